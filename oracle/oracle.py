"""ctypes view of the CPU oracle (libsg_oracle.so) -- TEST INFRASTRUCTURE.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use
this module, and only as the checker / CPU baseline.  The product library
never loads it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libsg_oracle.so")

F16_RUNTIME, F16_GGUF, F16_KERNELS = 0, 1, 2
ORDER_VNNI, ORDER_AVX2, ORDER_BLOCK_SERIAL, ORDER_ARM64 = 0, 1, 2, 3

_lib = None


class Config(ctypes.Structure):
    _fields_ = [("embed_dim", ctypes.c_int32), ("num_layers", ctypes.c_int32), ("num_heads", ctypes.c_int32),
                ("num_kv_heads", ctypes.c_int32), ("head_dim", ctypes.c_int32), ("interm_dim", ctypes.c_int32),
                ("max_seq_len", ctypes.c_int32), ("vocab_size", ctypes.c_int32), ("norm_eps", ctypes.c_float),
                ("rope_base", ctypes.c_float)]


class Taps(ctypes.Structure):
    _fields_ = [("att_in", ctypes.c_void_p), ("qkv", ctypes.c_void_p), ("att", ctypes.c_void_p),
                ("h", ctypes.c_void_p), ("n_layers", ctypes.c_int32), ("layer_rows", ctypes.c_int64)]


class Layer(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in (
        "attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down",
        "attn_norm", "attn_q_norm", "attn_k_norm", "post_attention_norm", "ffn_norm", "post_ffw_norm")]


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        build()
    lib = ctypes.CDLL(LIB_PATH)
    vp, i32, i64, f32 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_float
    protos = {
        "sgo_f16_to_f32": (f32, [ctypes.c_uint16, ctypes.c_int]),
        "sgo_f16_table": (None, [ctypes.c_int, vp]),
        "sgo_quantize_symmetric": (f32, [vp, i64, vp]),
        "sgo_extract_q8_0_scales": (None, [vp, ctypes.c_int, ctypes.c_int, vp]),
        "sgo_matmul_q8_0_int8": (None, [vp, vp, vp, vp, vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int]),
        "sgo_block_sums": (None, [vp, vp, vp, ctypes.c_int, ctypes.c_int, ctypes.c_int]),
        "sgo_dot_f32": (f32, [vp, vp, ctypes.c_int]),
        "sgo_rmsnorm": (None, [vp, vp, vp, ctypes.c_int, f32]),
        "sgo_fast_exp": (f32, [f32]),
        "sgo_gelu_quick": (None, [vp, vp, i64]),
        "sgo_softmax": (None, [vp, vp, ctypes.c_int]),
        "sgo_rope_cache": (None, [vp, vp, vp, ctypes.c_int, f32, ctypes.c_int]),
        "sgo_rope_apply": (None, [vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, vp, vp]),
        "sgo_attention": (None, [vp, vp, vp, vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, f32]),
        "sgo_mean_pool_partial": (None, [vp, vp, ctypes.c_int, ctypes.c_int, ctypes.c_int]),
        "sgo_l2_normalize": (None, [vp, ctypes.c_int]),
        "sgo_dequant_q8_0_row": (None, [vp, vp, ctypes.c_int]),
        "sgo_model_create": (vp, [ctypes.POINTER(Config), vp, vp, ctypes.POINTER(Layer)]),
        "sgo_model_free": (None, [vp]),
        "sgo_forward": (ctypes.c_int, [vp, vp, ctypes.c_int, ctypes.c_int, vp, ctypes.c_int, ctypes.c_int]),
        "sgo_forward_batch": (ctypes.c_int, [vp, vp, vp, ctypes.c_int, ctypes.c_int, vp, ctypes.c_int, ctypes.c_int]),
        "sgo_forward_taps": (ctypes.c_int, [vp, vp, vp, ctypes.c_int, ctypes.c_int, vp, ctypes.c_int, ctypes.c_int,
                                            ctypes.POINTER(Taps)]),
        "sgo_simd_level": (ctypes.c_int, []),
        "sgo_force_scalar": (None, [ctypes.c_int]),
        "sgo_set_gemm_threads": (None, [ctypes.c_int]),
        "sgo_bf_normalize": (None, [vp, ctypes.c_int]),
        "sgo_bf_quantize_i8": (None, [vp, ctypes.c_int, vp]),
        "sgo_bf_quantize_i16": (None, [vp, ctypes.c_int, vp]),
        "sgo_bf_dot": (f32, [vp, ctypes.c_int, i64, vp, ctypes.c_int]),
        "sgo_bf_search": (ctypes.c_int, [vp, ctypes.c_int, vp, ctypes.c_int, ctypes.c_int, vp, ctypes.c_int, vp, vp]),
    }
    for name, (res, args) in protos.items():
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = res, args
    _lib = lib
    return lib


def _p(a):
    return ctypes.c_void_p(a.ctypes.data)


def f16_to_f32(bits: int, variant: int) -> float:
    return load().sgo_f16_to_f32(bits, variant)


def f16_table(variant: int) -> np.ndarray:
    out = np.empty(65536, np.float32)
    load().sgo_f16_table(variant, _p(out))
    return out


def quantize(x: np.ndarray):
    x = np.ascontiguousarray(x, np.float32)
    q = np.empty(x.shape, np.int8)
    s = load().sgo_quantize_symmetric(_p(x), x.size, _p(q))
    return q, np.float32(s)


def extract_scales(raw: np.ndarray, rows: int, cols: int) -> np.ndarray:
    raw = np.ascontiguousarray(raw, np.uint8)
    out = np.empty((rows, cols // 32), np.float32)
    load().sgo_extract_q8_0_scales(_p(raw), rows, cols, _p(out))
    return out


def matmul(raw_w: np.ndarray, x_q: np.ndarray, row_scale, out_dim: int, order: int = ORDER_VNNI) -> np.ndarray:
    raw_w = np.ascontiguousarray(raw_w, np.uint8)
    x_q = np.ascontiguousarray(x_q, np.int8)
    batch, in_dim = x_q.shape
    rs = np.ascontiguousarray(np.broadcast_to(np.asarray(row_scale, np.float32), (batch,)))
    sc = extract_scales(raw_w, out_dim, in_dim)
    out = np.empty((batch, out_dim), np.float32)
    load().sgo_matmul_q8_0_int8(_p(out), _p(raw_w), _p(sc), _p(x_q), _p(rs), batch, in_dim, out_dim, order)
    return out


def block_sums(raw_w: np.ndarray, x_q: np.ndarray, out_dim: int) -> np.ndarray:
    raw_w = np.ascontiguousarray(raw_w, np.uint8)
    x_q = np.ascontiguousarray(x_q, np.int8)
    batch, in_dim = x_q.shape
    out = np.empty((batch, out_dim, in_dim // 32), np.int32)
    load().sgo_block_sums(_p(out), _p(raw_w), _p(x_q), batch, in_dim, out_dim)
    return out


def dot(a, b) -> np.float32:
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return np.float32(load().sgo_dot_f32(_p(a), _p(b), a.size))


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """Row-wise RMSNorm over the last axis."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    n = x.shape[-1]
    out = np.empty_like(x)
    xf, of = x.reshape(-1, n), out.reshape(-1, n)
    lib = load()
    for r in range(xf.shape[0]):
        lib.sgo_rmsnorm(ctypes.c_void_p(of[r:].ctypes.data), ctypes.c_void_p(xf[r:].ctypes.data), _p(w), n, eps)
    return out


def fast_exp(x: float) -> np.float32:
    return np.float32(load().sgo_fast_exp(x))


def gelu_quick(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    load().sgo_gelu_quick(_p(out), _p(x), x.size)
    return out


def softmax(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    load().sgo_softmax(_p(out), _p(x), x.size)
    return out


def rope_cache(head_dim: int, base: float, max_pos: int):
    half = head_dim // 2
    fr = np.empty(half, np.float32)
    c = np.empty((max_pos, half), np.float32)
    s = np.empty((max_pos, half), np.float32)
    load().sgo_rope_cache(_p(fr), _p(c), _p(s), head_dim, base, max_pos)
    return fr, c, s


def rope_apply(qk: np.ndarray, n_heads: int, head_dim: int, cos_t, sin_t) -> np.ndarray:
    """qk [S, n_heads*head_dim], positions 0..S-1; returns a rotated copy."""
    out = np.array(qk, np.float32, copy=True, order="C")
    load().sgo_rope_apply(_p(out), out.shape[0], n_heads, head_dim, _p(np.ascontiguousarray(cos_t)),
                          _p(np.ascontiguousarray(sin_t)))
    return out


def attention(q, k, v, n_heads, n_kv_heads, head_dim, scale=None) -> np.ndarray:
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    S = q.shape[0]
    if scale is None:
        scale = np.float32(1.0) / np.float32(np.sqrt(np.float64(head_dim)))
    out = np.empty((S, n_heads * head_dim), np.float32)
    load().sgo_attention(_p(out), _p(q), _p(k), _p(v), S, n_heads, n_kv_heads, head_dim, float(scale))
    return out


def mean_pool_l2(x: np.ndarray, out_dim: int, normalize: bool = True) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    S, d = x.shape
    out = np.empty(out_dim, np.float32)
    lib = load()
    lib.sgo_mean_pool_partial(_p(out), _p(x), S, d, out_dim)
    if normalize:
        lib.sgo_l2_normalize(_p(out), out_dim)
    return out


def dequant_row(raw_row: np.ndarray, n: int) -> np.ndarray:
    raw_row = np.ascontiguousarray(raw_row, np.uint8)
    out = np.empty(n, np.float32)
    load().sgo_dequant_q8_0_row(_p(out), _p(raw_row), n)
    return out


# ---- brute-force search (search/brute), sg_oracle_search.c ----------------
BF_F32, BF_I8, BF_I16 = 0, 1, 2
_BF_DTYPE = {BF_F32: np.float32, BF_I8: np.int8, BF_I16: np.int16}


def bf_normalize(v: np.ndarray) -> np.ndarray:
    """builder.go:131-141 on a copy of each row of v ([dim] or [n, dim])."""
    out = np.array(v, np.float32, copy=True, order="C")
    rows = out.reshape(-1, out.shape[-1])
    for r in rows:
        load().sgo_bf_normalize(_p(r), r.size)
    return out


def bf_quantize(v: np.ndarray, mode: int) -> np.ndarray:
    """quant.go:17-41 (rows already normalized); BF_F32 returns a float32 copy."""
    v = np.ascontiguousarray(v, np.float32)
    if mode == BF_F32:
        return v.copy()
    out = np.empty(v.shape, _BF_DTYPE[mode])
    fn = load().sgo_bf_quantize_i8 if mode == BF_I8 else load().sgo_bf_quantize_i16
    rows_in, rows_out = v.reshape(-1, v.shape[-1]), out.reshape(-1, v.shape[-1])
    for a, b in zip(rows_in, rows_out):
        fn(_p(a), a.size, _p(b))
    return out


def bf_scores(data: np.ndarray, mode: int, query: np.ndarray) -> np.ndarray:
    """Score of every stored row against one (normalized) query."""
    data = np.ascontiguousarray(data, _BF_DTYPE[mode])
    q = np.ascontiguousarray(query, np.float32)
    n, dim = data.shape
    lib = load()
    return np.array([lib.sgo_bf_dot(_p(data), mode, i, _p(q), dim) for i in range(n)], np.float32)


def bf_search(data: np.ndarray, mode: int, ids: np.ndarray, query: np.ndarray, top_k: int):
    """searchNormalized (index.go:53-147): (ids, distances) sorted, or None for top_k <= 0."""
    data = np.ascontiguousarray(data, _BF_DTYPE[mode])
    ids = np.ascontiguousarray(ids, np.int32)
    q = np.ascontiguousarray(query, np.float32)
    n, dim = data.shape
    out_i = np.empty(max(min(top_k, n), 1), np.int32)
    out_d = np.empty(max(min(top_k, n), 1), np.float32)
    r = load().sgo_bf_search(_p(data), mode, _p(ids), n, dim, _p(q), top_k, _p(out_i), _p(out_d))
    if r < 0:
        return None
    return out_i[:r].copy(), out_d[:r].copy()


class OracleModel:
    """sgo_model over a SynthModel's arrays (borrowed, like the reference's GGUF views)."""

    def __init__(self, model):
        c = model.config
        self.config = c
        self.model = model
        hd = c["embed_dim"] // c["num_heads"]
        self._keep = []

        def p(a):
            if a is None:
                return None
            a = np.ascontiguousarray(a)
            self._keep.append(a)
            return a.ctypes.data

        cfg = Config(c["embed_dim"], c["num_layers"], c["num_heads"], c["num_kv_heads"], hd, c["interm_dim"],
                     c["max_seq_len"], c["vocab_size"], c["norm_eps"], c["rope_base"])
        layers = (Layer * c["num_layers"])()
        for i, ly in enumerate(model.layers):
            for name, _ in Layer._fields_:
                setattr(layers[i], name, p(ly.get(name)))
        self._keep.append(layers)
        self.handle = load().sgo_model_create(ctypes.byref(cfg), p(model.token_embd), p(model.output_norm), layers)

    def close(self):
        if self.handle:
            load().sgo_model_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def forward(self, tokens, target_dim: int, order: int = ORDER_VNNI, stop_layer: int = -1):
        tokens = np.ascontiguousarray(tokens, np.int32)
        S = tokens.size
        if stop_layer >= 0:
            out = np.empty((S, self.config["embed_dim"]), np.float32)
        else:
            out = np.empty(max(target_dim, 1), np.float32)
        rc = load().sgo_forward(self.handle, _p(tokens), S, target_dim, _p(out), order, stop_layer)
        return rc, out

    def forward_batch(self, tokens, offsets, target_dim: int, order: int = ORDER_VNNI, n_threads: int = 8):
        tokens = np.ascontiguousarray(tokens, np.int32)
        offsets = np.ascontiguousarray(offsets, np.int32)
        n = offsets.size - 1
        out = np.empty((n, target_dim), np.float32)
        rc = load().sgo_forward_batch(self.handle, _p(tokens), _p(offsets), n, target_dim, _p(out), order,
                                      n_threads)
        return rc, out

    def forward_taps(self, tokens, offsets, target_dim: int, n_layers: int, att_in=None, qkv=False, att=False,
                     h=True, order: int = ORDER_BLOCK_SERIAL, n_threads: int = 8):
        """Batched forward with per-layer taps over the packed rows (see
        sgo_taps): returns (rc, out [n_seq, target_dim], dict of the requested
        arrays, each [n_layers, T, cols]).  att_in [n_layers, T, q_dim]
        replaces each layer's attention output (teacher forcing)."""
        c = self.config
        tokens = np.ascontiguousarray(tokens, np.int32)
        offsets = np.ascontiguousarray(offsets, np.int32)
        n, T = offsets.size - 1, int(offsets[-1])
        hd = c["embed_dim"] // c["num_heads"]
        qd, kvd = c["num_heads"] * hd, c["num_kv_heads"] * hd
        taps = Taps(None, None, None, None, n_layers, T)
        arrays = {}
        if att_in is not None:
            att_in = np.ascontiguousarray(att_in, np.float32)
            if att_in.shape != (n_layers, T, qd):
                raise ValueError(f"att_in must be [{n_layers}, {T}, {qd}]")
            taps.att_in = att_in.ctypes.data
        for name, want, cols in (("qkv", qkv, qd + 2 * kvd), ("att", att, qd), ("h", h, c["embed_dim"])):
            if want:
                arrays[name] = np.zeros((n_layers, T, cols), np.float32)
                setattr(taps, name, arrays[name].ctypes.data)
        out = np.empty((n, target_dim), np.float32)
        rc = load().sgo_forward_taps(self.handle, _p(tokens), _p(offsets), n, target_dim, _p(out), order, n_threads,
                                     ctypes.byref(taps))
        return rc, out, arrays
