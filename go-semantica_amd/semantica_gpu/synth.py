"""Deterministic synthetic EmbeddingGemma-300M Q8_0 weights and inputs.

The real GGUF is not available offline, so benchmarks and tests use random
tensors of the exact shapes and byte format the GGUF holds:
  * Q8_0 matrices: GGUF blocks of 34 bytes (little-endian fp16 scale, then 32
    int8), int8 uniform in [-127, 127], scale = fp16(|N(0, 1e-3)|) (about 5% of
    those scales are fp16 subnormals, which exercises the token-embedding
    converter quirk);
  * F32 norm weights uniform in [0.5, 1.5];
  * token IDs uniform in [2, vocab).
All draws use numpy's PCG64 with fixed seeds, so every process (and the CPU
oracle fed the same arrays) sees identical bytes.
"""
from __future__ import annotations

import dataclasses

import numpy as np

# gemma-embedding.* metadata of embeddinggemma-300m (the keys parseConfig
# reads, internal/runtime/model.go:424-517).
EMBEDDINGGEMMA_300M = dict(
    embed_dim=768, num_layers=24, num_heads=3, num_kv_heads=1, interm_dim=1152,
    max_seq_len=2048, vocab_size=262144, norm_eps=1e-6, rope_base=10000.0)

SEED_WEIGHTS = 5
SEED_NORMS = 2
SEED_TOKENS = 0

LAYER_Q8 = ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down")
LAYER_NORMS = ("attn_norm", "attn_q_norm", "attn_k_norm", "post_attention_norm", "ffn_norm", "post_ffw_norm")


def q8_0_random(rng: np.random.Generator, rows: int, cols: int) -> np.ndarray:
    """Raw Q8_0 bytes, shape [rows, cols/32, 34]."""
    assert cols % 32 == 0
    nb = cols // 32
    out = np.empty((rows, nb, 34), np.uint8)
    d = np.abs(rng.normal(0.0, 1e-3, size=(rows, nb))).astype(np.float16)
    out[:, :, 0:2] = d.astype("<f2").view(np.uint8).reshape(rows, nb, 2)
    out[:, :, 2:] = rng.integers(-127, 128, size=(rows, nb, 32), dtype=np.int8).view(np.uint8)
    return out


def q8_0_from_parts(scales_f16: np.ndarray, qs: np.ndarray) -> np.ndarray:
    """Builds raw Q8_0 bytes from fp16 scales [rows, nb] and int8 values [rows, nb*32]."""
    rows, nb = scales_f16.shape
    out = np.empty((rows, nb, 34), np.uint8)
    out[:, :, 0:2] = scales_f16.astype("<f2").view(np.uint8).reshape(rows, nb, 2)
    out[:, :, 2:] = qs.astype(np.int8).reshape(rows, nb, 32).view(np.uint8)
    return out


@dataclasses.dataclass
class SynthModel:
    config: dict
    token_embd: np.ndarray          # uint8 [vocab, d/32, 34]
    output_norm: np.ndarray         # f32 [d]
    layers: list                    # dicts: name -> array

    def layer_shapes(self):
        c = self.config
        d, ff = c["embed_dim"], c["interm_dim"]
        hd = d // c["num_heads"]
        qd, kvd = c["num_heads"] * hd, c["num_kv_heads"] * hd
        return {"attn_q": (qd, d), "attn_k": (kvd, d), "attn_v": (kvd, d), "attn_output": (d, qd),
                "ffn_gate": (ff, d), "ffn_up": (ff, d), "ffn_down": (d, ff)}


def make_model(config: dict | None = None, seed_weights: int = SEED_WEIGHTS,
               seed_norms: int = SEED_NORMS) -> SynthModel:
    c = dict(EMBEDDINGGEMMA_300M if config is None else config)
    d, ff, L = c["embed_dim"], c["interm_dim"], c["num_layers"]
    hd = d // c["num_heads"]
    qd, kvd = c["num_heads"] * hd, c["num_kv_heads"] * hd
    rw = np.random.default_rng(seed_weights)
    rn = np.random.default_rng(seed_norms)
    shapes = {"attn_q": (qd, d), "attn_k": (kvd, d), "attn_v": (kvd, d), "attn_output": (d, qd),
              "ffn_gate": (ff, d), "ffn_up": (ff, d), "ffn_down": (d, ff)}
    norm_len = {"attn_norm": d, "attn_q_norm": hd, "attn_k_norm": hd, "post_attention_norm": d,
                "ffn_norm": d, "post_ffw_norm": d}
    token_embd = q8_0_random(rw, c["vocab_size"], d)
    layers = []
    for _ in range(L):
        ly = {}
        for name in LAYER_Q8:
            ly[name] = q8_0_random(rw, *shapes[name])
        for name in LAYER_NORMS:
            ly[name] = rn.uniform(0.5, 1.5, size=norm_len[name]).astype(np.float32)
        layers.append(ly)
    output_norm = rn.uniform(0.5, 1.5, size=d).astype(np.float32)
    return SynthModel(c, token_embd, output_norm, layers)


def token_ids(n: int, vocab: int, seed: int = SEED_TOKENS) -> np.ndarray:
    return np.random.default_rng(seed).integers(2, vocab, size=n, dtype=np.int64).astype(np.int32)


def offsets_from_lengths(lengths) -> np.ndarray:
    off = np.zeros(len(lengths) + 1, np.int32)
    off[1:] = np.cumsum(np.asarray(lengths, np.int64))
    return off


def lengths_uniform(n: int, lo: int, hi: int, seed: int) -> np.ndarray:
    """Config 3: S ~ U[lo, hi] per row."""
    return np.random.default_rng(seed).integers(lo, hi + 1, size=n).astype(np.int32)


def lengths_log_uniform(n: int, lo: int, hi: int, seed: int) -> np.ndarray:
    """Config 4: S = round(exp(U[ln lo, ln hi]))."""
    u = np.random.default_rng(seed).uniform(np.log(lo), np.log(hi), size=n)
    return np.clip(np.round(np.exp(u)), lo, hi).astype(np.int32)


# ---------------------------------------------------------------- GGUF images

GGUF_DTYPE_F32, GGUF_DTYPE_Q8_0 = 0, 8
_GGUF_MTYPE = {"u8": 0, "i8": 1, "u16": 2, "i16": 3, "u32": 4, "i32": 5, "f32": 6, "bool": 7, "str": 8,
               "arr": 9, "u64": 10, "i64": 11, "f64": 12}
_GGUF_FMT = {"u8": "<B", "i8": "<b", "u16": "<H", "i16": "<h", "u32": "<I", "i32": "<i", "f32": "<f",
             "bool": "<?", "u64": "<Q", "i64": "<q", "f64": "<d"}


def _gguf_str(s: str) -> bytes:
    import struct
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _gguf_value(kind: str, value) -> bytes:
    import struct
    if kind == "str":
        return _gguf_str(value)
    if kind.startswith("arr:"):
        ek = kind[4:]
        out = struct.pack("<IQ", _GGUF_MTYPE["arr" if ek.startswith("arr:") else ek], len(value))
        return out + b"".join(_gguf_value(ek, v) for v in value)
    return struct.pack(_GGUF_FMT[kind], value)


def gguf_image(metadata: list, tensors: list, version: int = 3) -> bytes:
    """A GGUF image in the layout internal/gguf/reader.go:98-178 reads.

    metadata: [(key, kind, value)] with kind one of u8..f64, "str", "arr:<kind>".
    tensors: [(name, dims (ne0 first), dtype, raw bytes)].  Tensor data starts
    at the end of the infos rounded up to 32 bytes; each tensor is placed at a
    32-byte aligned offset from there.
    """
    import struct
    head = struct.pack("<IIQQ", 0x46554747, version, len(tensors), len(metadata))
    kv = b"".join(_gguf_str(k) + struct.pack("<I", _GGUF_MTYPE["arr" if kind.startswith("arr:") else kind]) +
                  _gguf_value(kind, v) for k, kind, v in metadata)
    infos, blobs, off = [], [], 0
    for name, dims, dtype, raw in tensors:
        raw = bytes(raw)
        infos.append(_gguf_str(name) + struct.pack("<I", len(dims)) + struct.pack(f"<{len(dims)}Q", *dims) +
                     struct.pack("<IQ", dtype, off))
        blobs.append(raw + b"\0" * ((-len(raw)) % 32))
        off += len(blobs[-1])
    body = head + kv + b"".join(infos)
    return body + b"\0" * ((-len(body)) % 32) + b"".join(blobs)


def model_gguf(model: SynthModel, **kw) -> bytes:
    """model_gguf_parts assembled into one image."""
    return gguf_image(*model_gguf_parts(model, **kw))


def model_gguf_parts(model: SynthModel, arch: str = "gemma-embedding", norms_q8: bool = False, vocab_tokens=True,
                     extra_metadata: list = ()):
    """The synthetic model as a GGUF image with the tensor names and metadata keys
    the reference loader reads (model.go:424-552, model_int8.go:54-119).  With
    norms_q8 the norm vectors are stored as Q8_0 (scale 1/64, exact for values
    that are multiples of 1/64 in [-1.98, 1.98])."""
    c = model.config
    p = arch + "."
    md = [("general.architecture", "str", arch),
          (p + "embedding_length", "u32", c["embed_dim"]), (p + "block_count", "u32", c["num_layers"]),
          (p + "attention.head_count", "u32", c["num_heads"]),
          (p + "attention.head_count_kv", "u32", c["num_kv_heads"]),
          (p + "feed_forward_length", "u32", c["interm_dim"]), (p + "context_length", "u32", c["max_seq_len"]),
          (p + "attention.layer_norm_rms_epsilon", "f32", c["norm_eps"]),
          (p + "rope.freq_base", "f32", c["rope_base"])]
    if vocab_tokens:
        md.append(("tokenizer.ggml.tokens", "arr:str", [f"t{i}" for i in range(c["vocab_size"])]))
    md += list(extra_metadata)

    def norm(name, v):
        v = np.asarray(v, np.float32)
        if not norms_q8:
            return (name, [v.size], GGUF_DTYPE_F32, v.astype("<f4").tobytes())
        q = np.round(v * 64).astype(np.int8)
        raw = q8_0_from_parts(np.full((1, v.size // 32), 1 / 64, np.float16), q.reshape(1, -1))
        return (name, [v.size], GGUF_DTYPE_Q8_0, raw.tobytes())

    d = c["embed_dim"]
    ts = [("token_embd.weight", [d, c["vocab_size"]], GGUF_DTYPE_Q8_0, model.token_embd.tobytes())]
    if model.output_norm is not None:
        ts.append(norm("output_norm.weight", model.output_norm))
    for i, ly in enumerate(model.layers):
        for name in LAYER_Q8:
            rows = ly[name].shape[0]
            cols = ly[name].shape[1] * 32
            ts.append((f"blk.{i}.{name}.weight", [cols, rows], GGUF_DTYPE_Q8_0, ly[name].tobytes()))
        for name in LAYER_NORMS:
            if ly.get(name) is not None:
                ts.append(norm(f"blk.{i}.{name}.weight", ly[name]))
    return md, ts


def quantized_norms(model: SynthModel) -> SynthModel:
    """Copy of the model whose norm vectors are multiples of 1/64 (exact in the
    Q8_0 form model_gguf(norms_q8=True) writes)."""
    layers = [{k: (np.round(v * 64) / 64).astype(np.float32) if k in LAYER_NORMS else v for k, v in ly.items()}
              for ly in model.layers]
    on = None if model.output_norm is None else (np.round(model.output_norm * 64) / 64).astype(np.float32)
    return SynthModel(dict(model.config), model.token_embd, on, layers)
