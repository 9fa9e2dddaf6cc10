"""Kernel-seam wrappers: the reference's internal/kernels entry points over
device tensors (torch is used only to hold HIP device memory and streams).

  quantize_symmetric_int8   <- QuantizeSymmetricINT8Into  internal/kernels/quantize.go:29
  Q8Weight + matmul_q8_0    <- MatMulQ8_0INT8             internal/kernels/quantize.go:346
  block_sums                <- the int32 block dots of matmulInnerLoop* (simd_amd64.s:241-304)
  rmsnorm                   <- RMSNorm                    internal/kernels/norm.go:8
  qknorm_rope               <- QK-norm + ApplyRoPECachedParallel (model_int8.go:371-452)
  attention                 <- MultiHeadAttentionChunked  internal/kernels/attention.go:88
  gelu_quick_mul            <- GELUQuickSIMD + VecMulF32  activation.go:47, matmul.go:238
  pool_l2                   <- MeanPoolingPartial + l2Normalize (attention.go:423, model.go:808)
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib


def _vp(t):
    return ctypes.c_void_p(t.data_ptr())


def _stream(stream):
    if stream is None:
        import torch
        return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    return ctypes.c_void_p(stream)


def _off(offsets):
    a = np.ascontiguousarray(offsets, np.int32)
    return a, ctypes.c_void_p(a.ctypes.data)


def _check_dev(*ts):
    for t in ts:
        if not t.is_cuda or not t.is_contiguous():
            raise ValueError("kernel-seam wrappers take contiguous device tensors")


class Q8Weight:
    """A raw Q8_0 matrix [out_dim][in_dim/32][34 B] repacked on the device."""

    def __init__(self, ctx, raw_q8: np.ndarray, out_dim: int, in_dim: int):
        self.ctx, self.lib = ctx, ctx.lib
        raw = np.ascontiguousarray(raw_q8, np.uint8)
        if raw.size != out_dim * (in_dim // 32) * 34:
            raise ValueError("raw Q8_0 size does not match out_dim x in_dim")
        h = ctypes.c_void_p()
        _lib.check(self.lib.sg_q8_weight_create(ctx.handle, ctypes.c_void_p(raw.ctypes.data), out_dim, in_dim,
                                                ctypes.byref(h)))
        self.handle, self.out_dim, self.in_dim = h, out_dim, in_dim

    def close(self):
        if self.handle:
            self.lib.sg_q8_weight_free(self.handle)
            self.handle = None


def quantize_symmetric_int8(ctx, x, offsets, q_out, scale_out, stream=None):
    _check_dev(x, q_out, scale_out)
    rows, cols = x.shape
    off, offp = _off(offsets)
    _lib.check(ctx.lib.sg_quantize_act(ctx.handle, _vp(x), rows, cols, offp, len(off) - 1, _vp(q_out),
                                       _vp(scale_out), _stream(stream)))


def matmul_q8_0(ctx, dst, w: Q8Weight, x, row_scale, stream=None):
    _check_dev(dst, x, row_scale)
    _lib.check(ctx.lib.sg_matmul_q8_0_int8(ctx.handle, _vp(dst), w.handle, _vp(x), _vp(row_scale), x.shape[0],
                                           _stream(stream)))


def matmul_q8_0_noalloc(ctx, dst, w: Q8Weight, x, row_scale, stream=None):
    """matmul_q8_0 with the operand relayout in the library's fixed per-device
    scratch (sg_matmul_q8_0_int8_noalloc): no device allocation."""
    _check_dev(dst, x, row_scale)
    _lib.check(ctx.lib.sg_matmul_q8_0_int8_noalloc(ctx.handle, _vp(dst), w.handle, _vp(x), _vp(row_scale),
                                                   x.shape[0], _stream(stream)))


def matmul_q8_0_kernel_us(ctx, dst, w: Q8Weight, x, row_scale, reps: int, stream=None) -> float:
    """Average time of the GEMM kernel alone over `reps` back-to-back launches
    (sg_matmul_q8_0_int8_bench; the operand relayout runs once, untimed)."""
    _check_dev(dst, x, row_scale)
    us = ctypes.c_float()
    _lib.check(ctx.lib.sg_matmul_q8_0_int8_bench(ctx.handle, _vp(dst), w.handle, _vp(x), _vp(row_scale), x.shape[0],
                                                 reps, _stream(stream), ctypes.byref(us)))
    return float(us.value)


def ffn_gate_up(ctx, dst, w_gate: Q8Weight, w_up: Q8Weight, x, row_scale, stream=None):
    """geluquick(x @ w_gate) * (x @ w_up) in one GEMM (model_int8.go:520-535)."""
    _check_dev(dst, x, row_scale)
    _lib.check(ctx.lib.sg_ffn_gate_up(ctx.handle, _vp(dst), w_gate.handle, w_up.handle, _vp(x), _vp(row_scale),
                                      x.shape[0], _stream(stream)))


def block_sums(ctx, out, w: Q8Weight, x, stream=None):
    _check_dev(out, x)
    _lib.check(ctx.lib.sg_q8_block_sums(ctx.handle, _vp(out), w.handle, _vp(x), x.shape[0], _stream(stream)))


def rmsnorm(ctx, dst, src, weight, eps, stream=None):
    _check_dev(dst, src, weight)
    rows, n = src.shape
    _lib.check(ctx.lib.sg_rmsnorm(ctx.handle, _vp(dst), _vp(src), _vp(weight), rows, n, ctypes.c_float(eps),
                                  _stream(stream)))


def qknorm_rope(ctx, q, k, q_norm, k_norm, n_heads, n_kv_heads, head_dim, eps, rope_base, max_seq_len, offsets,
                stream=None):
    _check_dev(q, k)
    off, offp = _off(offsets)
    _lib.check(ctx.lib.sg_qknorm_rope(ctx.handle, _vp(q), q.shape[1], _vp(k), k.shape[1],
                                      _vp(q_norm) if q_norm is not None else None,
                                      _vp(k_norm) if k_norm is not None else None, n_heads, n_kv_heads, head_dim,
                                      ctypes.c_float(eps), ctypes.c_float(rope_base), max_seq_len, offp, len(off) - 1,
                                      _stream(stream)))


def attention(ctx, out, q, k, v, n_heads, n_kv_heads, head_dim, offsets, stream=None):
    _check_dev(out, q, k, v)
    off, offp = _off(offsets)
    _lib.check(ctx.lib.sg_attention(ctx.handle, _vp(out), _vp(q), q.shape[1], _vp(k), _vp(v), k.shape[1], n_heads,
                                    n_kv_heads, head_dim, offp, len(off) - 1, _stream(stream)))


def attention_exact(ctx, out, q, k, v, n_heads, n_kv_heads, head_dim, offsets, stream=None):
    """attention() in the reference's float32 order (sg_attention_exact): bit-identical to it."""
    _check_dev(out, q, k, v)
    off, offp = _off(offsets)
    _lib.check(ctx.lib.sg_attention_exact(ctx.handle, _vp(out), _vp(q), q.shape[1], _vp(k), _vp(v), k.shape[1],
                                          n_heads, n_kv_heads, head_dim, offp, len(off) - 1, _stream(stream)))


def hbm_probe_us(ctx, kind: int, a, b, c, reps: int, stream=None) -> float:
    """sg_hbm_probe: average microseconds per launch of the streaming yardstick
    (kind 0: c = a + b fp32; kind 1: c = int8 codes of a)."""
    _check_dev(a, c)
    us = ctypes.c_float()
    _lib.check(ctx.lib.sg_hbm_probe(ctx.handle, kind, _vp(a), _vp(b) if b is not None else None, _vp(c),
                                    a.numel(), reps, _stream(stream), ctypes.byref(us)))
    return us.value


def issue_probe(ctx, kind: int, waves_per_simd: int, iters: int = 20000, stream=None):
    """sg_issue_probe: SIMD cycles per 32x32 subtile and K-block of the GEMM's
    arithmetic with no memory traffic (kind 0: MFMA + block-serial update;
    1: the VALU part; 2: the MFMA), and the shader clock in GHz."""
    cyc, ghz = ctypes.c_float(), ctypes.c_float()
    _lib.check(ctx.lib.sg_issue_probe(ctx.handle, kind, waves_per_simd, iters, _stream(stream), ctypes.byref(cyc),
                                      ctypes.byref(ghz)))
    return cyc.value, ghz.value


def gelu_quick_mul(ctx, dst, gate, up, stream=None):
    _check_dev(dst, gate, up)
    rows, cols = gate.shape
    _lib.check(ctx.lib.sg_gelu_quick_mul(ctx.handle, _vp(dst), dst.shape[1], _vp(gate), gate.shape[1], _vp(up),
                                         up.shape[1], rows, cols, _stream(stream)))


def embed_tokens(model, dst, tokens, stream=None):
    _check_dev(dst, tokens)
    _lib.check(model.lib.sg_embed_tokens(model.handle, _vp(dst), _vp(tokens), tokens.shape[0], _stream(stream)))


def pool_l2(ctx, out, x, out_dim, offsets, stream=None):
    _check_dev(out, x)
    off, offp = _off(offsets)
    _lib.check(ctx.lib.sg_pool_l2(ctx.handle, _vp(out), _vp(x), x.shape[1], out_dim, offp, len(off) - 1,
                                  _stream(stream)))
