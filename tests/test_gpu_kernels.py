"""Kernel-level parity: each HIP kernel (through the C ABI) against the oracle
on identical inputs.  Integer/byte results and every fp32 op whose reference
order the kernel reproduces are compared bit for bit; attention, which runs
its products on fp16 matrix cores, is compared with a stated tolerance."""
import sys

import numpy as np
import pytest

from conftest import rel_err

pytestmark = pytest.mark.gpu

GEMM_SHAPES = [(768, 768), (256, 768), (1152, 768), (768, 1152), (3072, 768), (768, 3072)]


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def _act_q(oracle, M, K, seed=3):
    """Config 1 activations: fp32 N(0,1) [M, K] quantized per tensor."""
    x = np.random.default_rng(seed).standard_normal((M, K)).astype(np.float32)
    return oracle.quantize(x)


@pytest.mark.parametrize("N,K", GEMM_SHAPES)
def test_gemm_block_sums_bit_exact(gpu_ctx, oracle, N, K):
    import torch
    from semantica_gpu import kernels, synth
    say(f"gemm block sums N={N} K={K} M=64 seed=5")
    raw = synth.q8_0_random(np.random.default_rng(5), N, K)
    xq, _ = _act_q(oracle, 64, K)
    w = kernels.Q8Weight(gpu_ctx, raw, N, K)
    out = torch.empty((64, N, K // 32), dtype=torch.int32, device="cuda")
    kernels.block_sums(gpu_ctx, out, w, dev(xq))
    got = host(out)
    w.close()
    assert np.array_equal(got, oracle.block_sums(raw, xq, N))


@pytest.mark.parametrize("N,K", GEMM_SHAPES)
def test_gemm_fp32_config1(gpu_ctx, oracle, N, K):
    """Config 1 at M = 2048: bit-exact to the block-serial FMA order (rows
    0..255 against the scalar oracle) and within 1e-5 (normwise) of the
    reference's AVX-512-VNNI accumulation order over all rows."""
    import torch
    from semantica_gpu import kernels, synth
    M = 2048
    say(f"gemm fp32 N={N} K={K} M={M} seeds w=5 x=3")
    raw = synth.q8_0_random(np.random.default_rng(5), N, K)
    xq, s = _act_q(oracle, M, K)
    w = kernels.Q8Weight(gpu_ctx, raw, N, K)
    y = torch.empty((M, N), dtype=torch.float32, device="cuda")
    kernels.matmul_q8_0(gpu_ctx, y, w, dev(xq), dev(np.full(M, s, np.float32)))
    got = host(y)
    w.close()
    serial = oracle.matmul(raw, xq[:256], s, N, oracle.ORDER_BLOCK_SERIAL)
    assert np.array_equal(got[:256].view(np.uint32), serial.view(np.uint32))
    vnni = oracle.matmul(raw, xq, s, N, oracle.ORDER_VNNI)
    assert rel_err(got, vnni) <= 1e-5
    avx2 = oracle.matmul(raw, xq, s, N, oracle.ORDER_AVX2)
    assert rel_err(got, avx2) <= 1e-5


def test_ffn_gate_up_interleave_cache(gpu_ctx):
    """sg_ffn_gate_up keeps the gate/up interleave on the gate weight and
    rebuilds it only when the up weight changes: one gate with two up weights,
    alternating, at M = 40 and 4200 and back, every call equal to the unfused
    GEMMs + GELU * up bit for bit."""
    import torch
    from semantica_gpu import kernels, synth
    N, K = 256, 768
    rng = np.random.default_rng(17)
    wg = kernels.Q8Weight(gpu_ctx, synth.q8_0_random(rng, N, K), N, K)
    ups = [kernels.Q8Weight(gpu_ctx, synth.q8_0_random(rng, N, K), N, K) for _ in range(2)]
    say("ffn gate/up interleave cache")
    try:
        for M, u in [(40, 0), (40, 0), (40, 1), (4200, 1), (4200, 0), (40, 0), (4200, 0)]:
            xq = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
            rs = rng.uniform(1e-3, 2e-2, M).astype(np.float32)
            gate = torch.empty((M, N), dtype=torch.float32, device="cuda")
            up, ref, got = torch.empty_like(gate), torch.empty_like(gate), torch.empty_like(gate)
            kernels.matmul_q8_0(gpu_ctx, gate, wg, dev(xq), dev(rs))
            kernels.matmul_q8_0(gpu_ctx, up, ups[u], dev(xq), dev(rs))
            kernels.gelu_quick_mul(gpu_ctx, ref, gate, up)
            kernels.ffn_gate_up(gpu_ctx, got, wg, ups[u], dev(xq), dev(rs))
            assert np.array_equal(host(got).view(np.uint32), host(ref).view(np.uint32)), (M, u)
    finally:
        wg.close()
        for w in ups:
            w.close()


@pytest.mark.parametrize("M,K", [(1, 768), (33, 768), (1100, 800), (2048, 768), (4500, 768), (8200, 768),
                                 (4500, 800)])
def test_ffn_gate_up_fused_bit_exact(gpu_ctx, oracle, M, K):
    """The fused gate/up GEMM with GELUQuick * up in its epilogue equals the
    unfused GEMMs followed by the GELU kernel bit for bit, and the first rows
    equal the oracle's block-serial GEMMs + geluquick * up.  The fused GEMM
    runs register-direct below 4096 rows and on the 8-wave direct-to-LDS
    kernel from there; K = 800 leaves 25 blocks (an odd last block after the
    register-direct block pairs, a partial last round of the ring-unrolled
    LDS loop)."""
    import torch
    from semantica_gpu import kernels, synth
    N = 1152
    rng = np.random.default_rng(M + K)
    say(f"ffn gate/up fused M={M} N={N} K={K}")
    raw_g, raw_u = synth.q8_0_random(rng, N, K), synth.q8_0_random(rng, N, K)
    xq = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
    rs = rng.uniform(1e-3, 2e-2, M).astype(np.float32)
    wg, wu = kernels.Q8Weight(gpu_ctx, raw_g, N, K), kernels.Q8Weight(gpu_ctx, raw_u, N, K)
    gate = torch.empty((M, N), dtype=torch.float32, device="cuda")
    up = torch.empty_like(gate)
    ref = torch.empty_like(gate)
    got = torch.empty_like(gate)
    kernels.matmul_q8_0(gpu_ctx, gate, wg, dev(xq), dev(rs))
    kernels.matmul_q8_0(gpu_ctx, up, wu, dev(xq), dev(rs))
    kernels.gelu_quick_mul(gpu_ctx, ref, gate, up)
    kernels.ffn_gate_up(gpu_ctx, got, wg, wu, dev(xq), dev(rs))
    wg.close()
    wu.close()
    g_host, r_host = host(got), host(ref)
    assert np.array_equal(g_host.view(np.uint32), r_host.view(np.uint32))
    m = min(M, 64)
    og = oracle.matmul(raw_g, xq[:m], rs[:m], N, oracle.ORDER_BLOCK_SERIAL)
    ou = oracle.matmul(raw_u, xq[:m], rs[:m], N, oracle.ORDER_BLOCK_SERIAL)
    want = oracle.gelu_quick(og) * ou
    assert np.array_equal(g_host[:m].view(np.uint32), want.view(np.uint32))


def test_ffn_gate_up_rejects_weights_of_another_context(gpu_ctx):
    """The gate weight caches its gate/up interleave under its own context's
    lock and scratch event, so a call through another context is refused."""
    import torch
    from semantica_gpu import Context, SemanticaError, _lib, kernels, synth
    rng = np.random.default_rng(5)
    N, K, M = 64, 64, 4
    other = Context(0)
    try:
        wg = kernels.Q8Weight(other, synth.q8_0_random(rng, N, K), N, K)
        wu = kernels.Q8Weight(other, synth.q8_0_random(rng, N, K), N, K)
        out = torch.empty((M, N), dtype=torch.float32, device="cuda")
        xq = dev(rng.integers(-127, 128, size=(M, K), dtype=np.int8))
        rs = dev(np.ones(M, np.float32))
        say("ffn gate/up with another context's weights")
        with pytest.raises(SemanticaError) as e:
            kernels.ffn_gate_up(gpu_ctx, out, wg, wu, xq, rs)
        assert e.value.code == _lib.SG_ERR_INVALID and "another context" in e.value.message
        kernels.ffn_gate_up(other, out, wg, wu, xq, rs)  # their own context accepts them
        torch.cuda.synchronize()
        wg.close()
        wu.close()
    finally:
        other.close()


@pytest.mark.parametrize("M", [6, 8200, 12300])
def test_gemm_order_pins(gpu_ctx, M):
    """The hand-derived order vectors of tests/gemm_pins.py: row i and
    column j hold pin i % 6's activations and pin j's weights, and the
    diagonal outputs must equal each pin's block-serial value exactly (which
    the VNNI, AVX2 and arm64 orders each miss on at least one pin).  M = 6
    runs the register-direct kernel, 8200 the 4-wave and 12300 the 8-wave
    direct-to-LDS kernel."""
    import torch
    import gemm_pins
    from semantica_gpu import kernels, synth
    pins = gemm_pins.PINS
    n = len(pins)
    ops = [p.operands() for p in pins]
    x = np.concatenate([o[0] for o in ops])
    raw = synth.q8_0_from_parts(np.concatenate([o[2] for o in ops]), np.concatenate([o[1] for o in ops]))
    xq = x[np.arange(M) % n]
    say(f"gemm order pins M={M} N={n} K=64")
    w = kernels.Q8Weight(gpu_ctx, raw.reshape(n, -1), n, 64)
    y = torch.empty((M, n), dtype=torch.float32, device="cuda")
    kernels.matmul_q8_0(gpu_ctx, y, w, dev(xq), dev(np.ones(M, np.float32)))
    got = host(y)
    w.close()
    for r in range(M):
        p = pins[r % n]
        assert got[r, r % n] == float(p.expected["block_serial"]), (M, r, p.name, got[r, r % n])


@pytest.mark.parametrize("M,N,K", [(2048, 768, 768), (2049, 768, 768), (6143, 256, 800), (33, 768, 1152)])
def test_gemm_mfma_ahead_threshold(gpu_ctx, oracle, M, N, K):
    """Register-direct launches of at most 384 workgroups run the MFMA-ahead
    loop (3-stage ring), larger ones the plain 2-stage loop: 2048 x 768 is
    exactly 384 64x64 tiles, 2049 rows 396; 6143 x 256 is 384 tiles with
    K = 800 (25 blocks: a partial last ring round); 33 x 768 x 1152 one row
    of tiles with 36 blocks.  The first and last 64 rows and every 37th row
    bit-exact to the block-serial order."""
    import torch
    from semantica_gpu import kernels, synth
    rng = np.random.default_rng(M + N + K)
    say(f"gemm MFMA-ahead threshold M={M} N={N} K={K}")
    raw = synth.q8_0_random(rng, N, K)
    xq = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
    rs = rng.uniform(1e-3, 2.0, size=M).astype(np.float32)
    w = kernels.Q8Weight(gpu_ctx, raw, N, K)
    y = torch.empty((M, N), dtype=torch.float32, device="cuda")
    kernels.matmul_q8_0(gpu_ctx, y, w, dev(xq), dev(rs))
    got = host(y)
    w.close()
    rows = np.unique(np.concatenate([np.arange(min(64, M)), np.arange(max(0, M - 64), M), np.arange(0, M, 37)]))
    ref = oracle.matmul(raw, xq[rows], rs[rows], N, oracle.ORDER_BLOCK_SERIAL)
    assert np.array_equal(got[rows].view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("M", [1280, 1408])
def test_ffn_gate_up_mfma_ahead_threshold(gpu_ctx, oracle, M):
    """The fused gate/up GEMM on both sides of the 384-workgroup MFMA-ahead
    threshold (128 x 64 tiles over 2 x 1152 columns: 1280 rows are 360
    workgroups, 1408 rows 396): bit-identical to the unfused GEMMs + GELU."""
    import torch
    from semantica_gpu import kernels, synth
    N, K = 1152, 768
    rng = np.random.default_rng(M)
    say(f"ffn gate/up MFMA-ahead threshold M={M}")
    wg = kernels.Q8Weight(gpu_ctx, synth.q8_0_random(rng, N, K), N, K)
    wu = kernels.Q8Weight(gpu_ctx, synth.q8_0_random(rng, N, K), N, K)
    xq = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
    rs = rng.uniform(1e-3, 2e-2, M).astype(np.float32)
    gate = torch.empty((M, N), dtype=torch.float32, device="cuda")
    up, ref, got = torch.empty_like(gate), torch.empty_like(gate), torch.empty_like(gate)
    kernels.matmul_q8_0(gpu_ctx, gate, wg, dev(xq), dev(rs))
    kernels.matmul_q8_0(gpu_ctx, up, wu, dev(xq), dev(rs))
    kernels.gelu_quick_mul(gpu_ctx, ref, gate, up)
    kernels.ffn_gate_up(gpu_ctx, got, wg, wu, dev(xq), dev(rs))
    wg.close()
    wu.close()
    assert np.array_equal(host(got).view(np.uint32), host(ref).view(np.uint32))


def test_gemm_ragged_m_and_extremes(gpu_ctx, oracle):
    """M not a multiple of any tile; blocks at +-127 extremes; per-row scales."""
    import torch
    from semantica_gpu import kernels, synth
    rng = np.random.default_rng(8)
    for M, N, K in ((1, 256, 768), (33, 1280, 768), (257, 2304, 768), (70, 768, 1152)):
        say(f"gemm ragged M={M} N={N} K={K}")
        raw = synth.q8_0_random(rng, N, K)
        xq = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
        xq[0, :] = 127
        rs = rng.uniform(1e-3, 2.0, size=M).astype(np.float32)
        w = kernels.Q8Weight(gpu_ctx, raw, N, K)
        y = torch.empty((M, N), dtype=torch.float32, device="cuda")
        kernels.matmul_q8_0(gpu_ctx, y, w, dev(xq), dev(rs))
        got = host(y)
        w.close()
        ref = np.stack([oracle.matmul(raw, xq[i:i + 1], rs[i], N, oracle.ORDER_BLOCK_SERIAL)[0] for i in range(M)])
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_gemm_seam_async_across_streams(gpu_ctx, oracle):
    """sg_matmul_q8_0_int8 returns once enqueued and shares the context's operand
    scratch: calls on two streams issued back to back (the second with a larger
    input, which regrows the scratch) must each produce their own result."""
    import torch
    from semantica_gpu import kernels, synth
    rng = np.random.default_rng(21)
    N, K = 768, 768
    raw = synth.q8_0_random(rng, N, K)
    w = kernels.Q8Weight(gpu_ctx, raw, N, K)
    xs = [rng.integers(-127, 128, size=(m, K), dtype=np.int8) for m in (300, 2100)]
    rs = [rng.uniform(1e-3, 2.0, size=x.shape[0]).astype(np.float32) for x in xs]
    dx = [dev(x) for x in xs]
    drs = [dev(r) for r in rs]
    ys = [torch.empty((x.shape[0], N), dtype=torch.float32, device="cuda") for x in xs]
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    say("gemm seam: two streams, M=300 then M=2100")
    for _ in range(3):
        kernels.matmul_q8_0(gpu_ctx, ys[0], w, dx[0], drs[0], stream=s1.cuda_stream)
        kernels.matmul_q8_0(gpu_ctx, ys[1], w, dx[1], drs[1], stream=s2.cuda_stream)
    torch.cuda.synchronize()
    w.close()
    for x, r, y in zip(xs, rs, ys):
        got = host(y)
        ref = np.stack([oracle.matmul(raw, x[i:i + 1], r[i], N, oracle.ORDER_BLOCK_SERIAL)[0] for i in range(0, len(x), 97)])
        assert np.array_equal(got[::97].view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("M", [300, 8200, 12300])
def test_gemm_unaligned_activations(gpu_ctx, M):
    """int8 activations at an odd address take the byte-wise relayout: same
    bits as the aligned call (register-direct at 300 rows, 4-wave
    direct-to-LDS at 8200, 8-wave at 12300)."""
    import torch
    from semantica_gpu import kernels, synth
    N, K = 768, 768
    rng = np.random.default_rng(M)
    say(f"gemm unaligned activations M={M}")
    raw = synth.q8_0_random(rng, N, K)
    xq = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
    rs = rng.uniform(1e-3, 2.0, size=M).astype(np.float32)
    w = kernels.Q8Weight(gpu_ctx, raw, N, K)
    buf = torch.zeros(M * K + 1, dtype=torch.int8, device="cuda")
    buf[1:] = torch.from_numpy(xq.reshape(-1)).cuda()
    x_odd = buf[1:].view(M, K)
    assert x_odd.data_ptr() % 16 != 0
    y0 = torch.empty((M, N), dtype=torch.float32, device="cuda")
    y1 = torch.empty((M, N), dtype=torch.float32, device="cuda")
    kernels.matmul_q8_0(gpu_ctx, y0, w, dev(xq), dev(rs))
    kernels.matmul_q8_0(gpu_ctx, y1, w, x_odd, dev(rs))
    a, b = host(y0), host(y1)
    w.close()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("M", [4500, 8200, 12300])
@pytest.mark.parametrize("N,K", [(1280, 768), (768, 1152), (768, 800)])
def test_gemm_large_m(gpu_ctx, oracle, M, N, K):
    """Large M: 4500 rows on the register-direct kernel, 8200 on the 4-wave
    (128 x 64 tiles, 6-stage ring) and 12300 on the 8-wave (256 x 128 tiles,
    3-stage ring) direct-to-LDS kernel; ragged last tiles; K = 800 leaves 25
    blocks (an odd last block after the register-direct block pairs, a
    partial last round of the ring-unrolled LDS loops): the first and last
    128 rows bit-exact to the block-serial order, every 7th row within 1e-5
    of AVX2's."""
    import torch
    from semantica_gpu import kernels, synth
    rng = np.random.default_rng(N + K)
    say(f"gemm large M={M} N={N} K={K}")
    raw = synth.q8_0_random(rng, N, K)
    xq = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
    rs = rng.uniform(1e-3, 2.0, size=M).astype(np.float32)
    w = kernels.Q8Weight(gpu_ctx, raw, N, K)
    y = torch.empty((M, N), dtype=torch.float32, device="cuda")
    kernels.matmul_q8_0(gpu_ctx, y, w, dev(xq), dev(rs))
    got = host(y)
    w.close()
    for lo, hi in ((0, 128), (M - 128, M)):
        ref = oracle.matmul(raw, xq[lo:hi], rs[lo:hi], N, oracle.ORDER_BLOCK_SERIAL)
        assert np.array_equal(got[lo:hi].view(np.uint32), ref.view(np.uint32))
    sub = np.arange(0, M, 7)
    assert rel_err(got[sub], oracle.matmul(raw, xq[sub], rs[sub], N, oracle.ORDER_AVX2)) <= 1e-5


@pytest.mark.parametrize("cols", [768, 1152])
def test_quantize_per_sequence_bit_exact(gpu_ctx, oracle, cols):
    import torch
    from semantica_gpu import kernels
    rng = np.random.default_rng(cols)
    lens = [1, 299, 0, 400, 37, 263]
    off = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    T = int(off[-1])
    say(f"quantize cols={cols} lens={lens}")
    x = (rng.standard_normal((T, cols)) * rng.uniform(0.01, 50, size=(T, 1))).astype(np.float32)
    x[off[3]:off[4]] = 0.0                      # an all-zero sequence
    x[off[1]:off[2]][0, :4] = [127.0, 2.5, -2.5, 0.5]   # exact ties inside a sequence
    x[off[1]:off[2]] = np.clip(x[off[1]:off[2]], -127, 127)
    q = torch.empty((T, cols), dtype=torch.int8, device="cuda")
    sc = torch.empty(len(lens), dtype=torch.float32, device="cuda")
    kernels.quantize_symmetric_int8(gpu_ctx, dev(x), off, q, sc)
    qg, sg = host(q), host(sc)
    for i in range(len(lens)):
        qo, so = oracle.quantize(x[off[i]:off[i + 1]])
        assert sg[i] == so, i
        assert np.array_equal(qg[off[i]:off[i + 1]], qo), i


def _near_ties(m):
    """Values x (|x| < m) whose float32 product with the kernel's inv =
    1/(m/127) lands exactly on k + 1/2, while the exact product (what the
    reference's float64 multiply gives) sits on, above or below that half:
    the cases where rounding the float32 product alone would go wrong."""
    inv = np.float32(1) / (np.float32(m) / np.float32(127))
    xs, lo_sign = [], []
    for k in range(-127, 127):
        x0 = np.float32((k + 0.5) / np.float64(inv))
        for d in range(-6, 7):
            x = (np.array([x0]).view(np.int32) + d).view(np.float32)[0]
            p = np.float64(x) * np.float64(inv)  # exact
            hi = np.float32(p)
            if np.float64(hi) == k + 0.5 and abs(x) < m:
                xs.append(x)
                lo_sign.append(np.sign(p - np.float64(hi)))
    return np.array(xs, np.float32), np.array(lo_sign)


def test_quantize_near_ties_bit_exact(gpu_ctx, oracle):
    """Round-half-away of the exact product x*inv, on the inputs where a
    float32 product rounds onto a half: one sequence per max value m."""
    import torch
    from semantica_gpu import kernels
    cols = 64
    rows, signs = [], []
    for m in (127.0, 63.5, 254.0, 1.0, 3.7, 50.3, 126.9, 0.0123, 1e-3):  # first three: exact ties
        xs, sg = _near_ties(m)
        signs.append(sg)
        n = -(-(len(xs) + 1) // cols) * cols
        v = np.zeros(n, np.float32)
        v[0] = m
        v[1:len(xs) + 1] = xs
        rows.append(v.reshape(-1, cols))
    signs = np.concatenate(signs)
    assert (signs > 0).sum() > 50 and (signs < 0).sum() > 50 and (signs == 0).sum() > 50
    lens = [len(r) for r in rows]
    off = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    x = np.concatenate(rows)
    say(f"quantize near ties: {len(signs)} values over {len(lens)} sequences")
    q = torch.empty(x.shape, dtype=torch.int8, device="cuda")
    sc = torch.empty(len(lens), dtype=torch.float32, device="cuda")
    kernels.quantize_symmetric_int8(gpu_ctx, dev(x), off, q, sc)
    qg, sgp = host(q), host(sc)
    for i in range(len(lens)):
        qo, so = oracle.quantize(x[off[i]:off[i + 1]])
        assert sgp[i] == so, i
        assert np.array_equal(qg[off[i]:off[i + 1]], qo), i


@pytest.mark.parametrize("n", [256, 768])
def test_rmsnorm_bit_exact(gpu_ctx, oracle, n):
    import torch
    from semantica_gpu import kernels
    rng = np.random.default_rng(n)
    x = (rng.standard_normal((1001, n)) * rng.uniform(1e-3, 100, size=(1001, 1))).astype(np.float32)
    w = rng.uniform(0.5, 1.5, n).astype(np.float32)
    say(f"rmsnorm n={n}")
    y = torch.empty_like(dev(x))
    kernels.rmsnorm(gpu_ctx, y, dev(x), dev(w), 1e-6)
    got = host(y)
    ref = oracle.rmsnorm(x, w, 1e-6)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_qknorm_rope_bit_exact(gpu_ctx, oracle):
    from semantica_gpu import kernels
    rng = np.random.default_rng(21)
    lens = [3, 64, 1, 700]
    off = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    T = int(off[-1])
    say(f"qknorm_rope lens={lens}")
    q = (rng.standard_normal((T, 768)) * 4).astype(np.float32)
    k = (rng.standard_normal((T, 256)) * 4).astype(np.float32)
    qw = rng.uniform(0.5, 1.5, 256).astype(np.float32)
    kw = rng.uniform(0.5, 1.5, 256).astype(np.float32)
    qd, kd = dev(q), dev(k)
    kernels.qknorm_rope(gpu_ctx, qd, kd, dev(qw), dev(kw), 3, 1, 256, 1e-6, 10000.0, 2048, off)
    gq, gk = host(qd), host(kd)
    _, c, s = oracle.rope_cache(256, 10000.0, 2048)
    for i in range(len(lens)):
        sl = slice(off[i], off[i + 1])
        rq = oracle.rope_apply(oracle.rmsnorm(q[sl].reshape(-1, 256), qw, 1e-6).reshape(-1, 768), 3, 256, c, s)
        rk = oracle.rope_apply(oracle.rmsnorm(k[sl], kw, 1e-6), 1, 256, c, s)
        assert np.array_equal(gq[sl].view(np.uint32), rq.view(np.uint32)), i
        assert np.array_equal(gk[sl].view(np.uint32), rk.view(np.uint32)), i


# Attention runs its products as split fp16 (hi + lo, ~2^-22 relative) with
# fp32 accumulation; the oracle is the reference's fp32 order.
ATTN_REL_TOL = 1e-5


# Batches whose longest sequence has at most 512 keys keep all of pass 1's
# scores in registers; a longer one switches the whole launch to the variant
# that spills the scores past 512 keys.
@pytest.mark.parametrize("lens", [[1, 31, 32, 33, 100, 517], [1, 31, 32, 33, 100, 512]])
def test_attention_vs_oracle(gpu_ctx, oracle, lens):
    import torch
    from semantica_gpu import kernels
    rng = np.random.default_rng(31)
    off = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    T = int(off[-1])
    say(f"attention lens={lens}")
    # post-QK-norm magnitudes: unit RMS rows times weights in [0.5, 1.5]
    q = (rng.standard_normal((T, 768)) * rng.uniform(0.5, 1.5, 768)).astype(np.float32)
    k = (rng.standard_normal((T, 256)) * rng.uniform(0.5, 1.5, 256)).astype(np.float32)
    v = (rng.standard_normal((T, 256)) * 2).astype(np.float32)
    out = torch.empty((T, 768), dtype=torch.float32, device="cuda")
    kernels.attention(gpu_ctx, out, dev(q), dev(k), dev(v), 3, 1, 256, off)
    got = host(out)
    for i in range(len(lens)):
        sl = slice(off[i], off[i + 1])
        ref = oracle.attention(q[sl], k[sl], v[sl], 3, 1, 256)
        assert rel_err(got[sl], ref) < ATTN_REL_TOL, (i, rel_err(got[sl], ref))
        assert np.max(np.abs(got[sl] - ref)) < 1e-4 * np.max(np.abs(v[sl])), i


# Past 512 keys the tiles beyond the register-held ones keep their scores in a
# global spill buffer (slots only for the workgroups of sequences that long, per
# kv head) and reach pass 2 through the V^T items' copies: the longest sequence
# (2048 keys, 48 spilled tiles), a sequence ending one key into a tile, grouped
# kv heads, and long sequences among many short ones.
@pytest.mark.parametrize("lens,heads", [([2048, 700, 1, 513], (3, 1)), ([1000, 40, 545], (4, 2)),
                                        ([33] * 30 + [1500] + [7] * 20 + [600], (3, 1))])
def test_attention_spilled_scores_vs_oracle(gpu_ctx, oracle, lens, heads):
    import torch
    from semantica_gpu import kernels
    H, HKV = heads
    rng = np.random.default_rng(32)
    off = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    T = int(off[-1])
    say(f"attention spilled scores lens={lens} heads={heads}")
    q = (rng.standard_normal((T, H * 256)) * rng.uniform(0.5, 1.5, H * 256)).astype(np.float32)
    k = (rng.standard_normal((T, HKV * 256)) * rng.uniform(0.5, 1.5, HKV * 256)).astype(np.float32)
    v = (rng.standard_normal((T, HKV * 256)) * 2).astype(np.float32)
    out = torch.empty((T, H * 256), dtype=torch.float32, device="cuda")
    kernels.attention(gpu_ctx, out, dev(q), dev(k), dev(v), H, HKV, 256, off)
    got = host(out)
    for i in range(len(lens)):
        sl = slice(off[i], off[i + 1])
        ref = oracle.attention(q[sl], k[sl], v[sl], H, HKV, 256)
        assert rel_err(got[sl], ref) < ATTN_REL_TOL, (i, rel_err(got[sl], ref))
        assert np.max(np.abs(got[sl] - ref)) < 1e-4 * np.max(np.abs(v[sl])), i


@pytest.mark.parametrize("lens,heads,nonfinite", [([1, 3, 7, 64, 65, 300, 513], (3, 1), False),
                                                  ([1100, 2048], (3, 1), False),
                                                  ([130, 5, 64], (4, 2), False),
                                                  ([90, 200], (3, 1), True)])
def test_attention_exact_bit_exact(gpu_ctx, oracle, lens, heads, nonfinite):
    """sg_attention_exact against the oracle's restatement of
    multiHeadAttentionInternal (attention.go:101-363), bit for bit: lengths
    across the 64-key score tiles, the 4-key softmax groups and their tails,
    up to 2048 keys, and a grouped-query shape with two KV heads.  Some query
    rows are scaled up so that their score ranges pass fastExp's -10 clamp:
    those weights are exact zeros and their keys are skipped.  In the last
    case some values are infinite or NaN, where skipping a zero-weight key
    (rather than adding 0 * v) decides the result (any NaN matches any NaN)."""
    import torch
    from semantica_gpu import kernels
    H, HKV = heads
    rng = np.random.default_rng(sum(lens) + H)
    off = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    T = int(off[-1])
    say(f"exact attention lens={lens} heads={H}/{HKV}")
    q = (rng.standard_normal((T, H * 256)) * rng.uniform(0.5, 1.5, H * 256)).astype(np.float32)
    q[::5] *= 6.0  # wide score ranges: clamped weights
    k = (rng.standard_normal((T, HKV * 256)) * rng.uniform(0.5, 1.5, HKV * 256)).astype(np.float32)
    v = (rng.standard_normal((T, HKV * 256)) * 2).astype(np.float32)
    if nonfinite:
        v[7, 3], v[50, 100], v[150, 9] = np.inf, -np.inf, np.nan
    out = torch.full((T, H * 256), float("nan"), dtype=torch.float32, device="cuda")
    kernels.attention_exact(gpu_ctx, out, dev(q), dev(k), dev(v), H, HKV, 256, off)
    got = host(out)
    clamped = 0
    for i in range(len(lens)):
        sl = slice(off[i], off[i + 1])
        ref = oracle.attention(q[sl], k[sl], v[sl], H, HKV, 256)
        same = (got[sl].view(np.uint32) == ref.view(np.uint32)) | (np.isnan(got[sl]) & np.isnan(ref))
        assert same.all(), (i, lens[i])
        if nonfinite:  # finite and non-finite outputs both occur
            assert np.isfinite(ref).any() and not np.isfinite(ref).all()
        if lens[i] > 1:
            s = (q[sl][:, :256].astype(np.float64) @ k[sl][:, :256].T.astype(np.float64)) / 16
            clamped += int(np.sum(s - s.max(axis=1, keepdims=True) < -10))
    say(f"  bit-identical; {clamped} clamped (query, key) pairs in head 0")
    if max(lens) > 64:
        assert clamped > 0


def test_attention_register_scores_match_spilling_launch(gpu_ctx):
    """The same sequences with and without a 600-key companion (which moves the
    launch to the kernel variant that spills scores past 512 keys) give
    identical bits."""
    import torch
    from semantica_gpu import kernels
    rng = np.random.default_rng(77)
    lens = [512, 1, 300, 47, 480, 33]
    long_len = 600
    T0 = sum(lens)
    T = T0 + long_len
    say(f"attention register-only vs spilling launch lens={lens} + [{long_len}]")
    q = (rng.standard_normal((T, 768)) * rng.uniform(0.5, 1.5, 768)).astype(np.float32)
    k = (rng.standard_normal((T, 256)) * rng.uniform(0.5, 1.5, 256)).astype(np.float32)
    v = (rng.standard_normal((T, 256)) * 2).astype(np.float32)
    off_a = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    off_b = np.concatenate([[0], np.cumsum(lens + [long_len])]).astype(np.int32)
    out_a = torch.empty((T0, 768), dtype=torch.float32, device="cuda")
    out_b = torch.empty((T, 768), dtype=torch.float32, device="cuda")
    kernels.attention(gpu_ctx, out_a, dev(q[:T0]), dev(k[:T0]), dev(v[:T0]), 3, 1, 256, off_a)
    kernels.attention(gpu_ctx, out_b, dev(q), dev(k), dev(v), 3, 1, 256, off_b)
    a, b = host(out_a), host(out_b)[:T0]
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_attention_clamped_keys_are_exact_zero(gpu_ctx, oracle):
    """A key 25 above the rest (after scaling) gives the others weight exactly
    0 (fastExp's -10 clamp), so the output is exactly that key's V row."""
    import torch
    from semantica_gpu import kernels
    S = 70
    rng = np.random.default_rng(5)
    q = np.zeros((S, 768), np.float32)
    q[:, 0] = q[:, 256] = q[:, 512] = 1.0
    k = np.zeros((S, 256), np.float32)
    k[40, 0] = 400.0
    v = rng.standard_normal((S, 256)).astype(np.float32)
    v = v.astype(np.float16).astype(np.float32)  # exactly representable in fp16
    out = torch.empty((S, 768), dtype=torch.float32, device="cuda")
    say("attention clamp case S=70")
    kernels.attention(gpu_ctx, out, dev(q), dev(k), dev(v), 3, 1, 256, np.array([0, S], np.int32))
    got = host(out)
    for h in range(3):
        assert np.array_equal(got[:, 256 * h:256 * (h + 1)], np.tile(v[40], (S, 1)))


def test_gelu_quick_mul_bit_exact(gpu_ctx, oracle):
    import torch
    from semantica_gpu import kernels
    rng = np.random.default_rng(41)
    gate = (rng.standard_normal((513, 1152)) * 4).astype(np.float32)
    gate[0, :8] = [0.0, -0.0, 10.0, -10.0, 6.0, -6.0, 5.9, -5.9]
    up = rng.standard_normal((513, 1152)).astype(np.float32)
    say("gelu_quick_mul 513x1152")
    out = torch.empty((513, 1152), dtype=torch.float32, device="cuda")
    kernels.gelu_quick_mul(gpu_ctx, out, dev(gate), dev(up))
    got = host(out)
    ref = oracle.gelu_quick(gate) * up
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_elementwise_pins_on_gpu(gpu_ctx):
    """The hand-derived bit-level pins (tests/elementwise_pins.py) through the
    GPU's GELUQuick*up seam (up = 1, so g is GELUQuick's value, fastExp on both
    sigmoid branches) and its RMSNorm seam (n = 768): the GPU gives each pin's
    bits, without the oracle in between."""
    import torch
    import elementwise_pins as ep
    from semantica_gpu import kernels
    gel = [p for p in ep.PINS if p.fn == "gelu"]
    xs = [u for p in gel for u in p.inputs]
    gate = np.zeros((3, 1152), np.float32)
    gate[1, :len(xs)] = np.array(xs, np.uint32).view(np.float32)
    up = np.ones_like(gate)
    say("elementwise pins: gelu")
    out = torch.empty(gate.shape, dtype=torch.float32, device="cuda")
    kernels.gelu_quick_mul(gpu_ctx, out, dev(gate), dev(up))
    got = host(out)[1, :len(xs)].view(np.uint32)
    want = [u for p in gel for u in p.expected]
    assert [int(v) for v in got] == want, [hex(int(v)) for v in got]

    for pin in (p for p in ep.PINS if p.fn == "rmsnorm"):
        x, w = ep.rmsnorm_operands(pin)
        xr = np.zeros((5, ep.RMS_N), np.float32)
        xr[2] = [float(v) for v in x]
        wr = np.array([float(v) for v in w], np.float32)
        say(f"elementwise pins: {pin.name}")
        y = torch.empty_like(dev(xr))
        kernels.rmsnorm(gpu_ctx, y, dev(xr), dev(wr), float(ep.EPS))
        got = host(y)[2, :2].view(np.uint32)
        assert tuple(int(v) for v in got) == pin.expected, (pin.name, [hex(int(v)) for v in got])


def test_gelu_quick_all_floats_bit_exact(gpu_ctx, oracle):
    """GELUQuick on every one of the 2^32 float32 bit patterns (every exponent,
    both signs, subnormals, infinities, NaNs) times up = 1, against the oracle
    bit for bit (any NaN matches any NaN), in 64 chunks of 2^26.  This covers
    fastExp on both sigmoid branches everywhere and pins the short correctly
    rounded division of the sigmoid (Markstein's scheme in sg_div_sigmoid)
    over the whole input range.  The oracle runs on 16 host threads."""
    import ctypes
    from concurrent.futures import ThreadPoolExecutor
    import torch
    from semantica_gpu import kernels
    lib = oracle.load()
    chunk, rows = 1 << 26, 1 << 16
    up = torch.ones((rows, chunk // rows), dtype=torch.float32, device="cuda")
    out = torch.empty_like(up)
    x = np.empty(chunk, np.uint32)
    ref = np.empty(chunk, np.float32)
    nt = 16
    part = chunk // nt
    fp = lambda a: a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))  # noqa: E731
    bad = 0
    with ThreadPoolExecutor(nt) as ex:
        for c in range(1 << 32 >> 26):
            if c % 16 == 0:
                say(f"gelu_quick all floats: chunk {c}/64")
            x[:] = np.arange(c * chunk, (c + 1) * chunk, dtype=np.uint64).astype(np.uint32)
            xf = x.view(np.float32)
            g = dev(xf.reshape(rows, -1))
            kernels.gelu_quick_mul(gpu_ctx, out, g, up)
            list(ex.map(lambda i: lib.sgo_gelu_quick(fp(ref[i * part:]), fp(xf[i * part:]), part), range(nt)))
            got = host(out).reshape(-1)
            same = (got.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(got) & np.isnan(ref))
            if not same.all():
                bad += int((~same).sum())
                say(f"  chunk {c}: {int((~same).sum())} mismatches, e.g. {x[~same][:4]}")
    assert bad == 0


@pytest.mark.parametrize("out_dim", [768, 256, 1])
def test_pool_l2_bit_exact(gpu_ctx, oracle, out_dim):
    import torch
    from semantica_gpu import kernels
    rng = np.random.default_rng(out_dim)
    lens = [1, 9, 512, 77]
    off = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    x = rng.standard_normal((int(off[-1]), 768)).astype(np.float32)
    say(f"pool_l2 out_dim={out_dim}")
    out = torch.empty((len(lens), out_dim), dtype=torch.float32, device="cuda")
    kernels.pool_l2(gpu_ctx, out, dev(x), out_dim, off)
    got = host(out)
    for i in range(len(lens)):
        ref = oracle.mean_pool_l2(x[off[i]:off[i + 1]], out_dim)
        assert np.array_equal(got[i].view(np.uint32), ref.view(np.uint32)), i


def test_issue_probe(gpu_ctx):
    """sg_issue_probe (the GEMM arithmetic's compute floor): every kind returns a
    positive cycle count at a plausible shader clock; the MFMA alone takes about
    its 32-cycle issue interval; the MFMA plus the block-serial update takes at
    least as long as either half."""
    from semantica_gpu import kernels
    got = {}
    for kind in (0, 1, 2):
        cyc, ghz = kernels.issue_probe(gpu_ctx, kind, 4, iters=4000)
        say(f"issue probe kind {kind}: {cyc:.1f} SIMD cycles per subtile-block at {ghz:.2f} GHz")
        assert 0.5 < ghz < 4.0
        got[kind] = cyc
    assert 24.0 < got[2] < 48.0
    assert got[0] >= 0.95 * max(got[1], got[2])
