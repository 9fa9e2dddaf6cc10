"""sg_matmul_q8_0_int8_noalloc (the GEMM seam without device allocation)
against sg_matmul_q8_0_int8, through the C ABI."""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _run(ctx, fn, w, xq, rs, N, check_free=False):
    """One call of fn; with check_free, the device's free memory must be the
    same before and after (every buffer is allocated before the first read)."""
    import torch
    y = torch.full((xq.shape[0], N), float("nan"), dtype=torch.float32, device="cuda")
    x, r = torch.from_numpy(xq).cuda(), torch.from_numpy(rs).cuda()
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    fn(ctx, y, w, x, r)
    torch.cuda.synchronize()
    if check_free:
        assert torch.cuda.mem_get_info()[0] == free0
    return y.cpu().numpy()


@pytest.mark.parametrize("sizes", [(12300, 8200), (8200, 300), (3000, 33)])
def test_noalloc_matches_matmul_two_calls(gpu_ctx, sizes):
    """Two calls in a row, the second with a smaller input (so the shared
    scratch still holds the first call's operand past the second's rows):
    each output equals the allocating entry point's bit for bit.  12300 rows
    take the 8-wave direct-to-LDS kernel, 8200 the 4-wave one and 300 / 3000 /
    33 the register-direct one."""
    from semantica_gpu import kernels, synth
    N, K = 1152, 768
    rng = np.random.default_rng(sizes[0])
    raw = synth.q8_0_random(rng, N, K)
    w = kernels.Q8Weight(gpu_ctx, raw, N, K)
    try:
        for M in sizes:
            say(f"noalloc gemm M={M} N={N} K={K}")
            xq = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
            rs = rng.uniform(1e-3, 2e-2, M).astype(np.float32)
            want = _run(gpu_ctx, kernels.matmul_q8_0, w, xq, rs, N)
            got = _run(gpu_ctx, kernels.matmul_q8_0_noalloc, w, xq, rs, N, check_free=True)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), M
    finally:
        w.close()


def test_noalloc_rejects_inputs_beyond_the_scratch(gpu_ctx):
    """An input whose operand would not fit the fixed scratch is refused with
    SG_ERR_INVALID before anything is launched (the output is untouched)."""
    import torch
    from semantica_gpu import SemanticaError, _lib, kernels, synth
    N, K = 256, 4096
    raw = synth.q8_0_random(np.random.default_rng(1), N, K)
    w = kernels.Q8Weight(gpu_ctx, raw, N, K)
    try:
        M = 16640  # 16640 rows x 4096 bytes = 65 MiB of int8 operand > 64 MiB
        say(f"noalloc gemm over the limit M={M} K={K}")
        x = torch.zeros((M, K), dtype=torch.int8, device="cuda")
        rs = torch.ones(M, dtype=torch.float32, device="cuda")
        y = torch.full((M, N), 7.0, dtype=torch.float32, device="cuda")
        with pytest.raises(SemanticaError) as ei:
            kernels.matmul_q8_0_noalloc(gpu_ctx, y, w, x, rs)
        assert ei.value.code == _lib.SG_ERR_INVALID and "limit" in ei.value.message
        torch.cuda.synchronize()
        assert bool(torch.all(y == 7.0))
    finally:
        w.close()


def test_noalloc_under_graph_capture(gpu_ctx):
    """The no-alloc call captured in a HIP graph (torch.cuda.graph: capture
    on torch's side stream, kernel launches only, no allocation) and replayed
    three times, with new activations copied into the captured input between
    replays and eager work and synchronizations in between: every replay
    equals the allocating entry point on the same input bit for bit.  The
    caller's current device is the same after each call."""
    import torch
    from semantica_gpu import kernels, synth
    N, K, M = 768, 768, 2100
    rng = np.random.default_rng(12)
    w = kernels.Q8Weight(gpu_ctx, synth.q8_0_random(rng, N, K), N, K)
    try:
        x = torch.zeros((M, K), dtype=torch.int8, device="cuda")
        rs = torch.zeros(M, dtype=torch.float32, device="cuda")
        y = torch.zeros((M, N), dtype=torch.float32, device="cuda")
        dev0 = torch.cuda.current_device()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):  # warm once outside the capture
            kernels.matmul_q8_0_noalloc(gpu_ctx, y, w, x, rs, stream=side.cuda_stream)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        say(f"noalloc gemm under graph capture M={M} N={N} K={K}")
        with torch.cuda.graph(g):
            kernels.matmul_q8_0_noalloc(gpu_ctx, y, w, x, rs, stream=torch.cuda.current_stream().cuda_stream)
        assert torch.cuda.current_device() == dev0
        for rep in range(3):
            xq = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
            r = rng.uniform(1e-3, 2e-2, M).astype(np.float32)
            x.copy_(torch.from_numpy(xq))
            rs.copy_(torch.from_numpy(r))
            y.fill_(float("nan"))
            torch.cuda.synchronize()
            say(f"  replay {rep}")
            g.replay()
            torch.cuda.synchronize()
            got = y.cpu().numpy()
            want = _run(gpu_ctx, kernels.matmul_q8_0, w, xq, r, N)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), rep
        del g
    finally:
        w.close()
