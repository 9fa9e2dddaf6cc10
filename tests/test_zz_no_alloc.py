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


@pytest.mark.parametrize("sizes", [(8200, 300), (3000, 33)])
def test_noalloc_matches_matmul_two_calls(gpu_ctx, sizes):
    """Two calls in a row, the second with a smaller input (so the shared
    scratch still holds the first call's operand past the second's rows):
    each output equals the allocating entry point's bit for bit.  8200 rows
    take the 4-wave direct-to-LDS kernel and 300 / 3000 / 33 the register-direct one."""
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
