"""End-to-end parity of the batched GPU forward with the oracle's
forwardINT8WithDim restatement, plus size-independent properties at the
benchmark's full size.

Tolerance (from the north star): max |gpu - ref| <= 1e-3 and cosine >= 0.9999
per embedding.  The GEMMs, norms, RoPE, GELU, quantization and pooling follow
the reference op for op; attention runs on fp16 matrix cores, so the
embeddings are close, not bit-identical.
"""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

MAX_ABS = 1e-3
MIN_COS = 0.9999


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _check(got, ref, tag=""):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape
    for i in range(got.shape[0]):
        cos = float(got[i] @ ref[i] / (np.linalg.norm(got[i]) * np.linalg.norm(ref[i])))
        mad = float(np.max(np.abs(got[i] - ref[i])))
        assert mad <= MAX_ABS and cos >= MIN_COS, f"{tag} seq {i}: max-abs {mad:.3e} cos {cos:.7f}"


@pytest.fixture(scope="module")
def tiny_gpu(gpu_ctx, tiny_model):
    from semantica_gpu import Model
    m = Model(gpu_ctx, tiny_model)
    yield m
    m.close()


@pytest.fixture(scope="module")
def full_model():
    from semantica_gpu import synth
    return synth.make_model()


@pytest.fixture(scope="module")
def full_gpu(gpu_ctx, full_model):
    from semantica_gpu import Model
    m = Model(gpu_ctx, full_model)
    yield m
    m.close()


def test_tiny_forward_vs_oracle(tiny_gpu, tiny_model, oracle):
    from semantica_gpu import synth
    lens = [1, 7, 32, 33, 128, 300]
    off = synth.offsets_from_lengths(lens)
    toks = synth.token_ids(int(off[-1]), tiny_model.config["vocab_size"], seed=7)
    say(f"tiny forward lens={lens}")
    for dim in (768, 256):
        got = tiny_gpu.forward_packed(toks, off, dim)
        rc, ref = oracle.OracleModel(tiny_model).forward_batch(toks, off, dim, n_threads=8)
        assert rc == 0
        _check(got, ref, f"tiny dim={dim}")


def test_forward_errors(tiny_gpu):
    from semantica_gpu import SemanticaError, _lib
    say("forward error cases")
    cases = [
        (lambda: tiny_gpu.forward_batch([[3, 4], []], 768), _lib.SG_ERR_EMPTY, "empty input"),
        (lambda: tiny_gpu.forward_batch([[5] * 2049], 768), _lib.SG_ERR_TOO_LONG, "sequence too long: 2049 > 2048"),
        (lambda: tiny_gpu.forward_batch([[3, 4], [9, 4096, 2]], 768), _lib.SG_ERR_TOKEN,
         "token ID out of range: 4096"),
        (lambda: tiny_gpu.forward_batch([[3, 4]], 0), _lib.SG_ERR_DIM, "target dimension 0 out of range (1..768)"),
        (lambda: tiny_gpu.forward_batch([[3, 4]], 769), _lib.SG_ERR_DIM, "target dimension 769"),
    ]
    for fn, code, msg in cases:
        with pytest.raises(SemanticaError) as ei:
            fn()
        assert ei.value.code == code and msg in ei.value.message
    # the model still works after errors
    assert tiny_gpu.forward_batch([[3, 4, 5]], 768).shape == (1, 768)


def test_device_path_reports_bad_token(tiny_gpu):
    import torch
    from semantica_gpu import SemanticaError, _lib
    say("device-path token validation")
    toks = torch.tensor([3, 4, 99999], dtype=torch.int32, device="cuda")
    out = torch.empty((1, 768), dtype=torch.float32, device="cuda")
    with pytest.raises(SemanticaError) as ei:
        tiny_gpu.forward_device(toks.data_ptr(), np.array([0, 3], np.int32), 768, out.data_ptr())
    assert ei.value.code == _lib.SG_ERR_TOKEN


def test_config0_full_model_vs_oracle(full_gpu, full_model, oracle):
    """Config 0: 1 x 32 tokens, seed 0, all 24 layers."""
    from semantica_gpu import synth
    toks = synth.token_ids(32, 262144, seed=0)
    say("config0 1x32 full model")
    got = full_gpu.forward_batch([toks], 768)
    rc, ref = oracle.OracleModel(full_model).forward(toks, 768)
    assert rc == 0
    _check(got, ref[None], "c0")


def test_config4_ragged_matryoshka_vs_oracle(full_gpu, full_model, oracle):
    """Config 4 shape (log-uniform lengths in [8, 512], seed 1, 256 dims) on a
    16-sequence slice, compared per row."""
    from semantica_gpu import synth
    lens = synth.lengths_log_uniform(256, 8, 512, seed=1)[:16]
    off = synth.offsets_from_lengths(lens)
    toks = synth.token_ids(int(off[-1]), 262144, seed=1)
    say(f"config4 slice lens={lens.tolist()}")
    got = full_gpu.forward_packed(toks, off, 256)
    rc, ref = oracle.OracleModel(full_model).forward_batch(toks, off, 256, n_threads=16)
    assert rc == 0
    _check(got, ref, "c4")


def test_long_sequence_vs_oracle(gpu_ctx, oracle):
    """Config 3's attention-heavy length range on a 2-layer model."""
    from semantica_gpu import Model, synth
    cfg = dict(synth.EMBEDDINGGEMMA_300M, num_layers=2, vocab_size=8192)
    mdl = synth.make_model(cfg, seed_weights=9)
    lens = [1500, 2048]
    off = synth.offsets_from_lengths(lens)
    toks = synth.token_ids(int(off[-1]), 8192, seed=4)
    say(f"long sequences {lens}")
    m = Model(gpu_ctx, mdl)
    try:
        got = m.forward_packed(toks, off, 768)
    finally:
        m.close()
    rc, ref = oracle.OracleModel(mdl).forward_batch(toks, off, 768, n_threads=2)
    assert rc == 0
    _check(got, ref, "long")


def test_config2_full_size_properties(full_gpu):
    """Config 2 (64 x 512): unit norm, and every sequence's embedding is
    independent of its batch neighbours (bit-identical alone and packed)."""
    from semantica_gpu import synth
    toks = synth.token_ids(64 * 512, 262144, seed=0)
    off = np.arange(0, 64 * 512 + 1, 512, dtype=np.int32)
    say("config2 64x512 properties")
    y = full_gpu.forward_packed(toks, off, 768)
    assert np.all(np.isfinite(y))
    assert np.max(np.abs(np.sum(y.astype(np.float64) ** 2, axis=1) - 1)) < 1e-5
    for i in (0, 17, 63):
        alone = full_gpu.forward_packed(toks[512 * i:512 * (i + 1)], np.array([0, 512], np.int32), 768)[0]
        assert np.array_equal(alone.view(np.uint32), y[i].view(np.uint32)), i
    # permuting the batch permutes the output
    perm = np.array([5, 0, 63, 12], np.int64)
    toks_p = np.concatenate([toks[512 * i:512 * (i + 1)] for i in perm])
    yp = full_gpu.forward_packed(toks_p, np.arange(0, 4 * 512 + 1, 512, dtype=np.int32), 768)
    assert np.array_equal(yp.view(np.uint32), y[perm].view(np.uint32))
