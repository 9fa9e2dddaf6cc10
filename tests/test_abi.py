"""C ABI surface and host-side logic (no GPU calls)."""
import ctypes
import re

import numpy as np
import pytest


def _declared():
    from semantica_gpu import _lib
    src = open(_lib.HEADER_PATH).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(sg_[a-z0-9_]+)\s*\(", src)))


def test_library_exports_every_declared_symbol():
    from semantica_gpu import _lib
    lib = ctypes.CDLL(_lib.LIB_PATH)
    names = _declared()
    assert len(names) >= 19
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # the ctypes prototypes cover exactly the declared functions
    assert _lib.exported_names() == names


def test_abi_version_and_error_string():
    from semantica_gpu import _lib
    lib = _lib.load()
    assert lib.sg_abi_version() == 2
    assert isinstance(lib.sg_last_error(), bytes)


def test_null_arguments_return_codes_without_gpu():
    """Argument checks happen before any device call."""
    from semantica_gpu import _lib
    lib = _lib.load()
    assert lib.sg_model_load(None, None, None) == _lib.SG_ERR_INVALID
    assert lib.sg_forward(None, None, None, 0, 0, None) == _lib.SG_ERR_INVALID
    assert lib.sg_init(0, None) == _lib.SG_ERR_INVALID
    assert b"NULL" in lib.sg_last_error()


def test_resolve_dim():
    """ResolveDim pkg/ggufembed/tasks.go:101-110."""
    from semantica_gpu import resolve_dim, supported_dims
    assert resolve_dim(0) == 512
    for d in (768, 512, 256, 128):
        assert resolve_dim(d) == d
    for d in (1, 64, 300, 1024):
        with pytest.raises(ValueError, match="unsupported embed dim"):
            resolve_dim(d)
    assert supported_dims() == [768, 512, 256, 128]


def test_synthetic_model_format_and_determinism():
    from semantica_gpu import synth
    cfg = dict(synth.EMBEDDINGGEMMA_300M, num_layers=1, vocab_size=64)
    a = synth.make_model(cfg)
    b = synth.make_model(cfg)
    assert a.token_embd.shape == (64, 24, 34)
    assert np.array_equal(a.token_embd, b.token_embd)
    for name, (rows, cols) in a.layer_shapes().items():
        raw = a.layers[0][name]
        assert raw.shape == (rows, cols // 32, 34) and raw.dtype == np.uint8
        d = raw[:, :, 0:2].copy().view("<f2")
        assert np.all(d >= 0) and np.all(np.isfinite(d.astype(np.float32)))
        q = raw[:, :, 2:].view(np.int8)
        assert q.min() >= -127 and q.max() <= 127
    # |N(0, 1e-3)| scales: a few percent land in fp16 subnormals
    d = a.token_embd[:, :, 0:2].copy().view("<f2").astype(np.float32)
    frac_sub = np.mean((d > 0) & (d < 2.0 ** -14))
    assert 0.01 < frac_sub < 0.1
    t = synth.token_ids(1000, 262144)
    assert t.min() >= 2 and t.max() < 262144 and np.array_equal(t, synth.token_ids(1000, 262144))
    ll = synth.lengths_log_uniform(256, 8, 512, seed=1)
    assert ll.min() >= 8 and ll.max() <= 512
