"""Shared test setup.

CPU tests (`-m "not gpu"`) pin the oracle against the reference's known
answers and mathematical invariants, and check the host logic and the C ABI
surface.  GPU tests (`-m gpu`) compare the HIP library, called through its C
ABI, with the oracle on identical inputs.
"""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "oracle"), os.path.join(ROOT, "go-semantica_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")


@pytest.fixture(scope="session")
def oracle():
    import oracle as o
    o.load()
    return o


# A 2-layer EmbeddingGemma (real widths, small vocabulary) that the oracle
# runs in well under a second per sequence.
TINY = dict(embed_dim=768, num_layers=2, num_heads=3, num_kv_heads=1, interm_dim=1152,
            max_seq_len=2048, vocab_size=4096, norm_eps=1e-6, rope_base=10000.0)


@pytest.fixture(scope="session")
def tiny_model():
    from semantica_gpu import synth
    return synth.make_model(TINY)


@pytest.fixture(scope="session")
def gpu_ctx():
    import torch  # noqa: F401  (initializes HIP device memory plumbing for tests)
    from semantica_gpu import Context
    ctx = Context(0)
    yield ctx
    ctx.close()


def rel_err(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))
