"""Plants single mistakes in a temporary copy of the oracle's C source and
checks that the bit-level pins (tests/elementwise_pins.py) reject each build.

The mutations are the restatement mistakes the pins are meant to catch:
fastExp with floor() for the int32 conversion (activation.go:115) or the
comment's 6-digit coefficients (:117 vs :121-124), GELUQuick's positive
sigmoid form on both sides (:64-72), Softmax's sum accumulated one by one
(:192), a division by the sum (:209-212), RMSNorm folding the weight into
the reciprocal (norm.go:26-28) or rounding 1/sqrt once (:21-22), and a fused
RoPE rotation (rope_cache.go:102-103).  The unmodified source must pass, so
a mutation that stops matching the source text fails the test instead of
silently passing.
"""
import ctypes
import os
import shutil
import subprocess

import numpy as np
import pytest

import elementwise_pins as ep

ORACLE_DIR = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle")

MUTATIONS = {
    "fast_exp_floor": ("int32_t ip = (int32_t)y;", "int32_t ip = (int32_t)floorf(y);"),
    "fast_exp_6digit": ("const float c1 = 0.693147180559945f, c2 = 0.240226506959101f;\n"
                        "  const float c3 = 0.055504108664821f, c4 = 0.009676036358193f;",
                        "const float c1 = 0.693147f, c2 = 0.240227f;\n"
                        "  const float c3 = 0.055504f, c4 = 0.009676f;"),
    "gelu_one_branch": ("if (sx >= 0.0f) {", "if (1) {"),
    "softmax_serial_sum": ("sum = sum + (((e0 + e1) + e2) + e3);", "sum = (((sum + e0) + e1) + e2) + e3;"),
    "softmax_divide": ("dst[k] = dst[k] * inv;", "dst[k] = dst[k] / sum;"),
    "rmsnorm_fold_w": ("float t = src[i] * inv;\n    dst[i] = t * w[i];", "dst[i] = src[i] * (inv * w[i]);"),
    "rmsnorm_rsqrt_once": ("float rms = (float)sqrt((double)(ms + eps));\n  float inv = 1.0f / rms;",
                           "float inv = (float)(1.0 / sqrt((double)(ms + eps)));"),
    "rope_fused": ("v[i] = a - b;", "v[i] = fmaf(v0, c[i], -b);"),
}


class _Lib:
    """The pin-relevant oracle entry points of one build (ctypes)."""

    def __init__(self, path):
        L = ctypes.CDLL(path)
        fp = ctypes.POINTER(ctypes.c_float)
        L.sgo_fast_exp.restype = ctypes.c_float
        L.sgo_fast_exp.argtypes = [ctypes.c_float]
        L.sgo_gelu_quick.argtypes = [fp, fp, ctypes.c_int64]
        L.sgo_softmax.argtypes = [fp, fp, ctypes.c_int]
        L.sgo_rmsnorm.argtypes = [fp, fp, fp, ctypes.c_int, ctypes.c_float]
        L.sgo_rope_apply.argtypes = [fp, ctypes.c_int, ctypes.c_int, ctypes.c_int, fp, fp]
        self.L = L

    @staticmethod
    def _p(a):
        return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))

    def eval(self, pin):
        f32 = lambda b: np.array(b, np.uint32).view(np.float32)  # noqa: E731
        bits = lambda a: tuple(int(u) for u in np.asarray(a, np.float32).reshape(-1).view(np.uint32))  # noqa: E731
        if pin.fn == "fast_exp":
            return bits([self.L.sgo_fast_exp(float(v)) for v in f32(pin.inputs)])
        if pin.fn in ("gelu", "softmax"):
            x = f32(pin.inputs).copy()
            y = np.empty_like(x)
            if pin.fn == "gelu":
                self.L.sgo_gelu_quick(self._p(y), self._p(x), x.size)
            else:
                self.L.sgo_softmax(self._p(y), self._p(x), x.size)
            return bits(y)
        if pin.fn == "rmsnorm":
            x, w = ep.rmsnorm_operands(pin)
            xs = np.array([float(v) for v in x], np.float32)
            ws = np.array([float(v) for v in w], np.float32)
            y = np.empty_like(xs)
            self.L.sgo_rmsnorm(self._p(y), self._p(xs), self._p(ws), xs.size, float(ep.EPS))
            return bits(y[:2])
        if pin.fn == "rope":
            n = len(pin.inputs)
            row = np.array([float(p[0]) for p in pin.inputs] + [float(p[1]) for p in pin.inputs], np.float32)
            c = np.array([float(p[2]) for p in pin.inputs], np.float32)
            s = np.array([float(p[3]) for p in pin.inputs], np.float32)
            self.L.sgo_rope_apply(self._p(row), 1, 1, 2 * n, self._p(c), self._p(s))
            return bits(row)
        raise ValueError(pin.fn)


def _build(tmp, name, src_text):
    d = tmp / name
    d.mkdir()
    for f in ("sg_oracle.h", "sg_oracle_search.c"):
        shutil.copy(os.path.join(ORACLE_DIR, f), d / f)
    (d / "sg_oracle.c").write_text(src_text)
    so = d / "lib.so"
    # the flags of oracle/Makefile
    subprocess.run(["gcc", "-O2", "-fPIC", "-std=gnu11", "-ffp-contract=off", "-fno-fast-math", "-shared",
                    "-o", str(so), str(d / "sg_oracle.c"), str(d / "sg_oracle_search.c"), "-lm", "-lpthread"],
                   check=True, capture_output=True)
    return _Lib(str(so))


@pytest.fixture(scope="module")
def oracle_src():
    if shutil.which("gcc") is None:
        pytest.skip("no gcc")
    with open(os.path.join(ORACLE_DIR, "sg_oracle.c")) as f:
        return f.read()


def test_unmodified_copy_passes_the_pins(oracle_src, tmp_path):
    lib = _build(tmp_path, "clean", oracle_src)
    for pin in ep.PINS:
        assert lib.eval(pin) == pin.expected, pin.name


@pytest.mark.parametrize("name", sorted(MUTATIONS))
def test_planted_mistake_fails_a_pin(oracle_src, tmp_path, name):
    old, new = MUTATIONS[name]
    assert oracle_src.count(old) == 1, f"mutation {name} no longer matches the oracle source"
    lib = _build(tmp_path, name, oracle_src.replace(old, new))
    failed = [p.name for p in ep.PINS if lib.eval(p) != p.expected]
    assert failed, f"{name}: every pin still passes"
