"""Pins the CPU oracle (the checker the GPU library is compared against).

Each check is one of: a known-answer case from the reference's own tests
(file:line cited), an exhaustive or brute-force enumeration, or a property
the mathematics fixes (closed form, invariant, special case).  None of them
re-types the oracle's formula.
"""
import numpy as np
import pytest

from conftest import rel_err


# ---------------------------------------------------------------- fp16 ----

def test_f16_runtime_converter_is_ieee_exhaustive(oracle):
    """model_int8.go:571-597 must equal IEEE fp16->fp32 on all 65536 patterns."""
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ieee = bits.view(np.float16).astype(np.float32)
    got = oracle.f16_table(oracle.F16_RUNTIME)
    nan = np.isnan(ieee)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ieee[~nan].view(np.uint32))


@pytest.mark.parametrize("variant", ["F16_GGUF", "F16_KERNELS"])
def test_f16_halving_converters_differ_only_on_subnormals(oracle, variant):
    """gguf/tensor.go:207-240 and kernels/matmul.go:261-288: exp starts at
    127-15 with no +1, so every subnormal comes out at exactly half."""
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ieee = bits.view(np.float16).astype(np.float32)
    got = oracle.f16_table(getattr(oracle, variant))
    sub = ((bits & 0x7C00) == 0) & ((bits & 0x03FF) != 0)
    nan = np.isnan(ieee)
    assert np.array_equal(got[sub], ieee[sub] * np.float32(0.5))
    ok = ~sub & ~nan
    assert np.array_equal(got[ok].view(np.uint32), ieee[ok].view(np.uint32))
    assert sub.sum() == 2 * 1023


def test_extract_scales_known_values(oracle):
    """TestExtractQ8_0Scales/Basic100Blocks (model_int8_test.go:67-131)."""
    from semantica_gpu.synth import q8_0_from_parts
    vals = np.array([0.01, 1.0, 10.0, -0.5] * 25, np.float32)
    qs = np.tile(np.arange(-16, 16, dtype=np.int8), 100).reshape(1, 100 * 32)
    raw = q8_0_from_parts(vals.astype(np.float16).reshape(1, 100), qs)
    sc = oracle.extract_scales(raw, 1, 100 * 32)[0]
    assert np.max(np.abs(sc - vals)) <= 1e-3
    # whole values are exact in fp16
    assert sc[1] == 1.0 and sc[2] == 10.0 and sc[3] == -0.5


# ------------------------------------------------------------ quantize ----

def test_quantize_all_zero(oracle):
    """quantize.go:50-58: max 0 -> scale 1, all zeros."""
    q, s = oracle.quantize(np.zeros(100, np.float32))
    assert s == 1.0 and not q.any()


def test_quantize_ties_round_half_away_from_zero(oracle):
    """math.Round semantics: with max|x| = 127 the scale is exactly 1, so
    +-2.5 and +-0.5 are exact ties; half-away gives +-3 and +-1 (half-even
    would give +-2 and 0)."""
    x = np.array([127.0, 2.5, -2.5, 0.5, -0.5, 1.49999, -126.5], np.float32)
    q, s = oracle.quantize(x)
    assert s == 1.0
    assert q.tolist() == [127, 3, -3, 1, -1, 1, -127]


def test_quantize_properties_random(oracle):
    rng = np.random.default_rng(11)
    for scale in (1e-3, 1.0, 37.0):
        x = (rng.standard_normal(4099) * scale).astype(np.float32)
        q, s = oracle.quantize(x)
        m = np.max(np.abs(x))
        assert s == np.float32(m / np.float32(127.0))
        i = int(np.argmax(np.abs(x)))
        assert abs(int(q[i])) == 127 and np.sign(q[i]) == np.sign(x[i])
        assert np.all(np.abs(q.astype(np.int32)) <= 127)
        # reconstruction error is at most half a quantum (plus fp32 slack on the scale)
        err = np.abs(x.astype(np.float64) - q.astype(np.float64) * np.float64(s))
        assert np.max(err) <= 0.5 * s * (1 + 1e-5)
        # odd symmetry of round-half-away
        q2, s2 = oracle.quantize(-x)
        assert s2 == s and np.array_equal(q2, -q)


# ----------------------------------------------------------------- GEMM ----

def _rand_q8(rng, rows, cols, scale_lo=0.5, scale_hi=1.0):
    from semantica_gpu.synth import q8_0_from_parts
    d = rng.uniform(scale_lo, scale_hi, size=(rows, cols // 32)).astype(np.float16)
    qs = rng.integers(-127, 128, size=(rows, cols), dtype=np.int8)
    return q8_0_from_parts(d, qs), d.astype(np.float32), qs


def test_block_sums_brute_force(oracle):
    rng = np.random.default_rng(3)
    raw, _, qs = _rand_q8(rng, 40, 96)
    x = rng.integers(-127, 128, size=(7, 96), dtype=np.int8)
    got = oracle.block_sums(raw, x, 40)
    ref = np.einsum("mbk,nbk->mnb", x.reshape(7, 3, 32).astype(np.int64), qs.reshape(40, 3, 32).astype(np.int64))
    assert np.array_equal(got, ref)
    # extreme block: 32 * 127 * 127 and its negation are representable
    from semantica_gpu.synth import q8_0_from_parts
    raw2 = q8_0_from_parts(np.ones((1, 1), np.float16), np.full((1, 32), -127, np.int8))
    x2 = np.full((1, 32), 127, np.int8)
    assert oracle.block_sums(raw2, x2, 1)[0, 0, 0] == -32 * 127 * 127


@pytest.mark.parametrize("order", [0, 1, 2])
def test_matmul_vnni_simple_case(oracle, order):
    """matmul_vnni_test.go:16-34: 32 x (1 * -1) * 1.0 = -32 exactly."""
    from semantica_gpu.synth import q8_0_from_parts
    raw = q8_0_from_parts(np.ones((1, 1), np.float16), np.full((1, 32), -1, np.int8))
    x = np.ones((1, 32), np.int8)
    y = oracle.matmul(raw, x, 1.0, 1, order)
    assert y[0, 0] == -32.0


def test_matmul_orders_vs_float64(oracle):
    """Every accumulation order is within fp32 rounding of the exact value;
    VNNI vs AVX2 within the reference's 1e-3 (matmul_vnni_test.go:36-58)."""
    rng = np.random.default_rng(1234)
    for blocks in range(1, 9):
        K = 32 * blocks
        raw, d, qs = _rand_q8(rng, 64, K)
        x = rng.integers(-127, 128, size=(16, K), dtype=np.int8)
        P = np.einsum("mbk,nbk->mnb", x.reshape(16, blocks, 32).astype(np.int64),
                      qs.reshape(64, blocks, 32).astype(np.int64)).astype(np.float64)
        exact = np.einsum("mnb,nb->mn", P, d.astype(np.float64)) * np.float64(np.float32(0.37))
        ys = [oracle.matmul(raw, x, np.float32(0.37), 64, o) for o in (0, 1, 2)]
        for y in ys:
            assert rel_err(y, exact) < 1e-6
        a, b = ys[0].astype(np.float64), ys[1].astype(np.float64)
        assert np.all(np.abs(a - b) <= 1e-3 * np.maximum(1.0, np.maximum(np.abs(a), np.abs(b))))


def _pin_eval(oracle, pin, order_name):
    from semantica_gpu.synth import q8_0_from_parts
    x, w, d = pin.operands()
    raw = q8_0_from_parts(d, w)
    code = {"vnni": oracle.ORDER_VNNI, "avx2": oracle.ORDER_AVX2, "block_serial": oracle.ORDER_BLOCK_SERIAL,
            "arm64": oracle.ORDER_ARM64}[order_name]
    return float(oracle.matmul(raw, x, np.float32(1.0), 1, code)[0, 0])


@pytest.mark.parametrize("scalar", [False, True])
def test_matmul_orders_pinned_by_hand_vectors(oracle, scalar):
    """Each accumulation order reproduces the hand-derived value of every
    vector in tests/gemm_pins.py (derivations in each vector's docstring),
    with the AVX2 speed-up paths and with the scalar definitions."""
    import gemm_pins
    lib = oracle.load()
    lib.sgo_force_scalar(1 if scalar else 0)
    try:
        for pin in gemm_pins.PINS:
            for o in gemm_pins.ORDERS:
                got = _pin_eval(oracle, pin, o)
                assert got == float(pin.expected[o]), (pin.name, o, got, pin.expected[o])
    finally:
        lib.sgo_force_scalar(0)


def test_matmul_pins_separate_the_orders():
    """For every order there is a vector on which its value differs from all
    three other orders' values, so swapping in another order's lane bytes,
    rounding or accumulator fails a pin."""
    import gemm_pins
    for o in gemm_pins.ORDERS:
        unique = [p.name for p in gemm_pins.PINS
                  if all(p.expected[o] != p.expected[q] for q in gemm_pins.ORDERS if q != o)]
        assert unique, f"no vector tells {o} apart from the other orders"


def test_matmul_pins_catch_single_mistakes():
    """An exact-arithmetic model with the reference's configuration of each
    order reproduces the hand values; changing any one knob (lane bytes,
    hsum tree, fused vs. mul+add) changes at least one pinned value."""
    import gemm_pins
    from gemm_pins import CONFIG, PINS, model
    for o, cfg in CONFIG.items():
        for pin in PINS:
            assert model(pin, *cfg) == pin.expected[o], (o, pin.name)
        lane, tree, fused = cfg
        mutants = [(lm, tree, fused) for lm in gemm_pins.LANE_MAPS if lm != lane]
        mutants.append((lane, tree, not fused))
        if lane != "single":
            mutants += [(lane, t, fused) for t in ("pairs", "seq")]
        for mcfg in mutants:
            caught = [p.name for p in PINS if model(p, *mcfg) != p.expected[o]]
            assert caught, f"{o}: mutation {mcfg} passes every pin"


def test_matmul_threaded_columns_equal_serial(oracle):
    """Column chunks over threads (the reference's matMulQ8_0INT8Tiled tasks)
    give every element the serial bits, in all four orders."""
    lib = oracle.load()
    rng = np.random.default_rng(17)
    raw, _, _ = _rand_q8(rng, 1152, 768, 1e-4, 1e-3)
    x = rng.integers(-127, 128, size=(5, 768), dtype=np.int8)
    for order in (0, 1, 2, 3):
        serial = oracle.matmul(raw, x, np.float32(0.02), 1152, order)
        lib.sgo_set_gemm_threads(7)
        try:
            threaded = oracle.matmul(raw, x, np.float32(0.02), 1152, order)
        finally:
            lib.sgo_set_gemm_threads(1)
        assert np.array_equal(serial.view(np.uint32), threaded.view(np.uint32)), order


def test_matmul_simd_equals_scalar(oracle):
    """The AVX2 speed-up paths must give the scalar definition's bits."""
    lib = oracle.load()
    if not lib.sgo_simd_level():
        pytest.skip("no AVX2+FMA on this host")
    rng = np.random.default_rng(5)
    raw, _, _ = _rand_q8(rng, 96, 768, 1e-4, 1e-3)
    x = rng.integers(-127, 128, size=(9, 768), dtype=np.int8)
    for order in (0, 1, 2, 3):
        fast = oracle.matmul(raw, x, np.float32(0.013), 96, order)
        lib.sgo_force_scalar(1)
        try:
            slow = oracle.matmul(raw, x, np.float32(0.013), 96, order)
        finally:
            lib.sgo_force_scalar(0)
        assert np.array_equal(fast.view(np.uint32), slow.view(np.uint32))


# -------------------------------------------------------------- RMSNorm ----

def test_rmsnorm_known_answer(oracle):
    """TestRMSNorm kernels_test.go:47-64."""
    y = oracle.rmsnorm(np.array([[1, 2, 3, 4]], np.float32), np.ones(4, np.float32), 1e-6)[0]
    ref = np.array([1, 2, 3, 4]) / np.sqrt(7.5)
    assert np.max(np.abs(y - ref)) <= 1e-4


def test_rmsnorm_closed_form(oracle):
    rng = np.random.default_rng(7)
    for n in (256, 768):
        x = rng.standard_normal((13, n)).astype(np.float32) * 3
        w = rng.uniform(0.5, 1.5, n).astype(np.float32)
        y = oracle.rmsnorm(x, w, 1e-6)
        x64 = x.astype(np.float64)
        ref = x64 / np.sqrt(np.mean(x64 * x64, axis=1, keepdims=True) + 1e-6) * w
        assert rel_err(y, ref) < 3e-7
        # RMS(y / w) == 1 up to eps
        r = np.sqrt(np.mean((y / w).astype(np.float64) ** 2, axis=1))
        assert np.all(np.abs(r - 1) < 1e-6)


def test_dot_order_is_eight_lane(oracle):
    """For n >= 8 the reduction is eight FMA lanes (simd_amd64.s:36-46): a
    vector whose lane partial sums are exact shows the hsum grouping: lane 0
    holds 2^24, lane 4 holds 1 and lane 1 holds -2^24, so
    ((l0+l4)+(l1+l5)) = (2^24+1 -> 2^24) - 2^24 = 0, while the serial order
    (2^24 - 2^24) + 1 would be 1."""
    a = np.zeros(8, np.float32)
    a[0], a[4], a[1] = 4096.0, 1.0, 4096.0
    b = np.zeros(8, np.float32)
    b[0], b[4], b[1] = 4096.0, 1.0, -4096.0
    assert oracle.dot(a, b) == 0.0
    # tail elements (n % 8) are added serially after the reduction
    a2 = np.concatenate([a, [1.0]]).astype(np.float32)
    b2 = np.concatenate([b, [1.0]]).astype(np.float32)
    assert oracle.dot(a2, b2) == 1.0


# ------------------------------------------------------- fastExp / GELU ----

def test_fast_exp_bounds_and_accuracy(oracle):
    assert oracle.fast_exp(0.0) == 1.0
    assert oracle.fast_exp(-10.001) == 0.0
    assert oracle.fast_exp(-10.0) > 0.0
    assert oracle.fast_exp(10.5) == np.float32(22026.4657948)
    xs = np.linspace(-10, 10, 20001).astype(np.float32)
    got = np.array([oracle.fast_exp(float(v)) for v in xs], np.float64)
    rel = np.abs(got / np.exp(xs.astype(np.float64)) - 1)
    # "Accurate to ~0.5% for |x| < 5" (activation.go:99); a dropped polynomial
    # term or wrong log2(e) pushes this above 1e-2.
    assert rel.max() < 3e-3


GELU_CASES = {  # TestGELUQuickSIMD kernels_test.go:304-363
    "zeros": [0] * 8, "positive": [0.1, 0.5, 1.0, 2.0, 3.0, 4.0, 5.0, 6.0],
    "negative": [-0.1, -0.5, -1.0, -2.0, -3.0, -4.0, -5.0, -6.0],
    "mixed": [-3.0, -2.0, -1.0, -0.5, 0.0, 0.5, 1.0, 2.0],
    "large_positive": [5.0, 6.0, 7.0, 8.0, 9.0, 10.0, 11.0, 12.0],
    "large_negative": [-5.0, -6.0, -7.0, -8.0, -9.0, -10.0, -11.0, -12.0],
    "small": [0.001, 0.01, 0.1, 0.2, 0.3, 0.4, 0.5, 0.6], "unaligned": [1.0, 2.0, 3.0, 4.0, 5.0]}


@pytest.mark.parametrize("case", sorted(GELU_CASES))
def test_gelu_quick_vs_exact(oracle, case):
    x = np.array(GELU_CASES[case], np.float32)
    got = oracle.gelu_quick(x).astype(np.float64)
    x64 = x.astype(np.float64)
    ref = x64 / (1 + np.exp(-1.702 * x64))
    assert np.max(np.abs(got - ref)) <= 0.01
    assert np.sqrt(np.mean((got - ref) ** 2)) <= 0.005


def test_gelu_quick_properties(oracle):
    """TestGELUQuickSIMDProperties kernels_test.go:365-417."""
    assert abs(oracle.gelu_quick(np.zeros(1, np.float32))[0]) <= 1e-5
    for x in (5.0, 10.0):
        r = oracle.gelu_quick(np.array([x], np.float32))[0] / x
        assert 0.95 <= r <= 1.0
    assert np.all(np.abs(oracle.gelu_quick(np.array([-5.0, -10.0], np.float32))) <= 0.01)
    y = oracle.gelu_quick(np.array([0.0, 0.5, 1.0, 2.0, 3.0, 4.0, 5.0], np.float32))
    assert np.all(np.diff(y) > 0)


# -------------------------------------------------------------- softmax ----

def test_softmax_known(oracle):
    """TestSoftmax kernels_test.go:66-87."""
    y = oracle.softmax(np.array([1, 2, 3, 4], np.float32))
    assert abs(float(np.sum(y, dtype=np.float32)) - 1) <= 1e-5
    assert np.all(np.diff(y) > 0)


def test_softmax_approximation_accuracy(oracle):
    """TestSoftmaxApproximationAccuracy kernels_test.go:89-189 (same sizes,
    trials and value buckets; numpy's RNG in place of Go's)."""
    rng = np.random.default_rng(1234)
    max_abs = max_rel = 0.0
    for n in (1, 2, 3, 4, 8, 16, 32, 64, 128):
        for trial in range(256):
            scale = (1.0, 10.0, 40.0)[trial % 3]
            x = ((rng.random(n) * 2 - 1) * scale).astype(np.float32)
            got = oracle.softmax(x)
            e = np.exp((x - x.max()).astype(np.float64))
            ref = (e.astype(np.float32) * np.float32(1.0 / e.sum())).astype(np.float64)
            diff = np.abs(got - ref)
            max_abs = max(max_abs, diff.max())
            big = np.abs(ref) > 5e-5
            if big.any():
                max_rel = max(max_rel, (diff[big] / np.abs(ref[big])).max())
            assert abs(float(np.sum(got, dtype=np.float32)) - 1) <= 1e-4
    assert max_abs <= 6e-4 and max_rel <= 3e-3


def test_softmax_clamp_gives_exact_zeros(oracle):
    """fastExp returns 0 below -10 (activation.go:104-106): such entries are 0."""
    y = oracle.softmax(np.array([0.0, -10.5, -3.0, -30.0], np.float32))
    assert y[1] == 0.0 and y[3] == 0.0 and y[2] > 0.0


# ----------------------------------------------------------------- RoPE ----

def test_rope_cache_values(oracle):
    fr, c, s = oracle.rope_cache(256, 10000.0, 2048)
    assert fr[0] == 1.0
    i = np.arange(128)
    assert np.allclose(fr, 10000.0 ** (-2.0 * i / 256), rtol=1e-7, atol=0)
    assert np.all(c[0] == 1.0) and np.all(s[0] == 0.0)
    th = (np.float32(1500) * fr).astype(np.float32).astype(np.float64)
    assert np.max(np.abs(c[1500] - np.cos(th))) <= 6e-8
    assert np.max(np.abs(s[1500] - np.sin(th))) <= 6e-8


def test_rope_apply_identity_and_norm(oracle):
    rng = np.random.default_rng(9)
    fr, c, s = oracle.rope_cache(256, 10000.0, 64)
    x = rng.standard_normal((40, 3 * 256)).astype(np.float32)
    y = oracle.rope_apply(x, 3, 256, c, s)
    assert np.array_equal(y[0], x[0])  # p = 0 is the identity
    xp = x.reshape(40, 3, 2, 128).astype(np.float64)
    yp = y.reshape(40, 3, 2, 128).astype(np.float64)
    n_in = np.hypot(xp[:, :, 0], xp[:, :, 1])
    n_out = np.hypot(yp[:, :, 0], yp[:, :, 1])
    assert np.max(np.abs(n_out - n_in) / np.maximum(n_in, 1e-3)) < 1e-6
    # pairs are (i, i+128) (NeoX), rotated by the position's angle
    ang = np.arctan2(yp[5, 0, 1, 7], yp[5, 0, 0, 7]) - np.arctan2(xp[5, 0, 1, 7], xp[5, 0, 0, 7])
    assert abs(np.angle(np.exp(1j * (ang - 5 * fr[7])))) < 1e-5


# ------------------------------------------ elementwise bit-level pins ----

def _bits(a) -> tuple:
    return tuple(int(u) for u in np.asarray(a, np.float32).reshape(-1).view(np.uint32))


def _f32(bits) -> np.ndarray:
    return np.array(bits, np.uint32).view(np.float32)


def pin_eval_oracle(oracle, pin) -> tuple:
    """Runs the oracle function a pin targets on the pin's inputs; returns the
    output bit patterns in the pin's order."""
    import elementwise_pins as ep
    if pin.fn == "fast_exp":
        return tuple(_bits(oracle.fast_exp(float(v)))[0] for v in _f32(pin.inputs))
    if pin.fn == "gelu":
        return _bits(oracle.gelu_quick(_f32(pin.inputs)))
    if pin.fn == "softmax":
        return _bits(oracle.softmax(_f32(pin.inputs)))
    if pin.fn == "rmsnorm":
        x, w = ep.rmsnorm_operands(pin)
        xs = np.array([float(v) for v in x], np.float32)[None]
        ws = np.array([float(v) for v in w], np.float32)
        return _bits(oracle.rmsnorm(xs, ws, float(ep.EPS))[0, :2])
    if pin.fn == "rope":
        n = len(pin.inputs)
        row = np.array([float(p[0]) for p in pin.inputs] + [float(p[1]) for p in pin.inputs], np.float32)[None]
        cos_t = np.array([[float(p[2]) for p in pin.inputs]], np.float32)
        sin_t = np.array([[float(p[3]) for p in pin.inputs]], np.float32)
        return _bits(oracle.rope_apply(row, 1, 2 * n, cos_t, sin_t))
    raise ValueError(pin.fn)


def test_elementwise_literals_are_the_go_float32_constants():
    """The float32 values of the Go constants in activation.go:48,101,121-124,
    :110 and the GGUF default eps, each by two routes: numpy's correctly
    rounded decimal parse and the exact-rational rounding the pins use."""
    import elementwise_pins as ep
    for text, bits in ep.LITERALS.items():
        assert int(np.float32(text).view(np.uint32)) == bits, text
        assert ep.to_bits(ep.r32(ep.F(text))) == bits, text


def test_exact_rounding_helpers_match_ieee():
    """The derivation engine: rational -> float32 rounding equals numpy's
    float64 -> float32 cast (correctly rounded, ties to even) on random
    doubles, subnormal and tie cases included; the rounded sqrt equals
    libm's sqrt in float64 and numpy's in float32."""
    import math
    import elementwise_pins as ep
    rng = np.random.default_rng(77)
    ds = np.concatenate([rng.standard_normal(3000) * 10.0 ** rng.integers(-40, 38, 3000),
                         (rng.integers(1, 1 << 24, 300) * 2 + 1) * 2.0 ** -25,   # float32 ties
                         rng.uniform(0, 2e-38, 200)])                             # subnormals
    for d in ds:
        assert ep.to_bits(ep.r32(ep.F(float(d)))) == int(np.float32(d).view(np.uint32)), d
    for d in np.abs(rng.standard_normal(500)) * 10.0 ** rng.integers(-30, 30, 500):
        assert ep.sqrt_rnd(ep.F(float(d)), 53) == ep.F(math.sqrt(float(d)))
        f = np.float32(d)
        assert ep.sqrt_rnd(ep.F(float(f)), 24) == ep.F(float(np.sqrt(f)))


def test_elementwise_pins_model_rederives_every_value():
    """The exact-rational model of the Go statements reproduces each pin's
    hand-derived bits (the docstrings walk the steps)."""
    import elementwise_pins as ep
    for pin in ep.PINS:
        assert ep.model_eval(pin) == pin.expected, pin.name


@pytest.mark.parametrize("scalar", [False, True], ids=["simd", "scalar"])
def test_elementwise_pins_oracle(oracle, scalar):
    """fastExp, GELUQuick, Softmax, RMSNorm and the RoPE rotation of the oracle
    give every pin's bits, on its AVX2 paths and on its scalar definitions."""
    import elementwise_pins as ep
    lib = oracle.load()
    lib.sgo_force_scalar(1 if scalar else 0)
    try:
        for pin in ep.PINS:
            got = pin_eval_oracle(oracle, pin)
            assert got == pin.expected, (pin.name, [hex(v) for v in got])
    finally:
        lib.sgo_force_scalar(0)


def test_elementwise_pins_catch_single_mistakes():
    """Every plausible restatement mistake changes at least one pinned value:
    fastExp with floor for int32(), the comment's 6-digit coefficients, fused
    or float64 Horner steps, a float64 log2e, `x <= -10` for the clamp;
    GELUQuick with either sigmoid form on both sides or the double 1.702;
    Softmax summed one by one or pairwise, or divided by the sum; RMSNorm as
    x*(inv*w), with 1/sqrt rounded once, or the mean by a reciprocal; any one
    of the four RoPE products fused into its add."""
    import elementwise_pins as ep
    for fn, mutants in ep.MUTANTS.items():
        pins = [p for p in ep.PINS if p.fn == fn]
        assert pins, fn
        for name, knobs in mutants.items():
            caught = [p.name for p in pins if ep.model_eval(p, **knobs) != p.expected]
            assert caught, f"{fn}: mutant {name} passes every pin"


# ------------------------------------------------------------ attention ----

def _attn64(q, k, v, H, HKV, hd):
    S = q.shape[0]
    out = np.zeros((S, H * hd))
    g = H // HKV
    for h in range(H):
        kv = h // g
        qs = q[:, h * hd:(h + 1) * hd].astype(np.float64)
        ks = k[:, kv * hd:(kv + 1) * hd].astype(np.float64)
        vs = v[:, kv * hd:(kv + 1) * hd].astype(np.float64)
        sc = qs @ ks.T / np.sqrt(hd)
        e = np.exp(sc - sc.max(axis=1, keepdims=True))
        out[:, h * hd:(h + 1) * hd] = (e / e.sum(axis=1, keepdims=True)) @ vs
    return out


def test_attention_special_cases(oracle):
    rng = np.random.default_rng(2)
    hd = 256
    # S = 1: the only weight is exactly 1
    q = rng.standard_normal((1, 3 * hd)).astype(np.float32)
    k = rng.standard_normal((1, hd)).astype(np.float32)
    v = rng.standard_normal((1, hd)).astype(np.float32)
    out = oracle.attention(q, k, v, 3, 1, hd)
    assert np.array_equal(out, np.tile(v, (1, 3)))
    # one dominating key (gap > 10 after scaling): the rest get weight exactly 0
    S = 9
    q = np.zeros((S, 3 * hd), np.float32)
    q[:, 0] = 1.0
    k = np.zeros((S, hd), np.float32)
    k[4, 0] = 400.0  # score 400/16 = 25 vs 0
    v = rng.standard_normal((S, hd)).astype(np.float32)
    out = oracle.attention(q, k, v, 3, 1, hd)
    assert np.array_equal(out[:, :hd], np.tile(v[4], (S, 1)))
    # equal scores: uniform weights -> the mean of V
    out = oracle.attention(np.zeros((S, 3 * hd), np.float32), k, v, 3, 1, hd)
    assert np.max(np.abs(out[:, :hd] - v.astype(np.float64).mean(0))) < 1e-5


def test_attention_vs_float64(oracle):
    """fastExp's relative error (< 0.3%) bounds the deviation from exact softmax."""
    rng = np.random.default_rng(4)
    S, hd = 37, 256
    q = rng.standard_normal((S, 3 * hd)).astype(np.float32)
    k = rng.standard_normal((S, hd)).astype(np.float32)
    v = rng.standard_normal((S, hd)).astype(np.float32)
    out = oracle.attention(q, k, v, 3, 1, hd)
    ref = _attn64(q, k, v, 3, 1, hd)
    assert rel_err(out, ref) < 5e-3
    # GQA: head h reads kv head h // (H/HKV) -- head 2 alone matches a 1-head call
    one = oracle.attention(np.ascontiguousarray(q[:, 2 * hd:]), k, v, 1, 1, hd)
    assert np.array_equal(one, out[:, 2 * hd:])


# ------------------------------------------------------------- pool, L2 ----

def test_pool_l2_closed_form(oracle):
    x = np.tile(np.arange(1, 769, dtype=np.float32), (5, 1))
    p = oracle.mean_pool_l2(x, 768, normalize=False)
    assert np.array_equal(p, np.arange(1, 769, dtype=np.float32))
    u = oracle.mean_pool_l2(x, 256)
    ref = np.arange(1, 257) / np.linalg.norm(np.arange(1, 257))
    assert np.max(np.abs(u - ref)) < 1e-6
    assert abs(np.sum(u.astype(np.float64) ** 2) - 1) < 1e-6
    z = oracle.mean_pool_l2(np.zeros((3, 8), np.float32), 8)
    assert not z.any()  # l2Normalize leaves a zero vector unchanged


def test_dequant_row_uses_halving_converter(oracle):
    from semantica_gpu.synth import q8_0_from_parts
    sub = np.array([[np.float16(2.0 ** -20), np.float16(0.5)]], np.float16)  # subnormal, normal
    qs = np.tile(np.arange(-16, 16, dtype=np.int8), 2).reshape(1, 64)
    raw = q8_0_from_parts(sub, qs)
    y = oracle.dequant_row(raw[0].reshape(-1), 64)
    assert np.array_equal(y[:32], qs[0, :32].astype(np.float32) * np.float32(2.0 ** -21))
    assert np.array_equal(y[32:], qs[0, 32:].astype(np.float32) * np.float32(0.5))


# -------------------------------------------------------------- forward ----

def test_forward_errors_and_norm(oracle, tiny_model):
    from semantica_gpu import synth
    m = oracle.OracleModel(tiny_model)
    toks = synth.token_ids(20, tiny_model.config["vocab_size"])
    rc, y = m.forward(toks, 768)
    assert rc == 0 and abs(np.sum(y.astype(np.float64) ** 2) - 1) < 1e-5
    rc2, y2 = m.forward(toks, 768)
    assert np.array_equal(y, y2)
    assert m.forward(np.zeros(0, np.int32), 768)[0] == -1
    assert m.forward(np.full(2049, 5, np.int32), 768)[0] == -2
    assert m.forward(np.array([3, 4096], np.int32), 768)[0] == -3
    assert m.forward(np.array([3, -1], np.int32), 768)[0] == -3
    assert m.forward(toks, 0)[0] == -4 and m.forward(toks, 769)[0] == -4
    # Matryoshka truncation pools the first outDim dims then re-normalizes
    rc, y128 = m.forward(toks, 128)
    assert rc == 0 and abs(np.sum(y128.astype(np.float64) ** 2) - 1) < 1e-5


def test_forward_batch_equals_singles(oracle, tiny_model):
    from semantica_gpu import synth
    m = oracle.OracleModel(tiny_model)
    lens = [5, 17, 1, 33]
    off = synth.offsets_from_lengths(lens)
    toks = synth.token_ids(int(off[-1]), tiny_model.config["vocab_size"], seed=3)
    rc, yb = m.forward_batch(toks, off, 256, n_threads=3)
    assert rc == 0
    for i in range(len(lens)):
        rc, ys = m.forward(toks[off[i]:off[i + 1]], 256)
        assert np.array_equal(ys, yb[i])


def test_forward_taps_teacher_forcing(oracle, tiny_model):
    """The tapped forward equals the plain one; forcing each layer's attention
    output with the oracle's own values changes nothing, bit for bit; forcing
    one perturbed value changes that layer's residual stream and all later
    ones (so the injected values are really the ones used)."""
    from semantica_gpu import synth
    m = oracle.OracleModel(tiny_model)
    lens = [5, 17, 1, 33]
    off = synth.offsets_from_lengths(lens)
    toks = synth.token_ids(int(off[-1]), tiny_model.config["vocab_size"], seed=3)
    L = tiny_model.config["num_layers"]
    for order in (oracle.ORDER_BLOCK_SERIAL, oracle.ORDER_VNNI):
        rc, plain = m.forward_batch(toks, off, 768, order=order, n_threads=2)
        assert rc == 0
        rc, out, taps = m.forward_taps(toks, off, 768, L, qkv=True, att=True, h=True, order=order, n_threads=2)
        assert rc == 0 and np.array_equal(out.view(np.uint32), plain.view(np.uint32))
        for i in range(len(lens)):  # h after the last layer is the stop_layer tap
            rc, hs = m.forward(toks[off[i]:off[i + 1]], 768, order=order, stop_layer=L)
            assert np.array_equal(hs.view(np.uint32), taps["h"][L - 1, off[i]:off[i + 1]].view(np.uint32))
        rc, out2, taps2 = m.forward_taps(toks, off, 768, L, att_in=taps["att"], qkv=True, att=True, h=True,
                                         order=order, n_threads=2)
        assert rc == 0 and np.array_equal(out2.view(np.uint32), out.view(np.uint32))
        for k in ("qkv", "att", "h"):
            assert np.array_equal(taps2[k].view(np.uint32), taps[k].view(np.uint32)), k
    bad = taps["att"].copy()
    bad[0, 20, 100] = np.nextafter(bad[0, 20, 100], np.float32(np.inf)) * np.float32(1.5)
    rc, out3, taps3 = m.forward_taps(toks, off, 768, L, att_in=bad, h=True, order=oracle.ORDER_VNNI, n_threads=2)
    seq = int(np.searchsorted(off, 20, side="right")) - 1
    a, b = off[seq], off[seq + 1]
    assert not np.array_equal(taps3["h"][0, a:b], taps["h"][0, a:b])
    assert not np.array_equal(out3[seq], out[seq])
