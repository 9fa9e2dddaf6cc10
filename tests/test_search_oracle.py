"""Pins of the CPU oracle's brute-force search (oracle/sg_oracle_search.c)
against the reference's own tests (search/brute/index_test.go), closed forms
and hand-derived cases.  CPU only.

The reference's tests draw their vectors from Go's math/rand, which is not
reproduced here: the same tests run on numpy draws of the same shape and
distribution, with the reference's tolerances."""
import numpy as np
import pytest

import oracle as o

MODES = [o.BF_F32, o.BF_I8, o.BF_I16]


def _index(vecs, mode):
    return o.bf_quantize(o.bf_normalize(vecs), mode)


def test_known_answer_builder_search():
    """TestBuilderSearchAndRoundTrip (index_test.go:10-36): ids 10, 11, 12 on
    the unit axes (in either insertion order); query e0 -> id 10 first."""
    vecs = np.eye(3, dtype=np.float32)
    for order in ([0, 1, 2], [2, 0, 1], [1, 2, 0]):
        data = _index(vecs[order], o.BF_I8)
        ids = np.array([10, 11, 12], np.int32)[order]
        got_ids, got_d = o.bf_search(data, o.BF_I8, ids, o.bf_normalize(np.array([1, 0, 0], np.float32)), 2)
        assert got_ids[0] == 10 and len(got_ids) == 2
        assert got_d[0] == np.float32(127) * np.float32(1 / 127)  # code 127 times its scale, times 1.0


@pytest.mark.parametrize("mode,tol", [(o.BF_I8, 0.02), (o.BF_I16, 0.01)])
def test_quantized_dot_matches_float32(mode, tol):
    """TestDotInt8MatchesFloat32 / TestDotInt16MatchesFloat32 (index_test.go:106-156):
    dim 128, 100 normalized N(0,1) pairs, |quantized - float32| <= tol."""
    rng = np.random.default_rng(123)
    for _ in range(100):
        v = o.bf_normalize(rng.standard_normal(128).astype(np.float32))
        q = o.bf_normalize(rng.standard_normal(128).astype(np.float32))
        got = o.bf_scores(o.bf_quantize(v.reshape(1, -1), mode), mode, q)[0]
        want = o.bf_scores(v.reshape(1, -1), o.BF_F32, q)[0]
        assert abs(float(got) - float(want)) <= tol


def test_float32_dot_matches_naive():
    """TestDotFloat32MatchesReference (index_test.go:158-183): within 1e-5 of
    a plain serial float32 sum, dim 256."""
    rng = np.random.default_rng(654)
    for _ in range(50):
        v = o.bf_normalize(rng.standard_normal(256).astype(np.float32))
        q = o.bf_normalize(rng.standard_normal(256).astype(np.float32))
        want = np.float32(0)
        for a, b in zip(v, q):
            want = np.float32(want + np.float32(a * b))
        assert abs(float(o.bf_scores(v.reshape(1, -1), o.BF_F32, q)[0]) - float(want)) <= 1e-5


@pytest.mark.parametrize("mode,tol", [(o.BF_I8, 0.02), (o.BF_I16, 0.01)])
def test_quantized_top1_matches_float32(mode, tol):
    """TestSearchNormalizedMatchesFloat32 (index_test.go:185-251): dim 64,
    256 vectors, top 10, 20 queries; the quantized top-1 distance is within
    0.05 of float32's.  The reference asserts equal top-1 ids on its own Go
    draws; on other draws two candidates closer than the quantization error
    can swap, so the ids must agree whenever float32's top-1/top-2 gap exceeds
    twice the dot tolerance above, and otherwise the quantized top-1 must be
    one of float32's candidates within that band."""
    rng = np.random.default_rng(456)
    vecs = o.bf_normalize(rng.standard_normal((256, 64)).astype(np.float32))
    ids = np.arange(256, dtype=np.int32)
    f = _index(vecs, o.BF_F32)
    qd = _index(vecs, mode)
    for _ in range(20):
        q = o.bf_normalize(rng.standard_normal(64).astype(np.float32))
        fi, fd = o.bf_search(f, o.BF_F32, ids, q, 10)
        qi, qdist = o.bf_search(qd, mode, ids, q, 10)
        assert abs(float(fd[0]) - float(qdist[0])) <= 0.05
        if float(fd[0] - fd[1]) > 2 * tol:
            assert fi[0] == qi[0]
        else:
            assert qi[0] in fi[fd >= fd[0] - 2 * tol]


def test_normalize_and_quantize_closed_forms():
    """builder.go:131-141 and quant.go:17-41 on values with known answers."""
    v = o.bf_normalize(np.array([3, 4], np.float32))
    norm = np.float32(1 / np.sqrt(25.0))  # float32(1/sqrt(float64 sum))
    assert np.array_equal(v, np.array([np.float32(3) * norm, np.float32(4) * norm]))
    z = o.bf_normalize(np.zeros(5, np.float32))  # zero vector stays as is
    assert np.array_equal(z, np.zeros(5, np.float32))
    x = np.array([1.0, -1.0, 2.0, -3.0, 0.5, -0.5, 0.0, 0.25], np.float32)
    # clamp to [-1, 1]; 0.5*127 = 63.5 and 0.25*127 = 31.75: round half away from zero
    assert o.bf_quantize(x, o.BF_I8).tolist() == [127, -127, 127, -127, 64, -64, 0, 32]
    assert o.bf_quantize(x, o.BF_I16).tolist() == [32767, -32767, 32767, -32767, 16384, -16384, 0, 8192]


@pytest.mark.parametrize("dim", [1, 3, 4, 5, 7, 8, 9, 12, 15, 16, 21, 64])
def test_float32_dot_exact_on_small_integers(dim):
    """With small integer values every float32 product and partial sum is
    exact, so any summation order gives the integer dot product: pins the
    element indexing of the 8-lane part and of the tail."""
    rng = np.random.default_rng(dim)
    a = rng.integers(-9, 10, (20, dim)).astype(np.float32)
    q = rng.integers(-9, 10, dim).astype(np.float32)
    want = (a.astype(np.int64) @ q.astype(np.int64)).astype(np.float32)
    assert np.array_equal(o.bf_scores(a, o.BF_F32, q), want)


@pytest.mark.parametrize("mode", [o.BF_I8, o.BF_I16])
@pytest.mark.parametrize("dim", [1, 3, 4, 5, 7, 8, 9, 12, 15, 16, 21, 64, 768])
def test_quantized_dot_within_rounding_bound(mode, dim):
    """Against the float64 value sum(code * inv * x): the float32 error of a
    dim-term sum of rounded products is at most ~(dim + 2) * 2^-24 * sum|terms|;
    a dropped or misindexed term is far outside that."""
    rng = np.random.default_rng(100 + dim)
    codes = rng.integers(-127 if mode == o.BF_I8 else -32767, 128 if mode == o.BF_I8 else 32768, (30, dim))
    data = codes.astype(np.int8 if mode == o.BF_I8 else np.int16)
    q = rng.standard_normal(dim).astype(np.float32)
    inv = np.float64(np.float32(1 / 127) if mode == o.BF_I8 else np.float32(1 / 32767))
    terms = codes.astype(np.float64) * inv * q.astype(np.float64)
    want = terms.sum(axis=1)
    bound = (dim + 3) * 2.0 ** -24 * np.abs(terms).sum(axis=1) + 1e-30
    got = o.bf_scores(data, mode, q).astype(np.float64)
    assert np.all(np.abs(got - want) <= bound)


def test_most_negative_code_in_tail_is_clamped():
    """The scalar tail goes through int8ToFloat32 (quant.go:57-68), which maps
    -128 to -127; the AVX2 part (dot_amd64.s) does not clamp."""
    q = np.ones(9, np.float32)
    data = np.full((1, 9), -128, np.int8)
    inv = np.float32(1 / 127)
    got = o.bf_scores(data, o.BF_I8, q)[0]
    eight = np.float32(8) * np.float32(np.float32(-128) * inv)  # 8 equal lanes: every partial sum exact
    assert got == np.float32(eight + np.float32(np.float32(-127) * inv))
    assert got != np.float32(eight + np.float32(np.float32(-128) * inv))


def _tie_index():
    # scores against e0 by construction: a = b = 0.5 (the same vector), c = 0.7
    a = np.array([0.5, np.sqrt(0.75)], np.float32)
    c = np.array([0.7, np.sqrt(0.51)], np.float32)
    return a, c


def test_streaming_tie_rule_hand_derived():
    """index.go:84-131 by hand.  Stored a, b, c with a == b < c and k = 2:
    [a, b] fill the list, c replaces the FIRST slot holding the minimum (a), so
    the result is {c, b}.  Stored c, a, b: [c, a] fill it, b is not strictly
    larger than the minimum and is skipped, so the result is {c, a}."""
    a, c = _tie_index()
    q = np.array([1, 0], np.float32)
    data = _index(np.stack([a, a, c]), o.BF_F32)
    ids, _ = o.bf_search(data, o.BF_F32, np.array([100, 101, 102], np.int32), q, 2)
    assert ids.tolist() == [102, 101]
    data = _index(np.stack([c, a, a]), o.BF_F32)
    ids, _ = o.bf_search(data, o.BF_F32, np.array([102, 100, 101], np.int32), q, 2)
    assert ids.tolist() == [102, 100]


def test_result_order_ties_by_id():
    """index.go:133-137: equal distances are ordered by id ascending."""
    a, _ = _tie_index()
    data = _index(np.stack([a, a, a]), o.BF_I8)
    ids, d = o.bf_search(data, o.BF_I8, np.array([7, 3, 5], np.int32), np.array([1, 0], np.float32), 3)
    assert ids.tolist() == [3, 5, 7] and d[0] == d[1] == d[2]


def test_top_k_edge_cases():
    """index.go:29-31,55-61: top_k <= 0 is an error, top_k > count is clipped."""
    data = _index(np.eye(4, dtype=np.float32), o.BF_I8)
    ids = np.arange(4, dtype=np.int32)
    q = np.array([1, 0, 0, 0], np.float32)
    assert o.bf_search(data, o.BF_I8, ids, q, 0) is None
    got, _ = o.bf_search(data, o.BF_I8, ids, q, 10)
    assert len(got) == 4 and got[0] == 0
