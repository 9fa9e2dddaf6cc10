"""GPU brute-force search (k_search.hip, sg_search.cpp) against the CPU
oracle's restatement of search/brute: every score bit-exact, the top-k
identical (ids and distances, ties included), the storage format byte-exact.
"""
import struct
import sys

import numpy as np
import pytest

import oracle as o

pytestmark = pytest.mark.gpu

MODES = [0, 1, 2]  # float32, int8, int16 (brute.QuantizationMode)
MODE_NAMES = {0: "f32", 1: "i8", 2: "i16"}


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _build(ctx, ids, vecs, mode):
    from semantica_gpu import search
    b = search.Builder(ctx, dimension=vecs.shape[1], quantization=mode)
    b.add_vectors(ids, vecs)
    return b.build()


def _oracle(vecs, ids, mode, queries, k, normalized):
    data = o.bf_quantize(o.bf_normalize(vecs), mode)
    out = []
    for q in queries:
        out.append(o.bf_search(data, mode, ids, q if normalized else o.bf_normalize(q), k))
    return data, out


def _check(idx, vecs, ids, mode, queries, k, normalized, tag):
    gi, gd, gn = idx.search_batch(queries, k, normalized=normalized)
    _, want = _oracle(vecs, ids, mode, queries, k, normalized)
    for q, (wi, wd) in enumerate(want):
        assert gn[q] == len(wi), (tag, q)
        assert np.array_equal(gi[q, :gn[q]], wi), (tag, q)
        assert np.array_equal(gd[q, :gn[q]].view(np.uint32), wd.view(np.uint32)), (tag, q)


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("dim", [1, 3, 4, 5, 7, 8, 9, 12, 64, 127, 768])
def test_every_score_bit_exact(gpu_ctx, mode, dim):
    """top_k = count returns every score, in the reference's order: all of
    them must equal the oracle's bit for bit (the 8-lane part, its reduction
    and the scalar tail for every dim % 8)."""
    rng = np.random.default_rng(dim * 3 + mode)
    n, nq = 700, 9  # 9 queries: one block of 8 and one of 1
    vecs = (rng.standard_normal((n, dim)) * rng.uniform(0.1, 10, (n, 1))).astype(np.float32)
    ids = rng.permutation(10 * n)[:n].astype(np.int32) - 3 * n
    queries = rng.standard_normal((nq, dim)).astype(np.float32)
    say(f"scores mode={MODE_NAMES[mode]} dim={dim}")
    idx = _build(gpu_ctx, ids, vecs, mode)
    try:
        _check(idx, vecs, ids, mode, queries, n, False, "all")
    finally:
        idx.close()


@pytest.mark.parametrize("mode", MODES)
def test_top_k_matches_oracle(gpu_ctx, mode):
    rng = np.random.default_rng(40 + mode)
    n, dim = 20000, 256
    vecs = rng.standard_normal((n, dim)).astype(np.float32)
    ids = np.arange(n, dtype=np.int32) * 7 + 1
    queries = rng.standard_normal((21, dim)).astype(np.float32)
    idx = _build(gpu_ctx, ids, vecs, mode)
    try:
        for k in (1, 10, 100, 1000):
            for normalized in (False, True):
                say(f"top-k mode={MODE_NAMES[mode]} k={k} normalized={normalized}")
                q = o.bf_normalize(queries) if normalized else queries
                _check(idx, vecs, ids, mode, q, k, normalized, f"k={k}")
    finally:
        idx.close()


@pytest.mark.parametrize("mode", MODES)
def test_ties_straddling_the_kth_place(gpu_ctx, mode):
    """Every vector stored three times under different ids (shuffled): equal
    scores straddle the k-th place for most k, which the reference resolves
    by its slot order (index.go:84-131).  The GPU must keep the same ids."""
    rng = np.random.default_rng(90 + mode)
    base = rng.standard_normal((500, 48)).astype(np.float32)
    rep = np.repeat(base, 3, axis=0)
    perm = rng.permutation(rep.shape[0])
    vecs = rep[perm]
    ids = (np.arange(vecs.shape[0], dtype=np.int32) * 13) % 100003
    queries = rng.standard_normal((16, 48)).astype(np.float32)
    idx = _build(gpu_ctx, ids, vecs, mode)
    try:
        for k in (1, 2, 3, 4, 5, 10, 31, 64, 65, 100, 1499, 1500):
            say(f"ties mode={MODE_NAMES[mode]} k={k}")
            _check(idx, vecs, ids, mode, queries, k, False, f"k={k}")
    finally:
        idx.close()


def test_zero_scores_of_both_signs_tie(gpu_ctx):
    """Vectors orthogonal to the query score +0 or -0 (a product with a
    negative code is -0); the reference compares them as equal.  k lands
    inside that run of zeros."""
    rng = np.random.default_rng(5)
    dim = 16
    pos = np.abs(rng.standard_normal((40, dim))).astype(np.float32)
    zero = rng.standard_normal((200, dim)).astype(np.float32)
    zero[:, 0] = 0.0
    vecs = np.concatenate([pos, zero])[rng.permutation(240)]
    ids = np.arange(240, dtype=np.int32)[::-1].copy()
    q = np.zeros((2, dim), np.float32)
    q[:, 0] = 1.0
    q[1, 0] = -1.0
    for mode in MODES:
        idx = _build(gpu_ctx, ids, vecs, mode)
        try:
            for k in (39, 40, 41, 60, 239, 240):
                _check(idx, vecs, ids, mode, q, k, False, f"{MODE_NAMES[mode]} k={k}")
        finally:
            idx.close()


def test_reference_known_answer_and_round_trip(gpu_ctx):
    """TestBuilderSearchAndRoundTrip (search/brute/index_test.go:10-36)."""
    from semantica_gpu import search
    b = search.Builder(gpu_ctx, dimension=3, quantization=search.QUANTIZE_INT8)
    for i, v in {10: [1, 0, 0], 11: [0, 1, 0], 12: [0, 0, 1]}.items():
        b.add_vector(i, v)
    idx = b.build()
    res = idx.search_vector([1, 0, 0], 2)
    assert res[0].id == 10 and len(res) == 2
    data = search.Serializer().serialize(idx)
    loaded = search.Serializer().deserialize(gpu_ctx, data)
    assert loaded.dimension() == idx.dimension() == 3
    assert loaded.count() == 3
    for i in (10, 11, 12):
        vec, ok = loaded.vector(i)
        assert ok and len(vec) == 3
    assert loaded.vector(99) == (None, False)
    idx.close()
    loaded.close()


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("dim", [5, 8, 13, 768])
def test_storage_format_byte_exact(gpu_ctx, mode, dim):
    """storage.go:47-91: "BRUT", version 1 (u16), dim (u16), count (u32),
    mode (u8), 7 zero bytes, ids (i32), row-major data -- little-endian.
    Serialize must produce exactly that; Deserialize of it must search like
    the built index; Vector must dequantize as quant.go:43-55 does."""
    from semantica_gpu import search
    rng = np.random.default_rng(dim + 10 * mode)
    n = 300
    vecs = rng.standard_normal((n, dim)).astype(np.float32)
    ids = rng.permutation(5000)[:n].astype(np.int32)
    idx = _build(gpu_ctx, ids, vecs, mode)
    data = o.bf_quantize(o.bf_normalize(vecs), mode)
    want = b"BRUT" + struct.pack("<HHIB7x", 1, dim, n, mode) + ids.tobytes() + data.tobytes()
    got = search.Serializer().serialize(idx)
    assert got == want
    loaded = search.Serializer().deserialize(gpu_ctx, want)
    q = rng.standard_normal((3, dim)).astype(np.float32)
    a, b = idx.search_batch(q, 17), loaded.search_batch(q, 17)
    assert all(np.array_equal(x, y) for x, y in zip(a, b))
    scale = {0: None, 1: np.float32(1 / 127), 2: np.float32(1 / 32767)}[mode]
    for j in (0, n // 2, n - 1):
        vec, ok = loaded.vector(int(ids[j]))
        expect = data[j].astype(np.float32) * scale if scale is not None else data[j]
        assert ok and np.array_equal(vec, expect)
    seen = []
    loaded.for_each(lambda i, v: seen.append((i, v)))
    assert [i for i, _ in seen] == ids.tolist()
    idx.close()
    loaded.close()


def test_deserialize_errors(gpu_ctx):
    """readIndex (storage.go:94-153) error cases and an empty index."""
    from semantica_gpu import SemanticaError, search
    ser = search.Serializer()
    good = b"BRUT" + struct.pack("<HHIB7x", 1, 4, 2, 1) + np.array([1, 2], np.int32).tobytes() + bytes(8)

    def err(data):
        with pytest.raises(SemanticaError) as e:
            ser.deserialize(gpu_ctx, data)
        return str(e.value)

    assert "EOF" in err(b"") and "unexpected" not in err(b"")
    assert "unexpected EOF" in err(good[:10])
    assert 'brute: invalid magic: "BRUX"' in err(b"BRUX" + good[4:])
    assert 'invalid magic: "\\x00AB\\n"' in err(b"\x00AB\n" + good[4:])
    assert "brute: unsupported version 2" in err(good[:4] + struct.pack("<H", 2) + good[6:])
    assert "EOF" in err(good[:20]) and "unexpected" not in err(good[:20])
    assert "unexpected EOF" in err(good[:22])
    assert "unexpected EOF" in err(good[:-1])
    assert "brute: unsupported quantization 3" in err(good[:12] + bytes([3]) + good[13:])
    empty = ser.deserialize(gpu_ctx, b"BRUT" + struct.pack("<HHIB7x", 1, 4, 0, 1))
    assert empty.count() == 0 and empty.search_vector([1, 0, 0, 0], 5) == []
    empty.close()
    idx = ser.deserialize(gpu_ctx, good)
    assert idx.count() == 2 and len(idx.search_vector([1, 0, 0, 0], 5)) == 2
    idx.close()


def test_builder_and_search_errors(gpu_ctx):
    """builder.go:52-80 and index.go:27-51 error cases."""
    from semantica_gpu import SemanticaError, search
    b = search.Builder(gpu_ctx, quantization=search.QUANTIZE_INT16)
    with pytest.raises(SemanticaError, match="brute: no vectors added"):
        b.build()
    b.add_vector(1, [1, 2, 3])
    with pytest.raises(SemanticaError, match="brute: duplicate id 1"):
        b.add_vector(1, [1, 2, 3])
    with pytest.raises(SemanticaError, match="brute: vector dimension mismatch: got 2 want 3"):
        b.add_vector(2, [1, 2])
    idx = b.build()
    with pytest.raises(SemanticaError, match="brute: builder already built"):
        b.build()
    with pytest.raises(SemanticaError, match="brute: topK must be positive"):
        idx.search_vector([1, 0, 0], 0)
    with pytest.raises(SemanticaError, match="brute: query dimension mismatch: got 2 want 3"):
        idx.search_vector([1, 0], 3)
    bad = search.Builder(gpu_ctx, quantization=7)
    bad.add_vector(1, [1, 0])
    with pytest.raises(SemanticaError, match="brute: unsupported quantization 7"):
        bad.build()
    idx.close()


def test_device_build_matches_host_build(gpu_ctx):
    """Index.from_device (vectors already in HBM) stores the same bytes as the
    Builder path."""
    import torch
    from semantica_gpu import search
    rng = np.random.default_rng(77)
    n, dim = 5000, 768
    vecs = rng.standard_normal((n, dim)).astype(np.float32)
    ids = np.arange(n, dtype=np.int32)
    for mode in MODES:
        host = _build(gpu_ctx, ids, vecs, mode)
        padded = torch.zeros((n, dim + 3), dtype=torch.float32, device="cuda")
        padded[:, :dim] = torch.from_numpy(vecs).cuda()
        torch.cuda.synchronize()
        devi = search.Index.from_device(gpu_ctx, ids, padded.data_ptr(), dim, n, mode, ld=dim + 3)
        ser = search.Serializer()
        assert ser.serialize(host) == ser.serialize(devi), mode
        host.close()
        devi.close()


def test_large_index(gpu_ctx):
    """300k x 768 int8 vectors (the embedding width), 40 queries in one call
    (query blocks of 8), top 10: three queries against the oracle in full, and
    every returned distance equal to the oracle's score of the returned id."""
    rng = np.random.default_rng(11)
    n, dim = 300_000, 768
    vecs = rng.standard_normal((n, dim), dtype=np.float32)
    ids = rng.permutation(n).astype(np.int32)
    queries = rng.standard_normal((40, dim), dtype=np.float32)
    say("large index build")
    idx = _build(gpu_ctx, ids, vecs, 1)
    try:
        gi, gd, gn = idx.search_batch(queries, 10)
        assert np.all(gn == 10)
        data = o.bf_quantize(o.bf_normalize(vecs), 1)
        pos = np.empty(n, np.int64)
        pos[ids] = np.arange(n)
        for q in range(40):
            qn = o.bf_normalize(queries[q])
            for j in range(10):
                s = np.float32(o.load().sgo_bf_dot(o._p(data), 1, int(pos[gi[q, j]]), o._p(qn), dim))
                assert s.view(np.uint32) == gd[q, j].view(np.uint32)
            assert np.all(np.diff(gd[q]) <= 0)
        for q in (0, 17, 39):
            say(f"large index oracle query {q}")
            wi, wd = o.bf_search(data, 1, ids, o.bf_normalize(queries[q]), 10)
            assert np.array_equal(gi[q], wi) and np.array_equal(gd[q].view(np.uint32), wd.view(np.uint32))
    finally:
        idx.close()
