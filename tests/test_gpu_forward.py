"""End-to-end parity of the batched GPU forward with the oracle's restatement
of forwardINT8WithDim (runtime/model_int8.go:148-256).

Parity is proven in two parts.  Teacher forcing (_teacher_forced) shows
every kernel except attention's two products bit-exact at full depth, and
attention within 1e-5 at every layer.  End to end, against the path the
reference takes on the GPU box's host (AVX-512 VNNI), north_star's
1e-3 / 0.9999 bar is reported per case, and the envelope below is asserted.

Why the end-to-end criterion is an envelope and not a fixed 1e-3 / 0.9999:
every layer re-quantizes four activations to int8 with a per-sequence scale
(model_int8.go:197,219,503,533), so a last-bit difference anywhere upstream
flips an int8 code by a whole quantum once in a while, and the flips compound
over 24 layers.  The reference itself shows this: its own GEMM paths (AVX-512
VNNI vs AVX2 on amd64, simd_amd64.s:164-304, and arm64 SDOT,
simd_arm64_matmul.s:6-56) differ only in fp32 summation order, yet their
embeddings for the same input differ by up to ~6e-3 max-abs (cosine down to
~0.9997) on the synthetic model.  The GPU is therefore held to:
  * the layer taps: the embedding layer bit-exact; the residual stream after
    one layer within 1e-5 of the oracle (observed ~1e-7: no int8 code has
    flipped yet); after two layers most sequences still within 1e-5 (a first
    flip shows up as ~1e-3 on its sequence);
  * the final embeddings: deviation from the oracle's VNNI path no larger than
    the reference's own cross-path spread (AVX2, arm64 and block-FMA orders vs
    VNNI), with a factor of 2 on max-abs and 3 on (1 - cosine) for the
    randomness of where the first flip lands, and cosine >= 0.999 always.
"""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

REF_ORDERS = {"avx2": 1, "block_fma": 2, "arm64": 3}
# north_star's end-to-end bar.  It is reported per case against the path the
# reference takes on an AVX-512-VNNI host; the reference's own other paths
# are reported against it too.  What is asserted at that depth is the
# envelope below, and, under teacher forcing, bit-identity of every kernel
# except attention (_teacher_forced).
NORTH_STAR_MAX_ABS, NORTH_STAR_COS = 1e-3, 0.9999


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _stats(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    mad = np.max(np.abs(a - b), axis=1)
    cos = np.sum(a * b, 1) / (np.linalg.norm(a, axis=1) * np.linalg.norm(b, axis=1))
    return mad, 1.0 - cos


def _check_envelope(got, oracle_model, toks, off, dim, tag, threads=16):
    refs = {}
    for name, order in [("vnni", 0)] + list(REF_ORDERS.items()):
        rc, refs[name] = oracle_model.forward_batch(toks, off, dim, order=order, n_threads=threads)
        assert rc == 0
    g_mad, g_dc = _stats(got, refs["vnni"])
    env = [_stats(refs[n], refs["vnni"]) for n in REF_ORDERS]
    e_mad = np.max([e[0] for e in env], axis=0)
    e_dc = np.max([e[1] for e in env], axis=0)
    say(f"{tag}: gpu-vs-vnni max-abs max {g_mad.max():.2e} mean {g_mad.mean():.2e} 1-cos max {g_dc.max():.2e} "
        f"mean {g_dc.mean():.2e} | reference spread max-abs max {e_mad.max():.2e} mean {e_mad.mean():.2e} "
        f"1-cos max {e_dc.max():.2e} mean {e_dc.mean():.2e}")

    def verdict(mad, dc):
        ok = mad.max() <= NORTH_STAR_MAX_ABS and dc.max() <= 1.0 - NORTH_STAR_COS
        return "met" if ok else "NOT met"
    say(f"{tag}: north_star bar (max-abs <= {NORTH_STAR_MAX_ABS:g}, cos >= {NORTH_STAR_COS}) against the VNNI path: "
        f"GPU {verdict(g_mad, g_dc)}; the reference's own AVX2 / block-FMA / arm64 paths: "
        + ", ".join(f"{n} {verdict(*e)}" for n, e in zip(REF_ORDERS, env)))
    # Against the path the GPU reproduces (the block-serial fallback order,
    # matmul_inner_loop_fallback.go:16-43, through model_int8.go:148-256):
    # every kernel but attention's two products is bit-exact to it
    # (_teacher_forced), so what is left is attention's fp32-class rounding
    # (<= 1e-5 relative per layer) carried through the int8 re-quantizations.
    b_mad, b_dc = _stats(got, refs["block_fma"])
    say(f"{tag}: gpu-vs-block-serial max-abs max {b_mad.max():.2e} mean {b_mad.mean():.2e} "
        f"1-cos max {b_dc.max():.2e} mean {b_dc.mean():.2e}; north_star bar against the block-serial path: "
        f"GPU {verdict(b_mad, b_dc)}")
    assert b_mad.max() <= 2.0 * e_mad.max() + 1e-4
    assert b_mad.mean() <= 2.0 * e_mad.mean() + 1e-4
    assert b_dc.max() <= 4.0 * e_dc.max() + 1e-6
    assert b_dc.max() <= 1e-3
    # The spread comes from int8 re-quantization flips, whose number per
    # sequence is random; a systematic error would sit far above these bounds.
    assert g_mad.max() <= 2.0 * e_mad.max() + 1e-4
    assert g_mad.mean() <= 2.0 * e_mad.mean() + 1e-4
    assert g_dc.max() <= 4.0 * e_dc.max() + 1e-6
    assert g_dc.mean() <= 3.0 * e_dc.mean() + 1e-6
    assert g_dc.max() <= 1e-3
    assert np.allclose(np.sum(np.asarray(got, np.float64) ** 2, axis=1), 1.0, atol=1e-5)


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
def full_oracle(full_model, oracle):
    return oracle.OracleModel(full_model)


@pytest.fixture(scope="module")
def full_gpu(gpu_ctx, full_model):
    from semantica_gpu import Model
    m = Model(gpu_ctx, full_model)
    yield m
    m.close()


def test_layer_taps_vs_oracle(full_gpu, full_oracle):
    """Residual stream after 0, 1 and 2 layers, before int8 flips compound."""
    import torch
    from semantica_gpu import synth
    lens = [32, 5, 100, 1]
    off = synth.offsets_from_lengths(lens)
    toks = synth.token_ids(int(off[-1]), 262144, seed=0)
    d_tok = torch.from_numpy(toks).cuda()
    hid = torch.empty((int(off[-1]), 768), dtype=torch.float32, device="cuda")
    rels = {}
    for n in (0, 1, 2):
        say(f"layer tap n_layers={n} lens={lens}")
        full_gpu.forward_hidden(d_tok.data_ptr(), off, n, hid.data_ptr())
        torch.cuda.synchronize()
        got = hid.cpu().numpy()
        for i in range(len(lens)):
            rc, ref = full_oracle.forward(toks[off[i]:off[i + 1]], 768, order=0, stop_layer=n)
            assert rc == 0
            g = got[off[i]:off[i + 1]]
            if n == 0:
                assert np.array_equal(g.view(np.uint32), ref.view(np.uint32)), i
                continue
            rel = np.linalg.norm(g.astype(np.float64) - ref) / np.linalg.norm(ref)
            rels.setdefault(n, []).append(rel)
            say(f"  seq {i} (S={lens[i]}): rel diff {rel:.2e}")
    assert max(rels[1]) <= 1e-5, rels[1]
    assert np.median(rels[2]) <= 1e-5 and max(rels[2]) <= 1e-2, rels[2]


def test_tiny_forward_envelope(tiny_gpu, tiny_model, oracle):
    from semantica_gpu import synth
    # edge lengths (1, partial and exact 32-row tiles) plus 18 seeded ragged ones
    lens = [1, 7, 32, 33, 128, 300] + [int(x) for x in synth.lengths_log_uniform(18, 2, 300, seed=11)]
    off = synth.offsets_from_lengths(lens)
    toks = synth.token_ids(int(off[-1]), tiny_model.config["vocab_size"], seed=7)
    say(f"tiny forward lens={lens}")
    om = oracle.OracleModel(tiny_model)
    for dim in (768, 256):
        _check_envelope(tiny_gpu.forward_packed(toks, off, dim), om, toks, off, dim, f"tiny dim={dim}")


def test_gguf_load_matches_descriptor_load(gpu_ctx, tiny_gpu, tiny_model, tmp_path):
    """LoadModelFromBytes / LoadModel over the synthetic GGUF image give the
    same weights as the descriptor load: embeddings identical bit for bit;
    Q8_0-stored norms are dequantized like gguf.DequantizeQ8_0."""
    from semantica_gpu import Model, SemanticaError, _lib, synth
    lens = [5, 40, 1, 33]
    off = synth.offsets_from_lengths(lens)
    toks = synth.token_ids(int(off[-1]), tiny_model.config["vocab_size"], seed=3)
    say("gguf load: bytes, file, Q8_0 norms, wrong dtype")
    want = tiny_gpu.forward_packed(toks, off, 768)
    image = synth.model_gguf(tiny_model)
    m = Model.from_gguf(gpu_ctx, image)
    assert m.config["vocab_size"] == 4096 and m.config["num_layers"] == 2
    assert np.array_equal(m.forward_packed(toks, off, 768).view(np.uint32), want.view(np.uint32))
    m.close()
    path = tmp_path / "tiny.gguf"
    path.write_bytes(image)
    m = Model.from_gguf(gpu_ctx, str(path))
    assert np.array_equal(m.forward_packed(toks, off, 768).view(np.uint32), want.view(np.uint32))
    m.close()
    qm = synth.quantized_norms(tiny_model)
    a, b = Model(gpu_ctx, qm), Model.from_gguf(gpu_ctx, synth.model_gguf(qm, norms_q8=True))
    assert np.array_equal(a.forward_packed(toks, off, 256).view(np.uint32),
                          b.forward_packed(toks, off, 256).view(np.uint32))
    a.close()
    b.close()
    md, ts = synth.model_gguf_parts(tiny_model)
    ts = [(n, dims, 1 if n == "blk.0.attn_q.weight" else dt, raw) for n, dims, dt, raw in ts]
    with pytest.raises(SemanticaError) as ei:
        Model.from_gguf(gpu_ctx, synth.gguf_image(md, ts))
    assert ei.value.code == _lib.SG_ERR_INVALID
    assert "expected Q8_0, got F16 for blk.0.attn_q.weight" in ei.value.message


def test_hand_assembled_gguf_payloads_vs_oracle(gpu_ctx, oracle, tmp_path):
    """GGUF payload parity independent of the repository's writer and loader
    (reader.go:98-178, model.go:424-552, model_int8.go:54-140).  The image is
    assembled field by field in tests/gguf_hand.py: a 2-layer model with the
    token embedding, every Q8_0 matrix and norm at unaligned, out-of-order
    offsets, one Q8_0-stored norm, three optional norms absent and an unused
    tensor between them.  The GPU loads it through sg_model_load_gguf (from
    bytes and from a file); the oracle gets each matrix's bytes straight out
    of the image at the offset the assembler put them.  Teacher-forced, the
    two agree bit for bit on Q|K|V and the residual stream at both layers and
    on the final embeddings, with attention within 1e-5."""
    import gguf_hand
    from semantica_gpu import Model, synth
    image, cfg, placed, norms = gguf_hand.hand_model_image()
    om = oracle.OracleModel(gguf_hand.oracle_model(image, cfg, placed, norms))
    lens = [1, 9, 32, 77, 200, 3]
    off = synth.offsets_from_lengths(lens)
    toks = np.random.default_rng(4).integers(0, cfg["vocab_size"], size=int(off[-1])).astype(np.int32)
    say(f"hand-assembled gguf: {len(image)} bytes, {len(placed)} tensors, lens={lens}")
    gm = Model.from_gguf(gpu_ctx, image)
    try:
        assert gm.config == pytest.approx(cfg)
        _teacher_forced(gm, om, toks, off, 768, cfg["num_layers"], "hand gguf")
        want = gm.forward_packed(toks, off, 256)
        rc, ref = om.forward_batch(toks, off, 256, order=oracle.ORDER_BLOCK_SERIAL, n_threads=4)
        assert rc == 0
        mad, dc = _stats(want, ref)
        say(f"hand gguf free-running vs block-serial oracle, dim 256: max-abs {mad.max():.2e} 1-cos {dc.max():.2e}")
        assert mad.max() <= NORTH_STAR_MAX_ABS and dc.max() <= 1.0 - NORTH_STAR_COS
    finally:
        gm.close()
    path = tmp_path / "hand.gguf"
    path.write_bytes(image)
    fm = Model.from_gguf(gpu_ctx, str(path))
    try:
        assert np.array_equal(fm.forward_packed(toks, off, 256).view(np.uint32), want.view(np.uint32))
    finally:
        fm.close()
    om.close()


def test_forward_errors(tiny_gpu):
    from semantica_gpu import SemanticaError, _lib
    say("forward error cases")
    cases = [
        (lambda: tiny_gpu.forward_batch([[3, 4], []], 768), _lib.SG_ERR_EMPTY, "empty input"),
        (lambda: tiny_gpu.forward_batch([[5] * 2049], 768), _lib.SG_ERR_TOO_LONG, "sequence too long: 2049 > 2048"),
        (lambda: tiny_gpu.forward_batch([[3, 4], [9, 4096, 2]], 768), _lib.SG_ERR_TOKEN,
         "token ID out of range: 4096"),
        (lambda: tiny_gpu.forward_batch([[3, -7], []], 768), _lib.SG_ERR_TOKEN, "token ID out of range: -7"),
        (lambda: tiny_gpu.forward_batch([[3, 4]], 0), _lib.SG_ERR_DIM, "target dimension 0 out of range (1..768)"),
        (lambda: tiny_gpu.forward_batch([[3, 4]], 769), _lib.SG_ERR_DIM, "target dimension 769"),
    ]
    for fn, code, msg in cases:
        with pytest.raises(SemanticaError) as ei:
            fn()
        assert ei.value.code == code and msg in ei.value.message
    # the model still works after errors
    assert tiny_gpu.forward_batch([[3, 4, 5]], 768).shape == (1, 768)


def test_device_path_errors_match_host_path(tiny_gpu):
    """sg_forward_device (tokens already in HBM) reports the same error as the
    host path, in the reference's request order (api.go:286-292: the first
    request with an error wins; model_int8.go:150-171: within a request,
    empty / too long before its first out-of-range token), with the
    offending id in the message."""
    import torch
    from semantica_gpu import SemanticaError, _lib
    say("device-path error order")
    cases = [  # (sequences, expected code, expected message)
        ([[3, 4], [9, 4096, 2], [5] * 2049], _lib.SG_ERR_TOKEN, "token ID out of range: 4096"),
        ([[5] * 2049, [9, 4096]], _lib.SG_ERR_TOO_LONG, "sequence too long: 2049 > 2048"),
        ([[3], [], [1, -3]], _lib.SG_ERR_EMPTY, "empty input"),
        ([[1, -5, 2, 300000]], _lib.SG_ERR_TOKEN, "token ID out of range: -5"),
        ([[1, 2], [7, 8, 99999], [4, -1]], _lib.SG_ERR_TOKEN, "token ID out of range: 99999"),
        ([[1, 2], [7, 8], [], [4, -1]], _lib.SG_ERR_EMPTY, "empty input"),
    ]
    for seqs, code, msg in cases:
        toks = np.array([t for q in seqs for t in q], np.int32)
        off = np.cumsum([0] + [len(q) for q in seqs]).astype(np.int32)
        d_tok = torch.from_numpy(toks if toks.size else np.zeros(1, np.int32)).cuda()
        out = torch.empty((len(seqs), 768), dtype=torch.float32, device="cuda")
        with pytest.raises(SemanticaError) as eh:
            tiny_gpu.forward_packed(toks, off, 768)
        with pytest.raises(SemanticaError) as ed:
            tiny_gpu.forward_device(d_tok.data_ptr(), off, 768, out.data_ptr())
        say(f"  {[len(q) for q in seqs]}: host '{eh.value.message}' device '{ed.value.message}'")
        assert (eh.value.code, eh.value.message) == (ed.value.code, ed.value.message) == (code, msg)
    assert tiny_gpu.forward_batch([[3, 4, 5]], 768).shape == (1, 768)

def test_sequence_groups_match_one_stream(tiny_gpu):
    """From 8192 tokens the forward runs as two contiguous sequence groups, each on
    its own stream, so the kernels of the two groups overlap on the GPU.  Each
    sequence's arithmetic is unchanged.  Ragged batches of 8k to 35k tokens are
    bit-identical to the same batch on one stream (the profiled path runs one
    group).  The batches of ~10k and ~13k tokens also compare the two forms of
    the O/down projection + residual post-norm: one group of 8192+ rows runs the
    fused whole-row GEMM kernel (o never stored), each half-size group the GEMM
    and k_post_res_norm as two launches.  With out-of-range tokens in both
    groups, the one in group 0 is reported, and with one only in group 1 that
    one, as the reference's request order does (api.go:286-292), on both the
    host and the device entry points."""
    import torch
    from semantica_gpu import SemanticaError, _lib
    rng = np.random.default_rng(11)
    for n, hi in ((10, 2048), (13, 2048), (60, 1100), (200, 300)):
        lens = rng.integers(1, hi + 1, size=n)
        off = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
        T = int(off[-1])
        toks = rng.integers(0, 4096, size=T).astype(np.int32)
        say(f"sequence groups: {n} sequences, {T} tokens")
        y = tiny_gpu.forward_packed(toks, off, 768)
        tiny_gpu.profile_enable(True)
        try:
            y1 = tiny_gpu.forward_packed(toks, off, 768)
        finally:
            tiny_gpu.profile_enable(False)
        assert np.array_equal(y.view(np.uint32), y1.view(np.uint32))
        if T < 16384:
            continue
        # the groups split at the sequence edge nearest T/2: sequence n//4 ends
        # near T/4 (group 0), sequence 0.9n starts near 0.9T (group 1)
        i1, i2 = n // 4, int(n * 0.9)
        assert off[i1 + 1] < T // 2 < off[i2]
        both = toks.copy()
        both[off[i2]] = 5000
        both[off[i1 + 1] - 1] = 4096 + i1
        second = toks.copy()
        second[off[i2]] = 5000
        for bad, tok, where in ((both, 4096 + i1, f"sequences {i1} and {i2}"), (second, 5000, f"sequence {i2}")):
            with pytest.raises(SemanticaError) as eh:
                tiny_gpu.forward_packed(bad, off, 768)
            d_tok = torch.from_numpy(bad).cuda()
            out = torch.empty((n, 768), dtype=torch.float32, device="cuda")
            with pytest.raises(SemanticaError) as ed:
                tiny_gpu.forward_device(d_tok.data_ptr(), off, 768, out.data_ptr())
            say(f"  errors at {where}: host '{eh.value.message}' device '{ed.value.message}'")
            expect = (_lib.SG_ERR_TOKEN, f"token ID out of range: {tok}")
            assert (eh.value.code, eh.value.message) == (ed.value.code, ed.value.message) == expect


@pytest.mark.parametrize("mode", ["fast", "exact"])
def test_short_sequence_fusions_match_unfused(full_gpu, mode):
    """Short sequences take fused launches.  When every sequence of a batch
    lies inside one 32-row workgroup of the row kernels, the post-norms
    quantize the next GEMM operand themselves (k_post_res_norm_q), and when
    every sequence is one attention work item (at most 32 tokens with 3 query
    heads) the attention kernel quantizes its own output (fast mode).  A
    sequence's embedding does not depend on the rest of its batch, so the same
    sequences embedded in batches that take both fused forms, only the
    attention one (a sequence crosses a 32-row boundary), or neither (a
    40-token sequence crosses it and needs two attention items) agree bit for
    bit, over 24 layers at full size."""
    from semantica_gpu import _lib
    rng = np.random.default_rng(31)
    x1, x2, x3, x40 = (rng.integers(2, 262144, size=n).astype(np.int32) for n in (32, 7, 19, 40))
    batches = {
        "fused (one 32-token sequence)": [x1],
        "fused (7 + 19 tokens in one row block)": [x2, x3],
        "fused (four sequences in row blocks)": [x1, x2, x3, x2[:5]],
        "attention-fused only (7 + 32: a sequence crosses row 32)": [x2, x1, x3],
        "unfused (a 40-token sequence first)": [x40, x1, x2, x3],
    }
    full_gpu.set_attention_mode(_lib.SG_ATTN_EXACT if mode == "exact" else _lib.SG_ATTN_FAST)
    try:
        got = {}
        for name, seqs in batches.items():
            toks = np.concatenate(seqs)
            off = np.concatenate([[0], np.cumsum([len(q) for q in seqs])]).astype(np.int32)
            say(f"short-sequence fusions ({mode}): {name}")
            y = full_gpu.forward_packed(toks, off, 768)
            for q, e in zip(seqs, y):
                got.setdefault(q.tobytes(), []).append((name, e))
    finally:
        full_gpu.set_attention_mode(_lib.SG_ATTN_FAST)
    for key, runs in got.items():
        ref_name, ref = runs[0]
        for name, e in runs[1:]:
            assert np.array_equal(e.view(np.uint32), ref.view(np.uint32)), (len(key) // 4, ref_name, name)


@pytest.mark.parametrize("lens", [
    [512] * 20 + [32, 992, 64, 2048, 96, 37],                    # 13,509 tokens: the 8-wave GEMM kernel
    [256] * 20 + [32, 480, 1024, 37],                            # 6,693 tokens: the 4-wave GEMM kernel
    [512] * 20 + [37, 1000, 511, 513, 1, 33, 2048, 64, 95, 700],  # starts off 32-row boundaries: not fused
])
def test_qkv_gemm_writes_vt_operand(tiny_gpu, lens):
    """From 6144 tokens, when every sequence starts on a 32-row boundary, the
    QKV GEMM's epilogue writes the V columns straight as the attention's V^T
    operand (hi/lo fp16, keys in the MMA order; whole 32-key tiles as 16-byte
    chunks, the last sequence's partial tile value by value) and k_kv_prep
    prepares only K.  Tracing Q|K|V turns that off (the fp32 V is then stored
    and split by k_kv_prep), so the residual stream traced with and without
    the Q|K|V tap compares the two forms: bit-identical after every layer.
    The batch embedded normally (two sequence groups from 8192 tokens) is
    pinned to single sequences (register-direct GEMMs, never fused) by batch
    invariance."""
    import torch
    rng = np.random.default_rng(21)
    off = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    T, L = int(off[-1]), 2
    toks = rng.integers(0, 4096, size=T).astype(np.int32)
    say(f"QKV GEMM V^T epilogue: {len(lens)} sequences, {T} tokens")
    d_tok = torch.from_numpy(toks).cuda()
    h_fused = torch.empty((L, T, 768), dtype=torch.float32, device="cuda")
    h_plain = torch.empty_like(h_fused)
    qkv = torch.empty((L, T, 1280), dtype=torch.float32, device="cuda")
    tiny_gpu.forward_trace(d_tok.data_ptr(), off, L, d_h_ptr=h_fused.data_ptr())
    tiny_gpu.forward_trace(d_tok.data_ptr(), off, L, d_qkv_ptr=qkv.data_ptr(), d_h_ptr=h_plain.data_ptr())
    torch.cuda.synchronize()
    a, b = h_fused.cpu().numpy(), h_plain.cpu().numpy()
    for l in range(L):
        assert np.array_equal(a[l].view(np.uint32), b[l].view(np.uint32)), l
    y = tiny_gpu.forward_packed(toks, off, 768)
    _batch_invariance(tiny_gpu, toks, off, 768, y, (0, len(lens) - 3, len(lens) - 1))


def test_concurrent_callers_match_serial(tiny_gpu):
    """TestConcurrentBufferPooling (internal/runtime/pooling_test.go:34-75):
    seven host threads call sg_forward on one model at once, four times each
    (ctypes releases the GIL for the call, so the calls overlap in the
    library).  Each result equals the same call made alone, bit for bit,
    whatever else runs; one thread's batches hold an out-of-range token, and
    that thread gets its own error message (sg_last_error is per thread)
    while the others succeed.  One batch of ~9k tokens runs as two sequence
    groups; the dims differ per thread."""
    import threading
    from semantica_gpu import SemanticaError, _lib, synth
    rng = np.random.default_rng(31)
    jobs = []
    for j in range(6):
        lens = rng.integers(300, 600, size=20) if j == 5 else rng.integers(1, 400, size=int(rng.integers(1, 40)))
        off = synth.offsets_from_lengths(lens)
        toks = rng.integers(0, 4096, size=int(off[-1])).astype(np.int32)
        jobs.append((toks, off, (768, 256, 128)[j % 3]))
    bad = jobs[0][0].copy()
    bad[-1] = 4096 + 7
    say(f"concurrent callers: batches of {[int(o[-1]) for _, o, _ in jobs]} tokens + one with a bad token")
    serial = [tiny_gpu.forward_packed(t, o, d) for t, o, d in jobs]
    results, errors, crashed = {}, {}, []

    def worker(j):
        try:
            for it in range(4):
                if j == 6:
                    try:
                        tiny_gpu.forward_packed(bad, jobs[0][1], 768)
                        errors[it] = None
                    except SemanticaError as e:
                        errors[it] = (e.code, e.message)
                else:
                    t, o, d = jobs[j]
                    results[(j, it)] = tiny_gpu.forward_packed(t, o, d)
        except Exception as e:  # noqa: BLE001  (reported below, on the main thread)
            crashed.append((j, repr(e)))

    threads = [threading.Thread(target=worker, args=(j,)) for j in range(7)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not crashed, crashed
    for (j, it), y in results.items():
        assert np.array_equal(y.view(np.uint32), serial[j].view(np.uint32)), (j, it)
    assert len(results) == 24
    assert all(errors[it] == (_lib.SG_ERR_TOKEN, "token ID out of range: 4103") for it in range(4)), errors


def _teacher_forced(gpu, om, toks, off, dim, n_layers, tag, seam_layers=(), threads=16):
    """Teacher-forced parity at every layer.  The GPU's per-layer trace
    (sg_forward_trace) gives each layer's Q|K|V GEMM output, attention output
    and residual stream.  The oracle (block-serial GEMM order) then reruns the
    forward with each layer's attention output replaced by the GPU's, so both
    sides feed identical values into everything after attention.  Asserted:
      * Q|K|V and the residual stream after every layer are bit-identical:
        every kernel other than attention's two products is exact, at any
        depth (embedding, pre-norm + quantize, the GEMMs, post-norm +
        residual, GELU * up and its quantize);
      * the oracle's own attention on those (bit-identical) inputs is within
        1e-5 relative of the GPU's, per sequence and layer;
      * for `seam_layers`, the forward's fused attention prologue (Q's
        QK-norm + RoPE + split) and K/V^T preparation give the same bits as the
        kernel seam's k_qknorm_rope (bit-exact to the oracle) + sg_attention;
      * with all layers traced, the final embeddings are bit-identical too.
    Returns the per-layer maxima of the attention relative error."""
    import torch
    from semantica_gpu import kernels
    c = om.config
    T, d = int(off[-1]), c["embed_dim"]
    hd = d // c["num_heads"]
    qd, kvd = c["num_heads"] * hd, c["num_kv_heads"] * hd
    d_tok = torch.from_numpy(np.ascontiguousarray(toks)).cuda()
    qkv = torch.empty((n_layers, T, qd + 2 * kvd), dtype=torch.float32, device="cuda")
    att = torch.empty((n_layers, T, qd), dtype=torch.float32, device="cuda")
    h = torch.empty((n_layers, T, d), dtype=torch.float32, device="cuda")
    say(f"{tag}: GPU trace of {n_layers} layers, {len(off) - 1} sequences, {T} tokens")
    gpu.forward_trace(d_tok.data_ptr(), off, n_layers, qkv.data_ptr(), att.data_ptr(), h.data_ptr())
    torch.cuda.synchronize()
    for l in seam_layers:
        q = qkv[l, :, :qd].contiguous()
        k = qkv[l, :, qd:qd + kvd].contiguous()
        v = qkv[l, :, qd + kvd:].contiguous()
        ly = om_layers(om)[l]
        qn = torch.from_numpy(ly["attn_q_norm"]).cuda()
        kn = torch.from_numpy(ly["attn_k_norm"]).cuda()
        kernels.qknorm_rope(gpu.ctx, q, k, qn, kn, c["num_heads"], c["num_kv_heads"], hd, c["norm_eps"],
                            c["rope_base"], c["max_seq_len"], off)
        seam = torch.empty((T, qd), dtype=torch.float32, device="cuda")
        kernels.attention(gpu.ctx, seam, q, k, v, c["num_heads"], c["num_kv_heads"], hd, off)
        torch.cuda.synchronize()
        same = torch.equal(seam.view(torch.int32), att[l].view(torch.int32))
        say(f"  layer {l}: fused prologue vs seam QK-norm/RoPE + attention bit-identical: {same}")
        assert same, l
    g_qkv, g_att, g_h = qkv.cpu().numpy(), att.cpu().numpy(), h.cpu().numpy()
    del qkv, att, h
    full = n_layers == c["num_layers"]
    g_out = gpu.forward_packed(toks, off, dim) if full else None
    rc, o_out, arr = om.forward_taps(toks, off, dim, n_layers, att_in=g_att, qkv=True, att=True, h=True,
                                     n_threads=threads)
    assert rc == 0
    att_err = []
    for l in range(n_layers):
        assert np.array_equal(arr["qkv"][l].view(np.uint32), g_qkv[l].view(np.uint32)), f"{tag}: Q|K|V layer {l}"
        assert np.array_equal(arr["h"][l].view(np.uint32), g_h[l].view(np.uint32)), f"{tag}: h after layer {l}"
        rel = [np.linalg.norm(g_att[l, a:b].astype(np.float64) - arr["att"][l, a:b]) /
               max(np.linalg.norm(arr["att"][l, a:b].astype(np.float64)), 1e-30) for a, b in zip(off[:-1], off[1:])]
        att_err.append(max(rel))
    say(f"{tag}: Q|K|V and h bit-identical after each of {n_layers} layers; attention rel err per layer "
        f"max {max(att_err):.2e} (layers: {' '.join(f'{e:.1e}' for e in att_err)})")
    assert max(att_err) <= 1e-5
    if full:
        assert np.array_equal(o_out.view(np.uint32), g_out.view(np.uint32)), f"{tag}: final embeddings"
        say(f"{tag}: final embeddings (dim {dim}) bit-identical under teacher forcing")
    return att_err


def _exact_forward(gpu, om, toks, off, dim, tag, threads=16):
    """The GPU forward with SG_ATTN_EXACT against the oracle's block-serial
    forward (matmul_inner_loop_fallback.go:16-43 through model_int8.go:148-256):
    every embedding bit-identical.  Restores the default mode."""
    from semantica_gpu import _lib
    gpu.set_attention_mode(_lib.SG_ATTN_EXACT)
    try:
        say(f"{tag}: exact-attention forward, {len(off) - 1} sequences, {int(off[-1])} tokens, dim {dim}")
        got = gpu.forward_packed(toks, off, dim)
    finally:
        gpu.set_attention_mode(_lib.SG_ATTN_FAST)
    import oracle as o
    say(f"{tag}: oracle block-serial forward on {threads} threads")
    rc, ref = om.forward_batch(toks, off, dim, order=o.ORDER_BLOCK_SERIAL, n_threads=threads)
    assert rc == 0
    same = np.all(got.view(np.uint32) == ref.view(np.uint32), axis=1)
    mad, dc = _stats(got, ref)
    say(f"{tag}: {int(same.sum())}/{len(same)} embeddings bit-identical to the block-serial path "
        f"(max-abs {mad.max():.1e}); north_star bar: {'met' if mad.max() <= NORTH_STAR_MAX_ABS else 'NOT met'}")
    assert same.all(), np.nonzero(~same)[0][:10]


def test_exact_attention_forward_config0(full_gpu, full_oracle):
    """Config 0 shape (8 rows of 32 tokens, seed 0), 24 layers, exact attention:
    bit-identical to the oracle's block-serial forward."""
    from semantica_gpu import synth
    toks = synth.token_ids(8 * 32, 262144, seed=0)
    off = np.arange(0, 8 * 32 + 1, 32, dtype=np.int32)
    _exact_forward(full_gpu, full_oracle, toks, off, 768, "c0 exact")


@pytest.mark.parametrize("case", ["short_mixed", "long_mixed", "many_tiny", "singletons", "one_row_block"])
def test_exact_attention_forward_random_batches(full_gpu, full_oracle, case):
    """Exact attention makes every embedding comparable bit for bit with the
    oracle's block-serial forward, so ragged batches chosen to cross the
    forward's dispatch boundaries are checked that way over all 24 layers:
    short mixed lengths (register-direct GEMMs with and without the
    MFMA-ahead loop, attention items of one and several workgroups), long
    sequences next to short ones (spilled attention scores, 2048 keys),
    hundreds of tiny sequences, single-token sequences (the short-sequence
    fused post-norm quantize), and one 32-row block of several sequences."""
    rng = np.random.default_rng({"short_mixed": 41, "long_mixed": 42, "many_tiny": 43, "singletons": 44,
                                 "one_row_block": 45}[case])
    if case == "short_mixed":
        lens = np.exp(rng.uniform(0, np.log(300), size=37)).astype(int) + 1
    elif case == "long_mixed":
        lens = np.array([1, 2048, 700, 33, 1200, 513])
    elif case == "many_tiny":
        lens = rng.integers(1, 65, size=200)
    elif case == "singletons":
        lens = np.ones(3, int)
    else:
        lens = np.array([5, 11, 2, 14])
    off = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    toks = rng.integers(2, 262144, size=int(off[-1])).astype(np.int32)
    _exact_forward(full_gpu, full_oracle, toks, off, 768, f"random batch {case}")


@pytest.mark.parametrize("interm", [1088, 1120])
def test_exact_attention_forward_ragged_k_blocks(gpu_ctx, oracle, interm):
    """Small batches run the forward's GEMMs on the register-direct kernel with
    a 6-stage load ring (cold weights); the model's own widths (24 and 36
    K-blocks) fill its rounds exactly, so FFN widths of 34 and 35 blocks leave
    partial last rounds of 4 and 5 blocks in the down GEMM.  Two layers, exact
    attention, bit-identical to the oracle's block-serial forward."""
    from semantica_gpu import Model, synth
    cfg = dict(synth.EMBEDDINGGEMMA_300M, num_layers=2, vocab_size=4096, interm_dim=interm)
    mdl = synth.make_model(cfg, seed_weights=13)
    m = Model(gpu_ctx, mdl)
    try:
        for lens in ([32], [7, 19, 3, 40]):
            off = synth.offsets_from_lengths(lens)
            toks = synth.token_ids(int(off[-1]), 4096, seed=3)
            _exact_forward(m, oracle.OracleModel(mdl), toks, off, 768, f"ffn {interm} lens {lens}", threads=4)
    finally:
        m.close()


def test_exact_attention_forward_config4(full_gpu, full_oracle):
    """Config 4 at full size: 256 log-uniform lengths in [8, 512] (seed 1),
    Matryoshka dim 256, 24 layers, two sequence groups on two streams, exact
    attention: every embedding bit-identical to the block-serial path."""
    from semantica_gpu import synth
    lens = synth.lengths_log_uniform(256, 8, 512, seed=1)
    off = synth.offsets_from_lengths(lens)
    toks = synth.token_ids(int(off[-1]), 262144, seed=1)
    _exact_forward(full_gpu, full_oracle, toks, off, 256, "c4 exact")


def test_exact_attention_forward_config2(full_gpu, full_oracle):
    """The headline shape, config 2: 64 x 512 tokens (seed 0), 24 layers, the
    fused GEMM + residual post-norm kernels and two sequence groups, exact
    attention: all 64 embeddings bit-identical to the block-serial path."""
    from semantica_gpu import synth
    toks = synth.token_ids(64 * 512, 262144, seed=0)
    off = np.arange(0, 64 * 512 + 1, 512, dtype=np.int32)
    _exact_forward(full_gpu, full_oracle, toks, off, 768, "c2 exact")


def test_exact_attention_forward_config3(full_gpu, full_oracle):
    """Config 3 at full size: 8 sequences of U[1024, 2048] tokens (seed 4),
    past the fast path's 512-key register kernel, 24 layers, exact attention:
    every embedding bit-identical to the block-serial path."""
    from semantica_gpu import synth
    lens = synth.lengths_uniform(8, 1024, 2048, seed=4)
    off = synth.offsets_from_lengths(lens)
    toks = synth.token_ids(int(off[-1]), 262144, seed=4)
    _exact_forward(full_gpu, full_oracle, toks, off, 768, "c3 exact")


def om_layers(om):
    return om.model.layers


def test_teacher_forced_config0(full_gpu, full_oracle):
    """Config 0 shape (32-token rows, seed 0), 8 rows, all 24 layers."""
    from semantica_gpu import synth
    toks = synth.token_ids(8 * 32, 262144, seed=0)
    off = np.arange(0, 8 * 32 + 1, 32, dtype=np.int32)
    _teacher_forced(full_gpu, full_oracle, toks, off, 768, 24, "c0 forced", seam_layers=(0, 23))


def test_teacher_forced_config4_slice(full_gpu, full_oracle):
    """Config 4's first 24 ragged rows (log-uniform lengths, seed 1), 256 dims, all 24 layers."""
    from semantica_gpu import synth
    lens = synth.lengths_log_uniform(256, 8, 512, seed=1)[:24]
    off = synth.offsets_from_lengths(lens)
    toks = synth.token_ids(int(off[-1]), 262144, seed=1)
    _teacher_forced(full_gpu, full_oracle, toks, off, 256, 24, "c4 slice forced", seam_layers=(5,))


def test_teacher_forced_long_sequences(gpu_ctx, oracle):
    """Config 3's lengths past 512 keys (attention with the scores past 512 keys spilled), 4 layers."""
    from semantica_gpu import Model, synth
    cfg = dict(synth.EMBEDDINGGEMMA_300M, num_layers=4, vocab_size=8192)
    mdl = synth.make_model(cfg, seed_weights=9)
    lens = [1500, 2048, 1024, 600]
    off = synth.offsets_from_lengths(lens)
    toks = synth.token_ids(int(off[-1]), 8192, seed=4)
    m = Model(gpu_ctx, mdl)
    try:
        _teacher_forced(m, oracle.OracleModel(mdl), toks, off, 768, 4, "c3 lengths forced", seam_layers=(1,),
                        threads=4)
    finally:
        m.close()


def test_config0_envelope(full_gpu, full_oracle):
    """Config 0: 1 x 32 tokens (seed 0), plus 7 more 32-token rows for statistics."""
    from semantica_gpu import synth
    toks = synth.token_ids(8 * 32, 262144, seed=0)
    off = np.arange(0, 8 * 32 + 1, 32, dtype=np.int32)
    say("config0 8x32 full model")
    _check_envelope(full_gpu.forward_packed(toks, off, 768), full_oracle, toks, off, 768, "c0")


def test_config4_ragged_matryoshka_envelope(full_gpu, full_oracle):
    """Config 4 shape (log-uniform lengths in [8, 512], seed 1, 256 dims) on a 24-row slice."""
    from semantica_gpu import synth
    lens = synth.lengths_log_uniform(256, 8, 512, seed=1)[:24]
    off = synth.offsets_from_lengths(lens)
    toks = synth.token_ids(int(off[-1]), 262144, seed=1)
    say(f"config4 slice lens={lens.tolist()}")
    _check_envelope(full_gpu.forward_packed(toks, off, 256), full_oracle, toks, off, 256, "c4")


def test_long_sequence_envelope(gpu_ctx, oracle):
    """Config 3's attention-heavy lengths on a 2-layer model."""
    from semantica_gpu import Model, synth
    cfg = dict(synth.EMBEDDINGGEMMA_300M, num_layers=2, vocab_size=8192)
    mdl = synth.make_model(cfg, seed_weights=9)
    lens = [1500, 2048, 1024]
    off = synth.offsets_from_lengths(lens)
    toks = synth.token_ids(int(off[-1]), 8192, seed=4)
    say(f"long sequences {lens}")
    m = Model(gpu_ctx, mdl)
    try:
        got = m.forward_packed(toks, off, 768)
    finally:
        m.close()
    _check_envelope(got, oracle.OracleModel(mdl), toks, off, 768, "long", threads=3)


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
    perm = np.array([5, 0, 63, 12], np.int64)
    toks_p = np.concatenate([toks[512 * i:512 * (i + 1)] for i in perm])
    yp = full_gpu.forward_packed(toks_p, np.arange(0, 4 * 512 + 1, 512, dtype=np.int32), 768)
    assert np.array_equal(yp.view(np.uint32), y[perm].view(np.uint32))


def _batch_invariance(gpu, toks, off, out_dim, y, rows):
    """Each listed sequence embedded alone is bit-identical to its row of the packed batch.
    The GEMM kernels are chosen by a sequence group's token count, so a sequence alone
    and the packed batch often run different kernels: this also pins them to each
    other."""
    for i in rows:
        a, b = int(off[i]), int(off[i + 1])
        alone = gpu.forward_packed(toks[a:b], np.array([0, b - a], np.int32), out_dim)[0]
        assert np.array_equal(alone.view(np.uint32), y[i].view(np.uint32)), i


def test_config3_full_size_properties(full_gpu):
    """Config 3 (8 sequences, lengths U[1024, 2048] seed 4, full model): finite, unit
    norm, and batch invariance for every sequence."""
    from semantica_gpu import synth
    lens = synth.lengths_uniform(8, 1024, 2048, seed=4)
    off = synth.offsets_from_lengths(lens)
    toks = synth.token_ids(int(off[-1]), 262144, seed=4)
    say(f"config3 lens={lens.tolist()}")
    y = full_gpu.forward_packed(toks, off, 768)
    assert y.shape == (8, 768) and np.all(np.isfinite(y))
    assert np.max(np.abs(np.sum(y.astype(np.float64) ** 2, axis=1) - 1)) < 1e-5
    _batch_invariance(full_gpu, toks, off, 768, y, range(8))


def test_config4_full_size_properties(full_gpu):
    """Config 4 at full size (256 sequences, log-uniform lengths in [8, 512] seed 1,
    Matryoshka 256 dims): finite, unit norm over the 256 dims, and batch invariance on
    a spread of rows."""
    from semantica_gpu import synth
    lens = synth.lengths_log_uniform(256, 8, 512, seed=1)
    off = synth.offsets_from_lengths(lens)
    toks = synth.token_ids(int(off[-1]), 262144, seed=1)
    say(f"config4 full: 256 sequences, {int(off[-1])} tokens")
    y = full_gpu.forward_packed(toks, off, 256)
    assert y.shape == (256, 256) and np.all(np.isfinite(y))
    assert np.max(np.abs(np.sum(y.astype(np.float64) ** 2, axis=1) - 1)) < 1e-5
    _batch_invariance(full_gpu, toks, off, 256, y, (0, 1, 100, 255))


@pytest.mark.parametrize("lens,rows", [
    ([2048, 1, 2047], (0, 1, 2)),                         # T = 4096: gate/up on the 8-wave LDS kernel
    ([2048, 2048, 2047, 1, 2048, 2048, 2048], (2, 3, 4)),  # two groups of 6144: the 4-wave LDS kernel
])
def test_gemm_kernel_thresholds(full_gpu, lens, rows):
    """Packed batches whose sequence groups sit just past a GEMM kernel
    threshold, against the same sequences alone (on the register-direct
    kernels): equal bits for every listed sequence.  The 8-wave kernel of the
    other GEMMs (groups from 12288 tokens) is pinned the same way by the
    config 2 test."""
    from semantica_gpu import synth
    off = synth.offsets_from_lengths(lens)
    toks = synth.token_ids(int(off[-1]), 262144, seed=9)
    say(f"gemm kernel thresholds lens={lens} (T={int(off[-1])})")
    y = full_gpu.forward_packed(toks, off, 768)
    _batch_invariance(full_gpu, toks, off, 768, y, rows)


def test_embed_texts_end_to_end(tiny_gpu, tiny_model):
    """pkg/ggufembed over text (api.go:94-209): OpenBytes of one GGUF image
    carrying the weights and a tokenizer vocabulary; EmbedInputs with mixed
    tasks and dimensions must equal tokenizing each prompt with the oracle
    tokenizer and running the descriptor-loaded model on those IDs, bit for
    bit, in input order."""
    import tokenizer_ref as ref
    from semantica_gpu import embed, synth
    rng = np.random.default_rng(8)
    letters = list("abcdefghijklmnopqrstuvwxyz:|▁")
    pieces = set()
    while len(pieces) < 4096 - 494:
        pieces.add("".join(rng.choice(letters, size=int(rng.integers(2, 6)))))
    vocab = ["<pad>", "<eos>", "<bos>"] + letters + [f"<u{i}>" for i in range(238 - 3 - len(letters))] + \
        [f"<0x{b:02X}>" for b in range(256)] + sorted(pieces)
    assert len(vocab) == 4096
    scores = [0.0] * 238 + [-10.0] * 256 + (-np.arange(len(vocab) - 494, dtype=np.float32) / 100).tolist()
    types = [3, 3, 3] + [1] * 235 + [6] * 256 + [1] * (len(vocab) - 494)
    md = [("tokenizer.ggml.tokens", "arr:str", vocab), ("tokenizer.ggml.scores", "arr:f32", scores),
          ("tokenizer.ggml.token_type", "arr:i32", types), ("tokenizer.ggml.bos_token_id", "u32", 2),
          ("tokenizer.ggml.eos_token_id", "u32", 1), ("tokenizer.ggml.padding_token_id", "u32", 0)]
    image = synth.gguf_image(*synth.model_gguf_parts(tiny_model, vocab_tokens=False, extra_metadata=md))
    say("embed: open_bytes + embed_inputs")
    rt = embed.open_bytes(image)
    try:
        inputs = [embed.EmbedInput(embed.Task.SEARCH_QUERY, "hello world", dim=768),
                  embed.EmbedInput(embed.Task.SEARCH_DOCUMENT, "the quick brown fox", title="fox", dim=256),
                  embed.EmbedInput(embed.Task.NONE, "  plain text, ü and 😀 ", dim=0),
                  embed.EmbedInput(embed.Task.CLUSTERING, "group these", dim=128),
                  embed.EmbedInput(embed.Task.SEARCH_QUERY, "hello world", dim=256)]
        got = rt.embed_inputs(inputs)
        tok = ref.Tokenizer(vocab, scores, types, add_bos=True, nfkc=True, bos_id=2, eos_id=1, pad_id=0)
        for inp, g in zip(inputs, got):
            ids = tok.encode(embed.build_prompt(inp))
            want = tiny_gpu.forward_batch([ids], embed.resolve_dim(inp.dim))[0]
            assert g.shape == want.shape and np.array_equal(g.view(np.uint32), want.view(np.uint32)), inp
        assert [len(v) for v in rt.embed(["a", "b c"])] == [512, 512]
        assert rt.embed([]) is None and rt.embed_dim() == 768 and rt.max_seq_len() == 2048
        with pytest.raises(embed.EmbedError, match=r"sequence too long: \d+ > 2048"):
            rt.embed_single("é" * 1100)  # not in the vocabulary: two byte tokens each
        with pytest.raises(embed.EmbedError, match="build prompt for input 1: content must not be empty"):
            rt.embed_inputs([embed.EmbedInput(content="a"), embed.EmbedInput(content=" ")])
        with pytest.raises(embed.EmbedError, match="input 0: unsupported embed dim 300"):
            rt.embed_inputs([embed.EmbedInput(content="a", dim=300)])
    finally:
        rt.close()


@pytest.mark.parametrize("lens", [
    [40, 64, 33],          # small batch: register-direct GEMMs, separate post-norm kernel
    [1024] * 16,           # 16384 tokens: the LDS GEMMs and the fused GEMM + residual post-norm
])
def test_teacher_forced_zero_activations(gpu_ctx, oracle, lens):
    """Sequences whose activations are exactly zero.  Token IDs below 64 get an
    all-zero embedding row (Q8_0 scale 0, codes 0).  Sequence 0 uses only those
    tokens, so every quantize site sees a per-sequence max of 0 (scale 1, codes
    0: quantize.go's m == 0 case), its attention scores are all 0 (uniform
    weights), and its pooled vector is zero, which L2 normalization leaves as
    is (model.go:808-820).  Sequence 1 mixes zero rows into ordinary ones
    (RMSNorm of a zero row inside a sequence with a non-zero max).  The rest
    are ordinary.  Teacher-forced through both layers of the 2-layer model:
    Q|K|V, h and the final embeddings bit-identical to the oracle."""
    import dataclasses
    from semantica_gpu import Model, synth
    from conftest import TINY
    base = synth.make_model(TINY)
    emb = base.token_embd.copy()
    emb[:64] = 0
    mdl = dataclasses.replace(base, token_embd=emb)
    off = synth.offsets_from_lengths(lens)
    T = int(off[-1])
    toks = synth.token_ids(T, TINY["vocab_size"], seed=11)
    rng = np.random.default_rng(12)
    toks[off[0]:off[1]] = rng.integers(0, 64, lens[0])
    s1 = np.arange(off[1], off[2])
    toks[s1[::3]] = rng.integers(0, 64, len(s1[::3]))
    m = Model(gpu_ctx, mdl)
    try:
        _teacher_forced(m, oracle.OracleModel(mdl), toks, off, 768, TINY["num_layers"], f"zero rows T={T}")
        y = m.forward_packed(toks, off, 768)
    finally:
        m.close()
    assert not np.any(y[0]), "an all-zero sequence embeds to the zero vector"
    assert np.all(np.isfinite(y))
