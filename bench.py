#!/usr/bin/env python3
"""Benchmark: EmbeddingGemma-300M Q8_0 forward, config 2 (64 x 512 tokens) on
one MI355X.  Prints ONE JSON line.

A step is one batched forward (sg_forward_device) over the 64 packed
sequences, token IDs already resident in HBM, embeddings left in HBM.
`value` is embeddings/sec over the K timed steps, which run uninstrumented
(the library runs a batch this size as two sequence groups on two streams,
whose kernels overlap).  Then the same K steps run again with a HIP event
pair around every launch: the profiled forward runs as one group on the
library's stream, so every kernel is timed alone, and the per-kernel-class
breakdown and `roofline` come from that pass (event records between launches
cost ~10% of the step, so they stay out of the timed region).  `roofline` is the Q8_0 GEMM (the
dominant kernel class): algorithmic int8 ops (2*M*N*K per launch) of every
Q8_0 GEMM launch (the plain ones and the O/down GEMMs fused with the residual
post-norm) over their event-measured time, against MI355X's dense int8 peak;
`plain_only` gives the plain launches alone.  `traffic` is read from
profiles/gemm_traffic.json (FETCH_SIZE and WRITE_SIZE counter passes of the
command it names, scaled by a copy kernel of known size), not measured by
this run.
`cpu_baseline` is the CPU oracle (a restatement
of the reference's Go path; the reference itself cannot run here) timed on
this host on a bounded sample of the same workload.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (os.path.join(ROOT, "go-semantica_amd"), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)

METRIC = "embeddings/sec (64×512 tok, Q8_0) on 1 MI355X; Q8_0 GEMM % of int8 peak"
INT8_PEAK_TOPS = 5000.0   # MI355X dense int8 (5.0 POP/s)
HBM_PEAK_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--batch", type=int, default=64)
    ap.add_argument("--seq-len", type=int, default=512)
    ap.add_argument("--cpu-threads", type=int, default=0,
                    help="0: min(16, host CPUs) -- 16 is one GPU's CPU share on the GPU boxes")
    ap.add_argument("--cpu-warmup", type=int, default=2, help="c2 CPU warm-up runs (the reference's: 5)")
    ap.add_argument("--cpu-runs", type=int, default=8,
                    help="c2 CPU timed runs, P50 reported (the reference's: 20; 8 keeps the sample near 20 s)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-search", action="store_true", help="skip the brute-force search measurement")
    ap.add_argument("--no-extras", action="store_true",
                    help="skip the small-batch latency and config-1 GEMM legs (profiles then hold only config-2 steps)")
    ap.add_argument("--search-vectors", type=int, default=1_000_000)
    ap.add_argument("--search-batch", type=int, default=64)
    ap.add_argument("--config-only", type=int, choices=(3, 4), default=0,
                    help="run only the config-3 or config-4 leg and print its object (profiling runs)")
    ap.add_argument("--search-only", action="store_true",
                    help="run only the search measurement and print its JSON (for profiling)")
    ap.add_argument("--no-gpu-events", action="store_true",
                    help="search timing by wall clock only (HIP events on a side stream do not work under rocprofv3)")
    ap.add_argument("--copy-calib-mib", type=int, default=0,
                    help="after the timed region, run a plain fp32 copy kernel (y = -x) of this many MiB "
                         "three times, so a counter run can scale FETCH_SIZE/WRITE_SIZE to bytes")
    return ap.parse_args()


def _cpu_model_name():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _p50(values):
    """calculateStats's P50 (cmd/benchmark/main.go:571-600): sorted[int(n * 0.5)]."""
    v = sorted(values)
    return v[min(int(len(v) * 0.5), len(v) - 1)]


def cpu_baseline(model, toks, seq_len, threads, c2_warmup, c2_runs):
    """The oracle's forward (C restatement of the reference's INT8 Go path; the
    VNNI accumulation order on AVX-512 VNNI intrinsics when the host has them,
    as simd_amd64.go:41-45 dispatches) timed on this host.
      c2: runs of `threads` 512-token rows of the workload, one worker per
          sequence as embedPrompts fans out (api.go:237-295); embeddings/s from
          the P50 run time after c2_warmup warm-up runs.
      c0: one 32-token sequence (the first 32 tokens of the workload), its GEMMs
          split into column chunks over `threads` threads like
          matMulQ8_0INT8Tiled (model_int8.go:258-346); 5 warm-ups, P50 of 20
          runs (measureSingleDocLatency, cmd/benchmark/main.go:553-637).
    CPU time is getrusage(RUSAGE_SELF) over each run."""
    import resource
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np
    import oracle
    lib = oracle.load()
    om = oracle.OracleModel(model)

    def timed(fn):
        r0, t0 = resource.getrusage(resource.RUSAGE_SELF), time.perf_counter()
        rc = fn()
        t1, r1 = time.perf_counter(), resource.getrusage(resource.RUSAGE_SELF)
        if rc != 0:
            raise RuntimeError(f"oracle forward failed: {rc}")
        return t1 - t0, (r1.ru_utime - r0.ru_utime) + (r1.ru_stime - r0.ru_stime)

    n_seq = threads
    if n_seq * seq_len > toks.size:
        raise ValueError("CPU sample exceeds the workload")
    off = np.arange(0, n_seq * seq_len + 1, seq_len, dtype=np.int32)
    sample = np.ascontiguousarray(toks[: n_seq * seq_len])
    c2 = []
    for i in range(c2_warmup + c2_runs):
        r = timed(lambda: om.forward_batch(sample, off, 768, n_threads=threads)[0])
        if i >= c2_warmup:
            c2.append(r)
    wall2 = _p50([w for w, _ in c2])
    cpu2 = _p50([c for _, c in c2])

    off0 = np.array([0, 32], np.int32)
    tok0 = np.ascontiguousarray(toks[:32])
    lib.sgo_set_gemm_threads(threads)
    try:
        c0 = []
        for i in range(25):
            r = timed(lambda: om.forward_batch(tok0, off0, 768, n_threads=1)[0])
            if i >= 5:
                c0.append(r)
    finally:
        lib.sgo_set_gemm_threads(1)
    om.close()
    isa = {2: "AVX-512 VNNI", 1: "AVX2 (VNNI lane order emulated)", 0: "scalar"}[lib.sgo_simd_level()]
    return {"value": round(n_seq / wall2, 3), "unit": "embeddings/sec", "cores": threads, "kind": "port",
            "host": {"nproc": os.cpu_count(), "model_name": _cpu_model_name(), "threads_used": threads},
            "c2": {"embeddings_per_s": round(n_seq / wall2, 3), "p50_run_s": round(wall2, 3),
                   "p50_cpu_s_per_embedding": round(cpu2 / n_seq, 3), "warmup": c2_warmup, "runs": c2_runs,
                   "run": f"{n_seq} sequences x {seq_len} tokens (rows 0..{n_seq - 1} of the workload), "
                          f"one worker per sequence"},
            "c0": {"p50_ms": round(_p50([w for w, _ in c0]) * 1e3, 2),
                   "p50_cpu_ms": round(_p50([c for _, c in c0]) * 1e3, 2), "warmup": 5, "runs": 20,
                   "run": f"1 x 32 tokens, GEMM column chunks over {threads} threads"},
            "sample": f"C oracle (restatement of the reference's INT8 Go path), VNNI-order GEMM on {isa}, "
                      f"{threads} threads; c2 P50 of {c2_runs} runs after {c2_warmup} warm-ups, "
                      f"c0 P50 of 20 runs after 5 warm-ups",
            "method_deviation": None if (c2_warmup, c2_runs) == (5, 20) else
            f"c2 uses {c2_warmup} warm-ups and the P50 of {c2_runs} runs where cmd/benchmark/main.go:553-637 uses 5 "
            f"and 20, to keep the CPU leg near 20 s of the bench; --cpu-warmup 5 --cpu-runs 20 runs the reference's"}


def search_leg(ctx, n, dim, batch, top_k, steps, with_cpu, gpu_events=True):
    """Brute-force search (search/brute) on the GPU: an int8 index of n
    random vectors (normalized and quantized on the device), queried in
    batches of `batch` and one query at a time.  GPU time by HIP events on
    the stream the search runs on; the host-side id mapping and final sort of
    the k results per query are inside the wall time only."""
    import numpy as np
    import torch
    from semantica_gpu import search
    vecs = torch.empty((n, dim), device="cuda", dtype=torch.float32)
    rng = np.random.default_rng(3)
    for r0 in range(0, n, 65536):  # N(0,1) vectors, generated on the host in chunks
        m = min(65536, n - r0)
        vecs[r0:r0 + m].copy_(torch.from_numpy(rng.standard_normal((m, dim), dtype=np.float32)))
    ids = np.arange(n, dtype=np.int32)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    idx = search.Index.from_device(ctx, ids, vecs.data_ptr(), dim, n, search.QUANTIZE_INT8)
    build_s = time.perf_counter() - t0
    del vecs
    rng = np.random.default_rng(4)
    queries = rng.standard_normal((batch, dim)).astype(np.float32)
    st = torch.cuda.Stream()
    out_i = np.zeros((batch, top_k), np.int32)
    out_d = np.zeros((batch, top_k), np.float32)
    found = np.zeros(batch, np.int32)
    lib = idx.lib

    def run(nq):
        qv = np.ascontiguousarray(queries[:nq])
        rc = lib.sg_index_search(idx.handle, qv.ctypes.data, nq, top_k, 1, out_i.ctypes.data, out_d.ctypes.data,
                                 found.ctypes.data, st.cuda_stream)
        if rc != 0:
            raise RuntimeError(lib.sg_last_error())

    out = {}
    for nq, reps in ((batch, steps), (1, 4 * steps)):
        run(nq)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        w0 = time.perf_counter()
        if gpu_events:
            e0.record(st)
        for _ in range(reps):
            run(nq)
        if gpu_events:
            e1.record(st)
            e1.synchronize()
        wall = (time.perf_counter() - w0) / reps
        gpu_ms = e0.elapsed_time(e1) / reps if gpu_events else float("nan")
        out[nq] = (wall, gpu_ms)
    wall_b, gpu_b = out[batch]
    wall_1, gpu_1 = out[1]
    res = {
        "workload": f"int8 index of {n} x {dim} N(0,1) vectors (seed 3; normalized + quantized on the GPU), top-{top_k}, "
                    f"queries normalized (SearchVector)",
        "build_s": round(build_s, 3),
        "batch": batch,
        "queries_per_s": round(batch / wall_b, 1),
        "ms_per_batch": round(wall_b * 1e3, 3),
        "gpu_ms_per_batch": round(gpu_b, 3),
        "single_query_ms": round(wall_1 * 1e3, 3),
        "single_query_gpu_ms": round(gpu_1, 3),
        "single_query_index_GB_s": round(n * dim / (gpu_1 * 1e-3) / 1e9, 1),
        "score_ops_per_query": 2 * n * dim,
    }
    idx.close()
    if with_cpu:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle
        m = min(n, 100_000)
        host = np.random.default_rng(5).standard_normal((m, dim)).astype(np.float32)
        data = oracle.bf_quantize(oracle.bf_normalize(host), oracle.BF_I8)
        qn = oracle.bf_normalize(queries[0])
        t0 = time.perf_counter()
        reps = 3
        for _ in range(reps):
            oracle.bf_search(data, oracle.BF_I8, np.arange(m, dtype=np.int32), qn, top_k)
        per = (time.perf_counter() - t0) / reps * (n / m)
        res["cpu_baseline"] = {"ms_per_query": round(per * 1e3, 2), "cores": 1, "kind": "port",
                               "sample": f"C oracle (AVX2-order restatement of searchNormalized), one thread, "
                                         f"{m} vectors x {reps} queries, scaled to {n}"}
    return res


def small_batch_latency(model, shapes=((1, 32), (8, 32), (1, 512), (8, 512)), reps=10):
    """Wall time of one device-resident forward (tokens already in HBM, embeddings
    left there) at small batches, where the forward is a chain of ~290 short
    kernels rather than a throughput job: the serving latency of EmbedSingle-like
    calls.  Same synthetic model and token stream as the headline."""
    import numpy as np
    import torch
    from semantica_gpu import synth
    res = {}
    for b, s in shapes:
        toks = torch.from_numpy(synth.token_ids(b * s, 262144, seed=0)).cuda()
        off = np.arange(0, b * s + 1, s, dtype=np.int32)
        out = torch.empty((b, 768), dtype=torch.float32, device="cuda")
        for _ in range(3):
            model.forward_device(toks.data_ptr(), off, 768, out.data_ptr())
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            model.forward_device(toks.data_ptr(), off, 768, out.data_ptr())
        torch.cuda.synchronize()
        res[f"{b}x{s}_ms"] = round((time.perf_counter() - t0) / reps * 1e3, 3)
    return res


def ragged_config_leg(model, which, steps=10, warmup=3):
    """Config 3 (8 sequences, lengths U[1024, 2048] seed 4, the attention-heavy
    case: every launch past the 512 keys held in registers) or config 4 (256
    sequences, log-uniform lengths in [8, 512] seed 1, Matryoshka 256 dims):
    device-resident forwards timed like the headline, then one instrumented pass
    (one sequence group) for the attention and GEMM classes.  Same synthetic
    model and token stream as the headline."""
    import numpy as np
    import torch
    from semantica_gpu import synth
    if which == 3:
        lens, out_dim, desc = synth.lengths_uniform(8, 1024, 2048, seed=4), 768, "8 x U[1024, 2048] (seed 4)"
    else:
        lens, out_dim, desc = synth.lengths_log_uniform(256, 8, 512, seed=1), 256, \
            "256 x log-uniform [8, 512] (seed 1), 256 dims"
    off = synth.offsets_from_lengths(lens)
    T, n = int(off[-1]), len(lens)
    toks = torch.from_numpy(synth.token_ids(T, 262144, seed=0)).cuda()
    out = torch.empty((n, out_dim), dtype=torch.float32, device="cuda")
    for _ in range(warmup):
        model.forward_device(toks.data_ptr(), off, out_dim, out.data_ptr())
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        model.forward_device(toks.data_ptr(), off, out_dim, out.data_ptr())
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    model.profile_enable(True)
    model.forward_device(toks.data_ptr(), off, out_dim, out.data_ptr())
    torch.cuda.synchronize()
    prof = model.profile_read()
    model.profile_enable(False)
    emb = out.cpu().numpy()
    assert np.all(np.isfinite(emb)) and np.allclose(np.sum(emb.astype(np.float64) ** 2, axis=1), 1.0, atol=1e-4)
    res = {"workload": f"config {which}: {desc}, {T} tokens", "steps": steps, "ms_per_step": round(dt * 1e3, 3),
           "embeddings_per_s": round(n / dt, 2), "tokens_per_s": round(T / dt)}
    for name in ("attention", "gemm", "gemm_norm"):
        p = prof.get(name)
        if p and p["launches"]:
            rate = p["work"] / (p["ms"] * 1e-3) / 1e12
            res[f"{name}_one_group_ms"] = round(p["ms"], 3)
            res[f"{name}_{'TFLOPS' if name == 'attention' else 'TOPS_int8'}"] = round(rate, 2)
    return res


C1_SHAPES = (("Q/O", 768, 768), ("K/V", 256, 768), ("gate/up", 1152, 768), ("down", 768, 1152),
             ("3072x768", 3072, 768), ("768x3072", 768, 3072))


def gemm_c1_leg(ctx, m=2048, reps=200):
    """Config 1: the isolated Q8_0 GEMMs at the model's layer shapes with M = 2048
    rows.  The GEMM kernel alone: sg_matmul_q8_0_int8_bench relays the int8
    activations into the operand layout once, then times `reps` back-to-back
    launches of the kernel sg_matmul_q8_0_int8 runs, between two HIP events on
    one stream.  Work = 2*M*N*K int8 ops; bytes = int8 A + Q8_0 W (34/32 B per
    weight) + fp32 Y + fp32 row scales, each once.  Each shape is also set
    against its time at the int8 peak and at 8 TB/s."""
    import numpy as np
    import torch
    from semantica_gpu import kernels, synth
    rng = np.random.default_rng(3)
    stream = torch.cuda.Stream()
    res = []
    for name, n, k in C1_SHAPES:
        w = kernels.Q8Weight(ctx, synth.q8_0_random(rng, n, k), n, k)
        xf = rng.standard_normal((m, k)).astype(np.float32)
        x = torch.from_numpy(np.clip(np.round(xf * (127.0 / np.abs(xf).max())), -127, 127).astype(np.int8)).cuda()
        rs = torch.full((m,), 0.01, dtype=torch.float32, device="cuda")
        y = torch.empty((m, n), dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()  # inputs made on the default stream are complete
        us = kernels.matmul_q8_0_kernel_us(ctx, y, w, x, rs, reps, stream=stream.cuda_stream)
        ops, nbytes = 2.0 * m * n * k, m * k + n * k * 34 / 32 + m * n * 4 + m * 4
        res.append({"gemm": name, "N": n, "K": k, "kernel_us": round(us, 2), "TOPS_int8": round(ops / us / 1e6, 1),
                    "frac_int8_peak": round(ops / us / 1e6 / INT8_PEAK_TOPS, 4),
                    "GB_s": round(nbytes / us / 1e3, 1), "frac_hbm": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4),
                    "us_at_int8_peak": round(ops / INT8_PEAK_TOPS / 1e6, 2),
                    "us_at_8TBs": round(nbytes / HBM_PEAK_GBS / 1e3, 2)})
        w.close()
    return {"workload": f"config 1: isolated Q8_0 GEMM kernels, M = {m}, seed-random Q8_0 weights, "
                        f"{reps} back-to-back launches per shape (operand relayout outside the timed region)",
            "shapes": res}


def exact_attention_leg(model, d_tok, off, d_out, steps, B):
    """The same config-2 forward with SG_ATTN_EXACT (attention in the
    reference's float32 order on the VALU; the embeddings are then
    bit-identical to the block-serial path, tests/test_gpu_forward.py::
    test_exact_attention_forward_config2): timed like the headline, then one
    instrumented pass for the attention class's time."""
    import torch
    from semantica_gpu import _lib
    model.set_attention_mode(_lib.SG_ATTN_EXACT)
    try:
        model.forward_device(d_tok.data_ptr(), off, 768, d_out.data_ptr())
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            model.forward_device(d_tok.data_ptr(), off, 768, d_out.data_ptr())
        torch.cuda.synchronize()
        dt = (time.perf_counter() - t0) / steps
        model.profile_enable(True)
        model.forward_device(d_tok.data_ptr(), off, 768, d_out.data_ptr())
        torch.cuda.synchronize()
        prof = model.profile_read()
        model.profile_enable(False)
    finally:
        model.set_attention_mode(_lib.SG_ATTN_FAST)
    a = prof["attention"]
    return {"mode": "SG_ATTN_EXACT", "steps": steps, "embeddings_per_s": round(B / dt, 2),
            "ms_per_step": round(dt * 1e3, 3), "attention_ms_per_step": round(a["ms"], 3),
            "attention_TFLOPS_algorithmic": round(a["work"] / (a["ms"] * 1e-3) / 1e12, 2) if a["ms"] > 0 else None,
            "parity": "embeddings bit-identical to the oracle's block-serial forward at this config"}


def hbm_reference_leg(ctx, T, d=768, reps=20):
    """What plain streaming kernels reach on this GPU, the yardstick for the
    bandwidth-bound row kernels, on [T, d] fp32 tensors: the library's
    sg_hbm_probe kernels (one float4 per lane: c = a + b, 12 B per element,
    the residual add's I/O; and the int8 codes of a, 5 B per element, the
    quantizers' I/O; HIP events on the launch stream inside the library), and
    torch's add and fp32 -> int8 conversion (events on torch's stream)."""
    import torch
    from semantica_gpu import kernels
    a = torch.randn((T, d), device="cuda")
    b = torch.randn((T, d), device="cuda")
    c = torch.empty_like(a)
    q = torch.empty((T, d), dtype=torch.int8, device="cuda")
    torch.cuda.synchronize()
    res = {}
    for name, kind, out, nbytes in (("probe_add", 0, c, 12 * T * d), ("probe_quant", 1, q, 5 * T * d)):
        us = kernels.hbm_probe_us(ctx, kind, a, b, out, reps)
        res[name] = {"us": round(us, 2), "bytes": nbytes, "GB_s": round(nbytes / us / 1e3, 1)}
    for name, fn, nbytes in (("torch_add", lambda: torch.add(a, b, out=c), 12 * T * d),
                             ("torch_to_int8", lambda: q.copy_(a), 5 * T * d)):
        fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        e1.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / reps
        res[name] = {"us": round(us, 2), "bytes": nbytes, "GB_s": round(nbytes / us / 1e3, 1)}
    del a, b, c, q
    return {"workload": f"[{T}, {d}] fp32 tensors, {reps} launches each", **res}


def issue_probe_leg(ctx):
    """The compute floor of the Q8_0 GEMM kernels: SIMD cycles per 32x32 output
    subtile and K-block of their arithmetic alone (sg_issue_probe: one int8
    MFMA, then the block-serial update of 16 subtractions + 16 v_fmac, no
    memory traffic), of its VALU and MFMA halves alone, at 2 and 4 waves per
    SIMD (the GEMM kernels run 4).  The MFMA is 32 cycles of the matrix pipe
    (its issue interval at the dense int8 peak), so 32 / (cycles of kind 0)
    is the largest fraction of the int8 peak these kernels can reach.  Also the
    attention's v_mfma_f32_16x16x32_f16 streamed alone (kind 3): cycles per
    instruction and the fp16 rate it reaches on the 1024 SIMDs."""
    from semantica_gpu import kernels
    res = {}
    for w in (2, 4):
        row = {}
        for kind, name in ((0, "mfma_plus_update"), (1, "update_only"), (2, "mfma_only")):
            cyc, ghz = kernels.issue_probe(ctx, kind, w)
            row[name] = round(cyc, 1)
        row["clock_GHz"] = round(ghz, 2)
        row["int8_peak_frac_ceiling"] = round(32.0 / row["mfma_plus_update"], 3)
        # the attention's fp16 MFMA stream: one 16x16x32 MFMA (8192 MACs) per reported "block"
        cyc3, ghz3 = kernels.issue_probe(ctx, 3, w)
        row["f16_mfma_16x16x32_cycles"] = round(cyc3, 1)
        row["f16_mfma_PFLOPs"] = round(2 * 8192 / cyc3 * 1024 * ghz3 * 1e9 / 1e15, 2)
        res[f"{w}_waves_per_simd"] = row
    return {"unit": "SIMD cycles per 32x32 subtile and K-block", **res}


def tokenizer_leg(n_texts=64, chars=2000):
    """The host tokenizer (sg_tokenizer_*, internal/tokenizer) on a synthetic
    262,144-token vocabulary (the real one is not available offline): texts of
    random words, about one c2 batch of prompts."""
    import numpy as np
    from semantica_gpu.tokenizer import Tokenizer
    rng = np.random.default_rng(6)
    letters = np.array(list("abcdefghijklmnopqrstuvwxyz▁"))
    pieces = set()
    while len(pieces) < 262144 - 494:
        pieces.add("".join(rng.choice(letters, size=int(rng.integers(2, 8)))))
    vocab = ["<pad>", "<eos>", "<bos>"] + [f"<u{i}>" for i in range(235)] + [f"<0x{b:02X}>" for b in range(256)] + \
        sorted(pieces)
    scores = [0.0] * 238 + [-10.0] * 256 + (-rng.random(len(vocab) - 494)).tolist()
    tok = Tokenizer.new(vocab, scores, add_bos=True, nfkc=True, bos_id=2, eos_id=1)
    words = ["".join(rng.choice(letters[:26], size=int(rng.integers(2, 10)))) for _ in range(5000)]
    texts = []
    for _ in range(n_texts):
        t = []
        while sum(len(w) + 1 for w in t) < chars:
            t.append(words[int(rng.integers(0, len(words)))])
        texts.append("task: search result | query: " + " ".join(t))
    tok.encode_batch(texts[:2])
    t0 = time.perf_counter()
    ids, off = tok.encode_batch(texts)
    dt = time.perf_counter() - t0
    tok.close()
    return {"workload": f"{n_texts} prompts of ~{chars} characters, synthetic 262144-token vocabulary, host threads",
            "texts_per_s": round(n_texts / dt, 1), "tokens_per_s": round(int(off[-1]) / dt, 1),
            "tokens_per_text": round(int(off[-1]) / n_texts, 1)}


def main():
    a = parse()
    if a.gpus != 1:
        print(f"bench.py: this build measures one GPU only (--gpus {a.gpus} requested); the path shards as "
              "pure data parallelism over sequences (each rank embeds its own bin of sequences with the "
              "replicated weights; only the embeddings are gathered)", file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch
    from semantica_gpu import Context, Model, synth

    if a.search_only:
        ctx = Context(0)
        res = search_leg(ctx, a.search_vectors, 768, a.search_batch, 10, max(3, a.steps // 2),
                         not a.no_cpu_baseline, gpu_events=not a.no_gpu_events)
        ctx.close()
        print(json.dumps({"search": res}), flush=True)
        return

    if a.config_only:
        ctx = Context(0)
        model = Model(ctx, synth.make_model())
        res = ragged_config_leg(model, a.config_only, steps=a.steps, warmup=a.warmup)
        model.close()
        ctx.close()
        print(json.dumps({f"config{a.config_only}": res}), flush=True)
        return

    B, S = a.batch, a.seq_len
    mdl = synth.make_model()
    toks = synth.token_ids(B * S, mdl.config["vocab_size"], seed=0)
    off = np.arange(0, B * S + 1, S, dtype=np.int32)
    ctx = Context(0)
    model = Model(ctx, mdl)
    d_tok = torch.from_numpy(toks).cuda()
    d_out = torch.empty((B, 768), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    for _ in range(a.warmup):
        model.forward_device(d_tok.data_ptr(), off, 768, d_out.data_ptr())
    torch.cuda.synchronize()

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(a.steps):
        model.forward_device(d_tok.data_ptr(), off, 768, d_out.data_ptr())
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0

    model.profile_enable(True)  # the instrumented pass: per-launch HIP events
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    for _ in range(a.steps):
        model.forward_device(d_tok.data_ptr(), off, 768, d_out.data_ptr())
    torch.cuda.synchronize()
    dt_prof = time.perf_counter() - t1
    prof = model.profile_read()
    model.profile_enable(False)

    if a.copy_calib_mib:
        n = a.copy_calib_mib * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.neg(src, out=dst)
        torch.cuda.synchronize()
        del src, dst

    emb = d_out.cpu().numpy()
    assert np.all(np.isfinite(emb)) and np.allclose(np.sum(emb.astype(np.float64) ** 2, axis=1), 1.0, atol=1e-4)

    g = prof["gemm"]
    gn = prof.get("gemm_norm", {"ms": 0.0, "work": 0.0, "launches": 0})
    gemm_tops = g["work"] / (g["ms"] * 1e-3) / 1e12 if g["ms"] > 0 else 0.0
    # The headline covers every Q8_0 GEMM launch: the plain ones (QKV, gate/up
    # + GELU) and the O and down GEMMs fused with the residual post-norm, whose
    # launch time includes that epilogue.
    all_ms, all_work, all_launches = g["ms"] + gn["ms"], g["work"] + gn["work"], g["launches"] + gn["launches"]
    all_tops = all_work / (all_ms * 1e-3) / 1e12 if all_ms > 0 else 0.0
    kernels = {}
    for name, p in prof.items():
        if p["launches"] == 0:
            continue
        k = {"ms_per_step": round(p["ms"] / a.steps, 4), "launches_per_step": p["launches"] // a.steps}
        if name == "gemm":
            k["TOPS_int8"] = round(gemm_tops, 2)
        elif name == "gemm_norm":  # GEMM + residual post-norm in one launch: the GEMM's int8 ops per second
            k["TOPS_int8"] = round(p["work"] / (p["ms"] * 1e-3) / 1e12, 2)
        elif name == "attention":
            k["TFLOPS"] = round(p["work"] / (p["ms"] * 1e-3) / 1e12, 2)
        else:
            k["GB_s"] = round(p["work"] / (p["ms"] * 1e-3) / 1e9, 1)
        kernels[name] = k

    # Algorithmic HBM bytes of one step's GEMMs (A and W operands, fp32 block scales,
    # fp32 row scales, fp32 output; the gate/up GEMM writes only g = geluquick(gate)*up).
    # Both operands are int8.
    c = mdl.config
    d, ff, T = c["embed_dim"], c["interm_dim"], B * S
    hd = d // c["num_heads"]
    qd, kvd = c["num_heads"] * hd, c["num_kv_heads"] * hd
    def gemm_bytes(N, K, out_cols):
        return T * K + N * K + N * (K // 32) * 4 + T * 4 + T * out_cols * 4

    # The O and down GEMMs run as plain GEMM launches only when the library does
    # not fuse them with the residual post-norm (class "gemm_norm": o is not
    # written; the epilogue reads and writes h, 8 B per element).
    fused = gn["launches"] > 0
    plain_bytes = c["num_layers"] * (gemm_bytes(qd + 2 * kvd, d, qd + 2 * kvd) + gemm_bytes(2 * ff, d, ff) +
                                     (0 if fused else gemm_bytes(d, qd, d) + gemm_bytes(d, ff, d)))
    norm_bytes = c["num_layers"] * (gemm_bytes(d, qd, 0) + gemm_bytes(d, ff, 0) + 2 * 8 * T * d) if fused else 0
    step_gemm_bytes = plain_bytes + norm_bytes
    gemm_gbs = step_gemm_bytes * a.steps / (all_ms * 1e-3) / 1e9 if all_ms > 0 else 0.0

    traffic, traffic_src = None, None  # HBM bytes per GEMM launch, from committed rocprofv3 counter passes
    tp = os.path.join(ROOT, "profiles", "gemm_traffic.json")
    if os.path.exists(tp):
        with open(tp) as f:
            tj = json.load(f)
        traffic = tj.get("traffic_bytes_per_launch_all_gemm")
        traffic_src = (f"committed counter passes ({tj['source']}), not this run: mean HBM bytes per Q8_0 GEMM "
                       f"launch over the plain and the fused GEMM + post-norm launches")

    line = {
        "metric": METRIC,
        "value": round(B * a.steps / dt, 2),
        "unit": "embeddings/sec",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(dt / a.steps * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": "config 2: EmbeddingGemma-300M Q8_0 forward, 64 x 512 tokens",
                   "batch": B, "seq_len": S, "tokens": "U[2,262144) seed 0",
                   "weights": "random Q8_0 (int8 U[-127,127], fp16 |N(0,1e-3)|) seed 5; norms U[0.5,1.5] seed 2"},
        "roofline": {"bound": "mfma", "achieved": round(all_tops, 2), "peak": INT8_PEAK_TOPS,
                     "unit": "TFLOP/s", "frac": round(all_tops / INT8_PEAK_TOPS, 4), "traffic": traffic,
                     "traffic_source": traffic_src,
                     "kernel": ("every Q8_0 GEMM launch: k_gemm_q8_lds (QKV; gate/up + GELU) and k_gemm_q8_resnorm "
                                "(O, down + residual post-norm, epilogue time included); int8 TOP/s" if fused
                                else "k_gemm_q8_lds / k_gemm_q8_rd (all Q8_0 GEMM launches; int8 TOP/s)"),
                     "avg_launch_ms": round(all_ms / max(all_launches, 1), 4),
                     "launches_per_step": all_launches // a.steps,
                     "algorithmic_bytes_per_launch": round(step_gemm_bytes * a.steps / max(all_launches, 1)),
                     "plain_only": {"kernel": "k_gemm_q8_lds (QKV, gate/up + GELU)", "achieved": round(gemm_tops, 2),
                                    "frac": round(gemm_tops / INT8_PEAK_TOPS, 4),
                                    "avg_launch_ms": round(g["ms"] / max(g["launches"], 1), 4)},
                     "hbm_view": {"achieved": round(gemm_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                  "frac": round(gemm_gbs / HBM_PEAK_GBS, 4)}},
        "kernels": kernels,
        "instrumented_ms_per_step": round(dt_prof / a.steps * 1e3, 3),
        "gemm_frac_of_step": round(all_ms / (dt_prof * 1e3), 3),
    }
    if not a.no_extras:
        line["exact_attention"] = exact_attention_leg(model, d_tok, off, d_out, max(2, a.steps // 4), B)
        line["hbm_reference"] = hbm_reference_leg(ctx, B * S)
        line["gemm_issue_floor"] = issue_probe_leg(ctx)
        line["latency"] = small_batch_latency(model)
        line["gemm_c1"] = gemm_c1_leg(ctx)
        line["config3"] = ragged_config_leg(model, 3)
        line["config4"] = ragged_config_leg(model, 4)
    model.close()
    if not a.no_search:
        line["tokenizer"] = tokenizer_leg()
        line["search"] = search_leg(ctx, a.search_vectors, 768, a.search_batch, 10, max(3, a.steps // 2),
                                    not a.no_cpu_baseline, gpu_events=not a.no_gpu_events)
    ctx.close()
    if not a.no_cpu_baseline:
        threads = a.cpu_threads or min(16, os.cpu_count() or 1)
        line["cpu_baseline"] = cpu_baseline(mdl, toks, S, min(threads, B), a.cpu_warmup, a.cpu_runs)
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
