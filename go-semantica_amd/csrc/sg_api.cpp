// sg_api.cpp -- the C ABI of libsemantica_gpu.so: context, model upload and
// repack, the batched forward orchestration and the kernel-seam entry points.
//
// The forward replaces forwardINT8WithDim (internal/runtime/model_int8.go:148-256)
// for a packed batch of sequences.  Per layer the reference op order is kept:
//   RMSNorm -> quantize -> Q/K/V GEMM -> QK-norm -> RoPE -> attention -> quantize
//   -> O GEMM -> post-norm -> +residual -> RMSNorm -> quantize -> gate/up GEMM
//   -> GELUQuick*up -> quantize -> down GEMM -> post-norm -> +residual
// with Q/K/V and gate/up fused into one GEMM each (weights concatenated by
// row; every output column is computed exactly as before) and each
// post-norm + residual fused with the following pre-norm.
#include "semantica_gpu.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdint>
#include <cstdlib>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "sg_internal.h"
#include "sg_kernels.h"

namespace {
thread_local std::string g_err;
}  // namespace

namespace sgi {
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}
}  // namespace sgi

namespace {

using sgi::fail;

using sgi::DevBuf;
using sgi::HostBuf;

// Per-call sequence metadata built on the host from CSR offsets.
struct Meta {
  int T = 0, n_seq = 0, n_items = 0, n_vtiles = 0;
  int Tp = 0;         // V^T columns: every sequence padded to whole 32-key tiles
  int max_len = 0;    // longest sequence
  double sum_sq = 0;  // sum over sequences of S^2 (attention work)
  // Every sequence inside one row-kernel workgroup's rows / one attention
  // work item: the post-norms and the attention then quantize the next GEMM
  // operand themselves (the short-sequence serving case).
  bool seq_in_row_block = false, seq_one_item = false;
  // Every sequence starts on a 32-row boundary (so the QKV GEMM's 32-row
  // subtiles are whole 32-key V^T tiles, except a last sequence's tail).
  bool seq_start32 = false;
  // device views into one buffer
  int32_t* row_seq = nullptr;
  int32_t* row_pos = nullptr;
  int32_t* seq_off = nullptr;
  int32_t* voff = nullptr;   // [n_seq + 1] V^T column of each sequence
  sg_item* items = nullptr;  // attention workgroups (sequence, first chunk)
  sg_item* vtiles = nullptr; // V^T split tiles (sequence, first key)
  int32_t* spill_off = nullptr;  // [n_seq] first attention spill tile of each sequence
  int spill_total = 0;           // attention spill tiles per kv head
};

// Attention workgroups of one sequence: G*ceil(S/16) chunks, kAttnChunks each.
int seq_groups(int S, int G) {
  const int chunks = G * ((S + sgk::kAttnChunkRows - 1) / sgk::kAttnChunkRows);
  return (chunks + sgk::kAttnChunks - 1) / sgk::kAttnChunks;
}

// Fills `host` with [row_seq | row_pos | seq_off | voff | items | vtiles |
// spill_off] and
// copies it to `dev` on stream s, asynchronously: kernels launched on s after
// this see the metadata, and the next stage_meta waits for the copy before it
// rewrites `host`.
// G: query heads per kv head.
//
// Workgroup order.  Workgroup i of a launch runs on XCD i % 8 (the dispatcher
// deals workgroups round-robin over the eight XCDs, each with its own L2), so
// sequences are binned to XCDs (largest first, onto the least-loaded bin) and
// the list interleaves the bins: all workgroups of a sequence then share one
// L2 copy of its K and V^T.
constexpr int kAttnLptItems = 512;  // two rounds of attention workgroups on 256 CUs

int stage_meta(const int32_t* off, int n_seq, int G, HostBuf& host, DevBuf& dev, hipStream_t s, Meta& m) {
  constexpr int kXcd = 8;
  const int T = off[n_seq];
  int n_items = 0, n_vt = 0;
  int64_t n_spill = 0;
  for (int i = 0; i < n_seq; i++) {
    const int S = off[i + 1] - off[i];
    n_items += seq_groups(S, G);
    n_vt += (S + 31) / 32;
    n_spill += (int64_t)seq_groups(S, G) * sgk::attention_spill_tiles(S);
  }
  if (n_spill > INT32_MAX) return fail(SG_ERR_INVALID, "batch too large for the attention spill layout");
  const size_t bytes = sizeof(int32_t) * ((size_t)2 * T + 2 * (n_seq + 1)) +
                       sizeof(sg_item) * ((size_t)n_items + n_vt) + sizeof(int32_t) * (size_t)n_seq + 64;
  SG_TRY(host.ensure(bytes));
  SG_TRY(dev.ensure(bytes));
  int32_t* h = host.as<int32_t>();
  int32_t* rs = h;
  int32_t* rp = rs + T;
  int32_t* so = rp + T;
  int32_t* vo = so + n_seq + 1;
  sg_item* it = reinterpret_cast<sg_item*>(vo + n_seq + 1);
  sg_item* vt = it + n_items;
  int32_t* sp = reinterpret_cast<int32_t*>(vt + n_vt);
  int nv = 0, ns = 0;
  vo[0] = 0;
  for (int i = 0; i < n_seq; i++) {
    const int S = off[i + 1] - off[i];
    so[i] = off[i];
    vo[i + 1] = vo[i] + sgk::attn_key_pad(S);
    for (int r = off[i]; r < off[i + 1]; r++) {
      rs[r] = i;
      rp[r] = r - off[i];
    }
    for (int k0 = 0; k0 < S; k0 += 32) vt[nv++] = sg_item{i, k0};
    sp[i] = ns;
    ns += seq_groups(S, G) * sgk::attention_spill_tiles(S);
  }
  so[n_seq] = off[n_seq];
  {
    std::vector<int> order(n_seq);
    for (int i = 0; i < n_seq; i++) order[i] = i;
    auto work = [&](int i) { return (double)seq_groups(off[i + 1] - off[i], G) * (off[i + 1] - off[i]); };
    std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return work(a) > work(b); });
    std::vector<std::vector<sg_item>> bin(kXcd);
    double load[kXcd] = {};
    for (int i : order) {
      int b = 0;
      for (int x = 1; x < kXcd; x++)
        if (load[x] < load[b]) b = x;
      load[b] += work(i);
      for (int c0 = 0, n = seq_groups(off[i + 1] - off[i], G); c0 < n * sgk::kAttnChunks; c0 += sgk::kAttnChunks)
        bin[b].push_back(sg_item{i, c0});
    }
    size_t pos[kXcd] = {};
    for (int k = 0; k < n_items; k++) {
      int b = k % kXcd;
      if (pos[b] == bin[b].size()) {  // this bin ran dry: take from the fullest one
        for (int x = 0; x < kXcd; x++)
          if (bin[x].size() - pos[x] > bin[b].size() - pos[b]) b = x;
      }
      it[k] = bin[b][pos[b]++];
    }
    // A workgroup's time grows with its sequence's length.  In a launch of at
    // most two rounds (one workgroup per CU) the last round's workgroups set
    // its end, so there the longest go first (stable: equal lengths keep the
    // XCD binning) and the last round holds the short ones.  Longer launches
    // keep the binning, whose shared L2 copies are worth more than the tail.
    if (n_items <= kAttnLptItems)
      std::stable_sort(it, it + n_items, [&](const sg_item& a, const sg_item& b) {
        return off[a.seq + 1] - off[a.seq] > off[b.seq + 1] - off[b.seq];
      });
  }
  SG_HIP(hipMemcpyAsync(dev.p, host.p, bytes, hipMemcpyHostToDevice, s));
  SG_TRY(host.record(s));
  int32_t* d = dev.as<int32_t>();
  m.T = T;
  m.n_seq = n_seq;
  m.sum_sq = 0;
  m.max_len = 0;
  for (int i = 0; i < n_seq; i++) {
    m.sum_sq += (double)(off[i + 1] - off[i]) * (off[i + 1] - off[i]);
    m.max_len = std::max(m.max_len, off[i + 1] - off[i]);
  }
  m.n_items = n_items;
  m.n_vtiles = n_vt;
  m.seq_one_item = n_items == n_seq;
  m.seq_in_row_block = true;
  for (int i = 0; i < n_seq; i++)
    if (off[i + 1] > off[i] && off[i] / sgk::kRowKernelRows != (off[i + 1] - 1) / sgk::kRowKernelRows)
      m.seq_in_row_block = false;
  m.seq_start32 = true;
  for (int i = 0; i < n_seq; i++)
    if (off[i] % 32) m.seq_start32 = false;
  m.Tp = vo[n_seq];
  m.row_seq = d;
  m.row_pos = d + T;
  m.seq_off = d + 2 * T;
  m.voff = d + 2 * T + n_seq + 1;
  m.items = reinterpret_cast<sg_item*>(d + 2 * T + 2 * (n_seq + 1));
  m.vtiles = m.items + n_items;
  m.spill_off = reinterpret_cast<int32_t*>(m.vtiles + n_vt);
  m.spill_total = ns;
  return SG_OK;
}

// Offsets sanity for the kernel seam (sizes only; the model seam applies the
// reference's error cases).
int check_offsets(const int32_t* off, int n_seq, int rows) {
  if (!off || n_seq <= 0) return fail(SG_ERR_INVALID, "seq_offsets must describe at least one sequence");
  if (off[0] != 0) return fail(SG_ERR_INVALID, "seq_offsets[0] must be 0");
  for (int i = 0; i < n_seq; i++)
    if (off[i + 1] < off[i]) return fail(SG_ERR_INVALID, "seq_offsets must be non-decreasing");
  if (rows >= 0 && off[n_seq] != rows)
    return fail(SG_ERR_INVALID, "seq_offsets[n_seq]=%d does not match rows=%d", off[n_seq], rows);
  return SG_OK;
}

// NewRoPECache (internal/kernels/rope_cache.go:15-44): freq_i =
// float32(1/pow(base, 2i/hd)) in float64; theta = float32(p) * freq_i in
// float32; cos/sin evaluated in float64 and rounded to float32.
void rope_tables(int hd, float base, int max_pos, std::vector<float>& c, std::vector<float>& s) {
  const int half = hd / 2;
  std::vector<float> freq(half);
  for (int i = 0; i < half; i++) freq[i] = (float)(1.0 / std::pow((double)base, (double)(2 * i) / (double)hd));
  c.resize((size_t)max_pos * half);
  s.resize((size_t)max_pos * half);
  for (int p = 0; p < max_pos; p++) {
    const float pf = (float)p;
    for (int i = 0; i < half; i++) {
      const float th = pf * freq[i];
      c[(size_t)p * half + i] = (float)std::cos((double)th);
      s[(size_t)p * half + i] = (float)std::sin((double)th);
    }
  }
}

}  // namespace

struct sg_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  std::mutex mu;  // guards the scratch below for the kernel seam
  HostBuf meta_h;
  DevBuf meta_d, a8, amax, tab;
  DevBuf split;  // sg_attention's split operands
  // Last use of a8 (and of a gate weight's gate/up interleave) by an
  // asynchronous GEMM call (sg_matmul_q8_0_int8, sg_ffn_gate_up): the next
  // such call waits for it on its own stream.
  hipEvent_t gemm_done = nullptr;
  bool gemm_pending = false;
};

namespace sgi {
int ctx_device(const sg_ctx* c) { return c->device; }
hipStream_t ctx_stream(const sg_ctx* c, void* stream) {
  return stream ? static_cast<hipStream_t>(stream) : c->stream;
}
}  // namespace sgi

namespace {

struct LayerDev {
  int8_t *wqkv = nullptr, *wo = nullptr, *wgu = nullptr, *wd = nullptr;  // block-major int8 [K/32][N][32]
  float *sqkv = nullptr, *so = nullptr, *sgu = nullptr, *sd = nullptr;
  float *attn_norm = nullptr, *q_norm = nullptr, *k_norm = nullptr;
  float *post_attn = nullptr, *ffn_norm = nullptr, *post_ffw = nullptr;
};

hipStream_t pick(sg_ctx* c, void* stream) { return stream ? static_cast<hipStream_t>(stream) : c->stream; }

// The asynchronous GEMM seam shares the context's operand scratch: a call
// orders its stream after the previous call's last use (GPU-side, no host
// wait) and marks its own.  Growing a scratch buffer synchronizes the device
// before freeing the old one (DevBuf::ensure), so a reallocation never pulls
// memory from under work in flight.
int gemm_scratch_begin(sg_ctx* c, hipStream_t s) {
  if (c->gemm_pending) SG_HIP(hipStreamWaitEvent(s, c->gemm_done, 0));
  return SG_OK;
}
int gemm_scratch_end(sg_ctx* c, hipStream_t s) {
  SG_HIP(hipEventRecord(c->gemm_done, s));
  c->gemm_pending = true;
  return SG_OK;
}

// Held by a GEMM entry point from gemm_scratch_begin on: every return path,
// errors included, orders what the call enqueued on `s` before the next use
// of the context's GEMM scratch (a8, the gate/up interleave).  The success
// path calls finish(); an early return ends the use in the destructor
// without touching the error message already set.  If the event cannot be
// recorded, the stream is drained instead.
struct ScratchUse {
  sg_ctx* c;
  hipStream_t s;
  bool done = false;
  ScratchUse(sg_ctx* c_, hipStream_t s_) : c(c_), s(s_) {}
  ScratchUse(const ScratchUse&) = delete;
  ScratchUse& operator=(const ScratchUse&) = delete;
  int finish() {
    done = true;
    const int r = gemm_scratch_end(c, s);
    if (r != SG_OK) (void)hipStreamSynchronize(s);
    return r;
  }
  ~ScratchUse() {
    if (done) return;
    if (hipEventRecord(c->gemm_done, s) == hipSuccess) c->gemm_pending = true;
    else (void)hipStreamSynchronize(s);
  }
};

int set_device(sg_ctx* c) {
  SG_HIP(hipSetDevice(c->device));
  return SG_OK;
}

}  // namespace

// Event-bracketed launch accounting for sg_profile_* (events are pooled and
// reused across forwards; records are folded in after each forward's sync).
struct Profiler {
  bool on = false;
  std::vector<hipEvent_t> pool;
  size_t used = 0;
  struct Rec {
    int cls;
    hipEvent_t a, b;
    double work;
  };
  std::vector<Rec> recs;
  sg_profile acc{};
  hipEvent_t next() {
    if (used == pool.size()) {
      hipEvent_t e = nullptr;
      if (hipEventCreate(&e) != hipSuccess) return nullptr;
      pool.push_back(e);
    }
    return pool[used++];
  }
  int fold() {
    for (const Rec& r : recs) {
      float ms = 0.f;
      SG_HIP(hipEventElapsedTime(&ms, r.a, r.b));
      acc.ms[r.cls] += ms;
      acc.work[r.cls] += r.work;
      acc.launches[r.cls] += 1;
    }
    recs.clear();
    used = 0;
    return SG_OK;
  }
  ~Profiler() {
    for (hipEvent_t e : pool) (void)hipEventDestroy(e);
  }
};

// One sequence group's forward: activation workspace (grown on demand),
// metadata staging, the token-error flag, and for groups after the first a
// stream of its own (created on first use, non-blocking, default priority) with
// the event that joins it back to the caller's stream.
struct Lane {
  DevBuf h, xn, qkv, att, o, g, a8, sx, amax, meta_d, err;
  DevBuf ks, vt;  // attention operands, hi/lo fp16 (K row-major; V^T); Q is split inside the attention kernel
  DevBuf qs;      // Q hi/lo for launches too small to fill the GPU (attn_q_presplit)
  DevBuf xp;      // exact-order attention: scores / weights [H][T][ldp] (SG_ATTN_EXACT only)
  DevBuf spill;   // attention scores past the kernel's register tiles (sequences > 512 keys)
  HostBuf meta_h, io_h;
  hipStream_t stream = nullptr;
  hipEvent_t done = nullptr;
  int open_stream() {
    if (!stream && hipStreamCreateWithFlags(&stream, hipStreamNonBlocking) != hipSuccess) {
      stream = nullptr;
      return fail(SG_ERR_DEVICE, "hipStreamCreateWithFlags failed");
    }
    if (!done && hipEventCreateWithFlags(&done, hipEventDisableTiming) != hipSuccess) {
      done = nullptr;
      return fail(SG_ERR_DEVICE, "hipEventCreateWithFlags failed");
    }
    return SG_OK;
  }
  ~Lane() {
    for (DevBuf* b : {&h, &xn, &qkv, &att, &o, &g, &a8, &sx, &amax, &meta_d, &err, &ks, &vt, &qs, &xp, &spill})
      b->release();
    meta_h.release();
    io_h.release();
    if (done) (void)hipEventDestroy(done);
    if (stream) (void)hipStreamDestroy(stream);
  }
};

// A large batch runs as up to kLanes sequence groups on as many streams: the
// groups' kernels overlap on the GPU (each kernel's ramp-up and tail filled by
// the other group's work, and at times one group's bandwidth-bound row kernels
// beside the other's GEMMs), with every sequence's arithmetic unchanged.  A
// group gets at least kLaneMinTokens tokens.  Two groups measured best at
// 64 x 512 tokens on MI355X (first: 19.2 ms per batch against 20.1 for one,
// 19.4 for three; with the fused GEMM + residual post-norm kernels: 16.80
// against 17.56 for three; four leave two streams on one of the process's
// four hardware queues and lose to one group).
constexpr int kLanes = 2;
constexpr int kLaneMinTokens = 4096;

struct sg_model {
  sg_ctx* ctx = nullptr;
  Profiler prof;
  sg_model_config cfg{};
  int hd = 0, qd = 0, kvd = 0, nqkv = 0;
  float attn_scale = 0.f, sqrt_d = 0.f;
  std::vector<void*> allocs;
  int8_t* emb_q = nullptr;
  float* emb_s = nullptr;
  float* out_norm = nullptr;
  float *cos_t = nullptr, *sin_t = nullptr;
  std::vector<LayerDev> layers;
  Lane lanes[kLanes];
  hipEvent_t fork = nullptr;  // the caller's stream position the groups start from
  DevBuf tokens, out;         // sg_forward's staging of host tokens and embeddings
  int attn_mode = SG_ATTN_FAST;  // sg_model_set_attention_mode
  std::mutex mu;

  template <typename T>
  int alloc(T** p, size_t count) {
    void* q = nullptr;
    if (hipMalloc(&q, sizeof(T) * count) != hipSuccess) return fail(SG_ERR_NOMEM, "hipMalloc failed (model)");
    allocs.push_back(q);
    *p = static_cast<T*>(q);
    return SG_OK;
  }
  ~sg_model() {
    for (void* p : allocs) (void)hipFree(p);
    tokens.release();
    out.release();
    if (fork) (void)hipEventDestroy(fork);
  }
};

namespace {

int upload_f32(sg_model* m, float** dst, const float* src, int n) {
  if (!src) {
    *dst = nullptr;
    return SG_OK;
  }
  SG_TRY(m->alloc(dst, (size_t)n));
  SG_HIP(hipMemcpy(*dst, src, sizeof(float) * n, hipMemcpyHostToDevice));
  return SG_OK;
}

// Copies one raw Q8_0 matrix through `stage` and repacks it into rows
// [row_off, row_off+rows) of w8 / columns of st.
// grp/gstride: row grouping of repack_q8_0 (0: rows stay contiguous).
int upload_q8(const void* raw, int rows, int cols, DevBuf& stage, int8_t* w8, float* st, int ld_st, int row_off,
              hipStream_t s, int grp = 0, int gstride = 0) {
  if (!raw) return fail(SG_ERR_INVALID, "missing Q8_0 tensor");
  const size_t bytes = (size_t)rows * (cols / 32) * 34;
  SG_TRY(stage.ensure(bytes));
  SG_HIP(hipMemcpyAsync(stage.p, raw, bytes, hipMemcpyHostToDevice, s));
  SG_HIP(sgk::repack_q8_0(stage.as<uint8_t>(), rows, cols, w8, st, ld_st, row_off, grp ? grp : rows, gstride, s));
  SG_HIP(hipStreamSynchronize(s));
  return SG_OK;
}

int validate_config(const sg_model_config& c) {
  if (c.embed_dim <= 0 || c.num_layers <= 0 || c.num_heads <= 0 || c.num_kv_heads <= 0 || c.interm_dim <= 0 ||
      c.max_seq_len <= 0 || c.vocab_size <= 0)
    return fail(SG_ERR_INVALID, "model config has a non-positive dimension");
  if (c.embed_dim % c.num_heads) return fail(SG_ERR_INVALID, "embed_dim %% num_heads != 0");
  const int hd = c.embed_dim / c.num_heads;
  if (hd != 256) return fail(SG_ERR_INVALID, "head_dim %d unsupported (kernels are built for 256)", hd);
  if (c.num_heads % c.num_kv_heads || c.num_heads / c.num_kv_heads > 4)
    return fail(SG_ERR_INVALID, "num_heads/num_kv_heads must be an integer <= 4");
  if (c.embed_dim != 256 && c.embed_dim != 512 && c.embed_dim != 768 && c.embed_dim != 1024)
    return fail(SG_ERR_INVALID, "embed_dim %d unsupported (256/512/768/1024)", c.embed_dim);
  if (c.interm_dim % 32) return fail(SG_ERR_INVALID, "feed_forward_length must be a multiple of 32");
  return SG_OK;
}

// Launch wrapper: with profiling on, brackets the launch with events on `s`.
#define SG_LAUNCH(cls, work, call)                                   \
  do {                                                               \
    hipEvent_t a_ = nullptr;                                         \
    if (m->prof.on && (a_ = m->prof.next())) SG_HIP(hipEventRecord(a_, s)); \
    SG_HIP(call);                                                    \
    if (a_) {                                                        \
      hipEvent_t b_ = m->prof.next();                                \
      if (b_) {                                                      \
        SG_HIP(hipEventRecord(b_, s));                               \
        m->prof.recs.push_back(Profiler::Rec{cls, a_, b_, (double)(work)}); \
      }                                                              \
    }                                                                \
  } while (0)

// The per-layer launch sequence.  amax sites per layer: 0 pre-attention
// norm, 1 attention output, 2 pre-FFN norm, 3 GELU*up; each [n_seq].
// Work figures are the algorithmic ones: 2*M*N*K int8 ops per GEMM,
// 4*H*hd*S^2 flops per sequence for attention, and bytes read + written at
// the reference's dtypes (fp32 activations, int8 quantized) elsewhere.
// Per-layer copies for sg_forward_trace: layer l's rows at l * T rows.
struct Trace {
  float *qkv = nullptr, *att = nullptr, *h = nullptr;
};

// Attention launches of fewer workgroups than the GPU has CUs run latency-
// bound, and there the in-kernel Q prologue (one memory round trip, the QK-norm
// through the LDS tile, RoPE, the split: over half of a 32-token sequence's
// workgroup) is on the critical path.  Such launches take Q pre-split from
// k_kv_prep (the same arithmetic, bit-identical operands), which prepares it
// over many more threads; larger launches keep the prologue, which saves
// writing Q's operands and reading them back.
constexpr int kAttnQPresplitItems = 256;
bool attn_q_presplit(const sg_model* m, const Meta& meta) {
  return m->attn_mode != SG_ATTN_EXACT && (int64_t)meta.n_items * m->cfg.num_kv_heads < kAttnQPresplitItems;
}

// Layers [l0, l1) of one sequence group's forward on lane w, stream s: the
// embedding first when l0 == 0, the pooled embeddings into d_out after the
// last layer.  stop >= 0: return after `stop` layers with the residual stream
// copied to d_out (when non-null).  tr: per-layer copies of the first `stop`
// layers.
int run_forward(sg_model* m, Lane& w, const int32_t* d_tokens, const Meta& meta, int out_dim, float* d_out,
                hipStream_t s, int l0, int l1, int stop = -1, const Trace* tr = nullptr) {
  const sg_model_config& c = m->cfg;
  const int T = meta.T, ns = meta.n_seq, d = c.embed_dim, ff = c.interm_dim, L = c.num_layers;
  const int qd = m->qd, kvd = m->kvd, nqkv = m->nqkv;
  float* h = w.h.as<float>();
  float* xn = w.xn.as<float>();
  float* qkv = w.qkv.as<float>();
  float* att = w.att.as<float>();
  float* o = w.o.as<float>();
  float* g = w.g.as<float>();
  int8_t* a8 = w.a8.as<int8_t>();
  const int ar = sgk::gemm_pad_rows(T);
  _Float16* ks_h = w.ks.as<_Float16>();
  _Float16* ks_l = ks_h + (size_t)T * kvd;
  _Float16* vt_h = w.vt.as<_Float16>();
  const int ldvt = 2 * meta.Tp;  // per dim: each 32-key tile's hi then lo halves
  float* sx = w.sx.as<float>();
  float* amax = w.amax.as<float>();
  auto site = [&](int l, int k) { return amax + ((size_t)4 * l + k) * ns; };
  const float eps = c.norm_eps;
  const double t = T;
  auto gemm_ops = [&](int N, int K) { return 2.0 * t * N * K; };
  auto quant_bytes = [&](int K) { return t * K * 5.0; };
  const double attn_flops = 4.0 * c.num_heads * m->hd * meta.sum_sq;
  const double attn_bytes = t * (2.0 * qd + 2.0 * kvd) * 4.0;
  (void)attn_bytes;
  auto norm_q = [&](const float* w, float* am) {
    return sgk::norm_quantize(h, w, eps, T, d, meta.row_seq, am, a8, ar, sx, s);
  };
  auto quant = [&](const float* x, int cols, float* am) {
    return sgk::quantize(x, cols, T, cols, meta.row_seq, am, a8, ar, nullptr, sx, s);
  };
  auto tap = [&](float* dst, const float* src, int l, int cols) {
    return hipMemcpyAsync(dst + (size_t)l * T * cols, src, sizeof(float) * (size_t)T * cols, hipMemcpyDeviceToDevice,
                          s);
  };
  auto gemm = [&](const int8_t* w8, const float* st, float* y, int N, int K) {
    return sgk::gemm_q8(a8, ar, w8, st, sx, y, nullptr, T, N, K, s, true);
  };
  // The QKV GEMM writes V straight into the attention's V^T operand (the
  // direct-to-LDS kernels' epilogue), so k_kv_prep only prepares K: for
  // batches whose sequences all start on 32-row boundaries, where the
  // epilogue's subtiles are whole key tiles (other subtiles go out value by
  // value: for 256 ragged sequences of 8-512 tokens the GEMM class then took
  // 8.1 instead of 6.4 ms per forward, far more than k_kv_prep's V half
  // saves).  Not in exact mode
  // (its attention reads V in fp32) nor when Q|K|V is traced.
  const bool vt_fused = m->attn_mode != SG_ATTN_EXACT && !(tr && tr->qkv) && sgk::gemm_writes_vt(T) &&
                        meta.seq_start32;
  const sgk::sg_vt_out vto{vt_h, ldvt, qd + kvd, meta.row_seq, meta.seq_off, meta.voff};
  // Small attention launches take Q pre-split by k_kv_prep (attn_q_presplit).
  const bool q_pre = attn_q_presplit(m, meta);
  _Float16* qs_h = q_pre ? w.qs.as<_Float16>() : nullptr;
  _Float16* qs_l = q_pre ? qs_h + (size_t)T * qd : nullptr;

  if (l0 == 0) {
    SG_LAUNCH(SG_K_OTHER, 4.0 * 4 * L * ns, sgk::fill_f32(amax, 0.0f, (int64_t)4 * L * ns, s));
    // V^T positions past each sequence's end stay zero through the layers
    // (the fused epilogue writes only the sequences' keys).
    if (vt_fused)
      SG_LAUNCH(SG_K_OTHER, 4.0 * kvd * meta.Tp,
                sgk::fill_i32(reinterpret_cast<int32_t*>(vt_h), 0, (int64_t)kvd * meta.Tp, s));
    SG_LAUNCH(SG_K_OTHER, 4.0, sgk::fill_i32(w.err.as<int32_t>(), INT32_MAX, 1, s));
    SG_LAUNCH(SG_K_NORM, t * (34.0 * d / 32 + 4.0 * d),
              sgk::embed_norm(d_tokens, T, m->emb_q, m->emb_s, c.vocab_size, d, m->sqrt_d, m->layers[0].attn_norm,
                              eps, meta.row_seq, h, nullptr, site(0, 0), w.err.as<int32_t>(), s));
  }
  // Short sequences (each inside one row-kernel workgroup / attention item):
  // the unfused post-norms quantize the next GEMM operand in the same launch,
  // and the attention its own output, so the separate quantizer launches go.
  // a8_ready: the operand of the next QKV GEMM is already in a8.
  const bool q_rows = meta.seq_in_row_block;
  const bool q_attn = meta.seq_one_item && c.num_kv_heads == 1 && meta.max_len <= sgk::kAttnRegKeys;
  bool a8_ready = false;
  auto post_norm_q = [&](const float* w_post, const float* w_next, float* am) {
    return sgk::post_res_norm_quantize(o, h, w_post, w_next, eps, T, d, meta.row_seq, am, a8, ar, sx, s);
  };
  for (int l = l0; l < l1; l++) {
    if (l == stop) break;
    const LayerDev& ly = m->layers[l];
    // The pre-norm's output xn is never stored: recomputed from h while quantizing.
    if (!a8_ready) SG_LAUNCH(SG_K_QUANTIZE, quant_bytes(d), norm_q(ly.attn_norm, site(l, 0)));
    a8_ready = false;
    SG_LAUNCH(SG_K_GEMM, gemm_ops(nqkv, d),
              sgk::gemm_q8(a8, ar, ly.wqkv, ly.sqkv, sx, qkv, nullptr, T, nqkv, d, s, true, vt_fused ? &vto : nullptr));
    if (tr && tr->qkv) SG_HIP(tap(tr->qkv, qkv, l, nqkv));
    if (m->attn_mode == SG_ATTN_EXACT) {
      // The reference's float32 order throughout: QK-norm + RoPE in place on
      // the QKV output, then the VALU attention (which folds the sequences'
      // max|o| into amax for the quantizer).
      SG_LAUNCH(SG_K_NORM, t * (qd + kvd) * 8.0,
                sgk::qknorm_rope(qkv, nqkv, qkv + qd, nqkv, ly.q_norm, ly.k_norm, c.num_heads, c.num_kv_heads, T,
                                 meta.row_pos, m->cos_t, m->sin_t, eps, nullptr, nullptr, 0, nullptr, nullptr, 0, s));
      SG_LAUNCH(SG_K_ATTENTION, attn_flops,
                sgk::attention_exact(qkv, nqkv, qkv + qd, qkv + qd + kvd, nqkv, att, qd, meta.seq_off, meta.row_seq,
                                     ns, T, c.num_heads, c.num_kv_heads, m->hd, m->attn_scale, meta.max_len,
                                     w.xp.as<float>(), site(l, 1), s));
    } else {
      // K's QK-norm + RoPE + split and V's V^T split in one launch; Q's norm and
      // RoPE run inside the attention kernel.
      const sgk::sg_kv_q qpart{qkv, nqkv, ly.q_norm, c.num_heads, qs_h, qs_l, qd};
      SG_LAUNCH(SG_K_NORM, t * ((vt_fused ? 8.0 : 16.0) * kvd + (q_pre ? 8.0 * qd : 0.0)),
                sgk::kv_prep(qkv + qd, qkv + qd + kvd, nqkv, ly.k_norm, c.num_kv_heads, T, meta.row_pos, m->cos_t,
                             m->sin_t, eps, ks_h, ks_l, kvd, meta.seq_off, meta.voff, meta.vtiles,
                             vt_fused ? 0 : meta.n_vtiles, vt_h, ldvt, s, q_pre ? &qpart : nullptr));
      const sg_attn_qpre qpre{qkv, nqkv, ly.q_norm, m->cos_t, m->sin_t, eps};
      const sg_attn_qout qout{a8, ar, sx};
      const sg_attn_spill spill{w.spill.as<float>(), meta.spill_off, meta.spill_total};
      SG_LAUNCH(SG_K_ATTENTION, attn_flops,
                sgk::attention(q_pre ? qs_h : nullptr, q_pre ? qs_l : nullptr, q_pre ? qd : 0, ks_h, ks_l, kvd, vt_h,
                               ldvt, att, qd, meta.seq_off, meta.voff, meta.items, meta.n_items, c.num_heads,
                               c.num_kv_heads, m->hd, m->attn_scale, site(l, 1), meta.max_len, s,
                               q_pre ? nullptr : &qpre, q_attn ? &qout : nullptr, &spill));
    }
    if (tr && tr->att) SG_HIP(tap(tr->att, att, l, qd));
    if (!(q_attn && m->attn_mode != SG_ATTN_EXACT))
      SG_LAUNCH(SG_K_QUANTIZE, quant_bytes(qd), quant(att, qd, site(l, 1)));
    // The O projection and the residual post-norm: one launch for large
    // batches (o stays on chip), else the GEMM then k_post_res_norm.
    if (sgk::gemm_res_norm_fused(T, d, ly.post_attn, ly.ffn_norm)) {
      SG_LAUNCH(SG_K_GEMM_NORM, gemm_ops(d, qd),
                sgk::gemm_q8_res_norm(a8, ar, ly.wo, ly.so, sx, o, T, d, qd, h, ly.post_attn, ly.ffn_norm, eps,
                                      nullptr, meta.row_seq, site(l, 2), s));
    } else if (q_rows) {
      SG_LAUNCH(SG_K_GEMM, gemm_ops(d, qd), gemm(ly.wo, ly.so, o, d, qd));
      SG_LAUNCH(SG_K_NORM, t * d * 13.0, post_norm_q(ly.post_attn, ly.ffn_norm, site(l, 2)));
    } else {
      SG_LAUNCH(SG_K_GEMM, gemm_ops(d, qd), gemm(ly.wo, ly.so, o, d, qd));
      SG_LAUNCH(SG_K_NORM, t * d * 12.0,
                sgk::post_res_norm(o, h, ly.post_attn, ly.ffn_norm, eps, T, d, nullptr, meta.row_seq, site(l, 2), s));
    }
    if (!(q_rows && !sgk::gemm_res_norm_fused(T, d, ly.post_attn, ly.ffn_norm)))
      SG_LAUNCH(SG_K_QUANTIZE, quant_bytes(d), norm_q(ly.ffn_norm, site(l, 2)));
    SG_LAUNCH(SG_K_GEMM, gemm_ops(2 * ff, d),
              sgk::gemm_q8_gelu(a8, ar, ly.wgu, ly.sgu, sx, g, T, ff, d, meta.row_seq, site(l, 3), s, true));
    SG_LAUNCH(SG_K_QUANTIZE, quant_bytes(ff), quant(g, ff, site(l, 3)));
    const bool last = l + 1 == L;
    const float* w_next = last ? m->out_norm : m->layers[l + 1].attn_norm;
    if (sgk::gemm_res_norm_fused(T, d, ly.post_ffw, w_next)) {
      SG_LAUNCH(SG_K_GEMM_NORM, gemm_ops(d, ff),
                sgk::gemm_q8_res_norm(a8, ar, ly.wd, ly.sd, sx, o, T, d, ff, h, ly.post_ffw, w_next, eps,
                                      last ? xn : nullptr, meta.row_seq, last ? nullptr : site(l + 1, 0), s));
    } else if (q_rows && !last) {
      SG_LAUNCH(SG_K_GEMM, gemm_ops(d, ff), gemm(ly.wd, ly.sd, o, d, ff));
      SG_LAUNCH(SG_K_NORM, t * d * 13.0, post_norm_q(ly.post_ffw, w_next, site(l + 1, 0)));
      a8_ready = true;
    } else {
      SG_LAUNCH(SG_K_GEMM, gemm_ops(d, ff), gemm(ly.wd, ly.sd, o, d, ff));
      SG_LAUNCH(SG_K_NORM, t * d * (last ? 16.0 : 12.0),
                sgk::post_res_norm(o, h, ly.post_ffw, w_next, eps, T, d, last ? xn : nullptr, meta.row_seq,
                                   last ? nullptr : site(l + 1, 0), s));
    }
    if (tr && tr->h) SG_HIP(tap(tr->h, h, l, d));
  }
  if (stop >= 0) {
    if (d_out) SG_HIP(hipMemcpyAsync(d_out, h, sizeof(float) * (size_t)T * d, hipMemcpyDeviceToDevice, s));
    return SG_OK;
  }
  if (l1 == L)
    SG_LAUNCH(SG_K_POOL, 4.0 * out_dim * (t + ns), sgk::pool_l2(d_out, xn, d, out_dim, meta.seq_off, ns, s));
  return SG_OK;
}

// Reference error cases.  ForwardWithDim (model.go:661-667) checks the
// dimension first; then every request carries its own error
// (forwardINT8WithDim, model_int8.go:150-171: empty, too long, then its first
// out-of-range token) and embedPrompts returns the first request's error in
// request order (api.go:286-292).  Here: the dimension and the offsets'
// shape, then *len_err_seq = the first sequence that is empty or too long
// (n_seq if none).  Token errors of the sequences before it come first; the
// caller checks them on the device.
int check_forward_args(const sg_model* m, const int32_t* off, int n_seq, int out_dim, int* len_err_seq) {
  const sg_model_config& c = m->cfg;
  if (out_dim <= 0 || out_dim > c.embed_dim)
    return fail(SG_ERR_DIM, "target dimension %d out of range (1..%d)", out_dim, c.embed_dim);
  if (!off || n_seq <= 0) return fail(SG_ERR_INVALID, "no sequences");
  if (off[0] != 0) return fail(SG_ERR_INVALID, "seq_offsets[0] must be 0");
  for (int i = 0; i < n_seq; i++)
    if (off[i + 1] < off[i]) return fail(SG_ERR_INVALID, "seq_offsets must be non-decreasing");
  *len_err_seq = n_seq;
  for (int i = 0; i < n_seq; i++) {
    const int S = off[i + 1] - off[i];
    if (S == 0 || S > c.max_seq_len) {
      *len_err_seq = i;
      break;
    }
  }
  return SG_OK;
}

int length_error(const sg_model* m, int S) {
  if (S == 0) return fail(SG_ERR_EMPTY, "empty input");
  return fail(SG_ERR_TOO_LONG, "sequence too long: %d > %d", S, m->cfg.max_seq_len);
}

// *row (device, written by an embedding kernel or first_bad_token; a row of
// d_tokens) -> the reference's message with the offending id, or SG_OK when
// no row was recorded.
int token_error(Lane& w, const int32_t* d_tokens, hipStream_t s) {
  SG_TRY(w.io_h.ensure(64));
  int32_t* h = w.io_h.as<int32_t>();
  SG_HIP(hipMemcpyAsync(h, w.err.p, sizeof(int32_t), hipMemcpyDeviceToHost, s));
  SG_HIP(hipStreamSynchronize(s));
  if (h[0] == INT32_MAX) return SG_OK;
  const int32_t row = h[0];
  SG_HIP(hipMemcpyAsync(h + 1, d_tokens + row, sizeof(int32_t), hipMemcpyDeviceToHost, s));
  SG_HIP(hipStreamSynchronize(s));
  return fail(SG_ERR_TOKEN, "token ID out of range: %d", h[1]);
}


int ensure_workspace(const sg_model* m, Lane& w, const Meta& meta) {
  const int T = meta.T, n_seq = meta.n_seq, Tp = meta.Tp;
  const sg_model_config& c = m->cfg;
  const size_t t = (size_t)T;
  const int amax_cols = c.embed_dim > c.interm_dim ? c.embed_dim : c.interm_dim;
  const int a_cols = amax_cols > m->qd ? amax_cols : m->qd;
  SG_TRY(w.h.ensure(sizeof(float) * t * c.embed_dim));
  SG_TRY(w.xn.ensure(sizeof(float) * t * c.embed_dim));
  SG_TRY(w.qkv.ensure(sizeof(float) * t * m->nqkv));
  SG_TRY(w.att.ensure(sizeof(float) * t * m->qd));
  SG_TRY(w.o.ensure(sizeof(float) * t * c.embed_dim));
  SG_TRY(w.g.ensure(sizeof(float) * t * c.interm_dim));
  SG_TRY(w.a8.ensure((size_t)sgk::gemm_pad_rows(T) * a_cols));
  if (attn_q_presplit(m, meta)) SG_TRY(w.qs.ensure(2 * sizeof(_Float16) * t * m->qd));
  SG_TRY(w.sx.ensure(sizeof(float) * t));
  SG_TRY(w.amax.ensure(sizeof(float) * 4 * (size_t)c.num_layers * n_seq));
  SG_TRY(w.ks.ensure(2 * sizeof(_Float16) * t * m->kvd));
  SG_TRY(w.vt.ensure(2 * sizeof(_Float16) * (size_t)m->kvd * Tp));
  SG_TRY(w.err.ensure(64));
  if (m->attn_mode == SG_ATTN_EXACT)
    SG_TRY(w.xp.ensure(sgk::attention_exact_scratch(T, c.num_heads, meta.max_len)));
  else
    SG_TRY(w.spill.ensure((size_t)c.num_kv_heads * meta.spill_total * sgk::kAttnSpillTileBytes));
  return SG_OK;
}

// Splits sequences [0, n_seq) into G contiguous groups [b[g], b[g+1]), each
// non-empty, with boundaries at the sequence edges nearest to g * T / G.
void lane_split(const int32_t* off, int n_seq, int G, int* b) {
  const int64_t T = off[n_seq];
  b[0] = 0;
  b[G] = n_seq;
  for (int g = 1; g < G; g++) {
    const int64_t target = T * g / G;
    int k = b[g - 1] + 1;
    while (k < n_seq - (G - g) && std::llabs((int64_t)off[k + 1] - target) <= std::llabs((int64_t)off[k] - target)) k++;
    b[g] = k;
  }
}

int forward_device_locked(sg_model* m, const int32_t* d_tokens, const int32_t* off, int n_seq, int out_dim,
                          float* d_out, hipStream_t s, int stop = -1, const Trace* tr = nullptr) {
  int len_err_seq = n_seq;
  SG_TRY(check_forward_args(m, off, n_seq, out_dim, &len_err_seq));
  SG_TRY(set_device(m->ctx));
  Lane& w0 = m->lanes[0];
  if (len_err_seq < n_seq) {  // the tokens of the sequences before it decide first
    SG_TRY(w0.err.ensure(64));
    SG_HIP(sgk::fill_i32(w0.err.as<int32_t>(), INT32_MAX, 1, s));
    SG_HIP(sgk::first_bad_token(d_tokens, off[len_err_seq], m->cfg.vocab_size, w0.err.as<int32_t>(), s));
    SG_TRY(token_error(w0, d_tokens, s));
    return length_error(m, off[len_err_seq + 1] - off[len_err_seq]);
  }
  const int T = off[n_seq], L = m->cfg.num_layers, GQ = m->cfg.num_heads / m->cfg.num_kv_heads;
  // Sequence groups: one for the per-layer and profiled paths (their outputs
  // and timings cover the whole batch in order), else up to kLanes.
  int G = 1;
  if (stop < 0 && !tr && !m->prof.on) G = std::max(1, std::min(std::min(kLanes, n_seq), T / kLaneMinTokens));
  int b[kLanes + 1];
  lane_split(off, n_seq, G, b);
  hipStream_t st[kLanes];
  st[0] = s;
  if (G > 1) {
    if (!m->fork && hipEventCreateWithFlags(&m->fork, hipEventDisableTiming) != hipSuccess) {
      m->fork = nullptr;
      return fail(SG_ERR_DEVICE, "hipEventCreateWithFlags failed");
    }
    SG_HIP(hipEventRecord(m->fork, s));  // the groups start after the caller's prior work on s
    for (int g = 1; g < G; g++) {
      SG_TRY(m->lanes[g].open_stream());
      st[g] = m->lanes[g].stream;
      SG_HIP(hipStreamWaitEvent(st[g], m->fork, 0));
    }
  }
  Meta meta[kLanes];
  std::vector<int32_t> sub;
  for (int g = 0; g < G; g++) {
    const int n = b[g + 1] - b[g];
    sub.resize(n + 1);
    for (int i = 0; i <= n; i++) sub[i] = off[b[g] + i] - off[b[g]];
    Lane& w = m->lanes[g];
    SG_TRY(stage_meta(sub.data(), n, GQ, w.meta_h, w.meta_d, st[g], meta[g]));
    SG_TRY(ensure_workspace(m, w, meta[g]));
  }
  int rc = SG_OK;
  if (G == 1) {
    rc = run_forward(m, w0, d_tokens, meta[0], out_dim, d_out, s, 0, L, stop, tr);
  } else {
    // Each group's ~20 launches per layer go out from a host thread of its
    // own (the calling thread takes the first group): one thread issuing every
    // group's launches cannot keep up with the GPU.
    int lrc[kLanes] = {};
    std::string lmsg[kLanes];
    auto group = [&](int g) {
      int r = set_device(m->ctx);
      if (r == SG_OK)
        r = run_forward(m, m->lanes[g], d_tokens + off[b[g]], meta[g], out_dim, d_out + (size_t)b[g] * out_dim,
                        st[g], 0, L);
      if (r == SG_OK && g > 0 && hipEventRecord(m->lanes[g].done, st[g]) != hipSuccess)
        r = fail(SG_ERR_DEVICE, "hipEventRecord failed (sequence group %d)", g);
      lrc[g] = r;
      if (r != SG_OK) lmsg[g] = g_err;  // this thread's message
    };
    std::vector<std::thread> th;
    th.reserve(G - 1);
    for (int g = 1; g < G; g++) th.emplace_back(group, g);
    group(0);
    for (std::thread& x : th) x.join();
    for (int g = 0; g < G && rc == SG_OK; g++)
      if (lrc[g] != SG_OK) rc = fail(lrc[g], "%s", lmsg[g].c_str());
    for (int g = 1; g < G && rc == SG_OK; g++)
      if (hipStreamWaitEvent(s, m->lanes[g].done, 0) != hipSuccess)
        rc = fail(SG_ERR_DEVICE, "joining sequence group %d failed", g);
  }
  if (rc != SG_OK) {  // nothing of this call may still run when it returns
    for (int g = 0; g < G; g++) (void)hipStreamSynchronize(st[g]);
    return rc;
  }
  SG_HIP(hipStreamSynchronize(s));
  if (m->prof.on) SG_TRY(m->prof.fold());
  // Token errors in request order: the first group with one holds the first
  // failing sequence.
  for (int g = 0; g < G; g++) SG_TRY(token_error(m->lanes[g], d_tokens + off[b[g]], s));
  return SG_OK;
}

}  // namespace

extern "C" {

const char* sg_last_error(void) { return g_err.c_str(); }
int sg_abi_version(void) { return SG_ABI_VERSION; }

int sg_init(int device_ordinal, sg_ctx** out) {
  if (!out) return fail(SG_ERR_INVALID, "out is NULL");
  *out = nullptr;
  int n = 0;
  SG_HIP(hipGetDeviceCount(&n));
  if (device_ordinal < 0 || device_ordinal >= n)
    return fail(SG_ERR_INVALID, "device %d out of range (%d devices)", device_ordinal, n);
  SG_HIP(hipSetDevice(device_ordinal));
  SG_TRY(sgi::noalloc_setup(device_ordinal));
  sg_ctx* c = new sg_ctx;
  c->device = device_ordinal;
  // A blocking stream (default flags and priority): it orders with the legacy
  // default stream, so callers that stage data there need no extra sync.
  if (hipStreamCreate(&c->stream) != hipSuccess) {
    delete c;
    return fail(SG_ERR_DEVICE, "hipStreamCreate failed");
  }
  if (hipEventCreateWithFlags(&c->gemm_done, hipEventDisableTiming) != hipSuccess) {
    (void)hipStreamDestroy(c->stream);
    delete c;
    return fail(SG_ERR_DEVICE, "hipEventCreateWithFlags failed");
  }
  *out = c;
  return SG_OK;
}

void sg_shutdown(sg_ctx* c) {
  if (!c) return;
  (void)hipSetDevice(c->device);
  (void)hipStreamSynchronize(c->stream);
  c->meta_h.release();
  c->meta_d.release();
  c->a8.release();
  c->amax.release();
  c->tab.release();
  c->split.release();
  (void)hipEventDestroy(c->gemm_done);
  (void)hipStreamDestroy(c->stream);
  delete c;
}

int sg_model_load(sg_ctx* ctx, const sg_model_desc* desc, sg_model** out) {
  if (!ctx || !desc || !out) return fail(SG_ERR_INVALID, "NULL argument");
  *out = nullptr;
  SG_TRY(validate_config(desc->config));
  if (!desc->token_embd || !desc->layers) return fail(SG_ERR_INVALID, "token_embd and layers are required");
  SG_TRY(set_device(ctx));
  sg_model* m = new sg_model;
  m->ctx = ctx;
  m->cfg = desc->config;
  const sg_model_config& c = m->cfg;
  m->hd = c.embed_dim / c.num_heads;
  m->qd = c.num_heads * m->hd;
  m->kvd = c.num_kv_heads * m->hd;
  m->nqkv = m->qd + 2 * m->kvd;
  m->attn_scale = 1.0f / (float)std::sqrt((double)m->hd);  // parseConfig model.go:475
  m->sqrt_d = (float)std::sqrt((double)c.embed_dim);       // model_int8.go:181
  hipStream_t s = ctx->stream;
  DevBuf stage;
  auto done = [&](int r) {
    stage.release();
    if (r != SG_OK) delete m;
    return r;
  };
  const int d = c.embed_dim, ff = c.interm_dim, qd = m->qd, kvd = m->kvd;
  int r;
  // token table
  if ((r = m->alloc(&m->emb_q, (size_t)c.vocab_size * d)) || (r = m->alloc(&m->emb_s, (size_t)c.vocab_size * (d / 32))))
    return done(r);
  {
    const size_t bytes = (size_t)c.vocab_size * (d / 32) * 34;
    if ((r = stage.ensure(bytes))) return done(r);
    if (hipMemcpy(stage.p, desc->token_embd, bytes, hipMemcpyHostToDevice) != hipSuccess)
      return done(fail(SG_ERR_DEVICE, "token_embd upload failed"));
    if (sgk::repack_embd(stage.as<uint8_t>(), c.vocab_size, d, m->emb_q, m->emb_s, s) != hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess)
      return done(fail(SG_ERR_DEVICE, "token_embd repack failed"));
  }
  if ((r = upload_f32(m, &m->out_norm, desc->output_norm, d))) return done(r);
  {
    std::vector<float> ct, st;
    rope_tables(m->hd, c.rope_base, c.max_seq_len, ct, st);
    if ((r = m->alloc(&m->cos_t, ct.size())) || (r = m->alloc(&m->sin_t, st.size()))) return done(r);
    if (hipMemcpy(m->cos_t, ct.data(), sizeof(float) * ct.size(), hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(m->sin_t, st.data(), sizeof(float) * st.size(), hipMemcpyHostToDevice) != hipSuccess)
      return done(fail(SG_ERR_DEVICE, "rope table upload failed"));
  }
  m->layers.resize(c.num_layers);
  for (int l = 0; l < c.num_layers; l++) {
    const sg_layer_desc& ld = desc->layers[l];
    LayerDev& ly = m->layers[l];
    const int nqkv = m->nqkv;
    if ((r = m->alloc(&ly.wqkv, (size_t)nqkv * d)) || (r = m->alloc(&ly.sqkv, (size_t)(d / 32) * nqkv)) ||
        (r = m->alloc(&ly.wo, (size_t)d * qd)) || (r = m->alloc(&ly.so, (size_t)(qd / 32) * d)) ||
        (r = m->alloc(&ly.wgu, (size_t)2 * ff * d)) || (r = m->alloc(&ly.sgu, (size_t)(d / 32) * 2 * ff)) ||
        (r = m->alloc(&ly.wd, (size_t)d * ff)) || (r = m->alloc(&ly.sd, (size_t)(ff / 32) * d)))
      return done(r);
    if ((r = upload_q8(ld.attn_q, qd, d, stage, ly.wqkv, ly.sqkv, nqkv, 0, s)) ||
        (r = upload_q8(ld.attn_k, kvd, d, stage, ly.wqkv, ly.sqkv, nqkv, qd, s)) ||
        (r = upload_q8(ld.attn_v, kvd, d, stage, ly.wqkv, ly.sqkv, nqkv, qd + kvd, s)) ||
        (r = upload_q8(ld.attn_output, d, qd, stage, ly.wo, ly.so, d, 0, s)) ||
        // gate and up interleaved in groups of 32 rows for the fused GELU GEMM
        (r = upload_q8(ld.ffn_gate, ff, d, stage, ly.wgu, ly.sgu, 2 * ff, 0, s, sgk::kGeluGroup,
                       2 * sgk::kGeluGroup)) ||
        (r = upload_q8(ld.ffn_up, ff, d, stage, ly.wgu, ly.sgu, 2 * ff, sgk::kGeluGroup, s, sgk::kGeluGroup,
                       2 * sgk::kGeluGroup)) ||
        (r = upload_q8(ld.ffn_down, d, ff, stage, ly.wd, ly.sd, d, 0, s)))
      return done(r);
    if (!ld.attn_norm || !ld.ffn_norm) return done(fail(SG_ERR_INVALID, "layer %d: attn_norm/ffn_norm required", l));
    if ((r = upload_f32(m, &ly.attn_norm, ld.attn_norm, d)) || (r = upload_f32(m, &ly.q_norm, ld.attn_q_norm, m->hd)) ||
        (r = upload_f32(m, &ly.k_norm, ld.attn_k_norm, m->hd)) ||
        (r = upload_f32(m, &ly.post_attn, ld.post_attention_norm, d)) ||
        (r = upload_f32(m, &ly.ffn_norm, ld.ffn_norm, d)) || (r = upload_f32(m, &ly.post_ffw, ld.post_ffw_norm, d)))
      return done(r);
  }
  *out = m;
  return done(SG_OK);
}

void sg_model_free(sg_model* m) {
  if (!m) return;
  (void)hipSetDevice(m->ctx->device);
  (void)hipDeviceSynchronize();
  delete m;
}

int sg_forward_device(sg_model* m, const int32_t* d_tokens, const int32_t* seq_offsets, int32_t n_seq,
                      int32_t out_dim, float* d_out, void* stream) {
  if (!m || !d_tokens || !d_out) return fail(SG_ERR_INVALID, "NULL argument");
  std::lock_guard<std::mutex> lk(m->mu);
  return forward_device_locked(m, d_tokens, seq_offsets, n_seq, out_dim, d_out, pick(m->ctx, stream));
}

int sg_forward_hidden(sg_model* m, const int32_t* d_tokens, const int32_t* seq_offsets, int32_t n_seq,
                      int32_t n_layers, float* d_hidden, void* stream) {
  if (!m || !d_tokens || !d_hidden) return fail(SG_ERR_INVALID, "NULL argument");
  if (n_layers < 0 || n_layers > m->cfg.num_layers)
    return fail(SG_ERR_INVALID, "n_layers %d out of range (0..%d)", n_layers, m->cfg.num_layers);
  std::lock_guard<std::mutex> lk(m->mu);
  return forward_device_locked(m, d_tokens, seq_offsets, n_seq, m->cfg.embed_dim, d_hidden, pick(m->ctx, stream),
                               n_layers);
}

int sg_forward_trace(sg_model* m, const int32_t* d_tokens, const int32_t* seq_offsets, int32_t n_seq,
                     int32_t n_layers, float* d_qkv, float* d_att, float* d_h, void* stream) {
  if (!m || !d_tokens) return fail(SG_ERR_INVALID, "NULL argument");
  if (n_layers < 1 || n_layers > m->cfg.num_layers)
    return fail(SG_ERR_INVALID, "n_layers %d out of range (1..%d)", n_layers, m->cfg.num_layers);
  std::lock_guard<std::mutex> lk(m->mu);
  Trace tr;
  tr.qkv = d_qkv;
  tr.att = d_att;
  tr.h = d_h;
  return forward_device_locked(m, d_tokens, seq_offsets, n_seq, m->cfg.embed_dim, nullptr, pick(m->ctx, stream),
                               n_layers, &tr);
}

int sg_forward(sg_model* m, const int32_t* tokens, const int32_t* off, int32_t n_seq, int32_t out_dim, float* out) {
  if (!m || !tokens || !out) return fail(SG_ERR_INVALID, "NULL argument");
  std::lock_guard<std::mutex> lk(m->mu);
  if (out_dim <= 0 || out_dim > m->cfg.embed_dim)
    return fail(SG_ERR_DIM, "target dimension %d out of range (1..%d)", out_dim, m->cfg.embed_dim);
  SG_TRY(check_offsets(off, n_seq, -1));
  const int T = off[n_seq];
  // Sequences are checked in order, each fully (length, then tokens), so the
  // error returned is the one the reference's request-ordered fan-out reports
  // first (api.go:286-292; model_int8.go:150-171).
  for (int sq = 0; sq < n_seq; sq++) {
    const int S = off[sq + 1] - off[sq];
    if (S == 0) return fail(SG_ERR_EMPTY, "empty input");
    if (S > m->cfg.max_seq_len) return fail(SG_ERR_TOO_LONG, "sequence too long: %d > %d", S, m->cfg.max_seq_len);
    for (int i = off[sq]; i < off[sq + 1]; i++)
      if (tokens[i] < 0 || tokens[i] >= m->cfg.vocab_size)
        return fail(SG_ERR_TOKEN, "token ID out of range: %d", tokens[i]);
  }
  SG_TRY(set_device(m->ctx));
  hipStream_t s = m->ctx->stream;
  SG_TRY(m->tokens.ensure(sizeof(int32_t) * (size_t)T));
  SG_TRY(m->out.ensure(sizeof(float) * (size_t)n_seq * out_dim));
  SG_HIP(hipMemcpyAsync(m->tokens.p, tokens, sizeof(int32_t) * (size_t)T, hipMemcpyHostToDevice, s));
  SG_TRY(forward_device_locked(m, m->tokens.as<int32_t>(), off, n_seq, out_dim, m->out.as<float>(), s));
  SG_HIP(hipMemcpyAsync(out, m->out.p, sizeof(float) * (size_t)n_seq * out_dim, hipMemcpyDeviceToHost, s));
  SG_HIP(hipStreamSynchronize(s));
  return SG_OK;
}

int sg_profile_enable(sg_model* m, int on) {
  if (!m) return fail(SG_ERR_INVALID, "NULL argument");
  std::lock_guard<std::mutex> lk(m->mu);
  m->prof.on = on != 0;
  m->prof.recs.clear();
  m->prof.used = 0;
  m->prof.acc = sg_profile{};
  return SG_OK;
}

int sg_profile_read(sg_model* m, sg_profile* out) {
  if (!m || !out) return fail(SG_ERR_INVALID, "NULL argument");
  std::lock_guard<std::mutex> lk(m->mu);
  SG_TRY(set_device(m->ctx));
  SG_HIP(hipStreamSynchronize(m->ctx->stream));
  SG_TRY(m->prof.fold());
  *out = m->prof.acc;
  return SG_OK;
}

// ---- kernel seam ----------------------------------------------------------

int sg_q8_weight_create(sg_ctx* ctx, const void* q8, int32_t out_dim, int32_t in_dim, sg_q8_weight** out) {
  if (!ctx || !q8 || !out) return fail(SG_ERR_INVALID, "NULL argument");
  *out = nullptr;
  if (out_dim <= 0 || in_dim <= 0 || in_dim % 32) return fail(SG_ERR_INVALID, "in_dim must be a positive multiple of 32");
  SG_TRY(set_device(ctx));
  static std::atomic<uint64_t> next_id{1};
  sg_q8_weight* w = new sg_q8_weight;
  w->ctx = ctx;
  w->id = next_id.fetch_add(1);
  w->N = out_dim;
  w->K = in_dim;
  DevBuf stage;
  int r = SG_OK;
  if (hipMalloc(&w->w8, (size_t)out_dim * in_dim) != hipSuccess ||
      hipMalloc(&w->st, sizeof(float) * (size_t)out_dim * (in_dim / 32)) != hipSuccess)
    r = fail(SG_ERR_NOMEM, "hipMalloc failed (weight)");
  if (r == SG_OK) r = upload_q8(q8, out_dim, in_dim, stage, w->w8, w->st, out_dim, 0, ctx->stream);
  stage.release();
  if (r != SG_OK) {
    sg_q8_weight_free(w);
    return r;
  }
  *out = w;
  return SG_OK;
}

void sg_q8_weight_free(sg_q8_weight* w) {
  if (!w) return;
  if (w->w8) (void)hipFree(w->w8);
  if (w->st) (void)hipFree(w->st);
  w->pair.release();
  delete w;
}

int sg_quantize_act(sg_ctx* ctx, const float* x, int32_t rows, int32_t cols, const int32_t* off, int32_t n_seq,
                    int8_t* q_out, float* scale_out, void* stream) {
  if (!ctx || !x || !q_out || !scale_out) return fail(SG_ERR_INVALID, "NULL argument");
  if (cols <= 0 || cols % 4) return fail(SG_ERR_INVALID, "cols must be a positive multiple of 4");
  SG_TRY(check_offsets(off, n_seq, rows));
  std::lock_guard<std::mutex> lk(ctx->mu);
  SG_TRY(set_device(ctx));
  hipStream_t s = pick(ctx, stream);
  Meta meta;
  SG_TRY(stage_meta(off, n_seq, 1, ctx->meta_h, ctx->meta_d, s, meta));
  SG_TRY(ctx->amax.ensure(sizeof(float) * ((size_t)n_seq + (size_t)rows)));
  float* amax = ctx->amax.as<float>();
  float* row_scale = amax + n_seq;
  SG_HIP(sgk::fill_f32(amax, 0.0f, n_seq, s));
  SG_HIP(sgk::absmax_rows(x, cols, rows, cols, meta.row_seq, amax, s));
  SG_HIP(sgk::quantize(x, cols, rows, cols, meta.row_seq, amax, nullptr, 0, q_out, row_scale, s));
  SG_HIP(sgk::seq_scales(amax, n_seq, scale_out, s));
  SG_HIP(hipStreamSynchronize(s));
  return SG_OK;
}

static int matmul_common(sg_ctx* ctx, float* dst, int32_t* sums, const sg_q8_weight* w, const int8_t* x,
                         const float* row_scale, int32_t batch, void* stream) {
  if (!ctx || !w || !x || (!dst && !sums)) return fail(SG_ERR_INVALID, "NULL argument");
  if (batch < 0) return fail(SG_ERR_INVALID, "batch < 0");
  if (batch == 0) return SG_OK;
  if (!sums && !row_scale) return fail(SG_ERR_INVALID, "row_scale is NULL");
  std::lock_guard<std::mutex> lk(ctx->mu);
  SG_TRY(set_device(ctx));
  hipStream_t s = pick(ctx, stream);
  const int ar = sgk::gemm_pad_rows(batch);
  SG_TRY(ctx->a8.ensure((size_t)ar * w->K));
  SG_TRY(gemm_scratch_begin(ctx, s));
  ScratchUse use(ctx, s);
  int8_t* a8 = ctx->a8.as<int8_t>();
  SG_HIP(sgk::i8_blocked(x, batch, w->K, a8, ar, s));
  if (sums) {  // parity dump: synchronous (a temporary output buffer)
    SG_TRY(ctx->amax.ensure(sizeof(float) * (size_t)batch));
    float* ones = ctx->amax.as<float>();
    SG_HIP(sgk::fill_f32(ones, 1.0f, batch, s));
    DevBuf y;
    SG_TRY(y.ensure(sizeof(float) * (size_t)batch * w->N));
    hipError_t e = sgk::gemm_q8(a8, ar, w->w8, w->st, ones, y.as<float>(), sums, batch, w->N, w->K, s);
    hipError_t e2 = hipStreamSynchronize(s);
    y.release();
    SG_HIP(e);
    SG_HIP(e2);
    return SG_OK;
  }
  SG_HIP(sgk::gemm_q8(a8, ar, w->w8, w->st, row_scale, dst, nullptr, batch, w->N, w->K, s));
  return use.finish();
}

int sg_matmul_q8_0_int8(sg_ctx* ctx, float* dst, const sg_q8_weight* w, const int8_t* x, const float* row_scale,
                        int32_t batch, void* stream) {
  return matmul_common(ctx, dst, nullptr, w, x, row_scale, batch, stream);
}

int sg_matmul_q8_0_int8_bench(sg_ctx* ctx, float* dst, const sg_q8_weight* w, const int8_t* x, const float* row_scale,
                              int32_t batch, int32_t reps, void* stream, float* us_per_launch) {
  if (!ctx || !w || !x || !dst || !row_scale || !us_per_launch) return fail(SG_ERR_INVALID, "NULL argument");
  if (batch <= 0 || reps <= 0) return fail(SG_ERR_INVALID, "batch and reps must be positive");
  std::lock_guard<std::mutex> lk(ctx->mu);
  SG_TRY(set_device(ctx));
  hipStream_t s = pick(ctx, stream);
  const int ar = sgk::gemm_pad_rows(batch);
  SG_TRY(ctx->a8.ensure((size_t)ar * w->K));
  SG_TRY(gemm_scratch_begin(ctx, s));
  ScratchUse use(ctx, s);
  int8_t* a8 = ctx->a8.as<int8_t>();
  SG_HIP(sgk::i8_blocked(x, batch, w->K, a8, ar, s));
  auto gemm = [&]() { return sgk::gemm_q8(a8, ar, w->w8, w->st, row_scale, dst, nullptr, batch, w->N, w->K, s); };
  SG_HIP(gemm());  // warm
  hipEvent_t e0 = nullptr, e1 = nullptr;
  if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) {
    if (e0) (void)hipEventDestroy(e0);
    return fail(SG_ERR_DEVICE, "hipEventCreate failed");
  }
  hipError_t e = hipEventRecord(e0, s);
  for (int i = 0; i < reps && e == hipSuccess; i++) e = gemm();
  if (e == hipSuccess) e = hipEventRecord(e1, s);
  if (e == hipSuccess) e = hipEventSynchronize(e1);
  float ms = 0.f;
  if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  SG_HIP(e);
  *us_per_launch = ms * 1000.0f / (float)reps;
  return use.finish();
}

int sg_hbm_probe(sg_ctx* ctx, int32_t kind, const float* a, const float* b, void* c, int64_t n, int32_t reps,
                 void* stream, float* us_per_launch) {
  if (!ctx || !a || !c || !us_per_launch || (kind == 0 && !b)) return fail(SG_ERR_INVALID, "NULL argument");
  if (kind < 0 || kind > 1) return fail(SG_ERR_INVALID, "unknown probe kind %d", kind);
  if (n <= 0 || n % 4 || reps <= 0) return fail(SG_ERR_INVALID, "n must be a positive multiple of 4, reps positive");
  if ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b) | reinterpret_cast<uintptr_t>(c)) & 15)
    return fail(SG_ERR_INVALID, "buffers must be 16-byte aligned");
  SG_TRY(set_device(ctx));
  hipStream_t s = pick(ctx, stream);
  SG_HIP(sgk::stream_probe(kind, a, b, c, n, s));  // warm
  hipEvent_t e0 = nullptr, e1 = nullptr;
  if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) {
    if (e0) (void)hipEventDestroy(e0);
    return fail(SG_ERR_DEVICE, "hipEventCreate failed");
  }
  hipError_t e = hipEventRecord(e0, s);
  for (int i = 0; i < reps && e == hipSuccess; i++) e = sgk::stream_probe(kind, a, b, c, n, s);
  if (e == hipSuccess) e = hipEventRecord(e1, s);
  if (e == hipSuccess) e = hipEventSynchronize(e1);
  float ms = 0.f;
  if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  if (e != hipSuccess) (void)hipStreamSynchronize(s);
  SG_HIP(e);
  *us_per_launch = ms * 1000.0f / (float)reps;
  return SG_OK;
}

int sg_issue_probe(sg_ctx* ctx, int32_t kind, int32_t waves_per_simd, int32_t iters, void* stream,
                   float* simd_cycles_per_block, float* clock_ghz) {
  if (!ctx || !simd_cycles_per_block || !clock_ghz) return fail(SG_ERR_INVALID, "NULL argument");
  if (kind < 0 || kind > 3) return fail(SG_ERR_INVALID, "unknown probe kind %d", kind);
  if (waves_per_simd < 1 || waves_per_simd > 8 || iters < 2 || iters % 2 || iters > (1 << 24))
    return fail(SG_ERR_INVALID, "waves_per_simd 1..8, iters even in 2..2^24");
  SG_TRY(set_device(ctx));
  hipStream_t s = pick(ctx, stream);
  int cus = 0, wall_khz = 0;
  SG_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, ctx->device));
  SG_HIP(hipDeviceGetAttribute(&wall_khz, hipDeviceAttributeWallClockRate, ctx->device));
  if (cus <= 0 || wall_khz <= 0) return fail(SG_ERR_DEVICE, "device attributes unavailable");
  const int blocks = cus * waves_per_simd;  // 4 waves per workgroup: waves_per_simd per SIMD
  float* sink = nullptr;
  long long* clk = nullptr;
  SG_HIP(hipMalloc(&sink, sizeof(float) * 256 * (size_t)blocks));
  if (hipMalloc(&clk, sizeof(long long) * 8 * (size_t)blocks) != hipSuccess) {
    (void)hipFree(sink);
    return fail(SG_ERR_NOMEM, "hipMalloc failed");
  }
  hipEvent_t e0 = nullptr, e1 = nullptr;
  hipError_t e = sgk::issue_probe(kind, blocks, sink, clk, iters, s);  // warm
  if (e == hipSuccess) e = hipEventCreate(&e0);
  if (e == hipSuccess) e = hipEventCreate(&e1);
  if (e == hipSuccess) e = hipEventRecord(e0, s);
  if (e == hipSuccess) e = sgk::issue_probe(kind, blocks, sink, clk, iters, s);
  if (e == hipSuccess) e = hipEventRecord(e1, s);
  if (e == hipSuccess) e = hipEventSynchronize(e1);
  float ms = 0.f;
  if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
  std::vector<long long> h((size_t)8 * blocks);
  if (e == hipSuccess) e = hipMemcpy(h.data(), clk, sizeof(long long) * h.size(), hipMemcpyDeviceToHost);
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  if (e != hipSuccess) (void)hipStreamSynchronize(s);
  (void)hipFree(sink);
  (void)hipFree(clk);
  SG_HIP(e);
  double cyc = 0, ticks = 0;
  for (int i = 0; i < 4 * blocks; i++) {
    cyc += (double)h[2 * i];
    ticks += (double)h[2 * i + 1];
  }
  if (ticks <= 0 || ms <= 0) return fail(SG_ERR_DEVICE, "probe clocks unavailable");
  const double ghz = cyc / (ticks / (wall_khz * 1e3)) / 1e9;
  // every SIMD ran waves_per_simd waves of iters steps, two subtile-blocks each
  *simd_cycles_per_block = (float)(ms * 1e-3 * ghz * 1e9 / ((double)iters * 2 * waves_per_simd));
  *clock_ghz = (float)ghz;
  return SG_OK;
}

int sg_q8_block_sums(sg_ctx* ctx, int32_t* out, const sg_q8_weight* w, const int8_t* x, int32_t batch, void* stream) {
  return matmul_common(ctx, nullptr, out, w, x, nullptr, batch, stream);
}

int sg_ffn_gate_up(sg_ctx* ctx, float* dst, const sg_q8_weight* w_gate, const sg_q8_weight* w_up, const int8_t* x,
                   const float* row_scale, int32_t batch, void* stream) {
  if (!ctx || !dst || !w_gate || !w_up || !x || !row_scale) return fail(SG_ERR_INVALID, "NULL argument");
  if (w_gate->N != w_up->N || w_gate->K != w_up->K || w_gate->N % sgk::kGeluGroup)
    return fail(SG_ERR_INVALID, "gate and up must have the same shape, out_dim a multiple of 32");
  // The interleave cache on the gate weight is guarded by its context's
  // mutex and ordered on that context's GEMM scratch event only.
  if (w_gate->ctx != ctx || w_up->ctx != ctx) return fail(SG_ERR_INVALID, "weights belong to another context");
  if (batch < 0) return fail(SG_ERR_INVALID, "batch < 0");
  if (batch == 0) return SG_OK;
  std::lock_guard<std::mutex> lk(ctx->mu);
  SG_TRY(set_device(ctx));
  hipStream_t s = pick(ctx, stream);
  const int N = w_gate->N, K = w_gate->K, ar = sgk::gemm_pad_rows(batch);
  // Interleave gate and up rows in groups of 32 (the model does this at load).
  // Block-major [K/32][N][32]: each 32-row group of one block is one 1-KB
  // chunk (128 B of scales), and chunks of gate and up alternate.  The
  // interleave is kept on the gate weight for its last up weight and rebuilt
  // only when that changes; it is written on `s` after gemm_scratch_begin, so
  // every later call (ordered after this one) sees it complete.
  const size_t wch = (size_t)sgk::kGeluGroup * 32, sch = sgk::kGeluGroup * sizeof(float);
  const size_t nch = (size_t)(K / 32) * (N / sgk::kGeluGroup);
  SG_TRY(ctx->a8.ensure((size_t)ar * K));
  SG_TRY(gemm_scratch_begin(ctx, s));
  ScratchUse use(ctx, s);
  const bool rebuild = w_gate->pair_up != w_up->id;
  if (rebuild) {
    w_gate->pair_up = 0;  // invalid until the copies below are enqueued
    SG_TRY(w_gate->pair.ensure(2 * nch * (wch + sch)));
  }
  uint8_t* wi = w_gate->pair.as<uint8_t>();
  uint8_t* si = wi + 2 * nch * wch;
  if (rebuild) {
    SG_HIP(hipMemcpy2DAsync(wi, 2 * wch, w_gate->w8, wch, wch, nch, hipMemcpyDeviceToDevice, s));
    SG_HIP(hipMemcpy2DAsync(wi + wch, 2 * wch, w_up->w8, wch, wch, nch, hipMemcpyDeviceToDevice, s));
    SG_HIP(hipMemcpy2DAsync(si, 2 * sch, w_gate->st, sch, sch, nch, hipMemcpyDeviceToDevice, s));
    SG_HIP(hipMemcpy2DAsync(si + sch, 2 * sch, w_up->st, sch, sch, nch, hipMemcpyDeviceToDevice, s));
    w_gate->pair_up = w_up->id;
  }
  int8_t* a8 = ctx->a8.as<int8_t>();
  SG_HIP(sgk::i8_blocked(x, batch, K, a8, ar, s));
  SG_HIP(sgk::gemm_q8_gelu(a8, ar, reinterpret_cast<const int8_t*>(wi), reinterpret_cast<const float*>(si), row_scale,
                           dst, batch, N, K, nullptr, nullptr, s));
  return use.finish();
}

int sg_rmsnorm(sg_ctx* ctx, float* dst, const float* src, const float* weight, int32_t rows, int32_t n, float eps,
               void* stream) {
  if (!ctx || !dst || !src || !weight) return fail(SG_ERR_INVALID, "NULL argument");
  if (rows < 0) return fail(SG_ERR_INVALID, "rows < 0");
  SG_TRY(set_device(ctx));
  hipError_t e = sgk::rmsnorm(dst, src, weight, rows, n, eps, nullptr, nullptr, pick(ctx, stream));
  if (e == hipErrorInvalidValue) return fail(SG_ERR_INVALID, "row length %d unsupported (256/512/768/1024/1152)", n);
  SG_HIP(e);
  return SG_OK;
}

int sg_qknorm_rope(sg_ctx* ctx, float* q, int32_t ldq, float* k, int32_t ldk, const float* q_norm, const float* k_norm,
                   int32_t n_heads, int32_t n_kv_heads, int32_t head_dim, float eps, float rope_base,
                   int32_t max_seq_len, const int32_t* off, int32_t n_seq, void* stream) {
  if (!ctx || !q || !k) return fail(SG_ERR_INVALID, "NULL argument");
  if (head_dim != 256) return fail(SG_ERR_INVALID, "head_dim must be 256");
  SG_TRY(check_offsets(off, n_seq, -1));
  for (int i = 0; i < n_seq; i++)
    if (off[i + 1] - off[i] > max_seq_len) return fail(SG_ERR_TOO_LONG, "sequence longer than max_seq_len");
  std::lock_guard<std::mutex> lk(ctx->mu);
  SG_TRY(set_device(ctx));
  hipStream_t s = pick(ctx, stream);
  Meta meta;
  SG_TRY(stage_meta(off, n_seq, 1, ctx->meta_h, ctx->meta_d, s, meta));
  std::vector<float> ct, st;
  rope_tables(head_dim, rope_base, max_seq_len, ct, st);
  SG_TRY(ctx->tab.ensure(sizeof(float) * (ct.size() + st.size())));
  float* tc = ctx->tab.as<float>();
  SG_HIP(hipMemcpy(tc, ct.data(), sizeof(float) * ct.size(), hipMemcpyHostToDevice));
  SG_HIP(hipMemcpy(tc + ct.size(), st.data(), sizeof(float) * st.size(), hipMemcpyHostToDevice));
  SG_HIP(sgk::qknorm_rope(q, ldq, k, ldk, q_norm, k_norm, n_heads, n_kv_heads, meta.T, meta.row_pos, tc,
                          tc + ct.size(), eps, nullptr, nullptr, 0, nullptr, nullptr, 0, s));
  SG_HIP(hipStreamSynchronize(s));
  return SG_OK;
}

int sg_attention(sg_ctx* ctx, float* out, const float* q, int32_t ldq, const float* k, const float* v, int32_t ldkv,
                 int32_t n_heads, int32_t n_kv_heads, int32_t head_dim, const int32_t* off, int32_t n_seq,
                 void* stream) {
  if (!ctx || !out || !q || !k || !v) return fail(SG_ERR_INVALID, "NULL argument");
  if (head_dim != 256 || n_kv_heads <= 0 || n_heads % n_kv_heads || n_heads / n_kv_heads > 4)
    return fail(SG_ERR_INVALID, "unsupported attention shape");
  SG_TRY(check_offsets(off, n_seq, -1));
  std::lock_guard<std::mutex> lk(ctx->mu);
  SG_TRY(set_device(ctx));
  hipStream_t s = pick(ctx, stream);
  Meta meta;
  SG_TRY(stage_meta(off, n_seq, n_heads / n_kv_heads, ctx->meta_h, ctx->meta_d, s, meta));
  const float scale = 1.0f / (float)std::sqrt((double)head_dim);
  // Split operands as the forward's producers write them.
  const size_t T = (size_t)meta.T, qd = (size_t)n_heads * head_dim, kvd = (size_t)n_kv_heads * head_dim;
  const size_t split_bytes = (2 * sizeof(_Float16) * (T * qd + T * kvd + kvd * (size_t)meta.Tp) + 255) & ~(size_t)255;
  SG_TRY(ctx->split.ensure(split_bytes + (size_t)n_kv_heads * meta.spill_total * sgk::kAttnSpillTileBytes));
  SG_TRY(gemm_scratch_begin(ctx, s));  // after the asynchronous GEMM calls of this context
  _Float16* qs_h = ctx->split.as<_Float16>();
  _Float16* qs_l = qs_h + T * qd;
  _Float16* ks_h = qs_l + T * qd;
  _Float16* ks_l = ks_h + T * kvd;
  _Float16* vt_h = ks_l + T * kvd;
  const int ldvt = 2 * meta.Tp;  // per dim: each 32-key tile's hi then lo halves
  SG_HIP(sgk::split_rows(q, ldq, meta.T, (int)qd, sgk::kAttnQKScale, qs_h, qs_l, (int)qd, s));
  SG_HIP(sgk::split_rows(k, ldkv, meta.T, (int)kvd, sgk::kAttnQKScale, ks_h, ks_l, (int)kvd, s));
  SG_HIP(sgk::v_split_t(v, ldkv, meta.seq_off, meta.voff, meta.vtiles, meta.n_vtiles, n_kv_heads, vt_h, ldvt, s));
  const sg_attn_spill spill{reinterpret_cast<float*>(ctx->split.as<unsigned char>() + split_bytes), meta.spill_off,
                            meta.spill_total};
  SG_HIP(sgk::attention(qs_h, qs_l, (int)qd, ks_h, ks_l, (int)kvd, vt_h, ldvt, out, (int)qd, meta.seq_off,
                        meta.voff, meta.items, meta.n_items, n_heads, n_kv_heads, head_dim, scale, nullptr,
                        meta.max_len, s, nullptr, nullptr, &spill));
  SG_HIP(hipStreamSynchronize(s));
  return SG_OK;
}

int sg_attention_exact(sg_ctx* ctx, float* out, const float* q, int32_t ldq, const float* k, const float* v,
                       int32_t ldkv, int32_t n_heads, int32_t n_kv_heads, int32_t head_dim, const int32_t* off,
                       int32_t n_seq, void* stream) {
  if (!ctx || !out || !q || !k || !v) return fail(SG_ERR_INVALID, "NULL argument");
  if (head_dim != 256 || n_kv_heads <= 0 || n_heads % n_kv_heads)
    return fail(SG_ERR_INVALID, "unsupported attention shape");
  if ((ldq & 3) || (ldkv & 3) || (reinterpret_cast<uintptr_t>(q) & 15) || (reinterpret_cast<uintptr_t>(k) & 15))
    return fail(SG_ERR_INVALID, "q and k rows must be 16-byte aligned (strides multiples of 4)");
  SG_TRY(check_offsets(off, n_seq, -1));
  if ((int64_t)n_seq * n_heads > 65535) return fail(SG_ERR_INVALID, "n_seq * n_heads above 65535");
  std::lock_guard<std::mutex> lk(ctx->mu);
  SG_TRY(set_device(ctx));
  hipStream_t s = pick(ctx, stream);
  Meta meta;
  SG_TRY(stage_meta(off, n_seq, n_heads / n_kv_heads, ctx->meta_h, ctx->meta_d, s, meta));
  if (meta.max_len > 2048) return fail(SG_ERR_INVALID, "sequences longer than 2048 keys are not supported");
  const float scale = 1.0f / (float)std::sqrt((double)head_dim);
  SG_TRY(ctx->split.ensure(sgk::attention_exact_scratch(meta.T, n_heads, meta.max_len)));
  SG_TRY(gemm_scratch_begin(ctx, s));  // after the asynchronous GEMM calls of this context
  SG_HIP(sgk::attention_exact(q, ldq, k, v, ldkv, out, n_heads * head_dim, meta.seq_off, meta.row_seq, n_seq, meta.T,
                              n_heads, n_kv_heads, head_dim, scale, meta.max_len, ctx->split.as<float>(), nullptr,
                              s));
  SG_HIP(hipStreamSynchronize(s));
  return SG_OK;
}

int sg_model_set_attention_mode(sg_model* m, int mode) {
  if (!m) return fail(SG_ERR_INVALID, "NULL argument");
  if (mode != SG_ATTN_FAST && mode != SG_ATTN_EXACT) return fail(SG_ERR_INVALID, "unknown attention mode %d", mode);
  if (mode == SG_ATTN_EXACT && m->cfg.max_seq_len > 2048)
    return fail(SG_ERR_INVALID, "exact attention supports sequences up to 2048 keys (model: %d)", m->cfg.max_seq_len);
  std::lock_guard<std::mutex> lk(m->mu);
  m->attn_mode = mode;
  return SG_OK;
}

int sg_gelu_quick_mul(sg_ctx* ctx, float* dst, int32_t ldd, const float* gate, int32_t ldg, const float* up,
                      int32_t ldu, int32_t rows, int32_t cols, void* stream) {
  if (!ctx || !dst || !gate || !up) return fail(SG_ERR_INVALID, "NULL argument");
  SG_TRY(set_device(ctx));
  hipError_t e = sgk::gelu_mul(dst, ldd, gate, ldg, up, ldu, rows, cols, nullptr, nullptr, pick(ctx, stream));
  if (e == hipErrorInvalidValue) return fail(SG_ERR_INVALID, "cols and strides must be multiples of 4");
  SG_HIP(e);
  return SG_OK;
}

int sg_embed_tokens(sg_model* m, float* dst, const int32_t* d_tokens, int32_t n_tokens, void* stream) {
  if (!m || !dst || !d_tokens) return fail(SG_ERR_INVALID, "NULL argument");
  std::lock_guard<std::mutex> lk(m->mu);
  SG_TRY(set_device(m->ctx));
  hipStream_t s = pick(m->ctx, stream);
  Lane& w = m->lanes[0];
  SG_TRY(w.err.ensure(64));
  SG_HIP(sgk::fill_i32(w.err.as<int32_t>(), INT32_MAX, 1, s));
  SG_HIP(sgk::embed_only(d_tokens, n_tokens, m->emb_q, m->emb_s, m->cfg.vocab_size, m->cfg.embed_dim, m->sqrt_d, dst,
                         w.err.as<int32_t>(), s));
  return token_error(w, d_tokens, s);
}

int sg_pool_l2(sg_ctx* ctx, float* out, const float* x, int32_t ldx, int32_t out_dim, const int32_t* off, int32_t n_seq,
               void* stream) {
  if (!ctx || !out || !x) return fail(SG_ERR_INVALID, "NULL argument");
  if (out_dim <= 0 || out_dim > 1024 || out_dim > ldx) return fail(SG_ERR_DIM, "out_dim %d out of range", out_dim);
  SG_TRY(check_offsets(off, n_seq, -1));
  for (int i = 0; i < n_seq; i++)
    if (off[i + 1] == off[i]) return fail(SG_ERR_EMPTY, "empty input");
  std::lock_guard<std::mutex> lk(ctx->mu);
  SG_TRY(set_device(ctx));
  hipStream_t s = pick(ctx, stream);
  Meta meta;
  SG_TRY(stage_meta(off, n_seq, 1, ctx->meta_h, ctx->meta_d, s, meta));
  SG_HIP(sgk::pool_l2(out, x, ldx, out_dim, meta.seq_off, n_seq, s));
  SG_HIP(hipStreamSynchronize(s));
  return SG_OK;
}

}  // extern "C"
