// sg_search.cpp -- the brute-force vector index (search/brute) on the GPU:
// Builder/Build, Serializer, Vector and SearchVector/SearchNormalized over a
// batch of queries, behind the C ABI.
//
// The vectors live in HBM in the scoring layout of k_search.hip; the host
// keeps the ids (and an id -> position map, index.go:14-15).  A search scores
// a batch of queries against every vector and selects each query's top-k on
// the GPU (sgk::bf_score, sgk::bf_select); the host maps positions to ids and
// applies the reference's final ordering, distance descending then id
// ascending (index.go:133-137), to the k results of each query.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "semantica_gpu.h"
#include "sg_internal.h"
#include "sg_kernels.h"

using sgi::DevBuf;
using sgi::fail;
using sgi::HostBuf;

struct sg_index {
  sg_ctx* ctx = nullptr;
  int dim = 0, mode = 0, count = 0;
  std::vector<int32_t> ids;
  std::unordered_map<int32_t, int> pos;
  DevBuf grp, tail;                                  // the vectors
  DevBuf stage, queries, scores, state, hist, oidx, odist;  // call workspace
  HostBuf h_in, h_out;
  std::mutex mu;
  ~sg_index() {
    for (DevBuf* b : {&grp, &tail, &stage, &queries, &scores, &state, &hist, &oidx, &odist}) b->release();
    h_in.release();
    h_out.release();
  }
};

namespace {

constexpr size_t kStageBytes = size_t(64) << 20;   // host <-> device chunks
constexpr size_t kScoreBytes = size_t(256) << 20;  // scores of one query batch

// storage.go:14-27: magic "BRUT", version 1, then the header fields packed
// little-endian with 7 bytes of padding (20 bytes), ids, vector data.
constexpr uint16_t kBruteVersion = 1;
constexpr size_t kHeaderBytes = 20;

size_t elem_bytes(int mode) { return mode == sgk::kBfF32 ? 4 : (mode == sgk::kBfI8 ? 1 : 2); }

int check_mode(int mode) {
  if (mode != sgk::kBfF32 && mode != sgk::kBfI8 && mode != sgk::kBfI16)
    return fail(SG_ERR_INVALID, "brute: unsupported quantization %d", mode);
  return SG_OK;
}

// Index shell with ids and the device layout allocated.
int make_index(sg_ctx* ctx, int dim, int mode, const int32_t* ids, int n, sg_index** out) {
  sg_index* x = new sg_index;
  x->ctx = ctx;
  x->dim = dim;
  x->mode = mode;
  x->count = n;
  x->ids.assign(ids, ids + n);
  x->pos.reserve((size_t)n);
  for (int i = 0; i < n; i++) x->pos[ids[i]] = i;
  const size_t eb = elem_bytes(mode);
  int r = x->grp.ensure(eb * (size_t)(dim / 8) * 8 * (size_t)n + 16);
  if (r == SG_OK) r = x->tail.ensure(eb * (size_t)(dim % 8) * (size_t)n + 16);
  if (r != SG_OK) {
    delete x;
    return r;
  }
  *out = x;
  return SG_OK;
}

// Go's %q of the 4 magic bytes (storage.go:103).
std::string quote4(const uint8_t* b) {
  std::string out = "\"";
  char tmp[8];
  for (int i = 0; i < 4; i++) {
    const uint8_t c = b[i];
    if (c == '"' || c == '\\') {
      out += '\\';
      out += (char)c;
    } else if (c >= 0x20 && c < 0x7f) {
      out += (char)c;
    } else {
      const char* esc = c == '\a' ? "\\a" : c == '\b' ? "\\b" : c == '\f' ? "\\f" : c == '\n' ? "\\n"
                      : c == '\r' ? "\\r" : c == '\t' ? "\\t" : c == '\v' ? "\\v" : nullptr;
      if (esc) {
        out += esc;
      } else {
        snprintf(tmp, sizeof tmp, "\\x%02x", c);
        out += tmp;
      }
    }
  }
  return out + "\"";
}

// io.ReadFull's error for a section of `need` bytes with `have` left.
int short_read(size_t have) { return fail(SG_ERR_INVALID, have ? "unexpected EOF" : "EOF"); }

// Rows per host<->device chunk for `row_bytes`-byte rows.
int chunk_rows(size_t row_bytes) { return (int)std::max<size_t>(1, kStageBytes / std::max<size_t>(row_bytes, 1)); }

int check_build_args(int dim, int mode, const int32_t* ids, int n) {
  SG_TRY(check_mode(mode));
  if (n <= 0) return fail(SG_ERR_INVALID, "brute: no vectors added");
  if (!ids) return fail(SG_ERR_INVALID, "NULL ids");
  if (dim <= 0) return fail(SG_ERR_INVALID, "brute: vector dimension must be positive");
  std::unordered_map<int32_t, int> seen;
  seen.reserve((size_t)n);
  for (int i = 0; i < n; i++)  // AddVector (builder.go:58-60)
    if (!seen.emplace(ids[i], i).second) return fail(SG_ERR_INVALID, "brute: duplicate id %d", ids[i]);
  return SG_OK;
}

}  // namespace

extern "C" {

int sg_index_build(sg_ctx* ctx, int32_t dim, int32_t quantization, const int32_t* ids, const float* vectors,
                   int32_t n, sg_index** out) {
  if (!ctx || !out) return fail(SG_ERR_INVALID, "NULL argument");
  *out = nullptr;
  SG_TRY(check_build_args(dim, quantization, ids, n));
  if (!vectors) return fail(SG_ERR_INVALID, "NULL vectors");
  SG_HIP(hipSetDevice(sgi::ctx_device(ctx)));
  hipStream_t s = sgi::ctx_stream(ctx, nullptr);
  sg_index* x = nullptr;
  SG_TRY(make_index(ctx, dim, quantization, ids, n, &x));
  const int rows = chunk_rows(sizeof(float) * (size_t)dim);
  int r = x->stage.ensure(sizeof(float) * (size_t)dim * std::min(rows, n));
  for (int r0 = 0; r == SG_OK && r0 < n; r0 += rows) {
    const int m = std::min(rows, n - r0);
    hipError_t e = hipMemcpyAsync(x->stage.p, vectors + (size_t)r0 * dim, sizeof(float) * (size_t)m * dim,
                                  hipMemcpyHostToDevice, s);
    if (e == hipSuccess)
      e = sgk::bf_build(quantization, x->stage.as<float>(), dim, m, dim, r0, n, x->grp.p, x->tail.p, true, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) r = fail(SG_ERR_DEVICE, "index build: %s", hipGetErrorString(e));
  }
  x->stage.release();
  if (r != SG_OK) {
    delete x;
    return r;
  }
  *out = x;
  return SG_OK;
}

int sg_index_build_device(sg_ctx* ctx, int32_t dim, int32_t quantization, const int32_t* ids,
                          const float* d_vectors, int64_t ld, int32_t n, void* stream, sg_index** out) {
  if (!ctx || !out) return fail(SG_ERR_INVALID, "NULL argument");
  *out = nullptr;
  SG_TRY(check_build_args(dim, quantization, ids, n));
  if (!d_vectors) return fail(SG_ERR_INVALID, "NULL vectors");
  if (ld < dim) return fail(SG_ERR_INVALID, "row stride %lld < dim %d", (long long)ld, dim);
  SG_HIP(hipSetDevice(sgi::ctx_device(ctx)));
  hipStream_t s = sgi::ctx_stream(ctx, stream);
  sg_index* x = nullptr;
  SG_TRY(make_index(ctx, dim, quantization, ids, n, &x));
  hipError_t e = sgk::bf_build(quantization, d_vectors, ld, n, dim, 0, n, x->grp.p, x->tail.p, true, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  if (e != hipSuccess) {
    delete x;
    return fail(SG_ERR_DEVICE, "index build: %s", hipGetErrorString(e));
  }
  *out = x;
  return SG_OK;
}

int sg_index_deserialize(sg_ctx* ctx, const void* data, size_t size, sg_index** out) {
  if (!ctx || !out || (!data && size)) return fail(SG_ERR_INVALID, "NULL argument");
  *out = nullptr;
  const uint8_t* p = static_cast<const uint8_t*>(data);
  // readIndex (storage.go:94-153); a short image is io.ReadFull's error.
  if (size < kHeaderBytes) return short_read(size);
  if (memcmp(p, "BRUT", 4) != 0) return fail(SG_ERR_INVALID, "brute: invalid magic: %s", quote4(p).c_str());
  uint16_t version, dim;
  uint32_t count;
  memcpy(&version, p + 4, 2);
  memcpy(&dim, p + 6, 2);
  memcpy(&count, p + 8, 4);
  const int mode = p[12];
  if (version != kBruteVersion) return fail(SG_ERR_INVALID, "brute: unsupported version %d", version);
  if (count > (uint32_t)INT32_MAX) return fail(SG_ERR_INVALID, "brute: count %u too large", count);
  const size_t ids_bytes = (size_t)count * 4;
  if (size - kHeaderBytes < ids_bytes) return short_read(size - kHeaderBytes);
  SG_TRY(check_mode(mode));
  const size_t row_bytes = elem_bytes(mode) * dim;
  const size_t data_bytes = row_bytes * count;
  if (size - kHeaderBytes - ids_bytes < data_bytes) return short_read(size - kHeaderBytes - ids_bytes);
  if (count > 0 && dim == 0) return fail(SG_ERR_INVALID, "brute: zero dimension");
  std::vector<int32_t> ids(count);
  if (count) memcpy(ids.data(), p + kHeaderBytes, ids_bytes);
  SG_HIP(hipSetDevice(sgi::ctx_device(ctx)));
  hipStream_t s = sgi::ctx_stream(ctx, nullptr);
  sg_index* x = nullptr;
  SG_TRY(make_index(ctx, dim, mode, ids.data(), (int)count, &x));
  const uint8_t* rows = p + kHeaderBytes + ids_bytes;
  const int per = chunk_rows(row_bytes);
  int r = count ? x->stage.ensure(row_bytes * std::min<size_t>(per, count)) : SG_OK;
  for (int r0 = 0; r == SG_OK && r0 < (int)count; r0 += per) {
    const int m = std::min(per, (int)count - r0);
    hipError_t e = hipMemcpyAsync(x->stage.p, rows + row_bytes * r0, row_bytes * m, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = sgk::bf_relayout(mode, x->stage.p, m, dim, r0, (int)count, x->grp.p, x->tail.p, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) r = fail(SG_ERR_DEVICE, "index upload: %s", hipGetErrorString(e));
  }
  x->stage.release();
  if (r != SG_OK) {
    delete x;
    return r;
  }
  *out = x;
  return SG_OK;
}

int sg_index_serialize(sg_index* x, void* buf, size_t cap, size_t* size) {
  if (!x || !size) return fail(SG_ERR_INVALID, "NULL argument");
  std::lock_guard<std::mutex> lk(x->mu);
  const size_t row_bytes = elem_bytes(x->mode) * x->dim;
  const size_t total = kHeaderBytes + (size_t)x->count * 4 + row_bytes * x->count;
  *size = total;
  if (!buf) return SG_OK;
  if (cap < total) return fail(SG_ERR_INVALID, "buffer of %zu bytes, %zu needed", cap, total);
  if (x->dim > 0xffff) return fail(SG_ERR_INVALID, "brute: dimension %d does not fit the v1 header", x->dim);
  uint8_t* p = static_cast<uint8_t*>(buf);
  memset(p, 0, kHeaderBytes);
  memcpy(p, "BRUT", 4);
  const uint16_t version = kBruteVersion, dim = (uint16_t)x->dim;
  const uint32_t count = (uint32_t)x->count;
  memcpy(p + 4, &version, 2);
  memcpy(p + 6, &dim, 2);
  memcpy(p + 8, &count, 4);
  p[12] = (uint8_t)x->mode;
  if (x->count) memcpy(p + kHeaderBytes, x->ids.data(), (size_t)x->count * 4);
  uint8_t* rows = p + kHeaderBytes + (size_t)x->count * 4;
  SG_HIP(hipSetDevice(sgi::ctx_device(x->ctx)));
  hipStream_t s = sgi::ctx_stream(x->ctx, nullptr);
  const int per = chunk_rows(row_bytes);
  for (int r0 = 0; r0 < x->count; r0 += per) {
    const int m = std::min(per, x->count - r0);
    SG_TRY(x->stage.ensure(row_bytes * m));
    SG_HIP(sgk::bf_unpack(x->mode, x->grp.p, x->tail.p, r0, m, x->dim, x->count, x->stage.p, s));
    SG_HIP(hipMemcpyAsync(rows + row_bytes * r0, x->stage.p, row_bytes * m, hipMemcpyDeviceToHost, s));
    SG_HIP(hipStreamSynchronize(s));
  }
  return SG_OK;
}

int sg_index_info(const sg_index* x, int32_t* dim, int32_t* count, int32_t* quantization) {
  if (!x) return fail(SG_ERR_INVALID, "NULL index");
  if (dim) *dim = x->dim;
  if (count) *count = x->count;
  if (quantization) *quantization = x->mode;
  return SG_OK;
}

int sg_index_vector(sg_index* x, int32_t id, float* out) {
  if (!x || !out) return fail(SG_ERR_INVALID, "NULL argument");
  std::lock_guard<std::mutex> lk(x->mu);
  auto it = x->pos.find(id);
  if (it == x->pos.end()) return fail(SG_ERR_INVALID, "brute: no vector with id %d", id);
  const size_t row_bytes = elem_bytes(x->mode) * x->dim;
  SG_HIP(hipSetDevice(sgi::ctx_device(x->ctx)));
  hipStream_t s = sgi::ctx_stream(x->ctx, nullptr);
  SG_TRY(x->stage.ensure(row_bytes));
  SG_TRY(x->h_out.ensure(row_bytes));
  SG_HIP(sgk::bf_unpack(x->mode, x->grp.p, x->tail.p, it->second, 1, x->dim, x->count, x->stage.p, s));
  SG_HIP(hipMemcpyAsync(x->h_out.p, x->stage.p, row_bytes, hipMemcpyDeviceToHost, s));
  SG_HIP(hipStreamSynchronize(s));
  // dequantizeInt8/16 (quant.go:43-55): float32(v) * float32(1/127 or 1/32767)
  if (x->mode == sgk::kBfF32) {
    memcpy(out, x->h_out.p, row_bytes);
  } else if (x->mode == sgk::kBfI8) {
    const float sc = (float)(1.0 / 127.0);
    for (int i = 0; i < x->dim; i++) out[i] = (float)x->h_out.as<int8_t>()[i] * sc;
  } else {
    const float sc = (float)(1.0 / 32767.0);
    for (int i = 0; i < x->dim; i++) out[i] = (float)x->h_out.as<int16_t>()[i] * sc;
  }
  return SG_OK;
}

int sg_index_search(sg_index* x, const float* queries, int32_t n_queries, int32_t top_k, int32_t normalize,
                    int32_t* out_ids, float* out_dist, int32_t* n_found, void* stream) {
  if (!x) return fail(SG_ERR_INVALID, "NULL index");
  if (top_k <= 0) return fail(SG_ERR_INVALID, "brute: topK must be positive");  // index.go:29-31
  if (n_queries < 0) return fail(SG_ERR_INVALID, "n_queries < 0");
  if (n_queries == 0) return SG_OK;
  if (!queries || !out_ids || !out_dist || !n_found) return fail(SG_ERR_INVALID, "NULL argument");
  std::lock_guard<std::mutex> lk(x->mu);
  const int N = x->count, dim = x->dim;
  const int k = std::min(top_k, N);  // index.go:55-58
  if (k == 0) {
    for (int q = 0; q < n_queries; q++) n_found[q] = 0;
    return SG_OK;
  }
  SG_HIP(hipSetDevice(sgi::ctx_device(x->ctx)));
  hipStream_t s = sgi::ctx_stream(x->ctx, stream);
  const int qb = (int)std::max<size_t>(1, std::min<size_t>((size_t)n_queries, kScoreBytes / (sizeof(float) * N)));
  SG_TRY(x->queries.ensure(sizeof(float) * (size_t)qb * dim));
  SG_TRY(x->scores.ensure(sizeof(float) * (size_t)qb * N));
  SG_TRY(x->state.ensure(sizeof(int32_t) * 8 * (size_t)qb));
  SG_TRY(x->hist.ensure(sizeof(uint32_t) * 256 * (size_t)qb));
  SG_TRY(x->oidx.ensure(sizeof(int32_t) * (size_t)qb * k));
  SG_TRY(x->odist.ensure(sizeof(float) * (size_t)qb * k));
  SG_TRY(x->h_in.ensure(sizeof(float) * (size_t)qb * dim));
  SG_TRY(x->h_out.ensure((sizeof(int32_t) + sizeof(float)) * (size_t)qb * k));
  struct Res {
    int32_t id;
    float dist;
  };
  std::vector<Res> res((size_t)k);
  for (int q0 = 0; q0 < n_queries; q0 += qb) {
    const int nq = std::min(qb, n_queries - q0);
    memcpy(x->h_in.p, queries + (size_t)q0 * dim, sizeof(float) * (size_t)nq * dim);
    SG_HIP(hipMemcpyAsync(x->queries.p, x->h_in.p, sizeof(float) * (size_t)nq * dim, hipMemcpyHostToDevice, s));
    if (normalize) SG_HIP(sgk::bf_normalize(x->queries.as<float>(), nq, dim, s));
    SG_HIP(sgk::bf_score(x->mode, x->grp.p, x->tail.p, N, dim, x->queries.as<float>(), nq, x->scores.as<float>(), N,
                         s));
    SG_HIP(sgk::bf_select(x->scores.as<float>(), N, N, nq, k, x->state.as<int32_t>(), x->hist.as<uint32_t>(),
                          x->oidx.as<int32_t>(), x->odist.as<float>(), s));
    int32_t* hi = x->h_out.as<int32_t>();
    float* hd = reinterpret_cast<float*>(hi + (size_t)nq * k);
    SG_HIP(hipMemcpyAsync(hi, x->oidx.p, sizeof(int32_t) * (size_t)nq * k, hipMemcpyDeviceToHost, s));
    SG_HIP(hipMemcpyAsync(hd, x->odist.p, sizeof(float) * (size_t)nq * k, hipMemcpyDeviceToHost, s));
    SG_HIP(hipStreamSynchronize(s));
    for (int q = 0; q < nq; q++) {
      for (int j = 0; j < k; j++) {
        const int32_t p = hi[(size_t)q * k + j];
        if (p < 0 || p >= N) return fail(SG_ERR_DEVICE, "top-k selection left slot %d of query %d empty", j, q0 + q);
        res[j] = Res{x->ids[p], hd[(size_t)q * k + j]};
      }
      std::sort(res.begin(), res.end(), [](const Res& a, const Res& b) {
        return a.dist == b.dist ? a.id < b.id : a.dist > b.dist;  // index.go:133-137
      });
      for (int j = 0; j < k; j++) {
        out_ids[(size_t)(q0 + q) * top_k + j] = res[j].id;
        out_dist[(size_t)(q0 + q) * top_k + j] = res[j].dist;
      }
      n_found[q0 + q] = k;
    }
  }
  return SG_OK;
}

void sg_index_free(sg_index* x) {
  if (!x) return;
  (void)hipSetDevice(sgi::ctx_device(x->ctx));
  delete x;
}

}  // extern "C"
