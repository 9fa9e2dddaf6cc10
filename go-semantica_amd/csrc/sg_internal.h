// sg_internal.h -- helpers shared by the library's host translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>

#include <string>
#include <vector>

#include "semantica_gpu.h"

namespace sgi {
// Records a printf-style message for sg_last_error() (thread-local) and
// returns `code`.
__attribute__((visibility("hidden"))) int fail(int code, const char* fmt, ...);

// sg_ctx accessors (the struct lives in sg_api.cpp): device ordinal, and the
// stream a call runs on (the caller's, or the context's own when NULL).
__attribute__((visibility("hidden"))) int ctx_device(const sg_ctx* c);
__attribute__((visibility("hidden"))) hipStream_t ctx_stream(const sg_ctx* c, void* stream);

// Resolves, once per device and with that device current, the device address
// of the allocation-free entry points' static scratch (sg_noalloc.hip).
__attribute__((visibility("hidden"))) int noalloc_setup(int device);

// A tokenizer's vocabulary and settings (tokenizer.New's arguments plus the
// special ids LoadFromGGUF sets).  types empty = every token normal.
struct TokenizerSpec {
  std::vector<std::string> tokens;
  std::vector<float> scores;
  std::vector<int32_t> types;
  bool add_bos = false, add_eos = false, lowercase = false, remove_accents = false, nfkc = false;
  int32_t bos = -1, eos = -1, unk = -1, pad = -1;
};
// Reads the tokenizer metadata of a GGUF image (sg_gguf.cpp).
__attribute__((visibility("hidden"))) int gguf_tokenizer_spec(const void* data, size_t size, TokenizerSpec& out);

// Grow-only device buffer.  Growing waits for the device first, so work still
// in flight on any stream never loses the old buffer under it.
struct DevBuf {
  void* p = nullptr;
  size_t n = 0;
  template <typename T>
  T* as() const { return static_cast<T*>(p); }
  int ensure(size_t bytes) {
    if (bytes <= n) return SG_OK;
    if (p) {
      (void)hipDeviceSynchronize();
      (void)hipFree(p);
    }
    p = nullptr;
    n = 0;
    if (bytes == 0) return SG_OK;
    if (hipMalloc(&p, bytes) != hipSuccess) {
      p = nullptr;
      return fail(SG_ERR_NOMEM, "hipMalloc(%zu bytes) failed", bytes);
    }
    n = bytes;
    return SG_OK;
  }
  void release() {
    if (p) (void)hipFree(p);
    p = nullptr;
    n = 0;
  }
};

// Grow-only pinned host buffer (staging for metadata / small copies).
// Pinned host staging.  An asynchronous copy out of it is followed by
// record(stream); wait() (called by ensure and release too) blocks until that
// copy has read the buffer, so the next writer cannot race the DMA.
struct HostBuf {
  void* p = nullptr;
  size_t n = 0;
  hipEvent_t done = nullptr;
  template <typename T>
  T* as() const { return static_cast<T*>(p); }
  int wait() {
    if (done && hipEventSynchronize(done) != hipSuccess) return fail(SG_ERR_DEVICE, "hipEventSynchronize failed");
    return SG_OK;
  }
  int record(hipStream_t s) {
    if (!done && hipEventCreateWithFlags(&done, hipEventDisableTiming) != hipSuccess) {
      done = nullptr;
      return fail(SG_ERR_DEVICE, "hipEventCreateWithFlags failed");
    }
    if (hipEventRecord(done, s) != hipSuccess) return fail(SG_ERR_DEVICE, "hipEventRecord failed");
    return SG_OK;
  }
  int ensure(size_t bytes) {
    if (wait() != SG_OK) return SG_ERR_DEVICE;
    if (bytes <= n) return SG_OK;
    if (p) (void)hipHostFree(p);
    p = nullptr;
    n = 0;
    if (hipHostMalloc(&p, bytes, hipHostMallocDefault) != hipSuccess) {
      p = nullptr;
      return fail(SG_ERR_NOMEM, "hipHostMalloc(%zu bytes) failed", bytes);
    }
    n = bytes;
    return SG_OK;
  }
  void release() {
    (void)wait();
    if (done) (void)hipEventDestroy(done);
    done = nullptr;
    if (p) (void)hipHostFree(p);
    p = nullptr;
    n = 0;
  }
};
}  // namespace sgi

// A Q8_0 weight matrix repacked on the device (kernel seam).
struct sg_q8_weight {
  sg_ctx* ctx = nullptr;
  int N = 0, K = 0;
  uint64_t id = 0;       // unique per created weight
  int8_t* w8 = nullptr;  // block-major int8 [K/32][N][32]
  float* st = nullptr;   // [K/32][N]
  // sg_ffn_gate_up with this weight as the gate: the gate/up interleave it
  // last built (weights then scales), for the up weight with id pair_up.
  mutable sgi::DevBuf pair;
  mutable uint64_t pair_up = 0;
};

#define SG_HIP(call)                                                                                     \
  do {                                                                                                   \
    hipError_t e_ = (call);                                                                              \
    if (e_ != hipSuccess)                                                                                \
      return ::sgi::fail(e_ == hipErrorInvalidValue ? SG_ERR_INVALID : SG_ERR_DEVICE, "%s: %s (%s:%d)", #call, \
                         hipGetErrorString(e_), __FILE__, __LINE__);                                     \
  } while (0)

#define SG_TRY(expr)            \
  do {                          \
    int r_ = (expr);            \
    if (r_ != SG_OK) return r_; \
  } while (0)
