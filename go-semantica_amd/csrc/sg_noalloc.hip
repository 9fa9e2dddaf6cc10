// sg_noalloc.hip -- the allocation-free form of the GEMM seam,
// sg_matmul_q8_0_int8_noalloc, for callers that cannot allocate device memory
// (code under HIP graph capture, tight serving loops).
//
// sg_matmul_q8_0_int8 relays the int8 activations into the GEMM's
// block-major operand [K/32][pad(batch)][32] in a library-grown buffer.  Here
// that operand lives in `scratch`, a fixed array in every device's memory
// (held until the process ends).  Its device address is resolved once per
// device when sg_init runs with that device current; host code never passes
// the array's own name to a kernel or a copy (in host code it names a host
// stand-in, not device memory).
//
// Every call on a device shares that device's array and leaves its contents
// behind.  Nothing in it needs to start at zero: each call writes every row
// the GEMM's stored outputs read (the padding rows past `batch` only feed
// output rows that are never stored).  Calls that overlap on one device, e.g.
// on two streams, race on the array; callers serialize them.
#include <hip/hip_runtime.h>

#include <mutex>

#include "sg_internal.h"
#include "sg_kernels.h"

static __device__ __align__(256) unsigned char scratch[SG_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_ptr[kMaxDevices] = {};  // device address of `scratch`, per device ordinal

}  // namespace

namespace sgi {

int noalloc_setup(int device) {
  if (device < 0 || device >= kMaxDevices) return fail(SG_ERR_INVALID, "device %d out of range", device);
  std::lock_guard<std::mutex> lk(g_mu);
  if (g_ptr[device]) return SG_OK;
  void* p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !p)
    return fail(SG_ERR_DEVICE, "hipGetSymbolAddress(scratch) failed on device %d: %s", device, hipGetErrorString(e));
  g_ptr[device] = p;
  return SG_OK;
}

}  // namespace sgi

extern "C" int sg_matmul_q8_0_int8_noalloc(sg_ctx* ctx, float* dst, const sg_q8_weight* w, const int8_t* x,
                                           const float* row_scale, int32_t batch, void* stream) {
  using sgi::fail;
  if (!ctx || !w || !x || !dst || !row_scale) return fail(SG_ERR_INVALID, "NULL argument");
  if (batch < 0) return fail(SG_ERR_INVALID, "batch < 0");
  if (batch == 0) return SG_OK;
  const int dev = sgi::ctx_device(ctx);
  void* p = nullptr;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    p = dev >= 0 && dev < kMaxDevices ? g_ptr[dev] : nullptr;
  }
  if (!p) return fail(SG_ERR_DEVICE, "scratch not set up for device %d (sg_init not called for it)", dev);
  const int ar = sgk::gemm_pad_rows(batch);
  const size_t need = (size_t)ar * (size_t)w->K;
  if (need > SG_NOALLOC_SCRATCH_BYTES)
    return fail(SG_ERR_INVALID, "batch %d x in_dim %d needs %zu bytes of operand scratch; the limit is %u", batch,
                w->K, need, (unsigned)SG_NOALLOC_SCRATCH_BYTES);
  // The launches go to the context's device; the calling thread's current
  // device is put back before returning, on every path.
  int prev = -1;
  SG_HIP(hipGetDevice(&prev));
  if (prev != dev) SG_HIP(hipSetDevice(dev));
  const hipStream_t s = sgi::ctx_stream(ctx, stream);
  int8_t* a8 = static_cast<int8_t*>(p);
  hipError_t e = sgk::i8_blocked(x, batch, w->K, a8, ar, s);
  if (e == hipSuccess) e = sgk::gemm_q8(a8, ar, w->w8, w->st, row_scale, dst, nullptr, batch, w->N, w->K, s);
  const hipError_t er = prev != dev ? hipSetDevice(prev) : hipSuccess;
  SG_HIP(e);
  SG_HIP(er);
  return SG_OK;
}
