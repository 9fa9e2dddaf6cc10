#include <hip/hip_runtime.h>
typedef int i32x4_t __attribute__((ext_vector_type(4)));
__global__ void k(const float* src, float* out) {
  __shared__ __attribute__((aligned(16))) unsigned char lds[4096];
  const uint64_t base = (uint64_t)src;
  i32x4_t r = {(int)(uint32_t)base, (int)(uint32_t)(base >> 32), 0x7fffffff, 0x00020000};
  const uint32_t m0v = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char*)(lds + 1024 * (threadIdx.x >> 6));
  const uint32_t voff = threadIdx.x * 16;
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" :: "s"(__builtin_amdgcn_readfirstlane(m0v)), "v"(voff), "s"(r) : "memory", "m0");
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  out[threadIdx.x] = ((float*)lds)[threadIdx.x];
}
