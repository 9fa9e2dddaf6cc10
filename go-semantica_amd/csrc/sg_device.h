// sg_device.h -- device-side building blocks shared by the gfx950 kernels.
//
// Every function here restates one piece of reference arithmetic with the
// same rounding steps (the library is built with -ffp-contract=off, so a*b+c
// is two roundings unless fmaf() is written out, exactly as Go on amd64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

typedef int i32x4_t __attribute__((ext_vector_type(4)));

// Publishes a ring stage of the direct-to-LDS kernels: this wave's vector
// memory operations older than the last N have completed (vmcnt) and so have
// its LDS reads (lgkmcnt), so after the following s_barrier every wave's
// copies of the stage have landed and no wave still reads the stage the next
// copies overwrite.  (The compiler may place the last MFMAs of a step, and
// their lgkmcnt waits, after an s_barrier, so the read wait is explicit.)
template <int N>
__device__ __forceinline__ void sg_wait_vmcnt() {
  static_assert(N >= 0 && N <= 63, "vmcnt field");
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(N) : "memory");
}

// One 64-lane buffer_load_dwordx4 ... lds (1 KB to LDS at lds_addr + 16 *
// lane, lane l reading rsrc.base + voff_l + soff), issued from inline
// assembly.  The compiler then sees no LDS write, so it inserts no wait in
// front of the fragment reads of the other ring stages (it cannot tell them
// apart from the copies once several are in flight); the kernel orders copies
// and reads itself with sg_wait_vmcnt + s_barrier.  M0 (the copy's LDS base)
// is saved and restored around it.
__device__ __forceinline__ void sg_lds_copy16(uint32_t lds_addr, uint32_t voff, i32x4_t rsrc, uint32_t soff) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %2, %3, %4 offen lds\n\t"
      "s_nop 0\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(lds_addr), "v"(voff), "s"(rsrc), "s"(soff)
      : "memory");
}

// Raw buffer descriptor over [base, base + 2 GB): stride 0, the rest as
// __builtin_amdgcn_make_buffer_rsrc builds it (word 3: gfx9 raw buffer).
__device__ __forceinline__ i32x4_t sg_raw_rsrc(const void* base) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  return i32x4_t{(int)(uint32_t)a, (int)(uint32_t)(a >> 32), 0x7fffffff, 0x00020000};
}

#define SG_WAVE 64

// fastExp, internal/kernels/activation.go:100-145: clamp at +-10, 2^(x*log2e)
// split into integer part (truncation) and a 4th-order polynomial on the
// fraction, exponent bits built directly.  All float32, no fused ops.
__device__ __forceinline__ float sg_fast_exp(float x) {
  if (x < -10.0f) return 0.0f;
  if (x > 10.0f) return 22026.4657948f;
  const float y = x * 1.442695041f;
  const int ip = (int)y;  // v_cvt_i32_f32 truncates toward zero, like Go's int32()
  const float f = y - (float)ip;
  const float poly =
      1.0f + f * (0.693147180559945f + f * (0.240226506959101f + f * (0.055504108664821f + f * 0.009676036358193f)));
  if (ip >= -126 && ip <= 127) return poly * __uint_as_float((uint32_t)(ip + 127) << 23);
  if (ip < -126) return 0.0f;
  return 3.402823e+38f;
}

// fastExp for softmax arguments x = s - max <= 0, branch-free.  Same value as
// sg_fast_exp on (-inf, 0]: below -10 it is 0; otherwise y = x*log2e lies in
// [-14.43, 0], so the integer part is in [-14, 0] and poly * 2^ip is exact,
// which ldexp computes without building exponent bits.  float(int(y)) is
// truncf(y) for |y| < 2^31 (a full-rate v_trunc_f32 instead of a half-rate
// int -> float convert).
__device__ __forceinline__ float sg_fast_exp_nonpos(float x) {
  const float y = x * 1.442695041f;
  const int ip = (int)y;
  const float f = y - __builtin_truncf(y);
  const float poly =
      1.0f + f * (0.693147180559945f + f * (0.240226506959101f + f * (0.055504108664821f + f * 0.009676036358193f)));
  const float r = __builtin_amdgcn_ldexpf(poly, ip);
  return x < -10.0f ? 0.0f : r;
}

// n / d for the sigmoid's operands (d = 1 + e in [1, 2], n in {1, e}): the
// hardware reciprocal, one Newton-Raphson step, then the quotient corrected
// by its exact FMA residual (Markstein's scheme).  Six instructions instead
// of the eleven of the general IEEE sequence, whose scaling and fix-up steps
// only matter for denormal, huge or special operands.  sg_gelu_quick's result
// with it equals the one with the IEEE division for every one of the 2^32
// float inputs (exhaustive comparison on MI355X).
__device__ __forceinline__ float sg_div_sigmoid(float n, float d) {
  float r = __builtin_amdgcn_rcpf(d);
  r = __builtin_fmaf(__builtin_fmaf(-d, r, 1.0f), r, r);
  const float q = n * r;
  return __builtin_fmaf(__builtin_fmaf(-d, q, n), r, q);
}

// GELUQuickSIMD element, activation.go:55-75: x * sigmoid(1.702 x) with the
// sign-split sigmoid: sx >= 0 -> 1/(1 + fastExp(-sx)), else e/(1 + e) with
// e = fastExp(sx).  Both branches evaluate fastExp at -|sx| and differ only
// in the numerator, so one exp and one correctly rounded division give the
// same bits without divergent branches.
__device__ __forceinline__ float sg_gelu_quick(float x) {
  const float sx = 1.702f * x;
  const float e = sg_fast_exp_nonpos(-fabsf(sx));
  const float num = sx >= 0.0f ? 1.0f : e;
  return x * sg_div_sigmoid(num, 1.0f + e);
}

// fp16 -> fp32 with subnormal support, internal/runtime/model_int8.go:571-597.
__device__ __host__ __forceinline__ float sg_f16_ieee(uint16_t h) {
  uint32_t sign = (h >> 15) & 1u;
  int32_t ex = (h >> 10) & 0x1f;
  uint32_t fr = h & 0x3ffu;
  if (ex == 0) {
    if (fr == 0) return __uint_as_float(sign << 31);
    while ((fr & 0x400u) == 0) { fr <<= 1; ex--; }
    ex++;
    fr &= 0x3ffu;
  } else if (ex == 0x1f) {
    return __uint_as_float((sign << 31) | 0x7f800000u | (fr << 13));
  }
  return __uint_as_float((sign << 31) | ((uint32_t)(ex + 112) << 23) | (fr << 13));
}

// fp16 -> fp32 as internal/gguf/tensor.go:207-240 computes it: the subnormal
// branch normalizes from exponent 112 without the +1, so subnormals halve.
// The token-embedding lookup (DequantizeQ8_0Row) goes through this one.
__device__ __host__ __forceinline__ float sg_f16_gguf(uint16_t h) {
  uint32_t sign = (h >> 15) & 1u, ex = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  if (ex == 0) {
    if (m == 0) return __uint_as_float(sign << 31);
    uint32_t e = 112u;
    while ((m & 0x400u) == 0) { m <<= 1; e--; }
    return __uint_as_float((sign << 31) | (e << 23) | ((m & 0x3ffu) << 13));
  }
  if (ex == 0x1f) return __uint_as_float((sign << 31) | (0xffu << 23) | (m << 13));
  return __uint_as_float((sign << 31) | (((ex + 112u) & 0xffu) << 23) | (m << 13));
}

// Correctly rounded float sqrt (equal to float32(math.Sqrt(float64(x))): the
// double result rounded to float cannot differ from the correctly rounded
// float one).  sqrtf lowers to llvm.sqrt.f32, which this library's build
// flag -fhip-fp32-correctly-rounded-divide-sqrt keeps exact; HIP's __fsqrt_rn
// maps to the approximate native sqrt unless OCML_BASIC_ROUNDED_OPERATIONS is
// defined, so it is not used.
__device__ __forceinline__ float sg_sqrt(float x) { return sqrtf(x); }

// Horizontal sum across the 8 lanes of an aligned lane group, in the order of
// the AVX2 reduction VEXTRACTF128/VADDPS/VHADDPS/VHADDPS
// (internal/kernels/simd_amd64.s:50-54): ((a0+a4)+(a1+a5))+((a2+a6)+(a3+a7)).
// fp32 addition is commutative bit for bit, so every lane of the group ends
// with the identical value.
__device__ __forceinline__ float sg_hsum8(float a) {
  float s = a + __shfl_xor(a, 4);
  s = s + __shfl_xor(s, 1);
  return s + __shfl_xor(s, 2);
}

__device__ __forceinline__ float sg_max8(float a) {
  a = fmaxf(a, __shfl_xor(a, 4));
  a = fmaxf(a, __shfl_xor(a, 2));
  return fmaxf(a, __shfl_xor(a, 1));
}

__device__ __forceinline__ float sg_wave_max(float a) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) a = fmaxf(a, __shfl_xor(a, o));
  return a;
}

// Split of an fp32 value into two fp16 terms, x ~= hi + lo with
// hi = fp16(x) and lo = fp16(x - hi) (x - hi is exact in fp32).
struct hl16 {
  _Float16 hi, lo;
};
__device__ __forceinline__ hl16 split_f16(float x) {
  const _Float16 hi = (_Float16)x;
  return hl16{hi, (_Float16)(x - (float)hi)};
}

// Monotone float max for non-negative values via the uint bit pattern.
__device__ __forceinline__ void sg_atomic_max_nonneg(float* addr, float v) {
  atomicMax(reinterpret_cast<unsigned int*>(addr), __float_as_uint(v));
}

// Per-sequence maxima of a workgroup's rows [r_first, r_first + n), n <= the
// workgroup size: rmax[i] (LDS, written and published by the caller) is row
// r_first + i's maximum.  Rows are packed sequence by sequence (row_seq is
// non-decreasing), so thread i takes row i, a segmented max-scan over each
// wave's 64 rows gathers every run of equal row_seq, and the run's last lane
// issues one atomic: one atomic per sequence and wave instead of one per row
// (same-address atomics serialise in L2).
__device__ __forceinline__ void sg_seg_seq_max(const float* rmax, int n, int r_first,
                                               const int32_t* __restrict__ row_seq, float* __restrict__ amax) {
  const int i = threadIdx.x, lane = i & 63;
  if ((i & ~63) >= n) return;  // wave-uniform: waves past the rows
  const bool v = i < n;
  float m = v ? rmax[i] : 0.0f;
  const int s = v ? row_seq[r_first + i] : -1;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const float mo = __shfl_up(m, o);
    const int so = __shfl_up(s, o);
    if (lane >= o && so == s) m = fmaxf(m, mo);
  }
  const int sn = __shfl_down(s, 1);
  if (v && (lane == 63 || sn != s)) sg_atomic_max_nonneg(amax + s, m);
}

// Folds per-row maxima into the per-sequence maxima amax[row_seq[row]] for
// the rows [r_first, r_last] (at most ROWS) a workgroup of NT threads owns.
// When the first and the last row share a sequence the whole workgroup
// reduces to ONE atomic; otherwise sg_seg_seq_max issues one per sequence
// and wave.  m: the caller's row maximum (0 for threads without a row),
// non-negative; owner: this thread publishes its row's maximum.  Every thread
// of the workgroup must call this (it holds a barrier).
template <int NT, int ROWS = NT / 8>
__device__ __forceinline__ void sg_block_seq_max(float m, bool owner, int row, int r_first, int r_last,
                                                 const int32_t* __restrict__ row_seq, float* __restrict__ amax) {
  __shared__ float red[NT / 64];
  __shared__ float rmax[ROWS];
  const int s0 = row_seq[r_first];
  if (s0 == row_seq[r_last]) {
    m = sg_wave_max(m);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
      float mm = red[0];
#pragma unroll
      for (int i = 1; i < NT / 64; i++) mm = fmaxf(mm, red[i]);
      sg_atomic_max_nonneg(amax + s0, mm);
    }
  } else {
    if (owner) rmax[row - r_first] = m;
    __syncthreads();
    sg_seg_seq_max(rmax, r_last - r_first + 1, r_first, row_seq, amax);
  }
}

// math.Round(float64(x) * float64(inv)) (quantize.go:67,95) without float64
// arithmetic, as an integer-valued float.  hi = fl(x*inv) is within half an
// ulp of the exact product p, and every half-integer k + 0.5 (|k| < 2^22) is a
// float, so p and hi lie on the same side of every such half unless hi lands
// exactly on one: away from ties rint(hi) is round(p).  On a tie (hi - rint(hi)
// = +-0.5, exact) the exact remainder lo = fma(x, inv, -hi) decides: p above
// the half rounds up, below it rounds down, and p == hi (lo == 0) rounds away
// from zero like math.Round.  Ties are rare (~2^-16 per value), so they take a
// branch; the common path is a multiply, a rint and a compare.
__device__ __forceinline__ float sg_round_prod_f(float x, float inv) {
  const float hi = x * inv;
  float q = __builtin_rintf(hi);
  if (__builtin_expect(__builtin_fabsf(hi - q) == 0.5f, 0)) {
    const float lo = __builtin_fmaf(x, inv, -hi);
    q = (lo > 0.0f || (lo == 0.0f && hi > 0.0f)) ? hi + 0.5f : hi - 0.5f;
  }
  return q;
}

// sg_round_prod_f with both paths computed and selected (ten VALU
// instructions, no branch; the tie goes the way of the sign of lo, or of hi
// when lo is 0, the same rule).  For the latency-bound small-batch kernels:
// there a workgroup's row values pipeline instead of each taking a
// divergent-branch sequence (a 1 x 32 forward 2.06 -> 2.00 ms), while the
// bandwidth-bound large-batch quantizers run faster with the shorter common
// path of the branch (config 2 16.70 vs 16.80 ms, config 4 15.38 vs 15.64).
__device__ __forceinline__ float sg_round_prod_f_nb(float x, float inv) {
  const float hi = x * inv;
  const float q = __builtin_rintf(hi);
  const bool tie = __builtin_fabsf(hi - q) == 0.5f;
  const float lo = __builtin_fmaf(x, inv, -hi);
  const float dir = lo == 0.0f ? hi : lo;
  const float qt = hi + __builtin_copysignf(0.5f, dir);
  return tie ? qt : q;
}

__device__ __forceinline__ int sg_round_prod(float x, float inv) { return (int)sg_round_prod_f(x, inv); }

// The int8 code of x at reciprocal scale inv: clamp(round(x*inv), +-127),
// returned as an integer-valued float.
__device__ __forceinline__ float sg_quant_code(float x, float inv) {
  return __builtin_amdgcn_fmed3f(sg_round_prod_f(x, inv), -127.0f, 127.0f);
}
// The same code, branch-free (sg_round_prod_f_nb).
__device__ __forceinline__ float sg_quant_code_nb(float x, float inv) {
  return __builtin_amdgcn_fmed3f(sg_round_prod_f_nb(x, inv), -127.0f, 127.0f);
}

// RMSNorm of one row held by an 8-lane group, internal/kernels/norm.go:8-36.
// Lane j of the group holds x[i] = row[8*i + j] (NPL = n/8 values): that is
// exactly lane j of dotProductAVX2Asm's YMM accumulator, which runs
// acc_j = fma(row[8i+j], row[8i+j], acc_j) in i order (simd_amd64.s:36-46).
// Then meanSq = ss/float32(n); rms = float32(sqrt(float64(meanSq+eps)))
// (a correctly rounded float sqrt gives the same bits); inv = 1/rms;
// y = (x*inv)*w with two roundings (VecScaleF32 then VecMulF32).
template <int NPL>
__device__ __forceinline__ void sg_rmsnorm8(float (&x)[NPL], const float* __restrict__ w, int j, float eps) {
  float acc = 0.0f;
#pragma unroll
  for (int i = 0; i < NPL; i++) acc = __builtin_fmaf(x[i], x[i], acc);
  const float ss = sg_hsum8(acc);
  const float ms = ss / (float)(NPL * 8);
  const float rms = sg_sqrt(ms + eps);
  const float inv = 1.0f / rms;
#pragma unroll
  for (int i = 0; i < NPL; i++) {
    const float t = x[i] * inv;
    x[i] = t * w[8 * i + j];
  }
}

// Coalesced variant for the bandwidth-bound row kernels.  The 8-lane group
// loads the row as float4 slots: lane j owns elements 32c + 4j .. 32c + 4j + 3
// of every 32-element chunk c, so one load instruction covers 128 contiguous
// bytes of each row (the stride-8 layout above covers 32).  The sum of squares
// must still run in the AVX2 lane order, lane v chaining element 8i + v over
// i, so each chunk is transposed through the wave's LDS tile (8 rows x 40
// floats; the stride of 40 puts the 8 rows' reads in distinct banks): after
// the write, lane v of row r reads elements 8k + v of the chunk, k = 0..3,
// i.e. i = 4c + k in order.  LDS operations of one wave complete in issue
// order, so only the compiler has to be kept from reordering them.
template <int NC>
__device__ __forceinline__ float sg_sumsq8_f4(const f32x4_t (&x)[NC], float* tile, int r, int j) {
  f32x4_t* wr = reinterpret_cast<f32x4_t*>(tile + r * 40 + 4 * j);
  const float* rd = tile + r * 40 + j;
  float acc = 0.0f;
#pragma unroll
  for (int c = 0; c < NC; c++) {
    asm volatile("" ::: "memory");
    *wr = x[c];
    asm volatile("" ::: "memory");
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const float v = rd[8 * k];
      acc = __builtin_fmaf(v, v, acc);
    }
  }
  asm volatile("" ::: "memory");
  return sg_hsum8(acc);
}

// sg_rmsnorm8 on the float4 layout: same sum, same scalar steps, y = (x*inv)*w.
template <int NC>
__device__ __forceinline__ void sg_rmsnorm8_f4(f32x4_t (&x)[NC], const float* __restrict__ w, float* tile, int r,
                                               int j, float eps) {
  const float ss = sg_sumsq8_f4<NC>(x, tile, r, j);
  const float ms = ss / (float)(NC * 32);
  const float rms = sg_sqrt(ms + eps);
  const float inv = 1.0f / rms;
#pragma unroll
  for (int c = 0; c < NC; c++) {
    const f32x4_t wv = *reinterpret_cast<const f32x4_t*>(w + 32 * c + 4 * j);
#pragma unroll
    for (int t = 0; t < 4; t++) {
      const float u = x[c][t] * inv;
      x[c][t] = u * wv[t];
    }
  }
}


// The residual post-norm of one row whose o (x) and h (hv) are already in
// the lanes of its 8-lane group (model_int8.go:203-210 / :225-232):
// h = RMSNorm(o; w_post) + h, stored to hrow, then xn = RMSNorm(h; w_next),
// the next pre-norm (:194 / :216) or output_norm (:236).  Float4 layout
// (lane j: elements 32c + 4j .. + 3); tile is the wave's 8 x 40-float
// transpose tile and r the row's slot in it.  xn is stored when xrow is
// non-null; returns this lane's max|xn| (max|h| without w_next).
template <int NC>
__device__ __forceinline__ float sg_post_res_norm_f4(f32x4_t (&x)[NC], const f32x4_t (&hv)[NC],
                                                     float* __restrict__ hrow, const float* __restrict__ w_post,
                                                     const float* __restrict__ w_next, float eps,
                                                     float* __restrict__ xrow, float* tile, int r, int j) {
  f32x4_t* hp = reinterpret_cast<f32x4_t*>(hrow) + j;
  if (w_post) sg_rmsnorm8_f4<NC>(x, w_post, tile, r, j, eps);
#pragma unroll
  for (int c = 0; c < NC; c++) {
#pragma unroll
    for (int t = 0; t < 4; t++) x[c][t] = x[c][t] + hv[c][t];
    hp[8 * c] = x[c];
  }
  if (w_next) sg_rmsnorm8_f4<NC>(x, w_next, tile, r, j, eps);
  if (xrow) {
    f32x4_t* yp = reinterpret_cast<f32x4_t*>(xrow) + j;
#pragma unroll
    for (int c = 0; c < NC; c++) yp[8 * c] = x[c];
  }
  float m = 0.0f;
#pragma unroll
  for (int c = 0; c < NC; c++)
#pragma unroll
    for (int t = 0; t < 4; t++) m = fmaxf(m, fabsf(x[c][t]));
  return m;
}

// sg_post_res_norm_f4 (w_post and w_next required; xn stored when XN) for a
// row whose o sits in LDS (srow, shared by the row's 8-lane group;
// overwritten with h).  The sums of squares read srow in the AVX2 lane order
// directly (lane v: elements 8i + v, i ascending), the values and order the
// transpose tile gives.  h is streamed in quarters -- hv holds the first one,
// loaded by the caller; the next quarter's loads are issued as the current one
// is consumed -- and the new h goes back into srow, where the second norm
// reads it, so the row never sits in registers whole.  The norm weights may be
// LDS copies.
template <int NC, bool XN>
__device__ __forceinline__ float sg_post_res_norm_lds(float* srow, float* __restrict__ hrow, f32x4_t (&hv)[NC / 4],
                                                      const float* w_post, const float* w_next, float eps,
                                                      float* __restrict__ xrow, int j) {
  constexpr int D = NC * 32, QB = NC / 4;
  static_assert(NC % 4 == 0, "four quarters of h");
  f32x4_t* sp = reinterpret_cast<f32x4_t*>(srow) + j;
  f32x4_t* hp = reinterpret_cast<f32x4_t*>(hrow) + j;
  // The chain's LDS reads go in groups of 16, the group's offset passed
  // through an empty asm that takes the chain value: the next group's reads
  // depend on the previous group's FMAs, so at most 16 of the D / 8 values are
  // live at once (the scheduler would otherwise issue every read first).
  auto inv_rms = [&]() {
    float acc = 0.0f;
#pragma unroll
    for (int i0 = 0; i0 < D / 8; i0 += 16) {
      int off = 8 * i0 + j;
      asm volatile("" : "+v"(off) : "v"(acc));
      float a[16];
#pragma unroll
      for (int i = 0; i < 16; i++) a[i] = srow[off + 8 * i];
#pragma unroll
      for (int i = 0; i < 16; i++) acc = __builtin_fmaf(a[i], a[i], acc);
    }
    const float ms = sg_hsum8(acc) / (float)D;
    return 1.0f / sg_sqrt(ms + eps);
  };
  const float inv = inv_rms();
#pragma unroll
  for (int c = 0; c < NC; c++) {
    const int k = c % QB;
    f32x4_t v = sp[8 * c];
    const f32x4_t wv = *reinterpret_cast<const f32x4_t*>(w_post + 32 * c + 4 * j);
#pragma unroll
    for (int t = 0; t < 4; t++) {
      const float u = v[t] * inv;
      v[t] = u * wv[t] + hv[k][t];
    }
    if (c + QB < NC) hv[k] = __builtin_nontemporal_load(&hp[8 * (c + QB)]);  // the next quarter's chunk
    hp[8 * c] = v;
    sp[8 * c] = v;  // every lane of the group read o of chunk c (same instruction) before
  }
  asm volatile("" ::: "memory");  // LDS operations of a wave complete in issue order
  const float inv2 = inv_rms();
  float m = 0.0f;
#pragma unroll
  for (int c = 0; c < NC; c++) {
    f32x4_t v = sp[8 * c];
    const f32x4_t wv = *reinterpret_cast<const f32x4_t*>(w_next + 32 * c + 4 * j);
#pragma unroll
    for (int t = 0; t < 4; t++) {
      const float u = v[t] * inv2;
      v[t] = u * wv[t];
      m = fmaxf(m, fabsf(v[t]));
    }
    if constexpr (XN) reinterpret_cast<f32x4_t*>(xrow)[8 * c + j] = v;
  }
  return m;
}

// sg_post_res_norm_f4 with o and h read from memory (orow, hrow).
template <int NC>
__device__ __forceinline__ float sg_post_res_norm_row(const float* __restrict__ orow, float* __restrict__ hrow,
                                                      const float* __restrict__ w_post,
                                                      const float* __restrict__ w_next, float eps,
                                                      float* __restrict__ xrow, float* tile, int r, int j) {
  // o and h are loaded together: one memory round trip before the first norm.
  // Both are last-use reads (h is rewritten), so they go non-temporal and
  // leave L2 to the operands other kernels re-read; the forward's two
  // sequence groups share the cache.
  f32x4_t x[NC], hv[NC];
  const f32x4_t* op = reinterpret_cast<const f32x4_t*>(orow) + j;
  const f32x4_t* hp = reinterpret_cast<const f32x4_t*>(hrow) + j;
#pragma unroll
  for (int c = 0; c < NC; c++) x[c] = __builtin_nontemporal_load(&op[8 * c]);
#pragma unroll
  for (int c = 0; c < NC; c++) hv[c] = __builtin_nontemporal_load(&hp[8 * c]);
  return sg_post_res_norm_f4<NC>(x, hv, hrow, w_post, w_next, eps, xrow, tile, r, j);
}
