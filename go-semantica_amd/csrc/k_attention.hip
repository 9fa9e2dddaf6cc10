// k_attention.hip -- bidirectional MQA attention over packed variable-length
// sequences (MultiHeadAttentionChunked with mask=nil,
// internal/kernels/attention.go:88-363; GQA expansion model_int8.go:455-479).
//
// Reference semantics kept:
//   s_ij = (q_i . k_j) * scale                         (scale = 1/sqrt(head_dim))
//   m_i  = max_j s_ij                                  (exact, before any exp)
//   e_ij = fastExp(s_ij - m_i)  -- 0 when s_ij - m_i < -10 (activation.go:104-106)
//   o_i  = sum_j e_ij v_j / sum_j e_ij
// fastExp is not multiplicative and clamps, so an online (running-max)
// softmax would change which keys are zeroed; the kernel therefore makes two
// passes over the keys: pass 1 finds the exact row max, pass 2 forms e, the
// row sum and P.V.  The products run on fp16 matrix cores with fp32
// accumulation (q, k, v rounded to fp16; e scaled by 2^10 before rounding so
// small weights stay out of the fp16 subnormal range; the scale is undone
// exactly at the end).
//
// One workgroup = one (sequence, 32-query block, kv head); wave w handles
// query head kv*G + w, so every K/V tile staged in LDS serves all G query
// heads that share it.  Scores are computed transposed (S^T = K Q^T): each
// lane then owns one query and 16 of the 32 keys of a tile, the row max needs
// a single cross-lane step, and the score registers feed the P.V product as
// its B operand with no shuffles (P^T in O^T = V^T P^T).
#include "sg_device.h"
#include "sg_kernels.h"

namespace {

constexpr int BK = 32, KPAD = 8, VPAD = 8;  // 32 keys per tile; LDS row padding
constexpr float kPScale = 1024.0f, kPUnscale = 1.0f / 1024.0f;

template <int HD, int G>
__global__ __launch_bounds__(G* SG_WAVE) void k_attention(const float* __restrict__ q, int ldq,
                                                          const float* __restrict__ k, const float* __restrict__ v,
                                                          int ldkv, float* __restrict__ out, int ldo,
                                                          const int32_t* __restrict__ seq_off,
                                                          const sg_item* __restrict__ items, float scale,
                                                          float* __restrict__ amax) {
  __shared__ _Float16 Ks[BK][HD + KPAD];
  __shared__ _Float16 Vt[HD][BK + VPAD];
  constexpr int NT = G * SG_WAVE;
  constexpr int NC = HD / 16;  // 16-wide k chunks of the QK^T product
  constexpr int ND = HD / 32;  // 32-wide output column tiles of P.V

  const sg_item it = items[blockIdx.x];
  const int kvh = blockIdx.y;
  const int r0 = seq_off[it.seq];
  const int S = seq_off[it.seq + 1] - r0;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int lr = lane & 31, lh = lane >> 5;
  const int head = kvh * G + w;
  const int qrow = it.q0 + lr;
  const bool qvalid = qrow < S;

  // Q^T as the B operand: lane owns query qrow, dims 16c + 8*lh .. +8.
  half8_t qb[NC];
  {
    const float* qp = q + (int64_t)(r0 + (qvalid ? qrow : S - 1)) * ldq + head * HD + 8 * lh;
#pragma unroll
    for (int c = 0; c < NC; c++) {
      const f32x4_t x0 = *reinterpret_cast<const f32x4_t*>(qp + 16 * c);
      const f32x4_t x1 = *reinterpret_cast<const f32x4_t*>(qp + 16 * c + 4);
      half8_t h;
#pragma unroll
      for (int t = 0; t < 4; t++) {
        h[t] = (_Float16)x0[t];
        h[t + 4] = (_Float16)x1[t];
      }
      qb[c] = h;
    }
  }

  const float* kbase = k + (int64_t)r0 * ldkv + kvh * HD;
  const float* vbase = v + (int64_t)r0 * ldkv + kvh * HD;

  auto load_k = [&](int kt) {
    for (int idx = tid; idx < BK * HD / 4; idx += NT) {
      const int key = idx / (HD / 4), d4 = idx % (HD / 4);
      const int kr = kt + key < S ? kt + key : S - 1;
      const f32x4_t x = *reinterpret_cast<const f32x4_t*>(kbase + (int64_t)kr * ldkv + 4 * d4);
      half4_t h;
#pragma unroll
      for (int t = 0; t < 4; t++) h[t] = (_Float16)x[t];
      *reinterpret_cast<half4_t*>(&Ks[key][4 * d4]) = h;
    }
  };
  auto load_vt = [&](int kt) {
    for (int idx = tid; idx < BK * HD / 4; idx += NT) {
      const int key = idx % BK, d4 = idx / BK;
      const int kr = kt + key < S ? kt + key : S - 1;
      const f32x4_t x = *reinterpret_cast<const f32x4_t*>(vbase + (int64_t)kr * ldkv + 4 * d4);
#pragma unroll
      for (int t = 0; t < 4; t++) Vt[4 * d4 + t][key] = (_Float16)x[t];
    }
  };
  // S^T tile: lane owns query lr; register r holds key 8*(r/4) + 4*lh + r%4.
  auto scores = [&]() {
    f32x16_t acc = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int c = 0; c < NC; c++) {
      const half8_t a = *reinterpret_cast<const half8_t*>(&Ks[lr][16 * c + 8 * lh]);
      acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qb[c], acc, 0, 0, 0);
    }
    return acc;
  };

  // ---- pass 1: exact row max ----
  float m = -INFINITY;
  for (int kt = 0; kt < S; kt += BK) {
    __syncthreads();
    load_k(kt);
    __syncthreads();
    const f32x16_t sc = scores();
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int key = kt + 8 * (r >> 2) + 4 * lh + (r & 3);
      if (key < S) m = fmaxf(m, sc[r] * scale);
    }
  }
  m = fmaxf(m, __shfl_xor(m, 32));

  // ---- pass 2: e = fastExp(s - m), row sums, O^T += V^T P^T ----
  f32x16_t o[ND];
#pragma unroll
  for (int dc = 0; dc < ND; dc++)
#pragma unroll
    for (int r = 0; r < 16; r++) o[dc][r] = 0.0f;
  float lsum = 0.0f;
  for (int kt = 0; kt < S; kt += BK) {
    __syncthreads();
    load_k(kt);
    load_vt(kt);
    __syncthreads();
    const f32x16_t sc = scores();
    half8_t p0, p1;
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int key = kt + 8 * (r >> 2) + 4 * lh + (r & 3);
      const float e = key < S ? sg_fast_exp(sc[r] * scale - m) : 0.0f;
      lsum = lsum + e;
      const _Float16 ph = (_Float16)(e * kPScale);
      if (r < 8) p0[r] = ph; else p1[r - 8] = ph;
    }
    // A operand = V^T rows (dims) with the keys this lane half placed in its
    // P slots: slots 0..3 <- keys 4lh..4lh+3, 4..7 <- 8+4lh.. (p0); +16 for p1.
#pragma unroll
    for (int dc = 0; dc < ND; dc++) {
      const _Float16* vr = &Vt[32 * dc + lr][0];
      const half4_t x0 = *reinterpret_cast<const half4_t*>(vr + 4 * lh);
      const half4_t x1 = *reinterpret_cast<const half4_t*>(vr + 8 + 4 * lh);
      const half4_t x2 = *reinterpret_cast<const half4_t*>(vr + 16 + 4 * lh);
      const half4_t x3 = *reinterpret_cast<const half4_t*>(vr + 24 + 4 * lh);
      const half8_t a0 = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
      const half8_t a1 = {x2[0], x2[1], x2[2], x2[3], x3[0], x3[1], x3[2], x3[3]};
      o[dc] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, p0, o[dc], 0, 0, 0);
      o[dc] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, p1, o[dc], 0, 0, 0);
    }
  }
  lsum = lsum + __shfl_xor(lsum, 32);
  const float f = (1.0f / lsum) * kPUnscale;

  // O^T layout: lane owns query lr; register r of tile dc is dim 32dc + 8(r/4) + 4lh + r%4.
  float mx = 0.0f;
  if (qvalid) {
    float* op = out + (int64_t)(r0 + qrow) * ldo + head * HD + 4 * lh;
#pragma unroll
    for (int dc = 0; dc < ND; dc++) {
#pragma unroll
      for (int g4 = 0; g4 < 4; g4++) {
        f32x4_t y;
#pragma unroll
        for (int t = 0; t < 4; t++) {
          y[t] = o[dc][4 * g4 + t] * f;
          mx = fmaxf(mx, fabsf(y[t]));
        }
        *reinterpret_cast<f32x4_t*>(op + 32 * dc + 8 * g4) = y;
      }
    }
  }
  if (amax) {
    mx = sg_wave_max(mx);
    if (lane == 0) sg_atomic_max_nonneg(amax + it.seq, mx);
  }
}

}  // namespace

namespace sgk {

hipError_t attention(const float* q, int ldq, const float* k, const float* v, int ldkv, float* out, int ldo,
                     const int32_t* seq_off, const sg_item* items, int n_items, int H, int HKV, int hd, float scale,
                     float* amax, hipStream_t s) {
  if (n_items <= 0) return hipSuccess;
  if (hd != 256 || HKV <= 0 || H % HKV) return hipErrorInvalidValue;
  if ((ldq | ldkv | ldo) & 3) return hipErrorInvalidValue;
  const int G = H / HKV;
  dim3 grid(n_items, HKV);
  switch (G) {
    case 1: hipLaunchKernelGGL((k_attention<256, 1>), grid, dim3(64), 0, s, q, ldq, k, v, ldkv, out, ldo, seq_off, items, scale, amax); break;
    case 2: hipLaunchKernelGGL((k_attention<256, 2>), grid, dim3(128), 0, s, q, ldq, k, v, ldkv, out, ldo, seq_off, items, scale, amax); break;
    case 3: hipLaunchKernelGGL((k_attention<256, 3>), grid, dim3(192), 0, s, q, ldq, k, v, ldkv, out, ldo, seq_off, items, scale, amax); break;
    case 4: hipLaunchKernelGGL((k_attention<256, 4>), grid, dim3(256), 0, s, q, ldq, k, v, ldkv, out, ldo, seq_off, items, scale, amax); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace sgk
