// k_attention.hip -- bidirectional MQA attention over packed variable-length
// sequences (MultiHeadAttentionChunked with mask=nil,
// internal/kernels/attention.go:88-363; GQA expansion model_int8.go:455-479).
//
// Reference semantics kept:
//   s_ij = (q_i . k_j) * scale                         (scale = 1/sqrt(head_dim))
//   m_i  = max_j s_ij                                  (before any exp)
//   e_ij = fastExp(s_ij - m_i)  -- 0 when s_ij - m_i < -10 (activation.go:104-106)
//   o_i  = sum_j e_ij v_j / sum_j e_ij
// fastExp is not multiplicative and clamps, so an online (running-max)
// softmax would change the weights; the kernel makes two passes over the
// keys: pass 1 finds the row max, pass 2 forms e, the row sum and P.V.
//
// Precision.  The attention output is re-quantized to int8 with a
// per-sequence scale right after this kernel, so an error of 2^-12 (plain
// fp16 operands) flips a few percent of the int8 codes by a whole quantum and
// the flips compound over 24 layers.  Both products therefore run as split
// fp16 on the matrix cores: x = hi + lo with hi = fp16(x), lo = fp16(x - hi),
// and a.b = ah.bh + ah.bl + al.bh accumulated in fp32 (about 2^-22 relative,
// the level of the reference's own fp32 rounding).  Q and K are scaled by 8
// before splitting (exact) to keep lo out of the fp16 subnormal range; the
// weights e are scaled by 2^10 for the same reason; both scalings are undone
// exactly.  Pass 1 computes the same split scores, so the max is the max of
// the scores pass 2 exponentiates (a max that is off by even 1e-4 moves every
// fastExp argument and, through fastExp's polynomial error, the weights by
// ~1e-5).
//
// Work split: one workgroup = one (sequence, 32-query block, kv head), 6
// waves = 2 sub-blocks of 16 queries x G=3 query heads, so every K/V tile
// staged in LDS serves all heads that share it.  Scores are computed
// transposed (S^T = K Q^T, v_mfma_f32_16x16x32_f16): a lane owns one query
// and 4 keys of each 16-key subtile, and those registers are exactly the B
// operand slots of O^T = V^T P^T -- no shuffles between the two products.
#include "sg_device.h"
#include "sg_kernels.h"

namespace {

constexpr int BK = 32;          // keys per tile
constexpr int QW = 16;          // queries per wave
constexpr int QB = 32 / QW;     // query sub-blocks per workgroup
constexpr int KPAD = 8, VPAD = 8;
constexpr float kQKScale = 8.0f;
constexpr float kPScale = 1024.0f, kPUnscale = 1.0f / 1024.0f;

struct hl16 {
  _Float16 hi, lo;
};
__device__ __forceinline__ hl16 split_f16(float x) {
  const _Float16 hi = (_Float16)x;
  return hl16{hi, (_Float16)(x - (float)hi)};
}

__device__ __forceinline__ f32x4_t mfma16(half8_t a, half8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

template <int HD, int G>
__global__ __launch_bounds__(G* QB* SG_WAVE) void k_attention(const float* __restrict__ q, int ldq,
                                                              const float* __restrict__ k,
                                                              const float* __restrict__ v, int ldkv,
                                                              float* __restrict__ out, int ldo,
                                                              const int32_t* __restrict__ seq_off,
                                                              const sg_item* __restrict__ items, float scale,
                                                              float* __restrict__ amax) {
  __shared__ _Float16 Kh[BK][HD + KPAD], Kl[BK][HD + KPAD];
  __shared__ _Float16 Vh[HD][BK + VPAD], Vl[HD][BK + VPAD];  // V^T
  constexpr int NT = G * QB * SG_WAVE;
  constexpr int NC = HD / 32;  // 32-dim chunks (k of the QK^T MFMA)
  constexpr int ND = HD / 16;  // 16-dim output tiles of P.V

  const sg_item it = items[blockIdx.x];
  const int kvh = blockIdx.y;
  const int r0 = seq_off[it.seq];
  const int S = seq_off[it.seq + 1] - r0;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int lq = lane & 15, lg = lane >> 4;  // column (query) and row group of the 16x16 tiles
  const int head = kvh * G + (w % G);
  const int qrow = it.q0 + (w / G) * QW + lq;
  const bool qvalid = qrow < S;

  // Q^T as the B operand: lane owns query qrow, dims 32c + 8*lg .. +8 (scaled by 8, split).
  half8_t qh[NC], ql[NC];
  {
    const float* qp = q + (int64_t)(r0 + (qvalid ? qrow : S - 1)) * ldq + head * HD + 8 * lg;
#pragma unroll
    for (int c = 0; c < NC; c++) {
      const f32x4_t x0 = *reinterpret_cast<const f32x4_t*>(qp + 32 * c);
      const f32x4_t x1 = *reinterpret_cast<const f32x4_t*>(qp + 32 * c + 4);
#pragma unroll
      for (int t = 0; t < 4; t++) {
        const hl16 a = split_f16(x0[t] * kQKScale), b = split_f16(x1[t] * kQKScale);
        qh[c][t] = a.hi;
        ql[c][t] = a.lo;
        qh[c][t + 4] = b.hi;
        ql[c][t + 4] = b.lo;
      }
    }
  }

  const float* kbase = k + (int64_t)r0 * ldkv + kvh * HD;
  const float* vbase = v + (int64_t)r0 * ldkv + kvh * HD;

  auto load_k = [&](int kt) {
    for (int idx = tid; idx < BK * HD / 4; idx += NT) {
      const int key = idx / (HD / 4), d4 = idx % (HD / 4);
      const int kr = kt + key < S ? kt + key : S - 1;
      const f32x4_t x = *reinterpret_cast<const f32x4_t*>(kbase + (int64_t)kr * ldkv + 4 * d4);
      half4_t h, l;
#pragma unroll
      for (int t = 0; t < 4; t++) {
        const hl16 p = split_f16(x[t] * kQKScale);
        h[t] = p.hi;
        l[t] = p.lo;
      }
      *reinterpret_cast<half4_t*>(&Kh[key][4 * d4]) = h;
      *reinterpret_cast<half4_t*>(&Kl[key][4 * d4]) = l;
    }
  };
  auto load_v = [&](int kt) {
    for (int idx = tid; idx < BK * HD / 4; idx += NT) {
      const int key = idx % BK, d4 = idx / BK;
      const int kr = kt + key < S ? kt + key : S - 1;
      const f32x4_t x = *reinterpret_cast<const f32x4_t*>(vbase + (int64_t)kr * ldkv + 4 * d4);
#pragma unroll
      for (int t = 0; t < 4; t++) {
        const hl16 p = split_f16(x[t]);
        Vh[4 * d4 + t][key] = p.hi;
        Vl[4 * d4 + t][key] = p.lo;
      }
    }
  };

  // Scores of key subtile st of the staged tile, split product (scaled by 64).
  // S^T subtile: lane holds query lq, keys 16*st + 4*lg + r (r = 0..3).
  auto scores = [&](int st) {
    f32x4_t acc = {0, 0, 0, 0};
#pragma unroll
    for (int c = 0; c < NC; c++) {
      const half8_t ah = *reinterpret_cast<const half8_t*>(&Kh[16 * st + lq][32 * c + 8 * lg]);
      const half8_t al = *reinterpret_cast<const half8_t*>(&Kl[16 * st + lq][32 * c + 8 * lg]);
      acc = mfma16(ah, qh[c], acc);
      acc = mfma16(ah, ql[c], acc);
      acc = mfma16(al, qh[c], acc);
    }
    return acc;
  };
  const float sscale = scale / (kQKScale * kQKScale);

  // ---- pass 1: row max ----
  float m = -INFINITY;
  for (int kt = 0; kt < S; kt += BK) {
    __syncthreads();
    load_k(kt);
    __syncthreads();
#pragma unroll
    for (int st = 0; st < 2; st++) {
      const f32x4_t acc = scores(st);
#pragma unroll
      for (int r = 0; r < 4; r++)
        if (kt + 16 * st + 4 * lg + r < S) m = fmaxf(m, acc[r] * sscale);
    }
  }
  m = fmaxf(m, __shfl_xor(m, 16));
  m = fmaxf(m, __shfl_xor(m, 32));

  // ---- pass 2: e = fastExp(s - m), row sums, O^T += V^T P^T ----
  f32x4_t o[ND];
#pragma unroll
  for (int dt = 0; dt < ND; dt++) o[dt] = f32x4_t{0, 0, 0, 0};
  float lsum = 0.0f;
  for (int kt = 0; kt < S; kt += BK) {
    __syncthreads();
    load_k(kt);
    load_v(kt);
    __syncthreads();
    half8_t ph, pl;  // slots 0..3: keys 4lg+r of subtile 0; slots 4..7: 16+4lg+r
#pragma unroll
    for (int st = 0; st < 2; st++) {
      const f32x4_t acc = scores(st);
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const float e = kt + 16 * st + 4 * lg + r < S ? sg_fast_exp(acc[r] * sscale - m) : 0.0f;
        lsum = lsum + e;
        const hl16 p = split_f16(e * kPScale);
        ph[4 * st + r] = p.hi;
        pl[4 * st + r] = p.lo;
      }
    }
#pragma unroll
    for (int dt = 0; dt < ND; dt++) {
      const _Float16* vh = &Vh[16 * dt + lq][0];
      const _Float16* vl = &Vl[16 * dt + lq][0];
      const half4_t h0 = *reinterpret_cast<const half4_t*>(vh + 4 * lg);
      const half4_t h1 = *reinterpret_cast<const half4_t*>(vh + 16 + 4 * lg);
      const half4_t l0 = *reinterpret_cast<const half4_t*>(vl + 4 * lg);
      const half4_t l1 = *reinterpret_cast<const half4_t*>(vl + 16 + 4 * lg);
      const half8_t ah = {h0[0], h0[1], h0[2], h0[3], h1[0], h1[1], h1[2], h1[3]};
      const half8_t al = {l0[0], l0[1], l0[2], l0[3], l1[0], l1[1], l1[2], l1[3]};
      o[dt] = mfma16(ah, ph, o[dt]);
      o[dt] = mfma16(ah, pl, o[dt]);
      o[dt] = mfma16(al, ph, o[dt]);
    }
  }
  lsum = lsum + __shfl_xor(lsum, 16);
  lsum = lsum + __shfl_xor(lsum, 32);
  const float f = (1.0f / lsum) * kPUnscale;

  // O^T tile dt: lane holds query lq, dims 16*dt + 4*lg + r.
  float mx = 0.0f;
  if (qvalid) {
    float* op = out + (int64_t)(r0 + qrow) * ldo + head * HD + 4 * lg;
#pragma unroll
    for (int dt = 0; dt < ND; dt++) {
      f32x4_t y;
#pragma unroll
      for (int r = 0; r < 4; r++) {
        y[r] = o[dt][r] * f;
        mx = fmaxf(mx, fabsf(y[r]));
      }
      *reinterpret_cast<f32x4_t*>(op + 16 * dt) = y;
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
    case 1: hipLaunchKernelGGL((k_attention<256, 1>), grid, dim3(1 * QB * 64), 0, s, q, ldq, k, v, ldkv, out, ldo, seq_off, items, scale, amax); break;
    case 2: hipLaunchKernelGGL((k_attention<256, 2>), grid, dim3(2 * QB * 64), 0, s, q, ldq, k, v, ldkv, out, ldo, seq_off, items, scale, amax); break;
    case 3: hipLaunchKernelGGL((k_attention<256, 3>), grid, dim3(3 * QB * 64), 0, s, q, ldq, k, v, ldkv, out, ldo, seq_off, items, scale, amax); break;
    case 4: hipLaunchKernelGGL((k_attention<256, 4>), grid, dim3(4 * QB * 64), 0, s, q, ldq, k, v, ldkv, out, ldo, seq_off, items, scale, amax); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace sgk
