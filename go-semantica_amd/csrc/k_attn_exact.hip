// k_attn_exact.hip -- attention in the reference's exact float32 operation
// order, for callers that need the forward bit-identical to the reference's
// block-serial path (sg_model_set_attention_mode(SG_ATTN_EXACT),
// sg_attention_exact).  The default attention (k_attention.hip) runs its
// products on fp16 matrix cores and lands within 1e-5; this path runs every
// operation on the VALU in the order internal/kernels/attention.go fixes:
//
//   scores  computeAttentionScoresRange (attention.go:267-310) with
//           dotProductSIMD (simd_amd64.s:19-76): eight lanes, lane l chaining
//           fma(q[8i+l], k[8i+l], .) over i ascending, then the hsum
//           ((l0+l4)+(l1+l5))+((l2+l6)+(l3+l7)), then score * scale;
//   softmax Softmax (activation.go:161-213) per row: max, e = fastExp(x-max),
//           sum + (((e0+e1)+e2)+e3) per group of four in order, the tail one by
//           one, p = e * (1/sum) (uniform 1/n if the sum is 0);
//   P.V     processHeadRange (attention.go:235-262) + axpyAccum (:344-363):
//           o = 0, then over keys j ascending with p != 0, o = o + fl(p * v_j).
//
// GQA: head h reads K/V head h / (H / HKV) (model_int8.go:455-479).  The
// scores live in an fp32 buffer P[H][T][ldp] (row r of the packed batch,
// keys of its own sequence); the softmax turns them into weights in place.
// Everything is VALU-bound: about 4*H*hd*S^2 instructions per sequence, several
// times the matrix-core path's time.
#include <hip/hip_runtime.h>

#include "sg_device.h"
#include "sg_kernels.h"

namespace {

constexpr int kXT = 64;     // query rows and key rows per score tile
constexpr int kXD = 32;     // head dims staged in LDS per step (four 8-lane steps)
constexpr int kXHd = 256;   // head_dim
constexpr int kXRows = 32;  // query rows per P.V workgroup
constexpr int kXKeys = 64;  // keys per P.V LDS stage

// One 64 x 64 tile of one (sequence, head): 256 threads, thread (tx, ty) the
// 4 x 4 outputs of query rows ty + 16a and keys tx + 16b, each with its eight
// lane chains (consecutive lanes read consecutive LDS rows: with the 36-float
// row stride their 16-byte reads fall in distinct banks).
__global__ __launch_bounds__(256) void k_exact_scores(const float* __restrict__ q, int ldq,
                                                      const float* __restrict__ k, int ldk,
                                                      const int32_t* __restrict__ seq_off, int H, int group,
                                                      float scale, int tiles, float* __restrict__ P, int ldp, int T) {
  const int s = blockIdx.y / H, h = blockIdx.y % H;
  const int r0 = seq_off[s], S = seq_off[s + 1] - r0;
  const int qt = blockIdx.x / tiles, kt = blockIdx.x % tiles;
  if (qt * kXT >= S || kt * kXT >= S) return;  // uniform over the workgroup, before any barrier
  const int kvh = h / group;
  __shared__ __attribute__((aligned(16))) float qs[kXT][kXD + 4];
  __shared__ __attribute__((aligned(16))) float ks[kXT][kXD + 4];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  float acc[4][4][8];
#pragma unroll
  for (int a = 0; a < 4; a++)
#pragma unroll
    for (int b = 0; b < 4; b++)
#pragma unroll
      for (int l = 0; l < 8; l++) acc[a][b][l] = 0.0f;

  // 64 rows x 32 dims of Q and of K per chunk: 512 float4 each, two per
  // thread; the next chunk's are loaded into registers while this one computes.
  constexpr int kPer = kXT * kXD / 4 / 256;
  f32x4_t nq[kPer], nk[kPer];
  auto load_chunk = [&](int c) {
#pragma unroll
    for (int u = 0; u < kPer; u++) {
      const int e = threadIdx.x + 256 * u;
      const int row = e / (kXD / 4), c4 = e % (kXD / 4);
      const int qi = qt * kXT + row, kj = kt * kXT + row;
      nq[u] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      nk[u] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      if (qi < S) nq[u] = *reinterpret_cast<const f32x4_t*>(q + (int64_t)(r0 + qi) * ldq + h * kXHd + c + 4 * c4);
      if (kj < S) nk[u] = *reinterpret_cast<const f32x4_t*>(k + (int64_t)(r0 + kj) * ldk + kvh * kXHd + c + 4 * c4);
    }
  };
  load_chunk(0);
  for (int c = 0; c < kXHd; c += kXD) {
#pragma unroll
    for (int u = 0; u < kPer; u++) {
      const int e = threadIdx.x + 256 * u;
      const int row = e / (kXD / 4), c4 = e % (kXD / 4);
      *reinterpret_cast<f32x4_t*>(&qs[row][4 * c4]) = nq[u];
      *reinterpret_cast<f32x4_t*>(&ks[row][4 * c4]) = nk[u];
    }
    __syncthreads();
    if (c + kXD < kXHd) load_chunk(c + kXD);
#pragma unroll
    for (int t = 0; t < kXD; t += 8) {  // dims c+t .. c+t+7: step i = (c+t)/8 of every lane chain
      float qa[4][8], kb[4][8];
#pragma unroll
      for (int a = 0; a < 4; a++) {
        const f32x4_t v0 = *reinterpret_cast<const f32x4_t*>(&qs[ty + 16 * a][t]);
        const f32x4_t v1 = *reinterpret_cast<const f32x4_t*>(&qs[ty + 16 * a][t + 4]);
#pragma unroll
        for (int l = 0; l < 4; l++) {
          qa[a][l] = v0[l];
          qa[a][l + 4] = v1[l];
        }
      }
#pragma unroll
      for (int b = 0; b < 4; b++) {
        const f32x4_t v0 = *reinterpret_cast<const f32x4_t*>(&ks[tx + 16 * b][t]);
        const f32x4_t v1 = *reinterpret_cast<const f32x4_t*>(&ks[tx + 16 * b][t + 4]);
#pragma unroll
        for (int l = 0; l < 4; l++) {
          kb[b][l] = v0[l];
          kb[b][l + 4] = v1[l];
        }
      }
#pragma unroll
      for (int a = 0; a < 4; a++)
#pragma unroll
        for (int b = 0; b < 4; b++)
#pragma unroll
          for (int l = 0; l < 8; l++) acc[a][b][l] = __builtin_fmaf(qa[a][l], kb[b][l], acc[a][b][l]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int a = 0; a < 4; a++) {
    const int i = qt * kXT + ty + 16 * a;
    if (i >= S) continue;
    float* prow = P + ((int64_t)h * T + r0 + i) * ldp;
#pragma unroll
    for (int b = 0; b < 4; b++) {
      const int j = kt * kXT + tx + 16 * b;
      const float* L = acc[a][b];
      float sc = ((L[0] + L[4]) + (L[1] + L[5])) + ((L[2] + L[6]) + (L[3] + L[7]));
      sc = sc * scale;
      if (j < S) prow[j] = sc;
    }
  }
}

// Softmax of one score row per wave (4 rows per 256-thread workgroup).  Lane
// `lane` owns the groups of four keys g = 64c + lane (c < kMaxChunks); lane 0
// of the wave adds the group sums and the tail in the reference's order.
constexpr int kSmMaxKeys = 2048;
constexpr int kSmChunks = kSmMaxKeys / 4 / SG_WAVE;  // 8 chunks of 64 groups

__global__ __launch_bounds__(256) void k_exact_softmax(float* __restrict__ P, int ldp,
                                                       const int32_t* __restrict__ seq_off,
                                                       const int32_t* __restrict__ row_seq, int T, int H) {
  __shared__ __attribute__((aligned(16))) float gs[4][kSmMaxKeys / 4];
  __shared__ float tail[4][4];
  __shared__ float inv_s[4];
  __shared__ int uni_s[4];
  const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t w = (int64_t)blockIdx.x * 4 + wv;
  const bool valid = w < (int64_t)H * T;  // no early return: every wave reaches the barriers
  const int h = valid ? (int)(w / T) : 0, r = valid ? (int)(w % T) : 0;
  const int sq = valid ? row_seq[r] : 0;
  const int S = valid ? seq_off[sq + 1] - seq_off[sq] : 0;
  float* row = P + ((int64_t)h * T + r) * ldp;
  float e[kSmChunks][4];
  const int ng = S / 4;  // whole groups; keys 4*ng .. S-1 are the tail
  const int nch = (S + 4 * SG_WAVE - 1) / (4 * SG_WAVE);  // chunks of 64 groups the row needs
  // The row once, four keys per lane (16-byte loads; -inf past its end).
#pragma unroll
  for (int c = 0; c < kSmChunks; c++) {
    if (c >= nch) break;
    const int j = 4 * (c * SG_WAVE + lane);
    if (j + 3 < S) {
      const f32x4_t v = *reinterpret_cast<const f32x4_t*>(row + j);
#pragma unroll
      for (int t = 0; t < 4; t++) e[c][t] = v[t];
    } else {
#pragma unroll
      for (int t = 0; t < 4; t++) e[c][t] = j + t < S ? row[j + t] : -__builtin_inff();
    }
  }
  // the row's maximum (any order gives the sequential `>` scan's value)
  float m = -__builtin_inff();
#pragma unroll
  for (int c = 0; c < kSmChunks; c++) {
    if (c >= nch) break;
#pragma unroll
    for (int t = 0; t < 4; t++) m = fmaxf(m, e[c][t]);
  }
  m = sg_wave_max(m);
#pragma unroll
  for (int c = 0; c < kSmChunks; c++) {
    if (c >= nch) break;
    const int g = c * SG_WAVE + lane;
    const int j = 4 * g;
#pragma unroll
    for (int t = 0; t < 4; t++) e[c][t] = (j + t < S) ? sg_fast_exp(e[c][t] - m) : 0.0f;
    if (g < ng) gs[wv][g] = ((e[c][0] + e[c][1]) + e[c][2]) + e[c][3];
    else if (g == ng && j < S)
      for (int t = 0; t < 4; t++) tail[wv][t] = e[c][t];
  }
  __syncthreads();
  if (lane == 0 && valid) {
    // The serial sum: group sums read 16 at a time, so one LDS round trip
    // serves 16 dependent adds.
    float sum = 0.0f;
    int g = 0;
    for (; g + 16 <= ng; g += 16) {
      f32x4_t b[4];
#pragma unroll
      for (int u = 0; u < 4; u++) b[u] = *reinterpret_cast<const f32x4_t*>(&gs[wv][g + 4 * u]);
#pragma unroll
      for (int u = 0; u < 4; u++)
#pragma unroll
        for (int t = 0; t < 4; t++) sum = sum + b[u][t];
    }
    for (; g < ng; g++) sum = sum + gs[wv][g];
    for (int j = 4 * ng; j < S; j++) sum = sum + tail[wv][j - 4 * ng];
    uni_s[wv] = sum == 0.0f;
    inv_s[wv] = sum == 0.0f ? 1.0f / (float)S : 1.0f / sum;
  }
  __syncthreads();
  if (!valid) return;
  const float inv = inv_s[wv];
  const bool uni = uni_s[wv] != 0;
#pragma unroll
  for (int c = 0; c < kSmChunks; c++) {
    if (c >= nch) break;
    const int j = 4 * (c * SG_WAVE + lane);
    f32x4_t v;
#pragma unroll
    for (int t = 0; t < 4; t++) v[t] = uni ? inv : e[c][t] * inv;
    if (j + 3 < S) {
      *reinterpret_cast<f32x4_t*>(row + j) = v;
    } else {
#pragma unroll
      for (int t = 0; t < 4; t++)
        if (j + t < S) row[j + t] = v[t];
    }
  }
}

// out[r][h*256 + d] for 32 query rows of one (sequence, head): thread d, one
// chain per row over the keys in order.  The weights of 64 keys are staged in
// LDS per step; V's row j is one coalesced 1-KB read shared by the 32 rows.
__global__ __launch_bounds__(256) void k_exact_pv(const float* __restrict__ P, int ldp, const float* __restrict__ v,
                                                  int ldv, const int32_t* __restrict__ seq_off, int H, int group,
                                                  float* __restrict__ out, int ldo, int T, float* __restrict__ amax) {
  const int s = blockIdx.y / H, h = blockIdx.y % H;
  const int r0 = seq_off[s], S = seq_off[s + 1] - r0;
  const int i0 = blockIdx.x * kXRows;
  if (i0 >= S) return;  // uniform, before any barrier
  const int kvh = h / group, d = threadIdx.x;
  __shared__ __attribute__((aligned(16))) float ps[kXRows][kXKeys];
  float acc[kXRows];
#pragma unroll
  for (int i = 0; i < kXRows; i++) acc[i] = 0.0f;
  const float* vcol = v + (int64_t)r0 * ldv + kvh * kXHd + d;
  for (int j0 = 0; j0 < S; j0 += kXKeys) {
    // 32 rows x 64 keys of weights (zeros past the sequence's rows or keys)
#pragma unroll
    for (int e = threadIdx.x; e < kXRows * kXKeys; e += 256) {
      const int i = e / kXKeys, jj = e % kXKeys;
      float pv = 0.0f;
      if (i0 + i < S && j0 + jj < S) pv = P[((int64_t)h * T + r0 + i0 + i) * ldp + j0 + jj];
      ps[i][jj] = pv;
    }
    __syncthreads();
    const int nk = min(kXKeys, S - j0);
    // Keys in batches of 4: their V loads go out together, and each row's 4
    // weights are one LDS read.  Keys past nk carry weight 0 in ps and a
    // clamped (in-range) V row, so they take the skip like any zero weight.
    for (int jb = 0; jb < nk; jb += 4) {
      float vj[4];
#pragma unroll
      for (int u = 0; u < 4; u++) vj[u] = vcol[(int64_t)(j0 + min(jb + u, nk - 1)) * ldv];
      // The reference skips keys of weight 0.  With v finite that changes
      // nothing: the product is +-0, and o + (+-0) = o, since o starts at +0 and
      // a sum is -0 only when both terms are.  So the skip is taken only when
      // this wave's values of the batch include an infinity or a NaN.
      const bool finite = __builtin_isfinite(vj[0]) && __builtin_isfinite(vj[1]) && __builtin_isfinite(vj[2]) &&
                          __builtin_isfinite(vj[3]);
      if (__ballot(!finite) == 0 && jb + 4 <= nk) {
#pragma unroll
        for (int i = 0; i < kXRows; i++) {
          const f32x4_t pw = *reinterpret_cast<const f32x4_t*>(&ps[i][jb]);
#pragma unroll
          for (int u = 0; u < 4; u++) {
            const float t = vj[u] * pw[u];  // VecScaleF32: one rounding
            acc[i] = acc[i] + t;            // VecAddF32
          }
        }
      } else {
#pragma unroll
        for (int i = 0; i < kXRows; i++) {
          const f32x4_t pw = *reinterpret_cast<const f32x4_t*>(&ps[i][jb]);
#pragma unroll
          for (int u = 0; u < 4; u++) {
            const float t = vj[u] * pw[u];
            if (pw[u] != 0.0f) acc[i] = acc[i] + t;
          }
        }
      }
    }
    __syncthreads();
  }
  float m = 0.0f;
#pragma unroll
  for (int i = 0; i < kXRows; i++)
    if (i0 + i < S) {
      out[(int64_t)(r0 + i0 + i) * ldo + h * kXHd + d] = acc[i];
      m = fmaxf(m, fabsf(acc[i]));
    }
  if (amax) {  // the sequence's max|o| for the quantizer: one atomic per workgroup
    __shared__ float red[4];
    m = sg_wave_max(m);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) sg_atomic_max_nonneg(amax + s, fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])));
  }
}

inline unsigned ceil_div(int64_t n, int per) { return (unsigned)((n + per - 1) / per); }

}  // namespace

namespace sgk {

size_t attention_exact_scratch(int T, int H, int max_len) {
  const int ldp = (max_len + 63) / 64 * 64;
  return sizeof(float) * (size_t)H * (size_t)T * (size_t)ldp;
}

hipError_t attention_exact(const float* q, int ldq, const float* k, const float* v, int ldkv, float* out, int ldo,
                           const int32_t* seq_off, const int32_t* row_seq, int n_seq, int T, int H, int HKV, int hd,
                           float scale, int max_len, float* P, float* amax, hipStream_t s) {
  if (T <= 0 || n_seq <= 0) return hipSuccess;
  if (hd != kXHd || HKV <= 0 || H % HKV || max_len > kSmMaxKeys || max_len <= 0 || (int64_t)n_seq * H > 65535)
    return hipErrorInvalidValue;
  if ((ldq & 3) || (ldkv & 3) || (reinterpret_cast<uintptr_t>(q) & 15) || (reinterpret_cast<uintptr_t>(k) & 15))
    return hipErrorInvalidValue;  // float4 staging of Q and K rows
  const int ldp = (max_len + 63) / 64 * 64, group = H / HKV;
  const int tiles = (int)ceil_div(max_len, kXT);
  hipLaunchKernelGGL(k_exact_scores, dim3(tiles * tiles, n_seq * H), dim3(256), 0, s, q, ldq, k, ldkv, seq_off, H,
                     group, scale, tiles, P, ldp, T);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k_exact_softmax, dim3(ceil_div((int64_t)H * T, 4)), dim3(256), 0, s, P, ldp, seq_off, row_seq,
                     T, H);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k_exact_pv, dim3(ceil_div(max_len, kXRows), n_seq * H), dim3(256), 0, s, P, ldp, v, ldkv,
                     seq_off, H, group, out, ldo, T, amax);
  return hipGetLastError();
}

}  // namespace sgk
