// sg_kv_prep.h -- device bodies shared by the QK-norm/RoPE split kernel,
// the V^T split kernel and the kernel that does both in one launch.
#pragma once
#include "sg_device.h"
#include "sg_kernels.h"

namespace sgd {

constexpr int kKvThreads = 256;  // threads per workgroup of every kernel using these bodies
constexpr int kKvRows = 32;      // (token, head) rows per workgroup of the QK split: 8 lanes each
constexpr int kVtRowStride = 256 + 4;  // fp32 LDS row stride of the V tile

// Key order inside a V^T tile row.  Lane group g (lane/16) of an attention
// wave holds the S^T entries of keys 4g..4g+3 (first 16-key subtile) and
// 16+4g..16+4g+3 (second); as the B operand of a 32-key MFMA step its slots
// are positions 8g..8g+7, so key k is stored at position
// 8*((k&15)>>2) + 4*(k>>4) + (k&3) and position p holds key:
__device__ __forceinline__ int vt_key(int p) { return ((p & 4) << 2) | ((p & 24) >> 1) | (p & 3); }

// One 8-lane group per (token, head): g = token * (H + HKV) + head (query
// heads first).  RMSNorm with attn_q_norm/attn_k_norm (model_int8.go:374-440),
// then the cached NeoX rotation of pairs (i, i+128) at the token's position
// (rope_cache.go:85-104): x0' = x0*c - x1*s, x1' = x0*s + x1*c, every product
// rounded; then hi/lo fp16 of x * kAttnQKScale.  Lane j holds float4 slots
// 4j.. of every 32-element chunk, so element e and its partner e + 128 sit in
// the same lane and slot.  tile: this wave's 8 x 40-float LDS tile.
__device__ __forceinline__ void qk_split_group(int64_t g, int j, int r, float* tile, const float* __restrict__ q,
                                               int ldq, const float* __restrict__ k, int ldk,
                                               const float* __restrict__ qw, const float* __restrict__ kw, int H,
                                               int HKV, int T, const int32_t* __restrict__ row_pos,
                                               const float* __restrict__ cos_t, const float* __restrict__ sin_t,
                                               float eps, _Float16* __restrict__ qs_h, _Float16* __restrict__ qs_l,
                                               int ldqs, _Float16* __restrict__ ks_h, _Float16* __restrict__ ks_l,
                                               int ldks) {
  constexpr int NC = 8, HALF = 128;
  const int per = H + HKV;
  if (g >= (int64_t)T * per) return;  // whole 8-lane groups
  const int t = (int)(g / per), hh = (int)(g % per);
  const float* src = hh < H ? q + (int64_t)t * ldq + hh * 256 : k + (int64_t)t * ldk + (hh - H) * 256;
  f32x4_t x[NC];
  // The fp32 Q/K row's last read: non-temporal, leaving L2 to re-read operands.
#pragma unroll
  for (int c = 0; c < NC; c++)
    x[c] = __builtin_nontemporal_load(reinterpret_cast<const f32x4_t*>(src + 32 * c + 4 * j));
  const float* wn = hh < H ? qw : kw;
  if (wn) sg_rmsnorm8_f4<NC>(x, wn, tile, r, j, eps);
  const int pos = row_pos[t];
  const float* cr = cos_t + (int64_t)pos * HALF + 4 * j;
  const float* sr = sin_t + (int64_t)pos * HALF + 4 * j;
#pragma unroll
  for (int c = 0; c < NC / 2; c++) {
    const f32x4_t cv = *reinterpret_cast<const f32x4_t*>(cr + 32 * c);
    const f32x4_t sv = *reinterpret_cast<const f32x4_t*>(sr + 32 * c);
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const float v0 = x[c][u], v1 = x[c + NC / 2][u];
      const float a = v0 * cv[u], b = v1 * sv[u], cc = v0 * sv[u], dd = v1 * cv[u];
      x[c][u] = a - b;
      x[c + NC / 2][u] = cc + dd;
    }
  }
  _Float16 *dh, *dl;
  if (hh < H) {
    dh = qs_h + (int64_t)t * ldqs + hh * 256;
    dl = qs_l + (int64_t)t * ldqs + hh * 256;
  } else {
    dh = ks_h + (int64_t)t * ldks + (hh - H) * 256;
    dl = ks_l + (int64_t)t * ldks + (hh - H) * 256;
  }
#pragma unroll
  for (int c = 0; c < NC; c++) {
    half4_t hv, lv;
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const hl16 sp = split_f16(x[c][u] * sgk::kAttnQKScale);
      hv[u] = sp.hi;
      lv[u] = sp.lo;
    }
    *reinterpret_cast<half4_t*>(dh + 32 * c + 4 * j) = hv;
    *reinterpret_cast<half4_t*>(dl + 32 * c + 4 * j) = lv;
  }
}

// One 32-key tile of V [T][ldv] fp32 (kv head kvh at column 256*kvh) -> V^T
// fp16 [HKV*256][ldvt]: sequence s occupies key columns voff[s] ..
// voff[s] + 32*ceil(S/32), keys in vt_key order inside every 32-key tile,
// zeros past S; the tile at key column c of a dim row is halves 2c .. 2c+31
// (hi) and 2c+32 .. 2c+63 (lo), so ldvt >= 2 * (key columns).  The 32 x 256
// fp32 tile is loaded with coalesced float4 rows into LDS (tv:
// [32][kVtRowStride]); a thread then owns one (dim, 8-key chunk), reads its 8
// keys down the LDS column and stores the chunk's hi and lo halves as two
// 16-byte writes (4 threads cover one dim's 128 contiguous bytes).  Every
// thread of the workgroup must call this (it holds a barrier).
__device__ __forceinline__ void v_split_tile(sg_item t, int kvh, float (*tv)[kVtRowStride], const float* __restrict__ v,
                                             int ldv, const int32_t* __restrict__ seq_off,
                                             const int32_t* __restrict__ voff, _Float16* __restrict__ vt, int ldvt) {
  constexpr int kHD = 256;
  const int r0 = seq_off[t.seq], S = seq_off[t.seq + 1] - r0, k0 = t.c0;
  const int tid = threadIdx.x;
#pragma unroll
  for (int u = 0; u < 8; u++) {  // 32 keys x 64 float4
    const int idx = tid + kKvThreads * u;
    const int key = idx >> 6, d4 = idx & 63;
    f32x4_t x = {0, 0, 0, 0};
    if (k0 + key < S)  // the fp32 V row's last read: non-temporal
      x = __builtin_nontemporal_load(
          reinterpret_cast<const f32x4_t*>(v + (int64_t)(r0 + k0 + key) * ldv + kvh * kHD + 4 * d4));
    *reinterpret_cast<f32x4_t*>(&tv[key][4 * d4]) = x;
  }
  __syncthreads();
  const int64_t col = voff[t.seq] + k0;
#pragma unroll
  for (int u = 0; u < 4; u++) {  // 256 dims x 4 chunks of 8 key positions
    const int dim = (tid >> 2) + 64 * u, c = tid & 3;
    uint32_t hw[4], lw[4];
#pragma unroll
    for (int m = 0; m < 4; m++) {
      uint32_t hb[2], lb[2];
#pragma unroll
      for (int e = 0; e < 2; e++) {
        const int p = 8 * c + 2 * m + e;  // position in the tile row
        const int key = vt_key(p);
        const hl16 sp = split_f16(tv[key][dim]);
        hb[e] = __builtin_bit_cast(uint16_t, sp.hi);
        lb[e] = __builtin_bit_cast(uint16_t, sp.lo);
      }
      hw[m] = hb[0] | (hb[1] << 16);
      lw[m] = lb[0] | (lb[1] << 16);
    }
    const int64_t o = (int64_t)(kvh * kHD + dim) * ldvt + 2 * col + 8 * c;
    *reinterpret_cast<uint4*>(vt + o) = uint4{hw[0], hw[1], hw[2], hw[3]};
    *reinterpret_cast<uint4*>(vt + o + 32) = uint4{lw[0], lw[1], lw[2], lw[3]};
  }
}

}  // namespace sgd
