// k_gemm.hip -- Q8_0 weight x per-sequence-quantized activation GEMM for gfx950.
//
// Semantics (MatMulQ8_0INT8, internal/kernels/quantize.go:346-458):
//   P_b[m,n] = sum_{k in block b} x[m,k] * w[n,k]          (exact integer)
//   acc      = fma(float(P_b), d[n,b], acc)  for b = 0,1,..  (one rounding per block)
//   y[m,n]   = acc * row_scale[m]
//
// Block sums on the fp16 matrix cores: both operands hold int8 values stored
// as fp16 (exact), every product is an integer below 2^14 and every partial
// sum of a 32-wide block is an integer below 2^19, so the fp32 accumulation
// inside v_mfma_f32_32x32x16_f16 is exact in any order: two MFMAs (k 0..15,
// 16..31) started from a zero accumulator produce float(P_b) with no rounding
// at all.  That removes the int32->float conversion from the epilogue, which
// leaves one v_fma_f32 per (m, n, block): with the int8 MFMA the epilogue
// would need a convert and an FMA per element (2 VALU ops per 32 MACs) and
// would cap the matrix cores at a quarter of their int8 rate.
//
// Layout: A [M][K] fp16 row-major (the quantized activations), W [N][K] fp16
// row-major (repacked weight rows), St [K/32][N] fp32 block scales (transposed
// so a wave's 32 columns read one contiguous 128-byte line per block).
#include "sg_device.h"
#include "sg_kernels.h"

namespace {

// WM x WN waves per workgroup, each wave owns TM x TN tiles of 32x32 outputs.
template <int WM, int WN, int TM, int TN, bool SUMS>
__global__ __launch_bounds__(WM* WN* SG_WAVE) void k_gemm_q8(const _Float16* __restrict__ A,
                                                             const _Float16* __restrict__ W,
                                                             const float* __restrict__ St,
                                                             const float* __restrict__ row_scale,
                                                             float* __restrict__ Y, int32_t* __restrict__ sums, int M,
                                                             int N, int K) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int m_base = blockIdx.y * (WM * TM * 32) + wm * TM * 32;
  const int n_base = blockIdx.x * (WN * TN * 32) + wn * TN * 32;
  const int lr = lane & 31, lh = lane >> 5;
  const int nb = K >> 5;

  // Operand fetch: lane (lr, lh) supplies row lr of the 32-row group and the
  // 8 consecutive k at 8*lh (+16 for the second MFMA) of every block.  A and
  // B use the same (lane half, slot) -> k assignment, so each block's dot
  // product is complete whatever k order the matrix core applies.
  const _Float16* ap[TM];
  const _Float16* wp[TN];
  int scol[TN];
#pragma unroll
  for (int tm = 0; tm < TM; tm++) {
    int r = m_base + tm * 32 + lr;
    r = r < M ? r : M - 1;
    ap[tm] = A + (int64_t)r * K + lh * 8;
  }
#pragma unroll
  for (int tn = 0; tn < TN; tn++) {
    int c = n_base + tn * 32 + lr;
    c = c < N ? c : N - 1;
    wp[tn] = W + (int64_t)c * K + lh * 8;
    scol[tn] = c;
  }

  f32x16_t acc[TM][TN];
#pragma unroll
  for (int tm = 0; tm < TM; tm++)
#pragma unroll
    for (int tn = 0; tn < TN; tn++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[tm][tn][r] = 0.0f;

  const f32x16_t zero = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
  for (int b = 0; b < nb; b++) {
    half8_t a0[TM], a1[TM], w0[TN], w1[TN];
    float d[TN];
#pragma unroll
    for (int tm = 0; tm < TM; tm++) {
      a0[tm] = *reinterpret_cast<const half8_t*>(ap[tm] + b * 32);
      a1[tm] = *reinterpret_cast<const half8_t*>(ap[tm] + b * 32 + 16);
    }
#pragma unroll
    for (int tn = 0; tn < TN; tn++) {
      w0[tn] = *reinterpret_cast<const half8_t*>(wp[tn] + b * 32);
      w1[tn] = *reinterpret_cast<const half8_t*>(wp[tn] + b * 32 + 16);
      d[tn] = St[(int64_t)b * N + scol[tn]];
    }
#pragma unroll
    for (int tm = 0; tm < TM; tm++) {
#pragma unroll
      for (int tn = 0; tn < TN; tn++) {
        f32x16_t p = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0[tm], w0[tn], zero, 0, 0, 0);
        p = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1[tm], w1[tn], p, 0, 0, 0);
        if (SUMS) {
          const int col = n_base + tn * 32 + lr;
#pragma unroll
          for (int r = 0; r < 16; r++) {
            const int row = m_base + tm * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
            if (row < M && col < N) sums[((int64_t)row * N + col) * nb + b] = (int32_t)p[r];
          }
        }
#pragma unroll
        for (int r = 0; r < 16; r++) acc[tm][tn][r] = __builtin_fmaf(p[r], d[tn], acc[tm][tn][r]);
      }
    }
  }

  // 32x32 accumulator layout: lane holds column lr; register r holds row
  // 8*(r/4) + 4*lh + r%4 of the tile.
#pragma unroll
  for (int tm = 0; tm < TM; tm++) {
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int row = m_base + tm * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
      if (row >= M) continue;
      const float rs = row_scale[row];
#pragma unroll
      for (int tn = 0; tn < TN; tn++) {
        const int col = n_base + tn * 32 + lr;
        if (col < N) Y[(int64_t)row * N + col] = acc[tm][tn][r] * rs;
      }
    }
  }
}

template <int WM, int WN, int TM, int TN, bool SUMS>
hipError_t launch(const _Float16* A, const _Float16* W, const float* St, const float* rs, float* Y, int32_t* sums,
                  int M, int N, int K, hipStream_t s) {
  constexpr int BM = WM * TM * 32, BN = WN * TN * 32;
  dim3 grid((N + BN - 1) / BN, (M + BM - 1) / BM);
  hipLaunchKernelGGL((k_gemm_q8<WM, WN, TM, TN, SUMS>), grid, dim3(WM * WN * SG_WAVE), 0, s, A, W, St, rs, Y, sums,
                     M, N, K);
  return hipGetLastError();
}

}  // namespace

namespace sgk {

hipError_t gemm_q8(const _Float16* A, const _Float16* W, const float* St, const float* row_scale, float* Y,
                   int32_t* sums, int M, int N, int K, hipStream_t s) {
  if (M <= 0 || N <= 0) return hipSuccess;
  if (K <= 0 || K % 32) return hipErrorInvalidValue;
  if (sums) return launch<1, 1, 1, 1, true>(A, W, St, row_scale, Y, sums, M, N, K, s);
  // Large M: 128x128 workgroup tiles (4 waves of 64x64).  Small problems use
  // 64x64 tiles so that the grid still covers the 256 compute units.
  const int64_t tiles128 = (int64_t)((M + 127) / 128) * ((N + 127) / 128);
  if (tiles128 >= 512) return launch<2, 2, 2, 2, false>(A, W, St, row_scale, Y, nullptr, M, N, K, s);
  return launch<2, 2, 1, 1, false>(A, W, St, row_scale, Y, nullptr, M, N, K, s);
}

}  // namespace sgk
