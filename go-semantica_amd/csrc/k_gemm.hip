// k_gemm.hip -- Q8_0 weight x per-sequence-quantized activation GEMM for gfx950.
//
// Semantics (MatMulQ8_0INT8, internal/kernels/quantize.go:346-458):
//   P_b[m,n] = sum_{k in block b} x[m,k] * w[n,k]          (exact integer)
//   acc      = fma(float(P_b), d[n,b], acc)  for b = 0,1,..  (one rounding per block)
//   y[m,n]   = acc * row_scale[m]
//
// Block sums on the int8 matrix cores: one v_mfma_i32_32x32x32_i8 per 32x32
// subtile and K-block gives P_b exactly (|P_b| <= 32 * 127 * 127).  The
// int32 -> float conversion costs no v_cvt_f32_i32 (a half-rate VALU op on
// gfx950): the MFMA starts from the bit pattern of 1.5 * 2^23 (kMagicBits)
// in every lane, so its result read as a float is exactly 12582912 + P_b
// (|P_b| < 2^22 keeps the exponent at 23 and the mantissa exact) and one
// full-rate subtraction gives float(P_b); read as an integer, minus
// kMagicBits, it is P_b.  Per subtile and block the epilogue is then 16
// subtractions and 16 FMAs (128 VALU cycles) against one 32-cycle MFMA: the
// block-serial rounding, not the matrix core, bounds these kernels.
//
// Operand layout (written by the quantize kernels and the load-time repack):
// block-major int8 [K/32][rows][32], i.e. a K-block of a 32-row group is one
// contiguous 1 KB piece.  Lane l of an MFMA operand reads row l % 32, bytes
// 16*(l / 32) .. +15 of its 32-byte block.  A and W use the same assignment,
// so each block's dot product is complete whatever k order the matrix core
// applies internally.  Block scales are St [K/32][N] fp32 (32 consecutive
// columns = 128 bytes).
#include <type_traits>

#include "sg_device.h"
#include "sg_kernels.h"
#include "sg_kv_prep.h"

typedef int i32x16_t __attribute__((ext_vector_type(16)));
using sgk::sg_vt_out;

namespace {

constexpr float kMagic = 12582912.0f;   // 1.5 * 2^23
constexpr int kMagicBits = 0x4B400000;  // its bit pattern

// The MFMA start value: kMagicBits in every lane.  The asm keeps the constant
// in registers (no per-use rematerialisation).
__device__ __forceinline__ i32x16_t magic_bias() {
  i32x16_t bias;
#pragma unroll
  for (int r = 0; r < 16; r++) bias[r] = kMagicBits;
  asm volatile("" : "+v"(bias));
  return bias;
}

// acc[r] = fma(float(P_b[r]), d, acc[r]) for the 16 block sums of one 32x32
// subtile (pp: the MFMA result from the magic start value): the 16
// subtractions, then 16 v_fmac_f32 (inline assembly, so that the scheduler
// keeps them after all the subtractions).  Each FMA's operand was produced 16
// instructions earlier; the compiler's own schedule runs each subtraction into
// one temporary that the next FMA reads at once, so every pair waits out the
// VALU latency.  The subtractions stay compiled code: the compiler inserts the
// wait states an MFMA result needs before its first VALU read, which it does
// not do for inline assembly.  The arithmetic (x - 12582912, then one fused
// multiply-add) is unchanged.
__device__ __forceinline__ void block_fma16(const i32x16_t& pp, float d, f32x16_t& acc) {
  float p[16], a[16];
#pragma unroll
  for (int r = 0; r < 16; r++) {
    p[r] = __int_as_float(pp[r]) - kMagic;
    a[r] = acc[r];
  }
#pragma unroll
  for (int r = 0; r < 16; r++) asm("v_fmac_f32_e32 %0, %1, %2" : "+v"(a[r]) : "v"(p[r]), "v"(d));
#pragma unroll
  for (int r = 0; r < 16; r++) acc[r] = a[r];
}

// XCD-aware tile order.  Workgroups are handed to the 8 XCDs round-robin by
// linear id, and each XCD has its own L2.  All N-tiles of one M-tile read the
// same A rows, so they are mapped to one XCD: linear id p runs on XCD p % 8;
// that XCD's consecutive slots p / 8 walk its M-tiles (xcd, xcd+8, ...) with
// every N-tile of each.  A is then fetched from HBM about once instead of
// once per N-tile, and W (at most a few MB) stays resident in every L2.
__device__ __forceinline__ void xcd_tile(int& bx, int& by) {
  const int gx = gridDim.x, gy = gridDim.y;
  if ((gy & 7) == 0) {
    const int p = blockIdx.x + blockIdx.y * gx;
    const int xcd = p & 7, slot = p >> 3;
    by = (slot / gx) * 8 + xcd;
    bx = slot % gx;
  } else {
    bx = blockIdx.x;
    by = blockIdx.y;
  }
}

// Epilogue shared by the GEMM kernels: Y = acc * row_scale (or, with
// GELU, g = geluquick(gate) * up over the paired subtiles, with the
// sequences' max|g| folded into amax).  Wave tile rows mw.., workgroup row
// tile by, columns n0...
// stage (optional): this wave's own 32 x 32 float slice of LDS.  Each output
// subtile then goes out as row-contiguous float4 stores (lane l: row
// l / 8 + 8 i, columns 4 (l % 8) .. + 3; 4 instructions per subtile) after
// a transpose through the slice, instead of 16 single-float stores in the
// MFMA's column-per-lane layout.
// ROWMAX: also fold each of the lane's four rows' max|value| over the
// subtile's valid columns into rm[i] (row row0 + l / 8 + 8 i), complete in
// every lane of the row's 8-lane group.
template <bool ROWMAX = false>
__device__ __forceinline__ void store_subtile(float* stage, const float (&v)[16], float* __restrict__ Y, int ld,
                                              int row0, int col0, int rows, int cols, int lr, int lh, int lane,
                                              float* rm = nullptr) {
#pragma unroll
  for (int r = 0; r < 16; r++) stage[(8 * (r >> 2) + 4 * lh + (r & 3)) * 32 + lr] = v[r];
  const int c4 = (lane & 7) * 4;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int rl = (lane >> 3) + 8 * i;
    const f32x4_t o = *reinterpret_cast<const f32x4_t*>(stage + rl * 32 + c4);
    const int row = row0 + rl, col = col0 + c4;
    if (row < rows) {
      if (col + 3 < cols) {
        *reinterpret_cast<f32x4_t*>(Y + (int64_t)row * ld + col) = o;
      } else {
#pragma unroll
        for (int t = 0; t < 4; t++)
          if (col + t < cols) Y[(int64_t)row * ld + col + t] = o[t];
      }
    }
    if constexpr (ROWMAX) {
      float m = 0.0f;
#pragma unroll
      for (int t = 0; t < 4; t++) m = (row < rows && col + t < cols) ? fmaxf(m, fabsf(o[t])) : m;
#pragma unroll
      for (int x = 1; x < 8; x <<= 1) m = fmaxf(m, __shfl_xor(m, x));
      rm[i] = fmaxf(rm[i], m);
    }
  }
}

// One 32 x 32 subtile of V (tokens row0 .., dims dim0 ..) into V^T, through
// the wave's LDS slice.  A subtile whose 32 tokens are one whole 32-key tile
// of a sequence (the usual case for sequences that start on a 32-row
// boundary) goes out as 16-byte hi and lo chunks: lane l covers dim l % 32,
// positions 8c .. 8c + 7 (c = 2 (l / 32), + 1), each position p holding key
// vt_key(p), 128 contiguous bytes per dim.  Any other subtile is written value
// by value at its key's tile and position.
__device__ __forceinline__ void store_vt_subtile(float* stage, const float (&v)[16], const sg_vt_out& vo, int row0,
                                                 int dim0, int rows, int lr, int lh, int lane) {
#pragma unroll
  for (int r = 0; r < 16; r++) stage[(8 * (r >> 2) + 4 * lh + (r & 3)) * 32 + lr] = v[r];
  const int dim = lane & 31;
  const int s0 = vo.row_seq[min(row0, rows - 1)];
  const int key0 = row0 - vo.seq_off[s0];
  const bool whole = (key0 & 31) == 0 && row0 + 31 < rows && vo.row_seq[row0 + 31] == s0;  // wave-uniform
  if (whole) {
    _Float16* base = vo.vt + ((dim0 + dim) * vo.ldvt + 2 * (vo.voff[s0] + key0));  // < 2^31 (checked at launch)
#pragma unroll 1
    for (int cc = 0; cc < 2; cc++) {
      const int c = 2 * (lane >> 5) + cc;
      uint32_t hw[4], lw[4];
#pragma unroll
      for (int m = 0; m < 4; m++) {
        uint32_t hb[2], lb[2];
#pragma unroll
        for (int e = 0; e < 2; e++) {
          const hl16 sp = split_f16(stage[sgd::vt_key(8 * c + 2 * m + e) * 32 + dim]);
          hb[e] = __builtin_bit_cast(uint16_t, sp.hi);
          lb[e] = __builtin_bit_cast(uint16_t, sp.lo);
        }
        hw[m] = hb[0] | (hb[1] << 16);
        lw[m] = lb[0] | (lb[1] << 16);
      }
      *reinterpret_cast<uint4*>(base + 8 * c) = uint4{hw[0], hw[1], hw[2], hw[3]};
      *reinterpret_cast<uint4*>(base + 32 + 8 * c) = uint4{lw[0], lw[1], lw[2], lw[3]};
    }
  } else {
#pragma unroll 1
    for (int i = 0; i < 16; i++) {
      const int rl = 2 * i + (lane >> 5), t = row0 + rl;
      if (t < rows) {
        const int sq = vo.row_seq[t], key = t - vo.seq_off[sq];
        const int p = 8 * ((key & 15) >> 2) + 4 * ((key >> 4) & 1) + (key & 3);  // vt_key(p) == key & 31
        _Float16* base = vo.vt + ((dim0 + dim) * vo.ldvt + 2 * (vo.voff[sq] + (key & ~31)));
        const hl16 sp = split_f16(stage[rl * 32 + dim]);
        base[p] = sp.hi;
        base[32 + p] = sp.lo;
      }
    }
  }
}

template <int NW, int TM, int TN, bool GELU>
__device__ __forceinline__ void gemm_epilogue(const f32x16_t (&acc)[TM][TN], int mw, int by, int n0, int lr, int lh,
                                              int lane, int wave, int tid, int M, int N,
                                              const float* __restrict__ row_scale, float* __restrict__ Y,
                                              const int32_t* __restrict__ row_seq, float* __restrict__ amax,
                                              float* stage = nullptr,
                                              sg_vt_out vto = sg_vt_out{nullptr, 0, 0, nullptr, nullptr, nullptr}) {
  constexpr int BMW = TM * 32;
  if constexpr (GELU) {
    // Subtile pairs (2p, 2p+1) are gate and up of output columns
    // (n0 / 2) + 32p + lr.
    static_assert(TN % 2 == 0, "GELU pairs gate and up subtiles");
    __shared__ float red[NW];
    __shared__ float rmax[NW * BMW];
    const int Nh = N >> 1;
    const int r_first = by * NW * BMW, r_last = min(r_first + NW * BMW, M) - 1;
    const bool one_seq = amax && row_seq[r_first] == row_seq[r_last];  // workgroup-uniform
    float mx = 0.0f;
    // Rows of several sequences: per-row maxima into rmax.  With the staged
    // stores they come from the row-contiguous read-back (three lane
    // exchanges per row slot) instead of five per MFMA row.
    const bool staged_rmax = stage && amax && !one_seq;  // workgroup-uniform
#pragma unroll
    for (int tm = 0; tm < TM; tm++) {
      const int mb = mw + tm * 32;
      float gv[TN / 2][16];
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int row = mb + 8 * (r >> 2) + 4 * lh + (r & 3);
        const float rsr = row_scale[row < M ? row : M - 1];
        float a = 0.0f;
#pragma unroll
        for (int pr = 0; pr < TN / 2; pr++) {
          const int col = (n0 >> 1) + 32 * pr + lr;
          const float gate = acc[tm][2 * pr][r] * rsr, up = acc[tm][2 * pr + 1][r] * rsr;
          const float g = sg_gelu_quick(gate) * up;
          const bool ok = row < M && col < Nh;
          if (stage)
            gv[pr][r] = g;
          else if (ok)
            Y[(int64_t)row * Nh + col] = g;
          a = ok ? fmaxf(a, fabsf(g)) : a;
        }
        if (one_seq) {
          mx = fmaxf(mx, a);
        } else if (amax && !staged_rmax) {  // rows of several sequences: per-row maxima, folded below
#pragma unroll
          for (int o = 1; o < 32; o <<= 1) a = fmaxf(a, __shfl_xor(a, o));
          if (lr == 0) rmax[row - r_first] = a;
        }
      }
      if (staged_rmax) {
        float rm[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int pr = 0; pr < TN / 2; pr++)
          store_subtile<true>(stage, gv[pr], Y, Nh, mb, (n0 >> 1) + 32 * pr, M, Nh, lr, lh, lane, rm);
        if ((lane & 7) == 0) {
#pragma unroll
          for (int i = 0; i < 4; i++) {
            const int row = mb + (lane >> 3) + 8 * i;
            if (row <= r_last) rmax[row - r_first] = rm[i];
          }
        }
      } else if (stage) {
#pragma unroll
        for (int pr = 0; pr < TN / 2; pr++) store_subtile(stage, gv[pr], Y, Nh, mb, (n0 >> 1) + 32 * pr, M, Nh, lr, lh, lane);
      }
    }
    if (one_seq) {
      mx = sg_wave_max(mx);
      if (lane == 0) red[wave] = mx;
      __syncthreads();
      if (tid == 0) {
        float mm = red[0];
#pragma unroll
        for (int i = 1; i < NW; i++) mm = fmaxf(mm, red[i]);
        sg_atomic_max_nonneg(amax + row_seq[r_first], mm);
      }
    } else if (amax) {  // workgroup-uniform
      __syncthreads();
      sg_seg_seq_max(rmax, r_last - r_first + 1, r_first, row_seq, amax);
    }
  } else {
#pragma unroll
    for (int tm = 0; tm < TM; tm++) {
      const int mb = mw + tm * 32;
      float rs[16];
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int row = mb + 8 * (r >> 2) + 4 * lh + (r & 3);
        rs[r] = row_scale[row < M ? row : M - 1];
      }
      if (stage) {
        // Scaled values first, so the row scales die before the stores.
        float v[TN][16];
#pragma unroll
        for (int tn = 0; tn < TN; tn++)
#pragma unroll
          for (int r = 0; r < 16; r++) v[tn][r] = acc[tm][tn][r] * rs[r];
        if (vto.vt && n0 >= vto.col0) {  // workgroup-uniform: the tile is V columns only
#pragma unroll
          for (int tn = 0; tn < TN; tn++)
            store_vt_subtile(stage, v[tn], vto, mb, n0 + tn * 32 - vto.col0, M, lr, lh, lane);
        } else {
#pragma unroll
          for (int tn = 0; tn < TN; tn++) store_subtile(stage, v[tn], Y, N, mb, n0 + tn * 32, M, N, lr, lh, lane);
        }
        continue;
      }
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int row = mb + 8 * (r >> 2) + 4 * lh + (r & 3);
#pragma unroll
        for (int tn = 0; tn < TN; tn++) {
          const int col = n0 + tn * 32 + lr;
          if (row < M && col < N) Y[(int64_t)row * N + col] = acc[tm][tn][r] * rs[r];
        }
      }
    }
  }
}

// Register-direct kernel: every wave loads its own A and W fragments straight
// from global memory (16 bytes per lane and operand per K-block, L1/L2
// cached) into a ring of PF register stages -- blocks b+1 .. b+PF-1 are in
// flight while block b computes -- with no LDS and no barrier in the K loop.
// The prefetches are unconditional (past the last block they re-load block
// nb-1, never computed): a load under a branch makes the compiler's wait
// counting merge the two paths and wait for every load in flight, the
// prefetch included.  The occupancy bound (two workgroups per CU) caps the
// kernel at 256 VGPRs, which keeps the MFMA results in VGPRs; without it they
// land in AGPRs and every one is copied back by a v_accvgpr_read before its
// subtraction.  WM x WN waves per workgroup, each owning TM x TN subtiles of
// 32x32 outputs.  A has a_rows rows per K-block (>= the padded M the grid
// covers).  SUMS additionally dumps the exact block sums int32 [M][N][K/32].
// GELU (WN = 1, TN even): W holds gate and up rows interleaved in groups of
// 32 (kGeluGroup), subtile pairs (2p, 2p+1) of a wave are gate and up of the
// same features, and gemm_epilogue writes g [M][N/2] with the sequences'
// max|g| in amax.  PIPE (PF >= 3) issues each block's MFMAs one step ahead of
// its FMA chain, for grids too small to cover a wave's MFMA latency with
// other waves.
template <int TM, int TN>
struct Stage {
  i32x4_t a[TM], w[TN];
  float d[TN];
};

template <int TM, int TN>
__device__ __forceinline__ void fetch(Stage<TM, TN>& st, const int8_t* const (&ap)[TM],
                                      const int8_t* const (&wp)[TN], const float* const (&sp)[TN], int b,
                                      int64_t a_bstride, int64_t w_bstride, int N) {
#pragma unroll
  for (int tm = 0; tm < TM; tm++) st.a[tm] = *reinterpret_cast<const i32x4_t*>(ap[tm] + b * a_bstride);
#pragma unroll
  for (int tn = 0; tn < TN; tn++) {
    st.w[tn] = *reinterpret_cast<const i32x4_t*>(wp[tn] + b * w_bstride);
    st.d[tn] = sp[tn][(int64_t)b * N];
  }
}

template <int TM, int TN>
__device__ __forceinline__ void block_mfma(const Stage<TM, TN>& st, i32x16_t (&p)[TM][TN], const i32x16_t& bias) {
#pragma unroll
  for (int tm = 0; tm < TM; tm++)
#pragma unroll
    for (int tn = 0; tn < TN; tn++) p[tm][tn] = __builtin_amdgcn_mfma_i32_32x32x32_i8(st.a[tm], st.w[tn], bias, 0, 0, 0);
}

template <int TM, int TN, bool SUMS>
__device__ __forceinline__ void block_fma(const i32x16_t (&p)[TM][TN], const float (&d)[TN], f32x16_t (&acc)[TM][TN],
                                          int32_t* sums, int M, int N, int nb, int b, int m_base, int n_base, int lr,
                                          int lh) {
#pragma unroll
  for (int tm = 0; tm < TM; tm++)
#pragma unroll
    for (int tn = 0; tn < TN; tn++) {
      if (SUMS) {
        const int col = n_base + tn * 32 + lr;
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const int row = m_base + tm * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
          if (row < M && col < N) sums[((int64_t)row * N + col) * nb + b] = p[tm][tn][r] - kMagicBits;
        }
      }
      block_fma16(p[tm][tn], d[tn], acc[tm][tn]);
    }
}

template <int TM, int TN, bool SUMS>
__device__ __forceinline__ void compute(const Stage<TM, TN>& st, f32x16_t (&acc)[TM][TN], int32_t* sums, int M,
                                        int N, int nb, int b, int m_base, int n_base, int lr, int lh,
                                        const i32x16_t& bias) {
  i32x16_t p[TM][TN];
  block_mfma<TM, TN>(st, p, bias);
  block_fma<TM, TN, SUMS>(p, st.d, acc, sums, M, N, nb, b, m_base, n_base, lr, lh);
}

template <int WM, int WN, int TM, int TN, bool SUMS, bool GELU, int PF, bool PIPE>
__global__ __launch_bounds__(WM* WN* SG_WAVE, 2) void k_gemm_q8_rd(
    const int8_t* __restrict__ A, int a_rows, const int8_t* __restrict__ W, const float* __restrict__ St,
    const float* __restrict__ row_scale, float* __restrict__ Y, int32_t* __restrict__ sums, int M, int N, int K,
    const int32_t* __restrict__ row_seq, float* __restrict__ amax) {
  static_assert(!GELU || (WN == 1 && TN % 2 == 0 && !SUMS), "GELU pairs gate and up subtiles of one wave");
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / WN, wn = wave % WN;
  int bx, by;
  xcd_tile(bx, by);
  const int m_base = by * (WM * TM * 32) + wm * TM * 32;
  const int n_base = bx * (WN * TN * 32) + wn * TN * 32;
  const int lr = lane & 31, lh = lane >> 5;
  const int nb = K >> 5;
  const int64_t a_bstride = (int64_t)a_rows * 32, w_bstride = (int64_t)N * 32;

  const int8_t* ap[TM];
  const int8_t* wp[TN];
  const float* sp[TN];
#pragma unroll
  for (int tm = 0; tm < TM; tm++) ap[tm] = A + (int64_t)(m_base + tm * 32 + lr) * 32 + 16 * lh;
#pragma unroll
  for (int tn = 0; tn < TN; tn++) {
    int c = n_base + tn * 32 + lr;
    c = c < N ? c : N - 1;
    wp[tn] = W + (int64_t)c * 32 + 16 * lh;
    sp[tn] = St + c;
  }

  f32x16_t acc[TM][TN];
#pragma unroll
  for (int tm = 0; tm < TM; tm++)
#pragma unroll
    for (int tn = 0; tn < TN; tn++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[tm][tn][r] = 0.0f;
  const i32x16_t bias = magic_bias();

  // Ring of PF register stages: block b is in stage b % PF.  The prologue
  // fetches blocks 0 .. PF-2; each step fetches block b + PF - 1 into the
  // stage block b - 1 left, then computes block b.  The scheduling barrier
  // keeps every prefetch ahead of the compute that follows it (the scheduler
  // would otherwise sink the loads to their use and fold the stages into one
  // register set).
  Stage<TM, TN> st[PF];
  static_for<0, PF - 1>([&](auto ic) {
    constexpr int I = decltype(ic)::value;
    fetch<TM, TN>(st[I], ap, wp, sp, min(I, nb - 1), a_bstride, w_bstride, N);
  });
  int b = 0;
  if constexpr (PIPE) {
    // MFMA one block ahead: step b issues block b+1's MFMAs (its stage was
    // fetched PF - 2 >= 1 steps earlier) before block b's FMA chain, so a
    // wave's FMAs wait on no MFMA latency.  Past the last block the MFMAs
    // run on re-loaded or stale stages and their results are never used.
    static_assert(PF >= 3 && !SUMS, "the pipelined loop keeps a fetched stage between fetch and MFMA");
    i32x16_t p[TM][TN];
    block_mfma<TM, TN>(st[0], p, bias);
    for (; b + PF <= nb; b += PF)
      static_for<0, PF>([&](auto ic) {
        constexpr int I = decltype(ic)::value;
        fetch<TM, TN>(st[(I + PF - 1) % PF], ap, wp, sp, min(b + I + PF - 1, nb - 1), a_bstride, w_bstride, N);
        __builtin_amdgcn_sched_barrier(0);
        i32x16_t pn[TM][TN];
        block_mfma<TM, TN>(st[(I + 1) % PF], pn, bias);
        __builtin_amdgcn_sched_barrier(0);
        block_fma<TM, TN, false>(p, st[I].d, acc, nullptr, M, N, nb, b + I, m_base, n_base, lr, lh);
        static_for<0, TM>([&](auto mc) {
          static_for<0, TN>([&](auto nc) { p[decltype(mc)::value][decltype(nc)::value] = pn[decltype(mc)::value][decltype(nc)::value]; });
        });
      });
    static_for<0, PF - 1>([&](auto ic) {  // the last nb % PF blocks, already in stages 0 ..
      constexpr int I = decltype(ic)::value;
      if (b + I < nb) {
        i32x16_t pn[TM][TN];
        block_mfma<TM, TN>(st[(I + 1) % PF], pn, bias);
        __builtin_amdgcn_sched_barrier(0);
        block_fma<TM, TN, false>(p, st[I].d, acc, nullptr, M, N, nb, b + I, m_base, n_base, lr, lh);
        static_for<0, TM>([&](auto mc) {
          static_for<0, TN>([&](auto nc) { p[decltype(mc)::value][decltype(nc)::value] = pn[decltype(mc)::value][decltype(nc)::value]; });
        });
      }
    });
  } else {
    for (; b + PF <= nb; b += PF)
      static_for<0, PF>([&](auto ic) {
        constexpr int I = decltype(ic)::value;
        fetch<TM, TN>(st[(I + PF - 1) % PF], ap, wp, sp, min(b + I + PF - 1, nb - 1), a_bstride, w_bstride, N);
        __builtin_amdgcn_sched_barrier(0);
        compute<TM, TN, SUMS>(st[I], acc, sums, M, N, nb, b + I, m_base, n_base, lr, lh, bias);
      });
    static_for<0, PF - 1>([&](auto ic) {  // the last nb % PF blocks, already in stages 0 ..
      constexpr int I = decltype(ic)::value;
      if (b + I < nb) compute<TM, TN, SUMS>(st[I], acc, sums, M, N, nb, b + I, m_base, n_base, lr, lh, bias);
    });
  }

  gemm_epilogue<WM, TM, TN, GELU>(acc, m_base, by, n_base, lr, lh, lane, wave, threadIdx.x, M, N, row_scale, Y,
                                  row_seq, amax);
}

// Tiny-M kernel (a few 16-row groups: the serving batches of one or a few
// short texts).  The register-direct tiles above give a wave 32 rows x 32
// columns, so at M = 32 half of a 64-row tile's waves (three quarters of the
// GELU kernel's 128-row tile) compute padding rows, and each wave's 24 blocks
// x 32 outputs per lane of subtractions and FMAs form a long VALU stream on a
// SIMD with nothing else to run.  Here a wave owns 16 rows x 16 columns
// (v_mfma_i32_16x16x32_i8: 4 outputs per lane, 8 VALU instructions per
// block), a workgroup 4 waves side by side along N (16 rows x 64 columns), so
// the same work is spread over four times the waves.  Operand fragments:
// lane l holds row (or weight column) l % 16, bytes 8 (l / 16) .. + 7 of the
// 32-byte block, the same assignment for A and W; the result's lane l holds
// rows 4 (l / 16) .. + 3 of column l % 16.  The K loop is the register-direct
// kernel's MFMA-ahead ring (PF stages, unconditional prefetches).  GELU: the
// wave's gate and up tiles of the same 16 output columns (W rows paired in
// groups of kGeluGroup), g = geluquick(gate) * up, the sequences' max|g| into
// amax.
typedef int i32x4_mf __attribute__((ext_vector_type(4)));
template <int T>
struct TinyStage {
  long a, w[T];
  float d[T];
};

template <bool GELU, int PF>
__global__ __launch_bounds__(256, 2) void k_gemm_q8_tiny(const int8_t* __restrict__ A, int a_rows,
                                                         const int8_t* __restrict__ W, const float* __restrict__ St,
                                                         const float* __restrict__ row_scale, float* __restrict__ Y,
                                                         int M, int N, int K, const int32_t* __restrict__ row_seq,
                                                         float* __restrict__ amax) {
  constexpr int T = GELU ? 2 : 1;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int lr = lane & 15, lg = lane >> 4;
  const int m0 = blockIdx.y * 16;
  const int nout = GELU ? N / 2 : N;
  const int c0 = (blockIdx.x * 4 + wave) * 16;  // this wave's 16 output columns
  const bool active = c0 < nout;                // wave-uniform
  const int nb = K >> 5;
  const int64_t a_bstride = (int64_t)a_rows * 32, w_bstride = (int64_t)N * 32;
  const int8_t* ap = A + (int64_t)(m0 + lr) * 32 + 8 * lg;
  const int8_t* wp[T];
  const float* sp[T];
#pragma unroll
  for (int t = 0; t < T; t++) {
    int wr = GELU ? (c0 / sgk::kGeluGroup) * 2 * sgk::kGeluGroup + c0 % sgk::kGeluGroup + t * sgk::kGeluGroup + lr : c0 + lr;
    wr = wr < N ? wr : N - 1;
    wp[t] = W + (int64_t)wr * 32 + 8 * lg;
    sp[t] = St + wr;
  }
  auto fetch = [&](TinyStage<T>& st, int b) {
    st.a = *reinterpret_cast<const long*>(ap + b * a_bstride);
#pragma unroll
    for (int t = 0; t < T; t++) {
      st.w[t] = *reinterpret_cast<const long*>(wp[t] + b * w_bstride);
      st.d[t] = sp[t][(int64_t)b * N];
    }
  };
  i32x4_mf bias = {kMagicBits, kMagicBits, kMagicBits, kMagicBits};
  asm volatile("" : "+v"(bias));
  auto mfma = [&](const TinyStage<T>& st, i32x4_mf (&p)[T]) {
#pragma unroll
    for (int t = 0; t < T; t++) p[t] = __builtin_amdgcn_mfma_i32_16x16x32_i8(st.a, st.w[t], bias, 0, 0, 0);
  };
  float acc[T][4];
#pragma unroll
  for (int t = 0; t < T; t++)
#pragma unroll
    for (int r = 0; r < 4; r++) acc[t][r] = 0.0f;
  auto fma_block = [&](const i32x4_mf (&p)[T], const float (&d)[T]) {
    // Every subtraction, then every FMA (as block_fma16: no FMA waits on the
    // instruction just before it).
    float q[T][4];
#pragma unroll
    for (int t = 0; t < T; t++)
#pragma unroll
      for (int r = 0; r < 4; r++) q[t][r] = __int_as_float(p[t][r]) - kMagic;
#pragma unroll
    for (int t = 0; t < T; t++)
#pragma unroll
      for (int r = 0; r < 4; r++) asm("v_fmac_f32_e32 %0, %1, %2" : "+v"(acc[t][r]) : "v"(q[t][r]), "v"(d[t]));
  };

  if (active) {
    TinyStage<T> st[PF];
    static_for<0, PF - 1>([&](auto ic) {
      constexpr int I = decltype(ic)::value;
      fetch(st[I], min(I, nb - 1));
    });
    i32x4_mf p[T];
    mfma(st[0], p);
    int b = 0;
    for (; b + PF <= nb; b += PF)
      static_for<0, PF>([&](auto ic) {
        constexpr int I = decltype(ic)::value;
        fetch(st[(I + PF - 1) % PF], min(b + I + PF - 1, nb - 1));
        __builtin_amdgcn_sched_barrier(0);
        i32x4_mf pn[T];
        mfma(st[(I + 1) % PF], pn);
        __builtin_amdgcn_sched_barrier(0);
        fma_block(p, st[I].d);
#pragma unroll
        for (int t = 0; t < T; t++) p[t] = pn[t];
      });
    static_for<0, PF - 1>([&](auto ic) {  // the last nb % PF blocks, already in stages 0 ..
      constexpr int I = decltype(ic)::value;
      if (b + I < nb) {
        i32x4_mf pn[T];
        mfma(st[(I + 1) % PF], pn);
        __builtin_amdgcn_sched_barrier(0);
        fma_block(p, st[I].d);
#pragma unroll
        for (int t = 0; t < T; t++) p[t] = pn[t];
      }
    });
  }

  const int col = c0 + lr;
  // GELU: each row's max|g| over the wave's columns, then over the four
  // waves (LDS), then a segmented max over the workgroup's 16 rows (packed
  // sequence by sequence): one atomic per sequence and workgroup.
  __shared__ float rmax[GELU ? 4 : 1][16];
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const int row = m0 + 4 * lg + r;
    const float rs = row_scale[row < M ? row : M - 1];
    if constexpr (GELU) {
      const float gate = acc[0][r] * rs, up = acc[1][r] * rs;
      const float g = sg_gelu_quick(gate) * up;
      const bool ok = active && row < M && col < nout;
      if (ok) Y[(int64_t)row * nout + col] = g;
      float a = ok ? fabsf(g) : 0.0f;
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) a = fmaxf(a, __shfl_xor(a, o));
      if (lr == 0) rmax[wave][4 * lg + r] = a;
    } else {
      if (active && row < M && col < N) Y[(int64_t)row * N + col] = acc[0][r] * rs;
    }
  }
  if constexpr (GELU) {
    if (!amax) return;  // grid-uniform
    __syncthreads();
    if (threadIdx.x < 16) {
      const int row = m0 + threadIdx.x;
      float v = fmaxf(fmaxf(rmax[0][threadIdx.x], rmax[1][threadIdx.x]), fmaxf(rmax[2][threadIdx.x], rmax[3][threadIdx.x]));
      const int sq = row < M ? row_seq[row] : -1;
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) {
        const float vu = __shfl_up(v, o);
        const int su = __shfl_up(sq, o);
        if ((int)threadIdx.x >= o && su == sq) v = fmaxf(v, vu);
      }
      const int sn = __shfl_down(sq, 1);
      if (row < M && (threadIdx.x == 15 || sn != sq)) sg_atomic_max_nonneg(amax + sq, v);
    }
  }
}

template <bool GELU, int PF>
hipError_t launch_tiny(const int8_t* A, int a_rows, const int8_t* W, const float* St, const float* rs, float* Y,
                       int M, int N, int K, hipStream_t s, const int32_t* row_seq = nullptr, float* amax = nullptr) {
  const int gm = (M + 15) / 16;
  if ((int64_t)gm * 16 > a_rows) return hipErrorInvalidValue;  // A must cover the padded rows
  const int nout = GELU ? N / 2 : N;
  dim3 grid((nout + 63) / 64, gm);
  hipLaunchKernelGGL((k_gemm_q8_tiny<GELU, PF>), grid, dim3(256), 0, s, A, a_rows, W, St, rs, Y, M, N, K, row_seq,
                     amax);
  return hipGetLastError();
}

template <int WM, int WN, int TM, int TN, bool SUMS, bool GELU = false, int PF = 2, bool PIPE = false>
hipError_t launch_rd(const int8_t* A, int a_rows, const int8_t* W, const float* St, const float* rs, float* Y,
                     int32_t* sums, int M, int N, int K, hipStream_t s, const int32_t* row_seq = nullptr,
                     float* amax = nullptr) {
  constexpr int BM = WM * TM * 32, BN = WN * TN * 32;
  const int gm = (M + BM - 1) / BM;
  if ((int64_t)gm * BM > a_rows) return hipErrorInvalidValue;  // A must cover the padded rows
  dim3 grid((N + BN - 1) / BN, gm);
  hipLaunchKernelGGL((k_gemm_q8_rd<WM, WN, TM, TN, SUMS, GELU, PF, PIPE>), grid, dim3(WM * WN * SG_WAVE), 0, s, A, a_rows, W,
                     St, rs, Y, sums, M, N, K, row_seq, amax);
  return hipGetLastError();
}

constexpr int kBufWord3 = 0x00020000;  // raw buffer descriptor, gfx9 family
// f(integral_constant<int, I>) for I = I0 .. N-1, unrolled at compile time.
template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

// Direct-to-LDS kernel.  Workgroup: NW waves x 32 rows, 32*TN columns.
// Every K-block's A tile (each wave's own 32 rows), weight tile and scales are
// copied global -> LDS by buffer_load_dwordx4/dword ... lds (no staging
// registers) into a ring of STAGES buffers, STAGES-1 blocks ahead.  Each wave
// issues the same number of copies per block, CPB (clamped, redundant past
// the last block), so one constant s_waitcnt vmcnt covers "this wave's copies
// of block b have landed"; a bare s_barrier then publishes every wave's
// copies.  (__syncthreads' fence would wait for all copies in flight.)  Large
// M uses 8 waves, 4 subtiles, 3 stages (two workgroups per CU); mid-size M
// uses 4 waves with a deep ring, as its K loop is bound by copy latency.
//
// A copy costs no vector instruction: each K-block's buffer descriptors (base
// = this tile's part of the block slice) are built on the scalar unit and the
// per-lane byte offsets are loop-invariant.  The K loop is unrolled by the
// ring depth, so every LDS fragment read is a loop-invariant vector address
// plus an immediate; the LDS is laid out [A stages][W stages][scale stages]
// to keep those immediates under 64 KB.  LDS per stage: A [2 halves][BM
// rows][16 B], W [2][BN][16 B], scales [BN]; lane l of an MFMA operand reads
// row l % 32, bytes 16*(l / 32) .. +15 of its 32-byte block, so each fragment
// read is 1 KB of contiguous LDS.  Copies: NW / 2 waves per half, each
// copying 64 A rows (one 1-KB copy) and, with 32 lanes, 32 W rows
// (BN = 16 * NW).
template <int NW, int TN, bool GELU, int STAGES>
__global__ __launch_bounds__(NW * SG_WAVE, NW == 8 ? 4 : 1) void k_gemm_q8_lds(
    const int8_t* __restrict__ A, int a_rows, const int8_t* __restrict__ W, const float* __restrict__ St,
    const float* __restrict__ row_scale, float* __restrict__ Y, int M, int N, int K,
    const int32_t* __restrict__ row_seq, float* __restrict__ amax, sg_vt_out vto) {
  constexpr int NWH = NW / 2;
  constexpr int BM = NW * 32, BN = TN * 32;
  static_assert(NW % 2 == 0 && TN == NWH, "copy split: 64 A rows and 32 W rows per wave and half");
  constexpr int A_BYTES = BM * 32, W_BYTES = BN * 32, S_BYTES = BN * 4;
  constexpr int W_OFF = STAGES * A_BYTES, S_OFF = W_OFF + STAGES * W_BYTES;
  constexpr int SLANES = BN / NW;  // scales each wave copies
  constexpr int CPB = 3;           // copies per wave per K-block
  static_assert(STAGES >= 3 && (STAGES - 2) * CPB <= 63, "vmcnt covers the copies in flight");
  static_assert(STAGES * A_BYTES < 65536 && STAGES * W_BYTES < 65536 && STAGES * S_BYTES < 65536,
                "stage offsets fit the LDS immediate");
  __shared__ __attribute__((aligned(16))) unsigned char lds[S_OFF + STAGES * S_BYTES];
  typedef __attribute__((address_space(3))) void* lds_ptr;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 31, lh = lane >> 5;
  int bx, by;
  xcd_tile(bx, by);
  const int n0 = bx * BN;
  const int mw = by * BM + wave * 32;
  const int nb = K >> 5;
  const int ch = wave / NWH, cr = wave % NWH;  // this wave's copy half and row group
  const uint32_t aoff = (uint32_t)(64 * cr + lane) * 32u + 16u * ch;
  const uint32_t woff = (uint32_t)(min(n0 + 32 * cr + lr, N - 1) - n0) * 32u + 16u * ch;
  const uint32_t soff = (uint32_t)(min(n0 + SLANES * wave + lane, N - 1) - n0) * 4u;
  auto issue = [&](int b, int st) {
    __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(A + ((int64_t)b * a_rows + (int64_t)by * BM) * 32), 0, A_BYTES, kBufWord3);
    __amdgpu_buffer_rsrc_t rw =
        __builtin_amdgcn_make_buffer_rsrc((void*)(W + ((int64_t)b * N + n0) * 32), 0, W_BYTES, kBufWord3);
    __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void*)(St + (int64_t)b * N + n0), 0, S_BYTES, kBufWord3);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_ptr)(lds + st * A_BYTES + ch * (BM * 16) + 64 * cr * 16), 16,
                                             aoff, 0, 0, 0);
    if (lane < 32)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rw, (lds_ptr)(lds + W_OFF + st * W_BYTES + ch * (BN * 16) + 32 * cr * 16), 16, woff, 0, 0, 0);
    if (lane < SLANES)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr)(lds + S_OFF + st * S_BYTES + wave * (SLANES * 4)), 4,
                                               soff, 0, 0, 0);
  };
  // Fragment read addresses (stage 0; stage st adds st * *_BYTES).
  const uint32_t ra_f = lh * (BM * 16) + (wave * 32 + lr) * 16;
  const uint32_t rw_f = W_OFF + lh * (BN * 16) + lr * 16;
  const uint32_t rd = S_OFF + 4 * lr;

  f32x16_t acc[1][TN];
#pragma unroll
  for (int tn = 0; tn < TN; tn++)
#pragma unroll
    for (int r = 0; r < 16; r++) acc[0][tn][r] = 0.0f;
  const i32x16_t bias = magic_bias();
  auto step = [&](auto stc, int b) {
    constexpr int ST = decltype(stc)::value;
    sg_wait_vmcnt<(STAGES - 2) * CPB>();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    issue(min(b + STAGES - 1, nb - 1), (ST + STAGES - 1) % STAGES);
    const i32x4_t fa = *reinterpret_cast<const i32x4_t*>(lds + ra_f + ST * A_BYTES);
#pragma unroll
    for (int tn = 0; tn < TN; tn++) {
      const i32x4_t fw = *reinterpret_cast<const i32x4_t*>(lds + rw_f + ST * W_BYTES + tn * 512);
      const float d = *reinterpret_cast<const float*>(lds + rd + ST * S_BYTES + tn * 128);
      const i32x16_t pp = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa, fw, bias, 0, 0, 0);
      block_fma16(pp, d, acc[0][tn]);
    }
  };
  static_for<0, STAGES - 1>([&](auto ic) { issue(min((int)decltype(ic)::value, nb - 1), decltype(ic)::value); });
  for (int b = 0; b < nb; b += STAGES)
    static_for<0, STAGES>([&](auto ic) {
      if (b + decltype(ic)::value < nb) step(ic, b + decltype(ic)::value);
    });
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // redundant tail copies drained before exit
  // Every wave's last fragment reads and every copy are done: the ring's
  // first NW * 4 KB become the waves' store staging slices.
  static_assert(NW * 4096 <= S_OFF + STAGES * S_BYTES, "staging slices fit the ring");
  __syncthreads();
  gemm_epilogue<NW, 1, TN, GELU>(acc, mw, by, n0, lr, lh, lane, wave, tid, M, N, row_scale, Y, row_seq, amax,
                                 reinterpret_cast<float*>(lds) + wave * 1024, vto);
}

template <int NW, int TN, bool GELU, int STAGES>
hipError_t launch_lds(const int8_t* A, int a_rows, const int8_t* W, const float* St, const float* rs, float* Y,
                      int M, int N, int K, hipStream_t s, const int32_t* row_seq = nullptr, float* amax = nullptr,
                      const sg_vt_out* vto = nullptr) {
  constexpr int BM = NW * 32, BN = TN * 32;
  const int gm = (M + BM - 1) / BM;
  if ((int64_t)gm * BM > a_rows) return hipErrorInvalidValue;
  if (vto && (GELU || !vto->vt || vto->col0 <= 0 || vto->col0 % BN || vto->col0 >= N || (vto->ldvt & 7) ||
              !vto->row_seq || !vto->seq_off || !vto->voff || (reinterpret_cast<uintptr_t>(vto->vt) & 15) ||
              (int64_t)(N - vto->col0) * vto->ldvt > INT32_MAX))
    return hipErrorInvalidValue;  // whole V tiles; 16-byte chunk stores; 32-bit V^T offsets
  const sg_vt_out vo = vto ? *vto : sg_vt_out{nullptr, 0, 0, nullptr, nullptr, nullptr};
  dim3 grid((N + BN - 1) / BN, gm);
  hipLaunchKernelGGL((k_gemm_q8_lds<NW, TN, GELU, STAGES>), grid, dim3(NW * SG_WAVE), 0, s, A, a_rows, W, St, rs, Y,
                     M, N, K, row_seq, amax, vo);
  return hipGetLastError();
}


// GEMM + residual post-norm for the N = 768 projections (O and down).  In
// the forward the output o only feeds the residual post-norm
// (model_int8.go:203-210 / :225-232): h = RMSNorm(o; w_post) + h, then
// xn = RMSNorm(h; w_next) with the sequences' max|xn| folded into amax (or xn
// stored, after the last layer).  Here a workgroup computes whole rows -- 64
// rows x all 768 columns; wave w (16 of them) the rows 32 (w / 8) .. + 31 and
// the columns 96 (w % 8) .. + 95 (three 32x32 subtiles) -- so the norm runs in
// the same launch on the values gemm_q8 would store: each 32-row half of the
// tile is staged in LDS row-major and an 8-lane group per row runs the row
// kernel's arithmetic on it (sg_post_res_norm_lds).  o never reaches HBM, and
// the separate norm launch goes away.
//
// K loop: the direct-to-LDS ring of k_gemm_q8_lds (3 stages, two blocks
// ahead).  A block is 29 1-KB copies -- the A tile (2), the 768 columns'
// weight blocks (24) and their scales (3) -- issued as two per wave (three
// redundant re-copies fill the 32 slots), so one vmcnt says "this wave's
// copies of block b have landed" and the barrier after it publishes them.
constexpr int kResN = 768;
constexpr int kResBM = 64;
template <int STAGES, bool XN>
__global__ __launch_bounds__(1024, 4) void k_gemm_q8_resnorm(
    const int8_t* __restrict__ A, int a_rows, const int8_t* __restrict__ W, const float* __restrict__ St,
    const float* __restrict__ row_scale, int M, int K, float* __restrict__ h, const float* __restrict__ w_post,
    const float* __restrict__ w_next, float eps, float* __restrict__ xn, const int32_t* __restrict__ row_seq,
    float* __restrict__ amax) {
  constexpr int N = kResN, BM = kResBM, TNW = 3, NC = N / 32, CPW = 2;
  constexpr int A_BYTES = BM * 32, W_BYTES = N * 32, S_BYTES = N * 4;
  constexpr int W_OFF = A_BYTES, S_OFF = A_BYTES + W_BYTES, STAGE = A_BYTES + W_BYTES + S_BYTES;
  // Staged rows 808 floats apart (40 banks mod 64): the eight rows of a wave's
  // lane-order reads (lane (row q, v): element 8i + v) fall in distinct banks,
  // and the two rows of each staging store 32 banks apart.
  constexpr int OST = N + 40;
  constexpr int STG_BYTES = 32 * OST * 4;
  constexpr int LDS_BYTES = STAGES * STAGE > STG_BYTES ? STAGES * STAGE : STG_BYTES;
  static_assert((STAGES - 2) * CPW <= 63, "vmcnt covers the copies in flight");
  __shared__ __attribute__((aligned(16))) unsigned char lds[LDS_BYTES];
  __shared__ __attribute__((aligned(16))) float wl[2][N];  // w_post, w_next
  __shared__ float rmax[BM];
  __shared__ float rsl[BM];  // the tile's row scales, for the staging
  typedef __attribute__((address_space(3))) void* lds_ptr;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rg = wave >> 3, cg = wave & 7;
  // Row scales into LDS now (published by the K loop's first barrier): all
  // sixteen waves reach the staging together, where a global load would be
  // waited on in series with it (-3.5 % kernel time at 32768 rows).
  if (tid < BM) rsl[tid] = row_scale[min((int)blockIdx.x * BM + tid, M - 1)];
  // The norm weights into LDS (published by the K loop's first barrier): the
  // norm reads them per chunk, from LDS at LDS latency.
  for (int i = tid; i < N; i += 1024) {
    wl[0][i] = w_post[i];
    wl[1][i] = w_next[i];
  }
  const int lr = lane & 31, lh = lane >> 5;
  const int m0 = blockIdx.x * BM;
  const int nb = K >> 5;
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_ptr)lds;

  // Copy slot s = 2 wave + i: s < 24 the weight blocks of columns
  // 64 (s % 12) .. + 63, half s / 12; 24, 25 the A tile halves; 26..28 the
  // scales 256 (s - 26) .. + 255; 29..31 re-copy slots 26, 27, 24.
  auto issue = [&](int b, int st) {
    const uint32_t base = lds0 + (uint32_t)(st * STAGE);
#pragma unroll
    for (int i = 0; i < CPW; i++) {
      const int s = CPW * wave + i;  // wave-uniform
      if (s < 24) {
        const int hh = s / 12, g = s % 12;
        sg_lds_copy16(base + W_OFF + hh * (N * 16) + g * 1024, (uint32_t)lane * 32u + 16u * hh,
                      sg_raw_rsrc(W + ((int64_t)b * N + 64 * g) * 32), 0u);
      } else {
        const int u = s < 29 ? s - 24 : (s == 31 ? 0 : s - 27);  // 0, 1: A halves; 2..4: scales
        if (u < 2)
          sg_lds_copy16(base + u * 1024, (uint32_t)lane * 32u + 16u * u,
                        sg_raw_rsrc(A + ((int64_t)b * a_rows + m0) * 32), 0u);
        else
          sg_lds_copy16(base + S_OFF + (u - 2) * 1024, (uint32_t)lane * 16u,
                        sg_raw_rsrc(St + (int64_t)b * N + 256 * (u - 2)), 0u);
      }
    }
  };
  // Fragment reads (stage 0): A rows 32 rg + lr, half lh; W and scale of
  // column 96 cg + 32 t + lr.
  const uint32_t ra_f = lh * (BM * 16) + (32 * rg + lr) * 16;
  const uint32_t rw_f = W_OFF + lh * (N * 16) + (96 * cg + lr) * 16;
  const uint32_t rd_f = S_OFF + (96 * cg + lr) * 4;

  f32x16_t acc[TNW];
#pragma unroll
  for (int t = 0; t < TNW; t++)
#pragma unroll
    for (int r = 0; r < 16; r++) acc[t][r] = 0.0f;
  const i32x16_t bias = magic_bias();
  auto step = [&](auto stc, int b) {
    constexpr int ST = decltype(stc)::value;
    sg_wait_vmcnt<(STAGES - 2) * CPW>();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    issue(min(b + STAGES - 1, nb - 1), (ST + STAGES - 1) % STAGES);
    const i32x4_t fa = *reinterpret_cast<const i32x4_t*>(lds + ra_f + ST * STAGE);
#pragma unroll
    for (int t = 0; t < TNW; t++) {
      const i32x4_t fw = *reinterpret_cast<const i32x4_t*>(lds + rw_f + ST * STAGE + t * 512);
      const float d = *reinterpret_cast<const float*>(lds + rd_f + ST * STAGE + t * 128);
      const i32x16_t pp = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa, fw, bias, 0, 0, 0);
      block_fma16(pp, d, acc[t]);
    }
  };
  static_for<0, STAGES - 1>([&](auto ic) { issue(min((int)decltype(ic)::value, nb - 1), decltype(ic)::value); });
  for (int b = 0; b < nb; b += STAGES)
    static_for<0, STAGES>([&](auto ic) {
      if (b + decltype(ic)::value < nb) step(ic, b + decltype(ic)::value);
    });
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // redundant tail copies landed: the ring is free
  __syncthreads();

  float* stg = reinterpret_cast<float*>(lds);
  // Half p of the tile, o = acc * row_scale as gemm_q8 stores it, into LDS.
  auto stage = [&](int p) {
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int rl = 8 * (r >> 2) + 4 * lh + (r & 3);
      const float rs = rsl[32 * p + rl];
#pragma unroll
      for (int t = 0; t < TNW; t++) stg[rl * OST + 96 * cg + 32 * t + lr] = acc[t][r] * rs;
    }
  };
  // Rows 8 cg + q of half rg (waves cg < 4), an 8-lane group each; the first
  // quarter of each row's h is loaded ahead of the half's staging.
  const int q = lane >> 3, j = lane & 7, rl = 8 * cg + q, nrow = m0 + 32 * rg + rl;
  const bool nvalid = cg < 4 && nrow < M;
  f32x4_t hv0[NC / 4];
  auto load_h = [&]() {
    if (nvalid) {
      const f32x4_t* hp = reinterpret_cast<const f32x4_t*>(h + (int64_t)nrow * N) + j;
#pragma unroll
      for (int k = 0; k < NC / 4; k++) hv0[k] = __builtin_nontemporal_load(&hp[8 * k]);
    }
  };
  auto norm_rows = [&](int p) {
    if (cg >= 4) return;
    float m = 0.0f;
    if (nvalid)
      m = sg_post_res_norm_lds<NC, XN>(stg + rl * OST, h + (int64_t)nrow * N, hv0, wl[0], wl[1], eps,
                                       XN ? xn + (int64_t)nrow * N : nullptr, j);
    m = sg_max8(m);
    if (j == 0) rmax[32 * p + rl] = m;
  };
  // The waves of each half stage it and norm it in turn; the branch is
  // wave-uniform and both sides pass four barriers, and a wave's
  // accumulators die at its staging.
  if (rg == 0) {
    load_h();
    stage(0);
    __syncthreads();
    norm_rows(0);
    __syncthreads();
    __syncthreads();
    __syncthreads();
  } else {
    __syncthreads();
    __syncthreads();  // half 0 normed: the staging area is free
    load_h();
    stage(1);
    __syncthreads();
    norm_rows(1);
    __syncthreads();
  }
  if (amax) {  // the rows' max|xn| into their sequences' maxima
    const int r_last = min(m0 + BM, M) - 1;
    if (row_seq[m0] == row_seq[r_last]) {
      if (wave == 0) {
        const float v = sg_wave_max(rmax[lane]);
        if (lane == 0) sg_atomic_max_nonneg(amax + row_seq[m0], v);
      }
    } else {
      sg_seg_seq_max(rmax, r_last - m0 + 1, m0, row_seq, amax);
    }
  }
}

// Issue-rate yardstick for the K loop's arithmetic (sg_issue_probe), with no
// memory traffic: per step a wave issues two independent int8 MFMAs
// (kind 0 and 2), then converts and accumulates the previous step's two
// block-sum subtiles as block_fma16 does (kind 0 and 1: 32 subtractions and
// 32 v_fmac).  Kind 0 is the K loop's per-subtile work; 1 and 2 its VALU and
// matrix halves alone.  Each wave records its shader-clock cycles (s_memtime)
// and constant-rate wall clock (s_memrealtime) over `iters` steps.
template <int KIND>
__global__ __launch_bounds__(256) void k_issue_probe(float* __restrict__ sink, long long* __restrict__ clk, int iters) {
  const int lane = threadIdx.x & 63;
  if constexpr (KIND == 3) {
    // The attention's matrix instruction alone: four independent chains of
    // v_mfma_f32_16x16x32_f16 (16 cycles each at the 2.5 PFLOP/s dense fp16
    // peak), two per probe "subtile" step.
    typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
    h8_t x, y;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      x[i] = (_Float16)(lane * 0.01f + i);
      y[i] = (_Float16)(i * 0.5f);
    }
    f32x4_t c0 = {0, 0, 0, 0}, c1 = c0, c2 = c0, c3 = c0;
    __syncthreads();
    const long long t0 = clock64(), r0 = wall_clock64();
    for (int i = 0; i < iters; i += 2) {
      c0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(x, y, c0, 0, 0, 0);
      c1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(y, x, c1, 0, 0, 0);
      c2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(x, x, c2, 0, 0, 0);
      c3 = __builtin_amdgcn_mfma_f32_16x16x32_f16(y, y, c3, 0, 0, 0);
    }
    const long long t1 = clock64(), r1 = wall_clock64();
    sink[blockIdx.x * 256 + threadIdx.x] = c0[0] + c1[1] + c2[2] + c3[3];
    if (lane == 0) {
      const int wv = blockIdx.x * 4 + (threadIdx.x >> 6);
      clk[2 * wv] = t1 - t0;
      clk[2 * wv + 1] = r1 - r0;
    }
    return;
  }
  i32x4_t a = {lane, 3, 5, 7}, w = {11, lane, 13, 17};
  const i32x16_t bias = magic_bias();
  f32x16_t acc0, acc1;
#pragma unroll
  for (int r = 0; r < 16; r++) {
    acc0[r] = 0.0f;
    acc1[r] = 0.0f;
  }
  i32x16_t p0 = bias, p1 = bias;
  p0[0] += lane;
  p1[1] += lane;
  const float d = 1.0f + lane * 1e-7f;
  __syncthreads();
  const long long t0 = clock64(), r0 = wall_clock64();
  for (int i = 0; i < iters; i += 2) {
    i32x16_t q0 = p0, q1 = p1;
    if (KIND != 1) {
      q0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, w, bias, 0, 0, 0);
      q1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(w, a, bias, 0, 0, 0);
      if (KIND == 2) asm volatile("" ::"v"(q0), "v"(q1));  // results kept live without the update
    }
    if (KIND != 2) {
      block_fma16(p0, d, acc0);
      block_fma16(p1, d, acc1);
    }
    a.x += 1;
    if (KIND != 1) {
      p0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, w, bias, 0, 0, 0);
      p1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(w, a, bias, 0, 0, 0);
    } else {
      p0 = q1;
      p1 = q0;
      asm volatile("" : "+v"(p0), "+v"(p1));
    }
    if (KIND != 2) {
      block_fma16(q0, d, acc0);
      block_fma16(q1, d, acc1);
    }
    a.x += 1;
  }
  const long long t1 = clock64(), r1 = wall_clock64();
  float s = 0.0f;
#pragma unroll
  for (int r = 0; r < 16; r++) s += acc0[r] + acc1[r] + (float)p0[r] + (float)p1[r];
  sink[blockIdx.x * 256 + threadIdx.x] = s;
  if (lane == 0) {
    const int wv = blockIdx.x * 4 + (threadIdx.x >> 6);
    clk[2 * wv] = t1 - t0;
    clk[2 * wv + 1] = r1 - r0;
  }
}

}  // namespace

namespace sgk {

// Kernel choice by M, from tile sweeps on MI355X at the model's shapes
// (M = 256 .. 32768, the forward's N and K) and, for the sizes where the
// forward runs two sequence groups at once, from the two-group step time:
// below kRdRows the register-direct 64x64 tiles (2x2 waves of 32x32), then
// the 4-wave direct-to-LDS kernel (128 x 64 tiles, 6-stage ring) and from
// kLds8Rows the 8-wave one (256 x 128 tiles, 3-stage ring).  Standalone the
// register-direct 64x128 tiles beat both LDS kernels up to ~24k rows (QKV at
// M = 16384: 43.3 vs 46.2 us), but two groups of 16384 tokens running them
// side by side took 19.3 ms per config-2 step against 18.9 with the LDS
// kernels: the LDS kernels read each operand tile from L2 once per workgroup,
// the register-direct ones once per wave.  The gate/up GEMM (N = 2 x 1152,
// gate and up subtiles paired in one wave) takes register-direct 4-wave
// 128 x 64 tiles below kGeluLdsRows rows (sizes that only occur as one
// group: 22.0 vs 26.3 us at M = 2048), then the 8-wave kernel.
constexpr int kRdRows = 6144, kLds8Rows = 12288, kGeluLdsRows = 4096;
// gemm_q8_res_norm: the fused kernel from kResRows rows (below, gemm_q8 and
// post_res_norm run as two launches).
constexpr int kResRows = 8192;
// Register-direct launches of at most kPipeTiles workgroups -- fewer than
// two waves per SIMD, so the other waves cannot fill a wave's MFMA latency --
// take the MFMA-ahead loop with a 3-stage ring (at M = 32: 4.8 vs 5.4 us for
// K = 768; at M = 2048, N = 256: 5.5 vs 6.0 us); larger grids keep the plain
// 2-stage loop, whose lower register count gives more waves per SIMD (QKV at
// M = 2048: 10.3 vs 10.8 us).  With cold weights (the forward: every layer's
// weights were last read a whole forward earlier, so their loads come from
// MALL or HBM) those small grids take a 6-stage ring instead, which keeps
// twice the blocks' loads in flight per wave: a 1 x 32 forward 2.24 -> 2.05
// ms, 1 x 512 3.52 -> 3.36 ms.  With the weights in L2 (one weight called
// again and again) the 3-stage ring is faster (M = 2048: Q/O 7.5 vs 8.2 us).
constexpr int kPipeTiles = 384;
// Batches of at most kTinyRows rows take k_gemm_q8_tiny.
constexpr int kTinyRows = 256;
inline int rd_tiles(int M, int N, int BM, int BN) { return ((M + BM - 1) / BM) * ((N + BN - 1) / BN); }

bool gemm_writes_vt(int M) { return M >= kRdRows; }

hipError_t gemm_q8(const int8_t* A, int a_rows, const int8_t* W, const float* St, const float* row_scale, float* Y,
                   int32_t* sums, int M, int N, int K, hipStream_t s, bool cold_weights, const sg_vt_out* vto) {
  if (M <= 0 || N <= 0) return hipSuccess;
  if (K <= 0 || K % 32) return hipErrorInvalidValue;
  if (vto && (sums || !gemm_writes_vt(M))) return hipErrorInvalidValue;
  if (sums) return launch_rd<1, 1, 1, 1, true>(A, a_rows, W, St, row_scale, Y, sums, M, N, K, s);
  if (M <= kTinyRows) return launch_tiny<false, 8>(A, a_rows, W, St, row_scale, Y, M, N, K, s);
  if (M < kRdRows) {
    if (rd_tiles(M, N, 64, 64) <= kPipeTiles)
      return cold_weights
                 ? launch_rd<2, 2, 1, 1, false, false, 6, true>(A, a_rows, W, St, row_scale, Y, nullptr, M, N, K, s)
                 : launch_rd<2, 2, 1, 1, false, false, 3, true>(A, a_rows, W, St, row_scale, Y, nullptr, M, N, K, s);
    return launch_rd<2, 2, 1, 1, false>(A, a_rows, W, St, row_scale, Y, nullptr, M, N, K, s);
  }
  if (M < kLds8Rows) return launch_lds<4, 2, false, 6>(A, a_rows, W, St, row_scale, Y, M, N, K, s, nullptr, nullptr, vto);
  return launch_lds<8, 4, false, 3>(A, a_rows, W, St, row_scale, Y, M, N, K, s, nullptr, nullptr, vto);
}

hipError_t gemm_q8_gelu(const int8_t* A, int a_rows, const int8_t* W, const float* St, const float* row_scale,
                        float* G, int M, int Nh, int K, const int32_t* row_seq, float* amax, hipStream_t s,
                        bool cold_weights) {
  if (M <= 0 || Nh <= 0) return hipSuccess;
  if (K <= 0 || K % 32 || Nh % 32) return hipErrorInvalidValue;
  if (amax && !row_seq) return hipErrorInvalidValue;
  if (M <= kTinyRows) return launch_tiny<true, 8>(A, a_rows, W, St, row_scale, G, M, 2 * Nh, K, s, row_seq, amax);
  if (M < kGeluLdsRows && rd_tiles(M, 2 * Nh, 128, 64) <= kPipeTiles)
    return cold_weights ? launch_rd<4, 1, 1, 2, false, true, 6, true>(A, a_rows, W, St, row_scale, G, nullptr, M,
                                                                      2 * Nh, K, s, row_seq, amax)
                        : launch_rd<4, 1, 1, 2, false, true, 3, true>(A, a_rows, W, St, row_scale, G, nullptr, M,
                                                                      2 * Nh, K, s, row_seq, amax);
  if (M < kGeluLdsRows)
    return launch_rd<4, 1, 1, 2, false, true>(A, a_rows, W, St, row_scale, G, nullptr, M, 2 * Nh, K, s, row_seq,
                                              amax);
  return launch_lds<8, 4, true, 3>(A, a_rows, W, St, row_scale, G, M, 2 * Nh, K, s, row_seq, amax);
}


bool gemm_res_norm_fused(int M, int N, const float* w_post, const float* w_next) {
  return N == kResN && M >= kResRows && w_post && w_next;
}

hipError_t gemm_q8_res_norm(const int8_t* A, int a_rows, const int8_t* W, const float* St, const float* row_scale,
                            float* o, int M, int N, int K, float* h, const float* w_post, const float* w_next, float eps,
                            float* xn, const int32_t* row_seq, float* amax, hipStream_t s) {
  if (M <= 0) return hipSuccess;
  if (K <= 0 || K % 32) return hipErrorInvalidValue;
  if (amax && !row_seq) return hipErrorInvalidValue;
  if (!gemm_res_norm_fused(M, N, w_post, w_next)) {
    const hipError_t e = gemm_q8(A, a_rows, W, St, row_scale, o, nullptr, M, N, K, s);
    if (e != hipSuccess) return e;
    return post_res_norm(o, h, w_post, w_next, eps, M, N, xn, row_seq, amax, s);
  }
  const int gm = (M + kResBM - 1) / kResBM;
  if ((int64_t)gm * kResBM > a_rows) return hipErrorInvalidValue;
  if (xn)
    hipLaunchKernelGGL((k_gemm_q8_resnorm<3, true>), dim3(gm), dim3(1024), 0, s, A, a_rows, W, St, row_scale, M, K, h,
                       w_post, w_next, eps, xn, row_seq, amax);
  else
    hipLaunchKernelGGL((k_gemm_q8_resnorm<3, false>), dim3(gm), dim3(1024), 0, s, A, a_rows, W, St, row_scale, M, K,
                       h, w_post, w_next, eps, xn, row_seq, amax);
  return hipGetLastError();
}

hipError_t issue_probe(int kind, int blocks, float* sink, long long* clk, int iters, hipStream_t s) {
  if (blocks <= 0 || iters <= 0 || iters % 2) return hipErrorInvalidValue;
  switch (kind) {
    case 0:
      hipLaunchKernelGGL(k_issue_probe<0>, dim3(blocks), dim3(256), 0, s, sink, clk, iters);
      break;
    case 1:
      hipLaunchKernelGGL(k_issue_probe<1>, dim3(blocks), dim3(256), 0, s, sink, clk, iters);
      break;
    case 2:
      hipLaunchKernelGGL(k_issue_probe<2>, dim3(blocks), dim3(256), 0, s, sink, clk, iters);
      break;
    case 3:
      hipLaunchKernelGGL(k_issue_probe<3>, dim3(blocks), dim3(256), 0, s, sink, clk, iters);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace sgk

