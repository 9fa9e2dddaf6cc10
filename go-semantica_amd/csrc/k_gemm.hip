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
// inside v_mfma_f32_32x32x16_f16 is exact in any order: two MFMAs started
// from a zero accumulator produce float(P_b) with no rounding at all.  That
// removes the int32->float conversion from the epilogue, which leaves one
// v_fma_f32 per (m, n, block); with the int8 MFMA the epilogue would need a
// convert and an FMA per element (2 VALU ops per 32 MACs) and cap the matrix
// cores at a quarter of their int8 rate.  Per 32x32 tile and block: 2 MFMAs
// (64 cycles) against 16 FMAs (64 cycles) -- the two pipes are balanced.
//
// Operand layout (written by the quantize kernel and the load-time repack):
// block-major fp16 [K/32][rows][32], i.e. a K-block of a 32-row group is one
// contiguous 2 KB piece.  Lane (r, h) of a wave reads the 32 bytes
// k = 16h..16h+15 of row r: the first MFMA takes k 16h..16h+7, the second
// 16h+8..16h+15.  A and W use the same assignment, so each block's dot
// product is complete whatever k order the matrix core applies internally.
// Block scales are St [K/32][N] fp32 (32 consecutive columns = 128 bytes).
#include <type_traits>

#include "sg_device.h"
#include "sg_kernels.h"

typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x16_t __attribute__((ext_vector_type(16)));

namespace {

struct Frag {
  half8_t lo, hi;
};

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

template <int TM, int TN>
struct Stage {
  Frag a[TM], w[TN];
  float d[TN];
};

template <int TM, int TN>
__device__ __forceinline__ void fetch(Stage<TM, TN>& st, const _Float16* const (&ap)[TM],
                                      const _Float16* const (&wp)[TN], const float* const (&sp)[TN], int b,
                                      int64_t a_bstride, int64_t w_bstride, int N) {
#pragma unroll
  for (int tm = 0; tm < TM; tm++) {
    const _Float16* p = ap[tm] + b * a_bstride;
    st.a[tm].lo = *reinterpret_cast<const half8_t*>(p);
    st.a[tm].hi = *reinterpret_cast<const half8_t*>(p + 8);
  }
#pragma unroll
  for (int tn = 0; tn < TN; tn++) {
    const _Float16* p = wp[tn] + b * w_bstride;
    st.w[tn].lo = *reinterpret_cast<const half8_t*>(p);
    st.w[tn].hi = *reinterpret_cast<const half8_t*>(p + 8);
    st.d[tn] = sp[tn][(int64_t)b * N];
  }
}

template <int TM, int TN, bool SUMS>
__device__ __forceinline__ void compute(const Stage<TM, TN>& st, f32x16_t (&acc)[TM][TN], int32_t* sums, int M,
                                        int N, int nb, int b, int m_base, int n_base, int lr, int lh) {
  const f32x16_t zero = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
  f32x16_t p[TM][TN];
#pragma unroll
  for (int tm = 0; tm < TM; tm++)
#pragma unroll
    for (int tn = 0; tn < TN; tn++) {
      p[tm][tn] = __builtin_amdgcn_mfma_f32_32x32x16_f16(st.a[tm].lo, st.w[tn].lo, zero, 0, 0, 0);
      p[tm][tn] = __builtin_amdgcn_mfma_f32_32x32x16_f16(st.a[tm].hi, st.w[tn].hi, p[tm][tn], 0, 0, 0);
    }
#pragma unroll
  for (int tm = 0; tm < TM; tm++)
#pragma unroll
    for (int tn = 0; tn < TN; tn++) {
      if (SUMS) {
        const int col = n_base + tn * 32 + lr;
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const int row = m_base + tm * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
          if (row < M && col < N) sums[((int64_t)row * N + col) * nb + b] = (int32_t)p[tm][tn][r];
        }
      }
#pragma unroll
      for (int r = 0; r < 16; r++) acc[tm][tn][r] = __builtin_fmaf(p[tm][tn][r], st.d[tn], acc[tm][tn][r]);
    }
}

// WM x WN waves per workgroup, each wave owns TM x TN tiles of 32x32 outputs.
// A has a_rows rows per K-block (>= the padded M the grid covers).
template <int WM, int WN, int TM, int TN, bool SUMS>
__global__ __launch_bounds__(WM* WN* SG_WAVE) void k_gemm_q8(const _Float16* __restrict__ A, int a_rows,
                                                             const _Float16* __restrict__ W,
                                                             const float* __restrict__ St,
                                                             const float* __restrict__ row_scale,
                                                             float* __restrict__ Y, int32_t* __restrict__ sums, int M,
                                                             int N, int K) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / WN, wn = wave % WN;
  int bx, by;
  xcd_tile(bx, by);
  const int m_base = by * (WM * TM * 32) + wm * TM * 32;
  const int n_base = bx * (WN * TN * 32) + wn * TN * 32;
  const int lr = lane & 31, lh = lane >> 5;
  const int nb = K >> 5;
  const int64_t a_bstride = (int64_t)a_rows * 32, w_bstride = (int64_t)N * 32;

  const _Float16* ap[TM];
  const _Float16* wp[TN];
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

  // Register double buffer: block b+1 is in flight while block b computes.
  Stage<TM, TN> s0, s1;
  fetch<TM, TN>(s0, ap, wp, sp, 0, a_bstride, w_bstride, N);
  int b = 0;
  for (; b + 2 <= nb; b += 2) {
    fetch<TM, TN>(s1, ap, wp, sp, b + 1, a_bstride, w_bstride, N);
    compute<TM, TN, SUMS>(s0, acc, sums, M, N, nb, b, m_base, n_base, lr, lh);
    if (b + 2 < nb) fetch<TM, TN>(s0, ap, wp, sp, b + 2, a_bstride, w_bstride, N);
    compute<TM, TN, SUMS>(s1, acc, sums, M, N, nb, b + 1, m_base, n_base, lr, lh);
  }
  if (b < nb) compute<TM, TN, SUMS>(s0, acc, sums, M, N, nb, b, m_base, n_base, lr, lh);

  // 32x32 accumulator layout: lane holds column lr; register r holds row
  // 8*(r/4) + 4*lh + r%4 of the tile.  The row scales are fetched for all
  // rows first (clamped index, no branch) so the loads overlap.
#pragma unroll
  for (int tm = 0; tm < TM; tm++) {
    float rs[16];
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int row = m_base + tm * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
      rs[r] = row_scale[row < M ? row : M - 1];
    }
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int row = m_base + tm * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
#pragma unroll
      for (int tn = 0; tn < TN; tn++) {
        const int col = n_base + tn * 32 + lr;
        if (row < M && col < N) Y[(int64_t)row * N + col] = acc[tm][tn][r] * rs[r];
      }
    }
  }
}

// Split-path variant: a workgroup of NW waves covers NW*TM*32 rows x TN*32
// columns.  Each wave streams its own A fragments straight from global
// memory (through the vector L1), while the workgroup's small W tile of each
// K-block (TN*32 rows x 64 B) and its block scales are staged once in a
// double-buffered LDS ring and read by all NW waves.  Operand traffic is
// split between the L1 path (A, 32 MAC per byte for TN = 2) and the LDS path
// (W, 16*TM MAC per byte), instead of all of it going through one.
// Epilogue shared by the split-path kernels: Y = acc * row_scale (or, with
// GELU, g = geluquick(gate) * up over the paired subtiles, with the
// sequences' max|g| folded into amax).  Wave tile rows mw.., workgroup row
// tile by, columns n0...
template <int NW, int TM, int TN, bool GELU>
__device__ __forceinline__ void gemm_epilogue(const f32x16_t (&acc)[TM][TN], int mw, int by, int n0, int lr, int lh,
                                              int lane, int wave, int tid, int M, int N,
                                              const float* __restrict__ row_scale, float* __restrict__ Y,
                                              const int32_t* __restrict__ row_seq, float* __restrict__ amax) {
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
#pragma unroll
    for (int tm = 0; tm < TM; tm++) {
      const int mb = mw + tm * 32;
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
          if (ok) Y[(int64_t)row * Nh + col] = g;
          a = ok ? fmaxf(a, fabsf(g)) : a;
        }
        if (one_seq) {
          mx = fmaxf(mx, a);
        } else if (amax) {  // rows of several sequences: per-row maxima, folded below
#pragma unroll
          for (int o = 1; o < 32; o <<= 1) a = fmaxf(a, __shfl_xor(a, o));
          if (lr == 0) rmax[row - r_first] = a;
        }
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

// GELU: the FFN's gate/up GEMM with GELUQuickSIMD * up in the epilogue
// (model_int8.go:520-535).  W holds gate and up rows interleaved in groups
// of 32 (rows 64j..64j+31 = gate 32j.., rows 64j+32.. = up 32j..), so the
// two 32-column subtiles of a wave are gate and up of the same features.
// Each value is rounded exactly as the unfused path rounds it (gate and up
// stored as acc * row_scale, then k_gelu_mul's arithmetic), so Y = g [M][N/2]
// is bit-identical; the sequences' max|g| is folded into amax (row_seq).
template <int NW, int TM, int TN, bool GELU>
__global__ __launch_bounds__(NW* SG_WAVE) void k_gemm_q8_sp(const _Float16* __restrict__ A, int a_rows,
                                                            const _Float16* __restrict__ W,
                                                            const float* __restrict__ St,
                                                            const float* __restrict__ row_scale,
                                                            float* __restrict__ Y, int M, int N, int K,
                                                            const int32_t* __restrict__ row_seq,
                                                            float* __restrict__ amax) {
  constexpr int NT = NW * SG_WAVE;
  constexpr int BN = TN * 32, BMW = TM * 32;
  constexpr int W_V = BN * 32 / 4;  // 8-byte pieces of the W tile (BN rows x 32 halfs)
  constexpr int WPT = (W_V + NT - 1) / NT;
  __shared__ __attribute__((aligned(16))) _Float16 Ws[2][BN * 32];
  __shared__ float Ss[2][BN];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lr = lane & 31, lh = lane >> 5;
  int bx, by;
  xcd_tile(bx, by);
  const int n0 = bx * BN;
  const int mw = by * NW * BMW + wave * BMW;  // this wave's first row
  const int nb = K >> 5;
  const int64_t a_bstride = (int64_t)a_rows * 32, w_bstride = (int64_t)N * 32;

  // W piece v of the tile: row n0 + v/8, halfs 4*(v%8) .. +4.
  const _Float16* wsrc[WPT];
#pragma unroll
  for (int i = 0; i < WPT; i++) {
    const int v = tid + i * NT;
    const int row = n0 + (v >> 3) < N ? n0 + (v >> 3) : N - 1;
    wsrc[i] = W + (int64_t)row * 32 + 4 * (v & 7);
  }
  const int s_col = n0 + tid < N ? n0 + tid : N - 1;
  struct WReg {
    half4_t w[WPT];
    float s;
  };
  auto wload = [&](WReg& r, int b) {
#pragma unroll
    for (int i = 0; i < WPT; i++)
      if (tid + i * NT < W_V) r.w[i] = *reinterpret_cast<const half4_t*>(wsrc[i] + b * w_bstride);
    if (tid < BN) r.s = St[(int64_t)b * N + s_col];
  };
  // LDS W layout: row r (64 B = four 16-byte chunks c) stores chunk c at slot
  // c ^ ((r >> 2) & 3), so a 16-lane fragment read (16 consecutive rows, one
  // chunk) touches 16 distinct bank groups.
  auto wslot = [](int r, int c) { return r * 32 + ((c ^ ((r >> 2) & 3)) << 3); };
  auto wstore = [&](const WReg& r, int buf) {
#pragma unroll
    for (int i = 0; i < WPT; i++) {
      const int v = tid + i * NT;  // piece v: row v/8, chunk (v%8)/2, half (v%2)
      if (v < W_V) *reinterpret_cast<half4_t*>(&Ws[buf][wslot(v >> 3, (v & 7) >> 1) + 4 * (v & 1)]) = r.w[i];
    }
    if (tid < BN) Ss[buf][tid] = r.s;
  };

  const _Float16* ap[TM];
#pragma unroll
  for (int tm = 0; tm < TM; tm++) ap[tm] = A + (int64_t)(mw + tm * 32 + lr) * 32 + 16 * lh;
  auto aload = [&](Frag (&f)[TM], int b) {
#pragma unroll
    for (int tm = 0; tm < TM; tm++) {
      const _Float16* p = ap[tm] + b * a_bstride;
      f[tm].lo = *reinterpret_cast<const half8_t*>(p);
      f[tm].hi = *reinterpret_cast<const half8_t*>(p + 8);
    }
  };

  f32x16_t acc[TM][TN];
#pragma unroll
  for (int tm = 0; tm < TM; tm++)
#pragma unroll
    for (int tn = 0; tn < TN; tn++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[tm][tn][r] = 0.0f;

  auto compute = [&](const Frag (&fa)[TM], int buf) {
    const f32x16_t zero = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    Frag fw[TN];
    float d[TN];
#pragma unroll
    for (int tn = 0; tn < TN; tn++) {
      const int row = tn * 32 + lr;
      fw[tn].lo = *reinterpret_cast<const half8_t*>(&Ws[buf][wslot(row, 2 * lh)]);
      fw[tn].hi = *reinterpret_cast<const half8_t*>(&Ws[buf][wslot(row, 2 * lh + 1)]);
      d[tn] = Ss[buf][row];
    }
    f32x16_t p[TM][TN];
#pragma unroll
    for (int tm = 0; tm < TM; tm++)
#pragma unroll
      for (int tn = 0; tn < TN; tn++) {
        p[tm][tn] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[tm].lo, fw[tn].lo, zero, 0, 0, 0);
        p[tm][tn] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[tm].hi, fw[tn].hi, p[tm][tn], 0, 0, 0);
      }
#pragma unroll
    for (int tm = 0; tm < TM; tm++)
#pragma unroll
      for (int tn = 0; tn < TN; tn++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[tm][tn][r] = __builtin_fmaf(p[tm][tn][r], d[tn], acc[tm][tn][r]);
  };

  // W ring: LDS buffer (b & 1) holds block b; w0/w1 carry blocks b+1, b+2.
  // A: registers fa0/fa1 alternate, one block ahead.
  WReg w0, w1;
  Frag fa0[TM], fa1[TM];
  wload(w0, 0);
  if (nb > 1) wload(w1, 1);
  aload(fa0, 0);
  wstore(w0, 0);
  if (nb > 2) wload(w0, 2);
  __syncthreads();
  for (int b = 0; b < nb; b += 2) {
    if (b + 1 < nb) aload(fa1, b + 1);
    compute(fa0, 0);
    if (b + 1 < nb) {
      wstore(w1, 1);
      if (b + 3 < nb) wload(w1, b + 3);
    }
    __syncthreads();
    if (b + 1 >= nb) break;
    if (b + 2 < nb) aload(fa0, b + 2);
    compute(fa1, 1);
    if (b + 2 < nb) {
      wstore(w0, 0);
      if (b + 4 < nb) wload(w0, b + 4);
    }
    __syncthreads();
  }

  gemm_epilogue<NW, TM, TN, GELU>(acc, mw, by, n0, lr, lh, lane, wave, tid, M, N, row_scale, Y, row_seq, amax);
}

// Direct-to-LDS kernel.  Workgroup: NW waves x 32 rows, 32*TN columns.
// Every K-block's A tile (each wave's own 32 rows), weight tile and scales are
// copied global -> LDS by buffer_load_dwordx4/dword ... lds (no staging
// registers) into a ring of STAGES buffers, STAGES-1 blocks ahead.  Each wave
// issues the same number of copies per block, CPB (clamped, redundant past
// the last block), so one constant s_waitcnt vmcnt covers "this wave's copies
// of block b have landed"; a bare s_barrier then publishes every wave's
// copies.  (__syncthreads' fence would wait for all copies in flight.)  Rows
// are stored in 64-byte lines with the 16-byte chunks XOR-swizzled by row, so
// fragment reads are conflict-free; the swizzle is applied by choosing which
// global chunk each lane copies.  Large M uses 8 waves, 4 subtiles, 3 stages
// (two workgroups per CU); mid-size M uses 4 waves with a deep ring, as its K
// loop is bound by copy latency, not by throughput.
//
// A copy costs no vector instruction: each K-block's buffer descriptors (64-bit
// base = this tile's part of the block slice) are built on the scalar unit,
// the per-lane byte offsets are loop-invariant and M0 is scalar.  (The flat
// global_load_lds form needed a 64-bit vector add and a readfirstlane per
// copy.)  The K loop is unrolled by the ring depth, so every LDS fragment read
// is a loop-invariant vector address plus an immediate; the LDS is laid out
// [A stages][W stages][scale stages] to keep those immediates under 64 KB.
// Only the MFMAs and the FMAs of the block-serial epilogue are vector work.
// Publishes a ring stage: this wave's copies older than the last N have
// landed (vmcnt) and its own LDS fragment reads have completed (lgkmcnt), so
// after the following barrier no wave still reads the stage the next copies
// overwrite.  (The compiler may place the last MFMAs of the previous step, and
// their lgkmcnt waits, after an s_barrier, so the read wait is explicit.)
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(N) : "memory");
}

constexpr int kBufWord3 = 0x00020000;  // raw buffer descriptor, gfx9 family
constexpr float kMagic = 12582912.0f;   // 1.5 * 2^23
constexpr int kMagicBits = 0x4B400000;  // its bit pattern

// f(integral_constant<int, I>) for I = I0 .. N-1, unrolled at compile time.
template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

template <int NW, int TN, bool GELU, int STAGES>
__global__ __launch_bounds__(NW * SG_WAVE, NW == 8 ? 4 : 1) void k_gemm_q8_bl(
    const _Float16* __restrict__ A, int a_rows, const _Float16* __restrict__ W, const float* __restrict__ St,
    const float* __restrict__ row_scale, float* __restrict__ Y, int M, int N, int K,
    const int32_t* __restrict__ row_seq, float* __restrict__ amax) {
  constexpr int BM = NW * 32, BN = TN * 32;
  constexpr int A_BYTES = BM * 64, W_BYTES = BN * 64, S_BYTES = BN * 4;
  constexpr int W_OFF = STAGES * A_BYTES, S_OFF = W_OFF + STAGES * W_BYTES;
  constexpr int WROWS = BN / NW;              // weight rows each wave copies (64 B each)
  constexpr int SLANES = BN / NW;             // scales each wave copies
  constexpr int CPB = 2 + 1 + 1;              // copies per wave per K-block
  static_assert(BN % NW == 0 && SLANES <= SG_WAVE, "weight tile split over the waves");
  static_assert((STAGES - 1) * A_BYTES < 65536 && (STAGES - 1) * W_BYTES + W_BYTES < 65536 &&
                    STAGES * S_BYTES < 65536,
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
  auto swz = [](int r, int c) { return c ^ ((r >> 2) & 3); };  // chunk slot of chunk c in row r

  // Copy sources: byte offsets inside this tile's part of block b: its BM
  // rows of A's block slice ([a_rows][32] halves), its BN rows of W's
  // ([N][32]) and its BN scales ([N] floats).  The descriptors' 64-bit bases
  // carry the rest, so no size limit applies.
  uint32_t aoff[2];
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int r = 16 * j + (lane >> 2);
    aoff[j] = (uint32_t)(wave * 32 + r) * 64u + 16u * swz(r, lane & 3);
  }
  // One 1-KB weight copy per wave.  (A guarded loop over an array of copy
  // offsets here made the host pass drop the kernel's launch stub.)
  static_assert(WROWS == 16, "one 1-KB weight copy per wave");
  const int wrow = WROWS * wave + (lane >> 2);
  const uint32_t woff = (uint32_t)(min(n0 + wrow, N - 1) - n0) * 64u + 16u * swz(wrow, lane & 3);
  const uint32_t soff = (uint32_t)(min(n0 + SLANES * wave + lane, N - 1) - n0) * 4u;

  auto issue = [&](int b, int st) {
    __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(A + ((int64_t)b * a_rows + (int64_t)by * BM) * 32), 0, A_BYTES, kBufWord3);
    __amdgpu_buffer_rsrc_t rw =
        __builtin_amdgcn_make_buffer_rsrc((void*)(W + ((int64_t)b * N + n0) * 32), 0, W_BYTES, kBufWord3);
    __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void*)(St + (int64_t)b * N + n0), 0, S_BYTES, kBufWord3);
#pragma unroll
    for (int j = 0; j < 2; j++)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_ptr)(lds + st * A_BYTES + wave * 2048 + j * 1024), 16,
                                               aoff[j], 0, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lds_ptr)(lds + W_OFF + st * W_BYTES + WROWS * 64 * wave), 16, woff, 0,
                                             0, 0);
    if (lane < SLANES)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr)(lds + S_OFF + st * S_BYTES + wave * (SLANES * 4)), 4,
                                               soff, 0, 0, 0);
  };

  // Fragment read addresses (stage 0; stage st adds st * *_BYTES).
  const int a_row = wave * 32 + lr;
  const uint32_t ra_lo = a_row * 64 + 16 * swz(a_row, 2 * lh), ra_hi = a_row * 64 + 16 * swz(a_row, 2 * lh + 1);
  const uint32_t rw_lo = W_OFF + lr * 64 + 16 * swz(lr, 2 * lh), rw_hi = W_OFF + lr * 64 + 16 * swz(lr, 2 * lh + 1);
  const uint32_t rd = S_OFF + 4 * lr;

  f32x16_t acc[1][TN];
#pragma unroll
  for (int tn = 0; tn < TN; tn++)
#pragma unroll
    for (int r = 0; r < 16; r++) acc[0][tn][r] = 0.0f;
  const f32x16_t zero = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};

  auto step = [&](auto stc, int b) {
    constexpr int ST = decltype(stc)::value;
    wait_vmcnt<(STAGES - 2) * CPB>();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    issue(min(b + STAGES - 1, nb - 1), (ST + STAGES - 1) % STAGES);
    Frag fa;
    fa.lo = *reinterpret_cast<const half8_t*>(lds + ra_lo + ST * A_BYTES);
    fa.hi = *reinterpret_cast<const half8_t*>(lds + ra_hi + ST * A_BYTES);
#pragma unroll
    for (int tn = 0; tn < TN; tn++) {
      // rows 32tn + lr share lr's swizzle ((32tn + lr) >> 2 differs by a multiple of 8)
      const half8_t wlo = *reinterpret_cast<const half8_t*>(lds + rw_lo + ST * W_BYTES + tn * 2048);
      const half8_t whi = *reinterpret_cast<const half8_t*>(lds + rw_hi + ST * W_BYTES + tn * 2048);
      const float d = *reinterpret_cast<const float*>(lds + rd + ST * S_BYTES + tn * 128);
      f32x16_t pp = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa.lo, wlo, zero, 0, 0, 0);
      pp = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa.hi, whi, pp, 0, 0, 0);
#pragma unroll
      for (int r = 0; r < 16; r++) acc[0][tn][r] = __builtin_fmaf(pp[r], d, acc[0][tn][r]);
    }
  };

  static_assert(STAGES >= 3 && (STAGES - 2) * CPB <= 63, "vmcnt covers the copies in flight");
  static_for<0, STAGES - 1>([&](auto ic) { issue(min((int)decltype(ic)::value, nb - 1), decltype(ic)::value); });
  for (int b = 0; b < nb; b += STAGES)
    static_for<0, STAGES>([&](auto ic) {
      if (b + decltype(ic)::value < nb) step(ic, b + decltype(ic)::value);
    });
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // redundant tail copies drained before exit
  gemm_epilogue<NW, 1, TN, GELU>(acc, mw, by, n0, lr, lh, lane, wave, tid, M, N, row_scale, Y, row_seq, amax);
}

template <int NW, int TN, bool GELU, int STAGES>
hipError_t launch_bl(const _Float16* A, int a_rows, const _Float16* W, const float* St, const float* rs, float* Y,
                     int M, int N, int K, hipStream_t s, const int32_t* row_seq = nullptr, float* amax = nullptr) {
  constexpr int BM = NW * 32, BN = TN * 32;
  const int gm = (M + BM - 1) / BM;
  if ((int64_t)gm * BM > a_rows) return hipErrorInvalidValue;
  dim3 grid((N + BN - 1) / BN, gm);
  hipLaunchKernelGGL((k_gemm_q8_bl<NW, TN, GELU, STAGES>), grid, dim3(NW * SG_WAVE), 0, s, A, a_rows, W, St, rs, Y, M, N, K,
                     row_seq, amax);
  return hipGetLastError();
}

// int8-operand form of k_gemm_q8_bl: A and W hold the int8 values
// themselves (A [K/32][a_rows][32], W [K/32][N][32]), and one
// v_mfma_i32_32x32x32_i8 per subtile and block gives the exact block sum
// P_b as int32 (|P_b| <= 516,128, so its conversion to float is exact); the
// per-block FMA is unchanged, so the outputs are bit-identical to the fp16
// form.  Half the bytes are copied and read from LDS, one MFMA replaces two,
// and 16 converts per subtile and block are added.  LDS per stage:
// A [2 halves][BM rows][16 B], W [2][BN][16 B], scales [BN]: lane l of an
// MFMA operand reads row l % 32, bytes 16*(l / 32) .. +15 of its 32-byte
// block, so each fragment read is 1 KB of contiguous LDS.  Copies: NW / 2
// waves per half, each copying 64 A rows (one 1-KB copy) and, with 32
// lanes, 32 W rows (BN = 16 * NW); the other scheme (scalar descriptors,
// ring unrolled by STAGES, one vmcnt per block) is k_gemm_q8_bl's.
template <int NW, int TN, bool GELU, int STAGES>
__global__ __launch_bounds__(NW * SG_WAVE, NW == 8 ? 4 : 1) void k_gemm_q8_i8(
    const int8_t* __restrict__ A, int a_rows, const int8_t* __restrict__ W, const float* __restrict__ St,
    const float* __restrict__ row_scale, float* __restrict__ Y, int M, int N, int K,
    const int32_t* __restrict__ row_seq, float* __restrict__ amax) {
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
  // int32 -> float without v_cvt_f32_i32 (a half-rate VALU op on gfx950): the
  // MFMA starts from the bit pattern of 1.5 * 2^23 in every lane, so its int32
  // result read as a float is exactly 12582912 + P_b (|P_b| <= 32 * 128 * 127
  // < 2^22 keeps the exponent at 23 and the mantissa exact), and one
  // full-rate subtraction gives float(P_b) exactly.  The asm keeps the
  // constant in registers (no per-use rematerialisation).
  i32x16_t bias;
#pragma unroll
  for (int r = 0; r < 16; r++) bias[r] = kMagicBits;
  asm volatile("" : "+v"(bias));
  auto step = [&](auto stc, int b) {
    constexpr int ST = decltype(stc)::value;
    wait_vmcnt<(STAGES - 2) * CPB>();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    issue(min(b + STAGES - 1, nb - 1), (ST + STAGES - 1) % STAGES);
    const i32x4_t fa = *reinterpret_cast<const i32x4_t*>(lds + ra_f + ST * A_BYTES);
#pragma unroll
    for (int tn = 0; tn < TN; tn++) {
      const i32x4_t fw = *reinterpret_cast<const i32x4_t*>(lds + rw_f + ST * W_BYTES + tn * 512);
      const float d = *reinterpret_cast<const float*>(lds + rd + ST * S_BYTES + tn * 128);
      const i32x16_t pp = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa, fw, bias, 0, 0, 0);
#pragma unroll
      for (int r = 0; r < 16; r++)
        acc[0][tn][r] = __builtin_fmaf(__int_as_float(pp[r]) - kMagic, d, acc[0][tn][r]);
    }
  };
  static_for<0, STAGES - 1>([&](auto ic) { issue(min((int)decltype(ic)::value, nb - 1), decltype(ic)::value); });
  for (int b = 0; b < nb; b += STAGES)
    static_for<0, STAGES>([&](auto ic) {
      if (b + decltype(ic)::value < nb) step(ic, b + decltype(ic)::value);
    });
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // redundant tail copies drained before exit
  gemm_epilogue<NW, 1, TN, GELU>(acc, mw, by, n0, lr, lh, lane, wave, tid, M, N, row_scale, Y, row_seq, amax);
}

template <int NW, int TN, bool GELU, int STAGES>
hipError_t launch_i8(const int8_t* A, int a_rows, const int8_t* W, const float* St, const float* rs, float* Y, int M,
                     int N, int K, hipStream_t s, const int32_t* row_seq = nullptr, float* amax = nullptr) {
  constexpr int BM = NW * 32, BN = TN * 32;
  const int gm = (M + BM - 1) / BM;
  if ((int64_t)gm * BM > a_rows) return hipErrorInvalidValue;
  dim3 grid((N + BN - 1) / BN, gm);
  hipLaunchKernelGGL((k_gemm_q8_i8<NW, TN, GELU, STAGES>), grid, dim3(NW * SG_WAVE), 0, s, A, a_rows, W, St, rs, Y,
                     M, N, K, row_seq, amax);
  return hipGetLastError();
}

template <int NW, int TM, int TN, bool GELU = false>
hipError_t launch_sp(const _Float16* A, int a_rows, const _Float16* W, const float* St, const float* rs, float* Y,
                     int M, int N, int K, hipStream_t s, const int32_t* row_seq = nullptr, float* amax = nullptr) {
  constexpr int BM = NW * TM * 32, BN = TN * 32;
  const int gm = (M + BM - 1) / BM;
  if ((int64_t)gm * BM > a_rows) return hipErrorInvalidValue;
  dim3 grid((N + BN - 1) / BN, gm);
  hipLaunchKernelGGL((k_gemm_q8_sp<NW, TM, TN, GELU>), grid, dim3(NW * SG_WAVE), 0, s, A, a_rows, W, St, rs, Y, M, N,
                     K, row_seq, amax);
  return hipGetLastError();
}

template <int WM, int WN, int TM, int TN, bool SUMS>
hipError_t launch(const _Float16* A, int a_rows, const _Float16* W, const float* St, const float* rs, float* Y,
                  int32_t* sums, int M, int N, int K, hipStream_t s) {
  constexpr int BM = WM * TM * 32, BN = WN * TN * 32;
  const int gm = (M + BM - 1) / BM;
  if ((int64_t)gm * BM > a_rows) return hipErrorInvalidValue;  // A must cover the padded rows
  dim3 grid((N + BN - 1) / BN, gm);
  hipLaunchKernelGGL((k_gemm_q8<WM, WN, TM, TN, SUMS>), grid, dim3(WM * WN * SG_WAVE), 0, s, A, a_rows, W, St, rs,
                     Y, sums, M, N, K);
  return hipGetLastError();
}

// Workgroups of the 8-wave direct-to-LDS launch.
inline int64_t dl8_blocks(int M, int N) { return (int64_t)((M + 255) / 256) * ((N + 127) / 128); }

}  // namespace

namespace sgk {

hipError_t gemm_q8(const _Float16* A, int a_rows, const _Float16* W, const float* St, const float* row_scale,
                   float* Y, int32_t* sums, int M, int N, int K, hipStream_t s) {
  if (M <= 0 || N <= 0) return hipSuccess;
  if (K <= 0 || K % 32) return hipErrorInvalidValue;
  if (sums) return launch<1, 1, 1, 1, true>(A, a_rows, W, St, row_scale, Y, sums, M, N, K, s);
  // Direct-to-LDS workgroups of 8 waves (256 rows x 128 columns, 3-stage
  // copy ring, buffer-load copies) once they cover half the compute units;
  // below that, from 4096
  // rows, 4 waves x 64 columns with a 6-stage ring; otherwise 64x64
  // register-direct tiles, whose grid still covers the chip (tile sweeps on
  // MI355X at the model's shapes, M = 32 .. 4096).
  if (M >= 8192 || dl8_blocks(M, N) >= 128) return launch_bl<8, 4, false, 3>(A, a_rows, W, St, row_scale, Y, M, N, K, s);
  if (M >= 4096) return launch_bl<4, 2, false, 6>(A, a_rows, W, St, row_scale, Y, M, N, K, s);
  return launch<2, 2, 1, 1, false>(A, a_rows, W, St, row_scale, Y, nullptr, M, N, K, s);
}

hipError_t gemm_q8_i8(const int8_t* A, int a_rows, const int8_t* W, const float* St, const float* row_scale, float* Y,
                      int M, int N, int K, hipStream_t s) {
  if (M <= 0 || N <= 0) return hipSuccess;
  if (K <= 0 || K % 32) return hipErrorInvalidValue;
  if (M >= 8192 || dl8_blocks(M, N) >= 128) return launch_i8<8, 4, false, 3>(A, a_rows, W, St, row_scale, Y, M, N, K, s);
  return launch_i8<4, 2, false, 6>(A, a_rows, W, St, row_scale, Y, M, N, K, s);
}

hipError_t gemm_q8_gelu_i8(const int8_t* A, int a_rows, const int8_t* W, const float* St, const float* row_scale,
                           float* G, int M, int Nh, int K, const int32_t* row_seq, float* amax, hipStream_t s) {
  if (M <= 0 || Nh <= 0) return hipSuccess;
  if (K <= 0 || K % 32 || Nh % 32) return hipErrorInvalidValue;
  if (amax && !row_seq) return hipErrorInvalidValue;
  return launch_i8<8, 4, true, 3>(A, a_rows, W, St, row_scale, G, M, 2 * Nh, K, s, row_seq, amax);
}

hipError_t gemm_q8_gelu(const _Float16* A, int a_rows, const _Float16* W, const float* St, const float* row_scale,
                        float* G, int M, int Nh, int K, const int32_t* row_seq, float* amax, hipStream_t s) {
  if (M <= 0 || Nh <= 0) return hipSuccess;
  if (K <= 0 || K % 32 || Nh % 32) return hipErrorInvalidValue;
  if (amax && !row_seq) return hipErrorInvalidValue;
  if (M >= 8192 || dl8_blocks(M, 2 * Nh) >= 128)
    return launch_bl<8, 4, true, 3>(A, a_rows, W, St, row_scale, G, M, 2 * Nh, K, s, row_seq, amax);
  return launch_sp<4, 1, 2, true>(A, a_rows, W, St, row_scale, G, M, 2 * Nh, K, s, row_seq, amax);
}

}  // namespace sgk
