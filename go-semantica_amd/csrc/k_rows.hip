// k_rows.hip -- bandwidth-bound per-row kernels: token embedding, RMSNorm
// (pre, post, final), per-sequence int8 quantization, QK-norm + RoPE,
// GELUQuick * up, mean-pool + L2, and the load-time Q8_0 repack.
//
// Row kernels give each row to an aligned group of 8 lanes (a wave covers 8
// rows): lane j of the group owns elements j, j+8, j+16, ... which is the lane
// structure of the reference's AVX2 fp32 dot product, so RMSNorm's sum of
// squares is reproduced bit for bit (see sg_rmsnorm8 in sg_device.h).
#include <type_traits>

#include "sg_device.h"
#include "sg_kernels.h"
#include "sg_kv_prep.h"

namespace {

constexpr int kRowsPerBlock = 32;  // 256 threads, 8 lanes per row
static_assert(kRowsPerBlock == sgk::kRowKernelRows, "row kernels' workgroup rows");
constexpr int kThreads = 256;
constexpr int kQuantNbRows = 8192;  // the quantizers' branch-free form below this many rows

__device__ __forceinline__ uint16_t rd_u16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

// ---------------------------------------------------------------- repack --

// One thread per Q8_0 block: 2-byte fp16 scale + 32 int8 values
// (GGUF Q8_0 layout; extractQ8_0Scales model_int8.go:543-569 reads the same bytes).
__global__ void k_repack_q8_0(const uint8_t* __restrict__ raw, int rows, int cols, int8_t* __restrict__ w8,
                              float* __restrict__ st, int ld, int row_off, int grp, int gstride) {
  const int nb = cols / 32;
  const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= (int64_t)rows * nb) return;
  const int r = (int)(id / nb), b = (int)(id % nb);
  const int dr = row_off + (r / grp) * gstride + r % grp;
  const uint8_t* blk = raw + id * 34;
  st[(int64_t)b * ld + dr] = sg_f16_ieee(rd_u16(blk));
  int8_t* d8 = w8 + ((int64_t)b * ld + dr) * 32;
#pragma unroll
  for (int i = 0; i < 32; i++) d8[i] = (int8_t)blk[2 + i];
}

// int8 x[M][K] -> block-major int8 y[K/32][a_rows][32]: one thread moves a
// 16-byte half block (vec: x 16-byte aligned; otherwise byte by byte).
__global__ void k_i8_blocked(const int8_t* __restrict__ x, int M, int K, int8_t* __restrict__ y, int a_rows,
                             bool vec) {
  const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int kq = K / 16;
  if (id >= (int64_t)M * kq) return;
  const int m = (int)(id / kq), q = (int)(id % kq);
  const int8_t* src = x + (int64_t)m * K + 16 * q;
  int8_t* dst = y + ((int64_t)(q >> 1) * a_rows + m) * 32 + 16 * (q & 1);
  if (vec) {
    *reinterpret_cast<uint4*>(dst) = *reinterpret_cast<const uint4*>(src);
  } else {
#pragma unroll
    for (int i = 0; i < 16; i++) dst[i] = src[i];
  }
}

// Token table: int8 values plus the block scale through the gguf converter
// (ParseQ8_0Block gguf/tensor.go:94-112).
__global__ void k_repack_embd(const uint8_t* __restrict__ raw, int vocab, int d, int8_t* __restrict__ q,
                              float* __restrict__ sc) {
  const int nb = d / 32;
  const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= (int64_t)vocab * nb) return;
  const uint8_t* blk = raw + id * 34;
  sc[id] = sg_f16_gguf(rd_u16(blk));
  int8_t* dst = q + id * 32;
#pragma unroll
  for (int i = 0; i < 32; i++) dst[i] = (int8_t)blk[2 + i];
}

__global__ void k_fill(float* __restrict__ p, float v, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

__global__ void k_fill_i32(int32_t* __restrict__ p, int32_t v, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

// The first row r < T whose token is outside [0, vocab), folded into *first
// (atomicMin; *first starts at T or above).
__global__ void k_first_bad_token(const int32_t* __restrict__ tokens, int T, int vocab, int32_t* __restrict__ first) {
  const int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r < T && (tokens[r] < 0 || tokens[r] >= vocab)) atomicMin(first, r);
}

// ------------------------------------------------------------- embedding --

// Embedding (model_int8.go:166-184): h = float32(q) * d' (d' through the
// halving converter), then h *= float32(sqrt(d)) as a second rounding.
template <int NPL>
__device__ __forceinline__ int gather_row(const int32_t* tokens, int row, const int8_t* __restrict__ eq,
                                          const float* __restrict__ es, int vocab, float sqrt_d, int j,
                                          float (&x)[NPL], int32_t* err) {
  constexpr int D = NPL * 8;
  int id = tokens[row];
  if (id < 0 || id >= vocab) {
    if (j == 0) atomicMin(err, row);  // the first offending row (rows run in request order)
    id = 0;  // keep the access in bounds; the call reports SG_ERR_TOKEN
  }
  const int8_t* qr = eq + (int64_t)id * D;
  const float* sr = es + (int64_t)id * (D / 32);
#pragma unroll
  for (int i = 0; i < NPL; i++) {
    const int c = 8 * i + j;
    const float v = (float)qr[c] * sr[c >> 5];
    x[i] = v * sqrt_d;
  }
  return id;
}

template <int NPL>
__global__ __launch_bounds__(kThreads) void k_embed_norm(const int32_t* __restrict__ tokens, int T,
                                                         const int8_t* __restrict__ eq, const float* __restrict__ es,
                                                         int vocab, float sqrt_d, const float* __restrict__ w,
                                                         float eps, const int32_t* __restrict__ row_seq,
                                                         float* __restrict__ h, float* __restrict__ xn,
                                                         float* __restrict__ amax, int32_t* __restrict__ err) {
  constexpr int D = NPL * 8;
  const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 3);
  const int j = threadIdx.x & 7;
  const bool valid = row < T;
  float m = 0.0f;
  if (valid) {
    float x[NPL];
    gather_row<NPL>(tokens, row, eq, es, vocab, sqrt_d, j, x, err);
    float* hr = h + (int64_t)row * D;
#pragma unroll
    for (int i = 0; i < NPL; i++) hr[8 * i + j] = x[i];
    sg_rmsnorm8<NPL>(x, w, j, eps);
    if (xn) {
      float* yr = xn + (int64_t)row * D;
#pragma unroll
      for (int i = 0; i < NPL; i++) yr[8 * i + j] = x[i];
    }
#pragma unroll
    for (int i = 0; i < NPL; i++) m = fmaxf(m, fabsf(x[i]));
  }
  if (amax) {
    m = sg_max8(m);
    const int r0 = blockIdx.x * kRowsPerBlock;
    sg_block_seq_max<kThreads>(m, valid && j == 0, row, r0, min(r0 + kRowsPerBlock, T) - 1, row_seq, amax);
  }
}

template <int NPL>
__global__ __launch_bounds__(kThreads) void k_embed_only(const int32_t* __restrict__ tokens, int T,
                                                         const int8_t* __restrict__ eq, const float* __restrict__ es,
                                                         int vocab, float sqrt_d, float* __restrict__ h,
                                                         int32_t* __restrict__ err) {
  constexpr int D = NPL * 8;
  const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 3);
  const int j = threadIdx.x & 7;
  if (row >= T) return;
  float x[NPL];
  gather_row<NPL>(tokens, row, eq, es, vocab, sqrt_d, j, x, err);
  float* hr = h + (int64_t)row * D;
#pragma unroll
  for (int i = 0; i < NPL; i++) hr[8 * i + j] = x[i];
}

// -------------------------------------------------------------- quantize --

// Four codes as int8 (one 4-byte store).
__device__ __forceinline__ void store_codes4(int8_t* p, const float (&c)[4]) {
  uint32_t u = 0;
#pragma unroll
  for (int t = 0; t < 4; t++) u |= (uint32_t)(uint8_t)(int8_t)(int)c[t] << (8 * t);
  *reinterpret_cast<uint32_t*>(p) = u;
}

// quantize.go:29-103 with the tensor max replaced by the per-sequence max
// gathered into amax (one reference call quantizes one sequence):
// scale = m/127 (fp32), inv = 1/scale (fp32),
// q = clamp(round_half_away(float64(x)*float64(inv)), +-127) (sg_quant_code);
// m == 0 -> scale 1, q 0.
// One row per wave (4 rows per workgroup): the row's scale and reciprocal are
// computed once, then the wave walks the row in coalesced float4 slots.  The
// codes go to the block-major GEMM operand qb [cols/32][a_rows][32] (qb !=
// null) or row-major to qi [rows][cols].
__global__ __launch_bounds__(kThreads) void k_quantize(const float* __restrict__ x, int ldx, int rows, int cols,
                                                       const int32_t* __restrict__ row_seq,
                                                       const float* __restrict__ amax, int8_t* __restrict__ qb,
                                                       int a_rows, int8_t* __restrict__ qi,
                                                       float* __restrict__ row_scale) {
  const int row = blockIdx.x * (kThreads / SG_WAVE) + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const float m = amax[row_seq[row]];
  float scale = 1.0f, inv = 0.0f;
  if (m != 0.0f) {
    scale = m / 127.0f;
    inv = 1.0f / scale;
  }
  if (lane == 0) row_scale[row] = scale;
  const float* xr = x + (int64_t)row * ldx;
  for (int c4 = lane; c4 < (cols >> 2); c4 += SG_WAVE) {
    const f32x4_t v = *reinterpret_cast<const f32x4_t*>(xr + 4 * c4);
    float qv[4];
#pragma unroll
    for (int t = 0; t < 4; t++) qv[t] = sg_quant_code(v[t], inv);  // m == 0: inv == 0 gives 0
    const int k = 4 * c4;
    store_codes4(qb ? qb + ((int64_t)(k >> 5) * a_rows + row) * 32 + (k & 31) : qi + (int64_t)row * cols + k, qv);
  }
}

// The next GEMM's operand straight from the residual stream: xn = RMSNorm(h; w)
// recomputed with the lanes and order k_post_res_norm / k_embed_norm used
// when they folded max|xn| into amax (so every value, and the scale, is the
// one the unfused path quantizes), then quantized as k_quantize does
// (model_int8.go:194-199 / :216-221: RMSNorm, then QuantizeSymmetricINT8 of
// the normed sequence).  Saves writing xn and reading it back.  NB: the
// branch-free codes, for small launches.
template <int NC, bool NB>
__global__ __launch_bounds__(kThreads) void k_norm_quantize(const float* __restrict__ h, const float* __restrict__ w,
                                                            float eps, int T, const int32_t* __restrict__ row_seq,
                                                            const float* __restrict__ amax,
                                                            int8_t* __restrict__ qf, int a_rows,
                                                            float* __restrict__ row_scale) {
  constexpr int D = NC * 32;
  __shared__ __attribute__((aligned(16))) float tiles[kThreads / SG_WAVE][8 * 40];
  const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 3);
  const int j = threadIdx.x & 7, r = (threadIdx.x >> 3) & 7;
  if (row >= T) return;  // whole 8-lane groups: the group reductions stay complete
  // The sequence's maximum first: its two dependent loads then overlap the
  // row's loads instead of following the norm (whose LDS steps they cannot
  // cross).
  const float m = amax[row_seq[row]];
  f32x4_t x[NC];
  const f32x4_t* hr = reinterpret_cast<const f32x4_t*>(h + (int64_t)row * D) + j;
#pragma unroll
  // Non-temporal: h is next read after the following GEMMs, and L2 is better
  // left to the operands they re-read (two sequence groups share it).
  for (int c = 0; c < NC; c++) x[c] = __builtin_nontemporal_load(&hr[8 * c]);
  sg_rmsnorm8_f4<NC>(x, w, tiles[threadIdx.x / SG_WAVE], r, j, eps);
  float scale = 1.0f, inv = 0.0f;
  if (m != 0.0f) {
    scale = m / 127.0f;
    inv = 1.0f / scale;
  }
  if (j == 0) row_scale[row] = scale;
  // chunk c is K-block c; lane j holds its elements 4j..4j+3
  int8_t* qr = qf + (int64_t)row * 32 + 4 * j;
#pragma unroll
  for (int c = 0; c < NC; c++) {
    float cv[4];
#pragma unroll
    for (int t = 0; t < 4; t++) cv[t] = NB ? sg_quant_code_nb(x[c][t], inv) : sg_quant_code(x[c][t], inv);
    store_codes4(qr + (int64_t)c * a_rows * 32, cv);
  }
}

// The GEMM-operand form of k_quantize on the float4 row layout: an 8-lane
// group per row, lane j handling elements 32c + 4j .. + 3 of every chunk c
// (chunk c is K-block c), so a wave's stores cover 8 consecutive rows' 64-byte
// block pieces: 512 contiguous bytes per instruction.  NB: the branch-free
// codes, for small launches (latency-bound rather than bandwidth-bound).
template <int NC, bool NB>
__global__ __launch_bounds__(kThreads) void k_quantize_blocked(const float* __restrict__ x, int ldx, int rows,
                                                               const int32_t* __restrict__ row_seq,
                                                               const float* __restrict__ amax,
                                                               int8_t* __restrict__ qf, int a_rows,
                                                               float* __restrict__ row_scale) {
  const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 3);
  const int j = threadIdx.x & 7;
  if (row >= rows) return;
  const float m = amax[row_seq[row]];
  float scale = 1.0f, inv = 0.0f;
  if (m != 0.0f) {
    scale = m / 127.0f;
    inv = 1.0f / scale;
  }
  if (j == 0) row_scale[row] = scale;
  const f32x4_t* xr = reinterpret_cast<const f32x4_t*>(x + (int64_t)row * ldx) + j;
  f32x4_t v[NC];  // every load in flight before the first store; last use of x: non-temporal
#pragma unroll
  for (int c = 0; c < NC; c++) v[c] = __builtin_nontemporal_load(&xr[8 * c]);
  int8_t* qr = qf + (int64_t)row * 32 + 4 * j;
#pragma unroll
  for (int c = 0; c < NC; c++) {
    float cv[4];
#pragma unroll
    for (int t = 0; t < 4; t++) cv[t] = NB ? sg_quant_code_nb(v[c][t], inv) : sg_quant_code(v[c][t], inv);
    store_codes4(qr + (int64_t)c * a_rows * 32, cv);
  }
}

__global__ void k_seq_scales(const float* __restrict__ amax, int n, float* __restrict__ out) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float m = amax[i];
  out[i] = m == 0.0f ? 1.0f : m / 127.0f;
}

// --------------------------------------------------------------- RMSNorm --

template <int NPL>
__global__ __launch_bounds__(kThreads) void k_rmsnorm(float* dst, const float* src, const float* __restrict__ w,
                                                      int rows, float eps, const int32_t* __restrict__ row_seq,
                                                      float* __restrict__ amax) {
  constexpr int D = NPL * 8;
  const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 3);
  const int j = threadIdx.x & 7;
  const bool valid = row < rows;
  float m = 0.0f;
  if (valid) {
    float x[NPL];
    const float* sr = src + (int64_t)row * D;
#pragma unroll
    for (int i = 0; i < NPL; i++) x[i] = sr[8 * i + j];
    sg_rmsnorm8<NPL>(x, w, j, eps);
    float* dr = dst + (int64_t)row * D;
#pragma unroll
    for (int i = 0; i < NPL; i++) {
      dr[8 * i + j] = x[i];
      m = fmaxf(m, fabsf(x[i]));
    }
  }
  if (amax) {
    m = sg_max8(m);
    const int r0 = blockIdx.x * kRowsPerBlock;
    sg_block_seq_max<kThreads>(m, valid && j == 0, row, r0, min(r0 + kRowsPerBlock, rows) - 1, row_seq, amax);
  }
}

// h = RMSNorm(o; w_post) + h (model_int8.go:203-210 / :225-232), then
// xn = RMSNorm(h; w_next) -- the next pre-norm (:194/:216) or output_norm (:236).
// Float4 row layout (sg_post_res_norm_row): NC chunks of 32 elements per row.
template <int NC>
__global__ __launch_bounds__(kThreads) void k_post_res_norm(const float* __restrict__ o, float* __restrict__ h,
                                                            const float* __restrict__ w_post,
                                                            const float* __restrict__ w_next, float eps, int T,
                                                            float* __restrict__ xn,
                                                            const int32_t* __restrict__ row_seq,
                                                            float* __restrict__ amax) {
  constexpr int D = NC * 32;
  __shared__ __attribute__((aligned(16))) float tiles[kThreads / SG_WAVE][8 * 40];
  const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 3);
  const int j = threadIdx.x & 7, r = (threadIdx.x >> 3) & 7;
  const bool valid = row < T;
  float m = 0.0f;
  if (valid)
    m = sg_post_res_norm_row<NC>(o + (int64_t)row * D, h + (int64_t)row * D, w_post, w_next, eps,
                                 xn ? xn + (int64_t)row * D : nullptr, tiles[threadIdx.x / SG_WAVE], r, j);
  if (amax) {
    m = sg_max8(m);
    const int r0 = blockIdx.x * kRowsPerBlock;
    sg_block_seq_max<kThreads>(m, valid && j == 0, row, r0, min(r0 + kRowsPerBlock, T) - 1, row_seq, amax);
  }
}

// k_post_res_norm followed by the next GEMM's operand, in one launch, for
// batches in which every sequence's rows lie inside one workgroup's
// kRowsPerBlock rows (the caller checks; short sequences, the serving case).
// Each sequence's max|xn| is then complete inside the workgroup, so xn --
// still in the lanes that formed it -- is quantized with it right away, as
// k_norm_quantize would quantize the xn it recomputes from h: the same values,
// scale, reciprocal and codes (quantize.go:29-103 per sequence), into the
// block-major operand q8 [D/32][a_rows][32] and row_scale.  The sequences'
// maxima also go to amax, as k_post_res_norm leaves them.
template <int NC>
__global__ __launch_bounds__(kThreads) void k_post_res_norm_q(const float* __restrict__ o, float* __restrict__ h,
                                                              const float* __restrict__ w_post,
                                                              const float* __restrict__ w_next, float eps, int T,
                                                              const int32_t* __restrict__ row_seq,
                                                              float* __restrict__ amax, int8_t* __restrict__ q8,
                                                              int a_rows, float* __restrict__ row_scale) {
  constexpr int D = NC * 32;
  __shared__ __attribute__((aligned(16))) float tiles[kThreads / SG_WAVE][8 * 40];
  __shared__ float rmax[kRowsPerBlock];
  __shared__ int rseq[kRowsPerBlock];
  const int rl = threadIdx.x >> 3, row = blockIdx.x * kRowsPerBlock + rl;
  const int j = threadIdx.x & 7, r = rl & 7;
  const bool valid = row < T;
  // The row's sequence now: its load overlaps the row loads instead of
  // following the norms.
  const int sq = valid ? row_seq[row] : -1;
  f32x4_t x[NC];
  float m = 0.0f;
  if (valid) {
    f32x4_t hv[NC];
    const f32x4_t* op = reinterpret_cast<const f32x4_t*>(o + (int64_t)row * D) + j;
    const f32x4_t* hp = reinterpret_cast<const f32x4_t*>(h + (int64_t)row * D) + j;
#pragma unroll
    for (int c = 0; c < NC; c++) x[c] = __builtin_nontemporal_load(&op[8 * c]);
#pragma unroll
    for (int c = 0; c < NC; c++) hv[c] = __builtin_nontemporal_load(&hp[8 * c]);
    m = sg_post_res_norm_f4<NC>(x, hv, h + (int64_t)row * D, w_post, w_next, eps, nullptr,
                                tiles[threadIdx.x / SG_WAVE], r, j);
  }
  m = sg_max8(m);
  if (j == 0) {
    rmax[rl] = m;  // 0 for rows past T
    rseq[rl] = sq;
  }
  __syncthreads();
  if (!valid) return;
  // The row's sequence maximum over this workgroup's rows (all of them).
  float sm = 0.0f;
  for (int i = 0; i < kRowsPerBlock; i++) sm = rseq[i] == sq ? fmaxf(sm, rmax[i]) : sm;
  const bool first = rl == 0 || rseq[rl - 1] != sq;
  if (amax && first && j == 0) sg_atomic_max_nonneg(amax + sq, sm);
  float scale = 1.0f, inv = 0.0f;
  if (sm != 0.0f) {
    scale = sm / 127.0f;
    inv = 1.0f / scale;
  }
  if (j == 0) row_scale[row] = scale;
  int8_t* qr = q8 + (int64_t)row * 32 + 4 * j;
#pragma unroll
  for (int c = 0; c < NC; c++) {
    float cv[4];
#pragma unroll
    for (int t = 0; t < 4; t++) cv[t] = sg_quant_code_nb(x[c][t], inv);
    store_codes4(qr + (int64_t)c * a_rows * 32, cv);
  }
}

// -------------------------------------------------------- QK-norm + RoPE --

// Per (token, head) 8-lane group: RMSNorm over head_dim=256 with
// attn_q_norm/attn_k_norm (model_int8.go:374-440), then the cached NeoX
// rotation of pairs (i, i+128) at position p (rope_cache.go:85-104):
// x0' = x0*c - x1*s, x1' = x0*s + x1*c, every product rounded.  Element
// 8i+j and its partner 8(i+16)+j live in the same lane.
__global__ __launch_bounds__(kThreads) void k_qknorm_rope(float* __restrict__ q, int ldq, float* __restrict__ k,
                                                          int ldk, const float* __restrict__ qw,
                                                          const float* __restrict__ kw, int H, int HKV, int T,
                                                          const int32_t* __restrict__ row_pos,
                                                          const float* __restrict__ cos_t,
                                                          const float* __restrict__ sin_t, float eps,
                                                          _Float16* __restrict__ qs_h, _Float16* __restrict__ qs_l,
                                                          int ldqs, _Float16* __restrict__ ks_h,
                                                          _Float16* __restrict__ ks_l, int ldks) {
  constexpr int NPL = 32, HALF = 128;
  const int g = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 3);
  const int j = threadIdx.x & 7;
  const int per = H + HKV;
  if (g >= T * per) return;
  const int t = g / per, hh = g % per;
  float* p;
  const float* w;
  if (hh < H) {
    p = q + (int64_t)t * ldq + hh * 256;
    w = qw;
  } else {
    p = k + (int64_t)t * ldk + (hh - H) * 256;
    w = kw;
  }
  float x[NPL];
#pragma unroll
  for (int i = 0; i < NPL; i++) x[i] = p[8 * i + j];
  if (w) sg_rmsnorm8<NPL>(x, w, j, eps);
  const int pos = row_pos[t];
  const float* cr = cos_t + (int64_t)pos * HALF;
  const float* sr = sin_t + (int64_t)pos * HALF;
#pragma unroll
  for (int i = 0; i < NPL / 2; i++) {
    const int e = 8 * i + j;
    const float c = cr[e], s = sr[e];
    const float v0 = x[i], v1 = x[i + NPL / 2];
    const float a = v0 * c, b = v1 * s, cc = v0 * s, dd = v1 * c;
    x[i] = a - b;
    x[i + NPL / 2] = cc + dd;
  }
  if (!qs_h) {
#pragma unroll
    for (int i = 0; i < NPL; i++) p[8 * i + j] = x[i];
    return;
  }
  // Attention operands: hi/lo fp16 of x * kAttnQKScale.
  _Float16 *dh, *dl;
  if (hh < H) {
    dh = qs_h + (int64_t)t * ldqs + hh * 256;
    dl = qs_l + (int64_t)t * ldqs + hh * 256;
  } else {
    dh = ks_h + (int64_t)t * ldks + (hh - H) * 256;
    dl = ks_l + (int64_t)t * ldks + (hh - H) * 256;
  }
#pragma unroll
  for (int i = 0; i < NPL; i++) {
    const hl16 sp = split_f16(x[i] * sgk::kAttnQKScale);
    dh[8 * i + j] = sp.hi;
    dl[8 * i + j] = sp.lo;
  }
}

// The same per-(token, head) arithmetic as k_qknorm_rope, writing the split
// attention operands, in the float4 row layout (sg_rmsnorm8_f4): lane j of
// the row's 8-lane group holds elements 32c + 4j .. 32c + 4j + 3, so loads
// are 128 contiguous bytes per row and the RoPE partner e + 128 of element e
// (chunk c + 4) sits in the same lane and slot.  Stores are 8-byte half4 hi
// and lo pieces, 64 contiguous bytes per row and chunk.
__global__ __launch_bounds__(kThreads) void k_qknorm_rope_split(
    const float* __restrict__ q, int ldq, const float* __restrict__ k, int ldk, const float* __restrict__ qw,
    const float* __restrict__ kw, int H, int HKV, int T, const int32_t* __restrict__ row_pos,
    const float* __restrict__ cos_t, const float* __restrict__ sin_t, float eps, _Float16* __restrict__ qs_h,
    _Float16* __restrict__ qs_l, int ldqs, _Float16* __restrict__ ks_h, _Float16* __restrict__ ks_l, int ldks) {
  static_assert(kThreads == sgd::kKvThreads && kRowsPerBlock == sgd::kKvRows, "one 8-lane group per row");
  __shared__ __attribute__((aligned(16))) float tiles[kThreads / SG_WAVE][8 * 40];
  const int64_t g = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 3);
  sgd::qk_split_group(g, threadIdx.x & 7, (threadIdx.x >> 3) & 7, tiles[threadIdx.x / SG_WAVE], q, ldq, k, ldk, qw,
                      kw, H, HKV, T, row_pos, cos_t, sin_t, eps, qs_h, qs_l, ldqs, ks_h, ks_l, ldks);
}

// ------------------------------------------------------------ GELU * up --

// GELUQuickSIMD (activation.go:47-95) then VecMulF32 (matmul.go:238-259):
// g = geluquick(gate) * up over kGeluRows rows per workgroup (the float4
// slots of those rows are dealt to the threads in turn), plus the sequences'
// max|g|.  A workgroup inside one sequence folds its maximum with one atomic;
// one straddling two sequences folds each row's maximum separately.
constexpr int kGeluRows = 8;
__global__ __launch_bounds__(kThreads) void k_gelu_mul(float* __restrict__ g, int ldd, const float* __restrict__ gate,
                                                       int ldg, const float* __restrict__ up, int ldu, int rows,
                                                       int cols, const int32_t* __restrict__ row_seq,
                                                       float* __restrict__ amax) {
  const int r0 = blockIdx.x * kGeluRows;
  const int nr = min(kGeluRows, rows - r0);
  const int c4n = cols >> 2;
  const bool one_seq = amax && row_seq[r0] == row_seq[r0 + nr - 1];
  float m = 0.0f;
  for (int idx = threadIdx.x; idx < nr * c4n; idx += kThreads) {
    const int row = r0 + idx / c4n, c4 = idx % c4n;
    const f32x4_t a = *reinterpret_cast<const f32x4_t*>(gate + (int64_t)row * ldg + 4 * c4);
    const f32x4_t b = *reinterpret_cast<const f32x4_t*>(up + (int64_t)row * ldu + 4 * c4);
    f32x4_t r;
    float mr = 0.0f;
#pragma unroll
    for (int t = 0; t < 4; t++) {
      r[t] = sg_gelu_quick(a[t]) * b[t];
      mr = fmaxf(mr, fabsf(r[t]));
    }
    *reinterpret_cast<f32x4_t*>(g + (int64_t)row * ldd + 4 * c4) = r;
    if (one_seq)
      m = fmaxf(m, mr);
    else if (amax)
      sg_atomic_max_nonneg(amax + row_seq[row], mr);
  }
  if (one_seq) sg_block_seq_max<kThreads>(m, false, r0, r0, r0 + nr - 1, row_seq, amax);
}


// Per-row max|x| folded into the row's sequence maximum (absMaxScalar,
// quantize.go:80-90, over a whole sequence).
__global__ __launch_bounds__(kThreads) void k_absmax_rows(const float* __restrict__ x, int ldx, int cols,
                                                          const int32_t* __restrict__ row_seq,
                                                          float* __restrict__ amax) {
  __shared__ float red[kThreads / SG_WAVE];
  const float* xr = x + (int64_t)blockIdx.x * ldx;
  float m = 0.0f;
  for (int c = threadIdx.x; c < cols; c += kThreads) m = fmaxf(m, fabsf(xr[c]));
  m = sg_wave_max(m);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    float mm = red[0];
    for (int i = 1; i < kThreads / SG_WAVE; i++) mm = fmaxf(mm, red[i]);
    sg_atomic_max_nonneg(amax + row_seq[blockIdx.x], mm);
  }
}

// ---------------------------------------------------------- pool and L2 --

// MeanPoolingPartial (attention.go:423-445): per column, serial sum over the
// sequence's rows then * (1/float32(S)); l2Normalize (runtime/model.go:808-820):
// serial sum of squares, norm = float32(sqrt(float64(ss))), v /= norm.
// MeanPoolingPartial (attention.go:423-445): p[c] = (sum_s x[s][c]) * (1/S),
// the sum running over s in order for each column.  A workgroup owns 64
// columns of one sequence; 64-row slabs are staged through LDS by all 256
// threads (coalesced, many loads in flight), then 64 threads extend their
// column's serial sum.  Writes the unnormalized means to out.
constexpr int kPoolCols = 64, kPoolRows = 64;
__global__ __launch_bounds__(kThreads) void k_pool_mean(float* __restrict__ out, const float* __restrict__ x, int ldx,
                                                        int out_dim, const int32_t* __restrict__ seq_off) {
  __shared__ float tile[kPoolRows][kPoolCols + 1];
  const int sq = blockIdx.x, c0 = blockIdx.y * kPoolCols;
  const int r0 = seq_off[sq], S = seq_off[sq + 1] - r0;
  const int lc = threadIdx.x % kPoolCols, rq = threadIdx.x / kPoolCols;  // rq: 0..3
  const int c = min(c0 + lc, out_dim - 1);
  float acc = 0.0f;
  for (int s0 = 0; s0 < S; s0 += kPoolRows) {
    const int n = min(kPoolRows, S - s0);
#pragma unroll
    for (int i = 0; i < kPoolRows / 4; i++) {
      const int rr = rq * (kPoolRows / 4) + i;
      tile[rr][lc] = x[(int64_t)(r0 + s0 + min(rr, n - 1)) * ldx + c];
    }
    __syncthreads();
    if (rq == 0)
      for (int i = 0; i < n; i++) acc = acc + tile[i][lc];
    __syncthreads();
  }
  if (rq == 0 && c0 + lc < out_dim) out[(int64_t)sq * out_dim + c0 + lc] = acc * (1.0f / (float)S);
}

// l2Normalize (runtime/model.go:808-820) of each pooled row in place: serial
// fp32 sum of squares, n = sqrt, v / n; an all-zero row is left as is.  The
// row is staged in LDS with coalesced loads so the one thread that runs the
// serial sum reads LDS, not a chain of global loads.
constexpr int kL2MaxDim = 1024;
__global__ __launch_bounds__(kThreads) void k_l2_rows(float* __restrict__ out, int out_dim) {
  __shared__ float row[kL2MaxDim];
  __shared__ float nrm;
  float* v = out + (int64_t)blockIdx.x * out_dim;
  for (int c = threadIdx.x; c < out_dim; c += kThreads) row[c] = v[c];
  __syncthreads();
  if (threadIdx.x == 0) {
    float ss = 0.0f;
    for (int c = 0; c < out_dim; c++) {
      const float t = row[c] * row[c];
      ss = ss + t;
    }
    nrm = ss == 0.0f ? 0.0f : sg_sqrt(ss);
  }
  __syncthreads();
  const float n = nrm;
  if (n != 0.0f)
    for (int c = threadIdx.x; c < out_dim; c += kThreads) v[c] = row[c] / n;
}

// Streaming yardsticks for the bandwidth-bound kernels (sg_hbm_probe): one
// float4 per lane, no reuse.  c = a + b (8 B read, 4 B written per element),
// and the quantizers' I/O: 4 B read, one int8 code written, q = the code of
// x at reciprocal scale inv (sg_quant_code, exact rounding included).
__global__ __launch_bounds__(256) void k_stream_add(const f32x4_t* __restrict__ a, const f32x4_t* __restrict__ b,
                                                    f32x4_t* __restrict__ c, int64_t n4) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n4) c[i] = a[i] + b[i];
}

__global__ __launch_bounds__(256) void k_stream_quant(const f32x4_t* __restrict__ a, float inv,
                                                      int8_t* __restrict__ q, int64_t n4) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n4) return;
  const f32x4_t v = __builtin_nontemporal_load(&a[i]);
  float cv[4];
#pragma unroll
  for (int t = 0; t < 4; t++) cv[t] = sg_quant_code(v[t], inv);
  store_codes4(q + 4 * i, cv);
}

inline unsigned blocks_for(int64_t n, int per) { return (unsigned)((n + per - 1) / per); }

}  // namespace

namespace sgk {

hipError_t repack_q8_0(const uint8_t* raw, int rows, int cols, int8_t* w8, float* st, int ld, int row_off, int grp,
                       int gstride, hipStream_t s) {
  const int64_t n = (int64_t)rows * (cols / 32);
  if (grp <= 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_repack_q8_0, dim3(blocks_for(n, 256)), dim3(256), 0, s, raw, rows, cols, w8, st, ld, row_off,
                     grp, gstride);
  return hipGetLastError();
}

hipError_t repack_embd(const uint8_t* raw, int vocab, int d, int8_t* q, float* sc, hipStream_t s) {
  const int64_t n = (int64_t)vocab * (d / 32);
  hipLaunchKernelGGL(k_repack_embd, dim3(blocks_for(n, 256)), dim3(256), 0, s, raw, vocab, d, q, sc);
  return hipGetLastError();
}

hipError_t i8_blocked(const int8_t* x, int M, int K, int8_t* y, int a_rows, hipStream_t s) {
  const int64_t n = (int64_t)M * K;
  if (n <= 0) return hipSuccess;
  if (K % 32 || a_rows < M) return hipErrorInvalidValue;
  const bool vec = (reinterpret_cast<uintptr_t>(x) & 15) == 0;
  hipLaunchKernelGGL(k_i8_blocked, dim3(blocks_for(n / 16, 256)), dim3(256), 0, s, x, M, K, y, a_rows, vec);
  return hipGetLastError();
}

hipError_t fill_f32(float* p, float v, int64_t n, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_fill, dim3(blocks_for(n, 256)), dim3(256), 0, s, p, v, n);
  return hipGetLastError();
}

hipError_t fill_i32(int32_t* p, int32_t v, int64_t n, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_fill_i32, dim3(blocks_for(n, 256)), dim3(256), 0, s, p, v, n);
  return hipGetLastError();
}

hipError_t first_bad_token(const int32_t* tokens, int T, int vocab, int32_t* first, hipStream_t s) {
  if (T <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_first_bad_token, dim3(blocks_for(T, 256)), dim3(256), 0, s, tokens, T, vocab, first);
  return hipGetLastError();
}

#define SG_DISPATCH_NPL(n, NPLV, ...)         \
  switch (n) {                                \
    case 256: { constexpr int NPLV = 32; __VA_ARGS__; break; }  \
    case 512: { constexpr int NPLV = 64; __VA_ARGS__; break; }  \
    case 768: { constexpr int NPLV = 96; __VA_ARGS__; break; }  \
    case 1024: { constexpr int NPLV = 128; __VA_ARGS__; break; } \
    case 1152: { constexpr int NPLV = 144; __VA_ARGS__; break; } \
    default: return hipErrorInvalidValue;     \
  }

hipError_t embed_norm(const int32_t* tokens, int T, const int8_t* eq, const float* es, int vocab, int d,
                      float sqrt_d, const float* w, float eps, const int32_t* row_seq, float* h, float* xn,
                      float* amax, int32_t* err, hipStream_t s) {
  if (T <= 0) return hipSuccess;
  SG_DISPATCH_NPL(d, NPL,
                  hipLaunchKernelGGL(k_embed_norm<NPL>, dim3(blocks_for(T, kRowsPerBlock)), dim3(kThreads), 0, s,
                                     tokens, T, eq, es, vocab, sqrt_d, w, eps, row_seq, h, xn, amax, err));
  return hipGetLastError();
}

hipError_t embed_only(const int32_t* tokens, int T, const int8_t* eq, const float* es, int vocab, int d,
                      float sqrt_d, float* h, int32_t* err, hipStream_t s) {
  if (T <= 0) return hipSuccess;
  SG_DISPATCH_NPL(d, NPL,
                  hipLaunchKernelGGL(k_embed_only<NPL>, dim3(blocks_for(T, kRowsPerBlock)), dim3(kThreads), 0, s,
                                     tokens, T, eq, es, vocab, sqrt_d, h, err));
  return hipGetLastError();
}

hipError_t quantize(const float* x, int ldx, int rows, int cols, const int32_t* row_seq, const float* amax,
                    int8_t* q8, int a_rows, int8_t* i8, float* row_scale, hipStream_t s) {
  if (rows <= 0) return hipSuccess;
  if (cols % 4 || ldx % 4 || (!q8 && !i8)) return hipErrorInvalidValue;
  if (q8 && (cols % 32 || a_rows < rows)) return hipErrorInvalidValue;
  if (q8 && (reinterpret_cast<uintptr_t>(x) & 15) == 0) {
    const unsigned nb = blocks_for(rows, kRowsPerBlock);
    // At most one round of workgroups: latency-bound, the branch-free codes.
    const bool small = rows < kQuantNbRows;
    switch (cols) {  // the widths the forward quantizes: attention output, hidden, FFN
#define SG_QB(C)                                                                                                   \
  case C:                                                                                                          \
    if (small)                                                                                                     \
      hipLaunchKernelGGL((k_quantize_blocked<C / 32, true>), dim3(nb), dim3(kThreads), 0, s, x, ldx, rows, row_seq, \
                         amax, q8, a_rows, row_scale);                                                             \
    else                                                                                                           \
      hipLaunchKernelGGL((k_quantize_blocked<C / 32, false>), dim3(nb), dim3(kThreads), 0, s, x, ldx, rows,        \
                         row_seq, amax, q8, a_rows, row_scale);                                                    \
    return hipGetLastError();
      SG_QB(256) SG_QB(512) SG_QB(768) SG_QB(1024) SG_QB(1152)
#undef SG_QB
      default:
        break;
    }
  }
  hipLaunchKernelGGL(k_quantize, dim3(blocks_for(rows, kThreads / SG_WAVE)), dim3(kThreads), 0, s, x, ldx, rows, cols,
                     row_seq, amax, q8, a_rows, q8 ? nullptr : i8, row_scale);
  return hipGetLastError();
}

hipError_t norm_quantize(const float* h, const float* w, float eps, int T, int d, const int32_t* row_seq,
                         const float* amax, int8_t* q8, int a_rows, float* row_scale, hipStream_t s) {
  if (T <= 0) return hipSuccess;
  if (a_rows < T) return hipErrorInvalidValue;
  if (T < kQuantNbRows) {
    SG_DISPATCH_NPL(d, NPL,
                    hipLaunchKernelGGL((k_norm_quantize<NPL / 4, true>), dim3(blocks_for(T, kRowsPerBlock)),
                                       dim3(kThreads), 0, s, h, w, eps, T, row_seq, amax, q8, a_rows, row_scale));
  } else {
    SG_DISPATCH_NPL(d, NPL,
                    hipLaunchKernelGGL((k_norm_quantize<NPL / 4, false>), dim3(blocks_for(T, kRowsPerBlock)),
                                       dim3(kThreads), 0, s, h, w, eps, T, row_seq, amax, q8, a_rows, row_scale));
  }
  return hipGetLastError();
}

hipError_t seq_scales(const float* amax, int n_seq, float* out, hipStream_t s) {
  hipLaunchKernelGGL(k_seq_scales, dim3(blocks_for(n_seq, 256)), dim3(256), 0, s, amax, n_seq, out);
  return hipGetLastError();
}

hipError_t rmsnorm(float* dst, const float* src, const float* w, int rows, int n, float eps, const int32_t* row_seq,
                   float* amax, hipStream_t s) {
  if (rows <= 0) return hipSuccess;
  SG_DISPATCH_NPL(n, NPL,
                  hipLaunchKernelGGL(k_rmsnorm<NPL>, dim3(blocks_for(rows, kRowsPerBlock)), dim3(kThreads), 0, s,
                                     dst, src, w, rows, eps, row_seq, amax));
  return hipGetLastError();
}

hipError_t qknorm_rope(float* q, int ldq, float* k, int ldk, const float* qw, const float* kw, int H, int HKV, int T,
                       const int32_t* row_pos, const float* cos_t, const float* sin_t, float eps, _Float16* qs_h,
                       _Float16* qs_l, int ldqs, _Float16* ks_h, _Float16* ks_l, int ldks, hipStream_t s) {
  if (T <= 0) return hipSuccess;
  const bool split = ks_h != nullptr;
  if (split && (!ks_l || (H > 0 && (!qs_h || !qs_l)))) return hipErrorInvalidValue;
  const int64_t groups = (int64_t)T * (H + HKV);
  if (groups <= 0) return hipSuccess;
  if (split) {
    if ((ldks & 7) || (ldk & 3) || (reinterpret_cast<uintptr_t>(k) & 15) ||
        (H > 0 && ((ldqs & 7) || (ldq & 3) || (reinterpret_cast<uintptr_t>(q) & 15))))
      return hipErrorInvalidValue;  // float4 loads of every head row
    hipLaunchKernelGGL(k_qknorm_rope_split, dim3(blocks_for(groups, kRowsPerBlock)), dim3(kThreads), 0, s, q, ldq, k,
                       ldk, qw, kw, H, HKV, T, row_pos, cos_t, sin_t, eps, qs_h, qs_l, ldqs, ks_h, ks_l, ldks);
  } else {
    hipLaunchKernelGGL(k_qknorm_rope, dim3(blocks_for(groups, kRowsPerBlock)), dim3(kThreads), 0, s, q, ldq, k, ldk,
                       qw, kw, H, HKV, T, row_pos, cos_t, sin_t, eps, nullptr, nullptr, 0, nullptr, nullptr, 0);
  }
  return hipGetLastError();
}

hipError_t post_res_norm(const float* o, float* h, const float* w_post, const float* w_next, float eps, int T, int d,
                         float* xn, const int32_t* row_seq, float* amax, hipStream_t s) {
  if (T <= 0) return hipSuccess;
  SG_DISPATCH_NPL(d, NPL,
                  hipLaunchKernelGGL(k_post_res_norm<NPL / 4>, dim3(blocks_for(T, kRowsPerBlock)), dim3(kThreads),
                                     0, s, o, h, w_post, w_next, eps, T, xn, row_seq, amax));
  return hipGetLastError();
}

hipError_t post_res_norm_quantize(const float* o, float* h, const float* w_post, const float* w_next, float eps,
                                  int T, int d, const int32_t* row_seq, float* amax, int8_t* q8, int a_rows,
                                  float* row_scale, hipStream_t s) {
  if (T <= 0) return hipSuccess;
  if (!q8 || !row_scale || !w_next || a_rows < T) return hipErrorInvalidValue;
  SG_DISPATCH_NPL(d, NPL,
                  hipLaunchKernelGGL(k_post_res_norm_q<NPL / 4>, dim3(blocks_for(T, kRowsPerBlock)), dim3(kThreads),
                                     0, s, o, h, w_post, w_next, eps, T, row_seq, amax, q8, a_rows, row_scale));
  return hipGetLastError();
}

hipError_t gelu_mul(float* g, int ldd, const float* gate, int ldg, const float* up, int ldu, int rows, int cols,
                    const int32_t* row_seq, float* amax, hipStream_t s) {
  if (rows <= 0) return hipSuccess;
  if (cols % 4 || ldd % 4 || ldg % 4 || ldu % 4) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_gelu_mul, dim3(blocks_for(rows, kGeluRows)), dim3(kThreads), 0, s, g, ldd, gate, ldg, up, ldu,
                     rows, cols, row_seq, amax);
  return hipGetLastError();
}

hipError_t pool_l2(float* out, const float* x, int ldx, int out_dim, const int32_t* seq_off, int n_seq,
                   hipStream_t s) {
  if (n_seq <= 0) return hipSuccess;
  if (out_dim > kL2MaxDim) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_pool_mean, dim3(n_seq, blocks_for(out_dim, kPoolCols)), dim3(kThreads), 0, s, out, x, ldx,
                     out_dim, seq_off);
  hipLaunchKernelGGL(k_l2_rows, dim3(n_seq), dim3(kThreads), 0, s, out, out_dim);
  return hipGetLastError();
}

hipError_t stream_probe(int kind, const float* a, const float* b, void* c, int64_t n, hipStream_t s) {
  if (n <= 0 || n % 4) return hipErrorInvalidValue;
  const int64_t n4 = n / 4;
  if (kind == 0)
    hipLaunchKernelGGL(k_stream_add, dim3(blocks_for(n4, 256)), dim3(256), 0, s,
                       reinterpret_cast<const f32x4_t*>(a), reinterpret_cast<const f32x4_t*>(b),
                       reinterpret_cast<f32x4_t*>(c), n4);
  else if (kind == 1)
    hipLaunchKernelGGL(k_stream_quant, dim3(blocks_for(n4, 256)), dim3(256), 0, s,
                       reinterpret_cast<const f32x4_t*>(a), 12.7f, static_cast<int8_t*>(c), n4);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t absmax_rows(const float* x, int ldx, int rows, int cols, const int32_t* row_seq, float* amax,
                       hipStream_t s) {
  if (rows <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_absmax_rows, dim3(rows), dim3(kThreads), 0, s, x, ldx, cols, row_seq, amax);
  return hipGetLastError();
}

}  // namespace sgk
