// sg_kernels.h -- host-side launchers for the gfx950 kernels (internal to the
// library; the public surface is include/semantica_gpu.h).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

// One unit of per-sequence work: attention workgroup (sequence, first 32-row
// chunk) or V^T split tile (sequence, first key).
struct sg_item { int32_t seq, c0; };
// Q's QK-norm + RoPE done inside the attention kernel: fp32 q [T][ldq] as the
// QKV GEMM wrote it, attn_q_norm weights (null: no norm) and the RoPE tables
// [pos][128].  A row's position is its index within its sequence (positions
// restart at 0 in every sequence, as the forward's row_pos holds them).
struct sg_attn_qpre {
  const float* q;
  int ldq;
  const float* w;
  const float* cos_t;
  const float* sin_t;
  float eps;
};

// Optional attention epilogue: the attention output quantized per sequence
// into the block-major GEMM operand q8[H*hd/32][a_rows][32] and row_scale
// (quantize's arithmetic on the values written to out), for launches in which
// one workgroup holds every row and head of its sequence (one work item per
// sequence and a single kv head); the caller checks.
struct sg_attn_qout {
  int8_t* q8;
  int a_rows;
  float* row_scale;
};

// Where attention() keeps the scores of the tiles past its register-held ones
// (sequences longer than sgk::kAttnRegKeys keys): per kv head, `total` tiles of
// sgk::kAttnSpillTileBytes at buf (16-byte aligned); sequence i's workgroups
// at tile off[i] + (c0 / sgk::kAttnChunks) * sgk::attention_spill_tiles(S_i).
struct sg_attn_spill {
  float* buf;
  const int32_t* off;
  int total;
};

namespace sgk {

// GEMM operands are block-major int8 [K/32][rows][32]; activation buffers hold
// gemm_pad_rows(M) rows per K-block so that every workgroup tile reads
// allocated memory (rows past M are never stored).
constexpr int kGemmRowPad = 256;
inline int gemm_pad_rows(int M) { return (M + kGemmRowPad - 1) / kGemmRowPad * kGemmRowPad; }

// ---- load-time repack (k_rows.hip) ----
// Raw Q8_0 rows [rows][cols/32][34 B] -> block-major int8 weights
// w8[b][dst(r)][32] (ld rows per block) and fp32 block scales (IEEE
// converter) st[b][dst(r)] (ld per block), dst(r) = row_off + (r / grp) *
// gstride + r % grp (grp = rows, gstride = 0: plain row_off + r).
hipError_t repack_q8_0(const uint8_t* raw, int rows, int cols, int8_t* w8, float* st, int ld, int row_off, int grp,
                       int gstride, hipStream_t s);
// token_embd: int8 values q[v][d] and per-block scales (gguf halving converter) sc[v][d/32].
hipError_t repack_embd(const uint8_t* raw, int vocab, int d, int8_t* q, float* sc, hipStream_t s);
// int8 x[M][K] -> block-major int8 y[K/32][a_rows][32] (the GEMM operand).
hipError_t i8_blocked(const int8_t* x, int M, int K, int8_t* y, int a_rows, hipStream_t s);
hipError_t fill_f32(float* p, float v, int64_t n, hipStream_t s);
hipError_t fill_i32(int32_t* p, int32_t v, int64_t n, hipStream_t s);
// The first row r < T with tokens[r] outside [0, vocab), folded into *first by
// atomicMin (the embedding kernels record theirs the same way).
hipError_t first_bad_token(const int32_t* tokens, int T, int vocab, int32_t* first, hipStream_t s);

// ---- per-row kernels (k_rows.hip) ----
// Embedding gather * sqrt(d) -> h; then RMSNorm(w) -> xn (stored when xn != null) and
// per-sequence max|xn| -> amax.  A token outside [0, vocab) is read as token 0
// and its row folded into *err by atomicMin (*err starts at INT32_MAX).
hipError_t embed_norm(const int32_t* tokens, int T, const int8_t* eq, const float* es, int vocab, int d,
                      float sqrt_d, const float* w, float eps, const int32_t* row_seq, float* h, float* xn,
                      float* amax, int32_t* err, hipStream_t s);
// Per-sequence symmetric quantization of x[rows][cols] (stride ldx) using amax[row_seq[r]].
// Writes the int8 codes block-major q8[cols/32][a_rows][32] (q8 != null, the GEMM
// operand) or row-major i8[rows][cols] (q8 == null), and row_scale[rows].
hipError_t quantize(const float* x, int ldx, int rows, int cols, const int32_t* row_seq, const float* amax,
                    int8_t* q8, int a_rows, int8_t* i8, float* row_scale, hipStream_t s);
// xn = RMSNorm(h; w) recomputed row by row exactly as post_res_norm / embed_norm
// formed it, quantized with amax[row_seq[r]] into the block-major int8 GEMM
// operand q8[d/32][a_rows][32] and row_scale[T] (quantize's arithmetic).
hipError_t norm_quantize(const float* h, const float* w, float eps, int T, int d, const int32_t* row_seq,
                         const float* amax, int8_t* q8, int a_rows, float* row_scale, hipStream_t s);
hipError_t absmax_rows(const float* x, int ldx, int rows, int cols, const int32_t* row_seq, float* amax,
                       hipStream_t s);
hipError_t seq_scales(const float* amax, int n_seq, float* out, hipStream_t s);
// RMSNorm rows in the reference's order; amax (optional) collects per-sequence max|y|.
hipError_t rmsnorm(float* dst, const float* src, const float* w, int rows, int n, float eps,
                   const int32_t* row_seq, float* amax, hipStream_t s);
// QK-norm + RoPE; head_dim 256.  In place (fp32) when ks_h is null, else
// written as the attention operands: hi/lo fp16 of x * kAttnQKScale into
// qs_h/qs_l [T][ldqs] and ks_h/ks_l [T][ldks] (q and k are only read; H = 0
// processes K alone, for attention() with qpre).
hipError_t qknorm_rope(float* q, int ldq, float* k, int ldk, const float* qw, const float* kw, int H, int HKV,
                       int T, const int32_t* row_pos, const float* cos_t, const float* sin_t, float eps,
                       _Float16* qs_h, _Float16* qs_l, int ldqs, _Float16* ks_h, _Float16* ks_l, int ldks,
                       hipStream_t s);
// h = RMSNorm(o; w_post) + h ; xn = RMSNorm(h; w_next) (stored when xn != null) ;
// amax (optional) per sequence of max|xn|.
hipError_t post_res_norm(const float* o, float* h, const float* w_post, const float* w_next, float eps, int T,
                         int d, float* xn, const int32_t* row_seq, float* amax, hipStream_t s);
// Rows per workgroup of the row kernels (post_res_norm, norm_quantize, ...).
constexpr int kRowKernelRows = 32;
// post_res_norm, then xn quantized per sequence into the block-major GEMM
// operand q8[d/32][a_rows][32] and row_scale[T] -- the values, scale and codes
// norm_quantize would produce from the new h -- in one launch.  Valid only when
// every sequence's rows lie inside one block of kRowKernelRows rows
// (off[s] / kRowKernelRows == (off[s+1] - 1) / kRowKernelRows); amax (optional)
// receives the sequences' max|xn| as post_res_norm leaves them.
hipError_t post_res_norm_quantize(const float* o, float* h, const float* w_post, const float* w_next, float eps,
                                  int T, int d, const int32_t* row_seq, float* amax, int8_t* q8, int a_rows,
                                  float* row_scale, hipStream_t s);
// g = geluquick(gate)*up over rows x cols; amax (optional) per sequence of max|g|.
hipError_t gelu_mul(float* g, int ldd, const float* gate, int ldg, const float* up, int ldu, int rows, int cols,
                    const int32_t* row_seq, float* amax, hipStream_t s);
hipError_t pool_l2(float* out, const float* x, int ldx, int out_dim, const int32_t* seq_off, int n_seq,
                   hipStream_t s);
hipError_t embed_only(const int32_t* tokens, int T, const int8_t* eq, const float* es, int vocab, int d,
                      float sqrt_d, float* h, int32_t* err, hipStream_t s);
// Streaming yardsticks over n floats (n % 4 == 0, 16-byte aligned): kind 0
// c = a + b (fp32), kind 1 c = int8 codes of a (b unused).
hipError_t stream_probe(int kind, const float* a, const float* b, void* c, int64_t n, hipStream_t s);
// k_issue_probe<kind> on `blocks` workgroups of 4 waves: sink [blocks * 256]
// floats, clk [blocks * 4 * 2] (per wave: shader cycles, wall-clock ticks).
hipError_t issue_probe(int kind, int blocks, float* sink, long long* clk, int iters, hipStream_t s);

// ---- GEMM (k_gemm.hip) ----
// Y[M][N] = (sum_b float(P_b) * St[b][n]) * row_scale[m] with A int8 [M][K]
// block-major [K/32][a_rows][32] (a_rows >= gemm_pad_rows(M)), W int8 [N][K]
// block-major [K/32][N][32], St [K/32][N].  sums != null additionally dumps
// the exact block sums int32 [M][N][K/32].  cold_weights: W is not expected
// in L2 (the forward, one layer after another), which selects deeper load
// pipelines for small grids; the results are the same either way.
// The V columns [col0, N) of the QKV GEMM written straight as attention's
// V^T operand (hi/lo fp16 in the layout and key order k_kv_prep's V half
// writes: per sequence s at key columns voff[s] ..) instead of fp32 into Y;
// the bits are the same.  Positions past a sequence's end are not written.
struct sg_vt_out {
  _Float16* vt;
  int ldvt;
  int col0;
  const int32_t* row_seq;
  const int32_t* seq_off;
  const int32_t* voff;
};
// Whether gemm_q8 takes an sg_vt_out at M rows (the direct-to-LDS kernels).
bool gemm_writes_vt(int M);
hipError_t gemm_q8(const int8_t* A, int a_rows, const int8_t* W, const float* St, const float* row_scale, float* Y,
                   int32_t* sums, int M, int N, int K, hipStream_t s, bool cold_weights = false,
                   const sg_vt_out* vto = nullptr);
// FFN gate/up GEMM with GELUQuick(gate) * up in the epilogue: W holds 2*Nh rows,
// gate and up interleaved in groups of kGeluGroup (see repack_q8_0's grouping);
// G[M][Nh] is bit-identical to the unfused GEMMs + gelu_mul; amax (optional,
// with row_seq) collects the sequences' max|g|.
hipError_t gemm_q8_gelu(const int8_t* A, int a_rows, const int8_t* W, const float* St, const float* row_scale,
                        float* G, int M, int Nh, int K, const int32_t* row_seq, float* amax, hipStream_t s,
                        bool cold_weights = false);
// gemm_q8 followed by post_res_norm on its output (N = d): o = the GEMM, then
// h = RMSNorm(o; w_post) + h, xn = RMSNorm(h; w_next) (stored when xn !=
// null), amax (optional, with row_seq) per sequence of max|xn|.  For N = 768
// and large M one launch computes whole rows and norms them without storing o
// (o is then left untouched); h, xn and amax are bit-identical either way.
hipError_t gemm_q8_res_norm(const int8_t* A, int a_rows, const int8_t* W, const float* St, const float* row_scale,
                            float* o, int M, int N, int K, float* h, const float* w_post, const float* w_next, float eps,
                            float* xn, const int32_t* row_seq, float* amax, hipStream_t s);
// Whether gemm_q8_res_norm runs as one launch for these arguments.
bool gemm_res_norm_fused(int M, int N, const float* w_post, const float* w_next);
// Gate/up interleaving used by gemm_q8_gelu: source row r of a matrix goes to
// row row_off + (r / 32) * 64 + r % 32 (gate: row_off 0, up: row_off 32).
constexpr int kGeluGroup = 32;

// ---- attention (k_attention.hip) ----
constexpr float kAttnQKScale = 8.0f;  // Q and K are split after scaling by 8 (exact)
constexpr int kAttnChunkRows = 16;    // (head, query) rows per attention chunk (one wave)
constexpr int kAttnChunks = 8;        // chunks per attention workgroup
constexpr int kAttnRegKeys = 512;     // longest sequence whose scores pass 1 keeps in registers
// Columns of V^T a sequence of S keys occupies (whole 32-key tiles).
inline int attn_key_pad(int S) { return (S + 31) / 32 * 32; }
// V fp32 [T][ldv] -> V^T fp16 [HKV*256][ldvt] (sequence s at key column voff[s],
// keys permuted within 32-key tiles, zero past S; the tile at key column c of
// a dim row holds its hi halves at 2c .. 2c+31 and its lo halves at 2c+32 ..
// 2c+63, so ldvt >= 2 * key columns); vtiles: (seq, key0) per 32 keys.
hipError_t v_split_t(const float* v, int ldv, const int32_t* seq_off, const int32_t* voff, const sg_item* vtiles,
                     int n_vtiles, int HKV, _Float16* vt, int ldvt, hipStream_t s);
// qknorm_rope's K-only split (H = 0) and v_split_t in one launch: K and V
// share the row stride ldkv (columns of the QKV output).  n_vtiles = 0: K
// only (V^T written by the QKV GEMM, sg_vt_out).
// Optional Q part of kv_prep: the H query heads' norm (qw), RoPE and hi/lo
// split as well (k_qknorm_rope_split's arithmetic), into qs_h / qs_l
// [T][ldqs], for launches that run the attention on pre-split Q.
struct sg_kv_q {
  const float* q;
  int ldq;
  const float* qw;
  int H;
  _Float16* qs_h;
  _Float16* qs_l;
  int ldqs;
};
hipError_t kv_prep(const float* k, const float* v, int ldkv, const float* kw, int HKV, int T, const int32_t* row_pos,
                   const float* cos_t, const float* sin_t, float eps, _Float16* ks_h, _Float16* ks_l, int ldks,
                   const int32_t* seq_off, const int32_t* voff, const sg_item* vtiles, int n_vtiles, _Float16* vt,
                   int ldvt, hipStream_t s, const sg_kv_q* qpart = nullptr);
// rows x cols of x -> hi/lo fp16 of x*scale (row stride ldo).
hipError_t split_rows(const float* x, int ldx, int rows, int cols, float scale, _Float16* hi, _Float16* lo, int ldo,
                      hipStream_t s);
// out[T][ldo] = attention over the split operands; items: (seq, first chunk)
// per workgroup, chunk c of a sequence = (head c / ceil(S/16), rows 16*(c % ceil(S/16))).
// qpre != null: Q is taken from qpre (fp32, normed and rotated in the kernel
// exactly as qknorm_rope does) and qh/ql/ldq are ignored.  max_len: the
// longest sequence of the launch.  Pass 1's scores stay in registers up to
// kAttnRegKeys keys; a longer sequence keeps the rest in spill (required
// when max_len exceeds kAttnRegKeys).  A sequence gives the same bits
// whatever the launch's max_len.
hipError_t attention(const _Float16* qh, const _Float16* ql, int ldq, const _Float16* kh, const _Float16* kl, int ldk,
                     const _Float16* vt, int ldvt, float* out, int ldo, const int32_t* seq_off,
                     const int32_t* voff, const sg_item* items, int n_items, int H, int HKV, int hd, float scale,
                     float* amax, int max_len, hipStream_t s, const sg_attn_qpre* qpre = nullptr,
                     const sg_attn_qout* qout = nullptr, const sg_attn_spill* spill = nullptr);
// Score tiles a sequence of S keys spills per attention workgroup (one 32-key
// tile of one workgroup: kAttnSpillTileBytes).
constexpr int kAttnSpillTileBytes = kAttnChunks * 2048;
inline int attention_spill_tiles(int S) {
  const int t = (S + 31) / 32 - kAttnRegKeys / 32;
  return t > 0 ? t : 0;
}

// ---- attention in the reference's float32 order (k_attn_exact.hip) ----
// out[T][ldo] (head h at h*hd) from q[T][ldq], k/v[T][ldkv] (kv head h / (H/HKV)),
// every operation in attention.go's order; P: attention_exact_scratch bytes;
// amax (optional) collects each sequence's max|out| (atomic max, >= 0).
// hd must be 256, max_len <= 2048, q/k rows 16-byte aligned; n_seq * H <= 65535.
size_t attention_exact_scratch(int T, int H, int max_len);
hipError_t attention_exact(const float* q, int ldq, const float* k, const float* v, int ldkv, float* out, int ldo,
                           const int32_t* seq_off, const int32_t* row_seq, int n_seq, int T, int H, int HKV, int hd,
                           float scale, int max_len, float* P, float* amax, hipStream_t s);

// ---- brute-force search (k_search.hip) ----
// Storage modes, the values of brute.QuantizationMode (search/brute/quant.go:8-15).
constexpr int kBfF32 = 0, kBfI8 = 1, kBfI16 = 2;
// Index layout: grp [dim/8][N][8] elements, tail [N][dim%8] elements.
// Rows row0..row0+n of the index from float vectors src[n][ld]: normalized
// (builder.go:131-141) when `normalize`, then quantized (quant.go:17-41).
hipError_t bf_build(int mode, const float* src, int64_t ld, int n, int dim, int row0, int N, void* grp, void* tail,
                    bool normalize, hipStream_t s);
// builder.go:131-141 in place on n rows [n][dim].
hipError_t bf_normalize(float* x, int n, int dim, hipStream_t s);
// Stored rows (row-major [n][dim], as serialized) -> rows row0.. of the layout.
hipError_t bf_relayout(int mode, const void* rows, int n, int dim, int row0, int N, void* grp, void* tail,
                       hipStream_t s);
// Rows row0..row0+n of the layout -> row-major [n][dim].
hipError_t bf_unpack(int mode, const void* grp, const void* tail, int row0, int n, int dim, int N, void* rows,
                     hipStream_t s);
// scores[q][ld_scores] for nq normalized queries [nq][dim] against all N vectors.
hipError_t bf_score(int mode, const void* grp, const void* tail, int N, int dim, const float* queries, int nq,
                    float* scores, int64_t ld_scores, hipStream_t s);
// The reference's top-k of every query's scores (k <= N): out_idx/out_dist [nq][k]
// in arbitrary order (positions, not ids).  state: int32 [nq][8]; hist: [nq][256].
hipError_t bf_select(const float* scores, int64_t ld_scores, int N, int nq, int k, int32_t* state, uint32_t* hist,
                     int32_t* out_idx, float* out_dist, hipStream_t s);

}  // namespace sgk
