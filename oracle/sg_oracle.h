/*
 * sg_oracle.h -- CPU restatement of go-semantica's INT8 EmbeddingGemma forward
 * path (test infrastructure only).
 *
 * This is the checker that the HIP library is compared against.  It is NOT
 * part of the product: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg load it.  Every function names the reference file:line it
 * restates (paths relative to the go-semantica source tree).
 */
#ifndef SG_ORACLE_H
#define SG_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* fp16 -> fp32 converters.  The reference carries three copies:
 *   RUNTIME: internal/runtime/model_int8.go:571-597  (IEEE-correct, used for
 *            the GEMM block scales via extractQ8_0Scales :543-569)
 *   GGUF:    internal/gguf/tensor.go:207-240          (subnormals come out
 *            halved; used by DequantizeQ8_0Row for the token embedding)
 *   KERNELS: internal/kernels/matmul.go:261-288       (same quirk as GGUF)  */
enum { SGO_F16_RUNTIME = 0, SGO_F16_GGUF = 1, SGO_F16_KERNELS = 2 };
float sgo_f16_to_f32(uint16_t h, int variant);
void sgo_f16_table(int variant, float *out65536);

/* QuantizeSymmetricINT8Into, internal/kernels/quantize.go:29-103.
 * One scale for the whole [n] tensor.  Returns the scale. */
float sgo_quantize_symmetric(const float *x, int64_t n, int8_t *dst);

/* extractQ8_0Scales, internal/runtime/model_int8.go:543-569 */
void sgo_extract_q8_0_scales(const uint8_t *q8, int rows, int cols, float *scales);

/* GEMM accumulation orders (internal/kernels/simd_amd64.go:39-49):
 *   VNNI: matmulInnerLoopVNNIAsm simd_amd64.s:241-304 (8 lanes of 4 consecutive bytes)
 *   AVX2: matmulInnerLoopAsm     simd_amd64.s:164-237 (lane l = bytes 2l,2l+1,16+2l,17+2l)
 *   BLOCK_SERIAL: acc = fma(float(P_b), d_b, acc) over whole-block sums, the order
 *                 the GPU kernel uses (also the arm64 / fallback structure,
 *                 matmul_inner_loop_fallback.go:25-36, with a fused multiply-add). */
enum { SGO_ORDER_VNNI = 0, SGO_ORDER_AVX2 = 1, SGO_ORDER_BLOCK_SERIAL = 2, SGO_ORDER_ARM64 = 3 };
/*   ARM64: matmulInnerLoopAsm simd_arm64_matmul.s:6-56 -- whole-block SDOT sum,
 *          SCVTF, then FMULS and FADDS (two roundings per block). */

/* MatMulQ8_0INT8, internal/kernels/quantize.go:346-458.
 * dst[batch][out_dim]; w = raw Q8_0 rows [out_dim][in_dim/32][34 B];
 * scales [out_dim][in_dim/32] (runtime converter); x int8 [batch][in_dim];
 * row_scale[batch] = the activation scale applied to each row (the reference
 * applies the single tensor scale: pass the same value for every row).
 * in_dim must be a multiple of 32. */
void sgo_matmul_q8_0_int8(float *dst, const uint8_t *w, const float *scales,
                          const int8_t *x, const float *row_scale,
                          int batch, int in_dim, int out_dim, int order);

/* Exact int32 block dot products P[m][n][b] = sum_{k in block b} x[m,k]*w[n,k]. */
void sgo_block_sums(int32_t *out, const uint8_t *w, const int8_t *x,
                    int batch, int in_dim, int out_dim);

/* dotProductSIMD with the AVX2 asm order, simd_amd64.go:59-76 + simd_amd64.s:19-76 */
float sgo_dot_f32(const float *a, const float *b, int n);

/* RMSNorm, internal/kernels/norm.go:8-36 (dst may alias src) */
void sgo_rmsnorm(float *dst, const float *src, const float *w, int n, float eps);

/* fastExp activation.go:100-145, GELUQuickSIMD :47-95, Softmax :161-213 */
float sgo_fast_exp(float x);
void sgo_gelu_quick(float *dst, const float *src, int64_t n);
void sgo_softmax(float *dst, const float *src, int n);

/* NewRoPECache rope_cache.go:15-44: cos/sin [max_pos][head_dim/2], freqs [head_dim/2] */
void sgo_rope_cache(float *freqs, float *cos_tab, float *sin_tab,
                    int head_dim, float base, int max_pos);
/* ApplyRoPECached rope_cache.go:47-107, positions 0..seq_len-1 */
void sgo_rope_apply(float *qk, int seq_len, int n_heads, int head_dim,
                    const float *cos_tab, const float *sin_tab);

/* MultiHeadAttentionChunked with mask=nil, attention.go:88-363, after the
 * GQA expansion of model_int8.go:455-479.  q,out: [S][n_heads*hd]; k,v:
 * [S][n_kv*hd].  Chunking/head-parallel splits in the reference do not change
 * any value, so this is the serial schedule. */
void sgo_attention(float *out, const float *q, const float *k, const float *v,
                   int seq_len, int n_heads, int n_kv_heads, int head_dim, float scale);

/* MeanPoolingPartial attention.go:423-445; l2Normalize runtime/model.go:808-820 */
void sgo_mean_pool_partial(float *dst, const float *src, int seq_len, int emb_dim, int out_dim);
void sgo_l2_normalize(float *v, int n);

/* DequantizeQ8_0Row gguf/tensor.go:157-178 (GGUF converter) */
void sgo_dequant_q8_0_row(float *dst, const uint8_t *row, int n);

/* ---- model ---- */
typedef struct sgo_config {
  int32_t embed_dim, num_layers, num_heads, num_kv_heads, head_dim, interm_dim;
  int32_t max_seq_len, vocab_size;
  float norm_eps, rope_base;
} sgo_config;

typedef struct sgo_layer {
  const uint8_t *attn_q, *attn_k, *attn_v, *attn_output, *ffn_gate, *ffn_up, *ffn_down;
  const float *attn_norm, *attn_q_norm, *attn_k_norm, *post_attention_norm, *ffn_norm, *post_ffw_norm;
} sgo_layer;

typedef struct sgo_model sgo_model;

/* Pointers are borrowed (zero-copy, like the reference's GGUF views). */
sgo_model *sgo_model_create(const sgo_config *cfg, const uint8_t *token_embd,
                            const float *output_norm, const sgo_layer *layers);
void sgo_model_free(sgo_model *m);

/* forwardINT8WithDim, runtime/model_int8.go:148-256.  Returns 0 or a negative
 * error code (-1 empty, -2 too long, -3 token out of range, -4 bad dim).
 * stop_layer < 0 runs the whole model and writes out[target_dim]; otherwise the
 * hidden state [S][embed_dim] after `stop_layer` layers is written to out
 * (before the final norm) -- a debugging tap. */
int sgo_forward(const sgo_model *m, const int32_t *tokens, int seq_len, int target_dim,
                float *out, int order, int stop_layer);

/* embedPrompts-style fan-out, pkg/ggufembed/api.go:237-295: n_threads workers
 * over contiguous sequence ranges.  seq_offsets[n_seq+1] (CSR); out[n_seq][target_dim]. */
int sgo_forward_batch(const sgo_model *m, const int32_t *tokens, const int32_t *seq_offsets,
                      int n_seq, int target_dim, float *out, int order, int n_threads);

/* Per-layer taps of the batched forward (a checker's view; the reference keeps
 * these internal).  Arrays are packed over the batch like the GPU library's
 * trace: row r (0..T-1, sequences concatenated) of layer l at row
 * l * layer_rows + r, with layer_rows = T.  Only layers < n_layers are tapped.
 *   att_in: replaces each layer's attention output before it is quantized
 *           (teacher forcing: model_int8.go:349-507 continues on these values)
 *   qkv:    Q|K|V GEMM outputs per row, before QK-norm and RoPE
 *   att:    the oracle's own attention output (computed even when forced)
 *   h:      the residual stream after the layer (model_int8.go:232) */
typedef struct sgo_taps {
  const float *att_in;
  float *qkv, *att, *h;
  int32_t n_layers;
  int64_t layer_rows;
} sgo_taps;
int sgo_forward_taps(const sgo_model *m, const int32_t *tokens, const int32_t *seq_offsets,
                     int n_seq, int target_dim, float *out, int order, int n_threads, const sgo_taps *taps);

/* 1 when the AVX2+FMA fast paths are in use on this host, 2 when the VNNI
 * order also runs on AVX-512 VNNI (results are bit-identical to the scalar
 * definitions either way). */
int sgo_simd_level(void);
void sgo_force_scalar(int on);
/* Threads per GEMM call (column chunks); 1 = serial (the default). */
void sgo_set_gemm_threads(int n);

/* Brute-force vector search (search/brute), sg_oracle_search.c.
 * Storage modes: QuantizationMode, search/brute/quant.go:8-15. */
enum { SGO_BF_F32 = 0, SGO_BF_I8 = 1, SGO_BF_I16 = 2 };
void sgo_bf_normalize(float *v, int dim);                          /* builder.go:131-141 */
void sgo_bf_quantize_i8(const float *v, int dim, int8_t *out);     /* quant.go:17-29 */
void sgo_bf_quantize_i16(const float *v, int dim, int16_t *out);   /* quant.go:31-41 */
float sgo_bf_dot_i8(const int8_t *vec, const float *q, int dim);   /* quant.go:79-105 */
float sgo_bf_dot_i16(const int16_t *vec, const float *q, int dim); /* quant.go:107-135 */
float sgo_bf_dot_f32(const float *a, const float *b, int dim);     /* index.go:199-214 */
/* score of stored row `row` (data row-major [count][dim] in `mode`) */
float sgo_bf_dot(const void *data, int mode, int64_t row, const float *q, int dim);
/* searchNormalized, index.go:53-147 (query already normalized). */
int sgo_bf_search(const void *data, int mode, const int32_t *ids, int count, int dim, const float *query,
                  int top_k, int32_t *out_ids, float *out_dist);

#ifdef __cplusplus
}
#endif
#endif
