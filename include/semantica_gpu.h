/*
 * semantica_gpu.h -- C ABI of the MI355X (gfx950) EmbeddingGemma-300M Q8_0
 * forward library (libsemantica_gpu.so).
 *
 * Plain C types only: host or device pointers, sizes, int status codes.  No
 * exception or abort crosses this boundary; failures return a negative SG_ERR_*
 * code and sg_last_error() (thread-local) describes the most recent one.
 *
 * Each entry point replaces one seam of the reference Go implementation
 * (headlands-org/go-semantica); the citation is given beside it.  Paths are
 * relative to that source tree.
 */
#ifndef SEMANTICA_GPU_H
#define SEMANTICA_GPU_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SG_ABI_VERSION 2

/* Status codes.  The first four are the error cases of forwardINT8WithDim
 * (internal/runtime/model_int8.go:150-171) and ForwardWithDim
 * (internal/runtime/model.go:661-667). */
#define SG_OK 0
#define SG_ERR_EMPTY (-1)     /* "empty input": a sequence with no tokens        */
#define SG_ERR_TOO_LONG (-2)  /* "sequence too long: %d > %d"                    */
#define SG_ERR_TOKEN (-3)     /* "token ID out of range: %d"                     */
#define SG_ERR_DIM (-4)       /* "target dimension %d out of range (1..%d)"      */
#define SG_ERR_INVALID (-5)   /* bad argument / unsupported shape (kernel seams panic here) */
#define SG_ERR_DEVICE (-6)    /* HIP runtime failure                              */
#define SG_ERR_NOMEM (-7)     /* device or host allocation failed                 */

typedef struct sg_ctx sg_ctx;             /* one GPU: device ordinal + stream + scratch */
typedef struct sg_model sg_model;         /* weights resident in HBM + forward workspace */
typedef struct sg_q8_weight sg_q8_weight; /* one repacked Q8_0 matrix                    */

/* ModelConfig, internal/runtime/model.go:16-31 (fields parseConfig fills,
 * :424-517).  head_dim = embed_dim / num_heads and the attention scale
 * 1/sqrt(head_dim) are derived exactly as parseConfig derives them. */
typedef struct sg_model_config {
  int32_t embed_dim;    /* gemma-embedding.embedding_length  (768)  */
  int32_t num_layers;   /* block_count                        (24)   */
  int32_t num_heads;    /* attention.head_count               (3)    */
  int32_t num_kv_heads; /* attention.head_count_kv            (1)    */
  int32_t interm_dim;   /* feed_forward_length                (1152) */
  int32_t max_seq_len;  /* context_length                     (2048) */
  int32_t vocab_size;   /* len(tokenizer.ggml.tokens)         (262144) */
  float norm_eps;       /* attention.layer_norm_rms_epsilon   (1e-6) */
  float rope_base;      /* rope.freq_base                     (10000) */
} sg_model_config;

/* Host pointers to one layer's GGUF tensors, exactly as stored in the file
 * (loadLayerINT8, internal/runtime/model_int8.go:54-119): Q8_0 matrices are
 * raw 34-byte blocks, row-major [out][in/32]; norms are F32 vectors. */
typedef struct sg_layer_desc {
  const void *attn_q, *attn_k, *attn_v, *attn_output; /* blk.N.attn_{q,k,v,output}.weight */
  const void *ffn_gate, *ffn_up, *ffn_down;           /* blk.N.ffn_{gate,up,down}.weight  */
  const float *attn_norm, *attn_q_norm, *attn_k_norm; /* blk.N.attn_norm / attn_{q,k}_norm */
  const float *post_attention_norm, *ffn_norm, *post_ffw_norm;
} sg_layer_desc;

typedef struct sg_model_desc {
  sg_model_config config;
  const void *token_embd;     /* token_embd.weight, Q8_0 [vocab][embed_dim/32][34 B] */
  const float *output_norm;   /* output_norm.weight [embed_dim] */
  const sg_layer_desc *layers;/* num_layers entries */
} sg_model_desc;

/* ---- context ----------------------------------------------------------- */

/* Opens device `device_ordinal`, creates a default-priority stream.
 * (The reference has no device; this is the handle the Go cgo shim keeps.) */
int sg_init(int device_ordinal, sg_ctx **out);
void sg_shutdown(sg_ctx *ctx);
const char *sg_last_error(void);
int sg_abi_version(void);

/* ---- model seam --------------------------------------------------------- */

/* Replaces LoadModel/loadModel's weight setup (internal/runtime/model.go:233-315,
 * :520-552; model_int8.go:54-140): copies every tensor to HBM once, repacks
 * the Q8_0 matrices for the MFMA GEMM and extracts the fp32 block scales with
 * the IEEE converter (model_int8.go:543-597); the token embedding keeps the
 * halving converter of DequantizeQ8_0Row (gguf/tensor.go:157-240).  Host
 * buffers may be freed after return (unlike the Go zero-copy views). */
int sg_model_load(sg_ctx *ctx, const sg_model_desc *desc, sg_model **out);
void sg_model_free(sg_model *model);

/* ---- GGUF model images ---------------------------------------------------
 * parseConfig (internal/runtime/model.go:424-517) over a GGUF v3 image
 * (gguf/reader.go:98-178): fills *out from the metadata.  Host only; no
 * device call. */
int sg_gguf_read_config(const void *data, size_t size, sg_model_config *out);

/* LoadModelFromBytes (model.go:250-262) for the INT8 path: parses the image,
 * checks the tensors the forward reads (token_embd and the seven layer
 * matrices Q8_0; attn_norm/ffn_norm F32 or Q8_0; q/k norms, post norms and
 * output_norm optional) and calls sg_model_load.  The image may be released
 * after return.  No tokenizer is built: the library takes token IDs. */
int sg_model_load_gguf(sg_ctx *ctx, const void *data, size_t size, sg_model **out);

/* LoadModel (model.go:236-248): the same from a file, memory-mapped for the
 * duration of the call. */
int sg_model_load_gguf_file(sg_ctx *ctx, const char *path, sg_model **out);

/* Batched ForwardWithDim (internal/runtime/model.go:661-667 ->
 * forwardINT8WithDim model_int8.go:148-256) over n_seq packed sequences:
 * tokens[seq_offsets[i] .. seq_offsets[i+1]) is sequence i (CSR offsets,
 * seq_offsets[0] == 0).  out[n_seq][out_dim] receives each sequence's
 * mean-pooled, L2-normalized embedding truncated to out_dim (1..embed_dim).
 * Every sequence is computed exactly as the reference computes it alone
 * (per-sequence activation scales, attention and pooling).  Host buffers;
 * synchronous.  A model serves one call at a time (calls are serialized by a
 * per-model mutex), as the reference serves concurrent callers. */
int sg_forward(sg_model *model, const int32_t *tokens, const int32_t *seq_offsets,
               int32_t n_seq, int32_t out_dim, float *out);

/* Same, with tokens and out in device memory (tokens already resident in
 * HBM); seq_offsets stays on the host.  `stream` (hipStream_t, may be NULL
 * for the context stream) orders the work; the call returns after the
 * result is complete and token IDs have been validated on the device. */
int sg_forward_device(sg_model *model, const int32_t *d_tokens, const int32_t *seq_offsets,
                      int32_t n_seq, int32_t out_dim, float *d_out, void *stream);

/* Layer tap for parity work (no counterpart in the reference API; it mirrors
 * the CPU oracle's stop-layer tap): runs the embedding and the first
 * n_layers layers (0..num_layers) of the batched forward and copies the
 * residual stream h [T][embed_dim] (before the final norm) into d_hidden.
 * Same argument checks and synchronization as sg_forward_device. */
int sg_forward_hidden(sg_model *model, const int32_t *d_tokens, const int32_t *seq_offsets,
                      int32_t n_seq, int32_t n_layers, float *d_hidden, void *stream);

/* Per-layer trace of the batched forward, for parity checks: runs the first
 * n_layers layers (1..num_layers) as sg_forward_hidden does and writes, for
 * each layer l, rows l*T .. l*T + T - 1 (T = seq_offsets[n_seq]) of
 *   d_qkv [n_layers][T][q_dim + 2*kv_dim]: the Q|K|V GEMM output, before
 *         QK-norm and RoPE (runAttentionINT8, model_int8.go:357-372),
 *   d_att [n_layers][T][q_dim]: the attention output before it is quantized
 *         (model_int8.go:481-507),
 *   d_h   [n_layers][T][embed_dim]: the residual stream after the layer
 *         (model_int8.go:232).
 * Any of the three may be NULL.  No counterpart in the reference, which keeps
 * these values internal to forwardINT8WithDim (model_int8.go:148-256). */
int sg_forward_trace(sg_model *model, const int32_t *d_tokens, const int32_t *seq_offsets, int32_t n_seq,
                     int32_t n_layers, float *d_qkv, float *d_att, float *d_h, void *stream);

/* ---- measurement hook ---------------------------------------------------
 * No counterpart in the reference (its benchmark only times whole Embed
 * calls, cmd/benchmark/main.go:553-715).  While enabled, sg_forward*
 * brackets every kernel launch with HIP events on the launch stream and
 * accumulates, per kernel class, the event-measured time, the launch count
 * and the algorithmic work of those launches (int8 ops for the GEMM, flops
 * for attention's two products, bytes read+written at the reference dtypes
 * for the bandwidth kernels).  sg_profile_read synchronizes and returns the
 * totals since the last enable. */
enum {
  SG_K_GEMM = 0,      /* Q8_0 GEMMs (QKV, gate/up; O and down below the fused size) */
  SG_K_ATTENTION = 1, /* fused MQA attention                          */
  SG_K_QUANTIZE = 2,  /* per-sequence int8 quantization               */
  SG_K_NORM = 3,      /* embed+norm, post-norm+residual+norm, QK-norm+RoPE */
  SG_K_GELU = 4,      /* GELUQuick * up                               */
  SG_K_POOL = 5,      /* mean-pool + L2                               */
  SG_K_OTHER = 6,     /* fills                                        */
  SG_K_GEMM_NORM = 7, /* O / down GEMM with the residual post-norm in one launch
                         (work: the GEMM's int8 ops)                   */
  SG_K_CLASSES = 8
};
typedef struct sg_profile {
  double ms[SG_K_CLASSES];        /* summed event time of the class's launches */
  double work[SG_K_CLASSES];      /* ops (GEMM), flops (attention) or bytes    */
  int64_t launches[SG_K_CLASSES];
} sg_profile;
int sg_profile_enable(sg_model *model, int on);
int sg_profile_read(sg_model *model, sg_profile *out);

/* Attention arithmetic of the forward.  SG_ATTN_FAST (the default) runs the
 * score and weight products on fp16 matrix cores as hi/lo splits (within
 * 1e-5 relative of the reference's float32 attention).  SG_ATTN_EXACT runs
 * multiHeadAttentionInternal's float32 operations in its order on the vector
 * ALUs (attention.go:101-363 with dotProductSIMD's eight-lane sums,
 * activation.go:161-213, axpyAccum): with it the whole forward gives the bits
 * of forwardINT8WithDim on the block-serial GEMM path
 * (matmul_inner_loop_fallback.go:16-43, model_int8.go:148-256), several times
 * slower.  Needs max_seq_len <= 2048.  Takes effect from the next forward.
 * No counterpart in the reference (which has one attention): the switch is
 * for callers that need embeddings identical to it, such as parity checks. */
#define SG_ATTN_FAST 0
#define SG_ATTN_EXACT 1
int sg_model_set_attention_mode(sg_model *model, int mode);

/* ---- kernel seam (device pointers, work on `stream`) ---------------------
 * sg_matmul_q8_0_int8 and sg_ffn_gate_up are asynchronous: they return once
 * their work is enqueued on `stream`.  They share the context's operand
 * scratch, so each is ordered on the GPU after the previous one of the same
 * context (an event; no host wait), whatever streams they use.  The other
 * calls (they read host-side seq_offsets, or dump into temporary buffers)
 * return after their work on `stream` has completed. */

/* Repacks one raw Q8_0 matrix [out_dim][in_dim/32][34 B] (host pointer) into
 * the device layout used by the GEMM (the int8 values block-major, one
 * byte per weight, plus the fp32 block scales).  in_dim must be a multiple
 * of 32.
 * (extractQ8_0Scales model_int8.go:543-569 + the weight bytes it views.) */
int sg_q8_weight_create(sg_ctx *ctx, const void *q8, int32_t out_dim, int32_t in_dim,
                        sg_q8_weight **out);
void sg_q8_weight_free(sg_q8_weight *w);

/* QuantizeSymmetricINT8Into (internal/kernels/quantize.go:29-103) applied to
 * each sequence of a packed tensor: x[rows][cols] fp32, rows grouped by the
 * host CSR seq_offsets[n_seq+1].  One scale per sequence (max|x|/127; all-zero
 * input gives scale 1 and zeros).  q_out int8 [rows][cols], scale_out[n_seq]. */
int sg_quantize_act(sg_ctx *ctx, const float *x, int32_t rows, int32_t cols,
                    const int32_t *seq_offsets, int32_t n_seq,
                    int8_t *q_out, float *scale_out, void *stream);

/* MatMulQ8_0INT8 (internal/kernels/quantize.go:346-458):
 * dst[b][n] = (sum_blocks float(P_block) * d[n][block]) * row_scale[b] with
 * P_block the exact int32 dot of a 32-wide block, accumulated block by block
 * with a fused multiply-add.  x int8 [batch][in_dim]; row_scale[batch]
 * (the reference's single input.Scale, repeated per row of a sequence). */
int sg_matmul_q8_0_int8(sg_ctx *ctx, float *dst, const sg_q8_weight *w, const int8_t *x,
                        const float *row_scale, int32_t batch, void *stream);

/* sg_matmul_q8_0_int8 without any device allocation: the same kernels and the
 * same results, with the activation operand relaid in a fixed per-device
 * array of SG_NOALLOC_SCRATCH_BYTES (resolved by sg_init, held until the
 * process ends) instead of a library-grown buffer.  No counterpart in the
 * reference: for callers that cannot allocate (HIP graph capture, serving
 * loops).  Limit: gemm_pad(batch) x in_dim bytes, where gemm_pad rounds up
 * to 256 rows; larger inputs return SG_ERR_INVALID before any launch.  Calls
 * that overlap on one device (e.g. on two streams) race on the array. */
#define SG_NOALLOC_SCRATCH_BYTES (64u << 20)
int sg_matmul_q8_0_int8_noalloc(sg_ctx *ctx, float *dst, const sg_q8_weight *w, const int8_t *x,
                                const float *row_scale, int32_t batch, void *stream);

/* Measurement hook (no counterpart in the reference): the HBM yardstick the
 * bandwidth-bound kernels are set against.  kind 0: c = a + b over n fp32
 * (8 B read, 4 B written per element); kind 1: c = int8 codes of a at a fixed
 * scale (4 B read, 1 B written: the quantizers' I/O; b unused).  One float4
 * per lane, launched `reps` times back to back on `stream` between two HIP
 * events; returns the average time per launch.  n a multiple of 4, device
 * buffers 16-byte aligned.  Synchronizes the stream. */
int sg_hbm_probe(sg_ctx *ctx, int32_t kind, const float *a, const float *b, void *c, int64_t n,
                 int32_t reps, void *stream, float *us_per_launch);

/* Measurement hook (no counterpart in the reference): the issue rate of the
 * Q8_0 GEMM's per-K-block arithmetic with no memory traffic, the compute
 * floor of those kernels.  kind 0: per 32x32 output subtile and K-block one
 * v_mfma_i32_32x32x32_i8 and the block-serial update (16 subtractions + 16
 * v_fmac, as the GEMM kernels issue them); kind 1: the VALU part alone;
 * kind 2: the MFMA alone; kind 3: the attention's v_mfma_f32_16x16x32_f16
 * alone (four independent chains; one instruction per "subtile-block").
 * waves_per_simd (1..8) waves run `iters` steps of two subtiles each on every
 * SIMD.  Returns the SIMD cycles per subtile and K-block (the launch's event
 * time x the shader clock, which the waves' s_memtime / s_memrealtime counts
 * give, / subtile-blocks per SIMD) and that clock in GHz.  Allocates and frees its own small buffers; synchronizes the
 * stream. */
int sg_issue_probe(sg_ctx *ctx, int32_t kind, int32_t waves_per_simd, int32_t iters, void *stream,
                   float *simd_cycles_per_block, float *clock_ghz);

/* Measurement hook for the GEMM kernel alone (no counterpart in the
 * reference): relays x into the operand layout once, then launches the same
 * GEMM kernel sg_matmul_q8_0_int8 uses `reps` times back to back on `stream`
 * between two HIP events and returns the average time per launch.  dst is
 * written as by sg_matmul_q8_0_int8.  Synchronizes the stream. */
int sg_matmul_q8_0_int8_bench(sg_ctx *ctx, float *dst, const sg_q8_weight *w, const int8_t *x,
                              const float *row_scale, int32_t batch, int32_t reps, void *stream,
                              float *us_per_launch);

/* The exact int32 block dot products of the same GEMM, out[batch][out_dim][in_dim/32]
 * (what matmulInnerLoop* converts with VCVTDQ2PS, simd_amd64.s:290). */
int sg_q8_block_sums(sg_ctx *ctx, int32_t *out, const sg_q8_weight *w, const int8_t *x,
                     int32_t batch, void *stream);

/* The FFN's first half as one GEMM (model_int8.go:520-535: MatMulQ8_0INT8 with
 * ffn_gate and with ffn_up, GELUQuickSIMD on the gate output, VecMulF32 by up):
 * dst[b][n] = geluquick(gate[b][n]) * up[b][n], where gate and up are exactly
 * what sg_matmul_q8_0_int8 returns for w_gate and w_up (same shapes, out_dim a
 * multiple of 32); bit-identical to those two calls followed by
 * sg_gelu_quick_mul. */
int sg_ffn_gate_up(sg_ctx *ctx, float *dst, const sg_q8_weight *w_gate, const sg_q8_weight *w_up,
                   const int8_t *x, const float *row_scale, int32_t batch, void *stream);

/* RMSNorm per row (internal/kernels/norm.go:8-36), AVX2 8-lane order.
 * dst may equal src.  n must be a multiple of 8. */
int sg_rmsnorm(sg_ctx *ctx, float *dst, const float *src, const float *weight,
               int32_t rows, int32_t n, float eps, void *stream);

/* Per-head RMSNorm with attn_q_norm / attn_k_norm then RoPE (model_int8.go:371-452;
 * rope_cache.go:15-107) on q[rows][n_heads*head_dim] and k[rows][n_kv*head_dim]
 * (row strides ldq, ldk floats), in place.  Positions restart at 0 for each
 * sequence of the host CSR seq_offsets.  head_dim must be 256. */
int sg_qknorm_rope(sg_ctx *ctx, float *q, int32_t ldq, float *k, int32_t ldk,
                   const float *q_norm, const float *k_norm, int32_t n_heads, int32_t n_kv_heads,
                   int32_t head_dim, float eps, float rope_base, int32_t max_seq_len,
                   const int32_t *seq_offsets, int32_t n_seq, void *stream);

/* MultiHeadAttentionChunked with mask=nil (internal/kernels/attention.go:88-363) per
 * sequence: bidirectional MQA, scale 1/sqrt(head_dim), fastExp softmax.
 * q[rows][ldq] (heads at h*head_dim), k,v[rows][ldkv]; out[rows][n_heads*head_dim].
 * head_dim must be 256 and n_heads/n_kv_heads <= 4. */
int sg_attention(sg_ctx *ctx, float *out, const float *q, int32_t ldq, const float *k,
                 const float *v, int32_t ldkv, int32_t n_heads, int32_t n_kv_heads,
                 int32_t head_dim, const int32_t *seq_offsets, int32_t n_seq, void *stream);

/* sg_attention in the reference's float32 order (MultiHeadAttentionChunked,
 * attention.go:88-363, mask nil; see SG_ATTN_EXACT): bit-identical to it.
 * Same arguments; any n_heads / n_kv_heads ratio, sequences up to 2048 keys,
 * q and k 16-byte aligned with strides multiples of 4. */
int sg_attention_exact(sg_ctx *ctx, float *out, const float *q, int32_t ldq, const float *k,
                       const float *v, int32_t ldkv, int32_t n_heads, int32_t n_kv_heads,
                       int32_t head_dim, const int32_t *seq_offsets, int32_t n_seq, void *stream);

/* GELUQuickSIMD then VecMulF32 (activation.go:47-145, matmul.go:238-259):
 * dst[i] = geluquick(gate[i]) * up[i], for `rows` rows of `cols` (strides ldg, ldu, ldd). */
int sg_gelu_quick_mul(sg_ctx *ctx, float *dst, int32_t ldd, const float *gate, int32_t ldg,
                      const float *up, int32_t ldu, int32_t rows, int32_t cols, void *stream);

/* Token embedding lookup + sqrt(embed_dim) scaling (model_int8.go:166-184, with
 * DequantizeQ8_0Row's halving fp16 converter) for the model's token_embd. */
int sg_embed_tokens(sg_model *model, float *dst, const int32_t *d_tokens, int32_t n_tokens,
                    void *stream);

/* MeanPoolingPartial + l2Normalize (attention.go:423-445, runtime/model.go:808-820)
 * per sequence: x[rows][ldx], out[n_seq][out_dim]. */
int sg_pool_l2(sg_ctx *ctx, float *out, const float *x, int32_t ldx, int32_t out_dim,
               const int32_t *seq_offsets, int32_t n_seq, void *stream);

/* ---- tokenizer (internal/tokenizer) -------------------------------------
 * The reference's SentencePiece-style BPE tokenizer on the host: text ->
 * the token IDs sg_forward takes.  Same normalization (NFKC / accents /
 * lowercase), space handling, merge order (highest score, ties to the
 * rightmost pair), byte fallback and special tokens as tokenizer.go. */
typedef struct sg_tokenizer sg_tokenizer;

/* tokenizer.Config (tokenizer.go:46-53) plus the special ids
 * (LoadFromGGUF sets them from metadata, :570-595); -1 = none. */
typedef struct {
  int32_t add_bos, add_eos, lowercase, remove_accents, nfkc;
  int32_t bos_id, eos_id, unk_id, pad_id;
} sg_tokenizer_config;

/* tokenizer.New (tokenizer.go:56-97).  Token i is
 * token_data[token_offsets[i] .. token_offsets[i+1]) (UTF-8, any bytes);
 * token_types may be NULL (all normal).  "vocab and scores length mismatch"
 * cannot occur here (one n for both). */
int sg_tokenizer_create(const char *token_data, const int64_t *token_offsets, const float *scores,
                        const int32_t *token_types, int32_t n, const sg_tokenizer_config *cfg,
                        sg_tokenizer **out);

/* tokenizer.LoadFromGGUF (tokenizer.go:497-598) over a GGUF v3 image / file:
 * tokenizer.ggml.tokens, .scores, .token_type, .add_bos_token,
 * .add_eos_token and the special ids; NFKC on.  Same errors. */
int sg_tokenizer_from_gguf(const void *data, size_t size, sg_tokenizer **out);
int sg_tokenizer_from_gguf_file(const char *path, sg_tokenizer **out);

/* Tokenizer.Encode (tokenizer.go:99-133) of text[0..len): *n_ids receives the
 * number of IDs; the first min(n, cap) are written to ids (ids may be NULL to
 * query the count). */
int sg_tokenizer_encode(const sg_tokenizer *tok, const char *text, size_t len, int32_t *ids, int32_t cap,
                        int32_t *n_ids);

/* Encode of n_texts texts (text i = text_data[text_offsets[i] ..
 * text_offsets[i+1])) into one packed array: id_offsets[n_texts+1] receives
 * CSR offsets (the seq_offsets sg_forward takes); ids (capacity cap) may be
 * NULL to query the total, id_offsets[n_texts]. */
int sg_tokenizer_encode_batch(const sg_tokenizer *tok, const char *text_data, const int64_t *text_offsets,
                              int32_t n_texts, int32_t *ids, int64_t cap, int32_t *id_offsets);

/* Tokenizer.Decode (tokenizer.go:135-159): *len receives the byte length;
 * the first min(len, cap) bytes go to buf (not NUL-terminated). */
int sg_tokenizer_decode(const sg_tokenizer *tok, const int32_t *ids, int32_t n, char *buf, size_t cap,
                        size_t *len);

/* Tokenizer.VocabSize (tokenizer.go:438-440). */
int32_t sg_tokenizer_vocab_size(const sg_tokenizer *tok);

void sg_tokenizer_free(sg_tokenizer *tok);

/* ---- brute-force vector search (search/brute) ----------------------------
 * The reference's quantized brute-force index (search/brute/index.go,
 * builder.go, storage.go) with its vectors in HBM.  Scores are bit-identical
 * to the reference's amd64 AVX2 dot products (quant.go:79-135,
 * index.go:199-214, dot_amd64.s) and the top-k is the reference's streaming
 * selection (index.go:53-147), ties included; only the batching is new: one
 * call searches n_queries queries. */
typedef struct sg_index sg_index;

/* brute.QuantizationMode, search/brute/quant.go:8-15 */
#define SG_BF_FLOAT32 0
#define SG_BF_INT8 1
#define SG_BF_INT16 2

/* brute.NewBuilder(WithDimension(dim), WithQuantization(q)) + AddVector for each
 * (ids[i], vectors[i*dim ..]) + Build (builder.go:40-128): every vector is
 * L2-normalized (builder.go:131-141) and stored in mode q (quant.go:17-41).
 * Host vectors.  Errors as the reference: "brute: no vectors added" (n = 0),
 * "brute: duplicate id %d", "brute: unsupported quantization %d". */
int sg_index_build(sg_ctx *ctx, int32_t dim, int32_t quantization, const int32_t *ids,
                   const float *vectors, int32_t n, sg_index **out);

/* Same with the vectors in device memory (row stride ld floats), e.g. the
 * embeddings sg_forward_device left in HBM; ids stay on the host. */
int sg_index_build_device(sg_ctx *ctx, int32_t dim, int32_t quantization, const int32_t *ids,
                          const float *d_vectors, int64_t ld, int32_t n, void *stream, sg_index **out);

/* Serializer.Deserialize (storage.go:43-45,94-153) of a "BRUT" v1 image. */
int sg_index_deserialize(sg_ctx *ctx, const void *data, size_t size, sg_index **out);

/* Serializer.Serialize (storage.go:31-41,47-91): *size receives the image
 * size; with buf == NULL nothing else is done. */
int sg_index_serialize(sg_index *index, void *buf, size_t cap, size_t *size);

/* Index.Dimension / Count (index.go:149-153) and the storage mode. */
int sg_index_info(const sg_index *index, int32_t *dim, int32_t *count, int32_t *quantization);

/* Index.Vector (index.go:155-172): the dequantized vector stored under id;
 * SG_ERR_INVALID when there is none (the reference returns ok = false). */
int sg_index_vector(sg_index *index, int32_t id, float *out);

/* SearchVector (normalize = 1, index.go:27-41) or SearchNormalized
 * (normalize = 0, index.go:43-51) for n_queries queries [n_queries][dim]
 * (host).  Query q gets n_found[q] = min(top_k, count) results in
 * out_ids/out_dist[q*top_k ...], distance descending, ties by id ascending.
 * top_k <= 0: "brute: topK must be positive".  One call at a time per index
 * (a per-index mutex). */
int sg_index_search(sg_index *index, const float *queries, int32_t n_queries, int32_t top_k,
                    int32_t normalize, int32_t *out_ids, float *out_dist, int32_t *n_found,
                    void *stream);

void sg_index_free(sg_index *index);

#ifdef __cplusplus
}
#endif
#endif /* SEMANTICA_GPU_H */
