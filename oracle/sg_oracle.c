/*
 * sg_oracle.c -- CPU restatement of go-semantica's INT8 EmbeddingGemma
 * forward path.  TEST INFRASTRUCTURE ONLY: the parity checker for the HIP
 * library and the timed CPU baseline ("port") in bench.py.  Nothing in the
 * product links, loads or calls this file.
 *
 * Arithmetic follows the reference exactly, operation by operation, with the
 * rounding each Go/asm statement performs:
 *   - Go on amd64 (default GOAMD64=v1) does not contract a*b+c into an FMA, so
 *     this file is compiled with -ffp-contract=off and uses fmaf() only where
 *     the reference assembly issues VFMADD231PS.
 *   - float64 products and sqrt are done in double exactly where the Go code
 *     converts to float64.
 * The AVX2 paths below are speed-ups of the scalar definitions and produce the
 * same bits (tests/test_oracle.py checks that); sgo_force_scalar(1) disables them.
 */
#include "sg_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#if defined(__x86_64__)
#include <immintrin.h>
#define SGO_X86 1
#endif

static int g_force_scalar = 0;
static int g_simd = -1;
static int g_gemm_threads = 1;

void sgo_force_scalar(int on) { g_force_scalar = on; }

/* 0 scalar, 1 AVX2+FMA, 2 AVX2+FMA and AVX-512 VNNI (with VL), the ISA the
 * reference dispatches on (simd_amd64.go:9-13,41-45). */
int sgo_simd_level(void) {
  if (g_simd < 0) {
#if SGO_X86
    __builtin_cpu_init();
    g_simd = (__builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma")) ? 1 : 0;
    if (g_simd && __builtin_cpu_supports("avx512vnni") && __builtin_cpu_supports("avx512vl")) g_simd = 2;
#else
    g_simd = 0;
#endif
  }
  return g_force_scalar ? 0 : g_simd;
}

void sgo_set_gemm_threads(int n) { g_gemm_threads = n < 1 ? 1 : n; }

static inline float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* ---------------------------------------------------------------- fp16 ---- */

/* internal/runtime/model_int8.go:571-597 (IEEE-correct: note exponent++ at :585) */
static float f16_runtime(uint16_t h) {
  uint32_t sign = (h >> 15) & 1u;
  int32_t exponent = (h >> 10) & 0x1f;
  uint32_t fraction = h & 0x3ffu;
  if (exponent == 0) {
    if (fraction == 0) return bits_f32(sign << 31);
    while ((fraction & 0x400u) == 0) { fraction <<= 1; exponent--; }
    exponent++;
    fraction &= 0x3ffu;
  } else if (exponent == 0x1f) {
    return bits_f32((sign << 31) | 0x7f800000u | (fraction << 13));
  }
  uint32_t e32 = (uint32_t)(exponent + (127 - 15));
  return bits_f32((sign << 31) | (e32 << 23) | (fraction << 13));
}

/* internal/gguf/tensor.go:207-240 and internal/kernels/matmul.go:261-288:
 * the subnormal branch starts from exp = 127-15 with no +1, so every fp16
 * subnormal comes out at half its value. */
static float f16_halving(uint16_t h) {
  uint32_t sign = (h >> 15) & 1u, ex = (h >> 10) & 0x1fu, mant = h & 0x3ffu, bits;
  if (ex == 0) {
    if (mant == 0) {
      bits = sign << 31;
    } else {
      uint32_t e = 127u - 15u;
      while ((mant & 0x400u) == 0) { mant <<= 1; e--; }
      mant &= 0x3ffu;
      bits = (sign << 31) | (e << 23) | (mant << 13);
    }
  } else if (ex == 0x1f) {
    bits = (sign << 31) | (0xffu << 23) | (mant << 13);
  } else {
    bits = (sign << 31) | (((ex - 15u + 127u) & 0xffu) << 23) | (mant << 13);
  }
  return bits_f32(bits);
}

float sgo_f16_to_f32(uint16_t h, int variant) {
  return variant == SGO_F16_RUNTIME ? f16_runtime(h) : f16_halving(h);
}

void sgo_f16_table(int variant, float *out) {
  for (uint32_t i = 0; i < 65536u; i++) out[i] = sgo_f16_to_f32((uint16_t)i, variant);
}

static inline uint16_t rd_u16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* ------------------------------------------------------------ quantize ---- */

/* quantize.go:29-69 (QuantizeSymmetricINT8Into), :80-90 absMaxScalar, :92-103 quantizeInto */
float sgo_quantize_symmetric(const float *x, int64_t n, int8_t *dst) {
  if (n == 0) return 1.0f;
  float maxv = 0.0f;
  for (int64_t i = 0; i < n; i++) {
    float a = bits_f32(f32_bits(x[i]) & 0x7fffffffu);
    if (a > maxv) maxv = a;
  }
  if (maxv == 0.0f) {
    memset(dst, 0, (size_t)n);
    return 1.0f;
  }
  float scale = maxv / 127.0f;
  float inv = 1.0f / scale;
  for (int64_t i = 0; i < n; i++) {
    double s = (double)x[i] * (double)inv;
    int32_t q = (int32_t)round(s); /* math.Round: half away from zero */
    if (q > 127) q = 127; else if (q < -127) q = -127;
    dst[i] = (int8_t)q;
  }
  return scale;
}

/* model_int8.go:543-569 */
void sgo_extract_q8_0_scales(const uint8_t *q8, int rows, int cols, float *scales) {
  int nb = (cols + 31) / 32;
  for (int r = 0; r < rows; r++)
    for (int b = 0; b < nb; b++)
      scales[(int64_t)r * nb + b] = f16_runtime(rd_u16(q8 + ((int64_t)r * nb + b) * 34));
}

/* ---------------------------------------------------------------- GEMM ---- */

/* Horizontal sum used by every AVX2/VNNI asm routine (simd_amd64.s:50-54,
 * :229-232, :297-300): VEXTRACTF128 + VADDPS, then two VHADDPS. */
static inline float hsum8(const float a[8]) {
  return ((a[0] + a[4]) + (a[1] + a[5])) + ((a[2] + a[6]) + (a[3] + a[7]));
}

/* One output element over nb whole blocks: the scalar definition of the
 * three orders. xr: int8 activations of one row, wr: raw Q8_0 row. */
static float q8_dot_scalar(const int8_t *xr, const uint8_t *wr, const float *sc, int nb, int order) {
  if (order == SGO_ORDER_BLOCK_SERIAL || order == SGO_ORDER_ARM64) {
    float acc = 0.0f;
    for (int b = 0; b < nb; b++) {
      const int8_t *w = (const int8_t *)(wr + (int64_t)b * 34 + 2);
      const int8_t *x = xr + (int64_t)b * 32;
      int32_t p = 0;
      for (int k = 0; k < 32; k++) p += (int32_t)x[k] * (int32_t)w[k];
      if (order == SGO_ORDER_BLOCK_SERIAL) {
        acc = fmaf((float)p, sc[b], acc);
      } else { /* SDOT + ADDP, SCVTF, FMULS, FADDS: simd_arm64_matmul.s:25-46 */
        float t = (float)p * sc[b];
        acc = acc + t;
      }
    }
    return acc;
  }
  float lane[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int b = 0; b < nb; b++) {
    const int8_t *w = (const int8_t *)(wr + (int64_t)b * 34 + 2);
    const int8_t *x = xr + (int64_t)b * 32;
    for (int l = 0; l < 8; l++) {
      int32_t p = 0;
      if (order == SGO_ORDER_VNNI) {
        /* VPDPBUSD lane l covers bytes 4l..4l+3 (simd_amd64.s:279-288) */
        for (int t = 0; t < 4; t++) p += (int32_t)x[4 * l + t] * (int32_t)w[4 * l + t];
      } else {
        /* VPMOVSXBW + VPMADDWD on each 16-byte half, then VPADDD (:199-215) */
        p = ((int32_t)x[2 * l] * w[2 * l] + (int32_t)x[2 * l + 1] * w[2 * l + 1]) +
            ((int32_t)x[16 + 2 * l] * w[16 + 2 * l] + (int32_t)x[17 + 2 * l] * w[17 + 2 * l]);
      }
      lane[l] = fmaf((float)p, sc[b], lane[l]); /* VCVTDQ2PS + VFMADD231PS */
    }
  }
  return hsum8(lane);
}

#if SGO_X86
__attribute__((target("avx2,fma")))
static float q8_dot_avx2(const int8_t *xr, const uint8_t *wr, const float *sc, int nb, int order) {
  __m256 acc = _mm256_setzero_ps();
  for (int b = 0; b < nb; b++) {
    const __m128i *wp = (const __m128i *)(wr + (int64_t)b * 34 + 2);
    const __m128i *xp = (const __m128i *)(xr + (int64_t)b * 32);
    __m256i xlo = _mm256_cvtepi8_epi16(_mm_loadu_si128(xp));
    __m256i xhi = _mm256_cvtepi8_epi16(_mm_loadu_si128(xp + 1));
    __m256i wlo = _mm256_cvtepi8_epi16(_mm_loadu_si128(wp));
    __m256i whi = _mm256_cvtepi8_epi16(_mm_loadu_si128(wp + 1));
    __m256i plo = _mm256_madd_epi16(xlo, wlo); /* pairs (2i,2i+1), bytes 0..15 */
    __m256i phi = _mm256_madd_epi16(xhi, whi); /* pairs, bytes 16..31 */
    __m256i lanes;
    if (order == SGO_ORDER_VNNI) {
      /* lane l = bytes 4l..4l+3: hadd pairs, then undo hadd's 128-bit interleave */
      lanes = _mm256_permute4x64_epi64(_mm256_hadd_epi32(plo, phi), 0xD8);
    } else {
      lanes = _mm256_add_epi32(plo, phi);
    }
    acc = _mm256_fmadd_ps(_mm256_cvtepi32_ps(lanes), _mm256_set1_ps(sc[b]), acc);
  }
  float l[8];
  _mm256_storeu_ps(l, acc);
  return hsum8(l);
}

/* matmulInnerLoopVNNIAsm itself (simd_amd64.s:241-304) on an AVX-512-VNNI
 * host: VPDPBUSD of (w ^ 0x80) as unsigned bytes with x, minus 128 * sum(x)
 * from a second VPDPBUSD with ones, VCVTDQ2PS, VFMADD231PS, then the hsum.
 * The lane integers equal the AVX2 emulation's, so the results are the same
 * bits; this is the path the reference takes on such a host. */
__attribute__((target("avx2,fma,avx512vnni,avx512vl")))
static float q8_dot_vnni512(const int8_t *xr, const uint8_t *wr, const float *sc, int nb) {
  const __m256i sign = _mm256_set1_epi8((char)0x80), ones = _mm256_set1_epi8(1);
  __m256 acc = _mm256_setzero_ps();
  for (int b = 0; b < nb; b++) {
    __m256i x = _mm256_loadu_si256((const __m256i *)(xr + (int64_t)b * 32));
    __m256i w = _mm256_loadu_si256((const __m256i *)(wr + (int64_t)b * 34 + 2));
    __m256i dot = _mm256_dpbusd_epi32(_mm256_setzero_si256(), _mm256_xor_si256(w, sign), x);
    __m256i sx = _mm256_dpbusd_epi32(_mm256_setzero_si256(), ones, x);
    dot = _mm256_sub_epi32(dot, _mm256_slli_epi32(sx, 7));
    acc = _mm256_fmadd_ps(_mm256_cvtepi32_ps(dot), _mm256_set1_ps(sc[b]), acc);
  }
  float l[8];
  _mm256_storeu_ps(l, acc);
  return hsum8(l);
}

/* One accumulator over whole-block sums (block-serial fma, or arm64's
 * mul + add): the int32 block sum is exact whatever order its products are
 * added in, so it is formed with VPMADDWD and an integer reduction. */
__attribute__((target("avx2,fma")))
static float q8_dot_serial_avx2(const int8_t *xr, const uint8_t *wr, const float *sc, int nb, int fused) {
  float acc = 0.0f;
  for (int b = 0; b < nb; b++) {
    const __m128i *wp = (const __m128i *)(wr + (int64_t)b * 34 + 2);
    const __m128i *xp = (const __m128i *)(xr + (int64_t)b * 32);
    __m256i plo = _mm256_madd_epi16(_mm256_cvtepi8_epi16(_mm_loadu_si128(xp)),
                                    _mm256_cvtepi8_epi16(_mm_loadu_si128(wp)));
    __m256i phi = _mm256_madd_epi16(_mm256_cvtepi8_epi16(_mm_loadu_si128(xp + 1)),
                                    _mm256_cvtepi8_epi16(_mm_loadu_si128(wp + 1)));
    __m256i s8 = _mm256_add_epi32(plo, phi);
    __m128i t = _mm_add_epi32(_mm256_castsi256_si128(s8), _mm256_extracti128_si256(s8, 1));
    t = _mm_add_epi32(t, _mm_shuffle_epi32(t, 0x4E));
    t = _mm_add_epi32(t, _mm_shuffle_epi32(t, 0xB1));
    int32_t p = _mm_cvtsi128_si32(t);
    if (fused) {
      acc = fmaf((float)p, sc[b], acc);
    } else {
      float prod = (float)p * sc[b];
      acc = acc + prod;
    }
  }
  return acc;
}
#endif

/* matMulQ8_0INT8SerialRange, quantize.go:390-458 (whole blocks only), over
 * output columns [c0, c1): dst[i*N+j] = innerLoop(...) * inputScale */
static void matmul_cols(float *dst, const uint8_t *w, const float *scales, const int8_t *x,
                        const float *row_scale, int batch, int in_dim, int out_dim, int order,
                        int c0, int c1) {
  int nb = in_dim / 32;
  int64_t row_bytes = (int64_t)nb * 34;
  int simd = sgo_simd_level();
  int serial = order == SGO_ORDER_BLOCK_SERIAL || order == SGO_ORDER_ARM64;
  const int JT = 64; /* column tile: keeps a weight tile hot while rows stream */
  for (int j0 = c0; j0 < c1; j0 += JT) {
    int j1 = j0 + JT < c1 ? j0 + JT : c1;
    for (int i = 0; i < batch; i++) {
      const int8_t *xr = x + (int64_t)i * in_dim;
      float s = row_scale[i];
      for (int j = j0; j < j1; j++) {
        const uint8_t *wr = w + (int64_t)j * row_bytes;
        const float *sc = scales + (int64_t)j * nb;
        float v;
#if SGO_X86
        if (simd && serial) v = q8_dot_serial_avx2(xr, wr, sc, nb, order == SGO_ORDER_BLOCK_SERIAL); else
        if (simd == 2 && order == SGO_ORDER_VNNI) v = q8_dot_vnni512(xr, wr, sc, nb); else
        if (simd) v = q8_dot_avx2(xr, wr, sc, nb, order); else
#endif
        v = q8_dot_scalar(xr, wr, sc, nb, order);
        dst[(int64_t)i * out_dim + j] = v * s;
      }
    }
  }
}

typedef struct {
  float *dst;
  const uint8_t *w;
  const float *scales;
  const int8_t *x;
  const float *row_scale;
  int batch, in_dim, out_dim, order, c0, c1;
} mm_job;

static void *mm_worker(void *p) {
  mm_job *j = (mm_job *)p;
  matmul_cols(j->dst, j->w, j->scales, j->x, j->row_scale, j->batch, j->in_dim, j->out_dim, j->order, j->c0, j->c1);
  return NULL;
}

/* With sgo_set_gemm_threads(n > 1), the output columns are split into
 * contiguous chunks over n threads (matMulQ8_0INT8Tiled's column tasks,
 * model_int8.go:258-346); every element is computed exactly as serially. */
void sgo_matmul_q8_0_int8(float *dst, const uint8_t *w, const float *scales,
                          const int8_t *x, const float *row_scale,
                          int batch, int in_dim, int out_dim, int order) {
  int n = g_gemm_threads;
  if (n > 1 && out_dim >= 128) {
    int chunk = (out_dim + n - 1) / n;
    chunk = (chunk + 31) / 32 * 32;
    mm_job jobs[256];
    pthread_t th[256];
    int used = 0;
    for (int c0 = 0; c0 < out_dim && used < 256; c0 += chunk) {
      jobs[used] = (mm_job){dst, w, scales, x, row_scale, batch, in_dim, out_dim, order, c0,
                            c0 + chunk < out_dim ? c0 + chunk : out_dim};
      pthread_create(&th[used], NULL, mm_worker, &jobs[used]);
      used++;
    }
    for (int i = 0; i < used; i++) pthread_join(th[i], NULL);
    return;
  }
  matmul_cols(dst, w, scales, x, row_scale, batch, in_dim, out_dim, order, 0, out_dim);
}

void sgo_block_sums(int32_t *out, const uint8_t *w, const int8_t *x,
                    int batch, int in_dim, int out_dim) {
  int nb = in_dim / 32;
  for (int i = 0; i < batch; i++)
    for (int j = 0; j < out_dim; j++)
      for (int b = 0; b < nb; b++) {
        const int8_t *wq = (const int8_t *)(w + ((int64_t)j * nb + b) * 34 + 2);
        const int8_t *xq = x + (int64_t)i * in_dim + b * 32;
        int64_t p = 0;
        for (int k = 0; k < 32; k++) p += (int64_t)xq[k] * wq[k];
        out[((int64_t)i * out_dim + j) * nb + b] = (int32_t)p;
      }
}

/* ----------------------------------------------------------- fp32 dot ---- */

/* dotProductSIMD simd_amd64.go:59-85 -> dotProductAVX2Asm simd_amd64.s:19-76 */
static float dot_scalar(const float *a, const float *b, int n) {
  if (n < 8) { /* dotProductScalar: sum += a*b, unfused */
    float s = 0.0f;
    for (int i = 0; i < n; i++) s = s + a[i] * b[i];
    return s;
  }
  float lane[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  int n8 = n & ~7;
  for (int i = 0; i < n8; i += 8)
    for (int l = 0; l < 8; l++) lane[l] = fmaf(a[i + l], b[i + l], lane[l]);
  float s = hsum8(lane);
  for (int i = n8; i < n; i++) s = s + a[i] * b[i]; /* VMULSS, VADDSS */
  return s;
}

#if SGO_X86
__attribute__((target("avx2,fma")))
static float dot_avx2(const float *a, const float *b, int n) {
  if (n < 8) return dot_scalar(a, b, n);
  __m256 acc = _mm256_setzero_ps();
  int n8 = n & ~7;
  for (int i = 0; i < n8; i += 8)
    acc = _mm256_fmadd_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i), acc);
  float l[8];
  _mm256_storeu_ps(l, acc);
  float s = hsum8(l);
  for (int i = n8; i < n; i++) s = s + a[i] * b[i];
  return s;
}
#endif

float sgo_dot_f32(const float *a, const float *b, int n) {
#if SGO_X86
  if (sgo_simd_level()) return dot_avx2(a, b, n);
#endif
  return dot_scalar(a, b, n);
}

/* ------------------------------------------------------------- RMSNorm ---- */

/* norm.go:8-36: sumSq via dotProductSIMD (n>=8) or sumSquaresScalar (:105-111);
 * meanSq = sumSq/float32(n); rms = float32(sqrt(float64(meanSq+eps)));
 * invRms = 1/rms; dst = (src*invRms)*weight with two roundings. */
void sgo_rmsnorm(float *dst, const float *src, const float *w, int n, float eps) {
  float ss;
  if (n >= 8) ss = sgo_dot_f32(src, src, n);
  else { ss = 0.0f; for (int i = 0; i < n; i++) ss = ss + src[i] * src[i]; }
  float ms = ss / (float)n;
  float rms = (float)sqrt((double)(ms + eps));
  float inv = 1.0f / rms;
  for (int i = 0; i < n; i++) {
    float t = src[i] * inv;
    dst[i] = t * w[i];
  }
}

/* ----------------------------------------------------- fastExp & friends ---- */

/* activation.go:100-145 */
float sgo_fast_exp(float x) {
  const float log2e = 1.442695041f;
  if (x < -10.0f) return 0.0f;
  if (x > 10.0f) return 22026.4657948f;
  float y = x * log2e;
  int32_t ip = (int32_t)y; /* truncation toward zero */
  float f = y - (float)ip;
  const float c1 = 0.693147180559945f, c2 = 0.240226506959101f;
  const float c3 = 0.055504108664821f, c4 = 0.009676036358193f;
  float poly = 1.0f + f * (c1 + f * (c2 + f * (c3 + f * c4)));
  if (ip >= -126 && ip <= 127) return poly * bits_f32((uint32_t)(ip + 127) << 23);
  if (ip < -126) return 0.0f;
  return 3.402823e+38f;
}

/* GELUQuickSIMD activation.go:47-95 (the 8-wide blocking does not change values) */
void sgo_gelu_quick(float *dst, const float *src, int64_t n) {
  const float scale = 1.702f;
  for (int64_t i = 0; i < n; i++) {
    float x = src[i];
    float sx = scale * x, sig;
    if (sx >= 0.0f) {
      float e = sgo_fast_exp(-sx);
      sig = 1.0f / (1.0f + e);
    } else {
      float e = sgo_fast_exp(sx);
      sig = e / (1.0f + e);
    }
    dst[i] = x * sig;
  }
}

/* Softmax activation.go:161-213 (sum += e0+e1+e2+e3 evaluates ((e0+e1)+e2)+e3) */
void sgo_softmax(float *dst, const float *src, int n) {
  if (n == 0) return;
  float maxv = src[0];
  for (int i = 1; i < n; i++) if (src[i] > maxv) maxv = src[i];
  float sum = 0.0f;
  int i = 0;
  for (; i + 3 < n; i += 4) {
    float e0 = sgo_fast_exp(src[i] - maxv), e1 = sgo_fast_exp(src[i + 1] - maxv);
    float e2 = sgo_fast_exp(src[i + 2] - maxv), e3 = sgo_fast_exp(src[i + 3] - maxv);
    dst[i] = e0; dst[i + 1] = e1; dst[i + 2] = e2; dst[i + 3] = e3;
    sum = sum + (((e0 + e1) + e2) + e3);
  }
  for (; i < n; i++) {
    float e = sgo_fast_exp(src[i] - maxv);
    dst[i] = e;
    sum = sum + e;
  }
  if (sum == 0.0f) {
    float inv = 1.0f / (float)n;
    for (int k = 0; k < n; k++) dst[k] = inv;
    return;
  }
  float inv = 1.0f / sum;
  for (int k = 0; k < n; k++) dst[k] = dst[k] * inv;
}

/* ---------------------------------------------------------------- RoPE ---- */

/* rope_cache.go:15-44 */
void sgo_rope_cache(float *freqs, float *cos_tab, float *sin_tab,
                    int head_dim, float base, int max_pos) {
  int half = head_dim / 2;
  for (int i = 0; i < half; i++)
    freqs[i] = (float)(1.0 / pow((double)base, (double)(2 * i) / (double)head_dim));
  for (int p = 0; p < max_pos; p++) {
    float pf = (float)p;
    for (int i = 0; i < half; i++) {
      float th = pf * freqs[i];
      cos_tab[(int64_t)p * half + i] = (float)cos((double)th);
      sin_tab[(int64_t)p * half + i] = (float)sin((double)th);
    }
  }
}

/* rope_cache.go:47-107 (NeoX pairs (i, i+half); unfused products) */
void sgo_rope_apply(float *qk, int seq_len, int n_heads, int head_dim,
                    const float *cos_tab, const float *sin_tab) {
  int half = head_dim / 2;
  for (int s = 0; s < seq_len; s++) {
    const float *c = cos_tab + (int64_t)s * half, *sn = sin_tab + (int64_t)s * half;
    for (int h = 0; h < n_heads; h++) {
      float *v = qk + ((int64_t)s * n_heads + h) * head_dim;
      for (int i = 0; i < half; i++) {
        float v0 = v[i], v1 = v[i + half];
        float a = v0 * c[i], b = v1 * sn[i];
        float cc = v0 * sn[i], d = v1 * c[i];
        v[i] = a - b;
        v[i + half] = cc + d;
      }
    }
  }
}

/* ----------------------------------------------------------- attention ---- */

/* axpyAccum attention.go:344-363 with the AVX2 branch: scaled = vec*weight
 * (VecScaleF32), out = out + scaled (VecAddF32). */
static void axpy_scalar(float *out, const float *v, float wgt, int n) {
  for (int i = 0; i < n; i++) { float t = v[i] * wgt; out[i] = out[i] + t; }
}
#if SGO_X86
__attribute__((target("avx2,fma")))
static void axpy_avx2(float *out, const float *v, float wgt, int n) {
  __m256 w = _mm256_set1_ps(wgt);
  int i = 0;
  for (; i + 8 <= n; i += 8)
    _mm256_storeu_ps(out + i, _mm256_add_ps(_mm256_loadu_ps(out + i), _mm256_mul_ps(_mm256_loadu_ps(v + i), w)));
  for (; i < n; i++) { float t = v[i] * wgt; out[i] = out[i] + t; }
}
#endif

/* processHeadRange attention.go:178-265 + computeAttentionScoresRange :267-310,
 * mask == nil, on K/V expanded per model_int8.go:455-479 (kv head = h / group). */
void sgo_attention(float *out, const float *q, const float *k, const float *v,
                   int S, int H, int HKV, int hd, float scale) {
  int group = H / HKV;
  int qs = H * hd, ks = HKV * hd;
  float *sc = (float *)malloc(sizeof(float) * (size_t)S * (size_t)S);
  int simd = sgo_simd_level();
  for (int h = 0; h < H; h++) {
    int kvh = h / group;
    for (int i = 0; i < S; i++) {
      const float *qr = q + (int64_t)i * qs + h * hd;
      for (int j = 0; j < S; j++) {
        float s = sgo_dot_f32(qr, k + (int64_t)j * ks + kvh * hd, hd);
        sc[(int64_t)i * S + j] = s * scale;
      }
    }
    for (int i = 0; i < S; i++) sgo_softmax(sc + (int64_t)i * S, sc + (int64_t)i * S, S);
    for (int i = 0; i < S; i++) {
      float *orow = out + (int64_t)i * qs + h * hd;
      for (int d = 0; d < hd; d++) orow[d] = 0.0f;
      for (int j = 0; j < S; j++) {
        float p = sc[(int64_t)i * S + j];
        if (p == 0.0f) continue;
        const float *vr = v + (int64_t)j * ks + kvh * hd;
#if SGO_X86
        if (simd) { axpy_avx2(orow, vr, p, hd); continue; }
#endif
        axpy_scalar(orow, vr, p, hd);
      }
    }
  }
  free(sc);
}

/* --------------------------------------------------------- pool and L2 ---- */

/* attention.go:423-445 */
void sgo_mean_pool_partial(float *dst, const float *src, int S, int emb, int out_dim) {
  if (out_dim > emb) out_dim = emb;
  for (int i = 0; i < out_dim; i++) dst[i] = 0.0f;
  for (int s = 0; s < S; s++)
    for (int i = 0; i < out_dim; i++) dst[i] = dst[i] + src[(int64_t)s * emb + i];
  float sc = 1.0f / (float)S;
  for (int i = 0; i < out_dim; i++) dst[i] = dst[i] * sc;
}

/* runtime/model.go:808-820 */
void sgo_l2_normalize(float *v, int n) {
  float ss = 0.0f;
  for (int i = 0; i < n; i++) { float t = v[i] * v[i]; ss = ss + t; }
  if (ss == 0.0f) return;
  float nrm = (float)sqrt((double)ss);
  for (int i = 0; i < n; i++) v[i] = v[i] / nrm;
}

/* gguf/tensor.go:157-178 with ParseQ8_0Block :94-112 (halving converter) */
void sgo_dequant_q8_0_row(float *dst, const uint8_t *row, int n) {
  int nb = (n + 31) / 32;
  for (int b = 0; b < nb; b++) {
    const uint8_t *blk = row + (int64_t)b * 34;
    float d = f16_halving(rd_u16(blk));
    int e = (b + 1) * 32 < n ? (b + 1) * 32 : n;
    for (int i = b * 32; i < e; i++) dst[i] = (float)(int8_t)blk[2 + i - b * 32] * d;
  }
}

/* --------------------------------------------------------------- model ---- */

typedef struct {
  const uint8_t *w;
  float *scales;
  int rows, cols;
} q8w;

struct sgo_model {
  sgo_config cfg;
  const uint8_t *token_embd;
  const float *output_norm;
  sgo_layer *layers;
  q8w *lw; /* 7 per layer: q k v o gate up down */
  float *freqs, *cos_tab, *sin_tab;
};

static void q8w_init(q8w *t, const uint8_t *w, int rows, int cols) {
  t->w = w; t->rows = rows; t->cols = cols;
  t->scales = (float *)malloc(sizeof(float) * (size_t)rows * (size_t)(cols / 32));
  sgo_extract_q8_0_scales(w, rows, cols, t->scales);
}

sgo_model *sgo_model_create(const sgo_config *cfg, const uint8_t *token_embd,
                            const float *output_norm, const sgo_layer *layers) {
  sgo_model *m = (sgo_model *)calloc(1, sizeof(sgo_model));
  m->cfg = *cfg;
  m->token_embd = token_embd;
  m->output_norm = output_norm;
  int L = cfg->num_layers, d = cfg->embed_dim, kv = cfg->num_kv_heads * cfg->head_dim, ff = cfg->interm_dim;
  m->layers = (sgo_layer *)malloc(sizeof(sgo_layer) * (size_t)L);
  memcpy(m->layers, layers, sizeof(sgo_layer) * (size_t)L);
  m->lw = (q8w *)calloc((size_t)L * 7, sizeof(q8w));
  for (int l = 0; l < L; l++) {
    const sgo_layer *ly = &layers[l];
    q8w *t = m->lw + l * 7;
    q8w_init(&t[0], ly->attn_q, cfg->num_heads * cfg->head_dim, d);
    q8w_init(&t[1], ly->attn_k, kv, d);
    q8w_init(&t[2], ly->attn_v, kv, d);
    q8w_init(&t[3], ly->attn_output, d, cfg->num_heads * cfg->head_dim);
    q8w_init(&t[4], ly->ffn_gate, ff, d);
    q8w_init(&t[5], ly->ffn_up, ff, d);
    q8w_init(&t[6], ly->ffn_down, d, ff);
  }
  int half = cfg->head_dim / 2;
  m->freqs = (float *)malloc(sizeof(float) * (size_t)half);
  m->cos_tab = (float *)malloc(sizeof(float) * (size_t)half * (size_t)cfg->max_seq_len);
  m->sin_tab = (float *)malloc(sizeof(float) * (size_t)half * (size_t)cfg->max_seq_len);
  sgo_rope_cache(m->freqs, m->cos_tab, m->sin_tab, cfg->head_dim, cfg->rope_base, cfg->max_seq_len);
  return m;
}

void sgo_model_free(sgo_model *m) {
  if (!m) return;
  for (int i = 0; i < m->cfg.num_layers * 7; i++) free(m->lw[i].scales);
  free(m->lw); free(m->layers); free(m->freqs); free(m->cos_tab); free(m->sin_tab);
  free(m);
}

static void norm_rows(float *h, const float *w, int rows, int n, float eps) {
  if (!w) return; /* `if len(weight) > 0` guards, model_int8.go:203,225,236 */
  for (int r = 0; r < rows; r++) sgo_rmsnorm(h + (int64_t)r * n, h + (int64_t)r * n, w, n, eps);
}

static void gemm_seq(float *dst, const q8w *t, const int8_t *x, float xs, int S, float *rs, int order) {
  for (int i = 0; i < S; i++) rs[i] = xs;
  sgo_matmul_q8_0_int8(dst, t->w, t->scales, x, rs, S, t->cols, t->rows, order);
}

/* forwardINT8WithDim, runtime/model_int8.go:148-256; runAttentionINT8 :349-507;
 * runMLPINT8 :510-538.  `tp` (may be NULL) adds the taps of sgo_forward_taps:
 * row r of layer l of a tap array sits at row l * tp->layer_rows + r. */
static int forward_core(const sgo_model *m, const int32_t *tokens, int S, int target_dim,
                        float *out, int order, int stop_layer, const sgo_taps *tp) {
  const sgo_config *c = &m->cfg;
  int d = c->embed_dim, H = c->num_heads, HKV = c->num_kv_heads, hd = c->head_dim;
  int qd = H * hd, kvd = HKV * hd, ff = c->interm_dim, nqkv = qd + 2 * kvd;
  if (target_dim <= 0 || target_dim > d) return -4; /* ForwardWithDim model.go:661-667 */
  if (S == 0) return -1;
  if (S > c->max_seq_len) return -2;
  for (int i = 0; i < S; i++)
    if (tokens[i] < 0 || tokens[i] >= c->vocab_size) return -3;

  size_t Sd = (size_t)S * (size_t)d;
  float *hidden = (float *)malloc(sizeof(float) * Sd);
  float *resid = (float *)malloc(sizeof(float) * Sd);
  float *q = (float *)malloc(sizeof(float) * (size_t)S * qd);
  float *k = (float *)malloc(sizeof(float) * (size_t)S * kvd);
  float *v = (float *)malloc(sizeof(float) * (size_t)S * kvd);
  float *att = (float *)malloc(sizeof(float) * (size_t)S * qd);
  float *gate = (float *)malloc(sizeof(float) * (size_t)S * ff);
  float *up = (float *)malloc(sizeof(float) * (size_t)S * ff);
  int8_t *xq = (int8_t *)malloc((size_t)S * (size_t)(ff > qd ? (ff > d ? ff : d) : (qd > d ? qd : d)));
  float *rs = (float *)malloc(sizeof(float) * (size_t)S);

  /* embedding :166-184 */
  int64_t row_bytes = (int64_t)((d + 31) / 32) * 34;
  for (int i = 0; i < S; i++)
    sgo_dequant_q8_0_row(hidden + (int64_t)i * d, m->token_embd + (int64_t)tokens[i] * row_bytes, d);
  float sf = (float)sqrt((double)d);
  for (size_t i = 0; i < Sd; i++) hidden[i] = hidden[i] * sf;

  int L = stop_layer >= 0 && stop_layer < c->num_layers ? stop_layer : c->num_layers;
  float eps = c->norm_eps;
  for (int l = 0; l < L; l++) {
    const sgo_layer *ly = &m->layers[l];
    const q8w *t = m->lw + l * 7;
    int tap = tp && l < tp->n_layers;
    int64_t lrow = tap ? (int64_t)l * tp->layer_rows : 0;
    memcpy(resid, hidden, sizeof(float) * Sd);
    norm_rows(hidden, ly->attn_norm, S, d, eps);
    float xs = sgo_quantize_symmetric(hidden, (int64_t)Sd, xq);
    /* runAttentionINT8 */
    gemm_seq(q, &t[0], xq, xs, S, rs, order);
    gemm_seq(k, &t[1], xq, xs, S, rs, order);
    gemm_seq(v, &t[2], xq, xs, S, rs, order);
    if (tap && tp->qkv)
      for (int s = 0; s < S; s++) {
        float *dst = tp->qkv + (lrow + s) * nqkv;
        memcpy(dst, q + (int64_t)s * qd, sizeof(float) * qd);
        memcpy(dst + qd, k + (int64_t)s * kvd, sizeof(float) * kvd);
        memcpy(dst + qd + kvd, v + (int64_t)s * kvd, sizeof(float) * kvd);
      }
    if (ly->attn_q_norm)
      for (int s = 0; s < S; s++)
        for (int h = 0; h < H; h++) {
          float *p = q + (int64_t)s * qd + h * hd;
          sgo_rmsnorm(p, p, ly->attn_q_norm, hd, eps);
        }
    if (ly->attn_k_norm)
      for (int s = 0; s < S; s++)
        for (int h = 0; h < HKV; h++) {
          float *p = k + (int64_t)s * kvd + h * hd;
          sgo_rmsnorm(p, p, ly->attn_k_norm, hd, eps);
        }
    sgo_rope_apply(q, S, H, hd, m->cos_tab, m->sin_tab);
    sgo_rope_apply(k, S, HKV, hd, m->cos_tab, m->sin_tab);
    float ascale = 1.0f / (float)sqrt((double)hd); /* model.go:475 */
    if (!(tap && tp->att_in) || tp->att) {
      sgo_attention(att, q, k, v, S, H, HKV, hd, ascale);
      if (tap && tp->att) memcpy(tp->att + lrow * qd, att, sizeof(float) * (size_t)S * qd);
    }
    /* teacher forcing: the rest of the layer runs on the injected attention output */
    if (tap && tp->att_in) memcpy(att, tp->att_in + lrow * qd, sizeof(float) * (size_t)S * qd);
    float as = sgo_quantize_symmetric(att, (int64_t)S * qd, xq);
    gemm_seq(hidden, &t[3], xq, as, S, rs, order);
    norm_rows(hidden, ly->post_attention_norm, S, d, eps);
    for (size_t i = 0; i < Sd; i++) hidden[i] = hidden[i] + resid[i];
    /* MLP */
    memcpy(resid, hidden, sizeof(float) * Sd);
    norm_rows(hidden, ly->ffn_norm, S, d, eps);
    xs = sgo_quantize_symmetric(hidden, (int64_t)Sd, xq);
    gemm_seq(gate, &t[4], xq, xs, S, rs, order);
    gemm_seq(up, &t[5], xq, xs, S, rs, order);
    sgo_gelu_quick(gate, gate, (int64_t)S * ff);
    for (int64_t i = 0; i < (int64_t)S * ff; i++) gate[i] = gate[i] * up[i];
    float gs = sgo_quantize_symmetric(gate, (int64_t)S * ff, xq);
    gemm_seq(hidden, &t[6], xq, gs, S, rs, order);
    norm_rows(hidden, ly->post_ffw_norm, S, d, eps);
    for (size_t i = 0; i < Sd; i++) hidden[i] = hidden[i] + resid[i];
    if (tap && tp->h) memcpy(tp->h + lrow * d, hidden, sizeof(float) * Sd);
  }

  if (L < c->num_layers || stop_layer == c->num_layers) {
    memcpy(out, hidden, sizeof(float) * Sd);
  } else {
    norm_rows(hidden, m->output_norm, S, d, eps);
    sgo_mean_pool_partial(out, hidden, S, d, target_dim);
    sgo_l2_normalize(out, target_dim);
  }
  free(hidden); free(resid); free(q); free(k); free(v); free(att); free(gate); free(up);
  free(xq); free(rs);
  return 0;
}

int sgo_forward(const sgo_model *m, const int32_t *tokens, int S, int target_dim,
                float *out, int order, int stop_layer) {
  return forward_core(m, tokens, S, target_dim, out, order, stop_layer, NULL);
}

typedef struct {
  const sgo_model *m;
  const int32_t *tokens, *off;
  int begin, end, dim, order;
  float *out;
  const sgo_taps *taps; /* packed over the batch; NULL: none */
  int err;
} fwd_job;

static void *fwd_worker(void *p) {
  fwd_job *j = (fwd_job *)p;
  const sgo_config *c = &j->m->cfg;
  int qd = c->num_heads * c->head_dim, nqkv = qd + 2 * c->num_kv_heads * c->head_dim;
  for (int s = j->begin; s < j->end; s++) {
    sgo_taps t, *tp = NULL;
    if (j->taps) { /* this sequence's rows of every packed tap array */
      int64_t r0 = j->off[s];
      t = *j->taps;
      if (t.att_in) t.att_in += r0 * qd;
      if (t.qkv) t.qkv += r0 * nqkv;
      if (t.att) t.att += r0 * qd;
      if (t.h) t.h += r0 * c->embed_dim;
      tp = &t;
    }
    int r = forward_core(j->m, j->tokens + j->off[s], j->off[s + 1] - j->off[s], j->dim,
                         j->out + (int64_t)s * j->dim, j->order, -1, tp);
    if (r && !j->err) j->err = r;
  }
  return NULL;
}

/* embedPrompts api.go:237-295: workers = min(n_threads, n), contiguous ranges */
static int forward_batch(const sgo_model *m, const int32_t *tokens, const int32_t *off,
                         int n, int dim, float *out, int order, int n_threads, const sgo_taps *taps) {
  if (n <= 0) return 0;
  int workers = n_threads < n ? n_threads : n;
  if (workers < 1) workers = 1;
  int per = (n + workers - 1) / workers;
  fwd_job *jobs = (fwd_job *)calloc((size_t)workers, sizeof(fwd_job));
  pthread_t *th = (pthread_t *)calloc((size_t)workers, sizeof(pthread_t));
  int used = 0;
  for (int w = 0; w < workers; w++) {
    int b = w * per, e = b + per < n ? b + per : n;
    if (b >= n) break;
    jobs[w] = (fwd_job){m, tokens, off, b, e, dim, order, out, taps, 0};
    pthread_create(&th[w], NULL, fwd_worker, &jobs[w]);
    used++;
  }
  int err = 0;
  for (int w = 0; w < used; w++) {
    pthread_join(th[w], NULL);
    if (jobs[w].err && !err) err = jobs[w].err;
  }
  free(jobs); free(th);
  return err;
}

int sgo_forward_batch(const sgo_model *m, const int32_t *tokens, const int32_t *off,
                      int n, int dim, float *out, int order, int n_threads) {
  return forward_batch(m, tokens, off, n, dim, out, order, n_threads, NULL);
}

int sgo_forward_taps(const sgo_model *m, const int32_t *tokens, const int32_t *off,
                     int n, int dim, float *out, int order, int n_threads, const sgo_taps *taps) {
  return forward_batch(m, tokens, off, n, dim, out, order, n_threads, taps);
}
