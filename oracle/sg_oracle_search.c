/*
 * sg_oracle_search.c -- CPU restatement of go-semantica's brute-force vector
 * search (search/brute), TEST INFRASTRUCTURE ONLY: the checker the GPU index
 * is compared against.  Only tests/ and bench.py's cpu_baseline leg load it.
 *
 * Arithmetic follows the amd64 path of the reference (AVX2 + FMA present):
 *   normalize        search/brute/builder.go:131-141
 *   quantizeInt8/16  search/brute/quant.go:17-41
 *   dotInt8/16       search/brute/quant.go:79-135 + dot_amd64.s:12-73
 *   dotFloat32       search/brute/index.go:199-214 + dot_amd64.s:75-105
 *   searchNormalized search/brute/index.go:53-147
 * The 8-lane loops keep one accumulator per lane (lane j takes elements
 * j, j+8, ...) and reduce them as VEXTRACTF128 + VADDPS + 2x VHADDPS do:
 * ((l0+l4)+(l1+l5)) + ((l2+l6)+(l3+l7)).
 */
#include "sg_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* builder.go:131-141: float64 sum of float32 squares, then one float32 scale. */
void sgo_bf_normalize(float *v, int dim) {
  double sum = 0.0;
  for (int i = 0; i < dim; i++) {
    const float sq = v[i] * v[i];
    sum += (double)sq;
  }
  if (sum == 0.0) return;
  const float norm = (float)(1.0 / sqrt(sum));
  for (int i = 0; i < dim; i++) v[i] *= norm;
}

static float clamp1(float v) { return v > 1.0f ? 1.0f : (v < -1.0f ? -1.0f : v); }

/* quant.go:17-29 / 31-41: clamp to [-1, 1], math.Round(float64(v) * 127). */
void sgo_bf_quantize_i8(const float *v, int dim, int8_t *out) {
  for (int i = 0; i < dim; i++) out[i] = (int8_t)round((double)clamp1(v[i]) * 127.0);
}
void sgo_bf_quantize_i16(const float *v, int dim, int16_t *out) {
  for (int i = 0; i < dim; i++) out[i] = (int16_t)round((double)clamp1(v[i]) * 32767.0);
}

static float hsum8(const float *l) { return ((l[0] + l[4]) + (l[1] + l[5])) + ((l[2] + l[6]) + (l[3] + l[7])); }

/* dotInt8 / dotInt16 (quant.go:79-135).  The AVX2 part (dot_amd64.s:12-73)
 * converts, scales by inv (float32(1/127) or float32(1/32767)), multiplies by
 * the query and adds, each step rounded; the scalar tail goes through the
 * lookup tables (quant.go:57-77), which clamp the most negative code. */
static float dot_q(const void *vec, int bytes, const float *q, int dim) {
  const float inv = bytes == 1 ? (float)(1.0 / 127.0) : (float)(1.0 / 32767.0);
  const int8_t *v8 = (const int8_t *)vec;
  const int16_t *v16 = (const int16_t *)vec;
#define SGO_Q(i) (bytes == 1 ? (int)v8[i] : (int)v16[i])
  float sum = 0.0f;
  int i0 = 0;
  if (dim >= 8) {
    const int n = dim & ~7;
    float l[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int i = 0; i < n; i += 8)
      for (int j = 0; j < 8; j++) {
        const float d = (float)SGO_Q(i + j) * inv;
        const float p = d * q[i + j];
        l[j] = l[j] + p;
      }
    sum += hsum8(l);
    i0 = n;
  }
  const int lo = bytes == 1 ? -127 : -32767;
  float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
  int i = i0;
  for (; i + 4 <= dim; i += 4) {
    int c0 = SGO_Q(i), c1 = SGO_Q(i + 1), c2 = SGO_Q(i + 2), c3 = SGO_Q(i + 3);
    c0 = c0 < lo ? lo : c0; c1 = c1 < lo ? lo : c1; c2 = c2 < lo ? lo : c2; c3 = c3 < lo ? lo : c3;
    s0 += q[i] * ((float)c0 * inv);
    s1 += q[i + 1] * ((float)c1 * inv);
    s2 += q[i + 2] * ((float)c2 * inv);
    s3 += q[i + 3] * ((float)c3 * inv);
  }
  sum += s0 + s1 + s2 + s3;
  for (; i < dim; i++) {
    int c = SGO_Q(i);
    c = c < lo ? lo : c;
    sum += q[i] * ((float)c * inv);
  }
#undef SGO_Q
  return sum;
}

float sgo_bf_dot_i8(const int8_t *vec, const float *q, int dim) { return dot_q(vec, 1, q, dim); }
float sgo_bf_dot_i16(const int16_t *vec, const float *q, int dim) { return dot_q(vec, 2, q, dim); }

/* dotFloat32 (index.go:199-214): VFMADD231PS per lane (dot_amd64.s:85-95),
 * the same reduction, then sum += a*b for the rest (two roundings each). */
float sgo_bf_dot_f32(const float *a, const float *b, int dim) {
  float sum = 0.0f;
  int i0 = 0;
  if (dim >= 8) {
    const int n = dim & ~7;
    float l[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int i = 0; i < n; i += 8)
      for (int j = 0; j < 8; j++) l[j] = fmaf(a[i + j], b[i + j], l[j]);
    sum += hsum8(l);
    i0 = n;
  }
  for (int i = i0; i < dim; i++) {
    const float p = a[i] * b[i];
    sum += p;
  }
  return sum;
}

float sgo_bf_dot(const void *data, int mode, int64_t row, const float *q, int dim) {
  switch (mode) {
    case SGO_BF_F32: return sgo_bf_dot_f32((const float *)data + row * dim, q, dim);
    case SGO_BF_I8: return sgo_bf_dot_i8((const int8_t *)data + row * dim, q, dim);
    default: return sgo_bf_dot_i16((const int16_t *)data + row * dim, q, dim);
  }
}

typedef struct {
  int idx;
  float dist;
  int32_t id;
} cand;

static int cand_cmp(const void *pa, const void *pb) {
  const cand *a = (const cand *)pa, *b = (const cand *)pb;
  if (a->dist == b->dist) return a->id < b->id ? -1 : (a->id > b->id ? 1 : 0);
  return a->dist > b->dist ? -1 : 1;
}

/* searchNormalized (index.go:53-147): a streaming top-k over the stored order
 * -- the first k candidates fill the list, later ones replace the current
 * minimum (the first slot holding it) only when strictly larger -- then the
 * list sorted by distance descending, ties by id ascending.  Returns the
 * number of results, min(top_k, count); top_k <= 0 returns -1. */
int sgo_bf_search(const void *data, int mode, const int32_t *ids, int count, int dim, const float *query,
                  int top_k, int32_t *out_ids, float *out_dist) {
  if (top_k <= 0) return -1;
  if (top_k > count) top_k = count;
  if (top_k == 0) return 0;
  cand *best = (cand *)malloc(sizeof(cand) * (size_t)top_k);
  int n = 0, min_idx = -1;
  float min_dist = 1.0f;
  for (int i = 0; i < count; i++) {
    const float d = sgo_bf_dot(data, mode, i, query, dim);
    if (n < top_k) {
      best[n].idx = i;
      best[n].dist = d;
      n++;
      if (n == top_k) {
        min_idx = 0;
        min_dist = best[0].dist;
        for (int j = 1; j < n; j++)
          if (best[j].dist < min_dist) { min_dist = best[j].dist; min_idx = j; }
      }
      continue;
    }
    if (d <= min_dist) continue;
    best[min_idx].idx = i;
    best[min_idx].dist = d;
    min_idx = 0;
    min_dist = best[0].dist;
    for (int j = 1; j < n; j++)
      if (best[j].dist < min_dist) { min_dist = best[j].dist; min_idx = j; }
  }
  for (int j = 0; j < n; j++) best[j].id = ids[best[j].idx];
  qsort(best, (size_t)n, sizeof(cand), cand_cmp);
  for (int j = 0; j < n; j++) {
    out_ids[j] = best[j].id;
    out_dist[j] = best[j].dist;
  }
  free(best);
  return n;
}
