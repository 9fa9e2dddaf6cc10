// k_search.hip -- brute-force vector search (search/brute) for gfx950: index
// build (normalize + quantize), scoring of every stored vector against a
// batch of queries, and the exact top-k selection.
//
// Index layout in HBM.  The reference stores vectors row-major [N][dim]
// (index.go:11-25).  Here the first 8*G elements of every vector (G = dim/8)
// are stored as [G][N][8] -- group g of all vectors contiguous -- so the lane
// that scores vector n reads its group g with one 8/16/32-byte load and a
// wave's loads are 512 contiguous bytes (int8).  The last R = dim % 8
// elements of each vector sit in a tail array [N][R].  Groups follow the
// reference's 8-lane split exactly: lane j of the AVX2 loop owns elements
// 8g + j, and the tail is what its scalar loop handles.
//
// Arithmetic (bit-exact to the amd64 AVX2 path of the reference):
//   int8/int16  d = float(q) * inv  (inv = float32(1/127) / float32(1/32767)),
//               acc_j = acc_j + d * x  (three roundings, dot_amd64.s:24-34,52-62)
//   float32     acc_j = fma(v, x, acc_j)  (dot_amd64.s:85-95)
//   reduction   ((l0+l4)+(l1+l5)) + ((l2+l6)+(l3+l7))  (VEXTRACTF128/VADDPS/2xVHADDPS)
//   tail        int modes: one unrolled group of 4 partial sums, then singles,
//               through the clamping lookup tables (quant.go:57-135);
//               float32: sum += a*b (index.go:209-212)
#include "sg_device.h"
#include "sg_kernels.h"

namespace {

constexpr int kBfThreads = 256;

template <typename T>
struct BfElem;
template <>
struct BfElem<int8_t> {
  static constexpr bool kQuant = true;
  static constexpr int kLo = -127;
  __device__ static float inv() { return (float)(1.0 / 127.0); }
  __device__ static double scale() { return 127.0; }
};
template <>
struct BfElem<int16_t> {
  static constexpr bool kQuant = true;
  static constexpr int kLo = -32767;
  __device__ static float inv() { return (float)(1.0 / 32767.0); }
  __device__ static double scale() { return 32767.0; }
};
template <>
struct BfElem<float> {
  static constexpr bool kQuant = false;
};

// One group of 8 stored elements as loaded (8, 16 or 32 bytes), and its
// conversion to the AVX2 loop's per-lane operand (no clamp: VPMOVSX +
// VCVTDQ2PS take the code as it is; then the scale multiply, rounded).
template <typename T>
struct BfRaw;
template <>
struct BfRaw<int8_t> {
  uint2 w;
  __device__ void load(const int8_t* p) { w = *reinterpret_cast<const uint2*>(p); }
  __device__ void get(float (&v)[8]) const {
#pragma unroll
    for (int l = 0; l < 4; l++) {
      v[l] = (float)(int8_t)(w.x >> (8 * l)) * BfElem<int8_t>::inv();
      v[4 + l] = (float)(int8_t)(w.y >> (8 * l)) * BfElem<int8_t>::inv();
    }
  }
};
template <>
struct BfRaw<int16_t> {
  uint4 w;
  __device__ void load(const int16_t* p) { w = *reinterpret_cast<const uint4*>(p); }
  __device__ void get(float (&v)[8]) const {
    const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int l = 0; l < 4; l++) {
      v[2 * l] = (float)(int16_t)(u[l] & 0xffffu) * BfElem<int16_t>::inv();
      v[2 * l + 1] = (float)(int16_t)(u[l] >> 16) * BfElem<int16_t>::inv();
    }
  }
};
template <>
struct BfRaw<float> {
  float4 a, b;
  __device__ void load(const float* p) {
    a = *reinterpret_cast<const float4*>(p);
    b = *reinterpret_cast<const float4*>(p + 4);
  }
  __device__ void get(float (&v)[8]) const {
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  }
};

// Tail element through the lookup table of quant.go:57-77 (the most negative
// code clamps to -127 / -32767).
template <typename T>
__device__ __forceinline__ float bf_lut(T c) {
  int v = (int)c;
  v = v < BfElem<T>::kLo ? BfElem<T>::kLo : v;
  return (float)v * BfElem<T>::inv();
}

// ------------------------------------------------------------------ build --

// builder.go:131-141 on one row: float64 sum of the float32 squares in index
// order, norm = float32(1/sqrt(sum)), v *= norm (a zero vector stays as is);
// then quant.go:17-41: clamp to [-1, 1] and math.Round(float64(v) * 127 or
// 32767) (the product is exact in float64, so C round() of it is the same).
// One thread per vector (the float64 sum is sequential by definition).
template <typename T>
__global__ __launch_bounds__(kBfThreads) void k_bf_build(const float* __restrict__ src, int64_t ld, int n, int dim,
                                                        int row0, int N, T* __restrict__ grp, T* __restrict__ tail,
                                                        int normalize) {
  const int r = blockIdx.x * kBfThreads + threadIdx.x;
  if (r >= n) return;
  const float* v = src + (int64_t)r * ld;
  float norm = 1.0f;
  bool scale = false;
  if (normalize) {
    double sum = 0.0;
    for (int i = 0; i < dim; i++) {
      const float sq = v[i] * v[i];
      sum += (double)sq;
    }
    if (sum != 0.0) {
      norm = (float)(1.0 / sqrt(sum));
      scale = true;
    }
  }
  const int G = dim >> 3, R = dim & 7;
  const int64_t row = row0 + r;
  for (int i = 0; i < dim; i++) {
    float x = v[i];
    if (scale) x = x * norm;
    T q;
    if constexpr (BfElem<T>::kQuant) {
      x = x > 1.0f ? 1.0f : (x < -1.0f ? -1.0f : x);
      q = (T)round((double)x * BfElem<T>::scale());
    } else {
      q = x;
    }
    const int g = i >> 3;
    if (g < G)
      grp[((int64_t)g * N + row) * 8 + (i & 7)] = q;
    else
      tail[row * R + (i & 7)] = q;
  }
}

// builder.go:131-141 in place on rows of x (the queries of SearchVector,
// index.go:36-38).  One wave per row: the row is staged in LDS with
// coalesced loads, lane 0 runs the float64 sum in index order, and all lanes
// scale.
constexpr int kNormChunk = 1024;

__global__ __launch_bounds__(64) void k_bf_normalize(float* __restrict__ x, int dim) {
  __shared__ float buf[kNormChunk];
  __shared__ float norm;
  __shared__ int scale;
  float* v = x + (int64_t)blockIdx.x * dim;
  const int lane = threadIdx.x;
  double sum = 0.0;
  for (int c0 = 0; c0 < dim; c0 += kNormChunk) {
    const int cn = min(kNormChunk, dim - c0);
    for (int i = lane; i < cn; i += 64) buf[i] = v[c0 + i];
    __syncthreads();
    if (lane == 0)
      for (int i = 0; i < cn; i++) {
        const float sq = buf[i] * buf[i];
        sum += (double)sq;
      }
    __syncthreads();
  }
  if (lane == 0) {
    scale = sum != 0.0;
    norm = sum != 0.0 ? (float)(1.0 / sqrt(sum)) : 1.0f;
  }
  __syncthreads();
  if (!scale) return;
  for (int i = lane; i < dim; i += 64) v[i] = v[i] * norm;
}

// Stored rows (row-major, as serialized) -> the grouped layout, and back.
template <typename T>
__global__ void k_bf_relayout(const T* __restrict__ rows, int64_t n_elems, int dim, int row0, int N,
                              T* __restrict__ grp, T* __restrict__ tail) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= n_elems) return;
  const int64_t row = row0 + e / dim;
  const int i = (int)(e % dim);
  const int G = dim >> 3, R = dim & 7;
  const int g = i >> 3;
  if (g < G)
    grp[((int64_t)g * N + row) * 8 + (i & 7)] = rows[e];
  else
    tail[row * R + (i & 7)] = rows[e];
}

template <typename T>
__global__ void k_bf_unpack(const T* __restrict__ grp, const T* __restrict__ tail, int64_t n_elems, int dim,
                            int row0, int N, T* __restrict__ rows) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= n_elems) return;
  const int64_t row = row0 + e / dim;
  const int i = (int)(e % dim);
  const int G = dim >> 3, R = dim & 7;
  const int g = i >> 3;
  rows[e] = g < G ? grp[((int64_t)g * N + row) * 8 + (i & 7)] : tail[row * R + (i & 7)];
}

// ---------------------------------------------------------------- scoring --

// scores[q][n] for QB queries (rows q0.. of `queries`, already normalized)
// against every stored vector; lane = vector.  The workgroup stages the
// queries in LDS, kQChunk dimensions at a time, and every lane reads them by
// broadcast; each lane issues the loads of kBfBatch groups before using them.
constexpr int kQChunk = 256;
// Groups loaded together per lane: 32 bytes of int8 / int16, 64 of float32.
template <typename T>
constexpr int kBfBatch = sizeof(T) == 1 ? 4 : 2;

template <typename T, int QB>
__global__ __launch_bounds__(kBfThreads) void k_bf_score(const T* __restrict__ grp, const T* __restrict__ tail,
                                                        int N, int dim, const float* __restrict__ queries, int q0,
                                                        int nq, float* __restrict__ scores, int64_t ld_scores) {
  __shared__ __attribute__((aligned(16))) float qs[QB][kQChunk];
  const int n = blockIdx.x * kBfThreads + threadIdx.x;
  const bool live = n < N;
  const int nn = live ? n : N - 1;  // lanes past the end load a valid vector and store nothing
  const int G = dim >> 3, R = dim & 7;

  float acc[QB][8];
#pragma unroll
  for (int j = 0; j < QB; j++)
#pragma unroll
    for (int l = 0; l < 8; l++) acc[j][l] = 0.0f;

  const T* gp = grp + (int64_t)nn * 8;
  const int64_t gstride = (int64_t)N * 8;
  for (int c0 = 0; c0 < 8 * G; c0 += kQChunk) {
    const int cn = min(kQChunk, 8 * G - c0);
    __syncthreads();  // the previous chunk's reads are done
    for (int e = threadIdx.x; e < QB * cn; e += kBfThreads) {
      const int j = e / cn, i = e - j * cn;
      qs[j][i] = queries[(int64_t)min(q0 + j, nq - 1) * dim + c0 + i];
    }
    __syncthreads();
    const int g0 = c0 >> 3, gn = cn >> 3;
    for (int g = 0; g < gn; g += kBfBatch<T>) {
      BfRaw<T> raw[kBfBatch<T>];  // all of a batch's loads in flight at once
#pragma unroll
      for (int u = 0; u < kBfBatch<T>; u++)
        if (g + u < gn) raw[u].load(gp + (g0 + g + u) * gstride);
#pragma unroll
      for (int u = 0; u < kBfBatch<T>; u++) {
        if (g + u >= gn) break;
        float v[8];
        raw[u].get(v);
#pragma unroll
        for (int j = 0; j < QB; j++) {
          const float4 xa = *reinterpret_cast<const float4*>(&qs[j][8 * (g + u)]);
          const float4 xb = *reinterpret_cast<const float4*>(&qs[j][8 * (g + u) + 4]);
          const float x[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
#pragma unroll
          for (int l = 0; l < 8; l++) {
            if constexpr (BfElem<T>::kQuant) {
              const float p = v[l] * x[l];
              acc[j][l] = acc[j][l] + p;
            } else {
              acc[j][l] = __builtin_fmaf(v[l], x[l], acc[j][l]);
            }
          }
        }
      }
    }
  }
  if (!live) return;

  const T* tp = tail + (int64_t)n * R;
#pragma unroll
  for (int j = 0; j < QB; j++) {
    if (q0 + j >= nq) break;
    float sum = 0.0f;
    if (G > 0) {
      const float* l = acc[j];
      sum += ((l[0] + l[4]) + (l[1] + l[5])) + ((l[2] + l[6]) + (l[3] + l[7]));
    }
    const float* x = queries + (int64_t)(q0 + j) * dim + 8 * G;
    if constexpr (BfElem<T>::kQuant) {
      float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
      int i = 0;
      if (R >= 4) {
        s0 += x[0] * bf_lut<T>(tp[0]);
        s1 += x[1] * bf_lut<T>(tp[1]);
        s2 += x[2] * bf_lut<T>(tp[2]);
        s3 += x[3] * bf_lut<T>(tp[3]);
        i = 4;
      }
      sum += s0 + s1 + s2 + s3;
      for (; i < R; i++) sum += x[i] * bf_lut<T>(tp[i]);
    } else {
      for (int i = 0; i < R; i++) {
        const float p = (float)tp[i] * x[i];
        sum += p;
      }
    }
    scores[(int64_t)(q0 + j) * ld_scores + n] = sum;
  }
}

// -------------------------------------------------------------- selection --
//
// The reference keeps a k-slot list while streaming the scores in stored
// order (index.go:84-131): the first k fill it; later ones replace the
// current minimum (its first slot) only when strictly larger.  The list
// always holds the k largest values seen, so at the end it holds every score
// above the k-th largest value v_k plus some scores equal to v_k.  When
// exactly k scores are >= v_k the result is that set, whatever the order;
// only a tie straddling the k-th place makes the slot history matter.
// Hence: an exact radix select finds v_k and the counts above / at it; the
// common case collects the >= v_k set in parallel; a query with a straddling
// tie replays the reference's streaming loop (one wave, exact).
//
// Per-query state, int32[8]: 0 prefix (key bits fixed so far), 1 mask,
// 2 k_rem (places left inside the prefix), 3 above (count with key > prefix
// bits decided), 4 at (count in the final bin), 5 done-blocks counter,
// 6 collected, 7 tie flag.

// Order-preserving key of a score; -0 maps with +0 (they compare equal).
__device__ __forceinline__ uint32_t bf_key(float d) {
  const uint32_t u = __float_as_uint(d == 0.0f ? 0.0f : d);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

constexpr int kSelPerThread = 16;
constexpr int kSelBlock = kBfThreads * kSelPerThread;  // scores per workgroup

// One 8-bit digit of the radix select (digit 0 = bits 31..24).  Every
// workgroup histograms its range of one query's scores among the keys that
// match the prefix, adds it to hist[q]; the last workgroup to finish picks the
// bin holding the k-th largest key, updates the state and clears hist[q].
__global__ __launch_bounds__(kBfThreads) void k_bf_radix(const float* __restrict__ scores, int64_t ld_scores,
                                                        int N, int digit, int32_t* __restrict__ state,
                                                        uint32_t* __restrict__ hist) {
  const int q = blockIdx.y;
  const float* s = scores + (int64_t)q * ld_scores;
  int32_t* st = state + 8 * q;
  uint32_t* hq = hist + 256 * q;
  __shared__ uint32_t h[256];
  __shared__ uint32_t suf[256];
  __shared__ int last;
  h[threadIdx.x] = 0;
  const uint32_t prefix = (uint32_t)st[0], mask = (uint32_t)st[1];
  const int shift = 24 - 8 * digit;
  __syncthreads();
  const int base = blockIdx.x * kSelBlock;
  // Scores crowd into a few bins (the top digit holds sign and exponent), so
  // each wave adds its lanes bin by bin: one LDS atomic per distinct bin.
  const int lane = threadIdx.x & 63;
#pragma unroll 4
  for (int t = 0; t < kSelPerThread; t++) {
    const int i = base + t * kBfThreads + threadIdx.x;
    int bin = -1;
    if (i < N) {
      const uint32_t k = bf_key(s[i]);
      if ((k & mask) == prefix) bin = (int)((k >> shift) & 255u);
    }
    uint64_t todo = __ballot(bin >= 0);
    while (todo) {
      const int leader = __builtin_ctzll(todo);
      const int lb = __shfl(bin, leader);
      const uint64_t same = __ballot(bin == lb);
      if (lane == leader) atomicAdd(&h[lb], (uint32_t)__popcll(same));
      todo &= ~same;
    }
  }
  __syncthreads();
  // Every value shared between workgroups here is read and written with
  // device-scope atomics, so ordering needs no cache maintenance: each wave
  // waits until its bin additions are performed before the workgroup counts
  // itself done, and the last workgroup reads the bins with atomic loads.
  // (A __threadfence() per workgroup would write back and invalidate the L2
  // thousands of times per pass.)
  if (h[threadIdx.x]) atomicAdd(&hq[threadIdx.x], h[threadIdx.x]);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0) last = atomicAdd(&st[5], 1) == (int)gridDim.x - 1;
  __syncthreads();
  if (!last) return;
  // suffix sums over the bins, highest first
  const uint32_t c = __hip_atomic_load(&hq[threadIdx.x], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  suf[threadIdx.x] = c;
  __syncthreads();
  for (int off = 1; off < 256; off <<= 1) {
    const uint32_t add = threadIdx.x + off < 256 ? suf[threadIdx.x + off] : 0u;
    __syncthreads();
    suf[threadIdx.x] += add;
    __syncthreads();
  }
  const int k_rem = st[2];
  // the bin b with suf[b+1] < k_rem <= suf[b]
  const uint32_t above = threadIdx.x < 255 ? suf[threadIdx.x + 1] : 0u;
  if ((int64_t)above < k_rem && (int64_t)suf[threadIdx.x] >= k_rem) {
    st[0] = (int32_t)(prefix | ((uint32_t)threadIdx.x << shift));
    st[1] = (int32_t)(mask | (255u << shift));
    st[2] = k_rem - (int)above;
    st[3] += (int)above;
    st[4] = (int)c;
  }
  hq[threadIdx.x] = 0u;
  if (threadIdx.x == 0) st[5] = 0;
}

// Common case (exactly k scores >= v_k): every such score's position and
// value go to out[q][0..k) in arbitrary order.  With a straddling tie the
// query is flagged for k_bf_stream instead.
__global__ __launch_bounds__(kBfThreads) void k_bf_collect(const float* __restrict__ scores, int64_t ld_scores,
                                                          int N, int k, int32_t* __restrict__ state,
                                                          int32_t* __restrict__ out_idx, float* __restrict__ out_dist) {
  const int q = blockIdx.y;
  int32_t* st = state + 8 * q;
  const int above = st[3], at = st[4];
  if (above + at != k) {  // tie straddles the k-th place
    if (blockIdx.x == 0 && threadIdx.x == 0) st[7] = 1;
    return;
  }
  const uint32_t kk = (uint32_t)st[0];
  const float* s = scores + (int64_t)q * ld_scores;
  const int base = blockIdx.x * kSelBlock;
  for (int t = 0; t < kSelPerThread; t++) {
    const int i = base + t * kBfThreads + threadIdx.x;
    if (i < N) {
      const float d = s[i];
      if (bf_key(d) >= kk) {
        const int slot = atomicAdd(&st[6], 1);
        if (slot < k) {
          out_idx[(int64_t)q * k + slot] = i;
          out_dist[(int64_t)q * k + slot] = d;
        }
      }
    }
  }
}

// The reference's streaming loop (index.go:84-131) for the flagged queries,
// one wave each.  The k slots live in out[q]; (min, first slot of the min) is
// kept in registers and recomputed after each replacement.  Scores are read
// 64 at a time; a ballot of "score > min" skips the rejected ones.
__device__ __forceinline__ void bf_min_slot(const float* dist, int k, float& mn, int& mi) {
  const int lane = threadIdx.x;
  float m = __builtin_inff();
  int idx = 0x7fffffff;
  for (int j = lane; j < k; j += 64) {
    const float d = dist[j];
    if (d < m) {  // first slot of the minimum within this lane's slots
      m = d;
      idx = j;
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float m2 = __shfl_xor(m, o);
    const int i2 = __shfl_xor(idx, o);
    if (m2 < m || (m2 == m && i2 < idx)) {
      m = m2;
      idx = i2;
    }
  }
  mn = m;
  mi = idx;
}

__global__ __launch_bounds__(64) void k_bf_stream(const float* __restrict__ scores, int64_t ld_scores, int N, int k,
                                                 const int32_t* __restrict__ state, int32_t* __restrict__ out_idx,
                                                 float* __restrict__ out_dist) {
  const int q = blockIdx.x;
  if (state[8 * q + 7] == 0) return;
  const float* s = scores + (int64_t)q * ld_scores;
  int32_t* oi = out_idx + (int64_t)q * k;
  float* od = out_dist + (int64_t)q * k;
  const int lane = threadIdx.x;
  for (int j = lane; j < k; j += 64) {  // the first k fill the list
    oi[j] = j;
    od[j] = s[j];
  }
  __threadfence_block();
  float mn;
  int mi;
  bf_min_slot(od, k, mn, mi);
  for (int base = k; base < N; base += 64) {
    const int i = base + lane;
    const float d = i < N ? s[i] : -__builtin_inff();
    uint64_t live = __ballot(i < N && d > mn);
    while (live) {
      const int b = __builtin_ctzll(live);
      const float db = __shfl(d, b);
      if (lane == 0) {
        oi[mi] = base + b;
        od[mi] = db;
      }
      __threadfence_block();
      bf_min_slot(od, k, mn, mi);
      live &= ~((2ull << b) - 1ull);  // later lanes only
      live &= __ballot(i < N && d > mn);
    }
  }
}

__global__ void k_bf_fill_i32(int32_t* p, int64_t n, int32_t v) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

// state initial values: prefix 0, mask 0, k_rem k, above 0, at 0, 0, 0, 0.
__global__ void k_bf_state_init(int32_t* state, int nq, int k) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < nq * 8) state[i] = (i & 7) == 2 ? k : 0;
}

unsigned nblocks(int64_t n, int per) { return (unsigned)((n + per - 1) / per); }

template <typename T>
hipError_t score_t(const void* grp, const void* tail, int N, int dim, const float* queries, int nq, float* scores,
                   int64_t ld, hipStream_t s) {
  const T* g = static_cast<const T*>(grp);
  const T* t = static_cast<const T*>(tail);
  const unsigned nb = nblocks(N, kBfThreads);
  for (int q0 = 0; q0 < nq;) {
    const int left = nq - q0;
    if (left >= 8) {
      hipLaunchKernelGGL((k_bf_score<T, 8>), dim3(nb, 1), dim3(kBfThreads), 0, s, g, t, N, dim, queries, q0, nq,
                         scores, ld);
      q0 += 8;
    } else if (left >= 4) {
      hipLaunchKernelGGL((k_bf_score<T, 4>), dim3(nb, 1), dim3(kBfThreads), 0, s, g, t, N, dim, queries, q0, nq,
                         scores, ld);
      q0 += 4;
    } else if (left >= 2) {
      hipLaunchKernelGGL((k_bf_score<T, 2>), dim3(nb, 1), dim3(kBfThreads), 0, s, g, t, N, dim, queries, q0, nq,
                         scores, ld);
      q0 += 2;
    } else {
      hipLaunchKernelGGL((k_bf_score<T, 1>), dim3(nb, 1), dim3(kBfThreads), 0, s, g, t, N, dim, queries, q0, nq,
                         scores, ld);
      q0 += 1;
    }
  }
  return hipGetLastError();
}

}  // namespace

namespace sgk {

hipError_t bf_build(int mode, const float* src, int64_t ld, int n, int dim, int row0, int N, void* grp, void* tail,
                    bool normalize, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  const unsigned nb = nblocks(n, kBfThreads);
  const int nz = normalize ? 1 : 0;
  switch (mode) {
    case kBfF32:
      hipLaunchKernelGGL(k_bf_build<float>, dim3(nb), dim3(kBfThreads), 0, s, src, ld, n, dim, row0, N,
                         static_cast<float*>(grp), static_cast<float*>(tail), nz);
      break;
    case kBfI8:
      hipLaunchKernelGGL(k_bf_build<int8_t>, dim3(nb), dim3(kBfThreads), 0, s, src, ld, n, dim, row0, N,
                         static_cast<int8_t*>(grp), static_cast<int8_t*>(tail), nz);
      break;
    case kBfI16:
      hipLaunchKernelGGL(k_bf_build<int16_t>, dim3(nb), dim3(kBfThreads), 0, s, src, ld, n, dim, row0, N,
                         static_cast<int16_t*>(grp), static_cast<int16_t*>(tail), nz);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t bf_normalize(float* x, int n, int dim, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_bf_normalize, dim3(n), dim3(64), 0, s, x, dim);
  return hipGetLastError();
}

hipError_t bf_relayout(int mode, const void* rows, int n, int dim, int row0, int N, void* grp, void* tail,
                       hipStream_t s) {
  const int64_t ne = (int64_t)n * dim;
  if (ne <= 0) return hipSuccess;
  const unsigned nb = nblocks(ne, 256);
  switch (mode) {
    case kBfF32:
      hipLaunchKernelGGL(k_bf_relayout<float>, dim3(nb), dim3(256), 0, s, static_cast<const float*>(rows), ne, dim,
                         row0, N, static_cast<float*>(grp), static_cast<float*>(tail));
      break;
    case kBfI8:
      hipLaunchKernelGGL(k_bf_relayout<int8_t>, dim3(nb), dim3(256), 0, s, static_cast<const int8_t*>(rows), ne,
                         dim, row0, N, static_cast<int8_t*>(grp), static_cast<int8_t*>(tail));
      break;
    case kBfI16:
      hipLaunchKernelGGL(k_bf_relayout<int16_t>, dim3(nb), dim3(256), 0, s, static_cast<const int16_t*>(rows), ne,
                         dim, row0, N, static_cast<int16_t*>(grp), static_cast<int16_t*>(tail));
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t bf_unpack(int mode, const void* grp, const void* tail, int row0, int n, int dim, int N, void* rows,
                     hipStream_t s) {
  const int64_t ne = (int64_t)n * dim;
  if (ne <= 0) return hipSuccess;
  const unsigned nb = nblocks(ne, 256);
  switch (mode) {
    case kBfF32:
      hipLaunchKernelGGL(k_bf_unpack<float>, dim3(nb), dim3(256), 0, s, static_cast<const float*>(grp),
                         static_cast<const float*>(tail), ne, dim, row0, N, static_cast<float*>(rows));
      break;
    case kBfI8:
      hipLaunchKernelGGL(k_bf_unpack<int8_t>, dim3(nb), dim3(256), 0, s, static_cast<const int8_t*>(grp),
                         static_cast<const int8_t*>(tail), ne, dim, row0, N, static_cast<int8_t*>(rows));
      break;
    case kBfI16:
      hipLaunchKernelGGL(k_bf_unpack<int16_t>, dim3(nb), dim3(256), 0, s, static_cast<const int16_t*>(grp),
                         static_cast<const int16_t*>(tail), ne, dim, row0, N, static_cast<int16_t*>(rows));
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t bf_score(int mode, const void* grp, const void* tail, int N, int dim, const float* queries, int nq,
                    float* scores, int64_t ld_scores, hipStream_t s) {
  if (N <= 0 || nq <= 0) return hipSuccess;
  switch (mode) {
    case kBfF32: return score_t<float>(grp, tail, N, dim, queries, nq, scores, ld_scores, s);
    case kBfI8: return score_t<int8_t>(grp, tail, N, dim, queries, nq, scores, ld_scores, s);
    case kBfI16: return score_t<int16_t>(grp, tail, N, dim, queries, nq, scores, ld_scores, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t bf_select(const float* scores, int64_t ld_scores, int N, int nq, int k, int32_t* state, uint32_t* hist,
                     int32_t* out_idx, float* out_dist, hipStream_t s) {
  if (N <= 0 || nq <= 0 || k <= 0) return hipSuccess;
  if (k > N) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_bf_state_init, dim3(nblocks((int64_t)nq * 8, 256)), dim3(256), 0, s, state, nq, k);
  hipLaunchKernelGGL(k_bf_fill_i32, dim3(nblocks((int64_t)nq * 256, 256)), dim3(256), 0, s,
                     reinterpret_cast<int32_t*>(hist), (int64_t)nq * 256, 0);
  hipLaunchKernelGGL(k_bf_fill_i32, dim3(nblocks((int64_t)nq * k, 256)), dim3(256), 0, s, out_idx, (int64_t)nq * k,
                     -1);
  const dim3 grid(nblocks(N, kSelBlock), nq);
  for (int digit = 0; digit < 4; digit++)
    hipLaunchKernelGGL(k_bf_radix, grid, dim3(kBfThreads), 0, s, scores, ld_scores, N, digit, state, hist);
  hipLaunchKernelGGL(k_bf_collect, grid, dim3(kBfThreads), 0, s, scores, ld_scores, N, k, state, out_idx, out_dist);
  hipLaunchKernelGGL(k_bf_stream, dim3(nq), dim3(64), 0, s, scores, ld_scores, N, k, state, out_idx, out_dist);
  return hipGetLastError();
}

}  // namespace sgk
