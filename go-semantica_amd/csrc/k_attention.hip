// k_attention.hip -- bidirectional MQA attention over packed variable-length
// sequences (MultiHeadAttentionChunked with mask=nil,
// internal/kernels/attention.go:88-363; GQA expansion model_int8.go:455-479).
//
// Reference semantics kept:
//   s_ij = (q_i . k_j) * scale                         (scale = 1/sqrt(head_dim))
//   m_i  = max_j s_ij                                  (before any exp)
//   e_ij = fastExp(s_ij - m_i)  -- 0 when s_ij - m_i < -10 (activation.go:104-106)
//   o_i  = sum_j e_ij v_j / sum_j e_ij
// fastExp is not multiplicative and clamps, so an online (running-max)
// softmax would change the weights; the kernel makes two passes over the
// keys: pass 1 finds the row max, pass 2 forms e, the row sum and P.V.
//
// Precision.  The attention output is re-quantized to int8 with a
// per-sequence scale right after this kernel, so an error of 2^-12 (plain
// fp16 operands) flips a few percent of the int8 codes by a whole quantum and
// the flips compound over 24 layers.  Both products therefore run as split
// fp16 on the matrix cores: x = hi + lo with hi = fp16(x), lo = fp16(x - hi),
// and a.b = ah.bh + ah.bl + al.bh accumulated in fp32 (about 2^-22 relative,
// the level of the reference's own fp32 rounding).  Q and K are scaled by 8
// before splitting (exact) to keep lo out of the fp16 subnormal range; the
// weights e are scaled by 2^10 for the same reason; both scalings are undone
// exactly.  Pass 1 computes the same split scores, so the max is the max of
// the scores pass 2 exponentiates (a max that is off by even 1e-4 moves every
// fastExp argument and, through fastExp's polynomial error, the weights by
// ~1e-5).
//
// Operands arrive already split (the QK-norm/RoPE kernel writes Q and K hi/lo,
// k_v_split_t writes V^T hi/lo), so every workgroup only copies fp16 tiles.
//
// Work split.  The G query heads that share a kv head are stacked into
// G*ceil(S/16) chunks of 16 (head, query) rows.  A workgroup is 8 waves, one
// chunk each, two waves per SIMD (so one wave's softmax VALU overlaps the
// other's MFMAs); all eight stream the same 32-key K and V^T tiles through
// LDS.  A wave holds its chunk's Q^T (split, 64 VGPRs) and its O^T
// accumulators (256 dims x 16 queries, 64 VGPRs) for the whole run.  Scores
// are computed transposed, S^T = K Q^T on v_mfma_f32_16x16x32_f16: a lane owns
// one query and 8 keys of the tile, so row max and row sum are lane-local
// plus two exchanges, and those 8 registers are exactly the B operand of
// O^T += V^T P^T (one 32-key MFMA step) once V^T's keys are stored in the
// matching order (sgd::vt_key; the V^T split writes that order).
#include "sg_device.h"
#include "sg_kernels.h"
#include "sg_kv_prep.h"

namespace {

constexpr int kHD = 256;            // head_dim
constexpr int kBK = 32;             // keys per tile
constexpr int kQW = 16;             // (head, query) rows per wave
constexpr int kWaves = sgk::kAttnChunks;
constexpr int kNT = kWaves * SG_WAVE;
constexpr float kQKScale = sgk::kAttnQKScale;
constexpr float kPScale = 1024.0f, kPUnscale = 1.0f / 1024.0f;

// split_f16(x * scale) of two values x0, x1, packed, for a power-of-two
// scale: hi = {fp16(p0), fp16(p1)}, lo = {fp16(p0 - hi.x), fp16(p1 - hi.y)}
// with p = x * scale.  p is exact and so is p - fp16(p) (fp16(p) is p rounded
// to 11 significant bits), so each half is one v_fma_mix{lo,hi}_f16 of x
// rounded once to fp16: the bits of rounding p and p - hi, in four
// instructions, the lo pair reading hi's halves through op_sel (the compiler
// forms p, packs hi and recomputes it instead).
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void split_pair(float x0, float x1, float scale, uint32_t& hi, uint32_t& lo) {
  asm("v_fma_mixlo_f16 %0, %2, %4, 0\n\t"
      "v_fma_mixhi_f16 %0, %3, %4, 0\n\t"
      "v_fma_mixlo_f16 %1, %2, %4, -%0 op_sel_hi:[0,0,1]\n\t"
      "v_fma_mixhi_f16 %1, %3, %4, -%0 op_sel:[0,0,1] op_sel_hi:[0,0,1]"
      : "=&v"(hi), "=&v"(lo)
      : "v"(x0), "v"(x1), "s"(scale));
}

template <bool B>
struct bool_c {
  static constexpr bool value = B;
};
static_assert(sgk::kAttnChunkRows == kQW, "host chunking must match the kernel");

__device__ __forceinline__ f32x4_t mfma16(half8_t a, half8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// V^T tiles hold their keys in sgd::vt_key order (sg_kv_prep.h), which makes
// the eight S^T registers a lane holds per 32-key tile the B operand of one
// O^T += V^T P^T step.

constexpr int kRegTiles = sgk::kAttnRegKeys / kBK;

// Q^T as the B operand of one wave's 16 (head, query) rows: lane (query ln,
// group g4), k-step ks holds dims 32ks + 8g4 .. + 7 of row qr, scaled by 8
// and split hi/lo.  QPRE: Q arrives as the QKV GEMM's fp32 output and the wave
// applies attn_q_norm and RoPE to its 16 rows itself (the arithmetic of
// k_qknorm_rope_split, so the operands are bit-identical), which saves writing
// Q's hi/lo operands and reading them back; tile: the wave's 16 x 40 floats
// of LDS for the norm, wtile its 256 floats for the norm weights.  Otherwise
// Q arrives split (qh, ql).
template <bool QPRE>
__device__ __forceinline__ void q_operand(half8_t (&bqh)[kHD / 32], half8_t (&bql)[kHD / 32],
                                          const _Float16* __restrict__ qh, const _Float16* __restrict__ ql, int ldq,
                                          const sg_attn_qpre& qp, int qr, int pos, int head, int ln, int g4,
                                          int lane, float* tile, float* wtile) {
  if constexpr (QPRE) {
    // Every global load (the norm weights, Q, the RoPE table rows of the
    // row's position pos) is issued up front, so the prologue pays one memory
    // latency instead of one per phase; the registers are free this early.
    // Lane (ln, g4) holds elements e = 32ks + 8g4 + t of row ln.  The norm
    // weights, the same for every row, are one 16-byte load per lane (the
    // whole vector per wave) into wtile, read back as LDS broadcasts: loaded
    // per lane they took 16 of the wave's 48 load instructions, and the
    // prologue's time is its load instructions' (each wave's waits for the
    // other wave of its SIMD).
    float x[kHD / 32][8];
    const f32x4_t wl = qp.w ? reinterpret_cast<const f32x4_t*>(qp.w)[lane] : f32x4_t{0, 0, 0, 0};
    const float* src = qp.q + (int64_t)qr * qp.ldq + head * kHD + 8 * g4;
#pragma unroll
    for (int ks = 0; ks < kHD / 32; ks++) {
      // The fp32 Q row's last read: non-temporal, leaving L2 to the K/V tiles.
      const f32x4_t* s4 = reinterpret_cast<const f32x4_t*>(src + 32 * ks);
      *reinterpret_cast<f32x4_t*>(&x[ks][0]) = __builtin_nontemporal_load(s4);
      *reinterpret_cast<f32x4_t*>(&x[ks][4]) = __builtin_nontemporal_load(s4 + 1);
    }
    float cv[kHD / 64][8], sv[kHD / 64][8];
    const float* cr = qp.cos_t + (int64_t)pos * (kHD / 2) + 8 * g4;
    const float* sr = qp.sin_t + (int64_t)pos * (kHD / 2) + 8 * g4;
#pragma unroll
    for (int ks = 0; ks < kHD / 64; ks++) {
      *reinterpret_cast<f32x4_t*>(&cv[ks][0]) = *reinterpret_cast<const f32x4_t*>(cr + 32 * ks);
      *reinterpret_cast<f32x4_t*>(&cv[ks][4]) = *reinterpret_cast<const f32x4_t*>(cr + 32 * ks + 4);
      *reinterpret_cast<f32x4_t*>(&sv[ks][0]) = *reinterpret_cast<const f32x4_t*>(sr + 32 * ks);
      *reinterpret_cast<f32x4_t*>(&sv[ks][4]) = *reinterpret_cast<const f32x4_t*>(sr + 32 * ks + 4);
    }
    static_assert(kHD == 4 * SG_WAVE, "one float4 of the norm weights per lane");
    if (qp.w) reinterpret_cast<f32x4_t*>(wtile)[lane] = wl;
    if (qp.w) {
      // RMSNorm's sum of squares in the AVX2 lane order (sg_rmsnorm8): lane v
      // of a row chains element 8i + v over i.  Element e sits at i = 4ks + g4,
      // v = t here, so each 32-element chunk goes through the wave's 16 x
      // 40-float LDS tile; lane (row rA or rA + 8, v) then reads the chunk's
      // elements 8k + v, k = 0..3, in order.
      const int v = lane & 7, rA = lane >> 3;
      float accA = 0.0f, accB = 0.0f;
#pragma unroll
      for (int ks = 0; ks < kHD / 32; ks++) {
        asm volatile("" ::: "memory");
        *reinterpret_cast<f32x4_t*>(tile + ln * 40 + 8 * g4) = f32x4_t{x[ks][0], x[ks][1], x[ks][2], x[ks][3]};
        *reinterpret_cast<f32x4_t*>(tile + ln * 40 + 8 * g4 + 4) = f32x4_t{x[ks][4], x[ks][5], x[ks][6], x[ks][7]};
        asm volatile("" ::: "memory");
#pragma unroll
        for (int k = 0; k < 4; k++) {
          const float a = tile[rA * 40 + 8 * k + v];
          accA = __builtin_fmaf(a, a, accA);
          const float b = tile[(rA + 8) * 40 + 8 * k + v];
          accB = __builtin_fmaf(b, b, accB);
        }
      }
      asm volatile("" ::: "memory");
      const float invA = 1.0f / sg_sqrt(sg_hsum8(accA) / (float)kHD + qp.eps);
      const float invB = 1.0f / sg_sqrt(sg_hsum8(accB) / (float)kHD + qp.eps);
      const float iA = __shfl(invA, 8 * (ln & 7)), iB = __shfl(invB, 8 * (ln & 7));
      const float inv = ln < 8 ? iA : iB;
#pragma unroll
      for (int ks = 0; ks < kHD / 32; ks++) {
        const float* wv = wtile + 32 * ks + 8 * g4;
#pragma unroll
        for (int t = 0; t < 8; t++) {
          const float u = x[ks][t] * inv;
          x[ks][t] = u * wv[t];
        }
      }
    }
    // RoPE (rope_cache.go:85-104): pairs (e, e + 128) are chunks ks and ks + 4
    // of the same lane and slot.
#pragma unroll
    for (int ks = 0; ks < kHD / 64; ks++) {
#pragma unroll
      for (int t = 0; t < 8; t++) {
        const float v0 = x[ks][t], v1 = x[ks + kHD / 64][t];
        const float a = v0 * cv[ks][t], b = v1 * sv[ks][t], cc = v0 * sv[ks][t], dd = v1 * cv[ks][t];
        x[ks][t] = a - b;
        x[ks + kHD / 64][t] = cc + dd;
      }
    }
#pragma unroll
    for (int ks = 0; ks < kHD / 32; ks++) {
      u32x4_t uh, ul;
#pragma unroll
      for (int k = 0; k < 4; k++) {
        uint32_t h, l;
        split_pair(x[ks][2 * k], x[ks][2 * k + 1], kQKScale, h, l);
        uh[k] = h;
        ul[k] = l;
      }
      bqh[ks] = __builtin_bit_cast(half8_t, uh);
      bql[ks] = __builtin_bit_cast(half8_t, ul);
    }
  } else {
    const int64_t qo = (int64_t)qr * ldq + head * kHD + 8 * g4;
#pragma unroll
    for (int ks = 0; ks < kHD / 32; ks++) {
      bqh[ks] = *reinterpret_cast<const half8_t*>(qh + qo + 32 * ks);
      bql[ks] = *reinterpret_cast<const half8_t*>(ql + qo + 32 * ks);
    }
  }
}

constexpr int kTileBytes = 32 * 1024;  // one K or V^T tile, hi and lo halves
constexpr int kRing = 3;               // tile stages in LDS
constexpr int kScoreBytes = sgk::kAttnSpillTileBytes;  // one tile's scores, 8 floats per lane and wave
static_assert(kScoreBytes == kWaves * 2048, "spill tile layout");

// Two passes over a sequence's 32-key tiles: pass 1 keeps each lane's scaled
// scores in registers (8 per tile, 128 VGPRs for the first kRegTiles tiles)
// and pass 2 reads them back instead of recomputing S^T, so K is streamed once
// and a third of the MFMAs and LDS reads go away.  SPILL (a launch with a
// sequence longer than kRegKeys keys): the tiles past kRegTiles write their
// scores to a per-workgroup spill range in pass 1 and read them back in pass 2
// through LDS, carried by the V^T item before their own.  The tiles reach LDS
// by buffer_load ... lds (no staging registers): one stream of 2 nt items, the
// nt K tiles then the nt V^T tiles, item i in ring stage i % 3, issued two
// items ahead; each wave issues four 1-KB copies per item (six when it also
// carries scores; past the last item it re-copies that one into the free
// stage), so a vmcnt of the next item's copy count says "item i has landed"
// and the barrier after it publishes every wave's copies and retires the
// stage the next copies overwrite.
//
// LDS layouts, XOR-swizzled in 16-byte chunks so that the 16x16x32 fragment
// reads (16 rows x 4 lane groups) hit distinct banks with unpadded rows:
//   K stage:   row R = 32 hl + key (hl 0 hi, 1 lo), 512 B per row; chunk c
//              (dims 8c .. 8c + 7) at position c ^ (R & 15).
//   V^T stage: row d = dim, 128 B per row (hi keys then lo keys, the global
//              layout); chunk c at position c ^ ((d >> 1) & 7).
// A copy lane picks the global chunk its LDS position holds, so the swizzle
// costs nothing at copy time; fragment addresses are one XOR per k-step.
template <bool QPRE, bool SPILL>
__global__ __launch_bounds__(kNT, 2) void k_attn_rs(
    const _Float16* __restrict__ qh, const _Float16* __restrict__ ql, int ldq, const _Float16* __restrict__ kh,
    const _Float16* __restrict__ kl, int ldk, const _Float16* __restrict__ vt, int ldvt, float* __restrict__ out,
    int ldo, const int32_t* __restrict__ seq_off, const int32_t* __restrict__ voff, const sg_item* __restrict__ items,
    int G, float sscale, float* __restrict__ amax, sg_attn_qpre qp, sg_attn_qout qo, sg_attn_spill sp) {
  __shared__ __attribute__((aligned(16))) unsigned char lds[kRing * kTileBytes];
  __shared__ __attribute__((aligned(16))) unsigned char slds[SPILL ? kRing * kScoreBytes : 16];
  __shared__ float red[kWaves];
  typedef __attribute__((address_space(3))) void* lds_ptr;

  const sg_item it = items[blockIdx.x];
  const int kvh = blockIdx.y;
  const int r0 = seq_off[it.seq];
  const int S = seq_off[it.seq + 1] - r0;
  const int vo = voff[it.seq];
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6) & (kWaves - 1);
  const int ln = lane & 15, g4 = lane >> 4;
  const int nqb = (S + kQW - 1) / kQW;
  const int nt = (S + kBK - 1) / kBK;  // <= kRegTiles unless SPILL (the host checks the longest sequence)
  const int c = it.c0 + w;
  const bool active = c < G * nqb;  // wave-uniform
  const int hg = active ? c / nqb : 0;
  const int q0 = active ? (c % nqb) * kQW : 0;
  const int head = kvh * G + hg;
  const int qrow = q0 + ln;
  const bool qvalid = active && qrow < S;
  const int qr = r0 + min(qrow, S - 1);

  // ---- copies ----
  // Wave w's four copies of an item land at w * 4 KB + i * 1 KB of the stage.
  // K item: copy i moves rows R = 8w + 2i and 8w + 2i + 1 (hi for waves 0-3,
  // lo for waves 4-7); lane L takes row R = 8w + 2i + L / 32 and LDS position
  // L % 32, i.e. global chunk (L % 32) ^ (R & 15).  Keys past the sequence's
  // end are clamped to its last key and masked out of the scores below.
  // V^T item: copy i moves dims 32w + 8i .. + 7; lane L takes dim
  // d = 32w + 8i + L / 8, position L % 8, global chunk (L % 8) ^ ((d >> 1) & 7);
  // every tile of a sequence lies inside its padded V^T columns.
  const i32x4_t rk = sg_raw_rsrc((w < 4 ? kh : kl) + (int64_t)r0 * ldk + kvh * kHD);
  const i32x4_t rv = sg_raw_rsrc(vt + (int64_t)kvh * kHD * ldvt + 2 * vo);
  // Per-lane byte offsets, loop-invariant: K copy i at key row kkey(i) of a
  // tile (kvo; the tile's first row goes in the scalar offset), V^T copy i
  // (voffs; the tile's columns go in the scalar offset).
  auto kkey = [&](int i) { return ((8 * w + 2 * i) & 31) + (lane >> 5); };
  uint32_t kvo[4], voffs[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int R = 8 * w + 2 * i + (lane >> 5);
    kvo[i] = (uint32_t)kkey(i) * (uint32_t)ldk * 2u + 16u * (uint32_t)((lane & 31) ^ (R & 15));
    const int d = 32 * (w & 7) + 8 * i + (lane >> 3), cv = (lane & 7) ^ ((d >> 1) & 7);
    voffs[i] = (uint32_t)d * (uint32_t)ldvt * 2u + 16u * (uint32_t)cv;
  }
  // This wave's four copies of K tile `tile` (isk) or V^T tile `tile` into the
  // ring stage at dst.
  auto copy_tile = [&](uint32_t dst, bool isk, int tile) {
    if (!isk) {  // V^T: the tile's columns, 64 halves per 32 keys
      const uint32_t soff = (uint32_t)tile * kBK * 4u;
#pragma unroll
      for (int i = 0; i < 4; i++) sg_lds_copy16(dst + 1024u * i, voffs[i], rv, soff);
    } else if (tile * kBK + kBK <= S) {  // a whole K tile
      const uint32_t soff = (uint32_t)(tile * kBK) * (uint32_t)ldk * 2u;
#pragma unroll
      for (int i = 0; i < 4; i++) sg_lds_copy16(dst + 1024u * i, kvo[i], rk, soff);
    } else {  // a sequence's last K tile: rows past S re-read its last key
      const int kt = tile * kBK;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int key = min(kt + kkey(i), S - 1);
        sg_lds_copy16(dst + 1024u * i, kvo[i] + (uint32_t)(key - kkey(i)) * (uint32_t)ldk * 2u, rk, 0u);
      }
    }
  };
  // SPILL: this workgroup's spilled scores, nt - kRegTiles tiles of
  // kScoreBytes (wave w's 2 KB at w * 2048: lane l's keys 4g4 + r at 16 l,
  // 16 + 4g4 + r at 1024 + 16 l).  V^T item nt + t - 1 also carries tile t's
  // scores when t >= kRegTiles, two more copies per wave into the item's
  // score stage.
  float* const wspill =
      SPILL && nt > kRegTiles
          ? sp.buf + ((size_t)kvh * sp.total + sp.off[it.seq] + (size_t)(it.c0 / kWaves) * (nt - kRegTiles)) *
                         (kScoreBytes / 4)
          : nullptr;
  const i32x4_t rsp = sg_raw_rsrc(wspill);
  const int last = 2 * nt - 1;
  auto carries = [&](int src) { return SPILL && src >= nt + kRegTiles - 1 && src < last; };
  auto issue = [&](int item) {
    const int src = item < last ? item : last;
    const uint32_t dst = (uint32_t)(uintptr_t)(lds_ptr)(lds + ((unsigned)item % kRing) * kTileBytes + w * 4096);
    copy_tile(dst, src < nt, src < nt ? src : src - nt);
    if (carries(src)) {
      const uint32_t sd = (uint32_t)(uintptr_t)(lds_ptr)(slds + ((unsigned)item % kRing) * kScoreBytes + w * 2048);
      const uint32_t so = (uint32_t)((src - nt + 1 - kRegTiles) * kScoreBytes + w * 2048);
      sg_lds_copy16(sd, 16u * lane, rsp, so);
      sg_lds_copy16(sd + 1024u, 16u * lane + 1024u, rsp, so);
    }
  };
  // Wait until item i has landed, item i + 1 (4 copies per wave, or 6 when it
  // carries scores) may still be in flight.
  auto wait_item = [&](int i) {
    if (carries(i + 1 < last ? i + 1 : last))
      sg_wait_vmcnt<6>();
    else
      sg_wait_vmcnt<4>();
  };
  issue(0);
  issue(1);
  half8_t bqh[kHD / 32], bql[kHD / 32];
  // The Q prologue's LDS tiles sit in stage 2, which no copy touches before
  // the first barrier.
  static_assert(kWaves * (16 * 40 + kHD) * 4 <= kTileBytes, "prologue tiles fit stage 2");
  q_operand<QPRE>(bqh, bql, qh, ql, ldq, qp, qr, qr - r0, head, ln, g4, lane,
                  reinterpret_cast<float*>(lds + 2 * kTileBytes) + w * (16 * 40),
                  reinterpret_cast<float*>(lds + 2 * kTileBytes) + kWaves * (16 * 40) + w * kHD);

  auto key_of = [&](int kt, int st, int r) { return kt + 16 * st + 4 * g4 + r; };
  // ---- pass 1: S^T = K Q^T per tile, kept in registers; row max ----
  // K fragment (row R = 32 hl + 16 st + ln, chunk 4 ks + g4) at
  // R * 512 + 16 * ((4 ks + g4) ^ ln) = (xk ^ 64 ks) + 8192 st + 16384 hl.
  const uint32_t xk = (uint32_t)ln * 512u + 16u * (uint32_t)(g4 ^ (ln & 3)) + 64u * (uint32_t)(ln >> 2);
  auto scores2 = [&](const unsigned char* kb, f32x4_t& a0, f32x4_t& a1) {
    auto rd = [&](int st, int ks, half8_t& h, half8_t& l) {
      const unsigned char* p = kb + (xk ^ (64u * ks)) + 8192 * st;
      h = *reinterpret_cast<const half8_t*>(p);
      l = *reinterpret_cast<const half8_t*>(p + 16384);
    };
    a0 = f32x4_t{0, 0, 0, 0};
    a1 = f32x4_t{0, 0, 0, 0};
    half8_t h0, l0, h1, l1;
    rd(0, 0, h0, l0);
    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
    for (int ks = 0; ks < kHD / 32; ks++) {
      rd(1, ks, h1, l1);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      a0 = mfma16(h0, bqh[ks], a0);
      a0 = mfma16(h0, bql[ks], a0);
      a0 = mfma16(l0, bqh[ks], a0);
      __builtin_amdgcn_sched_group_barrier(0x008, 3, 0);
      if (ks + 1 < kHD / 32) {
        rd(0, ks + 1, h0, l0);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      }
      a1 = mfma16(h1, bqh[ks], a1);
      a1 = mfma16(h1, bql[ks], a1);
      a1 = mfma16(l1, bqh[ks], a1);
      __builtin_amdgcn_sched_group_barrier(0x008, 3, 0);
    }
  };
  float m = -INFINITY;
  f32x4_t sr[kRegTiles][2];
  // The scores are kept as s = raw * sscale (exact: sscale is a power of
  // two); a key past S (only in a sequence's last tile) keeps -inf, so pass
  // 2's fastExp clamp gives it a weight of exactly 0 without a per-key test
  // there.
#pragma unroll
  for (int t = 0; t < kRegTiles; t++) {
    if (t < nt) {
      wait_item(t);  // item t landed (item t + 1 may still be in flight)
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      issue(t + 2);
      // Every wave computes (an inactive wave's results are never stored).
      scores2(lds + (t % kRing) * kTileBytes, sr[t][0], sr[t][1]);
      const int kt = t * kBK;
      if (kt + kBK <= S) {
#pragma unroll
        for (int r = 0; r < 4; r++) {
          sr[t][0][r] *= sscale;
          sr[t][1][r] *= sscale;
          m = fmaxf(m, fmaxf(sr[t][0][r], sr[t][1][r]));
        }
      } else {
#pragma unroll
        for (int r = 0; r < 4; r++) {
          sr[t][0][r] = key_of(kt, 0, r) < S ? sr[t][0][r] * sscale : -INFINITY;
          sr[t][1][r] = key_of(kt, 1, r) < S ? sr[t][1][r] * sscale : -INFINITY;
          m = fmaxf(m, fmaxf(sr[t][0][r], sr[t][1][r]));
        }
      }
    }
  }
  if constexpr (SPILL) {
    // Tiles past kRegTiles: their scores go to this wave's spill slots.
    for (int t = kRegTiles; t < nt; t++) {
      wait_item(t);
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      issue(t + 2);
      f32x4_t s0, s1;
      scores2(lds + (t % kRing) * kTileBytes, s0, s1);
      const int kt = t * kBK;
      if (kt + kBK <= S) {
#pragma unroll
        for (int r = 0; r < 4; r++) {
          s0[r] *= sscale;
          s1[r] *= sscale;
          m = fmaxf(m, fmaxf(s0[r], s1[r]));
        }
      } else {
#pragma unroll
        for (int r = 0; r < 4; r++) {
          s0[r] = key_of(kt, 0, r) < S ? s0[r] * sscale : -INFINITY;
          s1[r] = key_of(kt, 1, r) < S ? s1[r] * sscale : -INFINITY;
          m = fmaxf(m, fmaxf(s0[r], s1[r]));
        }
      }
      float* sp = wspill + (size_t)(t - kRegTiles) * (kScoreBytes / 4) + w * 512 + 4 * lane;
      *reinterpret_cast<f32x4_t*>(sp) = s0;
      *reinterpret_cast<f32x4_t*>(sp + 256) = s1;
    }
  }
  m = fmaxf(m, __shfl_xor(m, 16));
  m = fmaxf(m, __shfl_xor(m, 32));

  // ---- pass 2: e = fastExp(s - m), row sums, O^T += V^T P^T ----
  // V^T fragment (dim 16 mt + ln, chunk g4 hi / 4 + g4 lo) at
  // (16 mt + ln) * 128 + 16 * (chunk ^ ((ln >> 1) & 7)): xv (+ 64 for lo)
  // + 2048 mt.
  const uint32_t xv = (uint32_t)ln * 128u + 16u * (uint32_t)(g4 ^ ((ln >> 1) & 7));
  f32x4_t o[kHD / 16];
#pragma unroll
  for (int mt = 0; mt < kHD / 16; mt++) o[mt] = f32x4_t{0, 0, 0, 0};
  float lsum = 0.0f;
  auto pv = [&](const unsigned char* vb, const half8_t& ph, const half8_t& pl) {
    const unsigned char* p0 = vb + xv;
    half8_t fr[3][2];  // [buffer][hi, lo]
    auto rd = [&](int mt, half8_t(&f)[2]) {
      f[0] = *reinterpret_cast<const half8_t*>(p0 + 2048 * mt);
      f[1] = *reinterpret_cast<const half8_t*>(vb + ((xv ^ 64u) + 2048u * mt));
    };
    rd(0, fr[0]);
    rd(1, fr[1]);
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
    for (int mt = 0; mt < kHD / 16; mt++) {
      if (mt + 2 < kHD / 16) {
        rd(mt + 2, fr[(mt + 2) % 3]);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      }
      const half8_t(&f)[2] = fr[mt % 3];
      o[mt] = mfma16(f[0], ph, o[mt]);
      o[mt] = mfma16(f[0], pl, o[mt]);
      o[mt] = mfma16(f[1], ph, o[mt]);
      __builtin_amdgcn_sched_group_barrier(0x008, 3, 0);
    }
  };
  // One tile of pass 2: the weights from its scores, then P.V on its V^T item.
  auto tile2 = [&](const f32x4_t& s0, const f32x4_t& s1, int t) {
    const int item = nt + t;
    float e[8];  // slots 0..3: keys 4g4+r, slots 4..7: 16+4g4+r
#pragma unroll
    for (int r = 0; r < 4; r++) {
      e[r] = sg_fast_exp_nonpos(s0[r] - m);
      e[4 + r] = sg_fast_exp_nonpos(s1[r] - m);
    }
#pragma unroll
    for (int k = 0; k < 8; k++) lsum = lsum + e[k];
    u32x4_t uh, ul;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      uint32_t h, l;
      split_pair(e[2 * k], e[2 * k + 1], kPScale, h, l);
      uh[k] = h;
      ul[k] = l;
    }
    const half8_t ph = __builtin_bit_cast(half8_t, uh), pl = __builtin_bit_cast(half8_t, ul);
    wait_item(item);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    issue(item + 2);
    pv(lds + ((unsigned)item % kRing) * kTileBytes, ph, pl);
  };
#pragma unroll
  for (int t = 0; t < kRegTiles; t++)
    if (t < nt) tile2(sr[t][0], sr[t][1], t);
  if constexpr (SPILL) {
    // Tile t's scores landed with item nt + t - 1 (published by its barrier);
    // the stage is overwritten only after the next barrier.
    for (int t = kRegTiles; t < nt; t++) {
      const unsigned char* sb = slds + ((unsigned)(nt + t - 1) % kRing) * kScoreBytes + w * 2048 + 16 * lane;
      tile2(*reinterpret_cast<const f32x4_t*>(sb), *reinterpret_cast<const f32x4_t*>(sb + 1024), t);
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the re-copies past the last item have landed
  lsum = lsum + __shfl_xor(lsum, 16);
  lsum = lsum + __shfl_xor(lsum, 32);
  const float f = (1.0f / lsum) * kPUnscale;

  // O^T tile mt: lane holds query ln, dims 16mt + 4g4 + r.
  float mx = 0.0f;
  if (qvalid) {
    float* op = out + (int64_t)(r0 + qrow) * ldo + head * kHD + 4 * g4;
#pragma unroll
    for (int mt = 0; mt < kHD / 16; mt++) {
      f32x4_t y;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        y[j] = o[mt][j] * f;
        mx = fmaxf(mx, fabsf(y[j]));
      }
      *reinterpret_cast<f32x4_t*>(op + 16 * mt) = y;
    }
  }
  if (amax) {  // all chunks of a workgroup belong to one sequence
    mx = sg_wave_max(mx);
    if (lane == 0) red[w] = mx;
    __syncthreads();
    if (tid == 0) {
      float mm = red[0];
#pragma unroll
      for (int i = 1; i < kWaves; i++) mm = fmaxf(mm, red[i]);
      sg_atomic_max_nonneg(amax + it.seq, mm);
    }
    // The workgroup holds the whole sequence (every row of every head; the
    // caller passes qo.q8 only then), so its maximum is the sequence's and
    // the output is quantized here, from the values just stored, as the
    // quantizer would quantize them: lane (query ln, group g4) codes dims
    // 16 mt + 4 g4 .. + 3 of its head, 4 bytes of K-block (head * 256 +
    // 16 mt) / 32 per mt.
    if (qo.q8 && qvalid) {
      float mm = red[0];
#pragma unroll
      for (int i = 1; i < kWaves; i++) mm = fmaxf(mm, red[i]);
      float scale = 1.0f, inv = 0.0f;
      if (mm != 0.0f) {
        scale = mm / 127.0f;
        inv = 1.0f / scale;
      }
      const int row = r0 + qrow;
      if (hg == 0 && g4 == 0) qo.row_scale[row] = scale;
#pragma unroll
      for (int mt = 0; mt < kHD / 16; mt++) {
        const int col = head * kHD + 16 * mt + 4 * g4;
        uint32_t u = 0;
#pragma unroll
        for (int j = 0; j < 4; j++)
          u |= (uint32_t)(uint8_t)(int8_t)(int)sg_quant_code_nb(o[mt][j] * f, inv) << (8 * j);
        *reinterpret_cast<uint32_t*>(qo.q8 + ((int64_t)(col >> 5) * qo.a_rows + row) * 32 + (col & 31)) = u;
      }
    }
  }
}

// V^T split, one 32-key tile per workgroup (sgd::v_split_tile); kv head blockIdx.y.
__global__ __launch_bounds__(sgd::kKvThreads) void k_v_split_t(const float* __restrict__ v, int ldv,
                                                             const int32_t* __restrict__ seq_off,
                                                             const int32_t* __restrict__ voff,
                                                             const sg_item* __restrict__ vtiles,
                                                             _Float16* __restrict__ vt, int ldvt) {
  __shared__ __attribute__((aligned(16))) float tv[kBK][sgd::kVtRowStride];
  sgd::v_split_tile(vtiles[blockIdx.x], blockIdx.y, tv, v, ldv, seq_off, voff, vt, ldvt);
}

// K's QK-norm/RoPE split and V's V^T split in one launch: workgroups
// [0, nkb) take 32 (token, kv head) rows of K each, the rest one (V tile,
// kv head) each, so the two halves' loads and stores overlap.
__global__ __launch_bounds__(sgd::kKvThreads) void k_kv_prep(
    const float* __restrict__ k, const float* __restrict__ v, int ldkv, const float* __restrict__ kw, int HKV, int T,
    const int32_t* __restrict__ row_pos, const float* __restrict__ cos_t, const float* __restrict__ sin_t, float eps,
    _Float16* __restrict__ ks_h, _Float16* __restrict__ ks_l, int ldks, int nkb, const int32_t* __restrict__ seq_off,
    const int32_t* __restrict__ voff, const sg_item* __restrict__ vtiles, int n_vtiles, _Float16* __restrict__ vt, int ldvt,
    sgk::sg_kv_q qp) {
  __shared__ __attribute__((aligned(16))) float tv[kBK][sgd::kVtRowStride];
  const int b = blockIdx.x;
  if (b < nkb) {  // workgroup-uniform
    const int64_t g = (int64_t)b * sgd::kKvRows + (threadIdx.x >> 3);
    float* tile = &tv[0][0] + (threadIdx.x / SG_WAVE) * (8 * 40);  // 8 x 40 floats per wave
    // (token, head) groups, query heads first.  With no query heads (qp.H =
    // 0) the Q arguments are never read; they then point at K (passing null
    // for them crashed this compiler's device pass).
    sgd::qk_split_group(g, threadIdx.x & 7, (threadIdx.x >> 3) & 7, tile, qp.q, qp.ldq, k, ldkv, qp.qw, kw, qp.H,
                        HKV, T, row_pos, cos_t, sin_t, eps, qp.qs_h, qp.qs_l, qp.ldqs, ks_h, ks_l, ldks);
  } else {
    const int vb = b - nkb;
    sgd::v_split_tile(vtiles[vb % n_vtiles], vb / n_vtiles, tv, v, ldkv, seq_off, voff, vt, ldvt);
  }
}

// Rows of x (fp32) -> hi/lo fp16 of x*scale.
__global__ __launch_bounds__(256) void k_split_rows(const float* __restrict__ x, int ldx, int cols, float scale,
                                                    _Float16* __restrict__ hi, _Float16* __restrict__ lo,
                                                    int ldo) {
  const int row = blockIdx.x;
  for (int c4 = threadIdx.x; c4 < cols / 4; c4 += 256) {
    const f32x4_t a = *reinterpret_cast<const f32x4_t*>(x + (int64_t)row * ldx + 4 * c4);
    half4_t vh, vl;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const hl16 s = split_f16(a[j] * scale);
      vh[j] = s.hi;
      vl[j] = s.lo;
    }
    *reinterpret_cast<half4_t*>(hi + (int64_t)row * ldo + 4 * c4) = vh;
    *reinterpret_cast<half4_t*>(lo + (int64_t)row * ldo + 4 * c4) = vl;
  }
}

}  // namespace

namespace sgk {

hipError_t v_split_t(const float* v, int ldv, const int32_t* seq_off, const int32_t* voff, const sg_item* vtiles,
                     int n_vtiles, int HKV, _Float16* vt, int ldvt, hipStream_t s) {
  if (n_vtiles <= 0) return hipSuccess;
  if ((ldv & 3) || (ldvt & 7)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_v_split_t, dim3(n_vtiles, HKV), dim3(256), 0, s, v, ldv, seq_off, voff, vtiles, vt,
                     ldvt);
  return hipGetLastError();
}

hipError_t kv_prep(const float* k, const float* v, int ldkv, const float* kw, int HKV, int T, const int32_t* row_pos,
                   const float* cos_t, const float* sin_t, float eps, _Float16* ks_h, _Float16* ks_l, int ldks,
                   const int32_t* seq_off, const int32_t* voff, const sg_item* vtiles, int n_vtiles, _Float16* vt, int ldvt, hipStream_t s,
                   const sg_kv_q* qpart) {
  if (T <= 0 || n_vtiles < 0 || HKV <= 0) return hipSuccess;
  if ((ldkv & 3) || (ldks & 7) || (ldvt & 7) || (reinterpret_cast<uintptr_t>(k) & 15) ||
      (reinterpret_cast<uintptr_t>(v) & 15) || (kw && (reinterpret_cast<uintptr_t>(kw) & 15)))
    return hipErrorInvalidValue;  // float4 loads of K and V rows and of the weights
  sgk::sg_kv_q qp{k, ldkv, kw, 0, ks_h, ks_l, ldks};
  if (qpart && qpart->H > 0) {
    if (!qpart->q || !qpart->qs_h || !qpart->qs_l || (qpart->ldq & 3) || (qpart->ldqs & 7) ||
        (reinterpret_cast<uintptr_t>(qpart->q) & 15) || (qpart->qw && (reinterpret_cast<uintptr_t>(qpart->qw) & 15)))
      return hipErrorInvalidValue;  // float4 loads of the Q rows and weights, 16-byte split stores
    qp = *qpart;
  }
  const int64_t nkb = ((int64_t)T * (qp.H + HKV) + sgd::kKvRows - 1) / sgd::kKvRows;
  const int64_t nb = nkb + (int64_t)n_vtiles * HKV;
  if (nb > INT32_MAX) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_kv_prep, dim3((unsigned)nb), dim3(sgd::kKvThreads), 0, s, k, v, ldkv, kw, HKV, T, row_pos, cos_t,
                     sin_t, eps, ks_h, ks_l, ldks, (int)nkb, seq_off, voff, vtiles, n_vtiles, vt, ldvt, qp);
  return hipGetLastError();
}

hipError_t split_rows(const float* x, int ldx, int rows, int cols, float scale, _Float16* hi, _Float16* lo, int ldo,
                      hipStream_t s) {
  if (rows <= 0) return hipSuccess;
  if ((ldx & 3) || (cols & 3) || (ldo & 3)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_split_rows, dim3(rows), dim3(256), 0, s, x, ldx, cols, scale, hi, lo, ldo);
  return hipGetLastError();
}

namespace {
template <bool QPRE, bool SPILL>
void launch_attn(dim3 grid, hipStream_t s, const _Float16* qh, const _Float16* ql, int ldq, const _Float16* kh,
                 const _Float16* kl, int ldk, const _Float16* vt, int ldvt, float* out, int ldo,
                 const int32_t* seq_off, const int32_t* voff, const sg_item* items, int G, float sscale, float* amax,
                 const sg_attn_qpre& qp, const sg_attn_qout& qo, const sg_attn_spill& sp) {
  hipLaunchKernelGGL((k_attn_rs<QPRE, SPILL>), grid, dim3(kNT), 0, s, qh, ql, ldq, kh, kl, ldk, vt, ldvt, out, ldo,
                     seq_off, voff, items, G, sscale, amax, qp, qo, sp);
}
}  // namespace

hipError_t attention(const _Float16* qh, const _Float16* ql, int ldq, const _Float16* kh, const _Float16* kl, int ldk,
                     const _Float16* vt, int ldvt, float* out, int ldo, const int32_t* seq_off,
                     const int32_t* voff, const sg_item* items, int n_items, int H, int HKV, int hd, float scale,
                     float* amax, int max_len, hipStream_t s, const sg_attn_qpre* qpre,
                     const sg_attn_qout* qout, const sg_attn_spill* spill) {
  if (n_items <= 0) return hipSuccess;
  if (hd != kHD || HKV <= 0 || H % HKV || max_len <= 0) return hipErrorInvalidValue;
  // The quantizing epilogue needs the register-scores kernel, one workgroup per
  // sequence (one kv head, every chunk of the sequence in one item) and amax.
  if (qout && (!qout->q8 || !qout->row_scale || HKV != 1 || max_len > kAttnRegKeys || !amax ||
               (H / HKV) * ((max_len + kQW - 1) / kQW) > kWaves))
    return hipErrorInvalidValue;
  const sg_attn_qout qo = qout ? *qout : sg_attn_qout{nullptr, 0, nullptr};
  if ((ldk | ldvt) & 7 || (ldo & 3)) return hipErrorInvalidValue;
  static_assert(kBK == 32 && kRegTiles == sgk::kAttnRegKeys / 32, "attention_spill_tiles");
  const bool spills = attention_spill_tiles(max_len) > 0;
  if (spills && (!spill || !spill->buf || !spill->off || spill->total <= 0 ||
                 (reinterpret_cast<uintptr_t>(spill->buf) & 15)))
    return hipErrorInvalidValue;
  const sg_attn_spill sp = spills ? *spill : sg_attn_spill{nullptr, nullptr, 0};
  const float sscale = scale / (kQKScale * kQKScale);
  const dim3 grid(n_items, HKV);
  sg_attn_qpre qp{};
  if (qpre) {
    if (!qpre->q || !qpre->cos_t || !qpre->sin_t || (qpre->ldq & 3) ||
        (reinterpret_cast<uintptr_t>(qpre->q) & 15) || (reinterpret_cast<uintptr_t>(qpre->w) & 15) ||
        (reinterpret_cast<uintptr_t>(qpre->cos_t) & 15) || (reinterpret_cast<uintptr_t>(qpre->sin_t) & 15))
      return hipErrorInvalidValue;  // float4 loads of Q rows, weights and table rows
    qp = *qpre;
  } else if (ldq & 7) {
    return hipErrorInvalidValue;
  }
  using fn = void (*)(dim3, hipStream_t, const _Float16*, const _Float16*, int, const _Float16*, const _Float16*, int,
                      const _Float16*, int, float*, int, const int32_t*, const int32_t*, const sg_item*, int, float,
                      float*, const sg_attn_qpre&, const sg_attn_qout&, const sg_attn_spill&);
  static const fn table[2][2] = {{launch_attn<false, false>, launch_attn<false, true>},
                                 {launch_attn<true, false>, launch_attn<true, true>}};
  table[qpre != nullptr][spills](grid, s, qh, ql, ldq, kh, kl, ldk, vt, ldvt, out, ldo, seq_off, voff, items, H / HKV,
                                 sscale, amax, qp, qo, sp);
  return hipGetLastError();
}

}  // namespace sgk
