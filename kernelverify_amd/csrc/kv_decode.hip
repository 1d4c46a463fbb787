// Quantized-KV decode attention for gfx950, split over cached positions.
//
// Replaces the reference's `kv_attn_decode` (kernelverify/pack/kv_attention.py:85-234):
// one decode step per (sequence, query head): scores q.dequant(K_t)/sqrt(DH)
// over the T cached positions plus the step's own new_k at full precision,
// an fp32 max-subtracted softmax over T+1, and out = sum_t p_t dequant(V_t)
// + p_new new_v. The reference holds the whole softmax in threadgroup memory
// and is capped at T <= 1024 (:77, :112-115); here any T up to t_stride runs:
//
//   kv_split_kernel   one block per (chunk of positions, KV head, sequence).
//                     Every load of its chunk (q, K, V codes and scales) is
//                     issued up front, so the V stream is in flight while
//                     the scores and the chunk softmax are computed.
//                     It serves all G = H/HKV query heads of that KV head, so
//                     each cache byte is read from HBM once (the reference
//                     re-reads the cache per query head, :286-289). For its
//                     chunk it writes per-head partials (m, l, o[DH]): the
//                     running max, sum of exp(s - m) and sum of
//                     exp(s - m) * v.
//   kv_combine_kernel one block per (sequence, query head, 16-dim slice)
//                     merges the chunk partials and the new entry with the
//                     log-sum-exp rule M = max(m_c, s_new),
//                     L = sum l_c e^(m_c-M) + e^(s_new-M),
//                     O = (sum o_c e^(m_c-M) + e^(s_new-M) new_v) / L.
//
// This is the online-softmax tiling of contract clause C3
// (kernelverify/tolerance/contract.py:31-46): exact in exact arithmetic,
// every intermediate fp32. The softmax runs in base 2: scores carry
// log2(e) / sqrt(DH) (one rounding), so e^(s-m) is exp2 of the scaled
// difference; the partials' m is in the same base-2 units.
//
// Score side: a lane owns one unit (16 bytes; 24 for 3-bit) of a K row, so a
// wave's K load instruction covers 64/U whole rows contiguously. The lane's
// query slice (all G heads) is held in registers in weight-word pair order,
// and unit_dot (shared with the qmv kernel) forms the G partial dot products
// with V_DOT2_F32_F16 on exact fp16-denormal codes; the U lanes of a row
// then add their partials.
//
// Value side: a lane owns one 8-code block of a V row (the reference's
// block, kv_attention.py:194-217) for every G head, accumulating
// (p * s) * q + p * b in fp32.
#include <math.h>

#include <mutex>
#include <type_traits>

#include "common.h"
#include "qmv_core.h"

namespace kvp {
namespace {

constexpr int kBlock = 256;
constexpr int kWaves = kBlock / kWave;

__host__ __device__ constexpr size_t partial_floats(int head_dim) { return 2 + (size_t)head_dim; }

// Largest chunk a block takes: bounds the registers that hold a chunk's
// prefetched K and V codes.
template <int BITS>
__host__ __device__ constexpr int max_chunk() { return 128; }

struct KvArgs {
  const f16* q;
  const uint32_t* k_wq;
  const uint16_t* k_s;
  const uint16_t* k_b;
  const uint32_t* v_wq;
  const uint16_t* v_s;
  const uint16_t* v_b;
  const f16* new_k;
  const f16* new_v;
  const int32_t* t_cached;
  float* part;           // [B][H][n_chunks + 1][2 + DH] per-chunk (m, l, o), m in base-2
                         // units; slot n_chunks holds the new entry (s_new, 1, new_v)
  void* out;
  int out_f32;
  int n_heads, n_kv_heads, t_stride, chunk, n_chunks, per_seq;
  float scale;           // log2(e) / sqrt(DH)
};

// The 8-code block j of a row (codes 8j .. 8j+7) as the low 8*BITS bits of
// a 32-bit field (2-, 3- and 4-bit rows).
template <int BITS>
__device__ __forceinline__ uint32_t load_block8(const uint32_t* __restrict__ row, int j) {
  const int bit = j * 8 * BITS;
  const int w = bit >> 5, sh = bit & 31;
  if (sh + 8 * BITS <= 32) return row[w] >> sh;
  return __builtin_amdgcn_alignbit(row[w + 1], row[w], sh);
}

// The new entry of a block's G query heads as one more partial, slot
// n_chunks: m = s_new = q . new_k * scale (base 2), l = 1, o = new_v. Chunk 0
// of every (sequence, KV head) writes it, also for an empty cache, so the
// combine merges partials only.
template <int DH, int G>
__device__ __forceinline__ void write_new_entry(const KvArgs& a, int b, int hk) {
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const f16* nk = a.new_k + ((size_t)b * a.n_kv_heads + hk) * DH;
  const f16* nv = a.new_v + ((size_t)b * a.n_kv_heads + hk) * DH;
  for (int g = wave; g < G; g += kWaves) {  // wave-uniform
    const int h = hk * G + g;
    const f16* qh = a.q + ((size_t)b * a.n_heads + h) * DH;
    float s = 0.0f;
    for (int d = lane; d < DH; d += kWave) s = fmaf((float)qh[d], (float)nk[d], s);
    s = wave_sum(s) * a.scale;
    float* pp =
        a.part + (((size_t)b * a.n_heads + h) * (a.n_chunks + 1) + a.n_chunks) * partial_floats(DH);
    for (int d = lane; d < DH; d += kWave) pp[2 + d] = (float)nv[d];
    if (lane == 0) {
      pp[0] = s;
      pp[1] = 1.0f;
    }
  }
}

// Merge of the chunk partials of one query head and the new entry:
// M = max(m_c, s_new), L = sum l_c 2^(m_c-M) + 2^(s_new-M),
// out = (sum o_c 2^(m_c-M) + 2^(s_new-M) new_v) / L   (base-2 units).
// One block per (sequence, head, 16-dim slice): the 256 threads are 16
// chunk groups x 16 dims. Each thread folds its chunks into a running
// (M, L, O) as it reads them (one pass, every load issued up front), the
// sixteen group results meet once in LDS, and the new entry's score is
// formed by wave 0 while those loads are in flight.
constexpr int kCombDims = 16;
constexpr int kCombGroups = kBlock / kCombDims;

template <int DH, typename OutT>
__global__ __launch_bounds__(kBlock) void kv_combine_kernel(KvArgs a) {
  const int z = blockIdx.x;  // b * H + h
  const int b = z / a.n_heads;
  const int d0 = blockIdx.y * kCombDims;
  const int T = min(max(a.t_cached[b], 0), a.t_stride);  // as the split kernel clamps it
  const int nc = (T + a.chunk - 1) / a.chunk;
  __shared__ float gm[kCombGroups], gl[kCombGroups];
  __shared__ float go[kCombGroups][kCombDims];

  // Slots 0 .. nc - 1 are the chunks, slot n_chunks the new token. Every
  // slot's loads go out with the length's (they need not wait for it); the
  // slots from nc to n_chunks - 1 hold no partial of this call and are
  // skipped, never used in arithmetic.
  const float* pz = a.part + (size_t)z * (a.n_chunks + 1) * partial_floats(DH);
  const int dd = threadIdx.x % kCombDims, grp = threadIdx.x / kCombDims;
  float M = -INFINITY, L = 0.0f, O = 0.0f;
#pragma unroll 4
  for (int c = grp; c <= a.n_chunks; c += kCombGroups) {
    const float* pc = pz + c * partial_floats(DH);
    const float mc = pc[0], lc = pc[1], oc = pc[2 + d0 + dd];
    if (c < nc || c == a.n_chunks) {
      const float mn = fmaxf(M, mc);
      const float ea = exp2f(M - mn), eb = exp2f(mc - mn);  // first entry: ea = 2^-inf = 0
      L = fmaf(L, ea, lc * eb);
      O = fmaf(O, ea, oc * eb);
      M = mn;
    }
  }
  go[grp][dd] = O;
  if (dd == 0) {
    gm[grp] = M;
    gl[grp] = L;
  }
  __syncthreads();
  if (threadIdx.x < kCombDims) {
    float Mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < kCombGroups; ++i) Mx = fmaxf(Mx, gm[i]);
    float v = 0.0f, Lx = 0.0f;
#pragma unroll
    for (int i = 0; i < kCombGroups; ++i) {
      const float e = gl[i] > 0.0f ? exp2f(gm[i] - Mx) : 0.0f;  // groups without entries
      v = fmaf(go[i][dd], e, v);
      Lx = fmaf(gl[i], e, Lx);
    }
    store_out<OutT>(static_cast<OutT*>(a.out) + (size_t)z * DH + d0 + dd, v / Lx);
  }
}

template <int BITS, int DH, int G>
__global__ __launch_bounds__(kBlock) void kv_split_kernel(KvArgs a) {
  using Gm = Geom<BITS>;
  constexpr int U = DH * BITS / (8 * Gm::kUnitWords * 4);  // units per K row
  static_assert(U >= 1 && kWave % U == 0, "a K row must split evenly over lanes");
  constexpr int kRowsPerPass = kWave / U;                   // K rows per wave pass
  constexpr int kRowWords = DH * BITS / 32;
  constexpr int kGroups = DH / 64;
  constexpr int kBlocks8 = DH / 8;                          // 8-code blocks per row
  constexpr int kVRowsPerPass = kWave / kBlocks8;           // V rows per wave pass
  constexpr int kXW = Gm::kUnitCodes / 2;                   // fp16 pairs of a unit
  constexpr int kMaxChunk = max_chunk<BITS>();
  constexpr int KP = (kMaxChunk + kWaves * kRowsPerPass - 1) / (kWaves * kRowsPerPass);
  constexpr int VP = (kMaxChunk + kWaves * kVRowsPerPass - 1) / (kWaves * kVRowsPerPass);
  constexpr int kVW = BITS == 8 ? 2 : 1;                    // words of an 8-code block

  extern __shared__ float sc[];  // [G][chunk] scores, then probabilities
  __shared__ float red[kWaves][G];
  __shared__ float stat_m[G], stat_l[G];
  __shared__ float obuf[kWaves][G][DH];

  const int c = blockIdx.x, hk = blockIdx.y, b = blockIdx.z;
  // Lengths outside [0, t_stride] are clamped: the cache is never read past
  // its allocation whatever the caller passes.
  const int T = min(max(a.t_cached[b], 0), a.t_stride);
  const int nc = (T + a.chunk - 1) / a.chunk;
  if (c == 0) write_new_entry<DH, G>(a, b, blockIdx.y);
  if (c >= nc) return;  // chunk past this sequence: no partial (block-uniform)

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int h0 = hk * G;

  {
    const int t0 = c * a.chunk;
    const int n = min(a.chunk, T - t0);
    const size_t cache_base = ((size_t)(a.per_seq ? b : 0) * a.n_kv_heads + hk) * a.t_stride + t0;
    const int part = lane % U;
    const int grp = (part * Gm::kUnitCodes) / 64;
    const int j = lane % kBlocks8;  // V: 8-code block, dims 8j .. 8j+7
    const int vgrp = (8 * j) / 64;

    // --- every load of the chunk goes out first: q, then K, then V --------
    uint32_t nat[G][kXW];
    {
      const uint32_t* qw =
          reinterpret_cast<const uint32_t*>(a.q + ((size_t)b * a.n_heads + h0) * DH);
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int i = 0; i < kXW; i += 4) {
          const u32x4 v =
              *reinterpret_cast<const u32x4*>(qw + (g * DH + part * Gm::kUnitCodes) / 2 + i);
          nat[g][i] = v.x; nat[g][i + 1] = v.y; nat[g][i + 2] = v.z; nat[g][i + 3] = v.w;
        }
    }
    uint32_t kw[KP][1][Gm::kUnitWords];
    f16x2 ksb[KP];
#pragma unroll
    for (int p = 0; p < KP; ++p) {
      const int tr = (p * kWaves + wave) * kRowsPerPass + lane / U;
      const size_t row = cache_base + min(tr, n - 1);
      load_unit<BITS>(a.k_wq + row * kRowWords + part * Gm::kUnitWords, kw[p][0]);
      ksb[p] = f16x2{__builtin_bit_cast(f16, a.k_s[row * kGroups + grp]),
                     __builtin_bit_cast(f16, a.k_b[row * kGroups + grp])};
    }
    uint32_t vw[VP][kVW];
    f16x2 vsb[VP];
#pragma unroll
    for (int p = 0; p < VP; ++p) {
      const int tr = (p * kWaves + wave) * kVRowsPerPass + lane / kBlocks8;
      const size_t row = cache_base + min(tr, n - 1);
      const uint32_t* vrow = a.v_wq + row * kRowWords;
      if constexpr (BITS == 8) {
        const u32x2 v = *reinterpret_cast<const u32x2*>(vrow + 2 * j);
        vw[p][0] = v.x;
        vw[p][1] = v.y;
      } else {
        vw[p][0] = load_block8<BITS>(vrow, j);
      }
      vsb[p] = f16x2{__builtin_bit_cast(f16, a.v_s[row * kGroups + vgrp]),
                     __builtin_bit_cast(f16, a.v_b[row * kGroups + vgrp])};
    }

    // --- query slice in weight-word pair order ------------------------------
    uint32_t qp[G * Gm::kUnitPairs];
    float qsum[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float s = 0.0f;
#pragma unroll
      for (int i = 0; i < kXW; ++i) s = dot2(nat[g][i], 0x3C003C00u, s);
      qsum[g] = s;
      if constexpr (Gm::kMagic) {
        constexpr int H = Gm::kPairsPerWord;
#pragma unroll
        for (int wi = 0; wi < Gm::kUnitWords; ++wi)
          pair_order<BITS>(&nat[g][wi * (Gm::kCodesPerWord / 2)], &qp[(g * Gm::kSlots + wi) * H]);
      } else {
#pragma unroll
        for (int i = 0; i < kXW; ++i) qp[g * kXW + i] = nat[g][i];
      }
    }

    // --- scores ---------------------------------------------------------------
#pragma unroll
    for (int p = 0; p < KP; ++p) {
      const int tr = (p * kWaves + wave) * kRowsPerPass + lane / U;
      if ((p * kWaves + wave) * kRowsPerPass >= n) break;  // wave-uniform
      float d[1][G];
      unit_dot<BITS, G, 1>(kw[p], qp, Gm::kSlotPairs, d);
      const float s = (float)ksb[p].x, bias = (float)ksb[p].y;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float v = fmaf(s, d[0][g], bias * qsum[g]);
#pragma unroll
        for (int off = 1; off < U; off <<= 1) v += __shfl_xor(v, off, U);
        if (part == 0 && tr < n) sc[g * a.chunk + tr] = v * a.scale;
      }
    }
    __syncthreads();

    // --- chunk softmax statistics per head ----------------------------------
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float m = -INFINITY;
      for (int t = threadIdx.x; t < n; t += kBlock) m = fmaxf(m, sc[g * a.chunk + t]);
      m = wave_max(m);
      if (lane == 0) red[wave][g] = m;
    }
    __syncthreads();
    if (threadIdx.x < G) {
      float m = red[0][threadIdx.x];
      for (int i = 1; i < kWaves; ++i) m = fmaxf(m, red[i][threadIdx.x]);
      stat_m[threadIdx.x] = m;
    }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float m = stat_m[g];
      float l = 0.0f;
      for (int t = threadIdx.x; t < n; t += kBlock) {
        const float e = exp2f(sc[g * a.chunk + t] - m);
        sc[g * a.chunk + t] = e;
        l += e;
      }
      l = wave_sum(l);
      if (lane == 0) red[wave][g] = l;
    }
    __syncthreads();
    if (threadIdx.x < G) {
      float l = 0.0f;
      for (int i = 0; i < kWaves; ++i) l += red[i][threadIdx.x];
      stat_l[threadIdx.x] = l;
    }

    // --- values: o[g][d] = sum_t p[g][t] * (s_t * q_td + b_t) ----------------
    float acc[G][8];
    float pbias[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      pbias[g] = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[g][i] = 0.0f;
    }
#pragma unroll
    for (int p = 0; p < VP; ++p) {
      if ((p * kWaves + wave) * kVRowsPerPass >= n) break;  // wave-uniform
      const int tr = (p * kWaves + wave) * kVRowsPerPass + lane / kBlocks8;
      const bool valid = tr < n;
      float codes[8];
      if constexpr (BITS == 8) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          codes[i] = (float)((vw[p][0] >> (8 * i)) & 0xFFu);
          codes[4 + i] = (float)((vw[p][1] >> (8 * i)) & 0xFFu);
        }
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) codes[i] = (float)((vw[p][0] >> (BITS * i)) & ((1u << BITS) - 1u));
      }
      const float s = (float)vsb[p].x, bias = (float)vsb[p].y;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float pr = valid ? sc[g * a.chunk + min(tr, n - 1)] : 0.0f;
        const float ps = pr * s;
        pbias[g] = fmaf(pr, bias, pbias[g]);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[g][i] = fmaf(ps, codes[i], acc[g][i]);
      }
    }
    // Lanes with the same block j hold disjoint positions: add them up.
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float v = acc[g][i] + pbias[g];
#pragma unroll
        for (int off = kBlocks8; off < kWave; off <<= 1) v += __shfl_xor(v, off, kWave);
        acc[g][i] = v;
      }
    if (lane < kBlocks8) {
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int i = 0; i < 8; ++i) obuf[wave][g][8 * j + i] = acc[g][i];
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < G * DH; idx += kBlock) {
      const int g = idx / DH, dd = idx - g * DH;
      float v = 0.0f;
#pragma unroll
      for (int i = 0; i < kWaves; ++i) v += obuf[i][g][dd];
      float* pp = a.part + (((size_t)b * a.n_heads + h0 + g) * (a.n_chunks + 1) + c) * partial_floats(DH);
      pp[2 + dd] = v;
      if (dd == 0) {
        pp[0] = stat_m[g];
        pp[1] = stat_l[g];
      }
    }
  }

}

// ---------------------------------------------------------------------------
// Matrix-core split kernel (4- and 8-bit caches, G <= 8 query heads per KV
// head): one block per (slice of positions, KV head, sequence). Its four
// waves work independently on steps of 64 positions (32 when G > 4; step t
// of the slice goes to wave t % 4), each keeping an exact online softmax per
// head in the base-2 domain, and merge once at the end.
//
// Scores: S[h][n] = sum_g s_n,g (Q K_g^T)[h][n] + b_n,g qsum_g[h] over the
// 64-dim groups g, on v_mfma_f32_16x16x32_f16 with the 16 rows of A taken
// by (position tile, head) pairs: 4 tiles x 4 heads (2 x 8 when G > 4). A's
// 32-wide k is split the same way, so A carries the query block-diagonally
// (a slice of a head's row where the tiles match, zeros elsewhere; read from
// a small LDS table) and B carries each tile's codes as exact fp16
// denormals (c -> c * 2^-24, folded into the score scale). The output then
// gives every lane its own position's scores for its heads: no padding
// rows, and the softmax works on 4 values per lane and step.
//
// Values, one v_mfma_f32_16x16x32_f16 per 16 dims and 32 positions:
//   O[h][d] = sum_n p[h][n] s_n,g(d) c[n][d] + sum_n p[h][n] b_n,g(d).
// The first sum runs on the matrix cores: B = the codes (exact fp16
// denormals), A = x = p * s * 2^E carried as an unevaluated sum of two fp16
// values, hi = rne(x) and lo = rne(x - hi) (22 significant bits; every
// product exact; fp32 accumulation). The 16 rows of A are the pairs
// (group, hi/lo, head), so one instruction serves every head and both
// parts; the two parts are added once at the end. E is a power-of-two range
// shift per group chosen from the largest V scale seen so far so that
// x < 2^15; a larger scale later lowers E and rescales the accumulators by
// the exact power of two. The second sum (p * b) stays on the VALU in fp32.
// A lane of the value instruction owns one code word of a V row (its column
// of 16 dims) at 8 consecutive positions (its K-rows).
// ---------------------------------------------------------------------------
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));


template <int BITS>
__device__ __forceinline__ f16x8 codes8_f16(const uint32_t* w) {
  // Eight codes (dims 8k .. 8k+7 of a row) as fp16 denormals, in order.
  uint32_t h[4];
  if constexpr (BITS == 4) {
    const uint32_t even = w[0] & 0x0F0F0F0Fu, odd = (w[0] >> 4) & 0x0F0F0F0Fu;
    h[0] = __builtin_amdgcn_perm(odd, even, 0x0C040C00u);
    h[1] = __builtin_amdgcn_perm(odd, even, 0x0C050C01u);
    h[2] = __builtin_amdgcn_perm(odd, even, 0x0C060C02u);
    h[3] = __builtin_amdgcn_perm(odd, even, 0x0C070C03u);
  } else {
    h[0] = __builtin_amdgcn_perm(0u, w[0], 0x0C010C00u);
    h[1] = __builtin_amdgcn_perm(0u, w[0], 0x0C030C02u);
    h[2] = __builtin_amdgcn_perm(0u, w[1], 0x0C010C00u);
    h[3] = __builtin_amdgcn_perm(0u, w[1], 0x0C030C02u);
  }
  return __builtin_bit_cast(f16x8, u32x4{h[0], h[1], h[2], h[3]});
}

// Reductions over the 16 lanes of a DPP row; every lane of the row gets the
// same (bit-identical) result.
// (Every source lane of these patterns lies inside the row, so bound_ctrl's
// zero fill never applies; it spares the old-value initialisation.)
__device__ __forceinline__ float lane_value(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}
// 2^e as a float for -126 <= e <= 127; 0 below.
__device__ __forceinline__ float exp2_int(int e) {
  return e < -126 ? 0.0f : __builtin_bit_cast(float, (uint32_t)(e + 127) << 23);
}

template <int BITS, int DH, int G>
struct KvShape {
  static constexpr int kGp = G <= 4 ? 4 : 8;        // score rows per tile: heads, padded
  static constexpr int kTPS = 16 / kGp;             // position tiles per step
  static constexpr int kP = 16 * kTPS;              // positions per step
  static constexpr int kHalves = kP / 32;           // 32-position blocks of the value side
  static constexpr int kSub = 4 / kTPS;             // 8-dim k-blocks per tile and instruction
  static constexpr int kDPM = 8 * kSub;             // dims of a tile per score instruction
  static constexpr int kNM = DH / kDPM;             // score instructions per step
  static constexpr int kGroups = DH / 64;
  static constexpr int kRowWords = DH * BITS / 32;
  static constexpr int kKW = BITS == 8 ? 2 : 1;     // words per 8 codes
  static constexpr int kKWords = kNM * kKW;         // K words a lane holds per step
  static constexpr int kVW = (BITS == 8 && DH == 128) ? 2 : 1;  // V words per lane and position
  static constexpr int kNB = DH / 16;               // value instructions per row set
  static constexpr int kHR = DH == 128 ? 4 : 8;     // heads per value row set
  static constexpr int kSets = (G + kHR - 1) / kHR;
};

// What a lane loads for one step.
template <int BITS, int DH, int G>
struct KvStepRegs {
  using S = KvShape<BITS, DH, G>;
  uint32_t kw[S::kKWords];              // K codes of the lane's score position (its k-blocks)
  uint32_t ks, kbias, vs, vbias;        // scales / biases there (groups packed)
  uint32_t vw[S::kHalves][8][S::kVW];   // V codes: positions 32 hf + 8 kb + j, column word
};

// Buffer resources over one block's slice of the six cache arrays. A read
// past the slice's last row returns zeros (the hardware range check), so
// the loads of a partial last step need no clamping: zero K codes and
// scales give finite scores that the step masks, zero V scales give x = 0.
struct SliceRsrc {
  __amdgpu_buffer_rsrc_t kw, ks, kb, vw, vs, vb;
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t slice_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

template <int BITS, int DH, int G>
__device__ __forceinline__ void load_step(KvStepRegs<BITS, DH, G>& R, const SliceRsrc& rs, int p0,
                                          int lane) {
  using S = KvShape<BITS, DH, G>;
  constexpr uint32_t kRB = S::kRowWords * 4;  // bytes per cache row
  const int n16 = lane % 16, kb = lane / 16;
  const int sub = kb % S::kSub;
  // The lane's score position: tile kb / kSub, row n16. Lane byte offsets;
  // the per-step part p0 * row bytes is uniform, the rest immediates.
  const uint32_t pos = (uint32_t)(p0 + 16 * (kb / S::kSub) + n16);
  const uint32_t ko = pos * kRB;
  if constexpr (S::kSub == 1) {  // the whole row, 16 bytes at a time
#pragma unroll
    for (int w = 0; w < S::kKWords; w += 4) {
      const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rs.kw, ko + 4 * w, 0, 0);
      R.kw[w] = v.x;
      R.kw[w + 1] = v.y;
      R.kw[w + 2] = v.z;
      R.kw[w + 3] = v.w;
    }
  } else {  // the lane's 8-dim block of every 16-dim chunk
#pragma unroll
    for (int s = 0; s < S::kNM; ++s) {
      const uint32_t o = ko + (uint32_t)((2 * s + sub) * S::kKW * 4);
      if constexpr (S::kKW == 1) {
        R.kw[s] = __builtin_amdgcn_raw_buffer_load_b32(rs.kw, o, 0, 0);
      } else {
        const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(rs.kw, o, 0, 0);
        R.kw[2 * s] = v.x;
        R.kw[2 * s + 1] = v.y;
      }
    }
  }
  const uint32_t so = pos * 2 * S::kGroups;
  if constexpr (S::kGroups == 2) {
    R.ks = __builtin_amdgcn_raw_buffer_load_b32(rs.ks, so, 0, 0);
    R.kbias = __builtin_amdgcn_raw_buffer_load_b32(rs.kb, so, 0, 0);
    R.vs = __builtin_amdgcn_raw_buffer_load_b32(rs.vs, so, 0, 0);
    R.vbias = __builtin_amdgcn_raw_buffer_load_b32(rs.vb, so, 0, 0);
  } else {
    R.ks = __builtin_amdgcn_raw_buffer_load_b16(rs.ks, so, 0, 0);
    R.kbias = __builtin_amdgcn_raw_buffer_load_b16(rs.kb, so, 0, 0);
    R.vs = __builtin_amdgcn_raw_buffer_load_b16(rs.vs, so, 0, 0);
    R.vbias = __builtin_amdgcn_raw_buffer_load_b16(rs.vb, so, 0, 0);
  }
  // The lane's column word: 4-bit DH 128 word n16 (dims 8 n16 ..), 8-bit
  // DH 128 words 2 n16, 2 n16 + 1 (dims 8 n16 ..), 4-bit DH 64 word n16 % 8,
  // 8-bit DH 64 word n16 (dims 4 n16 ..).
  const int col = (BITS == 4 && DH == 64) ? n16 % 8 : n16;
#pragma unroll
  for (int hf = 0; hf < S::kHalves; ++hf) {
    const uint32_t vo = (uint32_t)(p0 + 32 * hf + 8 * kb) * kRB + col * 4 * S::kVW;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if constexpr (S::kVW == 2) {
        const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(rs.vw, vo + j * kRB, 0, 0);
        R.vw[hf][j][0] = v.x;
        R.vw[hf][j][1] = v.y;
      } else {
        R.vw[hf][j][0] = __builtin_amdgcn_raw_buffer_load_b32(rs.vw, vo + j * kRB, 0, 0);
      }
    }
  }
}

// Dim of code `nb` in column n16 of the value instruction.
template <int BITS, int DH>
__device__ __forceinline__ int value_dim(int n16, int nb) {
  if constexpr (DH == 128) return 8 * n16 + nb;
  else if constexpr (BITS == 4) return 8 * (n16 % 8) + 4 * (n16 / 8) + nb;
  else return 4 * n16 + nb;
}

// B operand of value instruction nb: element j = code nb of the lane's
// column at position 8 kb + j, as an fp16 denormal. `pl` holds the 4-bit
// nibble planes (even, odd) or the 8-bit words.
template <int BITS, int DH, int NB>
__device__ __forceinline__ f16x8 value_codes(const uint32_t (&pl)[8][2]) {
  uint32_t h[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    if constexpr (BITS == 4) {
      constexpr int k = NB >> 1;  // byte of the plane
      constexpr uint32_t sel = 0x0C000C00u | ((4u + k) << 16) | (uint32_t)k;
      h[p] = __builtin_amdgcn_perm(pl[2 * p + 1][NB & 1], pl[2 * p][NB & 1], sel);
    } else {
      constexpr int k = NB & 3;
      constexpr uint32_t sel = 0x0C000C00u | ((4u + k) << 16) | (uint32_t)k;
      h[p] = __builtin_amdgcn_perm(pl[2 * p + 1][NB >> 2], pl[2 * p][NB >> 2], sel);
    }
  }
  return __builtin_bit_cast(f16x8, u32x4{h[0], h[1], h[2], h[3]});
}

// Wave-wide max of an int / float (every lane gets it).
__device__ __forceinline__ int wave_max_i(int v) {
  v = row16_max_i(v);
  return max(max(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
             max(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}

template <int BITS, int DH, int G>
__global__ __launch_bounds__(kBlock) void kv_mfma_split_kernel(KvArgs a) {
  using S = KvShape<BITS, DH, G>;
  constexpr int kGroups = S::kGroups, kGp = S::kGp, kP = S::kP, kHR = S::kHR, kSets = S::kSets;
  constexpr int kHp = kGp;                        // heads per LDS x row
  constexpr int kXS = kGroups * kHp;              // floats per position in xbuf
  constexpr int kXWave = kP * kXS + (kP / 8) * 8; // + 8 floats per 8 positions (bank spread)
  // Lazy rescale: the max in use may trail the running max by up to 2^kLazy
  // (p <= 2^kLazy), so accumulators are rescaled only when a score rises
  // further; the range shift leaves room for it (x < 2^15).
  constexpr float kLazy = 8.0f;
  constexpr int kEBase = 21;                      // E = kEBase - exponent field of max |s|
  static_assert(G <= 8, "at most 8 query heads per KV head");
  __shared__ __align__(16) _Float16 qtab[(G + 1) * DH];  // the G query rows, then zeros
  __shared__ float qss_sh[G][kGroups];
  __shared__ __align__(16) float xbuf[kWaves][kXWave];
  __shared__ float wm[kWaves][G], wl[kWaves][G];
  __shared__ __align__(16) float wo[kWaves][G][DH];   // hi parts, + p * b
  __shared__ __align__(16) float wol[kWaves][G][DH];  // lo parts

  const int c = blockIdx.x, hk = blockIdx.y, b = blockIdx.z;
  const int slice0 = c * a.chunk;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);  // wave-uniform
  const int n16 = lane % 16, q4 = lane / 16;
  const int h0 = hk * G;
  const size_t base = ((size_t)(a.per_seq ? b : 0) * a.n_kv_heads + hk) * a.t_stride + slice0;
  float* xw = xbuf[wave];
  auto xaddr = [](int pos, int g, int h) { return pos * kXS + (pos / 8) * 8 + g * kHp + h; };

  // With one sequence the slice's first cache loads do not wait for the
  // length: they cover the slice within t_stride (every block of the grid
  // starts inside it), the length load travels beside them, and positions
  // at or past T are masked out of the softmax (their scores are -inf, so
  // p = 0 and they add nothing). Only a block wholly past the sequence's end
  // wastes them. With several sequences of different lengths such blocks
  // are common (config 4: 11.7 MB of 120 MB fetched, 1.108 x the algorithmic
  // bytes), so there the loads wait for the length and stop at it (measured:
  // config 4 45.2 -> 44.2 us; one sequence 32k 16.17 -> 16.72 us without the
  // early loads).
  const bool early = gridDim.z == 1;  // grid-uniform
  const int n_max = min(a.chunk, a.t_stride - slice0);
  SliceRsrc rs;
  {
    const uint32_t rb = S::kRowWords * 4, sb = 2 * kGroups;
    rs.kw = slice_rsrc(a.k_wq + base * S::kRowWords, n_max * rb);
    rs.vw = slice_rsrc(a.v_wq + base * S::kRowWords, n_max * rb);
    rs.ks = slice_rsrc(a.k_s + base * kGroups, n_max * sb);
    rs.kb = slice_rsrc(a.k_b + base * kGroups, n_max * sb);
    rs.vs = slice_rsrc(a.v_s + base * kGroups, n_max * sb);
    rs.vb = slice_rsrc(a.v_b + base * kGroups, n_max * sb);
  }
  // Double-buffered: the next step's loads are in flight while this one is
  // processed. A step past the last one loads from one past the slice: out
  // of the buffers' range, it reads zeros without traffic.
  KvStepRegs<BITS, DH, G> RA, RB;
  // The small inputs go out before the first cache loads, so (returns being
  // in order) they are in registers while the cache is still in flight: the
  // query table (G rows, then a zero row; at most one 16-byte item per
  // thread) and, in chunk 0, the new entry's q . new_k operands and new_v.
  static_assert((G + 1) * (DH / 8) <= kBlock, "one query-table item per thread");
  const int qi_row = threadIdx.x / (DH / 8), qi_c8 = threadIdx.x % (DH / 8);
  u32x4 qv = {0, 0, 0, 0};
  if (qi_row < G)
    qv = *reinterpret_cast<const u32x4*>(a.q + ((size_t)b * a.n_heads + h0 + qi_row) * DH +
                                         8 * qi_c8);
  constexpr int kNE = (G + kWaves - 1) / kWaves, kND = DH / kWave;  // heads per wave, dims per lane
  float ne_q[kNE][kND], ne_k[kNE][kND], ne_v[kNE][kND];
  if (c == 0) {
#pragma unroll
    for (int e = 0; e < kNE; ++e) {
      const int g = min(wave + kWaves * e, G - 1);
      const f16* qh = a.q + ((size_t)b * a.n_heads + h0 + g) * DH;
      const f16* nk = a.new_k + ((size_t)b * a.n_kv_heads + hk) * DH;
      const f16* nv = a.new_v + ((size_t)b * a.n_kv_heads + hk) * DH;
#pragma unroll
      for (int i = 0; i < kND; ++i) {
        ne_q[e][i] = (float)qh[lane + kWave * i];
        ne_k[e][i] = (float)nk[lane + kWave * i];
        ne_v[e][i] = (float)nv[lane + kWave * i];
      }
    }
  }

  if (early && wave * kP < n_max) load_step<BITS, DH, G>(RA, rs, kP * wave, lane);
  const int T = min(max(a.t_cached[b], 0), a.t_stride);
  if (slice0 >= T) {  // block-uniform
    if (c == 0) write_new_entry<DH, G>(a, b, hk);
    return;
  }
  const int n = min(a.chunk, T - slice0);
  if (!early && wave * kP < n) load_step<BITS, DH, G>(RA, rs, kP * wave, lane);
  const int nsteps = (n + kP - 1) / kP;
  auto step_pos = [&](int t) { return t < nsteps ? kP * t : a.chunk + kP; };

  if (qi_row <= G) *reinterpret_cast<u32x4*>(&qtab[qi_row * DH + 8 * qi_c8]) = qv;
  // The new entry's partial (slot n_chunks: m = q . new_k * scale, l = 1,
  // o = new_v), while the first cache loads are in flight.
  if (c == 0) {
#pragma unroll
    for (int e = 0; e < kNE; ++e) {
      const int g = wave + kWaves * e;
      if (g < G) {  // wave-uniform
        float sdot = 0.0f;
#pragma unroll
        for (int i = 0; i < kND; ++i) sdot = fmaf(ne_q[e][i], ne_k[e][i], sdot);
        sdot = wave_sum(sdot) * a.scale;
        float* pp = a.part + (((size_t)b * a.n_heads + h0 + g) * (a.n_chunks + 1) + a.n_chunks) *
                                 partial_floats(DH);
#pragma unroll
        for (int i = 0; i < kND; ++i) pp[2 + lane + kWave * i] = ne_v[e][i];
        if (lane == 0) {
          pp[0] = sdot;
          pp[1] = 1.0f;
        }
      }
    }
  }
  __syncthreads();
  {
    const int item = threadIdx.x / 16, part = threadIdx.x % 16;  // 16 lanes per (head, group)
    float sq = 0.0f;
    if (item < G * kGroups) {
      const int hh = item / kGroups, g = item % kGroups;
#pragma unroll
      for (int k = 0; k < 4; ++k) sq += (float)qtab[hh * DH + 64 * g + 4 * part + k];
    }
    sq = row16_sum(sq);
    if (item < G * kGroups && part == 0) qss_sh[item / kGroups][item % kGroups] = sq * a.scale;
  }
  __syncthreads();

  // Score layout: lane holds position 16 (q4 / kSub) + n16 of the step for
  // heads hd(i) = (kGp == 4 ? i : 4 (q4 % 2) + i), i = 0..3.
  const int spos = 16 * (q4 / S::kSub) + n16;
  const int hbase = kGp == 4 ? 0 : 4 * (q4 % 2);
  float qss[kGroups][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int g = 0; g < kGroups; ++g) qss[g][i] = qss_sh[min(hbase + i, G - 1)][g];
  // Score A operand: row m = n16 is (tile m / kGp, head m % kGp), k-block q4
  // is (tile q4 / kSub, dims 8 (q4 % kSub) ..): the query slice on the
  // block diagonal, zeros elsewhere (the zero row of the table).
  const int qrow = (n16 / kGp == q4 / S::kSub && n16 % kGp < G) ? n16 % kGp : G;
  const _Float16* qa = &qtab[qrow * DH + 8 * (q4 % S::kSub)];

  float mrow[4], l[4], pb[4][kGroups];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    mrow[i] = -INFINITY;
    l[i] = 0.0f;
#pragma unroll
    for (int g = 0; g < kGroups; ++g) pb[i][g] = 0.0f;
  }
  f32x4 acc[kSets][S::kNB];
#pragma unroll
  for (int st = 0; st < kSets; ++st)
#pragma unroll
    for (int nb = 0; nb < S::kNB; ++nb) acc[st][nb] = f32x4{0, 0, 0, 0};
  int E0 = 127, E1 = 127;  // range shift of groups 0 / 1 (uniform); 127 = no nonzero scale yet
  uint32_t thr = 0;        // per 16-bit half: largest |V scale| bits the current E admits

  const float scale24 = a.scale * 16777216.0f;  // base-2 softmax scale x 2^24 (denormal codes)
  // Value A operand row of this lane: (group, hi/lo part, head).
  const int g_r = DH == 128 ? n16 >> 3 : 0;
  const int hl_r = DH == 128 ? (n16 & 3) : (n16 & 7);
  const float lo_r = (DH == 128 ? (n16 >> 2) & 1 : n16 >> 3) ? 1.0f : 0.0f;

  auto process = [&](const KvStepRegs<BITS, DH, G>& R, int t) {
    const int p0 = kP * t;
    // --- scores: kTPS tiles stacked on the rows of each instruction -----------
    f32x4 d[kGroups];
#pragma unroll
    for (int g = 0; g < kGroups; ++g) d[g] = f32x4{0, 0, 0, 0};
#pragma unroll
    for (int s = 0; s < S::kNM; ++s) {
      const f16x8 av = *reinterpret_cast<const f16x8*>(qa + S::kDPM * s);
      constexpr int kPerGroup = 64 / S::kDPM;
      d[s / kPerGroup] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
          av, codes8_f16<BITS>(&R.kw[s * S::kKW]), d[s / kPerGroup], 0, 0, 0);
    }
    float sv[4];
    {
      float sgS[kGroups], bg[kGroups];
#pragma unroll
      for (int g = 0; g < kGroups; ++g) {
        sgS[g] = f16_bits_to_f32((uint16_t)(R.ks >> (16 * g))) * scale24;
        bg[g] = f16_bits_to_f32((uint16_t)(R.kbias >> (16 * g)));
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float v = 0.0f;
#pragma unroll
        for (int g = 0; g < kGroups; ++g) v = fmaf(sgS[g], d[g][i], fmaf(bg[g], qss[g][i], v));
        sv[i] = v;
      }
    }
    // V scale and bias of this lane's score position; positions past the
    // sequence's end (read only in its partial last step) get zeros, so
    // whatever a padded cache holds there (even NaN patterns) adds nothing.
    uint32_t vs_l = R.vs, vb_l = R.vbias;
    if (p0 + kP > n) {  // the slice's partial last step (uniform)
      const bool valid = p0 + spos < n;
#pragma unroll
      for (int i = 0; i < 4; ++i) sv[i] = valid ? sv[i] : -INFINITY;
      vs_l = valid ? vs_l : 0u;
      vb_l = valid ? vb_l : 0u;
    }
    // --- the max in use: moves only when a score outruns it by 2^kLazy ---------
    uint64_t rise = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (kGp == 8 || i < G)  // heads past G (zero query rows) never move the max
        rise |= __builtin_amdgcn_ballot_w64(sv[i] > mrow[i] + kLazy);
    const bool raise = rise != 0;  // wave-uniform
    // --- range shift: a V scale larger than the current E admits -----------------
    const uint32_t ub = vs_l & 0x7FFF7FFFu;
    const bool over = __builtin_bit_cast(uint32_t, __builtin_elementwise_max(
                                                       __builtin_bit_cast(u16x2, ub),
                                                       __builtin_bit_cast(u16x2, thr))) != thr;
    // One rare, wave-uniform slow path for both: a new max in use and a
    // lower range shift, each an exact rescale of what has accumulated.
    if (raise || __builtin_amdgcn_ballot_w64(over) != 0) {
      const int e0 = wave_max_i((int)(ub & 0xFFFFu)) >> 10;
      const int n0 = min(E0, kEBase - e0);
      const float fE0 = exp2_int(n0 - E0);
      E0 = n0;
      uint32_t nthr = (uint32_t)(((kEBase + 1 - n0) << 10) - 1);
      float fE1 = fE0;
      if constexpr (kGroups == 2) {
        const int e1 = wave_max_i((int)(ub >> 16)) >> 10;
        const int n1 = min(E1, kEBase - e1);
        fE1 = exp2_int(n1 - E1);
        E1 = n1;
        nthr |= (uint32_t)(((kEBase + 1 - n1) << 10) - 1) << 16;
      }
      thr = nthr;
      float csel[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float mn = mrow[i];
        if (raise) {
          // max over the lanes holding head hd(i): the whole wave (kGp 4) or
          // score rows q4 and q4 ^ 2 (kGp 8)
          const float r = row16_max(sv[i]);
          const float rA = fmaxf(lane_value(r, 0), lane_value(r, 32));
          const float rB = fmaxf(lane_value(r, 16), lane_value(r, 48));
          const float hm = kGp == 4 ? fmaxf(rA, rB) : ((q4 & 1) ? rB : rA);
          mn = fmaxf(mrow[i], hm);
        }
        csel[i] = __builtin_amdgcn_exp2f(mrow[i] - mn);  // 1 without a raise
        mrow[i] = mn;
        l[i] *= csel[i];
#pragma unroll
        for (int g = 0; g < kGroups; ++g) pb[i][g] *= csel[i];
      }
#pragma unroll
      for (int st = 0; st < kSets; ++st) {
        float f[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          // value rows of this lane: head kHR st + i (DH 128) or 4 (q4 % 2) + i
          // (DH 64); their factor sits in score row st (kGp 8, DH 128) or in
          // this lane's own score row
          const float ch = (kGp == 8 && DH == 128) ? lane_value(csel[i], 16 * st) : csel[i];
          f[i] = ch * ((DH == 128 && (q4 >> 1)) ? fE1 : fE0);
        }
#pragma unroll
        for (int nb = 0; nb < S::kNB; ++nb)
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[st][nb][i] *= f[i];
      }
    }
    // --- p, l, p * b, and x = p * s * 2^E into LDS (position, group, head) ------
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      p[i] = __builtin_amdgcn_exp2f(sv[i] - mrow[i]);
      l[i] += p[i];
    }
    const float sE0 = exp2_int(E0), sE1 = exp2_int(E1);
#pragma unroll
    for (int g = 0; g < kGroups; ++g) {
      const float vsg = f16_bits_to_f32((uint16_t)(vs_l >> (16 * g))) * (g ? sE1 : sE0);
      const float vbg = f16_bits_to_f32((uint16_t)(vb_l >> (16 * g)));
      f32x4 x;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        x[i] = p[i] * vsg;
        pb[i][g] = fmaf(p[i], vbg, pb[i][g]);
      }
      *reinterpret_cast<f32x4*>(&xw[xaddr(spos, g, hbase)]) = x;
    }
    // The x rows written above are read below by other lanes of this wave: a
    // wave's LDS operations execute in program order, so keeping the compiler
    // from moving them across this point is enough.
    __builtin_amdgcn_wave_barrier();
    // --- values on the matrix cores, 32 positions per instruction --------------
#pragma unroll
    for (int hf = 0; hf < S::kHalves; ++hf) {
      uint32_t pl[8][2];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if constexpr (BITS == 4) {
          const uint32_t w = DH == 64 ? (n16 >= 8 ? R.vw[hf][j][0] >> 16 : R.vw[hf][j][0])
                                      : R.vw[hf][j][0];
          pl[j][0] = w & 0x0F0F0F0Fu;
          pl[j][1] = (w >> 4) & 0x0F0F0F0Fu;
        } else {
          pl[j][0] = R.vw[hf][j][0];
          pl[j][1] = S::kVW == 2 ? R.vw[hf][j][S::kVW - 1] : 0u;
        }
      }
#pragma unroll
      for (int st = 0; st < kSets; ++st) {
        const int h = min(kHR * st + hl_r, G - 1);  // rows past G repeat a real head
        f16x8 av;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float xv = xw[xaddr(32 * hf + 8 * q4 + j, g_r, h)];
          const _Float16 hi = (_Float16)xv;
          av[j] = (_Float16)fmaf(-lo_r, (float)hi, xv);
        }
        auto mm = [&](auto nbc) {
          constexpr int NB = decltype(nbc)::value;
          acc[st][NB] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, value_codes<BITS, DH, NB>(pl),
                                                              acc[st][NB], 0, 0, 0);
        };
        mm(std::integral_constant<int, 0>{});
        mm(std::integral_constant<int, 1>{});
        mm(std::integral_constant<int, 2>{});
        mm(std::integral_constant<int, 3>{});
        if constexpr (S::kNB == 8) {
          mm(std::integral_constant<int, 4>{});
          mm(std::integral_constant<int, 5>{});
          mm(std::integral_constant<int, 6>{});
          mm(std::integral_constant<int, 7>{});
        }
      }
    }
    __builtin_amdgcn_wave_barrier();  // xbuf is rewritten by the next step
  };

  if (wave < nsteps) {
    // The next step's loads are issued before this step's work,
    // unconditionally, so the wait before each step covers exactly the
    // older set.
    int t = wave;
    const int last = nsteps - 1;
    for (;;) {
      load_step<BITS, DH, G>(RB, rs, step_pos(t + kWaves), lane);
      process(RA, t);
      t += kWaves;
      if (t > last) break;
      load_step<BITS, DH, G>(RA, rs, step_pos(t + kWaves), lane);
      process(RB, t);
      t += kWaves;
      if (t > last) break;
    }
  }

  // --- wave results ---------------------------------------------------------------
  // Sums of l and p * b over the lanes holding each head: heads 0-3 in score
  // rows 0 and 2, 4-7 in rows 1 and 3 (kGp 8), all four rows for kGp 4.
  f32x4 lA, lB, pA0, pA1, pB0, pB1;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float ls = row16_sum(l[i]);
    const float p0s = row16_sum(pb[i][0]);
    const float p1s = row16_sum(pb[i][kGroups - 1]);
    auto rows = [](float v, int r0, int r1) { return lane_value(v, 16 * r0) + lane_value(v, 16 * r1); };
    if constexpr (kGp == 4) {
      lA[i] = rows(ls, 0, 2) + rows(ls, 1, 3);
      pA0[i] = rows(p0s, 0, 2) + rows(p0s, 1, 3);
      pA1[i] = rows(p1s, 0, 2) + rows(p1s, 1, 3);
      lB[i] = lA[i];
      pB0[i] = pA0[i];
      pB1[i] = pA1[i];
    } else {
      lA[i] = rows(ls, 0, 2);
      lB[i] = rows(ls, 1, 3);
      pA0[i] = rows(p0s, 0, 2);
      pB0[i] = rows(p0s, 1, 3);
      pA1[i] = rows(p1s, 0, 2);
      pB1[i] = rows(p1s, 1, 3);
    }
  }
  const float inv0 = exp2_int(24 - E0), inv1 = exp2_int(24 - E1);
  // The hi and lo parts of x land in different D rows (the lo rows one
  // 16-lane row up at DH 128, 32 lanes up at DH 64): each part goes to LDS
  // as it is (wo, wol) and the merge below adds them, with no lane exchange.
  const bool is_lo = DH == 128 ? (q4 & 1) != 0 : q4 >= 2;
#pragma unroll
  for (int st = 0; st < kSets; ++st)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      int h, d0;
      bool keep;
      float ig, pbv;
      if constexpr (DH == 128) {
        // rows 0/1 (group 0, dims 0-63) and 2/3 (group 1, dims 64-127)
        const int g = q4 >> 1;
        h = 4 * st + i;
        keep = (n16 >> 3) == g && h < G;
        const int hc = min(i, (st == 0 ? G : G - 4) - 1);
        ig = g ? inv1 : inv0;
        pbv = st == 0 ? (g ? pA1[hc] : pA0[hc]) : (g ? pB1[hc] : pB0[hc]);
        d0 = 8 * n16;
      } else {
        h = 4 * (q4 & 1) + i;
        keep = h < G;
        ig = inv0;
        if constexpr (G > 4)
          pbv = (q4 & 1) ? pB0[i] : pA0[i];
        else
          pbv = pA0[min(i, G - 1)];
        d0 = value_dim<BITS, DH>(n16, 0);
      }
      pbv = is_lo ? 0.0f : pbv;  // p * b enters once, with the hi part
      float* dst = is_lo ? &wol[wave][h][d0] : &wo[wave][h][d0];
      if (keep) {
#pragma unroll
        for (int v4 = 0; v4 < S::kNB / 4; ++v4) {
          const f32x4 o = {acc[st][4 * v4][i], acc[st][4 * v4 + 1][i], acc[st][4 * v4 + 2][i],
                           acc[st][4 * v4 + 3][i]};
          *reinterpret_cast<f32x4*>(dst + 4 * v4) =
              f32x4{fmaf(o[0], ig, pbv), fmaf(o[1], ig, pbv), fmaf(o[2], ig, pbv),
                    fmaf(o[3], ig, pbv)};
        }
      }
    }
  if (lane == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      wm[wave][h] = lane_value(mrow[h & 3], 16 * (h / 4));
      wl[wave][h] = wave < nsteps ? (h < 4 ? lA[h & 3] : lB[h & 3]) : 0.0f;
    }
  }
  __syncthreads();
  // --- merge the four waves (log-sum-exp, base 2) and write the slice partial ----
  for (int idx = threadIdx.x; idx < G * DH; idx += kBlock) {
    const int g = idx / DH, dd = idx - g * DH;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, wm[w][g]);
    float L = 0.0f, O = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float e = wl[w][g] > 0.0f ? exp2f(wm[w][g] - M) : 0.0f;  // idle waves hold -inf
      L = fmaf(wl[w][g], e, L);
      O = fmaf(wo[w][g][dd] + wol[w][g][dd], e, O);
    }
    float* pp = a.part + (((size_t)b * a.n_heads + h0 + g) * (a.n_chunks + 1) + c) * partial_floats(DH);
    pp[2 + dd] = O;
    if (dd == 0) {
      pp[0] = M;
      pp[1] = L;
    }
  }
}

bool use_mfma(int bits, int G) { return (bits == 4 || bits == 8) && G <= 8; }

int pick_chunk(int bits, int batch, int n_kv_heads, int t_stride, int G) {
  // Whole 64-position steps, at most the kernel's own bound. The matrix-core
  // kernel walks its slice step by step with four waves that each pay a
  // fixed set-up and merge: about one block per CU (256 over the longest
  // sequence) measured best. The register-prefetched kernel holds its whole
  // chunk (128 positions at most): about 1024 blocks.
  // Several sequences of mixed lengths leave many slices empty (the host
  // sizes by t_stride, not by the lengths on the device), so they take
  // longer slices (measured, 8 sequences of 1k-32k: 4096 beats 2048 by 10%,
  // 512 by 25%).
  const bool mfma = use_mfma(bits, G);
  const int cap = mfma ? (batch > 1 ? 4096 : 1024) : 128;
  const long target = (long)batch * n_kv_heads * t_stride / (mfma ? 256 : 1024);
  int chunk = 64;
  while (chunk < cap && chunk < target) chunk *= 2;
  return chunk;
}

template <int BITS, int DH, int G>
int launch_dh_g(const KvArgs& a, int batch, hipStream_t st) {
  {  // also for an empty cache: chunk 0 writes the new entry
    const dim3 grid(a.n_chunks, a.n_kv_heads, batch);
    if constexpr ((BITS == 4 || BITS == 8) && G <= 8) {
      hipLaunchKernelGGL((kv_mfma_split_kernel<BITS, DH, G>), grid, dim3(kBlock), 0, st, a);
    } else {
      const size_t lds = (size_t)G * a.chunk * sizeof(float);
      hipLaunchKernelGGL((kv_split_kernel<BITS, DH, G>), grid, dim3(kBlock), lds, st, a);
    }
    const int rc = check_launch("kvp_kv_decode (split)");
    if (rc != KVP_OK) return rc;
  }
  const dim3 cgrid(batch * a.n_heads, DH / kCombDims);
  if (a.out_f32)
    hipLaunchKernelGGL((kv_combine_kernel<DH, float>), cgrid, dim3(kBlock), 0, st, a);
  else
    hipLaunchKernelGGL((kv_combine_kernel<DH, f16>), cgrid, dim3(kBlock), 0, st, a);
  return check_launch("kvp_kv_decode (combine)");
}

template <int BITS, int DH>
int launch_dh(int G, const KvArgs& a, int batch, hipStream_t st) {
  switch (G) {
    case 1: return launch_dh_g<BITS, DH, 1>(a, batch, st);
    case 2: return launch_dh_g<BITS, DH, 2>(a, batch, st);
    case 4: return launch_dh_g<BITS, DH, 4>(a, batch, st);
    case 8: return launch_dh_g<BITS, DH, 8>(a, batch, st);
  }
  return set_error(KVP_UNSUPPORTED, "kvp_kv_decode: GQA ratio %d not in {1,2,4,8}", G);
}

template <int BITS>
int launch_bits(int dh, int G, const KvArgs& a, int batch, hipStream_t st) {
  if (!use_mfma(BITS, G) && a.chunk > max_chunk<BITS>())
    return set_error(KVP_INVALID, "kvp_kv_decode: chunk=%d above %d at %d bits", a.chunk,
                     max_chunk<BITS>(), BITS);
  if (dh == 64) return launch_dh<BITS, 64>(G, a, batch, st);
  return launch_dh<BITS, 128>(G, a, batch, st);
}

// ---------------------------------------------------------------------------
// Scratch of the allocation-free entry point (kvp_kv_decode_static): the
// split partials of one call live in this fixed device array instead of a
// caller workspace. Every GPU the library runs on holds its own copy until
// the process ends. In host code `scratch` names a host-side stand-in, never
// device memory: the device address comes from hipGetSymbolAddress, taken
// once per device with that device current, and only that address is passed
// to kernels. Nothing in it must start at zero (every partial a call reads
// is written by the same call), and calls that overlap on one GPU race.
// ---------------------------------------------------------------------------
constexpr size_t kStaticScratchBytes = size_t(4) << 20;
constexpr int kMaxDevices = 64;
__device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's address of `scratch`, looked up on first use.
int static_scratch(void** ptr) {
  int dev = -1;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess)
    return set_error(KVP_NO_DEVICE, "kvp_kv_decode_static: hipGetDevice: %s",
                     hipGetErrorString(err));
  if (dev < 0 || dev >= kMaxDevices)
    return set_error(KVP_UNSUPPORTED, "kvp_kv_decode_static: device %d beyond %d", dev,
                     kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err != hipSuccess || !p)
      return set_error(KVP_LAUNCH_ERROR, "kvp_kv_decode_static: hipGetSymbolAddress: %s",
                       hipGetErrorString(err));
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return KVP_OK;
}

}  // namespace
}  // namespace kvp

extern "C" size_t kvp_kv_decode_workspace_bytes(int batch, int n_heads, int head_dim,
                                                int t_stride, int chunk) {
  if (batch < 1 || n_heads < 1 || head_dim < 1 || t_stride < 0) return 0;
  if (chunk <= 0) chunk = 64;  // the smallest chunk the library picks
  const size_t n_chunks = t_stride > 0 ? (t_stride + chunk - 1) / chunk : 1;
  return (size_t)batch * n_heads * (n_chunks + 1) * kvp::partial_floats(head_dim) * sizeof(float);
}

extern "C" int kvp_kv_decode(const void* q, const uint32_t* k_wq, const void* k_scales,
                             const void* k_biases, const uint32_t* v_wq, const void* v_scales,
                             const void* v_biases, const void* new_k, const void* new_v,
                             const int32_t* t_cached, void* out, int out_dtype, int batch,
                             int n_heads, int n_kv_heads, int head_dim, int t_stride, int bits,
                             int cache_per_sequence, int chunk, void* workspace,
                             size_t workspace_bytes, void* stream) {
  using namespace kvp;
  clear_error();
  KVP_REQUIRE(q && new_k && new_v && t_cached && out, "kvp_kv_decode: null pointer argument");
  KVP_REQUIRE(batch >= 1 && n_heads >= 1 && n_kv_heads >= 1,
              "kvp_kv_decode: batch=%d n_heads=%d n_kv_heads=%d", batch, n_heads, n_kv_heads);
  KVP_REQUIRE(n_heads % n_kv_heads == 0, "kvp_kv_decode: n_heads %d not a multiple of %d",
              n_heads, n_kv_heads);
  KVP_REQUIRE(head_dim == 64 || head_dim == 128, "kvp_kv_decode: head_dim=%d not in {64,128}",
              head_dim);
  KVP_REQUIRE(out_dtype == KVP_F16 || out_dtype == KVP_F32, "kvp_kv_decode: out_dtype=%d",
              out_dtype);
  KVP_REQUIRE(t_stride >= 0, "kvp_kv_decode: t_stride=%d", t_stride);
  if (bits != 2 && bits != 3 && bits != 4 && bits != 8)
    return set_error(KVP_UNSUPPORTED, "kvp_kv_decode: bits=%d not in {2,3,4,8}", bits);
  const int G = n_heads / n_kv_heads;
  if (G != 1 && G != 2 && G != 4 && G != 8)
    return set_error(KVP_UNSUPPORTED, "kvp_kv_decode: GQA ratio %d not in {1,2,4,8}", G);
  if (chunk <= 0) chunk = pick_chunk(bits, batch, n_kv_heads, t_stride, G);
  KVP_REQUIRE(chunk % 64 == 0 && chunk >= 64, "kvp_kv_decode: chunk=%d (a multiple of 64)",
              chunk);
  const int n_chunks = t_stride > 0 ? (t_stride + chunk - 1) / chunk : 1;
  const size_t need = kvp_kv_decode_workspace_bytes(batch, n_heads, head_dim, t_stride, chunk);
  KVP_REQUIRE(workspace && workspace_bytes >= need,
              "kvp_kv_decode: workspace of %zu bytes, %zu needed", workspace_bytes, need);
  if (t_stride > 0)
    KVP_REQUIRE(k_wq && k_scales && k_biases && v_wq && v_scales && v_biases,
                "kvp_kv_decode: null cache pointer");

  KvArgs a;
  a.q = static_cast<const f16*>(q);
  a.k_wq = k_wq;
  a.k_s = static_cast<const uint16_t*>(k_scales);
  a.k_b = static_cast<const uint16_t*>(k_biases);
  a.v_wq = v_wq;
  a.v_s = static_cast<const uint16_t*>(v_scales);
  a.v_b = static_cast<const uint16_t*>(v_biases);
  a.new_k = static_cast<const f16*>(new_k);
  a.new_v = static_cast<const f16*>(new_v);
  a.t_cached = t_cached;
  a.part = static_cast<float*>(workspace);
  a.out = out;
  a.out_f32 = out_dtype == KVP_F32;
  a.n_heads = n_heads;
  a.n_kv_heads = n_kv_heads;
  a.t_stride = t_stride;
  a.chunk = chunk;
  a.n_chunks = n_chunks;
  a.per_seq = cache_per_sequence ? 1 : 0;
  // Base-2 softmax: scores carry log2(e) / sqrt(DH), rounded once.
  a.scale = (float)(1.4426950408889634 / sqrt((double)head_dim));
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (bits) {
    case 2: return launch_bits<2>(head_dim, G, a, batch, st);
    case 3: return launch_bits<3>(head_dim, G, a, batch, st);
    case 4: return launch_bits<4>(head_dim, G, a, batch, st);
    default: return launch_bits<8>(head_dim, G, a, batch, st);
  }
}

extern "C" size_t kvp_kv_decode_static_scratch_bytes(void) { return kvp::kStaticScratchBytes; }

extern "C" int kvp_kv_decode_static(const void* q, const uint32_t* k_wq, const void* k_scales,
                                    const void* k_biases, const uint32_t* v_wq,
                                    const void* v_scales, const void* v_biases,
                                    const void* new_k, const void* new_v,
                                    const int32_t* t_cached, void* out, int out_dtype,
                                    int batch, int n_heads, int n_kv_heads, int head_dim,
                                    int t_stride, int bits, int cache_per_sequence, int chunk,
                                    void* stream) {
  using namespace kvp;
  clear_error();
  // The chunk decides the scratch size, so resolve it first (the checks it
  // needs); kvp_kv_decode checks every argument again.
  KVP_REQUIRE(batch >= 1 && n_heads >= 1 && n_kv_heads >= 1 && n_heads % n_kv_heads == 0,
              "kvp_kv_decode_static: batch=%d n_heads=%d n_kv_heads=%d", batch, n_heads,
              n_kv_heads);
  KVP_REQUIRE(t_stride >= 0, "kvp_kv_decode_static: t_stride=%d", t_stride);
  if (chunk <= 0) chunk = pick_chunk(bits, batch, n_kv_heads, t_stride, n_heads / n_kv_heads);
  KVP_REQUIRE(chunk % 64 == 0 && chunk >= 64, "kvp_kv_decode_static: chunk=%d (a multiple of 64)",
              chunk);
  const size_t need = kvp_kv_decode_workspace_bytes(batch, n_heads, head_dim, t_stride, chunk);
  KVP_REQUIRE(need <= kStaticScratchBytes,
              "kvp_kv_decode_static: this call needs %zu bytes of scratch; the static scratch "
              "holds %zu (fewer sequences or heads, or a longer chunk)",
              need, kStaticScratchBytes);
  void* ws = nullptr;
  const int rc = static_scratch(&ws);
  if (rc != KVP_OK) return rc;
  return kvp_kv_decode(q, k_wq, k_scales, k_biases, v_wq, v_scales, v_biases, new_k, new_v,
                       t_cached, out, out_dtype, batch, n_heads, n_kv_heads, head_dim, t_stride,
                       bits, cache_per_sequence, chunk, ws, kStaticScratchBytes, stream);
}
