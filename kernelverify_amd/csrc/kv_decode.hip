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
// every intermediate fp32, exp via the accurate expf.
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
  float* part;           // [B][H][n_chunks][2 + DH] per-chunk (m, l, o)
  void* out;
  int out_f32;
  int n_heads, n_kv_heads, t_stride, chunk, n_chunks, per_seq;
  float scale;
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

// Merge of the chunk partials of one query head and the new entry:
// M = max(m_c, s_new), L = sum l_c e^(m_c-M) + e^(s_new-M),
// out = (sum o_c e^(m_c-M) + e^(s_new-M) new_v) / L.
// One block per (sequence, head, 16-dim slice): the 256 threads are 16
// chunk groups x 16 dims, so every partial a block needs is requested at
// once (coalesced 16-float rows) and the merge costs about one memory
// latency whatever the chunk count.
constexpr int kCombDims = 16;
constexpr int kCombGroups = kBlock / kCombDims;

template <int DH, typename OutT>
__global__ __launch_bounds__(kBlock) void kv_combine_kernel(KvArgs a) {
  const int z = blockIdx.x;  // b * H + h
  const int b = z / a.n_heads, h = z - b * a.n_heads;
  const int hk = h / (a.n_heads / a.n_kv_heads);
  const int d0 = blockIdx.y * kCombDims;
  const int T = min(max(a.t_cached[b], 0), a.t_stride);  // as the split kernel clamps it
  const int nc = (T + a.chunk - 1) / a.chunk;
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  __shared__ float red[kWaves];
  __shared__ float s_new_sh, M_sh;
  __shared__ float osum[kCombGroups][kCombDims];
  __shared__ float lsum[kCombGroups];

  const float* pz = a.part + (size_t)z * a.n_chunks * partial_floats(DH);
  if (wave == 0) {  // the new entry at full precision: s_new = q . new_k / sqrt(DH)
    const f16* qh = a.q + (size_t)z * DH;
    const f16* nk = a.new_k + ((size_t)b * a.n_kv_heads + hk) * DH;
    float s = 0.0f;
    for (int d = lane; d < DH; d += kWave) s = fmaf((float)qh[d], (float)nk[d], s);
    s = wave_sum(s) * a.scale;
    if (lane == 0) s_new_sh = s;
  }
  float m = -INFINITY;
  for (int c = threadIdx.x; c < nc; c += kBlock) m = fmaxf(m, pz[c * partial_floats(DH)]);
  m = wave_max(m);
  if (lane == 0) red[wave] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    float M = s_new_sh;
    for (int i = 0; i < kWaves; ++i) M = fmaxf(M, red[i]);
    M_sh = M;
  }
  __syncthreads();
  const float M = M_sh;
  const int dd = threadIdx.x % kCombDims, grp = threadIdx.x / kCombDims;
  float o = 0.0f, l = 0.0f;
#pragma unroll 8
  for (int c = grp; c < nc; c += kCombGroups) {
    const float* pc = pz + c * partial_floats(DH);
    const float e = expf(pc[0] - M);
    o = fmaf(pc[2 + d0 + dd], e, o);
    l = fmaf(pc[1], e, l);
  }
  osum[grp][dd] = o;
  if (dd == 0) lsum[grp] = l;
  __syncthreads();
  if (threadIdx.x < kCombDims) {
    const float e_new = expf(s_new_sh - M);
    const f16* nv = a.new_v + ((size_t)b * a.n_kv_heads + hk) * DH;
    float v = e_new * (float)nv[d0 + dd];
    float L = e_new;
    for (int i = 0; i < kCombGroups; ++i) {
      v += osum[i][dd];
      L += lsum[i];
    }
    store_out<OutT>(static_cast<OutT*>(a.out) + (size_t)z * DH + d0 + dd, v / L);
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
        const float e = expf(sc[g * a.chunk + t] - m);
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
      float* pp = a.part + (((size_t)b * a.n_heads + h0 + g) * a.n_chunks + c) * partial_floats(DH);
      pp[2 + dd] = v;
      if (dd == 0) {
        pp[0] = stat_m[g];
        pp[1] = stat_l[g];
      }
    }
  }

}

int pick_chunk(int bits, int batch, int n_kv_heads, int t_stride) {
  // About 1024 blocks over the longest sequence, whole 64-position steps,
  // at most the kernel's register-bounded chunk.
  const int cap = bits > 0 ? 128 : 128;
  long target = (long)batch * n_kv_heads * t_stride / 1024;
  int chunk = 64;
  while (chunk < cap && chunk < target) chunk *= 2;
  return chunk;
}

template <int BITS, int DH, int G>
int launch_dh_g(const KvArgs& a, int batch, hipStream_t st) {
  if (a.t_stride > 0) {
    const dim3 grid(a.n_chunks, a.n_kv_heads, batch);
    const size_t lds = (size_t)G * a.chunk * sizeof(float);
    hipLaunchKernelGGL((kv_split_kernel<BITS, DH, G>), grid, dim3(kBlock), lds, st, a);
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
  if (a.chunk > max_chunk<BITS>())
    return set_error(KVP_INVALID, "kvp_kv_decode: chunk=%d above %d at %d bits", a.chunk,
                     max_chunk<BITS>(), BITS);
  if (dh == 64) return launch_dh<BITS, 64>(G, a, batch, st);
  return launch_dh<BITS, 128>(G, a, batch, st);
}

}  // namespace
}  // namespace kvp

extern "C" size_t kvp_kv_decode_workspace_bytes(int batch, int n_heads, int head_dim,
                                                int t_stride, int chunk) {
  if (batch < 1 || n_heads < 1 || head_dim < 1 || t_stride < 0) return 0;
  if (chunk <= 0) chunk = 64;  // the smallest chunk the library picks
  const size_t n_chunks = t_stride > 0 ? (t_stride + chunk - 1) / chunk : 1;
  return (size_t)batch * n_heads * n_chunks * kvp::partial_floats(head_dim) * sizeof(float);
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
  if (chunk <= 0) chunk = pick_chunk(bits, batch, n_kv_heads, t_stride);
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
  a.scale = 1.0f / sqrtf((float)head_dim);
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (bits) {
    case 2: return launch_bits<2>(head_dim, G, a, batch, st);
    case 3: return launch_bits<3>(head_dim, G, a, batch, st);
    case 4: return launch_bits<4>(head_dim, G, a, batch, st);
    default: return launch_bits<8>(head_dim, G, a, batch, st);
  }
}
