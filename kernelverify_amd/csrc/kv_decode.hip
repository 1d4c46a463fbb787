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
//                     It serves all G = H/HKV query heads of that KV head, so
//                     each cache byte is read from HBM once (the reference
//                     re-reads the cache per query head, :286-289). For its
//                     chunk it writes per-head partials (m, l, o[DH]): the
//                     running max, sum of exp(s - m) and sum of
//                     exp(s - m) * v.
//   kv_combine_kernel one wave per (sequence, query head): merges the chunk
//                     partials and the new entry with the log-sum-exp rule
//                     M = max(m_c, s_new), L = sum l_c e^(m_c-M) + e^(s_new-M),
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

struct KvArgs {
  const f16* q;
  const uint32_t* k_wq;
  const uint16_t* k_s;
  const uint16_t* k_b;
  const uint32_t* v_wq;
  const uint16_t* v_s;
  const uint16_t* v_b;
  const int32_t* t_cached;
  float* part;  // [B][H][n_chunks][2 + DH]
  int n_heads, n_kv_heads, t_stride, chunk, n_chunks, per_seq;
  float scale;
};

// Reads the 8-code block j of a row (codes 8j .. 8j+7) as a 32-bit field
// (low 8*BITS bits), from a row of `row_words` words.
template <int BITS>
__device__ __forceinline__ uint32_t load_block8(const uint32_t* __restrict__ row, int j) {
  if constexpr (BITS == 8) {
    return 0;  // 8-bit blocks span two words and are read as a u32x2 pair
  } else {
    const int bit = j * 8 * BITS;
    const int w = bit >> 5, sh = bit & 31;
    if (sh + 8 * BITS <= 32) return row[w] >> sh;
    return __builtin_amdgcn_alignbit(row[w + 1], row[w], sh);
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

  const int c = blockIdx.x, hk = blockIdx.y, b = blockIdx.z;
  // Lengths outside [0, t_stride] are clamped: the cache is never read past
  // its allocation whatever the caller passes.
  const int T = min(max(a.t_cached[b], 0), a.t_stride);
  const int t0 = c * a.chunk;
  if (t0 >= T) return;  // chunk past this sequence: no partial (block-uniform)
  const int n = min(a.chunk, T - t0);

  __shared__ float sc[G][1024];  // scores, then probabilities (chunk <= 1024)
  __shared__ float red[kWaves][G];
  __shared__ float stat_m[G], stat_l[G];
  __shared__ float obuf[kWaves][G][DH];

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int h0 = hk * G;
  const size_t cache_base = ((size_t)(a.per_seq ? b : 0) * a.n_kv_heads + hk) * a.t_stride;

  // --- query slice of this lane's K unit, all G heads, in pair order -------
  const int part = lane % U;
  uint32_t qp[G * Gm::kUnitPairs];
  float qsum[G];
  {
    const uint32_t* qw = reinterpret_cast<const uint32_t*>(a.q + ((size_t)b * a.n_heads + h0) * DH);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      uint32_t nat[kXW];
#pragma unroll
      for (int i = 0; i < kXW; ++i) nat[i] = qw[(g * DH + part * Gm::kUnitCodes) / 2 + i];
      float s = 0.0f;
#pragma unroll
      for (int i = 0; i < kXW; ++i) s = dot2(nat[i], 0x3C003C00u, s);
      qsum[g] = s;
      if constexpr (Gm::kMagic) {
        constexpr int H = Gm::kPairsPerWord;
#pragma unroll
        for (int wi = 0; wi < Gm::kUnitWords; ++wi)
          pair_order<BITS>(&nat[wi * (Gm::kCodesPerWord / 2)], &qp[(g * Gm::kSlots + wi) * H]);
      } else {
#pragma unroll
        for (int i = 0; i < kXW; ++i) qp[g * kXW + i] = nat[i];
      }
    }
  }

  // --- scores over the chunk ------------------------------------------------
  const int grp = (part * Gm::kUnitCodes) / 64;
  for (int r0 = wave * kRowsPerPass; r0 < n; r0 += kWaves * kRowsPerPass) {
    const int tr = r0 + lane / U;
    const int t = t0 + min(tr, n - 1);
    const size_t row = cache_base + t;
    uint32_t w[1][Gm::kUnitWords];
    load_unit<BITS>(a.k_wq + row * kRowWords + part * Gm::kUnitWords, w[0]);
    const float s = f16_bits_to_f32(a.k_s[row * kGroups + grp]);
    const float bias = f16_bits_to_f32(a.k_b[row * kGroups + grp]);
    float d[1][G];
    unit_dot<BITS, G, 1>(w, qp, Gm::kSlotPairs, d);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float v = fmaf(s, d[0][g], bias * qsum[g]);
#pragma unroll
      for (int off = 1; off < U; off <<= 1) v += __shfl_xor(v, off, U);
      if (part == 0 && tr < n) sc[g][tr] = v * a.scale;
    }
  }
  __syncthreads();

  // --- chunk softmax statistics per head ------------------------------------
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float m = -INFINITY;
    for (int t = threadIdx.x; t < n; t += kBlock) m = fmaxf(m, sc[g][t]);
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
      const float e = expf(sc[g][t] - m);
      sc[g][t] = e;
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

  // --- values: o[g][d] = sum_t p[g][t] * (s_t * q_td + b_t) ------------------
  const int j = lane % kBlocks8;  // 8-code block: dims 8j .. 8j+7
  const int vgrp = (8 * j) / 64;
  float acc[G][8];
  float pb[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    pb[g] = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[g][i] = 0.0f;
  }
  for (int r0 = wave * kVRowsPerPass; r0 < n; r0 += kWaves * kVRowsPerPass) {
    const int tr = r0 + lane / kBlocks8;
    const bool valid = tr < n;
    const size_t row = cache_base + t0 + min(tr, n - 1);
    const uint32_t* vrow = a.v_wq + row * kRowWords;
    float codes[8];
    if constexpr (BITS == 8) {
      const u32x2 v = *reinterpret_cast<const u32x2*>(vrow + 2 * j);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        codes[i] = (float)((v.x >> (8 * i)) & 0xFFu);
        codes[4 + i] = (float)((v.y >> (8 * i)) & 0xFFu);
      }
    } else {
      const uint32_t f = load_block8<BITS>(vrow, j);
#pragma unroll
      for (int i = 0; i < 8; ++i) codes[i] = (float)((f >> (BITS * i)) & ((1u << BITS) - 1u));
    }
    const float s = f16_bits_to_f32(a.v_s[row * kGroups + vgrp]);
    const float bias = f16_bits_to_f32(a.v_b[row * kGroups + vgrp]);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float p = valid ? sc[g][min(tr, n - 1)] : 0.0f;
      const float ps = p * s;
      pb[g] = fmaf(p, bias, pb[g]);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[g][i] = fmaf(ps, codes[i], acc[g][i]);
    }
  }
  // Lanes with the same block j hold disjoint positions: add them up.
#pragma unroll
  for (int g = 0; g < G; ++g) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float v = acc[g][i] + pb[g];
#pragma unroll
      for (int off = kBlocks8; off < kWave; off <<= 1) v += __shfl_xor(v, off, kWave);
      acc[g][i] = v;
    }
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
    float* p = a.part + (((size_t)b * a.n_heads + h0 + g) * a.n_chunks + c) * partial_floats(DH);
    p[2 + dd] = v;
    if (dd == 0) {
      p[0] = stat_m[g];
      p[1] = stat_l[g];
    }
  }
}

template <int DH, typename OutT>
__global__ __launch_bounds__(kBlock) void kv_combine_kernel(const f16* __restrict__ q,
                                                            const f16* __restrict__ new_k,
                                                            const f16* __restrict__ new_v,
                                                            const int32_t* __restrict__ t_cached,
                                                            const float* __restrict__ part,
                                                            OutT* __restrict__ out, int batch,
                                                            int n_heads, int n_kv_heads,
                                                            int t_stride, int chunk, int n_chunks,
                                                            float scale) {
  constexpr int L = DH / kWave;  // dims per lane
  const int lane = threadIdx.x & (kWave - 1);
  const int z = blockIdx.x * kWaves + threadIdx.x / kWave;  // b * H + h
  if (z >= batch * n_heads) return;
  const int b = z / n_heads, h = z - b * n_heads;
  const int hk = h / (n_heads / n_kv_heads);
  const int T = min(max(t_cached[b], 0), t_stride);  // as the split kernel clamps it
  const int nc = (T + chunk - 1) / chunk;

  // The new entry at full precision: s_new = q . new_k / sqrt(DH).
  const f16* qh = q + (size_t)z * DH;
  const f16* nk = new_k + ((size_t)b * n_kv_heads + hk) * DH;
  const f16* nv = new_v + ((size_t)b * n_kv_heads + hk) * DH;
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < L; ++i) s = fmaf((float)qh[lane * L + i], (float)nk[lane * L + i], s);
  const float s_new = wave_sum(s) * scale;

  const float* pz = part + (size_t)z * n_chunks * partial_floats(DH);
  float M = s_new;
  for (int c = 0; c < nc; ++c) M = fmaxf(M, pz[c * partial_floats(DH)]);
  const float e_new = expf(s_new - M);
  float l_tot = e_new;
  float o[L];
#pragma unroll
  for (int i = 0; i < L; ++i) o[i] = e_new * (float)nv[lane * L + i];
  for (int c = 0; c < nc; ++c) {
    const float* pc = pz + c * partial_floats(DH);
    const float e = expf(pc[0] - M);
    l_tot = fmaf(pc[1], e, l_tot);
#pragma unroll
    for (int i = 0; i < L; ++i) o[i] = fmaf(pc[2 + lane * L + i], e, o[i]);
  }
#pragma unroll
  for (int i = 0; i < L; ++i) store_out<OutT>(out + (size_t)z * DH + lane * L + i, o[i] / l_tot);
}

int pick_chunk(int batch, int n_kv_heads, int t_stride) {
  // About 2048 blocks over the longest sequence; whole 64-position steps,
  // at most 1024 positions (the score buffer).
  long target = (long)batch * n_kv_heads * t_stride / 2048;
  int chunk = 64;
  while (chunk < 1024 && chunk < target) chunk *= 2;
  return chunk;
}

template <int BITS, int DH>
int launch_split_dh(int G, const KvArgs& a, int batch, hipStream_t st) {
  const dim3 grid(a.n_chunks, a.n_kv_heads, batch);
  switch (G) {
#define KVP_G(N)                                                                          \
  case N:                                                                                 \
    hipLaunchKernelGGL((kv_split_kernel<BITS, DH, N>), grid, dim3(kBlock), 0, st, a);     \
    return check_launch("kvp_kv_decode (split)");
    KVP_G(1) KVP_G(2) KVP_G(4) KVP_G(8)
#undef KVP_G
  }
  return set_error(KVP_UNSUPPORTED, "kvp_kv_decode: GQA ratio %d not in {1,2,4,8}", G);
}

template <int BITS>
int launch_split(int dh, int G, const KvArgs& a, int batch, hipStream_t st) {
  if (dh == 64) return launch_split_dh<BITS, 64>(G, a, batch, st);
  return launch_split_dh<BITS, 128>(G, a, batch, st);
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
  if (chunk <= 0) chunk = pick_chunk(batch, n_kv_heads, t_stride);
  KVP_REQUIRE(chunk % 64 == 0 && chunk <= 1024, "kvp_kv_decode: chunk=%d (multiple of 64, <= 1024)",
              chunk);
  const int n_chunks = t_stride > 0 ? (t_stride + chunk - 1) / chunk : 1;
  const size_t need = kvp_kv_decode_workspace_bytes(batch, n_heads, head_dim, t_stride, chunk);
  KVP_REQUIRE(workspace && workspace_bytes >= need,
              "kvp_kv_decode: workspace of %zu bytes, %zu needed", workspace_bytes, need);
  if (t_stride > 0)
    KVP_REQUIRE(k_wq && k_scales && k_biases && v_wq && v_scales && v_biases,
                "kvp_kv_decode: null cache pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const float scale = 1.0f / sqrtf((float)head_dim);

  KvArgs a;
  a.q = static_cast<const f16*>(q);
  a.k_wq = k_wq;
  a.k_s = static_cast<const uint16_t*>(k_scales);
  a.k_b = static_cast<const uint16_t*>(k_biases);
  a.v_wq = v_wq;
  a.v_s = static_cast<const uint16_t*>(v_scales);
  a.v_b = static_cast<const uint16_t*>(v_biases);
  a.t_cached = t_cached;
  a.part = static_cast<float*>(workspace);
  a.n_heads = n_heads;
  a.n_kv_heads = n_kv_heads;
  a.t_stride = t_stride;
  a.chunk = chunk;
  a.n_chunks = n_chunks;
  a.per_seq = cache_per_sequence ? 1 : 0;
  a.scale = scale;
  if (t_stride > 0) {
    int rc = KVP_OK;
    switch (bits) {
      case 2: rc = launch_split<2>(head_dim, G, a, batch, st); break;
      case 3: rc = launch_split<3>(head_dim, G, a, batch, st); break;
      case 4: rc = launch_split<4>(head_dim, G, a, batch, st); break;
      case 8: rc = launch_split<8>(head_dim, G, a, batch, st); break;
    }
    if (rc != KVP_OK) return rc;
  }
  const int blocks = (batch * n_heads + kWaves - 1) / kWaves;
  const f16* qq = static_cast<const f16*>(q);
  const f16* nk = static_cast<const f16*>(new_k);
  const f16* nv = static_cast<const f16*>(new_v);
  const float* part = static_cast<const float*>(workspace);
  if (head_dim == 64) {
    if (out_dtype == KVP_F16)
      hipLaunchKernelGGL((kv_combine_kernel<64, f16>), dim3(blocks), dim3(kBlock), 0, st, qq, nk,
                         nv, t_cached, part, static_cast<f16*>(out), batch, n_heads, n_kv_heads,
                         t_stride, chunk, n_chunks, scale);
    else
      hipLaunchKernelGGL((kv_combine_kernel<64, float>), dim3(blocks), dim3(kBlock), 0, st, qq,
                         nk, nv, t_cached, part, static_cast<float*>(out), batch, n_heads,
                         n_kv_heads, t_stride, chunk, n_chunks, scale);
  } else {
    if (out_dtype == KVP_F16)
      hipLaunchKernelGGL((kv_combine_kernel<128, f16>), dim3(blocks), dim3(kBlock), 0, st, qq,
                         nk, nv, t_cached, part, static_cast<f16*>(out), batch, n_heads,
                         n_kv_heads, t_stride, chunk, n_chunks, scale);
    else
      hipLaunchKernelGGL((kv_combine_kernel<128, float>), dim3(blocks), dim3(kBlock), 0, st, qq,
                         nk, nv, t_cached, part, static_cast<float*>(out), batch, n_heads,
                         n_kv_heads, t_stride, chunk, n_chunks, scale);
  }
  return check_launch("kvp_kv_decode (combine)");
}
