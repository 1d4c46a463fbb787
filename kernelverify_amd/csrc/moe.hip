// MoE decode for gfx950: routing, token permutation, expert gather-qmv,
// weighted scatter-add.
//
// Replaces the reference's `kv_moe_routing` and `kv_moe_dispatch`
// (kernelverify/pack/moe_dispatch.py:39-138), generalised from top-2 to
// top-k, and adds the SwiGLU expert MLP of BASELINE config 5.
//
//   route        one wave per token: fp32 logits (given, or x . router as
//                the reference, :47-54), max-subtracted fp32 softmax over all
//                experts, top-k BY PROBABILITY with ties to the lower index
//                (the reference's strict `>` scan, :60-78), renormalised.
//   permute      one block: stable counting sort of the n*k (token, slot)
//                pairs by expert, plus the list of routed ("active")
//                experts and each pair's position (inverse permutation).
//   expert gemv  one block per (active expert, rows): the expert's weight
//                rows stream from HBM once for all of that expert's tokens
//                (the reference reads each expert once per token, :101-129).
//                fp16 activations use the qmv core (codes as exact fp16
//                denormals through V_DOT2_F32_F16); the SwiGLU down
//                projection takes its fp32 hidden state through fp32 FMAs.
//   scatter      out[t] = sum_s gate[t, s] * y[t, s], slots in order s = 0..k-1.
#include <math.h>

#include "common.h"
#include "qmv_core.h"

namespace kvp {
namespace {

constexpr int kBlock = 256;
constexpr int kWaves = kBlock / kWave;
constexpr int kMaxExperts = 1024;
constexpr int kMaxK = 32;

// ---------------------------------------------------------------------------
// Routing
// ---------------------------------------------------------------------------
// Wave-wide argmax by (value desc, index asc): the winner every lane agrees on.
__device__ __forceinline__ void wave_argmax(float& v, int& i) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(v, off, kWave);
    const int oi = __shfl_xor(i, off, kWave);
    if (ov > v || (ov == v && oi < i)) {
      v = ov;
      i = oi;
    }
  }
}

// logits: E fp32 values of one token, held as E/64 per lane (lane-strided).
template <int EPL>
__device__ __forceinline__ void route_token(const float (&lg)[EPL], int n_experts, int k,
                                            uint32_t* __restrict__ idx, float* __restrict__ gate) {
  const int lane = threadIdx.x & (kWave - 1);
  float peak = -INFINITY;
#pragma unroll
  for (int j = 0; j < EPL; ++j)
    if (lane + j * kWave < n_experts) peak = fmaxf(peak, lg[j]);
  peak = wave_max(peak);
  float e[EPL];
  float denom = 0.0f;
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    e[j] = (lane + j * kWave < n_experts) ? expf(lg[j] - peak) : 0.0f;
    denom += e[j];
  }
  denom = wave_sum(denom);
  float p[EPL];
#pragma unroll
  for (int j = 0; j < EPL; ++j) p[j] = (lane + j * kWave < n_experts) ? e[j] / denom : -1.0f;
  // k rounds of a wave argmax; the chosen expert is knocked out (-inf).
  float chosen_p[kMaxK];
  int chosen_i[kMaxK];
  float total = 0.0f;
  for (int s = 0; s < k; ++s) {
    float bv = -INFINITY;
    int bi = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      const int ei = lane + j * kWave;
      if (p[j] > bv || (p[j] == bv && ei < bi)) {
        bv = p[j];
        bi = ei;
      }
    }
    wave_argmax(bv, bi);
#pragma unroll
    for (int j = 0; j < EPL; ++j)
      if (lane + j * kWave == bi) p[j] = -INFINITY;
    chosen_p[s] = bv;
    chosen_i[s] = bi;
  }
  // Renormalise over the k chosen, summed in slot order.
  for (int s = 0; s < k; ++s) total += chosen_p[s];
  if (lane == 0) {
    for (int s = 0; s < k; ++s) {
      idx[s] = (uint32_t)chosen_i[s];
      gate[s] = chosen_p[s] / total;
    }
  }
}

template <int EPL>
__global__ __launch_bounds__(kBlock) void route_logits_kernel(const float* __restrict__ logits,
                                                              uint32_t* __restrict__ idx,
                                                              float* __restrict__ gate, int n,
                                                              int n_experts, int k) {
  const int t = blockIdx.x * kWaves + threadIdx.x / kWave;
  if (t >= n) return;  // whole waves; no barrier
  const int lane = threadIdx.x & (kWave - 1);
  float lg[EPL];
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int e = lane + j * kWave;
    lg[j] = e < n_experts ? logits[(size_t)t * n_experts + e] : 0.0f;
  }
  route_token<EPL>(lg, n_experts, k, idx + (size_t)t * k, gate + (size_t)t * k);
}

// Routing from activations: logits = x @ router^T in fp32
// (kernelverify/reference/native_kernels.py:118-119), one block per token.
// Each wave computes a quarter of the experts' logits with its lanes split
// over d (coalesced router rows), into LDS; wave 0 then routes.
template <int EPL>
__global__ __launch_bounds__(kBlock) void route_x_kernel(const f16* __restrict__ x,
                                                         const f16* __restrict__ router,
                                                         uint32_t* __restrict__ idx,
                                                         float* __restrict__ gate, int d,
                                                         int n_experts, int k) {
  __shared__ float lg_sh[kMaxExperts];
  const int t = blockIdx.x;
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const f16* xr = x + (size_t)t * d;
  for (int e = wave; e < n_experts; e += kWaves) {
    const f16* rr = router + (size_t)e * d;
    float acc = 0.0f;
    for (int i = lane; i < d; i += kWave) acc = fmaf((float)xr[i], (float)rr[i], acc);
    acc = wave_sum(acc);
    if (lane == 0) lg_sh[e] = acc;
  }
  __syncthreads();
  if (wave != 0) return;  // after the only barrier
  float lg[EPL];
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int e = lane + j * kWave;
    lg[j] = e < n_experts ? lg_sh[e] : 0.0f;
  }
  route_token<EPL>(lg, n_experts, k, idx + (size_t)t * k, gate + (size_t)t * k);
}

// ---------------------------------------------------------------------------
// Permutation: stable counting sort of flat pairs by expert
// ---------------------------------------------------------------------------
// offsets[E + 1]; perm[n*k]: flat index token*k + slot, ascending within each
// expert; active (optional): count, then the routed experts ascending;
// slot_of (optional): each flat pair's position in perm (-1 if unplaced).
__global__ __launch_bounds__(1024) void permute_kernel(const uint32_t* __restrict__ idx,
                                                       int32_t* __restrict__ offsets,
                                                       int32_t* __restrict__ perm,
                                                       int32_t* __restrict__ active,
                                                       int32_t* __restrict__ slot_of, int pairs,
                                                       int n_experts) {
  __shared__ int32_t cnt[kMaxExperts];
  __shared__ int32_t off[kMaxExperts + 1];
  __shared__ uint32_t tile[1024];
  for (int e = threadIdx.x; e < n_experts; e += blockDim.x) cnt[e] = 0;
  // A pair naming no valid expert is never placed: its slot stays -1 and the
  // scatter skips it.
  if (slot_of)
    for (int i = threadIdx.x; i < pairs; i += blockDim.x) slot_of[i] = -1;
  __syncthreads();
  for (int i = threadIdx.x; i < pairs; i += blockDim.x) {
    const uint32_t e = idx[i];
    if (e < (uint32_t)n_experts) atomicAdd(&cnt[e], 1);  // counts are order-free
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int run = 0, act = 0;
    for (int e = 0; e < n_experts; ++e) {
      off[e] = run;
      run += cnt[e];
      if (cnt[e] > 0 && active) active[1 + act++] = e;
    }
    off[n_experts] = run;
    if (active) active[0] = act;
  }
  __syncthreads();
  for (int e = threadIdx.x; e <= n_experts; e += blockDim.x) offsets[e] = off[e];
  // Stable placement: one thread per expert walks the pairs in flat order.
  for (int e0 = 0; e0 < n_experts; e0 += blockDim.x) {
    const int e = e0 + threadIdx.x;
    int pos = e < n_experts ? off[e] : 0;
    for (int base = 0; base < pairs; base += 1024) {
      const int m = min(1024, pairs - base);
      __syncthreads();
      for (int i = threadIdx.x; i < m; i += blockDim.x) tile[i] = idx[base + i];
      __syncthreads();
      if (e < n_experts) {
        for (int i = 0; i < m; ++i) {
          if (tile[i] == (uint32_t)e) {
            perm[pos] = base + i;
            if (slot_of) slot_of[base + i] = pos;
            ++pos;
          }
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Expert GEMV over the pairs routed to one expert
// ---------------------------------------------------------------------------
struct ExpertArgs {
  const f16* x;            // [n][d_in] fp16 activations (gate/up, single linear)
  const float* xf;         // [pairs][d_in] fp32 activations in pair order (down)
  const uint32_t* wq0;     // [E][d_out][d_in*bits/32]  (gate, or the single linear)
  const uint16_t* s0;
  const uint16_t* b0;
  const uint32_t* wq1;     // up projection (SwiGLU only)
  const uint16_t* s1;
  const uint16_t* b1;
  const int32_t* offsets;  // [E+1]
  const int32_t* perm;     // [pairs]
  const int32_t* active;   // [1 + E]
  float* y;                // [pairs][d_out] fp32, pair order
  int k, d_in, d_out;
};

constexpr int kMT = 4;  // tokens per pass of an expert's rows
constexpr int kRW = 2;  // rows per wave
constexpr int kRowsPerBlock = kWaves * kRW;

__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }

// Stage the fp16 activations of up to MT tokens (gathered by token id) into
// LDS in the unit-slot pair order of qmv_core, plus per-unit sums.
template <int BITS, int MT>
__device__ void stage_tokens(const f16* __restrict__ x, const int* tok, int nt, int d_in,
                             uint32_t* xs, float* xsum) {
  using Gm = Geom<BITS>;
  const int units = d_in / Gm::kUnitCodes;
  const uint16_t* xh = reinterpret_cast<const uint16_t*>(x);
  for (int idx = threadIdx.x; idx < MT * units * Gm::kSlots; idx += kBlock) {
    const int slot = idx % Gm::kSlots;
    const int mu = idx / Gm::kSlots;
    const int m = mu / units, u = mu - m * units;
    const uint16_t* src = xh + (size_t)(m < nt ? tok[m] : tok[0]) * d_in + u * Gm::kUnitCodes;
    uint32_t* dst = xs + ((m * Gm::kSlots + slot) * units + u) * Gm::kSlotPairs;
    if constexpr (Gm::kMagic) {
      constexpr int C = Gm::kCodesPerWord, H = Gm::kPairsPerWord;
#pragma unroll
      for (int i = 0; i < H; ++i) {
        const uint32_t lo = m < nt ? src[slot * C + i] : 0u;
        const uint32_t hi = m < nt ? src[slot * C + i + H] : 0u;
        dst[i] = lo | (hi << 16);
      }
    } else {
      const uint32_t lo = m < nt ? src[2 * slot] : 0u, hi = m < nt ? src[2 * slot + 1] : 0u;
      dst[0] = lo | (hi << 16);
    }
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < MT * units; idx += kBlock) {
    const int m = idx / units, u = idx - m * units;
    float s = 0.0f;
    for (int slot = 0; slot < Gm::kSlots; ++slot)
#pragma unroll
      for (int i = 0; i < Gm::kSlotPairs; ++i)
        s = dot2(xs[((m * Gm::kSlots + slot) * units + u) * Gm::kSlotPairs + i], 0x3C003C00u, s);
    xsum[m * units + u] = s;
  }
  __syncthreads();
}

// acc[r][m] += x_m . dequant(W rows) for this wave's RW rows, over all units.
template <int BITS, int MT>
__device__ __forceinline__ void rows_dot(const uint32_t* __restrict__ wq,
                                         const uint16_t* __restrict__ sc,
                                         const uint16_t* __restrict__ bi, const int (&rows)[kRW],
                                         int d_in, const uint32_t* xs, const float* xsum,
                                         float (&acc)[kRW][MT]) {
  using Gm = Geom<BITS>;
  constexpr int kUnitsPerGroup = 64 / Gm::kUnitCodes;
  const int lane = threadIdx.x & (kWave - 1);
  const int units = d_in / Gm::kUnitCodes;
  const int row_words = units * Gm::kUnitWords;
  const int groups = d_in / 64;
  for (int u = lane; u < units; u += kWave) {
    uint32_t w[kRW][Gm::kUnitWords];
    float s[kRW], b[kRW];
#pragma unroll
    for (int r = 0; r < kRW; ++r) {
      load_unit<BITS>(wq + (size_t)rows[r] * row_words + (size_t)u * Gm::kUnitWords, w[r]);
      s[r] = f16_bits_to_f32(sc[(size_t)rows[r] * groups + u / kUnitsPerGroup]);
      b[r] = f16_bits_to_f32(bi[(size_t)rows[r] * groups + u / kUnitsPerGroup]);
    }
    float d[kRW][MT];
    unit_dot<BITS, MT, kRW>(w, xs + u * Gm::kSlotPairs, units * Gm::kSlotPairs, d);
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      const float xu = xsum[m * units + u];
#pragma unroll
      for (int r = 0; r < kRW; ++r) acc[r][m] = fmaf(s[r], d[r][m], fmaf(b[r], xu, acc[r][m]));
    }
  }
#pragma unroll
  for (int r = 0; r < kRW; ++r)
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[r][m] = wave_sum(acc[r][m]);
}

// fp16-activation experts: single linear (y = x W^T) or SwiGLU gate/up
// (y = silu(x Wg^T) * (x Wu^T)), both written to y in pair order.
template <int BITS, bool SWIGLU>
__global__ __launch_bounds__(kBlock) void expert_f16_kernel(ExpertArgs a) {
  using Gm = Geom<BITS>;
  const int act = blockIdx.y;
  if (act >= a.active[0]) return;  // block-uniform
  const int e = a.active[1 + act];
  const int p0 = a.offsets[e], p1 = a.offsets[e + 1];
  extern __shared__ __align__(16) uint32_t smem[];
  const int units = a.d_in / Gm::kUnitCodes;
  uint32_t* xs = smem;
  float* xsum = reinterpret_cast<float*>(smem + kMT * units * Gm::kUnitPairs);
  __shared__ int tok[kMT];

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int row0 = blockIdx.x * kRowsPerBlock + wave * kRW;
  int rows[kRW];
#pragma unroll
  for (int r = 0; r < kRW; ++r) rows[r] = e * a.d_out + min(row0 + r, a.d_out - 1);

  for (int g0 = p0; g0 < p1; g0 += kMT) {  // groups of MT pairs (block-uniform)
    const int nt = min(kMT, p1 - g0);
    __syncthreads();
    if (threadIdx.x < kMT) tok[threadIdx.x] = a.perm[g0 + min((int)threadIdx.x, nt - 1)] / a.k;
    __syncthreads();
    stage_tokens<BITS, kMT>(a.x, tok, nt, a.d_in, xs, xsum);
    float acc0[kRW][kMT] = {};
    rows_dot<BITS, kMT>(a.wq0, a.s0, a.b0, rows, a.d_in, xs, xsum, acc0);
    if constexpr (SWIGLU) {
      float acc1[kRW][kMT] = {};
      rows_dot<BITS, kMT>(a.wq1, a.s1, a.b1, rows, a.d_in, xs, xsum, acc1);
#pragma unroll
      for (int r = 0; r < kRW; ++r)
#pragma unroll
        for (int m = 0; m < kMT; ++m) acc0[r][m] = silu(acc0[r][m]) * acc1[r][m];
    }
    if (lane == 0) {
#pragma unroll
      for (int r = 0; r < kRW; ++r)
#pragma unroll
        for (int m = 0; m < kMT; ++m)
          if (m < nt && row0 + r < a.d_out) a.y[(size_t)(g0 + m) * a.d_out + row0 + r] = acc0[r][m];
    }
  }
}

// Codes of one unit as fp32 values, in code order.
template <int BITS>
__device__ __forceinline__ void unit_codes_f32(const uint32_t (&w)[Geom<BITS>::kUnitWords],
                                               float* c) {
  using Gm = Geom<BITS>;
  if constexpr (BITS == 8) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) c[4 * i + j] = (float)((w[i] >> (8 * j)) & 0xFFu);
  } else if constexpr (BITS == 4) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t lo = w[i] & 0x0F0F0F0Fu, hi = (w[i] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        c[8 * i + 2 * j] = (float)((lo >> (8 * j)) & 0xFFu);
        c[8 * i + 2 * j + 1] = (float)((hi >> (8 * j)) & 0xFFu);
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < Gm::kUnitCodes; ++i) {
      const int bit = i * BITS, word = bit >> 5, sh = bit & 31;
      const uint32_t f = (sh + BITS <= 32) ? (w[word] >> sh)
                                           : __builtin_amdgcn_alignbit(w[word + 1], w[word], sh);
      c[i] = (float)(f & ((1u << BITS) - 1u));
    }
  }
}

// fp32-activation experts (the SwiGLU down projection): y_pair = h_pair . W^T,
// with h in fp32 (pair order), codes converted to fp32 and fused as
// s * sum(h * q) + b * sum(h) per unit.
template <int BITS>
__global__ __launch_bounds__(kBlock) void expert_f32_kernel(ExpertArgs a) {
  using Gm = Geom<BITS>;
  constexpr int kUnitsPerGroup = 64 / Gm::kUnitCodes;
  const int act = blockIdx.y;
  if (act >= a.active[0]) return;
  const int e = a.active[1 + act];
  const int p0 = a.offsets[e], p1 = a.offsets[e + 1];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int row0 = blockIdx.x * kRowsPerBlock + wave * kRW;
  const int units = a.d_in / Gm::kUnitCodes;
  const int row_words = units * Gm::kUnitWords;
  const int groups = a.d_in / 64;
  int rows[kRW];
#pragma unroll
  for (int r = 0; r < kRW; ++r) rows[r] = e * a.d_out + min(row0 + r, a.d_out - 1);

  for (int g0 = p0; g0 < p1; g0 += kMT) {
    const int nt = min(kMT, p1 - g0);
    float acc[kRW][kMT] = {};
    for (int u = lane; u < units; u += kWave) {
      float hx[kMT][Gm::kUnitCodes];
      float hs[kMT];
#pragma unroll
      for (int m = 0; m < kMT; ++m) {
        const float* hrow = a.xf + (size_t)(g0 + min(m, nt - 1)) * a.d_in + u * Gm::kUnitCodes;
        hs[m] = 0.0f;
#pragma unroll
        for (int i = 0; i < Gm::kUnitCodes; i += 4) {
          const float4 v = *reinterpret_cast<const float4*>(hrow + i);
          hx[m][i] = v.x; hx[m][i + 1] = v.y; hx[m][i + 2] = v.z; hx[m][i + 3] = v.w;
        }
#pragma unroll
        for (int i = 0; i < Gm::kUnitCodes; ++i) hs[m] += hx[m][i];
      }
#pragma unroll
      for (int r = 0; r < kRW; ++r) {
        uint32_t w[Gm::kUnitWords];
        load_unit<BITS>(a.wq0 + (size_t)rows[r] * row_words + (size_t)u * Gm::kUnitWords, w);
        const float s = f16_bits_to_f32(a.s0[(size_t)rows[r] * groups + u / kUnitsPerGroup]);
        const float b = f16_bits_to_f32(a.b0[(size_t)rows[r] * groups + u / kUnitsPerGroup]);
        float c[Gm::kUnitCodes];
        unit_codes_f32<BITS>(w, c);
#pragma unroll
        for (int m = 0; m < kMT; ++m) {
          float d = 0.0f;
#pragma unroll
          for (int i = 0; i < Gm::kUnitCodes; ++i) d = fmaf(hx[m][i], c[i], d);
          acc[r][m] = fmaf(s, d, fmaf(b, hs[m], acc[r][m]));
        }
      }
    }
#pragma unroll
    for (int r = 0; r < kRW; ++r)
#pragma unroll
      for (int m = 0; m < kMT; ++m) {
        const float v = wave_sum(acc[r][m]);
        if (lane == 0 && m < nt && row0 + r < a.d_out)
          a.y[(size_t)(g0 + m) * a.d_out + row0 + r] = v;
      }
  }
}

// out[t][d] = sum_s gate[t][s] * y[slot_of[t*k + s]][d], s in order.
template <typename OutT>
__global__ __launch_bounds__(kBlock) void scatter_kernel(const float* __restrict__ y,
                                                         const int32_t* __restrict__ slot_of,
                                                         const float* __restrict__ gate,
                                                         OutT* __restrict__ out, int n, int k,
                                                         int d) {
  const long long i = (long long)blockIdx.x * kBlock + threadIdx.x;
  if (i >= (long long)n * d) return;
  const int t = (int)(i / d), dd = (int)(i - (long long)t * d);
  float acc = 0.0f;
  for (int s = 0; s < k; ++s) {
    const int slot = slot_of[t * k + s];
    if (slot >= 0) acc = fmaf(gate[t * k + s], y[(size_t)slot * d + dd], acc);
  }
  store_out<OutT>(out + i, acc);
}

// Single-linear dispatch, the reference's contract at any k
// (kernelverify/pack/moe_dispatch.py:84-138): one block per (token, rows);
// for each slot in order, the rows of that slot's expert against the
// token's staged activations; out = sum_s gate[t, s] * (x_t . W_e rows).
template <int BITS, typename OutT>
__global__ __launch_bounds__(kBlock) void dispatch_kernel(const f16* __restrict__ x,
                                                          const uint32_t* __restrict__ idx,
                                                          const float* __restrict__ gate,
                                                          const uint32_t* __restrict__ wq,
                                                          const uint16_t* __restrict__ sc,
                                                          const uint16_t* __restrict__ bi,
                                                          OutT* __restrict__ out, int k,
                                                          int n_experts, int d_out, int d_in) {
  using Gm = Geom<BITS>;
  extern __shared__ __align__(16) uint32_t smem[];
  const int units = d_in / Gm::kUnitCodes;
  uint32_t* xs = smem;
  float* xsum = reinterpret_cast<float*>(smem + units * Gm::kUnitPairs);
  const int t = blockIdx.y;
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int row0 = blockIdx.x * kRowsPerBlock + wave * kRW;
  const int tok[1] = {t};
  stage_tokens<BITS, 1>(x, tok, 1, d_in, xs, xsum);
  float total[kRW] = {};
  for (int s = 0; s < k; ++s) {
    const uint32_t e = min(idx[(size_t)t * k + s], (uint32_t)(n_experts - 1));
    const float g = gate[(size_t)t * k + s];
    int rows[kRW];
#pragma unroll
    for (int r = 0; r < kRW; ++r) rows[r] = e * d_out + min(row0 + r, d_out - 1);
    float acc[kRW][1] = {};
    rows_dot<BITS, 1>(wq, sc, bi, rows, d_in, xs, xsum, acc);
#pragma unroll
    for (int r = 0; r < kRW; ++r) total[r] = fmaf(g, acc[r][0], total[r]);
  }
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < kRW; ++r)
      if (row0 + r < d_out) store_out<OutT>(out + (size_t)t * d_out + row0 + r, total[r]);
  }
}

// ---------------------------------------------------------------------------
// Host helpers
// ---------------------------------------------------------------------------
size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

struct MoeLayout {
  size_t offsets, active, slot_of, perm, h, y, total;
};

MoeLayout layout(int n, int k, int n_experts, int d_model, int d_ffn) {
  MoeLayout L;
  const size_t pairs = (size_t)n * k;
  size_t at = 0;
  L.offsets = at; at += align256((n_experts + 1) * 4);
  L.active = at;  at += align256((n_experts + 1) * 4);
  L.slot_of = at; at += align256(pairs * 4);
  L.perm = at;    at += align256(pairs * 4);
  L.h = at;       at += align256(pairs * (size_t)d_ffn * 4);
  L.y = at;       at += align256(pairs * (size_t)d_model * 4);
  L.total = at;
  return L;
}

int launch_route_core(const float* logits, const f16* x, const f16* router, int d,
                      uint32_t* idx, float* gate, int n, int n_experts, int k, hipStream_t st) {
  const int epl = (n_experts + kWave - 1) / kWave;
#define KVP_EPL(N)                                                                            \
  if (epl <= N) {                                                                             \
    if (logits)                                                                               \
      hipLaunchKernelGGL(route_logits_kernel<N>, dim3((n + kWaves - 1) / kWaves), dim3(kBlock), \
                         0, st, logits, idx, gate, n, n_experts, k);                          \
    else                                                                                      \
      hipLaunchKernelGGL(route_x_kernel<N>, dim3(n), dim3(kBlock), 0, st, x, router, idx,     \
                         gate, d, n_experts, k);                                              \
    return check_launch("kvp_moe_route");                                                     \
  }
  KVP_EPL(1) KVP_EPL(2) KVP_EPL(4) KVP_EPL(8) KVP_EPL(16)
#undef KVP_EPL
  return set_error(KVP_INVALID, "kvp_moe_route: n_experts=%d above %d", n_experts, kMaxExperts);
}

int check_route_args(int n, int n_experts, int k) {
  KVP_REQUIRE(n >= 1, "kvp_moe_route: n=%d", n);
  KVP_REQUIRE(n_experts >= 1 && n_experts <= kMaxExperts,
              "kvp_moe_route: n_experts=%d outside 1..%d", n_experts, kMaxExperts);
  KVP_REQUIRE(k >= 1 && k <= kMaxK && k <= n_experts, "kvp_moe_route: k=%d (1..%d, <= n_experts)",
              k, kMaxK);
  return KVP_OK;
}

template <int BITS>
int launch_experts(const ExpertArgs& a, int max_active, bool swiglu_f16, bool f32_input,
                   hipStream_t st) {
  using Gm = Geom<BITS>;
  const dim3 grid((a.d_out + kRowsPerBlock - 1) / kRowsPerBlock, max_active);
  if (f32_input) {
    hipLaunchKernelGGL(expert_f32_kernel<BITS>, grid, dim3(kBlock), 0, st, a);
  } else {
    const size_t lds = (size_t)(a.d_in / Gm::kUnitCodes) * (kMT * Gm::kUnitPairs + kMT) * 4;
    if (swiglu_f16)
      hipLaunchKernelGGL((expert_f16_kernel<BITS, true>), grid, dim3(kBlock), lds, st, a);
    else
      hipLaunchKernelGGL((expert_f16_kernel<BITS, false>), grid, dim3(kBlock), lds, st, a);
  }
  return check_launch("kvp_moe expert gemv");
}

int launch_experts_bits(int bits, const ExpertArgs& a, int max_active, bool swiglu, bool f32_in,
                        hipStream_t st) {
  switch (bits) {
    case 2: return launch_experts<2>(a, max_active, swiglu, f32_in, st);
    case 3: return launch_experts<3>(a, max_active, swiglu, f32_in, st);
    case 4: return launch_experts<4>(a, max_active, swiglu, f32_in, st);
    case 8: return launch_experts<8>(a, max_active, swiglu, f32_in, st);
  }
  return set_error(KVP_UNSUPPORTED, "kvp_moe: bits=%d not in {2,3,4,8}", bits);
}

int launch_scatter(const float* y, const int32_t* slot_of, const float* gate, void* out,
                   int out_dtype, int n, int k, int d, hipStream_t st) {
  const long long total = (long long)n * d;
  const unsigned blocks = (unsigned)((total + kBlock - 1) / kBlock);
  if (out_dtype == KVP_F16)
    hipLaunchKernelGGL(scatter_kernel<f16>, dim3(blocks), dim3(kBlock), 0, st, y, slot_of, gate,
                       static_cast<f16*>(out), n, k, d);
  else
    hipLaunchKernelGGL(scatter_kernel<float>, dim3(blocks), dim3(kBlock), 0, st, y, slot_of,
                       gate, static_cast<float*>(out), n, k, d);
  return check_launch("kvp_moe scatter");
}

// Every per-expert kernel stages up to kMT tokens of d_in fp16 in LDS.
int check_expert_dims(const char* who, int d_in, int d_out, int bits) {
  KVP_REQUIRE(d_in >= 64 && d_in % 64 == 0, "%s: d_in=%d must be a positive multiple of 64", who,
              d_in);
  KVP_REQUIRE(d_out >= 1, "%s: d_out=%d", who, d_out);
  KVP_REQUIRE((size_t)d_in * kMT * 2 + (size_t)d_in * 4 <= 96 * 1024,
              "%s: d_in=%d too wide to stage %d tokens in LDS", who, d_in, kMT);
  if (bits != 2 && bits != 3 && bits != 4 && bits != 8)
    return set_error(KVP_UNSUPPORTED, "%s: bits=%d not in {2,3,4,8}", who, bits);
  return KVP_OK;
}

}  // namespace
}  // namespace kvp

using namespace kvp;

extern "C" int kvp_moe_route_logits(const float* logits, uint32_t* idx, float* gate, int n,
                                    int n_experts, int k, void* stream) {
  clear_error();
  KVP_REQUIRE(logits && idx && gate, "kvp_moe_route_logits: null pointer argument");
  if (int rc = check_route_args(n, n_experts, k)) return rc;
  return launch_route_core(logits, nullptr, nullptr, 0, idx, gate, n, n_experts, k,
                           static_cast<hipStream_t>(stream));
}

extern "C" int kvp_moe_route(const void* x, const void* router, uint32_t* idx, float* gate, int n,
                             int d, int n_experts, int k, void* stream) {
  clear_error();
  KVP_REQUIRE(x && router && idx && gate, "kvp_moe_route: null pointer argument");
  KVP_REQUIRE(d >= 1, "kvp_moe_route: d=%d", d);
  if (int rc = check_route_args(n, n_experts, k)) return rc;
  return launch_route_core(nullptr, static_cast<const f16*>(x), static_cast<const f16*>(router),
                           d, idx, gate, n, n_experts, k, static_cast<hipStream_t>(stream));
}

extern "C" int kvp_moe_permute(const uint32_t* idx, int32_t* offsets, int32_t* perm, int n, int k,
                               int n_experts, void* stream) {
  clear_error();
  KVP_REQUIRE(idx && offsets && perm, "kvp_moe_permute: null pointer argument");
  KVP_REQUIRE(n >= 1 && k >= 1 && n_experts >= 1 && n_experts <= kMaxExperts,
              "kvp_moe_permute: n=%d k=%d n_experts=%d", n, k, n_experts);
  hipLaunchKernelGGL(permute_kernel, dim3(1), dim3(1024), 0, static_cast<hipStream_t>(stream), idx,
                     offsets, perm, nullptr, nullptr, n * k, n_experts);
  return check_launch("kvp_moe_permute");
}

extern "C" size_t kvp_moe_swiglu_workspace_bytes(int n, int k, int n_experts, int d_model,
                                                 int d_ffn) {
  if (n < 1 || k < 1 || n_experts < 1 || d_model < 1 || d_ffn < 1) return 0;
  return layout(n, k, n_experts, d_model, d_ffn).total;
}

extern "C" int kvp_moe_dispatch(const void* x, const uint32_t* idx, const float* gate,
                                const uint32_t* w_q, const void* scales, const void* biases,
                                void* out, int out_dtype, int n, int k, int n_experts, int d_out,
                                int d_in, int bits, void* stream) {
  clear_error();
  KVP_REQUIRE(x && idx && gate && w_q && scales && biases && out,
              "kvp_moe_dispatch: null pointer argument");
  KVP_REQUIRE(n >= 1 && k >= 1 && k <= kMaxK && n_experts >= 1,
              "kvp_moe_dispatch: n=%d k=%d n_experts=%d", n, k, n_experts);
  KVP_REQUIRE(out_dtype == KVP_F16 || out_dtype == KVP_F32, "kvp_moe_dispatch: out_dtype=%d",
              out_dtype);
  if (int rc = check_expert_dims("kvp_moe_dispatch", d_in, d_out, bits)) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid((d_out + kRowsPerBlock - 1) / kRowsPerBlock, n);
  const f16* xx = static_cast<const f16*>(x);
  const uint16_t* sc = static_cast<const uint16_t*>(scales);
  const uint16_t* bi = static_cast<const uint16_t*>(biases);
#define KVP_DISPATCH(B)                                                                       \
  case B: {                                                                                   \
    const size_t lds = (size_t)(d_in / Geom<B>::kUnitCodes) * (Geom<B>::kUnitPairs + 1) * 4;  \
    if (out_dtype == KVP_F16)                                                                 \
      hipLaunchKernelGGL((dispatch_kernel<B, f16>), grid, dim3(kBlock), lds, st, xx, idx,     \
                         gate, w_q, sc, bi, static_cast<f16*>(out), k, n_experts, d_out,      \
                         d_in);                                                               \
    else                                                                                      \
      hipLaunchKernelGGL((dispatch_kernel<B, float>), grid, dim3(kBlock), lds, st, xx, idx,   \
                         gate, w_q, sc, bi, static_cast<float*>(out), k, n_experts, d_out,    \
                         d_in);                                                               \
    return check_launch("kvp_moe_dispatch");                                                  \
  }
  switch (bits) {
    KVP_DISPATCH(2) KVP_DISPATCH(3) KVP_DISPATCH(4) KVP_DISPATCH(8)
  }
#undef KVP_DISPATCH
  return set_error(KVP_UNSUPPORTED, "kvp_moe_dispatch: bits=%d", bits);
}

extern "C" int kvp_moe_swiglu(const void* x, const uint32_t* idx, const float* gate,
                              const uint32_t* gate_wq, const void* gate_scales,
                              const void* gate_biases, const uint32_t* up_wq,
                              const void* up_scales, const void* up_biases,
                              const uint32_t* down_wq, const void* down_scales,
                              const void* down_biases, void* out, int out_dtype, int n, int k,
                              int n_experts, int d_model, int d_ffn, int bits, void* workspace,
                              size_t workspace_bytes, void* stream) {
  clear_error();
  KVP_REQUIRE(x && idx && gate && gate_wq && gate_scales && gate_biases && up_wq && up_scales &&
                  up_biases && down_wq && down_scales && down_biases && out,
              "kvp_moe_swiglu: null pointer argument");
  KVP_REQUIRE(n >= 1 && k >= 1 && k <= kMaxK && n_experts >= 1 && n_experts <= kMaxExperts,
              "kvp_moe_swiglu: n=%d k=%d n_experts=%d", n, k, n_experts);
  KVP_REQUIRE(out_dtype == KVP_F16 || out_dtype == KVP_F32, "kvp_moe_swiglu: out_dtype=%d",
              out_dtype);
  if (int rc = check_expert_dims("kvp_moe_swiglu (gate/up)", d_model, d_ffn, bits)) return rc;
  if (int rc = check_expert_dims("kvp_moe_swiglu (down)", d_ffn, d_model, bits)) return rc;
  const MoeLayout L = layout(n, k, n_experts, d_model, d_ffn);
  KVP_REQUIRE(workspace && workspace_bytes >= L.total,
              "kvp_moe_swiglu: workspace of %zu bytes, %zu needed", workspace_bytes, L.total);
  hipStream_t st = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  int32_t* offsets = reinterpret_cast<int32_t*>(ws + L.offsets);
  int32_t* active = reinterpret_cast<int32_t*>(ws + L.active);
  int32_t* slot_of = reinterpret_cast<int32_t*>(ws + L.slot_of);
  int32_t* perm = reinterpret_cast<int32_t*>(ws + L.perm);
  float* h = reinterpret_cast<float*>(ws + L.h);
  float* y = reinterpret_cast<float*>(ws + L.y);
  const int pairs = n * k;
  hipLaunchKernelGGL(permute_kernel, dim3(1), dim3(1024), 0, st, idx, offsets, perm, active,
                     slot_of, pairs, n_experts);
  if (int rc = check_launch("kvp_moe_swiglu (permute)")) return rc;
  const int max_active = pairs < n_experts ? pairs : n_experts;

  ExpertArgs a{};
  a.x = static_cast<const f16*>(x);
  a.wq0 = gate_wq;
  a.s0 = static_cast<const uint16_t*>(gate_scales);
  a.b0 = static_cast<const uint16_t*>(gate_biases);
  a.wq1 = up_wq;
  a.s1 = static_cast<const uint16_t*>(up_scales);
  a.b1 = static_cast<const uint16_t*>(up_biases);
  a.offsets = offsets;
  a.perm = perm;
  a.active = active;
  a.y = h;
  a.k = k;
  a.d_in = d_model;
  a.d_out = d_ffn;
  if (int rc = launch_experts_bits(bits, a, max_active, true, false, st)) return rc;

  ExpertArgs dn{};
  dn.xf = h;
  dn.wq0 = down_wq;
  dn.s0 = static_cast<const uint16_t*>(down_scales);
  dn.b0 = static_cast<const uint16_t*>(down_biases);
  dn.offsets = offsets;
  dn.perm = perm;
  dn.active = active;
  dn.y = y;
  dn.k = k;
  dn.d_in = d_ffn;
  dn.d_out = d_model;
  if (int rc = launch_experts_bits(bits, dn, max_active, false, true, st)) return rc;
  return launch_scatter(y, slot_of, gate, out, out_dtype, n, k, d_model, st);
}
