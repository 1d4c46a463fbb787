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
//                For a few pairs on the matrix-core path this launch is
//                folded into the gate/up launch: each block builds its own
//                expert's part of the same tables in LDS (block_route).
//   expert gemv  one block per (active expert, rows): the expert's weight
//                rows stream from HBM once for all of that expert's tokens
//                (the reference reads each expert once per token, :101-129).
//                fp16 activations use the qmv core (codes as exact fp16
//                denormals through V_DOT2_F32_F16); the SwiGLU down
//                projection takes its fp32 hidden state through fp32 FMAs.
//   scatter      out[t] = sum_s gate[t, s] * y[t, s], slots in order s = 0..k-1.
#include <math.h>

#include "common.h"
#include "mfma_core.h"
#include "qmv_core.h"

namespace kvp {
namespace {

constexpr int kBlock = 256;
constexpr int kWaves = kBlock / kWave;
constexpr int kMaxExperts = 1024;
constexpr int kMaxK = 32;
constexpr int kPermuteTile = 8192;  // routed pairs (n * k) one permutation holds

// ---------------------------------------------------------------------------
// Routing
// ---------------------------------------------------------------------------
// logits: E fp32 values of one token, held as E/64 per lane (lane-strided).
template <int EPL>
__device__ __forceinline__ void route_token(const float (&lg)[EPL], int n_experts, int k,
                                            uint32_t* __restrict__ idx, float* __restrict__ gate,
                                            uint32_t* idx2 = nullptr, float* gate2 = nullptr) {
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
  // k rounds: the largest p (a wave max), then the lowest expert index
  // holding it (ballots, lane-strided index order), knocked out (-inf).
  // Lane s keeps slot s; the renormalising sum runs in slot order.
  float my_p = 0.0f;
  int my_i = 0;
  float total = 0.0f;
  for (int s = 0; s < k; ++s) {  // wave-uniform
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < EPL; ++j) m = fmaxf(m, p[j]);
    m = wave_max(m);
    int bi = -1;
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      const unsigned long long hit = __ballot(p[j] == m);
      if (bi < 0 && hit != 0ull) bi = j * kWave + __ffsll((long long)hit) - 1;
    }
#pragma unroll
    for (int j = 0; j < EPL; ++j)
      if (lane + j * kWave == bi) p[j] = -INFINITY;
    if (lane == s) {
      my_p = m;
      my_i = bi;
    }
    total += m;
  }
  if (lane < k) {
    const float g = my_p / total;
    idx[lane] = (uint32_t)my_i;
    gate[lane] = g;
    if (idx2) {
      idx2[lane] = (uint32_t)my_i;
      gate2[lane] = g;
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
  __shared__ int32_t act_pos[kMaxExperts];
  __shared__ uint32_t tile[kPermuteTile];
  for (int e = threadIdx.x; e < n_experts; e += blockDim.x) cnt[e] = 0;
  for (int i = threadIdx.x; i < pairs; i += blockDim.x) tile[i] = idx[i];
  __syncthreads();
  for (int i = threadIdx.x; i < pairs; i += blockDim.x) {
    const uint32_t e = tile[i];
    if (e < (uint32_t)n_experts) atomicAdd(&cnt[e], 1);  // counts are order-free
  }
  __syncthreads();
  // Exclusive scans of the counts and of the routed flags: wave 0, each lane
  // a contiguous run of experts, then a scan of the lane totals.
  if (threadIdx.x < kWave) {
    const int lane = threadIdx.x;
    const int per = (n_experts + kWave - 1) / kWave;
    const int e0 = min(lane * per, n_experts), e1 = min(e0 + per, n_experts);
    int c = 0, f = 0;
    for (int e = e0; e < e1; ++e) {
      c += cnt[e];
      f += cnt[e] > 0;
    }
    int ci = c, fi = f;  // inclusive scans over lanes
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
      const int cu = __shfl_up(ci, d, kWave), fu = __shfl_up(fi, d, kWave);
      if (lane >= d) {
        ci += cu;
        fi += fu;
      }
    }
    int run = ci - c, act = fi - f;
    for (int e = e0; e < e1; ++e) {
      off[e] = run;
      act_pos[e] = act;
      run += cnt[e];
      act += cnt[e] > 0;
    }
    if (lane == kWave - 1) {
      off[n_experts] = ci;
      if (active) active[0] = fi;
    }
  }
  __syncthreads();
  for (int e = threadIdx.x; e <= n_experts; e += blockDim.x) offsets[e] = off[e];
  if (active)
    for (int e = threadIdx.x; e < n_experts; e += blockDim.x)
      if (cnt[e] > 0) active[1 + act_pos[e]] = e;
  // Stable placement: a pair's rank among the earlier pairs of its expert.
  // A pair naming no valid expert is never placed (slot -1: the scatter
  // skips it).
  for (int i = threadIdx.x; i < pairs; i += blockDim.x) {
    const uint32_t e = tile[i];
    int pos = -1;
    if (e < (uint32_t)n_experts) {
      int rank = 0;
      for (int j = 0; j < i; ++j) rank += tile[j] == e;
      pos = off[e] + rank;
      perm[pos] = i;
    }
    if (slot_of) slot_of[i] = pos;
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
  // In-block routing (gate/up launch, pairs <= kFusedPairs): the flat expert
  // indices in, and the permute kernel's tables out for the launches after.
  const uint32_t* idx;     // [pairs]
  int pairs, n_experts;
  // In-block routing from logits (kvp_moe_route_swiglu, a few tokens): the
  // launch routes every token itself (the logits-door contract) instead of
  // reading idx; block (0, 0) also writes the routing to out_idx / out_gate.
  const float* logits;     // [n][n_experts] fp32, or null
  int n_tokens, epl;       // tokens (any in-block routing); experts per lane (1, 2 or 4)
  uint32_t* out_idx;       // [n][k]
  float* out_gate;         // [n][k]
  int32_t* t_offsets;      // [E+1]: entries e and e + 1 of every routed e
  int32_t* t_perm;         // [pairs]
  int32_t* t_active;       // [1 + E]
  int32_t* t_slot_of;      // [pairs]
};

// Pairs (n * k) up to which the gate/up launch builds its routing in-block.
constexpr int kFusedPairs = 512;
// Tokens up to which kvp_moe_route_swiglu routes inside the gate/up launch
// (each block routes every token, one per wave: measured, two per wave
// cost the gate/up blocks more than the routing launch they replace).
constexpr int kRouteTokensInBlock = 4;

struct BlockRoute {
  int e, p0, p1;           // the expert and its segment [p0, p1) of the sorted order
  const int32_t* seg;      // LDS: the segment's flat pair indices, in flat order
};

// Every token's routing, computed by this block from the logits (wave w
// routes tokens w, w + 4, ...), into the LDS tile; the launch's first block
// also writes it to the routing outputs.
template <int EPL>
__device__ void route_tokens_in_block(const ExpertArgs& a, uint32_t* tile, float* gate_sh,
                                      bool write_out) {
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  for (int t = wave; t < a.n_tokens; t += kWaves) {  // wave-uniform
    float lg[EPL];
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      const int e = lane + j * kWave;
      lg[j] = e < a.n_experts ? a.logits[(size_t)t * a.n_experts + e] : 0.0f;
    }
    route_token<EPL>(lg, a.n_experts, a.k, tile + t * a.k, gate_sh + t * a.k,
                     write_out ? a.out_idx + (size_t)t * a.k : nullptr,
                     write_out ? a.out_gate + (size_t)t * a.k : nullptr);
  }
}

// The permute kernel's result for one expert, built by one block from the
// flat indices: e is the act-th routed expert in ascending order, its pairs
// are the flat indices i with idx[i] == e in flat order (a stable sort),
// and p0 counts the valid pairs routed to experts below e. Every block of
// the launch builds the same table from the same indices; the first row
// block of each expert also writes its entries of offsets, active, perm and
// slot_of, the tables the down projection and the scatter read; block
// (0, 0) writes the count of routed experts and the -1 slots of invalid
// indices. False for a block past the routed experts. Called by every
// thread of the block.
__device__ bool block_route(const ExpertArgs& a, int act, BlockRoute& br) {
  __shared__ uint32_t tile[kFusedPairs];
  __shared__ uint32_t routed[kMaxExperts / 32];
  __shared__ int32_t seg[kFusedPairs];
  __shared__ int s_e, s_total, s_p0, s_n;
  const int pairs = a.pairs, n_experts = a.n_experts;
  for (int w = threadIdx.x; w < kMaxExperts / 32; w += kBlock) routed[w] = 0u;
  if (a.logits) {  // route here: wave w takes tokens w, w + 4, ...
    __shared__ float gate_sh[kFusedPairs];
    const bool first = blockIdx.x == 0 && blockIdx.y == 0;
    switch (a.epl) {
      case 1: route_tokens_in_block<1>(a, tile, gate_sh, first); break;
      case 2: route_tokens_in_block<2>(a, tile, gate_sh, first); break;
      default: route_tokens_in_block<4>(a, tile, gate_sh, first); break;
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < pairs; i += kBlock) {
    const uint32_t e = a.logits ? tile[i] : a.idx[i];
    tile[i] = e;
    if (e < (uint32_t)n_experts) atomicOr(&routed[e >> 5], 1u << (e & 31));
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int seen = 0, found = -1;
    for (int w = 0; w < (n_experts + 31) / 32; ++w) {
      uint32_t m = routed[w];
      const int c = __popc(m);
      if (found < 0 && act < seen + c) {
        for (int skip = act - seen; skip > 0; --skip) m &= m - 1u;  // drop the lowest set bit
        found = 32 * w + __ffs(m) - 1;
      }
      seen += c;
    }
    s_e = found;
    s_total = seen;
  }
  __syncthreads();
  const int e = s_e;
  if (blockIdx.x == 0 && act == 0) {  // also when no pair names a valid expert
    if (threadIdx.x == 0) a.t_active[0] = s_total;
    for (int i = threadIdx.x; i < pairs; i += kBlock)
      if (tile[i] >= (uint32_t)n_experts) a.t_slot_of[i] = -1;
  }
  if (e < 0) return false;  // block-uniform
  if (threadIdx.x < kWave) {  // wave 0: ballot compaction, 64 pairs a round
    const int lane = threadIdx.x;
    const unsigned long long below_lane = (1ull << lane) - 1ull;
    int lower = 0, mine = 0;
    for (int i0 = 0; i0 < pairs; i0 += kWave) {  // wave-uniform
      const int i = i0 + lane;
      const uint32_t ti = i < pairs ? tile[i] : 0xffffffffu;
      const unsigned long long hit = __ballot(ti == (uint32_t)e);
      const unsigned long long low = __ballot(ti < (uint32_t)e);
      if (ti == (uint32_t)e) seg[mine + __popcll(hit & below_lane)] = i;
      mine += __popcll(hit);
      lower += __popcll(low);
    }
    if (lane == 0) {
      s_p0 = lower;
      s_n = mine;
    }
  }
  __syncthreads();
  br = BlockRoute{e, s_p0, s_p0 + s_n, seg};
  if (blockIdx.x == 0) {
    for (int r = threadIdx.x; r < s_n; r += kBlock) {
      a.t_perm[br.p0 + r] = seg[r];
      a.t_slot_of[seg[r]] = br.p0 + r;
    }
    if (threadIdx.x == 0) {
      a.t_offsets[e] = br.p0;
      a.t_offsets[e + 1] = br.p1;  // the next routed expert writes the same value
      a.t_active[1 + act] = e;
    }
  }
  return true;
}

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

// Matrix-core expert GEMV (4/8-bit codes), the qmv_mfma layout per expert:
// a block is one 16-row tile of one routed expert; the four waves split the
// tile's groups; A rows are up to four activation rows of the expert's
// pairs, block-diagonal over the four k-octets so each lane quarter walks
// its own 64-code group. fp16 activations (gate/up) give four tokens per
// pass; the fp32 hidden state of the down projection enters as two tokens
// per pass, each as an exact fp16 hi/lo pair (h * 2^-E = hi + lo to 22 bits,
// E a power-of-two shift that keeps every value inside fp16), so no fp16
// intermediate replaces h (contract C1): D(hi) + D(lo) is the fp32 product.
// SwiGLU computes the gate and up tiles of the same rows together.
constexpr int kEMT = 4;                              // A rows per pass
constexpr int kEGroupSlots = 9;                      // 8 operand slots + 1 pad (banks)

template <int BITS, bool SWIGLU>
struct ExpertStep {
  uint32_t w[SWIGLU ? 2 : 1][MfmaShape<BITS, kEMT>::kWPL];
  uint16_t s[SWIGLU ? 2 : 1], b[SWIGLU ? 2 : 1];  // fp16 bits of the group scale and bias
};

// KQ waves share one tile's steps (KQ = 4: one tile per block, for long
// rows) or each wave runs all of its own tile's steps (KQ = 1: four tiles per
// block share one staging of the activations, for short rows).
// At 4 bits, four waves per SIMD in both forms: the allocator otherwise
// spends a few registers more and drops one. With KQ = 1 that is what two
// steps in flight allow (four took 168 registers, three waves: at n = 32
// only 768 of the gate/up launch's 1320 live blocks then ran at once, and
// the rest started as a second generation); each slot is refilled with the
// step two ahead as soon as it is used, so two stay in flight throughout
// (measured, config 5 n = 32 107.8 -> 104.6 us, n = 8 53.6 -> 53.2). 8-bit
// forms need more registers than that and keep the allocator's choice.
//
// SBX (gate/up, one tile per wave, G % 16 == 0): the group scales and
// biases reach the steps through a per-wave LDS tile instead of a 2-byte
// load per step and array. Lane (n, h) needs group 4 st + h of row n at
// step st, so each such load touched 16 rows for 128 bytes and was issued
// again every step; one 8-byte load per array now covers four steps (lane
// (n, h) loads groups 4 st0 + 4h .. + 3), and the four lanes of a row meet
// in LDS. Measured (config 5, 4-bit): a loads-only copy of the kernels ran
// 17 us faster at n = 32 without the per-step scale loads; with the tile,
// n = 32 100.4 -> 87.5 us and n = 8 52.4 -> 46.1. The form holds 164
// registers (three waves per SIMD): at four it spilled, and ran 91.8 us.
// The fp32-input down projection takes the same tile when its steps fit
// one batch (G <= 16): written once, it serves every pass (86.3 us).
template <int BITS, bool SWIGLU, bool F32IN, int KQ, bool ROUTE = false, bool SBX = false>
__global__ __launch_bounds__(kBlock)
__attribute__((amdgpu_waves_per_eu(BITS == 4 ? ((SBX && SWIGLU) ? 3 : 4) : 1)))
void expert_mfma_kernel(ExpertArgs a) {
  using S = MfmaShape<BITS, kEMT>;
  constexpr int NP = SWIGLU ? 2 : 1;            // projections per tile
  constexpr int TPP = F32IN ? kEMT / 2 : kEMT;  // tokens per pass
  constexpr int TB = kWaves / KQ;               // tiles per block
  // Steps in flight per wave. The one-tile-per-wave down projection holds
  // four: a tile of up to four steps (d_in <= 1024) then stays in registers
  // over all of its expert's passes (two tokens each) instead of streaming
  // once per pass (config 5 n = 32: down traffic 1.24 x its weights; 103.4
  // -> 101.3 us).
  constexpr int RS = (KQ == 1 && F32IN) ? 4 : 2;
  extern __shared__ __align__(16) uint4 lds[];
  __shared__ float red[kWaves][NP][kEMT][16];
  static_assert(!ROUTE || (SWIGLU && !F32IN), "in-block routing is the gate/up launch's");
  static_assert(!SBX || (KQ == 1 && (SWIGLU ? (!F32IN && RS == 2) : (F32IN && RS == 4))),
                "scale tiles: one wave per tile (gate/up, or the fp32-input down projection)");
  const int act = blockIdx.y;
  const int G = a.d_in / 64;  // a multiple of 4 (checked by the launcher)
  // In-block routing, up to kEMT tokens (every expert's pairs fit one pass):
  // thread t requests group t % G of token t / G before routing, so the
  // activations arrive while the block routes, and stages them right after
  // it (the pairs' tokens are then known), before the expert's weight loads
  // go out; otherwise they would return behind the weights.
  const bool pre_x = ROUTE && a.n_tokens <= kEMT && a.n_tokens * G <= kBlock;  // one pass
  const int x_tok = pre_x && (int)threadIdx.x < a.n_tokens * G ? (int)threadIdx.x / G : -1;
  const int x_g = pre_x ? (int)threadIdx.x % G : 0;
  u32x4 xv[8];
  if constexpr (ROUTE) {
    if (x_tok >= 0) {
      const uint32_t* src =
          reinterpret_cast<const uint32_t*>(a.x + (size_t)x_tok * a.d_in + x_g * 64);
#pragma unroll
      for (int q = 0; q < 8; ++q) xv[q] = *reinterpret_cast<const u32x4*>(src + 4 * q);
    }
  }
  int e, p0, p1;
  const int32_t* seg = nullptr;  // ROUTE: the expert's flat pair indices (LDS)
  if constexpr (ROUTE) {
    BlockRoute br;
    if (!block_route(a, act, br)) return;  // block-uniform
    e = br.e;
    p0 = br.p0;
    p1 = br.p1;
    seg = br.seg;
  } else {
    if (act >= a.active[0]) return;  // block-uniform
    e = a.active[1 + act];
    p0 = a.offsets[e];
    p1 = a.offsets[e + 1];
  }
  const int steps = G / S::kNB;
  const int m_stride = G * kEGroupSlots + 1;  // slots per A row
  uint4* xs = lds;
  uint4* zeros = lds + kEMT * m_stride;
  float* sums = reinterpret_cast<float*>(zeros + S::kT);  // [G][kEMT]
  float* mult = sums + G * kEMT;                           // [G][kEMT] (fp32 input only)
  // SBX: the wave's scale/bias tile of four steps, [array][row][20 halves]
  // (16 groups + pad: a 40-byte pitch puts a step's 64 reads on 32 banks)
  uint16_t* sbt = reinterpret_cast<uint16_t*>(mult + G * kEMT) +
                  __builtin_amdgcn_readfirstlane(threadIdx.x / kWave) * (4 * 16 * 20);

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int tl = wave / KQ, kq = wave - tl * KQ;
  const int n = lane & 15, h = lane >> 4;  // blk = h (MT = 4: one octet per block)
  const int row = (blockIdx.x * TB + tl) * 16 + n;
  const bool row_ok = row < a.d_out;
  const uint32_t row_bytes = (uint32_t)a.d_in * BITS / 8;
  const size_t erow = (size_t)e * a.d_out;
  const uint32_t wbytes = (uint32_t)(a.d_out * row_bytes), sbytes = (uint32_t)(a.d_out * G * 2);
  __amdgpu_buffer_rsrc_t wr[NP], sr[NP], br[NP];
  wr[0] = rsrc(a.wq0 + erow * (row_bytes / 4), wbytes);
  sr[0] = rsrc(a.s0 + erow * G, sbytes);
  br[0] = rsrc(a.b0 + erow * G, sbytes);
  if constexpr (SWIGLU) {
    wr[1] = rsrc(a.wq1 + erow * (row_bytes / 4), wbytes);
    sr[1] = rsrc(a.s1 + erow * G, sbytes);
    br[1] = rsrc(a.b1 + erow * G, sbytes);
  }
  const uint32_t code_base = row_ok ? (uint32_t)row * row_bytes + h * S::kGroupBytes : kOutOfRange;
  const uint32_t sb_base = row_ok ? ((uint32_t)row * G + h) * 2 : kOutOfRange;
  const bool a_live = (n >> 2) == h;  // A row n is (block n / 4, x row n % 4)
  const uint4* a_base = a_live ? xs + (n & 3) * m_stride + h * kEGroupSlots : zeros;
  const uint32_t a_mul = a_live ? 1u : 0u;

  auto load = [&](ExpertStep<BITS, SWIGLU>& R, int st) {
    const bool live = st < steps;  // wave-uniform
    const uint32_t co = code_base + (live ? (uint32_t)st * 4 * S::kGroupBytes : kOutOfRange);
    const uint32_t so = sb_base + (live ? (uint32_t)st * 4 * 2 : kOutOfRange);
#pragma unroll
    for (int pj = 0; pj < NP; ++pj) {
#pragma unroll
      for (int i = 0; i < S::kWPL; i += 4) {
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(wr[pj], co + 4 * i, 0, 0);
        R.w[pj][i] = v.x; R.w[pj][i + 1] = v.y; R.w[pj][i + 2] = v.z; R.w[pj][i + 3] = v.w;
      }
      if constexpr (!SBX) {
        R.s[pj] = buffer_load_h16(sr[pj], so);
        R.b[pj] = buffer_load_h16(br[pj], so);
      }
    }
  };
  // SBX: lane (n, h) loads groups 4 st0 + 4h .. + 3 of row n from each array
  // (one 8-byte load per array covers four steps; G % 16 == 0 keeps it
  // aligned) and writes them to the wave's tile, where step st0 + j reads
  // group 4 (st0 + j) + h, its own.
  const uint32_t sbx_base = row_ok ? ((uint32_t)row * G + 4 * h) * 2 : kOutOfRange;
  uint32_t sxc[NP][2][2];
  auto sbx_load = [&](int st0) {
    if constexpr (SBX) {
      // A lane whose step lies past the row's last (a tile of fewer than
      // four steps) loads nothing.
      const uint32_t so = st0 + h < steps ? sbx_base + (uint32_t)st0 * 8 : kOutOfRange;
#pragma unroll
      for (int pj = 0; pj < NP; ++pj) {
        const u32x2 s = __builtin_amdgcn_raw_buffer_load_b64(sr[pj], so, 0, 0);
        const u32x2 b = __builtin_amdgcn_raw_buffer_load_b64(br[pj], so, 0, 0);
        sxc[pj][0][0] = s.x; sxc[pj][0][1] = s.y; sxc[pj][1][0] = b.x; sxc[pj][1][1] = b.y;
      }
    }
  };
  auto sbx_commit = [&]() {
    if constexpr (SBX) {
#pragma unroll
      for (int pj = 0; pj < NP; ++pj)
#pragma unroll
        for (int k = 0; k < 2; ++k)
          *reinterpret_cast<u32x2*>(sbt + ((2 * pj + k) * 16 + n) * 20 + 4 * h) =
              u32x2{sxc[pj][k][0], sxc[pj][k][1]};
    }
  };
  // A wave's steps are kq, kq + KQ, ...; RS of them are in flight at a time
  // (the first RS are requested before anything else).
  const int nt0 = min(TPP, p1 - p0);
  if (pre_x) {  // the one pass, q0 = p0
    // The activations pass through an empty asm here, so no work on them
    // is scheduled before routing (which would wait for them first, then
    // for the logits, one memory round trip after the other).
#pragma unroll
    for (int q = 0; q < 8; ++q) asm volatile("" : "+v"(xv[q]));
    // Rows past the expert's pairs are zeros; row m < nt0 is its pair's
    // token, written by the thread holding that token's group.
    for (int it = threadIdx.x; it < kEMT * G; it += kBlock) {
      const int m = it / G, g = it - m * G;
      if (m >= nt0) {
        uint4* dst = xs + m * m_stride + g * kEGroupSlots;
#pragma unroll
        for (int q = 0; q < 8; ++q) dst[q] = uint4{0, 0, 0, 0};
        sums[g * kEMT + m] = 0.0f;
      }
    }
    if (x_tok >= 0) {
      u32x4 ow[8];
      float s0 = 0.0f, s1 = 0.0f;  // the two halves' sums, as the staging loop forms them
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        ow[q] = to_slot_order<BITS>(xv[q]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (q < 4) s0 = dot2(ow[q][j], 0x3C003C00u, s0);
          else s1 = dot2(ow[q][j], 0x3C003C00u, s1);
        }
      }
      const float sum = s0 + s1;
      for (int m = 0; m < nt0; ++m) {
        if (seg[m] / a.k != x_tok) continue;
        uint4* dst = xs + m * m_stride + x_g * kEGroupSlots;
#pragma unroll
        for (int q = 0; q < 8; ++q) dst[q] = uint4{ow[q].x, ow[q].y, ow[q].z, ow[q].w};
        sums[x_g * kEMT + m] = sum;
      }
    }
  }
  const int spw = (steps - kq + KQ - 1) / KQ;  // wave-uniform
  ExpertStep<BITS, SWIGLU> R[RS];
  sbx_load(0);
#pragma unroll
  for (int j = 0; j < RS; ++j) load(R[j], kq + KQ * j);
  if (threadIdx.x < S::kT) zeros[threadIdx.x] = uint4{0, 0, 0, 0};
  bool fresh = true;  // R holds this wave's first RS steps

  for (int q0 = p0; q0 < p1; q0 += TPP) {  // block-uniform passes over the expert's pairs
    const int nt = min(TPP, p1 - q0);
    if (pre_x) {
      // staged before the weight loads (above)
    } else if constexpr (!F32IN) {
      // Stage: item (token row m, group g) in two halves of 32 values on
      // adjacent lanes (every thread busy, half the registers; n = 32 102.4
      // -> 100.9 us); the group's sum is the two half sums added.
      for (int it2 = threadIdx.x; it2 < 2 * kEMT * G; it2 += kBlock) {
        const int it = it2 >> 1, hf = it2 & 1;
        const int m = it / G, g = it - m * G;
        uint4* dst = xs + m * m_stride + g * kEGroupSlots + 4 * hf;
        float sum = 0.0f;
        u32x4 v[4];
        const bool live = m < nt;
        const int pair = live ? (ROUTE ? seg[q0 - p0 + m] : a.perm[q0 + m]) : 0;
        const int tok = pair / a.k;
        const uint32_t* src =
            reinterpret_cast<const uint32_t*>(a.x + (size_t)tok * a.d_in + g * 64) + 16 * hf;
#pragma unroll
        for (int q = 0; q < 4; ++q)
          v[q] = live ? *reinterpret_cast<const u32x4*>(src + 4 * q) : u32x4{0, 0, 0, 0};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const u32x4 ow = to_slot_order<BITS>(v[q]);
#pragma unroll
          for (int j = 0; j < 4; ++j) sum = dot2(ow[j], 0x3C003C00u, sum);
          dst[q] = uint4{ow.x, ow.y, ow.z, ow.w};
        }
        sum += __shfl_xor(sum, 1);  // both lanes of an item take this iteration
        if (hf == 0) sums[g * kEMT + m] = sum;
      }
    } else {
      // Stage: item (token, group, quarter of 16 values), four lanes per
      // (token, group) that agree on its shift; each writes its two slots of
      // the hi row (2 tk) and the lo row (2 tk + 1).
      for (int it = threadIdx.x; it < TPP * G * 4; it += kBlock) {
        const int qq = it & 3, tg = it >> 2;
        const int tk = tg / G, g = tg - tk * G;
        const bool live = tk < nt;
        const float* src = a.xf + (size_t)(q0 + (live ? tk : 0)) * a.d_in + g * 64 + 16 * qq;
        float hv[16];
#pragma unroll
        for (int i = 0; i < 16; i += 4) {
          const float4 v = live ? *reinterpret_cast<const float4*>(src + i) : float4{0, 0, 0, 0};
          hv[i] = v.x; hv[i + 1] = v.y; hv[i + 2] = v.z; hv[i + 3] = v.w;
        }
        float mx = 0.0f, tot = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          mx = fmaxf(mx, fabsf(hv[i]));
          tot += hv[i];
        }
        mx = fmaxf(mx, __shfl_xor(mx, 1, 4));
        mx = fmaxf(mx, __shfl_xor(mx, 2, 4));
        tot += __shfl_xor(tot, 1, 4);
        tot += __shfl_xor(tot, 2, 4);
        // Shift so the largest |h| stays below 2^14: hi and lo then fit fp16.
        const int ex = mx > 0.0f ? max(0, ilogbf(mx) - 13) : 0;
        const float inv = ldexpf(1.0f, -ex);
        uint4* dhi = xs + (2 * tk) * m_stride + g * kEGroupSlots + 2 * qq;
        uint4* dlo = dhi + m_stride;
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          f16x8 hi8, lo8;
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const float hs = hv[8 * q + j] * inv;
            const _Float16 hi = (_Float16)hs;
            hi8[j] = hi;
            lo8[j] = (_Float16)(hs - (float)hi);
          }
          const u32x4 oh = to_slot_order<BITS>(__builtin_bit_cast(u32x4, hi8));
          const u32x4 ol = to_slot_order<BITS>(__builtin_bit_cast(u32x4, lo8));
          dhi[q] = uint4{oh.x, oh.y, oh.z, oh.w};
          dlo[q] = uint4{ol.x, ol.y, ol.z, ol.w};
        }
        if (qq == 0) {  // b * sum(h) rides on the hi row; both rows scale back by 2^E
          sums[g * kEMT + 2 * tk] = tot;
          sums[g * kEMT + 2 * tk + 1] = 0.0f;
          mult[g * kEMT + 2 * tk] = mult[g * kEMT + 2 * tk + 1] = ldexpf(1.0f, ex);
        }
      }
    }
    lds_barrier();

    f32x4 acc[NP];
#pragma unroll
    for (int pj = 0; pj < NP; ++pj) acc[pj] = f32x4{0, 0, 0, 0};
    auto step = [&](const ExpertStep<BITS, SWIGLU>& Rs, int st) {
      const int g = st * S::kNB + h;  // this lane's group (D rows and codes alike)
      const uint4* a_src = a_base + a_mul * (uint32_t)(st * S::kNB * kEGroupSlots);
      const f32x4 sm = *reinterpret_cast<const f32x4*>(sums + g * kEMT);
      f32x4 mu = {1.0f, 1.0f, 1.0f, 1.0f};
      if constexpr (F32IN) mu = *reinterpret_cast<const f32x4*>(mult + g * kEMT);
#pragma unroll
      for (int pj = 0; pj < NP; ++pj) {
        f32x4 d = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int t = 0; t < S::kT; ++t)
          d = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a_src[t]),
                                                     code_operand<BITS>(Rs.w[pj], t), d, 0, 0, 0);
        float sc, bi;
        if constexpr (SBX) {
          const uint16_t* t = sbt + (2 * pj * 16 + n) * 20 + 4 * (st & 3) + h;
          sc = h16_to_f32(t[0]) * 16777216.0f;  // c * 2^-24
          bi = h16_to_f32(t[16 * 20]);
        } else {
          sc = h16_to_f32(Rs.s[pj]) * 16777216.0f;
          bi = h16_to_f32(Rs.b[pj]);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[pj][r] = fmaf(sc * mu[r], d[r], fmaf(bi, sm[r], acc[pj][r]));
      }
    };
    if constexpr (SBX && SWIGLU) {
      // Batches of four steps (spw % 4 == 0): the batch's scale tile goes to
      // LDS, the next batch's (or the next pass's first) is requested, then
      // the four steps run with rolling refills of the two step slots.
      const bool more = q0 + TPP < p1;  // block-uniform: another pass follows
      for (int bb = 0; bb < spw; bb += 4) {  // wave-uniform
        sbx_commit();
        const int nb = bb + 4 < spw ? bb + 4 : (more ? 0 : steps);
        if (nb < steps) sbx_load(nb);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          step(R[j & 1], bb + j);
          const int nx = bb + j + RS;
          if (nx < spw) load(R[j & 1], nx);
          else if (more) load(R[j & 1], nx - spw);
        }
      }
    } else if constexpr (KQ == 1) {
      // Rolling: slot j is refilled with the step RS ahead right after its
      // use; after its last use in a pass, with the next pass's step j (the
      // first RS steps are requested before the first pass). With spw <= RS
      // every step keeps its slot from pass to pass.
      if constexpr (SBX) {  // down projection (spw <= 4): its scale tile once, kept in LDS
        if (q0 == p0) sbx_commit();
      }
      const bool more = q0 + TPP < p1;  // block-uniform: another pass follows
      for (int jb = 0; jb < spw; jb += RS) {  // wave-uniform
#pragma unroll
        for (int j = 0; j < RS; ++j) {
          if (jb + j < spw) {
            step(R[j], jb + j);
            const int nx = jb + j + RS;
            if (nx < spw) load(R[j], nx);
            else if (more && spw > RS) load(R[j], j);
          }
        }
      }
    } else {
      // Batches of RS steps per wave, requested together.
      for (int jb = 0; jb < spw; jb += RS) {  // wave-uniform
        if (!fresh) {
#pragma unroll
          for (int j = 0; j < RS; ++j) load(R[j], kq + KQ * (jb + j));
        }
        fresh = false;
#pragma unroll
        for (int j = 0; j < RS; ++j)
          if (jb + j < spw) step(R[j], kq + KQ * (jb + j));
      }
    }
    // Merge the four row blocks (other groups, same A rows), then the waves.
#pragma unroll
    for (int pj = 0; pj < NP; ++pj)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        acc[pj][r] += __shfl_xor(acc[pj][r], 16);
        acc[pj][r] += __shfl_xor(acc[pj][r], 32);
      }
    if (h == 0) {
#pragma unroll
      for (int pj = 0; pj < NP; ++pj)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[wave][pj][r][n] = acc[pj][r];
    }
    __syncthreads();
    if (threadIdx.x < TB * TPP * 16) {
      const int tt = threadIdx.x / (TPP * 16), tk = (threadIdx.x >> 4) % TPP, nn = threadIdx.x & 15;
      const int orow = (blockIdx.x * TB + tt) * 16 + nn;
      float v[NP];
#pragma unroll
      for (int pj = 0; pj < NP; ++pj) {
        v[pj] = 0.0f;
#pragma unroll
        for (int w = 0; w < KQ; ++w) {
          const int ww = tt * KQ + w;
          if constexpr (F32IN) v[pj] += red[ww][pj][2 * tk][nn] + red[ww][pj][2 * tk + 1][nn];
          else v[pj] += red[ww][pj][tk][nn];
        }
      }
      float out = v[0];
      if constexpr (SWIGLU) out = silu(v[0]) * v[1];
      if (tk < nt && orow < a.d_out) a.y[(size_t)(q0 + tk) * a.d_out + orow] = out;
    }
    __syncthreads();  // red and the staged rows are reused by the next pass
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

// Down projection and the gated sum in one launch, for a few tokens. A
// block is one 16-row tile of the output for one token; wave w takes the
// token's slots w, w + kDcWaves, ...: it stages the slot's hidden state as
// fp16 hi/lo rows (the down launch's split, h * 2^-E = hi + lo), walks its
// expert's tile on the matrix cores exactly as the down launch does (the
// same steps in the same order, so y_s is the same fp32 value) and leaves
// y_s in LDS; the block then forms out = sum_s gate_s * y_s in slot order,
// the scatter kernel's sum. Each token reads its experts' tiles itself, so
// this serves token counts whose routed experts barely repeat.
constexpr int kDcWaves = 8;

struct DownCombineArgs {
  const float* h;          // [pairs][d_in] fp32 hidden states, sorted pair order
  const int32_t* slot_of;  // [n][k]: row of h for (t, s), or -1
  const uint32_t* idx;     // [n][k] experts
  const float* gate;       // [n][k]
  const uint32_t* wq;      // [E][d_out][d_in*bits/32]
  const uint16_t* s;
  const uint16_t* b;
  void* out;               // [n][d_out]
  int k, n_experts, d_in, d_out;
};

// LDS bytes of one wave's staging (hi and lo rows, zero slots, sums, shifts).
__host__ __device__ constexpr size_t dc_wave_bytes(int G) {
  return (size_t)(2 * (G * kEGroupSlots + 1) + 8) * 16 + (size_t)G * kEMT * 8;
}

template <int BITS, typename OutT>
__global__ __launch_bounds__(64 * kDcWaves) void down_combine_kernel(DownCombineArgs a) {
  using S = MfmaShape<BITS, kEMT>;
  constexpr int RS = 4;  // steps in flight per wave
  extern __shared__ __align__(16) uint4 lds[];
  __shared__ float ys[kMaxK][16];
  __shared__ int valid[kMaxK];
  const int G = a.d_in / 64;  // a multiple of 4 (checked by the launcher)
  const int steps = G / S::kNB;
  const int m_stride = G * kEGroupSlots + 1;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int t = blockIdx.y;
  uint4* xs = lds + wave * (dc_wave_bytes(G) / 16);  // rows 0 (hi) and 1 (lo)
  uint4* zeros = xs + 2 * m_stride;
  float* sums = reinterpret_cast<float*>(zeros + 8);  // [G][kEMT]
  float* mult = sums + G * kEMT;                       // [G][kEMT]
  if (lane < S::kT) zeros[lane] = uint4{0, 0, 0, 0};

  const int n = lane & 15, hq = lane >> 4;  // weight row in the tile; k-octet and row block
  const int row = blockIdx.x * 16 + n;
  const bool row_ok = row < a.d_out;
  const uint32_t row_bytes = (uint32_t)a.d_in * BITS / 8;
  const uint32_t code_base = row_ok ? (uint32_t)row * row_bytes + hq * S::kGroupBytes : kOutOfRange;
  const uint32_t sb_base = row_ok ? ((uint32_t)row * G + hq) * 2 : kOutOfRange;
  // A row n is (block n / 4, row n % 4): rows 0 and 1 hold hi and lo, 2 and
  // 3 read the zero slots.
  const bool a_live = (n >> 2) == hq && (n & 3) < 2;
  const uint4* a_base = a_live ? xs + (n & 3) * m_stride + hq * kEGroupSlots : zeros;
  const uint32_t a_mul = a_live ? 1u : 0u;
  const uint32_t wbytes = (uint32_t)(a.d_out * row_bytes), sbytes = (uint32_t)(a.d_out * G * 2);

  for (int sl = wave; sl < a.k; sl += kDcWaves) {  // wave-uniform
    const int pair = t * a.k + sl;
    const uint32_t e = a.idx[pair];
    const int hrow = a.slot_of[pair];
    const bool use = e < (uint32_t)a.n_experts && hrow >= 0;  // wave-uniform
    if (lane == 0) valid[sl] = use ? 1 : 0;
    if (!use) continue;
    const size_t erow = (size_t)e * a.d_out;
    const __amdgpu_buffer_rsrc_t wr = rsrc(a.wq + erow * (row_bytes / 4), wbytes);
    const __amdgpu_buffer_rsrc_t sr = rsrc(a.s + erow * G, sbytes);
    const __amdgpu_buffer_rsrc_t br = rsrc(a.b + erow * G, sbytes);
    ExpertStep<BITS, false> R[RS];
    auto load = [&](ExpertStep<BITS, false>& Rs, int st) {
      const bool live = st < steps;  // wave-uniform
      const uint32_t co = code_base + (live ? (uint32_t)st * 4 * S::kGroupBytes : kOutOfRange);
      const uint32_t so = sb_base + (live ? (uint32_t)st * 4 * 2 : kOutOfRange);
#pragma unroll
      for (int i = 0; i < S::kWPL; i += 4) {
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(wr, co + 4 * i, 0, 0);
        Rs.w[0][i] = v.x; Rs.w[0][i + 1] = v.y; Rs.w[0][i + 2] = v.z; Rs.w[0][i + 3] = v.w;
      }
      Rs.s[0] = buffer_load_h16(sr, so);
      Rs.b[0] = buffer_load_h16(br, so);
    };
#pragma unroll
    for (int j = 0; j < RS; ++j) load(R[j], j);

    // Stage: item (group, quarter of 16 values); the four lanes of a group
    // agree on its shift (the largest |h| of the group below 2^14).
    __builtin_amdgcn_wave_barrier();  // the previous slot's operand reads come first
    for (int it = lane; it < 4 * G; it += kWave) {
      const int qq = it & 3, g = it >> 2;
      const float* src = a.h + (size_t)hrow * a.d_in + g * 64 + 16 * qq;
      float hv[16];
#pragma unroll
      for (int i = 0; i < 16; i += 4) {
        const float4 v = *reinterpret_cast<const float4*>(src + i);
        hv[i] = v.x; hv[i + 1] = v.y; hv[i + 2] = v.z; hv[i + 3] = v.w;
      }
      float mx = 0.0f, tot = 0.0f;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        mx = fmaxf(mx, fabsf(hv[i]));
        tot += hv[i];
      }
      mx = fmaxf(mx, __shfl_xor(mx, 1, 4));
      mx = fmaxf(mx, __shfl_xor(mx, 2, 4));
      tot += __shfl_xor(tot, 1, 4);
      tot += __shfl_xor(tot, 2, 4);
      const int ex = mx > 0.0f ? max(0, ilogbf(mx) - 13) : 0;
      const float inv = ldexpf(1.0f, -ex);
      uint4* dhi = xs + g * kEGroupSlots + 2 * qq;
      uint4* dlo = dhi + m_stride;
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        f16x8 hi8, lo8;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float hs = hv[8 * q + j] * inv;
          const _Float16 hi = (_Float16)hs;
          hi8[j] = hi;
          lo8[j] = (_Float16)(hs - (float)hi);
        }
        const u32x4 oh = to_slot_order<BITS>(__builtin_bit_cast(u32x4, hi8));
        const u32x4 ol = to_slot_order<BITS>(__builtin_bit_cast(u32x4, lo8));
        dhi[q] = uint4{oh.x, oh.y, oh.z, oh.w};
        dlo[q] = uint4{ol.x, ol.y, ol.z, ol.w};
      }
      if (qq == 0) {  // b * sum(h) rides on the hi row; both rows scale back by 2^E
        const f32x4 sm = {tot, 0.0f, 0.0f, 0.0f};
        const float m2 = ldexpf(1.0f, ex);
        const f32x4 mu = {m2, m2, 1.0f, 1.0f};
        *reinterpret_cast<f32x4*>(sums + g * kEMT) = sm;
        *reinterpret_cast<f32x4*>(mult + g * kEMT) = mu;
      }
    }
    // The rows written above are read below by other lanes of this wave: a
    // wave's LDS operations run in program order, so holding the compiler
    // at this point is enough.
    __builtin_amdgcn_wave_barrier();

    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int jb = 0; jb < steps; jb += RS) {  // wave-uniform
      if (jb > 0) {
#pragma unroll
        for (int j = 0; j < RS; ++j) load(R[j], jb + j);
      }
#pragma unroll
      for (int j = 0; j < RS; ++j) {
        const int st = jb + j;
        if (st < steps) {
          const int g = st * S::kNB + hq;
          const uint4* a_src = a_base + a_mul * (uint32_t)(st * S::kNB * kEGroupSlots);
          const f32x4 sm = *reinterpret_cast<const f32x4*>(sums + g * kEMT);
          const f32x4 mu = *reinterpret_cast<const f32x4*>(mult + g * kEMT);
          f32x4 d = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
          for (int tt = 0; tt < S::kT; ++tt)
            d = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a_src[tt]),
                                                       code_operand<BITS>(R[j].w[0], tt), d, 0, 0,
                                                       0);
          const float sc = h16_to_f32(R[j].s[0]) * 16777216.0f;  // c * 2^-24
          const float bi = h16_to_f32(R[j].b[0]);
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[r] = fmaf(sc * mu[r], d[r], fmaf(bi, sm[r], acc[r]));
        }
      }
    }
    // Merge the four row blocks (other groups, same A rows): y_s = hi + lo.
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      acc[r] += __shfl_xor(acc[r], 16);
      acc[r] += __shfl_xor(acc[r], 32);
    }
    if (lane < 16) ys[sl][n] = acc[0] + acc[1];
  }
  __syncthreads();
  if (threadIdx.x < 16) {
    const int orow = blockIdx.x * 16 + threadIdx.x;
    float v = 0.0f;
    for (int sl = 0; sl < a.k; ++sl)
      if (valid[sl]) v = fmaf(a.gate[t * a.k + sl], ys[sl][threadIdx.x], v);
    if (orow < a.d_out) store_out<OutT>(static_cast<OutT*>(a.out) + (size_t)t * a.d_out + orow, v);
  }
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
    const uint32_t e = idx[(size_t)t * k + s];
    if (e >= (uint32_t)n_experts) continue;  // names no expert: adds nothing (block-uniform)
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

// Matrix cores take the experts at 4 and 8 bits: four groups per step, at
// most 16 steps (d_in <= 4096). Tuning key moe_valu = 1 forces the VALU kernels.
bool mfma_experts(int bits, int d_in) {
  const int G = d_in / 64;
  return (bits == 4 || bits == 8) && G % 4 == 0 && G <= 64 && tuning(kTuneMoeValu, 0) == 0;
}

// a.idx set: the gate/up launch routes in-block (matrix-core path only).
template <int BITS>
int launch_experts(const ExpertArgs& a, int max_active, bool swiglu_f16, bool f32_input,
                   hipStream_t st) {
  using Gm = Geom<BITS>;
  const int G = a.d_in / 64;
  const bool route = a.idx != nullptr;
  if constexpr (BITS == 4 || BITS == 8) {
    if (mfma_experts(BITS, a.d_in)) {
      const int tiles = (a.d_out + 15) / 16;
      // One wave per tile and four tiles per block for short rows (at most
      // 4 steps of 4 groups per tile) and whenever many experts are active
      // (their x staging then spreads over four tiles; 2048-code rows,
      // measured: n = 8 61.2 against 62.0 us, n = 32 114.3 against 118.0);
      // four waves per tile for long rows of a few experts (n = 1: 27.4
      // against 32.2 us). Tuning key moe_kq (1 or 4) overrides for tiling sweeps.
      const int kq = tuning(kTuneMoeKq, (G / 4 <= 4 || max_active >= 32) ? 1 : 4);
      const bool short_rows = kq == 1;
      const dim3 grid(short_rows ? (tiles + 3) / 4 : tiles, max_active);
      // One tile per wave takes the per-wave LDS scale tiles (2560 bytes a
      // wave): gate/up with whole four-step batches, and the fp32-input down
      // projection when its tile is one batch kept over every pass (G <= 16;
      // config 5 n = 32 87.6 -> 86.3 us).
      const bool sbx = short_rows && ((swiglu_f16 && !f32_input && G % 16 == 0) || (f32_input && G <= 16));
      const size_t lds = ((size_t)kEMT * (G * kEGroupSlots + 1) + 8) * 16 + (size_t)G * kEMT * 8 +
                         (sbx ? (size_t)kWaves * 4 * 16 * 40 : 0);
#define KVP_EXPERT(SW, F32, KQ, RT)                                                           \
  hipLaunchKernelGGL((expert_mfma_kernel<BITS, SW, F32, KQ, RT>), grid, dim3(kBlock), lds, st, a)
#define KVP_EXPERT_SBX(RT)                                                                    \
  hipLaunchKernelGGL((expert_mfma_kernel<BITS, true, false, 1, RT, true>), grid, dim3(kBlock), lds, st, a)
      if (route && !(swiglu_f16 && !f32_input))
        return set_error(KVP_INVALID, "kvp_moe: in-block routing is for the gate/up launch");
      if (f32_input) {
        if (sbx) hipLaunchKernelGGL((expert_mfma_kernel<BITS, false, true, 1, false, true>), grid, dim3(kBlock), lds, st, a);
        else if (short_rows) KVP_EXPERT(false, true, 1, false); else KVP_EXPERT(false, true, 4, false);
      } else if (swiglu_f16 && route) {
        if (sbx) KVP_EXPERT_SBX(true);
        else if (short_rows) KVP_EXPERT(true, false, 1, true); else KVP_EXPERT(true, false, 4, true);
      } else if (swiglu_f16) {
        if (sbx) KVP_EXPERT_SBX(false);
        else if (short_rows) KVP_EXPERT(true, false, 1, false); else KVP_EXPERT(true, false, 4, false);
      } else {
        if (short_rows) KVP_EXPERT(false, false, 1, false); else KVP_EXPERT(false, false, 4, false);
      }
#undef KVP_EXPERT
#undef KVP_EXPERT_SBX
      return check_launch("kvp_moe expert gemv (matrix cores)");
    }
  }
  if (route) return set_error(KVP_INVALID, "kvp_moe: in-block routing needs the matrix cores");
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

// Tokens up to which the SwiGLU call fuses the down projection with the
// gated sum (tuning key moe_down_combine overrides): every token then reads
// its own experts' down tiles. Measured on MI355X, config 5 (128 experts,
// top-8, 2048 / 768, 4-bit), whole call with the fused launch against the
// down launch (weights held over its passes, scale tiles) + scatter:
// n = 1 16.5 / 19.0 us, 2 19.2 / 23.4, 4 27.2 / 30.3, 5 36.4 / 37.4,
// 6 37.6 / 39.1, 7 45.3 / 43.8, 8 45.9 / 45.5, 12 64.6 / 59.2 (the repeated
// expert reads then dominate).
constexpr int kDownCombineTokens = 6;

int launch_down_combine(int bits, int out_dtype, const DownCombineArgs& c, int n,
                        hipStream_t st) {
  const int G = c.d_in / 64;
  const size_t lds = (size_t)kDcWaves * dc_wave_bytes(G);
  const dim3 grid((c.d_out + 15) / 16, n);
  const dim3 block(64 * kDcWaves);
#define KVP_DC(B, T) hipLaunchKernelGGL((down_combine_kernel<B, T>), grid, block, lds, st, c)
  if (bits == 4) {
    if (out_dtype == KVP_F16) KVP_DC(4, f16); else KVP_DC(4, float);
  } else {
    if (out_dtype == KVP_F16) KVP_DC(8, f16); else KVP_DC(8, float);
  }
#undef KVP_DC
  return check_launch("kvp_moe down projection + gated sum");
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
  KVP_REQUIRE((long long)n * k <= kPermuteTile, "kvp_moe_permute: n*k=%lld above %d",
              (long long)n * k, kPermuteTile);
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

namespace kvp {
namespace {

// kvp_moe_swiglu and kvp_moe_route_swiglu. With `logits` the routing is
// computed here (into idx / gate): in the gate/up launch itself for a few
// tokens on the in-block path, else by the routing kernel first.
int swiglu_impl(const char* who, const float* logits, const void* x, uint32_t* idx, float* gate,
                const uint32_t* gate_wq, const void* gate_scales, const void* gate_biases,
                const uint32_t* up_wq, const void* up_scales, const void* up_biases,
                const uint32_t* down_wq, const void* down_scales, const void* down_biases,
                void* out, int out_dtype, int n, int k, int n_experts, int d_model, int d_ffn,
                int bits, void* workspace, size_t workspace_bytes, void* stream) {
  KVP_REQUIRE(x && idx && gate && gate_wq && gate_scales && gate_biases && up_wq && up_scales &&
                  up_biases && down_wq && down_scales && down_biases && out,
              "%s: null pointer argument", who);
  KVP_REQUIRE(n >= 1 && k >= 1 && k <= kMaxK && n_experts >= 1 && n_experts <= kMaxExperts,
              "%s: n=%d k=%d n_experts=%d", who, n, k, n_experts);
  KVP_REQUIRE((long long)n * k <= kPermuteTile, "%s: n*k=%lld above %d", who,
              (long long)n * k, kPermuteTile);
  KVP_REQUIRE(out_dtype == KVP_F16 || out_dtype == KVP_F32, "%s: out_dtype=%d", who,
              out_dtype);
  if (int rc = check_expert_dims("kvp_moe_swiglu (gate/up)", d_model, d_ffn, bits)) return rc;
  if (int rc = check_expert_dims("kvp_moe_swiglu (down)", d_ffn, d_model, bits)) return rc;
  const MoeLayout L = layout(n, k, n_experts, d_model, d_ffn);
  KVP_REQUIRE(workspace && workspace_bytes >= L.total,
              "%s: workspace of %zu bytes, %zu needed", who, workspace_bytes, L.total);
  hipStream_t st = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  int32_t* offsets = reinterpret_cast<int32_t*>(ws + L.offsets);
  int32_t* active = reinterpret_cast<int32_t*>(ws + L.active);
  int32_t* slot_of = reinterpret_cast<int32_t*>(ws + L.slot_of);
  int32_t* perm = reinterpret_cast<int32_t*>(ws + L.perm);
  float* h = reinterpret_cast<float*>(ws + L.h);
  float* y = reinterpret_cast<float*>(ws + L.y);
  const int pairs = n * k;
  // A few pairs on the matrix-core path: the gate/up launch builds the
  // permutation in-block (tuning key moe_permute = 1 forces the permute launch).
  const bool route_in_block = pairs <= kFusedPairs && mfma_experts(bits, d_model) &&
                              tuning(kTuneMoePermute, 0) == 0;
  // From logits, up to kRouteTokensInBlock tokens routed by every gate/up
  // block (one per wave); more tokens take the routing kernel first.
  const int epl = (n_experts + kWave - 1) / kWave;
  const bool logits_in_block = logits && route_in_block && n <= kRouteTokensInBlock && epl <= 4;
  if (logits) {
    if (int rc = check_route_args(n, n_experts, k)) return rc;
    if (!logits_in_block)
      if (int rc = launch_route_core(logits, nullptr, nullptr, 0, idx, gate, n, n_experts, k, st))
        return rc;
  }
  if (!route_in_block) {
    hipLaunchKernelGGL(permute_kernel, dim3(1), dim3(1024), 0, st, idx, offsets, perm, active,
                       slot_of, pairs, n_experts);
    if (int rc = check_launch("kvp_moe_swiglu (permute)")) return rc;
  }
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
  if (route_in_block) {
    a.idx = idx;
    a.n_tokens = n;
    if (logits_in_block) {
      a.logits = logits;
      a.epl = epl <= 1 ? 1 : (epl <= 2 ? 2 : 4);
      a.out_idx = idx;
      a.out_gate = gate;
    }
    a.pairs = pairs;
    a.n_experts = n_experts;
    a.t_offsets = offsets;
    a.t_perm = perm;
    a.t_active = active;
    a.t_slot_of = slot_of;
  }
  if (int rc = launch_experts_bits(bits, a, max_active, true, false, st)) return rc;

  // A few tokens: the down projection and the gated sum in one launch.
  const int G_dn = d_ffn / 64;
  const bool dc_fits = (bits == 4 || bits == 8) && mfma_experts(bits, d_ffn) &&
                       (size_t)kDcWaves * dc_wave_bytes(G_dn) <= 64 * 1024;
  const int dc = tuning(kTuneMoeDownCombine, n <= kDownCombineTokens ? 1 : 0);
  if (dc_fits && dc == 1) {
    DownCombineArgs c{};
    c.h = h;
    c.slot_of = slot_of;
    c.idx = idx;
    c.gate = gate;
    c.wq = down_wq;
    c.s = static_cast<const uint16_t*>(down_scales);
    c.b = static_cast<const uint16_t*>(down_biases);
    c.out = out;
    c.k = k;
    c.n_experts = n_experts;
    c.d_in = d_ffn;
    c.d_out = d_model;
    return launch_down_combine(bits, out_dtype, c, n, st);
  }

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

}  // namespace
}  // namespace kvp

extern "C" int kvp_moe_swiglu(const void* x, const uint32_t* idx, const float* gate,
                              const uint32_t* gate_wq, const void* gate_scales,
                              const void* gate_biases, const uint32_t* up_wq,
                              const void* up_scales, const void* up_biases,
                              const uint32_t* down_wq, const void* down_scales,
                              const void* down_biases, void* out, int out_dtype, int n, int k,
                              int n_experts, int d_model, int d_ffn, int bits, void* workspace,
                              size_t workspace_bytes, void* stream) {
  using namespace kvp;
  clear_error();
  return swiglu_impl("kvp_moe_swiglu", nullptr, x, const_cast<uint32_t*>(idx),
                     const_cast<float*>(gate), gate_wq, gate_scales, gate_biases, up_wq,
                     up_scales, up_biases, down_wq, down_scales, down_biases, out, out_dtype, n,
                     k, n_experts, d_model, d_ffn, bits, workspace, workspace_bytes, stream);
}

extern "C" int kvp_moe_route_swiglu(const float* logits, const void* x, uint32_t* idx,
                                    float* gate, const uint32_t* gate_wq,
                                    const void* gate_scales, const void* gate_biases,
                                    const uint32_t* up_wq, const void* up_scales,
                                    const void* up_biases, const uint32_t* down_wq,
                                    const void* down_scales, const void* down_biases, void* out,
                                    int out_dtype, int n, int k, int n_experts, int d_model,
                                    int d_ffn, int bits, void* workspace, size_t workspace_bytes,
                                    void* stream) {
  using namespace kvp;
  clear_error();
  KVP_REQUIRE(logits, "kvp_moe_route_swiglu: null logits");
  return swiglu_impl("kvp_moe_route_swiglu", logits, x, idx, gate, gate_wq, gate_scales,
                     gate_biases, up_wq, up_scales, up_biases, down_wq, down_scales, down_biases,
                     out, out_dtype, n, k, n_experts, d_model, d_ffn, bits, workspace,
                     workspace_bytes, stream);
}
