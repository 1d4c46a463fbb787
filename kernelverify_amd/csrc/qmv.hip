// Affine group-quantized matvec for gfx950: out[m, r] = x[m] . dequant(W[r]).
//
// Replaces the reference's `kv_wide_qmv` (kernelverify/pack/wide_qmv.py:65-135).
// Same arithmetic contract: per stretch of codes the fused form
// s * dot(x, q) + b * sum(x) accumulated in fp32, then a cross-lane reduction
// (wide_qmv.py:111-123, :126-134). The tiling is MI355X's own:
//
//   * A 256-thread block is four 64-lane waves; each wave owns RW output rows
//     and walks them together, so one staged activation read feeds RW rows.
//   * Lane l reads 16-byte units l, l+64, l+128, ... of a row: every load
//     instruction is a fully coalesced, non-temporal 1 KiB stream per wave.
//     (3-bit rows use one 24-byte unit per 64-code group instead.)
//   * The activations x (M rows) are staged once per block into LDS,
//     pre-permuted so that each 32-bit weight word's codes line up with fp16
//     activation pairs: with `c` codes per word, pair i is (x[i], x[i+c/2]),
//     which is exactly the pair the word's low and high 16-bit halves expose
//     after one mask. Per-unit activation sums sit beside them in fp32.
//   * Masked code fields are read as exact fp16 denormals, so V_DOT2_F32_F16
//     multiplies them by x with exact products and fp32 accumulation, and an
//     exact power-of-two rescale per unit restores their value. Nothing is
//     narrower than fp32 except the fp16 inputs themselves (contract C1).
//   * Activations larger than the LDS budget are staged in block-uniform
//     chunks of whole 64-unit lane rounds.
#include <stdlib.h>

#include "common.h"
#include "qmv_core.h"

namespace kvp {

bool qmv_mfma_fits(int bits);
int launch_qmv_mfma(int bits, bool f32_out, const void* x, const uint32_t* wq, const void* s,
                    const void* b, void* out, int m, int d_out, int d_in, hipStream_t st);

namespace {

constexpr int kBlock = 256;
constexpr int kWavesPerBlock = kBlock / kWave;
constexpr int kUPL = 2;  // units per lane per pipeline step
// LDS budget for staged activations, in 32-bit words (fp16 pairs), per block.
constexpr int kStageWords = 16384;  // 64 KiB: two blocks fit in a CU's 160 KiB

// Stage x[m][code0 : code0 + n_units * kUnitCodes] for all m into LDS
// (slot-major, pairs in weight-word order) plus the fp32 sum of every unit.
template <int BITS, int M>
__device__ __forceinline__ void stage_x(const f16* __restrict__ x, int d_in, int code0,
                                        int n_units, uint32_t* xs, float* xsum) {
  using G = Geom<BITS>;
  const uint32_t* xw = reinterpret_cast<const uint32_t*>(x);  // fp16 pairs, row m at m*d_in/2
  if constexpr (G::kMagic) {
    // Thread = one weight word's block of C codes; the four blocks of a unit
    // are four consecutive lanes, which also sum the unit's activations.
    constexpr int C = G::kCodesPerWord;
    constexpr int H = G::kPairsPerWord;
    const int total = M * n_units * 4;
    for (int idx = threadIdx.x; idx < total; idx += kBlock) {
      const int wi = idx & 3;
      const int mu = idx >> 2;
      const int m = mu / n_units;
      const int u = mu - m * n_units;
      const uint32_t* src = xw + ((size_t)m * d_in + code0 + (u * 4 + wi) * C) / 2;
      uint32_t hw[C / 2];  // C halves as C/2 words
      if constexpr (C == 8) {
        u32x4 v = *reinterpret_cast<const u32x4*>(src);
        hw[0] = v.x; hw[1] = v.y; hw[2] = v.z; hw[3] = v.w;
      } else if constexpr (C == 4) {
        u32x2 v = *reinterpret_cast<const u32x2*>(src);
        hw[0] = v.x; hw[1] = v.y;
      } else {
        u32x4 v0 = *reinterpret_cast<const u32x4*>(src);
        u32x4 v1 = *reinterpret_cast<const u32x4*>(src + 4);
        hw[0] = v0.x; hw[1] = v0.y; hw[2] = v0.z; hw[3] = v0.w;
        hw[4] = v1.x; hw[5] = v1.y; hw[6] = v1.z; hw[7] = v1.w;
      }
      uint32_t* dst = xs + ((m * G::kSlots + wi) * n_units + u) * H;
      float part = 0.0f;
#pragma unroll
      for (int i = 0; i < H; ++i) {
        const uint32_t lo = (hw[i / 2] >> (16 * (i & 1))) & 0xFFFFu;
        const uint32_t hi = (hw[(i + H) / 2] >> (16 * ((i + H) & 1))) & 0xFFFFu;
        const uint32_t pair = lo | (hi << 16);
        dst[i] = pair;
        part = dot2(pair, 0x3C003C00u, part);
      }
      part += __shfl_xor(part, 1, 4);
      part += __shfl_xor(part, 2, 4);
      if (wi == 0) xsum[m * n_units + u] = part;
    }
  } else {
    // 3-bit: slot p of a unit = natural activation word p; eight threads per
    // unit each move four words.
    const int total = M * n_units * 8;
    for (int idx = threadIdx.x; idx < total; idx += kBlock) {
      const int part_id = idx & 7;
      const int mu = idx >> 3;
      const int m = mu / n_units;
      const int u = mu - m * n_units;
      const uint32_t* src = xw + ((size_t)m * d_in + code0 + u * 64) / 2 + part_id * 4;
      u32x4 v = *reinterpret_cast<const u32x4*>(src);
      const uint32_t vw[4] = {v.x, v.y, v.z, v.w};
      float part = 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        xs[(m * G::kSlots + part_id * 4 + i) * n_units + u] = vw[i];
        part = dot2(vw[i], 0x3C003C00u, part);
      }
      part += __shfl_xor(part, 1, 8);
      part += __shfl_xor(part, 2, 8);
      part += __shfl_xor(part, 4, 8);
      if (part_id == 0) xsum[m * n_units + u] = part;
    }
  }
  __syncthreads();
}

// Early staging for the resident path: every activation fragment a thread
// stages is first loaded into registers, BEFORE the first weight loads are
// issued. Loads complete in order, so the block can stage x and pass its
// barrier as soon as x (an L2 hit) arrives, while the weights are still in
// flight; each wave then computes the moment its own weights land.
template <int BITS, int M>
struct EarlyX {
  using G = Geom<BITS>;
  // A fragment: the codes of one weight word (magic widths) or four
  // activation words (3-bit).
  static constexpr int kFragWords = G::kMagic ? G::kCodesPerWord / 2 : 4;
  static constexpr int kItemsPerUnit = G::kMagic ? 4 : 8;
  static constexpr int kMaxItems = 32 / kFragWords;  // <= 32 VGPRs held per thread

  static __device__ __forceinline__ bool fits(int units) {
    return M * units * kItemsPerUnit <= kMaxItems * kBlock;
  }

  // Straight-line loads (clamped indices, no branches) through a pointer
  // without restrict, so the fence that follows keeps them ahead of the
  // weight loads instead of letting them sink into commit().
  static __device__ __forceinline__ void fetch(const f16* x, int d_in, int units,
                                               uint32_t (&f)[kMaxItems][kFragWords]) {
    const uint32_t* xw = reinterpret_cast<const uint32_t*>(x);
    const int total = M * units * kItemsPerUnit;
    const int n_items = (total + kBlock - 1) / kBlock;  // block-uniform
#pragma unroll
    for (int i = 0; i < kMaxItems; ++i) {
      const int idx = min((int)threadIdx.x + i * kBlock, total - 1);
      if (i < n_items) {
        const int part = idx % kItemsPerUnit;
        const int mu = idx / kItemsPerUnit;
        const int m = mu / units;
        const int u = mu - m * units;
        const uint32_t* src;
        if constexpr (G::kMagic)
          src = xw + ((size_t)m * d_in + (u * 4 + part) * G::kCodesPerWord) / 2;
        else
          src = xw + ((size_t)m * d_in + u * 64) / 2 + part * 4;
        if constexpr (kFragWords == 2) {
          u32x2 v = *reinterpret_cast<const u32x2*>(src);
          f[i][0] = v.x; f[i][1] = v.y;
        } else {
#pragma unroll
          for (int j = 0; j < kFragWords; j += 4) {
            u32x4 v = *reinterpret_cast<const u32x4*>(src + j);
            f[i][j] = v.x; f[i][j + 1] = v.y; f[i][j + 2] = v.z; f[i][j + 3] = v.w;
          }
        }
      }
    }
  }

  static __device__ __forceinline__ void commit(const uint32_t (&f)[kMaxItems][kFragWords],
                                                int units, uint32_t* xs, float* xsum) {
    const int total = M * units * kItemsPerUnit;
#pragma unroll
    for (int i = 0; i < kMaxItems; ++i) {
      const int idx = threadIdx.x + i * kBlock;
      if (idx < total) {  // whole quads / octets are active together
        const int part = idx % kItemsPerUnit;
        const int mu = idx / kItemsPerUnit;
        const int m = mu / units;
        const int u = mu - m * units;
        float sum = 0.0f;
        if constexpr (G::kMagic) {
          constexpr int H = G::kPairsPerWord;
          uint32_t* dst = xs + ((m * G::kSlots + part) * units + u) * H;
#pragma unroll
          for (int k = 0; k < H; ++k) {
            const uint32_t lo = (f[i][k / 2] >> (16 * (k & 1))) & 0xFFFFu;
            const uint32_t hi = (f[i][(k + H) / 2] >> (16 * ((k + H) & 1))) & 0xFFFFu;
            const uint32_t pair = lo | (hi << 16);
            dst[k] = pair;
            sum = dot2(pair, 0x3C003C00u, sum);
          }
          sum += __shfl_xor(sum, 1, 4);
          sum += __shfl_xor(sum, 2, 4);
        } else {
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            xs[(m * G::kSlots + part * 4 + k) * units + u] = f[i][k];
            sum = dot2(f[i][k], 0x3C003C00u, sum);
          }
          sum += __shfl_xor(sum, 1, 8);
          sum += __shfl_xor(sum, 2, 8);
          sum += __shfl_xor(sum, 4, 8);
        }
        if (part == 0) xsum[m * units + u] = sum;
      }
    }
    __syncthreads();
  }
};

// One pipeline step's registers: kUPL units of RW rows, with their scales.
template <int BITS, int RW>
struct StepRegs {
  uint32_t w[kUPL][RW][Geom<BITS>::kUnitWords];
  // The unit's group scale and bias, each in its own register: packed into
  // one, the wave waits for both loads before it can issue the rest of the
  // step's (measured: 9728 x 2560 6.10 -> 5.86 us, 8192 x 4096 6.18 -> 5.91)
  f16 s[kUPL][RW], b[kUPL][RW];
  uint32_t valid;      // bit k: unit k of this step lies inside the row
};



// Position of a wave in its sequence of steps: chunk start c0 (units), chunk
// size cu, step index within the chunk.
struct StepPos {
  int c0, cu, step, steps;
};

template <int BITS, int RW>
__device__ __forceinline__ void load_step(StepRegs<BITS, RW>& R, const StepPos& p,
                                          const uint32_t* __restrict__ wq,
                                          const uint16_t* __restrict__ scales,
                                          const uint16_t* __restrict__ biases,
                                          const int (&rows)[RW], int row_words, int groups,
                                          int lane, int kp, int kw) {
  using G = Geom<BITS>;
  constexpr int kUnitsPerGroup = 64 / G::kUnitCodes;
  R.valid = 0;
#pragma unroll
  for (int k = 0; k < kUPL; ++k) {
    const int ul = ((p.step * kUPL + k) * kw + kp) * kWave + lane;
    R.valid |= (ul < p.cu ? 1u : 0u) << k;
    const int u = p.c0 + min(ul, p.cu - 1);  // clamped: masked through R.valid at use
    const int g = u / kUnitsPerGroup;
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      load_unit<BITS>(wq + (size_t)rows[r] * row_words + (size_t)u * G::kUnitWords, R.w[k][r]);
      R.s[k][r] = __builtin_bit_cast(f16, scales[(size_t)rows[r] * groups + g]);
      R.b[k][r] = __builtin_bit_cast(f16, biases[(size_t)rows[r] * groups + g]);
    }
  }
}

template <int BITS, int M, int RW, typename OutT>
__global__ __launch_bounds__(kBlock) void qmv_kernel(const f16* __restrict__ x,
                                                     const uint32_t* __restrict__ wq,
                                                     const uint16_t* __restrict__ scales,
                                                     const uint16_t* __restrict__ biases,
                                                     OutT* __restrict__ out, int d_in, int d_out,
                                                     int chunk_units, int kw) {
  using G = Geom<BITS>;
  extern __shared__ __align__(16) uint32_t smem[];
  uint32_t* xs = smem;
  float* xsum = reinterpret_cast<float*>(smem + M * chunk_units * G::kUnitPairs);
  __shared__ float red[kWavesPerBlock][RW * M];

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int sets = kWavesPerBlock / kw;  // row sets per block
  const int rs = wave / kw;              // this wave's row set
  const int kp = wave - rs * kw;         // this wave's share of every chunk
  const int row0 = (blockIdx.x * sets + rs) * RW;
  const int units = d_in / G::kUnitCodes;
  const int row_words = units * G::kUnitWords;
  const int groups = d_in / 64;
  const int per_step = kUPL * kw * kWave;  // units of a chunk one step covers

  int rows[RW];
#pragma unroll
  for (int r = 0; r < RW; ++r) rows[r] = min(row0 + r, d_out - 1);

  float acc[RW][M];
#pragma unroll
  for (int r = 0; r < RW; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m) acc[r][m] = 0.0f;

  StepPos pos;
  pos.c0 = 0;
  pos.cu = min(chunk_units, units);
  pos.step = 0;
  pos.steps = (pos.cu + per_step - 1) / per_step;
  StepRegs<BITS, RW> cur, nxt;
  // The first step's weights are requested before the activations are
  // staged, so HBM latency overlaps the staging.
  load_step<BITS, RW>(cur, pos, wq, scales, biases, rows, row_words, groups, lane, kp, kw);
  int staged = -1;
  while (true) {
    if (pos.c0 != staged) {  // block-uniform: every wave walks the same steps
      if (staged >= 0) __syncthreads();
      stage_x<BITS, M>(x, d_in, pos.c0 * G::kUnitCodes, pos.cu, xs, xsum);
      staged = pos.c0;
    }
    StepPos np = pos;
    if (++np.step == np.steps) {
      np.c0 += chunk_units;
      np.cu = min(chunk_units, units - np.c0);
      np.step = 0;
      np.steps = (np.cu + per_step - 1) / per_step;
    }
    const bool more = np.c0 < units;
    if (more) load_step<BITS, RW>(nxt, np, wq, scales, biases, rows, row_words, groups, lane, kp, kw);

#pragma unroll
    for (int k = 0; k < kUPL; ++k) {
      const int ul = min(((pos.step * kUPL + k) * kw + kp) * kWave + lane, pos.cu - 1);
      const bool valid = (cur.valid >> k) & 1u;  // a clamped unit adds exactly nothing
      float d[RW][M];
      unit_dot<BITS, M, RW>(cur.w[k], xs + ul * G::kSlotPairs, pos.cu * G::kSlotPairs, d);
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const float xs_u = xsum[m * pos.cu + ul];
#pragma unroll
        for (int r = 0; r < RW; ++r)
        {
          const float sc = valid ? (float)cur.s[k][r] : 0.0f;
          const float bi = valid ? (float)cur.b[k][r] : 0.0f;
          acc[r][m] = fmaf(sc, d[r][m], fmaf(bi, xs_u, acc[r][m]));
        }
      }
      if constexpr (M > 2) sched_fence();
    }
    if (!more) break;
    cur = nxt;
    pos = np;
  }

#pragma unroll
  for (int r = 0; r < RW; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m) acc[r][m] = wave_sum(acc[r][m]);

  if (kw == 1) {
    if (lane == 0) {
#pragma unroll
      for (int r = 0; r < RW; ++r)
#pragma unroll
        for (int m = 0; m < M; ++m)
          if (row0 + r < d_out) store_out<OutT>(out + (size_t)m * d_out + row0 + r, acc[r][m]);
    }
  } else {
    // Waves sharing a row set hold partial sums over disjoint units; add
    // them in wave order (deterministic) through LDS.
    if (lane == 0) {
#pragma unroll
      for (int r = 0; r < RW; ++r)
#pragma unroll
        for (int m = 0; m < M; ++m) red[wave][r * M + m] = acc[r][m];
    }
    __syncthreads();
    for (int t = threadIdx.x; t < sets * RW * M; t += kBlock) {
      const int set = t / (RW * M);
      const int rm = t - set * RW * M;
      const int r = rm / M, m = rm - r * M;
      float v = 0.0f;
      for (int j = 0; j < kw; ++j) v += red[set * kw + j][rm];
      const int row = (blockIdx.x * sets + set) * RW + r;
      if (row < d_out) store_out<OutT>(out + (size_t)m * d_out + row, v);
    }
  }
}

// ---------------------------------------------------------------------------
// Resident-x path: the whole activation block (M x d_in) is staged once per
// block and every block stays resident, looping over row sets. Each wave
// walks its own sequence of (row set, unit step) pairs with two register
// sets in ping-pong: the loads of step t+1 are in flight while step t
// computes, so HBM streaming and VALU work overlap for the whole kernel
// instead of meeting in one load-then-compute phase.
// ---------------------------------------------------------------------------
template <int BITS, int RW>
__device__ __forceinline__ void load_set_step(StepRegs<BITS, RW>& R, int set, int step,
                                              const uint32_t* __restrict__ wq,
                                              const uint16_t* __restrict__ scales,
                                              const uint16_t* __restrict__ biases, int d_out,
                                              int units, int row_words, int groups, int lane) {
  // Branch-free: a unit past the row end loads a clamped (valid) address and
  // is masked at use through R.valid, so no load waits inside a branch.
  using G = Geom<BITS>;
  constexpr int kUnitsPerGroup = 64 / G::kUnitCodes;
  R.valid = 0;
#pragma unroll
  for (int k = 0; k < kUPL; ++k) {
    const int ul = (step * kUPL + k) * kWave + lane;
    R.valid |= (ul < units ? 1u : 0u) << k;
    const int u = min(ul, units - 1);
    const int g = u / kUnitsPerGroup;
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      const int row = min(set * RW + r, d_out - 1);
      load_unit<BITS>(wq + (size_t)row * row_words + (size_t)u * G::kUnitWords, R.w[k][r]);
      R.s[k][r] = __builtin_bit_cast(f16, scales[(size_t)row * groups + g]);
      R.b[k][r] = __builtin_bit_cast(f16, biases[(size_t)row * groups + g]);
    }
  }
}

template <int BITS, int M, int RW>
__device__ __forceinline__ void compute_step(const StepRegs<BITS, RW>& R, int step, int units,
                                             const uint32_t* xs, const float* xsum, int lane,
                                             float (&acc)[RW][M]) {
  using G = Geom<BITS>;
#pragma unroll
  for (int k = 0; k < kUPL; ++k) {
    const int ul = min((step * kUPL + k) * kWave + lane, units - 1);
    const bool valid = (R.valid >> k) & 1u;  // a clamped unit adds exactly nothing
    float d[RW][M];
    unit_dot<BITS, M, RW>(R.w[k], xs + ul * G::kSlotPairs, units * G::kSlotPairs, d);
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const float xs_u = xsum[m * units + ul];
#pragma unroll
      for (int r = 0; r < RW; ++r) {
        const float sc = valid ? (float)R.s[k][r] : 0.0f;
        const float bi = valid ? (float)R.b[k][r] : 0.0f;
        acc[r][m] = fmaf(sc, d[r][m], fmaf(bi, xs_u, acc[r][m]));
      }
    }
    if constexpr (M > 2) sched_fence();
  }
}

template <int RW, int M, typename OutT>
__device__ __forceinline__ void finish_set(float (&acc)[RW][M], int set, int d_out, int lane,
                                           OutT* __restrict__ out) {
#pragma unroll
  for (int r = 0; r < RW; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const float v = wave_sum(acc[r][m]);
      acc[r][m] = 0.0f;
      if (lane == 0 && set * RW + r < d_out)
        store_out<OutT>(out + (size_t)m * d_out + set * RW + r, v);
    }
}

template <int BITS, int M, int RW, typename OutT>
__global__ __launch_bounds__(kBlock) void qmv_resident_kernel(
    const f16* __restrict__ x, const uint32_t* __restrict__ wq,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ biases,
    OutT* __restrict__ out, int d_in, int d_out) {
  using G = Geom<BITS>;
  extern __shared__ __align__(16) uint32_t smem[];
  const int units = d_in / G::kUnitCodes;
  uint32_t* xs = smem;
  float* xsum = reinterpret_cast<float*>(smem + M * units * G::kUnitPairs);

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = blockIdx.x * kWavesPerBlock + threadIdx.x / kWave;
  const int n_waves = gridDim.x * kWavesPerBlock;
  const int row_words = units * G::kUnitWords;
  const int groups = d_in / 64;
  const int sets = (d_out + RW - 1) / RW;
  const int steps_per_set = (units + kUPL * kWave - 1) / (kUPL * kWave);
  const int my_sets = wave < sets ? (sets - 1 - wave) / n_waves + 1 : 0;
  const int total = my_sets * steps_per_set;

  StepRegs<BITS, RW> A, B;
  using EX = EarlyX<BITS, M>;
  if (EX::fits(units)) {  // block-uniform
    uint32_t frag[EX::kMaxItems][EX::kFragWords];
    EX::fetch(x, d_in, units, frag);
    sched_fence();  // x requests go out before the weight requests
    // Unconditional (a wave without work loads a valid row and ignores it):
    // a branch here would make the compiler drain the x loads first.
    load_set_step<BITS, RW>(A, min(wave, sets - 1), 0, wq, scales, biases, d_out, units,
                            row_words, groups, lane);
    EX::commit(frag, units, xs, xsum);  // ends with a block barrier
  } else {
    if (total > 0)
      load_set_step<BITS, RW>(A, wave, 0, wq, scales, biases, d_out, units, row_words, groups,
                              lane);
    stage_x<BITS, M>(x, d_in, 0, units, xs, xsum);  // ends with a block barrier
  }

  float acc[RW][M];
#pragma unroll
  for (int r = 0; r < RW; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m) acc[r][m] = 0.0f;

  // Step t of this wave: set wave + (t / steps_per_set) * n_waves, unit step
  // t % steps_per_set.
  int set = wave, step = 0;
  for (int t = 0; t < total; t += 2) {
    int set1 = set, step1 = step + 1;
    if (step1 == steps_per_set) { step1 = 0; set1 += n_waves; }
    if (t + 1 < total)
      load_set_step<BITS, RW>(B, set1, step1, wq, scales, biases, d_out, units, row_words,
                              groups, lane);
    compute_step<BITS, M, RW>(A, step, units, xs, xsum, lane, acc);
    if (step == steps_per_set - 1) finish_set<RW, M, OutT>(acc, set, d_out, lane, out);
    if (t + 1 >= total) break;

    int set2 = set1, step2 = step1 + 1;
    if (step2 == steps_per_set) { step2 = 0; set2 += n_waves; }
    if (t + 2 < total)
      load_set_step<BITS, RW>(A, set2, step2, wq, scales, biases, d_out, units, row_words,
                              groups, lane);
    compute_step<BITS, M, RW>(B, step1, units, xs, xsum, lane, acc);
    if (step1 == steps_per_set - 1) finish_set<RW, M, OutT>(acc, set1, d_out, lane, out);
    set = set2;
    step = step2;
  }
}

// ---------------------------------------------------------------------------
// Streaming path (small M): no LDS and no barrier. Every wave loads the
// activation fragments of its own units (L1/L2-resident: all waves read the
// same x) together with its weights, builds the pair order in registers with
// byte permutes, and computes the moment its own loads land. Waves are
// independent, so the hardware overlaps one wave's math with the next
// wave's loads without any block-level synchronisation.
// ---------------------------------------------------------------------------
template <int BITS, int M, int RW>
struct StreamRegs {
  static constexpr int kXWords = Geom<BITS>::kUnitCodes / 2;  // natural fp16 pairs of a unit
  uint32_t w[RW][Geom<BITS>::kUnitWords];
  // Scale and bias of the unit's group, each in its own register so the
  // wave need not wait for them before issuing the rest of a step's loads;
  // 2-bit keeps them packed in one, which holds its streaming kernel at 168
  // VGPRs (three waves per SIMD; one register more drops it to two).
  static constexpr bool kPacked = BITS == 2;
  f16 s[RW], b[RW];  // unpacked
  f16x2 sb[RW];      // packed (.x scale, .y bias)
  __device__ __forceinline__ void set_sb(int r, uint16_t sc, uint16_t bi) {
    if constexpr (kPacked) {
      sb[r] = f16x2{__builtin_bit_cast(f16, sc), __builtin_bit_cast(f16, bi)};
    } else {
      s[r] = __builtin_bit_cast(f16, sc);
      b[r] = __builtin_bit_cast(f16, bi);
    }
  }
  __device__ __forceinline__ float scale(int r) const { return kPacked ? (float)sb[r].x : (float)s[r]; }
  __device__ __forceinline__ float bias(int r) const { return kPacked ? (float)sb[r].y : (float)b[r]; }
  uint32_t x[M][kXWords];
  bool valid;
};

template <int BITS, int M, int RW>
__device__ __forceinline__ void stream_load(StreamRegs<BITS, M, RW>& R, int set, int ul,
                                            const f16* __restrict__ x,
                                            const uint32_t* __restrict__ wq,
                                            const uint16_t* __restrict__ scales,
                                            const uint16_t* __restrict__ biases, int d_in,
                                            int d_out, int units, int row_words, int groups) {
  using G = Geom<BITS>;
  constexpr int kUnitsPerGroup = 64 / G::kUnitCodes;
  constexpr int kXW = StreamRegs<BITS, M, RW>::kXWords;
  R.valid = ul < units;
  const int u = min(ul, units - 1);
  const int g = u / kUnitsPerGroup;
  const uint32_t* xw = reinterpret_cast<const uint32_t*>(x);
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int j = 0; j < kXW; j += 4) {
      u32x4 v = *reinterpret_cast<const u32x4*>(xw + ((size_t)m * d_in + u * G::kUnitCodes) / 2 + j);
      R.x[m][j] = v.x; R.x[m][j + 1] = v.y; R.x[m][j + 2] = v.z; R.x[m][j + 3] = v.w;
    }
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    const int row = min(set * RW + r, d_out - 1);
    load_unit<BITS>(wq + (size_t)row * row_words + (size_t)u * G::kUnitWords, R.w[r]);
    R.set_sb(r, scales[(size_t)row * groups + g], biases[(size_t)row * groups + g]);
  }
}

template <int BITS, int M, int RW>
__device__ __forceinline__ void stream_compute(const StreamRegs<BITS, M, RW>& R,
                                               float (&acc)[RW][M]) {
  using G = Geom<BITS>;
  constexpr int kXW = StreamRegs<BITS, M, RW>::kXWords;
  // Pair-ordered activations of this unit, slot-major like the LDS layout,
  // with slot stride kSlotPairs so unit_dot reads them unchanged.
  uint32_t xp[M * kXW];
  float xs_u[M];
#pragma unroll
  for (int m = 0; m < M; ++m) {
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < kXW; ++j) sum = dot2(R.x[m][j], 0x3C003C00u, sum);
    xs_u[m] = sum;
    if constexpr (G::kMagic) {
      constexpr int H = G::kPairsPerWord;
#pragma unroll
      for (int wi = 0; wi < G::kUnitWords; ++wi)
        pair_order<BITS>(&R.x[m][wi * (G::kCodesPerWord / 2)], &xp[(m * G::kSlots + wi) * H]);
    } else {
#pragma unroll
      for (int j = 0; j < kXW; ++j) xp[m * kXW + j] = R.x[m][j];
    }
  }
  float d[RW][M];
  unit_dot<BITS, M, RW>(R.w, xp, G::kSlotPairs, d);
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      const float sc = R.valid ? R.scale(r) : 0.0f;
      const float bi = R.valid ? R.bias(r) : 0.0f;
      acc[r][m] = fmaf(sc, d[r][m], fmaf(bi, xs_u[m], acc[r][m]));
    }
}

template <int BITS, int M, int RW, typename OutT>
__global__ __launch_bounds__(kBlock) void qmv_stream_kernel(
    const f16* __restrict__ x, const uint32_t* __restrict__ wq,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ biases,
    OutT* __restrict__ out, int d_in, int d_out) {
  using G = Geom<BITS>;
  const int lane = threadIdx.x & (kWave - 1);
  const int set = blockIdx.x * kWavesPerBlock + threadIdx.x / kWave;
  const int units = d_in / G::kUnitCodes;
  const int row_words = units * G::kUnitWords;
  const int groups = d_in / 64;
  const int steps = (units + kWave - 1) / kWave;
  const int sets = (d_out + RW - 1) / RW;
  if (set >= sets) return;  // whole waves; no barrier in this kernel

  float acc[RW][M];
#pragma unroll
  for (int r = 0; r < RW; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m) acc[r][m] = 0.0f;

  StreamRegs<BITS, M, RW> A, B;
  stream_load<BITS, M, RW>(A, set, lane, x, wq, scales, biases, d_in, d_out, units, row_words,
                           groups);
  for (int t = 0; t < steps; t += 2) {
    if (t + 1 < steps)
      stream_load<BITS, M, RW>(B, set, (t + 1) * kWave + lane, x, wq, scales, biases, d_in,
                               d_out, units, row_words, groups);
    stream_compute<BITS, M, RW>(A, acc);
    if (t + 1 >= steps) break;
    if (t + 2 < steps)
      stream_load<BITS, M, RW>(A, set, (t + 2) * kWave + lane, x, wq, scales, biases, d_in,
                               d_out, units, row_words, groups);
    stream_compute<BITS, M, RW>(B, acc);
  }
  finish_set<RW, M, OutT>(acc, set, d_out, lane, out);
}

// ---------------------------------------------------------------------------
// Persistent path (M = 1): a fixed grid of waves, each walking row sets
// wave, wave + n_waves, ... Its lane's activation units stay in registers,
// already in pair order with their sums, for every row it serves; the
// weights stream through a ring of PD row sets in flight; each row's 64-lane
// sum is four DPP steps per 16-lane row and one combination of the rows.
// ---------------------------------------------------------------------------
template <int BITS, int RW, int UPL>
struct PersistSet {
  uint32_t w[UPL][RW][Geom<BITS>::kUnitWords];
  uint16_t s[UPL][RW], b[UPL][RW];  // fp16 bits of the unit's group scale and bias
};

template <int BITS, int RW, int UPL, int PD, typename OutT>
__global__ __launch_bounds__(kBlock) void qmv_persist_kernel(
    const f16* __restrict__ x, const uint32_t* __restrict__ wq,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ biases,
    OutT* __restrict__ out, int d_in, int d_out) {
  using G = Geom<BITS>;
  constexpr int kXW = G::kUnitCodes / 2;  // activation words (natural fp16 pairs) of a unit
  constexpr uint32_t kOOR = 0x80000000u;  // buffer offset that reads as zero
  constexpr int kUnitsPerGroup = 64 / G::kUnitCodes;
  const int lane = threadIdx.x & (kWave - 1);
  const int wg = blockIdx.x * kWavesPerBlock + __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int n_waves = gridDim.x * kWavesPerBlock;
  const int units = d_in / G::kUnitCodes;
  const int groups = d_in / 64;
  const uint32_t row_bytes = (uint32_t)d_in * BITS / 8;
  const int sets = (d_out + RW - 1) / RW;
  auto mk = [](const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes,
                                             0x00020000);
  };
  const auto wr = mk(wq, (uint32_t)((size_t)d_out * row_bytes));
  const auto sr = mk(scales, (uint32_t)((size_t)d_out * groups * 2));
  const auto br = mk(biases, (uint32_t)((size_t)d_out * groups * 2));
  const auto xr = mk(x, (uint32_t)d_in * 2);

  auto load = [&](PersistSet<BITS, RW, UPL>& R, int set) {
    const bool live = set < sets;  // wave-uniform
#pragma unroll
    for (int j = 0; j < UPL; ++j) {
      const int u = lane + kWave * j;
#pragma unroll
      for (int r = 0; r < RW; ++r) {
        const int row = set * RW + r;
        const bool ok = live && row < d_out && u < units;
        const uint32_t co = ok ? (uint32_t)row * row_bytes + (uint32_t)u * 16 : kOOR;
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(wr, co, 0, 0);
        R.w[j][r][0] = v.x; R.w[j][r][1] = v.y; R.w[j][r][2] = v.z; R.w[j][r][3] = v.w;
        const uint32_t so = ok ? ((uint32_t)row * groups + u / kUnitsPerGroup) * 2 : kOOR;
        R.s[j][r] = buffer_load_h16(sr, so);
        R.b[j][r] = buffer_load_h16(br, so);
      }
    }
  };

  // This lane's activation units (requested before the weights, so their
  // wait does not hold for the ring), then pair-ordered with their sums.
  uint32_t nat[UPL][kXW];
#pragma unroll
  for (int j = 0; j < UPL; ++j) {
    const int u = lane + kWave * j;
    const uint32_t xo = u < units ? (uint32_t)u * G::kUnitCodes * 2 : kOOR;
#pragma unroll
    for (int i = 0; i < kXW; i += 4) {
      const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(xr, xo + 4 * i, 0, 0);
      nat[j][i] = v.x; nat[j][i + 1] = v.y; nat[j][i + 2] = v.z; nat[j][i + 3] = v.w;
    }
  }
  PersistSet<BITS, RW, UPL> ring[PD];
#pragma unroll
  for (int p = 0; p < PD; ++p) load(ring[p], wg + n_waves * p);

  uint32_t xp[UPL][kXW];
  float xsum[UPL];
#pragma unroll
  for (int j = 0; j < UPL; ++j) {
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < kXW; ++i) sum = dot2(nat[j][i], 0x3C003C00u, sum);
    xsum[j] = sum;
    constexpr int H = G::kPairsPerWord;
#pragma unroll
    for (int wi = 0; wi < G::kUnitWords; ++wi)
      pair_order<BITS>(&nat[j][wi * (G::kCodesPerWord / 2)], &xp[j][wi * H]);
  }

  for (int base = wg; base < sets; base += PD * n_waves) {  // wave-uniform
#pragma unroll
    for (int p = 0; p < PD; ++p) {
      const int set = base + p * n_waves;
      if (set < sets) {  // wave-uniform
        float acc[RW];
#pragma unroll
        for (int r = 0; r < RW; ++r) acc[r] = 0.0f;
#pragma unroll
        for (int j = 0; j < UPL; ++j) {
          float d[RW][1];
          unit_dot<BITS, 1, RW>(ring[p].w[j], xp[j], G::kSlotPairs, d);
#pragma unroll
          for (int r = 0; r < RW; ++r)
            acc[r] = fmaf(h16_to_f32(ring[p].s[j][r]), d[r][0],
                          fmaf(h16_to_f32(ring[p].b[j][r]), xsum[j], acc[r]));
        }
        load(ring[p], set + PD * n_waves);
#pragma unroll
        for (int r = 0; r < RW; ++r) {
          const int rs = __builtin_bit_cast(int, row16_sum(acc[r]));
          const float v = __builtin_bit_cast(float, __builtin_amdgcn_readlane(rs, 0)) +
                          __builtin_bit_cast(float, __builtin_amdgcn_readlane(rs, 16)) +
                          __builtin_bit_cast(float, __builtin_amdgcn_readlane(rs, 32)) +
                          __builtin_bit_cast(float, __builtin_amdgcn_readlane(rs, 48));
          if (lane == r && set * RW + r < d_out) store_out<OutT>(out + set * RW + r, v);
        }
      }
    }
  }
}

// Largest LDS footprint the resident path accepts: at least two blocks per CU.
constexpr size_t kResidentLdsMax = 64 * 1024;

template <int BITS, int M>
size_t resident_lds_bytes(int d_in) {
  using G = Geom<BITS>;
  const size_t units = d_in / G::kUnitCodes;
  return units * (size_t)(M * G::kUnitPairs + M) * 4;
}

template <int BITS, int M, int RW, typename OutT>
int launch_qmv(const void* x, const uint32_t* wq, const void* scales, const void* biases,
               void* out, int d_out, int d_in, hipStream_t stream) {
  using G = Geom<BITS>;
  const int units = d_in / G::kUnitCodes;
  const size_t res_lds = resident_lds_bytes<BITS, M>(d_in);
  // Path: 1 streaming (no LDS; M <= 2), 2 resident x, 3 chunked x. Auto
  // (measured on MI355X): streaming for M = 1 except tall 4-bit matrices of
  // short rows (below), resident when x fits, else chunked. The tuning
  // key qmv_path overrides for tiling sweeps.
  // Tall 4-bit M = 1 with rows of at most 4096 codes: x resident in LDS at
  // four blocks per CU (an equal share on every CU; 3.5 or 6 per CU lose),
  // two rows per wave. Measured against streaming: 14336 x 4096 8.46 / 8.85
  // us, 9728 x 2560 6.07 / 6.88, 8192 x 4096 6.15 / 6.41; 4096 x 4096 stays
  // streaming (5.07 / 4.47).
  const bool tall = M == 1 && BITS == 4 && d_in <= 4096 && d_out >= 8192;
  int path = tuning(kTuneQmvPath, 0);
  if (path == 0) path = (M == 1 && !tall) ? 1 : (res_lds <= kResidentLdsMax ? 2 : 3);
  if constexpr (M == 1 && G::kMagic) {
    const int upl = (units + kWave - 1) / kWave;
    // its buffer descriptors and offsets are 32-bit, with 2^31 as the
    // out-of-range sentinel: the code array must stay below 2 GiB
    const bool persist_fits = (size_t)d_out * d_in / 8 * BITS < (size_t(1) << 31);
    // Persistent waves pay off when each has many row sets to walk: very
    // tall matrices (measured: 151936 x 2560 at 4 bits, 51.5 against 68.7 us).
    if (persist_fits && (path == 5 || (path == 0 && d_out >= 65536)) && upl <= 4) {
      int dev = 0, cus = 0;
      hipGetDevice(&dev);
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
      const int sets = (d_out + 1) / 2;
      int blocks = cus * tuning(kTuneQmvPerCu, 2);
      blocks = min(blocks, (sets + kWavesPerBlock - 1) / kWavesPerBlock);
#define KVP_PERSIST(U)                                                                         \
  if (upl <= U) {                                                                              \
    hipLaunchKernelGGL((qmv_persist_kernel<BITS, 2, U, 4, OutT>), dim3(blocks), dim3(kBlock), 0, \
                       stream, static_cast<const f16*>(x), wq,                                 \
                       static_cast<const uint16_t*>(scales),                                   \
                       static_cast<const uint16_t*>(biases), static_cast<OutT*>(out), d_in,   \
                       d_out);                                                                 \
    return check_launch("kvp_qmv");                                                           \
  }
      KVP_PERSIST(1) KVP_PERSIST(2) KVP_PERSIST(4)
#undef KVP_PERSIST
    }
  }
  if constexpr (M <= 2) {
    if (path == 1) {
      const int sets = (d_out + RW - 1) / RW;
      const int blocks = (sets + kWavesPerBlock - 1) / kWavesPerBlock;
      hipLaunchKernelGGL((qmv_stream_kernel<BITS, M, RW, OutT>), dim3(blocks), dim3(kBlock), 0,
                         stream, static_cast<const f16*>(x), wq,
                         static_cast<const uint16_t*>(scales),
                         static_cast<const uint16_t*>(biases), static_cast<OutT*>(out), d_in,
                         d_out);
      return check_launch("kvp_qmv");
    }
  }
  if (res_lds <= kResidentLdsMax && path != 3) {
    // Grid = the blocks that fit on the device at once (cached per kernel
    // and footprint), capped by the row sets there are.
    static thread_local int cached_blocks = 0;
    static thread_local size_t cached_lds = 0;
    if (cached_lds != res_lds || cached_blocks == 0) {
      int per_cu = 0, dev = 0, cus = 0;
      hipGetDevice(&dev);
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
      if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
              &per_cu, reinterpret_cast<const void*>(qmv_resident_kernel<BITS, M, RW, OutT>),
              kBlock, res_lds) != hipSuccess || per_cu < 1)
        per_cu = 1;
      cached_blocks = per_cu * cus;
      cached_lds = res_lds;
    }
    const int sets = (d_out + RW - 1) / RW;
    int blocks = min(cached_blocks, (sets + kWavesPerBlock - 1) / kWavesPerBlock);
    if (tall) {
      int dev = 0, cus = 0;
      hipGetDevice(&dev);
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
      blocks = min(blocks, 4 * cus);
    }
    blocks = tuning(kTuneQmvBlocks, blocks);
    if (blocks < 1) return set_error(KVP_INVALID, "kvp_qmv: tuning qmv_blocks=%d", blocks);
    hipLaunchKernelGGL((qmv_resident_kernel<BITS, M, RW, OutT>), dim3(blocks), dim3(kBlock),
                       res_lds, stream, static_cast<const f16*>(x), wq,
                       static_cast<const uint16_t*>(scales), static_cast<const uint16_t*>(biases),
                       static_cast<OutT*>(out), d_in, d_out);
    return check_launch("kvp_qmv");
  }
  // Chunk = whole 64-unit lane rounds that fit the staging budget (fewer
  // units only when one round does not fit).
  const int words_per_unit = M * G::kUnitPairs + M;  // pairs + one fp32 sum per m
  int chunk_units = kStageWords / words_per_unit;
  if (chunk_units >= kWave) chunk_units = chunk_units / kWave * kWave;
  if (chunk_units > units) chunk_units = units;
  // Split each row's units over kw waves when rows alone leave the GPU
  // short of waves (about 4 per SIMD on 256 CUs), but never so far that a
  // wave has no full step of work.
  const int rounds = (units + kWave - 1) / kWave;
  const int row_waves = (d_out + RW - 1) / RW;
  int kw = 1;
  while (kw < kWavesPerBlock && row_waves * kw < 4096 && 2 * kw * kUPL <= rounds) kw *= 2;
  kw = tuning(kTuneQmvKw, kw);
  if (kw != 1 && kw != 2 && kw != 4) return set_error(KVP_INVALID, "kvp_qmv: tuning qmv_kw=%d", kw);
  const size_t lds = (size_t)chunk_units * words_per_unit * 4;
  const int rows_per_block = (kWavesPerBlock / kw) * RW;
  const int blocks = (d_out + rows_per_block - 1) / rows_per_block;
  hipLaunchKernelGGL((qmv_kernel<BITS, M, RW, OutT>), dim3(blocks), dim3(kBlock), lds, stream,
                     static_cast<const f16*>(x), wq, static_cast<const uint16_t*>(scales),
                     static_cast<const uint16_t*>(biases), static_cast<OutT*>(out), d_in, d_out,
                     chunk_units, kw);
  return check_launch("kvp_qmv");
}

// Rows per wave: the VGPR budget of RW * M accumulators. M <= 2 can run
// RW = 2 or 4 (tuning key qmv_rw picks for tiling sweeps); wider M steps down.
template <int BITS, int M, typename OutT>
int launch_qmv_rw(const void* x, const uint32_t* wq, const void* scales, const void* biases,
                  void* out, int d_out, int d_in, hipStream_t stream) {
  if constexpr (M <= 2) {
    // Two rows per wave; four (qmv_rw = 4) halve the activation work per
    // row of the streaming kernel, which measured faster only where the
    // resident kernel now serves (tall 4-bit M = 1 rows of <= 4096 codes).
    if (tuning(kTuneQmvRw, 2) == 4)
      return launch_qmv<BITS, M, 4, OutT>(x, wq, scales, biases, out, d_out, d_in, stream);
    return launch_qmv<BITS, M, 2, OutT>(x, wq, scales, biases, out, d_out, d_in, stream);
  } else {
    constexpr int RW = (M <= 8) ? 2 : 1;
    return launch_qmv<BITS, M, RW, OutT>(x, wq, scales, biases, out, d_out, d_in, stream);
  }
}

// The VALU kernels hold at most 8 rows of x (their accumulators and
// staged activations for more rows spill to scratch on gfx950): M = 9..16
// runs as two calls over rows 0..7 and 8..M-1, each reading the weights.
template <int BITS, typename OutT>
int dispatch_m(int m, const void* x, const uint32_t* wq, const void* s, const void* b, void* out,
               int d_out, int d_in, hipStream_t st) {
  if (m > 8) {
    if (int rc = dispatch_m<BITS, OutT>(8, x, wq, s, b, out, d_out, d_in, st)) return rc;
    return dispatch_m<BITS, OutT>(m - 8, static_cast<const f16*>(x) + (size_t)8 * d_in, wq, s, b,
                                  static_cast<OutT*>(out) + (size_t)8 * d_out, d_out, d_in, st);
  }
  switch (m) {
#define KVP_M(N) \
  case N: return launch_qmv_rw<BITS, N, OutT>(x, wq, s, b, out, d_out, d_in, st);
    KVP_M(1) KVP_M(2) KVP_M(3) KVP_M(4) KVP_M(5) KVP_M(6) KVP_M(7) KVP_M(8)
#undef KVP_M
  }
  return set_error(KVP_INVALID, "kvp_qmv: m=%d outside 1..16", m);
}

template <typename OutT>
int dispatch_bits(int bits, int m, const void* x, const uint32_t* wq, const void* s,
                  const void* b, void* out, int d_out, int d_in, hipStream_t st) {
  // Matrix cores at M >= 2 (qmv_mfma.hip): their cost does not grow with M.
  // At 4 and 8 bits and M = 2 over rows of at most 4096 codes the VALU paths
  // are still as fast or faster (measured on MI355X, 4-bit: 14336 x 4096 11.4
  // against 12.2 us, 4096 x 4096 5.9 against 6.2); at 2 and 3 bits the
  // matrix cores win from M = 2 (3-bit 14336 x 4096: 12.1 against 18.3).
  // qmv_path = 4 forces the matrix cores where they fit, 1..3 the VALU paths.
  const int path = tuning(kTuneQmvPath, 0);
  const bool fits = (size_t)d_out * d_in / 8 * bits < (size_t(1) << 31) &&  // 32-bit offsets
                    qmv_mfma_fits(bits);
  const bool mfma_auto = m >= 3 || (m == 2 && (bits <= 3 || d_in > 4096));
  if (fits && ((path == 0 && mfma_auto) || path == 4))
    return launch_qmv_mfma(bits, sizeof(OutT) == 4, x, wq, s, b, out, m, d_out, d_in, st);
  switch (bits) {
    case 2: return dispatch_m<2, OutT>(m, x, wq, s, b, out, d_out, d_in, st);
    case 3: return dispatch_m<3, OutT>(m, x, wq, s, b, out, d_out, d_in, st);
    case 4: return dispatch_m<4, OutT>(m, x, wq, s, b, out, d_out, d_in, st);
    case 8: return dispatch_m<8, OutT>(m, x, wq, s, b, out, d_out, d_in, st);
  }
  return set_error(KVP_UNSUPPORTED, "kvp_qmv: bits=%d not in {2,3,4,8}", bits);
}

}  // namespace
}  // namespace kvp

extern "C" int kvp_qmv(const void* x, const uint32_t* w_q, const void* scales,
                       const void* biases, void* out, int out_dtype, int m, int d_out, int d_in,
                       int bits, void* stream) {
  using namespace kvp;
  clear_error();
  KVP_REQUIRE(x && w_q && scales && biases && out, "kvp_qmv: null pointer argument");
  KVP_REQUIRE(m >= 1 && m <= 16, "kvp_qmv: m=%d outside 1..16", m);
  KVP_REQUIRE(d_out >= 1, "kvp_qmv: d_out=%d must be positive", d_out);
  KVP_REQUIRE(d_in >= 64 && d_in % 64 == 0, "kvp_qmv: d_in=%d must be a positive multiple of 64",
              d_in);
  KVP_REQUIRE(out_dtype == KVP_F16 || out_dtype == KVP_F32, "kvp_qmv: out_dtype=%d", out_dtype);
  KVP_REQUIRE(bits == 2 || bits == 3 || bits == 4 || bits == 8,
              "kvp_qmv: bits=%d not in {2,3,4,8}", bits);
  // Units must tile a row: 16-byte units need d_in * bits % 128 == 0.
  KVP_REQUIRE(bits == 3 || (d_in * bits) % 128 == 0,
              "kvp_qmv: a %d-bit row of d_in=%d is not a whole number of 16-byte units", bits,
              d_in);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (out_dtype == KVP_F16) return dispatch_bits<f16>(bits, m, x, w_q, scales, biases, out, d_out, d_in, st);
  return dispatch_bits<float>(bits, m, x, w_q, scales, biases, out, d_out, d_in, st);
}
