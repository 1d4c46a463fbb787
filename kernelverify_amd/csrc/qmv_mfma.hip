// Affine group-quantized matvec on the matrix cores, for M = 2..16 rows of x
// (2-, 3-, 4- and 8-bit codes). Same operator and contract as
// qmv.hip (reference kv_wide_qmv, kernelverify/pack/wide_qmv.py:65-135): per 64-code
// group s * dot(x, q) + b * sum(x), fp32 accumulation, one weight pass.
//
// Why a second kernel: the VALU path spends one V_DOT2 per code pair per row
// of x, so its instruction count grows with M and it turns VALU-bound from
// M = 4 on. Here the products run on V_MFMA_F32_16X16X32_F16, whose cost
// does not depend on M up to 16, and the VALU only unpacks codes and applies
// the per-group scale.
//
// One MFMA is D[16 x 16] = A[16 x 32] * B[32 x 16] with
//   B = codes of 16 weight rows (lane l: row l%16, k-octet l/16), as exact
//       fp16 denormals c * 2^-24 straight from a mask (no conversion);
//   A = activations, BLOCK-DIAGONAL: A row i = (block i / MT, x row i % MT),
//       nonzero only in the k-octets of its block.
// With MT = 4 the four k-octets are four independent blocks, so the four
// lane quarters can each walk a different 64-code group and one MFMA keeps
// their partial dots apart in the four row blocks of D (MT = 8: two blocks,
// MT = 16: one). Every lane of D then holds four x rows of ONE weight row and
// ONE group, so the group scale is one fp32 FMA per D register. A step of a
// wave covers 16 rows x 64 codes per lane quarter block.
//
// x for the step's groups is staged once per block in LDS, pre-permuted into
// the exact operand order the code masks produce (pairs (c_j, c_j+4) for a
// 4-bit word, (c_j, c_j+2) for an 8-bit word), with the fp32 sum of every
// (group, x row) beside it; lanes outside their block read a zero slot.
// Blocks are one 16-row tile; their waves split the tile's steps and merge
// the partial sums through LDS at the end, in a fixed order (deterministic).
#include "mfma_core.h"

namespace kvp {
namespace {

// x chunk budget per block: the whole row of x for M <= 8 at 4096 codes
// (77 KB at M = 8), so those run as one chunk with no hand-off barriers
// (measured, 14336 x 4096 M = 8: 17.0 us against 21.5 with a 64 KB budget);
// clamped to what the device lets a block allocate.
constexpr int kMfmaStageBytes = 96 * 1024;

template <int BITS, int MT>
struct MfmaStep {
  uint32_t w[MfmaShape<BITS, MT>::kWPL];
  uint16_t s, b;  // fp16 bits of this lane's group scale and bias (zero out of range)
};

// Staging of x[m][groups g0 .. g0 + kc) in operand order, with the fp32 sum
// of each (group, m), split in two so the loads can be issued early: a
// thread owns at most one (m, group) item (kc is sized for that), fetches its
// 128 bytes into registers, and commits them to LDS later. Issued before a
// wave's next weight loads, the fetch never waits for them (loads complete
// in order). Groups past the row and rows m >= M are zeros (buffer loads out
// of range read as zero: no branch).
template <int BITS, int MT>
__device__ __forceinline__ void mfma_fetch(__amdgpu_buffer_rsrc_t xr, int M, int d_in, int g0,
                                           int kc, int G, u32x4 (&v)[8]) {
  const int it = threadIdx.x;
  const int m = it / kc, gl = it - m * kc;
  const bool live = it < MT * kc && m < M && g0 + gl < G;
  const uint32_t off = live ? ((uint32_t)m * d_in + (uint32_t)(g0 + gl) * 64) * 2 : kOutOfRange;
#pragma unroll
  for (int q = 0; q < 8; ++q) v[q] = __builtin_amdgcn_raw_buffer_load_b128(xr, off + 16 * q, 0, 0);
}

template <int BITS, int MT>
__device__ __forceinline__ void mfma_commit(const u32x4 (&v)[8], int M, int kc, uint4* xs,
                                            float* xsum, int m_stride_slots) {
  const int it = threadIdx.x;
  if (it >= MT * kc) return;
  const int m = it / kc, gl = it - m * kc;
  float sum = 0.0f;
  uint4* dst = xs + min(m, M - 1) * m_stride_slots + gl * MfmaShape<BITS, MT>::kSlotsPerGroup;
  u32x4 op[8];
  group_slot_order<BITS>(v, op);
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const u32x4 ow = op[q];
#pragma unroll
    for (int j = 0; j < 4; ++j) sum = dot2(ow[j], 0x3C003C00u, sum);
    if (m < M) dst[q] = uint4{ow.x, ow.y, ow.z, ow.w};
  }
  xsum[gl * 16 + m] = sum;
}

// A block is TB row tiles of 16 rows; each tile's steps are split over KQ
// waves. A wave runs its steps through a ring of PD register sets, so PD
// steps of weight loads are in flight while it computes. Every per-step
// address is a per-lane base plus one wave-uniform offset (the buffer
// loads' scalar offset), so a step costs no index arithmetic on the VALU.
template <int BITS, int MT, int TB, int KQ, int PD, typename OutT>
__global__ __launch_bounds__(64 * TB * KQ) void qmv_mfma_kernel(
    const f16* __restrict__ x, const uint32_t* __restrict__ wq,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ biases,
    OutT* __restrict__ out, int M, int d_in, int d_out, int kc) {
  using S = MfmaShape<BITS, MT>;
  constexpr int W = TB * KQ;
  constexpr int kGroupSlots = S::kSlotsPerGroup;
  extern __shared__ __align__(16) uint4 lds[];
  __shared__ float red[W][16][16];
  const int G = d_in / 64;  // a multiple of kNB (checked by the launcher)
  const int m_stride = kc * kGroupSlots + 1;  // slots per x row (odd: spreads banks)
  uint4* xs = lds;
  uint4* zeros = lds + M * m_stride;  // kT zero slots: the A operand of lanes outside their block
  float* xsum = reinterpret_cast<float*>(zeros + S::kT);
  // Scale tiles (MT = 4 and 8, ring depth dividing four). Lane (n, h) needs
  // group base + blk of row n at every step, so a 2-byte load per step and
  // array touched 16 rows for 128 bytes and was issued again each step. Per
  // batch of four steps, lane (n, h) instead loads the kNB groups of step
  // jb + h for both arrays (one 8- or 4-byte load each), the four lanes of a
  // row meet in the wave's tile [array][row][kTP halves] (4 kNB groups + pad:
  // pitches of 40 and 20 bytes put a step's reads of 16 rows on distinct
  // banks), and each step reads its own value. Measured on MI355X (bit-
  // identical outputs): 14336 x 4096 4-bit M = 4 12.5 -> 11.2 us, M = 8
  // 17.0 -> 11.5, 8-bit M = 8 20.8 -> 16.3, 9728 x 2560 M = 8 11.2 -> 8.8.
  constexpr bool kTile = (MT == 4 || MT == 8) && 4 % PD == 0;
  constexpr int kTP = MT == 4 ? 20 : 10;
  uint16_t* tile = reinterpret_cast<uint16_t*>(xsum + kc * 16) +
                   __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) * (2 * 16 * kTP);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tl = wave / KQ, kq = wave - tl * KQ;  // tile in the block, share of its steps
  const int n = lane & 15;   // weight row in the tile (B and D), A row (A)
  const int h = lane >> 4;   // k-octet (A, B) and D row quarter
  const int blk = h / S::kOPB;      // the row block this lane's octet (and D rows) belong to
  const int share = h % S::kOPB;    // this octet's share of its block's group
  const int row = (blockIdx.x * TB + tl) * 16 + n;

  const uint32_t row_bytes = (uint32_t)d_in * BITS / 8;
  const __amdgpu_buffer_rsrc_t wr = rsrc(wq, (uint32_t)((size_t)d_out * row_bytes));
  const __amdgpu_buffer_rsrc_t sr = rsrc(scales, (uint32_t)((size_t)d_out * G * 2));
  const __amdgpu_buffer_rsrc_t br = rsrc(biases, (uint32_t)((size_t)d_out * G * 2));
  const __amdgpu_buffer_rsrc_t xr = rsrc(x, (uint32_t)((size_t)M * d_in * 2));

  // Per-lane bases; a step adds the wave-uniform group of its block 0.
  const bool row_ok = row < d_out;
  const uint32_t code_base =
      row_ok ? (uint32_t)row * row_bytes + blk * S::kGroupBytes + share * S::kShareBytes
             : kOutOfRange;
  const uint32_t sb_base = row_ok ? ((uint32_t)row * G + blk) * 2 : kOutOfRange;
  // A side: this lane's x row and whether its row block matches its octet.
  const int a_m = n % MT;
  const bool a_live = (n / MT == blk) && (a_m < M);
  const uint4* a_base = a_live ? xs + a_m * m_stride + blk * kGroupSlots + share * S::kT : zeros;
  const uint32_t a_mul = a_live ? 1u : 0u;  // lanes outside their block stay on the zero slots
  const float* sum_base = xsum + blk * 16 + (4 * h) % MT;

  const int chunks = (G + kc - 1) / kc;
  // Steps per chunk per wave, padded to whole rings (the padding is dead).
  constexpr int kJB = kTile ? 4 : PD;  // steps per batch (a multiple of the ring depth)
  const int J = ((kc / S::kNB + KQ - 1) / KQ + kJB - 1) / kJB * kJB;
  // Step jj of chunk c: block 0's group is c * kc + (kq + KQ * jj) * kNB.
  auto step_rel = [&](int jj) { return (kq + KQ * jj) * S::kNB; };
  auto load = [&](MfmaStep<BITS, MT>& R, int c, int jj) {
    const int rel = step_rel(jj);
    const int g = c * kc + rel;
    const bool live = c < chunks && rel < kc && g < G;  // wave-uniform
    const uint32_t so = live ? (uint32_t)g : kOutOfRange / S::kGroupBytes;
    const uint32_t co_s = so * S::kGroupBytes, sb_s = live ? (uint32_t)g * 2 : kOutOfRange;
    // The whole offset goes in the range-checked VGPR offset (never the
    // scalar one): a dead step or row lands past the buffer and reads zeros.
    const uint32_t co = code_base + co_s, sbo = sb_base + sb_s;
    if constexpr (S::kShareBytes == 6) {  // 3-bit, a quarter group: 2-byte aligned
      const uint32_t h0 = __builtin_amdgcn_raw_buffer_load_b16(wr, co, 0, 0);
      const uint32_t h1 = __builtin_amdgcn_raw_buffer_load_b16(wr, co + 2, 0, 0);
      R.w[1] = __builtin_amdgcn_raw_buffer_load_b16(wr, co + 4, 0, 0);
      R.w[0] = h0 | (h1 << 16);
    } else if constexpr (S::kWPL == 1) {
      R.w[0] = __builtin_amdgcn_raw_buffer_load_b32(wr, co, 0, 0);
    } else if constexpr (S::kWPL == 2) {
      const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(wr, co, 0, 0);
      R.w[0] = v.x; R.w[1] = v.y;
    } else if constexpr (S::kWPL == 3) {  // 3-bit, half a group: 4-byte aligned
#pragma unroll
      for (int i = 0; i < 3; ++i) R.w[i] = __builtin_amdgcn_raw_buffer_load_b32(wr, co + 4 * i, 0, 0);
    } else if constexpr (S::kWPL == 6) {  // 3-bit, a whole group: 8-byte aligned
#pragma unroll
      for (int i = 0; i < 6; i += 2) {
        const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(wr, co + 4 * i, 0, 0);
        R.w[i] = v.x; R.w[i + 1] = v.y;
      }
    } else {
#pragma unroll
      for (int i = 0; i < S::kWPL; i += 4) {
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(wr, co + 4 * i, 0, 0);
        R.w[i] = v.x; R.w[i + 1] = v.y; R.w[i + 2] = v.z; R.w[i + 3] = v.w;
      }
    }
    if constexpr (!kTile) {
      R.s = buffer_load_h16(sr, sbo);
      R.b = buffer_load_h16(br, sbo);
    }
  };
  // Tile batch (c, jb): lane (n, h) loads the kNB groups of step jb + h of
  // row n (G % kNB == 0 and a step's first group a multiple of kNB keep the
  // loads aligned); step jb + u reads group kNB u + blk of the row.
  u32x2 tsv, tbv;
  auto tile_load = [&](int c, int jb) {
    if constexpr (kTile) {
      const int rel = step_rel(jb + h);
      const int g = c * kc + rel;
      const bool live = c < chunks && rel < kc && g < G;
      const uint32_t o = row_ok && live ? ((uint32_t)row * G + (uint32_t)g) * 2 : kOutOfRange;
      if constexpr (MT == 4) {
        tsv = __builtin_amdgcn_raw_buffer_load_b64(sr, o, 0, 0);
        tbv = __builtin_amdgcn_raw_buffer_load_b64(br, o, 0, 0);
      } else {
        tsv.x = __builtin_amdgcn_raw_buffer_load_b32(sr, o, 0, 0);
        tbv.x = __builtin_amdgcn_raw_buffer_load_b32(br, o, 0, 0);
      }
    }
  };
  auto tile_commit = [&]() {
    if constexpr (kTile) {
      if constexpr (MT == 4) {
        *reinterpret_cast<u32x2*>(tile + n * kTP + 4 * h) = tsv;
        *reinterpret_cast<u32x2*>(tile + (16 + n) * kTP + 4 * h) = tbv;
      } else {
        *reinterpret_cast<uint32_t*>(tile + n * kTP + 2 * h) = tsv.x;
        *reinterpret_cast<uint32_t*>(tile + (16 + n) * kTP + 2 * h) = tbv.x;
      }
    }
  };

  u32x4 xv[8];
  mfma_fetch<BITS, MT>(xr, M, d_in, 0, kc, G, xv);  // x first: the weights must not hold it up
  MfmaStep<BITS, MT> ring[PD];
  tile_load(0, 0);
#pragma unroll
  for (int u = 0; u < PD; ++u) load(ring[u], 0, u);
  if (threadIdx.x < S::kT) zeros[threadIdx.x] = uint4{0, 0, 0, 0};
  mfma_commit<BITS, MT>(xv, M, kc, xs, xsum, m_stride);
  lds_barrier();

  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int c = 0; c < chunks; ++c) {
    const bool next_chunk = c + 1 < chunks;  // block-uniform
    if (next_chunk) mfma_fetch<BITS, MT>(xr, M, d_in, (c + 1) * kc, kc, G, xv);
    const int groups_c = min(kc, G - c * kc);
    for (int jb = 0; jb < J; jb += kJB) {
      if constexpr (kTile) {  // this batch's tile to LDS; the next batch's requested
        tile_commit();
        if (jb + 4 < J) tile_load(c, jb + 4);
        else if (next_chunk) tile_load(c + 1, 0);
      }
#pragma unroll
      for (int uu = 0; uu < kJB; ++uu) {
        const int u = uu % PD;  // ring slot
        const int jj = jb + uu;
        const int rel = step_rel(jj);
        if (rel < groups_c) {  // wave-uniform
          const uint4* a_src = a_base + a_mul * (uint32_t)(rel * kGroupSlots);
          f32x4 d = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
          for (int t = 0; t < S::kT; ++t) {
            d = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a_src[t]),
                                                       code_operand<BITS>(ring[u].w, t), d, 0, 0,
                                                       0);
          }
          // D rows 4h + r of this lane: x rows m = (4h + r) % MT of block blk.
          const f32x4 sums = *reinterpret_cast<const f32x4*>(sum_base + rel * 16);
          float sc, bi;
          if constexpr (kTile) {
            sc = h16_to_f32(tile[n * kTP + S::kNB * uu + blk]) * 16777216.0f;  // c * 2^-24
            bi = h16_to_f32(tile[(16 + n) * kTP + S::kNB * uu + blk]);
          } else {
            sc = h16_to_f32(ring[u].s) * 16777216.0f;
            bi = h16_to_f32(ring[u].b);
          }
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[r] = fmaf(sc, d[r], fmaf(bi, sums[r], acc[r]));
        }
        // The slot refills PD steps ahead, in this chunk or the next.
        const int jn = jj + PD;
        if (jn < J) load(ring[u], c, jn);
        else load(ring[u], c + 1, jn - J);
      }
    }
    if (next_chunk) {
      lds_barrier();  // every wave is done with this chunk
      mfma_commit<BITS, MT>(xv, M, kc, xs, xsum, m_stride);
      lds_barrier();
    }
  }

  // Merge the row blocks of D (they hold the same x rows for other groups).
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    if constexpr (MT == 4) {
      acc[r] += __shfl_xor(acc[r], 16);
      acc[r] += __shfl_xor(acc[r], 32);
    } else if constexpr (MT == 8) {
      acc[r] += __shfl_xor(acc[r], 32);
    }
  }
  if (blk == 0) {
#pragma unroll
    for (int r = 0; r < 4; ++r) red[wave][(4 * h + r) % MT][n] = acc[r];
  }
  __syncthreads();
  for (int t = threadIdx.x; t < TB * M * 16; t += 64 * W) {
    const int tt = t / (M * 16), m = (t >> 4) % M, nn = t & 15;
    const int orow = (blockIdx.x * TB + tt) * 16 + nn;
    float v = 0.0f;
#pragma unroll
    for (int k = 0; k < KQ; ++k) v += red[tt * KQ + k][m][nn];
    if (orow < d_out) store_out<OutT>(out + (size_t)m * d_out + orow, v);
  }
}

// Dynamic LDS a block may take on this device besides `static_bytes`.
inline int stage_budget(int static_bytes) {
  static thread_local int max_block = 0;
  if (max_block == 0) {
    int dev = 0, v = 0;
    hipGetDevice(&dev);
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess ||
        v <= 0)
      v = 64 * 1024;
    max_block = v;
  }
  return min(kMfmaStageBytes, max_block - static_bytes);
}

// Ring depth (steps of weight loads in flight per wave) for code words per
// lane and step `wpl`: about 4 KiB of weights per wave. Deeper rings
// (every step of a chunk in flight) measured slower on MI355X at M = 2 to 8:
// their VGPRs cost co-resident waves (4096 x 4096 M = 2: 8.5 against 6.2 us).
constexpr int ring_depth(int wpl) { return 16 / wpl < 2 ? 2 : 16 / wpl; }

template <int BITS, int MT, int TB, int KQ, int PD, typename OutT>
int launch_pd(const void* x, const uint32_t* wq, const void* s, const void* b, void* out, int m,
              int d_out, int d_in, int kc, size_t lds, hipStream_t stream) {
  const int tiles = (d_out + 15) / 16;
  const int blocks = (tiles + TB - 1) / TB;
  hipLaunchKernelGGL((qmv_mfma_kernel<BITS, MT, TB, KQ, PD, OutT>), dim3(blocks),
                     dim3(64 * TB * KQ), lds, stream, static_cast<const f16*>(x), wq,
                     static_cast<const uint16_t*>(s), static_cast<const uint16_t*>(b),
                     static_cast<OutT*>(out), m, d_in, d_out, kc);
  return check_launch("kvp_qmv (matrix cores)");
}

template <int BITS, int MT, int TB, int KQ, typename OutT>
int launch_mt(const void* x, const uint32_t* wq, const void* s, const void* b, void* out, int m,
              int d_out, int d_in, hipStream_t stream) {
  using S = MfmaShape<BITS, MT>;
  const int G = d_in / 64;
  // Groups per staged chunk: the LDS budget over (x rows x 9 slots + 16 sums),
  // a whole number of steps, at most the row.
  const int per_group = m * S::kSlotsPerGroup * 16 + 16 * 4;
  constexpr int PD = ring_depth(S::kWPL);
  const int tile_bytes =  // the waves' scale tiles (the kernel's kTile forms)
      (MT == 4 || MT == 8) && 4 % PD == 0 ? TB * KQ * 2 * 16 * (MT == 4 ? 40 : 20) : 0;
  const int budget = stage_budget(TB * KQ * 16 * 16 * 4 + tile_bytes);  // + the static merge buffer
  int kc = (budget - (m + S::kT) * 16) / per_group;
  kc = min(kc, 64 * TB * KQ / MT);  // one staging item per thread
  kc = kc / (S::kNB * KQ) * (S::kNB * KQ);
  if (kc < S::kNB * KQ) kc = S::kNB * KQ;
  const int g_pad = (G + S::kNB - 1) / S::kNB * S::kNB;
  if (kc > g_pad) kc = g_pad;
  const size_t lds = ((size_t)m * (kc * S::kSlotsPerGroup + 1) + S::kT) * 16 + (size_t)kc * 16 * 4 +
                     tile_bytes;
  return launch_pd<BITS, MT, TB, KQ, PD, OutT>(
      x, wq, s, b, out, m, d_out, d_in, kc, lds, stream);
}

template <int BITS, int MT, typename OutT>
int launch_tiles(const void* x, const uint32_t* wq, const void* s, const void* b, void* out,
                 int m, int d_out, int d_in, hipStream_t st) {
  // More tiles per block share one x staging (less staging per weight
  // byte) but leave fewer blocks. Measured on MI355X (4-bit, with the scale
  // tiles): four tiles for 768 to 4095 tiles and from 512 at M >= 5
  // (9728x2560 M = 6: 8.34 against 9.95 us on one, M = 5: 8.24 against
  // 9.67; at 2, 3 and 8 bits too), but two from M = 11 at 4
  // and 8 bits with d_in >= 4096 (14336x4096 M = 12: 33.1 against 37.5 us;
  // M = 9-10 and 2-bit M = 12 lose 4-6% there, and 9728x2560 keeps four:
  // 19.3 against 21.8); for 4096 tiles and more two at M = 5-8 and four
  // above (151936x2560 M = 6: 69.8 against 84.2 us on one, M = 5: 68.0
  // against 81.0, at every width; M = 16: 184 against 227 on two); else one
  // tile with eight waves on it to keep loads in flight.
  const int tiles = (d_out + 15) / 16;
  int pick = 1;
  if (tiles >= 4096) {
    if (m >= 5) pick = m > 8 ? 4 : 2;
  } else if (tiles >= 768 || (tiles >= 512 && m >= 5)) {
    pick = (BITS >= 4 && m > 10 && d_in >= 4096) ? 2 : 4;
  }
  const int v = tuning(kTuneQmvMfmaTiles, pick);
  if (v == 4) return launch_mt<BITS, MT, 4, 4, OutT>(x, wq, s, b, out, m, d_out, d_in, st);
  if (v == 2) return launch_mt<BITS, MT, 2, 4, OutT>(x, wq, s, b, out, m, d_out, d_in, st);
  if (tiles >= 512) return launch_mt<BITS, MT, 1, 4, OutT>(x, wq, s, b, out, m, d_out, d_in, st);
  return launch_mt<BITS, MT, 1, 8, OutT>(x, wq, s, b, out, m, d_out, d_in, st);
}

template <int BITS, typename OutT>
int launch_bits(const void* x, const uint32_t* wq, const void* s, const void* b, void* out, int m,
                int d_out, int d_in, hipStream_t st) {
  // A step covers 16 / MT whole groups, so the group count must divide.
  const int G = d_in / 64;
  if (m <= 4 && G % 4 == 0) return launch_tiles<BITS, 4, OutT>(x, wq, s, b, out, m, d_out, d_in, st);
  if (m <= 8 && G % 2 == 0) return launch_tiles<BITS, 8, OutT>(x, wq, s, b, out, m, d_out, d_in, st);
  return launch_tiles<BITS, 16, OutT>(x, wq, s, b, out, m, d_out, d_in, st);
}

}  // namespace

// Whether the matrix-core kernel takes this width.
bool qmv_mfma_fits(int bits) { return bits == 2 || bits == 3 || bits == 4 || bits == 8; }

// Host entry used by kvp_qmv's dispatcher (qmv.hip) at M >= 2.
int launch_qmv_mfma(int bits, bool f32_out, const void* x, const uint32_t* wq, const void* s,
                    const void* b, void* out, int m, int d_out, int d_in, hipStream_t st) {
  switch (bits) {
#define KVP_BITS(B)                                                                           \
  case B:                                                                                     \
    return f32_out ? launch_bits<B, float>(x, wq, s, b, out, m, d_out, d_in, st)             \
                   : launch_bits<B, f16>(x, wq, s, b, out, m, d_out, d_in, st);
    KVP_BITS(2) KVP_BITS(3) KVP_BITS(4) KVP_BITS(8)
#undef KVP_BITS
  }
  return set_error(KVP_UNSUPPORTED, "kvp_qmv (matrix cores): bits=%d", bits);
}

}  // namespace kvp
