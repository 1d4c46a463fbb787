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
#include "common.h"

namespace kvp {
namespace {

constexpr int kBlock = 256;
constexpr int kWavesPerBlock = kBlock / kWave;
// LDS budget for staged activations, in 32-bit words (fp16 pairs), per block.
constexpr int kStageWords = 16384;  // 64 KiB: two blocks fit in a CU's 160 KiB

template <int BITS>
struct Geom {
  static constexpr bool kMagic = (BITS == 2 || BITS == 4 || BITS == 8);
  // A unit is what one lane loads per step: 16 bytes, or one 3-bit group.
  static constexpr int kUnitWords = kMagic ? 4 : 6;
  static constexpr int kUnitCodes = kUnitWords * 32 / BITS;  // 64, 64, 32, 16
  static constexpr int kUnitPairs = kUnitCodes / 2;          // staged x words per unit
  static constexpr int kCodesPerWord = 32 / BITS;            // 2/4/8-bit only
  static constexpr int kPairsPerWord = kCodesPerWord / 2;
};

template <int BITS>
__device__ __forceinline__ void load_unit(const uint32_t* p, uint32_t (&w)[Geom<BITS>::kUnitWords]) {
  if constexpr (Geom<BITS>::kUnitWords == 4) {
    u32x4 v = load_stream16(p);
    w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
  } else {
    // 24-byte unit, 8-byte aligned.
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      u32x2 v = load_stream8(p + 2 * i);
      w[2 * i] = v.x;
      w[2 * i + 1] = v.y;
    }
  }
}

// Per-unit dot products d[r][m] = sum_i x[m][i] * q[r][i] over one unit.
//
// Codes are used as fp16 DENORMALS: a masked code field c placed in the low
// mantissa bits of an fp16 half is exactly c * 2^-24 (or c * 16 * 2^-24 when
// the field sits four bits up), so no offset or subtract is needed. Every
// product x * c * 2^-k is exact in fp32 and the fp32 sums are rescaled by an
// exact power of two at the end of the unit. This needs fp16 denormals to be
// honoured by V_DOT2_F32_F16, which is the gfx9 default (MODE f16 denorm on).
//
// 4-bit word (codes n0..n7 at bits 4i): pairs (n0,n4), (16 n1, 16 n5) from
// the word, (n2,n6), (16 n3, 16 n7) from the word shifted by 8: one shift,
// four ANDs and four dot2 per eight codes. The x pairs staged for this word
// are (x0,x4), (x1,x5), (x2,x6), (x3,x7).
template <int BITS, int M, int RW>
__device__ __forceinline__ void unit_dot(const uint32_t (&w)[RW][Geom<BITS>::kUnitWords],
                                         const uint32_t* __restrict__ xu, int m_stride,
                                         float (&d)[RW][M]) {
  using G = Geom<BITS>;
  constexpr float kDenormScale = 16777216.0f;  // 2^24
  if constexpr (BITS == 4) {
    float d1[RW][M], d16[RW][M];
#pragma unroll
    for (int r = 0; r < RW; ++r)
#pragma unroll
      for (int m = 0; m < M; ++m) d1[r][m] = d16[r][m] = 0.0f;
#pragma unroll
    for (int wi = 0; wi < 4; ++wi) {
      uint32_t xp[M][4];
#pragma unroll
      for (int m = 0; m < M; ++m)
#pragma unroll
        for (int i = 0; i < 4; ++i) xp[m][i] = xu[m * m_stride + wi * 4 + i];
#pragma unroll
      for (int r = 0; r < RW; ++r) {
        const uint32_t v = w[r][wi];
        const uint32_t v8 = v >> 8;
        const uint32_t a = v & 0x000F000Fu, b = v & 0x00F000F0u;
        const uint32_t c = v8 & 0x000F000Fu, e = v8 & 0x00F000F0u;
#pragma unroll
        for (int m = 0; m < M; ++m) {
          d1[r][m] = dot2(xp[m][0], a, d1[r][m]);
          d16[r][m] = dot2(xp[m][1], b, d16[r][m]);
          d1[r][m] = dot2(xp[m][2], c, d1[r][m]);
          d16[r][m] = dot2(xp[m][3], e, d16[r][m]);
        }
      }
    }
#pragma unroll
    for (int r = 0; r < RW; ++r)
#pragma unroll
      for (int m = 0; m < M; ++m) d[r][m] = fmaf(d16[r][m], 0.0625f, d1[r][m]) * kDenormScale;
  } else if constexpr (BITS == 8) {
    // Bytes b0..b3: (b0,b2) from the word, (b1,b3) from the word >> 8.
#pragma unroll
    for (int r = 0; r < RW; ++r)
#pragma unroll
      for (int m = 0; m < M; ++m) d[r][m] = 0.0f;
#pragma unroll
    for (int wi = 0; wi < 4; ++wi) {
      uint32_t xp[M][2];
#pragma unroll
      for (int m = 0; m < M; ++m)
#pragma unroll
        for (int i = 0; i < 2; ++i) xp[m][i] = xu[m * m_stride + wi * 2 + i];
#pragma unroll
      for (int r = 0; r < RW; ++r) {
        const uint32_t v = w[r][wi];
        const uint32_t a = v & 0x00FF00FFu, b = (v >> 8) & 0x00FF00FFu;
#pragma unroll
        for (int m = 0; m < M; ++m) {
          d[r][m] = dot2(xp[m][0], a, d[r][m]);
          d[r][m] = dot2(xp[m][1], b, d[r][m]);
        }
      }
    }
#pragma unroll
    for (int r = 0; r < RW; ++r)
#pragma unroll
      for (int m = 0; m < M; ++m) d[r][m] *= kDenormScale;
  } else {
    // 2-bit: pair i of a word = codes (i, i+8), field (w >> 2i) & 0x00030003.
    // 3-bit: pair p = codes (2p, 2p+1), a 6-bit field at bit 6p of the unit.
#pragma unroll
    for (int r = 0; r < RW; ++r)
#pragma unroll
      for (int m = 0; m < M; ++m) d[r][m] = 0.0f;
#pragma unroll
    for (int p = 0; p < G::kUnitPairs; ++p) {
      uint32_t xp[M];
#pragma unroll
      for (int m = 0; m < M; ++m) xp[m] = xu[m * m_stride + p];
#pragma unroll
      for (int r = 0; r < RW; ++r) {
        uint32_t q;
        if constexpr (BITS == 2) {
          q = (w[r][p / 8] >> (2 * (p % 8))) & 0x00030003u;
        } else {
          const int bit = 6 * p;
          const int word = bit >> 5;
          const int sh = bit & 31;
          const uint32_t f = (sh <= 26) ? (w[r][word] >> sh)
                                        : __builtin_amdgcn_alignbit(w[r][word + 1], w[r][word], sh);
          q = (f & 7u) | ((f << 13) & 0x70000u);
        }
#pragma unroll
        for (int m = 0; m < M; ++m) d[r][m] = dot2(xp[m], q, d[r][m]);
      }
    }
#pragma unroll
    for (int r = 0; r < RW; ++r)
#pragma unroll
      for (int m = 0; m < M; ++m) d[r][m] *= kDenormScale;
  }
}

// Stage x[m][code0 : code0 + n_units * kUnitCodes] for all m into LDS in the
// pair order above, and the fp32 activation sum of every unit.
template <int BITS, int M>
__device__ __forceinline__ void stage_x(const f16* __restrict__ x, int d_in, int code0,
                                        int n_units, uint32_t* xs, float* xsum) {
  using G = Geom<BITS>;
  const int pairs_per_m = n_units * G::kUnitPairs;
  if constexpr (G::kMagic) {
    // One "word block" = the kCodesPerWord codes of one weight word.
    constexpr int C = G::kCodesPerWord;
    constexpr int H = G::kPairsPerWord;
    const int blocks_per_m = n_units * G::kUnitWords;
    for (int idx = threadIdx.x; idx < M * blocks_per_m; idx += kBlock) {
      const int m = idx / blocks_per_m;
      const int blk = idx - m * blocks_per_m;
      const uint16_t* src =
          reinterpret_cast<const uint16_t*>(x) + (size_t)m * d_in + code0 + blk * C;
      uint32_t* dst = xs + m * pairs_per_m + blk * H;
#pragma unroll
      for (int i = 0; i < H; ++i) dst[i] = (uint32_t)src[i] | ((uint32_t)src[i + H] << 16);
    }
  } else {
    const int words_per_m = pairs_per_m;
    for (int idx = threadIdx.x; idx < M * words_per_m; idx += kBlock) {
      const int m = idx / words_per_m;
      const int wi = idx - m * words_per_m;
      const uint32_t* src = reinterpret_cast<const uint32_t*>(x + (size_t)m * d_in + code0);
      xs[m * pairs_per_m + wi] = src[wi];
    }
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < M * n_units; idx += kBlock) {
    const int m = idx / n_units;
    const int u = idx - m * n_units;
    const uint32_t* p = xs + m * pairs_per_m + u * G::kUnitPairs;
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < G::kUnitPairs; ++i) s = dot2(p[i], 0x3C003C00u, s);
    xsum[m * n_units + u] = s;
  }
  __syncthreads();
}

template <int BITS, int M, int RW, typename OutT>
__global__ __launch_bounds__(kBlock) void qmv_kernel(const f16* __restrict__ x,
                                                     const uint32_t* __restrict__ wq,
                                                     const uint16_t* __restrict__ scales,
                                                     const uint16_t* __restrict__ biases,
                                                     OutT* __restrict__ out, int d_in, int d_out,
                                                     int chunk_units) {
  using G = Geom<BITS>;
  extern __shared__ uint32_t smem[];
  uint32_t* xs = smem;
  float* xsum = reinterpret_cast<float*>(smem + M * chunk_units * G::kUnitPairs);

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int row0 = (blockIdx.x * kWavesPerBlock + wave) * RW;
  const int units = d_in / G::kUnitCodes;
  const int row_words = units * G::kUnitWords;
  const int groups = d_in / 64;
  constexpr int kUnitsPerGroup = 64 / G::kUnitCodes;  // 4, 2, 1 (3-bit: 1)

  int rows[RW];
#pragma unroll
  for (int r = 0; r < RW; ++r) rows[r] = min(row0 + r, d_out - 1);

  float acc[RW][M];
#pragma unroll
  for (int r = 0; r < RW; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m) acc[r][m] = 0.0f;

  for (int c0 = 0; c0 < units; c0 += chunk_units) {
    const int cu = min(chunk_units, units - c0);
    if (c0 > 0) __syncthreads();  // everyone is done with the previous chunk
    stage_x<BITS, M>(x, d_in, c0 * G::kUnitCodes, cu, xs, xsum);

    for (int ul = lane; ul < cu; ul += kWave) {
      const int u = c0 + ul;
      const int g = u / kUnitsPerGroup;
      uint32_t w[RW][G::kUnitWords];
      float s[RW], b[RW];
#pragma unroll
      for (int r = 0; r < RW; ++r) {
        load_unit<BITS>(wq + (size_t)rows[r] * row_words + u * G::kUnitWords, w[r]);
      }
#pragma unroll
      for (int r = 0; r < RW; ++r) {
        s[r] = f16_bits_to_f32(scales[(size_t)rows[r] * groups + g]);
        b[r] = f16_bits_to_f32(biases[(size_t)rows[r] * groups + g]);
      }
      float d[RW][M];
      unit_dot<BITS, M, RW>(w, xs + ul * G::kUnitPairs, cu * G::kUnitPairs, d);
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const float xs_u = xsum[m * cu + ul];
#pragma unroll
        for (int r = 0; r < RW; ++r) acc[r][m] = fmaf(s[r], d[r][m], fmaf(b[r], xs_u, acc[r][m]));
      }
    }
  }

#pragma unroll
  for (int r = 0; r < RW; ++r) {
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const float v = wave_sum(acc[r][m]);
      if (lane == 0 && row0 + r < d_out) store_out<OutT>(out + (size_t)m * d_out + row0 + r, v);
    }
  }
}

template <int BITS, int M, typename OutT>
int launch_qmv(const void* x, const uint32_t* wq, const void* scales, const void* biases,
               void* out, int d_out, int d_in, hipStream_t stream) {
  using G = Geom<BITS>;
  constexpr int RW = (M <= 2) ? 4 : (M <= 8 ? 2 : 1);
  const int units = d_in / G::kUnitCodes;
  // Chunk = whole 64-unit lane rounds that fit the staging budget (fewer
  // units only when one round does not fit).
  const int words_per_unit = M * G::kUnitPairs + M;  // pairs + one fp32 sum per m
  int chunk_units = kStageWords / words_per_unit;
  if (chunk_units >= kWave) chunk_units = chunk_units / kWave * kWave;
  if (chunk_units > units) chunk_units = units;
  const size_t lds = (size_t)chunk_units * words_per_unit * 4;
  const int rows_per_block = kWavesPerBlock * RW;
  const int blocks = (d_out + rows_per_block - 1) / rows_per_block;
  hipLaunchKernelGGL((qmv_kernel<BITS, M, RW, OutT>), dim3(blocks), dim3(kBlock), lds, stream,
                     static_cast<const f16*>(x), wq, static_cast<const uint16_t*>(scales),
                     static_cast<const uint16_t*>(biases), static_cast<OutT*>(out), d_in, d_out,
                     chunk_units);
  return check_launch("kvp_qmv");
}

template <int BITS, typename OutT>
int dispatch_m(int m, const void* x, const uint32_t* wq, const void* s, const void* b, void* out,
               int d_out, int d_in, hipStream_t st) {
  switch (m) {
#define KVP_M(N) \
  case N: return launch_qmv<BITS, N, OutT>(x, wq, s, b, out, d_out, d_in, st);
    KVP_M(1) KVP_M(2) KVP_M(3) KVP_M(4) KVP_M(5) KVP_M(6) KVP_M(7) KVP_M(8)
    KVP_M(9) KVP_M(10) KVP_M(11) KVP_M(12) KVP_M(13) KVP_M(14) KVP_M(15) KVP_M(16)
#undef KVP_M
  }
  return set_error(KVP_INVALID, "kvp_qmv: m=%d outside 1..16", m);
}

template <typename OutT>
int dispatch_bits(int bits, int m, const void* x, const uint32_t* wq, const void* s,
                  const void* b, void* out, int d_out, int d_in, hipStream_t st) {
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
