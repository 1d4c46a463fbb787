// Code-unpack and dot-product core shared by the qmv and KV-decode kernels.
//
// A "unit" is what one lane loads from a quantized row per step: 16 bytes
// (2-, 4- and 8-bit codes) or one 24-byte 3-bit group. unit_dot multiplies a
// unit's codes by M activation vectors held in the weight-word pair order
// (see pair_order), with fp32 accumulation.
#pragma once

#include "common.h"

namespace kvp {

template <int BITS>
struct Geom {
  static constexpr bool kMagic = (BITS == 2 || BITS == 4 || BITS == 8);
  // A unit is what one lane loads per step: 16 bytes, or one 3-bit group.
  static constexpr int kUnitWords = kMagic ? 4 : 6;
  static constexpr int kUnitCodes = kUnitWords * 32 / BITS;  // 64, 64, 32, 16
  static constexpr int kUnitPairs = kUnitCodes / 2;          // staged x words per unit
  static constexpr int kCodesPerWord = 32 / BITS;            // 2/4/8-bit only
  static constexpr int kPairsPerWord = kCodesPerWord / 2;
  // LDS slots of a unit: one per weight word (its pairs contiguous), or one
  // per code pair for 3-bit. Slot-major layout [m][slot][unit][pairs] keeps a
  // wave's 64 lanes on consecutive addresses for every read.
  static constexpr int kSlots = kMagic ? kUnitWords : kUnitPairs;
  static constexpr int kSlotPairs = kMagic ? kPairsPerWord : 1;
};

template <int BITS>
__device__ __forceinline__ void load_unit(const uint32_t* p, uint32_t* w) {
  if constexpr (Geom<BITS>::kUnitWords == 4) {
    u32x4 v = load_stream16(p);
    w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
  } else {
#pragma unroll
    for (int i = 0; i < 3; ++i) {  // 24-byte unit, 8-byte aligned
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
//
// `xu` points at slot 0 of this unit for m = 0; slot j of activation row m
// is at xu + (m * kSlots + j) * slot_stride (in words).
template <int BITS, int M, int RW>
__device__ __forceinline__ void unit_dot(const uint32_t (&w)[RW][Geom<BITS>::kUnitWords],
                                         const uint32_t* __restrict__ xu, int slot_stride,
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
      u32x4 xp[M];
#pragma unroll
      for (int m = 0; m < M; ++m)
        xp[m] = *reinterpret_cast<const u32x4*>(xu + (m * G::kSlots + wi) * slot_stride);
#pragma unroll
      for (int r = 0; r < RW; ++r) {
        const uint32_t v = w[r][wi];
        const uint32_t v8 = v >> 8;
        const uint32_t a = v & 0x000F000Fu, b = v & 0x00F000F0u;
        const uint32_t c = v8 & 0x000F000Fu, e = v8 & 0x00F000F0u;
#pragma unroll
        for (int m = 0; m < M; ++m) {
          d1[r][m] = dot2(xp[m].x, a, d1[r][m]);
          d16[r][m] = dot2(xp[m].y, b, d16[r][m]);
          d1[r][m] = dot2(xp[m].z, c, d1[r][m]);
          d16[r][m] = dot2(xp[m].w, e, d16[r][m]);
        }
      }
      if constexpr (M > 4) sched_fence();
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
      u32x2 xp[M];
#pragma unroll
      for (int m = 0; m < M; ++m)
        xp[m] = *reinterpret_cast<const u32x2*>(xu + (m * G::kSlots + wi) * slot_stride);
#pragma unroll
      for (int r = 0; r < RW; ++r) {
        const uint32_t v = w[r][wi];
        const uint32_t a = v & 0x00FF00FFu, b = (v >> 8) & 0x00FF00FFu;
#pragma unroll
        for (int m = 0; m < M; ++m) {
          d[r][m] = dot2(xp[m].x, a, d[r][m]);
          d[r][m] = dot2(xp[m].y, b, d[r][m]);
        }
      }
      if constexpr (M > 4) sched_fence();
    }
#pragma unroll
    for (int r = 0; r < RW; ++r)
#pragma unroll
      for (int m = 0; m < M; ++m) d[r][m] *= kDenormScale;
  } else if constexpr (BITS == 2) {
    // Pair i of a word = codes (i, i+8), field (w >> 2i) & 0x00030003.
#pragma unroll
    for (int r = 0; r < RW; ++r)
#pragma unroll
      for (int m = 0; m < M; ++m) d[r][m] = 0.0f;
#pragma unroll
    for (int wi = 0; wi < 4; ++wi) {
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        u32x4 xp[M];
#pragma unroll
        for (int m = 0; m < M; ++m)
          xp[m] = *reinterpret_cast<const u32x4*>(xu + (m * G::kSlots + wi) * slot_stride +
                                                  4 * half);
#pragma unroll
        for (int r = 0; r < RW; ++r) {
          const uint32_t v = w[r][wi] >> (8 * half);
#pragma unroll
          for (int m = 0; m < M; ++m) {
            d[r][m] = dot2(xp[m].x, v & 0x00030003u, d[r][m]);
            d[r][m] = dot2(xp[m].y, (v >> 2) & 0x00030003u, d[r][m]);
            d[r][m] = dot2(xp[m].z, (v >> 4) & 0x00030003u, d[r][m]);
            d[r][m] = dot2(xp[m].w, (v >> 6) & 0x00030003u, d[r][m]);
          }
        }
        if constexpr (M > 2) sched_fence();
      }
    }
#pragma unroll
    for (int r = 0; r < RW; ++r)
#pragma unroll
      for (int m = 0; m < M; ++m) d[r][m] *= kDenormScale;
  } else {
    // 3-bit: pair p = codes (2p, 2p+1), a 6-bit field at bit 6p of the unit.
#pragma unroll
    for (int r = 0; r < RW; ++r)
#pragma unroll
      for (int m = 0; m < M; ++m) d[r][m] = 0.0f;
#pragma unroll
    for (int p = 0; p < G::kUnitPairs; ++p) {
      uint32_t xp[M];
#pragma unroll
      for (int m = 0; m < M; ++m) xp[m] = xu[(m * G::kSlots + p) * slot_stride];
#pragma unroll
      for (int r = 0; r < RW; ++r) {
        const int bit = 6 * p;
        const int word = bit >> 5;
        const int sh = bit & 31;
        const uint32_t f = (sh <= 26) ? (w[r][word] >> sh)
                                      : __builtin_amdgcn_alignbit(w[r][word + 1], w[r][word], sh);
        const uint32_t q = (f & 7u) | ((f << 13) & 0x70000u);
#pragma unroll
        for (int m = 0; m < M; ++m) d[r][m] = dot2(xp[m], q, d[r][m]);
      }
      if constexpr (M > 4) sched_fence();
    }
#pragma unroll
    for (int r = 0; r < RW; ++r)
#pragma unroll
      for (int m = 0; m < M; ++m) d[r][m] *= kDenormScale;
  }
}

// Natural pairs (x0,x1),(x2,x3),... of one weight word's codes -> the pair
// order of unit_dot: (x_i, x_{i+c/2}).
template <int BITS>
__device__ __forceinline__ void pair_order(const uint32_t* nat, uint32_t* out) {
  constexpr int H = Geom<BITS>::kPairsPerWord;  // pairs per word
#pragma unroll
  for (int i = 0; i < H; ++i) {
    // low half of pair i = half i, high half = half i + H
    const uint32_t a = nat[i / 2], b = nat[(i + H) / 2];
    const uint32_t lo = (i & 1) ? (a >> 16) : (a & 0xFFFFu);
    const uint32_t hi = ((i + H) & 1) ? (b & 0xFFFF0000u) : (b << 16);
    out[i] = lo | hi;
  }
}

}  // namespace kvp
