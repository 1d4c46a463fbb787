// Matrix-core helpers shared by the quantized GEMV kernels (qmv_mfma.hip,
// moe.hip): V_MFMA_F32_16X16X32_F16 with weight codes as exact fp16
// denormals (c * 2^-24) in the B operand and activations in the A operand.
//
// Operand layouts of one 16x16x32 instruction (lane l of a 64-lane wave):
//   A: row l % 16, k-octet l / 16 (8 fp16);  B: k-octet l / 16, column l % 16;
//   D: rows 4 (l / 16) .. + 3, column l % 16 (4 fp32).
// The code masks yield codes in pair order, (c_j, c_j+4) per 4-bit word and
// (c0, c2), (c1, c3) per 8-bit word; activations are staged in that order.
#pragma once

#include <stdlib.h>

#include "common.h"

namespace kvp {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kOutOfRange = 0x80000000u;  // buffer offset that reads as zero

// Raw buffer resource over [p, p + bytes): reads past the end return zero.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

template <int BITS, int MT>
struct MfmaShape {
  static constexpr int kNB = 16 / MT;            // row blocks of A (independent groups per step)
  static constexpr int kOPB = 4 / kNB;           // k-octets per block
  static constexpr int kT = 2 * kNB;             // MFMAs per step
  static constexpr int kCPL = 16 * kNB;          // codes per lane per step
  static constexpr int kWPL = (kCPL * BITS + 31) / 32;  // code words per lane per step
  static constexpr int kShareBytes = kCPL * BITS / 8;   // code bytes per lane per step
  static constexpr int kGroupBytes = 8 * BITS;   // one 64-code group of a row
  static constexpr int kSlotsPerGroup = 9;       // 8 slots of 8 codes + 1 pad slot (banks)
};

// Pair order of one 8-code slot: operand position p holds x[slot_src(p)].
template <int BITS>
__device__ __forceinline__ int slot_src(int p) {
  // 4-bit (w >> 4j) & 0x000F000F -> (c_j, c_j+4); 8-bit (w >> 8j) & 0x00FF00FF
  // over two words -> (c0, c2), (c1, c3), (c4, c6), (c5, c7).
  if constexpr (BITS == 4) return (p & 1) ? (p >> 1) + 4 : (p >> 1);
  else return (p < 4 ? 0 : 4) + ((p & 1) ? 2 : 0) + ((p >> 1) & 1);
}

// The B operand of MFMA t from this lane's code words. Operand order, per
// width (what the activation staging reproduces, group_slot_order below):
//   2-bit: word t/2, element p = code 4 (t%2) + p/2 + 8 (p%2) of the word
//          ((w >> 2j) & 0x00030003 pairs codes j and j + 8);
//   3-bit: codes 8t .. 8t + 7 in natural order, bit-field extracts from the
//          24 bits at bit 24t of the lane's words (a group is 6 words, a
//          lane's quarter of one 48 bits in two words);
//   4-bit: word t, pairs (c_j, c_j+4);  8-bit: words 2t, 2t + 1, pairs
//          (c0, c2), (c1, c3).
template <int BITS>
__device__ __forceinline__ f16x8 code_operand(const uint32_t* w, int t) {
  u32x4 r;
  if constexpr (BITS == 2) {
    const uint32_t v = w[t >> 1];
    const int base = 8 * (t & 1);
    r.x = (v >> base) & 0x00030003u;
    r.y = (v >> (base + 2)) & 0x00030003u;
    r.z = (v >> (base + 4)) & 0x00030003u;
    r.w = (v >> (base + 6)) & 0x00030003u;
  } else if constexpr (BITS == 3) {
    const int bit = 24 * t, wi = bit >> 5, sh = bit & 31;
    const uint32_t v = sh <= 8 ? (w[wi] >> sh) : __builtin_amdgcn_alignbit(w[wi + 1], w[wi], sh);
    r.x = __builtin_amdgcn_ubfe(v, 0, 3) | (__builtin_amdgcn_ubfe(v, 3, 3) << 16);
    r.y = __builtin_amdgcn_ubfe(v, 6, 3) | (__builtin_amdgcn_ubfe(v, 9, 3) << 16);
    r.z = __builtin_amdgcn_ubfe(v, 12, 3) | (__builtin_amdgcn_ubfe(v, 15, 3) << 16);
    r.w = __builtin_amdgcn_ubfe(v, 18, 3) | (__builtin_amdgcn_ubfe(v, 21, 3) << 16);
  } else if constexpr (BITS == 4) {
    const uint32_t v = w[t];
    r.x = v & 0x000F000Fu;
    r.y = (v >> 4) & 0x000F000Fu;
    r.z = (v >> 8) & 0x000F000Fu;
    r.w = (v >> 12) & 0x000F000Fu;
  } else {
    const uint32_t v0 = w[2 * t], v1 = w[2 * t + 1];
    r.x = v0 & 0x00FF00FFu;
    r.y = (v0 >> 8) & 0x00FF00FFu;
    r.z = v1 & 0x00FF00FFu;
    r.w = (v1 >> 8) & 0x00FF00FFu;
  }
  return __builtin_bit_cast(f16x8, r);
}

// Eight fp16 activations in natural order -> the slot's operand order.
template <int BITS>
__device__ __forceinline__ u32x4 to_slot_order(u32x4 natural) {
  const f16x8 nat = __builtin_bit_cast(f16x8, natural);
  f16x8 op;
#pragma unroll
  for (int p = 0; p < 8; ++p) op[p] = nat[slot_src<BITS>(p)];
  return __builtin_bit_cast(u32x4, op);
}

// A 64-code group of activations, eight slots of eight in natural order ->
// the eight operand slots (slot u feeds MFMA u of a lane that holds the whole
// group, or MFMA u - kT share of a lane holding a share of it).
template <int BITS>
__device__ __forceinline__ void group_slot_order(const u32x4 (&nat)[8], u32x4 (&op)[8]) {
  if constexpr (BITS == 2) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const f16x8 lo = __builtin_bit_cast(f16x8, nat[2 * (u >> 1)]);
      const f16x8 hi = __builtin_bit_cast(f16x8, nat[2 * (u >> 1) + 1]);
      f16x8 o;
#pragma unroll
      for (int p = 0; p < 8; ++p) {
        const int c = 4 * (u & 1) + (p >> 1) + 8 * (p & 1);  // code in the 16-code window
        o[p] = c < 8 ? lo[c] : hi[c - 8];
      }
      op[u] = __builtin_bit_cast(u32x4, o);
    }
  } else if constexpr (BITS == 3) {
#pragma unroll
    for (int u = 0; u < 8; ++u) op[u] = nat[u];
  } else {
#pragma unroll
    for (int u = 0; u < 8; ++u) op[u] = to_slot_order<BITS>(nat[u]);
  }
}

// Workgroup barrier for LDS hand-offs only: waits for this wave's LDS
// accesses, not for its weight loads in flight (a fence would drain those).
__device__ __forceinline__ void lds_barrier() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);  // compiler ordering only, no wait
  __builtin_amdgcn_s_waitcnt(0xC07F);       // lgkmcnt(0); vmcnt, expcnt untouched
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

}  // namespace kvp
