// Shared device helpers and host-side status plumbing for libkvpack.
//
// Everything here is gfx950 (CDNA4) code: 64-lane wavefronts, packed fp16
// VALU ops and V_DOT2_F32_F16. No other target is built.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/kvpack.h"

namespace kvp {

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// Host side: status and the thread-local diagnostic behind kvp_last_error().
// ---------------------------------------------------------------------------
int set_error(int status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

#define KVP_REQUIRE(cond, ...)                                  \
  do {                                                          \
    if (!(cond)) return ::kvp::set_error(KVP_INVALID, __VA_ARGS__); \
  } while (0)

// Launch-time failures (hipGetLastError after the launch) become
// KVP_LAUNCH_ERROR with the runtime's own message.
int check_launch(const char* what);

// ---------------------------------------------------------------------------
// Device side
// ---------------------------------------------------------------------------

// fp32 += a.x*b.x + a.y*b.y with both fp16 products exact in fp32
// (V_DOT2_F32_F16). Operands arrive as raw 32-bit words.
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a),
                                __builtin_bit_cast(f16x2, b), c, false);
}

// Two codes sitting in the low bits of each 16-bit half of `v` (already
// masked) become the exact fp16 pair (q_lo, q_hi): OR-ing 0x6400 makes the
// fp16 value 1024 + q, and subtracting 1024 is exact for q < 1024.
__device__ __forceinline__ uint32_t codes_to_f16x2(uint32_t masked) {
  f16x2 v = __builtin_bit_cast(f16x2, masked | 0x64006400u);
  v = v - f16x2{(f16)1024.0f, (f16)1024.0f};
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
  return (float)__builtin_bit_cast(f16, h);
}

// Sum over the 64 lanes of a wavefront; every lane receives the total.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

// Compiler-only barrier: keeps LDS reads of one unrolled step from being
// hoisted above the previous step's math (bounds live registers at wide M).
__device__ __forceinline__ void sched_fence() { asm volatile("" ::: "memory"); }

// Non-temporal 16-byte load for streamed-once data (weights, cache pages):
// it should not evict the activations other waves still need from L2.
__device__ __forceinline__ u32x4 load_stream16(const uint32_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ u32x2 load_stream8(const uint32_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
}

template <typename T>
__device__ __forceinline__ void store_out(T* p, float v);
template <>
__device__ __forceinline__ void store_out<float>(float* p, float v) { *p = v; }
template <>
__device__ __forceinline__ void store_out<f16>(f16* p, float v) { *p = (f16)v; }

}  // namespace kvp
