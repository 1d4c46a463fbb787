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

// Kernel-selection overrides set through kvp_set_tuning (include/kvpack.h):
// tuning(key, fallback) is the caller's value when one is set, else the
// library's own choice `fallback`. Nothing else (no environment variable)
// changes which kernel a call runs.
enum TuneKey {
  kTuneQmvPath,        // 1 streaming, 2 resident, 3 chunked, 4 matrix cores, 5 persistent
  kTuneQmvPerCu,       // persistent M = 1 kernel: blocks per CU
  kTuneQmvBlocks,      // resident kernel: grid size
  kTuneQmvKw,          // chunked kernel: waves per row (1, 2, 4)
  kTuneQmvRw,          // M <= 2 VALU kernels: rows per wave (2 or 4)
  kTuneQmvMfmaTiles,   // matrix-core qmv: 16-row tiles per block (1, 2, 4)
  kTuneMoeValu,        // 1: MoE experts on the VALU kernels
  kTuneMoeKq,          // matrix-core experts: 1 tile per wave, or 4 waves per tile
  kTuneMoePermute,     // 1: the separate permute launch even where in-block routing applies
  kTuneMoeDownCombine, // SwiGLU down projection: 1 fused with the gated sum, 0 the two launches
  kTuneCount
};
int tuning(TuneKey key, int fallback);

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

// fp16 scales and biases loaded ahead of use (16-bit buffer loads into
// 32-bit registers) are converted by one instruction that reads only the low
// half, written as such: through a 16-bit type the compiler either masks the
// loaded register or packs two of them into one, right after the loads,
// which makes the wave wait for those loads (and every load issued before
// them) long before the values are used.
__device__ __forceinline__ uint16_t buffer_load_h16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
}
__device__ __forceinline__ float h16_to_f32(uint16_t v) {
  float f;
  asm("v_cvt_f32_f16 %0, %1" : "=v"(f) : "v"(v));
  return f;
}

// Sum over the 64 lanes of a wavefront; every lane receives the total.


// DPP lane moves within 16-lane rows (bound_ctrl: lanes without a source
// read zero), and the row-wide reductions built from them: after four steps
// every lane of a row holds the row's result.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(float,
                            __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, true);
}
constexpr int kQuadSwap1 = 0xB1;    // quad_perm [1,0,3,2]
constexpr int kQuadSwap2 = 0x4E;    // quad_perm [2,3,0,1]
constexpr int kHalfMirror = 0x141;  // row_half_mirror
constexpr int kRowMirror = 0x140;   // row_mirror

__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_f<kQuadSwap1>(v));
  v = fmaxf(v, dpp_f<kQuadSwap2>(v));
  v = fmaxf(v, dpp_f<kHalfMirror>(v));
  return fmaxf(v, dpp_f<kRowMirror>(v));
}
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_f<kQuadSwap1>(v);
  v += dpp_f<kQuadSwap2>(v);
  v += dpp_f<kHalfMirror>(v);
  return v + dpp_f<kRowMirror>(v);
}
__device__ __forceinline__ int row16_max_i(int v) {
  v = max(v, dpp_i<kQuadSwap1>(v));
  v = max(v, dpp_i<kQuadSwap2>(v));
  v = max(v, dpp_i<kHalfMirror>(v));
  return max(v, dpp_i<kRowMirror>(v));
}

// Max over the 64 lanes, the same value in every lane (as wave_sum).
__device__ __forceinline__ float wave_max(float v) {
  const int r = __builtin_bit_cast(int, row16_max(v));
  return fmaxf(fmaxf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(r, 0)),
                     __builtin_bit_cast(float, __builtin_amdgcn_readlane(r, 16))),
               fmaxf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(r, 32)),
                     __builtin_bit_cast(float, __builtin_amdgcn_readlane(r, 48))));
}

// Sum over the 64 lanes, the same value in every lane: DPP steps within each
// 16-lane row, then the four row sums read as scalars.
__device__ __forceinline__ float wave_sum(float v) {
  const int r = __builtin_bit_cast(int, row16_sum(v));
  return (__builtin_bit_cast(float, __builtin_amdgcn_readlane(r, 0)) +
          __builtin_bit_cast(float, __builtin_amdgcn_readlane(r, 16))) +
         (__builtin_bit_cast(float, __builtin_amdgcn_readlane(r, 32)) +
          __builtin_bit_cast(float, __builtin_amdgcn_readlane(r, 48)));
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
