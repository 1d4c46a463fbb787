// MLX-affine group quantization on the GPU, writing the kernel layout
// directly: packed code stream + fp16 scale and bias per 64-value group.
//
// Replaces the reference's CPU artefact path: canonical_quantize
// (kernelverify/schemas/quant_contract.py:60-104) followed by pack_codes
// (kernelverify/pack/wide_qmv.py:185-201), and quantize_cache
// (kernelverify/pack/kv_attention.py:270-283) for KV caches. The arithmetic
// is the contract's, in fp32 with IEEE division, in the same order:
//   lo = min(group), hi = max(max(group), 0)
//   step = max((hi - lo) / (2^bits - 1), 1e-7), negated unless |lo| > |hi|
//   edge = lo if |lo| > |hi| else hi; q0 = round_half_away(edge / step)
//   q0 != 0: step = edge / q0, bias = edge; else bias = 0
//   q = min(round_half_away((w - bias) / step), 2^bits - 1)
// with scale and bias rounded to fp16 only when stored. One thread owns one
// group: a group is a whole number of 32-bit code words at every width, so
// no two threads write the same word.
#include <math.h>

#include "common.h"

namespace kvp {
namespace {

__device__ __forceinline__ float round_half_away(float v) {
  return copysignf(floorf(fabsf(v) + 0.5f), v);
}

template <int BITS>
__global__ __launch_bounds__(256) void quantize_kernel(const uint16_t* __restrict__ w,
                                                       uint32_t* __restrict__ wq,
                                                       uint16_t* __restrict__ scales,
                                                       uint16_t* __restrict__ biases,
                                                       long long n_groups) {
  constexpr int kWords = 2 * BITS;  // 64 codes * BITS / 32
  const long long gid = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= n_groups) return;
  const u32x4* src = reinterpret_cast<const u32x4*>(w + gid * 64);
  float v[64];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const u32x4 p = src[i];
    const uint32_t pw[4] = {p.x, p.y, p.z, p.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[8 * i + 2 * j] = f16_bits_to_f32((uint16_t)(pw[j] & 0xFFFFu));
      v[8 * i + 2 * j + 1] = f16_bits_to_f32((uint16_t)(pw[j] >> 16));
    }
  }
  float lo = v[0], hi = v[0];
#pragma unroll
  for (int i = 1; i < 64; ++i) {
    lo = fminf(lo, v[i]);
    hi = fmaxf(hi, v[i]);
  }
  hi = fmaxf(hi, 0.0f);
  const float top = (float)((1 << BITS) - 1);
  float step = fmaxf((hi - lo) / top, 1e-7f);
  const bool low_side = fabsf(lo) > fabsf(hi);
  step = low_side ? step : -step;
  const float edge = low_side ? lo : hi;
  const float q0 = round_half_away(edge / step);
  float bias = 0.0f;
  if (q0 != 0.0f) {
    step = edge / q0;
    bias = edge;
  }
  uint32_t words[kWords];
#pragma unroll
  for (int i = 0; i < kWords; ++i) words[i] = 0u;
#pragma unroll
  for (int i = 0; i < 64; ++i) {
    const float qf = fminf(round_half_away((v[i] - bias) / step), top);
    const uint32_t q = (uint32_t)(int)qf;  // q >= 0 (-0.0 included) by the contract's sides
    const int bit = i * BITS, word = bit >> 5, off = bit & 31;
    words[word] |= q << off;
    if (off + BITS > 32) words[word + 1] |= q >> (32 - off);
  }
  uint32_t* dst = wq + gid * kWords;
#pragma unroll
  for (int i = 0; i < kWords; ++i) dst[i] = words[i];
  scales[gid] = __builtin_bit_cast(uint16_t, (f16)step);
  biases[gid] = __builtin_bit_cast(uint16_t, (f16)bias);
}

}  // namespace
}  // namespace kvp

extern "C" int kvp_quantize_affine(const void* w, int rows, int cols, int bits, uint32_t* w_q,
                                   void* scales, void* biases, void* stream) {
  using namespace kvp;
  clear_error();
  KVP_REQUIRE(w && w_q && scales && biases, "kvp_quantize_affine: null pointer argument");
  KVP_REQUIRE(rows >= 0 && cols >= 64 && cols % 64 == 0,
              "kvp_quantize_affine: rows=%d cols=%d (cols a positive multiple of 64)", rows, cols);
  if (bits != 2 && bits != 3 && bits != 4 && bits != 8)
    return set_error(KVP_UNSUPPORTED, "kvp_quantize_affine: bits=%d not in {2,3,4,8}", bits);
  const long long n_groups = (long long)rows * (cols / 64);
  if (n_groups == 0) return KVP_OK;
  const unsigned blocks = (unsigned)((n_groups + 255) / 256);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const uint16_t* src = static_cast<const uint16_t*>(w);
  uint16_t* s = static_cast<uint16_t*>(scales);
  uint16_t* b = static_cast<uint16_t*>(biases);
  switch (bits) {
    case 2: hipLaunchKernelGGL(quantize_kernel<2>, dim3(blocks), dim3(256), 0, st, src, w_q, s, b, n_groups); break;
    case 3: hipLaunchKernelGGL(quantize_kernel<3>, dim3(blocks), dim3(256), 0, st, src, w_q, s, b, n_groups); break;
    case 4: hipLaunchKernelGGL(quantize_kernel<4>, dim3(blocks), dim3(256), 0, st, src, w_q, s, b, n_groups); break;
    case 8: hipLaunchKernelGGL(quantize_kernel<8>, dim3(blocks), dim3(256), 0, st, src, w_q, s, b, n_groups); break;
  }
  return check_launch("kvp_quantize_affine");
}
