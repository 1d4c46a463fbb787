// Roofline probe kernels: the machine ceilings the pack is scored against.
//
// Re-targets the reference's Metal probe (bench/metal/roofline_probe.mm:35-144:
// stream read, stream copy, fp32 / fp16 FMA peaks; selected by
// bench/roofline.py:95-138) to gfx950, with the shapes of the pack's own
// work as sweep parameters instead of one fixed launch:
//
//   probe_read_tiled_kernel  a block reads whole tiles of blockDim x UNROLL
//                            16-byte units (every lane's UNROLL loads are
//                            issued before any is used), tiles taken
//                            grid-strided or as one contiguous range per
//                            block; loads plain, non-temporal or buffer.
//   probe_fma_kernel         eight independent fp32 FMA chains per lane.
//   probe_dot2_kernel        eight independent V_DOT2_F32_F16 chains.
//   probe_mfma_kernel        four independent V_MFMA_F32_16X16X32_F16 chains.
//
// Every kernel ends by storing one value per block, so no load or chain can
// be removed; all accesses stay inside [src, src + n_bytes).
#include "common.h"
#include "mfma_core.h"

namespace kvp {
namespace {

enum { kLoadPlain = 0, kLoadNonTemporal = 1, kLoadBuffer = 2 };

template <int KIND>
__device__ __forceinline__ u32x4 probe_load(const u32x4* base, size_t i) {
  if constexpr (KIND == kLoadNonTemporal) return __builtin_nontemporal_load(base + i);
  else return base[i];
}

__device__ __forceinline__ uint32_t fold(u32x4 v) { return v.x ^ v.y ^ v.z ^ v.w; }

template <int UNROLL, int KIND>
__global__ __launch_bounds__(1024) void probe_read_tiled_kernel(const u32x4* __restrict__ src,
                                                                size_t n16, int contiguous,
                                                                float* __restrict__ sink) {
  const size_t tile = (size_t)blockDim.x * UNROLL;  // 16-byte units per tile
  const size_t n_tiles = n16 / tile;
  size_t t0 = blockIdx.x, t1 = n_tiles, dt = gridDim.x;
  if (contiguous) {  // block b: tiles [b * per, (b + 1) * per)
    const size_t per = (n_tiles + gridDim.x - 1) / gridDim.x;
    t0 = (size_t)blockIdx.x * per;
    t1 = t0 + per < n_tiles ? t0 + per : n_tiles;
    dt = 1;
  }
  uint32_t acc = 0;
  for (size_t t = t0; t < t1; t += dt) {
    u32x4 v[UNROLL];
    if constexpr (KIND == kLoadBuffer) {
      // one descriptor per tile: offsets stay far below the 32-bit range
      const __amdgpu_buffer_rsrc_t r = rsrc(src + t * tile, (uint32_t)(tile * 16));
#pragma unroll
      for (int u = 0; u < UNROLL; ++u)
        v[u] = __builtin_amdgcn_raw_buffer_load_b128(r, (threadIdx.x + u * blockDim.x) * 16, 0, 0);
    } else {
      const u32x4* p = src + t * tile + threadIdx.x;
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) v[u] = probe_load<KIND>(p, (size_t)u * blockDim.x);
    }
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) acc ^= fold(v[u]);
  }
  // the ragged end past the last whole tile
  for (size_t i = n_tiles * tile + (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16;
       i += (size_t)gridDim.x * blockDim.x)
    acc ^= fold(src[i]);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) acc ^= (uint32_t)__shfl_xor((int)acc, off, kWave);
  if (threadIdx.x == 0) sink[blockIdx.x] = (float)(acc & 0xFFFF);
}

constexpr int kChains = 8;

__global__ __launch_bounds__(256) void probe_fma_kernel(int iters, float seed,
                                                        float* __restrict__ sink) {
  float a[kChains];
#pragma unroll
  for (int c = 0; c < kChains; ++c) a[c] = seed + 1e-3f * (float)(threadIdx.x + c);
  const float m = 0.999f + 1e-9f * seed, k = 1e-4f * seed;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int c = 0; c < kChains; ++c) a[c] = fmaf(a[c], m, k);
  }
  float s = 0.0f;
#pragma unroll
  for (int c = 0; c < kChains; ++c) s += a[c];
  if (s == 12345.678f || threadIdx.x == 0) sink[blockIdx.x] = s;
}

__global__ __launch_bounds__(256) void probe_dot2_kernel(int iters, float seed,
                                                         float* __restrict__ sink) {
  const f16 h = (f16)(0.5f + 1e-3f * seed);
  const uint32_t x = __builtin_bit_cast(uint32_t, f16x2{h, (f16)(-1.0f) * h});
  const uint32_t y = __builtin_bit_cast(uint32_t, f16x2{(f16)(0.25f), (f16)(0.25f)});
  float a[kChains];
#pragma unroll
  for (int c = 0; c < kChains; ++c) a[c] = seed + (float)(threadIdx.x + c);
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int c = 0; c < kChains; ++c) a[c] = dot2(x, y, a[c]);
  }
  float s = 0.0f;
#pragma unroll
  for (int c = 0; c < kChains; ++c) s += a[c];
  if (s == 12345.678f || threadIdx.x == 0) sink[blockIdx.x] = s;
}

constexpr int kMfmaChains = 4;

__global__ __launch_bounds__(256) void probe_mfma_kernel(int iters, float seed,
                                                         float* __restrict__ sink) {
  f16x8 av, bv;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    av[i] = (f16)(1e-3f * (float)((threadIdx.x + i) & 7) * seed);
    bv[i] = (f16)(1e-3f * (float)((threadIdx.x * 3 + i) & 7));
  }
  f32x4 acc[kMfmaChains];
#pragma unroll
  for (int c = 0; c < kMfmaChains; ++c) acc[c] = f32x4{seed, 0.0f, 0.0f, (float)c};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int c = 0; c < kMfmaChains; ++c)
      acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, acc[c], 0, 0, 0);
  }
  float s = 0.0f;
#pragma unroll
  for (int c = 0; c < kMfmaChains; ++c) s += acc[c][0] + acc[c][1] + acc[c][2] + acc[c][3];
  if (s == 12345.678f || threadIdx.x == 0) sink[blockIdx.x] = s;
}

template <int KIND>
int launch_read(int unroll, dim3 grid, dim3 block, hipStream_t st, const u32x4* src, size_t n16,
                int contiguous, float* sink) {
  switch (unroll) {
    case 1: hipLaunchKernelGGL((probe_read_tiled_kernel<1, KIND>), grid, block, 0, st, src, n16, contiguous, sink); break;
    case 2: hipLaunchKernelGGL((probe_read_tiled_kernel<2, KIND>), grid, block, 0, st, src, n16, contiguous, sink); break;
    case 4: hipLaunchKernelGGL((probe_read_tiled_kernel<4, KIND>), grid, block, 0, st, src, n16, contiguous, sink); break;
    case 8: hipLaunchKernelGGL((probe_read_tiled_kernel<8, KIND>), grid, block, 0, st, src, n16, contiguous, sink); break;
    default: hipLaunchKernelGGL((probe_read_tiled_kernel<16, KIND>), grid, block, 0, st, src, n16, contiguous, sink); break;
  }
  return check_launch("kvp_probe_read_tiled");
}

}  // namespace
}  // namespace kvp

extern "C" int kvp_probe_read_tiled(const void* src, size_t n_bytes, float* sink, int blocks,
                                    int threads, int unroll, int flags, void* stream) {
  using namespace kvp;
  clear_error();
  KVP_REQUIRE(src && sink, "kvp_probe_read_tiled: null pointer");
  KVP_REQUIRE(n_bytes % 16 == 0 && n_bytes > 0, "kvp_probe_read_tiled: n_bytes %% 16");
  KVP_REQUIRE(blocks > 0, "kvp_probe_read_tiled: blocks=%d", blocks);
  KVP_REQUIRE(threads == 64 || threads == 128 || threads == 256 || threads == 512 ||
                  threads == 1024,
              "kvp_probe_read_tiled: threads=%d", threads);
  KVP_REQUIRE(unroll == 1 || unroll == 2 || unroll == 4 || unroll == 8 || unroll == 16,
              "kvp_probe_read_tiled: unroll=%d", unroll);
  const int kind = flags & 3;
  KVP_REQUIRE(kind <= kLoadBuffer, "kvp_probe_read_tiled: flags=%d", flags);
  const int contiguous = (flags >> 2) & 1;
  const auto* s = static_cast<const u32x4*>(src);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const size_t n16 = n_bytes / 16;
  if (kind == kLoadPlain) return launch_read<kLoadPlain>(unroll, blocks, threads, st, s, n16, contiguous, sink);
  if (kind == kLoadNonTemporal) return launch_read<kLoadNonTemporal>(unroll, blocks, threads, st, s, n16, contiguous, sink);
  return launch_read<kLoadBuffer>(unroll, blocks, threads, st, s, n16, contiguous, sink);
}

extern "C" double kvp_probe_compute_flops(int kind, int blocks, int iters) {
  // flops per lane per iteration: FMA 2, dot2 4 (two fused products);
  // per wave per iteration for the matrix cores: 16 x 16 x 32 x 2 each.
  const double lanes = (double)blocks * 256.0, waves = (double)blocks * 4.0;
  switch (kind) {
    case 0: return lanes * iters * kvp::kChains * 2.0;
    case 1: return lanes * iters * kvp::kChains * 4.0;
    case 2: return waves * iters * kvp::kMfmaChains * 16.0 * 16.0 * 32.0 * 2.0;
  }
  return 0.0;
}

extern "C" int kvp_probe_compute(int kind, int blocks, int iters, float* sink, void* stream) {
  using namespace kvp;
  clear_error();
  KVP_REQUIRE(sink, "kvp_probe_compute: null sink");
  KVP_REQUIRE(blocks > 0 && iters > 0, "kvp_probe_compute: blocks=%d iters=%d", blocks, iters);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const float seed = 1.0f;
  switch (kind) {
    case 0: hipLaunchKernelGGL(probe_fma_kernel, dim3(blocks), dim3(256), 0, st, iters, seed, sink); break;
    case 1: hipLaunchKernelGGL(probe_dot2_kernel, dim3(blocks), dim3(256), 0, st, iters, seed, sink); break;
    case 2: hipLaunchKernelGGL(probe_mfma_kernel, dim3(blocks), dim3(256), 0, st, iters, seed, sink); break;
    default: return set_error(KVP_INVALID, "kvp_probe_compute: kind=%d not in {0,1,2}", kind);
  }
  return check_launch("kvp_probe_compute");
}
