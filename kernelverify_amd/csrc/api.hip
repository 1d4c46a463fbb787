// Library-wide entry points: version, diagnostics, device facts, and the
// HBM roofline probe kernels.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <string>

#include "common.h"

namespace kvp {

namespace {
thread_local std::string g_last_error;
}

int set_error(int status, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return status;
}

// Entry points start here: the message is reset, and so is the runtime's
// per-thread last error, which an earlier unrelated HIP call on this thread
// (a failed symbol lookup, say) may have left behind for check_launch to
// misreport as this entry's launch failure.
void clear_error() {
  g_last_error.clear();
  (void)hipGetLastError();
}

namespace {
// Each slot holds value + 1; 0 (static zero-initialisation) means unset.
std::atomic<int> g_tuning[kTuneCount];
constexpr const char* kTuneNames[kTuneCount] = {
    "qmv_path", "qmv_per_cu", "qmv_blocks", "qmv_kw", "qmv_rw", "qmv_mfma_tiles",
    "moe_valu", "moe_kq", "moe_permute", "moe_down_combine"};

int tuning_index(const char* key) {
  for (int i = 0; key && i < kTuneCount; ++i)
    if (strcmp(key, kTuneNames[i]) == 0) return i;
  return -1;
}
}  // namespace

int tuning(TuneKey key, int fallback) {
  const int v = g_tuning[key].load(std::memory_order_relaxed);
  return v == 0 ? fallback : v - 1;
}

int check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    return set_error(KVP_LAUNCH_ERROR, "%s: launch failed: %s", what, hipGetErrorString(err));
  }
  return KVP_OK;
}

namespace {

// Streaming read: four independent accumulators per thread over a
// grid-stride loop of 16-byte non-temporal loads; one float per block is
// stored so the loads stay live (roofline_probe.mm:35-144 measures the same
// two ceilings, read and copy, on Apple GPUs).
__global__ __launch_bounds__(256) void probe_read_kernel(const u32x4* __restrict__ src,
                                                         size_t n16, float* __restrict__ sink) {
  uint32_t a0 = 0, a1 = 0, a2 = 0, a3 = 0;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (; i + 3 * stride < n16; i += 4 * stride) {
    u32x4 v0 = __builtin_nontemporal_load(src + i);
    u32x4 v1 = __builtin_nontemporal_load(src + i + stride);
    u32x4 v2 = __builtin_nontemporal_load(src + i + 2 * stride);
    u32x4 v3 = __builtin_nontemporal_load(src + i + 3 * stride);
    a0 ^= v0.x ^ v0.y ^ v0.z ^ v0.w;
    a1 ^= v1.x ^ v1.y ^ v1.z ^ v1.w;
    a2 ^= v2.x ^ v2.y ^ v2.z ^ v2.w;
    a3 ^= v3.x ^ v3.y ^ v3.z ^ v3.w;
  }
  for (; i < n16; i += stride) {
    u32x4 v = __builtin_nontemporal_load(src + i);
    a0 ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  uint32_t a = a0 ^ a1 ^ a2 ^ a3;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) a ^= (uint32_t)__shfl_xor((int)a, off, kWave);
  if (threadIdx.x == 0) sink[blockIdx.x] = (float)(a & 0xFFFF);
}

__global__ __launch_bounds__(256) void probe_copy_kernel(const u32x4* __restrict__ src,
                                                         u32x4* __restrict__ dst, size_t n16) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride) {
    __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
  }
}

}  // namespace
}  // namespace kvp

extern "C" {

const char* kvp_version(void) { return "kvpack 0.1.0 gfx950"; }

size_t kvp_last_error(char* buf, size_t cap) {
  const std::string& e = kvp::g_last_error;
  if (buf && cap) {
    size_t n = e.size() < cap - 1 ? e.size() : cap - 1;
    memcpy(buf, e.data(), n);
    buf[n] = '\0';
  }
  return e.size();
}

int kvp_device_info(int device, char* name, size_t name_cap, char* arch, size_t arch_cap,
                    int* compute_units, int* max_threads_per_block, size_t* lds_per_block,
                    size_t* global_mem_bytes, int* clock_khz) {
  kvp::clear_error();
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || count == 0) {
    return kvp::set_error(KVP_NO_DEVICE, "kvp_device_info: no HIP device visible");
  }
  KVP_REQUIRE(device >= 0 && device < count, "kvp_device_info: device %d of %d", device, count);
  hipDeviceProp_t p;
  hipError_t err = hipGetDeviceProperties(&p, device);
  if (err != hipSuccess) {
    return kvp::set_error(KVP_NO_DEVICE, "kvp_device_info: %s", hipGetErrorString(err));
  }
  if (name && name_cap) snprintf(name, name_cap, "%s", p.name);
  if (arch && arch_cap) snprintf(arch, arch_cap, "%s", p.gcnArchName);
  if (compute_units) *compute_units = p.multiProcessorCount;
  if (max_threads_per_block) *max_threads_per_block = p.maxThreadsPerBlock;
  if (lds_per_block) *lds_per_block = p.sharedMemPerBlock;
  if (global_mem_bytes) *global_mem_bytes = p.totalGlobalMem;
  if (clock_khz) *clock_khz = p.clockRate;
  if (strncmp(p.gcnArchName, "gfx950", 6) != 0) {
    return kvp::set_error(KVP_NO_DEVICE, "kvp_device_info: device %d is %s, not gfx950", device,
                          p.gcnArchName);
  }
  return KVP_OK;
}

int kvp_set_tuning(const char* key, int value) {
  kvp::clear_error();
  const int i = kvp::tuning_index(key);
  KVP_REQUIRE(i >= 0, "kvp_set_tuning: unknown key %s", key ? key : "(null)");
  KVP_REQUIRE(value >= -1, "kvp_set_tuning: value %d (-1 restores the library's choice)", value);
  kvp::g_tuning[i].store(value < 0 ? 0 : value + 1, std::memory_order_relaxed);
  return KVP_OK;
}

int kvp_get_tuning(const char* key, int* value) {
  kvp::clear_error();
  const int i = kvp::tuning_index(key);
  KVP_REQUIRE(i >= 0 && value, "kvp_get_tuning: unknown key %s", key ? key : "(null)");
  *value = kvp::tuning(static_cast<kvp::TuneKey>(i), -1);
  return KVP_OK;
}

int kvp_probe_stream_read(const void* src, size_t n_bytes, float* read_sink, int blocks,
                          void* stream) {
  kvp::clear_error();
  KVP_REQUIRE(src && read_sink, "kvp_probe_stream_read: null pointer");
  KVP_REQUIRE(n_bytes % 16 == 0 && n_bytes > 0, "kvp_probe_stream_read: n_bytes %% 16");
  KVP_REQUIRE(blocks > 0, "kvp_probe_stream_read: blocks=%d", blocks);
  hipLaunchKernelGGL(kvp::probe_read_kernel, dim3(blocks), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const kvp::u32x4*>(src),
                     n_bytes / 16, read_sink);
  return kvp::check_launch("kvp_probe_stream_read");
}

int kvp_probe_stream_copy(const void* src, void* dst, size_t n_bytes, int blocks, void* stream) {
  kvp::clear_error();
  KVP_REQUIRE(src && dst, "kvp_probe_stream_copy: null pointer");
  KVP_REQUIRE(n_bytes % 16 == 0 && n_bytes > 0, "kvp_probe_stream_copy: n_bytes %% 16");
  KVP_REQUIRE(blocks > 0, "kvp_probe_stream_copy: blocks=%d", blocks);
  hipLaunchKernelGGL(kvp::probe_copy_kernel, dim3(blocks), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const kvp::u32x4*>(src),
                     static_cast<kvp::u32x4*>(dst), n_bytes / 16);
  return kvp::check_launch("kvp_probe_stream_copy");
}

}  // extern "C"
