// HBM ceilings: the plain streaming read and the plain streaming copy that
// the bandwidth-bound kernels are held against.
//
// Read: n bytes read once, the yardstick of the kernels whose time is one
// pass over their operands (the decode GEMVs read every weight byte once).
// 2048 workgroups of 256 threads walk the buffer grid-stride, each thread
// with 8 non-temporal 16-byte loads in flight per trip, xor-fold what they
// read and write one word per workgroup (so the loads cannot be dropped).
// Grid and depth are the fastest of a sweep on MI355X (grids 256..4096 x
// 2..8 loads in flight; 33.6..201 MB buffers that the Infinity Cache cannot
// hold): wider grids or deeper trips gained nothing.
//
// Copy: n bytes read once and written once, the yardstick of the norm and
// RoPE kernels (each reads its input once and writes its output once).  A
// one-shot grid, each thread 2 non-temporal 16-byte loads in flight, then 2
// non-temporal stores: the fastest of a sweep on MI355X at 48 and 160 MiB a
// side (1, 2, 4, 8, 16 loads per thread; plain or non-temporal loads and
// stores): 5.35 and 5.98 TB/s, against 4.8-5.1 and 5.3-5.8 for the others.
#include "common.hpp"

namespace umic {
namespace {

constexpr int kReadThreads = 256;
constexpr int kReadDepth = 8;
constexpr int kCopyThreads = 256;
constexpr int kCopyDepth = 2;

__global__ __launch_bounds__(kReadThreads) void stream_read_kernel(const u32x4* __restrict__ p,
                                                                   int64_t n16, uint32_t* fold) {
  const int64_t trip = (int64_t)gridDim.x * kReadThreads * kReadDepth;
  uint32_t acc = 0;
  for (int64_t base = (int64_t)blockIdx.x * kReadThreads * kReadDepth + threadIdx.x; base < n16;
       base += trip) {
    u32x4 v[kReadDepth];
#pragma unroll
    for (int u = 0; u < kReadDepth; ++u) {
      const int64_t i = base + (int64_t)u * kReadThreads;
      v[u] = i < n16 ? __builtin_nontemporal_load(p + i) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < kReadDepth; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  __shared__ uint32_t part[kReadThreads];
  part[threadIdx.x] = acc;
  __syncthreads();
  if (threadIdx.x < kWave) {
    uint32_t a = part[threadIdx.x] ^ part[threadIdx.x + 64] ^ part[threadIdx.x + 128] ^
                 part[threadIdx.x + 192];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) a ^= (uint32_t)__shfl_xor((int)a, o, kWave);
    if (threadIdx.x == 0) fold[blockIdx.x] = a;
  }
}

__global__ __launch_bounds__(kCopyThreads) void stream_copy_kernel(const u32x4* __restrict__ src,
                                                                   u32x4* __restrict__ dst,
                                                                   int64_t n16) {
  const int64_t base = (int64_t)blockIdx.x * kCopyThreads * kCopyDepth + threadIdx.x;
  u32x4 v[kCopyDepth];
#pragma unroll
  for (int u = 0; u < kCopyDepth; ++u) {
    const int64_t i = base + (int64_t)u * kCopyThreads;
    if (i < n16) v[u] = __builtin_nontemporal_load(src + i);
  }
#pragma unroll
  for (int u = 0; u < kCopyDepth; ++u) {
    const int64_t i = base + (int64_t)u * kCopyThreads;
    if (i < n16) __builtin_nontemporal_store(v[u], dst + i);
  }
}

}  // namespace
}  // namespace umic

using namespace umic;

extern "C" int umic_stream_read(const void* p, int64_t bytes, void* fold, void* stream) {
  if (bytes < 0) return UMIC_ERR_INVALID_ARG;
  if (bytes == 0) return UMIC_OK;
  if (!p || !fold) return UMIC_ERR_INVALID_ARG;
  if (bytes % 16 || ((uintptr_t)p & 15u) || ((uintptr_t)fold & 3u)) return UMIC_ERR_UNSUPPORTED;
  hipLaunchKernelGGL(stream_read_kernel, dim3(UMIC_STREAM_READ_GRID), dim3(kReadThreads), 0,
                     as_stream(stream), static_cast<const u32x4*>(p), bytes / 16,
                     static_cast<uint32_t*>(fold));
  return launch_status();
}

extern "C" int umic_stream_copy(const void* src, void* dst, int64_t bytes, void* stream) {
  if (bytes < 0) return UMIC_ERR_INVALID_ARG;
  if (bytes == 0) return UMIC_OK;
  if (!src || !dst) return UMIC_ERR_INVALID_ARG;
  const uintptr_t s = (uintptr_t)src, d = (uintptr_t)dst;
  if (s < d + (uintptr_t)bytes && d < s + (uintptr_t)bytes) return UMIC_ERR_INVALID_ARG;
  if (bytes % 16 || (s & 15u) || (d & 15u)) return UMIC_ERR_UNSUPPORTED;
  const int64_t n16 = bytes / 16;
  const int64_t per = (int64_t)kCopyThreads * kCopyDepth;
  const int64_t grid = (n16 + per - 1) / per;
  if (grid > INT32_MAX) return UMIC_ERR_UNSUPPORTED;
  hipLaunchKernelGGL(stream_copy_kernel, dim3((unsigned)grid), dim3(kCopyThreads), 0,
                     as_stream(stream), static_cast<const u32x4*>(src), static_cast<u32x4*>(dst),
                     n16);
  return launch_status();
}
