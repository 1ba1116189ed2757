// Streaming ceilings of this GPU's HBM for the access patterns of the
// HBM-bound hot-path kernels: pure read, pure write, and copy (read n bytes,
// write n bytes -- the pattern of every norm and RoPE kernel, which read each
// input once and write each output once).  16-byte vector accesses,
// grid-stride loops (every index checked against the element count),
// non-temporal loads; timed with HIP events over back-to-back launches that
// rotate over buffers of >= 1 GiB in total, so nothing is served from the
// 256 MB Infinity Cache.  The copy sizes are the byte counts the norm
// kernels move at the BASELINE shapes.  One JSON line per measurement.
//
//   umic-alpamayo_amd/umic/lib/hbm_ceiling      (built by build.py)
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <vector>

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

#define CHECK(x)                                                                     \
  do {                                                                               \
    hipError_t e_ = (x);                                                             \
    if (e_ != hipSuccess) {                                                          \
      std::fprintf(stderr, "%s failed: %s\n", #x, hipGetErrorString(e_));             \
      return 1;                                                                      \
    }                                                                                \
  } while (0)

__global__ void read_kernel(const u32x4* __restrict__ a, size_t n, uint32_t* sink) {
  u32x4 acc = {0u, 0u, 0u, 0u};
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += stride)
    acc ^= __builtin_nontemporal_load(a + i);
  // keeps every load live; the buffers are filled so that this never holds
  if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x9e3779b9u) sink[0] = 1u;
}

__global__ void write_kernel(u32x4* __restrict__ a, size_t n) {
  const u32x4 v = {1u, 2u, 3u, (uint32_t)blockIdx.x};
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += stride) a[i] = v;
}

__global__ void copy_kernel(const u32x4* __restrict__ a, u32x4* __restrict__ b, size_t n) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += stride)
    b[i] = __builtin_nontemporal_load(a + i);
}

int main() {
  int cus = 0;
  CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0));
  uint32_t* sink = nullptr;
  CHECK(hipMalloc(&sink, sizeof(uint32_t)));
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  // bytes per side (read = write for the copy): the norm kernels' moved
  // bytes / 2 (RMSNorm, LayerNorm, add+RMSNorm, add+LayerNorm), then 1 GiB
  const size_t sides[] = {25399296, 41945600, 50794496, 83888640, size_t(1) << 30};
  const int kReps = 16;
  for (size_t bytes : sides) {
    const size_t n = bytes / 16;
    const int nbuf = (int)(((size_t(1) << 30) + bytes - 1) / bytes) + 1;
    std::vector<u32x4*> src(nbuf), dst(nbuf);
    for (int i = 0; i < nbuf; ++i) {
      CHECK(hipMalloc(&src[i], n * 16));
      CHECK(hipMalloc(&dst[i], n * 16));
      CHECK(hipMemset(src[i], 0x5a, n * 16));
      CHECK(hipMemset(dst[i], 0, n * 16));
    }
    for (int pattern = 0; pattern < 3; ++pattern) {
      for (int bpc : {4, 8, 16}) {
        const int grid = cus * bpc;
        auto launch = [&](int r) {
          if (pattern == 0) read_kernel<<<grid, 256>>>(src[r % nbuf], n, sink);
          if (pattern == 1) write_kernel<<<grid, 256>>>(dst[r % nbuf], n);
          if (pattern == 2) copy_kernel<<<grid, 256>>>(src[r % nbuf], dst[r % nbuf], n);
        };
        for (int r = 0; r < 2; ++r) launch(r);
        CHECK(hipDeviceSynchronize());
        CHECK(hipEventRecord(e0, 0));
        for (int r = 0; r < kReps; ++r) launch(r);
        CHECK(hipEventRecord(e1, 0));
        CHECK(hipEventSynchronize(e1));
        float ms = 0.f;
        CHECK(hipEventElapsedTime(&ms, e0, e1));
        const double us = ms * 1e3 / kReps;
        const double moved = pattern == 2 ? 2.0 * n * 16 : 1.0 * n * 16;
        static const char* names[] = {"read", "write", "copy"};
        std::printf("{\"pattern\": \"%s\", \"bytes_moved\": %.0f, \"blocks_per_cu\": %d, "
                    "\"us\": %.2f, \"tbps\": %.3f}\n",
                    names[pattern], moved, bpc, us, moved / us / 1e6);
        std::fflush(stdout);
      }
    }
    for (int i = 0; i < nbuf; ++i) {
      CHECK(hipFree(src[i]));
      CHECK(hipFree(dst[i]));
    }
  }
  return 0;
}
