// Writes the gfx950 v_rcp_f32 and v_rsq_f32 results that torch-ROCm's
// LayerNorm uses (count reciprocals and the final rstd), for the CPU oracle:
//   rcp: every integer 1..65536 (raw floats)
//   rsq: every float of [1, 4) (raw floats; both instructions are exactly
//        exponent-scale invariant on the device, so one binade pair covers
//        all normal inputs).
// Usage: gfx950_tables OUT_RCP OUT_RSQ
#include <hip/hip_runtime.h>
#include <cstdio>
#include <vector>

__global__ void rcp_ints(float* out, int n) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
    out[i] = __builtin_amdgcn_rcpf((float)(i + 1));
}

__global__ void rsq_binades(float* out, int n) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
    out[i] = __builtin_amdgcn_rsqf(__uint_as_float(0x3f800000u + (unsigned)i));
}

static int dump(const char* path, const std::vector<float>& v) {
  FILE* f = fopen(path, "wb");
  if (!f) return 1;
  const size_t w = fwrite(v.data(), sizeof(float), v.size(), f);
  fclose(f);
  return w != v.size();
}

int main(int argc, char** argv) {
  if (argc != 3) return 1;
  const int NR = 65536, NS = 1 << 24;
  float *dr = nullptr, *ds = nullptr;
  if (hipMalloc(&dr, NR * sizeof(float)) != hipSuccess) return 2;
  if (hipMalloc(&ds, NS * sizeof(float)) != hipSuccess) return 2;
  hipLaunchKernelGGL(rcp_ints, dim3(256), dim3(256), 0, 0, dr, NR);
  hipLaunchKernelGGL(rsq_binades, dim3(1024), dim3(256), 0, 0, ds, NS);
  if (hipDeviceSynchronize() != hipSuccess) return 3;
  std::vector<float> hr(NR), hs(NS);
  if (hipMemcpy(hr.data(), dr, NR * sizeof(float), hipMemcpyDeviceToHost) != hipSuccess) return 3;
  if (hipMemcpy(hs.data(), ds, NS * sizeof(float), hipMemcpyDeviceToHost) != hipSuccess) return 3;
  if (hipFree(dr) != hipSuccess || hipFree(ds) != hipSuccess) return 3;
  return dump(argv[1], hr) | dump(argv[2], hs);
}
