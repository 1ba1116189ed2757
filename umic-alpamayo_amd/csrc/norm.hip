// Row normalisation kernels for gfx950: RMSNorm, residual-add + RMSNorm,
// LayerNorm (affine, bias) and residual-add + LayerNorm, all bf16 in/out.
//
// HBM-bound design: every element is read once and written once.  A row is
// owned by an aligned group of LPR lanes of one wavefront; each lane holds
// up to MAXV 16-byte vectors of the row in registers (lane-interleaved, so
// every load/store instruction of the group covers LPR*16 contiguous bytes).
// Row statistics are reduced with cross-lane butterflies only -- no LDS, no
// barriers -- and the normalised values are written straight from the
// registers the row was loaded into.  Rows that fit neither the 16-byte
// vector layout nor 16*64*8 elements take a block-per-row generic kernel.
//
// Numerics.  Row statistics come from exact double sums of x and x^2 (a
// bf16 square is exact in fp32; the double sums of bf16-derived terms are
// exact for activation-range data, hence independent of summation order):
// mean = sum/n and var = sumsq/n - mean^2 in double, each rounded once to
// fp32, rstd = 1/sqrt(var + eps) in double rounded once.  Every bf16
// rounding point of the eager op chain is kept:
//   RMSNorm     y = bf16(w * bf16(x * rstd))          (HF Qwen3VLTextRMSNorm)
//   LayerNorm   y = bf16(fma(w, rstd * (x - mean), b)) (torch layer_norm)
//   add+norm    s = bf16(x + r), then the norm of the ROUNDED s (eager adds
//               the residual as its own bf16 op before the norm).
#include "common.hpp"

namespace umic {
namespace {

enum NormOp { kRms = 0, kAddRms = 1, kLn = 2, kAddLn = 3 };

constexpr bool has_add(int op) { return op == kAddRms || op == kAddLn; }
constexpr bool is_ln(int op) { return op == kLn || op == kAddLn; }

struct NormArgs {
  const uint16_t* x;
  const uint16_t* r;  // residual (add ops)
  const uint16_t* w;
  const uint16_t* b;  // bias (LayerNorm ops)
  uint16_t* y;        // normalised output
  uint16_t* s;        // summed output (add ops)
  int64_t rows, n, ldx, ldr, ldy, lds;
  float eps;
};

// ---- register-resident fast path -----------------------------------------

// RPG rows per group: rows of one or two vectors per lane (e.g. the
// [S*H, 128] per-head q/k norms) leave a wavefront only 1-2 KB of loads in
// flight, too little to cover HBM latency; a group then takes RPG
// consecutive rows and issues all their loads before reducing any.
template <int OP, int LPR, int MAXV, int RPG>
__global__ __launch_bounds__(256) void norm_rows_kernel(NormArgs a, int nvec, int vpl) {
  const int rows_per_block = (int)blockDim.x / LPR * RPG;
  const int lane = threadIdx.x & (LPR - 1);
  const int64_t row0 = (int64_t)blockIdx.x * rows_per_block + (threadIdx.x / LPR) * RPG;
  // All LPR lanes of a group share its rows, so a group exits as a whole and
  // the butterflies below only ever read lanes of a live group.
  if (row0 >= a.rows) return;

  // The rows' source values stay packed as bf16 (16 B per 8 elements) in
  // registers between the statistics pass and the output pass.  Loads are
  // issued unconditionally (a dead slot re-reads vector 0, a row past the
  // end re-reads row0; both are zeroed or never stored): predicated loads
  // would sit in branches, and every branch join costs a full vmcnt drain
  // -- the loads must all be in flight together.
  const u32x4 zero = {0u, 0u, 0u, 0u};
  bool live[MAXV];
  int cix[MAXV];
#pragma unroll
  for (int i = 0; i < MAXV; ++i) {
    const int c = i * LPR + lane;
    live[i] = i < vpl && c < nvec;
    cix[i] = live[i] ? c : 0;
  }
  bool rlive[RPG];
  int64_t rows[RPG];
#pragma unroll
  for (int r = 0; r < RPG; ++r) {
    rlive[r] = r == 0 || row0 + r < a.rows;  // row0 is live (checked above)
    rows[r] = rlive[r] ? row0 + r : row0;
  }
  u32x4 sv[RPG][MAXV];
#pragma unroll
  for (int r = 0; r < RPG; ++r) {
    const u32x4* xp = reinterpret_cast<const u32x4*>(a.x + rows[r] * a.ldx);
#pragma unroll
    for (int i = 0; i < MAXV; ++i) sv[r][i] = ld_stream(xp + cix[i]);
  }
  if constexpr (has_add(OP)) {
    u32x4 rv[RPG][MAXV];
#pragma unroll
    for (int r = 0; r < RPG; ++r) {
      const u32x4* rp = reinterpret_cast<const u32x4*>(a.r + rows[r] * a.ldr);
#pragma unroll
      for (int i = 0; i < MAXV; ++i) rv[r][i] = ld_stream(rp + cix[i]);
    }
#pragma unroll
    for (int r = 0; r < RPG; ++r) {
#pragma unroll
      for (int i = 0; i < MAXV; ++i) {
        float xf[8], rf[8];
        unpack8(sv[r][i], xf);
        unpack8(rv[r][i], rf);
#pragma unroll
        for (int e = 0; e < 8; ++e) xf[e] = xf[e] + rf[e];
        sv[r][i] = pack8(xf);  // bf16(x + r): the eager residual add
      }
      u32x4* sp = reinterpret_cast<u32x4*>(a.s + rows[r] * a.lds);
#pragma unroll
      for (int i = 0; i < MAXV; ++i)
        if (live[i] && rlive[r]) st_stream(sp + cix[i], sv[r][i]);
    }
  }

  const u32x4* wp = reinterpret_cast<const u32x4*>(a.w);
  const u32x4* bp = reinterpret_cast<const u32x4*>(a.b);
  u32x4 wv[MAXV], bv[MAXV];
  const double inv_n = 1.0 / (double)a.n;
#pragma unroll
  for (int r = 0; r < RPG; ++r) {
#pragma unroll
    for (int i = 0; i < MAXV; ++i) sv[r][i] = live[i] ? sv[r][i] : zero;

    // Exact double sums (zero-filled tail vectors contribute nothing).  Four
    // independent accumulators keep the f64 add chains short; the sums are
    // exact, so the grouping does not change them.
    double sum4[4] = {0.0, 0.0, 0.0, 0.0}, ssq4[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
    for (int i = 0; i < MAXV; ++i) {
      float f[8];
      unpack8(sv[r][i], f);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if constexpr (is_ln(OP)) sum4[e & 3] += (double)f[e];
        ssq4[e & 3] += (double)(f[e] * f[e]);  // a bf16 square is exact in fp32
      }
    }
    double sum = (sum4[0] + sum4[1]) + (sum4[2] + sum4[3]);
    double ssq = (ssq4[0] + ssq4[1]) + (ssq4[2] + ssq4[3]);
    float rstd, mean = 0.f;
    if constexpr (is_ln(OP)) {
      sum = group_sum<LPR>(sum);
      ssq = group_sum<LPR>(ssq);
      const double mean_d = sum * inv_n;
      mean = (float)mean_d;
      rstd = rsqrt_cr((float)(ssq * inv_n - mean_d * mean_d) + a.eps);
    } else {
      rstd = rsqrt_cr((float)(group_sum<LPR>(ssq) * inv_n) + a.eps);
    }
    if (r == 0) {
      // weights (and bias), L2-resident, loaded once the first row's
      // statistics are done: issued with the row loads they measured slower
#pragma unroll
      for (int i = 0; i < MAXV; ++i) {
        wv[i] = wp[cix[i]];
        if constexpr (is_ln(OP)) bv[i] = bp[cix[i]];
      }
    }

    u32x4* yp = reinterpret_cast<u32x4*>(a.y + rows[r] * a.ldy);
#pragma unroll
    for (int i = 0; i < MAXV; ++i) {
      if (!live[i] || !rlive[r]) continue;
      const int c = cix[i];
      float f[8], wf[8], o[8];
      unpack8(sv[r][i], f);
      unpack8(wv[i], wf);
      if constexpr (is_ln(OP)) {
        float bf[8];
        unpack8(bv[i], bf);
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = __builtin_fmaf(wf[e], rstd * (f[e] - mean), bf[e]);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = wf[e] * rbf(f[e] * rstd);
      }
      st_stream(yp + c, pack8(o));
    }
  }
}

// ---- generic path: one 256-thread block per row, scalar elements ---------

__device__ double block_sum(double v, double* red) {
  v = group_sum<kWave>(v);
  const int wid = threadIdx.x / kWave;
  __syncthreads();  // `red` may still be read from a previous reduction
  if ((threadIdx.x & (kWave - 1)) == 0) red[wid] = v;
  __syncthreads();
  double t = 0.0;
  for (int i = 0; i < (int)(blockDim.x / kWave); ++i) t += red[i];
  return t;
}

// Element j of the row the statistics are taken over: x, or bf16(x + r).
// Recomputed on every pass (cheap, identical result) rather than re-read
// from the summed output.
template <int OP>
__device__ __forceinline__ float src_val(const NormArgs& a, int64_t row, int64_t j) {
  const float xf = bf2f(a.x[row * a.ldx + j]);
  if constexpr (has_add(OP)) return rbf(xf + bf2f(a.r[row * a.ldr + j]));
  return xf;
}

template <int OP>
__global__ __launch_bounds__(256) void norm_generic_kernel(NormArgs a) {
  __shared__ double red[256 / kWave];
  const int64_t row = blockIdx.x;
  if constexpr (has_add(OP)) {
    uint16_t* sr = a.s + row * a.lds;
    for (int64_t j = threadIdx.x; j < a.n; j += blockDim.x)
      sr[j] = (uint16_t)f2bf(src_val<OP>(a, row, j));
  }
  const double inv_n = 1.0 / (double)a.n;
  float rstd, mean = 0.f;
  double sum = 0.0, ssq = 0.0;
  for (int64_t j = threadIdx.x; j < a.n; j += blockDim.x) {
    const float f = src_val<OP>(a, row, j);
    if constexpr (is_ln(OP)) sum += (double)f;
    ssq += (double)(f * f);
  }
  if constexpr (is_ln(OP)) {
    const double mean_d = block_sum(sum, red) * inv_n;
    mean = (float)mean_d;
    rstd = rsqrt_cr((float)(block_sum(ssq, red) * inv_n - mean_d * mean_d) + a.eps);
  } else {
    rstd = rsqrt_cr((float)(block_sum(ssq, red) * inv_n) + a.eps);
  }
  uint16_t* yr = a.y + row * a.ldy;
  for (int64_t j = threadIdx.x; j < a.n; j += blockDim.x) {
    const float f = src_val<OP>(a, row, j);
    const float w = bf2f(a.w[j]);
    float o;
    if constexpr (is_ln(OP)) o = __builtin_fmaf(w, rstd * (f - mean), bf2f(a.b[j]));
    else o = w * rbf(f * rstd);
    yr[j] = (uint16_t)f2bf(o);
  }
}

// ---- host dispatch --------------------------------------------------------

// Block size: the hardware spreads workgroups evenly over the 256 CUs only
// when there are many of them, so small row counts get 64- or 128-thread
// blocks (the largest block that still yields >= 8 blocks per CU).
template <int OP, int LPR, int MAXV, int RPG = 1>
int launch_rows(const NormArgs& a, int nvec, int vpl, hipStream_t st) {
  int threads = 256;
  while (threads > 64 && (a.rows * LPR / RPG + threads - 1) / threads < 8 * 256) threads >>= 1;
  const int rows_per_block = threads / LPR * RPG;
  const int64_t blocks = (a.rows + rows_per_block - 1) / rows_per_block;
  if (blocks > 0x7fffffffLL) return UMIC_ERR_UNSUPPORTED;
  hipLaunchKernelGGL((norm_rows_kernel<OP, LPR, MAXV, RPG>), dim3((unsigned)blocks), dim3(threads),
                     0, st, a, nvec, vpl);
  return launch_status();
}

// One- and two-vector rows take 4 or 2 rows per group when the grouped
// launch still has >= 16 wavefronts per CU (measured on the [S*H, 128]
// per-head norms: 99200 rows gain ~10%, 24800 rows lose ~18% with grouping);
// smaller launches keep one row per group, spread over more wavefronts.
constexpr int64_t kRpgMinThreads = (int64_t)256 * 16 * 64;

template <int OP, int LPR, int MAXV>
int launch_small_rows(const NormArgs& a, int nvec, int vpl, hipStream_t st) {
  constexpr int kRpg = MAXV == 1 ? 4 : 2;
  if (a.rows * LPR / kRpg >= kRpgMinThreads)
    return launch_rows<OP, LPR, MAXV, kRpg>(a, nvec, vpl, st);
  return launch_rows<OP, LPR, MAXV>(a, nvec, vpl, st);
}

template <int OP, int LPR>
int launch_lpr(const NormArgs& a, int nvec, int vpl, hipStream_t st) {
  switch (vpl) {
    case 1: return launch_small_rows<OP, LPR, 1>(a, nvec, vpl, st);
    case 2: return launch_small_rows<OP, LPR, 2>(a, nvec, vpl, st);
    case 3: return launch_rows<OP, LPR, 3>(a, nvec, vpl, st);
    case 4: return launch_rows<OP, LPR, 4>(a, nvec, vpl, st);
    case 5: return launch_rows<OP, LPR, 5>(a, nvec, vpl, st);
    case 6: return launch_rows<OP, LPR, 6>(a, nvec, vpl, st);
    case 7:
    case 8: return launch_rows<OP, LPR, 8>(a, nvec, vpl, st);
    case 9:
    case 10: return launch_rows<OP, LPR, 10>(a, nvec, vpl, st);
    case 11:
    case 12: return launch_rows<OP, LPR, 12>(a, nvec, vpl, st);
    default: return launch_rows<OP, LPR, 16>(a, nvec, vpl, st);
  }
}

template <int OP>
int launch_norm(const NormArgs& a, hipStream_t st) {
  bool vec = a.n % 8 == 0 && a.ldx % 8 == 0 && a.ldy % 8 == 0 && aligned16(a.x) &&
             aligned16(a.y) && aligned16(a.w);
  if (has_add(OP)) vec = vec && a.ldr % 8 == 0 && a.lds % 8 == 0 && aligned16(a.r) && aligned16(a.s);
  if (is_ln(OP)) vec = vec && aligned16(a.b);
  const int64_t nvec = a.n / 8;
  if (vec && nvec >= 8 && nvec <= 64 * 16) {
    // Lanes per row: the widest group that splits the row evenly into at
    // most 16 vectors per lane; else the widest group with a ragged tail.
    int lpr = 0;
    for (int g = 64; g >= 8 && !lpr; g >>= 1)
      if (nvec % g == 0 && nvec / g <= 16) lpr = g;
    if (!lpr) {
      lpr = 8;
      while (lpr * 2 <= 64 && lpr * 2 <= nvec) lpr *= 2;
    }
    const int vpl = (int)((nvec + lpr - 1) / lpr);
    if (vpl <= 16) {
      switch (lpr) {
        case 64: return launch_lpr<OP, 64>(a, (int)nvec, vpl, st);
        case 32: return launch_lpr<OP, 32>(a, (int)nvec, vpl, st);
        case 16: return launch_lpr<OP, 16>(a, (int)nvec, vpl, st);
        default: return launch_lpr<OP, 8>(a, (int)nvec, vpl, st);
      }
    }
  }
  if (a.rows > 0x7fffffffLL) return UMIC_ERR_UNSUPPORTED;
  hipLaunchKernelGGL((norm_generic_kernel<OP>), dim3((unsigned)a.rows), dim3(256), 0, st, a);
  return launch_status();
}

template <int OP>
int norm_entry(NormArgs a, void* stream) {
  if (a.rows < 0 || a.n <= 0) return UMIC_ERR_INVALID_ARG;
  if (a.rows == 0) return UMIC_OK;  // empty tensors may carry null pointers
  if (!a.x || !a.w || !a.y) return UMIC_ERR_INVALID_ARG;
  if (has_add(OP) && (!a.r || !a.s)) return UMIC_ERR_INVALID_ARG;
  if (is_ln(OP) && !a.b) return UMIC_ERR_INVALID_ARG;
  if (a.ldx < a.n || a.ldy < a.n) return UMIC_ERR_INVALID_ARG;
  if (has_add(OP) && (a.ldr < a.n || a.lds < a.n)) return UMIC_ERR_INVALID_ARG;
  return launch_norm<OP>(a, as_stream(stream));
}

}  // namespace
}  // namespace umic

using namespace umic;

extern "C" int umic_rmsnorm_bf16(const void* x, const void* w, void* y, int64_t rows, int64_t n,
                                 int64_t ldx, int64_t ldy, float eps, void* stream) {
  NormArgs a{(const uint16_t*)x, nullptr, (const uint16_t*)w, nullptr, (uint16_t*)y, nullptr,
             rows, n, ldx, 0, ldy, 0, eps};
  return norm_entry<kRms>(a, stream);
}

extern "C" int umic_add_rmsnorm_bf16(const void* x, const void* r, const void* w, void* normed,
                                     void* summed, int64_t rows, int64_t n, int64_t ldx,
                                     int64_t ldr, int64_t ldn, int64_t lds, float eps,
                                     void* stream) {
  NormArgs a{(const uint16_t*)x, (const uint16_t*)r, (const uint16_t*)w, nullptr,
             (uint16_t*)normed, (uint16_t*)summed, rows, n, ldx, ldr, ldn, lds, eps};
  return norm_entry<kAddRms>(a, stream);
}

extern "C" int umic_layernorm_bf16(const void* x, const void* w, const void* b, void* y,
                                   int64_t rows, int64_t n, int64_t ldx, int64_t ldy, float eps,
                                   void* stream) {
  NormArgs a{(const uint16_t*)x, nullptr, (const uint16_t*)w, (const uint16_t*)b, (uint16_t*)y,
             nullptr, rows, n, ldx, 0, ldy, 0, eps};
  return norm_entry<kLn>(a, stream);
}

extern "C" int umic_add_layernorm_bf16(const void* x, const void* r, const void* w,
                                       const void* b, void* normed, void* summed, int64_t rows,
                                       int64_t n, int64_t ldx, int64_t ldr, int64_t ldn,
                                       int64_t lds, float eps, void* stream) {
  NormArgs a{(const uint16_t*)x, (const uint16_t*)r, (const uint16_t*)w, (const uint16_t*)b,
             (uint16_t*)normed, (uint16_t*)summed, rows, n, ldx, ldr, ldn, lds, eps};
  return norm_entry<kAddLn>(a, stream);
}
