/*
 * umic_oracle.c -- CPU restatement of the UMIC hot-path arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP
 * kernels in libumic_hip.so.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it, and only as the checker (or the
 * timed CPU baseline); the product path never calls it.
 *
 * What it restates.  The reference (soonhong99/umic-alpamayo) swaps HF
 * transformers' eager modules for fused kernels; "parity" means matching the
 * eager op chain each kernel replaces.  That chain lives in the third-party
 * packages torch (reference pin >=2.8, pyproject.toml:11) and transformers
 * (pin >=4.56, pyproject.toml:12; checked against 5.15.0 here), file
 * transformers/models/qwen3_vl/modeling_qwen3_vl.py, cited below as "HF:".
 * Every bf16 rounding point of the eager chain is reproduced explicitly with
 * round-to-nearest-even; fp32 steps are single IEEE operations (the file is
 * compiled with -ffp-contract=off, and fmaf() is used exactly where the
 * eager GPU kernel contracts).
 *
 * Row statistics follow torch-ROCm's own fp32 reduction order on the GPU
 * (see "torch-ROCm's fp32 row reductions" below), so the restated norms
 * equal eager on the GPU bit for bit.
 *
 * bf16 values travel as uint16_t bit patterns.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ---- bf16 <-> fp32 ----------------------------------------------------- */

static inline float bf2f(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* Round-to-nearest-even fp32 -> bf16, NaN kept quiet (torch's
 * c10::BFloat16 round_to_nearest_even). */
static inline uint16_t f2bf(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static inline float rbf(float f) { return bf2f(f2bf(f)); }

/* Correctly rounded fp32 1/sqrt(v). */
static inline float rsqrt_cr(float v) { return (float)(1.0 / sqrt((double)v)); }

void orc_f32_to_bf16(const float* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = f2bf(in[i]);
}

void orc_bf16_to_f32(const uint16_t* in, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = bf2f(in[i]);
}

/* ---- torch-ROCm's fp32 row reductions ----------------------------------
 *
 * The eager norms reduce on the GPU in fp32, in an order fixed by torch's
 * kernels; a statistic one fp32 ulp off moves bf16 outputs by up to two
 * ulps, so the oracle restates that order exactly.
 *
 * RMSNorm: HF:400-405 computes v = x.float().pow(2).mean(-1) with aten's
 * generic reduction (ATen/native/hip/Reduce.cuh, shipped with torch:
 * setReduceConfig, ReduceOp::input_vectorized_thread_reduce_impl,
 * thread_reduce_impl, block_x_reduce, block_y_reduce; MeanOps in
 * ATen/native/SharedReduceOps.h), then torch.rsqrt(v + eps), which is
 * correctly rounded on this platform (all 2^24 floats of [1, 4) checked on
 * the device, tests/golden/eager_gpu_stats.npz).  The plan below is
 * setReduceConfig for a contiguous [rows, n] fp32 tensor reduced over its
 * last dim (warp size 64, 256 CUs, 512 threads per block); block_x_reduce's
 * shuffle loop runs its offsets upward (1, 2, 4, ...) in the ROCm build.
 *
 * LayerNorm: torch.nn.functional.layer_norm on bf16 launches aten's
 * vectorized_layer_norm_kernel (kernel name and its 64x4 block read from a
 * rocprofv3 kernel trace): per-thread Welford over 4-element vectors, a
 * shuffle-down tree per wavefront and a shared-memory tree over the four
 * wavefronts.  Fitted bit-exactly against torch's own mean/rstd outputs on
 * 13 shapes and structured rows (tests/golden/make_eager_gpu.py); the fit
 * fixed which products the ROCm build fuses and that the count reciprocals
 * and the final rstd are the hardware v_rcp_f32 / v_rsq_f32, which the
 * oracle takes from measured tables (tests/golden/make_gfx950_tables.py). */

typedef struct {
  int vec;    /* 4-element vector loads along the row (n >= 128) */
  int bw;     /* threads across the row (block width) */
  int bh;     /* block height */
  int split;  /* the row is also split across the bh wavefronts */
} rms_plan_t;

static int last_pow2(int64_t v) {
  int p = 1;
  while ((int64_t)p * 2 <= v) p *= 2;
  return p;
}

/* setReduceConfig (Reduce.cuh) for inputs_per_output = n, num_outputs = rows.
 * Returns 0, or -1 when the launch would also split rows across blocks
 * (global reduction; only for n >= 131072). */
static int rms_plan_for(int64_t rows, int64_t n, rms_plan_t* p) {
  const int max_threads = 512;
  int64_t dim0 = n, dim1 = rows;
  p->vec = dim0 >= 128;
  if (p->vec) dim0 /= 4;
  const int d0 = dim0 < max_threads ? last_pow2(dim0) : max_threads;
  const int d1 = dim1 < max_threads ? last_pow2(dim1) : max_threads;
  int bw = d0 < 64 ? d0 : 64;
  int bh = d1 < max_threads / bw ? d1 : max_threads / bw;
  bw = d0 < max_threads / bh ? d0 : max_threads / bh;
  const int64_t vpt = (n + bw - 1) / bw;
  const int64_t thr = (int64_t)bh * 16 < 256 ? (int64_t)bh * 16 : 256;
  p->bw = bw;
  p->bh = bh;
  p->split = vpt >= thr;
  if (p->split && (n + (int64_t)bw * bh - 1) / ((int64_t)bw * bh) >= 256) return -1;
  return 0;
}

/* Partial sum of squares of one reducing thread (lane x, wavefront y) over
 * the fp32 row q[0..n) whose first element sits `shift` elements past a
 * 16-byte boundary (row r of a contiguous fp32 tensor: (r * n) % 4). */
static float rms_thread(const float* q, int64_t n, int shift, const rms_plan_t* p, int x, int y) {
  const int64_t step = (int64_t)p->bw * (p->split ? p->bh : 1);
  const int64_t idx0 = x + (int64_t)(p->split ? y : 0) * p->bw;
  const int tail_ok = !p->split || y == 0;
  if (p->vec) {
    const float* d = q;
    int64_t end = n;
    float v0 = 0.0f;
    if (shift > 0) {  /* head elements before the first aligned vector */
      d -= shift;
      end += shift;
      if (x >= shift && x < 4 && tail_ok) v0 = v0 + d[x] * d[x];
      end -= 4;
      d += 4;
    }
    float a[4] = {v0, 0.0f, 0.0f, 0.0f};
    int64_t idx = idx0;
    while (idx * 4 + 3 < end) {
      for (int i = 0; i < 4; ++i) a[i] = a[i] + d[idx * 4 + i] * d[idx * 4 + i];
      idx += step;
    }
    const int64_t tail_start = end - end % 4;
    if (tail_ok && tail_start + x < end) a[0] = a[0] + d[tail_start + x] * d[tail_start + x];
    return ((a[0] + a[1]) + a[2]) + a[3];
  }
  /* thread_reduce_impl: vt0 = 4 accumulators over idx, idx + stride, ... */
  float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  int64_t idx = idx0;
  while (idx + 3 * step < n) {
    for (int i = 0; i < 4; ++i) a[i] = a[i] + q[idx + i * step] * q[idx + i * step];
    idx += 4 * step;
  }
  for (int i = 0; i < 4 && idx < n; ++i, idx += step) a[i] = a[i] + q[idx] * q[idx];
  return ((a[0] + a[1]) + a[2]) + a[3];
}

/* block_x_reduce over t[0..bw): a shared-memory halving down to 64 lanes,
 * then the shuffle-down tree with offsets 1, 2, 4, ... (lane 0's value). */
static float rms_block_x(float* t, int bw) {
  for (int off = bw / 2; off >= 64; off /= 2)
    for (int i = 0; i < off; ++i) t[i] = t[i] + t[i + off];
  const int w = bw < 64 ? bw : 64;
  for (int off = 1; off < w; off *= 2)
    for (int i = 0; i + off < w; i += 2 * off) t[i] = t[i] + t[i + off];
  return t[0];
}

/* torch's fp32 mean of squares of one row (HF:403), given the plan of the
 * whole [rows, n] tensor; factor is MeanOps' float(rows) / float(rows * n). */
static float rms_var_torch(const float* q, int64_t n, int shift, const rms_plan_t* p,
                           float factor, float* scratch) {
  float yv[16];
  const int nb = p->split ? p->bh : 1;
  for (int y = 0; y < nb; ++y) {
    for (int x = 0; x < p->bw; ++x) scratch[x] = rms_thread(q, n, shift, p, x, y);
    yv[y] = rms_block_x(scratch, p->bw);
  }
  for (int off = nb / 2; off > 0; off /= 2)  /* block_y_reduce */
    for (int y = 0; y < off; ++y) yv[y] = yv[y] + yv[y + off];
  return yv[0] * factor;
}

/* Normalised output of HF:404-405: bf16(w * bf16(x * rstd)). */
static void rms_out(const uint16_t* x, const uint16_t* w, uint16_t* y, int64_t n, float rstd) {
  for (int64_t j = 0; j < n; ++j) y[j] = f2bf(bf2f(w[j]) * rbf(bf2f(x[j]) * rstd));
}

/* RMSNorm of `rows` contiguous rows, HF:400-405 (Qwen3VLTextRMSNorm) with
 * torch-ROCm's reduction order; x is the bf16 input (for the add variant,
 * the rounded sum).  Returns -1 for shapes whose reduction spans blocks. */
static int rms_rows(const uint16_t* x, const uint16_t* w, uint16_t* y, int64_t rows,
                    int64_t n, float eps) {
  rms_plan_t p;
  if (rms_plan_for(rows, n, &p)) return -1;
  const float factor = (float)rows / (float)(rows * n);
  float* q = (float*)malloc((size_t)(n + 8) * sizeof(float));
  float* scratch = (float*)malloc(512 * sizeof(float));
  if (!q || !scratch) {
    free(q);
    free(scratch);
    return -2;
  }
  for (int64_t r = 0; r < rows; ++r) {
    const int shift = (int)((r * n) % 4);
    float* qr = q + 4;  /* room for the head elements before the row */
    for (int64_t j = 0; j < n; ++j) qr[j] = bf2f(x[r * n + j]);
    const float var = rms_var_torch(qr, n, p.vec ? shift : 0, &p, factor, scratch);
    rms_out(x + r * n, w, y + r * n, n, rsqrt_cr(var + eps));
  }
  free(q);
  free(scratch);
  return 0;
}

/* Reference kernel: kernels/rmsnorm.py:32-51; module chain HF:391-405. */
int orc_rmsnorm(const uint16_t* x, const uint16_t* w, uint16_t* y, int64_t rows, int64_t n,
                float eps) {
  return rms_rows(x, w, y, rows, n, eps);
}

/* The fp32 variance alone (for the statistic fixtures), same plan. */
int orc_rms_var(const uint16_t* x, float* var, int64_t rows, int64_t n) {
  rms_plan_t p;
  if (rms_plan_for(rows, n, &p)) return -1;
  const float factor = (float)rows / (float)(rows * n);
  float* q = (float*)malloc((size_t)(n + 8) * sizeof(float));
  float* scratch = (float*)malloc(512 * sizeof(float));
  if (!q || !scratch) {
    free(q);
    free(scratch);
    return -2;
  }
  for (int64_t r = 0; r < rows; ++r) {
    float* qr = q + 4;
    for (int64_t j = 0; j < n; ++j) qr[j] = bf2f(x[r * n + j]);
    var[r] = rms_var_torch(qr, n, p.vec ? (int)((r * n) % 4) : 0, &p, factor, scratch);
  }
  free(q);
  free(scratch);
  return 0;
}

/* Residual add then RMSNorm, as the eager decoder layer runs it:
 * `hidden_states = residual + hidden_states` (HF:559, one bf16 rounding)
 * followed by post_attention_layernorm (HF:563) on the ROUNDED sum.
 * Reference kernel: kernels/rmsnorm.py:75-101; caller integrate.py:205. */
int orc_add_rmsnorm(const uint16_t* x, const uint16_t* r, const uint16_t* w, uint16_t* normed,
                    uint16_t* summed, int64_t rows, int64_t n, float eps) {
  for (int64_t i = 0; i < rows * n; ++i) summed[i] = f2bf(bf2f(x[i]) + bf2f(r[i]));
  return rms_rows(summed, w, normed, rows, n, eps);
}

/* ---- LayerNorm --------------------------------------------------------- */

/* gfx950's v_rcp_f32 on integer counts and v_rsq_f32, as deltas (in ulps)
 * from the correctly rounded values, installed from the measured tables
 * (tests/golden/gfx950_rcp_rsq.npz) by orc_set_hw_tables. */
static const int8_t* g_rcp_delta;   /* n = 1 .. g_rcp_n */
static int64_t g_rcp_n;
static const uint8_t* g_rsq_delta2; /* 2 bits per float of [1, 4) */

void orc_set_hw_tables(const int8_t* rcp_delta, int64_t rcp_n, const uint8_t* rsq_delta2) {
  g_rcp_delta = rcp_delta;
  g_rcp_n = rcp_n;
  g_rsq_delta2 = rsq_delta2;
}

static inline float add_ulps(float v, int d) {
  int32_t u;
  memcpy(&u, &v, 4);
  u += d;
  memcpy(&v, &u, 4);
  return v;
}

/* Tests plant a mistake by clearing this: the Welford order with correctly
 * rounded reciprocals and rsqrt instead of the hardware instructions. */
static int g_use_hw = 1;

/* v_rcp_f32 of an integer count 1..g_rcp_n. */
static inline float hw_rcp_count(float c) {
  const int64_t n = (int64_t)c;
  const float cr = (float)(1.0 / (double)n);
  return g_use_hw ? add_ulps(cr, g_rcp_delta[n - 1]) : cr;
}

/* v_rsq_f32 of a positive normal float: the [1, 4) table scaled by the
 * exponent (the instruction is exactly exponent-scale invariant). */
static inline float hw_rsq(float v) {
  int e = 0;
  float m = frexpf(v, &e);  /* v = m * 2^e, m in [0.5, 1) */
  m = ldexpf(m, 1);
  e -= 1;                   /* m in [1, 2) */
  if (e & 1) {
    m = ldexpf(m, 1);
    e -= 1;                 /* m in [2, 4), e even */
  }
  uint32_t u;
  memcpy(&u, &m, 4);
  const uint32_t i = u - 0x3f800000u;
  const int d = (int)((g_rsq_delta2[i >> 2] >> ((i & 3) * 2)) & 3) - 1;
  return g_use_hw ? add_ulps(rsqrt_cr(v), d) : rsqrt_cr(v);
}

typedef struct {
  float mean, m2, n;
} wf_t;

/* One Welford step (cuWelfordOnlineSum): the mean update fused, the m2
 * update as two roundings. */
static inline wf_t wf_push(wf_t a, float v) {
  const float delta = v - a.mean;
  const float cnt = a.n + 1.0f;
  const float mean = fmaf(delta, hw_rcp_count(cnt), a.mean);
  const float m2 = a.m2 + delta * (v - mean);
  return (wf_t){mean, m2, cnt};
}

/* cuWelfordCombine(b = own, a = other).  The ROCm build contracts the mean
 * as fma(nA, meanA, nB * meanB) in the wavefront tree and as
 * fma(nB, meanB, nA * meanA) in the cross-wavefront tree (`intra`
 * selects); the m2 term as fma(delta^2 * countA, nB, m2A + m2B). */
static inline wf_t wf_combine(wf_t b, wf_t a, int intra) {
  const float delta = b.mean - a.mean;
  const float cnt = a.n + b.n;
  if (!(cnt > 0.0f)) return (wf_t){0.0f, 0.0f, cnt};
  const float coef = hw_rcp_count(cnt);
  const float na = a.n * coef, nb = b.n * coef;
  const float mean = intra ? fmaf(na, a.mean, nb * b.mean) : fmaf(nb, b.mean, na * a.mean);
  const float m2 = fmaf((delta * delta) * a.n, nb, a.m2 + b.m2);
  return (wf_t){mean, m2, cnt};
}

/* torch-ROCm's LayerNorm statistics of one bf16 row (n % 4 == 0): 256
 * threads (4 wavefronts of 64), thread t pushes the 4-element vectors
 * t, t + 256, ... in order; shuffle-down tree per wavefront (offsets 32 .. 1,
 * lane 0 keeps the result), then the wavefront tree (offsets 2, 1);
 * var = m2 / n (correctly rounded), rstd = v_rsq_f32(var + eps). */
static void ln_stats_torch(const uint16_t* x, int64_t n, float eps, float* mean, float* rstd) {
  wf_t t[256];
  const int64_t nv = n / 4;
  for (int i = 0; i < 256; ++i) t[i] = (wf_t){0.0f, 0.0f, 0.0f};
  for (int64_t v = 0; v < nv; ++v)
    for (int e = 0; e < 4; ++e) t[v % 256] = wf_push(t[v % 256], bf2f(x[v * 4 + e]));
  wf_t wv[4];
  for (int w = 0; w < 4; ++w) {
    wf_t* s = t + 64 * w;
    for (int off = 32; off > 0; off /= 2)
      for (int i = 0; i < off; ++i) s[i] = wf_combine(s[i], s[i + off], 1);
    wv[w] = s[0];
  }
  for (int off = 2; off > 0; off /= 2)
    for (int i = 0; i < off; ++i) wv[i] = wf_combine(wv[i], wv[i + off], 0);
  *mean = wv[0].mean;
  *rstd = hw_rsq(wv[0].m2 / (float)n + eps);
}

/* torch-ROCm's other LayerNorm statistics kernel (RowwiseMomentsCUDAKernel),
 * which eager runs when the vectorized one cannot (n % 4 != 0, or x, w, b
 * off 8-byte alignment): 512 threads per row (8 wavefronts), thread t folds
 * elements t, t + 512, ... with WelfordOps::reduce (ATen/native/
 * SharedReduceOps.h: new_mean = mean + delta / n, m2 += delta * (x -
 * new_mean)), then cuda_utils::BlockReduce (ATen/native/hip/block_reduce.cuh):
 * a shuffle-down tree per wavefront with WelfordOps::combine(own, other)
 * (delta = b.mean - a.mean, nb/n = b.n / (a.n + b.n), mean = a.mean +
 * delta * nb/n, m2 = a.m2 + b.m2 + delta^2 * a.n * nb/n; an empty side
 * returns the other), lane 0 of each into shared memory, then the same tree
 * over the 8 wavefront results (the other 56 lanes the empty identity);
 * var = m2 / n, rstd = rsqrt(var + eps).  `variant` bits select the
 * arithmetic forms fitted against eager's recorded statistics:
 *   1: the reduce's division as fma(delta, v_rcp_f32(n), mean), not a/b
 *   2: the reduce's m2 term contracted to an fma
 *   4: the combine's mean and m2 terms contracted to fmas
 *   8: the combine's nb/n as b.n * v_rcp_f32(n)
 *  16: rsqrt as v_rsq_f32 (else correctly rounded)
 *  32: 256 threads per row instead of 512 (a planted mistake) */
typedef struct {
  float mean, m2, nf;
} wfs_t;

static wfs_t wfs_reduce(wfs_t a, float x, int variant) {
  const float nf = a.nf + 1.0f;
  const float delta = x - a.mean;
  const float mean = (variant & 1) ? fmaf(delta, hw_rcp_count(nf), a.mean) : a.mean + delta / nf;
  const float nd = x - mean;
  const float m2 = (variant & 2) ? fmaf(delta, nd, a.m2) : a.m2 + delta * nd;
  return (wfs_t){mean, m2, nf};
}

static wfs_t wfs_combine(wfs_t a, wfs_t b, int variant) {
  if (a.nf == 0.0f) return b;
  if (b.nf == 0.0f) return a;
  const float delta = b.mean - a.mean;
  const float cnt = a.nf + b.nf;
  const float nbn = (variant & 8) ? b.nf * hw_rcp_count(cnt) : b.nf / cnt;
  float mean, m2;
  if (variant & 4) {
    mean = fmaf(delta, nbn, a.mean);
    m2 = fmaf((delta * delta) * a.nf, nbn, a.m2 + b.m2);
  } else {
    mean = a.mean + delta * nbn;
    m2 = (a.m2 + b.m2) + ((delta * delta) * a.nf) * nbn;
  }
  return (wfs_t){mean, m2, cnt};
}

static void wfs_warp(wfs_t* v, int variant) {  /* 64 lanes, lane 0 keeps the result */
  for (int off = 32; off > 0; off /= 2)
    for (int i = 0; i < off; ++i) v[i] = wfs_combine(v[i], v[i + off], variant);
}

static void ln_stats_torch_scalar(const uint16_t* x, int64_t n, float eps, int variant,
                                  float* mean, float* rstd) {
  const int threads = (variant & 32) ? 256 : 512, waves = threads / 64;
  wfs_t t[512];
  for (int i = 0; i < threads; ++i) t[i] = (wfs_t){0.0f, 0.0f, 0.0f};
  for (int64_t j = 0; j < n; ++j) t[j % threads] = wfs_reduce(t[j % threads], bf2f(x[j]), variant);
  wfs_t s[64];
  for (int w = 0; w < waves; ++w) {
    wfs_warp(t + 64 * w, variant);
    s[w] = t[64 * w];
  }
  for (int i = waves; i < 64; ++i) s[i] = (wfs_t){0.0f, 0.0f, 0.0f};
  wfs_warp(s, variant);
  *mean = s[0].mean;
  const float var = s[0].m2 / s[0].nf;
  *rstd = (variant & 16) ? hw_rsq(var + eps) : rsqrt_cr(var + eps);
}

/* The forms eager's kernel takes on gfx950 (fitted: every recorded mean and
 * rstd of the scalar-path fixtures bit for bit): a / b divisions, the
 * reduce's and the combine's m2 and mean updates contracted, v_rsq_f32. */
#define LN_SCALAR_EAGER (2 | 4 | 16)

/* Test entry: the statistics above for rows of n, in one of the variants
 * (LN_SCALAR_EAGER is eager's; the others are planted mistakes). */
int orc_ln_scalar_stats(const uint16_t* x, float* mean, float* rstd, int64_t rows, int64_t n,
                        float eps, int variant) {
  if (!g_rcp_delta || !g_rsq_delta2 || n > g_rcp_n || n <= 0) return -1;
  g_use_hw = 1;
  for (int64_t r = 0; r < rows; ++r) ln_stats_torch_scalar(x + r * n, n, eps, variant, mean + r,
                                                          rstd + r);
  return 0;
}

/* Exact statistics (double sums of x and x^2 of bf16 data, rounded once;
 * rsqrt correctly rounded): a planted mistake for the tests, which show that
 * eager's kernels round differently on some rows. */
static void ln_stats_exact(const uint16_t* x, int64_t n, float eps, float* mean, float* rstd) {
  double s = 0.0, q = 0.0;
  for (int64_t j = 0; j < n; ++j) {
    const float f = bf2f(x[j]);
    s += (double)f;
    q += (double)(f * f);
  }
  const double mean_d = s / (double)n;
  *mean = (float)mean_d;
  *rstd = rsqrt_cr((float)(q / (double)n - mean_d * mean_d) + eps);
}

/* Affine output of torch's layer_norm: bf16(fma(w, rstd * (x - mean), b)). */
static void ln_out(const uint16_t* x, const uint16_t* w, const uint16_t* b, uint16_t* y,
                   int64_t n, float mean, float rstd) {
  for (int64_t j = 0; j < n; ++j)
    y[j] = f2bf(fmaf(bf2f(w[j]), rstd * (bf2f(x[j]) - mean), bf2f(b[j])));
}

/* torch.nn.functional.layer_norm on bf16 rows with bf16 affine params
 * (nn.LayerNorm in the ViT blocks, HF:283-284).  torch_order 1 selects the
 * vectorized kernel's statistics (needs n % 4 == 0 and the tables), 3 the
 * scalar kernel's (eager's choice for other widths and misaligned rows),
 * 0 the exact ones and 2 the vectorized order with correctly rounded
 * reciprocals (both planted mistakes for the tests).  mean/rstd may be NULL.
 * Reference kernel: kernels/layernorm.py:30-52. */
int orc_layernorm(const uint16_t* x, const uint16_t* w, const uint16_t* b, uint16_t* y,
                  float* mean, float* rstd, int64_t rows, int64_t n, float eps,
                  int torch_order) {
  if (torch_order == 3) {
    if (!g_rsq_delta2 || n <= 0) return -1;
  } else if (torch_order && (n % 4 || !g_rcp_delta || !g_rsq_delta2 || n > g_rcp_n)) {
    return -1;
  }
  g_use_hw = torch_order != 2;
  for (int64_t r = 0; r < rows; ++r) {
    float mu, rs;
    if (torch_order == 3) ln_stats_torch_scalar(x + r * n, n, eps, LN_SCALAR_EAGER, &mu, &rs);
    else if (torch_order) ln_stats_torch(x + r * n, n, eps, &mu, &rs);
    else ln_stats_exact(x + r * n, n, eps, &mu, &rs);
    if (mean) mean[r] = mu;
    if (rstd) rstd[r] = rs;
    ln_out(x + r * n, w, b, y + r * n, n, mu, rs);
  }
  return 0;
}

/* Vision-block residual add then LayerNorm: `hidden_states = hidden_states
 * + attn(...)` (HF:299-304, bf16 rounding) then norm2 on the rounded sum
 * (HF:305).  Reference kernel: kernels/layernorm.py:70-100; callers
 * integrate.py:581-582, 589-590, 602-603. */
int orc_add_layernorm(const uint16_t* x, const uint16_t* r, const uint16_t* w,
                      const uint16_t* b, uint16_t* normed, uint16_t* summed, int64_t rows,
                      int64_t n, float eps, int torch_order) {
  for (int64_t i = 0; i < rows * n; ++i) summed[i] = f2bf(bf2f(x[i]) + bf2f(r[i]));
  return orc_layernorm(summed, w, b, normed, NULL, NULL, rows, n, eps, torch_order);
}

/* ---- RoPE -------------------------------------------------------------- */

/* Text RoPE, HF:412-435 (apply_rotary_pos_emb) with rotate_half HF:138-142,
 * on bf16 q and bf16 cos/sin (HF:370 casts them to the activation dtype):
 *   out = bf16( bf16(x * cos) + bf16(rotate_half(x) * sin) )
 * Every product and the sum round to bf16 (each is a separate bf16 op).
 * x, out: [S, H, D] contiguous; cos, sin: [S, D].
 * Reference kernel: kernels/rope.py:30-60 via make_text_rope :86-107. */
void orc_rope_text(const uint16_t* x, const uint16_t* cos_, const uint16_t* sin_,
                   uint16_t* out, int64_t S, int64_t H, int64_t D) {
  int64_t half = D / 2;
  for (int64_t s = 0; s < S; ++s)
    for (int64_t h = 0; h < H; ++h) {
      const uint16_t* xr = x + (s * H + h) * D;
      uint16_t* o = out + (s * H + h) * D;
      for (int64_t d = 0; d < D; ++d) {
        float xd = bf2f(xr[d]);
        float rot = d < half ? -bf2f(xr[d + half]) : bf2f(xr[d - half]);
        float a = rbf(xd * bf2f(cos_[s * D + d]));
        float b = rbf(rot * bf2f(sin_[s * D + d]));
        o[d] = f2bf(a + b);
      }
    }
}

/* Vision RoPE, HF:145-156 (apply_rotary_pos_emb_vision): q.float(), fp32
 * cos/sin, (q*cos) + (rotate_half(q)*sin) as three separately rounded fp32
 * ops, then .to(bf16).  x, out: [S, H, D] contiguous; cos, sin: [S, D] fp32.
 * Reference kernel: kernels/rope.py:30-60 via apply_rotary_vision_triton
 * :78-84. */
void orc_rope_vision(const uint16_t* x, const float* cos_, const float* sin_,
                     uint16_t* out, int64_t S, int64_t H, int64_t D) {
  int64_t half = D / 2;
  for (int64_t s = 0; s < S; ++s)
    for (int64_t h = 0; h < H; ++h) {
      const uint16_t* xr = x + (s * H + h) * D;
      uint16_t* o = out + (s * H + h) * D;
      for (int64_t d = 0; d < D; ++d) {
        float xd = bf2f(xr[d]);
        float rot = d < half ? -bf2f(xr[d + half]) : bf2f(xr[d - half]);
        float a = xd * cos_[s * D + d];
        float b = rot * sin_[s * D + d];
        o[d] = f2bf(a + b);
      }
    }
}

/* ---- GEMMs ------------------------------------------------------------- */

/* out[m, n] = sum_k x[m, k] * w[n, k] accumulated in double, rounded once to
 * fp32.  x: [M, K], w: [N, K] (nn.Linear layout), out: [M, N] fp32. */
void orc_gemm_nt_f32(const uint16_t* x, const uint16_t* w, float* out,
                     int64_t M, int64_t N, int64_t K) {
  for (int64_t m = 0; m < M; ++m)
    for (int64_t n = 0; n < N; ++n) {
      double acc = 0.0;
      const uint16_t* xr = x + m * K;
      const uint16_t* wr = w + n * K;
      for (int64_t k = 0; k < K; ++k) acc += (double)bf2f(xr[k]) * (double)bf2f(wr[k]);
      out[m * N + n] = (float)acc;
    }
}

static inline float silu_f(float g) { return g / (1.0f + expf(-g)); }
static inline float gelu_erf_f(float v) {
  return 0.5f * v * (1.0f + erff(v * 0.70710678118654752f));
}
/* torch's gelu(approximate="tanh") in fp32 (HF gelu_pytorch_tanh), with its
 * operation order: inner = sqrt(2/pi) * (v + 0.044715 * v^3). */
static inline float gelu_tanh_f(float v) {
  const float cube = v * v * v;
  const float inner = 0.7978845608028654f * (v + 0.044715f * cube);
  return 0.5f * v * (1.0f + tanhf(inner));
}

/* P5: silu(x @ wg^T) * (x @ wu^T).
 * fused = 1: the reference kernel's numerics, kernels/fused_ffn.py:71-91
 *   (fp32 accumulators, silu*mul in fp32, ONE bf16 rounding).
 * fused = 0: the eager chain HF:522 / kernels/fused_ffn.py:31-43
 *   (gate and up GEMM outputs rounded to bf16, silu rounded, product rounded).
 * wg, wu: [N, K]. */
void orc_gate_silu_mul(const uint16_t* x, const uint16_t* wg, const uint16_t* wu,
                       uint16_t* out, int64_t M, int64_t N, int64_t K, int fused) {
  for (int64_t m = 0; m < M; ++m)
    for (int64_t n = 0; n < N; ++n) {
      double ag = 0.0, au = 0.0;
      const uint16_t* xr = x + m * K;
      const uint16_t* gr = wg + n * K;
      const uint16_t* ur = wu + n * K;
      for (int64_t k = 0; k < K; ++k) {
        double xv = (double)bf2f(xr[k]);
        ag += xv * (double)bf2f(gr[k]);
        au += xv * (double)bf2f(ur[k]);
      }
      float g = (float)ag, u = (float)au;
      if (fused) {
        out[m * N + n] = f2bf(silu_f(g) * u);
      } else {
        float gs = rbf(silu_f(rbf(g)));
        out[m * N + n] = f2bf(gs * rbf(u));
      }
    }
}

/* Linear with optional bias and erf-GELU epilogue, reference kernel
 * kernels/linear.py:32-90 (acc + bias, GELU, one rounding).
 * fused = 0 restates the eager pair F.linear -> bf16, then GELU -> bf16.
 * bias may be NULL.  act: 0 none, 1 erf GELU, 2 tanh-approximate GELU (the
 * activation of the Qwen3-VL ViT MLP; the reference's epilogue has no such
 * mode, kernels/linear.py:83-86 always applies the erf form). */
void orc_linear(const uint16_t* x, const uint16_t* w, const uint16_t* bias,
                uint16_t* out, int64_t M, int64_t N, int64_t K, int act,
                int fused) {
  for (int64_t m = 0; m < M; ++m)
    for (int64_t n = 0; n < N; ++n) {
      double acc = 0.0;
      const uint16_t* xr = x + m * K;
      const uint16_t* wr = w + n * K;
      for (int64_t k = 0; k < K; ++k) acc += (double)bf2f(xr[k]) * (double)bf2f(wr[k]);
      float v = (float)acc;
      if (bias) v = v + bf2f(bias[n]);
      if (!fused) v = rbf(v);
      if (act == 1) v = gelu_erf_f(v);
      if (act == 2) v = gelu_tanh_f(v);
      out[m * N + n] = f2bf(v);
    }
}
