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
 * Row statistics (sum of squares, mean, variance) are accumulated in double
 * and rounded once to fp32; rsqrt is 1/sqrt evaluated in double then
 * rounded.  For bf16 data the double sums are exact, so these are the
 * correctly rounded fp32 statistics whatever the summation order.  An eager fp32
 * reduction lands within a few fp32 ulps of these, which moves a bf16 output
 * by at most one ulp in rare ties (tests/test_oracle.py measures this
 * against torch directly).
 *
 * bf16 values travel as uint16_t bit patterns.
 */
#include <math.h>
#include <stdint.h>
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

/* ---- RMSNorm ----------------------------------------------------------- */

/* One row of HF:400-405 (Qwen3VLTextRMSNorm.forward):
 *   h = x.float(); var = h.pow(2).mean(-1); h = h * rsqrt(var + eps)
 *   return weight * h.to(bf16)
 * x*x of a bf16 value is exact in fp32, so the double sum is exact. */
static void rms_row(const uint16_t* x, const uint16_t* w, uint16_t* y,
                    int64_t n, float eps) {
  double ss = 0.0;
  for (int64_t j = 0; j < n; ++j) {
    float f = bf2f(x[j]);
    ss += (double)(f * f);
  }
  float var = (float)(ss / (double)n);
  float rstd = rsqrt_cr(var + eps);
  for (int64_t j = 0; j < n; ++j) {
    float h = rbf(bf2f(x[j]) * rstd);
    y[j] = f2bf(bf2f(w[j]) * h);
  }
}

/* Reference kernel: kernels/rmsnorm.py:32-51; module chain HF:391-405. */
void orc_rmsnorm(const uint16_t* x, const uint16_t* w, uint16_t* y,
                 int64_t rows, int64_t n, float eps) {
  for (int64_t i = 0; i < rows; ++i) rms_row(x + i * n, w, y + i * n, n, eps);
}

/* Residual add then RMSNorm, as the eager decoder layer runs it:
 * `hidden_states = residual + hidden_states` (HF:559, one bf16 rounding)
 * followed by post_attention_layernorm (HF:563) on the ROUNDED sum.
 * Reference kernel: kernels/rmsnorm.py:75-101; caller integrate.py:205. */
void orc_add_rmsnorm(const uint16_t* x, const uint16_t* r, const uint16_t* w,
                     uint16_t* normed, uint16_t* summed,
                     int64_t rows, int64_t n, float eps) {
  for (int64_t i = 0; i < rows; ++i) {
    uint16_t* s = summed + i * n;
    for (int64_t j = 0; j < n; ++j)
      s[j] = f2bf(bf2f(x[i * n + j]) + bf2f(r[i * n + j]));
    rms_row(s, w, normed + i * n, n, eps);
  }
}

/* ---- LayerNorm --------------------------------------------------------- */

/* torch.nn.functional.layer_norm on a bf16 row with bf16 affine params
 * (nn.LayerNorm in the ViT blocks, HF:283-284, eps 1e-6): fp32 mean and
 * biased variance, rstd = rsqrt(var + eps), and the per-element affine
 * y = w * (rstd * (x - mean)) + b contracted to one fma, rounded once.
 * Statistics: exact double sums of x and x^2 (x^2 of a bf16 is exact in
 * fp32), mean = sum/n and var = sumsq/n - mean^2 in double, each rounded
 * once to fp32. */
static void ln_row(const uint16_t* x, const uint16_t* w, const uint16_t* b,
                   uint16_t* y, int64_t n, float eps) {
  double s = 0.0, q = 0.0;
  for (int64_t j = 0; j < n; ++j) {
    float f = bf2f(x[j]);
    s += (double)f;
    q += (double)(f * f);
  }
  double mean_d = s / (double)n;
  float mean = (float)mean_d;
  float var = (float)(q / (double)n - mean_d * mean_d);
  float rstd = rsqrt_cr(var + eps);
  for (int64_t j = 0; j < n; ++j) {
    float t = rstd * (bf2f(x[j]) - mean);
    y[j] = f2bf(fmaf(bf2f(w[j]), t, bf2f(b[j])));
  }
}

/* Reference kernel: kernels/layernorm.py:30-52. */
void orc_layernorm(const uint16_t* x, const uint16_t* w, const uint16_t* b,
                   uint16_t* y, int64_t rows, int64_t n, float eps) {
  for (int64_t i = 0; i < rows; ++i) ln_row(x + i * n, w, b, y + i * n, n, eps);
}

/* Vision-block residual add then LayerNorm: `hidden_states = hidden_states
 * + attn(...)` (HF:299-304, bf16 rounding) then norm2 on the rounded sum
 * (HF:305).  Reference kernel: kernels/layernorm.py:70-100; callers
 * integrate.py:581-582, 589-590, 602-603. */
void orc_add_layernorm(const uint16_t* x, const uint16_t* r, const uint16_t* w,
                       const uint16_t* b, uint16_t* normed, uint16_t* summed,
                       int64_t rows, int64_t n, float eps) {
  for (int64_t i = 0; i < rows; ++i) {
    uint16_t* s = summed + i * n;
    for (int64_t j = 0; j < n; ++j)
      s[j] = f2bf(bf2f(x[i * n + j]) + bf2f(r[i * n + j]));
    ln_row(s, w, b, normed + i * n, n, eps);
  }
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
