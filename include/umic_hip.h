/*
 * umic_hip.h -- C ABI of libumic_hip.so, the MI355X (gfx950) kernel library
 * behind the UMIC fused hot path.
 *
 * Every entry point is a plain C function over device pointers and sizes:
 * no torch types, no allocation, no synchronisation, no host reads of device
 * memory.  Each call enqueues its kernel(s) on `stream` (a hipStream_t passed
 * as void*, NULL = the legacy default stream) and returns immediately, so
 * the calls are safe inside HIP stream / graph capture.
 *
 * Conventions
 *   - bf16 tensors are passed as raw 16-bit storage (uint16_t bit patterns).
 *   - Leading dimensions / strides are in ELEMENTS, not bytes.  The innermost
 *     dimension of every tensor is contiguous (stride 1).
 *   - Return value: UMIC_OK (0) on success; a negative UMIC_ERR_* code when
 *     the arguments are rejected before any launch (nothing was enqueued);
 *     a positive hipError_t value when the launch itself failed.
 *     umic_error_string() names either kind.  The library never aborts.
 *   - Numerics follow the eager PyTorch / HF transformers op chains that the
 *     reference's Triton kernels replace (rounding points noted per call).
 *
 * Reference interfaces (soonhong99/umic-alpamayo, path:line under src/umic/)
 * that each call replaces are cited on its declaration.
 */
#ifndef UMIC_HIP_H
#define UMIC_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define UMIC_OK 0
#define UMIC_ERR_INVALID_ARG (-1)  /* null pointer, negative size, bad enum */
#define UMIC_ERR_UNSUPPORTED (-2)  /* shape / stride / alignment not handled */
#define UMIC_ERR_SCRATCH (-3)      /* shape needs more than the static scratch */

/* Byte offset, in a stream-K workspace, of its sticky status word (int32):
 * 0 while every split tile's reduction has completed; 1 + t after the last
 * workgroup to reach tile t gave up waiting for the tile's other segments
 * (a bounded wait of well under a second: the workspace's counters were
 * inconsistent, e.g. calls overlapping on one workspace).  Tile t's output
 * is then left unwritten and its counters reset; the launch ends normally.
 * No launch clears the word: the caller reads it (and clears it) when it
 * wants to know. */
#define UMIC_SK_STATUS_OFFSET 8192

/* Library version string, e.g. "umic-hip 0.1.0 gfx950". */
const char* umic_version(void);

/* Human-readable text for a return code of any entry point. */
const char* umic_error_string(int code);

/*
 * RMSNorm over the last dim, one row of n elements per output row.
 *   y[i,:] = bf16( w * bf16( x[i,:] * rsqrt(mean(x[i,:]^2) + eps) ) )
 * i.e. the HF Qwen3VLTextRMSNorm chain (normalise in fp32, round to bf16,
 * then multiply by the bf16 weight and round again).
 * x: [rows, n] row stride ldx; w: [n]; y: [rows, n] row stride ldy.
 * Replaces: kernels/rmsnorm.py:53-73 (rmsnorm_triton) and its kernel
 * kernels/rmsnorm.py:32-51; caller integrate.py:134-141.
 */
int umic_rmsnorm_bf16(const void* x, const void* w, void* y,
                      int64_t rows, int64_t n, int64_t ldx, int64_t ldy,
                      float eps, void* stream);

/*
 * Residual add fused into RMSNorm.
 *   summed = bf16(x + r);  normed = rmsnorm(summed) as above.
 * Outputs both the normalised MLP input and the new residual stream.
 * Replaces: kernels/rmsnorm.py:103-134 (add_rmsnorm_triton), kernel
 * kernels/rmsnorm.py:75-101; caller integrate.py:205-206.
 */
int umic_add_rmsnorm_bf16(const void* x, const void* r, const void* w,
                          void* normed, void* summed,
                          int64_t rows, int64_t n,
                          int64_t ldx, int64_t ldr, int64_t ldn, int64_t lds,
                          float eps, void* stream);

/*
 * LayerNorm over the last dim with affine weight and bias (biased variance).
 *   y = bf16( fma(w, rstd * (x - mean), b) ),  fp32 statistics.
 * Replaces: kernels/layernorm.py:54-68 (layernorm_triton), kernel
 * kernels/layernorm.py:30-52; caller integrate.py:234-238.
 */
int umic_layernorm_bf16(const void* x, const void* w, const void* b, void* y,
                        int64_t rows, int64_t n, int64_t ldx, int64_t ldy,
                        float eps, void* stream);

/*
 * Residual add fused into LayerNorm.
 *   summed = bf16(x + r);  normed = layernorm(summed) as above.
 * Replaces: kernels/layernorm.py:102-124 (add_layernorm_triton), kernel
 * kernels/layernorm.py:70-100; callers integrate.py:581-582,589-590,602-603.
 */
int umic_add_layernorm_bf16(const void* x, const void* r, const void* w,
                            const void* b, void* normed, void* summed,
                            int64_t rows, int64_t n,
                            int64_t ldx, int64_t ldr, int64_t ldn, int64_t lds,
                            float eps, void* stream);

/* RoPE arithmetic modes for umic_rope_qk_bf16. */
#define UMIC_ROPE_TEXT 0   /* every op rounded to bf16 (HF apply_rotary_pos_emb) */
#define UMIC_ROPE_VISION 1 /* fp32 math, one rounding (HF apply_rotary_pos_emb_vision) */

/*
 * Rotary position embedding of q and k in ONE launch (cos/sin read once).
 *   out[..., d] = x[..., d] * cos[d] + rotate_half(x)[..., d] * sin[d]
 *   rotate_half(x) = cat(-x[..., D/2:], x[..., :D/2])
 * Tensors are addressed as [B, S, H, D] with arbitrary element strides for
 * the batch (sb), position (ss) and head (sh) dims; D is contiguous.
 *   q, q_out: B x S x Hq x D; k, k_out: B x S x Hk x D (Hk may be 0, then
 *   k / k_out are ignored);  cos, sin: B x S x D with strides (cs_sb, cs_ss).
 * cs_fp32 = 1: cos/sin are fp32, else bf16.  mode UMIC_ROPE_TEXT requires
 * bf16 cos/sin.  D must be even.
 * Replaces: kernels/rope.py:62-76 (_apply_one, launched once per tensor),
 * kernels/rope.py:78-84 (apply_rotary_vision_triton) and
 * kernels/rope.py:86-107 (make_text_rope); kernel kernels/rope.py:30-60.
 */
int umic_rope_qk_bf16(const void* q, const void* k, void* q_out, void* k_out,
                      const void* cos, const void* sin, int cs_fp32, int mode,
                      int64_t B, int64_t S, int64_t Hq, int64_t Hk, int64_t D,
                      int64_t q_sb, int64_t q_ss, int64_t q_sh,
                      int64_t k_sb, int64_t k_ss, int64_t k_sh,
                      int64_t qo_sb, int64_t qo_ss, int64_t qo_sh,
                      int64_t ko_sb, int64_t ko_ss, int64_t ko_sh,
                      int64_t cs_sb, int64_t cs_ss, void* stream);

/*
 * Text RoPE fused with the append into an in-place KV cache, one launch:
 *   q_out            = rope(q)   [B, S, Hq, D], strides (qo_sb, qo_ss, qo_sh)
 *   k_cache[b,h,P+s] = rope(k)   cache [B, Hk, capacity, D],
 *   v_cache[b,h,P+s] = v         strides (c_sb, c_sh, c_ss), shared by both
 * with P = pos + (*pos_dev if pos_dev is non-NULL; a device int64, so one
 * captured graph can append at a new position on every replay).  Rotation
 * numerics are UMIC_ROPE_TEXT's (bf16 cos/sin, every op rounded to bf16),
 * bit-identical to umic_rope_qk_bf16; v is moved bit for bit.  q, k, v are
 * [B, S, H, D] with element strides (sb, ss, sh) like umic_rope_qk_bf16.
 * Requires D % 16 == 0, every stride a multiple of 8 elements and 16-byte
 * aligned pointers (else UMIC_ERR_UNSUPPORTED).  Without pos_dev, a write
 * past the cache (pos < 0 or pos + S > capacity) is UMIC_ERR_INVALID_ARG
 * and nothing is enqueued; with pos_dev, cache rows outside [0, capacity)
 * are not written.
 * Replaces: kernels/rope.py:86-107 (make_text_rope) followed by the cache
 * append of cache.py:50-80 (InplaceLayer.update: slice assignment, or
 * index_copy_ at a device position in graph mode, cache.py:53-63), as
 * called from HF Qwen3VLTextAttention.forward (apply_rotary_pos_emb, then
 * past_key_values.update).
 */
int umic_rope_kv_append_bf16(const void* q, const void* k, const void* v,
                             void* q_out, void* k_cache, void* v_cache,
                             const void* cos, const void* sin,
                             int64_t B, int64_t S, int64_t Hq, int64_t Hk, int64_t D,
                             int64_t q_sb, int64_t q_ss, int64_t q_sh,
                             int64_t k_sb, int64_t k_ss, int64_t k_sh,
                             int64_t v_sb, int64_t v_ss, int64_t v_sh,
                             int64_t qo_sb, int64_t qo_ss, int64_t qo_sh,
                             int64_t c_sb, int64_t c_sh, int64_t c_ss, int64_t capacity,
                             int64_t pos, const int64_t* pos_dev,
                             int64_t cs_sb, int64_t cs_ss, void* stream);

/*
 * The text attention's per-head RMSNorm (q_norm, k_norm) fused into the text
 * RoPE: each head row of q and k is normalised,
 *   y = bf16( w * bf16( x * rsqrt(mean(x^2) + eps) ) )   (HF
 *   Qwen3VLTextRMSNorm, the umic_rmsnorm_bf16 numerics, w = q_w or k_w, [D]),
 * then rotated as umic_rope_qk_bf16 in UMIC_ROPE_TEXT mode, in one launch:
 * q and k are read once and written once.  Same arguments as
 * umic_rope_qk_bf16 (TEXT mode, bf16 cos/sin) plus the two norm weights and
 * eps.  Requires D = 128 or 256 (head sizes whose eager q_norm / k_norm
 * reduction order the kernel reproduces), every stride a multiple of 8
 * elements and 16-byte aligned pointers, weights included (else
 * UMIC_ERR_UNSUPPORTED).  Results are bit-identical to umic_rmsnorm_bf16 on
 * the [B*S*Hq, D] q rows and [B*S*Hk, D] k rows followed by
 * umic_rope_qk_bf16, and to the eager chain.
 * Replaces: the q_norm / k_norm forwards (integrate.py:134-141 on the
 * q_norm / k_norm modules of HF Qwen3VLTextAttention) followed by
 * kernels/rope.py:86-107 (make_text_rope) -- three launches.
 */
int umic_qk_rmsnorm_rope_bf16(const void* q, const void* k, void* q_out, void* k_out,
                              const void* q_w, const void* k_w, float eps,
                              const void* cos, const void* sin,
                              int64_t B, int64_t S, int64_t Hq, int64_t Hk, int64_t D,
                              int64_t q_sb, int64_t q_ss, int64_t q_sh,
                              int64_t k_sb, int64_t k_ss, int64_t k_sh,
                              int64_t qo_sb, int64_t qo_ss, int64_t qo_sh,
                              int64_t ko_sb, int64_t ko_ss, int64_t ko_sh,
                              int64_t cs_sb, int64_t cs_ss, void* stream);

/*
 * umic_rope_kv_append_bf16 with the q / k head-row RMSNorm of
 * umic_qk_rmsnorm_rope_bf16 applied before the rotation (v is copied
 * unchanged): the text attention's q_norm, k_norm, RoPE and in-place cache
 * append in one launch.  Arguments as umic_rope_kv_append_bf16, with the
 * norm weights (q_w, k_w: [D] bf16, 16-byte aligned) and eps after sin; the
 * same shape rules as both.
 * Replaces: the q_norm / k_norm forwards, kernels/rope.py:86-107 and the
 * cache append of cache.py:50-80.
 */
int umic_qk_rmsnorm_rope_kv_append_bf16(const void* q, const void* k, const void* v,
                                        void* q_out, void* k_cache, void* v_cache,
                                        const void* cos, const void* sin,
                                        const void* q_w, const void* k_w, float eps,
                                        int64_t B, int64_t S, int64_t Hq, int64_t Hk, int64_t D,
                                        int64_t q_sb, int64_t q_ss, int64_t q_sh,
                                        int64_t k_sb, int64_t k_ss, int64_t k_sh,
                                        int64_t v_sb, int64_t v_ss, int64_t v_sh,
                                        int64_t qo_sb, int64_t qo_ss, int64_t qo_sh,
                                        int64_t c_sb, int64_t c_sh, int64_t c_ss,
                                        int64_t capacity, int64_t pos, const int64_t* pos_dev,
                                        int64_t cs_sb, int64_t cs_ss, void* stream);

/* Epilogue activations for umic_linear_bf16. */
#define UMIC_ACT_NONE 0
#define UMIC_ACT_GELU 1      /* exact erf GELU */
#define UMIC_ACT_GELU_TANH 2 /* tanh-approximate GELU (torch approximate="tanh") */

/*
 * out = act(x @ w^T + bias), bf16 in/out, fp32 accumulation on MFMA.
 * x: [M, K] row stride ldx; w: [N, K] (nn.Linear layout) row stride ldw;
 * bias: [N] bf16 or NULL; out: [M, N] row stride ldo.
 * act: UMIC_ACT_NONE, UMIC_ACT_GELU (the reference's act="gelu") or
 * UMIC_ACT_GELU_TANH (no counterpart in the reference: the tanh GELU of the
 * Qwen3-VL ViT MLP); the bias add and the activation run in fp32 on the
 * accumulator, one bf16 rounding.  Any other act: UMIC_ERR_INVALID_ARG.
 * M <= 8 (decode) runs a weight-streaming GEMV kernel instead of the MFMA
 * tiles; same arguments, results and epilogue numerics (fp32 sums in
 * another order).
 * Requires K % 32 == 0, N % 8 == 0, ldx/ldw/ldo % 8 == 0 and 16-byte
 * aligned pointers (else UMIC_ERR_UNSUPPORTED).
 * Replaces: kernels/linear.py:118-145 (linear_triton), kernel
 * kernels/linear.py:32-90; caller integrate.py:98-107.
 */
int umic_linear_bf16(const void* x, const void* w, const void* bias, void* out,
                     int64_t M, int64_t N, int64_t K,
                     int64_t ldx, int64_t ldw, int64_t ldo,
                     int act, void* stream);

/*
 * Bytes of device workspace umic_linear_ws_bf16 uses for this shape on the
 * current device: nonzero when the output's 256 x 256 tiles leave enough of
 * the device's CUs idle and the K loop is long (then a stream-K schedule
 * spreads the K loop over the idle CUs too: for few tiles, and with
 * K % 64 == 0 up to 11/16 of the CUs' count in tiles, over up to twice as
 * many workgroups; beyond that, with K % 64 == 0 and K >= 8192, the K loop
 * tails of every tile over the CUs the tiles leave idle), 0 when the
 * data-parallel kernel is used and no workspace is needed.
 * Host-only query; enqueues nothing.
 */
int64_t umic_linear_workspace_bytes(int64_t M, int64_t N, int64_t K);

/*
 * umic_linear_bf16 with a caller-provided workspace for the stream-K
 * schedule.  Same arguments, numerics and shape rules; results are
 * deterministic (split tiles sum their K segments in a fixed order).
 * workspace: >= umic_linear_workspace_bytes(M, N, K) bytes, 256-byte
 * aligned, ALL ZERO before its first use; every call leaves its counters at
 * zero again, so one workspace serves any number of calls that do not
 * overlap in time (e.g. all calls on one stream).  Calls that may run
 * concurrently need separate workspaces: overlapping calls on one workspace
 * may give wrong results, or make a tile's reduction wait give up (see
 * UMIC_SK_STATUS_OFFSET), leaving that tile unwritten.  A smaller (or NULL)
 * workspace, or a shape the data-parallel kernel serves better, runs
 * umic_linear_bf16.
 * Replaces: kernels/linear.py:118-145 (linear_triton), as umic_linear_bf16;
 * caller integrate.py:98-107.
 */
int umic_linear_ws_bf16(const void* x, const void* w, const void* bias, void* out,
                        int64_t M, int64_t N, int64_t K,
                        int64_t ldx, int64_t ldw, int64_t ldo,
                        int act, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * umic_linear_ws_bf16 without a workspace argument and without allocating:
 * the stream-K schedule runs on a static device scratch array of the
 * library (64 MiB per device, held from the library's first use on that
 * device until the process ends).  Same arguments (minus the workspace),
 * numerics, shape rules and results as umic_linear_ws_bf16 with a large
 * enough workspace; shapes the data-parallel kernel or the GEMV serve run
 * those, as there.  A shape whose stream-K workspace
 * (umic_linear_workspace_bytes) exceeds 64 MiB -- the schedule for
 * fewer tiles with more than 127 output tiles of 256 x 256 -- returns
 * UMIC_ERR_SCRATCH before any launch.  At N = 4096, K = 12288 (the MLP
 * down projection) that admits M <= 1792 and, on the schedule for tiles
 * that fill most CUs (which always fits), M from 2817 to 3968, the BASELINE
 * prefill (M = 3100, 208 tiles, 63.8 MiB) included; M from 1793 to 2816
 * needs umic_linear_ws_bf16.  The device's first call clears the scratch's
 * counter region with a kernel (no memset); every launch leaves it cleared.
 * All calls on one device share its scratch: calls that may overlap in time
 * on one device (different streams without ordering) may give wrong
 * results, or make a tile's reduction wait give up after well under a
 * second and leave that tile unwritten (the scratch's status word, not
 * readable through this API, is then set); calls on one stream are safe.
 * No counterpart in the reference: an entry point for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops that
 * forbid allocation).
 */
int umic_linear_sk_static_bf16(const void* x, const void* w, const void* bias, void* out,
                               int64_t M, int64_t N, int64_t K,
                               int64_t ldx, int64_t ldw, int64_t ldo,
                               int act, void* stream);

/*
 * Up to three linears over one x in one launch, the decode GEMV path only:
 * out_i = act(x @ w_i^T + bias_i) for i < count (count 1..3), each with its
 * own N_i, weight leading dim ldw_i and output leading dim ldo_i; bias may
 * be NULL, or an array whose entries may be NULL.  M must be 1..8 (else
 * UMIC_ERR_UNSUPPORTED; M == 0 is a no-op); shape and alignment rules are
 * umic_linear_bf16's, per segment.  Results equal umic_linear_bf16 on each
 * linear (the same kernel and summation order).
 * No counterpart in the reference, which runs the text attention's q_proj,
 * k_proj and v_proj (transformers modeling_qwen3_vl
 * Qwen3VLTextAttention.forward) as three vendor GEMVs at decode.
 */
int umic_linear_multi_bf16(const void* x, int64_t M, int64_t K, int64_t ldx, int count,
                           const void* const* w, const void* const* bias, void* const* out,
                           const int64_t* N, const int64_t* ldw, const int64_t* ldo, int act,
                           void* stream);

/*
 * out = residual + (x @ w^T + bias) with the eager chain's two bf16
 * roundings (the linear's output, then the sum): the decoder layer's MLP
 * residual add folded into the down projection at decode.  M must be 1..8
 * (the GEMV path; else UMIC_ERR_UNSUPPORTED; M == 0 is a no-op).  residual:
 * [M, N] bf16, row stride ldr; out may alias residual only if ldr == ldo.
 * Other rules as umic_linear_bf16.  No counterpart in the reference, whose
 * decoder layer (transformers Qwen3VLTextDecoderLayer.forward) adds the MLP
 * output to the residual stream in a separate op.
 */
int umic_linear_add_bf16(const void* x, const void* w, const void* bias, const void* residual,
                         void* out, int64_t M, int64_t N, int64_t K, int64_t ldx, int64_t ldw,
                         int64_t ldr, int64_t ldo, void* stream);

/*
 * Fused P5 MLP front half: out = silu(x @ wg^T) * (x @ wu^T), one bf16
 * rounding of the fp32 product.  wg, wu: [N, K] nn.Linear weights (the
 * reference passes them as .t() views; same memory).
 * Same shape / alignment rules, and the same M <= 8 GEMV path, as
 * umic_linear_bf16.
 * Replaces: kernels/fused_ffn.py:93-126 (gate_silu_mul_triton /
 * gate_silu_mul), kernel kernels/fused_ffn.py:48-91; caller
 * integrate.py:44-55.
 */
int umic_gate_silu_mul_bf16(const void* x, const void* wg, const void* wu,
                            void* out, int64_t M, int64_t N, int64_t K,
                            int64_t ldx, int64_t ldwg, int64_t ldwu,
                            int64_t ldo, void* stream);

/*
 * Decode-step RMSNorm fused into the q/k/v multi-linear GEMV:
 *   y = RMSNorm(x) with norm_w and eps (umic_rmsnorm_bf16's numerics on the
 *   M x K rows), then out_i = y @ w_i^T + bias_i as umic_linear_multi_bf16
 *   (act none) -- one launch, no trip of y through memory: every workgroup
 *   normalizes the rows itself from L2 while its first weight loads are in
 *   flight.  Results are bit-identical to umic_rmsnorm_bf16 followed by
 *   umic_linear_multi_bf16.  normed: optional [M, >= ldn] copy of y (NULL:
 *   not written; written only when some N_i > 0), which must not overlap x.
 *   Requires 1 <= M <= 2 and a row length K whose eager reduction plan is
 *   the single-block one without a row split and at most four 4-vectors
 *   per thread (with K % 32 == 0: every K from 512 to 4096), 8-byte
 *   aligned norm_w and normed (ldn % 4 == 0), plus umic_linear_multi_bf16's
 *   rules; else UMIC_ERR_UNSUPPORTED.
 * No single counterpart in the reference: replaces the decoder layer's
 * input_layernorm forward (integrate.py:134-141 on Qwen3VLTextRMSNorm)
 * followed by the q/k/v projections (integrate.py:91, 98-107; in the
 * reference three linear launches) at the decode steps.
 */
int umic_rmsnorm_linear_multi_bf16(const void* x, const void* norm_w, void* normed,
                                   int64_t M, int64_t K, int64_t ldx, int64_t ldn,
                                   float eps, int count, const void* const* w,
                                   const void* const* bias, void* const* out,
                                   const int64_t* N, const int64_t* ldw, const int64_t* ldo,
                                   void* stream);

/*
 * Decode-step residual add + RMSNorm fused into the P5 GEMV:
 *   summed = bf16(x + r); normed = RMSNorm(summed) (umic_add_rmsnorm_bf16's
 *   numerics); out = silu(normed @ wg^T) * (normed @ wu^T) as
 *   umic_gate_silu_mul_bf16 -- one launch.  Bit-identical to
 *   umic_add_rmsnorm_bf16 followed by umic_gate_silu_mul_bf16.  normed and
 *   summed are optional outputs (NULL: not written) that must not overlap x
 *   or r.  Same row rules as umic_rmsnorm_linear_multi_bf16 (r 8-byte
 *   aligned, ldr % 4 == 0), plus umic_gate_silu_mul_bf16's.
 * No single counterpart in the reference: replaces the decoder layer's
 * residual add and post_attention_layernorm forward followed by
 * kernels/fused_ffn.py:93-118 (gate_silu_mul_triton) at the decode steps.
 */
int umic_add_rmsnorm_gate_silu_mul_bf16(const void* x, const void* r, const void* norm_w,
                                        void* normed, void* summed, const void* wg,
                                        const void* wu, void* out, int64_t M, int64_t N,
                                        int64_t K, int64_t ldx, int64_t ldr, int64_t ldn,
                                        int64_t lds, int64_t ldwg, int64_t ldwu, int64_t ldo,
                                        float eps, void* stream);

/*
 * Measurement helper: reads `bytes` bytes at p once (16-byte non-temporal
 * loads; p 16-byte aligned, bytes a multiple of 16, else
 * UMIC_ERR_UNSUPPORTED) and writes one xor-fold word per workgroup to
 * fold[0 .. UMIC_STREAM_READ_GRID) (4-byte aligned).  Its time is the
 * practical ceiling of a kernel that streams the same bytes from HBM, the
 * yardstick bench.py holds the decode GEMVs (one pass over their weights)
 * against.  No counterpart in the reference; nothing on the fused path
 * calls it.
 */
#define UMIC_STREAM_READ_GRID 2048
int umic_stream_read(const void* p, int64_t bytes, void* fold, void* stream);

/*
 * Measurement helper: copies `bytes` bytes from src to dst (16-byte
 * non-temporal loads and stores, one-shot grid; both 16-byte aligned and
 * bytes a multiple of 16, else UMIC_ERR_UNSUPPORTED; overlapping ranges
 * UMIC_ERR_INVALID_ARG).  Its time is the practical ceiling of a kernel that
 * reads bytes once and writes bytes once, the yardstick bench.py holds the
 * norm and RoPE kernels against.  No counterpart in the reference; nothing
 * on the fused path calls it.
 */
int umic_stream_copy(const void* src, void* dst, int64_t bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* UMIC_HIP_H */
