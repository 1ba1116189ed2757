// Row normalisation kernels for gfx950: RMSNorm, residual-add + RMSNorm,
// LayerNorm (affine, bias) and residual-add + LayerNorm, all bf16 in/out.
//
// Numerics: eager's, bit for bit.  The eager modules these kernels replace
// (HF Qwen3VLTextRMSNorm, torch layer_norm) take their row statistics on
// the GPU in fp32, in an order fixed by torch's own kernels, and a
// statistic one fp32 ulp away from eager's moves a bf16 output by up to two
// ulps.  So every kernel here reproduces torch-ROCm's order exactly:
//
//   RMSNorm   mean(x^2) is aten's generic reduction (ATen/native/hip/
//             Reduce.cuh): setReduceConfig picks, from [rows, n], the
//             threads across a row (bw), whether each thread reads 4-element
//             vectors, and whether a row is also split over wavefronts;
//             each thread keeps 4 accumulators, combines them in order, and
//             the threads combine in a fixed tree (a shared-memory halving
//             down to 64, then shuffles with offsets 1, 2, 4, ... on ROCm).
//             The mean is sum * (rows / (rows * n)); rsqrt is correctly
//             rounded (torch.rsqrt on this platform).
//   LayerNorm aten's vectorized_layer_norm_kernel (64x4 threads): thread t
//             runs Welford over the 4-element vectors t, t + 256, ...; the
//             wavefronts combine with shuffle-down offsets 32 .. 1, then
//             across the four wavefronts; count reciprocals are v_rcp_f32,
//             rstd is v_rsq_f32(m2 / n + eps), and the fused products are
//             the ones the ROCm build contracts.  Rows torch sends to its
//             scalar LayerNorm kernel (n % 4 != 0, or x, weight or bias
//             off 8-byte alignment) follow that kernel's order instead:
//             512 reducing threads per row, IEEE divisions, v_rsq_f32.
//
// Layouts.  The register paths keep each row in registers, so a row is read
// once and written once:
//   RMSNorm   a group of bw/2 lanes owns a row; lane l holds the vectors
//             l, l + bw/2, ... -- exactly the data of torch's reducing
//             threads 2l and 2l + 1, so the per-thread sums are formed in
//             place and the tree is the pair, then a lane butterfly.
//   LayerNorm 16 lanes own a row; lane l holds torch's threads l + 16k of
//             each wavefront (4-element vectors), so the first two steps of
//             torch's shuffle tree and its cross-wavefront tree run in-lane
//             and the rest is a 16-lane butterfly with the tree's (own,
//             other) orientation kept.
// Every other shape takes a block-per-row kernel that runs the same
// reduction with one hardware thread per torch thread.
//
// Eager's bf16 rounding points are kept:
//   RMSNorm     y = bf16(w * bf16(x * rstd))            (HF Qwen3VLTextRMSNorm)
//   LayerNorm   y = bf16(fma(w, rstd * (x - mean), b))  (torch layer_norm)
//   add+norm    s = bf16(x + r), then the norm of the ROUNDED s.
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
  float factor;  // RMSNorm: aten MeanOps factor, float(rows) / float(rows * n)
};


// ---- LayerNorm Welford pieces (torch-ROCm's arithmetic) -------------------

struct Wf {
  float mean, m2, n;
};

// v_rcp_f32 of a count.  The empty asm keeps the count opaque: in the
// unrolled register path the counts are compile-time constants (every
// Welford state starts at 0), and the compiler folds the instruction on a
// constant to the correctly rounded 1/c -- which differs from the hardware
// result on ~10% of counts, and eager runs the instruction.
__device__ __forceinline__ float hw_rcp(float c) {
  asm volatile("" : "+v"(c));
  return __builtin_amdgcn_rcpf(c);
}

// One element: the mean update fused with the hardware count reciprocal,
// the m2 update as two roundings (cuWelfordOnlineSum as the ROCm build
// compiles it).
__device__ __forceinline__ Wf wf_push(Wf a, float v) {
  const float delta = v - a.mean;
  const float cnt = a.n + 1.0f;
  const float mean = __builtin_fmaf(delta, hw_rcp(cnt), a.mean);
  const float m2 = a.m2 + delta * (v - mean);
  return Wf{mean, m2, cnt};
}

// cuWelfordCombine(b = own, a = other).  INTRA: the wavefront tree contracts
// the mean as fma(nA, meanA, nB * meanB); the cross-wavefront tree as
// fma(nB, meanB, nA * meanA).  m2 takes fma(delta^2 * countA, nB, m2A + m2B).
template <bool INTRA>
__device__ __forceinline__ Wf wf_combine(Wf b, Wf a) {
  const float delta = b.mean - a.mean;
  const float cnt = a.n + b.n;
  if (!(cnt > 0.0f)) return Wf{0.0f, 0.0f, cnt};
  const float coef = hw_rcp(cnt);
  const float na = a.n * coef, nb = b.n * coef;
  const float mean = INTRA ? __builtin_fmaf(na, a.mean, nb * b.mean)
                           : __builtin_fmaf(nb, b.mean, na * a.mean);
  const float m2 = __builtin_fmaf((delta * delta) * a.n, nb, a.m2 + b.m2);
  return Wf{mean, m2, cnt};
}

// The partner lane (lane ^ K, K <= 16) through ds_swizzle's bitmask mode.
template <int K>
__device__ __forceinline__ float swz_xor(float v) {
  return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), (K << 10) | 0x1F));
}

// One butterfly step of the wavefront tree over lane bit K: both lanes of a
// pair compute combine(lower lane's state, upper lane's state).
template <int K>
__device__ __forceinline__ Wf wf_step(Wf s, bool upper) {
  const Wf o{swz_xor<K>(s.mean), swz_xor<K>(s.m2), swz_xor<K>(s.n)};
  return upper ? wf_combine<true>(o, s) : wf_combine<true>(s, o);
}

// ---- register path: RMSNorm ----------------------------------------------

// LPR = bw/2 lanes own a row; lane l holds the 16-byte vectors l + LPR*j,
// the data of torch's reducing threads 2l (elements 0..3 of each vector) and
// 2l + 1 (elements 4..7).  RPG rows per group: rows of one or two vectors per
// lane (e.g. the [S*H, 128] per-head q/k norms) leave a wavefront only 1-2 KB
// of loads in flight, too little to cover HBM latency; a group then takes
// RPG consecutive rows and issues all their loads before reducing any.
// FULL: every lane's MAXV slots hold vectors of the row (nvec == MAXV * LPR,
// vpl == MAXV), so the per-slot liveness tests are compile-time true.
template <bool ADD, int LPR, int MAXV, int RPG, bool FULL = false>
__global__ __launch_bounds__(256) void rms_rows_kernel(NormArgs a, int nvec, int vpl) {
  const int rows_per_block = (int)blockDim.x / LPR * RPG;
  const int lane = threadIdx.x & (LPR - 1);
  const int64_t row0 = (int64_t)blockIdx.x * rows_per_block + (threadIdx.x / LPR) * RPG;
  // All LPR lanes of a group share its rows, so a group exits as a whole and
  // the butterflies below only ever read lanes of a live group.
  if (row0 >= a.rows) return;

  // Loads are issued unconditionally (a dead slot re-reads vector 0, a row
  // past the end re-reads row0; both are zeroed or never stored): predicated
  // loads would sit in branches, and every branch join costs a full vmcnt
  // drain -- the loads must all be in flight together.
  const u32x4 zero = {0u, 0u, 0u, 0u};
  bool live[MAXV];
  int cix[MAXV];
#pragma unroll
  for (int i = 0; i < MAXV; ++i) {
    const int c = i * LPR + lane;
    live[i] = FULL || (i < vpl && c < nvec);
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
  if constexpr (ADD) {
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
  u32x4 wv[MAXV];
#pragma unroll
  for (int r = 0; r < RPG; ++r) {
    // torch's per-thread sums: thread 2l keeps acc[0..3] over elements 0..3 of
    // its vectors, thread 2l + 1 acc[4..7] over elements 4..7, in vector order
    // (a dead slot adds +0, which changes nothing).
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < MAXV; ++i) {
      if (!live[i]) sv[r][i] = zero;
      float f[8];
      unpack8(sv[r][i], f);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = acc[e] + f[e] * f[e];
    }
    const float t_even = ((acc[0] + acc[1]) + acc[2]) + acc[3];
    const float t_odd = ((acc[4] + acc[5]) + acc[6]) + acc[7];
    // the shuffle tree over bw threads: the adjacent pair, then lane pairs
    const float ssq = group_sum<LPR>(t_even + t_odd);
    const float rstd = rsqrt_cr(ssq * a.factor + a.eps);
    if (r == 0) {
      // weights, L2-resident, loaded once the first row's statistic is
      // done: issued with the row loads they measured slower
#pragma unroll
      for (int i = 0; i < MAXV; ++i) wv[i] = wp[cix[i]];
    }

    u32x4* yp = reinterpret_cast<u32x4*>(a.y + rows[r] * a.ldy);
#pragma unroll
    for (int i = 0; i < MAXV; ++i) {
      if (!live[i] || !rlive[r]) continue;
      float f[8], wf[8], o[8];
      unpack8(sv[r][i], f);
      unpack8(wv[i], wf);
#pragma unroll
      for (int e = 0; e < 8; e += 2) {  // bf16(x * rstd) in pairs (one conversion each)
        float p0 = f[e] * rstd, p1 = f[e + 1] * rstd;
        rbf2(p0, p1);
        o[e] = wf[e] * p0;
        o[e + 1] = wf[e + 1] * p1;
      }
      st_stream(yp + cix[i], pack8(o));
    }
  }
}

// ---- register path: LayerNorm --------------------------------------------

// Word 3 of a raw buffer resource (the one gemm.hip uses): untyped dword
// access with range checking against num_records.
constexpr int kRsrcWord3 = 0x00020000;

// Sixteen lanes per row.  Torch's thread t = 64w + x (wavefront w, lane x)
// reads the 4-element vectors t, t + 256, ...; here lane l of a row's group
// holds the threads x = l + 16k, k = 0..3, of every wavefront w, so torch's
// first two shuffle steps (offsets 32 and 16: bit 1 and bit 0 of k) run
// in-lane, the next four (offsets 8 .. 1) are a lane butterfly over the 16
// lanes, and the cross-wavefront tree (w with w + 2, then 0 with 1) is
// in-lane again -- about 31 combines per lane and row.  Vector t + 256j of
// thread (w, l + 16k) is element group 16m + l with m = 4w + k + 16j: slot m
// of lane l, the slots below 4 * M4 = 4 * ceil(n / 256) held in registers.
// Loads and stores are 8-byte chunks, 128 contiguous bytes per group, through
// buffer resources over the wavefront's four rows.  The pushes take their
// count reciprocals from a table of v_rcp_f32 results.
// FULL: the row fills every slot (n = 256 * M4, as the ViT width 1280 with
// M4 = 5), so the per-slot guards are compile-time true.  Without them the
// launch at [16384, 1280] measured 16.4-17.2 against 17.6-18.6 us: the
// statistics between a row's loads and its stores are on the critical path.
template <bool ADD, int M4, bool FULL = false>
__global__ __launch_bounds__(256) void ln_rows_kernel(NormArgs a, int nvec4) {
  constexpr int G = 16, M = 4 * M4, kRowsPerWave = kWave / G;
  constexpr int kNt = 2;  // buffer access cache policy: non-temporal (streamed once)
  const int l = threadIdx.x & (G - 1);
  // the wavefront's first row (uniform) and this group's row within its four
  const int64_t wrow0 = __builtin_amdgcn_readfirstlane(
      (int)((int64_t)blockIdx.x * (blockDim.x / G) + (threadIdx.x / kWave) * kRowsPerWave));
  const int rw = (threadIdx.x & (kWave - 1)) / G;
  const int64_t row = wrow0 + rw;
  if (row >= a.rows) return;  // a group exits as a whole: its butterflies stay in it
  const int64_t wrows = a.rows - wrow0 < kRowsPerWave ? a.rows - wrow0 : kRowsPerWave;

  // Buffer resources over the wavefront's rows (uniform, so every access is
  // one instruction): a slot past its row's end reads the gap or the next row
  // (never pushed) or, past the last row, zeros; stores check the slot.
  auto span = [&](const uint16_t* base, int64_t ld) {
    return __builtin_amdgcn_make_buffer_rsrc((void*)(base + wrow0 * ld), (short)0,
                                             (int)(((wrows - 1) * ld + a.n) * 2), kRsrcWord3);
  };
  const int lx = (int)(rw * a.ldx * 2) + l * 8;  // byte offset of slot 0; slot m adds 128 m
  const __amdgpu_buffer_rsrc_t xr = span(a.x, a.ldx);
  u32x2 xv[M];
#pragma unroll
  for (int m = 0; m < M; ++m) xv[m] = __builtin_amdgcn_raw_buffer_load_b64(xr, lx + 128 * m, 0, kNt);
  if constexpr (ADD) {
    const __amdgpu_buffer_rsrc_t rr = span(a.r, a.ldr);
    const __amdgpu_buffer_rsrc_t sr = span(a.s, a.lds);
    const int lr = (int)(rw * a.ldr * 2) + l * 8, ls = (int)(rw * a.lds * 2) + l * 8;
    u32x2 rv[M];
#pragma unroll
    for (int m = 0; m < M; ++m) rv[m] = __builtin_amdgcn_raw_buffer_load_b64(rr, lr + 128 * m, 0, kNt);
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float xf[4], rf[4];
      unpack4(xv[m], xf);
      unpack4(rv[m], rf);
#pragma unroll
      for (int e = 0; e < 4; ++e) xf[e] = xf[e] + rf[e];
      xv[m] = pack4(xf);  // bf16(x + r): the eager residual add
      if (FULL || 16 * m + l < nvec4)
        __builtin_amdgcn_raw_buffer_store_b64(xv[m], sr, ls + 128 * m, 0, kNt);
    }
  }

  // v_rcp_f32 of the counts a thread's pushes reach (at most 4 per 16 slots)
  constexpr int kMaxCount = 4 * ((M + 15) / 16);
  float rc[kMaxCount];
#pragma unroll
  for (int c = 0; c < kMaxCount; ++c) rc[c] = hw_rcp((float)(c + 1));

  Wf wv[4];
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    Wf st[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      Wf t{0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int j = 0; 4 * w + k + 16 * j < M; ++j) {
        const int m = 4 * w + k + 16 * j;
        if (!FULL && 16 * m + l >= nvec4) break;  // a thread's vectors are a prefix of j
        float f[4];
        unpack4(xv[m], f);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float delta = f[e] - t.mean;
          t.mean = __builtin_fmaf(delta, rc[4 * j + e], t.mean);
          t.m2 = t.m2 + delta * (f[e] - t.mean);
        }
        t.n = (float)(4 * (j + 1));
      }
      st[k] = t;
    }
    // torch offsets 32 and 16 (k bit 1, then bit 0), own state first
    st[0] = wf_combine<true>(st[0], st[2]);
    st[1] = wf_combine<true>(st[1], st[3]);
    Wf sw = wf_combine<true>(st[0], st[1]);
    // offsets 8, 4, 2, 1: the lane bits
    sw = wf_step<8>(sw, l & 8);
    sw = wf_step<4>(sw, l & 4);
    sw = wf_step<2>(sw, l & 2);
    sw = wf_step<1>(sw, l & 1);
    wv[w] = sw;
  }
  // the cross-wavefront tree: w with w + 2, then 0 with 1
  const Wf t = wf_combine<false>(wf_combine<false>(wv[0], wv[2]),
                                 wf_combine<false>(wv[1], wv[3]));
  const float mean = t.mean;
  const float rstd = __builtin_amdgcn_rsqf(t.m2 / (float)a.n + a.eps);

  const int w_bytes = (int)(a.n * 2);
  const __amdgpu_buffer_rsrc_t wr =
      __builtin_amdgcn_make_buffer_rsrc((void*)a.w, (short)0, w_bytes, kRsrcWord3);
  const __amdgpu_buffer_rsrc_t br =
      __builtin_amdgcn_make_buffer_rsrc((void*)a.b, (short)0, w_bytes, kRsrcWord3);
  const __amdgpu_buffer_rsrc_t yr = span(a.y, a.ldy);
  const int ly = (int)(rw * a.ldy * 2) + l * 8;
  // LayerNorm: slot m + 1's weight and bias are loaded before slot m's store
  // (slots past the row read zeros: the resources end at n), so each load
  // overlaps a slot's arithmetic.  Measured in one process at [16384, 1280],
  // bit-identical, over two boxes: LayerNorm 15.2-16.6 us against 16.0-17.7
  // us with the loads beside their own slot.  add+LayerNorm, whose
  // summed-output stores are still draining here, ran 33.4-35.0 against
  // 32.2-34.1 us with the look-ahead, so it keeps the per-slot loads.
  constexpr bool kLookahead = !ADD;
  u32x2 wn = __builtin_amdgcn_raw_buffer_load_b64(wr, l * 8, 0, 0);
  u32x2 bn = __builtin_amdgcn_raw_buffer_load_b64(br, l * 8, 0, 0);
#pragma unroll
  for (int m = 0; m < M; ++m) {
    if (!kLookahead && m > 0) {
      wn = __builtin_amdgcn_raw_buffer_load_b64(wr, l * 8 + 128 * m, 0, 0);
      bn = __builtin_amdgcn_raw_buffer_load_b64(br, l * 8 + 128 * m, 0, 0);
    }
    const u32x2 wc = wn, bc = bn;
    if (kLookahead && m + 1 < M) {
      wn = __builtin_amdgcn_raw_buffer_load_b64(wr, l * 8 + 128 * (m + 1), 0, 0);
      bn = __builtin_amdgcn_raw_buffer_load_b64(br, l * 8 + 128 * (m + 1), 0, 0);
    }
    if (!FULL && 16 * m + l >= nvec4) continue;
    float f[4], wf[4], bf[4], o[4];
    unpack4(xv[m], f);
    unpack4(wc, wf);
    unpack4(bc, bf);
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = __builtin_fmaf(wf[e], rstd * (f[e] - mean), bf[e]);
    __builtin_amdgcn_raw_buffer_store_b64(pack4(o), yr, ly + 128 * m, 0, kNt);
  }
}

// ---- block-per-row paths -------------------------------------------------

// Element j of the row the statistics are taken over: x, or bf16(x + r).
// Recomputed on every pass (cheap, identical result) rather than re-read
// from the summed output.
template <bool ADD>
__device__ __forceinline__ float src_val(const NormArgs& a, int64_t row, int64_t j) {
  const float xf = bf2f(a.x[row * a.ldx + j]);
  if constexpr (ADD) return rbf(xf + bf2f(a.r[row * a.ldr + j]));
  return xf;
}

template <bool ADD>
__device__ __forceinline__ float sq(const NormArgs& a, int64_t row, int64_t j) {
  const float f = src_val<ADD>(a, row, j);
  return f * f;
}

template <bool ADD>
__device__ void write_sum(const NormArgs& a, int64_t row) {
  if constexpr (ADD) {
    uint16_t* sr = a.s + row * a.lds;
    for (int64_t j = threadIdx.x; j < a.n; j += blockDim.x)
      sr[j] = (uint16_t)f2bf(src_val<ADD>(a, row, j));
  }
}

// RMSNorm with torch's reduction for any plan: one hardware thread per
// reducing thread (x = lane across the row, y = wavefront when the row is
// split), the per-thread loops of Reduce.cuh's vectorized (with the head
// and tail of a row off 16-byte alignment in the fp32 copy eager reduces:
// row r starts (r * n) % 4 elements past it) and scalar forms, then
// block_x_reduce and block_y_reduce through LDS.
template <bool ADD>
__global__ __launch_bounds__(512) void rms_block_kernel(NormArgs a, RmsPlan p) {
  __shared__ float red[512];
  __shared__ float yred[16];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  const int x = tid % p.bw, y = tid / p.bw;
  write_sum<ADD>(a, row);
  const int64_t n = a.n;
  const int64_t step = (int64_t)p.bw * (p.split ? p.bh : 1);
  const int64_t idx0 = x + (int64_t)(p.split ? y : 0) * p.bw;
  const bool tail_ok = !p.split || y == 0;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  if (p.vec) {
    const int shift = (int)((row * n) % 4);
    int64_t j0 = 0, end = n;  // row elements j0 + [0, end) are vector-aligned
    if (shift > 0) {
      if (x >= shift && x < 4 && tail_ok) acc[0] = sq<ADD>(a, row, x - shift);
      j0 = 4 - shift;
      end = n - j0;
    }
    for (int64_t idx = idx0; idx * 4 + 3 < end; idx += step) {
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] = acc[i] + sq<ADD>(a, row, j0 + idx * 4 + i);
    }
    const int64_t tail = end - end % 4;
    if (tail_ok && tail + x < end) acc[0] = acc[0] + sq<ADD>(a, row, j0 + tail + x);
  } else {
    int64_t idx = idx0;
    for (; idx + 3 * step < n; idx += 4 * step) {
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] = acc[i] + sq<ADD>(a, row, idx + i * step);
    }
    for (int i = 0; i < 4 && idx < n; ++i, idx += step) acc[i] = acc[i] + sq<ADD>(a, row, idx);
  }
  red[tid] = ((acc[0] + acc[1]) + acc[2]) + acc[3];
  __syncthreads();
  for (int off = p.bw / 2; off >= kWave; off >>= 1) {  // shared-memory halving
    if (x < off) red[tid] = red[tid] + red[tid + off];
    __syncthreads();
  }
  const int w = p.bw < kWave ? p.bw : kWave;
  for (int off = 1; off < w; off <<= 1) {  // the shuffle tree, offsets upward
    if (x % (2 * off) == 0 && x + off < w) red[tid] = red[tid] + red[tid + off];
    __syncthreads();
  }
  float total = red[0];
  if (p.split) {
    if (x == 0) yred[y] = red[tid];
    __syncthreads();
    for (int off = p.bh / 2; off > 0; off >>= 1) {  // block_y_reduce
      if (tid < off) yred[tid] = yred[tid] + yred[tid + off];
      __syncthreads();
    }
    total = yred[0];
  }
  const float rstd = rsqrt_cr(total * a.factor + a.eps);
  uint16_t* yr = a.y + row * a.ldy;
  for (int64_t j = tid; j < n; j += blockDim.x)
    yr[j] = (uint16_t)f2bf(bf2f(a.w[j]) * rbf(src_val<ADD>(a, row, j) * rstd));
}

// RMSNorm rows of the plans with 128..512 reducing threads across a row and
// no split (one to seven rows: the decode steps), with the block kernel's
// summation order and vector access: thread x holds the 4-element vectors
// x, x + BW, ... (K4 of them at most) in registers, sums their squares into
// its four accumulators, and the block reduces as block_x_reduce does --
// shared-memory halving BW/2 .. 64 (wavefront w + W/2 into w, ...), done by
// wavefront 0 from one LDS pass, then the in-wavefront tree (offsets 1 .. 32
// upward; the butterfly gives lane 0 the same sums) -- so two barriers
// instead of one per halving step.  Requires n % 4 == 0 and 8-byte aligned
// rows (x, y, w; r and s for the add form).
template <bool ADD, int BW, int K4>
__global__ __launch_bounds__(BW) void rms_wide_kernel(NormArgs a) {
  constexpr int W = BW / kWave;
  __shared__ float red[BW];
  __shared__ float stat;
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int nv = (int)(a.n / 4);
  const uint16_t* xr = a.x + row * a.ldx;
  u32x2 v[K4];
#pragma unroll
  for (int k = 0; k < K4; ++k) {
    const int idx = tid + k * BW;
    if (idx < nv) v[k] = *reinterpret_cast<const u32x2*>(xr + idx * 4);
  }
  if constexpr (ADD) {
    const uint16_t* rr = a.r + row * a.ldr;
    uint16_t* sr = a.s + row * a.lds;
#pragma unroll
    for (int k = 0; k < K4; ++k) {
      const int idx = tid + k * BW;
      if (idx >= nv) continue;
      float xf[4], rf[4];
      unpack4(v[k], xf);
      unpack4(*reinterpret_cast<const u32x2*>(rr + idx * 4), rf);
#pragma unroll
      for (int e = 0; e < 4; ++e) xf[e] = xf[e] + rf[e];
      v[k] = pack4(xf);  // bf16(x + r): the eager residual add
      *reinterpret_cast<u32x2*>(sr + idx * 4) = v[k];
    }
  }
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int k = 0; k < K4; ++k) {
    if (tid + k * BW >= nv) break;
    float f[4];
    unpack4(v[k], f);
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] = acc[i] + f[i] * f[i];
  }
  red[tid] = ((acc[0] + acc[1]) + acc[2]) + acc[3];
  __syncthreads();
  if (tid < kWave) {
    float r[W];
#pragma unroll
    for (int w = 0; w < W; ++w) r[w] = red[w * kWave + lane];
#pragma unroll
    for (int h = W / 2; h >= 1; h >>= 1)
#pragma unroll
      for (int w = 0; w < h; ++w) r[w] = r[w] + r[w + h];
    const float total = group_sum<kWave>(r[0]);
    if (tid == 0) stat = rsqrt_cr(total * a.factor + a.eps);
  }
  __syncthreads();
  const float rstd = stat;
  const uint16_t* wr = a.w;
  uint16_t* yr = a.y + row * a.ldy;
#pragma unroll
  for (int k = 0; k < K4; ++k) {
    const int idx = tid + k * BW;
    if (idx >= nv) break;
    float f[4], wf[4], o[4];
    unpack4(v[k], f);
    unpack4(*reinterpret_cast<const u32x2*>(wr + idx * 4), wf);
#pragma unroll
    for (int e = 0; e < 4; e += 2) {  // bf16(x * rstd) in pairs
      float p0 = f[e] * rstd, p1 = f[e + 1] * rstd;
      rbf2(p0, p1);
      o[e] = wf[e] * p0;
      o[e + 1] = wf[e + 1] * p1;
    }
    *reinterpret_cast<u32x2*>(yr + idx * 4) = pack4(o);
  }
}

// LayerNorm with torch's vectorized kernel order for any n % 4 == 0: 256
// threads per row, thread t pushes the 4-element vectors t, t + 256, ...; the
// wavefront tree by shuffle-down (a lane past the end reads itself, as in
// torch), the four wavefront results combined by thread 0.
template <bool ADD>
__global__ __launch_bounds__(256) void ln_torch_block_kernel(NormArgs a) {
  __shared__ float wres[4][3];
  __shared__ float stat[2];
  const int64_t row = blockIdx.x;
  const int t = threadIdx.x, lane = t & (kWave - 1);
  write_sum<ADD>(a, row);
  Wf s{0.0f, 0.0f, 0.0f};
  for (int64_t v = t; v < a.n / 4; v += 256) {
#pragma unroll
    for (int e = 0; e < 4; ++e) s = wf_push(s, src_val<ADD>(a, row, v * 4 + e));
  }
  for (int off = 32; off > 0; off >>= 1) {
    const Wf o{__shfl_down(s.mean, off, kWave), __shfl_down(s.m2, off, kWave),
               __shfl_down(s.n, off, kWave)};
    s = wf_combine<true>(s, o);
  }
  if (lane == 0) {
    wres[t / kWave][0] = s.mean;
    wres[t / kWave][1] = s.m2;
    wres[t / kWave][2] = s.n;
  }
  __syncthreads();
  if (t == 0) {
    Wf w4[4];
    for (int i = 0; i < 4; ++i) w4[i] = Wf{wres[i][0], wres[i][1], wres[i][2]};
    w4[0] = wf_combine<false>(w4[0], w4[2]);
    w4[1] = wf_combine<false>(w4[1], w4[3]);
    w4[0] = wf_combine<false>(w4[0], w4[1]);
    stat[0] = w4[0].mean;
    stat[1] = __builtin_amdgcn_rsqf(w4[0].m2 / (float)a.n + a.eps);
  }
  __syncthreads();
  const float mean = stat[0], rstd = stat[1];
  uint16_t* yr = a.y + row * a.ldy;
  for (int64_t j = t; j < a.n; j += blockDim.x) {
    const float f = src_val<ADD>(a, row, j);
    yr[j] = (uint16_t)f2bf(__builtin_fmaf(bf2f(a.w[j]), rstd * (f - mean), bf2f(a.b[j])));
  }
}

// LayerNorm rows eager sends down its scalar kernel (n % 4 != 0, or x,
// weight or bias off 8-byte alignment) in that kernel's order
// (RowwiseMomentsCUDAKernel, layer_norm_kernel.cu): 512 reducing threads per
// row, thread t folding elements t, t + 512, ... by Welford updates with IEEE
// divisions; a shuffle-down tree per 64-thread group; the same tree over the
// 8 group results; var = m2 / n, rstd by v_rsq_f32.  Here one wavefront
// takes a row: lane l carries the states of reducing threads l + 64 v
// (v = 0..7) side by side and runs the 8 group trees together, so a short
// row costs one wavefront rather than a 512-thread block.
struct Ws {
  float mean, m2, nf;
};

// WelfordOps::combine (SharedReduceOps.h): an empty side yields the other;
// the mean and m2 updates contract to fmas on gfx950.
__device__ __forceinline__ Ws ws_combine(Ws a, Ws b) {
  if (a.nf == 0.0f) return b;
  if (b.nf == 0.0f) return a;
  const float delta = b.mean - a.mean;
  const float cnt = a.nf + b.nf;
  const float nbn = b.nf / cnt;
  return Ws{__builtin_fmaf(delta, nbn, a.mean),
            __builtin_fmaf((delta * delta) * a.nf, nbn, a.m2 + b.m2), cnt};
}

template <bool ADD>
__global__ __launch_bounds__(256) void ln_scalar_rows_kernel(NormArgs a) {
  const int lane = (int)threadIdx.x & (kWave - 1);
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= a.rows) return;
  Ws s[8];
  int cnt[8];
#pragma unroll
  for (int v = 0; v < 8; ++v) {
    s[v] = Ws{0.0f, 0.0f, 0.0f};
    cnt[v] = 0;
  }
  for (int64_t j0 = 0; j0 < a.n; j0 += 512) {
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      const int64_t j = j0 + 64 * v + lane;
      if (j < a.n) {
        const float f = src_val<ADD>(a, row, j);
        if constexpr (ADD) a.s[row * a.lds + j] = (uint16_t)f2bf(f);
        const float nf = (float)++cnt[v];
        const float delta = f - s[v].mean;
        const float mean = s[v].mean + delta / nf;
        s[v] = Ws{mean, __builtin_fmaf(delta, f - mean, s[v].m2), nf};
      }
    }
  }
  for (int off = 32; off > 0; off >>= 1) {
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      const Ws o{__shfl_down(s[v].mean, off, kWave), __shfl_down(s[v].m2, off, kWave),
                 __shfl_down(s[v].nf, off, kWave)};
      s[v] = ws_combine(s[v], o);
    }
  }
  // lane 0 holds the 8 group results; in eager's second tree offsets 32..8
  // pair them with empty lanes (no change), offsets 4, 2, 1 pair v, v + off
#pragma unroll
  for (int off = 4; off > 0; off >>= 1)
#pragma unroll
    for (int v = 0; v < off; ++v) s[v] = ws_combine(s[v], s[v + off]);
  const float mean = __shfl(s[0].mean, 0, kWave);
  const float var = __shfl(s[0].m2, 0, kWave) / __shfl(s[0].nf, 0, kWave);
  const float rstd = __builtin_amdgcn_rsqf(var + a.eps);
  uint16_t* yr = a.y + row * a.ldy;
  for (int64_t j = lane; j < a.n; j += kWave) {
    const float f = src_val<ADD>(a, row, j);
    yr[j] = (uint16_t)f2bf(__builtin_fmaf(bf2f(a.w[j]), rstd * (f - mean), bf2f(a.b[j])));
  }
}

// ---- host dispatch --------------------------------------------------------

// Block size: the hardware spreads workgroups evenly over the 256 CUs only
// when there are many of them, so small row counts get 64- or 128-thread
// blocks (the largest block that still yields >= 8 blocks per CU).
inline int block_threads(int64_t lanes_total) {
  int threads = 256;
  while (threads > 64 && (lanes_total + threads - 1) / threads < 8 * 256) threads >>= 1;
  return threads;
}

template <bool ADD, int LPR, int MAXV, int RPG = 1>
int launch_rms_rows(const NormArgs& a, int nvec, int vpl, hipStream_t st) {
  const int threads = block_threads(a.rows * LPR / RPG);
  const int rows_per_block = threads / LPR * RPG;
  const int64_t blocks = (a.rows + rows_per_block - 1) / rows_per_block;
  if (blocks > 0x7fffffffLL) return UMIC_ERR_UNSUPPORTED;
  if (vpl == MAXV && nvec == MAXV * LPR)
    hipLaunchKernelGGL((rms_rows_kernel<ADD, LPR, MAXV, RPG, true>), dim3((unsigned)blocks),
                       dim3(threads), 0, st, a, nvec, vpl);
  else
    hipLaunchKernelGGL((rms_rows_kernel<ADD, LPR, MAXV, RPG, false>), dim3((unsigned)blocks),
                       dim3(threads), 0, st, a, nvec, vpl);
  return launch_status();
}

// One- and two-vector rows take 4 or 2 rows per group when the grouped
// launch still has >= 16 wavefronts per CU (measured on the [S*H, 128]
// per-head norms: 99200 rows gain ~10%, 24800 rows lose ~18% with grouping);
// smaller launches keep one row per group, spread over more wavefronts.
constexpr int64_t kRpgMinThreads = (int64_t)256 * 16 * 64;

template <bool ADD, int LPR, int MAXV>
int launch_rms_small(const NormArgs& a, int nvec, int vpl, hipStream_t st) {
  constexpr int kRpg = MAXV == 1 ? 4 : 2;
  if (a.rows * LPR / kRpg >= kRpgMinThreads)
    return launch_rms_rows<ADD, LPR, MAXV, kRpg>(a, nvec, vpl, st);
  return launch_rms_rows<ADD, LPR, MAXV>(a, nvec, vpl, st);
}

constexpr int kRmsMaxVpl = 24;  // vectors per lane the register path holds

template <bool ADD, int LPR>
int launch_rms_lpr(const NormArgs& a, int nvec, int vpl, hipStream_t st) {
  switch (vpl) {
    case 1: return launch_rms_small<ADD, LPR, 1>(a, nvec, vpl, st);
    case 2: return launch_rms_small<ADD, LPR, 2>(a, nvec, vpl, st);
    case 3: return launch_rms_rows<ADD, LPR, 3>(a, nvec, vpl, st);
    case 4: return launch_rms_rows<ADD, LPR, 4>(a, nvec, vpl, st);
    case 5: return launch_rms_rows<ADD, LPR, 5>(a, nvec, vpl, st);
    case 6: return launch_rms_rows<ADD, LPR, 6>(a, nvec, vpl, st);
    case 7:
    case 8: return launch_rms_rows<ADD, LPR, 8>(a, nvec, vpl, st);
    case 9:
    case 10: return launch_rms_rows<ADD, LPR, 10>(a, nvec, vpl, st);
    case 11:
    case 12: return launch_rms_rows<ADD, LPR, 12>(a, nvec, vpl, st);
    case 13:
    case 14:
    case 15:
    case 16: return launch_rms_rows<ADD, LPR, 16>(a, nvec, vpl, st);
    case 17:
    case 18:
    case 19:
    case 20: return launch_rms_rows<ADD, LPR, 20>(a, nvec, vpl, st);
    default: return launch_rms_rows<ADD, LPR, 24>(a, nvec, vpl, st);
  }
}

template <bool ADD>
int launch_rms(NormArgs a, hipStream_t st) {
  RmsPlan p;
  if (!rms_plan(a.rows, a.n, p) || (p.split && p.bh > 16)) return UMIC_ERR_UNSUPPORTED;
  a.factor = (float)a.rows / (float)(a.rows * a.n);
  bool vec = p.vec && !p.split && p.bw <= kWave && a.n % 8 == 0 && a.ldx % 8 == 0 &&
             a.ldy % 8 == 0 && aligned16(a.x) && aligned16(a.y) && aligned16(a.w);
  if (ADD) vec = vec && a.ldr % 8 == 0 && a.lds % 8 == 0 && aligned16(a.r) && aligned16(a.s);
  const int64_t nvec = a.n / 8;
  const int lpr = p.bw / 2;
  const int64_t vpl = vec ? (nvec + lpr - 1) / lpr : 0;
  if (vec && vpl <= kRmsMaxVpl) {
    if (lpr == 32) return launch_rms_lpr<ADD, 32>(a, (int)nvec, (int)vpl, st);
    if (lpr == 16) return launch_rms_lpr<ADD, 16>(a, (int)nvec, (int)vpl, st);
  }
  if (a.rows > 0x7fffffffLL) return UMIC_ERR_UNSUPPORTED;
  // the wide rows (one to seven rows) with 8-byte vectors
  bool wide = p.vec && !p.split && p.bw >= 128 && a.n % 4 == 0 && a.ldx % 4 == 0 &&
              a.ldy % 4 == 0 && aligned8(a.x) && aligned8(a.y) && aligned8(a.w);
  if (ADD) wide = wide && a.ldr % 4 == 0 && a.lds % 4 == 0 && aligned8(a.r) && aligned8(a.s);
  const int64_t k4 = (a.n / 4 + p.bw - 1) / p.bw;
  if (wide && k4 <= 8) {
    const dim3 grid((unsigned)a.rows);
#define UMIC_RMS_WIDE(BW, K)                                                               \
  if (p.bw == BW && k4 <= K) {                                                              \
    hipLaunchKernelGGL((rms_wide_kernel<ADD, BW, K>), grid, dim3(BW), 0, st, a);           \
    return launch_status();                                                                 \
  }
    UMIC_RMS_WIDE(512, 2) UMIC_RMS_WIDE(512, 4) UMIC_RMS_WIDE(512, 8)
    UMIC_RMS_WIDE(256, 2) UMIC_RMS_WIDE(256, 4) UMIC_RMS_WIDE(256, 8)
    UMIC_RMS_WIDE(128, 2) UMIC_RMS_WIDE(128, 4) UMIC_RMS_WIDE(128, 8)
#undef UMIC_RMS_WIDE
  }
  const int threads = p.bw * (p.split ? p.bh : 1);
  hipLaunchKernelGGL((rms_block_kernel<ADD>), dim3((unsigned)a.rows), dim3(threads), 0, st, a,
                     p);
  return launch_status();
}

template <bool ADD, int M4>
int launch_ln_rows(const NormArgs& a, int nvec4, hipStream_t st) {
  const int threads = block_threads(a.rows * 16);
  const int rows_per_block = threads / 16;
  const int64_t blocks = (a.rows + rows_per_block - 1) / rows_per_block;
  if (blocks > 0x7fffffffLL) return UMIC_ERR_UNSUPPORTED;
  if (nvec4 == 64 * M4)
    hipLaunchKernelGGL((ln_rows_kernel<ADD, M4, true>), dim3((unsigned)blocks), dim3(threads), 0,
                       st, a, nvec4);
  else
    hipLaunchKernelGGL((ln_rows_kernel<ADD, M4, false>), dim3((unsigned)blocks), dim3(threads), 0,
                       st, a, nvec4);
  return launch_status();
}

template <bool ADD>
int launch_ln(const NormArgs& a, hipStream_t st) {
  if (a.rows > 0x7fffffffLL) return UMIC_ERR_UNSUPPORTED;
  // eager's layer_norm reads x itself when it is contiguous (else a fresh,
  // aligned copy; the add form normalises a fresh sum), and takes its
  // vectorized kernel for n % 4 == 0 with 8-byte aligned x, weight and bias
  const bool contiguous = a.rows == 1 || a.ldx == a.n;
  const bool torch_vec = a.n % 4 == 0 && a.n <= (1 << 24) && aligned8(a.w) && aligned8(a.b) &&
                         (ADD || !contiguous || aligned8(a.x));
  if (!torch_vec) {
    hipLaunchKernelGGL((ln_scalar_rows_kernel<ADD>), dim3((unsigned)((a.rows + 3) / 4)),
                       dim3(256), 0, st, a);
    return launch_status();
  }
  bool vec = a.ldx % 4 == 0 && a.ldy % 4 == 0 && aligned8(a.x) && aligned8(a.y);
  if (ADD) vec = vec && a.ldr % 4 == 0 && a.lds % 4 == 0 && aligned8(a.r) && aligned8(a.s);
  const int nvec4 = (int)(a.n / 4);
  if (vec) {
    switch ((nvec4 + 63) / 64) {  // register slots / 4
      case 1: return launch_ln_rows<ADD, 1>(a, nvec4, st);
      case 2: return launch_ln_rows<ADD, 2>(a, nvec4, st);
      case 3: return launch_ln_rows<ADD, 3>(a, nvec4, st);
      case 4: return launch_ln_rows<ADD, 4>(a, nvec4, st);
      case 5: return launch_ln_rows<ADD, 5>(a, nvec4, st);
      case 6: return launch_ln_rows<ADD, 6>(a, nvec4, st);
      case 7:
      case 8: return launch_ln_rows<ADD, 8>(a, nvec4, st);
      case 9:
      case 10: return launch_ln_rows<ADD, 10>(a, nvec4, st);
      case 11:
      case 12: return launch_ln_rows<ADD, 12>(a, nvec4, st);
      case 13:
      case 14:
      case 15:
      case 16: return launch_ln_rows<ADD, 16>(a, nvec4, st);
      default: break;
    }
  }
  hipLaunchKernelGGL((ln_torch_block_kernel<ADD>), dim3((unsigned)a.rows), dim3(256), 0, st, a);
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
  if constexpr (is_ln(OP)) return launch_ln<has_add(OP)>(a, as_stream(stream));
  return launch_rms<has_add(OP)>(a, as_stream(stream));
}

}  // namespace
}  // namespace umic

using namespace umic;

extern "C" int umic_rmsnorm_bf16(const void* x, const void* w, void* y, int64_t rows, int64_t n,
                                 int64_t ldx, int64_t ldy, float eps, void* stream) {
  NormArgs a{(const uint16_t*)x, nullptr, (const uint16_t*)w, nullptr, (uint16_t*)y, nullptr,
             rows, n, ldx, 0, ldy, 0, eps, 0.0f};
  return norm_entry<kRms>(a, stream);
}

extern "C" int umic_add_rmsnorm_bf16(const void* x, const void* r, const void* w, void* normed,
                                     void* summed, int64_t rows, int64_t n, int64_t ldx,
                                     int64_t ldr, int64_t ldn, int64_t lds, float eps,
                                     void* stream) {
  NormArgs a{(const uint16_t*)x, (const uint16_t*)r, (const uint16_t*)w, nullptr,
             (uint16_t*)normed, (uint16_t*)summed, rows, n, ldx, ldr, ldn, lds, eps, 0.0f};
  return norm_entry<kAddRms>(a, stream);
}

extern "C" int umic_layernorm_bf16(const void* x, const void* w, const void* b, void* y,
                                   int64_t rows, int64_t n, int64_t ldx, int64_t ldy, float eps,
                                   void* stream) {
  NormArgs a{(const uint16_t*)x, nullptr, (const uint16_t*)w, (const uint16_t*)b, (uint16_t*)y,
             nullptr, rows, n, ldx, 0, ldy, 0, eps, 0.0f};
  return norm_entry<kLn>(a, stream);
}

extern "C" int umic_add_layernorm_bf16(const void* x, const void* r, const void* w,
                                       const void* b, void* normed, void* summed, int64_t rows,
                                       int64_t n, int64_t ldx, int64_t ldr, int64_t ldn,
                                       int64_t lds, float eps, void* stream) {
  NormArgs a{(const uint16_t*)x, (const uint16_t*)r, (const uint16_t*)w, (const uint16_t*)b,
             (uint16_t*)normed, (uint16_t*)summed, rows, n, ldx, ldr, ldn, lds, eps, 0.0f};
  return norm_entry<kAddLn>(a, stream);
}
