// bf16 GEMMs on gfx950 MFMA for the UMIC projection sites:
//   linear         out = act(x @ w^T + bias)              (q_proj / o_proj)
//   gate_silu_mul  out = silu(x @ wg^T) * (x @ wu^T)      (P5 MLP front half)
// x: [M, K] row-major, weights [N, K] row-major (nn.Linear layout): both
// operands are K-contiguous, which is the native MFMA operand order, so no
// transpose or copy of the weights is ever made.
//
// Tiling.  A 256-thread workgroup (4 wavefronts, 2 x 2) owns a 256 (x rows)
// x 256 (weight rows) tile of the K loop.  For the linear that is a
// 256 x 256 output tile; for P5 the 256 weight rows are 128 gate rows and
// the SAME 128 up rows, so one staged x tile feeds both products and the
// two fp32 accumulators for an output element sit in the same lane and
// register slot -- silu(g) * u is applied in registers and only the product
// is written.  Each wavefront computes 128 weight rows x 128 x rows with a
// 4 x 4 grid of v_mfma_f32_32x32x16_bf16 (256 fp32 accumulators per lane).
//
// Data movement.  Tiles move global -> LDS with direct-to-LDS buffer loads
// (buffer_load_dwordx4 ... lds, no register staging) through a multi-stage
// LDS ring, one barrier per K step; LDS rows are XOR-swizzled so fragment
// reads are bank-conflict free (see Geo).  The MFMA A operand is the weight tile, B the x tile,
// so each lane's 16 outputs are 4 runs of 4 consecutive output columns:
// the epilogue writes 8-byte packed bf16 runs.
//
// Workgroup order.  Hardware hands consecutive workgroup ids to the 8 XCDs
// round-robin; the id is remapped so every XCD works through a contiguous
// run of a grouped tile order (4 tile rows at a time, m fastest), so the
// tiles one XCD runs together share x and weight slabs in its 4 MB L2.
#include "common.hpp"

namespace umic {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr int kBM = 256;     // x rows per tile
constexpr int kBW = 256;     // weight rows per tile (gate+up for P5)
constexpr int kGroupM = 4;   // tile rows per L2 locality group

struct GemmArgs {
  const uint16_t* x;
  const uint16_t* w0;  // linear weight, or gate weight
  const uint16_t* w1;  // up weight (P5)
  const uint16_t* bias;
  uint16_t* out;
  int64_t M, N, K, ldx, ldw0, ldw1, ldo;
  int tiles_m, tiles;
};

// LDS geometry for a K step of BK elements.  A tile row is BK bf16 = BK*2
// bytes = CPR 16-byte chunks; one direct-to-LDS wave instruction moves
// 64 x 16 B = 1 KB = RPI consecutive rows.  gfx950's LDS serves 16 lanes x
// 16 B = 256 B (64 banks) per cycle, and an MFMA fragment read has those 16
// lanes on 16 consecutive rows at one chunk, so the chunk is XOR-swizzled
// to give every row of a 256-byte bank line group a distinct 16-byte slot:
// 128 B rows pair up per bank line, so rows r and r+2, r+4, ... r+14 must
// differ -> (row >> 1) & 7; 64 B rows come four to a bank line -> (row >> 2) & 3.
template <int BK>
struct Geo {
  static constexpr int CPR = BK / 8;
  static constexpr int RPI = 64 / CPR;
  static __device__ __forceinline__ int swz(int row) {
    if constexpr (BK == 64) return (row >> 1) & 7;
    else return (row >> 2) & 3;
  }
  static __device__ __forceinline__ int slot(int row, int chunk) {
    return row * CPR + (chunk ^ swz(row));
  }
};

// Workgroup barrier for the LDS pipeline: wait until at most PENDING of this
// wave's direct-to-LDS loads are still in flight (the older ones -- the next
// stage -- have landed) and its LDS reads are done, then s_barrier.  Written
// out (rather than __syncthreads, whose fence drains every load) so the
// deeper stages stay in flight across the barrier; the asm is a compiler
// memory barrier, so no LDS access moves across it.
template <int PENDING>
__device__ __forceinline__ void stage_barrier() {
  static_assert(PENDING >= 0 && PENDING < 64, "vmcnt is 6 bits");
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(PENDING) : "memory");
}

// SCHED selects how the MFMA stream is interleaved with LDS reads and the
// direct-to-LDS loads inside a K step: 0 leaves it to the compiler, 1 and 2
// are the compiler's built-in GEMM strategies (iglp_opt 0 / 1), 3 pins one
// LDS read (and on the first slice one load) after each of the first MFMAs
// and fences each K slice, 4 only fences each K slice, 5 is 3 with the K
// step's loads issued an equal share per slice, spread between the MFMAs.
template <int NB, int ACT, bool BIAS, int BK, int STAGES, int SCHED>
__global__ __launch_bounds__(256, 1) void gemm_kernel(GemmArgs g) {
  using G = Geo<BK>;
  constexpr int CPR = G::CPR, RPI = G::RPI;
  constexpr int KK = BK / 16;                  // MFMA K slices per stage
  constexpr int L = 2 * (64 / RPI);            // DMA instructions per wave per stage
  // [stage][operand: 0 weights, 1 x][row * CPR + slot], 16-byte units
  __shared__ u32x4 lds[STAGES][2][kBM * CPR];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // wave-uniform (scalar) wave index: the operand pointers chosen from it
  // must live in SGPRs for the buffer resources
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 1, wn = wave >> 1;

  // XCD-aware remap: physical ids b, b+8, b+16, ... (one XCD) take
  // consecutive logical tiles; logical tiles run in groups of kGroupM tile
  // rows, m fastest inside a group, so the ~32 tiles an XCD holds at once
  // form a kGroupM x 8 block whose x and weight slabs its L2 shares.
  const int per_xcd = (g.tiles + 7) >> 3;
  const int logical = (int)(blockIdx.x & 7) * per_xcd + (int)(blockIdx.x >> 3);
  if (logical >= g.tiles) return;
  const int tiles_n = g.tiles / g.tiles_m;
  const int group = logical / (kGroupM * tiles_n);
  const int first_m = group * kGroupM;
  const int gm = min(g.tiles_m - first_m, kGroupM);
  const int in_group = logical - group * kGroupM * tiles_n;
  const int tm = first_m + in_group % gm;
  const int tn = in_group / gm;
  const int m0 = tm * kBM;
  const int n0 = tn * (NB == 1 ? kBW : kBW / 2);

  // Buffer resources: rows past M / N read as zero (hardware range check),
  // so ragged edge tiles need no clamping or predication in the K loop.
  const __amdgpu_buffer_rsrc_t rx =
      __builtin_amdgcn_make_buffer_rsrc((void*)g.x, (short)0, (int)(g.M * g.ldx * 2), 0x00020000);
  const uint16_t* wsrc = (NB == 2 && wave >= 2) ? g.w1 : g.w0;
  const int64_t ldw = (NB == 2 && wave >= 2) ? g.ldw1 : g.ldw0;
  const __amdgpu_buffer_rsrc_t rw =
      __builtin_amdgcn_make_buffer_rsrc((void*)wsrc, (short)0, (int)(g.N * ldw * 2), 0x00020000);

  // This wave DMAs tile rows [wave*64, wave*64+64) of both operands.  Lane
  // l writes LDS slot l % CPR of row l / CPR of each 1 KB group, so it
  // fetches the chunk that the swizzle places there (the swizzle of row
  // wave*64 + j*RPI + lr depends only on j and lr).
  const int lr = lane / CPR;
  const int wrow0 = NB == 1 ? n0 + wave * 64 : n0 + (wave & 1) * 64;
  const int xrow0 = m0 + wave * 64;
  const int woff = (int)((int64_t)(wrow0 + lr) * ldw * 2);
  const int xoff = (int)((int64_t)(xrow0 + lr) * g.ldx * 2);
  const int wstep = (int)(RPI * ldw * 2), xstep = (int)(RPI * g.ldx * 2);
  auto chunk_off = [&](int j) { return ((lane % CPR) ^ G::swz(j * RPI + lr)) * 16; };

  // Issue rows-blocks [j0, j1) of this wave's share of a K step's tiles.
  auto issue_part = [&](int stage, int k0, int j0, int j1) {
    lds_void* dw = (lds_void*)&lds[stage][0][wave * 64 * CPR];
    lds_void* dx = (lds_void*)&lds[stage][1][wave * 64 * CPR];
#pragma unroll
    for (int j = j0; j < j1; ++j) {
      const int co = chunk_off(j) + k0 * 2;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lds_void*)((__attribute__((address_space(3))) char*)dw + j * 1024),
                                               16, woff + j * wstep + co, 0, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_void*)((__attribute__((address_space(3))) char*)dx + j * 1024),
                                               16, xoff + j * xstep + co, 0, 0, 0);
    }
  };
  auto issue = [&](int stage, int k0) { issue_part(stage, k0, 0, 64 / RPI); };

  // Fragment rows: a-blocks (weights) and b-blocks (x), 32 rows each.
  int arow[4], brow[4];
#pragma unroll
  for (int a = 0; a < 4; ++a) {
    arow[a] = NB == 1 ? wn * 128 + a * 32 : (a >> 1) * 128 + wn * 64 + (a & 1) * 32;
    brow[a] = wm * 128 + a * 32;
  }
  const int frow = lane & 31;
  const int fk = lane >> 5;  // which 8-element half of a 16-wide K slice

  f32x16_t acc[4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.f;

  bf16x8_t fa[2][4], fb[2][4];
  auto frags = [&](int buf, int stage, int kk) {
    const int ch = kk * 2 + fk;
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      fa[buf][a] = __builtin_bit_cast(bf16x8_t, lds[stage][0][G::slot(arow[a] + frow, ch)]);
      fb[buf][a] = __builtin_bit_cast(bf16x8_t, lds[stage][1][G::slot(brow[a] + frow, ch)]);
    }
  };
  auto mma = [&](int buf) {
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int b = 0; b < 4; ++b)
        acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[buf][a], fb[buf][b], acc[a][b], 0, 0, 0);
  };

  const int KT = (int)(g.K / BK);
  // Prologue: STAGES-1 K steps in flight, wait for the first.
#pragma unroll
  for (int s = 0; s < STAGES - 1; ++s)
    if (s < KT) issue(s, s * BK);
  if (KT >= STAGES - 1) stage_barrier<(STAGES - 2) * L>();
  else stage_barrier<0>();
  frags(0, 0, 0);

  // The loop body is branch-free (one basic block the scheduler can
  // interleave): the last STAGES-1 steps still refill a buffer that is never
  // read again, from offsets past K -- in-range garbage or range-checked
  // zeros -- and the last step reads next-stage fragments it never uses.
  for (int kt = 0; kt < KT; ++kt) {
    const int st = kt % STAGES;
    // Refill the buffer consumed in the previous step (all waves are past
    // the barrier that ended their reads of it): all at once, or (SCHED 5)
    // an equal share in each K slice so the loads issue evenly between MFMAs.
    constexpr int kJ = 64 / RPI;  // row blocks per operand per wave
    if constexpr (SCHED != 5) issue((kt + STAGES - 1) % STAGES, (kt + STAGES - 1) * BK);
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      const int cur = kk & 1;
      if constexpr (SCHED == 5)
        issue_part((kt + STAGES - 1) % STAGES, (kt + STAGES - 1) * BK, kk * kJ / KK,
                   (kk + 1) * kJ / KK);
      if constexpr (SCHED == 1) __builtin_amdgcn_iglp_opt(0);
      if constexpr (SCHED == 2) __builtin_amdgcn_iglp_opt(1);
      if (kk < KK - 1) {
        frags(cur ^ 1, st, kk + 1);
      } else {
        // Step kt+1's tile must have landed (the STAGES-2 younger steps'
        // loads may stay in flight), then everyone may start reading it.
        stage_barrier<(STAGES - 2) * L>();
        frags(cur ^ 1, (kt + 1) % STAGES, 0);
      }
      mma(cur);
      if constexpr (SCHED == 3) {
        // 16 MFMAs of this slice: the first 8 each followed by one fragment
        // read for the next slice; on the first slice the step's
        // direct-to-LDS loads (2 * 64 / RPI per wave) ride between them too.
        constexpr int kLoads = 2 * (64 / RPI);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
          if (i < 8) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
          if (kk == 0 && i < kLoads) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM
        }
      }
      if constexpr (SCHED == 5) {
        // 16 MFMAs of this slice, one fragment read after each of the first
        // 8 and this slice's share of the loads spread evenly between them.
        constexpr int kLoadsPerSlice = 2 * kJ / KK;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
          if (i < 8) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
          if (i % (16 / kLoadsPerSlice) == 0) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
        }
      }
      // Nothing crosses a slice boundary: the next slice's MFMAs cannot be
      // hoisted onto fragments still in flight, so those fragments load
      // under this slice's MFMAs (a real double buffer).
      if constexpr (SCHED >= 3) __builtin_amdgcn_sched_barrier(0);
    }
  }
  // No direct-to-LDS load may still be in flight when the workgroup's LDS
  // is released.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // Epilogue.  acc[a][b][r]: weight row 8*(r/4) + 4*(lane/32) + r%4 of
  // a-block a, x row lane%32 of b-block b.
  constexpr int kOutBlocks = NB == 1 ? 4 : 2;
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const int64_t m = (int64_t)m0 + brow[b] + frow;
    if (m >= g.M) continue;
    uint16_t* orow = g.out + m * g.ldo;
#pragma unroll
    for (int a = 0; a < kOutBlocks; ++a) {
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int64_t n = n0 + (NB == 1 ? arow[a] : wn * 64 + a * 32) + rr * 8 + fk * 4;
        if (n >= g.N) continue;
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float v = acc[a][b][rr * 4 + e];
          if constexpr (NB == 2) {
            // silu(g) * u with the hardware exp2 / reciprocal (~1 ulp each,
            // far inside the bf16 output rounding); large |g| saturates
            // correctly: exp -> inf gives rcp -> 0, exp -> 0 gives rcp -> 1.
            const float u = acc[a + 2][b][rr * 4 + e];
            const float den = 1.0f + __builtin_amdgcn_exp2f(v * -1.4426950408889634f);
            v = v * __builtin_amdgcn_rcpf(den) * u;
          } else {
            if constexpr (BIAS) v = v + bf2f(g.bias[n + e]);
            if constexpr (ACT == UMIC_ACT_GELU) v = 0.5f * v * (1.0f + erff(v * 0.70710678118654752f));
          }
          o[e] = v;
        }
        uint2 pk;
        pk.x = pack2(o[0], o[1]);
        pk.y = pack2(o[2], o[3]);
        *reinterpret_cast<uint2*>(orow + n) = pk;
      }
    }
  }
}

constexpr int kBK = 32;
constexpr int kStages = 4;
constexpr int kSched = 5;

template <int NB, int ACT, bool BIAS>
int launch_gemm(GemmArgs g, hipStream_t st) {
  const int64_t bn = NB == 1 ? kBW : kBW / 2;
  const int64_t tm = (g.M + kBM - 1) / kBM;
  const int64_t tn = (g.N + bn - 1) / bn;
  if (tm * tn > (int64_t)1 << 28) return UMIC_ERR_UNSUPPORTED;
  g.tiles_m = (int)tm;
  g.tiles = (int)(tm * tn);
  const int64_t grid = ((g.tiles + 7) / 8) * 8;
  hipLaunchKernelGGL((gemm_kernel<NB, ACT, BIAS, kBK, kStages, kSched>), dim3((unsigned)grid),
                     dim3(256), 0, st, g);
  return launch_status();
}

// Buffer-resource offsets are 32-bit: every operand (rows x leading dim),
// plus the K overrun of the last steps' refills (STAGES-1 steps past K),
// must stay below 2 GiB.
bool gemm_shape_ok(const void* x, const void* w0, const void* w1, const void* out, int64_t M,
                   int64_t N, int64_t K, int64_t ldx, int64_t ldw0, int64_t ldw1, int64_t ldo) {
  if (K % kBK != 0 || N % 8 != 0) return false;
  if (ldx % 8 || ldw0 % 8 || ldw1 % 8 || ldo % 8) return false;
  if (!aligned16(x) || !aligned16(w0) || !aligned16(w1) || !aligned16(out)) return false;
  const int64_t lim = (int64_t)1 << 30;  // elements (2 GiB of bf16)
  const int64_t mpad = (M + kBM - 1) / kBM * kBM, npad = (N + kBW - 1) / kBW * kBW;
  const int64_t slack = (int64_t)kStages * kBK;
  if (mpad * ldx + slack >= lim || npad * ldw0 + slack >= lim || npad * ldw1 + slack >= lim)
    return false;
  return true;
}

}  // namespace
}  // namespace umic

using namespace umic;

extern "C" int umic_linear_bf16(const void* x, const void* w, const void* bias, void* out,
                                int64_t M, int64_t N, int64_t K, int64_t ldx, int64_t ldw,
                                int64_t ldo, int act, void* stream) {
  if (M < 0 || N < 0 || K < 0) return UMIC_ERR_INVALID_ARG;
  if (act != UMIC_ACT_NONE && act != UMIC_ACT_GELU) return UMIC_ERR_INVALID_ARG;
  if (M == 0 || N == 0) return UMIC_OK;  // empty tensors may carry null pointers
  if (!x || !w || !out) return UMIC_ERR_INVALID_ARG;
  if (ldx < K || ldw < K || ldo < N) return UMIC_ERR_INVALID_ARG;
  if (K == 0) return UMIC_ERR_UNSUPPORTED;
  if (!gemm_shape_ok(x, w, w, out, M, N, K, ldx, ldw, ldw, ldo)) return UMIC_ERR_UNSUPPORTED;
  if (bias && ((uintptr_t)bias & 7u)) return UMIC_ERR_UNSUPPORTED;
  GemmArgs g{(const uint16_t*)x, (const uint16_t*)w, (const uint16_t*)w, (const uint16_t*)bias,
             (uint16_t*)out, M, N, K, ldx, ldw, ldw, ldo, 0, 0};
  hipStream_t st = as_stream(stream);
  if (act == UMIC_ACT_GELU)
    return bias ? launch_gemm<1, UMIC_ACT_GELU, true>(g, st) : launch_gemm<1, UMIC_ACT_GELU, false>(g, st);
  return bias ? launch_gemm<1, UMIC_ACT_NONE, true>(g, st) : launch_gemm<1, UMIC_ACT_NONE, false>(g, st);
}

extern "C" int umic_gate_silu_mul_bf16(const void* x, const void* wg, const void* wu, void* out,
                                       int64_t M, int64_t N, int64_t K, int64_t ldx,
                                       int64_t ldwg, int64_t ldwu, int64_t ldo, void* stream) {
  if (M < 0 || N < 0 || K < 0) return UMIC_ERR_INVALID_ARG;
  if (M == 0 || N == 0) return UMIC_OK;  // empty tensors may carry null pointers
  if (!x || !wg || !wu || !out) return UMIC_ERR_INVALID_ARG;
  if (ldx < K || ldwg < K || ldwu < K || ldo < N) return UMIC_ERR_INVALID_ARG;
  if (K == 0) return UMIC_ERR_UNSUPPORTED;
  if (!gemm_shape_ok(x, wg, wu, out, M, N, K, ldx, ldwg, ldwu, ldo)) return UMIC_ERR_UNSUPPORTED;
  GemmArgs g{(const uint16_t*)x, (const uint16_t*)wg, (const uint16_t*)wu, nullptr,
             (uint16_t*)out, M, N, K, ldx, ldwg, ldwu, ldo, 0, 0};
  return launch_gemm<2, UMIC_ACT_NONE, false>(g, as_stream(stream));
}
