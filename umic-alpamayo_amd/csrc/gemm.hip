// bf16 GEMMs on gfx950 MFMA for the UMIC projection sites:
//   linear         out = act(x @ w^T + bias)              (q_proj / o_proj)
//   gate_silu_mul  out = silu(x @ wg^T) * (x @ wu^T)      (P5 MLP front half)
// x: [M, K] row-major, weights [N, K] row-major (nn.Linear layout): both
// operands are K-contiguous, which is the native MFMA operand order, so no
// transpose or copy of the weights is ever made.
//
// Tile.  A workgroup owns 256 x rows x 256 weight rows of the K loop.  For
// the linear that is a 256 x 256 output tile; for P5 the 256 weight rows are
// 128 gate rows and the SAME 128 up rows, so one staged x tile feeds both
// products and the two fp32 accumulators of an output element sit in the
// same lane and register slot -- silu(g) * u is applied in registers and
// only the product is written.
//
// Waves.  Eight wavefronts, two per SIMD.  SIMD q (waves q and q + 4) owns
// a 128 x 128 quadrant; its two waves split it along x rows, 64 each, and
// compute 128 weight rows x 64 x rows as 8 x 4 blocks of
// v_mfma_f32_16x16x32_bf16 (128 fp32 accumulators per lane).  The 16x16x32
// form carries half the accumulator register traffic per FLOP of the
// 32x32x16 form; these GEMMs run at the board's power limit, where that
// buys clock (measured ~14% faster P5 at the same power).
//
// Ping-pong.  The two groups of four waves alternate roles each phase:
// while group 0 runs the 32 MFMAs of K step j from fragments it holds,
// group 1 reads its step-j fragments from LDS and issues the weight half
// of the direct-to-LDS loads of step j + D; the next phase swaps them
// (group 0 reads step j+1 fragments and loads the x half).  A barrier ends
// each phase, so every SIMD always has one wave with MFMAs ready and the
// other doing the memory work.
//
// Data movement.  Tiles move global -> LDS with direct-to-LDS buffer loads
// (buffer_load_dwordx4 ... lds, no register staging) through a ring of
// S = D + 1 stages of BK = 32 (5 x 32 KB = all 160 KB of LDS).  Buffer
// resources range-check rows past M / N to zero, so ragged edge tiles need
// no clamps.  LDS rows are XOR-swizzled so fragment reads are bank-conflict
// free (see Geo).  The MFMA A operand is the weight tile, B the x tile, so
// each lane's 4 results per block are 4 consecutive output columns: the
// epilogue writes 8-byte packed bf16 runs.
//
// Workgroup order.  Hardware hands consecutive workgroup ids to the 8 XCDs
// round-robin; the id is remapped so every XCD works through a contiguous
// run of a grouped tile order (4 tile rows at a time, m fastest), so the
// tiles one XCD runs together share x and weight slabs in its 4 MB L2.
#include "common.hpp"

namespace umic {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) char lds_char;

constexpr int kBM = 256;     // x rows per tile
constexpr int kBW = 256;     // weight rows per tile (gate+up for P5)
constexpr int kGroupM = 4;   // tile rows per L2 locality group
constexpr int kBK = 32;      // K per step (one 16x16x32 MFMA deep)
constexpr int kAhead = 4;    // steps in flight ahead of the one consumed
constexpr int kStages = kAhead + 1;
constexpr int kThreads = 512;

struct GemmArgs {
  const uint16_t* x;
  const uint16_t* w0;  // linear weight, or gate weight
  const uint16_t* w1;  // up weight (P5)
  const uint16_t* bias;
  uint16_t* out;
  int64_t M, N, K, ldx, ldw0, ldw1, ldo;
  int tiles_m, tiles;
};

// LDS geometry of one operand tile of a K step: a row is BK bf16 = 64 bytes
// = CPR 16-byte chunks; one direct-to-LDS wave instruction moves 64 x 16 B
// = 1 KB = RPI consecutive rows.  A fragment read (ds_read_b128) has lane l
// on row l % 16, chunk l / 16.  The chunk is XOR-swizzled by (row >> 1) & 3:
// measured with SQ_LDS_BANK_CONFLICT on gfx950, that read pattern is
// conflict-free under this swizzle, 2-way under (row >> 2) & 3, row & 3 or
// none.  Direct-to-LDS writes are 1 KB contiguous and conflict-free.
struct Geo {
  static constexpr int CPR = kBK / 8;
  static constexpr int RPI = 64 / CPR;
  static __device__ __forceinline__ int swz(int row) { return (row >> 1) & 3; }
  static __device__ __forceinline__ int slot(int row, int chunk) {
    return row * CPR + (chunk ^ swz(row));
  }
};

// Wait until at most PENDING of this wave's direct-to-LDS loads are still
// in flight (the older ones have landed) and its LDS reads are done, then
// s_barrier.  Written out (rather than __syncthreads, whose fence drains
// every load) so the younger stages stay in flight across the barrier; the
// asm is a compiler memory barrier, so no LDS access moves across it.
template <int PENDING>
__device__ __forceinline__ void stage_barrier() {
  static_assert(PENDING >= 0 && PENDING < 64, "vmcnt is 6 bits");
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(PENDING) : "memory");
}

// Hazards of the ring.  Step j's stage is read in phases 2j-1 (group 0) and
// 2j (group 1) and refilled (as step j + S) in phases 2j+2 / 2j+3, after
// two barriers, each preceded by lgkmcnt(0).  Step j+1's two load batches
// were issued in phases 2(j+1-D) (weights, group 1) and 2(j+1-D)+1 (x,
// group 0).  At the barrier ending phase 2j, group 1 has D batches
// outstanding at most and waits for all but D-1; group 0 has issued one
// batch fewer and waits for all but D-2: both halves of step j+1 have
// landed before anyone reads it in phase 2j+1.  Barriers ending odd phases
// need no load wait (the same counts are already met there).
template <int NB, int ACT, bool BIAS>
__global__ __launch_bounds__(kThreads, 1) void gemm_kernel(GemmArgs g) {
  using G = Geo;
  constexpr int CPR = G::CPR, RPI = G::RPI;
  constexpr int D = kAhead, S = kStages;
  constexpr int LB = 64 / RPI;  // direct-to-LDS loads per wave per batch
  // [stage][operand: 0 weights, 1 x][row * CPR + slot], 16-byte units
  __shared__ u32x4 lds[S][2][kBM * CPR];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // wave-uniform (scalar) wave index: the operand pointer chosen from it
  // must live in SGPRs for the buffer resource
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wave >> 2, q = wave & 3;
  const int wm = q & 1, wn = q >> 1;

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

  // The operand this wave streams: group 1 the weight tile (for P5 waves
  // 0-1 of the group the gate rows, 2-3 the up rows), group 0 the x tile,
  // 64 rows per wave.  Rows past M / N read as zero.
  const int opnd = grp ? 0 : 1;
  const bool up = NB == 2 && grp && q >= 2;
  const uint16_t* src = grp ? (up ? g.w1 : g.w0) : g.x;
  const int64_t ld = grp ? (up ? g.ldw1 : g.ldw0) : g.ldx;
  const int64_t nrows = grp ? g.N : g.M;
  const int row0 = grp ? (NB == 1 ? n0 + q * 64 : n0 + (q & 1) * 64) : m0 + q * 64;
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc((void*)src, (short)0, (int)(nrows * ld * 2), 0x00020000);
  // Lane l writes LDS slot l % CPR of row l / CPR of each 1 KB group, so it
  // fetches the chunk the swizzle places there (the swizzle of tile row
  // q*64 + j*RPI + lr depends only on lr).
  const int lr = lane / CPR;
  const int off0 = (int)((int64_t)(row0 + lr) * ld * 2);
  const int rstep = (int)(RPI * ld * 2);
  auto issue = [&](int stage, int k0) {
    lds_char* d = (lds_char*)&lds[stage][opnd][q * 64 * CPR];
#pragma unroll
    for (int j = 0; j < LB; ++j) {
      const int co = ((lane % CPR) ^ G::swz(j * RPI + lr)) * 16 + k0 * 2;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)(d + j * 1024), 16,
                                               off0 + j * rstep + co, 0, 0, 0);
    }
  };

  // Fragment blocks of 16 rows: weights (A) -- linear: rows wn*128 + a*16;
  // P5: gate rows wn*64 + a*16 (a < 4) and the matching up rows
  // 128 + wn*64 + (a-4)*16 -- and x (B): rows wm*128 + grp*64 + b*16.
  int arow[8], brow[4];
#pragma unroll
  for (int a = 0; a < 8; ++a)
    arow[a] = NB == 1 ? wn * 128 + a * 16 : (a >> 2) * 128 + wn * 64 + (a & 3) * 16;
#pragma unroll
  for (int b = 0; b < 4; ++b) brow[b] = wm * 128 + grp * 64 + b * 16;
  const int frow = lane & 15;  // fragment row of this lane
  const int fch = lane >> 4;   // its 8-element K chunk

  f32x4_t acc[8][4];
#pragma unroll
  for (int a = 0; a < 8; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[a][b][r] = 0.f;

  bf16x8_t fa[8], fb[4];
  auto frags = [&](int stage) {
#pragma unroll
    for (int a = 0; a < 8; ++a)
      fa[a] = __builtin_bit_cast(bf16x8_t, lds[stage][0][G::slot(arow[a] + frow, fch)]);
#pragma unroll
    for (int b = 0; b < 4; ++b)
      fb[b] = __builtin_bit_cast(bf16x8_t, lds[stage][1][G::slot(brow[b] + frow, fch)]);
  };
  auto compute = [&]() {
#pragma unroll
    for (int a = 0; a < 8; ++a)
#pragma unroll
      for (int b = 0; b < 4; ++b)
        acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[a], fb[b], acc[a][b], 0, 0, 0);
  };

  const int KT = (int)(g.K / kBK);
  // Prologue: D steps in flight, step 0 landed, group 0 holds its step-0
  // fragments.  The loop stays branch-free: the last D steps still refill
  // stages that are never read again, from offsets past K (in-range data or
  // range-checked zeros), and group 0 reads step-KT fragments it never uses.
#pragma unroll
  for (int s = 0; s < D; ++s) issue(s, s * kBK);
  stage_barrier<(D - 1) * LB>();
  if (grp == 0) frags(0);
  stage_barrier<(D - 1) * LB>();

  // One straight loop per group (the hardware barrier counts arrivals, not
  // program points; both loops pass the same barriers), so the fragments
  // stay loop-carried in place.  sched_barrier keeps every MFMA in its phase.
  if (grp == 0) {
    for (int j = 0; j < KT; ++j) {
      compute();
      __builtin_amdgcn_sched_barrier(0);
      stage_barrier<(D - 2) * LB>();
      __builtin_amdgcn_sched_barrier(0);
      frags((j + 1) % S);
      issue((j + D) % S, (j + D) * kBK);
      __builtin_amdgcn_sched_barrier(0);
      stage_barrier<(D - 1) * LB>();
      __builtin_amdgcn_sched_barrier(0);
    }
  } else {
    for (int j = 0; j < KT; ++j) {
      frags(j % S);
      issue((j + D) % S, (j + D) * kBK);
      __builtin_amdgcn_sched_barrier(0);
      stage_barrier<(D - 1) * LB>();
      __builtin_amdgcn_sched_barrier(0);
      compute();
      __builtin_amdgcn_sched_barrier(0);
      stage_barrier<(D - 1) * LB>();
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // No direct-to-LDS load may still be in flight when the workgroup's LDS
  // is released.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // Epilogue.  acc[a][b][e]: x row brow[b] + lane % 16, weight row
  // arow[a] + 4 * (lane / 16) + e.
  constexpr int kOutBlocks = NB == 1 ? 8 : 4;
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const int64_t m = (int64_t)m0 + brow[b] + frow;
    if (m >= g.M) continue;
    uint16_t* orow = g.out + m * g.ldo;
#pragma unroll
    for (int a = 0; a < kOutBlocks; ++a) {
      const int64_t n = n0 + (NB == 1 ? arow[a] : wn * 64 + a * 16) + fch * 4;
      if (n >= g.N) continue;
      float o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float v = acc[a][b][e];
        if constexpr (NB == 2) {
          // silu(g) * u with the hardware exp2 / reciprocal (~1 ulp each,
          // far inside the bf16 output rounding); large |g| saturates
          // correctly: exp -> inf gives rcp -> 0, exp -> 0 gives rcp -> 1.
          const float u = acc[a + 4][b][e];
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

template <int NB, int ACT, bool BIAS>
int launch_gemm(GemmArgs g, hipStream_t st) {
  const int64_t bn = NB == 1 ? kBW : kBW / 2;
  const int64_t tm = (g.M + kBM - 1) / kBM;
  const int64_t tn = (g.N + bn - 1) / bn;
  if (tm * tn > (int64_t)1 << 28) return UMIC_ERR_UNSUPPORTED;
  g.tiles_m = (int)tm;
  g.tiles = (int)(tm * tn);
  const int64_t grid = ((g.tiles + 7) / 8) * 8;
  hipLaunchKernelGGL((gemm_kernel<NB, ACT, BIAS>), dim3((unsigned)grid), dim3(kThreads), 0, st, g);
  return launch_status();
}

// Buffer-resource offsets are 32-bit: every operand (rows x leading dim),
// plus the K overrun of the last steps' refills (kAhead steps past K), must
// stay below 2 GiB.
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
