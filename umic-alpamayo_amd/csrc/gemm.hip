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

#include <algorithm>
#include <type_traits>
#include <map>
#include <mutex>
#include <utility>

namespace umic {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) char lds_char;

constexpr int kBM = 256;     // x rows per tile
constexpr int kBW = 256;     // weight rows per tile (gate+up for P5)
// tile rows per L2 locality group of data-parallel launches: multi-round
// launches (P5: 4.9 rounds) read the fewest L2-miss bytes with 4 (1.29 GB per
// P5 launch against 1.40 GB with 7, at equal speed); single-round launches
// (q/o) run 2-3% faster with 7
constexpr int kGroupMRounds = 4;
constexpr int kGroupMOne = 7;
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
  int bm;  // x rows a tile owns: M spread evenly over tiles_m, a multiple of 16, <= kBM
  int gm;  // tile rows per L2 locality group of the tile order
};

// The row-tile height for M rows when the tiles span several rounds of the
// CUs: the ceil(M / kBM) tiles a kBM-row tiling needs, each taking an even
// share rounded up to whole 16-row fragments.  At M = 3100 that is 13 tiles
// of 240 rows instead of 12 full ones and one of 28 live rows, whose tiles
// loaded a whole weight tile for 1% of the work in a slot of a later round.
// Measured in one process against fixed 256-row tiles: P5 (1248 tiles) 2.6%
// faster; the single-round q/o launch (208 tiles) 8% slower, so launches
// that fit one round, and the stream-K schedule, keep kBM-row tiles.
inline int tile_rows(int64_t M) {
  const int64_t tm = (M + kBM - 1) / kBM;
  const int64_t share = (M + tm - 1) / tm;
  return (int)std::min<int64_t>(kBM, (share + 15) / 16 * 16);
}

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

typedef u32x4 LdsRing[kStages][2][kBM * Geo::CPR];

// Exact-erf GELU for the linear's epilogue, formed as eager does:
// GELU(x) = 0.5 * x * (1 + erf(x / sqrt2)) in fp32.  erf(|u|) is taken as
// 1 - erfc(|u|) rounded to fp32, with erfc(z) = t * exp(-z^2 + P(t)),
// t = 1 / (1 + z/2) -- the functional form of Numerical Recipes' erfcc
// (W. H. Press et al., 2nd ed., sec. 6.2).  The coefficients of P are this
// library's own least-squares fit in float64 of log(erfc(z) / t) + z^2 on
// z in [0, 10]; evaluated in fp32 with the hardware reciprocal and exp2,
// erfc is within 1.5e-5 relative on [0, 10], so the fp32 erf matches a
// correctly rounded erff to about an ulp (tests/test_gelu_epilogue.py
// re-checks these constants).  Forming 1 + erf in fp32 keeps eager's
// behaviour for very negative x, where it cancels to 0 or to one ulp of 1
// (the more accurate x/2 * erfc(|u|) would differ from eager there by many
// bf16 ulps).  About 17 VALU operations against the library erff's branches.
__device__ __forceinline__ float gelu_erf(float x) {
  const float z = __builtin_fabsf(x) * 0.70710678118654752f;
  const float t = __builtin_amdgcn_rcpf(1.0f + 0.5f * z);
  float p = 1.449302137e-01f;
  p = __builtin_fmaf(p, t, -6.808271779e-01f);
  p = __builtin_fmaf(p, t, 1.156733757e+00f);
  p = __builtin_fmaf(p, t, -6.962518993e-01f);
  p = __builtin_fmaf(p, t, -8.028043184e-02f);
  p = __builtin_fmaf(p, t, 1.267586182e-03f);
  p = __builtin_fmaf(p, t, 3.460280007e-02f);
  p = __builtin_fmaf(p, t, 3.866404121e-01f);
  p = __builtin_fmaf(p, t, 9.986327833e-01f);
  p = __builtin_fmaf(p, t, -1.265447997e+00f);
  const float erfc_z = t * __builtin_amdgcn_exp2f((p - z * z) * 1.4426950408889634f);
  const float erf_abs = 1.0f - erfc_z;
  return 0.5f * x * (1.0f + (x < 0.0f ? -erf_abs : erf_abs));
}

// tanh-approximate GELU, as torch's gelu(approximate="tanh") (HF
// gelu_pytorch_tanh, the Qwen3-VL ViT MLP's activation) forms it in fp32:
// 0.5 x (1 + tanh(y)), y = sqrt(2/pi) (x + 0.044715 x^3) in the same
// operation order.  tanh|y| = 1 - 2 / (1 + exp(2|y|)) with the hardware exp2
// and reciprocal: the final subtraction puts it on the fp32 grid of [0.5, 1),
// as tanhf's result, so 1 + tanh(y) cancels in the negative tail exactly as
// eager's does; it is exactly 1 where exp overflows.
__device__ __forceinline__ float gelu_tanh(float x) {
  const float y = 0.7978845608028654f * (x + 0.044715f * (x * x * x));
  const float e = __builtin_amdgcn_exp2f(__builtin_fabsf(y) * 2.8853900817779268f);  // exp(2|y|)
  const float th_abs = 1.0f - 2.0f * __builtin_amdgcn_rcpf(1.0f + e);
  return 0.5f * x * (1.0f + (y < 0.0f ? -th_abs : th_abs));
}

// Tile origin of logical tile t in the grouped order: groups of g.gm tile
// rows, m fastest inside a group.
__device__ __forceinline__ void tile_origin(const GemmArgs& g, int t, int bw, int& m0, int& n0) {
  const int tiles_n = g.tiles / g.tiles_m;
  const int group = t / (g.gm * tiles_n);
  const int first_m = group * g.gm;
  const int gm = min(g.tiles_m - first_m, g.gm);
  const int in_group = t - group * g.gm * tiles_n;
  m0 = (first_m + in_group % gm) * g.bm;
  n0 = (in_group / gm) * bw;
}

// XCD-aware remap of a physical workgroup id: ids b, b+8, b+16, ... (one
// XCD, which the hardware fills round-robin) take consecutive logical ids,
// so what one XCD runs together is a contiguous run of the grouped order
// (for tiles: a block of g.gm tile rows by a few columns whose x and weight
// slabs its L2 shares).
__device__ __forceinline__ int xcd_remap(int count) {
  const int per_xcd = (count + 7) >> 3;
  return (int)(blockIdx.x & 7) * per_xcd + (int)(blockIdx.x >> 3);
}

// One wavefront's share of the ping-pong pipeline for one tile: which
// operand rows it streams into LDS, which fragments it reads, and its
// 8 x 4 blocks of 16x16 accumulators.
//
// Hazards of the ring (per K segment run by run()).  Step j's stage is read
// in phases 2j-1 (group 0) and 2j (group 1) and refilled (as step j + S) in
// phases 2j+2 / 2j+3, after two barriers, each preceded by lgkmcnt(0).
// Step j+1's two load batches were issued in phases 2(j+1-D) (weights,
// group 1) and 2(j+1-D)+1 (x, group 0).  At the barrier ending phase 2j,
// group 1 has D batches outstanding at most and waits for all but D-1;
// group 0 has issued one batch fewer and waits for all but D-2: both halves
// of step j+1 have landed before anyone reads it in phase 2j+1.  Barriers
// ending odd phases need no load wait (the same counts are already met).
template <int NB>
struct Pipe {
  static constexpr int CPR = Geo::CPR, RPI = Geo::RPI;
  static constexpr int D = kAhead, S = kStages;
  static constexpr int LB = 64 / RPI;  // direct-to-LDS loads per wave per batch

  int lane, grp, q, wm, wn, frow, fch, lr, opnd;
  int nbv;  // x fragments of this wave with rows inside M (wave-uniform, 0..4)
  int arow[8], brow[4];
  // The streamed operand; its buffer resource is built inside run() (a
  // resource held in this struct loses its wave-uniformity and every load
  // turns into a waterfall loop).
  const uint16_t* src;
  int nbytes, off0, rstep;
  f32x4_t acc[8][4];
  bf16x8_t fa[8], fb[4];

  __device__ __forceinline__ void init(int tid) {
    lane = tid & 63;
    // wave-uniform (scalar) wave index: the operand pointer chosen from it
    // must live in SGPRs for the buffer resource
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    grp = wave >> 2;
    q = wave & 3;
    wm = q & 1;
    wn = q >> 1;
    opnd = grp ? 0 : 1;
    lr = lane / CPR;
    frow = lane & 15;  // fragment row of this lane
    fch = lane >> 4;   // its 8-element K chunk
    // Fragment blocks of 16 rows: weights (A) -- linear: rows wn*128 +
    // a*16; P5: gate rows wn*64 + a*16 (a < 4) and the matching up rows
    // 128 + wn*64 + (a-4)*16 -- and x (B): rows wm*128 + grp*64 + b*16.
#pragma unroll
    for (int a = 0; a < 8; ++a)
      arow[a] = NB == 1 ? wn * 128 + a * 16 : (a >> 2) * 128 + wn * 64 + (a & 3) * 16;
#pragma unroll
    for (int b = 0; b < 4; ++b) brow[b] = wm * 128 + grp * 64 + b * 16;
  }

  // The operand this wave streams for the tile at (m0, n0): group 1 the
  // weight tile (for P5 waves 0-1 of the group the gate rows, 2-3 the up
  // rows), group 0 the x tile, 64 rows per wave.  Rows past M / N read as
  // zero.  Lane l writes LDS slot l % CPR of row l / CPR of each 1 KB
  // group, so it fetches the chunk the swizzle places there (the swizzle of
  // tile row q*64 + j*RPI + lr depends only on lr).
  __device__ __forceinline__ void bind(const GemmArgs& g, int m0, int n0) {
    // x rows of this wave's fragments: m0 + wm*128 + grp*64 + b*16 + [0, 16);
    // the tile owns rows [m0, mlim)
    const int64_t mlim = std::min<int64_t>(g.M, (int64_t)m0 + g.bm);
    const int64_t rows_left = mlim - m0 - (wm * 128 + grp * 64);
    nbv = rows_left <= 0 ? 0 : rows_left >= 64 ? 4 : (int)((rows_left + 15) / 16);
    const bool up = NB == 2 && grp && q >= 2;
    src = grp ? (up ? g.w1 : g.w0) : g.x;
    const int64_t ld = grp ? (up ? g.ldw1 : g.ldw0) : g.ldx;
    const int64_t nrows = grp ? g.N : mlim;  // x rows past the tile read as zero
    const int row0 = grp ? (NB == 1 ? n0 + q * 64 : n0 + (q & 1) * 64) : m0 + q * 64;
    nbytes = (int)(nrows * ld * 2);
    off0 = (int)((int64_t)(row0 + lr) * ld * 2);
    rstep = (int)(RPI * ld * 2);
  }

  __device__ __forceinline__ void issue(LdsRing& lds, __amdgpu_buffer_rsrc_t rs, int stage,
                                        int k0) {
    lds_char* d = (lds_char*)&lds[stage][opnd][q * 64 * CPR];
#pragma unroll
    for (int j = 0; j < LB; ++j) {
      const int co = ((lane % CPR) ^ Geo::swz(j * RPI + lr)) * 16 + k0 * 2;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)(d + j * 1024), 16,
                                               off0 + j * rstep + co, 0, 0, 0);
    }
  }

  // Fragments and MFMAs of the first NBV x fragments only: x rows past M
  // would multiply range-checked zeros (the last row tile of M = 3100 has 28
  // live rows of 256), and at the board's power limit skipped work is clock
  // for the rest.
  template <int NBV>
  __device__ __forceinline__ void frags(LdsRing& lds, int stage) {
    if constexpr (NBV > 0) {
#pragma unroll
      for (int a = 0; a < 8; ++a)
        fa[a] = __builtin_bit_cast(bf16x8_t, lds[stage][0][Geo::slot(arow[a] + frow, fch)]);
    }
#pragma unroll
    for (int b = 0; b < NBV; ++b)
      fb[b] = __builtin_bit_cast(bf16x8_t, lds[stage][1][Geo::slot(brow[b] + frow, fch)]);
  }

  template <int NBV>
  __device__ __forceinline__ void compute() {
#pragma unroll
    for (int a = 0; a < 8; ++a)
#pragma unroll
      for (int b = 0; b < NBV; ++b)
        acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[a], fb[b], acc[a][b], 0, 0, 0);
  }

  // The K loop of one group for NBV live x fragments (see run()).  Every
  // NBV passes the same barriers: the phases differ only in the MFMAs and
  // fragment reads they contain.
  template <int NBV>
  __device__ __forceinline__ void loop(LdsRing& lds, __amdgpu_buffer_rsrc_t rs, int k0, int n) {
    if (grp == 0) frags<NBV>(lds, 0);
    stage_barrier<(D - 1) * LB>();
    if (grp == 0) {
      for (int j = 0; j < n; ++j) {
        compute<NBV>();
        __builtin_amdgcn_sched_barrier(0);
        stage_barrier<(D - 2) * LB>();
        __builtin_amdgcn_sched_barrier(0);
        frags<NBV>(lds, (j + 1) % S);
        issue(lds, rs, (j + D) % S, (k0 + j + D) * kBK);
        __builtin_amdgcn_sched_barrier(0);
        stage_barrier<(D - 1) * LB>();
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
      for (int j = 0; j < n; ++j) {
        frags<NBV>(lds, j % S);
        issue(lds, rs, (j + D) % S, (k0 + j + D) * kBK);
        __builtin_amdgcn_sched_barrier(0);
        stage_barrier<(D - 1) * LB>();
        __builtin_amdgcn_sched_barrier(0);
        compute<NBV>();
        __builtin_amdgcn_sched_barrier(0);
        stage_barrier<(D - 1) * LB>();
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }

  // acc = the tile's products over K steps [k0, k1) (k1 > k0).  Prologue: D
  // steps in flight, step k0 landed, group 0 holds its first fragments.  The
  // loop stays branch-free: the last D steps still refill stages that are
  // never read again, from offsets past k1 (in-range data or range-checked
  // zeros), and group 0 reads fragments one step past k1 that it never uses.
  // Returns with every load of every wave landed and every LDS read done:
  // the last steps' refills land asynchronously, and each wave's
  // s_waitcnt covers only its own, so a barrier follows before anyone
  // writes the ring (staged output, the arrival word, the next prologue).
  template <bool SKIP_DEAD_ROWS = true>
  __device__ __forceinline__ void run(LdsRing& lds, int k0, int k1) {
#pragma unroll
    for (int a = 0; a < 8; ++a)
#pragma unroll
      for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[a][b][r] = 0.f;
    const int n = k1 - k0;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void*)src, (short)0, nbytes, 0x00020000);
#pragma unroll
    for (int s = 0; s < D; ++s) issue(lds, rs, s, (k0 + s) * kBK);
    stage_barrier<(D - 1) * LB>();
    // One straight loop per group (the hardware barrier counts arrivals,
    // not program points; both loops pass the same barriers), so the
    // fragments stay loop-carried in place.  sched_barrier keeps every MFMA
    // in its phase.  The loop is instantiated per count of live x fragments
    // (wave-uniform, fixed for the tile): 4 everywhere but the last row tile.
    // (The stream-K kernel keeps one full loop: the extra instantiations'
    // register state would spill there.)
    if constexpr (SKIP_DEAD_ROWS) {
      switch (nbv) {
        case 4: loop<4>(lds, rs, k0, n); break;
        case 3: loop<3>(lds, rs, k0, n); break;
        case 2: loop<2>(lds, rs, k0, n); break;
        case 1: loop<1>(lds, rs, k0, n); break;
        default: loop<0>(lds, rs, k0, n); break;
      }
    } else {
      loop<4>(lds, rs, k0, n);
    }
    stage_barrier<0>();
  }

  // Epilogue.  acc[a][b][e]: x row brow[b] + lane % 16, weight row
  // arow[a] + 4 * (lane / 16) + e.  The output tile is staged in LDS (the
  // ring is idle once run() has returned) as row-major bf16 rows padded by
  // 16 bytes, then streamed to HBM as whole rows with 16-byte stores: stored
  // straight from the fragment layout, each store instruction would touch
  // 16 rows (16 partial cache lines), which measured ~7 us per tile against
  // ~1 us this way.
  static constexpr int kOutCols = NB == 1 ? kBW : kBW / 2;  // output columns per tile
  static constexpr int kOutRow = kOutCols * 2 + 16;         // staged bytes per row
  static_assert(kBM * kOutRow <= (int)sizeof(LdsRing), "staged tile must fit the ring");

  __device__ __forceinline__ int out_col(int a) const {
    return (NB == 1 ? arow[a] : wn * 64 + a * 16) + fch * 4;
  }

  // Bias of this lane's 4 output columns of column block a: 4 consecutive
  // bf16, 8-byte aligned (bias and N are multiples of 4 elements); columns
  // past N are never written out.
  template <bool BIAS>
  __device__ __forceinline__ f32x4_t load_bias(const GemmArgs& g, int n0, int a) const {
    f32x4_t bias = {0.f, 0.f, 0.f, 0.f};
    if constexpr (NB == 1 && BIAS) {
      if (n0 + out_col(a) < g.N) {
        const uint2 bw = *reinterpret_cast<const uint2*>(g.bias + n0 + out_col(a));
        bias[0] = bf_lo(bw.x);
        bias[1] = bf_hi(bw.x);
        bias[2] = bf_lo(bw.y);
        bias[3] = bf_hi(bw.y);
      }
    }
    return bias;
  }

  // Block (a, b) of the tile from fp32 v (P5: gate v, up u): bias, GELU or
  // silu(g)*u, one bf16 rounding, into the staged tile.
  template <int ACT, bool BIAS>
  __device__ __forceinline__ void stage_block(LdsRing& lds, int a, int b, f32x4_t v, f32x4_t u,
                                              f32x4_t bias) {
    const int row = brow[b] + frow;
    const int col = out_col(a);
    float o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float x = v[e];
      if constexpr (NB == 2) {
        // silu(g) * u with the hardware exp2 / reciprocal (~1 ulp each, far
        // inside the bf16 output rounding); large |g| saturates correctly:
        // exp -> inf gives rcp -> 0, exp -> 0 gives rcp -> 1.
        const float den = 1.0f + __builtin_amdgcn_exp2f(x * -1.4426950408889634f);
        x = x * __builtin_amdgcn_rcpf(den) * u[e];
      } else {
        if constexpr (BIAS) x = x + bias[e];
        if constexpr (ACT == UMIC_ACT_GELU) x = gelu_erf(x);
        if constexpr (ACT == UMIC_ACT_GELU_TANH) x = gelu_tanh(x);
      }
      o[e] = x;
    }
    uint2 pk;
    pk.x = pack2(o[0], o[1]);
    pk.y = pack2(o[2], o[3]);
    *reinterpret_cast<uint2*>(reinterpret_cast<char*>(&lds[0][0][0]) + row * kOutRow + col * 2) = pk;
  }

  // Stream the staged tile to out[m0.., n0..]: each thread moves 16-byte
  // chunks, a wavefront whole contiguous rows.  Barriers on both sides: the
  // tile must be complete, and the ring may be refilled afterwards.
  __device__ __forceinline__ void flush(LdsRing& lds, const GemmArgs& g, int m0, int n0) {
    __syncthreads();
    constexpr int kChunks = kOutCols / 8;  // 16-byte chunks per row
    constexpr int kRowsPerPass = kThreads / kChunks;
    const int c = threadIdx.x % kChunks;
    const int64_t n = n0 + c * 8;
    const char* base = reinterpret_cast<const char*>(&lds[0][0][0]);
    // staged rows past the tile's own (the next tile's rows) are never stored
    const int64_t mlim = std::min<int64_t>(g.M, (int64_t)m0 + g.bm);
    if (n < g.N) {
#pragma unroll 4
      for (int r = threadIdx.x / kChunks; r < kBM; r += kRowsPerPass) {
        const int64_t m = (int64_t)m0 + r;
        if (m >= mlim) break;
        // Plain (cached) stores: the next op reads this output (P5's h feeds
        // down_proj), and it can still be served from the Infinity Cache.
        // Non-temporal stores measured up to 2% faster for an isolated
        // kernel but made the config-5 layer prefill 1.3% slower.
        *reinterpret_cast<u32x4*>(g.out + m * g.ldo + n) =
            *reinterpret_cast<const u32x4*>(base + r * kOutRow + c * 16);
      }
    }
    __syncthreads();
  }

  template <int ACT, bool BIAS>
  __device__ __forceinline__ void store(LdsRing& lds, const GemmArgs& g, int m0, int n0) {
    constexpr int kOutBlocks = NB == 1 ? 8 : 4;
#pragma unroll
    for (int a = 0; a < kOutBlocks; ++a) {
      const f32x4_t bias = load_bias<BIAS>(g, n0, a);
#pragma unroll
      for (int b = 0; b < 4; ++b)
        stage_block<ACT, BIAS>(lds, a, b, acc[a][b], acc[NB == 2 ? a + 4 : a][b], bias);
    }
    flush(lds, g, m0, n0);
  }
};

// Data-parallel: one workgroup per tile, the whole K loop.
template <int NB, int ACT, bool BIAS>
__global__ __launch_bounds__(kThreads, 1) void gemm_kernel(GemmArgs g) {
  __shared__ LdsRing lds;
  const int t = xcd_remap(g.tiles);
  if (t >= g.tiles) return;
  int m0, n0;
  tile_origin(g, t, NB == 1 ? kBW : kBW / 2, m0, n0);
  Pipe<NB> p;
  p.init(threadIdx.x);
  p.bind(g, m0, n0);
  p.run(lds, 0, (int)(g.K / kBK));
  p.template store<ACT, BIAS>(lds, g, m0, n0);
}

// ---- Four-wave core (K a multiple of 64) ---------------------------------
//
// The data-parallel kernel for K % 64 == 0.  Same tile (256 x rows by 256
// weight rows), tile order, operand layout and arithmetic as gemm_kernel --
// every output is bit-identical to it -- with a different division of the
// tile and K loop:
//
// Waves.  Four wavefronts, one per SIMD.  Wave w owns a 128 x 128 block
// (x rows from wm * 128, weight rows from wn * 128; for P5 64 gate rows and
// the same 64 up rows), 8 x 8 blocks of v_mfma_f32_16x16x32_bf16 with its
// 256 fp32 accumulators in AGPRs.  Per 32 of K a wave reads 16 fragments
// for 64 MFMAs (gemm_kernel's waves read 12 for 32): a third fewer LDS
// reads per MFMA.
//
// MFMAs as inline asm.  Each MFMA is issued with its accumulator as a tied
// "+a" operand, so the accumulator stays in one AGPR for the whole tile.
// Left to the compiler, 256 live accumulators in a 256-entry AGPR file were
// renamed and copied (v_accvgpr_read/write/mov) between MFMAs -- 236 copies
// per 128 MFMAs.  The compiler's hazard tracking does not see into asm, so
// the kernel supplies the two wait states it needs itself: the tile's first
// MFMAs take srcC = 0 (no accumulator initialisation to wait for), and the
// reads of the results come after 32 wait states in asm statements that take
// every accumulator as an operand (nothing can be moved above them).
//
// Stages of K = 64.  A staged row is 128 bytes, a whole cache line, and one
// direct-to-LDS wave load moves 8 rows of it: the requests are whole lines
// (gemm_kernel's 32-deep stages move half lines).  Two stages of 64 KB
// fill 128 KB of LDS.  Stage j's first half (32 of K) runs its 64 MFMAs
// while the wave reads its fragments of the second half; then each wave
// waits for its own loads of stage j+1 and the block meets at a barrier
// (everyone's loads have landed, everyone's reads of stage j are done);
// the second half runs its MFMAs while the wave loads stage j+2 into stage
// j's buffer and reads its fragments of stage j+1.  One barrier per 64 of
// K; loads are issued one stage (128 MFMAs per wave) ahead.  Rows are
// XOR-swizzled by (row >> 1) & 7 (16-byte chunks within the 128-byte row):
// measured 2-3% bank-conflict cycles against 37-43% unswizzled.
//
// Dead fragments.  A wave whose x rows lie (partly) past the tile's live
// rows runs the K loop instantiated for its count of live fragments
// (0..8), so the last row tile of M = 3100 and the even 240-row tiles of a
// multi-round launch multiply no zero rows; every instantiation issues the
// same loads and meets the same barriers.
constexpr int kW4Threads = 256;
constexpr int kW4BK = 64;                        // K per stage
constexpr int kW4Row = kW4BK * 2;                // staged bytes per row
constexpr int kW4OpBytes = kBW * kW4Row;         // one operand of a stage (32 KB)
constexpr int kW4StageBytes = 2 * kW4OpBytes;    // 64 KB
constexpr int kW4LdsBytes = 160 * 1024;          // two stages; the staged output needs 135 KB

__device__ __forceinline__ int w4_swz(int row) { return (row >> 1) & 7; }

// s_waitcnt vmcnt(VM) lgkmcnt(LGKM) through the builtin, so the compiler's
// own waitcnt pass sees the counters it clears (an asm s_waitcnt left it
// assuming LDS reads were still in flight, and it added waits of its own
// before the next MFMAs); the empty asm statements keep memory accesses
// from moving across.
template <int VM, int LGKM>
__device__ __forceinline__ void w4_wait() {
  static_assert(VM >= 0 && VM < 64 && LGKM >= 0 && LGKM < 16, "waitcnt fields");
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt((VM & 15) | (7 << 4) | (LGKM << 8) | ((VM >> 4) << 14));
  asm volatile("" ::: "memory");
}

__device__ __forceinline__ void w4_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Where one tile's operand rows come from: the buffer resources (x rows past
// the tile's own, and rows past N, read as zero) and a lane's byte offsets
// (row, swizzled chunk) for its even and odd loads.
struct W4Src {
  __amdgpu_buffer_rsrc_t rx, rw;
  int xoff0, xoff1, woff0, woff1;
};

template <int NB>
struct W4Tile {
  lds_char* lds;
  int wave, wm, wn, frow, fch;
  int fo0, fo1;      // a lane's fragment offset inside a 16-row block, K halves 0 / 1
  int xbase;         // first x row of this wave's fragments
  W4Src src;         // the tile being loaded
  int xstep, wstep;  // bytes between 8-row load groups (wave-uniform)
  int kbase;         // first K element of the segment the K loop runs
  f32x4_t acc[8][8];
  bf16x8_t fa[2][8], fb[2][8];

  // Lane-invariant set-up (everything but the tile).
  __device__ __forceinline__ void init(void* smem, const GemmArgs& g) {
    lds = (lds_char*)smem;
    const int lane = threadIdx.x & 63;
    wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    wm = wave & 1;
    wn = wave >> 1;
    frow = lane & 15;
    fch = lane >> 4;
    // a fragment's 16 rows start at a multiple of 16: the swizzle of its
    // rows depends on the lane only
    fo0 = frow * kW4Row + ((fch ^ w4_swz(frow)) * 16);
    fo1 = frow * kW4Row + (((4 + fch) ^ w4_swz(frow)) * 16);
    xbase = wm * 128;  // wave pair wm takes x rows [wm * 128, ...) of the tile
    kbase = 0;
    const bool up = NB == 2 && wave >= 2;
    xstep = __builtin_amdgcn_readfirstlane((int)(8 * g.ldx * 2));
    wstep = __builtin_amdgcn_readfirstlane((int)(8 * (up ? g.ldw1 : g.ldw0) * 2));
  }

  // The load addressing of the tile at (m0, n0) owning x rows [m0, mlim).
  __device__ __forceinline__ W4Src bind(const GemmArgs& g, int m0, int n0, int64_t mlim) const {
    const int lane = threadIdx.x & 63;
    const bool up = NB == 2 && wave >= 2;
    const uint16_t* wsrc = up ? g.w1 : g.w0;
    const int64_t ldw = up ? g.ldw1 : g.ldw0;
    const int wrow0 = NB == 1 ? n0 + wave * 64 : n0 + (wave & 1) * 64;
    W4Src r;
    r.rx = __builtin_amdgcn_make_buffer_rsrc((void*)g.x, (short)0, (int)(mlim * g.ldx * 2),
                                             0x00020000);
    r.rw = __builtin_amdgcn_make_buffer_rsrc((void*)wsrc, (short)0, (int)(g.N * ldw * 2),
                                             0x00020000);
    // staged row wave*64 + q*8 + lr: its swizzle depends on lr and q's parity
    const int lr = lane >> 3, lc = lane & 7;
    const int c0 = (lc ^ w4_swz(lr)) * 16, c1 = (lc ^ w4_swz(8 + lr)) * 16;
    const int xoff = (int)((int64_t)(m0 + wave * 64 + lr) * g.ldx * 2);
    const int woff = (int)((int64_t)(wrow0 + lr) * ldw * 2);
    r.xoff0 = xoff + c0;
    r.xoff1 = xoff + c1;
    r.woff0 = woff + c0;
    r.woff1 = woff + c1;
    return r;
  }

  // Weight row of fragment block a: linear wn*128 + a*16; P5 gate rows
  // wn*64 + a*16 (a < 4) and the matching up rows 128 + wn*64 + (a-4)*16.
  __device__ __forceinline__ int arow(int a) const {
    return NB == 1 ? wn * 128 + a * 16 : (a >> 2) * 128 + wn * 64 + (a & 3) * 16;
  }

  // Load q (0..15) of a stage: 0..7 the weight rows wave*64 + q*8 .. + 8,
  // 8..15 the x rows wave*64 + (q-8)*8 .. + 8 (rows past the tile's own, or
  // past M / N, read as range-checked zeros).  Lane l writes LDS slot l % 8
  // of row l / 8, so it fetches the 16-byte chunk the swizzle puts there.
  __device__ __forceinline__ void issue(const W4Src& r, int stage, int k, int q) {
    lds_char* d = lds + stage * kW4StageBytes + (q >> 3) * kW4OpBytes +
                  (wave * 64 + (q & 7) * 8) * kW4Row;
    if (q < 8)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r.rw, (lds_void*)d, 16, (q & 1) ? r.woff1 : r.woff0,
                                               k * 2 + (q & 7) * wstep, 0, 0);
    else
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r.rx, (lds_void*)d, 16, (q & 1) ? r.xoff1 : r.xoff0,
                                               k * 2 + (q & 7) * xstep, 0, 0);
  }
  __device__ __forceinline__ void issue(int stage, int k, int q) {
    issue(src, stage, kbase + k, q);
  }

  // Fragment f (0..7: weight blocks, 8..15: x blocks) of K half h of a stage.
  __device__ __forceinline__ void read(int buf, int stage, int h, int f) {
    const lds_char* base = lds + stage * kW4StageBytes + (h ? fo1 : fo0);
    if (f < 8)
      fa[buf][f] = *(const bf16x8_t*)(base + arow(f) * kW4Row);
    else
      fb[buf][f - 8] = *(const bf16x8_t*)(base + kW4OpBytes + (xbase + (f - 8) * 16) * kW4Row);
  }

  // The 8 x NBX MFMAs of one K half on fragment buffer B; body(i) places
  // memory work after MFMA i.  ZERO: the tile's first half, srcC = 0.
  template <int NBX, int B, bool ZERO, typename Body>
  __device__ __forceinline__ void mfmas(Body body) {
#pragma unroll
    for (int i = 0; i < 64; ++i) {
      const int a = i >> 3, b = i & 7;
      if (b < NBX) {
        if constexpr (ZERO)
          asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, 0"
                       : "=a"(acc[a][b]) : "v"(fa[B][a]), "v"(fb[B][b]));
        else
          asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0"
                       : "+a"(acc[a][b]) : "v"(fa[B][a]), "v"(fb[B][b]));
      }
      body(i);
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // The K loop over n stages (stages 0 and 1 already in flight, stage 0
  // landed block-wide).  Returns with every load landed and every MFMA
  // result readable.
  template <int NBX>
  __device__ __forceinline__ void kloop(int n) {
    constexpr bool kAny = NBX > 0;
    auto wanted = [](int f) { return kAny && (f < 8 || f - 8 < NBX); };
#pragma unroll
    for (int f = 0; f < 16; ++f)
      if (wanted(f)) read(0, 0, 0, f);
    w4_wait<63, 0>();
    // Stage j; stage 0 (ZERO) is peeled off the loop, so every accumulator
    // has one definition reaching the loop and keeps its register.
    auto stage = [&](int j, auto zero) {
      const int sj = j & 1, sn = sj ^ 1;
      mfmas<NBX, 0, decltype(zero)::value>([&](int i) {
        if (i >= 1 && i < 17 && wanted(i - 1)) read(1, sj, 1, i - 1);
      });
      w4_wait<0, 0>();
      w4_barrier();
      // Past the last stage the refills read in-range data or range-checked
      // zeros, and the reads take fragments that are never used.
      mfmas<NBX, 1, false>([&](int i) {
        if (i % 4 == 1) issue(sj, (j + 2) * kW4BK, i / 4);
        if (i >= 2 && i < 18 && wanted(i - 2)) read(0, sn, 0, i - 2);
      });
      w4_wait<63, 0>();
    };
    stage(0, std::true_type{});
    for (int j = 1; j < n; ++j) stage(j, std::false_type{});
    w4_wait<0, 0>();
    w4_barrier();
    fence_results<NBX>();
  }

  // The MFMA results are read next: 32 wait states, then a statement per
  // live accumulator (blocks b < NBX; the others are never written or read)
  // that takes it, so no read moves above the wait states -- and no value
  // of an accumulator the K loop did not write is kept alive (a loop over
  // tiles of different NBX would otherwise carry them all across its
  // iterations).
  template <int NBX>
  __device__ __forceinline__ void fence_results() {
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
#pragma unroll
    for (int a = 0; a < 8; ++a)
#pragma unroll
      for (int b = 0; b < NBX; ++b) asm volatile("" : "+a"(acc[a][b]));
  }

  static constexpr int kOutCols = NB == 1 ? kBW : kBW / 2;
  static constexpr int kOutRow = kOutCols * 2 + 16;  // staged bytes per output row
  static_assert(kBM * kOutRow <= kW4LdsBytes, "staged tile must fit the LDS");

  // The linear's bias chunk of fragment block a (4 output columns of this lane).
  template <bool BIAS>
  __device__ __forceinline__ f32x4_t bias_of(const GemmArgs& g, int n0, int a) const {
    f32x4_t bias = {0.f, 0.f, 0.f, 0.f};
    if constexpr (NB == 1 && BIAS) {
      const int col = arow(a) + fch * 4;
      if (n0 + col < g.N) {
        const uint2 bw = *reinterpret_cast<const uint2*>(g.bias + n0 + col);
        bias[0] = bf_lo(bw.x);
        bias[1] = bf_hi(bw.x);
        bias[2] = bf_lo(bw.y);
        bias[3] = bf_hi(bw.y);
      }
    }
    return bias;
  }

  // Stage block (a, b) of the output tile, v its fp32 sums (P5: the gate
  // sums, u the up sums), as bf16 in LDS: bias, GELU or silu(g) * u in fp32,
  // one rounding, as gemm_kernel's epilogue.
  template <int ACT, bool BIAS>
  __device__ __forceinline__ void stage_block(int a, int b, const f32x4_t& v, const f32x4_t& u,
                                              const f32x4_t& bias) {
    char* out = (char*)lds;
    const int col = (NB == 1 ? arow(a) : wn * 64 + a * 16) + fch * 4;
    float o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float x = v[e];
      if constexpr (NB == 2) {
        const float den = 1.0f + __builtin_amdgcn_exp2f(x * -1.4426950408889634f);
        x = x * __builtin_amdgcn_rcpf(den) * u[e];
      } else {
        if constexpr (BIAS) x = x + bias[e];
        if constexpr (ACT == UMIC_ACT_GELU) x = gelu_erf(x);
        if constexpr (ACT == UMIC_ACT_GELU_TANH) x = gelu_tanh(x);
      }
      o[e] = x;
    }
    uint2 pk;
    pk.x = pack2(o[0], o[1]);
    pk.y = pack2(o[2], o[3]);
    *reinterpret_cast<uint2*>(out + (xbase + b * 16 + frow) * kOutRow + col * 2) = pk;
  }

  // Stage the tile's live fragments as bf16 rows in LDS.
  template <int NBX, int ACT, bool BIAS>
  __device__ __forceinline__ void stage_out(const GemmArgs& g, int n0) {
    constexpr int kOutBlocks = NB == 1 ? 8 : 4;
#pragma unroll
    for (int a = 0; a < kOutBlocks; ++a) {
      const f32x4_t bias = bias_of<BIAS>(g, n0, a);
#pragma unroll
      for (int b = 0; b < NBX; ++b) {
        stage_block<ACT, BIAS>(a, b, acc[a][b], acc[NB == 2 ? a + 4 : a][b], bias);
        __builtin_amdgcn_sched_barrier(0);  // one block's reads at a time
      }
    }
  }

  // Stream-K partials (linear only).  A lane's share of a partial is its
  // wave's 64 KB region, [a][b][lane] (block (a, b) at (a * 8 + b) * 64
  // f32x4 from the lane's base, so four consecutive blocks are reached with
  // immediate offsets of one address), written and read with device-scope
  // (sc1) accesses.  Called after fence_results().  A store of more than 8
  // bytes reads its data registers after issue, and the compiler's hazard
  // checks do not see into the asm: the s_nop keeps the next instruction
  // (typically the copy of the next block into the same registers) from
  // overwriting them first.
  template <int NBX>
  __device__ __forceinline__ void store_partial(f32x4_t* p) {
#pragma unroll
    for (int a = 0; a < 8; ++a)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        f32x4_t* const q = p + (a * 8 + h * 4) * 64;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (h * 4 + i < NBX)
            asm volatile("global_store_dwordx4 %0, %1, off offset:%2 sc1\n\ts_nop 1"
                         ::"v"(q), "v"(acc[a][h * 4 + i]), "n"(i * 1024) : "memory");
      }
  }

  // Stage the tile with its tail partials added: acc (K steps [0, ks)) +
  // the lower tail piece p1 (+ the higher one, p2, when `two`), summed in
  // that order.
  template <int NBX, int ACT, bool BIAS>
  __device__ __forceinline__ void stage_out_sum(const GemmArgs& g, int n0, const f32x4_t* p1,
                                                const f32x4_t* p2, bool two) {
    static_assert(NB == 1, "stream-K runs the linear");
    if (!two) {
#pragma unroll
      for (int a = 0; a < 8; a += 2) {
        f32x4_t q[16];
        w4_load16(q, p1 + a * 512, p1 + (a + 1) * 512);
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          const f32x4_t bias = bias_of<BIAS>(g, n0, a + r);
#pragma unroll
          for (int b = 0; b < NBX; ++b) {
            stage_block<ACT, BIAS>(a + r, b, acc[a + r][b] + q[r * 8 + b], q[0], bias);
            __builtin_amdgcn_sched_barrier(0);
          }
        }
      }
    } else {
#pragma unroll
      for (int a = 0; a < 8; ++a) {
        f32x4_t q[16];
        w4_load16(q, p1 + a * 512, p2 + a * 512);
        const f32x4_t bias = bias_of<BIAS>(g, n0, a);
#pragma unroll
        for (int b = 0; b < NBX; ++b) {
          stage_block<ACT, BIAS>(a, b, (acc[a][b] + q[b]) + q[8 + b], q[0], bias);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
  }

  // Two partial rows (8 blocks each, at u and v), device-scope loads issued
  // and waited for inside ONE asm statement: the outputs are valid when it
  // returns (a load left in flight across statements is unsafe: the
  // compiler may move or spill its destination before the data arrives).
  static __device__ __forceinline__ void w4_load16(f32x4_t (&q)[16], const f32x4_t* u,
                                                   const f32x4_t* v) {
    asm volatile(
        "global_load_dwordx4 %0, %16, off sc1\n\t"
        "global_load_dwordx4 %1, %16, off offset:1024 sc1\n\t"
        "global_load_dwordx4 %2, %16, off offset:2048 sc1\n\t"
        "global_load_dwordx4 %3, %16, off offset:3072 sc1\n\t"
        "global_load_dwordx4 %4, %17, off sc1\n\t"
        "global_load_dwordx4 %5, %17, off offset:1024 sc1\n\t"
        "global_load_dwordx4 %6, %17, off offset:2048 sc1\n\t"
        "global_load_dwordx4 %7, %17, off offset:3072 sc1\n\t"
        "global_load_dwordx4 %8, %18, off sc1\n\t"
        "global_load_dwordx4 %9, %18, off offset:1024 sc1\n\t"
        "global_load_dwordx4 %10, %18, off offset:2048 sc1\n\t"
        "global_load_dwordx4 %11, %18, off offset:3072 sc1\n\t"
        "global_load_dwordx4 %12, %19, off sc1\n\t"
        "global_load_dwordx4 %13, %19, off offset:1024 sc1\n\t"
        "global_load_dwordx4 %14, %19, off offset:2048 sc1\n\t"
        "global_load_dwordx4 %15, %19, off offset:3072 sc1\n\t"
        "s_waitcnt vmcnt(0)"
        : "=&v"(q[0]), "=&v"(q[1]), "=&v"(q[2]), "=&v"(q[3]), "=&v"(q[4]), "=&v"(q[5]),
          "=&v"(q[6]), "=&v"(q[7]), "=&v"(q[8]), "=&v"(q[9]), "=&v"(q[10]), "=&v"(q[11]),
          "=&v"(q[12]), "=&v"(q[13]), "=&v"(q[14]), "=&v"(q[15])
        : "v"(u), "v"(u + 256), "v"(v), "v"(v + 256)
        : "memory");
  }
};

// Stream the tile staged in LDS out as whole rows of 16-byte stores (rows
// [m0, mlim) of the output).
template <int NB>
__device__ __forceinline__ void w4_flush(const char* smem, const GemmArgs& g, int m0, int n0,
                                         int64_t mlim) {
  constexpr int kOutCols = W4Tile<NB>::kOutCols;
  constexpr int kOutRow = W4Tile<NB>::kOutRow;
  constexpr int kChunks = kOutCols / 8;
  constexpr int kRowsPerPass = kW4Threads / kChunks;
  const int cc = threadIdx.x % kChunks;
  const int64_t col = n0 + cc * 8;
  if (col < g.N) {
#pragma unroll 4
    for (int r = threadIdx.x / kChunks; r < kBM; r += kRowsPerPass) {
      const int64_t m = (int64_t)m0 + r;
      if (m >= mlim) break;
      *reinterpret_cast<u32x4*>(g.out + m * g.ldo + col) =
          *reinterpret_cast<const u32x4*>(smem + r * kOutRow + cc * 16);
    }
  }
}

template <int NB, int NBX, int ACT, bool BIAS>
__device__ __forceinline__ void w4_tile(W4Tile<NB>& c, const GemmArgs& g, int n, int n0) {
  c.template kloop<NBX>(n);
  c.template stage_out<NBX, ACT, BIAS>(g, n0);
}

template <int NB, int ACT, bool BIAS>
__global__ __launch_bounds__(kW4Threads, 1) void gemm_w4_kernel(GemmArgs g) {
  __shared__ __attribute__((aligned(16))) char smem[kW4LdsBytes];
  const int t = xcd_remap(g.tiles);
  if (t >= g.tiles) return;
  int m0, n0;
  tile_origin(g, t, NB == 1 ? kBW : kBW / 2, m0, n0);

  W4Tile<NB> c;
  c.init(smem, g);
  // the tile owns x rows [m0, mlim)
  const int64_t mlim = std::min<int64_t>(g.M, (int64_t)m0 + g.bm);
  c.src = c.bind(g, m0, n0, mlim);
  const int live = (int)(mlim - m0) - c.xbase;
  const int nbx = __builtin_amdgcn_readfirstlane(live <= 0 ? 0 : min(8, (live + 15) / 16));
  const int n = (int)(g.K / kW4BK);
#pragma unroll
  for (int q = 0; q < 16; ++q) c.issue(0, 0, q);
#pragma unroll
  for (int q = 0; q < 16; ++q) c.issue(1, kW4BK, q);
  w4_wait<16, 0>();  // this wave's loads of stage 0
  w4_barrier();      // everyone's
  switch (nbx) {
    case 8: w4_tile<NB, 8, ACT, BIAS>(c, g, n, n0); break;
    case 7: w4_tile<NB, 7, ACT, BIAS>(c, g, n, n0); break;
    case 6: w4_tile<NB, 6, ACT, BIAS>(c, g, n, n0); break;
    case 5: w4_tile<NB, 5, ACT, BIAS>(c, g, n, n0); break;
    case 4: w4_tile<NB, 4, ACT, BIAS>(c, g, n, n0); break;
    case 3: w4_tile<NB, 3, ACT, BIAS>(c, g, n, n0); break;
    case 2: w4_tile<NB, 2, ACT, BIAS>(c, g, n, n0); break;
    case 1: w4_tile<NB, 1, ACT, BIAS>(c, g, n, n0); break;
    default: w4_tile<NB, 0, ACT, BIAS>(c, g, n, n0); break;
  }
  __syncthreads();
  w4_flush<NB>(smem, g, m0, n0, mlim);
}

// Stream-K linear, K-aligned.  With T tiles < G workgroups (one per CU),
// every workgroup gets the same number of K steps, ks = floor(T*KT / G):
// T "main" workgroups run K steps [0, ks) of one tile each -- in lockstep,
// so concurrent tiles share x and weight slabs in L2 exactly as in the
// data-parallel kernel -- and the other G - T "tail" workgroups split the
// remaining T x (KT - ks) steps (the [ks, KT) range of every tile, in tile
// order) evenly between them, stream-K style.  A tile whose K range one
// workgroup covers is stored directly.  A split tile's segments (the main
// one, then its tail pieces in K order) are reduced by whichever workgroup
// arrives last: the others store their fp32 partial in the tile's slot for
// their arrival order (the first arriver slot 0, the second slot 1; the last
// stores none, so a tile of kSkMaxSeg segments needs kSkSlots slots), tag
// the slot with their segment index and count themselves "written"; the
// last waits for that count -- every workgroup it waits for has already
// arrived, so it is running and finishes its store without waiting on
// anything -- then, through the tags, sums the segments in segment order
// (deterministic whatever the arrival order), applies the epilogue and
// resets the tile's two counters, so the workspace is all-zero counters
// again after every launch.
struct SkArgs {
  int* counters;   // [2 * T]: arrived, written (zero between launches)
  int* status;     // sticky status word (0: every wait completed)
  int* tags;       // [T][kSkSlots]: the segment whose partial a slot holds
  f32x4_t* slots;  // [T][kSkSlots][kSlotVec]: partials, by arrival order
  int T, KT, ks;   // tiles, K steps per tile, main steps per tile
  int G;           // workgroups (T main + G - T tail)
};
constexpr int kSlotVec = kBM * kBW / 4;  // f32x4 per partial tile (256 KB)
constexpr int kSkMaxSeg = 3;             // segments per tile (checked on the host)
constexpr int kSkSlots = kSkMaxSeg - 1;  // stored partials per tile
// Workspace layout: the tile counters in a region of fixed size, then the
// partial slots.  One workspace serves calls of any shape in turn, so no
// call's slots may overlap another call's counters: with the counter region
// sized by the call's own tile count, a call with few tiles stored partials
// where a later call with more tiles kept (and trusted) zero counters.
// The region also holds one sticky status word after the counters, at byte
// kSkStatusOffset: a last arriver whose wait gives up (below) stores 1 + its
// tile index there; nothing else writes it and no launch clears it.  The
// slot tags follow it; a tag is written before its slot is counted and read
// only after, so tags need no clearing.
constexpr int kSkMaxTiles = 1024;        // stream-K needs fewer tiles than CUs
constexpr int64_t kSkStatusOffset = 2 * kSkMaxTiles * (int64_t)sizeof(int);
constexpr int64_t kSkTagOffset = kSkStatusOffset + 256;
constexpr int64_t kSkCounterBytes = kSkTagOffset + kSkSlots * kSkMaxTiles * (int64_t)sizeof(int);
static_assert(kSkStatusOffset == UMIC_SK_STATUS_OFFSET, "status word offset of the C ABI");
static_assert(kSkCounterBytes % 256 == 0, "partial slots stay 256-byte aligned");

// Bound of the last arriver's wait.  The segments it waits for have already
// arrived, so they are resident and finish their 256 KB partial store within
// microseconds; a count that never arrives means a corrupted workspace (or
// calls overlapping on one), and the wait then gives up instead of holding
// the GPU.  Each poll is one device-scope load (an L2 round trip, about
// 0.5-1 us under load) plus s_sleep(2) (2 x 64 clocks); 2^19 polls last at
// least 2^19 x 128 clocks = 28 ms at 2.4 GHz and, with the load latency,
// well under a second (0.7 s even at a 100 MHz clock without it).
constexpr int kSkSpinLimit = 1 << 19;

// Tail units: v = t * L + r is step ks + r of tile t (L = KT - ks); tail
// workgroup j owns [j*Ut/Gt, (j+1)*Ut/Gt), Ut = T*L, Gt = G - T (Ut*Gt < 2^31,
// checked on the host).
struct SkTail {
  int L, Ut, Gt;
  __device__ __forceinline__ explicit SkTail(const SkArgs& s)
      : L(s.KT - s.ks), Ut(s.T * (s.KT - s.ks)), Gt(s.G - s.T) {}
  __device__ __forceinline__ int start(int j) const { return j * Ut / Gt; }
  __device__ __forceinline__ int owner(int v) const { return ((v + 1) * Gt - 1) / Ut; }
};

// Device-scope (sc1) 16-byte loads of one accumulator row's partials,
// p[b * kThreads] for b = 0..3, issued and waited for inside ONE asm
// statement: the outputs are valid when it returns.  (A load left in flight
// across statements is unsafe: the compiler may move or spill its destination
// register before the data arrives.)  Early-clobber outputs keep the
// destinations off the address registers.
__device__ __forceinline__ void load_row_sc1(f32x4_t (&q)[4], const f32x4_t* p) {
  asm volatile(
      "global_load_dwordx4 %0, %4, off sc1\n\t"
      "global_load_dwordx4 %1, %5, off sc1\n\t"
      "global_load_dwordx4 %2, %6, off sc1\n\t"
      "global_load_dwordx4 %3, %7, off sc1\n\t"
      "s_waitcnt vmcnt(0)"
      : "=&v"(q[0]), "=&v"(q[1]), "=&v"(q[2]), "=&v"(q[3])
      : "v"(p), "v"(p + kThreads), "v"(p + 2 * kThreads), "v"(p + 3 * kThreads)
      : "memory");
}

// The same for two segments' rows at once (eight loads, one wait).
__device__ __forceinline__ void load_row_sc1(f32x4_t (&q)[4], f32x4_t (&r)[4],
                                             const f32x4_t* p, const f32x4_t* u) {
  asm volatile(
      "global_load_dwordx4 %0, %8, off sc1\n\t"
      "global_load_dwordx4 %1, %9, off sc1\n\t"
      "global_load_dwordx4 %2, %10, off sc1\n\t"
      "global_load_dwordx4 %3, %11, off sc1\n\t"
      "global_load_dwordx4 %4, %12, off sc1\n\t"
      "global_load_dwordx4 %5, %13, off sc1\n\t"
      "global_load_dwordx4 %6, %14, off sc1\n\t"
      "global_load_dwordx4 %7, %15, off sc1\n\t"
      "s_waitcnt vmcnt(0)"
      : "=&v"(q[0]), "=&v"(q[1]), "=&v"(q[2]), "=&v"(q[3]),
        "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3])
      : "v"(p), "v"(p + kThreads), "v"(p + 2 * kThreads), "v"(p + 3 * kThreads),
        "v"(u), "v"(u + kThreads), "v"(u + 2 * kThreads), "v"(u + 3 * kThreads)
      : "memory");
}

template <int ACT, bool BIAS>
__global__ __launch_bounds__(kThreads, 1) void gemm_sk_kernel(GemmArgs g, SkArgs s) {
  __shared__ LdsRing lds;
  // The arrival order is broadcast through the ring's first word: between
  // segments the ring is idle (run() returns with every read done and every
  // load landed) and the next prologue refills it only after two barriers.
  int* arrival = reinterpret_cast<int*>(&lds[0][0][0]);
  const int w = xcd_remap(s.G);
  if (w >= s.G) return;
  const int tid = threadIdx.x;
  const SkTail tl(s);
  Pipe<1> p;
  // Main workgroup: one segment.  Tail workgroup j: units [v, vend).
  const bool main_wg = w < s.T;
  int v = main_wg ? 0 : tl.start(w - s.T);
  const int vend = main_wg ? 1 : tl.start(w - s.T + 1);
  while (v < vend) {
    int t, k0, k1, seg;
    if (main_wg) {
      t = w;
      k0 = 0;
      k1 = s.ks;
      seg = 0;
      v = vend;
    } else {
      t = v / tl.L;
      const int r = v - t * tl.L;
      const int len = min(tl.L - r, vend - v);
      k0 = s.ks + r;
      k1 = k0 + len;
      seg = 1 + (w - s.T) - tl.owner(t * tl.L);
      v += len;
    }
    int m0, n0;
    tile_origin(g, t, kBW, m0, n0);
    // The per-wave invariants (fragment addresses, ...) are derived from an
    // opaque copy of the thread index, so they are recomputed per segment
    // instead of staying live (and spilled) across the segment epilogue.
    int vt = tid;
    asm volatile("" : "+v"(vt));
    p.init(vt);
    p.bind(g, m0, n0);
    p.template run<false>(lds, k0, k1);
    const int nseg = s.ks == s.KT ? 1
                                  : 2 + tl.owner(t * tl.L + tl.L - 1) - tl.owner(t * tl.L);
    if (nseg == 1) {
      p.template store<ACT, BIAS>(lds, g, m0, n0);
      continue;
    }
    int* arrived = s.counters + 2 * t;
    int* written = arrived + 1;
    if (tid == 0)
      *arrival = __hip_atomic_fetch_add(arrived, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    const int order = *arrival;
    __syncthreads();  // the word is refilled by the next segment's loads
    // Partials move with device-scope relaxed atomic stores and loads (one
    // dword each, lane-contiguous), so publishing one needs no L2
    // write-back and reading one no L2 invalidate (either would stall every
    // CU of the XCD): a partial is visible device-wide once its stores have
    // completed.  Layout: [slot][block a*4+b][element e][thread].
    if (order < nseg - 1) {
      // Not last: publish this segment's partial in slot `order`, tagged
      // with the segment, then count it.
      if (tid == 0)
        __hip_atomic_store(s.tags + t * kSkSlots + order, seg, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      f32x4_t* const dst = reinterpret_cast<f32x4_t*>(
                               s.slots + ((int64_t)t * kSkSlots + order) * kSlotVec) + vt;
#pragma unroll
      for (int a = 0; a < 8; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b)
          asm volatile("global_store_dwordx4 %0, %1, off sc1\n\ts_nop 1"  // store-data hazard
                       :: "v"(dst + (a * 4 + b) * kThreads), "v"(p.acc[a][b]) : "memory");
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      if (tid == 0) __hip_atomic_fetch_add(written, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      continue;
    }
    // Last: wait (device-scope relaxed loads) for the other nseg - 1, at
    // most kSkSpinLimit polls.  A wait that gives up records the tile in
    // the sticky status word, resets the tile's counters and leaves the
    // tile's output unwritten; the launch still ends normally.
    if (tid == 0) {
      int polls = 0;
      while (__hip_atomic_load(written, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != nseg - 1 &&
             ++polls < kSkSpinLimit)
        __builtin_amdgcn_s_sleep(2);
      *arrival = polls < kSkSpinLimit;
      // which segment each stored slot holds (written before it was counted)
      arrival[1] = __hip_atomic_load(s.tags + t * kSkSlots, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT);
      if (polls >= kSkSpinLimit) {
        __hip_atomic_store(s.status, 1 + t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(arrived, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(written, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    __syncthreads();
    const bool complete = arrival[0];
    const int tag0 = arrival[1];
    __syncthreads();  // the words are staged output space below
    if (!complete) continue;
    // The slots of the (one or two) other segments in segment order: the
    // lower one, o1, and the higher (with one stored partial it is slot 0).
    const int o1 = seg == 0 ? 1 : 0;
    const int slot1 = tag0 == o1 ? 0 : 1, slot2 = 1 - slot1;
    const f32x4_t* const tbase =
        reinterpret_cast<const f32x4_t*>(s.slots + (int64_t)t * kSkSlots * kSlotVec) + vt;
    const f32x4_t* const src1 = tbase + (int64_t)(nseg == 2 ? 0 : slot1) * kSlotVec;
    const f32x4_t* const src2 = tbase + (int64_t)slot2 * kSlotVec;
    // One accumulator row (a) at a time: load its partials (loads and wait in
    // one asm statement, so its outputs are complete when it returns), sum
    // each block in segment order -- fp32 add is commutative, so putting this
    // segment's acc in its place gives the segment-order sum -- and stage the
    // block at once.
#pragma unroll
    for (int a = 0; a < 8; ++a) {
      const f32x4_t bias = p.template load_bias<BIAS>(g, n0, a);
      f32x4_t q1[4], q2[4];
      if (nseg == 3) {
        load_row_sc1(q1, q2, src1 + a * 4 * kThreads, src2 + a * 4 * kThreads);
      } else {
        load_row_sc1(q1, src1 + a * 4 * kThreads);
#pragma unroll
        for (int b = 0; b < 4; ++b) q2[b] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const f32x4_t A = p.acc[a][b];
        f32x4_t r;
        if (seg == 0) r = A + q1[b];          // s0 = acc, s1
        else if (seg == 1) r = q1[b] + A;     // s0, s1 = acc
        else r = q1[b] + q2[b];               // s0, s1 (s2 = acc below)
        if (nseg == 3) r = seg == 2 ? r + A : r + q2[b];
        p.template stage_block<ACT, BIAS>(lds, a, b, r, r, bias);
      }
    }
    p.flush(lds, g, m0, n0);
    if (tid == 0) {
      __hip_atomic_store(arrived, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(written, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// ---- Stream-K on the four-wave core ---------------------------------------
//
// For K % 64 == 0, a long K loop (K >= 8192, w4sk_plan) and tiles that fill
// most but not all CUs (down_proj at M = 3100: 208 tiles on 256 CUs), the
// data-parallel four-wave kernel leaves the remaining CUs idle.  Here Gt
// "tail" workgroups (a multiple of 8, at
// most T) take the last L = KT - ks stages of every tile while T "main"
// workgroups run the first ks stages of one tile each, in lockstep as in the
// data-parallel kernel.  Tail j owns units [j*Ut/Gt, (j+1)*Ut/Gt) of the
// Ut = T*L (tile, stage) pairs, tile-major, so with Gt <= T a tile's tail
// stages are covered by one or two pieces (tails owner(t*L) ..
// owner(t*L + L - 1)); piece (j, t) stores its fp32 partial in slot j + t
// (pieces run along the unit line, each step advancing j or t or both, so
// the slots are distinct: T + Gt - 1 of them) and counts itself on the
// tile's counter.  The main workgroup always reduces: after its K loop it
// waits for the tile's piece count, adds the pieces in K order (main, lower
// piece, higher piece: deterministic whatever the arrival order), applies
// the epilogue, stores the tile and clears the counter.  Tails take the
// lowest workgroup ids, which the hardware dispatches first, and never wait,
// so a waiting main's tails are running or done; the wait is still bounded
// by kSkSpinLimit polls, recording 1 + tile in the status word on expiry
// (the tile is then left unwritten and the launch ends normally).
// Workspace: the stream-K counter region (counters[t] at 4t bytes, the
// status word at kSkStatusOffset), then the slots, each [wave][a][b][lane]
// f32x4 (256 KB).
struct W4SkArgs {
  int* counters;   // [T]: tail pieces stored (zero between launches)
  int* status;     // sticky status word (0: every wait completed)
  f32x4_t* slots;  // [T + Gt - 1][kW4SlotVec]
  int T, KT, ks, Gt;
};
constexpr int kW4SlotVec = 64 * kW4Threads;  // f32x4 per partial (256 KB)
constexpr int kW4SkFlag = 150 * 1024;        // LDS word past the staged output
static_assert(kW4SkFlag >= kBM * W4Tile<1>::kOutRow && kW4SkFlag + 4 <= kW4LdsBytes &&
                  kW4SkFlag >= 2 * kW4StageBytes,
              "the wait flag lies past the staged output and the K-loop stages");

// Tail workgroup owning unit v, and tail j's first unit.
__device__ __forceinline__ int w4sk_owner(int64_t v, int64_t Ut, int Gt) {
  return (int)(((v + 1) * Gt - 1) / Ut);
}
__device__ __forceinline__ int w4sk_start(int j, int64_t Ut, int Gt) {
  return (int)((int64_t)j * Ut / Gt);
}

template <int NBX>
__device__ __forceinline__ void w4sk_piece(W4Tile<1>& c, int n, f32x4_t* dst) {
  c.template kloop<NBX>(n);
  c.template store_partial<NBX>(dst);
}

// The main workgroup's tile: K loop over [0, ks), the wait for its np tail
// pieces, the reduction and staging.  Returns false when the wait gave up.
template <int NBX, int ACT, bool BIAS>
__device__ __forceinline__ bool w4sk_main(W4Tile<1>& c, const GemmArgs& g, const W4SkArgs& s,
                                          int t, int n0, int np, const f32x4_t* p1,
                                          const f32x4_t* p2, int* flag) {
  c.template kloop<NBX>(s.ks);
  if (threadIdx.x == 0) {
    int* const cnt = s.counters + t;
    int polls = 0;
    while (__hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != np &&
           ++polls < kSkSpinLimit)
      __builtin_amdgcn_s_sleep(2);
    *flag = polls < kSkSpinLimit;
    if (polls >= kSkSpinLimit)
      __hip_atomic_store(s.status, 1 + t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!*flag) return false;
  c.template stage_out_sum<NBX, ACT, BIAS>(g, n0, p1, p2, np == 2);
  return true;
}

template <int ACT, bool BIAS>
__global__ __launch_bounds__(kW4Threads, 1) void gemm_w4sk_kernel(GemmArgs g, W4SkArgs s) {
  __shared__ __attribute__((aligned(16))) char smem[kW4LdsBytes];
  const int h = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int L = s.KT - s.ks;
  const int64_t Ut = (int64_t)s.T * L;
  W4Tile<1> c;
  c.init(smem, g);
  auto begin = [&](int t, int k0, int& m0, int& n0, int64_t& mlim) {
    tile_origin(g, t, kBW, m0, n0);
    mlim = std::min<int64_t>(g.M, (int64_t)m0 + g.bm);
    c.src = c.bind(g, m0, n0, mlim);
    c.kbase = k0 * kW4BK;
    const int live = (int)(mlim - m0) - c.xbase;
#pragma unroll
    for (int q = 0; q < 16; ++q) c.issue(0, 0, q);
#pragma unroll
    for (int q = 0; q < 16; ++q) c.issue(1, kW4BK, q);
    w4_wait<16, 0>();
    w4_barrier();
    return __builtin_amdgcn_readfirstlane(live <= 0 ? 0 : min(8, (live + 15) / 16));
  };
  if (h < s.Gt) {
    // Tail h: its pieces in unit order.
    for (int v = w4sk_start(h, Ut, s.Gt), vend = w4sk_start(h + 1, Ut, s.Gt); v < vend;) {
      const int t = v / L, r = v - t * L, len = min(L - r, vend - v);
      int m0, n0;
      int64_t mlim;
      const int nbx = begin(t, s.ks + r, m0, n0, mlim);
      f32x4_t* const dst = s.slots + (int64_t)(h + t) * kW4SlotVec + c.wave * 4096 + lane;
      switch (nbx) {
        case 8: w4sk_piece<8>(c, len, dst); break;
        case 7: w4sk_piece<7>(c, len, dst); break;
        case 6: w4sk_piece<6>(c, len, dst); break;
        case 5: w4sk_piece<5>(c, len, dst); break;
        case 4: w4sk_piece<4>(c, len, dst); break;
        case 3: w4sk_piece<3>(c, len, dst); break;
        case 2: w4sk_piece<2>(c, len, dst); break;
        case 1: w4sk_piece<1>(c, len, dst); break;
        default: w4sk_piece<0>(c, len, dst); break;
      }
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      if (threadIdx.x == 0)
        __hip_atomic_fetch_add(s.counters + t, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      v += len;
    }
    return;
  }
  // Main workgroup u: tile t in the XCD-grouped order (Gt % 8 == 0, so u
  // and h share their XCD).
  const int u = h - s.Gt;
  const int per_xcd = (s.T + 7) >> 3;
  const int t = (u & 7) * per_xcd + (u >> 3);
  if (t >= s.T) return;
  int m0, n0;
  int64_t mlim;
  const int nbx = begin(t, 0, m0, n0, mlim);
  const int j0 = w4sk_owner((int64_t)t * L, Ut, s.Gt);
  const int j1 = w4sk_owner((int64_t)t * L + L - 1, Ut, s.Gt);
  const int np = j1 - j0 + 1;
  const f32x4_t* const p1 = s.slots + (int64_t)(j0 + t) * kW4SlotVec + c.wave * 4096 + lane;
  const f32x4_t* const p2 = s.slots + (int64_t)(j1 + t) * kW4SlotVec + c.wave * 4096 + lane;
  int* const flag = reinterpret_cast<int*>(smem + kW4SkFlag);
  bool ok;
  switch (nbx) {
    case 8: ok = w4sk_main<8, ACT, BIAS>(c, g, s, t, n0, np, p1, p2, flag); break;
    case 7: ok = w4sk_main<7, ACT, BIAS>(c, g, s, t, n0, np, p1, p2, flag); break;
    case 6: ok = w4sk_main<6, ACT, BIAS>(c, g, s, t, n0, np, p1, p2, flag); break;
    case 5: ok = w4sk_main<5, ACT, BIAS>(c, g, s, t, n0, np, p1, p2, flag); break;
    case 4: ok = w4sk_main<4, ACT, BIAS>(c, g, s, t, n0, np, p1, p2, flag); break;
    case 3: ok = w4sk_main<3, ACT, BIAS>(c, g, s, t, n0, np, p1, p2, flag); break;
    case 2: ok = w4sk_main<2, ACT, BIAS>(c, g, s, t, n0, np, p1, p2, flag); break;
    case 1: ok = w4sk_main<1, ACT, BIAS>(c, g, s, t, n0, np, p1, p2, flag); break;
    default: ok = w4sk_main<0, ACT, BIAS>(c, g, s, t, n0, np, p1, p2, flag); break;
  }
  if (!ok) return;
  __syncthreads();
  w4_flush<1>(smem, g, m0, n0, mlim);
}

// ---- Few-row (decode) path --------------------------------------------
//
// With M <= kGemvMaxRows the product is a weight stream: every weight byte is
// used M times, so MFMA tiles (one 256-row x tile mostly padding) waste the
// machine; hipBLASLt's GEMV kernels reach 0.6-3.6 TB/s on the config-5
// decode shapes (N = 1024 .. 12288, K = 4096 / 12288).  Here one workgroup
// owns kGemvCols consecutive output columns and streams their weight rows
// (for P5: the gate and the up row of each column) in 1 KB coalesced wave
// loads; its kGemvWaves waves split K (slab j of 64 16-byte chunks goes to
// wave j mod kGemvWaves), so even N = 1024 gives 2048 waves, 8 per CU, and
// each lane keeps U slabs in flight.  x rows are re-read per slab from L2
// (at most 8 x 24 KB).  fp32 FMAs per lane, a butterfly over the 64 lanes,
// the four waves' partials summed through LDS, then the GEMM's epilogue
// (bias, GELU, silu(g) * u) and one bf16 rounding.
constexpr int kGemvMaxRows = 8;
constexpr int kGemvCols = 2;
constexpr int kGemvWaves = 4;  // per 256-thread workgroup

template <int NB, int ACT, bool BIAS>
__device__ __forceinline__ float gemv_epilogue(float v, float u, float bias) {
  if constexpr (NB == 2) {
    // as the GEMM epilogue: silu(g) * u with the hardware exp2 / reciprocal
    const float den = 1.0f + __builtin_amdgcn_exp2f(v * -1.4426950408889634f);
    return v * __builtin_amdgcn_rcpf(den) * u;
  } else {
    if constexpr (BIAS) v = v + bias;
    if constexpr (ACT == UMIC_ACT_GELU) v = gelu_erf(v);
    if constexpr (ACT == UMIC_ACT_GELU_TANH) v = gelu_tanh(v);
    return v;
  }
}

// The GEMV kernel's one argument: x, and up to kGemvMaxSegs linears over it
// in one launch (the attention's q/k/v projections at decode).  Segment i
// owns workgroups [first[i], first[i + 1]) and has its own weights, bias,
// output, N and leading dims; a single linear, or P5 with its gate/up pair
// in w0/w1, is one segment.  Every operand the kernel reads comes from here.
constexpr int kGemvMaxSegs = 3;
struct GemvSeg {
  const uint16_t* w0;    // linear weight, or P5's gate weight
  const uint16_t* w1;    // P5's up weight (read only when NB == 2)
  const uint16_t* bias;  // or NULL
  uint16_t* out;
  int64_t N, ldw0, ldw1, ldo;
};
// The RMSNorm (optionally after a residual add) that a norm-prologue launch
// applies to x before the GEMV: y = bf16(w * bf16(v * rstd)), v = x or
// bf16(x + r), rstd from the sum of v^2 in the order of torch's wide
// reduction plan (bw reducing threads, k4 4-vectors each, norm.hip's
// rms_wide_kernel).  Workgroup 0 writes v (s, ADD) and y when asked.
struct GemvNorm {
  const uint16_t* w;  // [K] norm weight
  const uint16_t* r;  // residual rows (add form)
  uint16_t* s;        // bf16(x + r) rows out (add form), or NULL
  uint16_t* y;        // normalized rows out, or NULL
  int64_t ldr, lds, ldy;
  float factor, eps;
  int bw, k4;
};
struct GemvJob {
  const uint16_t* x;
  const uint16_t* resid;  // out = bf16(resid + bf16(result)), or NULL
  int64_t M, K, ldx, ldr;
  GemvSeg seg[kGemvMaxSegs];
  int64_t first[kGemvMaxSegs + 1];
  int count;
  GemvNorm nrm;  // used by the norm-prologue instantiations only
};

// Rows and LDS of the norm-prologue launches: each workgroup keeps the
// normalized rows (MR x K bf16) in LDS.
constexpr int kGemvNormMaxRows = 2;
constexpr int64_t kGemvNormMaxLds = 64 << 10;

// FULL: K is a whole number of passes (every slab of every pass is inside
// K: K a multiple of 2048 U, as 4096 and 12288), so the per-slab bounds
// tests are compile-time true -- a branch inside the streaming loop.
// Bit-identical; 1-2% faster at the config-5 decode sites.
template <int NB, int ACT, bool BIAS, int MR, bool FULL = false>
__global__ __launch_bounds__(kGemvWaves * 64) void gemv_kernel(GemvJob job) {
  int si = 0;  // launch-uniform per workgroup
#pragma unroll
  for (int i = 1; i < kGemvMaxSegs; ++i)
    if (i < job.count && (int64_t)blockIdx.x >= job.first[i]) si = i;
  const GemvSeg& sg = job.seg[si];
  const int64_t N = sg.N, K = job.K, M = job.M;
  constexpr int R = kGemvCols;
  // Slabs in flight per lane.  With U = 4 a workgroup's waves cover 1024
  // chunks per pass, but K = 4096 has 512: half the waves sat idle, and the
  // config-5 decode sites ran 11-22% slower than with U = 2 (graph-timed on
  // MI355X).  Eight rows hold eight x slabs per weight slab: U = 1 there.
  constexpr int U = MR >= 8 ? 1 : 2;
  __shared__ float part[kGemvWaves][MR * NB * R];
  const int lane = (int)threadIdx.x & 63;
  const int wave = (int)threadIdx.x >> 6;
  const int64_t n0 = ((int64_t)blockIdx.x - job.first[si]) * R;  // each segment covers its N
  const int64_t chunks = K / 8;
  // Columns past N (when N % R != 0) and x rows past M re-read the last
  // valid row; their results are not stored.
  const uint16_t* wr[NB][R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t n = n0 + r < N ? n0 + r : N - 1;
    wr[0][r] = sg.w0 + n * sg.ldw0;
    if constexpr (NB == 2) wr[NB - 1][r] = sg.w1 + n * sg.ldw1;
  }
  const uint16_t* xr[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) xr[m] = job.x + (m < M ? m : M - 1) * job.ldx;
  float acc[MR][NB][R];
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int r = 0; r < R; ++r) acc[m][b][r] = 0.0f;
  for (int64_t c0 = lane + (int64_t)64 * U * wave; c0 < chunks; c0 += 64 * U * kGemvWaves) {
    u32x4 wv[U][NB][R], xv[U][MR];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t c = FULL || c0 + 64 * u < chunks ? c0 + 64 * u : c0;  // c0 < chunks
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int r = 0; r < R; ++r)
          wv[u][b][r] = ld_stream(reinterpret_cast<const u32x4*>(wr[b][r] + c * 8));
#pragma unroll
      for (int m = 0; m < MR; ++m) xv[u][m] = *reinterpret_cast<const u32x4*>(xr[m] + c * 8);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (!FULL && c0 + 64 * u >= chunks) break;
      float xf[MR][8];
#pragma unroll
      for (int m = 0; m < MR; ++m) unpack8(xv[u][m], xf[m]);
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int r = 0; r < R; ++r) {
          float wf[8];
          unpack8(wv[u][b][r], wf);
#pragma unroll
          for (int m = 0; m < MR; ++m)
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[m][b][r] = __builtin_fmaf(wf[e], xf[m][e], acc[m][b][r]);
        }
    }
  }
  // every lane ends with the column totals
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int s = 32; s >= 1; s >>= 1) acc[m][b][r] += __shfl_xor(acc[m][b][r], s, kWave);
  // the waves' K parts, summed in a fixed order by wave 0
  if (lane == 0) {
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int r = 0; r < R; ++r) part[wave][(m * NB + b) * R + r] = acc[m][b][r];
  }
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float t = part[0][(m * NB + b) * R + r];
#pragma unroll
        for (int w = 1; w < kGemvWaves; ++w) t += part[w][(m * NB + b) * R + r];
        acc[m][b][r] = t;
      }
  // lane m stores row m (static indices: a select per row, no dynamic
  // register indexing)
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    if (lane != m || m >= M) continue;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t n = n0 + r;
      if (n >= N) continue;
      const float bias = BIAS && sg.bias ? bf2f(sg.bias[n]) : 0.0f;
      float o = gemv_epilogue<NB, ACT, BIAS>(acc[m][0][r], acc[m][NB - 1][r], bias);
      // the eager residual add after the linear: two bf16 roundings
      if (job.resid) o = rbf(o) + bf2f(job.resid[m * job.ldr + n]);
      sg.out[m * sg.ldo + n] = (uint16_t)f2bf(o);
    }
  }
}

template <int NB, int ACT, bool BIAS, int MR>
void launch_gemv_mr(const GemvJob& job, dim3 gd, dim3 bd, hipStream_t st) {
  constexpr int64_t pass = (int64_t)2048 * (MR >= 8 ? 1 : 2);  // K per pass of the waves
  if (job.K % pass == 0)
    hipLaunchKernelGGL((gemv_kernel<NB, ACT, BIAS, MR, true>), gd, bd, 0, st, job);
  else
    hipLaunchKernelGGL((gemv_kernel<NB, ACT, BIAS, MR, false>), gd, bd, 0, st, job);
}

template <int NB, int ACT, bool BIAS>
int launch_gemv_job(const GemvJob& job, hipStream_t st) {
  const int64_t grid = job.first[job.count];
  if (grid <= 0 || grid > 0x7fffffffLL) return UMIC_ERR_UNSUPPORTED;
  const dim3 gd((unsigned)grid), bd(kGemvWaves * 64);
  if (job.M <= 1)
    launch_gemv_mr<NB, ACT, BIAS, 1>(job, gd, bd, st);
  else if (job.M <= 2)
    launch_gemv_mr<NB, ACT, BIAS, 2>(job, gd, bd, st);
  else if (job.M <= 4)
    launch_gemv_mr<NB, ACT, BIAS, 4>(job, gd, bd, st);
  else
    launch_gemv_mr<NB, ACT, BIAS, 8>(job, gd, bd, st);
  return launch_status();
}

// A one-segment job: one linear (or the P5 pair), one workgroup per
// kGemvCols output columns; resid/ldr for the residual-add epilogue.
GemvJob gemv_job(const GemmArgs& g, const uint16_t* resid = nullptr, int64_t ldr = 0) {
  GemvJob job{};
  job.x = g.x;
  job.resid = resid;
  job.M = g.M;
  job.K = g.K;
  job.ldx = g.ldx;
  job.ldr = ldr;
  job.seg[0] = GemvSeg{g.w0, g.w1, g.bias, g.out, g.N, g.ldw0, g.ldw1, g.ldo};
  job.count = 1;
  job.first[0] = 0;
  job.first[1] = (g.N + kGemvCols - 1) / kGemvCols;
  return job;
}

// Compute units of the current device (cached per device).
int device_cus() {
  static int cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cus[dev] = n;
  }
  return cus[dev];
}

// ---- Norm-folded GEMV (decode) --------------------------------------------
//
// The decode GEMV with the RMSNorm of its input (after a residual add, ADD)
// folded in.  The norm's statistic spans the whole row, so every workgroup
// computes it itself, from L2, once: the launch is persistent (a grid that
// fits on the device at once), and each workgroup normalizes the MR rows into
// LDS, then walks the column groups blockIdx.x, + gridDim.x, ...  The norm's
// loads are issued before the first group's weight loads (a wait for them
// then does not wait for the weights), kept in registers, and the
// normalization is exactly rms_wide_kernel<ADD, bw, k4>'s (norm.hip): thread
// t plays reducing threads t and t + 256, each summing the squares of its
// 4-vectors vt, vt + bw, ... into four accumulators, ((a0 + a1) + a2) + a3,
// wavefront 0 halving the bw / 64 wavefront columns and finishing with the
// in-wavefront tree, the correctly rounded rsqrt, then bf16(w * bf16(v *
// rstd)) in pairs.  The products, their order and the epilogue are
// gemv_kernel's (act none, optional bias), so results are bit-identical to
// the RMSNorm launch followed by the GEMV launch.
constexpr int kNormPV = 4;  // 4-vectors per thread and row

template <int NB, bool BIAS, int MR, bool FULL, bool ADD>
__global__ __launch_bounds__(kGemvWaves * 64) void gemv_norm_kernel(GemvJob job) {
  extern __shared__ __attribute__((aligned(16))) uint16_t xs[];  // [MR][K] normalized rows
  __shared__ float red[512];
  __shared__ float stat[MR];
  constexpr int R = kGemvCols;
  constexpr int U = 2;
  __shared__ float part[kGemvWaves][MR * NB * R];
  const int t = (int)threadIdx.x, lane = t & 63, wave = t >> 6;
  const int64_t K = job.K, chunks = K / 8;
  const int64_t total = job.first[job.count];
  const GemvNorm& nm = job.nrm;
  const int bw = nm.bw, k4 = nm.k4, nv = (int)(K / 4);
  const int nvt = bw > 256 ? 2 : (t < bw ? 1 : 0);  // reducing threads played by t
  // 1. the norm's operands of this thread: vector j is reducing thread
  //    t + (j / k4) * 256's k = j % k4 th
  int pidx[kNormPV];
  bool pok[kNormPV];
  u32x2 px[MR][kNormPV], pw[kNormPV];
  [[maybe_unused]] u32x2 pr[MR][kNormPV];
#pragma unroll
  for (int j = 0; j < kNormPV; ++j) {
    const int a = j / k4, k = j - a * k4;
    const int idx = t + a * 256 + k * bw;
    pok[j] = a < nvt && idx < nv;
    pidx[j] = pok[j] ? idx : 0;
    if (pok[j]) {
      pw[j] = *reinterpret_cast<const u32x2*>(nm.w + pidx[j] * 4);
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        px[m][j] = *reinterpret_cast<const u32x2*>(job.x + m * job.ldx + pidx[j] * 4);
        if constexpr (ADD) pr[m][j] = *reinterpret_cast<const u32x2*>(nm.r + m * nm.ldr + pidx[j] * 4);
      }
    }
  }
  // 2. the first group's weights
  int64_t blk = blockIdx.x;
  const uint16_t* wr[NB][R];
  int64_t n0 = 0;
  int si = 0;
  auto setup = [&](int64_t b) {
    si = 0;
#pragma unroll
    for (int i = 1; i < kGemvMaxSegs; ++i)
      if (i < job.count && b >= job.first[i]) si = i;
    const GemvSeg& sg = job.seg[si];
    n0 = (b - job.first[si]) * R;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t n = n0 + r < sg.N ? n0 + r : sg.N - 1;
      wr[0][r] = sg.w0 + n * sg.ldw0;
      if constexpr (NB == 2) wr[NB - 1][r] = sg.w1 + n * sg.ldw1;
    }
  };
  u32x4 wv[U][NB][R];
  auto load_w = [&](int64_t cb) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t c = FULL || cb + 64 * u < chunks ? cb + 64 * u : cb;  // cb < chunks
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int r = 0; r < R; ++r)
          wv[u][b][r] = ld_stream(reinterpret_cast<const u32x4*>(wr[b][r] + c * 8));
    }
  };
  const int64_t c0 = lane + (int64_t)64 * U * wave;
  setup(blk);
  if (c0 < chunks) load_w(c0);
  // 3. the norm, row by row, into xs
  const bool lead = blockIdx.x == 0;
  auto vals = [&](int m, int j, float f[4]) {
    unpack4(px[m][j], f);
    if constexpr (ADD) {
      float rf[4];
      unpack4(pr[m][j], rf);
#pragma unroll
      for (int e = 0; e < 4; ++e) f[e] = rbf(f[e] + rf[e]);
    }
  };
#pragma unroll
  for (int m = 0; m < MR; ++m) {
#pragma unroll
    for (int a = 0; a < 2; ++a) {
      float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < kNormPV; ++j) {
        if (j / k4 != a || !pok[j]) continue;
        float f[4];
        vals(m, j, f);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = acc[i] + f[i] * f[i];
      }
      if (a < nvt) red[t + a * 256] = ((acc[0] + acc[1]) + acc[2]) + acc[3];
    }
    __syncthreads();
    if (t < kWave) {
      for (int h = bw / kWave / 2; h >= 1; h >>= 1)
        for (int w = 0; w < h; ++w)
          red[w * kWave + lane] = red[w * kWave + lane] + red[(w + h) * kWave + lane];
      const float tot = group_sum<kWave>(red[lane]);
      if (t == 0) stat[m] = rsqrt_cr(tot * nm.factor + nm.eps);
    }
    __syncthreads();
    const float rstd = stat[m];
#pragma unroll
    for (int j = 0; j < kNormPV; ++j) {
      if (!pok[j]) continue;
      float f[4], wf[4], o[4];
      vals(m, j, f);
      if (ADD && lead && nm.s) *reinterpret_cast<u32x2*>(nm.s + m * nm.lds + pidx[j] * 4) = pack4(f);
      unpack4(pw[j], wf);
#pragma unroll
      for (int e = 0; e < 4; e += 2) {  // bf16(v * rstd) in pairs
        float p0 = f[e] * rstd, p1 = f[e + 1] * rstd;
        rbf2(p0, p1);
        o[e] = wf[e] * p0;
        o[e + 1] = wf[e + 1] * p1;
      }
      const u32x2 y = pack4(o);
      *reinterpret_cast<u32x2*>(xs + m * K + pidx[j] * 4) = y;
      if (lead && nm.y) *reinterpret_cast<u32x2*>(nm.y + m * nm.ldy + pidx[j] * 4) = y;
    }
  }
  __syncthreads();
  // 4. the column groups: gemv_kernel's products and epilogue on xs.  A
  //    group's first-pass weights were loaded before it starts (the next
  //    group's go out right after this group's products, so they are in
  //    flight through its reduction and stores).
  while (true) {
    const int cur_si = si;
    const int64_t cur_n0 = n0;
    float acc[MR][NB][R];
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int r = 0; r < R; ++r) acc[m][b][r] = 0.0f;
    for (int64_t cb = c0; cb < chunks; cb += 64 * U * kGemvWaves) {
      if (cb != c0) load_w(cb);
      u32x4 xv[U][MR];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t c = FULL || cb + 64 * u < chunks ? cb + 64 * u : cb;
#pragma unroll
        for (int m = 0; m < MR; ++m) xv[u][m] = *reinterpret_cast<const u32x4*>(xs + m * K + c * 8);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (!FULL && cb + 64 * u >= chunks) break;
        float xf[MR][8];
#pragma unroll
        for (int m = 0; m < MR; ++m) unpack8(xv[u][m], xf[m]);
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
          for (int r = 0; r < R; ++r) {
            float wf[8];
            unpack8(wv[u][b][r], wf);
#pragma unroll
            for (int m = 0; m < MR; ++m)
#pragma unroll
              for (int e = 0; e < 8; ++e) acc[m][b][r] = __builtin_fmaf(wf[e], xf[m][e], acc[m][b][r]);
          }
      }
    }
    const int64_t next = blk + gridDim.x;
    if (next < total) {
      setup(next);
      if (c0 < chunks) load_w(c0);
    }
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
          for (int s = 32; s >= 1; s >>= 1) acc[m][b][r] += __shfl_xor(acc[m][b][r], s, kWave);
    if (lane == 0) {
#pragma unroll
      for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
          for (int r = 0; r < R; ++r) part[wave][(m * NB + b) * R + r] = acc[m][b][r];
    }
    __syncthreads();
    if (wave == 0) {
      const GemvSeg& sg = job.seg[cur_si];
#pragma unroll
      for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
          for (int r = 0; r < R; ++r) {
            float v = part[0][(m * NB + b) * R + r];
#pragma unroll
            for (int w = 1; w < kGemvWaves; ++w) v += part[w][(m * NB + b) * R + r];
            acc[m][b][r] = v;
          }
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        if (lane != m) continue;
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const int64_t n = cur_n0 + r;
          if (n >= sg.N) continue;
          const float bias = BIAS && sg.bias ? bf2f(sg.bias[n]) : 0.0f;
          const float o = gemv_epilogue<NB, UMIC_ACT_NONE, BIAS>(acc[m][0][r], acc[m][NB - 1][r], bias);
          sg.out[m * sg.ldo + n] = (uint16_t)f2bf(o);
        }
      }
    }
    if (next >= total) break;
    blk = next;
    __syncthreads();  // part is refilled by the next group
  }
}

// Workgroups of a persistent launch that fit on the device at once.  The
// occupancy query is cached per (kernel, LDS size): a decode loop asks the
// same few every step.
int64_t resident_grid(void (*kern)(GemvJob), size_t lds) {
  static std::mutex mu;
  static std::map<std::pair<const void*, size_t>, int> cache;
  const auto key = std::make_pair(reinterpret_cast<const void*>(kern), lds);
  int per_cu = 0;
  {
    std::lock_guard<std::mutex> lock(mu);
    const auto it = cache.find(key);
    if (it != cache.end()) per_cu = it->second;
  }
  if (per_cu == 0) {
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, kGemvWaves * 64, lds) !=
            hipSuccess || per_cu < 1)
      per_cu = 1;
    std::lock_guard<std::mutex> lock(mu);
    cache[key] = per_cu;
  }
  return (int64_t)device_cus() * per_cu;
}

template <int NB, bool BIAS, int MR, bool ADD>
int launch_gemv_norm_mr(const GemvJob& job, hipStream_t st) {
  const size_t lds = (size_t)(MR * job.K * 2);
  const int64_t total = job.first[job.count];
  if (job.K % 4096 == 0) {
    auto kern = gemv_norm_kernel<NB, BIAS, MR, true, ADD>;
    const int64_t grid = std::min<int64_t>(total, resident_grid(kern, lds));
    hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(kGemvWaves * 64), lds, st, job);
  } else {
    auto kern = gemv_norm_kernel<NB, BIAS, MR, false, ADD>;
    const int64_t grid = std::min<int64_t>(total, resident_grid(kern, lds));
    hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(kGemvWaves * 64), lds, st, job);
  }
  return launch_status();
}

template <int NB, bool BIAS, bool ADD>
int launch_gemv_norm(const GemvJob& job, hipStream_t st) {
  const int64_t total = job.first[job.count];
  if (total <= 0 || total > 0x7fffffffLL || device_cus() <= 0) return UMIC_ERR_UNSUPPORTED;
  if (job.M == 1) return launch_gemv_norm_mr<NB, BIAS, 1, ADD>(job, st);
  if (job.M == 2) return launch_gemv_norm_mr<NB, BIAS, 2, ADD>(job, st);
  return UMIC_ERR_UNSUPPORTED;
}

template <int NB, int ACT, bool BIAS>
int launch_gemm(GemmArgs g, hipStream_t st) {
  if (g.M <= kGemvMaxRows) return launch_gemv_job<NB, ACT, BIAS>(gemv_job(g), st);
  const int64_t bn = NB == 1 ? kBW : kBW / 2;
  const int64_t tm = (g.M + kBM - 1) / kBM;
  const int64_t tn = (g.N + bn - 1) / bn;
  if (tm * tn > (int64_t)1 << 28) return UMIC_ERR_UNSUPPORTED;
  g.tiles_m = (int)tm;
  g.tiles = (int)(tm * tn);
  const int cus = device_cus();
  const bool rounds = cus > 0 && g.tiles > cus;
  g.bm = rounds ? tile_rows(g.M) : kBM;
  g.gm = rounds ? kGroupMRounds : kGroupMOne;
  const int64_t grid = ((g.tiles + 7) / 8) * 8;
  if (g.K % kW4BK == 0)
    hipLaunchKernelGGL((gemm_w4_kernel<NB, ACT, BIAS>), dim3((unsigned)grid), dim3(kW4Threads), 0,
                       st, g);
  else
    hipLaunchKernelGGL((gemm_kernel<NB, ACT, BIAS>), dim3((unsigned)grid), dim3(kThreads), 0, st,
                       g);
  return launch_status();
}

// Stream-K pays when the tiles leave CUs idle and the K loop is long: a
// split tile costs about 20 us of fixed work (partial stores, the
// reduction's device-scope loads, extra prologues), measured on MI355X, so
// the main segment must be at least kSkMinMain steps (q/o at K = 4096 stays
// data-parallel; down_proj at K = 12288 gains ~10%); every tail workgroup
// keeps at least kSkMinSteps steps.  This schedule runs on the eight-wave
// core, the data-parallel kernel on the faster four-wave core (K % 64 == 0),
// so it is planned only while the tiles leave most CUs idle: at N = 4096,
// K = 12288 (MI355X, 256 CUs, us data-parallel / eight-wave stream-K)
// M = 512 (32 tiles): 263 / 169, 2048 (128): 270 / 219, 2560 (160): 274 /
// 250, 2816 (176): 279 / 267, 3100 (208): 252 / 269 -- up to 11/16 of the
// CUs; beyond that the four-wave core's own stream-K schedule (w4sk_plan)
// takes long-K shapes.
constexpr int kSkMinSteps = 16;
constexpr int kSkMinMain = 192;
constexpr int kSkMaxTileShare16 = 11;  // tiles <= CUs * 11 / 16

struct SkPlan {
  int64_t tiles;
  int G, KT, ks;
  int64_t counter_bytes, bytes;
  int kind;  // 1: the eight-wave schedule (gemm_sk_kernel), 2: the four-wave one
  int Gt;    // four-wave: tail workgroups
};

// The four-wave schedule (gemm_w4sk_kernel) for K % 64 == 0 shapes whose T
// tiles fill more than kSkMaxTileShare16 / 16 of the CUs but leave some
// idle, with a long K loop: Gt = min(T, CUs - T rounded up to 8), rounded
// down to a multiple of 8, tail workgroups, and the main segment ks (stages
// of 64) the even share T*KT/(T + Gt) plus kW4SkTailExtra stages for the
// tails' per-piece prologues and partial stores.  Measured on MI355X at
// M = 3100, N = 4096, in one process against the data-parallel four-wave
// kernel: down_proj (K = 12288, 208 tiles, Gt = 48) 228-234 against 234-242
// us over ks = 160..165 (157: no gain, 170+: slower; fewer tails, Gt = 40
// .. 16, slower step by step: 234 .. 249 against 230 us); q/o (K = 4096)
// 95-99 against 87-89 us at every ks tried -- the partials' stores and the
// main workgroup's device-scope reads cost more than the idle CUs return,
// so the schedule needs kW4SkMinKT stages.
constexpr int kW4SkTailExtra = 4;
constexpr int kW4SkMinKT = 128;  // K >= 8192
constexpr int kW4SkMinTail = 4;  // tail stages per tile, at least

SkPlan w4sk_plan(int64_t T, int64_t K, int64_t cus) {
  SkPlan pl{0, 0, 0, 0, 0, 0, 0, 0};
  const int64_t KT = K / kW4BK;
  const int64_t T8 = (T + 7) / 8 * 8;
  const int64_t Gt = std::min<int64_t>(T, cus - T8) / 8 * 8;
  if (KT < kW4SkMinKT || Gt < 8 || T > kSkMaxTiles || T * KT >= ((int64_t)1 << 31) / 8)
    return pl;
  const int64_t ks = (T * KT + (T + Gt) / 2) / (T + Gt) + kW4SkTailExtra;
  if (KT - ks < kW4SkMinTail) return pl;
  pl.tiles = T;
  pl.G = (int)(Gt + T8);
  pl.Gt = (int)Gt;
  pl.KT = (int)KT;
  pl.ks = (int)ks;
  pl.kind = 2;
  pl.counter_bytes = kSkCounterBytes;
  pl.bytes = kSkCounterBytes + (T + Gt - 1) * kW4SlotVec * (int64_t)sizeof(f32x4_t);
  return pl;
}

// Workspace layout and grid of the stream-K launch for this shape, or
// bytes = 0 when the data-parallel kernel is the better (or only) choice.
// Stream-K needs fewer tiles T than CUs; G = min(CUs, 2T - 1) workgroups,
// so every tail workgroup covers more than one tile's tail and a tile has
// at most kSkMaxSeg = 3 segments (main, two tail pieces); every workgroup
// keeps at least kSkMinSteps steps.
SkPlan sk_plan(int64_t M, int64_t N, int64_t K) {
  SkPlan pl{0, 0, 0, 0, 0, 0, 0, 0};
  if (M <= kGemvMaxRows || N <= 0 || K <= 0 || K % kBK) return pl;  // few rows: the GEMV
  const int64_t cus = device_cus();
  const int64_t T = ((M + kBM - 1) / kBM) * ((N + kBW - 1) / kBW);
  const int64_t KT = K / kBK;
  const int64_t G = std::min<int64_t>(cus, 2 * T - 1);
  if (cus <= 0 || G <= T || T * KT * G >= ((int64_t)1 << 31)) return pl;
  if (T > kSkMaxTiles) return pl;
  if (K % kW4BK == 0 && T * 16 > cus * kSkMaxTileShare16) return w4sk_plan(T, K, cus);
  // Main workgroups take a sixth of the tail beyond the even share, which
  // offsets the tail workgroups' extra segment prologues and partial stores
  // and makes a main workgroup usually the last to arrive at its tile.
  const int64_t even = T * KT / G;
  const int64_t ks = even + (KT - even) / 6;
  const int64_t L = KT - ks;           // tail steps per tile
  const int64_t per = T * L / (G - T); // tail steps per tail workgroup, at least
  if (ks < kSkMinMain || L <= 0 || per < kSkMinSteps) return pl;
  if (1 + (L + per - 1) / per + 1 > kSkMaxSeg) return pl;
  pl.tiles = T;
  pl.G = (int)G;
  pl.KT = (int)KT;
  pl.ks = (int)ks;
  pl.counter_bytes = kSkCounterBytes;
  pl.bytes = pl.counter_bytes + T * kSkSlots * kSlotVec * (int64_t)sizeof(f32x4_t);
  pl.kind = 1;
  return pl;
}

template <int ACT, bool BIAS>
int launch_gemm_sk(GemmArgs g, const SkPlan& pl, void* ws, hipStream_t st) {
  g.tiles_m = (int)((g.M + kBM - 1) / kBM);
  g.tiles = (int)pl.tiles;
  g.bm = kBM;
  // whole tile columns, m fastest: down_proj at M = 3100 ran 266-269 us
  // against 280-282 us with groups of four tile rows (one process)
  g.gm = g.tiles_m;
  char* const base = static_cast<char*>(ws);
  SkArgs s{reinterpret_cast<int*>(base), reinterpret_cast<int*>(base + kSkStatusOffset),
           reinterpret_cast<int*>(base + kSkTagOffset),
           reinterpret_cast<f32x4_t*>(base + pl.counter_bytes), (int)pl.tiles, pl.KT, pl.ks,
           pl.G};
  const int64_t grid = ((pl.G + 7) / 8) * 8;
  hipLaunchKernelGGL((gemm_sk_kernel<ACT, BIAS>), dim3((unsigned)grid), dim3(kThreads), 0, st, g, s);
  return launch_status();
}

template <int ACT, bool BIAS>
int launch_gemm_w4sk(GemmArgs g, const SkPlan& pl, void* ws, hipStream_t st) {
  g.tiles_m = (int)((g.M + kBM - 1) / kBM);
  g.tiles = (int)pl.tiles;
  g.bm = kBM;
  g.gm = kGroupMOne;
  char* const base = static_cast<char*>(ws);
  W4SkArgs s{reinterpret_cast<int*>(base), reinterpret_cast<int*>(base + kSkStatusOffset),
             reinterpret_cast<f32x4_t*>(base + pl.counter_bytes), (int)pl.tiles, pl.KT, pl.ks,
             pl.Gt};
  hipLaunchKernelGGL((gemm_w4sk_kernel<ACT, BIAS>), dim3((unsigned)pl.G), dim3(kW4Threads), 0, st,
                     g, s);
  return launch_status();
}

template <int ACT, bool BIAS>
int launch_sk(const GemmArgs& g, const SkPlan& pl, void* ws, hipStream_t st) {
  return pl.kind == 2 ? launch_gemm_w4sk<ACT, BIAS>(g, pl, ws, st)
                      : launch_gemm_sk<ACT, BIAS>(g, pl, ws, st);
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

// ---- Allocation-free stream-K --------------------------------------------
//
// umic_linear_sk_static_bf16 runs the stream-K schedule on this file-scope
// scratch instead of a caller's workspace, for callers that cannot allocate
// (code under graph capture, serving loops).  Each device holds its own copy
// for the life of the process.  Host code never passes `scratch` itself --
// on the host the name is a stand-in, not a device address -- only the
// per-device address hipGetSymbolAddress returns (scratch_address).
constexpr int64_t kScratchBytes = (int64_t)64 << 20;
constexpr int kScratchDevices = 64;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

// The device address of `scratch` on the current device, looked up once per
// device with that device current; 0 or a hipError_t value.  *first is true
// for the one call that looked the address up on this device.
int scratch_address(void** out, bool* first) {
  static std::mutex mu;
  static void* addr[kScratchDevices];
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kScratchDevices) return UMIC_ERR_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(mu);
  *first = !addr[dev];
  if (!addr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (!p) return UMIC_ERR_SCRATCH;
    addr[dev] = p;
  }
  *out = addr[dev];
  return UMIC_OK;
}

// Zeroes n ints (the stream-K tile counters) with vector stores: a kernel,
// not a memset, so a captured graph replays it like any other node.
__global__ __launch_bounds__(256) void zero_ints_kernel(int* p, int n) {
  const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (i < n) p[i] = 0;
}

}  // namespace
}  // namespace umic

using namespace umic;

extern "C" int umic_linear_bf16(const void* x, const void* w, const void* bias, void* out,
                                int64_t M, int64_t N, int64_t K, int64_t ldx, int64_t ldw,
                                int64_t ldo, int act, void* stream) {
  if (M < 0 || N < 0 || K < 0) return UMIC_ERR_INVALID_ARG;
  if (act != UMIC_ACT_NONE && act != UMIC_ACT_GELU && act != UMIC_ACT_GELU_TANH)
    return UMIC_ERR_INVALID_ARG;
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
  if (act == UMIC_ACT_GELU_TANH)
    return bias ? launch_gemm<1, UMIC_ACT_GELU_TANH, true>(g, st)
                : launch_gemm<1, UMIC_ACT_GELU_TANH, false>(g, st);
  return bias ? launch_gemm<1, UMIC_ACT_NONE, true>(g, st) : launch_gemm<1, UMIC_ACT_NONE, false>(g, st);
}

extern "C" int64_t umic_linear_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  return sk_plan(M, N, K).bytes;
}

namespace umic {
namespace {

// Argument checks of the stream-K launch (the data-parallel path does its own).
int sk_args_ok(const void* x, const void* w, const void* bias, const void* out, int64_t M,
               int64_t N, int64_t K, int64_t ldx, int64_t ldw, int64_t ldo, int act) {
  if (act != UMIC_ACT_NONE && act != UMIC_ACT_GELU && act != UMIC_ACT_GELU_TANH)
    return UMIC_ERR_INVALID_ARG;
  if (!x || !w || !out) return UMIC_ERR_INVALID_ARG;
  if (ldx < K || ldw < K || ldo < N) return UMIC_ERR_INVALID_ARG;
  if (!gemm_shape_ok(x, w, w, out, M, N, K, ldx, ldw, ldw, ldo)) return UMIC_ERR_UNSUPPORTED;
  if (bias && ((uintptr_t)bias & 7u)) return UMIC_ERR_UNSUPPORTED;
  return UMIC_OK;
}

// The stream-K launch on workspace ws (>= pl.bytes, 256-byte aligned, zero
// counters), after sk_args_ok.
int run_linear_sk(const void* x, const void* w, const void* bias, void* out, int64_t M, int64_t N,
                  int64_t K, int64_t ldx, int64_t ldw, int64_t ldo, int act, const SkPlan& pl,
                  void* workspace, hipStream_t st) {
  GemmArgs g{(const uint16_t*)x, (const uint16_t*)w, (const uint16_t*)w, (const uint16_t*)bias,
             (uint16_t*)out, M, N, K, ldx, ldw, ldw, ldo, 0, 0};
  if (act == UMIC_ACT_GELU)
    return bias ? launch_sk<UMIC_ACT_GELU, true>(g, pl, workspace, st)
                : launch_sk<UMIC_ACT_GELU, false>(g, pl, workspace, st);
  if (act == UMIC_ACT_GELU_TANH)
    return bias ? launch_sk<UMIC_ACT_GELU_TANH, true>(g, pl, workspace, st)
                : launch_sk<UMIC_ACT_GELU_TANH, false>(g, pl, workspace, st);
  return bias ? launch_sk<UMIC_ACT_NONE, true>(g, pl, workspace, st)
              : launch_sk<UMIC_ACT_NONE, false>(g, pl, workspace, st);
}

}  // namespace
}  // namespace umic

extern "C" int umic_linear_ws_bf16(const void* x, const void* w, const void* bias, void* out,
                                   int64_t M, int64_t N, int64_t K, int64_t ldx, int64_t ldw,
                                   int64_t ldo, int act, void* workspace,
                                   int64_t workspace_bytes, void* stream) {
  if (workspace_bytes < 0) return UMIC_ERR_INVALID_ARG;
  const SkPlan pl = sk_plan(M, N, K);
  if (pl.bytes == 0 || workspace_bytes < pl.bytes || !workspace ||
      ((uintptr_t)workspace & 255u))  // data-parallel path
    return umic_linear_bf16(x, w, bias, out, M, N, K, ldx, ldw, ldo, act, stream);
  const int rc = sk_args_ok(x, w, bias, out, M, N, K, ldx, ldw, ldo, act);
  if (rc != UMIC_OK) return rc;
  return run_linear_sk(x, w, bias, out, M, N, K, ldx, ldw, ldo, act, pl, workspace,
                       as_stream(stream));
}

extern "C" int umic_linear_sk_static_bf16(const void* x, const void* w, const void* bias,
                                          void* out, int64_t M, int64_t N, int64_t K,
                                          int64_t ldx, int64_t ldw, int64_t ldo, int act,
                                          void* stream) {
  if (M < 0 || N < 0 || K < 0) return UMIC_ERR_INVALID_ARG;
  if (M == 0 || N == 0) return UMIC_OK;  // empty tensors may carry null pointers
  int rc = sk_args_ok(x, w, bias, out, M, N, K, ldx, ldw, ldo, act);
  if (rc != UMIC_OK) return rc;
  const SkPlan pl = sk_plan(M, N, K);
  if (pl.bytes == 0)  // the data-parallel kernel or the GEMV: no scratch needed
    return umic_linear_bf16(x, w, bias, out, M, N, K, ldx, ldw, ldo, act, stream);
  if (pl.bytes > kScratchBytes) return UMIC_ERR_SCRATCH;
  void* ws = nullptr;
  bool first = false;
  rc = scratch_address(&ws, &first);
  if (rc != UMIC_OK) return rc;
  hipStream_t st = as_stream(stream);
  // The counter region (tile counters and the status word) is cleared once,
  // ahead of the device's first stream-K launch on it; every launch leaves
  // the counters at zero, so later calls find them cleared.  Clearing on
  // every call instead would zero counters that a call still running on
  // another stream is waiting on.
  if (first) {
    const int n = (int)(kSkCounterBytes / sizeof(int));
    hipLaunchKernelGGL(zero_ints_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                       static_cast<int*>(ws), n);
    rc = launch_status();
    if (rc != UMIC_OK) return rc;
  }
  return run_linear_sk(x, w, bias, out, M, N, K, ldx, ldw, ldo, act, pl, ws, st);
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

// The segments of a multi-linear GEMV job, with umic_linear_multi_bf16's
// argument checks; job.first[count] = 0 when every N is 0.
int multi_job(GemvJob& job, const void* x, int64_t M, int64_t K, int64_t ldx, int count,
              const void* const* w, const void* const* bias, void* const* out, const int64_t* N,
              const int64_t* ldw, const int64_t* ldo, bool& any_bias) {
  job.x = (const uint16_t*)x;
  job.M = M;
  job.K = K;
  job.ldx = ldx;
  job.count = count;
  any_bias = false;
  int64_t first = 0;
  for (int i = 0; i < count; ++i) {
    job.first[i] = first;
    if (N[i] == 0) continue;  // empty segment: no workgroups, pointers unused
    if (!w[i] || !out[i] || ldw[i] < K || ldo[i] < N[i]) return UMIC_ERR_INVALID_ARG;
    if (!gemm_shape_ok(x, w[i], w[i], out[i], M, N[i], K, ldx, ldw[i], ldw[i], ldo[i]))
      return UMIC_ERR_UNSUPPORTED;
    const void* b = bias ? bias[i] : nullptr;
    if (b && ((uintptr_t)b & 7u)) return UMIC_ERR_UNSUPPORTED;
    any_bias = any_bias || b;
    job.seg[i] = GemvSeg{(const uint16_t*)w[i], (const uint16_t*)w[i], (const uint16_t*)b,
                         (uint16_t*)out[i], N[i], ldw[i], ldw[i], ldo[i]};
    first += (N[i] + kGemvCols - 1) / kGemvCols;
  }
  job.first[count] = first;
  return UMIC_OK;
}

extern "C" int umic_linear_multi_bf16(const void* x, int64_t M, int64_t K, int64_t ldx, int count,
                                      const void* const* w, const void* const* bias,
                                      void* const* out, const int64_t* N, const int64_t* ldw,
                                      const int64_t* ldo, int act, void* stream) {
  if (M < 0 || K < 0 || count < 1 || count > kGemvMaxSegs) return UMIC_ERR_INVALID_ARG;
  if (!w || !out || !N || !ldw || !ldo) return UMIC_ERR_INVALID_ARG;
  if (act != UMIC_ACT_NONE && act != UMIC_ACT_GELU && act != UMIC_ACT_GELU_TANH)
    return UMIC_ERR_INVALID_ARG;
  for (int i = 0; i < count; ++i)
    if (N[i] < 0) return UMIC_ERR_INVALID_ARG;
  if (M == 0) return UMIC_OK;
  if (M > kGemvMaxRows) return UMIC_ERR_UNSUPPORTED;
  if (!x || ldx < K) return UMIC_ERR_INVALID_ARG;
  if (K == 0) return UMIC_ERR_UNSUPPORTED;
  GemvJob job{};
  bool any_bias = false;
  const int rc = multi_job(job, x, M, K, ldx, count, w, bias, out, N, ldw, ldo, any_bias);
  if (rc != UMIC_OK) return rc;
  if (job.first[count] == 0) return UMIC_OK;
  hipStream_t st = as_stream(stream);
  if (act == UMIC_ACT_GELU)
    return any_bias ? launch_gemv_job<1, UMIC_ACT_GELU, true>(job, st)
                    : launch_gemv_job<1, UMIC_ACT_GELU, false>(job, st);
  if (act == UMIC_ACT_GELU_TANH)
    return any_bias ? launch_gemv_job<1, UMIC_ACT_GELU_TANH, true>(job, st)
                    : launch_gemv_job<1, UMIC_ACT_GELU_TANH, false>(job, st);
  return any_bias ? launch_gemv_job<1, UMIC_ACT_NONE, true>(job, st)
                  : launch_gemv_job<1, UMIC_ACT_NONE, false>(job, st);
}

// torch's reduction plan for an M x K RMSNorm when launch_rms (norm.hip)
// runs it as the wide kernel, which the norm prologue reproduces; false for
// any other plan, or rows / LDS beyond the prologue's limits.
bool gemv_norm_plan(int64_t M, int64_t K, GemvNorm& nm) {
  RmsPlan p;
  if (M < 1 || M > kGemvNormMaxRows || K <= 0 || K % 8 || M * K * 2 > kGemvNormMaxLds)
    return false;
  if (!rms_plan(M, K, p) || !p.vec || p.split || p.bw < 128 || p.bw > 512) return false;
  const int64_t k4 = (K / 4 + p.bw - 1) / p.bw;
  if ((p.bw > 256 ? 2 : 1) * k4 > kNormPV) return false;  // the kernel's vectors per thread
  nm.bw = p.bw;
  nm.k4 = (int)k4;
  nm.factor = (float)M / (float)(M * K);
  return true;
}

// Bytes spanned by M rows of K bf16 at leading dim ld.
inline int64_t row_span(int64_t M, int64_t K, int64_t ld) { return ((M - 1) * ld + K) * 2; }

extern "C" int umic_rmsnorm_linear_multi_bf16(const void* x, const void* norm_w, void* normed,
                                              int64_t M, int64_t K, int64_t ldx, int64_t ldn,
                                              float eps, int count, const void* const* w,
                                              const void* const* bias, void* const* out,
                                              const int64_t* N, const int64_t* ldw,
                                              const int64_t* ldo, void* stream) {
  if (M < 0 || K < 0 || count < 1 || count > kGemvMaxSegs) return UMIC_ERR_INVALID_ARG;
  if (!w || !out || !N || !ldw || !ldo) return UMIC_ERR_INVALID_ARG;
  for (int i = 0; i < count; ++i)
    if (N[i] < 0) return UMIC_ERR_INVALID_ARG;
  if (M == 0) return UMIC_OK;
  if (!x || !norm_w || ldx < K || (normed && ldn < K)) return UMIC_ERR_INVALID_ARG;
  if (K == 0) return UMIC_ERR_UNSUPPORTED;
  GemvJob job{};
  if (!gemv_norm_plan(M, K, job.nrm) || !aligned8(norm_w)) return UMIC_ERR_UNSUPPORTED;
  if (normed && (!aligned8(normed) || ldn % 4)) return UMIC_ERR_UNSUPPORTED;
  // every workgroup reads x while workgroup 0 writes normed
  if (normed && overlaps(normed, row_span(M, K, ldn), x, row_span(M, K, ldx)))
    return UMIC_ERR_INVALID_ARG;
  bool any_bias = false;
  const int rc = multi_job(job, x, M, K, ldx, count, w, bias, out, N, ldw, ldo, any_bias);
  if (rc != UMIC_OK) return rc;
  if (job.first[count] == 0) return UMIC_OK;
  job.nrm.w = (const uint16_t*)norm_w;
  job.nrm.y = (uint16_t*)normed;
  job.nrm.ldy = ldn;
  job.nrm.eps = eps;
  hipStream_t st = as_stream(stream);
  return any_bias ? launch_gemv_norm<1, true, false>(job, st)
                  : launch_gemv_norm<1, false, false>(job, st);
}

extern "C" int umic_add_rmsnorm_gate_silu_mul_bf16(
    const void* x, const void* r, const void* norm_w, void* normed, void* summed, const void* wg,
    const void* wu, void* out, int64_t M, int64_t N, int64_t K, int64_t ldx, int64_t ldr,
    int64_t ldn, int64_t lds, int64_t ldwg, int64_t ldwu, int64_t ldo, float eps, void* stream) {
  if (M < 0 || N < 0 || K < 0) return UMIC_ERR_INVALID_ARG;
  if (M == 0 || N == 0) return UMIC_OK;  // empty tensors may carry null pointers
  if (!x || !r || !norm_w || !wg || !wu || !out) return UMIC_ERR_INVALID_ARG;
  if (ldx < K || ldr < K || ldwg < K || ldwu < K || ldo < N) return UMIC_ERR_INVALID_ARG;
  if ((normed && ldn < K) || (summed && lds < K)) return UMIC_ERR_INVALID_ARG;
  if (K == 0) return UMIC_ERR_UNSUPPORTED;
  if (!gemm_shape_ok(x, wg, wu, out, M, N, K, ldx, ldwg, ldwu, ldo)) return UMIC_ERR_UNSUPPORTED;
  GemmArgs g{(const uint16_t*)x, (const uint16_t*)wg, (const uint16_t*)wu, nullptr,
             (uint16_t*)out, M, N, K, ldx, ldwg, ldwu, ldo, 0, 0};
  GemvJob job = gemv_job(g);
  if (!gemv_norm_plan(M, K, job.nrm) || !aligned8(norm_w) || !aligned8(r) || ldr % 4)
    return UMIC_ERR_UNSUPPORTED;
  if ((normed && (!aligned8(normed) || ldn % 4)) || (summed && (!aligned8(summed) || lds % 4)))
    return UMIC_ERR_UNSUPPORTED;
  // every workgroup reads x and r while workgroup 0 writes normed and summed
  const int64_t sx = row_span(M, K, ldx), sr = row_span(M, K, ldr);
  const int64_t sn = normed ? row_span(M, K, ldn) : 0, ss = summed ? row_span(M, K, lds) : 0;
  if (overlaps(normed, sn, x, sx) || overlaps(normed, sn, r, sr) || overlaps(summed, ss, x, sx) ||
      overlaps(summed, ss, r, sr))
    return UMIC_ERR_INVALID_ARG;
  job.nrm.w = (const uint16_t*)norm_w;
  job.nrm.r = (const uint16_t*)r;
  job.nrm.ldr = ldr;
  job.nrm.s = (uint16_t*)summed;
  job.nrm.lds = lds;
  job.nrm.y = (uint16_t*)normed;
  job.nrm.ldy = ldn;
  job.nrm.eps = eps;
  return launch_gemv_norm<2, false, true>(job, as_stream(stream));
}

extern "C" int umic_linear_add_bf16(const void* x, const void* w, const void* bias,
                                    const void* residual, void* out, int64_t M, int64_t N,
                                    int64_t K, int64_t ldx, int64_t ldw, int64_t ldr, int64_t ldo,
                                    void* stream) {
  if (M < 0 || N < 0 || K < 0) return UMIC_ERR_INVALID_ARG;
  if (M == 0 || N == 0) return UMIC_OK;
  if (M > kGemvMaxRows) return UMIC_ERR_UNSUPPORTED;
  if (!x || !w || !residual || !out) return UMIC_ERR_INVALID_ARG;
  if (ldx < K || ldw < K || ldr < N || ldo < N) return UMIC_ERR_INVALID_ARG;
  if (K == 0) return UMIC_ERR_UNSUPPORTED;
  if (!gemm_shape_ok(x, w, w, out, M, N, K, ldx, ldw, ldw, ldo)) return UMIC_ERR_UNSUPPORTED;
  if (bias && ((uintptr_t)bias & 7u)) return UMIC_ERR_UNSUPPORTED;
  GemmArgs g{(const uint16_t*)x, (const uint16_t*)w, (const uint16_t*)w, (const uint16_t*)bias,
             (uint16_t*)out, M, N, K, ldx, ldw, ldw, ldo, 0, 0};
  const GemvJob job = gemv_job(g, (const uint16_t*)residual, ldr);
  hipStream_t st = as_stream(stream);
  return bias ? launch_gemv_job<1, UMIC_ACT_NONE, true>(job, st)
              : launch_gemv_job<1, UMIC_ACT_NONE, false>(job, st);
}
