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
// Data movement.  K advances in steps of 64: every thread fetches eight
// 16-byte chunks of the weight tile and eight of the x tile per step
// (global_load_dwordx4), parks them in registers while the MFMAs of the
// previous step run, then writes them to the other half of a double-buffered
// LDS (2 x 64 KB) -- one barrier per K step.  LDS rows are 128 bytes with the
// 16-byte chunk index XOR-swizzled by (row & 7), so both the row-wise writes
// and the 32-row fragment reads hit 8 distinct chunk slots per 8 lanes
// (bank-conflict free).  The MFMA A operand is the weight tile, B the x tile,
// so each lane's 16 outputs are 4 runs of 4 consecutive output columns:
// the epilogue writes 8-byte packed bf16 runs.
//
// Workgroup order.  Hardware hands consecutive workgroup ids to the 8 XCDs
// round-robin; the id is remapped so every XCD works through a contiguous
// run of the m-fastest tile order, i.e. the workgroups sharing a weight tile
// run on the same XCD at the same time and the weights stream from HBM
// about once (x is small and stays L2/MALL resident).
#include "common.hpp"

namespace umic {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kBM = 256;     // x rows per tile
constexpr int kBW = 256;     // weight rows per tile (gate+up for P5)
constexpr int kBK = 64;      // K per pipeline step
constexpr int kChunks = kBK / 8;  // 16-byte chunks per LDS row

struct GemmArgs {
  const uint16_t* x;
  const uint16_t* w0;  // linear weight, or gate weight
  const uint16_t* w1;  // up weight (P5)
  const uint16_t* bias;
  uint16_t* out;
  int64_t M, N, K, ldx, ldw0, ldw1, ldo;
  int tiles_m, tiles;
};

__device__ __forceinline__ int swz(int row, int chunk) { return row * kChunks + (chunk ^ (row & 7)); }

template <int NB, int ACT, bool BIAS>
__global__ __launch_bounds__(256, 1) void gemm_kernel(GemmArgs g) {
  // [stage][operand: 0 weights, 1 x][row][chunk] as 16-byte units (128 KB)
  __shared__ u32x4 lds[2][2][kBM * kChunks];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;

  // XCD-aware remap: physical ids b, b+8, b+16, ... (one XCD) take
  // consecutive logical tiles.
  const int per_xcd = (g.tiles + 7) >> 3;
  const int logical = (int)(blockIdx.x & 7) * per_xcd + (int)(blockIdx.x >> 3);
  if (logical >= g.tiles) return;
  const int tm = logical % g.tiles_m;
  const int tn = logical / g.tiles_m;
  const int64_t m0 = (int64_t)tm * kBM;
  const int64_t n0 = (int64_t)tn * (NB == 1 ? kBW : kBW / 2);

  // This thread's 8 weight chunks and 8 x chunks per K step: tile row
  // i*32 + tid/8, chunk tid%8.  Rows past the matrix edge re-read the last
  // row (in bounds); their results are never stored.
  const int crow = tid >> 3, cchunk = tid & 7;
  const uint16_t* wsrc[8];
  const uint16_t* xsrc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int r = i * 32 + crow;
    int64_t wr;
    const uint16_t* wb;
    int64_t ldw;
    if (NB == 1 || r < kBW / 2) {
      wr = n0 + r;
      wb = g.w0;
      ldw = g.ldw0;
    } else {
      wr = n0 + r - kBW / 2;
      wb = g.w1;
      ldw = g.ldw1;
    }
    wr = wr < g.N ? wr : g.N - 1;
    const int64_t xr = (m0 + r) < g.M ? (m0 + r) : g.M - 1;
    wsrc[i] = wb + wr * ldw + cchunk * 8;
    xsrc[i] = g.x + xr * g.ldx + cchunk * 8;
  }

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

  u32x4 wst[8], xst[8];
  auto fetch = [&](int64_t k0) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      wst[i] = *reinterpret_cast<const u32x4*>(wsrc[i] + k0);
      xst[i] = *reinterpret_cast<const u32x4*>(xsrc[i] + k0);
    }
  };
  auto stash = [&](int s) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = i * 32 + crow;
      lds[s][0][swz(r, cchunk)] = wst[i];
      lds[s][1][swz(r, cchunk)] = xst[i];
    }
  };

  const int ksteps = (int)(g.K / kBK);
  fetch(0);
  stash(0);
  __syncthreads();

  for (int kt = 0; kt < ksteps; ++kt) {
    const int s = kt & 1;
    if (kt + 1 < ksteps) fetch((int64_t)(kt + 1) * kBK);
#pragma unroll
    for (int kk = 0; kk < kBK / 16; ++kk) {
      bf16x8_t af[4], bfr[4];
      const int ch = kk * 2 + fk;
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        af[a] = __builtin_bit_cast(bf16x8_t, lds[s][0][swz(arow[a] + frow, ch)]);
        bfr[a] = __builtin_bit_cast(bf16x8_t, lds[s][1][swz(brow[a] + frow, ch)]);
      }
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b)
          acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[a], bfr[b], acc[a][b], 0, 0, 0);
    }
    if (kt + 1 < ksteps) stash(s ^ 1);
    __syncthreads();
  }

  // Epilogue.  acc[a][b][r]: weight row 8*(r/4) + 4*(lane/32) + r%4 of
  // a-block a, x row lane%32 of b-block b.
  constexpr int kOutBlocks = NB == 1 ? 4 : 2;
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const int64_t m = m0 + brow[b] + frow;
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
            const float u = acc[a + 2][b][rr * 4 + e];
            v = v / (1.0f + __expf(-v)) * u;
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

template <int NB, int ACT, bool BIAS>
int launch_gemm(GemmArgs g, hipStream_t st) {
  const int64_t bn = NB == 1 ? kBW : kBW / 2;
  const int64_t tm = (g.M + kBM - 1) / kBM;
  const int64_t tn = (g.N + bn - 1) / bn;
  if (tm * tn > (int64_t)1 << 28) return UMIC_ERR_UNSUPPORTED;
  g.tiles_m = (int)tm;
  g.tiles = (int)(tm * tn);
  const int64_t grid = ((g.tiles + 7) / 8) * 8;
  hipLaunchKernelGGL((gemm_kernel<NB, ACT, BIAS>), dim3((unsigned)grid), dim3(256), 0, st, g);
  return launch_status();
}

bool gemm_shape_ok(const void* x, const void* w0, const void* w1, const void* out, int64_t M,
                   int64_t N, int64_t K, int64_t ldx, int64_t ldw0, int64_t ldw1, int64_t ldo) {
  if (K % kBK != 0 || N % 8 != 0) return false;
  if (ldx % 8 || ldw0 % 8 || ldw1 % 8 || ldo % 8) return false;
  if (!aligned16(x) || !aligned16(w0) || !aligned16(w1) || !aligned16(out)) return false;
  return true;
}

}  // namespace
}  // namespace umic

using namespace umic;

extern "C" int umic_linear_bf16(const void* x, const void* w, const void* bias, void* out,
                                int64_t M, int64_t N, int64_t K, int64_t ldx, int64_t ldw,
                                int64_t ldo, int act, void* stream) {
  if (!x || !w || !out || M < 0 || N < 0 || K < 0) return UMIC_ERR_INVALID_ARG;
  if (act != UMIC_ACT_NONE && act != UMIC_ACT_GELU) return UMIC_ERR_INVALID_ARG;
  if (M > 0 && N > 0 && (ldx < K || ldw < K || ldo < N)) return UMIC_ERR_INVALID_ARG;
  if (M == 0 || N == 0) return UMIC_OK;
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
  if (!x || !wg || !wu || !out || M < 0 || N < 0 || K < 0) return UMIC_ERR_INVALID_ARG;
  if (M > 0 && N > 0 && (ldx < K || ldwg < K || ldwu < K || ldo < N)) return UMIC_ERR_INVALID_ARG;
  if (M == 0 || N == 0) return UMIC_OK;
  if (K == 0) return UMIC_ERR_UNSUPPORTED;
  if (!gemm_shape_ok(x, wg, wu, out, M, N, K, ldx, ldwg, ldwu, ldo)) return UMIC_ERR_UNSUPPORTED;
  GemmArgs g{(const uint16_t*)x, (const uint16_t*)wg, (const uint16_t*)wu, nullptr,
             (uint16_t*)out, M, N, K, ldx, ldwg, ldwu, ldo, 0, 0};
  return launch_gemm<2, UMIC_ACT_NONE, false>(g, as_stream(stream));
}
