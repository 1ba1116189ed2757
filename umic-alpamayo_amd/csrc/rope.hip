// Rotary position embedding for q and k in one gfx950 launch.
//
//   out[d]        = x[d]        * cos[d]        - x[d + D/2] * sin[d]
//   out[d + D/2]  = x[d + D/2]  * cos[d + D/2]  + x[d]       * sin[d + D/2]
// (HF rotate_half convention).  Three work layouts:
//   head group -- (bf16 tables read from global, 16-byte chunks, D a
//                 multiple of 128) a thread owns chunk c of R head rows of
//                 one position: the chunk pair [8c, 8c+8) and the same chunk
//                 shifted by D/2 of each row, so both halves of every
//                 rotation pair are in the same lane, and the position's
//                 cos/sin chunks are loaded once for R rows.  Consecutive
//                 threads walk the chunks, then the head groups, then the
//                 positions; at D = 128 each instruction covers whole
//                 128-byte half rows.
//   item pair  -- (staged tables, or 4- / 2-byte chunks) a work item owns
//                 one head row's chunk pair as above; consecutive items walk
//                 the chunks of a head, then the heads of a position.
//   lane chunk -- (16-byte chunks, D/8 <= 64) a lane owns one contiguous
//                 chunk, a wavefront whole head rows (low halves in lanes
//                 0..31, high halves in 32..63), and the rotation partner
//                 is lane ^ 32: every instruction covers one contiguous run.
//                 Used whenever D is not a multiple of 128: vision (D = 80,
//                 160-byte rows) runs 33 against 40 us in the item-pair
//                 form.
//
// Tables.  cos/sin are read once from HBM for q AND k (the reference's
// per-tensor launches read them twice).  fp32 tables (vision) are staged
// into LDS per block: the block stages the cos/sin rows of the positions its
// range touches, and rotates every item from registers.  bf16 tables (text,
// [S, 128] = 0.8 MB each, L2-resident) are instead read straight from
// global by the head-group form -- 16 bytes per half, once per R rows: as
// fast as the lane-chunk form with staged tables already with one row per
// thread (15.3-16.5 against 15.9-17.0 us at q[1,32,3100,128]), with no
// staging loop and no barrier.  For fp32 tables the per-row reads would be
// 4x the row's own bytes and staging wins.  Activations are streamed with
// non-temporal loads: each element is read once and written once.
//
// Arithmetic modes (no fp contraction anywhere in this library):
//   TEXT   -- every op rounds to bf16, as the eager bf16 chain does:
//             bf16( bf16(x*cos) + bf16(rot*sin) )   (cos/sin bf16)
//   VISION -- fp32 ops, one final rounding: bf16( x*cos + rot*sin ) with the
//             two products and the sum each rounded in fp32 (HF's q.float()
//             path; cos/sin fp32, or bf16 widened exactly).
#include "common.hpp"

#include <algorithm>

namespace umic {
namespace {

struct RopeArgs {
  const uint16_t* q;
  const uint16_t* k;
  uint16_t* qo;
  uint16_t* ko;
  const void* cos;
  const void* sin;
  int64_t B, S, Hq, Hk, D;
  int64_t q_sb, q_ss, q_sh, k_sb, k_ss, k_sh;
  int64_t qo_sb, qo_ss, qo_sh, ko_sb, ko_ss, ko_sh;
  int64_t cs_sb, cs_ss;
  // launch-uniform divisors of the item decomposition: items per position,
  // chunks per half row, head dim (set per launch; see SmallDiv)
  SmallDiv ipp, chunks, dim;
  // RMSNorm of q / k head rows before the rotation (norm kernels only)
  const uint16_t* qw;
  const uint16_t* kw;
  float eps;
  float fq, fk;          // MeanOps factors of the q and k head rows (see rms_norm_chunks)
};

// Items per position are bounded (checked on the host) so that every
// in-block item offset divided by them stays below 2^22 (SmallDiv's range).
constexpr int64_t kMaxItemsPerPos = (int64_t)1 << 21;

constexpr int kMaxCsFloats = 6144;  // LDS budget per staged table (cos, sin): 24 KB each
constexpr int kMaxHeadDim = 1024;
constexpr int kItems = 4;           // work items per thread per pass

// Staged table rows keep each 8-element chunk in 12 floats (48 bytes): the
// chunks one wavefront instruction reads from a row then fall in distinct
// LDS banks (measured with SQ_LDS_BANK_CONFLICT on the vision shape: 97%
// fewer conflict cycles than 8-float chunks, whose chunks c and c + 4 share
// banks).  An item's VEC elements never cross a chunk (VEC divides 8 and
// every item offset is a multiple of VEC).
__host__ __device__ __forceinline__ int cs_slot(int d) { return d + (d >> 3) * 4; }
__host__ __device__ __forceinline__ int cs_row(int D) { return (D + 7) / 8 * 12; }

template <int VEC>
struct Chunk;
template <>
struct Chunk<8> {
  static __device__ __forceinline__ void load(const uint16_t* p, float f[8]) {
    unpack8(ld_stream(reinterpret_cast<const u32x4*>(p)), f);
  }
  // Plain (cached) stores: a head row's two halves are written by two store
  // instructions, and with D/2 not a multiple of 64 elements they share
  // 128-byte lines, which L2 must merge before writing back.
  static __device__ __forceinline__ void store(uint16_t* p, const float f[8]) {
    *reinterpret_cast<u32x4*>(p) = pack8(f);
  }
};
template <>
struct Chunk<2> {
  static __device__ __forceinline__ void load(const uint16_t* p, float f[2]) {
    const uint32_t w = *reinterpret_cast<const uint32_t*>(p);
    f[0] = bf_lo(w);
    f[1] = bf_hi(w);
  }
  static __device__ __forceinline__ void store(uint16_t* p, const float f[2]) {
    *reinterpret_cast<uint32_t*>(p) = pack2(f[0], f[1]);
  }
};

template <>
struct Chunk<1> {
  static __device__ __forceinline__ void load(const uint16_t* p, float f[1]) { f[0] = bf2f(*p); }
  static __device__ __forceinline__ void store(uint16_t* p, const float f[1]) {
    *p = (uint16_t)f2bf(f[0]);
  }
};

// 8 consecutive table values (fp32 or bf16) at element offset off.
template <bool CS32>
__device__ __forceinline__ void load_cs8(const void* base, int64_t off, float f[8]) {
  if constexpr (CS32) {
    const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(base) + off);
    const float4 lo = p[0], hi = p[1];
    f[0] = lo.x; f[1] = lo.y; f[2] = lo.z; f[3] = lo.w;
    f[4] = hi.x; f[5] = hi.y; f[6] = hi.z; f[7] = hi.w;
  } else {
    unpack8(*reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(base) + off), f);
  }
}

template <int MODE, int VEC>
__device__ __forceinline__ void rotate(const float* xl, const float* xh, const float* cl,
                                       const float* ch, const float* sl, const float* sh,
                                       float* ol, float* oh) {
#pragma unroll
  for (int e = 0; e < VEC; ++e) {
    if constexpr (MODE == UMIC_ROPE_TEXT) {
      // the low and high halves' products rounded in pairs
      float cl_p = xl[e] * cl[e], ch_p = xh[e] * ch[e];
      float sl_p = (-xh[e]) * sl[e], sh_p = xl[e] * sh[e];
      rbf2(cl_p, ch_p);
      rbf2(sl_p, sh_p);
      ol[e] = cl_p + sl_p;
      oh[e] = ch_p + sh_p;
    } else {
      ol[e] = xl[e] * cl[e] + (-xh[e]) * sl[e];
      oh[e] = xh[e] * ch[e] + xl[e] * sh[e];
    }
  }
}

template <int MODE, bool CS32, int VEC>
__global__ __launch_bounds__(256) void rope_qk_kernel(RopeArgs a, int ipb, int np_max) {
  // the two staged tables, np_max rows of cs_row(D) floats each (dynamic
  // LDS sized by the host to the rows a block can touch)
  extern __shared__ float tables_l[];
  const int rs = cs_row((int)a.D);
  float* const cs_l = tables_l;
  float* const sn_l = tables_l + np_max * rs;
  const int64_t npos = a.B * a.S;
  const int D = (int)a.D;
  const int half = D / 2;
  const int ipp = a.ipp.d;
  const int nq = (int)a.Hq * a.chunks.d;
  // This block's flat item range [i0, i1) over (position, head, chunk) and
  // the positions [p0, p1] it touches.  Block-level values in 64 bits once;
  // per item only small offsets from (p0, r0) are divided (SmallDiv).
  const int64_t nitems = npos * ipp;
  const int64_t i0 = (int64_t)blockIdx.x * ipb;
  const int nloc = (int)((i0 + ipb < nitems ? i0 + ipb : nitems) - i0);
  const int64_t p0 = i0 / ipp;
  const int r0 = (int)(i0 - p0 * ipp);
  int rlast;
  const int np = div_small(a.ipp, r0 + nloc - 1, rlast) + 1;

  // Stage cos/sin rows of the touched positions (fp32 in LDS; bf16 widens
  // exactly, so TEXT mode still multiplies by the bf16 values).  Run after
  // the first pass's q/k loads are in flight, so both latencies overlap.
  auto stage_tables = [&]() {
    for (int i = threadIdx.x; i < np * D; i += blockDim.x) {
      int d;
      const int pp = div_small(a.dim, i, d);
      const int64_t p = p0 + pp;
      int64_t b = 0, sidx = p;
      if (a.B != 1) {
        b = p / a.S;
        sidx = p - b * a.S;
      }
      const int64_t off = b * a.cs_sb + sidx * a.cs_ss + d;
      const int slot = pp * rs + cs_slot(d);
      if constexpr (CS32) {
        cs_l[slot] = static_cast<const float*>(a.cos)[off];
        sn_l[slot] = static_cast<const float*>(a.sin)[off];
      } else {
        cs_l[slot] = bf2f(static_cast<const uint16_t*>(a.cos)[off]);
        sn_l[slot] = bf2f(static_cast<const uint16_t*>(a.sin)[off]);
      }
    }
  };

  // Each thread takes kItems items per pass; all their loads are issued
  // before any is consumed (an item past the range re-reads item i0, always
  // valid, and stores nothing).
  for (int lbase = 0; lbase < nloc; lbase += kItems * 256) {
    const uint16_t* xs[kItems];
    uint16_t* os[kItems];
    int cofs[kItems], dls[kItems];
    bool ok[kItems];
#pragma unroll
    for (int u = 0; u < kItems; ++u) {
      int l = lbase + u * 256 + (int)threadIdx.x;
      ok[u] = l < nloc;
      if (!ok[u]) l = 0;
      int j;
      const int pp = div_small(a.ipp, r0 + l, j);
      const int64_t p = p0 + pp;
      int64_t b = 0, sidx = p;
      if (a.B != 1) {
        b = p / a.S;
        sidx = p - b * a.S;
      }
      const bool isq = j < nq;
      const int jj = isq ? j : j - nq;
      int c;
      const int h = div_small(a.chunks, jj, c);
      if (isq) {
        xs[u] = a.q + b * a.q_sb + sidx * a.q_ss + h * a.q_sh;
        os[u] = a.qo + b * a.qo_sb + sidx * a.qo_ss + h * a.qo_sh;
      } else {
        xs[u] = a.k + b * a.k_sb + sidx * a.k_ss + h * a.k_sh;
        os[u] = a.ko + b * a.ko_sb + sidx * a.ko_ss + h * a.ko_sh;
      }
      dls[u] = c * VEC;
      cofs[u] = pp * rs;
    }
    float xl[kItems][VEC], xh[kItems][VEC];
#pragma unroll
    for (int u = 0; u < kItems; ++u) {
      Chunk<VEC>::load(xs[u] + dls[u], xl[u]);
      Chunk<VEC>::load(xs[u] + half + dls[u], xh[u]);
    }
    if (lbase == 0) {  // uniform: every thread takes the first pass
      stage_tables();
      __syncthreads();
    }
#pragma unroll
    for (int u = 0; u < kItems; ++u) {
      if (!ok[u]) continue;
      float ol[VEC], oh[VEC];
      const float* cb = cs_l + cofs[u];
      const float* sb = sn_l + cofs[u];
      const int dl = dls[u], dh = half + dls[u];
      const int tl = cs_slot(dl), th = cs_slot(dh);
      rotate<MODE, VEC>(xl[u], xh[u], cb + tl, cb + th, sb + tl, sb + th, ol, oh);
      Chunk<VEC>::store(os[u] + dl, ol);
      Chunk<VEC>::store(os[u] + dh, oh);
    }
  }
}

// Lane-per-chunk form for 16-byte chunks when a head row (D/8 chunks) fits
// a wavefront.  A lane owns ONE contiguous chunk: the low-half chunks of a
// wavefront's hpw head rows sit in lanes 0..31 (row r's chunk c at lane
// r*hh + c, hh = D/16 chunks per half), their high-half partners in the same
// places of lanes 32..63.  Each load and store instruction then covers the
// hpw rows whole -- one contiguous run -- where the head-group and
// item-pair forms above cover the two halves of every row with two instructions, each touching
// twice the cache lines (for D = 80 the halves are 80-byte pieces of
// 160-byte rows).  The rotation partner is lane ^ 32, swapped in by
// v_permlane32_swap (VALU, no LDS).  cos/sin rows of the positions a block
// touches are staged in LDS once per block; a chunk at column 8t reads table
// elements 8t .. 8t + 7 of its position, stored in cs_slot's 12-float chunk
// slots so the chunks of a row one instruction reads sit in distinct banks.
// kLaneItems row groups per wavefront, all loads issued before the staging
// barrier.
constexpr int kLaneItems = 4;

template <int MODE, bool CS32, bool CS_VEC, bool FULL>
__device__ __forceinline__ void lanes_block(const RopeArgs& a, int hpw, int np_max);

// Lanes past the wavefront's hpw rows (lane & 31 >= hpw * hh, e.g. 2 + 2 of
// 64 at D = 80) repeat the last row's chunks: they and their partners load,
// rotate and store exactly what the owning lanes do, so no lane needs a store
// guard; with every row of the block in range (all blocks but the last) the
// block runs without guards.
template <int MODE, bool CS32, bool CS_VEC>
__global__ __launch_bounds__(256) void rope_lanes_kernel(RopeArgs a, int hpw, int np_max) {
  const int64_t nrows = a.B * a.S * a.ipp.d;
  if ((int64_t)(blockIdx.x + 1) * (4 * kLaneItems * hpw) <= nrows)
    lanes_block<MODE, CS32, CS_VEC, true>(a, hpw, np_max);
  else
    lanes_block<MODE, CS32, CS_VEC, false>(a, hpw, np_max);
}

template <int MODE, bool CS32, bool CS_VEC, bool FULL>
__device__ __forceinline__ void lanes_block(const RopeArgs& a, int hpw, int np_max) {
  extern __shared__ float4 tables_v[];  // float4: 16-byte aligned rows
  float* const tables_l = reinterpret_cast<float*>(tables_v);
  const int D = (int)a.D;
  const int rs = cs_row(D);  // a multiple of 12 floats: rows stay 16-byte aligned
  float* const cs_l = tables_l;
  float* const sn_l = tables_l + np_max * rs;
  const int lane = (int)threadIdx.x & (kWave - 1);
  const int wave = (int)threadIdx.x / kWave;
  const bool upper = lane >= 32;
  int tt;
  const int hw_l = div_small(a.chunks, lane & 31, tt);  // row within the group, chunk in half
  const int hw = hw_l < hpw ? hw_l : hpw - 1;           // spare lanes repeat the last row
  const int hh = a.chunks.d;                          // chunks per half row
  const int t = tt + (upper ? hh : 0);                // chunk within the row
  const int hpp = a.ipp.d;                            // head rows per position
  const int64_t npos = a.B * a.S;
  const int64_t nrows = npos * hpp;
  const int rpb = 4 * kLaneItems * hpw;  // head rows per block
  const int64_t b0 = (int64_t)blockIdx.x * rpb;
  const int64_t p0 = b0 / hpp;
  const int r0 = (int)(b0 - p0 * hpp);

  uint16_t* os[kLaneItems];
  u32x4 xv[kLaneItems];
  int tofs[kLaneItems];
  bool ok[kLaneItems];
#pragma unroll
  for (int u = 0; u < kLaneItems; ++u) {
    const int off = (wave * kLaneItems + u) * hpw + hw;
    ok[u] = FULL || b0 + off < nrows;
    int head;
    const int pp = div_small(a.ipp, ok[u] ? r0 + off : r0, head);
    const int64_t p = p0 + pp;
    int64_t b = 0, sidx = p;
    if (a.B != 1) {
      b = p / a.S;
      sidx = p - b * a.S;
    }
    const uint16_t* xs;
    if (head < a.Hq) {
      xs = a.q + b * a.q_sb + sidx * a.q_ss + head * a.q_sh + t * 8;
      os[u] = a.qo + b * a.qo_sb + sidx * a.qo_ss + head * a.qo_sh + t * 8;
    } else {
      const int h = head - (int)a.Hq;
      xs = a.k + b * a.k_sb + sidx * a.k_ss + h * a.k_sh + t * 8;
      os[u] = a.ko + b * a.ko_sb + sidx * a.ko_ss + h * a.ko_sh + t * 8;
    }
    xv[u] = ld_stream(reinterpret_cast<const u32x4*>(xs));
    tofs[u] = pp * rs + cs_slot(t * 8);
  }

  // stage the touched positions' rows (bf16 tables widen exactly)
  const int np = (int)(npos - p0 < np_max ? npos - p0 : np_max);
  if constexpr (CS_VEC) {
    // rows aligned for 4-element moves (fp32: 16 bytes, bf16: 8).  Chunk C (8 floats) of the
    // staged rows sits at slot 12 C, its halves at +0 and +4 floats.  Each
    // 16-lane group writes the same half of 16 consecutive chunks, whose
    // slots 12 C cover the 64 banks once each.
    const int nc = np * (D / 8);
    const int ncp = (nc + 15) & ~15;
    for (int i = (int)threadIdx.x; i < 4 * ncp; i += blockDim.x) {
      const int which = i >= 2 * ncp;
      const int k = which ? i - 2 * ncp : i;
      const int h = (k >> 4) & 1;
      const int C = (k >> 5) * 16 + (k & 15);
      if (C >= nc) continue;
      int d4;
      const int pp = div_small(a.dim, C * 8 + 4 * h, d4);
      const int64_t p = p0 + pp;
      int64_t b = 0, sidx = p;
      if (a.B != 1) {
        b = p / a.S;
        sidx = p - b * a.S;
      }
      const int64_t off = b * a.cs_sb + sidx * a.cs_ss + d4;
      float4 v;
      if constexpr (CS32) {
        v = *reinterpret_cast<const float4*>(static_cast<const float*>(which ? a.sin : a.cos) +
                                             off);
      } else {  // bf16 rows, 8-byte aligned halves, widened exactly
        const u32x2 w = *reinterpret_cast<const u32x2*>(
            static_cast<const uint16_t*>(which ? a.sin : a.cos) + off);
        v = float4{bf_lo(w.x), bf_hi(w.x), bf_lo(w.y), bf_hi(w.y)};
      }
      *reinterpret_cast<float4*>((which ? sn_l : cs_l) + 12 * C + 4 * h) = v;
    }
  } else {
    for (int i = (int)threadIdx.x; i < np * D; i += blockDim.x) {
      int d;
      const int pp = div_small(a.dim, i, d);
      const int64_t p = p0 + pp;
      int64_t b = 0, sidx = p;
      if (a.B != 1) {
        b = p / a.S;
        sidx = p - b * a.S;
      }
      const int64_t off = b * a.cs_sb + sidx * a.cs_ss + d;
      const int slot = pp * rs + cs_slot(d);
      if constexpr (CS32) {
        cs_l[slot] = static_cast<const float*>(a.cos)[off];
        sn_l[slot] = static_cast<const float*>(a.sin)[off];
      } else {
        cs_l[slot] = bf2f(static_cast<const uint16_t*>(a.cos)[off]);
        sn_l[slot] = bf2f(static_cast<const uint16_t*>(a.sin)[off]);
      }
    }
  }
  __syncthreads();

#pragma unroll
  for (int u = 0; u < kLaneItems; ++u) {
    // the partner chunk (lane ^ 32): every lane takes part in the swap
    u32x4 pv;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const auto sw = __builtin_amdgcn_permlane32_swap(xv[u][w], xv[u][w], false, false);
      pv[w] = upper ? sw[0] : sw[1];
    }
    float x[8], xp[8], c[8], sn[8], o[8];
    unpack8(xv[u], x);
    unpack8(pv, xp);
    const float4* cp = reinterpret_cast<const float4*>(cs_l + tofs[u]);
    const float4* sp = reinterpret_cast<const float4*>(sn_l + tofs[u]);
    const float4 c0 = cp[0], c1 = cp[1], s0 = sp[0], s1 = sp[1];
    c[0] = c0.x; c[1] = c0.y; c[2] = c0.z; c[3] = c0.w;
    c[4] = c1.x; c[5] = c1.y; c[6] = c1.z; c[7] = c1.w;
    sn[0] = s0.x; sn[1] = s0.y; sn[2] = s0.z; sn[3] = s0.w;
    sn[4] = s1.x; sn[5] = s1.y; sn[6] = s1.z; sn[7] = s1.w;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float rot = upper ? xp[e] : -xp[e];  // rotate_half: (-x_hi, x_lo)
      if constexpr (MODE == UMIC_ROPE_TEXT) {
        float xc = x[e] * c[e], rs_ = rot * sn[e];
        rbf2(xc, rs_);
        o[e] = xc + rs_;
      }
      else o[e] = x[e] * c[e] + rot * sn[e];
    }
    if (FULL || ok[u]) *reinterpret_cast<u32x4*>(os[u]) = pack8(o);
  }
}

// bf16 tables, 16-byte chunks, read straight from global (see the header):
// head groups.  A thread owns chunk c of R head rows of one kind (q, k; v for
// the cache append) at one position -- the chunk pair [8c, 8c + 8) and
// [D/2 + 8c, +8) of each row -- so the position's cos/sin chunks (and norm
// weights) are loaded once for R rows instead of once per row.  All of a
// thread's loads (4 table chunks, 2 weight chunks, then 2R activation chunks)
// are issued before any arithmetic; row r's arithmetic waits only for the
// tables and its own chunks.
// Consecutive threads walk the chunks, then the head groups (q first), then
// the positions: the chunk lanes of one head row are adjacent and start at a
// multiple of D/16 (the head-row norm's reduction), and at D = 128 one load
// instruction covers whole 128-byte half rows.  R is the largest of 4, 2, 1
// that divides every head count.  Measured at q[1,32,3100,128] +
// k[1,8,...] in one process: plain RoPE 13.2-13.6 us at R = 4 against
// 13.6-14.1 us with one row per thread; with the head-row norm 15.4-16.5
// against 17.1-18.5 us; R = 8 (112 / 136 VGPRs) 14.1 / 17.1-17.9 us.
// The KV append keeps one head row per thread (kKvItems): head groups there,
// for the q rows only or for every kind, measured 16.0-16.4 against
// 15.3-15.9 us plain and 20.3 against 18.5-19.1 us with the norm.
constexpr int kMaxGroupRows = 4;
constexpr int kKvItems = 1;

int group_rows(int64_t Hq, int64_t Hk) {
  for (int r = kMaxGroupRows; r > 1; r /= 2)
    if (Hq % r == 0 && Hk % r == 0) return r;
  return 1;
}

// Thread -> (batch b, position s in the sequence, head group g, chunk c) for
// tpp threads per position; the block's first position is found once, each
// thread's offset from it with small divisions (SmallDiv).
struct GroupItem {
  int64_t b, s;
  int g, c;
};

__device__ __forceinline__ GroupItem group_item(const SmallDiv& tpp, const SmallDiv& chunks,
                                                int64_t B, int64_t S) {
  const int64_t base = (int64_t)blockIdx.x * 256;
  const int64_t pb = base / tpp.d;
  const int rb = (int)(base - pb * tpp.d);
  int j;
  const int64_t p = pb + div_small(tpp, rb + (int)threadIdx.x, j);
  GroupItem it;
  it.b = 0;
  it.s = p;
  if (B != 1) {
    it.b = p / S;
    it.s = p - it.b * S;
  }
  it.g = div_small(chunks, j, it.c);
  return it;
}

// HF Qwen3VLTextRMSNorm of one head row ahead of its rotation (the text
// attention's q_norm / k_norm), in place.  A head row is spread over G = D/16
// consecutive lanes that start at a multiple of G (a row's chunks are
// consecutive threads, and every position's thread count is a multiple of
// G): lane c holds
// the chunks [8c, 8c + 8) (xl) and [D/2 + 8c, +8) (xh); w holds the matching
// weight chunks.  Called with the whole row active (rows are skipped or kept
// as a unit).  The statistic follows torch-ROCm's reduction for
// rows of D = 128 or 256 (aten Reduce.cuh, 4-element vectors, D/4 reducing
// threads of one vector each): thread t sums the squares of elements 4t..4t+3
// in order; the threads combine in adjacent pairs, pairs of pairs, ... --
// here threads 2c, 2c + 1 in-lane, then a butterfly over the G lanes for
// each half row, and last the two halves.  mean = sum * factor (MeanOps:
// float(rows) / float(rows * D)), rstd correctly rounded, then
// bf16(w * bf16(x * rstd)).  G is launch-uniform.
__device__ __forceinline__ float quad_sq(const float* v) {
  return ((v[0] * v[0] + v[1] * v[1]) + v[2] * v[2]) + v[3] * v[3];
}

__device__ __forceinline__ float row_sum_dpp(float v, int G) {
  v += dpp_move<0xB1>(v);                // quad_perm [1,0,3,2]: lane ^ 1
  v += dpp_move<0x4E>(v);                // quad_perm [2,3,0,1]: lane ^ 2
  v += dpp_move<0x141>(v);               // row_half_mirror: the other quad of 8
  if (G >= 16) v += dpp_move<0x140>(v);  // row_mirror: the other 8 of 16
  return v;
}

__device__ __forceinline__ void rms_norm_chunks(float (&xl)[8], float (&xh)[8],
                                                const u32x4 (&w)[2], int G, float factor,
                                                float eps) {
  const float lo = row_sum_dpp(quad_sq(xl) + quad_sq(xl + 4), G);
  const float hi = row_sum_dpp(quad_sq(xh) + quad_sq(xh + 4), G);
  const float rstd = rsqrt_cr((lo + hi) * factor + eps);
  float wl[8], wh[8];
  unpack8(w[0], wl);
  unpack8(w[1], wh);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float l = xl[e] * rstd, h = xh[e] * rstd;
    rbf2(l, h);
    l = wl[e] * l;
    h = wh[e] * h;
    rbf2(l, h);
    xl[e] = l;
    xh[e] = h;
  }
}

// One 16-byte bf16 chunk at element offset off of base.
__device__ __forceinline__ u32x4 ld_chunk(const void* base, int64_t off) {
  return *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(base) + off);
}

// The cos/sin chunks of an item (low and high half of each table) and, for
// the norm kernels, its row's weight chunks.
struct ItemTables {
  u32x4 cs[4];  // cos lo, cos hi, sin lo, sin hi
  u32x4 w[2];   // norm weight lo, hi
};

template <bool NORM>
__device__ __forceinline__ void load_item_tables(ItemTables& t, const void* cos, const void* sin,
                                                 int64_t cso, int dl, int half,
                                                 const uint16_t* w) {
  t.cs[0] = ld_chunk(cos, cso + dl);
  t.cs[1] = ld_chunk(cos, cso + half + dl);
  t.cs[2] = ld_chunk(sin, cso + dl);
  t.cs[3] = ld_chunk(sin, cso + half + dl);
  if constexpr (NORM) {
    t.w[0] = ld_chunk(w, dl);
    t.w[1] = ld_chunk(w, half + dl);
  }
}

// q / k rotation (after the head-row norm when NORM) of R head rows per
// thread; a.chunks = D/16, tpp = (Hq/R + Hk/R) * D/16 threads per position,
// gq = Hq/R q groups, nthreads = B * S * tpp.
template <int MODE, bool NORM, int R>
__global__ __launch_bounds__(256) void rope_qk_direct_kernel(RopeArgs a, SmallDiv tpp, int gq,
                                                             int64_t nthreads) {
  // a head row's chunk lanes leave together (nthreads is a multiple of D/16)
  if ((int64_t)blockIdx.x * 256 + (int64_t)threadIdx.x >= nthreads) return;
  const GroupItem it = group_item(tpp, a.chunks, a.B, a.S);
  const bool isq = it.g < gq;
  const int64_t h0 = (int64_t)(isq ? it.g : it.g - gq) * R;
  const int half = (int)a.D / 2;
  const int dl = it.c * 8;
  const uint16_t* x;
  uint16_t* o;
  int64_t xsh, osh;
  if (isq) {
    x = a.q + it.b * a.q_sb + it.s * a.q_ss + h0 * a.q_sh + dl;
    o = a.qo + it.b * a.qo_sb + it.s * a.qo_ss + h0 * a.qo_sh + dl;
    xsh = a.q_sh;
    osh = a.qo_sh;
  } else {
    x = a.k + it.b * a.k_sb + it.s * a.k_ss + h0 * a.k_sh + dl;
    o = a.ko + it.b * a.ko_sb + it.s * a.ko_ss + h0 * a.ko_sh + dl;
    xsh = a.k_sh;
    osh = a.ko_sh;
  }
  // The tables (L2 hits) first, then the rows in order, and every load
  // issued before the first use: row r's arithmetic then waits only for the
  // tables and its own chunks, and its stores overlap the later rows' loads.
  // (Left to itself the scheduler split the row loads around the first
  // row's arithmetic in one build; with the rows first, every row waited for
  // all loads.)
  ItemTables tb;
  load_item_tables<NORM>(tb, a.cos, a.sin, it.b * a.cs_sb + it.s * a.cs_ss, dl, half,
                         isq ? a.qw : a.kw);
  // held packed until use (8 registers per half chunk instead of 16)
  u32x4 rl[R], rh[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    rl[r] = ld_stream(reinterpret_cast<const u32x4*>(x + r * xsh));
    rh[r] = ld_stream(reinterpret_cast<const u32x4*>(x + r * xsh + half));
  }
  __builtin_amdgcn_sched_barrier(0);
  float cl[8], ch[8], sl[8], sh[8];
  unpack8(tb.cs[0], cl);
  unpack8(tb.cs[1], ch);
  unpack8(tb.cs[2], sl);
  unpack8(tb.cs[3], sh);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    float xl[8], xh[8], ol[8], oh[8];
    unpack8(rl[r], xl);
    unpack8(rh[r], xh);
    if constexpr (NORM)
      rms_norm_chunks(xl, xh, tb.w, a.chunks.d, isq ? a.fq : a.fk, a.eps);
    rotate<MODE, 8>(xl, xh, cl, ch, sl, sh, ol, oh);
    Chunk<8>::store(o + r * osh, ol);
    Chunk<8>::store(o + r * osh + half, oh);
  }
}

// Text RoPE fused with the append into an in-place KV cache.  Per position
// the items are q heads, then k heads, then v heads (16-byte chunk pairs as
// above): q is rotated into q_out, k is rotated straight into the k cache and
// v is moved bit for bit into the v cache, both at cache position P + s,
// P = pos + (*pos_dev if given) -- a device-side P lets one captured graph
// append at a different position on every replay.  Cache stores outside
// [0, cap) are dropped (the host rejects them up front when P is known).
struct KvArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* qo;
  uint16_t* kc;
  uint16_t* vc;
  const uint16_t* cos;
  const uint16_t* sin;
  const int64_t* pos_dev;
  int64_t B, S, Hq, Hk, D;
  int64_t q_sb, q_ss, q_sh, k_sb, k_ss, k_sh, v_sb, v_ss, v_sh;
  int64_t qo_sb, qo_ss, qo_sh;
  int64_t c_sb, c_sh, c_ss, cap, pos;
  int64_t cs_sb, cs_ss;
  SmallDiv ipp, chunks;  // items per position, chunks per half row
  const uint16_t* qw;    // RMSNorm of q / k head rows (norm kernel only)
  const uint16_t* kw;
  float eps;
  float fq, fk;          // MeanOps factors of the q and k head rows
};

template <bool NORM = false>
__global__ __launch_bounds__(256) void rope_kv_append_kernel(KvArgs a) {
  constexpr int VEC = 8;
  const int half = (int)a.D / 2;
  const int nq = (int)a.Hq * a.chunks.d;
  const int nk = (int)a.Hk * a.chunks.d;
  const int ipp = a.ipp.d;  // nq + 2 * nk
  const int64_t nitems = a.B * a.S * ipp;
  const int64_t P = a.pos + (a.pos_dev ? a.pos_dev[0] : 0);
  // block-level decomposition once, per item small divisions (SmallDiv)
  const int64_t base = (int64_t)blockIdx.x * (kKvItems * 256);
  const int64_t pb = base / ipp;
  const int rb = (int)(base - pb * ipp);
  const uint16_t* xs[kKvItems];
  uint16_t* os[kKvItems];
  int64_t cso[kKvItems];
  int dls[kKvItems], kind[kKvItems];  // kind: 0 q, 1 k, 2 v
  bool ok[kKvItems];
#pragma unroll
  for (int u = 0; u < kKvItems; ++u) {
    const int l = u * 256 + (int)threadIdx.x;
    ok[u] = base + l < nitems;
    int j;
    const int pp = div_small(a.ipp, rb + l, j);
    int64_t p = pb + pp;
    if (!ok[u]) p = 0, j = 0;  // re-reads item 0 (always valid) and stores nothing
    int64_t b = 0, sidx = p;
    if (a.B != 1) {
      b = p / a.S;
      sidx = p - b * a.S;
    }
    kind[u] = j < nq ? 0 : j < nq + nk ? 1 : 2;
    const int jj = kind[u] == 0 ? j : kind[u] == 1 ? j - nq : j - nq - nk;
    int c;
    const int h = div_small(a.chunks, jj, c);
    const int64_t t = P + sidx;  // cache position of k / v
    if (kind[u] == 0) {
      xs[u] = a.q + b * a.q_sb + sidx * a.q_ss + h * a.q_sh;
      os[u] = a.qo + b * a.qo_sb + sidx * a.qo_ss + h * a.qo_sh;
    } else {
      ok[u] = ok[u] && t >= 0 && t < a.cap;
      const int64_t co = b * a.c_sb + h * a.c_sh + t * a.c_ss;
      if (kind[u] == 1) {
        xs[u] = a.k + b * a.k_sb + sidx * a.k_ss + h * a.k_sh;
        os[u] = a.kc + co;
      } else {
        xs[u] = a.v + b * a.v_sb + sidx * a.v_ss + h * a.v_sh;
        os[u] = a.vc + co;
      }
    }
    dls[u] = c * VEC;
    cso[u] = b * a.cs_sb + sidx * a.cs_ss;
  }
  u32x4 rl[kKvItems], rh[kKvItems];
  ItemTables tb[kKvItems];
#pragma unroll
  for (int u = 0; u < kKvItems; ++u) {
    rl[u] = ld_stream(reinterpret_cast<const u32x4*>(xs[u] + dls[u]));
    rh[u] = ld_stream(reinterpret_cast<const u32x4*>(xs[u] + half + dls[u]));
  }
#pragma unroll
  for (int u = 0; u < kKvItems; ++u)  // v items load (unused) tables too: no branch
    load_item_tables<NORM>(tb[u], a.cos, a.sin, cso[u], dls[u], half,
                           kind[u] == 0 ? a.qw : a.kw);
  // every load issued before the first use: without the fence the paired
  // roundings' schedule moved a table load behind the first wait (prefill
  // append 17.6-18.6 against 15.4-16.1 us)
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int u = 0; u < kKvItems; ++u) {
    if (!ok[u]) continue;
    u32x4* lo = reinterpret_cast<u32x4*>(os[u] + dls[u]);
    u32x4* hi = reinterpret_cast<u32x4*>(os[u] + half + dls[u]);
    if (kind[u] == 2) {
      *lo = rl[u];
      *hi = rh[u];
      continue;
    }
    float xl[VEC], xh[VEC], cl[VEC], ch[VEC], sl[VEC], sh[VEC], ol[VEC], oh[VEC];
    unpack8(rl[u], xl);
    unpack8(rh[u], xh);
    if constexpr (NORM)
      rms_norm_chunks(xl, xh, tb[u].w, a.chunks.d, kind[u] == 0 ? a.fq : a.fk, a.eps);
    unpack8(tb[u].cs[0], cl);
    unpack8(tb[u].cs[1], ch);
    unpack8(tb[u].cs[2], sl);
    unpack8(tb[u].cs[3], sh);
    rotate<UMIC_ROPE_TEXT, VEC>(xl, xh, cl, ch, sl, sh, ol, oh);
    *lo = pack8(ol);
    *hi = pack8(oh);
  }
}

// The launch-uniform divisors for vector width VEC.
template <int VEC>
RopeArgs with_divisors(const RopeArgs& a) {
  RopeArgs b = a;
  b.chunks = small_div((int)(a.D / 2 / VEC));
  b.ipp = small_div((int)((a.Hq + a.Hk) * (a.D / 2 / VEC)));
  b.dim = small_div((int)a.D);
  return b;
}

// LDS budget of the lane-per-chunk form's two staged tables
constexpr size_t kLanesMaxLds = 48 * 1024;

// The lane-per-chunk form (16-byte chunks, a head row within a wavefront),
// or UMIC_ERR_UNSUPPORTED when it does not apply.
template <int MODE, bool CS32>
int launch_lanes(const RopeArgs& a0, hipStream_t st) {
  const int64_t hh = a0.D / 16;  // chunks per half row
  if (a0.D % 16 != 0 || hh > 32) return UMIC_ERR_UNSUPPORTED;
  RopeArgs a = a0;
  a.chunks = small_div((int)hh);
  a.ipp = small_div((int)(a.Hq + a.Hk));
  a.dim = small_div((int)a.D);
  const int64_t npos = a.B * a.S;
  const int64_t hpp = a.Hq + a.Hk;
  const int hpw = (int)(32 / hh);  // head rows per wavefront
  const int64_t rpb = (int64_t)4 * kLaneItems * hpw;
  // a block's rpb head rows touch at most rpb / hpp + 2 positions
  const int64_t np_max = std::min<int64_t>(rpb / hpp + 2, npos);
  const size_t lds = (size_t)(2 * np_max * cs_row((int)a.D)) * sizeof(float);
  if (lds > kLanesMaxLds) return UMIC_ERR_UNSUPPORTED;
  const int64_t blocks = (npos * hpp + rpb - 1) / rpb;
  if (blocks > 0x7fffffffLL) return UMIC_ERR_UNSUPPORTED;
  const uintptr_t cs_align = CS32 ? 16 : 8;
  const bool cs_vec = a.cs_sb % 4 == 0 && a.cs_ss % 4 == 0 &&
                      (uintptr_t)a.cos % cs_align == 0 && (uintptr_t)a.sin % cs_align == 0;
  if (cs_vec)
    hipLaunchKernelGGL((rope_lanes_kernel<MODE, CS32, true>), dim3((unsigned)blocks), dim3(256),
                       lds, st, a, hpw, (int)np_max);
  else
    hipLaunchKernelGGL((rope_lanes_kernel<MODE, CS32, false>), dim3((unsigned)blocks),
                       dim3(256), lds, st, a, hpw, (int)np_max);
  return launch_status();
}

template <int MODE, bool CS32, int VEC>
int launch_staged(const RopeArgs& a0, hipStream_t st) {
  if constexpr (VEC == 8) {
    const int rc = launch_lanes<MODE, CS32>(a0, st);
    if (rc != UMIC_ERR_UNSUPPORTED) return rc;
  }
  const RopeArgs a = with_divisors<VEC>(a0);
  const int64_t npos = a.B * a.S;
  const int64_t ipp = (a.Hq + a.Hk) * (a.D / 2 / VEC);
  // kItems items per thread in one pass; the positions a range touches
  // (at most ipb / ipp + 2) must fit the LDS tables.
  int64_t ipb = kItems * 256;
  const int64_t rs = cs_row((int)a.D);
  const int64_t max_pos = kMaxCsFloats / rs;
  if (ipb / ipp + 2 > max_pos) ipb = (max_pos - 2) * ipp;
  if (ipb < 1) return UMIC_ERR_UNSUPPORTED;
  const int64_t blocks = (npos * ipp + ipb - 1) / ipb;
  if (blocks > 0x7fffffffLL) return UMIC_ERR_UNSUPPORTED;
  // a range of ipb items touches at most ipb / ipp + 2 positions
  const int64_t np_max = std::min<int64_t>(ipb / ipp + 2, npos);
  const size_t lds = (size_t)(2 * np_max * rs) * sizeof(float);
  hipLaunchKernelGGL((rope_qk_kernel<MODE, CS32, VEC>), dim3((unsigned)blocks), dim3(256), lds,
                     st, a, (int)ipb, (int)np_max);
  return launch_status();
}

// The head-group kernel for R rows per thread; a carries its divisors.
template <int MODE, bool NORM, int R>
int launch_direct_r(const RopeArgs& a, hipStream_t st) {
  const int gq = (int)(a.Hq / R), gk = (int)(a.Hk / R);
  const SmallDiv tpp = small_div((gq + gk) * a.chunks.d);
  const int64_t nthreads = a.B * a.S * tpp.d;
  const int64_t blocks = (nthreads + 255) / 256;
  if (blocks > 0x7fffffffLL) return UMIC_ERR_UNSUPPORTED;
  hipLaunchKernelGGL((rope_qk_direct_kernel<MODE, NORM, R>), dim3((unsigned)blocks), dim3(256),
                     0, st, a, tpp, gq, nthreads);
  return launch_status();
}

// Few positions (decode steps: one position, 40 head rows) take one row per
// thread: the launch is a latency chain, and R rows per thread put R rows'
// arithmetic (the norm's reduction and rsqrt) in series on one lane.
constexpr int64_t kDirectGroupMinThreads = 256 * 256;

template <int MODE, bool NORM>
int launch_direct(const RopeArgs& a, hipStream_t st) {
  if (a.B * a.S * (a.Hq + a.Hk) * a.chunks.d <= kDirectGroupMinThreads)
    return launch_direct_r<MODE, NORM, 1>(a, st);
  switch (group_rows(a.Hq, a.Hk)) {
    case 4: return launch_direct_r<MODE, NORM, 4>(a, st);
    case 2: return launch_direct_r<MODE, NORM, 2>(a, st);
    default: return launch_direct_r<MODE, NORM, 1>(a, st);
  }
}

// direct_ok: the bf16 tables allow 16-byte reads (aligned bases, row
// strides multiples of 8 elements); otherwise they are staged.  The
// head-group and item-pair forms are kept for head dims whose half rows are whole 128-byte
// lines (D a multiple of 128); any other D with 16-byte chunks takes the
// lane-chunk form (at D = 80 with bf16 tables 33-37 against 38-41 us, at
// text D = 64 9.5 against 14.4-15.3 us).
template <int MODE, bool CS32, int VEC>
int launch_rope(const RopeArgs& a, bool direct_ok, hipStream_t st) {
  if constexpr (VEC == 8) {
    if (a.D % 128 != 0) {
      const int rc = launch_lanes<MODE, CS32>(a, st);
      if (rc != UMIC_ERR_UNSUPPORTED) return rc;
    }
  }
  if constexpr (!CS32 && VEC == 8) {
    if (!direct_ok) return launch_staged<MODE, CS32, VEC>(a, st);
    return launch_direct<MODE, false>(with_divisors<VEC>(a), st);
  } else {
    return launch_staged<MODE, CS32, VEC>(a, st);
  }
}

template <int MODE, bool CS32>
int dispatch_vec(const RopeArgs& a, int vec, bool direct_ok, hipStream_t st) {
  if (vec == 8) return launch_rope<MODE, CS32, 8>(a, direct_ok, st);
  if (vec == 2) return launch_staged<MODE, CS32, 2>(a, st);
  return launch_staged<MODE, CS32, 1>(a, st);
}

}  // namespace
}  // namespace umic

using namespace umic;

extern "C" int umic_rope_qk_bf16(const void* q, const void* k, void* q_out, void* k_out,
                                 const void* cos, const void* sin, int cs_fp32, int mode,
                                 int64_t B, int64_t S, int64_t Hq, int64_t Hk, int64_t D,
                                 int64_t q_sb, int64_t q_ss, int64_t q_sh, int64_t k_sb,
                                 int64_t k_ss, int64_t k_sh, int64_t qo_sb, int64_t qo_ss,
                                 int64_t qo_sh, int64_t ko_sb, int64_t ko_ss, int64_t ko_sh,
                                 int64_t cs_sb, int64_t cs_ss, void* stream) {
  if (mode != UMIC_ROPE_TEXT && mode != UMIC_ROPE_VISION) return UMIC_ERR_INVALID_ARG;
  if (B < 0 || S < 0 || Hq < 0 || Hk < 0 || D <= 0) return UMIC_ERR_INVALID_ARG;
  if (mode == UMIC_ROPE_TEXT && cs_fp32) return UMIC_ERR_UNSUPPORTED;
  if (D % 2 != 0 || D > kMaxHeadDim) return UMIC_ERR_UNSUPPORTED;
  if ((Hq + Hk) * (D / 2) >= kMaxItemsPerPos) return UMIC_ERR_UNSUPPORTED;
  if (B * S == 0 || Hq + Hk == 0) return UMIC_OK;  // empty: pointers may be null
  if (!cos || !sin) return UMIC_ERR_INVALID_ARG;
  if (Hq > 0 && (!q || !q_out)) return UMIC_ERR_INVALID_ARG;
  if (Hk > 0 && (!k || !k_out)) return UMIC_ERR_INVALID_ARG;

  RopeArgs a{(const uint16_t*)q, (const uint16_t*)k, (uint16_t*)q_out, (uint16_t*)k_out,
             cos, sin, B, S, Hq, Hk, D,
             q_sb, q_ss, q_sh, k_sb, k_ss, k_sh,
             qo_sb, qo_ss, qo_sh, ko_sb, ko_ss, ko_sh, cs_sb, cs_ss};
  if (Hq == 0) a.q = a.qo = nullptr;
  if (Hk == 0) a.k = a.ko = nullptr;

  // 16-byte chunks need 8 | D/2, every stride a multiple of 8 and 16-byte
  // aligned bases; 4-byte pairs the same with 2; single elements always work.
  auto all_mult = [&](int64_t m) {
    bool ok = (D / 2) % m == 0;
    if (Hq) ok = ok && q_sb % m == 0 && q_ss % m == 0 && q_sh % m == 0 && qo_sb % m == 0 &&
                 qo_ss % m == 0 && qo_sh % m == 0;
    if (Hk) ok = ok && k_sb % m == 0 && k_ss % m == 0 && k_sh % m == 0 && ko_sb % m == 0 &&
                 ko_ss % m == 0 && ko_sh % m == 0;
    return ok;
  };
  auto all_aligned = [&](uintptr_t m) {
    bool ok = true;
    if (Hq) ok = ok && ((uintptr_t)q % m == 0) && ((uintptr_t)q_out % m == 0);
    if (Hk) ok = ok && ((uintptr_t)k % m == 0) && ((uintptr_t)k_out % m == 0);
    return ok;
  };
  const int vec = (all_mult(8) && all_aligned(16)) ? 8 : (all_mult(2) && all_aligned(4)) ? 2 : 1;
  if (vec == 1 && !all_aligned(2)) return UMIC_ERR_UNSUPPORTED;

  const bool direct_ok = cs_sb % 8 == 0 && cs_ss % 8 == 0 && (uintptr_t)cos % 16 == 0 &&
                         (uintptr_t)sin % 16 == 0;
  hipStream_t st = as_stream(stream);
  if (mode == UMIC_ROPE_TEXT) return dispatch_vec<UMIC_ROPE_TEXT, false>(a, vec, direct_ok, st);
  if (cs_fp32) return dispatch_vec<UMIC_ROPE_VISION, true>(a, vec, direct_ok, st);
  return dispatch_vec<UMIC_ROPE_VISION, false>(a, vec, direct_ok, st);
}

namespace umic {
namespace {

// head_dim values the fused RMSNorm takes: D = 128 or 256, whose eager
// reduction (one 4-element vector per reducing thread, whatever the row
// count) rms_norm_chunks reproduces; other head sizes normalise with
// umic_rmsnorm_bf16 first.
bool norm_dim_ok(int64_t D) { return D == 128 || D == 256; }

// aten MeanOps factor of `rows` head rows of D: float(rows) / float(rows * D)
float mean_factor(int64_t rows, int64_t D) {
  return rows > 0 ? (float)rows / (float)(rows * D) : 0.0f;
}

// The in-place cache append, optionally with the q / k RMSNorm (qw, kw
// non-null).  Shared by umic_rope_kv_append_bf16 and its norm variant.
int kv_append_impl(const void* q, const void* k, const void* v, void* q_out, void* k_cache,
                   void* v_cache, const void* cos, const void* sin, const void* qw,
                   const void* kw, float eps, bool norm, int64_t B, int64_t S, int64_t Hq,
                   int64_t Hk, int64_t D, int64_t q_sb, int64_t q_ss, int64_t q_sh,
                   int64_t k_sb, int64_t k_ss, int64_t k_sh, int64_t v_sb, int64_t v_ss,
                   int64_t v_sh, int64_t qo_sb, int64_t qo_ss, int64_t qo_sh, int64_t c_sb,
                   int64_t c_sh, int64_t c_ss, int64_t capacity, int64_t pos,
                   const int64_t* pos_dev, int64_t cs_sb, int64_t cs_ss, void* stream) {
  if (B < 0 || S < 0 || Hq < 0 || Hk < 0 || D <= 0 || capacity < 0) return UMIC_ERR_INVALID_ARG;
  // a known write position must fit the cache (the reference raises on overflow)
  if (!pos_dev && (pos < 0 || pos + S > capacity)) return UMIC_ERR_INVALID_ARG;
  if (D % 16 != 0) return UMIC_ERR_UNSUPPORTED;  // 16-byte chunks of each half row
  if ((Hq + 2 * Hk) * (D / 16) >= kMaxItemsPerPos) return UMIC_ERR_UNSUPPORTED;
  if (B * S == 0 || Hq + Hk == 0) return UMIC_OK;
  if (!cos || !sin) return UMIC_ERR_INVALID_ARG;
  if (Hq > 0 && (!q || !q_out)) return UMIC_ERR_INVALID_ARG;
  if (Hk > 0 && (!k || !v || !k_cache || !v_cache)) return UMIC_ERR_INVALID_ARG;
  if (norm) {
    if ((Hq > 0 && !qw) || (Hk > 0 && !kw)) return UMIC_ERR_INVALID_ARG;
    if (!norm_dim_ok(D) || (qw && (uintptr_t)qw % 16) || (kw && (uintptr_t)kw % 16))
      return UMIC_ERR_UNSUPPORTED;
  }

  KvArgs a{(const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v, (uint16_t*)q_out,
           (uint16_t*)k_cache, (uint16_t*)v_cache, (const uint16_t*)cos, (const uint16_t*)sin,
           pos_dev, B, S, Hq, Hk, D, q_sb, q_ss, q_sh, k_sb, k_ss, k_sh, v_sb, v_ss, v_sh,
           qo_sb, qo_ss, qo_sh, c_sb, c_sh, c_ss, capacity, pos, cs_sb, cs_ss,
           small_div((int)((Hq + 2 * Hk) * (D / 16))), small_div((int)(D / 16)),
           (const uint16_t*)qw, (const uint16_t*)kw, eps, mean_factor(B * S * Hq, D),
           mean_factor(B * S * Hk, D)};
  bool ok = cs_sb % 8 == 0 && cs_ss % 8 == 0 && (uintptr_t)cos % 16 == 0 &&
            (uintptr_t)sin % 16 == 0;
  if (Hq) {
    ok = ok && q_sb % 8 == 0 && q_ss % 8 == 0 && q_sh % 8 == 0 && qo_sb % 8 == 0 &&
         qo_ss % 8 == 0 && qo_sh % 8 == 0 && (uintptr_t)q % 16 == 0 && (uintptr_t)q_out % 16 == 0;
  } else {
    a.q = a.qo = nullptr;
  }
  if (Hk) {
    ok = ok && k_sb % 8 == 0 && k_ss % 8 == 0 && k_sh % 8 == 0 && v_sb % 8 == 0 &&
         v_ss % 8 == 0 && v_sh % 8 == 0 && c_sb % 8 == 0 && c_sh % 8 == 0 && c_ss % 8 == 0 &&
         (uintptr_t)k % 16 == 0 && (uintptr_t)v % 16 == 0 && (uintptr_t)k_cache % 16 == 0 &&
         (uintptr_t)v_cache % 16 == 0;
  } else {
    a.k = a.v = nullptr;
    a.kc = a.vc = nullptr;
  }
  if (!ok) return UMIC_ERR_UNSUPPORTED;
  const int64_t nitems = B * S * (Hq + 2 * Hk) * (D / 16);
  const int64_t blocks = (nitems + kKvItems * 256 - 1) / (kKvItems * 256);
  if (blocks > 0x7fffffffLL) return UMIC_ERR_UNSUPPORTED;
  if (norm)
    hipLaunchKernelGGL(rope_kv_append_kernel<true>, dim3((unsigned)blocks), dim3(256), 0,
                       as_stream(stream), a);
  else
    hipLaunchKernelGGL(rope_kv_append_kernel<false>, dim3((unsigned)blocks), dim3(256), 0,
                       as_stream(stream), a);
  return launch_status();
}

}  // namespace
}  // namespace umic

extern "C" int umic_rope_kv_append_bf16(
    const void* q, const void* k, const void* v, void* q_out, void* k_cache, void* v_cache,
    const void* cos, const void* sin, int64_t B, int64_t S, int64_t Hq, int64_t Hk, int64_t D,
    int64_t q_sb, int64_t q_ss, int64_t q_sh, int64_t k_sb, int64_t k_ss, int64_t k_sh,
    int64_t v_sb, int64_t v_ss, int64_t v_sh, int64_t qo_sb, int64_t qo_ss, int64_t qo_sh,
    int64_t c_sb, int64_t c_sh, int64_t c_ss, int64_t capacity, int64_t pos,
    const int64_t* pos_dev, int64_t cs_sb, int64_t cs_ss, void* stream) {
  return kv_append_impl(q, k, v, q_out, k_cache, v_cache, cos, sin, nullptr, nullptr, 0.f,
                        false, B, S, Hq, Hk, D, q_sb, q_ss, q_sh, k_sb, k_ss, k_sh, v_sb, v_ss,
                        v_sh, qo_sb, qo_ss, qo_sh, c_sb, c_sh, c_ss, capacity, pos, pos_dev,
                        cs_sb, cs_ss, stream);
}

extern "C" int umic_qk_rmsnorm_rope_kv_append_bf16(
    const void* q, const void* k, const void* v, void* q_out, void* k_cache, void* v_cache,
    const void* cos, const void* sin, const void* q_w, const void* k_w, float eps, int64_t B,
    int64_t S, int64_t Hq, int64_t Hk, int64_t D, int64_t q_sb, int64_t q_ss, int64_t q_sh,
    int64_t k_sb, int64_t k_ss, int64_t k_sh, int64_t v_sb, int64_t v_ss, int64_t v_sh,
    int64_t qo_sb, int64_t qo_ss, int64_t qo_sh, int64_t c_sb, int64_t c_sh, int64_t c_ss,
    int64_t capacity, int64_t pos, const int64_t* pos_dev, int64_t cs_sb, int64_t cs_ss,
    void* stream) {
  return kv_append_impl(q, k, v, q_out, k_cache, v_cache, cos, sin, q_w, k_w, eps, true, B, S,
                        Hq, Hk, D, q_sb, q_ss, q_sh, k_sb, k_ss, k_sh, v_sb, v_ss, v_sh, qo_sb,
                        qo_ss, qo_sh, c_sb, c_sh, c_ss, capacity, pos, pos_dev, cs_sb, cs_ss,
                        stream);
}

extern "C" int umic_qk_rmsnorm_rope_bf16(const void* q, const void* k, void* q_out, void* k_out,
                                        const void* q_w, const void* k_w, float eps,
                                        const void* cos, const void* sin, int64_t B, int64_t S,
                                        int64_t Hq, int64_t Hk, int64_t D, int64_t q_sb,
                                        int64_t q_ss, int64_t q_sh, int64_t k_sb, int64_t k_ss,
                                        int64_t k_sh, int64_t qo_sb, int64_t qo_ss,
                                        int64_t qo_sh, int64_t ko_sb, int64_t ko_ss,
                                        int64_t ko_sh, int64_t cs_sb, int64_t cs_ss,
                                        void* stream) {
  if (B < 0 || S < 0 || Hq < 0 || Hk < 0 || D <= 0) return UMIC_ERR_INVALID_ARG;
  if (!norm_dim_ok(D)) return UMIC_ERR_UNSUPPORTED;
  if ((Hq + Hk) * (D / 2) >= kMaxItemsPerPos) return UMIC_ERR_UNSUPPORTED;
  if (B * S == 0 || Hq + Hk == 0) return UMIC_OK;  // empty: pointers may be null
  if (!cos || !sin) return UMIC_ERR_INVALID_ARG;
  if (Hq > 0 && (!q || !q_out || !q_w)) return UMIC_ERR_INVALID_ARG;
  if (Hk > 0 && (!k || !k_out || !k_w)) return UMIC_ERR_INVALID_ARG;
  // the direct text kernel only: 16-byte chunks everywhere
  bool ok = cs_sb % 8 == 0 && cs_ss % 8 == 0 && (uintptr_t)cos % 16 == 0 &&
            (uintptr_t)sin % 16 == 0;
  if (Hq)
    ok = ok && q_sb % 8 == 0 && q_ss % 8 == 0 && q_sh % 8 == 0 && qo_sb % 8 == 0 &&
         qo_ss % 8 == 0 && qo_sh % 8 == 0 && (uintptr_t)q % 16 == 0 &&
         (uintptr_t)q_out % 16 == 0 && (uintptr_t)q_w % 16 == 0;
  if (Hk)
    ok = ok && k_sb % 8 == 0 && k_ss % 8 == 0 && k_sh % 8 == 0 && ko_sb % 8 == 0 &&
         ko_ss % 8 == 0 && ko_sh % 8 == 0 && (uintptr_t)k % 16 == 0 &&
         (uintptr_t)k_out % 16 == 0 && (uintptr_t)k_w % 16 == 0;
  if (!ok) return UMIC_ERR_UNSUPPORTED;
  RopeArgs a{(const uint16_t*)q, (const uint16_t*)k, (uint16_t*)q_out, (uint16_t*)k_out,
             cos, sin, B, S, Hq, Hk, D,
             q_sb, q_ss, q_sh, k_sb, k_ss, k_sh,
             qo_sb, qo_ss, qo_sh, ko_sb, ko_ss, ko_sh, cs_sb, cs_ss};
  if (Hq == 0) a.q = a.qo = nullptr;
  if (Hk == 0) a.k = a.ko = nullptr;
  a = with_divisors<8>(a);
  a.qw = (const uint16_t*)q_w;
  a.kw = (const uint16_t*)k_w;
  a.eps = eps;
  a.fq = mean_factor(B * S * Hq, D);
  a.fk = mean_factor(B * S * Hk, D);
  return launch_direct<UMIC_ROPE_TEXT, true>(a, as_stream(stream));
}
