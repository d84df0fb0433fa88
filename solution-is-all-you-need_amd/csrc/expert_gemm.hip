// expert_gemm.hip -- grouped int4 (Q4_0) expert SwiGLU FFN for gfx950,
// prefill regime: each expert segment is dense enough (tens to hundreds of
// tokens) to be a real GEMM, so the work runs on the matrix cores.
//
// Reference operator: kernels/sparse_moe/sparse_matmul.cu:120-215 and its
// dense branch (:322-365, cuBLAS GEMMs for gate/up and down, SwiGLU between),
// with the expert weights of python/phantom/loader/gguf_loader.py:362-381.
//
// Operands are exact, as in the decode regime, and fp16 for
// v_mfma_f32_16x16x32_f16, so the products are exact and only the fp32
// accumulation rounds:
//   A  gate/up: x rounded bf16 -> fp16 by the router's prep (exact for
//      2^-17 <= |x| < 65504, the fp16 range a bf16 value fits); down: h as
//      the fp16 pair hi + lo written by the gate/up epilogue.
//   B  the weight q * d with q = n - 8 and the fp16 scale split d = dh + dl,
//      dh = d with its 3 low mantissa bits cleared: q has at most 3
//      significant bits, so q * dh (<= 11 bits) and q * dl (<= 6 bits) are
//      both exact fp16 values (for normal d and |q d| < 65504).  The nibble
//      becomes the fp16 value 1024 + n (one v_and_or_b32 per pair), one
//      v_pk_add_f16 gives q, two v_pk_mul_f16 give the two operands.
// gate/up: acc += A.Bh + A.Bl (2 MFMAs per group, chained in the
// accumulators).  down: acc += hi.Bh + hi.Bl + lo.Bh (3 MFMAs; lo.Bl is below
// 2^-20 of the product and dropped).  The scale lives inside the operands, so
// there is no per-group vector-ALU work on the accumulators.
//
// Two tile pipelines share these tiles and this arithmetic.  The default,
// gemm_tile3 (gemm_*_kernel2, 8 waves), stages both operands into a 3-stage
// LDS ring with direct-to-LDS loads two quads ahead; gemm_tile (4 waves,
// PHANTOM_MOE_GEMM_KERNEL=v1) stages A through registers one quad ahead.
//
// Tiling.  A workgroup of kGemmWaves waves owns BM consecutive positions of
// one expert segment and a block of weight rows.  Per K quad (128), the
// positions' A rows are staged in LDS (double-buffered; 16-byte units XOR-
// swizzled by row so the ds_read_b128 of 16 rows hit distinct banks) and every
// wave multiplies them with NB weight row tiles of its own, dequantised
// from its own 128-bit loads (the repacked layout hands each lane exactly its
// B operand).  Each B operand feeds BM / 16 MFMAs.
//   gate/up (BM 128): wave w takes one 32-row group of I (two 16-row tiles)
//            for both gate and up (4 B operands), so its SwiGLU epilogue
//            produces whole down-operand chunks (hi + lo, written via LDS).
//   down (BM 64): wave w takes two 16-row tiles of H.
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "expert_common.h"
#include "moe_common.h"
#include "moe_launch.h"

namespace pmoe {

constexpr int kGemmWaves = 4;
constexpr int kGemmNBGateUp = 2;               // B operands per wave: gate and up of one 16-row tile
constexpr int kGemmNBDown = 2;                 // B operands per wave: two 16-row tiles of H
constexpr int kGemmBMGateUp = 128;             // segment positions per gate/up tile
constexpr int kGemmBMDown = 64;                // segment positions per down tile
constexpr int kGemmRowsGU = kGemmWaves * 16;   // rows of I per gate/up workgroup (two groups)
constexpr int kGemmRowsDown = kGemmWaves * 32; // rows of H per down workgroup
constexpr bool kGemmSplitGateUp = true;        // split-scale operands (else fp32 scaling)
constexpr bool kGemmSplitDown = true;
// LDS bytes of the double-buffered A tile: BM rows x 16 chunks x AW x 16 B
constexpr int kGemmLdsA = 2 * kGemmBMGateUp * 16 * 16;
static_assert(kGemmLdsA == 2 * kGemmBMDown * 32 * 16, "both tiles use the same LDS");

struct GemmK {
  SegSrc seg;
  const uint16_t* a_src;  // fp16 rows [rows][Kq][16 chunks][AW x 8] in MFMA operand order
  int64_t a_zero_row;     // an all-zero row of a_src
  int a_by_token;         // 1: A row = token of the position (x); 0: A row = position (h)
  int64_t Kq;             // quads of K
  int64_t Kg;             // real 32-groups of K (padded groups of a_src are ignored)
  int64_t N;              // rows of the weight matrices (I for gate/up, H for down)
  // weights: [E][N/16][Kq][1 KiB] nibbles, [E][N/16][Kq][64] fp16 scales;
  // w1 = gate (or down), w2 = up (gate/up only); sh_* the shared expert's
  const uint8_t* nib1;
  const uint16_t* sc1;
  const uint8_t* nib2;
  const uint16_t* sc2;
  const uint8_t* sh_nib1;
  const uint16_t* sh_sc1;
  const uint8_t* sh_nib2;
  const uint16_t* sh_sc2;
  // gate/up output: h as fp16 hi + lo [rows + 1][KqI][16 chunks][hi 8, lo 8],
  // the decode regime's down operand (its half-group sums are not written)
  uint16_t* hq16;
  int64_t KqI;
  int64_t h_zero_row;
  // down output: fp32 [rows][H]
  float* outbuf;
};

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));

// B operand of one 32-group: the lane's four nibble bytes w (bytes 4p..4p+3 of
// the group's qs for its row) -> the eight fp16 integers n - 8 in kmap order.
__device__ inline u32x4 dequant_int_f16(uint32_t w, uint32_t mask) {
  const h2_t off = {(_Float16)1032.0f, (_Float16)1032.0f};
  const uint32_t r[4] = {and_or(w, mask, 0x64006400u), and_or(w >> 4, mask, 0x64006400u),
                         and_or(w >> 8, mask, 0x64006400u), and_or(w >> 12, mask, 0x64006400u)};
  u32x4 out;
#pragma unroll
  for (int i = 0; i < 4; ++i) out[i] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2_t, r[i]) - off);
  return out;
}

// B operands of one 32-group: the lane's four nibble bytes w (bytes 4p..4p+3
// of the group's qs for its row) and the group's fp16 scale bits d -> the
// eight q * dh and the eight q * dl, fp16, in kmap order.
__device__ inline void dequant_split_f16(uint32_t w, uint32_t d, uint32_t mask, u32x4& bh, u32x4& bl) {
  const h2_t off = {(_Float16)1032.0f, (_Float16)1032.0f};
  const uint32_t dh = d & 0xFFF8u;
  const _Float16 dlv = __builtin_bit_cast(_Float16, (uint16_t)d) - __builtin_bit_cast(_Float16, (uint16_t)dh);
  const h2_t dh2 = __builtin_bit_cast(h2_t, dh | (dh << 16));
  const h2_t dl2 = {dlv, dlv};
  const uint32_t r[4] = {and_or(w, mask, 0x64006400u), and_or(w >> 4, mask, 0x64006400u),
                         and_or(w >> 8, mask, 0x64006400u), and_or(w >> 12, mask, 0x64006400u)};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const h2_t q = __builtin_bit_cast(h2_t, r[i]) - off;  // n - 8, exact
    bh[i] = __builtin_bit_cast(uint32_t, q * dh2);       // exact
    bl[i] = __builtin_bit_cast(uint32_t, q * dl2);       // exact
  }
}

// SwiGLU of one output, silu(g) * u, from the hardware exp2 and reciprocal
// (v_exp_f32, v_rcp_f32; about 1 ulp each, against some 35 instructions for
// expf and an IEEE division): the relative difference is ~1e-7.
__device__ inline float swiglu_fast(float g, float u) {
  const float e = __builtin_amdgcn_exp2f(-g * 1.44269504088896341f);
  return g * __builtin_amdgcn_rcpf(1.0f + e) * u;
}

// Item space: for each active segment u, ceil(len_u / BM) position blocks
// times n_nb row blocks.  s_mb[u] = first position block of segment u (an
// exclusive prefix over segments, computed by wave 0).
template <int BM>
__device__ inline int64_t plan_items(const int4* s_desc, int n_act, int* s_mb) {
  if (threadIdx.x < kWave) {
    const int lane = threadIdx.x;
    int carry = 0;
    for (int u0 = 0; u0 < n_act; u0 += kWave) {
      const int u = u0 + lane;
      const int len = u < n_act ? s_desc[u].z - s_desc[u].y : 0;
      const int v = (len + BM - 1) / BM;
      int inc = v;
#pragma unroll
      for (int off = 1; off < kWave; off <<= 1) {
        const int t = __shfl_up(inc, off, kWave);
        if (lane >= off) inc += t;
      }
      if (u < n_act) s_mb[u] = carry + inc - v;
      carry += __shfl(inc, kWave - 1, kWave);
    }
    if (lane == 0) s_mb[n_act] = carry;
  }
  __syncthreads();
  return s_mb[n_act];
}

// Segment holding position block mb: the last u with s_mb[u] <= mb (binary
// search; every lane computes the same answer).
__device__ inline int segment_of_block(const int* s_mb, int n_act, int64_t mb) {
  int lo = 0, hi = n_act - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) / 2;
    if (s_mb[mid] <= mb) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

// One (segment, position block, row block) tile: acc[b][tt] += sum over K of
// A(positions 16 tt ..) x B_b, B operand b of the wave being weight row tile
// rt[b] of matrix (nib[b], sc[b]).  A rows hold AW 16-byte units per chunk
// (1: fp16 x; 2: fp16 hi then lo of h).
template <int BM, int AW, int NB, bool SPLIT>
__device__ inline void gemm_tile(const GemmK& a, const int64_t* s_row, u32x4* lds_a,
                                 const uint8_t* const nib[NB], const uint16_t* const sc[NB],
                                 const int64_t rt[NB], f32x4 acc[NB][BM / 16]) {
  constexpr int TT = BM / 16;
  constexpr int PITCH = 16 * AW;          // 16-byte units per LDS row
  constexpr int TPR = 256 / BM;           // staging threads per row
  constexpr int UPT = 16 * AW / TPR;      // 16-byte units each staging thread moves
  // Unit u of row r is stored at u ^ swz(r): the 16 rows a ds_read_b128 of one
  // 16-lane group touches then sit in 16 distinct bank quads.
  auto swz = [](int row) { return (row & 15) * AW; };
  static_assert(TPR * UPT == 16 * AW && UPT >= 1, "staging threads cover a row");
  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int n = lane % 16;
  const int p = lane / 16;
  const uint32_t mask = vgpr_const(0x000F000Fu);
  const int r = tid / TPR;
  const int u0 = (tid % TPR) * UPT;       // first unit of the row this thread moves
  const uint16_t* arow = a.a_src + s_row[r] * a.Kq * (128 * AW) + u0 * 8;
  u32x4 an[UPT];
  u32x4 bw[NB], bn[NB];
  uint2 bs[NB], bsn[NB];
  auto load_a = [&](int64_t q) {
#pragma unroll
    for (int i = 0; i < UPT; ++i) an[i] = reinterpret_cast<const u32x4*>(arow + q * (128 * AW))[i];
  };
  auto store_a = [&](int64_t q, int buf) {
    const u32x4 zero = {0u, 0u, 0u, 0u};
    u32x4* dst = lds_a + (buf * BM + r) * PITCH;
#pragma unroll
    for (int i = 0; i < UPT; ++i) {
      const int gi = ((u0 + i) / AW) % 4;  // chunk (p, gi): padded groups read 0
      dst[(u0 + i) ^ swz(r)] = (4 * q + gi < a.Kg) ? an[i] : zero;
    }
  };
  auto load_b = [&](int64_t q, u32x4* w, uint2* sv) {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const int64_t tq = rt[b] * a.Kq + q;
      w[b] = *reinterpret_cast<const u32x4*>(nib[b] + tq * kQuadNibBytes + lane * 16);
      sv[b] = *reinterpret_cast<const uint2*>(sc[b] + tq * kQuadScales + n * 4);
    }
  };
  load_a(0);
  load_b(0, bw, bs);
  store_a(0, 0);
  __syncthreads();
  for (int64_t q = 0; q < a.Kq; ++q) {
    const int cur = (int)(q & 1);
    const bool more = q + 1 < a.Kq;
    if (more) {
      load_a(q + 1);
      load_b(q + 1, bn, bsn);
    }
    const u32x4* la = lds_a + cur * BM * PITCH;
    // the scaled form keeps one group's MFMA results live at a time
    constexpr int kGroupUnroll = SPLIT ? 4 : 1;
#pragma unroll kGroupUnroll
    for (int gi = 0; gi < 4; ++gi) {
      if constexpr (SPLIT) {
        u32x4 bh[NB], bl[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          const uint32_t s2 = gi < 2 ? bs[b].x : bs[b].y;
          dequant_split_f16(bw[b][gi], (gi % 2) ? (s2 >> 16) : (s2 & 0xffffu), mask, bh[b], bl[b]);
        }
#pragma unroll
        for (int tt = 0; tt < TT; ++tt) {
          const u32x4* row = la + (tt * 16 + n) * PITCH;
          const int unit = (p * 4 + gi) * AW;
          const u32x4 ah = row[unit ^ swz(n)];
#pragma unroll
          for (int b = 0; b < NB; ++b) {
            acc[b][tt] = mfma_f16_16x16x32(ah, bh[b], acc[b][tt]);
            acc[b][tt] = mfma_f16_16x16x32(ah, bl[b], acc[b][tt]);
          }
          if constexpr (AW == 2) {
            const u32x4 al = row[(unit + 1) ^ swz(n)];
#pragma unroll
            for (int b = 0; b < NB; ++b) acc[b][tt] = mfma_f16_16x16x32(al, bh[b], acc[b][tt]);
          }
        }
      } else {
        // exact group sums P = A . (n - 8), then acc += d * P in fp32
        u32x4 bq[NB];
        float d[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          float dv[4];
          unpack_scales(bs[b], dv);
          d[b] = dv[gi];
          bq[b] = dequant_int_f16(bw[b][gi], mask);
        }
        const f32x4 z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int tt = 0; tt < TT; ++tt) {
          const u32x4* row = la + (tt * 16 + n) * PITCH;
          const int unit = (p * 4 + gi) * AW;
          const u32x4 ah = row[unit ^ swz(n)];
          u32x4 al = ah;
          if constexpr (AW == 2) al = row[(unit + 1) ^ swz(n)];
#pragma unroll
          for (int b = 0; b < NB; ++b) {
            f32x4 pv = mfma_f16_16x16x32(ah, bq[b], z);
            if constexpr (AW == 2) pv = mfma_f16_16x16x32(al, bq[b], pv);
            acc[b][tt] += d[b] * pv;
          }
        }
      }
    }
    if (more) {
      store_a(q + 1, cur ^ 1);
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        bw[b] = bn[b];
        bs[b] = bsn[b];
      }
    }
    __syncthreads();
  }
}

// XCD-aware item order.  Workgroups are dispatched to the 8 XCDs round-robin
// (workgroup b on XCD b % 8), each XCD with its own L2.  Position block mb is
// handled only by the workgroups of XCD mb % 8, all its row blocks by
// neighbouring workgroups there, so the block's A rows come from HBM once and
// then from that L2.  Blocks (not segments) are dealt out, so one large
// segment still spreads over every XCD.
struct XcdPlan {
  int nx, x;
  int64_t l, nl, n_items;
};

__device__ inline XcdPlan xcd_plan(int64_t n_mb, int64_t n_nb) {
  XcdPlan q;
  q.nx = gridDim.x < 8 ? (int)gridDim.x : 8;
  q.x = (int)(blockIdx.x % q.nx);
  q.l = blockIdx.x / q.nx;
  q.nl = ((int64_t)gridDim.x - q.x + q.nx - 1) / q.nx;
  const int64_t mbs = n_mb > q.x ? (n_mb - q.x + q.nx - 1) / q.nx : 0;  // blocks of this XCD
  q.n_items = mbs * n_nb;
  return q;
}

// Shared prologue of both kernels: descriptors, item plan, and the A row of
// every position of the tile.
struct TileCoord {
  int e;
  int64_t m0, end;
  int64_t nb;
};

template <int BM>
__device__ inline TileCoord tile_coord(const GemmK& a, const int4* s_desc, const int* s_mb, int n_act,
                                       const XcdPlan& xp, int64_t item, int64_t n_nb, int64_t* s_row) {
  TileCoord c;
  const int64_t mb = (item / n_nb) * xp.nx + xp.x;
  c.nb = item % n_nb;
  const int u = segment_of_block(s_mb, n_act, mb);
  const int4 d = s_desc[u];
  c.e = __builtin_amdgcn_readfirstlane(d.x);
  c.m0 = (int64_t)d.y + (mb - s_mb[u]) * BM;
  c.end = d.z;
  if (threadIdx.x < BM) {
    const int64_t pos = c.m0 + threadIdx.x;
    int64_t row = a.a_zero_row;
    if (pos < c.end) row = a.a_by_token ? (int64_t)a.seg.seg_tok[pos] : pos;
    s_row[threadIdx.x] = row;
  }
  __syncthreads();
  return c;
}

__global__ __launch_bounds__(kGemmWaves * kWave) void gemm_gate_up_kernel(GemmK a) {
  constexpr int BM = kGemmBMGateUp;
  constexpr int TT = BM / 16;
  __shared__ u32x4 lds_a[kGemmLdsA / 16];
  __shared__ int4 s_desc[kMaxExperts + 1];
  __shared__ int s_mb[kMaxExperts + 2];
  __shared__ int64_t s_row[BM];
  __shared__ int s_nact;
  const int lane = threadIdx.x % kWave;
  const int w = threadIdx.x / kWave;
  const int n = lane % 16;
  const int p = lane / 16;
  if (blockIdx.x == 0) {
    // the all-zero down-operand row read for positions past a segment
    for (int64_t i = threadIdx.x; i < a.KqI * 256; i += blockDim.x) a.hq16[a.h_zero_row * a.KqI * 256 + i] = 0;
  }
  const int n_act = load_descriptors(a.seg, s_desc, &s_nact);
  const int64_t n_mb = plan_items<BM>(s_desc, n_act, s_mb);
  const int64_t n_nb = ceil_div(a.N, kGemmRowsGU);
  const XcdPlan xp = xcd_plan(n_mb, n_nb);
  for (int64_t item = xp.l; item < xp.n_items; item += xp.nl) {
    const TileCoord c = tile_coord<BM>(a, s_desc, s_mb, n_act, xp, item, n_nb, s_row);
    const int64_t n_tiles = a.N / kRowTile;
    const int64_t t = c.nb * kGemmWaves + w;             // this wave's 16-row tile of I
    const int64_t tc = t < n_tiles ? t : n_tiles - 1;    // a tile past I computes, unstored
    const int64_t nib_stride = a.N * a.Kq * 64, sc_stride = a.N * a.Kq * 4;
    const bool routed = c.e < a.seg.E;
    const uint8_t* const nib[2] = {routed ? a.nib1 + c.e * nib_stride : a.sh_nib1,
                                   routed ? a.nib2 + c.e * nib_stride : a.sh_nib2};
    const uint16_t* const sc[2] = {routed ? a.sc1 + c.e * sc_stride : a.sh_sc1,
                                   routed ? a.sc2 + c.e * sc_stride : a.sh_sc2};
    const int64_t rt[2] = {tc, tc};
    f32x4 acc[2][TT];
    const f32x4 z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int tt = 0; tt < TT; ++tt) acc[b][tt] = z;
    gemm_tile<BM, 1, 2, kGemmSplitGateUp>(a, s_row, lds_a, nib, sc, rt, acc);

    // SwiGLU, then h as the fp16 pair hi + lo into LDS in down-operand chunk
    // order [group of the workgroup][position][part p'][hi 8, lo 8]: element
    // cc = half * 16 + n of a group sits at j' = kmap^-1(p', cc), half = w % 2.
    uint16_t* hs = reinterpret_cast<uint16_t*>(lds_a);
    const int gl = w / 2;  // group of the workgroup this wave's tile belongs to
    const int half = w % 2;
    const int pp = n / 4;
    const int rr = n % 4;
    const int jj = half == 0 ? ((rr & 1) ? 4 : 0) + (rr >> 1) : ((rr & 1) ? 6 : 2) + (rr >> 1);
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int m = tt * 16 + 4 * p + j;
        const float gv = acc[0][tt][j];
        const float uv = acc[1][tt][j];
        const float hv = swiglu_fast(gv, uv);
        const uint32_t hb = float_to_half_bits(hv);
        const uint32_t lb = float_to_half_bits(hv - half_bits_to_float32(hb));
        uint16_t* chunk = hs + ((gl * BM + m) * 4 + pp) * 16;
        chunk[jj] = (uint16_t)hb;
        chunk[8 + jj] = (uint16_t)lb;
      }
    }
    __syncthreads();
    // the workgroup's two groups: BM positions x 4 parts x 2 groups chunks
    for (int cidx = threadIdx.x; cidx < 2 * BM * 4; cidx += blockDim.x) {
      const int g2 = cidx / (BM * 4);
      const int m = (cidx / 4) % BM;
      const int p2 = cidx % 4;
      const int64_t g = c.nb * 2 + g2;  // group of I
      const int64_t pos = c.m0 + m;
      if (pos < c.end && 2 * g + 1 < n_tiles) {
        const u32x4* src = reinterpret_cast<const u32x4*>(hs + ((g2 * BM + m) * 4 + p2) * 16);
        u32x4* dst = reinterpret_cast<u32x4*>(a.hq16 + ((pos * a.KqI + g / 4) * 16 + p2 * 4 + g % 4) * 16);
        dst[0] = src[0];
        dst[1] = src[1];
      }
    }
    __syncthreads();
  }
}

__global__ __launch_bounds__(kGemmWaves * kWave) void gemm_down_kernel(GemmK a) {
  constexpr int BM = kGemmBMDown;
  constexpr int TT = BM / 16;
  __shared__ u32x4 lds_a[kGemmLdsA / 16];
  __shared__ int4 s_desc[kMaxExperts + 1];
  __shared__ int s_mb[kMaxExperts + 2];
  __shared__ int64_t s_row[BM];
  __shared__ int s_nact;
  const int lane = threadIdx.x % kWave;
  const int w = threadIdx.x / kWave;
  const int n = lane % 16;
  const int p = lane / 16;
  const int n_act = load_descriptors(a.seg, s_desc, &s_nact);
  const int64_t n_mb = plan_items<BM>(s_desc, n_act, s_mb);
  const int64_t n_nb = ceil_div(a.N, kGemmRowsDown);
  const int64_t n_tiles = a.N / kRowTile;
  const XcdPlan xp = xcd_plan(n_mb, n_nb);
  for (int64_t item = xp.l; item < xp.n_items; item += xp.nl) {
    const TileCoord c = tile_coord<BM>(a, s_desc, s_mb, n_act, xp, item, n_nb, s_row);
    const int64_t nib_stride = a.N * a.Kq * 64, sc_stride = a.N * a.Kq * 4;
    const bool routed = c.e < a.seg.E;
    const uint8_t* d_nib = routed ? a.nib1 + c.e * nib_stride : a.sh_nib1;
    const uint16_t* d_sc = routed ? a.sc1 + c.e * sc_stride : a.sh_sc1;
    const uint8_t* nib[kGemmNBDown];
    const uint16_t* sc[kGemmNBDown];
    int64_t rt[kGemmNBDown];
#pragma unroll
    for (int b = 0; b < kGemmNBDown; ++b) {
      nib[b] = d_nib;
      sc[b] = d_sc;
      const int64_t t = (c.nb * kGemmWaves + w) * kGemmNBDown + b;
      rt[b] = t < n_tiles ? t : n_tiles - 1;  // a tile past H computes, unstored
    }
    f32x4 acc[kGemmNBDown][TT];
    const f32x4 z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int b = 0; b < kGemmNBDown; ++b)
#pragma unroll
      for (int tt = 0; tt < TT; ++tt) acc[b][tt] = z;
    gemm_tile<BM, 2, kGemmNBDown, kGemmSplitDown>(a, s_row, lds_a, nib, sc, rt, acc);
#pragma unroll
    for (int b = 0; b < kGemmNBDown; ++b) {
      const int64_t t = (c.nb * kGemmWaves + w) * kGemmNBDown + b;
      if (t >= n_tiles) continue;
#pragma unroll
      for (int tt = 0; tt < TT; ++tt) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int64_t pos = c.m0 + tt * 16 + 4 * p + j;
          if (pos < c.end) a.outbuf[pos * a.N + t * 16 + n] = acc[b][tt][j];
        }
      }
    }
  }
}

// ------------------------------------------------- tile pipeline, LDS ring
//
// The same tiles and arithmetic as gemm_tile, with both operands staged by
// direct-to-LDS loads into a ring of kG2Stages LDS stages two quads ahead of
// the MFMAs: per quad and wave, the wave's share of the A rows and its own B
// operands (nibbles and scales).  The loads are issued from inline assembly
// (dma_b128_unseen), so the compiler adds no waits of its own; per quad there
// is one workgroup barrier, preceded by a wait for the wave's copies of the
// quad about to be read (the newer quad's copies stay in flight), which also
// guarantees every wave has left the stage about to be refilled.  A rows are
// stored with unit s of row r at s ^ (r & 15), so the 16 rows one
// ds_read_b128 group touches fall in distinct banks for both operand widths.
// Padded groups of K (I not a multiple of 128 in the down projection, whose
// operand rows leave them unwritten) are skipped.
constexpr int kG2Waves = 8;
constexpr int kG2Stages = 3;
constexpr int kG2AUnits = 2048;  // 16-byte units of A per stage: BM x 16 x AW (128 x 16, 64 x 32)
constexpr int kG2NB = 2;         // B operands per wave in both kernels
constexpr int kG2BUnits = kG2Waves * kG2NB * kWave;  // nibbles: one 1 KiB unit row per operand
constexpr int kG2SUnits = kG2Waves * kG2NB * 8;      // scales: 128 B per operand
constexpr int kG2StageUnits = kG2AUnits + kG2BUnits + kG2SUnits;
constexpr int kG2LoadsPerQuad = kG2AUnits / kWave / kG2Waves + 2 * kG2NB;  // per wave

// s_waitcnt vmcnt(N) lgkmcnt(0), gfx9 encoding.
template <int N>
__device__ inline void wait_vm_lgkm0() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4));
}

// Active segment count (active slots come first; wave 0 scans, the others
// wait at the barrier) without copying the descriptors to LDS.
__device__ inline int count_active(const SegSrc& seg, int* s_nact) {
  if (threadIdx.x < kWave) {
    int cnt = 0;
    for (int u0 = 0; u0 < seg.max_slots; u0 += kWave) {
      const int u = u0 + (int)threadIdx.x;
      const bool act = u < seg.max_slots && seg.desc[u < seg.max_slots ? u : 0].x >= 0;
      cnt += __popcll(__ballot(act));
    }
    if (threadIdx.x == 0) *s_nact = cnt;
  }
  __syncthreads();
  return *s_nact;
}

// SPLIT: the split-scale operands (2 MFMAs per group and position tile for
// gate/up, 3 for down); else one MFMA per A operand against the integers
// n - 8 (exact group sums), scaled into the accumulators with fp32 FMAs.
// VT: the leading 16-position tiles of the block that are multiplied (the
// caller rounds the tiles holding a segment position up to 2, 4 or 8); the
// rest lie past the segment end, so their MFMAs, A reads and scaling are
// skipped, and their accumulators stay zero and are never stored.  A
// compile-time count keeps the loop branch-free: a run-time test per tile
// broke the software pipelining and cost 30%.
template <int BM, int AW, bool SPLIT, int VT>
__device__ inline void gemm_tile3(const GemmK& a, const int64_t* s_row, u32x4* lds, const i32x4& ar,
                                  const i32x4 (&nr)[kG2NB], const i32x4 (&sr)[kG2NB], const int64_t (&rt)[kG2NB],
                                  f32x4 acc[kG2NB][BM / 16]) {
  static_assert(VT >= 1 && VT <= BM / 16, "tiles to multiply");
  constexpr int NB = kG2NB;
  constexpr int TT = BM / 16;
  constexpr int UPR = 16 * AW;                // 16-byte units per A row
  constexpr int RPD = kWave / UPR;            // A rows per direct-to-LDS load
  constexpr int ND = kG2AUnits / kWave / kG2Waves;  // A loads per wave per quad
  static_assert(BM * UPR == kG2AUnits && ND >= 1, "one stage holds the tile");
  const int lane = threadIdx.x % kWave;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int n = lane % 16;
  const int p = lane / 16;
  const uint32_t mask = vgpr_const(0x000F000Fu);
  const uint32_t row_bytes = (uint32_t)(a.Kq * 256 * AW);
  // this wave's A loads j = w + kG2Waves * i: lane l fills slot l % UPR of row
  // j * RPD + l / UPR with logical unit (slot ^ (row & 15))
  uint32_t voff[ND];
#pragma unroll
  for (int i = 0; i < ND; ++i) {
    const int j = w + kG2Waves * i;
    const int row = j * RPD + lane / UPR;
    const int unit = (lane % UPR) ^ (row & 15);
    voff[i] = (uint32_t)s_row[row] * row_bytes + (uint32_t)unit * 16u;
  }
  const uint32_t lds0 = lds_addr(lds);
  auto uni = [](uint32_t v) { return (uint32_t)__builtin_amdgcn_readfirstlane((int)v); };
  auto copy = [&](int64_t q) {
    const uint32_t st = lds0 + (uint32_t)(q % kG2Stages) * (kG2StageUnits * 16);
    const uint32_t aoff = uni((uint32_t)q * 256u * AW);
#pragma unroll
    for (int i = 0; i < ND; ++i)
      dma_b128_unseen(ar, uni(st + (uint32_t)(w + kG2Waves * i) * kWave * 16), voff[i], aoff);
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const uint32_t tq = uni((uint32_t)(rt[b] * a.Kq + q));
      dma_b128_unseen(nr[b], uni(st + (uint32_t)(kG2AUnits + (w * NB + b) * kWave) * 16), (uint32_t)lane * 16u,
                      tq * kQuadNibBytes);
      // the 128 scale bytes: eight lanes
      if (lane < 8)
        dma_b128_unseen(sr[b], uni(st + (uint32_t)(kG2AUnits + kG2BUnits + (w * NB + b) * 8) * 16),
                        (uint32_t)lane * 16u, tq * (kQuadScales * 2));
    }
  };
  copy(0);
  if (a.Kq > 1) copy(1);
  for (int64_t q = 0; q < a.Kq; ++q) {
    asm volatile("" ::: "memory");
    if (q + 1 < a.Kq) wait_vm_lgkm0<kG2LoadsPerQuad>();  // quad q's copies done, q + 1's may fly
    else wait_vm_lgkm0<0>();
    __builtin_amdgcn_s_barrier();  // every wave's copies are in; stage (q - 1) % 3 is free
    asm volatile("" ::: "memory");
    if (q + 2 < a.Kq) copy(q + 2);
    const u32x4* st = lds + (q % kG2Stages) * kG2StageUnits;
    const u32x4* la = st;
    u32x4 bw[NB];
    uint2 bs[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      bw[b] = st[kG2AUnits + (w * NB + b) * kWave + lane];
      bs[b] = reinterpret_cast<const uint2*>(st + kG2AUnits + kG2BUnits + (w * NB + b) * 8)[n];
    }
#pragma unroll
    for (int gi = 0; gi < 4; ++gi) {
      if (4 * q + gi >= a.Kg) continue;  // padded group (uniform)
      if constexpr (SPLIT) {
        u32x4 bh[NB], bl[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          const uint32_t s2 = gi < 2 ? bs[b].x : bs[b].y;
          dequant_split_f16(bw[b][gi], (gi % 2) ? (s2 >> 16) : (s2 & 0xffffu), mask, bh[b], bl[b]);
        }
#pragma unroll
        for (int tt = 0; tt < VT; ++tt) {
          const u32x4* row = la + (tt * 16 + n) * UPR;
          const int unit = (p * 4 + gi) * AW;
          const u32x4 ah = row[unit ^ n];
#pragma unroll
          for (int b = 0; b < NB; ++b) {
            acc[b][tt] = mfma_f16_16x16x32(ah, bh[b], acc[b][tt]);
            acc[b][tt] = mfma_f16_16x16x32(ah, bl[b], acc[b][tt]);
          }
          if constexpr (AW == 2) {
            const u32x4 al = row[(unit + 1) ^ n];
#pragma unroll
            for (int b = 0; b < NB; ++b) acc[b][tt] = mfma_f16_16x16x32(al, bh[b], acc[b][tt]);
          }
        }
      } else {
        u32x4 bq[NB];
        float d[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          const uint32_t s2 = gi < 2 ? bs[b].x : bs[b].y;
          d[b] = half_bits_to_float((uint16_t)((gi % 2) ? (s2 >> 16) : (s2 & 0xffffu)));
          bq[b] = dequant_int_f16(bw[b][gi], mask);
        }
        const f32x4 z = {0.f, 0.f, 0.f, 0.f};
        // Software-pipelined by one position tile: the fp32 scaling of tile
        // tt - 1 is issued after the MFMAs of tile tt, so it runs while they
        // execute instead of stalling on the result it reads.
        f32x4 pv[2][NB];
        // the group's A operands, all read from LDS before its first MFMA
        u32x4 ahv[VT], alv[VT];
#pragma unroll
        for (int tt = 0; tt < VT; ++tt) {
          const u32x4* row = la + (tt * 16 + n) * UPR;
          const int unit = (p * 4 + gi) * AW;
          ahv[tt] = row[unit ^ n];
          alv[tt] = ahv[tt];
          if constexpr (AW == 2) alv[tt] = row[(unit + 1) ^ n];
        }
#pragma unroll
        for (int tt = 0; tt < VT; ++tt) {
          const u32x4 ah = ahv[tt];
          const u32x4 al = alv[tt];
          // the lo MFMAs follow all the hi ones, so no MFMA waits on the one before it
#pragma unroll
          for (int b = 0; b < NB; ++b) pv[tt & 1][b] = mfma_f16_16x16x32(ah, bq[b], z);
          if constexpr (AW == 2) {
#pragma unroll
            for (int b = 0; b < NB; ++b) pv[tt & 1][b] = mfma_f16_16x16x32(al, bq[b], pv[tt & 1][b]);
          }
          if (tt > 0) {
#pragma unroll
            for (int b = 0; b < NB; ++b) acc[b][tt - 1] += d[b] * pv[(tt - 1) & 1][b];
          }
        }
#pragma unroll
        for (int b = 0; b < NB; ++b) acc[b][VT - 1] += d[b] * pv[(VT - 1) & 1][b];
      }
    }
  }
  lds_barrier();  // every wave has left the ring before it is reused
}

template <bool SPLIT>
__global__ __launch_bounds__(kG2Waves * kWave) void gemm_gate_up_kernel2(GemmK a) {
  constexpr int BM = kGemmBMGateUp;
  constexpr int TT = BM / 16;
  constexpr int kRows = kG2Waves * 16;  // rows of I per workgroup (kG2Waves / 2 groups)
  __shared__ u32x4 lds_a[kG2Stages * kG2StageUnits];
  __shared__ int s_mb[kMaxExperts + 2];
  __shared__ int64_t s_row[BM];
  __shared__ int s_nact;
  const int lane = threadIdx.x % kWave;
  const int w = threadIdx.x / kWave;
  const int n = lane % 16;
  const int p = lane / 16;
  if (blockIdx.x == 0) {
    for (int64_t i = threadIdx.x; i < a.KqI * 256; i += blockDim.x) a.hq16[a.h_zero_row * a.KqI * 256 + i] = 0;
  }
  const i32x4 ar = buf_rsrc_words(a.a_src, (uint32_t)((a.a_zero_row + 1) * a.Kq * 256));
  const int n_act = count_active(a.seg, &s_nact);
  const int64_t n_mb = plan_items<BM>(a.seg.desc, n_act, s_mb);
  const int64_t n_nb = ceil_div(a.N, kRows);
  const XcdPlan xp = xcd_plan(n_mb, n_nb);
  const uint32_t nib_bytes = (uint32_t)(a.N * a.Kq * 64), sc_bytes = (uint32_t)(a.N * a.Kq * 8);
  for (int64_t item = xp.l; item < xp.n_items; item += xp.nl) {
    const TileCoord c = tile_coord<BM>(a, a.seg.desc, s_mb, n_act, xp, item, n_nb, s_row);
    const int64_t n_tiles = a.N / kRowTile;
    const int64_t t = c.nb * kG2Waves + w;
    const int64_t tc = t < n_tiles ? t : n_tiles - 1;
    const bool routed = c.e < a.seg.E;
    const i32x4 nr[2] = {buf_rsrc_words(routed ? a.nib1 + (int64_t)c.e * nib_bytes : a.sh_nib1, nib_bytes),
                         buf_rsrc_words(routed ? a.nib2 + (int64_t)c.e * nib_bytes : a.sh_nib2, nib_bytes)};
    const i32x4 sr[2] = {
        buf_rsrc_words(routed ? reinterpret_cast<const uint8_t*>(a.sc1) + (int64_t)c.e * sc_bytes
                              : reinterpret_cast<const uint8_t*>(a.sh_sc1), sc_bytes),
        buf_rsrc_words(routed ? reinterpret_cast<const uint8_t*>(a.sc2) + (int64_t)c.e * sc_bytes
                              : reinterpret_cast<const uint8_t*>(a.sh_sc2), sc_bytes)};
    const int64_t rt[2] = {tc, tc};
    f32x4 acc[2][TT];
    const f32x4 z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int tt = 0; tt < TT; ++tt) acc[b][tt] = z;
    const int vt = __builtin_amdgcn_readfirstlane((int)ceil_div(c.end - c.m0, (int64_t)16));
    if (vt > 4) gemm_tile3<BM, 1, SPLIT, 8>(a, s_row, lds_a, ar, nr, sr, rt, acc);
    else if (vt > 2) gemm_tile3<BM, 1, SPLIT, 4>(a, s_row, lds_a, ar, nr, sr, rt, acc);
    else gemm_tile3<BM, 1, SPLIT, 2>(a, s_row, lds_a, ar, nr, sr, rt, acc);

    // SwiGLU, h as fp16 hi + lo into LDS in down-operand chunk order, as in
    // gemm_gate_up_kernel (kG2Waves / 2 groups of I per workgroup)
    uint16_t* hs = reinterpret_cast<uint16_t*>(lds_a);
    const int gl = w / 2;
    const int half = w % 2;
    const int pp = n / 4;
    const int rr = n % 4;
    const int jj = half == 0 ? ((rr & 1) ? 4 : 0) + (rr >> 1) : ((rr & 1) ? 6 : 2) + (rr >> 1);
    // tiles past the segment (tt >= vt) hold no position that is stored
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) {
      if (tt >= vt) break;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int m = tt * 16 + 4 * p + j;
        const float gv = acc[0][tt][j];
        const float uv = acc[1][tt][j];
        const float hv = swiglu_fast(gv, uv);
        const uint32_t hb = float_to_half_bits(hv);
        const uint32_t lb = float_to_half_bits(hv - half_bits_to_float32(hb));
        uint16_t* chunk = hs + ((gl * BM + m) * 4 + pp) * 16;
        chunk[jj] = (uint16_t)hb;
        chunk[8 + jj] = (uint16_t)lb;
      }
    }
    lds_barrier();
    constexpr int kGroups = kG2Waves / 2;
    for (int cidx = threadIdx.x; cidx < kGroups * BM * 4; cidx += blockDim.x) {
      const int g2 = cidx / (BM * 4);
      const int m = (cidx / 4) % BM;
      const int p2 = cidx % 4;
      const int64_t g = c.nb * kGroups + g2;  // group of I
      const int64_t pos = c.m0 + m;
      if (pos < c.end && 2 * g + 1 < n_tiles) {
        const u32x4* src = reinterpret_cast<const u32x4*>(hs + ((g2 * BM + m) * 4 + p2) * 16);
        u32x4* dst = reinterpret_cast<u32x4*>(a.hq16 + ((pos * a.KqI + g / 4) * 16 + p2 * 4 + g % 4) * 16);
        dst[0] = src[0];
        dst[1] = src[1];
      }
    }
    lds_barrier();
  }
}

template <bool SPLIT>
__global__ __launch_bounds__(kG2Waves * kWave) void gemm_down_kernel2(GemmK a) {
  constexpr int BM = kGemmBMDown;
  constexpr int TT = BM / 16;
  constexpr int NB = kG2NB;
  constexpr int kRows = kG2Waves * 16 * NB;  // rows of H per workgroup
  __shared__ u32x4 lds_a[kG2Stages * kG2StageUnits];
  __shared__ int s_mb[kMaxExperts + 2];
  __shared__ int64_t s_row[BM];
  __shared__ int s_nact;
  const int lane = threadIdx.x % kWave;
  const int w = threadIdx.x / kWave;
  const int n = lane % 16;
  const int p = lane / 16;
  const i32x4 ar = buf_rsrc_words(a.a_src, (uint32_t)((a.a_zero_row + 1) * a.Kq * 512));
  const int n_act = count_active(a.seg, &s_nact);
  const int64_t n_mb = plan_items<BM>(a.seg.desc, n_act, s_mb);
  const int64_t n_nb = ceil_div(a.N, kRows);
  const int64_t n_tiles = a.N / kRowTile;
  const XcdPlan xp = xcd_plan(n_mb, n_nb);
  const uint32_t nib_bytes = (uint32_t)(a.N * a.Kq * 64), sc_bytes = (uint32_t)(a.N * a.Kq * 8);
  for (int64_t item = xp.l; item < xp.n_items; item += xp.nl) {
    const TileCoord c = tile_coord<BM>(a, a.seg.desc, s_mb, n_act, xp, item, n_nb, s_row);
    const bool routed = c.e < a.seg.E;
    const i32x4 nw = buf_rsrc_words(routed ? a.nib1 + (int64_t)c.e * nib_bytes : a.sh_nib1, nib_bytes);
    const i32x4 sw = buf_rsrc_words(routed ? reinterpret_cast<const uint8_t*>(a.sc1) + (int64_t)c.e * sc_bytes
                                           : reinterpret_cast<const uint8_t*>(a.sh_sc1), sc_bytes);
    const i32x4 nr[NB] = {nw, nw};
    const i32x4 sr[NB] = {sw, sw};
    int64_t rt[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const int64_t t = (c.nb * kG2Waves + w) * NB + b;
      rt[b] = t < n_tiles ? t : n_tiles - 1;
    }
    f32x4 acc[NB][TT];
    const f32x4 z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int tt = 0; tt < TT; ++tt) acc[b][tt] = z;
    const int vt = __builtin_amdgcn_readfirstlane((int)ceil_div(c.end - c.m0, (int64_t)16));
    if (vt > 2) gemm_tile3<BM, 2, SPLIT, 4>(a, s_row, lds_a, ar, nr, sr, rt, acc);
    else gemm_tile3<BM, 2, SPLIT, 2>(a, s_row, lds_a, ar, nr, sr, rt, acc);
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const int64_t t = (c.nb * kG2Waves + w) * NB + b;
      if (t >= n_tiles) continue;
#pragma unroll
      for (int tt = 0; tt < TT; ++tt) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int64_t pos = c.m0 + tt * 16 + 4 * p + j;
          if (pos < c.end) a.outbuf[pos * a.N + t * 16 + n] = acc[b][tt][j];
        }
      }
    }
  }
}

bool gemm_regime(int64_t T, int k, int E) {
  const int64_t slots = T * k;
  const int64_t seg_max = slots < E ? slots : E;
  return slots >= kGemmMinSlotsPerExpert * seg_max;
}

// PHANTOM_MOE_GEMM_KERNEL=v1 selects the register-staged tile pipeline
// (gemm_tile, 4 waves) instead of the LDS ring (gemm_tile2, 8 waves).
static bool gemm_v1() {
  const char* v = getenv("PHANTOM_MOE_GEMM_KERNEL");
  return v && strcmp(v, "v1") == 0;
}

bool gemm_uses_ring() { return !gemm_v1(); }

// The ring kernels scale exact integer group sums in fp32 (one MFMA per A
// operand and group; 10% faster than the split-scale operands at Qwen3 shape,
// 4096 tokens: gate/up 479 -> 433 us, down 372 -> 333 us);
// PHANTOM_MOE_GEMM_SCALE=split selects the split-scale operands.
static bool gemm_split() {
  const char* v = getenv("PHANTOM_MOE_GEMM_SCALE");
  return v && strcmp(v, "split") == 0;
}

static int64_t gemm_max_items(const ExpertArgs& x, int BM, int64_t n_nb) {
  const int64_t rows = x.T * x.k + (x.has_shared ? x.T : 0);
  return (ceil_div(rows, BM) + max_active_experts(x)) * n_nb;
}

hipError_t launch_gemm_gate_up(const ExpertArgs& x, const Workspace& ws, hipStream_t stream) {
  GemmK g = {};
  g.seg = segments_of(x, ws);
  g.a_src = ws.xq;
  g.a_zero_row = x.T;
  g.a_by_token = 1;
  g.Kq = ceil_div(x.H, kQuad);
  g.Kg = x.H / kGroup;
  g.N = x.I;
  g.nib1 = x.gate_nib;
  g.sc1 = x.gate_scale;
  g.nib2 = x.up_nib;
  g.sc2 = x.up_scale;
  g.sh_nib1 = x.sh_gate_nib;
  g.sh_sc1 = x.sh_gate_scale;
  g.sh_nib2 = x.sh_up_nib;
  g.sh_sc2 = x.sh_up_scale;
  g.hq16 = ws.hq;
  g.KqI = ceil_div(x.I, kQuad);
  g.h_zero_row = x.T * x.k + (x.has_shared ? x.T : 0);
  if (gemm_v1()) {
    const int64_t max_items = gemm_max_items(x, kGemmBMGateUp, ceil_div(x.I, kGemmRowsGU));
    hipLaunchKernelGGL(gemm_gate_up_kernel, dim3(resident_grid(gemm_gate_up_kernel, kGemmWaves * kWave, max_items)),
                       dim3(kGemmWaves * kWave), 0, stream, g);
  } else {
    const int64_t max_items = gemm_max_items(x, kGemmBMGateUp, ceil_div(x.I, kG2Waves * 16));
    if (gemm_split())
      hipLaunchKernelGGL(gemm_gate_up_kernel2<true>,
                         dim3(resident_grid(gemm_gate_up_kernel2<true>, kG2Waves * kWave, max_items)),
                         dim3(kG2Waves * kWave), 0, stream, g);
    else
      hipLaunchKernelGGL(gemm_gate_up_kernel2<false>,
                         dim3(resident_grid(gemm_gate_up_kernel2<false>, kG2Waves * kWave, max_items)),
                         dim3(kG2Waves * kWave), 0, stream, g);
  }
  return hipGetLastError();
}

hipError_t launch_gemm_down(const ExpertArgs& x, const Workspace& ws, hipStream_t stream) {
  GemmK g = {};
  g.seg = segments_of(x, ws);
  g.a_src = ws.hq;
  g.a_zero_row = x.T * x.k + (x.has_shared ? x.T : 0);
  g.a_by_token = 0;
  g.Kq = ceil_div(x.I, kQuad);
  g.Kg = x.I / kGroup;
  g.N = x.H;
  g.nib1 = x.down_nib;
  g.sc1 = x.down_scale;
  g.sh_nib1 = x.sh_down_nib;
  g.sh_sc1 = x.sh_down_scale;
  g.outbuf = ws.outbuf;
  if (gemm_v1()) {
    const int64_t max_items = gemm_max_items(x, kGemmBMDown, ceil_div(x.H, kGemmRowsDown));
    hipLaunchKernelGGL(gemm_down_kernel, dim3(resident_grid(gemm_down_kernel, kGemmWaves * kWave, max_items)),
                       dim3(kGemmWaves * kWave), 0, stream, g);
  } else {
    const int64_t max_items = gemm_max_items(x, kGemmBMDown, ceil_div(x.H, kG2Waves * 16 * kGemmNBDown));
    if (gemm_split())
      hipLaunchKernelGGL(gemm_down_kernel2<true>, dim3(resident_grid(gemm_down_kernel2<true>, kG2Waves * kWave, max_items)),
                         dim3(kG2Waves * kWave), 0, stream, g);
    else
      hipLaunchKernelGGL(gemm_down_kernel2<false>,
                         dim3(resident_grid(gemm_down_kernel2<false>, kG2Waves * kWave, max_items)),
                         dim3(kG2Waves * kWave), 0, stream, g);
  }
  return hipGetLastError();
}

}  // namespace pmoe
