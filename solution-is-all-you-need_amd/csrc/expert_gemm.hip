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
//      the fp16 pair hi + lo written by the gate/up epilogue
//      (|h - hi - lo| <= 2^-22 |h|).
//   B  the integers q = n - 8 as fp16: the nibble becomes the fp16 value
//      1024 + n (one v_and_or_b32 per pair) and one v_pk_add_f16 gives q.
// Per 32-group g, an MFMA gives the exact group sums P = A . q (fp32), and
// acc += d[n][g] * P scales them in fp32 (four FMAs per MFMA output tile).
// (Weights rounded to fp16 as q * d, one MFMA and no scaling, cost 9e-3 of
// max-abs error on outputs of magnitude 40 per rounded stage; the layer
// tolerance is 1e-2.)
//
// Tile pipeline.  Both operands are staged by direct-to-LDS loads into a ring
// of kG2Stages LDS stages two K quads ahead of the MFMAs: per quad, waves 0-3
// copy the A rows and the B operands (nibbles and scales) of all eight waves,
// so waves 4-7 never wait on vmcnt and their global stores stay in flight.
// The loads are issued from inline assembly (dma_b128_unseen), so the
// compiler adds no waits of its own; per quad there is one workgroup barrier,
// preceded by each copying wave's wait for its copies of the quad about to
// be read (the newer quad's copies stay in flight), which also guarantees
// every wave has left the stage about to be refilled.  A rows are stored with unit s of row
// r at s ^ a_swizzle(r & 15), so that no ds_read_b128 of the A operands
// has a bank conflict (see a_swizzle).  Padded groups of K (a ragged last quad of H or I) are
// skipped.
//
// Tiling.  A workgroup of kG2Waves waves owns BM consecutive positions of
// one expert segment and a block of weight rows; every wave multiplies all BM
// positions with NB = 2 weight row tiles of its own, so each B operand feeds
// up to BM / 16 (times AW) MFMAs, one per 16-position tile that holds a
// segment position.
//   gate/up (BM 128, AW 1): wave w takes the gate and the up operand of one
//            16-row tile of I, so its SwiGLU epilogue has both factors of
//            every output; the workgroup's 8 tiles are 4 whole 32-groups of
//            I, written as down-operand chunks (hi + lo) via LDS, stored by
//            waves 4-7.
//   down (BM 64, AW 2):  wave w takes two 16-row tiles of H.
//
// Schedule.  Per group the wave needs VT (times AW) A operands from LDS; the
// reads of group g + 1 are issued while the MFMAs of group g run, and the
// fp32 scaling of a tile's sums runs while the next tile's MFMAs execute, so
// no instruction waits on the one just issued.  (Left to itself the compiler
// issued each A read right before its two MFMAs, with a wait for it: one LDS
// round trip per two MFMAs.)
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <type_traits>

#include "expert_common.h"
#include "moe_common.h"
#include "moe_launch.h"

namespace pmoe {

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
  // the down GEMM's A operand
  uint16_t* hq16;
  int64_t KqI;
  int64_t h_zero_row;
  // down output: fp32 [rows][H]
  float* outbuf;
};

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));

// B operand of one 32-group: the lane's four nibble bytes w (bytes 4p..4p+3 of
// the group's qs for its row) -> the eight fp16 integers n - 8 in kmap order.
// mask holds 0x000F000F.
__device__ inline u32x4 dequant_int_f16(uint32_t w, uint32_t mask) {
  const h2_t off = {(_Float16)1032.0f, (_Float16)1032.0f};
  const uint32_t r[4] = {and_or(w, mask, 0x64006400u), and_or(w >> 4, mask, 0x64006400u),
                         and_or(w >> 8, mask, 0x64006400u), and_or(w >> 12, mask, 0x64006400u)};
  u32x4 out;
#pragma unroll
  for (int i = 0; i < 4; ++i) out[i] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2_t, r[i]) - off);
  return out;
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

// XCD-aware item order.  Workgroups are dispatched to the 8 XCDs round-robin
// (workgroup b on XCD b % 8), each XCD with its own L2.  The position blocks,
// in segment order, are cut into 8 contiguous ranges, one per XCD, and an
// XCD's items run block by block with the row blocks innermost.  The
// workgroups of an XCD that run at one time then share the A rows of each
// block (its row blocks run side by side) and the weights of each segment
// (its position blocks are neighbours in the range), so both come from HBM
// about once.  (Blocks dealt round-robin over the XCDs put the 2-3 blocks of
// a segment on different XCDs, each streaming the segment's weights.)
struct XcdPlan {
  int nx, x;
  int64_t l, nl, b0, n_items;
};

__device__ inline XcdPlan xcd_plan(int64_t n_mb, int64_t n_nb) {
  XcdPlan q;
  q.nx = gridDim.x < 8 ? (int)gridDim.x : 8;
  q.x = (int)(blockIdx.x % q.nx);
  q.l = blockIdx.x / q.nx;
  q.nl = ((int64_t)gridDim.x - q.x + q.nx - 1) / q.nx;
  q.b0 = n_mb * q.x / q.nx;
  q.n_items = (n_mb * (q.x + 1) / q.nx - q.b0) * n_nb;
  return q;
}

// Shared prologue of both kernels: descriptors, item plan, and the A row of
// every position of the tile.
struct TileCoord {
  int e;
  int64_t m0, end;
  int64_t nb;
};

// half >= 0: only positions [BM / 2 half, BM / 2 (half + 1)) of the block.
// The active slots' descriptors in LDS, copied once per launch: read there,
// an item's set-up issues no global load, after which the compiler would
// wait for every outstanding store of the wave (the gate/up kernel's storing
// waves keep theirs in flight into the next item).
struct SegLds {
  int e[kMaxExperts + 1], beg[kMaxExperts + 1], end[kMaxExperts + 1];
};

__device__ inline void seg_to_lds(const SegSrc& seg, int n_act, SegLds* sl) {
  for (int u = threadIdx.x; u < n_act; u += blockDim.x) {
    const int4 d = seg.desc[u];
    sl->e[u] = d.x;
    sl->beg[u] = d.y;
    sl->end[u] = d.z;
  }
}

template <int BM>
__device__ inline TileCoord tile_coord(const GemmK& a, const SegLds* sl, const int* s_mb, int n_act,
                                       const XcdPlan& xp, int64_t item, int64_t n_nb, int64_t* s_row,
                                       int half = -1) {
  TileCoord c;
  const int64_t mb = xp.b0 + item / n_nb;
  c.nb = item % n_nb;
  const int u = segment_of_block(s_mb, n_act, mb);
  c.e = __builtin_amdgcn_readfirstlane(sl->e[u]);
  c.m0 = (int64_t)sl->beg[u] + (mb - s_mb[u]) * BM;
  c.end = sl->end[u];
  if (half >= 0) {
    c.m0 += (int64_t)half * (BM / 2);
    c.end = c.end < c.m0 + BM / 2 ? c.end : c.m0 + BM / 2;
  }
  if (threadIdx.x < BM) {
    const int64_t pos = c.m0 + threadIdx.x;
    int64_t row = a.a_zero_row;
    if (pos < c.end) row = a.a_by_token ? (int64_t)a.seg.seg_tok[pos] : pos;
    s_row[threadIdx.x] = row;
  }
  __syncthreads();
  return c;
}

// ------------------------------------------------------------ the kernels
constexpr int kGemmBMGateUp = 128;  // segment positions per gate/up tile
constexpr int kGemmBMDown = 64;     // segment positions per down tile
constexpr int kG2Waves = 8;
constexpr int kG2Stages = 3;
constexpr int kG2AUnits = 2048;  // 16-byte units of A per stage: BM x 16 x AW (128 x 16, 64 x 32)
constexpr int kG2NB = 2;         // B operands per wave in both kernels
constexpr int kG2BUnits = kG2Waves * kG2NB * kWave;  // nibbles: one 1 KiB unit row per operand
constexpr int kG2SUnits = kG2Waves * kG2NB * 8;      // scales: 128 B per operand
constexpr int kG2StageUnits = kG2AUnits + kG2BUnits + kG2SUnits;

// Column swizzle of the A rows in LDS.  gfx950 serves a wave's ds_read_b128
// in four cycles of 16 lanes, lane l in cycle group (b0 ^ b1 ^ b2, b3) of its
// quad q = l / 4 (measured: two lanes conflict exactly when they share a
// group, a 16-byte column of a 256-byte LDS row, and not the row).  Lane
// (n, p) of an A read takes row n + 16 tt and logical unit AW (4p + gi) (+1);
// storing logical unit s of row r at s ^ a_swizzle(r & 15) puts the 16 lanes
// of every group in distinct columns for both kernels (AW 1 and 2), where the
// plain s ^ (r & 15) left two lanes per column (twice the LDS cycles).
// a_swizzle swaps bits 1 and 2 of r and folds bit 3 into bit 1.
__device__ inline uint32_t a_swizzle(uint32_t r) {
  return (r & 9u) | ((r & 2u) << 1) | (((r & 4u) >> 1) ^ ((r & 8u) >> 2));
}

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

// The multiply-accumulate of one K quad from LDS stage st into acc (shared
// by both kernels).  VT: the leading 16-position tiles of the block that are
// multiplied (the caller passes the number of tiles that hold a segment
// position); the rest lie past the segment end, so their MFMAs, A reads and
// scaling are skipped, and their accumulators stay zero and are never
// stored.  A compile-time count keeps the loop branch-free: a run-time test
// per tile broke the software pipelining and cost 30%.  RAGGED: groups at or
// past Kg (uniform) are skipped.  a_unit[gi]: this lane's LDS unit of A group
// gi (see gemm_tile3).
template <int BM, int AW, int VT, bool RAGGED>
__device__ __attribute__((always_inline)) inline void quad_math(const u32x4* st, uint32_t q, uint32_t Kg,
                                                                const uint32_t (&a_unit)[4], uint32_t mask,
                                                                f32x4 acc[kG2NB][BM / 16]) {
  static_assert(VT >= 1 && VT <= BM / 16, "tiles to multiply");
  constexpr int NB = kG2NB;
  constexpr int UPR = 16 * AW;  // 16-byte units per A row
  const int lane = threadIdx.x % kWave;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int n = lane % 16;
  const f32x4 z = {0.f, 0.f, 0.f, 0.f};
  // One group: MFMAs of every tile (hi then lo), the scaling of tile tt - 1
  // after the MFMAs of tile tt.
  auto group_math = [&](const u32x4 (&ah)[VT], const u32x4 (&al)[VT], const u32x4 (&bq)[NB], const float (&d)[NB]) {
    f32x4 pv[2][NB];
#pragma unroll
    for (int tt = 0; tt < VT; ++tt) {
#pragma unroll
      for (int b = 0; b < NB; ++b) pv[tt & 1][b] = mfma_f16_16x16x32(ah[tt], bq[b], z);
      if constexpr (AW == 2) {
#pragma unroll
        for (int b = 0; b < NB; ++b) pv[tt & 1][b] = mfma_f16_16x16x32(al[tt], bq[b], pv[tt & 1][b]);
      }
      if (tt > 0) {
#pragma unroll
        for (int b = 0; b < NB; ++b) acc[b][tt - 1] += d[b] * pv[(tt - 1) & 1][b];
      }
    }
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[b][VT - 1] += d[b] * pv[(VT - 1) & 1][b];
  };
  auto read_a = [&](int gi, u32x4 (&ah)[VT], u32x4 (&al)[VT]) {
#pragma unroll
    for (int tt = 0; tt < VT; ++tt) {
      ah[tt] = st[a_unit[gi] + tt * 16 * UPR];
      if constexpr (AW == 2) al[tt] = st[(a_unit[gi] ^ 1u) + tt * 16 * UPR];
      else al[tt] = ah[tt];
    }
  };
  auto operands = [&](const uint2 (&bs)[NB], const u32x4 (&bw)[NB], int gi, u32x4 (&bq)[NB], float (&d)[NB]) {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const uint32_t s2 = gi < 2 ? bs[b].x : bs[b].y;
      d[b] = half_bits_to_float((uint16_t)((gi % 2) ? (s2 >> 16) : (s2 & 0xffffu)));
      // the scale as fp32 in a register: the scaling is then v_fmac_f32,
      // not the slower mixed-precision v_fma_mix_f32 the compiler would
      // fold the conversion into
      asm volatile("" : "+v"(d[b]));
      bq[b] = dequant_int_f16(bw[b][gi], mask);
    }
  };
  // B operands, then the four groups, the A reads of group gi + 1 issued
  // before the MFMAs of group gi
  u32x4 bw[NB];
  uint2 bs[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    bw[b] = st[kG2AUnits + (w * NB + b) * kWave + lane];
    bs[b] = reinterpret_cast<const uint2*>(st + kG2AUnits + kG2BUnits + (w * NB + b) * 8)[n];
  }
  if constexpr (!RAGGED) {
    u32x4 ah[2][VT], al[2][VT];
    read_a(0, ah[0], al[0]);
#pragma unroll
    for (int gi = 0; gi < 4; ++gi) {
      if (gi < 3) read_a(gi + 1, ah[(gi + 1) & 1], al[(gi + 1) & 1]);
      u32x4 bq[NB];
      float d[NB];
      operands(bs, bw, gi, bq, d);
      group_math(ah[gi & 1], al[gi & 1], bq, d);
    }
  } else {
#pragma unroll
    for (int gi = 0; gi < 4; ++gi) {
      if (4 * q + gi >= Kg) break;
      u32x4 ah[VT], al[VT];
      read_a(gi, ah, al);
      u32x4 bq[NB];
      float d[NB];
      operands(bs, bw, gi, bq, d);
      group_math(ah, al, bq, d);
    }
  }
}

// The LDS offsets (16-byte units) of lane (n, p)'s A operands of group gi,
// tile 0: hi at n * UPR + ((p * 4 + gi) * AW ^ a_swizzle(n)), lo at that unit
// ^ 1 (AW * (p * 4 + gi) is even, so the pair stays adjacent); tile tt adds
// tt * 16 * UPR.
template <int AW>
__device__ inline void a_units(uint32_t (&a_unit)[4]) {
  const int lane = threadIdx.x % kWave;
  const uint32_t n = (uint32_t)(lane % 16), p = (uint32_t)(lane / 16);
#pragma unroll
  for (int gi = 0; gi < 4; ++gi) a_unit[gi] = n * 16 * AW + (((p * 4 + gi) * AW) ^ a_swizzle(n));
}

// One item's K loop through the LDS ring: both operands staged two quads
// ahead, one barrier per quad.  CW waves issue the copies: with CW = 8 each
// wave copies its own B operands and a share of A; with CW = 4 waves 0-3 copy
// everything (wave w the B operands of waves w and w + 4, rt[o] those of wave
// w + 4 o) and only they wait on vmcnt, so waves 4-7 may keep global stores
// in flight through the loop (gfx9 counts loads and stores in one vmcnt, and
// a wait for a copy would also wait for them).
template <int BM, int AW, int VT, int CW = kG2Waves>
__device__ inline void gemm_tile3(const GemmK& a, const int64_t* s_row, u32x4* lds, const i32x4& ar,
                                  const i32x4 (&nr)[kG2NB], const i32x4 (&sr)[kG2NB],
                                  const int64_t (&rt)[kG2Waves / CW][kG2NB], f32x4 acc[kG2NB][BM / 16]) {
  constexpr int NB = kG2NB;
  constexpr int OWN = kG2Waves / CW;          // waves whose B operands a copying wave loads
  constexpr int UPR = 16 * AW;                // 16-byte units per A row
  constexpr int RPD = kWave / UPR;            // A rows per direct-to-LDS load
  constexpr int ND = kG2AUnits / kWave / CW;  // A loads per copying wave per quad
  static_assert(BM * UPR == kG2AUnits && ND >= 1 && CW * OWN == kG2Waves, "one stage holds the tile");
  // A load i of the copying waves fills rows [CW RPD i, CW RPD (i + 1)); only
  // the loads that reach a multiplied tile (rows below 16 VT) are issued: the
  // rest would copy rows that no MFMA reads (at 64 positions to a
  // 128-position block, half of the A bytes)
  constexpr int NDV = (16 * VT + CW * RPD - 1) / (CW * RPD);
  static_assert(NDV >= 1 && NDV <= ND, "A loads issued");
  constexpr int kLoads = NDV + 2 * OWN * NB;  // copies per copying wave per quad
  const int lane = threadIdx.x % kWave;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const bool copier = w < CW;
  const uint32_t mask = vgpr_const(0x000F000Fu);
  const uint32_t row_bytes = (uint32_t)(a.Kq * 256 * AW);
  const uint32_t Kq = (uint32_t)a.Kq;
  // this wave's A loads j = w + CW * i: lane l fills slot l % UPR of row
  // j * RPD + l / UPR with logical unit (slot ^ a_swizzle(row & 15))
  uint32_t voff[ND];
#pragma unroll
  for (int i = 0; i < ND; ++i) {
    const int j = (copier ? w : 0) + CW * i;
    const int row = j * RPD + lane / UPR;
    const int unit = (lane % UPR) ^ (int)a_swizzle((uint32_t)row & 15u);
    voff[i] = (uint32_t)s_row[row] * row_bytes + (uint32_t)unit * 16u;
  }
  uint32_t a_unit[4];
  a_units<AW>(a_unit);
  const uint32_t lds0 = lds_addr(lds);
  auto uni = [](uint32_t v) { return (uint32_t)__builtin_amdgcn_readfirstlane((int)v); };
  auto copy = [&](uint32_t q, uint32_t stage) {
    if (!copier) return;
    const uint32_t st = lds0 + stage * (kG2StageUnits * 16);
    const uint32_t aoff = uni(q * 256u * AW);
#pragma unroll
    for (int i = 0; i < NDV; ++i)
      dma_b128_unseen(ar, uni(st + (uint32_t)(w + CW * i) * kWave * 16), voff[i], aoff);
#pragma unroll
    for (int o = 0; o < OWN; ++o) {
      const int ow = w + CW * o;
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const uint32_t tq = uni((uint32_t)rt[o][b] * Kq + q);
        dma_b128_unseen(nr[b], uni(st + (uint32_t)(kG2AUnits + (ow * NB + b) * kWave) * 16), (uint32_t)lane * 16u,
                        tq * kQuadNibBytes);
        // the 128 scale bytes: eight lanes
        if (lane < 8)
          dma_b128_unseen(sr[b], uni(st + (uint32_t)(kG2AUnits + kG2BUnits + (ow * NB + b) * 8) * 16),
                          (uint32_t)lane * 16u, tq * (kQuadScales * 2));
      }
    }
  };
  copy(0, 0);
  if (Kq > 1) copy(1, 1);
  // quads whose four groups are all real; a ragged last quad (H or I not a
  // multiple of 128) is done after the loop, so the accumulators keep one
  // register assignment through it
  const uint32_t Kq_full = (uint32_t)a.Kg / 4;
  uint32_t stage = 0;
  auto top = [&](uint32_t q) {
    asm volatile("" ::: "memory");
    if (copier) {
      if (q + 1 < Kq) wait_vm_lgkm0<kLoads>();  // quad q's copies done, q + 1's may fly
      else wait_vm_lgkm0<0>();
    } else {
      wait_vm_lgkm0<63>();  // LDS only: this wave's stores stay in flight
    }
    __builtin_amdgcn_s_barrier();  // every copy of quad q is in; stage (q - 1) % 3 is free
    asm volatile("" ::: "memory");
    if (q + 2 < Kq) copy(q + 2, stage == 0 ? 2u : stage - 1u);
    const u32x4* st = lds + stage * kG2StageUnits;
    stage = stage == kG2Stages - 1 ? 0u : stage + 1u;
    return st;
  };
  for (uint32_t q = 0; q < Kq_full; ++q) quad_math<BM, AW, VT, false>(top(q), q, (uint32_t)a.Kg, a_unit, mask, acc);
  if (Kq_full < Kq) quad_math<BM, AW, VT, true>(top(Kq_full), Kq_full, (uint32_t)a.Kg, a_unit, mask, acc);
  lds_barrier();  // every wave has left the ring before it is reused
}

__global__ __launch_bounds__(kG2Waves * kWave) void gemm_gate_up_kernel(GemmK a) {
  constexpr int BM = kGemmBMGateUp;
  constexpr int TT = BM / 16;
  constexpr int kRows = kG2Waves * 16;  // rows of I per workgroup (kG2Waves / 2 groups)
  __shared__ u32x4 lds_a[kG2Stages * kG2StageUnits];
  __shared__ int s_mb[kMaxExperts + 2];
  __shared__ int64_t s_row[BM];
  __shared__ SegLds s_seg;
  __shared__ int s_nact;
  const int lane = threadIdx.x % kWave;
  const int w = threadIdx.x / kWave;
  const int n = lane % 16;
  const int p = lane / 16;
  if (blockIdx.x == 0) {
    // the all-zero down-operand row read for positions past a segment
    for (int64_t i = threadIdx.x; i < a.KqI * 256; i += blockDim.x) a.hq16[a.h_zero_row * a.KqI * 256 + i] = 0;
  }
  const i32x4 ar = buf_rsrc_words(a.a_src, (uint32_t)((a.a_zero_row + 1) * a.Kq * 256));
  const int n_act = count_active(a.seg, &s_nact);
  seg_to_lds(a.seg, n_act, &s_seg);
  const int64_t n_mb = plan_items<BM>(a.seg.desc, n_act, s_mb);  // its barrier publishes s_seg too
  const int64_t n_nb = ceil_div(a.N, kRows);
  const XcdPlan xp = xcd_plan(n_mb, n_nb);
  const uint32_t nib_bytes = (uint32_t)(a.N * a.Kq * 64), sc_bytes = (uint32_t)(a.N * a.Kq * 8);
  // The XCD's items end in a partial round of r = n_items % nl items, which
  // r of its nl workgroups run while the rest idle.  When 2 r <= nl those r
  // items run as 2 r halves of BM / 2 positions each (still the XCD's last
  // items, so their weights are the ones in its L2): the last round then
  // takes about half an item (at 4096 tokens 8 -> 7.5 item times).
  const int64_t r_last = xp.n_items % xp.nl;
  const int64_t n_split = (r_last > 0 && 2 * r_last <= xp.nl) ? r_last : 0;
  const int64_t n_whole = xp.n_items - n_split;
  for (int64_t ent = xp.l; ent < xp.n_items + n_split; ent += xp.nl) {
    const int64_t item = ent < n_whole ? ent : n_whole + (ent - n_whole) / 2;
    const int part = ent < n_whole ? -1 : (int)((ent - n_whole) % 2);
    const TileCoord c = tile_coord<BM>(a, &s_seg, s_mb, n_act, xp, item, n_nb, s_row, part);
    if (c.m0 >= c.end) continue;  // the empty second half of a block of <= BM / 2 positions
    const int64_t n_tiles = a.N / kRowTile;
    const int64_t t = c.nb * kG2Waves + w;
    const int64_t tc = t < n_tiles ? t : n_tiles - 1;  // a tile past I computes, unstored
    const int64_t t4 = t + 4;                           // wave w + 4's tile, copied by wave w < 4
    const int64_t tc4 = t4 < n_tiles ? t4 : n_tiles - 1;
    const bool routed = c.e < a.seg.E;
    const i32x4 nr[2] = {buf_rsrc_words(routed ? a.nib1 + (int64_t)c.e * nib_bytes : a.sh_nib1, nib_bytes),
                         buf_rsrc_words(routed ? a.nib2 + (int64_t)c.e * nib_bytes : a.sh_nib2, nib_bytes)};
    const i32x4 sr[2] = {
        buf_rsrc_words(routed ? reinterpret_cast<const uint8_t*>(a.sc1) + (int64_t)c.e * sc_bytes
                              : reinterpret_cast<const uint8_t*>(a.sh_sc1), sc_bytes),
        buf_rsrc_words(routed ? reinterpret_cast<const uint8_t*>(a.sc2) + (int64_t)c.e * sc_bytes
                              : reinterpret_cast<const uint8_t*>(a.sh_sc2), sc_bytes)};
    const int64_t rt[2][2] = {{tc, tc}, {tc4, tc4}};
    f32x4 acc[2][TT];
    const f32x4 z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int tt = 0; tt < TT; ++tt) acc[b][tt] = z;
    const int vt = __builtin_amdgcn_readfirstlane((int)ceil_div(c.end - c.m0, (int64_t)16));
    // exactly the tiles that hold a position (a block of 65 positions takes 5
    // tiles, not 8: at about 64 positions an expert, DeepSeek-V3's prefill
    // multiplied half again its positions with rounding to 2, 4 or 8)
    switch (vt) {
      case 1: gemm_tile3<BM, 1, 1, 4>(a, s_row, lds_a, ar, nr, sr, rt, acc); break;
      case 2: gemm_tile3<BM, 1, 2, 4>(a, s_row, lds_a, ar, nr, sr, rt, acc); break;
      case 3: gemm_tile3<BM, 1, 3, 4>(a, s_row, lds_a, ar, nr, sr, rt, acc); break;
      case 4: gemm_tile3<BM, 1, 4, 4>(a, s_row, lds_a, ar, nr, sr, rt, acc); break;
      case 5: gemm_tile3<BM, 1, 5, 4>(a, s_row, lds_a, ar, nr, sr, rt, acc); break;
      case 6: gemm_tile3<BM, 1, 6, 4>(a, s_row, lds_a, ar, nr, sr, rt, acc); break;
      case 7: gemm_tile3<BM, 1, 7, 4>(a, s_row, lds_a, ar, nr, sr, rt, acc); break;
      default: gemm_tile3<BM, 1, 8, 4>(a, s_row, lds_a, ar, nr, sr, rt, acc); break;
    }

    // SwiGLU, then h as the fp16 pair hi + lo into LDS in down-operand chunk
    // order [group of the workgroup][position][part p'][hi 8, lo 8]: element
    // cc = half * 16 + n of a group sits at j' = kmap^-1(p', cc), half = w % 2.
    uint16_t* hs = reinterpret_cast<uint16_t*>(lds_a);
    const int gl = w / 2;  // group of the workgroup this wave's tile belongs to
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
        const float hv = swiglu_fast(acc[0][tt][j], acc[1][tt][j]);
        const uint32_t hb = float_to_half_bits(hv);
        const uint32_t lb = float_to_half_bits(hv - half_bits_to_float32(hb));
        uint16_t* chunk = hs + ((gl * BM + m) * 4 + pp) * 16;
        chunk[jj] = (uint16_t)hb;
        chunk[8 + jj] = (uint16_t)lb;
      }
    }
    lds_barrier();
    // the stores from waves 4-7, which issue no copies (see gemm_tile3): they
    // drain while the next item's copies and MFMAs run
    constexpr int kGroups = kG2Waves / 2;
    constexpr int kStoreThreads = kG2Waves / 2 * kWave;
    for (int cidx = (int)threadIdx.x - kStoreThreads; cidx >= 0 && cidx < kGroups * BM * 4; cidx += kStoreThreads) {
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

__global__ __launch_bounds__(kG2Waves * kWave) void gemm_down_kernel(GemmK a) {
  constexpr int BM = kGemmBMDown;
  constexpr int TT = BM / 16;
  constexpr int NB = kG2NB;
  constexpr int kRows = kG2Waves * 16 * NB;  // rows of H per workgroup
  __shared__ u32x4 lds_a[kG2Stages * kG2StageUnits];
  __shared__ int s_mb[kMaxExperts + 2];
  __shared__ int64_t s_row[BM];
  __shared__ SegLds s_seg;
  __shared__ int s_nact;
  const int lane = threadIdx.x % kWave;
  const int w = threadIdx.x / kWave;
  const int n = lane % 16;
  const int p = lane / 16;
  const i32x4 ar = buf_rsrc_words(a.a_src, (uint32_t)((a.a_zero_row + 1) * a.Kq * 512));
  const int n_act = count_active(a.seg, &s_nact);
  seg_to_lds(a.seg, n_act, &s_seg);
  const int64_t n_mb = plan_items<BM>(a.seg.desc, n_act, s_mb);  // its barrier publishes s_seg too
  const int64_t n_nb = ceil_div(a.N, kRows);
  const int64_t n_tiles = a.N / kRowTile;
  const XcdPlan xp = xcd_plan(n_mb, n_nb);
  const uint32_t nib_bytes = (uint32_t)(a.N * a.Kq * 64), sc_bytes = (uint32_t)(a.N * a.Kq * 8);
  for (int64_t item = xp.l; item < xp.n_items; item += xp.nl) {
    const TileCoord c = tile_coord<BM>(a, &s_seg, s_mb, n_act, xp, item, n_nb, s_row);
    const bool routed = c.e < a.seg.E;
    const i32x4 nw = buf_rsrc_words(routed ? a.nib1 + (int64_t)c.e * nib_bytes : a.sh_nib1, nib_bytes);
    const i32x4 sw = buf_rsrc_words(routed ? reinterpret_cast<const uint8_t*>(a.sc1) + (int64_t)c.e * sc_bytes
                                           : reinterpret_cast<const uint8_t*>(a.sh_sc1), sc_bytes);
    const i32x4 nr[NB] = {nw, nw};
    const i32x4 sr[NB] = {sw, sw};
    // waves 0-3 copy their own operands and wave w + 4's (rt[1])
    int64_t rt[2][NB];
#pragma unroll
    for (int o = 0; o < 2; ++o)
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const int64_t t = (c.nb * kG2Waves + w + 4 * o) * NB + b;
        rt[o][b] = t < n_tiles ? t : n_tiles - 1;  // a tile past H computes, unstored
      }
    f32x4 acc[NB][TT];
    const f32x4 z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int tt = 0; tt < TT; ++tt) acc[b][tt] = z;
    const int vt = __builtin_amdgcn_readfirstlane((int)ceil_div(c.end - c.m0, (int64_t)16));
    switch (vt) {
      case 1: gemm_tile3<BM, 2, 1, 4>(a, s_row, lds_a, ar, nr, sr, rt, acc); break;
      case 2: gemm_tile3<BM, 2, 2, 4>(a, s_row, lds_a, ar, nr, sr, rt, acc); break;
      case 3: gemm_tile3<BM, 2, 3, 4>(a, s_row, lds_a, ar, nr, sr, rt, acc); break;
      default: gemm_tile3<BM, 2, 4, 4>(a, s_row, lds_a, ar, nr, sr, rt, acc); break;
    }
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const int64_t t = (c.nb * kG2Waves + w) * NB + b;
      if (t >= n_tiles) continue;
#pragma unroll
      for (int tt = 0; tt < TT; ++tt) {
        if (tt >= vt) break;
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
  const int64_t max_items = gemm_max_items(x, kGemmBMGateUp, ceil_div(x.I, kG2Waves * 16));
  hipLaunchKernelGGL(gemm_gate_up_kernel, dim3(resident_grid(gemm_gate_up_kernel, kG2Waves * kWave, max_items)),
                     dim3(kG2Waves * kWave), 0, stream, g);
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
  const int64_t max_items = gemm_max_items(x, kGemmBMDown, ceil_div(x.H, kG2Waves * 16 * kG2NB));
  hipLaunchKernelGGL(gemm_down_kernel, dim3(resident_grid(gemm_down_kernel, kG2Waves * kWave, max_items)),
                     dim3(kG2Waves * kWave), 0, stream, g);
  return hipGetLastError();
}

}  // namespace pmoe
