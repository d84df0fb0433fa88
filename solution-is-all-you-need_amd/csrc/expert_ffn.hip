// expert_ffn.hip -- grouped int4 (Q4_0) expert SwiGLU FFN for gfx950, decode
// regime, plus the weighted combine.
//
// Reference operator: kernels/sparse_moe/sparse_matmul.cu:120-215 (gate and up
// projections, h = silu(g) * u in fp32, down projection) with the expert
// weights of python/phantom/loader/gguf_loader.py:362-381 (Q4_0).
//
// Work decomposition.  The router's permute groups tokens per expert into
// segments and writes one descriptor {expert, begin, end} per launch slot
// (expert -1 for slots beyond the active count), and, for the token-tile
// kernels, a table of 16-position token tiles.  Two kernel pairs:
//   K-split (gate_up_kernel, down_kernel): an item is RT 16-row tiles of one
//     segment's expert; up to four waves split K, each loading one or two
//     quads per step, and their partials are summed in LDS in wave order;
//   token-tile (gate_up_tile_kernel, down_tile_kernel): a workgroup copies
//     one token tile's activation operand into LDS once, and each wave
//     streams whole row tiles through a ring of weight chunks in registers.
// Results do not depend on timing.  Every weight byte of an active expert is
// read from HBM once per token tile; later tiles of a long segment mostly
// find it in L2 or the MALL.
//
// Arithmetic per 32-group g, token m, weight row n (see moe_common.h):
//   P = mfma(a_m, 1 + nib_n / 16)               exact products, fp32 sums
//   acc[m][n] += 16 d[n][g] * P                  fp32 FMA
//   corr[m][n] += S[m][g] * d[n][g]              fp32 MFMA over the 4 groups
//   result = acc - 24 * corr = sum_g d * sum_k a_k * (nib_k - 8)
// The gate/up activations x are exact bf16.  The down activations h are fp32;
// the gate/up epilogue stores each h as an fp16 pair hi + lo (|h - hi - lo| <=
// 2^-22 |h|) already in MFMA operand order, plus half-group sums, so the down
// kernel only loads operands (two fp16 MFMAs per group; one in the K-split
// kernel for tiles of at most 8 positions, whose hi and lo share an MFMA as
// adjacent rows).  fp16 bounds |h| to below 65504.
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <type_traits>

#include "expert_common.h"
#include "moe_common.h"
#include "moe_launch.h"

namespace pmoe {

struct GateUpK {
  SegSrc seg;
  int64_t T;  // tokens; row T of xq / xs is the all-zero activation row
  const uint16_t* xq;
  const float* xs;
  const uint8_t* gate_nib;
  const uint16_t* gate_sc;
  const uint8_t* up_nib;
  const uint16_t* up_sc;
  const uint8_t* sh_gate_nib;
  const uint16_t* sh_gate_sc;
  const uint8_t* sh_up_nib;
  const uint16_t* sh_up_sc;
  int64_t I;    // rows of gate/up
  int64_t Kq;   // quads of H
  int64_t KqI;  // quads of I (down operand layout)
  uint16_t* hq; // [rows + 1][KqI][4 p][4 gi][hi, lo][8] fp16 bits; row `zero_row` is zero
  float* hs;    // [rows + 1][KqI * 4 groups][2 halves] sums of hi + lo
  int64_t zero_row;
  const int32_t* tiles;    // token tiles of the segments (router permute), or null
  const int32_t* n_tiles;
};

struct DownK {
  SegSrc seg;
  const uint16_t* hq;
  const float* hs;
  const uint8_t* down_nib;
  const uint16_t* down_sc;
  const uint8_t* sh_down_nib;
  const uint16_t* sh_down_sc;
  int64_t H;         // rows of down
  int64_t I;         // K of down
  int64_t Kq;        // quads of I
  int64_t zero_row;  // hq / hs row that holds zeros
  float* outbuf;
  const int32_t* tiles;  // token tiles of the segments (router permute), or null
  const int32_t* n_tiles;
};

// ------------------------------------------------------------------ gate/up

// Workgroups of up to kGateUpWaves waves loop over items (active expert,
// 16-row tile of I).  Wave ks of the ksplit waves takes quads ks,
// ks + ksplit, ... of K in chunks of NQ, issuing all loads of a chunk at once,
// and contributes a partial tile; partials are summed in LDS in wave order,
// so results do not depend on timing.  The weight addresses depend only on
// the descriptor (wave-uniform), the activation addresses on one token id.
constexpr int kGateUpWaves = 8;

// One 16-row tile, token tiles [m0, m0 + 16 TP) of the segment ending at
// seg_end.  Token tiles are taken TP at a time: each dequantised weight
// operand feeds TP MFMAs, so the nibble expansion is paid once per 16 TP
// tokens.
// A pass is one 16-token tile of RT 16-row tiles of I of one segment.  Each
// wave works a pass one quad of K at a time.  Passes are software-pipelined:
// right after a pass's MFMAs, and before its epilogue, every wave issues the
// loads of the next pass's first chunk, so their latency overlaps the
// cross-wave reduction and the epilogue, and the epilogue's stores (younger
// than those loads) never sit in the wait for them.
struct GUPass {
  int e;             // expert (E = the shared expert)
  int64_t end;       // segment end position
  int64_t m0;        // first position of the tile
  int64_t rt;        // 16-row tile of I
  uint32_t xoff;     // this lane's activation row (times Kq)
};

// One quad of K for RT row tiles: their gate and up nibbles and scales, and
// the 16 tokens' activation operand they share.
template <int RT>
struct GUChunk {
  u32x4 gw[RT], uw[RT];
  uint2 gs[RT], us[RT];
  u32x4 xa[4];
  float sx;
};

template <bool TOK_LDS>
__device__ __attribute__((always_inline)) inline GUPass gu_pass(const GateUpK& a, const int* s_tok, const int4 d, int64_t m0, int64_t rt) {
  GUPass ps;
  ps.e = __builtin_amdgcn_readfirstlane(d.x);
  ps.end = __builtin_amdgcn_readfirstlane(d.z);
  ps.m0 = m0;
  ps.rt = rt;
  // token of the lane's position: from the LDS copy when the kernel made
  // one, else one unconditional global load (clamped index); row T is zero
  const int64_t pm = m0 + threadIdx.x % 16;
  const int64_t pc = pm < ps.end ? pm : ps.end - 1;
  int64_t tv;
  if constexpr (TOK_LDS) tv = s_tok[pc];
  else tv = a.seg.seg_tok[pc];
  ps.xoff = (uint32_t)((pm < ps.end ? tv : a.T) * a.Kq);
  return ps;
}

// Loads of quad q of the pass's RT row tiles (rt0 .. rt0 + RT - 1).
template <int RT>
__device__ __attribute__((always_inline)) inline void gu_load(const GateUpK& a, const GUPass& ps, int64_t q, GUChunk<RT>& c) {
  const int lane = threadIdx.x % kWave;
  const int n = lane % 16;
  const int p = lane / 16;
  const int64_t nib_stride = a.I * a.Kq * 64;
  const int64_t sc_stride = a.I * a.Kq * 4;
  const bool routed = ps.e < a.seg.E;
  const uint8_t* gnib = routed ? a.gate_nib + ps.e * nib_stride : a.sh_gate_nib;
  const uint16_t* gsc = routed ? a.gate_sc + ps.e * sc_stride : a.sh_gate_sc;
  const uint8_t* unib = routed ? a.up_nib + ps.e * nib_stride : a.sh_up_nib;
  const uint16_t* usc = routed ? a.up_sc + ps.e * sc_stride : a.sh_up_sc;
  // Wave-uniform bases plus 32-bit lane offsets: each load is one SGPR-base
  // access with a single VGPR offset instead of a per-lane 64-bit address.
  const uint32_t o_nib = (uint32_t)lane * 16u;
  const uint32_t o_sc = (uint32_t)n * 8u;
#pragma unroll
  for (int r = 0; r < RT; ++r) {
    const int64_t tq = (ps.rt + r) * a.Kq + q;  // wave-uniform
    const char* gb = uniform_ptr(reinterpret_cast<const char*>(gnib) + tq * kQuadNibBytes);
    const char* ub = uniform_ptr(reinterpret_cast<const char*>(unib) + tq * kQuadNibBytes);
    const char* gsb = uniform_ptr(reinterpret_cast<const char*>(gsc) + tq * kQuadScales * 2);
    const char* usb = uniform_ptr(reinterpret_cast<const char*>(usc) + tq * kQuadScales * 2);
    // explicitly global: the routed / shared pointer select would make these
    // flat loads, after which every wait is a wait for all outstanding loads
    c.gw[r] = gload_nt<u32x4>(gb + o_nib);
    c.uw[r] = gload_nt<u32x4>(ub + o_nib);
    c.gs[r] = gload_u2(gsb + o_sc);
    c.us[r] = gload_u2(usb + o_sc);
  }
  // Positions past the segment read the all-zero row T.  (Buffer loads with
  // an out-of-range offset for them, which return zeros without a memory
  // access, were slower here: DeepSeek-V3 8 tokens gate/up 183 -> 214 us,
  // 64 tokens 724 -> 809 us.)
  const uint32_t xrow = ps.xoff + (uint32_t)q;  // (token, quad) row of xq / xs
  const char* xb = reinterpret_cast<const char*>(a.xq);
  const uint32_t o_x = (xrow * 16u + (uint32_t)p * 4u) * 16u;
#pragma unroll
  for (int gi = 0; gi < 4; ++gi) c.xa[gi] = *reinterpret_cast<const u32x4*>(xb + (o_x + gi * 16u));
  c.sx = *reinterpret_cast<const float*>(reinterpret_cast<const char*>(a.xs) + (xrow * 4u + (uint32_t)p) * 4u);
}

template <int RT>
__device__ __attribute__((always_inline)) inline void gu_math(const GUChunk<RT>& c, f32x4 (&ag)[RT], f32x4 (&au)[RT], f32x4 (&cg)[RT],
                               f32x4 (&cu)[RT]) {
  const int p = (threadIdx.x % kWave) / 16;
  const uint32_t mask = vgpr_const(0x00780078u);
  const f32x4 z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int r = 0; r < RT; ++r) {
    float dg[4], du[4];
    unpack_scales(c.gs[r], dg);
    unpack_scales(c.us[r], du);
    const uint32_t gwv[4] = {c.gw[r].x, c.gw[r].y, c.gw[r].z, c.gw[r].w};
    const uint32_t uwv[4] = {c.uw[r].x, c.uw[r].y, c.uw[r].z, c.uw[r].w};
#pragma unroll
    for (int gi = 0; gi < 4; ++gi) {
      const u32x4 bg = dequant_unit_bf16(gwv[gi], mask);
      const u32x4 bu = dequant_unit_bf16(uwv[gi], mask);
      ag[r] += dg[gi] * mfma_bf16_16x16x32(c.xa[gi], bg, z);
      au[r] += du[gi] * mfma_bf16_16x16x32(c.xa[gi], bu, z);
    }
    cg[r] = mfma_f32_16x16x4(c.sx, dg[p], cg[r]);
    cu[r] = mfma_f32_16x16x4(c.sx, du[p], cu[r]);
  }
}

// SwiGLU of the pass from the wave partials in red, written as the down
// kernel's operand: fp16 pair hi + lo of h in MFMA operand order, plus the
// half-group sums of hi + lo.
template <int RT>
__device__ __attribute__((always_inline)) inline void gu_epilogue(const GateUpK& a, const GUPass& ps, float (*red)[RT][2][16][16]) {
  const int ksplit = blockDim.x / kWave;
  for (int o = threadIdx.x; o < RT * 256; o += blockDim.x) {
    const int r = o / 256;
    const int mm = (o % 256) / 16;
    const int nn = o % 16;
    float g = 0.0f, uu = 0.0f;
    for (int s2 = 0; s2 < ksplit; ++s2) {
      g += red[s2][r][0][mm][nn];
      uu += red[s2][r][1][mm][nn];
    }
    const float h = g * (1.0f / (1.0f + expf(-g))) * uu;
    const uint32_t hb = float_to_half_bits(h);
    const float hf = half_bits_to_float32(hb);
    const uint32_t lb = float_to_half_bits(h - hf);
    const float lf = half_bits_to_float32(lb);
    const int64_t pos = ps.m0 + mm;
    const bool ok = pos < ps.end;
    const int64_t i = (ps.rt + r) * 16 + nn;
    const int64_t g32 = i / kGroup;
    const int cc = (int)(i % kGroup);
    const int half = cc / 16;
    const int pp = (cc % 16) / 4;
    const int rr = cc % 4;
    // kmap(p, j) = 4p + {0, 2, 16, 18, 1, 3, 17, 19}[j], inverted per half
    const int j = half == 0 ? ((rr & 1) ? 4 : 0) + (rr >> 1) : ((rr & 1) ? 6 : 2) + (rr >> 1);
    if (ok) {
      uint16_t* dst = a.hq + (((pos * a.KqI + g32 / 4) * 16 + pp * 4 + (g32 % 4)) * 16);
      dst[j] = (uint16_t)hb;
      dst[8 + j] = (uint16_t)lb;
    }
    // The tile's 16 rows are one half of one group: sum hi + lo over them
    // (16 consecutive lanes, fixed butterfly order).
    float sum = hf + lf;
    sum += __shfl_xor(sum, 8, kWave);
    sum += __shfl_xor(sum, 4, kWave);
    sum += __shfl_xor(sum, 2, kWave);
    sum += __shfl_xor(sum, 1, kWave);
    if (nn == 0 && ok) a.hs[(pos * a.KqI * 4 + g32) * 2 + half] = sum;
  }
}

// Segment-position token ids kept in LDS when they fit (decode batches).
constexpr int kTokLds = 2048;

template <int RT, bool TOK_LDS>
__global__ __launch_bounds__(kGateUpWaves * kWave, RT == 1 ? 4 : 2) void gate_up_kernel(GateUpK a) {
  __shared__ float red[kGateUpWaves][RT][2][16][16];  // [wave][row tile][gate/up]
  __shared__ int4 s_desc[kMaxExperts + 1];
  __shared__ int s_tok[TOK_LDS ? kTokLds : 1];
  __shared__ int s_nact;
  const int lane = threadIdx.x % kWave;
  const int ks = threadIdx.x / kWave;
  const int ksplit = blockDim.x / kWave;
  const int n = lane % 16;
  const int p = lane / 16;
  if (blockIdx.x == 0) {
    // the all-zero down-operand row read for positions past a segment
    for (int64_t i = threadIdx.x; i < a.KqI * 256; i += blockDim.x) a.hq[a.zero_row * a.KqI * 256 + i] = 0;
    for (int64_t i = threadIdx.x; i < a.KqI * 8; i += blockDim.x) a.hs[a.zero_row * a.KqI * 8 + i] = 0.0f;
  }
  // descriptors and (when they fit) the positions' tokens, in one round trip
  const int n_act = load_descriptors(a.seg, s_desc, &s_nact, TOK_LDS ? s_tok : nullptr, TOK_LDS ? a.zero_row : 0);
  const int64_t n_blk = a.I / (kRowTile * RT);  // RT-tile blocks of I per expert
  const int64_t n_items = (int64_t)n_act * n_blk;
  int64_t item = blockIdx.x;
  if (item >= n_items) return;
  // this wave's quads of K: ks, ks + ksplit, ... (nch of them)
  const int64_t nch = ks < a.Kq ? (a.Kq - ks + ksplit - 1) / ksplit : 0;
  GUPass ps = gu_pass<TOK_LDS>(a, s_tok, s_desc[item / n_blk], s_desc[item / n_blk].y, (item % n_blk) * RT);
  GUChunk<RT> ck;
  if (nch > 0) gu_load<RT>(a, ps, ks, ck);
  for (;;) {
    const f32x4 z = {0.f, 0.f, 0.f, 0.f};
    f32x4 ag[RT], au[RT], cg[RT], cu[RT];
#pragma unroll
    for (int r = 0; r < RT; ++r) ag[r] = au[r] = cg[r] = cu[r] = z;
    for (int64_t c = 0; c < nch; ++c) {
      gu_math<RT>(ck, ag, au, cg, cu);
      if (c + 1 < nch) gu_load<RT>(a, ps, ks + (c + 1) * ksplit, ck);
    }
#pragma unroll
    for (int r = 0; r < RT; ++r) {
      // sum_g d * sum_k a (n - 8) = 16 * sum_g d P - 24 * sum_g d S
      const f32x4 rg = kUnitScale * ag[r] - kUnitBias * cg[r];
      const f32x4 ru = kUnitScale * au[r] - kUnitBias * cu[r];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        red[ks][r][0][4 * p + j][n] = rg[j];
        red[ks][r][1][4 * p + j][n] = ru[j];
      }
    }
    __syncthreads();
    // next pass: the segment's next token tile, else the next item
    GUPass nx = ps;
    bool more = true;
    if (ps.m0 + 16 < ps.end) {
      nx = gu_pass<TOK_LDS>(a, s_tok, s_desc[item / n_blk], ps.m0 + 16, ps.rt);
    } else {
      item += gridDim.x;
      more = item < n_items;
      if (more)
        nx = gu_pass<TOK_LDS>(a, s_tok, s_desc[item / n_blk], s_desc[item / n_blk].y, (item % n_blk) * RT);
    }
    if (more && nch > 0) gu_load<RT>(a, nx, ks, ck);
    gu_epilogue<RT>(a, ps, red);
    __syncthreads();
    if (!more) break;
    ps = nx;
  }
}

// ------------------------------------------------------- gate/up, token tiles
//
// A workgroup takes one token tile of the router's tile table (16 positions
// of one segment) and a block of its 16-row tiles of I.  It gathers the
// tile's activation operand for all of K into LDS once, in MFMA operand order
// ([quad][group][lane] 16-byte pieces, conflict-free reads), with
// direct-to-LDS loads, so neighbouring waves no longer each gather the same
// 16 scattered token rows per quad.  Each wave owns whole row tiles (all of K,
// no cross-wave reduction) and streams their weights through a ring of D
// chunk buffers in registers: after the math of chunk j it issues the loads
// of chunk j + D, which may belong to its next row tile.  Loads go through
// buffer resources, so a chunk costs no vector address arithmetic.
// Two workgroups fit a CU's LDS at H = 2048, so two waves per SIMD: the
// register budget is 256.
constexpr int kTileWaves = 4;

struct WChunk {  // one quad of one row tile: gate and up nibbles and scales
  u32x4 gw, uw;
  uint2 gs, us;
};

struct WSrc {  // weight resources of one expert
  BufRsrc g, u, gs, us;
};

__device__ __attribute__((always_inline)) inline void wchunk_load(const WSrc& s, uint32_t tq_in, WChunk& c) {
  // wave-uniform already; the compiler is told so (a buffer offset it takes
  // for divergent would be issued once per distinct value)
  const uint32_t tq = (uint32_t)__builtin_amdgcn_readfirstlane((int)tq_in);
  const int lane = threadIdx.x % kWave;
  const uint32_t o_nib = (uint32_t)lane * 16u;
  const uint32_t o_sc = (uint32_t)(lane % 16) * 8u;
  c.gw = buf_load_b128_nt(s.g, o_nib, tq * kQuadNibBytes);
  c.uw = buf_load_b128_nt(s.u, o_nib, tq * kQuadNibBytes);
  c.gs = buf_load_b64(s.gs, o_sc, tq * (kQuadScales * 2));
  c.us = buf_load_b64(s.us, o_sc, tq * (kQuadScales * 2));
}

// The math of gu_math for one row tile, the activation operand of quad q
// read from LDS.
__device__ __attribute__((always_inline)) inline void wchunk_math(const WChunk& c, const u32x4* s_xq, const float* s_sxq,
                                                                  f32x4& ag, f32x4& au, f32x4& cg, f32x4& cu) {
  const int lane = threadIdx.x % kWave;
  const int p = lane / 16;
  const uint32_t mask = vgpr_const(0x00780078u);
  const f32x4 z = {0.f, 0.f, 0.f, 0.f};
  float dg[4], du[4];
  unpack_scales(c.gs, dg);
  unpack_scales(c.us, du);
  const uint32_t gwv[4] = {c.gw.x, c.gw.y, c.gw.z, c.gw.w};
  const uint32_t uwv[4] = {c.uw.x, c.uw.y, c.uw.z, c.uw.w};
  // all eight MFMAs first, then their scaling: an FMA right behind the MFMA
  // whose result it reads would stall the wave for the MFMA's latency
  f32x4 pg[4], pu[4];
#pragma unroll
  for (int gi = 0; gi < 4; ++gi) {
    const u32x4 xa = s_xq[gi * kWave + lane];
    pg[gi] = mfma_bf16_16x16x32(xa, dequant_unit_bf16(gwv[gi], mask), z);
    pu[gi] = mfma_bf16_16x16x32(xa, dequant_unit_bf16(uwv[gi], mask), z);
  }
#pragma unroll
  for (int gi = 0; gi < 4; ++gi) {
    ag += dg[gi] * pg[gi];
    au += du[gi] * pu[gi];
  }
  const float sx = s_sxq[lane];
  cg = mfma_f32_16x16x4(sx, dg[p], cg);
  cu = mfma_f32_16x16x4(sx, du[p], cu);
}

// SwiGLU of one row tile rt of the token tile [m0, end) from the wave's own
// accumulators (lane (n, p) holds positions m0 + 4p + j of row n), stored as
// the down kernel's operand.
__device__ inline void tile_epilogue(const GateUpK& a, BufRsrc hqr, BufRsrc hsr, int64_t m0, int64_t end, uint32_t rt,
                                     const f32x4& ag, const f32x4& au, const f32x4& cg, const f32x4& cu) {
  const int lane = threadIdx.x % kWave;
  const int n = lane % 16;
  const int p = lane / 16;
  const uint32_t pos_bytes = (uint32_t)(a.KqI * 512);  // hq bytes per position
  const f32x4 rg = kUnitScale * ag - kUnitBias * cg;
  const f32x4 ru = kUnitScale * au - kUnitBias * cu;
  const uint32_t i = rt * 16u + (uint32_t)n;  // row of I
  const uint32_t g32 = i / kGroup;
  const int half = (int)((i % kGroup) / 16);
  const int pp = n / 4, rr = n % 4;
  // kmap(p, j) = 4p + {0, 2, 16, 18, 1, 3, 17, 19}[j], inverted per half
  const int j = half == 0 ? ((rr & 1) ? 4 : 0) + (rr >> 1) : ((rr & 1) ? 6 : 2) + (rr >> 1);
  const uint32_t o_row = ((((g32 / 4) * 16 + pp * 4 + (g32 % 4)) * 16) + j) * 2;
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) {
    const float g = rg[jj], u = ru[jj];
    const float h = g * (1.0f / (1.0f + expf(-g))) * u;
    const uint32_t hb = float_to_half_bits(h);
    const float hf = half_bits_to_float32(hb);
    const uint32_t lb = float_to_half_bits(h - hf);
    const float lf = half_bits_to_float32(lb);
    const int64_t pos = m0 + 4 * p + jj;
    const bool ok = pos < end;
    const uint32_t o = (uint32_t)pos * pos_bytes + o_row;
    if (ok) {
      __builtin_amdgcn_raw_buffer_store_b16((unsigned short)hb, hqr, (int)o, 0, 0);
      __builtin_amdgcn_raw_buffer_store_b16((unsigned short)lb, hqr, (int)(o + 16u), 0, 0);
    }
    // the 16 rows of the tile are one half of one group: sum hi + lo over
    // them (16 consecutive lanes, fixed butterfly order)
    float sum = hf + lf;
    sum += __shfl_xor(sum, 8, kWave);
    sum += __shfl_xor(sum, 4, kWave);
    sum += __shfl_xor(sum, 2, kWave);
    sum += __shfl_xor(sum, 1, kWave);
    if (n == 0 && ok)
      __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, sum), hsr,
                                            (int)((((uint32_t)pos * (uint32_t)a.KqI * 4u + g32) * 2u + half) * 4u), 0, 0);
  }
}

// Dynamic LDS: x operand [Kq][4 groups][64 lanes] x 16 bytes, then group sums
// [Kq][64 lanes] floats.
inline size_t tile_lds_bytes(int64_t Kq) { return (size_t)Kq * (256 * 16 + 64 * 4); }

// Job geometry of a token-tile launch: row tiles per job, at most M per wave,
// and jobs per token tile, chosen so that the jobs about fill `slots`
// workgroups.
struct TileJobs {
  uint32_t M, per_job, jpt, n_jobs;
};

__device__ inline TileJobs tile_jobs(uint32_t n_tiles, uint32_t n_rt, uint32_t slots, uint32_t nw = kTileWaves,
                                     bool flex = true) {
  TileJobs j;
  if (!flex) {
    // jobs of whole rounds of nw row tiles (M per wave), about `slots` of them
    // (the down projection measured 1% faster so than with flex jobs)
    const uint32_t M = (n_tiles * n_rt + nw * slots - 1) / (nw * slots);
    j.M = M < 1 ? 1 : M;
    j.per_job = nw * j.M;
    j.jpt = (n_rt + j.per_job - 1) / j.per_job;
    j.n_jobs = n_tiles * j.jpt;
    return j;
  }
  // row tiles per job: as few as keep the jobs within one round of the slots
  // (jobs per tile <= slots / tiles), at least one per wave and not
  // necessarily a multiple of nw (then the first waves take one row tile
  // more), so that the jobs fill the slots (Mixtral at 16 tokens: 256 jobs of
  // 28 row tiles rather than 224 of 32)
  const uint32_t jmax = n_tiles ? slots / n_tiles : 1;
  uint32_t pj = jmax ? (n_rt + jmax - 1) / jmax : n_rt;
  if (pj < nw) pj = nw;
  if (pj > n_rt) pj = n_rt;
  j.per_job = pj;
  j.M = (pj + nw - 1) / nw;
  j.jpt = (n_rt + j.per_job - 1) / j.per_job;
  j.n_jobs = n_tiles * j.jpt;
  return j;
}

// One gate/up job: token tile gt, row tiles part * per_job + w + NW * i for
// wave w, up to the job's end (part + 1) * per_job or the last row tile.
// Ends with the waves' last stores issued and LDS still in use; the caller
// synchronises before the next job.
template <int D, int NW = kTileWaves>
__device__ __attribute__((always_inline)) inline void gate_up_tile_job(const GateUpK& a, u32x4* s_x, float* s_sx, uint32_t gt,
                                                                       uint32_t part, const TileJobs& jb) {
  const int lane = threadIdx.x % kWave;
  const int p = lane / 16;
  const uint32_t w = (uint32_t)__builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const uint32_t Kq = (uint32_t)a.Kq;
  const uint32_t n_rt = (uint32_t)(a.I / kRowTile);
  const BufRsrc xr = buf_rsrc(a.xq, (uint32_t)((a.T + 1) * a.Kq * 256));
  const BufRsrc xsr = buf_rsrc(a.xs, (uint32_t)((a.T + 1) * a.Kq * 16));
  const BufRsrc hqr = buf_rsrc(a.hq, (uint32_t)((a.zero_row + 1) * a.KqI * 512));
  const BufRsrc hsr = buf_rsrc(a.hs, (uint32_t)((a.zero_row + 1) * a.KqI * 32));
  const uint32_t nib_bytes = (uint32_t)(a.I * a.Kq * 64);
  const uint32_t sc_bytes = (uint32_t)(a.I * a.Kq * 8);

  const int32_t* tw = a.tiles + (int64_t)gt * kTileWords;
  const int tok_w = tw[4 + lane % 16];
  const int e = __builtin_amdgcn_readfirstlane(tw[0]);
  const int64_t m0 = __builtin_amdgcn_readfirstlane(tw[1]);
  const int64_t end = __builtin_amdgcn_readfirstlane(tw[2]);
  // token of the lane's A-operand row; positions past the segment read the
  // all-zero row T
  const int tok = m0 + lane % 16 < end ? tok_w : (int)a.T;
  const bool routed = e < a.seg.E;
  WSrc ws;
  ws.g = buf_rsrc(routed ? a.gate_nib + (int64_t)e * nib_bytes : a.sh_gate_nib, nib_bytes);
  ws.u = buf_rsrc(routed ? a.up_nib + (int64_t)e * nib_bytes : a.sh_up_nib, nib_bytes);
  ws.gs = buf_rsrc(routed ? reinterpret_cast<const uint8_t*>(a.gate_sc) + (int64_t)e * sc_bytes
                          : reinterpret_cast<const uint8_t*>(a.sh_gate_sc), sc_bytes);
  ws.us = buf_rsrc(routed ? reinterpret_cast<const uint8_t*>(a.up_sc) + (int64_t)e * sc_bytes
                          : reinterpret_cast<const uint8_t*>(a.sh_up_sc), sc_bytes);
  // this wave's row tiles: rt0 + NW * i, i < n_mine
  const uint32_t rt0 = part * jb.per_job + w;
  const uint32_t lim = part * jb.per_job + jb.per_job < n_rt ? part * jb.per_job + jb.per_job : n_rt;
  const uint32_t n_mine = rt0 < lim ? (lim - rt0 + NW - 1) / NW : 0;
  const int64_t total = (int64_t)n_mine * Kq;  // chunks of this wave in this job

  // the tile's activation operand -> LDS (every wave takes a share)
  {
    const uint32_t row = (uint32_t)tok * Kq;
    const uint32_t xv = row * 256u + (uint32_t)p * 64u;
    const uint32_t sv = row * 16u + (uint32_t)p * 4u;
    for (uint32_t b = w; b < Kq * 4; b += NW)
      dma_b128(xr, s_x + b * kWave, xv, (b / 4) * 256u + (b % 4) * 16u);
    for (uint32_t q = w; q < Kq; q += NW) dma_b32(xsr, s_sx + q * kWave, sv, q * 16u);
  }
  asm volatile("" ::: "memory");  // the operand loads stay older than the weight loads below

  // ring prologue (the load cursor stops at the last chunk; refills past
  // the end reload it and are never used)
  uint32_t li = 0, lq = 0;
  int64_t loaded = 0;
  auto advance = [&]() {
    if (loaded + 1 < total) {
      ++loaded;
      if (++lq == Kq) {
        lq = 0;
        ++li;
      }
    }
  };
  WChunk buf[D];
  if (total > 0) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      wchunk_load(ws, (rt0 + NW * li) * Kq + lq, buf[d]);
      advance();
    }
    // the DMA is older than the D chunks just issued
    wait_vmcnt<4 * D>();
  } else {
    wait_vmcnt<0>();
  }
  // every wave's share of the operand is in LDS; no LDS access may move
  // across the barrier
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");

  uint32_t ci = 0, cq = 0;
  const f32x4 z = {0.f, 0.f, 0.f, 0.f};
  f32x4 ag = z, au = z, cg = z, cu = z;
  auto consume = [&](WChunk& c, bool refill) {
    wchunk_math(c, s_x + cq * 256, s_sx + cq * kWave, ag, au, cg, cu);
    if (refill) {
      wchunk_load(ws, (rt0 + NW * li) * Kq + lq, c);
      advance();
    }
    if (++cq == Kq) {
      tile_epilogue(a, hqr, hsr, m0, end, rt0 + NW * ci, ag, au, cg, cu);
      ag = au = cg = cu = z;
      cq = 0;
      ++ci;
    }
  };
  const int64_t n_full = total / D;
  for (int64_t j = 0; j < n_full; ++j) {
#pragma unroll
    for (int d = 0; d < D; ++d) consume(buf[d], true);
  }
  const int rem = (int)(total - n_full * D);
#pragma unroll
  for (int d = 0; d < D - 1; ++d)
    if (d < rem) consume(buf[d], false);
}

template <int D, int NW>
__global__ __launch_bounds__(NW * kWave) __attribute__((amdgpu_waves_per_eu(2))) void gate_up_tile_kernel(GateUpK a) {
  extern __shared__ u32x4 s_x[];
  float* s_sx = reinterpret_cast<float*>(s_x + (uint32_t)a.Kq * 256);
  if (blockIdx.x == 0) {
    // the all-zero down-operand row read for positions past a segment
    for (int64_t i = threadIdx.x; i < a.KqI * 256; i += blockDim.x) a.hq[a.zero_row * a.KqI * 256 + i] = 0;
    for (int64_t i = threadIdx.x; i < a.KqI * 8; i += blockDim.x) a.hs[a.zero_row * a.KqI * 8 + i] = 0.0f;
  }
  const uint32_t n_tiles = (uint32_t)__builtin_amdgcn_readfirstlane(*a.n_tiles);
  const TileJobs jb = tile_jobs(n_tiles, (uint32_t)(a.I / kRowTile), gridDim.x, NW);
  for (uint32_t job = blockIdx.x; job < jb.n_jobs; job += gridDim.x) {
    const uint32_t gt = job / jb.jpt;
    gate_up_tile_job<D, NW>(a, s_x, s_sx, gt, job - gt * jb.jpt, jb);
    __syncthreads();  // the operand is read by every wave before the next job overwrites it
  }
}

// ------------------------------------------------------------------ down

// Same decomposition as gate_up_kernel with RT 16-row tiles of H per item:
// the activation operand of a quad (16 positions x 128 of I as fp16 hi/lo)
// is loaded once and used for all RT tiles.  Positions past the segment
// read zeros.
constexpr int kDownWaves = 4;

template <int NQ, int RT>
__device__ inline void down_item(const DownK& a, const int4 d, const int64_t rt0, float (*red)[RT][16][16]) {
  const int lane = threadIdx.x % kWave;
  const int ks = threadIdx.x / kWave;
  const int ksplit = blockDim.x / kWave;
  const int n = lane % 16;
  const int p = lane / 16;
  const int e = __builtin_amdgcn_readfirstlane(d.x);
  const int64_t beg = __builtin_amdgcn_readfirstlane(d.y);
  const int64_t end = __builtin_amdgcn_readfirstlane(d.z);
  const int64_t nib_stride = a.H * a.Kq * 64;
  const int64_t sc_stride = a.H * a.Kq * 4;
  const uint8_t* dnib = e < a.seg.E ? a.down_nib + e * nib_stride : a.sh_down_nib;
  const uint16_t* dsc = e < a.seg.E ? a.down_sc + e * sc_stride : a.sh_down_sc;
  const int64_t Kg = a.I / kGroup;
  const u32x4 zero = {0u, 0u, 0u, 0u};
  const uint32_t mask = vgpr_const(0x03C003C0u);

  // the operand through buffer resources over this segment's positions only
  // (its size is then far below 4 GiB whatever the layer's; the launch
  // checks it), positions past the segment reading zeros from beyond the
  // buffer instead of the all-zero row, with no memory access (DeepSeek-V3
  // 8 tokens 133.4 -> 131.9 us, 64 tokens 529.5 -> 524.7)
  const BufRsrc hqr = buf_rsrc(a.hq + beg * a.Kq * 256, (uint32_t)((end - beg) * a.Kq * 512));
  const BufRsrc hsr = buf_rsrc(a.hs + beg * a.Kq * 8, (uint32_t)((end - beg) * a.Kq * 32));
  // One 16-position tile [m0, min(m0 + 16, end)).  With PK (at most 8
  // positions) MFMA row 2i holds the fp16 hi of position m0 + i and row
  // 2i + 1 its lo, so a group takes one operand load and one MFMA instead of
  // two of each; the group-sum correction sits in the hi rows, and each
  // position's output adds its two rows.
  auto tile = [&](int64_t m0, auto pk) {
    constexpr bool PK = decltype(pk)::value;
    const int64_t pm0 = PK ? m0 + n / 2 : m0 + n;
    const bool preal = pm0 < end;
    const uint32_t pm = (uint32_t)(preal ? pm0 - beg : 0);  // position within the segment
    const uint32_t hsel = PK ? (uint32_t)(n & 1) : 0u;  // PK: this row's half (0 hi, 1 lo)
    const f32x4 z = {0.f, 0.f, 0.f, 0.f};
    f32x4 acc[RT], corr[RT];
#pragma unroll
    for (int r = 0; r < RT; ++r) acc[r] = corr[r] = z;
    for (int64_t q0 = ks; q0 < a.Kq; q0 += (int64_t)NQ * ksplit) {
      u32x4 bw[NQ][RT];
      uint2 bs[NQ][RT];
      u32x4 ah[NQ][4], al[NQ][PK ? 1 : 4];
      float sp[NQ];
      bool qok[NQ];
#pragma unroll
      for (int i = 0; i < NQ; ++i) {
        int64_t q = q0 + (int64_t)i * ksplit;
        qok[i] = q < a.Kq;
        q = qok[i] ? q : a.Kq - 1;
#pragma unroll
        for (int r = 0; r < RT; ++r) {
          const int64_t tq = (rt0 + r) * a.Kq + q;  // wave-uniform
          bw[i][r] = gload_nt<u32x4>(dnib + (tq * kWave + lane) * 16);
          bs[i][r] = *reinterpret_cast<const uint2*>(dsc + tq * kQuadScales + n * 4);
        }
        const uint32_t o_h = preal ? ((pm * (uint32_t)a.Kq + (uint32_t)q) * 16u + (uint32_t)p * 4u) * 32u : kOutOfRange;
        const uint32_t o_s = preal && hsel == 0u
                                 ? ((pm * (uint32_t)a.Kq * 4u + 4u * (uint32_t)q + (uint32_t)p) * 2u) * 4u
                                 : kOutOfRange;
#pragma unroll
        for (int gi = 0; gi < 4; ++gi) {
          const bool real = 4 * q + gi < Kg;  // padded groups hold no h
          if constexpr (PK) {
            const u32x4 v = buf_load_b128(hqr, o_h + ((uint32_t)(2 * gi) + hsel) * 16u, 0);
            ah[i][gi] = real ? v : zero;
          } else {
            const u32x4 h = buf_load_b128(hqr, o_h + (uint32_t)(2 * gi) * 16u, 0);
            const u32x4 l = buf_load_b128(hqr, o_h + (uint32_t)(2 * gi + 1) * 16u, 0);
            ah[i][gi] = real ? h : zero;
            al[i][gi] = real ? l : zero;
          }
        }
        const uint2 hs2 = buf_load_b64(hsr, o_s, 0);
        const float s0 = __builtin_bit_cast(float, hs2.x), s1 = __builtin_bit_cast(float, hs2.y);
        sp[i] = (4 * q + p < Kg) ? s0 + s1 : 0.0f;
      }
      // per-chunk partials, added to the totals once (short fp32 chains)
      f32x4 part[RT];
#pragma unroll
      for (int r = 0; r < RT; ++r) part[r] = z;
#pragma unroll
      for (int i = 0; i < NQ; ++i) {
        if (!qok[i]) continue;
#pragma unroll
        for (int r = 0; r < RT; ++r) {
          float dv[4];
          unpack_scales(bs[i][r], dv);
          const uint32_t bwv[4] = {bw[i][r].x, bw[i][r].y, bw[i][r].z, bw[i][r].w};
#pragma unroll
          for (int gi = 0; gi < 4; ++gi) {
            const u32x4 bb = dequant_unit_f16(bwv[gi], mask);
            f32x4 pp = mfma_f16_16x16x32(ah[i][gi], bb, z);
            if constexpr (!PK) pp = mfma_f16_16x16x32(al[i][gi], bb, pp);
            part[r] += dv[gi] * pp;
          }
          corr[r] = mfma_f32_16x16x4(sp[i], dv[p], corr[r]);
        }
      }
#pragma unroll
      for (int r = 0; r < RT; ++r) acc[r] += part[r];
    }
#pragma unroll
    for (int r = 0; r < RT; ++r) {
      const f32x4 res = kUnitScale * acc[r] - kUnitBias * corr[r];
      if constexpr (PK) {
        // rows 4p, 4p + 1 are position 2p's hi and lo, rows 4p + 2, 4p + 3
        // position 2p + 1's
        red[ks][r][2 * p][n] = res[0] + res[1];
        red[ks][r][2 * p + 1][n] = res[2] + res[3];
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) red[ks][r][4 * p + j][n] = res[j];
      }
    }
    __syncthreads();
    for (int o = threadIdx.x; o < RT * 256; o += blockDim.x) {
      const int r = o / 256;
      const int mm = (o % 256) / 16;
      const int nn = o % 16;
      float y = 0.0f;
      for (int s2 = 0; s2 < ksplit; ++s2) y += red[s2][r][mm][nn];
      if (m0 + mm < end) a.outbuf[(m0 + mm) * a.H + (rt0 + r) * 16 + nn] = y;
    }
    __syncthreads();
  };
  for (int64_t m0 = beg; m0 < end; m0 += 16) {
    if (end - m0 <= 8) tile(m0, std::true_type{});
    else tile(m0, std::false_type{});
  }
}

template <int NQ, int RT>
__global__ __launch_bounds__(kDownWaves * kWave) void down_kernel(DownK a) {
  __shared__ float red[kDownWaves][RT][16][16];
  __shared__ int4 s_desc[kMaxExperts + 1];
  __shared__ int s_nact;
  const int n_act = load_descriptors(a.seg, s_desc, &s_nact);
  const int64_t n_items = a.H / (kRowTile * RT);
  for (int64_t item = blockIdx.x; item < (int64_t)n_act * n_items; item += gridDim.x)
    down_item<NQ, RT>(a, s_desc[item / n_items], (item % n_items) * RT, red);
}

// --------------------------------------------------------- down, token tiles
//
// As gate_up_tile_kernel, for the down projection: a workgroup takes one token
// tile (16 consecutive segment positions) and a block of the 16-row tiles of
// H.  The tile's activation operand (fp16 hi and lo of h for all of I, plus the
// half-group sums) is copied into LDS once with direct-to-LDS loads, in MFMA
// operand order; each wave streams whole row tiles of W_down (all of I)
// through a ring of D chunks and writes its expert-output rows.  Positions
// past the segment read the all-zero operand row, and groups of the padded
// last quad of I are zeroed at use.
struct DChunk {  // one quad of one row tile of W_down
  u32x4 w;
  uint2 s;
};

// Dynamic LDS: operand [KqI][4 groups][hi, lo][64 lanes] x 16 bytes, then the
// half-group sums [KqI][2 halves][64 lanes] floats.
inline size_t down_tile_lds_bytes(int64_t KqI) { return (size_t)KqI * (8 * 64 * 16 + 2 * 64 * 4); }

// One down job: token tile gt, row tiles of H part * per_job + w + NW * i, up
// to the job's end or the last row tile.
template <int D, int NW = kTileWaves>
__device__ __attribute__((always_inline)) inline void down_tile_job(const DownK& a, u32x4* s_h, float* s_hs, uint32_t gt,
                                                                    uint32_t part, const TileJobs& jb) {
  const int lane = threadIdx.x % kWave;
  const int n = lane % 16;
  const int p = lane / 16;
  const uint32_t w = (uint32_t)__builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const uint32_t Kq = (uint32_t)a.Kq;  // quads of I
  const int64_t Kg = a.I / kGroup;
  const uint32_t n_rt = (uint32_t)(a.H / kRowTile);
  const BufRsrc hqr = buf_rsrc(a.hq, (uint32_t)((a.zero_row + 1) * a.Kq * 512));
  const BufRsrc hsr = buf_rsrc(a.hs, (uint32_t)((a.zero_row + 1) * a.Kq * 32));
  const uint32_t nib_bytes = (uint32_t)(a.H * a.Kq * 64);
  const uint32_t sc_bytes = (uint32_t)(a.H * a.Kq * 8);
  const uint32_t mask = vgpr_const(0x03C003C0u);
  const u32x4 zero4 = {0u, 0u, 0u, 0u};

  const int32_t* tw = a.tiles + (int64_t)gt * kTileWords;
  const int e = __builtin_amdgcn_readfirstlane(tw[0]);
  const int64_t m0 = __builtin_amdgcn_readfirstlane(tw[1]);
  const int64_t end = __builtin_amdgcn_readfirstlane(tw[2]);
  const bool routed = e < a.seg.E;
  const BufRsrc wr = buf_rsrc(routed ? a.down_nib + (int64_t)e * nib_bytes : a.sh_down_nib, nib_bytes);
  const BufRsrc sr = buf_rsrc(routed ? reinterpret_cast<const uint8_t*>(a.down_sc) + (int64_t)e * sc_bytes
                                     : reinterpret_cast<const uint8_t*>(a.sh_down_sc), sc_bytes);
  const uint32_t rt0 = part * jb.per_job + w;
  const uint32_t lim = part * jb.per_job + jb.per_job < n_rt ? part * jb.per_job + jb.per_job : n_rt;
  const uint32_t n_mine = rt0 < lim ? (lim - rt0 + NW - 1) / NW : 0;
  const uint32_t total = n_mine * Kq;

  // the tile's operand -> LDS: block b = (q, gi, h) is one 16-byte piece per
  // lane; the blocks of padded groups (4q + gi >= Kg, only in a ragged last
  // quad of I) are zeroed instead, so the chunk math needs no test
  auto copy_operand = [&]() {
    const int64_t pos = m0 + n < end ? m0 + n : a.zero_row;
    const uint32_t hv = (uint32_t)pos * Kq * 512u + (uint32_t)p * 128u;
    const uint32_t sv = (uint32_t)pos * Kq * 32u + (uint32_t)p * 8u;
    for (uint32_t b = w; b < Kq * 8; b += NW) {
      if (4 * (b / 8) + (b / 2) % 4 < (uint32_t)Kg)
        dma_b128(hqr, s_h + b * kWave, hv, (b / 8) * 512u + ((b / 2) % 4) * 32u + (b % 2) * 16u);
      else
        s_h[b * kWave + lane] = zero4;
    }
    for (uint32_t b = w; b < Kq * 2; b += NW) dma_b32(hsr, s_hs + b * kWave, sv, (b / 2) * 32u + (b % 2) * 4u);
  };
  copy_operand();
  asm volatile("" ::: "memory");  // the operand loads stay older than the weight loads below

  uint32_t li = 0, lq = 0, loaded = 0;
  auto advance = [&]() {
    if (loaded + 1 < total) {
      ++loaded;
      if (++lq == Kq) {
        lq = 0;
        ++li;
      }
    }
  };
  auto load = [&](DChunk& c) {
    const uint32_t tq = (uint32_t)__builtin_amdgcn_readfirstlane((int)((rt0 + NW * li) * Kq + lq));
    c.w = buf_load_b128_nt(wr, (uint32_t)lane * 16u, tq * kQuadNibBytes);
    c.s = buf_load_b64(sr, (uint32_t)n * 8u, tq * (kQuadScales * 2));
  };
  DChunk buf[D];
  if (total > 0) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      load(buf[d]);
      advance();
    }
  }
  if (total > 0) wait_vmcnt<2 * D>();  // the operand copies are older than the D chunks
  else wait_vmcnt<0>();
  lds_barrier();  // this wave's copies and zero stores have landed; so have every other wave's

  uint32_t ci = 0, cq = 0;
  const f32x4 z = {0.f, 0.f, 0.f, 0.f};
  f32x4 acc = z, corr = z;
  auto consume = [&](DChunk& c, bool refill) {
    float dv[4];
    unpack_scales(c.s, dv);
    const uint32_t bwv[4] = {c.w.x, c.w.y, c.w.z, c.w.w};
    const u32x4* hq_q = s_h + cq * 512;
    // the four hi MFMAs, then the four lo ones (each four behind the MFMA it
    // accumulates onto), then the scaling: no instruction waits on the one
    // just issued
    u32x4 bb[4];
    f32x4 pp[4];
#pragma unroll
    for (int gi = 0; gi < 4; ++gi) {
      bb[gi] = dequant_unit_f16(bwv[gi], mask);
      pp[gi] = mfma_f16_16x16x32(hq_q[(gi * 2) * kWave + lane], bb[gi], z);
    }
#pragma unroll
    for (int gi = 0; gi < 4; ++gi) pp[gi] = mfma_f16_16x16x32(hq_q[(gi * 2 + 1) * kWave + lane], bb[gi], pp[gi]);
#pragma unroll
    for (int gi = 0; gi < 4; ++gi) acc += dv[gi] * pp[gi];
    // padded groups' sums (not copied for them) count as zero
    const float sp = 4 * cq + (uint32_t)p < (uint32_t)Kg ? s_hs[(cq * 2) * kWave + lane] + s_hs[(cq * 2 + 1) * kWave + lane] : 0.0f;
    corr = mfma_f32_16x16x4(sp, dv[p], corr);
    if (refill) {
      load(c);
      advance();
    }
    if (++cq == Kq) {
      const f32x4 res = kUnitScale * acc - kUnitBias * corr;
      const uint32_t rt = rt0 + NW * ci;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t pos = m0 + 4 * p + j;
        if (pos < end) a.outbuf[pos * a.H + rt * 16 + n] = res[j];
      }
      acc = corr = z;
      cq = 0;
      ++ci;
    }
  };
  const uint32_t n_full = total / D;
  for (uint32_t j = 0; j < n_full; ++j) {
#pragma unroll
    for (int d = 0; d < D; ++d) consume(buf[d], true);
  }
  const uint32_t rem = total - n_full * D;
#pragma unroll
  for (int d = 0; d < D - 1; ++d)
    if ((uint32_t)d < rem) consume(buf[d], false);
}

template <int D, int NW>
__global__ __launch_bounds__(NW * kWave) __attribute__((amdgpu_waves_per_eu(2))) void down_tile_kernel(DownK a) {
  extern __shared__ u32x4 s_h[];
  float* s_hs = reinterpret_cast<float*>(s_h + (uint32_t)a.Kq * 512);
  const uint32_t n_tiles = (uint32_t)__builtin_amdgcn_readfirstlane(*a.n_tiles);
  const TileJobs jb = tile_jobs(n_tiles, (uint32_t)(a.H / kRowTile), gridDim.x, NW, false);
  for (uint32_t job = blockIdx.x; job < jb.n_jobs; job += gridDim.x) {
    const uint32_t gt = job / jb.jpt;
    down_tile_job<D, NW>(a, s_h, s_hs, gt, job - gt * jb.jpt, jb);
    __syncthreads();  // the operand is read by every wave before the next job overwrites it
  }
}

// y[t] = sum_j w[t,j] * out[slot_pos[t*k+j]] (+ out[T*k + t] for the shared
// expert), j in slot order, fp32.  Slots are taken KB at a time: the KB
// positions and weights are loaded together, then the KB output rows, so a
// token costs two memory round trips per KB slots instead of two per slot.
constexpr int kCombineSlots = 8;

__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ outbuf,
                                                      const int32_t* __restrict__ slot_pos,
                                                      const float* __restrict__ topk_w, int64_t T,
                                                      int k, int64_t H, int has_shared,
                                                      float* __restrict__ y) {
  constexpr int KB = kCombineSlots;
  const int64_t H4 = H / 4;
  const int64_t total = T * H4;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = i / H4;
    const int64_t c = (i % H4) * 4;
    float4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int j0 = 0; j0 < k; j0 += KB) {
      int64_t pos[KB];
      float wt[KB];
#pragma unroll
      for (int jj = 0; jj < KB; ++jj) {
        const int j = j0 + jj < k ? j0 + jj : k - 1;  // clamped: every load unconditional
        pos[jj] = slot_pos[t * k + j];
        wt[jj] = topk_w[t * k + j];
      }
      float4 o[KB];
#pragma unroll
      for (int jj = 0; jj < KB; ++jj) {
        // read once: nontemporal, so the stream does not displace cached lines
        const f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(outbuf + pos[jj] * H + c));
        o[jj] = make_float4(v[0], v[1], v[2], v[3]);
      }
#pragma unroll
      for (int jj = 0; jj < KB; ++jj) {
        if (j0 + jj < k) {
          acc.x += wt[jj] * o[jj].x;
          acc.y += wt[jj] * o[jj].y;
          acc.z += wt[jj] * o[jj].z;
          acc.w += wt[jj] * o[jj].w;
        }
      }
    }
    if (has_shared) {
      const float4 o = *reinterpret_cast<const float4*>(outbuf + (T * k + t) * H + c);
      acc.x += o.x;
      acc.y += o.y;
      acc.z += o.z;
      acc.w += o.w;
    }
    __builtin_nontemporal_store(f32x4{acc.x, acc.y, acc.z, acc.w}, reinterpret_cast<f32x4*>(y + t * H + c));
  }
}

// K split: ksplit waves (at most max_waves) take about two quads each (few
// waves per item keep the cross-wave reduction short; two quads in flight per
// wave keep enough loads outstanding), issued NQ = 2 at a time.
struct Split {
  int ksplit, nq;
};

static Split choose_split(int64_t Kq, int max_waves) {
  Split s;
  const int64_t half = ceil_div(Kq, 2);
  s.ksplit = (int)(half < max_waves ? half : max_waves);
  s.nq = Kq > 1 ? 2 : 1;
  return s;
}

// Optional override "ksplit,rt,nq" for tuning sweeps (read once from the
// environment, see Tuning); unset leaves the shape-chosen tiling.
static void tiling_override(const int t[3], int* ksplit, int* rt, int* nq) {
  if (t[0] == 0) return;
  *ksplit = t[0];
  *rt = t[1];
  *nq = t[2];
}

// The token-tile kernel needs the tile table (written by the permute in the
// decode regime), the tile's operand in LDS, and every buffer it reads or
// writes addressable with 32-bit offsets.
// The K-split kernel can be forced (option PHANTOM_MOE_OPT_DECODE_KSPLIT).
bool gate_up_tile_regime(int64_t T, int64_t H, int64_t I, int E, int k, int has_shared) {
  if (lib_config().force_ksplit) return false;
  const int64_t lim = (int64_t)1 << 31;
  const int64_t Kq = ceil_div(H, kQuad), KqI = ceil_div(I, kQuad);
  const int64_t rows = T * k + (has_shared ? T : 0);
  // one wave per row tile of a token tile: with fewer row tiles than four
  // per CU (a single token, few experts) the K-split kernel fills the chip
  const int64_t row_items = max_token_tiles(T, k, E, has_shared) * (I / kRowTile);
  return row_items >= 4 * (int64_t)device_cus() && tile_lds_bytes(Kq) <= 160 * 1024 && I % kRowTile == 0 &&
         (T + 1) * Kq * 256 < lim && I * Kq * 64 < lim && (rows + 1) * KqI * 512 < lim;
}

static bool tile_fits(const ExpertArgs& x, const GateUpK& g) {
  return g.tiles != nullptr && gate_up_tile_regime(x.T, x.H, x.I, x.E, x.k, x.has_shared);
}

// Ring depth 3, or 2 from rows of 32 quads of H on (a tuning override may set
// 2..4): Qwen3 at 32 tokens (16 quads) 54.2 us a layer with 3 against 54.8
// with 2 or 4; Mixtral at 16 tokens (32 quads) 162.5 with 2 against 164.2
// (165.3 against 166.2 on another box).
static hipError_t launch_gate_up_tile(const ExpertArgs& x, const GateUpK& g, hipStream_t stream) {
  const int depth = tuning().gu_depth ? tuning().gu_depth : (g.Kq >= 32 ? 2 : 3);
  // Eight waves per workgroup, one workgroup per CU (two waves per SIMD, as
  // with two 4-wave workgroups): each CU copies a tile's operand to LDS once
  // rather than twice (Qwen3 shapes, 32 tokens: 24.5 -> 23.7 us).
  constexpr int nw = 8;
  const size_t lds = tile_lds_bytes(g.Kq);
  const int block = nw * kWave;
  const int64_t max_jobs = max_token_tiles(x.T, x.k, x.E, x.has_shared) * ceil_div(x.I / kRowTile, nw);
#define PMOE_TILE(D_, NW_)                                                                               \
  do {                                                                                                   \
    static bool attr_set = false;                                                                        \
    if (!attr_set) {                                                                                     \
      hipError_t e_ = hipFuncSetAttribute(reinterpret_cast<const void*>(&gate_up_tile_kernel<D_, NW_>),  \
                                          hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);       \
      if (e_ != hipSuccess) return e_;                                                                   \
      attr_set = true;                                                                                   \
    }                                                                                                    \
    int per_cu = 0;                                                                                      \
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, gate_up_tile_kernel<D_, NW_>, block, lds) != \
            hipSuccess || per_cu < 1)                                                                    \
      per_cu = 1;                                                                                        \
    int64_t grid = (int64_t)device_cus() * per_cu;                                                       \
    if (grid > max_jobs) grid = max_jobs;                                                                \
    hipLaunchKernelGGL((gate_up_tile_kernel<D_, NW_>), dim3((unsigned)(grid < 1 ? 1 : grid)), dim3(block), \
                       lds, stream, g);                                                                  \
  } while (0)
  if (depth == 2) PMOE_TILE(2, nw);
  else if (depth == 3) PMOE_TILE(3, nw);
  else PMOE_TILE(4, nw);
#undef PMOE_TILE
  return hipGetLastError();
}

static DownK make_down_k(const ExpertArgs& x, const Workspace& ws) {
  DownK d;
  d.seg = segments_of(x, ws);
  d.hq = ws.hq;
  d.hs = ws.hs;
  d.down_nib = x.down_nib;
  d.down_sc = x.down_scale;
  d.sh_down_nib = x.sh_down_nib;
  d.sh_down_sc = x.sh_down_scale;
  d.H = x.H;
  d.I = x.I;
  d.Kq = ceil_div(x.I, kQuad);
  d.zero_row = x.T * x.k + (x.has_shared ? x.T : 0);
  d.outbuf = ws.outbuf;
  d.tiles = ws.tiles;
  d.n_tiles = ws.n_tiles;
  return d;
}

static GateUpK make_gate_up_k(const ExpertArgs& x, const Workspace& ws) {
  GateUpK g;
  g.seg = segments_of(x, ws);
  g.T = x.T;
  g.xq = ws.xq;
  g.xs = ws.xs;
  g.gate_nib = x.gate_nib;
  g.gate_sc = x.gate_scale;
  g.up_nib = x.up_nib;
  g.up_sc = x.up_scale;
  g.sh_gate_nib = x.sh_gate_nib;
  g.sh_gate_sc = x.sh_gate_scale;
  g.sh_up_nib = x.sh_up_nib;
  g.sh_up_sc = x.sh_up_scale;
  g.I = x.I;
  g.Kq = ceil_div(x.H, kQuad);
  g.KqI = ceil_div(x.I, kQuad);
  g.hq = ws.hq;
  g.hs = ws.hs;
  g.zero_row = x.T * x.k + (x.has_shared ? x.T : 0);
  g.tiles = ws.tiles;
  g.n_tiles = ws.n_tiles;
  return g;
}

hipError_t launch_gate_up(const ExpertArgs& x, const Workspace& ws, hipStream_t stream) {
  const GateUpK g = make_gate_up_k(x, ws);
  if (tile_fits(x, g)) return launch_gate_up_tile(x, g, stream);
  // K split: about four quads per wave (fewer waves per item keep more items
  // in flight per CU), one quad of loads outstanding per wave at a time.
  const int64_t q4 = ceil_div(g.Kq, 4);
  int ksplit = (int)(q4 < kGateUpWaves ? q4 : kGateUpWaves);
  int rt = 1, nq = 1;
  // With 4096+ single-tile items (H 7168, I 2048 from 8 tokens on), items of
  // two row tiles (each quad's activation operand loaded once for both) on
  // four waves: 196 vs 229 us at 8 tokens, 751 vs 891 us at 64; with fewer
  // items (one token) the halved item count loses (46 vs 43 us).
  if ((int64_t)max_active_experts(x) * (x.I / kRowTile) >= 4096) {
    rt = 2;
    ksplit = ksplit < 4 ? ksplit : 4;
  }
  tiling_override(tuning().gu_tiling, &ksplit, &rt, &nq);
  if (rt != 2 || (x.I / kRowTile) % 2) rt = 1;  // RT 4 would spill
  const int block = kWave * ksplit;
  const int64_t max_items = (int64_t)max_active_experts(x) * (x.I / (kRowTile * rt));
  // segment positions (T*k + shared T) = g.zero_row; their token ids go to LDS when they fit
#define PMOE_GU(RT_)                                                                                     \
  do {                                                                                                   \
    if (g.zero_row <= kTokLds)                                                                           \
      hipLaunchKernelGGL((gate_up_kernel<RT_, true>),                                                    \
                         dim3(resident_grid(gate_up_kernel<RT_, true>, block, max_items)), dim3(block), 0, \
                         stream, g);                                                                     \
    else                                                                                                 \
      hipLaunchKernelGGL((gate_up_kernel<RT_, false>),                                                   \
                         dim3(resident_grid(gate_up_kernel<RT_, false>, block, max_items)), dim3(block), 0, \
                         stream, g);                                                                     \
  } while (0)
  if (rt == 2) PMOE_GU(2);
  else PMOE_GU(1);
#undef PMOE_GU
  return hipGetLastError();
}

bool down_tile_regime(int64_t T, int64_t H, int64_t I, int E, int k, int has_shared) {
  if (lib_config().force_ksplit) return false;
  const int64_t lim = (int64_t)1 << 31;
  const int64_t KqI = ceil_div(I, kQuad);
  const int64_t rows = T * k + (has_shared ? T : 0);
  // Its waves stream short rows (I / 128 chunks of 1 KB each), so it needs
  // two workgroups per CU (operand within half the LDS) and at least eight
  // row tiles per CU to beat the K-split kernel (measured at H 7168, I 2048:
  // one workgroup per CU, 2.8x slower; at a single token of Qwen3, 7% slower).
  const int64_t row_items = max_token_tiles(T, k, E, has_shared) * (H / kRowTile);
  return row_items >= 8 * (int64_t)device_cus() && down_tile_lds_bytes(KqI) <= 80 * 1024 && H % kRowTile == 0 &&
         H * KqI * 64 < lim && (rows + 1) * KqI * 512 < lim;
}

// Ring depth 2 (a tuning override may set 4 or 6).
static hipError_t launch_down_tile(const ExpertArgs& x, const DownK& d, hipStream_t stream) {
  const int depth = tuning().dn_depth ? tuning().dn_depth : 2;
  const size_t lds = down_tile_lds_bytes(d.Kq);
  const int block = kTileWaves * kWave;
  const int64_t max_jobs = max_token_tiles(x.T, x.k, x.E, x.has_shared) * ceil_div(x.H / kRowTile, kTileWaves);
#define PMOE_DTILE(D_)                                                                                   \
  do {                                                                                                   \
    static bool attr_set = false;                                                                        \
    if (!attr_set) {                                                                                     \
      hipError_t e_ = hipFuncSetAttribute(reinterpret_cast<const void*>(&down_tile_kernel<D_, kTileWaves>), \
                                          hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);       \
      if (e_ != hipSuccess) return e_;                                                                   \
      attr_set = true;                                                                                   \
    }                                                                                                    \
    int per_cu = 0;                                                                                      \
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, down_tile_kernel<D_, kTileWaves>, block, lds) != \
            hipSuccess || per_cu < 1)                                                                    \
      per_cu = 1;                                                                                        \
    int64_t grid = (int64_t)device_cus() * per_cu;                                                       \
    if (grid > max_jobs) grid = max_jobs;                                                                \
    hipLaunchKernelGGL((down_tile_kernel<D_, kTileWaves>), dim3((unsigned)(grid < 1 ? 1 : grid)), dim3(block), \
                       lds, stream, d);                                                                  \
  } while (0)
  if (depth == 2) PMOE_DTILE(2);
  else if (depth == 4) PMOE_DTILE(4);
  else PMOE_DTILE(6);
#undef PMOE_DTILE
  return hipGetLastError();
}

hipError_t launch_down(const ExpertArgs& x, const Workspace& ws, hipStream_t stream) {
  const DownK d = make_down_k(x, ws);
  if (d.tiles && down_tile_regime(x.T, x.H, x.I, x.E, x.k, x.has_shared)) return launch_down_tile(x, d, stream);
  // the K-split kernel reads a segment's operand (at most T positions)
  // through one buffer resource, which must stay under 2 GiB
  if (x.T * d.Kq * 512 >= ((int64_t)1 << 31)) return hipErrorInvalidValue;
  Split sp = choose_split(d.Kq, kDownWaves);
  int rt = 2;  // H is a multiple of 32: an even number of 16-row tiles
  // Two quads of loads in flight per wave pay off only when items are few
  // (one token: 7.7 vs 8.4 us at Qwen3 shape, 28.6 vs 29.8 at H 7168, I 2048);
  // with many items the occupancy NQ = 1 allows wins (158 vs 162 us at 8 tokens),
  // and from 8192 items on two waves per item beat four (H 7168, I 2048: 150
  // vs 161 us at 8 tokens, 572 vs 609 us at 64; with few items they lose).
  // Below 512 items (two experts of H 4096, one token) single row tiles
  // double the items and one quad in flight per wave beats two (Mixtral shape:
  // 31.2 vs 34.7 us).  With long rows of I (16+ quads), four row tiles per
  // item share each quad's activation operand, with two quads in flight
  // (Mixtral at 16 tokens: 80.1 vs 91.9 us; H 7168, I 2048: 28.6 vs 29.1 us
  // at one token, 138.8 vs 148.4 at 8, 538 vs 571 at 64).
  const int64_t items = (int64_t)max_active_experts(x) * (x.H / (kRowTile * rt));
  sp.nq = items <= 4096 ? 2 : 1;
  if (items >= 8192) sp.ksplit = sp.ksplit < 2 ? sp.ksplit : 2;
  if (items < 512) {
    rt = 1;
    sp.nq = 1;
  } else if (d.Kq >= 16) {
    rt = 4;
    sp.nq = 2;
  }
  tiling_override(tuning().dn_tiling, &sp.ksplit, &rt, &sp.nq);
  if (rt == 4 && (x.H / kRowTile) % 4) rt = 2;
  const int block = kWave * sp.ksplit;
  const int64_t max_items = (int64_t)max_active_experts(x) * (x.H / (kRowTile * rt));
#define PMOE_DOWN(NQ_, RT_)                                                                             \
  hipLaunchKernelGGL((down_kernel<NQ_, RT_>),                                          \
              dim3(resident_grid(down_kernel<NQ_, RT_>, block, max_items)), dim3(block), 0, stream, d)
  if (sp.nq == 1) {
    if (rt == 1) PMOE_DOWN(1, 1);
    else if (rt == 2) PMOE_DOWN(1, 2);
    else PMOE_DOWN(1, 4);
  } else {
    if (rt == 1) PMOE_DOWN(2, 1);
    else if (rt == 2) PMOE_DOWN(2, 2);
    else PMOE_DOWN(2, 4);
  }
#undef PMOE_DOWN
  return hipGetLastError();
}

hipError_t launch_combine(const ExpertArgs& x, const Workspace& ws, hipStream_t stream) {
  const int64_t total = x.T * (x.H / 4);
  int64_t blocks = ceil_div(total, 256);
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(combine_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, ws.outbuf,
              static_cast<const int32_t*>(ws.slot_pos), x.topk_w, x.T, x.k, x.H, x.has_shared, x.y);
  return hipGetLastError();
}

hipError_t launch_experts(const ExpertArgs& x, const Workspace& ws, hipStream_t stream) {
  hipError_t err = launch_gate_up(x, ws, stream);
  if (err != hipSuccess) return err;
  err = launch_down(x, ws, stream);
  if (err != hipSuccess) return err;
  return launch_combine(x, ws, stream);
}

}  // namespace pmoe
