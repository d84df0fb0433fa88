// expert_ffn.hip -- grouped int4 (Q4_0) expert SwiGLU FFN for gfx950, decode
// regime, plus the weighted combine.
//
// Reference operator: kernels/sparse_moe/sparse_matmul.cu:120-215 (gate and up
// projections, h = silu(g) * u in fp32, down projection) with the expert
// weights of python/phantom/loader/gguf_loader.py:362-381 (Q4_0).
//
// Work decomposition.  The router's permute groups tokens per expert into
// segments and writes one descriptor {expert, begin, end} per launch slot
// (expert -1 for slots beyond the active count).  A workgroup owns one 16-row
// tile of one slot's expert and splits K across up to 16 waves, each issuing
// the loads of its one to four quads at once; there are no loops over K and
// no dependent chains beyond descriptor -> token id -> activation, so the
// many short waves keep HBM busy the way a plain streaming read does.  Wave
// partials are summed in LDS in wave order, so results do not depend on
// timing.  Every weight byte of an active expert is read from HBM once; later
// 16-token tiles of a long segment re-read it from L2.
//
// Arithmetic per 32-group g, token m, weight row n (see moe_common.h):
//   P = mfma(a_m, 1 + nib_n / 16)               exact products, fp32 sums
//   acc[m][n] += 16 d[n][g] * P                  fp32 FMA
//   corr[m][n] += S[m][g] * d[n][g]              fp32 MFMA over the 4 groups
//   result = acc - 24 * corr = sum_g d * sum_k a_k * (nib_k - 8)
// The gate/up activations x are exact bf16.  The down activations h are fp32;
// the gate/up epilogue stores each h as an fp16 pair hi + lo (|h - hi - lo| <=
// 2^-22 |h|) already in MFMA operand order, plus half-group sums, so the down
// kernel only loads operands (two fp16 MFMAs per group).  fp16 bounds |h| to
// below 65504.
#include <math.h>
#include <stdio.h>
#include <stdlib.h>

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
template <int NQ, int TP>
__device__ inline void gate_up_pass(const GateUpK& a, const int e, const int64_t seg_end, const int64_t m0,
                                    const int64_t rt, float (*red)[1][2][16][16]) {
  const int lane = threadIdx.x % kWave;
  const int ks = threadIdx.x / kWave;
  const int ksplit = blockDim.x / kWave;
  const int n = lane % 16;
  const int p = lane / 16;
  const uint32_t mask = vgpr_const(0x00780078u);
  const int64_t nib_stride = a.I * a.Kq * 64;
  const int64_t sc_stride = a.I * a.Kq * 4;
  const uint8_t* gnib = e < a.seg.E ? a.gate_nib + e * nib_stride : a.sh_gate_nib;
  const uint16_t* gsc = e < a.seg.E ? a.gate_sc + e * sc_stride : a.sh_gate_sc;
  const uint8_t* unib = e < a.seg.E ? a.up_nib + e * nib_stride : a.sh_up_nib;
  const uint16_t* usc = e < a.seg.E ? a.up_sc + e * sc_stride : a.sh_up_sc;
  uint32_t xoff[TP];  // element offset of this lane's activation row
#pragma unroll
  for (int t = 0; t < TP; ++t) {
    const int64_t pm = m0 + 16 * t + n;
    const int64_t tok = pm < seg_end ? (int64_t)a.seg.seg_tok[pm] : a.T;  // row T is all zero
    xoff[t] = (uint32_t)(tok * a.Kq);
  }
  const f32x4 z = {0.f, 0.f, 0.f, 0.f};
  f32x4 ag[TP], au[TP], cg[TP], cu[TP];
#pragma unroll
  for (int t = 0; t < TP; ++t) ag[t] = au[t] = cg[t] = cu[t] = z;
  for (int64_t q0 = ks; q0 < a.Kq; q0 += (int64_t)NQ * ksplit) {
    u32x4 gw[NQ], uw[NQ];
    uint2 gs[NQ], us[NQ];
    u32x4 xa[NQ][TP][4];
    float sx[NQ][TP];
    bool qok[NQ];
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      int q = (int)(q0 + (int64_t)i * ksplit);
      qok[i] = q < a.Kq;
      q = qok[i] ? q : (int)a.Kq - 1;
      const int64_t tq = rt * a.Kq + q;  // wave-uniform
      gw[i] = *reinterpret_cast<const u32x4*>(gnib + tq * kQuadNibBytes + lane * 16);
      uw[i] = *reinterpret_cast<const u32x4*>(unib + tq * kQuadNibBytes + lane * 16);
      gs[i] = *reinterpret_cast<const uint2*>(gsc + tq * kQuadScales + n * 4);
      us[i] = *reinterpret_cast<const uint2*>(usc + tq * kQuadScales + n * 4);
#pragma unroll
      for (int t = 0; t < TP; ++t) {
        const u32x4* xp =
            reinterpret_cast<const u32x4*>(a.xq + ((uint64_t)(xoff[t] + q) * 16 + p * 4) * 8);
#pragma unroll
        for (int gi = 0; gi < 4; ++gi) xa[i][t][gi] = xp[gi];
        sx[i][t] = a.xs[(uint64_t)(xoff[t] + q) * 4 + p];
      }
    }
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      if (!qok[i]) continue;
      float dg[4], du[4];
      unpack_scales(gs[i], dg);
      unpack_scales(us[i], du);
      const uint32_t gwv[4] = {gw[i].x, gw[i].y, gw[i].z, gw[i].w};
      const uint32_t uwv[4] = {uw[i].x, uw[i].y, uw[i].z, uw[i].w};
#pragma unroll
      for (int gi = 0; gi < 4; ++gi) {
        const u32x4 bg = dequant_unit_bf16(gwv[gi], mask);
        const u32x4 bu = dequant_unit_bf16(uwv[gi], mask);
#pragma unroll
        for (int t = 0; t < TP; ++t) {
          ag[t] += dg[gi] * mfma_bf16_16x16x32(xa[i][t][gi], bg, z);
          au[t] += du[gi] * mfma_bf16_16x16x32(xa[i][t][gi], bu, z);
        }
      }
#pragma unroll
      for (int t = 0; t < TP; ++t) {
        cg[t] = mfma_f32_16x16x4(sx[i][t], dg[p], cg[t]);
        cu[t] = mfma_f32_16x16x4(sx[i][t], du[p], cu[t]);
      }
    }
  }
#pragma unroll
  for (int t = 0; t < TP; ++t) {
    // sum_g d * sum_k a (n - 8) = 16 * sum_g d P - 24 * sum_g d S
    const f32x4 rg = kUnitScale * ag[t] - kUnitBias * cg[t];
    const f32x4 ru = kUnitScale * au[t] - kUnitBias * cu[t];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      red[ks][t][0][4 * p + j][n] = rg[j];
      red[ks][t][1][4 * p + j][n] = ru[j];
    }
  }
  __syncthreads();
  for (int o = threadIdx.x; o < TP * 256; o += blockDim.x) {
    const int t = o / 256;
    const int mm = (o % 256) / 16;
    const int nn = o % 16;
    float g = 0.0f, uu = 0.0f;
    for (int s2 = 0; s2 < ksplit; ++s2) {
      g += red[s2][t][0][mm][nn];
      uu += red[s2][t][1][mm][nn];
    }
    const float h = g * (1.0f / (1.0f + expf(-g))) * uu;
    // fp16 pair hi + lo of h, placed where the down kernel's MFMA operand
    // for (segment position, group, part) expects element i of I.
    const uint32_t hb = float_to_half_bits(h);
    const float hf = half_bits_to_float32(hb);
    const uint32_t lb = float_to_half_bits(h - hf);
    const float lf = half_bits_to_float32(lb);
    const int64_t pos = m0 + 16 * t + mm;
    const bool ok = pos < seg_end;
    const int64_t i = rt * 16 + nn;
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
  __syncthreads();
}

template <int NQ>
__device__ inline void gate_up_item(const GateUpK& a, const int4 d, const int64_t rt,
                                    float (*red)[1][2][16][16]) {
  const int e = __builtin_amdgcn_readfirstlane(d.x);
  const int64_t beg = __builtin_amdgcn_readfirstlane(d.y);
  const int64_t end = __builtin_amdgcn_readfirstlane(d.z);
  // One 16-token tile at a time: a longer segment re-reads the tile's
  // weights from L2, which costs less than the registers of a paired pass.
  for (int64_t m0 = beg; m0 < end; m0 += 16) gate_up_pass<NQ, 1>(a, e, end, m0, rt, red);
}

template <int NQ>
__global__ __launch_bounds__(kGateUpWaves * kWave, 4) void gate_up_kernel(GateUpK a) {
  __shared__ float red[kGateUpWaves][1][2][16][16];  // [wave][token tile][gate/up]
  __shared__ int4 s_desc[kMaxExperts + 1];
  __shared__ int s_nact;
  if (blockIdx.x == 0) {
    // the all-zero down-operand row read for positions past a segment
    for (int64_t i = threadIdx.x; i < a.KqI * 256; i += blockDim.x) a.hq[a.zero_row * a.KqI * 256 + i] = 0;
    for (int64_t i = threadIdx.x; i < a.KqI * 8; i += blockDim.x) a.hs[a.zero_row * a.KqI * 8 + i] = 0.0f;
  }
  const int n_act = load_descriptors(a.seg, s_desc, &s_nact);
  const int64_t n_rt = a.I / kRowTile;
  for (int64_t item = blockIdx.x; item < (int64_t)n_act * n_rt; item += gridDim.x)
    gate_up_item<NQ>(a, s_desc[item / n_rt], item % n_rt, red);
}


// ------------------------------------------------------------------ down

// Same decomposition as gate_up_kernel with RT 16-row tiles of H per item:
// the activation operand of a quad (16 positions x 128 of I as fp16 hi/lo)
// is loaded once and used for all RT tiles.  Positions past the segment
// read the all-zero operand row of hq / hs.
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

  for (int64_t m0 = beg; m0 < end; m0 += 16) {
    const int64_t pm0 = m0 + n;
    const int64_t pm = pm0 < end ? pm0 : a.zero_row;
    const f32x4 z = {0.f, 0.f, 0.f, 0.f};
    f32x4 acc[RT], corr[RT];
#pragma unroll
    for (int r = 0; r < RT; ++r) acc[r] = corr[r] = z;
    for (int64_t q0 = ks; q0 < a.Kq; q0 += (int64_t)NQ * ksplit) {
      u32x4 bw[NQ][RT];
      uint2 bs[NQ][RT];
      u32x4 ah[NQ][4], al[NQ][4];
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
          bw[i][r] = *reinterpret_cast<const u32x4*>(dnib + (tq * kWave + lane) * 16);
          bs[i][r] = *reinterpret_cast<const uint2*>(dsc + tq * kQuadScales + n * 4);
        }
        const u32x4* src = reinterpret_cast<const u32x4*>(a.hq + ((pm * a.Kq + q) * 16 + p * 4) * 16);
#pragma unroll
        for (int gi = 0; gi < 4; ++gi) {
          const bool real = 4 * q + gi < Kg;  // padded groups hold no h
          const u32x4 h = src[2 * gi];
          const u32x4 l = src[2 * gi + 1];
          ah[i][gi] = real ? h : zero;
          al[i][gi] = real ? l : zero;
        }
        const float* hsrc = a.hs + (pm * a.Kq * 4 + 4 * q + p) * 2;
        const float s0 = hsrc[0], s1 = hsrc[1];
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
            pp = mfma_f16_16x16x32(al[i][gi], bb, pp);
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
#pragma unroll
      for (int j = 0; j < 4; ++j) red[ks][r][4 * p + j][n] = res[j];
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

// y[t] = sum_j w[t,j] * out[slot_pos[t*k+j]] (+ out[T*k + t] for the shared
// expert), j in slot order, fp32.
__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ outbuf,
                                                      const int32_t* __restrict__ slot_pos,
                                                      const float* __restrict__ topk_w, int64_t T,
                                                      int k, int64_t H, int has_shared,
                                                      float* __restrict__ y) {
  const int64_t H4 = H / 4;
  const int64_t total = T * H4;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = i / H4;
    const int64_t c = (i % H4) * 4;
    float4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int j = 0; j < k; ++j) {
      const int64_t pos = slot_pos[t * k + j];
      const float wt = topk_w[t * k + j];
      const float4 o = *reinterpret_cast<const float4*>(outbuf + pos * H + c);
      acc.x += wt * o.x;
      acc.y += wt * o.y;
      acc.z += wt * o.z;
      acc.w += wt * o.w;
    }
    if (has_shared) {
      const float4 o = *reinterpret_cast<const float4*>(outbuf + (T * k + t) * H + c);
      acc.x += o.x;
      acc.y += o.y;
      acc.z += o.z;
      acc.w += o.w;
    }
    *reinterpret_cast<float4*>(y + t * H + c) = acc;
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

// Optional override "ksplit,rt,nq" for tuning sweeps (PHANTOM_MOE_GATE_UP_TILING /
// PHANTOM_MOE_DOWN_TILING); values outside the supported set are ignored.
static void tiling_override(const char* name, int max_waves, int* ksplit, int* rt, int* nq) {
  const char* v = getenv(name);
  if (!v) return;
  int a = 0, b = 0, c = 0;
  if (sscanf(v, "%d,%d,%d", &a, &b, &c) == 3 && a >= 1 && a <= max_waves && (b == 1 || b == 2 || b == 4) &&
      (c == 1 || c == 2)) {
    *ksplit = a;
    *rt = b;
    *nq = c;
  }
}

hipError_t launch_gate_up(const ExpertArgs& x, const Workspace& ws, hipStream_t stream) {
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
  Split sp = choose_split(g.Kq, kGateUpWaves);
  int rt = 1;
  tiling_override("PHANTOM_MOE_GATE_UP_TILING", kGateUpWaves, &sp.ksplit, &rt, &sp.nq);
  const int block = kWave * sp.ksplit;
  const int64_t max_items = (int64_t)max_active_experts(x) * (x.I / kRowTile);
  if (sp.nq == 1)
    hipLaunchKernelGGL(gate_up_kernel<1>, dim3(resident_grid(gate_up_kernel<1>, block, max_items)), dim3(block), 0,
                stream, g);
  else
    hipLaunchKernelGGL(gate_up_kernel<2>, dim3(resident_grid(gate_up_kernel<2>, block, max_items)), dim3(block), 0,
                stream, g);
  return hipGetLastError();
}

hipError_t launch_down(const ExpertArgs& x, const Workspace& ws, hipStream_t stream) {
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
  Split sp = choose_split(d.Kq, kDownWaves);
  sp.nq = 1;   // measured faster than NQ = 2 at the occupancy NQ = 1 allows
  int rt = 2;  // H is a multiple of 32: an even number of 16-row tiles
  tiling_override("PHANTOM_MOE_DOWN_TILING", kDownWaves, &sp.ksplit, &rt, &sp.nq);
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
