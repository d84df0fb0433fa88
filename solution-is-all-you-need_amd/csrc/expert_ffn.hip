// expert_ffn.hip -- grouped int4 (Q4_0) expert SwiGLU FFN for gfx950, decode
// regime, plus the weighted combine.
//
// Reference operator: kernels/sparse_moe/sparse_matmul.cu:120-215 (gate and up
// projections, h = silu(g) * u in fp32, down projection) with the expert
// weights of python/phantom/loader/gguf_loader.py:362-381 (Q4_0).
//
// Work decomposition.  Tokens are grouped per expert by the router's permute
// (segment [offsets[e], offsets[e+1]) of sorted slots).  A workgroup of four
// waves owns one 16-row tile of one active expert and walks that expert's
// segment 16 tokens at a time; the four waves split K (quads q = w, w+4, ...)
// and their partial tiles are summed in LDS in wave order, so the result does
// not depend on timing.  Every weight byte of an active expert is read from
// HBM by exactly one workgroup; the second and later 16-token tiles of a
// segment re-read it from L2.
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

#include "moe_common.h"
#include "moe_launch.h"

namespace pmoe {

struct SegmentK {
  const int32_t* offsets;
  const int32_t* active;
  const int32_t* n_active;
  const int32_t* sorted_slots;
  int64_t T;
  int k, E;
};

struct GateUpK {
  SegmentK seg;
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
  int64_t I;   // rows of gate/up
  int64_t Kq;  // quads of H
  int64_t KqI; // quads of I (down operand layout)
  uint16_t* hq;  // [rows][KqI][4 p][4 gi][hi, lo][8] fp16 bits
  float* hs;     // [rows][KqI * 4 groups][2 halves] sums of hi + lo
};

struct DownK {
  SegmentK seg;
  const uint16_t* hq;
  const float* hs;
  const uint8_t* down_nib;
  const uint16_t* down_sc;
  const uint8_t* sh_down_nib;
  const uint16_t* sh_down_sc;
  int64_t H;   // rows of down
  int64_t I;   // K of down
  int64_t Kq;  // quads of I
  float* outbuf;
};

__device__ inline void unpack_scales(uint2 s, float d[4]) {
  d[0] = half_bits_to_float((uint16_t)(s.x & 0xffffu));
  d[1] = half_bits_to_float((uint16_t)(s.x >> 16));
  d[2] = half_bits_to_float((uint16_t)(s.y & 0xffffu));
  d[3] = half_bits_to_float((uint16_t)(s.y >> 16));
}

__device__ inline int64_t token_of(const SegmentK& s, int64_t pos) {
  const int64_t nslots = s.T * s.k;
  return (pos < nslots) ? (int64_t)(s.sorted_slots[pos] / s.k) : pos - nslots;
}

__global__ __launch_bounds__(256) void gate_up_kernel(GateUpK a) {
  const int u = blockIdx.y;
  if (u >= *a.seg.n_active) return;
  const int e = a.seg.active[u];
  const int64_t seg_beg = a.seg.offsets[e];
  const int64_t seg_end = a.seg.offsets[e + 1];
  const int64_t nib_stride = a.I * a.Kq * 64;  // bytes per expert
  const int64_t sc_stride = a.I * a.Kq * 4;    // fp16 scales per expert
  const uint8_t* gnib;
  const uint16_t* gsc;
  const uint8_t* unib;
  const uint16_t* usc;
  if (e < a.seg.E) {
    gnib = a.gate_nib + e * nib_stride;
    gsc = a.gate_sc + e * sc_stride;
    unib = a.up_nib + e * nib_stride;
    usc = a.up_sc + e * sc_stride;
  } else {
    gnib = a.sh_gate_nib;
    gsc = a.sh_gate_sc;
    unib = a.sh_up_nib;
    usc = a.sh_up_sc;
  }
  const int64_t rt = blockIdx.x;
  const int lane = threadIdx.x % kWave;
  const int w = threadIdx.x / kWave;
  const int n = lane % 16;
  const int p = lane / 16;
  __shared__ float red[4][2][16][16];

  for (int64_t m0 = seg_beg; m0 < seg_end; m0 += 16) {
    const int64_t pm = m0 + n;
    const bool valid = pm < seg_end;
    const int64_t tok = valid ? token_of(a.seg, pm) : 0;
    f32x4 accg = {0.f, 0.f, 0.f, 0.f}, accu = accg, cg = accg, cu = accg;
    for (int64_t q = w; q < a.Kq; q += 4) {
      const int64_t tq = rt * a.Kq + q;
      const u32x4 gw = *reinterpret_cast<const u32x4*>(gnib + (tq * kWave + lane) * 16);
      const u32x4 uw = *reinterpret_cast<const u32x4*>(unib + (tq * kWave + lane) * 16);
      const uint2 gs = *reinterpret_cast<const uint2*>(gsc + tq * kQuadScales + n * 4);
      const uint2 us = *reinterpret_cast<const uint2*>(usc + tq * kQuadScales + n * 4);
      u32x4 xa[4];
      float sx = 0.0f;
      if (valid) {
        const u32x4* xp = reinterpret_cast<const u32x4*>(a.xq + ((tok * a.Kq + q) * 16 + p * 4) * 8);
#pragma unroll
        for (int gi = 0; gi < 4; ++gi) xa[gi] = xp[gi];
        sx = a.xs[tok * a.Kq * 4 + 4 * q + p];
      } else {
#pragma unroll
        for (int gi = 0; gi < 4; ++gi) xa[gi] = u32x4{0u, 0u, 0u, 0u};
      }
      float dg[4], du[4];
      unpack_scales(gs, dg);
      unpack_scales(us, du);
      const uint32_t gwv[4] = {gw.x, gw.y, gw.z, gw.w};
      const uint32_t uwv[4] = {uw.x, uw.y, uw.z, uw.w};
#pragma unroll
      for (int gi = 0; gi < 4; ++gi) {
        const f32x4 z = {0.f, 0.f, 0.f, 0.f};
        const f32x4 pg = mfma_bf16_16x16x32(xa[gi], dequant_unit_bf16(gwv[gi]), z);
        accg += (kUnitScale * dg[gi]) * pg;
        const f32x4 pu = mfma_bf16_16x16x32(xa[gi], dequant_unit_bf16(uwv[gi]), z);
        accu += (kUnitScale * du[gi]) * pu;
      }
      cg = mfma_f32_16x16x4(sx, dg[p], cg);
      cu = mfma_f32_16x16x4(sx, du[p], cu);
    }
    const f32x4 rg = accg - kUnitBias * cg;
    const f32x4 ru = accu - kUnitBias * cu;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      red[w][0][4 * p + r][n] = rg[r];
      red[w][1][4 * p + r][n] = ru[r];
    }
    __syncthreads();
    {
      const int mm = threadIdx.x / 16;
      const int nn = threadIdx.x % 16;
      const float g = ((red[0][0][mm][nn] + red[1][0][mm][nn]) + red[2][0][mm][nn]) + red[3][0][mm][nn];
      const float uu = ((red[0][1][mm][nn] + red[1][1][mm][nn]) + red[2][1][mm][nn]) + red[3][1][mm][nn];
      const float h = g * (1.0f / (1.0f + expf(-g))) * uu;
      // fp16 pair hi + lo of h, placed where the down kernel's MFMA operand
      // for (token, group, part) expects element i of I.
      const uint32_t hb = float_to_half_bits(h);
      const float hf = half_bits_to_float32(hb);
      const uint32_t lb = float_to_half_bits(h - hf);
      const float lf = half_bits_to_float32(lb);
      const int64_t pos = m0 + mm;
      const int64_t i = rt * 16 + nn;
      const int64_t g32 = i / kGroup;
      const int c = (int)(i % kGroup);
      const int half = c / 16;
      const int pp = (c % 16) / 4;
      const int r = c % 4;
      // kmap(p, j) = 4p + {0, 2, 16, 18, 1, 3, 17, 19}[j], inverted per half
      const int j = half == 0 ? ((r & 1) ? 4 : 0) + (r >> 1) : ((r & 1) ? 6 : 2) + (r >> 1);
      if (pos < seg_end) {
        uint16_t* dst = a.hq + (((pos * a.KqI + g32 / 4) * 16 + pp * 4 + (g32 % 4)) * 16);
        dst[j] = (uint16_t)hb;
        dst[8 + j] = (uint16_t)lb;
      }
      // The tile's 16 rows are one half of one group: sum hi + lo over them
      // (16 consecutive lanes, fixed butterfly order).
      float s = hf + lf;
      s += __shfl_xor(s, 8, kWave);
      s += __shfl_xor(s, 4, kWave);
      s += __shfl_xor(s, 2, kWave);
      s += __shfl_xor(s, 1, kWave);
      if (nn == 0 && pos < seg_end) a.hs[(pos * a.KqI * 4 + g32) * 2 + half] = s;
    }
    __syncthreads();
  }
}

__global__ __launch_bounds__(256) void down_kernel(DownK a) {
  const int u = blockIdx.y;
  if (u >= *a.seg.n_active) return;
  const int e = a.seg.active[u];
  const int64_t seg_beg = a.seg.offsets[e];
  const int64_t seg_end = a.seg.offsets[e + 1];
  const int64_t nib_stride = a.H * a.Kq * 64;
  const int64_t sc_stride = a.H * a.Kq * 4;
  const uint8_t* dnib;
  const uint16_t* dsc;
  if (e < a.seg.E) {
    dnib = a.down_nib + e * nib_stride;
    dsc = a.down_sc + e * sc_stride;
  } else {
    dnib = a.sh_down_nib;
    dsc = a.sh_down_sc;
  }
  const int64_t Kg = a.I / kGroup;
  const int64_t rt = blockIdx.x;
  const int lane = threadIdx.x % kWave;
  const int w = threadIdx.x / kWave;
  const int n = lane % 16;
  const int p = lane / 16;
  __shared__ float red[4][16][16];

  for (int64_t m0 = seg_beg; m0 < seg_end; m0 += 16) {
    const int64_t pm = m0 + n;
    const bool valid = pm < seg_end;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f}, corr = acc;
    for (int64_t q = w; q < a.Kq; q += 4) {
      const int64_t tq = rt * a.Kq + q;
      const u32x4 bw = *reinterpret_cast<const u32x4*>(dnib + (tq * kWave + lane) * 16);
      const uint2 bs = *reinterpret_cast<const uint2*>(dsc + tq * kQuadScales + n * 4);
      float dv[4];
      unpack_scales(bs, dv);
      const uint32_t bwv[4] = {bw.x, bw.y, bw.z, bw.w};
      u32x4 ah[4], al[4];
      float sp = 0.0f;
      const u32x4 zero = {0u, 0u, 0u, 0u};
      if (valid) {
        const u32x4* src = reinterpret_cast<const u32x4*>(a.hq + ((pm * a.Kq + q) * 16 + p * 4) * 16);
#pragma unroll
        for (int gi = 0; gi < 4; ++gi) {
          const bool real = 4 * q + gi < Kg;  // padded groups hold no h
          ah[gi] = real ? src[2 * gi] : zero;
          al[gi] = real ? src[2 * gi + 1] : zero;
        }
        if (4 * q + p < Kg) {
          const float* hsrc = a.hs + (pm * a.Kq * 4 + 4 * q + p) * 2;
          sp = hsrc[0] + hsrc[1];
        }
      } else {
#pragma unroll
        for (int gi = 0; gi < 4; ++gi) ah[gi] = al[gi] = zero;
      }
#pragma unroll
      for (int gi = 0; gi < 4; ++gi) {
        const u32x4 b = dequant_unit_f16(bwv[gi]);
        const f32x4 z = {0.f, 0.f, 0.f, 0.f};
        f32x4 pp = mfma_f16_16x16x32(ah[gi], b, z);
        pp = mfma_f16_16x16x32(al[gi], b, pp);
        acc += (kUnitScale * dv[gi]) * pp;
      }
      corr = mfma_f32_16x16x4(sp, dv[p], corr);
    }
    const f32x4 res = acc - kUnitBias * corr;
#pragma unroll
    for (int r = 0; r < 4; ++r) red[w][4 * p + r][n] = res[r];
    __syncthreads();
    {
      const int mm = threadIdx.x / 16;
      const int nn = threadIdx.x % 16;
      const float y = ((red[0][mm][nn] + red[1][mm][nn]) + red[2][mm][nn]) + red[3][mm][nn];
      if (m0 + mm < seg_end) a.outbuf[(m0 + mm) * a.H + rt * 16 + nn] = y;
    }
    __syncthreads();
  }
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

hipError_t launch_experts(const ExpertArgs& x, const Workspace& ws, hipStream_t stream) {
  SegmentK seg;
  seg.offsets = ws.offsets;
  seg.active = ws.active;
  seg.n_active = ws.n_active;
  seg.sorted_slots = ws.sorted_slots;
  seg.T = x.T;
  seg.k = x.k;
  seg.E = x.E;
  const int64_t nslots = x.T * x.k;
  const int64_t max_active = ((nslots < x.E) ? nslots : x.E) + (x.has_shared ? 1 : 0);

  GateUpK g;
  g.seg = seg;
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
  hipLaunchKernelGGL(gate_up_kernel, dim3((unsigned)(x.I / kRowTile), (unsigned)max_active),
                     dim3(256), 0, stream, g);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;

  DownK d;
  d.seg = seg;
  d.hq = ws.hq;
  d.hs = ws.hs;
  d.down_nib = x.down_nib;
  d.down_sc = x.down_scale;
  d.sh_down_nib = x.sh_down_nib;
  d.sh_down_sc = x.sh_down_scale;
  d.H = x.H;
  d.I = x.I;
  d.Kq = ceil_div(x.I, kQuad);
  d.outbuf = ws.outbuf;
  hipLaunchKernelGGL(down_kernel, dim3((unsigned)(x.H / kRowTile), (unsigned)max_active),
                     dim3(256), 0, stream, d);
  err = hipGetLastError();
  if (err != hipSuccess) return err;

  const int64_t total = x.T * (x.H / 4);
  int64_t blocks = ceil_div(total, 256);
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(combine_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, ws.outbuf,
                     ws.slot_pos, x.topk_w, x.T, x.k, x.H, x.has_shared, x.y);
  return hipGetLastError();
}

}  // namespace pmoe
