// decode_stream.hip -- the whole MoE layer for one token in one launch, for
// experts too large to stage whole in LDS (the Mixtral-8x7B- and
// DeepSeek-V3-shaped layers): every wave streams its share of the weights
// through a private ring of direct-to-LDS copies.
//
// Reference semantics as the staged path: router tests/test_moe_routing.py:
// 56-72 (logits x W^T, top-k, softmax or sigmoid-renorm over the k), expert
// FFN kernels/sparse_moe/sparse_matmul.cu:120-215 (SwiGLU, fp32 math) on
// Q4_0 weights (python/phantom/loader/gguf_loader.py:362-381), combine in
// slot order.  It replaces five launches (logits, top-k + permute, gate/up,
// down, combine; sparse_matmul.cu:256-363 launches per stage and waits on
// the host) with one.
//
// Grid: one 8-wave workgroup per CU (all resident; every wait is bounded).
//   0. Logit e by wave e / G of workgroup e % G (the router's fixed-order fp64
//      dot), published device-scope as a tagged slot; the x operand of the
//      token into LDS.
//   1. The last wave of every workgroup polls the E slots and selects and
//      weighs the experts with wave_topk_row, the staged router's own
//      instructions: identical routing bits on both paths.
//   2. Gate/up: item u = (slot j, 16-row tile r of I), slots j < k routed
//      and j = k the shared expert; item u goes to wave u / G of workgroup
//      u % G.  The wave streams the tile's gate and up quads over all of H
//      through its ring (copies of a quad issued `ns` quads ahead), MFMAs on
//      exact operands (bf16 x, 1 + n/16), SwiGLU, and publishes h as tagged
//      device-scope units {hi(i) | hi(i+1), tag, lo(i) | lo(i+1), ~tag}.
//   3. Down: workgroup b serves slot j(b) (the workgroups split evenly over
//      the slots) and a contiguous range of 16-row tiles of H; with fewer
//      tiles than waves, the waves of a tile split I and their partials are
//      summed in LDS in slice order.  The first ring stages are issued before
//      h is polled into LDS; outputs d_j are published as tagged units.
//   4. Combine: workgroup b owns rows [b R, b R + R) of y:
//      y = sum_j w_j d_j (j = 0 .. k-1 in slot order) + d_shared.
//   5. The next call's tag (as the other single-launch kernels).
#include <math.h>
#include <stdint.h>

#include "expert_common.h"
#include "fused_common.h"
#include "moe_common.h"
#include "moe_launch.h"
#include "topk_common.h"

namespace pmoe {

namespace {

constexpr uint32_t kSGuStage = 2304;  // gate nibbles 1 KiB | up nibbles 1 KiB | gate scales 128 B | up scales 128 B
constexpr uint32_t kSDnStage = 1152;  // down nibbles 1 KiB | scales 128 B
constexpr int kSGuCopies = 4;         // copy instructions per gate/up stage
constexpr int kSDnCopies = 2;         // per down stage
// Ring depths (quads in flight per wave).  Shallow rings stream faster here:
// with every wave of the chip streaming at once, deeper rings only add
// requests the memory system queues (gate/up 3 and down 4 stages against as
// deep as the LDS allows: Mixtral-shaped layer 49.0 against 52.8 us,
// DeepSeek-V3-shaped 59.6 against 62.3 us).
constexpr int kSGuMaxStages = 3;
constexpr int kSDnMaxStages = 4;

struct StreamK {
  const uint16_t* x;  // [H] bf16
  const float* W;     // [E, H]
  const float* bias;  // [E] or null
  int H, I, E, k, score_mode, has_shared;
  int Kq, KqI, S;  // quads of H and of I; slots with work (k + shared)
  int kx;          // slices of I the down work of a slot is cut into
  const uint8_t* gate_nib;
  const uint16_t* gate_sc;
  const uint8_t* up_nib;
  const uint16_t* up_sc;
  const uint8_t* down_nib;
  const uint16_t* down_sc;
  const uint8_t* sh_gate_nib;
  const uint16_t* sh_gate_sc;
  const uint8_t* sh_up_nib;
  const uint16_t* sh_up_sc;
  const uint8_t* sh_down_nib;
  const uint16_t* sh_down_sc;
  float* y;
  int32_t* topk_idx;
  float* topk_w;
  uint32_t* ctl;
  uint64_t* presence;
  uint32_t* slots;  // [E] tagged logits, kStreamSlotStride bytes apart
  uint32_t* hv;     // [S][I / 2][4] tagged h units
  uint32_t* dv;     // [S][H / 2][4] tagged expert outputs
  StreamLds lds;
  uint32_t* host_status;
  uint32_t wait_polls;
  uint32_t skew_route;
  uint32_t skew_h;
  uint32_t skew_gen;
};

// Down work of workgroup b: the G workgroups are cut into S contiguous
// ranges, workgroup b serving slot j(b) = floor(b S / G).  A slot's
// workgroups are dealt round robin over kx slices of I (slice kk = li % kx
// for the li-th workgroup of the range); those of one slice cut the NT row
// tiles of H evenly.  A workgroup then needs h only for its slice of I.
struct DnWork {
  int slot, kk, t0, nt;  // slot, slice of I, first tile, tiles
};
__device__ inline DnWork dn_work(int b, int G, int S, int NT, int kx) {
  DnWork d;
  d.slot = (int)(((int64_t)b * S) / G);
  const int g0 = (int)(((int64_t)d.slot * G + S - 1) / S);  // first workgroup of the slot
  const int g1 = (int)(((int64_t)(d.slot + 1) * G + S - 1) / S);
  const int nw = g1 - g0, li = b - g0;
  d.kk = li % kx;
  const int ng = (nw - d.kk + kx - 1) / kx, tg = li / kx;  // workgroups of the slice; this one's rank
  d.t0 = (int)(((int64_t)tg * NT) / ng);
  d.nt = (int)(((int64_t)(tg + 1) * NT) / ng) - d.t0;
  return d;
}

__global__ __launch_bounds__(kFThreads) void moe_decode_stream_kernel(StreamK a) {
  __shared__ int s_sel_idx[kMaxTopK + 1];
  __shared__ float s_sel_w[kMaxTopK + 1];
  __shared__ int s_pfail;
  extern __shared__ u32x4 s_dyn[];
  char* lds = reinterpret_cast<char*>(s_dyn);
  const int lane = threadIdx.x % kWave;
  const int w = uni(threadIdx.x / kWave);
  const int n = lane % 16;
  const int p = lane / 16;
  const int G = (int)gridDim.x;
  const int b = (int)blockIdx.x;
  const int H = a.H, I = a.I, E = a.E, k = a.k, Kq = a.Kq, KqI = a.KqI, S = a.S;
  const int NTI = I / kRowTile, NTH = H / kRowTile;
  u32x4* s_xop = reinterpret_cast<u32x4*>(lds + a.lds.x);  // [Kq][4 p][4 gi]
  float* s_xs = reinterpret_cast<float*>(lds + a.lds.xs);  // [Kq][4 p]
  double* s_lv = reinterpret_cast<double*>(lds + a.lds.lv);
  char* s_tk = lds + a.lds.topk;
  char* s_h = lds + a.lds.h;  // this workgroup's quads [qa, qb) of h: [quad - qa][4 p][4 gi][hi | lo] x 16 B
  float* s_red = reinterpret_cast<float*>(lds + a.lds.red);  // [8 waves][16]
  const uint32_t ring = lds_addr(lds + a.lds.ring) + (uint32_t)w * a.lds.ring_wave;
  const char* ring_p = lds + a.lds.ring + w * a.lds.ring_wave;
  const f32x4 z = {0.f, 0.f, 0.f, 0.f};

  // ---- 0. generation; logits; x operand ---------------------------------------
  const uint32_t tag = launch_tag(a.ctl, &a.presence[b], b == G - 1 ? a.skew_gen : 0u);
  const BufRsrc slot_r = buf_rsrc(a.slots, (uint32_t)E * kStreamSlotStride);
  {
    const int e = w * G + b;
    if (e < E) {
      double logit = fixed_dot_bf16(a.x, a.W + (int64_t)e * H, H);
      if (a.bias) logit = logit + (double)a.bias[e];
      if (lane == 0) {
        const uint64_t bits = __builtin_bit_cast(uint64_t, logit);
        u32x4 v;
        v.x = (uint32_t)bits;
        v.y = tag;
        v.z = (uint32_t)(bits >> 32);
        v.w = ~tag;
        __builtin_amdgcn_raw_buffer_store_b128(v, slot_r, e * (int)kStreamSlotStride, 0, kDeviceScope);
      }
    }
  }
  // the x operand (one thread per (quad, group)) and its group sums, as the
  // other single-launch kernels build them
  for (int j = threadIdx.x; j < Kq * 4; j += kFThreads) {
    const int q = j / 4, gi = j % 4, g = 4 * q + gi;
    const bool valid = g < H / kGroup;
    const uint16_t* xr = a.x + (int64_t)(valid ? g : 0) * kGroup;
    float sp[4];
#pragma unroll
    for (int pp = 0; pp < 4; ++pp) {
      uint2 lo = *reinterpret_cast<const uint2*>(xr + 4 * pp);
      uint2 hi = *reinterpret_cast<const uint2*>(xr + 16 + 4 * pp);
      if (!valid) lo = hi = make_uint2(0u, 0u);
      u32x4 v;
      v.x = (lo.x & 0xffffu) | (lo.y << 16);
      v.y = (hi.x & 0xffffu) | (hi.y << 16);
      v.z = (lo.x >> 16) | (lo.y & 0xffff0000u);
      v.w = (hi.x >> 16) | (hi.y & 0xffff0000u);
      s_xop[(q * 4 + pp) * 4 + gi] = v;
      sp[pp] = ((bf16_bits_to_float(lo.x & 0xffffu) + bf16_bits_to_float(lo.x >> 16)) +
                (bf16_bits_to_float(lo.y & 0xffffu) + bf16_bits_to_float(lo.y >> 16))) +
               ((bf16_bits_to_float(hi.x & 0xffffu) + bf16_bits_to_float(hi.x >> 16)) +
                (bf16_bits_to_float(hi.y & 0xffffu) + bf16_bits_to_float(hi.y >> 16)));
    }
    s_xs[q * 4 + gi] = (sp[0] + sp[1]) + (sp[2] + sp[3]);
  }

  // ---- 1. selection (last wave) while the other waves start the shared expert --
  // Gate/up items: item u is the 16-row tile r = u % NTI of I of slot
  // j = u / NTI (slot k is the shared expert); workgroup b owns items
  // u = b + m G, m = 0 .. nI - 1, of which the first nR are routed.  The
  // shared expert's items need no routing, so waves 0 .. 6 stream them while
  // the last wave selects the experts; the routed items follow on all eight
  // waves.  Within each of the two groups the items' quads, in item order,
  // are cut into equal contiguous ranges, one per wave, streamed through the
  // wave's ring without a break at item boundaries; an item inside one
  // wave's range is finished by that wave, an item cut between waves is
  // summed from their partials (LDS, in wave order) after a barrier.  Every
  // row of the MFMAs' A operand holds the token's x, so every row of a
  // result holds the token's sums: element 0 of every lane is row 16 r + n
  // of I, and only that element is scaled and summed (per group: scale
  // times the sum over x (1 + n/16), and scale times the sum of x).
  lds_barrier();  // the x operand is in LDS
  const BufRsrc hv_r = buf_rsrc(a.hv, (uint32_t)(S * (I / 2) * 16));
  const int ns_gu = a.lds.ns_gu;
  const uint32_t bmask = vgpr_const(0x00780078u);
  const int nI = b < S * NTI ? (S * NTI - b + G - 1) / G : 0;
  const int nR = b < k * NTI ? (k * NTI - b + G - 1) / G : 0;
  // partials of items cut between waves: [kFW waves][first | last segment][16 rows][ag, au, cg, cu],
  // one array for the shared items and one for the routed ones
  float* s_gpart_sh = s_red;
  float* s_gpart_rt = s_red + kFW * 2 * 16 * 4;
  bool route_failed = false;  // known after the selection's barrier
  // h of item m from every lane's sums for row 16 r + n (NaN when !ok)
  auto publish = [&](int m, float ag, float au, float cg, float cu, bool ok) {
    const int u = b + m * G, j = u / NTI, r = u - j * NTI;
    float h = __builtin_nanf("");
    if (ok) {
      const float g = kUnitScale * ag - kUnitBias * cg;
      const float uu = kUnitScale * au - kUnitBias * cu;
      h = g * (1.0f / (1.0f + expf(-g))) * uu;
    }
    const uint32_t hb = float_to_half_bits(h);
    const uint32_t lb = float_to_half_bits(h - half_bits_to_float32(hb));
    const uint32_t hb2 = __shfl_down(hb, 1, kWave), lb2 = __shfl_down(lb, 1, kWave);
    if (p == 0 && (n & 1) == 0) {
      u32x4 v;
      v.x = hb | (hb2 << 16);
      v.y = tag;
      v.z = lb | (lb2 << 16);
      v.w = ~tag;
      __builtin_amdgcn_raw_buffer_store_b128(v, hv_r, (j * (I / 2) + (kRowTile * r + n) / 2) * 16, 0, kDeviceScope);
    }
  };
  const uint32_t nib_b = (uint32_t)I * (uint32_t)Kq * 64u, sc_b = (uint32_t)I * (uint32_t)Kq * 8u;
  // items m in [mb, mb + nit) over waves 0 .. nwv - 1; run: stream and sum
  // (else every item this wave finishes is published as NaN)
  auto run_items = [&](int mb, int nit, int nwv, float* gpart, bool run, bool ok) {
    const int Tq = nit * Kq;
    const int g0 = w < nwv ? (int)(((int64_t)w * Tq) / nwv) : Tq;
    const int n_w = w < nwv ? (int)(((int64_t)(w + 1) * Tq) / nwv) - g0 : 0;
    // copy cursor: item im, quad iq, and the item's buffers
    int im = g0 / Kq, iq = g0 - (g0 / Kq) * Kq;
    i32x4 gnr = {0, 0, 0, 0}, unr = gnr, gsr = gnr, usr = gnr;
    uint32_t itq0 = 0;
    auto item_buffers = [&]() {
      const int u = b + (mb + im) * G, j = u / NTI, r = u - j * NTI;
      const int e = j < k ? uni(s_sel_idx[j]) : -1;
      const bool sh = e < 0;
      const uint8_t* gn = sh ? a.sh_gate_nib : a.gate_nib + (size_t)e * nib_b;
      const uint8_t* un = sh ? a.sh_up_nib : a.up_nib + (size_t)e * nib_b;
      const char* gs = reinterpret_cast<const char*>(sh ? a.sh_gate_sc : a.gate_sc) + (sh ? 0 : (size_t)e * sc_b);
      const char* us = reinterpret_cast<const char*>(sh ? a.sh_up_sc : a.up_sc) + (sh ? 0 : (size_t)e * sc_b);
      gnr = buf_rsrc_words(gn, nib_b);
      unr = buf_rsrc_words(un, nib_b);
      gsr = buf_rsrc_words(gs, sc_b);
      usr = buf_rsrc_words(us, sc_b);
      itq0 = (uint32_t)r * (uint32_t)Kq;
    };
    auto issue_next = [&](int stage) {
      const uint32_t st = ring + (uint32_t)stage * kSGuStage;
      const uint32_t tq = (uint32_t)uni((int)(itq0 + (uint32_t)iq));
      dma_b128_stream(gnr, st, (uint32_t)lane * 16u, tq * kQuadNibBytes);
      dma_b128_stream(unr, st + 1024u, (uint32_t)lane * 16u, tq * kQuadNibBytes);
      if (lane < 8) {
        dma_b128_stream(gsr, st + 2048u, (uint32_t)lane * 16u, tq * 128u);
        dma_b128_stream(usr, st + 2176u, (uint32_t)lane * 16u, tq * 128u);
      }
      if (++iq == Kq) {
        iq = 0;
        if (++im < nit) item_buffers();
      }
    };
    if (run && n_w > 0) {
      item_buffers();
      const int pro = ns_gu < n_w ? ns_gu : n_w;
      for (int i = 0; i < pro; ++i) issue_next(i);
    }
    int cm = g0 / Kq, cq = g0 - (g0 / Kq) * Kq;  // quad being summed
    int seg_q0 = cq, seg_slot = 0;             // start quad of the segment; partial slot
    float ag = 0.0f, au = 0.0f, cg = 0.0f, cu = 0.0f;
    int stage = 0;  // ring stage of the quad being summed
    for (int i = 0; i < n_w; ++i) {
      if (run) {
        // this quad's copies in; the younger ones (up to ns - 1 quads) may fly
        const int younger = (i + ns_gu < n_w ? ns_gu : n_w - i) - 1;
        wait_vmcnt_le(kSGuCopies * younger);
        poll_clobber();
        const char* st = ring_p + stage * (int)kSGuStage;
        const u32x4 gw = *reinterpret_cast<const u32x4*>(st + lane * 16);
        const u32x4 uw = *reinterpret_cast<const u32x4*>(st + 1024 + lane * 16);
        const uint2 gsv = *reinterpret_cast<const uint2*>(st + 2048 + n * 8);
        const uint2 usv = *reinterpret_cast<const uint2*>(st + 2176 + n * 8);
        const u32x4* xo = s_xop + (cq * 4 + p) * 4;
        const u32x4 xa[4] = {xo[0], xo[1], xo[2], xo[3]};
        const f32x4 xs = *reinterpret_cast<const f32x4*>(s_xs + cq * 4);
        float dg[4], du[4];
        unpack_scales(gsv, dg);
        unpack_scales(usv, du);
        const uint32_t gwv[4] = {gw.x, gw.y, gw.z, gw.w};
        const uint32_t uwv[4] = {uw.x, uw.y, uw.z, uw.w};
        f32x4 pg[4], pu[4];
#pragma unroll
        for (int gi = 0; gi < 4; ++gi) {
          pg[gi] = mfma_bf16_16x16x32(xa[gi], dequant_unit_bf16(gwv[gi], bmask), z);
          pu[gi] = mfma_bf16_16x16x32(xa[gi], dequant_unit_bf16(uwv[gi], bmask), z);
        }
#pragma unroll
        for (int gi = 0; gi < 4; ++gi) {
          ag += dg[gi] * pg[gi][0];
          au += du[gi] * pu[gi][0];
          cg += dg[gi] * xs[gi];
          cu += du[gi] * xs[gi];
        }
        // the stage is read (the MFMAs consumed it) before it is refilled
        if (i + ns_gu < n_w) issue_next(stage);
        stage = stage + 1 == ns_gu ? 0 : stage + 1;
      }
      if (++cq == Kq || i == n_w - 1) {  // end of a segment
        if (seg_q0 == 0 && cq == Kq) {
          publish(mb + cm, ag, au, cg, cu, ok);
        } else if (p == 0) {
          const f32x4 v = {ag, au, cg, cu};
          *reinterpret_cast<f32x4*>(gpart + ((w * 2 + seg_slot) * 16 + n) * 4) = v;
        }
        ag = au = cg = cu = 0.0f;
        seg_q0 = 0;
        seg_slot = 1;
        if (cq == Kq) {
          cq = 0;
          ++cm;
        }
      }
    }
  };
  // after a barrier: items cut between waves, wave m % kFW summing item m's
  // partials in wave order
  auto finish_cut_items = [&](int mb, int nit, int nwv, const float* gpart, bool ok) {
    const int Tq = nit * Kq;
    auto range_lo = [&](int ww) { return ww < nwv ? (int)(((int64_t)ww * Tq) / nwv) : Tq; };
    for (int m = w; m < nit; m += kFW) {
      const int lo = m * Kq, hi = lo + Kq;
      bool whole = false;
      for (int ww = 0; ww < nwv; ++ww) whole = whole || (range_lo(ww) <= lo && range_lo(ww + 1) >= hi);
      if (whole) continue;
      float sg = 0.0f, su = 0.0f, sgc = 0.0f, suc = 0.0f;
      for (int ww = 0; ww < nwv; ++ww) {
        const int a0 = range_lo(ww), a1 = range_lo(ww + 1);
        if (a1 <= lo || a0 >= hi || a1 <= a0) continue;
        // item m is the first segment of wave ww when the wave starts inside it
        const f32x4 v = *reinterpret_cast<const f32x4*>(gpart + ((ww * 2 + (a0 >= lo ? 0 : 1)) * 16 + n) * 4);
        sg += v[0];
        su += v[1];
        sgc += v[2];
        suc += v[3];
      }
      publish(mb + m, sg, su, sgc, suc, ok);
    }
  };
  if (w == kFW - 1) {
    const uint32_t want = tag + a.skew_route;
    constexpr int kNV = kMaxExperts / kWave;
    bool done[kNV];
#pragma unroll
    for (int v = 0; v < kNV; ++v) done[v] = lane + v * kWave >= E;
    bool failed = false;
    for (uint32_t it = 0;; ++it) {
      poll_clobber();
      u32x4 sv[kNV];
#pragma unroll
      for (int v = 0; v < kNV; ++v)
        if (!done[v])
          sv[v] = __builtin_amdgcn_raw_buffer_load_b128(slot_r, (lane + v * kWave) * (int)kStreamSlotStride, 0,
                                                        kDevicePoll);
      bool all = true;
#pragma unroll
      for (int v = 0; v < kNV; ++v) {
        if (!done[v] && tag_ok(sv[v], want)) {
          s_lv[lane + v * kWave] = __builtin_bit_cast(double, ((uint64_t)sv[v].z << 32) | sv[v].x);
          done[v] = true;
        }
        all = all && done[v];
      }
      if (__all(all)) break;
      if (it >= a.wait_polls) {
        failed = true;
        if (lane == 0) set_status(a.ctl, a.host_status, kStatusRouteWait);
        break;
      }
    }
    if (!failed) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      uint64_t* s_ck = reinterpret_cast<uint64_t*>(s_tk);
      double* s_cv = reinterpret_cast<double*>(s_tk + 8 * k);
      double* s_val = reinterpret_cast<double*>(s_tk + 16 * k);
      double* s_e = reinterpret_cast<double*>(s_tk + 24 * k);
      int* s_ci = reinterpret_cast<int*>(s_tk + 32 * k);
      int* s_idx = reinterpret_cast<int*>(s_tk + 36 * k);
      if (E <= 64) wave_topk_row<1>(s_lv, E, k, a.score_mode, s_ck, s_cv, s_ci, s_val, s_idx, s_e, s_sel_idx, s_sel_w, nullptr);
      else if (E <= 128) wave_topk_row<2>(s_lv, E, k, a.score_mode, s_ck, s_cv, s_ci, s_val, s_idx, s_e, s_sel_idx, s_sel_w, nullptr);
      else if (E <= 256) wave_topk_row<4>(s_lv, E, k, a.score_mode, s_ck, s_cv, s_ci, s_val, s_idx, s_e, s_sel_idx, s_sel_w, nullptr);
      else wave_topk_row<8>(s_lv, E, k, a.score_mode, s_ck, s_cv, s_ci, s_val, s_idx, s_e, s_sel_idx, s_sel_w, nullptr);
    }
    if (lane == 0) {
      s_pfail = failed ? 1 : 0;
      s_sel_idx[k] = -1;  // the shared expert's slot
      s_sel_w[k] = 1.0f;
    }
  }
  // the shared expert's items, on waves 0 .. kFW - 2 (the last wave selects)
  run_items(nR, nI - nR, kFW - 1, s_gpart_sh, true, true);
  asm volatile("" ::"s"(tag));  // this wave's counter and presence loads have returned
  lds_barrier();
  if (threadIdx.x == 0) __hip_atomic_store(&a.presence[b], tag64(tag), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  route_failed = uni(s_pfail) != 0;
  if (b == 0 && (int)threadIdx.x < k) {
    a.topk_idx[threadIdx.x] = route_failed ? -1 : s_sel_idx[threadIdx.x];
    a.topk_w[threadIdx.x] = route_failed ? __builtin_nanf("") : s_sel_w[threadIdx.x];
  }

  // ---- 2. gate/up: the routed items, on all waves ---------------------------------
  finish_cut_items(nR, nI - nR, kFW - 1, s_gpart_sh, true);
  run_items(0, nR, kFW, s_gpart_rt, !route_failed, !route_failed);
  lds_barrier();
  finish_cut_items(0, nR, kFW, s_gpart_rt, !route_failed);

  // ---- 3. down: this workgroup's slot and tiles -----------------------------------
  const int kx = a.kx;
  const DnWork dw = dn_work(b, G, S, NTH, kx);
  // this workgroup's quads of I
  const int qa = (int)(((int64_t)dw.kk * KqI) / kx), qb = (int)(((int64_t)(dw.kk + 1) * KqI) / kx);
  // waves per tile (a power of two) when the tiles are fewer than the waves:
  // they split the quads of I in contiguous slices
  int ks = 1;
  while (ks < kFW && dw.nt * ks * 2 <= kFW) ks *= 2;
  const int ns_dn = a.lds.ns_dn;
  const uint32_t fmask = vgpr_const(0x000F000Fu);
  const int e_dn = route_failed ? 0 : uni(s_sel_idx[dw.slot]);
  const bool sh_dn = e_dn < 0;
  const uint32_t dnib_b = (uint32_t)H * (uint32_t)KqI * 64u, dsc_b = (uint32_t)H * (uint32_t)KqI * 8u;
  const i32x4 dnr = buf_rsrc_words(sh_dn ? a.sh_down_nib : a.down_nib + (size_t)e_dn * dnib_b, dnib_b);
  const i32x4 dsr = buf_rsrc_words(reinterpret_cast<const char*>(sh_dn ? a.sh_down_sc : a.down_sc) +
                                       (sh_dn ? 0 : (size_t)e_dn * dsc_b), dsc_b);
  const int slice = w % ks;                    // this wave's slice of I
  const int q0 = qa + (int)(((int64_t)slice * (qb - qa)) / ks), q1 = qa + (int)(((int64_t)(slice + 1) * (qb - qa)) / ks);
  const int nq = q1 - q0;
  // this wave's tiles: t0 + w / ks, then + kFW / ks
  const int tstep = kFW / ks;
  const int tl_first = w / ks;
  // this wave's stream: its tiles (rounds rr < nr_w) times the quads of its
  // slice, copied without a break between tiles
  const int nr_w = (!route_failed && nq > 0 && tl_first < dw.nt) ? (dw.nt - tl_first + tstep - 1) / tstep : 0;
  const int n_dn = nr_w * nq;
  int d_ir = 0, d_iq = 0;  // copy cursor: round, quad
  auto dn_issue_next = [&](int stage) {
    const uint32_t st = ring + (uint32_t)stage * kSDnStage;
    const uint32_t tq = (uint32_t)uni((dw.t0 + tl_first + d_ir * tstep) * KqI + q0 + d_iq);
    dma_b128_stream(dnr, st, (uint32_t)lane * 16u, tq * kQuadNibBytes);
    if (lane < 8) dma_b128_stream(dsr, st + 1024u, (uint32_t)lane * 16u, tq * 128u);
    if (++d_iq == nq) {
      d_iq = 0;
      ++d_ir;
    }
  };
  // the first ring stages, before h is polled (they need no h)
  for (int i = 0; i < (ns_dn < n_dn ? ns_dn : n_dn); ++i) dn_issue_next(i);
  // h of the slot's rows in this workgroup's quads [qa, qb) of I into LDS
  // (all threads), from the gate/up items' units: unit v holds rows i0 = 2v
  // and i0 + 1, at K positions kmap(pp, s), kmap(pp, s + 4) of part
  // pp = (i0 % 16) / 4 of group i0 / 32
  __shared__ int s_hfail;
  if (threadIdx.x == 0) s_hfail = 0;
  // zero first: groups past I (a ragged last quad) meet q = 0 there, and
  // whatever the LDS held could be NaN
  for (int i = (int)threadIdx.x; i < (qb - qa) * 128; i += kFThreads) reinterpret_cast<uint32_t*>(s_h)[i] = 0u;
  lds_barrier();
  const int va = qa * (kQuad / 2), vb = qb * (kQuad / 2) < I / 2 ? qb * (kQuad / 2) : I / 2;  // units
  if (!route_failed) {
    const uint32_t want = tag + a.skew_h;
    for (int v0 = va; v0 < vb; v0 += kFThreads) {
      const int v = v0 + (int)threadIdx.x;
      const bool mine = v < vb;
      u32x4 hvv = {0u, 0u, 0u, 0u};
      bool ok = !mine;
      if (mine) {
        hvv = __builtin_amdgcn_raw_buffer_load_b128(hv_r, (dw.slot * (I / 2) + v) * 16, 0, kDevicePoll);
        ok = tag_ok(hvv, want);
      }
      for (uint32_t it = 0;; ++it) {
        if (__all(ok)) break;
        if (it >= a.wait_polls) {
          if (lane == 0) {
            s_hfail = 1;
            set_status(a.ctl, a.host_status, kStatusExpertWait);
          }
          break;
        }
        poll_clobber();
        if (!ok) {
          hvv = __builtin_amdgcn_raw_buffer_load_b128(hv_r, (dw.slot * (I / 2) + v) * 16, 0, kDevicePoll);
          ok = tag_ok(hvv, want);
        }
      }
      if (mine) {
        if (!ok) {  // fp16 NaN
          hvv.x = 0x7E007E00u;
          hvv.z = 0x7E007E00u;
        }
        const int i0 = 2 * v, g32 = i0 / kGroup, jj = i0 % kGroup;
        const int pp = (jj % 16) / 4, off = jj - 4 * pp;  // 0, 2, 16 or 18
        const int s = ((off & 2) ? 1 : 0) + (off >= 16 ? 2 : 0);
        uint16_t* e16 = reinterpret_cast<uint16_t*>(s_h + (((g32 / 4 - qa) * 4 + pp) * 4 + g32 % 4) * 32);
        e16[s] = (uint16_t)(hvv.x & 0xffffu);
        e16[s + 4] = (uint16_t)(hvv.x >> 16);
        e16[8 + s] = (uint16_t)(hvv.z & 0xffffu);
        e16[8 + s + 4] = (uint16_t)(hvv.z >> 16);
      }
    }
  }
  lds_barrier();
  const bool h_failed = uni(s_hfail) != 0;
  const BufRsrc dv_r = buf_rsrc(a.dv, (uint32_t)(S * kx * (H / 2) * 16));
  // every wave runs the same number of tile rounds, so the K-split barrier
  // below is reached by all
  const int rounds = (dw.nt + tstep - 1) / tstep;
  int stage = 0;  // ring stage of the quad being summed
  for (int rr = 0; rr < rounds; ++rr) {
    const int tl = tl_first + rr * tstep;
    // A operand rows alternate h hi (even rows) and h lo (odd rows), so
    // elements 0 and 1 of every lane are the hi and lo sums of output row
    // 16 tile + n; only those are scaled and summed
    float acc_hi = 0.0f, acc_lo = 0.0f;
    if (rr < nr_w) {
      for (int q = 0; q < nq; ++q) {
        const int i = rr * nq + q;
        const int younger = (i + ns_dn < n_dn ? ns_dn : n_dn - i) - 1;
        wait_vmcnt_le(kSDnCopies * younger);
        poll_clobber();
        const char* st = ring_p + stage * (int)kSDnStage;
        const u32x4 wv = *reinterpret_cast<const u32x4*>(st + lane * 16);
        float dv[4];
        unpack_scales(*reinterpret_cast<const uint2*>(st + 1024 + n * 8), dv);
        const char* hq = s_h + (((q0 + q - qa) * 4 + p) * 4) * 32 + (n & 1) * 16;
        const u32x4 hh[4] = {*reinterpret_cast<const u32x4*>(hq), *reinterpret_cast<const u32x4*>(hq + 32),
                             *reinterpret_cast<const u32x4*>(hq + 64), *reinterpret_cast<const u32x4*>(hq + 96)};
        const uint32_t wvv[4] = {wv.x, wv.y, wv.z, wv.w};
        f32x4 pv[4];
#pragma unroll
        for (int gi = 0; gi < 4; ++gi) pv[gi] = mfma_f16_16x16x32(hh[gi], dequant_unit_f16s(wvv[gi], fmask), z);
#pragma unroll
        for (int gi = 0; gi < 4; ++gi) {
          acc_hi += dv[gi] * pv[gi][0];
          acc_lo += dv[gi] * pv[gi][1];
        }
        if (i + ns_dn < n_dn) dn_issue_next(stage);
        stage = stage + 1 == ns_dn ? 0 : stage + 1;
      }
    }
    const float part = acc_hi + acc_lo;
    if (ks > 1) {
      if (p == 0) s_red[w * 16 + n] = part;
      lds_barrier();
    }
    if (slice == 0 && tl < dw.nt) {
      float d = __builtin_nanf("");
      if (!route_failed && !h_failed) {
        d = part;
        for (int s2 = 1; s2 < ks; ++s2) d += s_red[(w + s2) * 16 + n];
      }
      const float d2 = __shfl_down(d, 1, kWave);
      if (p == 0 && (n & 1) == 0) {
        u32x4 v;
        v.x = __builtin_bit_cast(uint32_t, d);
        v.y = tag;
        v.z = __builtin_bit_cast(uint32_t, d2);
        v.w = ~tag;
        const int row = (dw.t0 + tl) * kRowTile + n;
        __builtin_amdgcn_raw_buffer_store_b128(v, dv_r, ((dw.slot * kx + dw.kk) * (H / 2) + row / 2) * 16, 0,
                                               kDeviceScope);
      }
    }
    if (ks > 1) lds_barrier();  // s_red is free for the next round
  }

  // ---- 4. combine: rows [b R, b R + R) of y ---------------------------------------
  if (w == 1) {
    const int R = a.lds.yrows;
    const int r0 = b * R;
    const int nr = r0 + R <= H ? R : (H > r0 ? H - r0 : 0);
    // lane l: rows r0 + 2 (l % (R / 2)) .. + 1 of part jk = l / (R / 2) (slot
    // jk / kx, slice of I jk % kx), then more parts in later rounds; the
    // values go through LDS (s_red)
    const int upr = R / 2;  // units per part
    float* s_d = s_red;     // [S][kx][R] expert outputs of the rows, by slice of I (reused)
    const uint32_t want = tag + a.skew_h;
    for (int c0 = 0; c0 < S * kx * upr; c0 += kWave) {
      const int c = c0 + lane;
      const int j = c / upr, uu = c - j * upr;
      const bool mine = c < S * kx * upr && 2 * uu < nr;
      u32x4 v = {0u, 0u, 0u, 0u};
      bool ok = !mine || route_failed;
      const int off = (j * (H / 2) + r0 / 2 + uu) * 16;
      if (!ok) {
        v = __builtin_amdgcn_raw_buffer_load_b128(dv_r, off, 0, kDevicePoll);
        ok = tag_ok(v, want);
      }
      for (uint32_t it = 0;; ++it) {
        if (__all(ok)) break;
        if (it >= a.wait_polls) {
          if (lane == 0) set_status(a.ctl, a.host_status, kStatusExpertWait);
          break;
        }
        poll_clobber();
        if (!ok) {
          v = __builtin_amdgcn_raw_buffer_load_b128(dv_r, off, 0, kDevicePoll);
          ok = tag_ok(v, want);
        }
      }
      if (mine) {
        const uint32_t d0 = ok ? v.x : 0x7FC00000u, d1 = ok ? v.z : 0x7FC00000u;
        s_d[j * R + 2 * uu] = __builtin_bit_cast(float, d0);
        s_d[j * R + 2 * uu + 1] = __builtin_bit_cast(float, d1);
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    // d_j = its slices' parts summed in slice order; y = sum_j w_j d_j in
    // slot order, plus the shared expert's d
    auto d_of = [&](int j, int rr) {
      float d = s_d[(j * kx) * R + rr];
      for (int kk = 1; kk < kx; ++kk) d += s_d[(j * kx + kk) * R + rr];
      return d;
    };
    for (int rr = lane; rr < nr; rr += kWave) {
      float yv = 0.0f;
      for (int j = 0; j < k; ++j) yv += s_sel_w[j] * d_of(j, rr);
      if (a.has_shared) yv += d_of(k, rr);
      a.y[r0 + rr] = route_failed ? __builtin_nanf("") : yv;
    }
  }

  // ---- 5. the next call's tag -------------------------------------------------------
  if (b == 0 && w == 2) {
    for (int i0 = 0; i0 < G; i0 += kWave) {
      const int i = i0 + lane;
      bool done = i >= G;
      for (uint32_t it = 0;; ++it) {
        if (!done) done = __hip_atomic_load(&a.presence[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == tag64(tag);
        if (__all(done)) break;
        if (it >= a.wait_polls) {
          if (lane == 0) set_status(a.ctl, a.host_status, kStatusPresenceWait);
          break;
        }
        __builtin_amdgcn_s_sleep(2);
      }
    }
    if (lane == 0) __hip_atomic_store(&a.ctl[0], tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

}  // namespace

int stream_kx_max(int64_t KqI) {
  // at most 16 quads of h (16 KiB of tagged units) per workgroup, up to 8 slices
  int kx = 1;
  while (kx < 8 && KqI > 16 * (int64_t)kx) kx *= 2;
  return kx;
}

int stream_kx(int64_t KqI, int G, int S) {
  int kx = stream_kx_max(KqI);
  while (kx > 1 && kx > G / S) kx /= 2;  // every slice of every slot gets a workgroup
  return kx;
}

bool stream_shape_ok(int64_t T, int64_t H, int64_t I, int E, int k, int has_shared) {
  if (T != 1 || E < 1 || E > kMaxExperts || k < 1 || k > kMaxTopK || k > E) return false;
  if (H < kGroup || H % kGroup || I < kGroup || I % kGroup) return false;
  const int64_t Kq = ceil_div(H, kQuad), KqI = ceil_div(I, kQuad);
  // 32-bit buffer sizes of one expert's matrices and of the hand-off regions
  if ((uint64_t)I * Kq * 64 >= kMaxRsrcBytes || (uint64_t)H * KqI * 64 >= kMaxRsrcBytes) return false;
  const int64_t S = k + (has_shared ? 1 : 0);
  if (S * (I / 2) * 16 >= ((int64_t)1 << 31) || S * stream_kx_max(KqI) * (H / 2) * 16 >= ((int64_t)1 << 31)) return false;
  return true;
}

StreamPlan stream_plan(int64_t T, int64_t H, int64_t I, int E, int k, int has_shared) {
  StreamPlan pl = {};
  pl.ok = false;
  const LibConfig cfg = lib_config();
  if (!cfg.decode_fused || !cfg.decode_stream || !stream_shape_ok(T, H, I, E, k, has_shared)) return pl;
  int G = device_cus();
  if (G > kFusedMaxGrid) G = kFusedMaxGrid;
  const int S = k + (has_shared ? 1 : 0);
  if (G < 2 || G < S || (int64_t)G * kFW < E) return pl;
  StreamLds l = {};
  const uint32_t Kq = (uint32_t)((H + kQuad - 1) / kQuad), KqI = (uint32_t)((I + kQuad - 1) / kQuad);
  l.yrows = (int)((H + G - 1) / G);
  l.yrows += l.yrows % 2;  // whole units of two rows
  l.x = 0;
  l.xs = align_lds(Kq * 256u);
  l.lv = align_lds(l.xs + Kq * 16u);
  l.topk = align_lds(l.lv + (uint32_t)E * 8u);
  // a workgroup holds h only for its slice of I, at most ceil(KqI / kx) quads
  const int kx = stream_kx(KqI, G, S);
  l.h = align_lds(l.topk + (uint32_t)k * 40u);
  l.red = align_lds(l.h + ((KqI + (uint32_t)kx - 1u) / (uint32_t)kx) * 512u);
  // the down phase's K-split partials, the combine's expert outputs, and
  // before them the gate/up partials of items cut between waves
  uint32_t red_floats = (uint32_t)(S * kx * l.yrows > kFW * 16 ? S * kx * l.yrows : kFW * 16);
  if (red_floats < (uint32_t)kFW * 2 * 16 * 4 * 2) red_floats = (uint32_t)kFW * 2 * 16 * 4 * 2;
  const uint32_t red_bytes = red_floats * 4u;
  l.ring = align_lds(l.red + red_bytes);
  if (l.ring >= kFusedDynLdsMax) return pl;
  l.ring_wave = ((uint32_t)kFusedDynLdsMax - l.ring) / kFW / 256u * 256u;
  l.ns_gu = (int)(l.ring_wave / kSGuStage);
  l.ns_dn = (int)(l.ring_wave / kSDnStage);
  if (l.ns_gu > kSGuMaxStages) l.ns_gu = kSGuMaxStages;
  if (l.ns_dn > kSDnMaxStages) l.ns_dn = kSDnMaxStages;
  if (l.ns_gu < 2 || l.ns_dn < 2) return pl;
  l.bytes = l.ring + kFW * l.ring_wave;
  pl.G = G;
  pl.kx = kx;
  pl.lds = l;
  pl.ok = true;
  return pl;
}

hipError_t launch_decode_stream(const StreamPlan& pl, const RouteArgs& r, const ExpertArgs& x, const FusedWs& ws,
                                hipStream_t stream) {
  if (!ws.sslots || !ws.hv || !ws.sdv) return hipErrorInvalidValue;  // a workspace planned for another shape
  StreamK a = {};
  a.x = static_cast<const uint16_t*>(r.x);
  a.W = r.router_w;
  a.bias = r.router_bias;
  a.H = (int)r.H;
  a.I = (int)x.I;
  a.E = r.E;
  a.k = r.k;
  a.score_mode = r.score_mode;
  a.has_shared = x.has_shared;
  a.Kq = (int)ceil_div(r.H, kQuad);
  a.KqI = (int)ceil_div(x.I, kQuad);
  a.S = r.k + (x.has_shared ? 1 : 0);
  a.kx = pl.kx;
  a.gate_nib = x.gate_nib;
  a.gate_sc = x.gate_scale;
  a.up_nib = x.up_nib;
  a.up_sc = x.up_scale;
  a.down_nib = x.down_nib;
  a.down_sc = x.down_scale;
  a.sh_gate_nib = x.sh_gate_nib;
  a.sh_gate_sc = x.sh_gate_scale;
  a.sh_up_nib = x.sh_up_nib;
  a.sh_up_sc = x.sh_up_scale;
  a.sh_down_nib = x.sh_down_nib;
  a.sh_down_sc = x.sh_down_scale;
  a.y = x.y;
  a.topk_idx = r.topk_idx;
  a.topk_w = r.topk_w;
  a.ctl = ws.ctl;
  a.presence = ws.presence;
  a.slots = ws.sslots;
  a.hv = ws.hv;
  a.dv = ws.sdv;
  a.lds = pl.lds;
  const LibConfig cfg = lib_config();
  a.host_status = host_status_word();
  a.wait_polls = cfg.fused_wait_polls;
  a.skew_route = (cfg.fused_fault & 1u) ? 1u : 0u;
  a.skew_h = (cfg.fused_fault & 2u) ? 1u : 0u;
  a.skew_gen = (cfg.fused_fault & 4u) ? 1u : 0u;
  static bool attr_set = false;
  if (!attr_set) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(moe_decode_stream_kernel),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)kFusedDynLdsMax);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  hipLaunchKernelGGL(moe_decode_stream_kernel, dim3(pl.G), dim3(kFThreads), pl.lds.bytes, stream, a);
  return hipGetLastError();
}

}  // namespace pmoe
