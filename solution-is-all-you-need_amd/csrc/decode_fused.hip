// decode_fused.hip -- the whole sparse-MoE layer for decode batches of a few
// tokens in ONE launch: router logits, top-k and weights, expert segments,
// gate/up with SwiGLU, and the down projection with the weighted combine.
//
// Reference path: PhantomTopKRouter.forward (tests/test_moe_routing.py:56-72),
// the Q4_0 expert weights (python/phantom/loader/gguf_loader.py:362-381), the
// SwiGLU FFN operator (kernels/sparse_moe/sparse_matmul.cu:120-215) and the
// combine transformers' MoE blocks perform (python/phantom/phantom_cli.py:
// 1393-1430).  It replaces the reference's launch-per-stage, host-blocking
// operator structure (sparse_matmul.cu:256-363, cuda_utils.h:253-257).
//
// Why one launch.  A batch-1 Qwen3-shaped layer reads 22 MB, about 3 us at
// HBM peak, so five dependent launches (each a dispatch plus at least one
// memory round trip) dominate it.  Here every workgroup of one resident grid
// (one per CU) runs the same program, and the program is a chain of phases
// whose length is set by memory round trips and by how many instructions one
// wave issues in a row (a wave issues at most one instruction every four
// cycles), so every phase spreads its work over waves and lanes:
//   0. Waves that own a (token, expert) logit compute it (the router's
//      fixed-order fp64 contract) and publish it at once as a tagged 16-byte
//      slot; the other waves build the MFMA-ordered x operand in LDS.
//   1. Every workgroup polls all T*E slots into LDS and ranks each logit
//      among its token's (value descending, NaN last, ties to the lower
//      index) with all of its threads.
//   2. Wave 0 turns the ranks into expert segments (experts ascending,
//      tokens ascending: the stable permute) while the other waves compute
//      each token's routing weights.  Every workgroup does this from the same
//      logits with the same instructions, so all agree bit for bit.
//   3. Every wave issues all of its weight copies into LDS with direct-to-LDS
//      loads (no registers held, every byte of the layer requested right after
//      routing): gate/up items (segment x 16-row tile of I, K split over the 8
//      waves; item i to workgroup i mod G) and down items (16-row tile of H:
//      every segment x quad of I, contiguous ranges per wave; item d to
//      workgroup G - 1 - d mod G, so the workgroups with fewer gate/up items
//      take them).  The copy list of a wave is worked out lane-parallel first.
//   4. Slot positions and segment tokens, while the copies are in flight.
//   5. Gate/up items as their copies land: MFMA (only the lanes of real
//      segment positions read the x operand), cross-wave sum in wave order,
//      SwiGLU, and h stored device-scope as tagged units {hi|lo of row i, tag,
//      hi|lo of row i + 2, ~tag}: data and readiness in one store, no flag and
//      no wait for the stores to complete.
//   6. Down items: expand the down weights into MFMA operands in registers,
//      then poll the tagged h units of every segment position straight into
//      the down operand in LDS (one memory round trip after the last store),
//      MFMA per (segment, quad), and per output row
//      y[t] = sum_j w[t,j] * (sum_q part[q]) (+ shared expert), j in slot
//      order: the combine is fused, no expert-output round trip.
//
// Hand-off protocol (no memset, no host involvement, graph-replay safe).
// Word 0 of the workspace is a generation counter.  Every wave reads it once
// at start; this call's tag is gen + 1.  Logit slots and h units hold
// {lo32, tag, hi32, ~tag} (one 16-byte store; both halves carry the tag, so a
// torn read cannot pass); presence words hold {tag, ~tag}.  Workgroup 0
// bumps the counter to the tag once every workgroup has published its
// presence (so every wave has read the counter); the next call therefore
// uses a fresh tag and never mistakes this call's data for its own.
// Hand-offs use device-scope (SC1) stores and loads: a device-scope store is
// written through to where every XCD reads, and a device-scope load is never
// served from a stale line of this XCD's L2, so no cache write-back or
// invalidation is needed.
// Every wait is bounded (LibConfig::fused_wait_polls polls); a wait that gives
// up sets a bit of the status word (workspace word 1, read by
// phantom_moe_workspace_status) and its workgroup writes NaN to the outputs
// it owns, so a failure is never silent.  The grid never exceeds one
// workgroup per CU, so with the GPU otherwise idle no wait can deadlock.
#include <math.h>
#include <stdint.h>

#include "expert_common.h"
#include "fused_common.h"
#include "moe_common.h"
#include "moe_launch.h"
#include "topk_common.h"  // logit_key

namespace pmoe {

namespace {

constexpr uint32_t kGuChunkLds = 2304;  // gate nib 1 KB, up nib 1 KB, gate scales 128 B, up scales 128 B
constexpr uint32_t kDnChunkLds = 1152;  // down nib 1 KB, scales 128 B
constexpr int kFusedMaxItems = 4;       // gate/up items per workgroup
constexpr int kPreDq = 5;               // down chunks per wave expanded into registers before h arrives
constexpr int kHUnits = 8;              // tagged h units a thread polls at once

// n / d for 0 <= n < 2^16 and 1 <= d < 2^16 with m = ceil(2^32 / d): the
// error term n * (m - 2^32/d) / 2^32 is below 2^-16 <= 1/d, so the floor is
// exact.
__host__ __device__ inline uint64_t div_magic(uint32_t d) { return ((1ull << 32) + d - 1) / d; }
__device__ inline int fdiv(int n, uint64_t m) { return (int)(((uint64_t)(uint32_t)n * m) >> 32); }

struct FusedK {
  const uint16_t* x;  // [T, H] bf16
  const float* W;     // [E, H]
  const float* bias;  // [E] or null
  int T, H, I, E, k, score_mode, has_shared;
  int Kq, KqI;  // quads of H and of I
  uint64_t md_E, md_nrtI, md_KqI, md_Kq4, md_upos, md_G;  // div_magic of E, I/16, KqI, 4*Kq, 64*KqI, G
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
  uint32_t* ctl;       // [0] generation, [1] status bits
  uint64_t* presence;  // [gridDim.x]
  uint32_t* slots;     // [T * E][4] tagged logits
  uint32_t* hv;        // [T*k + T][I / 2][4] tagged h units
  FusedLds lds;        // dynamic LDS layout
  uint32_t* host_status;  // pinned host word set on a failure, or null
  uint32_t wait_polls;  // bound of every wait
  uint32_t skew_route;  // added to the tag the logit wait expects (non-zero only to test the failure path)
  uint32_t skew_h;      // the same for the h wait
  uint32_t skew_gen;    // added to the counter the last workgroup reads (non-zero only to test a late start)
};


// Position-row stride of the h operand in LDS, padded by 16 bytes so the 16
// rows of an MFMA operand fall in different banks.
__host__ __device__ inline uint32_t h_row_bytes(int KqI) { return (uint32_t)KqI * 512u + 16u; }


// Routing scratch (dead before the first weight copy is issued): the
// logits [T*E] and their order keys [T*E], each wave's top-k scratch (k
// candidate keys, values and indices, k ranked values and indices, k
// exponentials: 40 k bytes), the expert token masks [E] and the ranks of one
// token's logits [E].
struct RouteScratch {
  uint32_t lv, key, topk, topk_wave, emask, rank, bytes;
};
__host__ __device__ inline RouteScratch route_scratch(int T, int k, int E) {
  RouteScratch r;
  r.lv = 0;
  r.key = align_lds((uint32_t)(T * E) * 8u);
  r.topk = r.key + align_lds((uint32_t)(T * E) * 8u);
  r.topk_wave = align_lds((uint32_t)k * 40u);
  r.emask = r.topk + kFW * r.topk_wave;
  r.rank = r.emask + align_lds((uint32_t)E * 8u);
  r.bytes = r.rank + align_lds((uint32_t)E * 4u);
  return r;
}

}  // namespace

// Dynamic LDS layout for ng gate/up and nd down items per workgroup, S_max
// segments:
//   [x operand][gate/up staging][down staging]
// The routing scratch is dead before the first weight copy is issued, so it
// sits over the staging regions.  The h operand and the down partials are
// written after the workgroup's gate/up work is done, so they sit over the x
// operand and the gate/up staging when those are large enough (else after
// the down staging).
FusedLds fused_lds_layout(int T, int k, int E, int has_shared, int H, int I, int ng, int nd, int S_max) {
  FusedLds l = {};
  const uint32_t Kq = (uint32_t)((H + kQuad - 1) / kQuad), KqI = (uint32_t)((I + kQuad - 1) / kQuad);
  const uint32_t npos = (uint32_t)(T * k + (has_shared ? T : 0));
  const uint32_t route = route_scratch(T, k, E).bytes;
  const uint32_t x_op = align_lds((uint32_t)(T + 1) * Kq * 256u) + align_lds((uint32_t)(T + 1) * Kq * 16u);
  // staging slots are indexed (item, wave slot, wave): a wave takes quads
  // w, w + 8, ... of a gate/up item (nq slots) and (segment, quad) pairs
  // [w * per, w * per + per) of a down item
  const uint32_t nq = (Kq + kFW - 1) / kFW;
  const uint32_t per = ((uint32_t)S_max * KqI + kFW - 1) / kFW;
  const uint32_t wgu = (uint32_t)ng * nq * kFW * kGuChunkLds;
  const uint32_t wdn = (uint32_t)nd * per * kFW * kDnChunkLds;
  const uint32_t h_op = align_lds(npos * h_row_bytes((int)KqI));
  const uint32_t dred = align_lds(npos * KqI * 16u * 4u);
  l.x = 0;
  l.wgu = x_op;
  l.wdn = align_lds(l.wgu + wgu);
  const uint32_t w_end = l.wdn + wdn;
  l.route = l.wgu;
  l.h = (h_op + dred <= l.wdn) ? 0u : align_lds(w_end);
  l.dred = l.h + h_op;
  uint32_t end = w_end;
  if (l.route + route > end) end = l.route + route;
  if (l.dred + dred > end) end = l.dred + dred;
  l.bytes = end;
  return l;
}

namespace {

// Expert segments of up to 64 slots (T*k <= 64), built by one wave from
// ballots: slot s (lane s) of expert e goes to position #{slots of experts
// < e} + #{earlier slots of e} (experts ascending, tokens ascending within an
// expert: the stable permute); its segment is #{distinct experts < e}.
// Writes every slot's position, every position's token, the segments
// (expert, begin, size, and the shared expert last) and their count.
__device__ inline void ballot_segments(int T, int k, int E, int has_shared, const int* s_sel_idx, int* s_slot_pos,
                                       int* s_seg_tok, int* s_seg_e, int* s_seg_beg, int* s_seg_cnt, short* s_e2u,
                                       int* s_nseg) {
  const int lane = threadIdx.x % kWave;
  const int nsl = T * k;
  const bool valid = lane < nsl;
  const int e = valid ? s_sel_idx[lane] : 0;
  int nbits = 1;
  while ((1 << nbits) < E) ++nbits;
  const uint64_t lt = (1ull << lane) - 1ull;
  const uint64_t vmask = __ballot(valid);
  uint64_t same = vmask;
  for (int bt = 0; bt < nbits; ++bt) {
    const bool bit = (e >> bt) & 1;
    const uint64_t bb = __ballot(valid && bit);
    same &= bit ? bb : ~bb;
  }
  const int in_seg = __popcll(same & lt);
  const bool first = valid && in_seg == 0;
  const uint64_t firsts = __ballot(first);
  uint64_t m_all = vmask, m_first = firsts;
  int below_all = 0, below_first = 0;
  for (int bt = nbits - 1; bt >= 0; --bt) {
    const uint64_t bb = __ballot(valid && ((e >> bt) & 1));
    if ((e >> bt) & 1) {
      below_all += __popcll(m_all & ~bb);
      below_first += __popcll(m_first & ~bb);
      m_all &= bb;
      m_first &= bb;
    } else {
      m_all &= ~bb;
      m_first &= ~bb;
    }
  }
  const int pos = below_all + in_seg;
  if (valid) {
    s_slot_pos[lane] = pos;
    s_seg_tok[pos] = lane / k;
  }
  if (first) {
    s_seg_e[below_first] = e;
    s_seg_beg[below_first] = below_all;
    s_seg_cnt[below_first] = __popcll(same);
    s_e2u[e] = (short)below_first;
  }
  const int nu = __popcll(firsts);
  if (has_shared && lane < T) s_seg_tok[T * k + lane] = lane;
  if (lane == 0) {
    if (has_shared) {
      s_seg_e[nu] = E;
      s_seg_cnt[nu] = T;
      s_seg_beg[nu] = T * k;
    }
    *s_nseg = nu + (has_shared ? 1 : 0);
  }
}

// The tagged h units [0, nun) of positions pos0, pos0 + 1, ... (upos units a
// position, padding groups included), unit i polled by thread tid + stride * m
// (device scope) and written into the down operand in LDS: unit (g32, half,
// p, r) of a position holds rows cc = 16 half + 4p + r and cc + 2 of group
// g32, which sit at operand entries jj and jj + 1 of group unit
// (p, g32 % 4).  Units of the groups past I are zero.  A wait that gives up
// sets *s_fail and the status bit.
template <int I_>
__device__ inline void poll_h_units(int pos0, int nun, int tid, int stride, BufRsrc hv_r, uint32_t want,
                                    uint32_t wait_polls, uint32_t* ctl, uint32_t* host_status, int* s_fail,
                                    char* s_hb, uint32_t hrow,
                                    int hunits, int upos, int KgI, uint64_t md_upos) {
  const int lane = threadIdx.x % kWave;
  for (int i0 = 0; i0 < nun; i0 += stride * kHUnits) {
    u32x4 v[kHUnits];
    bool ok[kHUnits];
    uint32_t off[kHUnits];
#pragma unroll
    for (int j = 0; j < kHUnits; ++j) {
      const int i = i0 + j * stride + tid;
      const int dp = I_ ? i / (64 * ((I_ + kQuad - 1) / kQuad)) : fdiv(i, md_upos);
      const int uu = i - dp * upos;
      const bool real = i < nun && uu / 16 < KgI;
      off[j] = real ? (uint32_t)(((pos0 + dp) * hunits + uu) * 16) : 0xFFFFF000u;  // past the end: reads zero
      v[j] = __builtin_amdgcn_raw_buffer_load_b128(hv_r, (int)off[j], 0, kDevicePoll);
      ok[j] = !real || tag_ok(v[j], want);
    }
    for (uint32_t it = 0;; ++it) {
      bool all = true;
#pragma unroll
      for (int j = 0; j < kHUnits; ++j) all = all && ok[j];
      if (__all(all)) break;
      if (it >= wait_polls) {
        if (lane == 0) {
          *s_fail = 1;
          set_status(ctl, host_status, kStatusExpertWait);
        }
        break;
      }
      poll_clobber();
#pragma unroll
      for (int j = 0; j < kHUnits; ++j) {
        if (!ok[j]) {
          v[j] = __builtin_amdgcn_raw_buffer_load_b128(hv_r, (int)off[j], 0, kDevicePoll);
          ok[j] = tag_ok(v[j], want);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < kHUnits; ++j) {
      const int i = i0 + j * stride + tid;
      const int dp = I_ ? i / (64 * ((I_ + kQuad - 1) / kQuad)) : fdiv(i, md_upos);
      const int uu = i - dp * upos;
      const bool real = i < nun && uu / 16 < KgI;
      const uint32_t v0 = real ? v[j].x : 0u, v1 = real ? v[j].z : 0u;
      const int g32 = uu / 16, hh = (uu / 8) % 2, pq = (uu / 2) % 4, r = uu % 2;
      if (i < nun) {
        const int jj = hh == 0 ? (r ? 4 : 0) : (r ? 6 : 2);
        char* d = s_hb + (size_t)(pos0 + dp) * hrow + (g32 / 4) * 512 + pq * 128 + (g32 % 4) * 32 + jj * 2;
        *reinterpret_cast<uint32_t*>(d) = (v0 & 0xffffu) | (v1 << 16);
        *reinterpret_cast<uint32_t*>(d + 16) = (v0 >> 16) | (v1 & 0xffff0000u);
      }
    }
  }
}

// Shape parameters known at compile time (0, or -1 for SH, = read at run
// time from the arguments): the generic instantiation reads them all; the
// batch-1 Qwen3-30B-A3B-shaped one knows them all, so every division, loop
// bound and bookkeeping step of a phase folds to constants.
template <int T_, int H_, int I_, int E_, int K_, int SH_>
__global__ __launch_bounds__(kFThreads) void moe_decode_fused_kernel(FusedK a) {
  __shared__ int s_sel_idx[kFusedMaxSlots];
  __shared__ float s_sel_w[kFusedMaxSlots];
  __shared__ double s_sel_v[kMaxTopK];  // one token: the selected logits in slot order
  __shared__ int s_slot_pos[kFusedMaxSlots];
  __shared__ int s_seg_tok[kFusedMaxSlots + kFusedMaxT];
  __shared__ int s_seg_e[kFusedMaxSlots + 1];
  __shared__ int s_seg_beg[kFusedMaxSlots + 1];
  __shared__ int s_seg_cnt[kFusedMaxSlots + 1];
  __shared__ short s_e2u[kMaxExperts];
  // combine: per slot (then per token of the shared expert) the down
  // partials' first index, the step between parts, and the number of parts
  __shared__ int s_cb_base[kFusedMaxSlots + kFusedMaxT];
  __shared__ int s_cb_step[kFusedMaxSlots + kFusedMaxT];
  __shared__ int s_cb_np[kFusedMaxSlots + kFusedMaxT];
  __shared__ int s_nseg;
  __shared__ int s_fail;
  __shared__ int s_pfail[kFusedMaxT];
  extern __shared__ u32x4 s_dyn[];

  const int lane = threadIdx.x % kWave;
  const int w = uni(threadIdx.x / kWave);
  const int n = lane % 16;
  const int p = lane / 16;
  const int G = (int)gridDim.x;
  const int b = (int)blockIdx.x;
  const int T = T_ ? T_ : a.T, H = H_ ? H_ : a.H, I = I_ ? I_ : a.I, E = E_ ? E_ : a.E, k = K_ ? K_ : a.k;
  const int has_sh = SH_ >= 0 ? SH_ : a.has_shared;
  const int Kq = H_ ? (H_ + kQuad - 1) / kQuad : a.Kq, KqI = I_ ? (I_ + kQuad - 1) / kQuad : a.KqI;
  auto div_E = [&](int v) { return E_ ? v / E_ : fdiv(v, a.md_E); };
  auto div_Kq4 = [&](int v) { return H_ ? v / (4 * ((H_ + kQuad - 1) / kQuad)) : fdiv(v, a.md_Kq4); };
  auto div_nrtI = [&](int v) { return I_ ? v / (I_ / kRowTile) : fdiv(v, a.md_nrtI); };
  auto div_KqI = [&](int v) { return I_ ? v / ((I_ + kQuad - 1) / kQuad) : fdiv(v, a.md_KqI); };
  const int Kg = H / kGroup, KgI = I / kGroup;
  const int npos = T * k + (has_sh ? T : 0);
  char* lds = reinterpret_cast<char*>(s_dyn);
  char* rs = lds + a.lds.route;  // routing scratch
  const RouteScratch rl = route_scratch(T, k, E);
  double* s_lv = reinterpret_cast<double*>(rs + rl.lv);
  uint64_t* s_key = reinterpret_cast<uint64_t*>(rs + rl.key);
  uint64_t* s_emask = reinterpret_cast<uint64_t*>(rs + rl.emask);
  int* s_rank = reinterpret_cast<int*>(rs + rl.rank);
  u32x4* s_xop = reinterpret_cast<u32x4*>(lds + a.lds.x);  // [(T+1) Kq][4 p][4 gi]
  float* s_xs = reinterpret_cast<float*>(lds + a.lds.x + align_lds((uint32_t)(T + 1) * Kq * 256u));

  // ---- 0. generation; logits published as computed; x operand -------------
  const uint32_t tag = launch_tag(a.ctl, &a.presence[b], b == G - 1 ? a.skew_gen : 0u);
  const BufRsrc slot_r = buf_rsrc(a.slots, (uint32_t)(T * E * 16));
  // at most one (token, expert) logit per wave: the grid has >= T*E waves
  const int task = w * G + b;
  if (task < T * E) {
    const int t = div_E(task), e = task - t * E;
    double logit = fixed_dot_bf16(a.x + (int64_t)t * H, a.W + (int64_t)e * H, H);
    if (a.bias) logit = logit + (double)a.bias[e];
    if (lane == 0) {
      const uint64_t bits = __builtin_bit_cast(uint64_t, logit);
      u32x4 v;
      v.x = (uint32_t)bits;
      v.y = tag;
      v.z = (uint32_t)(bits >> 32);
      v.w = ~tag;
      __builtin_amdgcn_raw_buffer_store_b128(v, slot_r, task * 16, 0, kDeviceScope);
    }
  }
  // ---- 1. top-k of every token: wave kFW - 1 - t polls token t's logits
  // from the start (the last waves hold no logit unless T*E > 7G) and selects
  // and weighs its experts with the staged router's own instructions
  // (wave_topk_row), so both paths route bit for bit alike.
  const int tpoll = kFW - 1 - w;
  bool poll_failed = false;
  if (tpoll < T) {
    const int t = tpoll;
    const uint32_t want = tag + a.skew_route;
    // every slot of the token in flight at once, then the checks
    constexpr int kNV = kMaxExperts / kWave;
    bool done[kNV];
#pragma unroll
    for (int v = 0; v < kNV; ++v) done[v] = lane + v * kWave >= E;
    for (uint32_t it = 0;; ++it) {
      poll_clobber();
      u32x4 sv[kNV];
#pragma unroll
      for (int v = 0; v < kNV; ++v)
        if (!done[v]) sv[v] = __builtin_amdgcn_raw_buffer_load_b128(slot_r, (t * E + lane + v * kWave) * 16, 0, kDevicePoll);
      bool all = true;
#pragma unroll
      for (int v = 0; v < kNV; ++v) {
        if (!done[v] && tag_ok(sv[v], want)) {
          const double lv = __builtin_bit_cast(double, ((uint64_t)sv[v].z << 32) | sv[v].x);
          s_lv[t * E + lane + v * kWave] = lv;
          s_key[t * E + lane + v * kWave] = logit_key(lv);
          done[v] = true;
        }
        all = all && done[v];
      }
      if (__all(all)) break;
      if (it >= a.wait_polls) {
        poll_failed = true;
        if (lane == 0) set_status(a.ctl, a.host_status, kStatusRouteWait);
        break;
      }
    }
    if (!poll_failed && T == 1) {
      // one token: the whole workgroup ranks its logits (below)
      for (int e = lane; e < E; e += kWave) s_rank[e] = 0;
    } else if (!poll_failed) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      char* tk = rs + rl.topk + (uint32_t)w * rl.topk_wave;
      uint64_t* s_ck = reinterpret_cast<uint64_t*>(tk);
      double* s_cv = reinterpret_cast<double*>(tk + 8 * k);
      double* s_val = reinterpret_cast<double*>(tk + 16 * k);
      double* s_e = reinterpret_cast<double*>(tk + 24 * k);
      int* s_ci = reinterpret_cast<int*>(tk + 32 * k);
      int* s_idx = reinterpret_cast<int*>(tk + 36 * k);
      const double* row = s_lv + t * E;
      int* oi = s_sel_idx + t * k;
      float* ow = s_sel_w + t * k;
      if (E <= 64) wave_topk_row<1>(row, E, k, a.score_mode, s_ck, s_cv, s_ci, s_val, s_idx, s_e, oi, ow, nullptr);
      else if (E <= 128) wave_topk_row<2>(row, E, k, a.score_mode, s_ck, s_cv, s_ci, s_val, s_idx, s_e, oi, ow, nullptr);
      else if (E <= 256) wave_topk_row<4>(row, E, k, a.score_mode, s_ck, s_cv, s_ci, s_val, s_idx, s_e, oi, ow, nullptr);
      else wave_topk_row<8>(row, E, k, a.score_mode, s_ck, s_cv, s_ci, s_val, s_idx, s_e, oi, ow, nullptr);
    }
  }
  // The MFMA-ordered x operand of every token (and an all-zero row T) and its
  // group sums, from the waves in increasing order: one
  // thread per (token, quad, group), the 4 parts p in order; the group sum
  // adds the parts as (p0 + p1) + (p2 + p3), each part ((x0 + x1) + (x2 + x3))
  // + ((x16 + x17) + (x18 + x19)) over its 8 elements.
  for (int j = threadIdx.x; j < (T + 1) * Kq * 4; j += kFThreads) {
    const int tok = div_Kq4(j);
    const int rem = j - tok * Kq * 4;
    const int q = rem / 4;
    const int gi = rem % 4;
    const int g = 4 * q + gi;
    const bool valid = tok < T && g < Kg;
    const uint16_t* xr = a.x + (int64_t)(valid ? tok : 0) * H + (int64_t)(valid ? g : 0) * kGroup;
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
      s_xop[((tok * Kq + q) * 4 + pp) * 4 + gi] = v;
      sp[pp] = ((bf16_bits_to_float(lo.x & 0xffffu) + bf16_bits_to_float(lo.x >> 16)) +
                (bf16_bits_to_float(lo.y & 0xffffu) + bf16_bits_to_float(lo.y >> 16))) +
               ((bf16_bits_to_float(hi.x & 0xffffu) + bf16_bits_to_float(hi.x >> 16)) +
                (bf16_bits_to_float(hi.y & 0xffffu) + bf16_bits_to_float(hi.y >> 16)));
    }
    s_xs[(tok * Kq + q) * 4 + gi] = (sp[0] + sp[1]) + (sp[2] + sp[3]);
  }
  if (threadIdx.x == 0) s_fail = 0;
  if (tpoll < T && lane == 0) s_pfail[tpoll] = poll_failed ? 1 : 0;
  asm volatile("" ::"s"(tag));  // this wave's counter and presence loads have returned
  lds_barrier();                // every wave of the workgroup has read the generation
  if (threadIdx.x == 0) __hip_atomic_store(&a.presence[b], tag64(tag), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  int pf = 0;
  for (int t = 0; t < T; ++t) pf |= s_pfail[t];
  const bool route_failed = uni(pf) != 0;

  // One token: every logit's rank among the E (the number of logits before
  // it in the order of wave_topk_row: value descending, NaN last, ties to the
  // lower index), P threads per logit over E/P keys each; rank r < k is slot
  // r.  Then wave 0 takes the winners to their slots and segments (experts
  // ascending) while wave 1 gathers the selected logits in slot order; the
  // weights (only the combine and the routing outputs need them) are
  // computed after the weight copies are issued, exactly as wave_topk_row
  // computes them, so the selection, its order and the weights equal the
  // staged router's bit for bit.
  if (T == 1 && !route_failed) {
    int P = 1;
    while (2 * P * E <= kFThreads) P *= 2;
    const int span = (E + P - 1) / P;
    if ((int)threadIdx.x < E * P) {
      const int pp = div_E(threadIdx.x);
      const int e = (int)threadIdx.x - pp * E;
      const uint64_t ke = s_key[e];
      const int j0 = pp * span;
      const int j1 = j0 + span < E ? j0 + span : E;
      int cnt = 0;
      int j = j0;
      for (; j + 8 <= j1; j += 8) {
        uint64_t kk[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) kk[q] = s_key[j + q];
#pragma unroll
        for (int q = 0; q < 8; ++q) cnt += (kk[q] > ke || (kk[q] == ke && j + q < e)) ? 1 : 0;
      }
      for (; j < j1; ++j) {
        const uint64_t kj = s_key[j];
        cnt += (kj > ke || (kj == ke && j < e)) ? 1 : 0;
      }
      if (P == 1) s_rank[e] = cnt;
      else atomicAdd(&s_rank[e], cnt);
    }
    lds_barrier();
    if (w == 0) {
      const uint64_t lt = (1ull << lane) - 1ull;
      int nsel = 0;
      for (int e0 = 0; e0 < E; e0 += kWave) {
        const int e = e0 + lane;
        const int r = e < E ? s_rank[e] : k;
        const bool sel = r < k;
        const uint64_t bal = __ballot(sel);
        if (sel) {
          const int u = nsel + __popcll(bal & lt);
          s_seg_e[u] = e;
          s_seg_beg[u] = u;
          s_seg_cnt[u] = 1;
          s_seg_tok[u] = 0;
          s_e2u[e] = (short)u;
          s_sel_idx[r] = e;
          s_slot_pos[r] = u;
        }
        nsel += __popcll(bal);
      }
      if (lane == 0) {
        if (has_sh) {
          s_seg_e[k] = E;
          s_seg_cnt[k] = 1;
          s_seg_beg[k] = k;
          s_seg_tok[k] = 0;
        }
        s_nseg = k + (has_sh ? 1 : 0);
      }
    } else if (w == 1) {
      for (int e = lane; e < E; e += kWave) {
        const int r = s_rank[e];
        if (r < k) s_sel_v[r] = s_lv[e];
      }
    }
    lds_barrier();
  }

  // ---- 2. expert segments (experts ascending, tokens ascending within one:
  // the stable permute) -------------------------------------------------------
  if (!route_failed && T > 1) {
    if (T * k <= kWave) {
      if (w == 0)
        ballot_segments(T, k, E, has_sh, s_sel_idx, s_slot_pos, s_seg_tok, s_seg_e, s_seg_beg, s_seg_cnt,
                        s_e2u, &s_nseg);
    } else {
      for (int e = threadIdx.x; e < E; e += kFThreads) s_emask[e] = 0;
      lds_barrier();
      for (int s2 = threadIdx.x; s2 < T * k; s2 += kFThreads)
        __hip_atomic_fetch_or(&s_emask[s_sel_idx[s2]], 1ull << (s2 / k), __ATOMIC_RELAXED,
                              __HIP_MEMORY_SCOPE_WORKGROUP);
      lds_barrier();
      if (w == 0) {
        // active experts in increasing id, their segment sizes and offsets
        const uint64_t lt = (1ull << lane) - 1ull;
        int nu = 0, run = 0;
        for (int e0 = 0; e0 < E; e0 += kWave) {
          const int e = e0 + lane;
          const uint64_t m = e < E ? s_emask[e] : 0ull;
          const int c = __popcll(m);
          const uint64_t bal = __ballot(m != 0ull);
          int inc = c;
#pragma unroll
          for (int off = 1; off < kWave; off <<= 1) {
            const int o = __shfl_up(inc, off, kWave);
            if (lane >= off) inc += o;
          }
          if (m != 0ull) {
            const int u = nu + __popcll(bal & lt);
            s_seg_e[u] = e;
            s_seg_cnt[u] = c;
            s_seg_beg[u] = run + inc - c;
            s_e2u[e] = (short)u;
          }
          nu += __popcll(bal);
          run += __shfl(inc, kWave - 1, kWave);
        }
        if (lane == 0) {
          if (has_sh) {
            s_seg_e[nu] = E;
            s_seg_cnt[nu] = T;
            s_seg_beg[nu] = T * k;
          }
          s_nseg = nu + (has_sh ? 1 : 0);
        }
      }
      lds_barrier();
      // every slot's segment position and every position's token
      for (int s2 = threadIdx.x; s2 < T * k; s2 += kFThreads) {
        const int t = s2 / k;
        const int e = s_sel_idx[s2];
        const int pos = s_seg_beg[s_e2u[e]] + __popcll(s_emask[e] & ((1ull << t) - 1ull));
        s_slot_pos[s2] = pos;
        s_seg_tok[pos] = t;
      }
      if (has_sh)
        for (int t = threadIdx.x; t < T; t += kFThreads) s_seg_tok[T * k + t] = t;
    }
    lds_barrier();
  }

  // ---- 3. work lists; every weight chunk of the workgroup -> LDS ------------
  // One token: k segments of one position each (segment u at position u),
  // plus the shared expert's; known without reading the routing results.
  const bool one_tok = T == 1;
  const int S = route_failed ? 0 : (one_tok ? k + has_sh : uni(s_nseg));
  auto seg_beg = [&](int u) { return one_tok ? u : uni(s_seg_beg[u]); };
  auto seg_cnt = [&](int u) { return one_tok ? 1 : uni(s_seg_cnt[u]); };
  const int nrtI = I / kRowTile;
  const int n_gu = S * nrtI;
  const int n_dn = H / kRowTile;
  // gate/up items b, b + G, ...; down items G - 1 - b, G - 1 - b + G, ...
  const int ng = b < n_gu ? fdiv(n_gu - b + G - 1, a.md_G) : 0;
  const int dn_first = G - 1 - b;
  const int nd = (S > 0 && dn_first < n_dn) ? fdiv(n_dn - dn_first + G - 1, a.md_G) : 0;
  // gate/up: wave w takes quads w, w + 8, ... (nqw of them) of each item
  const int nq = (Kq + kFW - 1) / kFW;
  const int nqw = Kq > w ? (Kq - 1 - w) / kFW + 1 : 0;
  // down: wave w takes (segment, quad) pairs [w * per, w * per + cnt_w) of each item
  const int n_c = S * KqI;
  const int per = (n_c + kFW - 1) / kFW;
  const int cnt_w = (n_c - w * per) < per ? ((n_c - w * per) > 0 ? n_c - w * per : 0) : per;
  const int gu_copies = ng * nqw * 4;  // vmcnt entries: gate nibbles, up nibbles, gate scales, up scales

  // each gate/up item's row tile of I and segment
  int it_rt[kFusedMaxItems], it_e[kFusedMaxItems], it_beg[kFusedMaxItems], it_cnt[kFusedMaxItems];
#pragma unroll
  for (int ii = 0; ii < kFusedMaxItems; ++ii) {
    it_rt[ii] = it_e[ii] = it_beg[ii] = it_cnt[ii] = 0;
    if (ii < ng) {
      const int item = b + ii * G;
      const int u = div_nrtI(item);
      it_rt[ii] = item - u * nrtI;
      it_e[ii] = uni(s_seg_e[u]);
      it_beg[ii] = seg_beg(u);
      it_cnt[ii] = seg_cnt(u);
    }
  }
  // lane c < cnt_w: the expert and quad of this wave's c-th down pair
  int my_e = 0, my_q = 0;
  if (nd > 0 && lane < cnt_w) {
    const int pair = w * per + lane;
    const int u = div_KqI(pair);
    my_q = pair - u * KqI;
    my_e = s_seg_e[u];
  }

  const uint32_t gnib_bytes = (uint32_t)I * (uint32_t)Kq * 64u;  // one expert's gate (or up) nibbles
  const uint32_t gsc_bytes = (uint32_t)I * (uint32_t)Kq * 8u;
  const uint32_t dnib_bytes = (uint32_t)H * (uint32_t)KqI * 64u;
  const uint32_t dsc_bytes = (uint32_t)H * (uint32_t)KqI * 8u;
  auto stack = [&](uint32_t one) {
    const uint64_t t = (uint64_t)one * (uint64_t)E;
    return (uint32_t)(t < kMaxRsrcBytes ? t : kMaxRsrcBytes);
  };
  char* wgu = lds + a.lds.wgu;
  char* wdn = lds + a.lds.wdn;
#pragma unroll
  for (int ii = 0; ii < kFusedMaxItems; ++ii) {
    if (ii < ng) {
      const int e = it_e[ii];
      const bool routed = e < E;
      const BufRsrc gn = routed ? buf_rsrc(a.gate_nib, stack(gnib_bytes)) : buf_rsrc(a.sh_gate_nib, gnib_bytes);
      const BufRsrc un = routed ? buf_rsrc(a.up_nib, stack(gnib_bytes)) : buf_rsrc(a.sh_up_nib, gnib_bytes);
      const BufRsrc gs = routed ? buf_rsrc(a.gate_sc, stack(gsc_bytes)) : buf_rsrc(a.sh_gate_sc, gsc_bytes);
      const BufRsrc us = routed ? buf_rsrc(a.up_sc, stack(gsc_bytes)) : buf_rsrc(a.sh_up_sc, gsc_bytes);
      const uint32_t eo_n = routed ? (uint32_t)e * gnib_bytes : 0u;
      const uint32_t eo_s = routed ? (uint32_t)e * gsc_bytes : 0u;
      for (int qq = 0; qq < nqw; ++qq) {
        const int q = w + kFW * qq;
        const uint32_t tq = (uint32_t)(it_rt[ii] * Kq + q);
        char* slot = wgu + ((ii * nq + qq) * kFW + w) * kGuChunkLds;
        dma_b128(gn, slot, (uint32_t)lane * 16u, eo_n + tq * kQuadNibBytes);
        dma_b128(un, slot + 1024, (uint32_t)lane * 16u, eo_n + tq * kQuadNibBytes);
        // scales: 32 lanes x 4 bytes each for gate, the other 32 for up
        if (lane < 32) dma_b32(gs, slot + 2048, (uint32_t)lane * 4u, eo_s + tq * (kQuadScales * 2));
        else dma_b32(us, slot + 2048, (uint32_t)(lane - 32) * 4u, eo_s + tq * (kQuadScales * 2));
      }
    }
  }
  // The down copies go out once this workgroup's h stores are issued (at
  // once without gate/up items): the gate/up weights, which the h hand-off
  // waits for, then share HBM with little else, and the down weights land
  // during the hand-off (Qwen3 batch 1: 18.3 -> 17.5 us).
  auto issue_down = [&]() {
  for (int dd = 0; dd < nd; ++dd) {
    const int rH = dn_first + dd * G;
    for (int cc = 0; cc < cnt_w; ++cc) {
      const int e = __builtin_amdgcn_readlane(my_e, cc);
      const int q = __builtin_amdgcn_readlane(my_q, cc);
      const bool routed = e < E;
      const BufRsrc dn = routed ? buf_rsrc(a.down_nib, stack(dnib_bytes)) : buf_rsrc(a.sh_down_nib, dnib_bytes);
      const BufRsrc ds = routed ? buf_rsrc(a.down_sc, stack(dsc_bytes)) : buf_rsrc(a.sh_down_sc, dsc_bytes);
      const uint32_t tq = (uint32_t)(rH * KqI + q);
      char* slot = wdn + ((dd * per + cc) * kFW + w) * kDnChunkLds;
      dma_b128(dn, slot, (uint32_t)lane * 16u, (routed ? (uint32_t)e * dnib_bytes : 0u) + tq * kQuadNibBytes);
      if (lane < 32)
        dma_b32(ds, slot + 1024, (uint32_t)lane * 4u, (routed ? (uint32_t)e * dsc_bytes : 0u) + tq * (kQuadScales * 2));
    }
  }
  };
  if (ng == 0) issue_down();

  // ---- 4. routing outputs and the combine's tables, while the copies land ----
  if (T == 1 && !route_failed && w == 1) {
    // one token's weights (softmax over the selected logits, or sigmoid
    // renormalised), summed in slot order as wave_topk_row sums them
    double ej = 0.0;
    if (lane < k) {
      const double v = s_sel_v[lane];
      ej = (a.score_mode == 0) ? exp(v - s_sel_v[0]) : 1.0 / (1.0 + exp(-v));
    }
    double sum = 0.0;
    for (int i = 0; i < k; ++i) sum += __shfl(ej, i, kWave);
    if (lane < k) {
      const float wt = (float)(ej / sum);
      s_sel_w[lane] = wt;
      if (b == 0) a.topk_w[lane] = wt;
    }
  }
  if (b == 0)
    for (int i = threadIdx.x; i < T * k; i += kFThreads) {
      a.topk_idx[i] = route_failed ? -1 : s_sel_idx[i];
      if (T > 1 || route_failed) a.topk_w[i] = route_failed ? __builtin_nanf("") : s_sel_w[i];
    }
  // the combine's tables: slot s at position pos of segment u reads part pt
  // of output row nn at (beg * KqI + pt * cnt + pos - beg) * 16 + nn, u's
  // parts being the waves its (segment, quad) pairs fall to
  if (S > 0 && nd > 0) {
    for (int s = threadIdx.x; s < T * k + (has_sh ? T : 0); s += kFThreads) {
      const bool sh = s >= T * k;
      const int u = sh ? S - 1 : s_e2u[s_sel_idx[s]];
      const int pos = sh ? s : s_slot_pos[s];
      const int beg = one_tok ? u : s_seg_beg[u], cnt = one_tok ? 1 : s_seg_cnt[u];  // u differs across lanes
      s_cb_base[s] = (beg * KqI + pos - beg) * 16;
      s_cb_step[s] = cnt * 16;
      s_cb_np[s] = ((u + 1) * KqI - 1) / per - (u * KqI) / per + 1;
    }
  }

  // ---- 5. gate/up items ----------------------------------------------------
  // Items in copy order, each as soon as its copies have landed, the
  // accumulators in registers; then one reduction for all items: each wave
  // writes its partial sums over its own first staging slot of the item
  // (read by nobody else, and dead once the wave's MFMAs are done), one
  // barrier, and the SwiGLU epilogue of every item spread over the workgroup.
  const int hunits = I / 2;  // tagged h units per segment position
  const BufRsrc hv_r = buf_rsrc(a.hv, (uint32_t)(npos * hunits * 16));
  const f32x4 z = {0.f, 0.f, 0.f, 0.f};
  // The down weights of a single item are expanded into MFMA operands
  // (fp16 n - 8 and fp32 scales) while h is on its way, so that only MFMAs
  // remain once it has arrived.
  const uint32_t dmask = vgpr_const(0x000F000Fu);
  const bool pre = nd == 1;  // the first kPreDq chunks of a single item
  u32x4 pbb[kPreDq][4];
  float pdv[kPreDq][4];
  auto expand_down = [&]() {
    wait_vmcnt<0>();  // this wave's down copies
    if (pre) {
#pragma unroll
      for (int c = 0; c < kPreDq; ++c) {
        if (c < cnt_w) {
          const char* slot = wdn + (c * kFW + w) * kDnChunkLds;
          const u32x4 wv = *reinterpret_cast<const u32x4*>(slot + lane * 16);
          unpack_scales(*reinterpret_cast<const uint2*>(slot + 1024 + n * 8), pdv[c]);
          pbb[c][0] = dequant_unit_f16s(wv.x, dmask);
          pbb[c][1] = dequant_unit_f16s(wv.y, dmask);
          pbb[c][2] = dequant_unit_f16s(wv.z, dmask);
          pbb[c][3] = dequant_unit_f16s(wv.w, dmask);
        }
      }
    }
  };
  if (ng > 0) {
    const uint32_t mask = vgpr_const(0x00780078u);
    f32x4 ag[kFusedMaxItems], au[kFusedMaxItems], cg[kFusedMaxItems], cu[kFusedMaxItems];
    // Only the lanes of real segment positions read the x operand; the
    // others keep whatever they hold: an MFMA row of A feeds only the same
    // row of the result, and those rows are never read.
    u32x4 xa[4] = {{0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}};
    float sx = 0.0f;
#pragma unroll
    for (int ii = 0; ii < kFusedMaxItems; ++ii) {
      ag[ii] = au[ii] = cg[ii] = cu[ii] = z;
      if (ii < ng) {
        const bool pv = n < it_cnt[ii];
        const int tok = pv ? s_seg_tok[it_beg[ii] + n] : 0;
        wait_vmcnt_le(gu_copies - (ii + 1) * nqw * 4);  // this item's copies
        for (int qq = 0; qq < nqw; ++qq) {
          const int q = w + kFW * qq;
          const char* slot = wgu + ((ii * nq + qq) * kFW + w) * kGuChunkLds;
          const u32x4 gw = *reinterpret_cast<const u32x4*>(slot + lane * 16);
          const u32x4 uw = *reinterpret_cast<const u32x4*>(slot + 1024 + lane * 16);
          const uint2 gsv = *reinterpret_cast<const uint2*>(slot + 2048 + n * 8);
          const uint2 usv = *reinterpret_cast<const uint2*>(slot + 2176 + n * 8);
          if (pv) {
            const u32x4* xo = s_xop + ((tok * Kq + q) * 4 + p) * 4;
            xa[0] = xo[0];
            xa[1] = xo[1];
            xa[2] = xo[2];
            xa[3] = xo[3];
            sx = s_xs[(tok * Kq + q) * 4 + p];
          }
          float dg[4], du[4];
          unpack_scales(gsv, dg);
          unpack_scales(usv, du);
          const uint32_t gwv[4] = {gw.x, gw.y, gw.z, gw.w};
          const uint32_t uwv[4] = {uw.x, uw.y, uw.z, uw.w};
          f32x4 pg[4], pu[4];
#pragma unroll
          for (int gi = 0; gi < 4; ++gi) {
            pg[gi] = mfma_bf16_16x16x32(xa[gi], dequant_unit_bf16(gwv[gi], mask), z);
            pu[gi] = mfma_bf16_16x16x32(xa[gi], dequant_unit_bf16(uwv[gi], mask), z);
          }
          cg[ii] = mfma_f32_16x16x4(sx, dg[p], cg[ii]);
          cu[ii] = mfma_f32_16x16x4(sx, du[p], cu[ii]);
#pragma unroll
          for (int gi = 0; gi < 4; ++gi) {
            ag[ii] += dg[gi] * pg[gi];
            au[ii] += du[gi] * pu[gi];
          }
        }
      }
    }
#pragma unroll
    for (int ii = 0; ii < kFusedMaxItems; ++ii) {
      if (ii < ng) {
        float* red = reinterpret_cast<float*>(wgu + ((ii * nq) * kFW + w) * kGuChunkLds);  // [gate/up][16][16]
        const f32x4 rg = kUnitScale * ag[ii] - kUnitBias * cg[ii];
        const f32x4 ru = kUnitScale * au[ii] - kUnitBias * cu[ii];
        // lane (n, p) holds positions 4p + j of output row n; only real
        // positions are read back
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (4 * p + j < it_cnt[ii]) {
            red[(4 * p + j) * 16 + n] = rg[j];
            red[256 + (4 * p + j) * 16 + n] = ru[j];
          }
        }
      }
    }
    lds_barrier();
    for (int o = threadIdx.x; o < ng * 256; o += kFThreads) {
      const int ii = o / 256;  // wave-uniform
      const int mm = (o % 256) / 16;
      const int nn = o % 16;
      const int item = b + ii * G;
      const int u = div_nrtI(item);
      const int rt = item - u * nrtI;
      const int beg = seg_beg(u), cnt = seg_cnt(u);
      const bool ok = mm < cnt;
      uint32_t v = 0u;
      if (ok) {
        const float* red0 = reinterpret_cast<const float*>(wgu + ((ii * nq) * kFW) * kGuChunkLds);
        float gv[kFW], uv[kFW];
#pragma unroll
        for (int s2 = 0; s2 < kFW; ++s2) {
          gv[s2] = red0[s2 * (kGuChunkLds / 4) + mm * 16 + nn];
          uv[s2] = red0[s2 * (kGuChunkLds / 4) + 256 + mm * 16 + nn];
        }
        float g = 0.0f, uu = 0.0f;
#pragma unroll
        for (int s2 = 0; s2 < kFW; ++s2) {
          g += gv[s2];
          uu += uv[s2];
        }
        const float h = g * (1.0f / (1.0f + expf(-g))) * uu;
        const uint32_t hb = float_to_half_bits(h);
        const uint32_t lb = float_to_half_bits(h - half_bits_to_float32(hb));
        v = hb | (lb << 16);
      }
      // the unit of rows cc and cc + 2 of a half-group (cc % 4 < 2) is
      // stored by the lane of row cc with its partner's value
      const uint32_t v2 = __shfl_down(v, 2, kWave);
      if (ok && (nn & 2) == 0) {
        const int i = rt * 16 + nn;  // row of I
        const int unit = (i / kGroup) * 16 + (rt & 1) * 8 + (nn >> 2) * 2 + (nn & 1);
        u32x4 hvv;
        hvv.x = v;
        hvv.y = tag;
        hvv.z = v2;
        hvv.w = ~tag;
        __builtin_amdgcn_raw_buffer_store_b128(hvv, hv_r, ((beg + mm) * hunits + unit) * 16, 0, kDeviceScope);
      }
    }
  }
  if (ng > 0 && nd > 0) issue_down();
  if (nd > 0) expand_down();

  // ---- 6. down items with the combine --------------------------------------
  if (nd > 0) {
    lds_barrier();  // every wave's gate/up epilogue has read its partials: the h region is free
    // h of every segment position, polled into the down operand (poll_h_units)
    const uint32_t hrow = h_row_bytes(KqI);
    char* s_hb = lds + a.lds.h;
    float* s_dred = reinterpret_cast<float*>(lds + a.lds.dred);
    const int upos = KqI * 64;  // h units per position, padding groups included
    // When every wave's (segment, quad) pairs are exactly one segment (wave w:
    // segment w), each wave polls the h of its own segment and goes on to its
    // MFMAs as soon as that has arrived; otherwise the workgroup polls all of
    // h and meets at a barrier.
    const bool seg_wave = per == KqI;
    if (seg_wave) {
      if (w < S)
        poll_h_units<I_>(seg_beg(w), seg_cnt(w) * upos, lane, kWave, hv_r, tag + a.skew_h, a.wait_polls,
                         a.ctl, a.host_status, &s_fail, s_hb, hrow, hunits, upos, KgI, a.md_upos);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
    } else {
      poll_h_units<I_>(0, npos * upos, (int)threadIdx.x, kFThreads, hv_r, tag + a.skew_h, a.wait_polls, a.ctl,
                       a.host_status, &s_fail, s_hb, hrow, hunits, upos, KgI, a.md_upos);
      lds_barrier();
    }
    // The h operand of position m of a segment sits in MFMA rows 2m (fp16 hi)
    // and 2m + 1 (fp16 lo), so one MFMA per group multiplies both halves
    // (segments hold at most 8 positions).  Only those lanes read it; the
    // others keep whatever they hold (those result rows are never used).
    u32x4 hh[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) hh[r] = u32x4{0u, 0u, 0u, 0u};
    for (int dd = 0; dd < nd; ++dd) {
      // The wave's pairs [w * per, w * per + per) in (segment, quad) order:
      // consecutive quads of one segment accumulate in registers; at a
      // segment's last pair in the range the partial sum goes to LDS as part
      // w - (first wave of the segment), real positions only.
      f32x4 acc = z;
      auto chunk = [&](int cc, const u32x4 (&bb)[4], const float (&dv)[4]) {
        const int pair = w * per + cc;
        const int u = div_KqI(pair);
        const int q = pair - u * KqI;
        const int beg = seg_beg(u), cnt = seg_cnt(u);
        if (n < 2 * cnt) {
          const u32x4* ho = reinterpret_cast<const u32x4*>(s_hb + (size_t)(beg + n / 2) * hrow + q * 512 + p * 128 +
                                                            (n & 1) * 16);
#pragma unroll
          for (int gi = 0; gi < 4; ++gi) hh[gi] = ho[2 * gi];
        }
#pragma unroll
        for (int gi = 0; gi < 4; ++gi) acc += dv[gi] * mfma_f16_16x16x32(hh[gi], bb[gi], z);
        if (q == KqI - 1 || cc == per - 1 || pair + 1 == n_c) {
          const int part = w - (u * KqI) / per;
          // lane (n, p) holds rows 4p + j of output row n: positions 2p
          // (hi + lo in rows 4p, 4p + 1) and 2p + 1
          const float r0 = acc[0] + acc[1], r1 = acc[2] + acc[3];
          float* dst = s_dred + (beg * KqI + part * cnt) * 16 + n;
          if (2 * p < cnt) dst[(2 * p) * 16] = r0;
          if (2 * p + 1 < cnt) dst[(2 * p + 1) * 16] = r1;
          acc = z;
        }
      };
      int c0 = 0;
      if (pre) {
#pragma unroll
        for (int c = 0; c < kPreDq; ++c)
          if (c < cnt_w) chunk(c, pbb[c], pdv[c]);
        c0 = kPreDq;
      }
      for (int cc = c0; cc < cnt_w; ++cc) {
        const char* slot = wdn + ((dd * per + cc) * kFW + w) * kDnChunkLds;
        const u32x4 wv = *reinterpret_cast<const u32x4*>(slot + lane * 16);
        float dv[4];
        unpack_scales(*reinterpret_cast<const uint2*>(slot + 1024 + n * 8), dv);
        const u32x4 bb[4] = {dequant_unit_f16s(wv.x, dmask), dequant_unit_f16s(wv.y, dmask),
                             dequant_unit_f16s(wv.z, dmask), dequant_unit_f16s(wv.w, dmask)};
        chunk(cc, bb, dv);
      }
      lds_barrier();
      const bool h_failed = uni(s_fail) != 0;
      const int rH = dn_first + dd * G;
      if (threadIdx.x < T * 16) {
        // the slots' tables and partials are independent loads, issued eight
        // slots at a time; the sums run in slot order
        const int t = threadIdx.x / 16;
        const int nn = threadIdx.x % 16;
        float acc_y = 0.0f;
        for (int j0 = 0; j0 < k; j0 += 8) {
          float sq[8], wj[8];
#pragma unroll
          for (int jj = 0; jj < 8; ++jj) {
            const int s = t * k + (j0 + jj < k ? j0 + jj : k - 1);
            const int base = s_cb_base[s] + nn, step = s_cb_step[s], np = s_cb_np[s];
            wj[jj] = s_sel_w[s];
            sq[jj] = s_dred[base];
            for (int pt = 1; pt < np; ++pt) sq[jj] += s_dred[base + pt * step];
          }
#pragma unroll
          for (int jj = 0; jj < 8; ++jj)
            if (j0 + jj < k) acc_y += wj[jj] * sq[jj];
        }
        if (has_sh) {
          const int s = T * k + t;
          const int base = s_cb_base[s] + nn, step = s_cb_step[s], np = s_cb_np[s];
          float sq = s_dred[base];
          for (int pt = 1; pt < np; ++pt) sq += s_dred[base + pt * step];
          acc_y += sq;
        }
        a.y[(int64_t)t * H + rH * 16 + nn] = h_failed ? __builtin_nanf("") : acc_y;
      }
      lds_barrier();  // s_dred is free for the next item
    }
  }
  if (S == 0 && dn_first < n_dn) {
    // routing failed: this workgroup's rows of y are NaN
    for (int dd = dn_first; dd < n_dn; dd += G)
      for (int i = threadIdx.x; i < T * 16; i += kFThreads) a.y[(int64_t)(i / 16) * H + dd * 16 + i % 16] = __builtin_nanf("");
  }

  // ---- 7. the next call's tag --------------------------------------------------
  if (b == 0 && w == 0) {
    // every wave has read the generation once its workgroup's presence is here
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

// ---------------------------------------------- batch 1, top-8, one XCD a slot
//
// One token with eight routed experts and no shared expert on an 8-XCD part
// (the batch-1 Qwen3-30B-A3B-shaped layer).  Selected expert j (slot j of
// the top-k order) runs entirely on XCD j, on the 32 workgroups the
// dispatcher places there.  It deals workgroups to the XCDs round-robin, so
// b, b + 8, b + 16, ... share an XCD, but the XCD the deal starts on varies
// between launches (graph replays start elsewhere than eager launches): each
// workgroup reads its XCD from the hardware XCC_ID register and takes
// b / 8 as its rank on it.  Every hand-off after routing but the last then
// stays inside one XCD's L2 and moves a few KB:
//   0. Logit e is computed once, by wave 0 of workgroup e (the router's
//      fixed-order fp64 contract), and published device-scope as a tagged
//      slot; the slots sit kX8SlotStride bytes apart, so the polls of all
//      256 workgroups spread over the memory channels.
//   1. Every workgroup polls the E slots and ranks the logits (branch-free
//      counts of larger keys, then equal keys ordered by index) and computes
//      the weights exactly as the generic kernel does.
//   2. The workgroup's weight copies, every wave its own share: gate/up in
//      half tiles (8 rows of I of gate and the same 8 rows of up make one
//      MFMA B operand, so the 96 half tiles of an expert are 3 per
//      workgroup) over the 16 quads of H; then, once those have landed, 4
//      row tiles of H of down over all of I.
//   3. Gate/up as the generic kernel computes it (bf16 offset operands, the
//      offset by one fp32 MFMA), the 8 waves' K-split partials summed in wave
//      order, SwiGLU, and h stored to the XCD's L2 as tagged units
//      {hi(i) | hi(i+1), tag, lo(i) | lo(i+1), ~tag}.
//   4. With its down weights already expanded into registers, every
//      workgroup polls the I / 2 h units of its XCD into the down operand
//      (MFMA rows 0 and 1 = fp16 hi and lo of h).
//   5. Down rows [64 rho, 64 rho + 64) of slot j's expert (rho = b / 8); the
//      partial outputs go out device-scope as tagged units, and workgroup
//      (j, rho) combines rows 64 rho + 8 j .. + 8 over the 8 slots in slot
//      order, y = sum_j w_j d_j: the only cross-XCD hand-off after routing.
// A workgroup that gives up a wait still publishes what the others wait for
// (NaN values), so a failure costs one bounded wait, sets a status bit and
// leaves NaN in the outputs it touches.
namespace {

constexpr int kX8Xcds = 8;
constexpr int kX8Grid = 256;
constexpr int kX8PerXcd = kX8Grid / kX8Xcds;
constexpr uint32_t kX8Chunk = 1152;  // 1 KiB of nibbles + 128 B of scales
// Byte stride of the device-scope logit slots.  Every workgroup polls all
// of them; slots 16 bytes apart put all those polls on a few memory
// channels (C1 13.95 us a layer, against 13.63 at 256 bytes and 13.82 with
// one poller per XCD relaying the logits through its L2).
constexpr uint32_t kX8SlotStride = 256;
// Cache policy of a poll of data another CU of this XCD stored: SC0 (not
// served by this CU's L1; this XCD's L2 holds the latest copy), with the
// intrinsic's volatile bit as in kDevicePoll.
constexpr int kXcdPoll = 1 | (int)0x80000000u;

struct X8K {
  const uint16_t* x;
  const float* W;
  const float* bias;
  int score_mode;
  const uint8_t* gate_nib;
  const uint16_t* gate_sc;
  const uint8_t* up_nib;
  const uint16_t* up_sc;
  const uint8_t* down_nib;
  const uint16_t* down_sc;
  float* y;
  int32_t* topk_idx;
  float* topk_w;
  uint32_t* ctl;
  uint64_t* presence;
  uint32_t* xslots;  // [E] device-scope tagged logits, kX8SlotStride bytes apart
  uint32_t* xh;      // [8][I / 2][4] tagged h units
  uint32_t* xpart;   // [8][H / 2][4] tagged down partials (device scope)
  uint32_t* host_status;
  uint32_t wait_polls;
  uint32_t skew_route;
  uint32_t skew_h;
  uint32_t skew_gen;
};

// The nibble expansions of dequant_unit_bf16 and dequant_unit_f16s as plain
// expressions.  Instructions written in inline assembly are invisible to the
// compiler's hazard checks, and this kernel keeps one element of its MFMA
// results (the token's row), so the compiler reuses the other elements'
// registers right after an MFMA issues: an inline-assembly write there is
// not held back, and the MFMA's own later write of that register then
// clobbers it (seen as wrong, run-to-run varying gate/up sums).
__device__ inline u32x4 x8_dequant_bf16(uint32_t w) {
  u32x4 r;
  r.x = ((w << 3) & 0x00780078u) | 0x3F803F80u;
  r.y = ((w >> 1) & 0x00780078u) | 0x3F803F80u;
  r.z = ((w >> 5) & 0x00780078u) | 0x3F803F80u;
  r.w = ((w >> 9) & 0x00780078u) | 0x3F803F80u;
  return r;
}
__device__ inline uint32_t x8_nib_pair_f16s(uint32_t w) {
  const f16x2 off = {(_Float16)-1032.0f, (_Float16)-1032.0f};
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, (w & 0x000F000Fu) | 0x64006400u) + off);
}
__device__ inline u32x4 x8_dequant_f16s(uint32_t w) {
  u32x4 r;
  r.x = x8_nib_pair_f16s(w);
  r.y = x8_nib_pair_f16s(w >> 4);
  r.z = x8_nib_pair_f16s(w >> 8);
  r.w = x8_nib_pair_f16s(w >> 12);
  return r;
}

constexpr int x8_rank_threads(int E) {
  int P = 1;
  while (2 * P * E <= kFThreads) P *= 2;
  return P;
}

// Dynamic LDS layout (bytes).
template <int H, int I, int E>
struct X8Lds {
  static constexpr int Kq = H / kQuad, KqI = I / kQuad;
  static constexpr int htPer = I / 8 / kX8PerXcd;         // gate/up half tiles per workgroup
  static constexpr int qPerW = Kq / kFW;                  // quads of H per wave and half tile
  static constexpr int GU = htPer * qPerW;                // gate/up (half tile, quad) pairs per wave
  static constexpr int tdPer = H / kRowTile / kX8PerXcd;  // down row tiles per workgroup
  static constexpr int DN = KqI / 2;                      // down (tile, quad) pairs per wave
  static constexpr uint32_t xop = 0;                      // [Kq][4 p][4 gi] x 16 B
  static constexpr uint32_t xs = xop + Kq * 256;          // [Kq][4] fp32 group sums
  static constexpr uint32_t gu = xs + Kq * 16;            // [8 waves][GU] chunks
  static constexpr uint32_t dn = gu + kFW * GU * kX8Chunk;  // [8 waves][DN] chunks
  static constexpr uint32_t hop = dn + kFW * DN * kX8Chunk; // [KqI][4 p][4 gi][hi, lo] x 16 B
  static constexpr uint32_t gred = hop + KqI * 512;         // [8 waves][htPer][16] fp32
  static constexpr uint32_t dred = gred + kFW * htPer * 64; // [8 waves][16] fp32
  static constexpr uint32_t lv = dred + kFW * 64;           // [E] fp64 logits
  static constexpr uint32_t key = lv + E * 8;               // [E] order keys
  static constexpr uint32_t rank = key + E * 8;             // [E] ranks
  static constexpr uint32_t bytes = rank + E * 4;
};

template <int H_, int I_, int E_>
__global__ __launch_bounds__(kFThreads) void moe_decode_x8_kernel(X8K a) {
  constexpr int H = H_, I = I_, E = E_, K = kX8Xcds;
  using L = X8Lds<H, I, E>;
  constexpr int Kq = L::Kq, KqI = L::KqI, htPer = L::htPer, qPerW = L::qPerW, GU = L::GU, tdPer = L::tdPer,
                DN = L::DN;
  constexpr int yRows = H / kX8Grid;      // rows of y each workgroup combines
  constexpr int P = x8_rank_threads(E);  // threads per logit in the ranking
  static_assert(H % (kQuad * kFW) == 0 && I % (8 * kX8PerXcd) == 0 && H % (kRowTile * kX8PerXcd) == 0 &&
                    I % kQuad == 0,
                "whole quads of H per wave, whole half tiles and row tiles per workgroup");
  static_assert(tdPer * 2 == kFW && KqI % 2 == 0, "down: two waves per row tile, half of I each");
  static_assert(tdPer * kRowTile == kWave, "one partial row per lane of wave 0");
  static_assert(E <= kX8Grid && E % kWave == 0 && E * P <= kFThreads, "logits");
  static_assert(htPer * 8 <= kWave && I / 2 <= kFThreads && yRows * K / 2 <= kWave && yRows <= kWave, "lanes");
  static_assert(L::bytes <= kFusedDynLdsMax, "LDS");

  __shared__ int s_sel_idx[K];
  __shared__ double s_sel_v[K];
  __shared__ float s_sel_w[K];
  __shared__ int s_pfail, s_hfail;
  extern __shared__ u32x4 s_dyn[];
  char* lds = reinterpret_cast<char*>(s_dyn);
  u32x4* s_xop = reinterpret_cast<u32x4*>(lds + L::xop);
  float* s_xs = reinterpret_cast<float*>(lds + L::xs);
  char* s_hop = lds + L::hop;
  float* s_gred = reinterpret_cast<float*>(lds + L::gred);
  float* s_dred = reinterpret_cast<float*>(lds + L::dred);
  double* s_lv = reinterpret_cast<double*>(lds + L::lv);
  uint64_t* s_key = reinterpret_cast<uint64_t*>(lds + L::key);
  int* s_rank = reinterpret_cast<int*>(lds + L::rank);

  const int lane = threadIdx.x % kWave;
  const int w = uni(threadIdx.x / kWave);
  const int n = lane % 16;
  const int p = lane / 16;
  const int b = (int)blockIdx.x;
  const int xcd = (int)(__builtin_amdgcn_s_getreg((3 << 11) | 20) & 0x7u);  // HW_REG_XCC_ID, bits 2:0
  const int rho = b / kX8Xcds;
  const f32x4 z = {0.f, 0.f, 0.f, 0.f};

  // ---- 0. generation; logits; x operand ---------------------------------------
  const uint32_t tag = launch_tag(a.ctl, &a.presence[b], b == kX8Grid - 1 ? a.skew_gen : 0u);
  if (threadIdx.x == 0) s_hfail = 0;
  // Logit e is computed once, by wave 0 of workgroup e (the router's
  // fixed-order contract), and published device-scope in slot e; every
  // workgroup polls all E slots and ranks the logits itself.
  const BufRsrc lg_r = buf_rsrc(a.xslots, (uint32_t)(E * kX8SlotStride));
  if (w == 0 && b < E) {
    double logit = fixed_dot_bf16(a.x, a.W + (int64_t)b * H, H);
    if (a.bias) logit = logit + (double)a.bias[b];
    if (lane == 0) {
      const uint64_t bits = __builtin_bit_cast(uint64_t, logit);
      u32x4 v;
      v.x = (uint32_t)bits;
      v.y = tag;
      v.z = (uint32_t)(bits >> 32);
      v.w = ~tag;
      __builtin_amdgcn_raw_buffer_store_b128(v, lg_r, b * kX8SlotStride, 0, kDeviceScope);
    }
  } else if (w == 4) {
    // the MFMA-ordered x operand and its group sums, as the generic kernel
    // builds them: one lane per (quad, group)
    for (int j = lane; j < Kq * 4; j += kWave) {
      const int q = j / 4, gi = j % 4;
      const uint16_t* xr = a.x + (int64_t)(4 * q + gi) * kGroup;
      float sp[4];
#pragma unroll
      for (int pp = 0; pp < 4; ++pp) {
        const uint2 lo = *reinterpret_cast<const uint2*>(xr + 4 * pp);
        const uint2 hi = *reinterpret_cast<const uint2*>(xr + 16 + 4 * pp);
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
  } else if (w == kFW - 1) {
    // ---- 1. the E logits into LDS
    const uint32_t want = tag + a.skew_route;
    constexpr int kNV = E / kWave;
    bool done[kNV];
#pragma unroll
    for (int v = 0; v < kNV; ++v) done[v] = false;
    bool failed = false;
    for (uint32_t it = 0;; ++it) {
      poll_clobber();
      u32x4 sv[kNV];
#pragma unroll
      for (int v = 0; v < kNV; ++v)
        if (!done[v])
          sv[v] = __builtin_amdgcn_raw_buffer_load_b128(lg_r, (lane + v * kWave) * kX8SlotStride, 0, kDevicePoll);
      bool all = true;
#pragma unroll
      for (int v = 0; v < kNV; ++v) {
        if (!done[v] && tag_ok(sv[v], want)) {
          const double lv = __builtin_bit_cast(double, ((uint64_t)sv[v].z << 32) | sv[v].x);
          s_lv[lane + v * kWave] = lv;
          s_key[lane + v * kWave] = logit_key(lv);
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
    for (int e = lane; e < E; e += kWave) s_rank[e] = 0;
    if (lane == 0) s_pfail = failed ? 1 : 0;
  }
  asm volatile("" ::"s"(tag));  // this wave's counter and presence loads have returned
  lds_barrier();                // every wave has read the generation; logits and x operand in LDS
  if (threadIdx.x == 0) __hip_atomic_store(&a.presence[b], tag64(tag), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const bool route_failed = uni(s_pfail) != 0;

  {
    if (!route_failed) {
      // rank of logit e in wave_topk_row's order (value descending, NaN
      // last, ties to the lower index): the number of larger keys, counted
      // without branches by P threads per logit (keys j0 .. j0 + span are
      // the same for the whole wave, so the LDS reads broadcast; all are
      // issued before the first comparison), plus the number of equal keys
      // at lower indices.  Sorted by key, position i has a count of at most
      // i, equal to i unless it ties with an earlier one; so when exactly K
      // logits have a count below K and those counts add up to K (K - 1) / 2,
      // the counts are the ranks.  Otherwise (equal keys among the top K)
      // wave 0 orders the equal counts by index with ballots (equal counts
      // mean equal keys).
      constexpr int span = E / P;
      static_assert(E % P == 0 && E == 2 * kWave && K == 8, "two logits per lane of the selecting wave");
      if ((int)threadIdx.x < E * P) {
        const int pp = uni((int)threadIdx.x / E);
        const int e = (int)threadIdx.x - pp * E;
        const uint64_t ke = s_key[e];
        const int j0 = pp * span;
        uint64_t kk[span];
#pragma unroll
        for (int q = 0; q < span; ++q) kk[q] = s_key[j0 + q];
        __builtin_amdgcn_sched_barrier(0);
        int cnt = 0;
#pragma unroll
        for (int q = 0; q < span; ++q) cnt += (int)(kk[q] > ke);
        if (P == 1) s_rank[e] = cnt;
        else atomicAdd(&s_rank[e], cnt);
      }
      lds_barrier();
      if (w == 0) {
        const int c0 = s_rank[lane], c1 = s_rank[lane + kWave];
        const uint64_t in0 = __ballot(c0 < K), in1 = __ballot(c1 < K);
        int csum = 0;
#pragma unroll
        for (int bt = 0; bt < 3; ++bt)
          csum += (__popcll(__ballot(c0 < K && ((c0 >> bt) & 1))) + __popcll(__ballot(c1 < K && ((c1 >> bt) & 1)))) << bt;
        if (__popcll(in0) + __popcll(in1) == K && csum == K * (K - 1) / 2) {
          if (c0 < K) {
            s_sel_idx[c0] = lane;
            s_sel_v[c0] = s_lv[lane];
          }
          if (c1 < K) {
            s_sel_idx[c1] = lane + kWave;
            s_sel_v[c1] = s_lv[lane + kWave];
          }
        } else {
        uint64_t m00 = __ballot(c0 < K), m01 = __ballot(c1 < K);  // half 0 / half 1 lanes with a count below K
        uint64_t m10 = m00, m11 = m01;
#pragma unroll
        for (int bt = 0; bt < 3; ++bt) {
          const uint64_t b0 = __ballot((c0 >> bt) & 1), b1 = __ballot((c1 >> bt) & 1);
          m00 &= ((c0 >> bt) & 1) ? b0 : ~b0;
          m01 &= ((c0 >> bt) & 1) ? b1 : ~b1;
          m10 &= ((c1 >> bt) & 1) ? b0 : ~b0;
          m11 &= ((c1 >> bt) & 1) ? b1 : ~b1;
        }
        const uint64_t lt = (1ull << lane) - 1ull;
        const int r0 = c0 + __popcll(m00 & lt);                   // e = lane
        const int r1 = c1 + __popcll(m10) + __popcll(m11 & lt);   // e = lane + 64
        (void)m01;
        if (c0 < K && r0 < K) {
          s_sel_idx[r0] = lane;
          s_sel_v[r0] = s_lv[lane];
        }
        if (c1 < K && r1 < K) {
          s_sel_idx[r1] = lane + kWave;
          s_sel_v[r1] = s_lv[lane + kWave];
        }
        }
      }
      lds_barrier();
    }
  }
  const int ex = route_failed ? 0 : uni(s_sel_idx[xcd]);  // this XCD's expert

  // ---- 2. this wave's weight copies ------------------------------------------
  // Gate/up pair c = 2 i + qq: half tile ht = htPer * rho + i (rows 8 ht ..
  // 8 ht + 7 of I: row tile ht / 2, half ht % 2) and quad 2 w + qq.  A
  // wave's gate/up staging holds the gate scales of its pairs (64 bytes
  // each), the up scales, then per half tile the gate units of both quads
  // (512 bytes each: unit 8p + r = row 8 (ht % 2) + r, part p) and the up
  // units.  Down pair c: row tile tdPer * rho + w / 2, quad DN * (w % 2) + c;
  // its staging holds the scales of the pairs (128 bytes each), then their
  // 1 KiB nibble units.  Every copy is one instruction: a wave issues
  // 2 + 2 htPer gate/up copies here, scales first, and its 1 + DN down
  // copies once its gate/up data has landed (they are needed only after the
  // h hand-off, and issued with the gate/up copies they delayed them:
  // 14.03 -> 13.82 us a layer).
  constexpr uint32_t kGuSc = GU * 64;  // bytes of one kind of gate/up scales
  static_assert(qPerW == 2 && GU * 4 <= kWave && DN * 8 <= kWave, "one copy instruction per kind");
  const uint32_t s_gu = lds_addr(lds + L::gu) + (uint32_t)w * GU * kX8Chunk;
  const uint32_t s_dn = lds_addr(lds + L::dn) + (uint32_t)w * DN * kX8Chunk;
  const char* gu_w = lds + L::gu + w * GU * kX8Chunk;
  const char* dn_w = lds + L::dn + w * DN * kX8Chunk;
  if (!route_failed) {
    constexpr uint32_t gnib = (uint32_t)I * Kq * 64u, gsc = (uint32_t)I * Kq * 8u;
    const i32x4 gn = buf_rsrc_words(a.gate_nib + (size_t)ex * gnib, gnib);
    const i32x4 un = buf_rsrc_words(a.up_nib + (size_t)ex * gnib, gnib);
    const i32x4 gs = buf_rsrc_words(reinterpret_cast<const char*>(a.gate_sc) + (size_t)ex * gsc, gsc);
    const i32x4 us = buf_rsrc_words(reinterpret_cast<const char*>(a.up_sc) + (size_t)ex * gsc, gsc);
    // scales: lane l < 4 GU takes 16 bytes (two rows) of pair l / 4
    if (lane < GU * 4) {
      const int c = lane / 4, ht = htPer * rho + c / 2;
      const uint32_t off = (uint32_t)(((ht / 2) * Kq + 2 * w + c % 2) * 128 + 64 * (ht % 2) + 16 * (lane % 4));
      dma_b128_stream(gs, s_gu, off, 0u);
      dma_b128_stream(us, s_gu + kGuSc, off, 0u);
    }
    // nibbles of half tile i: lane l takes unit l % 32 of quad 2 w + l / 32
    const uint32_t unit = (uint32_t)(16 * ((lane % 32) / 8) + lane % 8) * 16u + (uint32_t)(lane / 32) * kQuadNibBytes;
#pragma unroll
    for (int i = 0; i < htPer; ++i) {
      const int ht = htPer * rho + i;
      const uint32_t soff = (uint32_t)uni(((ht / 2) * Kq + 2 * w) * kQuadNibBytes + 128 * (ht % 2));
      dma_b128_stream(gn, s_gu + 2 * kGuSc + (uint32_t)i * 2048u, unit, soff);
      dma_b128_stream(un, s_gu + 2 * kGuSc + (uint32_t)i * 2048u + 1024u, unit, soff);
    }
  }

  // ---- routing outputs, while the copies land --------------------------------
  if (!route_failed && w == 1) {
    // softmax over the selected logits (or sigmoid renormalised), summed in
    // slot order as wave_topk_row sums them
    double ej = 0.0;
    if (lane < K) {
      const double v = s_sel_v[lane];
      ej = (a.score_mode == 0) ? exp(v - s_sel_v[0]) : 1.0 / (1.0 + exp(-v));
    }
    double sum = 0.0;
    for (int i = 0; i < K; ++i) sum += __shfl(ej, i, kWave);
    if (lane < K) {
      const float wt = (float)(ej / sum);
      s_sel_w[lane] = wt;
      if (b == 0) a.topk_w[lane] = wt;
    }
  }
  if (b == 0 && threadIdx.x < K) {
    a.topk_idx[threadIdx.x] = route_failed ? -1 : s_sel_idx[threadIdx.x];
    if (route_failed) a.topk_w[threadIdx.x] = __builtin_nanf("");
  }

  // ---- 3. gate/up ---------------------------------------------------------------
  if (!route_failed) {
    f32x4 ag[htPer], cg[htPer];
#pragma unroll
    for (int i = 0; i < htPer; ++i) ag[i] = cg[i] = z;
    // only lane row 0 (the token) reads the x operand; the other rows stay
    // zero (an MFMA row of A feeds only the same row of the result)
    u32x4 xa[4] = {{0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}};
    float sx = 0.0f;
#pragma unroll
    for (int c = 0; c < GU; ++c) {
      const int i = c / qPerW;
      const int q = qPerW * w + c % qPerW;
      // this half tile's copies (the younger ones may fly)
      if (c % qPerW == 0) {
        wait_vmcnt_le(2 * (htPer - 1 - i));
        poll_clobber();
      }
      const u32x4 gw = *reinterpret_cast<const u32x4*>(gu_w + 2 * kGuSc + i * 2048 + (n >= 8 ? 1024 : 0) +
                                                        (c % qPerW) * 512 + (8 * p + (n & 7)) * 16);
      const uint2 dsv = *reinterpret_cast<const uint2*>(gu_w + (n >= 8 ? kGuSc : 0) + c * 64 + (n & 7) * 8);
      if (n == 0) {
        const u32x4* xo = s_xop + (q * 4 + p) * 4;
        xa[0] = xo[0];
        xa[1] = xo[1];
        xa[2] = xo[2];
        xa[3] = xo[3];
        sx = s_xs[q * 4 + p];
      }
      float d[4];
      unpack_scales(dsv, d);
      const uint32_t gwv[4] = {gw.x, gw.y, gw.z, gw.w};
      f32x4 pg[4];
#pragma unroll
      for (int gi = 0; gi < 4; ++gi) pg[gi] = mfma_bf16_16x16x32(xa[gi], x8_dequant_bf16(gwv[gi]), z);
      cg[i] = mfma_f32_16x16x4(sx, d[p], cg[i]);
#pragma unroll
      for (int gi = 0; gi < 4; ++gi) ag[i] += d[gi] * pg[gi];
    }
    {
      // this wave's down copies (see the copy section)
      constexpr uint32_t dnib = (uint32_t)H * KqI * 64u, dsc = (uint32_t)H * KqI * 8u;
      const i32x4 dn = buf_rsrc_words(a.down_nib + (size_t)ex * dnib, dnib);
      const i32x4 ds = buf_rsrc_words(reinterpret_cast<const char*>(a.down_sc) + (size_t)ex * dsc, dsc);
    const uint32_t tq0 = (uint32_t)uni((tdPer * rho + w / 2) * KqI + DN * (w % 2));
    if (lane < DN * 8) dma_b128_stream(ds, s_dn, (uint32_t)lane * 16u, tq0 * 128u);
#pragma unroll
    for (int c = 0; c < DN; ++c)
      dma_b128_stream(dn, s_dn + (uint32_t)DN * 128u + (uint32_t)c * kQuadNibBytes, (uint32_t)lane * 16u,
                      (tq0 + (uint32_t)c) * kQuadNibBytes);
    }
    // lane (n, 0) holds result row 0 (the token) of column n: gate row n of
    // the half for n < 8, up row n - 8 for n >= 8
    if (p == 0) {
#pragma unroll
      for (int i = 0; i < htPer; ++i) s_gred[(w * htPer + i) * 16 + n] = kUnitScale * ag[i][0] - kUnitBias * cg[i][0];
    }
  }
  lds_barrier();
  const BufRsrc xh_r = buf_rsrc(a.xh + (size_t)xcd * (I / 2) * 4, (uint32_t)(I / 2 * 16));
  if (w == 0) {
    // SwiGLU of the workgroup's 8 htPer rows of I, the wave partials summed
    // in wave order; units of rows (i, i + 1) go to this XCD's L2
    uint32_t hb = 0u, lb = 0u;
    if (lane < htPer * 8) {
      const int i = lane / 8, r = lane % 8;
      float h = __builtin_nanf("");
      if (!route_failed) {
        float g = 0.0f, u = 0.0f;
#pragma unroll
        for (int s2 = 0; s2 < kFW; ++s2) {
          g += s_gred[(s2 * htPer + i) * 16 + r];
          u += s_gred[(s2 * htPer + i) * 16 + 8 + r];
        }
        h = g * (1.0f / (1.0f + expf(-g))) * u;
      }
      hb = float_to_half_bits(h);
      lb = float_to_half_bits(h - half_bits_to_float32(hb));
    }
    const uint32_t hb2 = __shfl_down(hb, 1, kWave), lb2 = __shfl_down(lb, 1, kWave);
    if (lane < htPer * 8 && (lane & 1) == 0) {
      const int row = 8 * (htPer * rho + lane / 8) + lane % 8;  // even row of I
      u32x4 v;
      v.x = hb | (hb2 << 16);
      v.y = tag;
      v.z = lb | (lb2 << 16);
      v.w = ~tag;
      __builtin_amdgcn_raw_buffer_store_b128(v, xh_r, (row / 2) * 16, 0, 0);
    }
  }

  // ---- 4. down weights into registers, then h into the down operand -----------
  u32x4 bb[DN][4];
  float dv[DN][4];
  if (!route_failed) {
    wait_vmcnt<0>();  // this wave's down copies
    poll_clobber();
#pragma unroll
    for (int c = 0; c < DN; ++c) {
      const u32x4 wv = *reinterpret_cast<const u32x4*>(dn_w + DN * 128 + c * kQuadNibBytes + lane * 16);
      unpack_scales(*reinterpret_cast<const uint2*>(dn_w + c * 128 + n * 8), dv[c]);
      bb[c][0] = x8_dequant_f16s(wv.x);
      bb[c][1] = x8_dequant_f16s(wv.y);
      bb[c][2] = x8_dequant_f16s(wv.z);
      bb[c][3] = x8_dequant_f16s(wv.w);
    }
  }
  if ((int)threadIdx.x < I / 2) {
    // unit u holds rows i0 = 2u and i0 + 1: in group i0 / 32 they sit at K
    // positions kmap(pp, s) and kmap(pp, s + 4) of part pp = (i0 % 16) / 4
    const int u = (int)threadIdx.x;
    const uint32_t want = tag + a.skew_h;
    u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(xh_r, u * 16, 0, kXcdPoll);
    bool ok = tag_ok(v, want);
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
        v = __builtin_amdgcn_raw_buffer_load_b128(xh_r, u * 16, 0, kXcdPoll);
        ok = tag_ok(v, want);
      }
    }
    // fp16 NaN, in two statements: hipcc compiled the chained form
    // v.x = v.z = c in a poll loop of this shape into code that also copied
    // v.x into v.z when ok
    if (!ok) {
      v.x = 0x7E007E00u;
      v.z = 0x7E007E00u;
    }
    const int i0 = 2 * u, g32 = i0 / kGroup, jj = i0 % kGroup;
    const int pp = (jj % 16) / 4, off = jj - 4 * pp;  // 0, 2, 16 or 18
    const int s = ((off & 2) ? 1 : 0) + (off >= 16 ? 2 : 0);
    uint16_t* e16 = reinterpret_cast<uint16_t*>(s_hop + (((g32 / 4) * 4 + pp) * 4 + g32 % 4) * 32);
    e16[s] = (uint16_t)(v.x & 0xffffu);
    e16[s + 4] = (uint16_t)(v.x >> 16);
    e16[8 + s] = (uint16_t)(v.z & 0xffffu);
    e16[8 + s + 4] = (uint16_t)(v.z >> 16);
  }
  lds_barrier();
  const bool h_failed = uni(s_hfail) != 0;

  // ---- 5. down, then the combine over the XCDs ---------------------------------
  if (!route_failed) {
    f32x4 acc = z;
    u32x4 hh[4] = {{0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}};
#pragma unroll
    for (int c = 0; c < DN; ++c) {
      const int q = DN * (w % 2) + c;
      if (n < 2) {
#pragma unroll
        for (int gi = 0; gi < 4; ++gi)
          hh[gi] = *reinterpret_cast<const u32x4*>(s_hop + ((q * 4 + p) * 4 + gi) * 32 + n * 16);
      }
#pragma unroll
      for (int gi = 0; gi < 4; ++gi) acc += dv[c][gi] * mfma_f16_16x16x32(hh[gi], bb[c][gi], z);
    }
    // lane (n, 0): result rows 0 (h hi) and 1 (h lo) of output row n
    if (p == 0) s_dred[w * 16 + n] = acc[0] + acc[1];
  }
  lds_barrier();
  const BufRsrc pt_r = buf_rsrc(a.xpart, (uint32_t)(kX8Xcds * H / 2 * 16));
  if (w == 0) {
    // rows 64 rho + lane of slot xcd's output, the two waves of each row tile
    // in order; units of rows (r, r + 1) go out device-scope
    float d = __builtin_nanf("");
    if (!route_failed && !h_failed) {
      const int i = lane / 16, nn = lane % 16;
      d = s_dred[(2 * i) * 16 + nn] + s_dred[(2 * i + 1) * 16 + nn];
    }
    const float d2 = __shfl_down(d, 1, kWave);
    if ((lane & 1) == 0) {
      const int row = tdPer * kRowTile * rho + lane;
      u32x4 v;
      v.x = __builtin_bit_cast(uint32_t, d);
      v.y = tag;
      v.z = __builtin_bit_cast(uint32_t, d2);
      v.w = ~tag;
      __builtin_amdgcn_raw_buffer_store_b128(v, pt_r, ((xcd * H + row) / 2) * 16, 0, kDeviceScope);
    }
  } else if (w == 1) {
    // rows row0 .. row0 + yRows of y: lane t < K * yRows / 2 polls unit t % 4
    // of slot t / 4 (of yRows / 2 units), then lane r < yRows sums its row
    // over the slots in slot order
    constexpr int UPS = yRows / 2;
    const int row0 = tdPer * kRowTile * rho + yRows * xcd;
    const bool mine = lane < K * UPS;
    const int j = lane / UPS, uu = lane % UPS;
    const uint32_t off = mine ? (uint32_t)(((j * H + row0) / 2 + uu) * 16) : 0u;
    u32x4 v = {0u, 0u, 0u, 0u};
    bool ok = !mine;
    if (mine) {
      v = __builtin_amdgcn_raw_buffer_load_b128(pt_r, (int)off, 0, kDevicePoll);
      ok = tag_ok(v, tag);
    }
    for (uint32_t it = 0;; ++it) {
      if (__all(ok)) break;
      if (it >= a.wait_polls) {
        if (lane == 0) set_status(a.ctl, a.host_status, kStatusExpertWait);
        break;
      }
      poll_clobber();
      if (!ok) {
        v = __builtin_amdgcn_raw_buffer_load_b128(pt_r, (int)off, 0, kDevicePoll);
        ok = tag_ok(v, tag);
      }
    }
    if (!ok) {  // NaN
      v.x = 0x7FC00000u;
      v.z = 0x7FC00000u;
    }
    float yv = 0.0f;
#pragma unroll
    for (int jj = 0; jj < K; ++jj) {
      const int src = jj * UPS + (lane % yRows) / 2;
      const uint32_t lo = (uint32_t)__shfl((int)v.x, src, kWave), hi = (uint32_t)__shfl((int)v.z, src, kWave);
      const float dj = __builtin_bit_cast(float, (lane & 1) ? hi : lo);
      yv += (route_failed ? 0.0f : s_sel_w[jj]) * dj;
    }
    if (lane < yRows) a.y[row0 + lane] = route_failed ? __builtin_nanf("") : yv;
  }

  // ---- 6. the next call's tag ---------------------------------------------------
  if (b == 0 && w == 2) {
    for (int i0 = 0; i0 < kX8Grid; i0 += kWave) {
      const int i = i0 + lane;
      bool done = false;
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

bool fused_shape_ok(int64_t T, int64_t H, int64_t I, int E, int k, int has_shared) {
  if (T < 1 || T > kFusedMaxT || T * E > kFusedMaxLogits || T * k > kFusedMaxSlots) return false;
  if (E < 1 || E > kMaxExperts || k < 1 || k > kMaxTopK || k > E) return false;
  if (H < kGroup || H % kGroup || I < kGroup || I % kGroup) return false;
  const int64_t Kq = ceil_div(H, kQuad), KqI = ceil_div(I, kQuad);
  // 32-bit buffer offsets over each stacked matrix and over h
  if ((uint64_t)E * (uint64_t)I * Kq * 64 >= kMaxRsrcBytes || (uint64_t)E * (uint64_t)H * KqI * 64 >= kMaxRsrcBytes)
    return false;
  if ((T * k + T) * (I / 2) * 16 >= ((int64_t)1 << 31)) return false;
  // the magic divisions: every dividend and divisor below 2^16
  if ((T + 1) * Kq * 4 >= 65536 || (T * k + T) * KqI * 64 + kFThreads * kHUnits >= 65536) return false;
  // the smallest layout: one item of each kind per workgroup; a wave's down
  // pairs fit one lane each
  const int S_max = (int)((T * k < E ? T * k : E) + (has_shared ? 1 : 0));
  if (ceil_div((int64_t)S_max * KqI, kFW) > kWave) return false;
  return fused_lds_layout((int)T, k, E, has_shared, (int)H, (int)I, 1, 1, S_max).bytes <= kFusedDynLdsMax;
}

bool x8_shape(int64_t T, int64_t H, int64_t I, int E, int k, int has_shared) {
  return T == 1 && H == 2048 && I == 768 && E == 128 && k == kX8Xcds && !has_shared;
}

namespace {

// XCDs of the current device (0 when the runtime cannot tell).
int device_xccs() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeNumberOfXccs, dev) != hipSuccess || n <= 0) n = -1;
    cached[dev] = n;
  }
  return cached[dev] > 0 ? cached[dev] : 0;
}

}  // namespace

FusedPlan fused_plan(int64_t T, int64_t H, int64_t I, int E, int k, int has_shared) {
  FusedPlan pl = {};
  pl.ok = false;
  const LibConfig cfg = lib_config();
  if (!cfg.decode_fused || !fused_shape_ok(T, H, I, E, k, has_shared)) return pl;
  if (cfg.decode_stream == 2 && T == 1) return pl;  // the streaming kernel takes every one-token shape
  if (cfg.decode_x8 && x8_shape(T, H, I, E, k, has_shared) && device_cus() == kX8Grid &&
      device_xccs() == kX8Xcds) {
    pl.G = kX8Grid;
    pl.spec = kFusedSpecX8;
    pl.lds = FusedLds{};
    pl.lds.bytes = X8Lds<2048, 768, 128>::bytes;
    pl.ok = true;
    return pl;
  }
  int G = device_cus();
  if (G > kFusedMaxGrid) G = kFusedMaxGrid;
  if ((int64_t)G * kFW < T * E || G < 2) return pl;  // one logit per wave at most
  const int S_max = (int)((T * k < E ? T * k : E) + (has_shared ? 1 : 0));
  const int n_gu = S_max * (int)(I / kRowTile);
  const int n_dn = (int)(H / kRowTile);
  if (n_gu + G >= 65536 || n_dn + G >= 65536) return pl;  // the magic divisions
  const int ng = (int)ceil_div(n_gu, G), nd = (int)ceil_div(n_dn, G);
  if (ng > kFusedMaxItems) return pl;  // the gate/up accumulators of one workgroup live in registers
  pl.lds = fused_lds_layout((int)T, k, E, has_shared, (int)H, (int)I, ng, nd, S_max);
  if (pl.lds.bytes > kFusedDynLdsMax) return pl;
  pl.G = G;
  pl.spec = (T == 1 && H == 2048 && I == 768 && E == 128 && k == 8 && !has_shared) ? kFusedSpecQwen3T1 : 0;
  pl.ok = true;
  return pl;
}

template <int T_, int H_, int I_, int E_, int K_, int SH_>
static hipError_t launch_fused_as(const FusedK& a, const FusedPlan& pl, hipStream_t stream) {
  static bool attr_set = false;
  auto kernel = moe_decode_fused_kernel<T_, H_, I_, E_, K_, SH_>;
  if (!attr_set) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)kFusedDynLdsMax);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  hipLaunchKernelGGL(kernel, dim3(pl.G), dim3(kFThreads), pl.lds.bytes, stream, a);
  return hipGetLastError();
}

static hipError_t launch_x8(const FusedPlan& pl, const RouteArgs& r, const ExpertArgs& x, const FusedWs& ws,
                            hipStream_t stream) {
  if (!ws.xslots || !ws.xh || !ws.xpart) return hipErrorInvalidValue;  // a workspace planned for another shape
  X8K a = {};
  a.x = static_cast<const uint16_t*>(r.x);
  a.W = r.router_w;
  a.bias = r.router_bias;
  a.score_mode = r.score_mode;
  a.gate_nib = x.gate_nib;
  a.gate_sc = x.gate_scale;
  a.up_nib = x.up_nib;
  a.up_sc = x.up_scale;
  a.down_nib = x.down_nib;
  a.down_sc = x.down_scale;
  a.y = x.y;
  a.topk_idx = r.topk_idx;
  a.topk_w = r.topk_w;
  a.ctl = ws.ctl;
  a.presence = ws.presence;
  a.xslots = ws.xslots;
  a.xh = ws.xh;
  a.xpart = ws.xpart;
  const LibConfig cfg = lib_config();
  a.wait_polls = cfg.fused_wait_polls;
  a.skew_route = (cfg.fused_fault & 1u) ? 1u : 0u;
  a.skew_h = (cfg.fused_fault & 2u) ? 1u : 0u;
  a.skew_gen = (cfg.fused_fault & 4u) ? 1u : 0u;
  a.host_status = host_status_word();
  static bool attr_set = false;
  auto kernel = moe_decode_x8_kernel<2048, 768, 128>;
  if (!attr_set) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)kFusedDynLdsMax);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  hipLaunchKernelGGL(kernel, dim3(kX8Grid), dim3(kFThreads), pl.lds.bytes, stream, a);
  return hipGetLastError();
}

static hipError_t launch_fused(const FusedK& a, const FusedPlan& pl, hipStream_t stream) {
  if (pl.spec == kFusedSpecQwen3T1) return launch_fused_as<1, 2048, 768, 128, 8, 0>(a, pl, stream);
  return launch_fused_as<0, 0, 0, 0, 0, -1>(a, pl, stream);
}

hipError_t launch_decode_fused(const FusedPlan& pl, const RouteArgs& r, const ExpertArgs& x, const FusedWs& ws,
                               hipStream_t stream) {
  if (pl.spec == kFusedSpecX8) return launch_x8(pl, r, x, ws, stream);
  FusedK a = {};
  a.x = static_cast<const uint16_t*>(r.x);
  a.W = r.router_w;
  a.bias = r.router_bias;
  a.T = (int)r.T;
  a.H = (int)r.H;
  a.I = (int)x.I;
  a.E = r.E;
  a.k = r.k;
  a.score_mode = r.score_mode;
  a.has_shared = x.has_shared;
  a.Kq = (int)ceil_div(r.H, kQuad);
  a.KqI = (int)ceil_div(x.I, kQuad);
  a.md_E = div_magic((uint32_t)a.E);
  a.md_nrtI = div_magic((uint32_t)(a.I / kRowTile));
  a.md_KqI = div_magic((uint32_t)a.KqI);
  a.md_Kq4 = div_magic((uint32_t)(4 * a.Kq));
  a.md_upos = div_magic((uint32_t)(64 * a.KqI));
  a.md_G = div_magic((uint32_t)pl.G);
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
  a.slots = ws.slots;
  a.hv = ws.hv;
  a.lds = pl.lds;
  const LibConfig cfg = lib_config();
  a.wait_polls = cfg.fused_wait_polls;
  a.skew_route = (cfg.fused_fault & 1u) ? 1u : 0u;
  a.skew_h = (cfg.fused_fault & 2u) ? 1u : 0u;
  a.skew_gen = (cfg.fused_fault & 4u) ? 1u : 0u;
  a.host_status = host_status_word();
  return launch_fused(a, pl, stream);
}

}  // namespace pmoe
