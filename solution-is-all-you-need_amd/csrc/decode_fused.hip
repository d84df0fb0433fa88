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
// (one per CU) runs the same program:
//   1. Its waves compute logits (the router's fixed-order fp64 contract, one
//      wave per (token, expert)) and publish each as a tagged 16-byte slot.
//   2. It waits until all T*E slots carry this call's tag and runs the top-k
//      and weights itself, from the same logits with the same instructions as
//      every other workgroup, so all agree bit for bit without a second
//      hand-off.  It then builds the expert segments (stable permute) in LDS.
//   3. It copies ALL its weights into LDS at once with direct-to-LDS loads
//      (the copies need no registers, so every byte of the layer is requested
//      right after routing): those of its gate/up items (segment x 16-row
//      tile of I, K split over the 8 waves; item i to workgroup i mod G) and
//      of its down items (16-row tile of H: every segment x quad of I; item d
//      to workgroup G - 1 - d mod G, so the workgroups with fewer gate/up
//      items take them).  Every workgroup thus shares both phases.
//   4. Gate/up items: MFMA, cross-wave sum in wave order, SwiGLU, h stored
//      device-scope as the fp16 hi/lo down operand; then one tagged flag per
//      item.
//   5. Down items: expand the down weights into MFMA operands in registers
//      while waiting for every gate/up flag, copy h of all segment positions
//      into LDS, MFMA per (segment, quad), then per output row
//      y[t] = sum_j w[t,j] * (sum_q part[q]) (+ shared expert), j in slot
//      order: the combine is fused, no expert-output round trip.
// Each wave reads back only the LDS it loaded itself, so the copies need a
// wait for the wave's own loads and no barrier.  Loops run over the wave's
// chunks without unrolling: the kernel stays a few thousand instructions,
// inside the instruction cache (a first version that kept every chunk in
// registers unrolled its epilogues per chunk to 15k instructions and spent
// most of its time in instruction fetch).
//
// Hand-off protocol (no memset, no host involvement, graph-replay safe).
// Word 0 of the workspace is a generation counter.  Every workgroup reads it
// once at start; this call's tag is gen + 1.  Logit slots hold
// {lo32, tag, hi32, ~tag} (one 16-byte store; both halves carry the tag, so a
// torn read cannot pass), flags and presence words {tag, ~tag}.  Workgroup 0
// bumps the counter to the tag once every workgroup has published its
// presence (so every workgroup has read the counter); the next call therefore
// uses a fresh tag and never mistakes this call's slots for its own.  Data
// hand-offs use device-scope (SC1) stores and loads: a device-scope store is
// written through to where every XCD reads, and a device-scope load is never
// served from a stale line of this XCD's L2, so no cache write-back or
// invalidation is needed; a writer waits for its data stores to complete
// before it stores a flag, and a reader issues its data loads only after the
// flag has arrived.
// Every wait is bounded (LibConfig::fused_wait_polls polls); a wait that gives
// up sets a bit of the status word (workspace word 1, read by
// phantom_moe_workspace_status) and its workgroup writes NaN to the outputs
// it owns, so a failure is never silent.  The grid never exceeds one
// workgroup per CU, so with the GPU otherwise idle no wait can deadlock.
#include <math.h>
#include <stdint.h>

#include "expert_common.h"
#include "moe_common.h"
#include "moe_launch.h"
#include "topk_common.h"  // logit_key

namespace pmoe {

namespace {

constexpr int kFW = 8;  // waves per workgroup
constexpr int kFThreads = kFW * kWave;
constexpr uint32_t kGuChunkLds = 2304;  // gate nib 1 KB, up nib 1 KB, gate scales 128 B, up scales 128 B
constexpr uint32_t kDnChunkLds = 1152;  // down nib 1 KB, scales 128 B
constexpr int kFusedMaxItems = 4;       // gate/up items per workgroup
constexpr int kPreDq = 4;               // down chunks per wave expanded into registers ahead of the hand-off

struct FusedK {
  const uint16_t* x;  // [T, H] bf16
  const float* W;     // [E, H]
  const float* bias;  // [E] or null
  int T, H, I, E, k, score_mode, has_shared;
  int Kq, KqI;  // quads of H and of I
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
  uint32_t* slots;     // [T * E][4]
  uint64_t* flags;     // [max gate/up items]
  uint16_t* hq;        // [positions][KqI * 256] fp16 hi/lo of h, down operand order
  float* hs;           // [positions][KqI * 8] half-group sums
  FusedLds lds;        // dynamic LDS layout
  uint32_t wait_polls;  // bound of every wait
  uint32_t skew_route;  // added to the tag the logit wait expects (non-zero only to test the failure path)
  uint32_t skew_flags;  // the same for the gate/up flag wait
};

__device__ inline uint64_t tag64(uint32_t t) { return (uint64_t)t | ((uint64_t)(~t) << 32); }

// A tagged 8-byte word {tag, ~tag} through a buffer resource, device scope.
__device__ inline void store_tag(BufRsrc r, uint32_t off, uint32_t t) {
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  const u32x2 v = {t, ~t};
  __builtin_amdgcn_raw_buffer_store_b64(v, r, (int)off, 0, kDeviceScope);
}

__device__ inline bool tag_is(BufRsrc r, uint32_t off, uint32_t t) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, kDeviceScope);
  return (uint32_t)v[0] == t && (uint32_t)v[1] == ~t;
}

// A value every lane of the wave holds alike (LDS reads of shared
// bookkeeping, wave indices): stated as uniform, so the compiler keeps it in
// an SGPR and branches and buffer offsets built from it stay scalar.
__device__ inline int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }

// s_waitcnt vmcnt(n) for a wave-uniform n known only at run time (n above
// 47 waits for everything).
__device__ inline void wait_vmcnt_le(int n) {
#define PMOE_W(N) \
  case N:         \
    wait_vmcnt<N>(); \
    break;
  switch (n) {
    PMOE_W(0) PMOE_W(1) PMOE_W(2) PMOE_W(3) PMOE_W(4) PMOE_W(5) PMOE_W(6) PMOE_W(7) PMOE_W(8) PMOE_W(9)
    PMOE_W(10) PMOE_W(11) PMOE_W(12) PMOE_W(13) PMOE_W(14) PMOE_W(15) PMOE_W(16) PMOE_W(17) PMOE_W(18)
    PMOE_W(19) PMOE_W(20) PMOE_W(21) PMOE_W(22) PMOE_W(23) PMOE_W(24) PMOE_W(25) PMOE_W(26) PMOE_W(27)
    PMOE_W(28) PMOE_W(29) PMOE_W(30) PMOE_W(31) PMOE_W(32) PMOE_W(33) PMOE_W(34) PMOE_W(35) PMOE_W(36)
    PMOE_W(37) PMOE_W(38) PMOE_W(39) PMOE_W(40) PMOE_W(41) PMOE_W(42) PMOE_W(43) PMOE_W(44) PMOE_W(45)
    PMOE_W(46) PMOE_W(47)
    default:
      wait_vmcnt<0>();
  }
#undef PMOE_W
}

__device__ inline void set_status(uint32_t* ctl, uint32_t bit) {
  __hip_atomic_fetch_or(&ctl[1], bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The router's fixed-order fp64 dot of x[t] (bf16) and W[e] (router.hip):
// lane l accumulates h = 256c + 4l + i in increasing h, then the xor tree
// s = 32..1 adds the 64 partials (commutative adds, so every lane ends with
// the same bits).
__device__ inline double fixed_dot_bf16(const uint16_t* xr, const float* wr, int H) {
  const int lane = threadIdx.x % kWave;
  constexpr int CB = 8;
  const int nch = (H + 255) / 256;
  double acc = 0.0;
  for (int c0 = 0; c0 < nch; c0 += CB) {
    float4 wv[CB];
    uint2 xv[CB];
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
      const int h0 = (c0 + cb) * 256 + 4 * lane;
      const bool ok = c0 + cb < nch && h0 < H;
      const int hc = ok ? h0 : 0;
      wv[cb] = *reinterpret_cast<const float4*>(wr + hc);
      xv[cb] = *reinterpret_cast<const uint2*>(xr + hc);
      if (!ok) {
        wv[cb] = make_float4(0.f, 0.f, 0.f, 0.f);
        xv[cb] = make_uint2(0u, 0u);
      }
    }
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
      acc += (double)bf16_bits_to_float(xv[cb].x & 0xffffu) * (double)wv[cb].x;
      acc += (double)bf16_bits_to_float(xv[cb].x >> 16) * (double)wv[cb].y;
      acc += (double)bf16_bits_to_float(xv[cb].y & 0xffffu) * (double)wv[cb].z;
      acc += (double)bf16_bits_to_float(xv[cb].y >> 16) * (double)wv[cb].w;
    }
  }
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) acc = acc + shfl_xor_f64(acc, s);
  return acc;
}

// The offset 32-bit buffer offsets cannot reach; no stacked matrix is
// allowed to come near it.
constexpr uint32_t kMaxRsrcBytes = 0xFFFFE000u;

// Position-row stride of the h operand in LDS, padded by 16 bytes so the 16
// rows of an MFMA operand fall in different banks.
__host__ __device__ inline uint32_t h_row_bytes(int KqI) { return (uint32_t)KqI * 512u + 16u; }

__host__ __device__ inline uint32_t align_lds(uint32_t v) { return (v + 255u) & ~255u; }

// Routing scratch: logits and their order keys [T*E], ranks [T*E], the
// selected logits and their exponentials [T*k], expert token masks [E].
struct RouteScratch {
  uint32_t lv, key, rank, selv, ej, emask, bytes;
};
__host__ __device__ inline RouteScratch route_scratch(int T, int k, int E) {
  RouteScratch r;
  r.lv = 0;
  r.key = r.lv + align_lds((uint32_t)(T * E) * 8u);
  r.rank = r.key + align_lds((uint32_t)(T * E) * 8u);
  r.selv = r.rank + align_lds((uint32_t)(T * E) * 4u);
  r.ej = r.selv + align_lds((uint32_t)(T * k) * 8u);
  r.emask = r.ej + align_lds((uint32_t)(T * k) * 8u);
  r.bytes = r.emask + align_lds((uint32_t)E * 8u);
  return r;
}
__host__ __device__ inline uint32_t route_scratch_bytes(int T, int k, int E) { return route_scratch(T, k, E).bytes; }

}  // namespace

// Dynamic LDS layout for ng gate/up and nd down items per workgroup, S_max
// segments:
//   [x operand][gate/up staging][down staging]
// The routing scratch (logits, keys, ranks, selection) is dead before the
// first weight copy is issued, so it sits over the staging regions; the h
// operand and the down partials are written after the workgroup's gate/up
// work is done, so they sit over the x operand and the gate/up staging when
// those are large enough (else after the down staging).
FusedLds fused_lds_layout(int T, int k, int E, int has_shared, int H, int I, int ng, int nd, int S_max) {
  FusedLds l = {};
  const uint32_t Kq = (uint32_t)((H + kQuad - 1) / kQuad), KqI = (uint32_t)((I + kQuad - 1) / kQuad);
  const uint32_t npos = (uint32_t)(T * k + (has_shared ? T : 0));
  const uint32_t route = route_scratch_bytes(T, k, E);
  const uint32_t x_op = align_lds((uint32_t)(T + 1) * Kq * 256u) + align_lds((uint32_t)(T + 1) * Kq * 16u);
  // staging slots are indexed (item, wave slot, wave): a wave takes quads
  // w, w + 8, ... of a gate/up item (nq slots) and (segment, quad) pairs
  // [w * per, w * per + per) of a down item
  const uint32_t nq = (Kq + kFW - 1) / kFW;
  const uint32_t per = ((uint32_t)S_max * KqI + kFW - 1) / kFW;
  const uint32_t wgu = (uint32_t)ng * nq * kFW * kGuChunkLds;
  const uint32_t wdn = (uint32_t)nd * per * kFW * kDnChunkLds;
  const uint32_t h_op = align_lds((npos + 1) * h_row_bytes((int)KqI)) + align_lds((npos + 1) * KqI * 32u);
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

__global__ __launch_bounds__(kFThreads) void moe_decode_fused_kernel(FusedK a) {
  __shared__ int s_sel_idx[kFusedMaxSlots];
  __shared__ float s_sel_w[kFusedMaxSlots];
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
  __shared__ uint32_t s_epoch;
  __shared__ int s_nseg;
  __shared__ int s_fail;
  extern __shared__ u32x4 s_dyn[];

  const int lane = threadIdx.x % kWave;
  const int w = uni(threadIdx.x / kWave);
  const int n = lane % 16;
  const int p = lane / 16;
  const int G = (int)gridDim.x;
  const int b = (int)blockIdx.x;
  const int T = a.T, H = a.H, I = a.I, E = a.E, k = a.k;
  const int Kq = a.Kq, KqI = a.KqI;
  const int Kg = H / kGroup, KgI = I / kGroup;
  char* lds = reinterpret_cast<char*>(s_dyn);
  char* rs = lds + a.lds.route;  // routing scratch
  const RouteScratch rl = route_scratch(T, k, E);
  double* s_lv = reinterpret_cast<double*>(rs + rl.lv);
  uint64_t* s_key = reinterpret_cast<uint64_t*>(rs + rl.key);
  int* s_rank = reinterpret_cast<int*>(rs + rl.rank);
  double* s_selv = reinterpret_cast<double*>(rs + rl.selv);
  double* s_ej = reinterpret_cast<double*>(rs + rl.ej);
  uint64_t* s_emask = reinterpret_cast<uint64_t*>(rs + rl.emask);
  u32x4* s_xop = reinterpret_cast<u32x4*>(lds + a.lds.x);  // [(T+1) Kq][4 p][4 gi]
  float* s_xs = reinterpret_cast<float*>(lds + a.lds.x + align_lds((uint32_t)(T + 1) * Kq * 256u));

  // ---- 0. generation (thread 0), router task, x operand ---------------
  uint32_t gen = 0;
  if (threadIdx.x == 0) {
    gen = __hip_atomic_load(&a.ctl[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_fail = 0;
  }
  // at most one (token, expert) logit per wave: the grid has >= T*E waves
  const int task = w * G + b;
  double logit = 0.0;
  if (task < T * E) {
    const int t = task / E, e = task % E;
    logit = fixed_dot_bf16(a.x + (int64_t)t * H, a.W + (int64_t)e * H, H);
    if (a.bias) logit = logit + (double)a.bias[e];
  }
  // the MFMA-ordered x operand of every token (and an all-zero row T) and its
  // group sums, built while the logits are in flight elsewhere: one thread per
  // (token, quad, group), the 4 parts p in order; the group sum adds the parts
  // as (p0 + p1) + (p2 + p3), each part ((x0 + x1) + (x2 + x3)) + ((x16 + x17)
  // + (x18 + x19)) over its 8 elements
  for (int j = threadIdx.x; j < (T + 1) * Kq * 4; j += kFThreads) {
    const int tok = j / (Kq * 4);
    const int q = (j / 4) % Kq;
    const int gi = j % 4;
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
  if (threadIdx.x == 0) {
    const uint32_t tg = gen + 1;
    s_epoch = tg;
    __hip_atomic_store(&a.presence[b], tag64(tg), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  lds_barrier();
  const uint32_t tag = (uint32_t)uni((int)s_epoch);

  // ---- 1. publish the logit ---------------------------------------------
  const BufRsrc slot_r = buf_rsrc(a.slots, (uint32_t)(T * E * 16));
  if (task < T * E && lane == 0) {
    const uint64_t bits = __builtin_bit_cast(uint64_t, logit);
    u32x4 v;
    v.x = (uint32_t)bits;
    v.y = tag;
    v.z = (uint32_t)(bits >> 32);
    v.w = ~tag;
    __builtin_amdgcn_raw_buffer_store_b128(v, slot_r, (int)(task * 16), 0, kDeviceScope);
  }

  // ---- 2. wait for every logit; top-k; segments ----------------------------
  // One poll per lane in flight: a load left in flight at the exit would
  // make the first later instruction that reuses its registers wait for it
  // (a memory round trip).
  {
    const uint32_t want = tag + a.skew_route;
    for (int i0 = w * kWave; i0 < T * E; i0 += kFThreads) {
      const int i = i0 + lane;
      bool done = i >= T * E;
      for (uint32_t it = 0;; ++it) {
        if (!done) {
          const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(slot_r, (int)((uint32_t)i * 16u), 0, kDeviceScope);
          if (v.y == want && v.w == ~want) {
            const double lv = __builtin_bit_cast(double, ((uint64_t)v.z << 32) | v.x);
            s_lv[i] = lv;
            s_key[i] = logit_key(lv);
            done = true;
          }
        }
        if (__all(done)) break;
        if (it >= a.wait_polls) {
          if (lane == 0) {
            s_fail = 1;
            set_status(a.ctl, kStatusRouteWait);
          }
          break;
        }
      }
    }
  }
  for (int i = threadIdx.x; i < T * E; i += kFThreads) s_rank[i] = 0;
  lds_barrier();
  const bool route_failed = uni(s_fail) != 0;
  if (!route_failed) {
    // Top-k of every token by rank counting over the whole workgroup: the
    // rank of logit i is the number of logits of its token before it in the
    // order (value descending, NaN last, ties to the lower index; the order
    // keys of topk_common.h), split over P threads per logit, the keys read
    // eight at a time.  Rank r < k lands in slot r: the selection and order
    // of wave_topk_row, and its weights below, bit for bit.
    const int n_el = T * E;
    int P = 1;
    while (2 * P * n_el <= kFThreads && 2 * P <= E) P *= 2;
    const int span = (E + P - 1) / P;
    for (int r = threadIdx.x; r < n_el * P; r += kFThreads) {
      const int el = r % n_el, pp = r / n_el;
      const int t = el / E, i = el % E;
      const uint64_t ki = s_key[el];
      const uint64_t* row = s_key + t * E;
      const int j0 = pp * span;
      const int j1 = j0 + span < E ? j0 + span : E;
      int cnt = 0;
      int j = j0;
      for (; j + 8 <= j1; j += 8) {
        uint64_t kk[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) kk[q] = row[j + q];
#pragma unroll
        for (int q = 0; q < 8; ++q) cnt += (kk[q] > ki || (kk[q] == ki && j + q < i)) ? 1 : 0;
      }
      for (; j < j1; ++j) {
        const uint64_t kj = row[j];
        cnt += (kj > ki || (kj == ki && j < i)) ? 1 : 0;
      }
      if (P == 1) s_rank[el] = cnt;
      else atomicAdd(&s_rank[el], cnt);
    }
    lds_barrier();
    // one wave per token: its k winners to their slots, then the weights,
    // softmax exp(l_j - l_0) or sigmoid(l_j) normalised by their sum over the
    // k slots in slot order, in fp64, stored as fp32
    for (int t = w; t < T; t += kFW) {
      for (int e0 = 0; e0 < E; e0 += kWave) {
        const int e = e0 + lane;
        if (e < E) {
          const int rk = s_rank[t * E + e];
          if (rk < k) {
            s_sel_idx[t * k + rk] = e;
            s_selv[t * k + rk] = s_lv[t * E + e];
          }
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      double ej = 0.0;
      if (lane < k) {
        const double v = s_selv[t * k + lane];
        ej = (a.score_mode == 0) ? exp(v - s_selv[t * k]) : 1.0 / (1.0 + exp(-v));
        s_ej[t * k + lane] = ej;
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      if (lane < k) {
        double sum = 0.0;
        for (int i = 0; i < k; ++i) sum += s_ej[t * k + i];
        s_sel_w[t * k + lane] = (float)(ej / sum);
      }
    }
  }
  lds_barrier();
  if (route_failed) {
    // no routing: this workgroup's outputs cannot be computed
    if (b == 0)
      for (int i = threadIdx.x; i < T * k; i += kFThreads) {
        a.topk_idx[i] = -1;
        a.topk_w[i] = __builtin_nanf("");
      }
  } else {
    if (b == 0)
      for (int i = threadIdx.x; i < T * k; i += kFThreads) {
        a.topk_idx[i] = s_sel_idx[i];
        a.topk_w[i] = s_sel_w[i];
      }
    if (T * k <= kWave) {
      // Up to 64 slots: one wave builds the segments from ballots.  Slot s
      // (lane s) of expert e goes to position #{slots of experts < e} +
      // #{earlier slots of e} (experts ascending, tokens ascending within an
      // expert: the stable permute); its segment is #{distinct experts < e}.
      if (w == 0) {
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
        if (a.has_shared && lane < T) s_seg_tok[T * k + lane] = lane;
        if (lane == 0) {
          if (a.has_shared) {
            s_seg_e[nu] = E;
            s_seg_cnt[nu] = T;
            s_seg_beg[nu] = T * k;
          }
          s_nseg = nu + (a.has_shared ? 1 : 0);
        }
      }
    } else {
      for (int e = threadIdx.x; e < E; e += kFThreads) s_emask[e] = 0;
      lds_barrier();
      for (int s = threadIdx.x; s < T * k; s += kFThreads)
        __hip_atomic_fetch_or(&s_emask[s_sel_idx[s]], 1ull << (s / k), __ATOMIC_RELAXED,
                              __HIP_MEMORY_SCOPE_WORKGROUP);
      lds_barrier();
      if (w == 0) {
        // active experts in increasing id, their segment sizes and offsets
        const uint64_t lt = (1ull << lane) - 1ull;
        int nu = 0;
        for (int e0 = 0; e0 < E; e0 += kWave) {
          const int e = e0 + lane;
          const uint64_t m = e < E ? s_emask[e] : 0ull;
          const uint64_t bal = __ballot(m != 0ull);
          if (m != 0ull) {
            const int u = nu + __popcll(bal & lt);
            s_seg_e[u] = e;
            s_seg_cnt[u] = __popcll(m);
            s_e2u[e] = (short)u;
          }
          nu += __popcll(bal);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        int run = 0;
        for (int u0 = 0; u0 < nu; u0 += kWave) {
          const int u = u0 + lane;
          const int c = u < nu ? s_seg_cnt[u] : 0;
          int inc = c;
#pragma unroll
          for (int off = 1; off < kWave; off <<= 1) {
            const int o = __shfl_up(inc, off, kWave);
            if (lane >= off) inc += o;
          }
          if (u < nu) s_seg_beg[u] = run + inc - c;
          run += __shfl(inc, kWave - 1, kWave);
        }
        if (lane == 0) {
          if (a.has_shared) {
            s_seg_e[nu] = E;
            s_seg_cnt[nu] = T;
            s_seg_beg[nu] = T * k;
          }
          s_nseg = nu + (a.has_shared ? 1 : 0);
        }
      }
      lds_barrier();
      // every slot's segment position (tokens in increasing order within a
      // segment: the stable permute) and every position's token
      for (int s = threadIdx.x; s < T * k; s += kFThreads) {
        const int t = s / k;
        const int e = s_sel_idx[s];
        const int pos = s_seg_beg[s_e2u[e]] + __popcll(s_emask[e] & ((1ull << t) - 1ull));
        s_slot_pos[s] = pos;
        s_seg_tok[pos] = t;
      }
      if (a.has_shared)
        for (int t = threadIdx.x; t < T; t += kFThreads) s_seg_tok[T * k + t] = t;
    }
  }
  lds_barrier();  // the routing scratch is dead from here on

  // ---- 3. work lists; every weight chunk of the workgroup -> LDS ------------
  const int S = route_failed ? 0 : uni(s_nseg);
  const int nrtI = I / kRowTile;
  const int n_gu = S * nrtI;
  const int n_dn = H / kRowTile;
  // gate/up items b, b + G, ...; down items G - 1 - b, G - 1 - b + G, ...
  const int ng = b < n_gu ? (n_gu - b + G - 1) / G : 0;
  const int dn_first = G - 1 - b;
  const int nd = (S > 0 && dn_first < n_dn) ? (n_dn - dn_first + G - 1) / G : 0;
  // gate/up: wave w takes quads w, w + 8, ... (nq slots) of each item
  const int nq = (Kq + kFW - 1) / kFW;
  // down: wave w takes (segment, quad) pairs [w * per, w * per + per) of each item
  const int n_c = S * KqI;
  const int per = (n_c + kFW - 1) / kFW;
  // this wave's pairs per down item, and its down copies (nibbles + scales)
  const int cnt_w = (n_c - w * per) < per ? ((n_c - w * per) > 0 ? n_c - w * per : 0) : per;
  const int dn_copies = nd * cnt_w * 2;

  // the combine's tables, while the routing results are at hand: slot s at
  // position pos of segment u reads part pt of output row nn at
  // (beg * KqI + pt * cnt + pos - beg) * 16 + nn, u's parts being the waves
  // its (segment, quad) pairs fall to
  if (S > 0 && nd > 0) {
    for (int s = threadIdx.x; s < T * k + (a.has_shared ? T : 0); s += kFThreads) {
      const bool sh = s >= T * k;
      const int u = sh ? S - 1 : s_e2u[s_sel_idx[s]];
      const int pos = sh ? T * k + (s - T * k) : s_slot_pos[s];
      const int beg = s_seg_beg[u], cnt = s_seg_cnt[u];
      s_cb_base[s] = (beg * KqI + pos - beg) * 16;
      s_cb_step[s] = cnt * 16;
      s_cb_np[s] = ((u + 1) * KqI - 1) / per - (u * KqI) / per + 1;
    }
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
  if (ng > 0) {
    for (int ii = 0; ii < ng; ++ii) {
      const int item = b + ii * G;
      const int u = item / nrtI, rt = item % nrtI;
      const int e = uni(s_seg_e[u]);
      const bool routed = e < E;
      const BufRsrc gn = routed ? buf_rsrc(a.gate_nib, stack(gnib_bytes)) : buf_rsrc(a.sh_gate_nib, gnib_bytes);
      const BufRsrc un = routed ? buf_rsrc(a.up_nib, stack(gnib_bytes)) : buf_rsrc(a.sh_up_nib, gnib_bytes);
      const BufRsrc gs = routed ? buf_rsrc(a.gate_sc, stack(gsc_bytes)) : buf_rsrc(a.sh_gate_sc, gsc_bytes);
      const BufRsrc us = routed ? buf_rsrc(a.up_sc, stack(gsc_bytes)) : buf_rsrc(a.sh_up_sc, gsc_bytes);
      const uint32_t eo_n = routed ? (uint32_t)e * gnib_bytes : 0u;
      const uint32_t eo_s = routed ? (uint32_t)e * gsc_bytes : 0u;
      for (int qq = 0; qq < nq; ++qq) {
        const int q = w + kFW * qq;
        if (q >= Kq) break;
        const uint32_t tq = (uint32_t)(rt * Kq + q);
        char* slot = wgu + ((ii * nq + qq) * kFW + w) * kGuChunkLds;
        dma_b128(gn, slot, (uint32_t)lane * 16u, eo_n + tq * kQuadNibBytes);
        dma_b128(un, slot + 1024, (uint32_t)lane * 16u, eo_n + tq * kQuadNibBytes);
        // scales: 32 lanes x 4 bytes each for gate, the other 32 for up
        if (lane < 32) dma_b32(gs, slot + 2048, (uint32_t)lane * 4u, eo_s + tq * (kQuadScales * 2));
        else dma_b32(us, slot + 2048, (uint32_t)(lane - 32) * 4u, eo_s + tq * (kQuadScales * 2));
      }
    }
  }
  if (nd > 0) {
    for (int dd = 0; dd < nd; ++dd) {
      const int rH = dn_first + dd * G;
      for (int cc = 0; cc < per; ++cc) {
        const int pair = w * per + cc;
        if (pair >= n_c) break;
        const int u = pair / KqI, q = pair % KqI;
        const int e = uni(s_seg_e[u]);
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
  }

  // ---- 4. gate/up items ----------------------------------------------------
  // Every item's chunks first, its accumulators in registers (at most
  // kFusedMaxItems items), then one reduction for all items: each wave writes
  // its partial sums over its own first staging slot of the item (read by
  // nobody else, and dead once the wave's MFMAs are done), one barrier, and
  // the SwiGLU epilogue of every item spread over the workgroup.
  const BufRsrc hq_r = buf_rsrc(a.hq, (uint32_t)((T * k + T) * KqI * 512));
  const BufRsrc hs_r = buf_rsrc(a.hs, (uint32_t)((T * k + T) * KqI * 32));
  const BufRsrc flag_r = buf_rsrc(a.flags, (uint32_t)(n_gu > 0 ? n_gu * 8 : 8));
  if (ng > 0) {
    const uint32_t mask = vgpr_const(0x00780078u);
    const f32x4 z = {0.f, 0.f, 0.f, 0.f};
    int tok[kFusedMaxItems];
#pragma unroll
    for (int ii = 0; ii < kFusedMaxItems; ++ii) {
      tok[ii] = T;
      if (ii < ng) {
        const int u = (b + ii * G) / nrtI;
        const int beg = uni(s_seg_beg[u]), cnt = uni(s_seg_cnt[u]);
        if (n < cnt) tok[ii] = s_seg_tok[beg + n];
      }
    }
    // this wave's gate/up copies have landed (each wave reads only its own;
    // its down copies, issued after them, may still be in flight)
    wait_vmcnt_le(dn_copies);
    f32x4 ag[kFusedMaxItems], au[kFusedMaxItems], cg[kFusedMaxItems], cu[kFusedMaxItems];
#pragma unroll
    for (int ii = 0; ii < kFusedMaxItems; ++ii) {
      ag[ii] = au[ii] = cg[ii] = cu[ii] = z;
      if (ii < ng) {
        for (int qq = 0; qq < nq; ++qq) {
          const int q = w + kFW * qq;
          if (q >= Kq) break;
          const char* slot = wgu + ((ii * nq + qq) * kFW + w) * kGuChunkLds;
          const u32x4 gw = *reinterpret_cast<const u32x4*>(slot + lane * 16);
          const u32x4 uw = *reinterpret_cast<const u32x4*>(slot + 1024 + lane * 16);
          const uint2 gsv = *reinterpret_cast<const uint2*>(slot + 2048 + n * 8);
          const uint2 usv = *reinterpret_cast<const uint2*>(slot + 2176 + n * 8);
          const u32x4* xo = s_xop + ((tok[ii] * Kq + q) * 4 + p) * 4;
          const u32x4 xa[4] = {xo[0], xo[1], xo[2], xo[3]};
          const float sx = s_xs[(tok[ii] * Kq + q) * 4 + p];
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
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          red[(4 * p + j) * 16 + n] = rg[j];
          red[256 + (4 * p + j) * 16 + n] = ru[j];
        }
      }
    }
    lds_barrier();
    for (int o = threadIdx.x; o < ng * 256; o += kFThreads) {
      const int ii = o / 256;
      const int mm = (o % 256) / 16;
      const int nn = o % 16;
      const int item = b + ii * G;
      const int u = item / nrtI, rt = item % nrtI;
      const int beg = s_seg_beg[u], cnt = s_seg_cnt[u];
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
      const float hf = half_bits_to_float32(hb);
      const uint32_t lb = float_to_half_bits(h - hf);
      const float lf = half_bits_to_float32(lb);
      const bool ok = mm < cnt;
      const int pos = beg + mm;
      const int i = rt * 16 + nn;  // row of I
      const int g32 = i / kGroup;
      const int cc = i % kGroup;
      const int half = cc / 16;
      const int pp = (cc % 16) / 4;
      const int rr = cc % 4;
      // kmap(p, j) = 4p + {0, 2, 16, 18, 1, 3, 17, 19}[j], inverted per half
      const int jj = half == 0 ? ((rr & 1) ? 4 : 0) + (rr >> 1) : ((rr & 1) ? 6 : 2) + (rr >> 1);
      const uint32_t off = (uint32_t)((((pos * KqI + g32 / 4) * 16 + pp * 4 + (g32 % 4)) * 16 + jj) * 2);
      if (ok) {
        __builtin_amdgcn_raw_buffer_store_b16((unsigned short)hb, hq_r, (int)off, 0, kDeviceScope);
        __builtin_amdgcn_raw_buffer_store_b16((unsigned short)lb, hq_r, (int)(off + 16u), 0, kDeviceScope);
      }
      // the 16 rows of the tile are one half of one group: sum hi + lo
      // over them (16 consecutive lanes, fixed butterfly order)
      float sum = hf + lf;
      sum += __shfl_xor(sum, 8, kWave);
      sum += __shfl_xor(sum, 4, kWave);
      sum += __shfl_xor(sum, 2, kWave);
      sum += __shfl_xor(sum, 1, kWave);
      if (nn == 0 && ok)
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, sum), hs_r,
                                              (int)(((pos * KqI * 4 + g32) * 2 + half) * 4), 0, kDeviceScope);
    }
    // every h store of the workgroup has completed before any flag is set
    __builtin_amdgcn_s_waitcnt(0);
    lds_barrier();
    if (threadIdx.x < ng) store_tag(flag_r, (uint32_t)(b + (int)threadIdx.x * G) * 8u, tag);
  }

  // ---- 5. down items with the combine --------------------------------------
  if (nd > 0) {
    // The down weights of a single item are expanded into MFMA operands now
    // (fp16 1 + n/16 and fp32 scales), while the gate/up results are still
    // on their way, so that only MFMAs remain after the hand-off.
    const uint32_t dmask = vgpr_const(0x03C003C0u);
    const bool pre = nd == 1;  // the first kPreDq chunks of a single item (more would spill)
    u32x4 pbb[kPreDq][4];
    float pdv[kPreDq][4];
    wait_vmcnt<0>();  // this wave's down copies
    if (pre) {
#pragma unroll
      for (int c = 0; c < kPreDq; ++c) {
        if (c < cnt_w) {
          const char* slot = wdn + (c * kFW + w) * kDnChunkLds;
          const u32x4 wv = *reinterpret_cast<const u32x4*>(slot + lane * 16);
          unpack_scales(*reinterpret_cast<const uint2*>(slot + 1024 + n * 8), pdv[c]);
          pbb[c][0] = dequant_unit_f16(wv.x, dmask);
          pbb[c][1] = dequant_unit_f16(wv.y, dmask);
          pbb[c][2] = dequant_unit_f16(wv.z, dmask);
          pbb[c][3] = dequant_unit_f16(wv.w, dmask);
        }
      }
    }
    // wait for every gate/up item of the layer (one poll per lane in flight)
    const uint32_t want = tag + a.skew_flags;
    for (int i0 = w * kWave; i0 < n_gu; i0 += kFThreads) {
      const int i = i0 + lane;
      bool done = i >= n_gu;
      for (uint32_t it = 0;; ++it) {
        if (!done) done = tag_is(flag_r, (uint32_t)i * 8u, want);
        if (__all(done)) break;
        if (it >= a.wait_polls) {
          if (lane == 0) {
            s_fail = 1;
            set_status(a.ctl, kStatusExpertWait);
          }
          break;
        }
      }
    }
    lds_barrier();
    const bool h_failed = uni(s_fail) != 0;
    // h of every segment position -> LDS (device-scope loads, issued after the
    // flags arrived), plus an all-zero row; groups past I are zero
    const int npos = T * k + (a.has_shared ? T : 0);
    const uint32_t hrow = h_row_bytes(KqI);
    char* s_hb = lds + a.lds.h;
    float* s_hs = reinterpret_cast<float*>(s_hb + align_lds((uint32_t)(npos + 1) * hrow));
    float* s_dred = reinterpret_cast<float*>(lds + a.lds.dred);
    {
      const int nu16 = (npos + 1) * KqI * 32;  // 16-byte units
      constexpr int U = 4;
      for (int i0 = threadIdx.x; i0 < nu16; i0 += kFThreads * U) {
        u32x4 v[U];
#pragma unroll
        for (int r = 0; r < U; ++r) {
          const int i = i0 + r * kFThreads;
          const int pos = i / (KqI * 32);
          const int rem = i % (KqI * 32);
          const int g = 4 * (rem / 32) + ((rem % 32) / 2) % 4;  // units of a quad: [p 4][gi 4][hi, lo]
          const bool ok = i < nu16 && pos < npos && g < KgI;
          v[r] = __builtin_amdgcn_raw_buffer_load_b128(hq_r, ok ? (uint32_t)(pos * KqI * 512 + rem * 16) : 0xFFFFF000u,
                                                        0, kDeviceScope);
        }
#pragma unroll
        for (int r = 0; r < U; ++r) {
          const int i = i0 + r * kFThreads;
          if (i < nu16) {
            const int pos = i / (KqI * 32);
            const int rem = i % (KqI * 32);
            *reinterpret_cast<u32x4*>(s_hb + (size_t)pos * hrow + rem * 16) = v[r];
          }
        }
      }
      const int nsum = (npos + 1) * KqI * 8;
      for (int i = threadIdx.x; i < nsum; i += kFThreads) {
        const int pos = i / (KqI * 8);
        const int g = (i % (KqI * 8)) / 2;
        const bool ok = pos < npos && g < KgI;
        s_hs[i] = __builtin_bit_cast(
            float, __builtin_amdgcn_raw_buffer_load_b32(hs_r, ok ? (uint32_t)(i * 4) : 0xFFFFF000u, 0, kDeviceScope));
      }
    }
    wait_vmcnt<0>();  // the h copies
    lds_barrier();
    const f32x4 z = {0.f, 0.f, 0.f, 0.f};
    for (int dd = 0; dd < nd; ++dd) {
      // The wave's pairs [w * per, w * per + per) in (segment, quad) order:
      // consecutive quads of one segment accumulate in registers; at a
      // segment's last pair in the range the partial sum goes to LDS as part
      // w - (first wave of the segment), real positions only.
      f32x4 acc = z, corr = z;
      auto chunk = [&](int cc, const u32x4 (&bb)[4], const float (&dv)[4]) {
        const int pair = w * per + cc;
        const int u = pair / KqI;
        const int q = pair % KqI;
        const int beg = uni(s_seg_beg[u]), cnt = uni(s_seg_cnt[u]);
        const int pos = n < cnt ? beg + n : npos;  // row npos is zero
        const u32x4* ho = reinterpret_cast<const u32x4*>(s_hb + (size_t)pos * hrow + q * 512 + p * 128);
        const u32x4 hh[8] = {ho[0], ho[1], ho[2], ho[3], ho[4], ho[5], ho[6], ho[7]};
        const float sp = s_hs[(pos * KqI + q) * 8 + p * 2] + s_hs[(pos * KqI + q) * 8 + p * 2 + 1];
        f32x4 pp[4];
#pragma unroll
        for (int gi = 0; gi < 4; ++gi) pp[gi] = mfma_f16_16x16x32(hh[2 * gi], bb[gi], z);
#pragma unroll
        for (int gi = 0; gi < 4; ++gi) pp[gi] = mfma_f16_16x16x32(hh[2 * gi + 1], bb[gi], pp[gi]);
        corr = mfma_f32_16x16x4(sp, dv[p], corr);
#pragma unroll
        for (int gi = 0; gi < 4; ++gi) acc += dv[gi] * pp[gi];
        if (q == KqI - 1 || cc == per - 1 || pair + 1 == n_c) {
          const f32x4 res = kUnitScale * acc - kUnitBias * corr;
          const int part = w - (u * KqI) / per;
          // lane (n, p) holds positions 4p + j of output row n
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int m = 4 * p + j;
            if (m < cnt) s_dred[((beg * KqI + part * cnt) + m) * 16 + n] = res[j];
          }
          acc = corr = z;
        }
      };
      int c0 = 0;
      if (pre) {
#pragma unroll
        for (int c = 0; c < kPreDq; ++c)
          if (c < cnt_w) chunk(c, pbb[c], pdv[c]);
        c0 = kPreDq;
      }
      {
        for (int cc = c0; cc < cnt_w; ++cc) {
          const char* slot = wdn + ((dd * per + cc) * kFW + w) * kDnChunkLds;
          const u32x4 wv = *reinterpret_cast<const u32x4*>(slot + lane * 16);
          float dv[4];
          unpack_scales(*reinterpret_cast<const uint2*>(slot + 1024 + n * 8), dv);
          const u32x4 bb[4] = {dequant_unit_f16(wv.x, dmask), dequant_unit_f16(wv.y, dmask),
                               dequant_unit_f16(wv.z, dmask), dequant_unit_f16(wv.w, dmask)};
          chunk(cc, bb, dv);
        }
      }
      lds_barrier();
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
        if (a.has_shared) {
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

  // ---- 6. the next call's tag --------------------------------------------------
  if (b == 0 && w == 0) {
    // every workgroup has read the generation once its presence is here
    for (int i0 = 0; i0 < G; i0 += kWave) {
      const int i = i0 + lane;
      bool done = i >= G;
      for (uint32_t it = 0;; ++it) {
        if (!done) done = __hip_atomic_load(&a.presence[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == tag64(tag);
        if (__all(done)) break;
        if (it >= a.wait_polls) {
          if (lane == 0) set_status(a.ctl, kStatusPresenceWait);
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
  if ((T * k + T) * KqI * 512 >= ((int64_t)1 << 31)) return false;
  // the smallest layout: one item of each kind per workgroup
  const int S_max = (int)((T * k < E ? T * k : E) + (has_shared ? 1 : 0));
  return fused_lds_layout((int)T, k, E, has_shared, (int)H, (int)I, 1, 1, S_max).bytes <= kFusedDynLdsMax;
}

FusedPlan fused_plan(int64_t T, int64_t H, int64_t I, int E, int k, int has_shared) {
  FusedPlan pl = {};
  pl.ok = false;
  if (!lib_config().decode_fused || !fused_shape_ok(T, H, I, E, k, has_shared)) return pl;
  int G = device_cus();
  if (G > kFusedMaxGrid) G = kFusedMaxGrid;
  if ((int64_t)G * kFW < T * E || G < 2) return pl;  // one logit per wave at most
  const int S_max = (int)((T * k < E ? T * k : E) + (has_shared ? 1 : 0));
  const int n_gu = S_max * (int)(I / kRowTile);
  const int n_dn = (int)(H / kRowTile);
  const int ng = (int)ceil_div(n_gu, G), nd = (int)ceil_div(n_dn, G);
  if (ng > kFusedMaxItems) return pl;  // the gate/up accumulators of one workgroup live in registers
  pl.lds = fused_lds_layout((int)T, k, E, has_shared, (int)H, (int)I, ng, nd, S_max);
  if (pl.lds.bytes > kFusedDynLdsMax) return pl;
  pl.G = G;
  pl.ok = true;
  return pl;
}

static hipError_t launch_fused(const FusedK& a, const FusedPlan& pl, hipStream_t stream) {
  static bool attr_set = false;
  if (!attr_set) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&moe_decode_fused_kernel),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)kFusedDynLdsMax);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  hipLaunchKernelGGL(moe_decode_fused_kernel, dim3(pl.G), dim3(kFThreads), pl.lds.bytes, stream, a);
  return hipGetLastError();
}

hipError_t launch_decode_fused(const FusedPlan& pl, const RouteArgs& r, const ExpertArgs& x, const FusedWs& ws,
                               hipStream_t stream) {
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
  a.flags = ws.flags;
  a.hq = ws.hq;
  a.hs = ws.hs;
  a.lds = pl.lds;
  const LibConfig cfg = lib_config();
  a.wait_polls = cfg.fused_wait_polls;
  a.skew_route = (cfg.fused_fault & 1u) ? 1u : 0u;
  a.skew_flags = (cfg.fused_fault & 2u) ? 1u : 0u;
  return launch_fused(a, pl, stream);
}

}  // namespace pmoe
