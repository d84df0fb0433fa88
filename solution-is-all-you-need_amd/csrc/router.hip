// router.hip -- MoE router for gfx950: gate GEMV (fp64, fixed order), top-k
// selection, softmax / sigmoid weights, and the stable expert permute.
//
// Reference semantics: PhantomTopKRouter.forward, tests/test_moe_routing.py:56-72
// (logits = x W^T; torch.topk(largest, sorted); softmax over the k selected).
//
// Logit arithmetic (identical in the CPU oracle, so selection is bit-exact):
//   products x*w are exact in fp64; 64 partial sums, partial l taking the
//   h with (h mod 256)/4 == l in increasing h; partials combined by the tree
//   p[l] += p[l ^ s] for s = 32..1 (commutative IEEE adds, so every pairing
//   order of one level gives the same bits); then + bias.
// Each wave computes TT tokens x EW experts.  Lane l owns partial l of every
// pair, so the 64 partials live one per lane; the tree is evaluated by a
// transposing butterfly: at level s each lane keeps half of its pairs and
// trades the other half with lane l ^ s, which yields exactly the tree above
// while spending one shuffle-add per pair per lane in total.
//
// Launches.  route_logits_kernel computes logits (and, spread over all its
// workgroups, the MFMA-ordered copy of x) with no inter-workgroup
// communication.  route_select_kernel gives one wave per token: a radix
// descent over the 64-bit order keys finds the k-th largest key, the k
// winners are ranked among themselves, then the weights.  For up to
// kFusedSelectBlocks select workgroups (decode) the last workgroup to finish
// runs the permute; beyond that permute_kernel does (one workgroup), and from
// kPermMultiSlots slots on three many-workgroup launches do (count, scan,
// place).  The hand-off costs one agent-scope release per select workgroup
// (an L2 write-back on a multi-XCD part), which is why it is reserved for
// small grids.
// Permute: per-wave expert counts, an (expert, wave)-major exclusive scan, and
// a second pass that places every slot at base + rank-within-round, where the
// rank comes from ballots over the bits of the expert id.  Placement depends
// only on slot order, never on atomics, so the permutation is deterministic
// and stable.
#include <float.h>
#include <math.h>

#include "moe_common.h"
#include "moe_launch.h"
#include "topk_common.h"

namespace pmoe {

struct RouteK {
  const void* x;
  const float* W;
  const float* bias;
  int64_t T, H;
  int E, k, score_mode;
  int32_t* topk_idx;
  float* topk_w;
  double* logits;
  // x preparation
  uint16_t* xq;
  float* xs;
  int64_t Kq;  // quads of H (padded)
  int prep_x;
  int prep_fp16;  // xq holds fp16 (rounded from bf16) instead of bf16
  // permute
  int do_permute;
  int has_shared;
  int32_t* offsets;       // [E + 2]
  int32_t* offsets_user;  // [E + 1] or null
  int32_t* active;        // [E + 1]
  int32_t* n_active;
  int32_t* sorted_slots;
  int32_t* slot_pos;
  int4* desc;        // [E + 1] {expert, begin, end, 0} per active segment, or null
  int32_t* seg_tok;  // [T*k + T] token of each segment position, or null
  int32_t* tiles;    // token tiles (see kTileWords), or null
  int32_t* n_tiles;
  int32_t* counter;  // select workgroups finished (fused permute); zeroed by the logits launch
  int fuse_permute;
  // many-slot permute: the select launch counts each slot into
  // perm_cnt[e * perm_nb + slot / perm_chunk] (zeroed by the first route
  // launch), which the count launch would otherwise do; null when it does not
  int32_t* perm_cnt;
  int64_t perm_chunk;
  int perm_nb;
};

template <typename XT>
__device__ inline void load_x4(const XT* x, int64_t off, float v[4]);

template <>
__device__ inline void load_x4<uint16_t>(const uint16_t* x, int64_t off, float v[4]) {
  const uint2 r = *reinterpret_cast<const uint2*>(x + off);
  v[0] = bf16_bits_to_float(r.x & 0xffffu);
  v[1] = bf16_bits_to_float(r.x >> 16);
  v[2] = bf16_bits_to_float(r.y & 0xffffu);
  v[3] = bf16_bits_to_float(r.y >> 16);
}

template <>
__device__ inline void load_x4<float>(const float* x, int64_t off, float v[4]) {
  const float4 r = *reinterpret_cast<const float4*>(x + off);
  v[0] = r.x;
  v[1] = r.y;
  v[2] = r.z;
  v[3] = r.w;
}

// Block-wide exclusive scan of three values at once (256 threads or more,
// one pair of barriers); s_tmp holds 3 ints per wave.  Returns the exclusive
// prefixes and writes the block totals to *total.
__device__ inline int3 block_exclusive_scan3(int3 v, int* s_tmp, int3* total) {
  const int lane = threadIdx.x % kWave;
  const int w = threadIdx.x / kWave;
  int3 inc = v;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int nx = __shfl_up(inc.x, off, kWave);
    const int ny = __shfl_up(inc.y, off, kWave);
    const int nz = __shfl_up(inc.z, off, kWave);
    if (lane >= off) {
      inc.x += nx;
      inc.y += ny;
      inc.z += nz;
    }
  }
  if (lane == kWave - 1) {
    s_tmp[3 * w] = inc.x;
    s_tmp[3 * w + 1] = inc.y;
    s_tmp[3 * w + 2] = inc.z;
  }
  lds_barrier();
  int3 prefix = make_int3(0, 0, 0), tot = make_int3(0, 0, 0);
  for (int i = 0; i < (int)(blockDim.x / kWave); ++i) {
    const int3 s = make_int3(s_tmp[3 * i], s_tmp[3 * i + 1], s_tmp[3 * i + 2]);
    if (i < w) {
      prefix.x += s.x;
      prefix.y += s.y;
      prefix.z += s.z;
    }
    tot.x += s.x;
    tot.y += s.y;
    tot.z += s.z;
  }
  lds_barrier();
  *total = tot;
  return make_int3(prefix.x + inc.x - v.x, prefix.y + inc.y - v.y, prefix.z + inc.z - v.z);
}

// Lanes of the wave holding the same expert id as this lane (valid lanes only).
__device__ inline uint64_t match_expert(int e, bool valid, int nbits) {
  uint64_t m = __ballot(valid);
  for (int b = 0; b < nbits; ++b) {
    const bool bit = valid && ((e >> b) & 1);
    const uint64_t bb = __ballot(bit);
    m &= bit ? bb : ~bb;
  }
  return m;
}

// Stable counting sort of n slots by expert, one workgroup of up to 1024
// threads (NW = blockDim / 64 waves).
//
// Besides offsets / sorted_slots / slot_pos it can emit, for the expert
// kernels, one descriptor {expert, begin, end} per active segment (the shared
// expert last, covering positions [T*k, T*k + T)), the token of every
// segment position, and the segments' 16-position token tiles.
__device__ __attribute__((always_inline)) inline void block_permute(const int32_t* __restrict__ idx, int64_t n, int k, int E, int64_t T,
                              int has_shared, int32_t* offsets, int32_t* offsets_user,
                              int32_t* active, int32_t* n_active, int32_t* sorted_slots,
                              int32_t* slot_pos, int4* desc, int32_t* seg_tok, int32_t* tiles,
                              int32_t* n_tiles) {
  constexpr int kMaxWaves = 16;
  __shared__ int s_cnt[kMaxWaves][kMaxExperts];
  __shared__ int s_tmp[3 * kMaxWaves];
  __shared__ int s_tb[kMaxExperts];   // first token tile of each expert's segment
  __shared__ int s_beg[kMaxExperts];  // first position of each expert's segment
  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int w = tid / kWave;
  const int NW = blockDim.x / kWave;
  int nbits = 1;
  while ((1 << nbits) < E) ++nbits;

  for (int i = tid; i < NW * kMaxExperts; i += blockDim.x) s_cnt[i / kMaxExperts][i % kMaxExperts] = 0;
  lds_barrier();

  const int64_t chunk = round_up(ceil_div(n, NW), kWave);
  const int64_t beg = w * chunk;
  const int64_t end = (beg + chunk < n) ? beg + chunk : n;

  // Expert ids of the wave's first kCached rounds are loaded together (from
  // clamped indices, so no load sits under a branch) and kept for pass 2.
  const uint64_t lt_mask = (1ull << lane) - 1ull;
  constexpr int kCached = 4;
  int cached[kCached];
#pragma unroll
  for (int i = 0; i < kCached; ++i) {
    const int64_t sl = beg + (int64_t)i * kWave + lane;
    const int v = idx[sl < n ? sl : n - 1];
    cached[i] = sl < end ? v : -1;
  }

  // Expert ids of rounds past the cached ones are loaded kBatch rounds at a
  // time (from clamped indices, all issued before any is used), so a long
  // chunk costs one memory round trip per kBatch rounds instead of one per
  // round; the rounds are still processed in order.
  constexpr int kBatch = 8;
  auto load_batch = [&](int64_t r0, int (&ev)[kBatch]) {
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const int64_t sl = r0 + (int64_t)j * kWave + lane;
      const int v = idx[sl < end ? sl : (end > 0 ? end - 1 : 0)];
      ev[j] = sl < end ? v : -1;
    }
  };

  // Pass 1: per-wave counts.
  auto count_round = [&](int e) {
    const bool valid = (e >= 0 && e < E);
    const uint64_t m = match_expert(e, valid, nbits);
    if (valid && (m & lt_mask) == 0) s_cnt[w][e] += __popcll(m);
  };
  {
    int64_t r0 = beg;
#pragma unroll
    for (int i = 0; i < kCached; ++i, r0 += kWave)
      if (r0 < end) count_round(cached[i]);
    for (; r0 < end; r0 += (int64_t)kBatch * kWave) {
      int ev[kBatch];
      load_batch(r0, ev);
#pragma unroll
      for (int j = 0; j < kBatch; ++j)
        if (r0 + (int64_t)j * kWave < end) count_round(ev[j]);
    }
  }
  lds_barrier();

  // Scan over experts: thread t owns experts t, t + blockDim, ... (at most
  // kMaxExperts / 256 = 2 per thread for 256 threads).
  constexpr int kPer = kMaxExperts / 256;
  int tot[kPer], act[kPer];
  int my_tot = 0, my_act = 0;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int e = tid * kPer + i;
    int t = 0;
    if (e < E && tid * kPer < kMaxExperts) {
      for (int ww = 0; ww < NW; ++ww) t += s_cnt[ww][e];
    }
    tot[i] = t;
    act[i] = (t > 0) ? 1 : 0;
    my_tot += t;
    my_act += act[i];
  }
  int my_tc = 0;
#pragma unroll
  for (int i = 0; i < kPer; ++i) my_tc += (tot[i] + 15) / 16;
  // positions, active experts and token tiles before this thread's experts
  int3 tot3;
  const int3 ex3 = block_exclusive_scan3(make_int3(my_tot, my_act, my_tc), s_tmp, &tot3);
  const int total = tot3.x, total_act = tot3.y, total_tiles = tot3.z;
  int run = ex3.x, arun = ex3.y, trun = ex3.z;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int e = tid * kPer + i;
    if (e < E) {
      offsets[e] = run;
      if (offsets_user) offsets_user[e] = run;
      if (act[i]) {
        active[arun] = e;
        if (desc) desc[arun] = make_int4(e, run, run + tot[i], 0);
      }
      s_tb[e] = trun;
      s_beg[e] = run;
      if (tiles) {
        // headers (pass 2 writes the tokens; words past the segment end are
        // left as they are and never read)
        for (int j = 0; j < (tot[i] + 15) / 16; ++j) {
          *reinterpret_cast<int4*>(tiles + (int64_t)(trun + j) * kTileWords) = make_int4(e, run + 16 * j, run + tot[i], 0);
        }
      }
      trun += (tot[i] + 15) / 16;
      int b = run;
      for (int ww = 0; ww < NW; ++ww) {
        const int c = s_cnt[ww][e];
        s_cnt[ww][e] = b;  // becomes the running base of (expert, wave)
        b += c;
      }
    }
    run += tot[i];
    arun += act[i];
  }
  if (tid == 0) {
    offsets[E] = total;
    if (offsets_user) offsets_user[E] = total;
    offsets[E + 1] = total + (has_shared ? (int)T : 0);
    if (has_shared) {
      active[total_act] = E;
      if (desc) desc[total_act] = make_int4(E, total, total + (int)T, 0);
    }
    *n_active = total_act + (has_shared ? 1 : 0);
  }
  if (has_shared && seg_tok) {
    for (int64_t t = tid; t < T; t += blockDim.x) seg_tok[n + t] = (int32_t)t;
  }
  if (tiles) {
    const int64_t n_sh = has_shared ? (T + 15) / 16 : 0;
    for (int64_t j = tid; j < n_sh; j += blockDim.x) {
      int32_t* tw = tiles + (total_tiles + j) * kTileWords;
      *reinterpret_cast<int4*>(tw) = make_int4(E, total + (int)(16 * j), total + (int)T, 0);
      for (int jj = 0; jj < 16 && 16 * j + jj < T; ++jj) tw[4 + jj] = (int32_t)(16 * j + jj);
    }
    if (tid == 0) {
      n_tiles[0] = total_tiles + (int)n_sh;
    }
  }
  if (desc) {
    // unused slots up to the launch bound min(E, n) + shared carry expert -1
    const int n_act = total_act + (has_shared ? 1 : 0);
    const int max_active = (int)((n < E) ? n : E) + (has_shared ? 1 : 0);
    for (int u = n_act + tid; u < max_active; u += blockDim.x) desc[u] = make_int4(-1, 0, 0, 0);
  }
  lds_barrier();

  // Pass 2: placement.
  auto place_round = [&](int64_t r0, int e) {
    const int64_t sl = r0 + lane;
    const bool valid = (e >= 0 && e < E);
    const uint64_t m = match_expert(e, valid, nbits);
    if (valid) {
      const uint64_t below = m & lt_mask;
      const int pos = s_cnt[w][e] + __popcll(below);
      sorted_slots[pos] = (int32_t)sl;
      slot_pos[sl] = pos;
      if (seg_tok) seg_tok[pos] = (int32_t)(sl / k);
      if (tiles) {
        const int rel = pos - s_beg[e];
        tiles[(int64_t)(s_tb[e] + rel / 16) * kTileWords + 4 + rel % 16] = (int32_t)(sl / k);
      }
      // Every lane of the group has read the base before the leader bumps
      // it: LDS operations of one wave complete in program order, and the
      // read above precedes this write in every lane's program.
      if (below == 0) s_cnt[w][e] = s_cnt[w][e] + __popcll(m);
    } else if (sl < end) {
      slot_pos[sl] = -1;
    }
  };
  {
    int64_t r0 = beg;
#pragma unroll
    for (int i = 0; i < kCached; ++i, r0 += kWave)
      if (r0 < end) place_round(r0, cached[i]);
    for (; r0 < end; r0 += (int64_t)kBatch * kWave) {
      int ev[kBatch];
      load_batch(r0, ev);
#pragma unroll
      for (int j = 0; j < kBatch; ++j)
        if (r0 + (int64_t)j * kWave < end) place_round(r0 + (int64_t)j * kWave, ev[j]);
    }
  }
}

// Top-k and weights of token t (topk_common.h), from the logits in the
// workspace to the caller's topk_idx / topk_w (and s_out when non-null).
template <int NV>
__device__ void wave_topk(const RouteK& a, int64_t t, uint64_t* s_ck, double* s_cv, int* s_ci,
                          double* s_val, int* s_idx, double* s_e, int* s_out) {
  wave_topk_row<NV>(a.logits + t * a.E, a.E, a.k, a.score_mode, s_ck, s_cv, s_ci, s_val, s_idx, s_e,
                    a.topk_idx + t * a.k, a.topk_w + t * a.k, s_out ? s_out + t * a.k : nullptr);
}

// MFMA-ordered copy of x (bf16) and fp32 group sums for tokens [t0, t0+TT),
// spread over the nparts workgroups that share this token tile (this one is
// number part), by nthreads threads of each (this one is number tid).
// Layout [t][q][p][gi][8]: one 16-byte chunk per (token, quad, part, group);
// chunk (p, gi) of quad q holds elements kmap(p, 0..7) of group 4q + gi, read
// as two 8-byte runs (4p..4p+3 and 4p+16..4p+19).  A group's sum adds its
// four parts' 8-element sums by an xor butterfly over p (lanes 4 and 8 apart).
// A thread's chunks come kPrepBatch at a time, all their loads issued before
// the first store: the compiler cannot move a load of x above a store to the
// copy (it cannot prove they do not alias), so a chunk at a time paid one
// memory round trip per chunk (16 of them per thread for 4096 tokens).
constexpr int kPrepBatch = 8;
__device__ void prep_x_tile(const RouteK& a, int64_t t0, int TT, int part, int nparts, int tid, int nthreads) {
  const uint16_t* x = static_cast<const uint16_t*>(a.x);
  const int Kg = (int)(a.H / kGroup);
  const int per_tok = (int)a.Kq * 16;
  const int n = TT * per_tok;
  const int lane = tid % kWave;
  const int stride = nparts * nthreads;
  const int wave0 = part * nthreads + (tid / kWave) * kWave;
  for (int c00 = wave0; c00 < n; c00 += kPrepBatch * stride) {  // wave-uniform
    uint2 lo[kPrepBatch], hi[kPrepBatch];
#pragma unroll
    for (int u = 0; u < kPrepBatch; ++u) {
      const int c = c00 + u * stride + lane;
      const int ti = c / per_tok;
      const int cc = c - ti * per_tok;
      const int64_t t = t0 + ti;
      const int g = 4 * (cc >> 4) + (cc & 3);
      lo[u] = hi[u] = make_uint2(0u, 0u);
      if (c < n && t < a.T && g < Kg) {
        const uint16_t* xr = x + t * a.H + (int64_t)g * kGroup + 4 * ((cc >> 2) & 3);
        lo[u] = *reinterpret_cast<const uint2*>(xr);
        hi[u] = *reinterpret_cast<const uint2*>(xr + 16);
      }
    }
#pragma unroll
    for (int u = 0; u < kPrepBatch; ++u) {
      const int c = c00 + u * stride + lane;
      const int ti = c / per_tok;
      const int cc = c - ti * per_tok;
      const int64_t t = t0 + ti;
      const bool valid = c < n && t < a.T;
      const int gi = cc & 3;
      const int p = (cc >> 2) & 3;
      const int g = 4 * (cc >> 4) + gi;
      u32x4 v;
      v.x = (lo[u].x & 0xffffu) | (lo[u].y << 16);
      v.y = (hi[u].x & 0xffffu) | (hi[u].y << 16);
      v.z = (lo[u].x >> 16) | (lo[u].y & 0xffff0000u);
      v.w = (hi[u].x >> 16) | (hi[u].y & 0xffff0000u);
      float sum = ((bf16_bits_to_float(lo[u].x & 0xffffu) + bf16_bits_to_float(lo[u].x >> 16)) +
                   (bf16_bits_to_float(lo[u].y & 0xffffu) + bf16_bits_to_float(lo[u].y >> 16))) +
                  ((bf16_bits_to_float(hi[u].x & 0xffffu) + bf16_bits_to_float(hi[u].x >> 16)) +
                   (bf16_bits_to_float(hi[u].y & 0xffffu) + bf16_bits_to_float(hi[u].y >> 16)));
      if (a.prep_fp16) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t b2 = v[i];
          v[i] = float_to_half_bits(bf16_bits_to_float(b2 & 0xffffu)) |
                 (float_to_half_bits(bf16_bits_to_float(b2 >> 16)) << 16);
        }
      }
      sum += __shfl_xor(sum, 4, kWave);
      sum += __shfl_xor(sum, 8, kWave);
      if (valid) {
        *reinterpret_cast<u32x4*>(a.xq + (t * per_tok + cc) * 8) = v;
        if (p == 0) a.xs[t * a.Kq * 4 + g] = sum;
      }
    }
  }
}

// Transposing butterfly over P pairs (P a power of two <= 64), see top.  Level
// S halves the live pairs (CNT -> CNT/2) until one remains, then plain
// butterfly levels finish the tree.  Recursion keeps every index a constant.
template <int S, int CNT, int P>
struct TreeLevel {
  __device__ static inline void run(double (&v)[P], int lane) {
    if constexpr (CNT > 1) {
      constexpr int HALF = CNT / 2;
      const bool hi = (lane & S) != 0;
#pragma unroll
      for (int i = 0; i < HALF; ++i) {
        const double send = hi ? v[i] : v[i + HALF];
        const double keep = hi ? v[i + HALF] : v[i];
        v[i] = keep + shfl_xor_f64(send, S);
      }
      if constexpr (S > 1) TreeLevel<S / 2, HALF, P>::run(v, lane);
    } else {
      v[0] = v[0] + shfl_xor_f64(v[0], S);
      if constexpr (S > 1) TreeLevel<S / 2, 1, P>::run(v, lane);
    }
  }
};

template <int P>
__device__ inline double tree_reduce_pairs(double (&v)[P]) {
  TreeLevel<32, P, P>::run(v, threadIdx.x % kWave);
  return v[0];
}

template <int P>
__device__ inline int tree_pair_of_lane(int lane) {
  int pair = 0, half = P / 2, s = 32;
  while (half >= 1) {
    if (lane & s) pair += half;
    half /= 2;
    s /= 2;
  }
  return pair;
}

template <typename XT, int TT, int EW, int CB>
__global__ __launch_bounds__(256) void route_logits_kernel(RouteK a) {
  constexpr int P = TT * EW;
  static_assert((P & (P - 1)) == 0 && P <= 64, "pairs per wave must be a power of two <= 64");
  const int lane = threadIdx.x % kWave;
  const int w = threadIdx.x / kWave;
  const int64_t t0 = (int64_t)blockIdx.y * TT;
  const int e0 = blockIdx.x * (4 * EW) + w * EW;
  const XT* x = static_cast<const XT*>(a.x);
  if (a.counter && blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) *a.counter = 0;
  // The bias of the expert this lane may write, fetched ahead of the GEMV.
  float bias_e = 0.0f;
  if (a.bias) {
    const int e = e0 + tree_pair_of_lane<P>(lane) % EW;
    bias_e = a.bias[e < a.E ? e : a.E - 1];
  }

  double acc[P];
#pragma unroll
  for (int i = 0; i < P; ++i) acc[i] = 0.0;

  // Chunks are loaded CB at a time (all loads of a batch issued before its
  // FMAs), then accumulated in increasing h as the contract requires.  Loads
  // are unconditional, from clamped addresses: a load under a branch gets its
  // own vmcnt(0) wait, which would serialise the batch.  Pairs of a clamped
  // expert or token are never stored, so only h needs a range: a batch of
  // whole in-range chunks adds its values as loaded, and only the batch that
  // reaches past H zeroes both operands of the lanes beyond it (so a
  // non-finite value read from the clamped address adds nothing).
  const int64_t nchunks = ceil_div(a.H, 256);
  const int64_t nfull = a.H / 256;  // chunks in range for every lane
  for (int64_t c0 = 0; c0 < nchunks; c0 += CB) {
    float wv[CB][EW][4];
    float xv[CB][TT][4];
    bool hok[CB];
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
      const int64_t h0 = (c0 + cb) * 256 + 4 * lane;
      hok[cb] = (c0 + cb) < nchunks && h0 < a.H;
      const int64_t hc = hok[cb] ? h0 : 0;
#pragma unroll
      for (int ei = 0; ei < EW; ++ei) {
        const int64_t ec = e0 + ei < a.E ? e0 + ei : a.E - 1;
        const float4 r = *reinterpret_cast<const float4*>(a.W + ec * a.H + hc);
        wv[cb][ei][0] = r.x;
        wv[cb][ei][1] = r.y;
        wv[cb][ei][2] = r.z;
        wv[cb][ei][3] = r.w;
      }
#pragma unroll
      for (int ti = 0; ti < TT; ++ti) {
        const int64_t tc = t0 + ti < a.T ? t0 + ti : a.T - 1;
        load_x4<XT>(x, tc * a.H + hc, xv[cb][ti]);
      }
    }
    // the MFMA-ordered copy of x, its loads in flight with the first batch's
    if (c0 == 0 && a.prep_x)
      prep_x_tile(a, t0, TT, (int)blockIdx.x, (int)gridDim.x, (int)threadIdx.x, (int)blockDim.x);
    if (c0 + CB > nfull) {
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
          for (int ei = 0; ei < EW; ++ei) wv[cb][ei][i] = hok[cb] ? wv[cb][ei][i] : 0.0f;
#pragma unroll
          for (int ti = 0; ti < TT; ++ti) xv[cb][ti][i] = hok[cb] ? xv[cb][ti][i] : 0.0f;
        }
      }
    }
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
#pragma unroll
      for (int ti = 0; ti < TT; ++ti) {
#pragma unroll
        for (int ei = 0; ei < EW; ++ei) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            acc[ti * EW + ei] += (double)xv[cb][ti][i] * (double)wv[cb][ei][i];
          }
        }
      }
    }
  }

  const double tot = tree_reduce_pairs<P>(acc);
  {
    constexpr int kLowBits = (P == 1) ? 6 : (P == 2) ? 5 : (P == 4) ? 4 : (P == 8) ? 3 : (P == 16) ? 2 : (P == 32) ? 1 : 0;
    if ((lane & ((1 << kLowBits) - 1)) == 0) {
      const int pair = tree_pair_of_lane<P>(lane);
      const int ti = pair / EW;
      const int ei = pair % EW;
      const int64_t t = t0 + ti;
      const int e = e0 + ei;
      if (t < a.T && e < a.E) {
        double v = tot;
        if (a.bias) v = v + (double)bias_e;
        a.logits[t * a.E + e] = v;
      }
    }
  }

  if (a.prep_x && blockIdx.x == 1 % gridDim.x && blockIdx.y == 0) {
    // all-zero activation row T, read by expert lanes past a segment
    for (int64_t i = threadIdx.x; i < a.Kq * 128; i += blockDim.x) a.xq[a.T * a.Kq * 128 + i] = 0;
    for (int64_t i = threadIdx.x; i < a.Kq * 4; i += blockDim.x) a.xs[a.T * a.Kq * 4 + i] = 0.0f;
  }
}

// Top-k and weights, one wave per token (grid-stride).  With do_permute, a
// launch of one workgroup continues with the permute, and a fused launch hands
// the permute to the last workgroup to finish.  (One workgroup of up to 16
// waves for up to 64 tokens, its selection handed to the permute in LDS,
// measured slower than the hand-off: route 24.4 vs 19.2 us at 32 tokens,
// 57 vs 39 us at 64 tokens of H 7168.)
constexpr int kSelectWaves = 4;
constexpr int kFusedSelectBlocks = 16;

template <int NV>
__global__ __launch_bounds__(256) void route_select_kernel(RouteK a) {
  __shared__ uint64_t s_ck[kSelectWaves][kMaxTopK];
  __shared__ double s_cv[kSelectWaves][kMaxTopK];
  __shared__ int s_ci[kSelectWaves][kMaxTopK];
  __shared__ double s_val[kSelectWaves][kMaxTopK];
  __shared__ double s_e[kSelectWaves][kMaxTopK];
  __shared__ int s_idx[kSelectWaves][kMaxTopK];
  __shared__ int s_sel[kSelectWaves * kMaxTopK];  // one workgroup: every token's selection, for the permute
  __shared__ int s_last;
  const int w = threadIdx.x / kWave;
  const int nw = blockDim.x / kWave;
  const bool single = gridDim.x == 1 && a.T <= kSelectWaves;
  const int lane = threadIdx.x % kWave;
  for (int64_t t = (int64_t)blockIdx.x * nw + w; t < a.T; t += (int64_t)gridDim.x * nw) {
    wave_topk<NV>(a, t, s_ck[w], s_cv[w], s_ci[w], s_val[w], s_idx[w], s_e[w], single ? s_sel : nullptr);
    // slot t k + j (j = lane) counted for the many-slot permute; the
    // selection of slot j is in s_idx[j] (this wave's own LDS stores)
    if (a.perm_cnt && lane < a.k) {
      const int e = s_idx[w][lane];
      if (e >= 0 && e < a.E) atomicAdd(a.perm_cnt + (int64_t)e * a.perm_nb + (t * a.k + lane) / a.perm_chunk, 1);
    }
  }
  if (!a.do_permute) return;
  if (single) {
    // the selection reaches the permute through LDS, not a global round trip
    lds_barrier();
    block_permute(s_sel, a.T * a.k, a.k, a.E, a.T, a.has_shared, a.offsets, a.offsets_user, a.active,
                  a.n_active, a.sorted_slots, a.slot_pos, a.desc, a.seg_tok, a.tiles, a.n_tiles);
    return;
  }
  if (gridDim.x > 1) {
    if (!a.fuse_permute) return;
    // Every wave's top-k stores have reached L2 before the barrier; thread 0
    // then writes the XCD's L2 back (agent-scope release) and counts in.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
      __threadfence();
      s_last = atomicAdd(a.counter, 1) == (int)gridDim.x - 1;
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();  // acquire: the other workgroups' top-k
  }
  __syncthreads();
  block_permute(a.topk_idx, a.T * a.k, a.k, a.E, a.T, a.has_shared, a.offsets, a.offsets_user, a.active,
                a.n_active, a.sorted_slots, a.slot_pos, a.desc, a.seg_tok, a.tiles, a.n_tiles);
}

__global__ __launch_bounds__(1024) void permute_kernel(const int32_t* idx, int64_t T, int k, int E,
                                                       int has_shared, int32_t* offsets,
                                                       int32_t* offsets_user, int32_t* active,
                                                       int32_t* n_active, int32_t* sorted_slots,
                                                       int32_t* slot_pos, int4* desc,
                                                       int32_t* seg_tok, int32_t* tiles, int32_t* n_tiles) {
  block_permute(idx, T * k, k, E, T, has_shared, offsets, offsets_user, active, n_active,
                sorted_slots, slot_pos, desc, seg_tok, tiles, n_tiles);
}

// Logits for many tokens (prefill): the same per-lane partials and tree as
// route_logits_kernel, with TT tokens x EW experts per wave and the loads of
// chunk c + 1 in flight while chunk c is summed.  x stays packed (bf16 pairs)
// in registers until its FMAs, so two chunks of operands fit beside the
// 2 * TT * EW fp64 accumulators.
// tokens x experts per wave of the many-token logits kernel
constexpr int kBigTT = 8;
constexpr int kBigEW = 4;

template <typename XT>
struct XRaw;
template <>
struct XRaw<uint16_t> {
  uint2 v;
  __device__ inline void load(const uint16_t* x, int64_t off) { v = *reinterpret_cast<const uint2*>(x + off); }
  __device__ inline float get(int i) const {
    const uint32_t w = i < 2 ? v.x : v.y;
    return bf16_bits_to_float((i & 1) ? (w >> 16) : (w & 0xffffu));
  }
};
template <>
struct XRaw<float> {
  float4 v;
  __device__ inline void load(const float* x, int64_t off) { v = *reinterpret_cast<const float4*>(x + off); }
  __device__ inline float get(int i) const { return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w)); }
};

template <typename XT, int TT, int EW>
struct LogitsChunk {
  float4 w[EW];
  XRaw<XT> x[TT];
  bool hok;
};

template <typename XT, int TT, int EW>
__device__ inline void logits_load(const RouteK& a, const XT* x, int64_t c, int64_t nchunks, int64_t t0, int e0,
                                   LogitsChunk<XT, TT, EW>& k) {
  const int lane = threadIdx.x % kWave;
  const int64_t h0 = c * 256 + 4 * lane;
  k.hok = c < nchunks && h0 < a.H;
  const int64_t hc = k.hok ? h0 : 0;
#pragma unroll
  for (int ei = 0; ei < EW; ++ei) {
    const int64_t ec = e0 + ei < a.E ? e0 + ei : a.E - 1;
    k.w[ei] = *reinterpret_cast<const float4*>(a.W + ec * a.H + hc);
  }
#pragma unroll
  for (int ti = 0; ti < TT; ++ti) {
    const int64_t tc = t0 + ti < a.T ? t0 + ti : a.T - 1;
    k.x[ti].load(x, tc * a.H + hc);
  }
}

template <typename XT, int TT, int EW>
__global__ __launch_bounds__(256) void route_logits_big_kernel(RouteK a) {
  constexpr int P = TT * EW;
  static_assert((P & (P - 1)) == 0 && P <= 64, "pairs per wave must be a power of two <= 64");
  const int lane = threadIdx.x % kWave;
  const int w = threadIdx.x / kWave;
  const int64_t t0 = (int64_t)blockIdx.y * TT;
  const int e0 = blockIdx.x * (4 * EW) + w * EW;
  const XT* x = static_cast<const XT*>(a.x);
  if (a.prep_x) prep_x_tile(a, t0, TT, (int)blockIdx.x, (int)gridDim.x, (int)threadIdx.x, (int)blockDim.x);
  if (a.counter && blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) *a.counter = 0;
  float bias_e = 0.0f;
  if (a.bias) {
    const int e = e0 + tree_pair_of_lane<P>(lane) % EW;
    bias_e = a.bias[e < a.E ? e : a.E - 1];
  }
  double acc[P];
#pragma unroll
  for (int i = 0; i < P; ++i) acc[i] = 0.0;
  const int64_t nchunks = ceil_div(a.H, 256);
  LogitsChunk<XT, TT, EW> cur, nxt;
  logits_load<XT, TT, EW>(a, x, 0, nchunks, t0, e0, cur);
  for (int64_t c = 0; c < nchunks; ++c) {
    logits_load<XT, TT, EW>(a, x, c + 1, nchunks, t0, e0, nxt);
    // out-of-range experts and tokens are never stored, so only the h range
    // needs masking (both operands, so a non-finite weight read from the
    // clamped address adds nothing); partials add in increasing h as the
    // contract requires
    float4 wm[EW];
#pragma unroll
    for (int ei = 0; ei < EW; ++ei)
      wm[ei] = cur.hok ? cur.w[ei] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int ti = 0; ti < TT; ++ti) {
      double xd[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) xd[i] = cur.hok ? (double)cur.x[ti].get(i) : 0.0;
#pragma unroll
      for (int ei = 0; ei < EW; ++ei) {
        const float4 wv = wm[ei];
        acc[ti * EW + ei] += xd[0] * (double)wv.x;
        acc[ti * EW + ei] += xd[1] * (double)wv.y;
        acc[ti * EW + ei] += xd[2] * (double)wv.z;
        acc[ti * EW + ei] += xd[3] * (double)wv.w;
      }
    }
    cur = nxt;
  }
  const double tot = tree_reduce_pairs<P>(acc);
  {
    constexpr int kLowBits = (P == 1) ? 6 : (P == 2) ? 5 : (P == 4) ? 4 : (P == 8) ? 3 : (P == 16) ? 2 : (P == 32) ? 1 : 0;
    if ((lane & ((1 << kLowBits) - 1)) == 0) {
      const int pair = tree_pair_of_lane<P>(lane);
      const int64_t t = t0 + pair / EW;
      const int e = e0 + pair % EW;
      if (t < a.T && e < a.E) {
        double v = tot;
        if (a.bias) v = v + (double)bias_e;
        a.logits[t * a.E + e] = v;
      }
    }
  }
}

// ------------------------------------------------- many-token router, two passes
//
// For prefill batches the fixed-order fp64 logits of every (token, expert)
// pair cost 100 us at 4096 tokens of H 2048, E 128 -- while only the top k
// of each token, and the experts near the k-th, decide anything.  So:
//   route_approx_kernel: L~ = x . (w_hi + w_lo) on the matrix cores for every
//     pair, with w_hi = bf16(w) and w_lo = bf16(w - w_hi) (both rounded to
//     nearest), plus the norms |x_t| and |w_e|;
//   route_candidates_kernel (one wave per token; four more waves per
//     workgroup write the GEMM's copy of x meanwhile): the error bound
//     |L~ - L| <= C(H) |x_t| |w_e| gives every expert an interval; experts
//     whose upper end reaches the k-th largest lower end are the candidates
//     (a superset of the exact top k: any expert below that has k others
//     strictly above it); the others' logits are set to -inf;
//   route_exact_kernel (per expert and block of tokens): the fixed-order
//     fp64 logits (contract above) of the candidate pairs, 16 tokens per wave
//     so each lane's slice of the weight row is loaded once per 16 pairs;
//   route_select_kernel: the exact selection and weights, unchanged.
// The bound.  Rounding: w - w_hi is exact in fp32, so |w - w_hi - w_lo| <=
// 2^-8 |w - w_hi| <= 2^-16 |w| (an 8-bit significand rounds to within 2^-8
// of the value), and |w_hi| + |w_lo| <= (1 + 2^-7) |w|.  Arithmetic: the
// products of two bf16 values are exact in fp32; each 32-wide K step s is
// summed by two chained MFMAs from zero (64 products, at most 63 roundings
// of 2^-24, taken 4x for whatever order and internal precision the matrix
// cores use: 252 u), and the S = ceil(H / 32) step sums are added in fp32
// on the vector ALU (S u more).  With Cauchy-Schwarz, sum |x| |w| <= |x| |w|,
// so C(H) = 2^-16 + (252 + S) 2^-24 (1 + 2^-7), with margin; |x| and |w| are
// taken as their computed fp32 norms plus sqrt(H + 8) 2^-63, which covers
// what squares and sums below 2^-126 can lose (so rows of tiny entries get a
// bound, not 0), and denormal inputs or products the matrix cores may flush
// add an absolute term.  Tokens with a non-finite approximate logit or norm
// take every expert as a candidate (the full exact row), so NaN and inf
// follow the contract exactly as on the one-pass path.
constexpr int kApproxTok = 64;     // tokens per approx workgroup (4 waves x 16)
constexpr int kApproxExp = 16;     // experts per approx workgroup (one tile of 16; 512 workgroups at E 128)
constexpr int kApproxChunk = 256;  // K staged in LDS per step
constexpr int kApproxUnits = kApproxExp * kApproxChunk / 8 / 256;  // 8-wide W units per thread per chunk
constexpr int kExactTok = 1024;    // tokens scanned per exact workgroup (a multiple of 256)
constexpr int kExactP = 16;        // token pairs per wave pass

// Workgroup b of a one-dimensional grid of n_eb x n_tt runs on XCD b % 8.
// When the token tiles divide evenly over the XCDs, XCD x takes token tiles
// x, x + 8, ... with every expert block of each, so a tile's x is fetched
// into that XCD's L2 once and read there by all n_eb workgroups (the plain
// order put a tile's expert blocks on n_eb different XCDs, each fetching it).
__device__ inline void xcd_tile_map(int64_t b, int64_t n_eb, int64_t n_tt, int64_t* eb, int64_t* tt) {
  if (n_tt % 8 == 0) {
    const int64_t j = b / 8;
    *tt = b % 8 + 8 * (j / n_eb);
    *eb = j % n_eb;
  } else {
    *tt = b / n_eb;
    *eb = b % n_eb;
  }
}

__global__ __launch_bounds__(256) void route_approx_kernel(RouteK a, float* approx, float* nx, float* nw) {
  // W chunk as bf16 B operands w_hi and w_lo: [expert tile][K step][lane] 16-byte units
  __shared__ u32x4 s_w[(kApproxExp / 16) * (kApproxChunk / 32) * kWave];
  __shared__ u32x4 s_wl[(kApproxExp / 16) * (kApproxChunk / 32) * kWave];
  __shared__ float s_nw[kApproxExp];
  const int lane = threadIdx.x % kWave;
  const int w = threadIdx.x / kWave;
  const int64_t n_eb = ceil_div(a.E, kApproxExp);
  int64_t eb, tt;
  xcd_tile_map(blockIdx.x, n_eb, ceil_div(a.T, kApproxTok), &eb, &tt);
  const int64_t t0 = tt * kApproxTok;
  const int e0 = (int)eb * kApproxExp;
  const uint16_t* x = static_cast<const uint16_t*>(a.x);
  if (a.counter && blockIdx.x == 0 && threadIdx.x == 0) *a.counter = 0;
  if (a.perm_cnt)
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < (int64_t)a.E * a.perm_nb;
         i += (int64_t)gridDim.x * blockDim.x)
      a.perm_cnt[i] = 0;
  // A rows: token t0 + 16 w + lane % 16 (clamped), K 8 (lane / 16) .. + 8 of each step
  const int64_t tr = t0 + 16 * w + lane % 16;
  const uint16_t* xrow = x + (tr < a.T ? tr : a.T - 1) * a.H + 8 * (lane / 16);
  f32x4 acc[kApproxExp / 16];
#pragma unroll
  for (int i = 0; i < kApproxExp / 16; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  float sx = 0.0f;                // this lane's share of |x|^2
  float sw[kApproxUnits];         // |w_e|^2 shares of the units this thread converts
#pragma unroll
  for (int i = 0; i < kApproxUnits; ++i) sw[i] = 0.0f;
  // unit u = threadIdx.x + 256 i: expert u / 32, 8-wide K block u % 32 of the chunk
  float4 wr[kApproxUnits][2];
  u32x4 ar[kApproxChunk / 32];
  auto load = [&](int64_t c0) {
    const int kc = (int)(a.H - c0 < kApproxChunk ? a.H - c0 : kApproxChunk);
#pragma unroll
    for (int i = 0; i < kApproxUnits; ++i) {
      const int u = threadIdx.x + 256 * i;
      const int e = u / 32, kb = u % 32;
      const int ec = e0 + e < a.E ? e0 + e : a.E - 1;
      const int kbc = 8 * kb < kc ? kb : 0;  // past the end: a valid address, zeroed at the store
      const float4* src = reinterpret_cast<const float4*>(a.W + (int64_t)ec * a.H + c0 + 8 * kbc);
      wr[i][0] = src[0];
      wr[i][1] = src[1];
    }
#pragma unroll
    for (int s = 0; s < kApproxChunk / 32; ++s)
      ar[s] = 32 * s < kc ? *reinterpret_cast<const u32x4*>(xrow + c0 + 32 * s) : u32x4{0u, 0u, 0u, 0u};
  };
  load(0);
  for (int64_t c0 = 0; c0 < a.H; c0 += kApproxChunk) {
    const int kc = (int)(a.H - c0 < kApproxChunk ? a.H - c0 : kApproxChunk);  // multiple of 32
#pragma unroll
    for (int i = 0; i < kApproxUnits; ++i) {
      const int u = threadIdx.x + 256 * i;
      const int e = u / 32, kb = u % 32;
      u32x4 v = {0u, 0u, 0u, 0u}, vl = {0u, 0u, 0u, 0u};
      if (8 * kb < kc) {
        const float f[8] = {wr[i][0].x, wr[i][0].y, wr[i][0].z, wr[i][0].w,
                            wr[i][1].x, wr[i][1].y, wr[i][1].z, wr[i][1].w};
#pragma unroll
        for (int j = 0; j < 8; ++j) sw[i] = __builtin_fmaf(f[j], f[j], sw[i]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t h0 = float_to_bf16_bits(f[2 * j]), h1 = float_to_bf16_bits(f[2 * j + 1]);
          v[j] = h0 | (h1 << 16);
          vl[j] = float_to_bf16_bits(f[2 * j] - bf16_bits_to_float(h0)) |
                  (float_to_bf16_bits(f[2 * j + 1] - bf16_bits_to_float(h1)) << 16);
        }
      }
      const int slot = ((e / 16) * (kApproxChunk / 32) + kb / 4) * kWave + (e % 16) + 16 * (kb % 4);
      s_w[slot] = v;
      s_wl[slot] = vl;
    }
    u32x4 av[kApproxChunk / 32];
#pragma unroll
    for (int s = 0; s < kApproxChunk / 32; ++s) av[s] = ar[s];
    __syncthreads();
    if (c0 + kApproxChunk < a.H) load(c0 + kApproxChunk);  // the next chunk flies during this one's MFMAs
#pragma unroll
    for (int s = 0; s < kApproxChunk / 32; ++s) {
      if (32 * s >= kc) break;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float lo = bf16_bits_to_float(av[s][j] & 0xffffu), hi = bf16_bits_to_float(av[s][j] >> 16);
        sx = __builtin_fmaf(lo, lo, sx);
        sx = __builtin_fmaf(hi, hi, sx);
      }
      // each step's sum from zero, added on the vector ALU (the bound's
      // S u term; chained MFMAs would add H roundings)
#pragma unroll
      for (int et = 0; et < kApproxExp / 16; ++et) {
        const int slot = (et * (kApproxChunk / 32) + s) * kWave + lane;
        f32x4 ps = mfma_bf16_16x16x32(av[s], s_w[slot], f32x4{0.f, 0.f, 0.f, 0.f});
        ps = mfma_bf16_16x16x32(av[s], s_wl[slot], ps);
        acc[et] += ps;
      }
    }
    __syncthreads();  // every wave has read the B operands before the next chunk overwrites them
  }
  // |x_t|^2: the four lanes of a row hold disjoint shares
  sx += __shfl_xor(sx, 16, kWave);
  sx += __shfl_xor(sx, 32, kWave);
  // |w_e|^2: the 32 threads of expert e (u / 32 == e, consecutive lanes)
#pragma unroll
  for (int i = 0; i < kApproxUnits; ++i) {
    float v = sw[i];
    v += __shfl_xor(v, 1, kWave);
    v += __shfl_xor(v, 2, kWave);
    v += __shfl_xor(v, 4, kWave);
    v += __shfl_xor(v, 8, kWave);
    v += __shfl_xor(v, 16, kWave);
    if (lane % 32 == 0) s_nw[(threadIdx.x + 256 * i) / 32] = v;
  }
  __syncthreads();
  // outputs: lane (n, g) of tile et holds tokens 16 w + 4 g + j, expert 16 et + n
#pragma unroll
  for (int et = 0; et < kApproxExp / 16; ++et) {
    const int e = e0 + 16 * et + lane % 16;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t t = t0 + 16 * w + 4 * (lane / 16) + j;
      if (t < a.T && e < a.E) approx[t * a.E + e] = acc[et][j];
    }
  }
  if (eb == 0 && lane < 16 && tr < a.T) nx[tr] = sqrtf(sx);
  if (tt == 0 && threadIdx.x < kApproxExp && e0 + (int)threadIdx.x < a.E)
    nw[e0 + threadIdx.x] = sqrtf(s_nw[threadIdx.x]);
}

// Order-preserving 32-bit key of a finite or infinite fp32 value.
__device__ inline uint32_t f32_key(float v) {
  const uint32_t b = __builtin_bit_cast(uint32_t, v == 0.0f ? 0.0f : v);
  return (b >> 31) ? ~b : (b | 0x80000000u);
}

// Candidates of each token (one wave per token): cand[e * T + t] = 1 for a
// candidate, else 0 and logits[t][e] = -inf.
template <int NV>
__global__ __launch_bounds__(512) void route_candidates_kernel(RouteK a, const float* approx, const float* nx,
                                                               const float* nw, uint8_t* cand) {
  const int lane = threadIdx.x % kWave;
  const int w = threadIdx.x / kWave;
  // C(H) of the bound, with 2^-8 relative room for the rounding of the norms
  const float S = (float)((a.H + 31) / 32);
  const float cH = (1.0f / 65536.0f + (252.0f + S) * (1.0f / 16777216.0f) * 1.02f) * (1.0f + 1.0f / 256.0f);
  const float sqrtH = sqrtf((float)a.H) * 1.01f;
  // The norms are fp32 sums of H + 8 squares.  Squares and partial sums below
  // 2^-126 may be flushed or lose bits, at most 2^-126 each, so the true
  // |v|^2 <= computed + (H + 8) 2^-126 and |v| <= computed + sqrt(H + 8) 2^-63:
  // that slack is added to both norms.  Without it a token (or an expert row)
  // of entries below about 2^-75 would get a norm of 0 and a bound far below
  // the bf16 rounding error of its approximate logits.
  const float slack = sqrtf((float)a.H + 8.0f) * 1.0842022e-19f * 1.01f;
  if (w >= 4) {
    // Waves 4-7 write the workgroup's tokens' MFMA-ordered x copy and group
    // sums meanwhile: the candidate waves are latency-bound and leave memory
    // idle (in the approximate-logit launch the copy cost 7 us at 4096 tokens
    // of H 2048 and 17.5 us at 2048 of H 7168)
    if (a.prep_x)
      for (int64_t t0 = (int64_t)blockIdx.x * 4; t0 < a.T; t0 += (int64_t)gridDim.x * 4)
        prep_x_tile(a, t0, 4, 0, 1, (int)threadIdx.x - 4 * kWave, 4 * kWave);
    return;
  }
  for (int64_t t = (int64_t)blockIdx.x * 4 + w; t < a.T; t += (int64_t)gridDim.x * 4) {
    const float nxt = nx[t] + slack;
    float lo[NV], hi[NV];
    bool all = !isfinite(nxt);
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const int e = lane + kWave * v;
      const int ec = e < a.E ? e : a.E - 1;
      const float l = approx[t * a.E + ec];
      const float b = a.bias ? a.bias[ec] : 0.0f;
      const float m = l + b;
      // + fp32 rounding of m and of the interval ends, + inputs the matrix
      // cores may flush as denormals (each |x| or |w| < 2^-126, so their
      // products sum to at most 2^-126 sqrt(H) (|x| + |w|))
      const float nwe = nw[ec] + slack;
      const float bnd = cH * nxt * nwe + (fabsf(l) + fabsf(b)) * (1.0f / 4194304.0f) +
                        sqrtH * 2.4e-38f * (nxt + nwe) + 1e-30f;
      all = all || (e < a.E && !(isfinite(m) && isfinite(bnd)));
      lo[v] = m - bnd;
      hi[v] = m + bnd;
    }
    all = __ballot(all) != 0ull;
    // the k-th largest lower end: radix descent over 32-bit keys
    uint32_t kth = 0;
    if (!all) {
      uint32_t key[NV];
#pragma unroll
      for (int v = 0; v < NV; ++v) key[v] = lane + kWave * v < a.E ? f32_key(lo[v]) : 0u;
      for (int bit = 31; bit >= 0; --bit) {
        const uint32_t c = kth | (1u << bit);
        int cnt = 0;
#pragma unroll
        for (int v = 0; v < NV; ++v) cnt += __popcll(__ballot(key[v] >= c));
        if (cnt >= a.k) kth = c;
      }
    }
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const int e = lane + kWave * v;
      if (e < a.E) {
        const bool c = all || f32_key(hi[v]) >= kth;
        cand[(int64_t)e * a.T + t] = c ? 1 : 0;
        if (!c) a.logits[t * a.E + e] = -INFINITY;
      }
    }
  }
}

// Exact logits of the candidate pairs of expert blockIdx.y among tokens
// [kExactTok * blockIdx.x, + kExactTok): the tokens are compacted in LDS, then
// each wave takes 16 at a time (the last group padded by repeating its last
// token): lane l sums, for each token, the h with (h mod 256) / 4 == l in
// increasing h, with its slice of the weight row loaded once for the 16.
__global__ __launch_bounds__(256) void route_exact_kernel(RouteK a, const uint8_t* cand) {
  constexpr int kSub = kExactTok / 256;  // 256-token sub-blocks, one token per thread each
  __shared__ int s_tok[kExactTok];
  __shared__ int s_cnt[4 * kSub];
  const int lane = threadIdx.x % kWave;
  const int w = threadIdx.x / kWave;
  const int e = blockIdx.y;
  const int64_t t0 = (int64_t)blockIdx.x * kExactTok;
  // compaction in token order: in sub-block sb, wave w takes tokens
  // t0 + 256 sb + 64 w + lane
  bool c[kSub];
  uint64_t m[kSub];
#pragma unroll
  for (int sb = 0; sb < kSub; ++sb) {
    const int64_t t = t0 + 256 * sb + 64 * w + lane;
    c[sb] = t < a.T && cand[(int64_t)e * a.T + t] != 0;
    m[sb] = __ballot(c[sb]);
    if (lane == 0) s_cnt[sb * 4 + w] = __popcll(m[sb]);
  }
  __syncthreads();
  int n = 0;
  for (int i = 0; i < 4 * kSub; ++i) n += s_cnt[i];
#pragma unroll
  for (int sb = 0; sb < kSub; ++sb) {
    int base = 0;
    for (int i = 0; i < sb * 4 + w; ++i) base += s_cnt[i];
    if (c[sb]) s_tok[base + __popcll(m[sb] & ((1ull << lane) - 1ull))] = 256 * sb + 64 * w + lane;
  }
  __syncthreads();
  const uint16_t* x = static_cast<const uint16_t*>(a.x);
  const float* wrow = a.W + (int64_t)e * a.H;
  const double bias = a.bias ? (double)a.bias[e] : 0.0;
  for (int g0 = kExactP * w; g0 < n; g0 += kExactP * 4) {
    int64_t tk[kExactP];
#pragma unroll
    for (int j = 0; j < kExactP; ++j) tk[j] = t0 + s_tok[g0 + j < n ? g0 + j : n - 1];
    double acc[kExactP];
#pragma unroll
    for (int j = 0; j < kExactP; ++j) acc[j] = 0.0;
    // the loads of chunk h0 + 256 are issued before chunk h0's FMAs
    float4 wn = make_float4(0.f, 0.f, 0.f, 0.f);
    uint2 xn[kExactP];
    auto load = [&](int64_t h0) {
      wn = *reinterpret_cast<const float4*>(wrow + h0);
#pragma unroll
      for (int j = 0; j < kExactP; ++j) xn[j] = *reinterpret_cast<const uint2*>(x + tk[j] * a.H + h0);
    };
    if (4 * lane < a.H) load(4 * lane);
    for (int64_t h0 = 4 * lane; h0 < a.H; h0 += 256) {
      const float4 wv = wn;
      uint2 xv[kExactP];
#pragma unroll
      for (int j = 0; j < kExactP; ++j) xv[j] = xn[j];
      if (h0 + 256 < a.H) load(h0 + 256);
      const double wd[4] = {(double)wv.x, (double)wv.y, (double)wv.z, (double)wv.w};
#pragma unroll
      for (int j = 0; j < kExactP; ++j) {
        acc[j] += (double)bf16_bits_to_float(xv[j].x & 0xffffu) * wd[0];
        acc[j] += (double)bf16_bits_to_float(xv[j].x >> 16) * wd[1];
        acc[j] += (double)bf16_bits_to_float(xv[j].y & 0xffffu) * wd[2];
        acc[j] += (double)bf16_bits_to_float(xv[j].y >> 16) * wd[3];
      }
    }
    const double tot = tree_reduce_pairs<kExactP>(acc);
    if ((lane & 3) == 0) {
      const int pair = tree_pair_of_lane<kExactP>(lane);
      double v = tot;
      if (a.bias) v = v + bias;
      a.logits[tk[pair] * a.E + e] = v;
    }
  }
}

// ------------------------------------------------- permute, many workgroups
//
// For large batches the one-workgroup permute is bound by one CU's issue
// rate (65 us for 32768 slots).  The same stable counting sort then runs as
// up to three launches:
//   permute_count_kernel: workgroup b counts, per expert, the slots of its
//     contiguous chunk into cnt[e][b] (after a two-pass route with a small
//     count table the select launch has counted them instead);
//   permute_scan_kernel (one workgroup): expert totals, the offsets, active
//     list, descriptors, token-tile headers and shared segment exactly as the
//     one-workgroup permute writes them, and cnt[e][b] replaced by the
//     position where chunk b's first slot of expert e goes;
//   permute_place_kernel: workgroup b re-counts its chunk per wave and places
//     every slot at its chunk base + the counts of earlier waves + its rank
//     within the round;
//   permute_scan_place_kernel replaces the last two when the count table is
//     small (E * chunks <= kFusedScanInts): each placing workgroup scans it.
// Chunks, waves, rounds and lanes follow slot order, so every expert's slots
// land in increasing slot order: the same permutation as block_permute.
// (from kPermMultiSlots slots on; chunks of about 1024 slots, perm_blocks)
constexpr int kPermWaves = 4;

// The slots [lo, hi) of this wave, counted per expert into cnt_w (LDS), or
// (place) placed at cnt_w[e] + rank, cnt_w then advancing.  Expert ids are
// loaded kPermBatch rounds at a time and the rounds processed in order.
template <bool PLACE>
__device__ __attribute__((always_inline)) inline void perm_wave_rounds(
    const int32_t* __restrict__ idx, int64_t lo, int64_t hi, int k, int E, int nbits, int* cnt_w,
    int32_t* sorted_slots, int32_t* slot_pos, int32_t* seg_tok, int32_t* tiles, const int* s_beg, const int* s_tb) {
  constexpr int kPermBatch = 8;
  const int lane = threadIdx.x % kWave;
  const uint64_t lt_mask = (1ull << lane) - 1ull;
  for (int64_t r0 = lo; r0 < hi; r0 += (int64_t)kPermBatch * kWave) {
    int ev[kPermBatch];
#pragma unroll
    for (int j = 0; j < kPermBatch; ++j) {
      const int64_t sl = r0 + (int64_t)j * kWave + lane;
      const int v = idx[sl < hi ? sl : hi - 1];
      ev[j] = sl < hi ? v : -1;
    }
#pragma unroll
    for (int j = 0; j < kPermBatch; ++j) {
      if (r0 + (int64_t)j * kWave >= hi) break;  // uniform
      const int64_t sl = r0 + (int64_t)j * kWave + lane;
      const int e = ev[j];
      const bool valid = (e >= 0 && e < E);
      const uint64_t m = match_expert(e, valid, nbits);
      const uint64_t below = m & lt_mask;
      if constexpr (PLACE) {
        if (valid) {
          const int pos = cnt_w[e] + __popcll(below);
          sorted_slots[pos] = (int32_t)sl;
          slot_pos[sl] = pos;
          if (seg_tok) seg_tok[pos] = (int32_t)(sl / k);
          if (tiles) {
            const int rel = pos - s_beg[e];
            tiles[(int64_t)(s_tb[e] + rel / 16) * kTileWords + 4 + rel % 16] = (int32_t)(sl / k);
          }
          // every lane of the group read the base before the leader bumps it
          if (below == 0) cnt_w[e] = cnt_w[e] + __popcll(m);
        } else if (sl < hi) {
          slot_pos[sl] = -1;
        }
      } else {
        if (valid && below == 0) cnt_w[e] += __popcll(m);
      }
    }
  }
}

__device__ inline int perm_nbits(int E) {
  int nbits = 1;
  while ((1 << nbits) < E) ++nbits;
  return nbits;
}

__global__ __launch_bounds__(kPermWaves * kWave) void permute_count_kernel(const int32_t* idx, int64_t n, int E,
                                                                           int64_t chunk, int32_t* cnt) {
  __shared__ int s_cnt[kPermWaves][kMaxExperts];
  const int w = threadIdx.x / kWave;
  const int nb = gridDim.x;
  for (int i = threadIdx.x; i < kPermWaves * kMaxExperts; i += blockDim.x) s_cnt[i / kMaxExperts][i % kMaxExperts] = 0;
  lds_barrier();
  const int64_t lo = (int64_t)blockIdx.x * chunk;
  const int64_t hi = lo + chunk < n ? lo + chunk : n;
  const int64_t wc = round_up(ceil_div(hi > lo ? hi - lo : 0, kPermWaves), kWave);
  const int64_t wlo = lo + w * wc;
  const int64_t whi = wlo + wc < hi ? wlo + wc : hi;
  perm_wave_rounds<false>(idx, wlo, whi, 0, E, perm_nbits(E), s_cnt[w], nullptr, nullptr, nullptr, nullptr, nullptr,
                          nullptr);
  lds_barrier();
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    int t = 0;
#pragma unroll
    for (int ww = 0; ww < kPermWaves; ++ww) t += s_cnt[ww][e];
    cnt[(int64_t)e * nb + blockIdx.x] = t;
  }
}

// One workgroup of 1024 threads.  Expert e is owned by a group of G
// consecutive threads (scan_group_size: 1024 / E rounded down to a power of
// two, at most 16, so a group never straddles a wave); thread j of the group
// takes the contiguous chunks [j per, j per + per) of cnt[e][*].  Its loads
// are issued together (held in registers up to kScanRun chunks), the expert
// total and the in-group prefix come from shuffles, and the scan over the
// experts runs on the group leaders.  (One thread per expert summing its
// chunks one dependent load at a time took 11 us at 32 chunks.)
constexpr int kScanRun = 8;

__device__ inline int scan_group_size(int E) {
  int g = 1;
  while (g < 16 && 2 * g * E <= 1024) g *= 2;
  return g;
}

__global__ __launch_bounds__(1024) void permute_scan_kernel(int64_t n, int64_t T, int E, int nb, int has_shared,
                                                            int32_t* cnt, int32_t* tb_out, int32_t* offsets,
                                                            int32_t* offsets_user, int32_t* active, int32_t* n_active,
                                                            int4* desc, int32_t* seg_tok, int32_t* tiles,
                                                            int32_t* n_tiles) {
  __shared__ int s_tmp[3 * 16];
  const int G = scan_group_size(E);
  const int lane = (int)threadIdx.x % kWave;
  const int e = (int)threadIdx.x / G;
  const int j = (int)threadIdx.x % G;
  const int gl = lane - j;  // the group leader's lane
  const bool own = e < E;
  const int per = (nb + G - 1) / G;
  const int b0 = j * per;
  const int b1 = b0 + per < nb ? b0 + per : nb;
  int32_t* ce = cnt + (int64_t)(own ? e : 0) * nb;
  int v[kScanRun];
  int part = 0;
  if (per <= kScanRun) {
#pragma unroll
    for (int i = 0; i < kScanRun; ++i) {
      const int x = ce[b0 + i < nb ? b0 + i : nb - 1];
      v[i] = (own && b0 + i < b1) ? x : 0;
    }
#pragma unroll
    for (int i = 0; i < kScanRun; ++i) part += v[i];
  } else if (own) {
    for (int b = b0; b < b1; ++b) part += ce[b];
  }
  int inc = part;
  for (int off = 1; off < G; off <<= 1) {
    const int t = __shfl_up(inc, off, kWave);
    if (j >= off) inc += t;
  }
  const int tot = __shfl(inc, gl + G - 1, kWave);
  const int pre = inc - part;  // this thread's chunks start here within expert e
  const bool lead = own && j == 0;
  int3 tot3;
  const int3 ex0 = block_exclusive_scan3(make_int3(lead ? tot : 0, (lead && tot > 0) ? 1 : 0,
                                                   lead ? (tot + 15) / 16 : 0), s_tmp, &tot3);
  const int total = tot3.x, total_act = tot3.y, total_tiles = tot3.z;
  const int run = __shfl(ex0.x, gl, kWave);
  const int ex_act = __shfl(ex0.y, gl, kWave);
  const int ex_tile = __shfl(ex0.z, gl, kWave);
  if (own) {
    if (j == 0) {
      offsets[e] = run;
      if (offsets_user) offsets_user[e] = run;
      if (tot > 0) {
        active[ex_act] = e;
        if (desc) desc[ex_act] = make_int4(e, run, run + tot, 0);
      }
      if (tb_out) tb_out[e] = ex_tile;
    }
    if (tiles) {
      const int ntl = (tot + 15) / 16;
      for (int t = j; t < ntl; t += G)
        *reinterpret_cast<int4*>(tiles + (int64_t)(ex_tile + t) * kTileWords) = make_int4(e, run + 16 * t, run + tot, 0);
    }
    // chunk bases of expert e, in chunk order
    int base = run + pre;
    if (per <= kScanRun) {
#pragma unroll
      for (int i = 0; i < kScanRun; ++i) {
        if (b0 + i < b1) {
          ce[b0 + i] = base;
          base += v[i];
        }
      }
    } else {
      for (int b = b0; b < b1; ++b) {
        const int x = ce[b];
        ce[b] = base;
        base += x;
      }
    }
  }
  if (threadIdx.x == 0) {
    offsets[E] = total;
    if (offsets_user) offsets_user[E] = total;
    offsets[E + 1] = total + (has_shared ? (int)T : 0);
    if (has_shared) {
      active[total_act] = E;
      if (desc) desc[total_act] = make_int4(E, total, total + (int)T, 0);
    }
    *n_active = total_act + (has_shared ? 1 : 0);
  }
  if (has_shared && seg_tok) {
    for (int64_t t = threadIdx.x; t < T; t += blockDim.x) seg_tok[n + t] = (int32_t)t;
  }
  if (tiles) {
    const int64_t n_sh = has_shared ? (T + 15) / 16 : 0;
    for (int64_t j = threadIdx.x; j < n_sh; j += blockDim.x) {
      int32_t* tw = tiles + (total_tiles + j) * kTileWords;
      *reinterpret_cast<int4*>(tw) = make_int4(E, total + (int)(16 * j), total + (int)T, 0);
      for (int jj = 0; jj < 16 && 16 * j + jj < T; ++jj) tw[4 + jj] = (int32_t)(16 * j + jj);
    }
    if (threadIdx.x == 0) {
      n_tiles[0] = total_tiles + (int)n_sh;
    }
  }
  if (desc) {
    const int n_act = total_act + (has_shared ? 1 : 0);
    const int max_active = (int)((n < E) ? n : E) + (has_shared ? 1 : 0);
    for (int u = n_act + threadIdx.x; u < max_active; u += blockDim.x) desc[u] = make_int4(-1, 0, 0, 0);
  }
}

__global__ __launch_bounds__(kPermWaves * kWave) void permute_place_kernel(const int32_t* idx, int64_t n, int k, int E,
                                                                           int64_t chunk, const int32_t* cnt,
                                                                           const int32_t* offsets, const int32_t* tb,
                                                                           int32_t* sorted_slots, int32_t* slot_pos,
                                                                           int32_t* seg_tok, int32_t* tiles) {
  __shared__ int s_cnt[kPermWaves][kMaxExperts];
  __shared__ int s_beg[kMaxExperts];
  __shared__ int s_tb[kMaxExperts];
  const int w = threadIdx.x / kWave;
  const int nb = gridDim.x;
  const int nbits = perm_nbits(E);
  for (int i = threadIdx.x; i < kPermWaves * kMaxExperts; i += blockDim.x) s_cnt[i / kMaxExperts][i % kMaxExperts] = 0;
  lds_barrier();
  const int64_t lo = (int64_t)blockIdx.x * chunk;
  const int64_t hi = lo + chunk < n ? lo + chunk : n;
  const int64_t wc = round_up(ceil_div(hi > lo ? hi - lo : 0, kPermWaves), kWave);
  const int64_t wlo = lo + w * wc;
  const int64_t whi = wlo + wc < hi ? wlo + wc : hi;
  perm_wave_rounds<false>(idx, wlo, whi, 0, E, nbits, s_cnt[w], nullptr, nullptr, nullptr, nullptr, nullptr, nullptr);
  lds_barrier();
  // per-wave bases: the chunk's base plus the counts of earlier waves
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    int b = cnt[(int64_t)e * nb + blockIdx.x];
#pragma unroll
    for (int ww = 0; ww < kPermWaves; ++ww) {
      const int c = s_cnt[ww][e];
      s_cnt[ww][e] = b;
      b += c;
    }
    if (tiles) {
      s_beg[e] = offsets[e];
      s_tb[e] = tb[e];
    }
  }
  lds_barrier();
  perm_wave_rounds<true>(idx, wlo, whi, k, E, nbits, s_cnt[w], sorted_slots, slot_pos, seg_tok, tiles, s_beg, s_tb);
}

// Placement with the scan folded in, when the per-block counts are few
// (E * nb <= kFusedScanInts): every workgroup copies the whole count table
// into LDS, forms the segment offsets, active experts and token-tile bases
// (the exclusive scan of block_permute) and its own per-expert bases (the
// counts of the blocks before it), then places its chunk as
// permute_place_kernel does.  Workgroup 0 also writes what the scan launch
// writes: offsets, active experts, descriptors, tile headers and count; the
// shared segment's tokens are spread over all workgroups.  This saves the
// single-workgroup scan launch and its wait between count and place.
constexpr int kFusedScanInts = 8192;

__global__ __launch_bounds__(kPermWaves * kWave) void permute_scan_place_kernel(
    const int32_t* idx, int64_t n, int64_t T, int k, int E, int has_shared, int64_t chunk, const int32_t* cnt,
    int32_t* offsets, int32_t* offsets_user, int32_t* active, int32_t* n_active, int4* desc, int32_t* sorted_slots,
    int32_t* slot_pos, int32_t* seg_tok, int32_t* tiles, int32_t* n_tiles) {
  __shared__ int s_all[kFusedScanInts];  // cnt[e * nb + b]
  __shared__ int s_cnt[kPermWaves][kMaxExperts];
  __shared__ int s_beg[kMaxExperts];
  __shared__ int s_tb[kMaxExperts];
  __shared__ int s_tmp[3 * kPermWaves];
  const int tid = threadIdx.x;
  const int w = tid / kWave;
  const int nb = gridDim.x;
  const int blk = blockIdx.x;
  const int nbits = perm_nbits(E);
  for (int i = tid; i < kPermWaves * kMaxExperts; i += blockDim.x) s_cnt[i / kMaxExperts][i % kMaxExperts] = 0;
  // the count table's loads are all issued first (clamped indices) and land
  // while the chunk's expert ids are loaded and counted
  const int ncnt = E * nb;
  constexpr int kRun = kFusedScanInts / (kPermWaves * kWave);
  int v[kRun];
#pragma unroll
  for (int j = 0; j < kRun; ++j) {
    const int i = j * kPermWaves * kWave + tid;
    v[j] = cnt[i < ncnt ? i : ncnt - 1];
  }
  lds_barrier();
  const int64_t lo = (int64_t)blk * chunk;
  const int64_t hi = lo + chunk < n ? lo + chunk : n;
  const int64_t wc = round_up(ceil_div(hi > lo ? hi - lo : 0, kPermWaves), kWave);
  const int64_t wlo = lo + w * wc;
  const int64_t whi = wlo + wc < hi ? wlo + wc : hi;
  perm_wave_rounds<false>(idx, wlo, whi, 0, E, nbits, s_cnt[w], nullptr, nullptr, nullptr, nullptr, nullptr, nullptr);
#pragma unroll
  for (int j = 0; j < kRun; ++j) {
    const int i = j * kPermWaves * kWave + tid;
    if (i < ncnt) s_all[i] = v[j];
  }
  lds_barrier();
  // Scan over experts: thread t owns experts t kPer .. t kPer + kPer - 1.
  constexpr int kPer = kMaxExperts / (kPermWaves * kWave);
  int tot[kPer], pre[kPer];
  int my_tot = 0, my_act = 0, my_tc = 0;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int e = tid * kPer + i;
    int t = 0, p = 0;
    if (e < E) {
      // eight independent LDS reads at a time, not one dependent read per block
      const int* ce = s_all + e * nb;
      for (int b0 = 0; b0 < nb; b0 += 8) {
        int c[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) c[j] = b0 + j < nb ? ce[b0 + j] : 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          t += c[j];
          p += b0 + j < blk ? c[j] : 0;
        }
      }
    }
    tot[i] = t;
    pre[i] = p;
    my_tot += t;
    my_act += t > 0 ? 1 : 0;
    my_tc += (t + 15) / 16;
  }
  int3 tot3;
  const int3 ex3 = block_exclusive_scan3(make_int3(my_tot, my_act, my_tc), s_tmp, &tot3);  // has barriers
  const int total = tot3.x, total_act = tot3.y, total_tiles = tot3.z;
  int run = ex3.x, arun = ex3.y, trun = ex3.z;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int e = tid * kPer + i;
    if (e < E) {
      s_beg[e] = run;
      s_tb[e] = trun;
      if (blk == 0) {
        offsets[e] = run;
        if (offsets_user) offsets_user[e] = run;
        if (tot[i] > 0) {
          active[arun] = e;
          if (desc) desc[arun] = make_int4(e, run, run + tot[i], 0);
        }
        if (tiles)
          for (int j = 0; j < (tot[i] + 15) / 16; ++j)
            *reinterpret_cast<int4*>(tiles + (int64_t)(trun + j) * kTileWords) =
                make_int4(e, run + 16 * j, run + tot[i], 0);
      }
      // this block's waves place expert e from here on, in wave order
      int b = run + pre[i];
      for (int ww = 0; ww < kPermWaves; ++ww) {
        const int c = s_cnt[ww][e];
        s_cnt[ww][e] = b;
        b += c;
      }
    }
    run += tot[i];
    arun += tot[i] > 0 ? 1 : 0;
    trun += (tot[i] + 15) / 16;
  }
  if (blk == 0) {
    if (tid == 0) {
      offsets[E] = total;
      if (offsets_user) offsets_user[E] = total;
      offsets[E + 1] = total + (has_shared ? (int)T : 0);
      if (has_shared) {
        active[total_act] = E;
        if (desc) desc[total_act] = make_int4(E, total, total + (int)T, 0);
      }
      *n_active = total_act + (has_shared ? 1 : 0);
      if (tiles) n_tiles[0] = total_tiles + (has_shared ? (int)((T + 15) / 16) : 0);
    }
    if (desc) {
      const int n_act = total_act + (has_shared ? 1 : 0);
      const int max_active = (int)((n < E) ? n : E) + (has_shared ? 1 : 0);
      for (int u = n_act + tid; u < max_active; u += blockDim.x) desc[u] = make_int4(-1, 0, 0, 0);
    }
  }
  if (has_shared && seg_tok)
    for (int64_t t = (int64_t)blk * blockDim.x + tid; t < T; t += (int64_t)nb * blockDim.x) seg_tok[n + t] = (int32_t)t;
  if (has_shared && tiles) {
    for (int64_t j = (int64_t)blk * blockDim.x + tid; j < (T + 15) / 16; j += (int64_t)nb * blockDim.x) {
      int32_t* tw = tiles + (total_tiles + j) * kTileWords;
      *reinterpret_cast<int4*>(tw) = make_int4(E, total + (int)(16 * j), total + (int)T, 0);
      for (int jj = 0; jj < 16 && 16 * j + jj < T; ++jj) tw[4 + jj] = (int32_t)(16 * j + jj);
    }
  }
  lds_barrier();
  perm_wave_rounds<true>(idx, wlo, whi, k, E, nbits, s_cnt[w], sorted_slots, slot_pos, seg_tok, tiles, s_beg, s_tb);
}

// Count, then the fused scan and placement (few blocks) or the scan and
// placement launches; cnt needs E * perm_blocks(T * k) ints, tb E ints.
static hipError_t launch_permute_multi(const int32_t* idx, int64_t T, int k, int E, int has_shared,
                                       int32_t* offsets, int32_t* offsets_user, int32_t* active, int32_t* n_active,
                                       int32_t* sorted_slots, int32_t* slot_pos, int4* desc, int32_t* seg_tok,
                                       int32_t* tiles, int32_t* n_tiles, int32_t* cnt,
                                       int32_t* tb, hipStream_t stream, bool counted = false) {
  const int64_t n = T * k;
  const int64_t nb = perm_blocks(n);
  const int64_t chunk = ceil_div(n, nb);
  if (!counted)
    hipLaunchKernelGGL(permute_count_kernel, dim3((unsigned)nb), dim3(kPermWaves * kWave), 0, stream, idx, n, E,
                       chunk, cnt);
  if ((int64_t)E * nb <= kFusedScanInts) {
    hipLaunchKernelGGL(permute_scan_place_kernel, dim3((unsigned)nb), dim3(kPermWaves * kWave), 0, stream, idx, n, T,
                       k, E, has_shared, chunk, cnt, offsets, offsets_user, active, n_active, desc, sorted_slots,
                       slot_pos, seg_tok, tiles, n_tiles);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(permute_scan_kernel, dim3(1), dim3(1024), 0, stream, n, T, E, (int)nb, has_shared, cnt, tb,
                     offsets, offsets_user, active, n_active, desc, seg_tok, tiles, n_tiles);
  hipLaunchKernelGGL(permute_place_kernel, dim3((unsigned)nb), dim3(kPermWaves * kWave), 0, stream, idx, n, k, E,
                     chunk, cnt, offsets, tb, sorted_slots, slot_pos, seg_tok, tiles);
  return hipGetLastError();
}

// Tokens per logits wave.  Small tiles give the grid more workgroups to
// stream W with, large ones re-read W less.  Measured routes (us), tiles of
// 1 / 2 / 4 tokens: DeepSeek-V3 8 tokens 22.5 / 24.8 / 29.7, Mixtral 16
// tokens 15.6 / 18.7 / 22.2, Qwen3 32 tokens 21.8 / 17.7 / 19.7 (with
// batches of eight chunks).  At 64 tokens of DeepSeek-V3 (H 7168, E 256)
// four tokens with batches of four chunks take 32.7 against 40.8 us for two
// tokens; eight tokens a wave took 35.0.
int router_token_tile(int64_t T) {
  if (T <= 16) return 1;
  if (T <= 32) return 2;
  if (T <= 64) return 4;
  return kBigTT;
}

template <typename XT>
static hipError_t launch_logits_t(const RouteK& k, int TT, int n_ttiles, hipStream_t stream) {
  if (TT == 1) {
    dim3 grid((unsigned)ceil_div(k.E, 4 * 1), (unsigned)n_ttiles);
    hipLaunchKernelGGL((route_logits_kernel<XT, 1, 1, 8>), grid, dim3(256), 0, stream, k);
  } else if (TT == 2) {
    dim3 grid((unsigned)ceil_div(k.E, 4 * 2), (unsigned)n_ttiles);
    hipLaunchKernelGGL((route_logits_kernel<XT, 2, 2, 8>), grid, dim3(256), 0, stream, k);
  } else if (TT == 4) {
    // batches of four chunks: with eight the bf16 kernel needs 256 registers
    // (one wave a SIMD) and the 64-token route took 43.4 us, with four 203
    dim3 grid((unsigned)ceil_div(k.E, 4 * 2), (unsigned)n_ttiles);
    hipLaunchKernelGGL((route_logits_kernel<XT, 4, 2, 4>), grid, dim3(256), 0, stream, k);
  } else {
    dim3 grid((unsigned)ceil_div(k.E, 4 * kBigEW), (unsigned)n_ttiles);
    hipLaunchKernelGGL((route_logits_big_kernel<XT, kBigTT, kBigEW>), grid, dim3(256), 0, stream, k);
  }
  return hipGetLastError();
}

// The two-pass router (approximate logits, candidates, exact candidate
// logits, then the usual selection) from this many bf16 tokens on (E >= 16).
static hipError_t launch_route_two_pass(const RouteK& k, const Workspace& ws, hipStream_t stream) {
  float* approx = ws.approx;
  float* nx = approx + k.T * k.E;
  float* nw = nx + k.T;
  hipLaunchKernelGGL(route_approx_kernel, dim3((unsigned)(ceil_div(k.E, kApproxExp) * ceil_div(k.T, kApproxTok))),
                     dim3(256), 0, stream, k, approx, nx, nw);
  const dim3 grid((unsigned)ceil_div(k.T, 4)), block(512);  // 4 candidate waves + 4 copying x
  if (k.E <= 64) hipLaunchKernelGGL(route_candidates_kernel<1>, grid, block, 0, stream, k, approx, nx, nw, ws.cand);
  else if (k.E <= 128) hipLaunchKernelGGL(route_candidates_kernel<2>, grid, block, 0, stream, k, approx, nx, nw, ws.cand);
  else if (k.E <= 256) hipLaunchKernelGGL(route_candidates_kernel<4>, grid, block, 0, stream, k, approx, nx, nw, ws.cand);
  else hipLaunchKernelGGL(route_candidates_kernel<8>, grid, block, 0, stream, k, approx, nx, nw, ws.cand);
  hipLaunchKernelGGL(route_exact_kernel, dim3((unsigned)ceil_div(k.T, kExactTok), (unsigned)k.E), dim3(256), 0, stream,
                     k, static_cast<const uint8_t*>(ws.cand));
  return hipGetLastError();
}

hipError_t launch_route(const RouteArgs& r, const Workspace& ws, hipStream_t stream) {
  RouteK k;
  k.x = r.x;
  k.W = r.router_w;
  k.bias = r.router_bias;
  k.T = r.T;
  k.H = r.H;
  k.E = r.E;
  k.k = r.k;
  k.score_mode = r.score_mode;
  k.topk_idx = r.topk_idx;
  k.topk_w = r.topk_w;
  k.logits = ws.logits;
  const int TT = router_token_tile(r.T);
  const int n_ttiles = (int)ceil_div(r.T, TT);
  k.xq = ws.xq;
  k.xs = ws.xs;
  k.Kq = ceil_div(r.H, kQuad);
  k.prep_x = r.prep_x ? 1 : 0;
  k.prep_fp16 = r.prep_fp16 ? 1 : 0;
  k.do_permute = r.do_permute ? 1 : 0;
  k.has_shared = r.has_shared;
  k.offsets = ws.offsets;
  k.offsets_user = r.offsets_out;
  k.active = ws.active;
  k.n_active = ws.n_active;
  k.sorted_slots = r.sorted_slots_out ? r.sorted_slots_out : ws.sorted_slots;
  k.slot_pos = r.slot_pos_out ? r.slot_pos_out : ws.slot_pos;
  k.desc = r.do_permute ? ws.desc : nullptr;
  k.seg_tok = r.do_permute ? ws.seg_tok : nullptr;
  // the token tiles feed the token-tile gate/up kernel only
  const bool want_tiles = r.do_permute && r.want_tiles;
  k.tiles = want_tiles ? ws.tiles : nullptr;
  k.n_tiles = want_tiles ? ws.n_tiles : nullptr;
  const unsigned sel_blocks = (unsigned)ceil_div(r.T, kSelectWaves);
  k.fuse_permute = (r.do_permute && sel_blocks > 1 && sel_blocks <= kFusedSelectBlocks) ? 1 : 0;
  k.counter = k.fuse_permute ? ws.counter : nullptr;
  const bool two_pass = two_pass_route(r.T, r.E, r.x_dtype) && ws.approx && ws.cand && !k.fuse_permute;
  // With two passes and a fused scan the select launch does the permute's
  // counting (the approximate-logit launch zeroes the counts first).
  const int64_t n_slots = r.T * r.k;
  const bool sel_count = two_pass && r.do_permute && sel_blocks > 1 && n_slots >= kPermMultiSlots &&
                         (int64_t)r.E * perm_blocks(n_slots) <= kFusedScanInts;
  k.perm_cnt = sel_count ? ws.perm_cnt : nullptr;
  k.perm_nb = (int)perm_blocks(n_slots);
  k.perm_chunk = ceil_div(n_slots, perm_blocks(n_slots));
  hipError_t err = two_pass
                       ? launch_route_two_pass(k, ws, stream)
                       : ((r.x_dtype == 0) ? launch_logits_t<uint16_t>(k, TT, n_ttiles, stream)
                                           : launch_logits_t<float>(k, TT, n_ttiles, stream));
  if (err != hipSuccess) return err;
  // One wave per token, four tokens per workgroup, so selection is spread
  // over many CUs.  The permute runs in the select launch up to
  // kFusedSelectBlocks workgroups, in its own single-workgroup launch beyond.
  const dim3 sb(kWave * kSelectWaves);
  if (r.E <= 64) hipLaunchKernelGGL(route_select_kernel<1>, dim3(sel_blocks), sb, 0, stream, k);
  else if (r.E <= 128) hipLaunchKernelGGL(route_select_kernel<2>, dim3(sel_blocks), sb, 0, stream, k);
  else if (r.E <= 256) hipLaunchKernelGGL(route_select_kernel<4>, dim3(sel_blocks), sb, 0, stream, k);
  else hipLaunchKernelGGL(route_select_kernel<8>, dim3(sel_blocks), sb, 0, stream, k);
  err = hipGetLastError();
  if (err != hipSuccess || !r.do_permute || sel_blocks == 1 || k.fuse_permute) return err;
  if (r.T * r.k >= kPermMultiSlots)
    return launch_permute_multi(k.topk_idx, r.T, r.k, r.E, r.has_shared, ws.offsets, r.offsets_out, ws.active,
                                ws.n_active, k.sorted_slots, k.slot_pos, k.desc, k.seg_tok, k.tiles, k.n_tiles,
                                ws.perm_cnt, ws.perm_tb, stream, sel_count);
  hipLaunchKernelGGL(permute_kernel, dim3(1), dim3(1024), 0, stream, k.topk_idx, r.T, r.k,
              r.E, r.has_shared, ws.offsets, r.offsets_out, ws.active, ws.n_active, k.sorted_slots, k.slot_pos,
              k.desc, k.seg_tok, k.tiles, k.n_tiles);
  return hipGetLastError();
}

hipError_t launch_permute(const int32_t* topk_idx, int64_t T, int k, int E, int has_shared,
                          int32_t* offsets, int32_t* sorted_slots, int32_t* slot_pos,
                          const Workspace& ws, hipStream_t stream) {
  if (T * k >= kPermMultiSlots)
    return launch_permute_multi(topk_idx, T, k, E, has_shared, ws.offsets, offsets, ws.active, ws.n_active,
                                sorted_slots, slot_pos, nullptr, nullptr, nullptr, nullptr, ws.perm_cnt,
                                ws.perm_tb, stream);
  hipLaunchKernelGGL(permute_kernel, dim3(1), dim3(1024), 0, stream, topk_idx, T, k, E, has_shared,
                     ws.offsets, offsets, ws.active, ws.n_active, sorted_slots, slot_pos,
                     static_cast<int4*>(nullptr), static_cast<int32_t*>(nullptr), static_cast<int32_t*>(nullptr),
                     static_cast<int32_t*>(nullptr));
  return hipGetLastError();
}

}  // namespace pmoe
