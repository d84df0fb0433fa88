// router.hip -- fused MoE router for gfx950: gate GEMV (fp64, fixed order),
// top-k selection, softmax / sigmoid weights, and the stable expert permute,
// in one launch.
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
// Launches.  route_logits_kernel computes logits (and the MFMA-ordered copy
// of x) with no inter-workgroup communication.  route_select_kernel gives one
// wave per token: k rounds of a wave-wide arg-max over (logit desc, index
// asc), then the weights.  When the whole batch fits one workgroup (decode),
// the same workgroup then runs the permute; otherwise permute_kernel does.
// No device-scope fences anywhere: on a multi-XCD part an agent-scope release
// writes back the XCD's L2, which costs microseconds per workgroup.
// Permute: per-wave expert counts, an (expert, wave)-major exclusive scan, and
// a second pass that places every slot at base + rank-within-round, where the
// rank comes from ballots over the bits of the expert id.  Placement depends
// only on slot order, never on atomics, so the permutation is deterministic
// and stable.
#include <float.h>
#include <math.h>

#include "moe_common.h"
#include "moe_launch.h"

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
};

__device__ inline bool ranks_before(double va, int ia, double vb, int ib) {
  const bool na = isnan(va), nb = isnan(vb);
  if (na || nb) return (na && nb) ? (ia < ib) : nb;
  return (va > vb) || (va == vb && ia < ib);
}

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

// Block-wide exclusive scan for 256 threads.  Returns the exclusive prefix and
// writes the block total to *total.
__device__ inline int block_exclusive_scan(int v, int* s_tmp, int* total) {
  const int lane = threadIdx.x % kWave;
  const int w = threadIdx.x / kWave;
  int inc = v;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int n = __shfl_up(inc, off, kWave);
    if (lane >= off) inc += n;
  }
  if (lane == kWave - 1) s_tmp[w] = inc;
  __syncthreads();
  int prefix = 0, tot = 0;
  for (int i = 0; i < (int)(blockDim.x / kWave); ++i) {
    if (i < w) prefix += s_tmp[i];
    tot += s_tmp[i];
  }
  __syncthreads();
  *total = tot;
  return prefix + inc - v;
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
// expert last, covering positions [T*k, T*k + T)) and the token of every
// segment position.
__device__ void block_permute(const int32_t* __restrict__ idx, int64_t n, int k, int E, int64_t T,
                              int has_shared, int32_t* offsets, int32_t* offsets_user,
                              int32_t* active, int32_t* n_active, int32_t* sorted_slots,
                              int32_t* slot_pos, int4* desc, int32_t* seg_tok) {
  constexpr int kMaxWaves = 16;
  __shared__ int s_cnt[kMaxWaves][kMaxExperts];
  __shared__ int s_tmp[kMaxWaves];
  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int w = tid / kWave;
  const int NW = blockDim.x / kWave;
  int nbits = 1;
  while ((1 << nbits) < E) ++nbits;

  for (int i = tid; i < NW * kMaxExperts; i += blockDim.x) s_cnt[i / kMaxExperts][i % kMaxExperts] = 0;
  __syncthreads();

  const int64_t chunk = round_up(ceil_div(n, NW), kWave);
  const int64_t beg = w * chunk;
  const int64_t end = (beg + chunk < n) ? beg + chunk : n;

  // Pass 1: per-wave counts.
  for (int64_t r0 = beg; r0 < end; r0 += kWave) {
    const int64_t s = r0 + lane;
    int e = (s < end) ? idx[s] : -1;
    const bool valid = (e >= 0 && e < E);
    const uint64_t m = match_expert(e, valid, nbits);
    if (valid) {
      const uint64_t below = m & ((1ull << lane) - 1ull);
      if (below == 0) s_cnt[w][e] += __popcll(m);
    }
  }
  __syncthreads();

  // Scan over experts: thread t owns experts t, t + blockDim, ... (at most
  // kMaxExperts / 256 = 2 per thread for 256 threads).
  constexpr int kPer = kMaxExperts / 256;
  int tot[kPer], act[kPer];
  int my_tot = 0, my_act = 0;
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
  int total = 0, total_act = 0;
  const int ex = block_exclusive_scan(my_tot, s_tmp, &total);
  const int ax = block_exclusive_scan(my_act, s_tmp, &total_act);
  int run = ex, arun = ax;
  for (int i = 0; i < kPer; ++i) {
    const int e = tid * kPer + i;
    if (e < E) {
      offsets[e] = run;
      if (offsets_user) offsets_user[e] = run;
      if (act[i]) {
        active[arun] = e;
        if (desc) desc[arun] = make_int4(e, run, run + tot[i], 0);
      }
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
  if (desc) {
    // unused slots up to the launch bound min(E, n) + shared carry expert -1
    const int n_act = total_act + (has_shared ? 1 : 0);
    const int max_active = (int)((n < E) ? n : E) + (has_shared ? 1 : 0);
    for (int u = n_act + tid; u < max_active; u += blockDim.x) desc[u] = make_int4(-1, 0, 0, 0);
  }
  __syncthreads();

  // Pass 2: placement.
  for (int64_t r0 = beg; r0 < end; r0 += kWave) {
    const int64_t s = r0 + lane;
    int e = (s < end) ? idx[s] : -1;
    const bool valid = (e >= 0 && e < E);
    const uint64_t m = match_expert(e, valid, nbits);
    if (valid) {
      const uint64_t below = m & ((1ull << lane) - 1ull);
      const int pos = s_cnt[w][e] + __popcll(below);
      sorted_slots[pos] = (int32_t)s;
      slot_pos[s] = pos;
      if (seg_tok) seg_tok[pos] = (int32_t)(s / k);
      // Every lane of the group has read the base before the leader bumps
      // it: LDS operations of one wave complete in program order, and the
      // read above precedes this write in every lane's program.
      if (below == 0) s_cnt[w][e] = s_cnt[w][e] + __popcll(m);
    } else if (s < end) {
      slot_pos[s] = -1;
    }
  }
}

// Order-preserving integer key of a logit: a > b (as numbers) iff
// key(a) > key(b), -0.0 and +0.0 share a key, and NaN maps to 0, below every
// number, so equal keys are exactly the ties the oracle breaks by index.
__device__ inline uint64_t logit_key(double v) {
  if (isnan(v)) return 0ull;
  if (v == 0.0) v = 0.0;  // -0.0 -> +0.0
  const uint64_t b = __builtin_bit_cast(uint64_t, v);
  return (b >> 63) ? ~b : (b | 0x8000000000000000ull);
}

// Top-k of one token by rank counting (called by all 64 lanes of one wave).
// The token's E keys sit in LDS; lane l ranks experts l, l + 64, ...:
// rank(e) = #{e' : key(e') > key(e) or (key(e') == key(e) and e' < e)}, which
// is e's position in (value desc, index asc) order.  Experts of rank < k are
// written straight to their slot.  No cross-lane dependency chains: each
// comparison reads a broadcast LDS word.
template <int NV>
__device__ void wave_topk(const RouteK& a, int64_t t, uint64_t* s_key, double* s_val, int* s_idx,
                          double* s_e) {
  const int lane = threadIdx.x % kWave;
  for (int e = lane; e < a.E; e += kWave) s_key[e] = logit_key(a.logits[t * a.E + e]);
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  uint64_t mine[NV];
  int rank[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int e = lane + kWave * v;
    mine[v] = e < a.E ? s_key[e] : 0ull;
    rank[v] = 0;
  }
  for (int e2 = 0; e2 < a.E; ++e2) {
    const uint64_t k2 = s_key[e2];
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const int e = lane + kWave * v;
      rank[v] += (k2 > mine[v] || (k2 == mine[v] && e2 < e)) ? 1 : 0;
    }
  }
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int e = lane + kWave * v;
    if (e < a.E && rank[v] < a.k) {
      s_idx[rank[v]] = e;
      s_val[rank[v]] = a.logits[t * a.E + e];
    }
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  // Weights: lane i (< k) owns slot i; every lane sums the k terms in slot
  // order, so the normaliser is the same sequential fp64 sum as the oracle's.
  double ej = 0.0;
  if (lane < a.k) {
    const double v = s_val[lane];
    ej = (a.score_mode == 0) ? exp(v - s_val[0]) : 1.0 / (1.0 + exp(-v));
    s_e[lane] = ej;
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  if (lane < a.k) {
    double sum = 0.0;
    for (int i = 0; i < a.k; ++i) sum += s_e[i];
    a.topk_idx[t * a.k + lane] = s_idx[lane];
    a.topk_w[t * a.k + lane] = (float)(ej / sum);
  }
  __builtin_amdgcn_wave_barrier();
}

// MFMA-ordered copy of x (bf16) and fp32 group sums for tokens [t0, t0+TT).
// Layout [t][q][p][gi][8]: one 16-byte chunk per (token, quad, part, group).
__device__ void prep_x_tile(const RouteK& a, int64_t t0, int TT) {
  const uint16_t* x = static_cast<const uint16_t*>(a.x);
  const int Kg = (int)(a.H / kGroup);
  const int per_tok = (int)a.Kq * 16;
  for (int ti = 0; ti < TT; ++ti) {
    const int64_t t = t0 + ti;
    if (t >= a.T) break;
    const uint16_t* xt = x + t * a.H;
    for (int c = threadIdx.x; c < per_tok; c += blockDim.x) {
      const int gi = c & 3;
      const int p = (c >> 2) & 3;
      const int q = c >> 4;
      const int g = 4 * q + gi;
      uint32_t wds[4] = {0, 0, 0, 0};
      if (g < Kg) {
        const uint16_t* xr = xt + g * kGroup;
        for (int j = 0; j < 8; j += 2) wds[j / 2] = (uint32_t)xr[kmap(p, j)] | ((uint32_t)xr[kmap(p, j + 1)] << 16);
      }
      u32x4 v = {wds[0], wds[1], wds[2], wds[3]};
      *reinterpret_cast<u32x4*>(a.xq + (t * a.Kq * 16 + c) * 8) = v;
    }
    const int ng = (int)a.Kq * 4;
    for (int g = threadIdx.x; g < ng; g += blockDim.x) {
      float sum = 0.0f;
      if (g < Kg) {
        const uint32_t* xr = reinterpret_cast<const uint32_t*>(xt + g * kGroup);
        for (int j = 0; j < kGroup / 2; ++j) {
          const uint32_t two = xr[j];
          sum += bf16_bits_to_float(two & 0xffffu);
          sum += bf16_bits_to_float(two >> 16);
        }
      }
      a.xs[t * ng + g] = sum;
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

  double acc[P];
#pragma unroll
  for (int i = 0; i < P; ++i) acc[i] = 0.0;

  // Chunks are loaded CB at a time (all loads of a batch issued before its
  // FMAs), then accumulated in increasing h as the contract requires.
  const int64_t nchunks = ceil_div(a.H, 256);
  for (int64_t c0 = 0; c0 < nchunks; c0 += CB) {
    float wv[CB][EW][4];
    float xv[CB][TT][4];
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
      const int64_t h0 = (c0 + cb) * 256 + 4 * lane;
      const bool hok = (c0 + cb) < nchunks && h0 < a.H;
#pragma unroll
      for (int ei = 0; ei < EW; ++ei) {
        const int e = e0 + ei;
        if (hok && e < a.E) {
          const float4 r = *reinterpret_cast<const float4*>(a.W + (int64_t)e * a.H + h0);
          wv[cb][ei][0] = r.x;
          wv[cb][ei][1] = r.y;
          wv[cb][ei][2] = r.z;
          wv[cb][ei][3] = r.w;
        } else {
          wv[cb][ei][0] = wv[cb][ei][1] = wv[cb][ei][2] = wv[cb][ei][3] = 0.0f;
        }
      }
#pragma unroll
      for (int ti = 0; ti < TT; ++ti) {
        const int64_t t = t0 + ti;
        if (hok && t < a.T) {
          load_x4<XT>(x, t * a.H + h0, xv[cb][ti]);
        } else {
          xv[cb][ti][0] = xv[cb][ti][1] = xv[cb][ti][2] = xv[cb][ti][3] = 0.0f;
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
        if (a.bias) v = v + (double)a.bias[e];
        a.logits[t * a.E + e] = v;
      }
    }
  }

  if (a.prep_x && blockIdx.x == 0) prep_x_tile(a, t0, TT);
  if (a.prep_x && blockIdx.x == 1 % gridDim.x && blockIdx.y == 0) {
    // all-zero activation row T, read by expert lanes past a segment
    for (int64_t i = threadIdx.x; i < a.Kq * 128; i += blockDim.x) a.xq[a.T * a.Kq * 128 + i] = 0;
    for (int64_t i = threadIdx.x; i < a.Kq * 4; i += blockDim.x) a.xs[a.T * a.Kq * 4 + i] = 0.0f;
  }
}

// Top-k and weights, one wave per token (grid-stride); a launch with one
// workgroup continues with the permute.
constexpr int kSelectWaves = 4;

template <int NV>
__global__ __launch_bounds__(256) void route_select_kernel(RouteK a) {
  __shared__ uint64_t s_key[kSelectWaves][kMaxExperts];
  __shared__ double s_val[kSelectWaves][kMaxTopK];
  __shared__ double s_e[kSelectWaves][kMaxTopK];
  __shared__ int s_idx[kSelectWaves][kMaxTopK];
  const int w = threadIdx.x / kWave;
  const int nw = blockDim.x / kWave;
  for (int64_t t = (int64_t)blockIdx.x * nw + w; t < a.T; t += (int64_t)gridDim.x * nw)
    wave_topk<NV>(a, t, s_key[w], s_val[w], s_idx[w], s_e[w]);
  if (!a.do_permute || gridDim.x != 1) return;
  __syncthreads();
  block_permute(a.topk_idx, a.T * a.k, a.k, a.E, a.T, a.has_shared, a.offsets, a.offsets_user, a.active,
                a.n_active, a.sorted_slots, a.slot_pos, a.desc, a.seg_tok);
}

__global__ __launch_bounds__(1024) void permute_kernel(const int32_t* idx, int64_t T, int k, int E,
                                                       int has_shared, int32_t* offsets,
                                                       int32_t* offsets_user, int32_t* active,
                                                       int32_t* n_active, int32_t* sorted_slots,
                                                       int32_t* slot_pos, int4* desc,
                                                       int32_t* seg_tok) {
  block_permute(idx, T * k, k, E, T, has_shared, offsets, offsets_user, active, n_active,
                sorted_slots, slot_pos, desc, seg_tok);
}

int router_token_tile(int64_t T) {
  if (T <= 1) return 1;
  if (T <= 64) return 4;
  return 16;
}

template <typename XT>
static hipError_t launch_logits_t(const RouteK& k, int TT, int n_ttiles, hipStream_t stream) {
  if (TT == 1) {
    dim3 grid((unsigned)ceil_div(k.E, 4 * 1), (unsigned)n_ttiles);
    hipLaunchKernelGGL((route_logits_kernel<XT, 1, 1, 8>), grid, dim3(256), 0, stream, k);
  } else if (TT == 4) {
    dim3 grid((unsigned)ceil_div(k.E, 4 * 2), (unsigned)n_ttiles);
    hipLaunchKernelGGL((route_logits_kernel<XT, 4, 2, 8>), grid, dim3(256), 0, stream, k);
  } else {
    dim3 grid((unsigned)ceil_div(k.E, 4 * 4), (unsigned)n_ttiles);
    hipLaunchKernelGGL((route_logits_kernel<XT, 16, 4, 1>), grid, dim3(256), 0, stream, k);
  }
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
  hipError_t err = (r.x_dtype == 0) ? launch_logits_t<uint16_t>(k, TT, n_ttiles, stream)
                                    : launch_logits_t<float>(k, TT, n_ttiles, stream);
  if (err != hipSuccess) return err;
  // One wave per token, four tokens per workgroup, so selection is spread
  // over many CUs; the permute then runs in its own single-workgroup launch.
  // A batch of at most four tokens is routed and permuted by one workgroup.
  const unsigned sel_blocks = (unsigned)ceil_div(r.T, kSelectWaves);
  const dim3 sb(kWave * kSelectWaves);
  if (r.E <= 64) hipLaunchKernelGGL(route_select_kernel<1>, dim3(sel_blocks), sb, 0, stream, k);
  else if (r.E <= 128) hipLaunchKernelGGL(route_select_kernel<2>, dim3(sel_blocks), sb, 0, stream, k);
  else if (r.E <= 256) hipLaunchKernelGGL(route_select_kernel<4>, dim3(sel_blocks), sb, 0, stream, k);
  else hipLaunchKernelGGL(route_select_kernel<8>, dim3(sel_blocks), sb, 0, stream, k);
  err = hipGetLastError();
  if (err != hipSuccess || !r.do_permute || sel_blocks == 1) return err;
  hipLaunchKernelGGL(permute_kernel, dim3(1), dim3(1024), 0, stream, k.topk_idx, r.T, r.k, r.E,
                     r.has_shared, ws.offsets, r.offsets_out, ws.active, ws.n_active, k.sorted_slots,
                     k.slot_pos, k.desc, k.seg_tok);
  return hipGetLastError();
}

hipError_t launch_permute(const int32_t* topk_idx, int64_t T, int k, int E, int has_shared,
                          int32_t* offsets, int32_t* sorted_slots, int32_t* slot_pos,
                          const Workspace& ws, hipStream_t stream) {
  hipLaunchKernelGGL(permute_kernel, dim3(1), dim3(1024), 0, stream, topk_idx, T, k, E, has_shared,
                     ws.offsets, offsets, ws.active, ws.n_active, sorted_slots, slot_pos,
                     static_cast<int4*>(nullptr), static_cast<int32_t*>(nullptr));
  return hipGetLastError();
}

}  // namespace pmoe
