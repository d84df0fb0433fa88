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
// Top-k: the last workgroup to finish a token tile (atomic ticket after a
// device-scope fence) selects for those tokens, one wave per token: k rounds
// of a wave-wide arg-max over (logit desc, index asc).  The last token tile to
// finish then runs the permute in one workgroup: per-wave expert counts,
// an (expert, wave)-major exclusive scan, and a second pass that places every
// slot at base + rank-within-round, where the rank comes from ballots over the
// bits of the expert id.  Placement depends only on slot order, never on
// atomics, so the permutation is deterministic and stable.
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
  int32_t* counters;
  int n_ttiles;
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

// Stable counting sort of n slots by expert, one workgroup of 256 threads.
__device__ void block_permute(const int32_t* __restrict__ idx, int64_t n, int E, int64_t T,
                              int has_shared, int32_t* offsets, int32_t* offsets_user,
                              int32_t* active, int32_t* n_active, int32_t* sorted_slots,
                              int32_t* slot_pos) {
  __shared__ int s_cnt[4][kMaxExperts];
  __shared__ int s_tmp[8];
  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int w = tid / kWave;
  int nbits = 1;
  while ((1 << nbits) < E) ++nbits;

  for (int i = tid; i < 4 * kMaxExperts; i += blockDim.x) (&s_cnt[0][0])[i] = 0;
  __syncthreads();

  const int64_t chunk = round_up(ceil_div(n, 4), kWave);
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

  // Scan: each thread owns experts 2*tid and 2*tid+1 (E <= 512).
  int tot2[2], act2[2];
  for (int i = 0; i < 2; ++i) {
    const int e = 2 * tid + i;
    int t = 0;
    if (e < E) t = s_cnt[0][e] + s_cnt[1][e] + s_cnt[2][e] + s_cnt[3][e];
    tot2[i] = t;
    act2[i] = (t > 0) ? 1 : 0;
  }
  int total = 0, total_act = 0;
  const int ex = block_exclusive_scan(tot2[0] + tot2[1], s_tmp, &total);
  const int ax = block_exclusive_scan(act2[0] + act2[1], s_tmp, &total_act);
  int run = ex, arun = ax;
  for (int i = 0; i < 2; ++i) {
    const int e = 2 * tid + i;
    if (e < E) {
      offsets[e] = run;
      if (offsets_user) offsets_user[e] = run;
      if (act2[i]) active[arun] = e;
      int b = run;
      for (int ww = 0; ww < 4; ++ww) {
        const int c = s_cnt[ww][e];
        s_cnt[ww][e] = b;  // becomes the running base of (expert, wave)
        b += c;
      }
    }
    run += tot2[i];
    arun += act2[i];
  }
  if (tid == 0) {
    offsets[E] = total;
    if (offsets_user) offsets_user[E] = total;
    offsets[E + 1] = total + (has_shared ? (int)T : 0);
    if (has_shared) active[total_act] = E;
    *n_active = total_act + (has_shared ? 1 : 0);
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
      // Every lane of the group has read the base before the leader bumps
      // it: LDS operations of one wave complete in program order, and the
      // read above precedes this write in every lane's program.
      if (below == 0) s_cnt[w][e] = s_cnt[w][e] + __popcll(m);
    } else if (s < end) {
      slot_pos[s] = -1;
    }
  }
}

// Wave-wide top-k for token t (called by all 64 lanes of one wave).
__device__ void wave_topk(const RouteK& a, int64_t t, double* s_vals, int* s_idx, double* s_e) {
  const int lane = threadIdx.x % kWave;
  constexpr int NV = kMaxExperts / kWave;
  double val[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int e = lane + kWave * v;
    val[v] = (e < a.E) ? a.logits[t * a.E + e] : 0.0;
  }
  uint32_t taken = 0;
  for (int j = 0; j < a.k; ++j) {
    double bv = __builtin_nan("");
    int bi = 0x7fffffff;
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const int e = lane + kWave * v;
      if (e < a.E && !((taken >> v) & 1u) && ranks_before(val[v], e, bv, bi)) {
        bv = val[v];
        bi = e;
      }
    }
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) {
      const double ov = shfl_xor_f64(bv, s);
      const int oi = __shfl_xor(bi, s, kWave);
      if (ranks_before(ov, oi, bv, bi)) {
        bv = ov;
        bi = oi;
      }
    }
    if (bi != 0x7fffffff && (bi % kWave) == lane) taken |= 1u << (bi / kWave);
    if (lane == 0) {
      s_vals[j] = bv;
      s_idx[j] = bi;
    }
  }
  // Weights: lane j (< k) owns slot j; every lane sums the k terms in slot
  // order from LDS, so the normaliser is the same sequential fp64 sum as the
  // oracle's.
  double ej = 0.0;
  if (lane < a.k) {
    const double v = s_vals[lane];
    ej = (a.score_mode == 0) ? exp(v - s_vals[0]) : 1.0 / (1.0 + exp(-v));
    s_e[lane] = ej;
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  if (lane < a.k) {
    double sum = 0.0;
    for (int j = 0; j < a.k; ++j) sum += s_e[j];
    a.topk_idx[t * a.k + lane] = s_idx[lane];
    a.topk_w[t * a.k + lane] = (float)(ej / sum);
  }
}

// MFMA-ordered copy of x (bf16) and fp32 group sums for tokens [t0, t0+TT).
__device__ void prep_x_tile(const RouteK& a, int64_t t0, int TT) {
  const uint16_t* x = static_cast<const uint16_t*>(a.x);
  const int64_t Kg = a.H / kGroup;
  const int64_t chunks = (int64_t)TT * a.Kq * 16;  // (t, q, p, gi) -> 8 bf16
  for (int64_t i = threadIdx.x; i < chunks; i += blockDim.x) {
    const int gi = (int)(i % 4);
    const int p = (int)((i / 4) % 4);
    const int64_t q = (i / 16) % a.Kq;
    const int64_t t = t0 + i / (16 * a.Kq);
    if (t >= a.T) continue;
    const int64_t g = 4 * q + gi;
    uint32_t wds[4] = {0, 0, 0, 0};
    if (g < Kg) {
      const uint16_t* xr = x + t * a.H + g * kGroup;
      for (int j = 0; j < 8; j += 2) {
        wds[j / 2] = (uint32_t)xr[kmap(p, j)] | ((uint32_t)xr[kmap(p, j + 1)] << 16);
      }
    }
    u32x4 v = {wds[0], wds[1], wds[2], wds[3]};
    // layout [t][q][p][gi][8]
    *reinterpret_cast<u32x4*>(a.xq + ((t * a.Kq + q) * 16 + p * 4 + gi) * 8) = v;
  }
  const int64_t ng = a.Kq * 4;
  for (int64_t i = threadIdx.x; i < (int64_t)TT * ng; i += blockDim.x) {
    const int64_t t = t0 + i / ng;
    const int64_t g = i % ng;
    if (t >= a.T) continue;
    float s = 0.0f;
    if (g < Kg) {
      const uint16_t* xr = x + t * a.H + g * kGroup;
      for (int j = 0; j < kGroup; ++j) s += bf16_bits_to_float(xr[j]);
    }
    a.xs[t * ng + g] = s;
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

template <typename XT, int TT, int EW>
__global__ __launch_bounds__(256) void route_kernel(RouteK a) {
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

  const int64_t nchunks = ceil_div(a.H, 256);
  for (int64_t c = 0; c < nchunks; ++c) {
    const int64_t h0 = c * 256 + 4 * lane;
    if (h0 < a.H) {
      float wv[EW][4];
#pragma unroll
      for (int ei = 0; ei < EW; ++ei) {
        const int e = e0 + ei;
        if (e < a.E) {
          const float4 r = *reinterpret_cast<const float4*>(a.W + (int64_t)e * a.H + h0);
          wv[ei][0] = r.x;
          wv[ei][1] = r.y;
          wv[ei][2] = r.z;
          wv[ei][3] = r.w;
        } else {
          wv[ei][0] = wv[ei][1] = wv[ei][2] = wv[ei][3] = 0.0f;
        }
      }
#pragma unroll
      for (int ti = 0; ti < TT; ++ti) {
        const int64_t t = t0 + ti;
        float xv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (t < a.T) load_x4<XT>(x, t * a.H + h0, xv);
#pragma unroll
        for (int ei = 0; ei < EW; ++ei) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            acc[ti * EW + ei] += (double)xv[i] * (double)wv[ei][i];
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

  // Ticket: the last expert tile of this token tile selects its top-k.
  __shared__ int s_last;
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    const int prev = atomicAdd(&a.counters[blockIdx.y], 1);
    s_last = (prev == (int)gridDim.x - 1);
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();

  __shared__ double s_vals[4][kMaxTopK];
  __shared__ double s_e[4][kMaxTopK];
  __shared__ int s_idx[4][kMaxTopK];
  for (int ti = w; ti < TT; ti += 4) {
    const int64_t t = t0 + ti;
    if (t < a.T) wave_topk(a, t, s_vals[w], s_idx[w], s_e[w]);
  }
  if (threadIdx.x == 0) a.counters[blockIdx.y] = 0;
  if (!a.do_permute) return;

  // Ticket: the last token tile runs the permute over all T*k slots.
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    const int prev = atomicAdd(&a.counters[a.n_ttiles], 1);
    s_last = (prev == a.n_ttiles - 1);
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  if (threadIdx.x == 0) a.counters[a.n_ttiles] = 0;
  block_permute(a.topk_idx, a.T * a.k, a.E, a.T, a.has_shared, a.offsets, a.offsets_user, a.active,
                a.n_active, a.sorted_slots, a.slot_pos);
}

__global__ __launch_bounds__(256) void permute_kernel(const int32_t* idx, int64_t T, int k, int E,
                                                      int has_shared, int32_t* offsets,
                                                      int32_t* offsets_user, int32_t* active,
                                                      int32_t* n_active, int32_t* sorted_slots,
                                                      int32_t* slot_pos) {
  block_permute(idx, T * k, E, T, has_shared, offsets, offsets_user, active, n_active,
                sorted_slots, slot_pos);
}

int router_token_tile(int64_t T) {
  if (T <= 1) return 1;
  if (T <= 64) return 4;
  return 16;
}

template <typename XT>
static hipError_t launch_route_t(const RouteK& k, int TT, hipStream_t stream) {
  if (TT == 1) {
    dim3 grid((unsigned)ceil_div(k.E, 4 * 1), (unsigned)k.n_ttiles);
    hipLaunchKernelGGL((route_kernel<XT, 1, 1>), grid, dim3(256), 0, stream, k);
  } else if (TT == 4) {
    dim3 grid((unsigned)ceil_div(k.E, 4 * 2), (unsigned)k.n_ttiles);
    hipLaunchKernelGGL((route_kernel<XT, 4, 2>), grid, dim3(256), 0, stream, k);
  } else {
    dim3 grid((unsigned)ceil_div(k.E, 4 * 4), (unsigned)k.n_ttiles);
    hipLaunchKernelGGL((route_kernel<XT, 16, 4>), grid, dim3(256), 0, stream, k);
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
  k.counters = ws.counters;
  const int TT = router_token_tile(r.T);
  k.n_ttiles = (int)ceil_div(r.T, TT);
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
  if (r.x_dtype == 0) return launch_route_t<uint16_t>(k, TT, stream);
  return launch_route_t<float>(k, TT, stream);
}

hipError_t launch_permute(const int32_t* topk_idx, int64_t T, int k, int E, int has_shared,
                          int32_t* offsets, int32_t* sorted_slots, int32_t* slot_pos,
                          const Workspace& ws, hipStream_t stream) {
  hipLaunchKernelGGL(permute_kernel, dim3(1), dim3(256), 0, stream, topk_idx, T, k, E, has_shared,
                     ws.offsets, offsets, ws.active, ws.n_active, sorted_slots, slot_pos);
  return hipGetLastError();
}

}  // namespace pmoe
