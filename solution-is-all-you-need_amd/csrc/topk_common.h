// topk_common.h -- top-k selection and routing weights of one token, one wave.
//
// Shared by the router's select kernel (router.hip) and the single-launch
// decode layer (decode_fused.hip), so both select and weigh experts with the
// same instructions.
//
// Reference semantics: torch.topk(logits, k, largest=True, sorted=True) then
// softmax over the k selected (tests/test_moe_routing.py:68-71); the order is
// descending by value, ties go to the lower expert index, NaN ranks below
// every number, -0 ties +0.
#pragma once

#include <math.h>
#include <stdint.h>

#include "moe_common.h"

namespace pmoe {

// Order-preserving integer key of a logit: a > b (as numbers) iff
// key(a) > key(b), -0.0 and +0.0 share a key, and NaN maps to 1, below every
// number (-inf has key 0x000F...F), so equal keys are exactly the ties the
// oracle breaks by index.  Key 0 is left for padding lanes.
__device__ inline uint64_t logit_key(double v) {
  if (isnan(v)) return 1ull;
  if (v == 0.0) v = 0.0;  // -0.0 -> +0.0
  const uint64_t b = __builtin_bit_cast(uint64_t, v);
  return (b >> 63) ? ~b : (b | 0x8000000000000000ull);
}

// Top-k of one token (called by all 64 lanes of one wave); `row` holds the
// token's E logits (global or LDS), lane l takes experts l, l + 64, ...
//  1. Radix descent over the key bits towards the largest x with
//     #{key >= x} >= k, the k-th largest key (two bits a step, one ballot +
//     popcount per threshold and register), stopping early at any x with
//     exactly k keys >= x.
//  2. Winners: every key > x, then keys == x in increasing expert index until
//     k are taken -- the (value desc, index asc) order's first k.
//  3. The k winners are compacted to LDS in index order and lane i < k ranks
//     winner i among them (the other winners read from their lanes); rank r
//     goes to slot r.
//  With at most kRankCountMaxE experts, steps 1-3 are one count per lane
//  instead: the keys ranked above its own (larger, or equal at a lower index).
//  4. Weights, fp64: softmax exp(l_j - l_0) / sum_i exp(l_i - l_0), or
//     sigmoid(l_j) / sum_i sigmoid(l_i), the sum taken in slot order; stored
//     as fp32.
// Outputs (slot j = lane < k): out_idx[j], out_w[j], and out_idx2[j] when
// out_idx2 is non-null.  The s_* arrays are this wave's LDS scratch of k
// entries each.
// Expert counts up to which one wave ranks by counting instead of the descent.
constexpr int kRankCountMaxE = 32;

template <int NV>
__device__ __attribute__((always_inline)) inline void wave_topk_row(const double* row, int E, int k, int score_mode,
                                                                    uint64_t* s_ck, double* s_cv, int* s_ci,
                                                                    double* s_val, int* s_idx, double* s_e,
                                                                    int32_t* out_idx, float* out_w,
                                                                    int32_t* out_idx2) {
  const int lane = threadIdx.x % kWave;
  const uint64_t lt_mask = (1ull << lane) - 1ull;
  uint64_t key[NV];
  double val[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int e = lane + kWave * v;
    const double lv = row[e < E ? e : E - 1];  // unconditional load
    val[v] = e < E ? lv : 0.0;
    key[v] = e < E ? logit_key(lv) : 0ull;
  }
  if (NV == 1 && E <= kRankCountMaxE) {
    // Few experts (one key per lane): each lane counts the keys ranked above
    // its own -- larger, or equal at a lower index -- from lane broadcasts;
    // rank r < k goes to slot r.  The same order as the descent below, in
    // about 7 instructions a key instead of one ballot chain per two bits.
    int r = 0;
    for (int j = 0; j < E; ++j) {
      const uint64_t kj = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(key[0] >> 32), j) << 32) |
                          (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)key[0], j);
      r += (kj > key[0] || (kj == key[0] && j < lane)) ? 1 : 0;
    }
    if (lane < E && r < k) {
      s_idx[r] = lane;
      s_val[r] = val[0];
    }
  } else {
  // Invariant: #{key >= kth} >= k.  Once it is exactly k the winners are
  // known (every other key is below kth), so the descent stops there --
  // usually at the first bits that separate the k-th and (k+1)-th keys.  Two
  // bits a step: the three thresholds' counts are independent, so a step
  // costs about one count's latency (each step waits on ballots and
  // popcounts; one bit a step ran about 150 cycles a bit).
  uint64_t kth = 0;
  int at_kth = kWave * NV;
  for (int bit = 63; bit >= 1 && at_kth != k; bit -= 2) {
    const uint64_t hb = 1ull << bit, lb = 1ull << (bit - 1);
    const uint64_t c1 = kth | lb, c2 = kth | hb, c3 = kth | hb | lb;
    int n1 = 0, n2 = 0, n3 = 0;
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      n1 += __popcll(__ballot(key[v] >= c1));
      n2 += __popcll(__ballot(key[v] >= c2));
      n3 += __popcll(__ballot(key[v] >= c3));
    }
    if (n3 >= k) {
      kth = c3;
      at_kth = n3;
    } else if (n2 >= k) {
      kth = c2;
      at_kth = n2;
    } else if (n1 >= k) {
      kth = c1;
      at_kth = n1;
    }
  }
  int n_gt = 0;
#pragma unroll
  for (int v = 0; v < NV; ++v) n_gt += __popcll(__ballot(key[v] > kth));
  const int take_eq = k - n_gt;  // >= 1 by the choice of kth
  int eq_before = 0, sel_before = 0;
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const bool eq = key[v] == kth;
    const uint64_t meq = __ballot(eq);
    const bool sel = key[v] > kth || (eq && eq_before + __popcll(meq & lt_mask) < take_eq);
    const uint64_t msel = __ballot(sel);
    if (sel) {
      const int pos = sel_before + __popcll(msel & lt_mask);
      s_ck[pos] = key[v];
      s_cv[pos] = val[v];
      s_ci[pos] = lane + kWave * v;
    }
    eq_before += __popcll(meq);
    sel_before += __popcll(msel);
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  // lane i < k holds winner i (index order) and ranks it among the k, the
  // others' keys and indices broadcast from their lanes
  uint64_t mk = 0ull;
  int me = 0;
  double mv = 0.0;
  if (lane < k) {
    mk = s_ck[lane];
    me = s_ci[lane];
    mv = s_cv[lane];
  }
  int r = 0;
  for (int j = 0; j < k; ++j) {
    const uint64_t kj = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(mk >> 32), j) << 32) |
                        (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)mk, j);
    const int cj = __builtin_amdgcn_readlane(me, j);
    r += (kj > mk || (kj == mk && cj < me)) ? 1 : 0;
  }
  if (lane < k) {
    s_idx[r] = me;
    s_val[r] = mv;
  }
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  // Weights: lane i (< k) owns slot i; the k terms are summed in slot order,
  // so the normaliser is the same sequential fp64 sum as the oracle's.
  double ej = 0.0;
  int oi = 0;
  if (lane < k) {
    const double v = s_val[lane];
    ej = (score_mode == 0) ? exp(v - s_val[0]) : 1.0 / (1.0 + exp(-v));
    oi = s_idx[lane];
  }
  double sum = 0.0;
  for (int i = 0; i < k; ++i) {
    const uint64_t b = __builtin_bit_cast(uint64_t, ej);
    sum += __builtin_bit_cast(double, ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(b >> 32), i) << 32) |
                                          (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, i));
  }
  if (lane < k) {
    out_idx[lane] = oi;
    if (out_idx2) out_idx2[lane] = oi;
    out_w[lane] = (float)(ej / sum);
  }
  (void)s_e;
  __builtin_amdgcn_wave_barrier();
}

}  // namespace pmoe
