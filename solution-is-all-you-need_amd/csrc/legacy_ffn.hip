// legacy_ffn.hip -- the reference's neuron-sparse fp16 FFN operator and its
// activation predictor, on gfx950, behind the reference's own symbols
// (declared in include/phantom_legacy.h):
//   sparse_mlp_forward      kernels/sparse_moe/sparse_matmul.cu:240-365
//   predict_active_neurons  kernels/sparse_moe/gate_predict.cu:200-242
//   get_sparsity_stats      kernels/sparse_moe/gate_predict.cu:253-271
//
// The reference runs one thread per output with a sequential fp32 loop over
// the dot product and row-per-thread (uncoalesced) weight reads
// (sparse_matmul.cu:56-100, :187-215), a single-thread compaction per batch
// row (gate_predict.cu:153-177), cuBLAS for the dense branch, and cudaMalloc
// / cudaFree / cuBLAS handle creation on every call.  Here:
//   - lg_rows_kernel: one wave per few weight rows; the 64 lanes split the
//     dot product, each streaming 16-byte loads (the 64 lanes of a wave read
//     1 KiB of a row at once, fully coalesced), then a fixed xor tree.  It
//     computes the predictor gate (sigmoid + threshold), or the gate and up
//     projections of the FFN with the SwiGLU epilogue fused in, for either
//     every neuron (dense branch, several batch rows per wave) or the list
//     positions of one batch row (sparse branch).
//   - lg_compact_kernel: wave prefix sums over the mask, one workgroup per
//     batch row, in increasing neuron order.
//   - lg_count_kernel + lg_down_kernel: the multiplicity of every neuron in
//     the active list, then a GEMV over the columns of W_down against
//     multiplicity x activation, streamed with the same coalesced 16-byte
//     loads (one pass over W_down per tile of up to 8 batch rows).
// Arithmetic: fp16 x fp16 products are exact in fp32, so each fmaf below is
// one rounded fp32 addition; the summation order is fixed (header of
// phantom_legacy.h), so results do not depend on timing.
#include <math.h>
#include <mutex>
#include <vector>

#include "moe_common.h"
#include "moe_launch.h"
#include "phantom_legacy.h"
#include "phantom_moe.h"

namespace pmoe {

constexpr int kLgWaves = 4;         // waves per workgroup
constexpr int kLgChunk = kWave * 8; // dot-product elements per lane pass: 8 per lane
constexpr int kLgRowsPredict = 8;   // predictor rows per wave
constexpr int kLgRowsFfn = 4;       // dense branch: neurons (gate and up rows) per wave
constexpr int kLgRowsSparse = 2;    // sparse branch: list positions per wave
constexpr int kLgRowsDown = 4;      // down rows per wave
constexpr int kLgCompactThreads = 1024;

enum LgMode { kLgPredict = 0, kLgDense = 1, kLgSparse = 2 };

struct LgRowsK {
  const uint16_t* x;    // [B, D] fp16
  const uint16_t* w1;   // [D_ffn, D] predictor gate, or FFN gate
  const uint16_t* b1;   // [D_ffn] or null
  const uint16_t* w2;   // [D_ffn, D] FFN up (FFN modes)
  const uint16_t* b2;
  const int32_t* idx;   // [B, D_ffn] active lists (sparse mode)
  const int32_t* count; // [B]
  int64_t B, D, D_ffn;
  int64_t cover;        // list positions the reference's grid covers (sparse mode)
  bool vec;             // D % 8 == 0 and x / w rows 16-byte aligned (picks the VEC kernels)
  float threshold;
  float* gate_out;      // [B, D_ffn] or null (predict)
  uint8_t* mask;        // [B, D_ffn] (predict)
  uint16_t* act;        // [B, D_ffn] fp16 by neuron (FFN modes)
};

__device__ inline float lg_sigmoid(float a) {
  return static_cast<float>(1.0 / (1.0 + exp(-static_cast<double>(a))));
}

// Eight fp16 values of a row starting at element d0, as raw bits (zeros past
// D).  The address is clamped so the load itself is unconditional.  VEC:
// D % 8 == 0 and 16-byte aligned rows, one 128-bit load; else eight element
// loads.
template <bool VEC>
__device__ inline uint4 lg_load8(const uint16_t* row, int64_t d0, int64_t D) {
  if (VEC) {
    const int64_t dc = d0 < D ? d0 : D - 8;
    const uint4 v = *reinterpret_cast<const uint4*>(row + dc);
    return d0 < D ? v : make_uint4(0u, 0u, 0u, 0u);
  } else {
    uint32_t h[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t d = d0 + j;
      const uint32_t v = row[d < D ? d : D - 1];
      h[j] = d < D ? v : 0u;
    }
    return make_uint4(h[0] | h[1] << 16, h[2] | h[3] << 16, h[4] | h[5] << 16, h[6] | h[7] << 16);
  }
}

// Element j (0..7) of eight packed fp16 values, as fp32.
__device__ inline float lg_elem(const uint4& v, int j) {
  const uint32_t w = j < 2 ? v.x : (j < 4 ? v.y : (j < 6 ? v.z : v.w));
  return half_bits_to_float32((j & 1) ? (w >> 16) : (w & 0xffffu));
}

__device__ inline float lg_tree(float v) {
#pragma unroll
  for (int s = kWave / 2; s >= 1; s >>= 1) v += __shfl_xor(v, s, kWave);
  return v;
}

__device__ inline float lg_bias(const uint16_t* b, int64_t n) {
  return b ? half_bits_to_float(b[n]) : 0.0f;
}

// NR weight rows x BT batch rows of dot products over D, in the fixed order:
// lane l adds elements d = 512 c + 8 l + j in increasing (c, j), then the
// xor tree.  Every lane returns every sum.  U chunks are loaded before any of
// them is summed (chunks past D load as zeros, which add nothing to a
// partial that started at +0.0).
template <int NR, int BT, bool VEC, int U>
__device__ inline void lg_dots(const uint16_t* const (&rows)[NR], const uint16_t* const (&xr)[BT], int64_t D,
                               float (&acc)[NR][BT]) {
  const int lane = threadIdx.x % kWave;
#pragma unroll
  for (int r = 0; r < NR; ++r)
#pragma unroll
    for (int b = 0; b < BT; ++b) acc[r][b] = 0.0f;
  for (int64_t c0 = 0; c0 < D; c0 += U * kLgChunk) {
    uint4 xv[U][BT], wv[U][NR];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t d0 = c0 + u * kLgChunk + 8 * lane;
#pragma unroll
      for (int b = 0; b < BT; ++b) xv[u][b] = lg_load8<VEC>(xr[b], d0, D);
#pragma unroll
      for (int r = 0; r < NR; ++r) wv[u][r] = lg_load8<VEC>(rows[r], d0, D);
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int r = 0; r < NR; ++r)
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
          for (int b = 0; b < BT; ++b)
            acc[r][b] = fmaf(lg_elem(wv[u][r], j), lg_elem(xv[u][b], j), acc[r][b]);
  }
#pragma unroll
  for (int r = 0; r < NR; ++r)
#pragma unroll
    for (int b = 0; b < BT; ++b) acc[r][b] = lg_tree(acc[r][b]);
}

// An fp32 value as rounded to fp32: the empty asm keeps the compiler from
// fusing the product that made it into a following fp16 conversion
// (v_fma_mixlo_f16 rounds once, straight to fp16, which moves ties away from
// the reference's fp32-then-fp16 rounding).
__device__ inline float lg_fp32(float v) {
  asm volatile("" : "+v"(v));
  return v;
}

// silu(g) * u as sparse_matmul.cu:141-145 (fp16 g and u read back as fp32),
// with this build's sigmoid.
__device__ inline uint16_t lg_swiglu(float g_acc, float u_acc) {
  const float g = half_bits_to_float32(float_to_half_bits(lg_fp32(g_acc)));
  const float u = half_bits_to_float32(float_to_half_bits(lg_fp32(u_acc)));
  const float silu = g * lg_sigmoid(g);
  return static_cast<uint16_t>(float_to_half_bits(lg_fp32(silu * u)));
}

// Picks acc[i / BT][i % BT] for lane i without indexing registers.
template <int NR, int BT>
__device__ inline float lg_pick(const float (&acc)[NR][BT], int i) {
  float v = acc[0][0];
#pragma unroll
  for (int r = 0; r < NR; ++r)
#pragma unroll
    for (int b = 0; b < BT; ++b) v = (i == r * BT + b) ? acc[r][b] : v;
  return v;
}

// Predictor: R consecutive neurons x BT batch rows per wave.
template <int BT, bool VEC, int U>
__global__ __launch_bounds__(kLgWaves* kWave) void lg_predict_kernel(LgRowsK p) {
  constexpr int R = kLgRowsPredict;
  const int lane = threadIdx.x % kWave;
  const int64_t n0 = ((int64_t)blockIdx.x * kLgWaves + threadIdx.x / kWave) * R;
  const int64_t b0 = (int64_t)blockIdx.y * BT;
  if (n0 >= p.D_ffn) return;
  const uint16_t* rows[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t n = n0 + r < p.D_ffn ? n0 + r : p.D_ffn - 1;
    rows[r] = p.w1 + n * p.D;
  }
  const uint16_t* xr[BT];
#pragma unroll
  for (int b = 0; b < BT; ++b) xr[b] = p.x + (b0 + b < p.B ? b0 + b : p.B - 1) * p.D;
  float acc[R][BT];
  lg_dots<R, BT, VEC, U>(rows, xr, p.D, acc);
  if (lane < R * BT) {
    const int r = lane / BT, b = lane % BT;
    const int64_t n = n0 + r, bb = b0 + b;
    if (n < p.D_ffn && bb < p.B) {
      const float a = lg_pick<R, BT>(acc, lane) + lg_bias(p.b1, n);
      const float g = lg_sigmoid(a);
      const int64_t o = bb * p.D_ffn + n;
      if (p.gate_out) p.gate_out[o] = g;
      p.mask[o] = g >= p.threshold ? 1 : 0;
    }
  }
}

// FFN gate + up + SwiGLU.  Dense: R consecutive neurons x BT batch rows, no
// biases.  Sparse: R list positions of one batch row, with biases.
template <int MODE, int R, int BT, bool VEC, int U>
__global__ __launch_bounds__(kLgWaves* kWave) void lg_ffn_rows_kernel(LgRowsK p) {
  const int lane = threadIdx.x % kWave;
  const int64_t i0 = ((int64_t)blockIdx.x * kLgWaves + threadIdx.x / kWave) * R;
  const int64_t b0 = (int64_t)blockIdx.y * BT;
  int64_t lim = p.D_ffn;
  if (MODE == kLgSparse) {
    int64_t c = p.count[b0];
    c = c < 0 ? 0 : (c > p.D_ffn ? p.D_ffn : c);
    lim = c < p.cover ? c : p.cover;
  }
  if (i0 >= lim) return;
  int64_t n[R];
  bool ok[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t i = i0 + r;
    if (MODE == kLgSparse) {
      const int64_t v = p.idx[b0 * p.D_ffn + (i < lim ? i : lim - 1)];
      ok[r] = i < lim && v >= 0 && v < p.D_ffn;
      n[r] = ok[r] ? v : 0;
    } else {
      ok[r] = i < lim;
      n[r] = ok[r] ? i : lim - 1;
    }
  }
  const uint16_t* rows[2 * R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    rows[r] = p.w1 + n[r] * p.D;
    rows[R + r] = p.w2 + n[r] * p.D;
  }
  const uint16_t* xr[BT];
#pragma unroll
  for (int b = 0; b < BT; ++b) xr[b] = p.x + (b0 + b < p.B ? b0 + b : p.B - 1) * p.D;
  float acc[2 * R][BT];
  lg_dots<2 * R, BT, VEC, U>(rows, xr, p.D, acc);
  if (lane < R * BT) {
    const int r = lane / BT, b = lane % BT;
    // gate rows are 0..R-1 and up rows R..2R-1 of acc: pick both for (r, b)
    float g = acc[0][0], u = acc[R][0];
#pragma unroll
    for (int rr = 0; rr < R; ++rr)
#pragma unroll
      for (int bb = 0; bb < BT; ++bb) {
        g = (lane == rr * BT + bb) ? acc[rr][bb] : g;
        u = (lane == rr * BT + bb) ? acc[R + rr][bb] : u;
      }
    bool live = false;
    int64_t nn = 0;
#pragma unroll
    for (int rr = 0; rr < R; ++rr)
      if (rr == r) {
        live = ok[rr];
        nn = n[rr];
      }
    const int64_t bb = b0 + b;
    if (live && bb < p.B) {
      if (MODE == kLgSparse) {
        g += lg_bias(p.b1, nn);
        u += lg_bias(p.b2, nn);
      }
      p.act[bb * p.D_ffn + nn] = lg_swiglu(g, u);
    }
  }
}

// Multiplicity of every neuron in the first count[b] list entries of batch
// row b (sparse branch): the down projection sums over list entries, so a
// neuron listed twice contributes twice.  Integer atomics, so the counts do
// not depend on timing.
__global__ __launch_bounds__(256) void lg_count_kernel(const int32_t* __restrict__ idx,
                                                        const int32_t* __restrict__ count,
                                                        int32_t* __restrict__ mult, int64_t D_ffn) {
  const int64_t b = blockIdx.y;
  int64_t lim = count[b];
  lim = lim < 0 ? 0 : (lim > D_ffn ? D_ffn : lim);
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < lim; i += (int64_t)gridDim.x * blockDim.x) {
    const int32_t n = idx[b * D_ffn + i];
    if (n >= 0 && n < D_ffn) atomicAdd(&mult[b * D_ffn + n], 1);
  }
}

// m_n * act[n] as fp32, and whether column n takes part (m_n > 0; dense
// branch: every column, m_n = 1).
template <int MODE, bool VEC>
__device__ inline void lg_down_operand(const uint16_t* arow, const int32_t* mrow, int64_t n0, int64_t D_ffn,
                                       float a[8], bool on[8]) {
  const uint4 av = lg_load8<VEC>(arow, n0, D_ffn);
  if (MODE == kLgSparse) {
    int32_t m[8];
    if (VEC) {
      const int64_t nc = n0 < D_ffn ? n0 : D_ffn - 8;
      const int4 m0 = *reinterpret_cast<const int4*>(mrow + nc);
      const int4 m1 = *reinterpret_cast<const int4*>(mrow + nc + 4);
      const int32_t mm[8] = {m0.x, m0.y, m0.z, m0.w, m1.x, m1.y, m1.z, m1.w};
#pragma unroll
      for (int j = 0; j < 8; ++j) m[j] = n0 < D_ffn ? mm[j] : 0;
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int64_t n = n0 + j;
        const int32_t v = mrow[n < D_ffn ? n : D_ffn - 1];
        m[j] = n < D_ffn ? v : 0;
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      on[j] = m[j] > 0;
      a[j] = (float)m[j] * lg_elem(av, j);
    }
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      on[j] = n0 + j < D_ffn;
      a[j] = lg_elem(av, j);
    }
  }
}

// y[b, d] = sum over columns n of Wd[d, n] * (m_n act[b, n]), columns with
// m_n = 0 skipped; lane l adds the columns with (n mod 512) / 8 == l in
// increasing n (the predictor's order), then the xor tree.  R output rows x
// BT batch rows per wave: each 16-byte weight load serves BT batch rows, so
// W_down is streamed once per batch tile with coalesced loads, whatever the
// active lists look like (a row-major W_down has every 64-column line touched
// by any list denser than a few percent anyway).
template <int MODE, int R, int BT, bool VEC, int U>
__global__ __launch_bounds__(kLgWaves* kWave) void lg_down_kernel(const uint16_t* __restrict__ act,
                                                                  const int32_t* __restrict__ mult,
                                                                  const uint16_t* __restrict__ wd,
                                                                  uint16_t* __restrict__ y, int64_t B, int64_t D,
                                                                  int64_t D_ffn) {
  const int lane = threadIdx.x % kWave;
  const int64_t d0 = ((int64_t)blockIdx.x * kLgWaves + threadIdx.x / kWave) * R;
  const int64_t b0 = (int64_t)blockIdx.y * BT;
  if (d0 >= D) return;
  const uint16_t* wrow[R];
#pragma unroll
  for (int r = 0; r < R; ++r) wrow[r] = wd + (d0 + r < D ? d0 + r : D - 1) * D_ffn;
  const uint16_t* arow[BT];
  const int32_t* mrow[BT];
#pragma unroll
  for (int b = 0; b < BT; ++b) {
    const int64_t bb = b0 + b < B ? b0 + b : B - 1;
    arow[b] = act + bb * D_ffn;
    mrow[b] = mult + bb * D_ffn;
  }
  float acc[R][BT];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int b = 0; b < BT; ++b) acc[r][b] = 0.0f;
  for (int64_t c0 = 0; c0 < D_ffn; c0 += U * kLgChunk) {
    uint4 wv[U][R];
    float a[U][BT][8];
    bool on[U][BT][8];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t n0 = c0 + u * kLgChunk + 8 * lane;
#pragma unroll
      for (int r = 0; r < R; ++r) wv[u][r] = lg_load8<VEC>(wrow[r], n0, D_ffn);
#pragma unroll
      for (int b = 0; b < BT; ++b) lg_down_operand<MODE, VEC>(arow[b], mrow[b], n0, D_ffn, a[u][b], on[u][b]);
    }
    // skipped columns add an exact +0 product (their activation is zero),
    // which leaves a partial that started at +0.0 unchanged
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float w = lg_elem(wv[u][r], j);
#pragma unroll
          for (int b = 0; b < BT; ++b) acc[r][b] = fmaf(on[u][b][j] ? w : 0.0f, a[u][b][j], acc[r][b]);
        }
  }
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int b = 0; b < BT; ++b) acc[r][b] = lg_tree(acc[r][b]);
  if (lane < R * BT) {
    const int r = lane / BT, b = lane % BT;
    if (d0 + r < D && b0 + b < B) y[(b0 + b) * D + d0 + r] = static_cast<uint16_t>(float_to_half_bits(lg_pick<R, BT>(acc, lane)));
  }
}

// Active neuron list of one batch row per workgroup, in increasing order.
__global__ __launch_bounds__(kLgCompactThreads) void lg_compact_kernel(const uint8_t* __restrict__ mask,
                                                                       int32_t* __restrict__ idx,
                                                                       int32_t* __restrict__ count,
                                                                       int64_t D_ffn) {
  constexpr int kWaves = kLgCompactThreads / kWave;
  __shared__ int s_wave[kWaves];
  const int tid = threadIdx.x, lane = tid % kWave, w = tid / kWave;
  const uint8_t* m = mask + (int64_t)blockIdx.x * D_ffn;
  int32_t* out = idx + (int64_t)blockIdx.x * D_ffn;
  int64_t base = 0;
  for (int64_t t0 = 0; t0 < D_ffn; t0 += 4 * kLgCompactThreads) {
    const int64_t e0 = t0 + 4 * tid;
    bool on[4];
    int cnt = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t e = e0 + j;
      const uint8_t v = m[e < D_ffn ? e : D_ffn - 1];
      on[j] = e < D_ffn && v != 0;
      cnt += on[j] ? 1 : 0;
    }
    int incl = cnt;
#pragma unroll
    for (int s = 1; s < kWave; s <<= 1) {
      const int o = __shfl_up(incl, s, kWave);
      incl += lane >= s ? o : 0;
    }
    if (lane == kWave - 1) s_wave[w] = incl;
    __syncthreads();
    int before = 0, total = 0;
#pragma unroll
    for (int v = 0; v < kWaves; ++v) {
      before += v < w ? s_wave[v] : 0;
      total += s_wave[v];
    }
    int64_t pos = base + before + incl - cnt;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (on[j]) out[pos++] = (int32_t)(e0 + j);
    base += total;
    __syncthreads();
  }
  if (tid == 0) count[blockIdx.x] = (int32_t)base;
}

__global__ void lg_zero_kernel(uint4* __restrict__ p, int64_t n16) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = make_uint4(0u, 0u, 0u, 0u);
}

// ---------------------------------------------------------------------------
// host side

namespace {

int batch_tile(int64_t B) { return B >= 8 ? 8 : (B >= 4 ? 4 : (B >= 2 ? 2 : 1)); }

// Loads in flight per lane: U chunks x (rows + batch rows) x 16 bytes.
template <int BT, bool VEC>
hipError_t launch_predict_bt(const LgRowsK& p, hipStream_t s) {
  constexpr int U = BT == 1 ? 2 : 1;
  const dim3 grid((unsigned)ceil_div(p.D_ffn, (int64_t)kLgWaves * kLgRowsPredict), (unsigned)ceil_div(p.B, BT));
  hipLaunchKernelGGL((lg_predict_kernel<BT, VEC, U>), grid, dim3(kLgWaves * kWave), 0, s, p);
  return hipGetLastError();
}

template <int MODE, int BT, bool VEC>
hipError_t launch_ffn_rows_bt(const LgRowsK& p, hipStream_t s) {
  // sparse: one batch row, few list positions per wave and deep loads;
  // dense: neighbouring neurons of several batch rows share each row load
  constexpr int R = MODE == kLgSparse ? kLgRowsSparse : kLgRowsFfn;
  constexpr int U = MODE == kLgSparse ? 4 : (BT == 1 ? 2 : 1);
  const int64_t rows = MODE == kLgSparse ? (p.cover < p.D_ffn ? p.cover : p.D_ffn) : p.D_ffn;
  const dim3 grid((unsigned)ceil_div(rows, (int64_t)kLgWaves * R), (unsigned)ceil_div(p.B, BT));
  hipLaunchKernelGGL((lg_ffn_rows_kernel<MODE, R, BT, VEC, U>), grid, dim3(kLgWaves * kWave), 0, s, p);
  return hipGetLastError();
}

template <int MODE, int BT>
hipError_t launch_ffn_rows(const LgRowsK& p, hipStream_t s) {
  return p.vec ? launch_ffn_rows_bt<MODE, BT, true>(p, s) : launch_ffn_rows_bt<MODE, BT, false>(p, s);
}

template <int MODE, int BT, bool VEC>
hipError_t launch_down_bt(const uint16_t* act, const int32_t* mult, const uint16_t* wd, uint16_t* y, int64_t B,
                          int64_t D, int64_t D_ffn, hipStream_t s) {
  constexpr int U = BT == 1 ? 2 : 1;
  const dim3 grid((unsigned)ceil_div(D, (int64_t)kLgWaves * kLgRowsDown), (unsigned)ceil_div(B, BT));
  hipLaunchKernelGGL((lg_down_kernel<MODE, kLgRowsDown, BT, VEC, U>), grid, dim3(kLgWaves * kWave), 0, s, act, mult,
                     wd, y, B, D, D_ffn);
  return hipGetLastError();
}

template <int MODE>
hipError_t launch_down(const uint16_t* act, const int32_t* mult, const uint16_t* wd, uint16_t* y, int64_t B,
                       int64_t D, int64_t D_ffn, bool vec, hipStream_t s) {
  switch (batch_tile(B)) {
    case 8: return vec ? launch_down_bt<MODE, 8, true>(act, mult, wd, y, B, D, D_ffn, s)
                       : launch_down_bt<MODE, 8, false>(act, mult, wd, y, B, D, D_ffn, s);
    case 4: return vec ? launch_down_bt<MODE, 4, true>(act, mult, wd, y, B, D, D_ffn, s)
                       : launch_down_bt<MODE, 4, false>(act, mult, wd, y, B, D, D_ffn, s);
    case 2: return vec ? launch_down_bt<MODE, 2, true>(act, mult, wd, y, B, D, D_ffn, s)
                       : launch_down_bt<MODE, 2, false>(act, mult, wd, y, B, D, D_ffn, s);
    default: return vec ? launch_down_bt<MODE, 1, true>(act, mult, wd, y, B, D, D_ffn, s)
                        : launch_down_bt<MODE, 1, false>(act, mult, wd, y, B, D, D_ffn, s);
  }
}

// Per-device state of the legacy entry points: the activation buffers and the
// timing events.  Eager calls wait for their own work before returning (as the
// reference's do), so their buffer is idle between calls; a process-wide mutex
// keeps calls one at a time.  Calls recorded under stream capture use a second
// buffer, `cap`, so graph replays never share memory with eager calls.  Every
// eager call makes both buffers large enough for its size.  Once a capture has
// recorded `cap`, a graph may replay it at any later time: a larger `cap` is
// then allocated beside it and the held one is kept, never freed, until the
// process ends.
struct LgBuf {
  uint16_t* p = nullptr;
  size_t bytes = 0;
};
struct LgDevice {
  LgBuf act;
  LgBuf cap;
  bool cap_held = false;
  std::vector<void*> retired;
  hipEvent_t ev[2] = {nullptr, nullptr};
};
std::mutex g_lg_mutex;
LgDevice g_lg_dev[64];

// Makes `b` hold at least `need` bytes (rounded up to 1 MiB).  A buffer that
// a captured graph references is retired instead of freed.
bool lg_reserve(LgBuf* b, size_t need, bool* held, std::vector<void*>* retired) {
  if (b->bytes >= need) return true;
  if (b->p) {
    if (held && *held) {
      retired->push_back(b->p);
      *held = false;
    } else {
      (void)hipFree(b->p);
    }
    b->p = nullptr;
    b->bytes = 0;
  }
  const size_t bytes = (size_t)round_up((int64_t)need, (int64_t)1 << 20);
  if (hipMalloc(reinterpret_cast<void**>(&b->p), bytes) != hipSuccess) {
    b->p = nullptr;
    return false;
  }
  b->bytes = bytes;
  return true;
}

bool capturing(hipStream_t s) {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &st) != hipSuccess) return false;
  return st != hipStreamCaptureStatusNone;
}

struct LgCall {
  LgDevice* dev = nullptr;
  bool timed = false;
};

// Device state and the start event; returns a message on failure.
const char* lg_begin(hipStream_t s, LgCall* c) {
  int d = 0;
  if (hipGetDevice(&d) != hipSuccess || d < 0 || d >= 64) return "no current HIP device";
  c->dev = &g_lg_dev[d];
  c->timed = !capturing(s);
  if (c->timed) {
    for (int i = 0; i < 2; ++i)
      if (!c->dev->ev[i] && hipEventCreate(&c->dev->ev[i]) != hipSuccess) return "hipEventCreate failed";
    if (hipEventRecord(c->dev->ev[0], s) != hipSuccess) return "hipEventRecord failed";
  }
  return nullptr;
}

// Stop event, wait, elapsed milliseconds (0 under capture); <0 on failure.
float lg_end(hipStream_t s, const LgCall& c) {
  if (!c.timed) return 0.0f;
  float ms = 0.0f;
  if (hipEventRecord(c.dev->ev[1], s) != hipSuccess || hipEventSynchronize(c.dev->ev[1]) != hipSuccess ||
      hipEventElapsedTime(&ms, c.dev->ev[0], c.dev->ev[1]) != hipSuccess)
    return -1.0f;
  return ms;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

template <bool VEC>
hipError_t launch_lg_predict_v(const LgRowsK& p, hipStream_t s) {
  switch (batch_tile(p.B)) {
    case 8: return launch_predict_bt<8, VEC>(p, s);
    case 4: return launch_predict_bt<4, VEC>(p, s);
    case 2: return launch_predict_bt<2, VEC>(p, s);
    default: return launch_predict_bt<1, VEC>(p, s);
  }
}

hipError_t launch_lg_predict(const LgRowsK& p, hipStream_t s) {
  return p.vec ? launch_lg_predict_v<true>(p, s) : launch_lg_predict_v<false>(p, s);
}

}  // namespace pmoe

using namespace pmoe;

extern "C" {

PHANTOM_LEGACY_API float predict_active_neurons(const phantom_half* d_input, const phantom_half* d_gate_weights,
                                                const phantom_half* d_gate_bias, uint8_t* d_active_mask,
                                                int* d_active_indices, int* d_active_count, float* d_gate_output,
                                                int B, int D, int D_ffn, float threshold, hipStream_t stream) {
  if ((D > 0 && (!d_input || !d_gate_weights)) || !d_active_mask || !d_active_indices || !d_active_count)
    return (float)set_error(PHANTOM_MOE_EINVAL, "predict_active_neurons: input, weights, mask, indices and count must be non-null");
  if (B < 1 || D < 0 || D_ffn < 1)
    return (float)set_error(PHANTOM_MOE_EINVAL, "predict_active_neurons: need B >= 1, D >= 0, D_ffn >= 1 (got %d, %d, %d)", B, D, D_ffn);
  std::lock_guard<std::mutex> lock(g_lg_mutex);
  LgCall call;
  if (const char* m = lg_begin(stream, &call)) return (float)set_error(PHANTOM_MOE_ELAUNCH, "predict_active_neurons: %s", m);
  LgRowsK p{};
  p.x = d_input;
  p.w1 = d_gate_weights;
  p.b1 = d_gate_bias;
  p.B = B;
  p.D = D;
  p.D_ffn = D_ffn;
  p.vec = D % 8 == 0 && aligned16(d_input) && aligned16(d_gate_weights);
  p.threshold = threshold;
  p.gate_out = d_gate_output;
  p.mask = d_active_mask;
  hipError_t e = launch_lg_predict(p, stream);
  if (e == hipSuccess) {
    hipLaunchKernelGGL(lg_compact_kernel, dim3(B), dim3(kLgCompactThreads), 0, stream, d_active_mask,
                       d_active_indices, d_active_count, (int64_t)D_ffn);
    e = hipGetLastError();
  }
  if (e != hipSuccess) return (float)set_error(PHANTOM_MOE_ELAUNCH, "predict_active_neurons: %s", hipGetErrorString(e));
  const float ms = lg_end(stream, call);
  if (ms < 0.0f) return (float)set_error(PHANTOM_MOE_ELAUNCH, "predict_active_neurons: timing events failed");
  clear_error();
  return ms;
}

PHANTOM_LEGACY_API float sparse_mlp_forward(const phantom_half* d_input, const phantom_half* d_gate_weight,
                                            const phantom_half* d_gate_bias, const phantom_half* d_up_weight,
                                            const phantom_half* d_up_bias, const phantom_half* d_down_weight,
                                            const int* d_active_indices, const int* d_active_count,
                                            phantom_half* d_output, int B, int D, int D_ffn, float sparsity_pct,
                                            hipStream_t stream) {
  if (D > 0 && (!d_input || !d_gate_weight || !d_up_weight || !d_down_weight || !d_output))
    return (float)set_error(PHANTOM_MOE_EINVAL, "sparse_mlp_forward: input, weights and output must be non-null");
  if (B < 1 || D < 0 || D_ffn < 1)
    return (float)set_error(PHANTOM_MOE_EINVAL, "sparse_mlp_forward: need B >= 1, D >= 0, D_ffn >= 1 (got %d, %d, %d)", B, D, D_ffn);
  // Branch and coverage exactly as the reference's host code computes them
  // (fp32 arithmetic, truncation toward zero).
  const float frac = sparsity_pct / 100.0f;
  const bool dense = frac < 0.30f;
  int64_t cover = D_ffn;
  if (!dense) {
    const float m = (1.0f - frac) * (float)D_ffn;
    if (!(m > -256.0f)) return (float)set_error(PHANTOM_MOE_EINVAL, "sparse_mlp_forward: sparsity_pct %g leaves no list position to compute", (double)sparsity_pct);
    int64_t max_active = (int64_t)m + 32;
    if (max_active > D_ffn) max_active = D_ffn;
    cover = max_active > 0 ? ceil_div(max_active, 256) * 256 : 0;
    if (cover < 1) return (float)set_error(PHANTOM_MOE_EINVAL, "sparse_mlp_forward: sparsity_pct %g leaves no list position to compute", (double)sparsity_pct);
    if (!d_active_indices || !d_active_count)
      return (float)set_error(PHANTOM_MOE_EINVAL, "sparse_mlp_forward: the sparse branch needs active indices and counts");
  }
  std::lock_guard<std::mutex> lock(g_lg_mutex);
  LgCall call;
  if (const char* m = lg_begin(stream, &call)) return (float)set_error(PHANTOM_MOE_ELAUNCH, "sparse_mlp_forward: %s", m);
  // pool: act fp16 [B, D_ffn] (16-byte rows padded as a whole), then the
  // neuron multiplicities int32 [B, D_ffn]
  const size_t act_bytes = (size_t)round_up((int64_t)B * D_ffn, 8) * sizeof(uint16_t);
  const size_t need = act_bytes + (size_t)round_up((int64_t)B * D_ffn, 4) * sizeof(int32_t);
  uint16_t* act = nullptr;
  if (call.timed) {
    if (!lg_reserve(&call.dev->act, need, nullptr, nullptr) ||
        !lg_reserve(&call.dev->cap, need, &call.dev->cap_held, &call.dev->retired))
      return (float)set_error(PHANTOM_MOE_ELAUNCH, "sparse_mlp_forward: cannot allocate %zu bytes", need);
    act = call.dev->act.p;
  } else {
    if (call.dev->cap.bytes < need)
      return (float)set_error(PHANTOM_MOE_EUNSUPPORTED, "sparse_mlp_forward: no activation buffer for B * D_ffn = %lld under stream capture; call once at this size outside capture first", (long long)B * D_ffn);
    call.dev->cap_held = true;
    act = call.dev->cap.p;
  }
  int32_t* mult = reinterpret_cast<int32_t*>(reinterpret_cast<char*>(act) + act_bytes);
  LgRowsK p{};
  p.x = d_input;
  p.w1 = d_gate_weight;
  p.w2 = d_up_weight;
  p.b1 = dense ? nullptr : d_gate_bias;
  p.b2 = dense ? nullptr : d_up_bias;
  p.idx = d_active_indices;
  p.count = d_active_count;
  p.B = B;
  p.D = D;
  p.D_ffn = D_ffn;
  p.cover = cover;
  p.vec = D % 8 == 0 && aligned16(d_input) && aligned16(d_gate_weight) && aligned16(d_up_weight);
  p.act = act;
  hipError_t e = hipSuccess;
  if (dense) {
    switch (batch_tile(B)) {
      case 8: e = launch_ffn_rows<kLgDense, 8>(p, stream); break;
      case 4: e = launch_ffn_rows<kLgDense, 4>(p, stream); break;
      case 2: e = launch_ffn_rows<kLgDense, 2>(p, stream); break;
      default: e = launch_ffn_rows<kLgDense, 1>(p, stream); break;
    }
  } else {
    hipLaunchKernelGGL(lg_zero_kernel, dim3(1024), dim3(256), 0, stream, reinterpret_cast<uint4*>(p.act),
                       (int64_t)(need / 16));
    e = hipGetLastError();
    if (e == hipSuccess) {
      hipLaunchKernelGGL(lg_count_kernel, dim3((unsigned)ceil_div(D_ffn, 256), (unsigned)B), dim3(256), 0, stream,
                         d_active_indices, d_active_count, mult, (int64_t)D_ffn);
      e = hipGetLastError();
    }
    if (e == hipSuccess) e = launch_ffn_rows<kLgSparse, 1>(p, stream);
  }
  if (e == hipSuccess && D > 0) {
    const bool dvec = D_ffn % 8 == 0 && aligned16(d_down_weight);
    e = dense ? launch_down<kLgDense>(p.act, mult, d_down_weight, d_output, B, D, D_ffn, dvec, stream)
              : launch_down<kLgSparse>(p.act, mult, d_down_weight, d_output, B, D, D_ffn, dvec, stream);
  }
  if (e != hipSuccess) return (float)set_error(PHANTOM_MOE_ELAUNCH, "sparse_mlp_forward: %s", hipGetErrorString(e));
  const float ms = lg_end(stream, call);
  if (ms < 0.0f) return (float)set_error(PHANTOM_MOE_ELAUNCH, "sparse_mlp_forward: timing events failed");
  clear_error();
  return ms;
}

PHANTOM_LEGACY_API float get_sparsity_stats(const int* d_active_count, int B, int D_ffn, hipStream_t stream) {
  if (B < 0) return (float)set_error(PHANTOM_MOE_EINVAL, "get_sparsity_stats: B must be >= 0, got %d", B);
  if (B > 0 && !d_active_count) return (float)set_error(PHANTOM_MOE_EINVAL, "get_sparsity_stats: d_active_count is null");
  float total_active = 0.0f;
  if (B > 0) {
    int32_t small[256];
    int32_t* h = small;
    int32_t* heap = nullptr;
    if (B > 256) {
      heap = static_cast<int32_t*>(malloc(sizeof(int32_t) * (size_t)B));
      if (!heap) return (float)set_error(PHANTOM_MOE_ELAUNCH, "get_sparsity_stats: host allocation failed");
      h = heap;
    }
    hipError_t e = hipMemcpyAsync(h, d_active_count, sizeof(int32_t) * (size_t)B, hipMemcpyDeviceToHost, stream);
    if (e == hipSuccess) e = hipStreamSynchronize(stream);
    if (e != hipSuccess) {
      free(heap);
      return (float)set_error(PHANTOM_MOE_ELAUNCH, "get_sparsity_stats: %s", hipGetErrorString(e));
    }
    for (int b = 0; b < B; ++b) total_active += (float)h[b];
    free(heap);
  }
  const float avg_active = total_active / (float)B;
  clear_error();
  return (1.0f - avg_active / (float)D_ffn) * 100.0f;
}

}  // extern "C"
