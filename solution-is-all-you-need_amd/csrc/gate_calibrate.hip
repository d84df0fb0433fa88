// gate_calibrate.hip -- the reference's sparsity-gate calibration
// (kernels/sparse_moe/gate_calibrate.cu:228-340) on gfx950, behind its own
// symbol calibrate_sparsity_gate (declared in include/phantom_legacy.h).
//
// The operator trains, for one FFN layer, one linear gate per neuron,
// gate = sigmoid(W x + b), to predict which neurons are active: a neuron is
// active on a sample when |activation| >= 0.01 * max(max_row |activation|,
// 1e-10) (gate_calibrate.cu:54-85).  W and b start at zero and take 50
// full-batch gradient steps of binary cross-entropy, lr 1e-3
// (:105-210, :283-307); then the F1 score of (gate >= 0.5) against the masks
// decides whether sparse routing is enabled (F1 >= 0.70, :309-334).
//
// Kernels: cal_mask_kernel (one workgroup per sample: row max, masks, active
// count), cal_forward_kernel (predictions, the legacy GEMV's fixed order on
// fp32 operands: one wave per 8 gate rows x up to 8 samples, lanes split D),
// cal_update_kernel (gradient and step: one thread per weight, samples summed
// in order, the reference's own decomposition, which is already coalesced
// over d).  fmaf everywhere (the products of fp32 operands are not exact, so
// the fused form is part of the contract); the sigmoid is the fp32 rounding
// of the fp64 expression, clamped to [1e-7, 1 - 1e-7] as :134.
#include <math.h>
#include <mutex>
#include <stdlib.h>
#include <string.h>

#include "moe_common.h"
#include "moe_launch.h"
#include "phantom_legacy.h"
#include "phantom_moe.h"

namespace pmoe {

constexpr int kCalEpochs = 50;             // gate_calibrate.cu:35
constexpr float kCalLr = 1e-3f;            // :34
constexpr float kCalF1Threshold = 0.70f;   // :36
constexpr float kCalActFrac = 0.01f;       // :37
constexpr int kCalWaves = 4;
constexpr int kCalRows = 8;                // gate rows per forward wave
constexpr int kCalChunk = kWave * 8;       // dot elements per lane pass

__global__ __launch_bounds__(256) void cal_mask_kernel(const float* __restrict__ act, uint8_t* __restrict__ masks,
                                                       int32_t* __restrict__ row_active, int64_t D_ffn) {
  __shared__ float s_max[256 / kWave];
  __shared__ int s_cnt[256 / kWave];
  const int64_t s = blockIdx.x;
  const float* row = act + s * D_ffn;
  float m = 0.0f;
  for (int64_t i = threadIdx.x; i < D_ffn; i += blockDim.x) m = fmaxf(m, fabsf(row[i]));
#pragma unroll
  for (int o = kWave / 2; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, kWave));
  if (threadIdx.x % kWave == 0) s_max[threadIdx.x / kWave] = m;
  __syncthreads();
  float rmax = s_max[0];
  for (int w = 1; w < (int)(blockDim.x / kWave); ++w) rmax = fmaxf(rmax, s_max[w]);
  rmax = fmaxf(rmax, 1e-10f);
  const float thr = kCalActFrac * rmax;
  int cnt = 0;
  for (int64_t i = threadIdx.x; i < D_ffn; i += blockDim.x) {
    const uint8_t on = fabsf(row[i]) >= thr ? 1 : 0;
    masks[s * D_ffn + i] = on;
    cnt += on;
  }
#pragma unroll
  for (int o = kWave / 2; o >= 1; o >>= 1) cnt += __shfl_xor(cnt, o, kWave);
  if (threadIdx.x % kWave == 0) s_cnt[threadIdx.x / kWave] = cnt;
  __syncthreads();
  if (threadIdx.x == 0) {
    int t = 0;
    for (int w = 0; w < (int)(blockDim.x / kWave); ++w) t += s_cnt[w];
    row_active[s] = t;
  }
}

__global__ void cal_zero_kernel(float* __restrict__ p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0.0f;
}

__device__ inline float cal_tree(float v) {
#pragma unroll
  for (int s = kWave / 2; s >= 1; s >>= 1) v += __shfl_xor(v, s, kWave);
  return v;
}

// pred[s][n] = clamp(sigmoid(w_n . x_s + b_n)); lane l adds the products
// with (d mod 512) / 8 == l in increasing d (fmaf from +0.0), xor tree, then
// the bias.  BT samples x 8 gate rows per wave.
template <int BT>
__global__ __launch_bounds__(kCalWaves* kWave) void cal_forward_kernel(const float* __restrict__ x,
                                                                       const float* __restrict__ w,
                                                                       const float* __restrict__ b,
                                                                       float* __restrict__ pred, int64_t N,
                                                                       int64_t D, int64_t D_ffn) {
  const int lane = threadIdx.x % kWave;
  const int64_t n0 = ((int64_t)blockIdx.x * kCalWaves + threadIdx.x / kWave) * kCalRows;
  const int64_t s0 = (int64_t)blockIdx.y * BT;
  if (n0 >= D_ffn) return;
  const float* wr[kCalRows];
#pragma unroll
  for (int r = 0; r < kCalRows; ++r) wr[r] = w + (n0 + r < D_ffn ? n0 + r : D_ffn - 1) * D;
  const float* xr[BT];
#pragma unroll
  for (int t = 0; t < BT; ++t) xr[t] = x + (s0 + t < N ? s0 + t : N - 1) * D;
  float acc[kCalRows][BT];
#pragma unroll
  for (int r = 0; r < kCalRows; ++r)
#pragma unroll
    for (int t = 0; t < BT; ++t) acc[r][t] = 0.0f;
  for (int64_t c0 = 0; c0 < D; c0 += kCalChunk) {
    const int64_t d0 = c0 + 8 * lane;
    float xv[BT][8];
#pragma unroll
    for (int t = 0; t < BT; ++t)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int64_t dd = d0 + j;
        const float v = xr[t][dd < D ? dd : D - 1];
        xv[t][j] = dd < D ? v : 0.0f;
      }
#pragma unroll
    for (int r = 0; r < kCalRows; ++r) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int64_t dd = d0 + j;
        const float wv0 = wr[r][dd < D ? dd : D - 1];
        const float wv = dd < D ? wv0 : 0.0f;
#pragma unroll
        for (int t = 0; t < BT; ++t) acc[r][t] = fmaf(wv, xv[t][j], acc[r][t]);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < kCalRows; ++r)
#pragma unroll
    for (int t = 0; t < BT; ++t) acc[r][t] = cal_tree(acc[r][t]);
  if (lane < kCalRows * BT) {
    const int r = lane / BT, t = lane % BT;
    float v = acc[0][0];
#pragma unroll
    for (int rr = 0; rr < kCalRows; ++rr)
#pragma unroll
      for (int tt = 0; tt < BT; ++tt) v = (lane == rr * BT + tt) ? acc[rr][tt] : v;
    const int64_t n = n0 + r, s = s0 + t;
    if (n < D_ffn && s < N) {
      const float a = v + b[n];
      float p = static_cast<float>(1.0 / (1.0 + exp(-static_cast<double>(a))));
      p = fmaxf(1e-7f, fminf(1.0f - 1e-7f, p));
      pred[s * D_ffn + n] = p;
    }
  }
}

// One gradient step (gate_calibrate.cu:164-210): g = sum over samples, in
// order, of (pred - y) * x (fmaf from +0.0), divided by N, then
// w = fmaf(-lr, g, w); the bias the same with x = 1.
__global__ __launch_bounds__(256) void cal_update_kernel(const float* __restrict__ x,
                                                         const float* __restrict__ pred,
                                                         const uint8_t* __restrict__ masks, float* __restrict__ w,
                                                         float* __restrict__ b, int64_t N, int64_t D,
                                                         int64_t D_ffn) {
  const int64_t n = blockIdx.x;
  const int64_t d = (int64_t)blockIdx.y * blockDim.x + threadIdx.x;
  const bool bias_lane = blockIdx.y == 0 && threadIdx.x == 0;
  float gw = 0.0f, gb = 0.0f;
  const int64_t dc = d < D ? d : D - 1;
  for (int64_t s = 0; s < N; ++s) {
    const float e = pred[s * D_ffn + n] - (float)masks[s * D_ffn + n];
    gw = fmaf(e, x[s * D + dc], gw);
    gb += e;
  }
  const float fN = (float)N;
  if (d < D) w[n * D + d] = fmaf(-kCalLr, gw / fN, w[n * D + d]);
  if (bias_lane) b[n] = fmaf(-kCalLr, gb / fN, b[n]);
}

namespace {

// Scratch of the calibration call: masks, predictions and per-sample
// counts, in one per-device buffer that grows on demand (the call is
// blocking, as the reference's is, so the buffer is idle between calls).
struct CalDevice {
  void* buf = nullptr;
  size_t bytes = 0;
};
std::mutex g_cal_mutex;
CalDevice g_cal_dev[64];

size_t a256(size_t v) { return (v + 255) & ~(size_t)255; }

}  // namespace

}  // namespace pmoe

using namespace pmoe;

extern "C" {

PHANTOM_LEGACY_API int calibrate_sparsity_gate(const float* d_inputs, const float* d_mlp_activations, int N_samples,
                                               int D, int D_ffn, float* d_gate_w, float* d_gate_b, bool* h_enabled,
                                               float* h_f1_score, float* h_sparsity, hipStream_t stream) {
  if (!d_inputs || !d_mlp_activations || !d_gate_w || !d_gate_b || !h_enabled || !h_f1_score || !h_sparsity)
    return set_error(PHANTOM_MOE_EINVAL, "calibrate_sparsity_gate: every pointer must be non-null");
  if (N_samples < 1 || D < 1 || D_ffn < 1)
    return set_error(PHANTOM_MOE_EINVAL, "calibrate_sparsity_gate: need N_samples, D, D_ffn >= 1 (got %d, %d, %d)",
                     N_samples, D, D_ffn);
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &cap) == hipSuccess && cap != hipStreamCaptureStatusNone)
    return set_error(PHANTOM_MOE_EUNSUPPORTED, "calibrate_sparsity_gate waits for its results; not under capture");
  const int64_t N = N_samples, ND = (int64_t)N_samples * D_ffn;
  std::lock_guard<std::mutex> lock(g_cal_mutex);
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
    return set_error(PHANTOM_MOE_ELAUNCH, "calibrate_sparsity_gate: no current HIP device");
  CalDevice& cd = g_cal_dev[dev];
  const size_t o_mask = 0, o_pred = a256((size_t)ND), o_cnt = o_pred + a256(sizeof(float) * (size_t)ND);
  const size_t need = o_cnt + a256(sizeof(int32_t) * (size_t)N);
  if (cd.bytes < need) {
    if (cd.buf) (void)hipFree(cd.buf);
    cd.buf = nullptr;
    cd.bytes = 0;
    if (hipMalloc(&cd.buf, need) != hipSuccess)
      return set_error(PHANTOM_MOE_ELAUNCH, "calibrate_sparsity_gate: cannot allocate %zu bytes", need);
    cd.bytes = need;
  }
  uint8_t* masks = static_cast<uint8_t*>(cd.buf) + o_mask;
  float* pred = reinterpret_cast<float*>(static_cast<char*>(cd.buf) + o_pred);
  int32_t* cnt = reinterpret_cast<int32_t*>(static_cast<char*>(cd.buf) + o_cnt);

  hipError_t e = hipSuccess;
  hipLaunchKernelGGL(cal_mask_kernel, dim3((unsigned)N), dim3(256), 0, stream, d_mlp_activations, masks, cnt,
                     (int64_t)D_ffn);
  e = hipGetLastError();
  if (e == hipSuccess) {
    hipLaunchKernelGGL(cal_zero_kernel, dim3(1024), dim3(256), 0, stream, d_gate_w, (int64_t)D_ffn * D);
    hipLaunchKernelGGL(cal_zero_kernel, dim3(64), dim3(256), 0, stream, d_gate_b, (int64_t)D_ffn);
    e = hipGetLastError();
  }
  const int BT = N >= 8 ? 8 : (N >= 4 ? 4 : (N >= 2 ? 2 : 1));
  auto forward = [&]() -> hipError_t {
    const dim3 grid((unsigned)ceil_div(D_ffn, kCalWaves * kCalRows), (unsigned)ceil_div(N, BT));
    const dim3 block(kCalWaves * kWave);
    switch (BT) {
      case 8: hipLaunchKernelGGL(cal_forward_kernel<8>, grid, block, 0, stream, d_inputs, d_gate_w, d_gate_b, pred, N, (int64_t)D, (int64_t)D_ffn); break;
      case 4: hipLaunchKernelGGL(cal_forward_kernel<4>, grid, block, 0, stream, d_inputs, d_gate_w, d_gate_b, pred, N, (int64_t)D, (int64_t)D_ffn); break;
      case 2: hipLaunchKernelGGL(cal_forward_kernel<2>, grid, block, 0, stream, d_inputs, d_gate_w, d_gate_b, pred, N, (int64_t)D, (int64_t)D_ffn); break;
      default: hipLaunchKernelGGL(cal_forward_kernel<1>, grid, block, 0, stream, d_inputs, d_gate_w, d_gate_b, pred, N, (int64_t)D, (int64_t)D_ffn); break;
    }
    return hipGetLastError();
  };
  for (int ep = 0; ep < kCalEpochs && e == hipSuccess; ++ep) {
    e = forward();
    if (e == hipSuccess) {
      hipLaunchKernelGGL(cal_update_kernel, dim3((unsigned)D_ffn, (unsigned)ceil_div(D, 256)), dim3(256), 0, stream,
                         d_inputs, pred, masks, d_gate_w, d_gate_b, N, (int64_t)D, (int64_t)D_ffn);
      e = hipGetLastError();
    }
  }
  if (e == hipSuccess) e = forward();
  if (e != hipSuccess) return set_error(PHANTOM_MOE_ELAUNCH, "calibrate_sparsity_gate: %s", hipGetErrorString(e));

  // host side, as gate_calibrate.cu:260-270 and :314-334 compute it
  uint8_t* hm = static_cast<uint8_t*>(malloc((size_t)ND));
  float* hp = static_cast<float*>(malloc(sizeof(float) * (size_t)ND));
  int32_t* hc = static_cast<int32_t*>(malloc(sizeof(int32_t) * (size_t)N));
  if (!hm || !hp || !hc) {
    free(hm);
    free(hp);
    free(hc);
    return set_error(PHANTOM_MOE_ELAUNCH, "calibrate_sparsity_gate: host allocation failed");
  }
  e = hipMemcpyAsync(hm, masks, (size_t)ND, hipMemcpyDeviceToHost, stream);
  if (e == hipSuccess) e = hipMemcpyAsync(hp, pred, sizeof(float) * (size_t)ND, hipMemcpyDeviceToHost, stream);
  if (e == hipSuccess) e = hipMemcpyAsync(hc, cnt, sizeof(int32_t) * (size_t)N, hipMemcpyDeviceToHost, stream);
  if (e == hipSuccess) e = hipStreamSynchronize(stream);
  if (e != hipSuccess) {
    free(hm);
    free(hp);
    free(hc);
    return set_error(PHANTOM_MOE_ELAUNCH, "calibrate_sparsity_gate: %s", hipGetErrorString(e));
  }
  long long active_total = 0;
  for (int64_t s = 0; s < N; ++s) active_total += hc[s];
  const float baseline = 1.0f - (float)active_total / ((float)N_samples * D_ffn);
  *h_sparsity = baseline * 100.0f;
  long long tp = 0, fp = 0, fn = 0;
  for (int64_t i = 0; i < ND; ++i) {
    const bool pr = hp[i] >= 0.5f, ac = hm[i] > 0;
    if (pr && ac) ++tp;
    else if (pr && !ac) ++fp;
    else if (!pr && ac) ++fn;
  }
  const float precision = (tp + fp > 0) ? (float)tp / (float)(tp + fp) : 0.0f;
  const float recall = (tp + fn > 0) ? (float)tp / (float)(tp + fn) : 0.0f;
  const float f1 = (precision + recall > 0) ? 2.0f * precision * recall / (precision + recall) : 0.0f;
  *h_f1_score = f1;
  *h_enabled = f1 >= kCalF1Threshold;
  free(hm);
  free(hp);
  free(hc);
  clear_error();
  return PHANTOM_MOE_OK;
}

}  // extern "C"
