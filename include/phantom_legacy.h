/*
 * phantom_legacy.h -- the reference's neuron-sparse FFN C ABI, on gfx950
 * (exported by libphantom_moe.so next to the MoE-layer ABI of phantom_moe.h).
 *
 * The three symbols keep the reference's names, parameter order, argument
 * meaning and float return value, so a caller written against
 * kernels/sparse_moe/ links unchanged; the stream is a hipStream_t where the
 * reference takes a cudaStream_t.  fp16 tensors are passed as pointers to
 * their 16-bit patterns (phantom_half).
 *
 *   sparse_mlp_forward      kernels/sparse_moe/sparse_matmul.cu:240-255
 *   predict_active_neurons  kernels/sparse_moe/gate_predict.cu:200-213
 *   get_sparsity_stats      kernels/sparse_moe/gate_predict.cu:253-258
 *   calibrate_sparsity_gate kernels/sparse_moe/gate_calibrate.cu:228-240
 *
 * Behaviour kept from the reference:
 *   - sparse_mlp_forward and predict_active_neurons time themselves with two
 *     events on the stream, wait for the second and return the elapsed
 *     milliseconds (kernels/common/cuda_utils.h:235-260).  Under stream
 *     capture they record nothing, do not wait, and return 0.
 *   - sparse_mlp_forward takes the dense branch when sparsity_pct / 100 is
 *     below 0.30 (sparse_matmul.cu:29, :259-305): every neuron, gate and up
 *     biases ignored, the active lists ignored.  Otherwise it computes the
 *     list positions below min(active_count[b], C), where C is the launch
 *     coverage of the reference's grid, C = ceil(M / 256) * 256 with
 *     M = min((int)((1 - sparsity_pct/100) * D_ffn) + 32, D_ffn)
 *     (sparse_matmul.cu:320-333); the down projection then sums over all
 *     active_count[b] list entries, the uncovered ones contributing zero.
 *   - get_sparsity_stats copies the counts to the host, waits for the
 *     stream and returns (1 - mean(count) / D_ffn) * 100 in fp32.
 *
 * Differences, all supersets or replacements of process exit:
 *   - On invalid arguments or a failed launch the functions return a
 *     negative value, the PHANTOM_MOE_E* status of phantom_moe.h as a float
 *     (-1 invalid argument, -3 launch or runtime failure, -4 unsupported),
 *     and set phantom_moe_last_error(); the reference prints and exits
 *     (cuda_utils.h:31-52).  get_sparsity_stats with B = 0 returns NaN, as
 *     the reference's 0/0 does.
 *   - A NULL bias reads as zero; a NULL d_gate_output is not written.
 *   - Active indices outside [0, D_ffn) are skipped; counts are clamped to
 *     [0, D_ffn].
 *   - No allocation per call: the fp16 activation vector of
 *     sparse_mlp_forward lives in per-device buffers that grow on demand
 *     (allocation happens only when a larger B * D_ffn is first seen, and
 *     never under stream capture).  Eager calls and calls recorded under
 *     stream capture use separate buffers; every eager call reserves both at
 *     its size, and a capture at a size no eager call has reserved returns
 *     -4 (unsupported).  A buffer a captured graph holds is never freed
 *     while the process runs, so graphs stay valid across later, larger
 *     eager calls.  Calls run one at a time per process; replays of graphs
 *     that hold sparse_mlp_forward share one buffer per device, so they must
 *     not overlap one another (they may overlap eager calls).
 *
 * Arithmetic (the reference accumulates each dot product sequentially in
 * fp32; this build uses a fixed parallel order with the same fp32 rounding
 * per addition, so results agree to fp32 rounding, which the fp16 outputs
 * mostly absorb):
 *   - fp16 x fp16 products are exact in fp32.  Dot products over D: 64
 *     partial sums, partial l adding, in increasing d and from +0.0, the
 *     products with (d mod 512) / 8 == l; partials combined by
 *     p[l] += p[l xor s] for s = 32, 16, 8, 4, 2, 1; then the bias added.
 *   - Down projection: over the columns n of W_down, weighting act[n] by
 *     m_n, the number of times n appears among the first active_count[b]
 *     list entries (1 for every n in the dense branch); columns with m_n = 0
 *     are skipped; partial l takes fmaf(W[d, n], m_n * act[n], .) for
 *     (n mod 512) / 8 == l in increasing n, same tree.  In exact arithmetic
 *     this is the reference's sum over list entries, duplicates included.
 *   - sigmoid(a) = (float)(1 / (1 + exp(-(double)a))); silu and the SwiGLU
 *     product in fp32 as sparse_matmul.cu:141-145; fp16 stores round to
 *     nearest even.
 */
#ifndef PHANTOM_LEGACY_H
#define PHANTOM_LEGACY_H

#include <stdbool.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#define PHANTOM_LEGACY_API __attribute__((visibility("default")))

#ifdef __cplusplus
extern "C" {
#endif

typedef uint16_t phantom_half; /* IEEE binary16 bit pattern */

/* y[b] = W_down (silu(W_g x[b] + b_g) * (W_u x[b] + b_u)) over the active
 * neurons of row b.  d_input [B, D]; d_gate_weight, d_up_weight [D_ffn, D];
 * biases [D_ffn]; d_down_weight [D, D_ffn]; d_active_indices [B, D_ffn]
 * (row stride D_ffn, first active_count[b] entries used); d_active_count [B];
 * d_output [B, D].  All fp16 except the int32 lists.
 * Replaces kernels/sparse_moe/sparse_matmul.cu:240-365. */
PHANTOM_LEGACY_API float sparse_mlp_forward(const phantom_half* d_input, const phantom_half* d_gate_weight,
                                            const phantom_half* d_gate_bias, const phantom_half* d_up_weight,
                                            const phantom_half* d_up_bias, const phantom_half* d_down_weight,
                                            const int* d_active_indices, const int* d_active_count,
                                            phantom_half* d_output, int B, int D, int D_ffn, float sparsity_pct,
                                            hipStream_t stream);

/* gate[b, n] = sigmoid(W_gate[n] . x[b] + bias[n]) (fp32, to d_gate_output);
 * mask[b, n] = gate >= threshold; d_active_indices[b, 0 .. count-1] = the
 * active n in increasing order; d_active_count[b] = count.
 * Replaces kernels/sparse_moe/gate_predict.cu:49-88, :153-177, :200-242. */
PHANTOM_LEGACY_API float predict_active_neurons(const phantom_half* d_input, const phantom_half* d_gate_weights,
                                                const phantom_half* d_gate_bias, uint8_t* d_active_mask,
                                                int* d_active_indices, int* d_active_count, float* d_gate_output,
                                                int B, int D, int D_ffn, float threshold, hipStream_t stream);

/* Mean sparsity in percent over the B counts (blocks on the stream).
 * Replaces kernels/sparse_moe/gate_predict.cu:253-271. */
PHANTOM_LEGACY_API float get_sparsity_stats(const int* d_active_count, int B, int D_ffn, hipStream_t stream);

/* Trains the predictor gates of one FFN layer (blocks on the stream).
 * d_inputs [N, D] fp32, d_mlp_activations [N, D_ffn] fp32; writes
 * d_gate_w [D_ffn, D] and d_gate_b [D_ffn] (fp32, device) and, on the host,
 * *h_enabled (F1 >= 0.70), *h_f1_score and *h_sparsity (percent of inactive
 * neurons).  A neuron is active on a sample when |activation| >= 0.01 *
 * max(row max |activation|, 1e-10); the gates start at zero and take 50
 * full-batch gradient steps of binary cross-entropy at lr 1e-3; F1 compares
 * gate >= 0.5 with the masks.  Arithmetic: the forward dot products in the
 * fixed order above with fmaf on fp32 operands, then the bias; gradients
 * summed over samples in order with fmaf, divided by N, applied as
 * w = fmaf(-lr, g, w); the sigmoid as above, clamped to [1e-7, 1 - 1e-7].
 * Returns 0 or a negative PHANTOM_MOE_E* status; the reference returns void
 * (so its callers ignore the status), prints progress and exits on error.
 * Replaces kernels/sparse_moe/gate_calibrate.cu:228-340. */
PHANTOM_LEGACY_API int calibrate_sparsity_gate(const float* d_inputs, const float* d_mlp_activations, int N_samples,
                                               int D, int D_ffn, float* d_gate_w, float* d_gate_b, bool* h_enabled,
                                               float* h_f1_score, float* h_sparsity, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* PHANTOM_LEGACY_H */
