/*
 * phantom_moe.h -- C ABI of the MI355X (gfx950) sparse-MoE layer library
 * (libphantom_moe.so).
 *
 * All pointers are device pointers unless stated otherwise; every entry point
 * is asynchronous on the caller's stream, performs no device allocation and
 * no host synchronisation, and returns 0 on success or a negative
 * PHANTOM_MOE_E* status (the message is available from
 * phantom_moe_last_error()).  Nothing here exits or aborts the process.
 *
 * Reference interfaces replaced (paths relative to the reference repository):
 *   - the router module PhantomTopKRouter.forward
 *       tests/test_moe_routing.py:43-72
 *   - the Q4_0 block format and its dequantisation
 *       python/phantom/loader/gguf_loader.py:72, :362-381, :588-596
 *   - the sparse SwiGLU FFN operator C ABI
 *       kernels/sparse_moe/sparse_matmul.cu:240-255 (sparse_mlp_forward)
 *   - the active-set compaction
 *       kernels/sparse_moe/gate_predict.cu:153-177, :200-213
 *   - the expert combine, which the reference delegates to transformers'
 *     MoE blocks (python/phantom/phantom_cli.py:1393-1430)
 *
 * Data formats
 *   x            [T, H] bf16 (x_dtype 0) or fp32 (x_dtype 1), row major.
 *   router_w     [E, H] fp32 (nn.Linear weight layout: out x in).
 *   router_bias  [E] fp32 or NULL; added to the logit before selection.
 *   Q4_0         GGUF Q4_0 rows: each row of K weights is K/32 blocks of
 *                18 bytes (fp16 scale d, then 16 bytes; byte j holds
 *                element j in its low nibble and element j+16 in its high
 *                nibble; value = (nibble - 8) * d).
 *   repacked     the device layout produced by phantom_q4_0_repack: rows are
 *                grouped 16 at a time and K is padded to a multiple of 128;
 *                "nib" holds the nibble bytes (rows * Kpad / 2 bytes) in the
 *                order the gfx950 MFMA operand loads consume them, "scale"
 *                holds the fp16 scales (rows * Kpad / 32 values).
 *                Stacked experts are stored back to back.
 */
#ifndef PHANTOM_MOE_H
#define PHANTOM_MOE_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#define PHANTOM_MOE_API __attribute__((visibility("default")))

#ifdef __cplusplus
extern "C" {
#endif

#define PHANTOM_MOE_OK 0
#define PHANTOM_MOE_EINVAL (-1)   /* bad shape, dtype, mode or null pointer */
#define PHANTOM_MOE_EWORKSPACE (-2) /* workspace missing or too small */
#define PHANTOM_MOE_ELAUNCH (-3)  /* a HIP launch or runtime call failed */
#define PHANTOM_MOE_EUNSUPPORTED (-4) /* valid but outside this build's limits */

#define PHANTOM_MOE_X_BF16 0
#define PHANTOM_MOE_X_F32 1

#define PHANTOM_MOE_SCORE_SOFTMAX 0 /* softmax over the k selected logits */
#define PHANTOM_MOE_SCORE_SIGMOID 1 /* sigmoid(l_j) / sum_i sigmoid(l_i) over the k */

/* Message describing the most recent failure on the calling thread. */
PHANTOM_MOE_API const char* phantom_moe_last_error(void);

/* Library version string. */
PHANTOM_MOE_API const char* phantom_moe_version(void);

/* Stage timing.  With a non-null array of PHANTOM_MOE_PROFILE_EVENTS events
 * set on the calling thread, phantom_moe_forward records events[0] before the
 * router, [1] before gate/up, [2] before down, [3] before the combine and
 * [4] after it, on the call's stream (no synchronisation).  The gate/up and
 * down stages are one kernel each, so [1]-[2] and [2]-[3] bracket single
 * launches.  The array is read by every later call on the thread, so it must
 * stay valid until it is replaced or cleared; NULL turns timing off.  The
 * non-blocking counterpart of the reference's per-call CudaTimer
 * (kernels/common/cuda_utils.h:235-260, used at sparse_matmul.cu:256-257). */
#define PHANTOM_MOE_PROFILE_EVENTS 5
PHANTOM_MOE_API int phantom_moe_set_profile_events(hipEvent_t* events, int n_events);

/* Names of the kernels phantom_moe_forward launches for the gate/up and down
 * stages at this shape, as "gate_up=<kernel>;down=<kernel>" (thread-local
 * storage, valid until the next call on the thread), so a profile can be
 * matched to its launches.  Diagnostic only: no counterpart in the reference. */
PHANTOM_MOE_API const char* phantom_moe_expert_kernels(int64_t T, int64_t H, int64_t I, int E, int top_k,
                                                       int has_shared);

/* ---------------------------------------------------------------- */
/* Q4_0 repack                                                       */
/* ---------------------------------------------------------------- */

/* Bytes of the repacked nibble and scale buffers for a [rows, K] Q4_0
 * matrix (rows % 16 == 0, K % 32 == 0); -1 on invalid shape. */
PHANTOM_MOE_API int64_t phantom_q4_0_nib_bytes(int64_t rows, int64_t K);
PHANTOM_MOE_API int64_t phantom_q4_0_scale_bytes(int64_t rows, int64_t K);

/* GGUF Q4_0 bytes [rows, K/32, 18] -> repacked (nib, scale).  Lossless.
 * Replaces the load-time dequantisation of gguf_loader.py:362-381 /
 * :588-596: weights stay 4-bit in HBM and are expanded in registers. */
PHANTOM_MOE_API int phantom_q4_0_repack(const uint8_t* q4_0, int64_t rows, int64_t K, uint8_t* nib, uint16_t* scale,
                        hipStream_t stream);

/* Inverse of phantom_q4_0_repack: reproduces the original bytes exactly. */
PHANTOM_MOE_API int phantom_q4_0_unrepack(const uint8_t* nib, const uint16_t* scale, int64_t rows, int64_t K,
                          uint8_t* q4_0, hipStream_t stream);

/* Q4_0 bytes -> fp32 values [rows, K] (the arithmetic of
 * gguf_loader.py:369-378, kept in fp32 instead of the bf16 cast at :380). */
PHANTOM_MOE_API int phantom_q4_0_dequant_f32(const uint8_t* q4_0, int64_t rows, int64_t K, float* out,
                             hipStream_t stream);

/* ---------------------------------------------------------------- */
/* Router, permute, layer                                            */
/* ---------------------------------------------------------------- */

/* Workspace bytes needed by phantom_moe_route / _permute / _forward for
 * these sizes.  The workspace must be 256-byte aligned and must not be used
 * by calls that may run concurrently.  Zero-fill it once before its first
 * use (hipMemset, torch.zeros) and leave it to the library afterwards: its
 * first 256 bytes keep a call counter that the single-launch decode path
 * (below) derives its hand-off tags from, so no later call needs a memset;
 * everything else is per-call scratch.  (A workspace that was never zeroed
 * still works; only a 2^-32-per-word chance remains that stale bytes pass
 * for a tag on its first call.) */
PHANTOM_MOE_API size_t phantom_moe_workspace_bytes(int64_t T, int64_t H, int64_t I, int E, int top_k, int has_shared);

/* Status bits that the single-launch decode path left in this workspace
 * (0: every call since the last query completed normally; bit 0: a
 * workgroup gave up waiting for the router logits, bit 1 for the gate/up
 * results or the down partials, bit 2 for every workgroup to start).  A call that sets a bit
 * also writes NaN to the outputs it could not compute.  Waits for the
 * stream, clears the bits, and must not be captured into a graph.  No
 * counterpart in the reference, whose errors exit the process
 * (kernels/common/cuda_utils.h:31-52). */
PHANTOM_MOE_API int phantom_moe_workspace_status(void* workspace, size_t workspace_bytes, uint32_t* status,
                                                 hipStream_t stream);

/* A process-wide pinned host word (hipHostMalloc, mapped, coherent; 256
 * bytes, allocated on the first call and kept until the process ends) into
 * which every later launch of the single-launch decode path stores a
 * non-zero status bit when one of its waits gives up, as it also sets the
 * workspace's bits.  The host reads it with a plain load, without
 * synchronising, and writes 0 to clear it: a failure of any earlier call
 * (graph replays included) becomes visible at the next check, where
 * phantom_moe_workspace_status would have to wait for the stream.  Launches
 * made before the first call do not write it.  Returns null (and sets
 * phantom_moe_last_error) if the allocation fails.  No counterpart in the
 * reference, whose errors exit the process (kernels/common/cuda_utils.h:31-52). */
PHANTOM_MOE_API uint32_t* phantom_moe_status_word(void);

/* Library options (process-wide; initialised from the environment on first
 * use: PHANTOM_MOE_DECODE=staged, PHANTOM_MOE_DECODE_KSPLIT=1,
 * PHANTOM_MOE_DECODE_X8=0, PHANTOM_MOE_DECODE_STREAM=0|2).  A/B and
 * test switches with no counterpart in the reference. */
#define PHANTOM_MOE_OPT_DECODE_FUSED 1 /* 1: decode batches that fit take the single-launch path (default) */
#define PHANTOM_MOE_OPT_DECODE_KSPLIT 2 /* 1: staged decode expert stages always as the K-split kernels (default 0) */
#define PHANTOM_MOE_OPT_FUSED_WAIT_POLLS 3 /* bound of each wait of the single-launch path (default 2^18 polls) */
/* Failure injection for tests of the error path: bit 0 makes the logit wait,
 * bit 1 the gate/up wait, expect a tag nobody writes, so it gives up after
 * FUSED_WAIT_POLLS polls (every wave still exits; outputs NaN, status set);
 * bit 2 makes the last workgroup read the generation counter one ahead, as a
 * workgroup that starts after workgroup 0 gave up waiting for it would (it
 * must still take its own launch's tag: outputs unchanged, no status). */
#define PHANTOM_MOE_OPT_FUSED_FAULT 4
/* 1: a batch-1, top-8 decode without a shared expert (compiled for H 2048,
 * I 768, E 128) runs with expert slot j on XCD j of an 8-XCD, 256-CU part
 * (default); 0: in the generic single-launch kernel. */
#define PHANTOM_MOE_OPT_DECODE_X8 5
/* The one-token layer as one launch that streams the weights (experts too
 * large for the single launch above, e.g. Mixtral-8x7B- or
 * DeepSeek-V3-shaped): 1 where no other single launch fits (default), 2 for
 * every one-token shape (in place of the kernels above), 0 never. */
#define PHANTOM_MOE_OPT_DECODE_STREAM 6
PHANTOM_MOE_API int phantom_moe_set_option(int option, int value);
PHANTOM_MOE_API int phantom_moe_get_option(int option, int* value);

/* Router: logits = x W^T (+ bias) under the fixed-order fp64 contract,
 * top-k descending with ties to the lower expert index, weights by
 * score_mode.  Replaces PhantomTopKRouter.forward
 * (tests/test_moe_routing.py:56-72).  A NaN logit ranks below every number,
 * -inf included (torch.topk in the reference ranks NaN above every number);
 * -0 ties +0.  Outputs topk_idx [T, top_k] int32 and topk_w [T, top_k] fp32. */
PHANTOM_MOE_API int phantom_moe_route(const void* x, int x_dtype, const float* router_w, const float* router_bias,
                      int64_t T, int64_t H, int E, int top_k, int score_mode, int32_t* topk_idx,
                      float* topk_w, void* workspace, size_t workspace_bytes, hipStream_t stream);

/* Stable counting sort of the T*top_k (token, slot) pairs by expert.
 * expert_offsets [E+1]: exclusive prefix sum of per-expert counts;
 * sorted_slots [T*top_k]: slot ids s = t*top_k + j in (expert, s) order;
 * slot_pos [T*top_k]: inverse permutation.  The device-side analogue of the
 * compaction in kernels/sparse_moe/gate_predict.cu:153-177, made parallel and
 * deterministic. */
PHANTOM_MOE_API int phantom_moe_permute(const int32_t* topk_idx, int64_t T, int top_k, int E, int32_t* expert_offsets,
                        int32_t* sorted_slots, int32_t* slot_pos, void* workspace,
                        size_t workspace_bytes, hipStream_t stream);

/* The whole MoE layer:
 *   y[t] = sum_j w[t,j] * W_down_e (silu(W_gate_e x_t) * (W_up_e x_t)) + shared(x_t)
 * with e = topk_idx[t,j].  x must be bf16.  Expert weights are repacked Q4_0:
 * gate/up are E stacked [I, H] matrices, down E stacked [H, I] matrices.
 * The sh_* pointers describe one always-on shared expert of the same shapes
 * (weight 1.0), or are all NULL.  Outputs: y [T, H] fp32, topk_idx, topk_w.
 * The FFN operator semantics follow kernels/sparse_moe/sparse_matmul.cu:120-215
 * (SwiGLU, fp32 math) with 4-bit weights.
 * Decode batches of a few tokens whose experts fit its register and LDS
 * budgets (the batch-1 Qwen3-shaped layer among them) run as ONE kernel:
 * router, top-k, permute, gate/up, down and combine without returning to the
 * host, replacing the launch-per-stage structure of sparse_matmul.cu:256-363;
 * other shapes run router, gate/up, down and combine as separate launches.
 * Both give the same routing (bit for bit) and outputs within the layer
 * tolerance.  The single launch is a persistent grid of one workgroup per
 * CU whose workgroups wait on each other, so it needs every workgroup
 * resident at once: the GPU must not be shared with other work (other
 * streams or processes holding CUs, CU masks) while it runs.  It is launched
 * as an ordinary kernel (so it can be captured into a graph); if workgroups
 * are not co-resident, the bounded waits give up, the outputs they own are
 * NaN, and the status bits are set in the workspace and in the word of
 * phantom_moe_status_word.  PHANTOM_MOE_DECODE=staged (or the option
 * PHANTOM_MOE_OPT_DECODE_FUSED) turns the single launch off.  Alignment: nibble buffers 16 bytes, scale buffers 8, x 8,
 * router_w 16, workspace 256.  Below 64 positions per expert (the decode
 * regime), T * ceil(I / 128) * 512 must stay under 2^31 (one expert
 * segment's down operand), else PHANTOM_MOE_EUNSUPPORTED. */
PHANTOM_MOE_API int phantom_moe_forward(const void* x, int x_dtype, int64_t T, int64_t H, int64_t I, int E, int top_k,
                        int score_mode, const float* router_w, const float* router_bias,
                        const uint8_t* gate_nib, const uint16_t* gate_scale, const uint8_t* up_nib,
                        const uint16_t* up_scale, const uint8_t* down_nib, const uint16_t* down_scale,
                        const uint8_t* sh_gate_nib, const uint16_t* sh_gate_scale,
                        const uint8_t* sh_up_nib, const uint16_t* sh_up_scale,
                        const uint8_t* sh_down_nib, const uint16_t* sh_down_scale, float* y,
                        int32_t* topk_idx, float* topk_w, void* workspace, size_t workspace_bytes,
                        hipStream_t stream);

/* phantom_moe_forward without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  The
 * scratch is a 16 MiB array in the library's device memory, one per GPU,
 * held until the process ends; the call allocates nothing.  Sizes whose
 * workspace (phantom_moe_workspace_bytes) exceeds 16 MiB return
 * PHANTOM_MOE_EWORKSPACE -- with H 2048, I 768, E 128, top-8 that is
 * T <= 128 tokens.  Every call on one GPU shares that GPU's array, so calls
 * that may overlap on one GPU (different streams without ordering between
 * them) race and must not be issued.  The workspace status of the
 * single-launch path is not readable here: a wait that gives up shows as NaN
 * outputs (and topk_idx -1 when the routing was lost), and in the word of
 * phantom_moe_status_word once that has been called. */
PHANTOM_MOE_API int phantom_moe_forward_static(const void* x, int x_dtype, int64_t T, int64_t H, int64_t I, int E,
                                               int top_k, int score_mode, const float* router_w,
                                               const float* router_bias, const uint8_t* gate_nib,
                                               const uint16_t* gate_scale, const uint8_t* up_nib,
                                               const uint16_t* up_scale, const uint8_t* down_nib,
                                               const uint16_t* down_scale, const uint8_t* sh_gate_nib,
                                               const uint16_t* sh_gate_scale, const uint8_t* sh_up_nib,
                                               const uint16_t* sh_up_scale, const uint8_t* sh_down_nib,
                                               const uint16_t* sh_down_scale, float* y, int32_t* topk_idx,
                                               float* topk_w, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* PHANTOM_MOE_H */
