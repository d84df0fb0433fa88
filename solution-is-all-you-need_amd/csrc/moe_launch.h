// moe_launch.h -- host-side launch helpers and the workspace layout shared by
// the kernel translation units and the C ABI (capi.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace pmoe {

// Limits of this build (checked by the C ABI before any launch).
constexpr int kMaxExperts = 512;  // router top-k keeps E/64 <= 8 logits per lane
constexpr int kMaxTopK = 32;

// Token tiles: the permute cuts every segment into tiles of 16 positions and
// writes, per tile, {expert, first position, segment end, 0} followed by the
// token of each of the 16 positions (T, the all-zero activation row, past the
// segment end).  Routed segments come in expert order, the shared one last.
constexpr int kTileWords = 20;
constexpr int kCtlStride = 32;  // ints per 128-byte line: counters that atomics hit get a line each
inline int64_t max_token_tiles(int64_t T, int k, int E, int has_shared) {
  const int64_t nslots = T * k;
  return (nslots + 15) / 16 + (nslots < E ? nslots : E) + (has_shared ? (T + 15) / 16 : 0);
}

// ---- the single-launch decode layer (decode_fused.hip) ----------------------
// Limits of the shapes it takes (the others run the staged launches).
constexpr int kFusedMaxT = 8;
constexpr int kFusedMaxLogits = 2048;  // T * E
constexpr int kFusedMaxSlots = 256;    // T * k
// Dynamic LDS of one workgroup (the static part is about 8 KB of routing
// results; a CU has 160 KB).
constexpr size_t kFusedDynLdsMax = 148 * 1024;
constexpr int kFusedMaxGrid = 1024;  // workgroups (presence words)
// Status bits of workspace word 1 (phantom_moe_workspace_status).
constexpr uint32_t kStatusRouteWait = 1u;     // a workgroup gave up waiting for the logits
constexpr uint32_t kStatusExpertWait = 2u;    // a down workgroup gave up waiting for the h of gate/up
constexpr uint32_t kStatusPresenceWait = 4u;  // workgroup 0 gave up waiting for every workgroup's start
// Bytes at the start of every workspace: word 0 the generation counter of the
// single-launch path, word 1 the status bits.
constexpr size_t kCtlBytes = 256;

// Byte offsets of the dynamic LDS regions (decode_fused.hip).
struct FusedLds {
  uint32_t x, wgu, wdn;  // x operand, gate/up and down weight staging
  uint32_t route;        // routing scratch (over the staging, dead before the copies start)
  uint32_t h, dred;      // h operand and down partials (after the workgroup's gate/up work)
  uint32_t bytes;        // total
};
// Instantiations of the single-launch kernel: 0 reads the shape at run time;
// kFusedSpecQwen3T1 is compiled for T 1, H 2048, I 768, E 128, top-8, no
// shared expert (the batch-1 Qwen3-30B-A3B-shaped layer).
constexpr int kFusedSpecQwen3T1 = 1;
// The per-XCD batch-1 kernel (moe_decode_x8_kernel): one token, top-8, no
// shared expert, on a part with 8 XCDs of 32 CUs, expert slot j on XCD j;
// compiled for H 2048, I 768, E 128.
constexpr int kFusedSpecX8 = 2;
bool x8_shape(int64_t T, int64_t H, int64_t I, int E, int k, int has_shared);
struct FusedPlan {
  bool ok;
  int G;     // workgroups (one per CU)
  int spec;  // kernel instantiation
  FusedLds lds;
};
struct FusedWs {
  uint32_t* ctl = nullptr;       // workspace words 0 (generation) and 1 (status)
  uint64_t* presence = nullptr;  // [kFusedMaxGrid]
  uint32_t* slots = nullptr;     // [T * E][4] tagged logits
  uint32_t* hv = nullptr;        // [T*k + T][I / 2][4] tagged h units (fp16 hi/lo of two rows)
  // the per-XCD kernel's (null unless x8_shape)
  uint32_t* xslots = nullptr;  // [E] tagged logits, 256 bytes apart
  uint32_t* xh = nullptr;      // [8][I / 2][4] tagged h units
  uint32_t* xpart = nullptr;   // [8][H / 2][4] tagged down partials
  // the streaming one-token kernel's (null unless stream_shape_ok)
  uint32_t* sslots = nullptr;  // [E] tagged logits, kStreamSlotStride bytes apart
  uint32_t* sdv = nullptr;     // [k + shared][slices of I][H / 2][4] tagged expert output parts (hv holds h)
};
// Device-independent shape limits (the workspace plan reserves the fused
// regions for these shapes).
bool fused_shape_ok(int64_t T, int64_t H, int64_t I, int E, int k, int has_shared);
// The launch plan on the current device; .ok false means the staged launches.
FusedPlan fused_plan(int64_t T, int64_t H, int64_t I, int E, int k, int has_shared);
// The dynamic LDS layout for ng gate/up and nd down items per workgroup.
FusedLds fused_lds_layout(int T, int k, int E, int has_shared, int H, int I, int ng, int nd, int S_max);

// ---- the single-launch layer for one token with experts too large to stage
// whole (decode_stream.hip): every wave streams its weights through its own
// ring of direct-to-LDS copies.
constexpr uint32_t kStreamSlotStride = 128;  // bytes between its device-scope logit slots
struct StreamLds {
  uint32_t x, xs, lv, topk, h, red, ring;  // byte offsets: x operand, its sums, logits, top-k scratch, h, reduction, rings
  uint32_t ring_wave, bytes;              // ring bytes per wave, total
  int ns_gu, ns_dn;                       // ring stages (quads in flight) of gate/up and of down
  int yrows;                              // rows of y each workgroup combines
};
struct StreamPlan {
  bool ok;
  int G;   // workgroups (one per CU)
  int kx;  // slices of I a slot's down work is cut into (stream_kx)
  StreamLds lds;
};
// Device-independent shape limits (the workspace reserves its regions for them).
bool stream_shape_ok(int64_t T, int64_t H, int64_t I, int E, int k, int has_shared);
// Slices of I (quads KqI) a slot's down work is cut into: the workspace bound
// (device-independent), and the count on a device of G workgroups for S slots.
int stream_kx_max(int64_t KqI);
int stream_kx(int64_t KqI, int G, int S);
// The launch plan on the current device; .ok false means another path.
StreamPlan stream_plan(int64_t T, int64_t H, int64_t I, int E, int k, int has_shared);

// Library options: initialised once from the environment on first use,
// changed afterwards only by phantom_moe_set_option:
//   PHANTOM_MOE_DECODE=staged       never take the single-launch decode path
//   PHANTOM_MOE_DECODE_KSPLIT=1     decode expert stages always as the K-split
//                                   kernels (not the token-tile ones)
//   PHANTOM_MOE_DECODE_X8=0         batch-1 top-8 decode in the generic
//                                   single-launch kernel, not per XCD
struct LibConfig {
  bool decode_fused;
  bool decode_x8;  // batch-1 top-8 decode per XCD where the shape and the device allow
  bool force_ksplit;
  uint32_t fused_wait_polls;  // bound of each wait of the single-launch path
  int decode_stream;  // one-token streaming single launch: 0 off, 1 where no other single launch fits, 2 for every one-token shape
  uint32_t fused_fault;       // failure injection for tests: bit 0 the logit wait, bit 1 the gate/up wait,
                              // bit 2 the last workgroup reads the generation one ahead (a late start)
};
// Tuning overrides for sweeps, read from the environment once, on first use
// (0 = the shape-chosen value):
//   PHANTOM_MOE_GATE_UP_DEPTH=2..4, PHANTOM_MOE_DOWN_DEPTH=2|4|6   token-tile weight-ring depths
//   PHANTOM_MOE_GATE_UP_TILING / PHANTOM_MOE_DOWN_TILING = "waves,row_tiles,quads"   K-split tiling
struct Tuning {
  int gu_depth = 0, dn_depth = 0;
  int gu_tiling[3] = {0, 0, 0};
  int dn_tiling[3] = {0, 0, 0};
};
const Tuning& tuning();
// Each poll is one device-scope round trip plus a short sleep (about 1-2 us),
// so the default bound is far beyond any real wait; it only guarantees that
// every wave exits.
constexpr uint32_t kFusedWaitPollsDefault = 1u << 18;
LibConfig lib_config();
void set_lib_config(const LibConfig& c);
// Device address of the pinned host word the single-launch kernels store a
// status bit into when a wait gives up (null until phantom_moe_status_word
// has allocated it).
uint32_t* host_status_word();

// Workspace carve-up.  Every region is 256-byte aligned.
struct Workspace {
  uint32_t* ctl = nullptr;  // [kCtlBytes / 4]: generation, status
  FusedWs fused;            // regions of the single-launch path (null when the shape is not fused)
  double* logits = nullptr;         // [T, E]
  uint16_t* xq = nullptr;           // [T, Kpad_h] bf16 bits, MFMA operand order
  float* xs = nullptr;              // [T, Kpad_h / 32] group sums of x
  int32_t* offsets = nullptr;       // [E + 2] segment offsets (+ shared segment)
  int32_t* active = nullptr;        // [E + 1] active expert ids, ascending (+ shared = E)
  int32_t* n_active = nullptr;      // [1]
  int32_t* sorted_slots = nullptr;  // [T * k]
  int32_t* slot_pos = nullptr;      // [T * k]
  int4* desc = nullptr;             // [E + 1] {expert, begin, end, 0} per active segment
  int32_t* seg_tok = nullptr;       // [T * k + T] token of each segment position
  int32_t* tiles = nullptr;         // [max_token_tiles][kTileWords] 16-position tiles of the segments
  int32_t* n_tiles = nullptr;       // [kCtlStride]: word 0 the token tile count
  uint16_t* hq = nullptr;          // [rows, Kpad_I * 2] fp16 hi/lo of h, MFMA operand order
  float* hs = nullptr;             // [rows, Kpad_I / 32, 2] half-group sums of h
  float* outbuf = nullptr;          // [T*k + T*shared, H] expert outputs, segment order
  int32_t* counter = nullptr;       // [1] router hand-off counter (reset by every route launch)
  int32_t* perm_cnt = nullptr;      // [E][perm_blocks(T * k)] per-chunk expert counts, then bases (large batches)
  int32_t* perm_tb = nullptr;       // [E] first token tile of each expert (large batches)
  float* approx = nullptr;          // [T * E + T + E] approximate logits, |x_t|, |w_e| (two-pass router)
  uint8_t* cand = nullptr;          // [E * T] candidate flags, expert-major (two-pass router)
};

// Batches of at least this many slots use the many-workgroup permute.
constexpr int64_t kPermMultiSlots = 8192;
inline int64_t perm_blocks(int64_t n) {
  const int64_t b = (n + 1023) / 1024;
  return b < 4096 ? (b < 1 ? 1 : b) : 4096;
}

// The thread-local message behind phantom_moe_last_error(): set_error
// formats it and returns `code`; clear_error empties it.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

size_t plan_workspace(int64_t T, int64_t H, int64_t I, int E, int k, int has_shared, void* base,
                      Workspace* ws);

// Router tiling: tokens per logits workgroup tile.
int router_token_tile(int64_t T);
// Batches routed in two passes (approximate logits with an error bound, then
// the exact logits of the candidates): bf16 x, T >= 128, E >= 16.  The
// workspace holds their regions (approx, cand) whenever T and E qualify.
constexpr int64_t kTwoPassMinT = 128;
inline bool two_pass_shape(int64_t T, int E) { return T >= kTwoPassMinT && E >= 16; }
inline bool two_pass_route(int64_t T, int E, int x_dtype) { return x_dtype == 0 && two_pass_shape(T, E); }

hipError_t launch_q4_repack(const uint8_t* src, int64_t rows, int64_t K, uint8_t* nib,
                            uint16_t* scale, hipStream_t stream);
hipError_t launch_q4_unrepack(const uint8_t* nib, const uint16_t* scale, int64_t rows, int64_t K,
                              uint8_t* dst, hipStream_t stream);
hipError_t launch_q4_dequant_f32(const uint8_t* src, int64_t n_blocks, float* out,
                                 hipStream_t stream);

// Logits (+ optional MFMA-ordered copy of x and its group sums), top-k, and
// optionally the permute: two launches up to 64 tokens (the permute runs in
// the select launch), three beyond.
struct RouteArgs {
  const void* x;
  int x_dtype;
  const float* router_w;
  const float* router_bias;
  int64_t T, H;
  int E, k, score_mode;
  int32_t* topk_idx;
  float* topk_w;
  bool prep_x;       // write ws.xq / ws.xs
  bool prep_fp16;    // ws.xq as fp16 (GEMM regime) instead of bf16 (GEMV regime)
  bool do_permute;   // write offsets / sorted_slots / slot_pos / active
  int has_shared;    // append the shared-expert segment to offsets / active
  bool want_tiles;   // write ws.tiles / ws.n_tiles (the token-tile gate/up kernel reads them)
  int32_t* offsets_out;       // optional user copy of offsets [E+1]
  int32_t* sorted_slots_out;  // where to write sorted slots (default ws)
  int32_t* slot_pos_out;      // where to write slot positions (default ws)
};
hipError_t launch_route(const RouteArgs& a, const Workspace& ws, hipStream_t stream);

// Permute only (topk_idx given).
hipError_t launch_permute(const int32_t* topk_idx, int64_t T, int k, int E, int has_shared,
                          int32_t* offsets, int32_t* sorted_slots, int32_t* slot_pos,
                          const Workspace& ws, hipStream_t stream);

struct ExpertArgs {
  int64_t T, H, I;
  int E, k, has_shared;
  const uint8_t* gate_nib;
  const uint16_t* gate_scale;
  const uint8_t* up_nib;
  const uint16_t* up_scale;
  const uint8_t* down_nib;
  const uint16_t* down_scale;
  const uint8_t* sh_gate_nib;
  const uint16_t* sh_gate_scale;
  const uint8_t* sh_up_nib;
  const uint16_t* sh_up_scale;
  const uint8_t* sh_down_nib;
  const uint16_t* sh_down_scale;
  const float* topk_w;
  float* y;
};
// Prefill regime: when the average segment holds at least this many slots,
// the expert stages run as grouped MFMA GEMMs (expert_gemm.hip) on fp16
// operands; below it, as the grouped GEMV (expert_ffn.hip).
constexpr int kGemmMinSlotsPerExpert = 64;
bool gemm_regime(int64_t T, int k, int E);
hipError_t launch_gemm_gate_up(const ExpertArgs& a, const Workspace& ws, hipStream_t stream);
hipError_t launch_gemm_down(const ExpertArgs& a, const Workspace& ws, hipStream_t stream);

// Whether the decode-regime gate/up stage runs as the token-tile kernel (which
// needs the permute's token tiles) for this shape.
bool gate_up_tile_regime(int64_t T, int64_t H, int64_t I, int E, int k, int has_shared);
// The same for the down stage.
bool down_tile_regime(int64_t T, int64_t H, int64_t I, int E, int k, int has_shared);

// The whole layer in one launch (decode_fused.hip); plan from fused_plan.
hipError_t launch_decode_stream(const StreamPlan& pl, const RouteArgs& r, const ExpertArgs& x, const FusedWs& ws,
                                hipStream_t stream);
hipError_t launch_decode_fused(const FusedPlan& pl, const RouteArgs& r, const ExpertArgs& x, const FusedWs& ws,
                               hipStream_t stream);

// The three expert stages; launch_experts runs them back to back.
hipError_t launch_gate_up(const ExpertArgs& a, const Workspace& ws, hipStream_t stream);
hipError_t launch_down(const ExpertArgs& a, const Workspace& ws, hipStream_t stream);
hipError_t launch_combine(const ExpertArgs& a, const Workspace& ws, hipStream_t stream);
hipError_t launch_experts(const ExpertArgs& a, const Workspace& ws, hipStream_t stream);

}  // namespace pmoe
