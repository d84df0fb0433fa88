// capi.hip -- extern "C" entry points of libphantom_moe.so (declared in
// include/phantom_moe.h).  Validates every argument on the host, carves the
// caller's workspace, and launches the kernels asynchronously on the caller's
// stream.  Never allocates, synchronises, exits or aborts: the reference's
// CUDA_CHECK exits the process on error (kernels/common/cuda_utils.h:31-52)
// and its host API blocks on a timer event (cuda_utils.h:253-257); here every
// failure is a return code plus a thread-local message.
#include <stdarg.h>

#include <atomic>
#include <mutex>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "moe_common.h"
#include "moe_launch.h"
#include "phantom_moe.h"

namespace {

thread_local char g_err[512] = "";

// Optional stage events (phantom_moe_set_profile_events), per thread.
thread_local hipEvent_t* g_prof_events = nullptr;

hipError_t record_stage(int i, hipStream_t stream) {
  if (!g_prof_events) return hipSuccess;
  return hipEventRecord(g_prof_events[i], stream);
}

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int ok() {
  g_err[0] = '\0';
  return PHANTOM_MOE_OK;
}

int launch_status(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(PHANTOM_MOE_ELAUNCH, "%s: %s", what, hipGetErrorString(e));
  return ok();
}

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

int check_route_shapes(const void* x, int x_dtype, const float* router_w, int64_t T, int64_t H,
                       int E, int top_k, int score_mode) {
  if (!x || !router_w) return fail(PHANTOM_MOE_EINVAL, "x and router_w must be non-null");
  if (x_dtype != PHANTOM_MOE_X_BF16 && x_dtype != PHANTOM_MOE_X_F32)
    return fail(PHANTOM_MOE_EINVAL, "x_dtype must be 0 (bf16) or 1 (fp32), got %d", x_dtype);
  if (T < 1) return fail(PHANTOM_MOE_EINVAL, "T must be >= 1, got %lld", (long long)T);
  if (T > (int64_t)1 << 24) return fail(PHANTOM_MOE_EUNSUPPORTED, "T above 2^24 is not supported");
  if (H < 32 || H % 32) return fail(PHANTOM_MOE_EINVAL, "H must be a positive multiple of 32, got %lld", (long long)H);
  if (E < 1 || E > pmoe::kMaxExperts)
    return fail(E < 1 ? PHANTOM_MOE_EINVAL : PHANTOM_MOE_EUNSUPPORTED, "E must be in [1, %d], got %d",
                pmoe::kMaxExperts, E);
  if (top_k < 1 || top_k > E) return fail(PHANTOM_MOE_EINVAL, "top_k must be in [1, E=%d], got %d", E, top_k);
  if (top_k > pmoe::kMaxTopK)
    return fail(PHANTOM_MOE_EUNSUPPORTED, "top_k above %d is not supported", pmoe::kMaxTopK);
  if (score_mode != PHANTOM_MOE_SCORE_SOFTMAX && score_mode != PHANTOM_MOE_SCORE_SIGMOID)
    return fail(PHANTOM_MOE_EINVAL, "score_mode must be 0 (softmax) or 1 (sigmoid), got %d", score_mode);
  if (T * (int64_t)top_k > ((int64_t)1 << 30))
    return fail(PHANTOM_MOE_EUNSUPPORTED, "T*top_k too large");
  return 0;
}

}  // namespace

namespace pmoe {

namespace {

LibConfig config_from_env() {
  LibConfig c;
  const char* d = getenv("PHANTOM_MOE_DECODE");
  c.decode_fused = !(d && strcmp(d, "staged") == 0);
  const char* k = getenv("PHANTOM_MOE_DECODE_KSPLIT");
  c.force_ksplit = k && strcmp(k, "1") == 0;
  const char* x8 = getenv("PHANTOM_MOE_DECODE_X8");
  c.decode_x8 = !(x8 && strcmp(x8, "0") == 0);
  const char* st = getenv("PHANTOM_MOE_DECODE_STREAM");
  c.decode_stream = (st && strcmp(st, "0") == 0) ? 0 : (st && strcmp(st, "2") == 0) ? 2 : 1;
  c.fused_wait_polls = kFusedWaitPollsDefault;
  c.fused_fault = 0;
  return c;
}

// "a,b,c" with a in [1, max_waves], b in {1, 2, 4}, c in {1, 2}; else unset.
void parse_tiling(const char* name, int max_waves, int out[3]) {
  const char* v = getenv(name);
  int a = 0, b = 0, c = 0;
  if (v && sscanf(v, "%d,%d,%d", &a, &b, &c) == 3 && a >= 1 && a <= max_waves && (b == 1 || b == 2 || b == 4) &&
      (c == 1 || c == 2)) {
    out[0] = a;
    out[1] = b;
    out[2] = c;
  }
}

Tuning tuning_from_env() {
  Tuning t;
  if (const char* v = getenv("PHANTOM_MOE_GATE_UP_DEPTH")) {
    const int d = atoi(v);
    if (d >= 2 && d <= 4) t.gu_depth = d;
  }
  if (const char* v = getenv("PHANTOM_MOE_DOWN_DEPTH")) {
    const int d = atoi(v);
    if (d == 2 || d == 4 || d == 6) t.dn_depth = d;
  }
  parse_tiling("PHANTOM_MOE_GATE_UP_TILING", 8, t.gu_tiling);
  parse_tiling("PHANTOM_MOE_DOWN_TILING", 4, t.dn_tiling);
  return t;
}

// Options live in atomics so a change from another thread is never torn;
// they are read once per call.  The environment is read once, on first use.
std::atomic<int> g_opt_fused{1};
std::atomic<int> g_opt_ksplit{0};
std::atomic<int> g_opt_x8{1};
std::atomic<int> g_opt_stream{1};
std::atomic<uint32_t> g_opt_polls{kFusedWaitPollsDefault};
std::atomic<uint32_t> g_opt_fault{0};
std::once_flag g_opt_once;
Tuning g_tuning;

void init_options() {
  std::call_once(g_opt_once, [] {
    const LibConfig c = config_from_env();
    g_opt_fused.store(c.decode_fused ? 1 : 0);
    g_opt_ksplit.store(c.force_ksplit ? 1 : 0);
    g_opt_x8.store(c.decode_x8 ? 1 : 0);
    g_opt_stream.store(c.decode_stream);
    g_opt_polls.store(c.fused_wait_polls);
    g_opt_fault.store(c.fused_fault);
    g_tuning = tuning_from_env();
  });
}

}  // namespace

LibConfig lib_config() {
  init_options();
  LibConfig c;
  c.decode_fused = g_opt_fused.load(std::memory_order_relaxed) != 0;
  c.force_ksplit = g_opt_ksplit.load(std::memory_order_relaxed) != 0;
  c.decode_x8 = g_opt_x8.load(std::memory_order_relaxed) != 0;
  c.decode_stream = g_opt_stream.load(std::memory_order_relaxed);
  c.fused_wait_polls = g_opt_polls.load(std::memory_order_relaxed);
  c.fused_fault = g_opt_fault.load(std::memory_order_relaxed);
  return c;
}

void set_lib_config(const LibConfig& c) {
  init_options();
  g_opt_fused.store(c.decode_fused ? 1 : 0);
  g_opt_ksplit.store(c.force_ksplit ? 1 : 0);
  g_opt_x8.store(c.decode_x8 ? 1 : 0);
  g_opt_stream.store(c.decode_stream);
  g_opt_polls.store(c.fused_wait_polls);
  g_opt_fault.store(c.fused_fault);
}

const Tuning& tuning() {
  init_options();
  return g_tuning;
}

namespace {
std::atomic<uint32_t*> g_host_status_dev{nullptr};
uint32_t* g_host_status_host = nullptr;
std::mutex g_host_status_mu;
}  // namespace

uint32_t* host_status_word() { return g_host_status_dev.load(std::memory_order_acquire); }

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_err[0] = '\0'; }

size_t plan_workspace(int64_t T, int64_t H, int64_t I, int E, int k, int has_shared, void* base,
                      Workspace* ws) {
  const int64_t Kpad = round_up(H, kQuad);
  const int64_t nslots = T * k;
  const int64_t rows = nslots + (has_shared ? T : 0);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t o = off;
    off = align256(off + bytes);
    return o;
  };
  // Every plan starts with the same control words, which only the
  // single-launch path writes; its own regions follow when the shape takes it.
  const size_t o_ctl = take(kCtlBytes);
  const bool fused = I > 0 && fused_shape_ok(T, H, I, E, k, has_shared);
  const bool strm = I > 0 && stream_shape_ok(T, H, I, E, k, has_shared);
  size_t o_pres = 0, o_slots = 0, o_hv = 0, o_xsl = 0, o_xh = 0, o_xpt = 0, o_ssl = 0, o_sdv = 0;
  const bool x8 = fused && x8_shape(T, H, I, E, k, has_shared);
  if (fused || strm) {
    o_pres = take(sizeof(uint64_t) * (size_t)kFusedMaxGrid);
    o_slots = take((size_t)16 * (size_t)(T * E));
    o_hv = take((size_t)16 * (size_t)((T * k + T) * (I / 2)));
  }
  if (strm) {
    o_ssl = take((size_t)kStreamSlotStride * (size_t)E);
    o_sdv = take((size_t)16 * (size_t)(k + 1) * (size_t)stream_kx_max(ceil_div(I, kQuad)) * (size_t)(H / 2));
  }
  if (x8) {
    o_xsl = take((size_t)256 * (size_t)E);  // device-scope logit slots, 256 bytes apart
    o_xh = take((size_t)16 * 8 * (size_t)(I / 2));
    o_xpt = take((size_t)16 * 8 * (size_t)(H / 2));
  }
  const size_t o_log = take(sizeof(double) * (size_t)(T * E));
  // x operand rows 0..T-1 plus an all-zero row T
  const size_t o_xq = take(sizeof(uint16_t) * (size_t)((T + 1) * Kpad));
  const size_t o_xs = take(sizeof(float) * (size_t)((T + 1) * (Kpad / kGroup)));
  const size_t o_off = take(sizeof(int32_t) * (size_t)(E + 2));
  const size_t o_act = take(sizeof(int32_t) * (size_t)(E + 1));
  const size_t o_nact = take(sizeof(int32_t));
  const size_t o_ss = take(sizeof(int32_t) * (size_t)nslots);
  const size_t o_sp = take(sizeof(int32_t) * (size_t)nslots);
  const size_t o_desc = take(sizeof(int4) * (size_t)(E + 1));
  const size_t o_tok = take(sizeof(int32_t) * (size_t)rows);
  const size_t o_tiles = take(sizeof(int32_t) * (size_t)(max_token_tiles(T, k, E, has_shared) * kTileWords));
  const size_t o_ntiles = take(sizeof(int32_t) * kCtlStride);
  const int64_t KpadI = I > 0 ? round_up(I, kQuad) : 0;
  // down operand rows plus an all-zero row
  const size_t o_hq = take(sizeof(uint16_t) * (size_t)((rows + 1) * KpadI * 2));
  const size_t o_hs = take(sizeof(float) * (size_t)((rows + 1) * (KpadI / kGroup) * 2));
  const size_t o_out = take(sizeof(float) * (size_t)(rows * (I > 0 ? H : 0)));
  const size_t o_cnt = take(sizeof(int32_t));
  const size_t o_pcnt = take(sizeof(int32_t) * (size_t)E * (size_t)perm_blocks(T * k));
  const size_t o_ptb = take(sizeof(int32_t) * (size_t)E);
  const bool two_pass = two_pass_shape(T, E);
  const size_t o_apx = two_pass ? take(sizeof(float) * (size_t)(T * E + T + E)) : 0;
  const size_t o_cand = two_pass ? take((size_t)(T * E)) : 0;
  if (ws && base) {
    char* b = static_cast<char*>(base);
    ws->ctl = reinterpret_cast<uint32_t*>(b + o_ctl);
    ws->fused = FusedWs();
    if (fused || strm) {
      ws->fused.ctl = ws->ctl;
      ws->fused.presence = reinterpret_cast<uint64_t*>(b + o_pres);
      ws->fused.slots = reinterpret_cast<uint32_t*>(b + o_slots);
      ws->fused.hv = reinterpret_cast<uint32_t*>(b + o_hv);
    }
    if (strm) {
      ws->fused.sslots = reinterpret_cast<uint32_t*>(b + o_ssl);
      ws->fused.sdv = reinterpret_cast<uint32_t*>(b + o_sdv);
    }
    if (x8) {
      ws->fused.xslots = reinterpret_cast<uint32_t*>(b + o_xsl);
      ws->fused.xh = reinterpret_cast<uint32_t*>(b + o_xh);
      ws->fused.xpart = reinterpret_cast<uint32_t*>(b + o_xpt);
    }
    ws->logits = reinterpret_cast<double*>(b + o_log);
    ws->xq = reinterpret_cast<uint16_t*>(b + o_xq);
    ws->xs = reinterpret_cast<float*>(b + o_xs);
    ws->offsets = reinterpret_cast<int32_t*>(b + o_off);
    ws->active = reinterpret_cast<int32_t*>(b + o_act);
    ws->n_active = reinterpret_cast<int32_t*>(b + o_nact);
    ws->sorted_slots = reinterpret_cast<int32_t*>(b + o_ss);
    ws->slot_pos = reinterpret_cast<int32_t*>(b + o_sp);
    ws->desc = reinterpret_cast<int4*>(b + o_desc);
    ws->seg_tok = reinterpret_cast<int32_t*>(b + o_tok);
    ws->tiles = reinterpret_cast<int32_t*>(b + o_tiles);
    ws->n_tiles = reinterpret_cast<int32_t*>(b + o_ntiles);
    ws->hq = reinterpret_cast<uint16_t*>(b + o_hq);
    ws->hs = reinterpret_cast<float*>(b + o_hs);
    ws->outbuf = reinterpret_cast<float*>(b + o_out);
    ws->counter = reinterpret_cast<int32_t*>(b + o_cnt);
    ws->perm_cnt = reinterpret_cast<int32_t*>(b + o_pcnt);
    ws->perm_tb = reinterpret_cast<int32_t*>(b + o_ptb);
    ws->approx = two_pass ? reinterpret_cast<float*>(b + o_apx) : nullptr;
    ws->cand = two_pass ? reinterpret_cast<uint8_t*>(b + o_cand) : nullptr;
  }
  return off;
}

}  // namespace pmoe


// Scratch of phantom_moe_forward_static: one copy per GPU, held until the
// process ends.  Static storage starts zeroed, which is the state a fresh
// workspace must start in (its first 256 bytes hold the call counter of the
// single-launch path).  In host code `scratch` only names the symbol; its
// device address comes from hipGetSymbolAddress, per device.
constexpr size_t kStaticScratchBytes = (size_t)16 << 20;
static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mu;

// The device address of the current device's scratch, looked up on the
// device's first call.
int static_scratch(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return launch_status(e, "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return fail(PHANTOM_MOE_EUNSUPPORTED, "device %d above %d", dev, kMaxDevices - 1);
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (!p) {
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess) return launch_status(e, "hipGetSymbolAddress(scratch)");
      if (!p || reinterpret_cast<uintptr_t>(p) % 256)
        return fail(PHANTOM_MOE_ELAUNCH, "static scratch address %p is not 256-byte aligned", p);
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return 0;
}

bool misaligned(const void* p, uintptr_t a) { return p && reinterpret_cast<uintptr_t>(p) % a != 0; }

// The arguments of one layer call (both forward entry points).
struct ForwardCall {
  const void* x;
  int x_dtype;
  int64_t T, H, I;
  int E, top_k, score_mode;
  const float* router_w;
  const float* router_bias;
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
  float* y;
  int32_t* topk_idx;
  float* topk_w;
  int has_shared;  // set by check_forward
};

int check_forward(ForwardCall& c) {
  if (int rc = check_route_shapes(c.x, c.x_dtype, c.router_w, c.T, c.H, c.E, c.top_k, c.score_mode)) return rc;
  if (c.x_dtype != PHANTOM_MOE_X_BF16)
    return fail(PHANTOM_MOE_EUNSUPPORTED, "phantom_moe_forward takes bf16 activations (x_dtype 0)");
  if (c.I < 32 || c.I % 32)
    return fail(PHANTOM_MOE_EINVAL, "I must be a positive multiple of 32, got %lld", (long long)c.I);
  if (!c.gate_nib || !c.gate_scale || !c.up_nib || !c.up_scale || !c.down_nib || !c.down_scale)
    return fail(PHANTOM_MOE_EINVAL, "expert weight pointers must be non-null");
  if (!c.y || !c.topk_idx || !c.topk_w) return fail(PHANTOM_MOE_EINVAL, "y, topk_idx and topk_w must be non-null");
  const int n_sh = (c.sh_gate_nib != nullptr) + (c.sh_gate_scale != nullptr) + (c.sh_up_nib != nullptr) +
                   (c.sh_up_scale != nullptr) + (c.sh_down_nib != nullptr) + (c.sh_down_scale != nullptr);
  if (n_sh != 0 && n_sh != 6)
    return fail(PHANTOM_MOE_EINVAL, "shared expert pointers must be all null or all non-null");
  c.has_shared = n_sh == 6 ? 1 : 0;
  // the kernels read nibbles with 16-byte and scales with 8-byte loads
  if (misaligned(c.gate_nib, 16) || misaligned(c.up_nib, 16) || misaligned(c.down_nib, 16) ||
      misaligned(c.sh_gate_nib, 16) || misaligned(c.sh_up_nib, 16) || misaligned(c.sh_down_nib, 16))
    return fail(PHANTOM_MOE_EINVAL, "repacked nibble buffers must be 16-byte aligned");
  if (misaligned(c.gate_scale, 8) || misaligned(c.up_scale, 8) || misaligned(c.down_scale, 8) ||
      misaligned(c.sh_gate_scale, 8) || misaligned(c.sh_up_scale, 8) || misaligned(c.sh_down_scale, 8))
    return fail(PHANTOM_MOE_EINVAL, "repacked scale buffers must be 8-byte aligned");
  if (misaligned(c.x, 8) || misaligned(c.router_w, 16))
    return fail(PHANTOM_MOE_EINVAL, "x must be 8-byte and router_w 16-byte aligned");
  // the decode-regime down kernel reads one expert segment's operand (at
  // most T positions of I as fp16 hi and lo) through a 32-bit buffer resource
  if (!pmoe::gemm_regime(c.T, c.top_k, c.E) && c.T * ((c.I + 127) / 128) * 512 >= ((int64_t)1 << 31))
    return fail(PHANTOM_MOE_EUNSUPPORTED, "T*I too large for the decode regime (one segment's down operand above 2 GiB)");
  return 0;
}

// Launch the layer on a workspace already checked to be large enough.
int run_forward(const ForwardCall& c, void* workspace, hipStream_t stream) {
  const int64_t T = c.T, H = c.H, I = c.I;
  const int E = c.E, top_k = c.top_k, has_shared = c.has_shared;
  pmoe::Workspace ws;
  pmoe::plan_workspace(T, H, I, E, top_k, has_shared, workspace, &ws);

  pmoe::RouteArgs r = {};
  r.x = c.x;
  r.x_dtype = c.x_dtype;
  r.router_w = c.router_w;
  r.router_bias = c.router_bias;
  r.T = T;
  r.H = H;
  r.E = E;
  r.k = top_k;
  r.score_mode = c.score_mode;
  r.topk_idx = c.topk_idx;
  r.topk_w = c.topk_w;
  pmoe::ExpertArgs a = {};
  a.T = T;
  a.H = H;
  a.I = I;
  a.E = E;
  a.k = top_k;
  a.has_shared = has_shared;
  a.gate_nib = c.gate_nib;
  a.gate_scale = c.gate_scale;
  a.up_nib = c.up_nib;
  a.up_scale = c.up_scale;
  a.down_nib = c.down_nib;
  a.down_scale = c.down_scale;
  a.sh_gate_nib = c.sh_gate_nib;
  a.sh_gate_scale = c.sh_gate_scale;
  a.sh_up_nib = c.sh_up_nib;
  a.sh_up_scale = c.sh_up_scale;
  a.sh_down_nib = c.sh_down_nib;
  a.sh_down_scale = c.sh_down_scale;
  a.topk_w = c.topk_w;
  a.y = c.y;

  // Decode batches of a few tokens: the whole layer in one launch.  Its
  // profile events bracket that launch as the gate/up stage (the router,
  // down and combine stages are then empty).
  if (ws.fused.ctl) {
    const pmoe::FusedPlan pl = pmoe::fused_plan(T, H, I, E, top_k, has_shared);
    if (pl.ok) {
      if (int rc = launch_status(record_stage(0, stream), "profile event")) return rc;
      if (int rc = launch_status(record_stage(1, stream), "profile event")) return rc;
      if (int rc = launch_status(pmoe::launch_decode_fused(pl, r, a, ws.fused, stream), "decode_fused")) return rc;
      for (int i = 2; i < PHANTOM_MOE_PROFILE_EVENTS; ++i)
        if (int rc = launch_status(record_stage(i, stream), "profile event")) return rc;
      return ok();
    }
    // one token with experts too large to stage whole: the streaming single launch
    const pmoe::StreamPlan sp = ws.fused.sslots ? pmoe::stream_plan(T, H, I, E, top_k, has_shared)
                                                : pmoe::StreamPlan{};
    if (sp.ok) {
      if (int rc = launch_status(record_stage(0, stream), "profile event")) return rc;
      if (int rc = launch_status(record_stage(1, stream), "profile event")) return rc;
      if (int rc = launch_status(pmoe::launch_decode_stream(sp, r, a, ws.fused, stream), "decode_stream")) return rc;
      for (int i = 2; i < PHANTOM_MOE_PROFILE_EVENTS; ++i)
        if (int rc = launch_status(record_stage(i, stream), "profile event")) return rc;
      return ok();
    }
  }

  const bool gemm = pmoe::gemm_regime(T, top_k, E);
  r.prep_x = true;
  r.prep_fp16 = gemm;
  r.do_permute = true;
  r.has_shared = has_shared;
  r.want_tiles = !gemm && (pmoe::gate_up_tile_regime(T, H, I, E, top_k, has_shared) ||
                           pmoe::down_tile_regime(T, H, I, E, top_k, has_shared));
  if (int rc = launch_status(record_stage(0, stream), "profile event")) return rc;
  if (int rc = launch_status(pmoe::launch_route(r, ws, stream), "route")) return rc;

  if (int rc = launch_status(record_stage(1, stream), "profile event")) return rc;
  if (int rc = launch_status(gemm ? pmoe::launch_gemm_gate_up(a, ws, stream) : pmoe::launch_gate_up(a, ws, stream),
                             "gate_up"))
    return rc;
  if (int rc = launch_status(record_stage(2, stream), "profile event")) return rc;
  if (int rc = launch_status(gemm ? pmoe::launch_gemm_down(a, ws, stream) : pmoe::launch_down(a, ws, stream),
                             "down"))
    return rc;
  if (int rc = launch_status(record_stage(3, stream), "profile event")) return rc;
  if (int rc = launch_status(pmoe::launch_combine(a, ws, stream), "combine")) return rc;
  return launch_status(record_stage(4, stream), "profile event");
}

}  // namespace

extern "C" {

const char* phantom_moe_last_error(void) { return g_err; }

const char* phantom_moe_version(void) { return "phantom_moe 0.1.0 gfx950"; }

const char* phantom_moe_expert_kernels(int64_t T, int64_t H, int64_t I, int E, int top_k, int has_shared) {
  static thread_local char buf[96];
  const char *gu, *dn;
  const pmoe::FusedPlan fp = pmoe::fused_plan(T, H, I, E, top_k, has_shared ? 1 : 0);
  if (fp.ok) {
    // the whole layer is one launch
    gu = dn = fp.spec == pmoe::kFusedSpecX8 ? "moe_decode_x8_kernel" : "moe_decode_fused_kernel";
  } else if (pmoe::stream_plan(T, H, I, E, top_k, has_shared ? 1 : 0).ok) {
    gu = dn = "moe_decode_stream_kernel";
  } else if (pmoe::gemm_regime(T, top_k, E)) {
    gu = "gemm_gate_up_kernel";
    dn = "gemm_down_kernel";
  } else {
    gu = pmoe::gate_up_tile_regime(T, H, I, E, top_k, has_shared) ? "gate_up_tile_kernel" : "gate_up_kernel";
    dn = pmoe::down_tile_regime(T, H, I, E, top_k, has_shared) ? "down_tile_kernel" : "down_kernel";
  }
  snprintf(buf, sizeof(buf), "gate_up=%s;down=%s", gu, dn);
  return buf;
}

int phantom_moe_set_profile_events(hipEvent_t* events, int n_events) {
  if (events == nullptr) {
    g_prof_events = nullptr;
    return ok();
  }
  if (n_events < PHANTOM_MOE_PROFILE_EVENTS)
    return fail(PHANTOM_MOE_EINVAL, "profile events: need %d events, got %d", PHANTOM_MOE_PROFILE_EVENTS, n_events);
  for (int i = 0; i < PHANTOM_MOE_PROFILE_EVENTS; ++i)
    if (!events[i]) return fail(PHANTOM_MOE_EINVAL, "profile events: event %d is null", i);
  g_prof_events = events;
  return ok();
}

int64_t phantom_q4_0_nib_bytes(int64_t rows, int64_t K) {
  if (rows < 0 || K < 0 || rows % 16 || K % 32) return -1;
  return rows * pmoe::round_up(K, pmoe::kQuad) / 2;
}

int64_t phantom_q4_0_scale_bytes(int64_t rows, int64_t K) {
  if (rows < 0 || K < 0 || rows % 16 || K % 32) return -1;
  return rows * pmoe::round_up(K, pmoe::kQuad) / 32 * 2;
}

int phantom_q4_0_repack(const uint8_t* q4_0, int64_t rows, int64_t K, uint8_t* nib, uint16_t* scale,
                        hipStream_t stream) {
  if (rows < 0 || K < 0 || rows % 16 || K % 32)
    return fail(PHANTOM_MOE_EINVAL, "repack needs rows %% 16 == 0 and K %% 32 == 0 (rows=%lld K=%lld)",
                (long long)rows, (long long)K);
  if (rows == 0 || K == 0) return ok();
  if (!q4_0 || !nib || !scale) return fail(PHANTOM_MOE_EINVAL, "repack: null pointer");
  if (reinterpret_cast<uintptr_t>(nib) % 16 || reinterpret_cast<uintptr_t>(scale) % 8)
    return fail(PHANTOM_MOE_EINVAL, "repack: nib must be 16-byte and scale 8-byte aligned");
  return launch_status(pmoe::launch_q4_repack(q4_0, rows, K, nib, scale, stream), "q4_repack");
}

int phantom_q4_0_unrepack(const uint8_t* nib, const uint16_t* scale, int64_t rows, int64_t K,
                          uint8_t* q4_0, hipStream_t stream) {
  if (rows < 0 || K < 0 || rows % 16 || K % 32)
    return fail(PHANTOM_MOE_EINVAL, "unrepack needs rows %% 16 == 0 and K %% 32 == 0");
  if (rows == 0 || K == 0) return ok();
  if (!q4_0 || !nib || !scale) return fail(PHANTOM_MOE_EINVAL, "unrepack: null pointer");
  return launch_status(pmoe::launch_q4_unrepack(nib, scale, rows, K, q4_0, stream), "q4_unrepack");
}

int phantom_q4_0_dequant_f32(const uint8_t* q4_0, int64_t rows, int64_t K, float* out,
                             hipStream_t stream) {
  if (rows < 0 || K < 0 || K % 32) return fail(PHANTOM_MOE_EINVAL, "dequant needs K %% 32 == 0");
  if (rows == 0 || K == 0) return ok();
  if (!q4_0 || !out) return fail(PHANTOM_MOE_EINVAL, "dequant: null pointer");
  return launch_status(pmoe::launch_q4_dequant_f32(q4_0, rows * (K / 32), out, stream), "q4_dequant");
}

size_t phantom_moe_workspace_bytes(int64_t T, int64_t H, int64_t I, int E, int top_k, int has_shared) {
  if (T < 1 || H < 1 || E < 1 || top_k < 1 || I < 0) return 0;
  return pmoe::plan_workspace(T, H, I, E, top_k, has_shared ? 1 : 0, nullptr, nullptr);
}

int phantom_moe_set_option(int option, int value) {
  pmoe::LibConfig c = pmoe::lib_config();
  switch (option) {
    case PHANTOM_MOE_OPT_DECODE_FUSED:
      if (value != 0 && value != 1) return fail(PHANTOM_MOE_EINVAL, "DECODE_FUSED takes 0 or 1, got %d", value);
      c.decode_fused = value != 0;
      break;
    case PHANTOM_MOE_OPT_DECODE_KSPLIT:
      if (value != 0 && value != 1) return fail(PHANTOM_MOE_EINVAL, "DECODE_KSPLIT takes 0 or 1, got %d", value);
      c.force_ksplit = value != 0;
      break;
    case PHANTOM_MOE_OPT_FUSED_WAIT_POLLS:
      if (value < 1) return fail(PHANTOM_MOE_EINVAL, "FUSED_WAIT_POLLS takes a positive bound, got %d", value);
      c.fused_wait_polls = (uint32_t)value;
      break;
    case PHANTOM_MOE_OPT_FUSED_FAULT:
      if (value < 0 || value > 7) return fail(PHANTOM_MOE_EINVAL, "FUSED_FAULT takes 0..7, got %d", value);
      c.fused_fault = (uint32_t)value;
      break;
    case PHANTOM_MOE_OPT_DECODE_X8:
      if (value != 0 && value != 1) return fail(PHANTOM_MOE_EINVAL, "DECODE_X8 takes 0 or 1, got %d", value);
      c.decode_x8 = value != 0;
      break;
    case PHANTOM_MOE_OPT_DECODE_STREAM:
      if (value < 0 || value > 2) return fail(PHANTOM_MOE_EINVAL, "DECODE_STREAM takes 0, 1 or 2, got %d", value);
      c.decode_stream = value;
      break;
    default:
      return fail(PHANTOM_MOE_EINVAL, "unknown option %d", option);
  }
  pmoe::set_lib_config(c);
  return ok();
}

int phantom_moe_get_option(int option, int* value) {
  if (!value) return fail(PHANTOM_MOE_EINVAL, "get_option: null value");
  const pmoe::LibConfig c = pmoe::lib_config();
  switch (option) {
    case PHANTOM_MOE_OPT_DECODE_FUSED: *value = c.decode_fused ? 1 : 0; break;
    case PHANTOM_MOE_OPT_DECODE_KSPLIT: *value = c.force_ksplit ? 1 : 0; break;
    case PHANTOM_MOE_OPT_FUSED_WAIT_POLLS: *value = (int)c.fused_wait_polls; break;
    case PHANTOM_MOE_OPT_FUSED_FAULT: *value = (int)c.fused_fault; break;
    case PHANTOM_MOE_OPT_DECODE_X8: *value = c.decode_x8 ? 1 : 0; break;
    case PHANTOM_MOE_OPT_DECODE_STREAM: *value = c.decode_stream; break;
    default: return fail(PHANTOM_MOE_EINVAL, "unknown option %d", option);
  }
  return ok();
}

uint32_t* phantom_moe_status_word(void) {
  std::lock_guard<std::mutex> lk(pmoe::g_host_status_mu);
  if (pmoe::g_host_status_host) {
    ok();
    return pmoe::g_host_status_host;
  }
  void* h = nullptr;
  hipError_t e = hipHostMalloc(&h, 256, hipHostMallocMapped | hipHostMallocPortable | hipHostMallocCoherent);
  if (e != hipSuccess) {
    launch_status(e, "status_word: hipHostMalloc");
    return nullptr;
  }
  memset(h, 0, 256);
  void* d = nullptr;
  e = hipHostGetDevicePointer(&d, h, 0);
  if (e != hipSuccess) {
    (void)hipHostFree(h);
    launch_status(e, "status_word: hipHostGetDevicePointer");
    return nullptr;
  }
  pmoe::g_host_status_host = static_cast<uint32_t*>(h);
  pmoe::g_host_status_dev.store(static_cast<uint32_t*>(d), std::memory_order_release);
  ok();
  return pmoe::g_host_status_host;
}

int phantom_moe_workspace_status(void* workspace, size_t workspace_bytes, uint32_t* status, hipStream_t stream) {
  if (!workspace || !status) return fail(PHANTOM_MOE_EINVAL, "workspace_status: null pointer");
  if (workspace_bytes < pmoe::kCtlBytes) return fail(PHANTOM_MOE_EWORKSPACE, "workspace_status: workspace too small");
  uint32_t* word = static_cast<uint32_t*>(workspace) + 1;
  uint32_t v = 0;
  hipError_t e = hipMemcpyAsync(&v, word, sizeof(v), hipMemcpyDeviceToHost, stream);
  if (e == hipSuccess) e = hipStreamSynchronize(stream);
  if (e == hipSuccess && v != 0) {
    static const uint32_t zero = 0;
    e = hipMemcpyAsync(word, &zero, sizeof(zero), hipMemcpyHostToDevice, stream);
    if (e == hipSuccess) e = hipStreamSynchronize(stream);
  }
  if (e != hipSuccess) return launch_status(e, "workspace_status");
  *status = v;
  return ok();
}

int phantom_moe_route(const void* x, int x_dtype, const float* router_w, const float* router_bias,
                      int64_t T, int64_t H, int E, int top_k, int score_mode, int32_t* topk_idx,
                      float* topk_w, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (int rc = check_route_shapes(x, x_dtype, router_w, T, H, E, top_k, score_mode)) return rc;
  if (!topk_idx || !topk_w) return fail(PHANTOM_MOE_EINVAL, "topk_idx and topk_w must be non-null");
  const size_t need = pmoe::plan_workspace(T, H, 0, E, top_k, 0, nullptr, nullptr);
  if (!workspace || workspace_bytes < need)
    return fail(PHANTOM_MOE_EWORKSPACE, "workspace of %zu bytes required, %zu given", need,
                workspace ? workspace_bytes : (size_t)0);
  pmoe::Workspace ws;
  pmoe::plan_workspace(T, H, 0, E, top_k, 0, workspace, &ws);
  pmoe::RouteArgs r = {};
  r.x = x;
  r.x_dtype = x_dtype;
  r.router_w = router_w;
  r.router_bias = router_bias;
  r.T = T;
  r.H = H;
  r.E = E;
  r.k = top_k;
  r.score_mode = score_mode;
  r.topk_idx = topk_idx;
  r.topk_w = topk_w;
  r.prep_x = false;
  r.do_permute = false;
  return launch_status(pmoe::launch_route(r, ws, stream), "route");
}

int phantom_moe_permute(const int32_t* topk_idx, int64_t T, int top_k, int E, int32_t* expert_offsets,
                        int32_t* sorted_slots, int32_t* slot_pos, void* workspace,
                        size_t workspace_bytes, hipStream_t stream) {
  if (!topk_idx || !expert_offsets || !sorted_slots || !slot_pos)
    return fail(PHANTOM_MOE_EINVAL, "permute: null pointer");
  if (T < 1 || top_k < 1 || E < 1 || top_k > E)
    return fail(PHANTOM_MOE_EINVAL, "permute: need T >= 1 and 1 <= top_k <= E");
  if (E > pmoe::kMaxExperts) return fail(PHANTOM_MOE_EUNSUPPORTED, "permute: E above %d", pmoe::kMaxExperts);
  if (T * (int64_t)top_k > ((int64_t)1 << 30)) return fail(PHANTOM_MOE_EUNSUPPORTED, "permute: T*top_k too large");
  const size_t need = pmoe::plan_workspace(T, 32, 0, E, top_k, 0, nullptr, nullptr);
  if (!workspace || workspace_bytes < need)
    return fail(PHANTOM_MOE_EWORKSPACE, "workspace of %zu bytes required", need);
  pmoe::Workspace ws;
  pmoe::plan_workspace(T, 32, 0, E, top_k, 0, workspace, &ws);
  return launch_status(
      pmoe::launch_permute(topk_idx, T, top_k, E, 0, expert_offsets, sorted_slots, slot_pos, ws, stream),
      "permute");
}

int phantom_moe_forward(const void* x, int x_dtype, int64_t T, int64_t H, int64_t I, int E, int top_k,
                        int score_mode, const float* router_w, const float* router_bias,
                        const uint8_t* gate_nib, const uint16_t* gate_scale, const uint8_t* up_nib,
                        const uint16_t* up_scale, const uint8_t* down_nib, const uint16_t* down_scale,
                        const uint8_t* sh_gate_nib, const uint16_t* sh_gate_scale,
                        const uint8_t* sh_up_nib, const uint16_t* sh_up_scale,
                        const uint8_t* sh_down_nib, const uint16_t* sh_down_scale, float* y,
                        int32_t* topk_idx, float* topk_w, void* workspace, size_t workspace_bytes,
                        hipStream_t stream) {
  ForwardCall c = {x, x_dtype, T, H, I, E, top_k, score_mode, router_w, router_bias,
                   gate_nib, gate_scale, up_nib, up_scale, down_nib, down_scale,
                   sh_gate_nib, sh_gate_scale, sh_up_nib, sh_up_scale, sh_down_nib, sh_down_scale,
                   y, topk_idx, topk_w, 0};
  if (int rc = check_forward(c)) return rc;
  if (misaligned(workspace, 256)) return fail(PHANTOM_MOE_EINVAL, "workspace must be 256-byte aligned");
  const size_t need = pmoe::plan_workspace(T, H, I, E, top_k, c.has_shared, nullptr, nullptr);
  if (!workspace || workspace_bytes < need)
    return fail(PHANTOM_MOE_EWORKSPACE, "workspace of %zu bytes required, %zu given", need,
                workspace ? workspace_bytes : (size_t)0);
  return run_forward(c, workspace, stream);
}

int phantom_moe_forward_static(const void* x, int x_dtype, int64_t T, int64_t H, int64_t I, int E, int top_k,
                               int score_mode, const float* router_w, const float* router_bias,
                               const uint8_t* gate_nib, const uint16_t* gate_scale, const uint8_t* up_nib,
                               const uint16_t* up_scale, const uint8_t* down_nib, const uint16_t* down_scale,
                               const uint8_t* sh_gate_nib, const uint16_t* sh_gate_scale,
                               const uint8_t* sh_up_nib, const uint16_t* sh_up_scale,
                               const uint8_t* sh_down_nib, const uint16_t* sh_down_scale, float* y,
                               int32_t* topk_idx, float* topk_w, hipStream_t stream) {
  ForwardCall c = {x, x_dtype, T, H, I, E, top_k, score_mode, router_w, router_bias,
                   gate_nib, gate_scale, up_nib, up_scale, down_nib, down_scale,
                   sh_gate_nib, sh_gate_scale, sh_up_nib, sh_up_scale, sh_down_nib, sh_down_scale,
                   y, topk_idx, topk_w, 0};
  if (int rc = check_forward(c)) return rc;
  const size_t need = pmoe::plan_workspace(T, H, I, E, top_k, c.has_shared, nullptr, nullptr);
  if (need > kStaticScratchBytes)
    return fail(PHANTOM_MOE_EWORKSPACE,
                "phantom_moe_forward_static: these sizes need %zu bytes of scratch, the static scratch holds %zu "
                "(use phantom_moe_forward with a workspace)",
                need, kStaticScratchBytes);
  void* base = nullptr;
  if (int rc = static_scratch(&base)) return rc;
  return run_forward(c, base, stream);
}

}  // extern "C"
