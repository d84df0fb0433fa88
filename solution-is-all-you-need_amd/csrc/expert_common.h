// expert_common.h -- pieces shared by the two expert regimes (expert_ffn.hip,
// the grouped GEMV for decode, and expert_gemm.hip, the grouped MFMA GEMM for
// prefill): segment descriptors, scale unpacking, and the resident-grid sizing
// of strided item loops.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "moe_common.h"
#include "moe_launch.h"

namespace pmoe {

// Where the router's permute left the expert segments.
struct SegSrc {
  const int4* desc;        // [max_slots] {expert, begin, end, 0}; expert -1 = unused slot
  const int32_t* seg_tok;  // token of each segment position
  int E;
  int max_slots;           // min(E, T*k) + shared
};

__device__ inline void unpack_scales(uint2 s, float d[4]) {
  d[0] = half_bits_to_float((uint16_t)(s.x & 0xffffu));
  d[1] = half_bits_to_float((uint16_t)(s.x >> 16));
  d[2] = half_bits_to_float((uint16_t)(s.y & 0xffffu));
  d[3] = half_bits_to_float((uint16_t)(s.y >> 16));
}

// Copies the launch slots' segment descriptors into LDS, and with s_tok the
// token of each of the first n_tok segment positions too; returns how many
// slots are in use (they come first; unused slots carry expert -1; at least
// one is in use, so exactly one thread finds the boundary and writes the
// count).  All loads of an iteration are issued before its stores, so the
// copies cost one memory round trip and one barrier.
__device__ inline int load_descriptors(const SegSrc& seg, int4* s_desc, int* s_nact, int* s_tok = nullptr,
                                       int64_t n_tok = 0) {
  const int64_t n = (s_tok && n_tok > seg.max_slots) ? n_tok : seg.max_slots;
  for (int64_t u = threadIdx.x; u < n; u += blockDim.x) {
    const bool ds = u < seg.max_slots;
    const bool ts = s_tok && u < n_tok;
    int4 d = make_int4(-1, 0, 0, 0);
    int nx = -1, tk = 0;
    if (ds) {
      d = seg.desc[u];
      if (u + 1 < seg.max_slots) nx = seg.desc[u + 1].x;
    }
    if (ts) tk = seg.seg_tok[u];
    if (ds) {
      s_desc[u] = d;
      if (d.x >= 0 && nx < 0) *s_nact = (int)u + 1;
    }
    if (ts) s_tok[u] = tk;
  }
  __syncthreads();
  return *s_nact;
}

// Launch slots: at most min(E, T*k) routed segments, plus the shared expert.
inline unsigned max_active_experts(const ExpertArgs& x) {
  const int64_t nslots = x.T * x.k;
  return (unsigned)(((nslots < x.E) ? nslots : x.E) + (x.has_shared ? 1 : 0));
}

inline SegSrc segments_of(const ExpertArgs& x, const Workspace& ws) {
  SegSrc seg;
  seg.desc = ws.desc;
  seg.seg_tok = ws.seg_tok;
  seg.E = x.E;
  seg.max_slots = (int)max_active_experts(x);
  return seg;
}

inline int device_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

// Workgroups for a strided item loop: those resident at once (occupancy of
// this kernel at this block size, cached per kernel since the query is slow),
// capped by the largest possible item count.
template <typename Kernel>
unsigned resident_grid(Kernel kernel, int block, int64_t max_items) {
  struct Entry {
    const void* fn;
    int block, per_cu;
  };
  static thread_local Entry cache[32];
  static thread_local int n_cache = 0;
  int per_cu = 0;
  for (int i = 0; i < n_cache; ++i)
    if (cache[i].fn == reinterpret_cast<const void*>(kernel) && cache[i].block == block) per_cu = cache[i].per_cu;
  if (per_cu == 0) {
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, block, 0) != hipSuccess || per_cu < 1)
      per_cu = 1;
    if (n_cache < 32) cache[n_cache++] = Entry{reinterpret_cast<const void*>(kernel), block, per_cu};
  }
  int64_t g = (int64_t)device_cus() * per_cu;
  if (g > max_items) g = max_items;
  return (unsigned)(g < 1 ? 1 : g);
}

}  // namespace pmoe
