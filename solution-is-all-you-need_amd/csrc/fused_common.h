// fused_common.h -- device helpers shared by the single-launch decode
// kernels (decode_fused.hip, decode_stream.hip): the tagged device-scope
// hand-offs, bounded waits, the launch tag, the router's fixed-order dot and
// the fp16 integer expansion of the weights.
#pragma once

#include <math.h>
#include <stdint.h>

#include "moe_common.h"
#include "moe_launch.h"

namespace pmoe {

namespace {

// LDS region offsets are rounded up to 256 bytes.
__host__ __device__ inline uint32_t align_lds(uint32_t v) { return (v + 255u) & ~255u; }

// The offset 32-bit buffer offsets cannot reach; no stacked matrix is
// allowed to come near it.
constexpr uint32_t kMaxRsrcBytes = 0xFFFFE000u;

constexpr int kFW = 8;  // waves per workgroup
constexpr int kFThreads = kFW * kWave;
// 4 qs bytes (little endian word) -> 8 fp16 values n - 8, exactly, in the
// nibble order of dequant_unit_f16 (kmap order): each nibble goes into the
// low mantissa bits of 1024.0 (fp16 0x6400, whose mantissa step is 1), and
// 1032 is subtracted.  The MFMA then sums h * q with no offset correction.
// mask must hold 0x000F000F (in a VGPR).
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
__device__ inline uint32_t nib_pair_f16s(uint32_t w, uint32_t mask) {
  const f16x2 off = {(_Float16)-1032.0f, (_Float16)-1032.0f};
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, and_or(w, mask, 0x64006400u)) + off);
}
__device__ inline u32x4 dequant_unit_f16s(uint32_t w, uint32_t mask) {
  u32x4 r;
  r.x = nib_pair_f16s(w, mask);
  r.y = nib_pair_f16s(w >> 4, mask);
  r.z = nib_pair_f16s(w >> 8, mask);
  r.w = nib_pair_f16s(w >> 12, mask);
  return r;
}

// Start of a poll retry: to the compiler, memory the kernel arguments point
// to may have changed here, so the polled loads after it are issued again
// each iteration (a poll loop otherwise writes no memory, and its loads
// could be hoisted out of it).
__device__ inline void poll_clobber() { asm volatile("" ::: "memory"); }

__device__ inline uint64_t tag64(uint32_t t) { return (uint64_t)t | ((uint64_t)(~t) << 32); }

__device__ inline bool tag_ok(const u32x4& v, uint32_t t) { return v.y == t && v.w == ~t; }

// A value every lane of the wave holds alike (LDS reads of shared
// bookkeeping, wave indices): stated as uniform, so the compiler keeps it in
// an SGPR and branches and buffer offsets built from it stay scalar.
__device__ inline int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }

// s_waitcnt vmcnt(n) for a wave-uniform n known only at run time (n above
// 47 waits for everything).
__device__ inline void wait_vmcnt_le(int n) {
#define PMOE_W(N) \
  case N:         \
    wait_vmcnt<N>(); \
    break;
  switch (n) {
    PMOE_W(0) PMOE_W(1) PMOE_W(2) PMOE_W(3) PMOE_W(4) PMOE_W(5) PMOE_W(6) PMOE_W(7) PMOE_W(8) PMOE_W(9)
    PMOE_W(10) PMOE_W(11) PMOE_W(12) PMOE_W(13) PMOE_W(14) PMOE_W(15) PMOE_W(16) PMOE_W(17) PMOE_W(18)
    PMOE_W(19) PMOE_W(20) PMOE_W(21) PMOE_W(22) PMOE_W(23) PMOE_W(24) PMOE_W(25) PMOE_W(26) PMOE_W(27)
    PMOE_W(28) PMOE_W(29) PMOE_W(30) PMOE_W(31) PMOE_W(32) PMOE_W(33) PMOE_W(34) PMOE_W(35) PMOE_W(36)
    PMOE_W(37) PMOE_W(38) PMOE_W(39) PMOE_W(40) PMOE_W(41) PMOE_W(42) PMOE_W(43) PMOE_W(44) PMOE_W(45)
    PMOE_W(46) PMOE_W(47)
    default:
      wait_vmcnt<0>();
  }
#undef PMOE_W
}

// A wait gave up: the bit goes into the workspace's status word, and, where
// the process registered one (phantom_moe_status_word), into a pinned host
// word that the host reads without synchronising (a plain system-scope
// store: any non-zero value tells the host to look).  Only failure paths
// call this.
__device__ inline void set_status(uint32_t* ctl, uint32_t* host, uint32_t bit) {
  __hip_atomic_fetch_or(&ctl[1], bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (host) __hip_atomic_store(host, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// This launch's hand-off tag.  Normally the generation counter + 1.  The
// counter only advances at the end of a launch, once workgroup 0 has seen
// every workgroup's presence word carry the launch's tag, or once that wait
// gave up: a workgroup that starts after it gave up (it was not resident)
// reads the advanced counter, one ahead of its launch.  Its own presence
// word then still holds the previous launch's tag, which is counter - 1 from
// where it stands, and it takes the counter's value: its launch's tag, not
// the next launch's (so it never publishes stale data under a tag a later
// launch will accept).  A fresh (zero) or foreign presence word fails the
// {t, ~t} check and gives the normal tag.  skew is added to the counter
// read (non-zero only where a test forces the late-start case).
__device__ inline uint32_t launch_tag(const uint32_t* ctl, const uint64_t* own_presence, uint32_t skew) {
  const uint32_t g =
      (uint32_t)uni((int)__hip_atomic_load(&ctl[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) + skew;
  const uint64_t pr = __hip_atomic_load(own_presence, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const uint32_t plo = (uint32_t)uni((int)(uint32_t)pr), phi = (uint32_t)uni((int)(uint32_t)(pr >> 32));
  const bool late = phi == ~plo && plo + 1u == g;
  return late ? g : g + 1u;
}

// The router's fixed-order fp64 dot of x[t] (bf16) and W[e] (router.hip):
// lane l accumulates h = 256c + 4l + i in increasing h, then the xor tree
// s = 32..1 adds the 64 partials (commutative adds, so every lane ends with
// the same bits).
__device__ inline double fixed_dot_bf16(const uint16_t* xr, const float* wr, int H) {
  const int lane = threadIdx.x % kWave;
  constexpr int CB = 8;
  const int nch = (H + 255) / 256;
  double acc = 0.0;
  for (int c0 = 0; c0 < nch; c0 += CB) {
    float4 wv[CB];
    uint2 xv[CB];
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
      const int h0 = (c0 + cb) * 256 + 4 * lane;
      const bool ok = c0 + cb < nch && h0 < H;
      const int hc = ok ? h0 : 0;
      wv[cb] = *reinterpret_cast<const float4*>(wr + hc);
      xv[cb] = *reinterpret_cast<const uint2*>(xr + hc);
      if (!ok) {
        wv[cb] = make_float4(0.f, 0.f, 0.f, 0.f);
        xv[cb] = make_uint2(0u, 0u);
      }
    }
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
      acc += (double)bf16_bits_to_float(xv[cb].x & 0xffffu) * (double)wv[cb].x;
      acc += (double)bf16_bits_to_float(xv[cb].x >> 16) * (double)wv[cb].y;
      acc += (double)bf16_bits_to_float(xv[cb].y & 0xffffu) * (double)wv[cb].z;
      acc += (double)bf16_bits_to_float(xv[cb].y >> 16) * (double)wv[cb].w;
    }
  }
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) acc = acc + shfl_xor_f64(acc, s);
  return acc;
}

}  // namespace

}  // namespace pmoe
