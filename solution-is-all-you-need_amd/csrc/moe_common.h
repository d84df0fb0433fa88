// moe_common.h -- shared device helpers for the gfx950 sparse-MoE kernels.
//
// Repacked Q4_0 layout (see phantom_q4_0_repack):
//   A [rows, K] Q4_0 matrix is cut into row tiles of 16 rows and K quads of
//   128 elements (4 Q4_0 groups).  One (row tile, quad) is 1 KiB of nibbles:
//   lane l of a wave owns 16 bytes, which hold, for each of the quad's 4
//   groups gi, the 4 qs bytes [4*p, 4*p+3] (p = l / 16) of row 16*rt + l%16.
//   Its scales are 128 bytes: [16 rows][4 groups] fp16.
//
// MFMA operand mapping (v_mfma_f32_16x16x32_bf16):
//   lane l holds 8 bf16 of A row (l % 16) and of B column (l % 16), both for
//   the same 8 K positions of the 32-wide group, chosen by p = l / 16.  The 4
//   qs bytes of part p expand (dequant_unit_bf16 / _f16) to the K positions
//       kmap(p) = {4p, 4p+2, 16+4p, 18+4p, 4p+1, 4p+3, 17+4p, 19+4p}
//   and activations are laid out in the same order, so the MFMA reduces over
//   exactly the 32 elements of the group.
//
// Magic-number expansion: placing a nibble n in the top mantissa bits of the
// constant 1.0 gives the exact value 1 + n/16 (bf16 pattern 0x3F80 | n << 3,
// fp16 pattern 0x3C00 | n << 6), so 8 nibbles become MFMA operands with one
// shift and one AND-OR per pair.  With q = n - 8,
//     sum_k a_k q_k = 16 * sum_k a_k (1 + n_k/16) - 24 * sum_k a_k,
// so each group's MFMA result is scaled by 16*d (exact) and the correction
// 24 * d * S (S = group sum of the activations) is applied once per output
// with an fp32 MFMA over groups.  The offset costs about 5x the signed
// result's rounding error (mean |1 + n/16| / rms |q/16|), not more.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pmoe {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;
constexpr int kRowTile = 16;
constexpr int kQuad = 128;       // K elements per quad
constexpr int kGroup = 32;       // Q4_0 group
constexpr int kQuadNibBytes = 1024;
constexpr int kQuadScales = 64;  // fp16 values per (row tile, quad)
constexpr float kUnitScale = 16.0f;  // (1 + n/16) * 16 = n + 16
constexpr float kUnitBias = 24.0f;   // 16 + 8: q = 16 (1 + n/16) - 24

__host__ __device__ inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
__host__ __device__ inline int64_t round_up(int64_t a, int64_t b) { return ceil_div(a, b) * b; }

// Position within a 32-group of element j (0..7) of MFMA part p (0..3).
__host__ __device__ inline int kmap(int p, int j) {
  // j: 0 1 2 3 4 5 6 7 -> 4p+{0, 2, 16, 18, 1, 3, 17, 19}
  const int off[8] = {0, 2, 16, 18, 1, 3, 17, 19};
  return 4 * p + off[j];
}

// (a & m) | c, which the compiler forms as one v_and_or_b32 (gfx9 VOP3
// reads at most one scalar or literal operand, so the caller keeps the mask
// in a VGPR, hoisted out of loops).  Written as an expression, not inline
// assembly: the compiler's hazard checks do not see inline assembly, and an
// inline v_and_or_b32 placed next to in-flight MFMAs has produced wrong
// results (NaN outputs) once a change of register allocation put it there.
__device__ inline uint32_t and_or(uint32_t a, uint32_t m_vgpr, uint32_t c_sgpr) { return (a & m_vgpr) | c_sgpr; }

// 4 qs bytes (little endian word) -> 8 bf16 values 1 + n/16, in kmap order.
// mask must hold 0x00780078 (in a VGPR).
__device__ inline u32x4 dequant_unit_bf16(uint32_t w, uint32_t mask) {
  u32x4 r;
  r.x = and_or(w << 3, mask, 0x3F803F80u);
  r.y = and_or(w >> 1, mask, 0x3F803F80u);
  r.z = and_or(w >> 5, mask, 0x3F803F80u);
  r.w = and_or(w >> 9, mask, 0x3F803F80u);
  return r;
}

// Same expansion as fp16 values 1 + n/16; mask must hold 0x03C003C0.
__device__ inline u32x4 dequant_unit_f16(uint32_t w, uint32_t mask) {
  u32x4 r;
  r.x = and_or(w << 6, mask, 0x3C003C00u);
  r.y = and_or(w << 2, mask, 0x3C003C00u);
  r.z = and_or(w >> 2, mask, 0x3C003C00u);
  r.w = and_or(w >> 6, mask, 0x3C003C00u);
  return r;
}

// A pointer the compiler cannot prove wave-uniform, made uniform (it must
// already hold the same value in every lane), so loads from it plus a 32-bit
// lane offset use the SGPR-base form.
template <typename T>
__device__ inline const T* uniform_ptr(const T* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return reinterpret_cast<const T*>(((uint64_t)hi << 32) | lo);
}

// A value the compiler must keep in a VGPR (for and_or masks).  The empty
// assembly statement emits no instruction: the compiler moves the constant
// into the VGPR itself (so its hazard checks see the write) and can no longer
// fold it, which keeps and_or a single v_and_or_b32.
__device__ inline uint32_t vgpr_const(uint32_t v) {
  asm volatile("" : "+v"(v));
  return v;
}

__device__ inline f32x4 mfma_bf16_16x16x32(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

__device__ inline f32x4 mfma_f16_16x16x32(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

__device__ inline f32x4 mfma_f32_16x16x4(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ inline float half_bits_to_float(uint16_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

__device__ inline float bf16_bits_to_float(uint32_t b) {
  return __builtin_bit_cast(float, b << 16);
}

// Round-to-nearest-even fp32 -> bf16 bits (finite inputs).
__device__ inline uint32_t float_to_bf16_bits(float f) {
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<__bf16>(f)));
}

__device__ inline uint32_t float_to_half_bits(float f) {
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(f)));
}

__device__ inline float half_bits_to_float32(uint32_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h)));
}

// A load through an explicitly global (address space 1) pointer.  A pointer
// chosen with ?: between two kernel arguments, one of which may be null, is
// generic to the compiler; generic (flat) loads count against both vmcnt and
// lgkmcnt, so every wait after one becomes a wait for all outstanding loads.
template <typename T>
__device__ inline T gload(const void* ptr) {
  typedef const __attribute__((address_space(1))) T* global_ptr;
  return *(global_ptr)ptr;
}

// The 8-byte case as one 64-bit load (a uint2 struct load through the cast
// pointer is lowered as a generic copy).
__device__ inline uint2 gload_u2(const void* ptr) {
  const uint64_t v = gload<uint64_t>(ptr);
  return make_uint2((uint32_t)v, (uint32_t)(v >> 32));
}

__device__ inline double shfl_xor_f64(double v, int mask) {
  return __shfl_xor(v, mask, kWave);
}

// Raw buffer access: a 128-bit resource (base, size in bytes) held in SGPRs,
// a per-lane 32-bit offset and a wave-uniform 32-bit offset.  A load whose
// lane offsets are fixed for many chunks then costs no vector address
// arithmetic per chunk; accesses at or past `bytes` read zero and do not
// write.  Word 3 is the gfx9 raw-buffer format (32-bit data).
typedef __amdgpu_buffer_rsrc_t BufRsrc;

__device__ inline BufRsrc buf_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}

// A lane offset past every resource the library builds (each under 2 GiB):
// the load returns zeros and accesses no memory.  The range check covers the
// lane offset only, not the scalar one.
constexpr uint32_t kOutOfRange = 0x80000000u;

__device__ inline u32x4 buf_load_b128(BufRsrc r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0);
}

__device__ inline uint2 buf_load_b64(BufRsrc r, uint32_t voff, uint32_t soff) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)voff, (int)soff, 0);
  return make_uint2(v[0], v[1]);
}

// Weight loads with the nontemporal hint (cache policy nt): a decode step
// streams each active expert's weights once, and without the hint that
// stream displaces the lines its hand-offs and activations reuse (C2 59.4 ->
// 57.4 us, Mixtral T = 1 77.4 -> 73.8, DSV3 T = 1 91.5 -> 86.1).
constexpr int kLoadNt = 2;
__device__ inline u32x4 buf_load_b128_nt(BufRsrc r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, kLoadNt);
}
template <typename T>
__device__ inline T gload_nt(const void* ptr) {
  typedef const __attribute__((address_space(1))) T* global_ptr;
  return __builtin_nontemporal_load((global_ptr)ptr);
}

__device__ inline float buf_load_f32(BufRsrc r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, 0));
}


// Cache policy of a buffer access (the `aux` operand): SC1 alone makes it a
// device-scope access, the form the compiler gives agent-scope atomic loads
// and stores.  A device-scope store is written through to where every XCD
// reads it, and a device-scope load is served from there, never from a
// possibly stale line of this CU's L1 or this XCD's L2.  Data handed between
// workgroups of one launch this way needs no L2 write-back or invalidation.
constexpr int kDeviceScope = 16;
// The same for a load that polls for another workgroup's store, with the
// intrinsic's volatile bit (bit 31, dropped when the instruction is built):
// a plain buffer load in a loop that writes no memory may be hoisted out of
// the loop by the compiler, which would then spin on a stale register.
constexpr int kDevicePoll = kDeviceScope | (int)0x80000000u;

// Direct-to-LDS buffer loads: each lane's 16 (or 4) bytes land at
// lds + lane * 16 (or 4); lds must be wave-uniform.  They count in vmcnt like
// other loads and are not tracked by the compiler's waits for LDS reads, so
// the reader waits explicitly (wait_vmcnt) before a barrier.
template <int AUX = 0>
__device__ inline void dma_b128(BufRsrc r, void* lds, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, (int)voff,
                                           (int)soff, 0, AUX);
}

template <int AUX = 0>
__device__ inline void dma_b32(BufRsrc r, void* lds, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 4, (int)voff,
                                           (int)soff, 0, AUX);
}

// The same 16-byte direct-to-LDS load issued from inline assembly, so the
// compiler does not see an LDS write: a kernel that refills one stage of an
// LDS ring while it reads another then gets no conservative vmcnt(0) before
// its reads (the compiler cannot tell the stages apart).  The caller owns
// the ordering: it waits with wait_vmcnt / s_waitcnt before a barrier.  M0
// is written right before the load and declared clobbered, so the compiler
// reloads it before any later use of its own; the resource is raw SGPR words.
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

__device__ inline i32x4 buf_rsrc_words(const void* base, uint32_t bytes) {
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  const i32x4 r = {(int32_t)(uint32_t)b, (int32_t)((b >> 32) & 0xFFFFu), (int32_t)bytes, 0x00020000};
  return r;
}

__device__ inline uint32_t lds_addr(const void* p) {
  return (uint32_t)reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const void*)p);
}

// The same copy with the nontemporal hint (nt), for weights streamed once per
// call: the batch-1 layer reads each selected expert once, and the hint keeps
// that stream from displacing cached lines (C1 13.6 -> 13.1 us a layer).
__device__ inline void dma_b128_stream(const i32x4& r, uint32_t lds_byte, uint32_t voff, uint32_t soff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen nt lds"
               :: "s"(lds_byte), "v"(voff), "s"(r), "s"(soff) : "memory", "m0");
}

__device__ inline void dma_b128_unseen(const i32x4& r, uint32_t lds_byte, uint32_t voff, uint32_t soff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :: "s"(lds_byte), "v"(voff), "s"(r), "s"(soff) : "memory", "m0");
}

// s_waitcnt vmcnt(N) alone (expcnt and lgkmcnt left at their maxima), gfx9 encoding.
template <int N>
__device__ inline void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Workgroup barrier for LDS data only: waits for this wave's LDS accesses,
// not for its outstanding global loads and stores (which no wave of the
// workgroup reads back), as a __syncthreads() fence would.  The fences are
// workgroup-scope release/acquire restricted to the local address space
// (lgkmcnt(0) and nothing else), and they are real fences to the compiler:
// an empty asm with a memory clobber is not, since alias analysis may assume
// it cannot touch a __shared__ variable whose address never escapes, and
// then fold another wave's store into this thread's view of the variable.
__device__ inline void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

}  // namespace pmoe
