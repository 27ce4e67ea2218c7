// Device-side helpers shared by every kernel (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "plan_params.h"

namespace vafa {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_inff();

// Online softmax with a lazily updated running max (forward kernels): a
// lane's P sum over one tile at or below kLazyMax (2^8) keeps the running max,
// since every P is then below 2^8, far inside fp32 and 16-bit range.  A larger
// sum (or an infinite one, from the initial running max -kHuge) sends the wave
// through the path that takes the tile's row max and rescales.
constexpr float kLazyMax = 256.0f;
// Initial running max.  Finite, so that masked scores (-inf) still give
// exp2(-inf) = 0 on the first tile instead of -inf + inf = NaN.
constexpr float kHuge = 1e30f;

typedef __bf16 bf16;
typedef _Float16 f16;
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8;
typedef __attribute__((__vector_size__(4 * sizeof(_Float16)))) _Float16 f16x4;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4;
typedef __attribute__((__vector_size__(2 * sizeof(uint32_t)))) uint32_t u32x2;

// ---- scalar conversions ---------------------------------------------------
template <typename T>
__device__ __forceinline__ float to_f(T x) {
  return static_cast<float>(x);
}
template <typename T>
__device__ __forceinline__ T from_f(float x) {
  return static_cast<T>(x);
}
// Round an fp32 value to T and back (models feeding T-typed matrix inputs).
template <typename T>
__device__ __forceinline__ float round_to(float x) {
  return static_cast<float>(static_cast<T>(x));
}

// ---- wave reductions (64 lanes) --------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

// ---- raw buffer loads ----------------------------------------------------
// A buffer resource covering `bytes` from `base`; loads at offsets >= bytes
// return zero, which replaces per-lane bounds branches on tile tails.  The
// base must be wave-uniform and the range below 4 GiB.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
__device__ __forceinline__ rsrc_t make_rsrc(const void *base, int64_t bytes) {
  const int32_t n = bytes > 0x7fffffff ? 0x7fffffff : (int32_t)(bytes < 0 ? 0 : bytes);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, n, 0x00020000);
}
// The same for a wave-uniform byte count below 2^31 (no 64-bit clamp).
__device__ __forceinline__ rsrc_t make_rsrc32(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int32_t)bytes,
                                           0x00020000);
}
__device__ __forceinline__ u32x4 buf_load16(rsrc_t r, int32_t byte_off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0));
}

// 16-byte LDS-DMA load: lane l's 16 bytes from `rsrc` at byte offset `voff`
// land at LDS address lds_base + 16*l (out-of-range offsets write zeros).
// Written as inline asm so that the compiler's automatic waits do not treat
// every later LDS read as dependent on it; callers order it with explicit
// s_waitcnt vmcnt(N) + barrier.  An SALU write of M0 needs one wait state
// before an LDS-DMA instruction reads it, and the compiler does not pad
// inside inline asm, hence the s_nop.
// Raw buffer descriptor words (base, stride 0, num_records, gfx9 flags) for
// use in inline asm.
__device__ __forceinline__ u32x4 rsrc_words(const void *base, int64_t bytes) {
  const uint64_t a = (uint64_t)(uintptr_t)base;
  u32x4 r;
  r[0] = (uint32_t)a;
  r[1] = (uint32_t)(a >> 32) & 0xffffu;
  r[2] = (uint32_t)(bytes > 0x7fffffff ? 0x7fffffff : (bytes < 0 ? 0 : bytes));
  r[3] = 0x00020000u;
  return r;
}

// The same for a wave-uniform byte count below 2^31, formed on the scalar
// unit (no 64-bit clamp: SALU has no signed 64-bit compare, so the clamp of
// rsrc_words runs on the vector unit).
__device__ __forceinline__ u32x4 rsrc_words32(const void *base, uint32_t bytes) {
  const uint64_t a = (uint64_t)(uintptr_t)base;
  u32x4 r;
  r[0] = (uint32_t)a;
  r[1] = (uint32_t)(a >> 32) & 0xffffu;
  r[2] = bytes;
  r[3] = 0x00020000u;
  return r;
}

// A wave-uniform pointer computed on the vector unit (a 64-bit multiply,
// which the scalar unit lacks), moved back to scalar registers so that the
// buffer descriptors built from it stay scalar.
template <typename P>
__device__ __forceinline__ P *uniform_ptr(P *p) {
  const uint64_t a = (uint64_t)(uintptr_t)p;
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)a);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32));
  return reinterpret_cast<P *>((uintptr_t)(((uint64_t)hi << 32) | lo));
}

// min(max(n, 0), hi), made wave-uniform: a clamp compiles to v_med3_i32,
// which would drag the byte counts formed from it (and their 64-bit
// multiplies) onto the vector unit.
__device__ __forceinline__ int uniform_clamp(int n, int hi) {
  n = n < hi ? n : hi;
  n = n > 0 ? n : 0;
  return __builtin_amdgcn_readfirstlane(n);
}

// LDS-DMA (buffer_load ... lds) takes its LDS base in M0, which the asm
// below writes.  M0 is a reserved register, so clang ignores it in a clobber
// list (and warns, silenced here); this is sound only while compiler code in
// these kernels never keeps a value in M0, which tests/test_abi.py checks in
// the generated assembly of every source that uses these helpers.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void lds_dma16(u32x4 r, uint32_t lds_base, int32_t voff) {
  // (an ext_vector_type operand is what binds to an SGPR quad under "s")
  typedef uint32_t sgpr4 __attribute__((ext_vector_type(4)));
  sgpr4 q;
  q.x = (uint32_t)__builtin_amdgcn_readfirstlane((int)r[0]);
  q.y = (uint32_t)__builtin_amdgcn_readfirstlane((int)r[1]);
  q.z = (uint32_t)__builtin_amdgcn_readfirstlane((int)r[2]);
  q.w = (uint32_t)__builtin_amdgcn_readfirstlane((int)r[3]);
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(lds_base), "v"(voff), "s"(q)
               : "memory", "m0");
}

// 4-byte LDS-DMA load: lane l's dword from `rsrc` at byte offset `voff` lands
// at LDS address lds_base + 4*l (out-of-range offsets write zeros).
__device__ __forceinline__ void lds_dma4(u32x4 r, uint32_t lds_base, int32_t voff) {
  typedef uint32_t sgpr4 __attribute__((ext_vector_type(4)));
  sgpr4 q;
  q.x = (uint32_t)__builtin_amdgcn_readfirstlane((int)r[0]);
  q.y = (uint32_t)__builtin_amdgcn_readfirstlane((int)r[1]);
  q.z = (uint32_t)__builtin_amdgcn_readfirstlane((int)r[2]);
  q.w = (uint32_t)__builtin_amdgcn_readfirstlane((int)r[3]);
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dword %1, %2, 0 offen lds"
               :
               : "s"(lds_base), "v"(voff), "s"(q)
               : "memory", "m0");
}
#pragma clang diagnostic pop

// 32-bit LDS address of a pointer into __shared__ memory.
template <typename P>
__device__ __forceinline__ uint32_t lds_addr(const P *p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) P *)(p);
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Max over the lane pairs (l, l^16) and (l, l^32) in registers, without the
// LDS round trip of a shuffle: v_permlane16_swap leaves x holding rows
// (0,0,2,2) and y rows (1,1,3,3) of the 16-lane rows of x, v_permlane32_swap
// leaves x = (lo,lo) and y = (hi,hi) halves.  Inline asm with explicit wait
// states around the swap (the compiler's builtin model of these swaps does
// not track that both outputs change).
__device__ __forceinline__ float max_xor16(float x) {
  float y;
  asm volatile("v_mov_b32 %1, %0\n\ts_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1"
               : "+v"(x), "=&v"(y));
  return fmaxf(x, y);
}
__device__ __forceinline__ float max_xor32(float x) {
  float y;
  asm volatile("v_mov_b32 %1, %0\n\ts_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1"
               : "+v"(x), "=&v"(y));
  return fmaxf(x, y);
}

// Wave-uniform "any lane" vote.
__device__ __forceinline__ bool wave_any(bool p) { return __builtin_amdgcn_ballot_w64(p) != 0; }

// A 32-byte plan item (see plan.cpp for the per-section field meaning).
struct alignas(16) PlanItem {
  int32_t v[8];
};

// Every lane of a workgroup reads the same item; readfirstlane makes that
// visible to the compiler, so item-derived ranges, addresses and buffer
// descriptors live in scalar registers and steer scalar branches.
__device__ __forceinline__ PlanItem load_item(const int32_t *plan, int64_t idx) {
  const u32x4 *p = reinterpret_cast<const u32x4 *>(plan + idx * 8);
  u32x4 a = p[0], b = p[1];
  PlanItem it;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    it.v[i] = __builtin_amdgcn_readfirstlane((int32_t)a[i]);
    it.v[4 + i] = __builtin_amdgcn_readfirstlane((int32_t)b[i]);
  }
  return it;
}

}  // namespace vafa
