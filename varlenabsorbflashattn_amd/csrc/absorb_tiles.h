// Shared tiling of the absorbed target-attention kernels (gfx950): raw X
// rows streamed through LDS as 32-key tiles by buffer_load ... lds.
#pragma once
#include "kernels.h"
#include "mfma.h"

namespace vafa {
namespace absorb {

constexpr int kWaves = kAbsorbRows / 32;  // 2 waves x 32 rows
constexpr int kThreads = 64 * kWaves;
constexpr int kBK = 32;                   // keys per LDS tile
constexpr int kNBuf = 3;                  // LDS ring depth
constexpr int kMaxF = 256;                // D_KV handled by this kernel (padded to 32)

#ifndef VAFA_ABS_XPAD
#define VAFA_ABS_XPAD 8
#endif

template <int FP>
struct AbsSmem {
  static constexpr int CPR = FP / 8;                 // 16-byte chunks per X row
  static constexpr int XS = FP + VAFA_ABS_XPAD;      // padded row stride (elements)
  static constexpr int kTile = kBK * XS;             // elements per tile
  static constexpr int kLoopBytes = kNBuf * kTile * 2;
  static constexpr int kEpiBytes = kAbsorbRows * XS * 2;
  static constexpr int kBytes = kLoopBytes > kEpiBytes ? kLoopBytes : kEpiBytes;
};

template <typename T>
struct Mfma16;
template <>
struct Mfma16<bf16> {
  static __device__ __forceinline__ f32x4 mma(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};
template <>
struct Mfma16<f16> {
  static __device__ __forceinline__ f32x4 mma(f16x8 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

// Issue the LDS-DMA loads of one 32-key tile: one instruction per X row,
// lanes 0..CPR-1 each move one 16-byte chunk to the row's padded LDS slot
// (keys past k_end and chunks past D_KV arrive as zeros).  Every wave issues
// kBK / kWaves instructions per tile, which keeps vmcnt accounting uniform.
template <typename T, int FP>
__device__ __forceinline__ void issue_tile(const T *__restrict__ X, int kb, int k_end, int F,
                                           T *tile, int wave, int lane) {
  using S = AbsSmem<FP>;
  const int rows = k_end - kb < kBK ? (k_end - kb > 0 ? k_end - kb : 0) : kBK;
  const u32x4 rx = rsrc_words(X + (int64_t)kb * F, (int64_t)rows * F * 2);
  // chunks past D_KV get an offset >= 2^31, past any buffer range
  const uint32_t off = lane < F / 8 ? (uint32_t)lane * 16u : 0x80000000u;
  const uint32_t base = lds_addr(tile);
  if (lane < S::CPR) {
#pragma unroll
    for (int n = 0; n < kBK / kWaves; ++n) {
      const int r = wave * (kBK / kWaves) + n;
      lds_dma16(rx, base + r * S::XS * 2, (int32_t)(off + (uint32_t)(r * F * 2)));
    }
  }
}

// LDS-address-space views: offsets from one per-lane base fold into the
// instructions' immediate offsets instead of living in registers.
template <typename T>
using lds_cptr = const __attribute__((address_space(3))) T *;

template <typename T>
__device__ __forceinline__ lds_cptr<T> as_lds(const T *p) {
  return (lds_cptr<T>)(p);
}
template <typename T>
__device__ __forceinline__ u32x4 lds_ld16(lds_cptr<T> p) {
  return *(lds_cptr<u32x4>)(p);
}
template <typename T>
__device__ __forceinline__ u32x2 lds_tr8(lds_cptr<T> p) {
  typedef __attribute__((address_space(3))) v4s16 *tr_ptr;
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((tr_ptr)(p)));
}

inline int padded_f(int F) { return (F + 31) / 32 * 32; }

}  // namespace absorb
}  // namespace vafa
