// Shared tiling of the absorbed target-attention kernels (gfx950): raw X
// rows streamed through LDS as 32-key tiles by buffer_load ... lds.
#pragma once
#include "kernels.h"
#include "mfma.h"

namespace vafa {
namespace absorb {

constexpr int kBK = 32;     // keys per LDS tile
constexpr int kNBuf = 3;    // LDS ring depth
constexpr int kMaxF = 256;  // D_KV of the compiled widths up to 256 (padded to 32)
constexpr int kMaxFwdF = 512;  // above kMaxF: FP = 512 (2-deep forward ring, one du / dX
                               // workgroup per CU)

// Row padding of the staged tiles (elements), by operand read pattern,
// measured on gfx950 at 12 waves per CU with FP = 256: the 16x16x32 kernels
// read 16 rows x 4 chunks (ds_read_b128) and 16x16 transposed operands
// (ds_read_b64_tr_b16), both fastest at a stride of 16*odd elements (FP + 16:
// 29 and 17 cycles per read against 52 and 29 at FP + 8); the 32x32x16
// kernels read 32 rows x 2 chunks, fastest at 8*odd (FP + 8: 29 against 52).
constexpr int kXPad16 = 16;
constexpr int kXPad32 = 8;

template <int FP, int Pad = kXPad16>
struct AbsSmem {
  static constexpr int CPR = FP / 8;                 // 16-byte chunks per X row
  static constexpr int XS = FP + Pad;                // padded row stride (elements)
  static constexpr int kTile = kBK * XS;             // elements per tile
  // ring depth: 3 tiles, or 2 above 256 features (three 34 KB tiles would
  // leave room for one workgroup per CU)
  static constexpr int kRing = FP > kMaxF ? 2 : kNBuf;
  static constexpr int kLoopBytes = kRing * kTile * 2;
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

// LDS-DMA of 32 consecutive rows [F] of a row slab (src, bytes) into a
// padded [32][XS] LDS block (rows past the slab and chunks past F arrive as
// zeros); each of the workgroup's NW waves moves 32/NW rows, one instruction
// per row.  One descriptor covers the block's valid bytes and the row offset
// sits in the lane offset (the range check covers the lane offset, not
// soffset), added by one volatile VALU add per row so that the compiler does
// not hoist the rows' offsets into separate registers.  Chunks past F carry an
// offset of 2^31 and read as zeros.
template <int FP, int NW, int XS>
__device__ __forceinline__ void dma_block(const void *src, uint32_t bytes, int F, uint32_t base,
                                          int wave, int lane) {
  const u32x4 rs = rsrc_words32(src, bytes);
  const uint32_t off = lane < F / 8 ? (uint32_t)lane * 16u : 0x80000000u;
  if (lane < FP / 8) {
#pragma unroll
    for (int n = 0; n < 32 / NW; ++n) {
      const int r = wave * (32 / NW) + n;
      int32_t voff;
      asm volatile("v_add_u32 %0, %1, %2" : "=v"(voff) : "s"(r * F * 2), "v"(off));
      lds_dma16(rs, base + r * XS * 2, voff);
    }
  }
}

// F padded up to the next width the matrix-core kernels are compiled for
// (64, 128, 192, 224, 256, 512): the padding reads as zeros
// and every store is bounded by F itself, so any F % 8 == 0 up to the
// largest width runs on one of them.
inline int padded_f(int F) {
  const int f32 = (F + 31) / 32 * 32;
  if (f32 <= 64) return 64;
  if (f32 <= 128) return 128;
  if (f32 <= 192) return 192;
  if (f32 <= 224) return 224;
  return f32 <= 256 ? 256 : 512;
}

}  // namespace absorb
}  // namespace vafa
