// Matrix-core helpers for gfx950: 32x32x16 MFMA on 16-bit inputs.
//
// Operand layout of v_mfma_f32_32x32x16_{bf16,f16} (wave64):
//   A (32 x 16): lane l holds A[l % 32][(l / 32) * 8 + t], t = 0..7
//   B (16 x 32): lane l holds B[(l / 32) * 8 + t][l % 32]
//   C (32 x 32): lane l holds C[(r / 4) * 8 + (l / 32) * 4 + r % 4][l % 32],
//                r = 0..15
// The kernels compute transposed products (S^T = K Q^T, O^T = V^T P^T) so
// that the C column -- one query row -- is owned by one lane pair (l, l^32)
// and the softmax statistics stay in registers.  The P^T accumulator is fed
// back as the B operand of the next product by relabelling the key axis:
// B slot (l/32)*8 + t of 16-key chunk m is key 16m + (t/4)*8 + (l/32)*4 + t%4,
// which is exactly what C register r = 8m + t of that lane holds.
#pragma once
#include "common.h"

namespace vafa {

template <typename T>
struct Mfma;

template <>
struct Mfma<bf16> {
  typedef bf16x8 v8;
  static __device__ __forceinline__ f32x16 mma(v8 a, v8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};

template <>
struct Mfma<f16> {
  typedef f16x8 v8;
  static __device__ __forceinline__ f32x16 mma(v8 a, v8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

// Pack 8 fp32 values (registers r0..r0+7 of an accumulator) to a 16-bit x8.
template <typename T>
__device__ __forceinline__ typename Mfma<T>::v8 pack8(const f32x16 &x, int r0) {
  typename Mfma<T>::v8 out;
#pragma unroll
  for (int t = 0; t < 8; ++t) out[t] = static_cast<T>(x[r0 + t]);
  return out;
}

// Reinterpret 16 bytes as an MFMA 16-bit x8 operand.
template <typename T>
__device__ __forceinline__ typename Mfma<T>::v8 as_v8(u32x4 x) {
  return __builtin_bit_cast(typename Mfma<T>::v8, x);
}

__device__ __forceinline__ u32x4 join(u32x2 a, u32x2 b) {
  u32x4 r;
  r[0] = a[0];
  r[1] = a[1];
  r[2] = b[0];
  r[3] = b[1];
  return r;
}

// 16-bit element e (0..7) of a 16-byte chunk.
__device__ __forceinline__ uint32_t half_of(const u32x4 &x, int e) {
  return (x[e >> 1] >> ((e & 1) * 16)) & 0xffffu;
}

}  // namespace vafa
