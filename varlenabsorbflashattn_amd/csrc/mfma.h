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

// ---- transposed operand reads from row-major LDS tiles -------------------
// ds_read_b64_tr_b16: within each 16-lane group, source lane 4e+a supplies
// 4 consecutive elements (row e, columns 4a..4a+3 of a 4 x 16 block) and
// output lane i receives column i of that block (rows e = 0..3).
typedef short v4s16 __attribute__((ext_vector_type(4)));
template <typename T>
__device__ __forceinline__ u32x2 lds_tr16(const T *p) {
  typedef v4s16 __attribute__((address_space(3))) * lds_ptr;
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_ptr)(p)));
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

// A operand of a 32x32x16 MFMA whose row index is a column c0 + (l % 32) of
// a row-major LDS tile (stride elements per row) and whose reduction index
// runs over tile rows k0 .. k0+15 in the relabelled order of the C layout:
// B slot (l/32)*8 + t <-> row k0 + (t/4)*8 + (l/32)*4 + t%4.  Two transposed
// reads cover t = 0..3 and t = 4..7.
template <typename T>
__device__ __forceinline__ typename Mfma<T>::v8 tr_operand(const T *tile, int stride, int k0,
                                                           int c0, int lane) {
  const int i = lane & 15, g = lane >> 4;
  const T *p = tile + (k0 + 4 * (g >> 1) + (i >> 2)) * stride + c0 + (g & 1) * 16 + 4 * (i & 3);
  const u32x2 lo = lds_tr16(p);
  const u32x2 hi = lds_tr16(p + 8 * stride);
  return as_v8<T>(join(lo, hi));
}

// 16-bit element e (0..7) of a 16-byte chunk.
__device__ __forceinline__ uint32_t half_of(const u32x4 &x, int e) {
  return (x[e >> 1] >> ((e & 1) * 16)) & 0xffffu;
}

}  // namespace vafa
