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

// ---- row stores of transposed accumulators -------------------------------
// A wave's output block of 32 rows x 32*NDT columns held as NDT transposed
// 32x32 accumulators (acc[i] = columns 32i .. 32i+31 as C rows, the 32
// output rows as C columns): lane l holds row l % 32 at columns
// 32i + 8g + 4(l/32) + e, g, e < 4.  Stored straight from the registers,
// every instruction writes 16 (or, for fp32, 32) bytes into each of 32 rows.
// StagedRows sends the block through the wave's own LDS region instead, so
// every store instruction writes whole rows, 16 bytes per lane.
template <typename O, int NDT>
struct StagedRows {
  static constexpr int kW = 32 * NDT;                        // columns
  // row stride: 16-byte aligned for the row reads, 16 bytes of padding
  static constexpr int kStride = kW * (int)sizeof(O) + 16;   // bytes
  static constexpr int kBytes = 32 * kStride;                // per wave
  static constexpr int kLanesPerRow = kW * (int)sizeof(O) / 16;
  static constexpr int kRowsPerStep = 64 / kLanesPerRow;

  // Writes conv(acc) into `stage` (kBytes, this wave's), then stores row r
  // of the block at out + r * row_stride (elements) for r < rows.  The caller
  // makes `stage` free of other waves' accesses; LDS operations of one wave
  // execute in order, so the reads see this wave's writes.  The lane index is
  // formed here (mbcnt), not taken from the kernel's, so that nothing of the
  // epilogue's addressing is computed ahead of a kernel's main loop and held
  // in registers across it.
  template <typename F>
  static __device__ __forceinline__ void store(const f32x16 (&acc)[NDT], F conv,
                                               unsigned char *stage, O *out,
                                               int64_t row_stride, int rows) {
    static_assert(kLanesPerRow >= 1 && kLanesPerRow <= 64 && 64 % kLanesPerRow == 0,
                  "row width");
    const int lane = (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
    const int r = lane & 31, hf = lane >> 5;
    typedef __attribute__((__vector_size__(4 * sizeof(O)))) O O4;
#pragma unroll
    for (int i = 0; i < NDT; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        O4 w;
#pragma unroll
        for (int e = 0; e < 4; ++e) w[e] = conv(acc[i][g * 4 + e]);
        *reinterpret_cast<O4 *>(stage + r * kStride + (32 * i + 8 * g + 4 * hf) * sizeof(O)) = w;
      }
    asm volatile("" ::: "memory");
    const int c = lane % kLanesPerRow, r0 = lane / kLanesPerRow;
#pragma unroll
    for (int s = 0; s < 32 / kRowsPerStep; ++s) {
      const int rr = s * kRowsPerStep + r0;
      const u32x4 v = *reinterpret_cast<const u32x4 *>(stage + rr * kStride + c * 16);
      if (rr < rows)
        *reinterpret_cast<u32x4 *>(out + rr * row_stride + c * (16 / (int)sizeof(O))) = v;
    }
    asm volatile("" ::: "memory");
  }
};

// A wave's block as 16-bit rows (one pass) or as fp32 rows (split partials:
// two passes over column halves when there are two or more column tiles), in
// a per-wave region of kBytes.
template <typename T, int ND>
struct RowStore {
  using R16 = StagedRows<T, ND>;
  static constexpr int kHalves = ND % 2 == 0 ? 2 : 1;
  using R32 = StagedRows<float, ND / kHalves>;
  static constexpr int kBytes = R16::kBytes > R32::kBytes ? R16::kBytes : R32::kBytes;

  template <typename F>
  static __device__ __forceinline__ void rows16(const f32x16 (&acc)[ND], F conv,
                                                unsigned char *stage, T *out,
                                                int64_t row_stride, int rows) {
    R16::store(acc, conv, stage, out, row_stride, rows);
  }
  // fp32 rows of acc * mul
  static __device__ __forceinline__ void rows32(const f32x16 (&acc)[ND], float mul,
                                                unsigned char *stage, float *out,
                                                int64_t row_stride, int rows) {
    constexpr int NH = ND / kHalves;
#pragma unroll
    for (int hh = 0; hh < kHalves; ++hh)
      R32::store(*reinterpret_cast<const f32x16(*)[NH]>(&acc[hh * NH]),
                 [&](float x) { return x * mul; }, stage, out + hh * NH * 32, row_stride,
                 rows);
  }
};

// 16-bit element e (0..7) of a 16-byte chunk.
__device__ __forceinline__ uint32_t half_of(const u32x4 &x, int e) {
  return (x[e >> 1] >> ((e & 1) * 16)) & 0xffffu;
}

}  // namespace vafa
