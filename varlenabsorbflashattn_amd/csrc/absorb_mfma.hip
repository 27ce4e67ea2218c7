// Absorbed ragged target attention forward on gfx950 matrix cores
// (replaces ta/kernels.py:185-284, the default "alpha" forward).
//
// One workgroup = 4 waves owns up to 128 (token, head) rows of one sample --
// all H heads of 128/H consecutive tokens, token-major, so the rows are one
// contiguous slab of u -- and one key range.  Each 32-key tile of raw X is
// read from HBM once per workgroup (not once per head) and staged in LDS both
// row-major (A operand of S^T = X U^T) and transposed (A operand of
// aX^T += X^T P^T).  After the key loop aX/l is rounded to the input dtype,
// regrouped head-major in LDS and projected by W_V with 16x16x32 MFMAs.
#include "kernels.h"
#include "mfma.h"

namespace vafa {

namespace {

constexpr int kRows = kAbsorbRows;  // 128 rows per workgroup
constexpr int kBK = 32;             // keys per LDS tile
constexpr int kMaxF = 256;          // D_KV handled by this kernel (padded to 32)

template <int FP>
struct AbsSmem {
  static constexpr int XS = FP + 8;   // row-major X stride
  static constexpr int TS = kBK + 4;  // transposed X stride
  static constexpr int kXs = kBK * XS, kXt = FP * TS;
  static constexpr int kBuf = kXs + kXt;
  static constexpr int kLoopBytes = 2 * kBuf * 2;
  static constexpr int kEpiBytes = kRows * XS * 2;  // head-major aX rows
  static constexpr int kBytes = kLoopBytes > kEpiBytes ? kLoopBytes : kEpiBytes;
};

typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f4;

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

// W_V [F, H, DH] -> wvt [H, DH, FP] (zero-padded over f), the B-operand
// layout of the projection (8 consecutive f per lane).
template <typename T>
__global__ __launch_bounds__(256) void transpose_wv_kernel(const T *__restrict__ wv,
                                                           T *__restrict__ wvt, int H, int F,
                                                           int DH, int FP) {
  const int64_t n = (int64_t)H * DH * FP;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const int f = (int)(i % FP);
  const int d = (int)((i / FP) % DH);
  const int h = (int)(i / ((int64_t)FP * DH));
  wvt[i] = f < F ? wv[((int64_t)f * H + h) * DH + d] : static_cast<T>(0.f);
}

template <typename T, int FP, int DH>
__global__ __launch_bounds__(256, 1) void absorb_fwd_kernel(
    const T *__restrict__ u, const T *__restrict__ X, const T *__restrict__ wvt,
    T *__restrict__ O, float *__restrict__ lse, float *__restrict__ part_o,
    float *__restrict__ part_lse, const int32_t *__restrict__ items, int H, int F, float c) {
  using M = Mfma<T>;
  using S = AbsSmem<FP>;
  constexpr int NC = FP / 16;   // S^T reduction chunks
  constexpr int NF = FP / 32;   // aX^T row tiles
  constexpr int CPR = FP / 8;   // 16-byte chunks per padded X row
  extern __shared__ __align__(16) unsigned char smem_raw[];
  T *smem = reinterpret_cast<T *>(smem_raw);

  const PlanItem it = load_item(items, blockIdx.x);
  const int t0 = it.v[0], t1 = it.v[1], k0 = it.v[2], k1 = it.v[3], pbase = it.v[4];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int lrow = lane & 31, lhalf = lane >> 5;
  const int nrows = (t1 - t0) * H;
  const int row = wave * 32 + lrow;  // local (token-major) row
  const bool row_ok = row < nrows;
  const bool wave_active = wave * 32 < nrows;
  const int fchunks = F / 8;         // valid 16-byte chunks per X / u row

  // U^T fragments (B operand of S^T = X U^T)
  typename M::v8 uf[NC];
  const T *urow = u + ((int64_t)t0 * H + row) * F;
#pragma unroll
  for (int cc = 0; cc < NC; ++cc) {
    const int ch = cc * 2 + lhalf;
    u32x4 val = {0u, 0u, 0u, 0u};
    if (row_ok && ch < fchunks) val = *reinterpret_cast<const u32x4 *>(urow + ch * 8);
    uf[cc] = as_v8<T>(val);
  }
  f32x16 acc[NF];
#pragma unroll
  for (int i = 0; i < NF; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[i][r] = 0.f;
  float m_run = kNegInf, l_part = 0.f;

  // tile staging: 4-key x 8-feature quads, (kBK/4)*CPR of them
  constexpr int kQuads = (kBK / 4) * CPR;
  constexpr int kPer = (kQuads + 255) / 256;
  u32x4 stg[kPer][4];
  auto fetch = [&](int kb) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int qi = tid + 256 * i;
      const int kq = qi / CPR, dc = qi % CPR;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int key = kb + kq * 4 + e;
        u32x4 val = {0u, 0u, 0u, 0u};
        if (qi < kQuads && key < k1 && dc < fchunks)
          val = *reinterpret_cast<const u32x4 *>(X + (int64_t)key * F + dc * 8);
        stg[i][e] = val;
      }
    }
  };
  auto put = [&](int buf) {
    T *xs = smem + buf * S::kBuf;
    T *xt = xs + S::kXs;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int qi = tid + 256 * i;
      if (qi >= kQuads) continue;
      const int kq = qi / CPR, dc = qi % CPR;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        *reinterpret_cast<u32x4 *>(xs + (kq * 4 + e) * S::XS + dc * 8) = stg[i][e];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        u32x2 w;
        w[0] = half_of(stg[i][0], e) | (half_of(stg[i][1], e) << 16);
        w[1] = half_of(stg[i][2], e) | (half_of(stg[i][3], e) << 16);
        *reinterpret_cast<u32x2 *>(xt + (dc * 8 + e) * S::TS + kq * 4) = w;
      }
    }
  };

  const int nt = (k1 - k0 + kBK - 1) / kBK;
  if (nt > 0) {
    fetch(k0);
    put(0);
  }
  __syncthreads();
  for (int j = 0; j < nt; ++j) {
    const int kb = k0 + j * kBK;
    if (j + 1 < nt) fetch(kb + kBK);
    if (wave_active) {
      const T *xs = smem + (j & 1) * S::kBuf;
      const T *xt = xs + S::kXs;
      f32x16 s;
#pragma unroll
      for (int r = 0; r < 16; ++r) s[r] = 0.f;
#pragma unroll
      for (int cc = 0; cc < NC; ++cc) {
        const u32x4 a = *reinterpret_cast<const u32x4 *>(xs + lrow * S::XS + cc * 16 + lhalf * 8);
        s = M::mma(as_v8<T>(a), uf[cc], s);
      }
      const bool tail = kb + kBK > k1;
      float mx = kNegInf;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float t = s[r] * c;
        if (tail && kb + (r >> 2) * 8 + lhalf * 4 + (r & 3) >= k1) t = kNegInf;
        s[r] = t;
        mx = fmaxf(mx, t);
      }
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float m_new = fmaxf(m_run, mx);
      const float alpha = fast_exp2(m_run - m_new);
      m_run = m_new;
      float psum = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = fast_exp2(s[r] - m_new);
        s[r] = p;
        psum += p;
      }
      l_part = l_part * alpha + psum;
#pragma unroll
      for (int i = 0; i < NF; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][r] *= alpha;
      typename M::v8 pb[2];
#pragma unroll
      for (int mm = 0; mm < 2; ++mm) pb[mm] = pack8<T>(s, mm * 8);
#pragma unroll
      for (int ft = 0; ft < NF; ++ft) {
        const T *xrow = xt + (ft * 32 + lrow) * S::TS + lhalf * 4;
#pragma unroll
        for (int mm = 0; mm < 2; ++mm) {
          const u32x2 lo = *reinterpret_cast<const u32x2 *>(xrow + mm * 16);
          const u32x2 hi = *reinterpret_cast<const u32x2 *>(xrow + mm * 16 + 8);
          acc[ft] = M::mma(as_v8<T>(join(lo, hi)), pb[mm], acc[ft]);
        }
      }
    }
    if (j + 1 < nt) put((j + 1) & 1);
    __syncthreads();
  }

  // ---- epilogue: aX/l -> LDS (head-major rows, input dtype), then W_V ----
  const float l = l_part + __shfl_xor(l_part, 32, 64);
  const float inv = l > 0.f ? 1.f / l : 0.f;
  const int TT = kRows / H;               // tokens per workgroup
  const int tl = row / H, hh = row % H;   // token / head of this lane's row
  if (row_ok && lhalf == 0) {
    const float lse_v = l > 0.f ? m_run + fast_log2(l) : kNegInf;
    if (pbase < 0)
      lse[(int64_t)t0 * H + row] = lse_v;
    else
      part_lse[(int64_t)(pbase + tl) * H + hh] = lse_v;
  }
  T *axs = smem;  // [kRows][XS], row h*TT + t
  if (wave_active) {
    T *dst = axs + (hh * TT + tl) * S::XS;
#pragma unroll
    for (int ft = 0; ft < NF; ++ft)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        typedef __attribute__((__vector_size__(4 * sizeof(T)))) T T4;
        T4 w;
#pragma unroll
        for (int e = 0; e < 4; ++e) w[e] = static_cast<T>(row_ok ? acc[ft][g * 4 + e] * inv : 0.f);
        *reinterpret_cast<T4 *>(dst + ft * 32 + g * 8 + lhalf * 4) = w;
      }
  }
  __syncthreads();
  // projection: per (head, 16-token tile, 16-wide d tile) one 16x16 output
  const int l16 = lane & 15, lq = lane >> 4;
  const int ntok = t1 - t0;
  const int tiles_per_head = (TT + 15) / 16;
  const int n_tiles = H * tiles_per_head * (DH / 16);
  for (int tile = wave; tile < n_tiles; tile += 4) {
    const int dtile = tile % (DH / 16);
    const int tt = (tile / (DH / 16)) % tiles_per_head;
    const int h = tile / ((DH / 16) * tiles_per_head);
    if (tt * 16 >= ntok) continue;
    f32x4 o = {0.f, 0.f, 0.f, 0.f};
    const T *arow = axs + (h * TT + tt * 16 + l16) * S::XS + lq * 8;
    const T *brow = wvt + ((int64_t)h * DH + dtile * 16 + l16) * FP + lq * 8;
#pragma unroll
    for (int kc = 0; kc < FP / 32; ++kc) {
      const u32x4 a = (tt * 16 + l16 < TT) ? *reinterpret_cast<const u32x4 *>(arow + kc * 32)
                                          : u32x4{0u, 0u, 0u, 0u};
      const u32x4 b = *reinterpret_cast<const u32x4 *>(brow + kc * 32);
      o = Mfma16<T>::mma(as_v8<T>(a), as_v8<T>(b), o);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int tok = tt * 16 + lq * 4 + r;
      if (tok >= ntok) continue;
      const int d = dtile * 16 + l16;
      if (pbase < 0)
        O[((int64_t)(t0 + tok) * H + h) * DH + d] = static_cast<T>(o[r]);
      else
        part_o[((int64_t)(pbase + tok) * H + h) * DH + d] = o[r];
    }
  }
}

template <typename T, int FP, int DH>
void launch_fp(const AbsorbArgs &a, const T *wvt, hipStream_t st) {
  const int smem = AbsSmem<FP>::kBytes;
  hipFuncSetAttribute(reinterpret_cast<const void *>(&absorb_fwd_kernel<T, FP, DH>),
                      hipFuncAttributeMaxDynamicSharedMemorySize, smem);
  hipLaunchKernelGGL((absorb_fwd_kernel<T, FP, DH>), dim3((unsigned)a.n_items), dim3(256), smem,
                     st, (const T *)a.u, (const T *)a.X, wvt, (T *)a.O, a.lse, a.part_o,
                     a.part_lse, a.items, a.H, a.F, a.scale * kLog2e);
}

template <typename T, int DH>
void launch_dh(const AbsorbArgs &a, const T *wvt, int FP, hipStream_t st) {
  switch (FP) {
    case 64: launch_fp<T, 64, DH>(a, wvt, st); break;
    case 128: launch_fp<T, 128, DH>(a, wvt, st); break;
    case 192: launch_fp<T, 192, DH>(a, wvt, st); break;
    case 224: launch_fp<T, 224, DH>(a, wvt, st); break;
    case 256: launch_fp<T, 256, DH>(a, wvt, st); break;
    default: break;
  }
}

inline int padded_f(int F) { return (F + 31) / 32 * 32; }

}  // namespace

// The matrix-core path takes H | 128 with 128/H >= 16 tokens per workgroup,
// D_KV a multiple of 8 that pads (to 32) onto one of the compiled widths,
// and D_H in {16, 32, 64, 128}.
template <typename T>
bool mfma_absorb_supported(int H, int F, int DH) {
  const int FP = padded_f(F);
  const bool f_ok = F % 8 == 0 && F <= kMaxF &&
                    (FP == 64 || FP == 128 || FP == 192 || FP == 224 || FP == 256);
  const bool h_ok = H >= 1 && H <= 8 && (kRows % H) == 0;
  const bool d_ok = DH == 16 || DH == 32 || DH == 64 || DH == 128;
  return f_ok && h_ok && d_ok;
}

int64_t mfma_absorb_wvt_elems(int H, int F, int DH) { return (int64_t)H * DH * padded_f(F); }

template <typename T>
void launch_mfma_absorb_fwd(const AbsorbArgs &a, hipStream_t st) {
  const int FP = padded_f(a.F);
  T *wvt = reinterpret_cast<T *>(a.wvt);
  const int64_t n = (int64_t)a.H * a.DH * FP;
  hipLaunchKernelGGL(transpose_wv_kernel<T>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                     (const T *)a.wv, wvt, a.H, a.F, a.DH, FP);
  if (a.n_items == 0) return;
  switch (a.DH) {
    case 16: launch_dh<T, 16>(a, wvt, FP, st); break;
    case 32: launch_dh<T, 32>(a, wvt, FP, st); break;
    case 64: launch_dh<T, 64>(a, wvt, FP, st); break;
    case 128: launch_dh<T, 128>(a, wvt, FP, st); break;
    default: break;
  }
}

template bool mfma_absorb_supported<bf16>(int, int, int);
template bool mfma_absorb_supported<f16>(int, int, int);
template void launch_mfma_absorb_fwd<bf16>(const AbsorbArgs &, hipStream_t);
template void launch_mfma_absorb_fwd<f16>(const AbsorbArgs &, hipStream_t);

}  // namespace vafa
