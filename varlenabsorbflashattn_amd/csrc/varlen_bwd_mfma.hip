// Packed varlen FlashAttention backward on gfx950 matrix cores.
//
// Two deterministic kernels (no atomics), both recomputing P = exp2(S*c - LSE)
// from the forward's log2-domain LSE (fa/kernels.py:233-494):
//   * dK/dV, key-major: a workgroup owns 128 keys of one head (32 per wave,
//     K and V held in registers as MFMA operands) and walks the segment's
//     queries in blocks of 32 staged row-major in LDS (the transposed
//     operands Q^T, dO^T come from ds_read_b64_tr_b16):
//       S = Q K^T, dP = dO V^T, dS = P (dP - delta),
//       dV^T += dO^T P,  dK^T += Q^T dS           (4 products per block)
//   * dQ, query-major over the forward's plan items (including split-K
//     partials): S^T = K Q^T, dP^T = V dO^T, dQ^T += K^T dS^T.
// The row statistics of the dQ kernel stay per lane (lane <-> query row);
// the dK/dV kernel reads LSE and delta of its 32-row block from LDS.
#include "kernels.h"
#include "mfma.h"

namespace vafa {

namespace {

constexpr int kRB = 32;  // rows per staged block (queries for dK/dV, keys for dQ)

// A [kRB x D] block of a [T, H, D] tensor staged through registers: 16-byte
// chunks, rows past the buffer range read as zero.
template <int D, int NT>
struct Rows {
  static constexpr int kChunks = kRB * D / 8;
  static constexpr int kPer = (kChunks + NT - 1) / NT;
  u32x4 v[kPer];
};

template <typename T, int D, int NT>
__device__ __forceinline__ void load_rows(Rows<D, NT> &s, const T *__restrict__ src, int r0,
                                          int r_end, int H, int h, int t) {
  constexpr int CPR = D / 8;
  const int rows = r_end - r0 < kRB ? r_end - r0 : kRB;
  const rsrc_t rs = make_rsrc(src + (int64_t)r0 * H * D, (int64_t)rows * H * D * 2);
#pragma unroll
  for (int i = 0; i < Rows<D, NT>::kPer; ++i) {
    const int ci = t + NT * i;
    const int row = ci < Rows<D, NT>::kChunks ? ci / CPR : kRB;
    s.v[i] = buf_load16(rs, (row * H + h) * D * 2 + (ci % CPR) * 16);
  }
}

template <typename T, int D, int NT>
__device__ __forceinline__ void store_rows(const Rows<D, NT> &s, T *dst, int RS, int t) {
  constexpr int CPR = D / 8;
#pragma unroll
  for (int i = 0; i < Rows<D, NT>::kPer; ++i) {
    const int ci = t + NT * i;
    if (ci < Rows<D, NT>::kChunks)
      *reinterpret_cast<u32x4 *>(dst + (ci / CPR) * RS + (ci % CPR) * 8) = s.v[i];
  }
}

template <int D>
struct DkvSmem {
  static constexpr int RS = D + 8;
  static constexpr int kQs = kRB * RS;                        // Q (or dO) row-major
  static constexpr int kBufBytes = 2 * kQs * 2 + 2 * kRB * 4;  // Q, dO, LSE, delta
  static constexpr int kBytes = 2 * kBufBytes;
};

template <typename T, int D>
__global__ __launch_bounds__(256, 2) void varlen_dkv_kernel(
    const T *__restrict__ q, const T *__restrict__ k, const T *__restrict__ v,
    const T *__restrict__ dout, const float *__restrict__ lse, const float *__restrict__ delta,
    T *__restrict__ dk, T *__restrict__ dv, const int32_t *__restrict__ items, int H, float c,
    float scale) {
  using M = Mfma<T>;
  using S = DkvSmem<D>;
  constexpr int NC = D / 16, ND = D / 32;
  extern __shared__ __align__(16) unsigned char smem_raw[];

  const int item = blockIdx.x / H, h = blockIdx.x % H;
  const PlanItem it = load_item(items, item);
  const int k0 = it.v[0], k1 = it.v[1], q0 = it.v[2], q1 = it.v[3];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int lrow = lane & 31, lhalf = lane >> 5;
  const int key = k0 + wave * 32 + lrow;
  const bool key_ok = key < k1;
  const bool wave_active = k0 + wave * 32 < k1;

  typename M::v8 kf[NC], vf[NC];
  {
    const int nk = k1 - k0;
    const rsrc_t rk = make_rsrc(k + (int64_t)k0 * H * D, (int64_t)nk * H * D * 2);
    const rsrc_t rv = make_rsrc(v + (int64_t)k0 * H * D, (int64_t)nk * H * D * 2);
    const int off = ((wave * 32 + lrow) * H + h) * D * 2 + lhalf * 16;
#pragma unroll
    for (int cc = 0; cc < NC; ++cc) {
      kf[cc] = as_v8<T>(buf_load16(rk, off + cc * 32));
      vf[cc] = as_v8<T>(buf_load16(rv, off + cc * 32));
    }
  }
  f32x16 adk[ND], adv[ND];
#pragma unroll
  for (int i = 0; i < ND; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) adk[i][r] = adv[i][r] = 0.f;

  // threads 0..127 stage Q, 128..255 stage dO; threads < 32 also fetch LSE and
  // delta (past-the-end rows get LSE=+inf so their P is exactly 0)
  const bool stage_q = tid < 128;
  const int st = tid & 127;
  const T *src = stage_q ? q : dout;
  Rows<D, 128> stg;
  float st_lse = 0.f, st_dl = 0.f;
  auto fetch = [&](int qb) {
    load_rows<T, D, 128>(stg, src, qb, q1, H, h, st);
    if (tid < kRB) {
      const int row = qb + tid;
      st_lse = row < q1 ? lse[(int64_t)row * H + h] : __builtin_inff();
      st_dl = row < q1 ? delta[(int64_t)row * H + h] : 0.f;
    }
  };
  auto put = [&](int buf) {
    unsigned char *base = smem_raw + buf * S::kBufBytes;
    T *qs = reinterpret_cast<T *>(base);
    store_rows<T, D, 128>(stg, stage_q ? qs : qs + S::kQs, S::RS, st);
    float *ls = reinterpret_cast<float *>(base + 2 * S::kQs * 2);
    if (tid < kRB) {
      ls[tid] = st_lse;
      ls[kRB + tid] = st_dl;
    }
  };

  const int nblk = (q1 - q0 + kRB - 1) / kRB;
  if (nblk > 0) {
    fetch(q0);
    put(0);
  }
  __syncthreads();
  for (int j = 0; j < nblk; ++j) {
    if (j + 1 < nblk) fetch(q0 + (j + 1) * kRB);
    if (wave_active) {
      const unsigned char *base = smem_raw + (j & 1) * S::kBufBytes;
      const T *qs = reinterpret_cast<const T *>(base);
      const T *ds_ = qs + S::kQs;
      const float *ls = reinterpret_cast<const float *>(base + 2 * S::kQs * 2);
      f32x16 s, dp;
#pragma unroll
      for (int r = 0; r < 16; ++r) s[r] = dp[r] = 0.f;
#pragma unroll
      for (int cc = 0; cc < NC; ++cc) {
        const u32x4 a = *reinterpret_cast<const u32x4 *>(qs + lrow * S::RS + cc * 16 + lhalf * 8);
        s = M::mma(as_v8<T>(a), kf[cc], s);
        const u32x4 b = *reinterpret_cast<const u32x4 *>(ds_ + lrow * S::RS + cc * 16 + lhalf * 8);
        dp = M::mma(as_v8<T>(b), vf[cc], dp);
      }
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x4 L = *reinterpret_cast<const f32x4 *>(ls + g * 8 + lhalf * 4);
        const f32x4 Dl = *reinterpret_cast<const f32x4 *>(ls + kRB + g * 8 + lhalf * 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = g * 4 + e;
          const float p = key_ok ? fast_exp2(__builtin_fmaf(s[r], c, -L[e])) : 0.f;
          s[r] = p;
          dp[r] = p * (dp[r] - Dl[e]);
        }
      }
      typename M::v8 pb[2], sb[2];
#pragma unroll
      for (int mm = 0; mm < 2; ++mm) {
        pb[mm] = pack8<T>(s, mm * 8);
        sb[mm] = pack8<T>(dp, mm * 8);
      }
#pragma unroll
      for (int dtile = 0; dtile < ND; ++dtile)
#pragma unroll
        for (int mm = 0; mm < 2; ++mm) {
          adv[dtile] = M::mma(tr_operand<T>(ds_, S::RS, mm * 16, dtile * 32, lane), pb[mm],
                              adv[dtile]);
          adk[dtile] = M::mma(tr_operand<T>(qs, S::RS, mm * 16, dtile * 32, lane), sb[mm],
                              adk[dtile]);
        }
    }
    if (j + 1 < nblk) put((j + 1) & 1);
    __syncthreads();
  }

  if (!key_ok) return;
  typedef __attribute__((__vector_size__(4 * sizeof(T)))) T T4;
  T *dkr = dk + ((int64_t)key * H + h) * D;
  T *dvr = dv + ((int64_t)key * H + h) * D;
#pragma unroll
  for (int dtile = 0; dtile < ND; ++dtile)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      T4 wk, wv;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        wk[e] = static_cast<T>(adk[dtile][g * 4 + e] * scale);
        wv[e] = static_cast<T>(adv[dtile][g * 4 + e]);
      }
      const int d = dtile * 32 + g * 8 + lhalf * 4;
      *reinterpret_cast<T4 *>(dkr + d) = wk;
      *reinterpret_cast<T4 *>(dvr + d) = wv;
    }
}

template <int D>
struct DqSmem {
  static constexpr int RS = D + 8;
  static constexpr int kKs = kRB * RS;
  static constexpr int kBuf = 2 * kKs;  // K and V row-major
  static constexpr int kBytes = 2 * kBuf * 2;
};

template <typename T, int D>
__global__ __launch_bounds__(256, D >= 256 ? 1 : 2) void varlen_dq_kernel(
    const T *__restrict__ q, const T *__restrict__ k, const T *__restrict__ v,
    const T *__restrict__ dout, const float *__restrict__ lse, const float *__restrict__ delta,
    T *__restrict__ dq, float *__restrict__ part_dq, const int32_t *__restrict__ items, int H,
    float c, float scale) {
  using M = Mfma<T>;
  using S = DqSmem<D>;
  constexpr int NC = D / 16, ND = D / 32;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  T *smem = reinterpret_cast<T *>(smem_raw);

  const int item = blockIdx.x / H, h = blockIdx.x % H;
  const PlanItem it = load_item(items, item);
  const int q0 = it.v[0], q1 = it.v[1], k0 = it.v[2], k1 = it.v[3], pbase = it.v[4];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int lrow = lane & 31, lhalf = lane >> 5;
  const int qrow = q0 + wave * 32 + lrow;
  const bool row_ok = qrow < q1;
  const bool wave_active = q0 + wave * 32 < q1;

  typename M::v8 qf[NC], dof[NC];
  {
    const int64_t nb = (int64_t)(q1 - q0) * H * D * 2;
    const rsrc_t rq = make_rsrc(q + (int64_t)q0 * H * D, nb);
    const rsrc_t rd = make_rsrc(dout + (int64_t)q0 * H * D, nb);
    const int off = ((wave * 32 + lrow) * H + h) * D * 2 + lhalf * 16;
#pragma unroll
    for (int cc = 0; cc < NC; ++cc) {
      qf[cc] = as_v8<T>(buf_load16(rq, off + cc * 32));
      dof[cc] = as_v8<T>(buf_load16(rd, off + cc * 32));
    }
  }
  const float Lr = row_ok ? lse[(int64_t)qrow * H + h] : __builtin_inff();
  const float Dr = row_ok ? delta[(int64_t)qrow * H + h] : 0.f;
  f32x16 acc[ND];
#pragma unroll
  for (int i = 0; i < ND; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[i][r] = 0.f;

  // threads 0..127 stage K, 128..255 stage V (both row-major)
  const bool stage_k = tid < 128;
  const int st = tid & 127;
  const T *src = stage_k ? k : v;
  Rows<D, 128> stg;
  const int nblk = (k1 - k0 + kRB - 1) / kRB;
  auto put = [&](int buf) {
    T *ks = smem + buf * S::kBuf;
    store_rows<T, D, 128>(stg, stage_k ? ks : ks + S::kKs, S::RS, st);
  };
  if (nblk > 0) {
    load_rows<T, D, 128>(stg, src, k0, k1, H, h, st);
    put(0);
  }
  __syncthreads();
  for (int j = 0; j < nblk; ++j) {
    const int kb = k0 + j * kRB;
    if (j + 1 < nblk) load_rows<T, D, 128>(stg, src, kb + kRB, k1, H, h, st);
    if (wave_active) {
      const T *ks = smem + (j & 1) * S::kBuf;
      const T *vs = ks + S::kKs;
      f32x16 s, dp;
#pragma unroll
      for (int r = 0; r < 16; ++r) s[r] = dp[r] = 0.f;
#pragma unroll
      for (int cc = 0; cc < NC; ++cc) {
        const u32x4 a = *reinterpret_cast<const u32x4 *>(ks + lrow * S::RS + cc * 16 + lhalf * 8);
        s = M::mma(as_v8<T>(a), qf[cc], s);
        const u32x4 b = *reinterpret_cast<const u32x4 *>(vs + lrow * S::RS + cc * 16 + lhalf * 8);
        dp = M::mma(as_v8<T>(b), dof[cc], dp);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = fast_exp2(__builtin_fmaf(s[r], c, -Lr));
        dp[r] = p * (dp[r] - Dr);
      }
      if (kb + kRB > k1) {
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (kb + (r >> 2) * 8 + lhalf * 4 + (r & 3) >= k1) dp[r] = 0.f;
      }
      typename M::v8 sb[2];
#pragma unroll
      for (int mm = 0; mm < 2; ++mm) sb[mm] = pack8<T>(dp, mm * 8);
#pragma unroll
      for (int dtile = 0; dtile < ND; ++dtile)
#pragma unroll
        for (int mm = 0; mm < 2; ++mm)
          acc[dtile] = M::mma(tr_operand<T>(ks, S::RS, mm * 16, dtile * 32, lane), sb[mm],
                              acc[dtile]);
    }
    if (j + 1 < nblk) put((j + 1) & 1);
    __syncthreads();
  }

  if (!row_ok) return;
  if (pbase < 0) {
    typedef __attribute__((__vector_size__(4 * sizeof(T)))) T T4;
    T *row = dq + ((int64_t)qrow * H + h) * D;
#pragma unroll
    for (int dtile = 0; dtile < ND; ++dtile)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        T4 w;
#pragma unroll
        for (int e = 0; e < 4; ++e) w[e] = static_cast<T>(acc[dtile][g * 4 + e] * scale);
        *reinterpret_cast<T4 *>(row + dtile * 32 + g * 8 + lhalf * 4) = w;
      }
  } else {
    float *row = part_dq + ((int64_t)(pbase + qrow - q0) * H + h) * D;
#pragma unroll
    for (int dtile = 0; dtile < ND; ++dtile)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        f32x4 w;
#pragma unroll
        for (int e = 0; e < 4; ++e) w[e] = acc[dtile][g * 4 + e] * scale;
        *reinterpret_cast<f32x4 *>(row + dtile * 32 + g * 8 + lhalf * 4) = w;
      }
  }
}

}  // namespace

template <typename T, int D>
void launch_mfma_varlen_dkv(const VarlenArgs &a, hipStream_t st) {
  if (a.n_kv == 0) return;
  const int smem = DkvSmem<D>::kBytes;
  hipFuncSetAttribute(reinterpret_cast<const void *>(&varlen_dkv_kernel<T, D>),
                      hipFuncAttributeMaxDynamicSharedMemorySize, smem);
  hipLaunchKernelGGL((varlen_dkv_kernel<T, D>), dim3((unsigned)(a.n_kv * a.H)), dim3(256), smem,
                     st, (const T *)a.q, (const T *)a.k, (const T *)a.v, (const T *)a.dout,
                     a.lse_in, a.delta, (T *)a.dk, (T *)a.dv, a.kv_items, a.H, a.scale * kLog2e,
                     a.scale);
}

template <typename T, int D>
void launch_mfma_varlen_dq(const VarlenArgs &a, hipStream_t st) {
  if (a.n_items == 0) return;
  const int smem = DqSmem<D>::kBytes;
  hipFuncSetAttribute(reinterpret_cast<const void *>(&varlen_dq_kernel<T, D>),
                      hipFuncAttributeMaxDynamicSharedMemorySize, smem);
  hipLaunchKernelGGL((varlen_dq_kernel<T, D>), dim3((unsigned)(a.n_items * a.H)), dim3(256),
                     smem, st, (const T *)a.q, (const T *)a.k, (const T *)a.v,
                     (const T *)a.dout, a.lse_in, a.delta, (T *)a.dq, a.part_o, a.items, a.H,
                     a.scale * kLog2e, a.scale);
}

#define VAFA_INST(T, D)                                                           \
  template void launch_mfma_varlen_dkv<T, D>(const VarlenArgs &, hipStream_t);    \
  template void launch_mfma_varlen_dq<T, D>(const VarlenArgs &, hipStream_t);
VAFA_INST(bf16, 32)
VAFA_INST(bf16, 64)
VAFA_INST(bf16, 128)
VAFA_INST(f16, 32)
VAFA_INST(f16, 64)
VAFA_INST(f16, 128)
#undef VAFA_INST

}  // namespace vafa
