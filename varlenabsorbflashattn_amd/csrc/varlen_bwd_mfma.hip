// Packed varlen FlashAttention backward on gfx950 matrix cores.
//
// Two deterministic kernels (no atomics), both recomputing P = exp2(S*c - LSE)
// from the forward's log2-domain LSE (fa/kernels.py:233-494):
//   * dK/dV, key-major: a workgroup owns 128 keys of one head (32 per wave,
//     K and V held in registers as MFMA operands) and walks the segment's
//     queries in blocks of 32 staged in LDS (row-major and transposed):
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
constexpr int kTP = 4;   // transposed-row padding (elements)

// Registers of a [kRB x D] row block staged as 4-row x 8-column quads.
template <int D, int NT>
struct Quads {
  static constexpr int kQuads = (kRB / 4) * (D / 8);
  static constexpr int kPer = (kQuads + NT - 1) / NT;
  u32x4 v[kPer][4];
};

template <typename T, int D, int NT>
__device__ __forceinline__ void load_quads(Quads<D, NT> &s, const T *__restrict__ src, int r0,
                                           int r_end, int H, int h, int t) {
  constexpr int CPR = D / 8;
#pragma unroll
  for (int i = 0; i < Quads<D, NT>::kPer; ++i) {
    const int qi = t + NT * i;
    const int rq = qi / CPR, dc = qi % CPR;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = r0 + rq * 4 + e;
      u32x4 val = {0u, 0u, 0u, 0u};
      if (qi < Quads<D, NT>::kQuads && row < r_end)
        val = *reinterpret_cast<const u32x4 *>(src + ((int64_t)row * H + h) * D + dc * 8);
      s.v[i][e] = val;
    }
  }
}

// Row-major copy (stride RS) and/or transposed copy (stride TS) into LDS.
template <typename T, int D, int NT>
__device__ __forceinline__ void store_quads(const Quads<D, NT> &s, T *rm, int RS, T *tr, int TS,
                                            int t) {
  constexpr int CPR = D / 8;
#pragma unroll
  for (int i = 0; i < Quads<D, NT>::kPer; ++i) {
    const int qi = t + NT * i;
    if (qi >= Quads<D, NT>::kQuads) continue;
    const int rq = qi / CPR, dc = qi % CPR;
    if (rm != nullptr) {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        *reinterpret_cast<u32x4 *>(rm + (rq * 4 + e) * RS + dc * 8) = s.v[i][e];
    }
    if (tr != nullptr) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        u32x2 w;
        w[0] = half_of(s.v[i][0], e) | (half_of(s.v[i][1], e) << 16);
        w[1] = half_of(s.v[i][2], e) | (half_of(s.v[i][3], e) << 16);
        *reinterpret_cast<u32x2 *>(tr + (dc * 8 + e) * TS + rq * 4) = w;
      }
    }
  }
}

// A operand of a transposed product over a 32-row block: lane (lrow, lhalf)
// needs rows 16m + lhalf*4 + {0..3} and 16m + 8 + lhalf*4 + {0..3} of column
// `col` from a transposed LDS tile (row = column index, stride TS).
template <typename T>
__device__ __forceinline__ typename Mfma<T>::v8 tr_operand_t(const T *tr, int TS, int col, int m,
                                                           int lhalf) {
  const T *p = tr + col * TS + m * 16 + lhalf * 4;
  const u32x2 lo = *reinterpret_cast<const u32x2 *>(p);
  const u32x2 hi = *reinterpret_cast<const u32x2 *>(p + 8);
  return as_v8<T>(join(lo, hi));
}

template <int D>
struct DkvSmem {
  static constexpr int RS = D + 8, TS = kRB + kTP;
  static constexpr int kQs = kRB * RS;          // Q row-major
  static constexpr int kQt = D * TS;            // Q transposed
  static constexpr int kElems = 2 * (kQs + kQt);  // Q and dO, both layouts
  static constexpr int kBufBytes = kElems * 2 + 2 * kRB * 4;  // + LSE and delta
  static constexpr int kBytes = 2 * kBufBytes;
};

template <typename T, int D>
__global__ __launch_bounds__(256, D >= 128 ? 1 : 2) void varlen_dkv_kernel(
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
#pragma unroll
  for (int cc = 0; cc < NC; ++cc) {
    u32x4 a = {0u, 0u, 0u, 0u}, b = {0u, 0u, 0u, 0u};
    if (key_ok) {
      const int64_t off = ((int64_t)key * H + h) * D + cc * 16 + lhalf * 8;
      a = *reinterpret_cast<const u32x4 *>(k + off);
      b = *reinterpret_cast<const u32x4 *>(v + off);
    }
    kf[cc] = as_v8<T>(a);
    vf[cc] = as_v8<T>(b);
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
  Quads<D, 128> stg;
  float st_lse = 0.f, st_dl = 0.f;
  auto fetch = [&](int qb) {
    load_quads<T, D, 128>(stg, src, qb, q1, H, h, st);
    if (tid < kRB) {
      const int row = qb + tid;
      st_lse = row < q1 ? lse[(int64_t)row * H + h] : __builtin_inff();
      st_dl = row < q1 ? delta[(int64_t)row * H + h] : 0.f;
    }
  };
  auto put = [&](int buf) {
    unsigned char *base = smem_raw + buf * S::kBufBytes;
    T *qs = reinterpret_cast<T *>(base);
    T *qt = qs + S::kQs;
    T *ds = qt + S::kQt;
    T *dt = ds + S::kQs;
    float *ls = reinterpret_cast<float *>(base + S::kElems * 2);
    if (stage_q)
      store_quads<T, D, 128>(stg, qs, S::RS, qt, S::TS, st);
    else
      store_quads<T, D, 128>(stg, ds, S::RS, dt, S::TS, st);
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
      const T *qt = qs + S::kQs;
      const T *ds_ = qt + S::kQt;
      const T *dt_ = ds_ + S::kQs;
      const float *ls = reinterpret_cast<const float *>(base + S::kElems * 2);
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
          const float p = key_ok ? fast_exp2(s[r] * c - L[e]) : 0.f;
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
      for (int dtile = 0; dtile < ND; ++dtile) {
        const int col = dtile * 32 + lrow;
#pragma unroll
        for (int mm = 0; mm < 2; ++mm) {
          adv[dtile] = M::mma(tr_operand_t<T>(dt_, S::TS, col, mm, lhalf), pb[mm], adv[dtile]);
          adk[dtile] = M::mma(tr_operand_t<T>(qt, S::TS, col, mm, lhalf), sb[mm], adk[dtile]);
        }
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
  static constexpr int RS = D + 8, TS = kRB + kTP;
  static constexpr int kKs = kRB * RS, kKt = D * TS, kVs = kRB * RS;
  static constexpr int kBuf = kKs + kKt + kVs;
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
#pragma unroll
  for (int cc = 0; cc < NC; ++cc) {
    u32x4 a = {0u, 0u, 0u, 0u}, b = {0u, 0u, 0u, 0u};
    if (row_ok) {
      const int64_t off = ((int64_t)qrow * H + h) * D + cc * 16 + lhalf * 8;
      a = *reinterpret_cast<const u32x4 *>(q + off);
      b = *reinterpret_cast<const u32x4 *>(dout + off);
    }
    qf[cc] = as_v8<T>(a);
    dof[cc] = as_v8<T>(b);
  }
  const float Lr = row_ok ? lse[(int64_t)qrow * H + h] : __builtin_inff();
  const float Dr = row_ok ? delta[(int64_t)qrow * H + h] : 0.f;
  f32x16 acc[ND];
#pragma unroll
  for (int i = 0; i < ND; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[i][r] = 0.f;

  // threads 0..127 stage K (row-major + transposed), 128..255 stage V (row-major)
  const bool stage_k = tid < 128;
  const int st = tid & 127;
  Quads<D, 128> stg;
  const int nblk = (k1 - k0 + kRB - 1) / kRB;
  auto put = [&](int buf) {
    T *ks = smem + buf * S::kBuf;
    T *kt = ks + S::kKs;
    T *vs = kt + S::kKt;
    if (stage_k)
      store_quads<T, D, 128>(stg, ks, S::RS, kt, S::TS, st);
    else
      store_quads<T, D, 128>(stg, vs, S::RS, nullptr, 0, st);
  };
  if (nblk > 0) {
    load_quads<T, D, 128>(stg, stage_k ? k : v, k0, k1, H, h, st);
    put(0);
  }
  __syncthreads();
  for (int j = 0; j < nblk; ++j) {
    const int kb = k0 + j * kRB;
    if (j + 1 < nblk) load_quads<T, D, 128>(stg, stage_k ? k : v, kb + kRB, k1, H, h, st);
    if (wave_active) {
      const T *ks = smem + (j & 1) * S::kBuf;
      const T *kt = ks + S::kKs;
      const T *vs = kt + S::kKt;
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
      const bool tail = kb + kRB > k1;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float p = fast_exp2(s[r] * c - Lr);
        if (tail && kb + (r >> 2) * 8 + lhalf * 4 + (r & 3) >= k1) p = 0.f;
        dp[r] = p * (dp[r] - Dr);
      }
      typename M::v8 sb[2];
#pragma unroll
      for (int mm = 0; mm < 2; ++mm) sb[mm] = pack8<T>(dp, mm * 8);
#pragma unroll
      for (int dtile = 0; dtile < ND; ++dtile) {
        const int col = dtile * 32 + lrow;
#pragma unroll
        for (int mm = 0; mm < 2; ++mm)
          acc[dtile] = M::mma(tr_operand_t<T>(kt, S::TS, col, mm, lhalf), sb[mm], acc[dtile]);
      }
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
