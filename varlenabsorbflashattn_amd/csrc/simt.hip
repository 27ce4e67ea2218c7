// Wave-per-row kernels for every dtype and head size.
//
// One wave64 owns one (query row, head) -- or one (key, head) in the dK/dV
// pass -- and its lanes split the feature axis; dot products are wave
// reductions and the online softmax runs in the log2 domain exactly like the
// matrix-core kernels.  These kernels carry the fp32 path (absorb with
// bf16=False, ta/interface.py:371, 422-427; varlen with fp32 inputs,
// fa/interface.py:163) and every shape the matrix-core kernels do not take.
// They read the same plans and write the same partial / combine layouts.
#include "common.h"
#include "kernels.h"

namespace vafa {

namespace {

constexpr int kMaxPerLane = 8;  // feature widths up to 512

// ---------------------------------------------------------------------------
// Varlen forward.  Item {q0,q1,k0,k1,pbase,...}; grid = n_items * H.
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void simt_varlen_fwd(
    const T *__restrict__ q, const T *__restrict__ k, const T *__restrict__ v,
    T *__restrict__ o, float *__restrict__ lse, float *__restrict__ part_o,
    float *__restrict__ part_lse, const int32_t *__restrict__ items, int H, int D, float c) {
  const int item = blockIdx.x / H, h = blockIdx.x % H;
  const PlanItem it = load_item(items, item);
  const int q0 = it.v[0], q1 = it.v[1], k0 = it.v[2], k1 = it.v[3], pbase = it.v[4];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int per = (D + 63) / 64;
  for (int row = q0 + wave; row < q1; row += 4) {
    float qv[kMaxPerLane], acc[kMaxPerLane];
    for (int i = 0; i < per; ++i) {
      int d = lane + 64 * i;
      qv[i] = d < D ? to_f(q[((int64_t)row * H + h) * D + d]) : 0.f;
      acc[i] = 0.f;
    }
    float m = kNegInf, l = 0.f;
    for (int j = k0; j < k1; ++j) {
      const T *kr = k + ((int64_t)j * H + h) * D;
      float s = 0.f;
      for (int i = 0; i < per; ++i) {
        int d = lane + 64 * i;
        if (d < D) s += qv[i] * to_f(kr[d]);
      }
      const float t = wave_sum(s) * c;
      const float mn = fmaxf(m, t);
      const float alpha = fast_exp2(m - mn);
      const float p = fast_exp2(t - mn);
      l = l * alpha + p;
      const float pr = round_to<T>(p);
      const T *vr = v + ((int64_t)j * H + h) * D;
      for (int i = 0; i < per; ++i) {
        int d = lane + 64 * i;
        acc[i] = acc[i] * alpha + (d < D ? pr * to_f(vr[d]) : 0.f);
      }
      m = mn;
    }
    const float inv = l > 0.f ? 1.f / l : 0.f;
    const float lse_v = l > 0.f ? m + fast_log2(l) : kNegInf;
    if (pbase < 0) {
      for (int i = 0; i < per; ++i) {
        int d = lane + 64 * i;
        if (d < D) o[((int64_t)row * H + h) * D + d] = from_f<T>(acc[i] * inv);
      }
      if (lane == 0) lse[(int64_t)row * H + h] = lse_v;
    } else {
      const int64_t pr_row = pbase + (row - q0);
      for (int i = 0; i < per; ++i) {
        int d = lane + 64 * i;
        if (d < D) part_o[(pr_row * H + h) * D + d] = acc[i] * inv;
      }
      if (lane == 0) part_lse[pr_row * H + h] = lse_v;
    }
  }
}

// ---------------------------------------------------------------------------
// Varlen dQ (same items as the forward).  Split items write scaled fp32
// partial rows that combine_sum adds up in split order.
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void simt_varlen_dq(
    const T *__restrict__ q, const T *__restrict__ k, const T *__restrict__ v,
    const T *__restrict__ dout, const float *__restrict__ lse,
    const float *__restrict__ delta, T *__restrict__ dq, float *__restrict__ part_dq,
    const int32_t *__restrict__ items, int H, int D, float c, float scale) {
  const int item = blockIdx.x / H, h = blockIdx.x % H;
  const PlanItem it = load_item(items, item);
  const int q0 = it.v[0], q1 = it.v[1], k0 = it.v[2], k1 = it.v[3], pbase = it.v[4];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int per = (D + 63) / 64;
  for (int row = q0 + wave; row < q1; row += 4) {
    float qv[kMaxPerLane], dov[kMaxPerLane], acc[kMaxPerLane];
    for (int i = 0; i < per; ++i) {
      int d = lane + 64 * i;
      qv[i] = d < D ? to_f(q[((int64_t)row * H + h) * D + d]) : 0.f;
      dov[i] = d < D ? to_f(dout[((int64_t)row * H + h) * D + d]) : 0.f;
      acc[i] = 0.f;
    }
    const float L = lse[(int64_t)row * H + h], dl = delta[(int64_t)row * H + h];
    for (int j = k0; j < k1; ++j) {
      const T *kr = k + ((int64_t)j * H + h) * D;
      const T *vr = v + ((int64_t)j * H + h) * D;
      float s = 0.f, dp = 0.f;
      for (int i = 0; i < per; ++i) {
        int d = lane + 64 * i;
        if (d < D) {
          s += qv[i] * to_f(kr[d]);
          dp += dov[i] * to_f(vr[d]);
        }
      }
      s = wave_sum(s);
      dp = wave_sum(dp);
      const float p = fast_exp2(s * c - L);
      const float ds = round_to<T>(p * (dp - dl));
      for (int i = 0; i < per; ++i) {
        int d = lane + 64 * i;
        if (d < D) acc[i] += ds * to_f(kr[d]);
      }
    }
    for (int i = 0; i < per; ++i) {
      int d = lane + 64 * i;
      if (d >= D) continue;
      if (pbase < 0)
        dq[((int64_t)row * H + h) * D + d] = from_f<T>(acc[i] * scale);
      else
        part_dq[((int64_t)(pbase + row - q0) * H + h) * D + d] = acc[i] * scale;
    }
  }
}

// ---------------------------------------------------------------------------
// Varlen dK/dV.  Item {k0,k1,q0,q1,...}; one wave per (key, head).
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void simt_varlen_dkv(
    const T *__restrict__ q, const T *__restrict__ k, const T *__restrict__ v,
    const T *__restrict__ dout, const float *__restrict__ lse,
    const float *__restrict__ delta, T *__restrict__ dk, T *__restrict__ dv,
    const int32_t *__restrict__ items, int H, int D, float c, float scale) {
  const int item = blockIdx.x / H, h = blockIdx.x % H;
  const PlanItem it = load_item(items, item);
  const int k0 = it.v[0], k1 = it.v[1], q0 = it.v[2], q1 = it.v[3];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int per = (D + 63) / 64;
  for (int key = k0 + wave; key < k1; key += 4) {
    float kv[kMaxPerLane], vv[kMaxPerLane], adk[kMaxPerLane], adv[kMaxPerLane];
    for (int i = 0; i < per; ++i) {
      int d = lane + 64 * i;
      kv[i] = d < D ? to_f(k[((int64_t)key * H + h) * D + d]) : 0.f;
      vv[i] = d < D ? to_f(v[((int64_t)key * H + h) * D + d]) : 0.f;
      adk[i] = adv[i] = 0.f;
    }
    for (int row = q0; row < q1; ++row) {
      const T *qr = q + ((int64_t)row * H + h) * D;
      const T *dor = dout + ((int64_t)row * H + h) * D;
      float s = 0.f, dp = 0.f;
      for (int i = 0; i < per; ++i) {
        int d = lane + 64 * i;
        if (d < D) {
          s += kv[i] * to_f(qr[d]);
          dp += vv[i] * to_f(dor[d]);
        }
      }
      s = wave_sum(s);
      dp = wave_sum(dp);
      const float p = fast_exp2(s * c - lse[(int64_t)row * H + h]);
      const float ds = round_to<T>(p * (dp - delta[(int64_t)row * H + h]));
      const float pr = round_to<T>(p);
      for (int i = 0; i < per; ++i) {
        int d = lane + 64 * i;
        if (d < D) {
          adv[i] += pr * to_f(dor[d]);
          adk[i] += ds * to_f(qr[d]);
        }
      }
    }
    for (int i = 0; i < per; ++i) {
      int d = lane + 64 * i;
      if (d >= D) continue;
      dk[((int64_t)key * H + h) * D + d] = from_f<T>(adk[i] * scale);
      dv[((int64_t)key * H + h) * D + d] = from_f<T>(adv[i]);
    }
  }
}

// ---------------------------------------------------------------------------
// Absorb forward.  Item {t0,t1,k0,k1,pbase,...}; grid = n_items; one wave per
// (token, head) row; lanes split D_KV.  Output rows are projected with W_V
// after rounding aX/l to T (ta/kernels.py:276-277).
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void simt_absorb_fwd(
    const T *__restrict__ u, const T *__restrict__ X, const T *__restrict__ wv,
    T *__restrict__ O, float *__restrict__ lse, float *__restrict__ part_o,
    float *__restrict__ part_lse, const int32_t *__restrict__ items, int H, int F, int DH,
    float c) {
  const PlanItem it = load_item(items, blockIdx.x);
  const int t0 = it.v[0], t1 = it.v[1], k0 = it.v[2], k1 = it.v[3], pbase = it.v[4];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int per = (F + 63) / 64;
  const int nrows = (t1 - t0) * H;
  for (int r = wave; r < nrows; r += 4) {
    const int t = t0 + r / H, h = r % H;
    float uv[kMaxPerLane], ax[kMaxPerLane];
    for (int i = 0; i < per; ++i) {
      int f = lane + 64 * i;
      uv[i] = f < F ? to_f(u[((int64_t)t * H + h) * F + f]) : 0.f;
      ax[i] = 0.f;
    }
    float m = kNegInf, l = 0.f;
    for (int j = k0; j < k1; ++j) {
      const T *xr = X + (int64_t)j * F;
      float s = 0.f;
      for (int i = 0; i < per; ++i) {
        int f = lane + 64 * i;
        if (f < F) s += uv[i] * to_f(xr[f]);
      }
      const float tt = wave_sum(s) * c;
      const float mn = fmaxf(m, tt);
      const float alpha = fast_exp2(m - mn), p = fast_exp2(tt - mn);
      l = l * alpha + p;
      const float pr = round_to<T>(p);
      for (int i = 0; i < per; ++i) {
        int f = lane + 64 * i;
        ax[i] = ax[i] * alpha + (f < F ? pr * to_f(xr[f]) : 0.f);
      }
      m = mn;
    }
    const float inv = l > 0.f ? 1.f / l : 0.f;
    const float lse_v = l > 0.f ? m + fast_log2(l) : kNegInf;
    for (int i = 0; i < per; ++i) ax[i] = round_to<T>(ax[i] * inv);
    for (int d = 0; d < DH; ++d) {
      float s = 0.f;
      for (int i = 0; i < per; ++i) {
        int f = lane + 64 * i;
        if (f < F) s += ax[i] * to_f(wv[((int64_t)f * H + h) * DH + d]);
      }
      s = wave_sum(s);
      if (lane == 0) {
        if (pbase < 0)
          O[((int64_t)t * H + h) * DH + d] = from_f<T>(s);
        else
          part_o[((int64_t)(pbase + t - t0) * H + h) * DH + d] = s;
      }
    }
    if (lane == 0) {
      if (pbase < 0)
        lse[(int64_t)t * H + h] = lse_v;
      else
        part_lse[(int64_t)(pbase + t - t0) * H + h] = lse_v;
    }
  }
}

// ---------------------------------------------------------------------------
// Absorb backward, query side: per (token, head) wave, with dAX = dO W_V^T
//   already in the workspace: du = scale * sum_j dS X_j and aX = sum_j P X_j
//   (the fp32 aX is kept for dW_V).
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void simt_absorb_du(
    const T *__restrict__ u, const T *__restrict__ X, const float *__restrict__ lse,
    const float *__restrict__ delta, T *__restrict__ du, const T *__restrict__ dax_ws,
    float *__restrict__ ax_ws, const int32_t *__restrict__ cu_items, int H, int F, float c,
    float scale) {
  // cu_items: one item per token tile, {t0, t1, k0, k1}: the segment's keys.
  const PlanItem it = load_item(cu_items, blockIdx.x);
  const int t0 = it.v[0], t1 = it.v[1], k0 = it.v[2], k1 = it.v[3];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int per = (F + 63) / 64;
  const int nrows = (t1 - t0) * H;
  for (int r = wave; r < nrows; r += 4) {
    const int t = t0 + r / H, h = r % H;
    const int64_t row = (int64_t)t * H + h;
    float uv[kMaxPerLane], dax[kMaxPerLane], adu[kMaxPerLane], aax[kMaxPerLane];
    for (int i = 0; i < per; ++i) {
      int f = lane + 64 * i;
      uv[i] = f < F ? to_f(u[row * F + f]) : 0.f;
      dax[i] = f < F ? to_f(dax_ws[row * F + f]) : 0.f;
      adu[i] = aax[i] = 0.f;
    }
    const float L = lse[row], dl = delta[row];
    for (int j = k0; j < k1; ++j) {
      const T *xr = X + (int64_t)j * F;
      float s = 0.f, dp = 0.f;
      for (int i = 0; i < per; ++i) {
        int f = lane + 64 * i;
        if (f < F) {
          float x = to_f(xr[f]);
          s += uv[i] * x;
          dp += dax[i] * x;
        }
      }
      s = wave_sum(s);
      dp = wave_sum(dp);
      const float p = fast_exp2(s * c - L);
      const float ds = p * (dp - dl);
      for (int i = 0; i < per; ++i) {
        int f = lane + 64 * i;
        if (f < F) {
          float x = to_f(xr[f]);
          adu[i] += ds * x;
          aax[i] += p * x;
        }
      }
    }
    for (int i = 0; i < per; ++i) {
      int f = lane + 64 * i;
      if (f >= F) continue;
      du[row * F + f] = from_f<T>(adu[i] * scale);
      ax_ws[row * F + f] = aax[i];
    }
  }
}

// Absorb dX: item {k0,k1,t0,t1,...}; one wave per key, loops over the
// segment's (token, head) rows.
template <typename T>
__global__ __launch_bounds__(256) void simt_absorb_dx(
    const T *__restrict__ u, const T *__restrict__ X, const float *__restrict__ lse,
    const float *__restrict__ delta, const T *__restrict__ dax_ws, T *__restrict__ dX,
    const int32_t *__restrict__ items, int H, int F, float c, float scale) {
  const PlanItem it = load_item(items, blockIdx.x);
  const int k0 = it.v[0], k1 = it.v[1], t0 = it.v[2], t1 = it.v[3];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int per = (F + 63) / 64;
  for (int j = k0 + wave; j < k1; j += 4) {
    float xv[kMaxPerLane], acc[kMaxPerLane];
    for (int i = 0; i < per; ++i) {
      int f = lane + 64 * i;
      xv[i] = f < F ? to_f(X[(int64_t)j * F + f]) : 0.f;
      acc[i] = 0.f;
    }
    for (int64_t row = (int64_t)t0 * H; row < (int64_t)t1 * H; ++row) {
      float s = 0.f, dp = 0.f;
      for (int i = 0; i < per; ++i) {
        int f = lane + 64 * i;
        if (f < F) {
          s += xv[i] * to_f(u[row * F + f]);
          dp += xv[i] * to_f(dax_ws[row * F + f]);
        }
      }
      s = wave_sum(s);
      dp = wave_sum(dp);
      const float p = fast_exp2(s * c - lse[row]);
      const float ds = p * (dp - delta[row]) * scale;
      for (int i = 0; i < per; ++i) {
        int f = lane + 64 * i;
        if (f < F) acc[i] += ds * to_f(u[row * F + f]) + p * to_f(dax_ws[row * F + f]);
      }
    }
    for (int i = 0; i < per; ++i) {
      int f = lane + 64 * i;
      if (f < F) dX[(int64_t)j * F + f] = from_f<T>(acc[i]);
    }
  }
}

}  // namespace

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
template <typename T>
void launch_simt_varlen_fwd(const VarlenArgs &a, hipStream_t st) {
  if (a.n_items == 0) return;
  hipLaunchKernelGGL(simt_varlen_fwd<T>, dim3(a.n_items * a.H), dim3(256), 0, st,
                     (const T *)a.q, (const T *)a.k, (const T *)a.v, (T *)a.o, a.lse, a.part_o,
                     a.part_lse, a.items, a.H, a.D, a.scale * kLog2e);
}

template <typename T>
void launch_simt_varlen_dq(const VarlenArgs &a, hipStream_t st) {
  if (a.n_items == 0) return;
  hipLaunchKernelGGL(simt_varlen_dq<T>, dim3(a.n_items * a.H), dim3(256), 0, st,
                     (const T *)a.q, (const T *)a.k, (const T *)a.v, (const T *)a.dout,
                     a.lse_in, a.delta, (T *)a.dq, a.part_o, a.items, a.H, a.D,
                     a.scale * kLog2e, a.scale);
}

template <typename T>
void launch_simt_varlen_dkv(const VarlenArgs &a, hipStream_t st) {
  if (a.n_kv == 0) return;
  hipLaunchKernelGGL(simt_varlen_dkv<T>, dim3(a.n_kv * a.H), dim3(256), 0, st,
                     (const T *)a.q, (const T *)a.k, (const T *)a.v, (const T *)a.dout,
                     a.lse_in, a.delta, (T *)a.dk, (T *)a.dv, a.kv_items, a.H, a.D,
                     a.scale * kLog2e, a.scale);
}

template <typename T>
void launch_simt_absorb_fwd(const AbsorbArgs &a, hipStream_t st) {
  if (a.n_items == 0) return;
  hipLaunchKernelGGL(simt_absorb_fwd<T>, dim3(a.n_items), dim3(256), 0, st, (const T *)a.u,
                     (const T *)a.X, (const T *)a.wv, (T *)a.O, a.lse, a.part_o, a.part_lse,
                     a.items, a.H, a.F, a.DH, a.scale * kLog2e);
}

template <typename T>
void launch_simt_absorb_du(const AbsorbArgs &a, hipStream_t st) {
  if (a.n_qseg == 0) return;
  hipLaunchKernelGGL(simt_absorb_du<T>, dim3(a.n_qseg), dim3(256), 0, st, (const T *)a.u,
                     (const T *)a.X, a.lse_in, a.delta, (T *)a.du, (const T *)a.dax, a.ax,
                     a.qseg_items, a.H, a.F, a.scale * kLog2e, a.scale);
}

template <typename T>
void launch_simt_absorb_dx(const AbsorbArgs &a, hipStream_t st) {
  if (a.n_kv == 0) return;
  hipLaunchKernelGGL(simt_absorb_dx<T>, dim3(a.n_kv), dim3(256), 0, st, (const T *)a.u,
                     (const T *)a.X, a.lse_in, a.delta, (const T *)a.dax, (T *)a.dX, a.kv_items, a.H, a.F,
                     a.scale * kLog2e, a.scale);
}

#define VAFA_INST(T)                                                          \
  template void launch_simt_varlen_fwd<T>(const VarlenArgs &, hipStream_t);  \
  template void launch_simt_varlen_dq<T>(const VarlenArgs &, hipStream_t);   \
  template void launch_simt_varlen_dkv<T>(const VarlenArgs &, hipStream_t);  \
  template void launch_simt_absorb_fwd<T>(const AbsorbArgs &, hipStream_t);  \
  template void launch_simt_absorb_du<T>(const AbsorbArgs &, hipStream_t);   \
  template void launch_simt_absorb_dx<T>(const AbsorbArgs &, hipStream_t);
VAFA_INST(float)
VAFA_INST(f16)
VAFA_INST(bf16)
#undef VAFA_INST

}  // namespace vafa
