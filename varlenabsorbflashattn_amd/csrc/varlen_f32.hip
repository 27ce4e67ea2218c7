// Packed varlen FlashAttention in fp32 on gfx950 fp32 matrix cores
// (v_mfma_f32_32x32x2_f32, IEEE fp32 products; replaces fa/kernels.py:64-175
// and 516-628 for fp32 inputs, fa/interface.py:163).
//
// Forward: one workgroup = NW waves (the plan's query tile / 32) of one head,
// each wave owning 32 query rows; 32-key K/V tiles staged in LDS through
// registers (the next tile's loads in flight under the current tile's
// products, double-buffered LDS).  Per tile a wave forms
//   S^T = K Q^T        (D/2 products, K rows as A, Q^T held in registers)
//   O^T += V^T P^T     (D/2 products, V^T as A, P^T straight from S^T)
// The reduction index of every product is relabelled so that each lane's
// operands are 16-byte LDS reads:
//   * S^T step s: lane half lh supplies d = lh*D/2 + s (A: K[key][d], B:
//     Q[row][d]), four consecutive steps from one ds_read_b128 of a K row;
//   * O^T step s: lane half lh supplies key 8*(s/4) + 4*lh + s%4 -- exactly
//     the keys the S^T accumulator holds in its element s for that lane, so
//     P^T needs no exchange, and V is staged transposed ([d][key]) so the
//     four keys of s = 4j..4j+3 are one ds_read_b128.
// The online softmax runs in the log2 domain (LSE = m + log2 l), as the
// 16-bit kernels; split items write normalized fp32 partial rows.
#include "common.h"
#include "kernels.h"

namespace vafa {

namespace {

constexpr int kF32BK = 32;  // keys per tile

__device__ __forceinline__ f32x16 mma32f(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

template <int D>
struct F32FwdSmem {
  static constexpr int KS = D + 4;            // K row stride (floats): 16 rows hit 16 bank groups
  static constexpr int VS = kF32BK + 4;       // V^T row stride (floats)
  static constexpr int kK = kF32BK * KS;      // floats per K tile
  static constexpr int kV = D * VS;           // floats per V^T tile
  static constexpr int kBuf = kK + kV;
  static constexpr int kBytes = 2 * kBuf * 4;  // double buffered
};

// Register stage of one 32-key K/V tile over NT threads: 16-byte chunks,
// zeros past k_end.
template <int D, int NT>
struct F32Tile {
  static constexpr int kChunks = kF32BK * D / 4;              // per tensor
  static constexpr int kPer = (kChunks + NT - 1) / NT;        // per thread
  f32x4 kc[kPer], vc[kPer];
};

template <int D, int NT>
__device__ __forceinline__ void f32_load_tile(F32Tile<D, NT> &r, const float *k, const float *v,
                                              int kbase, int k_end, int H, int h, int tid) {
  using R = F32Tile<D, NT>;
  constexpr int CPR = D / 4;
  const int nk = k_end - kbase < kF32BK ? k_end - kbase : kF32BK;
  const int64_t nbytes = (int64_t)nk * H * D * 4;
  const rsrc_t rk = make_rsrc(k + (int64_t)kbase * H * D, nbytes);
  const rsrc_t rv = make_rsrc(v + (int64_t)kbase * H * D, nbytes);
#pragma unroll
  for (int i = 0; i < R::kPer; ++i) {
    const int ci = tid + NT * i;
    const int key = ci < R::kChunks ? ci / CPR : kF32BK, dc = ci % CPR;  // kF32BK: zeros
    const int off = (key * H + h) * D * 4 + dc * 16;
    r.kc[i] = __builtin_bit_cast(f32x4, buf_load16(rk, off));
    r.vc[i] = __builtin_bit_cast(f32x4, buf_load16(rv, off));
  }
}

template <int D, int NT>
__device__ __forceinline__ void f32_store_tile(const F32Tile<D, NT> &r, float *ks, float *vts,
                                               int tid) {
  using R = F32Tile<D, NT>;
  using S = F32FwdSmem<D>;
  constexpr int CPR = D / 4;
#pragma unroll
  for (int i = 0; i < R::kPer; ++i) {
    const int ci = tid + NT * i;
    if (R::kChunks % NT == 0 || ci < R::kChunks) {
      const int key = ci / CPR, d0 = (ci % CPR) * 4;
      *reinterpret_cast<f32x4 *>(ks + key * S::KS + d0) = r.kc[i];
#pragma unroll
      for (int e = 0; e < 4; ++e) vts[(d0 + e) * S::VS + key] = r.vc[i][e];
    }
  }
}

// two waves per SIMD (one at D = 256, whose Q^T operands and accumulators
// take 256 registers)
template <int D, int NW>
__global__ __launch_bounds__(64 * NW, NW == 8 || D >= 256 ? 1 : 2) void varlen_fwd_f32_kernel(
    const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v,
    float *__restrict__ o, float *__restrict__ lse, float *__restrict__ part_o,
    float *__restrict__ part_lse, const int32_t *__restrict__ items, int H, float c) {
  using S = F32FwdSmem<D>;
  constexpr int NT = 64 * NW;
  constexpr int ND = D / 32;  // 32-row d tiles of O^T
  extern __shared__ __align__(16) unsigned char smem_raw[];
  float *smem = reinterpret_cast<float *>(smem_raw);

  const int item = blockIdx.x / H, h = blockIdx.x % H;
  const PlanItem it = load_item(items, item);
  const int q0 = it.v[0], q1 = it.v[1], k0 = it.v[2], k1 = it.v[3], pbase = it.v[4];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int l32 = lane & 31, lh = lane >> 5;
  const int qrow = q0 + wave * 32 + l32;
  const bool row_ok = qrow < q1;
  const bool wave_active = q0 + wave * 32 < q1;

  // Q^T operand: this lane's row at d = lh*D/2 + s, rows past q1 zero.  A
  // negative scale is folded into Q (exact sign flips), so c > 0 below.
  const float qsgn = c < 0.f ? -1.f : 1.f;
  c = fabsf(c);
  float qf[D / 2];
  {
    const rsrc_t rq = make_rsrc(q + ((int64_t)q0 * H + h) * D, (int64_t)(q1 - q0) * H * D * 4);
    const int lr = wave * 32 + l32;
#pragma unroll
    for (int t = 0; t < D / 8; ++t) {
      const f32x4 x = __builtin_bit_cast(f32x4, buf_load16(rq, (lr * H * D + lh * (D / 2) + 4 * t) * 4));
#pragma unroll
      for (int e = 0; e < 4; ++e) qf[4 * t + e] = x[e] * qsgn;
    }
  }
  f32x16 acc[ND];
#pragma unroll
  for (int i = 0; i < ND; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[i][r] = 0.f;
  float m_run = kNegInf, l_part = 0.f;

  const int nt = (k1 - k0 + kF32BK - 1) / kF32BK;
  F32Tile<D, NT> regs;
  if (nt > 0) {
    f32_load_tile<D, NT>(regs, k, v, k0, k1, H, h, tid);
    f32_store_tile<D, NT>(regs, smem, smem + S::kK, tid);
  }
  __syncthreads();
  for (int j = 0; j < nt; ++j) {
    const int kbase = k0 + j * kF32BK;
    if (j + 1 < nt) f32_load_tile<D, NT>(regs, k, v, kbase + kF32BK, k1, H, h, tid);
    const float *ks = smem + (j & 1) * S::kBuf;
    const float *vts = ks + S::kK;
    if (wave_active) {
      // S^T = K Q^T
      f32x16 s;
#pragma unroll
      for (int r = 0; r < 16; ++r) s[r] = 0.f;
      const float *krow = ks + l32 * S::KS + lh * (D / 2);
#pragma unroll
      for (int t = 0; t < D / 8; ++t) {
        const f32x4 a = *reinterpret_cast<const f32x4 *>(krow + 4 * t);
#pragma unroll
        for (int e = 0; e < 4; ++e) s = mma32f(a[e], qf[4 * t + e], s);
      }
      // element r: key kbase + 8*(r/4) + 4*lh + r%4 of this lane's row
      if (kbase + kF32BK > k1) {
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (kbase + 8 * (r >> 2) + 4 * lh + (r & 3) >= k1) s[r] = kNegInf;
      }
      float mx = s[0];
#pragma unroll
      for (int r = 1; r < 16; ++r) mx = fmaxf(mx, s[r]);
      mx = max_xor32(mx) * c;
      const float m_new = fmaxf(m_run, mx);
      // a fully masked tile cannot occur (nt covers [k0, k1)), so m_new is finite
      const float alpha = fast_exp2(m_run - m_new);
      m_run = m_new;
      l_part *= alpha;
#pragma unroll
      for (int i = 0; i < ND; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][r] *= alpha;
      float p[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        p[r] = fast_exp2(__builtin_fmaf(s[r], c, -m_new));
        l_part += p[r];
      }
      // O^T += V^T P^T: step s uses keys 8*(s/4) + 4*lh + s%4 (p[s] of this lane)
#pragma unroll
      for (int dt = 0; dt < ND; ++dt) {
        const float *vrow = vts + (dt * 32 + l32) * S::VS + 4 * lh;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const f32x4 a = *reinterpret_cast<const f32x4 *>(vrow + 8 * jj);
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[dt] = mma32f(a[e], p[4 * jj + e], acc[dt]);
        }
      }
    }
    // the other buffer held tile j-1, which every wave finished before the
    // barrier that ended the previous trip
    if (j + 1 < nt) {
      float *nks = smem + ((j + 1) & 1) * S::kBuf;
      f32_store_tile<D, NT>(regs, nks, nks + S::kK, tid);
    }
    __syncthreads();
  }

  if (!row_ok) return;
  const float l = l_part + __shfl_xor(l_part, 32, 64);
  const float inv = l > 0.f ? 1.f / l : 0.f;
  const float lse_v = l > 0.f ? m_run + fast_log2(l) : kNegInf;
  // element r of tile dt: d = 32*dt + 8*(r/4) + 4*lh + r%4
  float *orow = pbase < 0 ? o + ((int64_t)qrow * H + h) * D
                          : part_o + ((int64_t)(pbase + (qrow - q0)) * H + h) * D;
#pragma unroll
  for (int dt = 0; dt < ND; ++dt)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      f32x4 w;
#pragma unroll
      for (int e = 0; e < 4; ++e) w[e] = acc[dt][g * 4 + e] * inv;
      *reinterpret_cast<f32x4 *>(orow + dt * 32 + g * 8 + lh * 4) = w;
    }
  if (lh == 0) {
    if (pbase < 0)
      lse[(int64_t)qrow * H + h] = lse_v;
    else
      part_lse[(int64_t)(pbase + (qrow - q0)) * H + h] = lse_v;
  }
}

template <int D, int NW>
void launch_fwd_f32_nw(const VarlenArgs &a, hipStream_t st) {
  const int smem = F32FwdSmem<D>::kBytes;
  allow_dynamic_lds(reinterpret_cast<const void *>(&varlen_fwd_f32_kernel<D, NW>), smem);
  hipLaunchKernelGGL((varlen_fwd_f32_kernel<D, NW>), dim3((unsigned)(a.n_items * a.H)),
                     dim3(64 * NW), smem, st, (const float *)a.q, (const float *)a.k,
                     (const float *)a.v, (float *)a.o, a.lse, a.part_o, a.part_lse, a.items, a.H,
                     a.scale * kLog2e);
}

// the planner gives 256-row query tiles only to D <= 128
template <int D>
void launch_fwd_f32_d(const VarlenArgs &a, hipStream_t st) {
  if constexpr (D <= 128) {
    if (a.q_tile == kVarlenWideTile) return launch_fwd_f32_nw<D, 8>(a, st);
  }
  launch_fwd_f32_nw<D, 4>(a, st);
}

// ---------------------------------------------------------------------------
// Backward at D in {32, 64} (D = 128 and 256 below, on 16x16x4 products:
// here the operands held in registers and the accumulators would take more
// than half the register file at D = 128 and more than all of it at 256).
//
// dQ, query-major over the forward's items (split items write scaled fp32
// partial rows that the ordered sum adds): per 32-key tile
//   S^T = K Q^T, dP^T = V dO^T      (K, V rows as A from LDS, Q^T, dO^T in
//                                    registers, d relabelled as above)
//   P^T = exp2(S^T c - LSE), dS^T = P^T (dP^T - delta)   (lane = query row)
//   dQ^T += K^T dS^T                 (K^T staged transposed; step s takes the
//                                    keys of S^T's element s, as the forward's PV)
// An item's rows are walked 32*NW at a time (one pass for the items the plan
// gives these head dims).
// ---------------------------------------------------------------------------
template <int D>
struct F32DqSmem {
  static constexpr int KS = D + 4;
  static constexpr int TS = kF32BK + 4;
  static constexpr int kK = kF32BK * KS;       // K rows, then V rows
  static constexpr int kKT = D * TS;           // K^T
  static constexpr int kBuf = 2 * kK + kKT;
  static constexpr int kBytes = 2 * kBuf * 4;
};

template <int D, int NT>
__device__ __forceinline__ void f32_store_dq_tile(const F32Tile<D, NT> &r, float *ks, int tid) {
  using R = F32Tile<D, NT>;
  using S = F32DqSmem<D>;
  constexpr int CPR = D / 4;
  float *vs = ks + S::kK, *kts = ks + 2 * S::kK;
#pragma unroll
  for (int i = 0; i < R::kPer; ++i) {
    const int ci = tid + NT * i;
    if (R::kChunks % NT == 0 || ci < R::kChunks) {
      const int key = ci / CPR, d0 = (ci % CPR) * 4;
      *reinterpret_cast<f32x4 *>(ks + key * S::KS + d0) = r.kc[i];
      *reinterpret_cast<f32x4 *>(vs + key * S::KS + d0) = r.vc[i];
#pragma unroll
      for (int e = 0; e < 4; ++e) kts[(d0 + e) * S::TS + key] = r.kc[i][e];
    }
  }
}

template <int D, int NW>
__global__ __launch_bounds__(64 * NW, NW == 8 || D >= 128 ? 1 : 2) void varlen_dq_f32_kernel(
    const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v,
    const float *__restrict__ dout, const float *__restrict__ lse,
    const float *__restrict__ delta, float *__restrict__ dq, float *__restrict__ part_dq,
    const int32_t *__restrict__ items, int H, float c, float scale) {
  using S = F32DqSmem<D>;
  constexpr int NT = 64 * NW;
  constexpr int ND = D / 32;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  float *smem = reinterpret_cast<float *>(smem_raw);

  const int item = blockIdx.x / H, h = blockIdx.x % H;
  const PlanItem it = load_item(items, item);
  const int iq0 = it.v[0], q1 = it.v[1], k0 = it.v[2], k1 = it.v[3], pbase = it.v[4];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int l32 = lane & 31, lh = lane >> 5;
  for (int q0 = iq0; q0 < q1; q0 += 32 * NW) {
    const int qrow = q0 + wave * 32 + l32;
    const bool row_ok = qrow < q1;
    const bool wave_active = q0 + wave * 32 < q1;
    // Q^T and dO^T operands of this lane's row (zero past q1)
    float qf[D / 2], gf[D / 2];
    {
      const int64_t nb = (int64_t)(q1 - q0) * H * D * 4;
      const rsrc_t rq = make_rsrc(q + ((int64_t)q0 * H + h) * D, nb);
      const rsrc_t rg = make_rsrc(dout + ((int64_t)q0 * H + h) * D, nb);
      const int lr = wave * 32 + l32;
#pragma unroll
      for (int t = 0; t < D / 8; ++t) {
        const int off = (lr * H * D + lh * (D / 2) + 4 * t) * 4;
        const f32x4 x = __builtin_bit_cast(f32x4, buf_load16(rq, off));
        const f32x4 y = __builtin_bit_cast(f32x4, buf_load16(rg, off));
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          qf[4 * t + e] = x[e];
          gf[4 * t + e] = y[e];
        }
      }
    }
    const float L = row_ok ? lse[(int64_t)qrow * H + h] : 0.f;
    const float dl = row_ok ? delta[(int64_t)qrow * H + h] : 0.f;
    f32x16 acc[ND];
#pragma unroll
    for (int i = 0; i < ND; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][r] = 0.f;

    const int nt = (k1 - k0 + kF32BK - 1) / kF32BK;
    F32Tile<D, NT> regs;
    if (nt > 0) {
      f32_load_tile<D, NT>(regs, k, v, k0, k1, H, h, tid);
      f32_store_dq_tile<D, NT>(regs, smem, tid);
    }
    __syncthreads();
    for (int j = 0; j < nt; ++j) {
      const int kbase = k0 + j * kF32BK;
      if (j + 1 < nt) f32_load_tile<D, NT>(regs, k, v, kbase + kF32BK, k1, H, h, tid);
      const float *ks = smem + (j & 1) * S::kBuf;
      const float *vs = ks + S::kK, *kts = ks + 2 * S::kK;
      if (wave_active) {
        f32x16 s, dp;
#pragma unroll
        for (int r = 0; r < 16; ++r) s[r] = dp[r] = 0.f;
        const float *krow = ks + l32 * S::KS + lh * (D / 2);
        const float *vrow = vs + l32 * S::KS + lh * (D / 2);
#pragma unroll
        for (int t = 0; t < D / 8; ++t) {
          const f32x4 a = *reinterpret_cast<const f32x4 *>(krow + 4 * t);
          const f32x4 b = *reinterpret_cast<const f32x4 *>(vrow + 4 * t);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            s = mma32f(a[e], qf[4 * t + e], s);
            dp = mma32f(b[e], gf[4 * t + e], dp);
          }
        }
        // element r: key kbase + 8*(r/4) + 4*lh + r%4; P = 0 past k1
        float ds[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const bool kin = kbase + 8 * (r >> 2) + 4 * lh + (r & 3) < k1;
          const float p = kin ? fast_exp2(__builtin_fmaf(s[r], c, -L)) : 0.f;
          ds[r] = p * (dp[r] - dl);
        }
#pragma unroll
        for (int dt = 0; dt < ND; ++dt) {
          const float *trow = kts + (dt * 32 + l32) * S::TS + 4 * lh;
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            const f32x4 a = *reinterpret_cast<const f32x4 *>(trow + 8 * jj);
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[dt] = mma32f(a[e], ds[4 * jj + e], acc[dt]);
          }
        }
      }
      if (j + 1 < nt) {
        float *nks = smem + ((j + 1) & 1) * S::kBuf;
        f32_store_dq_tile<D, NT>(regs, nks, tid);
      }
      __syncthreads();
    }
    if (row_ok) {
      // element r of tile dt: d = 32*dt + 8*(r/4) + 4*lh + r%4
      float *orow = pbase < 0 ? dq + ((int64_t)qrow * H + h) * D
                              : part_dq + ((int64_t)(pbase + (qrow - iq0)) * H + h) * D;
#pragma unroll
      for (int dt = 0; dt < ND; ++dt)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          f32x4 w;
#pragma unroll
          for (int e = 0; e < 4; ++e) w[e] = acc[dt][g * 4 + e] * scale;
          *reinterpret_cast<f32x4 *>(orow + dt * 32 + g * 8 + lh * 4) = w;
        }
    }
    // the next sub-tile's first LDS store follows the last barrier above,
    // after which no wave reads LDS
  }
}

// dK/dV, key-major over the plan's key tiles (32 keys per wave): per 32-row
// query block (Q, dO staged row-major and transposed, LSE and delta)
//   S = Q K^T, dP = dO V^T           (Q, dO rows as A, K^T, V^T in registers:
//                                    lane = key, d relabelled)
//   P = exp2(S c - LSE), dS = P (dP - delta)   (element r: query row
//                                    8*(r/4) + 4*lh + r%4 of the block)
//   dV^T += dO^T P, dK^T += Q^T dS   (A from the transposed copies, B = P / dS
//                                    element s: no exchange)
template <int D>
struct F32DkvSmem {
  static constexpr int RS = D + 4;            // row-major Q / dO stride
  static constexpr int TS = kF32BK + 4;       // transposed stride
  static constexpr int kR = kF32BK * RS;
  static constexpr int kT = D * TS;
  static constexpr int kBuf = 2 * kR + 2 * kT + 2 * kF32BK;  // Q, dO, Q^T, dO^T, LSE, delta
  static constexpr int kBytes = 2 * kBuf * 4;
};

template <int D, int NT>
struct F32QBlk {
  static constexpr int kChunks = kF32BK * D / 4;
  static constexpr int kPer = (kChunks + NT - 1) / NT;
  f32x4 qc[kPer], gc[kPer];
  float lv, dv;
};

template <int D, int NT>
__device__ __forceinline__ void f32_load_qblk(F32QBlk<D, NT> &r, const float *q,
                                              const float *dout, const float *lse,
                                              const float *delta, int qb, int q_end, int H,
                                              int h, int tid) {
  using R = F32QBlk<D, NT>;
  constexpr int CPR = D / 4;
  const int nq = q_end - qb < kF32BK ? q_end - qb : kF32BK;
  const int64_t nbytes = (int64_t)nq * H * D * 4;
  const rsrc_t rq = make_rsrc(q + (int64_t)qb * H * D, nbytes);
  const rsrc_t rg = make_rsrc(dout + (int64_t)qb * H * D, nbytes);
#pragma unroll
  for (int i = 0; i < R::kPer; ++i) {
    const int ci = tid + NT * i;
    const int row = ci < R::kChunks ? ci / CPR : kF32BK, dc = ci % CPR;
    const int off = (row * H + h) * D * 4 + dc * 16;
    r.qc[i] = __builtin_bit_cast(f32x4, buf_load16(rq, off));
    r.gc[i] = __builtin_bit_cast(f32x4, buf_load16(rg, off));
  }
  // rows past q_end: LSE = +inf makes P = 0 (their Q and dO are zero too)
  const bool ok = tid < kF32BK && tid < nq;
  r.lv = ok ? lse[(int64_t)(qb + tid) * H + h] : __builtin_inff();
  r.dv = ok ? delta[(int64_t)(qb + tid) * H + h] : 0.f;
}

template <int D, int NT>
__device__ __forceinline__ void f32_store_qblk(const F32QBlk<D, NT> &r, float *base, int tid) {
  using R = F32QBlk<D, NT>;
  using S = F32DkvSmem<D>;
  constexpr int CPR = D / 4;
  float *qs = base, *gs = base + S::kR, *qt = base + 2 * S::kR, *gt = qt + S::kT;
  float *ls = gt + S::kT;
#pragma unroll
  for (int i = 0; i < R::kPer; ++i) {
    const int ci = tid + NT * i;
    if (R::kChunks % NT == 0 || ci < R::kChunks) {
      const int row = ci / CPR, d0 = (ci % CPR) * 4;
      *reinterpret_cast<f32x4 *>(qs + row * S::RS + d0) = r.qc[i];
      *reinterpret_cast<f32x4 *>(gs + row * S::RS + d0) = r.gc[i];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        qt[(d0 + e) * S::TS + row] = r.qc[i][e];
        gt[(d0 + e) * S::TS + row] = r.gc[i][e];
      }
    }
  }
  if (tid < kF32BK) {
    ls[tid] = r.lv;
    ls[kF32BK + tid] = r.dv;
  }
}

template <int D, int NW>
__global__ __launch_bounds__(64 * NW, NW == 8 || D >= 128 ? 1 : 2) void varlen_dkv_f32_kernel(
    const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v,
    const float *__restrict__ dout, const float *__restrict__ lse,
    const float *__restrict__ delta, float *__restrict__ dk, float *__restrict__ dv,
    const int32_t *__restrict__ items, int H, float c, float scale) {
  using S = F32DkvSmem<D>;
  constexpr int NT = 64 * NW;
  constexpr int ND = D / 32;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  float *smem = reinterpret_cast<float *>(smem_raw);

  const int item = blockIdx.x / H, h = blockIdx.x % H;
  const PlanItem it = load_item(items, item);
  const int kt0 = it.v[0], kt1 = it.v[1], q0 = it.v[2], q1 = it.v[3];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int l32 = lane & 31, lh = lane >> 5;
  const int nb = (q1 - q0 + kF32BK - 1) / kF32BK;
  // an item holds one key tile of NW*32 keys, or (fused-planned chunks) a
  // few: each sub-tile walks the query blocks on its own
  for (int k0 = kt0; k0 < kt1; k0 += 32 * NW) {
    const int k1 = kt1 - k0 < 32 * NW ? kt1 : k0 + 32 * NW;
    const int key = k0 + wave * 32 + l32;
    const bool key_ok = key < k1;
    const bool wave_active = k0 + wave * 32 < k1;

    // K^T and V^T operands of this lane's key (zero past k1)
    float kf[D / 2], vf[D / 2];
    {
      const int64_t nbk = (int64_t)(k1 - k0) * H * D * 4;
      const rsrc_t rk = make_rsrc(k + ((int64_t)k0 * H + h) * D, nbk);
      const rsrc_t rv = make_rsrc(v + ((int64_t)k0 * H + h) * D, nbk);
      const int lr = wave * 32 + l32;
#pragma unroll
      for (int t = 0; t < D / 8; ++t) {
        const int off = (lr * H * D + lh * (D / 2) + 4 * t) * 4;
        const f32x4 x = __builtin_bit_cast(f32x4, buf_load16(rk, off));
        const f32x4 y = __builtin_bit_cast(f32x4, buf_load16(rv, off));
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          kf[4 * t + e] = x[e];
          vf[4 * t + e] = y[e];
        }
      }
    }
    f32x16 adk[ND], adv[ND];
#pragma unroll
    for (int i = 0; i < ND; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) adk[i][r] = adv[i][r] = 0.f;

    F32QBlk<D, NT> regs;
    if (nb > 0) {
      f32_load_qblk<D, NT>(regs, q, dout, lse, delta, q0, q1, H, h, tid);
      f32_store_qblk<D, NT>(regs, smem, tid);
    }
    __syncthreads();
    for (int j = 0; j < nb; ++j) {
      const int qbase = q0 + j * kF32BK;
      if (j + 1 < nb)
        f32_load_qblk<D, NT>(regs, q, dout, lse, delta, qbase + kF32BK, q1, H, h, tid);
      const float *base = smem + (j & 1) * S::kBuf;
      const float *qs = base, *gs = base + S::kR, *qt = base + 2 * S::kR, *gt = qt + S::kT;
      const float *ls = gt + S::kT;
      if (wave_active) {
        f32x16 s, dp;
#pragma unroll
        for (int r = 0; r < 16; ++r) s[r] = dp[r] = 0.f;
        const float *qrow = qs + l32 * S::RS + lh * (D / 2);
        const float *grow = gs + l32 * S::RS + lh * (D / 2);
#pragma unroll
        for (int t = 0; t < D / 8; ++t) {
          const f32x4 a = *reinterpret_cast<const f32x4 *>(qrow + 4 * t);
          const f32x4 b = *reinterpret_cast<const f32x4 *>(grow + 4 * t);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            s = mma32f(a[e], kf[4 * t + e], s);
            dp = mma32f(b[e], vf[4 * t + e], dp);
          }
        }
        // element r: query row 8*(r/4) + 4*lh + r%4 of the block
        float p[16], ds[16];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const f32x4 L4 = *reinterpret_cast<const f32x4 *>(ls + 8 * g + 4 * lh);
          const f32x4 D4 = *reinterpret_cast<const f32x4 *>(ls + kF32BK + 8 * g + 4 * lh);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int r = 4 * g + e;
            p[r] = fast_exp2(__builtin_fmaf(s[r], c, -L4[e]));
            ds[r] = p[r] * (dp[r] - D4[e]);
          }
        }
#pragma unroll
        for (int dt = 0; dt < ND; ++dt) {
          const float *gtr = gt + (dt * 32 + l32) * S::TS + 4 * lh;
          const float *qtr = qt + (dt * 32 + l32) * S::TS + 4 * lh;
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            const f32x4 a = *reinterpret_cast<const f32x4 *>(gtr + 8 * jj);
            const f32x4 b = *reinterpret_cast<const f32x4 *>(qtr + 8 * jj);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              adv[dt] = mma32f(a[e], p[4 * jj + e], adv[dt]);
              adk[dt] = mma32f(b[e], ds[4 * jj + e], adk[dt]);
            }
          }
        }
      }
      if (j + 1 < nb) f32_store_qblk<D, NT>(regs, smem + ((j + 1) & 1) * S::kBuf, tid);
      __syncthreads();
    }
    if (key_ok) {
      // element r of tile dt: d = 32*dt + 8*(r/4) + 4*lh + r%4 of this lane's key
      float *krow = dk + ((int64_t)key * H + h) * D;
      float *vrow = dv + ((int64_t)key * H + h) * D;
#pragma unroll
      for (int dt = 0; dt < ND; ++dt)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          f32x4 wk, wv;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            wk[e] = adk[dt][g * 4 + e] * scale;
            wv[e] = adv[dt][g * 4 + e];
          }
          *reinterpret_cast<f32x4 *>(krow + dt * 32 + g * 8 + lh * 4) = wk;
          *reinterpret_cast<f32x4 *>(vrow + dt * 32 + g * 8 + lh * 4) = wv;
        }
    }
  }
}

// ---------------------------------------------------------------------------
// Backward at D in {128, 256} on v_mfma_f32_16x16x4_f32.  The 32x32x2
// kernels above hold a row's (or key's) whole Q^T / dO^T (or K^T / V^T)
// operands, 2 * D/2 floats, beside D/32 accumulator tiles: 512 registers and
// more at D = 256; at D = 128 they fit at one wave per SIMD, 4.4% slower
// than these kernels on C2's lengths (fp32 fwd+bwd 20.96 against 20.04 ms).
// With 16 rows (keys) per wave each lane group lq holds only the quarter of
// the features it reduces over (Q = D/4 per operand), as the fp32 absorb
// kernels do:
//   * products over d (S, dP): step i takes feature Q*lq + i in lane group
//     lq, so a lane reads Q consecutive floats of its LDS row;
//   * products over keys / rows (dQ^T, dV^T, dK^T): output tile (a, b) holds
//     feature 64a + 4m + b in its row m and step j4 takes the key / row
//     4*lq + j4 -- the one whose S / dS element j4 the lane holds -- so the A
//     operand is one 16-byte LDS read over b and the B operand needs no
//     exchange; a lane's accumulators hold features 64a + 16*lq + 4r + b,
//     stored as 16-byte runs.
// 16-row K / V (dQ) or Q / dO (dK/dV) tiles, double-buffered, staged by
// buffer_load ... lds, one instruction per row (D = 256 floats = 64 lanes x
// 16 bytes).
// ---------------------------------------------------------------------------
constexpr int kX4Rows = 16;  // rows per LDS tile

template <int D>
struct F32x4Smem {
  static constexpr int XS = D + 4;                  // row stride (floats)
  static constexpr int kTile = kX4Rows * XS;        // one tile
  static constexpr int kBuf = 2 * kTile + 2 * kX4Rows;  // two tiles (+ LSE, delta)
  static constexpr int kBytes = 2 * kBuf * 4;       // double buffered
};

// LDS-DMA of token rows [0, 16) of one head of a [T, H, D] fp32 tensor (row
// r at byte r*row_bytes from src; rows at or past `rows` read as zeros) into
// a [16][XS] LDS tile: each of the 4 waves moves 4 rows, one instruction per
// row and 64-lane run of 16-byte chunks.
template <int D, int XS>
__device__ __forceinline__ void dma_rows_x4(const float *src, int rows, int row_bytes,
                                            uint32_t base, int wave, int lane) {
  const u32x4 rs = rsrc_words(src, (int64_t)rows * row_bytes);
#pragma unroll
  for (int part = 0; part < (D / 4 + 63) / 64; ++part) {
    const int ch = part * 64 + lane;
    if (ch < D / 4) {
#pragma unroll
      for (int n = 0; n < kX4Rows / 4; ++n) {
        const int r = wave * (kX4Rows / 4) + n;
        int32_t voff;
        asm volatile("v_add_u32 %0, %1, %2" : "=v"(voff) : "s"(r * row_bytes), "v"(ch * 16));
        lds_dma16(rs, base + (r * XS + part * 256) * 4, voff);
      }
    }
  }
}

// The lane's Q = D/4 features [Q*lq, Q*lq + Q) of row `row` of one head of a
// [T, H, D] fp32 tensor; rows outside the descriptor's range read as zeros.
template <int D>
__device__ __forceinline__ void load_row_quarter(float (&dst)[D / 4], rsrc_t r,
                                                 int row_byte_off, int lq) {
  constexpr int Q = D / 4;
#pragma unroll
  for (int i4 = 0; i4 < Q / 4; ++i4) {
    const f32x4 v = __builtin_bit_cast(f32x4, buf_load16(r, row_byte_off + (Q * lq + 4 * i4) * 4));
#pragma unroll
    for (int e = 0; e < 4; ++e) dst[4 * i4 + e] = v[e];
  }
}

__device__ __forceinline__ f32x4 mma4f(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// dQ, query-major over the forward's items (split items write scaled fp32
// partial rows), 4 waves x 16 rows per pass (an item's rows in passes of
// 64): per 16-key tile S^T = K Q^T, dP^T = V dO^T (K, V rows as A from LDS,
// this lane's row quarter as B), P^T, dS^T, then dQ^T += K^T dS^T.
template <int D>
__global__ __launch_bounds__(256, 2) void varlen_dq_f32x4_kernel(
    const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v,
    const float *__restrict__ dout, const float *__restrict__ lse,
    const float *__restrict__ delta, float *__restrict__ dq, float *__restrict__ part_dq,
    const int32_t *__restrict__ items, int H, float c, float scale) {
  using S = F32x4Smem<D>;
  constexpr int Q = D / 4, NA = D / 64, XS = S::XS;
  extern __shared__ __align__(16) float smem_x4[];
  const int item = blockIdx.x / H, h = blockIdx.x % H;
  const PlanItem it = load_item(items, item);
  const int iq0 = it.v[0], q1 = it.v[1], k0 = it.v[2], k1 = it.v[3], pbase = it.v[4];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, lq = lane >> 4;
  const int row_bytes = H * D * 4;
  const int nt = (k1 - k0 + kX4Rows - 1) / kX4Rows;
  auto issue = [&](int kb, int buf) {
    const int rows = uniform_clamp(k1 - kb, kX4Rows);
    const int64_t off = ((int64_t)kb * H + h) * D;
    float *base = smem_x4 + buf * S::kBuf;
    dma_rows_x4<D, XS>(k + off, rows, row_bytes, lds_addr(base), wave, lane);
    dma_rows_x4<D, XS>(v + off, rows, row_bytes, lds_addr(base + S::kTile), wave, lane);
  };
  for (int q0 = iq0; q0 < q1; q0 += 4 * kX4Rows) {
    const int qrow = q0 + wave * kX4Rows + l16;
    const bool row_ok = qrow < q1;
    const bool wave_active = q0 + wave * kX4Rows < q1;
    if (nt > 0) issue(k0, 0);
    float qf[Q], gf[Q];
    {
      const int64_t nb = (int64_t)(q1 - q0) * row_bytes;
      const int64_t off = ((int64_t)q0 * H + h) * D;
      const int roff = (wave * kX4Rows + l16) * row_bytes;
      load_row_quarter<D>(qf, make_rsrc(q + off, nb), roff, lq);
      load_row_quarter<D>(gf, make_rsrc(dout + off, nb), roff, lq);
    }
    const float L = row_ok ? lse[(int64_t)qrow * H + h] : 0.f;
    const float dl = row_ok ? delta[(int64_t)qrow * H + h] : 0.f;
    f32x4 acc[NA][4];
#pragma unroll
    for (int a = 0; a < NA; ++a)
#pragma unroll
      for (int b = 0; b < 4; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int j = 0; j < nt; ++j) {
      wait_vmcnt<0>();
      __syncthreads();  // tile j landed; every wave is done with the other buffer
      if (j + 1 < nt) issue(k0 + (j + 1) * kX4Rows, (j + 1) & 1);
      const int kb = k0 + j * kX4Rows;
      if (wave_active) {
        const float *ks = smem_x4 + (j & 1) * S::kBuf;
        const float *vs = ks + S::kTile;
        // S^T, dP^T (16 keys x 16 rows): lane holds key kb + 4*lq + r of its row
        f32x4 s2[2], dp2[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) s2[e] = dp2[e] = f32x4{0.f, 0.f, 0.f, 0.f};
        const float *ka = ks + l16 * XS + Q * lq;
        const float *va = vs + l16 * XS + Q * lq;
#pragma unroll
        for (int i4 = 0; i4 < Q / 4; ++i4) {
          const f32x4 kv = *reinterpret_cast<const f32x4 *>(ka + 4 * i4);
          const f32x4 vv = *reinterpret_cast<const f32x4 *>(va + 4 * i4);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            s2[e & 1] = mma4f(kv[e], qf[4 * i4 + e], s2[e & 1]);
            dp2[e & 1] = mma4f(vv[e], gf[4 * i4 + e], dp2[e & 1]);
          }
        }
        const f32x4 s = s2[0] + s2[1], dp = dp2[0] + dp2[1];
        float ds[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const bool kin = kb + 4 * lq + r < k1;
          const float p = kin ? fast_exp2(__builtin_fmaf(s[r], c, -L)) : 0.f;
          ds[r] = p * (dp[r] - dl);
        }
        // dQ^T += K^T dS^T over the tile's 16 keys (slot lq <-> key 4*lq + j4)
#pragma unroll
        for (int j4 = 0; j4 < 4; ++j4) {
          const float *kt = ks + (4 * lq + j4) * XS + 4 * l16;
#pragma unroll
          for (int a = 0; a < NA; ++a) {
            const f32x4 kv = *reinterpret_cast<const f32x4 *>(kt + 64 * a);
#pragma unroll
            for (int b = 0; b < 4; ++b) acc[a][b] = mma4f(kv[b], ds[j4], acc[a][b]);
          }
        }
      }
    }
    if (row_ok) {
      // lane: row qrow, features 64a + 16*lq + 4r + b
      float *orow = pbase < 0 ? dq + ((int64_t)qrow * H + h) * D
                              : part_dq + ((int64_t)(pbase + (qrow - iq0)) * H + h) * D;
#pragma unroll
      for (int a = 0; a < NA; ++a)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          f32x4 w;
#pragma unroll
          for (int b = 0; b < 4; ++b) w[b] = acc[a][b][r] * scale;
          *reinterpret_cast<f32x4 *>(orow + 64 * a + 16 * lq + 4 * r) = w;
        }
    }
    __syncthreads();  // the next pass's first DMA overwrites buffer 0
  }
}

// dK/dV, key-major over the plan's key tiles, 4 waves x 16 keys per pass (an
// item's keys in passes of 64): per 16-row query block (Q, dO rows, LSE and
// delta in LDS) S = Q K^T, dP = dO V^T (Q, dO rows as A, this lane's key
// quarter as B), P = exp2(S c - LSE), dS = P (dP - delta), then
// dV^T += dO^T P and dK^T += Q^T dS.  Rows past the segment arrive as zero Q
// and dO rows, so both products vanish for them.
template <int D>
__global__ __launch_bounds__(256, 1) void varlen_dkv_f32x4_kernel(
    const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v,
    const float *__restrict__ dout, const float *__restrict__ lse,
    const float *__restrict__ delta, float *__restrict__ dk, float *__restrict__ dv,
    const int32_t *__restrict__ items, int H, float c, float scale) {
  using S = F32x4Smem<D>;
  constexpr int Q = D / 4, NA = D / 64, XS = S::XS;
  extern __shared__ __align__(16) float smem_x4[];
  const int item = blockIdx.x / H, h = blockIdx.x % H;
  const PlanItem it = load_item(items, item);
  const int kt0 = it.v[0], kt1 = it.v[1], q0 = it.v[2], q1 = it.v[3];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, lq = lane >> 4;
  const int row_bytes = H * D * 4;
  const int nb = (q1 - q0 + kX4Rows - 1) / kX4Rows;
  // block qb: Q and dO rows, then LSE (waves 0, 2) and delta (waves 1, 3:
  // the pairs write the same bytes), one 4-byte DMA per lane < 16
  auto issue = [&](int qb, int buf) {
    const int rows = uniform_clamp(q1 - qb, kX4Rows);
    const int64_t off = ((int64_t)qb * H + h) * D;
    float *base = smem_x4 + buf * S::kBuf;
    dma_rows_x4<D, XS>(q + off, rows, row_bytes, lds_addr(base), wave, lane);
    dma_rows_x4<D, XS>(dout + off, rows, row_bytes, lds_addr(base + S::kTile), wave, lane);
    const float *vec = (wave & 1) ? delta : lse;
    const u32x4 rv = rsrc_words32(vec + (int64_t)qb * H + h, (uint32_t)(rows * H * 4));
    if (lane < kX4Rows)
      lds_dma4(rv, lds_addr(base + 2 * S::kTile + (wave & 1) * kX4Rows), lane * H * 4);
  };
  for (int k0 = kt0; k0 < kt1; k0 += 4 * kX4Rows) {
    const int key = k0 + wave * kX4Rows + l16;
    const bool key_ok = key < kt1;
    const bool wave_active = k0 + wave * kX4Rows < kt1;
    if (nb > 0) issue(q0, 0);
    float kf[Q], vf[Q];
    {
      const int64_t nbk = (int64_t)(kt1 - k0) * row_bytes;
      const int64_t off = ((int64_t)k0 * H + h) * D;
      const int roff = (wave * kX4Rows + l16) * row_bytes;
      load_row_quarter<D>(kf, make_rsrc(k + off, nbk), roff, lq);
      load_row_quarter<D>(vf, make_rsrc(v + off, nbk), roff, lq);
    }
    f32x4 adk[NA][4], adv[NA][4];
#pragma unroll
    for (int a = 0; a < NA; ++a)
#pragma unroll
      for (int b = 0; b < 4; ++b) adk[a][b] = adv[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int j = 0; j < nb; ++j) {
      wait_vmcnt<0>();
      __syncthreads();  // block j landed; every wave is done with the other buffer
      if (j + 1 < nb) issue(q0 + (j + 1) * kX4Rows, (j + 1) & 1);
      if (wave_active) {
        const float *qs = smem_x4 + (j & 1) * S::kBuf;
        const float *gs = qs + S::kTile;
        const float *ls = qs + 2 * S::kTile;
        // S, dP (16 rows x 16 keys): lane holds row 4*lq + r of the block for its key
        f32x4 s2[2], dp2[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) s2[e] = dp2[e] = f32x4{0.f, 0.f, 0.f, 0.f};
        const float *qa = qs + l16 * XS + Q * lq;
        const float *ga = gs + l16 * XS + Q * lq;
#pragma unroll
        for (int i4 = 0; i4 < Q / 4; ++i4) {
          const f32x4 qv = *reinterpret_cast<const f32x4 *>(qa + 4 * i4);
          const f32x4 gv = *reinterpret_cast<const f32x4 *>(ga + 4 * i4);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            s2[e & 1] = mma4f(qv[e], kf[4 * i4 + e], s2[e & 1]);
            dp2[e & 1] = mma4f(gv[e], vf[4 * i4 + e], dp2[e & 1]);
          }
        }
        const f32x4 s = s2[0] + s2[1], dp = dp2[0] + dp2[1];
        const f32x4 L4 = *reinterpret_cast<const f32x4 *>(ls + 4 * lq);
        const f32x4 D4 = *reinterpret_cast<const f32x4 *>(ls + kX4Rows + 4 * lq);
        float p[4], ds[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          p[r] = fast_exp2(__builtin_fmaf(s[r], c, -L4[r]));
          ds[r] = p[r] * (dp[r] - D4[r]);
        }
        // dV^T += dO^T P, dK^T += Q^T dS over the block's 16 rows (slot lq <-> row 4*lq + j4)
#pragma unroll
        for (int j4 = 0; j4 < 4; ++j4) {
          const float *gt = gs + (4 * lq + j4) * XS + 4 * l16;
          const float *qt = qs + (4 * lq + j4) * XS + 4 * l16;
#pragma unroll
          for (int a = 0; a < NA; ++a) {
            const f32x4 gv = *reinterpret_cast<const f32x4 *>(gt + 64 * a);
            const f32x4 qv = *reinterpret_cast<const f32x4 *>(qt + 64 * a);
#pragma unroll
            for (int b = 0; b < 4; ++b) {
              adv[a][b] = mma4f(gv[b], p[j4], adv[a][b]);
              adk[a][b] = mma4f(qv[b], ds[j4], adk[a][b]);
            }
          }
        }
      }
    }
    if (key_ok) {
      // lane: key `key`, features 64a + 16*lq + 4r + b
      float *krow = dk + ((int64_t)key * H + h) * D;
      float *vrow = dv + ((int64_t)key * H + h) * D;
#pragma unroll
      for (int a = 0; a < NA; ++a)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          f32x4 wk, wv;
#pragma unroll
          for (int b = 0; b < 4; ++b) {
            wk[b] = adk[a][b][r] * scale;
            wv[b] = adv[a][b][r];
          }
          const int f = 64 * a + 16 * lq + 4 * r;
          *reinterpret_cast<f32x4 *>(krow + f) = wk;
          *reinterpret_cast<f32x4 *>(vrow + f) = wv;
        }
    }
    __syncthreads();  // the next pass's first DMA overwrites buffer 0
  }
}

template <int D>
void launch_dq_f32x4(const VarlenArgs &a, hipStream_t st) {
  const int smem = F32x4Smem<D>::kBytes;
  allow_dynamic_lds(reinterpret_cast<const void *>(&varlen_dq_f32x4_kernel<D>), smem);
  hipLaunchKernelGGL((varlen_dq_f32x4_kernel<D>), dim3((unsigned)(a.n_items * a.H)), dim3(256),
                     smem, st, (const float *)a.q, (const float *)a.k, (const float *)a.v,
                     (const float *)a.dout, a.lse_in, a.delta, (float *)a.dq, a.part_o, a.items,
                     a.H, a.scale * kLog2e, a.scale);
}

template <int D>
void launch_dkv_f32x4(const VarlenArgs &a, hipStream_t st) {
  const int smem = F32x4Smem<D>::kBytes;
  allow_dynamic_lds(reinterpret_cast<const void *>(&varlen_dkv_f32x4_kernel<D>), smem);
  hipLaunchKernelGGL((varlen_dkv_f32x4_kernel<D>), dim3((unsigned)(a.n_kv * a.H)), dim3(256),
                     smem, st, (const float *)a.q, (const float *)a.k, (const float *)a.v,
                     (const float *)a.dout, a.lse_in, a.delta, (float *)a.dk, (float *)a.dv,
                     a.kv_items, a.H, a.scale * kLog2e, a.scale);
}

template <int D, int NW>
void launch_dq_f32_nw(const VarlenArgs &a, hipStream_t st) {
  const int smem = F32DqSmem<D>::kBytes;
  allow_dynamic_lds(reinterpret_cast<const void *>(&varlen_dq_f32_kernel<D, NW>), smem);
  hipLaunchKernelGGL((varlen_dq_f32_kernel<D, NW>), dim3((unsigned)(a.n_items * a.H)),
                     dim3(64 * NW), smem, st, (const float *)a.q, (const float *)a.k,
                     (const float *)a.v, (const float *)a.dout, a.lse_in, a.delta,
                     (float *)a.dq, a.part_o, a.items, a.H, a.scale * kLog2e, a.scale);
}

template <int D, int NW>
void launch_dkv_f32_nw(const VarlenArgs &a, hipStream_t st) {
  const int smem = F32DkvSmem<D>::kBytes;
  allow_dynamic_lds(reinterpret_cast<const void *>(&varlen_dkv_f32_kernel<D, NW>), smem);
  hipLaunchKernelGGL((varlen_dkv_f32_kernel<D, NW>), dim3((unsigned)(a.n_kv * a.H)),
                     dim3(64 * NW), smem, st, (const float *)a.q, (const float *)a.k,
                     (const float *)a.v, (const float *)a.dout, a.lse_in, a.delta,
                     (float *)a.dk, (float *)a.dv, a.kv_items, a.H, a.scale * kLog2e, a.scale);
}

}  // namespace

bool f32_varlen_mfma_d(int D) { return D == 32 || D == 64 || D == 128 || D == 256; }
bool f32_varlen_bwd_mfma_d(int D) { return D == 32 || D == 64 || D == 128 || D == 256; }

void launch_f32_varlen_dq(const VarlenArgs &a, hipStream_t st) {
  if (a.n_items == 0) return;
  const bool wide = a.q_tile == kVarlenWideTile;
  switch (a.D) {
    case 32: wide ? launch_dq_f32_nw<32, 8>(a, st) : launch_dq_f32_nw<32, 4>(a, st); break;
    case 64: wide ? launch_dq_f32_nw<64, 8>(a, st) : launch_dq_f32_nw<64, 4>(a, st); break;
    case 128: launch_dq_f32x4<128>(a, st); break;
    case 256: launch_dq_f32x4<256>(a, st); break;
    default: break;
  }
}

// Key tiles of the plan on 4 waves; the 32x32x2 kernel walks longer items
// (fused-planned chunks at D <= 64) in 128-key steps, the 16x16x4 kernel any
// item in 64-key steps.
void launch_f32_varlen_dkv(const VarlenArgs &a, hipStream_t st) {
  if (a.n_kv == 0) return;
  switch (a.D) {
    case 32: launch_dkv_f32_nw<32, 4>(a, st); break;
    case 64: launch_dkv_f32_nw<64, 4>(a, st); break;
    case 128: launch_dkv_f32x4<128>(a, st); break;
    case 256: launch_dkv_f32x4<256>(a, st); break;
    default: break;
  }
}

void launch_f32_varlen_fwd(const VarlenArgs &a, hipStream_t st) {
  if (a.n_items == 0) return;
  switch (a.D) {
    case 32: launch_fwd_f32_d<32>(a, st); break;
    case 64: launch_fwd_f32_d<64>(a, st); break;
    case 128: launch_fwd_f32_d<128>(a, st); break;
    case 256: launch_fwd_f32_d<256>(a, st); break;
    default: break;
  }
}

}  // namespace vafa
