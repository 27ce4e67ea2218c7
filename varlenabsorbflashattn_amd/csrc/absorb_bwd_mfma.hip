// Absorbed ragged target attention backward on gfx950 matrix cores
// (replaces ta/kernels.py:354-498 and the dX family ta/kernels.py:528-900).
//
// With rows r = (token, head) pairs, P = exp2(c * u_r.X_j - LSE_r) rebuilt
// from the forward's log2-domain LSE, dP = dAX_r . X_j and dS = P (dP - delta):
//   * query side, absorb_du_kernel: one workgroup (4 waves x 16 rows) per
//     token tile with the sample's whole key range; raw X streams through a
//     3-deep LDS-DMA ring like the forward's.  Per 32-key tile, on 16x16x32
//     products (16 rows per wave keep both fp32 accumulators in registers):
//       S^T = X U^T, dP^T = X dAX^T   (X rows as A, U^T / dAX^T in registers)
//       du^T += X^T dS^T, aX^T += X^T P^T   (X^T from ds_read_b64_tr_b16)
//     du = scale * du is written in the input dtype, aX (for dW_V) in fp32.
//   * key side, absorb_dx_kernel: one workgroup (4 waves x 32 keys) per key
//     tile, X held in registers, walking the sample's rows in blocks of 32
//     staged row-major in LDS by DMA:
//       S = U X^T, dP = dAX X^T,  dX^T += U^T (scale dS) + dAX^T P
//     summed over heads in registers (no partial buffers, no atomics).
// dAX = dO W_V^T arrives in the input dtype: the reference rounds it to that
// dtype before every product it feeds (ta/kernels.py:480, 617-626).
#include "absorb_tiles.h"

namespace vafa {

namespace {

using namespace absorb;

// LDS-DMA of 32 consecutive rows [F] of a row slab into a padded [32][XS]
// LDS block (rows past the slab and chunks past F arrive as zeros); each of
// the workgroup's NW waves moves 32/NW rows, one instruction per row.
template <int FP, int NW>
__device__ __forceinline__ void dma_block(const u32x4 &rs, int F, uint32_t base, int wave,
                                          int lane) {
  constexpr int XS = AbsSmem<FP>::XS;
  const uint32_t off = lane < F / 8 ? (uint32_t)lane * 16u : 0x80000000u;
  if (lane < FP / 8) {
#pragma unroll
    for (int n = 0; n < 32 / NW; ++n) {
      const int r = wave * (32 / NW) + n;
      lds_dma16(rs, base + r * XS * 2, (int32_t)(off + (uint32_t)(r * F * 2)));
    }
  }
}

constexpr int kDuWaves = 4;  // 4 waves x 16 rows = one forward row tile

// A operand of a 16x16x32 product out of a row-major [keys][XS] tile,
// transposed: lane l gets column f0 + l%16 at the 8 keys of its k slots,
// slots (l/16)*8 + t <-> keys 4*(l/16) + t (t < 4) and 16 + 4*(l/16) + t - 4.
template <typename T>
__device__ __forceinline__ typename Mfma<T>::v8 tr_operand16(const T *tile, int stride, int f0,
                                                             int lane) {
  const int i = lane & 15, g = lane >> 4;
  const T *p = tile + (4 * g + (i >> 2)) * stride + f0 + 4 * (i & 3);
  return as_v8<T>(join(lds_tr16(p), lds_tr16(p + 16 * stride)));
}

template <typename T, int FP>
__global__ __launch_bounds__(64 * kDuWaves, 2) void absorb_du_kernel(
    const T *__restrict__ u, const T *__restrict__ X, const T *__restrict__ dax,
    const float *__restrict__ lse, const float *__restrict__ delta, T *__restrict__ du,
    float *__restrict__ ax, const int32_t *__restrict__ items, int H, int F, float c,
    float scale) {
  using M16 = Mfma16<T>;
  using v8 = typename Mfma<T>::v8;
  using S = AbsSmem<FP>;
  constexpr int NK = FP / 32;   // 32-wide reduction chunks of S^T / dP^T
  constexpr int NF = FP / 16;   // 16-row f tiles of aX^T / du^T
  constexpr int kPerWave = kBK / kDuWaves;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  T *smem = reinterpret_cast<T *>(smem_raw);

  const PlanItem it = load_item(items, blockIdx.x);
  const int t0 = it.v[0], t1 = it.v[1], k0 = it.v[2], k1 = it.v[3];
  if (t1 <= t0) return;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, lq = lane >> 4;
  const int nrows = (t1 - t0) * H;
  const int row = wave * 16 + l16;
  const bool row_ok = row < nrows;
  const bool wave_active = wave * 16 < nrows;
  const int nt = (k1 - k0 + kBK - 1) / kBK;

  auto issue = [&](int kb, int buf) {
    const int rows = k1 - kb < kBK ? (k1 - kb > 0 ? k1 - kb : 0) : kBK;
    dma_block<FP, kDuWaves>(rsrc_words(X + (int64_t)kb * F, (int64_t)rows * F * 2), F,
                            lds_addr(smem + buf * S::kTile), wave, lane);
  };
#pragma unroll
  for (int b = 0; b < kNBuf - 1; ++b) issue(k0 + b * kBK, b);

  // U^T and dAX^T fragments (B operands of S^T and dP^T), rows past the tile zero
  v8 uf[NK], gf[NK];
  float L, dl;
  {
    const int64_t nb = (int64_t)nrows * F * 2;
    const rsrc_t ru = make_rsrc(u + (int64_t)t0 * H * F, nb);
    const rsrc_t rg = make_rsrc(dax + (int64_t)t0 * H * F, nb);
    const int fchunks = F / 8;
#pragma unroll
    for (int kc = 0; kc < NK; ++kc) {
      const int ch = kc * 4 + lq;
      const int off = ch < fchunks ? row * F * 2 + ch * 16 : 0x7fffffff;
      u32x4 w = buf_load16(ru, off);
      u32x4 g = buf_load16(rg, off);
      // waited for here, in the prologue, not inside the key loop where a
      // compiler vmcnt wait would also drain the LDS-DMA ring
      asm volatile("" : "+v"(w), "+v"(g));
      uf[kc] = as_v8<T>(w);
      gf[kc] = as_v8<T>(g);
    }
    L = row_ok ? lse[(int64_t)t0 * H + row] : __builtin_inff();
    dl = row_ok ? delta[(int64_t)t0 * H + row] : 0.f;
    asm volatile("" : "+v"(L), "+v"(dl));
  }
  f32x4 adu[NF], aax[NF];
#pragma unroll
  for (int i = 0; i < NF; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) adu[i][r] = aax[i][r] = 0.f;

  for (int j = 0; j < nt; ++j) {
    wait_vmcnt<(kNBuf - 2) * kPerWave>();
    __syncthreads();
    issue(k0 + (j + kNBuf - 1) * kBK, (j + kNBuf - 1) % kNBuf);
    const int kb = k0 + j * kBK;
    const T *xs = smem + (j % kNBuf) * S::kTile;
    if (wave_active) {
      // S^T, dP^T: two 16-key halves; element r of half mt is key
      // kb + 16*mt + 4*lq + r of this lane's row
      f32x4 s[2], dp[2];
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
        for (int r = 0; r < 4; ++r) s[mt][r] = dp[mt][r] = 0.f;
#pragma unroll
        for (int kc = 0; kc < NK; ++kc) {
          const u32x4 a = *reinterpret_cast<const u32x4 *>(xs + (16 * mt + l16) * S::XS +
                                                           kc * 32 + lq * 8);
          s[mt] = M16::mma(as_v8<T>(a), uf[kc], s[mt]);
          dp[mt] = M16::mma(as_v8<T>(a), gf[kc], dp[mt]);
        }
      }
      const bool tail = kb + kBK > k1;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float p = fast_exp2(__builtin_fmaf(s[mt][r], c, -L));
          if (tail && kb + 16 * mt + 4 * lq + r >= k1) p = 0.f;
          s[mt][r] = p;
          dp[mt][r] = p * (dp[mt][r] - dl);
        }
      // B operands over the tile's keys: slot 8*lq + t <-> key 4*lq + t (t < 4),
      // 16 + 4*lq + t - 4 (t >= 4), matching tr_operand16
      v8 pb, sb;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        pb[r] = static_cast<T>(s[0][r]);
        pb[4 + r] = static_cast<T>(s[1][r]);
        sb[r] = static_cast<T>(dp[0][r]);
        sb[4 + r] = static_cast<T>(dp[1][r]);
      }
#pragma unroll
      for (int ft = 0; ft < NF; ++ft) {
        const v8 a = tr_operand16<T>(xs, S::XS, ft * 16, lane);
        aax[ft] = M16::mma(a, pb, aax[ft]);
        adu[ft] = M16::mma(a, sb, adu[ft]);
      }
    }
  }
  wait_vmcnt<0>();

  if (!row_ok) return;
  typedef __attribute__((__vector_size__(4 * sizeof(T)))) T T4;
  const int64_t ro = ((int64_t)t0 * H + row) * F;
#pragma unroll
  for (int ft = 0; ft < NF; ++ft) {
    const int f = ft * 16 + lq * 4;  // element r is f + r of this lane's row
    if (f >= F) continue;
    T4 wu;
#pragma unroll
    for (int e = 0; e < 4; ++e) wu[e] = static_cast<T>(adu[ft][e] * scale);
    *reinterpret_cast<T4 *>(du + ro + f) = wu;
    *reinterpret_cast<f32x4 *>(ax + ro + f) = aax[ft];
  }
}

constexpr int kDxWaves = 4;

template <int FP>
struct DxSmem {
  static constexpr int XS = AbsSmem<FP>::XS;
  static constexpr int kBlk = 32 * XS;                    // one [32][XS] row block
  static constexpr int kBufBytes = 2 * kBlk * 2 + 2 * 32 * 4;  // U, dAX, LSE, delta
  static constexpr int kBytes = 2 * kBufBytes;
};

template <typename T, int FP>
__global__ __launch_bounds__(64 * kDxWaves, 2) void absorb_dx_kernel(
    const T *__restrict__ u, const T *__restrict__ X, const T *__restrict__ dax,
    const float *__restrict__ lse, const float *__restrict__ delta, T *__restrict__ dX,
    const int32_t *__restrict__ items, int H, int F, float c, float scale) {
  using M = Mfma<T>;
  using S = DxSmem<FP>;
  constexpr int NC = FP / 16;
  constexpr int NF = FP / 32;
  constexpr int XS = S::XS;
  extern __shared__ __align__(16) unsigned char smem_raw[];

  const PlanItem it = load_item(items, blockIdx.x);
  const int k0 = it.v[0], k1 = it.v[1], t0 = it.v[2], t1 = it.v[3];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lrow = lane & 31, lhalf = lane >> 5;
  const int key = k0 + wave * 32 + lrow;
  const bool key_ok = key < k1;
  const bool wave_active = k0 + wave * 32 < k1;
  const int r0 = t0 * H, r1 = t1 * H;
  const int nblk = (r1 - r0 + 31) / 32;

  // stage one 32-row block of U, dAX, LSE and delta (rows past r1 are zero,
  // so they add nothing to dX: both products carry a zero U or dAX row)
  auto issue = [&](int blk, int buf) {
    unsigned char *base = smem_raw + buf * S::kBufBytes;
    const int rb = r0 + blk * 32;
    const int rows = r1 - rb < 32 ? r1 - rb : 32;
    const int64_t nb = (int64_t)rows * F * 2;
    dma_block<FP, kDxWaves>(rsrc_words(u + (int64_t)rb * F, nb), F, lds_addr(base), wave, lane);
    dma_block<FP, kDxWaves>(rsrc_words(dax + (int64_t)rb * F, nb), F,
                            lds_addr(base + S::kBlk * 2), wave, lane);
    // waves 0/2 move LSE and waves 1/3 delta (the pairs write identical bytes):
    // one 128-byte DMA per wave keeps every wave's vmcnt count equal
    const float *vec = (wave & 1) ? delta : lse;
    const u32x4 rv = rsrc_words(vec + rb, (int64_t)rows * 4);
    if (lane < 8)
      lds_dma16(rv, lds_addr(base + 2 * S::kBlk * 2 + (wave & 1) * 128), lane * 16);
  };

  if (nblk > 0) issue(0, 0);

  // X rows of this wave's 32 keys: B operand of S = U X^T and dP = dAX X^T
  typename M::v8 xf[NC];
  {
    const rsrc_t rx = make_rsrc(X + (int64_t)k0 * F, (int64_t)(k1 - k0) * F * 2);
    const int fchunks = F / 8;
#pragma unroll
    for (int cc = 0; cc < NC; ++cc) {
      const int ch = cc * 2 + lhalf;
      u32x4 w = buf_load16(rx, ch < fchunks ? (wave * 32 + lrow) * F * 2 + ch * 16 : 0x7fffffff);
      asm volatile("" : "+v"(w));
      xf[cc] = as_v8<T>(w);
    }
  }
  f32x16 acc[NF];
#pragma unroll
  for (int i = 0; i < NF; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[i][r] = 0.f;

  for (int j = 0; j < nblk; ++j) {
    wait_vmcnt<0>();
    __syncthreads();  // block j visible; every wave is done with block j-1's buffer
    if (j + 1 < nblk) issue(j + 1, (j + 1) & 1);
    if (wave_active) {
      const unsigned char *base = smem_raw + (j & 1) * S::kBufBytes;
      const T *us = reinterpret_cast<const T *>(base);
      const T *gs = us + S::kBlk;
      const float *ls = reinterpret_cast<const float *>(base + 2 * S::kBlk * 2);
      f32x16 s, dp;
#pragma unroll
      for (int r = 0; r < 16; ++r) s[r] = dp[r] = 0.f;
#pragma unroll
      for (int cc = 0; cc < NC; ++cc) {
        const u32x4 a = *reinterpret_cast<const u32x4 *>(us + lrow * XS + cc * 16 + lhalf * 8);
        s = M::mma(as_v8<T>(a), xf[cc], s);
        const u32x4 b = *reinterpret_cast<const u32x4 *>(gs + lrow * XS + cc * 16 + lhalf * 8);
        dp = M::mma(as_v8<T>(b), xf[cc], dp);
      }
      // element r holds row (r/4)*8 + lhalf*4 + r%4 of the block, this lane's key
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x4 Lv = *reinterpret_cast<const f32x4 *>(ls + g * 8 + lhalf * 4);
        const f32x4 Dv = *reinterpret_cast<const f32x4 *>(ls + 32 + g * 8 + lhalf * 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = g * 4 + e;
          const float p = fast_exp2(__builtin_fmaf(s[r], c, -Lv[e]));
          s[r] = p;
          dp[r] = p * (dp[r] - Dv[e]) * scale;
        }
      }
      typename M::v8 pb[2], sb[2];
#pragma unroll
      for (int mm = 0; mm < 2; ++mm) {
        pb[mm] = pack8<T>(s, mm * 8);
        sb[mm] = pack8<T>(dp, mm * 8);
      }
#pragma unroll
      for (int ft = 0; ft < NF; ++ft)
#pragma unroll
        for (int mm = 0; mm < 2; ++mm) {
          acc[ft] = M::mma(tr_operand<T>(gs, XS, mm * 16, ft * 32, lane), pb[mm], acc[ft]);
          acc[ft] = M::mma(tr_operand<T>(us, XS, mm * 16, ft * 32, lane), sb[mm], acc[ft]);
        }
    }
  }

  if (!key_ok) return;
  typedef __attribute__((__vector_size__(4 * sizeof(T)))) T T4;
  T *dst = dX + (int64_t)key * F;
#pragma unroll
  for (int ft = 0; ft < NF; ++ft)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int f = ft * 32 + g * 8 + lhalf * 4;
      if (f >= F) continue;
      T4 w;
#pragma unroll
      for (int e = 0; e < 4; ++e) w[e] = static_cast<T>(acc[ft][g * 4 + e]);
      *reinterpret_cast<T4 *>(dst + f) = w;
    }
}

template <typename T, int FP>
void launch_du_fp(const AbsorbArgs &a, hipStream_t st) {
  const int smem = AbsSmem<FP>::kLoopBytes;
  hipFuncSetAttribute(reinterpret_cast<const void *>(&absorb_du_kernel<T, FP>),
                      hipFuncAttributeMaxDynamicSharedMemorySize, smem);
  hipLaunchKernelGGL((absorb_du_kernel<T, FP>), dim3((unsigned)a.n_qseg), dim3(64 * kDuWaves), smem,
                     st, (const T *)a.u, (const T *)a.X, (const T *)a.dax, a.lse_in, a.delta,
                     (T *)a.du, a.ax, a.qseg_items, a.H, a.F, a.scale * kLog2e, a.scale);
}

template <typename T, int FP>
void launch_dx_fp(const AbsorbArgs &a, hipStream_t st) {
  const int smem = DxSmem<FP>::kBytes;
  hipFuncSetAttribute(reinterpret_cast<const void *>(&absorb_dx_kernel<T, FP>),
                      hipFuncAttributeMaxDynamicSharedMemorySize, smem);
  hipLaunchKernelGGL((absorb_dx_kernel<T, FP>), dim3((unsigned)a.n_kv), dim3(64 * kDxWaves),
                     smem, st, (const T *)a.u, (const T *)a.X, (const T *)a.dax, a.lse_in,
                     a.delta, (T *)a.dX, a.kv_items, a.H, a.F, a.scale * kLog2e, a.scale);
}

}  // namespace

template <typename T>
void launch_mfma_absorb_du(const AbsorbArgs &a, hipStream_t st) {
  if (a.n_qseg == 0) return;
  switch (padded_f(a.F)) {
    case 64: launch_du_fp<T, 64>(a, st); break;
    case 128: launch_du_fp<T, 128>(a, st); break;
    case 192: launch_du_fp<T, 192>(a, st); break;
    case 224: launch_du_fp<T, 224>(a, st); break;
    case 256: launch_du_fp<T, 256>(a, st); break;
    default: break;
  }
}

template <typename T>
void launch_mfma_absorb_dx(const AbsorbArgs &a, hipStream_t st) {
  if (a.n_kv == 0) return;
  switch (padded_f(a.F)) {
    case 64: launch_dx_fp<T, 64>(a, st); break;
    case 128: launch_dx_fp<T, 128>(a, st); break;
    case 192: launch_dx_fp<T, 192>(a, st); break;
    case 224: launch_dx_fp<T, 224>(a, st); break;
    case 256: launch_dx_fp<T, 256>(a, st); break;
    default: break;
  }
}

template void launch_mfma_absorb_du<bf16>(const AbsorbArgs &, hipStream_t);
template void launch_mfma_absorb_du<f16>(const AbsorbArgs &, hipStream_t);
template void launch_mfma_absorb_dx<bf16>(const AbsorbArgs &, hipStream_t);
template void launch_mfma_absorb_dx<f16>(const AbsorbArgs &, hipStream_t);

}  // namespace vafa
