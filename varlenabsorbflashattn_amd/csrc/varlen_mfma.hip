// Packed varlen FlashAttention on gfx950 matrix cores (bf16 / f16 inputs).
//
// Forward (replaces fa/kernels.py:64-175 and the split variant 516-628):
// one workgroup = 4 waves = 128 query rows of one head; each wave owns 32
// rows.  Key/value tiles of 64 keys are staged once per workgroup in LDS
// (K row-major, V transposed) with a register prefetch of the next tile, so
// each tile is read from HBM/L2 once for 128 queries.  Per 64-key tile a wave
// issues 16 MFMAs for S^T = K Q^T and 16 for O^T += V^T P^T (D=128).  The
// online softmax runs in the log2 domain, the row max needs one cross-lane
// exchange (lane l <-> l^32) and the row sum none until the end.
#include "kernels.h"
#include "mfma.h"

namespace vafa {

namespace {

constexpr int kBM = kVarlenQTile;  // 128 query rows per workgroup
constexpr int kBN = 64;            // keys per LDS tile
constexpr int kKPad = 8;           // K row padding (elements)
constexpr int kVPad = 4;           // V^T row padding (elements)

template <int D>
struct FwdSmem {
  static constexpr int kKs = kBN * (D + kKPad);  // elements per K buffer
  static constexpr int kVt = D * (kBN + kVPad);  // elements per V^T buffer
  static constexpr int kBuf = kKs + kVt;
  static constexpr int kBytes = 2 * kBuf * 2;    // double buffered, 2 B/elt
};

// Global -> register stage of one K/V tile (zero-filled past k_end).
template <int D>
struct TileRegs {
  static constexpr int kKChunks = kBN * D / 8 / 256;           // 16 B chunks per thread
  static constexpr int kVQuads = (kBN / 4) * (D / 8);          // 4-key x 8-d quads
  static constexpr int kVPer = (kVQuads + 255) / 256;
  u32x4 kc[kKChunks > 0 ? kKChunks : 1];
  u32x4 vq[kVPer][4];
};

template <typename T, int D>
__device__ __forceinline__ void load_tile(TileRegs<D> &r, const T *__restrict__ k,
                                          const T *__restrict__ v, int kbase, int k_end, int H,
                                          int h, int tid) {
  constexpr int CPR = D / 8;  // chunks per row
#pragma unroll
  for (int i = 0; i < TileRegs<D>::kKChunks; ++i) {
    const int ci = tid + 256 * i;
    const int key = ci / CPR, dc = ci % CPR;
    const int gk = kbase + key;
    u32x4 val = {0u, 0u, 0u, 0u};
    if (gk < k_end) val = *reinterpret_cast<const u32x4 *>(k + ((int64_t)gk * H + h) * D + dc * 8);
    r.kc[i] = val;
  }
#pragma unroll
  for (int i = 0; i < TileRegs<D>::kVPer; ++i) {
    const int qi = tid + 256 * i;
    const int kq = qi / CPR, dc = qi % CPR;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int gk = kbase + kq * 4 + e;
      u32x4 val = {0u, 0u, 0u, 0u};
      if (qi < TileRegs<D>::kVQuads && gk < k_end)
        val = *reinterpret_cast<const u32x4 *>(v + ((int64_t)gk * H + h) * D + dc * 8);
      r.vq[i][e] = val;
    }
  }
}

template <typename T, int D>
__device__ __forceinline__ void store_tile(const TileRegs<D> &r, T *ks, T *vt, int tid) {
  constexpr int CPR = D / 8;
  constexpr int KS = D + kKPad, VS = kBN + kVPad;
#pragma unroll
  for (int i = 0; i < TileRegs<D>::kKChunks; ++i) {
    const int ci = tid + 256 * i;
    const int key = ci / CPR, dc = ci % CPR;
    *reinterpret_cast<u32x4 *>(ks + key * KS + dc * 8) = r.kc[i];
  }
#pragma unroll
  for (int i = 0; i < TileRegs<D>::kVPer; ++i) {
    const int qi = tid + 256 * i;
    if (qi >= TileRegs<D>::kVQuads) continue;
    const int kq = qi / CPR, dc = qi % CPR;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      u32x2 w;
      w[0] = half_of(r.vq[i][0], e) | (half_of(r.vq[i][1], e) << 16);
      w[1] = half_of(r.vq[i][2], e) | (half_of(r.vq[i][3], e) << 16);
      *reinterpret_cast<u32x2 *>(vt + (dc * 8 + e) * VS + kq * 4) = w;
    }
  }
}

template <typename T, int D>
__global__ __launch_bounds__(256, D >= 256 ? 1 : 2) void varlen_fwd_kernel(
    const T *__restrict__ q, const T *__restrict__ k, const T *__restrict__ v,
    T *__restrict__ o, float *__restrict__ lse, float *__restrict__ part_o,
    float *__restrict__ part_lse, const int32_t *__restrict__ items, int H, float c) {
  using M = Mfma<T>;
  constexpr int NC = D / 16;   // 16-wide d chunks (S^T reduction)
  constexpr int ND = D / 32;   // 32-row d tiles of O^T
  constexpr int KS = D + kKPad, VS = kBN + kVPad;
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

  // Q^T fragments (B operand): rows past q1 are zero.
  typename M::v8 qf[NC];
#pragma unroll
  for (int cc = 0; cc < NC; ++cc) {
    u32x4 val = {0u, 0u, 0u, 0u};
    if (row_ok)
      val = *reinterpret_cast<const u32x4 *>(q + ((int64_t)qrow * H + h) * D + cc * 16 +
                                              lhalf * 8);
    qf[cc] = as_v8<T>(val);
  }

  f32x16 acc[ND];
#pragma unroll
  for (int i = 0; i < ND; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[i][r] = 0.f;
  float m_run = kNegInf, l_part = 0.f;

  const int nt = (k1 - k0 + kBN - 1) / kBN;
  TileRegs<D> regs;
  if (nt > 0) {
    load_tile<T, D>(regs, k, v, k0, k1, H, h, tid);
    store_tile<T, D>(regs, smem, smem + FwdSmem<D>::kKs, tid);
  }
  __syncthreads();

  for (int j = 0; j < nt; ++j) {
    const int kbase = k0 + j * kBN;
    if (j + 1 < nt) load_tile<T, D>(regs, k, v, kbase + kBN, k1, H, h, tid);
    const T *ks = smem + (j & 1) * FwdSmem<D>::kBuf;
    const T *vt = ks + FwdSmem<D>::kKs;
    if (wave_active) {
      // S^T = K Q^T for two 32-key sub-tiles.
      f32x16 s[2];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
        for (int r = 0; r < 16; ++r) s[kt][r] = 0.f;
#pragma unroll
        for (int cc = 0; cc < NC; ++cc) {
          const u32x4 a = *reinterpret_cast<const u32x4 *>(ks + (kt * 32 + lrow) * KS +
                                                           cc * 16 + lhalf * 8);
          s[kt] = M::mma(as_v8<T>(a), qf[cc], s[kt]);
        }
      }
      // scale into the log2 domain, mask the key tail, row max
      const bool tail = kbase + kBN > k1;
      float mx = kNegInf;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float t = s[kt][r] * c;
          if (tail) {
            const int key = kbase + kt * 32 + (r >> 2) * 8 + lhalf * 4 + (r & 3);
            if (key >= k1) t = kNegInf;
          }
          s[kt][r] = t;
          mx = fmaxf(mx, t);
        }
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float m_new = fmaxf(m_run, mx);
      const float alpha = fast_exp2(m_run - m_new);
      m_run = m_new;
      float psum = 0.f;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float p = fast_exp2(s[kt][r] - m_new);
          s[kt][r] = p;
          psum += p;
        }
      l_part = l_part * alpha + psum;
#pragma unroll
      for (int i = 0; i < ND; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][r] *= alpha;
      // O^T += V^T P^T
      typename M::v8 pb[2][2];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int mm = 0; mm < 2; ++mm) pb[kt][mm] = pack8<T>(s[kt], mm * 8);
#pragma unroll
      for (int dt = 0; dt < ND; ++dt) {
        const T *vrow = vt + (dt * 32 + lrow) * VS + lhalf * 4;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int mm = 0; mm < 2; ++mm) {
            const int kk = kt * 32 + mm * 16;
            const u32x2 lo = *reinterpret_cast<const u32x2 *>(vrow + kk);
            const u32x2 hi = *reinterpret_cast<const u32x2 *>(vrow + kk + 8);
            acc[dt] = M::mma(as_v8<T>(join(lo, hi)), pb[kt][mm], acc[dt]);
          }
      }
    }
    if (j + 1 < nt) {
      T *nks = smem + ((j + 1) & 1) * FwdSmem<D>::kBuf;
      store_tile<T, D>(regs, nks, nks + FwdSmem<D>::kKs, tid);
    }
    __syncthreads();
  }

  if (!row_ok) return;
  const float l = l_part + __shfl_xor(l_part, 32, 64);
  const float inv = l > 0.f ? 1.f / l : 0.f;
  const float lse_v = l > 0.f ? m_run + fast_log2(l) : kNegInf;
  if (pbase < 0) {
    T *orow = o + ((int64_t)qrow * H + h) * D;
#pragma unroll
    for (int dt = 0; dt < ND; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        typedef __attribute__((__vector_size__(4 * sizeof(T)))) T T4;
        T4 w;
#pragma unroll
        for (int e = 0; e < 4; ++e) w[e] = static_cast<T>(acc[dt][g * 4 + e] * inv);
        *reinterpret_cast<T4 *>(orow + dt * 32 + g * 8 + lhalf * 4) = w;
      }
    if (lhalf == 0) lse[(int64_t)qrow * H + h] = lse_v;
  } else {
    const int64_t prow = pbase + (qrow - q0);
    float *orow = part_o + (prow * H + h) * D;
#pragma unroll
    for (int dt = 0; dt < ND; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        f32x4 w;
#pragma unroll
        for (int e = 0; e < 4; ++e) w[e] = acc[dt][g * 4 + e] * inv;
        *reinterpret_cast<f32x4 *>(orow + dt * 32 + g * 8 + lhalf * 4) = w;
      }
    if (lhalf == 0) part_lse[prow * H + h] = lse_v;
  }
}

}  // namespace

template <typename T, int D>
void launch_mfma_varlen_fwd(const VarlenArgs &a, hipStream_t st) {
  if (a.n_items == 0) return;
  const int smem = FwdSmem<D>::kBytes;
  hipFuncSetAttribute(reinterpret_cast<const void *>(&varlen_fwd_kernel<T, D>),
                      hipFuncAttributeMaxDynamicSharedMemorySize, smem);
  hipLaunchKernelGGL((varlen_fwd_kernel<T, D>), dim3((unsigned)(a.n_items * a.H)), dim3(256),
                     smem, st, (const T *)a.q, (const T *)a.k, (const T *)a.v, (T *)a.o, a.lse,
                     a.part_o, a.part_lse, a.items, a.H, a.scale * kLog2e);
}

#define VAFA_INST(T, D) template void launch_mfma_varlen_fwd<T, D>(const VarlenArgs &, hipStream_t);
VAFA_INST(bf16, 32)
VAFA_INST(bf16, 64)
VAFA_INST(bf16, 128)
VAFA_INST(bf16, 256)
VAFA_INST(f16, 32)
VAFA_INST(f16, 64)
VAFA_INST(f16, 128)
VAFA_INST(f16, 256)
#undef VAFA_INST

}  // namespace vafa
