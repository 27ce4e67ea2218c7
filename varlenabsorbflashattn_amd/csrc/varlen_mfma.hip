// Packed varlen FlashAttention on gfx950 matrix cores (bf16 / f16 inputs).
//
// Forward (replaces fa/kernels.py:64-175 and the split variant 516-628):
// one workgroup = NW waves (4 or 8, the plan's query tile / 32) of one head;
// each wave owns 32 rows.  Key/value tiles of 64 keys are staged once per
// workgroup in LDS (both row-major; V^T operands come from transposing LDS
// reads) with a register prefetch of the next tile, so each tile is read
// from HBM/L2 once for 128 or 256 queries.  Per 64-key tile a wave
// issues 16 MFMAs for S^T = K Q^T and 16 for O^T += V^T P^T (D=128).  The
// online softmax runs in the log2 domain against a lazily updated running
// max: a tile's row max is taken (one cross-lane register swap, lane l <->
// l^32) only when the tile's P sum shows the running max is out of date, and
// the row sum needs no exchange until the end.
#include <type_traits>

#include "kernels.h"
#include "mfma.h"

namespace vafa {

namespace {

constexpr int kBN = 64;  // keys per LDS tile
// LDS row padding (elements).  K is read by ds_read_b128 (rows as the A
// operand) and V only by ds_read_b64_tr_b16 (V^T operands); measured on
// gfx950 the two want different row strides: 16-byte row reads are
// conflict-free when the stride is 8 * odd elements (D + 24), the transposed
// reads when it is 32 mod 128 elements (D + 32).
constexpr int kKPad = 24;
constexpr int kVPad = 32;

template <int D>
struct FwdSmem {
  static constexpr int KSK = D + kKPad;          // K row stride (elements)
  static constexpr int KSV = D + kVPad;          // V row stride (elements)
  static constexpr int kKs = kBN * KSK;          // elements per K buffer
  static constexpr int kVs = kBN * KSV;          // elements per V buffer
  static constexpr int kBuf = kKs + kVs;         // K then V
  static constexpr int kBytes = 2 * kBuf * 2;    // double buffered, 2 B/elt
};

// Global -> register stage of one K/V tile over NT threads (zero-filled past
// k_end; at D=32 with 512 threads half of them have no chunk).
template <int D, int NT>
struct TileRegs {
  static constexpr int kTotal = kBN * D / 8;                // 16 B chunks per tensor
  static constexpr int kKChunks = (kTotal + NT - 1) / NT;   // per thread
  u32x4 kc[kKChunks];
  u32x4 vc[kKChunks];
};

template <typename T, int D, int NT>
__device__ __forceinline__ void load_tile(TileRegs<D, NT> &r, const T *__restrict__ k,
                                          const T *__restrict__ v, int kbase, int k_end, int H,
                                          int h, int tid) {
  using R = TileRegs<D, NT>;
  constexpr int CPR = D / 8;  // chunks per row
  // one buffer resource per tile: rows past k_end read as zero
  const int64_t row_bytes = (int64_t)H * D * 2;
  const int64_t nbytes = (int64_t)(k_end - kbase < kBN ? k_end - kbase : kBN) * row_bytes;
  const rsrc_t rk = make_rsrc(k + (int64_t)kbase * H * D, nbytes);
  const rsrc_t rv = make_rsrc(v + (int64_t)kbase * H * D, nbytes);
#pragma unroll
  for (int i = 0; i < R::kKChunks; ++i) {
    const int ci = tid + NT * i;
    const int key = ci < R::kTotal ? ci / CPR : kBN, dc = ci % CPR;  // kBN: past the range
    r.kc[i] = buf_load16(rk, (key * H + h) * D * 2 + dc * 16);
  }
#pragma unroll
  for (int i = 0; i < R::kKChunks; ++i) {
    const int ci = tid + NT * i;
    const int key = ci < R::kTotal ? ci / CPR : kBN, dc = ci % CPR;
    r.vc[i] = buf_load16(rv, (key * H + h) * D * 2 + dc * 16);
  }
}

template <typename T, int D, int NT>
__device__ __forceinline__ void store_tile(const TileRegs<D, NT> &r, T *ks, T *vs, int tid) {
  using R = TileRegs<D, NT>;
  constexpr int CPR = D / 8;
#pragma unroll
  for (int i = 0; i < R::kKChunks; ++i) {
    const int ci = tid + NT * i;
    if (R::kTotal % NT == 0 || ci < R::kTotal) {
      const int key = ci / CPR, dc = ci % CPR;
      *reinterpret_cast<u32x4 *>(ks + key * FwdSmem<D>::KSK + dc * 8) = r.kc[i];
      *reinterpret_cast<u32x4 *>(vs + key * FwdSmem<D>::KSV + dc * 8) = r.vc[i];
    }
  }
}

// acc + x[2t] + x[2t+1] on the dot2 unit (fp32 accumulate): the row sum of
// P as rounded for the PV product, half the instructions of fp32 adds.
template <typename T>
__device__ __forceinline__ float dot2_ones(const typename Mfma<T>::v8 &x, int t, float acc);
template <>
__device__ __forceinline__ float dot2_ones<bf16>(const bf16x8 &x, int t, float acc) {
  typedef __bf16 b2 __attribute__((ext_vector_type(2)));
  const b2 v = {x[2 * t], x[2 * t + 1]};
  return __builtin_amdgcn_fdot2_f32_bf16(v, __builtin_bit_cast(b2, 0x3f803f80u), acc, false);
}
template <>
__device__ __forceinline__ float dot2_ones<f16>(const f16x8 &x, int t, float acc) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const h2 v = {x[2 * t], x[2 * t + 1]};
  return __builtin_amdgcn_fdot2(v, __builtin_bit_cast(h2, 0x3c003c00u), acc, false);
}

// One 64-key tile for the wave's 32 query rows: S^T = K Q^T, online softmax
// (scores scaled by c > 0), O^T += V^T P^T.  Keys >= k_end are masked on
// the (wave-uniform) tail tile only.
template <typename T, int D>
__device__ __forceinline__ void fwd_tile(const T *ks, const T *vs,
                                         const typename Mfma<T>::v8 (&qf)[D / 16],
                                         f32x16 (&acc)[D / 32], float &m_run, float &l_part,
                                         float c, int kbase, int k_end, int lane) {
  using M = Mfma<T>;
  constexpr int NC = D / 16, ND = D / 32;
  constexpr int KS = FwdSmem<D>::KSK, VS = FwdSmem<D>::KSV;
  const int lrow = lane & 31, lhalf = lane >> 5;
  // S^T for the two 32-key halves as two interleaved MFMA chains; K operands
  // are read kPre steps ahead so LDS latency hides behind earlier MFMAs.
  constexpr int kPre = 4;
  constexpr int NS = 2 * NC;
  f32x16 s[2];
#pragma unroll
  for (int kt = 0; kt < 2; ++kt)
#pragma unroll
    for (int r = 0; r < 16; ++r) s[kt][r] = 0.f;
  const T *kbase_p = ks + lrow * KS + lhalf * 8;
  auto kop = [&](int i) {  // i = cc * 2 + kt
    return *reinterpret_cast<const u32x4 *>(kbase_p + (i & 1) * 32 * KS + (i >> 1) * 16);
  };
  u32x4 ring[kPre];
#pragma unroll
  for (int i = 0; i < kPre; ++i) ring[i] = kop(i);
  // sched_barrier(0) pins the written order: the scheduler would otherwise
  // pull each LDS read down next to its MFMA and expose its latency
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < NS; ++i) {
    const u32x4 a = ring[i % kPre];
    s[i & 1] = M::mma(as_v8<T>(a), qf[i >> 1], s[i & 1]);
    if (i + kPre < NS) ring[i % kPre] = kop(i + kPre);
    __builtin_amdgcn_sched_barrier(0);
  }
  if (kbase + kBN > k_end) {
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (kbase + kt * 32 + (r >> 2) * 8 + lhalf * 4 + (r & 3) >= k_end) s[kt][r] = kNegInf;
  }
  // P against the running max first; the lane's sum of P as rounded to T
  // (dot2 with (1, 1), four chains) both accumulates the row sum and checks
  // the bound.  Only a tile whose sum exceeds kLazyMax (some P above 2^8, or
  // the first tile, where m_run = -kHuge) takes the row max, rescales the
  // accumulators and rebuilds P.
  typename M::v8 pb[2][2];
  float ps4[4];
  auto build_p = [&]() {
#pragma unroll
    for (int i = 0; i < 4; ++i) ps4[i] = 0.f;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int mm = 0; mm < 2; ++mm) {
        typename M::v8 x;
#pragma unroll
        for (int t = 0; t < 8; ++t)
          x[t] = static_cast<T>(fast_exp2(__builtin_fmaf(s[kt][mm * 8 + t], c, -m_run)));
        pb[kt][mm] = x;
#pragma unroll
        for (int t = 0; t < 4; ++t) ps4[t] = dot2_ones<T>(x, t, ps4[t]);
      }
  };
  build_p();
  float ps = (ps4[0] + ps4[1]) + (ps4[2] + ps4[3]);
  if (wave_any(!(ps <= kLazyMax))) {
    float m4[4] = {kNegInf, kNegInf, kNegInf, kNegInf};
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) m4[r & 3] = fmaxf(m4[r & 3], s[kt][r]);
    float mx = fmaxf(fmaxf(m4[0], m4[1]), fmaxf(m4[2], m4[3]));
    mx = max_xor32(mx) * c;
    const float m_new = fmaxf(m_run, mx);
    const float alpha = fast_exp2(m_run - m_new);
    m_run = m_new;
    l_part *= alpha;
#pragma unroll
    for (int i = 0; i < ND; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][r] *= alpha;
    build_p();
    ps = (ps4[0] + ps4[1]) + (ps4[2] + ps4[3]);
  }
  l_part += ps;
  // O^T += V^T P^T: 4*ND MFMAs ordered so consecutive ones hit different
  // accumulators, V^T operands read kPre steps ahead.
  constexpr int NP = 4 * ND;
  auto vop = [&](int i) {  // i = km * ND + dt, km = kt * 2 + mm
    const int km = i / ND, dt = i % ND;
    return tr_operand<T>(vs, VS, km * 16, dt * 32, lane);
  };
  typename M::v8 vring[kPre];
#pragma unroll
  for (int i = 0; i < kPre; ++i) vring[i] = vop(i);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    const typename M::v8 a = vring[i % kPre];
    const int km = i / ND, dt = i % ND;
    acc[dt] = M::mma(a, pb[km >> 1][km & 1], acc[dt]);
    if (i + kPre < NP) vring[i % kPre] = vop(i + kPre);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// two waves per SIMD (one at D=256, whose registers take the whole file)
template <typename T, int D, int NW>
__global__ __launch_bounds__(64 * NW, D >= 256 ? 1 : 2) void varlen_fwd_kernel(
    const T *__restrict__ q, const T *__restrict__ k, const T *__restrict__ v,
    T *__restrict__ o, float *__restrict__ lse, float *__restrict__ part_o,
    float *__restrict__ part_lse, const int32_t *__restrict__ items, int H, float c,
    int n_items, int xcd_heads) {
  using M = Mfma<T>;
  constexpr int NC = D / 16;   // 16-wide d chunks (S^T reduction)
  constexpr int ND = D / 32;   // 32-row d tiles of O^T
  extern __shared__ __align__(16) unsigned char smem_raw[];
  T *smem = reinterpret_cast<T *>(smem_raw);

  // grid: item-major with heads innermost, or (xcd_heads) the H workgroups of
  // an item on one XCD -- workgroup b runs on XCD b % kXcds
  int item, h;
  if (xcd_heads) {
    const int grp = blockIdx.x / (kXcds * H), rr = blockIdx.x % (kXcds * H);
    item = grp * kXcds + rr % kXcds;
    h = rr / kXcds;
    if (item >= n_items) return;  // padding of the last group
  } else {
    item = blockIdx.x / H;
    h = blockIdx.x % H;
  }
  const PlanItem it = load_item(items, item);
  const int q0 = it.v[0], q1 = it.v[1], k0 = it.v[2], k1 = it.v[3], pbase = it.v[4];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int lrow = lane & 31, lhalf = lane >> 5;
  const int qrow = q0 + wave * 32 + lrow;
  const bool row_ok = qrow < q1;
  const bool wave_active = q0 + wave * 32 < q1;

  // Q^T fragments (B operand): rows past q1 are zero.  A negative softmax
  // scale is folded into Q (sign flips are exact) so c > 0 below.
  const uint32_t qsign = c < 0.f ? 0x80008000u : 0u;
  c = fabsf(c);
  typename M::v8 qf[NC];
  {
    const rsrc_t rq = make_rsrc(q + ((int64_t)q0 * H + h) * D, (int64_t)(q1 - q0) * H * D * 2);
    const int lr = wave * 32 + lrow;
#pragma unroll
    for (int cc = 0; cc < NC; ++cc) {
      u32x4 val = buf_load16(rq, (lr * H) * D * 2 + cc * 32 + lhalf * 16);
#pragma unroll
      for (int w = 0; w < 4; ++w) val[w] ^= qsign;
      qf[cc] = as_v8<T>(val);
    }
  }

  f32x16 acc[ND];
#pragma unroll
  for (int i = 0; i < ND; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[i][r] = 0.f;
  float m_run = -kHuge, l_part = 0.f;

  constexpr int NT = 64 * NW;
  const int nt = (k1 - k0 + kBN - 1) / kBN;
  TileRegs<D, NT> regs;
  if (nt > 0) {
    load_tile<T, D, NT>(regs, k, v, k0, k1, H, h, tid);
    store_tile<T, D, NT>(regs, smem, smem + FwdSmem<D>::kKs, tid);
  }
  __syncthreads();

  // Two tiles per trip, so each tile's LDS buffer is a compile-time offset
  // that folds into the LDS instructions' immediates (a run-time (j & 1)
  // select cost address adds on every tile).
  auto step = [&](int j, auto buf) {
    constexpr int B = decltype(buf)::value;
    const int kbase = k0 + j * kBN;
    if (j + 1 < nt) load_tile<T, D, NT>(regs, k, v, kbase + kBN, k1, H, h, tid);
    const T *ks = smem + B * FwdSmem<D>::kBuf;
    const T *vs = ks + FwdSmem<D>::kKs;
    if (wave_active) fwd_tile<T, D>(ks, vs, qf, acc, m_run, l_part, c, kbase, k1, lane);
    if (j + 1 < nt) {
      T *nks = smem + (1 - B) * FwdSmem<D>::kBuf;
      store_tile<T, D, NT>(regs, nks, nks + FwdSmem<D>::kKs, tid);
    }
    __syncthreads();
  };
  for (int j = 0; j < nt; j += 2) {
    step(j, std::integral_constant<int, 0>{});
    if (j + 1 < nt) step(j + 1, std::integral_constant<int, 1>{});
  }

  if (!wave_active) return;
  const float l = l_part + __shfl_xor(l_part, 32, 64);
  const float inv = l > 0.f ? 1.f / l : 0.f;
  const float lse_v = l > 0.f ? m_run + fast_log2(l) : kNegInf;
  // O (or a split's fp32 partial rows) leaves as whole rows through the
  // wave's LDS region (the K/V buffers: every wave has passed the loop's last
  // barrier).  Stored from the accumulators, every instruction wrote 8 or 16
  // bytes into each of 32 rows, 8% of the C2 forward.
  using RS = RowStore<T, ND>;
  unsigned char *stage = smem_raw + wave * RS::kBytes;
  const int rows = uniform_clamp(q1 - (q0 + wave * 32), 32);
  if (pbase < 0) {
    RS::rows16(acc, [&](float x) { return static_cast<T>(x * inv); }, stage,
               o + ((int64_t)(q0 + wave * 32) * H + h) * D, (int64_t)H * D, rows);
    if (row_ok && lhalf == 0) lse[(int64_t)qrow * H + h] = lse_v;
  } else {
    const int64_t prow = pbase + wave * 32;
    RS::rows32(acc, inv, stage, part_o + (prow * H + h) * D, (int64_t)H * D, rows);
    if (row_ok && lhalf == 0) part_lse[(prow + lrow) * H + h] = lse_v;
  }
}

}  // namespace

// Dynamic LDS of the forward: the K/V buffers, or the per-wave row-store
// regions of the epilogue if those are larger.
template <typename T, int D, int NW>
constexpr int fwd_lds_bytes() {
  constexpr int kStage = NW * RowStore<T, D / 32>::kBytes;
  return FwdSmem<D>::kBytes > kStage ? FwdSmem<D>::kBytes : kStage;
}

template <typename T, int D, int NW>
void launch_fwd_nw(const VarlenArgs &a, hipStream_t st) {
  const int smem = fwd_lds_bytes<T, D, NW>();
  allow_dynamic_lds(reinterpret_cast<const void *>(&varlen_fwd_kernel<T, D, NW>), smem);
  const int64_t n_wg = a.xcd_heads ? (a.n_items + kXcds - 1) / kXcds * kXcds * a.H
                                   : a.n_items * a.H;
  hipLaunchKernelGGL((varlen_fwd_kernel<T, D, NW>), dim3((unsigned)n_wg), dim3(64 * NW), smem,
                     st, (const T *)a.q, (const T *)a.k, (const T *)a.v, (T *)a.o, a.lse,
                     a.part_o, a.part_lse, a.items, a.H, a.scale * kLog2e, (int)a.n_items,
                     a.xcd_heads);
}

// The plan's query tile sets the workgroup: 32 rows per wave.
template <typename T, int D>
void launch_mfma_varlen_fwd(const VarlenArgs &a, hipStream_t st) {
  if (a.n_items == 0) return;
  if constexpr (D <= 128) {
    if (a.q_tile == kVarlenWideTile) return launch_fwd_nw<T, D, 8>(a, st);
  }
  launch_fwd_nw<T, D, 4>(a, st);
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
