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
//     chunk, walked in 128-key sub-tiles with X held in registers (the next
//     sub-tile's rows load while the current one finishes), against the
//     sample's rows in blocks of 32 staged row-major in LDS by DMA (kept
//     resident when the sample has at most 64 rows):
//       S = U X^T, dP = dAX X^T,  dX^T += U^T (scale dS) + dAX^T P
//     summed over heads in registers (no partial buffers, no atomics).
// dAX = dO W_V^T arrives in the input dtype: the reference rounds it to that
// dtype before every product it feeds (ta/kernels.py:480, 617-626).
#include "absorb_tiles.h"

namespace vafa {

namespace {

using namespace absorb;

constexpr int kDuWaves = 4;  // 4 waves x 16 rows = one forward row tile

// Above 256 features (FP = 512) the du / aX accumulators of all 32 f tiles
// and the U^T / dAX^T operands would take 384 registers: there two
// workgroups share a token tile, each forming S and dP over every feature
// and accumulating du / aX for one half of the f tiles (NS = 2 slices).
// Grid of NS = 2: blocks b and b + 8 of each 16 are the two halves of one
// tile and run on one XCD, whose L2 serves the second stream of the tile's
// X.  One workgroup per CU at FP = 512, two below.
template <int FP>
struct DuSlices {
  static constexpr int NS = FP > kMaxF ? 2 : 1;
};

template <typename T, int FP>
__global__ __launch_bounds__(64 * kDuWaves, FP > kMaxF ? 1 : 2) void absorb_du_kernel(
    const T *__restrict__ u, const T *__restrict__ X, const T *__restrict__ dax,
    const float *__restrict__ lse, const float *__restrict__ delta, T *__restrict__ du,
    float *__restrict__ ax, const int32_t *__restrict__ items, int n_items, int H, int F,
    float c, float scale) {
  using M16 = Mfma16<T>;
  using v8 = typename Mfma<T>::v8;
  using S = AbsSmem<FP>;
  constexpr int NS = DuSlices<FP>::NS;
  constexpr int NK = FP / 32;        // 32-wide reduction chunks of S^T / dP^T
  constexpr int NF = FP / 16 / NS;   // 16-row f tiles of aX^T / du^T in this slice
  constexpr int kPerWave = kBK / kDuWaves;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  T *smem = reinterpret_cast<T *>(smem_raw);

  int item = blockIdx.x, ft0 = 0;  // first f tile of this workgroup's slice
  if constexpr (NS == 2) {
    const int b = blockIdx.x;
    item = (b / 16) * 8 + b % 8;
    ft0 = ((b / 8) & 1) * NF;
    if (item >= n_items) return;  // padding of the last group of 16
  }
  const PlanItem it = load_item(items, item);
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
    const int rows = uniform_clamp(k1 - kb, kBK);
    dma_block<FP, kDuWaves, S::XS>(X + (int64_t)kb * F, (uint32_t)(rows * F * 2), F,
                            lds_addr(smem + buf * S::kTile), wave, lane);
  };
  // only tiles of the key range are fetched (a tile past it would land as
  // zeros and cost a tile's DMA instructions)
#pragma unroll
  for (int b = 0; b < kNBuf - 1; ++b)
    if (b < nt) issue(k0 + b * kBK, b);

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

  // per-lane element offsets into a tile: X row l16 at f = 8*lq (A operand
  // of S^T / dP^T) and the origin of the transposed reads (below)
  const int a_off = l16 * S::XS + lq * 8;
  const int t_off = (4 * lq + (l16 >> 2)) * S::XS + 4 * (l16 & 3);
  constexpr int kPre = 4;
  constexpr int NA = 2 * NK;  // A reads of S^T / dP^T per tile
  int buf = 0;                // j % kNBuf
  for (int j = 0; j < nt; ++j) {
    // tile j landed (tile j+1, if there is one, may still be in flight)
    static_assert(kNBuf == 3, "one tile in flight behind the current one");
    if (j + 1 < nt)
      wait_vmcnt<(kNBuf - 2) * kPerWave>();
    else
      wait_vmcnt<0>();
    __syncthreads();
    if (j + kNBuf - 1 < nt) issue(k0 + (j + kNBuf - 1) * kBK, buf == 0 ? kNBuf - 1 : buf - 1);
    const int kb = k0 + j * kBK;
    if (wave_active) {
      const lds_cptr<T> xa = as_lds(smem + buf * S::kTile + a_off);
      const lds_cptr<T> xt = as_lds(smem + buf * S::kTile + t_off);
      // S^T, dP^T: two 16-key halves; element r of half mt is key
      // kb + 16*mt + 4*lq + r of this lane's row.  A read i covers half i / NK
      // and f chunk i % NK; reads run kPre ahead of their products, pinned by
      // sched_barrier so the scheduler does not sink them next to their use.
      auto aop = [&](int i) { return lds_ld16<T>(xa + (i / NK) * 16 * S::XS + (i % NK) * 32); };
      f32x4 s[2], dp[2];
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) s[mt][r] = dp[mt][r] = 0.f;
      u32x4 ring[kPre];
#pragma unroll
      for (int i = 0; i < kPre; ++i) ring[i] = aop(i);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < NA; ++i) {
        const v8 a = as_v8<T>(ring[i % kPre]);
        s[i / NK] = M16::mma(a, uf[i % NK], s[i / NK]);
        dp[i / NK] = M16::mma(a, gf[i % NK], dp[i / NK]);
        if (i + kPre < NA) ring[i % kPre] = aop(i + kPre);
        __builtin_amdgcn_sched_barrier(0);
      }
      // A operand of aX^T / du^T for f tile ft, X^T out of the row-major tile:
      // lane l gets column 16*ft + l%16 at the keys of its k slots 8*lq + t,
      // key 4*lq + t (t < 4) and 16 + 4*lq + t - 4 (t >= 4), from two
      // ds_read_b64_tr_b16.  The first kPre overlap the softmax arithmetic.
      auto top = [&](int ft) {
        return as_v8<T>(join(lds_tr8<T>(xt + ft * 16), lds_tr8<T>(xt + 16 * S::XS + ft * 16)));
      };
      v8 tring[kPre];
#pragma unroll
      for (int i = 0; i < kPre; ++i) tring[i] = top(ft0 + i);
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
      // B operands over the tile's keys in the same slot order
      v8 pb, sb;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        pb[r] = static_cast<T>(s[0][r]);
        pb[4 + r] = static_cast<T>(s[1][r]);
        sb[r] = static_cast<T>(dp[0][r]);
        sb[4 + r] = static_cast<T>(dp[1][r]);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int ft = 0; ft < NF; ++ft) {
        const v8 a = tring[ft % kPre];
        aax[ft] = M16::mma(a, pb, aax[ft]);
        adu[ft] = M16::mma(a, sb, adu[ft]);
        if (ft + kPre < NF) tring[ft % kPre] = top(ft0 + ft + kPre);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    buf = buf == kNBuf - 1 ? 0 : buf + 1;
  }
  wait_vmcnt<0>();

  if (!row_ok) return;
  typedef __attribute__((__vector_size__(4 * sizeof(T)))) T T4;
  const int64_t ro = ((int64_t)t0 * H + row) * F;
#pragma unroll
  for (int ft = 0; ft < NF; ++ft) {
    const int f = (ft0 + ft) * 16 + lq * 4;  // element r is f + r of this lane's row
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
  static constexpr int XS = AbsSmem<FP, kXPad32>::XS;  // 32-row operand reads
  static constexpr int kBlk = 32 * XS;                    // one [32][XS] row block
  static constexpr int kBufBytes = 2 * kBlk * 2 + 2 * 32 * 4;  // U, dAX, LSE, delta
  static constexpr int kBytes = 2 * kBufBytes;
};

// Shared pieces of the two dX kernels, for one workgroup's item.
template <typename T, int FP>
struct DxItem {
  using T_ = T;
  using M = Mfma<T>;
  using S = DxSmem<FP>;
  static constexpr int NC = FP / 16;
  static constexpr int NF = FP / 32;
  static constexpr int XS = S::XS;
  static constexpr int kSub = 32 * kDxWaves;  // keys per sub-tile (32 per wave)

  const T *u, *X, *dax;
  const float *lse, *delta;
  unsigned char *smem;
  int k0, k1, r0, r1, F, wave, lane, lrow, lhalf, a_off, t_off;

  __device__ DxItem(const T *u_, const T *X_, const T *dax_, const float *lse_,
                    const float *delta_, unsigned char *smem_, const PlanItem &it, int H, int F_)
      : u(u_), X(X_), dax(dax_), lse(lse_), delta(delta_), smem(smem_), F(F_) {
    k0 = it.v[0];
    k1 = it.v[1];
    r0 = it.v[2] * H;
    r1 = it.v[3] * H;
    lane = threadIdx.x & 63;
    wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    lrow = lane & 31;
    lhalf = lane >> 5;
    // row lrow at f = 8*lhalf (A of S and dP) and the origin of the
    // transposed reads (layout of tr_operand)
    a_off = lrow * XS + lhalf * 8;
    t_off = (4 * (lane >> 5) + ((lane & 15) >> 2)) * XS + ((lane >> 4) & 1) * 16 + 4 * (lane & 3);
  }
  __device__ int nblk() const { return (r1 - r0 + 31) / 32; }
  __device__ int nsub() const { return (k1 - k0 + kSub - 1) / kSub; }

  // stage 32-row block blk of U, dAX, LSE and delta into buffer buf (rows past
  // r1 are zero, so they add nothing to dX: both products carry a zero U or
  // dAX row).  Waves 0/2 move LSE and waves 1/3 delta (the pairs write
  // identical bytes): one 128-byte DMA per wave keeps vmcnt counts equal.
  __device__ void issue(int blk, int buf) const {
    unsigned char *base = smem + buf * S::kBufBytes;
    const int rb = r0 + blk * 32;
    const int rows = uniform_clamp(r1 - rb, 32);
    const uint32_t nb = (uint32_t)(rows * F * 2);
    dma_block<FP, kDxWaves, XS>(u + (int64_t)rb * F, nb, F, lds_addr(base), wave, lane);
    dma_block<FP, kDxWaves, XS>(dax + (int64_t)rb * F, nb, F, lds_addr(base + S::kBlk * 2), wave,
                            lane);
    const float *vec = (wave & 1) ? delta : lse;
    const u32x4 rv = rsrc_words32(vec + rb, (uint32_t)(rows * 4));
    if (lane < 8) lds_dma16(rv, lds_addr(base + 2 * S::kBlk * 2 + (wave & 1) * 128), lane * 16);
  }

  // X rows of this wave's 32 keys of sub-tile st: B operand of S = U X^T and
  // dP = dAX X^T; keys past k1 read as zero.  Waited for at first use.
  __device__ void load_x(typename M::v8 (&xf)[NC], int st) const {
    const int kb = k0 + st * kSub;
    const rsrc_t rx = make_rsrc(X + (int64_t)kb * F, (int64_t)(k1 - kb) * F * 2);
    const int fchunks = F / 8;
#pragma unroll
    for (int cc = 0; cc < NC; ++cc) {
      const int ch = cc * 2 + lhalf;
      xf[cc] = as_v8<T>(
          buf_load16(rx, ch < fchunks ? (wave * 32 + lrow) * F * 2 + ch * 16 : 0x7fffffff));
    }
  }

  // P and scale*dS of one staged row block against this wave's keys, packed
  // as B operands over the block's rows (relabelled C layout: element r of
  // the S / dP accumulators is row (r/4)*8 + lhalf*4 + r%4, this lane's key)
  template <int kPre>
  __device__ void block_p_ds(const typename M::v8 (&xf)[NC], int buf, float c, float scale,
                             typename M::v8 (&pb)[2], typename M::v8 (&sb)[2]) const {
    const unsigned char *base = smem + buf * S::kBufBytes;
    const lds_cptr<T> ub = as_lds(reinterpret_cast<const T *>(base));
    const lds_cptr<T> gb = ub + S::kBlk;
    const float *ls = reinterpret_cast<const float *>(base + 2 * S::kBlk * 2);
    // read i is chunk i/2 of the U (even i) or dAX (odd i) row; reads run
    // kPre ahead of their products (pinned by sched_barrier)
    auto aop = [&](int i) { return lds_ld16<T>(((i & 1) ? gb : ub) + a_off + (i >> 1) * 16); };
    f32x16 s, dp;
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = dp[r] = 0.f;
    u32x4 ring[kPre];
#pragma unroll
    for (int i = 0; i < kPre; ++i) ring[i] = aop(i);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < 2 * NC; ++i) {
      const typename M::v8 a = as_v8<T>(ring[i % kPre]);
      if (i & 1)
        dp = M::mma(a, xf[i >> 1], dp);
      else
        s = M::mma(a, xf[i >> 1], s);
      if (i + kPre < 2 * NC) ring[i % kPre] = aop(i + kPre);
      __builtin_amdgcn_sched_barrier(0);
    }
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
#pragma unroll
    for (int mm = 0; mm < 2; ++mm) {
      pb[mm] = pack8<T>(s, mm * 8);
      sb[mm] = pack8<T>(dp, mm * 8);
    }
  }

  // transposed A operand of dX^T from a staged block: f tile ft, row half mm,
  // U (which = 1) or dAX (which = 0)
  __device__ typename M::v8 top(int buf, int which, int mm, int ft) const {
    const lds_cptr<T> ub = as_lds(reinterpret_cast<const T *>(smem + buf * S::kBufBytes));
    const lds_cptr<T> q = (which ? ub : ub + S::kBlk) + t_off + mm * 16 * XS + ft * 32;
    return as_v8<T>(join(lds_tr8<T>(q), lds_tr8<T>(q + 8 * XS)));
  }

  // dX[key, f] for f tiles [f0t, f0t + N) of this wave's keys of the sub-tile
  // at kb, from accumulators with lanes along f: element r of tile i is key
  // kb + 32*wave + (r/4)*8 + lhalf*4 + r%4 at f = (f0t + i)*32 + lrow
  // Buffer stores: keys past k1 fall outside the descriptor and are dropped.
  // Each offset is one add of a scalar row term, written as volatile asm so
  // the compiler does not hoist all 16*N offsets into registers.
  template <int N>
  __device__ void store_rows(T *dX, int kb, int f0t, const f32x16 (&acc)[N]) const {
    const rsrc_t rs = make_rsrc(dX + (int64_t)kb * F, (int64_t)(k1 - kb) * F * 2);
    const int lane_off = ((wave * 32 + lhalf * 4) * F + lrow) * 2;
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int f = (f0t + i) * 32 + lrow;
      if (f >= F) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row_term = (((r >> 2) * 8 + (r & 3)) * F + (f0t + i) * 32) * 2;
        int off;
        asm volatile("v_add_u32 %0, %1, %2" : "=v"(off) : "s"(row_term), "v"(lane_off));
        __builtin_amdgcn_raw_buffer_store_b16(
            __builtin_bit_cast(unsigned short, static_cast<T>(acc[i][r])), rs, off, 0, 0);
      }
    }
  }

  // dX[key, f] for f tiles [f0t, f0t + n) from this lane's accumulators
  template <int N>
  __device__ void store(T *dX, int key, int f0t, const f32x16 (&acc)[N]) const {
    typedef __attribute__((__vector_size__(4 * sizeof(T)))) T T4;
    T *dst = dX + (int64_t)key * F;
#pragma unroll
    for (int i = 0; i < N; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int f = (f0t + i) * 32 + g * 8 + lhalf * 4;
        if (f >= F) continue;
        T4 w;
#pragma unroll
        for (int e = 0; e < 4; ++e) w[e] = static_cast<T>(acc[i][g * 4 + e]);
        *reinterpret_cast<T4 *>(dst + f) = w;
      }
  }
};

// dX over NB resident row blocks, in two f halves of (NF+1)/2 tiles each:
// dX[key, f] += P^T[key, row] dAX[row, f] + (scale dS)^T[key, row] U[row, f]
// with the packed P / scale*dS as A (their relabelled row order serves as the
// reduction index) and U / dAX columns from transposed reads as B.  The
// result has lanes along f, so each store writes 64 contiguous bytes of a
// key row.
template <int NB, typename D>
__device__ __forceinline__ void dx_halves(const D &d, typename D::T_ *dX, int kb,
                                          const typename D::M::v8 (&pb)[2][2],
                                          const typename D::M::v8 (&sb)[2][2]) {
  using v8 = typename D::M::v8;
  constexpr int NF = D::NF, NH = (NF + 1) / 2, kPre = 4;
  constexpr int NO = 4 * NB * NH;  // (block, which, mm) x f tiles of a half
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    f32x16 acc[NH];
#pragma unroll
    for (int i = 0; i < NH; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][r] = 0.f;
    // operand i: f tile h*NH + i % NH (clamped; products past NF are
    // skipped), block / which / mm from q = i / NH
    auto op = [&](int i) {
      const int q = i / NH, ft = h * NH + i % NH;
      return d.top(q >> 2, q & 1, (q >> 1) & 1, ft < NF ? ft : NF - 1);
    };
    v8 tring[kPre];
#pragma unroll
    for (int i = 0; i < kPre; ++i) tring[i] = op(i);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < NO; ++i) {
      const int q = i / NH, ft = h * NH + i % NH;
      const v8 a = tring[i % kPre];
      if (ft < NF) {
        const v8 aop = (q & 1) ? sb[q >> 2][(q >> 1) & 1] : pb[q >> 2][(q >> 1) & 1];
        acc[i % NH] = D::M::mma(aop, a, acc[i % NH]);
      }
      if (i + kPre < NO) tring[i % kPre] = op(i + kPre);
      __builtin_amdgcn_sched_barrier(0);
    }
    d.store_rows(dX, kb, h * NH, acc);
  }
}

// Items whose sample has at most 64 rows: both row blocks stay resident for
// the whole key chunk.  Per 128-key sub-tile each wave forms P and scale*dS
// for both blocks first (X operands then dead, so the next sub-tile's X loads
// right away), then accumulates dX^T in two f halves of 64 registers.
template <typename T, int FP>
__global__ __launch_bounds__(64 * kDxWaves, FP > kMaxF ? 1 : 2) void absorb_dx_res_kernel(
    const T *__restrict__ u, const T *__restrict__ X, const T *__restrict__ dax,
    const float *__restrict__ lse, const float *__restrict__ delta, T *__restrict__ dX,
    const int32_t *__restrict__ items, int H, int F, float c, float scale) {
  using D = DxItem<T, FP>;
  using v8 = typename D::M::v8;
  constexpr int kPre = 4;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const D d(u, X, dax, lse, delta, smem_raw, load_item(items, blockIdx.x), H, F);
  const int nblk = d.nblk();
  if (nblk * 32 > kDxResidentRows) return;  // streamed by absorb_dx_kernel
  const int nsub = d.nsub();
  if (nblk == 0) {
    // a sample without queries: its keys get zero gradient
    f32x16 zero[D::NF];
#pragma unroll
    for (int i = 0; i < D::NF; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) zero[i][r] = 0.f;
    for (int st = 0; st < nsub; ++st) {
      const int key = d.k0 + st * D::kSub + d.wave * 32 + d.lrow;
      if (key < d.k1) d.store(dX, key, 0, zero);
    }
    return;
  }
  for (int b = 0; b < nblk; ++b) d.issue(b, b);
  v8 xf[D::NC];
  d.load_x(xf, 0);
  wait_vmcnt<0>();
  __syncthreads();
  for (int st = 0; st < nsub; ++st) {
    const int kb = d.k0 + st * D::kSub;
    if (kb + d.wave * 32 >= d.k1) break;  // wave-uniform: no keys left for this wave
    v8 pb[2][2], sb[2][2];
    d.template block_p_ds<kPre>(xf, 0, c, scale, pb[0], sb[0]);
    if (nblk > 1) d.template block_p_ds<kPre>(xf, 1, c, scale, pb[1], sb[1]);
    __builtin_amdgcn_sched_barrier(0);
    if (st + 1 < nsub) d.load_x(xf, st + 1);
    __builtin_amdgcn_sched_barrier(0);
    if (nblk > 1)
      dx_halves<2>(d, dX, kb, pb, sb);
    else
      dx_halves<1>(d, dX, kb, pb, sb);
  }
  wait_vmcnt<0>();
}

// Items whose sample has more than 64 rows: per 128-key sub-tile the row
// blocks stream through two buffers and dX^T accumulates over all of them.
// At FP = 512 the accumulators of all 16 f tiles would take 256 registers:
// two workgroups share an item (blocks b and b + 8 of each 16, on one XCD),
// each forming S and dP over every feature and accumulating one half of the
// f tiles (the du kernel's slicing).
template <typename T, int FP>
__global__ __launch_bounds__(64 * kDxWaves, FP > kMaxF ? 1 : 2) void absorb_dx_kernel(
    const T *__restrict__ u, const T *__restrict__ X, const T *__restrict__ dax,
    const float *__restrict__ lse, const float *__restrict__ delta, T *__restrict__ dX,
    const int32_t *__restrict__ items, int n_items, int H, int F, float c, float scale) {
  using D = DxItem<T, FP>;
  using v8 = typename D::M::v8;
  constexpr int NS = DuSlices<FP>::NS;
  constexpr int NF = D::NF / NS;  // 32-wide f tiles of this workgroup's slice
  constexpr int kPre = FP >= 224 ? 1 : 4;  // operand prefetch depth within the register budget
  extern __shared__ __align__(16) unsigned char smem_raw[];
  int item = blockIdx.x, ft0 = 0;
  if constexpr (NS == 2) {
    const int b = blockIdx.x;
    item = (b / 16) * 8 + b % 8;
    ft0 = ((b / 8) & 1) * NF;
    if (item >= n_items) return;  // padding of the last group of 16
  }
  const D d(u, X, dax, lse, delta, smem_raw, load_item(items, item), H, F);
  const int nblk = d.nblk();
  if (nblk * 32 <= kDxResidentRows) return;  // resident items: absorb_dx_res_kernel
  const int nsub = d.nsub();
  v8 xf[D::NC];
  d.issue(0, 0);
  int jb = 0;  // streamed blocks consumed so far (buffer parity)
  for (int st = 0; st < nsub; ++st) {
    const int kb = d.k0 + st * D::kSub;
    const int key = kb + d.wave * 32 + d.lrow;
    const bool wave_active = kb + d.wave * 32 < d.k1;
    d.load_x(xf, st);
    f32x16 acc[NF];
#pragma unroll
    for (int i = 0; i < NF; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][r] = 0.f;
    for (int j = 0; j < nblk; ++j) {
      wait_vmcnt<0>();
      __syncthreads();  // block visible; every wave is done with the other buffer
      const int buf = jb & 1;
      // next streamed block: this sub-tile's j+1, or block 0 of the next one
      if (j + 1 < nblk)
        d.issue(j + 1, buf ^ 1);
      else if (st + 1 < nsub)
        d.issue(0, buf ^ 1);
      ++jb;
      if (!wave_active) continue;
      v8 pb[2], sb[2];
      d.template block_p_ds<kPre>(xf, buf, c, scale, pb, sb);
      v8 tring[kPre];
      auto op = [&](int i) { return d.top(buf, (i / NF) & 1, (i / NF) >> 1, ft0 + i % NF); };
#pragma unroll
      for (int i = 0; i < kPre; ++i) tring[i] = op(i);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < 4 * NF; ++i) {
        const int ft = i % NF, mm = (i / NF) >> 1;
        const v8 a = tring[i % kPre];
        acc[ft] = D::M::mma(a, ((i / NF) & 1) ? sb[mm] : pb[mm], acc[ft]);
        if (i + kPre < 4 * NF) tring[i % kPre] = op(i + kPre);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    if (wave_active && key < d.k1) d.store(dX, key, ft0, acc);
  }
  wait_vmcnt<0>();
}

// dAX[t,h,f] = sum_d dO[t,h,d] W_V[f,h,d] (ta/kernels.py:474-476), rounded to
// the input dtype.  One wave per (32 tokens, head, kDaxTiles f tiles): dAX =
// dO W_V^T with dO rows as A (32 tokens x 16 d) and W_V rows as B (16 d x 32 f).
// 32-wide f tiles per wave: 2 gives 4x the waves of one wave per full row
// (14.7 against 17.8 us for 8 tiles on a 9424-token launch)
constexpr int kDaxTiles = 2;

template <typename T, int DH>
__global__ __launch_bounds__(64) void absorb_dax_kernel(const T *__restrict__ dO,
                                                        const T *__restrict__ wv,
                                                        T *__restrict__ dax, int64_t T_q, int H,
                                                        int F, const T *__restrict__ O,
                                                        float *__restrict__ delta) {
  using M = Mfma<T>;
  constexpr int KC = DH / 16;
  const int lane = threadIdx.x, l32 = lane & 31, lh = lane >> 5;
  const int nft = (F + 31) / 32, nfg = (nft + kDaxTiles - 1) / kDaxTiles;
  const int fg = (int)(blockIdx.x % nfg);
  const int h = (int)((blockIdx.x / nfg) % H);
  const int64_t t0 = (int64_t)(blockIdx.x / nfg / H) * 32;
  const int nt = T_q - t0 < 32 ? (int)(T_q - t0) : 32;
  // tokens past T_q and W_V rows past F read as zero
  const rsrc_t rd = make_rsrc(dO + t0 * H * DH, (int64_t)nt * H * DH * 2);
  const rsrc_t rw = make_rsrc(wv, (int64_t)F * H * DH * 2);
  typename M::v8 a[KC];
#pragma unroll
  for (int kc = 0; kc < KC; ++kc)
    a[kc] = as_v8<T>(buf_load16(rd, ((l32 * H + h) * DH + kc * 16 + lh * 8) * 2));
  if (fg == 0) {
    // delta[t,h] = sum_d dO[t,h,d] O[t,h,d] (ta/kernels.py:298-325) from the
    // dO rows already in registers; each half-wave holds half of every row
    const rsrc_t ro = make_rsrc(O + t0 * H * DH, (int64_t)nt * H * DH * 2);
    float sd = 0.f;
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) {
      const typename M::v8 ov =
          as_v8<T>(buf_load16(ro, ((l32 * H + h) * DH + kc * 16 + lh * 8) * 2));
#pragma unroll
      for (int e = 0; e < 8; ++e) sd = __builtin_fmaf(to_f(a[kc][e]), to_f(ov[e]), sd);
    }
    sd += __shfl_xor(sd, 32, 64);
    if (lane < 32 && l32 < nt) delta[(t0 + l32) * H + h] = sd;
  }
  // the wave's [32 tokens, kDaxTiles*32 f] block is staged in LDS, then
  // written as contiguous row runs (16 bytes per lane when F % 8 == 0)
  constexpr int kW = kDaxTiles * 32;
  __shared__ __align__(16) T st[32][kW + 8];
  const int fbase = fg * kW, fw = F - fbase < kW ? F - fbase : kW;
  const int ft_end = (fg + 1) * kDaxTiles < nft ? (fg + 1) * kDaxTiles : nft;
  for (int ft = fg * kDaxTiles; ft < ft_end; ++ft) {
    f32x16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.f;
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) {
      const u32x4 b = buf_load16(rw, (((ft * 32 + l32) * H + h) * DH + kc * 16 + lh * 8) * 2);
      acc = M::mma(a[kc], as_v8<T>(b), acc);
    }
    // element r: token (r/4)*8 + lh*4 + r%4, f = ft*32 + l32
    const int fl = ft * 32 - fbase + l32;
#pragma unroll
    for (int r = 0; r < 16; ++r) st[(r >> 2) * 8 + lh * 4 + (r & 3)][fl] = static_cast<T>(acc[r]);
  }
  __syncthreads();
  T *out = dax + (t0 * H + h) * (int64_t)F + fbase;
  if (F % 8 == 0) {
    constexpr int kLanesPerRow = kW / 8, kRowsPerPass = 64 / kLanesPerRow;
    const int rr = lane / kLanesPerRow, cc = (lane % kLanesPerRow) * 8;
    if (cc < fw)
      for (int tk = rr; tk < nt; tk += kRowsPerPass)
        *reinterpret_cast<u32x4 *>(out + (int64_t)tk * H * F + cc) =
            *reinterpret_cast<const u32x4 *>(&st[tk][cc]);
  } else {
    for (int i = lane; i < nt * fw; i += 64) out[(int64_t)(i / fw) * H * F + i % fw] = st[i / fw][i % fw];
  }
}

template <typename T, int FP>
void launch_du_fp(const AbsorbArgs &a, hipStream_t st) {
  const int smem = kNBuf * AbsSmem<FP>::kTile * 2;  // the du ring is 3 deep at every FP
  allow_dynamic_lds(reinterpret_cast<const void *>(&absorb_du_kernel<T, FP>), smem);
  const int64_t grid = DuSlices<FP>::NS == 2 ? (a.n_qseg + 7) / 8 * 16 : a.n_qseg;
  hipLaunchKernelGGL((absorb_du_kernel<T, FP>), dim3((unsigned)grid), dim3(64 * kDuWaves), smem,
                     st, (const T *)a.u, (const T *)a.X, (const T *)a.dax, a.lse_in, a.delta,
                     (T *)a.du, a.ax, a.qseg_items, (int)a.n_qseg, a.H, a.F, a.scale * kLog2e,
                     a.scale);
}

template <typename T, int FP>
void launch_dx_fp(const AbsorbArgs &a, hipStream_t st) {
  const int smem = DxSmem<FP>::kBytes;
  // the plan puts the resident-row items first (items are 8 int32 each): each
  // kernel gets its own run of the key-chunk section and still skips any item
  // of the other kind
  const int64_t n_res = a.n_kv_res, n_str = a.n_kv - a.n_kv_res;
  if (n_res > 0) {
    allow_dynamic_lds(reinterpret_cast<const void *>(&absorb_dx_res_kernel<T, FP>), smem);
    hipLaunchKernelGGL((absorb_dx_res_kernel<T, FP>), dim3((unsigned)n_res), dim3(64 * kDxWaves),
                       smem, st, (const T *)a.u, (const T *)a.X, (const T *)a.dax, a.lse_in,
                       a.delta, (T *)a.dX, a.kv_items, a.H, a.F, a.scale * kLog2e, a.scale);
  }
  if (n_str > 0) {
    allow_dynamic_lds(reinterpret_cast<const void *>(&absorb_dx_kernel<T, FP>), smem);
    const int64_t grid = DuSlices<FP>::NS == 2 ? (n_str + 7) / 8 * 16 : n_str;
    hipLaunchKernelGGL((absorb_dx_kernel<T, FP>), dim3((unsigned)grid), dim3(64 * kDxWaves),
                       smem, st, (const T *)a.u, (const T *)a.X, (const T *)a.dax, a.lse_in,
                       a.delta, (T *)a.dX, a.kv_items + n_res * 8, (int)n_str, a.H, a.F,
                       a.scale * kLog2e, a.scale);
  }
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
    case 512: launch_du_fp<T, 512>(a, st); break;
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
    case 512: launch_dx_fp<T, 512>(a, st); break;
    default: break;
  }
}

template <typename T>
bool launch_mfma_absorb_dax(const AbsorbArgs &a, hipStream_t st) {
  if (a.T_q == 0) return true;
  const unsigned grid =
      (unsigned)(((a.T_q + 31) / 32) * a.H * ((((a.F + 31) / 32) + kDaxTiles - 1) / kDaxTiles));
  switch (a.DH) {
    case 16: hipLaunchKernelGGL((absorb_dax_kernel<T, 16>), dim3(grid), dim3(64), 0, st, (const T *)a.dO, (const T *)a.wv, (T *)a.dax, a.T_q, a.H, a.F, (const T *)a.O_in, a.delta); return true;
    case 32: hipLaunchKernelGGL((absorb_dax_kernel<T, 32>), dim3(grid), dim3(64), 0, st, (const T *)a.dO, (const T *)a.wv, (T *)a.dax, a.T_q, a.H, a.F, (const T *)a.O_in, a.delta); return true;
    case 64: hipLaunchKernelGGL((absorb_dax_kernel<T, 64>), dim3(grid), dim3(64), 0, st, (const T *)a.dO, (const T *)a.wv, (T *)a.dax, a.T_q, a.H, a.F, (const T *)a.O_in, a.delta); return true;
    case 128: hipLaunchKernelGGL((absorb_dax_kernel<T, 128>), dim3(grid), dim3(64), 0, st, (const T *)a.dO, (const T *)a.wv, (T *)a.dax, a.T_q, a.H, a.F, (const T *)a.O_in, a.delta); return true;
    case 256: hipLaunchKernelGGL((absorb_dax_kernel<T, 256>), dim3(grid), dim3(64), 0, st, (const T *)a.dO, (const T *)a.wv, (T *)a.dax, a.T_q, a.H, a.F, (const T *)a.O_in, a.delta); return true;
    default: return false;
  }
}

template bool launch_mfma_absorb_dax<bf16>(const AbsorbArgs &, hipStream_t);
template bool launch_mfma_absorb_dax<f16>(const AbsorbArgs &, hipStream_t);
template void launch_mfma_absorb_du<bf16>(const AbsorbArgs &, hipStream_t);
template void launch_mfma_absorb_du<f16>(const AbsorbArgs &, hipStream_t);
template void launch_mfma_absorb_dx<bf16>(const AbsorbArgs &, hipStream_t);
template void launch_mfma_absorb_dx<f16>(const AbsorbArgs &, hipStream_t);

}  // namespace vafa
