// Absorbed ragged target attention forward on gfx950 matrix cores
// (replaces ta/kernels.py:185-284, the default "alpha" forward).
//
// One workgroup = 4 waves x 16 rows owns up to 64 (token, head) rows of one
// sample -- all H heads of 64/H consecutive tokens, one contiguous slab of u
// -- and one key range.  Raw X is streamed once per workgroup (not once per
// head) through a 3-deep ring of 32-key LDS tiles
// filled by buffer_load ... lds, one instruction per padded row (no staging
// registers; rows past the key range arrive as zeros).  Per tile each wave
// issues S^T = X U^T (X rows as the A operand) and aX^T += X^T P^T (X^T from
// ds_read_b64_tr_b16) as 16x16x32 products, LDS operands read a few products
// ahead, with the online softmax in the log2 domain.  The workgroup's rows
// are head-major (a wave's 16 rows span few heads: two at H = 8), so after
// the key loop each wave rounds aX/l to the input dtype in registers and
// projects it by each of its heads' W_V (16x16x32 products, W_V^T stored in the accumulators'
// f order): no LDS staging and no barrier in the epilogue.
//
// Folded projection (FOLD): instead of reading u (T_q x H x D_KV, written by
// a projection launch), the prologue forms each lane's u row from q_proj
// (T_q x H x D_H, 1/8 of u's bytes at D_KV = 256, D_H = 32) and W_K on the
// matrix cores -- U^T_h = W_K,h q_proj_h^T per 16-row f tile, accumulated in
// fp32 over d and rounded once to the input dtype, the reference's u GEMM
// (ta/interface.py:435) -- so u never reaches HBM.
//
// Unprojected epilogue (the DH = 0 instantiation, for wide heads or many
// heads per wave): each wave would read its heads' W_V (up to 2 x D_KV x D_H
// at H = 8, 256 KB at D_H = 256) from L2 for only 16 rows, so instead the
// rounded aX/l rows are written out
// ([T_q, H, FP] in wvt's f order; split partials unrounded as fp32) and one
// row GEMM with wvt projects them after the split combine -- the same
// roundings as the reference's epilogue: aX/l rounded to the input dtype,
// then one fp32-accumulated product with W_V (ta/kernels.py:274-275).
#include <algorithm>

#include "absorb_tiles.h"

namespace vafa {

namespace {

using namespace absorb;


// W_V [F, H, DH] -> wvt [H, DH, FP] (zero-padded over f): the A operand of
// the projection O^T = W_V^T (aX/l)^T.  Within each 32-wide f chunk,
// position 8a + b holds f = 4a + b (b < 4) or 16 + 4a + b - 4 (b >= 4), the
// order in which the forward's accumulators present aX^T (rows 4a..4a+3 of
// the chunk's two 16-row tiles).
// With the folded projection the same launch also writes
// W_K [F, H, DH] -> wkt [H, FP, DHP] (DHP = max(DH, 32); zeros at f >= F and
// d >= DH): the rows of one head contiguous, so the u product's A operand
// (16 f rows x 16 bytes per lane group) reads whole cache lines.
template <typename T>
__global__ __launch_bounds__(256) void transpose_w_kernel(const T *__restrict__ wv,
                                                          T *__restrict__ wvt,
                                                          const T *__restrict__ wk,
                                                          T *__restrict__ wkt, int H, int F,
                                                          int DH, int FP, int DHP) {
  const int64_t nv = (int64_t)H * DH * FP;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < nv) {
    const int p = (int)(i % FP);
    const int d = (int)((i / FP) % DH);
    const int h = (int)(i / ((int64_t)FP * DH));
    const int a = (p & 31) >> 3, b = p & 7;
    const int f = (p & ~31) + (b < 4 ? 4 * a + b : 16 + 4 * a + b - 4);
    wvt[i] = f < F ? wv[((int64_t)f * H + h) * DH + d] : static_cast<T>(0.f);
    return;
  }
  if (wkt == nullptr) return;
  const int64_t j = i - nv;
  if (j >= (int64_t)H * FP * DHP) return;
  const int d = (int)(j % DHP);
  const int f = (int)((j / DHP) % FP);
  const int h = (int)(j / ((int64_t)DHP * FP));
  wkt[j] = (f < F && d < DH) ? wk[((int64_t)f * H + h) * DH + d] : static_cast<T>(0.f);
}

constexpr int kFwdWaves = 4;  // 4 waves x 16 rows = kAbsorbRows

// FOLD: 0 = read u; 1 = form u in the prologue, one head per wave (H <= 4);
// 2 = form u, two heads per wave (H = 8: 8 tokens per head, 16 rows a wave).
template <typename T, int FP, int DH, int FOLD>
__global__ __launch_bounds__(64 * kFwdWaves, 2) void absorb_fwd_kernel(
    const T *__restrict__ u, const T *__restrict__ wkt, const T *__restrict__ X,
    const T *__restrict__ wvt, T *__restrict__ O, float *__restrict__ lse,
    float *__restrict__ part_o, float *__restrict__ part_lse, const int32_t *__restrict__ items,
    int H, int F, float c) {
  using M16 = Mfma16<T>;
  using v8 = typename Mfma<T>::v8;
  using S = AbsSmem<FP>;
  constexpr int NK = FP / 32;   // 32-wide reduction chunks of S^T
  constexpr int NF = FP / 16;   // 16-row f tiles of aX^T
  constexpr int kPerWave = kBK / kFwdWaves;  // DMA instructions per wave per tile
  constexpr int NBUF = S::kRing;
  constexpr int kPre = 4;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  T *smem = reinterpret_cast<T *>(smem_raw);

  const PlanItem it = load_item(items, blockIdx.x);
  const int t0 = it.v[0], t1 = it.v[1], k0 = it.v[2], k1 = it.v[3], pbase = it.v[4];
  if (t1 <= t0) return;  // no-op slot of the XCD-aware layout
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, lq = lane >> 4;
  // Rows are head-major inside the workgroup: row r is token r % TT of head
  // r / TT, so a wave's 16 rows span ceil(16 / TT) or one more heads and the
  // W_V projection runs on the accumulators in registers, once per head.
  // TT = floor(64 / H) tokens per item: with H not dividing 64 the last
  // 64 - TT*H rows of the workgroup (head index >= H) stay idle.
  const int ntok = t1 - t0;
  const int nrows = ntok * H;
  const int TT = kAbsorbRows / H;
  const int row = wave * 16 + l16;
  const int tl = row % TT, hh = row / TT;  // token / head of this lane's row
  const bool row_ok = tl < ntok && hh < H;
  const bool wave_active = wave_any(row_ok);
  // heads among the wave's rows
  const int h_first = (wave * 16) / TT;
  const int h_last = min(H - 1, (wave * 16 + 15) / TT);
  const int nh = h_last - h_first + 1;
  const int nt = (k1 - k0 + kBK - 1) / kBK;

  auto issue = [&](int kb, int buf) {
    const int rows = uniform_clamp(k1 - kb, kBK);
    dma_block<FP, kFwdWaves, S::XS>(X + (int64_t)kb * F, (uint32_t)(rows * F * 2), F,
                             lds_addr(smem + buf * S::kTile), wave, lane);
  };
  // only tiles of the key range are fetched (a tile past it would land as
  // zeros and cost a tile's DMA instructions)
#pragma unroll
  for (int b = 0; b < NBUF - 1; ++b)
    if (b < nt) issue(k0 + b * kBK, b);

  // U^T fragments (B operand of S^T = X U^T): row `row`, f = 32*kc + 8*lq + t
  v8 uf[NK];
  if constexpr (FOLD != 0) {
    // q_proj fragments (B operand of U^T = W_K,h q_proj^T): row `row`,
    // d = 32*ks + 8*lq + t; rows past the item's tokens and d >= DH read zeros
    constexpr int DHP = DH < 32 ? 32 : DH;
    constexpr int NKS = DHP / 32;
    v8 qb[NKS];
    const rsrc_t rq = make_rsrc(u + (int64_t)t0 * H * DH, (int64_t)nrows * DH * 2);
    // (consumed in the prologue, so no wait is forced here: the first W_K
    // batch below is requested before the first product waits for q_proj)
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      const int d0 = 32 * ks + 8 * lq;
      qb[ks] = as_v8<T>(
          buf_load16(rq, d0 < DH && hh < H ? ((tl * H + hh) * DH + d0) * 2 : 0x7fffffff));
    }
    // Output tile (kc, s) of U^T: its row m holds f = 32*kc + 8*(m/4) + 4*s
    // + m%4, so lane (column l16, group lq) receives f = 32*kc + 8*lq + 4*s + r
    // (r < 4): elements 4*s + r of the B fragment uf[kc] above.  A wave's 16
    // rows span nh <= NHW = FOLD heads: every head's product is formed (the
    // A operand is per head) and each lane keeps its own head's.  A negative
    // scale is folded into u (an exact sign flip before the rounding).  The A
    // operands (16-byte rows of wkt, from L2) are loaded KB chunks at a
    // time, the next batch in flight while the current one is multiplied:
    // one L2 round trip of latency instead of one per chunk.
    constexpr int NHW = FOLD;                          // heads per wave (max)
    constexpr int UPC = 2 * NHW * NKS;                 // A loads per f chunk
    static_assert(UPC <= 8, "folded u product: at most 8 A loads per f chunk");
    constexpr int KB = UPC <= 4 ? 2 : 1;               // f chunks per batch
    constexpr int NB = (NK + KB - 1) / KB;             // the last may be short
    const float sgn = c < 0.f ? -1.f : 1.f;
    const int hsel = min(max(hh - h_first, 0), NHW - 1);  // this lane's head slot
    const int frow = 8 * (l16 >> 2) + (l16 & 3);
    const T *wa[NHW];
#pragma unroll
    for (int hx = 0; hx < NHW; ++hx)  // heads past H (idle rows) reuse the last
      wa[hx] = wkt + ((int64_t)min(h_first + hx, H - 1) * FP + frow) * DHP + 8 * lq;
    u32x4 abuf[2][KB][2][NHW][NKS];
    auto load_batch = [&](int b, int slot) {
#pragma unroll
      for (int kk = 0; kk < KB; ++kk)
        if (b * KB + kk < NK)
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
          for (int hx = 0; hx < NHW; ++hx)
#pragma unroll
            for (int ks = 0; ks < NKS; ++ks)
              abuf[slot][kk][s][hx][ks] = *reinterpret_cast<const u32x4 *>(
                  wa[hx] + (int64_t)(32 * (b * KB + kk) + 4 * s) * DHP + 32 * ks);
    };
    load_batch(0, 0);
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      if (b + 1 < NB) load_batch(b + 1, (b + 1) & 1);
#pragma unroll
      for (int kk = 0; kk < KB; ++kk) {
        const int kc = b * KB + kk;
        if (kc >= NK) break;
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          f32x4 r[NHW];
#pragma unroll
          for (int hx = 0; hx < NHW; ++hx) {
            r[hx] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < NKS; ++ks)
              r[hx] = M16::mma(as_v8<T>(abuf[b & 1][kk][s][hx][ks]), qb[ks], r[hx]);
          }
          f32x4 rr = r[0];
#pragma unroll
          for (int hx = 1; hx < NHW; ++hx)
#pragma unroll
            for (int e = 0; e < 4; ++e) rr[e] = hsel == hx ? r[hx][e] : rr[e];
#pragma unroll
          for (int e = 0; e < 4; ++e) uf[kc][4 * s + e] = static_cast<T>(rr[e] * sgn);
        }
      }
    }
  } else {
    const rsrc_t ru = make_rsrc(u + (int64_t)t0 * H * F, (int64_t)nrows * F * 2);
    const int fchunks = F / 8;
    // a negative scale is folded into u (sign flip of every element)
    const uint32_t usign = c < 0.f ? 0x80008000u : 0u;
#pragma unroll
    for (int kc = 0; kc < NK; ++kc) {
      const int ch = kc * 4 + lq;
      // rows past the item's tokens lie past the descriptor's range: zeros
      u32x4 w = buf_load16(ru, ch < fchunks && hh < H ? (tl * H + hh) * F * 2 + ch * 16
                                                       : 0x7fffffff);
      // waited for here, in the prologue, not inside the key loop where a
      // compiler vmcnt wait would also drain the LDS-DMA ring
      asm volatile("" : "+v"(w));
#pragma unroll
      for (int e = 0; e < 4; ++e) w[e] ^= usign;
      uf[kc] = as_v8<T>(w);
    }
  }
  c = fabsf(c);
  f32x4 acc[NF];
#pragma unroll
  for (int i = 0; i < NF; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[i][r] = 0.f;
  float m_run = -kHuge, l_part = 0.f;

  const int a_off = l16 * S::XS + lq * 8;
  const int t_off = (4 * lq + (l16 >> 2)) * S::XS + 4 * (l16 & 3);
  int buf = 0;  // j % NBUF
  for (int j = 0; j < nt; ++j) {
    // tile j landed (tile j+1, if there is one, may still be in flight),
    // visible to all waves, and every wave is done with tile j-1 whose slot
    // is refilled next
    // (3-deep ring: tile j+1 may stay in flight; 2-deep: none is)
    if (NBUF == 3 && j + 1 < nt)
      wait_vmcnt<(NBUF - 2) * kPerWave>();
    else
      wait_vmcnt<0>();
    __syncthreads();
    if (j + NBUF - 1 < nt) issue(k0 + (j + NBUF - 1) * kBK, buf == 0 ? NBUF - 1 : buf - 1);
    const int kb = k0 + j * kBK;
    if (wave_active) {
      const lds_cptr<T> xa = as_lds(smem + buf * S::kTile + a_off);
      const lds_cptr<T> xt = as_lds(smem + buf * S::kTile + t_off);
      // S^T in two 16-key halves: element r of half mt is key
      // kb + 16*mt + 4*lq + r of this lane's row; A reads run kPre ahead
      auto aop = [&](int i) { return lds_ld16<T>(xa + (i / NK) * 16 * S::XS + (i % NK) * 32); };
      f32x4 s[2];
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) s[mt][r] = 0.f;
      u32x4 ring[kPre];
#pragma unroll
      for (int i = 0; i < kPre; ++i) ring[i] = aop(i);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < 2 * NK; ++i) {
        s[i / NK] = M16::mma(as_v8<T>(ring[i % kPre]), uf[i % NK], s[i / NK]);
        if (i + kPre < 2 * NK) ring[i % kPre] = aop(i + kPre);
        __builtin_amdgcn_sched_barrier(0);
      }
      // X^T operands of aX^T: lane l gets column 16*ft + l%16 at the keys of
      // its k slots 8*lq + t <-> key 4*lq + t (t < 4), 16 + 4*lq + t - 4
      auto top = [&](int ft) {
        return as_v8<T>(join(lds_tr8<T>(xt + ft * 16), lds_tr8<T>(xt + 16 * S::XS + ft * 16)));
      };
      v8 tring[kPre];
#pragma unroll
      for (int i = 0; i < kPre; ++i) tring[i] = top(i);
      if (kb + kBK > k1) {
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (kb + 16 * mt + 4 * lq + r >= k1) s[mt][r] = kNegInf;
      }
      // P against the running max first; the lane's tile sum checks the
      // bound (P <= 2^8 everywhere, or the first tile with m_run = -kHuge)
      // and only an out-of-bound tile takes the row max and rescales.
      v8 pb;
      float ps;
      auto build_p = [&]() {
        float p2[2] = {0.f, 0.f};
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float p = fast_exp2(__builtin_fmaf(s[mt][r], c, -m_run));
            p2[r & 1] += p;
            pb[4 * mt + r] = static_cast<T>(p);
          }
        ps = p2[0] + p2[1];
      };
      build_p();
      if (wave_any(!(ps <= kLazyMax))) {
        float mx = fmaxf(fmaxf(fmaxf(s[0][0], s[0][1]), fmaxf(s[0][2], s[0][3])),
                         fmaxf(fmaxf(s[1][0], s[1][1]), fmaxf(s[1][2], s[1][3])));
        mx = max_xor32(max_xor16(mx)) * c;
        const float m_new = fmaxf(m_run, mx);
        const float alpha = fast_exp2(m_run - m_new);
        m_run = m_new;
        l_part *= alpha;
#pragma unroll
        for (int i = 0; i < NF; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[i][r] *= alpha;
        build_p();
      }
      l_part += ps;
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int ft = 0; ft < NF; ++ft) {
        acc[ft] = M16::mma(tring[ft % kPre], pb, acc[ft]);
        if (ft + kPre < NF) tring[ft % kPre] = top(ft + kPre);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    buf = buf == NBUF - 1 ? 0 : buf + 1;
  }
  wait_vmcnt<0>();

  // ---- epilogue: O = round(aX / l) W_V from the accumulators ----
  // The four lanes of a column hold its P-sum partials.
  float l = l_part + __shfl_xor(l_part, 16, 64);
  l += __shfl_xor(l, 32, 64);
  const float inv = l > 0.f ? 1.f / l : 0.f;
  if (row_ok && lq == 0) {
    const float lse_v = l > 0.f ? m_run + fast_log2(l) : kNegInf;
    if (pbase < 0)
      lse[(int64_t)(t0 + tl) * H + hh] = lse_v;
    else
      part_lse[(int64_t)(pbase + tl) * H + hh] = lse_v;
  }
  if (!wave_active) return;
  if constexpr (DH == 0) {
    // unprojected: position 32*kc + 8*lq + t of the row (wvt's f order, as
    // in bx below) is accumulator element [2kc + t/4][t%4]
    if (!row_ok) return;
    if (pbase < 0) {
      T *dst = O + ((int64_t)(t0 + tl) * H + hh) * FP + lq * 8;
#pragma unroll
      for (int kc = 0; kc < NK; ++kc) {
        v8 b;
#pragma unroll
        for (int t = 0; t < 8; ++t) b[t] = static_cast<T>(acc[2 * kc + (t >> 2)][t & 3] * inv);
        *reinterpret_cast<v8 *>(dst + kc * 32) = b;
      }
    } else {
      float *dst = part_o + ((int64_t)(pbase + tl) * H + hh) * FP + lq * 8;
#pragma unroll
      for (int kc = 0; kc < NK; ++kc)
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          f32x4 v;
#pragma unroll
          for (int r = 0; r < 4; ++r) v[r] = acc[2 * kc + s][r] * inv;
          *reinterpret_cast<f32x4 *>(dst + kc * 32 + 4 * s) = v;
        }
    }
    return;
  }
  // B operand of O^T = W_V^T (aX/l)^T for 32-wide f chunk kc: k slot t of
  // lane group lq is f = 32*kc + 4*lq + t (t < 4, from acc[2kc]) or
  // 32*kc + 16 + 4*lq + t - 4 (t >= 4, from acc[2kc+1]); wvt stores W_V^T in
  // that order, so the A operand is one 16-byte load.
  v8 bx[NK];
#pragma unroll
  for (int kc = 0; kc < NK; ++kc)
#pragma unroll
    for (int t = 0; t < 8; ++t)
      bx[kc][t] = static_cast<T>(acc[2 * kc + (t >> 2)][t & 3] * inv);
  constexpr int ND16 = DH / 16;
  typedef __attribute__((__vector_size__(4 * sizeof(T)))) T T4;
  for (int hx = 0; hx < nh; ++hx) {
    const int h = h_first + hx;
    const T *arow = wvt + ((int64_t)h * DH + l16) * FP + lq * 8;
#pragma unroll
    for (int dt = 0; dt < ND16; ++dt) {
      u32x4 wa[NK];
#pragma unroll
      for (int kc = 0; kc < NK; ++kc)
        wa[kc] = *reinterpret_cast<const u32x4 *>(arow + dt * 16 * FP + kc * 32);
      f32x4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kc = 0; kc < NK; ++kc) o = M16::mma(as_v8<T>(wa[kc]), bx[kc], o);
      // lane: row l16 (token tl of head hh), d = 16*dt + 4*lq + r
      if (row_ok && hh == h) {
        const int d = dt * 16 + lq * 4;
        if (pbase < 0) {
          T4 w;
#pragma unroll
          for (int r = 0; r < 4; ++r) w[r] = static_cast<T>(o[r]);
          *reinterpret_cast<T4 *>(O + ((int64_t)(t0 + tl) * H + hh) * DH + d) = w;
        } else {
          *reinterpret_cast<f32x4 *>(part_o + ((int64_t)(pbase + tl) * H + hh) * DH + d) = o;
        }
      }
    }
  }
}


template <typename T, int FP, int DH, int FOLD>
void launch_fold(const AbsorbArgs &a, const T *wvt, hipStream_t st) {
  const int smem = AbsSmem<FP>::kLoopBytes;
  allow_dynamic_lds(reinterpret_cast<const void *>(&absorb_fwd_kernel<T, FP, DH, FOLD>), smem);
  hipLaunchKernelGGL((absorb_fwd_kernel<T, FP, DH, FOLD>), dim3((unsigned)a.n_items),
                     dim3(64 * kFwdWaves), smem, st, (const T *)a.u, (const T *)a.wkt,
                     (const T *)a.X, wvt, (T *)(DH == 0 ? a.axf : a.O), a.lse, a.part_o,
                     a.part_lse, a.items, a.H,
                     a.F, a.scale * kLog2e);
}

template <typename T, int FP, int DH>
void launch_fp(const AbsorbArgs &a, const T *wvt, hipStream_t st) {
  if (!a.fold) return launch_fold<T, FP, DH, 0>(a, wvt, st);
  if constexpr (DH <= 128) {
    const int nhw = absorb_heads_per_wave(a.H);
    if (nhw == 1) return launch_fold<T, FP, DH, 1>(a, wvt, st);
    if constexpr (DH <= 64) {
      if (nhw == 2) return launch_fold<T, FP, DH, 2>(a, wvt, st);
    }
    if constexpr (DH <= 32) return launch_fold<T, FP, DH, 4>(a, wvt, st);
  }
}

template <typename T, int DH>
void launch_dh(const AbsorbArgs &a, const T *wvt, int FP, hipStream_t st) {
  switch (FP) {
    case 64: launch_fp<T, 64, DH>(a, wvt, st); break;
    case 128: launch_fp<T, 128, DH>(a, wvt, st); break;
    case 192: launch_fp<T, 192, DH>(a, wvt, st); break;
    case 224: launch_fp<T, 224, DH>(a, wvt, st); break;
    case 256: launch_fp<T, 256, DH>(a, wvt, st); break;
    case 512: launch_fold<T, 512, DH, 0>(a, wvt, st); break;
    default: break;
  }
}


}  // namespace

using absorb::padded_f;

// The matrix-core path takes H <= 64 (floor(64/H) >= 1 tokens per item; a
// wave's 16 rows span up to 16 heads, each projected in the epilogue), D_KV
// a multiple of 8 up to 256 (padded onto one of the compiled widths), and
// D_H in {16, 32, 64, 128, 256}.
template <typename T>
bool mfma_absorb_supported(int H, int F, int DH) {
  const bool f_ok = F >= 8 && F % 8 == 0 && F <= kMaxF;
  const bool h_ok = H >= 1 && H <= kAbsorbRows;
  const bool d_ok = DH == 16 || DH == 32 || DH == 64 || DH == 128 || DH == 256;
  return f_ok && h_ok && d_ok;
}

// The forward and backward kernels also take 256 < D_KV <= 512 (FP = 512:
// a 2-deep forward ring, one workgroup per CU in du and dX).
template <typename T>
bool mfma_absorb_fwd_supported(int H, int F, int DH) {
  if (F > kMaxF && F <= kMaxFwdF && F % 8 == 0) return mfma_absorb_supported<T>(H, 8, DH);
  return mfma_absorb_supported<T>(H, F, DH);
}

// Most heads among the 16 rows of one forward wave (rows head-major,
// floor(64/H) tokens per head).
int absorb_heads_per_wave(int H) {
  const int TT = kAbsorbRows / H;
  int m = 0;
  for (int w = 0; w < kFwdWaves; ++w) {
    const int a = (16 * w) / TT;
    if (a >= H) continue;
    const int b = std::min(H - 1, (16 * w + 15) / TT);
    m = std::max(m, b - a + 1);
  }
  return m;
}

// The folded forward forms u in the prologue: 2 * heads-per-wave * D_H/32
// A-operand loads per 32-wide f chunk must fit its register batch (<= 8),
// and above FP = 128 only the variants that keep three waves per SIMD
// without spilling (at most two heads per wave, D_H <= 64; gfx950 register
// counts of the compiled kernels) fold; other shapes read a projected u.
bool mfma_absorb_fold_supported(int H, int F, int DH) {
  if (!mfma_absorb_supported<bf16>(H, F, DH)) return false;  // F <= 256
  const int nhw = absorb_heads_per_wave(H);
  if (nhw > 4) return false;  // FOLD variants form at most 4 heads per wave
  const int nhw_t = nhw == 1 ? 1 : nhw == 2 ? 2 : 4;
  if (nhw_t * (DH < 32 ? 1 : DH / 32) > 4) return false;
  return padded_f(F) <= 128 || (nhw_t <= 2 && DH <= 64);
}

// Without the folded projection, shapes whose epilogue would read at least
// 128 x FP x 2 bytes of W_V per wave (heads per wave x D_H >= 128) write aX/l
// and project it in a separate row GEMM: per (token, head) row that is 4 FP
// bytes of HBM traffic (aX written and read back) against heads-per-wave x
// D_H x FP / 8 bytes of L2 reads, and measured on C4's lengths the row GEMM
// wins from a ratio of 4 on (H = 8: D_H >= 64; H = 16: D_H >= 32; H <= 4:
// D_H >= 128).  The combine covers widths up to 256.
bool mfma_absorb_unprojected(int H, int F, int DH, bool fold) {
  return absorb_heads_per_wave(H) * DH >= 128 && padded_f(F) <= 256 && !fold;
}

int64_t mfma_absorb_wvt_elems(int H, int F, int DH) { return (int64_t)H * DH * padded_f(F); }
int64_t mfma_absorb_wkt_elems(int H, int F, int DH) {
  return (int64_t)H * padded_f(F) * (DH < 32 ? 32 : DH);
}

template <typename T>
void launch_mfma_absorb_fwd(const AbsorbArgs &a, hipStream_t st) {
  const int FP = padded_f(a.F);
  T *wvt = reinterpret_cast<T *>(a.wvt);
  const int DHP = a.DH < 32 ? 32 : a.DH;
  const int64_t n = (int64_t)a.H * a.DH * FP + (a.fold ? (int64_t)a.H * FP * DHP : 0);
  hipLaunchKernelGGL(transpose_w_kernel<T>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                     (const T *)a.wv, wvt, (const T *)a.wk,
                     a.fold ? reinterpret_cast<T *>(a.wkt) : nullptr, a.H, a.F, a.DH, FP, DHP);
  if (a.n_items == 0) return;
  if (mfma_absorb_unprojected(a.H, a.F, a.DH, a.fold)) {
    switch (FP) {
      case 64: launch_fold<T, 64, 0, 0>(a, wvt, st); break;
      case 128: launch_fold<T, 128, 0, 0>(a, wvt, st); break;
      case 192: launch_fold<T, 192, 0, 0>(a, wvt, st); break;
      case 224: launch_fold<T, 224, 0, 0>(a, wvt, st); break;
      case 256: launch_fold<T, 256, 0, 0>(a, wvt, st); break;
      default: break;
    }
    return;
  }
  switch (a.DH) {
    case 16: launch_dh<T, 16>(a, wvt, FP, st); break;
    case 32: launch_dh<T, 32>(a, wvt, FP, st); break;
    case 64: launch_dh<T, 64>(a, wvt, FP, st); break;
    case 128: launch_dh<T, 128>(a, wvt, FP, st); break;
    case 256: launch_dh<T, 256>(a, wvt, FP, st); break;
    default: break;
  }
}

template bool mfma_absorb_supported<bf16>(int, int, int);
template bool mfma_absorb_supported<f16>(int, int, int);
template bool mfma_absorb_fwd_supported<bf16>(int, int, int);
template bool mfma_absorb_fwd_supported<f16>(int, int, int);
template void launch_mfma_absorb_fwd<bf16>(const AbsorbArgs &, hipStream_t);
template void launch_mfma_absorb_fwd<f16>(const AbsorbArgs &, hipStream_t);

}  // namespace vafa
