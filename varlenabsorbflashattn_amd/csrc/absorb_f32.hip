// Absorbed ragged target attention in fp32 on gfx950 matrix cores
// (v_mfma_f32_16x16x4_f32): the reference's documented call, which computes
// with fp32 inputs and IEEE fp32 dots (ta/interface.py:371, 389-391;
// ta/kernels.py:258-270).  Same work decomposition as the 16-bit kernels:
//   * forward (ta/kernels.py:185-284) and du/aX (ta/kernels.py:354-498): a
//     workgroup of 4 waves x 16 rows owns the H heads of floor(64/H) tokens
//     of one sample (head-major; with H not dividing 64 the last rows idle)
//     and streams the sample's X rows once through a 3-deep ring of 16-key
//     LDS tiles filled by buffer_load ... lds;
//   * dX (ta/kernels.py:528-900): a workgroup owns up to 512 keys of one
//     sample, 16 per wave per pass, and streams the sample's (token, head)
//     rows of u and dAX through LDS in blocks of 32, summing over heads in
//     registers (deterministic).
//
// Operand layout of v_mfma_f32_16x16x4_f32 (wave64; l16 = lane % 16,
// lq = lane / 16): A (16 x 4) lane holds A[l16][lq], B (4 x 16) lane holds
// B[lq][l16], C (16 x 16) lane holds C[4*lq + r][l16], r = 0..3.
// Two relabellings keep every operand read a contiguous 16-byte load:
//   * products that reduce over features (S = u.X, dP = dAX.X): product i
//     takes feature Q*lq + i in lane group lq (Q = FP/4), so a lane reads Q
//     consecutive floats of its row;
//   * products that reduce over keys or rows (aX^T, du^T, dX^T): the output
//     tile (a, b) holds feature 64a + 4m + b in its row m, so an A operand
//     read is 4 consecutive floats (b = 0..3) and a lane's accumulators hold
//     features 64a + 16*lq + 4r + b -- four consecutive floats per (a, r),
//     stored (and projected by W_V) as 16-byte runs.
#include "kernels.h"
#include "mfma.h"

namespace vafa {

namespace {

__device__ __forceinline__ f32x4 mma4(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

constexpr int kKT = 16;    // keys per LDS tile (forward, du)
constexpr int kNBuf = 3;   // LDS ring depth
constexpr int kRBlk = 32;  // (token, head) rows per LDS block (dX)

// padded feature width: a multiple of 64 (the aX^T / du^T / dX^T tiling) up
// to 256; 512 above (the forward only)
inline int fp64_of(int F) { return F > 256 ? 512 : (F + 63) / 64 * 64; }

// LDS row stride (floats): 16 consecutive rows read at one column by the
// S / dP products land on 16 distinct 16-byte bank groups
template <int FP>
struct F32Smem {
  static constexpr int XS = FP + 4;
  static constexpr int kTile = kKT * XS;
  static constexpr int kFwdBytes = kNBuf * kTile * 4;
  static constexpr int kDxBytes = 2 * kRBlk * XS * 4 + 2 * kRBlk * 4;
};

// LDS-DMA of rows [0, ROWS) of a row-major slab of F floats per row into a
// [ROWS][XS] LDS block: NW waves move ROWS/NW rows each, one instruction per
// 64 16-byte chunks of a row (two at FP = 512) with chunks < FP/4 active
// (chunks past F, and rows past the slab's `bytes`, read as zeros).
template <int FP, int NW, int ROWS, int XS>
__device__ __forceinline__ void dma_rows_f32(const float *src, int64_t bytes, int F, uint32_t base,
                                             int wave, int lane) {
  constexpr int NI = (FP / 4 + 63) / 64;  // instructions per row
  const u32x4 rs = rsrc_words(src, bytes);
#pragma unroll
  for (int part = 0; part < NI; ++part) {
    const int ch = part * 64 + lane;
    const uint32_t off = ch < F / 4 ? (uint32_t)ch * 16u : 0x80000000u;
    if (ch < FP / 4) {
#pragma unroll
      for (int n = 0; n < ROWS / NW; ++n) {
        const int r = wave * (ROWS / NW) + n;
        int32_t voff;
        asm volatile("v_add_u32 %0, %1, %2" : "=v"(voff) : "s"(r * F * 4), "v"(off));
        lds_dma16(rs, base + r * XS * 4 + part * 1024, voff);
      }
    }
  }
}

// The lane's Q = FP/4 features [Q*lq, Q*lq + Q) of one row of a [*, F] fp32
// tensor (zero past F and for rows outside the descriptor's range).
template <int FP>
__device__ __forceinline__ void load_quarter(float (&dst)[FP / 4], rsrc_t r, int row_byte_off,
                                             int F, int lq) {
  constexpr int Q = FP / 4;
#pragma unroll
  for (int i4 = 0; i4 < Q / 4; ++i4) {
    const int f = Q * lq + 4 * i4;
    // the whole 16 bytes are reinterpreted, then indexed (a bit cast of one
    // vector element, bit_cast(float, w[1]), reads element 0 in this clang)
    const f32x4 v = __builtin_bit_cast(f32x4, buf_load16(r, f < F ? row_byte_off + f * 4
                                                                  : 0x7fffffff));
    float x0 = v[0], x1 = v[1], x2 = v[2], x3 = v[3];
    asm volatile("" : "+v"(x0), "+v"(x1), "+v"(x2), "+v"(x3));  // waited for here
    dst[4 * i4] = x0;
    dst[4 * i4 + 1] = x1;
    dst[4 * i4 + 2] = x2;
    dst[4 * i4 + 3] = x3;
  }
}

// ---------------------------------------------------------------------------
// W_V [F, H, DH] -> wvt [H, DH, FP] fp32 (zero past F): the A operand of the
// forward's projection, read as 16-byte runs along f.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void transpose_wv_f32_kernel(const float *__restrict__ wv,
                                                               float *__restrict__ wvt, int H,
                                                               int F, int DH, int FP) {
  const int64_t n = (int64_t)H * DH * FP;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const int f = (int)(i % FP);
  const int d = (int)((i / FP) % DH);
  const int h = (int)(i / ((int64_t)FP * DH));
  wvt[i] = f < F ? wv[((int64_t)f * H + h) * DH + d] : 0.f;
}

// Row geometry of a 64-row workgroup (forward and du): row = wave*16 + l16
// is token row % TT of head row / TT, TT = floor(64 / H) tokens (rows past
// H * TT idle).  A wave's rows span heads h_first..h_last.
struct Rows64 {
  int TT, tl, hh, h_first, h_last;
  bool row_ok, wave_active;
  __device__ Rows64(int H, int ntok, int wave, int l16) {
    TT = kAbsorbRows / H;
    const int row = wave * 16 + l16;
    tl = row % TT;
    hh = row / TT;
    row_ok = tl < ntok && hh < H;
    wave_active = wave_any(row_ok);
    h_first = wave * 16 / TT;
    h_last = (wave * 16 + 15) / TT < H - 1 ? (wave * 16 + 15) / TT : H - 1;
  }
};

// ---------------------------------------------------------------------------
// Forward: O = softmax(c u X^T) X W_V per (token, head) row, online softmax
// in the log2 domain against a lazily updated running max; split items
// write projected fp32 partial rows + LSE for the combine.
// ---------------------------------------------------------------------------
// two workgroups per CU; one at FP = 512 (u operands and accumulators take
// 256 registers)
template <int FP>
__global__ __launch_bounds__(256, FP > 256 ? 1 : 2) void absorb_fwd_f32_kernel(
    const float *__restrict__ u, const float *__restrict__ X, const float *__restrict__ wvt,
    float *__restrict__ O, float *__restrict__ lse, float *__restrict__ part_o,
    float *__restrict__ part_lse, const int32_t *__restrict__ items, int H, int F, int DH,
    float c) {
  using S = F32Smem<FP>;
  constexpr int Q = FP / 4, NA = FP / 64, XS = S::XS;
  constexpr int kPerWave = kKT / 4 * ((FP / 4 + 63) / 64);  // DMA instructions per wave per tile
  extern __shared__ __align__(16) float smem_f[];

  const PlanItem it = load_item(items, blockIdx.x);
  const int t0 = it.v[0], t1 = it.v[1], k0 = it.v[2], k1 = it.v[3], pbase = it.v[4];
  if (t1 <= t0) return;  // no-op slot of the XCD-aware layout
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, lq = lane >> 4;
  const int ntok = t1 - t0;
  const Rows64 g(H, ntok, wave, l16);
  const int nt = (k1 - k0 + kKT - 1) / kKT;

  auto issue = [&](int kb, int buf) {
    const int rows = k1 - kb < kKT ? (k1 - kb > 0 ? k1 - kb : 0) : kKT;
    dma_rows_f32<FP, 4, kKT, XS>(X + (int64_t)kb * F, (int64_t)rows * F * 4, F,
                                 lds_addr(smem_f + buf * S::kTile), wave, lane);
  };
#pragma unroll
  for (int b = 0; b < kNBuf - 1; ++b) issue(k0 + b * kKT, b);

  // B operand of S^T = X U^T: this lane's row, features Q*lq .. Q*lq+Q-1; a
  // negative scale is folded into u
  float uf[Q];
  {
    const rsrc_t ru = make_rsrc(u + (int64_t)t0 * H * F, (int64_t)ntok * H * F * 4);
    load_quarter<FP>(uf, ru, g.row_ok ? (g.tl * H + g.hh) * F * 4 : 0x7fff0000, F, lq);
    if (c < 0.f) {
#pragma unroll
      for (int i = 0; i < Q; ++i) uf[i] = -uf[i];
    }
  }
  c = fabsf(c);
  f32x4 acc[NA][4];
#pragma unroll
  for (int a = 0; a < NA; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -kHuge, l_part = 0.f;

  int buf = 0;
  for (int j = 0; j < nt; ++j) {
    wait_vmcnt<(kNBuf - 2) * kPerWave>();
    __syncthreads();
    issue(k0 + (j + kNBuf - 1) * kKT, buf == 0 ? kNBuf - 1 : buf - 1);
    const int kb = k0 + j * kKT;
    if (g.wave_active) {
      const float *xs = smem_f + buf * S::kTile;
      // S^T (16 keys x 16 rows): lane holds key kb + 4*lq + r of its row;
      // four independent accumulation chains, summed at the end
      f32x4 s4[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) s4[e] = f32x4{0.f, 0.f, 0.f, 0.f};
      const float *xa = xs + l16 * XS + Q * lq;
#pragma unroll
      for (int i4 = 0; i4 < Q / 4; ++i4) {
        const f32x4 xv = *reinterpret_cast<const f32x4 *>(xa + 4 * i4);
#pragma unroll
        for (int e = 0; e < 4; ++e) s4[e] = mma4(xv[e], uf[4 * i4 + e], s4[e]);
      }
      f32x4 s = (s4[0] + s4[1]) + (s4[2] + s4[3]);
      if (kb + kKT > k1) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (kb + 4 * lq + r >= k1) s[r] = kNegInf;
      }
      float p[4], ps;
      auto build_p = [&]() {
#pragma unroll
        for (int r = 0; r < 4; ++r) p[r] = fast_exp2(__builtin_fmaf(s[r], c, -m_run));
        ps = (p[0] + p[1]) + (p[2] + p[3]);
      };
      build_p();
      if (wave_any(!(ps <= kLazyMax))) {
        float mx = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
        mx = max_xor32(max_xor16(mx)) * c;
        const float m_new = fmaxf(m_run, mx);
        const float alpha = fast_exp2(m_run - m_new);
        m_run = m_new;
        l_part *= alpha;
#pragma unroll
        for (int a = 0; a < NA; ++a)
#pragma unroll
          for (int b = 0; b < 4; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[a][b][r] *= alpha;
        build_p();
      }
      l_part += ps;
      // aX^T += X^T P^T over the tile's 16 keys in 4 slices (slot lq <-> key
      // 4*lq + j4, whose P this lane holds in p[j4])
#pragma unroll
      for (int j4 = 0; j4 < 4; ++j4) {
        const float *xt = xs + (4 * lq + j4) * XS + 4 * l16;
#pragma unroll
        for (int a = 0; a < NA; ++a) {
          const f32x4 xv = *reinterpret_cast<const f32x4 *>(xt + 64 * a);
#pragma unroll
          for (int b = 0; b < 4; ++b) acc[a][b] = mma4(xv[b], p[j4], acc[a][b]);
        }
      }
    }
    buf = buf == kNBuf - 1 ? 0 : buf + 1;
  }
  wait_vmcnt<0>();

  // ---- epilogue: O = (aX / l) W_V from the accumulators ----
  float l = l_part + __shfl_xor(l_part, 16, 64);
  l += __shfl_xor(l, 32, 64);
  const float inv = l > 0.f ? 1.f / l : 0.f;
  if (g.row_ok && lq == 0) {
    const float lse_v = l > 0.f ? m_run + fast_log2(l) : kNegInf;
    if (pbase < 0)
      lse[(int64_t)(t0 + g.tl) * H + g.hh] = lse_v;
    else
      part_lse[(int64_t)(pbase + g.tl) * H + g.hh] = lse_v;
  }
  if (!g.wave_active) return;
#pragma unroll
  for (int a = 0; a < NA; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[a][b][r] *= inv;
  // O^T (16 d x 16 rows) = W_V^T (16 d x f) (aX/l)^T: slice (a, r, b) takes
  // feature 64a + 16*lq + 4r + b in lane group lq -- the lane's own
  // accumulator acc[a][b][r] as B, wvt[h][d][64a + 16lq + 4r + b] as A
  for (int h = g.h_first; h <= g.h_last; ++h) {
    for (int dt = 0; dt < DH / 16; ++dt) {
      const float *wrow = wvt + ((int64_t)h * DH + dt * 16 + l16) * FP + 16 * lq;
      f32x4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int a = 0; a < NA; ++a)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const f32x4 w = *reinterpret_cast<const f32x4 *>(wrow + 64 * a + 4 * r);
#pragma unroll
          for (int b = 0; b < 4; ++b) o = mma4(w[b], acc[a][b][r], o);
        }
      // lane: row l16, d = 16*dt + 4*lq + r
      if (g.row_ok && g.hh == h) {
        const int d = dt * 16 + lq * 4;
        if (pbase < 0)
          *reinterpret_cast<f32x4 *>(O + ((int64_t)(t0 + g.tl) * H + g.hh) * DH + d) = o;
        else
          *reinterpret_cast<f32x4 *>(part_o + ((int64_t)(pbase + g.tl) * H + g.hh) * DH + d) = o;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Backward, query side (ta/kernels.py:354-498): per token tile with the
// sample's whole key range, P rebuilt from the saved LSE:
//   du = scale * sum_j dS_j X_j,  aX = sum_j P_j X_j (fp32, for dW_V),
//   dS = P (dP - delta), dP = dAX . X_j, dAX = dO W_V^T (workspace).
// ---------------------------------------------------------------------------
template <int FP>
__global__ __launch_bounds__(256, 1) void absorb_du_f32_kernel(
    const float *__restrict__ u, const float *__restrict__ X, const float *__restrict__ lse,
    const float *__restrict__ delta, const float *__restrict__ dax, float *__restrict__ du,
    float *__restrict__ ax_ws, const int32_t *__restrict__ items, int n_items, int H, int F,
    float c, float scale) {
  using S = F32Smem<FP>;
  // FP = 512: two workgroups of one XCD share a token tile (blocks b and
  // b + 8 of each 16), each forming S and dP over every feature and
  // accumulating du / aX for one half of the 64-feature groups
  constexpr int NS = FP > 256 ? 2 : 1;
  constexpr int Q = FP / 4, NA = FP / 64 / NS, XS = S::XS;
  constexpr int kPerWave = kKT / 4 * ((FP / 4 + 63) / 64);
  extern __shared__ __align__(16) float smem_f[];

  int item = blockIdx.x, a0 = 0;  // first 64-feature group of this slice
  if constexpr (NS == 2) {
    const int b = blockIdx.x;
    item = (b / 16) * 8 + b % 8;
    a0 = ((b / 8) & 1) * NA;
    if (item >= n_items) return;  // padding of the last group of 16
  }
  const PlanItem it = load_item(items, item);
  const int t0 = it.v[0], t1 = it.v[1], k0 = it.v[2], k1 = it.v[3];
  if (t1 <= t0) return;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, lq = lane >> 4;
  const int ntok = t1 - t0;
  const Rows64 g(H, ntok, wave, l16);
  const int nt = (k1 - k0 + kKT - 1) / kKT;

  auto issue = [&](int kb, int buf) {
    const int rows = k1 - kb < kKT ? (k1 - kb > 0 ? k1 - kb : 0) : kKT;
    dma_rows_f32<FP, 4, kKT, XS>(X + (int64_t)kb * F, (int64_t)rows * F * 4, F,
                                 lds_addr(smem_f + buf * S::kTile), wave, lane);
  };
#pragma unroll
  for (int b = 0; b < kNBuf - 1; ++b) issue(k0 + b * kKT, b);

  float uf[Q], df[Q];
  const int64_t grow = (int64_t)(t0 + g.tl) * H + g.hh;  // global (token, head) row
  {
    const int64_t nb = (int64_t)ntok * H * F * 4;
    const int off = g.row_ok ? (g.tl * H + g.hh) * F * 4 : 0x7fff0000;
    load_quarter<FP>(uf, make_rsrc(u + (int64_t)t0 * H * F, nb), off, F, lq);
    load_quarter<FP>(df, make_rsrc(dax + (int64_t)t0 * H * F, nb), off, F, lq);
  }
  float L = g.row_ok ? lse[grow] : 0.f;
  float Dl = g.row_ok ? delta[grow] : 0.f;
  asm volatile("" : "+v"(L), "+v"(Dl));
  f32x4 adu[NA][4], aax[NA][4];
#pragma unroll
  for (int a = 0; a < NA; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) adu[a][b] = aax[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};

  int buf = 0;
  for (int j = 0; j < nt; ++j) {
    wait_vmcnt<(kNBuf - 2) * kPerWave>();
    __syncthreads();
    issue(k0 + (j + kNBuf - 1) * kKT, buf == 0 ? kNBuf - 1 : buf - 1);
    const int kb = k0 + j * kKT;
    if (g.wave_active) {
      const float *xs = smem_f + buf * S::kTile;
      f32x4 s2[2], dp2[2];
#pragma unroll
      for (int e = 0; e < 2; ++e) s2[e] = dp2[e] = f32x4{0.f, 0.f, 0.f, 0.f};
      const float *xa = xs + l16 * XS + Q * lq;
#pragma unroll
      for (int i4 = 0; i4 < Q / 4; ++i4) {
        const f32x4 xv = *reinterpret_cast<const f32x4 *>(xa + 4 * i4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          s2[e & 1] = mma4(xv[e], uf[4 * i4 + e], s2[e & 1]);
          dp2[e & 1] = mma4(xv[e], df[4 * i4 + e], dp2[e & 1]);
        }
      }
      const f32x4 s = s2[0] + s2[1], dp = dp2[0] + dp2[1];
      float p[4], ds[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const bool ok = kb + 4 * lq + r < k1;
        p[r] = ok ? fast_exp2(__builtin_fmaf(s[r], c, -L)) : 0.f;
        ds[r] = p[r] * (dp[r] - Dl);
      }
#pragma unroll
      for (int j4 = 0; j4 < 4; ++j4) {
        const float *xt = xs + (4 * lq + j4) * XS + 4 * l16;
#pragma unroll
        for (int a = 0; a < NA; ++a) {
          const f32x4 xv = *reinterpret_cast<const f32x4 *>(xt + 64 * (a0 + a));
#pragma unroll
          for (int b = 0; b < 4; ++b) {
            adu[a][b] = mma4(xv[b], ds[j4], adu[a][b]);
            aax[a][b] = mma4(xv[b], p[j4], aax[a][b]);
          }
        }
      }
    }
    buf = buf == kNBuf - 1 ? 0 : buf + 1;
  }
  wait_vmcnt<0>();
  if (!g.wave_active || !g.row_ok) return;
  // lane: row grow, features 64a + 16*lq + 4r + b (b = 0..3 consecutive)
#pragma unroll
  for (int a = 0; a < NA; ++a)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int f = 64 * (a0 + a) + 16 * lq + 4 * r;
      if (f >= F) continue;
      f32x4 wu, wa;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        wu[b] = adu[a][b][r] * scale;
        wa[b] = aax[a][b][r];
      }
      *reinterpret_cast<f32x4 *>(du + grow * F + f) = wu;
      *reinterpret_cast<f32x4 *>(ax_ws + grow * F + f) = wa;
    }
}

// ---------------------------------------------------------------------------
// Backward, key side (ta/kernels.py:528-900): item {k0, k1, t0, t1, ...}
// covers up to 512 keys of one sample and all of its (token, head) rows
// R = t*H + h in [t0*H, t1*H):
//   dX_j = sum_R (scale * dS_Rj u_R + P_Rj dAX_R),
// summed over rows and heads in registers in a fixed order.  Each pass gives
// every wave 16 keys (their X rows are the B operand, in registers); the rows
// stream through LDS in blocks of 32 with their LSE and delta.
// ---------------------------------------------------------------------------
// two workgroups per CU; one at FP = 512 (X operands and dX accumulators
// take 256 registers)
template <int FP>
__global__ __launch_bounds__(256, FP > 256 ? 1 : 2) void absorb_dx_f32_kernel(
    const float *__restrict__ u, const float *__restrict__ X, const float *__restrict__ lse,
    const float *__restrict__ delta, const float *__restrict__ dax, float *__restrict__ dX,
    const int32_t *__restrict__ items, int H, int F, float c, float scale) {
  using S = F32Smem<FP>;
  constexpr int Q = FP / 4, NA = FP / 64, XS = S::XS;
  extern __shared__ __align__(16) float smem_f[];
  float *us = smem_f;                    // [kRBlk][XS] u rows
  float *ds_ = smem_f + kRBlk * XS;      // [kRBlk][XS] dAX rows
  float *lsd = smem_f + 2 * kRBlk * XS;  // [kRBlk] LSE, then [kRBlk] delta

  const PlanItem it = load_item(items, blockIdx.x);
  const int k0 = it.v[0], k1 = it.v[1], t0 = it.v[2], t1 = it.v[3];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, lq = lane >> 4;
  const int64_t R0 = (int64_t)t0 * H;
  const int nrows = (t1 - t0) * H;
  const int nblk = (nrows + kRBlk - 1) / kRBlk;

  for (int kp = k0; kp < k1; kp += 64) {
    const int kw = kp + wave * 16;  // this wave's 16 keys
    // X rows of the wave's keys (B operand): key kw + l16, features Q*lq..
    float xf[Q];
    {
      const int nk = k1 - kw;
      const rsrc_t rx = make_rsrc(X + (int64_t)kw * F, (int64_t)(nk > 0 ? nk : 0) * F * 4);
      load_quarter<FP>(xf, rx, l16 * F * 4, F, lq);
    }
    f32x4 acc[NA][4];
#pragma unroll
    for (int a = 0; a < NA; ++a)
#pragma unroll
      for (int b = 0; b < 4; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int rb = 0; rb < nblk; ++rb) {
      const int r0 = rb * kRBlk;
      const int rows = nrows - r0 < kRBlk ? nrows - r0 : kRBlk;
      __syncthreads();  // every wave is done with the previous block
      dma_rows_f32<FP, 4, kRBlk, XS>(u + (R0 + r0) * F, (int64_t)rows * F * 4, F, lds_addr(us),
                                     wave, lane);
      dma_rows_f32<FP, 4, kRBlk, XS>(dax + (R0 + r0) * F, (int64_t)rows * F * 4, F,
                                     lds_addr(ds_), wave, lane);
      if (wave < 2 && lane < kRBlk) {
        const float *vec = wave == 0 ? lse : delta;
        lds_dma4(rsrc_words(vec + R0 + r0, (int64_t)rows * 4), lds_addr(lsd + wave * kRBlk),
                 lane * 4);
      }
      wait_vmcnt<0>();
      __syncthreads();
      if (kw >= k1) continue;
#pragma unroll
      for (int half = 0; half < kRBlk / 16; ++half) {
        // S (16 rows x 16 keys), lane holds row 4*lq + r of the half, key
        // kw + l16; rows past the segment are zero (their dAX too, so they
        // add nothing)
        f32x4 s2[2], dp2[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) s2[e] = dp2[e] = f32x4{0.f, 0.f, 0.f, 0.f};
        const float *ua = us + (half * 16 + l16) * XS + Q * lq;
        const float *da = ds_ + (half * 16 + l16) * XS + Q * lq;
#pragma unroll
        for (int i4 = 0; i4 < Q / 4; ++i4) {
          const f32x4 uv = *reinterpret_cast<const f32x4 *>(ua + 4 * i4);
          const f32x4 dv = *reinterpret_cast<const f32x4 *>(da + 4 * i4);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            s2[e & 1] = mma4(uv[e], xf[4 * i4 + e], s2[e & 1]);
            dp2[e & 1] = mma4(dv[e], xf[4 * i4 + e], dp2[e & 1]);
          }
        }
        const f32x4 s = s2[0] + s2[1], dp = dp2[0] + dp2[1];
        const f32x4 L = *reinterpret_cast<const f32x4 *>(lsd + half * 16 + 4 * lq);
        const f32x4 Dl = *reinterpret_cast<const f32x4 *>(lsd + kRBlk + half * 16 + 4 * lq);
        float p[4], dsc[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          p[r] = fast_exp2(__builtin_fmaf(s[r], c, -L[r]));
          dsc[r] = p[r] * (dp[r] - Dl[r]) * scale;
        }
        // dX^T (f x keys) += u^T dS^T + dAX^T P^T over the half's rows in 4
        // slices (slot lq <-> row 4*lq + j4)
#pragma unroll
        for (int j4 = 0; j4 < 4; ++j4) {
          const float *ut = us + (half * 16 + 4 * lq + j4) * XS + 4 * l16;
          const float *dt = ds_ + (half * 16 + 4 * lq + j4) * XS + 4 * l16;
#pragma unroll
          for (int a = 0; a < NA; ++a) {
            const f32x4 uv = *reinterpret_cast<const f32x4 *>(ut + 64 * a);
            const f32x4 dv = *reinterpret_cast<const f32x4 *>(dt + 64 * a);
#pragma unroll
            for (int b = 0; b < 4; ++b) {
              acc[a][b] = mma4(uv[b], dsc[j4], acc[a][b]);
              acc[a][b] = mma4(dv[b], p[j4], acc[a][b]);
            }
          }
        }
      }
    }
    // lane: key kw + l16, features 64a + 16*lq + 4r + b
    const int key = kw + l16;
    if (key < k1) {
#pragma unroll
      for (int a = 0; a < NA; ++a)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int f = 64 * a + 16 * lq + 4 * r;
          if (f >= F) continue;
          f32x4 w;
#pragma unroll
          for (int b = 0; b < 4; ++b) w[b] = acc[a][b][r];
          *reinterpret_cast<f32x4 *>(dX + (int64_t)key * F + f) = w;
        }
    }
  }
}

template <int FP>
void launch_fwd_fp(const AbsorbArgs &a, const float *wvt, hipStream_t st) {
  const int smem = F32Smem<FP>::kFwdBytes;
  allow_dynamic_lds(reinterpret_cast<const void *>(&absorb_fwd_f32_kernel<FP>), smem);
  hipLaunchKernelGGL(absorb_fwd_f32_kernel<FP>, dim3((unsigned)a.n_items), dim3(256), smem, st,
                     (const float *)a.u, (const float *)a.X, wvt, (float *)a.O, a.lse, a.part_o,
                     a.part_lse, a.items, a.H, a.F, a.DH, a.scale * kLog2e);
}

template <int FP>
void launch_bwd_fp(const AbsorbArgs &a, hipStream_t st) {
  if (a.n_qseg > 0) {
    const int smem = F32Smem<FP>::kFwdBytes;
    allow_dynamic_lds(reinterpret_cast<const void *>(&absorb_du_f32_kernel<FP>), smem);
    const int64_t grid = FP > 256 ? (a.n_qseg + 7) / 8 * 16 : a.n_qseg;
    hipLaunchKernelGGL(absorb_du_f32_kernel<FP>, dim3((unsigned)grid), dim3(256), smem, st,
                       (const float *)a.u, (const float *)a.X, a.lse_in, a.delta,
                       (const float *)a.dax, (float *)a.du, a.ax, a.qseg_items, (int)a.n_qseg,
                       a.H, a.F, a.scale * kLog2e, a.scale);
  }
  if (a.n_kv > 0) {
    const int smem = F32Smem<FP>::kDxBytes;
    allow_dynamic_lds(reinterpret_cast<const void *>(&absorb_dx_f32_kernel<FP>), smem);
    hipLaunchKernelGGL(absorb_dx_f32_kernel<FP>, dim3((unsigned)a.n_kv), dim3(256), smem, st,
                       (const float *)a.u, (const float *)a.X, a.lse_in, a.delta,
                       (const float *)a.dax, (float *)a.dX, a.kv_items, a.H, a.F,
                       a.scale * kLog2e, a.scale);
  }
}

}  // namespace

// The fp32 matrix-core path takes H <= 64 (floor(64/H) tokens per forward /
// du workgroup), D_KV a multiple of 4 up to 256 (padded to a multiple of 64
// inside the kernels; up to 512 in the forward, padded to 512) and D_H a
// multiple of 16 up to 256.
namespace {

// dAX[t,h,f] = sum_d dO[t,h,d] W_V[f,h,d] in fp32 (ta/kernels.py:474-476, an
// IEEE dot there): one wave per (32 tokens, head, 64 f) on 16x16x4 fp32
// products, C[token][f] accumulated over 32-wide d blocks.  The reduction
// order is relabelled (k step ks, slot l/16 <-> d = 32*blk + 8*(l/16) + ks) so
// every operand comes from two contiguous 16-byte loads per lane: dO rows (A)
// and W_V rows (B).  The wave's [32, 64] block is staged in LDS and written
// as 16-byte row runs.
__global__ __launch_bounds__(64) void absorb_dax_f32_kernel(const float *__restrict__ dO,
                                                            const float *__restrict__ wv,
                                                            float *__restrict__ dax, int64_t T_q,
                                                            int H, int F, int DH) {
  const int lane = threadIdx.x, l16 = lane & 15, lq = lane >> 4;
  const int nfg = (F + 63) / 64;
  int64_t w = blockIdx.x;
  const int fg = (int)(w % nfg);
  w /= nfg;
  const int h = (int)(w % H);
  const int64_t t0 = (w / H) * 32;
  const int f0 = fg * 64;
  f32x4 acc[2][4];
#pragma unroll
  for (int hf = 0; hf < 2; ++hf)
#pragma unroll
    for (int ft = 0; ft < 4; ++ft) acc[hf][ft] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int db = 0; db < DH; db += 32) {
    const int d = db + 8 * lq;
    float a[2][8], b[4][8];
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const int64_t t = t0 + hf * 16 + l16;
      const bool ok = t < T_q && d < DH;
      const float *src = dO + (ok ? (t * H + h) * DH + d : 0);
      const f32x4 x0 = *reinterpret_cast<const f32x4 *>(src);
      const f32x4 x1 = *reinterpret_cast<const f32x4 *>(src + 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        a[hf][e] = ok ? x0[e] : 0.f;
        a[hf][4 + e] = ok ? x1[e] : 0.f;
      }
    }
#pragma unroll
    for (int ft = 0; ft < 4; ++ft) {
      const int f = f0 + ft * 16 + l16;
      const bool ok = f < F && d < DH;
      const float *src = wv + (ok ? ((int64_t)f * H + h) * DH + d : 0);
      const f32x4 x0 = *reinterpret_cast<const f32x4 *>(src);
      const f32x4 x1 = *reinterpret_cast<const f32x4 *>(src + 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        b[ft][e] = ok ? x0[e] : 0.f;
        b[ft][4 + e] = ok ? x1[e] : 0.f;
      }
    }
#pragma unroll
    for (int ks = 0; ks < 8; ++ks)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf)
#pragma unroll
        for (int ft = 0; ft < 4; ++ft) acc[hf][ft] = mma4(a[hf][ks], b[ft][ks], acc[hf][ft]);
  }
  // C: token 16*hf + 4*lq + r, f = f0 + 16*ft + l16
  __shared__ __align__(16) float st[32][64 + 4];
#pragma unroll
  for (int hf = 0; hf < 2; ++hf)
#pragma unroll
    for (int ft = 0; ft < 4; ++ft)
#pragma unroll
      for (int r = 0; r < 4; ++r) st[hf * 16 + 4 * lq + r][ft * 16 + l16] = acc[hf][ft][r];
  __syncthreads();
  const int rr = lane >> 4, cc = (lane & 15) * 4;
  if (f0 + cc < F)
    for (int tk = rr; tk < 32; tk += 4) {
      const int64_t t = t0 + tk;
      if (t < T_q)
        *reinterpret_cast<f32x4 *>(dax + (t * H + h) * F + f0 + cc) =
            *reinterpret_cast<const f32x4 *>(&st[tk][cc]);
    }
}

}  // namespace

void launch_f32_absorb_dax(const AbsorbArgs &a, hipStream_t st) {
  const int64_t waves = (a.T_q + 31) / 32 * a.H * ((a.F + 63) / 64);
  if (waves == 0) return;
  hipLaunchKernelGGL(absorb_dax_f32_kernel, dim3((unsigned)waves), dim3(64), 0, st,
                     (const float *)a.dO, (const float *)a.wv, (float *)a.dax, a.T_q, a.H, a.F,
                     a.DH);
}

bool f32_absorb_fwd_supported(int H, int F, int DH) {
  return H >= 1 && H <= kAbsorbRows && F >= 4 && F % 4 == 0 && F <= 512 && DH >= 16 &&
         DH % 16 == 0 && DH <= 256;
}

bool f32_absorb_supported(int H, int F, int DH) { return f32_absorb_fwd_supported(H, F, DH); }

int64_t f32_absorb_wvt_elems(int H, int F, int DH) { return (int64_t)H * DH * fp64_of(F); }

void launch_f32_absorb_fwd(const AbsorbArgs &a, hipStream_t st) {
  const int FP = fp64_of(a.F);
  float *wvt = reinterpret_cast<float *>(a.wvt);
  const int64_t n = (int64_t)a.H * a.DH * FP;
  hipLaunchKernelGGL(transpose_wv_f32_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                     (const float *)a.wv, wvt, a.H, a.F, a.DH, FP);
  if (a.n_items == 0) return;
  switch (FP) {
    case 64: launch_fwd_fp<64>(a, wvt, st); break;
    case 128: launch_fwd_fp<128>(a, wvt, st); break;
    case 192: launch_fwd_fp<192>(a, wvt, st); break;
    case 256: launch_fwd_fp<256>(a, wvt, st); break;
    case 512: launch_fwd_fp<512>(a, wvt, st); break;
    default: break;
  }
}

void launch_f32_absorb_du_dx(const AbsorbArgs &a, hipStream_t st) {
  switch (fp64_of(a.F)) {
    case 64: launch_bwd_fp<64>(a, st); break;
    case 128: launch_bwd_fp<128>(a, st); break;
    case 192: launch_bwd_fp<192>(a, st); break;
    case 256: launch_bwd_fp<256>(a, st); break;
    case 512: launch_bwd_fp<512>(a, st); break;
    default: break;
  }
}

}  // namespace vafa
