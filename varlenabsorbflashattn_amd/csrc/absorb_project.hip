// Projections of packed_target_attn around the absorbed attention
// (ta/interface.py:434-435: q_proj = q_raw W_Q, u = einsum('thd,khd->thk',
// q_proj, W_K)) and their backward, which the reference leaves to torch
// autograd.  Every product here is an "NT" row GEMM with the reduction index
// contiguous in both operands,
//     Y[t, g*ys + j] = sum_k X[t*ldx + g*xs + k] * W[g*ws + j*ldw + k],
// over groups g (the heads, or one group):
//   q_proj  = q_raw   . W_Q       X = q_raw [T, DQ],        W = W_Q^T [HD, DQ]
//   u       = q_proj  . W_K,h^T   X = q_proj [T, H, DH],    W = W_K [F, H, DH]
//   dq_proj = du      . W_K,h     X = du [T, H, F],          W = W_K^T [H, DH, F]
//   dq_raw  = dq_proj . W_Q^T     X = dq_proj [T, HD],       W = W_Q [DQ, HD]
// (HD = H*DH), fp32 accumulation and one rounding to the input dtype, as the
// reference's 16-bit GEMMs.  The weight gradients dW_K = sum_t du^T q_proj
// per head and dW_Q = sum_t q_raw^T dq_proj are token reductions and run on
// the chunked, ordered (deterministic) reduction of dW_V.
#include "absorb_tiles.h"

namespace vafa {

namespace {

using namespace absorb;

constexpr int kRgTok = 32;  // tokens per workgroup

// One workgroup (4 waves) computes a 32-token x 64*NJ-column block of Y for
// one group.  The 32 X rows of each 32*KS-wide reduction block are staged in
// LDS by contiguous 16-byte loads (each wave instruction covers whole row
// segments); each wave then runs Y^T = W X^T over its 16*NJ columns on
// 16x16x32 products, its W rows (the A operand, 8 consecutive k per lane)
// loaded straight from global memory before the block's barrier, the tokens
// (the B operand) read from LDS.  The result is rounded, staged in LDS and
// written back as contiguous 16-byte row segments.
template <typename T, int NJ, int KS>
__global__ __launch_bounds__(256) void rowgemm_nt_kernel(
    const T *__restrict__ X, const T *__restrict__ W, T *__restrict__ Y, int64_t T_q, int G,
    int J, int K, int64_t ldx, int64_t xs, int64_t ws, int64_t ldw, int64_t ldy, int64_t ys,
    int n_jb) {
  using M16 = Mfma16<T>;
  constexpr int kKBlk = 32 * KS;     // reduction block staged in LDS
  constexpr int kRgXS = kKBlk + 16;  // padded LDS row stride of the X block
  constexpr int kJB = 64 * NJ;       // columns per workgroup
  constexpr int kYS = kJB + 8;       // padded LDS row stride of the Y block
  constexpr int kSmem = kRgTok * (kRgXS > kYS ? kRgXS : kYS);
  __shared__ __align__(16) T smem[kSmem];
  const int tid = threadIdx.x, lane = tid & 63, l16 = lane & 15, lq = lane >> 4;
  const int wave = tid >> 6;
  int64_t b = blockIdx.x;
  const int jb = (int)(b % n_jb);
  b /= n_jb;
  const int g = (int)(b % G);
  const int64_t tb = (b / G) * kRgTok;
  const T *xg = X + g * xs;
  const T *wg = W + g * ws;
  // this wave's W rows
  int jrow[NJ];
  bool j_ok[NJ];
#pragma unroll
  for (int n = 0; n < NJ; ++n) {
    const int j = jb * kJB + wave * 16 * NJ + n * 16 + l16;
    j_ok[n] = j < J;
    jrow[n] = j_ok[n] ? j : 0;
  }
  f32x4 acc[NJ][2];
#pragma unroll
  for (int n = 0; n < NJ; ++n)
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) acc[n][hf] = f32x4{0.f, 0.f, 0.f, 0.f};
  constexpr int kCh = kKBlk / 8;  // 16-byte chunks per staged row
  for (int kb = 0; kb < K; kb += kKBlk) {
    // W operands of the block (issued before the X block lands)
    u32x4 wa[NJ][KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int k = kb + ks * 32 + lq * 8;
#pragma unroll
      for (int n = 0; n < NJ; ++n) {
        // branch-free: a clamped in-range load, then the select
        const bool ok = k < K && j_ok[n];
        const u32x4 v = *reinterpret_cast<const u32x4 *>(wg + (ok ? (int64_t)jrow[n] * ldw + k : 0));
        wa[n][ks] = ok ? v : u32x4{0u, 0u, 0u, 0u};
      }
    }
    if (kb > 0) __syncthreads();  // every wave is done with the previous block
    for (int idx = tid; idx < kRgTok * kCh; idx += 256) {
      const int r = idx / kCh, c = idx % kCh;
      const int64_t t = tb + r;
      const int k = kb + c * 8;
      u32x4 v = {0u, 0u, 0u, 0u};
      if (t < T_q && k < K) v = *reinterpret_cast<const u32x4 *>(xg + t * ldx + k);
      *reinterpret_cast<u32x4 *>(smem + r * kRgXS + c * 8) = v;
    }
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      u32x4 xb[2];
#pragma unroll
      for (int hf = 0; hf < 2; ++hf)
        xb[hf] = *reinterpret_cast<const u32x4 *>(smem + (hf * 16 + l16) * kRgXS + ks * 32 + lq * 8);
#pragma unroll
      for (int n = 0; n < NJ; ++n)
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
          acc[n][hf] = M16::mma(as_v8<T>(wa[n][ks]), as_v8<T>(xb[hf]), acc[n][hf]);
    }
  }
  __syncthreads();  // the X block is dead: its LDS holds the Y block next
  typedef __attribute__((__vector_size__(4 * sizeof(T)))) T T4;
  // lane: columns wave*16NJ + 16n + 4lq + r of token 16hf + l16
#pragma unroll
  for (int n = 0; n < NJ; ++n)
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      T4 o;
#pragma unroll
      for (int r = 0; r < 4; ++r) o[r] = static_cast<T>(acc[n][hf][r]);
      *reinterpret_cast<T4 *>(smem + (hf * 16 + l16) * kYS + wave * 16 * NJ + n * 16 + lq * 4) = o;
    }
  __syncthreads();
  const int jn = J - jb * kJB < kJB ? J - jb * kJB : kJB;
  constexpr int kYCh = kJB / 8;
#pragma unroll
  for (int i = 0; i < kRgTok * kYCh / 256; ++i) {
    const int idx = i * 256 + tid, r = idx / kYCh, c = idx % kYCh;
    const int64_t t = tb + r;
    if (t < T_q && c * 8 < jn)
      *reinterpret_cast<u32x4 *>(Y + t * ldy + g * ys + jb * kJB + c * 8) =
          *reinterpret_cast<const u32x4 *>(smem + r * kYS + c * 8);
  }
}

// K <= 256: one workgroup walks tiles_per_wg consecutive 32-token tiles of
// one (group, column block) with its W operands loaded once into registers;
// X tiles go through a double-buffered LDS ring (the next tile's 16-byte
// loads held in registers under the current tile's products), and each
// tile's Y block is staged in LDS and stored while the next X tile lands.
template <typename T, int NJ, int KS>
__global__ __launch_bounds__(256) void rowgemm_tiles_kernel(
    const T *__restrict__ X, const T *__restrict__ W, T *__restrict__ Y, int64_t T_q, int G,
    int J, int K, int64_t ldx, int64_t xs, int64_t ws, int64_t ldw, int64_t ldy, int64_t ys,
    int n_jb, int tiles_per_wg, int64_t n_tt) {
  using M16 = Mfma16<T>;
  constexpr int kKBlk = 32 * KS;
  constexpr int kXS = kKBlk + 16;
  constexpr int kJB = 64 * NJ;
  constexpr int kYS = kJB + 8;
  constexpr int kXElems = kRgTok * kXS;
  __shared__ __align__(16) T smem[2 * kXElems + kRgTok * kYS];
  T *ystage = smem + 2 * kXElems;
  const int tid = threadIdx.x, lane = tid & 63, l16 = lane & 15, lq = lane >> 4;
  const int wave = tid >> 6;
  int64_t b = blockIdx.x;
  const int jb = (int)(b % n_jb);
  b /= n_jb;
  const int g = (int)(b % G);
  const int64_t tt0 = (b / G) * tiles_per_wg;
  const int64_t tt1 = tt0 + tiles_per_wg < n_tt ? tt0 + tiles_per_wg : n_tt;
  const T *xg = X + g * xs;
  const T *wg = W + g * ws;

  // this wave's W operands, loaded once (branch-free: clamped, then zeroed)
  u32x4 wa[NJ][KS];
#pragma unroll
  for (int n = 0; n < NJ; ++n) {
    const int j = jb * kJB + wave * 16 * NJ + n * 16 + l16;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int k = ks * 32 + lq * 8;
      const bool ok = k < K && j < J;
      const u32x4 v = *reinterpret_cast<const u32x4 *>(wg + (ok ? (int64_t)j * ldw + k : 0));
      wa[n][ks] = ok ? v : u32x4{0u, 0u, 0u, 0u};
    }
  }
  constexpr int kCh = kKBlk / 8;                          // 16-byte chunks per X row
  constexpr int kXPer = (kRgTok * kCh + 255) / 256;       // per thread
  u32x4 rx[kXPer];
  auto load_x = [&](int64_t tt) {
#pragma unroll
    for (int i = 0; i < kXPer; ++i) {
      const int idx = i * 256 + tid, r = (idx / kCh) & (kRgTok - 1), c = idx % kCh;
      const int64_t t = tt * kRgTok + r;
      const bool ok = idx < kRgTok * kCh && t < T_q && c * 8 < K;
      const u32x4 v = *reinterpret_cast<const u32x4 *>(xg + (ok ? t * ldx + c * 8 : 0));
      rx[i] = ok ? v : u32x4{0u, 0u, 0u, 0u};
    }
  };
  auto store_x = [&](int buf) {
#pragma unroll
    for (int i = 0; i < kXPer; ++i) {
      const int idx = i * 256 + tid;
      if (idx < kRgTok * kCh)
        *reinterpret_cast<u32x4 *>(smem + buf * kXElems + (idx / kCh) * kXS + (idx % kCh) * 8) =
            rx[i];
    }
  };
  typedef __attribute__((__vector_size__(4 * sizeof(T)))) T T4;
  constexpr int kYCh = kJB / 8;
  const int jn = J - jb * kJB < kJB ? J - jb * kJB : kJB;
  if (tt0 < tt1) {
    load_x(tt0);
    store_x(0);
  }
  __syncthreads();
  for (int64_t tt = tt0; tt < tt1; ++tt) {
    const int buf = (int)((tt - tt0) & 1);
    if (tt + 1 < tt1) load_x(tt + 1);
    f32x4 acc[NJ][2];
#pragma unroll
    for (int n = 0; n < NJ; ++n)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) acc[n][hf] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      u32x4 xb[2];
#pragma unroll
      for (int hf = 0; hf < 2; ++hf)
        xb[hf] = *reinterpret_cast<const u32x4 *>(smem + buf * kXElems + (hf * 16 + l16) * kXS +
                                                  ks * 32 + lq * 8);
#pragma unroll
      for (int n = 0; n < NJ; ++n)
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
          acc[n][hf] = M16::mma(as_v8<T>(wa[n][ks]), as_v8<T>(xb[hf]), acc[n][hf]);
    }
    // lane: columns wave*16NJ + 16n + 4lq + r of token 16hf + l16
#pragma unroll
    for (int n = 0; n < NJ; ++n)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        T4 o;
#pragma unroll
        for (int r = 0; r < 4; ++r) o[r] = static_cast<T>(acc[n][hf][r]);
        *reinterpret_cast<T4 *>(ystage + (hf * 16 + l16) * kYS + wave * 16 * NJ + n * 16 +
                                lq * 4) = o;
      }
    __syncthreads();  // Y block staged; every wave is done with X buffer buf
#pragma unroll
    for (int i = 0; i < kRgTok * kYCh / 256; ++i) {
      const int idx = i * 256 + tid, r = idx / kYCh, c = idx % kYCh;
      const int64_t t = tt * kRgTok + r;
      if (t < T_q && c * 8 < jn)
        *reinterpret_cast<u32x4 *>(Y + t * ldy + g * ys + jb * kJB + c * 8) =
            *reinterpret_cast<const u32x4 *>(ystage + r * kYS + c * 8);
    }
    if (tt + 1 < tt1) store_x(buf ^ 1);
    __syncthreads();  // next X tile visible; the Y block is read out
  }
}

// Weight gradient of a projection on 16-bit matrix cores, one workgroup per
// (token chunk c, group g, 32-column block of d):
//   part[c, f, g, d] = sum_{t in chunk c} A[t, g, f] B[t, g, d]
// (dW_K: A = du [T, H, F], B = q_proj [T, H, DH]; dW_Q: one group, A = q_raw,
// B = dq_proj), and with DQ also the input gradient of the same A rows,
//   dq[t, g, d] = sum_f A[t, g, f] Wt[g, d, f]   (dq_proj = du W_K per head),
// so du is read once for both.  32-token tiles of A and B are staged in a
// double-buffered LDS ring (contiguous 16-byte row loads held in registers
// while the current tile is consumed; zeros past the chunk and past F); the
// token reduction reads both operands transposed (ds_read_b64_tr_b16: lane
// l gets column 16*tile + l%16 at tokens 4*(l/16) + 0..3 and 16 + 4*(l/16) +
// 0..3, the same token order for A and B), the dq product reads A rows as
// the B operand of dq^T = Wt A^T with this wave's Wt rows in registers.
constexpr int kWgTok = 32;          // tokens per tile
constexpr int kWgDB = 32;           // d columns per workgroup
constexpr int kWgBS = kWgDB + 16;   // padded LDS row stride of the B tile

template <int FP>
struct WgSmem {
  static constexpr int AS = FP + 16;                    // padded A row stride
  static constexpr int kStage = kWgTok * (AS + kWgBS);  // elements per stage
  static constexpr int kBytes = 2 * kStage * 2;
};

template <typename T, int FP, bool DQ>
__global__ __launch_bounds__(256) void wgrad_kernel(
    const T *__restrict__ A, const T *__restrict__ B, const T *__restrict__ Wt, T *__restrict__ dq,
    float *__restrict__ part, int64_t T_q, int64_t tchunk, int G, int F, int DH, int n_db) {
  using M16 = Mfma16<T>;
  using v8 = typename Mfma<T>::v8;
  using S = WgSmem<FP>;
  typedef __attribute__((__vector_size__(4 * sizeof(T)))) T T4;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  T *smem = reinterpret_cast<T *>(smem_raw);
  const int tid = threadIdx.x, lane = tid & 63, l16 = lane & 15, lq = lane >> 4;
  const int wave = tid >> 6;
  int64_t b = blockIdx.x;
  const int db = (int)(b % n_db);
  b /= n_db;
  const int g = (int)(b % G);
  const int64_t c = b / G;
  const int64_t ta = c * tchunk, tb = ta + tchunk < T_q ? ta + tchunk : T_q;
  const int d0 = db * kWgDB;
  const int dn = DH - d0 < kWgDB ? DH - d0 : kWgDB;

  constexpr int kACh = FP / 8;                    // 16-byte chunks per A row
  constexpr int kAPer = kWgTok * kACh / 256;      // A chunks per thread
  u32x4 ra[kAPer], rb = {0u, 0u, 0u, 0u};
  auto load = [&](int64_t t0) {
#pragma unroll
    for (int i = 0; i < kAPer; ++i) {
      const int idx = i * 256 + tid, r = idx / kACh, ch = idx % kACh;
      const int64_t t = t0 + r;
      const bool ok = t < tb && ch * 8 < F;
      const u32x4 v = *reinterpret_cast<const u32x4 *>(A + (ok ? (t * G + g) * F + ch * 8 : 0));
      ra[i] = ok ? v : u32x4{0u, 0u, 0u, 0u};
    }
    {
      const int r = (tid >> 2) & (kWgTok - 1), ch = tid & 3;
      const int64_t t = t0 + r;
      const bool ok = tid < kWgTok * 4 && t < tb && ch * 8 < dn;
      const u32x4 v = *reinterpret_cast<const u32x4 *>(
          B + (ok ? (t * G + g) * DH + d0 + ch * 8 : 0));
      rb = ok ? v : u32x4{0u, 0u, 0u, 0u};
    }
  };
  auto stage = [&](int s) {
    T *as = smem + s * S::kStage;
    T *bs = as + kWgTok * S::AS;
#pragma unroll
    for (int i = 0; i < kAPer; ++i) {
      const int idx = i * 256 + tid, r = idx / kACh, ch = idx % kACh;
      *reinterpret_cast<u32x4 *>(as + r * S::AS + ch * 8) = ra[i];
    }
    if (tid < kWgTok * 4)
      *reinterpret_cast<u32x4 *>(bs + (tid >> 2) * kWgBS + (tid & 3) * 8) = rb;
  };

  // dq: this wave's 16 d columns (d tile wave & 1) and 16 tokens (half wave >> 1)
  constexpr int kKs = FP / 32;
  const int dq_d = d0 + 16 * (wave & 1) + l16;
  const int dq_hf = wave >> 1;
  u32x4 wa[DQ ? kKs : 1];
  if constexpr (DQ) {
#pragma unroll
    for (int ks = 0; ks < kKs; ++ks) {
      // branch-free: a clamped in-range load, then the select (a load under
      // a branch makes the whole register array a phi of copies)
      const int k = ks * 32 + lq * 8;
      const bool ok = dq_d < DH && k < F;
      const u32x4 v = *reinterpret_cast<const u32x4 *>(
          Wt + (ok ? ((int64_t)g * DH + dq_d) * F + k : 0));
      wa[ks] = ok ? v : u32x4{0u, 0u, 0u, 0u};
    }
  }

  constexpr int kFt = FP / 64;  // f tiles per wave: wave + 4j
  f32x4 acc[kFt][2];
#pragma unroll
  for (int j = 0; j < kFt; ++j)
#pragma unroll
    for (int dt = 0; dt < 2; ++dt) acc[j][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int a_tr = (4 * lq + (l16 >> 2)) * S::AS + 4 * (l16 & 3);
  const int b_tr = (4 * lq + (l16 >> 2)) * kWgBS + 4 * (l16 & 3);
  const int nt = (int)((tb - ta + kWgTok - 1) / kWgTok);
  load(ta);
  stage(0);
  __syncthreads();
#pragma nounroll
  for (int i = 0; i < nt; ++i) {
    if (i + 1 < nt) load(ta + (int64_t)(i + 1) * kWgTok);
    const lds_cptr<T> as = as_lds(smem + (i & 1) * S::kStage);
    const lds_cptr<T> bs = as + kWgTok * S::AS;
    v8 bop[2];
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
      bop[dt] = as_v8<T>(join(lds_tr8<T>(bs + b_tr + 16 * dt),
                              lds_tr8<T>(bs + b_tr + 16 * kWgBS + 16 * dt)));
#pragma unroll
    for (int j = 0; j < kFt; ++j) {
      const int ft = wave + 4 * j;
      const v8 aop = as_v8<T>(join(lds_tr8<T>(as + a_tr + 16 * ft),
                                   lds_tr8<T>(as + a_tr + 16 * S::AS + 16 * ft)));
#pragma unroll
      for (int dt = 0; dt < 2; ++dt) acc[j][dt] = M16::mma(aop, bop[dt], acc[j][dt]);
    }
    if constexpr (DQ) {
      f32x4 q = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < kKs; ++ks) {
        const u32x4 x = lds_ld16<T>(as + (16 * dq_hf + l16) * S::AS + ks * 32 + lq * 8);
        q = M16::mma(as_v8<T>(wa[ks]), as_v8<T>(x), q);
      }
      // q^T: d = d0 + 16*(wave & 1) + 4*lq + r, token 16*dq_hf + l16 of the tile
      const int64_t t = ta + (int64_t)i * kWgTok + 16 * dq_hf + l16;
      const int dd = d0 + 16 * (wave & 1) + 4 * lq;
      if (t < tb && dd < DH) {
        T4 o;
#pragma unroll
        for (int r = 0; r < 4; ++r) o[r] = static_cast<T>(q[r]);
        *reinterpret_cast<T4 *>(dq + (t * G + g) * DH + dd) = o;
      }
    }
    if (i + 1 < nt) stage((i + 1) & 1);
    __syncthreads();
  }
  // C[f][d]: f = 16*ft + 4*lq + r, d = d0 + 16*dt + l16
#pragma unroll
  for (int j = 0; j < kFt; ++j)
#pragma unroll
    for (int dt = 0; dt < 2; ++dt) {
      const int d = 16 * dt + l16;
      if (d >= dn) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int f = 16 * (wave + 4 * j) + 4 * lq + r;
        if (f < F) part[((c * F + f) * G + g) * DH + d0 + d] = acc[j][dt][r];
      }
    }
}

// dst[c, r] = src[r, c] for a [R, C] matrix.
template <typename T>
__global__ __launch_bounds__(256) void transpose2d_kernel(const T *__restrict__ src,
                                                          T *__restrict__ dst, int R, int C) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)R * C) return;
  const int r = (int)(i % R), c = (int)(i / R);
  dst[i] = src[(int64_t)r * C + c];
}

// Workgroups of the tile-walking row GEMM: about this many in all.
constexpr int64_t kRgTargetWgs = 512;

template <typename T, int NJ, int KS>
void rowgemm_nj(const RowGemm &p, hipStream_t st) {
  const int n_jb = (p.J + 64 * NJ - 1) / (64 * NJ);
  const int64_t n_tt = (p.T_q + kRgTok - 1) / kRgTok;
  if (n_tt == 0) return;
  if (p.K <= 256) {
    const int64_t units = n_tt * p.G * n_jb;
    int64_t tpw = units / kRgTargetWgs;
    tpw = tpw < 1 ? 1 : (tpw > 16 ? 16 : tpw);
    const int64_t wgs = (n_tt + tpw - 1) / tpw * p.G * n_jb;
    hipLaunchKernelGGL((rowgemm_tiles_kernel<T, NJ, KS>), dim3((unsigned)wgs), dim3(256), 0, st,
                       (const T *)p.X, (const T *)p.W, (T *)p.Y, p.T_q, p.G, p.J, p.K, p.ldx,
                       p.xs, p.ws, p.ldw, p.ldy, p.ys, n_jb, (int)tpw, n_tt);
    return;
  }
  const int64_t wgs = n_tt * p.G * n_jb;
  hipLaunchKernelGGL((rowgemm_nt_kernel<T, NJ, KS>), dim3((unsigned)wgs), dim3(256), 0, st,
                     (const T *)p.X, (const T *)p.W, (T *)p.Y, p.T_q, p.G, p.J, p.K, p.ldx, p.xs,
                     p.ws, p.ldw, p.ldy, p.ys, n_jb);
}

template <typename T, int NJ>
void rowgemm_ks(const RowGemm &p, hipStream_t st) {
  if (p.K <= 32) rowgemm_nj<T, NJ, 1>(p, st);
  else if (p.K <= 64) rowgemm_nj<T, NJ, 2>(p, st);
  else if (p.K <= 128) rowgemm_nj<T, NJ, 4>(p, st);
  else rowgemm_nj<T, NJ, 8>(p, st);
}

template <typename T, int FP>
void wgrad_fp(const Wgrad &p, hipStream_t st) {
  const int n_db = (p.DH + kWgDB - 1) / kWgDB;
  const int64_t wgs = p.n_chunks * p.G * n_db;
  if (wgs == 0) return;
  constexpr int smem = WgSmem<FP>::kBytes;
  if (p.dq != nullptr) {
    allow_dynamic_lds(reinterpret_cast<const void *>(&wgrad_kernel<T, FP, true>), smem);
    hipLaunchKernelGGL((wgrad_kernel<T, FP, true>), dim3((unsigned)wgs), dim3(256), smem, st,
                       (const T *)p.A, (const T *)p.B, (const T *)p.Wt, (T *)p.dq, p.part, p.T_q,
                       p.tchunk, p.G, p.F, p.DH, n_db);
  } else {
    allow_dynamic_lds(reinterpret_cast<const void *>(&wgrad_kernel<T, FP, false>), smem);
    hipLaunchKernelGGL((wgrad_kernel<T, FP, false>), dim3((unsigned)wgs), dim3(256), smem, st,
                       (const T *)p.A, (const T *)p.B, nullptr, nullptr, p.part, p.T_q,
                       p.tchunk, p.G, p.F, p.DH, n_db);
  }
}

}  // namespace

bool rowgemm_supported(const RowGemm &p) {
  const bool pos = p.T_q >= 0 && p.G >= 1 && p.J >= 1 && p.K >= 8;
  const bool al = p.K % 8 == 0 && p.J % 8 == 0 && p.ldx % 8 == 0 && p.xs % 8 == 0 &&
                  p.ws % 8 == 0 && p.ldw % 8 == 0 && p.ldy % 8 == 0 && p.ys % 8 == 0;
  return pos && al;
}

// Widest column block (256, 128 or 64) that still gives at least 1024
// workgroups (four per CU), else the narrowest.
template <typename T>
void launch_rowgemm(const RowGemm &p, hipStream_t st) {
  const int64_t tiles = (p.T_q + kRgTok - 1) / kRgTok * p.G;
  auto wgs = [&](int jb) { return tiles * ((p.J + jb - 1) / jb); };
  if (wgs(256) >= 1024) rowgemm_ks<T, 4>(p, st);
  else if (wgs(128) >= 1024) rowgemm_ks<T, 2>(p, st);
  else rowgemm_ks<T, 1>(p, st);
}

bool wgrad16_supported(int F) { return F >= 8 && F <= 512 && F % 8 == 0; }

template <typename T>
void launch_wgrad16(const Wgrad &p, hipStream_t st) {
  if (p.F <= 64) wgrad_fp<T, 64>(p, st);
  else if (p.F <= 128) wgrad_fp<T, 128>(p, st);
  else if (p.F <= 256) wgrad_fp<T, 256>(p, st);
  else wgrad_fp<T, 512>(p, st);
  launch_chunk_sum<T>(p.part, p.out, (int64_t)p.F * p.G * p.DH, p.n_chunks, st);
}

template <typename T>
void launch_transpose2d(const void *src, void *dst, int R, int C, hipStream_t st) {
  const int64_t n = (int64_t)R * C;
  if (n == 0) return;
  hipLaunchKernelGGL(transpose2d_kernel<T>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                     (const T *)src, (T *)dst, R, C);
}

template void launch_rowgemm<bf16>(const RowGemm &, hipStream_t);
template void launch_rowgemm<f16>(const RowGemm &, hipStream_t);
template void launch_wgrad16<bf16>(const Wgrad &, hipStream_t);
template void launch_wgrad16<f16>(const Wgrad &, hipStream_t);
template void launch_transpose2d<bf16>(const void *, void *, int, int, hipStream_t);
template void launch_transpose2d<f16>(const void *, void *, int, int, hipStream_t);

}  // namespace vafa
