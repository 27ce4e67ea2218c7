// Small bandwidth-bound passes shared by both operators: the backward row
// dot (delta), the split-K merges and the absorb dAX / dW_V reductions.
// Every reduction runs in a fixed order, so results are bit-reproducible.
#include "common.h"
#include "kernels.h"
#include "plan_params.h"

namespace vafa {

namespace {

// delta[r] = sum_d o[r,d] * dout[r,d] in fp32 (fa/kernels.py:186-216,
// ta/kernels.py:298-325).  Each thread reads one 16-byte chunk of a row and
// sums it by fused multiply-adds in element order; the D/CH threads of a row
// reduce with a lane butterfly, so loads are coalesced.  The varlen dQ kernel
// reproduces this order when it forms delta itself.
template <typename T>
__global__ __launch_bounds__(256) void row_dot_kernel(const T *__restrict__ o,
                                                      const T *__restrict__ dout,
                                                      float *__restrict__ delta, int64_t rows,
                                                      int D) {
  constexpr int CH = 16 / sizeof(T);  // elements per 16-byte chunk
  const int tpr = D / CH;             // threads per row (power of two, <= 64)
  const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t r = g / tpr;
  const int part = (int)(g % tpr);
  float s = 0.f;
  if (r < rows) {
    const u32x4 a = *reinterpret_cast<const u32x4 *>(o + r * D + part * CH);
    const u32x4 b = *reinterpret_cast<const u32x4 *>(dout + r * D + part * CH);
    const T *x = reinterpret_cast<const T *>(&a);
    const T *y = reinterpret_cast<const T *>(&b);
#pragma unroll
    for (int e = 0; e < CH; ++e) s = __builtin_fmaf(to_f(x[e]), to_f(y[e]), s);
  }
  for (int off = tpr >> 1; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
  if (r < rows && part == 0) delta[r] = s;
}

// Split-K merges.  One wave per (row of a split tile, head) and kCombRows
// rows per block: the splits' LSEs are read one per lane, then the partial
// rows are streamed with the lanes along d and eight splits' loads in
// flight, accumulated in split order (a fixed order, so results repeat bit
// for bit).  A thread-per-element form re-reads every
// LSE per element and walks the splits with one dependent load at a time.
constexpr int kCombRows = 4;
constexpr int kCombMaxD = 256;                 // d = lane + 64 k, k < kCombMaxD / 64
constexpr int kCombBatch = 8;                  // split loads in flight per lane

// Log2-domain merge (fa/kernels.py:639-647):
//   m = max_s lse_s, w_s = exp2(lse_s - m), O = sum_s w_s O_s / sum_s w_s,
//   LSE = m + log2(sum_s w_s); all splits masked gives O = 0, LSE = -inf.
// RPW rows per wave: with D <= 32 each half-wave takes its own row, so a
// wave still moves 64 lanes' worth of every partial.
template <typename T, int RPW>
__global__ __launch_bounds__(64 * kCombRows) void lse_combine_kernel(
    const float *__restrict__ part_o, const float *__restrict__ part_lse, T *__restrict__ out,
    float *__restrict__ lse, const int32_t *__restrict__ items, int H, int D, int rblocks) {
  constexpr int CH = 64 / RPW;                           // lanes (and splits) per row group
  constexpr int KD = RPW == 1 ? kCombMaxD / 64 : 1;      // d = lg + CH k
  const int lane = threadIdx.x & 63;
  const int g = lane / CH, lg = lane % CH;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int rb = (int)blockIdx.x % rblocks, ih = (int)blockIdx.x / rblocks;
  const int item = ih / H, h = ih - item * H;
  const PlanItem it = load_item(items, item);
  const int q0 = it.v[0], q1 = it.v[1], pbase = it.v[2], ns = it.v[3];
  const int R = q1 - q0;
  const int r0 = (rb * kCombRows + wave) * RPW;  // the wave's first row
  if (r0 >= R) return;
  const int r = r0 + g;
  const bool row_ok = r < R;
  auto prow = [&](int sp) { return (int64_t)(pbase + sp * R + r) * H + h; };
  // lane g*CH + s of a chunk holds split s of row group g; readlane
  // broadcasts it (scalar, no LDS round trip) and keeps sums in split order
  auto bcast = [&](float x, int j) {
    float y = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), j));
    if (RPW == 2) {
      const float yb = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), CH + j));
      y = g ? yb : y;
    }
    return y;
  };
  auto load_batch = [&](int s0, int nc, int j0, float (&v)[kCombBatch][KD]) {
#pragma unroll
    for (int jj = 0; jj < kCombBatch; ++jj)
#pragma unroll
      for (int k = 0; k < KD; ++k) {
        const int d = lg + CH * k;
        v[jj][k] = (row_ok && j0 + jj < nc && d < D) ? part_o[prow(s0 + j0 + jj) * D + d] : 0.f;
      }
  };
  // The first chunk's LSEs and its first batch of partial rows are requested
  // together (the rows do not depend on the max), so a row with at most
  // kCombBatch splits costs one memory round trip.
  const int nc0 = ns < CH ? ns : CH;
  const float x0 = (row_ok && lg < nc0) ? part_lse[prow(lg)] : kNegInf;
  float v0[kCombBatch][KD];
  load_batch(0, nc0, 0, v0);
  float m = kNegInf;
  for (int jj = 0; jj < nc0; ++jj) m = fmaxf(m, bcast(x0, jj));
  for (int s0 = CH; s0 < ns; s0 += CH) {
    const int nc = ns - s0 < CH ? ns - s0 : CH;
    const float x = (row_ok && lg < nc) ? part_lse[prow(s0 + lg)] : kNegInf;
    for (int jj = 0; jj < nc; ++jj) m = fmaxf(m, bcast(x, jj));
  }
  const float ms = m == kNegInf ? 0.f : m;
  float acc[KD] = {};
  float l = 0.f;
  for (int s0 = 0; s0 < ns; s0 += CH) {
    const int nc = ns - s0 < CH ? ns - s0 : CH;
    const float x = s0 == 0 ? x0 : ((row_ok && lg < nc) ? part_lse[prow(s0 + lg)] : kNegInf);
    const float w = lg < nc ? fast_exp2(x - ms) : 0.f;
    for (int j0 = 0; j0 < nc; j0 += kCombBatch) {
      float v[kCombBatch][KD];
      if (s0 == 0 && j0 == 0) {
#pragma unroll
        for (int jj = 0; jj < kCombBatch; ++jj)
#pragma unroll
          for (int k = 0; k < KD; ++k) v[jj][k] = v0[jj][k];
      } else {
        load_batch(s0, nc, j0, v);
      }
#pragma unroll
      for (int jj = 0; jj < kCombBatch; ++jj) {
        if (j0 + jj >= nc) break;
        const float wj = bcast(w, j0 + jj);
        l += wj;
#pragma unroll
        for (int k = 0; k < KD; ++k) acc[k] += wj * v[jj][k];
      }
    }
  }
  if (!row_ok) return;
  const float ls = l == 0.f ? 1.f : l;
  const int64_t orow = (int64_t)(q0 + r) * H + h;
#pragma unroll
  for (int k = 0; k < KD; ++k) {
    const int d = lg + CH * k;
    if (d < D) out[orow * D + d] = from_f<T>(acc[k] / ls);
  }
  if (lg == 0) lse[orow] = m == kNegInf ? kNegInf : ms + fast_log2(ls);
}

// Ordered sum of split partials (dQ): out = sum_s part[s] (partials carry the
// softmax scale already).
template <typename T>
__global__ __launch_bounds__(64 * kCombRows) void sum_combine_kernel(
    const float *__restrict__ part, T *__restrict__ out, const int32_t *__restrict__ items, int H,
    int D, int rblocks) {
  constexpr int KD = kCombMaxD / 64;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int rb = (int)blockIdx.x % rblocks, ih = (int)blockIdx.x / rblocks;
  const int item = ih / H, h = ih - item * H;
  const PlanItem it = load_item(items, item);
  const int q0 = it.v[0], q1 = it.v[1], pbase = it.v[2], ns = it.v[3];
  const int R = q1 - q0;
  const int r = rb * kCombRows + wave;
  if (r >= R) return;
  float acc[KD] = {};
  for (int j0 = 0; j0 < ns; j0 += kCombBatch) {
    float v[kCombBatch][KD];
#pragma unroll
    for (int j = 0; j < kCombBatch; ++j)
#pragma unroll
      for (int k = 0; k < KD; ++k) {
        const int d = lane + 64 * k;
        v[j][k] = (j0 + j < ns && d < D)
                      ? part[((int64_t)(pbase + (j0 + j) * R + r) * H + h) * D + d]
                      : 0.f;
      }
#pragma unroll
    for (int j = 0; j < kCombBatch; ++j)
#pragma unroll
      for (int k = 0; k < KD; ++k) acc[k] += v[j][k];
  }
  const int64_t orow = (int64_t)(q0 + r) * H + h;
#pragma unroll
  for (int k = 0; k < KD; ++k) {
    const int d = lane + 64 * k;
    if (d < D) out[orow * D + d] = from_f<T>(acc[k]);
  }
}

// dAX[t,h,f] = sum_d dO[t,h,d] W_V[f,h,d]; one block per (t, h) row.
template <typename T>
__global__ __launch_bounds__(256) void absorb_dax_kernel(const T *__restrict__ dO,
                                                         const T *__restrict__ wv,
                                                         T *__restrict__ dax, int H, int F,
                                                         int DH) {
  const int64_t row = blockIdx.x;
  const int h = (int)(row % H);
  __shared__ float sdo[256];
  for (int d = threadIdx.x; d < DH; d += 256) sdo[d] = to_f(dO[row * DH + d]);
  __syncthreads();
  for (int f = threadIdx.x; f < F; f += 256) {
    const T *w = wv + ((int64_t)f * H + h) * DH;
    float s = 0.f;
    for (int d = 0; d < DH; ++d) s += sdo[d] * to_f(w[d]);
    dax[row * F + f] = from_f<T>(s);
  }
}

// Weight-gradient partial over one token chunk, part[c, f, h, d] =
// sum_{t in chunk} A[t,h,f] B[t,h,d] (dW_V: A = aX in fp32, B = dO; the
// projections' dW_K: A = du, B = q_proj; dW_Q: one group, A = q_raw, B =
// dq_proj), on fp32 matrix cores (v_mfma_f32_32x32x2f32).  One wave per
// (chunk, head, 32-wide f slice, 32-wide d tile): part^T[d, f] += B^T[d, t]
// A[t, f] two tokens per product, lane l feeding token t + l/32 at d (A
// operand) and f (B operand) = l % 32.
template <typename T>
__device__ __forceinline__ float bits_to_f(uint32_t b) {
  if constexpr (std::is_same<T, float>::value) return __uint_as_float(b);
  else if constexpr (std::is_same<T, bf16>::value) return __uint_as_float(b << 16);
  else return (float)__builtin_bit_cast(f16, (uint16_t)b);
}

template <typename TA, typename T>
__global__ __launch_bounds__(64) void absorb_dwv_part_kernel(
    const TA *__restrict__ ax, const T *__restrict__ dO, float *__restrict__ part,
    int64_t T_q, int64_t tchunk, int H, int F, int DH, int n_waves) {
  const int lane = threadIdx.x, l32 = lane & 31, kt = lane >> 5;
  const int nfs = (F + 31) / 32, nds = (DH + 31) / 32;
  // workgroup i runs on XCD i % kXcds: give each XCD a contiguous run of
  // waves, so the F/32 waves that read the same dO rows share one L2
  int w = blockIdx.x;
  w = (w % kXcds) * (int)(gridDim.x / kXcds) + w / kXcds;
  if (w >= n_waves) return;
  const int ds = w % nds;
  w /= nds;
  const int fs = w % nfs;
  w /= nfs;
  const int h = w % H;
  const int64_t c = w / H;
  const int64_t ta = c * tchunk, tb = ta + tchunk < T_q ? ta + tchunk : T_q;
  const int f = fs * 32 + l32, d = ds * 32 + l32;
  const bool f_ok = f < F, d_ok = d < DH;
  f32x16 acc;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = 0.f;
  constexpr int kU = 8;  // token pairs per batch of loads
  // Branch-free loads: every lane reads a clamped, in-range element and the
  // select to zero comes after all loads are issued, so a batch is one round
  // trip (predicated loads compile to branches that wait on each load).
  const int dc = d_ok ? d : DH - 1, fc = f_ok ? f : F - 1;
  auto load = [&](int64_t t, float(&av)[kU], float(&bv)[kU]) {
    // 16-bit elements go into separate 32-bit registers: loaded as T they
    // get packed two per register, and each load then waits on the previous
    using Bits = typename std::conditional<sizeof(T) == 2, uint16_t, uint32_t>::type;
    using BitsA = typename std::conditional<sizeof(TA) == 2, uint16_t, uint32_t>::type;
    uint32_t ra[kU], rb[kU];
#pragma unroll
    for (int i = 0; i < kU; ++i) {
      const int64_t tt = t + 2 * i + kt, tc = tt < tb ? tt : tb - 1;
      ra[i] = reinterpret_cast<const Bits *>(dO)[(tc * H + h) * DH + dc];
      rb[i] = reinterpret_cast<const BitsA *>(ax)[(tc * H + h) * F + fc];
    }
#pragma unroll
    for (int i = 0; i < kU; ++i) {
      const bool ok = t + 2 * i + kt < tb;
      av[i] = ok && d_ok ? bits_to_f<T>(ra[i]) : 0.f;
      bv[i] = ok && f_ok ? bits_to_f<TA>(rb[i]) : 0.f;
    }
  };
  auto product = [&](const float(&av)[kU], const float(&bv)[kU]) {
#pragma unroll
    for (int i = 0; i < kU; ++i) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i], bv[i], acc, 0, 0, 0);
  };
  // two register batches: the next batch's loads are in flight while the
  // matrix cores consume the current one
  float a0[kU], b0[kU], a1[kU], b1[kU];
  load(ta, a0, b0);
  for (int64_t t = ta; t < tb; t += 4 * kU) {
    load(t + 2 * kU, a1, b1);
    product(a0, b0);
    if (t + 2 * kU >= tb) break;
    load(t + 4 * kU, a0, b0);
    product(a1, b1);
  }
  // acc element r: d = ds*32 + (r/4)*8 + kt*4 + r%4, f = this lane's f
  if (!f_ok) return;
  float *dst = part + ((c * F + f) * H + h) * DH;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int d0 = ds * 32 + g * 8 + kt * 4;
    if (d0 >= DH) continue;
    f32x4 v = {acc[g * 4], acc[g * 4 + 1], acc[g * 4 + 2], acc[g * 4 + 3]};
    *reinterpret_cast<f32x4 *>(dst + d0) = v;
  }
}

// dW_V partials with the chunk's token tiles staged in LDS, one workgroup per
// (token chunk c, head h, 32-column block of d): part[c, f, h, d] = sum_t
// aX[t,h,f] dO[t,h,d] on v_mfma_f32_16x16x4f32 (aX stays fp32).  32-token
// tiles of aX [32][FP] and dO [32][32] (converted to fp32) sit in a double-
// buffered LDS ring, the next tile's 16-byte loads held in registers while the
// current one is consumed; every operand is one 4-byte LDS read (A: aX[t =
// 4*ks + l/16][f = 16*ft + l%16], B: dO[t][d = 16*dt + l%16], rows padded so
// the four token rows of a read fall in different banks).  Each wave owns f
// tiles wave + 4j and both d tiles.
constexpr int kDwTok = 32;
constexpr int kDwBS = 48;  // B tile row stride (floats)

template <int FP>
struct DwSmem {
  static constexpr int AS = FP + 16;  // A tile row stride (floats)
  static constexpr int kStage = kDwTok * (AS + kDwBS);
  static constexpr int kBytes = 2 * kStage * 4;
};

template <typename T, int FP>
__global__ __launch_bounds__(256) void absorb_dwv_lds_kernel(
    const float *__restrict__ ax, const T *__restrict__ dO, float *__restrict__ part,
    int64_t T_q, int64_t tchunk, int H, int F, int DH, int n_db) {
  static_assert(sizeof(T) == 2, "16-bit dO");
  using S = DwSmem<FP>;
  extern __shared__ __align__(16) float dw_smem[];
  const int tid = threadIdx.x, lane = tid & 63, l16 = lane & 15, lq = lane >> 4;
  const int wave = tid >> 6;
  int64_t b = blockIdx.x;
  const int db = (int)(b % n_db);
  b /= n_db;
  const int h = (int)(b % H);
  const int64_t c = b / H;
  const int64_t ta = c * tchunk, tb = ta + tchunk < T_q ? ta + tchunk : T_q;
  const int d0 = db * 32;
  const int dn = DH - d0 < 32 ? DH - d0 : 32;

  constexpr int kACh = FP / 4;                 // 16-byte chunks per aX row
  constexpr int kAPer = kDwTok * kACh / 256;   // per thread
  u32x4 ra[kAPer], rb = {0u, 0u, 0u, 0u};
  // branch-free loads: clamped in-range addresses, zeros selected afterwards
  auto load = [&](int64_t t0) {
#pragma unroll
    for (int i = 0; i < kAPer; ++i) {
      const int idx = i * 256 + tid, r = idx / kACh, ch = idx % kACh;
      const int64_t t = t0 + r;
      const bool ok = t < tb && ch * 4 < F;
      const u32x4 v = *reinterpret_cast<const u32x4 *>(ax + (ok ? (t * H + h) * F + ch * 4 : 0));
      ra[i] = ok ? v : u32x4{0u, 0u, 0u, 0u};
    }
    const int r = (tid >> 2) & (kDwTok - 1), ch = tid & 3;
    const int64_t t = t0 + r;
    const bool ok = tid < kDwTok * 4 && t < tb && ch * 8 < dn;
    const u32x4 v =
        *reinterpret_cast<const u32x4 *>(dO + (ok ? (t * H + h) * DH + d0 + ch * 8 : 0));
    rb = ok ? v : u32x4{0u, 0u, 0u, 0u};
  };
  auto stage = [&](int st) {
    float *as = dw_smem + st * S::kStage;
    float *bs = as + kDwTok * S::AS;
#pragma unroll
    for (int i = 0; i < kAPer; ++i) {
      const int idx = i * 256 + tid, r = idx / kACh, ch = idx % kACh;
      *reinterpret_cast<u32x4 *>(as + r * S::AS + ch * 4) = ra[i];
    }
    if (tid < kDwTok * 4) {
      const int r = tid >> 2, ch = tid & 3;
      f32x4 lo, hi;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        lo[e] = bits_to_f<T>((rb[e >> 1] >> ((e & 1) * 16)) & 0xffffu);
        hi[e] = bits_to_f<T>((rb[(e + 4) >> 1] >> ((e & 1) * 16)) & 0xffffu);
      }
      *reinterpret_cast<f32x4 *>(bs + r * kDwBS + ch * 8) = lo;
      *reinterpret_cast<f32x4 *>(bs + r * kDwBS + ch * 8 + 4) = hi;
    }
  };

  constexpr int kFt = FP / 64;  // f tiles per wave
  f32x4 acc[kFt][2];
#pragma unroll
  for (int j = 0; j < kFt; ++j)
#pragma unroll
    for (int dt = 0; dt < 2; ++dt) acc[j][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int nt = (int)((tb - ta + kDwTok - 1) / kDwTok);
  load(ta);
  stage(0);
  __syncthreads();
#pragma nounroll
  for (int i = 0; i < nt; ++i) {
    if (i + 1 < nt) load(ta + (int64_t)(i + 1) * kDwTok);
    const float *as = dw_smem + (i & 1) * S::kStage + lq * S::AS + wave * 16 + l16;
    const float *bs = dw_smem + (i & 1) * S::kStage + kDwTok * S::AS + lq * kDwBS + l16;
#pragma unroll
    for (int ks = 0; ks < kDwTok / 4; ++ks) {
      float bv[2], av[kFt];
#pragma unroll
      for (int dt = 0; dt < 2; ++dt) bv[dt] = bs[ks * 4 * kDwBS + 16 * dt];
#pragma unroll
      for (int j = 0; j < kFt; ++j) av[j] = as[ks * 4 * S::AS + 64 * j];
#pragma unroll
      for (int j = 0; j < kFt; ++j)
#pragma unroll
        for (int dt = 0; dt < 2; ++dt)
          acc[j][dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[j], bv[dt], acc[j][dt], 0, 0, 0);
    }
    if (i + 1 < nt) stage((i + 1) & 1);
    __syncthreads();
  }
  // C[f][d]: f = 16*(wave + 4j) + 4*lq + r, d = d0 + 16*dt + l16
#pragma unroll
  for (int j = 0; j < kFt; ++j)
#pragma unroll
    for (int dt = 0; dt < 2; ++dt) {
      const int d = 16 * dt + l16;
      if (d >= dn) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int f = 16 * (wave + 4 * j) + 4 * lq + r;
        if (f < F) part[((c * F + f) * H + h) * DH + d0 + d] = acc[j][dt][r];
      }
    }
}

template <typename T>
__global__ __launch_bounds__(256) void absorb_dwv_sum_kernel(const float *__restrict__ part,
                                                             T *__restrict__ dwv, int64_t n_out,
                                                             int64_t n_chunks) {
  const int64_t o = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (o >= n_out) return;
  // chunk order kept; eight independent loads in flight per batch
  constexpr int kB = 8;
  float s = 0.f;
  for (int64_t c0 = 0; c0 < n_chunks; c0 += kB) {
    float v[kB];
#pragma unroll
    for (int i = 0; i < kB; ++i) v[i] = c0 + i < n_chunks ? part[(c0 + i) * n_out + o] : 0.f;
#pragma unroll
    for (int i = 0; i < kB; ++i) s += v[i];
  }
  dwv[o] = from_f<T>(s);
}

// [rows, 16] -> [rows, 32] with zero columns 16..31, and back: D=16 runs on
// the D=32 matrix-core kernels.  A row of 16 elements is cpr 16-byte chunks
// (2 for 16-bit elements, 4 for fp32); its padded copy is 2 * cpr chunks.
__global__ __launch_bounds__(256) void pad16_kernel(const u32x4 *__restrict__ src,
                                                    u32x4 *__restrict__ dst, int64_t rows,
                                                    int cpr) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= rows * 2 * cpr) return;
  const int64_t r = i / (2 * cpr);
  const int c = (int)(i % (2 * cpr));
  u32x4 v = {0u, 0u, 0u, 0u};
  if (c < cpr) v = src[r * cpr + c];
  dst[r * 2 * cpr + c] = v;
}

__global__ __launch_bounds__(256) void unpad16_kernel(const u32x4 *__restrict__ src,
                                                      u32x4 *__restrict__ dst, int64_t rows,
                                                      int cpr) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= rows * cpr) return;
  const int64_t r = i / cpr;
  const int c = (int)(i % cpr);
  dst[r * cpr + c] = src[r * 2 * cpr + c];
}

// [rows, n] -> [rows, m] (m >= n) with zero columns n..m-1, and back
// (element type E of the operand's width: absorb D_KV padded to a whole
// number of 16-byte chunks)
template <typename E>
__global__ __launch_bounds__(256) void pad_cols_kernel(const E *__restrict__ src,
                                                       E *__restrict__ dst, int64_t rows,
                                                       int64_t n, int64_t m) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= rows * m) return;
  const int64_t r = i / m, c = i % m;
  dst[i] = c < n ? src[r * n + c] : E(0);
}

template <typename E>
__global__ __launch_bounds__(256) void unpad_cols_kernel(const E *__restrict__ src,
                                                         E *__restrict__ dst, int64_t rows,
                                                         int64_t n, int64_t m) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= rows * n) return;
  const int64_t r = i / n, c = i % n;
  dst[i] = src[r * m + c];
}

inline unsigned blocks_for(int64_t n) { return (unsigned)((n + 255) / 256); }

}  // namespace

template <typename T>
void launch_row_dot(const void *o, const void *dout, float *delta, int64_t rows, int D,
                    hipStream_t st) {
  if (rows == 0) return;
  const int64_t threads = rows * (D / (16 / (int)sizeof(T)));
  hipLaunchKernelGGL(row_dot_kernel<T>, dim3(blocks_for(threads)), dim3(256), 0, st,
                     (const T *)o, (const T *)dout, delta, rows, D);
}

template <typename T>
void launch_lse_combine(const float *part_o, const float *part_lse, void *out, float *lse,
                        const int32_t *comb_items, int64_t n_comb, int H, int D, int max_rows,
                        hipStream_t st) {
  if (n_comb == 0) return;
  if (D <= 32) {
    const int rblocks = (max_rows + 2 * kCombRows - 1) / (2 * kCombRows);
    hipLaunchKernelGGL((lse_combine_kernel<T, 2>), dim3((unsigned)(n_comb * H * rblocks)),
                       dim3(64 * kCombRows), 0, st, part_o, part_lse, (T *)out, lse, comb_items,
                       H, D, rblocks);
  } else {
    const int rblocks = (max_rows + kCombRows - 1) / kCombRows;
    hipLaunchKernelGGL((lse_combine_kernel<T, 1>), dim3((unsigned)(n_comb * H * rblocks)),
                       dim3(64 * kCombRows), 0, st, part_o, part_lse, (T *)out, lse, comb_items,
                       H, D, rblocks);
  }
}

template <typename T>
void launch_sum_combine(const float *part, void *out, const int32_t *comb_items, int64_t n_comb,
                        int H, int D, int max_rows, hipStream_t st) {
  if (n_comb == 0) return;
  const int rblocks = (max_rows + kCombRows - 1) / kCombRows;
  hipLaunchKernelGGL(sum_combine_kernel<T>, dim3((unsigned)(n_comb * H * rblocks)),
                     dim3(64 * kCombRows), 0, st, part, (T *)out, comb_items, H, D, rblocks);
}

template <typename T>
void launch_absorb_dax(const AbsorbArgs &a, hipStream_t st) {
  if (a.T_q == 0) return;
  hipLaunchKernelGGL(absorb_dax_kernel<T>, dim3((unsigned)(a.T_q * a.H)), dim3(256), 0, st,
                     (const T *)a.dO, (const T *)a.wv, (T *)a.dax, a.H, a.F, a.DH);
}

template <typename TA, typename T>
void launch_wgrad(const void *a, const void *b, float *part, void *out, int64_t T_q,
                  int64_t tchunk, int64_t n_chunks, int G, int F, int DH, hipStream_t st) {
  const int64_t n_out = (int64_t)F * G * DH;
  if (n_chunks > 0) {
    const int64_t waves = n_chunks * G * ((F + 31) / 32) * ((DH + 31) / 32);
    const int64_t grid = (waves + kXcds - 1) / kXcds * kXcds;
    hipLaunchKernelGGL((absorb_dwv_part_kernel<TA, T>), dim3((unsigned)grid), dim3(64), 0, st,
                       (const TA *)a, (const T *)b, part, T_q, tchunk, G, F, DH, (int)waves);
  }
  hipLaunchKernelGGL(absorb_dwv_sum_kernel<T>, dim3(blocks_for(n_out)), dim3(256), 0, st, part,
                     (T *)out, n_out, n_chunks);
}

template <typename T>
void launch_chunk_sum(const float *part, void *out, int64_t n_out, int64_t n_chunks,
                      hipStream_t st) {
  if (n_out == 0) return;
  hipLaunchKernelGGL(absorb_dwv_sum_kernel<T>, dim3(blocks_for(n_out)), dim3(256), 0, st, part,
                     (T *)out, n_out, n_chunks);
}

template <typename T, int FP>
void dwv_lds(const AbsorbArgs &a, hipStream_t st) {
  const int n_db = (a.DH + 31) / 32;
  const int64_t wgs = a.n_tchunks * a.H * n_db;
  if (wgs > 0) {
    constexpr int smem = DwSmem<FP>::kBytes;
    allow_dynamic_lds(reinterpret_cast<const void *>(&absorb_dwv_lds_kernel<T, FP>), smem);
    hipLaunchKernelGGL((absorb_dwv_lds_kernel<T, FP>), dim3((unsigned)wgs), dim3(256), smem, st,
                       a.ax, (const T *)a.dO, a.dwv_part, a.T_q, a.tchunk, a.H, a.F, a.DH, n_db);
  }
  launch_chunk_sum<T>(a.dwv_part, a.dwv, (int64_t)a.F * a.H * a.DH, a.n_tchunks, st);
}

// dW_V: the LDS-tiled kernel for 16-bit dO and D_KV <= 256 (a multiple of
// 4), the register-batched one otherwise.
template <typename T>
void launch_absorb_dwv(const AbsorbArgs &a, hipStream_t st) {
  if constexpr (sizeof(T) == 2) {
    if (a.F % 4 == 0 && a.F <= 256) {
      if (a.F <= 64) dwv_lds<T, 64>(a, st);
      else if (a.F <= 128) dwv_lds<T, 128>(a, st);
      else dwv_lds<T, 256>(a, st);
      return;
    }
  }
  launch_wgrad<float, T>(a.ax, a.dO, a.dwv_part, a.dwv, a.T_q, a.tchunk, a.n_tchunks, a.H, a.F,
                         a.DH, st);
}

void launch_pad16(const void *src, void *dst, int64_t rows, int elem_bytes, hipStream_t st) {
  if (rows <= 0) return;
  const int cpr = elem_bytes;  // 16 elements = elem_bytes 16-byte chunks
  hipLaunchKernelGGL(pad16_kernel, dim3(blocks_for(rows * 2 * cpr)), dim3(256), 0, st,
                     (const u32x4 *)src, (u32x4 *)dst, rows, cpr);
}

void launch_pad_cols(const void *src, void *dst, int64_t rows, int64_t n, int64_t m,
                     int elem_bytes, hipStream_t st) {
  if (rows <= 0 || m <= 0) return;
  if (elem_bytes == 4)
    hipLaunchKernelGGL(pad_cols_kernel<uint32_t>, dim3(blocks_for(rows * m)), dim3(256), 0, st,
                       (const uint32_t *)src, (uint32_t *)dst, rows, n, m);
  else
    hipLaunchKernelGGL(pad_cols_kernel<uint16_t>, dim3(blocks_for(rows * m)), dim3(256), 0, st,
                       (const uint16_t *)src, (uint16_t *)dst, rows, n, m);
}

void launch_unpad_cols(const void *src, void *dst, int64_t rows, int64_t n, int64_t m,
                       int elem_bytes, hipStream_t st) {
  if (rows <= 0 || n <= 0) return;
  if (elem_bytes == 4)
    hipLaunchKernelGGL(unpad_cols_kernel<uint32_t>, dim3(blocks_for(rows * n)), dim3(256), 0,
                       st, (const uint32_t *)src, (uint32_t *)dst, rows, n, m);
  else
    hipLaunchKernelGGL(unpad_cols_kernel<uint16_t>, dim3(blocks_for(rows * n)), dim3(256), 0,
                       st, (const uint16_t *)src, (uint16_t *)dst, rows, n, m);
}

void launch_unpad16(const void *src, void *dst, int64_t rows, int elem_bytes, hipStream_t st) {
  if (rows <= 0) return;
  const int cpr = elem_bytes;
  hipLaunchKernelGGL(unpad16_kernel, dim3(blocks_for(rows * cpr)), dim3(256), 0, st,
                     (const u32x4 *)src, (u32x4 *)dst, rows, cpr);
}

#define VAFA_INST(T)                                                                        \
  template void launch_row_dot<T>(const void *, const void *, float *, int64_t, int,        \
                                  hipStream_t);                                             \
  template void launch_lse_combine<T>(const float *, const float *, void *, float *,        \
                                      const int32_t *, int64_t, int, int, int, hipStream_t);\
  template void launch_sum_combine<T>(const float *, void *, const int32_t *, int64_t, int, \
                                      int, int, hipStream_t);                               \
  template void launch_absorb_dax<T>(const AbsorbArgs &, hipStream_t);                      \
  template void launch_absorb_dwv<T>(const AbsorbArgs &, hipStream_t);                      \
  template void launch_wgrad<T, T>(const void *, const void *, float *, void *, int64_t,    \
                                   int64_t, int64_t, int, int, int, hipStream_t);           \
  template void launch_chunk_sum<T>(const float *, void *, int64_t, int64_t, hipStream_t);
VAFA_INST(float)
VAFA_INST(f16)
VAFA_INST(bf16)
#undef VAFA_INST

}  // namespace vafa
