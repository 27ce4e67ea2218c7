// Packed varlen FlashAttention backward on gfx950 matrix cores.
//
// Deterministic kernels (no atomics), all recomputing P = exp2(S*c - LSE)
// from the forward's log2-domain LSE (fa/kernels.py:233-494):
//   * dK/dV, key-major: a workgroup owns the plan's key tile (128 or 256 keys)
//     of one head (32 per wave, K and V held in registers as MFMA operands)
//     and walks the segment's queries in blocks of 32 staged row-major in LDS
//     by buffer_load ... lds,
//     double-buffered (the transposed operands Q^T, dO^T come from
//     ds_read_b64_tr_b16):
//       S = Q K^T, dP = dO V^T, dS = P (dP - delta),
//       dV^T += dO^T P,  dK^T += Q^T dS           (4 products per block)
//   * dQ, query-major over the forward's plan items (including split-K
//     partials): S^T = K Q^T, dP^T = V dO^T, dQ^T += K^T dS^T.
//   * fused dQ/dK/dV, key-major (segments with one query block): a workgroup
//     walks a chunk of 128-key tiles with the query block staged once, forms
//     dK/dV per tile and dQ^T = K^T dS^T over the whole chunk, and writes one
//     set of scaled fp32 partial dQ rows per chunk, which an ordered sum turns
//     into dQ (the dead template of fa/kernels.py:923-1099).
// The dQ kernel stages K / V blocks through registers.  Its row statistics stay
// per lane (lane <-> query row); the dK/dV kernel reads LSE and delta of its
// 32-row block from LDS.  LDS operands are read a few products ahead of the
// MFMAs that consume them (sched_barrier keeps that order).
#include <type_traits>

#include "kernels.h"
#include "mfma.h"

namespace vafa {

namespace {

constexpr int kRB = 32;  // rows per staged block (queries for dK/dV, keys for dQ)
// LDS layout of a 32-row tile of 16-bit rows that is read both as rows
// (ds_read_b128: 16 lanes take one 16-byte chunk of 16 consecutive rows) and
// transposed (ds_read_b64_tr_b16: 32 lanes take 64 bytes of 4 consecutive
// rows).  With one row stride the two cannot both be conflict-free -- row
// reads want 4 x odd dwords, transposed reads 16 mod 64 dwords -- so rows sit
// in groups of four: P1 elements apart inside a group (P1/2 dwords = 16 mod
// 32: the 4 row pieces of a transposed read fill distinct banks) and P2 =
// 4*P1 + 8 elements from group to group (4 dwords past a multiple of the 64
// banks: 16 consecutive rows start on 16 distinct 4-bank groups).  The
// operand reads add row offsets that are multiples of 4 rows to a per-lane
// base, so those stay compile-time immediates.
template <int D>
struct GTile {
  static constexpr int P1 = (D / 2) % 32 == 16 ? D : D + 32;
  static constexpr int P2 = 4 * P1 + 8;
  static constexpr int kElems = (kRB / 4) * P2;  // 32 rows
  static __device__ __forceinline__ int row(int r) { return (r >> 2) * P2 + (r & 3) * P1; }
};

// A operand of a 32x32x16 MFMA read transposed from a GTile (columns c0 +
// l % 32 as the row index, tile rows k0 .. k0+15 as the reduction index in
// the relabelled order of the C layout; k0 a multiple of 4), as tr_operand
// does for a fixed row stride.
template <typename T, int D>
__device__ __forceinline__ typename Mfma<T>::v8 tr_operand_g(const T *tile, int k0, int c0,
                                                             int lane) {
  using L = GTile<D>;
  const int i = lane & 15, g = lane >> 4;
  const T *p = tile + (k0 >> 2) * L::P2 + L::row(4 * (g >> 1) + (i >> 2)) + c0 + (g & 1) * 16 +
               4 * (i & 3);
  return as_v8<T>(join(lds_tr16(p), lds_tr16(p + 2 * L::P2)));
}

template <int D>
struct DkvSmem {
  static constexpr int kQs = GTile<D>::kElems;                // Q (or dO) rows
  static constexpr int kBufBytes = 2 * kQs * 2 + 2 * kRB * 4;  // Q, dO, LSE, delta
  // + the span of the last full-width DMA instruction past its tile (the
  // instruction's masked lanes write nothing, the slack is never touched)
  static constexpr int kBytes = 2 * kBufBytes + 1024;
};

// Dynamic LDS of the dK/dV kernel: the query-block buffers, or the per-wave
// row-store regions of the epilogue if those are larger (D = 128 on 8 waves).
template <typename T, int D, int NW>
constexpr int dkv_lds_bytes() {
  constexpr int kNDO = D / 32 / (D >= 256 ? 2 : 1);
  constexpr int kStage = NW * StagedRows<T, kNDO>::kBytes;
  constexpr int kBase = DkvSmem<D>::kBytes > kStage ? DkvSmem<D>::kBytes : kStage;
  // D = 256: the partial S / dP exchange region after the query-block buffers
  return D >= 256 ? DkvSmem<D>::kBytes + NW * 64 * 32 * 4 : kBase;
}

// LDS-DMA of one head's rows [r0, r0 + 32) of a [T, H, D] tensor (rows at or
// past r_end read as zero) into a GTile block: wave w of NW moves
// rows RPW*w .. RPW*w + RPW-1 (RPW = 32/NW), one instruction per row with
// lanes < D/8 active.  One buffer descriptor covers the block's valid rows;
// the row sits in the lane offset.
template <typename T, int D, int NW>
__device__ __forceinline__ void dma_rows(const T *src, int r0, int r_end, int H, int h,
                                         uint32_t base, int wave, int lane) {
  constexpr int RPW = kRB / NW;
  const int rows = uniform_clamp(r_end - r0, kRB);
  const u32x4 rs = rsrc_words32(src + (int64_t)r0 * H * D, (uint32_t)(rows * H * D * 2));
  const int off = (wave * RPW * H + h) * D * 2 + lane * 16;
  if (lane < D / 8) {
#pragma unroll
    for (int n = 0; n < RPW; ++n) {
      // one add of a scalar row term (volatile: not hoisted into RPW registers)
      int voff;
      asm volatile("v_add_u32 %0, %1, %2" : "=v"(voff) : "s"(n * H * D * 2), "v"(off));
      lds_dma16(rs, base + GTile<D>::row(wave * RPW + n) * 2, voff);
    }
  }
}

// Query-block staging of the dK/dV and fused kernels: full width at D <= 64.
template <typename T, int D, int NW>
__device__ __forceinline__ void dma_block_rows(const T *src, int r0, int r_end, int H, int h,
                                               uint32_t base, int wave, int lane);

// The same block by full-width LDS-DMA: the instruction with index i writes
// the tile's LDS bytes [1024 i, 1024 i + 1024), lane l the 16 bytes at
// 1024 i + 16 l, so each lane fetches the (row, 16-byte chunk) that the GTile
// layout places there; lanes whose position is row padding or past the tile
// are masked off.  ceil(tile bytes / 1 KiB) instructions per block instead of
// one per row (D = 64: 6 against 32 with 8 of 64 lanes active).  Measured on
// the MI355X (A/B in one call): stage-1 replay (H=4, D=64) fwd+bwd 4.98 ->
// 4.61 ms; C2's D=128 dK/dV kernel (8 waves, 256-key tiles) 0.93 -> 0.97 ms,
// so D >= 128 keeps one instruction per row (16 or 32 active lanes).
template <typename T, int D, int NW>
__device__ __forceinline__ void dma_rows_wide(const T *src, int r0, int r_end, int H, int h,
                                              uint32_t base, int wave, int lane) {
  using L = GTile<D>;
  constexpr int kInstr = (L::kElems / 8 + 63) / 64;
  const int rows = uniform_clamp(r_end - r0, kRB);
  const u32x4 rs = rsrc_words32(src + (int64_t)r0 * H * D, (uint32_t)(rows * H * D * 2));
  for (int i = wave; i < kInstr; i += NW) {
    const int e = (i * 64 + lane) * 8;       // element offset of this lane's 16 bytes
    const int g = e / L::P2, w = e - g * L::P2;
    const int j = w / L::P1, wr = w - j * L::P1;
    if (e < L::kElems && j < 4 && wr < D) {
      // rows at or past `rows` lie past the descriptor's range: zeros
      const int voff = (((4 * g + j) * H + h) * D + wr) * 2;
      lds_dma16(rs, base + i * 1024, voff);
    }
  }
}

template <typename T, int D, int NW>
__device__ __forceinline__ void dma_block_rows(const T *src, int r0, int r_end, int H, int h,
                                               uint32_t base, int wave, int lane) {
  if constexpr (D <= 64)
    dma_rows_wide<T, D, NW>(src, r0, r_end, H, h, base, wave, lane);
  else
    dma_rows<T, D, NW>(src, r0, r_end, H, h, base, wave, lane);
}

template <typename T, int D, int NW>
__global__ __launch_bounds__(64 * NW, D >= 256 && NW < 8 ? 1 : 2) void varlen_dkv_kernel(
    const T *__restrict__ q, const T *__restrict__ k, const T *__restrict__ v,
    const T *__restrict__ dout, const float *__restrict__ lse, const float *__restrict__ delta,
    T *__restrict__ dk, T *__restrict__ dv, const int32_t *__restrict__ items, int H, float c,
    float scale) {
  using M = Mfma<T>;
  using S = DkvSmem<D>;
  using L = GTile<D>;
  constexpr int ND = D / 32;
  constexpr int kPre = D >= 128 ? 2 : 4;  // operand ring depth within the register budget
  // At D = 256 (8 waves) waves w and w + 4 share 32 keys, each holding K / V
  // and accumulating dK / dV for one half of d: each forms S and dP over its
  // half, the two partial sums meet through LDS, and both form the same P
  // and dS (full-width K / V operands beside the accumulators would not fit).
  constexpr bool kShare = D >= 256;
  static_assert(!kShare || NW == 8, "D = 256 runs on 8 waves");
  constexpr int NDO = kShare ? ND / 2 : ND;  // 32-wide d tiles of dK/dV per wave
  constexpr int NCS = 2 * NDO;               // 16-wide d chunks of the S / dP products
  constexpr bool kDeltaInChain = D <= 64;
  extern __shared__ __align__(16) unsigned char smem_raw[];

  const int item = blockIdx.x / H, h = blockIdx.x % H;
  const PlanItem it = load_item(items, item);
  const int k0 = it.v[0], k1 = it.v[1], q0 = it.v[2], q1 = it.v[3];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int kgrp = kShare ? (wave & 3) : wave;  // this wave's 32 keys
  const int dpart = kShare ? (wave >> 2) : 0;   // this wave's half of d (kShare)
  const int lrow = lane & 31, lhalf = lane >> 5;
  const bool wave_active = k0 + kgrp * 32 < k1;

  // stage query block qb: Q and dO rows by 16-byte DMA, LSE and delta (strided
  // by H) by one 4-byte DMA per lane -- even waves LSE, odd waves delta (the
  // same bytes from every even or odd wave), so every wave issues the same
  // count.  Rows past q1 arrive as zeros: Q = dO = 0 there makes both of
  // their products vanish whatever P is.
  auto issue = [&](int qb, int buf) {
    unsigned char *base = smem_raw + buf * S::kBufBytes;
    dma_block_rows<T, D, NW>(q, qb, q1, H, h, lds_addr(base), wave, lane);
    dma_block_rows<T, D, NW>(dout, qb, q1, H, h, lds_addr(base + S::kQs * 2), wave, lane);
    const float *vec = (wave & 1) ? delta : lse;
    const int rows = uniform_clamp(q1 - qb, kRB);
    const u32x4 rv = rsrc_words32(vec + (int64_t)qb * H + h, (uint32_t)(rows * H * 4));
    if (lane < kRB) lds_dma4(rv, lds_addr(base + 2 * S::kQs * 2 + (wave & 1) * kRB * 4), lane * H * 4);
  };
  const int nblk = (q1 - q0 + kRB - 1) / kRB;
  if (nblk > 0) issue(q0, 0);

  typename M::v8 kf[NCS], vf[NCS];
  {
    const int nk = k1 - k0;
    const rsrc_t rk = make_rsrc(k + (int64_t)k0 * H * D, (int64_t)nk * H * D * 2);
    const rsrc_t rv = make_rsrc(v + (int64_t)k0 * H * D, (int64_t)nk * H * D * 2);
    const int off = ((kgrp * 32 + lrow) * H + h) * D * 2 + lhalf * 16 + dpart * NDO * 64;
#pragma unroll
    for (int cc = 0; cc < NCS; ++cc) {
      u32x4 a = buf_load16(rk, off + cc * 32), b = buf_load16(rv, off + cc * 32);
      // waited for here, in the prologue, not inside the loop
      asm volatile("" : "+v"(a), "+v"(b));
      kf[cc] = as_v8<T>(a);
      // At D <= 64, V enters negated (an exact sign flip): the dP chain below
      // starts from delta and yields delta - dP, so dS = P (dP - delta) is
      // one multiply with a negated operand.  (At D = 128 the delta reads in
      // front of the chain cost more than the subtractions they remove.)
      if constexpr (kDeltaInChain) {
#pragma unroll
        for (int w = 0; w < 4; ++w) b[w] ^= 0x80008000u;
      }
      vf[cc] = as_v8<T>(b);
    }
  }
  f32x16 adk[NDO], adv[NDO];
#pragma unroll
  for (int i = 0; i < NDO; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) adk[i][r] = adv[i][r] = 0.f;

  // per-lane element offsets: row lrow at d = 8*lhalf (A of S and dP) and the
  // origin of the transposed reads (layout of tr_operand)
  const int a_off = L::row(lrow) + lhalf * 8 + dpart * NDO * 32;
  const int t_off = L::row(4 * (lane >> 5) + ((lane & 15) >> 2)) + ((lane >> 4) & 1) * 16 +
                    4 * (lane & 3);
  // Two query blocks per trip (below), so each block's LDS buffer is a
  // compile-time offset folded into the LDS reads' immediates.
  auto blk = [&](int j, auto bufc) {
    constexpr int B = decltype(bufc)::value;
    wait_vmcnt<0>();
    __syncthreads();  // block j visible; every wave is done with the other buffer
    if (j + 1 < nblk) issue(q0 + (j + 1) * kRB, 1 - B);
    const unsigned char *base = smem_raw + B * S::kBufBytes;
    const lds_cptr<T> qs = as_lds(reinterpret_cast<const T *>(base));
    const lds_cptr<T> ds_ = qs + S::kQs;
    const float *ls = reinterpret_cast<const float *>(base + 2 * S::kQs * 2);
    f32x16 s, dp;
    if (wave_active) {
      // S = Q K^T (even reads, Q rows) and dP = dO V^T (odd reads, dO rows);
      // with kDeltaInChain delta - dP = delta + dO (-V)^T, the chain starting
      // from the block's delta (row r of the accumulator is query
      // 8*(r/4) + 4*lhalf + r%4); kShare: over this wave's half of d
      auto aop = [&](int i) { return lds_ld16<T>(((i & 1) ? ds_ : qs) + a_off + (i >> 1) * 16); };
  #pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x4 d4 = kDeltaInChain
                             ? *reinterpret_cast<const f32x4 *>(ls + kRB + g * 8 + lhalf * 4)
                             : f32x4{0.f, 0.f, 0.f, 0.f};
  #pragma unroll
        for (int e = 0; e < 4; ++e) {
          s[4 * g + e] = 0.f;
          dp[4 * g + e] = d4[e];
        }
      }
      u32x4 ring[kPre];
  #pragma unroll
      for (int i = 0; i < kPre; ++i) ring[i] = aop(i);
      __builtin_amdgcn_sched_barrier(0);
  #pragma unroll
      for (int i = 0; i < 2 * NCS; ++i) {
        const typename M::v8 a = as_v8<T>(ring[i % kPre]);
        if (i & 1)
          dp = M::mma(a, vf[i >> 1], dp);
        else
          s = M::mma(a, kf[i >> 1], s);
        if (i + kPre < 2 * NCS) ring[i % kPre] = aop(i + kPre);
        __builtin_amdgcn_sched_barrier(0);
      }
      if constexpr (kShare) {
        // this wave's partial S and dP for the partner wave (wave ^ 4):
        // [register group][lane] as 16-byte pieces, 1 KiB per instruction
        // (byte offset formed here, volatile: no address register is held
        // across the block loop)
        int eo;
        asm volatile("v_lshl_add_u32 %0, %1, 4, %2"
                     : "=v"(eo)
                     : "v"(lane), "s"(S::kBytes + wave * 8 * 64 * 16));
        f32x4 *ex = reinterpret_cast<f32x4 *>(smem_raw + eo);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          ex[g * 64] = f32x4{s[4 * g], s[4 * g + 1], s[4 * g + 2], s[4 * g + 3]};
          ex[(4 + g) * 64] = f32x4{dp[4 * g], dp[4 * g + 1], dp[4 * g + 2], dp[4 * g + 3]};
        }
      }
    }
    if constexpr (kShare) {
      // every pair's partial sums written (waves w and w ^ 4 are active
      // together); the next block's writes come after its first barrier,
      // when every wave has read these
      __syncthreads();
      if (wave_active) {
        int eo;
        asm volatile("v_lshl_add_u32 %0, %1, 4, %2"
                     : "=v"(eo)
                     : "v"(lane), "s"(S::kBytes + (wave ^ 4) * 8 * 64 * 16));
        const f32x4 *ex = reinterpret_cast<const f32x4 *>(smem_raw + eo);
        // S = S_own + S_partner: fp32 addition commutes, so both waves of the
        // pair hold the same bits of S, dP and hence of P and dS
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const f32x4 a = ex[g * 64], b = ex[(4 + g) * 64];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            s[4 * g + e] += a[e];
            dp[4 * g + e] += b[e];
          }
        }
      }
    }
    if (wave_active) {
      // transposed operands: i -> this workgroup's d tile i % NDO, query half
      // mm = (i / NDO) >> 1, dO^T (for dV^T, with P) when (i / NDO) is even,
      // else Q^T (for dK^T, with dS)
      auto top = [&](int i) {
        const lds_cptr<T> p = (((i / NDO) & 1) ? qs : ds_) + t_off +
                              ((i / NDO) >> 1) * 4 * L::P2 + (dpart * NDO + i % NDO) * 32;
        return as_v8<T>(join(lds_tr8<T>(p), lds_tr8<T>(p + 2 * L::P2)));
      };
      typename M::v8 tring[kPre];
  #pragma unroll
      for (int i = 0; i < kPre; ++i) tring[i] = top(i);
      // P = exp2(S*c - LSE) and dS = P (dP - delta) (= -(P (delta - dP))
      // with kDeltaInChain) per accumulator row r (query 8*(r/4) + 4*lhalf +
      // r%4 of the block); keys past k1 have zero K and V rows, their dK / dV
      // columns are never stored, so their P needs no masking.
      auto ds_of = [&](float p, float acc, float dl) {
        if constexpr (kDeltaInChain)
          return -(p * acc);
        else
          return p * (acc - dl);
      };
      typename M::v8 pb[2], sb[2];
      // rows 0..7 (first 16 queries) before the products; rows 8..15 are
      // computed under the first half of the chain, which only reads rows 0..7,
      // their LSE (and delta) read one product ahead
  #pragma unroll
      for (int g = 0; g < 2; ++g) {
        const f32x4 L = *reinterpret_cast<const f32x4 *>(ls + g * 8 + lhalf * 4);
        const f32x4 Dl = kDeltaInChain
                             ? f32x4{0.f, 0.f, 0.f, 0.f}
                             : *reinterpret_cast<const f32x4 *>(ls + kRB + g * 8 + lhalf * 4);
  #pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = g * 4 + e;
          const float p = fast_exp2(__builtin_fmaf(s[r], c, -L[e]));
          s[r] = p;
          dp[r] = ds_of(p, dp[r], Dl[e]);
        }
      }
      pb[0] = pack8<T>(s, 0);
      sb[0] = pack8<T>(dp, 0);
      // the 8 second-half rows are spread over the first 2*NDO products:
      // kRowsPer rows at every kEvery-th product
      constexpr int kSteps = 2 * NDO < 8 ? 2 * NDO : 8;
      constexpr int kRowsPer = 8 / kSteps;
      constexpr int kEvery = 2 * NDO / kSteps;
      auto lse_at = [&](int r) { return ls[(r >> 2) * 8 + lhalf * 4 + (r & 3)]; };
      auto del_at = [&](int r) {
        return kDeltaInChain ? 0.f : ls[kRB + (r >> 2) * 8 + lhalf * 4 + (r & 3)];
      };
      float Ln[kRowsPer], Dn[kRowsPer];
  #pragma unroll
      for (int rr = 0; rr < kRowsPer; ++rr) Ln[rr] = lse_at(8 + rr), Dn[rr] = del_at(8 + rr);
      __builtin_amdgcn_sched_barrier(0);
  #pragma unroll
      for (int i = 0; i < 4 * NDO; ++i) {
        const int dt = i % NDO, q2 = i / NDO, mm = q2 >> 1;
        const typename M::v8 a = tring[i % kPre];
        if (q2 & 1)
          adk[dt] = M::mma(a, sb[mm], adk[dt]);
        else
          adv[dt] = M::mma(a, pb[mm], adv[dt]);
        if (i + kPre < 4 * NDO) tring[i % kPre] = top(i + kPre);
        if (i < 2 * NDO && i % kEvery == 0) {
          const int g = i / kEvery;
          float Lc[kRowsPer], Dc[kRowsPer];
  #pragma unroll
          for (int rr = 0; rr < kRowsPer; ++rr) {
            Lc[rr] = Ln[rr], Dc[rr] = Dn[rr];
            if (g + 1 < kSteps) {
              const int rn = 8 + (g + 1) * kRowsPer + rr;
              Ln[rr] = lse_at(rn);
              Dn[rr] = del_at(rn);
            }
          }
  #pragma unroll
          for (int rr = 0; rr < kRowsPer; ++rr) {
            const int r = 8 + g * kRowsPer + rr;
            const float p = fast_exp2(__builtin_fmaf(s[r], c, -Lc[rr]));
            s[r] = p;
            dp[r] = ds_of(p, dp[r], Dc[rr]);
          }
          if (g == kSteps - 1) {
            pb[1] = pack8<T>(s, 8);
            sb[1] = pack8<T>(dp, 8);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };
  for (int j = 0; j < nblk; j += 2) {
    blk(j, std::integral_constant<int, 0>{});
    if (j + 1 < nblk) blk(j + 1, std::integral_constant<int, 1>{});
  }
  wait_vmcnt<0>();

  // dK and dV leave as whole rows through per-wave LDS regions (over the
  // query-block buffers, free once every wave is past its last block):
  // stored from the accumulators, every instruction wrote 16 bytes into each
  // of 32 rows, which cost 14% of the kernel on the stage-1 replay shapes.
  __syncthreads();
  if (!wave_active) return;
  using SR = StagedRows<T, NDO>;
  unsigned char *stage = smem_raw + wave * SR::kBytes;
  const int rows = uniform_clamp(k1 - (k0 + kgrp * 32), 32);
  const int64_t off = ((int64_t)(k0 + kgrp * 32) * H + h) * D + dpart * NDO * 32;
  SR::store(adk, [&](float x) { return static_cast<T>(x * scale); }, stage, dk + off,
            (int64_t)H * D, rows);
  SR::store(adv, [](float x) { return static_cast<T>(x); }, stage, dv + off, (int64_t)H * D,
            rows);
}

// Fused K-major dQ/dK/dV for segments with at most kFusedMaxQ (<= 32)
// queries at D <= 64 (the dead template of fa/kernels.py:923-1099, planner
// fa/chunk_indices.py:290-460).  A workgroup owns one (segment, head) and a
// chunk of up to kFusedTiles 128-key tiles; the segment's single query block
// (Q, dO, LSE, delta) is staged once.  Per tile each wave holds its 32 keys'
// K / V rows as operands -- the next tile's are requested into the same
// registers once S and dP are formed -- forms S = Q K^T, dP = dO V^T, P and
// dS, accumulates
// dV^T += dO^T P and dK^T += Q^T dS (stored at the end of the tile) and
// dQ^T += K^T dS^T over all of its tiles in registers (dS rounded to T as
// for dK; K^T and dS^T operands read transposed from the wave's own LDS rows).
// At the end the four waves' dQ^T are summed in a fixed order through LDS and
// written, scaled, as the chunk's fp32 partial rows pbase + r, which
// sum_combine_kernel adds in chunk order.
template <int D>
struct FusedSmem {
  static constexpr int kTile = GTile<D>::kElems;
  static constexpr int kQOff = 0;                     // Q block (GTile)
  static constexpr int kDoOff = kTile * 2;            // dO block (GTile)
  static constexpr int kLsOff = 2 * kTile * 2;        // LSE [32], delta [32]
  static constexpr int kROff = kLsOff + 2 * kRB * 4;  // K rows (a slot per wave), later the dQ^T sums
  static constexpr int kRS = D + 4;                   // fp32 row stride of the sums
  // a wave's slot: its K rows (GTile), after the tile's dQ^T products the
  // dK / dV row-store region (StagedRows, 32 rows of D + 8 elements)
  static constexpr int kSlot = kTile * 2 > 32 * (D * 2 + 16) ? kTile * 2 : 32 * (D * 2 + 16);
  static constexpr int kKtBytes = 4 * kSlot;
  static constexpr int kRedBytes = 4 * 32 * kRS * 4;
  static constexpr int kDsS = 40;                     // dS^T [32 keys][40]
  static constexpr int kDsOff = kROff + (kKtBytes > kRedBytes ? kKtBytes : kRedBytes);
  static constexpr int kBytes = kDsOff + 4 * 32 * kDsS * 2;
};

template <typename T, int D>
__global__ __launch_bounds__(256, 2) void varlen_fkv_kernel(
    const T *__restrict__ q, const T *__restrict__ k, const T *__restrict__ v,
    const T *__restrict__ dout, const float *__restrict__ lse, const float *__restrict__ delta,
    T *__restrict__ dk, T *__restrict__ dv, const int32_t *__restrict__ items, int H, float c,
    float scale, float *__restrict__ part_dq) {
  using M = Mfma<T>;
  using S = FusedSmem<D>;
  using v8 = typename M::v8;
  using L = GTile<D>;
  constexpr int NC = D / 16, ND = D / 32;
  constexpr int kPre = 4;
  static_assert(D <= 64, "the fused kernel serves D <= 64");
  extern __shared__ __align__(16) unsigned char smem_raw[];

  const int item = blockIdx.x / H, h = blockIdx.x % H;
  const PlanItem it = load_item(items, item);
  const int k0 = it.v[0], k1 = it.v[1], q0 = it.v[2], q1 = it.v[3], pbase = it.v[5];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int lrow = lane & 31, lhalf = lane >> 5;

  // the query block (rows past q1 arrive as zeros: Q = dO = 0 there makes
  // all of their products vanish whatever P is); even waves DMA LSE, odd
  // waves delta
  dma_block_rows<T, D, 4>(q, q0, q1, H, h, lds_addr(smem_raw + S::kQOff), wave, lane);
  dma_block_rows<T, D, 4>(dout, q0, q1, H, h, lds_addr(smem_raw + S::kDoOff), wave, lane);
  {
    const float *vec = (wave & 1) ? delta : lse;
    const int rows = uniform_clamp(q1 - q0, kRB);
    const u32x4 rv = rsrc_words32(vec + (int64_t)q0 * H + h, (uint32_t)(rows * H * 4));
    if (lane < kRB)
      lds_dma4(rv, lds_addr(smem_raw + S::kLsOff + (wave & 1) * kRB * 4), lane * H * 4);
  }

  // K / V operands of tile t: this wave's 32 keys (keys past k1 read as zero;
  // their P needs no masking: zero K and V rows make their dQ contribution
  // vanish, and their dK / dV rows are never stored)
  // (a chunk holds at most kFusedTiles * 128 keys: its byte count is formed
  // on the scalar unit in 32 bits, which keeps the descriptors in SGPRs)
  const uint32_t kv_bytes = (uint32_t)(k1 - k0) * (uint32_t)(H * D * 2);
  const rsrc_t rk = make_rsrc32(uniform_ptr(k + (int64_t)k0 * H * D), kv_bytes);
  const rsrc_t rvv = make_rsrc32(uniform_ptr(v + (int64_t)k0 * H * D), kv_bytes);
  const int koff = ((wave * 32 + lrow) * H + h) * D * 2 + lhalf * 16;
  auto load_kv = [&](int t, v8 (&kk)[NC], v8 (&vv)[NC]) {
    const int off = koff + t * 128 * H * D * 2;
#pragma unroll
    for (int cc = 0; cc < NC; ++cc) {
      kk[cc] = as_v8<T>(buf_load16(rk, off + cc * 32));
      vv[cc] = as_v8<T>(buf_load16(rvv, off + cc * 32));
    }
  };
  v8 kf[NC], vf[NC];
  load_kv(0, kf, vf);

  f32x16 dqa[ND];  // dQ^T [d][query] over all of the chunk's keys
#pragma unroll
  for (int dt = 0; dt < ND; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) dqa[dt][r] = 0.f;

  const lds_cptr<T> qs = as_lds(reinterpret_cast<const T *>(smem_raw + S::kQOff));
  const lds_cptr<T> ds_ = as_lds(reinterpret_cast<const T *>(smem_raw + S::kDoOff));
  const float *ls = reinterpret_cast<const float *>(smem_raw + S::kLsOff);
  T *kt = reinterpret_cast<T *>(smem_raw + S::kROff + wave * S::kSlot);
  T *dst = reinterpret_cast<T *>(smem_raw + S::kDsOff) + wave * 32 * S::kDsS;
  const int a_off = L::row(lrow) + lhalf * 8;
  const int t_off = L::row(4 * (lane >> 5) + ((lane & 15) >> 2)) + ((lane >> 4) & 1) * 16 +
                    4 * (lane & 3);
  const int ntile = (k1 - k0 + 127) / 128;
  wait_vmcnt<0>();
  __syncthreads();  // the query block is visible

  // one tile; false when this wave has no keys in it (nor in later tiles)
  auto tile = [&](int t) -> bool {
    const int kw = k0 + t * 128 + wave * 32;  // this wave's first key
    if (kw >= k1) return false;
    // K rows to this wave's LDS rows, K^T operands of dQ^T read back
    // transposed (LDS operations of one wave execute in order)
#pragma unroll
    for (int cc = 0; cc < NC; ++cc)
      *reinterpret_cast<v8 *>(kt + L::row(lrow) + cc * 16 + lhalf * 8) = kf[cc];
    v8 ktf[2 * ND];
#pragma unroll
    for (int hk = 0; hk < 2; ++hk)
#pragma unroll
      for (int dt = 0; dt < ND; ++dt) ktf[hk * ND + dt] = tr_operand_g<T, D>(kt, 16 * hk, 32 * dt, lane);
    // S = Q K^T (even reads, Q rows) and dP = dO V^T (odd reads, dO rows)
    auto aop = [&](int i) { return lds_ld16<T>(((i & 1) ? ds_ : qs) + a_off + (i >> 1) * 16); };
    f32x16 s, dp;
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = dp[r] = 0.f;
    u32x4 ring[kPre];
#pragma unroll
    for (int i = 0; i < kPre; ++i) ring[i] = aop(i);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < 2 * NC; ++i) {
      const v8 a = as_v8<T>(ring[i % kPre]);
      if (i & 1)
        dp = M::mma(a, vf[i >> 1], dp);
      else
        s = M::mma(a, kf[i >> 1], s);
      if (i + kPre < 2 * NC) ring[i % kPre] = aop(i + kPre);
      __builtin_amdgcn_sched_barrier(0);
    }
    // K / V of the next tile, in flight under the rest of this one
    if (t + 1 < ntile) load_kv(t + 1, kf, vf);
    // P = exp2(S*c - LSE), dS = P (dP - delta); row r of a lane is query
    // 8*(r/4) + 4*lhalf + r%4 of the block
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const f32x4 L = *reinterpret_cast<const f32x4 *>(ls + g * 8 + lhalf * 4);
      const f32x4 Dl = *reinterpret_cast<const f32x4 *>(ls + kRB + g * 8 + lhalf * 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = g * 4 + e;
        const float p = fast_exp2(__builtin_fmaf(s[r], c, -L[e]));
        s[r] = p;
        dp[r] = p * (dp[r] - Dl[e]);
      }
    }
    v8 pb[2], sb[2];
#pragma unroll
    for (int mm = 0; mm < 2; ++mm) {
      pb[mm] = pack8<T>(s, 8 * mm);
      sb[mm] = pack8<T>(dp, 8 * mm);
    }
    // dS^T [key][query] of this wave, rounded to T as for dK
    typedef __attribute__((__vector_size__(4 * sizeof(T)))) T T4;
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      T4 w;
#pragma unroll
      for (int e = 0; e < 4; ++e) w[e] = static_cast<T>(dp[4 * r4 + e]);
      *reinterpret_cast<T4 *>(dst + lrow * S::kDsS + 8 * r4 + 4 * lhalf) = w;
    }
    // dV^T += dO^T P and dK^T += Q^T dS: operand i -> d tile i % ND, query
    // half (i / ND) >> 1, dO^T when (i / ND) is even, else Q^T
    f32x16 adk[ND], adv[ND];
#pragma unroll
    for (int i = 0; i < ND; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) adk[i][r] = adv[i][r] = 0.f;
    auto top = [&](int i) {
      const lds_cptr<T> p =
          (((i / ND) & 1) ? qs : ds_) + t_off + ((i / ND) >> 1) * 4 * L::P2 + (i % ND) * 32;
      return as_v8<T>(join(lds_tr8<T>(p), lds_tr8<T>(p + 2 * L::P2)));
    };
    v8 tring[kPre];
#pragma unroll
    for (int i = 0; i < kPre; ++i) tring[i] = top(i);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < 4 * ND; ++i) {
      const int dt = i % ND, q2 = i / ND, mm = q2 >> 1;
      if (q2 & 1)
        adk[dt] = M::mma(tring[i % kPre], sb[mm], adk[dt]);
      else
        adv[dt] = M::mma(tring[i % kPre], pb[mm], adv[dt]);
      if (i + kPre < 4 * ND) tring[i % kPre] = top(i + kPre);
      __builtin_amdgcn_sched_barrier(0);
    }
    // dQ^T += K^T dS^T over the wave's 32 keys (dS^T read transposed in the
    // key order of the K^T operands)
#pragma unroll
    for (int hk = 0; hk < 2; ++hk) {
      const v8 b = tr_operand<T>(dst, S::kDsS, 16 * hk, 0, lane);
#pragma unroll
      for (int dt = 0; dt < ND; ++dt) dqa[dt] = M::mma(ktf[hk * ND + dt], b, dqa[dt]);
    }
    // dK / dV leave as whole rows through the wave's slot (its K rows were
    // read into ktf at the top of the tile; LDS operations of one wave
    // execute in order)
    {
      using SR = StagedRows<T, ND>;
      static_assert(SR::kBytes <= S::kSlot, "row-store region");
      const int64_t off = ((int64_t)kw * H + h) * D;
      const int rows = uniform_clamp(k1 - kw, 32);
      unsigned char *stage = reinterpret_cast<unsigned char *>(kt);
      SR::store(adk, [&](float x) { return static_cast<T>(x * scale); }, stage, dk + off,
                (int64_t)H * D, rows);
      SR::store(adv, [](float x) { return static_cast<T>(x); }, stage, dv + off,
                (int64_t)H * D, rows);
    }
    return true;
  };
  // tile 0 peeled: every entry to the loop then comes after a tile whose
  // dK / dV stores follow its K / V requests, so the compiler's wait for the
  // K / V operands at the top of a tile leaves those stores in flight
  if (ntile > 0 && tile(0))
    for (int t = 1; t < ntile; ++t)
      if (!tile(t)) break;

  // ordered sum of the four waves' dQ^T (a wave without keys adds zeros),
  // scaled: the chunk's partial dQ rows
  __syncthreads();  // every wave is done with its K rows (region R is reused)
  {
    float *red = reinterpret_cast<float *>(smem_raw + S::kROff) + wave * 32 * S::kRS;
#pragma unroll
    for (int dt = 0; dt < ND; ++dt)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        f32x4 w;
#pragma unroll
        for (int e = 0; e < 4; ++e) w[e] = dqa[dt][4 * r4 + e];
        *reinterpret_cast<f32x4 *>(red + lrow * S::kRS + 32 * dt + 8 * r4 + 4 * lhalf) = w;
      }
  }
  __syncthreads();
  const int row = tid >> 3, cs = tid & 7;  // 32 rows x 8 column segments
  if (q0 + row < q1) {
    const float *red = reinterpret_cast<const float *>(smem_raw + S::kROff);
    float *prow = part_dq + ((int64_t)(pbase + row) * H + h) * D;
#pragma unroll
    for (int c4 = 0; c4 < D / 32; ++c4) {
      const int col = cs * (D / 8) + 4 * c4;
      f32x4 acc = *reinterpret_cast<const f32x4 *>(red + row * S::kRS + col);
#pragma unroll
      for (int w = 1; w < 4; ++w)
        acc += *reinterpret_cast<const f32x4 *>(red + (w * 32 + row) * S::kRS + col);
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[e] *= scale;
      *reinterpret_cast<f32x4 *>(prow + col) = acc;
    }
  }
}

// A [kRB x D] block of a [T, H, D] tensor staged through registers: 16-byte
// chunks, rows past the buffer range read as zero.
template <int D, int NT>
struct Rows {
  static constexpr int kChunks = kRB * D / 8;
  static constexpr int kPer = (kChunks + NT - 1) / NT;
  u32x4 v[kPer];
};

template <typename T, int D, int NT>
__device__ __forceinline__ void load_rows(Rows<D, NT> &s, const T *__restrict__ src, int r0,
                                          int r_end, int H, int h, int t) {
  constexpr int CPR = D / 8;
  const int rows = uniform_clamp(r_end - r0, kRB);
  const rsrc_t rs = make_rsrc32(src + (int64_t)r0 * H * D, (uint32_t)(rows * H * D * 2));
#pragma unroll
  for (int i = 0; i < Rows<D, NT>::kPer; ++i) {
    const int ci = t + NT * i;
    const int row = ci < Rows<D, NT>::kChunks ? ci / CPR : kRB;
    s.v[i] = buf_load16(rs, (row * H + h) * D * 2 + (ci % CPR) * 16);
  }
}

template <typename T, int D, int NT>
__device__ __forceinline__ void store_rows(const Rows<D, NT> &s, T *dst, int t) {
  constexpr int CPR = D / 8;
#pragma unroll
  for (int i = 0; i < Rows<D, NT>::kPer; ++i) {
    const int ci = t + NT * i;
    if (ci < Rows<D, NT>::kChunks)
      *reinterpret_cast<u32x4 *>(dst + GTile<D>::row(ci / CPR) + (ci % CPR) * 8) = s.v[i];
  }
}

template <int D>
struct DqSmem {
  static constexpr int kKs = GTile<D>::kElems;
  static constexpr int kBuf = 2 * kKs;  // K and V row-major
  static constexpr int kBytes = 2 * kBuf * 2;
};

template <typename T, int D, int NW>
__global__ __launch_bounds__(64 * NW, D >= 256 ? 1 : 2) void varlen_dq_kernel(
    const T *__restrict__ q, const T *__restrict__ k, const T *__restrict__ v,
    const T *__restrict__ dout, const float *__restrict__ lse, float *delta,
    const T *__restrict__ o_fused, T *__restrict__ dq, float *__restrict__ part_dq,
    const int32_t *__restrict__ items, int H, float c, float scale) {
  using M = Mfma<T>;
  using S = DqSmem<D>;
  using L = GTile<D>;
  constexpr int NC = D / 16, ND = D / 32;
  constexpr int kPre = 4;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  T *smem = reinterpret_cast<T *>(smem_raw);

  const int item = blockIdx.x / H, h = blockIdx.x % H;
  const PlanItem it = load_item(items, item);
  const int q0 = it.v[0], q1 = it.v[1], k0 = it.v[2], k1 = it.v[3], pbase = it.v[4];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int lrow = lane & 31, lhalf = lane >> 5;
  const int qrow = q0 + wave * 32 + lrow;
  const bool row_ok = qrow < q1;
  const bool wave_active = q0 + wave * 32 < q1;

  // key blocks staged through registers (the first half of the waves K, the
  // second V; rows past k1 read as zero): a block's loads are issued before
  // the previous block's compute and written to LDS after it.  (Per-row
  // LDS-DMA moves only D*2 bytes per instruction, which costs more than it
  // saves here.)
  constexpr int NS = 32 * NW;  // staging threads per tensor
  const bool stage_k = wave < NW / 2;
  const int st = tid & (NS - 1);
  const T *src = stage_k ? k : v;
  Rows<D, NS> stg;
  auto put = [&](int buf) {
    T *ks = smem + buf * S::kBuf;
    store_rows<T, D, NS>(stg, stage_k ? ks : ks + S::kKs, st);
  };
  const int nblk = (k1 - k0 + kRB - 1) / kRB;
  if (nblk > 0) load_rows<T, D, NS>(stg, src, k0, k1, H, h, st);

  typename M::v8 qf[NC], dof[NC];
  // O rows for delta (fused mode), requested with Q and dO: one round trip
  const bool fused = o_fused != nullptr;
  u32x4 ov[NC];
  {
    const int64_t nb = (int64_t)(q1 - q0) * H * D * 2;
    const rsrc_t rq = make_rsrc(q + (int64_t)q0 * H * D, nb);
    const rsrc_t rd = make_rsrc(dout + (int64_t)q0 * H * D, nb);
    const int off = ((wave * 32 + lrow) * H + h) * D * 2 + lhalf * 16;
    if (fused) {
      const rsrc_t ro = make_rsrc(o_fused + (int64_t)q0 * H * D, nb);
#pragma unroll
      for (int cc = 0; cc < NC; ++cc) ov[cc] = buf_load16(ro, off + cc * 32);
    }
#pragma unroll
    for (int cc = 0; cc < NC; ++cc) {
      u32x4 a = buf_load16(rq, off + cc * 32), b = buf_load16(rd, off + cc * 32);
      asm volatile("" : "+v"(a), "+v"(b));  // waited for in the prologue
      qf[cc] = as_v8<T>(a);
      dof[cc] = as_v8<T>(b);
    }
  }
  float Lr = row_ok ? lse[(int64_t)qrow * H + h] : __builtin_inff();
  float Dr;
  if (fused) {
    // delta = rowsum(O * dO) from the dO operands and the O rows read in the
    // same layout, summed in row_dot_kernel's order (per 16-byte chunk
    // sequentially, then a butterfly over the chunks; this lane holds chunks
    // 2*cc + lhalf) so both produce the same bits.  The item that owns the
    // rows' first key range writes it for dK/dV.
    float sc[NC];
#pragma unroll
    for (int cc = 0; cc < NC; ++cc) {
      const T *x = reinterpret_cast<const T *>(&ov[cc]);
      float acc_c = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc_c = __builtin_fmaf(to_f(x[e]), to_f(dof[cc][e]), acc_c);
      sc[cc] = acc_c;
    }
#pragma unroll
    for (int half = NC / 2; half >= 1; half /= 2)
#pragma unroll
      for (int cc = 0; cc < half; ++cc) sc[cc] = sc[cc] + sc[cc + half];
    Dr = sc[0] + __shfl_xor(sc[0], 32, 64);
    if (row_ok && lhalf == 0 && it.v[6] == 0) delta[(int64_t)qrow * H + h] = Dr;
  } else {
    Dr = row_ok ? delta[(int64_t)qrow * H + h] : 0.f;
  }
  asm volatile("" : "+v"(Lr), "+v"(Dr));
  // At D = 128 (registers to spare) the dO operands enter negated (an exact
  // sign flip, after delta is formed from them) and the dP^T chain starts
  // from a block holding this lane's delta: it yields delta - dP, and
  // dS = P (dP - delta) is one multiply with a negated operand.
  constexpr bool kDeltaInChain = D == 128;
  f32x16 drb;
#pragma unroll
  for (int r = 0; r < 16; ++r) drb[r] = kDeltaInChain ? Dr : 0.f;
  if constexpr (kDeltaInChain) {
#pragma unroll
    for (int cc = 0; cc < NC; ++cc) {
      u32x4 w = __builtin_bit_cast(u32x4, dof[cc]);
#pragma unroll
      for (int e = 0; e < 4; ++e) w[e] ^= 0x80008000u;
      dof[cc] = as_v8<T>(w);
    }
  }
  f32x16 acc[ND];
#pragma unroll
  for (int i = 0; i < ND; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[i][r] = 0.f;

  const int a_off = L::row(lrow) + lhalf * 8;
  const int t_off = L::row(4 * (lane >> 5) + ((lane & 15) >> 2)) + ((lane >> 4) & 1) * 16 +
                    4 * (lane & 3);
  if (nblk > 0) put(0);
  __syncthreads();
  // Only the last key block can reach past k1, and only there are the dS
  // columns of those keys masked: the loop body is instantiated twice so the
  // other blocks carry no per-element key compares (if-converted, they were
  // 48 VALU instructions per block).
  // bufc: the block's LDS buffer, a compile-time constant when the loop
  // below is paired, else j & 1
  auto block = [&](int j, auto masked, auto bufc) {
    const int B = bufc;
    const int kb = k0 + j * kRB;
    if (j + 1 < nblk) load_rows<T, D, NS>(stg, src, kb + kRB, k1, H, h, st);
    if (wave_active) {
      const lds_cptr<T> ks = as_lds(smem + B * S::kBuf);
      const lds_cptr<T> vs = ks + S::kKs;
      // S^T = K Q^T (even reads, K rows) and dP^T = V dO^T (odd reads, V
      // rows; delta - dP^T when kDeltaInChain)
      auto aop = [&](int i) { return lds_ld16<T>(((i & 1) ? vs : ks) + a_off + (i >> 1) * 16); };
      f32x16 s, dp = drb;
#pragma unroll
      for (int r = 0; r < 16; ++r) s[r] = 0.f;
      u32x4 ring[kPre];
#pragma unroll
      for (int i = 0; i < kPre; ++i) ring[i] = aop(i);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < 2 * NC; ++i) {
        const typename M::v8 a = as_v8<T>(ring[i % kPre]);
        if (i & 1)
          dp = M::mma(a, dof[i >> 1], dp);
        else
          s = M::mma(a, qf[i >> 1], s);
        if (i + kPre < 2 * NC) ring[i % kPre] = aop(i + kPre);
        __builtin_amdgcn_sched_barrier(0);
      }
      // K^T operands of dQ^T: i -> d tile i % ND, key half i / ND
      auto top = [&](int i) {
        const lds_cptr<T> p = ks + t_off + (i / ND) * 4 * L::P2 + (i % ND) * 32;
        return as_v8<T>(join(lds_tr8<T>(p), lds_tr8<T>(p + 2 * L::P2)));
      };
      typename M::v8 tring[kPre];
#pragma unroll
      for (int i = 0; i < kPre; ++i) tring[i] = top(i);
      // element r holds key kb + (r/4)*8 + lhalf*4 + r%4 of this lane's row
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = fast_exp2(__builtin_fmaf(s[r], c, -Lr));
        if constexpr (kDeltaInChain)
          dp[r] = -(p * dp[r]);
        else
          dp[r] = p * (dp[r] - Dr);
      }
      if constexpr (decltype(masked)::value) {
        if (kb + kRB > k1) {
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (kb + (r >> 2) * 8 + lhalf * 4 + (r & 3) >= k1) dp[r] = 0.f;
        }
      }
      typename M::v8 sb[2];
#pragma unroll
      for (int mm = 0; mm < 2; ++mm) sb[mm] = pack8<T>(dp, mm * 8);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < 2 * ND; ++i) {
        acc[i % ND] = M::mma(tring[i % kPre], sb[i / ND], acc[i % ND]);
        if (i + kPre < 2 * ND) tring[i % kPre] = top(i + kPre);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    if (j + 1 < nblk) put(1 - B);
    __syncthreads();
  };
  // At D >= 128 two blocks per trip, so each block's LDS buffer is a
  // compile-time offset folded into the LDS reads' immediates (at D = 64 the
  // paired body needs more registers than four waves per SIMD allow); the
  // last block is the masked one.
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  int j = 0;
  if constexpr (D >= 128) {
    for (; j + 2 < nblk; j += 2) {
      block(j, std::false_type{}, I0{});
      block(j + 1, std::false_type{}, I1{});
    }
    if (j + 1 < nblk) {
      block(j, std::false_type{}, I0{});
      block(j + 1, std::true_type{}, I1{});
    } else if (j < nblk) {
      block(j, std::true_type{}, I0{});
    }
  } else {
    for (; j + 1 < nblk; ++j) block(j, std::false_type{}, j & 1);
    if (j < nblk) block(j, std::true_type{}, j & 1);
  }

  if (!wave_active) return;
  // dQ (or a split's fp32 partial rows) leaves as whole rows through the
  // wave's LDS region (the K/V buffers, free after the loop's last barrier);
  // stored from the accumulators it cost 5% of the C2 dQ kernel.
  using RS = RowStore<T, ND>;
  unsigned char *stage = smem_raw + wave * RS::kBytes;
  const int rows = uniform_clamp(q1 - (q0 + wave * 32), 32);
  if (pbase < 0)
    RS::rows16(acc, [&](float x) { return static_cast<T>(x * scale); }, stage,
               dq + ((int64_t)(q0 + wave * 32) * H + h) * D, (int64_t)H * D, rows);
  else
    RS::rows32(acc, scale, stage, part_dq + ((int64_t)(pbase + wave * 32) * H + h) * D,
               (int64_t)H * D, rows);
}

}  // namespace

template <typename T, int D, int NW>
void launch_dkv_nw(const VarlenArgs &a, hipStream_t st) {
  const int smem = dkv_lds_bytes<T, D, NW>();
  allow_dynamic_lds(reinterpret_cast<const void *>(&varlen_dkv_kernel<T, D, NW>), smem);
  hipLaunchKernelGGL((varlen_dkv_kernel<T, D, NW>),
                     dim3((unsigned)(a.n_kv * a.H)), dim3(64 * NW), smem, st,
                     (const T *)a.q, (const T *)a.k, (const T *)a.v, (const T *)a.dout,
                     a.lse_in, a.delta, (T *)a.dk, (T *)a.dv, a.kv_items, a.H,
                     a.scale * kLog2e, a.scale);
}

// The plan's key tile sets the workgroup: 32 keys per wave.
template <typename T, int D>
void launch_mfma_varlen_dkv(const VarlenArgs &a, hipStream_t st) {
  if (a.n_kv == 0) return;
  if constexpr (D == 256) {
    launch_dkv_nw<T, D, 8>(a, st);  // 128 keys: two waves per 32 keys
  } else {
    if constexpr (D == 128) {
      if (a.k_tile == kVarlenWideTile) return launch_dkv_nw<T, D, 8>(a, st);
    }
    launch_dkv_nw<T, D, 4>(a, st);
  }
}

template <typename T, int D>
void launch_mfma_varlen_fkv(const VarlenArgs &a, hipStream_t st) {
  if (a.n_fkv == 0) return;
  const int smem = FusedSmem<D>::kBytes;
  allow_dynamic_lds(reinterpret_cast<const void *>(&varlen_fkv_kernel<T, D>), smem);
  hipLaunchKernelGGL((varlen_fkv_kernel<T, D>), dim3((unsigned)(a.n_fkv * a.H)), dim3(256),
                     smem, st, (const T *)a.q, (const T *)a.k, (const T *)a.v,
                     (const T *)a.dout, a.lse_in, a.delta, (T *)a.dk, (T *)a.dv, a.fkv_items, a.H,
                     a.scale * kLog2e, a.scale, a.part_fq);
}

// Dynamic LDS of the dQ kernel: the K/V block buffers, or the per-wave
// row-store regions of the epilogue if those are larger.
template <typename T, int D, int NW>
constexpr int dq_lds_bytes() {
  constexpr int kStage = NW * RowStore<T, D / 32>::kBytes;
  return DqSmem<D>::kBytes > kStage ? DqSmem<D>::kBytes : kStage;
}

template <typename T, int D, int NW>
void launch_dq_nw(const VarlenArgs &a, hipStream_t st) {
  const int smem = dq_lds_bytes<T, D, NW>();
  allow_dynamic_lds(reinterpret_cast<const void *>(&varlen_dq_kernel<T, D, NW>), smem);
  hipLaunchKernelGGL((varlen_dq_kernel<T, D, NW>), dim3((unsigned)(a.n_items * a.H)),
                     dim3(64 * NW), smem, st, (const T *)a.q, (const T *)a.k, (const T *)a.v,
                     (const T *)a.dout, a.lse_in, a.delta,
                     a.fuse_delta ? (const T *)a.o_in : nullptr, (T *)a.dq, a.part_o, a.items,
                     a.H, a.scale * kLog2e, a.scale);
}

// dQ runs over the forward's query tiles: 32 rows per wave.
template <typename T, int D>
void launch_mfma_varlen_dq(const VarlenArgs &a, hipStream_t st) {
  if (a.n_items == 0) return;
  if constexpr (D <= 128) {
    if (a.q_tile == kVarlenWideTile) return launch_dq_nw<T, D, 8>(a, st);
  }
  launch_dq_nw<T, D, 4>(a, st);
}

#define VAFA_INST(T, D)                                                           \
  template void launch_mfma_varlen_dkv<T, D>(const VarlenArgs &, hipStream_t);    \
  template void launch_mfma_varlen_dq<T, D>(const VarlenArgs &, hipStream_t);
#define VAFA_INST_F(T, D) \
  template void launch_mfma_varlen_fkv<T, D>(const VarlenArgs &, hipStream_t);
VAFA_INST(bf16, 32)
VAFA_INST(bf16, 64)
VAFA_INST(bf16, 128)
VAFA_INST(f16, 32)
VAFA_INST(f16, 64)
VAFA_INST(f16, 128)
VAFA_INST(bf16, 256)
VAFA_INST(f16, 256)
VAFA_INST_F(bf16, 32)
VAFA_INST_F(bf16, 64)
VAFA_INST_F(f16, 32)
VAFA_INST_F(f16, 64)
#undef VAFA_INST
#undef VAFA_INST_F

}  // namespace vafa
