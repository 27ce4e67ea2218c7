// Launch arguments and launcher declarations shared by the C ABI and the
// kernel translation units.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace vafa {

// Lets kernel `fn` be launched with `bytes` of dynamic LDS (above the 64 KB
// default).  A failure is not returned here: HIP keeps it as the thread's
// last error, so the launch that follows fails and every entry point reports
// it through check_launch (hipGetLastError) as VAFA_ERR_RUNTIME.
inline void allow_dynamic_lds(const void *fn, int bytes) {
  const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  (void)e;
}

struct VarlenArgs {
  const void *q, *k, *v, *o_in, *dout;
  void *o, *dq, *dk, *dv;
  float *lse;            // forward output [T_q, H]
  const float *lse_in;   // backward input [T_q, H]
  float *delta;          // [T_q, H] workspace (backward)
  float *part_o;         // split partial rows: O (fwd) or dQ (bwd), [rows, H, D]
  float *part_lse;       // split partial LSE [rows, H] (fwd)
  const int32_t *items, *comb_items, *kv_items;
  int64_t n_items, n_comb, n_kv;
  int comb_rows;         // most rows of one combine item
  int64_t T_q;
  int H, D;
  int q_tile, k_tile;  // the plan's tiles: forward / dQ rows and dK/dV keys per workgroup
  int xcd_heads;       // forward grid: an item's H workgroups on one XCD (1) or item-major
  float scale;
  int stage;  // backward stage (VAFA_BWD_*) or -1 for all
  // the matrix-core dQ kernel computes delta from O and dO itself and writes
  // it for dK/dV (no separate row_dot launch)
  bool fuse_delta;
  // backward: the dQ pass's items (forward items of the segments that are not
  // fused) and the fused K-major pass (key tiles, partial-dQ sums)
  const int32_t *dq_items, *dqc_items, *fkv_items, *fcomb_items;
  int64_t n_dq, n_dqc, n_fkv, n_fcomb;
  int dqc_rows, fcomb_rows;
  float *part_fq;  // fused dQ partial rows [n_fpart_rows, H, D] fp32
};

struct AbsorbArgs {
  const void *u, *X, *wv, *O_in, *dO;
  void *O, *du, *dX, *dwv;
  float *lse;
  const float *lse_in;
  float *delta;
  float *part_o, *part_lse;   // split partial rows [rows, H, D_H] / [rows, H]
  void *dax;                  // dO W_V^T [T_q, H, F] in the input dtype (backward)
  float *ax;                  // aX [T_q, H, F] fp32 (backward, for dW_V)
  float *dwv_part;            // [n_tchunks, F, H, D_H] fp32 (backward)
  void *wvt;                  // W_V re-laid out as [H, D_H, F padded to 32] (forward)
  // forward with mfma_absorb_unprojected: rounded aX/l rows [T_q, H, FP] in
  // wvt's f order (part_o then holds [rows, H, FP] unprojected partials)
  void *axf;
  // Folded projection (forward): `u` holds q_proj [T_q, H, D_H] instead of u,
  // and each workgroup forms its rows' u = q_proj_h W_K,h^T from `wk`
  // (W_K [F, H, D_H]) re-laid out into `wkt` ([H, F padded to 32, D_H padded
  // to 32], zeros in the padding).
  const void *wk;
  void *wkt;
  bool fold;
  const int32_t *items, *comb_items, *kv_items, *qseg_items;
  int64_t n_items, n_comb, n_kv, n_qseg;
  int64_t n_kv_res;           // leading kv items for absorb_dx_res_kernel
  int comb_rows;              // most tokens of one combine item
  int64_t T_q, T_k;
  int64_t n_tchunks, tchunk;
  int H, F, DH;
  float scale;
};

// varlen_f32.hip: fp32 varlen on fp32 matrix cores
bool f32_varlen_mfma_d(int D);      // D in {32, 64, 128, 256}
bool f32_varlen_bwd_mfma_d(int D);  // D in {32, 64, 128}
void launch_f32_varlen_fwd(const VarlenArgs &, hipStream_t);
void launch_f32_varlen_dq(const VarlenArgs &, hipStream_t);
void launch_f32_varlen_dkv(const VarlenArgs &, hipStream_t);

// simt.hip
template <typename T> void launch_simt_varlen_fwd(const VarlenArgs &, hipStream_t);
template <typename T> void launch_simt_varlen_dq(const VarlenArgs &, hipStream_t);
template <typename T> void launch_simt_varlen_dkv(const VarlenArgs &, hipStream_t);
template <typename T> void launch_simt_absorb_fwd(const AbsorbArgs &, hipStream_t);
template <typename T> void launch_simt_absorb_du(const AbsorbArgs &, hipStream_t);
template <typename T> void launch_simt_absorb_dx(const AbsorbArgs &, hipStream_t);

// reduce.hip
// delta[t,h] = sum_d O[t,h,d] * dO[t,h,d] (fa/kernels.py:186-216)
template <typename T>
void launch_row_dot(const void *o, const void *dout, float *delta, int64_t rows, int D,
                    hipStream_t);
// LSE-weighted merge of split partials into out / lse (fa/kernels.py:652-734);
// every combine item covers at most max_rows rows, D <= 256
template <typename T>
void launch_lse_combine(const float *part_o, const float *part_lse, void *out, float *lse,
                        const int32_t *comb_items, int64_t n_comb, int H, int D, int max_rows,
                        hipStream_t);
// Plain ordered sum of split partials (dQ): out = sum_s part[s]
template <typename T>
void launch_sum_combine(const float *part, void *out, const int32_t *comb_items, int64_t n_comb,
                        int H, int D, int max_rows, hipStream_t);
// dW_V = sum_t aX[t]^T dO[t] per head, two-level deterministic reduction.
template <typename T>
void launch_absorb_dwv(const AbsorbArgs &, hipStream_t);
// Weight gradient out[f, g, d] = sum_t A[t, g, f] B[t, g, d] (A [T, G, F], B
// [T, G, DH], out in B's dtype): ordered fp32 partials over n_chunks token
// chunks of tchunk tokens (part holds n_chunks * F * G * DH floats), then
// their sum in chunk order.  TA is float or T.
template <typename TA, typename T>
void launch_wgrad(const void *a, const void *b, float *part, void *out, int64_t T_q,
                  int64_t tchunk, int64_t n_chunks, int G, int F, int DH, hipStream_t);
// rows [rows, 16] -> zero-padded [rows, 32], and the first 16 columns back
// (elem_bytes: 2 for 16-bit elements, 4 for fp32)
void launch_pad16(const void *src, void *dst, int64_t rows, int elem_bytes, hipStream_t);
void launch_unpad16(const void *src, void *dst, int64_t rows, int elem_bytes, hipStream_t);
// rows [rows, n] -> zero-padded [rows, m] (m >= n), and the first n columns
// back (elem_bytes 2 or 4)
void launch_pad_cols(const void *src, void *dst, int64_t rows, int64_t n, int64_t m,
                     int elem_bytes, hipStream_t);
void launch_unpad_cols(const void *src, void *dst, int64_t rows, int64_t n, int64_t m,
                       int elem_bytes, hipStream_t);
// out[o] = sum_c part[c * n_out + o] in chunk order, rounded to T
template <typename T>
void launch_chunk_sum(const float *part, void *out, int64_t n_out, int64_t n_chunks, hipStream_t);
// dAX = dO W_V^T, fp32 [T_q, H, F]
template <typename T>
void launch_absorb_dax(const AbsorbArgs &, hipStream_t);

// varlen_mfma.hip (bf16 / f16, D in {32, 64, 128, 256})
template <typename T, int D> void launch_mfma_varlen_fwd(const VarlenArgs &, hipStream_t);
template <typename T, int D> void launch_mfma_varlen_dq(const VarlenArgs &, hipStream_t);
template <typename T, int D> void launch_mfma_varlen_dkv(const VarlenArgs &, hipStream_t);
// fused dQ/dK/dV over the fkv items (D <= 128): dK, dV and dQ partial rows
template <typename T, int D> void launch_mfma_varlen_fkv(const VarlenArgs &, hipStream_t);

// absorb_mfma.hip (bf16 / f16)
template <typename T> bool mfma_absorb_supported(int H, int F, int DH);
template <typename T> bool mfma_absorb_fwd_supported(int H, int F, int DH);
int64_t mfma_absorb_wvt_elems(int H, int F, int DH);
bool mfma_absorb_unprojected(int H, int F, int DH, bool fold);
bool mfma_absorb_fold_supported(int H, int F, int DH);
int absorb_heads_per_wave(int H);
int64_t mfma_absorb_wkt_elems(int H, int F, int DH);
template <typename T> void launch_mfma_absorb_fwd(const AbsorbArgs &, hipStream_t);

// absorb_project.hip (bf16 / f16): Y[t, g*ys + j] = sum_k X[t*ldx + g*xs + k]
// * W[g*ws + j*ldw + k] for t < T_q, g < G, j < J, k < K; fp32 accumulation,
// one rounding.  Needs K % 8 == 0, J % 8 == 0, every stride % 8 == 0 and
// 16-byte aligned X, W, Y.
struct RowGemm {
  const void *X, *W;
  void *Y;
  int64_t T_q;
  int G, J, K;
  int64_t ldx, xs, ws, ldw, ldy, ys;
};
bool rowgemm_supported(const RowGemm &);
// Weight gradient out[f, g, d] = sum_t A[t, g, f] B[t, g, d] on 16-bit
// matrix cores (A [T, G, F] with F <= 512, B [T, G, DH]): fp32 partials over
// n_chunks chunks of tchunk tokens (a multiple of 32; part holds n_chunks * F
// * G * DH floats) summed in chunk order into out.  With dq != nullptr also
// dq[t, g, d] = sum_f A[t, g, f] Wt[g, d, f] (Wt [G, DH, F]), rounded once.
struct Wgrad {
  const void *A, *B, *Wt;
  void *dq, *out;
  float *part;
  int64_t T_q, tchunk, n_chunks;
  int G, F, DH;
};
bool wgrad16_supported(int F);
template <typename T> void launch_wgrad16(const Wgrad &, hipStream_t);
template <typename T> void launch_rowgemm(const RowGemm &, hipStream_t);
// dst [C, R] = src [R, C]^T
template <typename T> void launch_transpose2d(const void *src, void *dst, int R, int C, hipStream_t);
// absorb_bwd_mfma.hip: du/aX (query side) and dX (key side) on matrix cores
template <typename T> void launch_mfma_absorb_du(const AbsorbArgs &, hipStream_t);
// dAX = dO W_V^T; false (nothing launched) for a D_H it does not cover
template <typename T> bool launch_mfma_absorb_dax(const AbsorbArgs &, hipStream_t);
template <typename T> void launch_mfma_absorb_dx(const AbsorbArgs &, hipStream_t);

// absorb_f32.hip: fp32 absorb on fp32 matrix cores (v_mfma_f32_16x16x4_f32)
bool f32_absorb_supported(int H, int F, int DH);      // backward (D_KV <= 256)
bool f32_absorb_fwd_supported(int H, int F, int DH);  // forward (D_KV <= 512)
int64_t f32_absorb_wvt_elems(int H, int F, int DH);
void launch_f32_absorb_fwd(const AbsorbArgs &, hipStream_t);
// dAX = dO W_V^T in fp32 on fp32 matrix cores (F % 4 == 0, D_H % 16 == 0)
void launch_f32_absorb_dax(const AbsorbArgs &, hipStream_t);
// du / aX (query side) and dX (key side); dAX and delta must be in the workspace
void launch_f32_absorb_du_dx(const AbsorbArgs &, hipStream_t);

}  // namespace vafa
