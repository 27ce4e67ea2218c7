/*
 * vafa.h -- C ABI of the MI355X (gfx950) implementation of packed varlen
 * FlashAttention and absorbed ragged target attention.
 *
 * Every entry point is plain C: device pointers, int64 sizes, a dtype enum,
 * a caller-owned workspace and a hipStream_t passed as void*.  Calls are
 * asynchronous on that stream, never allocate device memory and never sync
 * the host.  They return VAFA_OK (0) or a negative status; the message for
 * the last failure on the calling thread is available from
 * vafa_last_error().
 *
 * Reference interfaces replaced (paths relative to the reference checkout):
 *   fa/ = triton_fa_varlen_v2/triton_fa_varlen_v2/
 *   ta/ = triton_target_attn_absorb/triton_target_attn_absorb/
 */
#ifndef VAFA_H_
#define VAFA_H_

#include <stdint.h>

#if defined(__GNUC__) || defined(__clang__)
#define VAFA_API __attribute__((visibility("default")))
#else
#define VAFA_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------ */
#define VAFA_OK 0
#define VAFA_ERR_VALUE (-1)     /* maps to Python ValueError               */
#define VAFA_ERR_ASSERT (-2)    /* maps to Python AssertionError           */
#define VAFA_ERR_RUNTIME (-3)   /* HIP launch/runtime failure              */
#define VAFA_ERR_WORKSPACE (-4) /* workspace too small or misaligned       */
#define VAFA_ERR_CAPACITY (-5)  /* host output buffer too small            */

/* ---- dtypes -------------------------------------------------------------- */
#define VAFA_F32 0
#define VAFA_F16 1
#define VAFA_BF16 2

/* ---- misc ---------------------------------------------------------------- */
VAFA_API const char *vafa_version(void);
/* Message of the last failing call on this thread ("" if none). */
VAFA_API const char *vafa_last_error(void);

/* ======================================================================== */
/* Host metadata (pure C++, no device access; usable without a GPU).        */
/* ======================================================================== */

/* Replaces fa/interface.py:74-93 (_seqinfo_to_cu_seqlens).
 * seqinfo[n] -> cu_out[n+1] int32; VAFA_ERR_VALUE for n==0, a negative
 * length or a total above INT32_MAX. */
VAFA_API int vafa_seqinfo_to_cu(const int64_t *seqinfo, int64_t n, int32_t *cu_out);

/* Replaces fa/interface.py:96-118 (_validate_cu_seqlens of the varlen
 * operator): n1 >= 2, cu[0]==0, cu[n1-1]==T, non-decreasing.
 * `name` is used in the error message. */
VAFA_API int vafa_validate_cu(const int64_t *cu, int64_t n1, int64_t T, const char *name);

/* Replaces ta/interface.py:92-106 (_validate_cu_seqlens of the absorb
 * operator): the same checks in the same order, with that operator's error
 * texts ("<name>[0] must be 0", "<name> must be non-decreasing", ...). */
VAFA_API int vafa_validate_cu_absorb(const int64_t *cu, int64_t n1, int64_t T, const char *name);

/* Replaces ta/interface.py:109-116 (_validate_active_segments_have_keys). */
VAFA_API int vafa_check_active_have_keys(const int64_t *cu_q, const int64_t *cu_k, int64_t n1);

/* Replaces fa/chunk_indices.py:25-65 and ta/chunk_indices.py:19-54
 * (_prepare_chunk_indices): rows (seg, block) for block < ceil(L/BT).
 * out holds cap rows of 2 int32; *n_rows receives the row count (also when
 * VAFA_ERR_CAPACITY is returned). */
VAFA_API int vafa_chunk_indices(const int64_t *cu, int64_t n1, int32_t BT, int32_t *out,
                       int64_t cap, int64_t *n_rows);

/* ======================================================================== */
/* Work plans.                                                              */
/*                                                                          */
/* A plan is a flat int32 array built on the host from host copies of       */
/* cu_seqlens and copied once to the device.  It replaces the reference's   */
/* SplitIndices / chunk-index tables (fa/chunk_indices.py:144-287,          */
/* ta/chunk_indices.py:19-67).  Items hold absolute token offsets, are      */
/* ordered longest-first and every long-tail (segment, q-tile) is split     */
/* over the key axis; the combine tables merge the split partials.          */
/* ======================================================================== */

#define VAFA_ITEM_INTS 8 /* every work item is 8 int32 (32 bytes) */
#define VAFA_PLAN_MAGIC 0x56414641 /* "VAFA" */

typedef struct vafa_plan_info {
  int64_t magic;          /* VAFA_PLAN_MAGIC */
  int64_t kind;           /* 1 = varlen, 2 = absorb */
  int64_t n_seg;
  int64_t T_q, T_k, H;
  /* section offsets (in int32 units from the plan start) and item counts */
  int64_t off_fwd, n_fwd;         /* forward / dq items (query tiles)      */
  int64_t off_comb, n_comb;       /* combine items                         */
  int64_t off_kv, n_kv;           /* key-tile items (dK/dV, absorb dX)     */
  int64_t off_qt, n_qt;           /* unsplit query tiles (absorb dU pass)  */
  int64_t n_part_rows;            /* partial rows written by split items   */
  int64_t plan_ints;              /* total plan length in int32            */
  int64_t q_tile, k_tile;         /* tile sizes the plan was built for:
                                     varlen picks 128 or 256 per call (256
                                     only for the head dims whose kernels run
                                     it; entry points called with another D
                                     return VAFA_ERR_VALUE)                  */
  int64_t max_split;              /* largest number of splits of one tile  */
  int64_t max_comb_rows;          /* most rows (tokens) of one combine item */
  int64_t n_kv_res;               /* absorb: the leading key-tile items whose
                                     segment has at most 64 (token, head) rows */
  /* varlen backward: the dQ pass runs over the forward items of the
   * segments that are not fused (dq, dqc: filtered copies of fwd, comb);
   * fused segments (at most 16 queries, D <= 64) run dQ/dK/dV in one
   * K-major pass over fkv items whose fp32 dQ partials fcomb sums. */
  int64_t off_dq, n_dq;           /* dQ-pass items                          */
  int64_t off_dqc, n_dqc;         /* dQ-pass combine items                  */
  int64_t max_dqc_rows;
  int64_t off_fkv, n_fkv;         /* fused key-chunk items                  */
  int64_t off_fcomb, n_fcomb;     /* fused dQ-partial sums                  */
  int64_t n_fpart_rows;           /* fused dQ partial rows                  */
  int64_t max_fcomb_rows;
  /* varlen forward grid: 1 = the H heads of a forward item run on one XCD
   * (most of the work lies in segments of at most 128 queries, whose items
   * share no key range: the heads then read whole token rows together);
   * 0 = item-major with heads innermost (the query tiles of a segment share
   * its K/V in one XCD's L2) */
  int64_t xcd_heads;
} vafa_plan_info;

/* Plan for packed_varlen_attn (fa/interface.py:184-236, 293-338).
 * cu_q/cu_k: host int64 [n1].  D and the segment lengths select the tile
 * sizes: the plan serves calls with this head dim.  Call with plan==NULL to
 * size (info->plan_ints), then with a buffer of that many int32. */
VAFA_API int vafa_plan_varlen(const int64_t *cu_q, const int64_t *cu_k, int64_t n1, int64_t H,
                     int64_t D, int32_t *plan, int64_t plan_cap, vafa_plan_info *info);

/* Plan for packed_target_attn (ta/interface.py:191-216, 265-314). */
VAFA_API int vafa_plan_absorb(const int64_t *cu_q, const int64_t *cu_k, int64_t n1, int64_t H,
                     int64_t D_KV, int64_t D_H, int32_t *plan, int64_t plan_cap,
                     vafa_plan_info *info);

/* ======================================================================== */
/* Device entry points.  plan_dev is the plan copied to device memory.      */
/* workspace: device memory of at least the size the *_workspace query     */
/* returns, 256-byte aligned.  stream: hipStream_t.                          */
/* ======================================================================== */

/* Workspace bytes needed by vafa_varlen_fwd / vafa_varlen_bwd.  For D=16 this
 * includes zero-padded D=32 copies of the operands (sized for fp32 rows):
 * D=16 calls run on the D=32 matrix-core kernels over them. */
VAFA_API int64_t vafa_varlen_fwd_workspace(const vafa_plan_info *info, int64_t D);
VAFA_API int64_t vafa_varlen_bwd_workspace(const vafa_plan_info *info, int64_t D);

/* Replaces _PackedVarlenAttnFunction.forward (fa/interface.py:153-250):
 * q [T_q,H,D], k/v [T_k,H,D] contiguous, o [T_q,H,D] (same dtype),
 * lse [T_q,H] fp32 log2-domain.  D in {16,32,64,128,256}. */
VAFA_API int vafa_varlen_fwd(const void *q, const void *k, const void *v, void *o, float *lse,
                    const int32_t *plan_dev, const vafa_plan_info *info, int64_t D,
                    int32_t dtype, float scale, void *workspace, int64_t workspace_bytes,
                    void *stream);

/* Replaces _PackedVarlenAttnFunction.backward (fa/interface.py:252-341):
 * dO [T_q,H,D] -> dq, dk, dv (same dtype as q). Deterministic (no atomics).
 * Runs the stages below in order; on the matrix-core path the dQ stage forms
 * delta itself (bit-identical to stage 0) and leaves it for dK/dV. */
VAFA_API int vafa_varlen_bwd(const void *q, const void *k, const void *v, const void *o,
                    const void *dout, const float *lse, void *dq, void *dk, void *dv,
                    const int32_t *plan_dev, const vafa_plan_info *info, int64_t D,
                    int32_t dtype, float scale, void *workspace, int64_t workspace_bytes,
                    void *stream);

/* No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  vafa_varlen_fwd with its workspace replaced by a static
 * device array of VAFA_NOALLOC_SCRATCH_BYTES per GPU, held until the process
 * ends (it is part of the library's code object, so every GPU on which the
 * library is loaded holds it, whether or not this entry point is called):
 * same arguments otherwise, and the same kernels and results -- except for
 * D=16, which vafa_varlen_fwd runs on the D=32 matrix-core kernels
 * over zero-padded copies in its workspace and this entry point runs on the
 * wave-per-row kernels (no room for the copies): both are within the parity
 * bound of the reference, not bit-identical.  The caller still passes inputs,
 * outputs and the device plan.  Plans whose split partials need more scratch
 * than that return VAFA_ERR_WORKSPACE (use vafa_varlen_fwd with a
 * workspace).  Calls no hipMalloc/hipFree; the stream must belong to the
 * current device.  The first call on a device looks the array's address up
 * (hipGetSymbolAddress): make that call outside graph capture; later calls
 * may be captured (no memset nodes are recorded).  Every call on a GPU
 * shares that GPU's array, so calls that overlap on one GPU (other streams,
 * other threads) race: serialize them. */
#define VAFA_NOALLOC_SCRATCH_BYTES (64ll << 20)
VAFA_API int vafa_varlen_fwd_noalloc(const void *q, const void *k, const void *v, void *o,
                                     float *lse, const int32_t *plan_dev,
                                     const vafa_plan_info *info, int64_t D, int32_t dtype,
                                     float scale, void *stream);

/* One stage of vafa_varlen_bwd, for callers that schedule the backward
 * themselves (e.g. dQ and dK/dV on two streams) and for per-kernel timing:
 *   VAFA_BWD_DELTA (0): delta = rowsum(O * dO) into the workspace;
 *   VAFA_BWD_DQ    (1): dQ, including the ordered sum of split partials;
 *   VAFA_BWD_DKV   (2): dK and dV.
 * Stages 1 and 2 read the delta that stage 0 left in the same workspace and
 * are independent of each other.  Same arguments as vafa_varlen_bwd. */
#define VAFA_BWD_DELTA 0
#define VAFA_BWD_DQ 1
#define VAFA_BWD_DKV 2
VAFA_API int vafa_varlen_bwd_stage(int32_t stage, const void *q, const void *k, const void *v,
                                   const void *o, const void *dout, const float *lse, void *dq,
                                   void *dk, void *dv, const int32_t *plan_dev,
                                   const vafa_plan_info *info, int64_t D, int32_t dtype,
                                   float scale, void *workspace, int64_t workspace_bytes,
                                   void *stream);

/* Workspace bytes needed by vafa_absorb_fwd / vafa_absorb_bwd.  With
 * D_KV % 8 != 0 they include copies of u, X and W_V (and of the gradients)
 * whose D_KV is zero-padded to a multiple of 8, sized for fp32: calls whose
 * D_KV is not a whole number of 16-byte chunks run on the matrix-core
 * kernels over them. */
VAFA_API int64_t vafa_absorb_fwd_workspace(const vafa_plan_info *info, int64_t D_KV, int64_t D_H);
VAFA_API int64_t vafa_absorb_bwd_workspace(const vafa_plan_info *info, int64_t D_KV, int64_t D_H);

/* Replaces _TargetAttnFunction.forward (ta/interface.py:153-223):
 * u [T_q,H,D_KV], X [T_k,D_KV], W_V [D_KV,H,D_H] -> O [T_q,H,D_H],
 * lse [T_q,H] fp32 log2-domain. */
VAFA_API int vafa_absorb_fwd(const void *u, const void *X, const void *W_V, void *O, float *lse,
                    const int32_t *plan_dev, const vafa_plan_info *info, int64_t D_KV,
                    int64_t D_H, int32_t dtype, float scale, void *workspace,
                    int64_t workspace_bytes, void *stream);

/* Replaces _TargetAttnFunction.backward (ta/interface.py:225-321):
 * -> du [T_q,H,D_KV], dX [T_k,D_KV], dW_V [D_KV,H,D_H] (input dtype).
 * Deterministic: dX and dW_V are reduced in a fixed order (the reference
 * uses fp32 atomics for dW_V, ta/kernels.py:493). */
VAFA_API int vafa_absorb_bwd(const void *u, const void *X, const void *W_V, const void *O,
                    const void *dO, const float *lse, void *du, void *dX, void *dW_V,
                    const int32_t *plan_dev, const vafa_plan_info *info, int64_t D_KV,
                    int64_t D_H, int32_t dtype, float scale, void *workspace,
                    int64_t workspace_bytes, void *stream);

/* Workspace bytes needed by vafa_absorb_fwd_fold. */
VAFA_API int64_t vafa_absorb_fwd_fold_workspace(const vafa_plan_info *info, int64_t D_KV,
                                                int64_t D_H);

/* 1 if vafa_absorb_fwd_fold takes this shape (16-bit dtype, H dividing 64 up
 * to 8, D_KV a multiple of 8 padding onto one of the matrix-core widths up
 * to 256, D_H in {16, 32, 64, 128}), else 0. */
VAFA_API int vafa_absorb_fold_supported(int64_t H, int64_t D_KV, int64_t D_H, int32_t dtype);

/* The forward of packed_target_attn from q_proj on, with the u projection
 * folded into the attention kernel (replaces ta/interface.py:435 followed by
 * _TargetAttnFunction.forward, ta/interface.py:153-223): from
 * q_proj [T_q, H*D_H] (= q_raw W_Q, rounded to the 16-bit dtype, as
 * vafa_absorb_project_fwd writes it with u = NULL), W_K [D_KV,H,D_H],
 * X [T_k,D_KV], W_V [D_KV,H,D_H] -> O [T_q,H,D_H], lse [T_q,H] fp32
 * log2-domain.  Each workgroup forms u = q_proj_h W_K,h^T for its rows on the
 * matrix cores (fp32 accumulation, one rounding, as the reference's 16-bit
 * GEMM), so u is never written to memory.  Shapes outside
 * vafa_absorb_fold_supported return VAFA_ERR_VALUE; 16-byte aligned
 * operands. */
VAFA_API int vafa_absorb_fwd_fold(const void *q_proj, const void *W_K, const void *X,
                                  const void *W_V, void *O, float *lse, const int32_t *plan_dev,
                                  const vafa_plan_info *info, int64_t D_KV, int64_t D_H,
                                  int32_t dtype, float scale, void *workspace,
                                  int64_t workspace_bytes, void *stream);

/* The head projection of packed_target_attn, which the reference runs as a
 * torch einsum (ta/interface.py:434-435, 'thd,khd->thk'):
 * u[t,h,f] = sum_d q_proj[t, h*D_H + d] * W_K[f,h,d] with q_proj [T_q, H*D_H],
 * W_K [D_KV,H,D_H] -> u [T_q,H,D_KV], all in the given 16-bit dtype (fp32
 * accumulation, one rounding).  D_KV and D_H positive multiples of 8,
 * 16-byte aligned operands; other shapes and fp32 return VAFA_ERR_VALUE. */
VAFA_API int vafa_absorb_project_u(const void *q_proj, const void *W_K, void *u, int64_t T_q,
                                   int64_t H, int64_t D_KV, int64_t D_H, int32_t dtype,
                                   void *stream);

/* Workspace bytes of vafa_absorb_project_fwd (backward = 0) or
 * vafa_absorb_project_bwd (backward = 1); -1 for unsupported dimensions. */
VAFA_API int64_t vafa_absorb_project_workspace(int64_t T_q, int64_t H, int64_t D_Q, int64_t D_KV,
                                               int64_t D_H, int32_t backward);

/* Both projections of packed_target_attn (ta/interface.py:434-435):
 * q_proj [T_q, H*D_H] = q_raw [T_q, D_Q] . W_Q [D_Q, H*D_H] and
 * u [T_q, H, D_KV] = per head q_proj W_K[:,h,:]^T, each rounded once to the
 * 16-bit dtype (as the reference's two 16-bit GEMMs).  q_proj is written for
 * the backward.  u may be NULL: then only q_proj is formed (the input of
 * vafa_absorb_fwd_fold).  D_Q, D_KV, D_H positive multiples of 8, 16-byte
 * aligned operands and workspace. */
VAFA_API int vafa_absorb_project_fwd(const void *q_raw, const void *W_Q, const void *W_K,
                                     void *q_proj, void *u, int64_t T_q, int64_t H, int64_t D_Q,
                                     int64_t D_KV, int64_t D_H, int32_t dtype, void *workspace,
                                     int64_t workspace_bytes, void *stream);

/* Backward of the projections, which the reference leaves to torch autograd
 * (ta/interface.py:430-435): from du [T_q, H, D_KV],
 *   dq_proj = per head du W_K[:,h,:]     (rounded, kept in the workspace)
 *   dq_raw  = dq_proj W_Q^T              [T_q, D_Q]
 *   dW_Q    = q_raw^T dq_proj            [D_Q, H, D_H]
 *   dW_K    = per head du^T q_proj       [D_KV, H, D_H]
 * Any of dq_raw, dW_Q, dW_K may be NULL (not computed).  The weight
 * gradients are deterministic: fp32 partials over fixed token chunks summed
 * in chunk order. */
VAFA_API int vafa_absorb_project_bwd(const void *q_raw, const void *W_Q, const void *W_K,
                                     const void *q_proj, const void *du, void *dq_raw,
                                     void *dW_Q, void *dW_K, int64_t T_q, int64_t H, int64_t D_Q,
                                     int64_t D_KV, int64_t D_H, int32_t dtype, void *workspace,
                                     int64_t workspace_bytes, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* VAFA_H_ */
