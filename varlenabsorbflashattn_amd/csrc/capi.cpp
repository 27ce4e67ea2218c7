// extern "C" entry points: argument checks, workspace carving and kernel
// dispatch.  Compiled by hipcc (host code only; kernels live in *.hip).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <initializer_list>
#include <mutex>
#include <string>

#include "../../include/vafa.h"
#include "common.h"
#include "kernels.h"

// Device memory for the split-K partial rows of vafa_varlen_fwd_noalloc, for
// callers that cannot allocate.  Each GPU holds its own copy of the array (a
// code-object global) until the process ends.  Host code never passes
// `scratch` itself to a kernel -- in host code the name is a stand-in, not a
// device address: the device address is looked up once per device with
// hipGetSymbolAddress (scratch_ptr below) and that pointer is used instead.
static __device__ __align__(256) unsigned char scratch[VAFA_NOALLOC_SCRATCH_BYTES];

namespace vafa {
int fail(int code, const char *fmt, ...);

namespace {

constexpr int64_t kAlign = 256;
inline int64_t align_up(int64_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

// Sequential carve-out of a caller-provided workspace.
struct Carver {
  char *base;
  int64_t used = 0;
  explicit Carver(void *b) : base(static_cast<char *>(b)) {}
  template <typename P>
  P *take(int64_t bytes) {
    P *p = base ? reinterpret_cast<P *>(base + used) : nullptr;
    used += align_up(bytes);
    return p;
  }
};

int check_info(const vafa_plan_info *info, int64_t kind) {
  if (info == nullptr || info->magic != VAFA_PLAN_MAGIC || info->kind != kind)
    return fail(VAFA_ERR_VALUE, "plan does not belong to this operator");
  if (info->n_kv_res < 0 || info->n_kv_res > info->n_kv)
    return fail(VAFA_ERR_VALUE, "plan info is inconsistent (n_kv_res)");
  return VAFA_OK;
}

// A varlen plan's tiles must be ones the kernels of this head dim run: the
// planner picks 256-row query tiles only for D <= 128, 256-key tiles only
// for D = 128 (D=16 runs on the D=32 kernels), and fused key-major items
// (chunks of kFusedTiles key tiles) only for D <= kFusedMaxD -- the plain
// dK/dV kernels of a wider head dim cover one key tile per item.
int check_varlen_tiles(const vafa_plan_info *info, int64_t D) {
  const int64_t Dk = D == 16 ? 32 : D;
  const bool q_ok =
      info->q_tile == kVarlenTile || (info->q_tile == kVarlenWideTile && Dk <= 128);
  const bool k_ok =
      info->k_tile == kVarlenTile || (info->k_tile == kVarlenWideTile && Dk == 128);
  if (!q_ok || !k_ok)
    return fail(VAFA_ERR_VALUE,
                "plan tiles (%lld queries, %lld keys) do not fit head_dim %lld: build the "
                "plan with this head_dim",
                (long long)info->q_tile, (long long)info->k_tile, (long long)D);
  if (info->n_fkv > 0 && Dk > kFusedMaxD)
    return fail(VAFA_ERR_VALUE,
                "plan holds fused key-major items, which head_dim %lld does not run: build "
                "the plan with this head_dim",
                (long long)D);
  return VAFA_OK;
}

int check_launch(const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return fail(VAFA_ERR_RUNTIME, "%s: kernel launch failed: %s", what, hipGetErrorString(e));
  return VAFA_OK;
}

bool supported_d(int64_t D) {
  return D == 16 || D == 32 || D == 64 || D == 128 || D == 256;
}

// ---- varlen ---------------------------------------------------------------
struct VarlenWs {
  float *part_o = nullptr, *part_lse = nullptr, *delta = nullptr, *part_fq = nullptr;
  // D=16 on the matrix cores: zero-padded D=32 copies of the operands
  void *pq = nullptr, *pk = nullptr, *pv = nullptr, *po = nullptr, *pdo = nullptr,
       *pdq = nullptr, *pdk = nullptr, *pdv = nullptr;
  int64_t bytes = 0;
};

// D=16 runs on the D=32 matrix-core kernels over zero-padded copies (the
// zero columns add exact zeros to every product; the caller's scale is kept).
inline bool pad_d16(int64_t D, int32_t dtype) {
  return D == 16 && (dtype == VAFA_BF16 || dtype == VAFA_F16 || dtype == VAFA_F32);
}
inline int elem_bytes(int32_t dtype) { return dtype == VAFA_F32 ? 4 : 2; }

VarlenWs carve_varlen(void *ws, const vafa_plan_info *info, int64_t D, bool bwd, bool pad) {
  Carver c(ws);
  VarlenWs w;
  const int64_t Dc = pad ? 32 : D;
  const int64_t rows = info->n_part_rows * info->H;
  if (bwd) w.delta = c.take<float>(info->T_q * info->H * 4);
  w.part_o = c.take<float>(rows * Dc * 4);
  if (!bwd) w.part_lse = c.take<float>(rows * 4);
  if (bwd) w.part_fq = c.take<float>(info->n_fpart_rows * info->H * Dc * 4);
  if (pad) {
    // sized for fp32 rows: the workspace functions do not see the dtype
    const int64_t nq = info->T_q * info->H * 32 * 4, nk = info->T_k * info->H * 32 * 4;
    w.pq = c.take<void>(nq);
    w.pk = c.take<void>(nk);
    w.pv = c.take<void>(nk);
    w.po = c.take<void>(nq);
    if (bwd) {
      w.pdo = c.take<void>(nq);
      w.pdq = c.take<void>(nq);
      w.pdk = c.take<void>(nk);
      w.pdv = c.take<void>(nk);
    }
  }
  w.bytes = c.used;
  return w;
}

template <typename T>
void varlen_fwd_dispatch(const VarlenArgs &a, hipStream_t st) {
  if constexpr (sizeof(T) == 2) {
    switch (a.D) {
      case 32: launch_mfma_varlen_fwd<T, 32>(a, st); return;
      case 64: launch_mfma_varlen_fwd<T, 64>(a, st); return;
      case 128: launch_mfma_varlen_fwd<T, 128>(a, st); return;
      case 256: launch_mfma_varlen_fwd<T, 256>(a, st); return;
      default: break;
    }
  } else {
    if (f32_varlen_mfma_d(a.D)) return launch_f32_varlen_fwd(a, st);
  }
  launch_simt_varlen_fwd<T>(a, st);
}

template <typename T>
void varlen_fwd_all(const VarlenArgs &a, hipStream_t st) {
  varlen_fwd_dispatch<T>(a, st);
  launch_lse_combine<T>(a.part_o, a.part_lse, a.o, a.lse, a.comb_items, a.n_comb, a.H, a.D,
                        a.comb_rows, st);
}

// Backward stages.  Matrix-core kernels for D in {32, 64, 128, 256} (16-bit
// and fp32); D=16 (below the 32-wide output tiles) reaches them padded to 32
// from vafa_varlen_bwd, and the stage entry points' D=16 takes the
// wave-per-row kernels.  Segments the plan fuses (few queries, D <= 64) run
// dQ/dK/dV in the fused key-major kernel, whose dQ partials are summed in
// order; without it (fp32) their key tiles go to the plain dK/dV kernel and
// their dQ to the dQ pass over every forward item.
inline bool mfma_bwd_d(int D) { return D == 32 || D == 64 || D == 128 || D == 256; }

template <typename T>
bool fused_path(const VarlenArgs &a) {
  return sizeof(T) == 2 && a.n_fkv > 0 && (a.D == 32 || a.D == 64);
}

template <typename T>
void varlen_bwd_stage(int stage, const VarlenArgs &a, hipStream_t st) {
  const bool mfma = sizeof(T) == 2 && mfma_bwd_d(a.D);
  const bool fq = fused_path<T>(a);
  if (stage == VAFA_BWD_DELTA) {
    launch_row_dot<T>(a.o_in, a.dout, a.delta, a.T_q * a.H, a.D, st);
  } else if (stage == VAFA_BWD_DQ) {
    VarlenArgs d = a;
    if (fq) {  // the fused kernel owns the fused segments' dQ
      d.items = a.dq_items;
      d.n_items = a.n_dq;
      d.comb_items = a.dqc_items;
      d.n_comb = a.n_dqc;
      d.comb_rows = a.dqc_rows;
    }
    if constexpr (sizeof(T) == 2) {
      if (mfma) {
        if (a.D == 32) launch_mfma_varlen_dq<T, 32>(d, st);
        if (a.D == 64) launch_mfma_varlen_dq<T, 64>(d, st);
        if (a.D == 128) launch_mfma_varlen_dq<T, 128>(d, st);
        if (a.D == 256) launch_mfma_varlen_dq<T, 256>(d, st);
      }
    }
    if (!mfma) {
      if (sizeof(T) == 4 && f32_varlen_bwd_mfma_d(a.D))
        launch_f32_varlen_dq(d, st);
      else
        launch_simt_varlen_dq<T>(d, st);
    }
    launch_sum_combine<T>(d.part_o, d.dq, d.comb_items, d.n_comb, d.H, d.D, d.comb_rows, st);
  } else {
    if constexpr (sizeof(T) == 2) {
      if (mfma) {
        if (a.D == 32) launch_mfma_varlen_dkv<T, 32>(a, st);
        if (a.D == 64) launch_mfma_varlen_dkv<T, 64>(a, st);
        if (a.D == 128) launch_mfma_varlen_dkv<T, 128>(a, st);
        if (a.D == 256) launch_mfma_varlen_dkv<T, 256>(a, st);
      }
      if (fq) {
        if (a.D == 32) launch_mfma_varlen_fkv<T, 32>(a, st);
        if (a.D == 64) launch_mfma_varlen_fkv<T, 64>(a, st);
        launch_sum_combine<T>(a.part_fq, a.dq, a.fcomb_items, a.n_fcomb, a.H, a.D, a.fcomb_rows,
                              st);
      }
    }
    // fp32: the fp32 matrix-core kernels (D=16 only from the stage API, on
    // the wave-per-key kernel)
    const bool f32m = sizeof(T) == 4 && f32_varlen_bwd_mfma_d(a.D);
    if (!mfma) {
      if (f32m)
        launch_f32_varlen_dkv(a, st);
      else
        launch_simt_varlen_dkv<T>(a, st);
    }
    if (!fq && a.n_fkv > 0) {
      // fused-planned chunks without the fused kernel (fp32): both dK/dV
      // kernels walk any key range ({k0, k1, q0, q1} leads both item
      // formats).  16-bit operands always take the fused kernel here: a plan
      // holds fused items only for D <= kFusedMaxD (check_varlen_tiles).
      VarlenArgs kv = a;
      kv.kv_items = a.fkv_items;
      kv.n_kv = a.n_fkv;
      if (f32m)
        launch_f32_varlen_dkv(kv, st);
      else
        launch_simt_varlen_dkv<T>(kv, st);
    }
  }
}

// All stages in order.  The matrix-core dQ kernel forms delta itself (the
// same bits as the delta stage) and leaves it for dK/dV -- unless fused
// segments exist, whose rows it does not see: then the delta stage runs.
template <typename T>
void varlen_bwd_all(const VarlenArgs &a, hipStream_t st) {
  const bool mfma = sizeof(T) == 2 && mfma_bwd_d(a.D);
  VarlenArgs f = a;
  f.fuse_delta = mfma && !fused_path<T>(a);
  if (!f.fuse_delta) varlen_bwd_stage<T>(VAFA_BWD_DELTA, f, st);
  varlen_bwd_stage<T>(VAFA_BWD_DQ, f, st);
  varlen_bwd_stage<T>(VAFA_BWD_DKV, f, st);
}

// ---- absorb ---------------------------------------------------------------
struct AbsorbWs {
  float *part_o = nullptr, *part_lse = nullptr, *delta = nullptr, *dax = nullptr, *ax = nullptr,
        *dwv_part = nullptr;
  void *wvt = nullptr, *wkt = nullptr, *axf = nullptr;
  // D_KV padded to a multiple of 8: copies of u, X, W_V and (backward) the
  // padded du, dX, dW_V
  void *pu = nullptr, *pX = nullptr, *pW = nullptr, *pdu = nullptr, *pdX = nullptr,
       *pdW = nullptr;
  int64_t n_tchunks = 0, tchunk = 0;
  int64_t bytes = 0;
};

constexpr int64_t kDwvChunks = 64;

// D_KV that is not a whole number of 16-byte chunks (8 16-bit or 4 fp32
// elements) runs on the matrix-core kernels over copies of u, X and W_V
// whose D_KV is zero-padded to a multiple of 8, when they take the padded
// shape: the zero features add exact zeros to every product and leave zero
// columns in du, dX and dW_V, which are not copied back.
inline int64_t absorb_fpad(int64_t F) { return (F + 7) / 8 * 8; }

bool absorb_pad(int64_t H, int64_t F, int64_t DH, int32_t dtype, bool bwd) {
  if (F % (dtype == VAFA_F32 ? 4 : 8) == 0) return false;
  const int h = (int)H, fp = (int)absorb_fpad(F), dh = (int)DH;
  switch (dtype) {
    case VAFA_F32: return bwd ? f32_absorb_supported(h, fp, dh) : f32_absorb_fwd_supported(h, fp, dh);
    case VAFA_BF16: return mfma_absorb_fwd_supported<bf16>(h, fp, dh);
    case VAFA_F16: return mfma_absorb_fwd_supported<f16>(h, fp, dh);
    default: return false;
  }
}

// The workspace functions do not see the dtype: with D_KV % 8 != 0 they
// include the padded copies (sized for fp32) and size the internal buffers
// for the padded width.
AbsorbWs carve_absorb(void *ws, const vafa_plan_info *info, int64_t F0, int64_t DH, bool bwd,
                      bool fold = false) {
  Carver c(ws);
  AbsorbWs w;
  const int64_t H = info->H, Tq = info->T_q;
  const int64_t F = absorb_fpad(F0);  // >= F0; == F0 when F0 % 8 == 0
  if (F0 % 8 != 0) {
    w.pu = c.take<void>(Tq * H * F * 4);
    w.pX = c.take<void>(info->T_k * F * 4);
    w.pW = c.take<void>(F * H * DH * 4);
    if (bwd) {
      w.pdu = c.take<void>(Tq * H * F * 4);
      w.pdX = c.take<void>(info->T_k * F * 4);
      w.pdW = c.take<void>(F * H * DH * 4);
    }
  }
  if (!bwd) {
    // the unprojected 16-bit forward keeps split partials and aX/l rows at
    // the padded D_KV width
    const bool unproj = !fold && mfma_absorb_unprojected((int)H, (int)F, (int)DH, false);
    const int64_t fpw = mfma_absorb_wvt_elems(1, (int)F, 1);  // padded D_KV
    w.part_o = c.take<float>(info->n_part_rows * H * (unproj ? std::max(DH, fpw) : DH) * 4);
    w.part_lse = c.take<float>(info->n_part_rows * H * 4);
    if (unproj) w.axf = c.take<char>(Tq * H * fpw * 2);
    // W_V re-laid out for the projection: 16-bit (mfma_absorb_wvt_elems x 2
    // bytes) or fp32 (f32_absorb_wvt_elems x 4 bytes); sized for either
    const int64_t wvt16 = mfma_absorb_wvt_elems((int)H, (int)F, (int)DH) * 2;
    const int64_t wvt32 = f32_absorb_wvt_elems((int)H, (int)F, (int)DH) * 4;
    w.wvt = c.take<char>(wvt16 > wvt32 ? wvt16 : wvt32);
    // folded projection: W_K re-laid out per head (16-bit only)
    if (fold) w.wkt = c.take<char>(mfma_absorb_wkt_elems((int)H, (int)F, (int)DH) * 2);
  } else {
    w.delta = c.take<float>(Tq * H * 4);
    w.dax = c.take<float>(Tq * H * F * 4);
    w.ax = c.take<float>(Tq * H * F * 4);
    w.tchunk = Tq > 0 ? (Tq + kDwvChunks - 1) / kDwvChunks : 0;
    w.n_tchunks = Tq > 0 ? (Tq + w.tchunk - 1) / w.tchunk : 0;
    w.dwv_part = c.take<float>((w.n_tchunks > 0 ? w.n_tchunks : 1) * F * H * DH * 4);
  }
  w.bytes = c.used;
  return w;
}

template <typename T>
void absorb_fwd_all(const AbsorbArgs &a, hipStream_t st) {
  if constexpr (sizeof(T) == 2) {
    if (mfma_absorb_fwd_supported<T>(a.H, a.F, a.DH)) {
      launch_mfma_absorb_fwd<T>(a, st);
      if (mfma_absorb_unprojected(a.H, a.F, a.DH, a.fold)) {
        // combine the split partials into the aX/l rows, then O = aX W_V
        const int FP = (int)mfma_absorb_wvt_elems(1, a.F, 1);
        launch_lse_combine<T>(a.part_o, a.part_lse, a.axf, a.lse, a.comb_items, a.n_comb, a.H,
                              FP, a.comb_rows, st);
        RowGemm p{a.axf, a.wvt, a.O, a.T_q, a.H, a.DH, FP,
                  (int64_t)a.H * FP, FP, (int64_t)a.DH * FP, FP, (int64_t)a.H * a.DH, a.DH};
        launch_rowgemm<T>(p, st);
        return;
      }
    } else {
      launch_simt_absorb_fwd<T>(a, st);
    }
  } else {
    if (f32_absorb_fwd_supported(a.H, a.F, a.DH))
      launch_f32_absorb_fwd(a, st);
    else
      launch_simt_absorb_fwd<T>(a, st);
  }
  launch_lse_combine<T>(a.part_o, a.part_lse, a.O, a.lse, a.comb_items, a.n_comb, a.H, a.DH,
                        a.comb_rows, st);
}

template <typename T>
void absorb_bwd_all(const AbsorbArgs &a, hipStream_t st) {
  bool mfma = false;
  if constexpr (sizeof(T) == 2) mfma = mfma_absorb_fwd_supported<T>(a.H, a.F, a.DH);
  // the matrix-core dAX kernel also writes delta (sum_d dO O) for its rows
  bool dax_done = false;
  if constexpr (sizeof(T) == 2) dax_done = launch_mfma_absorb_dax<T>(a, st);
  if (!dax_done) {
    launch_row_dot<T>(a.O_in, a.dO, a.delta, a.T_q * a.H, a.DH, st);
    if (sizeof(T) == 4 && f32_absorb_supported(a.H, a.F, a.DH))
      launch_f32_absorb_dax(a, st);
    else
      launch_absorb_dax<T>(a, st);
  }
  if (mfma) {
    if constexpr (sizeof(T) == 2) {
      launch_mfma_absorb_du<T>(a, st);
      launch_mfma_absorb_dx<T>(a, st);
    }
  } else if (sizeof(T) == 4 && f32_absorb_supported(a.H, a.F, a.DH)) {
    launch_f32_absorb_du_dx(a, st);
  } else {
    launch_simt_absorb_du<T>(a, st);
    launch_simt_absorb_dx<T>(a, st);
  }
  launch_absorb_dwv<T>(a, st);
}

template <template <typename> class F, typename A>
int by_dtype(int32_t dtype, const A &a, hipStream_t st) {
  switch (dtype) {
    case VAFA_F32: F<float>::run(a, st); return VAFA_OK;
    case VAFA_F16: F<f16>::run(a, st); return VAFA_OK;
    case VAFA_BF16: F<bf16>::run(a, st); return VAFA_OK;
    default: return fail(VAFA_ERR_ASSERT, "unsupported dtype code %d", (int)dtype);
  }
}
template <typename T> struct VFwd { static void run(const VarlenArgs &a, hipStream_t s) { varlen_fwd_all<T>(a, s); } };
template <typename T> struct VBwd { static void run(const VarlenArgs &a, hipStream_t s) { varlen_bwd_all<T>(a, s); } };
template <typename T> struct VBwdStage {
  static void run(const VarlenArgs &a, hipStream_t s) { varlen_bwd_stage<T>(a.stage, a, s); }
};
template <typename T> struct AFwd { static void run(const AbsorbArgs &a, hipStream_t s) { absorb_fwd_all<T>(a, s); } };
template <typename T> struct ABwd { static void run(const AbsorbArgs &a, hipStream_t s) { absorb_bwd_all<T>(a, s); } };

// ---- scratch of vafa_varlen_fwd_noalloc (the array is at file scope above) --
constexpr int64_t kScratchBytes = VAFA_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;
void *g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mu;

// Device address of this GPU's scratch: looked up on the first call made
// while that device is current, then reused.
int scratch_ptr(void **out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess)
    return fail(VAFA_ERR_RUNTIME, "hipGetDevice failed: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(VAFA_ERR_RUNTIME, "device ordinal %d beyond the %d the library tracks", dev,
                kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(::scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(VAFA_ERR_RUNTIME, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                  hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return VAFA_OK;
}


// Projection shapes: every dimension a positive multiple of 8 (16-byte rows
// for the row GEMM's loads), H * D_H and the token count within int range.
int check_project_dims(const char *what, int64_t T_q, int64_t H, int64_t D_Q, int64_t D_KV,
                       int64_t D_H) {
  const bool ok = T_q >= 0 && T_q < (1ll << 31) && H >= 1 && H <= 1024 && D_Q >= 8 &&
                  D_Q <= 65536 && D_Q % 8 == 0 && D_KV >= 8 && D_KV <= 65536 && D_KV % 8 == 0 &&
                  D_H >= 8 && D_H % 8 == 0 && H * D_H <= 65536;
  if (!ok)
    return fail(VAFA_ERR_VALUE, "%s: T_q=%lld H=%lld D_Q=%lld D_KV=%lld D_H=%lld not supported "
                "(D_Q, D_KV, D_H positive multiples of 8, H*D_H <= 65536)", what, (long long)T_q,
                (long long)H, (long long)D_Q, (long long)D_KV, (long long)D_H);
  return VAFA_OK;
}

int check_aligned(const char *what, std::initializer_list<const void *> ptrs) {
  for (const void *p : ptrs)
    if (reinterpret_cast<uintptr_t>(p) % 16 != 0)
      return fail(VAFA_ERR_VALUE, "%s: operands must be 16-byte aligned", what);
  return VAFA_OK;
}

template <typename T>
void project_u(const void *q_proj, const void *W_K, void *u, int64_t T_q, int H, int F, int DH,
               hipStream_t st) {
  // u[t, h, f] = sum_d q_proj[t, h, d] W_K[f, h, d]
  const int64_t HD = (int64_t)H * DH;
  launch_rowgemm<T>(RowGemm{q_proj, W_K, u, T_q, H, F, DH, HD, DH, DH, HD, (int64_t)H * F, F}, st);
}

// Token chunks of a projection weight gradient: on the 16-bit kernel a
// multiple of 32 tokens, about kWgradWgs workgroups in all (wgs_per_chunk per
// chunk); on the fp32-product fallback (F > 512) 64 chunks.
constexpr int64_t kWgradWgs = 512;
struct Chunks {
  int64_t tchunk = 0, n = 0;
};
Chunks wgrad_chunks(int64_t T_q, int64_t F, int64_t wgs_per_chunk) {
  Chunks c;
  if (T_q <= 0) return c;
  if (!wgrad16_supported((int)F)) {
    c.tchunk = (T_q + 63) / 64;
  } else {
    const int64_t tiles = (T_q + 31) / 32;
    int64_t want = kWgradWgs / wgs_per_chunk;
    want = want < 1 ? 1 : (want > tiles ? tiles : want);
    c.tchunk = (tiles + want - 1) / want * 32;
  }
  c.n = (T_q + c.tchunk - 1) / c.tchunk;
  return c;
}

struct ProjectWs {
  void *wt = nullptr;      // W_Q^T [HD, D_Q] (forward) or W_K^T [HD, D_KV] (backward)
  void *dq_proj = nullptr; // [T_q, HD]
  float *part = nullptr;   // weight-gradient chunk partials
  Chunks ck, cq;           // chunks of dW_K and dW_Q
  int64_t bytes = 0;
};

ProjectWs carve_project(void *ws, int64_t T_q, int64_t H, int64_t D_Q, int64_t D_KV, int64_t D_H,
                        bool bwd) {
  Carver c(ws);
  ProjectWs w;
  const int64_t HD = H * D_H;
  w.wt = c.take<void>(HD * (bwd ? D_KV : D_Q) * 2);
  if (bwd) {
    w.dq_proj = c.take<void>(T_q * HD * 2);
    w.ck = wgrad_chunks(T_q, D_KV, H * ((D_H + 31) / 32));
    w.cq = wgrad_chunks(T_q, D_Q, (HD + 31) / 32);
    const int64_t pk = w.ck.n * D_KV * HD, pq = w.cq.n * D_Q * HD;
    w.part = c.take<float>((pk > pq ? pk : pq) * 4 + 4);
  }
  w.bytes = c.used;
  return w;
}

template <typename T>
void project_fwd(const void *q_raw, const void *W_Q, const void *W_K, void *q_proj, void *u,
                 int64_t T_q, int H, int DQ, int F, int DH, const ProjectWs &w, hipStream_t st) {
  const int HD = H * DH;
  // q_proj [T, HD] = q_raw [T, DQ] . W_Q [DQ, HD], through W_Q^T [HD, DQ]
  launch_transpose2d<T>(W_Q, w.wt, DQ, HD, st);
  launch_rowgemm<T>(RowGemm{q_raw, w.wt, q_proj, T_q, 1, HD, DQ, DQ, 0, 0, DQ, HD, 0}, st);
  if (u != nullptr) project_u<T>(q_proj, W_K, u, T_q, H, F, DH, st);
}

template <typename T>
void project_bwd(const void *q_raw, const void *W_Q, const void *W_K, const void *q_proj,
                 const void *du, void *dq_raw, void *dW_Q, void *dW_K, int64_t T_q, int H, int DQ,
                 int F, int DH, const ProjectWs &w, hipStream_t st) {
  const int HD = H * DH;
  const bool need_dq = dq_raw != nullptr || dW_Q != nullptr;
  // W_K^T [HD, F]: the dq_proj product's weight rows
  if (need_dq) launch_transpose2d<T>(W_K, w.wt, F, HD, st);
  // dW_K[f, h, d] = sum_t du[t, h, f] q_proj[t, h, d], and on the 16-bit
  // kernel dq_proj[t, h, d] = sum_f du[t, h, f] W_K[f, h, d] from the same du reads
  const bool fused = wgrad16_supported(F) && dW_K != nullptr;
  if (fused) {
    launch_wgrad16<T>(Wgrad{du, q_proj, w.wt, need_dq ? w.dq_proj : nullptr, dW_K, w.part, T_q,
                            w.ck.tchunk, w.ck.n, H, F, DH}, st);
  } else if (dW_K != nullptr) {
    launch_wgrad<T, T>(du, q_proj, w.part, dW_K, T_q, w.ck.tchunk, w.ck.n, H, F, DH, st);
  }
  if (!need_dq) return;
  if (!fused)
    launch_rowgemm<T>(RowGemm{du, w.wt, w.dq_proj, T_q, H, DH, F, (int64_t)H * F, F,
                              (int64_t)DH * F, F, HD, DH}, st);
  if (dq_raw != nullptr)  // dq_raw [T, DQ] = dq_proj [T, HD] . W_Q [DQ, HD]^T
    launch_rowgemm<T>(RowGemm{w.dq_proj, W_Q, dq_raw, T_q, 1, DQ, HD, HD, 0, 0, HD, DQ, 0}, st);
  if (dW_Q != nullptr) {  // dW_Q[c, hd] = sum_t q_raw[t, c] dq_proj[t, hd]
    if (wgrad16_supported(DQ))
      launch_wgrad16<T>(Wgrad{q_raw, w.dq_proj, nullptr, nullptr, dW_Q, w.part, T_q, w.cq.tchunk,
                              w.cq.n, 1, DQ, HD}, st);
    else
      launch_wgrad<T, T>(q_raw, w.dq_proj, w.part, dW_Q, T_q, w.cq.tchunk, w.cq.n, 1, DQ, HD, st);
  }
}

}  // namespace
}  // namespace vafa

using namespace vafa;

extern "C" {

const char *vafa_version(void) { return "vafa 0.1.0 gfx950"; }

// The workspace functions do not see the dtype: for D=16 they include the
// padded copies, sized for fp32 rows.
int64_t vafa_varlen_fwd_workspace(const vafa_plan_info *info, int64_t D) {
  if (check_info(info, 1)) return -1;
  return carve_varlen(nullptr, info, D, false, D == 16).bytes;
}

int64_t vafa_varlen_bwd_workspace(const vafa_plan_info *info, int64_t D) {
  if (check_info(info, 1)) return -1;
  return carve_varlen(nullptr, info, D, true, D == 16).bytes;
}

static int varlen_fwd_impl(const void *q, const void *k, const void *v, void *o, float *lse,
                           const int32_t *plan_dev, const vafa_plan_info *info, int64_t D,
                           int32_t dtype, float scale, void *workspace, int64_t workspace_bytes,
                           void *stream, bool allow_pad) {
  if (int rc = check_info(info, 1)) return rc;
  if (!supported_d(D))
    return fail(VAFA_ERR_ASSERT, "head_dim %lld not supported (try 64/128/256)", (long long)D);
  if (int rc = check_varlen_tiles(info, D)) return rc;
  const bool pad = allow_pad && pad_d16(D, dtype);
  VarlenWs w = carve_varlen(workspace, info, D, false, pad);
  if (workspace_bytes < w.bytes || (w.bytes > 0 && workspace == nullptr))
    return fail(VAFA_ERR_WORKSPACE, "workspace of %lld bytes, %lld needed",
                (long long)workspace_bytes, (long long)w.bytes);
  const hipStream_t st = (hipStream_t)stream;
  VarlenArgs a{};
  a.q = q; a.k = k; a.v = v; a.o = o; a.lse = lse;
  a.part_o = w.part_o; a.part_lse = w.part_lse;
  a.items = plan_dev + info->off_fwd; a.n_items = info->n_fwd;
  a.comb_items = plan_dev + info->off_comb; a.n_comb = info->n_comb;
  a.comb_rows = (int)info->max_comb_rows;
  a.kv_items = plan_dev + info->off_kv; a.n_kv = info->n_kv;
  a.T_q = info->T_q; a.H = (int)info->H; a.D = (int)D; a.scale = scale;
  a.q_tile = (int)info->q_tile; a.k_tile = (int)info->k_tile;
  a.xcd_heads = (int)info->xcd_heads;
  const int eb = elem_bytes(dtype);
  if (pad) {
    launch_pad16(q, w.pq, info->T_q * info->H, eb, st);
    launch_pad16(k, w.pk, info->T_k * info->H, eb, st);
    launch_pad16(v, w.pv, info->T_k * info->H, eb, st);
    a.q = w.pq; a.k = w.pk; a.v = w.pv; a.o = w.po; a.D = 32;
  }
  if (int rc = by_dtype<VFwd>(dtype, a, st)) return rc;
  if (pad) launch_unpad16(w.po, o, info->T_q * info->H, eb, st);
  return check_launch("vafa_varlen_fwd");
}

int vafa_varlen_fwd(const void *q, const void *k, const void *v, void *o, float *lse,
                    const int32_t *plan_dev, const vafa_plan_info *info, int64_t D,
                    int32_t dtype, float scale, void *workspace, int64_t workspace_bytes,
                    void *stream) {
  return varlen_fwd_impl(q, k, v, o, lse, plan_dev, info, D, dtype, scale, workspace,
                         workspace_bytes, stream, true);
}

int vafa_varlen_fwd_noalloc(const void *q, const void *k, const void *v, void *o, float *lse,
                            const int32_t *plan_dev, const vafa_plan_info *info, int64_t D,
                            int32_t dtype, float scale, void *stream) {
  if (int rc = check_info(info, 1)) return rc;
  if (!supported_d(D))
    return fail(VAFA_ERR_ASSERT, "head_dim %lld not supported (try 64/128/256)", (long long)D);
  // D=16 stays on the wave-per-row kernels here: the static scratch holds
  // the split partials only, not padded operand copies
  const int64_t need = carve_varlen(nullptr, info, D, false, false).bytes;
  if (need > kScratchBytes)
    return fail(VAFA_ERR_WORKSPACE,
                "vafa_varlen_fwd_noalloc: this plan's split partials need %lld bytes, the "
                "static scratch holds %lld; call vafa_varlen_fwd with a workspace instead",
                (long long)need, (long long)kScratchBytes);
  void *ws = nullptr;
  if (need > 0) {
    if (int rc = scratch_ptr(&ws)) return rc;
  }
  return varlen_fwd_impl(q, k, v, o, lse, plan_dev, info, D, dtype, scale, ws,
                         need > 0 ? kScratchBytes : 0, stream, false);
}

static int varlen_bwd_entry(int32_t stage, const void *q, const void *k, const void *v,
                            const void *o, const void *dout, const float *lse, void *dq, void *dk,
                            void *dv, const int32_t *plan_dev, const vafa_plan_info *info,
                            int64_t D, int32_t dtype, float scale, void *workspace,
                            int64_t workspace_bytes, void *stream) {
  if (int rc = check_info(info, 1)) return rc;
  if (!supported_d(D))
    return fail(VAFA_ERR_ASSERT, "head_dim %lld not supported (try 64/128/256)", (long long)D);
  if (stage < -1 || stage > VAFA_BWD_DKV)
    return fail(VAFA_ERR_VALUE, "unknown backward stage %d", (int)stage);
  if (int rc = check_varlen_tiles(info, D)) return rc;
  // the stage entry points (a test and profiling API) keep D=16 on the
  // wave-per-row kernels
  const bool pad = stage < 0 && pad_d16(D, dtype);
  VarlenWs w = carve_varlen(workspace, info, D, true, pad);
  if (workspace_bytes < w.bytes || (w.bytes > 0 && workspace == nullptr))
    return fail(VAFA_ERR_WORKSPACE, "workspace of %lld bytes, %lld needed",
                (long long)workspace_bytes, (long long)w.bytes);
  const hipStream_t st = (hipStream_t)stream;
  VarlenArgs a{};
  a.q = q; a.k = k; a.v = v; a.o_in = o; a.dout = dout; a.lse_in = lse;
  a.dq = dq; a.dk = dk; a.dv = dv;
  a.delta = w.delta; a.part_o = w.part_o; a.part_fq = w.part_fq;
  a.dq_items = plan_dev + info->off_dq; a.n_dq = info->n_dq;
  a.dqc_items = plan_dev + info->off_dqc; a.n_dqc = info->n_dqc;
  a.dqc_rows = (int)info->max_dqc_rows;
  a.fkv_items = plan_dev + info->off_fkv; a.n_fkv = info->n_fkv;
  a.fcomb_items = plan_dev + info->off_fcomb; a.n_fcomb = info->n_fcomb;
  a.fcomb_rows = (int)info->max_fcomb_rows;
  a.items = plan_dev + info->off_fwd; a.n_items = info->n_fwd;
  a.comb_items = plan_dev + info->off_comb; a.n_comb = info->n_comb;
  a.comb_rows = (int)info->max_comb_rows;
  a.kv_items = plan_dev + info->off_kv; a.n_kv = info->n_kv;
  a.T_q = info->T_q; a.H = (int)info->H; a.D = (int)D; a.scale = scale;
  a.q_tile = (int)info->q_tile; a.k_tile = (int)info->k_tile;
  a.xcd_heads = (int)info->xcd_heads;
  a.stage = stage;
  const int eb = elem_bytes(dtype);
  if (pad) {
    const int64_t rq = info->T_q * info->H, rk = info->T_k * info->H;
    launch_pad16(q, w.pq, rq, eb, st);
    launch_pad16(k, w.pk, rk, eb, st);
    launch_pad16(v, w.pv, rk, eb, st);
    launch_pad16(o, w.po, rq, eb, st);
    launch_pad16(dout, w.pdo, rq, eb, st);
    a.q = w.pq; a.k = w.pk; a.v = w.pv; a.o_in = w.po; a.dout = w.pdo;
    a.dq = w.pdq; a.dk = w.pdk; a.dv = w.pdv; a.D = 32;
  }
  const int rc = stage < 0 ? by_dtype<VBwd>(dtype, a, st) : by_dtype<VBwdStage>(dtype, a, st);
  if (rc) return rc;
  if (pad) {
    launch_unpad16(w.pdq, dq, info->T_q * info->H, eb, st);
    launch_unpad16(w.pdk, dk, info->T_k * info->H, eb, st);
    launch_unpad16(w.pdv, dv, info->T_k * info->H, eb, st);
  }
  return check_launch("vafa_varlen_bwd");
}

int vafa_varlen_bwd(const void *q, const void *k, const void *v, const void *o,
                    const void *dout, const float *lse, void *dq, void *dk, void *dv,
                    const int32_t *plan_dev, const vafa_plan_info *info, int64_t D,
                    int32_t dtype, float scale, void *workspace, int64_t workspace_bytes,
                    void *stream) {
  return varlen_bwd_entry(-1, q, k, v, o, dout, lse, dq, dk, dv, plan_dev, info, D, dtype,
                          scale, workspace, workspace_bytes, stream);
}

int vafa_varlen_bwd_stage(int32_t stage, const void *q, const void *k, const void *v,
                          const void *o, const void *dout, const float *lse, void *dq, void *dk,
                          void *dv, const int32_t *plan_dev, const vafa_plan_info *info,
                          int64_t D, int32_t dtype, float scale, void *workspace,
                          int64_t workspace_bytes, void *stream) {
  if (stage < 0) return fail(VAFA_ERR_VALUE, "unknown backward stage %d", (int)stage);
  return varlen_bwd_entry(stage, q, k, v, o, dout, lse, dq, dk, dv, plan_dev, info, D, dtype,
                          scale, workspace, workspace_bytes, stream);
}

int64_t vafa_absorb_fwd_workspace(const vafa_plan_info *info, int64_t D_KV, int64_t D_H) {
  if (check_info(info, 2)) return -1;
  return carve_absorb(nullptr, info, D_KV, D_H, false).bytes;
}

int64_t vafa_absorb_bwd_workspace(const vafa_plan_info *info, int64_t D_KV, int64_t D_H) {
  if (check_info(info, 2)) return -1;
  return carve_absorb(nullptr, info, D_KV, D_H, true).bytes;
}

static int check_absorb_dims(int64_t F, int64_t DH) {
  if (!(DH == 16 || DH == 32 || DH == 64 || DH == 128 || DH == 256))
    return fail(VAFA_ERR_ASSERT, "D_H %lld not supported", (long long)DH);
  if (F < 1 || F > 512)
    return fail(VAFA_ERR_ASSERT, "D_KV=%lld pads beyond 512, which is too large", (long long)F);
  return VAFA_OK;
}

int vafa_absorb_fwd(const void *u, const void *X, const void *W_V, void *O, float *lse,
                    const int32_t *plan_dev, const vafa_plan_info *info, int64_t D_KV,
                    int64_t D_H, int32_t dtype, float scale, void *workspace,
                    int64_t workspace_bytes, void *stream) {
  if (int rc = check_info(info, 2)) return rc;
  if (int rc = check_absorb_dims(D_KV, D_H)) return rc;
  AbsorbWs w = carve_absorb(workspace, info, D_KV, D_H, false);
  if (workspace_bytes < w.bytes || (w.bytes > 0 && workspace == nullptr))
    return fail(VAFA_ERR_WORKSPACE, "workspace of %lld bytes, %lld needed",
                (long long)workspace_bytes, (long long)w.bytes);
  const hipStream_t st = (hipStream_t)stream;
  AbsorbArgs a{};
  a.u = u; a.X = X; a.wv = W_V; a.O = O; a.lse = lse;
  a.part_o = w.part_o; a.part_lse = w.part_lse; a.wvt = w.wvt; a.axf = w.axf;
  int64_t F = D_KV;
  if (absorb_pad(info->H, D_KV, D_H, dtype, false)) {
    F = absorb_fpad(D_KV);
    const int eb = elem_bytes(dtype);
    launch_pad_cols(u, w.pu, info->T_q * info->H, D_KV, F, eb, st);
    launch_pad_cols(X, w.pX, info->T_k, D_KV, F, eb, st);
    launch_pad_cols(W_V, w.pW, 1, D_KV * info->H * D_H, F * info->H * D_H, eb, st);
    a.u = w.pu; a.X = w.pX; a.wv = w.pW;
  }
  a.items = plan_dev + info->off_fwd; a.n_items = info->n_fwd;
  a.comb_items = plan_dev + info->off_comb; a.n_comb = info->n_comb;
  a.comb_rows = (int)info->max_comb_rows;
  a.kv_items = plan_dev + info->off_kv; a.n_kv = info->n_kv; a.n_kv_res = info->n_kv_res;
  a.qseg_items = plan_dev + info->off_qt; a.n_qseg = info->n_qt;
  a.T_q = info->T_q; a.T_k = info->T_k;
  a.H = (int)info->H; a.F = (int)F; a.DH = (int)D_H; a.scale = scale;
  if (int rc = by_dtype<AFwd>(dtype, a, st)) return rc;
  return check_launch("vafa_absorb_fwd");
}

// The folded forward runs on the 16-bit matrix-core kernel only (the
// projection it folds is the 16-bit one of vafa_absorb_project_fwd).
static bool fold_supported(int64_t H, int64_t F, int64_t DH, int32_t dtype) {
  if (dtype != VAFA_BF16 && dtype != VAFA_F16) return false;
  if (H < 1 || H > 64 || F < 1 || F > 512 || DH < 1 || DH > 256) return false;
  return mfma_absorb_fold_supported((int)H, (int)F, (int)DH);
}

int vafa_absorb_fold_supported(int64_t H, int64_t D_KV, int64_t D_H, int32_t dtype) {
  return fold_supported(H, D_KV, D_H, dtype) ? 1 : 0;
}

int64_t vafa_absorb_fwd_fold_workspace(const vafa_plan_info *info, int64_t D_KV, int64_t D_H) {
  if (check_info(info, 2)) return -1;
  return carve_absorb(nullptr, info, D_KV, D_H, false, true).bytes;
}

int vafa_absorb_fwd_fold(const void *q_proj, const void *W_K, const void *X, const void *W_V,
                         void *O, float *lse, const int32_t *plan_dev,
                         const vafa_plan_info *info, int64_t D_KV, int64_t D_H, int32_t dtype,
                         float scale, void *workspace, int64_t workspace_bytes, void *stream) {
  if (int rc = check_info(info, 2)) return rc;
  if (int rc = check_absorb_dims(D_KV, D_H)) return rc;
  if (!fold_supported(info->H, D_KV, D_H, dtype))
    return fail(VAFA_ERR_VALUE,
                "absorb_fwd_fold: H=%lld, D_KV=%lld, D_H=%lld, dtype %d is not a shape of the "
                "folded kernel (vafa_absorb_fold_supported); use vafa_absorb_project_fwd + "
                "vafa_absorb_fwd",
                (long long)info->H, (long long)D_KV, (long long)D_H, (int)dtype);
  if (int rc = check_aligned("absorb_fwd_fold", {q_proj, W_K, X, W_V, O})) return rc;
  AbsorbWs w = carve_absorb(workspace, info, D_KV, D_H, false, true);
  if (workspace_bytes < w.bytes || (w.bytes > 0 && workspace == nullptr))
    return fail(VAFA_ERR_WORKSPACE, "workspace of %lld bytes, %lld needed",
                (long long)workspace_bytes, (long long)w.bytes);
  AbsorbArgs a{};
  a.u = q_proj; a.wk = W_K; a.wkt = w.wkt; a.fold = true;
  a.X = X; a.wv = W_V; a.O = O; a.lse = lse;
  a.part_o = w.part_o; a.part_lse = w.part_lse; a.wvt = w.wvt;
  a.items = plan_dev + info->off_fwd; a.n_items = info->n_fwd;
  a.comb_items = plan_dev + info->off_comb; a.n_comb = info->n_comb;
  a.comb_rows = (int)info->max_comb_rows;
  a.T_q = info->T_q; a.T_k = info->T_k;
  a.H = (int)info->H; a.F = (int)D_KV; a.DH = (int)D_H; a.scale = scale;
  if (int rc = by_dtype<AFwd>(dtype, a, (hipStream_t)stream)) return rc;
  return check_launch("vafa_absorb_fwd_fold");
}

int vafa_absorb_project_u(const void *q_proj, const void *W_K, void *u, int64_t T_q, int64_t H,
                          int64_t D_KV, int64_t D_H, int32_t dtype, void *stream) {
  if (int rc = check_project_dims("project_u", T_q, H, 8, D_KV, D_H)) return rc;
  if (int rc = check_aligned("project_u", {q_proj, W_K, u})) return rc;
  switch (dtype) {
    case VAFA_BF16:
      project_u<bf16>(q_proj, W_K, u, T_q, (int)H, (int)D_KV, (int)D_H, (hipStream_t)stream);
      break;
    case VAFA_F16:
      project_u<f16>(q_proj, W_K, u, T_q, (int)H, (int)D_KV, (int)D_H, (hipStream_t)stream);
      break;
    default:
      return fail(VAFA_ERR_VALUE, "project_u: 16-bit dtypes only (got %d)", (int)dtype);
  }
  return check_launch("vafa_absorb_project_u");
}

int64_t vafa_absorb_project_workspace(int64_t T_q, int64_t H, int64_t D_Q, int64_t D_KV,
                                      int64_t D_H, int32_t backward) {
  if (check_project_dims("project_workspace", T_q, H, D_Q, D_KV, D_H) != VAFA_OK) return -1;
  return carve_project(nullptr, T_q, H, D_Q, D_KV, D_H, backward != 0).bytes;
}

int vafa_absorb_project_fwd(const void *q_raw, const void *W_Q, const void *W_K, void *q_proj,
                            void *u, int64_t T_q, int64_t H, int64_t D_Q, int64_t D_KV,
                            int64_t D_H, int32_t dtype, void *workspace, int64_t workspace_bytes,
                            void *stream) {
  if (int rc = check_project_dims("project_fwd", T_q, H, D_Q, D_KV, D_H)) return rc;
  if (int rc = check_aligned("project_fwd", {q_raw, W_Q, W_K, q_proj, u, workspace})) return rc;
  const ProjectWs w = carve_project(workspace, T_q, H, D_Q, D_KV, D_H, false);
  if (workspace_bytes < w.bytes || workspace == nullptr)
    return fail(VAFA_ERR_WORKSPACE, "project_fwd: workspace of %lld bytes, %lld needed",
                (long long)workspace_bytes, (long long)w.bytes);
  const hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case VAFA_BF16:
      project_fwd<bf16>(q_raw, W_Q, W_K, q_proj, u, T_q, (int)H, (int)D_Q, (int)D_KV, (int)D_H, w, st);
      break;
    case VAFA_F16:
      project_fwd<f16>(q_raw, W_Q, W_K, q_proj, u, T_q, (int)H, (int)D_Q, (int)D_KV, (int)D_H, w, st);
      break;
    default:
      return fail(VAFA_ERR_VALUE, "project_fwd: 16-bit dtypes only (got %d)", (int)dtype);
  }
  return check_launch("vafa_absorb_project_fwd");
}

int vafa_absorb_project_bwd(const void *q_raw, const void *W_Q, const void *W_K,
                            const void *q_proj, const void *du, void *dq_raw, void *dW_Q,
                            void *dW_K, int64_t T_q, int64_t H, int64_t D_Q, int64_t D_KV,
                            int64_t D_H, int32_t dtype, void *workspace, int64_t workspace_bytes,
                            void *stream) {
  if (int rc = check_project_dims("project_bwd", T_q, H, D_Q, D_KV, D_H)) return rc;
  if (int rc = check_aligned("project_bwd", {q_raw, W_Q, W_K, q_proj, du, dq_raw, dW_Q, dW_K,
                                             workspace}))
    return rc;
  const ProjectWs w = carve_project(workspace, T_q, H, D_Q, D_KV, D_H, true);
  if (workspace_bytes < w.bytes || workspace == nullptr)
    return fail(VAFA_ERR_WORKSPACE, "project_bwd: workspace of %lld bytes, %lld needed",
                (long long)workspace_bytes, (long long)w.bytes);
  const hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case VAFA_BF16:
      project_bwd<bf16>(q_raw, W_Q, W_K, q_proj, du, dq_raw, dW_Q, dW_K, T_q, (int)H, (int)D_Q,
                        (int)D_KV, (int)D_H, w, st);
      break;
    case VAFA_F16:
      project_bwd<f16>(q_raw, W_Q, W_K, q_proj, du, dq_raw, dW_Q, dW_K, T_q, (int)H, (int)D_Q,
                       (int)D_KV, (int)D_H, w, st);
      break;
    default:
      return fail(VAFA_ERR_VALUE, "project_bwd: 16-bit dtypes only (got %d)", (int)dtype);
  }
  return check_launch("vafa_absorb_project_bwd");
}

int vafa_absorb_bwd(const void *u, const void *X, const void *W_V, const void *O,
                    const void *dO, const float *lse, void *du, void *dX, void *dW_V,
                    const int32_t *plan_dev, const vafa_plan_info *info, int64_t D_KV,
                    int64_t D_H, int32_t dtype, float scale, void *workspace,
                    int64_t workspace_bytes, void *stream) {
  if (int rc = check_info(info, 2)) return rc;
  if (int rc = check_absorb_dims(D_KV, D_H)) return rc;
  AbsorbWs w = carve_absorb(workspace, info, D_KV, D_H, true);
  if (workspace_bytes < w.bytes || (w.bytes > 0 && workspace == nullptr))
    return fail(VAFA_ERR_WORKSPACE, "workspace of %lld bytes, %lld needed",
                (long long)workspace_bytes, (long long)w.bytes);
  const hipStream_t st = (hipStream_t)stream;
  AbsorbArgs a{};
  a.u = u; a.X = X; a.wv = W_V; a.O_in = O; a.dO = dO; a.lse_in = lse;
  a.du = du; a.dX = dX; a.dwv = dW_V;
  const bool pad = absorb_pad(info->H, D_KV, D_H, dtype, true);
  const int64_t F = pad ? absorb_fpad(D_KV) : D_KV;
  const int eb = elem_bytes(dtype);
  if (pad) {
    launch_pad_cols(u, w.pu, info->T_q * info->H, D_KV, F, eb, st);
    launch_pad_cols(X, w.pX, info->T_k, D_KV, F, eb, st);
    launch_pad_cols(W_V, w.pW, 1, D_KV * info->H * D_H, F * info->H * D_H, eb, st);
    a.u = w.pu; a.X = w.pX; a.wv = w.pW;
    a.du = w.pdu; a.dX = w.pdX; a.dwv = w.pdW;
  }
  a.delta = w.delta; a.dax = w.dax; a.ax = w.ax; a.dwv_part = w.dwv_part;
  a.n_tchunks = w.n_tchunks; a.tchunk = w.tchunk;
  a.items = plan_dev + info->off_fwd; a.n_items = info->n_fwd;
  a.comb_items = plan_dev + info->off_comb; a.n_comb = info->n_comb;
  a.comb_rows = (int)info->max_comb_rows;
  a.kv_items = plan_dev + info->off_kv; a.n_kv = info->n_kv; a.n_kv_res = info->n_kv_res;
  a.qseg_items = plan_dev + info->off_qt; a.n_qseg = info->n_qt;
  a.T_q = info->T_q; a.T_k = info->T_k;
  a.H = (int)info->H; a.F = (int)F; a.DH = (int)D_H; a.scale = scale;
  if (int rc = by_dtype<ABwd>(dtype, a, st)) return rc;
  if (pad) {
    launch_unpad_cols(w.pdu, du, info->T_q * info->H, D_KV, F, eb, st);
    launch_unpad_cols(w.pdX, dX, info->T_k, D_KV, F, eb, st);
    launch_unpad_cols(w.pdW, dW_V, 1, D_KV * info->H * D_H, F * info->H * D_H, eb, st);
  }
  return check_launch("vafa_absorb_bwd");
}

}  // extern "C"
