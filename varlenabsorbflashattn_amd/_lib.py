"""ctypes binding of ``libvafa.so`` (the C ABI declared in include/vafa.h).

The library is built in-tree by ``varlenabsorbflashattn_amd.build``.  Loading
it is mandatory for every compute call: there is no CPU or eager fallback,
so a missing or stale library raises immediately.
"""
from __future__ import annotations

import ctypes as C
import os
import threading
from collections import OrderedDict
from typing import Optional, Tuple

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# VAFA_LIBRARY selects another build of the library (e.g. a tuning variant)
LIB_PATH = os.environ.get("VAFA_LIBRARY") or os.path.join(_HERE, "libvafa.so")

VAFA_OK = 0
VAFA_ERR_VALUE = -1
VAFA_ERR_ASSERT = -2
VAFA_ERR_RUNTIME = -3
VAFA_ERR_WORKSPACE = -4
VAFA_ERR_CAPACITY = -5

DT_F32, DT_F16, DT_BF16 = 0, 1, 2
# bytes of the static per-GPU scratch of vafa_varlen_fwd_noalloc
# (VAFA_NOALLOC_SCRATCH_BYTES in include/vafa.h)
NOALLOC_SCRATCH_BYTES = 64 << 20
PLAN_MAGIC = 0x56414641
ITEM_INTS = 8


class PlanInfo(C.Structure):
    _fields_ = [(n, C.c_int64) for n in (
        "magic", "kind", "n_seg", "T_q", "T_k", "H",
        "off_fwd", "n_fwd", "off_comb", "n_comb", "off_kv", "n_kv", "off_qt", "n_qt",
        "n_part_rows", "plan_ints", "q_tile", "k_tile", "max_split", "max_comb_rows", "n_kv_res",
        "off_dq", "n_dq", "off_dqc", "n_dqc", "max_dqc_rows", "off_fkv", "n_fkv",
        "off_fcomb", "n_fcomb", "n_fpart_rows", "max_fcomb_rows", "xcd_heads")]


_lib = None
_lock = threading.Lock()

_P = C.c_void_p
_I64 = C.c_int64
_I32 = C.c_int32
_PI64 = C.POINTER(C.c_int64)
_PI32 = C.POINTER(C.c_int32)
_PINFO = C.POINTER(PlanInfo)

_SIGS = {
    "vafa_version": (C.c_char_p, []),
    "vafa_last_error": (C.c_char_p, []),
    "vafa_seqinfo_to_cu": (C.c_int, [_PI64, _I64, _PI32]),
    "vafa_validate_cu": (C.c_int, [_PI64, _I64, _I64, C.c_char_p]),
    "vafa_validate_cu_absorb": (C.c_int, [_PI64, _I64, _I64, C.c_char_p]),
    "vafa_check_active_have_keys": (C.c_int, [_PI64, _PI64, _I64]),
    "vafa_chunk_indices": (C.c_int, [_PI64, _I64, _I32, _PI32, _I64, _PI64]),
    "vafa_plan_varlen": (C.c_int, [_PI64, _PI64, _I64, _I64, _I64, _PI32, _I64, _PINFO]),
    "vafa_plan_absorb": (C.c_int, [_PI64, _PI64, _I64, _I64, _I64, _I64, _PI32, _I64, _PINFO]),
    "vafa_varlen_fwd_workspace": (C.c_int64, [_PINFO, _I64]),
    "vafa_varlen_bwd_workspace": (C.c_int64, [_PINFO, _I64]),
    "vafa_absorb_fwd_workspace": (C.c_int64, [_PINFO, _I64, _I64]),
    "vafa_absorb_bwd_workspace": (C.c_int64, [_PINFO, _I64, _I64]),
    "vafa_absorb_fwd_fold_workspace": (C.c_int64, [_PINFO, _I64, _I64]),
    "vafa_absorb_fold_supported": (C.c_int, [_I64, _I64, _I64, _I32]),
    "vafa_varlen_fwd": (C.c_int, [_P, _P, _P, _P, _P, _P, _PINFO, _I64, _I32, C.c_float,
                                  _P, _I64, _P]),
    "vafa_varlen_fwd_noalloc": (C.c_int, [_P, _P, _P, _P, _P, _P, _PINFO, _I64, _I32, C.c_float,
                                          _P]),
    "vafa_varlen_bwd": (C.c_int, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _PINFO, _I64, _I32,
                                  C.c_float, _P, _I64, _P]),
    "vafa_varlen_bwd_stage": (C.c_int, [_I32, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _PINFO, _I64,
                                        _I32, C.c_float, _P, _I64, _P]),
    "vafa_absorb_project_u": (C.c_int, [_P, _P, _P, _I64, _I64, _I64, _I64, _I32, _P]),
    "vafa_absorb_project_workspace": (C.c_int64, [_I64, _I64, _I64, _I64, _I64, _I32]),
    "vafa_absorb_project_fwd": (C.c_int, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I32,
                                          _P, _I64, _P]),
    "vafa_absorb_project_bwd": (C.c_int, [_P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64,
                                          _I64, _I32, _P, _I64, _P]),
    "vafa_absorb_fwd": (C.c_int, [_P, _P, _P, _P, _P, _P, _PINFO, _I64, _I64, _I32, C.c_float,
                                  _P, _I64, _P]),
    "vafa_absorb_bwd": (C.c_int, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _PINFO, _I64, _I64,
                                  _I32, C.c_float, _P, _I64, _P]),
    "vafa_absorb_fwd_fold": (C.c_int, [_P, _P, _P, _P, _P, _P, _P, _PINFO, _I64, _I64, _I32,
                                       C.c_float, _P, _I64, _P]),
}

EXPORTED = tuple(_SIGS)


def lib():
    """Load (once) and return the ctypes handle of libvafa.so."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"{LIB_PATH} is missing: build it with "
                    "`python -m varlenabsorbflashattn_amd.build` (hipcc, gfx950)")
            # torch first, so the HIP runtime it ships is the one libvafa binds to
            import torch  # noqa: F401
            h = C.CDLL(LIB_PATH)
            for name, (res, args) in _SIGS.items():
                fn = getattr(h, name)
                fn.restype = res
                fn.argtypes = args
            _lib = h
    return _lib


def last_error() -> str:
    return lib().vafa_last_error().decode(errors="replace")


def check(rc: int) -> None:
    if rc == VAFA_OK:
        return
    msg = last_error()
    if rc == VAFA_ERR_VALUE:
        raise ValueError(msg)
    if rc == VAFA_ERR_ASSERT:
        raise AssertionError(msg)
    raise RuntimeError(f"vafa error {rc}: {msg}")


def _i64p(a: np.ndarray):
    return a.ctypes.data_as(_PI64)


def _i32p(a: np.ndarray):
    return a.ctypes.data_as(_PI32)


def as_host_i64(x) -> np.ndarray:
    """Host int64 copy of a cu_seqlens / seqinfo tensor or array (one D2H)."""
    try:
        import torch
        if isinstance(x, torch.Tensor):
            return np.ascontiguousarray(x.detach().to("cpu", torch.int64).numpy())
    except ImportError:  # pragma: no cover
        pass
    return np.ascontiguousarray(np.asarray(x, dtype=np.int64))


def as_host_i64_pair(a, b) -> Tuple[np.ndarray, np.ndarray]:
    """Host int64 copies of two cu_seqlens tensors with one device sync: the
    same tensor is copied once, two device tensors of one shape and dtype are
    stacked on the device and copied together."""
    import torch
    if a is b:
        h = as_host_i64(a)
        return h, h
    if (isinstance(a, torch.Tensor) and isinstance(b, torch.Tensor) and a.is_cuda and b.is_cuda
            and a.device == b.device and a.dtype == b.dtype and a.shape == b.shape
            and a.dim() == 1):
        h = as_host_i64(torch.stack((a.detach(), b.detach())))
        return np.ascontiguousarray(h[0]), np.ascontiguousarray(h[1])
    return as_host_i64(a), as_host_i64(b)


# ---- host metadata -----------------------------------------------------------

def seqinfo_to_cu(seqinfo: np.ndarray) -> np.ndarray:
    s = np.ascontiguousarray(seqinfo, dtype=np.int64)
    out = np.empty(max(s.size, 0) + 1, dtype=np.int32)
    check(lib().vafa_seqinfo_to_cu(_i64p(s), s.size, _i32p(out)))
    return out


def validate_cu(cu: np.ndarray, T: int, name: str) -> None:
    """The varlen operator's cu_seqlens checks and texts (fa/interface.py:96-118)."""
    c = np.ascontiguousarray(cu, dtype=np.int64)
    check(lib().vafa_validate_cu(_i64p(c), c.size, int(T), name.encode()))


def validate_cu_absorb(cu: np.ndarray, T: int, name: str) -> None:
    """The absorb operator's cu_seqlens checks and texts (ta/interface.py:92-106)."""
    c = np.ascontiguousarray(cu, dtype=np.int64)
    check(lib().vafa_validate_cu_absorb(_i64p(c), c.size, int(T), name.encode()))


def check_active_have_keys(cu_q: np.ndarray, cu_k: np.ndarray) -> None:
    a = np.ascontiguousarray(cu_q, dtype=np.int64)
    b = np.ascontiguousarray(cu_k, dtype=np.int64)
    check(lib().vafa_check_active_have_keys(_i64p(a), _i64p(b), a.size))


def chunk_indices(cu: np.ndarray, BT: int) -> np.ndarray:
    c = np.ascontiguousarray(cu, dtype=np.int64)
    n = C.c_int64(0)
    rc = lib().vafa_chunk_indices(_i64p(c), c.size, int(BT), None, 0, C.byref(n))
    if rc not in (VAFA_OK, VAFA_ERR_CAPACITY):
        check(rc)
    out = np.empty((n.value, 2), dtype=np.int32)
    check(lib().vafa_chunk_indices(_i64p(c), c.size, int(BT), _i32p(out), n.value, C.byref(n)))
    return out


class HostPlan:
    """A plan on the host: its info struct and int32 item array."""

    def __init__(self, info: PlanInfo, items: np.ndarray):
        self.info = info
        self.items = items

    def section(self, name: str) -> np.ndarray:
        off = getattr(self.info, "off_" + name)
        n = getattr(self.info, "n_" + name)
        return self.items[off:off + n * ITEM_INTS].reshape(n, ITEM_INTS)


def plan_varlen(cu_q: np.ndarray, cu_k: np.ndarray, H: int, D: int) -> HostPlan:
    a = np.ascontiguousarray(cu_q, dtype=np.int64)
    b = np.ascontiguousarray(cu_k, dtype=np.int64)
    if a.shape != b.shape:
        raise AssertionError(f"segment count mismatch: q has {a.size - 1}, k has {b.size - 1}")
    info = PlanInfo()
    check(lib().vafa_plan_varlen(_i64p(a), _i64p(b), a.size, H, D, None, 0, C.byref(info)))
    items = np.empty(info.plan_ints, dtype=np.int32)
    check(lib().vafa_plan_varlen(_i64p(a), _i64p(b), a.size, H, D, _i32p(items), items.size,
                                 C.byref(info)))
    return HostPlan(info, items)


def plan_absorb(cu_q: np.ndarray, cu_k: np.ndarray, H: int, F: int, DH: int) -> HostPlan:
    a = np.ascontiguousarray(cu_q, dtype=np.int64)
    b = np.ascontiguousarray(cu_k, dtype=np.int64)
    if a.shape != b.shape:
        raise AssertionError("segment count mismatch q vs k")
    info = PlanInfo()
    check(lib().vafa_plan_absorb(_i64p(a), _i64p(b), a.size, H, F, DH, None, 0, C.byref(info)))
    items = np.empty(info.plan_ints, dtype=np.int32)
    check(lib().vafa_plan_absorb(_i64p(a), _i64p(b), a.size, H, F, DH, _i32p(items),
                                 items.size, C.byref(info)))
    return HostPlan(info, items)


# ---- device plans (cached by cu_seqlens content) ------------------------------

class DevicePlan:
    def __init__(self, host: HostPlan, device):
        import torch
        self.host = host
        self.info = host.info
        t = torch.from_numpy(host.items)
        if host.items.size == 0:
            t = torch.zeros(ITEM_INTS, dtype=torch.int32)
        self.items = t.to(device, non_blocking=False)


_CACHE: "OrderedDict[tuple, DevicePlan]" = OrderedDict()
_CACHE_MAX = 64


def device_plan(kind: str, cu_q: np.ndarray, cu_k: np.ndarray, dims: tuple, device) -> DevicePlan:
    """The cached device plan for these cu_seqlens, marked as in use on the
    current stream: a plan evicted from the cache while a kernel on another
    stream still reads it keeps its memory until that stream's work is done."""
    import torch
    key = (kind, cu_q.tobytes(), cu_k.tobytes(), dims, str(device))
    with _lock:
        dp = _CACHE.get(key)
        if dp is not None:
            _CACHE.move_to_end(key)
    if dp is None:
        host = (plan_varlen(cu_q, cu_k, *dims) if kind == "varlen"
                else plan_absorb(cu_q, cu_k, *dims))
        dp = DevicePlan(host, device)
        with _lock:
            _CACHE[key] = dp
            while len(_CACHE) > _CACHE_MAX:
                _CACHE.popitem(last=False)
    if dp.items.is_cuda:
        dp.items.record_stream(torch.cuda.current_stream(dp.items.device))
    return dp


def dtype_code(dtype) -> int:
    import torch
    if dtype == torch.bfloat16:
        return DT_BF16
    if dtype == torch.float16:
        return DT_F16
    if dtype == torch.float32:
        return DT_F32
    raise AssertionError(f"dtype {dtype} not supported (float32, float16, bfloat16)")


def stream_ptr(device) -> int:
    import torch
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t) -> Optional[int]:
    return None if t is None else t.data_ptr()
