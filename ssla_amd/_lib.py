"""ctypes binding of libssla_amd.so (the C-ABI declared in include/ssla_amd.h).

Only plain pointers, sizes and a stream handle cross this boundary.  The
library is loaded lazily on first use; when it is missing or cannot be
loaded every entry point raises -- there is no fallback implementation.
"""
from __future__ import annotations

import ctypes as C
import os
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libssla_amd.so"

SSLA_OK = 0
SSLA_ERR_ARG = -1
SSLA_ERR_DTYPE = -2
SSLA_ERR_WORKSPACE = -3
SSLA_ERR_LAUNCH = -4
SSLA_ERR_UNSUPPORTED = -5

SSLA_F32, SSLA_BF16, SSLA_F16 = 0, 1, 2
DTYPE_CODE = {torch.float32: SSLA_F32, torch.bfloat16: SSLA_BF16, torch.float16: SSLA_F16}

_vp, _i32, _i64, _f32, _sz = C.c_void_p, C.c_int, C.c_int64, C.c_float, C.c_size_t


class HeadLevel(C.Structure):
    """ssla_head_level of include/ssla_amd.h."""
    _fields_ = [("grid", C.c_void_p), ("w_br", C.c_void_p), ("br_scale", C.c_void_p), ("br_shift", C.c_void_p),
                ("w_pred", C.c_void_p), ("b_pred", C.c_void_p), ("c", C.c_int), ("h", C.c_int), ("w", C.c_int),
                ("stride", C.c_int)]

class GridLevel(C.Structure):
    """ssla_grid_level of include/ssla_amd.h."""
    _fields_ = [("events", C.c_void_p), ("lengths", C.c_void_p), ("batch", C.c_void_p), ("h", C.c_void_p),
                ("w", C.c_void_p), ("grid", C.c_void_p), ("E", C.c_int64), ("G", C.c_int64), ("C", C.c_int),
                ("Hg", C.c_int), ("Wg", C.c_int)]


GRIDS_MAX_LEVELS, GRIDS_MAX_CELLS = 8, 16384

# name -> (restype, argtypes); must match include/ssla_amd.h
SIGNATURES = {
    "ssla_version": (_i32, []),
    "ssla_last_error": (C.c_char_p, []),
    "ssla_gla_chunk_workspace_size": (_sz, [_i32, _i64, _i32, _i32, _i32]),
    "ssla_gla_chunk_fwd": (_i32, [_vp, _vp, _vp, _vp, _i32, _vp, _i32, _i64, _i32, _i32, _i32,
                                  _f32, _vp, _vp, _vp, _i32, _vp, _sz, _vp]),
    "ssla_gla_chunk_fwd_noalloc": (_i32, [_vp, _vp, _vp, _vp, _i32, _vp, _i32, _i64, _i32, _i32, _i32,
                                          _f32, _vp, _vp, _vp, _i32, _vp]),
    "ssla_gla_chunk_f32_fwd": (_i32, [_vp, _vp, _vp, _vp, _vp, _i32, _i64, _i32, _i32, _i32, _f32, _vp, _vp, _vp,
                                       _vp]),
    "ssla_gla_chunk_f32_bwd_workspace_size": (_sz, [_i32, _i64, _i32]),
    "ssla_gla_chunk_f32_bwd": (_i32, [_vp, _vp, _vp, _vp, _vp, _i32, _i64, _i32, _i32, _i32, _f32, _vp, _vp, _vp,
                                       _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "ssla_gla_chunk_bwd_workspace_size": (_sz, [_i32, _i64, _i32, _i32, _i32]),
    "ssla_gla_chunk_bwd": (_i32, [_vp, _vp, _vp, _vp, _i32, _vp, _i32, _i64, _i32, _i32, _i32, _f32, _vp,
                                  _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _vp, _sz, _vp]),
    "ssla_gla_recurrent_workspace_size": (_sz, [_i32, _i64, _i32, _i32, _i32]),
    "ssla_gla_recurrent_fwd": (_i32, [_vp, _vp, _vp, _vp, _i32, _vp, _i32, _i64, _i32, _i32, _i32,
                                      _f32, _vp, _vp, _vp, _vp, _i32, _vp, _i32, _vp, _sz, _vp]),
    "ssla_diag_scan_fwd": (_i32, [_vp, _vp, _vp, _i32, _i64, _i32, _vp, _vp]),
    "ssla_diag_scan_bwd": (_i32, [_vp, _vp, _vp, _vp, _i32, _i64, _i32, _vp, _vp, _vp]),
    "ssla_sparse_gla_step": (_i32, [_vp, _i32, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32,
                                    _f32, _vp, _vp, _vp]),
    "ssla_status_read": (_i32, [_vp, C.POINTER(_i32), _vp]),
    "ssla_site_project": (_i32, [_vp, _i64, _i32, _vp, _i32, _f32, _vp, _vp, _vp, _vp, _vp]),
    "ssla_site_finish": (_i32, [_vp, _i64, _i32, _vp, _vp, _i32, _vp, _vp, _vp, _f32, _i32, _vp, _vp]),
    "ssla_site_gla_block_workspace_size": (_sz, [_i64, _i64, _i32, _i32]),
    "ssla_site_gla_block": (_i32, [_vp, _i64, _i32, _vp, _vp, _vp, _vp, _i64, _i32, _i32, _vp, _i32, _i32, _i32, _vp,
                                   _f32, _f32, _vp, _vp, _vp, _vp, _f32, _i32, _vp, _vp, _vp, _sz, _vp]),
    "ssla_detect_head": (_i32, [C.POINTER(HeadLevel), _i32, _i32, _i32, _i32, _vp, _vp]),
    "ssla_scatter_workspace_size": (_sz, [_i64, _i32, _i64]),
    "ssla_scatter_max": (_i32, [_vp, _vp, _i64, _i32, _i64, _i32, _vp, _vp, _vp, _sz, _vp]),
    "ssla_scatter_mean": (_i32, [_vp, _vp, _i64, _i32, _i64, _i32, _vp, _vp, _sz, _vp]),
    "ssla_scatter_check": (_i32, [_vp, C.POINTER(_i32), _vp]),
    "ssla_rf_lut_shape": (_i32, [_i32, _i32, _i32, _i32, _i32, _i32, C.POINTER(_i64)]),
    "ssla_rf_lut": (_i32, [_i32, _i32, _i32, _i32, _i32, _i32, _vp, _vp, _vp]),
    "ssla_events_counts": (_i32, [_vp, C.POINTER(_i64), _i32, C.POINTER(_i32), _vp]),
    "ssla_events_counts_async": (_i32, [_vp, _vp, _vp]),
    "ssla_group_events_workspace_size": (_sz, [_i32, _i64]),
    "ssla_group_events": (_i32, [_vp, _vp, _i32, _i64, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp,
                                 _vp, _sz, _vp]),
    "ssla_preprocess_events": (_i32, [_vp, _vp, _i32, _i64, _i32, _i32, _i32, _i32, _i64, _vp, _vp, _vp, _vp,
                                      _vp, _vp, _vp, _sz, _vp]),
    "ssla_rf_scatter_workspace_size": (_sz, [_i64, _i32, _i32, _i32, _i64, _i64]),
    "ssla_rf_scatter_plan": (_i32, [_vp, _vp, _vp, _vp, _i64, _vp, _i64, _i32, _i32, _i32, _vp, _i64, _i32, _i64,
                                    _vp, _sz, _vp]),
    "ssla_rf_scatter_fill": (_i32, [_vp, _i64, _vp, _i64, _i32, _i32, _i32, _vp, _i64, _i32, _i64, _i64, _i64,
                                    _i64, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "ssla_rf_scatter_fill_sorted": (_i32, [_vp, _vp, _vp, _vp, _i64, _vp, _i64, _i32, _i32, _i32, _vp, _i64, _i32,
                                           _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "ssla_gather_rows": (_i32, [_vp, _i64, _vp, _i64, _i32, _vp, _vp]),
    "ssla_index_add_rows_workspace_size": (_sz, [_i64]),
    "ssla_index_add_rows": (_i32, [_vp, _vp, _i64, _i32, _i64, _vp, _vp, _sz, _vp]),
    "ssla_mos_attention_workspace_size": (_sz, [_i64, _i32, _i32, _i32, _i64, _i64]),
    "ssla_mos_attention_lds_bytes": (_sz, [_i32, _i32, _i32, _i32, _i32]),
    "ssla_mos_attention_fwd": (_i32, [_vp, _i64, _i32, _vp, _vp, _i64, _vp, _i64, _i32, _vp, _i32, _vp, _vp, _vp,
                                      _vp, _vp, _i32, _vp, _vp, _vp, _f32, _i32, _vp, _vp, _sz, _vp]),
    "ssla_sort_pairs_workspace_size": (_sz, [_i64]),
    "ssla_sort_pairs": (_i32, [_vp, _vp, _i64, _i32, _vp, _vp, _vp, _sz, _vp]),
    "ssla_segments_workspace_size": (_sz, [_i64]),
    "ssla_truncate_packed": (_i32, [_vp, _vp, _i64, _i64, _i32, _i64, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "ssla_temporal_dropout_index": (_i32, [_vp, _i64, _i64, _vp, _i64, _vp, _vp, _sz, _vp]),
    "ssla_expand_segments": (_i32, [_vp, _vp, _i64, _i64, _vp, _vp, _sz, _vp]),
    "ssla_pool_segments": (_i32, [_vp, _vp, _i64, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "ssla_sparse_pool_workspace_size": (_sz, [_i64, _i64, _i32, _i32, _i32, _i64, _i32, _i64]),
    "ssla_sparse_pool_plan": (_i32, [_vp, _vp, _vp, _vp, _i64, _vp, _i64, _i32, _i32, _i32, _vp, _i64, _i32, _i64,
                                     C.POINTER(_i64), _vp, _sz, _vp]),
    "ssla_sparse_pool_plan_enqueue": (_i32, [_vp, _vp, _vp, _vp, _i64, _vp, _i64, _i32, _i32, _i32, _vp, _i64, _i32,
                                             _i64, _vp, _sz, _vp]),
    "ssla_sparse_pool_plan_finish": (_i32, [_vp, _i64, _vp, _i64, _i32, _i32, _i32, _vp, _i64, _i32, _i64,
                                            C.POINTER(_i64), _i32, C.POINTER(_i64), _vp, _sz, _vp]),
    "ssla_sparse_pool_emit": (_i32, [_vp, _i32, _i64, _i64, _i32, _i32, _i32, _i64, _i32, _i64, _vp, _i32, _i64,
                                     _i64, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "ssla_sparse_pool_emit_linear": (_i32, [_vp, _i32, _vp, _i32, _i64, _i64, _i32, _i32, _i32, _i64, _i32, _i64,
                                            _i32, _i64, _i64, _i64, _vp, _vp, _sz, _vp]),
    "ssla_pixel_delays": (_i32, [_vp, _i64, _i32, _vp, _i64, _vp, _sz, _vp]),
    "ssla_events_to_grid": (_i32, [_vp, _i64, _i32, _vp, _vp, _vp, _vp, _i64, _i32, _i32, _i32, _vp, _vp, _sz,
                                   _vp]),
    "ssla_events_to_grids": (_i32, [C.POINTER(GridLevel), _i32, _i32, _vp, _vp]),
    "ssla_dat_decode_batch": (_i32, [_vp, _i64, _vp, _i32, _i64, _i32, _vp, _vp]),
}

_lock = threading.Lock()
_lib = None


class SslaError(RuntimeError):
    """Launch or workspace failure reported by libssla_amd."""


def load() -> C.CDLL:
    """Load (once) and return the library; raise if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            path = Path(os.environ.get("SSLA_AMD_LIB", LIB_PATH))
            if not path.exists():
                raise ImportError(
                    f"{path} is missing: build it with `python -m ssla_amd.build` "
                    "(the HIP path has no fallback)")
            lib = C.CDLL(str(path))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def check(status: int, what: str) -> None:
    if status == SSLA_OK:
        return
    msg = load().ssla_last_error().decode(errors="replace") or what
    if status == SSLA_ERR_ARG:
        raise ValueError(msg)
    if status == SSLA_ERR_DTYPE:
        raise TypeError(msg)
    if status == SSLA_ERR_UNSUPPORTED:
        raise NotImplementedError(msg)
    raise SslaError(f"{msg} (status {status})")


def new_status(device) -> torch.Tensor:
    """A device status word set to SSLA_OK (see ssla_status_read)."""
    return torch.zeros(1, dtype=torch.int32, device=device)


def read_status(status: torch.Tensor) -> int:
    """Value of a device status word (synchronises its stream)."""
    v = C.c_int(0)
    check(load().ssla_status_read(status.data_ptr(), C.byref(v), stream_of(status)), "ssla_status_read")
    return v.value


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    """The raw handle of the current stream of t's device."""
    return torch._C._cuda_getCurrentRawStream(t.get_device())


class ParamWatch:
    """A cheap validity check for values derived from a module's parameters
    and buffers.  For every tensor read (a dotted path from ``root``) it
    keeps the dict that holds the tensor (``_parameters`` / ``_buffers`` of
    its module), the tensor, its version and data pointer, and for every
    module on the way the ``_modules`` dict that holds it: an in-place
    update, a reassigned parameter, a move (``.to``) or a replaced submodule
    fails ``valid()``."""
    __slots__ = ("items",)

    def __init__(self, root: torch.nn.Module, paths):
        items, seen = [], set()
        for path in paths:
            parts = path.split(".")
            m = root
            for name in parts[:-1]:
                child = m._modules[name]
                if (id(m._modules), name) not in seen:
                    seen.add((id(m._modules), name))
                    items.append((m._modules, name, child, None, None))
                m = child
            name = parts[-1]
            d = m._parameters if name in m._parameters else m._buffers
            t = d.get(name)
            items.append((d, name, t, None, None) if t is None else (d, name, t, t._version, t.data_ptr()))
        self.items = tuple(items)

    def valid(self) -> bool:
        for d, k, obj, ver, p in self.items:
            cur = d.get(k)
            if cur is not obj or (ver is not None and (cur._version != ver or cur.data_ptr() != p)):
                return False
        return True


def require_cuda(*tensors: torch.Tensor) -> torch.device:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError("ssla_amd kernels need device tensors (got a CPU tensor)")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} and {t.device}")
    return dev


def require_no_grad(name: str, *tensors: torch.Tensor) -> None:
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in tensors):
        raise NotImplementedError(f"{name}: only the forward pass is implemented "
                                  "(call it under torch.no_grad())")
