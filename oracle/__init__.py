"""CPU oracle for the SSLA hot path -- TEST INFRASTRUCTURE ONLY.

Restates the reference's (haohq19/ssla) arithmetic on the CPU so that the
HIP path can be checked against it.  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may
import this package, and only as the checker / baseline: the product
(``ssla_amd``) never routes through it.

* ``liboracle.so`` (oracle.c, fp64): GLA recurrent and chunked forms, the
  diagonal scan, the per-site sparse step, scatter max/mean.
* numpy here: the parallel (quadratic) GLA form and small helpers.

Parity pins of each function live in tests/test_oracle.py (closed forms,
cross-algorithm agreement, brute force); see the header of that file.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

_lib = None

_dp = np.ctypeslib.ndpointer
_f32 = _dp(dtype=np.float32, flags="C_CONTIGUOUS")
_f64 = _dp(dtype=np.float64, flags="C_CONTIGUOUS")
_i64 = _dp(dtype=np.int64, flags="C_CONTIGUOUS")
_i32 = _dp(dtype=np.int32, flags="C_CONTIGUOUS")


class _Opt:
    """ndpointer that also accepts None (NULL)."""

    def __init__(self, base):
        self.base = base

    def from_param(self, obj):
        if obj is None:
            return None
        return self.base.from_param(obj)


def load():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            from .build import build
            build()
        lib = C.CDLL(str(LIB_PATH))
        ci, cd, c64 = C.c_int, C.c_double, C.c_int64
        lib.oracle_gla_recurrent.argtypes = [_f32, _f32, _f32, _f32, _i64, ci, ci, ci, ci, cd,
                                             _Opt(_f32), _f64, _Opt(_f64)]
        lib.oracle_gla_recurrent_bwd.argtypes = [_f32, _f32, _f32, _f32, _i64, ci, ci, ci, ci, cd,
                                                 _Opt(_f32), _f32, _Opt(_f32), _f64, _f64, _f64, _f64,
                                                 _Opt(_f64)]
        lib.oracle_gla_chunk.argtypes = [_f32, _f32, _f32, _f32, _i64, ci, ci, ci, ci, cd,
                                         _Opt(_f32), ci, _f64, _Opt(_f64)]
        lib.oracle_diag_scan.argtypes = [_f32, _f32, _i64, ci, c64, ci, _f64]
        lib.oracle_diag_scan_bwd.argtypes = [_f32, _f32, _f32, _i64, ci, c64, ci, _f64, _f64]
        lib.oracle_sparse_gla_step.argtypes = [_i32, ci, _f32, _f32, _f32, _f32, _f32, ci, ci, ci,
                                               cd, _f64]
        lib.oracle_scatter_max.argtypes = [_f32, _i64, c64, ci, c64, _f32, _i64]
        lib.oracle_scatter_mean.argtypes = [_f32, _i64, c64, ci, c64, _f64]
        for fn in (lib.oracle_gla_recurrent, lib.oracle_gla_recurrent_bwd, lib.oracle_gla_chunk, lib.oracle_diag_scan, lib.oracle_diag_scan_bwd,
                   lib.oracle_sparse_gla_step, lib.oracle_scatter_max, lib.oracle_scatter_mean):
            fn.restype = None
        _lib = lib
    return _lib


def _f(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def gla_recurrent(q, k, v, g, cu_seqlens, scale=None, initial_state=None, output_final_state=True):
    """naive_gla_recurrent (reference ops/gla/naive.py:50-111) in fp64.
    Arrays: q, k, g [T,H,K]; v [T,H,V]; cu_seqlens [N+1]; state [N,H,K,V].
    Returns (o [T,H,V] fp64, final_state [N,H,K,V] fp64 or None)."""
    q, k, v, g = _f(q), _f(k), _f(v), _f(g)
    T, H, K = q.shape
    V = v.shape[-1]
    cu = np.ascontiguousarray(cu_seqlens, dtype=np.int64)
    N = cu.size - 1
    if scale is None:
        scale = K ** -0.5
    h0 = None if initial_state is None else _f(initial_state)
    o = np.zeros((T, H, V), np.float64)
    ht = np.zeros((N, H, K, V), np.float64) if output_final_state else None
    load().oracle_gla_recurrent(q, k, v, g, cu, N, H, K, V, float(scale), h0, o, ht)
    return o, ht


def gla_recurrent_bwd(q, k, v, g, cu_seqlens, do, scale=None, initial_state=None, dht=None):
    """Gradients (dq, dk, dv, dg, dh0) of naive_gla_recurrent (o and the
    final state) for output gradients do [T, H, V] and dht [N, H, K, V] (or
    None), fp64; dh0 is None without an initial state."""
    q, k, v, g, do = _f(q), _f(k), _f(v), _f(g), _f(do)
    T, H, K = q.shape
    V = v.shape[-1]
    cu = np.ascontiguousarray(cu_seqlens, dtype=np.int64)
    N = cu.size - 1
    scale = K ** -0.5 if scale is None else float(scale)
    h0 = None if initial_state is None else _f(initial_state)
    dht = None if dht is None else _f(dht)
    dq, dk, dg = (np.zeros((T, H, K)) for _ in range(3))
    dv = np.zeros((T, H, V))
    dh0 = np.zeros((N, H, K, V)) if h0 is not None else None
    load().oracle_gla_recurrent_bwd(q, k, v, g, cu, N, H, K, V, scale, h0, do, dht, dq, dk, dv, dg, dh0)
    return dq, dk, dv, dg, dh0


def gla_chunk(q, k, v, g, cu_seqlens, scale=None, initial_state=None, output_final_state=True,
              chunk_size=64):
    """chunk_gla_fwd's chunked algorithm (reference ops/gla/chunk.py:906-960) in fp64."""
    q, k, v, g = _f(q), _f(k), _f(v), _f(g)
    T, H, K = q.shape
    V = v.shape[-1]
    cu = np.ascontiguousarray(cu_seqlens, dtype=np.int64)
    N = cu.size - 1
    if scale is None:
        scale = K ** -0.5
    h0 = None if initial_state is None else _f(initial_state)
    o = np.zeros((T, H, V), np.float64)
    ht = np.zeros((N, H, K, V), np.float64) if output_final_state else None
    load().oracle_gla_chunk(q, k, v, g, cu, N, H, K, V, float(scale), h0, int(chunk_size), o, ht)
    return o, ht


def gla_parallel(q, k, v, g, cu_seqlens, scale=None):
    """naive_gla_parallel (reference ops/gla/naive.py:6-47) in fp64 numpy:
    global cumsum per sequence, A = sum_k q k exp(Gc_i - Gc_j) * scale,
    lower-triangular mask, o = A v.  No state in or out; O(T^2 K) memory,
    so only for small T."""
    q, k, v, g = (np.asarray(a, np.float64) for a in (q, k, v, g))
    T, H, K = q.shape
    if scale is None:
        scale = K ** -0.5
    cu = np.asarray(cu_seqlens, np.int64)
    out = np.zeros((T, H, v.shape[-1]), np.float64)
    for n in range(cu.size - 1):
        s, e = int(cu[n]), int(cu[n + 1])
        if e <= s:
            continue
        qn, kn, vn, gn = (a[s:e].transpose(1, 0, 2) for a in (q, k, v, g))  # [H, Tn, D]
        gc = np.cumsum(gn, axis=1)
        A = np.einsum("htk,hsk,htsk->hts", qn, kn,
                      np.exp(gc[:, :, None, :] - gc[:, None, :, :])) * scale
        A = np.tril(A)
        out[s:e] = np.einsum("hts,hsv->htv", A, vn).transpose(1, 0, 2)
    return out


def diag_scan(u, g, cu_seqlens):
    """sequential_scan_fwd (reference ops/common/scan.py:20-43) in fp64."""
    u, g = _f(u), _f(g)
    T, C_ = u.shape
    cu = np.ascontiguousarray(cu_seqlens, dtype=np.int64)
    h = np.zeros((T, C_), np.float64)
    load().oracle_diag_scan(u, g, cu, cu.size - 1, T, C_, h)
    return h


def diag_scan_bwd(u, g, dout, cu_seqlens):
    """sequential_scan_bwd (reference ops/common/scan.py:55-86) in fp64:
    (du, dg) for the output gradient dout."""
    u, g, dout = _f(u), _f(g), _f(dout)
    T, C_ = u.shape
    cu = np.ascontiguousarray(cu_seqlens, dtype=np.int64)
    du = np.zeros((T, C_), np.float64)
    dg = np.zeros((T, C_), np.float64)
    load().oracle_diag_scan_bwd(u, g, dout, cu, cu.size - 1, T, C_, du, dg)
    return du, dg


def sparse_gla_step(site_idx, q, k, v, g, state, scale=None):
    """One bin of the per-site update; `state` (fp32 numpy) is updated in
    place, returns o [n, H, V] fp64."""
    q, k, v, g = _f(q), _f(k), _f(v), _f(g)
    n, H, K = q.shape
    V = v.shape[-1]
    if scale is None:
        scale = K ** -0.5
    assert state.dtype == np.float32 and state.flags.c_contiguous
    o = np.zeros((n, H, V), np.float64)
    load().oracle_sparse_gla_step(np.ascontiguousarray(site_idx, np.int32), n, q, k, v, g, state,
                                  H, K, V, float(scale), o)
    return o


def scatter_max(src, index, n_out):
    """torch_scatter.scatter_max semantics, dim 0, first-index tie rule."""
    src = _f(src)
    E, C_ = src.shape
    out = np.zeros((n_out, C_), np.float32)
    arg = np.zeros((n_out, C_), np.int64)
    load().oracle_scatter_max(src, np.ascontiguousarray(index, np.int64), E, C_, n_out, out, arg)
    return out, arg


def scatter_mean(src, index, n_out):
    """torch_scatter.scatter_mean semantics, dim 0 (fp64 accumulation)."""
    src = _f(src)
    E, C_ = src.shape
    out = np.zeros((n_out, C_), np.float64)
    load().oracle_scatter_mean(src, np.ascontiguousarray(index, np.int64), E, C_, n_out, out)
    return out
