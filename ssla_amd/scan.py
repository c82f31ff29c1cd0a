"""Sparse sequential scans on MI355X.

* :func:`scan` -- drop-in for ``ops.common.scan.scan(u, g, cu_seqlens)``
  (reference ops/common/scan.py:140-163): varlen diagonal gated scan
  ``h_t = g_t * h_{t-1} + u_t`` with a zero state at each sequence start,
  with its backward (:class:`SequentialScan`).
* :func:`sparse_gla_step` -- one time bin of the per-site matrix-state GLA
  update at active sites only (no reference function; its math is
  ``naive_gla_recurrent``, reference ops/gla/naive.py:50-111, on a length-1
  sequence per active site whose initial state is the stored site state).
* :func:`sparse_gla_scan` -- the same update over many bins at once, as a
  varlen recurrence per site whose state is gathered from and scattered back
  to the resident state table.
"""
from __future__ import annotations

from typing import Optional

import torch

from . import _lib
from .gla import _recurrent

__all__ = ["scan", "SequentialScan", "sparse_gla_step", "sparse_gla_scan"]


def _scan_fwd(u: torch.Tensor, g: torch.Tensor, cu: torch.Tensor) -> torch.Tensor:
    T, C = u.shape
    h = torch.empty_like(u)
    st = _lib.load().ssla_diag_scan_fwd(_lib.ptr(u), _lib.ptr(g), _lib.ptr(cu), cu.numel() - 1, T, C,
                                        _lib.ptr(h), _lib.stream_of(u))
    _lib.check(st, "ssla_diag_scan_fwd")
    return h


class SequentialScan(torch.autograd.Function):
    """Forward and backward of the varlen diagonal scan (reference
    ops/common/scan.py:89-137): saves g and h, and the backward kernel
    returns (du, dg) with zeros on rows in no sequence."""

    @staticmethod
    def forward(ctx, u, g, cu_seqlens):
        h = _scan_fwd(u, g, cu_seqlens)
        ctx.save_for_backward(g, h, cu_seqlens)
        return h

    @staticmethod
    def backward(ctx, dout):
        g, h, cu = ctx.saved_tensors
        dout = dout.to(torch.float32).contiguous()
        T, C = h.shape
        du, dg = torch.empty_like(h), torch.empty_like(h)
        st = _lib.load().ssla_diag_scan_bwd(_lib.ptr(dout), _lib.ptr(g), _lib.ptr(h), _lib.ptr(cu), cu.numel() - 1,
                                            T, C, _lib.ptr(du), _lib.ptr(dg), _lib.stream_of(h))
        _lib.check(st, "ssla_diag_scan_bwd")
        return du, dg, None


def scan(u: torch.Tensor, g: torch.Tensor, cu_seqlens: torch.Tensor) -> torch.Tensor:
    """Varlen diagonal scan; u, g ``[T, C]`` -> h ``[T, C]`` in u's dtype
    (reference ops/common/scan.py:101, ``torch.zeros_like(u)``; rows in no
    sequence are zero).  The running state is fp32 and each stored row is
    rounded once to u's dtype, as the reference kernel's fp32 ``b_h`` is
    (scan.py:35-43).  Differentiable in u and g (``ssla_diag_scan_bwd``)."""
    if u.dim() != 2 or u.shape != g.shape:
        raise ValueError(f"scan: u and g must both be [T, C], got {tuple(u.shape)}, {tuple(g.shape)}")
    dev = _lib.require_cuda(u, g)
    out_dtype = u.dtype
    u = u.to(torch.float32).contiguous()
    g = g.to(torch.float32).contiguous()
    cu = cu_seqlens.to(device=dev, dtype=torch.int64).contiguous()
    if torch.is_grad_enabled() and (u.requires_grad or g.requires_grad):
        h = SequentialScan.apply(u, g, cu)
    else:
        h = _scan_fwd(u, g, cu)
    return h if out_dtype == torch.float32 else h.to(out_dtype)


def sparse_gla_step(site_idx: torch.Tensor, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                    g: torch.Tensor, state: torch.Tensor, scale: Optional[float] = None,
                    check: bool = False) -> torch.Tensor:
    """Update ``state[site_idx]`` in place for one time bin and return o.

    site_idx: int32 ``[n]`` (strictly increasing, inside ``[0, n_sites)``);
    q, k, g: fp32 ``[n, H, K]``; v: fp32 ``[n, H, V]``; state: fp32
    ``[n_sites, H, K, V]``.  Rows of inactive sites are neither read nor
    written.  An entry out of range or not above the one before it is
    skipped (its o rows are zero, no state changes).  ``check=True`` reads
    the status word back after the call (one host sync) and raises
    ValueError for such an entry; the default makes no host sync, so a
    caller stepping through many bins pays none.
    """
    n, H, K = q.shape
    V = v.shape[-1]
    if k.shape != q.shape or g.shape != q.shape or v.shape[:2] != (n, H):
        raise ValueError("sparse_gla_step: q, k, g must be [n, H, K] and v [n, H, V]")
    if state.dim() != 4 or state.shape[1:] != (H, K, V) or state.dtype != torch.float32:
        raise ValueError(f"sparse_gla_step: state must be fp32 [n_sites, {H}, {K}, {V}]")
    if not state.is_contiguous():
        raise ValueError("sparse_gla_step: state must be contiguous (it is updated in place)")
    if site_idx.shape != (n,):
        raise ValueError("sparse_gla_step: site_idx must be [n]")
    _lib.require_cuda(site_idx, q, k, v, g, state)
    _lib.require_no_grad("sparse_gla_step", q, k, v, g, state)
    if scale is None:
        scale = K ** -0.5
    sidx = site_idx.to(torch.int32).contiguous()
    q, k, v, g = (t.to(torch.float32).contiguous() for t in (q, k, v, g))
    o = torch.empty(n, H, V, device=q.device, dtype=torch.float32)
    lib = _lib.load()
    status = _lib.new_status(q.device) if check and n else None
    st = lib.ssla_sparse_gla_step(_lib.ptr(sidx), n, _lib.ptr(q), _lib.ptr(k), _lib.ptr(v),
                                  _lib.ptr(g), _lib.ptr(state), state.shape[0], H, K, V,
                                  float(scale), _lib.ptr(o), _lib.ptr(status), _lib.stream_of(q))
    _lib.check(st, "ssla_sparse_gla_step")
    if status is not None and _lib.read_status(status) != _lib.SSLA_OK:
        raise ValueError(f"sparse_gla_step: site_idx must be strictly increasing and inside [0, {state.shape[0]})")
    return o


def sparse_gla_scan(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, g: torch.Tensor,
                    cu_seqlens: torch.Tensor, seq_site: torch.Tensor, state: torch.Tensor,
                    scale: Optional[float] = None, check: bool = False) -> torch.Tensor:
    """Many bins at once: sequence n (rows ``cu_seqlens[n]:cu_seqlens[n+1]``,
    ordered in time) is the history of site ``seq_site[n]``; its state row
    is read from and written back to ``state`` in place.  Returns o with
    q's dtype.  ``seq_site`` must be strictly increasing and inside
    ``[0, n_sites)``; a sequence whose entry is not is skipped (zero o rows,
    state untouched); ``check=True`` reads the status back after the call
    (one host sync) and raises ValueError for such a sequence."""
    T, H, K = q.shape
    V = v.shape[-1]
    if state.dim() != 4 or state.shape[1:] != (H, K, V) or state.dtype != torch.float32 \
            or not state.is_contiguous():
        raise ValueError(f"sparse_gla_scan: state must be contiguous fp32 [n_sites, {H}, {K}, {V}]")
    dev = _lib.require_cuda(q, k, v, g, state, seq_site)
    _lib.require_no_grad("sparse_gla_scan", q, k, v, g, state)
    if scale is None:
        scale = K ** -0.5
    cu = cu_seqlens.to(device=dev, dtype=torch.int64).contiguous()
    sidx = seq_site.to(device=dev, dtype=torch.int32).contiguous()
    if sidx.numel() != cu.numel() - 1:
        raise ValueError("sparse_gla_scan: seq_site needs one entry per sequence")
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    g = g.to(torch.float32).contiguous() if g.dtype != q.dtype else g.contiguous()
    o = torch.empty(T, H, V, device=q.device, dtype=q.dtype)
    status = _lib.new_status(dev) if check and sidx.numel() else None
    _recurrent(q, k, v, g, cu, float(scale), state, o, state, sidx, state.shape[0], status)
    if status is not None and _lib.read_status(status) != _lib.SSLA_OK:
        raise ValueError(f"sparse_gla_scan: seq_site must be strictly increasing and inside [0, {state.shape[0]})")
    return o
