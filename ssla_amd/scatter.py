"""Scatter-reduce pooling on MI355X, drop-in for the two ``torch_scatter``
functions the reference imports (reference layers/sparse_pooling.py:5,33).

``scatter_max(src, index, dim=0, out=None, dim_size=None) -> (out, argmax)``
and ``scatter_mean(src, index, dim=0, out=None, dim_size=None) -> out``
reduce rows of a 2-D ``src [E, C]`` into ``[dim_size, C]`` by a per-row
index.  The index may be ``[E]`` or the ``[E, C]`` stride-0 broadcast
(``index.unsqueeze(1).expand(-1, C)``) that the reference passes.

Semantics (torch_scatter's documented behaviour): empty output rows are 0
(argmax = E); ``argmax`` picks the smallest event index among equal maxima
(deterministic, unlike atomic implementations); mean divides the sum by
``max(count, 1)``.

Both are differentiable in ``src`` as torch_scatter's are: the gradient of
``scatter_max`` goes to the winning event of every (row, channel) (none for
empty rows), that of ``scatter_mean`` is the row's gradient over its count.
``out=`` is not supported (torch_scatter reduces into the existing contents
of ``out``; the reference never passes it): it raises NotImplementedError.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _lib

__all__ = ["scatter_max", "scatter_mean"]


def _prep(name, src, index, dim, dim_size):
    if src.dim() == 1:
        src = src.unsqueeze(1)
        squeeze = True
    elif src.dim() == 2:
        squeeze = False
    else:
        raise NotImplementedError(f"{name}: only 1-D and 2-D src are supported")
    if dim not in (0, -src.dim() if not squeeze else -1) and not (squeeze and dim == -1):
        raise NotImplementedError(f"{name}: only dim=0 is supported")
    E, Cc = src.shape
    if index.dim() == 2:
        if index.shape != (E, Cc):
            raise ValueError(f"{name}: index shape {tuple(index.shape)} != src shape {(E, Cc)}")
        if Cc > 1 and index.stride(1) != 0:
            raise NotImplementedError(f"{name}: per-channel indices are not supported "
                                      "(pass the row index broadcast over channels)")
        index = index[:, 0]
    elif index.dim() != 1 or index.shape[0] != E:
        raise ValueError(f"{name}: index must be [E] or [E, C], got {tuple(index.shape)}")
    _lib.require_cuda(src, index)
    if src.dtype != torch.float32:
        raise TypeError(f"{name}: src must be fp32, got {src.dtype}")
    index = index.to(torch.int64).contiguous()
    if dim_size is None:
        dim_size = int(index.max().item()) + 1 if E > 0 else 0
    return src.contiguous(), index, int(dim_size), Cc, squeeze


def _run(name, fn, src, index, n_out, sorted_index, out, argmax, check):
    E, Cp = src.shape
    lib = _lib.load()
    ws_bytes = lib.ssla_scatter_workspace_size(E, Cp, n_out)
    ws = torch.empty(ws_bytes, device=src.device, dtype=torch.uint8)
    args = [_lib.ptr(src), _lib.ptr(index), E, Cp, n_out, 1 if sorted_index else 0, _lib.ptr(out)]
    if argmax is not None:
        args.append(_lib.ptr(argmax))
    args += [_lib.ptr(ws), ws_bytes, _lib.stream_of(src)]
    _lib.check(fn(*args), name)
    if check:
        import ctypes
        status = ctypes.c_int(0)
        _lib.check(lib.ssla_scatter_check(_lib.ptr(ws), ctypes.byref(status), _lib.stream_of(src)),
                   "ssla_scatter_check")
        if status.value != 0:
            raise ValueError(f"{name}: index out of range [0, {n_out})"
                             + (" or not sorted" if sorted_index else ""))


def _no_out(name, out):
    if out is not None:
        raise NotImplementedError(
            f"{name}: out= is not supported (torch_scatter would reduce into the existing contents of out); "
            "pass out=None and copy the result")


class _ScatterMax(torch.autograd.Function):
    @staticmethod
    def forward(ctx, src, idx, n_out, sorted_index, check):
        E, Cc = src.shape
        res = torch.empty(n_out, Cc, device=src.device, dtype=torch.float32)
        arg = torch.empty(n_out, Cc, device=src.device, dtype=torch.int64)
        _run("scatter_max", _lib.load().ssla_scatter_max, src, idx, n_out, sorted_index, res, arg, check)
        ctx.save_for_backward(arg)
        ctx.n_src = E
        ctx.mark_non_differentiable(arg)
        return res, arg

    @staticmethod
    def backward(ctx, d_out, _d_arg):
        (arg,) = ctx.saved_tensors
        grad = torch.zeros(ctx.n_src + 1, arg.shape[1], device=arg.device, dtype=d_out.dtype)
        grad.scatter_(0, arg, d_out.contiguous())   # argmax = E (empty row) lands in the dropped extra row
        return grad[:ctx.n_src], None, None, None, None


class _ScatterMean(torch.autograd.Function):
    @staticmethod
    def forward(ctx, src, idx, n_out, sorted_index, check):
        Cc = src.shape[1]
        res = torch.empty(n_out, Cc, device=src.device, dtype=torch.float32)
        _run("scatter_mean", _lib.load().ssla_scatter_mean, src, idx, n_out, sorted_index, res, None, check)
        ctx.save_for_backward(idx)
        ctx.n_out = n_out
        return res

    @staticmethod
    def backward(ctx, d_out):
        (idx,) = ctx.saved_tensors
        cnt = torch.bincount(idx, minlength=ctx.n_out).clamp_(min=1).to(d_out.dtype)
        return (d_out / cnt[:, None]).index_select(0, idx), None, None, None, None


def scatter_max(src: torch.Tensor, index: torch.Tensor, dim: int = -1,
                out: Optional[torch.Tensor] = None, dim_size: Optional[int] = None,
                sorted_index: bool = False, check: bool = True
                ) -> Tuple[torch.Tensor, torch.Tensor]:
    """Row-wise maximum and first-index argmax.  ``sorted_index=True``
    promises a non-decreasing index (e.g. a ``unique_consecutive`` inverse);
    ``check`` reports out-of-range (or unsorted) indices as ValueError."""
    _no_out("scatter_max", out)
    src_c, idx, n_out, _Cc, squeeze = _prep("scatter_max", src, index, dim, dim_size)
    res, arg = _ScatterMax.apply(src_c, idx, n_out, sorted_index, check)
    if squeeze:
        res, arg = res[:, 0], arg[:, 0]
    return res, arg


def scatter_mean(src: torch.Tensor, index: torch.Tensor, dim: int = -1,
                 out: Optional[torch.Tensor] = None, dim_size: Optional[int] = None,
                 sorted_index: bool = False, check: bool = True) -> torch.Tensor:
    """Row-wise mean (sum / max(count, 1))."""
    _no_out("scatter_mean", out)
    src_c, idx, n_out, _Cc, squeeze = _prep("scatter_mean", src, index, dim, dim_size)
    res = _ScatterMean.apply(src_c, idx, n_out, sorted_index, check)
    if squeeze:
        res = res[:, 0]
    return res
