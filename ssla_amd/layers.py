"""SSLA layers on MI355X, with the reference's class names, constructor
arguments, parameter / buffer names and dict interface (haohq19/ssla):

* :class:`MosAttention`      layers/mos_attention.py:12-167
* :class:`LinearAttention`   layers/linear_attention.py:11-102
* :class:`AsyncSparseModule` layers/async_sparse_module.py:7-41
* :class:`SparsePool`, :class:`SparseMaxPool`, :class:`SparseAvgPool`,
  :class:`SparseAdaptiveMaxPool`, :class:`SparseAdaptiveAvgPool`
                             layers/sparse_pooling.py:8-103
* :class:`TemporalDropout`   layers/temporal_dropout.py:6-59

The event glue, the diagonal scan and the pooling run the gfx950 kernels of
libssla_amd.so; the dense projections are plain library GEMMs and the
normalisation a library LayerNorm.  The layers train: the scan, the row
gathers / ordered index-adds and the scatter reductions have backward
passes, so autograd runs through the composed MosAttention forward,
LinearAttention and the SparsePool family (the fused MosAttention forward is
inference only and is skipped whenever a gradient is recorded; so is the
two-call SparsePool, ssla_sparse_pool_plan / _emit, which pools straight
from the pixel events without storing the receptive-field rows).

Deviations, all deliberate: every ordering is stable (the reference's
unstable field sorts have implementation-defined tie order); SparsePool does
not shift the caller's ``time`` tensor in place; lookup tables are built on
the device at the first forward (their shapes are registered at
construction, so state dicts stay interchangeable).
"""
from __future__ import annotations

import ctypes
import math
from typing import Dict, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _lib
from . import events as E
from .scan import scan
from .scatter import scatter_max, scatter_mean

__all__ = ["MosAttention", "LinearAttention", "AsyncSparseModule", "SparsePool", "SparseMaxPool",
           "SparseAvgPool", "SparseAdaptiveMaxPool", "SparseAdaptiveAvgPool", "TemporalDropout"]


def _lut_shape(frame_size, kernel_size, stride):
    n = ctypes.c_int64(0)
    _lib.check(_lib.load().ssla_rf_lut_shape(int(frame_size[0]), int(frame_size[1]), int(kernel_size[0]),
                                             int(kernel_size[1]), int(stride[0]), int(stride[1]), ctypes.byref(n)),
               "rf_lut_shape")
    return int(n.value)


def _out_hw(frame_size, kernel_size, stride):
    """Output grid (rows, cols) of the field table: the field count of each
    axis alone (a 1-wide axis with a 1-wide kernel has one field)."""
    Ho = _lut_shape((frame_size[0], 1), (kernel_size[0], 1), (stride[0], 1))
    Wo = _lut_shape((1, frame_size[1]), (1, kernel_size[1]), (1, stride[1]))
    return Ho, Wo


def _ensure_lut(module, lut_name, outc_name, frame_size, kernel_size, stride, device):
    """Build the lookup tables on `device` with the HIP kernel (once)."""
    if getattr(module, "_lut_ready", None) == device:
        return
    lut, outc = E.compute_rf2pixels(frame_size, kernel_size, stride, device=device)
    getattr(module, lut_name).data = lut
    if outc_name is not None:
        getattr(module, outc_name).data = outc
    module._lut_ready = device


def _grouped_linear(x: torch.Tensor, pos: torch.Tensor, weights: torch.Tensor) -> torch.Tensor:
    """out[e] = weights[pos[e]] @ x[e]: rows bucketed by position with the
    stable device sort, one library GEMM per bucket, rows put back."""
    A = weights.shape[0]
    n = x.shape[0]
    out = torch.empty(n, weights.shape[1], device=x.device, dtype=torch.float32)
    if n == 0:
        return out
    _, perm = E.sort_pairs(pos, end_bit=max(1, (A - 1).bit_length()))
    counts = torch.bincount(pos, minlength=A).tolist()
    xs = E.gather_rows(x, perm)
    ys = torch.empty_like(out)
    o = 0
    for a, c in enumerate(counts):
        if c:
            ys[o:o + c] = F.linear(xs[o:o + c], weights[a])
            o += c
    out.index_copy_(0, perm, ys)
    return out


# ---------------------------------------------------------------- attention --
class MosAttention(nn.Module):
    """Mixture-of-sparse (patch) linear attention layer; reference
    layers/mos_attention.py:12-167.  forward(dict) -> dict with the keys of
    group_events."""

    def __init__(self, input_size: int, hidden_size: int, frame_size: Tuple[int, int],
                 kernel_size: Tuple[int, int], stride: Tuple[int, int] = (1, 1), scatter_proj: bool = True,
                 gather_proj: bool = True):
        super().__init__()
        self.input_size = input_size
        self.hidden_size = hidden_size
        self.frame_size = tuple(frame_size)
        self.frame_output_size = tuple(frame_size)
        self.kernel_size = tuple(kernel_size)
        self.stride = tuple(stride)
        self.scatter_proj = scatter_proj
        self.gather_proj = gather_proj
        n_coords = self.kernel_size[0] * self.kernel_size[1]
        self.register_parameter("scatter_conv_weights", nn.Parameter(
            torch.zeros(n_coords if scatter_proj else 1, input_size * hidden_size)))
        self.register_parameter("gather_conv_weights", nn.Parameter(
            torch.zeros(n_coords if gather_proj else 1, hidden_size * hidden_size)))
        std = math.sqrt(2.0 / (input_size + hidden_size))   # Xavier, as the reference
        with torch.no_grad():
            self.scatter_conv_weights.normal_(0, std)
            self.gather_conv_weights.normal_(0, std)
        self.q_proj = nn.Linear(hidden_size, hidden_size, bias=False)
        self.v_proj = nn.Linear(hidden_size, hidden_size, bias=False)
        self.g_proj = nn.Linear(hidden_size, hidden_size, bias=False)
        self.o_proj = nn.Linear(hidden_size, hidden_size, bias=False)
        self.norm = nn.LayerNorm(hidden_size)
        n_patch = _lut_shape(self.frame_size, self.kernel_size, self.stride)
        self.register_buffer("patch2pixel_lut", torch.full((n_patch, n_coords), -1, dtype=torch.int64))
        self.register_buffer("patch_outcoord", torch.zeros(n_patch, 2, dtype=torch.int))
        self.input_proj = nn.Linear(input_size, hidden_size, bias=False) if input_size != hidden_size else None

    def _project(self, x, pos, weights, enabled, in_size):
        w = weights.reshape(-1, self.hidden_size, in_size)
        if not enabled:
            return F.linear(x, w[0])
        return _grouped_linear(x, pos, w)

    def _fused_ok(self, events):
        """The fused forward (ssla_mos_attention_fwd) runs when no gradient is
        recorded, the kernel has at most 49 positions and the sizes fit one of
        its paths: input and hidden <= 32 with the weights within 64 KB of LDS,
        or input and hidden multiples of 4 up to 128 (matrix cores)."""
        if torch.is_grad_enabled() and (events.requires_grad or any(p.requires_grad for p in self.parameters())):
            return False
        A = self.kernel_size[0] * self.kernel_size[1]
        if A > 49:
            return False
        lds = _lib.load().ssla_mos_attention_lds_bytes(self.input_size, self.hidden_size, A, int(self.scatter_proj),
                                                       int(self.gather_proj))
        return 0 < lds <= 64 * 1024

    def _forward_fused(self, inputs, dev):
        events = inputs["events"].to(torch.float32).contiguous()
        src, _tim, pos, _f_index, f_len, _n_rf = E._rf_scatter(inputs, self.frame_size, self.patch2pixel_lut)
        A = self.kernel_size[0] * self.kernel_size[1]
        n, R, P = events.shape[0], src.numel(), f_len.numel()
        lib = _lib.load()
        ws = E._ws(lib.ssla_mos_attention_workspace_size(n, self.input_size, self.hidden_size, A, R, P), dev)
        out = torch.empty(n, self.hidden_size, dtype=torch.float32, device=dev)
        f32 = lambda t: t.detach().to(torch.float32).contiguous()   # noqa: E731
        w = [f32(x) for x in (self.scatter_conv_weights, self.q_proj.weight, self.v_proj.weight, self.g_proj.weight,
                              self.o_proj.weight, self.gather_conv_weights, self.norm.weight, self.norm.bias)]
        w_in = f32(self.input_proj.weight) if self.input_proj is not None else None
        _lib.check(lib.ssla_mos_attention_fwd(
            _lib.ptr(events), n, self.input_size, _lib.ptr(src), _lib.ptr(pos), R, _lib.ptr(f_len), P, A,
            _lib.ptr(w[0]), int(self.scatter_proj), _lib.ptr(w[1]), _lib.ptr(w[2]), _lib.ptr(w[3]), _lib.ptr(w[4]),
            _lib.ptr(w[5]), int(self.gather_proj), _lib.ptr(w_in) if w_in is not None else None, _lib.ptr(w[6]),
            _lib.ptr(w[7]), float(self.norm.eps), self.hidden_size, _lib.ptr(out), _lib.ptr(ws), ws.numel(),
            _lib.stream_of(events)), "mos_attention_fwd")
        return out

    def forward(self, inputs, fused=None):
        """fused: None picks the fused forward whenever it applies; False
        forces the composed (differentiable) path; True requires the fused
        one (SslaError if it does not apply)."""
        events = inputs["events"]
        lengths = inputs["lengths"]
        dev = _lib.require_cuda(events, lengths)
        _ensure_lut(self, "patch2pixel_lut", None, self.frame_size, self.kernel_size, self.stride, dev)
        use_fused = self._fused_ok(events) if fused is None else bool(fused)
        if use_fused:
            if fused and not self._fused_ok(events):
                raise _lib.SslaError("fused MosAttention forward needs no grad, at most 49 kernel positions and input / "
                                     "hidden sizes <= 32 or multiples of 4 up to 128")
            out = self._forward_fused(inputs, dev)
            return {"events": out, "time": inputs["time"], "w": inputs["w"], "h": inputs["h"],
                    "batch_id": inputs["batch_id"], "lengths": lengths, "batch_size": inputs["batch_size"]}
        patch = E.scatter_group_events_to_patch(inputs, self.frame_size, self.patch2pixel_lut)
        p_len, p_ev, p_pos = patch["lengths"], patch["events"], patch["pos_id"]
        x = self._project(p_ev, p_pos, self.scatter_conv_weights, self.scatter_proj, self.input_size)
        qvg = F.linear(x, torch.cat([self.q_proj.weight, self.v_proj.weight, self.g_proj.weight], 0))
        q, v, g = qvg.split(self.hidden_size, dim=1)
        # empty patches add repeated offsets; the scan takes the distinct ones
        cu = torch.cat([torch.zeros(1, dtype=torch.int64, device=dev), torch.cumsum(p_len[p_len > 0], 0)])
        h = scan(v.contiguous(), torch.sigmoid(g).contiguous(), cu)
        o = self.o_proj(q * h)
        o = self._project(o, p_pos, self.gather_conv_weights, self.gather_proj, self.hidden_size)
        out = E.gather_patch_events_to_group(o, patch["orig_event_idx"], events.shape[0])
        residual = self.input_proj(events) if self.input_proj is not None else events
        out = self.norm(out + residual)
        return {"events": out, "time": inputs["time"], "w": inputs["w"], "h": inputs["h"],
                "batch_id": inputs["batch_id"], "lengths": lengths, "batch_size": inputs["batch_size"]}

    def compute_flops(self, inputs):
        """Analytic flop count of one forward on these inputs, term for term
        the reference's (layers/mos_attention.py:169-199): every pixel event
        is counted once per kernel position (k_h * k_w patch copies)."""
        n_group = int(inputs["events"].shape[0])
        n_patch = n_group * self.kernel_size[0] * self.kernel_size[1]
        hs, ins = self.hidden_size, self.input_size
        flops = n_patch * hs * (2 * ins - 1)            # scatter projection
        flops += 3 * n_patch * hs * (2 * hs - 1)        # q, v, g
        flops += n_patch * hs * 4                       # sigmoid
        flops += n_patch * hs * 2                       # h = g * h + u
        flops += n_patch * hs                           # q * h
        flops += n_patch * hs * (2 * hs - 1)            # output projection
        flops += n_patch * hs * (2 * hs - 1)            # gather projection
        flops += n_patch * hs                           # gather back (index_add)
        flops += n_group * hs * (2 * ins - 1) if self.input_proj is not None else 0
        flops += n_group * hs                           # residual
        flops += n_group * (8 * hs + 1)                 # layer norm
        return flops


class LinearAttention(nn.Module):
    """Per-sample linear attention over events ordered by time; reference
    layers/linear_attention.py:11-102."""

    def __init__(self, input_size: int, hidden_size: int, frame_size: Tuple[int, int]):
        super().__init__()
        self.input_size = input_size
        self.hidden_size = hidden_size
        self.frame_size = tuple(frame_size)
        self.frame_output_size = tuple(frame_size)
        self.q_proj = nn.Linear(hidden_size, hidden_size, bias=False)
        self.v_proj = nn.Linear(hidden_size, hidden_size, bias=False)
        self.g_proj = nn.Linear(hidden_size, hidden_size, bias=False)
        self.o_proj = nn.Linear(hidden_size, hidden_size, bias=False)
        self.norm = nn.LayerNorm(hidden_size)
        if input_size != hidden_size:
            self.input_proj = nn.Linear(input_size, hidden_size, bias=False)
            self.residual_proj = nn.Linear(input_size, hidden_size, bias=False)
        else:
            self.input_proj = None
            self.residual_proj = None

    def forward(self, inputs):
        x_in = inputs["events"]
        gr_time, gr_len, gr_b = inputs["time"], inputs["lengths"], inputs["batch_id"]
        B = int(inputs["batch_size"])
        dev = _lib.require_cuda(x_in, gr_time)
        x = self.input_proj(x_in) if self.input_proj is not None else x_in
        n = x.shape[0]
        ev_b = E.expand_segments(gr_b, gr_len, n)
        # (batch, time) order, ties in event order: one stable sort on the
        # composite key batch * span + (t - t_min)
        t_min, t_max = (int(v) for v in torch.aminmax(gr_time)) if n else (0, 0)
        span = t_max - t_min + 1
        if B * span >= 1 << 62:
            raise _lib.SslaError("LinearAttention: batch * time range exceeds the 62-bit sort key")
        key = ev_b * span + (gr_time.to(torch.int64) - t_min)
        _, sort_idx = E.sort_pairs(key, end_bit=max(1, (B * span).bit_length()))
        xs = E.gather_rows(x, sort_idx)
        lengths = torch.bincount(ev_b, minlength=B)
        cu = torch.cat([torch.zeros(1, dtype=torch.int64, device=dev), torch.cumsum(lengths[lengths > 0], 0)])
        qvg = F.linear(xs, torch.cat([self.q_proj.weight, self.v_proj.weight, self.g_proj.weight], 0))
        q, v, g = qvg.split(self.hidden_size, dim=1)
        h = scan(v.contiguous(), torch.sigmoid(g).contiguous(), cu)
        o = self.o_proj(q * h)
        out = torch.empty_like(o)
        out.index_copy_(0, sort_idx, o)
        residual = self.residual_proj(x_in) if self.residual_proj is not None else x_in
        out = self.norm(out + residual)
        return {"events": out, "time": gr_time, "w": inputs["w"], "h": inputs["h"], "batch_id": gr_b,
                "lengths": gr_len, "batch_size": B}

    def compute_flops(self, inputs):
        """Analytic flop count of one forward, with the terms of the
        reference (layers/linear_attention.py:105-124).  The reference
        method names two counts it never defines (``num_patch_events``,
        ``num_group_events``) and raises NameError; here both are the event
        count, since this layer scans every event once."""
        n = int(inputs["events"].shape[0])
        hs, ins = self.hidden_size, self.input_size
        flops = 3 * n * hs * (2 * hs - 1)               # q, v, g
        flops += n * hs * 4                             # sigmoid
        flops += n * hs * 2                             # h = g * h + u
        flops += n * hs                                 # q * h
        flops += n * hs * (2 * hs - 1)                  # output projection
        flops += n * hs * (2 * ins - 1) if self.input_proj is not None else 0
        flops += n * hs * (2 * ins - 1) if self.residual_proj is not None else 0
        flops += n * hs                                 # residual
        flops += n * (8 * hs + 1)                       # layer norm
        return flops


# ------------------------------------------------------------------ pooling --
class AsyncSparseModule(nn.Module):
    """Receptive-field plumbing shared by pooling and dropout; reference
    layers/async_sparse_module.py:7-41."""

    def __init__(self, frame_size, kernel_size=(1, 1), stride=(1, 1), max_events_per_rf=512):
        super().__init__()
        self.frame_size = tuple(frame_size)
        self.kernel_size = tuple(kernel_size)
        self.stride = tuple(stride)
        self.register_buffer("max_events_per_rf", torch.tensor(max_events_per_rf))
        n_rf = _lut_shape(self.frame_size, self.kernel_size, self.stride)
        self.register_buffer("rf2pixel_lut", torch.full((n_rf, self.kernel_size[0] * self.kernel_size[1]), -1,
                                                        dtype=torch.int64))
        self.register_buffer("rf_outcoord", torch.zeros(n_rf, 2, dtype=torch.int64))
        Ho, Wo = _out_hw(self.frame_size, self.kernel_size, self.stride)
        if Ho * Wo != n_rf:
            raise _lib.SslaError(f"rf table of {n_rf} fields is not {Ho} x {Wo}")
        self.frame_output_size = (Ho, Wo)

    def prepare_inputs(self, inputs, grouped_events):
        if not grouped_events:
            inputs = self.group_events(inputs)
        if not (self.kernel_size[0] == 1 and self.kernel_size[1] == 1 and self.stride[0] == 1 and self.stride[1] == 1):
            inputs = self.gather_receptive_fields(inputs)
        return inputs

    def group_events(self, inputs):
        with torch.no_grad():
            return E.group_events(inputs, self.frame_size)

    def gather_receptive_fields(self, inputs):
        dev = inputs["time"].device
        _ensure_lut(self, "rf2pixel_lut", "rf_outcoord", self.frame_size, self.kernel_size, self.stride, dev)
        return E.gather_receptive_fields(inputs, self.frame_size, self.rf2pixel_lut, self.rf_outcoord)

    def compute_flops(self, inputs, grouped_events=True):
        """Modules without a flop cost of their own count 0, as the
        reference's fallback does (layers/async_sparse_module.py:44-46)."""
        return 0


class SparsePool(AsyncSparseModule):
    """Pool the events of every receptive field that share a timestamp;
    reference layers/sparse_pooling.py:8-51."""

    def __init__(self, pool_func, *args, kernel_size=(1, 1), stride=None, **kwargs):
        stride = stride if stride else kernel_size
        super().__init__(*args, kernel_size=kernel_size, stride=stride, **kwargs)
        self.pool_func = pool_func

    def forward(self, inputs, grouped_events=True):
        if grouped_events and self._one_call(inputs):
            dev = inputs["time"].device
            _ensure_lut(self, "rf2pixel_lut", "rf_outcoord", self.frame_size, self.kernel_size, self.stride, dev)
            return E.sparse_pool(inputs, self.frame_size, self.rf2pixel_lut, self.rf_outcoord,
                                 mean=self.pool_func is scatter_mean, fields_per_pixel=self._fields_per_pixel())
        x = self.prepare_inputs(inputs, grouped_events)
        seg, seg_time, new_len = E.pool_segments(x["time"], x["lengths"])
        res = self.pool_func(x["events"], seg, dim=0, dim_size=int(seg_time.numel()), sorted_index=True)
        new_events = res[0] if isinstance(res, tuple) else res
        return {"events": new_events, "time": seg_time, "lengths": new_len, "batch_id": x["batch_id"],
                "h": x["h"], "w": x["w"], "batch_size": x["batch_size"]}

    def plan(self, inputs) -> "E.PoolPlan":
        """The structure half of forward (E.sparse_pool_plan) for grouped
        device inputs whose values come later: the pooled time, lengths,
        batch_id, h, w land in ``plan.structure``; ``apply_plan`` then pools
        the values.  Only for the one-call pooling (max or mean over a field
        larger than one pixel)."""
        if self.pool_func not in (scatter_max, scatter_mean) or (self.kernel_size == (1, 1)
                                                                 and self.stride == (1, 1)):
            raise ValueError("SparsePool.plan: needs max or mean pooling over fields larger than one pixel")
        dev = inputs["time"].device
        _ensure_lut(self, "rf2pixel_lut", "rf_outcoord", self.frame_size, self.kernel_size, self.stride, dev)
        return E.sparse_pool_plan(inputs, self.frame_size, self.rf2pixel_lut, self.rf_outcoord,
                                  fields_per_pixel=self._fields_per_pixel())

    def plan_enqueue(self, inputs) -> "E.PoolPlan":
        """``plan`` in two halves (E.sparse_pool_plan_enqueue): the plan's
        kernels and an asynchronous copy of its counts; ``plan_finish`` waits
        for the counts and emits the structure."""
        if self.pool_func not in (scatter_max, scatter_mean) or (self.kernel_size == (1, 1)
                                                                 and self.stride == (1, 1)):
            raise ValueError("SparsePool.plan: needs max or mean pooling over fields larger than one pixel")
        dev = inputs["time"].device
        _ensure_lut(self, "rf2pixel_lut", "rf_outcoord", self.frame_size, self.kernel_size, self.stride, dev)
        return E.sparse_pool_plan_enqueue(inputs, self.frame_size, self.rf2pixel_lut, self.rf_outcoord,
                                          fields_per_pixel=self._fields_per_pixel())

    @staticmethod
    def plan_finish(plan: "E.PoolPlan") -> "E.PoolPlan":
        return E.sparse_pool_plan_finish(plan)

    def apply_plan(self, plan: "E.PoolPlan", events: torch.Tensor) -> Dict[str, torch.Tensor]:
        """forward's output for the values ``events`` of the groups ``plan``
        was made from."""
        return {"events": E.sparse_pool_values(plan, events, mean=self.pool_func is scatter_mean),
                **plan.structure}

    def apply_plan_linear(self, plan: "E.PoolPlan", x: torch.Tensor,
                          weight_bf16: torch.Tensor) -> Dict[str, torch.Tensor]:
        """``apply_plan`` of ``F.linear(x.bfloat16(), weight_bf16).float()``
        (x fp32 [E, 2], weight bf16 [C, 2]) with the linear map folded into
        the pooling (E.sparse_pool_values_linear): bit-identical outputs."""
        return {"events": E.sparse_pool_values_linear(plan, x, weight_bf16, mean=self.pool_func is scatter_mean),
                **plan.structure}

    def _fields_per_pixel(self) -> int:
        return (-(-self.kernel_size[0] // self.stride[0])) * (-(-self.kernel_size[1] // self.stride[1]))

    def compute_flops(self, inputs, grouped_events=True, elementwise_agg_flops=0):
        """Flops of the aggregation (reference layers/sparse_pooling.py:53-70):
        every receptive-field event that joins another one of the same field
        and time costs ``elementwise_agg_flops`` per channel."""
        x = self.prepare_inputs(inputs, grouped_events)
        _seg, seg_time, _len = E.pool_segments(x["time"], x["lengths"])
        agg_n = int(x["time"].numel()) - int(seg_time.numel())
        return agg_n * int(x["events"].shape[-1]) * elementwise_agg_flops

    def _one_call(self, inputs) -> bool:
        """The two-call pooling (ssla_sparse_pool_plan / _emit) takes grouped
        fp32 device events with no gradient to record and a receptive field
        larger than one pixel (a 1 x 1 field pools the pixel groups as they
        are, without the gather)."""
        ev = inputs["events"]
        return (self.pool_func in (scatter_max, scatter_mean) and ev.is_cuda and ev.dim() == 2
                and ev.dtype == torch.float32 and not (torch.is_grad_enabled() and ev.requires_grad)
                and not (self.kernel_size == (1, 1) and self.stride == (1, 1)))


class SparseMaxPool(SparsePool):
    def __init__(self, *args, **kwargs):
        super().__init__(scatter_max, *args, **kwargs)

    def compute_flops(self, inputs, grouped_events=True):
        """One compare per aggregated channel (reference sparse_pooling.py:78-79)."""
        return super().compute_flops(inputs, grouped_events=grouped_events, elementwise_agg_flops=1)


class SparseAvgPool(SparsePool):
    def __init__(self, *args, **kwargs):
        super().__init__(scatter_mean, *args, **kwargs)

    def compute_flops(self, inputs, grouped_events=True):
        """An add and a divide per aggregated channel (reference sparse_pooling.py:86-87)."""
        return super().compute_flops(inputs, grouped_events=grouped_events, elementwise_agg_flops=2)


class SparseAdaptiveMaxPool(SparseMaxPool):
    def __init__(self, frame_size, output_size):
        if output_size[0] > frame_size[0] or output_size[1] > frame_size[1]:
            raise ValueError("SparseAdaptiveMaxPool cannot be used to unpool the input frame.")
        k = [math.ceil(frame_size[0] / output_size[0]), math.ceil(frame_size[1] / output_size[1])]
        super().__init__(frame_size, kernel_size=k)


class SparseAdaptiveAvgPool(SparseAvgPool):
    def __init__(self, frame_size, output_size):
        if output_size[0] > frame_size[0] or output_size[1] > frame_size[1]:
            raise ValueError("SparseAdaptiveMaxPool cannot be used to unpool the input frame.")
        k = [math.ceil(frame_size[0] / output_size[0]), math.ceil(frame_size[1] / output_size[1])]
        super().__init__(frame_size, kernel_size=k)


class TemporalDropout(AsyncSparseModule):
    """Keep every window_size-th event of each sequence (the last one always);
    reference layers/temporal_dropout.py:6-59."""

    def __init__(self, window_size, *args, **kwargs):
        super().__init__(*args, **kwargs)
        if window_size <= 0:
            raise ValueError("window_size must be greater than 0.")
        self.window_size = window_size

    def forward(self, inputs, grouped_events=True):
        x = self.prepare_inputs(inputs, grouped_events)
        idx, kl = E.temporal_dropout_index(x["lengths"], self.window_size, total=x["events"].shape[0])
        events = E.gather_rows(x["events"], idx)
        time = x["time"][idx]
        return {"events": events, "time": time, "lengths": kl, "batch_id": x["batch_id"], "h": x["h"], "w": x["w"],
                "batch_size": x["batch_size"]}
