"""Event-stream glue of the SSLA path on MI355X.

Drop-ins for the reference's index pipelines (haohq19/ssla), with the same
names, arguments and dict keys, running the gfx950 kernels of
``csrc/events.hip`` through libssla_amd.so (no CPU or torch fallback):

* :func:`group_events`                  utils/farsecnn_utils.py:130-174, utils/async_utils.py:10-84
* :func:`compute_rf2pixels`             utils/farsecnn_utils.py:95-128
* :func:`get_patch2pixel_lut`           utils/async_utils.py:96-122
* :func:`gather_receptive_fields`       utils/farsecnn_utils.py:177-265
* :func:`scatter_group_events_to_patch` utils/async_utils.py:125-240
* :func:`gather_patch_events_to_group`  utils/async_utils.py:243-264
* :func:`truncate_packed_sequence`      utils/farsecnn_utils.py:8-33
* :func:`temporal_dropout_index`        layers/temporal_dropout.py:30-53
* :func:`pool_segments`                 layers/sparse_pooling.py:26-48
* :func:`events_to_grid`                model_mos.py:212-228 (``events_to_grids``: several levels)
* :func:`preprocess_inputs`             model_mos.py:173-209

Every ordering is stable (ties keep enumeration order).  The reference's
field sorts use ``torch.sort(stable=False)``, whose tie order is
implementation-defined; where it is stable the results are identical.
Calls with data-dependent output sizes synchronise once to read the counts
(the reference's boolean-mask indexing and ``.item()`` calls do the same).
"""
from __future__ import annotations

import ctypes
from typing import Dict, List, Optional, Tuple

import numpy as np
import torch

from . import _lib

__all__ = [
    "group_events", "compute_rf2pixels", "get_patch2pixel_lut", "gather_receptive_fields",
    "scatter_group_events_to_patch", "gather_patch_events_to_group", "truncate_packed_sequence",
    "temporal_dropout_index", "pool_segments", "events_to_grid", "events_to_grids", "preprocess_inputs",
    "gather_rows", "sort_pairs", "expand_segments", "GatherRows", "IndexAddRows", "sparse_pool",
    "sparse_pool_values_linear",
]


def _ws(nbytes: int, device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


def _counts(ws: torch.Tensor, n: int, stream: int, what: str, check_bad: bool = True):
    out = (ctypes.c_int64 * n)()
    bad = ctypes.c_int(0)
    _lib.check(_lib.load().ssla_events_counts(_lib.ptr(ws), out, n, ctypes.byref(bad), stream), what)
    if check_bad and bad.value:
        raise ValueError(f"{what}: input indices or coordinates out of range")
    return [int(v) for v in out]


# Counts of a data-dependent call sit at the head of its workspace: int64
# words from byte 0 and the input-error flag as an int32 at byte 256.
_HEAD_BYTES = 260


class _CountSlot:
    """Pinned host memory for one counts head (with int64 / int32 views)
    and the event that marks its copy."""
    __slots__ = ("host", "i64", "i32", "event")

    def __init__(self):
        self.host = torch.zeros(_HEAD_BYTES + 4, dtype=torch.uint8, pin_memory=True)
        arr = self.host.numpy()
        self.i64, self.i32 = arr.view(np.int64), arr.view(np.int32)
        self.event = torch.cuda.Event()


# per device index: slots whose counts were read, ready for another copy
_free_slots: Dict[int, list] = {}


class PendingCounts:
    """The counts of a data-dependent call on their way to host memory: a
    copy of the workspace head into pinned memory, queued on the current
    stream behind the call's kernels, and the event after it.  ``read``
    waits on that event only, so work queued after the copy keeps the
    device busy meanwhile; its pinned slot then serves later copies."""
    __slots__ = ("slot", "dev")

    def __init__(self, ws: torch.Tensor):
        if ws.numel() < _HEAD_BYTES:
            raise ValueError(f"PendingCounts: workspace of {ws.numel()} bytes holds no counts head")
        dev = ws.get_device()
        free = _free_slots.setdefault(dev, [])
        if free:
            slot = free.pop()
        else:
            with torch.cuda.device(dev):
                slot = _CountSlot()
        _lib.check(_lib.load().ssla_events_counts_async(ws.data_ptr(), slot.host.data_ptr(), _lib.stream_of(ws)),
                   "events_counts_async")
        if dev == torch.cuda.current_device():
            slot.event.record()
        else:
            slot.event.record(torch.cuda.current_stream(ws.device))
        self.slot, self.dev = slot, dev

    def read(self, n: int):
        """(counts[0..n), input-error flag) once the copy has landed."""
        slot = self.slot
        if slot is None:
            raise RuntimeError("PendingCounts.read: the counts were read already")
        slot.event.synchronize()
        out = slot.i64[:n].tolist(), int(slot.i32[64])
        self.slot = None
        _free_slots[self.dev].append(slot)
        return out


def _i64(t: torch.Tensor) -> torch.Tensor:
    if t.dtype is torch.int64 and t.is_contiguous():
        return t
    return t.to(torch.int64).contiguous()


# ------------------------------------------------------------------ tables --
def compute_rf2pixels(frame_size, kernel_size, stride, device=None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Receptive-field lookup table and output coordinates ('same' padding,
    -1 for padded positions); reference utils/farsecnn_utils.py:95-128."""
    lib = _lib.load()
    H, W = int(frame_size[0]), int(frame_size[1])
    kh, kw = int(kernel_size[0]), int(kernel_size[1])
    sh, sw = int(stride[0]), int(stride[1])
    n_rf = ctypes.c_int64(0)
    _lib.check(lib.ssla_rf_lut_shape(H, W, kh, kw, sh, sw, ctypes.byref(n_rf)), "rf_lut_shape")
    dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    lut = torch.empty(n_rf.value, kh * kw, dtype=torch.int64, device=dev)
    outc = torch.empty(n_rf.value, 2, dtype=torch.int64, device=dev)
    _lib.check(lib.ssla_rf_lut(H, W, kh, kw, sh, sw, _lib.ptr(lut), _lib.ptr(outc), _lib.stream_of(lut)), "rf_lut")
    return lut, outc


def get_patch2pixel_lut(frame_size, kernel_size, stride, device=None) -> torch.Tensor:
    """Patch lookup table; reference utils/async_utils.py:96-122."""
    return compute_rf2pixels(frame_size, kernel_size, stride, device)[0]


# ---------------------------------------------------------------- grouping --
def group_events(inputs, frame_size, max_events_per_px: int = 512) -> Dict[str, torch.Tensor]:
    """Group padded events by pixel (reference utils/farsecnn_utils.py:130-174).

    inputs = (events [B, N, C>=4] with x, y, t, features..., lengths [B]).
    Returns dict(events, time, batch_id, h, w, lengths, batch_size)."""
    if not (isinstance(inputs, tuple) and len(inputs) == 2):
        raise ValueError("inputs should be a tuple of (events, lengths)")
    events, lengths = inputs
    if events.dim() != 3 or events.size(2) < 4:
        raise ValueError("events should be a (B, N, C) tensor with C >= 4")
    if lengths.dim() != 1 or lengths.size(0) != events.size(0):
        raise ValueError("lengths should be a (B,) tensor")
    dev = _lib.require_cuda(events, lengths)
    ev = events.to(torch.float32).contiguous()
    ln = _i64(lengths)
    B, N, C = ev.shape
    H, W = int(frame_size[0]), int(frame_size[1])
    lib = _lib.load()
    cap = B * N
    ws = _ws(lib.ssla_group_events_workspace_size(B, N), dev)
    out_ev = torch.empty(cap, C - 3, dtype=torch.float32, device=dev)
    out_t = torch.empty(cap, dtype=torch.int64, device=dev)
    gb, gh, gw, gl = (torch.empty(cap, dtype=torch.int64, device=dev) for _ in range(4))
    st = _lib.stream_of(ev)
    _lib.check(lib.ssla_group_events(_lib.ptr(ev), _lib.ptr(ln), B, N, C, H, W, int(max_events_per_px),
                                     _lib.ptr(out_ev), _lib.ptr(out_t), _lib.ptr(gb), _lib.ptr(gh), _lib.ptr(gw),
                                     _lib.ptr(gl), _lib.ptr(ws), ws.numel(), st), "group_events")
    G, E, _ = _counts(ws, 3, st, "group_events")
    return {"events": out_ev[:E], "time": out_t[:E], "batch_id": gb[:G], "h": gh[:G], "w": gw[:G],
            "lengths": gl[:G], "batch_size": B}


# ------------------------------------------------- fields / patches ----------
def _rf_scatter(inputs, frame_size, lut, force_sort=False, dst_map=False):
    """Field / patch rows of the pixel groups: (src, time, pos, f_index, f_len,
    n_rf[, dst]).  Pixel runs sorted by time (the plan counts the others)
    take the sort-free fill; force_sort=True always takes the radix-sort
    fill (the general path).  dst_map=True also returns the row of every
    (event, kernel position) pair ([E_in * A] int32, -1 if none; sort-free
    fill only, else None)."""
    lib = _lib.load()
    gb, gh, gw, gl = (_i64(inputs[k]) for k in ("batch_id", "h", "w", "lengths"))
    time = _i64(inputs["time"])
    dev = _lib.require_cuda(gb, gl, time, lut)
    B = int(inputs["batch_size"])
    H, W = int(frame_size[0]), int(frame_size[1])
    lut = _i64(lut)
    n_rf, A = lut.shape
    G, E_in = gl.numel(), time.numel()
    E_cap = A * E_in
    ws = _ws(lib.ssla_rf_scatter_workspace_size(G, B, H, W, n_rf, E_cap), dev)
    st = _lib.stream_of(time)
    _lib.check(lib.ssla_rf_scatter_plan(_lib.ptr(gb), _lib.ptr(gh), _lib.ptr(gw), _lib.ptr(gl), G, _lib.ptr(time),
                                        E_in, B, H, W, _lib.ptr(lut), n_rf, A, E_cap, _lib.ptr(ws), ws.numel(), st),
               "rf_scatter_plan")
    n_act, E_out, t_max, n_unsorted = _counts(ws, 4, st, "rf_scatter_plan")
    src = torch.empty(E_out, dtype=torch.int64, device=dev)
    tim = torch.empty(E_out, dtype=torch.int64, device=dev)
    pos = torch.empty(E_out, dtype=torch.int64, device=dev)
    f_index = torch.empty(n_act, dtype=torch.int64, device=dev)
    f_len = torch.empty(n_act, dtype=torch.int64, device=dev)
    dst = None
    if n_unsorted == 0 and not force_sort:
        inv = torch.empty(H * W * A, dtype=torch.int32, device=dev)
        dst = torch.empty(E_in * A, dtype=torch.int32, device=dev) if dst_map else None
        _lib.check(lib.ssla_rf_scatter_fill_sorted(
            _lib.ptr(gb), _lib.ptr(gh), _lib.ptr(gw), _lib.ptr(gl), G, _lib.ptr(time), E_in, B, H, W, _lib.ptr(lut),
            n_rf, A, E_cap, n_act, E_out, _lib.ptr(src), _lib.ptr(tim), _lib.ptr(pos), _lib.ptr(f_index),
            _lib.ptr(f_len), _lib.ptr(inv), _lib.ptr(dst), _lib.ptr(ws), ws.numel(), st),
            "rf_scatter_fill_sorted")
    else:
        _lib.check(lib.ssla_rf_scatter_fill(_lib.ptr(gl), G, _lib.ptr(time), E_in, B, H, W, _lib.ptr(lut), n_rf, A,
                                            E_cap, n_act, E_out, t_max, _lib.ptr(src), _lib.ptr(tim), _lib.ptr(pos),
                                            _lib.ptr(f_index), _lib.ptr(f_len), _lib.ptr(ws), ws.numel(), st),
                   "rf_scatter_fill")
    if dst_map:
        return src, tim, pos, f_index, f_len, n_rf, dst
    return src, tim, pos, f_index, f_len, n_rf


def _gather_rows(src: torch.Tensor, idx: torch.Tensor) -> torch.Tensor:
    C = src.shape[1] if src.dim() == 2 else 1
    out = torch.empty(idx.numel(), C, dtype=torch.float32, device=src.device)
    if idx.numel():
        _lib.check(_lib.load().ssla_gather_rows(_lib.ptr(src), src.shape[0], _lib.ptr(idx), idx.numel(), C,
                                                _lib.ptr(out), _lib.stream_of(src)), "gather_rows")
    return out


def _index_add_rows(src: torch.Tensor, idx: torch.Tensor, n_out: int) -> torch.Tensor:
    n, C = src.shape
    lib = _lib.load()
    ws = _ws(lib.ssla_index_add_rows_workspace_size(n), src.device)
    out = torch.empty(int(n_out), C, dtype=torch.float32, device=src.device)
    _lib.check(lib.ssla_index_add_rows(_lib.ptr(src), _lib.ptr(idx), n, C, int(n_out), _lib.ptr(out),
                                       _lib.ptr(ws), ws.numel(), _lib.stream_of(src)), "index_add_rows")
    return out


class GatherRows(torch.autograd.Function):
    """out = src[idx]; its backward sums the output gradient rows back into
    the source rows (the index_add kernel: ordered, deterministic)."""

    @staticmethod
    def forward(ctx, src, idx):
        ctx.save_for_backward(idx)
        ctx.n_src = src.shape[0]
        return _gather_rows(src, idx)

    @staticmethod
    def backward(ctx, dout):
        (idx,) = ctx.saved_tensors
        return _index_add_rows(dout.to(torch.float32).contiguous(), idx, ctx.n_src), None


class IndexAddRows(torch.autograd.Function):
    """out[r] = sum of src rows i with idx[i] == r; its backward gathers the
    output gradient rows (d src[i] = d out[idx[i]])."""

    @staticmethod
    def forward(ctx, src, idx, n_out):
        ctx.save_for_backward(idx)
        return _index_add_rows(src, idx, n_out)

    @staticmethod
    def backward(ctx, dout):
        (idx,) = ctx.saved_tensors
        return _gather_rows(dout.to(torch.float32).contiguous(), idx), None, None


def gather_rows(src: torch.Tensor, idx: torch.Tensor) -> torch.Tensor:
    """out[j] = src[idx[j]] for a 2-D fp32 src (the HIP row gather);
    differentiable in src."""
    src = src.to(torch.float32).contiguous()
    idx = _i64(idx)
    _lib.require_cuda(src, idx)
    if torch.is_grad_enabled() and src.requires_grad:
        return GatherRows.apply(src, idx)
    return _gather_rows(src, idx)


def gather_receptive_fields(inputs, frame_size, rf2pixel_lut, rf_outcoord) -> Dict[str, torch.Tensor]:
    """Pixel groups -> receptive-field sequences (reference
    utils/farsecnn_utils.py:177-265): dict(events, time, pos_id, lengths, h,
    w, batch_id, batch_size)."""
    src, tim, pos, f_index, f_len, n_rf = _rf_scatter(inputs, frame_size, rf2pixel_lut)
    ev = gather_rows(inputs["events"], src)
    rf = f_index % n_rf
    outc = _i64(rf_outcoord)
    return {"events": ev, "time": tim, "pos_id": pos, "lengths": f_len, "h": outc[rf, 1], "w": outc[rf, 0],
            "batch_id": f_index // n_rf, "batch_size": inputs["batch_size"]}


def scatter_group_events_to_patch(pixel_inputs, frame_size, patch2pixel_lut) -> Dict[str, torch.Tensor]:
    """Pixel groups -> patch sequences (reference utils/async_utils.py:125-240):
    dict(events, pos_id, lengths, batch_size, orig_event_idx)."""
    src, _tim, pos, _f_index, f_len, _ = _rf_scatter(pixel_inputs, frame_size, patch2pixel_lut)
    ev = gather_rows(pixel_inputs["events"], src)
    return {"events": ev, "pos_id": pos, "lengths": f_len, "batch_size": pixel_inputs["batch_size"],
            "orig_event_idx": src}


def gather_patch_events_to_group(patch_events: torch.Tensor, patch_event_to_pixel_event_idx: torch.Tensor,
                                 num_pixel_events: int) -> torch.Tensor:
    """Sum the patch copies of every pixel event (reference
    utils/async_utils.py:243-264); copies are added in increasing patch-event
    order from zero in fp32, as index_add_ does on the CPU."""
    pe = patch_events.to(torch.float32).contiguous()
    idx = _i64(patch_event_to_pixel_event_idx)
    _lib.require_cuda(pe, idx)
    if torch.is_grad_enabled() and pe.requires_grad:
        return IndexAddRows.apply(pe, idx, int(num_pixel_events))
    return _index_add_rows(pe, idx, int(num_pixel_events))


# ---------------------------------------------------------------- sequences --
def truncate_packed_sequence(data: torch.Tensor, seqlens: torch.Tensor, threshold: int,
                             others: Optional[torch.Tensor] = None):
    """Keep the first `threshold` rows of every packed sequence (reference
    utils/farsecnn_utils.py:8-33); returns (new_data, new_lengths[, new_others])."""
    d2 = data.to(torch.float32).reshape(data.shape[0], -1).contiguous()
    sl = _i64(seqlens)
    dev = _lib.require_cuda(d2, sl)
    E, C = d2.shape
    oth = None if others is None else _i64(others)
    lib = _lib.load()
    ws = _ws(lib.ssla_segments_workspace_size(sl.numel()), dev)
    out = torch.empty(E, max(C, 1), dtype=torch.float32, device=dev)
    out_l = torch.empty(sl.numel(), dtype=torch.int64, device=dev)
    out_o = None if oth is None else torch.empty(E, dtype=torch.int64, device=dev)
    st = _lib.stream_of(d2)
    _lib.check(lib.ssla_truncate_packed(_lib.ptr(d2), _lib.ptr(sl), sl.numel(), E, max(C, 1), int(threshold),
                                        _lib.ptr(oth), _lib.ptr(out), _lib.ptr(out_l), _lib.ptr(out_o), _lib.ptr(ws),
                                        ws.numel(), st), "truncate_packed")
    (n,) = _counts(ws, 1, st, "truncate_packed", check_bad=False)
    nd = out[:n].reshape((n,) + tuple(data.shape[1:])).to(data.dtype)
    if others is not None:
        return nd, out_l, out_o[:n].to(others.dtype)
    return nd, out_l


def temporal_dropout_index(lengths: torch.Tensor, window_size: int, total: Optional[int] = None):
    """Keep indices and new lengths of TemporalDropout (reference
    layers/temporal_dropout.py:30-53).  ``total`` is the number of rows the
    sequences index (the events tensor's rows): given, it sizes the output
    without reading sum(lengths) back from the device, and lengths that keep
    more rows than it allows raise ValueError."""
    ln = _i64(lengths)
    dev = _lib.require_cuda(ln)
    lib = _lib.load()
    ws = _ws(lib.ssla_segments_workspace_size(ln.numel()), dev)
    # capacity: sum(ceil(len / w)) <= sum(len) + n
    cap_t = (int(ln.sum().item()) if total is None else int(total)) + ln.numel()
    idx = torch.empty(max(cap_t, 1), dtype=torch.int64, device=dev)
    kl = torch.empty(ln.numel(), dtype=torch.int64, device=dev)
    st = _lib.stream_of(ln)
    _lib.check(lib.ssla_temporal_dropout_index(_lib.ptr(ln), ln.numel(), int(window_size), _lib.ptr(idx), cap_t,
                                               _lib.ptr(kl), _lib.ptr(ws), ws.numel(), st), "temporal_dropout_index")
    (n,) = _counts(ws, 1, st, "temporal_dropout_index", check_bad=False)
    if n > cap_t:
        raise ValueError(f"temporal_dropout_index: the lengths keep {n} rows, more than {cap_t} "
                         f"({total} rows and {ln.numel()} sequences) allow")
    return idx[:n], kl


def expand_segments(values: torch.Tensor, lengths: torch.Tensor, total: Optional[int] = None) -> torch.Tensor:
    """repeat_interleave(values, lengths) on the device."""
    v, ln = _i64(values), _i64(lengths)
    dev = _lib.require_cuda(v, ln)
    n = int(ln.sum().item()) if total is None else int(total)
    out = torch.empty(n, dtype=torch.int64, device=dev)
    lib = _lib.load()
    ws = _ws(lib.ssla_segments_workspace_size(ln.numel()), dev)
    _lib.check(lib.ssla_expand_segments(_lib.ptr(v), _lib.ptr(ln), ln.numel(), n, _lib.ptr(out), _lib.ptr(ws),
                                        ws.numel(), _lib.stream_of(v)), "expand_segments")
    return out


def sort_pairs(keys: torch.Tensor, end_bit: int = 64, values: Optional[torch.Tensor] = None):
    """Stable sort of uint64-valued keys (given as int64, non-negative);
    returns (sorted keys, permutation as int64)."""
    k = _i64(keys)
    dev = _lib.require_cuda(k)
    n = k.numel()
    lib = _lib.load()
    ws = _ws(lib.ssla_sort_pairs_workspace_size(n), dev)
    ko = torch.empty_like(k)
    vo = torch.empty(n, dtype=torch.int32, device=dev)
    vin = None if values is None else values.to(torch.int32).contiguous()
    _lib.check(lib.ssla_sort_pairs(_lib.ptr(k), _lib.ptr(vin), n, int(end_bit), _lib.ptr(ko), _lib.ptr(vo),
                                   _lib.ptr(ws), ws.numel(), _lib.stream_of(k)), "sort_pairs")
    return ko, vo.to(torch.int64)


def pool_segments(time: torch.Tensor, lengths: torch.Tensor):
    """SparsePool keys (reference layers/sparse_pooling.py:26-48): for
    field sequences laid out in order, the non-decreasing segment index of
    every event (events of a field with equal time share a segment), the
    time of every segment and the segment count of every field."""
    t, ln = _i64(time), _i64(lengths)
    dev = _lib.require_cuda(t, ln)
    E, n_f = t.numel(), ln.numel()
    lib = _lib.load()
    ws = _ws(lib.ssla_segments_workspace_size(max(n_f, E)), dev)
    field = torch.empty(max(E, 1), dtype=torch.int64, device=dev)
    seg = torch.empty(max(E, 1), dtype=torch.int64, device=dev)
    seg_t = torch.empty(max(E, 1), dtype=torch.int64, device=dev)
    seg_f = torch.empty(max(E, 1), dtype=torch.int64, device=dev)
    new_len = torch.empty(n_f, dtype=torch.int64, device=dev)
    st = _lib.stream_of(t)
    _lib.check(lib.ssla_pool_segments(_lib.ptr(t), _lib.ptr(ln), n_f, E, _lib.ptr(field), _lib.ptr(seg),
                                      _lib.ptr(seg_t), _lib.ptr(seg_f), _lib.ptr(new_len), _lib.ptr(ws), ws.numel(),
                                      st), "pool_segments")
    (n_seg,) = _counts(ws, 1, st, "pool_segments", check_bad=False)
    return seg[:E], seg_t[:n_seg], new_len


class PoolPlan:
    """A pooling plan (ssla_sparse_pool_plan) of one window's structure: the
    workspace that holds it, the call sizes, the counts and, once emitted,
    the pooled structure (time, lengths, batch_id, h, w, batch_size)."""
    __slots__ = ("ws", "sizes", "n_act", "n_seg", "E_out", "outc", "stream", "structure", "pending", "refs")

    def tensors(self):
        """The device tensors the plan holds (for Tensor.record_stream when
        another stream consumes it)."""
        return [self.ws, self.outc] + [v for v in self.structure.values() if isinstance(v, torch.Tensor)]


def _pool_plan_call(inputs, frame_size, rf2pixel_lut, rf_outcoord, fields_per_pixel,
                    enqueue_only: bool = False) -> PoolPlan:
    """ssla_sparse_pool_plan, or with ``enqueue_only`` its kernels alone and
    an asynchronous copy of the counts (finished by _pool_plan_finish)."""
    lib = _lib.load()
    gb, gh, gw, gl = (_i64(inputs[k]) for k in ("batch_id", "h", "w", "lengths"))
    time = _i64(inputs["time"])
    dev = _lib.require_cuda(gb, gl, time, rf2pixel_lut)
    B = int(inputs["batch_size"])
    H, W = int(frame_size[0]), int(frame_size[1])
    lut, outc = _i64(rf2pixel_lut), _i64(rf_outcoord)
    n_rf, A = lut.shape
    G, E_in = gl.numel(), time.numel()
    E_cap = E_in * min(A, int(fields_per_pixel) if fields_per_pixel else A)
    ws = _ws(lib.ssla_sparse_pool_workspace_size(G, E_in, B, H, W, n_rf, A, E_cap), dev)
    st = _lib.stream_of(time)
    plan = PoolPlan()
    plan.ws, plan.sizes, plan.outc, plan.stream = ws, (G, E_in, B, H, W, n_rf, A, E_cap), outc, st
    plan.structure = {"batch_size": inputs["batch_size"]}
    plan.pending, plan.refs = None, None
    if enqueue_only:
        _lib.check(lib.ssla_sparse_pool_plan_enqueue(_lib.ptr(gb), _lib.ptr(gh), _lib.ptr(gw), _lib.ptr(gl), G,
                                                     _lib.ptr(time), E_in, B, H, W, _lib.ptr(lut), n_rf, A, E_cap,
                                                     _lib.ptr(ws), ws.numel(), st), "sparse_pool_plan")
        plan.pending, plan.refs = PendingCounts(ws), (gl, time, lut)
        return plan
    cnt = (ctypes.c_int64 * 4)()
    _lib.check(lib.ssla_sparse_pool_plan(_lib.ptr(gb), _lib.ptr(gh), _lib.ptr(gw), _lib.ptr(gl), G, _lib.ptr(time),
                                         E_in, B, H, W, _lib.ptr(lut), n_rf, A, E_cap, cnt, _lib.ptr(ws), ws.numel(),
                                         st), "sparse_pool_plan")
    _pool_plan_counts(plan, cnt)
    return plan


def _pool_plan_counts(plan: PoolPlan, cnt):
    n_act, n_seg, E_out, bad = (int(v) for v in cnt)
    if bad:
        raise ValueError("sparse_pool: input indices or coordinates out of range")
    plan.n_act, plan.n_seg, plan.E_out = n_act, n_seg, E_out


def _pool_plan_finish(plan: PoolPlan):
    """The counts of an enqueued plan (waiting for their copy), checked by
    ssla_sparse_pool_plan_finish (which runs the sort fill when a pixel run
    was not sorted by time)."""
    head, bad = plan.pending.read(6)
    gl, time, lut = plan.refs
    G, E_in, B, H, W, n_rf, A, E_cap = plan.sizes
    hv = (ctypes.c_int64 * 6)(*head)
    cnt = (ctypes.c_int64 * 4)()
    _lib.check(_lib.load().ssla_sparse_pool_plan_finish(_lib.ptr(gl), G, _lib.ptr(time), E_in, B, H, W,
                                                       _lib.ptr(lut), n_rf, A, E_cap, hv, int(bad), cnt,
                                                       _lib.ptr(plan.ws), plan.ws.numel(), plan.stream),
               "sparse_pool_plan")
    plan.pending, plan.refs = None, None
    _pool_plan_counts(plan, cnt)


def _pool_emit(plan: PoolPlan, ev, mean, structure: bool):
    """One ssla_sparse_pool_emit call on the plan: the values when ``ev`` is
    given, the structure when ``structure``."""
    lib = _lib.load()
    G, E_in, B, H, W, n_rf, A, E_cap = plan.sizes
    dev = plan.ws.device
    out_ev = None
    if ev is not None:
        if ev.dim() != 2 or ev.dtype != torch.float32:
            raise TypeError("sparse_pool: events must be fp32 [E, C]")
        if ev.shape[0] != E_in:
            raise ValueError(f"sparse_pool: {ev.shape[0]} event rows for {E_in} times")
        ev = ev.contiguous()
        out_ev = torch.empty(plan.n_seg, ev.shape[1], dtype=torch.float32, device=dev)
    C = ev.shape[1] if ev is not None else 1
    out_t = fl = None
    if structure:
        out_t = torch.empty(plan.n_seg, dtype=torch.int64, device=dev)
        fl = torch.empty(4, plan.n_act, dtype=torch.int64, device=dev)
    P = _lib.ptr
    _lib.check(lib.ssla_sparse_pool_emit(P(ev), C, G, E_in, B, H, W, n_rf, A, E_cap, P(plan.outc),
                                         1 if mean else 0, plan.n_act, plan.n_seg, plan.E_out, P(out_ev), P(out_t),
                                         P(fl[0]) if fl is not None else None, P(fl[1]) if fl is not None else None,
                                         P(fl[2]) if fl is not None else None, P(fl[3]) if fl is not None else None,
                                         P(plan.ws), plan.ws.numel(), _lib.stream_of(plan.ws)), "sparse_pool_emit")
    if structure:
        plan.structure.update({"time": out_t, "lengths": fl[0], "batch_id": fl[1], "h": fl[2], "w": fl[3]})
    return out_ev


def sparse_pool_plan(inputs, frame_size, rf2pixel_lut, rf_outcoord,
                     fields_per_pixel: Optional[int] = None) -> PoolPlan:
    """The structure half of sparse_pool: the plan of the groups in
    ``inputs`` (batch_id, h, w, lengths, time, batch_size; no values needed)
    and the pooled structure, emitted into ``plan.structure``.  The values
    follow with sparse_pool_values on the same plan, so the structure of a
    window can be planned before the values that pass through it exist."""
    plan = _pool_plan_call(inputs, frame_size, rf2pixel_lut, rf_outcoord, fields_per_pixel)
    _pool_emit(plan, None, False, True)
    return plan


def sparse_pool_plan_enqueue(inputs, frame_size, rf2pixel_lut, rf_outcoord,
                             fields_per_pixel: Optional[int] = None) -> PoolPlan:
    """sparse_pool_plan in two halves: the plan's kernels and an
    asynchronous copy of its counts now, the counts and the structure in
    sparse_pool_plan_finish, so that work queued in between keeps the device
    busy while the host waits."""
    return _pool_plan_call(inputs, frame_size, rf2pixel_lut, rf_outcoord, fields_per_pixel, enqueue_only=True)


def sparse_pool_plan_finish(plan: PoolPlan) -> PoolPlan:
    _pool_plan_finish(plan)
    _pool_emit(plan, None, False, True)
    return plan


def sparse_pool_values(plan: PoolPlan, events: torch.Tensor, mean: bool = False) -> torch.Tensor:
    """The values half of sparse_pool on a plan from sparse_pool_plan:
    [segments, C] max (or mean) of every pooling segment."""
    return _pool_emit(plan, events, mean, False)


def sparse_pool_values_linear(plan: PoolPlan, x: torch.Tensor, weight_bf16: torch.Tensor,
                              mean: bool = False) -> torch.Tensor:
    """sparse_pool_values of ``F.linear(x.bfloat16(), weight_bf16).float()``
    without materialising the mapped events (ssla_sparse_pool_emit_linear):
    x fp32 [E, 2], weight_bf16 [C, 2] with C a multiple of 4; bit-identical
    to the two steps."""
    lib = _lib.load()
    G, E_in, B, H, W, n_rf, A, E_cap = plan.sizes
    dev = plan.ws.device
    if x.dim() != 2 or x.shape[1] != 2 or x.shape[0] != E_in:
        raise ValueError(f"sparse_pool_values_linear: x must be [{E_in}, 2], got {tuple(x.shape)}")
    if weight_bf16.dtype != torch.bfloat16 or weight_bf16.dim() != 2 or weight_bf16.shape[1] != 2:
        raise TypeError("sparse_pool_values_linear: weight must be bf16 [C, 2]")
    x = x.to(torch.float32).contiguous()
    w = weight_bf16.contiguous()
    C = w.shape[0]
    out = torch.empty(plan.n_seg, C, dtype=torch.float32, device=dev)
    _lib.check(lib.ssla_sparse_pool_emit_linear(_lib.ptr(x), 2, _lib.ptr(w), C, G, E_in, B, H, W, n_rf, A, E_cap,
                                                1 if mean else 0, plan.n_act, plan.n_seg, plan.E_out, _lib.ptr(out),
                                                _lib.ptr(plan.ws), plan.ws.numel(), _lib.stream_of(plan.ws)),
               "sparse_pool_emit_linear")
    return out


def sparse_pool(inputs, frame_size, rf2pixel_lut, rf_outcoord, mean: bool = False,
                fields_per_pixel: Optional[int] = None) -> Dict[str, torch.Tensor]:
    """SparsePool.forward on pixel groups (reference layers/sparse_pooling.py:
    14-48 after gather_receptive_fields) in two library calls, without
    gradient: the receptive-field rows are never stored as features.  The
    returned dict equals that of gather_receptive_fields -> pool_segments ->
    scatter_max / scatter_mean with a sorted index.  ``fields_per_pixel``
    bounds the fields one pixel belongs to (ceil(kh/sh) * ceil(kw/sw); the
    kernel positions when not given): it sizes the row capacity."""
    _lib.require_cuda(inputs["events"])
    plan = _pool_plan_call(inputs, frame_size, rf2pixel_lut, rf_outcoord, fields_per_pixel)
    out_ev = _pool_emit(plan, inputs["events"], mean, True)
    return {"events": out_ev, **plan.structure}


def events_to_grid(x: Dict[str, torch.Tensor], grid_size, channels: int) -> torch.Tensor:
    """The last event of every group at its cell of a dense [B, C, H, W]
    grid (reference model_mos.py:212-228)."""
    ev = x["events"].to(torch.float32).contiguous()
    ln, gb, gh, gw = (_i64(x[k]) for k in ("lengths", "batch_id", "h", "w"))
    dev = _lib.require_cuda(ev, ln)
    B = int(x["batch_size"])
    Hg, Wg = int(grid_size[0]), int(grid_size[1])
    if ev.shape[1] != channels:
        raise ValueError(f"events_to_grid: {ev.shape[1]} channels, expected {channels}")
    grid = torch.zeros(B, channels, Hg, Wg, dtype=torch.float32, device=dev)
    lib = _lib.load()
    ws = _ws(lib.ssla_segments_workspace_size(ln.numel()), dev)
    st = _lib.stream_of(ev)
    _lib.check(lib.ssla_events_to_grid(_lib.ptr(ev), ev.shape[0], channels, _lib.ptr(ln), _lib.ptr(gb),
                                       _lib.ptr(gh), _lib.ptr(gw), ln.numel(), B, Hg, Wg, _lib.ptr(grid),
                                       _lib.ptr(ws), ws.numel(), st), "events_to_grid")
    return grid


def events_to_grids(levels) -> List[torch.Tensor]:
    """``events_to_grid`` over several ``(x, grid_size, channels)`` levels of
    one batch in one launch (ssla_events_to_grids); each grid is written
    whole, so none is cleared first.  Levels with more than
    ``GRIDS_MAX_CELLS`` cells (B * Hg * Wg) go through ``events_to_grid``
    one by one."""
    if not levels:
        return []
    B = int(levels[0][0]["batch_size"])
    if len(levels) > _lib.GRIDS_MAX_LEVELS or any(
            B * int(gs[0]) * int(gs[1]) > _lib.GRIDS_MAX_CELLS or int(x["batch_size"]) != B for x, gs, _ in levels):
        return [events_to_grid(x, gs, c) for x, gs, c in levels]
    arr = (_lib.GridLevel * len(levels))()
    grids = []
    for i, (x, gs, c) in enumerate(levels):
        ev = x["events"].to(torch.float32).contiguous()
        ln, gb, gh, gw = (_i64(x[k]) for k in ("lengths", "batch_id", "h", "w"))
        dev = _lib.require_cuda(ev, ln)
        if ev.shape[1] != c:
            raise ValueError(f"events_to_grids: level {i} has {ev.shape[1]} channels, expected {c}")
        Hg, Wg = int(gs[0]), int(gs[1])
        grid = torch.empty(B, c, Hg, Wg, dtype=torch.float32, device=dev)
        arr[i] = _lib.GridLevel(_lib.ptr(ev), _lib.ptr(ln), _lib.ptr(gb), _lib.ptr(gh), _lib.ptr(gw), _lib.ptr(grid),
                                ev.shape[0], ln.numel(), c, Hg, Wg)
        grids.append(grid)
    _lib.check(_lib.load().ssla_events_to_grids(arr, len(levels), B, None, _lib.stream_of(grids[0])),
               "events_to_grids")
    return grids


def _preprocess_launch(events, lengths, frame_size, hot_pixel_thres, max_events_per_px: int = 512):
    """ssla_preprocess_events into capacity-sized outputs: (workspace,
    stream, outputs, batch size); the counts stay on the device."""
    ev = events.to(torch.float32).contiguous()
    ln = _i64(lengths)
    dev = _lib.require_cuda(ev, ln)
    B, N, C = ev.shape
    H, W = int(frame_size[0]), int(frame_size[1])
    lib = _lib.load()
    cap = B * N
    ws = _ws(lib.ssla_group_events_workspace_size(B, N), dev)
    out_ev = torch.empty(cap, C - 2, dtype=torch.float32, device=dev)
    out_t = torch.empty(cap, dtype=torch.int64, device=dev)
    grp = torch.empty(4, cap, dtype=torch.int64, device=dev)
    st = _lib.stream_of(ev)
    _lib.check(lib.ssla_preprocess_events(_lib.ptr(ev), _lib.ptr(ln), B, N, C, H, W, int(max_events_per_px),
                                          int(hot_pixel_thres), _lib.ptr(out_ev), _lib.ptr(out_t), _lib.ptr(grp[0]),
                                          _lib.ptr(grp[1]), _lib.ptr(grp[2]), _lib.ptr(grp[3]), _lib.ptr(ws),
                                          ws.numel(), st), "preprocess_events")
    return ws, st, (out_ev, out_t, grp), B


def _preprocess_result(outs, B, G: int, E: int):
    out_ev, out_t, grp = outs
    return {"events": out_ev[:E], "time": out_t[:E], "batch_id": grp[0, :G], "h": grp[1, :G], "w": grp[2, :G],
            "lengths": grp[3, :G], "batch_size": B}


def _preprocess_one_call(events, lengths, frame_size, hot_pixel_thres, max_events_per_px: int = 512):
    """preprocess_inputs as one library call (ssla_preprocess_events): the
    grouping, the delays and the truncation share one device pass and one
    read of the counts."""
    ws, st, outs, B = _preprocess_launch(events, lengths, frame_size, hot_pixel_thres, max_events_per_px)
    G, E, _ = _counts(ws, 3, st, "preprocess_events")
    return _preprocess_result(outs, B, G, E)


def preprocess_enqueue(events, lengths, frame_size, hot_pixel_thres: int = 50):
    """The first half of preprocess_inputs on a GPU (padded [B, N, >= 4]
    events): the library call and an asynchronous copy of its counts.
    preprocess_finish waits for the counts and returns what
    preprocess_inputs returns."""
    ws, _st, outs, B = _preprocess_launch(events, lengths, frame_size, hot_pixel_thres)
    return (PendingCounts(ws), ws, outs, B)


def preprocess_finish(pending) -> Dict[str, torch.Tensor]:
    counts, ws, outs, B = pending
    (G, E, _), bad = counts.read(3)
    if bad:
        raise ValueError("preprocess_events: input indices or coordinates out of range")
    return _preprocess_result(outs, B, G, E)


def preprocess_inputs(events: torch.Tensor, lengths: torch.Tensor, frame_size, hot_pixel_thres: int = 50):
    """MosModel.preprocess_inputs (reference model_mos.py:173-209):
    <x, y, t, p> -> grouped pixels with features <dt, p>, dt the per-pixel
    delay clamped at 100 ms and normalised to [0, 1] (1 for the first event
    of a pixel), hot pixels truncated to their first `hot_pixel_thres`."""
    if events.is_cuda and events.dim() == 3 and events.size(2) >= 4 and lengths.dim() == 1 \
            and lengths.size(0) == events.size(0):
        return _preprocess_one_call(events, lengths, frame_size, hot_pixel_thres)
    return _preprocess_composed(events, lengths, frame_size, hot_pixel_thres)


def _preprocess_composed(events, lengths, frame_size, hot_pixel_thres):
    """preprocess_inputs step by step: group_events of the duplicated-time
    layout, ssla_pixel_delays, truncate_packed_sequence."""
    ev = events.to(torch.float32)
    ev = torch.cat([ev[..., :3], ev[..., 2:3], ev[..., 3:]], dim=-1).contiguous()
    gr = group_events((ev, lengths), frame_size)
    feats = gr["events"]
    ln = gr["lengths"]
    lib = _lib.load()
    ws = _ws(lib.ssla_segments_workspace_size(ln.numel()), feats.device)
    _lib.check(lib.ssla_pixel_delays(_lib.ptr(feats), feats.shape[0], feats.shape[1], _lib.ptr(ln), ln.numel(),
                                     _lib.ptr(ws), ws.numel(), _lib.stream_of(feats)), "pixel_delays")
    if hot_pixel_thres > 0:
        gr["events"], gr["lengths"], gr["time"] = truncate_packed_sequence(
            gr["events"], gr["lengths"], threshold=hot_pixel_thres, others=gr["time"])
    return gr
