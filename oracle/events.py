"""CPU oracle of the event-glue rows -- TEST INFRASTRUCTURE ONLY.

numpy restatements of the reference's event grouping, receptive-field /
patch scatter-gather, truncation, temporal dropout and sparse pooling
(haohq19/ssla).  Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg may use this module, and only as the
checker.  Each function names the reference code it restates; all of them
are pinned against the vectors in ``tests/golden/event_fixtures.npz``, which
the reference's own functions produced (``tests/test_oracle_events.py``).

Ordering conventions (pinned by the fixtures): every sort is stable, so
ties keep the order in which the items were enumerated.
"""
from __future__ import annotations

import math

import numpy as np


def _stable_argsort(key):
    return np.argsort(np.asarray(key), kind="stable")


# --------------------------------------------------------------- grouping --
def group_events(events, lengths, frame_size, max_events_per_px=512):
    """utils/farsecnn_utils.py:130-174 (and the identical utils/async_utils.py:10-84).

    events [B, N, C>=4] (x, y, t, features...), lengths [B].  Events of a
    pixel are kept in input order and only the latest ``max_events_per_px``
    survive.  Returns dict(events, time, batch_id, h, w, lengths, batch_size)."""
    ev = np.asarray(events, dtype=np.float32)
    lengths = np.asarray(lengths, dtype=np.int64)
    B, N, _ = ev.shape
    H, W = frame_size
    rows = [ev[b, : int(lengths[b])] for b in range(B)]
    flat = np.concatenate(rows, axis=0) if rows else np.zeros((0, ev.shape[2]), np.float32)
    bid = np.repeat(np.arange(B), lengths)
    # the reference forms the id in float arithmetic (exact below 2^24)
    pid = (bid * (H * W)).astype(np.float32) + flat[:, 1] * np.float32(W) + flat[:, 0]
    order = _stable_argsort(pid)
    spid = pid[order]
    head = np.ones(spid.shape[0], bool)
    head[1:] = spid[1:] != spid[:-1]
    starts = np.flatnonzero(head)
    lens = np.diff(np.append(starts, spid.shape[0]))
    kept = np.minimum(lens, max_events_per_px)
    drop = lens - kept
    keep_idx = np.concatenate([np.arange(s + d, s + l) for s, d, l in zip(starts, drop, lens)]) \
        if starts.size else np.zeros(0, np.int64)
    sev = flat[order]
    first = sev[starts]
    return {
        "events": sev[keep_idx, 3:],
        "time": sev[keep_idx, 2].astype(np.int64),
        "batch_id": bid[order][starts].astype(np.int64),
        "h": first[:, 1].astype(np.int64),
        "w": first[:, 0].astype(np.int64),
        "lengths": kept.astype(np.int64),
        "batch_size": B,
    }


# ------------------------------------------------------------ lookup tables --
def padding_1d(in_size, kernel_size, stride):
    """'same' padding: ceil(in/stride) outputs (utils/farsecnn_utils.py:78-84)."""
    return (math.ceil(in_size / stride) - 1) * stride + kernel_size - in_size


def rf2pixels(frame_size, kernel_size, stride):
    """utils/farsecnn_utils.py:95-128 / utils/async_utils.py:96-122: for each
    receptive field (row-major over the output grid) the pixel index of each
    kernel coordinate (row-major), -1 for padding; and the <x, y> output
    coordinate of each field."""
    H, W = frame_size
    kh, kw = kernel_size
    sh, sw = stride
    ph, pw = padding_1d(H, kh, sh), padding_1d(W, kw, sw)
    top, left = math.floor(ph / 2), math.floor(pw / 2)
    Ho = (H + ph - kh) // sh + 1
    Wo = (W + pw - kw) // sw + 1
    oy, ox, ky, kx = np.meshgrid(np.arange(Ho), np.arange(Wo), np.arange(kh), np.arange(kw), indexing="ij")
    y = oy * sh - top + ky
    x = ox * sw - left + kx
    lut = np.where((y >= 0) & (y < H) & (x >= 0) & (x < W), y * W + x, -1).reshape(Ho * Wo, kh * kw)
    oyy, oxx = np.meshgrid(np.arange(Ho), np.arange(Wo), indexing="ij")
    outc = np.stack([oxx.reshape(-1), oyy.reshape(-1)], axis=1)
    return lut.astype(np.int64), outc.astype(np.int64)


# ------------------------------------------------- RF / patch scatter-gather --
def _rf_scatter(gr, frame_size, lut):
    """Shared core of gather_receptive_fields (utils/farsecnn_utils.py:177-265)
    and scatter_group_events_to_patch (utils/async_utils.py:125-240).

    Fields (b, rf) in order; a field is active when one of its pixels holds a
    group.  Its events are the runs of its active pixels in kernel-coordinate
    order, then stably sorted by time.  Returns per-output-event source index
    (into the pixel events), time, kernel position, and per active field its
    (b, rf) and event count."""
    H, W = frame_size
    B = gr["batch_size"]
    n_rf, A = lut.shape
    gid = np.asarray(gr["batch_id"]) * (H * W) + np.asarray(gr["h"]) * W + np.asarray(gr["w"])
    lens = np.asarray(gr["lengths"], np.int64)
    starts = np.concatenate([[0], np.cumsum(lens)[:-1]]) if lens.size else np.zeros(0, np.int64)
    pix2g = {int(p): g for g, p in enumerate(gid)}
    time = np.asarray(gr["time"], np.int64)
    src, tim, pos, rf_b, rf_i, rf_len = [], [], [], [], [], []
    for b in range(B):
        for r in range(n_rf):
            n0 = len(src)
            for a in range(A):
                p = int(lut[r, a])
                if p < 0:
                    continue
                g = pix2g.get(b * H * W + p)
                if g is None:
                    continue
                idx = np.arange(starts[g], starts[g] + lens[g])
                src.extend(idx.tolist())
                tim.extend(time[idx].tolist())
                pos.extend([a] * idx.size)
            if len(src) > n0 or any(pix2g.get(b * H * W + int(p)) is not None for p in lut[r] if p >= 0):
                rf_b.append(b)
                rf_i.append(r)
                rf_len.append(len(src) - n0)
    src, tim, pos = np.array(src, np.int64), np.array(tim, np.int64), np.array(pos, np.int64)
    rf_len = np.array(rf_len, np.int64)
    field = np.repeat(np.arange(rf_len.size), rf_len)
    stride = (tim.max() + 1) if tim.size else 1
    order = _stable_argsort(tim + field * stride)
    return src[order], tim[order], pos[order], np.array(rf_b, np.int64), np.array(rf_i, np.int64), rf_len


def gather_receptive_fields(gr, frame_size, lut, outcoord):
    """utils/farsecnn_utils.py:177-265."""
    src, tim, pos, rf_b, rf_i, rf_len = _rf_scatter(gr, frame_size, lut)
    ev = np.asarray(gr["events"])
    return {"events": ev[src], "time": tim, "pos_id": pos, "lengths": rf_len,
            "h": outcoord[rf_i, 1], "w": outcoord[rf_i, 0], "batch_id": rf_b, "batch_size": gr["batch_size"]}


def scatter_group_events_to_patch(gr, frame_size, lut):
    """utils/async_utils.py:125-240."""
    src, tim, pos, rf_b, rf_i, rf_len = _rf_scatter(gr, frame_size, lut)
    ev = np.asarray(gr["events"])
    return {"events": ev[src], "pos_id": pos, "lengths": rf_len, "batch_size": gr["batch_size"],
            "orig_event_idx": src}


def gather_patch_events_to_group(patch_events, orig_event_idx, num_pixel_events):
    """utils/async_utils.py:243-264: zeros + index_add_ (fp32, in index order)."""
    pe = np.asarray(patch_events, np.float32)
    out = np.zeros((num_pixel_events, pe.shape[1]), np.float32)
    for i, p in enumerate(np.asarray(orig_event_idx)):
        out[p] += pe[i]
    return out


# ---------------------------------------------------------------- A25 glue --
def truncate_packed_sequence(data, seqlens, threshold, others=None):
    """utils/farsecnn_utils.py:8-33: keep the first `threshold` of each sequence."""
    seqlens = np.asarray(seqlens, np.int64)
    intra = np.concatenate([np.arange(n) for n in seqlens]) if seqlens.size else np.zeros(0, np.int64)
    mask = intra < threshold
    res = (np.asarray(data)[mask], np.minimum(seqlens, threshold))
    if others is not None:
        res = res + (np.asarray(others)[mask],)
    return res


def temporal_dropout_index(lengths, window_size):
    """layers/temporal_dropout.py:30-53: per sequence keep ceil(len / w) events,
    every w-th one, aligned so that the last event is kept."""
    lengths = np.asarray(lengths, np.int64)
    starts = np.concatenate([[0], np.cumsum(lengths)[:-1]]) if lengths.size else np.zeros(0, np.int64)
    keep_len = -(-lengths // window_size)
    idx = []
    for s, n, k in zip(starts, lengths, keep_len):
        off = (n % window_size - 1) % window_size
        idx.extend((s + off + window_size * np.arange(k)).tolist())
    return np.array(idx, np.int64), keep_len


def preprocess_events(events, lengths, frame_size, hot_pixel_thres=50):
    """model_mos.py:173-209: <x,y,t,p> -> <x,y,t,t,p>, group by pixel, the
    duplicated t becomes the per-pixel delay (clamped at 1e5 us, normalised
    to [0, 1], 1 for the first event of each pixel), then hot pixels are
    truncated to their first `hot_pixel_thres` events."""
    ev = np.asarray(events, np.float32)
    ev = np.concatenate([ev[..., :3], ev[..., 2:3], ev[..., 3:]], axis=-1)
    gr = group_events(ev, lengths, frame_size)
    ts = gr["events"][:, 0].copy()
    d = ts.copy()
    d[1:] = ts[1:] - ts[:-1]
    d = np.minimum(d / np.float32(1e5), np.float32(1.0)).astype(np.float32)
    starts = np.concatenate([[0], np.cumsum(gr["lengths"])[:-1]]).astype(np.int64)
    d[starts] = 1.0
    gr["events"] = gr["events"].copy()
    gr["events"][:, 0] = d
    if hot_pixel_thres > 0:
        gr["events"], gr["lengths"], gr["time"] = truncate_packed_sequence(
            gr["events"], gr["lengths"], hot_pixel_thres, others=gr["time"])
    return gr


def event_to_grid(gr, grid_size, channels):
    """model_mos.py:212-228: the last event of every group, placed at its
    (b, h, w) cell of a dense [B, C, H, W] grid (zeros elsewhere)."""
    Hg, Wg = grid_size
    B = gr["batch_size"]
    last = np.cumsum(gr["lengths"]) - 1
    grid = np.zeros((B * Hg * Wg, channels), np.float32)
    cell = gr["batch_id"] * Hg * Wg + gr["h"] * Wg + gr["w"]
    np.add.at(grid, cell, np.asarray(gr["events"])[last])
    return grid.reshape(B, Hg, Wg, channels).transpose(0, 3, 1, 2)


def sparse_pool(rf, reduce="max"):
    """layers/sparse_pooling.py:14-51 after gather_receptive_fields: events of
    one field with the same timestamp are reduced (torch_scatter max / mean
    over the unique_consecutive inverse); returns dict with events, time and
    per-field lengths."""
    lens = np.asarray(rf["lengths"], np.int64)
    field = np.repeat(np.arange(lens.size), lens)
    t = np.asarray(rf["time"], np.int64)
    stride = (t.max() + 1) if t.size else 1
    key = t + field * stride
    head = np.ones(key.size, bool)
    head[1:] = key[1:] != key[:-1]
    seg = np.cumsum(head) - 1
    n_seg = int(seg[-1]) + 1 if seg.size else 0
    ev = np.asarray(rf["events"], np.float32)
    out = np.zeros((n_seg, ev.shape[1]), np.float64 if reduce == "mean" else np.float32)
    if reduce == "max":
        out[:] = -np.inf
        np.maximum.at(out, seg, ev)
    else:
        np.add.at(out, seg, ev.astype(np.float64))
        out /= np.bincount(seg, minlength=n_seg)[:, None]
    new_t = key[head] - field[head] * stride
    new_len = np.bincount(field[head], minlength=lens.size) if lens.size else np.zeros(0, np.int64)
    new_len = new_len[new_len > 0]
    return {"events": out, "time": new_t, "lengths": new_len}


# ------------------------------------------------------------- ingestion --
def dat_decode(rec):
    """utils/io/dat_events_tools.py:40-47: raw Event2D records (t u4, w i4)
    -> dict of t, x, y, p arrays (x = w & 16383, y = (w & 268419072) >> 14,
    p = (w & 268435456) >> 28)."""
    rec = np.asarray(rec)
    w = rec["_"].astype(np.int64)
    return {"t": rec["t"].copy(), "x": w & 16383, "y": (w & 268419072) >> 14,
            "p": (w & 268435456) >> 28}


def pad_batches(samples, dataset="Gen1"):
    """model_base.py:82-117 on decoded samples (dicts or structured arrays
    with t, x, y, p): each sample stacked as float32 [t, x, y, p] rows
    (numpy astype rounding), zero-padded to the longest, then for Gen1 /
    NCaltech101 reordered to <x, y, t, p> with p -> 2p - 1 (padding rows
    included).  Returns (events [B, L, 4] float32, lengths [B])."""
    rows = [np.stack([np.asarray(s[f]).astype(np.float32) for f in ("t", "x", "y", "p")], axis=-1)
            for s in samples]
    lens = [len(r) for r in rows]
    L = max(lens)
    ev = np.stack([np.pad(r, ((0, L - n), (0, 0)), mode="constant", constant_values=0)
                   for n, r in zip(lens, rows)], axis=0)
    if dataset in ("Gen1", "NCaltech101"):
        ev = ev[:, :, [1, 2, 0, 3]]
        ev[:, :, -1] = ev[:, :, -1] * 2 - 1
    return ev, np.asarray(lens, np.int64)
