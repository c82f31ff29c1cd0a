"""Event ingestion from Prophesee ``.dat`` files, ending in the padded batch
tensor on the device.

Drop-ins with the reference's names and behaviour:

* :func:`parse_header`, :func:`count_events`, :func:`load_td_data`
  (utils/io/dat_events_tools.py:21-47, :122-183);
* :class:`PSEELoader` (utils/io/psee_loader.py:7-242) for ``.dat`` files: the
  same cursor (``seek_time`` / ``seek_event`` / ``load_delta_t`` /
  ``load_n_events`` / ``current_time`` / ``done``) over a memory-mapped file;
* :func:`pad_batches` (model_base.py:82-125): the collate step, with the
  record decode, float32 conversion, zero padding, column reorder and
  polarity map done by one gfx950 kernel (``ssla_dat_decode_batch``) that
  writes the batch tensor in place on the device.

The loaders' ``*_raw`` methods return the window as the file's own 8-byte
records (a zero-copy view of the memory map); that is what
:func:`pad_batches` uploads.  The decoded structured arrays the reference
returns are still available from the plain methods (decoded on the host,
as the reference does), so code written against the reference keeps
working.  Records are 8 bytes (``EV_TYPE``); a header that declares another
size is rejected (the reference would read such a file with 8-byte records
at ``ev_size`` strides).
"""
from __future__ import annotations

import os
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np
import torch

from . import _lib

__all__ = ["EV_TYPE", "EV_STRING", "DECODE_DTYPE", "parse_header", "count_events", "load_td_data",
           "decode_records", "PSEELoader", "pad_batches", "pad_events"]

EV_TYPE = [("t", "u4"), ("_", "i4")]   # Event2D record (dat_events_tools.py:15)
EV_STRING = "Event2D"
DECODE_DTYPE = [("t", "u4"), ("x", "u2"), ("y", "u2"), ("p", "u1")]   # psee_loader.py:33-38

_LAYOUTS = {"xytp": 0, "txyp": 1}


def parse_header(f) -> Tuple[int, int, int, Tuple[Optional[int], Optional[int]]]:
    """(position after the header, event type, event size, (height, width)),
    as dat_events_tools.parse_header (:136-183): header lines start with
    "% "; when there is at least one, two bytes (type, size) follow it."""
    f.seek(0, os.SEEK_SET)
    size = [None, None]
    n_comment = 0
    while True:
        bod = f.tell()
        line = f.readline()
        if line.decode("latin-1")[:2] != "% ":
            break
        words = line.split()
        if len(words) > 1:
            if words[1] == b"Height":
                size[0] = int(words[2])
            if words[1] == b"Width":
                size[1] = int(words[2])
        n_comment += 1
    f.seek(bod, os.SEEK_SET)
    if n_comment > 0:
        ev_type = int(np.frombuffer(f.read(1), dtype=np.uint8)[0])
        ev_size = int(np.frombuffer(f.read(1), dtype=np.uint8)[0])
    else:
        ev_type, ev_size = 0, 8
    return f.tell(), ev_type, ev_size, (size[0], size[1])


def count_events(filename: str) -> int:
    """Records after the header (dat_events_tools.py:122-133)."""
    with open(filename, "rb") as f:
        bod, _, ev_size, _ = parse_header(f)
        f.seek(0, os.SEEK_END)
        eod = f.tell()
    if ev_size == 0 or (eod - bod) % ev_size != 0:
        raise Exception("unexpected format !")
    return (eod - bod) // ev_size


def decode_records(rec: np.ndarray, dtype=DECODE_DTYPE) -> np.ndarray:
    """Structured array (t, x, y, p) of raw records, the reference's host
    decode (dat_events_tools.py:40-47, :93-103)."""
    out = np.empty(rec.shape[0], dtype=dtype)
    w = rec["_"]
    out["t"] = rec["t"]
    out["x"] = np.bitwise_and(w, 16383)
    out["y"] = np.right_shift(np.bitwise_and(w, 268419072), 14)
    out["p"] = np.right_shift(np.bitwise_and(w, 268435456), 28)
    return out


def _records(filename: str):
    with open(filename, "rb") as f:
        bod, ev_type, ev_size, size = parse_header(f)
    if ev_size != 8:
        raise ValueError(f"{filename}: event size {ev_size}, only 8-byte Event2D records are supported")
    n = (os.path.getsize(filename) - bod) // 8
    rec = np.memmap(filename, dtype=EV_TYPE, mode="r", offset=bod, shape=(n,)) if n > 0 \
        else np.empty(0, dtype=EV_TYPE)
    return rec, ev_type, size


def load_td_data(filename: str, ev_count: int = -1, ev_start: int = 0) -> np.ndarray:
    """Events [ev_start, ev_start + ev_count) as (t, x, y, p) with x, y, p
    int16 (dat_events_tools.py:21-47)."""
    rec, _, _ = _records(filename)
    lo = min(max(ev_start, 0), rec.shape[0])
    hi = rec.shape[0] if ev_count < 0 else min(rec.shape[0], lo + ev_count)
    return decode_records(rec[lo:hi], [("t", "u4"), ("x", "i2"), ("y", "i2"), ("p", "i2")])


class PSEELoader:
    """Cursor over the events of a ``.dat`` file (psee_loader.py:7-242).

    The cursor is an event index; every method moves it exactly as the
    reference moves its file position, including ``seek_time``'s binary
    search (an exact timestamp hit while more than ``term_criterion`` events
    remain leaves the cursor one event past the hit, :201-208)."""

    def __init__(self, datfile: str):
        ext = datfile.split(".")[-1]
        if ext != "dat":
            raise NotImplementedError(f"input file path = {datfile}: only .dat files are supported")
        self._rec, self.ev_type, self._size = _records(datfile)
        self._ev_size = 8
        self._ev_count = int(self._rec.shape[0])
        self._pos = 0
        self.done = False
        self.current_time = 0
        self.duration_s = self.total_time() * 1e-6

    # -- state ------------------------------------------------------------
    def reset(self):
        self._pos = 0
        self.done = False
        self.current_time = 0

    def event_count(self) -> int:
        return self._ev_count

    def get_size(self):
        return self._size

    def __repr__(self):
        return ("PSEELoader:\n-----------\n" + f"Event Type: {EV_STRING}\n" + f"Event Size: {self._ev_size} bytes\n"
                + f"Event Count: {self._ev_count}\n" + f"Duration: {self.duration_s} s \n" + "-----------\n")

    def _t(self, i: int) -> int:
        return int(self._rec["t"][i])

    # -- loads (raw records: a zero-copy view) -----------------------------
    def load_n_events_raw(self, ev_count: int) -> np.ndarray:
        """psee_loader.py:86-105."""
        pos = self._pos
        count = self._ev_count - pos
        if ev_count >= count:
            self.done = True
            ev_count = count
            out = self._rec[pos:pos + ev_count]
            self.current_time = int(out["t"][ev_count - 1]) + 1 if ev_count > 0 else self.current_time
            self._pos = pos + ev_count
        else:
            out = self._rec[pos:pos + ev_count]
            self.current_time = self._t(pos + ev_count)
            self._pos = pos + ev_count
        return out

    def load_delta_t_raw(self, delta_t: int) -> np.ndarray:
        """Events with current_time <= t < current_time + delta_t from the
        cursor on (psee_loader.py:107-150; t is assumed sorted, as the
        reference's final searchsorted assumes)."""
        if delta_t < 1:
            raise ValueError("load_delta_t(): delta_t must be at least 1 micro-second: {}".format(delta_t))
        if self.done or self._pos >= self._ev_count:
            self.done = True
            return self._rec[0:0]
        final_time = self.current_time + delta_t
        start = self._pos
        t = self._rec["t"]
        # buffers of 100000 events until one ends at or after final_time
        batch = 100000
        pos = start
        tmp_time = self.current_time
        while tmp_time < final_time and pos < self._ev_count:
            end = min(self._ev_count, pos + batch)
            tmp_time = int(t[end - 1])
            last_lo = pos
            pos = end
        if tmp_time >= final_time:
            self.current_time = final_time
        else:
            self.current_time = tmp_time + 1
        hi = last_lo + int(np.searchsorted(t[last_lo:pos], final_time))
        self._pos = hi
        self.done = self._pos >= self._ev_count
        return self._rec[start:hi]

    # -- decoded loads (the reference's return values) ---------------------
    def load_n_events(self, ev_count: int) -> np.ndarray:
        return decode_records(self.load_n_events_raw(ev_count))

    def load_delta_t(self, delta_t: int) -> np.ndarray:
        return decode_records(self.load_delta_t_raw(delta_t))

    # -- seeks ----------------------------------------------------------------
    def seek_event(self, ev_count: int):
        """psee_loader.py:152-176."""
        if ev_count <= 0:
            self._pos = 0
            self.current_time = 0
        elif ev_count >= self._ev_count:
            self._pos = self._ev_count
            self.current_time = self._t(self._ev_count - 1) + 1
        else:
            self._pos = ev_count
            self.current_time = self._t(ev_count)
        self.done = self._pos >= self._ev_count

    def seek_time(self, final_time: int, term_criterion: int = 100000):
        """psee_loader.py:178-215."""
        if final_time > self.total_time():
            self._pos = self._ev_count
            self.done = True
            self.current_time = self.total_time() + 1
            return
        if final_time <= 0:
            self.reset()
            return
        low, high = 0, self._ev_count
        while high - low > term_criterion:
            middle = (low + high) // 2
            self.seek_event(middle)
            mid = self._t(middle)
            self._pos = middle + 1   # the reference reads the event at the cursor
            if mid > final_time:
                high = middle
            elif mid < final_time:
                low = middle + 1
            else:
                self.current_time = final_time
                self.done = self._pos >= self._ev_count
                return
        self.seek_event(low)
        idx = int(np.searchsorted(self._rec["t"][low:high], final_time))
        self.seek_event(low + idx)
        self.current_time = final_time
        self.done = self._pos >= self._ev_count

    def total_time(self) -> int:
        """Last event's timestamp (psee_loader.py:217-238)."""
        if not self._ev_count:
            return 0
        return self._t(self._ev_count - 1)


def _as_records(a: np.ndarray) -> np.ndarray:
    if a.dtype.names == ("t", "_"):
        return np.ascontiguousarray(a)
    if a.dtype.names is not None and {"t", "x", "y", "p"} <= set(a.dtype.names):
        rec = np.empty(a.shape[0], dtype=EV_TYPE)   # re-pack decoded events (writer's formula)
        rec["t"] = a["t"]
        rec["_"] = (a["x"].astype(np.int32) + np.left_shift(a["y"].astype(np.int32), 14)
                    + np.left_shift(a["p"].astype(np.int32), 28))
        return rec
    raise TypeError("events must be raw .dat records (EV_TYPE) or a structured array with t, x, y, p")


def pad_events(samples: Sequence[np.ndarray], device, layout: str = "xytp") -> Tuple[torch.Tensor, torch.Tensor]:
    """(events float32 [B, L, 4] on ``device``, lengths int64 [B]) from the
    samples' records: the events half of pad_batches.  layout "xytp": rows
    (x, y, t, 2p - 1), padding rows (0, 0, 0, -1) (Gen1 / NCaltech101);
    "txyp": rows (t, x, y, p), padding rows 0."""
    if layout not in _LAYOUTS:
        raise ValueError(f"unknown layout {layout!r}")
    recs = [_as_records(s) for s in samples]
    lens = [int(r.shape[0]) for r in recs]
    B, L = len(recs), (max(lens) if recs else 0)
    dev = torch.device(device)
    if dev.type != "cuda":
        raise ValueError("pad_events decodes on the device: pass a GPU device")
    events = torch.empty((B, L, 4), dtype=torch.float32, device=dev)
    lengths = torch.as_tensor(lens, dtype=torch.int64)
    if B == 0 or L == 0:
        if events.numel():
            events.zero_()
        return events, lengths
    total = sum(lens)
    start = np.zeros(B + 1, dtype=np.int64)
    np.cumsum(lens, out=start[1:])
    # one pinned staging buffer: the records, then the start offsets
    host = torch.empty(total * 8 + (B + 1) * 8, dtype=torch.uint8, pin_memory=True)
    hv = host.numpy()
    off = 0
    for r in recs:
        nb = r.shape[0] * 8
        hv[off:off + nb] = r.view(np.uint8)
        off += nb
    hv[off:].view(np.int64)[:] = start
    # (torch keeps the pinned block alive until the asynchronous copy is done)
    dbuf = host.to(dev, non_blocking=True)
    lib = _lib.load()
    st = torch.cuda.current_stream(dev).cuda_stream
    _lib.check(lib.ssla_dat_decode_batch(dbuf.data_ptr(), total, dbuf.data_ptr() + total * 8, B, L,
                                         _LAYOUTS[layout], events.data_ptr(), st), "ssla_dat_decode_batch")
    return events, lengths


def pad_batches(data: List[Tuple[np.ndarray, np.ndarray]], dataset: str = "Gen1", device="cuda") -> Dict[str, torch.Tensor]:
    """model_base.py:82-125: ``data`` is a list of (events, labels) samples;
    events as raw records or the loaders' structured arrays.  Returns the
    reference's dict: events float32 [B, L, 4] (on ``device``; <x, y, t, p>
    with p in {-1, 1} for Gen1 / NCaltech101, else <t, x, y, p>), labels
    padded with zeros, lengths and labels_lengths (host)."""
    layout = "xytp" if dataset in ("Gen1", "NCaltech101") else "txyp"
    events, lengths = pad_events([s[0] for s in data], device, layout)
    labels = [np.asarray(s[1]) for s in data]
    labels_lens = [len(l) for l in labels]
    max_len = max(labels_lens)
    labels = [np.pad(lb, ((0, max_len - ln), (0, 0)), mode="constant", constant_values=0)
              for ln, lb in zip(labels_lens, labels)]
    return {"events": events, "labels": torch.as_tensor(np.stack(labels, axis=0)), "lengths": lengths,
            "labels_lengths": torch.as_tensor(labels_lens)}
