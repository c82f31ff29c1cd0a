"""Writes Prophesee .dat files for the ingestion tests, in the format the
reference's writer produces (utils/io/dat_events_tools.py:186-222): "% "
header lines, then one byte event type and one byte event size, then 8-byte
records (uint32 t, int32 x + (y << 14) + (p << 28))."""
import numpy as np

EV_TYPE = [("t", "u4"), ("_", "i4")]


def encode(t, x, y, p):
    rec = np.empty(len(t), dtype=EV_TYPE)
    rec["t"] = np.asarray(t, np.uint32)
    rec["_"] = (np.asarray(x, np.int32) + np.left_shift(np.asarray(y, np.int32), 14)
                + np.left_shift(np.asarray(p, np.int32), 28))
    return rec


def write_dat(path, t, x, y, p, height=240, width=304, header=True):
    rec = encode(t, x, y, p)
    with open(path, "wb") as f:
        if header:
            f.write(b"% Data file containing Event2D events.\n% Version 2\n% Date 2020-01-01 00:00:00\n")
            f.write(("%% Height %d\n%% Width %d\n" % (height, width)).encode())
            f.write(np.array([0, 8], dtype=np.uint8).tobytes())
        f.write(rec.tobytes())
    return rec


def random_stream(n, seed=0, t_max=5_000_000, width=304, height=240, dup=True):
    """Sorted timestamps (with repeats when dup) and random pixels."""
    rng = np.random.default_rng(seed)
    t = np.sort(rng.integers(0, t_max, n)) if dup else np.sort(rng.choice(t_max, n, replace=False))
    x = rng.integers(0, width, n)
    y = rng.integers(0, height, n)
    p = rng.integers(0, 2, n)
    return t, x, y, p
