"""Ingestion on the host: .dat header and record format, the PSEELoader
cursor (reference utils/io/psee_loader.py), and the oracle of pad_batches
(model_base.py:82-117) pinned by hand-computed rows.  No GPU needed."""
import numpy as np
import pytest

import oracle.events as OE
from ssla_amd import io
from tests.dat_files import encode, random_stream, write_dat


# ----------------------------------------------------------- the oracle --
def test_oracle_pad_batches_known_rows():
    """Hand-computed rows: Gen1 order <x, y, t, 2p-1>; t = 2^24 + 1 rounds to
    2^24 in float32; padding rows become (0, 0, 0, -1)."""
    rec = encode([10, 2 ** 24 + 1], [3, 16383], [4, 16383], [1, 0])
    s0, s1 = OE.dat_decode(rec), OE.dat_decode(rec[:0])
    ev, lens = OE.pad_batches([s0, s1], "Gen1")
    want = np.array([[[3, 4, 10, 1], [16383, 16383, 16777216, -1]],
                     [[0, 0, 0, -1], [0, 0, 0, -1]]], np.float32)
    assert np.array_equal(ev, want) and list(lens) == [2, 0]
    ev2, _ = OE.pad_batches([s0, s1], "other")   # <t, x, y, p>, zero padding
    want2 = np.array([[[10, 3, 4, 1], [16777216, 16383, 16383, 0]], [[0, 0, 0, 0], [0, 0, 0, 0]]], np.float32)
    assert np.array_equal(ev2, want2)


def test_oracle_decode_inverts_the_writer():
    rng = np.random.default_rng(0)
    n = 5000
    t, x, y, p = (rng.integers(0, 2 ** 32, n, dtype=np.uint64), rng.integers(0, 16384, n),
                  rng.integers(0, 16384, n), rng.integers(0, 2, n))
    d = OE.dat_decode(encode(t, x, y, p))
    assert np.array_equal(d["t"], t) and np.array_equal(d["x"], x)
    assert np.array_equal(d["y"], y) and np.array_equal(d["p"], p)
    # the mirror's host decode agrees
    h = io.decode_records(encode(t, x, y, p))
    for f in "txyp":
        assert np.array_equal(h[f].astype(np.int64), np.asarray(d[f], np.int64))


# ---------------------------------------------------------------- files --
def test_parse_header_and_counts(tmp_path):
    f = tmp_path / "a.dat"
    t, x, y, p = random_stream(100, seed=1)
    write_dat(f, t, x, y, p, height=240, width=304)
    with open(f, "rb") as fh:
        bod, ev_type, ev_size, size = io.parse_header(fh)
    assert (ev_type, ev_size, size) == (0, 8, (240, 304))
    assert bod == f.stat().st_size - 100 * 8
    assert io.count_events(str(f)) == 100
    g = tmp_path / "b.dat"
    write_dat(g, t, x, y, p, header=False)   # no header: 8-byte records from byte 0
    with open(g, "rb") as fh:
        assert io.parse_header(fh) == (0, 0, 8, (None, None))
    d = io.load_td_data(str(f), ev_count=7, ev_start=20)
    assert list(d.dtype.names) == ["t", "x", "y", "p"] and d["x"].dtype == np.int16
    assert np.array_equal(d["t"], t[20:27]) and np.array_equal(d["x"], x[20:27])
    assert np.array_equal(io.load_td_data(str(f))["y"], y)
    assert io.load_td_data(str(f), ev_start=500).shape == (0,)


def test_other_record_size_rejected(tmp_path):
    f = tmp_path / "c.dat"
    with open(f, "wb") as fh:
        fh.write(b"% Version 2\n" + np.array([0, 12], np.uint8).tobytes() + bytes(24))
    with pytest.raises(ValueError):
        io.PSEELoader(str(f))
    with pytest.raises(NotImplementedError):
        io.PSEELoader(str(tmp_path / "c.npy"))


# --------------------------------------------------------------- cursor --
def _window(t, T, dt):
    """Events of the time window [T', T' + dt), T' = max(T, 0); none when T is
    past the last event (the loader's documented window semantics)."""
    if T > t[-1]:
        return np.zeros(0, np.int64)
    T = max(T, 0)
    return np.nonzero((t >= T) & (t < T + dt))[0]


@pytest.mark.parametrize("dup", [True, False])
def test_seek_time_then_load_delta_t_is_the_time_window(tmp_path, dup):
    f = tmp_path / "w.dat"
    t, x, y, p = random_stream(3000, seed=2, t_max=200_000, dup=dup)
    write_dat(f, t, x, y, p)
    ld = io.PSEELoader(str(f))
    assert ld.event_count() == 3000 and ld.total_time() == t[-1] and ld.get_size() == (240, 304)
    rng = np.random.default_rng(3)
    cases = [(-50, 1000), (0, 1), (int(t[0]), 10), (int(t[1234]), 5000), (int(t[-1]), 7), (int(t[-1]) + 1, 10)]
    cases += [(int(v), int(d)) for v, d in zip(rng.integers(-100, 210_000, 40), rng.integers(1, 50_000, 40))]
    for T, dt in cases:
        ld.seek_time(T)
        got = ld.load_delta_t_raw(dt)
        want = _window(t, T, dt)
        assert np.array_equal(got["t"], t[want]), (T, dt)
    # decoded form of the same window
    ld.seek_time(int(t[100]))
    d = ld.load_delta_t(1000)
    w = _window(t, int(t[100]), 1000)
    assert np.array_equal(d["x"], x[w]) and d["p"].dtype == np.uint8


def test_seek_time_exact_hit_skips_the_hit_event(tmp_path):
    """The reference's binary search returns on an exact timestamp hit with
    the file one event past it (psee_loader.py:196-208).  t = 10 i for 64
    events, term_criterion 4: the first probe is event 32 (t = 320)."""
    f = tmp_path / "q.dat"
    t = np.arange(64) * 10
    write_dat(f, t, np.zeros(64), np.zeros(64), np.zeros(64))
    ld = io.PSEELoader(str(f))
    ld.seek_time(320, term_criterion=4)
    assert ld.current_time == 320
    assert list(ld.load_delta_t_raw(25)["t"]) == [330, 340]
    ld.seek_time(325, term_criterion=4)   # no hit: first event at or after 325
    assert list(ld.load_delta_t_raw(25)["t"]) == [330, 340]
    ld.seek_time(320)                     # default criterion: plain search
    assert list(ld.load_delta_t_raw(25)["t"]) == [320, 330, 340]


def test_load_n_events_and_seek_event(tmp_path):
    f = tmp_path / "n.dat"
    t, x, y, p = random_stream(50, seed=4, t_max=1000)
    write_dat(f, t, x, y, p)
    ld = io.PSEELoader(str(f))
    a = ld.load_n_events(10)
    assert np.array_equal(a["t"], t[:10]) and ld.current_time == t[10] and not ld.done
    b = ld.load_n_events(100)
    assert np.array_equal(b["t"], t[10:]) and ld.done and ld.current_time == t[-1] + 1
    ld.seek_event(20)
    assert ld.current_time == t[20] and not ld.done
    assert np.array_equal(ld.load_n_events(1)["y"], y[20:21])
    ld.seek_event(10 ** 6)
    assert ld.done and ld.current_time == t[-1] + 1
    assert ld.load_delta_t_raw(5).shape == (0,)
    with pytest.raises(ValueError):
        ld.load_delta_t_raw(0)


def test_pad_events_needs_a_gpu_device():
    with pytest.raises(ValueError):
        io.pad_events([encode([1], [2], [3], [1])], "cpu")
