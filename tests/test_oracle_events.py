"""Pins of the event-glue oracle (oracle/events.py) against golden vectors
that the reference's own functions wrote (tests/golden/make_event_fixtures.py
runs them in the build container) plus closed forms.  CPU only."""
from pathlib import Path

import numpy as np
import pytest

from oracle import events as OE

FIX = Path(__file__).resolve().parent / "golden" / "event_fixtures.npz"


@pytest.fixture(scope="module")
def fx():
    return np.load(FIX, allow_pickle=False)


def _grouped(fx, cap=512):
    return OE.group_events(fx["ge_events"], fx["ge_lengths"], tuple(fx["ge_frame"]), cap)


@pytest.mark.parametrize("tag", ["mos", "farse"])
@pytest.mark.parametrize("cap", [4, 512])
def test_group_events(fx, tag, cap):
    gr = _grouped(fx, cap)
    for key in ("events", "time", "batch_id", "h", "w", "lengths"):
        np.testing.assert_array_equal(gr[key], fx[f"ge_{tag}_{cap}_{key}"], err_msg=key)


@pytest.mark.parametrize("name", ["12x15_k3s1", "7x10_k3s2", "9x5_k2s2", "6x8_k5s3"])
def test_lookup_tables(fx, name):
    fh, fw = (int(v) for v in name.split("_")[0].split("x"))
    k, s = int(name.split("_")[1][1]), int(name.split("_")[1][3])
    lut, outc = OE.rf2pixels((fh, fw), (k, k), (s, s))
    np.testing.assert_array_equal(lut, fx[f"lut_{name}"])
    np.testing.assert_array_equal(lut, fx[f"rf2p_{name}"])
    np.testing.assert_array_equal(outc, fx[f"rfout_{name}"])


def test_lookup_table_closed_form():
    """Stride-1 'same' 3x3 fields are centred on every pixel, so pixel (y, x)
    lies in (#centres within 1 row) x (#centres within 1 column) fields and
    field (y, x) holds pixel (y + dy) * W + (x + dx) at position (dy+1)*3+dx+1."""
    H, W = 11, 13
    lut, outc = OE.rf2pixels((H, W), (3, 3), (1, 1))
    counts = np.bincount(lut[lut >= 0], minlength=H * W).reshape(H, W)
    ny = np.array([min(y + 1, H - 1) - max(y - 1, 0) + 1 for y in range(H)])
    nx = np.array([min(x + 1, W - 1) - max(x - 1, 0) + 1 for x in range(W)])
    np.testing.assert_array_equal(counts, ny[:, None] * nx[None, :])
    y, x = 5, 7
    r = y * W + x
    np.testing.assert_array_equal(outc[r], [x, y])
    for dy in (-1, 0, 1):
        for dx in (-1, 0, 1):
            assert lut[r, (dy + 1) * 3 + dx + 1] == (y + dy) * W + (x + dx)


def _same_up_to_ties(ours, raw, field_lengths, time):
    """Equal after reordering rows within each (field, time) tie group."""
    field = np.repeat(np.arange(len(field_lengths)), field_lengths)
    key = field * (int(time.max()) + 1) + time
    for k in np.unique(key):
        sel = key == k
        o = np.asarray(ours)[sel].reshape(sel.sum(), -1)
        r = np.asarray(raw)[sel].reshape(sel.sum(), -1)
        assert sorted(map(tuple, o.tolist())) == sorted(map(tuple, r.tolist()))


@pytest.mark.parametrize("ks", [3, 2])
def test_patch_scatter_gather(fx, ks):
    gr = _grouped(fx)
    gr["events"] = fx["sp_pix_events"]
    res = OE.scatter_group_events_to_patch(gr, tuple(fx["ge_frame"]), fx[f"sp_lut_k{ks}"])
    for key in ("events", "pos_id", "lengths", "orig_event_idx"):
        np.testing.assert_array_equal(res[key], fx[f"sps_k{ks}_{key}"], err_msg=key)
    # the reference as it runs (unstable sort): same rows within each tie group
    np.testing.assert_array_equal(res["lengths"], fx[f"sp_k{ks}_lengths"])
    t = np.asarray(_grouped(fx)["time"])[res["orig_event_idx"]]
    rows = np.column_stack([res["orig_event_idx"], res["pos_id"]])
    raw = np.column_stack([fx[f"sp_k{ks}_orig_event_idx"], fx[f"sp_k{ks}_pos_id"]])
    _same_up_to_ties(rows, raw, res["lengths"], t)
    out = OE.gather_patch_events_to_group(fx[f"sp_k{ks}_gather_in"], res["orig_event_idx"],
                                          fx["sp_pix_events"].shape[0])
    np.testing.assert_array_equal(out.view(np.uint32), fx[f"sps_k{ks}_gather_out"].view(np.uint32))
    raw = OE.gather_patch_events_to_group(fx[f"sp_k{ks}_gather_in"], fx[f"sp_k{ks}_orig_event_idx"],
                                          fx["sp_pix_events"].shape[0])
    np.testing.assert_array_equal(raw.view(np.uint32), fx[f"sp_k{ks}_gather_out"].view(np.uint32))


@pytest.mark.parametrize("k,s", [(2, 2), (3, 2)])
def test_gather_receptive_fields(fx, k, s):
    gr = _grouped(fx)
    gr["events"] = fx["sp_pix_events"]
    lut, outc = OE.rf2pixels(tuple(fx["ge_frame"]), (k, k), (s, s))
    res = OE.gather_receptive_fields(gr, tuple(fx["ge_frame"]), lut, outc)
    for key in ("events", "time", "pos_id", "lengths", "h", "w", "batch_id"):
        np.testing.assert_array_equal(res[key], fx[f"grfs_k{k}s{s}_{key}"], err_msg=key)
    rows = np.column_stack([res["events"], res["pos_id"]])
    raw = np.column_stack([fx[f"grf_k{k}s{s}_events"], fx[f"grf_k{k}s{s}_pos_id"]])
    _same_up_to_ties(rows, raw, res["lengths"], res["time"])


def test_truncate(fx):
    nd, nl, no = OE.truncate_packed_sequence(fx["tr_data"], fx["tr_seqlens"], 4, others=fx["tr_other"])
    np.testing.assert_array_equal(nd, fx["tr_new_data"])
    np.testing.assert_array_equal(nl, fx["tr_new_lengths"])
    np.testing.assert_array_equal(no, fx["tr_new_other"])


@pytest.mark.parametrize("w", [1, 3, 4])
def test_temporal_dropout(fx, w):
    idx, kl = OE.temporal_dropout_index(fx["td_in_lengths"], w)
    np.testing.assert_array_equal(kl, fx[f"td_w{w}_lengths"])
    np.testing.assert_array_equal(fx["td_in_time"][idx], fx[f"td_w{w}_time"])
    np.testing.assert_array_equal(fx["sp_pix_events"][idx], fx[f"td_w{w}_events"])


def test_temporal_dropout_keeps_last():
    """Closed form: the last event of every sequence survives."""
    lens = np.array([1, 2, 5, 7, 9])
    idx, _ = OE.temporal_dropout_index(lens, 3)
    ends = np.cumsum(lens) - 1
    assert set(ends.tolist()) <= set(idx.tolist())


def test_gla_fixture_matches_fp64_oracle(fx):
    """The reference's naive_gla_recurrent output vs the fp64 C oracle."""
    import oracle
    o, ht = oracle.gla_recurrent(fx["gla_q"], fx["gla_k"], fx["gla_v"], fx["gla_g"], fx["gla_cu"], 1.0,
                                 fx["gla_h0"], True)
    np.testing.assert_allclose(o, fx["gla_o"], rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(ht, fx["gla_ht"], rtol=1e-4, atol=1e-5)


def test_sparse_pool_brute_force():
    """Segment max/mean against a direct loop on a tiny field set."""
    rf = {"events": np.array([[1, 2], [3, 0], [2, 5], [7, 7], [0, 1]], np.float32),
          "time": np.array([4, 4, 6, 1, 1]), "lengths": np.array([3, 2])}
    r = OE.sparse_pool(rf, "max")
    np.testing.assert_array_equal(r["events"], [[3, 2], [2, 5], [7, 7]])
    np.testing.assert_array_equal(r["time"], [4, 6, 1])
    np.testing.assert_array_equal(r["lengths"], [2, 1])
    m = OE.sparse_pool(rf, "mean")
    np.testing.assert_allclose(m["events"], [[2, 1], [2, 5], [3.5, 4]])


def test_preprocess_delays_direct_loop(fx):
    """model_mos.py:173-209 restated event by event: within each pixel group
    (in time order) feature 0 becomes min((t - t_prev) / 1e5, 1), 1 for the
    first event of the group; hot pixels keep their first 50 events."""
    ev = fx["ge_events"][..., [0, 1, 2, 4]]          # <x, y, t, p>
    lens = fx["ge_lengths"]
    H, W = (int(v) for v in fx["ge_frame"])
    gr = OE.preprocess_events(ev, lens, (H, W), hot_pixel_thres=3)
    # direct loop over the padded input
    per_pix = {}
    for b in range(ev.shape[0]):
        for n in range(int(lens[b])):
            x, y, t, p = ev[b, n]
            per_pix.setdefault((b, int(y), int(x)), []).append((t, p))
    want = []
    for key in sorted(per_pix):
        prev = None
        for i, (t, p) in enumerate(per_pix[key][-512:]):
            d = 1.0 if prev is None else min((np.float32(t) - np.float32(prev)) / np.float32(1e5), 1.0)
            prev = t
            if i < 3:
                want.append((d, p))
    want = np.array(want, np.float32)
    np.testing.assert_allclose(gr["events"][:, 0], want[:, 0], rtol=1e-6)
    np.testing.assert_array_equal(gr["events"][:, 1], want[:, 1])
    assert int(np.sum(gr["lengths"])) == want.shape[0]


def test_event_to_grid_direct_loop():
    """model_mos.py:212-228: the last event of each group at its cell."""
    gr = {"events": np.arange(12, dtype=np.float32).reshape(6, 2), "lengths": np.array([2, 3, 1]),
          "batch_id": np.array([0, 1, 1]), "h": np.array([1, 0, 2]), "w": np.array([2, 1, 0]), "batch_size": 2}
    grid = OE.event_to_grid(gr, (3, 3), 2)
    want = np.zeros((2, 2, 3, 3), np.float32)
    want[0, :, 1, 2] = gr["events"][1]
    want[1, :, 0, 1] = gr["events"][4]
    want[1, :, 2, 0] = gr["events"][5]
    np.testing.assert_array_equal(grid, want)
