"""GPU parity of the event glue (csrc/events.hip via the C-ABI) against the
golden vectors the reference's own functions wrote
(tests/golden/event_fixtures.npz) and, at larger seeded sizes, against the
CPU oracle (oracle/events.py).  Integer outputs and gathered rows are
compared bit-exactly."""
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import events as OE

pytestmark = pytest.mark.gpu
FIX = Path(__file__).resolve().parent / "golden" / "event_fixtures.npz"


@pytest.fixture(scope="module")
def fx():
    return np.load(FIX, allow_pickle=False)


def _np(t):
    return t.detach().cpu().numpy()


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _grouped(fx, dev, cap=512):
    from ssla_amd import events as E
    return E.group_events((_t(fx["ge_events"], dev), _t(fx["ge_lengths"], dev)), tuple(int(v) for v in fx["ge_frame"]),
                          max_events_per_px=cap)


@pytest.mark.parametrize("cap", [4, 512])
def test_group_events_fixture(dev, fx, cap):
    gr = _grouped(fx, dev, cap)
    for key in ("events", "time", "batch_id", "h", "w", "lengths"):
        np.testing.assert_array_equal(_np(gr[key]), fx[f"ge_farse_{cap}_{key}"], err_msg=key)


@pytest.mark.parametrize("name", ["12x15_k3s1", "7x10_k3s2", "9x5_k2s2", "6x8_k5s3"])
def test_lut_fixture(dev, fx, name):
    from ssla_amd import events as E
    fh, fw = (int(v) for v in name.split("_")[0].split("x"))
    k, s = int(name.split("_")[1][1]), int(name.split("_")[1][3])
    lut, outc = E.compute_rf2pixels((fh, fw), (k, k), (s, s), device=dev)
    np.testing.assert_array_equal(_np(lut), fx[f"rf2p_{name}"])
    np.testing.assert_array_equal(_np(outc), fx[f"rfout_{name}"])


@pytest.mark.parametrize("ks", [3, 2])
def test_patch_scatter_gather_fixture(dev, fx, ks):
    from ssla_amd import events as E
    gr = _grouped(fx, dev)
    gr["events"] = _t(fx["sp_pix_events"], dev)
    frame = tuple(int(v) for v in fx["ge_frame"])
    lut = E.get_patch2pixel_lut(frame, (ks, ks), (1, 1), device=dev)
    res = E.scatter_group_events_to_patch(gr, frame, lut)
    for key in ("events", "pos_id", "lengths", "orig_event_idx"):
        np.testing.assert_array_equal(_np(res[key]), fx[f"sps_k{ks}_{key}"], err_msg=key)
    out = E.gather_patch_events_to_group(_t(fx[f"sp_k{ks}_gather_in"], dev), res["orig_event_idx"],
                                         fx["sp_pix_events"].shape[0])
    np.testing.assert_array_equal(_np(out).view(np.uint32), fx[f"sps_k{ks}_gather_out"].view(np.uint32))


@pytest.mark.parametrize("k,s", [(2, 2), (3, 2)])
def test_gather_receptive_fields_fixture(dev, fx, k, s):
    from ssla_amd import events as E
    gr = _grouped(fx, dev)
    gr["events"] = _t(fx["sp_pix_events"], dev)
    frame = tuple(int(v) for v in fx["ge_frame"])
    lut, outc = E.compute_rf2pixels(frame, (k, k), (s, s), device=dev)
    res = E.gather_receptive_fields(gr, frame, lut, outc)
    for key in ("events", "time", "pos_id", "lengths", "h", "w", "batch_id"):
        np.testing.assert_array_equal(_np(res[key]), fx[f"grfs_k{k}s{s}_{key}"], err_msg=key)


def test_truncate_and_dropout_fixture(dev, fx):
    from ssla_amd import events as E
    nd, nl, no = E.truncate_packed_sequence(_t(fx["tr_data"], dev), _t(fx["tr_seqlens"], dev), 4,
                                            others=_t(fx["tr_other"], dev))
    np.testing.assert_array_equal(_np(nd), fx["tr_new_data"])
    np.testing.assert_array_equal(_np(nl), fx["tr_new_lengths"])
    np.testing.assert_array_equal(_np(no), fx["tr_new_other"])
    for w in (1, 3, 4):
        idx, kl = E.temporal_dropout_index(_t(fx["td_in_lengths"], dev), w)
        np.testing.assert_array_equal(_np(kl), fx[f"td_w{w}_lengths"])
        np.testing.assert_array_equal(fx["td_in_time"][_np(idx)], fx[f"td_w{w}_time"])


def _synthetic(seed, B, N, H, W, dev):
    gen = np.random.default_rng(seed)
    ev = np.zeros((B, N, 4), np.float32)
    lens = gen.integers(N // 2, N + 1, B)
    for b in range(B):
        n = int(lens[b])
        cx, cy = gen.uniform(0, W, 5), gen.uniform(0, H, 5)
        c = gen.integers(0, 5, n)
        x = np.clip(np.round(cx[c] + gen.normal(0, 3, n)), 0, W - 1)
        y = np.clip(np.round(cy[c] + gen.normal(0, 3, n)), 0, H - 1)
        t = np.sort(gen.integers(0, 20000, n)).astype(np.float32)
        ev[b, :n] = np.stack([x, y, t, np.where(gen.random(n) < 0.5, -1.0, 1.0)], 1)
    return ev, lens


def test_preprocess_and_fields_synthetic(dev):
    """Larger seeded window (2 samples, 64x80 frame): preprocess_inputs, a
    stride-2 pooling field scatter with its segment keys and scatter_max,
    and the dense grid, all against the oracle."""
    from ssla_amd import events as E
    from ssla_amd.scatter import scatter_max
    H, W = 64, 80
    ev, lens = _synthetic(7, 2, 3000, H, W, dev)
    gr = E.preprocess_inputs(_t(ev, dev), _t(lens, dev), (H, W), hot_pixel_thres=20)
    ro = OE.preprocess_events(ev, lens, (H, W), hot_pixel_thres=20)
    for key in ("events", "time", "batch_id", "h", "w", "lengths"):
        np.testing.assert_array_equal(_np(gr[key]), ro[key], err_msg=key)

    lut, outc = E.compute_rf2pixels((H, W), (2, 2), (2, 2), device=dev)
    rf = E.gather_receptive_fields(gr, (H, W), lut, outc)
    rro = OE.gather_receptive_fields(ro, (H, W), _np(lut), _np(outc))
    for key in ("events", "time", "pos_id", "lengths", "h", "w", "batch_id"):
        np.testing.assert_array_equal(_np(rf[key]), rro[key], err_msg=key)

    seg, seg_t, new_len = E.pool_segments(rf["time"], rf["lengths"])
    with torch.no_grad():
        pooled, _ = scatter_max(rf["events"], seg, dim=0, dim_size=int(seg_t.numel()), sorted_index=True)
    rp = OE.sparse_pool(rro, "max")
    np.testing.assert_array_equal(_np(pooled), rp["events"])
    np.testing.assert_array_equal(_np(seg_t), rp["time"])
    np.testing.assert_array_equal(_np(new_len), rp["lengths"])

    grid = E.events_to_grid(gr, (H, W), gr["events"].shape[1])
    np.testing.assert_array_equal(_np(grid), OE.event_to_grid(ro, (H, W), ro["events"].shape[1]))


def test_events_to_grids_levels(dev):
    """ssla_events_to_grids (all levels in one launch, every element written)
    against the oracle's index-add into zeros and the one-level call: two
    samples, one group per occupied cell, a channel count that is not a
    multiple of the 4-channel block, an empty level, and a level above the
    one-launch cell limit (taken one level at a time)."""
    from ssla_amd import events as E
    rng = np.random.default_rng(12)
    B = 2
    levels, ref = [], []
    for (Hg, Wg, C, n_grp) in ((30, 38, 64, 700), (15, 19, 22, 200), (8, 10, 256, 0), (100, 90, 8, 3000)):
        cells = rng.choice(B * Hg * Wg, size=n_grp, replace=False)
        cells.sort()
        lens = rng.integers(1, 5, size=n_grp).astype(np.int64)
        x = {"events": rng.standard_normal((int(lens.sum()), C)).astype(np.float32),
             "lengths": lens, "batch_id": (cells // (Hg * Wg)).astype(np.int64),
             "h": (cells % (Hg * Wg) // Wg).astype(np.int64), "w": (cells % Wg).astype(np.int64), "batch_size": B}
        ref.append(OE.event_to_grid(x, (Hg, Wg), C))
        xd = {k: (_t(v, dev) if isinstance(v, np.ndarray) else v) for k, v in x.items()}
        levels.append((xd, (Hg, Wg), C))
    print("events_to_grids: 4 levels", flush=True)
    grids = E.events_to_grids(levels)
    for i, (g, r) in enumerate(zip(grids, ref)):
        np.testing.assert_array_equal(_np(g), r, err_msg=f"level {i}")
        np.testing.assert_array_equal(_np(g), _np(E.events_to_grid(*levels[i])), err_msg=f"level {i}")
    grids3 = E.events_to_grids(levels[:3])   # one launch for all three
    for i in range(3):
        np.testing.assert_array_equal(_np(grids3[i]), ref[i], err_msg=f"one launch, level {i}")


def test_preprocess_large_vs_oracle(dev):
    """ssla_preprocess_events at a capacity of 2 x 40,000 events (its prefix
    sums run as multi-tile look-back scans) against the oracle, bit for
    bit, on the 304 x 240 sensor with a hot pixel over the 512-event cap."""
    from ssla_amd import events as E
    H, W = 240, 304
    gen = np.random.default_rng(31)
    N = 40_000
    lens = np.array([N, 31_000], np.int64)
    ev = np.zeros((2, N, 4), np.float32)
    for b in range(2):
        n = int(lens[b])
        ev[b, :n, 0] = gen.integers(0, W, n)
        ev[b, :n, 1] = gen.integers(0, H, n)
        ev[b, :n, 2] = np.sort(gen.integers(0, 50_000, n))
        ev[b, :n, 3] = np.where(gen.random(n) < 0.5, -1.0, 1.0)
    ev[0, :900, 0], ev[0, :900, 1] = 17.0, 9.0
    print("preprocess large", flush=True)
    one = E.preprocess_inputs(_t(ev, dev), _t(lens, dev), (H, W), hot_pixel_thres=50)
    ro = OE.preprocess_events(ev, lens, (H, W), hot_pixel_thres=50)
    assert ro["lengths"].size > 8192
    for key in ("events", "time", "batch_id", "h", "w", "lengths"):
        np.testing.assert_array_equal(_np(one[key]), ro[key], err_msg=key)


@pytest.mark.parametrize("B,H,W", [(8, 240, 304), (4, 480, 640), (32, 480, 640), (1, 8, 8), (1, 1, 1)],
                         ids=["20bit", "21bit", "24bit", "7bit", "1bit"])
def test_group_events_pixel_sort_widths(dev, B, H, W):
    """group_events' pixel sort (two stable counting passes; digits of 1 to
    12 bits, so 1 to 16 wavefronts per tile and a single pass for 1-bit
    keys) against the oracle's stable argsort, with ragged samples, repeated
    pixels and a few events outside the frame dropped by the lengths."""
    from ssla_amd import events as E
    gen = np.random.default_rng(B * 1000 + H)
    N = 600
    lens = gen.integers(0, N + 1, B).astype(np.int64)
    lens[0] = N
    ev = np.zeros((B, N, 4), np.float32)
    for b in range(B):
        n = int(lens[b])
        ev[b, :n, 0] = gen.integers(0, W, n)
        ev[b, :n, 1] = gen.integers(0, H, n)
        ev[b, :n, 2] = np.sort(gen.integers(0, 10_000, n))
        ev[b, :n, 3] = 1.0
        if n > 40:
            ev[b, 10:40, 0], ev[b, 10:40, 1] = ev[b, 5, 0], ev[b, 5, 1]   # a pixel with many events
    print(f"group_events pixel sort B={B} H={H} W={W}", flush=True)
    gr = E.group_events((_t(ev, dev), _t(lens, dev)), (H, W), max_events_per_px=16)
    ro = OE.group_events(ev, lens, (H, W), max_events_per_px=16)
    for key in ("events", "time", "batch_id", "h", "w", "lengths"):
        np.testing.assert_array_equal(_np(gr[key]), ro[key], err_msg=key)


@pytest.mark.parametrize("thres,extra", [(20, 0), (0, 0), (3, 2), (600, 0)])
def test_preprocess_one_call_vs_composed(dev, thres, extra):
    """ssla_preprocess_events (grouping, delays and truncation in one pass)
    against the step-by-step path and the oracle, with a hot pixel beyond the
    512-event cap (its latest 512 kept, then the first `thres` of those) and
    extra feature columns after p."""
    from ssla_amd import events as E
    H, W = 32, 40
    ev, lens = _synthetic(11, 3, 2500, H, W, dev)
    ev[1, :700, 0], ev[1, :700, 1] = 5.0, 7.0
    if extra:
        rng = np.random.default_rng(4)
        ev = np.concatenate([ev, rng.standard_normal(ev.shape[:2] + (extra,)).astype(np.float32)], -1)
    print(f"preprocess one call thres={thres} extra={extra}", flush=True)
    one = E.preprocess_inputs(_t(ev, dev), _t(lens, dev), (H, W), hot_pixel_thres=thres)
    comp = E._preprocess_composed(_t(ev, dev), _t(lens, dev), (H, W), thres)
    ro = OE.preprocess_events(ev, lens, (H, W), hot_pixel_thres=thres)
    for key in ("events", "time", "batch_id", "h", "w", "lengths"):
        np.testing.assert_array_equal(_np(one[key]), _np(comp[key]), err_msg=key)
        np.testing.assert_array_equal(_np(one[key]), ro[key], err_msg=key)
    assert int(_np(one["lengths"]).max()) == min(512, thres if thres > 0 else 512)


def test_patch_scatter_synthetic(dev):
    from ssla_amd import events as E
    H, W = 40, 48
    ev, lens = _synthetic(3, 3, 1500, H, W, dev)
    evc = np.concatenate([ev, np.random.default_rng(1).normal(size=ev.shape[:2] + (3,)).astype(np.float32)], -1)
    gr = E.group_events((_t(evc, dev), _t(lens, dev)), (H, W))
    ro = OE.group_events(evc, lens, (H, W))
    lut = E.get_patch2pixel_lut((H, W), (3, 3), (1, 1), device=dev)
    res = E.scatter_group_events_to_patch(gr, (H, W), lut)
    rres = OE.scatter_group_events_to_patch(ro, (H, W), _np(lut))
    for key in ("events", "pos_id", "lengths", "orig_event_idx"):
        np.testing.assert_array_equal(_np(res[key]), rres[key], err_msg=key)
    pe = np.random.default_rng(2).normal(size=(rres["events"].shape[0], 5)).astype(np.float32)
    out = E.gather_patch_events_to_group(_t(pe, dev), res["orig_event_idx"], ro["events"].shape[0])
    ref = OE.gather_patch_events_to_group(pe, rres["orig_event_idx"], ro["events"].shape[0])
    np.testing.assert_array_equal(_np(out).view(np.uint32), ref.view(np.uint32))


def test_empty_and_bad_inputs(dev):
    from ssla_amd import events as E
    ev = torch.zeros(2, 5, 4, device=dev)
    gr = E.group_events((ev, torch.zeros(2, dtype=torch.int64, device=dev)), (4, 4))
    assert gr["events"].shape[0] == 0 and gr["lengths"].numel() == 0
    bad = torch.zeros(1, 3, 4, device=dev)
    bad[0, 1, 0] = 9.0                       # x outside a 4-wide frame
    with pytest.raises(ValueError):
        E.group_events((bad, torch.tensor([3], device=dev)), (4, 4))


@pytest.mark.parametrize("k,s", [(3, 1), (1, 1), (2, 2), (3, 2), (5, 1)])
def test_sort_free_field_fill_equals_sort(dev, k, s):
    """The sort-free fill (pixel runs sorted by time, rows placed by counting)
    equals the radix-sort fill bit for bit on a clustered batch with many
    timestamp ties, and its (event, position) -> row map inverts the rows."""
    from ssla_amd import events as E
    H, W = 48, 56
    ev, lens = _synthetic(11 + k, 3, 4000, H, W, dev)
    ev[..., 2] = np.floor(ev[..., 2] / 50.0)   # coarse times: many ties across a field's runs
    gr = E.group_events((_t(ev, dev), _t(lens, dev)), (H, W))
    lut, _ = E.compute_rf2pixels((H, W), (k, k), (s, s), device=dev)
    print(f"sort-free fill k={k} s={s}: E={gr['time'].numel()}", flush=True)
    a = E._rf_scatter(gr, (H, W), lut, dst_map=True)
    b = E._rf_scatter(gr, (H, W), lut, force_sort=True)
    for name, x, y in zip(("src", "time", "pos", "f_index", "f_len"), a[:5], b[:5]):
        np.testing.assert_array_equal(_np(x), _np(y), err_msg=name)
    src, pos, dst = _np(a[0]), _np(a[2]), _np(a[6])
    A = k * k
    assert np.array_equal(dst[src * A + pos], np.arange(src.size))
    assert int((dst >= 0).sum()) == src.size


def test_unsorted_runs_take_the_sort_path(dev):
    """A pixel run out of time order (possible in a hand-built dict) is
    counted by the plan; the sort fill then gives the oracle's rows."""
    from ssla_amd import events as E
    H, W = 6, 7
    ev, lens = _synthetic(5, 1, 300, H, W, dev)
    evc = np.concatenate([ev, np.random.default_rng(4).normal(size=ev.shape[:2] + (2,)).astype(np.float32)], -1)
    gr = E.group_events((_t(evc, dev), _t(lens, dev)), (H, W))
    ro = OE.group_events(evc, lens, (H, W))
    g = int(np.argmax(ro["lengths"]))                 # reverse the longest run's times
    s0 = int(np.sum(ro["lengths"][:g]))
    n = int(ro["lengths"][g])
    ro["time"][s0:s0 + n] = ro["time"][s0:s0 + n][::-1].copy()
    gr["time"] = _t(ro["time"], dev)
    lut = E.get_patch2pixel_lut((H, W), (3, 3), (1, 1), device=dev)
    res = E.scatter_group_events_to_patch(gr, (H, W), lut)
    rres = OE.scatter_group_events_to_patch(ro, (H, W), _np(lut))
    for key in ("events", "pos_id", "lengths", "orig_event_idx"):
        np.testing.assert_array_equal(_np(res[key]), rres[key], err_msg=key)


@pytest.mark.parametrize("n", [1, 1000, 8191, 8192, 8193, 30000])
def test_prefix_sums_across_the_one_workgroup_limit(dev, n):
    """Prefix sums of up to 8192 values run in one workgroup, longer ones
    through rocPRIM: expand_segments (an exclusive scan of the lengths) and
    temporal_dropout_index (two scans) on both sides of the limit, against
    numpy's repeat and the CPU oracle."""
    from ssla_amd import events as E
    rng = np.random.default_rng(n)
    ln = rng.integers(0, 4, size=n)
    vals = rng.integers(-5, 5, size=n)
    got = E.expand_segments(torch.from_numpy(vals).to(dev), torch.from_numpy(ln).to(dev)).cpu().numpy()
    assert np.array_equal(got, np.repeat(vals, ln))
    idx, kl = E.temporal_dropout_index(torch.from_numpy(ln).to(dev), 3)
    want_idx, want_kl = OE.temporal_dropout_index(ln, 3)
    assert np.array_equal(kl.cpu().numpy(), want_kl)
    assert np.array_equal(idx.cpu().numpy(), want_idx)


def test_temporal_dropout_index_row_total(dev):
    """With the events' row count given (the path TemporalDropout takes, no
    read of sum(lengths)) the indices equal the oracle's; lengths that keep
    more rows than that count and the sequences allow raise ValueError."""
    from ssla_amd import events as E
    rng = np.random.default_rng(11)
    ln = rng.integers(0, 9, size=500)
    for w in (1, 3, 4):
        idx, kl = E.temporal_dropout_index(torch.from_numpy(ln).to(dev), w, total=int(ln.sum()))
        want_idx, want_kl = OE.temporal_dropout_index(ln, w)
        assert np.array_equal(kl.cpu().numpy(), want_kl)
        assert np.array_equal(idx.cpu().numpy(), want_idx)
    with pytest.raises(ValueError, match="more than"):
        E.temporal_dropout_index(torch.from_numpy(ln).to(dev), 1, total=10)
