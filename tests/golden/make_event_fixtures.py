"""Writes the golden vectors for the event-glue rows of the hot path by
running the reference's own pure-torch functions on the CPU of the build
container (the reference tree is not shipped; only these vectors are).

Run from the repository root, with the reference checked out at
/root/reference (override with SSLA_REFERENCE):

    python tests/golden/make_event_fixtures.py

Functions exercised (reference file:line):
* utils/async_utils.py:10-84     group_events (MOS variant)
* utils/farsecnn_utils.py:130-174 group_events (the one model_mos.py uses)
* utils/async_utils.py:96-122     get_patch2pixel_lut
* utils/async_utils.py:125-240    scatter_group_events_to_patch
* utils/async_utils.py:243-264    gather_patch_events_to_group
* utils/farsecnn_utils.py:95-128  compute_rf2pixels
* utils/farsecnn_utils.py:177-265 gather_receptive_fields
* utils/farsecnn_utils.py:8-33    truncate_packed_sequence
* layers/temporal_dropout.py:14-59 TemporalDropout.forward
* ops/gla/naive.py:50-111         naive_gla_recurrent
Inputs are small, seeded, and built to contain timestamp ties, pixels with
more events than the per-pixel cap, empty batch entries and border pixels.

scatter_group_events_to_patch and gather_receptive_fields sort with
torch.sort(stable=False), whose tie order is implementation-defined (the CPU
kernel is unstable below roughly 2e4 elements and stable above).  Their
vectors are therefore written twice: as the reference returns them ("raw",
pinned up to reordering within (field, time) ties) and with torch.sort
forced stable (pinned exactly; this is the order the reference produces
whenever its sort is stable).
"""
from __future__ import annotations

import os
import sys
from pathlib import Path

import numpy as np
import torch

REF = Path(os.environ.get("SSLA_REFERENCE", "/root/reference"))
OUT = Path(__file__).resolve().parent / "event_fixtures.npz"


def make_events(seed, B, N, H, W, n_hot=2, tie_every=3):
    """Padded [B, N, 5] float events <x, y, t, t, p> with time-sorted rows,
    repeated timestamps and a few hot pixels."""
    g = torch.Generator().manual_seed(seed)
    ev = torch.zeros(B, N, 5)
    lengths = torch.randint(N // 2, N + 1, (B,), generator=g)
    lengths[-1] = 0 if B > 2 else lengths[-1]      # an empty sample when B > 2
    for b in range(B):
        n = int(lengths[b])
        x = torch.randint(0, W, (n,), generator=g)
        y = torch.randint(0, H, (n,), generator=g)
        hot = torch.rand(n, generator=g) < 0.3
        hx = torch.randint(0, W, (n_hot,), generator=g)
        hy = torch.randint(0, H, (n_hot,), generator=g)
        pick = torch.randint(0, n_hot, (n,), generator=g)
        x = torch.where(hot, hx[pick], x)
        y = torch.where(hot, hy[pick], y)
        t = torch.sort(torch.randint(0, max(2, n // tie_every), (n,), generator=g) * 7).values
        p = torch.where(torch.rand(n, generator=g) < 0.5, -1.0, 1.0)
        ev[b, :n, 0] = x.float()
        ev[b, :n, 1] = y.float()
        ev[b, :n, 2] = t.float()
        ev[b, :n, 3] = t.float()
        ev[b, :n, 4] = p
    return ev, lengths


def main():
    sys.path.insert(0, str(REF))
    from utils import async_utils, farsecnn_utils
    from layers.temporal_dropout import TemporalDropout
    from ops.gla.naive import naive_gla_recurrent

    out = {}
    # ---- group_events (both variants), with a small per-pixel cap ---------
    H, W = 16, 20
    ev, lengths = make_events(0, 3, 120, H, W)
    out["ge_events"] = ev.numpy()
    out["ge_lengths"] = lengths.numpy()
    out["ge_frame"] = np.array([H, W])
    for tag, fn in (("mos", async_utils.group_events), ("farse", farsecnn_utils.group_events)):
        for cap in (4, 512):
            gr = fn((ev.clone(), lengths.clone()), (H, W), max_events_per_px=cap)
            for key in ("events", "time", "batch_id", "h", "w", "lengths"):
                out[f"ge_{tag}_{cap}_{key}"] = gr[key].numpy()

    # ---- patch scatter / gather (MOS), kernel 3 stride 1 and kernel 2 stride 1
    gr = farsecnn_utils.group_events((ev.clone(), lengths.clone()), (H, W), max_events_per_px=512)
    feats = torch.randn(gr["events"].shape[0], 3, generator=torch.Generator().manual_seed(5))
    gr_f = dict(gr)
    gr_f["events"] = feats
    out["sp_pix_events"] = feats.numpy()
    for ks in (3, 2):
        lut = async_utils.get_patch2pixel_lut((H, W), (ks, ks), (1, 1))
        out[f"sp_lut_k{ks}"] = lut.numpy()
        pi = async_utils.scatter_group_events_to_patch(gr_f, (H, W), lut)
        for key in ("events", "pos_id", "lengths", "orig_event_idx"):
            out[f"sp_k{ks}_{key}"] = pi[key].numpy()
        pe = torch.randn(pi["events"].shape[0], 3, generator=torch.Generator().manual_seed(6 + ks))
        out[f"sp_k{ks}_gather_in"] = pe.numpy()
        out[f"sp_k{ks}_gather_out"] = async_utils.gather_patch_events_to_group(
            pe, pi["orig_event_idx"], gr["events"].shape[0]).numpy()
    # LUT on a non-divisible frame and strides > 1
    for (fh, fw, k, s) in ((7, 10, 3, 2), (9, 5, 2, 2), (12, 15, 3, 1), (6, 8, 5, 3)):
        lut = async_utils.get_patch2pixel_lut((fh, fw), (k, k), (s, s))
        rf, oc = farsecnn_utils.compute_rf2pixels((fh, fw), (k, k), (s, s))
        out[f"lut_{fh}x{fw}_k{k}s{s}"] = lut.numpy()
        out[f"rf2p_{fh}x{fw}_k{k}s{s}"] = rf.numpy()
        out[f"rfout_{fh}x{fw}_k{k}s{s}"] = oc.numpy()

    # ---- gather_receptive_fields (SparsePool's input), k2 s2 and k3 s2 ------
    for (k, s) in ((2, 2), (3, 2)):
        rf, oc = farsecnn_utils.compute_rf2pixels((H, W), (k, k), (s, s))
        gi = dict(gr_f)
        gi["time"] = gr["time"].clone()
        ri = farsecnn_utils.gather_receptive_fields(gi, (H, W), rf, oc)
        for key in ("events", "time", "pos_id", "lengths", "h", "w", "batch_id"):
            out[f"grf_k{k}s{s}_{key}"] = ri[key].numpy()

    # ---- truncate_packed_sequence -----------------------------------------
    data = torch.arange(60, dtype=torch.float32).reshape(30, 2)
    seqlens = torch.tensor([5, 1, 0, 9, 3, 12])
    other = torch.arange(30) * 3
    nd, nl, no = farsecnn_utils.truncate_packed_sequence(data, seqlens, 4, others=other)
    out["tr_data"], out["tr_seqlens"], out["tr_other"] = data.numpy(), seqlens.numpy(), other.numpy()
    out["tr_new_data"], out["tr_new_lengths"], out["tr_new_other"] = nd.numpy(), nl.numpy(), no.numpy()

    # ---- TemporalDropout ----------------------------------------------------
    for wsz in (1, 3, 4):
        td = TemporalDropout(wsz, (H, W))
        inp = dict(gr_f)
        inp["time"] = gr["time"].clone()
        r = td(inp, grouped_events=True)
        for key in ("events", "time", "lengths"):
            out[f"td_w{wsz}_{key}"] = r[key].numpy()
    out["td_in_time"] = gr["time"].numpy()
    out["td_in_lengths"] = gr["lengths"].numpy()

    # ---- naive_gla_recurrent (small config-1 shaped case) --------------------
    gq = torch.Generator().manual_seed(0)
    T, Hh, K = 48, 2, 16
    q = torch.randn(T, Hh, K, generator=gq) * K ** -0.5
    kk = torch.randn(T, Hh, K, generator=gq)
    v = torch.randn(T, Hh, K, generator=gq)
    g = torch.nn.functional.logsigmoid(torch.randn(T, Hh, K, generator=gq) / 16)
    cu = torch.tensor([0, 30, 48])
    h0 = torch.randn(2, Hh, K, K, generator=gq) * 0.1
    o, ht = naive_gla_recurrent(q, kk, v, g, cu, scale=1.0, initial_state=h0, output_final_state=True)
    for name, t in (("q", q), ("k", kk), ("v", v), ("g", g), ("cu", cu), ("h0", h0), ("o", o), ("ht", ht)):
        out[f"gla_{name}"] = t.numpy()

    # ---- the two sort-based functions again with a stable torch.sort ------
    raw_sort = torch.sort

    def stable_sort(x, *a, **kw):
        kw["stable"] = True
        return raw_sort(x, *a, **kw)

    torch.sort = stable_sort
    try:
        for ks in (3, 2):
            lut = async_utils.get_patch2pixel_lut((H, W), (ks, ks), (1, 1))
            pi = async_utils.scatter_group_events_to_patch(gr_f, (H, W), lut)
            for key in ("events", "pos_id", "lengths", "orig_event_idx"):
                out[f"sps_k{ks}_{key}"] = pi[key].numpy()
            pe = torch.from_numpy(out[f"sp_k{ks}_gather_in"])
            out[f"sps_k{ks}_gather_out"] = async_utils.gather_patch_events_to_group(
                pe, pi["orig_event_idx"], gr["events"].shape[0]).numpy()
        for (k, s) in ((2, 2), (3, 2)):
            rf, oc = farsecnn_utils.compute_rf2pixels((H, W), (k, k), (s, s))
            gi = dict(gr_f)
            gi["time"] = gr["time"].clone()
            ri = farsecnn_utils.gather_receptive_fields(gi, (H, W), rf, oc)
            for key in ("events", "time", "pos_id", "lengths", "h", "w", "batch_id"):
                out[f"grfs_k{k}s{s}_{key}"] = ri[key].numpy()
    finally:
        torch.sort = raw_sort

    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(out)} arrays)")


if __name__ == "__main__":
    main()
