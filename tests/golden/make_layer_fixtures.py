"""Writes golden vectors for the attention layers of the hot path by running
the reference's own layer classes on the CPU of the build container (the
reference tree is not shipped; only these vectors are).

Run from the repository root, with the reference checked out at
/root/reference (override with SSLA_REFERENCE):

    python tests/golden/make_layer_fixtures.py

Layers exercised (reference file:line):
* layers/mos_attention.py:75-146     MosAttention.forward
* layers/linear_attention.py:39-102  LinearAttention.forward

The reference's ``scan`` (ops/common/scan.py:140-163) is a Triton kernel that
needs a GPU; for these vectors the layer modules' ``scan`` name is bound to a
plain torch loop of the recurrence the kernel documents,
``h_t = g_t * h_{t-1} + u_t`` restarted at every ``cu_seqlens`` boundary.
That recurrence is pinned on its own by closed forms in the oracle tests, so
the vectors pin the rest of each layer: patch scatter, the per-position
projections, q/v/g, o_proj, the gather back, the residual and LayerNorm.
torch.sort is forced stable (as in make_event_fixtures.py) so that the patch
order is the one the reference produces whenever its sort is stable.
"""
from __future__ import annotations

import os
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
REF = Path(os.environ.get("SSLA_REFERENCE", "/root/reference"))
OUT = HERE / "layer_fixtures.npz"
sys.path.insert(0, str(HERE))
from make_event_fixtures import make_events  # noqa: E402


def loop_scan(u, g, cu_seqlens):
    h = torch.zeros_like(u)
    cu = cu_seqlens.tolist()
    for s, e in zip(cu[:-1], cu[1:]):
        acc = torch.zeros(u.shape[1], dtype=u.dtype)
        for t in range(s, e):
            acc = g[t] * acc + u[t]
            h[t] = acc
    return h


def main():
    sys.path.insert(0, str(REF))
    from utils import farsecnn_utils
    import layers.mos_attention as mos_mod
    import layers.linear_attention as lin_mod
    mos_mod.scan = loop_scan
    lin_mod.scan = loop_scan

    raw_sort = torch.sort

    def stable_sort(x, *a, **kw):
        kw["stable"] = True
        return raw_sort(x, *a, **kw)

    torch.sort = stable_sort
    out = {}
    try:
        H, W = 16, 20
        ev, lengths = make_events(11, 3, 90, H, W)
        gr = farsecnn_utils.group_events((ev.clone(), lengths.clone()), (H, W), max_events_per_px=512)
        out["in_frame"] = np.array([H, W])
        for key in ("time", "batch_id", "h", "w", "lengths"):
            out[f"in_{key}"] = gr[key].numpy()
        out["in_batch_size"] = np.array(int(gr["batch_size"]))
        gen = torch.Generator().manual_seed(3)
        n = gr["time"].shape[0]
        feats = {6: torch.randn(n, 6, generator=gen), 8: torch.randn(n, 8, generator=gen)}
        for C, f in feats.items():
            out[f"in_events_c{C}"] = f.numpy()

        cases = (
            # tag, input, hidden, kernel, stride, scatter_proj, gather_proj
            ("mos_a", 6, 8, (3, 3), (1, 1), True, True),
            ("mos_b", 8, 8, (2, 2), (2, 2), True, True),
            ("mos_c", 6, 8, (3, 3), (1, 1), False, False),
        )
        for tag, ci, ch, k, s, sp, gp in cases:
            torch.manual_seed(100 + len(tag) + ci + k[0])
            layer = mos_mod.MosAttention(ci, ch, (H, W), k, s, scatter_proj=sp, gather_proj=gp)
            with torch.no_grad():
                layer.norm.weight.uniform_(0.5, 1.5)
                layer.norm.bias.uniform_(-0.5, 0.5)
            inp = dict(gr)
            inp["events"] = feats[ci].clone()
            with torch.no_grad():
                r = layer(inp)
            for name, t in layer.state_dict().items():
                out[f"{tag}_sd_{name}"] = t.numpy()
            out[f"{tag}_out"] = r["events"].numpy()

        for tag, ci, ch in (("lin_a", 6, 8), ("lin_b", 8, 8)):
            torch.manual_seed(200 + ci)
            layer = lin_mod.LinearAttention(ci, ch, (H, W))
            with torch.no_grad():
                layer.norm.weight.uniform_(0.5, 1.5)
                layer.norm.bias.uniform_(-0.5, 0.5)
            inp = dict(gr)
            inp["events"] = feats[ci].clone()
            with torch.no_grad():
                r = layer(inp)
            for name, t in layer.state_dict().items():
                out[f"{tag}_sd_{name}"] = t.numpy()
            out[f"{tag}_out"] = r["events"].numpy()
    finally:
        torch.sort = raw_sort

    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(out)} arrays)")


if __name__ == "__main__":
    main()
