"""CPU oracle of the attention layers -- TEST INFRASTRUCTURE ONLY.

fp64 numpy restatements of the reference's MosAttention and LinearAttention
forwards (haohq19/ssla), composed from the event-glue oracle
(``oracle.events``) and the diagonal-scan oracle (``oracle.diag_scan``).
Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may use this module, and only as the checker.  Both
functions are pinned against ``tests/golden/layer_fixtures.npz``, which the
reference's own layer classes produced (``tests/test_oracle_layers.py``).

``params`` is a layer's state dict as numpy arrays (the reference's names).
"""
from __future__ import annotations

import numpy as np

from . import diag_scan
from . import events as oe


def _sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def _layer_norm(x, w, b, eps=1e-5):
    mu = x.mean(axis=1, keepdims=True)
    var = ((x - mu) ** 2).mean(axis=1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * w + b


def _grouped(x, pos, weights, hidden, in_size, enabled):
    """layers/mos_attention.py:148-167: row e multiplied by the weight of its
    kernel position (one shared weight when the projection is disabled)."""
    w = np.asarray(weights, np.float64).reshape(-1, hidden, in_size)
    if not enabled:
        return x @ w[0].T
    return np.einsum("eoi,ei->eo", w[pos], x)


def mos_attention(params, gr, frame_size, kernel_size, stride, scatter_proj=True, gather_proj=True):
    """layers/mos_attention.py:75-146; returns the output events [E, hidden]."""
    hidden = params["q_proj.weight"].shape[0]
    in_size = np.asarray(gr["events"]).shape[1]
    lut, _ = oe.rf2pixels(frame_size, kernel_size, stride)
    patch = oe.scatter_group_events_to_patch(gr, frame_size, lut)
    x = np.asarray(patch["events"], np.float64)
    pos = np.asarray(patch["pos_id"], np.int64)
    x = _grouped(x, pos, params["scatter_conv_weights"], hidden, in_size, scatter_proj)
    q = x @ params["q_proj.weight"].astype(np.float64).T
    v = x @ params["v_proj.weight"].astype(np.float64).T
    g = _sigmoid(x @ params["g_proj.weight"].astype(np.float64).T)
    lens = np.asarray(patch["lengths"], np.int64)
    cu = np.unique(np.concatenate([[0], np.cumsum(lens)]))
    h = diag_scan(v, g, cu)
    o = (q * h) @ params["o_proj.weight"].astype(np.float64).T
    o = _grouped(o, pos, params["gather_conv_weights"], hidden, hidden, gather_proj)
    n_pix = np.asarray(gr["events"]).shape[0]
    out = np.zeros((n_pix, hidden), np.float64)
    np.add.at(out, np.asarray(patch["orig_event_idx"], np.int64), o)
    res = np.asarray(gr["events"], np.float64)
    if "input_proj.weight" in params:
        res = res @ params["input_proj.weight"].astype(np.float64).T
    return _layer_norm(out + res, params["norm.weight"], params["norm.bias"])


def linear_attention(params, gr):
    """layers/linear_attention.py:39-102; returns the output events [E, hidden]."""
    ev = np.asarray(gr["events"], np.float64)
    x = ev @ params["input_proj.weight"].astype(np.float64).T if "input_proj.weight" in params else ev
    lens = np.asarray(gr["lengths"], np.int64)
    ev_b = np.repeat(np.asarray(gr["batch_id"], np.int64), lens)
    t = np.asarray(gr["time"], np.int64)
    order = np.lexsort((np.arange(t.size), t, ev_b))      # (batch, time), ties in event order
    B = int(gr["batch_size"])
    counts = np.bincount(ev_b, minlength=B)
    cu = np.concatenate([[0], np.cumsum(counts[counts > 0])])
    xs = x[order]
    q = xs @ params["q_proj.weight"].astype(np.float64).T
    v = xs @ params["v_proj.weight"].astype(np.float64).T
    g = _sigmoid(xs @ params["g_proj.weight"].astype(np.float64).T)
    h = diag_scan(v, g, cu)
    o = (q * h) @ params["o_proj.weight"].astype(np.float64).T
    out = np.empty_like(o)
    out[order] = o
    res = ev @ params["residual_proj.weight"].astype(np.float64).T if "residual_proj.weight" in params else ev
    return _layer_norm(out + res, params["norm.weight"], params["norm.bias"])
