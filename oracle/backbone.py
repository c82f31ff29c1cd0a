"""CPU oracle of the asynchronous forward step (ssla_amd.backbone) -- TEST
INFRASTRUCTURE ONLY.

fp64 numpy restatement of one window of the per-site GLA backbone, composed
from the pinned oracle pieces: preprocessing and receptive-field pooling
(``oracle.events``: model_mos.py:173-209, utils/farsecnn_utils.py:177-265,
layers/sparse_pooling.py:14-51), the GLA recurrence (``oracle.gla_recurrent``:
ops/gla/naive.py:50-111, here per site with the stored state as the
initial state and the final state written back), the dense last-event grids
(model_mos.py:212-228) and the YOLOX head's inference path
(layers/yolox_head.py:100-256).  Only ``tests/`` and ``bench.py``'s
``cpu_baseline`` leg use this module, and only as the checker / baseline.

The GPU step computes its projections in bf16 (inputs and weights rounded to
bf16, fp32 accumulation, bf16 results) and keeps the residual stream, the
gates, the recurrence state and LayerNorm in fp32; the restatement rounds
the same operands and results to bf16 (``bf16``) and computes everything else
in fp64.  ``params`` is the module's state dict as numpy arrays.
"""
from __future__ import annotations

import numpy as np
import torch

from . import events as oe
from . import gla_recurrent


def bf16(a):
    """Round to bfloat16 (nearest even) and return the values as fp64."""
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).bfloat16().double().numpy()


def _linear_bf16(x, w):
    """bf16 GEMM: bf16 operands, result rounded to fp32 then to bf16."""
    return bf16((bf16(x) @ bf16(w).T).astype(np.float32))


def _logsigmoid(x):
    return np.minimum(x, 0.0) - np.log1p(np.exp(-np.abs(x)))


def _layer_norm(x, w, b, eps=1e-5):
    mu = x.mean(axis=1, keepdims=True)
    var = ((x - mu) ** 2).mean(axis=1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * w + b


# ------------------------------------------------------------ GLA block --
def block_project(p, x, heads, head_dim, gate_normalizer=16.0):
    """q, k, v (bf16 values) and fp32 log-gates of every event row."""
    n = x.shape[0]
    shp = (n, heads, head_dim)
    q, k, v = (_linear_bf16(x, p[f"{nm}_proj.weight"]).reshape(shp) for nm in ("q", "k", "v"))
    g = (_logsigmoid(_linear_bf16(x, p["g_proj.weight"])) / gate_normalizer).astype(np.float32).reshape(shp)
    return q, k, v, g


def block_scan(q, k, v, g, lengths, sites, state, scale):
    """Per-site recurrence: site sites[i] runs its lengths[i] rows from
    state[sites[i]]; its final state is stored back (fp32).  Rows of other
    sites are untouched.  Returns o (fp64)."""
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)
    sites = np.asarray(sites, np.int64)
    o, ht = gla_recurrent(q, k, v, g, cu, scale, state[sites], True)
    state[sites] = ht.astype(np.float32)
    return o


def block_finish(p, o_bf16, x):
    """LayerNorm(o_proj(o) + residual): bf16 projections, fp64 rest."""
    n = x.shape[0]
    y = _linear_bf16(o_bf16.reshape(n, -1), p["o_proj.weight"])
    if "res_proj.weight" in p:
        y = y + _linear_bf16(x, p["res_proj.weight"])
    else:
        y = y + np.asarray(x, np.float64)
    return _layer_norm(y, p["norm.weight"], p["norm.bias"])


def sites_of(gr, grid_size):
    Hg, Wg = grid_size
    return (np.asarray(gr["batch_id"]) * Hg + np.asarray(gr["h"])) * Wg + np.asarray(gr["w"])


def site_gla_block(p, gr, state, grid_size, heads=4, head_dim=32):
    x = np.asarray(gr["events"], np.float32)
    q, k, v, g = block_project(p, x, heads, head_dim)
    o = block_scan(q, k, v, g, gr["lengths"], sites_of(gr, grid_size), state, head_dim ** -0.5)
    out = dict(gr)
    out["events"] = block_finish(p, bf16(o.astype(np.float32)), x).astype(np.float32)
    return out


# -------------------------------------------------------------- pooling --
def max_pool(gr, frame_size, k):
    """SparseMaxPool(kernel k, stride k): receptive-field gather, then the
    max over events of one field with one timestamp."""
    lut, outc = oe.rf2pixels(frame_size, (k, k), (k, k))
    rf = oe.gather_receptive_fields(gr, frame_size, lut, outc)
    pooled = oe.sparse_pool(rf, "max")
    return {"events": pooled["events"], "time": pooled["time"], "lengths": pooled["lengths"],
            "h": rf["h"], "w": rf["w"], "batch_id": rf["batch_id"], "batch_size": gr["batch_size"]}


def stem(p, events, lengths, frame_size, k, hot_pixel_thres=50):
    gr = oe.preprocess_events(events, lengths, frame_size, hot_pixel_thres)
    gr["events"] = _linear_bf16(gr["events"], p["embed.weight"]).astype(np.float32)
    return max_pool(gr, frame_size, k)


# ----------------------------------------------------------------- head --
def head(p, grids, strides, eps=1e-5):
    """DetectionHead in fp64 from bf16 weights and inputs: [B, anchors, 5+C]."""
    def conv(x, pre):
        return np.einsum("oc,bchw->bohw", bf16(p[pre + ".weight"][:, :, 0, 0]), x) + \
            bf16(p[pre + ".bias"])[None, :, None, None]

    def branch(x, pre):
        y = conv(x, pre + ".0")
        m, var = bf16(p[pre + ".1.running_mean"]), bf16(p[pre + ".1.running_var"])
        y = (y - m[None, :, None, None]) / np.sqrt(var + eps)[None, :, None, None]
        y = y * bf16(p[pre + ".1.weight"])[None, :, None, None] + bf16(p[pre + ".1.bias"])[None, :, None, None]
        return y / (1.0 + np.exp(-y))

    outs = []
    for lvl, x in enumerate(grids):
        x = bf16(x)
        cf, rfeat = branch(x, f"cls_convs.{lvl}"), branch(x, f"reg_convs.{lvl}")
        out = np.concatenate([conv(rfeat, f"reg_preds.{lvl}"), conv(rfeat, f"obj_preds.{lvl}"),
                              conv(cf, f"cls_preds.{lvl}")], 1)
        B, C, Hh, Ww = out.shape
        out = out.transpose(0, 2, 3, 1).reshape(B, Hh * Ww, C)
        yv, xv = np.meshgrid(np.arange(Hh), np.arange(Ww), indexing="ij")
        cell = np.stack([xv, yv], 2).reshape(1, Hh * Ww, 2)
        s = strides[lvl]
        out = np.concatenate([(out[..., :2] + cell) * s, np.exp(out[..., 2:4]) * s, out[..., 4:]], -1)
        outs.append(out)
    return np.concatenate(outs, 1)


# ------------------------------------------------------------ one window --
def async_step(params, events, lengths, states, frame_size=(240, 304),
               stages=((32, 4), (64, 8), (128, 16), (256, 32)), heads=4, head_dim=32):
    """One window of AsyncSparseGLA: returns (head output, per-stage outputs)
    and updates `states` (list of fp32 arrays) in place."""
    def sub(prefix):
        n = len(prefix)
        return {k[n:]: v for k, v in params.items() if k.startswith(prefix)}

    grids_hw = [(-(-frame_size[0] // s), -(-frame_size[1] // s)) for _, s in stages]
    x = stem(params, events, lengths, frame_size, stages[0][1])
    feats = []
    for i in range(len(stages)):
        x = site_gla_block(sub(f"blocks.{i}."), x, states[i], grids_hw[i], heads, head_dim)
        feats.append(x)
        if i + 1 < len(stages):
            x = max_pool(x, grids_hw[i], stages[i + 1][1] // stages[i][1])
    levels = list(range(1, len(stages)))
    grids = [oe.event_to_grid(feats[i], grids_hw[i], stages[i][0]) for i in levels]
    return head(sub("head."), grids, [stages[i][1] for i in levels]), feats
