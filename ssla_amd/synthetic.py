"""Seeded synthetic inputs of the benchmark configurations.

The reference ships no datasets for this path, so every measurement and
full-size parity test runs on these generators (host numpy/torch, moved to
the device by the caller):

* :func:`chunk_gla_inputs` -- chunked GLA forward, B=8 sequences of 4096
  tokens, H=8, K=V=64 (q, k, v bf16 ~ N(0,1) with q pre-scaled by 1/8,
  gates logsigmoid(N(0,1)/16), h0 ~ N(0, 0.1)).
* :func:`sparse_scan_bins` -- per-site GLA scan over a 76x60 grid, 64 bins,
  10-30 % of sites active per bin as Gaussian blobs (sigma 6) around 5-15
  moving centres.
* :func:`pooling_events` -- 1e6 events on 304x240 (70 % in 20 Gaussian
  clusters of sigma 8 px, 30 % uniform) with C=64 fp32 features, pooled
  2x2 into the 152x120 cell grid.
* :func:`event_windows` -- a batch of Gen1 windows (304x240 sensor, 100 ms
  each, about 50k events per window from the same cluster mixture, t
  sorted and uniform in the window, polarity +-1 equiprobable) as the padded
  <x, y, t, p> batch the model's preprocessing takes.
* :func:`async_windows` -- consecutive 100 ms windows of one stream (the
  same cluster mixture, centres drifting across windows, absolute
  timestamps) for the asynchronous forward step that carries its per-site
  states from window to window.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import List

import numpy as np
import torch
import torch.nn.functional as F


def chunk_gla_inputs(B=8, T=4096, H=8, D=64, dtype=torch.bfloat16, seed=0, device="cpu"):
    gen = torch.Generator().manual_seed(seed)
    Tt = B * T
    q = torch.randn(Tt, H, D, generator=gen) * (D ** -0.5)
    k = torch.randn(Tt, H, D, generator=gen)
    v = torch.randn(Tt, H, D, generator=gen)
    g = F.logsigmoid(torch.randn(Tt, H, D, generator=gen) / 16)
    h0 = torch.randn(B, H, D, D, generator=gen) * 0.1
    cu = torch.arange(0, Tt + 1, T, dtype=torch.int64)
    return dict(q=q.to(dtype).to(device), k=k.to(dtype).to(device), v=v.to(dtype).to(device),
                g=g.to(device), cu_seqlens=cu.to(device), initial_state=h0.to(device), scale=1.0)


@dataclass
class SparseBins:
    grid: tuple                 # (W, H) in sites
    sites: List[np.ndarray]     # per bin: sorted unique int32 site ids
    q: List[torch.Tensor]       # per bin: [n_b, H, K] fp32
    k: List[torch.Tensor]
    v: List[torch.Tensor]
    g: List[torch.Tensor]
    state0: torch.Tensor        # [n_sites, H, K, V] fp32
    scale: float

    @property
    def n_sites(self):
        return self.grid[0] * self.grid[1]

    @property
    def site_steps(self):
        return int(sum(s.size for s in self.sites))


def sparse_scan_bins(n_bins=64, W=76, Hg=60, heads=4, D=32, seed=0, sigma=6.0) -> SparseBins:
    rng = np.random.default_rng(seed)
    n_sites = W * Hg
    n_c = int(rng.integers(5, 16))
    pos = rng.uniform([0, 0], [W, Hg], size=(n_c, 2))
    vel = rng.uniform(-1.0, 1.0, size=(n_c, 2))
    sites = []
    for _ in range(n_bins):
        frac = rng.uniform(0.10, 0.30)
        n_b = int(round(frac * n_sites))
        chosen = np.zeros(0, np.int64)
        while chosen.size < n_b:
            c = rng.integers(0, n_c, size=4 * n_b)
            p = pos[c] + rng.normal(0.0, sigma, size=(4 * n_b, 2))
            p = np.rint(p).astype(np.int64)
            ok = (p[:, 0] >= 0) & (p[:, 0] < W) & (p[:, 1] >= 0) & (p[:, 1] < Hg)
            ids = p[ok, 1] * W + p[ok, 0]
            allc = np.concatenate([chosen, ids])
            _, first = np.unique(allc, return_index=True)
            chosen = allc[np.sort(first)]
        sites.append(np.sort(chosen[:n_b]).astype(np.int32))
        pos = pos + vel
        for d, lim in ((0, W), (1, Hg)):        # reflect at the borders
            lo, hi = pos[:, d] < 0, pos[:, d] > lim - 1
            pos[lo, d] = -pos[lo, d]
            pos[hi, d] = 2 * (lim - 1) - pos[hi, d]
            vel[lo | hi, d] = -vel[lo | hi, d]
    gen = torch.Generator().manual_seed(seed)
    qs, ks, vs, gs = [], [], [], []
    for s in sites:
        n = s.size
        qs.append(torch.randn(n, heads, D, generator=gen))
        ks.append(torch.randn(n, heads, D, generator=gen))
        vs.append(torch.randn(n, heads, D, generator=gen))
        gs.append(F.logsigmoid(torch.randn(n, heads, D, generator=gen) / 16))
    state0 = torch.randn(n_sites, heads, D, D, generator=torch.Generator().manual_seed(seed + 1)) * 0.1
    return SparseBins((W, Hg), sites, qs, ks, vs, gs, state0, D ** -0.5)


def pooling_events(E=1_000_000, C=64, W=304, Hp=240, n_clusters=20, sigma=8.0, seed=0):
    """Returns (src fp32 [E, C], index int64 [E], n_out) with index = cell of
    the 2x2 pooling (cell = (y >> 1) * (W/2) + (x >> 1)), events shuffled."""
    rng = np.random.default_rng(seed)
    n_cl = int(round(0.7 * E))
    centres = rng.uniform([0, 0], [W, Hp], size=(n_clusters, 2))
    which = rng.integers(0, n_clusters, size=n_cl)
    xy_c = centres[which] + rng.normal(0.0, sigma, size=(n_cl, 2))
    xy_u = rng.uniform([0, 0], [W, Hp], size=(E - n_cl, 2))
    xy = np.rint(np.concatenate([xy_c, xy_u]))
    x = np.clip(xy[:, 0], 0, W - 1).astype(np.int64)
    y = np.clip(xy[:, 1], 0, Hp - 1).astype(np.int64)
    perm = rng.permutation(E)
    x, y = x[perm], y[perm]
    Wc = W // 2
    index = (y >> 1) * Wc + (x >> 1)
    gen = torch.Generator().manual_seed(seed)
    src = torch.randn(E, C, generator=gen)
    return src, torch.from_numpy(index), Wc * (Hp // 2)


def event_windows(B=8, n_mean=50_000, W=304, Hp=240, window_us=100_000, n_clusters=20, sigma=8.0, seed=0):
    """Returns (events fp32 [B, N, 4] as <x, y, t, p>, lengths int64 [B]):
    window b holds n_mean * (0.8 + 0.4 * b / (B - 1)) events (ragged
    batch), 70 % in Gaussian clusters (sigma px) around centres that drift
    across the window, 30 % uniform; t (microseconds) sorted uniform in
    [0, window_us); p = +-1; rows past a window's length are (0, 0, 0, -1),
    the padding of the reference's collate."""
    rng = np.random.default_rng(seed)
    lens = [int(n_mean * (0.8 + 0.4 * b / max(B - 1, 1))) for b in range(B)]
    N = max(lens)
    ev = np.zeros((B, N, 4), np.float32)
    for b, n in enumerate(lens):
        t = np.sort(rng.integers(0, window_us, n))
        c0 = rng.uniform([0, 0], [W, Hp], size=(n_clusters, 2))
        vel = rng.uniform(-30, 30, size=(n_clusters, 2))          # px per window
        n_cl = int(round(0.7 * n))
        pick = rng.permutation(n)
        cl, un = pick[:n_cl], pick[n_cl:]
        xy = np.empty((n, 2))
        which = rng.integers(0, n_clusters, size=n_cl)
        xy[cl] = c0[which] + vel[which] * (t[cl, None] / window_us) + rng.normal(0.0, sigma, size=(n_cl, 2))
        xy[un] = rng.uniform([0, 0], [W, Hp], size=(len(un), 2))
        xy = np.rint(xy)
        ev[b, :n, 0] = np.clip(xy[:, 0], 0, W - 1)
        ev[b, :n, 1] = np.clip(xy[:, 1], 0, Hp - 1)
        ev[b, :n, 2] = t
        ev[b, :n, 3] = 2 * rng.integers(0, 2, n) - 1
        ev[b, n:, 3] = -1
    return torch.from_numpy(ev), torch.tensor(lens, dtype=torch.int64)


def async_windows(n_windows=20, n_events=50_000, W=304, Hp=240, window_us=100_000, n_clusters=20, sigma=8.0,
                  seed=0) -> List[torch.Tensor]:
    """``n_windows`` consecutive windows of one event stream, each an fp32
    ``[1, n_events, 4]`` batch of <x, y, t, p> (t in microseconds from the
    stream start, sorted; window w covers [w, w + 1) * window_us).  70 % of
    the events fall in Gaussian clusters (sigma px) whose centres move at a
    constant velocity across the whole stream, 30 % are uniform; p = +-1
    equiprobable.  Clusters persisting from window to window make the same
    sites active again, so the carried per-site states matter."""
    rng = np.random.default_rng(seed)
    c0 = rng.uniform([0, 0], [W, Hp], size=(n_clusters, 2))
    vel = rng.uniform(-30, 30, size=(n_clusters, 2))            # px per window
    out = []
    for w in range(n_windows):
        t = np.sort(rng.integers(0, window_us, n_events)) + w * window_us
        n_cl = int(round(0.7 * n_events))
        pick = rng.permutation(n_events)
        cl, un = pick[:n_cl], pick[n_cl:]
        xy = np.empty((n_events, 2))
        which = rng.integers(0, n_clusters, size=n_cl)
        pos = c0[which] + vel[which] * (t[cl, None] / window_us)
        pos = np.abs(np.mod(pos, [2 * W, 2 * Hp]))                 # reflect at the borders
        pos = np.where(pos >= [W, Hp], [2 * W, 2 * Hp] - pos, pos)
        xy[cl] = pos + rng.normal(0.0, sigma, size=(n_cl, 2))
        xy[un] = rng.uniform([0, 0], [W, Hp], size=(len(un), 2))
        xy = np.rint(xy)
        ev = np.empty((1, n_events, 4), np.float32)
        ev[0, :, 0] = np.clip(xy[:, 0], 0, W - 1)
        ev[0, :, 1] = np.clip(xy[:, 1], 0, Hp - 1)
        ev[0, :, 2] = t
        ev[0, :, 3] = 2 * rng.integers(0, 2, n_events) - 1
        out.append(torch.from_numpy(ev))
    return out
