"""The asynchronous forward step of a sparse GLA backbone on MI355X: the
fifth configuration of the benchmark this package is measured on.

The reference's MosModel step (model_mos.py:157-170) preprocesses a window
of events into pixel groups (:173-209), runs its backbone of sparse layers,
turns the stride-8/16/32 outputs into dense grids (async_event_to_grid,
:212-228) and ends with a YOLOX head (layers/yolox_head.py:183-230).  Its
layers keep no state from one window to the next.  The configuration
measured here keeps one: every stage holds a per-site GLA state
``S[site] in R^{H x D x D}`` (fp32, resident in HBM) that is carried across
consecutive windows, and a window updates the states of the sites it
touches only.  For a site with events ``x_1..x_n`` (in time order) in this
window, with ``q, k, v = W x`` (bf16) and per-key log-gates
``g = logsigmoid(W_g x) / 16``:

    S <- diag(exp(g_t)) S + k_t v_t^T,   o_t = (D^-1/2 q_t)^T S      (t = 1..n)

which is the reference's ``naive_gla_recurrent`` (ops/gla/naive.py:50-111)
over the site's events with ``initial_state = S[site]`` and the final state
written back -- one ``ssla_gla_recurrent_fwd`` launch with ``state_idx``
per stage (``sparse_gla_scan``).  Sites without events keep their states
bit for bit.

Step (one window, B samples):
  preprocess (group_events, pixel delays, hot-pixel truncation)
  stem: per-event embedding 2 -> C1, SparseMaxPool k=4 (stride 4)
  stage s = 1..4 (C = 32/64/128/256 at stride 4/8/16/32, H = 4, D = 32):
      SiteGLABlock (projections in bf16, the per-site recurrence with fp32
      states, output projection, residual, LayerNorm in fp32), then
      SparseMaxPool k=2 for stages 1-3
  dense grids of the stage 2-4 outputs (last event of every site)
  DetectionHead (the YOLOX head's inference path, bf16)
"""
from __future__ import annotations

import math
from typing import Dict, List, Sequence, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _lib
from . import events as E
from .layers import SparseMaxPool
from .scan import sparse_gla_scan

__all__ = ["SiteGLABlock", "DetectionHead", "AsyncSparseGLA", "WindowPlan", "STAGES"]

# (channels, stride) of the four stages
STAGES: Tuple[Tuple[int, int], ...] = ((32, 4), (64, 8), (128, 16), (256, 32))


def grid_of(frame_size: Sequence[int], stride: int) -> Tuple[int, int]:
    """Output grid of 'same'-padded pooling by `stride` (ceil division)."""
    return (-(-int(frame_size[0]) // stride), -(-int(frame_size[1]) // stride))


class SiteGLABlock(nn.Module):
    """Per-site matrix-state GLA over the sites active in one window.

    ``forward(inputs, state, grid_size)`` takes a grouped-events dict whose
    groups are sites of a ``grid_size`` grid (one group per active site, its
    events in time order, groups in increasing (batch, row, column) order --
    the layout SparsePool produces) and ``state`` fp32
    ``[B * Hg * Wg, heads, head_dim, head_dim]``, updated in place.
    """

    def __init__(self, in_channels: int, out_channels: int, heads: int = 4, head_dim: int = 32,
                 gate_normalizer: float = 16.0):
        super().__init__()
        self.in_channels, self.out_channels = in_channels, out_channels
        self.heads, self.head_dim = heads, head_dim
        self.gate_normalizer = gate_normalizer
        hd = heads * head_dim
        self.q_proj = nn.Linear(in_channels, hd, bias=False)
        self.k_proj = nn.Linear(in_channels, hd, bias=False)
        self.v_proj = nn.Linear(in_channels, hd, bias=False)
        self.g_proj = nn.Linear(in_channels, hd, bias=False)
        self.o_proj = nn.Linear(hd, out_channels, bias=False)
        self.res_proj = nn.Linear(in_channels, out_channels, bias=False) if in_channels != out_channels else None
        self.norm = nn.LayerNorm(out_channels)

    def _bf16(self) -> Dict[str, torch.Tensor]:
        """bf16 copies of the projection weights, converted once and again
        only when a weight changes (in-place updates bump its version, a
        move or reassignment changes its storage)."""
        if torch.is_grad_enabled():
            mods = self._proj_modules()
            if any(m.weight.requires_grad for m in mods.values()):
                return {nm: m.weight.to(torch.bfloat16) for nm, m in mods.items()}   # differentiable, not cached
        cache = self.__dict__.get("_bf16_cache")
        if cache is not None and cache[0].valid() and ("r" in cache[1]) == (self._modules.get("res_proj") is not None):
            return cache[1]
        mods = self._proj_modules()
        with torch.no_grad():
            ws = {nm: m.weight.detach().to(torch.bfloat16).contiguous() for nm, m in mods.items()}
            ws["qkvg"] = torch.cat([ws[nm] for nm in ("q", "k", "v", "g")], 0).contiguous()
        names = {"q": "q_proj", "k": "k_proj", "v": "v_proj", "g": "g_proj", "o": "o_proj", "r": "res_proj"}
        self.__dict__["_bf16_cache"] = (_lib.ParamWatch(self, [f"{names[nm]}.weight" for nm in mods]), ws)
        return ws

    def _proj_modules(self) -> Dict[str, nn.Linear]:
        mods = {"q": self.q_proj, "k": self.k_proj, "v": self.v_proj, "g": self.g_proj, "o": self.o_proj}
        if self.res_proj is not None:
            mods["r"] = self.res_proj
        return mods

    def _fused(self, *tensors) -> bool:
        """The one-launch kernels (ssla_site_project / ssla_site_finish) take
        the block: device tensors, no gradient recorded, sizes they cover."""
        hd = self.heads * self.head_dim
        return (all(t.is_cuda for t in tensors) and not (torch.is_grad_enabled() and (
                    any(t.requires_grad for t in tensors) or any(p.requires_grad for p in self.parameters())))
                and self.in_channels % 32 == 0 and hd % 32 == 0
                and self.out_channels in (16, 32, 64, 96, 128, 192, 256))

    def project(self, x: torch.Tensor):
        """q, k, v (bf16 ``[n, H, D]``) and log-gates g (fp32 ``[n, H, D]``)."""
        n = x.shape[0]
        w = self._bf16()
        shp = (n, self.heads, self.head_dim)
        if self._fused(x):
            hd = self.heads * self.head_dim
            x = x.to(torch.float32).contiguous()
            q, k, v = (torch.empty(n, hd, dtype=torch.bfloat16, device=x.device) for _ in range(3))
            g = torch.empty(n, hd, dtype=torch.float32, device=x.device)
            _lib.check(_lib.load().ssla_site_project(
                _lib.ptr(x), n, self.in_channels, _lib.ptr(w["qkvg"]), hd, float(self.gate_normalizer),
                _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(g), _lib.stream_of(x)), "ssla_site_project")
            return q.view(shp), k.view(shp), v.view(shp), g.view(shp)
        xb = x.to(torch.bfloat16)
        q, k, v = (F.linear(xb, w[nm]).view(shp) for nm in ("q", "k", "v"))
        g = F.logsigmoid(F.linear(xb, w["g"]).float()) / self.gate_normalizer
        return q, k, v, g.view(shp)

    def finish(self, o: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
        """LayerNorm(o_proj(o) + residual) in fp32 (projections in bf16)."""
        n = x.shape[0]
        w = self._bf16()
        if self._fused(o, x) and o.dtype == torch.bfloat16:
            hd = self.heads * self.head_dim
            o = o.reshape(n, hd).contiguous()
            x = x.to(torch.float32).contiguous()
            y = torch.empty(n, self.out_channels, dtype=torch.float32, device=x.device)
            _lib.check(_lib.load().ssla_site_finish(
                _lib.ptr(o), n, hd, _lib.ptr(w["o"]), _lib.ptr(x), self.in_channels,
                _lib.ptr(w["r"]) if self.res_proj is not None else None, _lib.ptr(self.norm.weight),
                _lib.ptr(self.norm.bias), float(self.norm.eps), self.out_channels, _lib.ptr(y), _lib.stream_of(x)),
                "ssla_site_finish")
            return y
        y = F.linear(o.reshape(n, -1), w["o"]).float()
        if self.res_proj is not None:
            y = y + F.linear(x.to(torch.bfloat16), w["r"]).float()
        else:
            y = y + x
        return self.norm(y)

    @staticmethod
    def sites(inputs: Dict[str, torch.Tensor], grid_size: Sequence[int]) -> torch.Tensor:
        Hg, Wg = int(grid_size[0]), int(grid_size[1])
        return ((inputs["batch_id"] * Hg + inputs["h"]) * Wg + inputs["w"]).to(torch.int32)

    def forward(self, inputs: Dict[str, torch.Tensor], state: torch.Tensor, grid_size: Sequence[int],
                check: bool = False, mark=None) -> Dict[str, torch.Tensor]:
        """``mark(name)`` (optional) is called after each piece: "project",
        "scan", "finish" (a timing hook; it must not touch the tensors).
        Without it, a block the one-launch kernels take runs as one library
        call (ssla_site_gla_block)."""
        x = inputs["events"].to(torch.float32)
        if mark is None and self._fused(x):
            return self._forward_one_call(inputs, x, state, grid_size, check)
        lengths = inputs["lengths"]
        cu = F.pad(torch.cumsum(lengths, 0), (1, 0))
        q, k, v, g = self.project(x)
        if mark:
            mark("project")
        o = sparse_gla_scan(q, k, v, g, cu, self.sites(inputs, grid_size), state,
                            scale=self.head_dim ** -0.5, check=check)
        if mark:
            mark("scan")
        out = dict(inputs)
        out["events"] = self.finish(o, x)
        if mark:
            mark("finish")
        return out


    def _forward_one_call(self, inputs, x, state, grid_size, check):
        H, D = self.heads, self.head_dim
        if state.dim() != 4 or state.shape[1:] != (H, D, D) or state.dtype != torch.float32 \
                or not state.is_contiguous() or not state.is_cuda:
            raise ValueError(f"SiteGLABlock: state must be contiguous fp32 [n_sites, {H}, {D}, {D}] on the device")
        w = self._bf16()
        n = x.shape[0]
        x = x.contiguous()
        ln, gb, gh, gw = (E._i64(inputs[k]) for k in ("lengths", "batch_id", "h", "w"))
        G = ln.numel()
        lib = _lib.load()
        ws = torch.empty(max(lib.ssla_site_gla_block_workspace_size(n, G, H, D), 1), dtype=torch.uint8,
                         device=x.device)
        y = torch.empty(n, self.out_channels, dtype=torch.float32, device=x.device)
        status = _lib.new_status(x.device) if check and G else None
        _lib.check(lib.ssla_site_gla_block(
            _lib.ptr(x), n, self.in_channels, _lib.ptr(ln), _lib.ptr(gb), _lib.ptr(gh), _lib.ptr(gw), G,
            int(grid_size[0]), int(grid_size[1]), _lib.ptr(state), state.shape[0], H, D, _lib.ptr(w["qkvg"]),
            float(self.gate_normalizer), float(D ** -0.5), _lib.ptr(w["o"]), _lib.ptr(w.get("r")),
            _lib.ptr(self.norm.weight), _lib.ptr(self.norm.bias), float(self.norm.eps), self.out_channels,
            _lib.ptr(y), _lib.ptr(status), _lib.ptr(ws), ws.numel(), _lib.stream_of(x)), "ssla_site_gla_block")
        if status is not None and _lib.read_status(status) != _lib.SSLA_OK:
            raise ValueError(f"SiteGLABlock: site rows must be strictly increasing and inside [0, {state.shape[0]})")
        out = dict(inputs)
        out["events"] = y
        return out


class DetectionHead(nn.Module):
    """The YOLOX head's inference path (reference layers/yolox_head.py:
    100-182 structure, 183-230 forward, 234-256 decode): per level a 1x1
    conv + BatchNorm + SiLU branch for classes and one for boxes, 1x1
    predictions of boxes (4), objectness (1) and classes; outputs ``[B,
    anchors, 5 + classes]`` with box centres ``(t + cell) * stride`` and
    sizes ``exp(t) * stride``.  No losses (the step has no labels)."""

    def __init__(self, num_classes: int, strides: Sequence[int], in_channels: Sequence[int], width: int):
        super().__init__()
        self.num_classes, self.strides = num_classes, tuple(strides)

        def branch(c):
            return nn.Sequential(nn.Conv2d(c, width, 1), nn.BatchNorm2d(width), nn.SiLU())

        self.cls_convs = nn.ModuleList(branch(c) for c in in_channels)
        self.reg_convs = nn.ModuleList(branch(c) for c in in_channels)
        self.cls_preds = nn.ModuleList(nn.Conv2d(width, num_classes, 1) for _ in in_channels)
        self.reg_preds = nn.ModuleList(nn.Conv2d(width, 4, 1) for _ in in_channels)
        self.obj_preds = nn.ModuleList(nn.Conv2d(width, 1, 1) for _ in in_channels)
        prior = -math.log((1 - 0.01) / 0.01)
        for m in list(self.cls_preds) + list(self.obj_preds):
            nn.init.constant_(m.bias, prior)

    @staticmethod
    def _conv1x1(x, conv):
        return F.linear(x, conv.weight.view(conv.out_channels, conv.in_channels), conv.bias)

    def _branch(self, x, seq):
        conv, bn, _ = seq
        y = F.batch_norm(self._conv1x1(x, conv), bn.running_mean, bn.running_var, bn.weight, bn.bias, False, 0.0,
                         bn.eps)
        return F.silu(y)

    def forward(self, xin: List[torch.Tensor], fused: bool = True) -> torch.Tensor:
        """The head on dense maps ``xin`` (``[B, C_l, H_l, W_l]`` per level,
        fp32 or bf16).  On a GPU without autograd (and with ``fused``) all
        levels run as one kernel (ssla_detect_head: the two branches' 1x1
        convolutions as one bf16 GEMM, batch norm and SiLU in fp32, the
        predictions as a second GEMM, the decode); otherwise the module's
        bf16 ops run one by one."""
        if not (fused and xin and xin[0].is_cuda and not torch.is_grad_enabled() and self._kernel_fits(xin)):
            dt = self.cls_convs[0][0].weight.dtype
            return self._forward_eager([x.to(dt) for x in xin])
        prm = self._fused_params()
        B = int(xin[0].shape[0])
        grids = [x.to(torch.float32).contiguous() for x in xin]
        lv = (_lib.HeadLevel * len(grids))()
        for i, x in enumerate(grids):
            w_br, sc, sh, w_p, b_p = prm[i]
            lv[i] = _lib.HeadLevel(_lib.ptr(x), _lib.ptr(w_br), _lib.ptr(sc), _lib.ptr(sh), _lib.ptr(w_p),
                                   _lib.ptr(b_p), int(x.shape[1]), int(x.shape[2]), int(x.shape[3]),
                                   int(self.strides[i]))
        n_out = 5 + self.num_classes
        n_anchor = sum(int(x.shape[2]) * int(x.shape[3]) for x in grids)
        out = torch.empty(B, n_anchor, n_out, dtype=torch.bfloat16, device=grids[0].device)
        width = self.cls_convs[0][0].out_channels
        _lib.check(_lib.load().ssla_detect_head(lv, len(grids), B, n_out, width, _lib.ptr(out),
                                                _lib.stream_of(grids[0])), "ssla_detect_head")
        return out

    def _kernel_fits(self, xin) -> bool:
        """The sizes ssla_detect_head takes: at most SSLA_HEAD_MAX_LEVELS
        levels, 5 + classes <= 16 outputs, a branch width that is a multiple
        of 16 up to 256 and level channels that are multiples of 32; other
        heads (e.g. 80 classes) run the module's ops one by one."""
        width = self.cls_convs[0][0].out_channels
        return (len(xin) <= 4 and 5 + self.num_classes <= 16 and width % 16 == 0 and 0 < width <= 256
                and all(x.dim() == 4 and int(x.shape[1]) % 32 == 0 for x in xin))

    def _fused_params(self):
        """Per level: the two branch convolutions' weights stacked (bf16
        [2 width, C]), batch norm folded with the convolution bias into an
        fp32 scale and shift, and the predictions as one bf16 [16, 2 width]
        matrix (zero where a prediction does not read a branch) with fp32
        biases; recomputed only when a parameter or buffer changes."""
        # the watch covers exactly the tensors read below and the modules
        # that hold them (an in-place update, a replaced parameter or module,
        # or a move invalidates it); comparing a key built by walking the
        # modules cost about 40 µs of host time per call
        cache = self.__dict__.get("_fused_cache")
        if cache is not None and cache[0].valid():
            return cache[1]
        paths = []
        for lvl in range(len(self.strides)):
            for br in ("cls_convs", "reg_convs"):
                paths += [f"{br}.{lvl}.0.{n}" for n in ("weight", "bias")]
                # (batch norm's running statistics change in training
                # without a version bump; its batch counter does not)
                paths += [f"{br}.{lvl}.1.{n}" for n in ("weight", "bias", "running_mean", "running_var",
                                                         "num_batches_tracked")]
            for pr in ("reg_preds", "obj_preds", "cls_preds"):
                paths += [f"{pr}.{lvl}.{n}" for n in ("weight", "bias")]
        levels = []
        with torch.no_grad():
            for lvl in range(len(self.strides)):
                scs, shs, ws = [], [], []
                for seq in (self.cls_convs[lvl], self.reg_convs[lvl]):
                    conv, bn, _ = seq
                    w = conv.weight.view(conv.out_channels, conv.in_channels)
                    s = bn.weight.float() / torch.sqrt(bn.running_var.float() + bn.eps)
                    scs.append(s)
                    shs.append((conv.bias.float() - bn.running_mean.float()) * s + bn.bias.float())
                    ws.append(w.to(torch.bfloat16))
                width = ws[0].shape[0]
                w_br = torch.cat(ws, 0).contiguous()
                w_p = torch.zeros(16, 2 * width, dtype=torch.bfloat16, device=w_br.device)
                b_p = torch.zeros(16, dtype=torch.float32, device=w_br.device)
                reg, obj, cls = self.reg_preds[lvl], self.obj_preds[lvl], self.cls_preds[lvl]
                w_p[0:4, width:] = reg.weight.view(4, width)
                w_p[4:5, width:] = obj.weight.view(1, width)
                w_p[5:5 + self.num_classes, :width] = cls.weight.view(self.num_classes, width)
                b_p[0:4], b_p[4:5], b_p[5:5 + self.num_classes] = reg.bias.float(), obj.bias.float(), cls.bias.float()
                levels.append((w_br, torch.cat(scs).contiguous(), torch.cat(shs).contiguous(), w_p.contiguous(), b_p))
        self.__dict__["_fused_cache"] = (_lib.ParamWatch(self, paths), levels)
        return levels

    def _forward_eager(self, xin: List[torch.Tensor]) -> torch.Tensor:
        # A 1x1 convolution is a linear map of every cell's channels: the
        # maps are taken channel-last ([B * H * W, C], the order the outputs
        # are laid out in) and run as GEMMs; BatchNorm in eval mode and SiLU
        # are elementwise.
        outs = []
        for lvl, x in enumerate(xin):
            B, Cin, Hh, Ww = x.shape
            xc = x.permute(0, 2, 3, 1).reshape(B * Hh * Ww, Cin)
            cls_feat = self._branch(xc, self.cls_convs[lvl])
            reg_feat = self._branch(xc, self.reg_convs[lvl])
            out = torch.cat([self._conv1x1(reg_feat, self.reg_preds[lvl]), self._conv1x1(reg_feat, self.obj_preds[lvl]),
                             self._conv1x1(cls_feat, self.cls_preds[lvl])], 1)
            out = out.view(B, Hh * Ww, -1)
            yv, xv = torch.meshgrid(torch.arange(Hh, device=x.device), torch.arange(Ww, device=x.device),
                                    indexing="ij")
            cell = torch.stack((xv, yv), 2).reshape(1, Hh * Ww, 2).to(out.dtype)
            s = self.strides[lvl]
            out = torch.cat([(out[..., :2] + cell) * s, torch.exp(out[..., 2:4]) * s, out[..., 4:]], -1)
            outs.append(out)
        return torch.cat(outs, 1)


class WindowPlan:
    """The structure of one window (AsyncSparseGLA.plan): the preprocessed
    pixel groups and the pooling plans of the stem and stages 1-3."""
    __slots__ = ("grouped", "pools")

    def __init__(self, grouped: Dict[str, torch.Tensor], pools: List["E.PoolPlan"]):
        self.grouped, self.pools = grouped, pools

    def tensors(self) -> List[torch.Tensor]:
        out = [v for v in self.grouped.values() if isinstance(v, torch.Tensor)]
        for p in self.pools:
            out += p.tensors()
        return out


class AsyncSparseGLA(nn.Module):
    """Stem, four per-site GLA stages with pooling, dense grids and the
    detection head.  ``forward(events, lengths, states)`` runs one window
    (``events`` fp32 ``[B, N, 4]`` as <x, y, t, p> with ``lengths [B]``, the
    reference's collated batch) and updates ``states`` (``init_states``) in
    place; it returns the head output and the per-stage outputs."""

    def __init__(self, frame_size=(240, 304), num_classes: int = 2, stages=STAGES, heads: int = 4,
                 head_dim: int = 32, hot_pixel_thres: int = 50):
        super().__init__()
        self.frame_size = tuple(frame_size)
        self.stages = tuple(stages)
        self.heads, self.head_dim = heads, head_dim
        self.hot_pixel_thres = hot_pixel_thres
        self.grid_sizes = [grid_of(frame_size, s) for _, s in self.stages]
        c1 = self.stages[0][0]
        self.embed = nn.Linear(2, c1, bias=False)
        self.stem_pool = SparseMaxPool(self.frame_size, kernel_size=(self.stages[0][1],) * 2)
        blocks, pools = [], []
        c_prev = c1
        for i, (c, _) in enumerate(self.stages):
            blocks.append(SiteGLABlock(c_prev, c, heads, head_dim))
            if i + 1 < len(self.stages):
                k = self.stages[i + 1][1] // self.stages[i][1]
                pools.append(SparseMaxPool(self.grid_sizes[i], kernel_size=(k, k)))
            c_prev = c
        self.blocks = nn.ModuleList(blocks)
        self.pools = nn.ModuleList(pools)
        self.head_levels = list(range(1, len(self.stages)))          # strides 8, 16, 32
        chans = [self.stages[i][0] for i in self.head_levels]
        self.head = DetectionHead(num_classes, [self.stages[i][1] for i in self.head_levels], chans, chans[-1])
        self.head.to(torch.bfloat16)
        self.head.eval()

    def init_states(self, batch_size: int, device) -> List[torch.Tensor]:
        D = self.head_dim
        return [torch.zeros(batch_size * Hg * Wg, self.heads, D, D, dtype=torch.float32, device=device)
                for Hg, Wg in self.grid_sizes]

    def plan(self, events: torch.Tensor, lengths: torch.Tensor) -> "WindowPlan":
        """Everything of a window that depends only on its events'
        coordinates and times: the pixel groups with their <dt, p> features
        (preprocess_inputs) and the pooling plans and pooled structure of the
        stem and of stages 1-3 (the per-site stages keep the structure).  All
        of the window's reads of device counts happen here, so ``forward``
        with this plan enqueues its work without waiting on the device."""
        gr = E.preprocess_inputs(events, lengths, self.frame_size, self.hot_pixel_thres)
        pools = [self.stem_pool.plan(gr)]
        for pool in self.pools:
            pools.append(pool.plan(pools[-1].structure))
        return WindowPlan(gr, pools)

    def _embed_weight(self) -> torch.Tensor:
        """The embedding weight in bf16, converted again only when it
        changes (differentiable and not cached while it records a
        gradient)."""
        w = self.embed.weight
        if torch.is_grad_enabled() and w.requires_grad:
            return w.to(torch.bfloat16)
        key = (w.data_ptr(), w._version, w.device)
        cache = getattr(self, "_embed_bf16", None)
        if cache is None or cache[0] != key:
            with torch.no_grad():
                cache = (key, w.detach().to(torch.bfloat16))
            self._embed_bf16 = cache
        return cache[1]

    def _embed(self, gr: Dict[str, torch.Tensor]) -> torch.Tensor:
        return F.linear(gr["events"].to(torch.bfloat16), self._embed_weight()).float()

    def _stem_planned(self, plan: "WindowPlan") -> Dict[str, torch.Tensor]:
        """The stem of a planned window: without a gradient to record, the
        embedding runs inside the stem pool's value pass
        (SparsePool.apply_plan_linear, bit-identical); else embedding, then
        pooling."""
        x = plan.grouped["events"]
        w = self._embed_weight()
        if (not torch.is_grad_enabled() and x.is_cuda and x.dim() == 2 and x.shape[1] == 2
                and w.shape[0] % 4 == 0):
            return self.stem_pool.apply_plan_linear(plan.pools[0], x, w)
        return self.stem_pool.apply_plan(plan.pools[0], self._embed(plan.grouped))

    def stem(self, events: torch.Tensor, lengths: torch.Tensor) -> Dict[str, torch.Tensor]:
        gr = E.preprocess_inputs(events, lengths, self.frame_size, self.hot_pixel_thres)
        gr["events"] = self._embed(gr)
        return self.stem_pool(gr)

    def forward(self, events: torch.Tensor, lengths: torch.Tensor, states: List[torch.Tensor], mark=None,
                plan: "WindowPlan" = None):
        """``plan`` (from ``plan`` on this window) supplies the groups and the
        pooled structure, and the call then reads nothing back from the
        device; without it every stage is planned as it comes.  ``mark(name)``
        (optional) is called after each piece ("stem", "s<i>.project" /
        ".scan" / ".finish" / ".pool", "grids", "head"): a timing hook that
        must not touch the tensors."""
        pieces = self._pieces(events, lengths, states, mark, plan)
        while True:
            try:
                next(pieces)
            except StopIteration as done:
                return done.value

    def _pieces(self, events, lengths, states, mark, plan):
        """forward as a generator that pauses after the stem and after each
        of stages 0-2 (block and pooling) and returns (head output, stage
        outputs)."""
        # Without a plan each stage's pooling is planned right after the
        # stage's block is enqueued, so the plan's read of device counts
        # waits while the GPU runs that block.
        x = self.stem(events, lengths) if plan is None else self._stem_planned(plan)
        if mark:
            mark("stem")
        yield
        feats = []
        for i, blk in enumerate(self.blocks):
            x = blk(x, states[i], self.grid_sizes[i], mark=(lambda nm, i=i: mark(f"s{i}.{nm}")) if mark else None)
            feats.append(x)
            if i < len(self.pools):
                x = self.pools[i](x) if plan is None else self.pools[i].apply_plan(plan.pools[i + 1], x["events"])
                if mark:
                    mark(f"s{i}.pool")
                yield
        grids = E.events_to_grids([(feats[i], self.grid_sizes[i], self.stages[i][0]) for i in self.head_levels])
        if mark:
            mark("grids")
        out = self.head(grids)
        if mark:
            mark("head")
        return out, feats

    def _plan_steps(self, events: torch.Tensor, lengths: torch.Tensor):
        """``plan`` as a generator: each step queues its kernels and an
        asynchronous copy of its counts and pauses; resuming waits for those
        counts only (not for the stream), finishes the step and queues the
        next.  Returns the WindowPlan."""
        pending = E.preprocess_enqueue(events, lengths, self.frame_size, self.hot_pixel_thres)
        yield
        gr = E.preprocess_finish(pending)
        pending = self.stem_pool.plan_enqueue(gr)
        yield
        pools = [self.stem_pool.plan_finish(pending)]
        for pool in self.pools:
            pending = pool.plan_enqueue(pools[-1].structure)
            yield
            pools.append(pool.plan_finish(pending))
        return WindowPlan(gr, pools)

    def run(self, windows: Sequence[torch.Tensor], lengths: Sequence[torch.Tensor],
            states: List[torch.Tensor]) -> List[tuple]:
        """``forward`` over consecutive windows with ``states`` carried from
        one to the next (the same results as calling it on each window in
        turn), with no wait that drains the device: while window i's stages
        run, the next window is planned step by step on the same stream,
        each planning step queued ahead of one of window i's stages, so the
        device works on that stage while the host waits for the step's
        counts.  Returns forward's result per window."""
        outs = []
        if len(windows) == 0:
            return outs
        if not self._can_plan_ahead(windows, lengths):
            return [self.forward(w, ln, states) for w, ln in zip(windows, lengths)]
        plan = self.plan(windows[0], lengths[0])
        for i in range(len(windows)):
            steps = self._plan_steps(windows[i + 1], lengths[i + 1]) if i + 1 < len(windows) else None
            nxt = None

            def advance():
                nonlocal steps, nxt
                try:
                    next(steps)
                except StopIteration as done:
                    nxt, steps = done.value, None

            if steps is not None:
                advance()
            pieces = self._pieces(windows[i], lengths[i], states, None, plan)
            while True:
                try:
                    next(pieces)
                except StopIteration as done:
                    outs.append(done.value)
                    break
                if steps is not None:
                    advance()
            while steps is not None:
                advance()
            plan = nxt
        return outs

    def _can_plan_ahead(self, windows, lengths) -> bool:
        """Planning ahead takes the one-call preprocessing and pooling: padded
        fp32 device events and no gradient to record."""
        return (not torch.is_grad_enabled() and all(
            w.is_cuda and w.dim() == 3 and w.size(2) >= 4 and ln.dim() == 1 and ln.size(0) == w.size(0)
            for w, ln in zip(windows, lengths)))
