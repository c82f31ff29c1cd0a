"""Gated linear attention (GLA) forward on MI355X.

Drop-in for the reference's GLA API (haohq19/ssla ``ops/gla``):

* :func:`chunk_gla` -- ``chunk_gla(q, k, v, g, cu_seqlens, scale=None,
  initial_state=None, output_final_state=False) -> (o, final_state)``
  (reference ops/gla/chunk.py:1119-1167).
* :func:`fused_recurrent_gla` (alias :func:`naive_gla_recurrent`) -- the
  recurrent form with the signature of ``naive_gla_recurrent``
  (reference ops/gla/naive.py:50-111).

They run hand-written gfx950 kernels through libssla_amd.so; there is no
CPU or Triton fallback.  The chunk kernels work on 64 keys: other key
widths (multiples of 16 up to 256) run as groups of 64 keys, the last one
zero-padded -- the decay is per key, so each key group is an independent
GLA whose outputs add up (o = sum of the groups' o, ht = the groups' rows).
``chunk_gla`` is differentiable (:class:`ChunkGLAFunction`, backward
``ssla_gla_chunk_bwd`` / ``ssla_gla_chunk_f32_bwd``, run in groups of 64
keys by 64 value columns) for the shapes the chunk kernels take; fp32
inputs run fp32 chunk kernels in both directions.  The recurrent form is
forward-only.  Layouts are the
reference's packed varlen layouts: q, k, g ``[T, H, K]``, v ``[T, H, V]``,
``cu_seqlens`` int64 ``[N + 1]``, states ``[N, H, K, V]`` fp32.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _lib

__all__ = ["chunk_gla", "ChunkGLAFunction", "fused_recurrent_gla", "fused_recurrent_gla_rows", "naive_gla_recurrent",
           "chunk_kernel_supports", "chunk_backward_supports"]


KD = 64   # keys of one chunk-kernel call


def chunk_kernel_supports(q: torch.Tensor, v: torch.Tensor) -> bool:
    """True when the chunk kernels handle this dtype/shape: bf16/fp16 with K
    a multiple of 16 up to 256 (run in groups of 64 keys) and V a multiple
    of 16 up to 256 (the fused MFMA kernels), or fp32 with K and V up to
    256 (the fp32 chunk kernels, ``ssla_gla_chunk_f32_*``)."""
    K, V = q.shape[-1], v.shape[-1]
    if q.dtype == torch.float32:
        return 0 < K <= 256 and 0 < V <= 256
    return (q.dtype in (torch.bfloat16, torch.float16) and K % 16 == 0 and 0 < K <= 256
            and V % 16 == 0 and V <= 256)


VD = 64   # value columns of one chunk-backward call


def chunk_backward_supports(q: torch.Tensor, v: torch.Tensor) -> bool:
    """True when the chunk backward handles this dtype/shape: bf16/fp16 with
    K and V multiples of 16 up to 256, or fp32 with K and V up to 256
    (``ssla_gla_chunk_bwd`` / ``ssla_gla_chunk_f32_bwd`` run 64 keys by 64
    value columns; wider K and V run as groups of those)."""
    return chunk_kernel_supports(q, v)


def _key_groups(K: int):
    """(first key, keys) of the 64-key groups that cover K keys."""
    return [(s, min(KD, K - s)) for s in range(0, K, KD)]


def _keys_of(x: Optional[torch.Tensor], s: int, w: int, dim: int) -> Optional[torch.Tensor]:
    """Keys s .. s + w - 1 of x along ``dim``, zero-padded to KD keys."""
    if x is None:
        return None
    if s == 0 and w == KD and x.shape[dim] == KD:
        return x
    shape = list(x.shape)
    shape[dim] = KD
    out = x.new_zeros(shape)
    out.narrow(dim, 0, w).copy_(x.narrow(dim, s, w))
    return out


def _prep(name, q, k, v, g, cu_seqlens, initial_state, allow_grad=False):
    for t, nm in ((q, "q"), (k, "k"), (v, "v"), (g, "g")):
        if t.dim() != 3:
            raise ValueError(f"{name}: {nm} must be [T, H, D], got shape {tuple(t.shape)}")
    if q.shape != k.shape or q.shape != g.shape:
        raise ValueError(f"{name}: q, k, g shapes differ: {tuple(q.shape)}, {tuple(k.shape)}, "
                         f"{tuple(g.shape)}")
    if v.shape[:2] != q.shape[:2]:
        raise ValueError(f"{name}: v shape {tuple(v.shape)} does not match q {tuple(q.shape)}")
    if not (q.dtype == k.dtype == v.dtype):
        raise TypeError(f"{name}: q, k, v must share a dtype ({q.dtype}, {k.dtype}, {v.dtype})")
    if q.dtype not in _lib.DTYPE_CODE:
        raise TypeError(f"{name}: unsupported dtype {q.dtype}")
    dev = _lib.require_cuda(q, k, v, g, initial_state)
    if not allow_grad:
        _lib.require_no_grad(name, q, k, v, g, initial_state)
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    if g.dtype != torch.float32 and g.dtype != q.dtype:
        g = g.float()
    g = g.contiguous()
    cu = cu_seqlens.to(device=dev, dtype=torch.int64).contiguous()
    h0 = None
    if initial_state is not None:
        h0 = initial_state.to(dtype=torch.float32).contiguous()
    return q, k, v, g, cu, h0


def chunk_gla(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    g: torch.Tensor,
    cu_seqlens: torch.LongTensor,
    scale: Optional[float] = None,
    initial_state: Optional[torch.Tensor] = None,
    output_final_state: bool = False,
) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """Chunked GLA forward (reference ops/gla/chunk.py:1119-1167).

    Returns ``o`` (dtype of v, ``[T, H, V]``) and the fp32 final state
    ``[N, H, K, V]`` when ``output_final_state`` (else None).  Rows of o
    outside ``[cu_seqlens[0], cu_seqlens[-1])`` are unspecified, as in the
    reference (``torch.empty_like``).

    bf16/fp16 inputs with K a multiple of 16 up to 256 run the fused MFMA
    chunk kernels (in groups of 64 keys); fp32 inputs run the fp32 chunk
    kernels (chunks of 64 rows, fp32 products); other shapes run the fused
    recurrent kernel (same math, fp32 state, serial over time).
    """
    if initial_state is not None and initial_state.shape[0] != len(cu_seqlens) - 1:
        raise ValueError(
            f"The number of initial states is expected to be equal to the number of input sequences, "
            f"i.e., {len(cu_seqlens) - 1} rather than {initial_state.shape[0]}."
        )
    if scale is None:
        scale = q.shape[-1] ** -0.5
    grad = torch.is_grad_enabled() and any(
        t is not None and t.requires_grad for t in (q, k, v, g, initial_state))
    q, k, v, g, cu, h0 = _prep("chunk_gla", q, k, v, g, cu_seqlens, initial_state, allow_grad=grad)
    if grad:
        if not chunk_backward_supports(q, v):
            raise NotImplementedError(
                "chunk_gla backward needs K and V multiples of 16 up to 256 (up to 256 for fp32) "
                f"(got {q.dtype}, K={q.shape[-1]}, V={v.shape[-1]})")
        return ChunkGLAFunction.apply(q, k, v, g, float(scale), h0, output_final_state, cu)
    return _chunk_fwd(q, k, v, g, cu, float(scale), h0, output_final_state)


def _chunk_fwd(q, k, v, g, cu, scale, h0, output_final_state):
    T, H, K = q.shape
    V = v.shape[-1]
    N = cu.numel() - 1
    if h0 is not None and h0.shape != (N, H, K, V):
        raise ValueError(f"chunk_gla: initial_state must be {(N, H, K, V)}, got {tuple(h0.shape)}")
    if not chunk_kernel_supports(q, v):
        o = torch.empty_like(v)
        ht = torch.empty(N, H, K, V, device=q.device, dtype=torch.float32) if output_final_state else None
        return _recurrent(q, k, v, g, cu, float(scale), h0, o, ht, None, 0)
    if K == KD or (q.dtype == torch.float32 and K <= KD):
        return _chunk_call(q, k, v, g, cu, scale, h0, output_final_state)
    # key groups: o adds up over the groups (in fp32, rounded once more for
    # 16-bit inputs), ht stacks their key rows
    os, hts = [], []
    for s, w in _key_groups(K):
        o_i, ht_i = _chunk_call(_keys_of(q, s, w, 2), _keys_of(k, s, w, 2), v, _keys_of(g, s, w, 2), cu, scale,
                                _keys_of(h0, s, w, 2), output_final_state)
        os.append(o_i)
        if ht_i is not None:
            hts.append(ht_i[:, :, :w])
    o = os[0] if len(os) == 1 else torch.stack(os).float().sum(0).to(v.dtype)
    return o, (torch.cat(hts, dim=2) if output_final_state else None)


def _chunk_call(q, k, v, g, cu, scale, h0, output_final_state):
    """One ssla_gla_chunk_fwd call (K == KD), or one ssla_gla_chunk_f32_fwd
    call for fp32 inputs (K <= KD)."""
    T, H, K = q.shape
    V = v.shape[-1]
    N = cu.numel() - 1
    o = torch.empty_like(v)
    ht = torch.empty(N, H, K, V, device=q.device, dtype=torch.float32) if output_final_state else None
    lib = _lib.load()
    if q.dtype == torch.float32:
        st = lib.ssla_gla_chunk_f32_fwd(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(g), _lib.ptr(cu), N, T, H, K,
                                        V, float(scale), _lib.ptr(h0), _lib.ptr(o), _lib.ptr(ht), _lib.stream_of(q))
        _lib.check(st, "ssla_gla_chunk_f32_fwd")
        return o, ht
    ws_bytes = lib.ssla_gla_chunk_workspace_size(N, T, H, K, V)
    ws = torch.empty(ws_bytes, device=q.device, dtype=torch.uint8) if ws_bytes else None
    st = lib.ssla_gla_chunk_fwd(
        _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(g), _lib.DTYPE_CODE[g.dtype],
        _lib.ptr(cu), N, T, H, K, V, float(scale), _lib.ptr(h0), _lib.ptr(o), _lib.ptr(ht),
        _lib.DTYPE_CODE[q.dtype], _lib.ptr(ws), ws_bytes, _lib.stream_of(q))
    _lib.check(st, "ssla_gla_chunk_fwd")
    return o, ht


class ChunkGLAFunction(torch.autograd.Function):
    """Forward ``ssla_gla_chunk_fwd``, backward ``ssla_gla_chunk_bwd``
    (reference ChunkGLAFunction, ops/gla/chunk.py:1056-1116): the backward
    recomputes every chunk's state from q, k, v, g and h0 instead of saving
    them.  Returns dq, dk, dv in the input dtype, dg in g's dtype and dh0
    (fp32) when an initial state was given."""

    @staticmethod
    def forward(ctx, q, k, v, g, scale, initial_state, output_final_state, cu_seqlens):
        o, ht = _chunk_fwd(q, k, v, g, cu_seqlens, scale, initial_state, output_final_state)
        ctx.save_for_backward(q, k, v, g, initial_state, cu_seqlens)
        ctx.scale = scale
        return o, ht

    @staticmethod
    def backward(ctx, do, dht):
        q, k, v, g, h0, cu = ctx.saved_tensors
        do = do.to(v.dtype).contiguous()
        dht = None if dht is None else dht.to(torch.float32).contiguous()
        V = v.shape[-1]
        if V <= VD:
            dq, dk, dv, dg, dh0 = _bwd_keys(q, k, v, g, h0, cu, do, dht, ctx.scale)
            return dq, dk, dv, dg, None, dh0, None, None
        # value groups: each state column evolves on its own (the decay acts
        # on keys), so the V groups are independent GLAs sharing q, k, g;
        # their dq, dk, dg add up (in fp32, rounded once), dv and dh0 are the
        # groups' columns
        parts = [_bwd_keys(q, k, v[..., s:s + w].contiguous(), g, None if h0 is None else h0[..., s:s + w].contiguous(),
                           cu, do[..., s:s + w].contiguous(), None if dht is None else dht[..., s:s + w].contiguous(),
                           ctx.scale)
                 for s, w in _value_groups(V)]
        add = lambda i, like: torch.stack([p[i].float() for p in parts]).sum(0).to(like.dtype)   # noqa: E731
        dh0 = torch.cat([p[4] for p in parts], dim=3) if h0 is not None else None
        return (add(0, q), add(1, k), torch.cat([p[2] for p in parts], dim=2), add(3, g), None, dh0, None, None)


def _value_groups(V: int):
    """(first column, columns) of the 64-column groups that cover V."""
    return [(s, min(VD, V - s)) for s in range(0, V, VD)]


def _bwd_keys(q, k, v, g, h0, cu, do, dht, scale):
    """dq, dk, dv, dg, dh0 of one value group (V <= VD): one
    ssla_gla_chunk_bwd call per group of 64 keys."""
    K = q.shape[-1]
    if K == KD or (q.dtype == torch.float32 and K <= KD):
        return _chunk_bwd_call(q, k, v, g, h0, cu, do, dht, scale)
    # key groups: each group's gradients are its keys' rows; dv adds up
    parts = [_chunk_bwd_call(_keys_of(q, s, w, 2), _keys_of(k, s, w, 2), v, _keys_of(g, s, w, 2),
                             _keys_of(h0, s, w, 2), cu, do, _keys_of(dht, s, w, 2), scale)
             for s, w in _key_groups(K)]
    widths = [w for _, w in _key_groups(K)]
    cat = lambda i, dim: torch.cat([p[i].narrow(dim, 0, w) for p, w in zip(parts, widths)], dim=dim)   # noqa: E731
    dv = parts[0][2] if len(parts) == 1 else torch.stack([p[2] for p in parts]).float().sum(0).to(v.dtype)
    dh0 = cat(4, 2) if h0 is not None else None
    return cat(0, 2), cat(1, 2), dv, cat(3, 2), dh0


def _chunk_bwd_call(q, k, v, g, h0, cu, do, dht, scale):
    """One ssla_gla_chunk_bwd call (K == KD), or one ssla_gla_chunk_f32_bwd
    call for fp32 inputs: dq, dk, dv, dg, dh0."""
    T, H, K = q.shape
    V = v.shape[-1]
    N = cu.numel() - 1
    dq, dk = torch.empty_like(q), torch.empty_like(k)
    dv, dg = torch.empty_like(v), torch.empty_like(g)
    dh0 = torch.empty_like(h0) if h0 is not None else None
    lib = _lib.load()
    if q.dtype == torch.float32:
        g32 = g if g.dtype == torch.float32 else g.float()
        dg32 = dg if dg.dtype == torch.float32 else torch.empty_like(g32)
        ws_bytes = lib.ssla_gla_chunk_f32_bwd_workspace_size(N, T, H)
        ws = torch.empty(max(ws_bytes, 1), device=q.device, dtype=torch.uint8)
        st = lib.ssla_gla_chunk_f32_bwd(
            _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(g32), _lib.ptr(cu), N, T, H, K, V, float(scale),
            _lib.ptr(h0), _lib.ptr(do), _lib.ptr(dht), _lib.ptr(dq), _lib.ptr(dk), _lib.ptr(dv), _lib.ptr(dg32),
            _lib.ptr(dh0), _lib.ptr(ws), ws_bytes, _lib.stream_of(q))
        _lib.check(st, "ssla_gla_chunk_f32_bwd")
        if dg32 is not dg:
            dg.copy_(dg32)
        return dq, dk, dv, dg, dh0
    ws_bytes = lib.ssla_gla_chunk_bwd_workspace_size(N, T, H, K, V)
    ws = torch.empty(max(ws_bytes, 1), device=q.device, dtype=torch.uint8)
    st = lib.ssla_gla_chunk_bwd(
        _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(g), _lib.DTYPE_CODE[g.dtype], _lib.ptr(cu), N, T, H, K, V,
        float(scale), _lib.ptr(h0), _lib.ptr(do), _lib.ptr(dht), _lib.ptr(dq), _lib.ptr(dk), _lib.ptr(dv),
        _lib.ptr(dg), _lib.ptr(dh0), _lib.DTYPE_CODE[q.dtype], _lib.ptr(ws), ws_bytes, _lib.stream_of(q))
    _lib.check(st, "ssla_gla_chunk_bwd")
    return dq, dk, dv, dg, dh0


def _recurrent(q, k, v, g, cu, scale, h0, o, ht, state_idx, n_rows, status=None):
    T, H, K = q.shape
    V = v.shape[-1]
    N = cu.numel() - 1
    lib = _lib.load()
    ws_bytes = lib.ssla_gla_recurrent_workspace_size(N, T, H, K, V)
    ws = torch.empty(ws_bytes, device=q.device, dtype=torch.uint8) if ws_bytes else None
    st = lib.ssla_gla_recurrent_fwd(
        _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(g), _lib.DTYPE_CODE[g.dtype],
        _lib.ptr(cu), N, T, H, K, V, float(scale), _lib.ptr(h0), _lib.ptr(o), _lib.ptr(ht),
        _lib.ptr(state_idx), int(n_rows), _lib.ptr(status), _lib.DTYPE_CODE[q.dtype], _lib.ptr(ws), ws_bytes,
        _lib.stream_of(q))
    _lib.check(st, "ssla_gla_recurrent_fwd")
    return o, ht


def fused_recurrent_gla(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    g: torch.Tensor,
    cu_seqlens: torch.LongTensor,
    scale: Optional[float] = None,
    initial_state: Optional[torch.Tensor] = None,
    output_final_state: bool = False,
) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """Recurrent GLA forward with the signature and semantics of
    ``naive_gla_recurrent`` (reference ops/gla/naive.py:50-111):
    ``S_t = exp(g_t) * S_{t-1} + k_t v_t^T``, ``o_t = (scale q_t) . S_t``;
    o has q's dtype, the final state is fp32.  As the reference concatenates
    the outputs of its sequences (naive.py:106), o holds the rows
    ``cu_seqlens[0]:cu_seqlens[-1]``.  Finding them reads the two bounds
    back, one host sync per call (as the reference's ``.item()`` calls do),
    unless ``cu_seqlens`` is a CPU tensor; :func:`fused_recurrent_gla_rows`
    makes no sync and returns all T rows (for callers whose sequences cover
    the batch, e.g. under HIP graph capture)."""
    if scale is None:
        scale = q.shape[-1] ** -0.5
    q, k, v, g, cu, h0 = _prep("fused_recurrent_gla", q, k, v, g, cu_seqlens, initial_state)
    T, H, K = q.shape
    V = v.shape[-1]
    N = cu.numel() - 1
    if h0 is not None and h0.shape != (N, H, K, V):
        raise ValueError(f"fused_recurrent_gla: initial_state must be {(N, H, K, V)}, "
                         f"got {tuple(h0.shape)}")
    o = torch.empty(T, H, V, device=q.device, dtype=q.dtype)
    ht = torch.empty(N, H, K, V, device=q.device, dtype=torch.float32) if output_final_state else None
    o, ht = _recurrent(q, k, v, g, cu, float(scale), h0, o, ht, None, 0)
    lo, hi = (int(x) for x in cu_seqlens[[0, -1]].tolist()) if N > 0 else (0, 0)
    if (lo, hi) != (0, T):
        o = o[lo:hi]
    return o, ht


def fused_recurrent_gla_rows(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    g: torch.Tensor,
    cu_seqlens: torch.LongTensor,
    scale: Optional[float] = None,
    initial_state: Optional[torch.Tensor] = None,
    output_final_state: bool = False,
) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """:func:`fused_recurrent_gla` without the host sync: o has all T rows
    (rows outside every sequence are unspecified), so nothing is read back
    and the call can be captured in a HIP graph."""
    if scale is None:
        scale = q.shape[-1] ** -0.5
    q, k, v, g, cu, h0 = _prep("fused_recurrent_gla", q, k, v, g, cu_seqlens, initial_state)
    T, H, K = q.shape
    V = v.shape[-1]
    N = cu.numel() - 1
    if h0 is not None and h0.shape != (N, H, K, V):
        raise ValueError(f"fused_recurrent_gla: initial_state must be {(N, H, K, V)}, "
                         f"got {tuple(h0.shape)}")
    o = torch.empty(T, H, V, device=q.device, dtype=q.dtype)
    ht = torch.empty(N, H, K, V, device=q.device, dtype=torch.float32) if output_final_state else None
    return _recurrent(q, k, v, g, cu, float(scale), h0, o, ht, None, 0)


naive_gla_recurrent = fused_recurrent_gla
