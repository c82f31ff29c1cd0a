"""CPU emulation of the reference's chunked GLA forward with its rounding
points (test infrastructure only: no product path imports this file).

The fp64 recurrence in ``oracle.gla_recurrent`` is the exact answer.  This
module computes what the reference's Triton pipeline returns for bf16
inputs, so that a test can hold the HIP kernel to "at least as close to the
exact answer as the reference itself", rather than to a band measured on
the kernel.  It follows, step for step:

* ``chunk_local_cumsum`` (reference ops/utils/cumsum.py:61-90): G is the
  chunk-local inclusive cumsum of g in fp32 (``allow_tf32=False``).
* ``chunk_fwd_kernel_h`` (ops/common/chunk_h.py:60-128) with
  ``states_in_fp32=False`` (ops/gla/chunk.py:933): the state S is fp32; the
  state entering chunk c is stored as bf16 (``h``); then
  ``S <- S * exp(G_last)`` and ``S += bf16(k * exp(G_last - G))^T v`` (a
  bf16 dot, fp32 sums).  ht is the fp32 S.
* ``chunk_gla_fwd_A_kernel_intra_sub_inter`` (ops/gla/chunk.py:33-98): for
  16-row sub-chunks i > j, with gn = G at the first row of sub-chunk i,
  ``A_ij = (q_i exp(G_i - gn) scale) (k_j exp(gn - G_j))^T`` in fp32
  operands, which Triton's ``tl.dot`` rounds to TF32 (its default,
  ``allow_tf32=True``; round to nearest, ties away, 10 mantissa bits).
* ``chunk_gla_fwd_A_kernel_intra_sub_intra`` (ops/gla/chunk.py:112-176):
  the diagonal sub-chunks as an fp32 elementwise sum
  ``sum_k q k exp(G_r - G_c) scale`` for c <= r.
* ``chunk_gla_fwd_kernel_o`` (ops/gla/chunk.py:189-249):
  ``q' = bf16(q scale)``, ``qg = bf16(q' exp(G))``,
  ``o = qg bf16(h) + bf16(tril(A)) v`` (bf16 dots, fp32 sums), stored as
  bf16.

Chunks are 64 rows restarting at every sequence start (BT = 64, BC = 16).
"""
from __future__ import annotations

import numpy as np

BT, BC = 64, 16


def bf16(x):
    """Round fp32 values to bf16 (nearest, ties to even), returned as fp32."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    r = ((b >> 16) & 1) + np.uint32(0x7FFF)
    return ((b + r) & np.uint32(0xFFFF0000)).view(np.float32)


def tf32(x):
    """Round fp32 values to TF32 (10 mantissa bits; nearest, ties away from
    zero, as the cvt.rna conversion Triton uses for tf32 dots)."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    return ((b + np.uint32(0x1000)) & np.uint32(0xFFFFE000)).view(np.float32)


def _same(x):
    return np.asarray(x, dtype=np.float32)


def _chunk(q, k, v, G, S, scale, bf16=bf16, tf32=tf32):
    """One chunk of n <= 64 rows for all heads: q, k, G [n, H, K], v [n, H,
    V] fp32 (q, k, v bf16 values), S [H, K, V] fp32 entering state.
    Returns (o [n, H, V] as bf16 values, the state after the chunk)."""
    n, H, K = q.shape
    f = np.float32
    qh, kh, vh, Gh = (np.transpose(x, (1, 0, 2)) for x in (q, k, v, G))   # [H, n, D]
    # intra-chunk A (fp32 [H, n, n])
    A = np.zeros((H, n, n), dtype=f)
    for i in range(0, n, BC):
        ie = min(i + BC, n)
        gn = Gh[:, i:i + 1, :]                                     # [H, 1, K]
        qg = (qh[:, i:ie] * np.exp(Gh[:, i:ie] - gn) * f(scale)).astype(f)
        for j in range(0, i, BC):
            je = j + BC
            kg = (kh[:, j:je] * np.exp(gn - Gh[:, j:je])).astype(f)
            A[:, i:ie, j:je] = np.matmul(tf32(qg), np.transpose(tf32(kg), (0, 2, 1)))
        # diagonal sub-chunk: elementwise fp32 sums
        d = (qh[:, i:ie, None, :] * kh[:, None, i:ie, :]
             * np.exp(Gh[:, i:ie, None, :] - Gh[:, None, i:ie, :])).astype(f)
        blk = d.sum(-1, dtype=f) * f(scale)
        A[:, i:ie, i:ie] = np.tril(blk)
    A = np.tril(A)
    # output: bf16 operands, fp32 sums
    qs = bf16(qh * f(scale))
    qg = bf16(qs * np.exp(Gh))
    o = np.matmul(qg, bf16(S)) + np.matmul(bf16(A), vh)
    # state after the chunk
    g_last = Gh[:, n - 1:n, :]                                     # [H, 1, K]
    kd = bf16(kh * np.exp(g_last - Gh))                            # [H, n, K]
    S = S * np.exp(g_last[:, 0, :])[:, :, None] + np.matmul(np.transpose(kd, (0, 2, 1)), vh)
    return np.transpose(bf16(o), (1, 0, 2)), S.astype(f)


def chunk_gla(q, k, v, g, cu_seqlens, scale, h0=None, exact=False):
    """o [T, H, V] (bf16 values in fp32) and ht [N, H, K, V] fp32 as the
    reference's chunk pipeline computes them for bf16 q, k, v and fp32 g.
    ``exact=True`` drops every rounding step (the same algorithm in fp32),
    which must then equal the recurrence up to fp32 sums: the check that
    pins the chunk algebra of this emulation."""
    rb, rt = (_same, _same) if exact else (bf16, tf32)
    q, k, v = (rb(np.asarray(x, np.float32)) for x in (q, k, v))
    g = np.asarray(g, np.float32)
    cu = np.asarray(cu_seqlens, np.int64)
    T, H, K = q.shape
    V = v.shape[-1]
    N = cu.size - 1
    o = np.zeros((T, H, V), np.float32)
    ht = np.zeros((N, H, K, V), np.float32)
    for s in range(N):
        bos, eos = int(cu[s]), int(cu[s + 1])
        S = np.zeros((H, K, V), np.float32) if h0 is None else np.asarray(h0[s], np.float32).copy()
        for c0 in range(bos, eos, BT):
            c1 = min(c0 + BT, eos)
            G = np.cumsum(g[c0:c1], axis=0, dtype=np.float32)
            o[c0:c1], S = _chunk(q[c0:c1], k[c0:c1], v[c0:c1], G, S, scale, rb, rt)
        ht[s] = S
    return o, ht
