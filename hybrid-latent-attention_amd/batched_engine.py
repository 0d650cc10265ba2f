"""The HF rolling engine's attention over [latent history rows || exact current chunk]
(``hla/latent/batched_engine.py:154-182``, ``mixed_attention``) with the latent history on the MI355X K-hop kernels.

One softmax spans the current chunk's exact keys and every history block's latent rows. Written as an LSE merge of
its parts, which is the same softmax: the current chunk (per-head causal attention over the RoPE'd q / k of the
chunk, the standard attention the reference also computes with dense torch ops) gives ``(o_c, lse_c)``; each history
block gives ``(z_k, lse_k)`` from ``history_gemm.causal_history_gemm`` (bf16 MFMA kernels, differentiable in the
latent query and the packed rows) with the block's ``[B, N]`` mask shared by the chunk's queries; then
``out = w_c o_c + (sum_k w_k z_k) @ B`` with ``w = exp(lse - logsumexp(all lse))``. The reference rounds the joint
probabilities to bf16 before its products; here the parts are normalized in fp32 inside the kernels and z is
rounded once to bf16, so outputs agree within bf16 rounding.
"""
from __future__ import annotations

import math

import torch

from . import history_gemm


def rotate_half(x):
    """``[-x2, x1]`` of the two halves of the last dimension (``hla/latent/register.py:14-16``)."""
    x1, x2 = x.chunk(2, -1)
    return torch.cat((-x2, x1), -1)


def apply_rope(x, cos, sin):
    """``x cos + rotate_half(x) sin`` with cos / sin ``[B, n, d]`` broadcast over the heads of ``x [B, H, n, d]``
    (``hla/latent/register.py:19-20``)."""
    return x * cos.unsqueeze(1) + rotate_half(x) * sin.unsqueeze(1)


def _history_block(qc, ck, cv, mask, scale):
    """z ``[B, H, n, r]`` and lse ``[B, H, n]`` of the latent query qc ``[B, H, n, r]`` over the rows ck / cv
    ``[B, N, r]`` that mask ``[B, N]`` shows to every query of the chunk."""
    B, H, n, r = qc.shape
    q = qc.transpose(1, 2).contiguous()                       # [B, n, H, r]: token-linear rows for the MFMA kernel
    m = mask[:, None, :].expand(B, n, mask.shape[1]).contiguous()
    z, lse = history_gemm.causal_history_gemm(q, ck, cv, m, scale, precision='bf16')
    return z.transpose(1, 2), lse


def mixed_attention(sl, loop, q, k, v, cos, sin, valid, blocks, masks):
    """``hla/latent/batched_engine.py:154-182``: q, k, v ``[B, 16, n, head_dim]`` of the chunk, cos / sin ``[B, n,
    head_dim]``, valid ``[B, n]``, ``blocks`` the packed history rows ``[B, N_k, 1536]`` and ``masks`` their ``[B,
    N_k]`` visibility. ``sl`` is the layer's latent module (``register.LatentLayer``: ``query``, ``fields``,
    ``readers``, ``head_dim``). Returns ``[B, 16, n, head_dim]`` in v.dtype. Valid queries see the chunk's valid keys
    up to their own position; an invalid query sees every key of the chunk (its row stays finite and is never read)."""
    scale = 1 / math.sqrt(sl.head_dim)
    qrot, krot = apply_rope(q, cos, sin), apply_rope(k, cos, sin)
    n = valid.shape[1]
    visible = valid[:, None, None, :] & torch.ones(n, n, device=q.device, dtype=torch.bool).tril()
    visible = visible | ~valid[:, None, :, None]
    with torch.autocast(q.device.type, enabled=False):
        current = (qrot.float() @ krot.float().transpose(-1, -2).contiguous()) * scale
        current = current.masked_fill(~visible, float('-inf'))
        lse_c = torch.logsumexp(current, -1)                  # [B, 16, n]
        o_c = torch.softmax(current, -1) @ v.float()
    if not blocks:
        return o_c.to(v.dtype)
    qc = sl.query(loop, q, cos, sin)
    parts = []
    for block, mask in zip(blocks, masks):
        ck, cv = sl.fields(loop, block)
        parts.append(_history_block(qc, ck, cv, mask, scale))
    with torch.autocast(q.device.type, enabled=False):
        total = torch.logsumexp(torch.stack([lse_c] + [lse for _, lse in parts]), 0)
        out = torch.exp(lse_c - total)[..., None] * o_c
        z = None
        for zk, lse in parts:                                  # rows without a visible key carry lse = -inf: weight 0
            wz = torch.exp(lse - total)[..., None] * zk.float()
            z = wz if z is None else z + wz
        _, B_read, _ = sl.readers(loop)
        out = out + torch.einsum('bhir,hrd->bhid', z, B_read.float())
    return out.to(v.dtype)
