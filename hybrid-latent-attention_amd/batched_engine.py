"""The HF rolling engine's attention over [latent history rows || exact current chunk]
(``hla/latent/batched_engine.py:154-182``, ``mixed_attention``) on MI355X kernels, differentiable.

One softmax spans the current chunk's exact keys and every history block's latent rows. Written as an LSE merge of
its parts, which is the same softmax: the current chunk (per-head causal attention over the RoPE'd q / k of the
chunk with the reference's visibility rule) gives ``(o_c, lse_c)`` from the HIP chunk kernels
(``hla_s6_hf_chunk_forward`` / ``_backward``); each history block gives ``(z_k, lse_k)`` from
``history_gemm.causal_history_gemm`` (bf16 MFMA kernels, differentiable in the latent query and the packed rows)
with the block's ``[B, N]`` mask shared by the chunk's queries; then ``out = w_c o_c + (sum_k w_k z_k) @ B`` with
``w = exp(lse - logsumexp(all lse))``. The reference rounds the joint probabilities to bf16 before its products;
here the parts are normalized in fp32 inside the kernels and z is rounded once to bf16, so outputs agree within
bf16 rounding.
"""
from __future__ import annotations

import math

import torch
from torch.autograd.function import once_differentiable

from . import _lib, history_gemm, s6_ops


def rotate_half(x):
    """``[-x2, x1]`` of the two halves of the last dimension (``hla/latent/register.py:14-16``)."""
    x1, x2 = x.chunk(2, -1)
    return torch.cat((-x2, x1), -1)


def apply_rope(x, cos, sin):
    """``x cos + rotate_half(x) sin`` with cos / sin ``[B, n, d]`` broadcast over the heads of ``x [B, H, n, d]``
    (``hla/latent/register.py:19-20``)."""
    return x * cos.unsqueeze(1) + rotate_half(x) * sin.unsqueeze(1)


class _CurrentChunk(torch.autograd.Function):
    """Per-head softmax of the chunk's RoPE'd queries over its RoPE'd keys (``batched_engine.py:156-162``): q, k, v
    ``[B, 16, n, 128]``, valid ``[B, n]``; returns o ``[B, 16, n, 128]`` fp32 and lse ``[B, 16, n]`` fp32. bf16 MFMA
    operands, fp32 softmax and accumulation; backward on the HIP kernels (dq, dk, dv fp32)."""

    @staticmethod
    def forward(ctx, q, k, v, valid, scale):
        B, H, n, D = q.shape
        qb, kb, vb = (t.to(torch.bfloat16).contiguous() for t in (q, k, v))
        v8 = valid.to(torch.bool).contiguous().view(torch.uint8)
        o = torch.empty(B, H, n, D, dtype=torch.float32, device=q.device)
        lse = torch.empty(B, H, n, dtype=torch.float32, device=q.device)
        st = _lib.stream(q.device)
        _lib.call('hla_s6_hf_chunk_forward', _lib.ptr(qb), *qb.stride()[:3], _lib.ptr(kb), *kb.stride()[:3],
                  _lib.ptr(vb), *vb.stride()[:3], _lib.ptr(v8), v8.stride(0), B, H, n, D, float(scale), _lib.ptr(o),
                  *o.stride()[:3], _lib.ptr(lse), lse.stride(0), lse.stride(1), st)
        ctx.save_for_backward(qb, kb, vb, v8, o, lse)
        ctx.settings = (float(scale), q.dtype, k.dtype, v.dtype)
        return o, lse

    @staticmethod
    @once_differentiable
    def backward(ctx, do, dlse):
        qb, kb, vb, v8, o, lse = ctx.saved_tensors
        scale, q_dtype, k_dtype, v_dtype = ctx.settings
        B, H, n, D = qb.shape
        do = torch.zeros_like(o) if do is None else do.to(torch.float32).contiguous()
        dl = None if dlse is None else dlse.to(torch.float32).contiguous()
        delta = torch.empty_like(lse)
        dq, dk, dv = (torch.empty(B, H, n, D, dtype=torch.float32, device=qb.device) for _ in range(3))
        _lib.call('hla_s6_hf_chunk_backward', _lib.ptr(qb), *qb.stride()[:3], _lib.ptr(kb), *kb.stride()[:3],
                  _lib.ptr(vb), *vb.stride()[:3], _lib.ptr(v8), v8.stride(0), B, H, n, D, scale, _lib.ptr(o),
                  *o.stride()[:3], _lib.ptr(lse), lse.stride(0), lse.stride(1), _lib.ptr(do), *do.stride()[:3],
                  _lib.ptr(dl), _lib.ptr(delta), _lib.ptr(dq), _lib.ptr(dk), _lib.ptr(dv), *dq.stride()[:3],
                  _lib.stream(qb.device))
        return dq.to(q_dtype), dk.to(k_dtype), dv.to(v_dtype), None, None


def current_chunk_attention(q, k, v, valid, scale):
    """``(o [B, 16, n, 128] fp32, lse [B, 16, n] fp32)`` of the chunk's exact attention (RoPE'd q / k, valid
    ``[B, n]``) on the HIP chunk kernels, differentiable in q, k and v."""
    s6_ops._dev(q, k, v, valid)
    B, H, n, D = q.shape
    if H != 16 or D != 128 or k.shape != q.shape or v.shape != q.shape or tuple(valid.shape) != (B, n):
        raise ValueError(f'the chunk kernels take q / k / v [B, 16, n, 128] and valid [B, n] (got {tuple(q.shape)}, '
                         f'{tuple(k.shape)}, {tuple(v.shape)}, {tuple(valid.shape)})')
    return _CurrentChunk.apply(q, k, v, valid, float(scale))


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
    with torch.autocast(q.device.type, enabled=False):
        o_c, lse_c = current_chunk_attention(qrot, krot, v, valid, scale)
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
