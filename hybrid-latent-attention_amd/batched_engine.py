"""The HF rolling engine's attention over [latent history rows || exact current chunk]
(``hla/latent/batched_engine.py:154-182``, ``mixed_attention``) on MI355X kernels, differentiable.

One softmax spans the current chunk's exact keys and every history block's latent rows. Written as an LSE merge of
its parts, which is the same softmax: the current chunk (per-head causal attention over the chunk's q / k, RoPE'd
by one HIP launch for both, ``hla_s6_rope_rows_forward`` / ``_backward``, with the reference's visibility rule) gives
``(o_c, lse_c)`` from the HIP chunk kernels (``hla_s6_hf_chunk_forward`` / ``_backward``); each history block gives ``(z_k, lse_k)`` from
``history_gemm.causal_history_gemm`` (bf16 MFMA kernels, differentiable in the latent query and the packed rows)
with the block's ``[B, N]`` mask shared by the chunk's queries; then ``out = w_c o_c + bf16(sum_k w_k z_k) @ B``
with ``w = exp(lse - logsumexp(all lse))`` in one HIP launch (``hla_s6_mixed_merge_forward``; its backward
``hla_s6_mixed_merge_backward`` gives the gradients of every part). The reference rounds the joint probabilities to
bf16 before its products; here the parts are normalized in fp32 inside the kernels and z is rounded once to bf16, so
outputs agree within bf16 rounding. The kernels take bf16 operands: float32 q / k / v and latent queries are rounded
to bf16 once on entry (the reference computes in the input dtype), which keeps every result within the same bf16
rounding of the float32 reference.
"""
from __future__ import annotations

import ctypes
import math

import torch
from torch.autograd.function import once_differentiable

from . import _lib, history_gemm, s6_ops

# History blocks per call of the merge kernel
MAX_BLOCKS = 8


def rotate_half(x):
    """``[-x2, x1]`` of the two halves of the last dimension (``hla/latent/register.py:14-16``)."""
    x1, x2 = x.chunk(2, -1)
    return torch.cat((-x2, x1), -1)


def apply_rope(x, cos, sin):
    """``x cos + rotate_half(x) sin`` with cos / sin ``[B, n, d]`` broadcast over the heads of ``x [B, H, n, d]``
    (``hla/latent/register.py:19-20``)."""
    return x * cos.unsqueeze(1) + rotate_half(x) * sin.unsqueeze(1)


def _chunk_forward(qb, kb, vb, v8, scale):
    """o ``[B, 16, n, 128]`` fp32 and lse ``[B, 16, n]`` of the HIP chunk kernel for bf16 qb / kb / vb."""
    B, H, n, D = qb.shape
    o = torch.empty(B, H, n, D, dtype=torch.float32, device=qb.device)
    lse = torch.empty(B, H, n, dtype=torch.float32, device=qb.device)
    _lib.call('hla_s6_hf_chunk_forward', _lib.ptr(qb), *qb.stride()[:3], _lib.ptr(kb), *kb.stride()[:3],
              _lib.ptr(vb), *vb.stride()[:3], _lib.ptr(v8), v8.stride(0), B, H, n, D, float(scale), _lib.ptr(o),
              *o.stride()[:3], _lib.ptr(lse), lse.stride(0), lse.stride(1), _lib.stream(qb.device))
    return o, lse


def _chunk_backward(qb, kb, vb, v8, o, lse, do, dlse, scale):
    """fp32 dq, dk, dv of the chunk kernel's operands for the cotangents do (None = 0) and dlse (None = 0)."""
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
    return dq, dk, dv


class _CurrentChunk(torch.autograd.Function):
    """Per-head softmax of the chunk's RoPE'd queries over its RoPE'd keys (``batched_engine.py:156-162``): q, k, v
    ``[B, 16, n, 128]``, valid ``[B, n]``; returns o ``[B, 16, n, 128]`` fp32 and lse ``[B, 16, n]`` fp32. bf16 MFMA
    operands, fp32 softmax and accumulation; backward on the HIP kernels (dq, dk, dv fp32)."""

    @staticmethod
    def forward(ctx, q, k, v, valid, scale):
        qb, kb, vb = (t.to(torch.bfloat16).contiguous() for t in (q, k, v))
        v8 = valid.to(torch.bool).contiguous().view(torch.uint8)
        o, lse = _chunk_forward(qb, kb, vb, v8, scale)
        ctx.save_for_backward(qb, kb, vb, v8, o, lse)
        ctx.settings = (float(scale), q.dtype, k.dtype, v.dtype)
        return o, lse

    @staticmethod
    @once_differentiable
    def backward(ctx, do, dlse):
        qb, kb, vb, v8, o, lse = ctx.saved_tensors
        scale, q_dtype, k_dtype, v_dtype = ctx.settings
        dq, dk, dv = _chunk_backward(qb, kb, vb, v8, o, lse, do, dlse, scale)
        return dq.to(q_dtype), dk.to(k_dtype), dv.to(v_dtype), None, None


def _trig(cos, sin, B, n, D):
    """cos / sin broadcast to ``[B, n, D]`` with one layout for both (16-byte rows): bf16 when both tables are (torch
    then rotates in bf16), else fp32 (torch's precision for a bf16 x with fp32 or fp16 tables)."""
    dt = torch.bfloat16 if cos.dtype == sin.dtype == torch.bfloat16 else torch.float32
    c, s = (t.to(dt).expand(B, n, D) for t in (cos, sin))
    if (c.stride() != s.stride() or c.stride(-1) != 1 or c.stride(0) % 8 or c.stride(1) % 8 or c.data_ptr() % 16
            or s.data_ptr() % 16):
        c, s = c.contiguous(), s.contiguous()
    return c, s


def _rope_call(name, xs, ys, c, s):
    B, H, n, D = ys[0].shape
    _lib.call(name, len(xs), _ptrs(xs), _strides3(xs), _ptrs(ys), _strides3(ys), B, H, n, D, _lib.ptr(c),
              _lib.ptr(s), c.stride(0), c.stride(1), int(c.dtype == torch.bfloat16), _lib.stream(ys[0].device))


class _RopedChunk(torch.autograd.Function):
    """``apply_rope`` of the chunk's q and k (``batched_engine.py:156``: one HIP launch for both, bf16 results as the
    chunk kernel reads them, the products and sum rounded as torch rounds them) followed by the chunk attention;
    the backward takes the chunk kernel's fp32 dq / dk of the rotated operands through the RoPE backward kernel
    (autograd's roundings for bf16 q / k). Returns o fp32 and lse as ``_CurrentChunk`` does."""

    @staticmethod
    def forward(ctx, q, k, v, valid, cos, sin, scale):
        B, H, n, D = q.shape
        qb, kb = (t.to(torch.bfloat16) for t in (q, k))
        qb, kb = (t if t.stride(-1) == 1 and all(x % 8 == 0 for x in t.stride()[:3]) and t.data_ptr() % 16 == 0
                  else t.contiguous() for t in (qb, kb))
        c, s = _trig(cos, sin, B, n, D)
        qr, kr = (torch.empty(B, H, n, D, dtype=torch.bfloat16, device=q.device) for _ in range(2))
        _rope_call('hla_s6_rope_rows_forward', [qb, kb], [qr, kr], c, s)
        vb = v.to(torch.bfloat16).contiguous()
        v8 = valid.to(torch.bool).contiguous().view(torch.uint8)
        o, lse = _chunk_forward(qr, kr, vb, v8, scale)
        ctx.save_for_backward(qr, kr, vb, v8, o, lse, c, s)
        ctx.settings = (float(scale), q.dtype, k.dtype, v.dtype)
        return o, lse

    @staticmethod
    @once_differentiable
    def backward(ctx, do, dlse):
        qr, kr, vb, v8, o, lse, c, s = ctx.saved_tensors
        scale, q_dtype, k_dtype, v_dtype = ctx.settings
        dqr, dkr, dv = _chunk_backward(qr, kr, vb, v8, o, lse, do, dlse, scale)
        dq, dk = torch.empty_like(qr), torch.empty_like(kr)
        _rope_call('hla_s6_rope_rows_backward', [dqr, dkr], [dq, dk], c, s)
        return dq.to(q_dtype), dk.to(k_dtype), dv.to(v_dtype), None, None, None, None


def current_chunk_attention(q, k, v, valid, scale):
    """``(o [B, 16, n, 128] fp32, lse [B, 16, n] fp32)`` of the chunk's exact attention (RoPE'd q / k, valid
    ``[B, n]``) on the HIP chunk kernels, differentiable in q, k and v."""
    s6_ops._dev(q, k, v, valid)
    B, H, n, D = q.shape
    if H != 16 or D != 128 or k.shape != q.shape or v.shape != q.shape or tuple(valid.shape) != (B, n):
        raise ValueError(f'the chunk kernels take q / k / v [B, 16, n, 128] and valid [B, n] (got {tuple(q.shape)}, '
                         f'{tuple(k.shape)}, {tuple(v.shape)}, {tuple(valid.shape)})')
    return _CurrentChunk.apply(q, k, v, valid, float(scale))


def _history_block(qt, ck, cv, mask, scale):
    """z ``[B, H, n, r]`` (bf16, a view of token-linear rows) and lse ``[B, H, n]`` of the latent query qt ``[B, n,
    H, r]`` (bf16, token-linear) over the rows ck / cv ``[B, N, r]`` that mask ``[B, N]`` shows to every query of the
    chunk."""
    B, n = qt.shape[:2]
    m = mask[:, None, :].expand(B, n, mask.shape[1])  # (query stride 0: the kernels read one row per batch row)
    z, lse = history_gemm.causal_history_gemm(qt, ck, cv, m, scale, precision='bf16')
    return z.transpose(1, 2), lse


def _ptrs(ts):
    return (ctypes.c_void_p * max(len(ts), 1))(*[t.data_ptr() for t in ts])


def _strides3(ts):
    return (ctypes.c_int64 * max(3 * len(ts), 1))(*[s for t in ts for s in t.stride()[:3]])


def _merge_args(o_c, lse_c, zs, ls, b_read):
    B, H, n, D = o_c.shape
    return (B, H, n, zs[0].shape[-1], D, _lib.ptr(o_c), *o_c.stride()[:3], _lib.ptr(lse_c), len(zs), _ptrs(zs),
            _strides3(zs), _ptrs(ls), _lib.ptr(b_read), b_read.stride(0), b_read.stride(1))


class _Merge(torch.autograd.Function):
    """``out = bf16(w_c o_c + bf16(sum_p w_p z_p) @ B)`` with ``w = exp(lse - logsumexp(lse_c, lse_p, ..))``
    (``batched_engine.py:171-181``) on the HIP merge kernels: o_c ``[B, 16, n, 128]`` fp32 and lse_c ``[B, 16, n]``
    of the chunk, ``parts`` alternating z_p ``[B, 16, n, r]`` bf16 and lse_p ``[B, 16, n]`` of the history blocks, B
    ``[16, r, 128]``. The backward kernel gives the gradients of o_c, lse_c and every part; the gradient of B (when it
    is asked for) is the float32 product of the bf16 joint latent output with dout."""

    @staticmethod
    def forward(ctx, o_c, lse_c, b_read, *parts):
        zs = [z.to(torch.bfloat16) for z in parts[0::2]]
        zs = [z if z.stride(-1) == 1 and all(s % 8 == 0 for s in z.stride()[:3]) else z.contiguous() for z in zs]
        ls = [l.to(torch.float32).contiguous() for l in parts[1::2]]
        o_c, lse_c = o_c.to(torch.float32), lse_c.to(torch.float32).contiguous()
        if o_c.stride(-1) != 1 or any(s % 4 for s in o_c.stride()[:3]):
            o_c = o_c.contiguous()
        bb = b_read.to(torch.bfloat16)
        if bb.stride(-1) != 1 or any(s % 8 for s in bb.stride()[:2]):
            bb = bb.contiguous()
        out = torch.empty(o_c.shape, dtype=torch.bfloat16, device=o_c.device)
        _lib.call('hla_s6_mixed_merge_forward', *_merge_args(o_c, lse_c, zs, ls, bb), _lib.ptr(out),
                  *out.stride()[:3], _lib.stream(o_c.device))
        ctx.save_for_backward(o_c, lse_c, bb, *zs, *ls)
        ctx.dtypes = (b_read.dtype, [p.dtype for p in parts])
        return out

    @staticmethod
    @once_differentiable
    def backward(ctx, dout):
        o_c, lse_c, bb, *rest = ctx.saved_tensors
        k = len(rest) // 2
        zs, ls = rest[:k], rest[k:]
        b_dtype, part_dtypes = ctx.dtypes
        d = dout.to(torch.bfloat16).contiguous()
        doc = torch.empty(o_c.shape, dtype=torch.float32, device=o_c.device)
        dlc = torch.empty_like(lse_c)
        dzs = [torch.empty_like(z) for z in zs]
        dls = [torch.empty_like(l) for l in ls]
        _lib.call('hla_s6_mixed_merge_backward', *_merge_args(o_c, lse_c, zs, ls, bb), _lib.ptr(d), *d.stride()[:3],
                  _lib.ptr(doc), *doc.stride()[:3], _lib.ptr(dlc), _ptrs(dzs), _strides3(dzs), _ptrs(dls),
                  _lib.stream(o_c.device))
        db = None
        if ctx.needs_input_grad[2]:
            total = torch.logsumexp(torch.stack([lse_c, *ls]), 0)
            z = sum(torch.exp(l - total)[..., None] * zz.float() for zz, l in zip(zs, ls))
            db = torch.einsum('bhir,bhid->hrd', z.to(torch.bfloat16).float(), d.float()).to(b_dtype)
        grads = []
        for dz, dl, dzt, dlt in zip(dzs, dls, part_dtypes[0::2], part_dtypes[1::2]):
            grads += [dz.to(dzt), dl.to(dlt)]
        return (doc, dlc, db, *grads)


def mixed_attention(sl, loop, q, k, v, cos, sin, valid, blocks, masks):
    """``hla/latent/batched_engine.py:154-182``: q, k, v ``[B, 16, n, head_dim]`` of the chunk, cos / sin ``[B, n,
    head_dim]``, valid ``[B, n]``, ``blocks`` the packed history rows ``[B, N_k, 1536]`` and ``masks`` their ``[B,
    N_k]`` visibility. ``sl`` is the layer's latent module (``register.LatentLayer``: ``query``, ``fields``,
    ``readers``, ``head_dim``). Returns ``[B, 16, n, head_dim]`` in v.dtype. Valid queries see the chunk's valid keys
    up to their own position; an invalid query sees every key of the chunk (its row stays finite and is never read)."""
    scale = 1 / math.sqrt(sl.head_dim)
    s6_ops._dev(q, k, v, valid, cos, sin)
    B, H, n, D = q.shape
    if H != 16 or D != 128 or k.shape != q.shape or v.shape != q.shape or tuple(valid.shape) != (B, n):
        raise ValueError(f'the chunk kernels take q / k / v [B, 16, n, 128] and valid [B, n] (got {tuple(q.shape)}, '
                         f'{tuple(k.shape)}, {tuple(v.shape)}, {tuple(valid.shape)})')
    blocks, masks = list(blocks or ()), list(masks or ())
    if len(blocks) != len(masks):
        raise ValueError(f'mixed_attention: {len(blocks)} history blocks but {len(masks)} masks')
    if len(blocks) > MAX_BLOCKS:   # checked before any launch
        raise ValueError(f'mixed_attention: {len(blocks)} history blocks (the merge kernel takes at most {MAX_BLOCKS})')
    with torch.autocast(q.device.type, enabled=False):         # qrot, krot = apply_rope(q / k, cos, sin), then the chunk
        o_c, lse_c = _RopedChunk.apply(q, k, v, valid, cos, sin, float(scale))
    if not blocks:
        return o_c.to(v.dtype)
    qc = sl.query(loop, q, cos, sin)
    # the MFMA kernels' operands, made once for every block: token-linear bf16 rows [B, n, 16, r] (one copy, which
    # also rounds a float32 query as the kernels would)
    qt = torch.empty(qc.shape[0], qc.shape[2], qc.shape[1], qc.shape[3], dtype=torch.bfloat16, device=qc.device)
    qt.copy_(qc.transpose(1, 2))
    parts = []
    for block, mask in zip(blocks, masks):
        ck, cv = sl.fields(loop, block)
        parts.append(_history_block(qt, ck, cv, mask, scale))
    _, B_read, _ = sl.readers(loop)
    with torch.autocast(q.device.type, enabled=False):
        out = _Merge.apply(o_c, lse_c, B_read, *[t for part in parts for t in part])
    return out.to(v.dtype)
