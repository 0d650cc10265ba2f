"""History attention over contiguous latent rows with backward on MI355X: the interface of
``hla/latent/history_gemm.py`` (``causal_history_gemm``) and of ``hla/latent/fused_history.py`` (the single-query
``history_attention`` of lines 49-54 and the multi-query ``causal_history_attention`` of lines 126-153) over the HIP
kernels of ``khop.hip`` (``hla_s6_khop_bounds``, ``hla_s6_khop_forward``, ``hla_s6_khop_backward``) and
``history.hip`` (``hla_s6_masked_history``, the single-query forward).

Every query row ``(b, i, h)`` attends over the latent rows ``k[b, j], v[b, j]`` that ``mask[b, i, j]`` shows (all
heads share the rows). The kernels compute with bf16 GEMM operands and fp32 accumulation and softmax: the
reference's ``precision='bf16'`` mode, which callers select explicitly. The reference's default modes (``'fp32'``,
IEEE fp32 GEMMs, and ``'tf32'``; ``hla/latent/history_gemm.py:19-24,270-271``) and its fp32 CUDA-core ``'triton'``
backend (``hla/latent/fused_history.py:129-130``) have no kernels here and raise ``ValueError``, so that no call
narrows its arithmetic without asking. The kernels derive each query's key bound from the mask, so ``causal`` needs
no promise and only documents intent. No ``[B, H, Lq, N]`` tensor is ever formed.
"""
from __future__ import annotations

import torch
from torch.autograd.function import once_differentiable

from . import _lib, s6_ops

PRECISIONS = ('fp32', 'tf32', 'bf16')   # the reference's modes
KERNEL_PRECISIONS = ('bf16',)          # the modes the HIP kernels compute
DEFAULT_CHUNK = 128
DEFAULT_MAX_ELEMENTS = 1 << 26
KEY_ALIGN = 16
HEADS = 16
WIDTHS = (128, 256, 512)          # forward and backward
FORWARD_WIDTHS = WIDTHS + (1024,)  # 1024: forward only (token-linear rows, N a multiple of 16)


def bf16_fp32_output_supported(device) -> bool:
    """The HIP kernels always accumulate bf16 products in fp32 (``history_gemm.py:84-98`` probes torch for this)."""
    return True


def _check_precision(precision):
    """``ValueError`` unless ``precision`` is a mode the kernels compute (the reference's message for unknown modes,
    ``hla/latent/history_gemm.py:287-288``; a clear refusal for its fp32 / tf32 modes)."""
    if precision not in PRECISIONS:
        raise ValueError(f'Unknown precision {precision!r}; expected one of {PRECISIONS}')
    if precision not in KERNEL_PRECISIONS:
        raise ValueError(f'precision={precision!r} has no MI355X kernel: the HIP kernels compute with bf16 operands '
                         f'and fp32 accumulation; pass precision="bf16"')


def _bf16_rows(name, t):
    t = t.to(torch.bfloat16)
    if t.stride(-1) != 1 or any(s % 8 for s in t.stride()[:-1]) or t.data_ptr() % 16:
        t = t.contiguous()
    return t


def _key_splits(tiles: int, device, per_cu: int = 4) -> int:
    """Row ranges per key tile of the dk/dv kernel: about ``per_cu`` workgroups per CU (at most 16 ranges)."""
    cus = _lib.device_cus(device.index or 0)
    return max(1, min(16, round(per_cu * cus / max(1, tiles))))


class _CausalHistory(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, mask, scale):
        B, Lq, H, R = q.shape
        N = k.shape[1]
        dev = q.device
        qb, kb, vb = _bf16_rows('q', q), _bf16_rows('k', k), _bf16_rows('v', v)
        if qb.stride(0) != Lq * qb.stride(1):      # token-linear query rows: the multi-query kernels need them
            qb = qb.contiguous()
        if R == 1024:
            kb, vb = kb.contiguous(), vb.contiguous()
            if N % KEY_ALIGN:
                raise ValueError(f'width 1024 needs a key count that is a multiple of {KEY_ALIGN} (got {N})')
        m = mask if mask.dtype == torch.bool else mask.bool()
        if m.stride(-1) != 1:
            m = m.contiguous()
        m8 = m.view(torch.uint8)
        bound = torch.empty(B * Lq, dtype=torch.int32, device=dev)
        st = _lib.stream(dev)
        _lib.call('hla_s6_khop_bounds', _lib.ptr(m8), m8.stride(0), m8.stride(1), B, Lq, N, _lib.ptr(bound), st)
        z = torch.empty(B, Lq, H, R, dtype=torch.bfloat16, device=dev)
        lse = torch.empty(B, H, Lq, dtype=torch.float32, device=dev)
        _lib.call('hla_s6_khop_forward', _lib.ptr(qb), qb.stride(0), qb.stride(1), qb.stride(2), _lib.ptr(kb),
                  kb.stride(0), kb.stride(1), _lib.ptr(vb), vb.stride(0), vb.stride(1), _lib.ptr(m8), m8.stride(0),
                  m8.stride(1), _lib.ptr(bound), B, Lq, N, H, R, float(scale), _lib.ptr(z), z.stride(0), z.stride(1),
                  z.stride(2), _lib.ptr(lse), st)
        ctx.save_for_backward(qb, kb, vb, m8, bound, lse, z)
        ctx.settings = (float(scale), q.dtype, k.dtype, v.dtype)
        return z.to(q.dtype), lse

    @staticmethod
    @once_differentiable
    def backward(ctx, dz, dlse):
        qb, kb, vb, m8, bound, lse, z = ctx.saved_tensors
        scale, q_dtype, k_dtype, v_dtype = ctx.settings
        need_q, need_k, need_v = ctx.needs_input_grad[:3]
        if qb.shape[-1] not in WIDTHS:
            raise ValueError(f'causal_history_gemm backward: the HIP kernels take widths {WIDTHS} '
                             f'(got {qb.shape[-1]}; 1024 is forward only)')
        bf = q_dtype == k_dtype == v_dtype == torch.bfloat16
        dq, dk, dv = _backward(qb, kb, vb, m8, bound, lse, z, dz, dlse, scale, need_q, need_k or need_v, bf)
        return (dq.to(q_dtype) if need_q else None, dk.to(k_dtype) if need_k else None,
                dv.to(v_dtype) if need_v else None, None, None)


def _backward(qb, kb, vb, m8, bound, lse, z, dz, dlse, scale, need_q, need_kv, bf16_grads=False):
    """dq [B, Lq, 16, R], dk / dv [B, N, R] (fp32, or bf16 written by the kernels with ``bf16_grads``; None where not
    needed) of z, lse = forward(q [B, Lq, 16, R], k, v, mask bytes m8 [B, Lq, N]) for the cotangents dz
    [B, Lq, 16, R] and dlse [B, 16, Lq] (None = 0)."""
    B, Lq, H, R = qb.shape
    N = kb.shape[1]
    dev = qb.device
    dzb = _bf16_rows('dz', dz if dz is not None else torch.zeros_like(z))
    dl = None if dlse is None else dlse.to(torch.float32).contiguous()
    delta = torch.empty(B, H, Lq, dtype=torch.float32, device=dev)
    gd = torch.bfloat16 if bf16_grads else torch.float32
    dq = torch.empty(B, Lq, H, R, dtype=gd, device=dev) if need_q else None
    dk = torch.empty(B, N, R, dtype=gd, device=dev) if need_kv else None
    dv = torch.empty(B, N, R, dtype=gd, device=dev) if need_kv else None
    # key tiles of the dk / dv kernel: 64 keys on the multi-query form (widths 512 / 256, N a multiple of 16),
    # whose causal load is balanced best with about 8 workgroups per CU (12 ranges at B=4, L=2880: 3.78 ms
    # forward + backward against 4.15 ms with 6 and 4.11 ms with 32); 4 per CU on the 32-key form
    # (row ranges split a tile's query rows, which the kernels take two at a time: at most ceil(Lq / 2) of them).
    # Few queries over many keys (a chunk against history rows it sees alike) give every key tile the same work:
    # one workgroup per CU, no more ranges than fill the GPU (B=8, a 256-token chunk over 2048 rows: the
    # joint-attention step 2.40 -> 2.08 ms; with 8 per CU, 8 ranges and their fp32 partials)
    mq = R in (256, 512) and N % 16 == 0
    per_cu = (8 if 2 * Lq >= N else 1) if mq else 4
    splits = min(_key_splits(-(-N // (64 if mq else 32)) * B, dev, per_cu), -(-Lq // 2)) if need_kv else 1
    splits = max(1, splits)
    floats = _lib.load().hla_s6_khop_backward_workspace(B, Lq, N, R, splits)
    ws = torch.empty(floats, dtype=torch.float32, device=dev) if floats > 0 else None
    _lib.call('hla_s6_khop_backward', _lib.ptr(qb), qb.stride(0), qb.stride(1), qb.stride(2), _lib.ptr(kb),
              kb.stride(0), kb.stride(1), _lib.ptr(vb), vb.stride(0), vb.stride(1), _lib.ptr(m8), m8.stride(0),
              m8.stride(1), _lib.ptr(bound), B, Lq, N, H, R, scale, _lib.ptr(z), z.stride(0), z.stride(1),
              z.stride(2), _lib.ptr(lse), _lib.ptr(dzb), dzb.stride(0), dzb.stride(1), dzb.stride(2), _lib.ptr(dl),
              _lib.ptr(delta), _lib.ptr(dq), 0 if dq is None else dq.stride(0), 0 if dq is None else dq.stride(1),
              0 if dq is None else dq.stride(2), _lib.ptr(dk), 0 if dk is None else dk.stride(0),
              0 if dk is None else dk.stride(1), _lib.ptr(dv), 0 if dv is None else dv.stride(0),
              0 if dv is None else dv.stride(1), splits, _lib.ptr(ws), 0 if ws is None else ws.numel(),
              int(bf16_grads), _lib.stream(dev))
    return dq, dk, dv


def causal_history_gemm(q, k, v, mask, scale, *, causal=False, chunk=DEFAULT_CHUNK, precision='fp32',
                        max_elements=DEFAULT_MAX_ELEMENTS):
    """Causal history attention (``hla/latent/history_gemm.py:270-294``).

    q: [B, Lq, 16, R], k: [B, N, R], v: [B, N, R], mask: [B, Lq, N] (True = visible). Returns z [B, Lq, 16, R] in
    q.dtype and lse [B, 16, Lq] (fp32, -inf on rows with no visible history, where z is 0); differentiable in q, k
    and v. ``precision`` must be ``'bf16'`` (bf16 operands, fp32 accumulation); the reference's default ``'fp32'``
    and ``'tf32'`` raise ``ValueError``. ``causal`` asks for the reference's promise check only; ``chunk`` and
    ``max_elements`` are accepted for signature parity (the kernels do not chunk).
    """
    if q.ndim != 4 or k.ndim != 3 or v.ndim != 3 or mask.ndim != 3:
        raise ValueError(f'Expected Q[B,Lq,H,R], K[B,N,R], V[B,N,Rv], mask[B,Lq,N], got '
                         f'{tuple(q.shape)}, {tuple(k.shape)}, {tuple(v.shape)}, {tuple(mask.shape)}')
    B, Lq, H, Rk = q.shape
    N = k.shape[1]
    if (k.shape[0] != B or k.shape[-1] != Rk or v.shape[:2] != k.shape[:2]
            or tuple(mask.shape) != (B, Lq, N)):
        raise ValueError('Inconsistent history attention shapes')
    if causal and N < Lq:
        raise ValueError('Causal history requires at least as many keys as queries')
    _check_precision(precision)
    if chunk < 1 or max_elements < 1:
        raise ValueError('chunk and max_elements must be positive')
    if H != HEADS or v.shape[-1] != Rk or Rk not in FORWARD_WIDTHS:
        raise ValueError(f'the HIP kernels take {HEADS} heads and equal K/V widths in {FORWARD_WIDTHS} '
                         f'(got H={H}, Rk={Rk}, Rv={v.shape[-1]})')
    s6_ops._dev(q, k, v, mask)
    return _CausalHistory.apply(q, k, v, mask, float(scale))


SINGLE_WIDTHS = (128, 256, 512, 1024)  # forward; the backward takes WIDTHS


class _History(torch.autograd.Function):
    """``hla/latent/fused_history.py:23-46``: forward on the split kernel over contiguous rows with a key mask
    (``hla_s6_masked_history``), backward on the K-hop kernels with one query per batch row."""

    @staticmethod
    def forward(ctx, q, k, v, mask, scale):
        B, H, R = q.shape
        N = k.shape[1]
        dev = q.device
        qb, kb, vb = _bf16_rows('q', q), _bf16_rows('k', k), _bf16_rows('v', v)
        if kb.stride() != vb.stride():                # one row geometry for both (e.g. fields of packed rows)
            kb, vb = kb.contiguous(), vb.contiguous()
        m = mask if mask.dtype == torch.bool else mask.bool()
        m8 = m.contiguous().view(torch.uint8)
        bound = torch.empty(B, dtype=torch.int32, device=dev)
        st = _lib.stream(dev)
        _lib.call('hla_s6_khop_bounds', _lib.ptr(m8), m8.stride(0), N, B, 1, N, _lib.ptr(bound), st)
        splits = s6_ops.mi355x_kv_splits(N, B, _lib.device_cus(dev.index or 0), width=R)
        ws = torch.empty(B * splits * H * (R + 1), dtype=torch.float32, device=dev) if splits > 1 else None
        z = torch.empty(B, H, R, dtype=torch.bfloat16, device=dev)
        lse = torch.empty(B, H, dtype=torch.float32, device=dev)
        _lib.call('hla_s6_masked_history', _lib.ptr(qb), qb.stride(0), qb.stride(1), _lib.ptr(kb), _lib.ptr(vb),
                  kb.stride(0), kb.stride(1), _lib.ptr(m8), m8.stride(0), _lib.ptr(bound), B, N, H, R, float(scale),
                  splits, _lib.ptr(ws), 0 if ws is None else ws.numel(), _lib.ptr(z), z.stride(0), z.stride(1),
                  _lib.ptr(lse), st)
        ctx.save_for_backward(qb, kb, vb, m8, bound, lse, z)
        ctx.settings = (float(scale), q.dtype, k.dtype, v.dtype)
        return z.to(q.dtype), lse

    @staticmethod
    @once_differentiable
    def backward(ctx, dz, dlse):
        qb, kb, vb, m8, bound, lse, z = ctx.saved_tensors
        scale, q_dtype, k_dtype, v_dtype = ctx.settings
        need_q, need_k, need_v = ctx.needs_input_grad[:3]
        R = qb.shape[-1]
        if R not in WIDTHS:
            raise ValueError(f'history_attention backward: the HIP kernels take widths {WIDTHS} (got {R})')
        dq, dk, dv = _backward(qb[:, None], kb, vb, m8[:, None], bound, lse[:, :, None], z[:, None],
                               None if dz is None else dz[:, None], None if dlse is None else dlse[:, :, None],
                               scale, need_q, need_k or need_v, q_dtype == k_dtype == v_dtype == torch.bfloat16)
        return (dq[:, 0].to(q_dtype) if need_q else None, dk.to(k_dtype) if need_k else None,
                dv.to(v_dtype) if need_v else None, None, None)


def history_attention(q, k, v, mask, scale, reference_forward=False):
    """Single-query history attention (``hla/latent/fused_history.py:49-54``): q [B, 16, R] against the contiguous
    rows k, v [B, N, R] that mask [B, N] (True = visible) shows. Returns z [B, 16, R] in q.dtype and lse [B, 16]
    (fp32, natural log; z = 0 and lse = -inf for a row with no visible key), differentiable in q, k and v (the
    cache gradients keep in-window writers trainable). bf16 operands, fp32 accumulation and softmax.
    ``reference_forward`` (the reference's dense torch forward) is refused: the HIP forward is the only one here."""
    if (q.ndim != 3 or k.ndim != 3 or k.shape != v.shape or mask.shape != k.shape[:2] or q.shape[0] != k.shape[0]
            or q.shape[-1] != k.shape[-1]):
        raise ValueError('Expected Q[B,H,R], K/V[B,N,R], mask[B,N]')
    s6_ops._dev(q, k, v, mask)
    if k.shape[1] < 1:
        raise ValueError('History must contain a storage row')
    if reference_forward:
        raise ValueError('reference_forward: the dense torch forward is not part of the MI355X path')
    if q.shape[1] != HEADS or q.shape[-1] not in SINGLE_WIDTHS:
        raise ValueError(f'the HIP kernels take {HEADS} heads and widths {SINGLE_WIDTHS} '
                         f'(got H={q.shape[1]}, R={q.shape[-1]})')
    if q.shape[0] == 0:
        return q.new_zeros(q.shape), torch.empty(0, HEADS, dtype=torch.float32, device=q.device)
    return _History.apply(q, k, v, mask, float(scale))


HISTORY_BACKENDS = ('triton', 'reference', 'gemm')


def causal_history_attention(q, k, v, mask, scale, reference_forward=False, *, backend='triton', precision='fp32',
                             chunk=None, causal=False):
    """``hla/latent/fused_history.py:129-153``: ``backend='gemm'`` runs ``causal_history_gemm`` with ``precision``
    (``'bf16'``: the HIP kernels). The reference's default ``'triton'`` backend (fp32 CUDA-core kernels) and its
    ``'reference'`` backend (dense fp32 torch autograd) compute in fp32, which no kernel here does: both raise
    ``ValueError`` rather than run at bf16."""
    if q.ndim != 4 or k.ndim != 3 or v.ndim != 3 or mask.ndim != 3:
        raise ValueError(f'Expected Q[B,Lq,H,R], K/V[B,N,R], mask[B,Lq,N], got {tuple(q.shape)}, {tuple(k.shape)}, '
                         f'{tuple(v.shape)}, {tuple(mask.shape)}')
    if backend not in HISTORY_BACKENDS:
        raise ValueError(f'Unknown causal history backend {backend!r}; expected one of {HISTORY_BACKENDS}')
    if backend != 'gemm':
        raise ValueError(f'backend={backend!r} computes in fp32, which has no MI355X kernel: use backend="gemm", '
                         f'precision="bf16" (bf16 MFMA operands, fp32 accumulation)')
    return causal_history_gemm(q, k, v, mask, scale, causal=causal, chunk=chunk or DEFAULT_CHUNK,
                               precision=precision)


def flops(visible_pairs: int, heads: int, width: int, with_backward: bool = False) -> float:
    """Algorithmic FLOPs for ``visible_pairs`` visible (query, key) pairs, ``2 * heads * width`` per pair and GEMM:
    2 GEMMs forward (S, P V); the backward adds 5 (S again, dP, dV, dQ, dK)."""
    return 2.0 * heads * width * visible_pairs * (7 if with_backward else 2)
