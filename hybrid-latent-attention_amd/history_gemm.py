"""History attention over contiguous latent rows with backward on MI355X: the interface of
``hla/latent/history_gemm.py`` (``causal_history_gemm``) and of ``hla/latent/fused_history.py`` (the single-query
``history_attention`` of lines 49-54 and the multi-query ``causal_history_attention`` of lines 126-153) over the HIP
kernels of ``khop.hip`` / ``khop_f32.hip`` (``hla_s6_khop_bounds``, ``hla_s6_khop_forward[_f32]``,
``hla_s6_khop_backward[_f32]``) and ``history.hip`` (``hla_s6_masked_history``, the single-query forward).

Every query row ``(b, i, h)`` attends over the latent rows ``k[b, j], v[b, j]`` that ``mask[b, i, j]`` shows (all
heads share the rows). Two arithmetics, as the reference's precision modes (``hla/latent/history_gemm.py:19-24``):

* ``precision='fp32'`` (the reference's default) and ``'tf32'``: fp32 operands on fp32 MFMA, fp32 softmax and
  accumulation (``khop_f32.hip``); tf32 runs the same fp32 kernels (wider than tf32, never narrower). The
  reference's fp32 ``'triton'`` (default) and ``'reference'`` backends of ``causal_history_attention`` run them too.
  Inputs of any floating dtype are converted to fp32 once (the reference's ``.to(acc)``); float64 inputs, which the
  reference computes in float64, raise ``ValueError`` (no float64 kernel) rather than narrow.
* ``precision='bf16'``: bf16 GEMM operands with fp32 accumulation and softmax (``khop.hip`` and the multi-query
  history kernels); the width-1024 backward runs on the fp32 kernels (bf16 inputs, wider arithmetic).

The kernels derive each query's key bound from the mask, so ``causal`` needs no promise and only documents intent.
No ``[B, H, Lq, N]`` tensor is ever formed.
"""
from __future__ import annotations

import torch
from torch.autograd.function import once_differentiable

from . import _lib, s6_ops

PRECISIONS = ('fp32', 'tf32', 'bf16')   # the reference's modes
KERNEL_PRECISIONS = PRECISIONS           # every mode has kernels ('tf32' runs the fp32 ones)
DEFAULT_CHUNK = 128
DEFAULT_MAX_ELEMENTS = 1 << 26
KEY_ALIGN = 16
HEADS = 16
WIDTHS = (128, 256, 512)          # bf16 forward and backward on the bf16 kernels
FORWARD_WIDTHS = WIDTHS + (1024,)  # 1024: bf16 forward on the multi-query kernel (N a multiple of 16), backward on
                                   # the fp32 kernels
FP32_WIDTHS = (128, 256, 512, 1024)


def bf16_fp32_output_supported(device) -> bool:
    """The HIP kernels always accumulate bf16 products in fp32 (``history_gemm.py:84-98`` probes torch for this)."""
    return True


def _check_precision(precision):
    """``ValueError`` for a mode the reference does not know (its message, ``hla/latent/history_gemm.py:287-288``)."""
    if precision not in PRECISIONS:
        raise ValueError(f'Unknown precision {precision!r}; expected one of {PRECISIONS}')


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
        if qb.shape[-1] not in WIDTHS:   # width 1024: the fp32 kernels on the bf16 operands (wider arithmetic)
            f32 = lambda t: t.float().contiguous()
            dq, dk, dv = _backward_f32(f32(qb), f32(kb), f32(vb), m8, bound, lse, f32(z), dz, dlse, scale, need_q,
                                       need_k or need_v)
        else:
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


def _f32_rows(t):
    """fp32 rows for the fp32 kernels: 16-byte aligned, unit last stride (a copy only when needed)."""
    t = t.to(torch.float32)
    if t.stride(-1) != 1 or any(s % 4 for s in t.stride()[:-1]) or t.data_ptr() % 16:
        t = t.contiguous()
    return t


def _mask_bytes(mask, B, Lq, N, dev):
    """The mask as bytes with a unit last stride and each token's key bound (``hla_s6_khop_bounds``)."""
    m = mask if mask.dtype == torch.bool else mask.bool()
    if m.stride(-1) != 1:
        m = m.contiguous()
    m8 = m.view(torch.uint8)
    bound = torch.empty(B * Lq, dtype=torch.int32, device=dev)
    _lib.call('hla_s6_khop_bounds', _lib.ptr(m8), m8.stride(0), m8.stride(1), B, Lq, N, _lib.ptr(bound),
              _lib.stream(dev))
    return m8, bound


def _forward_f32(q32, k32, v32, m8, bound, scale):
    """z [B, Lq, 16, R] fp32 and lse [B, 16, Lq] of the fp32 kernels."""
    B, Lq, H, R = q32.shape
    N = k32.shape[1]
    dev = q32.device
    z = torch.empty(B, Lq, H, R, dtype=torch.float32, device=dev)
    lse = torch.empty(B, H, Lq, dtype=torch.float32, device=dev)
    _lib.call('hla_s6_khop_forward_f32', _lib.ptr(q32), q32.stride(0), q32.stride(1), q32.stride(2), _lib.ptr(k32),
              k32.stride(0), k32.stride(1), _lib.ptr(v32), v32.stride(0), v32.stride(1), _lib.ptr(m8), m8.stride(0),
              m8.stride(1), _lib.ptr(bound), B, Lq, N, H, R, float(scale), _lib.ptr(z), z.stride(0), z.stride(1),
              z.stride(2), _lib.ptr(lse), _lib.stream(dev))
    return z, lse


def _f32_key_splits(B, Lq, N, R, dev):
    """Token ranges per key block of the fp32 dk / dv kernel: about 4 workgroups per CU over the B * key blocks
    (16 * 8 / (R / 128) keys each), at most 16, each range at least 64 tokens."""
    blocks = B * -(-N // (16 * max(1, 1024 // R)))
    cus = _lib.device_cus(dev.index or 0)
    return max(1, min(16, -(-4 * cus // max(1, blocks)), max(1, Lq // 64)))


def _backward_f32(q32, k32, v32, m8, bound, lse, z32, dz, dlse, scale, need_q, need_kv):
    """dq [B, Lq, 16, R], dk / dv [B, N, R] (fp32; None where not needed) on the fp32 kernels, for the cotangents
    dz (any floating dtype, None = 0) and dlse [B, 16, Lq] (None = 0); delta = dz . z uses the fp32 forward
    output z32."""
    B, Lq, H, R = q32.shape
    N = k32.shape[1]
    dev = q32.device
    dz32 = _f32_rows(dz) if dz is not None else torch.zeros_like(z32)
    dl = None if dlse is None else dlse.to(torch.float32).contiguous()
    delta = torch.empty(B, H, Lq, dtype=torch.float32, device=dev)
    dq = torch.empty(B, Lq, H, R, dtype=torch.float32, device=dev) if need_q else None
    dk = torch.empty(B, N, R, dtype=torch.float32, device=dev) if need_kv else None
    dv = torch.empty(B, N, R, dtype=torch.float32, device=dev) if need_kv else None
    splits = _f32_key_splits(B, Lq, N, R, dev) if need_kv else 1
    floats = _lib.load().hla_s6_khop_backward_f32_workspace(B, Lq, N, R, splits)
    ws = torch.empty(floats, dtype=torch.float32, device=dev) if floats > 0 else None
    _lib.call('hla_s6_khop_backward_f32', _lib.ptr(q32), q32.stride(0), q32.stride(1), q32.stride(2), _lib.ptr(k32),
              k32.stride(0), k32.stride(1), _lib.ptr(v32), v32.stride(0), v32.stride(1), _lib.ptr(m8), m8.stride(0),
              m8.stride(1), _lib.ptr(bound), B, Lq, N, H, R, float(scale), _lib.ptr(z32), z32.stride(0),
              z32.stride(1), z32.stride(2), _lib.ptr(lse), _lib.ptr(dz32), dz32.stride(0), dz32.stride(1),
              dz32.stride(2), _lib.ptr(dl), _lib.ptr(delta), _lib.ptr(dq), 0 if dq is None else dq.stride(0),
              0 if dq is None else dq.stride(1), 0 if dq is None else dq.stride(2), _lib.ptr(dk),
              0 if dk is None else dk.stride(0), 0 if dk is None else dk.stride(1), _lib.ptr(dv),
              0 if dv is None else dv.stride(0), 0 if dv is None else dv.stride(1), splits, _lib.ptr(ws),
              0 if ws is None else ws.numel(), _lib.stream(dev))
    return dq, dk, dv


class _CausalHistoryF32(torch.autograd.Function):
    """fp32 arithmetic (``precision='fp32'`` / ``'tf32'``, and the fp32 backends of ``causal_history_attention``):
    z in q.dtype, lse fp32; gradients in the inputs' dtypes."""

    @staticmethod
    def forward(ctx, q, k, v, mask, scale):
        B, Lq, H, R = q.shape
        N = k.shape[1]
        q32, k32, v32 = _f32_rows(q), _f32_rows(k), _f32_rows(v)
        m8, bound = _mask_bytes(mask, B, Lq, N, q.device)
        z, lse = _forward_f32(q32, k32, v32, m8, bound, scale)
        ctx.save_for_backward(q32, k32, v32, m8, bound, lse, z)
        ctx.settings = (float(scale), q.dtype, k.dtype, v.dtype)
        return z.to(q.dtype), lse

    @staticmethod
    @once_differentiable
    def backward(ctx, dz, dlse):
        q32, k32, v32, m8, bound, lse, z = ctx.saved_tensors
        scale, q_dtype, k_dtype, v_dtype = ctx.settings
        need_q, need_k, need_v = ctx.needs_input_grad[:3]
        dq, dk, dv = _backward_f32(q32, k32, v32, m8, bound, lse, z, dz, dlse, scale, need_q, need_k or need_v)
        return (dq.to(q_dtype) if need_q else None, dk.to(k_dtype) if need_k else None,
                dv.to(v_dtype) if need_v else None, None, None)


def causal_history_gemm(q, k, v, mask, scale, *, causal=False, chunk=DEFAULT_CHUNK, precision='fp32',
                        max_elements=DEFAULT_MAX_ELEMENTS):
    """Causal history attention (``hla/latent/history_gemm.py:270-294``).

    q: [B, Lq, 16, R], k: [B, N, R], v: [B, N, R], mask: [B, Lq, N] (True = visible). Returns z [B, Lq, 16, R] in
    q.dtype and lse [B, 16, Lq] (fp32, -inf on rows with no visible history, where z is 0); differentiable in q, k
    and v. ``precision`` ``'fp32'`` (default) and ``'tf32'`` compute in fp32 (widths 128-1024), ``'bf16'`` with bf16
    operands and fp32 accumulation (widths 128-512, and 1024 with N a multiple of 16). ``causal`` asks for the
    reference's promise check only; ``chunk`` and ``max_elements`` are accepted for signature parity (the kernels
    do not chunk).
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
    return _apply(q, k, v, mask, scale, precision)


def _apply(q, k, v, mask, scale, precision):
    """The kernels of ``precision`` after the shape checks of the reference's entry points."""
    H, Rk = q.shape[2], q.shape[-1]
    widths = FORWARD_WIDTHS if precision == 'bf16' else FP32_WIDTHS
    if H != HEADS or v.shape[-1] != Rk or Rk not in widths:
        raise ValueError(f'the HIP kernels take {HEADS} heads and equal K/V widths in {widths} for precision '
                         f'{precision!r} (got H={H}, Rk={Rk}, Rv={v.shape[-1]})')
    s6_ops._dev(q, k, v, mask)
    if precision == 'bf16':
        return _CausalHistory.apply(q, k, v, mask, float(scale))
    if torch.float64 in (q.dtype, k.dtype, v.dtype):
        raise ValueError(f'precision={precision!r} computes float64 inputs in float64 in the reference; the MI355X '
                         f'kernels compute in fp32: pass float32 or bfloat16 inputs')
    return _CausalHistoryF32.apply(q, k, v, mask, float(scale))


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
        splits = s6_ops.mi355x_kv_splits(N, B, _lib.device_cus(dev.index or 0), width=R, min_keys_per_split=256)
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
    """``hla/latent/fused_history.py:129-153``: ``backend='gemm'`` runs ``causal_history_gemm`` with ``precision``;
    the reference's default ``'triton'`` backend (fp32 CUDA-core kernels) and its ``'reference'`` backend (dense
    fp32 torch autograd) compute in fp32, as the fp32 kernels here do (``precision`` and ``chunk`` apply to
    ``'gemm'`` only, as in the reference). ``reference_forward`` selects the reference's dense torch forward inside
    its Triton backend; both forwards compute the same fp32 attention, and here the fp32 kernel is the only one."""
    if q.ndim != 4 or k.ndim != 3 or v.ndim != 3 or mask.ndim != 3:
        raise ValueError(f'Expected Q[B,Lq,H,R], K/V[B,N,R], mask[B,Lq,N], got {tuple(q.shape)}, {tuple(k.shape)}, '
                         f'{tuple(v.shape)}, {tuple(mask.shape)}')
    if backend == 'gemm':
        return causal_history_gemm(q, k, v, mask, scale, causal=causal, chunk=chunk or DEFAULT_CHUNK,
                                   precision=precision)
    if backend not in HISTORY_BACKENDS:
        raise ValueError(f'Unknown causal history backend {backend!r}; expected one of {HISTORY_BACKENDS}')
    return _apply(q, k, v, mask, scale, 'fp32')


def flops(visible_pairs: int, heads: int, width: int, with_backward: bool = False) -> float:
    """Algorithmic FLOPs for ``visible_pairs`` visible (query, key) pairs, ``2 * heads * width`` per pair and GEMM:
    2 GEMMs forward (S, P V); the backward adds 5 (S again, dP, dV, dQ, dK)."""
    return 2.0 * heads * width * visible_pairs * (7 if with_backward else 2)
