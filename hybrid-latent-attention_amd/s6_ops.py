"""S6 serving ops on MI355X: the operator interface of ``hla/vllm_latent/s6_ops.py`` over hand-written HIP kernels.

Same names, argument meaning, output layouts and error behaviour as the reference module, with exactly one
implementation: the gfx950 kernels of ``libhla_s6.so`` (C ABI in ``include/hla_s6.h``). There is no torch
or CPU path; the only accepted ``backend`` string is ``'hip'`` and any other raises ``ValueError`` as the
reference does for an unknown backend. Contracts shared by all ops (``hla/vllm_latent/s6_ops.py:1-10``):
outputs are normalized attention outputs, ``lse`` is a contiguous fp32 ``[H, T]`` natural-log LSE over already
scaled scores, empty rows give ``lse = -inf`` and ``o = 0``, no NaN leaves a merge. Every op enqueues on the
current stream, allocates only its outputs (through torch's caching allocator) and never syncs with the host,
so every op is safe under HIP graph capture.
"""
from __future__ import annotations

from collections import namedtuple

import ctypes

import torch

from . import _lib

INF = float('inf')
HIP = 'hip'
Backends = namedtuple('Backends', 'history chunk merge rope')
HIP_BACKENDS = Backends(HIP, HIP, HIP, HIP)
BF16, I32, I64 = torch.bfloat16, torch.int32, torch.int64


def _backend(kind: str, backend: str) -> None:
    if backend != HIP:
        raise ValueError(f'Unknown {kind} backend {backend!r}')


def _dev(*tensors) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError('S6 ops run on the GPU only; got a tensor on ' + str(t.device))


def _bf16(name: str, t: torch.Tensor) -> None:
    if t.dtype != BF16:
        raise ValueError(f'{name} must be bfloat16, got {t.dtype}')
    if t.stride(-1) != 1:
        raise ValueError(f'{name} needs a unit last-dim stride')


def _int(name: str, t: torch.Tensor, dtype) -> torch.Tensor:
    if t.dtype != dtype:
        raise ValueError(f'{name} must be {dtype}, got {t.dtype}')
    return t if t.is_contiguous() else t.contiguous()


def _mask(t):
    if t is None:
        return None
    if t.dtype != torch.bool:
        raise ValueError('masks must be torch.bool')
    return t.contiguous()


# ----------------------------------------------------------------------------------------------------------------
# Latent RoPE (hla/vllm_latent/s6_ops.py:23-58)
# ----------------------------------------------------------------------------------------------------------------

def latent_rope(x, positions, table, backend):
    """Neox RoPE of ``x`` IN PLACE by ``table[positions]`` (``[max_position, w] = [cos | sin]``); returns ``x``.

    ``x`` is ``[T, w]``, ``[T, H, w]`` (any token/head stride, unit last stride) or ``[T, H*w]``; ``positions`` int64
    ``[T]``. Per element: ``x*cos + rotate_half(x)*sin`` with bf16 rounding after each product and the sum, the op
    order of the torch formula (``hla/vllm_latent/s6_ops.py:32-36``).
    """
    _backend('rope', backend)
    _dev(x, positions, table)
    _bf16('x', x)
    _bf16('table', table)
    w = table.shape[1]
    T = x.shape[0]
    if x.dim() == 3:
        if x.shape[-1] != w:
            raise ValueError(f'x width {x.shape[-1]} != table width {w}')
        heads, st, sh = x.shape[1], x.stride(0), x.stride(1)
    elif x.dim() == 2:
        if x.shape[1] % w:
            raise ValueError(f'x width {x.shape[1]} is not a multiple of the table width {w}')
        heads, st, sh = x.shape[1] // w, x.stride(0), w
    else:
        raise ValueError('x must be [T, w], [T, H, w] or [T, H*w]')
    pos = _int('positions', positions, I64)
    _lib.call('hla_s6_latent_rope', _lib.ptr(x), T, heads, w, st, sh, _lib.ptr(pos), _lib.ptr(table), table.shape[0],
              table.stride(0), _lib.stream(x.device))
    return x


def probe_latent_rope(table, heads=2, tokens=3):
    """Runtime check of the head-stride handling of the RoPE kernel (``hla/vllm_latent/s6_ops.py:44-58``).

    Rotates an einsum-shaped ``[T, H, w]`` view (head stride ``T*w``) and a contiguous ``[T, H*w]`` copy of the
    same values; returns ``(flat, exact)`` = ``(False, True)`` when both agree bit for bit and raises otherwise.
    """
    w = table.shape[1]
    gen = torch.Generator(device=table.device).manual_seed(0)
    x = torch.randn(heads, tokens, w, dtype=table.dtype, device=table.device, generator=gen).transpose(0, 1)
    pos = torch.randint(0, table.shape[0], (tokens,), device=table.device, generator=gen)
    flat = x.reshape(tokens, -1).clone()
    out = latent_rope(x.clone(), pos, table, HIP)   # clone() keeps the [T, H, w] transposed strides
    ref = latent_rope(flat, pos, table, HIP).view(tokens, heads, w)
    if not torch.equal(out, ref):
        raise RuntimeError('latent RoPE kernel disagrees between strided and flat layouts')
    return False, True


# ----------------------------------------------------------------------------------------------------------------
# Step metadata (hla/vllm_latent/s6_ops.py:61-114)
# ----------------------------------------------------------------------------------------------------------------

def token_requests(query_start_loc, num_tokens):
    """Request index per token (int64, clamped into range) and ``valid = arange(T) < query_start_loc[-1]``."""
    _dev(query_start_loc)
    qsl = _int('query_start_loc', query_start_loc, I32)
    R = qsl.shape[0] - 1
    req = torch.empty(num_tokens, dtype=I64, device=qsl.device)
    valid = torch.empty(num_tokens, dtype=torch.bool, device=qsl.device)
    _lib.call('hla_s6_step_metadata', _lib.ptr(qsl), R, None, num_tokens, 0, _lib.ptr(req), _lib.ptr(valid),
              None, None, None, None, _lib.stream(qsl.device))
    return req, valid


def history_lengths(seq_lens, query_start_loc):
    """Per-request history length ``seq_len - query_len``, clamped at 0 (negative at FULL-graph capture)."""
    _dev(seq_lens, query_start_loc)
    qsl = _int('query_start_loc', query_start_loc, I32)
    seq = _int('seq_lens', seq_lens, I32)
    R = qsl.shape[0] - 1
    hist = torch.empty(R, dtype=I32, device=qsl.device)
    _lib.call('hla_s6_step_metadata', _lib.ptr(qsl), R, _lib.ptr(seq), 0, 0, None, None, None, None, None,
              _lib.ptr(hist), _lib.stream(qsl.device))
    return hist


def num_kv_splits(max_seq_len, num_tokens, split_max_tokens, sm_count, head_blocks=1):
    """KV splits of the paged-history kernel for a step of ``num_tokens`` rows (``hla/vllm_latent/s6_ops.py:76-89``).

    1 above ``split_max_tokens``; otherwise enough ``rows x head_blocks x splits`` workgroups to cover every compute
    unit twice, floored by one split per 512 keys (rounded to a power of two) and capped at ``2 * sm_count`` and at
    one split per 32 keys. Depends on constants and the row count only, so a captured graph of a batch size
    always replays the split count it was captured with. ``sm_count`` is the CU count on MI355X (256).
    """
    if num_tokens > split_max_tokens:
        return 1
    by_length = 1 << (max(1, max_seq_len // 512) - 1).bit_length()
    by_occupancy = -(-2 * sm_count // (num_tokens * head_blocks))
    return max(1, min(max(by_length, by_occupancy), 2 * sm_count, -(-max_seq_len // 32)))


def mi355x_kv_splits(max_seq_len, num_tokens, cu_count=256, width=512, waves_per_cu=8, min_keys_per_split=128,
                     tokens_per_group=1, min_keys_per_group_split=256, small_step_tiles=768):
    """Split slots per row of the history kernel on MI355X for a ``width``-wide latent. The kernel runs one wave per
    128 latent columns, so a split is a workgroup of ``width / 128`` waves; about ``waves_per_cu`` resident waves per
    compute unit (8 keeps enough loads in flight to stream HBM on gfx950) make ``W = waves_per_cu * CUs / (width /
    128)`` busy workgroups. The kernel cuts every row in chunks sized so that about half of the ``num_tokens *
    slots`` workgroups get equal work whatever the row lengths (short rows use few slots, long rows many), so this
    returns ``2 * floor(W / num_tokens)`` slots (at least 2: the plan's ``num_tokens * slots / 2`` items never
    exceed W, where a ceiling gave a few CUs a third item and the launch waited on them), never more than two per
    ``min_keys_per_split`` keys of the longest row nor 1024. The kernel's plan gives every item at least 8 tiles of 16 keys (128 keys), or 4 tiles in a step
    of fewer than ``small_step_tiles`` tiles over all rows, where the history is latency-bound and shorter chains
    pay; a step that is that small even at the longest length (``num_tokens * ceil(max_seq_len / 16)`` below it)
    gets two slots per ``min_keys_per_split / 2`` keys, room for those 4-tile items. A function of constants and
    the row count only (graph-stable).

    Multi-query steps (``tokens_per_group`` 4) run one workgroup of eight tokens per (token group, slot), and every
    slot of the longest row holds work: ``ceil(2 * CUs / groups)`` slots for ``groups`` four-token groups make one
    busy workgroup per CU (8 waves at width 512, 4 at 256), never more than one per ``min_keys_per_group_split``
    keys of the longest row, at least 1 (with 512-token chunks of four requests, one slot: no split reduction at
    all)."""
    if tokens_per_group > 1:
        groups = -(-max(1, num_tokens) // tokens_per_group)
        by_length = max(1, -(-max_seq_len // min_keys_per_group_split))
        return max(1, min(-(-2 * cu_count // groups), by_length, 1024))
    waves_per_split = max(1, width // 128)
    busy = -(-waves_per_cu * cu_count // waves_per_split)
    by_occupancy = 2 * max(1, busy // max(1, num_tokens))
    small = max(1, num_tokens) * -(-max_seq_len // 16) < small_step_tiles
    keys = max(1, min_keys_per_split // 2) if small else min_keys_per_split
    by_length = max(1, 2 * -(-max_seq_len // keys))
    return max(1, min(by_occupancy, by_length, 1024))


class S6Workspace:
    """Persistent fp32 split-partials buffer of the history kernel (``hla/vllm_latent/s6_ops.py:92-114``).

    Sized for ``rows_x_splits`` (the largest ``num_tokens * num_kv_splits`` a step can request) at ``heads x
    (width_max + 1)`` floats per row-split, allocated once on first use and never grown: an oversized request
    raises ``RuntimeError`` instead of reallocating.
    """

    def __init__(self, heads, width_max, rows_x_splits):
        self.heads = heads
        self.floats = rows_x_splits * heads * (width_max + 1)
        self.buffer = None

    def ensure(self, device):
        if self.buffer is None:
            self.buffer = torch.empty(self.floats, dtype=torch.float32, device=device)
        return self.buffer

    @classmethod
    def for_splits(cls, heads, tokens, splits_by_width):
        """A workspace for ``tokens`` rows at every ``{width: splits}`` pair of ``splits_by_width``."""
        ws = cls(heads, 0, 0)
        ws.floats = max(tokens * heads * s * (w + 1) for w, s in splits_by_width.items())
        return ws

    def attn_logits(self, tokens, heads, splits, width, device=None):
        need = tokens * heads * splits * (width + 1)
        buffer = self.ensure(device)
        if need > buffer.numel():
            raise RuntimeError(f'S6 workspace overflow: need {need} floats, have {buffer.numel()}')
        return buffer[:need].view(tokens, heads, splits, width + 1)


# ----------------------------------------------------------------------------------------------------------------
# Paged latent history (hla/vllm_latent/s6_ops.py:117-222)
# ----------------------------------------------------------------------------------------------------------------

def history_attention(q_lat, cache, block_table, ctx, scale, num_kv_splits, workspace, k_scale, v_scale, backend,
                      empty=None):
    """Fully visible attention of ``q_lat[T,H,W]`` over the first ``ctx[t]`` paged latent rows of an MQA S6 cache.

    ``cache`` is the logical vLLM layout ``[num_blocks, 1, block, 2W]`` (K then V on the last dim, any strides).
    """
    W = q_lat.shape[-1]
    return history_attention_kv(q_lat, cache[..., :W], cache[..., W:], block_table, ctx, scale, num_kv_splits,
                                workspace, k_scale, v_scale, backend, empty)


def history_attention_kv(q, k, v, block_table, ctx, scale, num_kv_splits, workspace, k_scale, v_scale, backend,
                         empty=None, mla=False, bt_rows=None, tokens_per_group=1, shared_rows=False):
    """Fully visible attention of ``q[T,16,L]`` over the first ``ctx[t]`` paged rows of ``k``/``v``
    ``[num_blocks, 1, block, L]`` (MQA, page/row strides shared by K and V, unit last stride).

    ``block_table[T, max_blocks]`` int32 is per token (or per request with ``bt_rows[t]`` naming the row of token
    ``t``), ``ctx[T]`` int32. Only block-table columns ``< ceil(ctx[t] / block)`` are read. Returns
    ``(o[T,H,L] bf16, lse[H,T] fp32)``; empty rows give ``o = 0``, ``lse = -inf``. ``k_scale``/``v_scale`` belong
    to quantized caches, which the S6 adapter rejects (``hla/vllm_latent/ouro_latent.py:103-104``): they are
    accepted and unused. ``empty`` is derived from ``ctx`` inside the kernel and is accepted for signature parity.
    ``tokens_per_group`` (1, 2 or 4) lets one workgroup serve that many consecutive tokens that share a block-table
    row (the query rows of one request in a chunked-prefill step) from a single read of each K/V tile.
    ``shared_rows`` declares that several tokens read the same rows, so K/V loads are cached for the re-reads
    (decode steps read every row once and stream it past the caches).
    """
    _backend('history', backend)
    T, H, L, ctx, rows = _history_operands(q, k, v, block_table, ctx, mla, bt_rows)
    o = torch.empty(T, H, L, dtype=BF16, device=q.device)
    lse = torch.empty(H, T, dtype=torch.float32, device=q.device)
    splits = int(num_kv_splits)
    ws = None
    if splits > 1:
        if workspace is None:
            raise RuntimeError('history attention with num_kv_splits > 1 needs an S6Workspace')
        ws = workspace.attn_logits(T, H, splits, L, q.device)
    args = (_lib.ptr(q), T, H, L, q.stride(0), q.stride(1), _lib.ptr(k), _lib.ptr(v), k.stride(0), k.stride(2),
            k.shape[2], k.shape[0], _lib.ptr(block_table), block_table.stride(0), block_table.shape[1], _lib.ptr(rows),
            _lib.ptr(ctx), float(scale), splits, _lib.ptr(ws), 0 if ws is None else ws.numel(), _lib.ptr(o),
            o.stride(0), o.stride(1), _lib.ptr(lse))
    if int(tokens_per_group) == 1 and not shared_rows:
        _lib.call('hla_s6_history_attention', *args, _lib.stream(q.device))
    else:
        _lib.call('hla_s6_history_attention_grouped', *args, int(tokens_per_group), int(bool(shared_rows)),
                  _lib.stream(q.device))
    return o, lse


def history_partials(q, k, v, block_table, ctx, scale, num_kv_splits, workspace, bt_rows=None, plan=None):
    """Stage 1 of the history op alone, the split kernel (``hla/vllm_latent/s6_ops.py:186-196``): writes the
    normalized per-split partials and their lse to ``workspace`` for any ``num_kv_splits >= 1`` and returns the
    workspace view ``[T, H, splits, width + 1]`` (its layout is private to the HIP library). Operands and checks as
    ``history_attention_kv``; ``history_reduce`` completes the op bitwise. ``plan`` is an optional precomputed
    split plan (``split_plan``)."""
    T, H, L, ctx, rows = _history_operands(q, k, v, block_table, ctx, False, bt_rows)
    splits = int(num_kv_splits)
    if workspace is None:
        raise RuntimeError('history partials need an S6Workspace')
    ws = workspace.attn_logits(T, H, splits, L, q.device)
    _lib.call('hla_s6_history_partials', _lib.ptr(q), T, H, L, q.stride(0), q.stride(1), _lib.ptr(k), _lib.ptr(v),
              k.stride(0), k.stride(2), k.shape[2], k.shape[0], _lib.ptr(block_table), block_table.stride(0),
              block_table.shape[1], _lib.ptr(rows), _lib.ptr(ctx), float(scale), splits, _lib.ptr(ws), ws.numel(),
              _lib.ptr(plan), 0 if plan is None else plan.numel(), _lib.stream(q.device))
    return ws


def split_plan(ctx, cap, num_kv_splits, query_start_loc=None):
    """The split plan of the history kernels for history lengths ``ctx[T]`` (int32), ``cap`` addressable rows per
    token and ``num_kv_splits`` slots per row (``hla_s6_split_plan``): computed once on the GPU, reusable by every
    history call of the step with the same lengths. With ``query_start_loc``, the tokens of a short chunk (2..16
    tokens of a request with equal lengths) have their chunks listed together, so their shared rows are read from
    HBM once."""
    _dev(ctx, query_start_loc)
    ctx = _int('ctx', ctx, I32)
    qsl = None if query_start_loc is None else _int('query_start_loc', query_start_loc, I32)
    T, splits = ctx.shape[0], int(num_kv_splits)
    n = _lib.load().hla_s6_split_plan_ints(T, splits)
    plan = torch.empty(max(int(n), 1), dtype=I32, device=ctx.device)
    _lib.call('hla_s6_split_plan', _lib.ptr(ctx), T, int(cap), splits, _lib.ptr(qsl),
              0 if qsl is None else qsl.shape[0] - 1, _lib.ptr(plan), plan.numel(), _lib.stream(ctx.device))
    return plan


def split_plans(ctx, cap, splits, query_start_loc=None):
    """The plans of ``split_plan`` for several slot counts over the same lengths (a step's latent widths run
    different counts over the same rows) in one launch (``hla_s6_split_plans``, at most 4); returns them in the
    order of ``splits``."""
    _dev(ctx, query_start_loc)
    ctx = _int('ctx', ctx, I32)
    qsl = None if query_start_loc is None else _int('query_start_loc', query_start_loc, I32)
    T, splits = ctx.shape[0], [int(s) for s in splits]
    lib = _lib.load()
    plans = [torch.empty(max(int(lib.hla_s6_split_plan_ints(T, s)), 1), dtype=I32, device=ctx.device) for s in splits]
    n = len(plans)
    _lib.call('hla_s6_split_plans', _lib.ptr(ctx), T, int(cap), n, (ctypes.c_int32 * n)(*splits), _lib.ptr(qsl),
              0 if qsl is None else qsl.shape[0] - 1, (ctypes.c_void_p * n)(*[p.data_ptr() for p in plans]),
              (ctypes.c_int64 * n)(*[p.numel() for p in plans]), _lib.stream(ctx.device))
    return plans


def history_reduce(partials):
    """Stage 2 of the history op (``hla/vllm_latent/s6_ops.py:202``, ``_decode_softmax_reducev_fwd``): the LSE
    reduction of the split partials ``history_partials`` returned. Returns ``(o[T,H,L] bf16, lse[H,T] fp32)``."""
    _dev(partials)
    if partials.dtype != torch.float32 or partials.dim() != 4 or not partials.is_contiguous():
        raise ValueError('history_reduce expects the fp32 workspace view returned by history_partials')
    T, H, S, L1 = partials.shape
    L = L1 - 1
    o = torch.empty(T, H, L, dtype=BF16, device=partials.device)
    lse = torch.empty(H, T, dtype=torch.float32, device=partials.device)
    _lib.call('hla_s6_history_reduce', _lib.ptr(partials), partials.numel(), T, H, L, S, _lib.ptr(o), o.stride(0),
              o.stride(1), _lib.ptr(lse), _lib.stream(partials.device))
    return o, lse


def history_partials_grouped(q, k, v, block_table, ctx, scale, num_kv_splits, workspace, bt_rows=None,
                             tokens_per_group=4):
    """The split kernel of ``history_attention_kv(..., tokens_per_group=2 or 4)`` writing only its per-slot partials
    (every slot, empty ones with lse = -inf) to ``workspace``; returns the workspace view ``[T, H, splits, width + 1]``
    for ``split_epilogue``. Operands and checks as ``history_attention_kv``."""
    T, H, L, ctx, rows = _history_operands(q, k, v, block_table, ctx, False, bt_rows)
    splits = int(num_kv_splits)
    if workspace is None:
        raise RuntimeError('history partials need an S6Workspace')
    ws = workspace.attn_logits(T, H, splits, L, q.device)
    _lib.call('hla_s6_history_partials_grouped', _lib.ptr(q), T, H, L, q.stride(0), q.stride(1), _lib.ptr(k),
              _lib.ptr(v), k.stride(0), k.stride(2), k.shape[2], k.shape[0], _lib.ptr(block_table),
              block_table.stride(0), block_table.shape[1], _lib.ptr(rows), _lib.ptr(ctx), float(scale), splits,
              _lib.ptr(ws), ws.numel(), int(tokens_per_group), _lib.stream(q.device))
    return ws


def split_epilogue(partials, B, o_win, lse_win, invalid):
    """``merge_states(bf16(o_hist) @ B, lse_hist, o_win, lse_win, invalid)`` with ``(o_hist, lse_hist)`` the LSE
    reduction of the split partials (``history_partials_grouped``) in one launch, the epilogue of the fused decode
    step; ``num_kv_splits >= 2``. B ``[16, width, 128]``, o_win ``[T, 16, 128]`` bf16 and lse_win ``[16, T]``
    contiguous. Returns ``[T, 16, 128]`` bf16 with ``invalid`` rows zeroed."""
    _dev(partials, B, o_win, lse_win, invalid)
    if partials.dtype != torch.float32 or partials.dim() != 4 or not partials.is_contiguous():
        raise ValueError('split_epilogue expects the fp32 workspace view returned by history_partials_grouped')
    T, H, S, L1 = partials.shape
    _bf16('B', B)
    _bf16('o_win', o_win)
    if tuple(B.shape) != (H, L1 - 1, o_win.shape[-1]) or B.stride(-1) != 1:
        raise ValueError(f'B must be [{H}, {L1 - 1}, {o_win.shape[-1]}] with a unit last stride, got {tuple(B.shape)}')
    if not o_win.is_contiguous() or tuple(o_win.shape[:2]) != (T, H) or tuple(lse_win.shape) != (H, T):
        raise ValueError('o_win [T, 16, 128] and lse_win [16, T] must be contiguous partials of the same tokens')
    lse_win = lse_win.to(torch.float32).contiguous()
    inv = _mask(invalid)
    if inv is not None and tuple(inv.shape) != (T,):
        raise ValueError(f'invalid must be [{T}] bool')
    out = torch.empty(T, H, o_win.shape[-1], dtype=BF16, device=o_win.device)
    _lib.call('hla_s6_split_epilogue', _lib.ptr(partials), partials.numel(), T, H, L1 - 1, S, _lib.ptr(B),
              B.stride(0), B.stride(1), _lib.ptr(o_win), _lib.ptr(lse_win), _lib.ptr(inv), _lib.ptr(out),
              out.stride(0), out.stride(1), _lib.stream(o_win.device))
    return out


def _history_operands(q, k, v, block_table, ctx, mla, bt_rows):
    """Checks of the history operands; returns ``(T, H, L, ctx int32, bt_rows int64 or None)``."""
    if mla:
        raise ValueError('MLA-style rows (value = prefix of key) are not part of the S6 path')
    _dev(q, k, v, block_table, ctx)
    _bf16('q', q)
    _bf16('k', k)
    _bf16('v', v)
    T, H, L = q.shape
    if k.dim() != 4 or v.dim() != 4 or k.shape[1] != 1 or v.shape[1] != 1:
        raise ValueError('history attention expects an MQA cache [num_blocks, 1, block, width]')
    if k.shape[-1] != L or v.shape[-1] != L:
        raise ValueError(f'latent widths differ: q {L}, k {k.shape[-1]}, v {v.shape[-1]}')
    if k.stride(0) != v.stride(0) or k.stride(2) != v.stride(2):
        raise ValueError('K and V must share page and row strides (halves of one cache)')
    if block_table.dtype != I32 or block_table.stride(-1) != 1:
        raise ValueError('block_table must be int32 with a unit last stride')
    ctx = _int('ctx', ctx, I32)
    if ctx.shape[0] != T:
        raise ValueError(f'ctx has {ctx.shape[0]} rows for {T} tokens')
    if bt_rows is None and block_table.shape[0] < T:
        raise ValueError(f'block_table has {block_table.shape[0]} rows for {T} tokens')
    rows = None if bt_rows is None else _int('bt_rows', bt_rows, I64)
    return T, H, L, ctx, rows


# ----------------------------------------------------------------------------------------------------------------
# Current chunk, exact window and merges (hla/vllm_latent/s6_ops.py:234-361)
# ----------------------------------------------------------------------------------------------------------------

def chunk_attention(q, k, v, query_start_loc, max_query_len, invalid, scale, backend):
    """Causal attention within each request's current chunk (``q, k, v`` are ``[T,H,d]``).

    Returns ``(o[T,H,d] bf16, lse[H,T] fp32)``; tokens past ``query_start_loc[-1]`` (the ``invalid`` rows) give
    ``o = 0``, ``lse = -inf``. ``max_query_len`` and ``invalid`` are accepted for signature parity.
    """
    _backend('chunk', backend)
    _dev(q, k, v, query_start_loc)
    for name, t in (('q', q), ('k', k), ('v', v)):
        _bf16(name, t)
    qsl = _int('query_start_loc', query_start_loc, I32)
    T, H, d = q.shape
    o = torch.empty(T, H, d, dtype=BF16, device=q.device)
    lse = torch.empty(H, T, dtype=torch.float32, device=q.device)
    _lib.call('hla_s6_chunk_attention', _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), T, H, d, q.stride(0), q.stride(1),
              k.stride(0), k.stride(1), v.stride(0), v.stride(1), _lib.ptr(qsl), qsl.shape[0] - 1, float(scale),
              _lib.ptr(o), o.stride(0), o.stride(1), _lib.ptr(lse), _lib.stream(q.device))
    return o, lse


def chunk_window_attention(q, k, v, query_start_loc, seq_lens, cache, block_table, window, scale, backend):
    """``chunk_attention`` merged with ``window_history_fa`` in one softmax: every token of request ``r`` attends to
    the exact-cache history rows ``[ctx_r - window, ctx_r)`` (``ctx_r = seq_lens[r] - query length``, read through
    the per-request ``block_table``) and to its request's chunk tokens up to itself.

    Same outputs as ``merge_lse(chunk_attention(...), window_history_fa(...))`` up to the bf16 rounding of the two
    partial outputs, which the one-pass form does not make; ``cache`` is ``[num_blocks, H, block, 2d]`` (K then V).
    """
    _backend('chunk', backend)
    _dev(q, k, v, query_start_loc, seq_lens, cache, block_table)
    for name, t in (('q', q), ('k', k), ('v', v), ('cache', cache)):
        _bf16(name, t)
    qsl = _int('query_start_loc', query_start_loc, I32)
    sl = _int('seq_lens', seq_lens, I32)
    T, H, d = q.shape
    R = qsl.shape[0] - 1
    if cache.dim() != 4 or cache.shape[1] != H or cache.shape[-1] != 2 * d:
        raise ValueError(f'exact cache must be [num_blocks, {H}, block, {2 * d}], got {tuple(cache.shape)}')
    if block_table.dtype != I32 or block_table.stride(-1) != 1:
        raise ValueError('block_table must be int32 with a unit last stride')
    if block_table.shape[0] < R or sl.shape[0] < R:
        raise ValueError(f'per-request block_table / seq_lens need {R} rows')
    o = torch.empty(T, H, d, dtype=BF16, device=q.device)
    lse = torch.empty(H, T, dtype=torch.float32, device=q.device)
    _lib.call('hla_s6_chunk_window_attention', _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), T, H, d, q.stride(0),
              q.stride(1), k.stride(0), k.stride(1), v.stride(0), v.stride(1), _lib.ptr(qsl), _lib.ptr(sl), R,
              _lib.ptr(cache), _lib.ptr(cache[..., d:]), cache.stride(0), cache.stride(2), cache.stride(1),
              cache.shape[2], cache.shape[0], _lib.ptr(block_table), block_table.stride(0), block_table.shape[1],
              int(window), float(scale), _lib.ptr(o), o.stride(0), o.stride(1), _lib.ptr(lse), _lib.stream(q.device))
    return o, lse


def merge_states(o_hist, lse_hist, o_chunk, lse_chunk, invalid, backend):
    """LSE merge of two partial softmaxes; ``[T,H,D]`` outputs, ``[H,T]`` fp32 lse; ``invalid`` rows are zeroed.

    ``+inf`` lse counts as empty (the FA2 empty-key convention); both sides empty give 0.
    """
    _backend('merge', backend)
    _dev(o_hist, lse_hist, o_chunk, lse_chunk)
    _bf16('o_hist', o_hist)
    _bf16('o_chunk', o_chunk)
    T, H, D = o_chunk.shape
    out = torch.empty(T, H, D, dtype=BF16, device=o_chunk.device)
    lh, lc = lse_hist.float().contiguous(), lse_chunk.float().contiguous()
    _lib.call('hla_s6_merge_states', _lib.ptr(o_hist), o_hist.stride(0), o_hist.stride(1), _lib.ptr(lh),
              _lib.ptr(o_chunk), o_chunk.stride(0), o_chunk.stride(1), _lib.ptr(lc), _lib.ptr(_mask(invalid)), T, H, D,
              0, _lib.ptr(out), out.stride(0), out.stride(1), None, _lib.stream(out.device))
    return out


def merge_lse(o1, lse1, o2, lse2):
    """LSE merge that also returns the merged lse (``[T,H,d]`` outputs, ``[H,T]`` lse); both empty -> 0, -inf.
    NaN entries of either output (scratch rows) count as 0."""
    _dev(o1, lse1, o2, lse2)
    _bf16('o1', o1)
    _bf16('o2', o2)
    T, H, D = o1.shape
    out = torch.empty(T, H, D, dtype=BF16, device=o1.device)
    lse = torch.empty(H, T, dtype=torch.float32, device=o1.device)
    l1, l2 = lse1.float().contiguous(), lse2.float().contiguous()
    _lib.call('hla_s6_merge_states', _lib.ptr(o1), o1.stride(0), o1.stride(1), _lib.ptr(l1), _lib.ptr(o2),
              o2.stride(0), o2.stride(1), _lib.ptr(l2), None, T, H, D, 1, _lib.ptr(out), out.stride(0), out.stride(1),
              _lib.ptr(lse), _lib.stream(out.device))
    return out, lse


def _exact_call(q, cache, block_table, mode, qsl, seq_lens, ctx, window, scale, bt_rows=None):
    _dev(q, cache, block_table)
    _bf16('q', q)
    _bf16('cache', cache)
    T, H, d = q.shape
    if cache.dim() != 4 or cache.shape[1] != H or cache.shape[-1] != 2 * d:
        raise ValueError(f'exact cache must be [num_blocks, {H}, block, {2 * d}], got {tuple(cache.shape)}')
    if block_table.dtype != I32 or block_table.stride(-1) != 1:
        raise ValueError('block_table must be int32 with a unit last stride')
    R = 0 if qsl is None else qsl.shape[0] - 1
    if mode == 0 and (block_table.shape[0] < R or seq_lens.shape[0] < R):
        raise ValueError(f'per-request block_table / seq_lens need {R} rows')
    if mode == 1 and (ctx.shape[0] != T or (bt_rows is None and block_table.shape[0] < T)):
        raise ValueError(f'per-token block_table / ctx need {T} rows')
    o = torch.empty(T, H, d, dtype=BF16, device=q.device)
    lse = torch.empty(H, T, dtype=torch.float32, device=q.device)
    _lib.call('hla_s6_window_attention', _lib.ptr(q), T, H, d, q.stride(0), q.stride(1), _lib.ptr(cache),
              _lib.ptr(cache[..., d:]), cache.stride(0), cache.stride(2), cache.stride(1), cache.shape[2],
              cache.shape[0], _lib.ptr(block_table), block_table.stride(0), block_table.shape[1], _lib.ptr(bt_rows),
              mode, _lib.ptr(qsl),
              _lib.ptr(seq_lens), R, _lib.ptr(ctx), int(window), float(scale), _lib.ptr(o), o.stride(0), o.stride(1),
              _lib.ptr(lse), _lib.stream(q.device))
    return o, lse


def window_attention(q, cache, block_table, ctx, window, scale):
    """Exact attention of ``q[T,H,d]`` (roped) over history rows ``[ctx[t] - window, ctx[t])`` of a paged exact cache.

    ``cache`` is the TRITON_ATTN logical layout ``[num_blocks, H, block, 2d]`` (K then V), ``block_table[T, *]`` per
    token. Rows without window history give ``o = 0``, ``lse = -inf``.
    """
    return _exact_call(q, cache, block_table, 1, None, None, _int('ctx', ctx, I32), window, scale)


def window_attention_fa(q, cache, block_table, query_start_loc, seq_lens, window, scale, max_seqlen_k, invalid):
    """Decode exact window: keys ``[seq_len - 1 - window, seq_len - 1]`` (the window history plus the current token,
    already written) of a TRITON_ATTN cache ``[nb, H, block, 2d]``, per-request ``block_table`` / ``seq_lens``.

    Returns ``(o[T,H,d], lse[H,T] fp32)``; ``invalid`` rows (tokens past ``query_start_loc[-1]``) get ``o = 0``,
    ``lse = -inf``. ``max_seqlen_k`` and ``invalid`` are accepted for signature parity.
    """
    qsl = _int('query_start_loc', query_start_loc, I32)
    return _exact_call(q, cache, block_table, 0, qsl, _int('seq_lens', seq_lens, I32), None, window, scale)


def window_history_fa(q, cache, token_block_table, ctx, window, scale, max_seqlen_k, empty):
    """Exact window over history keys only (non-decode steps): token ``t`` reads rows ``[ctx[t] - window, ctx[t])``
    with a per-token table; rows without history (``empty``) give ``o = 0``, ``lse = -inf``."""
    return _exact_call(q, cache, token_block_table, 1, None, None, _int('ctx', ctx, I32), window, scale)


def select_backends(head_size=128):
    """The HIP kernel set; raises ``RuntimeError`` when no GPU or no library is available."""
    if not torch.cuda.is_available():
        raise RuntimeError('S6 serving ops require a GPU (gfx950)')
    if head_size != 128:
        raise RuntimeError(f'exact-window kernels are built for head_size 128, not {head_size}')
    _lib.load()
    return HIP_BACKENDS
