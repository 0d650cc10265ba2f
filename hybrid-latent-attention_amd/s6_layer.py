"""S6 attention of one layer x loop on MI355X: the interface of ``hla/vllm_latent/s6_layer.py`` over the HIP ops.

The adapter builds one ``StepContext`` per step and, per layer and loop, calls ``latent_query`` before the
(in-place) exact RoPE, then ``attend``, ``write_rows`` and ``committed_row``. Latent RoPE reads persistent per-width
``[max_position, w]`` tables built once by ``latent_rope_table``. Everything here is sync-free and loops over no
requests; ``sl`` is the layer's ``LatentLayer``-shaped module (``readers(loop)``, ``write1``, ``write_step``,
``rank``, ``rank1``, ``loops``; ``hla/latent/register.py:28-95``).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib, s6_ops


def latent_inv_freq(head_dim, theta):
    """The teacher's ``head_dim/2`` RoPE frequencies (HF/vLLM ``inv_freq``; ``hla/vllm_latent/s6_layer.py:16-18``)."""
    return 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64).float() / head_dim))


def latent_rope_table(max_position, inv_freq, width, dtype):
    """``[max_position, width]`` = ``[cos | sin]`` halves of the latent angles; the teacher frequencies are reused
    round-robin over the ``width/2`` rotation pairs, angle ``p * inv_freq`` in fp32, then cast
    (``hla/vllm_latent/s6_layer.py:21-29``)."""
    pair = torch.arange(width // 2, device=inv_freq.device) % inv_freq.shape[0]
    angle = torch.arange(max_position, device=inv_freq.device).float()[:, None] * inv_freq[pair][None, :]
    return torch.cat((angle.cos(), angle.sin()), -1).to(dtype)


def latent_query(q_pre_rope, A, positions, table, backend, flat=False):
    """``[T,H,d]`` pre-RoPE query -> latent-rotated ``[T,H,w]`` (contiguous) = RoPE(einsum('thd,hdr->thr', q, A)).

    One fused HIP launch (absorption GEMM on MFMA with the latent RoPE in its epilogue); follows
    ``hla/vllm_latent/s6_layer.py:32-40``. ``flat`` is accepted for signature parity: the kernel writes its own
    contiguous output.
    """
    s6_ops._backend('rope', backend)
    s6_ops._dev(q_pre_rope, A, positions, table)
    s6_ops._bf16('q_pre_rope', q_pre_rope)
    s6_ops._bf16('A', A)
    s6_ops._bf16('table', table)
    T, H, d = q_pre_rope.shape
    w = A.shape[-1]
    if A.shape[:2] != (H, d) or table.shape[1] != w:
        raise ValueError(f'A {tuple(A.shape)} / table {tuple(table.shape)} do not match q {tuple(q_pre_rope.shape)}')
    out = torch.empty(T, H, w, dtype=q_pre_rope.dtype, device=q_pre_rope.device)
    pos = s6_ops._int('positions', positions, torch.int64)
    _lib.call('hla_s6_absorb', _lib.ptr(q_pre_rope), T, H, d, q_pre_rope.stride(0), q_pre_rope.stride(1), _lib.ptr(A),
              A.stride(0), A.stride(1), w, _lib.ptr(out), out.stride(0), out.stride(1), _lib.ptr(pos), _lib.ptr(table),
              table.shape[0], table.stride(0), _lib.stream(out.device))
    return out


def absorb_out(o_lat, B):
    """``einsum('thr,hrd->thd', o_lat, B)`` on MFMA (the ``B_t`` projection of ``hla/vllm_latent/s6_layer.py:114``)."""
    s6_ops._bf16('o_lat', o_lat)
    s6_ops._bf16('B', B)
    T, H, r = o_lat.shape
    d = B.shape[-1]
    out = torch.empty(T, H, d, dtype=o_lat.dtype, device=o_lat.device)
    _lib.call('hla_s6_absorb', _lib.ptr(o_lat), T, H, r, o_lat.stride(0), o_lat.stride(1), _lib.ptr(B), B.stride(0),
              B.stride(1), d, _lib.ptr(out), out.stride(0), out.stride(1), None, None, 0, 0, _lib.stream(out.device))
    return out


class StepContext:
    """Per-step tensors shared by every layer and loop (``hla/vllm_latent/s6_layer.py:43-84``).

    ``query_start_loc=None`` means a metadata-less (profiling) step: one request spanning all tokens, no history and
    no cache writes (``md_present`` False), workspace still allocated. ``tables`` maps a latent width to its
    persistent ``[max_position, w]`` RoPE table. Token -> request, ``ctx`` and ``ctx_latent`` come from one HIP
    launch; all shapes depend only on ``num_tokens`` and host ints; nothing here syncs with the host.

    Split counts: the reference adapter passes one ``num_kv_splits`` for both latent widths
    (``hla/vllm_latent/ouro_latent.py:257``). The history kernel's occupancy depends on the width (one wave per 128
    columns), so when the step has metadata, ``max_seqlen_k`` and a workspace, each width takes the MI355X count
    ``s6_ops.mi355x_kv_splits(max_seqlen_k, num_tokens, CUs, width, history_group)`` if the workspace holds its
    partials, and ``num_kv_splits`` otherwise. Like the reference's count it depends on the row count and
    constants only (``max_query_len`` picks the kernel family, as ``history_group`` always has), so a graph captured
    for a batch size replays the counts it was captured with; a split count changes only the order of the fp32
    sums. ``kv_splits_by_width`` overrides the counts per width (the workspace must hold the largest of them).
    """

    def __init__(self, positions, query_start_loc, seq_lens, max_query_len, num_tokens, tables, scale, backends,
                 workspace=None, num_kv_splits=1, rope_flat=False, window=0, max_seqlen_k=0,
                 kv_splits_by_width=None):
        device = positions.device
        self.window, self.max_seqlen_k = window, max_seqlen_k
        self.positions, self.tables, self.scale, self.backends = positions, tables, scale, backends
        self.workspace, self.num_kv_splits, self.rope_flat = workspace, num_kv_splits, rope_flat
        self.kv_splits_by_width = dict(kv_splits_by_width or {})
        # query rows per workgroup of the history kernel: chunked-prefill steps with long chunks serve four tokens
        # of a request per workgroup (the MFMA multi-query kernel); short chunks keep one token per workgroup, which
        # gives the GPU more workgroups
        self.history_group = 4 if (max_query_len or 1) >= 16 else 1
        self.history_needed = True
        # chunks shorter than FUSED_CHUNK_TOKENS attend through the fused decode path, reading their own keys from
        # the exact cache (which the adapter writes before attending), and longer ones with split history reduce
        # their splits, apply B_t and merge in one epilogue; False: the reference's op sequence
        self.fused_chunks = True
        self.md_present = query_start_loc is not None
        if not self.md_present:
            query_start_loc = torch.tensor([0, num_tokens], dtype=torch.int32, device=device)
            seq_lens, max_query_len = query_start_loc[1:], num_tokens
        self.query_start_loc, self.seq_lens, self.max_query_len = query_start_loc, seq_lens, max_query_len
        qsl = s6_ops._int('query_start_loc', query_start_loc, torch.int32)
        seq = s6_ops._int('seq_lens', seq_lens, torch.int32)
        R = qsl.shape[0] - 1
        self.token_requests = torch.empty(num_tokens, dtype=torch.int64, device=device)
        self.valid = torch.empty(num_tokens, dtype=torch.bool, device=device)
        self.invalid = torch.empty(num_tokens, dtype=torch.bool, device=device)
        self.ctx = torch.empty(num_tokens, dtype=torch.int32, device=device)
        self.ctx_latent = torch.empty(num_tokens, dtype=torch.int32, device=device)
        _lib.call('hla_s6_step_metadata', _lib.ptr(qsl), R, _lib.ptr(seq), num_tokens, int(window or 0),
                  _lib.ptr(self.token_requests), _lib.ptr(self.valid), _lib.ptr(self.invalid), _lib.ptr(self.ctx),
                  _lib.ptr(self.ctx_latent), None, _lib.stream(device))
        self._empty = self._empty_latent = None
        self._block_tables = {}
        self._plans = {}
        self._slots = {}
        if workspace is not None:
            workspace.ensure(device)
            if kv_splits_by_width is None and self.md_present and max_seqlen_k:
                self.kv_splits_by_width = self._mi355x_splits(workspace, num_tokens, device)

    def _mi355x_splits(self, workspace, num_tokens, device):
        """``{width: splits}`` of the MI355X policy for every latent width with a RoPE table, where the workspace
        holds ``num_tokens * heads * splits * (width + 1)`` partials (other widths keep ``num_kv_splits``)."""
        cus = _lib.device_cus(device.index or 0)
        heads = getattr(workspace, 'heads', None) or 16
        out = {}
        for width in self.tables:
            s = s6_ops.mi355x_kv_splits(int(self.max_seqlen_k), int(num_tokens), cus, width=int(width),
                                        tokens_per_group=self.history_group)
            if s == 1 or num_tokens * heads * s * (int(width) + 1) <= workspace.floats:
                out[int(width)] = s
        return out

    @property
    def empty(self):
        """Tokens without history (``ctx == 0``), computed on first use: the fused steps never read it."""
        if self._empty is None:
            self._empty = self.ctx == 0
        return self._empty

    @property
    def empty_latent(self):
        """Tokens without latent history (``ctx_latent == 0``), computed on first use."""
        if self._empty_latent is None:
            self._empty_latent = self.ctx_latent == 0
        return self._empty_latent

    def kv_splits(self, width):
        """History split count for a latent of ``width`` columns."""
        return int(self.kv_splits_by_width.get(width, self.num_kv_splits))

    def split_plan(self, splits, cap):
        """The step's split plan of the latent history (``hla_s6_split_plan``) for ``splits`` slots per row and
        ``cap`` addressable rows, read by every layer. The first request of a step makes, in the same launch, the
        plans of the other latent widths' slot counts for the same ``cap`` (``hla_s6_split_plans``: the widths'
        tables address the same pages), so a step computes its plans with one launch."""
        key = (int(splits), int(cap))
        if key not in self._plans:
            qsl = self.query_start_loc if self.max_query_len > 1 else None   # short chunks share rows
            others = sorted({self.kv_splits(w) for w in self.tables} - {key[0]} -
                            {s for s, c in self._plans if c == key[1]})
            counts = [key[0]] + [s for s in others if s > 1][:3]
            for s, plan in zip(counts, s6_ops.split_plans(self.ctx_latent, key[1], counts, qsl)):
                self._plans[(s, key[1])] = plan
        return self._plans[key]

    def slots(self, table, block_size):
        """Commit slot of every token for a per-request block table (``slot_mapping``), once per table per step."""
        key = (table.data_ptr(), int(block_size))
        if key not in self._slots:
            self._slots[key] = slot_mapping(self, table, block_size)
        return self._slots[key]

    def block_table(self, table):
        """Per-token gather of a per-request block table, done once per distinct tensor per step."""
        key = table.data_ptr()
        if key not in self._block_tables:
            if table.dtype != torch.int32 or table.stride(-1) != 1:
                raise ValueError('block tables must be int32 with a unit last stride')
            T, cols = self.token_requests.shape[0], table.shape[1]
            out = torch.empty(T, cols, dtype=torch.int32, device=table.device)
            _lib.call('hla_s6_gather_block_table', _lib.ptr(table), table.stride(0), table.shape[0], cols,
                      _lib.ptr(self.token_requests), T, _lib.ptr(out), out.stride(0), _lib.stream(table.device))
            self._block_tables[key] = out
        return self._block_tables[key]

    def latent_query(self, sl, loop, q_pre_rope):
        A, _, width = sl.readers(loop)
        return latent_query(q_pre_rope, A, self.positions, self.tables[width], self.backends.rope, self.rope_flat)


# Steps whose longest chunk is shorter than this take the fused decode path (one token per history workgroup);
# longer chunks take the multi-query kernels (eight tokens of a request per workgroup).
FUSED_CHUNK_TOKENS = 16


def attend(sl, loop, q_lat, q_rope, k_rope, v, cache, block_table, k_scale, v_scale, ctx, window=None):
    """One softmax over the paged latent history (fully visible) and the causal current chunk
    (``hla/vllm_latent/s6_layer.py:87-115``).

    ``q_lat`` comes from ``StepContext.latent_query``; ``q_rope``, ``k_rope``, ``v`` are ``[T,H,d]``; ``cache`` is the
    layer's ``[num_blocks,1,block,2w]`` tensor or None (no history); ``block_table`` is the per-request table;
    ``window`` is ``(exact_cache, per-request block_table)`` or None. Returns ``[T,H,d]`` with ``~valid`` rows zeroed.
    Decode steps with history run as one fused call (history + exact window in one launch, the split reduction,
    then the ``B_t`` projection fused with the LSE merge). So do steps whose chunks are shorter than
    ``FUSED_CHUNK_TOKENS`` tokens (``ctx.fused_chunks``): their exact part is one softmax per query over the exact
    cache's rows ``[ctx - W, p]``, the window history and the chunk up to the query, which the adapter has written
    to the exact cache before attending (``hla/vllm_latent/ouro_latent.py:120-122``), so it equals the reference's
    causal chunk of ``k_rope`` / ``v`` merged with its window history. Longer chunks with split history
    (``kv_splits > 1``) compute their chunk + window partial as the reference does, then the history kernels' split
    partials, and one epilogue reduces the splits, applies ``B_t`` and merges (the decode step's epilogue). Other
    steps compose the single ops in the reference's order.
    """
    fused = window is not None and ctx.md_present and (ctx.max_query_len == 1 or
                                                       (ctx.fused_chunks and ctx.max_query_len < FUSED_CHUNK_TOKENS))
    has_history = cache is not None and ctx.md_present and ctx.history_needed
    if fused and has_history:
        return _attend_decode(sl, loop, q_lat, q_rope, cache, block_table, ctx, window)
    if fused:
        o_chunk, lse_chunk = s6_ops.window_attention_fa(q_rope, window[0], window[1], ctx.query_start_loc, ctx.seq_lens,
                                                        ctx.window, ctx.scale, ctx.max_seqlen_k, ctx.invalid)
    elif window is not None and has_history:  # the chunk and its exact window history in one softmax
        o_chunk, lse_chunk = s6_ops.chunk_window_attention(q_rope, k_rope, v, ctx.query_start_loc, ctx.seq_lens,
                                                           window[0], window[1], ctx.window, ctx.scale,
                                                           ctx.backends.chunk)
    else:
        o_chunk, lse_chunk = s6_ops.chunk_attention(q_rope, k_rope, v, ctx.query_start_loc, ctx.max_query_len,
                                                    ctx.invalid, ctx.scale, ctx.backends.chunk)
    if not has_history:
        return o_chunk.masked_fill_(ctx.invalid[:, None, None], 0)
    _, B, _ = sl.readers(loop)
    w = q_lat.shape[-1]
    if window is not None and ctx.fused_chunks and ctx.history_group > 1 and ctx.kv_splits(w) > 1:
        # multi-query step with split history: the grouped kernels' split partials, then the fused decode step's
        # epilogue (LSE reduction, B_t, merge with the chunk + window partial) in place of history_attention,
        # the B_t einsum and merge_states
        for kind in ('history', 'merge'):
            s6_ops._backend(kind, getattr(ctx.backends, kind))
        ws = s6_ops.history_partials_grouped(q_lat, cache[..., :w], cache[..., w:], block_table, ctx.ctx_latent,
                                             ctx.scale, ctx.kv_splits(w), ctx.workspace, bt_rows=ctx.token_requests,
                                             tokens_per_group=ctx.history_group)
        return s6_ops.split_epilogue(ws, B, o_chunk, lse_chunk, ctx.invalid)
    o_hist, lse_hist = s6_ops.history_attention_kv(q_lat, cache[..., :w], cache[..., w:], block_table, ctx.ctx_latent,
                                                   ctx.scale, ctx.kv_splits(w), ctx.workspace, k_scale, v_scale,
                                                   ctx.backends.history, ctx.empty_latent, bt_rows=ctx.token_requests,
                                                   tokens_per_group=ctx.history_group,
                                                   shared_rows=ctx.max_query_len > 1)
    o_hist = absorb_out(o_hist, B)
    return s6_ops.merge_states(o_hist, lse_hist, o_chunk, lse_chunk, ctx.invalid, ctx.backends.merge)


def _attend_decode(sl, loop, q_lat, q_rope, cache, block_table, ctx, window):
    """Decode branch with history (and short chunks): one ``hla_s6_attend_decode`` call (two launches: the split
    history kernel, whose last workgroups compute the exact windows, then the epilogue that reduces the splits,
    applies B_t and merges)."""
    for kind in ('history', 'merge', 'chunk'):
        s6_ops._backend(kind, getattr(ctx.backends, kind))
    _, B, _ = sl.readers(loop)
    exact, ex_table = window
    s6_ops._dev(q_lat, q_rope, cache, block_table, exact, ex_table, B)
    for name, t in (('q_lat', q_lat), ('q_rope', q_rope), ('cache', cache), ('exact cache', exact), ('B', B)):
        s6_ops._bf16(name, t)
    T, H, w = q_lat.shape
    d = q_rope.shape[-1]
    if cache.dim() != 4 or cache.shape[1] != 1 or cache.shape[-1] != 2 * w:
        raise ValueError(f'latent cache must be [num_blocks, 1, block, {2 * w}], got {tuple(cache.shape)}')
    if exact.dim() != 4 or exact.shape[1] != H or exact.shape[-1] != 2 * d:
        raise ValueError(f'exact cache must be [num_blocks, {H}, block, {2 * d}], got {tuple(exact.shape)}')
    if B.shape != (H, w, d):
        raise ValueError(f'B must be [{H}, {w}, {d}], got {tuple(B.shape)}')
    for name, tab in (('block_table', block_table), ('exact block_table', ex_table)):
        if tab.dtype != torch.int32 or tab.stride(-1) != 1:
            raise ValueError(f'{name} must be int32 with a unit last stride')
    qsl = s6_ops._int('query_start_loc', ctx.query_start_loc, torch.int32)
    seq = s6_ops._int('seq_lens', ctx.seq_lens, torch.int32)
    R = qsl.shape[0] - 1
    if block_table.shape[0] < R or ex_table.shape[0] < R or seq.shape[0] < R:
        raise ValueError(f'per-request tables and seq_lens need {R} rows')
    dev = q_lat.device
    o_hist = torch.empty(T, H, w, dtype=torch.bfloat16, device=dev)
    lse_hist = torch.empty(H, T, dtype=torch.float32, device=dev)
    o_win = torch.empty(T, H, d, dtype=torch.bfloat16, device=dev)
    lse_win = torch.empty(H, T, dtype=torch.float32, device=dev)
    out = torch.empty(T, H, d, dtype=torch.bfloat16, device=dev)
    splits = ctx.kv_splits(w)
    ws = plan = None
    if splits > 1:
        if ctx.workspace is None:
            raise RuntimeError('history attention with num_kv_splits > 1 needs an S6Workspace')
        ws = ctx.workspace.attn_logits(T, H, splits, w, dev)
        plan = ctx.split_plan(splits, block_table.shape[1] * cache.shape[2])
    _lib.call('hla_s6_attend_decode', _lib.ptr(q_lat), q_lat.stride(0), q_lat.stride(1), w, _lib.ptr(cache),
              _lib.ptr(cache[..., w:]), cache.stride(0), cache.stride(2), cache.shape[2], cache.shape[0],
              _lib.ptr(block_table), block_table.stride(0), block_table.shape[1], _lib.ptr(ctx.token_requests),
              _lib.ptr(ctx.ctx_latent), _lib.ptr(q_rope), q_rope.stride(0), q_rope.stride(1), _lib.ptr(exact),
              _lib.ptr(exact[..., d:]), exact.stride(0), exact.stride(2), exact.stride(1), exact.shape[2],
              exact.shape[0], _lib.ptr(ex_table), ex_table.stride(0), ex_table.shape[1], _lib.ptr(qsl), _lib.ptr(seq),
              R, int(ctx.window), _lib.ptr(B), B.stride(0), B.stride(1), _lib.ptr(ctx.invalid), T, H, float(ctx.scale),
              splits, int(ctx.max_query_len), _lib.ptr(ws), 0 if ws is None else ws.numel(), _lib.ptr(plan),
              0 if plan is None else plan.numel(),
              _lib.ptr(o_hist),
              _lib.ptr(lse_hist), _lib.ptr(o_win), _lib.ptr(lse_win), _lib.ptr(out), out.stride(0), out.stride(1),
              _lib.stream(dev))
    return out


@dataclass
class WriterState:
    reg: torch.Tensor | None = None
    first: torch.Tensor | None = None


def _writer_weight(sl, loop):
    """This loop's candidate projection: the ``[2w, hidden]`` nn.Linear weight and ``w`` (``cand1`` at loop 0,
    ``cand_s[loop - 1]`` after; ``hla/latent/register.py:37-38``)."""
    if loop == 0:
        lin, width = sl.cand1, sl.rank1
    else:
        if getattr(sl, 'rank_v', sl.rank) != sl.rank:
            raise ValueError(f'S6 rows need rank_v == rank (got {sl.rank_v} and {sl.rank})')
        lin, width = sl.cand_s[loop - 1], sl.rank
    weight = lin.weight
    if weight.shape[0] != 2 * width:
        raise ValueError(f'candidate projection has {weight.shape[0]} outputs, rows are 2 x {width} wide')
    return weight, width


def _write(h, weight, width, prev, reg, slots=None, positions=None, table=None, cache=None):
    """One ``hla_s6_write_rows`` launch (projection, accumulation and, with ``cache``, the row commit)."""
    s6_ops._dev(h, weight, prev, reg, cache)
    s6_ops._bf16('h', h)
    s6_ops._bf16('candidate weight', weight)
    T, hidden = h.shape
    if weight.shape[1] != hidden:
        raise ValueError(f'candidate weight takes {weight.shape[1]} inputs, h has {hidden}')
    if prev is not None:
        s6_ops._bf16('previous register', prev)
        if tuple(prev.shape) != (T, 2 * width):
            raise ValueError(f'previous register is {tuple(prev.shape)}, expected {(T, 2 * width)}')
    geo = (None, 0, 0, 0, 0)
    if cache is not None:
        s6_ops._bf16('cache', cache)
        s6_ops._bf16('rope table', table)
        if cache.shape[-1] != 2 * width or table.shape[1] != width:
            raise ValueError(f'cache rows ({cache.shape[-1]}) / RoPE table ({table.shape[1]}) do not fit width {width}')
        geo = (cache, cache.stride(0), cache.stride(2), cache.shape[2], cache.shape[0])
        positions = s6_ops._int('positions', positions, torch.int64)
        slots = s6_ops._int('slots', slots, torch.int64)
    _lib.call('hla_s6_write_rows', _lib.ptr(h), T, hidden, h.stride(0), _lib.ptr(weight), width, weight.stride(0),
              _lib.ptr(prev), 0 if prev is None else prev.stride(0), _lib.ptr(reg), 0 if reg is None else reg.stride(0),
              _lib.ptr(slots), _lib.ptr(positions), _lib.ptr(table), 0 if table is None else table.shape[0],
              0 if table is None else table.stride(0), _lib.ptr(geo[0]), geo[1], geo[2], geo[3], geo[4],
              _lib.stream(h.device))
    return reg


def write_rows(sl, loop, h, state=None):
    """Writer accumulation on the attention input ``h[T, hidden]`` of this loop (``LatentLayer.write_step``/``write1``;
    ``hla/vllm_latent/s6_layer.py:124-132``). Loop 0 produces the loop-1 row ``first``; later loops accumulate ``reg``.

    One HIP launch: the candidate projection on MFMA with the bf16 register update in its epilogue."""
    weight, width = _writer_weight(sl, loop)
    prev = None if loop == 0 or state is None else state.reg
    reg = torch.empty(h.shape[0], 2 * width, dtype=h.dtype, device=h.device)
    _write(h, weight, width, prev, reg)
    return WriterState(None, reg) if loop == 0 else WriterState(reg, None)


def write_commit(sl, loop, h, state, ctx, cache, block_table):
    """``write_rows`` + ``committed_row`` + the slot-mapped store of ``hla/vllm_latent/ouro_latent.py:127-129`` in ONE
    launch. At loop 0 and the last loop the committed row goes straight from the projection's epilogue into
    ``cache`` (``[num_blocks, 1, block, 2w]``; K half latent-rotated, padding tokens skipped) and the returned state
    holds no row, since nothing reads it again; other loops return the accumulated register as ``write_rows`` does.
    ``block_table`` is the per-request table of ``cache``."""
    if loop != 0 and loop != sl.loops - 1:
        return write_rows(sl, loop, h, state)
    weight, width = _writer_weight(sl, loop)
    prev = None if loop == 0 or state is None else state.reg
    slots = ctx.slots(block_table, cache.shape[2])
    _write(h, weight, width, prev, None, slots, ctx.positions, ctx.tables[width], cache)
    return WriterState(None, None)


def committed_row(sl, loop, state, ctx):
    """``(key[T,w], value[T,w])`` to store after this loop: loop-1 row at loop 0, main row at the last loop, else None
    (``hla/vllm_latent/s6_layer.py:135-147``). The K half is rotated in place by the latent RoPE kernel."""
    if loop == 0:
        row, width = state.first, sl.rank1
    elif loop == sl.loops - 1:
        row, width = state.reg, sl.rank
    else:
        return None
    return s6_ops.latent_rope(row[:, :width], ctx.positions, ctx.tables[width], ctx.backends.rope), row[:, width:]


def slot_mapping(ctx, block_table, block_size):
    """Cache slot per token (``table[req, pos // block] * block + pos % block``, -1 on padding) for the row commit."""
    T = ctx.token_requests.shape[0]
    slots = torch.empty(T, dtype=torch.int64, device=block_table.device)
    pos = s6_ops._int('positions', ctx.positions, torch.int64)
    _lib.call('hla_s6_slot_mapping', _lib.ptr(block_table), block_table.stride(0), block_table.shape[1],
              _lib.ptr(ctx.token_requests),
              _lib.ptr(ctx.valid), _lib.ptr(pos), T, int(block_size), _lib.ptr(slots), _lib.stream(block_table.device))
    return slots


def store_rows(key, value, slots, cache):
    """Slot-mapped store of ``[key | value]`` rows into a ``[num_blocks, 1, block, 2w]`` latent cache (negative slots
    skipped): the ``unified_kv_cache_update`` of ``hla/vllm_latent/ouro_latent.py:127-129``."""
    s6_ops._bf16('key', key)
    s6_ops._bf16('value', value)
    s6_ops._bf16('cache', cache)
    T, w = key.shape
    if cache.shape[-1] != 2 * w:
        raise ValueError(f'cache rows are {cache.shape[-1]} wide, rows to store are 2 x {w}')
    _lib.call('hla_s6_store_rows', _lib.ptr(key), key.stride(0), _lib.ptr(value), value.stride(0), T, w,
              _lib.ptr(slots), _lib.ptr(cache), cache.stride(0), cache.stride(2), cache.shape[2], cache.shape[0],
              _lib.stream(cache.device))
