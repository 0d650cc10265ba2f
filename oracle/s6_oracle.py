"""Numpy restatement of the S6 serving-path semantics. TEST INFRASTRUCTURE ONLY (see ``oracle/__init__``).

Conventions (``hla/vllm_latent/s6_ops.py:1-10``): outputs are normalized attention outputs; ``lse`` is a
contiguous ``[H, T]`` natural-log log-sum-exp of already-scaled scores; an empty row gives ``lse = -inf``
and ``o = 0``; no NaN leaves a merge. Floating-point inputs are float32 arrays holding bf16 values
(``oracle.bf16.to_f32``); arithmetic is float32 (or float64 with ``dtype=np.float64``). ``rounding=True``
reproduces the bf16 rounding points of the reference torch path (each op output that the reference
keeps in the query dtype is rounded to bf16).
"""
from __future__ import annotations

import math

import numpy as np

from .bf16 import round_bf16

INF = np.inf


# ----------------------------------------------------------------------------------------------------------------
# Step metadata (integer, bit-exact)
# ----------------------------------------------------------------------------------------------------------------

def token_requests(query_start_loc, num_tokens):
    """Request index per token (int64, clamped) and ``valid = arange(T) < qsl[-1]``.

    Follows ``hla/vllm_latent/s6_ops.py:61-68`` (``searchsorted(qsl[1:], idx, right=True).clamp(max=R-1)``).
    """
    qsl = np.asarray(query_start_loc, dtype=np.int64)
    idx = np.arange(num_tokens, dtype=np.int64)
    req = np.searchsorted(qsl[1:], idx, side='right')
    req = np.minimum(req, qsl.shape[0] - 2).astype(np.int64)
    return req, idx < qsl[-1]


def history_lengths(seq_lens, query_start_loc):
    """``max(seq_len - query_len, 0)`` per request; follows ``hla/vllm_latent/s6_ops.py:71-73``."""
    qsl = np.asarray(query_start_loc, dtype=np.int64)
    seq = np.asarray(seq_lens, dtype=np.int64)
    return np.maximum(seq - (qsl[1:] - qsl[:-1]), 0).astype(np.int32)


def num_kv_splits(max_seq_len, num_tokens, split_max_tokens, sm_count, head_blocks=1):
    """Split-count heuristic; follows ``hla/vllm_latent/s6_ops.py:76-89``."""
    if num_tokens > split_max_tokens:
        return 1
    ideal = 1 << (max(1, max_seq_len // 512) - 1).bit_length()
    fill = -(-2 * sm_count // (num_tokens * head_blocks))
    return max(1, min(max(ideal, fill), 2 * sm_count, -(-max_seq_len // 32)))


def workspace_floats(heads, width_max, rows_x_splits):
    """fp32 workspace size; follows ``S6Workspace.__init__`` (``hla/vllm_latent/s6_ops.py:100-102``)."""
    return rows_x_splits * heads * (width_max + 1)


def step_context(query_start_loc, seq_lens, num_tokens, window=0):
    """Per-token ``(token_requests, valid, ctx, ctx_latent)``; follows ``StepContext.__init__``
    (``hla/vllm_latent/s6_layer.py:59-70``). ``query_start_loc=None`` is the profiling step
    (one request spanning every token, no history).
    """
    if query_start_loc is None:
        query_start_loc = np.array([0, num_tokens], dtype=np.int32)
        seq_lens = query_start_loc[1:]
    req, valid = token_requests(query_start_loc, num_tokens)
    history = history_lengths(seq_lens, query_start_loc)
    ctx = np.where(valid, history[req], 0).astype(np.int32)
    ctx_latent = np.maximum(ctx - window, 0).astype(np.int32) if window else ctx.copy()
    return req, valid, ctx, ctx_latent


def token_block_table(table, token_requests_):
    """Per-token gather of a per-request block table; follows ``StepContext.block_table``
    (``hla/vllm_latent/s6_layer.py:75-80``)."""
    return np.asarray(table)[np.asarray(token_requests_)]


def slot_mapping(table, token_requests_, valid, positions, block):
    """Cache slot per token: ``table[req, pos // block] * block + pos % block``, -1 for padding tokens.

    Closed form of ``hla/tests/test_s6_serving.py:54``; negative slots are the padding convention of
    ``hla/vllm_latent/ouro_latent.py:8-9``.
    """
    table = np.asarray(table, dtype=np.int64)
    pos = np.asarray(positions, dtype=np.int64)
    req = np.asarray(token_requests_, dtype=np.int64)
    slots = table[req, pos // block] * block + pos % block
    return np.where(valid, slots, -1).astype(np.int64)


def store_rows(cache_rows, slots, key, value):
    """Slot-mapped store of ``[key | value]`` rows into a flat ``[num_slots, 2w]`` cache view, skipping
    negative slots (``unified_kv_cache_update`` at ``hla/vllm_latent/ouro_latent.py:127-129``)."""
    out = np.array(cache_rows, copy=True)
    for t, s in enumerate(np.asarray(slots)):
        if s >= 0:
            out[s] = np.concatenate((key[t], value[t]))
    return out


# ----------------------------------------------------------------------------------------------------------------
# Latent RoPE and absorption GEMMs
# ----------------------------------------------------------------------------------------------------------------

def latent_inv_freq(head_dim, theta):
    """Teacher RoPE frequencies; follows ``hla/vllm_latent/s6_layer.py:16-18`` (float32)."""
    exps = np.arange(0, head_dim, 2, dtype=np.int64).astype(np.float32) / np.float32(head_dim)
    return (np.float32(1.0) / (np.float32(theta) ** exps)).astype(np.float32)


def latent_rope_table(max_position, inv_freq, width):
    """``[max_position, width] = [cos | sin]`` with frequencies round-robin over the ``width/2`` pairs;
    follows ``hla/vllm_latent/s6_layer.py:21-29`` (float32 angle; cast by the caller)."""
    idx = np.arange(width // 2) % inv_freq.shape[0]
    angle = np.arange(max_position, dtype=np.float32)[:, None] * inv_freq[idx][None, :]
    return np.concatenate((np.cos(angle), np.sin(angle)), -1).astype(np.float32)


def rotate_half(x):
    """``cat(-x2, x1)``; follows ``hla/latent/register.py:14-16``."""
    a, b = np.split(x, 2, axis=-1)
    return np.concatenate((-b, a), -1)


def latent_rope(x, positions, table, rounding=True):
    """Neox rotation ``x*cos + rotate_half(x)*sin`` of ``x[T, ..., w]`` by ``table[positions]``.

    Follows the torch branch of ``hla/vllm_latent/s6_ops.py:32-36``; with ``rounding`` each of the three
    elementwise ops is rounded to bf16, as torch does for bf16 tensors.
    """
    w = table.shape[1]
    rows = table[np.asarray(positions)]
    cos = np.concatenate((rows[:, : w // 2], rows[:, : w // 2]), -1)
    sin = np.concatenate((rows[:, w // 2:], rows[:, w // 2:]), -1)
    shape = (x.shape[0],) + (1,) * (x.ndim - 2) + (w,)
    cos, sin = cos.reshape(shape), sin.reshape(shape)
    r = round_bf16 if rounding else (lambda v: v)
    return r(r(x * cos) + r(rotate_half(x) * sin))


def absorb(x, weight, rounding=True, dtype=np.float32):
    """``einsum('thd,hdr->thr', x, weight)`` with fp32 accumulation; follows the ``A_t`` einsum of
    ``hla/vllm_latent/s6_layer.py:37`` and the ``B_t`` einsum of ``hla/vllm_latent/s6_layer.py:114``.
    ``rounding`` rounds the output to bf16 (the einsum output dtype)."""
    out = np.einsum('thd,hdr->thr', x.astype(dtype), weight.astype(dtype))
    return round_bf16(out.astype(np.float32)) if rounding else out


def latent_query(q_pre_rope, A, positions, table, rounding=True):
    """Absorbed, latent-rotated query; follows ``hla/vllm_latent/s6_layer.py:32-40``."""
    return latent_rope(absorb(q_pre_rope, A, rounding), positions, table, rounding)


# ----------------------------------------------------------------------------------------------------------------
# Writer (candidate projection, register accumulation, committed row)
# ----------------------------------------------------------------------------------------------------------------

def write_step(h, weight, prev=None, dtype=np.float64):
    """One loop of the writer: ``update = h @ weight.T`` rounded to bf16 (an nn.Linear in bf16), then
    ``previous + update`` rounded to bf16. Follows ``LatentLayer.write_step`` / ``write1``
    (``hla/latent/register.py:45-49,60-61``) as ``write_rows`` calls them (``hla/vllm_latent/s6_layer.py:124-132``);
    ``weight`` is the ``[2w, hidden]`` nn.Linear weight."""
    update = round_bf16((h.astype(dtype) @ weight.astype(dtype).T).astype(np.float32))
    return update if prev is None else round_bf16(prev + update)


def write_trajectory(h_loops, weights):
    """The register after every loop (loop 0 adds nothing: ``write_step`` returns zeros there); follows
    ``LatentLayer.write`` (``hla/latent/register.py:51-58``). ``weights[l - 1]`` is ``cand_s[l - 1].weight``."""
    reg, rows = None, []
    for loop, h in enumerate(h_loops):
        if loop == 0:
            rows.append(np.zeros((h.shape[0], weights[0].shape[0]), np.float32))
            continue
        reg = write_step(h, weights[loop - 1], reg)
        rows.append(reg)
    return np.stack(rows)


def committed_row(row, width, positions, table):
    """``(RoPE_lat(row[:, :w]), row[:, w:])``: the key half rotated by the width's table, the value half as is;
    follows ``hla/vllm_latent/s6_layer.py:135-147`` (rounding as ``latent_rope``)."""
    return latent_rope(row[:, :width], positions, table), row[:, width:]


# ----------------------------------------------------------------------------------------------------------------
# Attention partials
# ----------------------------------------------------------------------------------------------------------------

def _softmax_partial(scores, values, dtype):
    """Normalized ``softmax(scores) @ values`` and natural-log lse of one query row set; all -inf -> (0, -inf)."""
    if scores.shape[-1] == 0 or not np.isfinite(scores).any():
        return np.zeros(scores.shape[:-1] + (values.shape[-1],), dtype), np.full(scores.shape[:-1], -INF, dtype)
    peak = scores.max(-1, keepdims=True)
    peak = np.where(np.isfinite(peak), peak, 0)
    probs = np.exp(scores - peak)
    den = probs.sum(-1, keepdims=True)
    out = (probs @ values) / np.where(den > 0, den, 1)
    lse = np.where(den[..., 0] > 0, np.log(np.where(den[..., 0] > 0, den[..., 0], 1)) + peak[..., 0], -INF)
    out = np.where(den > 0, out, 0)
    return out.astype(dtype), lse.astype(dtype)


def history_attention(q, k_cache, v_cache, block_table, ctx, scale, rounding=False, dtype=np.float32):
    """Fully visible attention of ``q[T, H, Lk]`` over the first ``ctx[t]`` paged rows.

    ``k_cache[nb, kvH, block, Lk]`` / ``v_cache[nb, kvH, block, Lv]`` (MQA when ``kvH == 1``), ``block_table[T, *]``
    per token. Only table columns ``< ceil(ctx / block)`` are read. Returns ``(o[T, H, Lv], lse[H, T])``; empty rows
    give ``o = 0``, ``lse = -inf``. Follows ``_history_reference`` (``hla/vllm_latent/s6_ops.py:204-222``);
    ``rounding`` rounds ``o`` to bf16 (the kernel's ``q.dtype`` output).
    """
    T, H, Lk = q.shape
    kvh, block, Lv = k_cache.shape[1], k_cache.shape[2], v_cache.shape[-1]
    group = H // kvh
    o = np.zeros((T, H, Lv), dtype)
    lse = np.full((H, T), -INF, dtype)
    for t in range(T):
        n = int(ctx[t])
        if n == 0:
            continue
        pages = np.asarray(block_table[t][: (n + block - 1) // block], dtype=np.int64)
        for g in range(kvh):
            rows_k = k_cache[pages, g].reshape(-1, Lk)[:n].astype(dtype)
            rows_v = v_cache[pages, g].reshape(-1, Lv)[:n].astype(dtype)
            qg = q[t, g * group:(g + 1) * group].astype(dtype)
            scores = (qg @ rows_k.T) * dtype(scale)
            out, l = _softmax_partial(scores, rows_v, dtype)
            o[t, g * group:(g + 1) * group] = out
            lse[g * group:(g + 1) * group, t] = l
    return (round_bf16(o.astype(np.float32)) if rounding else o), lse


def _exact_rows(cache_k, cache_v, table_row, positions, head):
    block = cache_k.shape[2]
    pages = np.asarray(table_row, dtype=np.int64)[positions // block]
    return cache_k[pages, head, positions % block], cache_v[pages, head, positions % block]


def window_decode(q, cache_k, cache_v, block_table, query_start_loc, seq_lens, window, scale, invalid,
                  rounding=False, dtype=np.float32):
    """Exact causal sliding-window attention over the request's exact paged cache (current token included).

    Query ``i`` of a request with ``Lq`` queries and ``seq_len`` keys sits at position ``p = seq_len - Lq + i`` and
    reads keys ``[max(0, p - window), p]``; for decode (``Lq = 1``) that is ``[seq_len - 1 - window, seq_len - 1]``.
    ``cache_k/cache_v`` are ``[nb, H, block, d]`` (the TRITON_ATTN logical layout split into its K and V halves),
    ``block_table`` is per request. Follows ``window_attention_fa`` (``hla/vllm_latent/s6_ops.py:317-331``:
    causal, ``window_size=(window, 0)``, bottom-right aligned); ``invalid`` rows give ``o = 0, lse = -inf``.
    """
    T, H, d = q.shape
    req, _ = token_requests(query_start_loc, T)
    qsl = np.asarray(query_start_loc, dtype=np.int64)
    o = np.zeros((T, H, d), dtype)
    lse = np.full((H, T), -INF, dtype)
    for t in range(T):
        if invalid[t]:
            continue
        r = int(req[t])
        lq = int(qsl[r + 1] - qsl[r])
        p = int(seq_lens[r]) - lq + (t - int(qsl[r]))
        if p < 0:
            continue
        keys = np.arange(max(0, p - window), p + 1)
        for h in range(H):
            kk, vv = _exact_rows(cache_k, cache_v, block_table[r], keys, h)
            scores = (kk.astype(dtype) @ q[t, h].astype(dtype)) * dtype(scale)
            out, l = _softmax_partial(scores[None], vv.astype(dtype), dtype)
            o[t, h], lse[h, t] = out[0], l[0]
    return (round_bf16(o.astype(np.float32)) if rounding else o), lse


def window_history(q, cache_k, cache_v, token_block_table, ctx, window, scale, rounding=False, dtype=np.float32):
    """Exact attention over history rows ``[ctx[t] - window, ctx[t])`` (no self key) with a per-token table.

    Follows ``window_attention`` (``hla/vllm_latent/s6_ops.py:290-314``) and ``window_history_fa`` (``334-350``);
    rows without window history give ``o = 0, lse = -inf``.
    """
    T, H, d = q.shape
    o = np.zeros((T, H, d), dtype)
    lse = np.full((H, T), -INF, dtype)
    for t in range(T):
        c = int(ctx[t])
        keys = np.arange(max(0, c - window), c)
        if keys.size == 0:
            continue
        for h in range(H):
            kk, vv = _exact_rows(cache_k, cache_v, token_block_table[t], keys, h)
            scores = (kk.astype(dtype) @ q[t, h].astype(dtype)) * dtype(scale)
            out, l = _softmax_partial(scores[None], vv.astype(dtype), dtype)
            o[t, h], lse[h, t] = out[0], l[0]
    return (round_bf16(o.astype(np.float32)) if rounding else o), lse


def chunk_attention(q, k, v, query_start_loc, invalid, scale, rounding=False, dtype=np.float32):
    """Causal attention inside each request's current chunk; follows ``_chunk_reference``
    (``hla/vllm_latent/s6_ops.py:251-259``). Invalid rows give ``o = 0, lse = -inf``."""
    T, H, d = q.shape
    req, _ = token_requests(query_start_loc, T)
    o = np.zeros((T, H, d), dtype)
    lse = np.full((H, T), -INF, dtype)
    for i in range(T):
        if invalid[i]:
            continue
        keys = np.nonzero((req == req[i]) & (np.arange(T) <= i))[0]
        for h in range(H):
            scores = (k[keys, h].astype(dtype) @ q[i, h].astype(dtype)) * dtype(scale)
            out, l = _softmax_partial(scores[None], v[keys, h].astype(dtype), dtype)
            o[i, h], lse[h, i] = out[0], l[0]
    return (round_bf16(o.astype(np.float32)) if rounding else o), lse


# ----------------------------------------------------------------------------------------------------------------
# Merges
# ----------------------------------------------------------------------------------------------------------------

def merge_states(o_hist, lse_hist, o_chunk, lse_chunk, invalid, rounding=False):
    """LSE merge of two partial softmaxes; ``+inf`` lse counts as empty, both empty -> 0, ``invalid`` rows -> 0.

    Follows ``merge_states`` / ``_merge_reference`` (``hla/vllm_latent/s6_ops.py:262-284``).
    """
    lh = np.where(lse_hist == INF, -INF, lse_hist).astype(np.float32)
    lc = np.where(lse_chunk == INF, -INF, lse_chunk).astype(np.float32)
    peak = np.maximum(lh, lc)
    peak = np.where(np.isinf(peak), 0, peak)
    with np.errstate(invalid='ignore', over='ignore'):
        wh, wc = np.exp(lh - peak), np.exp(lc - peak)
    total = wh + wc
    safe = np.where(total > 0, total, 1)
    wh, wc = np.where(total > 0, wh / safe, 0), np.where(total > 0, wc / safe, 0)
    out = o_hist.astype(np.float32) * wh.T[..., None] + o_chunk.astype(np.float32) * wc.T[..., None]
    out = round_bf16(out) if rounding else out
    out[np.asarray(invalid, dtype=bool)] = 0
    return out


def merge_lse(o1, lse1, o2, lse2, rounding=False):
    """LSE merge returning the merged lse too; follows ``merge_lse`` (``hla/vllm_latent/s6_ops.py:353-361``)."""
    peak = np.maximum(lse1, lse2)
    peak = np.where(np.isinf(peak), 0, peak)
    with np.errstate(invalid='ignore', over='ignore'):
        w1, w2 = np.exp(lse1 - peak), np.exp(lse2 - peak)
    total = w1 + w2
    safe = np.where(total > 0, total, 1)
    w1, w2 = (np.where(total > 0, w / safe, 0).T[..., None] for w in (w1, w2))
    out = np.nan_to_num(o1.astype(np.float32)) * w1 + np.nan_to_num(o2.astype(np.float32)) * w2
    with np.errstate(divide='ignore'):
        merged = peak + np.log(total)
    return (round_bf16(out) if rounding else out), merged.astype(np.float32)


# ----------------------------------------------------------------------------------------------------------------
# Composite: one layer x loop of the decode branch of ``s6_layer.attend``
# ----------------------------------------------------------------------------------------------------------------

def attend_decode(q_lat, q_rope, B, lat_k, lat_v, token_table, ctx_latent, ex_k, ex_v, request_table,
                  query_start_loc, seq_lens, window, scale, invalid, rounding=True, dtype=np.float32):
    """Decode branch of ``attend`` (``hla/vllm_latent/s6_layer.py:97-100,110-115``): exact window plus the current
    token, paged latent history, ``B_t`` projection of the history output, LSE merge. Returns ``[T, H, d]``."""
    o_c, lse_c = window_decode(q_rope, ex_k, ex_v, request_table, query_start_loc, seq_lens, window, scale, invalid,
                               rounding, dtype)
    o_h, lse_h = history_attention(q_lat, lat_k, lat_v, token_table, ctx_latent, scale, rounding, dtype)
    o_h = absorb(o_h, B, rounding, dtype)
    return merge_states(o_h, lse_h, o_c, lse_c, invalid, rounding)


def attend_chunk(q_lat, q_rope, k_rope, v, B, lat_k, lat_v, token_table, ctx, ctx_latent, query_start_loc, window,
                 scale, invalid, ex_k=None, ex_v=None, rounding=True, dtype=np.float32):
    """Prefill / mixed branch of ``attend`` (``hla/vllm_latent/s6_layer.py:101-115``): causal current chunk, optional
    exact window over history rows ``[ctx - W, ctx)`` merged by ``merge_lse``, then history + ``B_t`` + merge."""
    o_c, lse_c = chunk_attention(q_rope, k_rope, v, query_start_loc, invalid, scale, rounding, dtype)
    if ex_k is not None:
        o_w, lse_w = window_history(q_rope, ex_k, ex_v, token_table['exact'], ctx, window, scale, rounding, dtype)
        o_c, lse_c = merge_lse(o_c, lse_c, o_w, lse_w, rounding)
    o_h, lse_h = history_attention(q_lat, lat_k, lat_v, token_table['latent'], ctx_latent, scale, rounding, dtype)
    o_h = absorb(o_h, B, rounding, dtype)
    return merge_states(o_h, lse_h, o_c, lse_c, invalid, rounding)


# ----------------------------------------------------------------------------------------------------------------
# Multi-query causal history attention with backward (K-hop replay / chunked prefill on contiguous rows)
# ----------------------------------------------------------------------------------------------------------------

def _masked_scores(q, k, mask, scale, dtype):
    s = np.einsum('bihr,bjr->bihj', q.astype(dtype), k.astype(dtype)) * dtype(scale)
    vis = np.asarray(mask, bool)[:, :, None, :]
    return np.where(vis, s, -np.inf), vis


def causal_history(q, k, v, mask, scale, dtype=np.float64):
    """``z [B, Lq, H, Rv]`` and ``lse [B, H, Lq]`` of every query row (i, h) over the keys ``mask[b, i, :]``
    shows; rows without a visible key give ``z = 0``, ``lse = -inf``. Follows ``_forward``
    (``hla/latent/history_gemm.py:159-177``): peak-shifted exponentials, ``lse = log(den) + peak``,
    ``z = (prob @ v) / den``."""
    s, vis = _masked_scores(q, k, mask, scale, dtype)
    peak = s.max(-1, keepdims=True)
    peak = np.where(np.isfinite(peak), peak, 0.0)
    prob = np.where(vis, np.exp(s - peak), 0.0)
    den = prob.sum(-1, keepdims=True)
    with np.errstate(divide='ignore'):
        lse = (np.log(den) + peak)[..., 0]
    z = np.einsum('bihj,bjr->bihr', prob, v.astype(dtype)) / np.where(den == 0, 1.0, den)
    return z, lse.transpose(0, 2, 1)


def causal_history_backward(q, k, v, mask, scale, lse, dz, dlse=None, z=None, dtype=np.float64):
    """``(dq, dk, dv)`` of ``causal_history`` for output cotangents ``dz [B, Lq, H, Rv]`` and
    ``dlse [B, H, Lq]``. Follows ``_backward`` (``hla/latent/history_gemm.py:180-220``):
    ``P = exp(s - lse)`` (0 on rows without history), ``dv = P^T dz``, ``dP = dz v^T``,
    ``delta = sum(dz * z)`` when ``z`` is given, else ``sum(P * dP)``,
    ``dS = P (dP - delta + dlse) scale``, ``dq = dS k``, ``dk = dS^T q``."""
    s, vis = _masked_scores(q, k, mask, scale, dtype)
    lse_t = np.asarray(lse, dtype).transpose(0, 2, 1)[..., None]            # [B, Lq, H, 1]
    empty = ~np.isfinite(lse_t)
    prob = np.where(vis & ~empty, np.exp(s - np.where(empty, 0.0, lse_t)), 0.0)
    dz = np.asarray(dz, dtype)
    dv = np.einsum('bihj,bihr->bjr', prob, dz)
    dp = np.einsum('bihr,bjr->bihj', dz, v.astype(dtype))
    if z is not None:
        delta = (dz * np.asarray(z, dtype)).sum(-1, keepdims=True)
    else:
        delta = (dp * prob).sum(-1, keepdims=True)
    ds = dp - delta
    if dlse is not None:
        ds = ds + np.where(empty, 0.0, np.asarray(dlse, dtype).transpose(0, 2, 1)[..., None])
    ds = ds * prob * dtype(scale)
    dq = np.einsum('bihj,bjr->bihr', ds, k.astype(dtype))
    dk = np.einsum('bihj,bihr->bjr', ds, q.astype(dtype))
    return dq, dk, dv


def single_history(q, k, v, mask, scale, dtype=np.float64):
    """Single-query form (``reference`` of ``hla/latent/fused_history.py:11-20``): q ``[B, H, R]`` against k, v
    ``[B, N, R]`` with ``mask [B, N]``; returns ``z [B, H, R]`` and ``lse [B, H]`` (``z = 0``, ``lse = -inf`` on a
    row with no visible key). The multi-query form with one query per batch row."""
    z, lse = causal_history(np.asarray(q)[:, None], k, v, np.asarray(mask, bool)[:, None], scale, dtype)
    return z[:, 0], lse[:, :, 0]


def single_history_backward(q, k, v, mask, scale, lse, dz, dlse=None, dtype=np.float64):
    """``(dq [B, H, R], dk, dv [B, N, R])`` of ``single_history`` (the Triton ``_backward_q`` / ``_backward_kv`` of
    ``hla/latent/history_kernels.py:36-81``: ``dS = P (v.dz - delta + dlse)``, ``dq = scale dS k``)."""
    dq, dk, dv = causal_history_backward(np.asarray(q)[:, None], k, v, np.asarray(mask, bool)[:, None], scale,
                                         np.asarray(lse)[:, :, None], np.asarray(dz)[:, None],
                                         None if dlse is None else np.asarray(dlse)[:, :, None], dtype=dtype)
    return dq[:, 0], dk, dv


def rel_l2(a, b):
    """Relative L2 error ``||a - b|| / ||b||`` in float64."""
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    den = math.sqrt(float((b * b).sum()))
    return math.sqrt(float(((a - b) ** 2).sum())) / (den if den > 0 else 1.0)


# ----------------------------------------------------------------------------------------------------------------
# HF rolling engine: one softmax over latent history blocks and the exact current chunk, with its gradient
# ----------------------------------------------------------------------------------------------------------------

def hf_rope(x, cos, sin):
    """``x cos + rotate_half(x) sin`` with cos / sin ``[B, n, w]`` broadcast over the heads of ``x [B, H, n, w]``;
    follows ``apply_rope`` (``hla/latent/register.py:19-20``)."""
    return x * cos[:, None] + rotate_half(x) * sin[:, None]


def hf_rope_backward(dy, cos, sin):
    """Cotangent of ``x`` for ``y = hf_rope(x, cos, sin)``: ``dy cos + R^T (dy sin)`` where ``R = rotate_half``
    (``R [a, b] = [-b, a]``, so ``R^T [u, w] = [w, -u]``)."""
    u = dy * sin[:, None]
    a, b = np.split(u, 2, axis=-1)
    return dy * cos[:, None] + np.concatenate((b, -a), -1)


def rope_latent_tables(cos, sin, width):
    """The teacher's cos / sin ``[..., d]`` re-indexed for a latent of ``width`` columns: pair ``i`` takes frequency
    ``i % (d / 2)``, both halves alike; follows ``rope_latent`` (``hla/latent/register.py:23-25``)."""
    idx = np.arange(width // 2) % (cos.shape[-1] // 2)
    return (np.concatenate((cos[..., idx], cos[..., idx]), -1), np.concatenate((sin[..., idx], sin[..., idx]), -1))


def _mixed_parts(q, k, v, cos, sin, valid, hist_k, hist_v, masks, A, scale, dtype):
    f = lambda x: np.asarray(x, dtype)
    q, k, v, cos, sin = f(q), f(k), f(v), f(cos), f(sin)
    n = q.shape[2]
    qr, kr = hf_rope(q, cos, sin), hf_rope(k, cos, sin)
    valid = np.asarray(valid, bool)
    visible = (valid[:, None, None, :] & np.tril(np.ones((n, n), bool))) | ~valid[:, None, :, None]
    scores = []
    qc = None
    if hist_k:
        r = hist_k[0].shape[-1]
        c_r, s_r = rope_latent_tables(cos, sin, r)
        qc = hf_rope(np.einsum('bhid,hdr->bhir', q, f(A)), c_r, s_r)
        for ck, m in zip(hist_k, masks):
            s = np.einsum('bhir,bjr->bhij', qc, f(ck)) * dtype(scale)
            scores.append(np.where(np.asarray(m, bool)[:, None, None, :], s, -np.inf))
    scores.append(np.where(visible, np.einsum('bhid,bhjd->bhij', qr, kr) * dtype(scale), -np.inf))
    s = np.concatenate(scores, -1)
    peak = s.max(-1, keepdims=True)
    p = np.exp(s - peak)
    p = p / p.sum(-1, keepdims=True)
    return qr, kr, qc, p


def mixed_attention(q, k, v, cos, sin, valid, hist_k, hist_v, masks, A, B, scale, dtype=np.float64):
    """One softmax over ``[latent scores of every history block || causal exact scores of the chunk]``; follows
    ``mixed_attention`` (``hla/latent/batched_engine.py:154-182``) without its bf16 rounding points.

    q, k, v ``[B, H, n, d]`` (pre-RoPE q and k), cos / sin ``[B, n, d]``, valid ``[B, n]``; ``hist_k`` / ``hist_v``
    the history blocks' latent K / V fields ``[B, N_k, r]`` (``LatentLayer.fields``) with ``masks`` ``[B, N_k]``;
    ``A [H, d, r]`` / ``B [H, r, d]`` the loop's readers. Valid queries see the chunk's valid keys up to their own
    position and the visible rows of every block; an invalid query sees every key of the chunk. Returns
    ``[B, H, n, d]``: ``P_chunk v + (sum_k P_k cv_k) B``."""
    _, _, _, p = _mixed_parts(q, k, v, cos, sin, valid, hist_k, hist_v, masks, A, scale, dtype)
    n = q.shape[2]
    out = p[..., -n:] @ np.asarray(v, dtype)
    if hist_k:
        z, off = 0, 0
        for cv in hist_v:
            w = cv.shape[1]
            z = z + np.einsum('bhij,bjr->bhir', p[..., off:off + w], np.asarray(cv, dtype))
            off += w
        out = out + np.einsum('bhir,hrd->bhid', z, np.asarray(B, dtype))
    return out


def mixed_attention_backward(q, k, v, cos, sin, valid, hist_k, hist_v, masks, A, B, scale, dout, dtype=np.float64):
    """Gradients of ``sum(mixed_attention(...) * dout)`` with respect to ``q, k, v``, every block's ``hist_k`` /
    ``hist_v`` and the readers ``A``, ``B``: a dict ``{q, k, v, hist_k: [...], hist_v: [...], A, B}`` (``A`` / ``B``
    None without history). Softmax backward over the concatenated scores (``dS = P (dP - sum(P dP))``), then the
    chain through the products, the latent query absorption and both RoPEs."""
    f = lambda x: np.asarray(x, dtype)
    qr, kr, qc, p = _mixed_parts(q, k, v, cos, sin, valid, hist_k, hist_v, masks, A, scale, dtype)
    g = f(dout)
    n = q.shape[2]
    widths = [ck.shape[1] for ck in hist_k]
    offs = np.cumsum([0] + widths)
    p_cur = p[..., -n:]
    dp_cur = np.einsum('bhid,bhjd->bhij', g, f(v))
    res = {'v': np.einsum('bhij,bhid->bhjd', p_cur, g), 'hist_k': [], 'hist_v': [], 'A': None, 'B': None}
    dps = []
    if hist_k:
        z = sum(np.einsum('bhij,bjr->bhir', p[..., offs[i]:offs[i + 1]], f(cv)) for i, cv in enumerate(hist_v))
        dz = np.einsum('bhid,hrd->bhir', g, f(B))
        res['B'] = np.einsum('bhir,bhid->hrd', z, g)
        for i, cv in enumerate(hist_v):
            pk = p[..., offs[i]:offs[i + 1]]
            dps.append(np.einsum('bhir,bjr->bhij', dz, f(cv)))
            res['hist_v'].append(np.einsum('bhij,bhir->bjr', pk, dz))
    dp = np.concatenate(dps + [dp_cur], -1)
    ds = p * (dp - (p * dp).sum(-1, keepdims=True)) * dtype(scale)
    ds_cur = ds[..., -n:]
    dqr = np.einsum('bhij,bhjd->bhid', ds_cur, kr)
    res['k'] = hf_rope_backward(np.einsum('bhij,bhid->bhjd', ds_cur, qr), f(cos), f(sin))
    dq = hf_rope_backward(dqr, f(cos), f(sin))
    if hist_k:
        r = hist_k[0].shape[-1]
        c_r, s_r = rope_latent_tables(f(cos), f(sin), r)
        dqc = 0
        for i, ck in enumerate(hist_k):
            dsk = ds[..., offs[i]:offs[i + 1]]
            dqc = dqc + np.einsum('bhij,bjr->bhir', dsk, f(ck))
            res['hist_k'].append(np.einsum('bhij,bhir->bjr', dsk, qc))
        dpre = hf_rope_backward(dqc, c_r, s_r)
        dq = dq + np.einsum('bhir,hdr->bhid', dpre, f(A))
        res['A'] = np.einsum('bhid,bhir->hdr', f(q), dpre)
    res['q'] = dq
    return res
