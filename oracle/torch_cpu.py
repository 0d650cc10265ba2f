"""Vectorized torch-on-CPU restatement of the S6 attention path: the CPU baseline. TEST INFRASTRUCTURE ONLY.

The same semantics as ``oracle.s6_oracle.attend_decode`` / ``attend_chunk`` (and so as the reference's torch path,
``hla/vllm_latent/s6_ops.py:204-222,251-259,262-284,290-331`` composed as ``hla/vllm_latent/s6_layer.py:87-115``),
written the way the reference's own CPU oracles are written: whole-row torch GEMMs in float32 from bf16 inputs on
the host's cores (``torch.set_num_threads``), one Python iteration per token (decode) or per request (chunked
prefill) instead of the numpy oracle's per-(token, head) loops. ``bench.py`` times it as the CPU baseline of each
benchmark configuration; ``tests/test_oracle_torch_cpu.py`` pins it to the numpy oracle. Nothing in the product
imports it.

Tensors are CPU tensors: latent caches ``[num_blocks, 1, block, 2w]`` bf16 (K = ``[:w]``, V = ``[w:]``), exact caches
``[num_blocks, H, block, 2d]`` bf16 (K = ``[:d]``), int tables. Outputs are bf16 ``[T, H, d]``; rows of ``invalid``
tokens are 0. Rounding points follow the reference: the history output and the ``B_t`` product are bf16, the
window / chunk output is bf16, the merge is float32 then bf16.
"""
from __future__ import annotations

import torch

NEG_INF = float('-inf')


def latent_query(q_pre_rope, A, table_rows):
    """``RoPE_lat(einsum('thd,hdr->thr', q, A))`` with ``table_rows = table[positions]`` (``[T, w]`` = ``[cos |
    sin]`` halves): the A_t product rounded to bf16, then the neox rotation with each elementwise op rounded to
    bf16, as torch evaluates it on bf16 tensors."""
    x = torch.einsum('thd,hdr->thr', q_pre_rope.float(), A.float()).to(torch.bfloat16)
    w = x.shape[-1]
    cos = torch.cat((table_rows[:, : w // 2], table_rows[:, : w // 2]), -1)[:, None].to(torch.bfloat16)
    sin = torch.cat((table_rows[:, w // 2:], table_rows[:, w // 2:]), -1)[:, None].to(torch.bfloat16)
    rot = torch.cat((-x[..., w // 2:], x[..., : w // 2]), -1)
    return x * cos + rot * sin


def _softmax_rows(s):
    """(probabilities, lse) of the last dimension of float32 scores, rows without a finite score -> (0, -inf)."""
    lse = torch.logsumexp(s, -1)
    ok = torch.isfinite(lse)
    p = torch.exp(s - torch.where(ok, lse, torch.zeros_like(lse))[..., None])
    p = torch.where(ok[..., None], p, torch.zeros_like(p))
    return p, torch.where(ok, lse, torch.full_like(lse, NEG_INF))


def _history(q, rows, w, scale):
    """o [M, w] (float32) and lse [M] of query rows q [M, w] over latent rows [n, 2w]."""
    rows = rows.float()
    p, lse = _softmax_rows((q.float() @ rows[:, :w].T) * scale)
    return p @ rows[:, w:], lse


def _latent_rows(cache, table_row, n):
    block = cache.shape[2]
    pages = table_row[: -(-n // block)].long()
    return cache[pages, 0].reshape(-1, cache.shape[-1])[:n]


def _merge(o_h, lse_h, o_c, lse_c, invalid):
    """LSE merge of two partials ``[T, H, d]`` / ``[T, H]`` (float32); empty sides weigh 0; invalid rows 0."""
    peak = torch.maximum(lse_h, lse_c)
    peak = torch.where(torch.isfinite(peak), peak, torch.zeros_like(peak))
    wh, wc = torch.exp(lse_h - peak), torch.exp(lse_c - peak)
    total = wh + wc
    safe = torch.where(total > 0, total, torch.ones_like(total))
    out = (o_h * (wh / safe)[..., None] + o_c * (wc / safe)[..., None]).to(torch.bfloat16)
    out[invalid] = 0
    return out


def _absorb(o_hist, B):
    """``einsum('thr,hrd->thd')`` of the bf16-rounded history output with B_t, rounded to bf16."""
    o = o_hist.to(torch.bfloat16).float()
    return torch.einsum('thr,hrd->thd', o, B.float()).to(torch.bfloat16).float()


def attend_decode(q_lat, q_rope, B, lat_cache, lat_table, ctx_latent, ex_cache, ex_table, token_requests, seq_lens,
                  window, scale, invalid):
    """Decode branch of ``attend``: the paged latent history of each token (its first ``ctx_latent[t]`` rows through
    its row of ``lat_table``), ``B_t``, the exact window ``[seq - 1 - W, seq - 1]`` of its request (``ex_table`` per
    request), LSE merge."""
    T, H, w = q_lat.shape
    d = q_rope.shape[-1]
    o_h = torch.zeros(T, H, w)
    lse_h = torch.full((T, H), NEG_INF)
    for t in range(T):
        n = int(ctx_latent[t])
        if n > 0 and not invalid[t]:
            o_h[t], lse_h[t] = _history(q_lat[t], _latent_rows(lat_cache, lat_table[t], n), w, scale)
    o_h = _absorb(o_h, B)
    # exact window, all tokens at once: keys p - W .. p of the token's request
    req = token_requests.long()
    p = seq_lens.long()[req] - 1
    keys = p[:, None] - window + torch.arange(window + 1)[None]                      # [T, W + 1]
    ok = (keys >= 0) & ~invalid[:, None]
    kc = keys.clamp(min=0)
    block = ex_cache.shape[2]
    pages = ex_table.long()[req[:, None], kc // block]
    rows = ex_cache[pages, :, kc % block].float()                                    # [T, W + 1, H, 2d]
    s = torch.einsum('thd,tjhd->thj', q_rope.float(), rows[..., :d]) * scale
    s = s.masked_fill(~ok[:, None, :], NEG_INF)
    pw, lse_c = _softmax_rows(s)
    o_c = torch.einsum('thj,tjhd->thd', pw, rows[..., d:]).to(torch.bfloat16).float()
    return _merge(o_h, lse_h, o_c, lse_c, invalid.bool())


def attend_chunk(q_lat, q_rope, k_rope, v, B, lat_cache, lat_table, query_start_loc, ctx, ctx_latent, ex_cache,
                 ex_table, window, scale, invalid):
    """Prefill branch of ``attend`` for requests whose tokens share a history: per request, one GEMM of all its
    tokens' latent queries against its ``ctx_latent`` latent rows, the exact part as the reference computes it (the
    causal chunk from ``k_rope`` / ``v`` and the window history rows ``[ctx - W, ctx)`` of the exact cache, each
    rounded to bf16, merged by LSE), ``B_t``, LSE merge. ``lat_table`` / ``ex_table`` are per request; ``ctx`` /
    ``ctx_latent`` per request."""
    T, H, w = q_lat.shape
    d = q_rope.shape[-1]
    qsl = [int(x) for x in query_start_loc]
    o_h = torch.zeros(T, H, w)
    lse_h = torch.full((T, H), NEG_INF)
    o_c = torch.zeros(T, H, d)
    lse_c = torch.full((T, H), NEG_INF)
    block = ex_cache.shape[2]
    for r in range(len(qsl) - 1):
        a, b = qsl[r], qsl[r + 1]
        if a == b:
            continue
        n, c = int(ctx_latent[r]), int(ctx[r])
        if n > 0:
            oh, lh = _history(q_lat[a:b].reshape(-1, w), _latent_rows(lat_cache, lat_table[r], n), w, scale)
            o_h[a:b], lse_h[a:b] = oh.view(b - a, H, w), lh.view(b - a, H)
        q = q_rope[a:b].float()
        # causal chunk over the request's own k / v (bf16 output, as the varlen attention returns it)
        s = torch.einsum('ihd,jhd->hij', q, k_rope[a:b].float()) * scale                # [H, q, q]
        s = s.masked_fill(torch.ones(b - a, b - a, dtype=torch.bool).triu(1), NEG_INF)
        p, lse1 = _softmax_rows(s)
        o1 = torch.einsum('hij,jhd->ihd', p, v[a:b].float()).to(torch.bfloat16).float()
        # exact window history rows [ctx - W, ctx) of the exact cache (bf16 output), then their LSE merge
        pos = torch.arange(max(0, c - window), c)
        pages = ex_table[r].long()[pos // block]
        win = ex_cache[pages, :, pos % block].float()                                    # [nw, H, 2d]
        p, lse2 = _softmax_rows(torch.einsum('ihd,jhd->hij', q, win[..., :d]) * scale)
        o2 = torch.einsum('hij,jhd->ihd', p, win[..., d:]).to(torch.bfloat16).float()
        lse1, lse2 = lse1.T, lse2.T
        peak = torch.maximum(lse1, lse2)
        peak = torch.where(torch.isfinite(peak), peak, torch.zeros_like(peak))
        w1, w2 = torch.exp(lse1 - peak), torch.exp(lse2 - peak)
        total = w1 + w2
        safe = torch.where(total > 0, total, torch.ones_like(total))
        o_c[a:b] = (o1 * (w1 / safe)[..., None] + o2 * (w2 / safe)[..., None]).to(torch.bfloat16).float()
        lse_c[a:b] = peak + torch.log(total)
    return _merge(_absorb(o_h, B), lse_h, o_c, lse_c, invalid.bool())
