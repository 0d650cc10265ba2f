"""GPU parity of the decode step at the benchmark configurations' full shapes, against the oracle composite
(``O.attend_decode``: exact window + current token, paged latent history, B_t, LSE merge), all four loops of a layer:

* the headline step: 64 decode rows at context 8192 (+ 2 padding rows), 16 slots per row at width 512 and 32 at
  256 (the MI355X split policy at 64 rows, the bench's split plan), which runs the four-token epilogue;
* long context: 8 rows at context 32768, the history split over 8, 16 and 32 slots and the MI355X policy
  (128 / 256);
* ragged decode: 32 rows with contexts drawn from U[1024, 8192] on 65,536-page pools (2 GiB main latent, 1 GiB
  loop-1 latent: page ids up to 65,535, byte offsets past 2^31);
* short-chunk prefill: 4 requests x 3 tokens on 8192 latent rows (against ``O.attend_chunk``), on the fused path and
  the reference's op sequence, and a mixed step of decode rows and chunks of 2..15 tokens;
* steps whose longest chunk has 2 or 3 tokens over ragged histories (one-token requests beside them, an empty
  history, padding);
* a few-token decode step planned for a 32768-token model (hundreds of slots, mostly empty) and for its own length;
* chunked prefill of 4 requests x 512 and x 128 tokens over 8,192 latent rows (the multi-query configuration at
  full size), sampled tokens of every request.

Caches live on the device; page 0 and every page no request references are +inf-poisoned, so a read outside a row's
pages cannot go unseen. The oracle reads host copies of the referenced pages only (through a remapped table).
Bars: max-abs 2e-2 and rel-L2 5e-3 against the fp32 oracle; padding rows exactly zero."""
import math

import numpy as np
import pytest
import torch

from oracle import s6_oracle as O
from s6util import FakeLatentLayer, assert_attention_close, host_f32

pytestmark = pytest.mark.gpu
H, D, W, BLOCK = 16, 128, 32, 16
SCALE = 1 / math.sqrt(D)
WIDTHS = (512, 256)
POS_INF = float('inf')


class DeviceDecode:
    """A step of ``len(hist)`` requests (``lens`` new tokens each, default one: a decode step; ``pad`` padding
    tokens) with caches on the device: per width one latent cache of ``pool`` pages whose tables are slices of one
    random permutation, one small exact cache per loop holding the window pages and the step's tokens (the adapter
    writes them before attending), random readers of all four loops."""

    def __init__(self, hist, pad=0, pool=None, seed=0, lens=None):
        g = torch.Generator(device='cuda').manual_seed(seed)
        self.hist = np.asarray(hist, np.int64)
        self.lens = np.ones(len(hist), np.int64) if lens is None else np.asarray(lens, np.int64)
        self.qsl = np.concatenate(([0], np.cumsum(self.lens))).astype(np.int32)
        self.R, self.T = len(hist), int(self.lens.sum()) + pad
        self.seq = self.hist + self.lens                           # the step's tokens are already in the exact cache
        pages = -(-self.seq // BLOCK)
        self.cols = int(pages.max())
        self.pool = int(pool or pages.sum() + 1)
        assert self.pool > pages.sum()
        randn = lambda *s, std=1.0: (torch.randn(*s, generator=g, device='cuda') * std).to(torch.bfloat16)
        self.tables, self.lat = {}, {}
        for w in WIDTHS:
            perm = (torch.randperm(self.pool - 1, generator=g, device='cuda') + 1).to(torch.int32).cpu().numpy()
            table = np.zeros((self.R, self.cols), np.int32)
            used = 0
            for r in range(self.R):
                table[r, :pages[r]] = perm[used:used + pages[r]]
                used += pages[r]
            cache = torch.empty(self.pool, 1, BLOCK, 2 * w, dtype=torch.bfloat16, device='cuda').normal_(generator=g)
            referenced = torch.zeros(self.pool, dtype=torch.bool, device='cuda')
            referenced[torch.as_tensor(perm[:used], device='cuda').long()] = True
            cache[~referenced] = POS_INF                           # page 0 and every unreferenced page
            self.tables[w], self.lat[w] = table, cache
        first, last = np.maximum(self.hist - W, 0) // BLOCK, (self.seq - 1) // BLOCK
        ex_pool = int((last - first + 1).sum()) + 1
        self.ex_table = np.zeros((self.R, self.cols), np.int32)
        perm = np.random.default_rng(seed).permutation(np.arange(1, ex_pool)).astype(np.int32)
        used = 0
        for r in range(self.R):
            n = int(last[r] - first[r] + 1)
            self.ex_table[r, first[r]:last[r] + 1] = perm[used:used + n]
            used += n
        self.exact = []
        for _ in range(4):
            ex = randn(ex_pool, H, BLOCK, 2 * D)
            ex[0] = POS_INF
            self.exact.append(ex)
        std = 1 / math.sqrt(2048)
        self.sl = FakeLatentLayer(randn(H, D, 256, std=std), randn(H, 256, D, std=std), randn(3, H, D, 512, std=std),
                                  randn(3, H, 512, D, std=std))
        self.q_lat = [randn(self.T, H, 256 if loop == 0 else 512, std=(256 if loop == 0 else 512) ** -0.5)
                      for loop in range(4)]
        self.q_rope = [randn(self.T, H, D) for _ in range(4)]
        self.dev_tables = {w: torch.as_tensor(t, device='cuda') for w, t in self.tables.items()}
        self.dev_ex_table = torch.as_tensor(self.ex_table, device='cuda')

    def context(self, layer, ops, splits_by_width):
        positions = np.concatenate([np.arange(h, h + n) for h, n in zip(self.hist, self.lens)] +
                                   [np.ones(self.T - int(self.lens.sum()), np.int64)])
        ws = ops.S6Workspace.for_splits(H, self.T, splits_by_width)
        return layer.StepContext(torch.as_tensor(positions, device='cuda'), torch.as_tensor(self.qsl, device='cuda'),
                                 torch.as_tensor(self.seq.astype(np.int32), device='cuda'), int(self.lens.max()),
                                 self.T, {}, SCALE, ops.HIP_BACKENDS, ws, splits_by_width[512], window=W,
                                 max_seqlen_k=int(self.seq.max()), kv_splits_by_width=splits_by_width)

    def run(self, layer, ctx, loop):
        w = 256 if loop == 0 else 512
        k_rope = v = None
        if not (self.lens == 1).all():   # the reference's branch reads the chunk from k_rope / v
            req, valid, _, _ = O.step_context(self.qsl, self.seq, self.T, W)
            pos = np.where(valid, self.hist[req] + np.arange(self.T) - self.qsl[req], 0)
            pages = torch.as_tensor(self.ex_table[req, pos // BLOCK], device='cuda').long()
            rows = self.exact[loop][pages, :, torch.as_tensor(pos % BLOCK, device='cuda')]   # [T, H, 2D]
            k_rope, v = rows[..., :D].contiguous(), rows[..., D:].contiguous()
        return layer.attend(self.sl, loop, self.q_lat[loop], self.q_rope[loop], k_rope, v, self.lat[w],
                            self.dev_tables[w], None, None, ctx, (self.exact[loop], self.dev_ex_table))

    def oracle(self, loop, sample=None):
        """The oracle composite on host copies of the pages the rows reference (the table remapped to them):
        O.attend_decode for a decode step, O.attend_chunk (the reference's causal chunk of k_rope / v + window
        history + latent history) otherwise, with the chunk's k / v read back from the exact cache. ``sample`` (a
        token mask) limits a chunked step's oracle to those tokens (every valid token still serves as a key of the
        chunk); the other rows come back zero."""
        w = 256 if loop == 0 else 512
        table = self.tables[w]
        ctx_lat = np.maximum(self.hist - W, 0)
        need = -(-ctx_lat // BLOCK)
        used = np.unique(np.concatenate([table[r, :need[r]] for r in range(self.R)] + [np.zeros(1, np.int32)]))
        remap = np.zeros(self.pool, np.int64)
        remap[used] = np.arange(used.size)
        lat = self.lat[w][torch.as_tensor(used, device='cuda').long()].float().cpu().numpy()
        req, valid, ctx, ctx_lat_t = O.step_context(self.qsl, self.seq, self.T, W)
        tok_table = np.where(valid[:, None], remap[table][req], 0)
        ex = host_f32(self.exact[loop])
        B = host_f32(self.sl.readers(loop)[1])
        q_lat, q_rope = host_f32(self.q_lat[loop]), host_f32(self.q_rope[loop])
        if (self.lens == 1).all():
            return O.attend_decode(q_lat, q_rope, B, lat[..., :w], lat[..., w:], tok_table, ctx_lat_t, ex[..., :D],
                                   ex[..., D:], self.ex_table, self.qsl, self.seq, W, SCALE, ~valid, rounding=False)
        k_rope, v = np.zeros((self.T, H, D), np.float32), np.zeros((self.T, H, D), np.float32)
        for t in np.nonzero(valid)[0]:
            p = int(self.hist[req[t]] + t - self.qsl[req[t]])
            row = ex[self.ex_table[req[t], p // BLOCK], :, p % BLOCK]
            k_rope[t], v[t] = row[:, :D], row[:, D:]
        attend = valid if sample is None else valid & sample
        ctx, ctx_lat_t = np.where(attend, ctx, 0), np.where(attend, ctx_lat_t, 0)
        return O.attend_chunk(q_lat, q_rope, k_rope, v, B, lat[..., :w], lat[..., w:],
                              {'latent': tok_table, 'exact': self.ex_table[req]}, ctx, ctx_lat_t, self.qsl, W, SCALE,
                              ~attend, ex[..., :D], ex[..., D:], rounding=False)


def _check(case, layer, ops, splits_by_width, loops=range(4), wants=None, fused=True):
    ctx = case.context(layer, ops, splits_by_width)
    ctx.fused_chunks = fused
    wants = {} if wants is None else wants
    n = int(case.lens.sum())
    for loop in loops:
        print(f'case R={case.R} T={case.T} lens<={case.lens.max()} loop={loop} splits={splits_by_width} '
              f'fused={fused}', flush=True)
        out = host_f32(case.run(layer, ctx, loop))
        if loop not in wants:
            wants[loop] = case.oracle(loop)
        assert_attention_close(out[:n], wants[loop][:n], f'loop {loop}')
        assert (out[n:] == 0).all()
    return wants


@pytest.mark.parametrize('pad', [0, 2])
def test_headline_decode_step(ops, layer, pad):
    """64 rows at context 8192 (8160 latent rows + the 32-row window + the current token), all four loops, with the
    split counts the bench runs; 64 rows or more take the four-token epilogue."""
    cus = 256
    splits = {w: ops.mi355x_kv_splits(8193, 64, cus, width=w) for w in WIDTHS}
    assert splits == {512: 16, 256: 32}
    case = DeviceDecode([8192] * 64, pad=pad, seed=30 + pad)
    assert case.T >= 64
    _check(case, layer, ops, splits)


def test_long_context_split_counts(ops, layer):
    """8 rows at context 32768; the same step over 8, 16 and 32 slots per row and the MI355X policy (128 / 256)."""
    case = DeviceDecode([32768] * 8, pad=1, seed=40)
    policy = {w: ops.mi355x_kv_splits(32769, 8, 256, width=w) for w in WIDTHS}
    assert policy == {512: 128, 256: 256}
    wants = None
    for splits in ({512: 8, 256: 8}, {512: 16, 256: 16}, {512: 32, 256: 32}, policy):
        wants = _check(case, layer, ops, splits, wants=wants)


def test_ragged_decode_on_full_pools(ops, layer):
    """32 rows with contexts from U[1024, 8192] whose tables are slices of one permutation of a 65,536-page pool
    (the benchmark's pools: 2 GiB main latent, 1 GiB loop-1 latent), all four loops, the MI355X policy."""
    hist = np.random.default_rng(50).integers(1024, 8193, 32)
    case = DeviceDecode(hist, pad=2, pool=65536, seed=50)
    assert case.lat[512].numel() * 2 == 2 << 30 and case.lat[256].numel() * 2 == 1 << 30
    assert max(int(case.tables[w].max()) for w in WIDTHS) > 65000
    splits = {w: ops.mi355x_kv_splits(int(case.seq.max()), case.T, 256, width=w) for w in WIDTHS}
    _check(case, layer, ops, splits)


def test_few_token_steps_planned_for_a_long_model(ops, layer):
    """Three decode rows of 2048, 1500 and 40 history tokens (and a padding row) with the slot counts the policy gives
    for a model length of 32768, as the adapter plans a step (hundreds of slots, of which the plan's 4-tile items
    fill a few dozen per row: the empty ones get their lse from one coalesced range), and for the step's own length;
    all four loops, both against the oracle and the same results either way."""
    case = DeviceDecode([2048, 1500, 40], pad=1, seed=70)
    wide = {w: ops.mi355x_kv_splits(32768, case.T, 256, width=w) for w in WIDTHS}
    tight = {w: ops.mi355x_kv_splits(int(case.seq.max()), case.T, 256, width=w) for w in WIDTHS}
    assert min(wide.values()) >= 256 and max(tight.values()) <= 66
    wants = _check(case, layer, ops, wide)
    _check(case, layer, ops, tight, wants=wants)


def test_short_chunk_prefill(ops, layer):
    """Chunked prefill of 4 requests x 3 tokens on 8192 latent rows (+ the 32-row window): the K-hop-sized step,
    on the fused path (the chunk's keys from the exact cache) and on the reference's op sequence, all four loops;
    then a mixed step (decode rows, chunks of 2..15 tokens, a fresh prompt of 5, padding)."""
    case = DeviceDecode([8192 + W] * 4, pad=2, seed=60, lens=[3] * 4)
    splits = {w: ops.mi355x_kv_splits(8192 + W + 3, 12, 256, width=w) for w in WIDTHS}
    wants = _check(case, layer, ops, splits)
    _check(case, layer, ops, splits, wants=wants, fused=False)
    mixed = DeviceDecode([3000, 17, 900, 0, 5000, 40, 1200], pad=3, seed=61, lens=[1, 15, 4, 5, 2, 1, 9])
    splits = {w: ops.mi355x_kv_splits(int(mixed.seq.max()), mixed.T, 256, width=w) for w in WIDTHS}
    _check(mixed, layer, ops, splits, loops=(0, 1))


@pytest.mark.parametrize('hist,lens,pad', [([2000, 700, 4100, 33], [2, 2, 2, 2], 1),
                                           ([1500, 0, 3100, 260, 90], [3, 1, 2, 3, 3], 2),
                                           ([6000, 40, 2500], [2, 1, 2], 0)])
def test_two_and_three_token_chunks(ops, layer, hist, lens, pad):
    """Steps whose longest chunk has 2 or 3 tokens on the fused path (one token per history workgroup, the chunk's
    exact keys from the exact cache): ragged histories, one-token requests beside the chunks, an empty history and
    padding, all four loops, against the oracle and the reference's op sequence."""
    case = DeviceDecode([h + W for h in hist], pad=pad, seed=62 + len(hist), lens=lens)
    splits = {w: ops.mi355x_kv_splits(int(case.seq.max()), case.T, 256, width=w) for w in WIDTHS}
    wants = _check(case, layer, ops, splits)
    _check(case, layer, ops, splits, wants=wants, fused=False)


@pytest.mark.parametrize('queries', [512, 128])
def test_multi_query_prefill_full_size(ops, layer, queries):
    """Chunked prefill of 4 requests x ``queries`` tokens over 8,192 latent rows + the 32-row window (the
    multi-query configuration at its full size), all four loops, at the MI355X split policy: one slot at 512
    tokens per request (the multi-query history kernel, then the reference's op sequence), four at 128 (the split
    partials reduced with B_t and the merge in one epilogue). The first, middle and last 8 tokens of each request
    are checked against the oracle, every head; the chunk's other tokens still serve as its keys."""
    case = DeviceDecode([8192 + W] * 4, pad=1, seed=70 + queries, lens=[queries] * 4)
    splits = {w: ops.mi355x_kv_splits(int(case.seq.max()), case.T, 256, width=w, tokens_per_group=4) for w in WIDTHS}
    assert splits == ({512: 1, 256: 1} if queries == 512 else {512: 4, 256: 4})
    picks = np.concatenate([np.r_[0:8, queries // 2 - 4:queries // 2 + 4, queries - 8:queries] + r * queries
                            for r in range(4)])
    sample = np.zeros(case.T, bool)
    sample[picks] = True
    ctx = case.context(layer, ops, splits)
    assert ctx.history_group == 4
    for loop in range(4):
        print(f'case 4 x {queries} tokens over 8192 + {W} rows loop={loop} splits={splits}', flush=True)
        out = host_f32(case.run(layer, ctx, loop))
        want = case.oracle(loop, sample)
        assert_attention_close(out[picks], want[picks], f'loop {loop}')
        assert (out[case.T - 1:] == 0).all()
