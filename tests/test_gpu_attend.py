"""GPU parity of the composite S6 attention of one layer x loop (s6_layer.attend) against the oracle composite:
decode (exact window + current token, paged latent history, B_t, LSE merge), the prefill / mixed branch (causal
chunk + history-only window), all four loops of a layer, and HIP-graph replay of a decode step."""
import math

import numpy as np
import pytest
import torch

from oracle import bf16
from oracle import s6_oracle as O
from s6util import (FakeLatentLayer, assert_attention_close, dev_bf16, dev_i32, dev_i64, host_f32, latent_cache_bits,
                    random_bits)

pytestmark = pytest.mark.gpu
H, D, W, BLOCK = 16, 128, 32, 16
SCALE = 1 / math.sqrt(D)


class DecodeCase:
    """One decode step of R requests (one token each) on a layer: latent caches for both widths, one exact cache per
    loop, per-request block tables (latent and exact tables differ), absorbed readers of every loop."""

    def __init__(self, rng, history, pad_tokens=0, widths=(512, 256)):
        self.R = len(history)
        self.T = self.R + pad_tokens
        self.history = np.asarray(history, np.int32)
        self.seq_lens = self.history + 1                              # the current token is already in the cache
        self.qsl = np.arange(self.R + 1, dtype=np.int32)
        self.positions = np.concatenate((self.history, np.ones(pad_tokens, np.int64))).astype(np.int64)
        cols = -(-int(self.seq_lens.max()) // BLOCK)
        nb = self.R * cols + 8
        self.tables = {}
        for name in ('latent', 'exact'):
            perm = rng.permutation(np.arange(1, nb))
            self.tables[name] = perm[:self.R * cols].reshape(self.R, cols).astype(np.int32)
        self.lat = {w: latent_cache_bits(rng, nb, BLOCK, w) for w in widths}
        self.exact = [random_bits(rng, (nb, H, BLOCK, 2 * D)) for _ in range(4)]
        r, r1 = widths
        self.sl_bits = dict(A1=random_bits(rng, (H, D, r1), 1 / math.sqrt(2048)),
                            B1=random_bits(rng, (H, r1, D), 1 / math.sqrt(2048)),
                            A=random_bits(rng, (3, H, D, r), 1 / math.sqrt(2048)),
                            B=random_bits(rng, (3, H, r, D), 1 / math.sqrt(2048)))
        self.sl = FakeLatentLayer(*(dev_bf16(self.sl_bits[k]) for k in ('A1', 'B1', 'A', 'B')))
        self.dev = dict(lat={w: dev_bf16(c) for w, c in self.lat.items()}, exact=[dev_bf16(c) for c in self.exact],
                        lt=dev_i32(self.tables['latent']), et=dev_i32(self.tables['exact']))

    def context(self, layer, ops, splits):
        ws = ops.S6Workspace(H, max(self.lat), self.T * splits)
        return layer.StepContext(dev_i64(self.positions), dev_i32(self.qsl), dev_i32(self.seq_lens), 1, self.T,
                                 {}, SCALE, ops.HIP_BACKENDS, ws, splits, window=W, max_seqlen_k=int(self.seq_lens.max()))

    def reader_bits(self, loop):
        if loop == 0:
            return self.sl_bits['B1'], min(self.lat)
        return self.sl_bits['B'][loop - 1], max(self.lat)

    def oracle(self, loop, q_lat_bits, q_rope_bits):
        B, w = self.reader_bits(loop)
        lat = bf16.to_f32(self.lat[w])
        ex = bf16.to_f32(self.exact[loop])
        seq_all = self.seq_lens
        ctx_lat = np.maximum(self.history - W, 0)
        invalid = np.arange(self.T) >= self.R
        req, _ = O.token_requests(self.qsl, self.T)
        lat_tab = self.tables['latent'][req]
        ctx_lat_t = np.where(invalid, 0, ctx_lat[req])
        return O.attend_decode(bf16.to_f32(q_lat_bits), bf16.to_f32(q_rope_bits), bf16.to_f32(B), lat[..., :w],
                               lat[..., w:], lat_tab, ctx_lat_t, ex[..., :D], ex[..., D:], self.tables['exact'],
                               self.qsl, seq_all, W, SCALE, invalid, rounding=False)

    def run(self, layer, ops, ctx, loop, q_lat_bits, q_rope_bits):
        _, w = self.reader_bits(loop)
        return layer.attend(self.sl, loop, dev_bf16(q_lat_bits), dev_bf16(q_rope_bits), None, None, self.dev['lat'][w],
                            self.dev['lt'], None, None, ctx, (self.dev['exact'][loop], self.dev['et']))


def test_config1_single_decode(ops, layer):
    """B = 1, ctx 1024 = 992 latent history rows + the exact window of 32 rows + the current token."""
    rng = np.random.default_rng(0)
    case = DecodeCase(rng, [1024])
    ctx = case.context(layer, ops, 1)
    assert ctx.ctx.tolist() == [1024] and ctx.ctx_latent.tolist() == [992]
    q_lat = random_bits(rng, (1, H, 512), 1 / math.sqrt(512))
    q_rope = random_bits(rng, (1, H, D))
    out = case.run(layer, ops, ctx, 1, q_lat, q_rope)
    want = case.oracle(1, q_lat, q_rope)
    assert out.shape == (1, H, D) and out.dtype == torch.bfloat16
    assert_attention_close(host_f32(out), want)


@pytest.mark.parametrize('rows,splits', [(8, 1), (8, 8), (8, 64), (8, 300), (40, 24)])
def test_ragged_batch_all_loops(ops, layer, rows, splits):
    """Ragged decode rows (one without history, one with history inside the window only, two padding tokens);
    slot counts from one to more than the rows' chunks. These steps have fewer than 64 rows, so the epilogue runs
    one token per workgroup; steps of 64 rows or more (four tokens per workgroup) are in test_gpu_configs.py."""
    rng = np.random.default_rng(1 + splits + rows)
    history = rng.integers(1024, 4096, rows)
    history[2], history[5] = 0, 20                       # no history at all; history inside the window only
    case = DecodeCase(rng, history, pad_tokens=2)
    ctx = case.context(layer, ops, splits)
    for loop in range(4):
        print(f'case loop={loop} splits={splits}', flush=True)
        _, w = case.reader_bits(loop)
        q_lat = random_bits(rng, (case.T, H, w), 1 / math.sqrt(w))
        q_rope = random_bits(rng, (case.T, H, D))
        out = host_f32(case.run(layer, ops, ctx, loop, q_lat, q_rope))
        want = case.oracle(loop, q_lat, q_rope)
        assert_attention_close(out, want, f'loop {loop}')
        assert (out[case.R:] == 0).all()


def test_latent_query_then_attend_matches_fp32_reference(ops, layer):
    """The whole reader path from the pre-RoPE query: A_t + latent RoPE, attend, against the fp32 oracle (no
    intermediate bf16 rounding) at the north-star tolerance."""
    rng = np.random.default_rng(3)
    case = DecodeCase(rng, [3000, 1200, 64, 33])
    ctx = case.context(layer, ops, 4)
    inv = layer.latent_inv_freq(128, 1e6).to('cuda')
    tables = {w: layer.latent_rope_table(8192, inv, w, torch.bfloat16) for w in (512, 256)}
    ctx.tables = tables
    q_pre = random_bits(rng, (case.T, H, D))
    q_rope = random_bits(rng, (case.T, H, D))
    for loop in (0, 2):
        q_lat = ctx.latent_query(case.sl, loop, dev_bf16(q_pre))
        out = layer.attend(case.sl, loop, q_lat, dev_bf16(q_rope), None, None, case.dev['lat'][case.reader_bits(loop)[1]],
                           case.dev['lt'], None, None, ctx, (case.dev['exact'][loop], case.dev['et']))
        A = case.sl_bits['A1'] if loop == 0 else case.sl_bits['A'][loop - 1]
        w = A.shape[-1]
        q_lat32 = O.latent_query(bf16.to_f32(q_pre), bf16.to_f32(A), case.positions, host_f32(tables[w]), rounding=False)
        B, _ = case.reader_bits(loop)
        lat, ex = bf16.to_f32(case.lat[w]), bf16.to_f32(case.exact[loop])
        want = O.attend_decode(q_lat32, bf16.to_f32(q_rope), bf16.to_f32(B), lat[..., :w], lat[..., w:],
                               case.tables['latent'], np.maximum(case.history - W, 0), ex[..., :D], ex[..., D:],
                               case.tables['exact'], case.qsl, case.seq_lens, W, SCALE, np.zeros(case.T, bool),
                               rounding=False)
        assert_attention_close(host_f32(out), want, f'loop {loop}')


@pytest.mark.parametrize('lens,splits,fused', [((6, 1, 3), 1, True), ((6, 1, 3), 8, True), ((6, 1, 3), 4, False),
                                               ((15, 1, 2), 8, True), ((40, 1, 17), 1, True), ((40, 1, 17), 4, True),
                                               ((40, 1, 17), 4, False), ((70, 1, 20), 8, True),
                                               ((70, 1, 20), 8, False)])
def test_prefill_and_mixed_branch(ops, layer, lens, splits, fused):
    """max_query_len > 1: causal chunk + exact window over history rows [ctx - W, ctx) + latent history. Chunks
    shorter than 16 tokens take the fused decode path (exact rows [ctx - W, p] of the exact cache, which holds the
    chunk as the adapter writes it first); longer ones the multi-query history kernel (eight tokens of a request
    per workgroup) with the chunk from k_rope / v, and with split history (fused) the split partials reduced, B_t
    applied and merged in one epilogue (one and four tokens per epilogue workgroup: 60 and 93 rows), or (not fused)
    the reference's op sequence. All against the oracle's reference composite."""
    rng = np.random.default_rng(4 + sum(lens) + splits + fused)
    w = 512
    # request 0: prefill after 900 history rows; request 1: decode after 40; request 2: fresh prompt
    lens, hist = np.array(lens), np.array([900, 40, 0])
    qsl = np.concatenate(([0], np.cumsum(lens))).astype(np.int32)
    T = int(qsl[-1]) + 2
    seq = (hist + lens).astype(np.int32)
    positions = np.concatenate([np.arange(h, h + n) for h, n in zip(hist, lens)] + [np.ones(2, np.int64)])
    cols = -(-int(seq.max()) // BLOCK)
    nb = 3 * cols + 4
    lt = rng.permutation(np.arange(1, nb))[:3 * cols].reshape(3, cols).astype(np.int32)
    et = rng.permutation(np.arange(1, nb))[:3 * cols].reshape(3, cols).astype(np.int32)
    lat = latent_cache_bits(rng, nb, BLOCK, w)
    ex = random_bits(rng, (nb, H, BLOCK, 2 * D))
    B = random_bits(rng, (H, w, D), 1 / math.sqrt(2048))
    sl = FakeLatentLayer(dev_bf16(random_bits(rng, (H, D, 256))), dev_bf16(random_bits(rng, (H, 256, D))),
                         dev_bf16(random_bits(rng, (3, H, D, w))), dev_bf16(np.stack([B] * 3)))
    q_lat = random_bits(rng, (T, H, w), 1 / math.sqrt(w))
    q_rope, k_rope, v = (random_bits(rng, (T, H, D)) for _ in range(3))
    for r in range(3):   # the adapter writes the chunk's k / v to the exact cache before attending
        for i in range(int(lens[r])):
            pos, tok = int(hist[r]) + i, int(qsl[r]) + i
            ex[et[r, pos // BLOCK], :, pos % BLOCK, :D] = k_rope[tok]
            ex[et[r, pos // BLOCK], :, pos % BLOCK, D:] = v[tok]
    ws = ops.S6Workspace(H, w, T * splits)
    ctx = layer.StepContext(dev_i64(positions), dev_i32(qsl), dev_i32(seq), int(lens.max()), T, {}, SCALE,
                            ops.HIP_BACKENDS, ws, splits, window=W, max_seqlen_k=int(seq.max()))
    ctx.fused_chunks = fused
    assert ctx.history_group == (4 if lens.max() >= 16 else 1)
    out = layer.attend(sl, 1, dev_bf16(q_lat), dev_bf16(q_rope), dev_bf16(k_rope), dev_bf16(v), dev_bf16(lat),
                       dev_i32(lt), None, None, ctx, (dev_bf16(ex), dev_i32(et)))
    req, valid, c, cl = O.step_context(qsl, seq, T, W)
    latf, exf = bf16.to_f32(lat), bf16.to_f32(ex)
    want = O.attend_chunk(bf16.to_f32(q_lat), bf16.to_f32(q_rope), bf16.to_f32(k_rope), bf16.to_f32(v), bf16.to_f32(B),
                          latf[..., :w], latf[..., w:], {'latent': lt[req], 'exact': et[req]}, c, cl, qsl, W, SCALE,
                          ~valid, exf[..., :D], exf[..., D:], rounding=False)
    got = host_f32(out)
    assert_attention_close(got, want)
    assert (got[~valid] == 0).all()


def test_decode_step_replays_in_a_hip_graph(ops, layer):
    """Step metadata + A_t/RoPE + attend captured once; every replay (new query, new lengths) equals eager."""
    rng = np.random.default_rng(5)
    case = DecodeCase(rng, [2000, 1500, 700, 64, 5, 3000])
    inv = layer.latent_inv_freq(128, 1e6).to('cuda')
    tables = {w: layer.latent_rope_table(8192, inv, w, torch.bfloat16) for w in (512, 256)}
    splits = 8
    ws = ops.S6Workspace(H, 512, case.T * splits)
    pos = dev_i64(case.positions)
    qsl, seq = dev_i32(case.qsl), dev_i32(case.seq_lens)
    q_pre = dev_bf16(random_bits(rng, (case.T, H, D)))
    q_rope = dev_bf16(random_bits(rng, (case.T, H, D)))

    def step():
        ctx = layer.StepContext(pos, qsl, seq, 1, case.T, tables, SCALE, ops.HIP_BACKENDS, ws, splits, window=W,
                                max_seqlen_k=4096)
        q_lat = ctx.latent_query(case.sl, 2, q_pre)
        return layer.attend(case.sl, 2, q_lat, q_rope, None, None, case.dev['lat'][512], case.dev['lt'], None, None,
                            ctx, (case.dev['exact'][2], case.dev['et']))

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = step()
    for i in range(3):
        q_pre.copy_(dev_bf16(random_bits(rng, (case.T, H, D))))
        new_hist = rng.integers(0, 3000, case.R).astype(np.int32)
        seq.copy_(dev_i32(new_hist + 1))
        pos.copy_(dev_i64(new_hist))
        graph.replay()
        torch.cuda.synchronize()
        eager = step()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f'replay {i} differs from eager'
