"""GPU parity of the small ops through the C ABI: step metadata, block-table gather, slot mapping and row store
(bit-exact), latent RoPE (bit-exact to the torch op order), the A_t / B_t MFMA GEMMs, the exact-window and chunk
kernels and the LSE merges (north-star tolerances against the fp32 oracle)."""
import json
import math
import os

import numpy as np
import pytest
import torch

from oracle import bf16
from oracle import s6_oracle as O
from s6util import (assert_attention_close, assert_lse_close, dev_bf16, dev_i32, dev_i64, host_f32, random_bits)

pytestmark = pytest.mark.gpu
KNOWN = json.load(open(os.path.join(os.path.dirname(__file__), 'golden', 'known_answers.json')))
CUDA = 'cuda'


# ------------------------------------------------------------------------------------------------ metadata

@pytest.mark.parametrize('case', KNOWN['token_requests']['cases'], ids=lambda c: str(c['qsl']) + f"/T{c['num_tokens']}")
def test_token_requests_known_answers(ops, case):
    req, valid = ops.token_requests(dev_i32(case['qsl']), case['num_tokens'])
    assert req.dtype == torch.int64 and valid.dtype == torch.bool
    assert req.tolist() == case['req'] and valid.tolist() == [bool(v) for v in case['valid']]


@pytest.mark.parametrize('case', KNOWN['history_lengths']['cases'], ids=lambda c: str(c['qsl']))
def test_history_lengths_known_answers(ops, case):
    assert ops.history_lengths(dev_i32(case['seq_lens']), dev_i32(case['qsl'])).tolist() == case['expected']


def test_step_context_random_ragged_is_bit_exact(layer):
    rng = np.random.default_rng(0)
    for trial in range(5):
        R = int(rng.integers(1, 40))
        lens = rng.integers(0, 6, R)
        lens[rng.random(R) < 0.3] = 1
        qsl = np.concatenate(([0], np.cumsum(lens))).astype(np.int32)
        pad_req = int(rng.integers(0, 3))
        qsl = np.concatenate((qsl, [qsl[-1]] * pad_req)).astype(np.int32)
        T = int(qsl[-1]) + int(rng.integers(0, 4))
        seq = np.concatenate((lens + rng.integers(0, 9000, R), np.zeros(pad_req, np.int64))).astype(np.int32)
        window = int(rng.choice([0, 32]))
        ctx = layer.StepContext(dev_i64(np.arange(T)), dev_i32(qsl), dev_i32(seq), int(lens.max()), T, {}, 1.0,
                                None, window=window)
        req, valid, c, cl = O.step_context(qsl, seq, T, window)
        assert ctx.token_requests.tolist() == req.tolist(), trial
        assert ctx.valid.tolist() == valid.tolist() and ctx.ctx.tolist() == c.tolist()
        assert ctx.ctx_latent.tolist() == cl.tolist()
        assert torch.equal(ctx.invalid, ~ctx.valid) and torch.equal(ctx.empty, ctx.ctx == 0)
        table = rng.integers(0, 1000, (qsl.shape[0] - 1, 7)).astype(np.int32)
        got = ctx.block_table(dev_i32(table))
        assert got.tolist() == O.token_block_table(table, req).tolist()


def test_step_context_known_mixed_step(layer):
    g = KNOWN['step_context_mixed']
    ctx = layer.StepContext(dev_i64([5, 2, 1, 1]), dev_i32(g['qsl']), dev_i32(g['seq_lens']), 1, g['num_tokens'], {},
                            1.0, None)
    assert ctx.token_requests.tolist() == g['token_requests'] and ctx.ctx.tolist() == g['ctx']
    prof = layer.StepContext(dev_i64(np.arange(5)), None, None, None, 5, {}, 1.0, None)
    assert not prof.md_present and prof.valid.all() and (prof.ctx == 0).all() and prof.max_query_len == 5


def test_rollout_rows_slot_mapping_and_store(layer):
    """Slot mapping + row store reproduce the reference's bit-exact rollout-cache rows."""
    g = KNOWN['rollout_rows']
    bs = g['block_size']
    pos = np.array(g['positions'])
    ctx = layer.StepContext(dev_i64(pos), dev_i32([0, 3]), dev_i32([3]), 3, 3, {}, 1.0, None)
    rows = []
    for part in ('main', 'l1'):
        p = g[part]
        w = p['row_width'] // 2
        want_cache = torch.arange(p['num_blocks'] * bs * 2 * w, dtype=torch.float32).view(p['num_blocks'], 1, bs, 2 * w)
        slots = layer.slot_mapping(ctx, dev_i32([p['table']]), bs)
        assert slots.tolist() == O.slot_mapping(np.array([p['table']]), np.zeros(3, np.int64), np.ones(3, bool), pos,
                                                bs).tolist()
        # store the expected rows through the kernel into an empty cache, then read them back by slot
        src = want_cache.view(-1, 2 * w)[slots.cpu()].to(torch.bfloat16).to(CUDA)
        cache = torch.full((p['num_blocks'], 1, bs, 2 * w), float('nan'), dtype=torch.bfloat16, device=CUDA)
        layer.store_rows(src[:, :w].contiguous(), src[:, w:].contiguous(), slots, cache)
        rows.append(cache.view(-1, 2 * w)[slots].float().cpu())
    assert torch.cat(rows, -1).tolist() == [[float(x) for x in r] for r in g['expected_rows']]


def test_slot_mapping_padding_and_out_of_table_positions(layer):
    ctx = layer.StepContext(dev_i64([0, 5, 9, 1]), dev_i32([0, 1, 2, 3]), dev_i32([1, 6, 10]), 1, 4, {}, 1.0, None)
    slots = layer.slot_mapping(ctx, dev_i32([[3, 0], [7, 8], [4, 4]]), 4)
    assert slots.tolist() == [12, 33, -1, -1]     # pos 9 is past the 2-column table; token 3 is padding


# ------------------------------------------------------------------------------------------------ RoPE / GEMMs

def _table(layer, width, rows=4096, theta=1e6):
    inv = layer.latent_inv_freq(128, theta).to(CUDA)
    return layer.latent_rope_table(rows, inv, width, torch.bfloat16)


def _bf16_ulp(x):
    """Spacing of bf16 values at |x| (8 significant bits), in float64."""
    a = np.maximum(np.abs(np.asarray(x, np.float64)), 2.0 ** -126)
    return 2.0 ** (np.floor(np.log2(a)) - 7)


@pytest.mark.parametrize('width', [512, 256])
def test_latent_rope_table_on_the_device(layer, width):
    """The persistent [65536, w] bf16 table built on the device (hla/vllm_latent/s6_layer.py:16-29) against the
    oracle's. The frequencies come from torch's fp32 pow, as the reference's do; they must lie within 2 fp32 ulp of
    the correctly rounded theta^(-2i/128). Given the frequencies, the fp32 angles are IEEE products; cos / sin of the
    same fp32 angle differ between math libraries by about an fp32 ulp, which moves a bf16 rounding in a few entries
    in 10^5, so every entry must lie within one bf16 ulp of the float64 cos / sin of the fp32 angle and at least
    99.99 % of the entries must equal the oracle's table (built from the same frequencies) bit for bit. Row 0 is
    exactly [1 ... 1 | 0 ... 0] (hla/tests/test_s6_ops.py:36)."""
    inv = layer.latent_inv_freq(128, 1e6)
    inv_h = inv.numpy()
    exact_inv = (1.0 / (1e6 ** (np.arange(0, 128, 2) / 128.0))).astype(np.float32)
    assert inv_h.dtype == np.float32 and np.abs(inv_h.view(np.int32) - exact_inv.view(np.int32)).max() <= 2
    table = layer.latent_rope_table(65536, inv.to(CUDA), width, torch.bfloat16)
    inv_o = inv_h
    assert table.shape == (65536, width) and table.dtype == torch.bfloat16
    got = host_f32(table)
    want = bf16.round_bf16(O.latent_rope_table(65536, inv_o, width))
    idx = np.arange(width // 2) % 64
    angle = np.arange(65536, dtype=np.float32)[:, None] * inv_o[idx][None, :]
    exact = np.concatenate((np.cos(angle.astype(np.float64)), np.sin(angle.astype(np.float64))), -1)
    assert (got[0, :width // 2] == 1).all() and (got[0, width // 2:] == 0).all()
    err = np.abs(got.astype(np.float64) - exact)
    bad = err > _bf16_ulp(exact) + 2.0 ** -20
    assert not bad.any(), f'{int(bad.sum())} entries more than one bf16 ulp off, first at {np.argwhere(bad)[:3].tolist()}'
    same = float((got == want).mean())
    assert same >= 0.9999, f'only {same:.6f} of the entries equal the oracle table'
    # the pairing: column c and c + w/2 hold cos and sin of the same angle (frequency c % 64)
    np.testing.assert_allclose(got[:, :width // 2] ** 2 + got[:, width // 2:] ** 2, 1.0, atol=2e-2)


@pytest.mark.parametrize('width', [512, 256])
def test_latent_rope_layouts_bit_exact(ops, layer, width):
    rng = np.random.default_rng(4)
    T, H = 33, 16
    table = _table(layer, width)
    table_h = host_f32(table)
    pos = rng.integers(0, table.shape[0], T)
    q = dev_bf16(random_bits(rng, (H, T, width))).transpose(0, 1)          # einsum-shaped, head stride T*w
    row = dev_bf16(random_bits(rng, (T, 2 * width)))
    flat = q.reshape(T, -1).clone()
    want_q = O.latent_rope(host_f32(q), pos, table_h, rounding=True)
    want_row = O.latent_rope(host_f32(row[:, :width]), pos, table_h, rounding=True)
    v_before = row[:, width:].clone()
    got_q = ops.latent_rope(q.clone(), dev_i64(pos), table, 'hip')
    got_row = ops.latent_rope(row[:, :width], dev_i64(pos), table, 'hip')
    got_flat = ops.latent_rope(flat, dev_i64(pos), table, 'hip')
    assert got_row.data_ptr() == row.data_ptr() and got_row.stride() == (2 * width, 1)
    np.testing.assert_array_equal(host_f32(got_q), want_q)
    np.testing.assert_array_equal(host_f32(got_row), want_row)
    np.testing.assert_array_equal(host_f32(got_flat).reshape(T, H, width), want_q)
    assert torch.equal(row[:, width:], v_before)
    assert ops.probe_latent_rope(table, 16) == (False, True)


@pytest.mark.parametrize('T', [1, 64, 200])
@pytest.mark.parametrize('width', [512, 256])
def test_latent_query_fused_absorb_rope(layer, T, width):
    rng = np.random.default_rng(5)
    table = _table(layer, width)
    q = random_bits(rng, (T, 16, 128))
    A = random_bits(rng, (16, 128, width), 1 / math.sqrt(2048))
    pos = rng.integers(0, table.shape[0], T)
    got = layer.latent_query(dev_bf16(q), dev_bf16(A), dev_i64(pos), table, 'hip')
    want = O.latent_query(bf16.to_f32(q), bf16.to_f32(A), pos, host_f32(table), rounding=True)
    assert got.shape == (T, 16, width) and got.is_contiguous()
    assert_attention_close(host_f32(got), want, 'q_lat', max_abs=2e-2, rel=5e-3)


@pytest.mark.parametrize('T', [1, 64, 130])
@pytest.mark.parametrize('r', [512, 256])
def test_out_projection_gemm(layer, T, r):
    rng = np.random.default_rng(6)
    o = random_bits(rng, (T, 16, r))
    B = random_bits(rng, (16, r, 128), 1 / math.sqrt(2048))
    got = layer.absorb_out(dev_bf16(o), dev_bf16(B))
    want = O.absorb(bf16.to_f32(o), bf16.to_f32(B), rounding=False)
    assert_attention_close(host_f32(got), want, 'o_B')


# ------------------------------------------------------------------------------------------------ exact window / chunk

def _exact_cache(rng, nb, H, block, d):
    bits = random_bits(rng, (nb, H, block, 2 * d))
    bits[0] = 0x7F80
    return bits


@pytest.mark.parametrize('window', [0, 1, 32, 100])
def test_window_decode(ops, window):
    rng = np.random.default_rng(7)
    H, d, block, nb = 16, 128, 16, 300
    seq_lens = np.array([1, 2, 20, 33, 34, 200, 1000, 65], np.int32)
    R = len(seq_lens)
    pad_req = 2
    qsl = np.concatenate((np.arange(R + 1), [R] * pad_req)).astype(np.int32)
    T = R + 3                                        # three padding tokens
    seq_all = np.concatenate((seq_lens, np.zeros(pad_req, np.int32))).astype(np.int32)
    cache = _exact_cache(rng, nb, H, block, d)
    cols = 70
    table = np.zeros((R + pad_req, cols), np.int32)
    for r in range(R):
        need = -(-int(seq_lens[r]) // block)
        table[r, :need] = rng.integers(1, nb, need)
    q = random_bits(rng, (T, H, d))
    scale = 1 / math.sqrt(d)
    invalid = np.arange(T) >= R
    o, lse = ops.window_attention_fa(dev_bf16(q), dev_bf16(cache), dev_i32(table), dev_i32(qsl), dev_i32(seq_all),
                                     window, scale, 0, torch.as_tensor(invalid, device=CUDA))
    cf = bf16.to_f32(cache)
    want_o, want_lse = O.window_decode(bf16.to_f32(q), cf[..., :d], cf[..., d:], table, qsl, seq_all, window, scale,
                                       invalid)
    assert_attention_close(host_f32(o), want_o, 'window o')
    assert_lse_close(host_f32(lse), want_lse)
    assert (host_f32(o)[invalid] == 0).all()


@pytest.mark.parametrize('window', [1, 32])
def test_window_history(ops, window):
    rng = np.random.default_rng(8)
    H, d, block, nb = 16, 128, 16, 200
    ctx = np.array([0, 1, 5, 31, 32, 33, 500, 0, 77], np.int32)
    cache = _exact_cache(rng, nb, H, block, d)
    table = np.zeros((len(ctx), 40), np.int32)
    for t, c in enumerate(ctx):
        need = -(-int(c) // block)
        table[t, :need] = rng.integers(1, nb, need)
    q = random_bits(rng, (len(ctx), H, d))
    o, lse = ops.window_history_fa(dev_bf16(q), dev_bf16(cache), dev_i32(table), dev_i32(ctx), window, 0.1, 0,
                                   torch.as_tensor(ctx == 0, device=CUDA))
    cf = bf16.to_f32(cache)
    want_o, want_lse = O.window_history(bf16.to_f32(q), cf[..., :d], cf[..., d:], table, ctx, window, 0.1)
    assert_attention_close(host_f32(o), want_o, 'window-history o')
    assert_lse_close(host_f32(lse), want_lse)
    o2, lse2 = ops.window_attention(dev_bf16(q), dev_bf16(cache), dev_i32(table), dev_i32(ctx), window, 0.1)
    assert torch.equal(o, o2) and torch.equal(lse, lse2)


@pytest.mark.parametrize('qsl,T', [((0, 5, 6, 20, 20, 20), 24),        # empty requests, four padding tokens
                                   ((0, 100, 101, 400, 413), 420),      # long chunks crossing 16-token blocks
                                   ((0, 300, 301, 1000, 1100), 1104),   # 4-wave blocks (one per CU or more)
                                   ((0, 15, 45, 46, 70, 100, 131, 160, 190, 222, 250, 280, 300), 304)])
def test_chunk_attention(ops, qsl, T):
    """Single-wave 16-token blocks for steps of short requests (fewer than 64 tokens on average) whose 64-token
    blocks x 16 heads would leave CUs idle (the first and last cases), 4-wave 64-token blocks otherwise."""
    rng = np.random.default_rng(9 + T)
    H, d = 16, 128
    qsl = np.array(qsl, np.int32)
    q, k, v = (random_bits(rng, (T, H, d)) for _ in range(3))
    invalid = np.arange(T) >= qsl[-1]
    o, lse = ops.chunk_attention(dev_bf16(q), dev_bf16(k), dev_bf16(v), dev_i32(qsl), int(np.diff(qsl).max()),
                                 torch.as_tensor(invalid, device=CUDA), 1 / math.sqrt(d), 'hip')
    want_o, want_lse = O.chunk_attention(bf16.to_f32(q), bf16.to_f32(k), bf16.to_f32(v), qsl, invalid, 1 / math.sqrt(d))
    assert o.is_contiguous() and lse.is_contiguous() and lse.shape == (H, T)
    assert_attention_close(host_f32(o), want_o, 'chunk o')
    assert_lse_close(host_f32(lse), want_lse)


@pytest.mark.parametrize('lens,hist,pad', [((5, 1, 14, 0, 0), (0, 40, 7, 3, 0), 4),   # no history, short history,
                                           ((100, 1, 299, 13), (33, 90, 0, 17), 7),   # empty requests, padding
                                           ((600, 1, 450, 13), (33, 90, 0, 17), 7)])  # the 4-wave blocks
def test_chunk_window_attention(ops, lens, hist, pad):
    """The one-softmax chunk + exact window against the oracle's chunk, window history and LSE merge."""
    rng = np.random.default_rng(sum(lens) + pad)
    H, d, W, block = 16, 128, 32, 16
    lens, hist = np.array(lens, np.int64), np.array(hist, np.int64)
    R = len(lens)
    qsl = np.concatenate(([0], np.cumsum(lens))).astype(np.int32)
    T = int(qsl[-1]) + pad
    seq = (hist + lens).astype(np.int32)
    cols = int(-(-max(hist.max(), 1) // block))
    nb = R * cols + 3
    table = (1 + rng.permutation(nb - 1)[:R * cols]).reshape(R, cols).astype(np.int32)
    cache = random_bits(rng, (nb, H, block, 2 * d))
    q, k, v = (random_bits(rng, (T, H, d)) for _ in range(3))
    req, valid, ctx, _ = O.step_context(qsl, seq, T, W)
    invalid = ~valid
    scale = 1 / math.sqrt(d)
    o, lse = ops.chunk_window_attention(dev_bf16(q), dev_bf16(k), dev_bf16(v), dev_i32(qsl), dev_i32(seq),
                                        dev_bf16(cache), dev_i32(table), W, scale, 'hip')
    cf = bf16.to_f32(cache)
    o_c, l_c = O.chunk_attention(bf16.to_f32(q), bf16.to_f32(k), bf16.to_f32(v), qsl, invalid, scale)
    o_w, l_w = O.window_history(bf16.to_f32(q), cf[..., :d], cf[..., d:], table[req], ctx, W, scale)
    want_o, want_lse = O.merge_lse(o_c, l_c, o_w, l_w)
    assert o.shape == (T, H, d) and lse.shape == (H, T)
    assert_attention_close(host_f32(o), want_o, 'chunk+window o')
    assert_lse_close(host_f32(lse), want_lse)
    assert (host_f32(o)[invalid] == 0).all() and np.isneginf(host_f32(lse)[:, invalid]).all()


# ------------------------------------------------------------------------------------------------ merges

def test_merge_states_edge_cases(ops):
    rng = np.random.default_rng(10)
    T, H, D = 8, 16, 128
    oh, oc = random_bits(rng, (T, H, D)), random_bits(rng, (T, H, D))
    lh = (rng.standard_normal((H, T)) * 3).astype(np.float32)
    lc = (rng.standard_normal((H, T)) * 3).astype(np.float32)
    lh[:, 0] = -np.inf            # empty history -> chunk output
    lc[:, 1] = np.inf             # FA2 empty-key convention -> history output
    lh[:, 2] = lc[:, 2] = -np.inf  # both empty (padding row)
    invalid = np.zeros(T, bool)
    invalid[2] = invalid[7] = True
    out = ops.merge_states(dev_bf16(oh), torch.as_tensor(lh, device=CUDA), dev_bf16(oc),
                           torch.as_tensor(lc, device=CUDA), torch.as_tensor(invalid, device=CUDA), 'hip')
    want = O.merge_states(bf16.to_f32(oh), lh, bf16.to_f32(oc), lc, invalid)
    got = host_f32(out)
    assert_attention_close(got, want, 'merge')
    assert (got[2] == 0).all() and (got[7] == 0).all()
    np.testing.assert_array_equal(got[0], bf16.to_f32(oc)[0])
    np.testing.assert_array_equal(got[1], bf16.to_f32(oh)[1])


def test_merge_lse(ops):
    rng = np.random.default_rng(11)
    T, H, D = 6, 16, 128
    o1, o2 = random_bits(rng, (T, H, D)), random_bits(rng, (T, H, D))
    o1[0] = 0x7FC0                 # scratch NaN row of an empty side
    l1 = (rng.standard_normal((H, T)) * 2).astype(np.float32)
    l2 = (rng.standard_normal((H, T)) * 2).astype(np.float32)
    l1[:, 0] = -np.inf
    l1[:, 3] = l2[:, 3] = -np.inf
    out, lse = ops.merge_lse(dev_bf16(o1), torch.as_tensor(l1, device=CUDA), dev_bf16(o2), torch.as_tensor(l2, device=CUDA))
    want, want_lse = O.merge_lse(bf16.to_f32(o1), l1, bf16.to_f32(o2), l2)
    assert_attention_close(host_f32(out), want, 'merge_lse')
    assert_lse_close(host_f32(lse), want_lse)


def _plan_restated(ctx, cap, S, qsl=None):
    """The split plan's documented formula in plain Python (an independent restatement for the integer check): the
    chunk is the smallest one at or above max(ceil(max_tiles / S), ceil(2 * total_tiles / (T * S)), floor) that
    leaves at most T*S/2 items (or max_tiles), the floor 4 tiles below 768 tiles per step and 8 above (or
    max_tiles); the (row, chunk) items in row order, except that the rows of a request of 2..16
    tokens with equal slot counts list theirs chunk-major (chunk 0 of every row, then chunk 1, ...)."""
    tiles = [-(-min(int(c), cap) // 16) for c in ctx]
    T = len(ctx)
    chunk = max(1, -(-max(tiles) // S), -(-2 * sum(tiles) // (T * S)))
    chunk = max(chunk, min(max(tiles), 4 if sum(tiles) < 768 else 8))   # the floor: 4 tiles in small steps, else 8
    while chunk < max(tiles) and sum(-(-t // chunk) for t in tiles) > T * S // 2:
        chunk += 1
    used = [-(-t // chunk) for t in tiles]
    ni = T if S == 1 else -(-T * ((S + 1) // 2 + 1) // 8) * 8
    groups, r = [], 0                                        # runs of rows listed together
    bounds = [] if qsl is None else [(int(qsl[k]), int(qsl[k + 1])) for k in range(len(qsl) - 1)]
    for lo, hi in bounds:
        while r < lo:
            groups.append([r])
            r += 1
        if 2 <= hi - lo <= 16 and len({used[x] for x in range(lo, hi)}) == 1:
            groups.append(list(range(lo, hi)))
            r = hi
    groups += [[x] for x in range(r, T)]
    items = []
    for g in groups:
        for c in range(used[g[0]]):
            items += [(x, c) for x in g]
    rows, slots = [-1] * ni, [None] * ni
    q = -(-len(items) // 8)                                  # eight contiguous shares, one per XCD
    for i, (x, c) in enumerate(items):
        b = (i % q) * 8 + i // q
        rows[b], slots[b] = x, c
    return chunk, used, rows, slots


@pytest.mark.parametrize('T,S,grouped,hi', [(1, 2, False, 20000), (5, 7, False, 20000), (64, 16, False, 20000),
                                            (300, 32, False, 20000), (8, 1024, False, 20000), (700, 3, False, 20000),
                                            (60, 66, True, 20000), (300, 32, True, 20000),
                                            # few-tile steps: the 4-tile floor (below 768 tiles) and the 8-tile one
                                            (3, 34, False, 1100), (2, 66, False, 2200), (4, 130, False, 4400),
                                            (8, 128, False, 4400),
                                            # more rows than the plan kernel keeps in LDS: lengths read from memory
                                            (5000, 3, False, 20000)])
def test_split_plan_is_the_documented_balanced_list(ops, T, S, grouped, hi):
    rng = np.random.default_rng(T * 1000 + S)
    ctx = rng.integers(hi // 2 if hi < 20000 else 0, hi, T).astype(np.int32)
    ctx[::7] = 0                                            # rows without history
    qsl = None
    if grouped:   # requests of 1..20 tokens, most with one length per request (short chunks), two padding rows
        lens = rng.integers(1, 21, T)
        qsl = np.concatenate(([0], np.cumsum(lens)))
        qsl = qsl[qsl <= T - 2].astype(np.int32)
        for k in range(len(qsl) - 1):
            if k % 5:                                       # every fifth request keeps ragged lengths
                ctx[qsl[k]:qsl[k + 1]] = ctx[qsl[k]]
    cap = 16 * 1000                                         # rows past the table's reach are not read
    lib = ops._lib.load()
    n = lib.hla_s6_split_plan_ints(T, S)
    plan = torch.full((n,), -7, dtype=torch.int32, device='cuda')
    ctx_d = dev_i32(ctx)
    qsl_d = None if qsl is None else dev_i32(qsl)
    ops._lib.call('hla_s6_split_plan', ctx_d.data_ptr(), T, cap, S, None if qsl is None else qsl_d.data_ptr(),
                  0 if qsl is None else len(qsl) - 1, plan.data_ptr(), n, ops._lib.stream())
    got = plan.cpu().tolist()
    chunk, used, rows, slots = _plan_restated(ctx, cap, S, qsl)
    ni = len(rows)
    assert n == 1 + T + 2 * ni
    assert got[0] == chunk and got[1:1 + T] == used
    assert got[1 + T:1 + T + ni] == rows
    assert all(s is None or g == s for g, s in zip(got[1 + T + ni:], slots))
    assert max(used) <= S                                  # every row fits its slots
    tiles = [-(-min(int(c), cap) // 16) for c in ctx]
    assert all(u * chunk >= t > (u - 1) * chunk for u, t in zip(used, tiles) if t)
    assert sum(used) <= T * S // 2 or chunk == max(tiles)  # at most two items per CU at the policy's counts


@pytest.mark.parametrize('T,counts,grouped', [(64, (16, 32), False), (8, (128, 256), False), (32, (32, 64, 3), False),
                                               (60, (66, 130), True), (1, (34,), False)])
def test_split_plans_of_several_slot_counts_in_one_launch(ops, T, counts, grouped):
    """hla_s6_split_plans: every plan of the set equals hla_s6_split_plan's for its slot count (the widths of a
    step over the same lengths), with and without the request grouping of short chunks."""
    rng = np.random.default_rng(T + 7)
    ctx = rng.integers(1, 20000, T).astype(np.int32)
    qsl = None
    if grouped:
        lens = rng.integers(1, 5, T)
        qsl = np.concatenate(([0], np.cumsum(lens)))
        qsl = qsl[qsl <= T].astype(np.int32)
        for k in range(len(qsl) - 1):
            ctx[qsl[k]:qsl[k + 1]] = ctx[qsl[k]]
    ctx_d, qsl_d = dev_i32(ctx), None if qsl is None else dev_i32(qsl)
    cap = 16 * 1500
    plans = ops.split_plans(ctx_d, cap, counts, qsl_d)
    for S, plan in zip(counts, plans):
        want = ops.split_plan(ctx_d, cap, S, qsl_d).cpu().numpy()
        got = plan.cpu().numpy()
        ni = (len(want) - 1 - T) // 2
        rows = want[1 + T:1 + T + ni]
        assert (got[:1 + T + ni] == want[:1 + T + ni]).all(), S      # chunk, slot counts, item rows
        live = rows >= 0                                              # item slots (unused items leave theirs unset)
        assert (got[1 + T + ni:][live] == want[1 + T + ni:][live]).all(), S


def test_split_plans_reject_bad_sets(ops):
    ctx = torch.ones(4, dtype=torch.int32, device='cuda')
    plan = torch.empty(3, dtype=torch.int32, device='cuda')
    arr = lambda ct, *v: (ct * len(v))(*v)
    import ctypes
    with pytest.raises(ValueError, match='needs'):
        ops._lib.call('hla_s6_split_plans', ctx.data_ptr(), 4, 1024, 1, arr(ctypes.c_int32, 8), None, 0,
                      arr(ctypes.c_void_p, plan.data_ptr()), arr(ctypes.c_int64, plan.numel()), ops._lib.stream())
    with pytest.raises(ValueError, match='plan count'):
        ops._lib.call('hla_s6_split_plans', ctx.data_ptr(), 4, 1024, 5, arr(ctypes.c_int32, 8, 8, 8, 8, 8), None, 0,
                      arr(ctypes.c_void_p, *[plan.data_ptr()] * 5), arr(ctypes.c_int64, *[plan.numel()] * 5),
                      ops._lib.stream())


def test_split_plan_rejects_a_short_buffer(ops):
    plan = torch.empty(3, dtype=torch.int32, device='cuda')
    ctx = torch.ones(4, dtype=torch.int32, device='cuda')
    with pytest.raises(ValueError, match='need'):
        ops._lib.call('hla_s6_split_plan', ctx.data_ptr(), 4, 1024, 8, None, 0, plan.data_ptr(), plan.numel(),
                      ops._lib.stream())
