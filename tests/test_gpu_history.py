"""GPU parity of the paged latent-history kernel (split-KV, MFMA) against the fp32 oracle.

The grid follows the reference GPU test (hla/tests/test_s6_ops_gpu.py:43-57): widths, block sizes, split counts,
ctx pattern [5000, 1000, 17, 1, 0] and batch sizes 1 / 8 / 33, random block tables whose stale columns point at a
+inf-poisoned null page. Tolerance: max-abs 2e-2 and relative L2 5e-3 on o, 1e-3 on lse."""
import math

import numpy as np
import pytest
import torch

from oracle import bf16
from oracle import s6_oracle as O
from s6util import (NAN_BF16, assert_attention_close, assert_lse_close, dev_bf16, dev_i32, dev_i64, host_f32,
                    latent_cache_bits, random_bits, token_tables)

pytestmark = pytest.mark.gpu
SCALE = 1 / math.sqrt(128)


def run_history(ops, q_bits, cache_bits, table, ctx, splits, bt_rows=None):
    T, H, w = q_bits.shape
    q, cache = dev_bf16(q_bits), dev_bf16(cache_bits)
    ws = ops.S6Workspace(H, w, T * splits)
    o, lse = ops.history_attention_kv(q, cache[..., :w], cache[..., w:], dev_i32(table), dev_i32(ctx), SCALE, splits,
                                      ws, None, None, 'hip', bt_rows=None if bt_rows is None else dev_i64(bt_rows))
    return host_f32(o), host_f32(lse)


def oracle_history(q_bits, cache_bits, table, ctx):
    w = q_bits.shape[-1]
    cf = bf16.to_f32(cache_bits)
    return O.history_attention(bf16.to_f32(q_bits), cf[..., :w], cf[..., w:], table, ctx, SCALE)


def check(o, lse, want_o, want_lse, ctx):
    assert_attention_close(o, want_o)
    assert_lse_close(lse, want_lse)
    empty = np.asarray(ctx) == 0
    assert (o[empty] == 0).all() and np.isneginf(lse[:, empty]).all()


@pytest.mark.parametrize('width', [1024, 512, 256, 128])
@pytest.mark.parametrize('block', [16, 32])
@pytest.mark.parametrize('splits', [1, 4, 16])
def test_history_matches_oracle(ops, width, block, splits):
    rng = np.random.default_rng(width + block + splits)
    num_blocks = 1024 if block == 16 else 512
    cache = latent_cache_bits(rng, num_blocks, block, width)
    cols = -(-5000 // block)
    for batch in (1, 8, 33):
        print(f'case width={width} block={block} splits={splits} batch={batch}', flush=True)
        ctx = np.array(([5000, 1000, 17, 1, 0] * 7)[:batch], np.int32)
        table = token_tables(rng, ctx, block, num_blocks, cols)
        q = random_bits(rng, (batch, 16, width))
        o, lse = run_history(ops, q, cache, table, ctx, splits)
        check(o, lse, *oracle_history(q, cache, table, ctx), ctx)


@pytest.mark.parametrize('splits', [1, 7])
def test_history_nan_tails_and_page_ids_do_not_leak(ops, splits):
    """Rows past ctx inside a row's last page are NaN: they must not reach o or lse."""
    rng = np.random.default_rng(11)
    width, block, nb = 512, 16, 600
    ctx = np.array([1, 15, 16, 17, 33, 250, 1000, 31], np.int32)
    cache = latent_cache_bits(rng, nb, block, width)
    table = token_tables(rng, ctx, block, nb, 70, distinct=True)
    for t, n in enumerate(ctx):
        if n % block:
            cache[table[t, n // block], 0, n % block:] = NAN_BF16
    q = random_bits(rng, (len(ctx), 16, width))
    o, lse = run_history(ops, q, cache, table, ctx, splits)
    check(o, lse, *oracle_history(q, cache, table, ctx), ctx)   # the oracle reads rows < ctx only


def test_history_per_request_table_rows(ops):
    """bt_rows maps tokens onto a per-request table: same result as the gathered per-token table."""
    rng = np.random.default_rng(12)
    width, block, nb = 256, 16, 400
    req_ctx = np.array([700, 3, 0, 129], np.int32)
    table = token_tables(rng, req_ctx, block, nb, 50)
    cache = latent_cache_bits(rng, nb, block, width)
    rows = np.array([0, 0, 1, 3, 3, 3, 2], np.int64)
    ctx = req_ctx[rows]
    q = random_bits(rng, (len(rows), 16, width))
    o, lse = run_history(ops, q, cache, table, ctx, 4, bt_rows=rows)
    o2, lse2 = run_history(ops, q, cache, table[rows], ctx, 4)
    np.testing.assert_array_equal(o, o2)
    np.testing.assert_array_equal(lse, lse2)
    check(o, lse, *oracle_history(q, cache, table[rows], ctx), ctx)


def test_history_contiguous_rows_of_the_hf_engine(ops):
    """The HF engine's packed rows [B, N, 1536] = [K 512 | V 512 | K1 256 | V1 256] read with identity paging."""
    rng = np.random.default_rng(13)
    B, N = 3, 1024
    rows = random_bits(rng, (B, N, 1536))
    ctx = np.array([1024, 700, 9], np.int32)
    packed = dev_bf16(rows)
    pages = packed.view(B * N // 16, 1, 16, 1536)
    table = (np.arange(B)[:, None] * (N // 16) + np.arange(N // 16)[None]).astype(np.int32)
    for (k0, w) in ((0, 512), (1024, 256)):
        q = random_bits(rng, (B, 16, w))
        o, lse = ops.history_attention_kv(dev_bf16(q), pages[..., k0:k0 + w], pages[..., k0 + w:k0 + 2 * w],
                                          dev_i32(table), dev_i32(ctx), SCALE, 4, ops.S6Workspace(16, w, B * 4), None,
                                          None, 'hip')
        rf = bf16.to_f32(rows).reshape(B * N // 16, 1, 16, 1536)
        want_o, want_lse = O.history_attention(bf16.to_f32(q), rf[..., k0:k0 + w], rf[..., k0 + w:k0 + 2 * w], table,
                                               ctx, SCALE)
        check(host_f32(o), host_f32(lse), want_o, want_lse, ctx)


def test_split_counts_agree(ops):
    """The split partition changes only the summation order: every split count gives the same answer."""
    rng = np.random.default_rng(14)
    width, block, nb = 512, 16, 2048
    ctx = rng.integers(1024, 8192, 12).astype(np.int32)
    cache = latent_cache_bits(rng, nb, block, width)
    table = token_tables(rng, ctx, block, nb, 512)
    q = random_bits(rng, (len(ctx), 16, width), 1 / math.sqrt(512))
    ref = run_history(ops, q, cache, table, ctx, 1)
    for splits in (2, 16, 64, 200):
        o, lse = run_history(ops, q, cache, table, ctx, splits)
        assert_attention_close(o, ref[0], f'splits={splits}')
        assert_lse_close(lse, ref[1])


@pytest.mark.parametrize('width', [512, 256])
@pytest.mark.parametrize('splits', [1, 3, 8])
def test_two_stage_history_is_bitwise_the_op(ops, width, splits):
    """history_partials + history_reduce (the reference's stage-1 / stage-2 launches) give exactly the bytes of
    history_attention_kv, including empty rows, and match the oracle."""
    rng = np.random.default_rng(7 * width + splits)
    block, num_blocks = 16, 600
    cache_bits = latent_cache_bits(rng, num_blocks, block, width)
    ctx = np.array([4100, 999, 16, 1, 0, 2500], np.int32)
    table = token_tables(rng, ctx, block, num_blocks, -(-4100 // block))
    q_bits = random_bits(rng, (ctx.shape[0], 16, width))
    q, cache = dev_bf16(q_bits), dev_bf16(cache_bits)
    k, v, bt, c = cache[..., :width], cache[..., width:], dev_i32(table), dev_i32(ctx)
    ws = ops.S6Workspace(16, width, ctx.shape[0] * splits)
    o_ref, lse_ref = ops.history_attention_kv(q, k, v, bt, c, SCALE, splits, ws, None, None, 'hip')
    o_ref, lse_ref = o_ref.clone(), lse_ref.clone()
    part = ops.history_partials(q, k, v, bt, c, SCALE, splits, ws)
    assert tuple(part.shape) == (ctx.shape[0], 16, splits, width + 1)
    o, lse = ops.history_reduce(part)
    assert torch.equal(o.view(torch.int16), o_ref.view(torch.int16))
    assert torch.equal(lse, lse_ref)
    if splits > 1:  # the same work split through a precomputed plan
        plan = ops.split_plan(c, table.shape[1] * block, splits)
        o2, lse2 = ops.history_reduce(ops.history_partials(q, k, v, bt, c, SCALE, splits, ws, plan=plan))
        assert torch.equal(o2.view(torch.int16), o_ref.view(torch.int16)) and torch.equal(lse2, lse_ref)
    check(host_f32(o), host_f32(lse), *oracle_history(q_bits, cache_bits, table, ctx), ctx)
    with pytest.raises(RuntimeError, match='S6Workspace'):
        ops.history_partials(q, k, v, bt, c, SCALE, splits, None)


@pytest.mark.parametrize('width', [1024, 512, 256])
@pytest.mark.parametrize('splits', [1, 5])
@pytest.mark.parametrize('group', [1, 2, 4])
def test_grouped_history_matches_oracle(ops, width, splits, group):
    """Chunked-prefill shape: requests of 5, 3, 1, 8 and 2 query rows whose rows share the request's table row.
    Request 0 has one ctx for every row (vLLM prefill), request 1 a causal ctx per row (K-hop), request 2 no
    history, request 3 decreasing ctx, request 4 a short one. Groups straddle requests."""
    rng = np.random.default_rng(100 * width + 10 * splits + group)
    block, num_blocks = 16, 1200
    lens = [5, 3, 1, 8, 2]
    req = np.repeat(np.arange(len(lens)), lens)
    ctx = np.concatenate([np.full(5, 3000), 700 + np.arange(3), [0], 1200 - 37 * np.arange(8), [40, 41]])
    ctx = ctx.astype(np.int32)
    per_req = np.array([ctx[req == r].max() for r in range(len(lens))])
    table = token_tables(rng, per_req, block, num_blocks, -(-3000 // block))
    cache_bits = latent_cache_bits(rng, num_blocks, block, width)
    q_bits = random_bits(rng, (len(ctx), 16, width))
    q, cache = dev_bf16(q_bits), dev_bf16(cache_bits)
    ws = ops.S6Workspace(16, width, len(ctx) * splits)
    o, lse = ops.history_attention_kv(q, cache[..., :width], cache[..., width:], dev_i32(table), dev_i32(ctx), SCALE,
                                      splits, ws, None, None, 'hip', bt_rows=dev_i64(req), tokens_per_group=group,
                                      shared_rows=True)
    o, lse = host_f32(o), host_f32(lse)
    check(o, lse, *oracle_history(q_bits, cache_bits, table[req], ctx), ctx)
    o1, lse1 = run_history(ops, q_bits, cache_bits, table, ctx, splits, bt_rows=req)
    assert_attention_close(o, o1, 'grouped vs one token per workgroup')
    assert_lse_close(lse, lse1)


@pytest.mark.parametrize('width,T', [(512, 40), (256, 40), (512, 80)])
def test_grouped_partials_and_split_epilogue(ops, layer, width, T):
    """hla_s6_history_partials_grouped + hla_s6_history_reduce give the grouped history op's result (the reduce
    reads every slot, the op only the used ones: the same terms, summed in groups that can differ); the split
    epilogue over those partials equals merge_states(absorb_out(o_hist, B), lse_hist, o_win, lse_win, invalid) to the
    attention tolerance (its B_t product sums in another order), with invalid rows zeroed; bad arguments raise
    before any launch."""
    rng = np.random.default_rng(width + T)
    block, num_blocks, splits = 16, 500, 5
    lens = [T // 2, T // 4, T - T // 2 - T // 4]
    req = np.repeat(np.arange(3), lens)
    ctx = np.concatenate([np.full(lens[0], 2000), np.full(lens[1], 0), 300 + np.arange(lens[2])]).astype(np.int32)
    per_req = np.array([max(1, ctx[req == r].max()) for r in range(3)])
    table = token_tables(rng, per_req, block, num_blocks, -(-2000 // block))
    cache_bits = latent_cache_bits(rng, num_blocks, block, width)
    q = dev_bf16(random_bits(rng, (T, 16, width)))
    cache = dev_bf16(cache_bits)
    k, v, bt, c, rows = cache[..., :width], cache[..., width:], dev_i32(table), dev_i32(ctx), dev_i64(req)
    ws = ops.S6Workspace(16, width, T * splits)
    o_ref, lse_ref = ops.history_attention_kv(q, k, v, bt, c, SCALE, splits, ws, None, None, 'hip', bt_rows=rows,
                                              tokens_per_group=4, shared_rows=True)
    o_ref, lse_ref = o_ref.clone(), lse_ref.clone()
    part = ops.history_partials_grouped(q, k, v, bt, c, SCALE, splits, ws, bt_rows=rows, tokens_per_group=4)
    o, lse = ops.history_reduce(part)
    assert_attention_close(host_f32(o), host_f32(o_ref), 'grouped partials + reduce vs the grouped op')
    assert_lse_close(host_f32(lse), host_f32(lse_ref))
    B = dev_bf16(random_bits(rng, (16, width, 128), 1 / math.sqrt(2048)))
    o_win = dev_bf16(random_bits(rng, (T, 16, 128)))
    lse_win = torch.tensor(rng.standard_normal((16, T)).astype(np.float32), device='cuda')
    lse_win[:, 1] = -math.inf                       # a row whose chunk part is empty
    invalid = torch.zeros(T, dtype=torch.bool, device='cuda')
    invalid[-1] = True
    got = ops.split_epilogue(part, B, o_win, lse_win, invalid)
    want = ops.merge_states(layer.absorb_out(o_ref, B), lse_ref, o_win, lse_win, invalid, 'hip')
    assert_attention_close(host_f32(got), host_f32(want), 'split epilogue vs op sequence')
    assert (host_f32(got)[-1] == 0).all()
    with pytest.raises(ValueError, match='num_kv_splits'):
        ops.split_epilogue(ws.attn_logits(T, 16, 1, width, q.device), B, o_win, lse_win, invalid)
    with pytest.raises(ValueError, match='B must be'):
        ops.split_epilogue(part, B[:, :64], o_win, lse_win, invalid)
    with pytest.raises(ValueError, match='group'):
        ops.history_partials_grouped(q, k, v, bt, c, SCALE, splits, ws, bt_rows=rows, tokens_per_group=3)


@pytest.mark.parametrize('width,group', [(512, 4), (256, 4), (1024, 2)])
def test_grouped_history_fills_every_slot(ops, width, group):
    """The multi-token kernels run one workgroup per (token group, slot): every slot of the longest row holds
    work (a finite partial lse in the workspace), shorter rows a prefix of the slots, and the result matches the
    oracle."""
    rng = np.random.default_rng(width + group)
    block, num_blocks, splits = 16, 400, 6
    lens = [8, 4]
    req = np.repeat(np.arange(len(lens)), lens)
    ctx = np.concatenate([np.full(8, 3000), np.full(4, 1000)]).astype(np.int32)
    per_req = np.array([ctx[req == r].max() for r in range(len(lens))])
    table = token_tables(rng, per_req, block, num_blocks, -(-3000 // block))
    cache_bits = latent_cache_bits(rng, num_blocks, block, width)
    q_bits = random_bits(rng, (len(ctx), 16, width))
    q, cache = dev_bf16(q_bits), dev_bf16(cache_bits)
    ws = ops.S6Workspace(16, width, len(ctx) * splits)
    o, lse = ops.history_attention_kv(q, cache[..., :width], cache[..., width:], dev_i32(table), dev_i32(ctx), SCALE,
                                      splits, ws, None, None, 'hip', bt_rows=dev_i64(req), tokens_per_group=group,
                                      shared_rows=True)
    T = len(ctx)
    flat = ws.ensure(q.device)
    part_lse = host_f32(flat[T * splits * 16 * width:T * splits * 16 * (width + 1)]).reshape(T, splits, 16)
    tiles = -(-3000 // 16)
    chunk = -(-tiles // splits)
    for t in range(T):
        used = -(-(-(-int(ctx[t]) // 16)) // chunk)
        assert np.isfinite(part_lse[t, :used]).all(), (t, used)
        assert np.isneginf(part_lse[t, used:]).all(), (t, used)
    assert used < splits and np.isfinite(part_lse[0]).all()
    check(host_f32(o), host_f32(lse), *oracle_history(q_bits, cache_bits, table[req], ctx), ctx)


@pytest.mark.parametrize('width,block,long_ctx,splits', [(512, 16, 33000, 1),  # more pages than the LDS list holds
                                                         (512, 16, 33000, 3),
                                                         (512, 32, 5003, 1),   # pages of 32 rows
                                                         (512, 32, 5003, 4),
                                                         (256, 16, 33000, 1),
                                                         (256, 32, 5003, 4)])
def test_grouped_history_page_geometry(ops, width, block, long_ctx, splits):
    """Four-token groups over long rows and other page sizes: request 0 (11 rows) sees ``long_ctx`` rows, request 1
    (6 rows) ragged lengths ending inside a tile, request 2 (3 rows) rows of 1-40."""
    rng = np.random.default_rng(width + block + long_ctx + splits)
    num_blocks = -(-long_ctx // block) + 64
    lens = [11, 6, 3]
    req = np.repeat(np.arange(len(lens)), lens)
    ctx = np.concatenate([np.full(11, long_ctx), 517 + 5 * np.arange(6), [1, 17, 40]]).astype(np.int32)
    per_req = np.array([ctx[req == r].max() for r in range(len(lens))])
    cols = -(-long_ctx // block)
    table = np.zeros((len(lens), cols), np.int32)
    for r, n in enumerate(per_req):  # request 0 walks the whole pool in a random order, the others share pages
        need = -(-int(n) // block)
        table[r, :need] = rng.permutation(np.arange(1, num_blocks))[:need] if r == 0 else \
            rng.integers(1, num_blocks, need)
    cache_bits = latent_cache_bits(rng, num_blocks, block, width)
    q_bits = random_bits(rng, (len(ctx), 16, width))
    q, cache = dev_bf16(q_bits), dev_bf16(cache_bits)
    ws = ops.S6Workspace(16, width, len(ctx) * splits)
    o, lse = ops.history_attention_kv(q, cache[..., :width], cache[..., width:], dev_i32(table), dev_i32(ctx), SCALE,
                                      splits, ws, None, None, 'hip', bt_rows=dev_i64(req), tokens_per_group=4,
                                      shared_rows=True)
    check(host_f32(o), host_f32(lse), *oracle_history(q_bits, cache_bits, table[req], ctx), ctx)


@pytest.mark.parametrize('splits', [1, 5])
def test_grouped_history_scores_that_outgrow_the_first_tile(ops, splits):
    """Rows whose scores rise far above their first tile's (the online softmax raises its maximum and rescales the
    accumulators many times): requests 0 and 2 of the 512-wide multi-query kernel have keys from position 100 on
    scaled by 5 (their row maxima rise by 2^40 and more over the first 32 keys'), 1 and 3 do not; the first
    workgroup holds two passes (requests 0 and 1). Against the oracle and the one-token-per-workgroup kernel."""
    width, block, num_blocks = 512, 16, 400
    rng = np.random.default_rng(512 + splits)
    lens = [3, 6, 7, 5]
    req = np.repeat(np.arange(len(lens)), lens)
    ctx = np.concatenate([np.full(3, 600), 500 - 7 * np.arange(6), 640 + np.arange(7), np.full(5, 90)])
    ctx = ctx.astype(np.int32)
    per_req = np.array([ctx[req == r].max() for r in range(len(lens))])
    table = token_tables(rng, per_req, block, num_blocks, -(-700 // block), distinct=True)
    cache = bf16.to_f32(latent_cache_bits(rng, num_blocks, block, width))
    for r in (0, 2):
        for pos in range(100, int(per_req[r])):
            cache[table[r, pos // block], 0, pos % block, :width] *= 5
    cache_bits = bf16.from_f32(cache)
    q_bits = random_bits(rng, (len(ctx), 16, width))
    kf, qf = bf16.to_f32(cache_bits)[:, 0, :, :width], bf16.to_f32(q_bits)
    growth = []  # per token: the largest rise of a row's maximum (log2 units) over its first 32 keys' maximum
    for t, n in enumerate(ctx):
        pos = np.arange(n)
        sc = qf[t] @ kf[table[req[t], pos // block], pos % block].T * (SCALE * math.log2(math.e))
        growth.append((sc.max(-1) - sc[:, :32].max(-1)).max())
    growth = np.array(growth)
    assert (growth[req == 0] > 24).all() and (growth[req == 1] < 24).all()
    q, dcache = dev_bf16(q_bits), dev_bf16(cache_bits)
    ws = ops.S6Workspace(16, width, len(ctx) * splits)
    o, lse = ops.history_attention_kv(q, dcache[..., :width], dcache[..., width:], dev_i32(table), dev_i32(ctx),
                                      SCALE, splits, ws, None, None, 'hip', bt_rows=dev_i64(req), tokens_per_group=4,
                                      shared_rows=True)
    o, lse = host_f32(o), host_f32(lse)
    check(o, lse, *oracle_history(q_bits, cache_bits, table[req], ctx), ctx)
    o1, lse1 = run_history(ops, q_bits, cache_bits, table, ctx, splits, bt_rows=req)
    assert_attention_close(o, o1, 'grouped vs one token per workgroup')
    assert_lse_close(lse, lse1)


def test_grouped_history_width_256_both_wave_forms(ops):
    """At width 256 the multi-query kernel takes two tokens per wave when its grid has more workgroups than the
    device has CUs, else one: a step of 8 x (CUs + 8) tokens (the first form) and its first request's 16 tokens
    alone (the second form) both match the oracle on those tokens (the two forms may round the row sum's update
    differently, so they agree to the attention tolerance, not bit for bit)."""
    width, block, n_ctx = 256, 16, 100
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    T = 8 * (cus + 8)
    rng = np.random.default_rng(256)
    req = np.arange(T) // 16
    R = int(req[-1]) + 1
    num_blocks = 64
    table = rng.integers(1, num_blocks, (R, -(-n_ctx // block))).astype(np.int32)
    ctx = (n_ctx - (np.arange(T) % 16)).astype(np.int32)
    cache_bits = latent_cache_bits(rng, num_blocks, block, width)
    q_bits = random_bits(rng, (T, 16, width))
    cache = dev_bf16(cache_bits)
    outs = []
    for n in (T, 16):
        q = dev_bf16(q_bits[:n])
        o, lse = ops.history_attention_kv(q, cache[..., :width], cache[..., width:], dev_i32(table), dev_i32(ctx[:n]),
                                          SCALE, 1, None, None, None, 'hip', bt_rows=dev_i64(req[:n]),
                                          tokens_per_group=4, shared_rows=True)
        outs.append((o[:16].clone(), lse[:, :16].clone()))
    want = oracle_history(q_bits[:16], cache_bits, table[req[:16]], ctx[:16])
    for o, lse in outs:
        check(host_f32(o), host_f32(lse), *want, ctx[:16])
    assert_attention_close(host_f32(outs[0][0]), host_f32(outs[1][0]), 'two-token vs one-token waves')


def test_grouped_history_rejects_unsupported_group(ops):
    q = torch.zeros(2, 16, 512, dtype=torch.bfloat16, device='cuda')
    cache = torch.zeros(4, 1, 16, 1024, dtype=torch.bfloat16, device='cuda')
    table = torch.zeros(2, 1, dtype=torch.int32, device='cuda')
    ctx = torch.ones(2, dtype=torch.int32, device='cuda')
    with pytest.raises(ValueError, match='group'):
        ops.history_attention_kv(q, cache[..., :512], cache[..., 512:], table, ctx, SCALE, 1, None, None, None, 'hip',
                                 tokens_per_group=3)
