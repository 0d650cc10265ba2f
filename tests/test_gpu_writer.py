"""The writer kernel (``hla_s6_write_rows``): candidate projection + register accumulation + fused row commit,
against the numpy oracle (``LatentLayer.write_step`` / ``write1``, ``committed_row``; hla/latent/register.py:45-61,
hla/vllm_latent/s6_layer.py:124-147) and against the unfused composition of the same ops.

Bars: the projection is floating point (an fp32-accumulated GEMM rounded to bf16, so a sum whose fp32 value lies
next to a bf16 rounding boundary may round the other way): every element within one bf16 rounding step of the
float64 oracle (two for an accumulated register) and at least 99 % of elements bit-identical. Everything after the
projection (accumulate, RoPE, slot-mapped store) is checked bit-exactly: with a permutation weight the projection
is exact, and the fused commit must equal write_rows -> committed_row -> store_rows bit for bit.
"""
import importlib
import types

import numpy as np
import pytest
import torch

from oracle import bf16
from oracle import s6_oracle as O
from s6util import dev_bf16, dev_i32, dev_i64, host_f32, random_bits

pytestmark = pytest.mark.gpu

layer = importlib.import_module('hybrid-latent-attention_amd.s6_layer')
ops = importlib.import_module('hybrid-latent-attention_amd.s6_ops')

HIDDEN, HEAD_DIM, BLOCK = 2048, 128, 16


def writer_layer(rng, rank=512, rank1=256, loops=4, hidden=HIDDEN, weights=None):
    """A LatentLayer-shaped writer: ``cand1`` and ``cand_s[l]`` carry nn.Linear-layout weights [2w, hidden]."""
    if weights is None:
        weights = {'cand1': random_bits(rng, (2 * rank1, hidden), hidden ** -0.5),
                   'cand_s': [random_bits(rng, (2 * rank, hidden), hidden ** -0.5) for _ in range(loops - 1)]}
    sl = types.SimpleNamespace(rank=rank, rank_v=rank, rank1=rank1, loops=loops, head_dim=HEAD_DIM)
    sl.cand1 = types.SimpleNamespace(weight=dev_bf16(weights['cand1']))
    sl.cand_s = [types.SimpleNamespace(weight=dev_bf16(w)) for w in weights['cand_s']]
    return sl, weights


def assert_projection_close(got, want, update, what, steps=1, magnitude=None):
    """|got - want| <= steps bf16 rounding steps of the larger of |want| and |update|, plus twice the worst-case
    fp32 summation error ``K * 2^-24 * magnitude`` (``magnitude`` = |h| @ |W|^T, which matters where the sum
    cancels to near zero); >= 99 % bit-identical."""
    got, want, update = (np.asarray(x, np.float32) for x in (got, want, update))
    assert got.shape == want.shape, what
    assert np.isfinite(got).all(), f'{what}: non-finite'
    bound = steps * 2.0 ** -7 * np.maximum(np.abs(want), np.abs(update)) + 1e-30
    if magnitude is not None:
        bound = bound + 2 * HIDDEN * 2.0 ** -24 * magnitude
    err = np.abs(got - want)
    assert (err <= bound).all(), f'{what}: {int((err > bound).sum())} elements beyond {steps} bf16 step(s)'
    same = float((got == want).mean())
    assert same >= 0.99, f'{what}: only {same:.4f} of elements bit-identical'


@pytest.mark.parametrize('T', [1, 5, 64, 128, 130, 600])
@pytest.mark.parametrize('loop', [0, 1, 2])
def test_write_rows_matches_the_oracle(T, loop):
    rng = np.random.default_rng(100 + T + loop)
    sl, wts = writer_layer(rng)
    h = [random_bits(rng, (T, HIDDEN)) for _ in range(3)]
    state = None
    reg = None
    for l in range(loop + 1):
        state = layer.write_rows(sl, l, dev_bf16(h[l]), state)
        w = wts['cand1'] if l == 0 else wts['cand_s'][l - 1]
        prev = None if l <= 1 else reg
        upd = O.write_step(bf16.to_f32(h[l]), bf16.to_f32(w))
        want = O.write_step(bf16.to_f32(h[l]), bf16.to_f32(w), prev)
        got = state.first if l == 0 else state.reg
        assert got.shape == (T, 2 * (sl.rank1 if l == 0 else sl.rank)) and got.dtype == torch.bfloat16
        assert (state.reg is None) == (l == 0) and (state.first is None) == (l != 0)
        g = host_f32(got)
        mag = np.abs(bf16.to_f32(h[l])).astype(np.float64) @ np.abs(bf16.to_f32(w)).astype(np.float64).T
        assert_projection_close(g, want, upd, f'loop {l}', steps=1 if prev is None else 2, magnitude=mag)
        if l >= 1:
            reg = g                               # the next loop accumulates onto the kernel's own register


@pytest.mark.parametrize('width', [256, 512])
def test_permutation_weight_makes_the_writer_exact(width):
    """With one-hot rows the projection selects columns of h exactly: register, accumulation, RoPE and store are
    then checked bit-exactly against the oracle (column mapping, operand orientation, rotation pairs, slots)."""
    rng = np.random.default_rng(7 + width)
    T, num_blocks, max_pos = 70, 40, 4096
    perm = rng.permutation(HIDDEN)[:2 * width]
    W = np.zeros((2 * width, HIDDEN), np.uint16)
    W[np.arange(2 * width), perm] = 0x3F80                            # 1.0
    h = random_bits(rng, (T, HIDDEN))
    prev = random_bits(rng, (T, 2 * width))
    positions = rng.integers(0, max_pos, T)
    slots = rng.permutation(num_blocks * BLOCK)[:T].astype(np.int64)
    slots[[3, 11, 69]] = -1                                           # padding tokens are skipped
    table = O.latent_rope_table(max_pos, O.latent_inv_freq(HEAD_DIM, 1e6), width)
    table_bits = bf16.from_f32(table)
    cache_bits = random_bits(rng, (num_blocks, 1, BLOCK, 2 * width))

    reg_d = torch.empty(T, 2 * width, dtype=torch.bfloat16, device='cuda')
    cache_d = dev_bf16(cache_bits)
    layer._write(dev_bf16(h), dev_bf16(W), width, dev_bf16(prev), reg_d, dev_i64(slots), dev_i64(positions),
                 dev_bf16(table_bits), cache_d)
    want_reg = bf16.round_bf16(bf16.to_f32(prev) + bf16.to_f32(h)[:, perm])
    assert (host_f32(reg_d) == want_reg).all()
    key, val = O.committed_row(want_reg, width, positions, bf16.to_f32(table_bits))
    want_cache = O.store_rows(bf16.to_f32(cache_bits).reshape(-1, 2 * width), slots, key, val)
    assert (host_f32(cache_d).reshape(-1, 2 * width) == want_cache).all()


@pytest.mark.parametrize('T', [3, 64, 97, 700])
def test_fused_commit_equals_write_then_commit_then_store(T):
    """``write_commit`` at loop 0 and the last loop stores exactly what ``write_rows`` -> ``committed_row`` ->
    ``store_rows`` store (the reference's sequence in ouro_latent.forward), padding tokens included."""
    rng = np.random.default_rng(50 + T)
    sl, _ = writer_layer(rng)
    R = max(1, T // 2)
    lens = np.ones(R, np.int64)
    lens[-1] = T - (R - 1) - (1 if T > 2 else 0)                      # one padding token when T > 2
    qsl = np.concatenate(([0], np.cumsum(lens))).astype(np.int32)
    seq = rng.integers(20, 300, R).astype(np.int32)
    seq = np.maximum(seq, lens.astype(np.int32))
    positions = np.concatenate([np.arange(s - n, s) for s, n in zip(seq, lens)] + [np.zeros(T - qsl[-1], np.int64)])
    cols = int(-(-seq.max() // BLOCK))
    num_blocks = 2 + R * cols
    table = (1 + rng.permutation(num_blocks - 1)[:R * cols]).reshape(R, cols).astype(np.int32)
    max_pos = 1024
    inv = O.latent_inv_freq(HEAD_DIM, 1e6)
    tables = {w: dev_bf16(bf16.from_f32(O.latent_rope_table(max_pos, inv, w))) for w in (256, 512)}
    ctx = layer.StepContext(dev_i64(positions), dev_i32(qsl), dev_i32(seq), int(lens.max()), T, tables, 1.0,
                            ops.HIP_BACKENDS)
    hs = [dev_bf16(random_bits(rng, (T, HIDDEN))) for _ in range(sl.loops)]
    caches = {w: dev_bf16(random_bits(rng, (num_blocks, 1, BLOCK, 2 * w))) for w in (256, 512)}
    fused = {w: c.clone() for w, c in caches.items()}
    orig = {w: c.clone() for w, c in caches.items()}
    tab = dev_i32(table)

    state = fstate = None
    for loop in range(sl.loops):
        state = layer.write_rows(sl, loop, hs[loop], state)
        fstate = layer.write_commit(sl, loop, hs[loop], fstate, ctx, fused[256 if loop == 0 else 512], tab)
        if 0 < loop < sl.loops - 1:
            assert torch.equal(fstate.reg, state.reg)
        row = layer.committed_row(sl, loop, state, ctx)
        if row is not None:
            w = row[0].shape[1]
            layer.store_rows(row[0], row[1], layer.slot_mapping(ctx, tab, BLOCK), caches[w])
    torch.cuda.synchronize()
    for w in (256, 512):
        assert torch.equal(fused[w], caches[w]), f'width {w}: fused commit differs from the composed ops'
    # only the valid tokens' slots changed (closed form of the slot, hla/tests/test_s6_serving.py:54)
    req = np.searchsorted(qsl[1:], np.arange(T), side='right')
    n_valid = int(qsl[-1])
    slots = table[req[:n_valid], positions[:n_valid] // BLOCK] * BLOCK + positions[:n_valid] % BLOCK
    for w in (256, 512):
        rows_changed = (host_f32(fused[w]) != host_f32(orig[w])).reshape(-1, 2 * w).any(-1)
        assert set(np.flatnonzero(rows_changed).tolist()) <= set(slots.tolist())


def test_writer_rejects_unsupported_shapes():
    rng = np.random.default_rng(3)
    sl, _ = writer_layer(rng, hidden=640)
    h = dev_bf16(random_bits(rng, (4, 640)))
    with pytest.raises(ValueError, match='multiple of 512'):
        layer.write_rows(sl, 1, h)
    sl, _ = writer_layer(rng)
    with pytest.raises(ValueError, match='inputs'):
        layer.write_rows(sl, 1, dev_bf16(random_bits(rng, (4, 1024))))
    sl.rank_v = 256
    with pytest.raises(ValueError, match='rank_v'):
        layer.write_rows(sl, 1, dev_bf16(random_bits(rng, (4, HIDDEN))))
