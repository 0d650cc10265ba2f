"""Pins of the floating-point oracle functions: independent float64 per-token loops on tiny inputs, the
joint-softmax identity of the merges, closed forms of RoPE and the GEMMs, and planted mistakes that each pin
must catch. CPU only."""
import math

import numpy as np
import pytest

from oracle import bf16
from oracle import s6_oracle as O

INF = np.inf


def _softmax64(scores, values):
    scores = np.asarray(scores, np.float64)
    m = scores.max()
    p = np.exp(scores - m)
    return (p / p.sum()) @ np.asarray(values, np.float64), m + math.log(p.sum())


# ---------------------------------------------------------------------------------------------- history

def paged_setup(block, width, heads, kvh=1, num_blocks=64, ctx=(0, 1, 17, 40, 5, 0), seed=0):
    rng = np.random.default_rng(seed)
    cache = rng.standard_normal((num_blocks, kvh, block, 2 * width)).astype(np.float32)
    cache[0] = INF                           # null block: any unmasked read of it is loud
    q = rng.standard_normal((len(ctx), heads, width)).astype(np.float32)
    table = rng.integers(1, num_blocks, (len(ctx), 12)).astype(np.int32)
    ctx = np.array(ctx, np.int32)
    needed = (ctx + block - 1) // block
    table[np.arange(12)[None] >= needed[:, None]] = 0   # stale columns point at the poisoned block
    return q, cache, table, ctx


def check_history(o, lse, q, cache, table, ctx, scale, tol=1e-5):
    T, H, w = q.shape
    kvh, block = cache.shape[1], cache.shape[2]
    group = H // kvh
    assert o.shape == (T, H, w) and lse.shape == (H, T)
    for t, n in enumerate(ctx.tolist()):
        if n == 0:
            assert (o[t] == 0).all() and (lse[:, t] == -INF).all()
            continue
        for h in range(H):
            g = h // group
            rows = np.stack([cache[int(table[t, j // block]), g, j % block] for j in range(n)]).astype(np.float64)
            scores = rows[:, :w] @ q[t, h].astype(np.float64) * scale
            out, l = _softmax64(scores, rows[:, w:])
            np.testing.assert_allclose(lse[h, t], l, rtol=tol, atol=tol)
            np.testing.assert_allclose(o[t, h], out, rtol=tol, atol=tol)


@pytest.mark.parametrize('block', [4, 8, 16])
@pytest.mark.parametrize('heads,kvh', [(2, 1), (4, 2), (16, 1)])
def test_history_matches_explicit_softmax(block, heads, kvh):
    width = 8
    q, cache, table, ctx = paged_setup(block, width, heads, kvh)
    scale = 1 / math.sqrt(width)
    o, lse = O.history_attention(q, cache[..., :width], cache[..., width:], table, ctx, scale)
    assert np.isfinite(o).all() and not np.isnan(lse).any()
    check_history(o, lse, q, cache, table, ctx, scale)


# ---------------------------------------------------------------------------------------------- chunk

def test_chunk_is_block_diagonal_causal():
    heads, dim = 2, 8
    qsl, T = np.array([0, 3, 4, 6, 6], np.int32), 8     # prefill 3, decode 1, prefill 2, padded request, 2 padding tokens
    rng = np.random.default_rng(2)
    q, k, v = rng.standard_normal((3, T, heads, dim)).astype(np.float32)
    invalid = np.arange(T) >= 6
    o, lse = O.chunk_attention(q, k, v, qsl, invalid, 1 / math.sqrt(dim))
    assert (o[6:] == 0).all() and (lse[:, 6:] == -INF).all()
    for r in range(3):
        s, e = qsl[r], qsl[r + 1]
        for i in range(s, e):
            for h in range(heads):
                sc = k[s:i + 1, h].astype(np.float64) @ q[i, h].astype(np.float64) / math.sqrt(dim)
                out, l = _softmax64(sc, v[s:i + 1, h])
                np.testing.assert_allclose(lse[h, i], l, rtol=1e-5, atol=1e-6)
                np.testing.assert_allclose(o[i, h], out, rtol=1e-5, atol=1e-6)


# ---------------------------------------------------------------------------------------------- merges

def partial(scores, values):
    T, H, _ = scores.shape
    o = np.zeros((T, H, values.shape[-1]))
    lse = np.full((H, T), -INF)
    for t in range(T):
        for h in range(H):
            if np.isfinite(scores[t, h]).any():
                o[t, h], lse[h, t] = _softmax64(scores[t, h], values[t])
    return o, lse


def joint(s1, v1, s2, v2):
    return partial(np.concatenate((s1, s2), -1), np.concatenate((v1, v2), 1))


def test_merge_states_is_joint_softmax():
    T, H, D, n1, n2 = 6, 2, 8, 5, 3
    rng = np.random.default_rng(3)
    s1, s2 = rng.standard_normal((T, H, n1)) * 3, rng.standard_normal((T, H, n2)) * 3
    v1, v2 = rng.standard_normal((T, n1, D)), rng.standard_normal((T, n2, D))
    s1[1] = -INF
    s2[2] = -INF
    s1[3] = s2[3] = -INF
    o1, l1 = partial(s1, v1)
    o2, l2 = partial(s2, v2)
    invalid = np.array([0, 0, 0, 0, 0, 1], bool)
    out = O.merge_states(o1, l1, o2, l2, invalid)
    want, _ = joint(s1, v1, s2, v2)
    want[invalid] = 0
    np.testing.assert_allclose(out, want, rtol=2e-5, atol=2e-6)
    assert (out[3] == 0).all() and (out[5] == 0).all()


def test_merge_states_plus_inf_is_empty():
    rng = np.random.default_rng(4)
    o_h, o_c = rng.standard_normal((2, 1, 8)), rng.standard_normal((2, 1, 8))
    lse_h, lse_c = np.zeros((1, 2)), np.array([[INF, 0.0]])
    out = O.merge_states(o_h, lse_h, o_c, lse_c, np.zeros(2, bool))
    np.testing.assert_allclose(out[0], o_h[0], rtol=1e-6)
    np.testing.assert_allclose(out[1], (o_h[1] + o_c[1]) / 2, rtol=1e-6)


def test_merge_lse_is_joint_softmax_and_its_lse():
    T, H, D = 5, 3, 8
    rng = np.random.default_rng(5)
    s1, s2 = rng.standard_normal((T, H, 4)) * 2, rng.standard_normal((T, H, 6)) * 2
    v1, v2 = rng.standard_normal((T, 4, D)), rng.standard_normal((T, 6, D))
    s1[0] = -INF
    s1[4] = s2[4] = -INF
    o1, l1 = partial(s1, v1)
    o2, l2 = partial(s2, v2)
    o1[0] = np.nan                                # a scratch (empty) row of the first partial
    out, lse = O.merge_lse(o1, l1, o2, l2)
    want, want_lse = joint(s1, v1, s2, v2)
    np.testing.assert_allclose(out, want, rtol=2e-5, atol=2e-6)
    np.testing.assert_allclose(lse[:, :4], want_lse[:, :4], rtol=1e-6)
    assert (lse[:, 4] == -INF).all() and (out[4] == 0).all()


# ---------------------------------------------------------------------------------------------- exact window

def exact_cache(rng, num_blocks, heads, block, d):
    cache = rng.standard_normal((num_blocks, heads, block, 2 * d)).astype(np.float32)
    cache[0] = INF
    return cache


def test_window_decode_matches_explicit_keys():
    """Decode (one query per request): keys [seq_len - 1 - W, seq_len - 1] of the request's exact paged cache."""
    rng = np.random.default_rng(6)
    H, d, block, W = 2, 8, 4, 5
    seq_lens = np.array([1, 3, 6, 12, 9], np.int32)
    R = len(seq_lens)
    qsl = np.arange(R + 1, dtype=np.int32)
    T = R + 2                                       # two padding tokens
    cache = exact_cache(rng, 40, H, block, d)
    table = np.zeros((R, 4), np.int32)
    perm = rng.permutation(np.arange(1, 40))
    for r in range(R):
        need = (seq_lens[r] + block - 1) // block
        table[r, :need] = perm[4 * r:4 * r + need]
    q = rng.standard_normal((T, H, d)).astype(np.float32)
    invalid = np.arange(T) >= R
    scale = 0.3
    o, lse = O.window_decode(q, cache[..., :d], cache[..., d:], table, qsl, seq_lens, W, scale, invalid)
    for t in range(T):
        if invalid[t]:
            assert (o[t] == 0).all() and (lse[:, t] == -INF).all()
            continue
        keys = list(range(max(0, seq_lens[t] - 1 - W), seq_lens[t]))
        for h in range(H):
            rows = np.stack([cache[table[t, p // block], h, p % block] for p in keys]).astype(np.float64)
            out, l = _softmax64(rows[:, :d] @ q[t, h].astype(np.float64) * scale, rows[:, d:])
            np.testing.assert_allclose(o[t, h], out, rtol=1e-5, atol=1e-6)
            np.testing.assert_allclose(lse[h, t], l, rtol=1e-5, atol=1e-6)


def test_window_decode_multi_query_is_bottom_right_causal():
    """Lq > 1: query i of the request sits at seq_len - Lq + i (FA2 bottom-right alignment)."""
    rng = np.random.default_rng(7)
    H, d, block, W = 2, 8, 4, 3
    seq_lens, qsl = np.array([7], np.int32), np.array([0, 3], np.int32)
    cache = exact_cache(rng, 8, H, block, d)
    table = np.array([[3, 5]], np.int32)
    q = rng.standard_normal((3, H, d)).astype(np.float32)
    o, lse = O.window_decode(q, cache[..., :d], cache[..., d:], table, qsl, seq_lens, W, 1.0, np.zeros(3, bool))
    for i in range(3):
        p = 7 - 3 + i
        keys = list(range(max(0, p - W), p + 1))
        rows = np.stack([cache[table[0, k // block], 0, k % block] for k in keys]).astype(np.float64)
        out, _ = _softmax64(rows[:, :d] @ q[i, 0].astype(np.float64), rows[:, d:])
        np.testing.assert_allclose(o[i, 0], out, rtol=1e-5, atol=1e-6)


def test_window_history_rows_before_ctx():
    rng = np.random.default_rng(8)
    H, d, block, W = 2, 8, 4, 4
    ctx = np.array([0, 1, 3, 4, 9, 16], np.int32)
    cache = exact_cache(rng, 32, H, block, d)
    table = rng.integers(1, 32, (len(ctx), 4)).astype(np.int32)
    q = rng.standard_normal((len(ctx), H, d)).astype(np.float32)
    o, lse = O.window_history(q, cache[..., :d], cache[..., d:], table, ctx, W, 0.5)
    for t, c in enumerate(ctx):
        if c == 0:
            assert (o[t] == 0).all() and (lse[:, t] == -INF).all()
            continue
        keys = list(range(max(0, c - W), c))
        for h in range(H):
            rows = np.stack([cache[table[t, p // block], h, p % block] for p in keys]).astype(np.float64)
            out, l = _softmax64(rows[:, :d] @ q[t, h].astype(np.float64) * 0.5, rows[:, d:])
            np.testing.assert_allclose(o[t, h], out, rtol=1e-5, atol=1e-6)
            np.testing.assert_allclose(lse[h, t], l, rtol=1e-5, atol=1e-6)


# ---------------------------------------------------------------------------------------------- RoPE / GEMM

def test_latent_rope_is_pairwise_rotation():
    rng = np.random.default_rng(9)
    head_dim, width, max_pos, T, H = 16, 24, 64, 7, 3
    inv = O.latent_inv_freq(head_dim, 1e4)
    table = O.latent_rope_table(max_pos, inv, width)
    pos = rng.integers(0, max_pos, T)
    x = rng.standard_normal((T, H, width)).astype(np.float32)
    y = O.latent_rope(x, pos, table, rounding=False)
    half = width // 2
    for t in range(T):
        ang = pos[t] * inv[np.arange(half) % inv.shape[0]].astype(np.float64)
        c, s = np.cos(ang), np.sin(ang)
        x1, x2 = x[t, :, :half].astype(np.float64), x[t, :, half:].astype(np.float64)
        np.testing.assert_allclose(y[t, :, :half], x1 * c - x2 * s, rtol=1e-5, atol=1e-5)
        np.testing.assert_allclose(y[t, :, half:], x2 * c + x1 * s, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(np.linalg.norm(y, axis=-1), np.linalg.norm(x, axis=-1), rtol=1e-5)


def test_latent_rope_rounding_is_per_op_bf16():
    rng = np.random.default_rng(10)
    table = bf16.round_bf16(O.latent_rope_table(32, O.latent_inv_freq(16, 1e6), 16))
    x = bf16.round_bf16(rng.standard_normal((5, 2, 16)).astype(np.float32))
    pos = rng.integers(0, 32, 5)
    y = O.latent_rope(x, pos, table, rounding=True)
    assert (bf16.round_bf16(y) == y).all()
    yr = O.latent_rope(x, pos, table, rounding=False)
    assert np.abs(y - yr).max() <= 2 ** -7 * np.abs(yr).max() + 1e-6


def test_absorb_is_batched_gemm():
    rng = np.random.default_rng(11)
    x = rng.standard_normal((5, 3, 32)).astype(np.float32)
    w = rng.standard_normal((3, 32, 16)).astype(np.float32)
    out = O.absorb(x, w, rounding=False, dtype=np.float64)
    for t in range(5):
        for h in range(3):
            np.testing.assert_allclose(out[t, h], x[t, h].astype(np.float64) @ w[h].astype(np.float64), rtol=1e-12)


# ---------------------------------------------------------------------------------------------- writer

def test_write_step_is_rounded_linear_plus_rounded_sum():
    """update[t, n] = bf16(sum_k h[t, k] W[n, k]) by explicit float64 loops; register = bf16(prev + update)."""
    rng = np.random.default_rng(12)
    T, hidden, out = 3, 8, 6                 # W is [out, hidden]: a transposed operand cannot even multiply
    h = bf16.round_bf16(rng.standard_normal((T, hidden)).astype(np.float32))
    W = bf16.round_bf16(rng.standard_normal((out, hidden)).astype(np.float32))
    prev = bf16.round_bf16(rng.standard_normal((T, out)).astype(np.float32))
    u = O.write_step(h, W)
    r = O.write_step(h, W, prev)
    for t in range(T):
        for n in range(out):
            dot = sum(float(h[t, k]) * float(W[n, k]) for k in range(hidden))
            want_u = bf16.round_bf16(np.array([dot], np.float32))[0]
            assert u[t, n] == want_u
            assert r[t, n] == bf16.round_bf16(np.array([np.float32(prev[t, n]) + np.float32(want_u)], np.float32))[0]


def test_write_step_with_a_permutation_weight_selects_columns():
    rng = np.random.default_rng(13)
    h = bf16.round_bf16(rng.standard_normal((5, 16)).astype(np.float32))
    perm = rng.permutation(16)[:12]
    W = np.zeros((12, 16), np.float32)
    W[np.arange(12), perm] = 1.0
    assert (O.write_step(h, W) == h[:, perm]).all()


def _teacher_cos_sin(positions, inv):
    """HF rotary layout: ``cos = cat(cos(p*f), cos(p*f))`` over the head dimension (float32 angle)."""
    ang = np.asarray(positions, np.float32)[:, None] * inv[None, :]
    return np.concatenate((np.cos(ang), np.cos(ang)), -1), np.concatenate((np.sin(ang), np.sin(ang)), -1)


def _rope_latent(cos, sin, width):
    idx = np.arange(width // 2) % (cos.shape[-1] // 2)
    return np.concatenate((cos[..., idx], cos[..., idx]), -1), np.concatenate((sin[..., idx], sin[..., idx]), -1)


def test_committed_rows_equal_the_training_pack():
    """The rows committed at loop 0 and at the last loop equal the fields of the training writer's packed row,
    whose rotation is built from the teacher's cos/sin, not from the latent table (hla/latent/register.py:23-25,
    73-85; the equality is what hla/tests/test_s6_serving.py:80-83 asserts)."""
    rng = np.random.default_rng(14)
    T, hidden, head_dim, rank, rank1, loops = 4, 32, 16, 24, 12, 4
    inv = O.latent_inv_freq(head_dim, 1e6)
    pos = np.array([0, 3, 17, 40])
    h = [bf16.round_bf16(rng.standard_normal((T, hidden)).astype(np.float32)) for _ in range(loops)]
    cand = [bf16.round_bf16(rng.standard_normal((2 * rank, hidden)).astype(np.float32) / 6) for _ in range(loops - 1)]
    cand1 = bf16.round_bf16(rng.standard_normal((2 * rank1, hidden)).astype(np.float32) / 6)
    # serving order: write1 at loop 0, accumulate from loop 1, commit with the latent tables
    first = O.write_step(h[0], cand1)
    reg = O.write_trajectory(h, cand)[-1]
    l1_key, l1_val = O.committed_row(first, rank1, pos, O.latent_rope_table(64, inv, rank1))
    key, val = O.committed_row(reg, rank, pos, O.latent_rope_table(64, inv, rank))
    # training pack (independent rotation tables)
    cos, sin = _teacher_cos_sin(pos, inv)
    c, s = _rope_latent(cos, sin, rank)
    c1, s1 = _rope_latent(cos, sin, rank1)
    r = bf16.round_bf16
    packed = np.concatenate((r(r(reg[:, :rank] * c) + r(O.rotate_half(reg[:, :rank]) * s)), reg[:, rank:],
                             r(r(first[:, :rank1] * c1) + r(O.rotate_half(first[:, :rank1]) * s1)), first[:, rank1:]), -1)
    assert (np.concatenate((key, val), -1) == packed[:, :2 * rank]).all()
    assert (np.concatenate((l1_key, l1_val), -1) == packed[:, 2 * rank:]).all()
    assert (key[0] == reg[0, :rank]).all()             # position 0: cos = 1, sin = 0
    # the register is the sum of the three loops' updates (loop 0 adds nothing)
    total = sum(h[l].astype(np.float64) @ cand[l - 1].astype(np.float64).T for l in range(1, loops))
    assert np.abs(reg - total).max() <= 2 ** -6 * np.abs(total).max()
    # planted: rotating with the wrong half split fails the equality
    wrong = O.latent_rope(reg[:, :rank], pos, O.latent_rope_table(64, inv, rank)[:, ::-1].copy())
    assert not (wrong == packed[:, :rank]).all()


def test_bf16_conversions():
    vals = np.array([1.0, 1 + 2 ** -8, 1 + 3 * 2 ** -8, -2.5, 0.0, INF, -INF, 3.0e38], np.float32)
    bits = bf16.from_f32(vals)
    assert bf16.to_f32(bits).tolist()[:5] == [1.0, 1.0, 1 + 2 ** -6, -2.5, 0.0]   # ties to even
    assert bits[5] == 0x7F80 and bits[6] == 0xFF80
    assert np.isnan(bf16.to_f32(bf16.from_f32(np.array([np.nan], np.float32))))[0]
    r = np.random.default_rng(0).standard_normal(1000).astype(np.float32)
    assert (bf16.from_f32(bf16.to_f32(bf16.from_f32(r))) == bf16.from_f32(r)).all()


# ---------------------------------------------------------------------------------------------- composite

def test_attend_decode_is_one_joint_softmax():
    """History (through A_t/B_t absorption) + exact window + LSE merge equals one softmax over the union of keys,
    the semantics of the HF engine's mixed_attention (hla/latent/batched_engine.py:154-182) with a window."""
    rng = np.random.default_rng(12)
    H, d, r, block, W = 2, 8, 12, 4, 3
    seq_lens = np.array([9, 2, 14], np.int32)
    R = len(seq_lens)
    qsl = np.arange(R + 1, dtype=np.int32)
    ctx = seq_lens - 1
    ctx_lat = np.maximum(ctx - W, 0)
    lat = rng.standard_normal((30, 1, block, 2 * r)).astype(np.float32)
    ex = rng.standard_normal((30, H, block, 2 * d)).astype(np.float32)
    table = np.stack([rng.permutation(np.arange(1, 30))[:4] for _ in range(R)]).astype(np.int32)
    q_lat = rng.standard_normal((R, H, r)).astype(np.float32)
    q_rope = rng.standard_normal((R, H, d)).astype(np.float32)
    B = rng.standard_normal((H, r, d)).astype(np.float32)
    out = O.attend_decode(q_lat, q_rope, B, lat[..., :r], lat[..., r:], table, ctx_lat, ex[..., :d], ex[..., d:],
                          table, qsl, seq_lens, W, 0.4, np.zeros(R, bool), rounding=False, dtype=np.float64)
    for t in range(R):
        for h in range(H):
            hist = [lat[table[t, j // block], 0, j % block].astype(np.float64) for j in range(ctx_lat[t])]
            win = [ex[table[t, p // block], h, p % block].astype(np.float64)
                   for p in range(max(0, seq_lens[t] - 1 - W), seq_lens[t])]
            s = [row[:r] @ q_lat[t, h] * 0.4 for row in hist] + [row[:d] @ q_rope[t, h] * 0.4 for row in win]
            vals = [row[r:] @ B[h] for row in hist] + [row[d:] for row in win]
            want, _ = _softmax64(np.array(s), np.array(vals))
            np.testing.assert_allclose(out[t, h], want, rtol=1e-6, atol=1e-6)   # the merge is fp32, as in the reference


# ---------------------------------------------------------------------------------------------- planted mistakes

def test_planted_mistakes_fail_the_pins():
    """Plausible oracle mistakes (dropped key, wrong scale, swapped heads, sign of the rotation) fail a pin."""
    width, heads = 8, 2
    q, cache, table, ctx = paged_setup(8, width, heads)
    scale = 1 / math.sqrt(width)
    k, v = cache[..., :width], cache[..., width:]
    cases = {
        'dropped last key': lambda: O.history_attention(q, k, v, table, np.maximum(ctx - 1, 0), scale),
        'wrong scale': lambda: O.history_attention(q, k, v, table, ctx, scale * 1.01),
        'swapped heads': lambda: tuple(x[..., ::-1, :] if x.ndim == 3 else x[::-1]
                                       for x in O.history_attention(q, k, v, table, ctx, scale)),
        'K/V swapped': lambda: O.history_attention(q, v, k, table, ctx, scale),
    }
    for name, planted in cases.items():
        o, lse = planted()
        with pytest.raises(AssertionError):
            check_history(o, lse, q, cache, table, ctx, scale)
    rng = np.random.default_rng(9)
    inv = O.latent_inv_freq(16, 1e4)
    table_r = O.latent_rope_table(16, inv, 8)
    x = rng.standard_normal((3, 1, 8)).astype(np.float32)
    pos = np.array([1, 5, 9])
    wrong = x * np.concatenate((table_r[pos, :4], table_r[pos, :4]), -1)[:, None] - \
        O.rotate_half(x) * np.concatenate((table_r[pos, 4:], table_r[pos, 4:]), -1)[:, None]
    assert not np.allclose(wrong, O.latent_rope(x, pos, table_r, rounding=False), atol=1e-3)


# ---------------------------------------------------------------------------------------------- multi-query history

def _khop_case(seed, B=2, Lq=5, N=7, H=3, R=4, causal=True):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B, Lq, H, R))
    k = rng.standard_normal((B, N, R))
    v = rng.standard_normal((B, N, R))
    i = np.arange(Lq)[:, None]
    j = np.arange(N)[None, :]
    mask = np.broadcast_to(j < i + N - Lq, (B, Lq, N)).copy() if causal else rng.random((B, Lq, N)) < 0.6
    mask[0, 0] = False                          # one query row without history
    if B > 1:
        mask[1, :, N - 1] = False               # a padded key
    return q, k, v, mask


def test_causal_history_matches_per_row_softmax():
    q, k, v, mask = _khop_case(20, causal=False)
    scale = 0.37
    z, lse = O.causal_history(q, k, v, mask, scale)
    B, Lq, H, _ = q.shape
    for b in range(B):
        for i in range(Lq):
            for h in range(H):
                keys = np.flatnonzero(mask[b, i])
                if keys.size == 0:
                    assert (z[b, i, h] == 0).all() and lse[b, h, i] == -np.inf
                    continue
                out, l = _softmax64(k[b, keys] @ q[b, i, h] * scale, v[b, keys])
                np.testing.assert_allclose(z[b, i, h], out, rtol=1e-12, atol=1e-12)
                np.testing.assert_allclose(lse[b, h, i], l, rtol=1e-12)


@pytest.mark.parametrize('use_z', [False, True])
def test_causal_history_backward_is_the_gradient(use_z):
    """Central finite differences of L = sum(z * dz) + sum(lse * dlse) (finite lse only) in float64."""
    q, k, v, mask = _khop_case(21, B=2, Lq=4, N=6, H=2, R=3)
    rng = np.random.default_rng(22)
    scale = 0.6
    z, lse = O.causal_history(q, k, v, mask, scale)
    dz = rng.standard_normal(z.shape)
    dlse = rng.standard_normal(lse.shape)

    def objective(q_, k_, v_):
        z_, l_ = O.causal_history(q_, k_, v_, mask, scale)
        return float((z_ * dz).sum() + np.where(np.isfinite(l_), l_ * dlse, 0.0).sum())

    dq, dk, dv = O.causal_history_backward(q, k, v, mask, scale, lse, dz, dlse, z=z if use_z else None)
    eps = 1e-6
    for name, x, g in (('q', q, dq), ('k', k, dk), ('v', v, dv)):
        num = np.zeros_like(x)
        for idx in np.ndindex(x.shape):
            xp, xm = x.copy(), x.copy()
            xp[idx] += eps
            xm[idx] -= eps
            args = {'q': (xp, k, v), 'k': (q, xp, v), 'v': (q, k, xp)}[name]
            argm = {'q': (xm, k, v), 'k': (q, xm, v), 'v': (q, k, xm)}[name]
            num[idx] = (objective(*args) - objective(*argm)) / (2 * eps)
        np.testing.assert_allclose(g, num, rtol=1e-6, atol=1e-7, err_msg=name)


def test_causal_history_planted_mistakes_fail():
    """A dropped dlse term or a transposed key/query in dk fails the finite-difference pin."""
    q, k, v, mask = _khop_case(23, B=1, Lq=3, N=4, H=2, R=2)
    rng = np.random.default_rng(24)
    z, lse = O.causal_history(q, k, v, mask, 0.5)
    dz, dlse = rng.standard_normal(z.shape), rng.standard_normal(lse.shape)
    dq, dk, dv = O.causal_history_backward(q, k, v, mask, 0.5, lse, dz, dlse)
    dq0, _, _ = O.causal_history_backward(q, k, v, mask, 0.5, lse, dz, None)
    assert np.abs(dq - dq0).max() > 1e-3
    _, dkv, _ = O.causal_history_backward(q, v, k, mask, 0.5, lse, dz, dlse)
    assert np.abs(dk - dkv).max() > 1e-3


def test_single_history_matches_per_row_softmax_and_its_gradient():
    """The single-query form (fused_history.reference): per (b, h) softmax over the visible keys, an empty row gives
    z = 0 and lse = -inf, and its backward is the finite-difference gradient of sum(z dz) + sum(lse dlse)."""
    rng = np.random.default_rng(31)
    B, H, N, R = 3, 2, 7, 3
    q, k, v = rng.standard_normal((B, H, R)), rng.standard_normal((B, N, R)), rng.standard_normal((B, N, R))
    mask = rng.random((B, N)) < 0.5
    mask[0] = False
    mask[1, 2] = True
    scale = 0.45
    z, lse = O.single_history(q, k, v, mask, scale)
    assert z.shape == (B, H, R) and lse.shape == (B, H)
    for b in range(B):
        keys = np.flatnonzero(mask[b])
        for h in range(H):
            if keys.size == 0:
                assert (z[b, h] == 0).all() and lse[b, h] == -np.inf
                continue
            out, l = _softmax64(k[b, keys] @ q[b, h] * scale, v[b, keys])
            np.testing.assert_allclose(z[b, h], out, rtol=1e-12, atol=1e-12)
            np.testing.assert_allclose(lse[b, h], l, rtol=1e-12)
    dz, dlse = rng.standard_normal(z.shape), rng.standard_normal(lse.shape)

    def objective(q_, k_, v_):
        z_, l_ = O.single_history(q_, k_, v_, mask, scale)
        return float((z_ * dz).sum() + np.where(np.isfinite(l_), l_ * dlse, 0.0).sum())

    grads = O.single_history_backward(q, k, v, mask, scale, lse, dz, dlse)
    eps = 1e-6
    for pos, (x, g) in enumerate(zip((q, k, v), grads)):
        num = np.zeros_like(x)
        for idx in np.ndindex(x.shape):
            xp, xm = x.copy(), x.copy()
            xp[idx] += eps
            xm[idx] -= eps
            a, m = [q, k, v], [q, k, v]
            a[pos], m[pos] = xp, xm
            num[idx] = (objective(*a) - objective(*m)) / (2 * eps)
        np.testing.assert_allclose(g, num, rtol=1e-6, atol=1e-7, err_msg='qkv'[pos])
    assert (grads[0][0] == 0).all()


# ---------------------------------------------------------------------------------------------- prefill / mixed composite

def _chunk_case(seed=13):
    """Three requests of a prefill / mixed step (a chunk after history, a decode row, a fresh prompt) plus two
    padding tokens, on tiny shapes with distinct latent and exact page tables."""
    rng = np.random.default_rng(seed)
    H, d, r, block, W = 2, 8, 12, 4, 3
    lens, hist = np.array([4, 1, 3]), np.array([11, 5, 0])
    qsl = np.concatenate(([0], np.cumsum(lens))).astype(np.int32)
    T = int(qsl[-1]) + 2
    seq = (hist + lens).astype(np.int32)
    req, valid, ctx, ctx_lat = O.step_context(qsl, seq, T, W)
    lat = rng.standard_normal((40, 1, block, 2 * r)).astype(np.float32)
    ex = rng.standard_normal((40, H, block, 2 * d)).astype(np.float32)
    lat[0] = INF
    ex[0] = INF                                     # the null page: any read past a row's pages is loud
    lt = np.stack([rng.permutation(np.arange(1, 40))[:5] for _ in range(3)]).astype(np.int32)
    et = np.stack([rng.permutation(np.arange(1, 40))[:5] for _ in range(3)]).astype(np.int32)
    f = lambda *s: rng.standard_normal(s).astype(np.float32)
    case = dict(q_lat=f(T, H, r), q_rope=f(T, H, d), k_rope=f(T, H, d), v=f(T, H, d), B=f(H, r, d), lat=lat, ex=ex,
                lt=lt, et=et, req=req, valid=valid, ctx=ctx, ctx_lat=ctx_lat, qsl=qsl, W=W, scale=0.35, r=r, d=d,
                block=block, H=H, T=T)
    return case


def _attend_chunk(c):
    r, d = c['r'], c['d']
    return O.attend_chunk(c['q_lat'], c['q_rope'], c['k_rope'], c['v'], c['B'], c['lat'][..., :r], c['lat'][..., r:],
                          {'latent': c['lt'][c['req']], 'exact': c['et'][c['req']]}, c['ctx'], c['ctx_lat'], c['qsl'],
                          c['W'], c['scale'], ~c['valid'], c['ex'][..., :d], c['ex'][..., d:], rounding=False,
                          dtype=np.float64)


def _check_attend_chunk(out, c):
    """One float64 softmax per (token, head) over the union of its keys: the causal chunk of its request, the exact
    window rows [ctx - W, ctx) of the exact cache, and the latent rows [0, ctx - W) read through B[h]."""
    r, d, block, s = c['r'], c['d'], c['block'], c['scale']
    for t in range(c['T']):
        if not c['valid'][t]:
            assert (out[t] == 0).all()
            continue
        rq, n = int(c['req'][t]), int(c['ctx'][t])
        for h in range(c['H']):
            scores, vals = [], []
            for u in range(int(c['qsl'][rq]), t + 1):
                scores.append(float(c['k_rope'][u, h].astype(np.float64) @ c['q_rope'][t, h]) * s)
                vals.append(c['v'][u, h].astype(np.float64))
            for p in range(max(0, n - c['W']), n):
                row = c['ex'][c['et'][rq, p // block], h, p % block].astype(np.float64)
                scores.append(float(row[:d] @ c['q_rope'][t, h]) * s)
                vals.append(row[d:])
            for j in range(max(0, n - c['W'])):
                row = c['lat'][c['lt'][rq, j // block], 0, j % block].astype(np.float64)
                scores.append(float(row[:r] @ c['q_lat'][t, h]) * s)
                vals.append(row[r:] @ c['B'][h].astype(np.float64))
            want, _ = _softmax64(np.array(scores), np.array(vals))
            np.testing.assert_allclose(out[t, h], want, rtol=1e-6, atol=1e-6)


def test_attend_chunk_is_one_joint_softmax():
    """The prefill / mixed branch of attend (hla/vllm_latent/s6_layer.py:101-115): causal chunk + exact window over
    history rows [ctx - W, ctx) + latent history [0, ctx - W) through B_t equal one softmax over all of them."""
    c = _chunk_case()
    assert c['ctx'].tolist()[:8] == [11, 11, 11, 11, 5, 0, 0, 0] and c['ctx_lat'].tolist()[:5] == [8] * 4 + [2]
    _check_attend_chunk(_attend_chunk(c), c)


def test_attend_chunk_planted_mistakes_fail(monkeypatch):
    """Plausible wiring mistakes inside the composite, planted in the oracle one at a time, fail the pin."""
    c = _chunk_case()
    real = {name: getattr(O, name) for name in ('window_history', 'history_attention', 'chunk_attention', 'absorb')}

    def window_on_latent_ctx(q, k, v, table, ctx, *a, **kw):          # ctx_latent handed to the window
        return real['window_history'](q, k, v, table, np.maximum(ctx - c['W'], 0), *a, **kw)

    def history_over_ctx(q, k, v, table, ctx, *a, **kw):              # latent rows overlap the exact window
        return real['history_attention'](q, k, v, table, np.where(ctx > 0, ctx + c['W'], 0), *a, **kw)

    def window_shifted(q, k, v, table, ctx, *a, **kw):                # window one row early
        return real['window_history'](q, k, v, table, np.maximum(ctx - 1, 0), *a, **kw)

    def chunk_not_causal(q, k, v, qsl, invalid, scale, rounding=False, dtype=np.float32):
        qsl_all = np.array([0, q.shape[0]])                             # every token sees the whole step
        return real['chunk_attention'](q, k, v, qsl_all, invalid, scale, rounding, dtype)

    def readout_heads_swapped(x, w, *a, **kw):
        return real['absorb'](x, w[::-1], *a, **kw)

    for name, fn in (('window_history', window_on_latent_ctx), ('history_attention', history_over_ctx),
                     ('window_history', window_shifted), ('chunk_attention', chunk_not_causal),
                     ('absorb', readout_heads_swapped)):
        monkeypatch.setattr(O, name, fn)
        with pytest.raises(AssertionError):
            _check_attend_chunk(_attend_chunk(c), c)
        monkeypatch.setattr(O, name, real[name])
    _check_attend_chunk(_attend_chunk(c), c)


# ---------------------------------------------------------------------------------------------- HF engine joint softmax

def _rotate_pairs(x, cos_pair, sin_pair):
    """Rotation of the pairs (c, c + w/2) of x by the angles whose cos / sin are given per pair (explicit loop)."""
    w = x.shape[-1]
    y = np.empty(w)
    for c in range(w // 2):
        a, b = x[c], x[c + w // 2]
        y[c] = a * cos_pair[c] - b * sin_pair[c]
        y[c + w // 2] = b * cos_pair[c] + a * sin_pair[c]
    return y


def _mixed_case(seed, B=2, H=2, n=5, d=4, r=6, sizes=(6, 3)):
    rng = np.random.default_rng(seed)
    f = lambda *s: rng.standard_normal(s)
    q, k, v = f(B, H, n, d), f(B, H, n, d), f(B, H, n, d)
    pos = rng.integers(0, 50, B)[:, None] + np.arange(n)[None]
    inv = 1.0 / (100.0 ** (np.arange(0, d, 2) / d))
    ang = pos[..., None] * inv                                       # [B, n, d/2]
    cos, sin = np.concatenate((np.cos(ang),) * 2, -1), np.concatenate((np.sin(ang),) * 2, -1)
    valid = np.ones((B, n), bool)
    valid[0, :2] = False                                             # left padding
    hist_k = [f(B, N, r) for N in sizes]
    hist_v = [f(B, N, r) for N in sizes]
    masks = [rng.random((B, N)) < 0.7 for N in sizes]
    if masks:
        masks[0][1] = False                                          # a row that sees nothing of a block
    A, Bw = f(H, d, r) * 0.5, f(H, r, d) * 0.5
    return dict(q=q, k=k, v=v, cos=cos, sin=sin, valid=valid, hist_k=hist_k, hist_v=hist_v, masks=masks, A=A, B=Bw,
                scale=0.6, ang=ang)


def _mixed(c, **over):
    c = dict(c, **over)
    return O.mixed_attention(c['q'], c['k'], c['v'], c['cos'], c['sin'], c['valid'], c['hist_k'], c['hist_v'],
                             c['masks'], c['A'], c['B'], c['scale'])


def _check_mixed(out, c):
    """Per (b, h, i): one float64 softmax over the block rows the query's mask shows (latent query q A rotated pair
    by pair with teacher frequency c % (d/2), values through B[h]) and the chunk keys it sees (RoPE'd q / k)."""
    q, k, v, ang, valid, s = c['q'], c['k'], c['v'], c['ang'], c['valid'], c['scale']
    Bn, H, n, d = q.shape
    half = d // 2
    for b in range(Bn):
        for h in range(H):
            for i in range(n):
                qr = _rotate_pairs(q[b, h, i], np.cos(ang[b, i]), np.sin(ang[b, i]))
                scores, vals = [], []
                for ck, cv, m in zip(c['hist_k'], c['hist_v'], c['masks']):
                    r = ck.shape[-1]
                    idx = np.arange(r // 2) % half
                    qc = _rotate_pairs(q[b, h, i] @ c['A'][h], np.cos(ang[b, i, idx]), np.sin(ang[b, i, idx]))
                    for j in range(ck.shape[1]):
                        if m[b, j]:
                            scores.append(float(qc @ ck[b, j]) * s)
                            vals.append(cv[b, j] @ c['B'][h])
                for j in range(n):
                    if (valid[b, i] and valid[b, j] and j <= i) or not valid[b, i]:
                        kr = _rotate_pairs(k[b, h, j], np.cos(ang[b, j]), np.sin(ang[b, j]))
                        scores.append(float(qr @ kr) * s)
                        vals.append(v[b, h, j])
                want, _ = _softmax64(np.array(scores), np.array(vals))
                np.testing.assert_allclose(out[b, h, i], want, rtol=1e-9, atol=1e-9)


@pytest.mark.parametrize('sizes', [(6, 3), (), (4,)])
def test_mixed_attention_is_one_softmax_per_query(sizes):
    """The HF rolling engine's joint attention (hla/latent/batched_engine.py:154-182) against explicit per-query
    softmaxes (padding queries see the whole chunk; rows a block hides are skipped)."""
    c = _mixed_case(21 + len(sizes), sizes=sizes)
    _check_mixed(_mixed(c), c)


def test_mixed_attention_planted_mistakes_fail(monkeypatch):
    c = _mixed_case(22)
    real_tables, real_rope = O.rope_latent_tables, O.hf_rope

    def tables_clamped(cos, sin, width):                             # pairs past d/2 reuse the last frequency
        idx = np.minimum(np.arange(width // 2), cos.shape[-1] // 2 - 1)
        return np.concatenate((cos[..., idx],) * 2, -1), np.concatenate((sin[..., idx],) * 2, -1)

    def rope_wrong_sign(x, cos, sin):
        return x * cos[:, None] - O.rotate_half(x) * sin[:, None]

    for name, fn in (('rope_latent_tables', tables_clamped), ('hf_rope', rope_wrong_sign)):
        monkeypatch.setattr(O, name, fn)
        with pytest.raises(AssertionError):
            _check_mixed(_mixed(c), c)
    monkeypatch.setattr(O, 'rope_latent_tables', real_tables)
    monkeypatch.setattr(O, 'hf_rope', real_rope)
    with pytest.raises(AssertionError):                               # a block's mask ignored
        _check_mixed(_mixed(c, masks=[np.ones_like(m) for m in c['masks']]), c)
    with pytest.raises(AssertionError):                               # padding queries limited to valid keys
        _check_mixed(_mixed(c, valid=np.ones_like(c['valid'])), c)


def _fd_check(c, grads, eps=1e-6, tol=1e-6):
    """Central finite differences of sum(out * g) for every element of every differentiable input."""
    g = c['g']
    loss = lambda cc: float((_mixed(cc) * g).sum())
    leaves = {'q': c['q'], 'k': c['k'], 'v': c['v'], 'A': c['A'], 'B': c['B']}
    for i in range(len(c['hist_k'])):
        leaves[f'hist_k{i}'] = c['hist_k'][i]
        leaves[f'hist_v{i}'] = c['hist_v'][i]
    for name, x in leaves.items():
        want = grads[name[:6]][int(name[6:])] if name.startswith('hist') else grads[name]
        got = np.zeros_like(x)
        for idx in np.ndindex(x.shape):
            old = x[idx]
            x[idx] = old + eps
            up = loss(c)
            x[idx] = old - eps
            down = loss(c)
            x[idx] = old
            got[idx] = (up - down) / (2 * eps)
        np.testing.assert_allclose(want, got, rtol=tol, atol=tol, err_msg=name)


def test_mixed_attention_backward_is_the_gradient():
    c = _mixed_case(23, n=4, sizes=(5, 3))
    c['g'] = np.random.default_rng(3).standard_normal(c['q'].shape)
    grads = O.mixed_attention_backward(c['q'], c['k'], c['v'], c['cos'], c['sin'], c['valid'], c['hist_k'],
                                       c['hist_v'], c['masks'], c['A'], c['B'], c['scale'], c['g'])
    _fd_check(c, grads)
    c0 = _mixed_case(24, n=3, sizes=())                               # no history: A and B have no gradient
    c0['g'] = np.random.default_rng(4).standard_normal(c0['q'].shape)
    g0 = O.mixed_attention_backward(c0['q'], c0['k'], c0['v'], c0['cos'], c0['sin'], c0['valid'], [], [], [], c0['A'],
                                    c0['B'], c0['scale'], c0['g'])
    assert g0['A'] is None and g0['B'] is None
    g0['A'], g0['B'] = np.zeros_like(c0['A']), np.zeros_like(c0['B'])
    _fd_check(c0, g0)


def test_mixed_attention_backward_planted_mistake_fails(monkeypatch):
    c = _mixed_case(25, n=3, sizes=(4,))
    c['g'] = np.random.default_rng(5).standard_normal(c['q'].shape)

    def rope_backward_untransposed(dy, cos, sin):                      # R instead of R^T
        return dy * cos[:, None] + O.rotate_half(dy * sin[:, None])

    monkeypatch.setattr(O, 'hf_rope_backward', rope_backward_untransposed)
    grads = O.mixed_attention_backward(c['q'], c['k'], c['v'], c['cos'], c['sin'], c['valid'], c['hist_k'],
                                       c['hist_v'], c['masks'], c['A'], c['B'], c['scale'], c['g'])
    with pytest.raises(AssertionError):
        _fd_check(c, grads)
