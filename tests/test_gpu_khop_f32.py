"""Multi-query causal history attention in fp32 arithmetic (``history_gemm.causal_history_gemm`` with the reference's
default ``precision='fp32'``, ``'tf32'``, and ``causal_history_attention``'s fp32 ``'triton'`` / ``'reference'``
backends, over khop_f32.hip) against the float64 oracle (``oracle.s6_oracle.causal_history`` /
``causal_history_backward``, restating hla/latent/history_gemm.py:159-220) on fp32 inputs.

Bars: z, dq, dk, dv within relative L2 1e-5 of the float64 oracle (per tensor), lse within 2e-5; rows without a
visible key give exactly z = 0, lse = -inf and zero dq. Also: the width-1024 backward of bf16 mode (run on these
kernels) against the oracle at the bf16 bars, key ranges of the dk / dv kernel, broadcast masks, the modes that
share the kernels bitwise, and the inputs the fp32 kernels refuse.
"""
import importlib
import math

import numpy as np
import pytest
import torch

from oracle import bf16
from oracle import s6_oracle as O
from s6util import assert_attention_close, assert_lse_close, rel_l2

pytestmark = pytest.mark.gpu

hg = importlib.import_module('hybrid-latent-attention_amd.history_gemm')

REL = 1e-5
LSE_ATOL = 2e-5


def case(seed, B, Lq, N, R, kind):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B, Lq, 16, R)).astype(np.float32)
    k = rng.standard_normal((B, N, R)).astype(np.float32)
    v = rng.standard_normal((B, N, R)).astype(np.float32)
    if kind == 'benchmark':                    # hla/latent/benchmark_history_gemm.py:72-76
        assert Lq == N
        lengths = np.array([max(2, int(Lq * (1 - 0.1 * b))) for b in range(B)])
        valid = np.arange(Lq)[None] < lengths[:, None]
        order = np.arange(Lq)[:, None] > np.arange(Lq)[None]
        mask = valid[:, :, None] & valid[:, None, :] & order[None]
    elif kind == 'khop':                       # prompt P, window W: query i sees j < P + i - W
        P, W = N - Lq, 3
        mask = np.broadcast_to(np.arange(N)[None] < P + np.arange(Lq)[:, None] - W, (B, Lq, N)).copy()
    else:                                      # arbitrary, with rows that see nothing
        mask = rng.random((B, Lq, N)) < 0.3
        mask[:, 1] = False
    return q, k, v, mask


def run(q, k, v, mask, scale, dz, dlse, precision='fp32', dtype=torch.float32, **kw):
    leaves = [torch.tensor(x, device='cuda').to(dtype).requires_grad_(True) for x in (q, k, v)]
    z, lse = hg.causal_history_gemm(*leaves, torch.tensor(mask, device='cuda'), scale, precision=precision, **kw)
    g = torch.autograd.grad([z, lse], leaves, [torch.tensor(dz, device='cuda').to(z.dtype),
                                                torch.tensor(dlse, device='cuda')])
    host = lambda t: t.detach().float().cpu().numpy()
    return dict(z=host(z), lse=host(lse), dq=host(g[0]), dk=host(g[1]), dv=host(g[2]), dtype=z.dtype)


def oracle(q, k, v, mask, scale, dz, dlse):
    z, lse = O.causal_history(q, k, v, mask, scale)
    dq, dk, dv = O.causal_history_backward(q, k, v, mask, scale, lse, dz, dlse, z=z)
    return dict(z=z, lse=lse, dq=dq, dk=dk, dv=dv)


def assert_close(got, want, what, rel=REL):
    assert np.isfinite(got).all(), f'{what}: non-finite'
    r = rel_l2(got, want)
    assert r <= rel, f'{what}: rel-L2 {r:.3e} > {rel}'


@pytest.mark.parametrize('R', [128, 256, 512, 1024])
@pytest.mark.parametrize('kind,B,Lq,N', [('benchmark', 2, 45, 45), ('khop', 2, 21, 70), ('any', 2, 37, 50)])
def test_fp32_forward_and_backward_match_the_float64_oracle(R, kind, B, Lq, N):
    q, k, v, mask = case(13 * R + Lq, B, Lq, N, R, kind)
    scale = 1 / math.sqrt(128)
    rng = np.random.default_rng(R + N + 1)
    dz = rng.standard_normal((B, Lq, 16, R)).astype(np.float32)
    dlse = rng.standard_normal((B, 16, Lq)).astype(np.float32)
    print(f'case fp32 R={R} {kind} B={B} Lq={Lq} N={N}', flush=True)
    got = run(q, k, v, mask, scale, dz, dlse)
    want = oracle(q, k, v, mask, scale, dz, dlse)
    assert got['dtype'] == torch.float32
    for name in ('z', 'dq', 'dk', 'dv'):
        assert_close(got[name], want[name], name)
    assert_lse_close(got['lse'], want['lse'], atol=LSE_ATOL)
    empty = ~mask.any(-1)
    assert (got['z'][empty] == 0).all() and np.isneginf(got['lse'].transpose(0, 2, 1)[empty]).all()
    assert (got['dq'][empty] == 0).all()


def test_fp32_over_many_tiles_and_key_ranges(monkeypatch):
    """300 queries over 300 keys (19 key tiles, a causal mask with padding), dk / dv with key ranges forced to 1 and
    to 5 (partials summed in a fixed order): both match the oracle, and each is bitwise repeatable."""
    R, B, L = 512, 2, 300
    q, k, v, mask = case(77, B, L, L, R, 'benchmark')
    scale = 1 / math.sqrt(128)
    rng = np.random.default_rng(78)
    dz = rng.standard_normal((B, L, 16, R)).astype(np.float32)
    dlse = rng.standard_normal((B, 16, L)).astype(np.float32)
    want = oracle(q, k, v, mask, scale, dz, dlse)
    for splits in (1, 5):
        print(f'case fp32 key ranges={splits}', flush=True)
        monkeypatch.setattr(hg, '_f32_key_splits', lambda *a, s=splits: s)
        got = run(q, k, v, mask, scale, dz, dlse)
        again = run(q, k, v, mask, scale, dz, dlse)
        for name in ('z', 'dq', 'dk', 'dv'):
            assert_close(got[name], want[name], f'{name} ({splits} ranges)')
            assert np.array_equal(got[name], again[name]), f'{name} not repeatable'


def test_fp32_modes_and_backends_share_the_kernels():
    """The reference's default precision ('fp32'), 'tf32', and causal_history_attention's 'triton' and 'reference'
    backends give bitwise the same results; bf16 inputs get a bf16 z (the fp32 result rounded) and bf16 gradients."""
    R, B, Lq, N = 256, 2, 19, 64
    q, k, v, mask = case(5, B, Lq, N, R, 'khop')
    qt, kt, vt = (torch.tensor(x, device='cuda') for x in (q, k, v))
    mt = torch.tensor(mask, device='cuda')
    base = hg.causal_history_gemm(qt, kt, vt, mt, 0.1)                     # default precision: fp32
    others = [hg.causal_history_gemm(qt, kt, vt, mt, 0.1, precision='tf32'),
              hg.causal_history_attention(qt, kt, vt, mt, 0.1),            # default backend: triton
              hg.causal_history_attention(qt, kt, vt, mt, 0.1, backend='reference'),
              hg.causal_history_attention(qt, kt, vt, mt, 0.1, backend='gemm', precision='fp32')]
    for z, lse in others:
        assert torch.equal(z, base[0]) and torch.equal(lse, base[1])
    zo, lo = O.causal_history(q, k, v, mask, 0.1)
    assert_close(base[0].cpu().numpy(), zo, 'z')
    qb, kb, vb = (t.to(torch.bfloat16).requires_grad_(True) for t in (qt, kt, vt))
    zb, lb = hg.causal_history_gemm(qb, kb, vb, mt, 0.1)
    z32, l32 = hg.causal_history_gemm(qb.detach().float(), kb.detach().float(), vb.detach().float(), mt, 0.1)
    assert zb.dtype == torch.bfloat16 and torch.equal(zb, z32.to(torch.bfloat16)) and torch.equal(lb, l32)
    g = torch.autograd.grad(zb.float().sum(), [qb, kb, vb])
    assert all(x.dtype == torch.bfloat16 for x in g)


def test_fp32_broadcast_mask_and_no_query_gradient():
    """A [B, N] key mask expanded over the queries (query stride 0) gives bitwise the results of the copied mask;
    gradients of k / v alone (q not requiring grad) match the oracle."""
    R, B, Lq, N = 512, 3, 21, 50
    q, k, v, _ = case(9, B, Lq, N, R, 'any')
    rng = np.random.default_rng(10)
    rows = rng.random((B, N)) < 0.6
    rows[1] = False
    mask = np.broadcast_to(rows[:, None], (B, Lq, N)).copy()
    dz = rng.standard_normal((B, Lq, 16, R)).astype(np.float32)
    outs = []
    for broadcast in (False, True):
        qt = torch.tensor(q, device='cuda')
        kt, vt = (torch.tensor(x, device='cuda').requires_grad_(True) for x in (k, v))
        mt = torch.tensor(rows, device='cuda')[:, None].expand(B, Lq, N)
        mt = mt if broadcast else mt.contiguous()
        z, lse = hg.causal_history_gemm(qt, kt, vt, mt, 0.07)
        gk, gv = torch.autograd.grad(z, [kt, vt], torch.tensor(dz, device='cuda'))
        outs.append([x.detach().cpu() for x in (z, lse, gk, gv)])
    for name, a, b in zip(('z', 'lse', 'dk', 'dv'), *outs):
        assert torch.equal(a, b), name
    want = oracle(q, k, v, mask, 0.07, dz, np.zeros((B, 16, Lq), np.float32))
    assert_close(outs[1][2].numpy(), want['dk'], 'dk')
    assert_close(outs[1][3].numpy(), want['dv'], 'dv')


def test_fp32_refuses_float64_and_unsupported_widths():
    q = torch.zeros(1, 4, 16, 256, device='cuda', dtype=torch.float64)
    k = torch.zeros(1, 4, 256, device='cuda', dtype=torch.float64)
    m = torch.ones(1, 4, 4, dtype=torch.bool, device='cuda')
    with pytest.raises(ValueError, match='float64'):
        hg.causal_history_gemm(q, k, k, m, 1.0)
    with pytest.raises(ValueError, match='widths'):
        hg.causal_history_gemm(q.float()[..., :192], k.float()[..., :192], k.float()[..., :192], m, 1.0)


@pytest.mark.parametrize('kind,B,Lq,N', [('benchmark', 2, 48, 48), ('khop', 2, 19, 64), ('any', 3, 29, 96)])
def test_bf16_width_1024_backward_matches_the_oracle(kind, B, Lq, N):
    """bf16 mode at width 1024: forward on the multi-query kernel, backward on the fp32 kernels (the bf16 operands
    in fp32 arithmetic), against the oracle at the bf16 bars (z: attention tolerance; gradients rel-L2 1e-2)."""
    R = 1024
    q, k, v, mask = case(3 * N + Lq, B, Lq, N, R, kind)
    q, k, v = (bf16.round_bf16(x) for x in (q, k, v))
    scale = 1 / math.sqrt(128)
    rng = np.random.default_rng(N * Lq)
    dz = bf16.round_bf16(rng.standard_normal((B, Lq, 16, R)).astype(np.float32))
    dlse = rng.standard_normal((B, 16, Lq)).astype(np.float32)
    print(f'case bf16 R=1024 {kind}', flush=True)
    got = run(q, k, v, mask, scale, dz, dlse, precision='bf16', dtype=torch.bfloat16)
    want = oracle(q, k, v, mask, scale, dz, dlse)
    assert got['dtype'] == torch.bfloat16
    assert_attention_close(got['z'], want['z'], 'z')
    assert_lse_close(got['lse'], want['lse'])
    for name in ('dq', 'dk', 'dv'):
        assert_close(got[name], want[name], name, rel=1e-2)
