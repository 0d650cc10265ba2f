"""Multi-query causal history attention with backward (``history_gemm.causal_history_gemm`` over khop.hip) against
the float64 oracle (``oracle.s6_oracle.causal_history`` / ``causal_history_backward``, restating
hla/latent/history_gemm.py:159-220) on bf16-rounded inputs.

Bars: z within the attention tolerance (max-abs 2e-2, rel-L2 5e-3) and lse within 1e-3 of the oracle. Gradients
(bf16 GEMM operands, including the bf16-rounded P and dS that enter the second products, as the reference's bf16
mode) within relative L2 1e-2 per tensor and max-abs 2e-2 of its largest magnitude; empty rows give exactly
z = 0, lse = -inf and no gradient; results are bitwise repeatable.
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

GRAD_REL = 1e-2


def benchmark_mask(lengths, L):
    """The mask of hla/latent/benchmark_history_gemm.py:72-76: valid rows and keys, query i sees keys j < i."""
    lengths = np.asarray(lengths)
    valid = np.arange(L)[None] < lengths[:, None]
    order = np.arange(L)[:, None] > np.arange(L)[None]
    return valid[:, :, None] & valid[:, None, :] & order[None]


def case(seed, B, Lq, N, R, kind):
    rng = np.random.default_rng(seed)
    q = bf16.round_bf16(rng.standard_normal((B, Lq, 16, R)).astype(np.float32))
    k = bf16.round_bf16(rng.standard_normal((B, N, R)).astype(np.float32))
    v = bf16.round_bf16(rng.standard_normal((B, N, R)).astype(np.float32))
    if kind == 'benchmark':
        assert Lq == N
        mask = benchmark_mask([max(2, int(Lq * (1 - 0.1 * b))) for b in range(B)], Lq)
    elif kind == 'khop':                       # prompt P, window W: query i sees j < P + i - W (khop_replay.py:105)
        P, W = N - Lq, 3
        mask = np.broadcast_to(np.arange(N)[None] < P + np.arange(Lq)[:, None] - W, (B, Lq, N)).copy()
    else:                                      # arbitrary
        mask = rng.random((B, Lq, N)) < 0.3
        mask[:, 1] = False                     # rows without history
    return q, k, v, mask


def run(q, k, v, mask, scale, need_grad=True, dz=None, dlse=None):
    dev = lambda x, grad: torch.tensor(x, device='cuda').to(torch.bfloat16).requires_grad_(grad)
    qt, kt, vt = dev(q, need_grad), dev(k, need_grad), dev(v, need_grad)
    mt = torch.tensor(mask, device='cuda')
    z, lse = hg.causal_history_gemm(qt, kt, vt, mt, scale, causal=True, precision='bf16')
    out = {'z': z.detach().float().cpu().numpy(), 'lse': lse.detach().cpu().numpy()}
    if need_grad:
        dzt = torch.tensor(dz, device='cuda').to(torch.bfloat16)
        dlt = torch.tensor(dlse, device='cuda', dtype=torch.float32)
        obj = (z.float() * dzt.float()).sum() + torch.where(torch.isfinite(lse), lse * dlt, 0.).sum()
        g = torch.autograd.grad(obj, [qt, kt, vt])
        out.update(dq=g[0].float().cpu().numpy(), dk=g[1].float().cpu().numpy(), dv=g[2].float().cpu().numpy())
    return out


def assert_grad_close(got, want, what):
    assert np.isfinite(got).all(), f'{what}: non-finite'
    r = rel_l2(got, want)
    err = float(np.abs(got - want).max())
    assert r <= GRAD_REL, f'{what}: rel-L2 {r:.3e} > {GRAD_REL}'
    assert err <= 2e-2 * max(1.0, float(np.abs(want).max())), f'{what}: max-abs {err:.3e}'


@pytest.mark.parametrize('R', [128, 256, 512])
@pytest.mark.parametrize('kind,B,Lq,N', [('benchmark', 3, 45, 45), ('khop', 2, 21, 70), ('any', 2, 37, 50)])
def test_forward_and_backward_match_the_oracle(R, kind, B, Lq, N):
    q, k, v, mask = case(7 * R + Lq, B, Lq, N, R, kind)
    scale = 1 / math.sqrt(128)
    rng = np.random.default_rng(R + N)
    dz = bf16.round_bf16(rng.standard_normal((B, Lq, 16, R)).astype(np.float32))
    dlse = rng.standard_normal((B, 16, Lq)).astype(np.float32)
    got = run(q, k, v, mask, scale, dz=dz, dlse=dlse)
    z, lse = O.causal_history(q, k, v, mask, scale)
    assert_attention_close(got['z'], z, 'z')
    assert_lse_close(got['lse'], lse)
    empty = ~mask.any(-1)                                          # [B, Lq]
    assert (got['z'][empty] == 0).all() and np.isneginf(got['lse'].transpose(0, 2, 1)[empty]).all()
    dq, dk, dv = O.causal_history_backward(q, k, v, mask, scale, lse, dz, dlse)
    assert_grad_close(got['dq'], dq, 'dq')
    assert_grad_close(got['dk'], dk, 'dk')
    assert_grad_close(got['dv'], dv, 'dv')
    assert (got['dq'][empty] == 0).all()


@pytest.mark.parametrize('R', [256, 512])
@pytest.mark.parametrize('kind,B,Lq,N', [('benchmark', 2, 48, 48), ('khop', 2, 19, 64), ('any', 3, 29, 96)])
def test_key_counts_of_whole_pages_match_the_oracle(R, kind, B, Lq, N):
    """N a multiple of 16: the forward runs on the multi-query history kernel (eight tokens per workgroup, the mask
    bytes copied to LDS with each K tile); token counts that do not fill the last workgroup, rows without history."""
    q, k, v, mask = case(5 * R + N, B, Lq, N, R, kind)
    scale = 1 / math.sqrt(128)
    rng = np.random.default_rng(R * N)
    dz = bf16.round_bf16(rng.standard_normal((B, Lq, 16, R)).astype(np.float32))
    dlse = rng.standard_normal((B, 16, Lq)).astype(np.float32)
    got = run(q, k, v, mask, scale, dz=dz, dlse=dlse)
    z, lse = O.causal_history(q, k, v, mask, scale)
    assert_attention_close(got['z'], z, 'z')
    assert_lse_close(got['lse'], lse)
    empty = ~mask.any(-1)
    assert (got['z'][empty] == 0).all() and np.isneginf(got['lse'].transpose(0, 2, 1)[empty]).all()
    dq, dk, dv = O.causal_history_backward(q, k, v, mask, scale, lse, dz, dlse)
    assert_grad_close(got['dq'], dq, 'dq')
    assert_grad_close(got['dk'], dk, 'dk')
    assert_grad_close(got['dv'], dv, 'dv')


@pytest.mark.parametrize('R', [256, 512])
def test_mask_rows_off_16_byte_boundaries_and_no_mask(R):
    """A mask view whose rows do not start on 16-byte boundaries takes the other forward kernels; the C ABI without a
    mask (every key below the bound visible) takes the multi-query kernel's unmasked form. Same results as the
    oracle."""
    B, Lq, N = 2, 21, 64
    q, k, v, mask = case(17 + R, B, Lq, N, R, 'any')
    scale = 0.11
    wide = np.zeros((B, Lq, N + 8), bool)
    wide[..., :N] = mask
    qt, kt, vt = (torch.tensor(x, device='cuda').to(torch.bfloat16) for x in (q, k, v))
    mt = torch.tensor(wide, device='cuda')[..., :N]
    assert mt.stride(1) % 16 != 0
    z, lse = hg.causal_history_gemm(qt, kt, vt, mt, scale, precision='bf16')
    zo, lo = O.causal_history(q, k, v, mask, scale)
    assert_attention_close(z.float().cpu().numpy(), zo, 'z (strided mask)')
    assert_lse_close(lse.cpu().numpy(), lo)
    lib = hg._lib
    bound = torch.empty(B * Lq, dtype=torch.int32, device='cuda')
    st = lib.stream(qt.device)
    lib.call('hla_s6_khop_bounds', None, 0, 0, B, Lq, N, lib.ptr(bound), st)
    z2 = torch.empty(B, Lq, 16, R, dtype=torch.bfloat16, device='cuda')
    lse2 = torch.empty(B, 16, Lq, dtype=torch.float32, device='cuda')
    lib.call('hla_s6_khop_forward', lib.ptr(qt), qt.stride(0), qt.stride(1), qt.stride(2), lib.ptr(kt), kt.stride(0),
             kt.stride(1), lib.ptr(vt), vt.stride(0), vt.stride(1), None, 0, 0, lib.ptr(bound), B, Lq, N, 16, R,
             scale, lib.ptr(z2), z2.stride(0), z2.stride(1), z2.stride(2), lib.ptr(lse2), st)
    zo2, lo2 = O.causal_history(q, k, v, np.ones((B, Lq, N), bool), scale)
    assert_attention_close(z2.float().cpu().numpy(), zo2, 'z (no mask)')
    assert_lse_close(lse2.cpu().numpy(), lo2)
    # dq alone through the C ABI without a mask (dk, dv not asked for)
    rng = np.random.default_rng(R)
    dz = bf16.round_bf16(rng.standard_normal((B, Lq, 16, R)).astype(np.float32))
    dzt = torch.tensor(dz, device='cuda').to(torch.bfloat16)
    delta = torch.empty(B, 16, Lq, dtype=torch.float32, device='cuda')
    dq = torch.empty(B, Lq, 16, R, dtype=torch.float32, device='cuda')
    lib.call('hla_s6_khop_backward', lib.ptr(qt), qt.stride(0), qt.stride(1), qt.stride(2), lib.ptr(kt), kt.stride(0),
             kt.stride(1), lib.ptr(vt), vt.stride(0), vt.stride(1), None, 0, 0, lib.ptr(bound), B, Lq, N, 16, R, scale,
             lib.ptr(z2), z2.stride(0), z2.stride(1), z2.stride(2), lib.ptr(lse2), lib.ptr(dzt), dzt.stride(0),
             dzt.stride(1), dzt.stride(2), None, lib.ptr(delta), lib.ptr(dq), dq.stride(0), dq.stride(1), dq.stride(2),
             None, 0, 0, None, 0, 0, 1, None, 0, 0, st)
    dqo, _, _ = O.causal_history_backward(q, k, v, np.ones((B, Lq, N), bool), scale, lo2, dz, None,
                                          z=bf16.round_bf16(zo2.astype(np.float32)))
    assert_grad_close(dq.cpu().numpy(), dqo, 'dq (no mask)')


@pytest.mark.parametrize('R,N', [(256, 64), (512, 64), (512, 50), (256, 50), (1024, 64)])
def test_one_mask_row_per_batch_row_broadcast_over_queries(R, N):
    """A [B, N] key mask expanded over the queries (query stride 0, the joint-attention history blocks' form) gives
    bitwise the results of the same mask copied out per query, forward and (widths below 1024) backward, and
    matches the oracle."""
    B, Lq = 3, 21
    rng = np.random.default_rng(R + N)
    q, k, v, _ = case(R + N, B, Lq, N, R, 'any')
    rows = rng.random((B, N)) < 0.6
    rows[1] = False                            # a batch row without history
    rows[2, N // 3:] = False
    mask = np.broadcast_to(rows[:, None], (B, Lq, N)).copy()
    scale = 1 / math.sqrt(R)
    dz = bf16.round_bf16(rng.standard_normal((B, Lq, 16, R)).astype(np.float32))
    dlse = rng.standard_normal((B, 16, Lq)).astype(np.float32)
    outs = []
    for broadcast in (False, True):
        grad = R != 1024
        qt, kt, vt = (torch.tensor(x, device='cuda').to(torch.bfloat16).requires_grad_(grad) for x in (q, k, v))
        mt = torch.tensor(rows, device='cuda')[:, None].expand(B, Lq, N)
        if not broadcast:
            mt = mt.contiguous()
        assert (mt.stride(1) == 0) == broadcast
        z, lse = hg.causal_history_gemm(qt, kt, vt, mt, scale, precision='bf16')
        out = [z.detach().float().cpu(), lse.detach().cpu()]
        if grad:
            obj = (z.float() * torch.tensor(dz, device='cuda')).sum() + torch.where(
                torch.isfinite(lse), lse * torch.tensor(dlse, device='cuda'), 0.).sum()
            out += [g.float().cpu() for g in torch.autograd.grad(obj, [qt, kt, vt])]
        outs.append(out)
    for name, a, b in zip(('z', 'lse', 'dq', 'dk', 'dv'), *outs):
        assert torch.equal(a, b), f'{name}: broadcast mask differs from the per-query copy'
    zo, lo = O.causal_history(q, k, v, mask, scale)
    assert_attention_close(outs[1][0].numpy(), zo, 'z (broadcast mask)')
    assert_lse_close(outs[1][1].numpy(), lo)


def test_width_256_forward_in_both_wave_forms():
    """At width 256 the forward takes two tokens per wave when its grid has more 8-token workgroups than the device
    has CUs, else one: batch row 0 of a call with 8 x (CUs + 8) queries and row 0 alone both match the oracle."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    R, Lq, N = 256, 64, 96
    B = -(-8 * (cus + 8) // Lq)
    q, k, v, mask = case(5, B, Lq, N, R, 'any')
    scale = 1 / math.sqrt(R)
    qt, kt, vt = (torch.tensor(x, device='cuda').to(torch.bfloat16) for x in (q, k, v))
    mt = torch.tensor(mask, device='cuda')
    z_all, l_all = hg.causal_history_gemm(qt, kt, vt, mt, scale, precision='bf16')
    z_one, l_one = hg.causal_history_gemm(qt[:1], kt[:1], vt[:1], mt[:1], scale, precision='bf16')
    zo, lo = O.causal_history(q[:1], k[:1], v[:1], mask[:1], scale)
    for z, lse in ((z_all[:1], l_all[:1]), (z_one, l_one)):
        assert_attention_close(z.float().cpu().numpy(), zo, 'z')
        assert_lse_close(lse.cpu().numpy(), lo)


def test_backward_is_bitwise_repeatable_and_needs_only_what_is_asked():
    q, k, v, mask = case(3, 2, 30, 30, 256, 'benchmark')
    rng = np.random.default_rng(4)
    dz = bf16.round_bf16(rng.standard_normal(q.shape).astype(np.float32))
    dlse = rng.standard_normal((2, 16, 30)).astype(np.float32)
    a = run(q, k, v, mask, 0.1, dz=dz, dlse=dlse)
    b = run(q, k, v, mask, 0.1, dz=dz, dlse=dlse)
    for key in ('z', 'lse', 'dq', 'dk', 'dv'):
        assert np.array_equal(a[key], b[key]), key
    qt = torch.tensor(q, device='cuda').to(torch.bfloat16).requires_grad_(True)
    kt = torch.tensor(k, device='cuda').to(torch.bfloat16)
    vt = torch.tensor(v, device='cuda').to(torch.bfloat16)
    z, lse = hg.causal_history_gemm(qt, kt, vt, torch.tensor(mask, device='cuda'), 0.1, precision='bf16')
    (gq,) = torch.autograd.grad((z.float() * torch.tensor(dz, device='cuda')).sum()
                                + torch.where(torch.isfinite(lse), lse * torch.tensor(dlse, device='cuda'), 0.).sum(),
                                [qt])
    assert np.array_equal(gq.float().cpu().numpy(), a['dq'])


def test_unsplit_key_tiles_match_the_oracle(monkeypatch):
    """dk / dv accumulated by one workgroup per key tile (no row splits, no partial sums)."""
    monkeypatch.setattr(hg, '_key_splits', lambda tiles, device, per_cu=4: 1)
    q, k, v, mask = case(11, 2, 40, 40, 512, 'benchmark')
    rng = np.random.default_rng(12)
    dz = bf16.round_bf16(rng.standard_normal(q.shape).astype(np.float32))
    dlse = rng.standard_normal((2, 16, 40)).astype(np.float32)
    got = run(q, k, v, mask, 0.09, dz=dz, dlse=dlse)
    z, lse = O.causal_history(q, k, v, mask, 0.09)
    dq, dk, dv = O.causal_history_backward(q, k, v, mask, 0.09, lse, dz, dlse)
    assert_grad_close(got['dk'], dk, 'dk')
    assert_grad_close(got['dv'], dv, 'dv')
    assert_grad_close(got['dq'], dq, 'dq')


def test_fp32_inputs_and_transposed_query_view():
    """fp32 leaves (as in the reference benchmark) are rounded to bf16 operands; a [B,H,L,R] -> [B,L,H,R] view works."""
    rng = np.random.default_rng(9)
    B, L, R = 2, 33, 256
    q = torch.randn(B, 16, L, R, device='cuda').transpose(1, 2)
    k, v = torch.randn(B, L, R, device='cuda'), torch.randn(B, L, R, device='cuda')
    mask = torch.tensor(benchmark_mask([L, 20], L), device='cuda')
    z, lse = hg.causal_history_gemm(q, k, v, mask, 0.125, causal=True, precision='bf16')
    assert z.dtype == torch.float32 and lse.shape == (B, 16, L)
    qn, kn, vn = (bf16.round_bf16(t.contiguous().cpu().numpy()) for t in (q, k, v))
    zo, lo = O.causal_history(qn, kn, vn, mask.cpu().numpy(), 0.125)
    assert_attention_close(z.detach().cpu().numpy(), zo, 'z')
    assert_lse_close(lse.detach().cpu().numpy(), lo)
    del rng


def test_rejects_unsupported_shapes_and_precision():
    q = torch.zeros(1, 4, 16, 1024, device='cuda', dtype=torch.bfloat16)
    k = torch.zeros(1, 4, 1024, device='cuda', dtype=torch.bfloat16)
    m = torch.ones(1, 4, 4, dtype=torch.bool, device='cuda')
    with pytest.raises(ValueError, match='widths'):
        hg.causal_history_gemm(q[..., :768], k[..., :768], k[..., :768], m, 1.0, precision='bf16')
    with pytest.raises(ValueError, match='multiple of 16'):   # width 1024 takes whole 16-key groups
        hg.causal_history_gemm(q, k, k, m, 1.0, precision='bf16')
    with pytest.raises(ValueError, match='Unknown precision'):
        hg.causal_history_gemm(q[..., :256], k[..., :256], k[..., :256], m, 1.0, precision='fp16')
    with pytest.raises(ValueError, match='Unknown causal history backend'):
        hg.causal_history_attention(q[..., :256], k[..., :256], k[..., :256], m, 1.0, backend='cuda')
    z, _ = hg.causal_history_attention(q[..., :256], k[..., :256], k[..., :256], m, 1.0, backend='gemm',
                                       precision='bf16')
    assert z.shape == (1, 4, 16, 256)
    with pytest.raises(ValueError, match='Inconsistent'):
        hg.causal_history_gemm(q[..., :256], k[..., :256], k[:, :3, :256], m, 1.0, precision='bf16')


@pytest.mark.parametrize('kind,B,Lq,N', [('benchmark', 2, 48, 48), ('khop', 2, 19, 64), ('any', 3, 29, 96)])
def test_width_1024_forward_matches_the_oracle(kind, B, Lq, N):
    """Width 1024 (the reference benchmark's widest latent): forward on the four-token group kernel over contiguous
    rows with per-token masks (its backward: tests/test_gpu_khop_f32.py)."""
    R = 1024
    q, k, v, mask = case(3 * N + Lq, B, Lq, N, R, kind)
    scale = 1 / math.sqrt(128)
    got = run(q, k, v, mask, scale, need_grad=False)
    z, lse = O.causal_history(q, k, v, mask, scale)
    assert_attention_close(got['z'], z, 'z')
    assert_lse_close(got['lse'], lse)
    empty = ~mask.any(-1)
    assert (got['z'][empty] == 0).all() and np.isneginf(got['lse'].transpose(0, 2, 1)[empty]).all()


def test_transposed_query_view_of_the_reference_benchmark():
    """The reference benchmark's production query layout ([B, H, L, R] storage viewed as [B, L, H, R]) gives the
    same results as contiguous queries (it is made token-linear for the multi-query kernels)."""
    B, L, R = 2, 64, 512
    q, k, v, mask = case(91, B, L, L, R, 'benchmark')
    scale = 1 / math.sqrt(128)
    qt = torch.tensor(q, device='cuda').to(torch.bfloat16)
    qv = qt.transpose(1, 2).contiguous().transpose(1, 2)
    assert qv.stride(0) != L * qv.stride(1)
    kt, vt = (torch.tensor(x, device='cuda').to(torch.bfloat16) for x in (k, v))
    mt = torch.tensor(mask, device='cuda')
    z1, l1 = hg.causal_history_gemm(qt, kt, vt, mt, scale, precision='bf16')
    z2, l2 = hg.causal_history_gemm(qv, kt, vt, mt, scale, precision='bf16')
    assert torch.equal(z1, z2) and torch.equal(l1, l2)


@pytest.mark.parametrize('R,B,Lq,N,kind', [(128, 2, 21, 70, 'khop'), (256, 2, 48, 48, 'benchmark'),
                                           (512, 3, 29, 96, 'any'), (512, 4, 2, 256, 'any')])
def test_bf16_gradients_are_the_rounded_fp32_gradients(R, B, Lq, N, kind):
    """bf16 leaves get gradients written as bf16 by the kernels (no fp32 copy): bitwise the fp32 gradients of the
    same bf16 inputs rounded to nearest even, on the direct, row-range and key-range (one query) paths."""
    q, k, v, mask = case(R + Lq + N, B, Lq, N, R, kind)
    rng = np.random.default_rng(R * Lq)
    dz = torch.tensor(bf16.round_bf16(rng.standard_normal((B, Lq, 16, R)).astype(np.float32)), device='cuda')
    dl = torch.tensor(rng.standard_normal((B, 16, Lq)).astype(np.float32), device='cuda')
    mt = torch.tensor(mask, device='cuda')
    grads = {}
    for dt in (torch.float32, torch.bfloat16):
        leaves = [torch.tensor(x, device='cuda').to(torch.bfloat16).to(dt).requires_grad_(True) for x in (q, k, v)]
        z, lse = hg.causal_history_gemm(*leaves, mt, 0.08, precision='bf16')
        grads[dt] = torch.autograd.grad([z, lse], leaves, [dz.to(dt), dl])
    for name, g32, g16 in zip('qkv', grads[torch.float32], grads[torch.bfloat16]):
        assert g16.dtype == torch.bfloat16
        assert torch.equal(g32.to(torch.bfloat16).view(torch.int16), g16.view(torch.int16)), name
