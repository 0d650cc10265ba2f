"""Single-query history attention over contiguous rows with a key mask (``history_gemm.history_attention``, the
interface of hla/latent/fused_history.py:49-54 used by the HF rolling engine) against the float64 oracle
(``oracle.s6_oracle.single_history`` / ``single_history_backward``, restating fused_history.py:11-20 and
history_kernels.py:11-81) on bf16-rounded inputs.

Bars: z within the attention tolerance (max-abs 2e-2, rel-L2 5e-3) and lse within 1e-3 of the oracle; rows with no
visible key give exactly z = 0 and lse = -inf; gradients within relative L2 1e-2 per tensor and max-abs 2e-2 of
the largest magnitude; one split and several splits agree within the attention tolerance; results are bitwise
repeatable.
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


def case(seed, B, N, R, kind):
    rng = np.random.default_rng(seed)
    q = bf16.round_bf16(rng.standard_normal((B, 16, R)).astype(np.float32))
    k = bf16.round_bf16(rng.standard_normal((B, N, R)).astype(np.float32))
    v = bf16.round_bf16(rng.standard_normal((B, N, R)).astype(np.float32))
    if kind == 'prefix':                       # valid history lengths (the rolling engine's padding masks)
        mask = np.arange(N)[None] < np.maximum(1, (N * (1 - 0.3 * np.arange(B) / max(1, B - 1)))).astype(int)[:, None]
    else:                                      # arbitrary holes
        mask = rng.random((B, N)) < 0.4
    if B > 1:
        mask[1] = False                        # a row with no visible key
    if B > 2:
        mask[2] = True                         # a row that sees every key
    return q, k, v, mask


def run(q, k, v, mask, scale, splits=None, monkeypatch=None, dz=None, dlse=None):
    if splits is not None:
        monkeypatch.setattr(hg.s6_ops, 'mi355x_kv_splits', lambda *a, **kw: splits)
    grad = dz is not None
    qt, kt, vt = (torch.tensor(x, device='cuda').to(torch.bfloat16).requires_grad_(grad) for x in (q, k, v))
    mt = torch.tensor(mask, device='cuda')
    z, lse = hg.history_attention(qt, kt, vt, mt, scale)
    out = {'z': z.detach().float().cpu().numpy(), 'lse': lse.detach().cpu().numpy()}
    if grad:
        dzt = torch.tensor(dz, device='cuda').to(torch.bfloat16)
        dlt = torch.tensor(dlse, device='cuda', dtype=torch.float32)
        g = torch.autograd.grad([z, lse], [qt, kt, vt], [dzt, dlt])
        out.update(dq=g[0].float().cpu().numpy(), dk=g[1].float().cpu().numpy(), dv=g[2].float().cpu().numpy())
    return out


def assert_grad_close(got, want, what):
    assert np.isfinite(got).all(), f'{what}: non-finite'
    r = rel_l2(got, want)
    err = float(np.abs(got - want).max())
    assert r <= GRAD_REL, f'{what}: rel-L2 {r:.3e} > {GRAD_REL}'
    assert err <= 2e-2 * max(1.0, float(np.abs(want).max())), f'{what}: max-abs {err:.3e}'


def check_forward(got, q, k, v, mask, scale):
    z, lse = O.single_history(q, k, v, mask, scale)
    assert_attention_close(got['z'], z, 'z')
    assert_lse_close(got['lse'], lse)
    empty = ~mask.any(-1)
    assert (got['z'][empty] == 0).all() and np.isneginf(got['lse'][empty]).all()
    return z, lse


@pytest.mark.parametrize('R', [128, 256, 512, 1024])
@pytest.mark.parametrize('kind,B,N', [('any', 3, 37), ('prefix', 4, 300), ('any', 3, 1029)])
@pytest.mark.parametrize('splits', [1, 5])
def test_forward_matches_the_oracle(R, kind, B, N, splits, monkeypatch):
    """Mask rows of odd length (byte loads) and of a multiple of 4 (word loads), one split (direct output) and five
    (partials reduced by the combine kernel, with slots that see no key)."""
    q, k, v, mask = case(R + N + splits, B, N, R, kind)
    got = run(q, k, v, mask, 1 / math.sqrt(128), splits, monkeypatch)
    check_forward(got, q, k, v, mask, 1 / math.sqrt(128))


def test_forward_with_the_default_split_policy_at_a_long_history():
    B, N, R = 8, 4100, 512
    q, k, v, mask = case(11, B, N, R, 'any')
    got = run(q, k, v, mask, 0.09)
    check_forward(got, q, k, v, mask, 0.09)


@pytest.mark.parametrize('R', [128, 256, 512])
@pytest.mark.parametrize('kind,B,N', [('any', 3, 45), ('prefix', 3, 96)])
def test_forward_and_backward_match_the_oracle(R, kind, B, N, monkeypatch):
    q, k, v, mask = case(3 * R + N, B, N, R, kind)
    scale = 1 / math.sqrt(128)
    rng = np.random.default_rng(R * N)
    dz = bf16.round_bf16(rng.standard_normal((B, 16, R)).astype(np.float32))
    dlse = rng.standard_normal((B, 16)).astype(np.float32)
    got = run(q, k, v, mask, scale, 3, monkeypatch, dz=dz, dlse=dlse)
    z, lse = check_forward(got, q, k, v, mask, scale)
    dq, dk, dv = O.single_history_backward(q, k, v, mask, scale, lse, dz, dlse)
    assert_grad_close(got['dq'], dq, 'dq')
    assert_grad_close(got['dk'], dk, 'dk')
    assert_grad_close(got['dv'], dv, 'dv')
    assert (got['dq'][~mask.any(-1)] == 0).all()
    hidden = ~mask.any(0)                      # keys no row sees get no gradient
    assert (got['dk'][:, hidden] == 0).all() and (got['dv'][:, hidden] == 0).all()


def test_c_abi_splits_agree_and_repeat():
    """Through the C ABI: a mask view whose rows start off 4-byte boundaries, one split against seven, and a second
    call bitwise equal to the first."""
    B, N, R = 3, 200, 512
    q, k, v, mask = case(5, B, N, R, 'any')
    lib = hg._lib
    qt, kt, vt = (torch.tensor(x, device='cuda').to(torch.bfloat16) for x in (q, k, v))
    wide = torch.zeros(B, N + 3, dtype=torch.uint8, device='cuda')
    wide[:, 1:N + 1] = torch.tensor(mask, device='cuda').to(torch.uint8)
    m8 = wide[:, 1:N + 1]
    st = lib.stream(qt.device)
    bound = torch.empty(B, dtype=torch.int32, device='cuda')
    lib.call('hla_s6_khop_bounds', lib.ptr(m8), m8.stride(0), N, B, 1, N, lib.ptr(bound), st)
    assert bound.cpu().tolist() == [int(np.flatnonzero(r)[-1]) + 1 if r.any() else 0 for r in mask]
    outs = []
    for splits in (1, 7, 7):
        ws = torch.empty(B * splits * 16 * (R + 1), dtype=torch.float32, device='cuda')
        z = torch.empty(B, 16, R, dtype=torch.bfloat16, device='cuda')
        lse = torch.empty(B, 16, dtype=torch.float32, device='cuda')
        lib.call('hla_s6_masked_history', lib.ptr(qt), qt.stride(0), qt.stride(1), lib.ptr(kt), lib.ptr(vt),
                 kt.stride(0), kt.stride(1), lib.ptr(m8), m8.stride(0), lib.ptr(bound), B, N, 16, R, 0.07, splits,
                 lib.ptr(ws), ws.numel(), lib.ptr(z), z.stride(0), z.stride(1), lib.ptr(lse), st)
        torch.cuda.synchronize()
        outs.append((z.float().cpu().numpy(), lse.cpu().numpy()))
    zo, lo = O.single_history(q, k, v, mask, 0.07)
    for z, lse in outs:
        assert_attention_close(z, zo, 'z')
        assert_lse_close(lse, lo)
    assert_attention_close(outs[0][0], outs[1][0], 'one split vs seven')
    assert (outs[1][0] == outs[2][0]).all() and (outs[1][1] == outs[2][1]).all()


def test_errors_match_the_reference():
    q = torch.zeros(2, 16, 256, dtype=torch.bfloat16, device='cuda')
    k = torch.zeros(2, 5, 256, dtype=torch.bfloat16, device='cuda')
    mask = torch.ones(2, 5, dtype=torch.bool, device='cuda')
    with pytest.raises(ValueError, match='Expected Q'):
        hg.history_attention(q, k, k[:, :4], mask, 1.0)
    with pytest.raises(ValueError, match='Expected Q'):
        hg.history_attention(q, k, k, mask[:, :4], 1.0)
    with pytest.raises(ValueError, match='storage row'):
        hg.history_attention(q, k[:, :0], k[:, :0], mask[:, :0], 1.0)


@pytest.mark.parametrize('N', [1, 5, 16, 17, 100, 1000, 4099])
@pytest.mark.parametrize('offset', [0, 1, 3, 9])
def test_key_bounds_of_mask_rows(N, offset):
    """hla_s6_khop_bounds: 1 + the last nonzero byte of every mask row (any nonzero value is visible), for rows that
    start anywhere relative to 16-byte boundaries; all-zero rows give 0."""
    rng = np.random.default_rng(N * 10 + offset)
    B, Lq = 3, 7
    rows = np.zeros((B * Lq, N), np.uint8)
    for r in range(B * Lq):
        kind = r % 5
        if kind == 1:
            rows[r, rng.integers(0, N)] = rng.integers(1, 256)
        elif kind == 2:
            rows[r] = (rng.random(N) < 0.1) * rng.integers(1, 256, N)
        elif kind == 3:
            rows[r, N - 1] = 2
        elif kind == 4:
            rows[r, 0] = 255
    stride = N + 5
    flat = np.zeros(offset + B * Lq * stride + 16, np.uint8)
    for r in range(B * Lq):
        flat[offset + r * stride: offset + r * stride + N] = rows[r]
    buf = torch.tensor(flat, device='cuda')
    m8 = buf[offset:]
    bound = torch.empty(B * Lq, dtype=torch.int32, device='cuda')
    lib = hg._lib
    lib.call('hla_s6_khop_bounds', lib.ptr(m8), Lq * stride, stride, B, Lq, N, lib.ptr(bound), lib.stream(buf.device))
    want = [int(np.flatnonzero(r)[-1]) + 1 if r.any() else 0 for r in rows]
    assert bound.cpu().tolist() == want


def test_fields_of_packed_rows_without_copies():
    """K and V as the fields of the HF engine's packed rows [B, N, 1536] (row stride 1536): the same results as
    contiguous copies, forward and gradients."""
    rng = np.random.default_rng(77)
    B, N, R = 3, 160, 512
    packed = bf16.round_bf16(rng.standard_normal((B, N, 1536)).astype(np.float32))
    q = bf16.round_bf16(rng.standard_normal((B, 16, R)).astype(np.float32))
    mask = rng.random((B, N)) < 0.5
    pt = torch.tensor(packed, device='cuda').to(torch.bfloat16).requires_grad_(True)
    qt = torch.tensor(q, device='cuda').to(torch.bfloat16)
    mt = torch.tensor(mask, device='cuda')
    z, lse = hg.history_attention(qt, pt[..., :R], pt[..., R:2 * R], mt, 0.05)
    (gp,) = torch.autograd.grad([z], [pt], [torch.ones_like(z)])
    kc = pt.detach()[..., :R].contiguous().requires_grad_(True)
    vc = pt.detach()[..., R:2 * R].contiguous().requires_grad_(True)
    z2, lse2 = hg.history_attention(qt, kc, vc, mt, 0.05)
    gk, gv = torch.autograd.grad([z2], [kc, vc], [torch.ones_like(z2)])
    assert torch.equal(z, z2) and torch.equal(lse, lse2)
    assert torch.equal(gp[..., :R], gk) and torch.equal(gp[..., R:2 * R], gv)
    assert (gp[..., 2 * R:] == 0).all()
