"""Shared helpers of the test-suite: bf16 transfers between numpy (oracle) and torch (device), tolerances."""
from __future__ import annotations

import math

import numpy as np
import torch

from oracle import bf16

# Tolerances of the hot-path parity bar: attention output vs the fp32 oracle, LSE vs the fp32 oracle.
MAX_ABS = 2e-2
REL_L2 = 5e-3
LSE_ATOL = 1e-3

POS_INF_BF16 = 0x7F80
NAN_BF16 = 0x7FC0


def dev_bf16(bits: np.ndarray, device='cuda') -> torch.Tensor:
    """uint16 bf16 bit patterns -> torch bfloat16 tensor on ``device``."""
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).to(device)


def host_f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def dev_i32(a, device='cuda') -> torch.Tensor:
    return torch.as_tensor(np.asarray(a, dtype=np.int32), device=device)


def dev_i64(a, device='cuda') -> torch.Tensor:
    return torch.as_tensor(np.asarray(a, dtype=np.int64), device=device)


def rel_l2(a, b) -> float:
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    den = math.sqrt(float((b * b).sum()))
    return math.sqrt(float(((a - b) ** 2).sum())) / (den if den > 0 else 1.0)


def assert_attention_close(got, want, what='o', max_abs=MAX_ABS, rel=REL_L2):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    assert got.shape == want.shape, (what, got.shape, want.shape)
    assert np.isfinite(got).all(), f'{what}: non-finite values in the kernel output'
    err = float(np.abs(got - want).max()) if got.size else 0.0
    r = rel_l2(got, want)
    assert err <= max_abs, f'{what}: max-abs {err:.3e} > {max_abs}'
    assert r <= rel, f'{what}: rel-L2 {r:.3e} > {rel}'


def assert_lse_close(got, want, atol=LSE_ATOL, what='lse'):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    assert got.shape == want.shape, (what, got.shape, want.shape)
    assert not np.isnan(got).any(), f'{what}: NaN'
    inf_g, inf_w = np.isneginf(got), np.isneginf(want)
    assert (inf_g == inf_w).all(), f'{what}: -inf pattern differs at {np.argwhere(inf_g != inf_w)[:5].tolist()}'
    fin = ~inf_w
    if fin.any():
        err = float(np.abs(got[fin] - want[fin]).max())
        assert err <= atol, f'{what}: max-abs {err:.3e} > {atol}'


def random_bits(rng, shape, std=1.0):
    return bf16.random_bf16(rng, shape, std)


def latent_cache_bits(rng, num_blocks, block, width, poison_null=True):
    """Paged MQA latent cache [num_blocks, 1, block, 2w] as bf16 bits; block 0 is a +inf-poisoned null page."""
    bits = random_bits(rng, (num_blocks, 1, block, 2 * width))
    if poison_null:
        bits[0] = POS_INF_BF16
    return bits


def token_tables(rng, ctx, block, num_blocks, cols, distinct=False):
    """Per-token block tables: random pages in [1, num_blocks) for the columns each row needs, 0 (the poisoned
    null page) in the stale columns. ``distinct`` gives every row its own pages (no page shared by two rows)."""
    ctx = np.asarray(ctx)
    table = np.zeros((len(ctx), cols), np.int32)
    if distinct:
        pool = rng.permutation(np.arange(1, num_blocks))
        used = 0
    for t, n in enumerate(ctx):
        need = -(-int(n) // block)
        assert need <= cols
        if distinct:
            table[t, :need] = pool[used:used + need]
            used += need
        else:
            table[t, :need] = rng.integers(1, num_blocks, need)
    return table


class FakeLatentLayer:
    """The reader interface of a LatentLayer (hla/latent/register.py:63-66): per loop (A, B, width)."""

    def __init__(self, A1, B1, A, B, loops=4):
        self.A1, self.B1, self.A, self.B = A1, B1, A, B
        self.rank1, self.rank, self.loops = A1.shape[-1], A[0].shape[-1], loops

    def readers(self, loop):
        if loop == 0:
            return self.A1, self.B1, self.rank1
        return self.A[loop - 1], self.B[loop - 1], self.rank
