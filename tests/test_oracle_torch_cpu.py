"""The torch-on-CPU restatement (the benchmark's CPU baseline) against the numpy oracle: decode steps with ragged
histories, empty histories, histories inside the window and padding rows, and chunked-prefill steps, both latent
widths. They agree to float32 summation order and the shared bf16 rounding points; a window one row short, a
missing B_t or a non-causal chunk would miss by orders of magnitude more."""
import math

import numpy as np
import pytest
import torch

from oracle import bf16
from oracle import s6_oracle as O
from oracle import torch_cpu as TC
from s6util import assert_attention_close, latent_cache_bits, random_bits

H, D, W, BLOCK = 16, 128, 32, 16
SCALE = 1 / math.sqrt(D)


def cpu_bf16(bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16)


@pytest.mark.parametrize('w', [512, 256])
def test_decode_matches_the_numpy_oracle(w):
    rng = np.random.default_rng(11 + w)
    hist = np.array([700, 0, 20, 33, 1500, 64])
    R, pad = len(hist), 2
    T = R + pad
    seq = (hist + 1).astype(np.int32)
    qsl = np.arange(R + 1, dtype=np.int32)
    cols = -(-int(seq.max()) // BLOCK)
    nb = R * cols + 4
    lt = rng.permutation(np.arange(1, nb))[:R * cols].reshape(R, cols).astype(np.int32)
    et = rng.permutation(np.arange(1, nb))[:R * cols].reshape(R, cols).astype(np.int32)
    lat = latent_cache_bits(rng, nb, BLOCK, w)
    ex = random_bits(rng, (nb, H, BLOCK, 2 * D))
    B = random_bits(rng, (H, w, D), 1 / math.sqrt(2048))
    q_lat = random_bits(rng, (T, H, w), 1 / math.sqrt(w))
    q_rope = random_bits(rng, (T, H, D))
    req, valid, c, cl = O.step_context(qsl, seq, T, W)
    latf, exf = bf16.to_f32(lat), bf16.to_f32(ex)
    want = O.attend_decode(bf16.to_f32(q_lat), bf16.to_f32(q_rope), bf16.to_f32(B), latf[..., :w], latf[..., w:],
                           lt[req], cl, exf[..., :D], exf[..., D:], et, qsl, seq, W, SCALE, ~valid)
    got = TC.attend_decode(cpu_bf16(q_lat), cpu_bf16(q_rope), cpu_bf16(B), cpu_bf16(lat), torch.from_numpy(lt[req]),
                           torch.from_numpy(cl), cpu_bf16(ex), torch.from_numpy(et), torch.from_numpy(req),
                           torch.from_numpy(seq), W, SCALE, torch.from_numpy(~valid))
    assert_attention_close(got.float().numpy(), want, max_abs=1.6e-2, rel=1e-3)
    assert (got[R:] == 0).all()


@pytest.mark.parametrize('w', [512, 256])
def test_chunk_matches_the_numpy_oracle(w):
    rng = np.random.default_rng(21 + w)
    lens, hist = np.array([5, 17, 1, 9]), np.array([900, 40, 0, 10])
    R = len(lens)
    qsl = np.concatenate(([0], np.cumsum(lens))).astype(np.int32)
    T = int(qsl[-1]) + 1
    seq = (hist + lens).astype(np.int32)
    cols = -(-int(seq.max()) // BLOCK)
    nb = R * cols + 4
    lt = rng.permutation(np.arange(1, nb))[:R * cols].reshape(R, cols).astype(np.int32)
    et = rng.permutation(np.arange(1, nb))[:R * cols].reshape(R, cols).astype(np.int32)
    lat = latent_cache_bits(rng, nb, BLOCK, w)
    ex = random_bits(rng, (nb, H, BLOCK, 2 * D))
    B = random_bits(rng, (H, w, D), 1 / math.sqrt(2048))
    q_lat = random_bits(rng, (T, H, w), 1 / math.sqrt(w))
    q_rope, k_rope, v = (random_bits(rng, (T, H, D)) for _ in range(3))
    req, valid, c, cl = O.step_context(qsl, seq, T, W)
    latf, exf = bf16.to_f32(lat), bf16.to_f32(ex)
    want = O.attend_chunk(bf16.to_f32(q_lat), bf16.to_f32(q_rope), bf16.to_f32(k_rope), bf16.to_f32(v),
                          bf16.to_f32(B), latf[..., :w], latf[..., w:], {'latent': lt[req], 'exact': et[req]}, c, cl,
                          qsl, W, SCALE, ~valid, exf[..., :D], exf[..., D:])
    ctx_req, cl_req = hist, np.maximum(hist - W, 0)
    got = TC.attend_chunk(cpu_bf16(q_lat), cpu_bf16(q_rope), cpu_bf16(k_rope), cpu_bf16(v), cpu_bf16(B),
                          cpu_bf16(lat), torch.from_numpy(lt), qsl, ctx_req, cl_req, cpu_bf16(ex),
                          torch.from_numpy(et), W, SCALE, torch.from_numpy(~valid))
    assert_attention_close(got.float().numpy(), want, max_abs=1.6e-2, rel=1e-3)
    assert (got[~valid] == 0).all()


def test_latent_query_matches_the_numpy_oracle():
    """A_t product and latent RoPE with torch's bf16 rounding points: bit-identical to the oracle's rounding."""
    rng = np.random.default_rng(31)
    T, w = 9, 512
    inv = O.latent_inv_freq(D, 1e6)
    table = bf16.round_bf16(O.latent_rope_table(4096, inv, w).astype(np.float32))
    positions = rng.integers(0, 4096, T)
    q = random_bits(rng, (T, H, D))
    A = random_bits(rng, (H, D, w), 1 / math.sqrt(2048))
    want = O.latent_query(bf16.to_f32(q), bf16.to_f32(A), positions, table)
    rows = cpu_bf16(bf16.from_f32(table[positions]))
    got = TC.latent_query(cpu_bf16(q), cpu_bf16(A), rows)
    assert got.dtype == torch.bfloat16
    np.testing.assert_array_equal(got.float().numpy(), want)
