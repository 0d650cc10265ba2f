"""The HF rolling engine's joint attention (``batched_engine.mixed_attention``, hla/latent/batched_engine.py:154-182)
with the latent history on the K-hop kernels, against a float32 torch restatement of the reference's dense joint
softmax (one softmax over the concatenated [history block scores || causal current scores], probabilities times the
latent values, then the B reader), outputs and gradients.

Bars: outputs of valid queries within the attention tolerance (max-abs 2e-2, rel-L2 5e-3) of the float32 form;
gradients of q, k, v and the packed history rows within relative L2 2e-2 (bf16 operands of every kernel product).
The latent module is a stand-in with the shapes and field layout of ``register.LatentLayer`` (q absorption, latent
RoPE by ``rope_latent``, packed rows ``[K 512 | V 512 | K1 256 | V1 256]``).
"""
import importlib
import math

import numpy as np
import pytest
import torch

from s6util import assert_attention_close, rel_l2

pytestmark = pytest.mark.gpu

be = importlib.import_module('hybrid-latent-attention_amd.batched_engine')

HEADS, HD, RANK, RANK1 = 16, 128, 512, 256


def rope_latent(cos, sin, width):
    idx = torch.arange(width // 2, device=cos.device) % (cos.shape[-1] // 2)
    return torch.cat((cos[..., idx], cos[..., idx]), -1), torch.cat((sin[..., idx], sin[..., idx]), -1)


class Latent:
    """readers / query / fields of the latent module for one layer (matmul against contiguous readers)."""

    def __init__(self, gen, dtype):
        w = lambda *s: (torch.randn(*s, generator=gen, device='cuda') / math.sqrt(s[-2])).to(dtype)
        self.head_dim = HD
        self.A = [w(HEADS, HD, RANK1)] + [w(HEADS, HD, RANK) for _ in range(3)]
        self.B = [w(HEADS, RANK1, HD)] + [w(HEADS, RANK, HD) for _ in range(3)]

    def cast(self, dtype):
        other = Latent.__new__(Latent)
        other.head_dim = HD
        other.A = [a.to(dtype) for a in self.A]
        other.B = [b.to(dtype) for b in self.B]
        return other

    def readers(self, loop):
        return self.A[loop], self.B[loop], RANK1 if loop == 0 else RANK

    def query(self, loop, q, cos, sin):
        A, _, rank = self.readers(loop)
        c, s = rope_latent(cos, sin, rank)
        # (float32 product: the bf16 backward would take a transposed right operand)
        return be.apply_rope(torch.matmul(q.float(), A.float()[None]).to(q.dtype), c, s)

    def fields(self, loop, packed):
        if loop == 0:
            row = packed[..., 2 * RANK:]
            return row[..., :RANK1], row[..., RANK1:]
        return packed[..., :RANK], packed[..., RANK:2 * RANK]


def reference(sl, loop, q, k, v, cos, sin, valid, blocks, masks):
    """The reference's dense form in float32: one softmax over [block scores..., current scores]."""
    scale = 1 / math.sqrt(HD)
    qr, kr = be.apply_rope(q, cos, sin), be.apply_rope(k, cos, sin)
    n = valid.shape[1]
    visible = valid[:, None, None, :] & torch.ones(n, n, device='cuda', dtype=torch.bool).tril()
    visible = visible | ~valid[:, None, :, None]
    current = (qr @ kr.transpose(-1, -2).contiguous()) * scale
    scores, values = [], []
    qc = sl.query(loop, q, cos, sin)
    for block, mask in zip(blocks, masks):
        ck, cv = sl.fields(loop, block)
        s = torch.matmul(qc, ck.transpose(-1, -2).contiguous()[:, None]) * scale
        scores.append(s.masked_fill(~mask[:, None, None, :], float('-inf')))
        values.append(cv)
    scores.append(current.masked_fill(~visible, float('-inf')))
    probs = torch.softmax(torch.cat(scores, -1), -1)
    out = probs[..., -n:] @ v
    if blocks:
        z, off = 0, 0
        for cv in values:
            w = cv.shape[1]
            z = z + torch.matmul(probs[..., off:off + w], cv[:, None])
            off += w
        out = out + torch.matmul(z, sl.readers(loop)[1][None])
    return out


def rope_tables(B, n, start, gen):
    pos = start[:, None] + torch.arange(n, device='cuda')[None]
    inv = 1.0 / (1e6 ** (torch.arange(0, HD, 2, device='cuda').float() / HD))
    ang = pos[..., None].float() * inv
    emb = torch.cat((ang, ang), -1)
    return emb.cos(), emb.sin()


def make_case(seed, B, n, sizes, loop, valid_kind):
    gen = torch.Generator(device='cuda').manual_seed(seed)
    bf = lambda *s: torch.randn(*s, generator=gen, device='cuda').to(torch.bfloat16)
    q, k, v = bf(B, HEADS, n, HD), bf(B, HEADS, n, HD), bf(B, HEADS, n, HD)
    blocks = [bf(B, N, 2 * RANK + 2 * RANK1) * 0.5 for N in sizes]
    masks = []
    for i, N in enumerate(sizes):
        m = torch.rand(B, N, generator=gen, device='cuda') < 0.8
        if B > 1 and i == 0:
            m[1] = False                                       # a row that sees nothing of this block
        masks.append(m)
    valid = torch.ones(B, n, dtype=torch.bool, device='cuda')
    if valid_kind == 'left':
        valid[0, :3] = False                                    # left padding
    elif valid_kind == 'holes':
        valid[:, ::5] = False
        valid[:, 0] = True
    cos, sin = rope_tables(B, n, torch.tensor([sum(sizes)] * B, device='cuda'), gen)
    return Latent(gen, torch.bfloat16), q, k, v, cos, sin, valid, blocks, masks


@pytest.mark.parametrize('loop', [0, 2])
@pytest.mark.parametrize('B,n,sizes,valid_kind', [(2, 16, (160,), 'all'), (3, 9, (64, 48), 'left'),
                                                  (2, 33, (96, 37), 'holes'), (2, 7, (), 'left')])
def test_mixed_attention_matches_the_dense_joint_softmax(loop, B, n, sizes, valid_kind):
    sl, q, k, v, cos, sin, valid, blocks, masks = make_case(11 * n + loop, B, n, sizes, loop, valid_kind)
    leaves = [q, k, v, *blocks]
    ours = [x.clone().requires_grad_(True) for x in leaves]
    ref = [x.float().clone().requires_grad_(True) for x in leaves]
    out = be.mixed_attention(sl, loop, *ours[:3], cos, sin, valid, tuple(ours[3:]), tuple(masks))
    want = reference(sl.cast(torch.float32), loop, *ref[:3], cos, sin, valid, tuple(ref[3:]), tuple(masks))
    assert out.dtype == torch.bfloat16 and out.shape == (B, HEADS, n, HD)
    vq = valid.cpu().numpy()
    got_v = out.detach().float().cpu().numpy().transpose(0, 2, 1, 3)[vq]
    want_v = want.detach().cpu().numpy().transpose(0, 2, 1, 3)[vq]
    assert_attention_close(got_v, want_v, 'mixed attention')
    g = torch.randn(out.shape, generator=torch.Generator(device='cuda').manual_seed(5), device='cuda')
    g = g * valid[:, None, :, None]                             # the loss reads valid queries only
    grads = torch.autograd.grad(out.float(), ours, g)
    wants = torch.autograd.grad(want, ref, g)
    for name, a, b in zip(['q', 'k', 'v'] + [f'block{i}' for i in range(len(blocks))], grads, wants):
        a, b = a.float().cpu().numpy(), b.cpu().numpy()
        assert np.isfinite(a).all(), name
        r = rel_l2(a, b)
        assert r <= 2e-2, f'{name}: rel-L2 {r:.3e}'
