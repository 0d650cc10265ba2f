"""The HF rolling engine's joint attention (``batched_engine.mixed_attention``, hla/latent/batched_engine.py:154-182)
with the current chunk on the HIP chunk kernels and the latent history on the K-hop kernels, against the oracle's float64 joint softmax (``O.mixed_attention``, one
softmax over the concatenated [history block scores || causal current scores]) and its gradient
(``O.mixed_attention_backward``), both pinned on the CPU by per-query brute force and finite differences.

Bars: outputs of valid queries within the attention tolerance (max-abs 2e-2, rel-L2 5e-3) of the oracle;
gradients of q, k, v, the packed history rows and the A / B readers within relative L2 2e-2 (bf16 operands of every
kernel product). The latent module is a stand-in with the shapes and field layout of ``register.LatentLayer`` (q
absorption, latent RoPE by ``rope_latent``, packed rows ``[K 512 | V 512 | K1 256 | V1 256]``).
"""
import importlib
import math

import numpy as np
import pytest
import torch

from oracle import s6_oracle as O
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
    elif valid_kind == 'left20':
        valid[0, :20] = False                                   # a 16-row block of padding and valid queries whose
                                                                # first visible key lies in the block's own tile
    elif valid_kind == 'holes':
        valid[:, ::5] = False
        valid[:, 0] = True
    cos, sin = rope_tables(B, n, torch.tensor([sum(sizes)] * B, device='cuda'), gen)
    return Latent(gen, torch.bfloat16), q, k, v, cos, sin, valid, blocks, masks


def f64(t):
    return t.detach().double().cpu().numpy()


@pytest.mark.parametrize('loop', [0, 2])
@pytest.mark.parametrize('B,n,sizes,valid_kind', [(2, 16, (160,), 'all'), (3, 9, (64, 48), 'left'),
                                                  (2, 33, (96, 37), 'holes'), (2, 7, (), 'left'),
                                                  (2, 130, (), 'holes'), (1, 300, (80,), 'left'),
                                                  (2, 48, (64,), 'left20')])
def test_mixed_attention_matches_the_oracle(loop, B, n, sizes, valid_kind):
    sl, q, k, v, cos, sin, valid, blocks, masks = make_case(11 * n + loop, B, n, sizes, loop, valid_kind)
    print(f'case loop={loop} B={B} n={n} blocks={sizes} valid={valid_kind}', flush=True)
    ours = [x.clone().requires_grad_(True) for x in (q, k, v, *blocks)]
    sl.A[loop].requires_grad_(True)
    sl.B[loop].requires_grad_(True)
    out = be.mixed_attention(sl, loop, *ours[:3], cos, sin, valid, tuple(ours[3:]), tuple(masks))
    assert out.dtype == torch.bfloat16 and out.shape == (B, HEADS, n, HD)
    fields = [sl.fields(loop, f64(blk)) for blk in blocks]
    args = (f64(q), f64(k), f64(v), f64(cos), f64(sin), valid.cpu().numpy(), [a for a, _ in fields],
            [b for _, b in fields], [m.cpu().numpy() for m in masks], f64(sl.A[loop]), f64(sl.B[loop]), 1 / math.sqrt(HD))
    want = O.mixed_attention(*args)
    vq = valid.cpu().numpy()
    got_v = out.detach().float().cpu().numpy().transpose(0, 2, 1, 3)[vq]
    assert_attention_close(got_v, want.transpose(0, 2, 1, 3)[vq], 'mixed attention')
    g = torch.randn(out.shape, generator=torch.Generator(device='cuda').manual_seed(5), device='cuda')
    g = g * valid[:, None, :, None]                             # the loss reads valid queries only
    leaves = ours + ([sl.A[loop], sl.B[loop]] if blocks else [])
    grads = torch.autograd.grad(out.float(), leaves, g)
    wants = O.mixed_attention_backward(*args, f64(g))
    packed = []                                                 # block gradients: the loop's K / V fields of the rows
    for i, blk in enumerate(blocks):
        dblk = np.zeros(blk.shape)
        dk_, dv_ = sl.fields(loop, dblk)
        dk_[...] = wants['hist_k'][i]
        dv_[...] = wants['hist_v'][i]
        packed.append(dblk)
    want_list = [wants['q'], wants['k'], wants['v'], *packed] + ([wants['A'], wants['B']] if blocks else [])
    names = ['q', 'k', 'v'] + [f'block{i}' for i in range(len(blocks))] + (['A', 'B'] if blocks else [])
    for name, a, b in zip(names, grads, want_list):
        a = a.double().cpu().numpy()
        assert np.isfinite(a).all(), name
        r = rel_l2(a, b)
        assert r <= 2e-2, f'{name}: rel-L2 {r:.3e}'


@pytest.mark.parametrize('trig', [torch.float32, torch.bfloat16])
def test_chunk_rope_kernels_match_torch_bitwise(trig):
    """The RoPE kernels of the chunk's q / k equal torch's ``apply_rope(x, cos, sin).to(bf16)`` bit for bit (fp32 or
    bf16 tables, positions from 7 to 2000, a ragged chunk of 37 rows), and the backward kernel equals autograd's
    gradient of ``apply_rope`` for a bf16 x bit for bit."""
    gen = torch.Generator(device='cuda').manual_seed(3)
    B, n = 3, 37
    print(f'case rope trig={trig}', flush=True)
    q, k = (torch.randn(B, HEADS, n, HD, generator=gen, device='cuda').to(torch.bfloat16) for _ in range(2))
    cos, sin = rope_tables(B, n, torch.tensor([100, 2000, 7], device='cuda'), gen)
    cos, sin = cos.to(trig), sin.to(trig)
    c, s = be._trig(cos, sin, B, n, HD)
    qr, kr = torch.empty_like(q), torch.empty_like(k)
    be._rope_call('hla_s6_rope_rows_forward', [q, k], [qr, kr], c, s)
    for x, y in ((q, qr), (k, kr)):
        assert torch.equal(y, be.apply_rope(x, cos, sin).to(torch.bfloat16))
    x = q.clone().requires_grad_(True)
    out = be.apply_rope(x, cos, sin)
    dy = torch.randn(out.shape, generator=gen, device='cuda').to(out.dtype)
    want, = torch.autograd.grad(out, x, dy)
    dx = torch.empty_like(q)
    be._rope_call('hla_s6_rope_rows_backward', [dy.float().contiguous()], [dx], c, s)
    assert want.dtype == torch.bfloat16 and torch.equal(dx, want)


def test_mixed_attention_at_the_bench_shape():
    """The benchmark's shape: 8 rows of a 256-token loop-2 chunk (row 0 left-padded by 20 tokens) over history
    blocks of 2,048 and 256 packed rows, 80 % of them visible. Rows 0 and 5 (every head, every valid query) against
    the oracle's joint softmax (a row's output depends on that row's inputs only); the gradients are checked at the
    smaller shapes above, whose oracle backward finishes in seconds."""
    B, n, sizes, loop = 8, 256, (2048, 256), 2
    sl, q, k, v, cos, sin, valid, blocks, masks = make_case(97, B, n, sizes, loop, 'all')
    valid[0, :20] = False
    print('case bench shape B=8 n=256 blocks=(2048, 256) loop=2', flush=True)
    with torch.no_grad():
        out = be.mixed_attention(sl, loop, q, k, v, cos, sin, valid, tuple(blocks), tuple(masks))
    rows = [0, 5]
    pick = lambda t: t.detach()[rows].double().cpu().numpy()
    fields = [sl.fields(loop, pick(blk)) for blk in blocks]
    args = (pick(q), pick(k), pick(v), pick(cos), pick(sin), valid[rows].cpu().numpy(), [a for a, _ in fields],
            [b for _, b in fields], [m[rows].cpu().numpy() for m in masks], f64(sl.A[loop]), f64(sl.B[loop]),
            1 / math.sqrt(HD))
    want = O.mixed_attention(*args, dtype=np.float32)
    vq = valid[rows].cpu().numpy()
    got = out[rows].float().cpu().numpy().transpose(0, 2, 1, 3)[vq]
    assert_attention_close(got, want.transpose(0, 2, 1, 3)[vq], 'mixed attention at the bench shape')
