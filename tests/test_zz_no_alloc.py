"""hla_s6_attend_decode_static (the fused decode step with its buffers in the library's static device array) against
hla_s6_attend_decode (caller-allocated workspace, plan and intermediates), through the C ABI: two calls in a row, the
second smaller (fewer rows, fewer slots, the narrower latent), each bitwise equal to the allocating entry point
(same kernels, same split plan); and sizes past the array refused before any launch."""
import importlib
import math

import numpy as np
import pytest
import torch

from s6util import FakeLatentLayer

pytestmark = pytest.mark.gpu
H, D, W, BLOCK = 16, 128, 32, 16
SCALE = 1 / math.sqrt(D)

lib = importlib.import_module('hybrid-latent-attention_amd._lib')
layer = importlib.import_module('hybrid-latent-attention_amd.s6_layer')
ops = importlib.import_module('hybrid-latent-attention_amd.s6_ops')


class Step:
    """One step of ``len(hist)`` requests (+ ``pad`` padding rows) at one latent width, caches on the device: decode
    (one token per request), or ``lens[r]`` tokens of request r (short prefill chunks, whose keys the exact cache
    holds)."""

    def __init__(self, hist, pad, width, splits, seed, lens=None):
        g = torch.Generator(device='cuda').manual_seed(seed)
        hist = np.asarray(hist)
        lens = np.ones(len(hist), np.int64) if lens is None else np.asarray(lens, np.int64)
        self.R, self.n, self.Q, self.w, self.splits = len(hist), int(lens.sum()), int(lens.max()), width, splits
        self.T = self.n + pad
        seq = hist + lens
        cols = int(-(-seq.max() // BLOCK))
        pool = self.R * cols + 1
        rnd = lambda *s, std=1.0: (torch.randn(*s, generator=g, device='cuda') * std).to(torch.bfloat16)
        perm = (torch.randperm(pool - 1, generator=g, device='cuda') + 1).to(torch.int32)
        self.table = perm[:self.R * cols].view(self.R, cols).contiguous()
        self.ex_table = (torch.randperm(pool - 1, generator=g, device='cuda') + 1).to(torch.int32)[:self.R * cols]
        self.ex_table = self.ex_table.view(self.R, cols).contiguous()
        self.cache = rnd(pool, 1, BLOCK, 2 * width)
        self.exact = rnd(pool, H, BLOCK, 2 * D)
        self.q_lat = rnd(self.T, H, width, std=width ** -0.5)
        self.q_rope = rnd(self.T, H, D)
        self.B = rnd(H, width, D, std=1 / math.sqrt(2048))
        positions = np.concatenate([np.arange(h, h + n) for h, n in zip(hist, lens)] + [np.ones(pad, np.int64)])
        qsl = np.concatenate(([0], np.cumsum(lens))).astype(np.int32)
        ws = ops.S6Workspace(H, width, self.T * splits)
        self.ctx = layer.StepContext(torch.as_tensor(positions, device='cuda'), torch.as_tensor(qsl, device='cuda'),
                                     torch.as_tensor(seq.astype(np.int32), device='cuda'), self.Q, self.T, {}, SCALE,
                                     ops.HIP_BACKENDS, ws, splits, window=W, max_seqlen_k=int(seq.max()))
        A = rnd(H, D, width)
        if width == 512:
            self.loop, self.sl = 1, FakeLatentLayer(rnd(H, D, 256), rnd(H, 256, D), A[None].repeat(3, 1, 1, 1),
                                                    self.B[None].repeat(3, 1, 1, 1))
        else:
            self.loop, self.sl = 0, FakeLatentLayer(A, self.B, rnd(3, H, D, 512), rnd(3, H, 512, D))

    def allocating(self):
        """The existing path: s6_layer.attend's decode branch (hla_s6_attend_decode with the step's plan)."""
        return layer.attend(self.sl, self.loop, self.q_lat, self.q_rope, None, None, self.cache, self.table, None,
                            None, self.ctx, (self.exact, self.ex_table))

    def static(self):
        ctx, w, d = self.ctx, self.w, D
        out = torch.empty(self.T, H, D, dtype=torch.bfloat16, device='cuda')
        c, ex = self.cache, self.exact
        lib.call('hla_s6_attend_decode_static', lib.ptr(self.q_lat), self.q_lat.stride(0), self.q_lat.stride(1), w,
                 lib.ptr(c), lib.ptr(c[..., w:]), c.stride(0), c.stride(2), c.shape[2], c.shape[0],
                 lib.ptr(self.table), self.table.stride(0), self.table.shape[1], lib.ptr(ctx.token_requests),
                 lib.ptr(ctx.ctx_latent), lib.ptr(self.q_rope), self.q_rope.stride(0), self.q_rope.stride(1),
                 lib.ptr(ex), lib.ptr(ex[..., d:]), ex.stride(0), ex.stride(2), ex.stride(1), ex.shape[2],
                 ex.shape[0], lib.ptr(self.ex_table), self.ex_table.stride(0), self.ex_table.shape[1],
                 lib.ptr(ctx.query_start_loc), lib.ptr(ctx.seq_lens), self.R, W, lib.ptr(self.B), self.B.stride(0),
                 self.B.stride(1), lib.ptr(ctx.invalid), self.T, H, SCALE, self.splits, self.Q, lib.ptr(out),
                 out.stride(0), out.stride(1), lib.stream(out.device))
        return out


def test_static_entry_under_graph_capture():
    """The first call of the static entry point in this process is made under HIP graph capture (its per-device
    array lookup included); replays with new queries between them, each after eager work and a synchronization,
    are bitwise equal to the allocating entry point's eager result, and so is an eager call of the static entry
    point between replays (which shares the array with the graph's kernels)."""
    step = Step(np.random.default_rng(4).integers(1, 5000, 32), pad=1, width=512, splits=16, seed=4)
    step.allocating()                       # the step's plan and the library's kernels, loaded outside the capture
    torch.cuda.synchronize()
    print('case graph capture of the first static call (33 rows, width 512, 16 slots)', flush=True)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        out = step.static()
    torch.cuda.current_stream().wait_stream(side)
    g = torch.Generator(device='cuda').manual_seed(5)
    for i in range(3):
        step.q_lat.copy_((torch.randn(step.q_lat.shape, generator=g, device='cuda') * 512 ** -0.5).to(torch.bfloat16))
        graph.replay()
        torch.cuda.synchronize()
        want = step.allocating()
        torch.cuda.synchronize()
        assert torch.equal(out, want), f'replay {i}: max diff {(out.float() - want.float()).abs().max().item()}'
        eager = step.static()
        torch.cuda.synchronize()
        assert torch.equal(eager, want), f'eager static call after replay {i} differs'


def test_static_entry_equals_the_allocating_one_on_two_calls():
    big = Step(np.random.default_rng(1).integers(1, 6000, 64), pad=2, width=512, splits=16, seed=1)
    small = Step([700, 0, 45, 2900, 20], pad=1, width=256, splits=4, seed=2)
    for name, step in (('first call (66 rows, width 512, 16 slots)', big),
                       ('second call (6 rows, width 256, 4 slots)', small)):
        print(f'case {name}', flush=True)
        want = step.allocating()
        got = step.static()
        torch.cuda.synchronize()
        assert torch.isfinite(got.float()).all(), name
        assert torch.equal(got, want), f'{name}: max diff {(got.float() - want.float()).abs().max().item()}'
        assert (got[step.n:] == 0).all()
    # one slot: the one-slot history output and lse also live in the array
    one = Step([1500, 300, 0], pad=0, width=512, splits=1, seed=3)
    assert torch.equal(one.static(), one.allocating())


def test_static_entry_on_short_chunks():
    """Steps of short prefill chunks (the static entry's plan then lists a request's tokens chunk by chunk, as the
    step's own plan does): 4 x 3 tokens over about 8,000 history rows, then a smaller mixed step (decode rows and
    chunks of 2 .. 15 tokens, padding) at the narrower latent; each bitwise equal to the allocating entry point."""
    chunks = Step([8200, 7900, 8100, 8050], pad=2, width=512, splits=64, seed=6, lens=[3, 3, 3, 3])
    mixed = Step([3000, 17, 900, 0, 1200], pad=3, width=256, splits=16, seed=7, lens=[1, 15, 4, 2, 1])
    for name, step in (('4 x 3 tokens, width 512, 64 slots', chunks),
                       ('chunks of 1 .. 15 tokens, width 256, 16 slots', mixed)):
        print(f'case {name}', flush=True)
        want = step.allocating()
        got = step.static()
        torch.cuda.synchronize()
        assert torch.isfinite(got.float()).all(), name
        assert torch.equal(got, want), f'{name}: max diff {(got.float() - want.float()).abs().max().item()}'
        assert (got[step.n:] == 0).all()


def refusal_args(num_tokens, num_splits, width=512):
    """Arguments of hla_s6_attend_decode_static with null pointers and zero strides around the sizes."""
    args = [None if t is lib.P else 0 for t in lib.SIGNATURES['hla_s6_attend_decode_static']]
    args[3], args[36], args[37], args[38], args[39] = width, num_tokens, H, SCALE, num_splits
    return args


def test_static_entry_refuses_sizes_past_the_array():
    """4096 rows x 64 slots at width 512 need 8.6 GB of partials: refused before any launch or device access."""
    with pytest.raises(RuntimeError, match='static array holds'):
        lib.call('hla_s6_attend_decode_static', *refusal_args(4096, 64))
