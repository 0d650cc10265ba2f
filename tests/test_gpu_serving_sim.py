"""A few serving steps of one S6 layer end to end on the GPU, in the shape of hla/tests/test_s6_serving.py:27-106
(prefill, decode over the committed history, a page crossing, a mixed step with padding): per step and loop the
writer commits rows through the step's slots (write_commit), the exact cache takes the step's keys, and attend reads
the history committed by earlier steps through the same block tables. Every attend output is checked against the
oracle composite evaluated on host mirrors of the caches; the committed rows against the oracle writer.
"""
import math
import types

import numpy as np
import pytest
import torch

from oracle import bf16
from oracle import s6_oracle as O
from s6util import assert_attention_close, dev_bf16, dev_i32, dev_i64, host_f32, random_bits

pytestmark = pytest.mark.gpu

H, D, W, BLOCK, HIDDEN, R, R1 = 16, 128, 32, 16, 512, 512, 256
SCALE = 1 / math.sqrt(D)


class Layer:
    """A LatentLayer-shaped module: readers (A_t, B_t per loop) and writer projections (cand1, cand_s)."""

    def __init__(self, rng):
        self.rank, self.rank_v, self.rank1, self.loops, self.head_dim = R, R, R1, 4, D
        std = 1 / math.sqrt(HIDDEN)
        self.bits = dict(A1=random_bits(rng, (H, D, R1), std), B1=random_bits(rng, (H, R1, D), std),
                         A=random_bits(rng, (3, H, D, R), std), B=random_bits(rng, (3, H, R, D), std),
                         cand1=random_bits(rng, (2 * R1, HIDDEN), std),
                         cand_s=random_bits(rng, (3, 2 * R, HIDDEN), std))
        self.dev = {k: dev_bf16(v) for k, v in self.bits.items()}
        self.cand1 = types.SimpleNamespace(weight=self.dev['cand1'])
        self.cand_s = [types.SimpleNamespace(weight=self.dev['cand_s'][i]) for i in range(3)]

    def readers(self, loop):
        if loop == 0:
            return self.dev['A1'], self.dev['B1'], R1
        return self.dev['A'][loop - 1], self.dev['B'][loop - 1], R

    def weight_bits(self, loop):
        return self.bits['cand1'] if loop == 0 else self.bits['cand_s'][loop - 1]

    def b_bits(self, loop):
        return self.bits['B1'] if loop == 0 else self.bits['B'][loop - 1]


def test_prefill_decode_page_crossing_and_mixed_steps(ops, layer):
    rng = np.random.default_rng(31)
    sl = Layer(rng)
    num_reqs, cols = 3, 6
    nb = num_reqs * cols + 2
    lt = (1 + rng.permutation(nb - 1)[:num_reqs * cols]).reshape(num_reqs, cols).astype(np.int32)
    et = (1 + rng.permutation(nb - 1)[:num_reqs * cols]).reshape(num_reqs, cols).astype(np.int32)
    caches = {w: torch.zeros(nb, 1, BLOCK, 2 * w, dtype=torch.bfloat16, device='cuda') for w in (R, R1)}
    exact = [torch.zeros(nb, H, BLOCK, 2 * D, dtype=torch.bfloat16, device='cuda') for _ in range(4)]
    inv = layer.latent_inv_freq(D, 1e6).to('cuda')
    tables = {w: layer.latent_rope_table(256, inv, w, torch.bfloat16) for w in (R, R1)}
    history = [0] * num_reqs
    # (request, new tokens) per step; -1 marks a padding token appended to the step
    # request 0: a 47-token prompt, then decodes whose latent history (context - 32 rows) grows from 15 rows across the
    # first page boundary; request 1: a 37-token prompt in a mixed step; request 2: a prompt in a later mixed step
    steps = [[(0, 47)], [(0, 1), (1, 37)], [(0, 1), (1, 1), (-1, 1)], [(0, 1), (2, 12), (1, 1)], [(0, 1), (1, 1)]]
    for step_no, step in enumerate(steps):
        reqs = [r for r, _ in step if r >= 0]
        lens = np.array([n for r, n in step if r >= 0], np.int64)
        pad = sum(n for r, n in step if r < 0)
        qsl = np.concatenate(([0], np.cumsum(lens))).astype(np.int32)
        T = int(qsl[-1]) + pad
        seq = np.array([history[r] + n for r, n in zip(reqs, lens)], np.int32)
        positions = np.concatenate([np.arange(history[r], history[r] + n) for r, n in zip(reqs, lens)] +
                                   [np.zeros(pad, np.int64)]).astype(np.int64)
        lt_s, et_s = lt[reqs], et[reqs]
        splits = 4
        ws = ops.S6Workspace(H, R, T * splits)
        ctx = layer.StepContext(dev_i64(positions), dev_i32(qsl), dev_i32(seq), int(lens.max()), T, tables, SCALE,
                                ops.HIP_BACKENDS, ws, splits, window=W, max_seqlen_k=int(seq.max()))
        req, valid, c, cl = O.step_context(qsl, seq, T, W)
        lt_dev, et_dev = dev_i32(lt_s), dev_i32(et_s)
        state = None
        for loop in range(4):
            print(f'case step={step_no} loop={loop} T={T}', flush=True)
            w = R1 if loop == 0 else R
            h = random_bits(rng, (T, HIDDEN))
            prev_reg = None if state is None or state.reg is None else host_f32(state.reg)
            state = layer.write_commit(sl, loop, dev_bf16(h), state, ctx, caches[w], lt_dev)
            if loop in (0, 3):  # the committed rows of the valid tokens, against the oracle writer and rotation
                row = O.write_step(bf16.to_f32(h), bf16.to_f32(sl.weight_bits(loop)),
                                   None if loop == 0 else prev_reg)
                key, val = O.committed_row(row, w, positions, host_f32(tables[w]))
                flat = host_f32(caches[w]).reshape(-1, 2 * w)
                slots = lt_s[req[valid], positions[valid] // BLOCK] * BLOCK + positions[valid] % BLOCK
                want = np.concatenate((key, val), -1)[valid]
                got = flat[slots]
                bound = 2 * 2.0 ** -7 * np.abs(want) + 0.02
                assert (np.abs(got - want) <= bound).all() and (got == want).mean() > 0.9
            elif loop > 0:
                assert state.reg is not None
            q_pre = dev_bf16(random_bits(rng, (T, H, D)))
            q_lat = ctx.latent_query(sl, loop, q_pre)
            q_rope, k_rope, v = (random_bits(rng, (T, H, D)) for _ in range(3))
            # the exact cache takes this step's keys before attention (unified_kv_cache_update)
            ex_slots = et_s[req[valid], positions[valid] // BLOCK] * BLOCK + positions[valid] % BLOCK
            kv = np.concatenate((bf16.to_f32(k_rope), bf16.to_f32(v)), -1)[valid]
            flat_ex = exact[loop].permute(0, 2, 1, 3).reshape(-1, H, 2 * D)
            upd = flat_ex.clone()
            upd[torch.as_tensor(ex_slots, device='cuda')] = torch.tensor(kv, device='cuda').to(torch.bfloat16)
            exact[loop].copy_(upd.reshape(nb, BLOCK, H, 2 * D).permute(0, 2, 1, 3))
            out = layer.attend(sl, loop, q_lat, dev_bf16(q_rope), dev_bf16(k_rope), dev_bf16(v), caches[w], lt_dev,
                               None, None, ctx, (exact[loop], et_dev))
            lat = host_f32(caches[w])
            ex = host_f32(exact[loop])
            ql = host_f32(q_lat)
            B = bf16.to_f32(sl.b_bits(loop))
            if int(lens.max()) == 1:
                want = O.attend_decode(ql, bf16.to_f32(q_rope), B, lat[..., :w], lat[..., w:], lt_s[req],
                                       np.where(valid, cl, 0), ex[..., :D], ex[..., D:], et_s, qsl, seq, W, SCALE,
                                       ~valid, rounding=False)
            else:
                want = O.attend_chunk(ql, bf16.to_f32(q_rope), bf16.to_f32(k_rope), bf16.to_f32(v), B, lat[..., :w],
                                      lat[..., w:], {'latent': lt_s[req], 'exact': et_s[req]}, c, cl, qsl, W, SCALE,
                                      ~valid, ex[..., :D], ex[..., D:], rounding=False)
            got = host_f32(out)
            assert_attention_close(got, want, f'step {step_no} loop {loop}')
            assert (got[~valid] == 0).all()
        for r, n in zip(reqs, lens):
            history[r] += int(n)
    assert history == [51, 40, 12]
