"""The device gather of the s6-rollout-cache-v1 export (``hla_s6_gather_packed_rows``) against the reference's
known rows (hla/tests/test_rollout_cache.py:38-41, in tests/golden/known_answers.json) and against the oracle's
slot-mapped row gather on random multi-layer caches; bit-exact. Then the whole export -> file, read back with the
safe loader."""
import importlib
import json
import os

import numpy as np
import pytest
import torch

from oracle import bf16
from oracle import s6_oracle as O
from s6util import dev_bf16, host_f32, random_bits

pytestmark = pytest.mark.gpu

rc = importlib.import_module('hybrid-latent-attention_amd.rollout_cache')
GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), 'golden', 'known_answers.json')))


def test_known_rows_of_the_reference_test():
    g = GOLDEN['rollout_rows']
    bs = g['block_size']
    caches = []
    for part in ('main', 'l1'):
        p = g[part]
        vals = torch.arange(p['num_blocks'] * bs * p['row_width'], dtype=torch.float32)
        caches.append(vals.reshape(p['num_blocks'], 1, bs, p['row_width']).to(torch.bfloat16).cuda())
    out = rc.gather_packed_rows([tuple(caches)], g['main']['table'], g['l1']['table'], len(g['positions']))
    assert out.shape == (1, 3, 6)
    assert host_f32(out[0]).tolist() == g['expected_rows']


def _oracle_rows(caches_bits, blocks, bs, length):
    """Per layer: cat of the slot-mapped rows of both caches (slot = block[pos // bs] * bs + pos % bs)."""
    pos = np.arange(length)
    layers = []
    for pair in caches_bits:
        parts = []
        for c, b, s in zip(pair, blocks, bs):
            slots = O.slot_mapping(np.asarray([b]), np.zeros(length, np.int64), np.ones(length, bool), pos, s)
            parts.append(c.reshape(-1, c.shape[-1])[slots])
        layers.append(np.concatenate(parts, -1))
    return np.stack(layers)


@pytest.mark.parametrize('r,r1,bs,length', [(512, 256, 16, 1000), (512, 256, 16, 1), (12, 5, 4, 37)])
def test_random_layers_match_the_oracle_gather(r, r1, bs, length):
    rng = np.random.default_rng(r + length)
    L, nb = 5, -(-length // bs) + 7
    caches_bits = [(random_bits(rng, (nb, 1, bs, 2 * r)), random_bits(rng, (nb, 1, bs, 2 * r1))) for _ in range(L)]
    need = -(-length // bs)
    blocks = [rng.permutation(nb)[:need].astype(np.int32) for _ in range(2)]
    caches = [(dev_bf16(a), dev_bf16(b)) for a, b in caches_bits]
    out = rc.gather_packed_rows(caches, torch.as_tensor(blocks[0]), torch.as_tensor(blocks[1]), length)
    want = _oracle_rows(caches_bits, blocks, (bs, bs), length)
    got = out.cpu().view(torch.int16).numpy().view(np.uint16)
    assert got.shape == want.shape and (got == want).all()


def test_gather_rejects_short_block_lists():
    c = (torch.zeros(4, 1, 16, 8, dtype=torch.bfloat16, device='cuda'),
         torch.zeros(4, 1, 16, 4, dtype=torch.bfloat16, device='cuda'))
    with pytest.raises(ValueError, match='cannot hold'):
        rc.gather_packed_rows([c], [0], [0, 1], 17)
    with pytest.raises(RuntimeError, match='layout'):
        rc.gather_packed_rows([(c[0][:, 0], c[1])], [0, 1], [0, 1], 17)


def test_export_writes_the_gathered_rows(tmp_path):
    rng = np.random.default_rng(5)
    cfg = dict(num_layers=3, rank=512, rank_v=512, rank1=256)
    prompt, response = 40, 25
    length = prompt + response - 1
    nb, bs = 10, 16
    caches_bits = [(random_bits(rng, (nb, 1, bs, 1024)), random_bits(rng, (nb, 1, bs, 512))) for _ in range(3)]
    caches = [(dev_bf16(a), dev_bf16(b)) for a, b in caches_bits]
    blocks = [np.array([7, 2, 9, 4, 0], np.int32), np.array([1, 3, 5, 6, 8], np.int32)]
    logits = torch.randn(1, 1, 11)
    ids = rng.integers(0, 1000, prompt + response).tolist()
    ref = rc.export_request(tmp_path / '0.pt', caches, torch.as_tensor(blocks[0]).cuda(), blocks[1], length,
                            version=3, request_id='req-0', cfg=cfg, prompt_ids=ids[:prompt],
                            first_response_logits=logits)
    assert ref['length'] == length and ref['bytes'] > 3 * length * 1536 * 2 and ref['seconds'] > 0
    raw = torch.load(ref['path'], map_location='cpu', weights_only=True)
    assert raw['schema'] == 's6-rollout-cache-v1' and raw['version'] == 3 and raw['request_id'] == 'req-0'
    assert raw['cfg'] == cfg and raw['prompt_ids'] == ids[:prompt] and raw['length'] == length
    assert torch.equal(raw['first_response_logits'], logits)
    want = _oracle_rows(caches_bits, blocks, (bs, bs), length)
    assert len(raw['rows']) == 3
    for l in range(3):
        assert tuple(raw['rows'][l].shape) == (1, length, 1536) and raw['rows'][l].dtype == torch.bfloat16
        got = raw['rows'][l][0].view(torch.int16).numpy().view(np.uint16)
        assert (got == want[l]).all()
