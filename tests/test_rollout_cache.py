"""The s6-rollout-cache-v1 snapshot: the file written by ``rollout_cache.write_snapshot`` and read back with the
reference's guards (hla/tests/test_rollout_cache.py:73-96 cases; hla/latent/history_snapshot.py:78-105). CPU only:
the rows here are host tensors (the device gather is tested in test_gpu_rollout.py)."""
import importlib
from types import SimpleNamespace as NS

import pytest
import torch

rc = importlib.import_module('hybrid-latent-attention_amd.rollout_cache')

CFG = dict(num_layers=2, rank=2, rank_v=2, rank1=1)          # packed row width 2 + 2 + 2 * 1 = 6


def write(tmp_path, length=3, version=0, request_id='a', prompt=(4, 5)):
    rows = torch.arange(2 * length * 6, dtype=torch.float32).reshape(2, length, 6).to(torch.bfloat16)
    logits = torch.arange(9).float()[None, None]
    ref = rc.write_snapshot(tmp_path / '0.pt', rows, version=version, request_id=request_id, cfg=CFG,
                            prompt_ids=list(prompt), length=length, first_response_logits=logits)
    return rows, ref


def trajectory(ids, ref, prompt=2, version=0, request_id='a'):
    return NS(ids=torch.tensor([ids]), prompt=prompt, version=version, history_ref=ref, request_id=request_id,
              truncated=False)


def test_roundtrip(tmp_path):
    rows, ref = write(tmp_path)
    assert set(ref) == {'path', 'request_id', 'version', 'length', 'bytes'} and ref['length'] == 3
    raw = torch.load(ref['path'], map_location='cpu', weights_only=True)
    assert raw['schema'] == 's6-rollout-cache-v1' and raw['cfg'] == CFG and raw['prompt_ids'] == [4, 5]
    assert len(raw['rows']) == 2 and all(tuple(r.shape) == (1, 3, 6) for r in raw['rows'])
    ref['token_ids'] = [4, 5, 6, 7]
    snap = rc.load_rollout_snapshot(trajectory([4, 5, 6, 7], ref), NS(cfg=CFG))
    assert snap.source == 'vllm_rollout' and snap.prompt_length == 2 and snap.response_length == 2
    for l in range(2):
        assert torch.equal(snap.rows[l], rows[l:l + 1])
    assert torch.equal(snap.first_response_logits, torch.arange(9).float()[None, None])
    assert not (tmp_path / '0.tmp').exists()


@pytest.mark.parametrize('field,value,match', [
    ('version', 7, 'stale'), ('request_id', 'wrong', 'stale'),
    ('length', 99, 'length'), ('token_ids', [1], 'token ids')])
def test_reject_bad_reference(tmp_path, field, value, match):
    _, ref = write(tmp_path, length=2)
    ref['token_ids'] = [4, 5, 6]
    ref[field] = value
    with pytest.raises(ValueError, match=match):
        rc.load_rollout_snapshot(trajectory([4, 5, 6], ref), NS(cfg=CFG))


def test_reject_over_scheduled_export(tmp_path):
    """One extra executed token exports P+n rows for a P+n-1 trajectory (hla/tests/test_rollout_cache.py:81-93)."""
    _, ref = write(tmp_path, length=3)
    ref['token_ids'] = [4, 5, 6]
    with pytest.raises(ValueError, match='exported 3.*needs 2'):
        rc.load_rollout_snapshot(trajectory([4, 5, 6], ref), NS(cfg=CFG))


def test_reject_config_prompt_and_layout(tmp_path):
    _, ref = write(tmp_path)
    ref['token_ids'] = [4, 5, 6, 7]
    with pytest.raises(ValueError, match='config mismatch'):
        rc.load_rollout_snapshot(trajectory([4, 5, 6, 7], ref), NS(cfg=dict(CFG, rank1=2)))
    with pytest.raises(ValueError, match='prompt tokens'):
        ref2 = dict(ref, token_ids=[9, 5, 6, 7])
        rc.load_rollout_snapshot(trajectory([9, 5, 6, 7], ref2), NS(cfg=CFG))
    rows = torch.zeros(2, 3, 5, dtype=torch.bfloat16)          # a row one element short of the packed width
    bad = rc.write_snapshot(tmp_path / '1.pt', rows, version=0, request_id='a', cfg=CFG, prompt_ids=[4, 5], length=3,
                            first_response_logits=torch.zeros(1, 1, 9))
    bad['token_ids'] = [4, 5, 6, 7]
    with pytest.raises(ValueError, match='row layout'):
        rc.load_rollout_snapshot(trajectory([4, 5, 6, 7], bad), NS(cfg=CFG))


def test_export_requires_logits():
    with pytest.raises(RuntimeError, match='logits'):
        rc.export_request('unused.pt', [], [], [], 0, version=0, request_id='a', cfg=CFG, prompt_ids=[],
                          first_response_logits=None)
