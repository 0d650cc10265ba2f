"""The s6-rollout-cache-v1 file written by ``rollout_cache.write_snapshot`` (``hla/vllm_latent/cache_export.py:176-188``):
its fields, the packed row layout of every layer and the exporter's per-request record, checked directly on the file
with the safe loader. CPU only: the rows here are host tensors (the device gather is tested in test_gpu_rollout.py)."""
import importlib

import pytest
import torch

rc = importlib.import_module('hybrid-latent-attention_amd.rollout_cache')

CFG = dict(num_layers=2, rank=2, rank_v=2, rank1=1)          # packed row width 2 + 2 + 2 * 1 = 6
FIELDS = {'schema', 'version', 'request_id', 'cfg', 'prompt_ids', 'length', 'first_response_logits', 'rows'}


def write(tmp_path, length=3, version=0, request_id='a', prompt=(4, 5), name='0.pt'):
    rows = torch.arange(2 * length * 6, dtype=torch.float32).reshape(2, length, 6).to(torch.bfloat16)
    logits = torch.arange(9).float()[None, None]
    ref = rc.write_snapshot(tmp_path / name, rows, version=version, request_id=request_id, cfg=CFG,
                            prompt_ids=list(prompt), length=length, first_response_logits=logits)
    return rows, logits, ref


def test_file_fields_and_rows(tmp_path):
    rows, logits, ref = write(tmp_path, length=3, version=7, request_id='req-1', prompt=(4, 5))
    assert ref == dict(path=str(tmp_path / '0.pt'), request_id='req-1', version=7, length=3,
                       bytes=(tmp_path / '0.pt').stat().st_size)
    raw = torch.load(ref['path'], map_location='cpu', weights_only=True)
    assert set(raw) == FIELDS
    assert raw['schema'] == 's6-rollout-cache-v1' and raw['version'] == 7 and raw['request_id'] == 'req-1'
    assert raw['cfg'] == CFG and raw['prompt_ids'] == [4, 5] and raw['length'] == 3
    assert torch.equal(raw['first_response_logits'], logits)
    # one [1, length, rank + rank_v + 2 rank1] tensor per layer, bf16, equal to the rows handed in
    width = CFG['rank'] + CFG['rank_v'] + 2 * CFG['rank1']
    assert isinstance(raw['rows'], tuple) and len(raw['rows']) == CFG['num_layers']
    for l, row in enumerate(raw['rows']):
        assert tuple(row.shape) == (1, 3, width) and row.dtype == torch.bfloat16
        assert torch.equal(row[0], rows[l])
    assert not (tmp_path / '0.tmp').exists()                   # written through a temporary name, then renamed


def test_rewrite_replaces_the_file_atomically(tmp_path):
    write(tmp_path, length=2, version=0)
    _, _, ref = write(tmp_path, length=4, version=1)
    raw = torch.load(ref['path'], map_location='cpu', weights_only=True)
    assert raw['version'] == 1 and raw['length'] == 4 and raw['rows'][0].shape[1] == 4
    assert sorted(p.name for p in tmp_path.iterdir()) == ['0.pt']


def test_rows_must_match_the_length(tmp_path):
    with pytest.raises(ValueError, match='rows must be'):
        rc.write_snapshot(tmp_path / '0.pt', torch.zeros(2, 3, 6, dtype=torch.bfloat16), version=0, request_id='a',
                          cfg=CFG, prompt_ids=[4], length=2, first_response_logits=torch.zeros(1, 1, 9))
    with pytest.raises(ValueError, match='rows must be'):
        rc.write_snapshot(tmp_path / '0.pt', torch.zeros(3, 6, dtype=torch.bfloat16), version=0, request_id='a',
                          cfg=CFG, prompt_ids=[4], length=3, first_response_logits=torch.zeros(1, 1, 9))
    assert not list(tmp_path.iterdir())


def test_export_requires_logits():
    """The exporter's retirement guard (``cache_export.py:166-167``)."""
    with pytest.raises(RuntimeError, match='logits'):
        rc.export_request('unused.pt', [], [], [], 0, version=0, request_id='a', cfg=CFG, prompt_ids=[],
                          first_response_logits=None)
