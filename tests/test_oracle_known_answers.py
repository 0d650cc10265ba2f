"""The oracle against the known-answer values of the reference's own tests (tests/golden/known_answers.json)."""
import json
import os

import numpy as np
import pytest

from oracle import s6_oracle as O

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), 'golden', 'known_answers.json')))


@pytest.mark.parametrize('case', GOLDEN['token_requests']['cases'], ids=lambda c: str(c['qsl']) + f"/T{c['num_tokens']}")
def test_token_requests(case):
    req, valid = O.token_requests(case['qsl'], case['num_tokens'])
    assert req.dtype == np.int64 and valid.dtype == bool
    assert req.tolist() == case['req'] and valid.tolist() == [bool(v) for v in case['valid']]


@pytest.mark.parametrize('case', GOLDEN['history_lengths']['cases'], ids=lambda c: str(c['qsl']))
def test_history_lengths(case):
    assert O.history_lengths(case['seq_lens'], case['qsl']).tolist() == case['expected']


def test_step_context_after_mixed_step():
    g = GOLDEN['step_context_mixed']
    req, valid, ctx, ctx_latent = O.step_context(g['qsl'], g['seq_lens'], g['num_tokens'])
    assert req.tolist() == g['token_requests'] and valid.tolist() == [bool(v) for v in g['valid']]
    assert ctx.tolist() == g['ctx'] and ctx_latent.tolist() == g['ctx']
    _, _, ctx_w, lat_w = O.step_context(g['qsl'], g['seq_lens'], g['num_tokens'], window=3)
    assert ctx_w.tolist() == g['ctx'] and lat_w.tolist() == [2, 0, 0, 0]


def test_profiling_step_has_no_history():
    req, valid, ctx, _ = O.step_context(None, None, 5)
    assert valid.all() and (ctx == 0).all() and (req == 0).all()


@pytest.mark.parametrize('case', GOLDEN['num_kv_splits']['cases'], ids=lambda c: str(c['args']))
def test_num_kv_splits(case):
    assert O.num_kv_splits(*case['args']) == case['expected']


def test_workspace_size():
    g = GOLDEN['workspace']
    assert O.workspace_floats(g['heads'], g['width_max'], g['rows_x_splits']) == g['floats']
    t, h, s, w = g['view_args']
    assert t * h * s * (w + 1) <= g['floats'] and list(g['view_shape']) == [t, h, s, w + 1]
    t, h, s, w = g['overflow_args']
    assert t * h * s * (w + 1) > g['floats']


def test_latent_rope_table_row0():
    g = GOLDEN['latent_rope_table_row0']
    table = O.latent_rope_table(g['max_position'], O.latent_inv_freq(g['head_dim'], g['theta']), g['width'])
    assert table.shape == (g['max_position'], g['width'])
    assert table[0].tolist() == g['row0']


def test_rollout_rows_block_table_expansion():
    """Slot mapping + paged row gather reproduce the reference's bit-exact rollout-cache rows."""
    g = GOLDEN['rollout_rows']
    bs, pos = g['block_size'], np.array(g['positions'])
    rows = []
    for part in ('main', 'l1'):
        p = g[part]
        cache = np.arange(p['num_blocks'] * bs * p['row_width']).reshape(p['num_blocks'] * bs, p['row_width'])
        table = np.array([p['table']])
        slots = O.slot_mapping(table, np.zeros(len(pos), np.int64), np.ones(len(pos), bool), pos, bs)
        rows.append(cache[slots])
    assert np.concatenate(rows, -1).tolist() == g['expected_rows']
    slots = O.slot_mapping(np.array([g['main']['table']]), np.zeros(3, np.int64), np.array([1, 0, 1], bool), pos, bs)
    assert slots.tolist() == [4, -1, 0]
