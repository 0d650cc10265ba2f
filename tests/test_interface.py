"""CPU checks of the drop-in boundary: the C ABI library loads and exports every symbol of include/hla_s6.h with
the declared arity; the Python mirror keeps the reference's operator names and parameter lists and its host-side
error behaviour; the product package never reaches the oracle."""
import ast
import importlib
import inspect
import json
import os
import re

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, 'include', 'hla_s6.h')
PKG_DIR = os.path.join(ROOT, 'hybrid-latent-attention_amd')
IFACE = json.load(open(os.path.join(ROOT, 'tests', 'golden', 'reference_interface.json')))
KNOWN = json.load(open(os.path.join(ROOT, 'tests', 'golden', 'known_answers.json')))


def header_declarations():
    text = re.sub(r'/\*.*?\*/', '', open(HEADER).read(), flags=re.S)
    decls = {}
    for m in re.finditer(r'^(?:int|int64_t|const char \*)\s*(hla_s6_\w+)\s*\(([^)]*)\)\s*;', text, re.M):
        params = m.group(2).strip()
        decls[m.group(1)] = 0 if params in ('', 'void') else params.count(',') + 1
    return decls


def test_library_exports_every_declared_symbol(pkg):
    lib = pkg._lib.load()
    decls = header_declarations()
    assert len(decls) >= 12
    assert set(decls) == set(pkg._lib.SIGNATURES), 'header and ctypes binding disagree'
    for name, arity in decls.items():
        assert hasattr(lib, name), f'{name} not exported by libhla_s6.so'
        assert len(pkg._lib.SIGNATURES[name]) == arity, f'{name}: binding has {len(pkg._lib.SIGNATURES[name])} args'
    assert lib.hla_s6_abi_version() == pkg._lib.ABI_VERSION


def _params(obj):
    return list(inspect.signature(obj).parameters)


@pytest.mark.parametrize('module', ['s6_ops', 's6_layer', 'history_gemm', 'batched_engine'])
def test_reference_parameter_lists(pkg, module):
    mod = getattr(pkg, module)
    for qual, want in IFACE[module].items():
        obj = mod
        for part in qual.split('.'):
            obj = getattr(obj, part)
        got = _params(obj)
        assert got[:len(want)] == want, f'{module}.{qual}: {got} != {want}'
        for extra in list(inspect.signature(obj).parameters.values())[len(want):]:
            assert extra.default is not inspect.Parameter.empty, f'{module}.{qual}: extra {extra.name} has no default'


@pytest.mark.parametrize('module', ['s6_ops', 's6_layer', 'history_gemm', 'batched_engine'])
def test_reference_default_values(pkg, module):
    """Every parameter the reference gives a default keeps that default value (a caller relying on a default gets
    the reference's behaviour or an error, never a silently different mode)."""
    mod = getattr(pkg, module)
    for qual, defaults in IFACE['_defaults'][module].items():
        obj = mod
        for part in qual.split('.'):
            obj = getattr(obj, part)
        params = inspect.signature(obj).parameters
        for name, want in defaults.items():
            assert params[name].default == want, f'{module}.{qual}({name}=...): {params[name].default!r} != {want!r}'


def test_history_precisions_and_backends(pkg):
    """Every precision and backend of the reference has kernels: on host tensors each refuses with the GPU-only
    error (no CPU path); unknown names raise the reference's errors (hla/latent/history_gemm.py:287-288,
    fused_history.py:146-147)."""
    hg = pkg.history_gemm
    q, k, m = torch.zeros(1, 2, 16, 256), torch.zeros(1, 2, 256), torch.ones(1, 2, 2, dtype=torch.bool)
    for kwargs in ({}, {'precision': 'fp32'}, {'precision': 'tf32'}, {'precision': 'bf16'}):
        with pytest.raises(RuntimeError, match='GPU only'):
            hg.causal_history_gemm(q, k, k, m, 1.0, **kwargs)
    with pytest.raises(ValueError, match='Unknown precision'):
        hg.causal_history_gemm(q, k, k, m, 1.0, precision='fp16')
    for backend in ('triton', 'reference', 'gemm'):
        with pytest.raises(RuntimeError, match='GPU only'):
            hg.causal_history_attention(q, k, k, m, 1.0, backend=backend)
    with pytest.raises(ValueError, match='Unknown causal history backend'):
        hg.causal_history_attention(q, k, k, m, 1.0, backend='hip')
    assert hg.KERNEL_PRECISIONS == hg.PRECISIONS


@pytest.mark.parametrize('case', KNOWN['num_kv_splits']['cases'], ids=lambda c: str(c['args']))
def test_num_kv_splits_known_answers(ops, case):
    assert ops.num_kv_splits(*case['args']) == case['expected']


def test_mi355x_split_policy(ops):
    # 8 resident waves per CU: a 512-wide split is a 4-wave workgroup, a 256-wide one 2 waves, a 128-wide one 1 wave;
    # twice the busy workgroups in slots, of which the kernel's plan fills about half
    assert ops.mi355x_kv_splits(8192, 64, 256, width=512) == 16
    assert ops.mi355x_kv_splits(8192, 64, 256, width=256) == 32
    assert ops.mi355x_kv_splits(8192, 32, 256, width=512) == 32
    assert ops.mi355x_kv_splits(32768, 8, 256, width=512) == 128
    assert ops.mi355x_kv_splits(8192, 64, 256, width=128) == 64
    assert ops.mi355x_kv_splits(8192, 1, 256, width=512) == 256        # 512 tiles: 64-key slots
    assert ops.mi355x_kv_splits(8192, 2, 256, width=512) == 128        # 1024 tiles: 128-key slots
    assert ops.mi355x_kv_splits(8227, 12, 256, width=512) == 84        # 4 x 3-token chunks: by occupancy
    assert ops.mi355x_kv_splits(8192, 24, 256, width=512) == 42        # 504 items: at most two per CU
    assert ops.mi355x_kv_splits(8192, 600, 256, width=512) == 2
    assert ops.mi355x_kv_splits(8227, 12, 256, width=256) == 130       # and by length
    assert ops.mi355x_kv_splits(4097, 4, 256, width=512) == 66         # 1028 tiles at the longest length
    # steps below 768 tiles even at the longest length: room for the plan's 4-tile items (64 keys per slot)
    assert ops.mi355x_kv_splits(1025, 1, 256, width=512) == 34
    assert ops.mi355x_kv_splits(2049, 2, 256, width=512) == 66
    assert ops.mi355x_kv_splits(2049, 4, 256, width=512) == 66
    assert ops.mi355x_kv_splits(4097, 1, 256, width=512) == 130
    assert ops.mi355x_kv_splits(32769, 8, 256, width=256) == 256
    assert ops.mi355x_kv_splits(300, 1, 256) == 10
    assert ops.mi355x_kv_splits(1, 4096, 256) == 2
    # multi-query steps: one busy 8-token workgroup per CU, every slot filled, at least 256 keys per slot
    assert ops.mi355x_kv_splits(8704, 2048, 256, tokens_per_group=4) == 1
    assert ops.mi355x_kv_splits(8704, 1024, 256, tokens_per_group=4) == 2
    assert ops.mi355x_kv_splits(8704, 64, 256, tokens_per_group=4) == 32
    assert ops.mi355x_kv_splits(300, 64, 256, tokens_per_group=4) == 2
    assert ops.mi355x_kv_splits(10 ** 6, 1, 256, width=128) == 1024    # the kernel's maximum


def test_workspace_for_several_widths(ops):
    ws = ops.S6Workspace.for_splits(16, 64, {512: 8, 256: 16})
    assert ws.floats == max(64 * 16 * 8 * 513, 64 * 16 * 16 * 257)
    for w, s in ((512, 8), (256, 16)):
        assert tuple(ws.attn_logits(64, 16, s, w, 'cpu').shape) == (64, 16, s, w + 1)


def test_workspace_sizing_and_overflow(ops):
    g = KNOWN['workspace']
    ws = ops.S6Workspace(heads=g['heads'], width_max=g['width_max'], rows_x_splits=g['rows_x_splits'])
    assert ws.floats == g['floats'] and ws.buffer is None
    view = ws.attn_logits(*g['view_args'], torch.device('cpu'))
    assert list(view.shape) == g['view_shape'] and view.dtype == torch.float32
    assert view.data_ptr() == ws.buffer.data_ptr() and ws.ensure('cpu') is ws.buffer
    with pytest.raises(RuntimeError, match='overflow'):
        ws.attn_logits(*g['overflow_args'])


def test_unknown_backends_raise_value_error(ops, layer):
    ones = torch.ones(1, 1, 8)
    i32 = torch.zeros(1, dtype=torch.int32)
    with pytest.raises(ValueError):
        ops.history_attention(ones, ones[None], i32[None], i32, 1.0, 1, None, None, None, 'triton')
    with pytest.raises(ValueError):
        ops.chunk_attention(ones, ones, ones, torch.tensor([0, 1], dtype=torch.int32), 1,
                            torch.zeros(1, dtype=torch.bool), 1.0, 'flash')
    with pytest.raises(ValueError):
        ops.merge_states(ones, ones[0], ones, ones[0], torch.zeros(1, dtype=torch.bool), 'vllm')
    with pytest.raises(ValueError):
        ops.latent_rope(ones, torch.zeros(1, dtype=torch.int64), ones[0], 'torch')
    with pytest.raises(ValueError):
        layer.latent_query(ones, ones, torch.zeros(1, dtype=torch.int64), ones[0], 'vllm')


def test_cpu_tensors_are_rejected(ops):
    """No CPU path: a host tensor is an error, never a fallback."""
    q = torch.zeros(1, 16, 512, dtype=torch.bfloat16)
    cache = torch.zeros(2, 1, 16, 1024, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match='GPU only'):
        ops.history_attention(q, cache, torch.zeros(1, 1, dtype=torch.int32), torch.zeros(1, dtype=torch.int32),
                              1.0, 1, None, None, None, 'hip')
    with pytest.raises(RuntimeError, match='GPU only'):
        ops.history_partials_grouped(q, cache[..., :512], cache[..., 512:], torch.zeros(1, 1, dtype=torch.int32),
                                     torch.zeros(1, dtype=torch.int32), 1.0, 2, None)
    with pytest.raises(RuntimeError, match='GPU only'):
        ops.split_epilogue(torch.zeros(1, 16, 2, 513), torch.zeros(16, 512, 128, dtype=torch.bfloat16),
                           torch.zeros(1, 16, 128, dtype=torch.bfloat16), torch.zeros(16, 1), None)


def test_select_backends_needs_a_gpu(ops):
    if torch.cuda.is_available():
        assert ops.select_backends() == ops.HIP_BACKENDS
    else:
        with pytest.raises(RuntimeError):
            ops.select_backends()


def test_product_never_imports_the_oracle():
    for dirpath, _, files in os.walk(PKG_DIR):
        for f in files:
            if f.endswith('.py'):
                tree = ast.parse(open(os.path.join(dirpath, f)).read())
                for node in ast.walk(tree):
                    names = []
                    if isinstance(node, ast.Import):
                        names = [a.name for a in node.names]
                    elif isinstance(node, ast.ImportFrom):
                        names = [node.module or '']
                    assert not any(n.split('.')[0] == 'oracle' for n in names), f'{f} imports the oracle'


def test_library_status_codes_map_to_reference_exceptions(pkg):
    lib = pkg._lib
    with pytest.raises(ValueError):   # EUNSUPPORTED: 8 query heads
        lib.call('hla_s6_history_attention', None, 1, 8, 512, 0, 0, None, None, 0, 0, 16, 1, None, 0, 1, None, None,
                 1.0, 1, None, 0, None, 0, 0, None, None)
    with pytest.raises(RuntimeError, match='workspace overflow'):   # EWORKSPACE before any launch
        lib.call('hla_s6_history_attention', 16, 1, 16, 512, 512, 512, 16, 16, 1024, 1024, 16, 1, 16, 0, 1, None, 16,
                 1.0, 4, 16, 10, 16, 512, 512, 16, None)


def test_static_decode_refuses_sizes_past_its_array(pkg):
    """hla_s6_attend_decode_static checks its buffers against the static array before any device access: 4096 rows x
    64 slots at width 512 (8.6 GB of split partials) raise RuntimeError; a bad width raises ValueError."""
    lib = pkg._lib
    args = [None if t is lib.P else 0 for t in lib.SIGNATURES['hla_s6_attend_decode_static']]
    args[3], args[36], args[37], args[38], args[39] = 512, 4096, 16, 0.1, 64
    with pytest.raises(RuntimeError, match='static array holds'):
        lib.call('hla_s6_attend_decode_static', *args)
    args[3] = 384
    with pytest.raises(ValueError, match='width'):
        lib.call('hla_s6_attend_decode_static', *args)


def test_joint_attention_kernels_refuse_bad_shapes_before_any_launch(pkg):
    """The merge / B_t and RoPE entry points of the HF engine's joint attention check their sizes first: no history
    block or more than 8, a width outside {256, 512}, a head_dim other than 128 (merge) or not a multiple of 16
    (RoPE), a tensor count outside {1, 2} raise ValueError without touching the device."""
    lib = pkg._lib

    def merge_args(parts, width, head_dim):
        args = [None if t is lib.P else 0 for t in lib.SIGNATURES['hla_s6_mixed_merge_forward']]
        args[0], args[1], args[2], args[3], args[4], args[10] = 2, 16, 8, width, head_dim, parts
        return args

    for parts, width, head_dim, match in ((0, 512, 128, 'history blocks'), (9, 512, 128, 'history blocks'),
                                          (1, 384, 128, 'width'), (1, 512, 64, 'head_dim')):
        with pytest.raises(ValueError, match=match):
            lib.call('hla_s6_mixed_merge_forward', *merge_args(parts, width, head_dim))
        bwd = [None if t is lib.P else 0 for t in lib.SIGNATURES['hla_s6_mixed_merge_backward']]
        bwd[:5], bwd[10] = merge_args(parts, width, head_dim)[:5], parts
        with pytest.raises(ValueError, match=match):
            lib.call('hla_s6_mixed_merge_backward', *bwd)
    for name in ('hla_s6_rope_rows_forward', 'hla_s6_rope_rows_backward'):
        for count, head_dim, match in ((3, 128, 'tensor count'), (0, 128, 'tensor count'), (2, 120, 'multiple of 16')):
            args = [None if t is lib.P else 0 for t in lib.SIGNATURES[name]]
            args[0], args[5], args[6], args[7], args[8] = count, 2, 16, 8, head_dim
            with pytest.raises(ValueError, match=match):
                lib.call(name, *args)
    be = importlib.import_module('hybrid-latent-attention_amd.batched_engine')
    assert be.MAX_BLOCKS == 8
