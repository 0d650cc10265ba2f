"""The ``s6-rollout-cache-v1`` snapshot of one finished request: every layer's committed latent rows, gathered
from the paged caches through the request's block lists before vLLM reuses the blocks, written as one file for
training replay.

Writer: ``hla/vllm_latent/cache_export.py:159-188`` (``RolloutCacheExporter.export``). The file is a ``torch.save``
dict ``{schema, version, request_id, cfg, prompt_ids, length, first_response_logits, rows}`` with ``rows`` a tuple of
per-layer ``[1, length, 2r + 2r1]`` tensors in the packed row layout of ``hla/latent/register.py:73-79``, readable
with ``torch.load(weights_only=True)``; the training side reads it with its own loader
(``hla/latent/history_snapshot.py:78-105``), which is not part of this package.

On MI355X the gather of all layers is ONE HIP launch (``hla_s6_gather_packed_rows``) into a device buffer, followed
by one device-to-host copy into pinned memory; the per-layer rows of the file are views of that one host buffer.
The vLLM runner hooks that decide WHEN to export (scheduler callbacks) are the serving engine's business and are not
part of this module.
"""
from __future__ import annotations

import os
import time

import torch

from . import _lib, s6_ops

SCHEMA = 's6-rollout-cache-v1'


class PackedRowGather:
    """The device gather of one request's committed rows over a fixed set of layer caches.

    ``layer_caches``: per layer ``(main_cache, l1_cache)``, each ``[num_blocks, 1, block_size, 2w]`` bf16 (the
    TRITON_ATTN layout the reference checks, ``cache_export.py:171-172``). The geometry is validated and the table of
    cache addresses uploaded once, here; each call then is one launch (capturable in a HIP graph when the block
    lists are already int32 device tensors)."""

    def __init__(self, layer_caches):
        if not layer_caches:
            raise ValueError('no layers to export')
        main0, l10 = layer_caches[0]
        s6_ops._dev(main0)
        self.device, self.dtype = main0.device, main0.dtype
        geo = []
        for c in (main0, l10):
            if c.ndim != 4 or c.shape[1] != 1:
                raise RuntimeError('Unsupported TRITON_ATTN cache layout')
            s6_ops._bf16('cache', c)
            geo.append((c.stride(0), c.stride(2), c.shape[-1] // 2, c.shape[0], c.shape[2]))
        for main, l1 in layer_caches:
            for c, g in ((main, geo[0]), (l1, geo[1])):
                if c.ndim != 4 or c.device != self.device or c.dtype != self.dtype or c.stride(0) != g[0] or \
                        c.stride(2) != g[1] or c.shape[-1] != 2 * g[2] or c.shape[0] != g[3] or \
                        c.shape[2] != g[4] or c.stride(-1) != 1:
                    raise ValueError('every layer cache of a group must share one geometry')
        self.geo, self.layers = geo, len(layer_caches)
        self.width = 2 * (geo[0][2] + geo[1][2])
        self.addrs = torch.tensor([c.data_ptr() for pair in layer_caches for c in pair],
                                  dtype=torch.int64).to(self.device)
        self.vector_ok = all(c.data_ptr() % 16 == 0 for pair in layer_caches for c in pair)
        self._caches = layer_caches                  # the addresses stay valid while this object lives

    def __call__(self, main_blocks, l1_blocks, length, out=None):
        """``[layers, length, 2r + 2r1]``: row ``pos`` of layer ``l`` is
        ``cache[blocks[pos // block_size], 0, pos % block_size, :]`` of both caches (``cache_export.py:173-175``)."""
        blocks = []
        for b, g in ((main_blocks, self.geo[0]), (l1_blocks, self.geo[1])):
            b = torch.as_tensor(b, dtype=torch.int32).to(self.device).contiguous()
            if b.numel() * g[4] < length:
                raise ValueError(f'{b.numel()} blocks of {g[4]} rows cannot hold {length} rows')
            blocks.append(b)
        if out is None:
            out = torch.empty(self.layers, length, self.width, dtype=self.dtype, device=self.device)
        elif tuple(out.shape) != (self.layers, length, self.width) or out.dtype != self.dtype or out.stride(-1) != 1:
            raise ValueError(f'out must be [{self.layers}, {length}, {self.width}] {self.dtype}')
        g0, g1 = self.geo
        _lib.call('hla_s6_gather_packed_rows', _lib.ptr(self.addrs), self.layers, g0[0], g0[1], g0[2], g0[3],
                  _lib.ptr(blocks[0]), g0[4], g1[0], g1[1], g1[2], g1[3], _lib.ptr(blocks[1]), g1[4], int(length),
                  _lib.ptr(out), out.stride(0), out.stride(1), int(self.vector_ok), _lib.stream(self.device))
        return out


def gather_packed_rows(layer_caches, main_blocks, l1_blocks, length):
    """``[layers, length, 2r + 2r1]`` device tensor of one request's committed rows (one ``PackedRowGather``
    launch); ``main_blocks`` / ``l1_blocks`` are the request's physical block ids per cache group (any device)."""
    return PackedRowGather(layer_caches)(main_blocks, l1_blocks, length)


def write_snapshot(path, rows, *, version, request_id, cfg, prompt_ids, length, first_response_logits):
    """Write the ``s6-rollout-cache-v1`` file (through a temporary name, then an atomic rename, as
    ``cache_export.py:180-184``). ``rows`` is ``[layers, length, R]`` on any device; a device tensor crosses to
    the host in one copy into pinned memory. Returns the exporter's per-request record
    ``{path, request_id, version, length, bytes}``."""
    if rows.ndim != 3 or rows.shape[1] != length:
        raise ValueError(f'rows must be [layers, {length}, R], got {tuple(rows.shape)}')
    if rows.is_cuda:
        host = torch.empty(rows.shape, dtype=rows.dtype, pin_memory=True)
        host.copy_(rows)                      # synchronous: the blocks may be reused once this returns
    else:
        host = rows.contiguous()
    payload = dict(schema=SCHEMA, version=version, request_id=request_id, cfg=cfg, prompt_ids=list(prompt_ids),
                   length=int(length), first_response_logits=first_response_logits,
                   rows=tuple(host[l:l + 1] for l in range(host.shape[0])))
    path = os.fspath(path)
    temp = os.path.splitext(path)[0] + '.tmp'
    torch.save(payload, temp)
    os.replace(temp, path)
    return dict(path=path, request_id=request_id, version=version, length=int(length), bytes=os.path.getsize(path))


def export_request(path, layer_caches, main_blocks, l1_blocks, length, *, version, request_id, cfg, prompt_ids,
                   first_response_logits):
    """Gather and write one finished request (``RolloutCacheExporter.export``); returns the per-request record
    plus ``seconds`` spent. ``layer_caches`` is a list of per-layer cache pairs or a ``PackedRowGather``."""
    tick = time.perf_counter()
    if first_response_logits is None:
        raise RuntimeError('Missing prompt logits at request retirement')
    gather = layer_caches if isinstance(layer_caches, PackedRowGather) else PackedRowGather(layer_caches)
    rows = gather(main_blocks, l1_blocks, length)
    record = write_snapshot(path, rows, version=version, request_id=request_id, cfg=cfg, prompt_ids=prompt_ids,
                            length=length, first_response_logits=first_response_logits)
    record['seconds'] = time.perf_counter() - tick
    return record
