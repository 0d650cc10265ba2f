#!/usr/bin/env python3
"""Benchmark of the S6 latent decode-attention path on one MI355X (Ouro-1.4B shape, B = 64, context 8192).

One step = the attention path of one full S6 decode step: 24 layers x 4 loops, each loop running the absorbed query
(A_t GEMM + latent RoPE), the exact window over the last 32 tokens plus the current one, the paged latent history
(loop 0 reads the 256-wide loop-1 latent, loops 1-3 the 512-wide main latent), the B_t projection and the LSE merge.
Inputs are synthetic and random-init, resident in HBM before timing; the whole step is captured once in a HIP graph
and replayed. The step is driven as the reference adapter drives it (one split count for the step from the
reference formula and the workspace it allocates; the layer code picks each latent width's count). Prints one JSON
line (the value is microseconds per layer = step time / 24; lower is better); its "configs" key holds the same
measurement of the other configurations (B=1 at context 1024 for one main loop; B=32 ragged contexts over 65,536-page
pools; B=8 at context 32768; chunked prefill of 4 requests x 3 and x 512 tokens on 8192 latent rows), each with its
roofline fraction and a CPU baseline (a torch-on-CPU restatement of the same layer path on the host's cores).
"""
from __future__ import annotations

import argparse
import importlib
import json
import math
import os
import re
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = 'latent decode-attn µs/layer + HBM GB/s (% peak), Ouro-1.4B S6, B=64 ctx 8K'
PEAK_HBM_GBPS = 8000.0
PEAK_BF16_TFLOPS = 2500.0
PEAK_FP32_TFLOPS = 157.3
TRAFFIC_PROFILE = os.path.join(ROOT, 'profiles', 'history_split_512_b64_ctx8192_pmc.md')
LAYERS, LOOPS, HEADS, HEAD_DIM, RANK, RANK1, WINDOW, BLOCK = 24, 4, 16, 128, 512, 256, 32, 16
MAX_POSITION = 65536


def parse():
    p = argparse.ArgumentParser(description=__doc__)
    p.add_argument('--gpus', type=int, default=1)
    p.add_argument('--steps', type=int, default=20)
    p.add_argument('--warmup', type=int, default=3)
    p.add_argument('--workload', choices=('decode', 'single', 'ragged', 'long', 'prefill', 'writer', 'export', 'khop',
                                          'rows', 'mixed'),
                   default='decode',
                   help='decode: the headline decode step (B=64, context 8192, 24 layers x 4 loops); single: B=1 '
                        'at context 1024, one layer x one main loop; ragged: B=32 decode rows with contexts drawn '
                        'from U[1024, 8192] over 65,536-page pools; long: B=8 decode rows at context 32768; prefill: '
                        'B=4 requests of --queries new tokens each on a context-8192 history (ragged, long and '
                        'prefill: 4 loops over 4 / 4 / 8 layers with distinct caches, reported per layer); writer: '
                        'the row writer and commit; export: the rollout-cache gather; khop: multi-query history with '
                        'backward (B=4, L=2880); rows: single-query history over contiguous rows with a key mask '
                        '(B=8, 8192 rows); mixed: the HF rolling engine\'s joint attention of a chunk over its '
                        'history blocks with backward (B=8, 256-token chunk, blocks of 2048 and 256 rows). Only '
                        'decode prints the headline line.')
    p.add_argument('--batch', type=int, default=0, help='rows (default: 64 / 1 / 32 / 8 / 4 by workload)')
    p.add_argument('--context', type=int, default=0, help='history tokens before the step (default by workload)')
    p.add_argument('--queries', type=int, default=512, help='new tokens per request of --workload prefill')
    p.add_argument('--writer-queries', type=int, default=1, help='new tokens per request of --workload writer')
    p.add_argument('--layers', type=int, default=0, help='layers (default by workload: 24 / 1 / 4 / 4 / 8)')
    p.add_argument('--splits', type=int, default=0,
                   help='KV splits of every latent width (0: the reference count, which StepContext turns into the '
                        'MI355X count per width)')
    p.add_argument('--max-model-len', type=int, default=0,
                   help="the adapter's max_model_len, which sizes the split counts (0: the step's longest sequence)")
    p.add_argument('--kernel-only', action='store_true', help='only launch the history op (profiling)')
    p.add_argument('--width', type=int, default=512, choices=(256, 512, 1024),
                   help='latent width of --kernel-only (256 / 512) and --workload khop / rows (1024: forward only)')
    p.add_argument('--copy-calibration', action='store_true',
                   help='only run a plain 1 GiB device copy three times (scales the FETCH_SIZE / WRITE_SIZE counters '
                        'of a PMC profile to bytes)')
    p.add_argument('--no-cpu-baseline', action='store_true')
    p.add_argument('--settle', type=float, default=60.0,
                   help='seconds of GPU idle between the heavy configurations of the default run (outside the timed '
                        'regions; 0: none)')
    p.add_argument('--no-secondary', action='store_true',
                   help='decode: skip the other configurations (single decode, ragged, long context, multi-query Q=3 '
                        'and Q=512) that the default run measures before the headline and reports under "configs"')
    p.add_argument('--precision', choices=('bf16', 'fp32', 'tf32'), default='bf16',
                   help='--workload khop: the history GEMM precision (fp32 / tf32: fp32 leaves and fp32 kernels)')
    p.add_argument('--seed', type=int, default=0)
    p.add_argument('--table', choices=('random', 'identity'), default='random',
                   help='latent block tables: a random permutation of the page pool, or pages in order')
    return p.parse_args()


# The adapter's step constants (hla/vllm_latent/ouro_latent.py:205-212): the largest CUDA-graph batch (vLLM's
# default capture size) bounds the split steps, and the workspace covers the scheduler's token budget
SPLIT_MAX_TOKENS, MAX_BATCHED_TOKENS = 512, 8192


class Workload:
    """Random-init caches, tables and readers of the model's attention path for one step: request r has ``hist[r]``
    history tokens and ``queries`` new tokens (1: a decode step; more: a chunked-prefill step whose tokens are
    already written to the exact cache), ``layers`` layers (each with its own caches) x the loops in ``loops``, run
    loop-major as the model runs them (every layer's loop 0, then every layer's loop 1, ...).

    The latent page pool of each width holds ``lat_pool`` pages (at least the pages the step uses plus the null
    page); each width's table is a slice of one random permutation of its pool. The step is driven as the
    reference adapter drives it (``hla/vllm_latent/ouro_latent.py:203-212,257-265``): one ``num_kv_splits`` count
    for the step from the reference formula, the workspace the adapter allocates, ``max_seqlen_k`` = the model
    length (``max_model_len``, by default the step's longest sequence); ``StepContext`` picks each width's count
    itself. ``splits_override`` instead fixes every width's count (``kv_splits_by_width``)."""

    def __init__(self, ops, layer, hist, queries, seed, device, cus, table='random', layers=LAYERS, lat_pool=0,
                 splits_override=0, loops=tuple(range(LOOPS)), max_model_len=0):
        g = torch.Generator(device=device).manual_seed(seed)
        hist = [int(h) for h in hist]
        B, Q = len(hist), int(queries)
        self.B, self.Q, self.T, self.hist, self.layers, self.device = B, Q, B * Q, hist, layers, device
        self.loops = tuple(loops)
        self.seq = [h + Q for h in hist]                          # the step's tokens are already in the exact cache
        self.n_latent = [max(h - WINDOW, 0) for h in hist]
        cols = [-(-s // BLOCK) for s in self.seq]
        self.cols = max(cols)
        randn = lambda *shape, std=1.0: (torch.randn(*shape, generator=g, device=device, dtype=torch.float32) * std
                                         ).to(torch.bfloat16)
        perm = lambda n: (torch.randperm(n - 1, generator=g, device=device) + 1).to(torch.int32)
        lat_pages = perm if table == 'random' else (lambda n: torch.arange(1, n, dtype=torch.int32, device=device))
        self.pool = max(int(lat_pool), sum(cols) + 1)             # page 0: the null page

        def paged_table(first, last, pages):
            t = torch.zeros(B, self.cols, dtype=torch.int32, device=device)
            used = 0
            for r in range(B):
                n = last[r] - first[r] + 1
                t[r, first[r]:last[r] + 1] = pages[used:used + n]
                used += n
            return t

        self.lat_table = {w: paged_table([0] * B, [c - 1 for c in cols], lat_pages(self.pool)) for w in (RANK, RANK1)}
        self.lat = [{w: torch.empty(self.pool, 1, BLOCK, 2 * w, dtype=torch.bfloat16, device=device).normal_(
                     generator=g) for w in (RANK, RANK1)} for _ in range(layers)]
        # exact caches: the window rows and the step's tokens per request and loop; freed pages are the null page
        first = [max(0, h - WINDOW) // BLOCK for h in hist]
        last = [(s - 1) // BLOCK for s in self.seq]
        ex_pool = sum(l - f + 1 for f, l in zip(first, last)) + 1
        self.ex_table = [paged_table(first, last, perm(ex_pool)) for _ in range(LOOPS)]
        self.exact = [[randn(ex_pool, HEADS, BLOCK, 2 * HEAD_DIM) for _ in range(LOOPS)] for _ in range(layers)]
        std = 1 / math.sqrt(2048)
        self.readers = [_Reader(randn(HEADS, HEAD_DIM, RANK1, std=std), randn(HEADS, RANK1, HEAD_DIM, std=std),
                                randn(3, HEADS, HEAD_DIM, RANK, std=std), randn(3, HEADS, RANK, HEAD_DIM, std=std))
                        for _ in range(layers)]
        inv = layer.latent_inv_freq(HEAD_DIM, 1e6).to(device)
        self.tables = {w: layer.latent_rope_table(MAX_POSITION, inv, w, torch.bfloat16) for w in (RANK, RANK1)}
        T = self.T
        self.q_pre = [randn(T, HEADS, HEAD_DIM) for _ in range(LOOPS)]
        self.q_rope = [randn(T, HEADS, HEAD_DIM) for _ in range(LOOPS)]
        self.k_rope = [randn(T, HEADS, HEAD_DIM) for _ in range(LOOPS)] if Q > 1 else [None] * LOOPS
        self.v = [randn(T, HEADS, HEAD_DIM) for _ in range(LOOPS)] if Q > 1 else [None] * LOOPS
        self.positions = torch.tensor([h + i for h in hist for i in range(Q)], dtype=torch.int64, device=device)
        self.qsl = (torch.arange(B + 1, dtype=torch.int32, device=device) * Q).contiguous()
        self.seq_lens = torch.tensor(self.seq, dtype=torch.int32, device=device)
        self.ops, self.layer = ops, layer
        self.max_model_len = max(int(max_model_len), max(self.seq))
        if splits_override:
            self.by_width = {RANK: int(splits_override), RANK1: int(splits_override)}
            self.ref_splits = int(splits_override)
            self.workspace = ops.S6Workspace.for_splits(HEADS, T, self.by_width)
        else:
            self.by_width = None
            ref = lambda t: ops.num_kv_splits(self.max_model_len, t, SPLIT_MAX_TOKENS, cus)
            self.ref_splits = ref(T)
            rows = max(MAX_BATCHED_TOKENS, max(t * ref(t) for t in range(1, SPLIT_MAX_TOKENS + 1)))
            self.workspace = ops.S6Workspace(HEADS, RANK, rows)
        ctx = self.context()
        self.splits = {w: ctx.kv_splits(w) for w in (RANK, RANK1)}   # {latent width: KV splits} the step runs

    def context(self):
        """The step's StepContext, built with the adapter's arguments (``ouro_latent.py:263-265``)."""
        return self.layer.StepContext(self.positions, self.qsl, self.seq_lens, self.Q, self.T, self.tables,
                                      HEAD_DIM ** -0.5, self.ops.HIP_BACKENDS, self.workspace, self.ref_splits,
                                      window=WINDOW, max_seqlen_k=self.max_model_len,
                                      kv_splits_by_width=self.by_width)

    def step(self):
        ctx, layer = self.context(), self.layer
        outs = []
        for loop in self.loops:
            w = RANK1 if loop == 0 else RANK
            for i in range(self.layers):
                sl = self.readers[i]
                q_lat = ctx.latent_query(sl, loop, self.q_pre[loop])
                outs.append(layer.attend(sl, loop, q_lat, self.q_rope[loop], self.k_rope[loop], self.v[loop],
                                         self.lat[i][w], self.lat_table[w], None, None, ctx,
                                         (self.exact[i][loop], self.ex_table[loop])))
        return outs

    def setup(self):
        """The step's per-step launches alone: metadata and the split plan of each width that the fused path
        reads (shared by every layer of the step)."""
        ctx = self.context()
        if self.Q < self.layer.FUSED_CHUNK_TOKENS:
            for w in (RANK, RANK1):
                if any((RANK1 if l == 0 else RANK) == w for l in self.loops) and ctx.kv_splits(w) > 1:
                    ctx.split_plan(ctx.kv_splits(w), self.lat_table[w].shape[1] * BLOCK)

    def widths(self):
        return [RANK1 if loop == 0 else RANK for loop in self.loops]

    def history_bytes_per_layer(self):
        """Latent rows read once per request and loop: 2 x (256 or 512) bf16 columns per row."""
        return sum(self.n_latent) * sum(2 * w * 2 for w in self.widths())

    def history_flops_per_layer(self):
        """4 flops per (query row, latent row, latent column): scores and weighted values."""
        return sum(4 * self.Q * HEADS * n * sum(self.widths()) for n in self.n_latent)

    def window_bytes_per_layer(self):
        keys = sum(min(s, WINDOW + self.Q) for s in self.seq)
        return len(self.loops) * keys * HEADS * 2 * HEAD_DIM * 2


class _Reader:
    def __init__(self, A1, B1, A, B):
        self.A1, self.B1, self.A, self.B = A1, B1, A, B
        self.rank1, self.rank, self.loops = RANK1, RANK, LOOPS

    def readers(self, loop):
        return (self.A1, self.B1, RANK1) if loop == 0 else (self.A[loop - 1], self.B[loop - 1], RANK)


def time_graph(fn, steps, warmup):
    """Capture ``fn`` in a HIP graph, replay ``warmup`` times untimed, then time ``steps`` replays with events."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn()
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def measured_traffic(path=TRAFFIC_PROFILE):
    """HBM bytes per launch of the roofline kernel from its committed rocprofv3 PMC summary (FETCH_SIZE and
    WRITE_SIZE scaled by a plain-copy calibration), or None when the summary is absent."""
    try:
        with open(path) as f:
            m = re.search(r'^traffic_bytes_per_launch:\s*(\d+)', f.read(), re.M)
    except OSError:
        return None
    return int(m.group(1)) if m else None


def history_roofline(wl, iters=50, width=RANK):
    """The dominant kernel of the step, the split-KV history kernel (stage 1 of the history op, with the step's
    split plan as in the decode step), launched alone over the main latent of every layer in turn: its average
    duration from HIP events on the stream it runs on,
    the average duration of the stage-2 reduction likewise, and the algorithmic bytes stage 1 reads (every latent
    K and V row of every token once)."""
    ops = wl.ops
    ctx_lat = torch.tensor(wl.n_latent, dtype=torch.int32, device=wl.device)
    q = torch.randn(wl.B, HEADS, width, device=wl.device).to(torch.bfloat16) * (width ** -0.5)
    caches = [wl.lat[i][width] for i in range(wl.layers)]
    splits = wl.splits[width]
    plan = ops.split_plan(ctx_lat, wl.lat_table[width].shape[1] * BLOCK, splits) if splits > 1 else None

    def stage1(i):
        c = caches[i % len(caches)]
        return ops.history_partials(q, c[..., :width], c[..., width:], wl.lat_table[width], ctx_lat, HEAD_DIM ** -0.5,
                                    splits, wl.workspace, plan=plan)

    def timed(fn):
        for i in range(5):
            fn(i)
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for i in range(iters):
            fn(i)
        end.record(stream)
        torch.cuda.synchronize()
        return start.elapsed_time(end) * 1000 / iters

    us = timed(stage1)
    part = stage1(0)
    us_reduce = timed(lambda i: ops.history_reduce(part))
    nbytes = sum(wl.n_latent) * 2 * width * 2
    return us, us_reduce, nbytes


def cpu_baseline(wl, timed_loops, per_request=0):
    """The torch-on-CPU restatement of the layer's attention path (``oracle/torch_cpu.py``: A_t + latent RoPE, paged
    latent history, B_t, the exact window or chunk, LSE merge; float32 GEMMs from bf16 inputs on all of the host's
    cores) over layer 0's caches, one call per loop in ``timed_loops`` (median of 3 after a warm-up). Decode steps
    run every row; multi-query steps every request, on its first ``per_request`` tokens when that is set (scaled to
    all of its tokens). Loops not timed are the main-latent loop 1's time again (loops 1-3 read the same
    caches and shapes). Returns the baseline dict (microseconds per layer, or per call for a one-loop step)."""
    from oracle import torch_cpu as TC
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    cpu = lambda t: t.cpu()
    multi = wl.Q > 1
    take = per_request if (multi and per_request) else wl.Q
    tokens = torch.tensor([r * wl.Q + i for r in range(wl.B) for i in range(take)], device=wl.device)
    T = tokens.numel()
    timings = {}
    for loop in timed_loops:
        w = RANK1 if loop == 0 else RANK
        A, Bw, _ = wl.readers[0].readers(loop)
        cols = max(1, -(-max(wl.n_latent) // BLOCK))
        pages = wl.lat_table[w][:, :cols].long()                       # the pages the requests read, compacted
        lat_h = cpu(wl.lat[0][w][pages.reshape(-1)]).view(wl.B * cols, 1, BLOCK, 2 * w)
        lat_tab = torch.arange(wl.B * cols, dtype=torch.int32).view(wl.B, cols)
        ex_h, ex_tab = cpu(wl.exact[0][loop]), cpu(wl.ex_table[loop])
        q_pre, rows = cpu(wl.q_pre[loop][tokens]), cpu(wl.tables[w][wl.positions[tokens]])
        q_rope = cpu(wl.q_rope[loop][tokens])
        A, Bw = cpu(A), cpu(Bw)
        invalid = torch.zeros(T, dtype=torch.bool)
        n_lat = torch.tensor(wl.n_latent, dtype=torch.int32)
        if multi:
            k_rope, v = cpu(wl.k_rope[loop][tokens]), cpu(wl.v[loop][tokens])
            qsl = [r * take for r in range(wl.B + 1)]

            def run():
                q_lat = TC.latent_query(q_pre, A, rows)
                return TC.attend_chunk(q_lat, q_rope, k_rope, v, Bw, lat_h, lat_tab, qsl, wl.hist, n_lat, ex_h,
                                       ex_tab, WINDOW, HEAD_DIM ** -0.5, invalid)
        else:
            req = torch.arange(wl.B)
            seq = torch.tensor(wl.seq, dtype=torch.int32)

            def run():
                q_lat = TC.latent_query(q_pre, A, rows)
                return TC.attend_decode(q_lat, q_rope, Bw, lat_h, lat_tab, n_lat, ex_h, ex_tab, req, seq, WINDOW,
                                        HEAD_DIM ** -0.5, invalid)
        run()
        reps = []
        for _ in range(3):
            t0 = time.perf_counter()
            run()
            reps.append(time.perf_counter() - t0)
        timings[loop] = float(np.median(reps))
    per_loop = [timings.get(loop, timings.get(1)) for loop in wl.loops]
    scale = wl.Q / take
    value = sum(per_loop) * scale * 1e6
    whole = set(timed_loops) == set(wl.loops) and scale == 1
    what = (f'all {wl.B} decode rows' if not multi else
            f'all {wl.B} requests x {take} of their {wl.Q} tokens' if take < wl.Q else f'all {wl.T} tokens')
    note = ('the whole call' if whole else
            f'loops {list(timed_loops)} timed, the untimed main loops counted at loop 1\'s time'
            + (f', x{scale:.0f} tokens' if scale > 1 else '') + '; extrapolated')
    return {'value': round(value, 1), 'unit': 'us/call' if len(wl.loops) == 1 else 'us/layer', 'cores': cores,
            'kind': 'port',
            'sample': f'torch-on-CPU restatement of the layer path (A_t + latent RoPE, paged history, B_t, exact '
                      f'window or chunk, LSE merge; float32 GEMMs from bf16, {cores} threads) on {what} of layer 0, '
                      f'median of 3 after a warm-up: {note}'}


def secondary_metrics(name, kind, wl, B, context, queries, steps, warmup):
    """Step time and roofline fractions of a configuration other than the headline (HIP-graph replay). ``value`` is
    the step time per layer (per call when the step is one loop); the step's setup launches, shared by its layers
    as in the model, are timed alone beside it."""
    ms = time_graph(wl.step, steps, warmup)
    setup_ms = time_graph(wl.setup, steps, warmup)
    per = 'call' if len(wl.loops) == 1 else 'layer'
    us_layer = ms * 1000 / wl.layers
    hist_bytes, flops = wl.history_bytes_per_layer(), wl.history_flops_per_layer()
    gbps, tflops = hist_bytes / (us_layer * 1e3), flops / (us_layer * 1e6)
    return {'workload': name, 'value': round(us_layer, 2), 'unit': f'us/{per}', 'B': B, 'queries': queries,
            'context': context, 'contexts': wl.hist if kind == 'ragged' else None, 'layers': wl.layers,
            'loops': len(wl.loops), 'latent_pool_pages': wl.pool, 'kv_splits': wl.splits,
            'reference_kv_splits': wl.ref_splits, 'max_model_len': wl.max_model_len, 'steps': steps,
            'ms_per_step': round(ms, 4),
            'setup_us_per_step': round(setup_ms * 1000, 2),
            'history_bytes_per_layer': hist_bytes, 'history_gbps': round(gbps, 1),
            'hbm_frac': round(gbps / PEAK_HBM_GBPS, 4), 'history_flops_per_layer': flops,
            'history_tflops': round(tflops, 1), 'mfma_frac': round(tflops / PEAK_BF16_TFLOPS, 4),
            'bound': 'mfma' if kind == 'prefill' and queries >= 64 else 'hbm' if kind != 'single' else 'latency',
            'data': 'synthetic (random-init caches, readers and queries)', 'hip_graph': True}


# The benchmark configurations besides the headline (name: workload, B, context, queries, layers, latent pool pages,
# loops, CPU-baseline loops, CPU-baseline tokens per request), in the order the default run measures them (each heavy
# one after `--settle` seconds of GPU idle, see settle()). Layers are distinct caches run loop-major, so
# that a loop's history reads (over all the step's layers) exceed the 256 MB MALL as in the 24-layer model and no
# loop re-reads the previous loop's rows from it; the ragged step reads its rows from 65,536-page pools per width.
SECONDARY = (
    ('long_b8_ctx32768', 'long', 8, 32768, 1, 4, 0, (0, 1, 2, 3), (0, 1, 2, 3), 0),
    ('ragged_b32_ctx1024_8192', 'ragged', 32, 8192, 1, 4, 65536, (0, 1, 2, 3), (0, 1, 2, 3), 0),
    ('single_b1_ctx1024', 'single', 1, 1024, 1, 1, 0, (1,), (1,), 0),
    ('prefill_b4_q3_ctx8192', 'prefill', 4, 8192, 3, 8, 0, (0, 1, 2, 3), (0, 1, 2, 3), 0),
    ('prefill_b4_q512_ctx8192', 'prefill', 4, 8192, 512, 8, 0, (0, 1, 2, 3), (0, 1), 16),
)


def workload_shape(kind, B, context, seed):
    """History lengths of the requests of a workload."""
    if kind == 'ragged':
        return np.random.default_rng(seed).integers(1024, context + 1, B).tolist()
    if kind == 'prefill':
        return [context + WINDOW] * B                          # `context` latent rows + the exact window
    return [context] * B


def build_workload(ops, layer, kind, B, context, layers, queries, seed, device, cus, splits_override=0,
                   table='random', lat_pool=0, loops=tuple(range(LOOPS)), max_model_len=0):
    hist = workload_shape(kind, B, context, seed)
    print(f'bench: building workload {kind} B={B} queries={queries} max ctx={max(hist)} layers={layers} '
          f'pool={lat_pool} loops={loops} cus={cus}', file=sys.stderr, flush=True)
    wl = Workload(ops, layer, hist, queries, seed, device, cus, 'identity' if kind == 'single' else table, layers,
                  lat_pool, splits_override, loops, max_model_len)
    torch.cuda.synchronize()
    return wl


def settle(seconds, last, name):
    """Idle the GPU until ``seconds`` have passed since the previous heavy measurement ended (``last``, a
    time.monotonic() stamp; None: nothing measured yet). Within about a minute of a heavy HBM-bound step the next
    one ran 2-4 % slower on the MI355X (ragged decode 271.8 against 261-264 us/layer right after the long-context
    step), and 60 s idle restored the fresh-device rate. The wait is outside every timed region and overlaps the
    previous configuration's CPU baseline."""
    if last is None or seconds <= 0:
        return
    wait = seconds - (time.monotonic() - last)
    if wait > 0:
        print(f'bench: {wait:.0f} s idle before {name}', file=sys.stderr, flush=True)
        time.sleep(wait)


def measure_secondaries(ops, layer, args, device, cus, with_cpu):
    """Every configuration of SECONDARY, one after another (each workload freed before the next is built): a dict
    of their metrics (with their CPU baselines) for the headline line, and when the last heavy one ended."""
    out = {}
    last = None
    for name, kind, B, context, queries, layers, pool, loops, cpu_loops, cpu_tokens in SECONDARY:
        wl = build_workload(ops, layer, kind, B, context, layers, queries, args.seed, device, cus, lat_pool=pool,
                            loops=loops)
        if kind != 'single':
            settle(args.settle, last, name)
        out[name] = secondary_metrics(name, kind, wl, B, context, queries, args.steps, args.warmup)
        if kind != 'single':
            last = time.monotonic()
        if with_cpu:
            print(f'bench: cpu baseline of {name}', file=sys.stderr, flush=True)
            out[name]['cpu_baseline'] = cpu_baseline(wl, cpu_loops, cpu_tokens)
        del wl
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
    return out, last


def single_config(args, ops, layer, device, cus):
    """One JSON line for one configuration of SECONDARY (``--workload single|ragged|long|prefill``; prefill picks
    the entry of ``--queries`` tokens when there is one, else the 512-token entry's shape); ``--batch``,
    ``--context``, ``--layers`` and ``--splits`` override its shape."""
    entries = [e for e in SECONDARY if e[1] == args.workload]
    if args.workload == 'prefill':
        entries = [e for e in entries if e[4] == args.queries] or [e for e in entries if e[4] == 512]
    name, kind, B, context, queries, layers, pool, loops, cpu_loops, cpu_tokens = entries[0]
    if kind == 'prefill':
        queries = args.queries
        cpu_tokens = min(cpu_tokens, queries) if cpu_tokens else 0
    B, context, layers = args.batch or B, args.context or context, args.layers or layers
    wl = build_workload(ops, layer, kind, B, context, layers, queries, args.seed, device, cus, args.splits,
                        args.table, pool, loops, args.max_model_len)
    out = secondary_metrics(name, kind, wl, B, context, queries, args.steps, args.warmup)
    out['cpu_baseline'] = None if args.no_cpu_baseline else cpu_baseline(wl, cpu_loops, cpu_tokens)
    print(json.dumps(out), flush=True)


HIDDEN = 2048


def writer_workload(args, layer, device):
    """The writer of a step, per layer: loop 0 projects and commits the loop-1 row, loops 1-2 accumulate the register,
    loop 3 accumulates and commits the main row (``write_commit``: one launch per loop). ``--batch`` requests of
    ``--queries`` new tokens each (decode: 1), 24 layers, random-init nn.Linear weights; one JSON line."""
    import types
    B = args.batch or 64
    Q = args.writer_queries
    T, layers = B * Q, args.layers or LAYERS
    g = torch.Generator(device=device).manual_seed(args.seed)
    bf = torch.bfloat16

    def rnd(*shape, std=1.0):
        return (torch.randn(*shape, generator=g, device=device) * std).to(bf)

    sls = []
    for _ in range(layers):
        sl = types.SimpleNamespace(rank=RANK, rank_v=RANK, rank1=RANK1, loops=LOOPS, head_dim=HEAD_DIM)
        sl.cand1 = types.SimpleNamespace(weight=rnd(2 * RANK1, HIDDEN, std=HIDDEN ** -0.5))
        sl.cand_s = [types.SimpleNamespace(weight=rnd(2 * RANK, HIDDEN, std=HIDDEN ** -0.5)) for _ in range(LOOPS - 1)]
        sls.append(sl)
    hs = [rnd(T, HIDDEN) for _ in range(LOOPS)]
    seq = torch.full((B,), 8192, dtype=torch.int32, device=device)
    qsl = torch.arange(0, T + 1, Q, dtype=torch.int32, device=device)
    positions = (seq.long()[:, None] - Q + torch.arange(Q, device=device)[None]).reshape(-1)
    pages = (8192 + BLOCK - 1) // BLOCK
    pool = B * pages + 1
    table = (1 + torch.randperm(pool - 1, device=device)[:B * pages]).view(B, pages).to(torch.int32)
    inv = layer.latent_inv_freq(HEAD_DIM, 1e6).to(device)
    tables = {w: layer.latent_rope_table(MAX_POSITION, inv, w, bf) for w in (RANK, RANK1)}
    caches = {w: torch.zeros(pool, 1, BLOCK, 2 * w, dtype=bf, device=device) for w in (RANK, RANK1)}
    ctx = layer.StepContext(positions, qsl, seq, Q, T, tables, HEAD_DIM ** -0.5, layer.s6_ops.HIP_BACKENDS)
    ctx.slots(table, BLOCK)                                   # the step's slots, computed outside the timed graph

    def step():
        for sl in sls:
            state = None
            for loop in range(LOOPS):
                state = layer.write_commit(sl, loop, hs[loop], state, ctx, caches[RANK1 if loop == 0 else RANK], table)

    ms = time_graph(step, args.steps, args.warmup)
    us_layer = ms * 1000 / layers
    weight_bytes = (2 * RANK1 + 3 * 2 * RANK) * HIDDEN * 2
    act_bytes = 4 * T * HIDDEN * 2 + T * 2 * RANK * 2 * 4 + T * 2 * (RANK + RANK1) * 2   # h; register; rows
    nbytes = weight_bytes + act_bytes
    flops = 2 * T * HIDDEN * (2 * RANK1 + 3 * 2 * RANK)
    base = None
    if not args.no_cpu_baseline:
        from oracle import s6_oracle as O
        f32 = lambda t: t.float().cpu().numpy()
        W = [f32(sls[0].cand1.weight)] + [f32(w.weight) for w in sls[0].cand_s]
        H = [f32(h) for h in hs]
        pos = positions.cpu().numpy()
        tab_h = {w: f32(t) for w, t in tables.items()}

        def run():
            first = O.write_step(H[0], W[0], dtype=np.float32)
            O.committed_row(first, RANK1, pos, tab_h[RANK1])
            reg = None
            for loop in range(1, LOOPS):
                reg = O.write_step(H[loop], W[loop], reg, dtype=np.float32)
            return O.committed_row(reg, RANK, pos, tab_h[RANK])
        run()
        times = []
        for _ in range(3):
            t0 = time.perf_counter()
            run()
            times.append(time.perf_counter() - t0)
        base = {'value': round(float(np.median(times)) * 1e6, 1), 'unit': 'us/layer',
                'cores': len(os.sched_getaffinity(0)), 'kind': 'port',
                'sample': f'one layer (4 loops) of the writer on all {T} tokens, numpy float32 GEMMs, median of 3'}
    print(json.dumps({'workload': 'writer', 'value': round(us_layer, 2), 'unit': 'us/layer', 'tokens': T,
                      'layers': layers, 'launches_per_layer': LOOPS, 'steps': args.steps, 'ms_per_step': round(ms, 4),
                      'bytes_per_layer': nbytes, 'gbps': round(nbytes / (us_layer * 1e3), 1),
                      'hbm_frac': round(nbytes / (us_layer * 1e3) / PEAK_HBM_GBPS, 4), 'flops_per_layer': flops,
                      'tflops': round(flops / (us_layer * 1e6), 2),
                      'data': 'synthetic (random-init nn.Linear weights and hidden states)', 'hip_graph': True,
                      'cpu_baseline': base}), flush=True)


def export_workload(args, pkg, device):
    """The s6-rollout-cache-v1 export of one finished request of ``--context`` rows (default 8192): the one-launch
    gather of all 24 layers' main and loop-1 rows through random block lists (timed in a HIP graph: value, GB/s of
    read + write), then once the whole export (gather, one pinned device-to-host copy, torch.save) to a temporary
    file, reported beside it. One JSON line."""
    import tempfile
    rc = pkg.rollout_cache
    length, layers = args.context or 8192, args.layers or LAYERS
    pages = -(-length // BLOCK)
    pool = 4 * pages + 1
    g = torch.Generator(device=device).manual_seed(args.seed)
    caches = [tuple((torch.randn(pool, 1, BLOCK, 2 * w, generator=g, device=device)).to(torch.bfloat16)
                    for w in (RANK, RANK1)) for _ in range(layers)]
    blocks = [torch.randperm(pool, generator=g, device=device)[:pages].to(torch.int32) for _ in range(2)]
    gather = rc.PackedRowGather(caches)
    rows = torch.empty(layers, length, 2 * (RANK + RANK1), dtype=torch.bfloat16, device=device)

    def step():
        gather(blocks[0], blocks[1], length, out=rows)
    ms = time_graph(step, args.steps, args.warmup)
    nbytes = 2 * layers * length * 2 * (2 * RANK + 2 * RANK1)
    logits = torch.zeros(1, 1, 16)
    with tempfile.TemporaryDirectory() as tmp:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        ref = rc.export_request(os.path.join(tmp, '0.pt'), gather, blocks[0], blocks[1], length, version=0,
                                request_id='bench', cfg=dict(num_layers=layers, rank=RANK, rank_v=RANK, rank1=RANK1),
                                prompt_ids=[0], first_response_logits=logits)
        whole = time.perf_counter() - t0
    base = None
    if not args.no_cpu_baseline:
        # the same gather on host copies of layer 0's caches (numpy fancy indexing), scaled by the layers
        main_h, l1_h = (c.view(torch.int16).cpu().numpy() for c in caches[0])
        bl = [b.long().cpu().numpy() for b in blocks]
        pos = np.arange(length)

        def run():
            return np.concatenate((main_h[bl[0][pos // BLOCK], 0, pos % BLOCK], l1_h[bl[1][pos // BLOCK], 0, pos % BLOCK]),
                                  -1)
        run()
        times = []
        for _ in range(3):
            t0 = time.perf_counter()
            run()
            times.append(time.perf_counter() - t0)
        base = {'value': round(float(np.median(times)) * 1e6 * layers, 1), 'unit': 'us/request', 'cores': 1,
                'kind': 'port', 'sample': f'numpy gather of layer 0 ({length} rows of both caches) on host copies, '
                                          f'median of 3, x{layers} layers; extrapolated'}
    print(json.dumps({'workload': 'export', 'value': round(ms * 1000, 2), 'unit': 'us/request (device gather)',
                      'rows': length, 'layers': layers, 'row_bytes': 2 * (2 * RANK + 2 * RANK1),
                      'bytes_moved': nbytes, 'gbps': round(nbytes / (ms * 1e6), 1),
                      'hbm_frac': round(nbytes / (ms * 1e6) / PEAK_HBM_GBPS, 4), 'steps': args.steps,
                      'whole_export_ms': round(whole * 1000, 1), 'file_bytes': ref['bytes'],
                      'data': 'synthetic (random caches and block lists)', 'hip_graph': True,
                      'cpu_baseline': base}), flush=True)


def khop_workload(args, pkg, device):
    """Multi-query causal history attention with backward at the reference's operator benchmark shape
    (hla/latent/benchmark_history_gemm.py:79-101): B = 4, 16 heads, L = 2880 queries and keys, latent width
    ``--width`` (512 default), valid lengths L, 0.9 L, 0.8 L, 0.7 L, query i sees keys j < i. Times the forward (in
    a HIP graph) and the forward + backward (dq, dk, dv through autograd, returned as the reference's benchmark does
    with torch.autograd.grad) at ``--precision`` (bf16: bf16 leaves and operands; fp32 / tf32: fp32 leaves, the fp32
    kernels, as the reference benchmark's gemm-fp32 / gemm-tf32 rows); reports TFLOP/s of the algorithmic work (2
    GEMMs forward, 7 with the backward, over the visible pairs) against the dense MFMA peak of the arithmetic (bf16
    2.5 PFLOP/s, fp32 157.3 TFLOP/s) and the reference's published A100 times of the same backend and shape. One
    JSON line."""
    hg = pkg.history_gemm
    B, L, R = args.batch or 4, args.context or 2880, args.width
    g = torch.Generator(device=device).manual_seed(args.seed)
    prec = args.precision
    leaf = torch.bfloat16 if prec == 'bf16' else torch.float32
    q = torch.randn(B, L, HEADS, R, generator=g, device=device).to(leaf).requires_grad_(True)
    k = torch.randn(B, L, R, generator=g, device=device).to(leaf).requires_grad_(True)
    v = torch.randn(B, L, R, generator=g, device=device).to(leaf).requires_grad_(True)
    lengths = torch.tensor([max(2, int(L * (1 - 0.1 * i))) for i in range(B)], device=device)
    valid = torch.arange(L, device=device)[None] < lengths[:, None]
    order = torch.arange(L, device=device)[:, None] > torch.arange(L, device=device)[None]
    mask = valid[:, :, None] & valid[:, None, :] & order[None]
    pairs = int(mask.sum().item())
    scale = 1 / math.sqrt(HEAD_DIM)
    dz = torch.randn(B, L, HEADS, R, generator=g, device=device).to(leaf)
    dlse = torch.randn(B, HEADS, L, generator=g, device=device)

    def fwd():
        with torch.no_grad():
            hg.causal_history_gemm(q, k, v, mask, scale, causal=True, precision=prec)

    def train():  # gradients returned, not accumulated into .grad (as the reference's operator benchmark does)
        z, lse = hg.causal_history_gemm(q, k, v, mask, scale, causal=True, precision=prec)
        torch.autograd.grad([z, lse], [q, k, v], [dz, dlse])

    ms_f = time_graph(fwd, args.steps, args.warmup)
    ms_t = time_eager(train, args.steps, args.warmup)
    f_fwd, f_all = hg.flops(pairs, HEADS, R), hg.flops(pairs, HEADS, R, with_backward=True)
    base = None
    if not args.no_cpu_baseline:
        # the oracle's forward + backward (numpy float32) on the last 64 queries of request 0 over all its keys,
        # scaled by visible (query, key) pairs
        from oracle import s6_oracle as O
        f32 = lambda t: t.detach().float().cpu().numpy()
        n_q = 64
        qs, ks, vs = f32(q[:1, L - n_q:]), f32(k[:1]), f32(v[:1])
        ms_ = mask[:1, L - n_q:].cpu().numpy()
        dzs, dls = f32(dz[:1, L - n_q:]), f32(dlse[:1, :, L - n_q:])

        def run():
            z_, l_ = O.causal_history(qs, ks, vs, ms_, scale, dtype=np.float32)
            if ms_t is None:
                return z_
            return O.causal_history_backward(qs, ks, vs, ms_, scale, l_, dzs, dls, dtype=np.float32)
        run()
        times = []
        for _ in range(3):
            t0 = time.perf_counter()
            run()
            times.append(time.perf_counter() - t0)
        sample_pairs = int(ms_.sum())
        base = {'value': round(float(np.median(times)) * 1e3 * pairs / sample_pairs, 1),
                'unit': 'ms per forward+backward' if ms_t else 'ms per forward',
                'cores': len(os.sched_getaffinity(0)), 'kind': 'port',
                'sample': f'numpy oracle forward{" + backward" if ms_t else ""} (float32) on the last {n_q} '
                          f'queries of request 0 '
                          f'({sample_pairs} visible pairs), median of 3, scaled by visible pairs ({pairs}); '
                          f'extrapolated'}
    # the reference's published A100 times (ms) at this shape: forward, forward + backward of dq, dk, dv
    # (results/latent/history-gemm-bench-0923-summary.json, gemm-<precision> rows at length 2880)
    published = {('bf16', 1024): (19.02, 60.33), ('bf16', 256): (13.34, 38.34), ('fp32', 1024): (76.07, 261.84),
                 ('fp32', 256): (30.39, 99.20), ('tf32', 1024): (23.08, 73.50),
                 ('tf32', 256): (13.71, 39.18)}.get((prec, R)) if (B, L) == (4, 2880) else None
    peak = PEAK_BF16_TFLOPS if prec == 'bf16' else PEAK_FP32_TFLOPS
    print(json.dumps({'workload': 'khop', 'precision': prec, 'value': round(ms_t, 3),
                      'unit': 'ms per forward+backward', 'forward_ms': round(ms_f, 3), 'B': B, 'L': L,
                      'heads': HEADS, 'width': R, 'visible_pairs': pairs,
                      'forward_tflops': round(f_fwd / (ms_f * 1e9), 1), 'train_tflops': round(f_all / (ms_t * 1e9), 1),
                      'mfma_peak_tflops': peak, 'forward_mfma_frac': round(f_fwd / (ms_f * 1e9) / peak, 4),
                      'train_mfma_frac': round(f_all / (ms_t * 1e9) / peak, 4),
                      'reference_a100_ms': None if published is None else {'forward': published[0],
                                                                          'forward_backward': published[1]},
                      'steps': args.steps,
                      'data': 'synthetic (randn q, k, v, cotangents)', 'forward_hip_graph': True,
                      'cpu_baseline': base}), flush=True)


def rows_workload(args, pkg, device):
    """Single-query history attention over contiguous rows with a key mask: the HF rolling engine's history call
    (``hla/latent/fused_history.py:49-54``) at its decode shape, B = 8 rows of ``--context`` (8192) latent rows of
    width ``--width`` (512), padding masks (valid lengths N, 0.95 N, ..., and every 7th key of row 1 hidden). Times
    the forward (bounds, split kernel and reduction in a HIP graph; HBM GB/s of the rows up to each row's last
    visible key plus the mask) and the forward + backward through autograd (dq, dk, dv). One JSON line."""
    hg = pkg.history_gemm
    B, N, R = args.batch or 8, args.context or 8192, args.width
    g = torch.Generator(device=device).manual_seed(args.seed)
    q = (torch.randn(B, HEADS, R, generator=g, device=device) * R ** -0.5).to(torch.bfloat16).requires_grad_(True)
    k = torch.randn(B, N, R, generator=g, device=device).to(torch.bfloat16).requires_grad_(True)
    v = torch.randn(B, N, R, generator=g, device=device).to(torch.bfloat16).requires_grad_(True)
    lengths = torch.tensor([max(1, int(N * (1 - 0.05 * i))) for i in range(B)], device=device)
    mask = torch.arange(N, device=device)[None] < lengths[:, None]
    if B > 1:
        mask[1, ::7] = False
    scale = 1 / math.sqrt(HEAD_DIM)
    dz = torch.randn(B, HEADS, R, generator=g, device=device).to(torch.bfloat16)
    dlse = torch.randn(B, HEADS, generator=g, device=device)

    def fwd():
        with torch.no_grad():
            hg.history_attention(q, k, v, mask, scale)

    def train():
        z, lse = hg.history_attention(q, k, v, mask, scale)
        torch.autograd.grad([z, lse], [q, k, v], [dz, dlse])

    ms_f = time_graph(fwd, args.steps, args.warmup)
    ms_t = time_eager(train, args.steps, args.warmup)
    rows = int(lengths.sum().item())                       # rows up to each row's last visible key
    nbytes = rows * 2 * R * 2 + B * N
    base = None
    if not args.no_cpu_baseline:
        from oracle import s6_oracle as O
        f32 = lambda t: t.detach().float().cpu().numpy()
        qs, ks, vs, ms_ = f32(q[:1]), f32(k[:1]), f32(v[:1]), mask[:1].cpu().numpy()
        run = lambda: O.single_history(qs, ks, vs, ms_, scale, dtype=np.float32)
        run()
        times = []
        for _ in range(3):
            t0 = time.perf_counter()
            run()
            times.append(time.perf_counter() - t0)
        base = {'value': round(float(np.median(times)) * 1e6 * rows / int(lengths[0].item()), 1),
                'unit': 'us per forward', 'cores': len(os.sched_getaffinity(0)), 'kind': 'port',
                'sample': f'numpy oracle forward (float32) of row 0 ({int(lengths[0].item())} keys), median of 3, '
                          f'scaled by rows read ({rows}); extrapolated'}
    gbps = nbytes / (ms_f * 1e6)
    print(json.dumps({'workload': 'rows', 'value': round(ms_f * 1000, 2), 'unit': 'us per forward', 'B': B, 'N': N,
                      'heads': HEADS, 'width': R, 'rows_read': rows, 'bytes': nbytes, 'gbps': round(gbps, 1),
                      'hbm_frac': round(gbps / PEAK_HBM_GBPS, 4), 'train_ms': round(ms_t, 3), 'steps': args.steps,
                      'data': 'synthetic (randn q, k, v, cotangents; padding masks)', 'forward_hip_graph': True,
                      'cpu_baseline': base}), flush=True)


class EngineLatent:
    """Random-init latent module of one layer with the interface the HF rolling engine's attention reads
    (``register.LatentLayer``: ``readers``, ``query``, ``fields``, ``head_dim``): readers A_t / B_t per loop (loop 0
    at the loop-1 width), the latent query RoPE'd with the teacher's frequencies folded over the latent width, and
    the packed rows ``[K 512 | V 512 | K1 256 | V1 256]``."""

    def __init__(self, pkg, device, gen):
        w = lambda *s: (torch.randn(*s, generator=gen, device=device) / math.sqrt(s[-2])).to(torch.bfloat16)
        self.be, self.head_dim = pkg.batched_engine, HEAD_DIM
        self.A = [w(HEADS, HEAD_DIM, RANK1)] + [w(HEADS, HEAD_DIM, RANK) for _ in range(3)]
        self.B = [w(HEADS, RANK1, HEAD_DIM)] + [w(HEADS, RANK, HEAD_DIM) for _ in range(3)]

    def readers(self, loop):
        return self.A[loop], self.B[loop], RANK1 if loop == 0 else RANK

    def query(self, loop, q, cos, sin):
        """``apply_rope(einsum('bhid,hdr->bhir', q, A), c, s)`` in the dtype of q and A (bf16), as
        ``register.LatentLayer.query`` computes it (``hla/latent/register.py:68-71``)."""
        A, _, rank = self.readers(loop)
        idx = torch.arange(rank // 2, device=cos.device) % (cos.shape[-1] // 2)
        c, s = torch.cat((cos[..., idx], cos[..., idx]), -1), torch.cat((sin[..., idx], sin[..., idx]), -1)
        return self.be.apply_rope(torch.matmul(q.contiguous(), A.contiguous()[None]), c, s)

    def fields(self, loop, packed):
        if loop == 0:
            row = packed[..., 2 * RANK:]
            return row[..., :RANK1], row[..., RANK1:]
        return packed[..., :RANK], packed[..., RANK:2 * RANK]


def mixed_workload(args, pkg, device):
    """The HF rolling engine's joint attention (``hla/latent/batched_engine.py:154-182``) of a loop-2 (main-latent)
    chunk: B = 8 rows of a 256-token chunk, row 0 left-padded by 20 tokens, over two history blocks
    of 2048 and 256 packed rows (``--context`` sets the first) with 80 % of their rows visible. The chunk runs on the
    HIP chunk kernels, the blocks on the multi-query history kernels, both with backward. Times the forward and the
    forward + backward (gradients of q, k, v and the packed rows through autograd) eagerly, and reports the
    attention FLOPs (the chunk's causal pairs and the blocks' rows, two GEMMs each forward) per second. One JSON
    line."""
    be = pkg.batched_engine
    B, n, N0 = args.batch or 8, 256, args.context or 2048
    sizes = (N0, 256)
    g = torch.Generator(device=device).manual_seed(args.seed)
    bf = lambda *s: torch.randn(*s, generator=g, device=device).to(torch.bfloat16)
    sl = EngineLatent(pkg, device, g)
    q, k, v = (bf(B, HEADS, n, HEAD_DIM).requires_grad_(True) for _ in range(3))
    blocks = [(bf(B, N, 2 * RANK + 2 * RANK1) * 0.5).requires_grad_(True) for N in sizes]
    masks = [torch.rand(B, N, generator=g, device=device) < 0.8 for N in sizes]
    valid = torch.ones(B, n, dtype=torch.bool, device=device)
    valid[0, :20] = False
    pos = sum(sizes) + torch.arange(n, device=device)[None].expand(B, n)
    inv = 1.0 / (1e6 ** (torch.arange(0, HEAD_DIM, 2, device=device).float() / HEAD_DIM))
    ang = torch.cat((pos[..., None] * inv, pos[..., None] * inv), -1)
    cos, sin = ang.cos(), ang.sin()
    dout = bf(B, HEADS, n, HEAD_DIM)
    loop = 2

    def fwd():
        with torch.no_grad():
            be.mixed_attention(sl, loop, q, k, v, cos, sin, valid, blocks, masks)

    def train():
        out = be.mixed_attention(sl, loop, q, k, v, cos, sin, valid, blocks, masks)
        torch.autograd.grad(out, [q, k, v] + blocks, dout)

    ms_f = time_eager(fwd, args.steps, args.warmup)
    ms_t = time_eager(train, args.steps, args.warmup)
    pairs_chunk = B * HEADS * n * (n + 1) // 2
    rows_hist = sum(int(m.sum().item()) for m in masks) * HEADS * n
    flops = 4 * HEAD_DIM * pairs_chunk + 4 * RANK * rows_hist
    base = None
    if not args.no_cpu_baseline:
        from oracle import s6_oracle as O
        f32 = lambda t: t.detach().float().cpu().numpy()
        A, Bm, _ = sl.readers(loop)
        fields = [sl.fields(loop, b[:1]) for b in blocks]
        hk, hv = [f32(ck) for ck, _ in fields], [f32(cv) for _, cv in fields]
        args_o = (f32(q[:1]), f32(k[:1]), f32(v[:1]), f32(cos[:1]), f32(sin[:1]), valid[:1].cpu().numpy(), hk, hv,
                  [m[:1].cpu().numpy() for m in masks], f32(A), f32(Bm), 1 / math.sqrt(HEAD_DIM))
        run = lambda: O.mixed_attention(*args_o, dtype=np.float32)
        run()
        times = []
        for _ in range(3):
            t0 = time.perf_counter()
            run()
            times.append(time.perf_counter() - t0)
        base = {'value': round(float(np.median(times)) * 1e3 * B, 1), 'unit': 'ms per forward',
                'cores': len(os.sched_getaffinity(0)), 'kind': 'port',
                'sample': f'numpy oracle forward (float32) of row 0 of the {B}, median of 3, scaled x{B}; '
                          'extrapolated'}
    tflops = flops / (ms_f * 1e9)
    print(json.dumps({'workload': 'mixed', 'value': round(ms_f * 1000, 1), 'unit': 'us per forward', 'B': B,
                      'chunk': n, 'blocks': list(sizes), 'loop': loop, 'flops': flops,
                      'tflops': round(tflops, 1), 'mfma_frac': round(tflops / PEAK_BF16_TFLOPS, 4),
                      'train_ms': round(ms_t, 3), 'steps': args.steps,
                      'data': 'synthetic (randn q, k, v, packed rows, readers; 80 % visible rows; left padding)',
                      'cpu_baseline': base}), flush=True)


def time_eager(fn, steps, warmup):
    """Events around ``steps`` eager calls after ``warmup`` (for work that allocates, e.g. autograd backward)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def main():
    args = parse()
    world = int(os.environ.get('WORLD_SIZE', '1'))
    if args.gpus != 1 or world != 1:
        print('bench.py measures one GPU: the S6 decode path shards by sequence with no exchange, and this '
              'implementation has no multi-GPU path; run with --gpus 1', file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print('bench.py needs an MI355X GPU', file=sys.stderr)
        sys.exit(2)
    device = torch.device('cuda:0')
    torch.cuda.set_device(device)
    if args.copy_calibration:
        src = torch.ones(1 << 28, dtype=torch.int32, device=device)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({'copy_bytes': src.numel() * 4, 'copies': 3}), flush=True)
        return
    pkg = importlib.import_module('hybrid-latent-attention_amd')
    ops, layer = pkg.s6_ops, pkg.s6_layer
    if args.workload == 'writer':
        return writer_workload(args, layer, device)
    if args.workload == 'export':
        return export_workload(args, pkg, device)
    if args.workload == 'khop':
        return khop_workload(args, pkg, device)
    if args.workload == 'rows':
        return rows_workload(args, pkg, device)
    if args.workload == 'mixed':
        return mixed_workload(args, pkg, device)
    cus = pkg._lib.device_cus(0)
    if args.workload != 'decode' and not args.kernel_only:
        return single_config(args, ops, layer, device, cus)
    others, last = None, None
    if not args.no_secondary and not args.kernel_only:
        # the other configurations go first: for about a minute after the 24-layer step (92 GB of caches written and
        # streamed) HBM-bound work ran 2-4 % slower (long context 378 against 364 us/layer, recovered after 60 s
        # idle); each heavy measurement, this step's included, starts after `--settle` seconds of idle
        print('bench: the other configurations', file=sys.stderr, flush=True)
        others, last = measure_secondaries(ops, layer, args, device, cus, not args.no_cpu_baseline)
    B, context, layers = args.batch or 64, args.context or 8192, args.layers or LAYERS
    wl = build_workload(ops, layer, 'decode', B, context, layers, 1, args.seed, device, cus, args.splits, args.table,
                        max_model_len=args.max_model_len)
    splits = wl.splits
    if args.kernel_only:
        us, us_reduce, nbytes = history_roofline(wl, iters=max(args.steps, 1), width=args.width)
        print(json.dumps({'kernel': f'history_split width {args.width}', 'splits': splits[args.width],
                          'us_per_launch': us, 'gbps': nbytes / us / 1e3, 'reduce_us': us_reduce}), flush=True)
        return

    settle(args.settle, last, 'the decode step')
    print('bench: capturing the decode step', file=sys.stderr, flush=True)
    ms = time_graph(wl.step, args.steps, args.warmup)
    us_layer = ms * 1000 / layers
    hist_bytes, win_bytes = wl.history_bytes_per_layer(), wl.window_bytes_per_layer()
    layer_gbps = (hist_bytes + win_bytes) / (us_layer * 1e3)
    print('bench: history kernel roofline', file=sys.stderr, flush=True)
    op_us, reduce_us, op_bytes = history_roofline(wl)
    achieved = op_bytes / (op_us * 1e3)
    base = None
    if not args.no_cpu_baseline:
        print('bench: cpu baseline', file=sys.stderr, flush=True)
        base = cpu_baseline(wl, (0, 1))
    ref_splits = wl.ref_splits
    result = {
        'metric': METRIC, 'value': round(us_layer, 3), 'unit': 'us/layer', 'n_gpus': 1, 'steps': args.steps,
        'warmup': args.warmup, 'ms_per_step': round(ms, 4), 'higher_is_better': False, 'scaling': 'weak',
        'vs_baseline': None, 'dtype': 'bf16', 'data': 'synthetic (random-init caches, readers and queries)',
        'config': {'workload': f'Ouro-1.4B S6 decode attention path, {layers} layers x {LOOPS} loops, '
                               f'B={B}, context {context}, W={WINDOW}, block {BLOCK}',
                   'global_batch': B, 'seq_len': context, 'parallelism': 'none (1 GPU)',
                   'kv_splits': splits, 'reference_kv_splits': ref_splits,
                   'driven_as': 'the reference adapter drives it: one num_kv_splits count and its workspace; '
                                'StepContext picks the per-width counts', 'hip_graph': True},
        'tokens_per_s': round(B / (ms / 1000), 1),
        'hbm_gbps': round(layer_gbps, 1), 'hbm_frac': round(layer_gbps / PEAK_HBM_GBPS, 4),
        'bytes_per_layer': {'latent_history': hist_bytes, 'exact_window': win_bytes},
        'roofline': {'kernel': f'history_split<{RANK}> (split-KV latent history, {splits[RANK]} splits)',
                     'bound': 'hbm', 'achieved': round(achieved, 1), 'peak': PEAK_HBM_GBPS, 'unit': 'GB/s',
                     'frac': round(achieved / PEAK_HBM_GBPS, 4), 'traffic': measured_traffic(),
                     'us_per_launch': round(op_us, 2), 'algorithmic_bytes_per_launch': op_bytes,
                     'reduce_us_per_launch': round(reduce_us, 2)},
        'cpu_baseline': base,
        'configs': others,
    }
    print(json.dumps(result), flush=True)


if __name__ == '__main__':
    main()
