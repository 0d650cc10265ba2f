"""The benchmark driver's host logic (no GPU): the idle pause between heavy configurations and the refusal of a
multi-GPU run."""
import importlib.util
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope='module')
def bench():
    spec = importlib.util.spec_from_file_location('bench_under_test', os.path.join(ROOT, 'bench.py'))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_settle_waits_out_the_rest_of_the_pause(bench, monkeypatch):
    clock, slept = [100.0], []
    monkeypatch.setattr(bench.time, 'monotonic', lambda: clock[0])
    monkeypatch.setattr(bench.time, 'sleep', lambda s: slept.append(s))
    bench.settle(60.0, None, 'first')          # nothing measured yet: no pause
    bench.settle(0.0, 90.0, 'disabled')        # --settle 0: no pause
    bench.settle(60.0, 30.0, 'long ago')       # 70 s since the last heavy step: no pause
    assert slept == []
    bench.settle(60.0, 85.0, 'recent')         # 15 s since: the remaining 45 s
    assert slept == [pytest.approx(45.0)]


def test_more_than_one_gpu_is_refused():
    proc = subprocess.run([sys.executable, os.path.join(ROOT, 'bench.py'), '--gpus', '2'], capture_output=True,
                          text=True, timeout=300, cwd=ROOT)
    assert proc.returncode == 2
    assert 'one GPU' in proc.stderr
