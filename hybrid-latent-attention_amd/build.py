"""Build ``libhla_s6.so`` (the C-ABI HIP library) in-tree for gfx950 with hipcc.

Usage: ``python build.py`` from anywhere; ``build()`` from Python. Every call recompiles every source.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, 'csrc')
INCLUDE = os.path.join(ROOT, 'include')
LIB_NAME = 'libhla_s6.so'
ARCH = os.environ.get('HLA_OFFLOAD_ARCH', 'gfx950')

SOURCES = ('api.hip', 'history.hip', 'window.hip', 'elementwise.hip', 'absorb.hip', 'writer.hip', 'rollout.hip', 'khop.hip',
           'khop_f32.hip', 'hf_chunk.hip', 'mixed.hip')

FLAGS = [
    f'--offload-arch={ARCH}', '-O3', '-std=c++17', '-fPIC', '-Wall', '-Wno-unused-function',
    # packed fp32 (v_pk_*_f32) is kept out of every kernel on this platform
    '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops',
    f'-I{INCLUDE}', f'-I{CSRC}',
]


def hipcc() -> str:
    path = shutil.which('hipcc') or '/opt/rocm/bin/hipcc'
    if not os.path.exists(path):
        raise RuntimeError('hipcc not found: the ROCm toolchain is required to build libhla_s6.so')
    return path


def _compile(src: str, obj: str, defines=()) -> str:
    cmd = [hipcc(), *FLAGS, *(f'-D{d}' for d in defines), '-c', os.path.join(CSRC, src), '-o', obj]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f'hipcc failed on {src}:\n{proc.stdout}\n{proc.stderr}')
    return obj


def build(verbose: bool = False, out: str | None = None, defines=()) -> str:
    """Compile every HIP source for gfx950 and link ``libhla_s6.so`` (next to this file unless ``out`` names another
    path; ``defines`` are extra ``NAME=VALUE`` preprocessor definitions); returns its path."""
    out = out or os.path.join(HERE, LIB_NAME)
    with tempfile.TemporaryDirectory(prefix='hla_build_') as tmp:
        objs = [os.path.join(tmp, s.replace('.hip', '.o')) for s in SOURCES]
        with cf.ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 1)) as pool:
            list(pool.map(lambda so: _compile(*so, defines), zip(SOURCES, objs)))
        tmp_out = os.path.join(tmp, LIB_NAME)
        cmd = [hipcc(), f'--offload-arch={ARCH}', '-shared', '-fPIC', *objs, '-o', tmp_out,
               '-Wl,-rpath,/opt/rocm/lib']
        proc = subprocess.run(cmd, capture_output=True, text=True)
        if proc.returncode != 0:
            raise RuntimeError(f'hipcc link failed:\n{proc.stdout}\n{proc.stderr}')
        shutil.move(tmp_out, out)
    if verbose:
        print(f'built {out}', flush=True)
    return out


if __name__ == '__main__':
    build(verbose=True)
    sys.exit(0)
