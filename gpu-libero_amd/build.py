"""Build libmx_physics.so for gfx950 with hipcc (in-tree, next to this file).

Flags: -O3, FMA contraction as HIP's default (the reference builds with --fmad=true), IEEE
division and square root (HIP's default correctly rounded fp32 div/sqrt), no fast-math, no
flush-to-zero; packed FP32 instructions disabled (``-packed-fp32-ops``).
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent
LIBRARY = HERE / 'libmx_physics.so'
SOURCES = [HERE / 'csrc' / 'mx_step.hip', HERE / 'csrc' / 'mx_step_slab.hip', HERE / 'csrc' / 'mx_step_slab4.hip',
           HERE / 'csrc' / 'mx_step_f64.hip']
HEADERS = [HERE / 'csrc' / h for h in ('mx_math.h', 'mx_image.h', 'mx_collide.h', 'mx_convex.h')] + [ROOT / 'include' / 'mx_physics.h']

HIPCC_FLAGS = ['--offload-arch=gfx950', '-O3', '-std=c++17', '-fPIC', '-shared',
               '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops',
               '-fno-gpu-rdc', '-Wall', '-Wno-unused-function', '-Wno-unused-variable']


def hipcc():
    path = os.environ.get('HIPCC') or shutil.which('hipcc') or '/opt/rocm/bin/hipcc'
    if not Path(path).exists():
        raise RuntimeError('hipcc not found; set HIPCC')
    return path


def build(verbose=False):
    """Compile every HIP source into the in-tree shared library (always recompiles): the
    translation units compile in parallel into objects under a temporary directory, then link."""
    import tempfile
    tmp = LIBRARY.with_suffix('.so.tmp')
    with tempfile.TemporaryDirectory(prefix='mx_build_') as work:
        objects, jobs = [], []
        for src in SOURCES:
            obj = Path(work) / (src.stem + '.o')
            objects.append(str(obj))
            cmd = [hipcc()] + [f for f in HIPCC_FLAGS if f != '-shared'] + ['-c', '-o', str(obj), str(src)]
            jobs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)))
        failed = False
        for src, job in jobs:
            out, err = job.communicate()
            if job.returncode != 0:
                sys.stderr.write(out + err)
                failed = True
            elif verbose:
                sys.stderr.write(err)
        if failed:
            raise RuntimeError('hipcc failed for libmx_physics.so')
        result = subprocess.run([hipcc()] + HIPCC_FLAGS + ['-o', str(tmp)] + objects, capture_output=True, text=True)
        if result.returncode != 0:
            sys.stderr.write(result.stdout + result.stderr)
            raise RuntimeError('hipcc link failed for libmx_physics.so')
    os.replace(tmp, LIBRARY)
    return LIBRARY


if __name__ == '__main__':
    print(build(verbose='-v' in sys.argv))
