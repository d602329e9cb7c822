"""Builds libefgs_hip.so (hipcc, gfx950) in-tree and pre-populates the hipRTC code-object cache.

Usage: python build_lib.py [--arch gfx950] [--jobs 8]
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, 'csrc')
BUILD = os.path.join(HERE, '_build')
LIB = os.path.join(HERE, 'efgs', 'libefgs_hip.so')

# (source, extra flags). The decision-path files disable FP contraction so instance emission, blend replay and
# Adam follow the exact operation sequence of their definitions.
SOURCES = [
    ('api.cpp', []),
    ('rtc.cpp', []),
    ('scan.hip', []),
    ('raster.hip', ['-ffp-contract=off']),
    ('blend.hip', ['-ffp-contract=off']),
    ('adam.hip', ['-ffp-contract=off']),
    ('densification.hip', ['-ffp-contract=off']),
    ('ngsplat.hip', ['-ffp-contract=off']),
]

COMMON = ['-O3', '-std=c++17', '-fPIC', '-fhip-fp32-correctly-rounded-divide-sqrt',
          '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops', '-Wall', '-Wno-unused-function']


def _compile(src: str, extra: list[str], arch: str) -> str:
    obj = os.path.join(BUILD, src + '.o')
    cmd = ['hipcc', '-x', 'hip', f'--offload-arch={arch}', *COMMON, *extra, '-I', CSRC, '-c', os.path.join(CSRC, src), '-o', obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f'compiling {src} failed:\n{" ".join(cmd)}\n{r.stdout}\n{r.stderr}')
    return obj


def build(arch: str = 'gfx950', jobs: int = 8, verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s[0], s[1], arch), SOURCES))
    tmp = LIB + '.tmp'
    cmd = ['hipcc', f'--offload-arch={arch}', '-shared', '-fPIC', '-o', tmp, *objs, '-lhiprtc']
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f'linking failed:\n{" ".join(cmd)}\n{r.stdout}\n{r.stderr}')
    os.replace(tmp, LIB)
    if verbose:
        print(f'built {LIB}')
    return LIB


if __name__ == '__main__':
    ap = argparse.ArgumentParser()
    ap.add_argument('--arch', default='gfx950')
    ap.add_argument('--jobs', type=int, default=8)
    args = ap.parse_args()
    build(args.arch, args.jobs, verbose=True)
    sys.exit(0)
