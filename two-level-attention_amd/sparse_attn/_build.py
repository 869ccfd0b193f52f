"""Build libnfa_hip.so for gfx950 with hipcc (in-tree, next to the package).

``python -m sparse_attn._build`` (with ``two-level-attention_amd`` on the path)
or ``__graft_entry__.build()`` runs it.  Each source compiles to its own
object in parallel, then one link step produces ``lib/libnfa_hip.so``.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(PKG_ROOT, 'csrc')
LIB_DIR = os.path.join(PKG_ROOT, 'lib')
OBJ_DIR = os.path.join(PKG_ROOT, 'lib', 'obj')
SOURCES = ('nfa_select.hip', 'nfa_attn.hip', 'nfa_mla_attn.hip', 'nfa_write.hip',
           'nfa_decode_fused.hip', 'nfa_gate.hip')
ARCH = 'gfx950'

# Bit-exactness of the selector depends on these: no FMA contraction, IEEE
# fp32 division, fp32 denormals kept.  Packed fp32 instructions are disabled.
HIP_FLAGS = [
    f'--offload-arch={ARCH}', '-O3', '-std=c++17', '-fPIC',
    '-ffp-contract=off', '-fno-fast-math', '-fno-gpu-flush-denormals-to-zero',
    '-fhip-fp32-correctly-rounded-divide-sqrt',
    '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops',
]


def hipcc() -> str:
    path = shutil.which('hipcc') or '/opt/rocm/bin/hipcc'
    if not os.path.exists(path):
        raise RuntimeError('hipcc not found; ROCm is required to build')
    return path


def _compile(src: str) -> str:
    obj = os.path.join(OBJ_DIR, os.path.splitext(src)[0] + '.o')
    cmd = [hipcc(), *HIP_FLAGS, '-c', os.path.join(CSRC, src), '-o', obj]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f'hipcc failed for {src}:\n{proc.stderr}')
    return obj


def build(verbose: bool = True) -> str:
    os.makedirs(OBJ_DIR, exist_ok=True)
    with ThreadPoolExecutor(max_workers=len(SOURCES)) as pool:
        objs = list(pool.map(_compile, SOURCES))
    out = os.path.join(LIB_DIR, 'libnfa_hip.so')
    tmp = out + '.tmp'
    cmd = [hipcc(), f'--offload-arch={ARCH}', '-shared', '-fPIC', *objs,
           '-o', tmp]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f'link failed:\n{proc.stderr}')
    os.replace(tmp, out)
    if verbose:
        print(f'built {out}', file=sys.stderr)
    return out


if __name__ == '__main__':
    build()
