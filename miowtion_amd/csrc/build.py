"""Builds libveda_hip.so (all HIP sources of this directory) for gfx950.

Usage: python -m miowtion_amd.csrc.build   (or build() from Python)

Each .hip file is compiled to an object in parallel, then linked into
miowtion_amd/libveda_hip.so. No torch headers are involved: the library is a
plain C ABI (include/veda_hip.h) that the Python side loads with ctypes.
"""

from __future__ import annotations

import concurrent.futures
import os
import pathlib
import subprocess
import sys

HERE = pathlib.Path(__file__).resolve().parent
PKG = HERE.parent
ROOT = PKG.parent
LIB = PKG / 'libveda_hip.so'
BUILD_DIR = PKG / '_build'
HIPCC = os.environ.get('HIPCC', '/opt/rocm/bin/hipcc')
ARCH = 'gfx950'
# -packed-fp32-ops: hipcc must not emit packed fp32 arithmetic for this pool
# (the host pass warns that it does not know the feature; harmless).
FLAGS = ['-O3', '-std=c++17', '-fPIC', f'--offload-arch={ARCH}',
         '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops',
         f'-I{ROOT / "include"}']


# Per-source extra flags. attention.hip, heat.hip: MFMA results in VGPRs
# (the softmax / heat reads every score; the default AGPR form costs a copy
# per score).
EXTRA = {'attention.hip': ['-mllvm', '-amdgpu-mfma-vgpr-form'],
         'heat.hip': ['-mllvm', '-amdgpu-mfma-vgpr-form']}


def sources() -> list[pathlib.Path]:
    return sorted(HERE.glob('*.hip'))


def _compile(src: pathlib.Path) -> pathlib.Path:
    obj = BUILD_DIR / (src.stem + '.o')
    cmd = [HIPCC, *FLAGS, *EXTRA.get(src.name, []), '-c', str(src), '-o', str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f'hipcc failed on {src.name}:\n{proc.stderr}')
    return obj


def build(verbose: bool = True) -> pathlib.Path:
    """Compiles every source and links the shared library; returns its path."""
    BUILD_DIR.mkdir(exist_ok=True)
    srcs = sources()
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as pool:
        objs = list(pool.map(_compile, srcs))
    tmp = LIB.with_suffix('.so.tmp')
    cmd = [HIPCC, '-shared', f'--offload-arch={ARCH}', '-o', str(tmp), *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f'link failed:\n{proc.stderr}')
    os.replace(tmp, LIB)
    if verbose:
        print(f'built {LIB} from {len(srcs)} sources', file=sys.stderr)
    return LIB


if __name__ == '__main__':
    build()
