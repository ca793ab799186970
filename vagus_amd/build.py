"""Build libvagus_gdr.so in-tree with hipcc for gfx950.

    python -m vagus_amd.build            # compile every csrc/*.hip and link

Each translation unit is compiled to an object in parallel, then linked into
vagus_amd/libvagus_gdr.so.  The library is plain C ABI (include/vagus_gdr.h);
nothing links against torch.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, 'csrc')
LIB = os.path.join(PKG, 'libvagus_gdr.so')
ARCH = os.environ.get('VGDR_OFFLOAD_ARCH', 'gfx950')

HIPCC_FLAGS = [
    '-O3', '-std=c++17', '-fPIC', f'--offload-arch={ARCH}',
    # packed fp32 VALU ops are kept out of the generated code
    '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops',
    '-Wall', '-Wno-unused-function', '-Wno-unused-variable', '-Wno-pass-failed',
    f'-I{os.path.join(ROOT, "include")}',
]


def hipcc() -> str:
    for cand in (os.environ.get('HIPCC'), shutil.which('hipcc'), '/opt/rocm/bin/hipcc'):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError('hipcc not found (ROCm is required to build libvagus_gdr.so)')


def sources() -> list[str]:
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith('.hip'))


def _compile(src: str, obj: str) -> None:
    cmd = [hipcc(), *HIPCC_FLAGS, '-c', src, '-o', obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f'hipcc failed on {os.path.basename(src)}')
    # the host pass does not know the gfx950 feature flag above: drop that noise
    noise = "'-packed-fp32-ops' is not a recognized feature"
    for line in (r.stdout + r.stderr).splitlines():
        if line.strip() and noise not in line:
            sys.stderr.write(line + '\n')


def build(verbose: bool = True) -> str:
    """Compile all kernels and link the shared library; returns its path."""
    objdir = os.path.join(PKG, '_build')
    os.makedirs(objdir, exist_ok=True)
    srcs = sources()
    objs = [os.path.join(objdir, os.path.basename(s)[:-4] + '.o') for s in srcs]
    workers = min(len(srcs), max(1, (os.cpu_count() or 4) // 2))
    with cf.ThreadPoolExecutor(workers) as ex:
        list(ex.map(_compile, srcs, objs))
    tmp = LIB + '.tmp'
    cmd = [hipcc(), f'--offload-arch={ARCH}', '-shared', '-fPIC', *objs, '-o', tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError('hipcc link of libvagus_gdr.so failed')
    os.replace(tmp, LIB)
    if verbose:
        print(f'[vagus_amd] built {LIB}')
    return LIB


if __name__ == '__main__':
    build()
