"""Build ``libklsample.so`` (gfx950) in place with hipcc.

The library is two sources: ``csrc/sampling.hip`` (kernels) and ``csrc/api.cpp`` (the C
ABI declared in ``include/klsample.h``).  The result lands next to this file so it
travels with the source tree.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
ROOT = PACKAGE_DIR.parent.parent
CSRC = PACKAGE_DIR.parent / 'csrc'
INCLUDE = ROOT / 'include'
LIBRARY = PACKAGE_DIR / 'libklsample.so'
ARCH = 'gfx950'

# -ffp-contract=off keeps the penalty and temperature arithmetic free of fused
# multiply-adds (it must round exactly like the reference's separate fp32 operations);
# packed fp32 instructions are disabled for every HIP code object.
HIPCC_FLAGS = [
    f'--offload-arch={ARCH}', '-O3', '-std=c++17', '-fPIC', '-shared',
    '-ffp-contract=off',
    '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops',
    '-Wall', '-Wno-unused-function',
]


def hipcc() -> str:
    path = shutil.which('hipcc') or '/opt/rocm/bin/hipcc'
    if not os.path.exists(path):
        raise RuntimeError('hipcc not found; the ROCm toolchain is required to build klsample')
    return path


def sources() -> list[Path]:
    return [CSRC / 'sampling.hip', CSRC / 'api.cpp']


def build(verbose: bool = False) -> Path:
    """Compile the library; always recompiles.  Returns the library path."""
    tmp = LIBRARY.with_suffix('.so.tmp')
    cmd = [hipcc(), *HIPCC_FLAGS, f'-I{INCLUDE}', f'-I{CSRC}', '-o', str(tmp), *map(str, sources())]
    if verbose:
        print(' '.join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = 'packed-fp32-ops'  # the host pass does not know the device feature flag
    log = '\n'.join(line for line in (proc.stdout + proc.stderr).splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f'hipcc failed ({proc.returncode}):\n{log}')
    if verbose and log.strip():
        print(log, file=sys.stderr)
    os.replace(tmp, LIBRARY)
    return LIBRARY


if __name__ == '__main__':
    print(build(verbose=True))
