"""The C ABI layer (api.cpp) under the address and undefined-behaviour sanitizers (CPU).

api.cpp is compiled with g++ (host code only) together with tests/abi_sanitize/driver.cpp,
which drives every entry point through its argument checks and launch planning, and
tests/abi_sanitize/stubs.cpp, which stands in for the kernel launches of sampling.hip."""
import os
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HERE = ROOT / 'tests' / 'abi_sanitize'
ROCM_INCLUDE = Path(os.environ.get('ROCM_PATH', '/opt/rocm')) / 'include'


@pytest.mark.skipif(shutil.which('g++') is None or not (ROCM_INCLUDE / 'hip').exists(),
                    reason='needs g++ and the HIP headers')
def test_c_abi_under_asan_and_ubsan(tmp_path):
    exe = tmp_path / 'abi_sanitize'
    cmd = ['g++', '-std=c++17', '-O1', '-g', '-fno-omit-frame-pointer',
           '-fsanitize=address,undefined', '-fno-sanitize-recover=all', '-D__HIP_PLATFORM_AMD__',
           f'-I{ROCM_INCLUDE}', f'-I{ROOT / "include"}', f'-I{ROOT / "gpu-kernel-lab_amd" / "csrc"}', f'-I{HERE}',
           str(ROOT / 'gpu-kernel-lab_amd' / 'csrc' / 'api.cpp'), str(HERE / 'stubs.cpp'), str(HERE / 'driver.cpp'),
           '-pthread', '-o', str(exe)]
    build = subprocess.run(cmd, capture_output=True, text=True)
    assert build.returncode == 0, build.stderr[-4000:]
    # (verify_asan_link_order=0: a library the environment preloads may precede the
    # sanitizer runtime)
    env = dict(os.environ, ASAN_OPTIONS='detect_leaks=1:verify_asan_link_order=0', UBSAN_OPTIONS='print_stacktrace=1')
    run = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=120)
    assert run.returncode == 0 and run.stdout.strip() == 'ok', run.stdout[-2000:] + run.stderr[-4000:]
