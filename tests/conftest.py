"""Test configuration: import paths, the ``gpu`` marker and the built library."""
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT / 'gpu-kernel-lab_amd', ROOT, ROOT / 'tests'):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line('markers', 'gpu: needs an MI355X (gfx950) GPU')


@pytest.fixture(scope='session')
def lib():
    """The C ABI library; built here if it has not been built yet."""
    from klsample import _lib, build
    if not _lib.LIBRARY.exists():
        build.build()
    return _lib.load()
