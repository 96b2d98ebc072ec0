"""The C ABI without a GPU: exports, struct layout, validation (CPU only).

Every check here runs before the library's first HIP call, so no device is touched."""
import ctypes
import re
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

from klsample import _lib

HEADER = Path(__file__).resolve().parents[1] / 'include' / 'klsample.h'


def declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r'^\s*(?:const\s+)?\w+\s*\*?\s*(klsample_\w+)\s*\(', text, re.M)))


def test_header_declares_the_expected_entry_points():
    assert declared_functions() == sorted(_lib.EXPORTS)


def test_library_exports_every_declared_symbol(lib):
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert lib.klsample_abi_version() == _lib.ABI_VERSION
    assert _lib.last_error(lib) == '' or isinstance(_lib.last_error(lib), str)


@pytest.mark.skipif(shutil.which('gcc') is None, reason='gcc not available')
def test_struct_layout_matches_header(tmp_path):
    """Compile a probe against the header and compare sizes/offsets with the ctypes mirror."""
    fields = [f for f, _ in _lib.Batch._fields_]
    src = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', 'int main(void){',
           'printf("%zu %zu %zu\\n", sizeof(klsample_row_params), sizeof(klsample_row_info), sizeof(klsample_batch));']
    src += [f'printf("%zu\\n", offsetof(klsample_batch, {f}));' for f in fields]
    src += [f'printf("%zu\\n", offsetof(klsample_row_params, {f}));' for f in _lib.ROW_PARAMS_DTYPE.names]
    src += [f'printf("%zu\\n", offsetof(klsample_row_info, {f}));' for f in _lib.ROW_INFO_DTYPE.names]
    src += ['return 0;}']
    (tmp_path / 'probe.c').write_text('\n'.join(src))
    subprocess.run(['gcc', '-o', str(tmp_path / 'probe'), str(tmp_path / 'probe.c')], check=True)
    out = subprocess.run([str(tmp_path / 'probe')], capture_output=True, text=True, check=True).stdout.split()
    sizes = list(map(int, out[:3]))
    assert sizes == [_lib.ROW_PARAMS_DTYPE.itemsize, _lib.ROW_INFO_DTYPE.itemsize, ctypes.sizeof(_lib.Batch)]
    offs = list(map(int, out[3:]))
    n = len(fields)
    assert offs[:n] == [getattr(_lib.Batch, f).offset for f in fields]
    assert offs[n:n + len(_lib.ROW_PARAMS_DTYPE.names)] == [
        _lib.ROW_PARAMS_DTYPE.fields[f][1] for f in _lib.ROW_PARAMS_DTYPE.names]
    assert offs[n + len(_lib.ROW_PARAMS_DTYPE.names):] == [
        _lib.ROW_INFO_DTYPE.fields[f][1] for f in _lib.ROW_INFO_DTYPE.names]


def _size(lib, b, v, dt=0, k=0, n=0):
    out = ctypes.c_size_t(0)
    st = lib.klsample_workspace_size(b, v, dt, k, n, ctypes.byref(out))
    return st, out.value


def test_workspace_size_validation(lib):
    assert _size(lib, 1, 151936)[0] == _lib.OK
    assert _size(lib, 0, 10)[0] == _lib.ERR_INVALID_ARGUMENT
    assert 'batch' in _lib.last_error(lib)
    assert _size(lib, _lib.MAX_BATCH + 1, 10)[0] == _lib.ERR_INVALID_ARGUMENT
    assert _size(lib, 1, 0)[0] == _lib.ERR_INVALID_ARGUMENT
    assert _size(lib, 1, _lib.MAX_VOCAB + 1)[0] == _lib.ERR_INVALID_ARGUMENT
    assert _size(lib, 1, 10, dt=7)[0] == _lib.ERR_UNSUPPORTED_DTYPE
    assert _size(lib, 1, 10, k=-1)[0] == _lib.ERR_INVALID_ARGUMENT
    assert _size(lib, 1, 10, n=_lib.MAX_LOGPROBS + 1)[0] == _lib.ERR_INVALID_ARGUMENT
    assert lib.klsample_workspace_size(1, 10, 0, 0, 0, None) == _lib.ERR_INVALID_ARGUMENT


def test_phase_event_hook_validation(lib):
    """The hook only stores handles; nothing reaches HIP until a run records them."""
    assert lib.klsample_set_phase_events(None, 0) == _lib.OK
    assert lib.klsample_set_phase_events(None, 1) == _lib.ERR_INVALID_ARGUMENT
    assert 'events' in _lib.last_error(lib)
    handles = (ctypes.c_void_p * 5)()
    assert lib.klsample_set_phase_events(handles, 5) == _lib.ERR_INVALID_ARGUMENT
    assert lib.klsample_set_phase_events(handles, -1) == _lib.ERR_INVALID_ARGUMENT
    assert lib.klsample_set_phase_events(handles, 4) == _lib.OK   # all NULL: nothing recorded
    assert lib.klsample_set_phase_events(None, 0) == _lib.OK


def test_workspace_grows_with_work(lib):
    base = _size(lib, 8, 151936)[1]
    assert _size(lib, 256, 151936)[1] > base
    assert _size(lib, 8, 151936, k=1000)[1] >= base
    assert _size(lib, 8, 200000)[1] > base
    assert base % 256 == 0


def _valid_batch(ws_bytes=1 << 30):
    """A batch whose pointers are fake but non-NULL; only used for calls that must fail
    validation before any device access."""
    b = _lib.Batch()
    b.logits = 0x10000
    b.row_stride = 100
    b.dtype = _lib.FLOAT32
    b.batch = 2
    b.vocab = 100
    b.num_logprobs = 0
    b.max_top_k = 0
    b.options = 0
    b.params = 0x20000
    b.history_ids = None
    b.history_offsets = None
    b.token_ids = 0x30000
    b.logprobs = 0x40000
    b.top_ids = None
    b.top_logprobs = None
    b.probs = None
    b.row_info = None
    b.workspace = 0x100000
    b.workspace_bytes = ws_bytes
    return b


@pytest.mark.parametrize('mutate,status,needle', [
    (lambda b: setattr(b, 'batch', 0), _lib.ERR_INVALID_ARGUMENT, 'batch'),
    (lambda b: setattr(b, 'vocab', 0), _lib.ERR_INVALID_ARGUMENT, 'vocab'),
    (lambda b: setattr(b, 'dtype', 5), _lib.ERR_UNSUPPORTED_DTYPE, 'dtype'),
    (lambda b: setattr(b, 'logits', None), _lib.ERR_INVALID_ARGUMENT, 'logits'),
    (lambda b: setattr(b, 'row_stride', 99), _lib.ERR_INVALID_ARGUMENT, 'row_stride'),
    (lambda b: setattr(b, 'params', None), _lib.ERR_INVALID_ARGUMENT, 'params'),
    (lambda b: setattr(b, 'token_ids', None), _lib.ERR_INVALID_ARGUMENT, 'token_ids'),
    (lambda b: setattr(b, 'num_logprobs', 3), _lib.ERR_INVALID_ARGUMENT, 'top_ids'),
    (lambda b: setattr(b, 'num_logprobs', 300), _lib.ERR_INVALID_ARGUMENT, 'num_logprobs'),
    (lambda b: setattr(b, 'max_top_k', -2), _lib.ERR_INVALID_ARGUMENT, 'max_top_k'),
    (lambda b: setattr(b, 'history_offsets', 0x50000), _lib.ERR_INVALID_ARGUMENT, 'history_ids'),
    (lambda b: setattr(b, 'options', 64), _lib.ERR_INVALID_ARGUMENT, 'option'),
    (lambda b: setattr(b, 'workspace', None), _lib.ERR_WORKSPACE, 'workspace'),
    (lambda b: setattr(b, 'workspace', 0x100010), _lib.ERR_WORKSPACE, 'aligned'),
    (lambda b: setattr(b, 'workspace_bytes', 1024), _lib.ERR_WORKSPACE, 'too small'),
])
def test_run_rejects_invalid_arguments_before_touching_the_device(lib, mutate, status, needle):
    b = _valid_batch()
    mutate(b)
    assert lib.klsample_run(ctypes.byref(b), None) == status
    assert needle in _lib.last_error(lib)


def test_run_rejects_null_batch(lib):
    assert lib.klsample_run(None, None) == _lib.ERR_INVALID_ARGUMENT


def test_workspace_init_rejects_null(lib):
    assert lib.klsample_workspace_init(None, 16, None) == _lib.ERR_INVALID_ARGUMENT
    assert lib.klsample_workspace_init(ctypes.c_void_p(0x1000), 0, None) == _lib.OK


def test_errors_map_to_python_exceptions(lib):
    with pytest.raises(ValueError):
        _lib.check(lib, lib.klsample_workspace_size(0, 1, 0, 0, 0, ctypes.byref(ctypes.c_size_t())))
    with pytest.raises(_lib.KLSampleError):
        b = _valid_batch()
        b.workspace_bytes = 16
        _lib.check(lib, lib.klsample_run(ctypes.byref(b), None))


def test_row_params_dtype_is_32_bytes():
    assert _lib.ROW_PARAMS_DTYPE.itemsize == 32 and _lib.ROW_INFO_DTYPE.itemsize == 32
    assert np.zeros(1, _lib.ROW_PARAMS_DTYPE).nbytes == 32


@pytest.mark.parametrize('mutate,status,needle', [
    (lambda b: setattr(b, 'batch', 0), _lib.ERR_INVALID_ARGUMENT, 'batch'),
    (lambda b: setattr(b, 'logits', None), _lib.ERR_INVALID_ARGUMENT, 'logits'),
    (lambda b: setattr(b, 'num_logprobs', 3), _lib.ERR_INVALID_ARGUMENT, 'top_ids'),
    (lambda b: setattr(b, 'workspace', 0x100000), _lib.ERR_WORKSPACE, 'takes no workspace'),
    (lambda b: setattr(b, 'workspace_bytes', 4096), _lib.ERR_WORKSPACE, 'takes no workspace'),
    (lambda b: (setattr(b, 'batch', 4096), setattr(b, 'vocab', 151936), setattr(b, 'row_stride', 151936)),
     _lib.ERR_WORKSPACE, 'static scratch holds'),
])
def test_noalloc_rejects_before_touching_the_device(lib, mutate, status, needle):
    """The no-allocation entry point validates like klsample_run, takes no workspace, and
    refuses a call needing more than its static scratch, all before any HIP call."""
    b = _valid_batch()
    b.workspace = None
    b.workspace_bytes = 0
    mutate(b)
    assert lib.klsample_run_noalloc(ctypes.byref(b), None) == status
    assert needle in _lib.last_error(lib)
    assert lib.klsample_run_noalloc(None, None) == _lib.ERR_INVALID_ARGUMENT


def test_noalloc_capacity_matches_header():
    m = re.search(r'#define KLSAMPLE_NOALLOC_SCRATCH_BYTES \(\(size_t\)(\d+) << (\d+)\)', HEADER.read_text())
    assert m and int(m.group(1)) << int(m.group(2)) == _lib.NOALLOC_SCRATCH_BYTES
