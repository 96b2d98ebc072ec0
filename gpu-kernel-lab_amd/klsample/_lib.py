"""ctypes binding of ``libklsample.so`` (the C ABI in ``include/klsample.h``).

The library is loaded from this package directory only; there is no fallback.  A
missing or stale library raises ``RuntimeError`` instead of sampling some other way.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import numpy as np

LIBRARY = Path(__file__).resolve().parent / 'libklsample.so'
ABI_VERSION = 3

OK = 0
ERR_INVALID_ARGUMENT = -1
ERR_UNSUPPORTED_DTYPE = -2
ERR_WORKSPACE = -3
ERR_HIP = -4

FLOAT32 = 0
BFLOAT16 = 1

ROW_GREEDY = 1
ROW_REPETITION = 2
ROW_PRESENCE_FREQUENCY = 4
ROW_TOP_P = 8

OPT_FORCE_DENSE = 1
OPT_HISTORY_PAIRS = 2
OPT_HOST_PARAMS = 4
HOST_PARAMS_MAX_BATCH = 8

MAX_LOGPROBS = 256
MAX_BATCH = 65536
MAX_VOCAB = 1 << 24

EXPORTS = ('klsample_abi_version', 'klsample_workspace_size', 'klsample_workspace_init',
           'klsample_run', 'klsample_run_noalloc', 'klsample_set_phase_events', 'klsample_last_error',
           'klsample_lmhead_workspace_size', 'klsample_lmhead_run')
NOALLOC_SCRATCH_BYTES = 64 << 20

# klsample_row_params, 32 bytes
ROW_PARAMS_DTYPE = np.dtype([
    ('temperature', '<f4'), ('top_k', '<i4'), ('top_p', '<f4'), ('repetition_penalty', '<f4'),
    ('presence_penalty', '<f4'), ('frequency_penalty', '<f4'), ('uniform', '<f4'), ('flags', '<u4'),
])
# klsample_row_info, 32 bytes
ROW_INFO_DTYPE = np.dtype([
    ('max_score', '<f4'), ('cut_score', '<f4'), ('cut_index', '<i4'), ('kept', '<i4'),
    ('log_norm', '<f8'), ('path', '<i4'), ('mode', '<i4'),
])


class Batch(ctypes.Structure):
    """``klsample_batch``."""

    _fields_ = [
        ('logits', ctypes.c_void_p),
        ('row_stride', ctypes.c_int64),
        ('dtype', ctypes.c_int32),
        ('batch', ctypes.c_int32),
        ('vocab', ctypes.c_int32),
        ('num_logprobs', ctypes.c_int32),
        ('max_top_k', ctypes.c_int32),
        ('options', ctypes.c_uint32),
        ('params', ctypes.c_void_p),
        ('history_ids', ctypes.c_void_p),
        ('history_offsets', ctypes.c_void_p),
        ('token_ids', ctypes.c_void_p),
        ('logprobs', ctypes.c_void_p),
        ('top_ids', ctypes.c_void_p),
        ('top_logprobs', ctypes.c_void_p),
        ('probs', ctypes.c_void_p),
        ('row_info', ctypes.c_void_p),
        ('workspace', ctypes.c_void_p),
        ('workspace_bytes', ctypes.c_size_t),
        ('history_errors', ctypes.c_void_p),
        ('history_append', ctypes.c_void_p),
    ]


class LMHead(ctypes.Structure):
    """``klsample_lmhead``."""

    _fields_ = [('hidden', ctypes.c_void_p), ('weight', ctypes.c_void_p), ('dim', ctypes.c_int32),
                ('reserved', ctypes.c_int32)]


class KLSampleError(RuntimeError):
    """A non-zero status from the library."""

    def __init__(self, status: int, message: str):
        super().__init__(f'klsample status {status}: {message}')
        self.status = status


_lock = threading.Lock()
_lib = None


def load(path: Path | str | None = None) -> ctypes.CDLL:
    """Load the library (once) and declare its signatures."""
    global _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        target = Path(path) if path is not None else LIBRARY
        if not target.exists():
            raise RuntimeError(f'{target} is not built; run klsample.build.build() '
                               '(or __graft_entry__.build()) first')
        lib = ctypes.CDLL(str(target))
        lib.klsample_abi_version.restype = ctypes.c_int
        lib.klsample_abi_version.argtypes = []
        lib.klsample_last_error.restype = ctypes.c_char_p
        lib.klsample_last_error.argtypes = []
        lib.klsample_workspace_size.restype = ctypes.c_int
        lib.klsample_workspace_size.argtypes = [ctypes.c_int32] * 5 + [ctypes.POINTER(ctypes.c_size_t)]
        lib.klsample_workspace_init.restype = ctypes.c_int
        lib.klsample_workspace_init.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
        lib.klsample_run.restype = ctypes.c_int
        lib.klsample_run.argtypes = [ctypes.POINTER(Batch), ctypes.c_void_p]
        lib.klsample_run_noalloc.restype = ctypes.c_int
        lib.klsample_run_noalloc.argtypes = [ctypes.POINTER(Batch), ctypes.c_void_p]
        lib.klsample_lmhead_workspace_size.restype = ctypes.c_int
        lib.klsample_lmhead_workspace_size.argtypes = [ctypes.c_int32] * 4 + [ctypes.POINTER(ctypes.c_size_t)]
        lib.klsample_lmhead_run.restype = ctypes.c_int
        lib.klsample_lmhead_run.argtypes = [ctypes.POINTER(Batch), ctypes.POINTER(LMHead), ctypes.c_void_p]
        lib.klsample_set_phase_events.restype = ctypes.c_int
        lib.klsample_set_phase_events.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_int32]
        version = lib.klsample_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f'{target} has ABI version {version}, expected {ABI_VERSION}; rebuild it')
        if path is None:
            _lib = lib
        return lib


_hip = None


def hip() -> ctypes.CDLL:
    """The HIP runtime the process (torch) already has loaded, for the few calls made
    here directly."""
    global _hip
    if _hip is None:
        h = ctypes.CDLL('libamdhip64.so')
        h.hipHostGetDevicePointer.restype = ctypes.c_int
        h.hipHostGetDevicePointer.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_void_p, ctypes.c_uint]
        h.hipStreamSynchronize.restype = ctypes.c_int
        h.hipStreamSynchronize.argtypes = [ctypes.c_void_p]
        h.hipGetErrorString.restype = ctypes.c_char_p
        h.hipGetErrorString.argtypes = [ctypes.c_int]
        _hip = h
    return _hip


def mapped_pointer(host_ptr: int) -> int | None:
    """The device's address of pinned host memory (``hipHostGetDevicePointer``), or
    None if the runtime does not map it for the device."""
    dev = ctypes.c_void_p()
    if hip().hipHostGetDevicePointer(ctypes.byref(dev), ctypes.c_void_p(host_ptr), 0) != 0 or not dev.value:
        return None
    return dev.value


def stream_synchronize(stream: int) -> None:
    """Wait for the work enqueued on a raw hipStream_t (0: the null stream)."""
    e = hip().hipStreamSynchronize(stream)
    if e != 0:
        raise KLSampleError(ERR_HIP, 'hipStreamSynchronize: ' + hip().hipGetErrorString(e).decode())


def last_error(lib: ctypes.CDLL) -> str:
    return lib.klsample_last_error().decode('utf-8', 'replace')


def check(lib: ctypes.CDLL, status: int) -> None:
    if status != OK:
        message = last_error(lib)
        if status in (ERR_INVALID_ARGUMENT, ERR_UNSUPPORTED_DTYPE):
            raise ValueError(f'klsample status {status}: {message}')
        raise KLSampleError(status, message)


def lmhead_workspace_size(batch: int, vocab: int, max_top_k: int, num_logprobs: int) -> int:
    lib = load()
    out = ctypes.c_size_t(0)
    check(lib, lib.klsample_lmhead_workspace_size(batch, vocab, max_top_k, num_logprobs, ctypes.byref(out)))
    return int(out.value)


def workspace_size(batch: int, vocab: int, dtype: int, max_top_k: int, num_logprobs: int) -> int:
    lib = load()
    out = ctypes.c_size_t(0)
    check(lib, lib.klsample_workspace_size(batch, vocab, dtype, max_top_k, num_logprobs, ctypes.byref(out)))
    return int(out.value)
