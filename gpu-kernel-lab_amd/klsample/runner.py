"""Device-side execution of batched sampling calls through the C ABI.

A :class:`DeviceRunner` owns, per GPU and per host thread, the library workspace and
the staging buffers of a call.  Batches of up to ``HOST_PARAMS_MAX_BATCH`` rows hand
their row parameters and history offsets to the library in host memory, which carries
them in the kernel arguments; larger batches stage them, with any history ids, in one
pinned buffer brought up in a single copy.  The kernels write the outputs into a pinned
host buffer mapped for the device (or a device buffer brought back in one copy where
the device cannot address it).  Buffers only grow; a call allocates nothing once they
are large enough.
"""
from __future__ import annotations

import ctypes
import threading
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib

_DTYPES = {torch.float32: _lib.FLOAT32, torch.bfloat16: _lib.BFLOAT16}
_INT32_MAX = 2**31 - 1


def _align(n: int, a: int = 256) -> int:
    return (n + a - 1) // a * a


def normalize_history(history, vocab: int) -> np.ndarray:
    """History ids as int32 in ``[0, vocab)``.

    Mirrors ``scores[ids]`` in ``serving/sampling.py:48-49``: a negative id counts from
    the end and an id outside ``[-vocab, vocab)`` raises ``IndexError``.
    """
    ids = np.asarray(history, dtype=np.int64).reshape(-1)
    if ids.size:
        lo, hi = int(ids.min()), int(ids.max())
        if lo < -vocab or hi >= vocab:
            bad = ids[(ids < -vocab) | (ids >= vocab)][0]
            raise IndexError(f'index {int(bad)} is out of bounds for dimension 0 with size {vocab}')
        if lo < 0:
            ids = np.where(ids < 0, ids + vocab, ids)
    return ids.astype(np.int32, copy=False)


def row_flags(p) -> int:
    """``KLSAMPLE_ROW_*`` flags of one request: the reference's tests on the original
    Python values (``serving/sampling.py:47``, ``:50``, ``:56``)."""
    flags = 0
    if p.temperature == 0:
        flags |= _lib.ROW_GREEDY
    if p.repetition_penalty != 1:
        flags |= _lib.ROW_REPETITION
    if getattr(p, 'presence_penalty', 0.0) != 0 or getattr(p, 'frequency_penalty', 0.0) != 0:
        flags |= _lib.ROW_PRESENCE_FREQUENCY
    if p.top_p < 1:
        flags |= _lib.ROW_TOP_P
    return flags


def row_record(p, uniform: float = 0.0) -> np.ndarray:
    """One ``klsample_row_params`` record (an array of one).  The floats are the fp32
    roundings of the Python values, which is what the reference's tensor-by-scalar
    operations use."""
    rec = np.zeros(1, dtype=_lib.ROW_PARAMS_DTYPE)
    rec[0] = (p.temperature, min(int(p.top_k), _INT32_MAX), p.top_p, p.repetition_penalty,
              getattr(p, 'presence_penalty', 0.0), getattr(p, 'frequency_penalty', 0.0),
              0.0 if p.temperature == 0 else uniform, row_flags(p))
    return rec


def max_top_k_of(params_list, vocab: int) -> int:
    """Largest top-k of the sampled rows (sizes the candidate slots), 0 if none."""
    return max([min(int(p.top_k), vocab) for p in params_list if p.temperature != 0 and p.top_k > 0] or [0])


def pack_rows(params_list, histories, uniforms, vocab: int):
    """Row parameters (``klsample_row_params``), CSR history and ``max_top_k``."""
    B = len(params_list)
    rows = np.zeros(B, dtype=_lib.ROW_PARAMS_DTYPE)
    offsets = np.zeros(B + 1, dtype=np.int32)
    chunks = []
    total = 0
    for b, p in enumerate(params_list):
        rows[b] = row_record(p, 0.0 if uniforms is None else uniforms[b])[0]
        hist = histories[b] if histories is not None else ()
        if (int(rows['flags'][b]) & (_lib.ROW_REPETITION | _lib.ROW_PRESENCE_FREQUENCY)) and len(hist):
            ids = normalize_history(hist, vocab)
            chunks.append(ids)
            total += ids.size
        offsets[b + 1] = total
    if total > _INT32_MAX:
        raise ValueError('total history length exceeds the int32 CSR offsets')
    ids = np.concatenate(chunks) if chunks else np.zeros(0, dtype=np.int32)
    return rows, offsets, ids, max_top_k_of(params_list, vocab)


@dataclass
class BatchOutput:
    """Host copies of one call's outputs."""

    tokens: np.ndarray          # int64 [B]
    logprobs: np.ndarray        # float32 [B]
    top_ids: np.ndarray         # int32 [B, N]
    top_logprobs: np.ndarray    # float32 [B, N]
    info: np.ndarray | None     # ROW_INFO_DTYPE [B]
    probs: torch.Tensor | None  # device float32 [B, V]
    vocab: int

    def top(self, b: int, count: int):
        count = min(count, self.vocab, self.top_ids.shape[1])
        return tuple((int(self.top_ids[b, t]), float(self.top_logprobs[b, t])) for t in range(count))


class DeviceRunner:
    """Workspace and staging buffers of one (device, host thread)."""

    def __init__(self, device: torch.device):
        if not torch.cuda.is_available():
            raise RuntimeError('klsample runs on a ROCm GPU; no GPU is visible to torch')
        self.device = torch.device(device)
        self.index = self.device.index if self.device.index is not None else torch.cuda.current_device()
        self.lib = _lib.load()
        self.layouts = {}        # call shape -> record and output views (see _layout)
        self.pointers = {}       # id(host array) -> (array, address): arrays handed over repeatedly
        self.generation = 0      # bumped whenever a buffer is replaced
        self.workspace = None
        self.workspace_bytes = 0
        self.stage_dev = None
        self.stage_host = None
        self.out_dev = None
        self.out_host = None

    # -- buffers -------------------------------------------------------------------------
    def _ensure_workspace(self, nbytes: int, stream) -> None:
        if self.workspace_bytes >= nbytes:
            return
        nbytes = _align(max(nbytes, int(self.workspace_bytes * 1.25)), 1 << 20)
        self.generation += 1
        self.layouts.clear()   # (they point into the buffers being replaced)
        with torch.inference_mode(False):   # ordinary tensors: writable in and out of inference mode
            ws = torch.empty(nbytes + 256, dtype=torch.uint8, device=self.device)
        base = ws.data_ptr()
        offset = (-base) % 256
        self.workspace = ws
        self.workspace_ptr = base + offset
        self.workspace_bytes = nbytes
        _lib.check(self.lib, self.lib.klsample_workspace_init(
            ctypes.c_void_p(self.workspace_ptr), ctypes.c_size_t(nbytes), ctypes.c_void_p(stream)))

    def _ensure_stage(self, nbytes: int) -> None:
        if self.stage_dev is not None and self.stage_dev.numel() >= nbytes:
            return
        n = _align(max(nbytes, 4096), 4096)
        with torch.inference_mode(False):
            self.stage_dev = torch.empty(n, dtype=torch.uint8, device=self.device)
            self.stage_host = torch.empty(n, dtype=torch.uint8, pin_memory=True)

    def _ensure_out(self, nbytes: int) -> None:
        if self.out_host is not None and self.out_host.numel() >= nbytes:
            return
        n = _align(max(nbytes, 4096), 4096)
        self.generation += 1
        self.layouts.clear()
        with torch.inference_mode(False):
            self.out_host = torch.empty(n, dtype=torch.uint8, pin_memory=True)
            # the kernels write the outputs straight into this pinned buffer when the
            # device can address it; otherwise into a device twin copied back
            mapped = _lib.mapped_pointer(self.out_host.data_ptr())
            self.out_dev = None if mapped is not None else torch.empty(n, dtype=torch.uint8, device=self.device)
        self.out_ptr = mapped if mapped is not None else self.out_dev.data_ptr()

    # -- one call ------------------------------------------------------------------------
    def run(self, logits: torch.Tensor, params_list, histories, uniforms, num_logprobs: int, *,
            options: int = 0, want_probs: bool = False, want_info: bool = False) -> BatchOutput:
        """Sample every row of ``logits`` ([B, V] on this device) and wait for the result."""
        if logits.dim() != 2:
            raise ValueError('logits must be [batch, vocab]')
        B, V = logits.shape
        # the kernels read one parameter record, CSR offset pair and uniform per logits row
        if len(params_list) != B:
            raise ValueError(f'one SamplingParams per row is required ({len(params_list)} for {B} rows)')
        if histories is not None and len(histories) != B:
            raise ValueError(f'one history per row is required ({len(histories)} for {B} rows)')
        if uniforms is not None and len(uniforms) != B:
            raise ValueError(f'one uniform per row is required ({len(uniforms)} for {B} rows)')
        rows, offsets, ids, max_top_k = pack_rows(params_list, histories, uniforms, V)
        out = self.run_packed(logits, rows, max_top_k, int(num_logprobs),
                              offsets=offsets if ids.size else None, ids=ids if ids.size else None,
                              options=options, want_probs=want_probs, want_info=want_info)
        tokens, logprobs, top_ids, top_lp, info, probs = out
        return BatchOutput(tokens.copy(), logprobs.copy(), top_ids.copy(), top_lp.copy(),
                           info.copy() if info is not None else None, probs, V)

    def _layout(self, key):
        """Library call record and output views of one call shape (built once per shape
        and buffer generation; a call then sets only its pointers)."""
        B, V, dt, max_top_k, N, want_info, options, row_stride, head = key
        ws = _lib.lmhead_workspace_size(B, V, max_top_k, N) if head else _lib.workspace_size(B, V, dt, max_top_k, N)
        self._ensure_workspace(ws, self._stream())
        p_lp = _align(8 * B)
        p_tid = _align(p_lp + 4 * B)
        p_tlp = _align(p_tid + 4 * B * N)
        p_inf = _align(p_tlp + 4 * B * N)
        out_bytes = _align(p_inf + (_lib.ROW_INFO_DTYPE.itemsize * B if want_info else 0))
        self._ensure_out(out_bytes)
        batch = _lib.Batch()
        batch.row_stride = row_stride
        batch.dtype, batch.batch, batch.vocab, batch.num_logprobs, batch.max_top_k = dt, B, V, N, max_top_k
        batch.options = options
        obase = self.out_ptr
        batch.token_ids = obase
        batch.logprobs = obase + p_lp
        batch.top_ids = obase + p_tid if N else None
        batch.top_logprobs = obase + p_tlp if N else None
        batch.row_info = obase + p_inf if want_info else None
        batch.workspace = self.workspace_ptr
        batch.workspace_bytes = self.workspace_bytes
        h = self.out_host.numpy()
        views = (h[:8 * B].view(np.int64), h[p_lp:p_lp + 4 * B].view(np.float32),
                 h[p_tid:p_tid + 4 * B * N].view(np.int32).reshape(B, N),
                 h[p_tlp:p_tlp + 4 * B * N].view(np.float32).reshape(B, N),
                 h[p_inf:p_inf + _lib.ROW_INFO_DTYPE.itemsize * B].view(_lib.ROW_INFO_DTYPE) if want_info else None)
        lay = (self.generation, batch, ctypes.byref(batch), views, out_bytes)
        self.layouts[key] = lay
        return lay

    def _address(self, arr: np.ndarray) -> int:
        hit = self.pointers.get(id(arr))
        if hit is None or hit[0] is not arr:
            if len(self.pointers) > 4096:
                self.pointers.clear()
            hit = self.pointers[id(arr)] = (arr, arr.ctypes.data)
        return hit[1]

    def _stream(self) -> int:
        return torch._C._cuda_getCurrentRawStream(self.index)

    def run_packed(self, logits: torch.Tensor, rows: np.ndarray, max_top_k: int, N: int, *,
                   offsets: np.ndarray | None = None, ids: np.ndarray | None = None, ids_ptr: int | None = None,
                   append_ptr: int | None = None, options: int = 0, want_probs: bool = False,
                   want_info: bool = False, host_params: bool | None = None, head=None):
        """One library call on packed rows (``klsample_row_params`` records) and wait.

        ``logits`` is ``[B, V]`` (or one ``[V]`` row).  ``offsets`` are the history
        offsets (CSR, or begin/end pairs with ``OPT_HISTORY_PAIRS``) into ``ids`` (host,
        uploaded with the call) or into device ids at ``ids_ptr``; ``append_ptr`` is
        ``history_append``.  Up to ``HOST_PARAMS_MAX_BATCH`` rows hand their parameters
        and offsets over in host memory (carried in the kernel arguments: nothing is
        uploaded without host ids); ``host_params=False`` stages them as a larger batch's
        are.  Returns host views of tokens, logprobs, top ids, top logprobs and row info
        (valid until the next call on this runner) and the device probabilities.  With
        ``head`` (a ``klsample_lmhead``), ``logits`` is the fp32 output the LM head writes
        and the call is ``klsample_lmhead_run``."""
        if logits.dtype not in _DTYPES:
            logits = logits.float()
        if logits.dim() == 1:
            B, V = 1, logits.shape[0]
            if logits.stride(0) != 1:
                logits = logits.contiguous()
            row_stride = V
        else:
            B, V = logits.shape
            # rows must not overlap (a size-1 dimension may carry any stride)
            if logits.stride(1) != 1 or (B > 1 and logits.stride(0) < V):
                logits = logits.contiguous()
            row_stride = logits.stride(0) if B > 1 else V
        if host_params is None:
            host_params = B <= _lib.HOST_PARAMS_MAX_BATCH
        if host_params:
            options |= _lib.OPT_HOST_PARAMS
        key = (B, V, _DTYPES[logits.dtype], max_top_k, N, want_info, options, row_stride, head is not None)
        lay = self.layouts.get(key)
        if lay is None or lay[0] != self.generation:
            lay = self._layout(key)
        _, batch, ref, views, out_bytes = lay
        # one host-to-device copy, if any: params | offsets (larger batches) | ids
        o_off = 0 if host_params else _align(rows.nbytes)
        o_ids = o_off if offsets is None or host_params else _align(o_off + offsets.nbytes)
        stage_bytes = _align(o_ids + (ids.nbytes if ids is not None else 0))
        if stage_bytes:
            self._ensure_stage(stage_bytes)
            host = self.stage_host.numpy()
            if not host_params:
                host[:rows.nbytes] = rows.view(np.uint8)
                if offsets is not None:
                    host[o_off:o_off + offsets.nbytes] = offsets.view(np.uint8)
            if ids is not None:
                host[o_ids:o_ids + ids.nbytes] = ids.view(np.uint8)
            self.stage_dev[:stage_bytes].copy_(self.stage_host[:stage_bytes], non_blocking=True)
            dbase = self.stage_dev.data_ptr()
        if host_params:
            batch.params = self._address(rows)
            batch.history_offsets = self._address(offsets) if offsets is not None else None
        else:
            batch.params = dbase
            batch.history_offsets = dbase + o_off if offsets is not None else None
        batch.history_ids = dbase + o_ids if ids is not None else ids_ptr
        batch.history_append = append_ptr
        batch.logits = logits.data_ptr()
        probs = None
        if want_probs:
            probs = torch.empty((B, V), dtype=torch.float32, device=self.device)
            batch.probs = probs.data_ptr()
        else:
            batch.probs = None
        sptr = self._stream()
        if head is None:
            status = self.lib.klsample_run(ref, sptr)
        else:
            status = self.lib.klsample_lmhead_run(ref, ctypes.byref(head), sptr)
        if status:
            _lib.check(self.lib, status)
        if self.out_dev is not None:
            self.out_host[:out_bytes].copy_(self.out_dev[:out_bytes], non_blocking=True)
        _lib.stream_synchronize(sptr)
        return views + (probs,)


_local = threading.local()


def runner_for(device: torch.device) -> DeviceRunner:
    """The calling thread's runner for ``device`` (created on first use)."""
    runners = getattr(_local, 'runners', None)
    if runners is None:
        runners = _local.runners = {}
    key = (device.type, device.index)
    r = runners.get(key)
    if r is None:
        r = runners[key] = DeviceRunner(device)
    return r


def target_device(logits: torch.Tensor) -> torch.device:
    if logits.is_cuda:
        return logits.device
    if not torch.cuda.is_available():
        raise RuntimeError('klsample runs on a ROCm GPU; no GPU is visible to torch')
    return torch.device('cuda', torch.cuda.current_device())
