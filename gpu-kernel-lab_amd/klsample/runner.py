"""Device-side execution of batched sampling calls through the C ABI.

A :class:`DeviceRunner` owns, per GPU and per host thread, the library workspace and
the staging buffers of a call: one pinned host buffer carrying the row parameters and
the CSR history up in a single copy, and one device output arena brought back in a
single copy.  Buffers only grow; a call allocates nothing once they are large enough.
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


def pack_rows(params_list, histories, uniforms, vocab: int):
    """Row parameters (``klsample_row_params``), CSR history and ``max_top_k``.

    The flags carry the reference's tests on the original Python values
    (``serving/sampling.py:47``, ``:50``, ``:56``); the floats are their fp32 roundings,
    which is what the reference's tensor-by-scalar operations use.
    """
    B = len(params_list)
    rows = np.zeros(B, dtype=_lib.ROW_PARAMS_DTYPE)
    offsets = np.zeros(B + 1, dtype=np.int32)
    chunks = []
    total = 0
    max_top_k = 0
    for b, p in enumerate(params_list):
        flags = 0
        greedy = p.temperature == 0
        if greedy:
            flags |= _lib.ROW_GREEDY
        rep = p.repetition_penalty != 1
        pf = getattr(p, 'presence_penalty', 0.0) != 0 or getattr(p, 'frequency_penalty', 0.0) != 0
        if rep:
            flags |= _lib.ROW_REPETITION
        if pf:
            flags |= _lib.ROW_PRESENCE_FREQUENCY
        if p.top_p < 1:
            flags |= _lib.ROW_TOP_P
        top_k = min(int(p.top_k), _INT32_MAX)
        rows[b] = (p.temperature, top_k, p.top_p, p.repetition_penalty,
                   getattr(p, 'presence_penalty', 0.0), getattr(p, 'frequency_penalty', 0.0),
                   0.0 if uniforms is None or greedy else uniforms[b], flags)
        if not greedy and top_k > 0:
            max_top_k = max(max_top_k, min(top_k, vocab))
        hist = histories[b] if histories is not None else ()
        if (rep or pf) and len(hist):
            ids = normalize_history(hist, vocab)
            chunks.append(ids)
            total += ids.size
        offsets[b + 1] = total
    if total > _INT32_MAX:
        raise ValueError('total history length exceeds the int32 CSR offsets')
    ids = np.concatenate(chunks) if chunks else np.zeros(0, dtype=np.int32)
    return rows, offsets, ids, max_top_k


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
        self.lib = _lib.load()
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
        self.stage_dev = torch.empty(n, dtype=torch.uint8, device=self.device)
        self.stage_host = torch.empty(n, dtype=torch.uint8, pin_memory=True)

    def _ensure_out(self, nbytes: int) -> None:
        if self.out_dev is not None and self.out_dev.numel() >= nbytes:
            return
        n = _align(max(nbytes, 4096), 4096)
        self.out_dev = torch.empty(n, dtype=torch.uint8, device=self.device)
        self.out_host = torch.empty(n, dtype=torch.uint8, pin_memory=True)

    # -- one call ------------------------------------------------------------------------
    def run(self, logits: torch.Tensor, params_list, histories, uniforms, num_logprobs: int, *,
            options: int = 0, want_probs: bool = False, want_info: bool = False) -> BatchOutput:
        """Sample every row of ``logits`` ([B, V] on this device) and wait for the result."""
        if logits.dim() != 2:
            raise ValueError('logits must be [batch, vocab]')
        if logits.dtype not in _DTYPES:
            logits = logits.float()
        B, V = logits.shape
        # the kernels read one parameter record, CSR offset pair and uniform per logits row
        if len(params_list) != B:
            raise ValueError(f'one SamplingParams per row is required ({len(params_list)} for {B} rows)')
        if histories is not None and len(histories) != B:
            raise ValueError(f'one history per row is required ({len(histories)} for {B} rows)')
        if uniforms is not None and len(uniforms) != B:
            raise ValueError(f'one uniform per row is required ({len(uniforms)} for {B} rows)')
        # rows must not overlap (a size-1 dimension may carry any stride)
        if logits.stride(1) != 1 or (B > 1 and logits.stride(0) < V):
            logits = logits.contiguous()
        row_stride = logits.stride(0) if B > 1 else V
        N = int(num_logprobs)
        rows, offsets, ids, max_top_k = pack_rows(params_list, histories, uniforms, V)
        stream = torch.cuda.current_stream(self.device)
        sptr = stream.cuda_stream

        ws_bytes = _lib.workspace_size(B, V, _DTYPES[logits.dtype], max_top_k, N)
        self._ensure_workspace(ws_bytes, sptr)

        # one host-to-device copy: params | offsets | ids
        o_par = 0
        o_off = _align(o_par + rows.nbytes)
        o_ids = _align(o_off + offsets.nbytes)
        stage_bytes = _align(o_ids + ids.nbytes)
        self._ensure_stage(stage_bytes)
        host = self.stage_host.numpy()
        host[o_par:o_par + rows.nbytes] = rows.view(np.uint8)
        host[o_off:o_off + offsets.nbytes] = offsets.view(np.uint8)
        if ids.size:
            host[o_ids:o_ids + ids.nbytes] = ids.view(np.uint8)
        self.stage_dev[:stage_bytes].copy_(self.stage_host[:stage_bytes], non_blocking=True)
        dbase = self.stage_dev.data_ptr()

        # one device-to-host copy: tokens | logprobs | top ids | top logprobs | info
        p_tok = 0
        p_lp = _align(p_tok + 8 * B)
        p_tid = _align(p_lp + 4 * B)
        p_tlp = _align(p_tid + 4 * B * N)
        p_inf = _align(p_tlp + 4 * B * N)
        out_bytes = _align(p_inf + (_lib.ROW_INFO_DTYPE.itemsize * B if want_info else 0))
        self._ensure_out(out_bytes)
        obase = self.out_dev.data_ptr()
        probs = torch.empty((B, V), dtype=torch.float32, device=self.device) if want_probs else None

        batch = _lib.Batch()
        batch.logits = logits.data_ptr()
        batch.row_stride = row_stride
        batch.dtype = _DTYPES[logits.dtype]
        batch.batch = B
        batch.vocab = V
        batch.num_logprobs = N
        batch.max_top_k = max_top_k
        batch.options = options
        batch.params = dbase + o_par
        batch.history_ids = dbase + o_ids if ids.size else None
        batch.history_offsets = dbase + o_off if ids.size else None
        batch.token_ids = obase + p_tok
        batch.logprobs = obase + p_lp
        batch.top_ids = obase + p_tid if N else None
        batch.top_logprobs = obase + p_tlp if N else None
        batch.probs = probs.data_ptr() if probs is not None else None
        batch.row_info = obase + p_inf if want_info else None
        batch.workspace = self.workspace_ptr
        batch.workspace_bytes = self.workspace_bytes
        _lib.check(self.lib, self.lib.klsample_run(ctypes.byref(batch), ctypes.c_void_p(sptr)))

        self.out_host[:out_bytes].copy_(self.out_dev[:out_bytes], non_blocking=True)
        stream.synchronize()
        h = self.out_host.numpy()
        tokens = h[p_tok:p_tok + 8 * B].view(np.int64).copy()
        logprobs = h[p_lp:p_lp + 4 * B].view(np.float32).copy()
        top_ids = h[p_tid:p_tid + 4 * B * N].view(np.int32).reshape(B, N).copy()
        top_lp = h[p_tlp:p_tlp + 4 * B * N].view(np.float32).reshape(B, N).copy()
        info = h[p_inf:p_inf + _lib.ROW_INFO_DTYPE.itemsize * B].view(_lib.ROW_INFO_DTYPE).copy() if want_info else None
        return BatchOutput(tokens, logprobs, top_ids, top_lp, info, probs, V)


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
