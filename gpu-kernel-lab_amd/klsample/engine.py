"""The sampling side of a serving-engine step, batched (serving/engine.py:70-131).

The reference engine calls ``Sampler.sample`` once per row, with ``prompt + generated``
rebuilt as a host tuple every step (serving/engine.py:94, :105-106), on logits its
executor returns as a per-request dict split out of one ``[B, V]`` tensor
(serving/qwen_executor.py:136).  Here one step is one library call over the whole
device-resident ``[B, V]`` tensor:

* :class:`DeviceHistory` keeps every request's history (prompt, then each sampled token)
  in one device arena.  A call passes each row's ``[begin, end)`` range and the library
  appends the sampled token itself (``KLSAMPLE_OPT_HISTORY_PAIRS`` + ``history_append``),
  so a step uploads no history.
* :class:`BatchedStep` packs each request's parameters once (only the uniform changes
  per step) and makes the call through its own runner: small batches hand their
  parameters and ranges over in the kernel arguments, larger ones in one upload, and the
  outputs come back in pinned host memory the kernels write directly.
* :class:`TokenEvent` and :func:`sse_chunk` are the wire format of a sampled token
  (serving/engine.py:21-24, :127-128; serving/api.py:58-70).
* :class:`SamplingLoop` drives them like ``ServingEngine.step``: decode rows first, then
  the first token of each finished prefill with the prompt as its history; a request
  finishes on a stop token (``'stop'``) or at ``max_tokens`` (``'length'``), and any
  exception raised by a step fails every unfinished request of it
  (serving/engine.py:109-115).
"""
from __future__ import annotations

import json
from collections.abc import Mapping
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib
from .runner import _INT32_MAX, DeviceRunner, max_top_k_of, normalize_history, row_record
from .sampling import SampleResult, Sampler


class DeviceHistory:
    """Per-request token histories in one device arena of int32 ids.

    A request owns a segment of the arena; its history is the segment's first ``length``
    ids and the slot just past them is kept free for the token the next call appends.
    Segment bookkeeping lives in host arrays indexed by a per-request slot, so a step
    reads and advances the ranges of all its rows with array operations.  A full segment
    moves to one twice its size (device-to-device copy); the arena grows by copying into
    a larger one; released segments are reused.
    """

    def __init__(self, device, vocab: int, capacity: int = 1 << 20, reserve: int = 256):
        self.device = torch.device(device)
        self.vocab = int(vocab)
        self.reserve = max(int(reserve), 1)
        self.arena = torch.empty(max(int(capacity), 1024), dtype=torch.int32, device=self.device)
        self.top = 0
        self.free_segments = []      # (start, cap) of released segments
        self.slot = {}               # request id -> slot
        self.free_slots = []
        self.start = np.zeros(64, dtype=np.int64)
        self.length = np.zeros(64, dtype=np.int64)
        self.cap = np.zeros(64, dtype=np.int64)

    def _alloc(self, cap: int) -> int:
        for i, (start, c) in enumerate(self.free_segments):
            if c >= cap:
                self.free_segments.pop(i)
                if c > cap:
                    self.free_segments.append((start + cap, c - cap))
                return start
        if self.top + cap > self.arena.numel():
            if self.top + cap > _INT32_MAX:
                raise ValueError('the history arena would exceed int32 offsets')
            bigger = torch.empty(min(max(2 * self.arena.numel(), self.top + cap), _INT32_MAX),
                                 dtype=torch.int32, device=self.device)
            bigger[:self.top].copy_(self.arena[:self.top])
            self.arena = bigger
        start = self.top
        self.top += cap
        return start

    def register(self, rid, prompt_ids) -> None:
        """Start ``rid``'s history with its prompt ids (negative ids count from the end,
        ids outside ``[-vocab, vocab)`` raise ``IndexError``, as ``scores[ids]`` does in
        serving/sampling.py:48-49)."""
        if rid in self.slot:
            raise KeyError(f'request {rid!r} is already registered')
        ids = normalize_history(prompt_ids, self.vocab)
        cap = ids.size + self.reserve
        start = self._alloc(cap)
        if ids.size:
            self.arena[start:start + ids.size].copy_(torch.from_numpy(ids))
        if self.free_slots:
            s = self.free_slots.pop()
        else:
            s = len(self.slot)
            if s == self.start.size:
                self.start, self.length, self.cap = (np.concatenate([x, np.zeros_like(x)])
                                                     for x in (self.start, self.length, self.cap))
        self.slot[rid] = s
        self.start[s], self.length[s], self.cap[s] = start, ids.size, cap

    def slots(self, rids) -> np.ndarray:
        return np.fromiter((self.slot[r] for r in rids), dtype=np.int64, count=len(rids))

    def prepare(self, slots: np.ndarray, out: np.ndarray | None = None) -> np.ndarray:
        """Room for one more token in each of these requests; their ``[begin, end)``
        ranges as the library's history pairs (int32, 2 per row), in ``out`` if given."""
        full = slots[self.length[slots] >= self.cap[slots]]
        for s in full.tolist():
            start, length, cap = int(self.start[s]), int(self.length[s]), int(self.cap[s])
            new_start = self._alloc(2 * cap)
            self.arena[new_start:new_start + length].copy_(self.arena[start:start + length])
            self.free_segments.append((start, cap))
            self.start[s], self.cap[s] = new_start, 2 * cap
        if out is None or out.size != 2 * slots.size:
            out = np.empty(2 * slots.size, dtype=np.int32)
        out[0::2] = self.start[slots]
        out[1::2] = self.start[slots] + self.length[slots]
        return out

    def advance(self, slots: np.ndarray) -> None:
        """Each of these requests had one token appended by the last call."""
        self.length[slots] += 1

    def ids(self, rid) -> np.ndarray:
        s = self.slot[rid]
        start, length = int(self.start[s]), int(self.length[s])
        return self.arena[start:start + length].cpu().numpy()

    def release(self, rid) -> None:
        s = self.slot.pop(rid)
        self.free_segments.append((int(self.start[s]), int(self.cap[s])))
        self.length[s] = self.cap[s] = 0
        self.free_slots.append(s)


def as_batch(logits, rids) -> torch.Tensor:
    """``[B, V]`` logits of ``rids``: a tensor as is, or the executor's per-request dict
    (serving/qwen_executor.py:136).  Rows that are evenly spaced views of one tensor are
    used in place; others are stacked."""
    if not isinstance(logits, Mapping):
        return logits
    rows = [logits[r] for r in rids]
    if not rows:
        raise ValueError('no rows to sample')
    r0 = rows[0]
    if r0.dim() != 1:
        raise ValueError('logits must be floating vectors')
    if len(rows) == 1:
        return r0.unsqueeze(0)
    base = r0.untyped_storage().data_ptr()
    step = rows[1].storage_offset() - r0.storage_offset()
    if r0.stride(0) == 1 and step >= r0.numel() and all(
            r.dim() == 1 and r.dtype == r0.dtype and r.device == r0.device and r.numel() == r0.numel()
            and r.stride(0) == 1 and r.untyped_storage().data_ptr() == base
            and r.storage_offset() == r0.storage_offset() + i * step for i, r in enumerate(rows)):
        return r0.as_strided((len(rows), r0.numel()), (step, 1))
    return torch.stack(rows)


@dataclass
class StepOutput:
    """One step's results, row-aligned: host arrays (copies)."""

    tokens: np.ndarray          # int64 [B]
    logprobs: np.ndarray        # float32 [B]
    top_ids: np.ndarray         # int32 [B, N]
    top_logprobs: np.ndarray    # float32 [B, N]
    stopped: np.ndarray         # bool [B]: the token is one of the row's stop ids
    counts: list                # top-N entries each row asked for


class BatchedStep:
    """One sampling call for all rows of a device-resident ``[B, V]`` logits tensor.

    Row ``b`` is sampled with ``samplers[b]`` (its parameters and its own uniform stream)
    and, given a :class:`DeviceHistory`, with the device history of request ``rids[b]``,
    to which the library appends the sampled token.  The results equal ``B`` separate
    ``Sampler.sample`` calls with ``history = prompt + generated``.

    While a set of rows stays the same from step to step, the step holds each sampled
    request's pending uniforms (taken from its Sampler a block at a time, handed back
    when the set changes or on :meth:`release`), so a step reads its uniforms with one
    array gather."""

    def __init__(self, device, history: DeviceHistory | None = None):
        self.runner = DeviceRunner(torch.device(device))
        self.device = self.runner.device
        self.history = history
        self.records = {}       # id(sampler) -> (sampler, row record)
        self.key = None         # the current set's (samplers, rids, vocab) identity
        self.sampled = []

    def _record(self, s: Sampler) -> np.ndarray:
        hit = self.records.get(id(s))
        if hit is None or hit[0] is not s:
            hit = self.records[id(s)] = (s, row_record(s.params))
        return hit[1]

    def release(self) -> None:
        """Hand the pending uniforms back to their samplers."""
        for i, s in enumerate(self.sampled):
            s.return_uniforms(self.device, self.U[i, self.pos[i]:self.lim[i]])
        self.sampled = []
        self.key = None

    def forget(self, sampler: Sampler) -> None:
        self.release()
        self.records.pop(id(sampler), None)

    def _take(self, i: int) -> None:
        blk = self.sampled[i].take_uniforms(self.device)
        self.U[i, :blk.size] = blk
        self.pos[i], self.lim[i] = 0, blk.size

    def _compose(self, rids, samplers, V: int) -> None:
        self.release()
        self.rows = np.concatenate([self._record(s) for s in samplers])
        self.sampled_idx = np.array([b for b, s in enumerate(samplers) if s.params.temperature != 0], dtype=np.int64)
        self.sampled = [samplers[b] for b in self.sampled_idx.tolist()]
        n = len(self.sampled)
        self.U = np.zeros((n, 64), dtype=np.float32)
        self.pos = np.zeros(n, dtype=np.int64)
        self.lim = np.zeros(n, dtype=np.int64)
        self.ar = np.arange(n)
        for i in range(n):
            self._take(i)
        self.max_top_k = max_top_k_of([s.params for s in samplers], V)
        self.N = min(max(s.params.logprobs for s in samplers), _lib.MAX_LOGPROBS)
        self.counts = [min(s.params.logprobs, V, self.N) for s in samplers]
        self.stop_rows = [(b, s.params.stop_token_ids) for b, s in enumerate(samplers) if s.params.stop_token_ids]
        self.slots = self.history.slots(rids) if self.history is not None else None
        self.ranges = np.empty(2 * len(rids), dtype=np.int32)

    def run(self, rids, samplers, logits: torch.Tensor) -> StepOutput:
        if logits.dim() != 2 or not logits.is_floating_point():
            raise ValueError('logits must be a floating [batch, vocab] tensor')
        B, V = logits.shape
        if len(samplers) != B or (self.history is not None and len(rids) != B):
            raise ValueError(f'one request per row is required ({len(samplers)} samplers for {B} rows)')
        if logits.device != self.device:
            raise ValueError(f'logits must be on {self.device} (got {logits.device})')
        hist = self.history
        if hist is not None and V != hist.vocab:
            raise ValueError(f'logits have {V} columns, the history arena {hist.vocab}')
        key = (tuple(map(id, samplers)), tuple(rids) if hist is not None else None, V)
        if key != self.key:
            self._compose(rids, samplers, V)
            self.key = key
        rows, N = self.rows, self.N
        if self.sampled:
            for i in np.flatnonzero(self.pos == self.lim).tolist():
                self._take(i)
            rows['uniform'][self.sampled_idx] = self.U[self.ar, self.pos]
            self.pos += 1
        if hist is not None:
            ranges = hist.prepare(self.slots, self.ranges)
            arena = hist.arena.data_ptr()
            out = self.runner.run_packed(logits, rows, self.max_top_k, N, offsets=ranges, ids_ptr=arena,
                                         append_ptr=arena, options=_lib.OPT_HISTORY_PAIRS)
            hist.advance(self.slots)
        else:
            out = self.runner.run_packed(logits, rows, self.max_top_k, N)
        tokens = out[0].copy()
        stopped = np.zeros(B, dtype=bool)
        for b, stop in self.stop_rows:
            stopped[b] = int(tokens[b]) in stop
        return StepOutput(tokens, out[1].copy(), out[2].copy(), out[3].copy(), stopped, self.counts)

    def sample(self, rids, samplers, logits: torch.Tensor) -> list[SampleResult]:
        """:meth:`run` as one ``SampleResult`` per row."""
        o = self.run(rids, samplers, logits)
        tids, tlps = o.top_ids.tolist(), o.top_logprobs.tolist()
        return [SampleResult(t, lp, tuple(zip(ti[:n], tl[:n])), st)
                for t, lp, ti, tl, n, st in zip(o.tokens.tolist(), o.logprobs.tolist(), tids, tlps, o.counts,
                                                o.stopped.tolist())]


@dataclass(frozen=True)
class TokenEvent:
    """One streamed event of a request (serving/engine.py:21-24)."""

    request_id: str
    token_id: int | None = None
    logprob: float | None = None
    top_logprobs: tuple = ()
    finished: bool = False
    finish_reason: str | None = None
    error: str | None = None


SSE_DONE = 'data: [DONE]\n\n'


def sse_chunk(event: TokenEvent, text: str = '', chat: bool = False) -> str:
    """The server-sent-events line of one event (serving/api.py:58-70): a token's
    ``logprobs`` object holds its logprob and its top-N list of ``[id, logprob]`` pairs,
    best first, equal logprobs in ascending id order; a finished event carries the
    finish reason (and is followed by :data:`SSE_DONE`)."""
    obj = 'chat.completion.chunk' if chat else 'text_completion'
    if event.finished:
        choice = {'index': 0, 'delta': {} if chat else None, 'text': '' if not chat else None,
                  'finish_reason': event.finish_reason}
    else:
        choice = {'index': 0, 'finish_reason': None,
                  'logprobs': {'token_logprob': event.logprob, 'top_logprobs': event.top_logprobs}}
        if chat:
            choice['delta'] = {'content': text}
        else:
            choice['text'] = text
    return 'data: ' + json.dumps({'id': event.request_id, 'object': obj, 'choices': [choice]}) + '\n\n'


class SamplingLoop:
    """The sampling side of ``ServingEngine`` (serving/engine.py:47-131) over batched calls.

    ``submit`` registers a request (its prompt becomes its device history); ``step`` takes
    the decode rows' and the finished prefills' logits (each a ``[B, V]`` device tensor in
    ``rids`` order, or the executor's per-request dict) and makes one library call for
    each.  ``events[rid]`` lists the request's :class:`TokenEvent` s."""

    def __init__(self, device, vocab: int, **history_kw):
        self.history = DeviceHistory(device, vocab, **history_kw)
        self.sampling = BatchedStep(device, self.history)
        self.samplers, self.max_tokens, self.generated, self.state, self.events = {}, {}, {}, {}, {}

    def submit(self, rid, params, prompt_ids, max_tokens: int) -> None:
        if max_tokens < 1:
            raise ValueError('max_tokens must be >= 1')
        self.history.register(rid, prompt_ids)
        self.samplers[rid] = Sampler(params, device=self.sampling.device)
        self.max_tokens[rid] = int(max_tokens)
        self.generated[rid] = []
        self.state[rid] = 'prefill'
        self.events[rid] = []

    @property
    def finished(self) -> bool:
        return all(s in ('finished', 'failed') for s in self.state.values())

    def _finish(self, rid, reason, error=None) -> None:
        self.state[rid] = 'failed' if reason == 'error' else 'finished'
        self.events[rid].append(TokenEvent(rid, finished=True, finish_reason=reason, error=error))
        self.sampling.forget(self.samplers[rid])
        self.history.release(rid)

    def _sample(self, rids, logits, expect) -> None:
        for rid in rids:
            if self.state.get(rid) != expect:
                raise ValueError(f'request {rid!r} is not in the {expect} state')
        o = self.sampling.run(list(rids), [self.samplers[r] for r in rids], as_batch(logits, rids))
        tids, tlps = o.top_ids.tolist(), o.top_logprobs.tolist()
        for rid, token, lp, ti, tl, n, stopped in zip(rids, o.tokens.tolist(), o.logprobs.tolist(), tids, tlps,
                                                      o.counts, o.stopped.tolist()):
            self.generated[rid].append(token)
            self.state[rid] = 'decode'
            self.events[rid].append(TokenEvent(rid, token, lp, tuple(zip(ti[:n], tl[:n]))))
            if stopped or len(self.generated[rid]) >= self.max_tokens[rid]:
                self._finish(rid, 'stop' if stopped else 'length')

    def step(self, decode_rids=(), decode_logits=None, prefill_rids=(), prefill_logits=None) -> None:
        try:
            if decode_rids:
                self._sample(decode_rids, decode_logits, 'decode')
            if prefill_rids:
                self._sample(prefill_rids, prefill_logits, 'prefill')
        except Exception as error:
            for rid in (*decode_rids, *prefill_rids):
                if self.state.get(rid) in ('prefill', 'decode'):
                    self._finish(rid, 'error', str(error))
