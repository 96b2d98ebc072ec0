"""Drop-in replacement for the reference's ``serving/sampling.py``.

Same names, constructor, call signature, validation and results as
``serving/sampling.py:7-63``:

* ``SamplingParams`` keeps the reference's fields and positional order (the HTTP layer
  builds it positionally, ``serving/api.py:50-51``) and appends
  ``presence_penalty`` and ``frequency_penalty`` after ``logprobs``;
* ``Sampler(params, device='cpu').sample(logits, history=())`` returns a
  ``SampleResult``.

Every call runs on the GPU through ``libklsample.so``; logits that live on the host
are copied to the current GPU first.  The multinomial draw of
``serving/sampling.py:60`` becomes an inverse CDF on one uniform per sampled call,
drawn from the request's generator seeded with ``params.seed``, so a request's
tokens do not depend on how it is batched.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib
from .runner import row_record, runner_for, target_device

_UNIFORM_BLOCK = 64


@dataclass(frozen=True)
class SamplingParams:
    """Per-request sampling parameters (``serving/sampling.py:7-21``)."""

    temperature: float = 0.0
    top_k: int = 0
    top_p: float = 1.0
    repetition_penalty: float = 1.0
    stop_token_ids: frozenset[int] = frozenset()
    seed: int = 0
    logprobs: int = 0
    presence_penalty: float = 0.0
    frequency_penalty: float = 0.0

    def __post_init__(self):
        # serving/sampling.py:18-21
        if self.temperature < 0 or not math.isfinite(self.temperature):
            raise ValueError('temperature must be finite and nonnegative')
        if self.top_k < 0 or not 0 < self.top_p <= 1:
            raise ValueError('invalid top-k/top-p')
        if self.repetition_penalty <= 0 or not math.isfinite(self.repetition_penalty):
            raise ValueError('repetition penalty must be positive')
        if self.logprobs < 0:
            raise ValueError('logprobs must be nonnegative')
        # additions of this implementation
        if not (math.isfinite(self.presence_penalty) and math.isfinite(self.frequency_penalty)):
            raise ValueError('presence and frequency penalties must be finite')
        if self.logprobs > _lib.MAX_LOGPROBS:
            raise ValueError(f'logprobs must be at most {_lib.MAX_LOGPROBS}')


@dataclass(frozen=True)
class SampleResult:
    """One sampled token (``serving/sampling.py:24-29``)."""

    token_id: int
    logprob: float
    top_logprobs: tuple[tuple[int, float], ...]
    stopped: bool


class Sampler:
    """Per-request sampler (``serving/sampling.py:32-63``)."""

    def __init__(self, params: SamplingParams, device='cpu'):
        self.params = params
        self.generators = {}
        self.uniforms = {}    # device key -> [block of uniforms, next index]
        self.record = None    # the packed klsample_row_params of params
        if device is not None:
            self._generator(torch.device(device))

    def _generator(self, device):
        # One generator per device key, as in serving/sampling.py:37-41.  It is a CPU
        # generator whatever the device: it only supplies the draw's uniform.
        key = str(device)
        if key not in self.generators:
            self.generators[key] = torch.Generator(device='cpu').manual_seed(self.params.seed)
        return self.generators[key]

    def next_uniform(self, device) -> float:
        """The uniform of this request's next sampled call.

        Uniforms are drawn from the generator in blocks of 64 and served in order: a
        block draw yields the same sequence as 64 single draws, at the cost of about one.
        The generator's own state therefore runs up to 63 draws ahead of the calls."""
        key = str(device)
        block = self.uniforms.get(key)
        if block is None or block[1] == len(block[0]):
            block = self.uniforms[key] = [torch.rand(_UNIFORM_BLOCK, generator=self._generator(device)).tolist(), 0]
        u = block[0][block[1]]
        block[1] += 1
        return u

    def take_uniforms(self, device) -> np.ndarray:
        """Hand the rest of the current block of uniforms (a fresh block if it is spent)
        to a caller that consumes them in order, as fp32 values.  Until they are returned
        (:meth:`return_uniforms`), the request's draws belong to that caller."""
        key = str(device)
        block = self.uniforms.get(key)
        if block is None or block[1] == len(block[0]):
            out = torch.rand(_UNIFORM_BLOCK, generator=self._generator(device)).numpy()
        else:
            out = np.asarray(block[0][block[1]:], dtype=np.float32)
        self.uniforms[key] = [[], 0]
        return out

    def return_uniforms(self, device, rest) -> None:
        """Give back the unconsumed part of what :meth:`take_uniforms` handed out; the
        next draws continue from its first value."""
        self.uniforms[str(device)] = [[float(u) for u in rest], 0]

    @torch.inference_mode()
    def sample(self, logits: torch.Tensor, history=()) -> SampleResult:
        if logits.ndim != 1 or not logits.is_floating_point():
            raise ValueError('logits must be a floating vector')
        p = self.params
        u = self.next_uniform(logits.device) if p.temperature != 0 else 0.0
        if self.record is None:
            self.record = row_record(p)
        rec = self.record
        if (int(rec['flags'][0]) & (_lib.ROW_REPETITION | _lib.ROW_PRESENCE_FREQUENCY)) and len(history):
            return _run([logits], [p], [history], [u])[0]
        # no history to apply: the packed record goes to the library as it is
        device = target_device(logits)
        if logits.device != device:
            logits = logits.to(device)
        V = logits.numel()
        rec['uniform'][0] = u
        N = min(p.logprobs, _lib.MAX_LOGPROBS)
        top_k = min(int(p.top_k), V) if p.temperature != 0 and p.top_k > 0 else 0
        tokens, lps, tids, tlps, _, _ = runner_for(device).run_packed(logits, rec, top_k, N)
        token = int(tokens[0])
        n = min(p.logprobs, V, N)
        return SampleResult(token, float(lps[0]), tuple(zip(tids[0, :n].tolist(), tlps[0, :n].tolist())),
                            token in p.stop_token_ids)

    @staticmethod
    @torch.inference_mode()
    def sample_many(samplers, logits, histories) -> list[SampleResult]:
        """One batched call for many requests: ``logits`` is ``[B, V]`` (or a sequence
        of B vectors), row b sampled with ``samplers[b]`` and ``histories[b]``.  Each
        sampled row consumes one uniform of its own request's generator, so results
        equal B separate ``sample`` calls."""
        if isinstance(logits, torch.Tensor) and logits.dim() == 2:
            rows, devices = logits, [logits.device] * logits.shape[0]
        else:
            rows = list(logits)
            devices = [r.device for r in rows]
        if len(devices) != len(samplers):
            raise ValueError('one sampler per row is required')
        if histories is not None and len(histories) != len(samplers):
            raise ValueError('one history per row is required')
        params = [s.params for s in samplers]
        us = [s.next_uniform(d) if s.params.temperature != 0 else 0.0 for s, d in zip(samplers, devices)]
        return _run(rows, params, histories, us)


def _results(out, params_list) -> list[SampleResult]:
    res = []
    for b, p in enumerate(params_list):
        token = int(out.tokens[b])
        res.append(SampleResult(token, float(out.logprobs[b]), out.top(b, p.logprobs),
                                token in p.stop_token_ids))
    return res


def _stack(rows) -> torch.Tensor:
    if isinstance(rows, torch.Tensor):
        if rows.dim() != 2 or not rows.is_floating_point():
            raise ValueError('logits must be a floating [batch, vocab] tensor')
        return rows
    if not rows:
        raise ValueError('no rows to sample')
    for r in rows:
        if r.ndim != 1 or not r.is_floating_point():
            raise ValueError('logits must be a floating vector')
    if len(rows) == 1:
        return rows[0].unsqueeze(0)
    dtype = rows[0].dtype if all(r.dtype == rows[0].dtype for r in rows) else torch.float32
    return torch.stack([r.to(dtype) for r in rows])


def _run(rows, params_list, histories, uniforms, **kw) -> list[SampleResult]:
    logits = _stack(rows)
    device = target_device(logits)
    if logits.device != device:
        logits = logits.to(device)
    num_logprobs = max((p.logprobs for p in params_list), default=0)
    num_logprobs = min(num_logprobs, _lib.MAX_LOGPROBS)
    out = runner_for(device).run(logits, params_list, histories, uniforms, num_logprobs, **kw)
    return _results(out, params_list)


def sample_batch(logits: torch.Tensor, params_list, histories=None, uniforms=None, **kw):
    """Batched entry point: one token per row of ``logits`` ([B, V]) with per-row
    parameters, histories and caller-supplied uniforms (one float in [0, 1) per row;
    ignored for greedy rows).  Returns ``list[SampleResult]``."""
    B = logits.shape[0]
    if len(params_list) != B:
        raise ValueError('one SamplingParams per row is required')
    if histories is not None and len(histories) != B:
        raise ValueError('one history per row is required')
    if uniforms is None:
        if any(p.temperature != 0 for p in params_list):
            raise ValueError('uniforms are required for sampled rows')
        uniforms = [0.0] * B
    return _run(logits, params_list, histories, [float(u) for u in uniforms], **kw)
