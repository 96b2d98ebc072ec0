"""The LM head fused with the sampling call (prototype).

The reference's decode step computes ``self.model.lm_head(hidden)[:,0].float()``
(serving/qwen_executor.py:238), a bf16 ``[B, d] x [d, V]`` product, and the sampler then
reads the ``[B, V]`` logits back (serving/engine.py:94).  :func:`lmhead_sample` makes one
library call (``klsample_lmhead_run``) that computes the logits chunk by chunk with bf16
matrix cores and runs the sampler's streaming pass on each chunk while it is still on
chip; the logits are written out as well (fp32 holding the bf16-rounded values) for the
rows and options that re-read them.
"""
from __future__ import annotations

import torch

from . import _lib
from .runner import BatchOutput, pack_rows, runner_for


def lmhead_sample(hidden: torch.Tensor, weight: torch.Tensor, params_list, histories=None, uniforms=None,
                  num_logprobs: int | None = None, *, want_info: bool = False):
    """Sample one token per row of ``hidden @ weight.T``.

    ``hidden`` is ``[B, d]`` bf16 and ``weight`` ``[V, d]`` bf16 (``lm_head.weight``),
    both contiguous on one GPU, ``d`` a multiple of 64.  Rows take ``params_list``,
    ``histories`` and ``uniforms`` as in ``sample_batch``.  Returns the batch output and
    the ``[B, V]`` fp32 logits (bf16-rounded values)."""
    if hidden.dim() != 2 or weight.dim() != 2 or hidden.shape[1] != weight.shape[1]:
        raise ValueError('hidden must be [batch, dim] and weight [vocab, dim]')
    if hidden.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise ValueError('hidden and weight must be bfloat16')
    if not hidden.is_cuda or hidden.device != weight.device:
        raise ValueError('hidden and weight must be on one GPU')
    hidden, weight = hidden.contiguous(), weight.contiguous()
    B, d = hidden.shape
    V = weight.shape[0]
    if len(params_list) != B:
        raise ValueError('one SamplingParams per row is required')
    if uniforms is None:
        if any(p.temperature != 0 for p in params_list):
            raise ValueError('uniforms are required for sampled rows')
        uniforms = [0.0] * B
    N = min(max((p.logprobs for p in params_list), default=0) if num_logprobs is None else num_logprobs,
            _lib.MAX_LOGPROBS)
    rows, offsets, ids, max_top_k = pack_rows(params_list, histories, uniforms, V)
    logits = torch.empty((B, V), dtype=torch.float32, device=hidden.device)
    head = _lib.LMHead(hidden.data_ptr(), weight.data_ptr(), d, 0)
    tokens, logprobs, top_ids, top_lp, info, _ = runner_for(hidden.device).run_packed(
        logits, rows, max_top_k, N, offsets=offsets if ids.size else None, ids=ids if ids.size else None,
        want_info=want_info, head=head)
    out = BatchOutput(tokens.copy(), logprobs.copy(), top_ids.copy(), top_lp.copy(),
                      info.copy() if info is not None else None, None, V)
    return out, logits
