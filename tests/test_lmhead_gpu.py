"""The LM head fused with the sampling call (klsample_lmhead_run), on the GPU.

* The materialised logits against the exact product ``hidden @ weight.T`` (float64 on
  the CPU), as the reference's bf16 ``lm_head`` output (serving/qwen_executor.py:238):
  within half a bf16 step plus the fp32 accumulation bound ``d·2^-24·Σ|h_k·w_k|`` of the
  exact value, bf16 values, and equal to the exact value rounded to bf16 almost
  everywhere.
* The sampled rows against the oracle on those same logits, to the parity bar of the
  plain sampling call (tokens exact, logprobs within 1e-5, kept sets equal).
* The same rows through klsample_run on the materialised logits: identical tokens.
"""
import sys

import numpy as np
import pytest
import torch

from helpers import compare
from klsample import SamplingParams
from klsample.lmhead import lmhead_sample
from klsample.runner import runner_for
from oracle.cpu_sampler import sample_rows

pytestmark = pytest.mark.gpu

DEV = torch.device('cuda', 0)


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _params(B, V, seed, greedy_only=False):
    rng = np.random.default_rng(seed)
    kinds = [
        lambda: SamplingParams(logprobs=5),
        lambda: SamplingParams(temperature=0.8, top_k=50, seed=1, logprobs=5),
        lambda: SamplingParams(temperature=1.0, top_p=0.9, seed=2, logprobs=3),
        lambda: SamplingParams(temperature=0.7, top_k=40, top_p=0.95, repetition_penalty=1.2,
                               presence_penalty=0.3, frequency_penalty=0.2, seed=3, logprobs=2),
        lambda: SamplingParams(temperature=1.0, seed=4),
        lambda: SamplingParams(repetition_penalty=1.3, logprobs=1),
    ]
    params = [kinds[0]() if greedy_only else kinds[b % len(kinds)]() for b in range(B)]
    hist = [rng.integers(0, V, int(rng.integers(0, 300))).tolist() for _ in range(B)]
    uni = rng.random(B).astype(np.float32)
    return params, hist, uni


def _bf16_step(x: torch.Tensor) -> torch.Tensor:
    """The spacing of bf16 values at |x| (float64)."""
    return torch.ldexp(torch.ones_like(x), torch.frexp(x.abs().clamp_min(1e-30))[1] - 8)


@pytest.mark.parametrize('B,V,d,seed,greedy_only', [
    (1, 151936, 1024, 0, False),
    (3, 151936, 1024, 1, True),
    (6, 5003, 256, 2, False),
    (20, 32000, 512, 3, False),
])
def test_fused_lm_head_matches_the_product_and_the_oracle(B, V, d, seed, greedy_only):
    say(f'lmhead B={B} V={V} d={d} greedy_only={greedy_only}')
    g = torch.Generator().manual_seed(100 + seed)
    hidden = torch.randn(B, d, generator=g).bfloat16()
    weight = (torch.randn(V, d, generator=g) * (3.0 / d ** 0.5)).bfloat16()
    params, hist, uni = _params(B, V, seed, greedy_only)
    out, logits = lmhead_sample(hidden.to(DEV), weight.to(DEV), params, hist, uni, want_info=True)
    torch.cuda.synchronize()
    got = logits.cpu()
    exact = hidden.double() @ weight.double().T
    bound = d * 2.0 ** -24 * (hidden.double().abs() @ weight.double().abs().T)
    err = (got.double() - exact).abs()
    allowed = 0.5 * _bf16_step(torch.maximum(got.double().abs(), exact.abs() + bound)) + bound
    assert (err <= allowed).all(), f'worst excess {(err - allowed).max().item():.3g}'
    differ = (got != exact.to(torch.bfloat16).float()).double().mean().item()
    say(f'  logits differing from the exact value rounded to bf16: {differ:.2e}')
    assert differ < 1e-2
    assert torch.equal(got, got.bfloat16().float())           # bf16 values, as the reference's output
    rows = sample_rows(got, hist, params, uni)
    rep = compare(out, rows, params, tol=1e-5)
    say('  ' + ' '.join(f'{k}={v}' for k, v in rep.counts().items()))
    assert rep.ok(), '\n'.join(rep.failures[:20])
    plain = runner_for(DEV).run(logits, params, hist, uni, max(p.logprobs for p in params))
    assert np.array_equal(plain.tokens, out.tokens)


def test_fused_lm_head_argument_errors():
    h = torch.zeros(2, 48, dtype=torch.bfloat16, device=DEV)     # dim not a multiple of 64
    w = torch.zeros(100, 48, dtype=torch.bfloat16, device=DEV)
    from klsample._lib import KLSampleError
    with pytest.raises((ValueError, KLSampleError)):
        lmhead_sample(h, w, [SamplingParams()] * 2)
    with pytest.raises(ValueError):
        lmhead_sample(h.float(), w, [SamplingParams()] * 2)
