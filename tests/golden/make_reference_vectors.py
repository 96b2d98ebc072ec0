"""Write ``reference_vectors.json`` by running the reference sampler in the build container.

The reference sampler (``serving/sampling.py``) is loaded from its own file (the
package ``__init__`` is not executed) and called unchanged, except that for the
duration of each sampled call ``torch.multinomial`` is replaced by the inverse-CDF
draw on a supplied uniform (``oracle.cpu_sampler.inverse_cdf`` semantics, restated
here so the vectors do not depend on the oracle they pin).  The replacement also
records the probability vector the reference passes to the draw.

Only inputs and outputs are written.  The reference itself never leaves this
container; the GPU machines read the JSON fixture only.

Usage (build container only)::

    python tests/golden/make_reference_vectors.py [/root/reference]
"""
from __future__ import annotations

import base64
import importlib.util
import json
import math
import sys
from pathlib import Path

import numpy as np
import torch

OUT = Path(__file__).with_name('reference_vectors.json')


def load_reference(root: Path):
    spec = importlib.util.spec_from_file_location('reference_sampling', root / 'serving' / 'sampling.py')
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    return module


def _inverse_cdf(probs, u):
    c = np.cumsum(probs.detach().double().numpy())
    target = float(u) * c[-1]
    i = int(np.searchsorted(c, target, side='right'))
    if i >= c.size:
        i = int(np.flatnonzero(probs.double().numpy() > 0)[-1])
    return i


def run_case(ref, logits, history, params_kw, u):
    params = ref.SamplingParams(**params_kw)
    seen = {}
    real = torch.multinomial

    def fake_multinomial(probs, num_samples, generator=None):
        seen['probs'] = probs.clone()
        return torch.tensor([_inverse_cdf(probs, u)])

    torch.multinomial = fake_multinomial
    try:
        result = ref.Sampler(params).sample(logits, history)
    finally:
        torch.multinomial = real
    probs = seen.get('probs')
    return {
        'token_id': result.token_id,
        'logprob': result.logprob,
        'top_logprobs': [[i, v] for i, v in result.top_logprobs],
        'stopped': result.stopped,
        'probs': probs,
    }


def _f(x):
    """JSON-safe float (``-inf`` kept as a string)."""
    return x if math.isfinite(x) else repr(x)


def _b64(array, dtype):
    """Little-endian array bytes as base64 text."""
    return base64.b64encode(np.ascontiguousarray(array, dtype=dtype).tobytes()).decode('ascii')


def cases():
    rng = np.random.default_rng(20261201)
    out = []

    def add(name, logits, history, u, **kw):
        kw.setdefault('stop_token_ids', frozenset())
        out.append((name, np.asarray(logits, dtype=np.float32), list(history), kw, float(u)))

    # the reference's own known-answer test, serving/test_serving.py:101-107
    kat = [0., 1., 3., 2.]
    for u in (0.0, 0.25, 0.7128, 0.7129, 0.999):
        add(f'kat_u{u}', kat, [2], u, temperature=.8, top_k=3, top_p=.9, repetition_penalty=1.1,
            stop_token_ids=frozenset({2}), seed=7, logprobs=2)
    add('kat_greedy', kat, [], 0.5, stop_token_ids=frozenset({2}))
    # greedy ties resolve to the lowest index
    add('greedy_tie', [1., 5., 2., 5., 5.], [], 0.5, logprobs=3)
    add('greedy_penalised', [-3., 2., 4., -1., 4.1], [4, 4, 0], 0.5, repetition_penalty=1.3, logprobs=2)
    # negative scores are multiplied by the penalty, positive ones divided, zero stays
    add('repetition_signs', [-2., 0., 2., 1.5, -0.5, 3.], [0, 1, 2, 2, 5], 0.3,
        temperature=1.0, repetition_penalty=1.7, logprobs=6)
    add('repetition_below_one', [-2., 0.5, 2., 1.5], [0, 2], 0.6, temperature=0.5, repetition_penalty=0.6,
        logprobs=2)
    # top-k keeps every value tied with the k-th largest
    add('topk_ties', [3., 1., 3., 2., 3., 0., 2.], [], 0.8, temperature=1.0, top_k=2, logprobs=5)
    add('topk_over_vocab', [0.1, 0.4, -0.3], [], 0.2, temperature=2.0, top_k=10, logprobs=3)
    add('topk_one', [0.1, 0.4, -0.3, 0.4], [], 0.9, temperature=0.3, top_k=1, logprobs=4)
    # top-p: tiny p keeps only the largest; the crossing token is kept
    add('topp_tiny', [1., 2., 3., 4.], [], 0.99, temperature=1.0, top_p=1e-6, logprobs=2)
    add('topp_half', [1., 2., 3., 4., 0., -1.], [], 0.4, temperature=1.0, top_p=0.5, logprobs=6)
    # -inf logits (masked tokens)
    add('masked', [-math.inf, 1., -math.inf, 2., 0.5], [3], 0.7, temperature=0.7, top_p=0.9,
        repetition_penalty=1.2, logprobs=5)
    # random rows of several sizes and parameter mixes
    specs = [
        (64, dict(temperature=0.8, top_k=50, top_p=0.9)),
        (257, dict(temperature=1.3, top_k=0, top_p=0.95, repetition_penalty=1.1)),
        (1000, dict(temperature=0.7, top_k=20, top_p=1.0, repetition_penalty=1.2)),
        (1000, dict(temperature=1.0, top_k=0, top_p=1.0)),
        (4096, dict(temperature=0.9, top_k=100, top_p=0.95, repetition_penalty=1.2)),
        (4096, dict(temperature=0.0, repetition_penalty=1.1)),
        (4096, dict(temperature=1.5, top_k=1000, top_p=0.85, repetition_penalty=0.9)),
        (2048, dict(temperature=0.5, top_k=0, top_p=0.8)),
    ]
    for n, (v, kw) in enumerate(specs):
        x = (rng.standard_normal(v) * 2.5).astype(np.float32)
        hist = rng.integers(0, v, size=min(64, v)).tolist()
        for u in (float(rng.random()), float(rng.random())):
            add(f'random{n}_v{v}', x, hist, u, logprobs=5, **kw)
    # values on the bf16 grid: many exact ties
    x = torch.from_numpy((rng.standard_normal(3000) * 2).astype(np.float32)).bfloat16().float().numpy()
    for u in (0.1, 0.5, 0.9):
        add('bf16_ties_topk_topp', x, rng.integers(0, 3000, 40).tolist(), u, temperature=0.9, top_k=100,
            top_p=0.95, repetition_penalty=1.2, logprobs=8)
        add('bf16_ties_topp', x, [], u, temperature=0.9, top_p=0.5, logprobs=8)
    add('bf16_ties_greedy', x, rng.integers(0, 3000, 40).tolist(), 0.5, repetition_penalty=1.2, logprobs=8)
    # integer-valued logits: ties straddling the top-p cut
    x = rng.integers(-3, 4, size=200).astype(np.float32)
    for u in (0.05, 0.5, 0.95):
        add('integer_ties_topp', x, [], u, temperature=1.0, top_p=0.6, logprobs=10)
    return out


def main(root='/root/reference'):
    ref = load_reference(Path(root))
    records = []
    for name, logits, history, kw, u in cases():
        got = run_case(ref, torch.from_numpy(logits.copy()), history, kw, u)
        params = {k: (sorted(v) if isinstance(v, frozenset) else v) for k, v in kw.items()}
        probs = got.pop('probs')
        if probs is not None:
            p = probs.numpy()
            nz = np.flatnonzero(p)
            got['probs_nonzero'] = {'index_i32': _b64(nz, '<i4'), 'value_f32': _b64(p[nz], '<f4')}
        else:
            got['probs_nonzero'] = None
        records.append({
            'name': name,
            'vocab': int(logits.size),
            'logits_f32': _b64(logits, '<f4'),
            'history': history,
            'params': params,
            'u': u,
            'expected': {**got,
                         'logprob': _f(got['logprob']),
                         'top_logprobs': [[i, _f(v)] for i, v in got['top_logprobs']]},
        })
    meta = {'generator': 'tests/golden/make_reference_vectors.py',
            'reference_file': 'serving/sampling.py',
            'torch': torch.__version__,
            'draw': 'torch.multinomial replaced by inverse CDF on u (float64 cumsum, first index > u*sum)'}
    OUT.write_text(json.dumps({'meta': meta, 'cases': records}, separators=(',', ':')) + '\n')
    print(f'wrote {len(records)} cases to {OUT} ({OUT.stat().st_size} bytes)')


if __name__ == '__main__':
    main(*sys.argv[1:])
