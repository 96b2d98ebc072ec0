"""The engine-shaped step (klsample.engine) on the GPU: per-step tokens against the
per-row drop-in and the oracle, device histories, the FAILED path and the SSE wire format.
"""
import json

import numpy as np
import pytest
import torch

from klsample import Sampler, SamplingParams, _lib
from klsample import engine as eng
from oracle.cpu_sampler import restated_sample

pytestmark = pytest.mark.gpu

DEV = 'cuda:0'


def _params(V):
    return [
        SamplingParams(temperature=0.8, top_k=40, top_p=0.9, repetition_penalty=1.1, seed=1, logprobs=3),
        SamplingParams(repetition_penalty=1.3, logprobs=2),                                  # greedy
        SamplingParams(temperature=1.0, top_p=0.8, seed=2, logprobs=5),                      # top-p only
        SamplingParams(temperature=0.7, seed=3),                                             # full row
        SamplingParams(temperature=1.2, top_k=1, seed=4, logprobs=1),
        SamplingParams(temperature=0.9, top_k=V + 5, top_p=0.95, repetition_penalty=0.9,
                       presence_penalty=0.4, frequency_penalty=0.2, seed=5, logprobs=4),
    ]


def _check_row(got, row, history, params, u, what):
    """One engine row against a fresh per-row Sampler result and the oracle."""
    want = restated_sample(row.cpu(), history, params, u=u, stable=True)
    if got.token_id != want.token_id:
        assert want.boundary, f'{what}: token {got.token_id} != oracle {want.token_id}'
        assert want.in_kept(got.token_id)
        return
    if want.margin_row:
        return      # the reference's fp32 cut may sit one entry away: its normaliser differs by design
    assert abs(got.logprob - want.logprob) <= 1e-5 * max(1.0, abs(want.logprob)) + want.lse_error, what
    assert [i for i, _ in got.top_logprobs] == [i for i, _ in want.top_logprobs], what
    for (_, a), (_, b) in zip(got.top_logprobs, want.top_logprobs):
        assert abs(a - b) <= 1e-5 * max(1.0, abs(b)) + want.lse_error, what


@pytest.mark.parametrize('dtype', [torch.float32, torch.bfloat16])
def test_engine_steps_equal_per_row_sampler_and_oracle(dtype):
    """Prefill then decode steps of six requests (one call per step): every row equals a
    per-row Sampler.sample with history prompt + generated, and the oracle with the
    request's own uniform; the device history after each step is prompt + generated.
    A two-slot reserve and a 1024-id arena make segments move and the arena grow."""
    V = 32000
    rng = np.random.default_rng(7)
    params = _params(V)
    rids = [f'r{i}' for i in range(len(params))]
    prompts = {r: rng.integers(0, V, int(n)).tolist() for r, n in zip(rids, [0, 5, 300, 17, 1, 900])}
    max_tokens = dict(zip(rids, [8, 3, 8, 5, 8, 8]))
    loop = eng.SamplingLoop(DEV, V, capacity=1024, reserve=2)
    for r, p in zip(rids, params):
        loop.submit(r, p, prompts[r], max_tokens[r])
    single = {r: Sampler(p, device=DEV) for r, p in zip(rids, params)}
    uniforms = {r: Sampler(p, device=DEV) for r, p in zip(rids, params)}
    step = 0
    active = list(rids)
    while active:
        x = torch.from_numpy((rng.standard_normal((len(active), V)) * 3).astype(np.float32)).to(DEV, dtype)
        x[0, :8] = x[0, :8].max()       # a value tie at the top of one row
        phase = 'prefill' if step == 0 else 'decode'
        hist = {r: prompts[r] + loop.generated[r] for r in active}
        if phase == 'prefill':
            # the executor's per-request dict of rows of one tensor, used in place
            loop.step(prefill_rids=active, prefill_logits={r: x[i] for i, r in enumerate(active)})
        else:
            loop.step(decode_rids=active, decode_logits=x)
        for i, r in enumerate(active):
            ev = [e for e in loop.events[r] if not e.finished][-1]
            got = eng.SampleResult(ev.token_id, ev.logprob, ev.top_logprobs, ev.token_id in params[rids.index(r)].stop_token_ids)
            assert got == single[r].sample(x[i], hist[r]), f'step {step} {r}'
            p = params[rids.index(r)]
            u = uniforms[r].next_uniform(DEV) if p.temperature != 0 else 0.0
            _check_row(got, x[i], hist[r], p, u, f'step {step} {r}')
        for r in active:
            if loop.state[r] == 'decode':
                assert loop.history.ids(r).tolist() == prompts[r] + loop.generated[r]
        active = [r for r in active if loop.state[r] == 'decode']
        step += 1
    for r in rids:
        assert loop.state[r] == 'finished' and len(loop.generated[r]) == max_tokens[r]
        assert loop.events[r][-1].finish_reason == 'length'
    assert loop.history.arena.numel() > 1024


def test_engine_history_of_4096_tokens():
    """Long device histories (4096 ids per row, penalties on) through history ranges:
    tokens equal the per-row Sampler's and the oracle's; the arena holds prompt +
    generated after three steps."""
    V = 151936
    rng = np.random.default_rng(11)
    params = [SamplingParams(temperature=1.0, top_k=40, top_p=0.9, repetition_penalty=1.1, presence_penalty=0.5,
                             frequency_penalty=0.3, seed=20 + i, logprobs=2) for i in range(3)]
    params.append(SamplingParams(repetition_penalty=1.2))
    rids = list(range(4))
    prompts = {r: rng.integers(0, V, 4096).tolist() for r in rids}
    loop = eng.SamplingLoop(DEV, V)
    for r, p in zip(rids, params):
        loop.submit(r, p, prompts[r], 10)
    single = {r: Sampler(p, device=DEV) for r, p in zip(rids, params)}
    uni = {r: Sampler(p, device=DEV) for r, p in zip(rids, params)}
    for step in range(3):
        x = torch.from_numpy((rng.standard_normal((4, V)) * 2).astype(np.float32)).to(DEV)
        hist = {r: prompts[r] + loop.generated[r] for r in rids}
        if step == 0:
            loop.step(prefill_rids=rids, prefill_logits=x)
        else:
            loop.step(decode_rids=rids, decode_logits=x)
        for r in rids:
            ev = loop.events[r][-1]
            got = eng.SampleResult(ev.token_id, ev.logprob, ev.top_logprobs, False)
            assert got == single[r].sample(x[r], hist[r])
            u = uni[r].next_uniform(DEV) if params[r].temperature != 0 else 0.0
            _check_row(got, x[r], hist[r], params[r], u, f'step {step} row {r}')
            assert loop.history.ids(r).tolist() == hist[r] + [ev.token_id]


def test_a_failing_call_fails_every_request_of_the_step(monkeypatch):
    """A library error (here: a workspace smaller than the call needs, status -3, found
    before any launch) is a KLSampleError; as in serving/engine.py:109-115 every
    unfinished request of the step then gets one finished event with reason 'error'.
    Requests outside the step carry on."""
    V = 151936
    rng = np.random.default_rng(3)
    loop = eng.SamplingLoop(DEV, V)
    p = SamplingParams(temperature=1.0, top_p=0.9, seed=9)
    for r in ('a', 'b', 'c'):
        loop.submit(r, p, rng.integers(0, V, 10).tolist(), 4)
    need = _lib.workspace_size(2, V, _lib.FLOAT32, 0, 0)
    assert need > (1 << 20)     # the 1 MiB workspace allocated below is too small
    real = eng._lib.workspace_size
    monkeypatch.setattr(eng._lib, 'workspace_size', lambda *a: 256)
    x = torch.randn(2, V, device=DEV)
    loop.step(prefill_rids=['a', 'b'], prefill_logits=x)
    for r in ('a', 'b'):
        assert loop.state[r] == 'failed'
        (ev,) = loop.events[r]
        assert ev.finished and ev.finish_reason == 'error' and 'workspace' in ev.error
        assert r not in loop.history.slot
    monkeypatch.setattr(eng._lib, 'workspace_size', real)
    ref = Sampler(p, device=DEV)
    y = torch.randn(1, V, device=DEV)
    loop.step(prefill_rids=['c'], prefill_logits=y)
    assert loop.state['c'] == 'decode'
    assert loop.events['c'][-1].token_id == ref.sample(y[0], loop.history.ids('c')[:-1].tolist()).token_id


def test_sse_lines_carry_the_oracle_top_logprobs():
    """The SSE lines of a request (serving/api.py:58-70) parse as JSON and their
    ``top_logprobs`` pairs are the oracle's: ids best first, equal logprobs in ascending
    id order, values within 1e-5; the stream ends with the finish chunk and [DONE]."""
    V = 5000
    rng = np.random.default_rng(5)
    p = SamplingParams(temperature=0.9, top_k=50, seed=13, logprobs=6, stop_token_ids=frozenset({V + 1}))
    loop = eng.SamplingLoop(DEV, V)
    loop.submit('cmpl-1', p, [3, 4, 5], 3)
    uni = Sampler(p, device=DEV)
    rows, hists = [], []
    for step in range(3):
        x = torch.from_numpy((rng.standard_normal((1, V)) * 2).astype(np.float32))
        x[0, [40, 7, 900, 12]] = 9.0                     # four equal maxima
        hists.append([3, 4, 5] + loop.generated['cmpl-1'])
        xd = x.to(DEV)
        if step == 0:
            loop.step(prefill_rids=['cmpl-1'], prefill_logits=xd)
        else:
            loop.step(decode_rids=['cmpl-1'], decode_logits=xd)
        rows.append(x[0])
    lines = [eng.sse_chunk(e, text='t', chat=False) for e in loop.events['cmpl-1']] + [eng.SSE_DONE]
    assert lines[-1] == 'data: [DONE]\n\n' and all(l.startswith('data: ') and l.endswith('\n\n') for l in lines)
    payloads = [json.loads(l[6:]) for l in lines[:-1]]
    assert [q['choices'][0]['finish_reason'] for q in payloads] == [None, None, None, 'length']
    for q, row, h in zip(payloads[:3], rows, hists):
        assert q['id'] == 'cmpl-1' and q['object'] == 'text_completion'
        ch = q['choices'][0]
        want = restated_sample(row, h, p, u=uni.next_uniform(DEV), stable=True)
        got = ch['logprobs']['top_logprobs']
        assert [i for i, _ in got] == [i for i, _ in want.top_logprobs]
        assert [i for i, _ in got][:4] == [7, 12, 40, 900]
        for (_, a), (_, b) in zip(got, want.top_logprobs):
            assert abs(a - b) <= 1e-5 * max(1.0, abs(b))
        assert abs(ch['logprobs']['token_logprob'] - want.logprob) <= 1e-5 * max(1.0, abs(want.logprob))
    chat = json.loads(eng.sse_chunk(loop.events['cmpl-1'][0], text='hi', chat=True)[6:])
    assert chat['object'] == 'chat.completion.chunk' and chat['choices'][0]['delta'] == {'content': 'hi'}
