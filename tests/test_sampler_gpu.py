"""The drop-in ``Sampler`` API on the GPU (MI355X only)."""
import asyncio

import numpy as np
import pytest
import torch

from klsample import SampleResult, Sampler, SamplingParams, sample_batch
from oracle.cpu_sampler import restated_sample

pytestmark = pytest.mark.gpu


def test_reference_known_answer_through_the_drop_in():
    # serving/test_serving.py:101-107, unchanged
    params = SamplingParams(temperature=.8, top_k=3, top_p=.9, repetition_penalty=1.1,
                            stop_token_ids=frozenset({2}), seed=7, logprobs=2)
    logits = torch.tensor([0., 1., 3., 2.])
    a = Sampler(params).sample(logits, [2])
    b = Sampler(params).sample(logits, [2])
    assert a == b and len(a.top_logprobs) == 2
    assert a.token_id in (2, 3)
    assert dict(a.top_logprobs)[2] == pytest.approx(-0.33853459, abs=1e-5)
    assert dict(a.top_logprobs)[3] == pytest.approx(-1.24762559, abs=1e-5)
    greedy = Sampler(SamplingParams(stop_token_ids=frozenset({2}))).sample(logits)
    assert greedy.token_id == 2 and greedy.stopped


def test_sampler_matches_oracle_with_its_own_uniform():
    rng = np.random.default_rng(0)
    x = torch.from_numpy((rng.standard_normal(151936) * 2).astype(np.float32))
    params = SamplingParams(temperature=0.8, top_k=50, top_p=0.9, seed=123, logprobs=3)
    s = Sampler(params)
    gen = torch.Generator().manual_seed(123)
    for step in range(5):
        u = float(torch.rand((), generator=gen))
        want = restated_sample(x, [], params, u=u, stable=True)
        got = s.sample(x.cuda())
        assert got.token_id == want.token_id or want.boundary
        assert isinstance(got, SampleResult)


def test_batching_does_not_change_a_requests_tokens():
    rng = np.random.default_rng(1)
    x = torch.from_numpy((rng.standard_normal((6, 32000)) * 2).astype(np.float32)).cuda()
    params = [SamplingParams(temperature=0.9, top_k=40, top_p=0.95, seed=i, logprobs=2) for i in range(5)]
    params.append(SamplingParams(repetition_penalty=1.2, logprobs=2))
    hist = [rng.integers(0, 32000, 30).tolist() for _ in range(6)]
    single = [Sampler(p) for p in params]
    batched = [Sampler(p) for p in params]
    for step in range(3):
        one = [s.sample(x[i], hist[i]) for i, s in enumerate(single)]
        many = Sampler.sample_many(batched, x, hist)
        assert one == many


def test_entry_points_mix_inside_and_outside_inference_mode():
    """Sampler.sample runs under inference mode and makes the staging buffers there;
    sample_batch called afterwards outside inference mode reuses them."""
    x = torch.randn(2, 1000).cuda()
    a = Sampler(SamplingParams()).sample(x[0])
    res = sample_batch(x, [SamplingParams(), SamplingParams()])
    assert [r.token_id for r in res] == x.argmax(1).tolist() and a.token_id == res[0].token_id


def test_sample_batch_requires_uniforms_for_sampled_rows():
    x = torch.randn(2, 100).cuda()
    with pytest.raises(ValueError):
        sample_batch(x, [SamplingParams(temperature=1.0), SamplingParams()])
    res = sample_batch(x, [SamplingParams(), SamplingParams()])
    assert [r.token_id for r in res] == x.argmax(1).tolist()


def test_history_errors_mirror_indexing():
    s = Sampler(SamplingParams(repetition_penalty=1.2))
    with pytest.raises(IndexError):
        s.sample(torch.zeros(10), [10])
    # id -1 is the last token: with r=1.2 its score 9 becomes 7.5, below token 8
    assert s.sample(torch.arange(10.), [-1]).token_id == 8


class _FakeExecutor:
    """Returns constant host logits per request, like serving/test_serving.py:120-126."""

    async def decode(self, rids):
        await asyncio.sleep(0)
        return {r: torch.tensor([0., 1., 3., 2.]) for r in rids}


def test_engine_style_loop_runs_unchanged():
    """The per-row call pattern of serving/engine.py:92-96 and :105-107 with one
    Sampler per request created at submit time (serving/engine.py:53)."""
    async def main():
        samplers = {f'r{i}': Sampler(SamplingParams(stop_token_ids=frozenset({2}))) for i in range(3)}
        prompts = {r: (5, 6, 7) for r in samplers}
        generated = {r: [] for r in samplers}
        first = {r: samplers[r].sample(torch.tensor([0., 1., 3., 2.]), prompts[r]) for r in samplers}
        for r, res in first.items():
            generated[r].append(res.token_id)
        logits = await _FakeExecutor().decode(list(samplers))
        for r in samplers:
            res = samplers[r].sample(logits[r], prompts[r] + tuple(generated[r]))
            generated[r].append(res.token_id)
            assert res.stopped
        return generated
    assert asyncio.run(main()) == {f'r{i}': [2, 2] for i in range(3)}


def test_integration_ctypes_stub_matches_the_drop_in():
    """The raw ctypes binding printed in the repository's integration guide runs as
    written and returns the drop-in's tokens and logprobs."""
    import re
    from pathlib import Path

    from klsample import _lib, workloads
    from klsample.runner import runner_for

    root = Path(__file__).resolve().parents[1]
    blocks = re.findall(r'```python\n(.*?)```', (root / 'INTEGRATION.md').read_text(), re.S)
    stub = next(b for b in blocks if 'klsample_run' in b)
    stub = stub.replace('/path/to/repo/gpu-kernel-lab_amd/klsample/libklsample.so', str(_lib.LIBRARY))
    ns = {}
    exec(compile(stub, '<integration stub>', 'exec'), ns)
    w = workloads.make('cpu_reference_b8', num_logprobs=3)
    hist = [[5, 9, -1]] * w.batch
    params = [SamplingParams(p.temperature, p.top_k, p.top_p, 1.2, p.stop_token_ids, p.seed, 3) for p in w.params]
    logits = w.logits.cuda()
    tok, lp, top_ids, top_lp = ns['sample_rows'](logits, params, hist, w.uniforms, 3)
    want = runner_for(logits.device).run(logits, params, hist, w.uniforms, 3)
    assert np.array_equal(tok.numpy(), want.tokens)
    assert np.array_equal(lp.numpy(), want.logprobs)
    assert np.array_equal(top_ids.numpy(), want.top_ids)


@pytest.mark.parametrize('name', ['cpu_reference_b8', 'latency_b1', 'mixed_b64'])
def test_workload_digests_on_the_gpu_host(name):
    """The workloads generate the same bytes here as where the digests were committed."""
    import json
    from pathlib import Path
    from klsample import workloads
    want = json.loads((Path(__file__).resolve().parent / 'golden' / 'workload_digests.json').read_text())[name]
    assert workloads.digest(workloads.make(name)) == want


def test_out_of_range_history_ids_are_reported_through_the_c_abi():
    """Ids outside [0, V) that reach the C ABI are ignored and counted per penalised row in
    history_errors; the tokens equal those of the same call without them."""
    import ctypes
    from klsample import _lib
    from klsample.runner import pack_rows

    lib = _lib.load()
    dev = torch.device('cuda', 0)
    V = 5000
    rng = np.random.default_rng(3)
    logits = torch.from_numpy((rng.standard_normal((3, V)) * 2).astype(np.float32)).to(dev)
    params = [SamplingParams(repetition_penalty=1.5), SamplingParams(temperature=0.8, top_k=20),
              SamplingParams(temperature=0.9, repetition_penalty=1.3, frequency_penalty=0.4)]
    good = [[1, 2, 7, 7], [4], [10, 11]]
    bad = [[1, -5, 2, V, 7, 7, V + 100], [9999], [10, 11]]   # row 1 is not penalised
    u = np.float32([0.0, 0.4, 0.7])

    def call(hist):
        rows, _, _, max_top_k = pack_rows(params, good, u, V)   # flags and floats only
        ids = np.concatenate([np.asarray(h, np.int32) for h in hist])
        offs = np.cumsum([0] + [len(h) for h in hist]).astype(np.int32)
        d_rows = torch.from_numpy(rows.view(np.uint8).copy()).to(dev)
        d_ids = torch.from_numpy(ids).to(dev)
        d_off = torch.from_numpy(offs).to(dev)
        tok = torch.empty(3, dtype=torch.int64, device=dev)
        lp = torch.empty(3, dtype=torch.float32, device=dev)
        errs = torch.full((3,), 77, dtype=torch.int32, device=dev)
        ws_bytes = _lib.workspace_size(3, V, _lib.FLOAT32, max_top_k, 0)
        ws = torch.empty(ws_bytes + 256, dtype=torch.uint8, device=dev)
        b = _lib.Batch()
        b.logits, b.row_stride, b.dtype, b.batch, b.vocab = logits.data_ptr(), V, _lib.FLOAT32, 3, V
        b.max_top_k, b.params = max_top_k, d_rows.data_ptr()
        b.history_ids, b.history_offsets = d_ids.data_ptr(), d_off.data_ptr()
        b.token_ids, b.logprobs = tok.data_ptr(), lp.data_ptr()
        b.workspace = ws.data_ptr() + (-ws.data_ptr()) % 256
        b.workspace_bytes = ws_bytes
        b.history_errors = errs.data_ptr()
        _lib.check(lib, lib.klsample_run(ctypes.byref(b), None))
        torch.cuda.synchronize()
        return tok.cpu().numpy(), lp.cpu().numpy(), errs.cpu().numpy()

    t_good, lp_good, e_good = call(good)
    t_bad, lp_bad, e_bad = call(bad)
    assert e_good.tolist() == [0, 0, 0]
    assert e_bad.tolist() == [3, 0, 0]
    assert np.array_equal(t_good, t_bad) and np.array_equal(lp_good, lp_bad)
