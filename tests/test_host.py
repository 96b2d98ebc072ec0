"""Host-side logic of the drop-in API (CPU only)."""
import hashlib
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from klsample import SampleResult, Sampler, SamplingParams, _lib, workloads
from klsample.runner import normalize_history, pack_rows


def test_params_validation_matches_reference():
    # serving/sampling.py:17-21
    for bad in (dict(temperature=-0.1), dict(temperature=float('inf')), dict(top_k=-1), dict(top_p=0.0),
                dict(top_p=1.01), dict(repetition_penalty=0.0), dict(repetition_penalty=float('nan')),
                dict(logprobs=-1)):
        with pytest.raises(ValueError):
            SamplingParams(**bad)
    SamplingParams(temperature=0.0, top_k=0, top_p=1.0, repetition_penalty=1.0, logprobs=20)


def test_params_additions():
    with pytest.raises(ValueError):
        SamplingParams(presence_penalty=float('inf'))
    with pytest.raises(ValueError):
        SamplingParams(frequency_penalty=float('nan'))
    with pytest.raises(ValueError):
        SamplingParams(logprobs=_lib.MAX_LOGPROBS + 1)


def test_params_positional_order_is_the_references():
    # serving/api.py:50-51 builds the params positionally
    p = SamplingParams(0.7, 40, 0.9, 1.1, frozenset({3}), 5, 2)
    assert (p.temperature, p.top_k, p.top_p, p.repetition_penalty, p.stop_token_ids, p.seed, p.logprobs) == \
        (0.7, 40, 0.9, 1.1, frozenset({3}), 5, 2)
    assert p.presence_penalty == 0.0 and p.frequency_penalty == 0.0
    with pytest.raises(Exception):
        p.temperature = 1.0  # frozen


def test_result_type():
    r = SampleResult(1, -0.5, ((1, -0.5),), False)
    assert r == SampleResult(1, -0.5, ((1, -0.5),), False)


def test_pack_rows_flags_and_fp32_values():
    params = [SamplingParams(), SamplingParams(0.7, 40, 0.95, 1.1, presence_penalty=0.5),
              SamplingParams(1.0, 0, 0.99999999, 1.0, frequency_penalty=0.3)]
    rows, offsets, ids, max_top_k = pack_rows(params, [[1, 2], [3, -1, 3], [9]], [0.1, 0.2, 0.3], 10)
    assert rows['flags'].tolist() == [_lib.ROW_GREEDY,
                                      _lib.ROW_REPETITION | _lib.ROW_PRESENCE_FREQUENCY | _lib.ROW_TOP_P,
                                      _lib.ROW_PRESENCE_FREQUENCY | _lib.ROW_TOP_P]
    # fp32 rounds 0.99999999 to 1.0, the flag still says top-p applies (p < 1 in double)
    assert rows['top_p'][2] == np.float32(1.0)
    assert rows['temperature'][1] == np.float32(0.7) and rows['repetition_penalty'][1] == np.float32(1.1)
    assert rows['uniform'].tolist() == [0.0, np.float32(0.2), np.float32(0.3)]
    # history only for rows with a penalty; negative ids wrap
    assert offsets.tolist() == [0, 0, 3, 4] and ids.tolist() == [3, 9, 3, 9]
    assert max_top_k == 10  # min(top_k, vocab)


def test_history_is_ignored_without_penalties_like_the_reference():
    # the reference indexes history only when repetition_penalty != 1 (serving/sampling.py:47)
    rows, offsets, ids, _ = pack_rows([SamplingParams()], [[10**9]], None, 10)
    assert offsets.tolist() == [0, 0] and ids.size == 0
    with pytest.raises(IndexError):
        pack_rows([SamplingParams(repetition_penalty=1.2)], [[10]], None, 10)


def test_normalize_history():
    assert normalize_history([-1, 0, 9], 10).tolist() == [9, 0, 9]
    with pytest.raises(IndexError):
        normalize_history([-11], 10)


def test_sampler_fails_loudly_without_a_gpu():
    if torch.cuda.is_available():
        pytest.skip('a GPU is visible')
    s = Sampler(SamplingParams())
    with pytest.raises(RuntimeError):
        s.sample(torch.tensor([0., 1., 3., 2.]))


def test_sampler_rejects_bad_logits():
    s = Sampler(SamplingParams())
    with pytest.raises(ValueError):
        s.sample(torch.zeros(2, 2))
    with pytest.raises(ValueError):
        s.sample(torch.tensor([1, 2, 3]))


def test_sample_many_rejects_row_count_mismatches_before_drawing():
    """A padded [B, V] decode batch with fewer samplers (or histories) than rows is an
    error, raised before any uniform is drawn or any launch is made."""
    s = [Sampler(SamplingParams(temperature=1.0, seed=5)) for _ in range(2)]
    with pytest.raises(ValueError):
        Sampler.sample_many(s, torch.zeros(3, 10), [(), ()])
    with pytest.raises(ValueError):
        Sampler.sample_many(s, torch.zeros(2, 10), [(), (), ()])
    with pytest.raises(ValueError):
        Sampler.sample_many(s, [torch.zeros(10)], [()])
    fresh = Sampler(SamplingParams(temperature=1.0, seed=5))
    assert s[0].next_uniform('cpu') == fresh.next_uniform('cpu')   # no uniform was consumed


def test_device_runner_checks_rows_before_staging():
    from klsample.runner import DeviceRunner
    r = DeviceRunner.__new__(DeviceRunner)   # no device needed: the checks come first
    x = torch.zeros(3, 10)
    with pytest.raises(ValueError):
        r.run(x, [SamplingParams()] * 2, None, None, 0)
    with pytest.raises(ValueError):
        r.run(x, [SamplingParams()] * 3, [()] * 2, None, 0)
    with pytest.raises(ValueError):
        r.run(x, [SamplingParams()] * 3, None, [0.5] * 4, 0)


def test_uniform_stream_is_per_request_and_seeded():
    a, b = Sampler(SamplingParams(temperature=1.0, seed=3)), Sampler(SamplingParams(temperature=1.0, seed=3))
    ua = [a.next_uniform('cpu') for _ in range(4)]
    assert ua == [b.next_uniform('cpu') for _ in range(4)]
    assert len(set(ua)) == 4 and all(0 <= u < 1 for u in ua)
    c = Sampler(SamplingParams(temperature=1.0, seed=4))
    assert c.next_uniform('cpu') != ua[0]


def test_uniforms_served_from_blocks_equal_single_draws():
    """Sampler.next_uniform draws 64 at a time; the values it hands out, across block
    boundaries, are the ones single draws of a generator with the request's seed give."""
    s = Sampler(SamplingParams(temperature=1.0, seed=77))
    g = torch.Generator().manual_seed(77)
    got = [s.next_uniform('cpu') for _ in range(150)]
    want = [float(torch.rand((), generator=g)) for _ in range(150)]
    assert got == want
    # a second device key has a stream of its own, from the same seed
    assert s.next_uniform('cuda:0') == want[0]


def _digest(t: torch.Tensor) -> str:
    return hashlib.sha256(t.contiguous().view(torch.uint8).numpy().tobytes()).hexdigest()[:16]


@pytest.mark.parametrize('name,shape,dtype', [
    ('cpu_reference_b8', (8, 151936), torch.float32),
    ('latency_b1', (1, 151936), torch.bfloat16),
    ('mixed_b64', (64, 151936), torch.bfloat16),
])
def test_workloads_are_deterministic(name, shape, dtype):
    a = workloads.make(name)
    b = workloads.make(name)
    assert tuple(a.logits.shape) == shape and a.logits.dtype == dtype
    assert _digest(a.logits) == _digest(b.logits)
    assert np.array_equal(a.uniforms, b.uniforms)
    assert all(np.array_equal(x, y) for x, y in zip(a.histories, b.histories))
    assert a.algorithmic_bytes() == a.batch * a.vocab * a.logits.element_size() + 4 * a.history_tokens + 48 * a.batch


def test_workload_shapes_of_documented_configs():
    w = workloads.make('mixed_b64')
    assert {p.top_k for p in w.params} <= {0, 20, 50, 1000}
    assert all(0.5 <= p.temperature <= 1.5 and 0.8 <= p.top_p <= 1.0 for p in w.params)
    assert all(len(h) == 512 for h in w.histories)
    w1 = workloads.make('latency_b1')
    x = w1.logits.float()[0]
    assert float(x.max()) > 14  # the +8 heavy head tops the 3*N(0,1) bulk (max ~13)
    assert workloads.make('cpu_reference_b8', batch=3).batch == 3


DIGESTS = Path(__file__).resolve().parent / 'golden' / 'workload_digests.json'


@pytest.mark.parametrize('name', workloads.NAMES)
def test_workloads_match_the_committed_digests(name):
    """Every workload regenerates to the bytes whose SHA-256 is committed
    (tests/golden/make_workload_digests.py); the GPU tests repeat this on the GPU host."""
    want = json.loads(DIGESTS.read_text())[name]
    assert workloads.digest(workloads.make(name)) == want


def test_uniforms_taken_in_blocks_and_returned_keep_the_stream():
    """A batched step takes a request's pending uniforms and hands back what it did not
    use: the request's stream of uniforms is unchanged by that."""
    s = Sampler(SamplingParams(temperature=1.0, seed=5))
    g = torch.Generator().manual_seed(5)
    want = [float(torch.rand((), generator=g)) for _ in range(200)]
    got = [s.next_uniform('cpu') for _ in range(3)]
    blk = s.take_uniforms('cpu')
    assert blk.dtype == np.float32 and blk.size == 61
    got += blk[:10].tolist()
    s.return_uniforms('cpu', blk[10:])
    got += [s.next_uniform('cpu') for _ in range(60)]
    blk = s.take_uniforms('cpu')          # the rest of the block the draws above started
    got += blk.tolist()
    got += [s.next_uniform('cpu') for _ in range(10)]
    assert got == want[:len(got)]


def test_smoke_report_reads_the_parity_report():
    """smoke() prints its line from the same report the GPU tests build; a failing report
    raises."""
    import __graft_entry__ as entry
    from helpers import ParityReport
    rep = ParityReport(rows=2, greedy=1, sampled=1, exact=2)
    line = entry.smoke_report(np.array([3, 4]), rep)
    assert line.startswith('smoke ok: tokens=[3, 4]') and "'exact': 2" in line
    rep.failures.append('row 0: token 1 != oracle 2')
    with pytest.raises(AssertionError):
        entry.smoke_report(np.array([1]), rep)
