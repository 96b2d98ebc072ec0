"""Parity of the HIP sampling path with the CPU oracle (MI355X only).

The oracle runs with the stable tie order (equal scores in ascending index order, the
kernels' rule).  Token ids must be bit-exact on every row except boundary rows (top-p
mass or CDF step within 1e-6 of the cut, where the token must still be kept); a value
tie across the top-p cut is no exemption.  Kept sets are equal, logprobs and top-N
values within 1e-5 of the exact (float64) log-softmax, top-N ids equal, and the final
probabilities within 1e-5 relative of the exact softmax.

With ``KLSAMPLE_PARITY_LOG`` set to a path, every comparison appends one JSON line of
its counts (rows, boundary rows, mismatches, largest errors) to that file."""
import json
import math
import os
import sys

import numpy as np
import pytest
import torch

from helpers import close, compare, golden_cases
from klsample import SamplingParams, _lib, workloads
from klsample.runner import runner_for
from oracle.cpu_sampler import restated_sample, sample_rows

pytestmark = pytest.mark.gpu
DEV = torch.device('cuda', 0)
TOL = 1e-5


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def run(logits, params, histories, uniforms, *, options=0, probs=False, n=None):
    n = max((p.logprobs for p in params), default=0) if n is None else n
    say(f'  klsample_run B={logits.shape[0]} V={logits.shape[-1]} dtype={logits.dtype} N={n} options={options}')
    out = runner_for(DEV).run(logits.to(DEV), params, histories, uniforms, n, options=options,
                              want_probs=probs, want_info=True)
    torch.cuda.synchronize()
    return out


def check(out, rows, params, probs=False, label=None):
    rep = compare(out, rows, params, tol=TOL, probs=out.probs.cpu().numpy() if probs else None)
    counts = rep.counts()
    say('  ' + ' '.join(f'{k}={v}' for k, v in counts.items()))
    log = os.environ.get('KLSAMPLE_PARITY_LOG')
    if log:
        with open(log, 'a') as f:
            f.write(json.dumps({'case': label or os.environ.get('PYTEST_CURRENT_TEST', '?').split(' ')[0],
                                'probs': bool(probs), **counts}) + '\n')
    assert rep.ok(), '\n'.join(rep.failures[:20])
    return rep


def _with_logprobs(w, n):
    ps = [SamplingParams(p.temperature, p.top_k, p.top_p, p.repetition_penalty, p.stop_token_ids, p.seed, n,
                         p.presence_penalty, p.frequency_penalty) for p in w.params]
    return workloads.Workload(w.name, w.logits, ps, w.histories, w.uniforms)


# ---- the configured workloads -------------------------------------------------------------

@pytest.mark.parametrize('name,batch,n,probs', [
    ('cpu_reference_b8', None, 0, True),
    ('cpu_reference_b8', None, 5, True),
    ('latency_b1', None, 20, True),
    ('latency_b1_greedy', None, 3, True),
    ('mixed_b64', None, 5, True),
    ('throughput_b256_v128256', None, 0, True),
    ('throughput_b256_v151936', None, 3, True),
    ('tie_stress_b1024', None, 4, True),
])
def test_workload_parity(name, batch, n, probs):
    """Every configured workload at full size, with probabilities: zero tie exemptions."""
    say(f'workload {name} batch={batch} logprobs={n}')
    w = _with_logprobs(workloads.make(name, batch=batch), n)
    rows = sample_rows(w.logits, w.histories, w.params, w.uniforms)
    out = run(w.logits, w.params, w.histories, w.uniforms, probs=probs)
    rep = check(out, rows, w.params, probs=probs, label=f'workload {name} N={n}')
    # ties across the top-p cut are compared like any other row
    assert rep.exact + rep.boundary_mismatches == rep.rows


@pytest.mark.parametrize('name,batch', [
    ('cpu_reference_b8', None),
    ('latency_b1', None),
    ('mixed_b64', 16),
    ('throughput_b256_v151936', 8),
    ('tie_stress_b1024', 16),
])
def test_row_path_parity(name, batch):
    """Every row forced through the multi-pass row path (dense_kernel)."""
    say(f'row path {name} batch={batch}')
    w = _with_logprobs(workloads.make(name, batch=batch), 4)
    rows = sample_rows(w.logits, w.histories, w.params, w.uniforms)
    out = run(w.logits, w.params, w.histories, w.uniforms, options=_lib.OPT_FORCE_DENSE, probs=True)
    assert (out.info['path'] == 1).all()
    check(out, rows, w.params, probs=True)


def test_repeated_calls_are_deterministic():
    say('determinism mixed_b64[:16] x3')
    w = workloads.make('mixed_b64', batch=16)
    outs = [run(w.logits, w.params, w.histories, w.uniforms) for _ in range(3)]
    for o in outs[1:]:
        assert np.array_equal(o.tokens, outs[0].tokens)
        assert np.array_equal(o.logprobs, outs[0].logprobs)


@pytest.mark.parametrize('name,rows', [('cpu_reference_b8', 8), ('mixed_b64', 8), ('mixed_b64', 3),
                                       ('latency_b1', 1), ('latency_b1_greedy', 1), ('tie_stress_b1024', 5)])
def test_inline_parameters_equal_staged_parameters(name, rows):
    """Up to eight rows may hand their parameters and history offsets over in the kernel
    arguments (KLSAMPLE_OPT_HOST_PARAMS) instead of device memory.  Both give identical
    outputs, on either row path; the output buffer is overwritten with garbage before
    every call, so a call that left a row unwritten would show."""
    from klsample.runner import pack_rows
    say(f'inline parameters {name}[:{rows}]')
    w = workloads.make(name, batch=rows, num_logprobs=5)
    logits = w.logits.to(DEV)
    packed, offsets, ids, kmax = pack_rows(w.params, w.histories, w.uniforms, w.vocab)
    r = runner_for(DEV)
    outs = []
    for host, options in ((False, 0), (True, 0), (True, 0), (False, 0),
                          (False, _lib.OPT_FORCE_DENSE), (True, _lib.OPT_FORCE_DENSE)):
        if r.out_host is not None:
            r.out_host.numpy()[:] = 0xA5
        o = r.run_packed(logits, packed, kmax, 5, offsets=offsets if ids.size else None,
                         ids=ids if ids.size else None, options=options, want_info=True, host_params=host)
        outs.append((options, [x.copy() for x in o[:4]], o[4].copy()))
    for options, arrays, info in outs:
        base = next(x for x in outs if x[0] == options)
        for a, b in zip(arrays, base[1]):
            assert np.array_equal(a, b)
        assert info.tobytes() == base[2].tobytes()
    assert (outs[-1][2]['path'] == 1).all()


# ---- vectors written by the reference sampler ----------------------------------------------

CASES = golden_cases()


@pytest.mark.parametrize('case', CASES, ids=[c['name'] for c in CASES])
def test_reference_vectors_on_gpu(case):
    """The GPU against the stable-order oracle (full parity), and against the vectors the
    reference itself wrote.  Where the reference's unstable sort kept other members of a
    tie at the top-p cut, its kept probabilities must still be the GPU's as a multiset."""
    say(f'golden {case["name"]}')
    p = case['params']
    params = SamplingParams(p.temperature, p.top_k, p.top_p, p.repetition_penalty, p.stop_token_ids, p.seed,
                            p.logprobs)
    stable_row = restated_sample(case['logits'], case['history'], params, u=case['u'], stable=True)
    ref_row = restated_sample(case['logits'], case['history'], params, u=case['u'])
    out = run(case['logits'][None, :], [params], [case['history']], [case['u']], probs=True)
    check(out, [stable_row], [params], probs=True, label=f'golden {case["name"]}')
    tok = int(out.tokens[0])
    got = out.probs.cpu().numpy()[0]
    if ref_row.topp_tie:
        if case['probs'] is not None:
            want = np.sort(case['probs'][case['probs'] > 0])
            have = np.sort(got[got > 0])
            assert want.size == have.size
            np.testing.assert_allclose(have, want, rtol=TOL, atol=0)
        return
    if tok != case['token']:
        assert ref_row.boundary and not ref_row.greedy, (tok, case['token'])
        return
    assert close(float(out.logprobs[0]), case['logprob'], TOL)
    assert (tok in params.stop_token_ids) == case['stopped']
    got_top = out.top(0, params.logprobs)
    assert len(got_top) == len(case['top'])
    for (gi, gv), (wi, wv) in zip(got_top, case['top']):
        assert close(gv, wv, TOL)
    if case['probs'] is not None and not ref_row.boundary:
        np.testing.assert_array_equal(got > 0, case['probs'] > 0)
        m = case['probs'] > 1e-30
        np.testing.assert_allclose(got[m], case['probs'][m], rtol=TOL, atol=0)


# ---- edge cases ------------------------------------------------------------------------------

def _random_params(rng, kind):
    if kind == 'greedy':
        return SamplingParams(repetition_penalty=1.3, logprobs=4)
    if kind == 'topk':
        return SamplingParams(temperature=0.8, top_k=int(rng.integers(1, 60)), top_p=0.9, repetition_penalty=1.2,
                              logprobs=4, presence_penalty=0.4, frequency_penalty=0.2)
    if kind == 'topp':
        return SamplingParams(temperature=1.1, top_p=float(rng.uniform(0.3, 0.99)), repetition_penalty=0.9,
                              logprobs=4)
    return SamplingParams(temperature=0.6, logprobs=4, frequency_penalty=0.5)


@pytest.mark.parametrize('vocab', [1, 2, 3, 5, 17, 100, 1000, 4097, 10007, 70001])
@pytest.mark.parametrize('dtype', [torch.float32, torch.bfloat16])
def test_vocab_sizes_and_modes(vocab, dtype):
    say(f'edge vocab={vocab} dtype={dtype}')
    rng = np.random.default_rng(vocab)
    kinds = ['greedy', 'topk', 'topp', 'full'] * 2
    logits = torch.from_numpy((rng.standard_normal((len(kinds), vocab)) * 2).astype(np.float32)).to(dtype)
    params = [_random_params(rng, k) for k in kinds]
    hist = [rng.integers(0, vocab, int(rng.integers(0, 50))).tolist() for _ in kinds]
    u = rng.random(len(kinds)).astype(np.float32)
    rows = sample_rows(logits, hist, params, u)
    out = run(logits, params, hist, u, probs=True)
    check(out, rows, params, probs=True)


@pytest.mark.parametrize('dense', [False, True])
@pytest.mark.parametrize('dtype', [torch.float32, torch.bfloat16])
def test_long_histories_count_past_16_bits(dtype, dense):
    """Histories of 65536 ids or more take 32-bit counts over each half of a chunk in
    turn; an id repeated more than 65535 times keeps its exact count.  Forced through the
    multi-pass row path, a history this long is re-read per chunk rather than kept in LDS."""
    say(f'long histories dtype={dtype} dense={dense}')
    rng = np.random.default_rng(12)
    V = 151936
    kinds = ['greedy', 'topk', 'topp', 'full'] * 2
    logits = torch.from_numpy((rng.standard_normal((len(kinds), V)) * 2).astype(np.float32)).to(dtype)
    params = []
    for i, k in enumerate(kinds):
        t, tk, tp = {'greedy': (0.0, 0, 1.0), 'topk': (0.8, 50, 1.0), 'topp': (0.9, 0, 0.9),
                     'full': (1.1, 0, 1.0)}[k]
        params.append(SamplingParams(temperature=t, top_k=tk, top_p=tp, repetition_penalty=1.2,
                                     logprobs=3, presence_penalty=0.2, frequency_penalty=2e-5))
    hist = []
    for i in range(len(kinds)):
        hot = int(rng.integers(0, V))
        h = np.concatenate([np.full(66000 + 1000 * i, hot), rng.integers(0, V, 5000),
                            rng.integers(0, 64, 3000)])
        rng.shuffle(h)
        hist.append(h.tolist())
    # the hot id's penalty depends on its full count: 66000 * 2e-5 moves it by 1.32
    u = rng.random(len(kinds)).astype(np.float32)
    rows = sample_rows(logits, hist, params, u)
    out = run(logits, params, hist, u, probs=True, options=_lib.OPT_FORCE_DENSE if dense else 0)
    if dense:
        assert (out.info['path'] == 1).all()
    check(out, rows, params, probs=True)


@pytest.mark.parametrize('n', [0, 5])
def test_wide_vocab_top_p_rows_narrow_their_candidates(n):
    """Top-p rows over 74 chunks gather more candidates than the row's LDS list holds;
    the combine narrows them with a radix select before the histogram gather."""
    say(f'wide vocab top-p n={n}')
    rng = np.random.default_rng(13)
    V = 600001
    x = (rng.standard_normal((6, V)) * 2).astype(np.float32)
    x[1, rng.choice(V, 300, replace=False)] += 9.0          # heavy head
    x[3, rng.choice(V, 40, replace=False)] += 14.0
    logits = torch.from_numpy(x)
    params = [SamplingParams(temperature=t, top_p=tp, logprobs=n)
              for t, tp in ((0.8, 0.9), (0.7, 0.95), (1.0, 0.5), (0.9, 0.99), (1.3, 0.3), (0.6, 0.8))]
    u = rng.random(6).astype(np.float32)
    rows = sample_rows(logits, None, params, u)
    out = run(logits, params, None, u, probs=True)
    check(out, rows, params, probs=True)


@pytest.mark.parametrize('vocab', [151936, 100003, 20001, 600001])
@pytest.mark.parametrize('dtype', [torch.float32, torch.bfloat16])
def test_wide_top_p_rows(vocab, dtype):
    """Flat top-p rows whose kept set reaches far past the chunk candidates (thousands to
    most of the vocabulary) are resolved chunk by chunk from the chunks' histograms and
    final scores (row path 2), next to greedy, top-k and heavy-head rows of the same
    batch; value ties on a coarse grid put many equal scores into the cut."""
    say(f'wide top-p vocab={vocab} dtype={dtype}')
    rng = np.random.default_rng(vocab % 1000 + (7 if dtype == torch.bfloat16 else 0))
    specs = [(1.0, 0.9, 'flat'), (1.4, 0.97, 'flat'), (0.8, 0.8, 'flat'), (1.2, 0.999, 'flat'),
             (1.0, 0.95, 'grid'), (0.9, 0.9, 'grid8'), (0.7, 0.95, 'heavy'), (0.0, 1.0, 'flat'),
             (0.9, 0.9, 'topk'), (2.0, 0.5, 'flat')]
    x = (rng.standard_normal((len(specs), vocab)) * 2.5).astype(np.float32)
    params, hist = [], []
    for b, (t, tp, kind) in enumerate(specs):
        if kind == 'grid':
            x[b] = np.round(x[b] * 4) / 4          # ties: one score per 1/4
        elif kind == 'grid8':
            x[b] = np.round(x[b] * 64) / 64        # ties a little finer than the bins
        elif kind == 'heavy':
            x[b, rng.choice(vocab, 100, replace=False)] += 9.0
        k = 40 if kind == 'topk' else 0
        params.append(SamplingParams(temperature=t, top_k=k, top_p=tp, repetition_penalty=1.1,
                                     logprobs=int(rng.choice([0, 5, 64])), presence_penalty=0.3,
                                     frequency_penalty=0.2))
        hist.append(rng.integers(0, vocab, int(rng.integers(0, 3000))).tolist())
    logits = torch.from_numpy(x).to(dtype)
    u = rng.random(len(specs)).astype(np.float32)
    u[3] = 0.99999     # a draw near the end of the kept mass
    rows = sample_rows(logits, hist, params, u)
    out = run(logits, params, hist, u, probs=True)
    check(out, rows, params, probs=True)
    # the flat top-p rows never take the single-workgroup row path (1): the candidates
    # settle them (0) or the chunk histograms do (2), which the longer rows need
    paths = out.info['path'].tolist()
    assert all(paths[b] in (0, 2) for b in (0, 1, 2, 3, 9)), paths
    if vocab >= 100003:
        assert all(paths[b] == 2 for b in (0, 1, 3)), paths


def test_massive_ties_take_the_row_path():
    say('ties: constant rows')
    V = 50000
    logits = torch.zeros((4, V))
    params = [SamplingParams(logprobs=3), SamplingParams(temperature=1.0, top_k=5, logprobs=3),
              SamplingParams(temperature=1.0, top_p=0.5, logprobs=3), SamplingParams(temperature=1.0, logprobs=3)]
    u = np.float32([0.5, 0.5, 0.5, 0.999])
    rows = sample_rows(logits, None, params, u)
    out = run(logits, params, None, u, probs=True)
    assert int(out.tokens[0]) == 0
    assert int(out.info['kept'][1]) == V  # every tie with the k-th value survives top-k
    check(out, rows, params, probs=False)


def test_masked_and_infinite_logits():
    say('masked logits')
    V = 3000
    rng = np.random.default_rng(9)
    x = (rng.standard_normal((4, V)) * 2).astype(np.float32)
    x[:, rng.random(V) < 0.7] = -np.inf
    logits = torch.from_numpy(x)
    params = [SamplingParams(logprobs=5), SamplingParams(temperature=0.9, top_k=2000, logprobs=5),
              SamplingParams(temperature=0.9, top_p=0.8, logprobs=5), SamplingParams(temperature=0.9, logprobs=5)]
    u = rng.random(4).astype(np.float32)
    rows = sample_rows(logits, None, params, u)
    out = run(logits, params, None, u, probs=True)
    check(out, rows, params, probs=True)


def test_strided_and_unaligned_rows():
    say('strided / unaligned rows')
    rng = np.random.default_rng(10)
    V = 20001
    base = torch.from_numpy((rng.standard_normal((6, V + 7)) * 2).astype(np.float32))
    params = [SamplingParams(), SamplingParams(temperature=0.7, top_k=20, logprobs=2),
              SamplingParams(temperature=0.7, top_p=0.9), SamplingParams(temperature=0.7, top_k=3, logprobs=6),
              SamplingParams(repetition_penalty=1.5, logprobs=2), SamplingParams(temperature=2.0)]
    hist = [[0, 1, V - 1]] * 6
    u = rng.random(6).astype(np.float32)
    strided = base.to(DEV)[:, 3:3 + V]  # row stride V + 7, start offset 3 elements: no 16-byte alignment
    rows = sample_rows(base[:, 3:3 + V].contiguous(), hist, params, u)
    out = runner_for(DEV).run(strided, params, hist, u, 6, want_info=True)
    check(out, rows, params)


def test_other_float_dtypes_are_upcast():
    say('fp16 / fp64 inputs')
    rng = np.random.default_rng(11)
    x = torch.from_numpy((rng.standard_normal((2, 5000)) * 2).astype(np.float32))
    params = [SamplingParams(logprobs=2), SamplingParams(temperature=0.8, top_k=50, logprobs=2)]
    u = np.float32([0.3, 0.6])
    for dt in (torch.float16, torch.float64):
        xs = x.to(dt)
        rows = sample_rows(xs, None, params, u)
        out = run(xs, params, None, u)
        check(out, rows, params)


def test_large_top_k_and_top_n():
    say('large k and N')
    rng = np.random.default_rng(12)
    V = 151936
    x = torch.from_numpy((rng.standard_normal((3, V)) * 2.5).astype(np.float32))
    params = [SamplingParams(temperature=1.0, top_k=1000, top_p=0.95, logprobs=256),
              SamplingParams(temperature=1.0, top_k=5000, logprobs=20),
              SamplingParams(logprobs=256)]
    u = rng.random(3).astype(np.float32)
    rows = sample_rows(x, None, params, u)
    out = run(x, params, None, u)
    check(out, rows, params)


def test_top_k_quotient_ties():
    """Distinct scores one ulp apart around the k-th collapse to equal quotients after the
    division by T: the top set takes every candidate whose quotient reaches the k-th one,
    including scores below the k-th best (the combine's short path must step aside)."""
    say('top-k quotient ties')
    rng = np.random.default_rng(21)
    V, B = 30011, 24
    x = (rng.standard_normal((B, V)) * 2).astype(np.float32)
    params, u = [], rng.random(B).astype(np.float32)
    for b in range(B):
        k = int(rng.integers(5, 60))
        # a run of consecutive floats placed across the k-th largest position
        top = np.sort(x[b])[::-1]
        base = np.float32(top[k - 1] + 1.0)
        run_len = int(rng.integers(3, 12))
        vals = np.nextafter(np.full(run_len, base), np.float32(-np.inf))
        for j in range(1, run_len):
            vals[j] = np.nextafter(vals[j - 1], np.float32(-np.inf))
        pos = rng.choice(V, run_len + k, replace=False)
        x[b, pos[:k - 2]] = base + np.float32(5.0) + rng.random(k - 2).astype(np.float32)
        x[b, pos[k:k + run_len]] = vals
        t = float(rng.choice([7.0, 7.0, 5.0, 3.0, 0.3, 1.7, 1.0]))
        params.append(SamplingParams(temperature=t, top_k=k, top_p=float(rng.choice([1.0, 0.9, 0.5])), logprobs=4))
    logits = torch.from_numpy(x)
    rows = sample_rows(logits, None, params, u)
    out = run(logits, params, None, u, probs=True)
    check(out, rows, params, probs=True)


def test_top_p_kept_sets_around_the_short_list():
    """Top-p rows whose kept set has 30 to 80 entries: within the combine's first (best-48)
    list, just past it (second gather of the best 64), and past both (general path)."""
    say('top-p kept sets around 48 and 64')
    rng = np.random.default_rng(22)
    V = 151936
    heads = [30, 40, 46, 48, 50, 55, 60, 63, 64, 66, 72, 80]
    x = (rng.standard_normal((len(heads), V))).astype(np.float32)
    params = []
    for b, h in enumerate(heads):
        pos = rng.choice(V, h, replace=False)
        x[b, pos] = (12.0 + 0.05 * rng.standard_normal(h)).astype(np.float32)
        params.append(SamplingParams(temperature=1.0, top_p=float(rng.choice([0.9, 0.97, 0.995])), logprobs=3))
    u = rng.random(len(heads)).astype(np.float32)
    logits = torch.from_numpy(x)
    for dt in (torch.float32, torch.bfloat16):
        lt = logits.to(dt)
        rows = sample_rows(lt, None, params, u)
        out = run(lt, params, None, u, probs=True)
        check(out, rows, params, probs=True)


@pytest.mark.parametrize('elems', ['4', '8', '16'])
def test_other_chunk_sizes(elems, monkeypatch):
    """The smaller chunk variants (selected by KLSAMPLE_ELEMS_PER_THREAD, read per call)
    give the same results as the default."""
    say(f'chunk variant E={elems}')
    monkeypatch.setenv('KLSAMPLE_ELEMS_PER_THREAD', elems)
    for name, batch in (('mixed_b64', 16), ('throughput_b256_v151936', 8), ('latency_b1', None)):
        w = _with_logprobs(workloads.make(name, batch=batch), 4)
        rows = sample_rows(w.logits, w.histories, w.params, w.uniforms)
        out = run(w.logits, w.params, w.histories, w.uniforms, probs=True)
        check(out, rows, w.params, probs=True)


# ---- randomised configurations -----------------------------------------------------------


def _random_case(seed):
    """A seeded batch mixing vocab sizes, dtypes, score shapes (wide, heavy head, value
    ties on a 0.5 grid, mostly masked, nearly flat), every mode and penalty, histories
    with heavy repeats, and the full-row path."""
    rng = np.random.default_rng(seed)
    V = int(rng.choice([rng.integers(1, 300), rng.integers(300, 20000), rng.integers(20000, 160000), 151936]))
    B = int(rng.integers(1, 33)) if V <= 60000 else int(rng.integers(1, 13))
    dtype = torch.bfloat16 if rng.random() < 0.5 else torch.float32
    shape = str(rng.choice(['wide', 'heavy', 'ties', 'masked', 'flat']))
    x = rng.standard_normal((B, V)).astype(np.float32) * float(rng.uniform(0.3, 8.0))
    if shape == 'heavy':
        for b in range(B):
            x[b, rng.integers(0, V, size=min(V, int(rng.integers(1, 40))))] += rng.uniform(5, 25)
    elif shape == 'ties':
        x = np.round(x * 2) / 2
    elif shape == 'masked':
        x[rng.random((B, V)) < rng.uniform(0.1, 0.95)] = -np.inf
        x[:, 0] = np.maximum(x[:, 0], 0)
    elif shape == 'flat':
        x *= 0.01
    params, hist = [], []
    for _ in range(B):
        T = 0.0 if rng.random() < 0.2 else float(rng.choice([1.0, rng.uniform(0.2, 2.5)]))
        k = 0 if rng.random() < 0.4 else int(rng.choice([rng.integers(1, 64), rng.integers(64, 3000),
                                                         rng.integers(1, V + 5)]))
        p = 1.0 if rng.random() < 0.35 else float(rng.choice([rng.uniform(0.05, 0.999), rng.uniform(0.9, 0.9999)]))
        params.append(SamplingParams(
            temperature=T, top_k=k, top_p=p,
            repetition_penalty=1.0 if rng.random() < 0.4 else float(rng.uniform(0.7, 1.6)),
            logprobs=int(rng.choice([0, 1, 4, 20, rng.integers(0, 65)])),
            presence_penalty=0.0 if rng.random() < 0.5 else float(rng.uniform(-0.5, 1.0)),
            frequency_penalty=0.0 if rng.random() < 0.5 else float(rng.uniform(-0.3, 0.8))))
        n = int(rng.choice([0, rng.integers(0, 100), rng.integers(0, 3000)]))
        hist.append(rng.integers(0, min(V, 20) if rng.random() < 0.2 else V, n).tolist())
    u = rng.random(B).astype(np.float32)
    options = _lib.OPT_FORCE_DENSE if rng.random() < 0.15 else 0
    return torch.from_numpy(x).to(dtype), params, hist, u, options, shape


@pytest.mark.parametrize('block', range(6))
def test_randomised_configurations(block):
    """Forty seeded random batches per block against the oracle, with probabilities
    on every third."""
    for seed in range(40 * block, 40 * block + 40):
        logits, params, hist, u, options, shape = _random_case(90_000 + seed)
        say(f'random seed={90_000 + seed} shape={shape}')
        rows = sample_rows(logits, hist, params, u)
        out = run(logits, params, hist, u, options=options, probs=seed % 3 == 0)
        check(out, rows, params, probs=seed % 3 == 0)
