"""Pinning the CPU oracle (CPU only).

The oracle restates serving/sampling.py:44-63.  Each check below is independent of the
oracle's own code: the reference's known-answer test, vectors written by running the
reference sampler, or a closed form evaluated here with numpy.  Each is chosen so a
plausible slip (penalty sign, strict vs non-strict cut, dropped term, wrong rounding,
off-by-one in the CDF) changes the answer."""
import math

import numpy as np
import pytest
import torch

from helpers import GoldenParams, close, golden_cases
from oracle.cpu_sampler import inverse_cdf, normalize_history, restated_sample, sample_rows

P = GoldenParams
CASES = golden_cases()


def test_reference_known_answer_test():
    # serving/test_serving.py:101-107
    params = P(temperature=.8, top_k=3, top_p=.9, repetition_penalty=1.1, stop_token_ids=frozenset({2}),
               seed=7, logprobs=2)
    logits = torch.tensor([0., 1., 3., 2.])
    a = restated_sample(logits, [2], params, u=0.5)
    b = restated_sample(logits, [2], params, u=0.5)
    assert (a.token_id, a.logprob, a.top_logprobs, a.stopped) == (b.token_id, b.logprob, b.top_logprobs, b.stopped)
    assert len(a.top_logprobs) == 2
    greedy = restated_sample(logits, (), P(stop_token_ids=frozenset({2})))
    assert greedy.token_id == 2 and greedy.stopped


def test_known_answer_hand_derived_values():
    # numpy fp32 by hand: after r=1.1 on id 2 -> [0, 1, 2.7272727, 2]; /0.8 ->
    # [0, 1.25, 3.409091, 2.5]; k=3 drops id 0; top-p .9 drops id 1 (exclusive mass .924)
    params = P(temperature=.8, top_k=3, top_p=.9, repetition_penalty=1.1, logprobs=2)
    row = restated_sample(torch.tensor([0., 1., 3., 2.]), [2], params, u=0.5)
    probs = row.probs.numpy()
    assert probs[0] == 0 and probs[1] == 0
    assert probs[2] == pytest.approx(0.71281412, abs=1e-7)
    assert probs[3] == pytest.approx(0.28718588, abs=1e-7)
    assert dict(row.top_logprobs)[2] == pytest.approx(-0.33853459, abs=1e-7)
    assert dict(row.top_logprobs)[3] == pytest.approx(-1.24762559, abs=1e-7)
    assert restated_sample(torch.tensor([0., 1., 3., 2.]), [2], params, u=0.7128).token_id == 2
    assert restated_sample(torch.tensor([0., 1., 3., 2.]), [2], params, u=0.7129).token_id == 3


@pytest.mark.parametrize('case', CASES, ids=[c['name'] for c in CASES])
def test_reference_vectors(case):
    """Vectors written by running the reference sampler (tests/golden/make_reference_vectors.py)."""
    row = restated_sample(case['logits'], case['history'], case['params'], u=case['u'])
    assert row.token_id == case['token']
    assert row.stopped == case['stopped']
    assert close(row.logprob, case['logprob'], 1e-6)
    assert len(row.top_logprobs) == len(case['top'])
    for (gi, gv), (wi, wv) in zip(row.top_logprobs, case['top']):
        assert close(gv, wv, 1e-6)
        if math.isfinite(wv):
            assert gi == wi
    if case['probs'] is None:
        assert row.probs is None
    else:
        got = row.probs.numpy()
        np.testing.assert_array_equal(got > 0, case['probs'] > 0)
        np.testing.assert_allclose(got, case['probs'], rtol=1e-6, atol=0)


# ---- closed forms -----------------------------------------------------------------------

def _numpy_penalised(x, history, r, a=0.0, b=0.0):
    """fp32 closed form: repetition on distinct ids (multiply negatives, divide the rest),
    then s - fp32(fp32(b*count) + a)."""
    s = x.astype(np.float32).copy()
    ids, counts = np.unique(np.asarray(history, dtype=np.int64), return_counts=True)
    if r != 1 and ids.size:
        rr = np.float32(r)
        v = s[ids]
        s[ids] = np.where(v < 0, v * rr, v / rr).astype(np.float32)
    if (a != 0 or b != 0) and ids.size:
        t = (np.float32(b) * counts.astype(np.float32)).astype(np.float32)
        t = (t + np.float32(a)).astype(np.float32)
        s[ids] = (s[ids] - t).astype(np.float32)
    return s


def test_repetition_penalty_closed_form():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(300) * 3).astype(np.float32)
    x[:3] = [0.0, -0.0, -2.5]
    hist = list(rng.integers(0, 300, 80)) + [0, 1, 2, 2, 2]
    for r in (1.1, 1.7, 0.6):
        row = restated_sample(torch.from_numpy(x), hist, P(repetition_penalty=r))
        np.testing.assert_array_equal(row.scores.numpy(), _numpy_penalised(x, hist, r))
    # applied once per distinct id, and multiplying (not dividing) negative scores
    row = restated_sample(torch.tensor([-2.0, 2.0]), [0, 0, 1], P(repetition_penalty=2.0))
    assert row.scores.tolist() == [-4.0, 1.0]


def test_presence_frequency_closed_form_and_zero_invariant():
    rng = np.random.default_rng(2)
    x = (rng.standard_normal(500) * 2).astype(np.float32)
    hist = list(rng.integers(0, 500, 200)) + [7] * 9
    for a, b in ((0.5, 0.3), (0.0, 0.7), (-0.4, 0.0)):
        row = restated_sample(torch.from_numpy(x), hist, P(repetition_penalty=1.2, presence_penalty=a,
                                                          frequency_penalty=b))
        np.testing.assert_array_equal(row.scores.numpy(), _numpy_penalised(x, hist, 1.2, a, b))
    # brute-force count on a tiny history: id 1 seen 3 times, id 0 once
    row = restated_sample(torch.tensor([1.0, 1.0, 1.0]), [1, 0, 1, 1], P(presence_penalty=0.5, frequency_penalty=0.25))
    assert row.scores.tolist() == [1.0 - (0.25 * 1 + 0.5), 1.0 - (0.25 * 3 + 0.5), 1.0]
    # alpha == beta == 0 reproduces the reference exactly
    base = restated_sample(torch.from_numpy(x), hist, P(temperature=0.9, top_k=30, repetition_penalty=1.3), u=0.4)
    zero = restated_sample(torch.from_numpy(x), hist, P(temperature=0.9, top_k=30, repetition_penalty=1.3,
                                                       presence_penalty=0.0, frequency_penalty=0.0), u=0.4)
    assert torch.equal(base.scores, zero.scores) and base.token_id == zero.token_id


def test_temperature_is_ieee_fp32_division():
    x = (np.random.default_rng(7).standard_normal(4096) * 5).astype(np.float32)
    row = restated_sample(torch.from_numpy(x), (), P(temperature=0.7), u=0.3)
    np.testing.assert_array_equal(row.scores.numpy(), x / np.float32(0.7))
    # neither a reciprocal multiply nor a double-precision quotient gives these values
    assert not np.array_equal(row.scores.numpy(), x * np.float32(1 / 0.7))
    assert not np.array_equal(row.scores.numpy(), (x.astype(np.float64) / 0.7).astype(np.float32))


def test_topk_threshold_with_multiplicity_brute_force():
    rng = np.random.default_rng(3)
    for trial in range(30):
        v = int(rng.integers(2, 40))
        x = rng.integers(-4, 5, v).astype(np.float32)  # many ties
        k = int(rng.integers(1, v + 3))
        row = restated_sample(torch.from_numpy(x), (), P(temperature=1.0, top_k=k), u=0.5)
        kk = min(k, v)
        cutoff = np.sort(x)[::-1][kk - 1]
        np.testing.assert_array_equal(np.isfinite(row.scores.numpy()), x >= cutoff)


def test_topp_distinct_values_closed_form():
    rng = np.random.default_rng(4)
    for trial in range(40):
        v = int(rng.integers(2, 60))
        x = rng.permutation(np.linspace(-3, 3, v)).astype(np.float32)
        p = float(rng.uniform(0.05, 0.99))
        row = restated_sample(torch.from_numpy(x), (), P(temperature=1.0, top_p=p), u=0.5)
        order = np.argsort(-x.astype(np.float64))
        w = np.exp(x[order].astype(np.float64) - x.max())
        excl = (np.cumsum(w) - w) / w.sum()
        keep = np.zeros(v, bool)
        keep[order[excl <= np.float32(p)]] = True
        if np.min(np.abs(excl - np.float32(p))) < 1e-6:
            continue  # within the boundary tolerance fp32 rounding decides
        np.testing.assert_array_equal(np.isfinite(row.scores.numpy()), keep)
        assert keep[order[0]]  # the crossing token is kept: never empty


def test_logprob_is_log_softmax_of_final_scores():
    rng = np.random.default_rng(5)
    x = (rng.standard_normal(1000) * 2).astype(np.float32)
    row = restated_sample(torch.from_numpy(x), (), P(temperature=0.8, top_k=50, top_p=0.9, logprobs=5), u=0.6)
    s = row.scores.numpy().astype(np.float64)
    f = np.isfinite(s)
    lse = s[f].max() + np.log(np.exp(s[f] - s[f].max()).sum())
    assert row.logprob == pytest.approx(s[row.token_id] - lse, abs=2e-6)
    assert [i for i, _ in row.top_logprobs] == list(np.argsort(-s)[:5])
    greedy = restated_sample(torch.from_numpy(x), (), P(logprobs=1))
    lse_all = x.max() + np.log(np.exp(x.astype(np.float64) - x.max()).sum())
    assert greedy.logprob == pytest.approx(x.max() - lse_all, abs=2e-6)


def test_exact_log_normaliser_closed_forms():
    # equal scores: every logprob is -log(n) exactly; the reference's fp32 value is close
    flat = restated_sample(torch.zeros(100_000), (), P(logprobs=1))
    assert flat.exact_logprob == pytest.approx(-math.log(100_000), abs=1e-12)
    assert flat.lse_error == pytest.approx(abs(-flat.logprob - math.log(100_000)), abs=1e-12)
    assert flat.lse_error < 1e-4
    # two values a > b, n_b copies of b: log(1 / (1 + n_b e^(b - a))) at the argmax
    x = torch.full((50_001,), -3.0)
    x[7] = 4.0
    two = restated_sample(x, (), P(logprobs=1))
    assert two.token_id == 7
    assert two.exact_logprob == pytest.approx(-math.log1p(50_000 * math.exp(-7.0)), abs=1e-12)
    # masked entries take no part; a masked-out token has no exact value
    y = torch.tensor([1.0, 2.0, -math.inf, 0.5])
    r = restated_sample(y, (), P(temperature=1.0), u=0.0)
    assert r.token_id == 0
    assert r.exact_logprob == pytest.approx(1.0 - math.log(math.e + math.e ** 2 + math.e ** 0.5), abs=1e-12)


def test_greedy_takes_lowest_index_of_ties():
    assert restated_sample(torch.tensor([1., 5., 2., 5.]), (), P()).token_id == 1
    assert restated_sample(torch.tensor([-1., -1., -1.]), (), P()).token_id == 0


def test_inverse_cdf_brute_force_and_monotone():
    rng = np.random.default_rng(6)
    for trial in range(50):
        v = int(rng.integers(1, 30))
        p = rng.random(v).astype(np.float32)
        p[rng.random(v) < 0.3] = 0
        if p.sum() == 0:
            p[int(rng.integers(0, v))] = 1.0
        u = float(np.float32(rng.random()))
        total = float(np.sum(p.astype(np.float64)))
        acc, want = 0.0, None
        for i in range(v):
            acc += float(p[i])
            if acc > u * total:
                want = i
                break
        if want is None:
            want = int(np.flatnonzero(p)[-1])
        assert inverse_cdf(torch.from_numpy(p), u) == want
        assert p[want] > 0
    p = torch.tensor([0.1, 0.0, 0.4, 0.5])
    toks = [inverse_cdf(p, u) for u in np.linspace(0, 0.999, 200)]
    assert toks == sorted(toks) and set(toks) == {0, 2, 3}


def test_history_normalisation_matches_indexing():
    assert normalize_history([-1, 0, 3], 4).tolist() == [3, 0, 3]
    with pytest.raises(IndexError):
        normalize_history([4], 4)
    with pytest.raises(IndexError):
        normalize_history([-5], 4)


def test_boundary_classification():
    # an exact value tie straddling the top-p cut is flagged, but it is no boundary row:
    # the stable order keeps the lower index
    row = restated_sample(torch.tensor([2., 1., 1., 0.]), (), P(temperature=1.0, top_p=0.73), u=0.99, stable=True)
    assert row.topp_tie and not row.boundary
    assert torch.isfinite(row.scores).tolist() == [True, True, False, False]
    # the top-p mass at the cut within 1e-6 of p: a margin row
    w = np.array([0.5, 0.3, 0.2])
    x = torch.from_numpy(np.log(w).astype(np.float32))
    xd = x.double().numpy()
    mass = float(np.exp(xd[0]) / np.exp(xd).sum())
    row = restated_sample(x, (), P(temperature=1.0, top_p=mass + 2e-7), u=0.3, stable=True)
    assert row.margin_row and row.boundary
    # u * Z within 1e-6 of a CDF step
    full = restated_sample(x, (), P(temperature=1.0), u=0.3, stable=True)
    row = restated_sample(x, (), P(temperature=1.0), u=float(full.probs[0]) + 1e-7, stable=True)
    assert row.cdf_row and row.boundary and not row.margin_row
    # far from every cut
    row = restated_sample(torch.tensor([3., 1., 0.5, 0.]), (), P(temperature=1.0, top_p=0.5), u=0.2)
    assert not row.boundary


def test_faithful_mode_is_the_reference_draw():
    """Faithful mode draws with torch.multinomial from the seeded generator, as
    serving/sampling.py:60 does; equal seeds give equal tokens."""
    x = torch.randn(5000, generator=torch.Generator().manual_seed(0))
    params = P(temperature=1.0, top_k=0, top_p=0.95, seed=11)
    g1, g2 = torch.Generator().manual_seed(11), torch.Generator().manual_seed(11)
    a = [restated_sample(x, (), params, generator=g1).token_id for _ in range(5)]
    b = [restated_sample(x, (), params, generator=g2).token_id for _ in range(5)]
    assert a == b


def test_sample_rows_loops_rows():
    x = torch.tensor([[0., 1., 3., 2.], [3., 2., 1., 0.]])
    rows = sample_rows(x, [[2], []], [P(repetition_penalty=1.1), P()], None)
    assert [r.token_id for r in rows] == [2, 0]


# ---- the stable tie order and the parity checker itself ----------------------------------

def test_stable_tie_order_keeps_the_reference_count_and_lowest_indices():
    """Stable order changes only which of equal scores are kept at the top-p cut: the
    kept count, every probability and logprob stay the reference's."""
    rng = np.random.default_rng(31)
    for trial in range(40):
        v = int(rng.integers(5, 400))
        x = torch.from_numpy((np.round(rng.standard_normal(v) * 2) / 2).astype(np.float32))  # many ties
        params = P(temperature=float(rng.uniform(0.5, 1.5)), top_k=int(rng.choice([0, 10, 50])),
                   top_p=float(rng.uniform(0.3, 0.99)), logprobs=8)
        u = float(rng.random())
        ref = restated_sample(x, (), params, u=u)
        st = restated_sample(x, (), params, u=u, stable=True)
        assert ref.kept == st.kept
        # (the fp32 softmax sums the kept entries in vocab order, so the last bit may move)
        np.testing.assert_allclose(np.sort(ref.probs.numpy()), np.sort(st.probs.numpy()), rtol=1e-6, atol=0)
        fin = torch.isfinite(st.scores)
        if st.pre_topp is not None and st.kept:
            # the kept set is a prefix of (score descending, index ascending)
            order = sorted(range(v), key=lambda i: (-float(st.pre_topp[i]), i))
            assert set(order[:st.kept]) == set(torch.nonzero(fin).flatten().tolist())
        # the top-N list: by final score, equal scores by index, then -inf entries by index
        sc = st.scores
        want = sorted(range(v), key=lambda i: (-float(sc[i]), i))[:min(8, v)]
        assert [i for i, _ in st.top_logprobs] == want
        lp = sc.log_softmax(0)
        assert [b for _, b in st.top_logprobs] == [float(lp[i]) for i in want]


def test_exact_top_p_cut_closed_forms():
    """The exact (float64) cut: n equal scores keep floor(p*n) + 1 of them (exclusive mass
    j/n <= p), the lowest indices; weights 2^-j (scores -j ln 2) keep the smallest J with
    (1 - 2^-J) / (1 - 2^-n) > p."""
    n = 1000
    for p in (0.1, 0.25, 0.5, 0.731, 0.9, 0.99):
        row = restated_sample(torch.zeros(n), (), P(temperature=1.0, top_p=p), u=0.5, stable=True)
        k = math.floor(p * n) + 1
        if abs(p * n - round(p * n)) > 1e-3:   # away from an exact multiple
            assert row.topp_exact_kept == k
            assert row.topp_exact_cut == (0.0, k - 1)
    n = 40
    x = torch.from_numpy((-np.arange(n) * math.log(2)).astype(np.float32))
    xs = x.double().numpy()
    w = np.exp(xs - xs[0])
    for p in (0.3, 0.6, 0.8, 0.95, 0.999):
        row = restated_sample(x, (), P(temperature=1.0, top_p=p), u=0.5, stable=True)
        excl = (np.cumsum(w) - w) / w.sum()
        assert row.topp_exact_kept == int((excl <= np.float32(p)).sum())
        # closed form: excl(j) = (1 - 2^-j) / (1 - 2^-n) up to the fp32 rounding of -j ln 2
        closed = next(j for j in range(1, n + 1) if (1 - 2.0 ** -j) / (1 - 2.0 ** -n) > np.float32(p))
        assert row.topp_exact_kept == closed


def _fake_gpu_output(rows, vocab, n):
    """A BatchOutput holding exactly what the kernels' rules give, built from the stable
    oracle: tokens, exact logprobs, kept counts with (cut score, cut index), top-N."""
    from types import SimpleNamespace

    from klsample import _lib
    B = len(rows)
    info = np.zeros(B, dtype=_lib.ROW_INFO_DTYPE)
    top_ids = np.full((B, n), -1, np.int32)
    top_lp = np.full((B, n), -np.inf, np.float32)
    probs = np.zeros((B, vocab), np.float32)
    for b, r in enumerate(rows):
        s = r.scores.numpy()
        fin = np.isfinite(s)
        info['kept'][b] = int(fin.sum()) if not r.greedy else vocab
        if not r.greedy:
            cut = float(s[fin].min())
            info['cut_score'][b] = cut
            pre = (r.pre_topp if r.pre_topp is not None else r.scores).numpy()
            ties = np.flatnonzero(pre == cut)
            kept_ties = np.flatnonzero(s == cut)
            info['cut_index'][b] = vocab if ties.size == kept_ties.size else int(kept_ties.max())
            probs[b] = r.exact_probs.astype(np.float32)
        for t, (i, v) in enumerate(r.top_logprobs):
            top_ids[b, t], top_lp[b, t] = i, v
    return SimpleNamespace(tokens=np.array([r.token_id for r in rows]),
                           logprobs=np.array([r.exact_logprob for r in rows], np.float32),
                           info=info, top_ids=top_ids, top_logprobs=top_lp,
                           top=lambda b, c: tuple((int(top_ids[b, t]), float(top_lp[b, t]))
                                                  for t in range(min(c, vocab, n)))), probs


def test_parity_checker_accepts_the_kernel_rules_and_rejects_tie_swaps():
    """compare() passes an output that follows the documented rules (built from the
    oracle) on tie-heavy rows, and fails when a planted mistake in the oracle side swaps
    a tied token, drops a kept entry, or perturbs one probability by 2e-5."""
    from helpers import compare
    rng = np.random.default_rng(32)
    V, B = 3000, 12
    x = torch.from_numpy((np.round(rng.standard_normal((B, V)) * 4) / 4).astype(np.float32))
    params = [P(temperature=1.0, top_p=float(rng.uniform(0.5, 0.95)), logprobs=5) for _ in range(B - 2)]
    params += [P(logprobs=5), P(temperature=0.7, top_k=30, logprobs=5)]
    u = rng.random(B)
    rows = sample_rows(x, None, params, u)
    out, probs = _fake_gpu_output(rows, V, 5)
    rep = compare(out, rows, params, probs=probs)
    assert rep.ok(), rep.failures
    assert rep.tie_rows > 0 and rep.exact == B
    # plant: a tied neighbour of the token (same score, other index) for a row without margins
    b = next(i for i, r in enumerate(rows) if not r.greedy and not r.boundary
             and (r.scores == r.scores[r.token_id]).sum() > 1)
    twin = int(torch.nonzero(rows[b].scores == rows[b].scores[rows[b].token_id]).flatten()[-1])
    if twin == rows[b].token_id:
        twin = int(torch.nonzero(rows[b].scores == rows[b].scores[rows[b].token_id]).flatten()[0])
    bad = list(out.tokens)
    bad[b] = twin
    out.tokens = np.array(bad)
    assert not compare(out, rows, params, probs=probs).ok()
    out.tokens = np.array([r.token_id for r in rows])
    # plant: one kept entry fewer
    out.info['kept'][0] -= 1
    assert not compare(out, rows, params, probs=probs).ok()
    out.info['kept'][0] += 1
    # plant: a probability off by 2e-5 relative
    j = int(np.flatnonzero(probs[1] > 1e-3)[0])
    probs[1, j] *= np.float32(1 + 2e-5)
    assert not compare(out, rows, params, probs=probs).ok()


def test_stable_top_n_orders_by_score_when_logprobs_round_together():
    """Two scores one ulp apart share an fp32 logprob over a wide row; the higher score
    is still listed first (the kernels' order), whatever its index."""
    x = torch.zeros(100_000)
    c = np.float32(0.01)
    x[7] = float(c)
    x[3] = float(np.nextafter(c, np.float32(-1)))
    row = restated_sample(x, (), P(logprobs=3), stable=True)
    lp = x.log_softmax(0)
    assert float(lp[7]) == float(lp[3])
    assert [i for i, _ in row.top_logprobs] == [7, 3, 0]
