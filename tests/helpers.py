"""Shared test helpers: golden-vector decoding and the parity comparison."""
from __future__ import annotations

import base64
import json
import math
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np
import torch

GOLDEN = Path(__file__).resolve().parent / 'golden' / 'reference_vectors.json'


@dataclass(frozen=True)
class GoldenParams:
    """Plain parameter record (the fields ``SamplingParams`` has)."""

    temperature: float = 0.0
    top_k: int = 0
    top_p: float = 1.0
    repetition_penalty: float = 1.0
    stop_token_ids: frozenset = frozenset()
    seed: int = 0
    logprobs: int = 0
    presence_penalty: float = 0.0
    frequency_penalty: float = 0.0


def _arr(text, dtype):
    return np.frombuffer(base64.b64decode(text), dtype=dtype).copy()


def _num(x):
    return float(x) if not isinstance(x, str) else float(x)


def golden_cases():
    data = json.loads(GOLDEN.read_text())
    out = []
    for c in data['cases']:
        kw = dict(c['params'])
        kw['stop_token_ids'] = frozenset(kw.get('stop_token_ids', []))
        exp = c['expected']
        probs = None
        if exp['probs_nonzero'] is not None:
            probs = np.zeros(c['vocab'], dtype=np.float32)
            idx = _arr(exp['probs_nonzero']['index_i32'], '<i4')
            probs[idx] = _arr(exp['probs_nonzero']['value_f32'], '<f4')
        out.append(dict(
            name=c['name'], logits=torch.from_numpy(_arr(c['logits_f32'], '<f4')), history=c['history'],
            params=GoldenParams(**kw), u=c['u'], token=exp['token_id'], logprob=_num(exp['logprob']),
            top=[(i, _num(v)) for i, v in exp['top_logprobs']], stopped=exp['stopped'], probs=probs))
    return out


def close(a: float, b: float, tol: float = 1e-5) -> bool:
    if math.isinf(a) or math.isinf(b) or math.isnan(a) or math.isnan(b):
        return (a == b) or (math.isnan(a) and math.isnan(b))
    return abs(a - b) <= tol * max(1.0, abs(b))


@dataclass
class ParityReport:
    """Per-call parity counts.  ``boundary_mismatches`` are the only token differences
    allowed: rows whose top-p mass or CDF step lies within 1e-6 of the cut."""

    rows: int = 0
    greedy: int = 0
    sampled: int = 0
    exact: int = 0                 # rows whose token id equals the oracle's
    tie_rows: int = 0              # sampled rows with a value tie across the top-p cut (checked like any other)
    margin_rows: int = 0           # top-p mass within 1e-6 (+ the reference's fp32 delta) of p
    cdf_rows: int = 0              # u * Z within 1e-6 of a CDF step
    kept_differs: int = 0          # margin rows whose kept count differs from the reference's
    boundary_mismatches: int = 0   # token differs on a margin or CDF row (it must still be kept)
    probs_rows: int = 0            # rows whose probability vector was compared
    max_prob_rel: float = 0.0      # largest relative error against the exact softmax
    max_logprob_err: float = 0.0   # largest error against the exact log-softmax
    failures: list = field(default_factory=list)

    def ok(self) -> bool:
        return not self.failures

    def counts(self) -> dict:
        d = {k: getattr(self, k) for k in ('rows', 'greedy', 'sampled', 'exact', 'tie_rows', 'margin_rows',
                                           'cdf_rows', 'kept_differs', 'boundary_mismatches', 'probs_rows')}
        d['max_prob_rel'] = float(f'{self.max_prob_rel:.3g}')
        d['max_logprob_err'] = float(f'{self.max_logprob_err:.3g}')
        d['failures'] = len(self.failures)
        return d


def _exact_lse(scores: torch.Tensor) -> float:
    s = scores.double().numpy()
    fin = np.isfinite(s)
    if not fin.any():
        return math.nan
    m = s[fin].max()
    return float(m + math.log(np.exp(s[fin] - m).sum()))


def _kept_set_matches(o, info_b) -> bool:
    """The GPU's kept set, described by (cut_score, cut_index) over the scores entering
    top-p, equals the oracle's finite final scores."""
    final = o.scores.numpy()
    want = np.isfinite(final)
    cut, cidx = float(info_b['cut_score']), int(info_b['cut_index'])
    if cut == -math.inf:
        return int(want.sum()) == int(info_b['kept'])
    pre = (o.pre_topp if o.pre_topp is not None else o.scores).numpy()
    got = (pre > cut) | ((pre == cut) & (np.arange(pre.size) <= cidx))
    return bool(np.array_equal(got, want))


def compare(out, oracle_rows, params_list, *, tol: float = 1e-5, probs=None, check_top: bool = True) -> ParityReport:
    """Row-by-row parity of a GPU call against oracle rows (uniform mode, stable tie
    order: equal scores in ascending index order, which is the kernels' rule).

    * Token ids must be equal on every row.  The only exception is a sampled row whose
      top-p decision lies within ``1e-6 + |delta|`` of p (``delta`` is the reference's
      own fp32 normalisation error) and whose kept count therefore differs, or whose
      ``u * Z`` lies within 1e-6 of a CDF step; the GPU's token must then still be in
      the oracle's kept set or in the exact (float64) top-p cut's.
    * The kept count must equal the exact top-p cut's unless that cut is within 1e-6 of
      p, and the reference's unless the row is a margin row; with equal counts the kept
      set itself (the GPU's cut score and cut index) must equal the oracle's.
    * With the same token and kept set: logprobs within ``tol`` (relative, floor 1) of
      the exact (float64) log-softmax of the final scores, and within ``tol + eps`` of
      the reference's fp32 value (``eps``: that row's own fp32 log-normaliser error);
      top-N ids equal to the oracle's list entry for entry, values within ``tol`` of
      the exact log-softmax; probabilities (if given) within ``tol`` relative of the
      exact (float64) softmax of the final scores, and zero outside the kept set."""
    rep = ParityReport()
    info = out.info
    for b, (o, p) in enumerate(zip(oracle_rows, params_list)):
        rep.rows += 1
        tok = int(out.tokens[b])
        kept = int(info['kept'][b]) if info is not None else None
        same_set = True
        if o.greedy:
            rep.greedy += 1
            if tok != o.token_id:
                rep.failures.append(f'row {b}: greedy token {tok} != oracle {o.token_id}')
                continue
        else:
            rep.sampled += 1
            rep.tie_rows += int(o.topp_tie)
            rep.margin_rows += int(o.margin_row)
            rep.cdf_rows += int(o.cdf_row)
            if kept is not None:
                if o.topp_exact_kept is not None and o.topp_exact_margin >= 1e-6 and kept != o.topp_exact_kept:
                    rep.failures.append(f'row {b}: kept {kept} != exact top-p cut {o.topp_exact_kept}')
                if not o.margin_row and kept != o.kept:
                    rep.failures.append(f'row {b}: kept {kept} != oracle {o.kept}')
                same_set = kept == o.kept
                if not same_set:
                    rep.kept_differs += 1
                elif not _kept_set_matches(o, info[b]):
                    rep.failures.append(f'row {b}: kept set (cut {float(info["cut_score"][b])!r}, index '
                                        f'{int(info["cut_index"][b])}) differs from the oracle\'s')
            if tok != o.token_id:
                if not same_set or o.cdf_row:
                    rep.boundary_mismatches += 1
                    if not o.in_kept(tok):
                        rep.failures.append(f'row {b}: boundary-row token {tok} is not kept')
                    continue
                rep.failures.append(f'row {b}: token {tok} != oracle {o.token_id} (topp_margin={o.topp_margin:.3g}, '
                                    f'cdf_margin={o.cdf_margin:.3g}, tie={o.topp_tie})')
                continue
        rep.exact += 1
        if not same_set:
            continue  # the reference's rounding moved its cut: normalisers differ by design
        lp = float(out.logprobs[b])
        if not close(lp, o.logprob, tol + o.lse_error):
            rep.failures.append(f'row {b}: logprob {lp!r} != oracle {o.logprob!r}')
        elif not math.isnan(o.exact_logprob):
            if not close(lp, o.exact_logprob, tol):
                rep.failures.append(f'row {b}: logprob {lp!r} != exact {o.exact_logprob!r}')
            rep.max_logprob_err = max(rep.max_logprob_err, abs(lp - o.exact_logprob))
        if check_top and p.logprobs:
            got = out.top(b, p.logprobs)
            want = list(o.top_logprobs)
            lse = _exact_lse(o.scores)
            if [g[0] for g in got] != [w[0] for w in want]:
                rep.failures.append(f'row {b}: top ids {[g[0] for g in got][:6]}... != oracle '
                                    f'{[w[0] for w in want][:6]}...')
            else:
                s = o.scores
                for (gi, gv), (wi, wv) in zip(got, want):
                    ex = float(s[gi]) - lse if math.isfinite(wv) else -math.inf
                    if not close(gv, ex, tol) or not close(gv, wv, tol + o.lse_error):
                        rep.failures.append(f'row {b}: top logprob of {gi}: {gv!r} vs exact {ex!r} / oracle {wv!r}')
                        break
        if probs is not None and o.exact_probs is not None:
            # probabilities of 1e-30 and below carry no relative precision in fp32 (they
            # are compared as "kept or not" only)
            want = o.exact_probs
            got = probs[b].astype(np.float64)
            rep.probs_rows += 1
            if np.any((want == 0) & (got != 0)):
                rep.failures.append(f'row {b}: {int(((want == 0) & (got != 0)).sum())} probabilities outside the kept set')
            m = want > 1e-30
            if np.any(got[m] <= 0):
                rep.failures.append(f'row {b}: {int((got[m] <= 0).sum())} kept probabilities are zero')
            rel = np.abs(got[m] - want[m]) / want[m]
            if rel.size:
                rep.max_prob_rel = max(rep.max_prob_rel, float(rel.max()))
                if rel.max() > tol:
                    rep.failures.append(f'row {b}: probability rel err {rel.max():.3g} against the exact softmax')
    return rep
