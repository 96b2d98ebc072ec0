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


def top_matches(got, want, tol: float = 1e-5, cut_tie: bool = False) -> bool:
    """Top-logprob lists agree: same length, values within ``tol``, and the same ids
    for every group of equal values in ``want`` except the last group (the list may
    cut a tie at a different member) and -inf entries (their ids are
    implementation-defined).  With ``cut_tie`` (a value tie straddles the top-p cut,
    so which of its members are kept is implementation-defined) the last finite group
    is exempt as well."""
    if len(got) != len(want):
        return False
    for (gi, gv), (wi, wv) in zip(got, want):
        if not close(gv, wv, tol):
            return False
    i, n = 0, len(want)
    while i < n:
        j = i
        while j < n and want[j][1] == want[i][1]:
            j += 1
        last_finite = j < n and not math.isfinite(want[j][1])
        if j < n and math.isfinite(want[i][1]) and not (cut_tie and last_finite):
            if {g[0] for g in got[i:j]} != {w[0] for w in want[i:j]}:
                return False
        i = j
    return True


@dataclass
class ParityReport:
    rows: int = 0
    exact: int = 0
    boundary_rows: int = 0
    boundary_mismatches: int = 0
    failures: list = field(default_factory=list)

    def ok(self) -> bool:
        return not self.failures


def compare(out, oracle_rows, params_list, *, tol: float = 1e-5, probs=None, check_top: bool = True) -> ParityReport:
    """Row-by-row parity of a GPU call against oracle rows (uniform mode).

    * Token ids must be equal; a sampled row may differ only if the oracle classes it
      as a boundary row: the top-p cut within ``1e-6 + |delta|`` of p (``delta`` is the
      reference's own normalisation error), a value tie across the top-p cut, or the
      CDF step within 1e-6.
    * The kept count must equal the reference's when no boundary applies, and must
      equal the exact (float64) top-p cut's unless that cut is within 1e-6 of p.
    * With the same token and kept set: logprobs within ``tol`` (relative, floor 1) of
      the exact (float64) log-softmax of the final scores, and within ``tol + eps`` of
      the reference's, where ``eps`` is the reference's own fp32 log-normaliser error
      on that row; top-N lists equal up to ties within ``tol + eps``; probabilities
      (if given) within ``tol + |delta| + eps`` relative."""
    rep = ParityReport()
    for b, (o, p) in enumerate(zip(oracle_rows, params_list)):
        rep.rows += 1
        tok = int(out.tokens[b])
        rep.boundary_rows += int(o.boundary)
        kept = int(out.info['kept'][b]) if out.info is not None else None
        if kept is not None and not o.greedy:
            if o.topp_exact_kept is not None and o.topp_exact_margin >= 1e-6 and kept != o.topp_exact_kept:
                rep.failures.append(f'row {b}: kept {kept} != exact top-p cut {o.topp_exact_kept}')
            margin_row = o.topp_margin < 1e-6 + o.topp_norm_error
            if not margin_row and kept != o.kept:  # ties (class ii) keep the count too
                rep.failures.append(f'row {b}: kept {kept} != oracle {o.kept}')
        if tok != o.token_id:
            if o.boundary and not o.greedy:
                rep.boundary_mismatches += 1
                continue
            rep.failures.append(f'row {b}: token {tok} != oracle {o.token_id} (greedy={o.greedy}, '
                                f'topp_margin={o.topp_margin:.3g}, cdf_margin={o.cdf_margin:.3g})')
            continue
        rep.exact += 1
        if kept is not None and not o.greedy and kept != o.kept:
            continue  # the reference's rounding moved its cut: normalisers differ by design
        lp = float(out.logprobs[b])
        if not close(lp, o.logprob, tol + o.lse_error):
            rep.failures.append(f'row {b}: logprob {lp!r} != oracle {o.logprob!r}')
        elif not math.isnan(o.exact_logprob) and not close(lp, o.exact_logprob, tol):
            rep.failures.append(f'row {b}: logprob {lp!r} != exact {o.exact_logprob!r}')
        if check_top and p.logprobs:
            got = out.top(b, p.logprobs)
            if not top_matches(got, list(o.top_logprobs), tol + o.lse_error, cut_tie=o.topp_tie):
                rep.failures.append(f'row {b}: top logprobs {got[:4]}... != oracle {list(o.top_logprobs)[:4]}...')
        if probs is not None and o.probs is not None and not o.boundary:
            # probabilities below 1e-30 are compared as zero: fp32 softmax values that
            # small carry little relative precision in the reference; one side above 2e-30
            # and the other at or below 1e-30 is a support difference
            want = o.probs.numpy().astype(np.float64)
            got = probs[b].astype(np.float64)
            ptol = tol + o.topp_norm_error + o.lse_error
            split = ((want > 2e-30) & (got <= 1e-30)) | ((got > 2e-30) & (want <= 1e-30))
            if split.any():
                rep.failures.append(f'row {b}: kept support differs ({int((want > 1e-30).sum())} vs '
                                    f'{int((got > 1e-30).sum())})')
            else:
                m = (want > 2e-30) & (got > 2e-30)
                rel = np.abs(got[m] - want[m]) / want[m]
                if rel.size and rel.max() > ptol:
                    rep.failures.append(f'row {b}: probability rel err {rel.max():.3g}')
    return rep
