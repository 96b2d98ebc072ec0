"""CPU restatement of the reference sampler, used as the parity oracle.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

The reference (``serving/sampling.py:44-63``) processes one row per call with stock
PyTorch CPU operations.  This module runs the same operations in the same order,
so that on the same fp32 inputs it produces the same scores bit for bit, and adds:

* presence and frequency penalties, which the reference lacks (its
  ``SamplingParams`` stops at ``logprobs``, ``serving/sampling.py:8-15``), applied
  after the repetition penalty over the same history;
* ``uniform`` mode, where the multinomial draw (``serving/sampling.py:60``) becomes
  an inverse CDF on a caller-supplied uniform ``u``;
* per-row diagnostics that classify a row as a *boundary row* (the top-p crossing or
  the CDF step lies within ``1e-6`` of the cut), which is the only class of row whose
  token id may differ from a GPU implementation;
* an exact evaluation of the top-p cut (float64 weights and cumulative sum over the
  same sorted order);
* ``stable`` tie order: the reference sorts with an unstable ``sort``
  (``serving/sampling.py:57``) and takes its top-N with ``topk`` (``:62``), so which of
  several equal scores is kept at the top-p cut, and the order of equal top-N entries,
  are implementation-defined there.  With ``stable=True`` equal scores are taken in
  ascending index order in both places, the top-N list is ordered by final score (two
  scores one ulp apart can share an fp32 logprob), and top-N slots past the kept set
  list the smallest ids whose final score is ``-inf``.  The kept *count*, every probability and
  every logprob are the reference's; only the identities among equal scores are fixed.  The reference's fp32 ``softmax`` over a 151,936-entry row sums
  to ``1 + delta`` with ``|delta|`` up to ~3e-5 (measured: the last element of its own
  ``cumsum``), so its cut can differ from the exact one by a few tokens; the top-p
  boundary band is therefore ``1e-6 + |delta|`` wide, and implementations are also
  checked against the exact cut with the 1e-6 band.

PyTorch facts this restatement relies on (probed on the installed torch CPU build):
``tensor / python_float`` is IEEE fp32 division by ``fp32(value)``;
``tensor * python_float`` multiplies by ``fp32(value)``; ``tensor > python_float``
compares against ``fp32(value)``; ``cumsum`` on fp32 accumulates in double and
rounds each element to fp32.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np
import torch

BOUNDARY_EPS = 1e-6


@dataclass
class OracleRow:
    """Result of one restated ``Sampler.sample`` call plus diagnostics."""

    token_id: int
    logprob: float
    top_logprobs: tuple
    stopped: bool
    greedy: bool
    probs: torch.Tensor | None = None      # vector handed to the draw (sampled rows)
    scores: torch.Tensor | None = None     # final scores (after penalties, T, top-k/p)
    kept: int = 0                          # number of finite final scores
    exact_probs: np.ndarray | None = None  # float64 softmax of the final scores (sampled rows)
    pre_topp: torch.Tensor | None = None   # scores entering the top-p step (top_p < 1 rows)
    topp_exact_cut: tuple | None = None    # (score, index) of the last entry the exact cut keeps
    # boundary classification (sampled rows only)
    topp_margin: float = math.inf          # |excl_cumsum - p| nearest the cut (reference arithmetic)
    topp_norm_error: float = 0.0           # |sum of the reference's top-p probabilities - 1|
    topp_tie: bool = False                 # a value tie straddles the top-p cut
    topp_exact_kept: int | None = None     # kept count of the exact (float64) top-p cut
    topp_exact_margin: float = math.inf    # |exact excl - p| nearest the exact cut
    cdf_margin: float = math.inf           # |cdf step - u*Z| / Z nearest the token
    # the final log-softmax in exact arithmetic (float64 over the same fp32 final scores)
    exact_logprob: float = math.nan        # of the token
    lse_error: float = 0.0                 # |the reference's fp32 log-normaliser - the exact one|
    notes: list = field(default_factory=list)

    @property
    def margin_row(self) -> bool:
        """The top-p decision lies within 1e-6 of p, widened by the reference's own fp32
        normalisation error ``delta``: its cut may then fall one entry away from the
        exact (float64) cut."""
        return self.topp_margin < BOUNDARY_EPS + self.topp_norm_error

    @property
    def cdf_row(self) -> bool:
        """``u * Z`` lies within 1e-6 (relative) of a CDF step next to the token."""
        return self.cdf_margin < BOUNDARY_EPS

    @property
    def boundary(self) -> bool:
        """A row whose token id may differ from an implementation's: a top-p mass margin
        or a CDF-step margin.  A value tie across the cut is not one: with ``stable`` tie
        order the kept identities are fixed (ascending index)."""
        return self.margin_row or self.cdf_row

    def in_kept(self, token: int) -> bool:
        """Whether ``token`` is kept by this row's final scores or by the exact top-p cut."""
        if self.scores is not None and math.isfinite(float(self.scores[token])):
            return True
        if self.pre_topp is None or self.topp_exact_cut is None:
            return False
        s = float(self.pre_topp[token])
        cs, ci = self.topp_exact_cut
        return s > cs or (s == cs and token <= ci)


def normalize_history(history, vocab: int) -> np.ndarray:
    """History ids as int64 in ``[0, vocab)``.

    The reference indexes ``scores[ids]`` with the raw ids
    (``serving/sampling.py:48-49``): a negative id counts from the end, and an id
    outside ``[-vocab, vocab)`` raises ``IndexError``.
    """
    ids = np.asarray(list(history), dtype=np.int64).reshape(-1)
    if ids.size and (ids.min() < -vocab or ids.max() >= vocab):
        bad = ids[(ids < -vocab) | (ids >= vocab)][0]
        raise IndexError(f'index {int(bad)} is out of bounds for dimension 0 with size {vocab}')
    return np.where(ids < 0, ids + vocab, ids)


def inverse_cdf(probs: torch.Tensor, u: float) -> int:
    """Smallest vocab index ``i`` with ``sum(probs[:i+1]) > u * sum(probs)``.

    Replaces ``torch.multinomial(probs, 1, generator)`` (``serving/sampling.py:60``)
    with a draw driven by one caller-supplied uniform ``u`` in ``[0, 1)``.  The
    cumulative sum runs in float64 in vocab order.  If rounding leaves no index
    above the target, the last index with non-zero probability is returned.
    """
    p = probs.detach().double().numpy()
    c = np.cumsum(p)
    target = float(u) * c[-1]
    i = int(np.searchsorted(c, target, side='right'))
    if i >= p.size:
        i = int(np.flatnonzero(p > 0)[-1])
    return i


def _apply_penalties(scores: torch.Tensor, ids: np.ndarray, params) -> None:
    """Repetition penalty (``serving/sampling.py:47-49``), then presence/frequency."""
    r = params.repetition_penalty
    if r != 1 and ids.size:
        # serving/sampling.py:48 builds the sorted distinct ids; after normalising
        # negative ids the duplicates collapse to the same element, which the
        # reference also updates once (every copy writes the same value).
        uniq = torch.from_numpy(np.unique(ids))
        sel = scores[uniq]
        scores[uniq] = torch.where(sel < 0, sel * r, sel / r)
    a = getattr(params, 'presence_penalty', 0.0)
    b = getattr(params, 'frequency_penalty', 0.0)
    if (a != 0 or b != 0) and ids.size:
        uniq, counts = np.unique(ids, return_counts=True)
        idx = torch.from_numpy(uniq)
        # closed form, three fp32 roundings, no fused multiply-add:
        #   t = fp32(beta * count); t = fp32(t + alpha); s = fp32(s - t)
        t = torch.from_numpy(counts.astype(np.float32)) * b
        t = t + a
        scores[idx] = scores[idx] - t


def restated_sample(logits: torch.Tensor, history=(), params=None, *, u: float | None = None,
                    generator: torch.Generator | None = None, diagnostics: bool = True,
                    stable: bool = False) -> OracleRow:
    """One reference ``Sampler.sample`` call (``serving/sampling.py:44-63``).

    ``u`` selects uniform mode (inverse CDF); otherwise ``generator`` drives
    ``torch.multinomial`` exactly as the reference does.  ``stable`` fixes the order of
    equal scores (ascending index) in the top-p sort and the top-N list.
    """
    if logits.ndim != 1 or not logits.is_floating_point():        # :45
        raise ValueError('logits must be a floating vector')
    p = params
    scores = logits.detach().to('cpu').float().clone()             # :46
    vocab = scores.numel()
    ids = normalize_history(history, vocab)
    _apply_penalties(scores, ids, p)                               # :47-49 (+ presence/frequency)
    row = OracleRow(0, 0.0, (), False, p.temperature == 0)
    if p.temperature == 0:                                         # :50-51
        token = int(scores.argmax())
    else:
        scores /= p.temperature                                    # :53
        if p.top_k:                                                # :54-55
            k = min(p.top_k, vocab)
            cutoff = scores.topk(k).values[-1]
            scores.masked_fill_(scores < cutoff, -torch.inf)
        if p.top_p < 1:                                            # :56-59
            if diagnostics:
                row.pre_topp = scores.clone()
            ordered, index = scores.sort(descending=True, stable=stable)
            probabilities = ordered.softmax(0)
            cumulative = probabilities.cumsum(0)
            excl = cumulative - probabilities
            remove = excl > p.top_p
            if diagnostics:
                _topp_diagnostics(row, ordered, index, excl, remove, p.top_p, float(cumulative[-1]))
            scores[index[remove]] = -torch.inf
        probs = scores.softmax(0)                                  # :60
        row.probs = probs
        if u is not None:
            token = inverse_cdf(probs, u)
            if diagnostics:
                _cdf_diagnostics(row, probs, token, u)
        else:
            token = int(torch.multinomial(probs, 1, generator=generator))
    log_probabilities = scores.log_softmax(0)                      # :61
    count = min(p.logprobs, vocab)
    if not count:
        top = ()
    elif stable:
        # ordered by final score, equal scores in index order (two distinct scores may
        # round to one fp32 logprob; the score still orders them); past the kept set the
        # -inf entries in index order are the smallest ids not listed before them
        order = scores.sort(descending=True, stable=True).indices[:count]
        top = tuple((int(a), float(log_probabilities[a])) for a in order)
    else:
        top = tuple((int(i), float(v)) for v, i in zip(*log_probabilities.topk(count)))   # :62
    row.token_id = token
    row.logprob = float(log_probabilities[token])                  # :63
    if diagnostics:
        _lse_diagnostics(row, scores, token)
        if p.temperature != 0:
            s = scores.double().numpy()
            fin = np.isfinite(s)
            ep = np.zeros_like(s)
            if fin.any():
                m = s[fin].max()
                e = np.exp(s[fin] - m)
                ep[fin] = e / e.sum()
            row.exact_probs = ep
    row.top_logprobs = top
    row.stopped = token in p.stop_token_ids
    row.scores = scores
    row.kept = int(torch.isfinite(scores).sum()) if p.temperature != 0 else vocab
    return row


def _topp_diagnostics(row: OracleRow, ordered, index, excl, remove, top_p, total: float) -> None:
    """Distance of the top-p decision from its cut, the reference's normalisation
    error, ties across the cut, and the exact (float64) cut over the same order."""
    p32 = float(np.float32(top_p))            # torch compares against fp32(top_p)
    e = excl.double().numpy()
    rm = remove.numpy()
    n = e.size
    first_removed = int(np.argmax(rm)) if rm.any() else n
    margins = []
    for j in (first_removed - 1, first_removed):
        if 0 <= j < n and np.isfinite(ordered[j].item()):
            margins.append(abs(e[j] - p32))
    row.topp_margin = min(margins) if margins else math.inf
    if 0 < first_removed < n:
        row.topp_tie = bool(ordered[first_removed - 1].item() == ordered[first_removed].item())
    # the reference's probabilities are scaled by (1 + delta); its last cumsum entry is 1 + delta
    o = ordered.double().numpy()
    w = np.exp(o - o[0]) if np.isfinite(o[0]) else np.zeros_like(o)
    z = w.sum()
    if z > 0:
        ex = (np.cumsum(w) - w) / z
        row.topp_norm_error = abs(total - 1.0)
        keep = ex <= p32
        row.topp_exact_kept = int(keep.sum())
        cut = row.topp_exact_kept
        if cut > 0:
            row.topp_exact_cut = (float(o[cut - 1]), int(index[cut - 1]))
        em = [abs(ex[j] - p32) for j in (cut - 1, cut) if 0 <= j < n and w[j] > 0]
        row.topp_exact_margin = min(em) if em else math.inf


def _lse_diagnostics(row: OracleRow, scores, token: int) -> None:
    """The token's log-softmax in float64 over the final fp32 scores, and how far the
    reference's fp32 log-normaliser (``scores[token] - logprob``) lies from the exact
    one: over ~10^5 entries its fp32 sum carries a relative error of ~1e-5."""
    s = scores.double().numpy()
    fin = np.isfinite(s)
    if not fin.any() or not np.isfinite(s[token]):
        return
    m = s[fin].max()
    lse = m + math.log(np.exp(s[fin] - m).sum())
    row.exact_logprob = float(s[token] - lse)
    if math.isfinite(row.logprob):
        row.lse_error = abs((float(s[token]) - row.logprob) - lse)


def _cdf_diagnostics(row: OracleRow, probs, token: int, u: float) -> None:
    """Relative distance of ``u * Z`` from the CDF steps around the chosen token."""
    c = np.cumsum(probs.double().numpy())
    z = c[-1]
    target = float(u) * z
    steps = [c[token]]
    if token > 0:
        steps.append(c[token - 1])
    row.cdf_margin = min(abs(s - target) for s in steps) / z


def sample_rows(logits2d: torch.Tensor, histories, params_list, uniforms=None,
                generators=None, diagnostics: bool = True, stable: bool = True) -> list[OracleRow]:
    """Row loop over a ``[B, V]`` batch, one reference call per row (as
    ``serving/engine.py:92-96`` calls the sampler once per request row).  Parity uses
    the stable tie order by default (see ``restated_sample``)."""
    out = []
    for b in range(logits2d.shape[0]):
        u = None if uniforms is None else float(uniforms[b])
        g = None if generators is None else generators[b]
        out.append(restated_sample(logits2d[b], histories[b] if histories is not None else (),
                                   params_list[b], u=u, generator=g, diagnostics=diagnostics,
                                   stable=stable))
    return out
