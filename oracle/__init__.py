"""CPU oracle for the token-sampling path.

TEST INFRASTRUCTURE ONLY. Nothing in the product (the ``klsample`` package, its HIP
library or its C ABI) imports, links or calls this package. Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` use it, and
there only to check results (or as the timed CPU baseline), never as the path
measured or shipped.

``oracle.cpu_sampler`` restates the reference sampler (``serving/sampling.py:44-63``)
with the same PyTorch CPU operations, in two modes:

* ``uniform``: line 60's ``torch.multinomial`` is replaced by an inverse CDF on a
  caller-supplied uniform (the parity mode);
* ``faithful``: ``torch.multinomial`` with the request's seeded generator (the CPU
  baseline mode).

Pinning (what checks each function):

* ``restated_sample`` greedy branch, repetition penalty, temperature, top-k, top-p,
  log-softmax and top-logprobs: the reference's own known-answer test
  (``serving/test_serving.py:101-107``), the vectors in
  ``tests/golden/reference_vectors.json`` written by running the reference sampler
  in the build container, and closed-form checks (brute-force order statistics,
  exact descending-prefix mass, IEEE fp32 division) in ``tests/test_oracle.py``.
* presence / frequency penalties: no reference counterpart. Pinned by the closed
  form ``s - fp32(fp32(beta*count) + alpha)``, by brute-force counts on tiny
  histories, and by the invariant ``alpha == beta == 0`` reproduces the reference.
* ``inverse_cdf``: the build's own definition (no reference counterpart); pinned by
  brute force against a pure-Python loop and by its monotonicity in ``u``.
"""
