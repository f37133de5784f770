"""CPU oracle for the token-sampling hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package (``chenxing_amd``)
imports, calls or links anything under ``oracle/``; only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may,
and there only as the checker (or, in ``bench.py``, as the timed CPU baseline).

The oracle is a batched NumPy restatement of the reference's algorithm with
the random variates made explicit (the uniforms are arguments instead of
``Generator`` draws):

* :mod:`oracle.sampler_ref`  -- ``chenxing/core/sampler.py:63-127``
  (penalties, greedy, softmax + temperature, top-k / top-p / min-p /
  typical-p, inverse-CDF draw), plus the build-defined presence/frequency
  penalty, which reduces to the reference when both are 0.
* :mod:`oracle.speculative_ref` -- ``chenxing/engine/speculative.py:67-69``
  (``_softmax``) and ``:145-171`` (Leviathan accept/reject and the residual
  ``max(0, p - q)`` resample).
* :mod:`oracle.lmhead_ref` -- ``chenxing/model/transformer.py:102-104``
  (``x @ out_w.T``) on bf16 operands with exact products, then the greedy
  argmax of ``sampler.py:114-115``; with the device's accumulation bound.
* :mod:`oracle.bf16` -- exact bf16 <-> fp32 conversion (round to nearest even).

How each function is pinned (closed forms, the reference's own known-answer
tests, golden vectors written by importing the reference in the build
container, numpy behaviour pins and brute force) is listed in each module's
docstring and enforced by ``tests/test_oracle_*.py``.
"""
