"""CPU oracle for the MI355X Muon step — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the arithmetic of the reference's hot path
(tonyf/dtensor-muon, package ``muonium`` 0.2.0): the Newton-Schulz / Polar Express
iteration, the Muon / NorMuon update rules, the per-parameter and foreach drivers, and
the blockwise quantizers of the low-precision momentum state. Every function cites the
reference file:line it follows.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg
may import it, and only as the checker (or as the CPU baseline that is timed). The
product package (``dtensor-muon_amd/muonium_amd``) never imports, calls or links
anything here.

Pinning status (what fixes each function independently of its own formula):

* ``muon_ref.polar_iteration`` / ``pe_loop`` / ``ns_loop``: the reference's own
  property tests (orthogonality, SVD closeness, steps=0 prescale, manual one-step
  expansion with overridden coefficients, transpose symmetry, zero/rank-1 inputs,
  orthogonal fixed point, scale invariance, batched == unbatched) and the fp64 run of
  the same iteration.
* ``muon_ref.muon_update`` / ``split_*``: the closed-form known answers of the
  reference tests (test_optim.py:392-584, test_algorithms.py:315-393).
* ``muon_ref.normuon_normalize`` / ``normuon_update``: invariants of the method
  (Frobenius norm preserved, equal row norms from a zero variance, the EMA's fixed
  point, the same per split_sizes row block) and the known answers of
  test_algorithms.py:174-259; ``normuon_update``'s composition (normalize, then cautious
  wd on the normalized update, then the apply, normuon.py:118-134) by a 3 x 2 case worked
  by hand, which the other order fails.
* ``quant_ref``: the quantized-state arithmetic lives in torchao 0.17.0, which is not
  present here; the restatement follows torchao's published algorithm and is pinned
  by brute-force nearest-code search, map structure, round-trip error bounds and
  torch's own float8_e4m3fn cast. ``lp_momentum_step`` (muon.py:45-56 through the
  quantized state) by hand-worked cases for each format: Nesterov's input from the
  unquantized m', codes of m' by brute-force nearest code, and the next step starting
  from the dequantized state, with a block where requantization is lossy so the two
  readings differ. Bit parity with torchao itself is UNPINNED.
"""
