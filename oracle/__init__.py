"""CPU checker for the vnx MI355X kernels — TEST INFRASTRUCTURE ONLY.

Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of
`bench.py` may import this package, and only as the checker (or the timed CPU
baseline), never as the product path: `versenext_amd` never imports it.

Modules
-------
- `speculative`: the reference's greedy verify / commit (restated from
  packages/verse_nex/verse_nex/speculative.py) and the stochastic acceptance
  rule (Leviathan et al. 2023, arXiv:2211.17192, Alg. 1) in the exact
  arithmetic the kernels are specified to use.
- `rows`: temperature scaling, row softmax / log-sum-exp, argmax, top-k
  threshold (device.py:305-308, sampler.py:94-111).
- `_clib`: ctypes binding of `canon.c` (canonical exp, exact inverse-CDF).

Pinning status of each function is stated in its docstring and in the tests
under tests/test_oracle_*.py.
"""
