"""CPU oracle for the attention hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the naive PyTorch paths that the reference
repository (KiritoHugh/attention_kernel_triton) uses to check its kernels, plus
the kept-index selection of its test harness.  It exists to check the HIP
kernels; it is never shipped as, or called by, the product: only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg import it.

Modules:
  naive  -- attention restatements (prefill, var-len prefill, decode, paged,
            sparse, sparse paged, MagicPIG) with log-sum-exp outputs
  kept   -- kept-token index selection and page-table addressing (integer work)

Pinning (how each function is checked independently of its own formula) is
listed in the module docstrings and exercised by tests/test_oracle_*.py.
"""
