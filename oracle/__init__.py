"""CPU oracle for miniserve's paged-attention path -- TEST INFRASTRUCTURE ONLY.

This package restates, in plain torch / numpy on the CPU, the algorithms of
the reference's paged-attention hot path:

  paged_sdpa  PagedAttention.build_mask / _gather / write_kv / forward
              (miniserve/attention.py:111-250): the SDPA path, which is also
              the CPU baseline that bench.py times ("kind": "port").
  dense       float64 closed-form masked-softmax attention over the gathered
              rows (pattern of tests/test_parity.py:99-117): the numerical
              truth the HIP kernels are compared against.
  split_k     the split-K decomposition and log-sum-exp merge of
              kernels/paged_attn_triton.py:80-171.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import it, and only as the checker; the product (miniserve_amd) never does.
Each function is pinned by the checks in tests/test_oracle.py (known-answer
tests from the reference's tests, closed forms, invariants and brute force).
"""
