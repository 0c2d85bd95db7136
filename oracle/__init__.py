"""CPU restatement of the reference's INT8-attention / GGUF k-quant hot path (numpy).

TEST INFRASTRUCTURE ONLY. Nothing in the product package imports this; only
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, as the
checker (never as the thing measured on the GPU or shipped).

Every function cites the reference file:line it restates. How each function is
pinned (known answers, closed forms, brute force, invariants) is listed in
tests/test_oracle.py; no function here is left unpinned.
"""
from . import attention, kquant, lloydmax, q4k, quant  # noqa: F401
