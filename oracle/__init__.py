"""CPU oracle: a from-scratch restatement of nanoserve's PyTorch path for the decode token loop.

TEST INFRASTRUCTURE ONLY. Nothing in the product package (nanoserve_amd/) imports this package; only
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg do, and only as the checker (or, for
cpu_baseline, as the timed CPU restatement), never as the thing measured on the GPU.

Modules:
  ops     unfused token-wise ops, RoPE tables, gather+SDPA paged attention, fp64 brute force
  model   fp32/bf16 CPU Qwen2 forward (unfused, SDPA), paged KV, greedy generation

Each function cites the reference file:line it restates (darshanseenivasakumar/nanoserve). How each one is
pinned (HF transformers modules built locally, closed forms, fp64 brute force, known answers from the
reference's own tests) is in tests/test_oracle_*.py.
"""
