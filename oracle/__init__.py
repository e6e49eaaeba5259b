"""CPU oracle of the Dion optimizer step — TEST INFRASTRUCTURE ONLY.

A restatement, on host cores (torch CPU ops and numpy), of the reference's
PyTorch/Triton path for ``dionw.Dion(...).step()``: the momentum passes, row
selection, Gram / standard / quintic Newton-Schulz with the reference's
float16 / bfloat16 rounding points, NorMuon, the weight update, fused AdamW
and the EMA. Each function cites the reference file:line it follows.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import this package, and only as the checker (or the timed CPU
baseline); the product (``dionw_amd``) never does.

How each part is pinned (beyond agreeing with the HIP kernels) is listed in
``tests/test_oracle.py``: closed forms (the float64 polynomial and the exact
SVD polar factor), brute-force float64 sums, torch's own CPU ``_fused_adamw_``
and ``lerp``, and the reference's known-answer tables.
"""
