"""CPU oracle for the per-layer LLM kernels -- TEST INFRASTRUCTURE ONLY.

This package restates, in plain PyTorch on the CPU, the arithmetic of the
reference's own torch spellings of each kernel (jingchangshi/TileFoundry,
``examples/qwen3_1_7b-tilelang/fast/test_kernels.py``,
``examples/minicpm3_4b-cutedsl/kernels/reference_ops.py``) and of the authored
HIR models they are checked against. Every function cites the reference file
and lines it follows.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg
may import it, and only as the checker. The product path (``tilefoundry_amd``)
never imports it and has no CPU fallback.

Pinning (how each function is checked independently of its own formula) is
listed in each module's docstring; ``tests/test_oracle.py`` holds the checks.
"""
