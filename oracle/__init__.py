"""CPU oracle for the W4A16 GEMM -- test infrastructure only.

Importable by ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg.
The product path (``w4a16-gemm_amd/``) never imports it.
"""
