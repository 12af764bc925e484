"""ORACLE — test infrastructure only.

CPU restatements of the reference (poseidonchan/MPQ) algorithms on the
per-layer quantization path.  Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg may import anything here, and only as the
checker or as the timed CPU baseline; the product (``mpq_amd``) never does.
Every function names the reference file:line it follows.  Functions whose
result no golden vector, closed form or brute force pins say "parity
unpinned" in their docstring.
"""
