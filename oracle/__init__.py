"""CPU checker for the CDA hot path (test infrastructure only).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import this package, and only as the checker; ``sub0_amd`` never
imports it.
"""
