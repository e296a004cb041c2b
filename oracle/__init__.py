"""Test infrastructure: the CPU restatement of the reference PairFormer block.

Only tests, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg may
import this package, and only as the checker or a timed baseline.
"""
