"""CPU oracle for the VecMarket matching path (test infrastructure only).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package, and only as the checker or the timed CPU baseline.
"""
