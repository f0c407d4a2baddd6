"""Test infrastructure: CPU oracles for the attention hot path.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package, and only as the checker (never as the thing
measured or shipped). ``attention`` is the float64 brute force + closed-form
backward; ``cpu_path`` is the reference's own CPU attention path, timed as the
CPU baseline.
"""
