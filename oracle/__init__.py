"""CPU oracle for the quantized DiT attention path (test infrastructure only).

Nothing in the shipped package imports this directory. Only `tests/`, `__graft_entry__.smoke()` and the
`cpu_baseline` leg of `bench.py` use it, and only as the checker / the timed CPU baseline.
"""
