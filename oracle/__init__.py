"""CPU oracle for the EXL3 trellis linear and grouped-MoE path.

TEST INFRASTRUCTURE ONLY. Nothing in the product package imports this directory. Only `tests/`,
`__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` may load it, and only as the checker or as the
timed CPU baseline, never as a fallback for the HIP path.
"""
