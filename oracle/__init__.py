"""CPU oracle for the soft-triangle rasterizer — test infrastructure only.

`oracle.oracle` wraps `liboracle.so` (a plain-C restatement of the reference's
CPU algorithm, built by `oracle/Makefile`) with numpy in/out. Only `tests/`,
`__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` use it, to
check the GPU results against; the product package never imports anything from here.
"""
