"""TEST INFRASTRUCTURE ONLY: CPU oracles for the MI355X hot path.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this package, and only as the checker or as the reported CPU baseline. The
product (open-pacho_amd/openpacho and libpacho_hip.so) never imports, calls
or links anything here; a product path that did would void its parity claims.

Contents (each function cites the reference file:line it restates):
- philox:        Philox4x32-10 stream + distribution transforms
                 (reference _random.py:19-58), NumPy and C (philox_oracle.c).
- numpy_backend: the reference NumPy backend's matmul / two-pass norm / RNG
                 (backends.py:86-150, _norm.py:44-52), the reported CPU baseline.
- kernels:       bit-exact restatements of the reference CUDA custom kernels'
                 arithmetic order (GEMM sequential-K, GEMV 128-lane + tree,
                 DOT chunks, scaled-norm pair merge, reduce), giving the
                 "reference custom-kernel error" the parity bar is scaled by.
- exact:         exact (dyadic integer) and extended-precision references.
- padding:       closed-form padding plan metadata (_padding.py:80-109).

Pinning of each oracle function is recorded in tests/test_oracle_*.py; a
function without such a check is marked "parity unpinned" in its docstring.
"""
