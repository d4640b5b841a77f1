"""Writes int8_recipe_checksums.json: i32 checksums of C = A x B for the
reference benchmark's deterministic inputs
    val = ((i*N + j) % 127) - 64;  A[i,j] = B[j,i] = val
(simptensor/benchmarks/bench_int8_matmul_runner.cpp:33-64).

Sizes 64..2048 that the reference's own vnni_matmul_single_thread<N>
(simptensor/benchmarks/bench_int8_matmul_multicore.cpp:39-89) is instantiated
for come from it, compiled in place by `make -C oracle ref`.  The other sizes
benchmark_int8_matmul_<N> defines (32, 384, 768, 4096:
simptensor/benchmarks/bench_int8_matmul.sl:11-335) come from the oracle's VNNI
restatement, which equals the reference kernel bit for bit at every size both
cover.  Run here, where the reference
is mounted:  python tests/golden/make_int8_recipe_checksums.py
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))
import oracle  # noqa: E402

out = {"recipe": "val=((i*N+j)%127)-64; A[i,j]=B[j,i]=val; checksum = i32 wraparound sum of C",
       "checksums": {}, "source": {}}
ref = oracle.load_ref()
for n in (32, 64, 128, 256, 384, 512, 768, 1024, 2048, 4096):
    a, b = oracle.recipe_inputs(n)
    if ref is not None and n in (64, 128, 256, 512, 1024, 2048):
        bt = np.ascontiguousarray(b.T)
        c = np.zeros((n, n), np.int32)
        getattr(ref, f"ref_vnni_matmul_{n}")(a.ctypes.data, bt.ctypes.data, c.ctypes.data)
        src = "reference vnni_matmul_single_thread"
        c2, _ = oracle.matmul_i8_vnni(a, b, nthreads=8)
        assert (c2 == c).all(), n
    else:
        c, _ = oracle.matmul_i8_vnni(a, b, nthreads=8)
        src = "oracle orc_matmul_i8_vnni"
    out["checksums"][str(n)] = oracle.checksum_i32(c)
    out["source"][str(n)] = src
    print(n, out["checksums"][str(n)], src, flush=True)
json.dump(out, open(os.path.join(HERE, "int8_recipe_checksums.json"), "w"), indent=1)
