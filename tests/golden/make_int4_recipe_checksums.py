"""Writes int4_recipe_checksums.json: i16-sum checksums (as i32) of C = A x B for
the reference int4 benchmark's deterministic packed inputs
    A[i,k] = ((i*N + k) % 15) - 7 packed along k,  B[k,j] = ((j*N + k) % 15) - 7
    packed along j  (simptensor/benchmarks/bench_int4_matmul_runner.cpp:76-143).

Sizes 32, 64, 128 come from the reference's own packed_matmul_int4<N> and
scalar_matmul_int4<N> (both must agree), compiled in place by `make -C oracle
ref`.  Larger and odd sizes come from the oracle's restatement of the lowering
(ConvertSimpToMemRef.cpp:2953-3133), which equals the reference at every size
both cover.  Run here, where the reference is mounted:
    python tests/golden/make_int4_recipe_checksums.py
"""
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))
import oracle  # noqa: E402

out = {"recipe": "A[i,k]=((i*N+k)%15)-7 packed along k; B[k,j]=((j*N+k)%15)-7 packed along j; "
                 "C = i16(sum_k A*B); checksum = i32 sum of C",
       "checksums": {}, "source": {}}
for n in (32, 64, 128, 33, 255, 512, 1024):
    ap, bp = oracle.int4_recipe_inputs(n)
    mine = oracle.checksum_i16(oracle.matmul_i4(ap, bp, n, n, n))
    if oracle.ref is not None and n in (32, 64, 128):
        ref = getattr(oracle.ref, f"ref_packed_int4_{n}")()
        assert ref == getattr(oracle.ref, f"ref_scalar_int4_{n}")() == mine, n
        src = "reference packed_matmul_int4"
    else:
        src = "oracle orc_matmul_i4"
    out["checksums"][str(n)] = mine
    out["source"][str(n)] = src
    print(n, mine, src, flush=True)
json.dump(out, open(os.path.join(HERE, "int4_recipe_checksums.json"), "w"), indent=1)
