"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the checker.

Each test checks the oracle against something other than its own formula:
the reference's known answers, the reference's own code compiled in place
(oracle/_ref, only where the SimpLang sources are mounted), exact library
arithmetic (numpy int64 / float64), closed forms and invariants.
"""
import numpy as np
import pytest

RNG = np.random.default_rng(1234)


def _i64_matmul_wrap(a, b):
    """Exact int64 product wrapped to i32, the reference's accumulator width."""
    return (a.astype(np.int64) @ b.astype(np.int64)).astype(np.int32)


# --------------------------------------------------------------- vpdpbusd --
# Known answers of simptensor/tests/test_vnni_correctness.cpp:76-361.

def test_vpdpbusd_kats(orc):
    z16 = np.zeros(16, np.int32)
    assert (orc.vpdpbusd16(np.zeros(64), np.zeros(64), z16) == 0).all()
    assert (orc.vpdpbusd16(np.ones(64), np.ones(64), z16) == 4).all()
    assert (orc.vpdpbusd16(np.full(64, 255), np.full(64, 127), z16) == 129540).all()
    assert (orc.vpdpbusd16(np.full(64, 255), np.full(64, -128), z16) == -130560).all()
    acc = np.arange(16, dtype=np.int32) * 1000
    out = orc.vpdpbusd16(np.full(64, 10), np.full(64, 5), acc)
    assert (out == np.arange(16) * 1000 + 200).all()
    out = orc.vpdpbusd16(np.full(64, 200), np.full(64, 100), np.full(16, 2000000000, np.int32))
    assert (out == 2000080000).all()


def test_vpdpbusd_mixed_and_accumulate(orc):
    i = np.arange(64)
    a = (i + 1).astype(np.uint8)
    b = np.where(i % 2 == 0, i + 1, -(i + 1)).astype(np.int8)
    exp = (a.astype(np.int64) * b.astype(np.int64)).reshape(16, 4).sum(1)
    assert (orc.vpdpbusd16(a, b, np.zeros(16, np.int32)) == exp).all()
    # four accumulation steps (test_vnni_matmul_pattern)
    a = ((i % 16) + 1).astype(np.uint8)
    b = ((i // 16) + 1).astype(np.int8)
    acc = np.zeros(16, np.int32)
    for _ in range(4):
        acc = orc.vpdpbusd16(a, b, acc)
    assert (acc == 4 * (a.astype(np.int64) * b).reshape(16, 4).sum(1)).all()


def test_vpdpbusd_random_vs_reference(orc):
    for _ in range(200):
        a = RNG.integers(0, 256, 64).astype(np.uint8)
        b = RNG.integers(-128, 128, 64).astype(np.int8)
        acc = RNG.integers(-2**30, 2**30, 16).astype(np.int32)
        got = orc.vpdpbusd16(a, b, acc)
        exp = (acc.astype(np.int64) + (a.astype(np.int64) * b).reshape(16, 4).sum(1))
        assert (got == exp.astype(np.int32)).all()
        if orc.load_ref() is not None:
            ref = np.empty(16, np.int32)
            orc.load_ref().ref_scalar_vpdpbusd(a.ctypes.data, b.ctypes.data, acc.ctypes.data,
                                        ref.ctypes.data)
            assert (got == ref).all()


def test_reference_vnni_binary_passes(orc):
    """The reference's own KAT program, built in place, passes on this host."""
    import os
    import subprocess
    if not os.path.exists(orc.REF_VNNI_TEST):
        pytest.skip("reference not built here")
    flags = open("/proc/cpuinfo").read()
    if "avx512_vnni" not in flags:
        pytest.skip("host lacks AVX-512 VNNI")
    out = subprocess.run([orc.REF_VNNI_TEST], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0 and "Passed: 9/9" in out.stdout


# -------------------------------------------------------------- int8 GEMM --

@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (3, 5, 7), (17, 33, 130), (64, 48, 256)])
@pytest.mark.parametrize("a_unsigned", [False, True])
@pytest.mark.parametrize("b_nk", [False, True])
def test_matmul_i8_vs_int64(orc, M, N, K, a_unsigned, b_nk):
    a = RNG.integers(0, 256, (M, K)) if a_unsigned else RNG.integers(-128, 128, (M, K))
    a = a.astype(np.uint8 if a_unsigned else np.int8)
    b = RNG.integers(-128, 128, (K, N)).astype(np.int8)
    bb = np.ascontiguousarray(b.T) if b_nk else b
    c = orc.matmul_i8(a, bb, a_unsigned=a_unsigned, b_nk=b_nk)
    assert (c == _i64_matmul_wrap(a, b)).all()


def test_matmul_i8_closed_forms(orc):
    n = 37
    eye = np.eye(n, dtype=np.int8)
    b = RNG.integers(-128, 128, (n, 29)).astype(np.int8)
    assert (orc.matmul_i8(eye, b) == b.astype(np.int32)).all()          # I x B = B
    a = np.full((5, 300), -128, np.int8)
    bb = np.full((300, 6), -128, np.int8)
    assert (orc.matmul_i8(a, bb) == 300 * 16384).all()                  # constant
    au = np.full((5, 300), 255, np.uint8)
    assert (orc.matmul_i8(au, bb, a_unsigned=True) == 300 * 255 * -128).all()


@pytest.mark.parametrize("M,N,K", [(4, 8, 64), (7, 9, 200), (13, 64, 128), (1, 33, 70)])
@pytest.mark.parametrize("a_unsigned", [False, True])
@pytest.mark.parametrize("b_nk", [False, True])
def test_vnni_algorithm_equals_textbook(orc, M, N, K, a_unsigned, b_nk):
    """The VNNI-pass restatement (sign flip + bias, M/K tails) is bit-exact."""
    a = RNG.integers(0, 256, (M, K)).astype(np.uint8)
    if not a_unsigned:
        a = a.view(np.int8)
    b = RNG.integers(-128, 128, (K, N)).astype(np.int8)
    bb = np.ascontiguousarray(b.T) if b_nk else b
    c, _ = orc.matmul_i8_vnni(a, bb, a_unsigned=a_unsigned, b_nk=b_nk, nthreads=2)
    assert (c == orc.matmul_i8(a, bb, a_unsigned=a_unsigned, b_nk=b_nk)).all()


@pytest.mark.parametrize("n", [64, 128, 256, 512])
def test_vnni_vs_reference_kernel(orc, n):
    """Oracle == the reference's vnni_matmul_single_thread<N>, compiled in place."""
    if orc.load_ref() is None:
        pytest.skip("reference not built here")
    if "avx512_vnni" not in open("/proc/cpuinfo").read():
        pytest.skip("host lacks AVX-512 VNNI")
    for a, b in (orc.recipe_inputs(n),
                 (RNG.integers(-128, 128, (n, n)).astype(np.int8),
                  RNG.integers(-128, 128, (n, n)).astype(np.int8))):
        bt = np.ascontiguousarray(b.T)
        ref = np.zeros((n, n), np.int32)
        getattr(orc.load_ref(), f"ref_vnni_matmul_{n}")(a.ctypes.data, bt.ctypes.data, ref.ctypes.data)
        assert (orc.matmul_i8(a, b) == ref).all()
        c, _ = orc.matmul_i8_vnni(a, b, nthreads=4)
        assert (c == ref).all()


def test_checksum_recipe_fixture(orc):
    """Golden checksums of the reference's int8 benchmark recipe (tests/golden)."""
    import json
    import os
    gold = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                       "int8_recipe_checksums.json")))
    for n_str, want in gold["checksums"].items():
        n = int(n_str)
        if n > 512:
            continue  # covered on the GPU; the scalar oracle is slow there
        a, b = orc.recipe_inputs(n)
        c, _ = orc.matmul_i8_vnni(a, b, nthreads=4)
        assert orc.checksum_i32(c) == want, n


def test_int4_nibble_convention_vs_reference(orc):
    """F6 nibble unpack (low = even k, sign-extend >= 8) reproduces the
    reference's packed int4 GEMM checksum (bench_int4_matmul_runner.cpp:74-150)."""
    if orc.load_ref() is None:
        pytest.skip("reference not built here")
    for n in (32, 64, 128):
        idx = np.arange(n * n).reshape(n, n)
        a = ((idx % 15) - 7).astype(np.float32)                  # A[i,k]
        bt_vals = ((idx % 15) - 7)                                # B_T[j,k] = B[k,j]
        nib = (bt_vals & 15).astype(np.uint8)
        packed = (nib[:, 0::2] | (nib[:, 1::2] << 4)).astype(np.uint8)
        c = orc.matmul_w4s(packed, np.ones((n, n // 32 if n >= 32 else 1), np.float32),
                           a, gs=32)
        c16 = np.rint(c).astype(np.int64).astype(np.int16)      # i16 result type
        chk = np.int64(c16.astype(np.int64).sum()).astype(np.int32)
        assert int(chk) == int(getattr(orc.load_ref(), f"ref_packed_int4_{n}")())
        assert int(chk) == int(getattr(orc.load_ref(), f"ref_scalar_int4_{n}")())


def test_matmul_i4_recipe_fixture(orc):
    """i4 tensor_matmul checksums: 32/64/128 from the reference's own
    packed_matmul_int4 (tests/golden), the rest from the oracle's recipe run."""
    import json
    import os
    gold = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                       "int4_recipe_checksums.json")))
    for n_str, want in gold["checksums"].items():
        n = int(n_str)
        if n > 512:
            continue
        ap, bp = orc.int4_recipe_inputs(n)
        assert orc.checksum_i16(orc.matmul_i4(ap, bp, n, n, n)) == want, n
    if orc.load_ref() is not None:
        for n in (32, 64, 128):
            assert gold["checksums"][str(n)] == int(getattr(orc.load_ref(), f"ref_packed_int4_{n}")())


@pytest.mark.parametrize("M,N,K", [(5, 7, 9), (16, 33, 64), (33, 18, 101), (1, 1, 1)])
def test_matmul_i4_vs_int64_truncated(orc, M, N, K):
    """Closed form: nibbles unpacked by numpy, exact int64 product, wrapped to i16;
    odd K and N exercise the half-used last byte of a packed row."""
    rng = np.random.default_rng(M * 100 + N * 10 + K)
    a = rng.integers(-8, 8, (M, K))
    b = rng.integers(-8, 8, (K, N))
    ap, bp = orc.pack_i4(a, axis=1), orc.pack_i4(b, axis=1)
    assert ap.shape == (M, (K + 1) // 2) and bp.shape == (K, (N + 1) // 2)
    want = (a.astype(np.int64) @ b.astype(np.int64)).astype(np.int16)
    assert np.array_equal(orc.matmul_i4(ap, bp, M, N, K), want)


def test_matmul_i4_wraps_to_i16(orc):
    """K = 1100 rows of (-8)*(-8) = 70400 -> i16 wrap (70400 - 65536 = 4864)."""
    K = 1100
    a = np.full((1, K), -8)
    b = np.full((K, 2), -8)
    got = orc.matmul_i4(orc.pack_i4(a, 1), orc.pack_i4(b, 1), 1, 2, K)
    assert got.tolist() == [[4864, 4864]]
    # and a tiny brute force in plain Python loops
    a = [[3, -8, 7], [0, -1, 5]]
    b = [[1, -2], [7, 4], [-8, -3]]
    want = [[sum(a[i][k] * b[k][j] for k in range(3)) for j in range(2)] for i in range(2)]
    got = orc.matmul_i4(orc.pack_i4(np.array(a), 1), orc.pack_i4(np.array(b), 1), 2, 2, 3)
    assert got.tolist() == want


# ---------------------------------------------------------------- fp32 ops --

def test_matmul_f32_kat_and_accumulate(orc):
    a = np.arange(1, 11, dtype=np.float32)
    b = np.full(10, 2.0, np.float32)
    out = np.zeros(1, np.float32)
    orc.matmul_f32_acc(a, b, out, 1, 10, 1)
    assert out[0] == 110.0               # tests/test_tensor_matmul_runner.cpp:39
    orc.matmul_f32_acc(a, b, out, 1, 10, 1)
    assert out[0] == 220.0               # C += A*B accumulates (F4)
    m, k, n = 9, 33, 5
    A = RNG.standard_normal(3 + m * k).astype(np.float32)
    B = RNG.standard_normal(2 + k * n).astype(np.float32)
    C = np.zeros(4 + m * n, np.float32)
    orc.matmul_f32_acc(A, B, C, m, k, n, 3, 2, 4)
    exp = A[3:].reshape(m, k).astype(np.float64) @ B[2:].reshape(k, n).astype(np.float64)
    np.testing.assert_allclose(C[4:].reshape(m, n), exp, rtol=1e-5, atol=1e-5)
    assert (C[:4] == 0).all()


def test_rmsnorm_kat(orc):
    out = orc.rmsnorm(np.array([1, 2, 3, 4], np.float32), np.ones(4, np.float32), 1e-5)
    want = np.float32(1.0) / np.sqrt(np.float32(7.5) + np.float32(1e-5))
    assert abs(out[0] - want) < 1e-4     # examples/llama2/kernels/test_rmsnorm_host.cpp:34-48
    x = RNG.standard_normal(768).astype(np.float32)
    w = RNG.standard_normal(2 * 768).astype(np.float32)
    o1 = orc.rmsnorm(x, w, 1e-5, 768)
    exp = x / np.sqrt((x.astype(np.float64) ** 2).mean() + 1e-5) * w[768:]
    np.testing.assert_allclose(o1, exp, rtol=1e-5, atol=1e-6)
    o2 = orc.rmsnorm(x * 7.0, w, 0.0, 768)  # scale invariance at eps = 0
    np.testing.assert_allclose(o2, orc.rmsnorm(x, w, 0.0, 768), rtol=1e-5, atol=1e-6)


def test_softmax_kat_and_offsets(orc):
    out = orc.softmax(np.array([1, 2, 3, 4], np.float32))
    e = np.exp(np.array([-3, -2, -1, 0], np.float32))
    assert abs(out[0] - e[0] / e.sum()) < 1e-4   # test_softmax_host.cpp:34-45
    assert np.allclose(orc.softmax(np.full(17, 3.5, np.float32)), 1 / 17)
    x = RNG.standard_normal(50).astype(np.float32)
    out = orc.softmax(x, np.zeros(64, np.float32), size=20, in_off=7, out_off=11)
    ref = np.exp(x[7:27].astype(np.float64) - x[7:27].max())
    np.testing.assert_allclose(out[11:31], ref / ref.sum(), rtol=1e-5)
    assert (out[:11] == 0).all() and (out[31:] == 0).all()


def test_silu_kat(orc):
    out = orc.silu(np.array([1, 2, -1, 0], np.float32))
    assert abs(out[0] - 1 / (1 + np.exp(-1.0))) < 1e-4  # test_silu_host.cpp:32-43
    assert out[3] == 0.0
    x = RNG.standard_normal(1000).astype(np.float32) * 5
    np.testing.assert_allclose(orc.silu(x), x / (1 + np.exp(-x.astype(np.float64))),
                               rtol=1e-5, atol=1e-6)


# --------------------------------------------------------------------- W4 --

def test_quant_f5_roofline_kat(orc):
    """bench constants of examples/llama2/test_quant_roofline.cpp:71-92:
    bytes 0x55 (q = 5 in both nibbles), scale 0.01, zero 0 -> every w = 0.05."""
    rows, cols, gs = 12, 256, 128
    qw = np.full(rows * cols // 2, 0x55, np.uint8)
    sc = np.full(rows * cols // gs, 0.01, np.float32)
    ze = np.zeros(rows * cols // gs, np.float32)
    x = RNG.standard_normal(cols).astype(np.float32)
    out = orc.matmul_quant_f5(qw, sc, ze, x, rows, cols, gs)
    np.testing.assert_allclose(out, 0.05 * x.astype(np.float64).sum(), rtol=1e-4, atol=1e-5)


def _dequant_f5(qw, sc, ze, total, gs):
    q = np.empty(total, np.float64)
    q[0::2] = qw[: (total + 1) // 2] & 15
    q[1::2] = (qw[: total // 2] >> 4) & 15
    g = np.arange(total) // gs
    return q * sc[g] + ze[g]


def test_dequant_w4_pins(orc):
    """dequant_w4 (ConvertSimpToMemRef.cpp:2367-2429): the test_quant_roofline
    constants (0x55, scale 0.01, zero 0 -> 5 * 0.01f), agreement with
    matmul_quant on one-hot inputs element by element (a single product, so
    exact whatever the sum order; a swapped nibble or group index fails it),
    and the float64 value within one rounding of each step."""
    qw = np.full(64, 0x55, np.uint8)
    sc = np.full(4, 0.01, np.float32)
    ze = np.zeros(4, np.float32)
    assert (orc.dequant_w4(qw, sc, ze, 0, 128, 32) == np.float32(5) * np.float32(0.01)).all()
    rows, cols, gs, layers = 6, 256, 32, 3
    total = layers * rows * cols
    qw = RNG.integers(0, 256, total // 2).astype(np.uint8)
    sc = RNG.uniform(0.001, 0.02, total // gs).astype(np.float32)
    ze = RNG.uniform(-0.1, 0.1, total // gs).astype(np.float32)
    off = 2 * rows * cols
    deq = orc.dequant_w4(qw, sc, ze, off, rows * cols, gs).reshape(rows, cols)
    for k in (0, 1, 31, 32, 77, 255):
        x = np.zeros(cols, np.float32)
        x[k] = 1.0
        assert np.array_equal(orc.matmul_quant_f5(qw, sc, ze, x, rows, cols, gs, off), deq[:, k]), k
    want = _dequant_f5(qw, sc, ze, total, gs)
    got = orc.dequant_w4(qw, sc, ze, 0, total, gs)
    assert np.abs(got - want).max() <= 2 * np.finfo(np.float32).eps * np.abs(want).max()
    # an odd start and a range that crosses groups
    assert np.array_equal(orc.dequant_w4(qw, sc, ze, 37, 100, gs), got[37:137])


def test_quant_f5_vs_dequant_and_quantizer(orc):
    rows, cols, gs = 16, 512, 128
    w = RNG.uniform(-0.01, 0.01, rows * cols).astype(np.float32)  # bench_llama_quant.cpp:43-49
    qw, sc, ze = orc.quantize_f5(w, gs)
    deq = _dequant_f5(qw, sc, ze, w.size, gs)
    assert np.abs(deq - w).max() <= sc.max() / 2 + 1e-7          # round-to-nearest bound
    x = RNG.standard_normal(cols).astype(np.float32)
    out = orc.matmul_quant_f5(qw, sc, ze, x, rows, cols, gs)
    exp = deq.reshape(rows, cols) @ x.astype(np.float64)
    np.testing.assert_allclose(out, exp, rtol=1e-4, atol=1e-5)
    # weight offset: the second matrix in a concatenated buffer (D3 fixed)
    w2 = RNG.uniform(-0.01, 0.01, 2 * rows * cols).astype(np.float32)
    qw2, sc2, ze2 = orc.quantize_f5(w2, gs)
    out2 = orc.matmul_quant_f5(qw2, sc2, ze2, x, rows, cols, gs, rows * cols)
    deq2 = _dequant_f5(qw2, sc2, ze2, w2.size, gs)[rows * cols:]
    np.testing.assert_allclose(out2, deq2.reshape(rows, cols) @ x, rtol=1e-4, atol=1e-5)


def _rand_w4s(N, K, gs):
    q = RNG.integers(-8, 8, (N, K))
    nib = (q & 15).astype(np.uint8)
    packed = (nib[:, 0::2] | (nib[:, 1::2] << 4)).astype(np.uint8)
    sc = (np.abs(RNG.standard_normal((N, K // gs))) * 0.02 / 7).astype(np.float32)
    return q, packed, sc


def test_w4s_vs_dequant_and_f5_equivalence(orc):
    N, K, gs, M = 24, 320, 32, 3
    q, packed, sc = _rand_w4s(N, K, gs)
    x = RNG.standard_normal((M, K)).astype(np.float32)
    out = orc.matmul_w4s(packed, sc, x, gs)
    deq = (q.astype(np.float32) * np.repeat(sc, gs, axis=1)).astype(np.float64)
    np.testing.assert_allclose(out, x.astype(np.float64) @ deq.T, rtol=1e-6, atol=1e-7)
    # F6 == F5 with u = q + 8 and zero = -8 * scale (flat groups == row groups)
    u = (q + 8).astype(np.uint8)
    f5 = (u[:, 0::2] | (u[:, 1::2] << 4)).astype(np.uint8).ravel()
    f5_out = orc.matmul_quant_f5(f5, sc.ravel().copy(), (-8 * sc).ravel().copy(), x[0],
                                 N, K, gs)
    np.testing.assert_allclose(f5_out, out[0], rtol=1e-4, atol=1e-5)
    f32 = orc.matmul_w4s_f32(packed, sc, x, gs, nthreads=2)
    np.testing.assert_allclose(f32, out, rtol=1e-4, atol=1e-5)
    low = orc.matmul_w4s_lowering(packed, sc, x, gs, nthreads=2)   # the CPU baseline
    np.testing.assert_allclose(low, out, rtol=1e-4, atol=1e-5)


# ------------------------------------------------------------------- RoPE --

def test_rope_properties(orc):
    dim, hs = 64, 16
    q = RNG.standard_normal(dim).astype(np.float32)
    k = RNG.standard_normal(dim).astype(np.float32)
    q0, k0 = q.copy(), k.copy()
    orc.rope(q, k, dim, dim, hs, 0)
    assert np.allclose(q, q0) and np.allclose(k, k0)      # pos 0: identity
    pos = 5
    orc.rope(q, k, dim, dim // 2, hs, pos)
    pair = lambda v: v[0::2] ** 2 + v[1::2] ** 2
    np.testing.assert_allclose(pair(q), pair(q0), rtol=1e-5)   # rotation keeps norms
    # pair 0 of each head has freq 1: angle = pos
    c, s = np.cos(pos), np.sin(pos)
    np.testing.assert_allclose(q[0], q0[0] * c - q0[1] * s, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(q[hs], q0[hs] * c - q0[hs + 1] * s, rtol=1e-5, atol=1e-6)
    assert np.allclose(k[dim // 2:], k0[dim // 2:])             # only i < kv_dim rotated


def test_quantize_w4s_properties(orc):
    """Symmetric W4 (signed nibbles, one scale per group): every value within half a step of its
    dequantized value, the group maximum at +-7, an all-zero group at scale 1,
    two's-complement nibbles with the even index low."""
    rng = np.random.default_rng(11)
    rows, cols, gs = 9, 256, 32
    w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    w[2, 32:64] = 0.0
    q, s = orc.quantize_w4s(w, gs)
    nib = np.stack([q & 15, q >> 4], axis=-1).reshape(rows, cols).astype(np.int32)
    val = np.where(nib >= 8, nib - 16, nib)
    sc = np.repeat(s, gs, axis=1)
    assert val.min() >= -8 and val.max() <= 7
    assert np.all(np.abs(val * sc - w) <= sc / 2 * (1 + 1e-6))
    g = np.abs(w).reshape(rows, cols // gs, gs)
    arg = g.argmax(axis=2)
    top = np.take_along_axis(val.reshape(rows, cols // gs, gs), arg[..., None], 2)[..., 0]
    nz = g.max(axis=2) > 0
    assert np.all(np.abs(top[nz]) == 7)
    assert s[2, 1] == 1.0 and np.all(val[2, 32:64] == 0)


# ------------------------------------------------------ rank-3 / rank-4 --
# Known answers of simptensor/tests/test_matmul_dot.sl:135-290 and
# tests/test_tensor_matmul.sl:66-117.

def test_batch_matmul_kats(orc):
    a = np.arange(1, 13, dtype=np.float32).reshape(2, 2, 3)
    b = np.tile(np.array([1, 0, 0, 1, 1, 1], np.float32), 2).reshape(2, 3, 2)
    c = orc.batch_matmul(a, b)
    assert c[0, 0, 0] + c[1, 0, 0] == 20.0            # test_matmul_dot.sl:135-161
    eye = np.eye(3, dtype=np.float32)
    a = np.stack([eye, 2 * eye, 3 * eye])
    b = np.stack([5 * eye, 4 * eye, 2 * eye])
    c = orc.batch_matmul(a, b)
    assert c[0, 0, 0] + c[1, 1, 1] + c[2, 2, 2] == 19.0  # :164-199
    assert np.count_nonzero(c) == 9                   # diagonal products only
    # tests/test_tensor_matmul.sl:66-117 (f64): A[b,i,j] = (b+1)(i+j), B[b,i,j] = (b+1)(i+1)
    bb, ii, jj = np.meshgrid(np.arange(2), np.arange(3), np.arange(4), indexing="ij")
    A = ((bb + 1) * (ii + jj)).astype(np.float64)
    bb, ii, jj = np.meshgrid(np.arange(2), np.arange(4), np.arange(3), indexing="ij")
    B = ((bb + 1) * (ii + 1)).astype(np.float64)
    c = orc.batch_matmul(A, B)
    assert c[0, 0, 0] == 20.0                         # sum_j j (j+1), j < 4
    assert c[1, 2, 1] == 4 * sum((2 + j) * (j + 1) for j in range(4))


def test_batch_matmul_equals_2d_per_batch(orc):
    bt, m, k, n = 3, 7, 13, 5
    a = RNG.standard_normal((bt, m, k)).astype(np.float32)
    b = RNG.standard_normal((bt, k, n)).astype(np.float32)
    c = orc.batch_matmul(a, b)
    for i in range(bt):
        ref = np.zeros(m * n, np.float32)
        orc.matmul_f32_acc(a[i].ravel(), b[i].ravel(), ref, m, k, n)
        np.testing.assert_allclose(c[i].ravel(), ref, rtol=1e-5, atol=1e-5)
    c64 = orc.batch_matmul(a.astype(np.float64), b.astype(np.float64))
    np.testing.assert_allclose(c64, np.matmul(a.astype(np.float64), b.astype(np.float64)),
                               rtol=1e-13, atol=1e-13)


def test_batch_matmul_i8_vs_int64(orc):
    a = RNG.integers(-128, 128, (4, 9, 70), dtype=np.int8)
    b = RNG.integers(-128, 128, (4, 70, 11), dtype=np.int8)
    c = orc.batch_matmul(a, b)
    assert c.dtype == np.int32
    assert (c == np.matmul(a.astype(np.int64), b.astype(np.int64))).all()


def test_matmul_nhwc_kats(orc):
    x = np.arange(1, 25, dtype=np.float32).reshape(2, 2, 2, 3)
    w = np.array([[1, 0, 0], [0, 1, 0], [0, 0, 1], [.5, .5, .5]], np.float32)
    y = orc.matmul_nhwc(x, w)
    assert y.shape == (2, 2, 2, 4)
    assert y[0, 0, 0, 0] + y[0, 0, 0, 3] == 4.0       # test_matmul_dot.sl:204-236
    assert (y[..., :3] == x).all()                    # identity rows pass channels through
    x = np.repeat(np.arange(1, 19, dtype=np.float32), 2).reshape(2, 3, 3, 2)
    w = np.array([[1, 1], [2, 2], [3, 3]], np.float32)
    y = orc.matmul_nhwc(x, w)
    assert y[0, 0, 0, 0] + y[0, 0, 0, 1] + y[0, 0, 0, 2] == 12.0  # :239-268
    assert y[1, 2, 2, 2] == 3 * 2 * 18


# ---------------------------------------------------------- llama32 (int8) --

def _l32_dims(cfg):
    from _llama32 import DIMS
    return [cfg[k] for k in DIMS]


def test_llama32_zero_weights_closed_form(orc):
    """All-zero int8 layer weights: every projection is 0, the residual stream
    stays x = (float)x_i8 and logits = wcls . rmsnorm(x) (numpy, float64)."""
    from _llama32 import CFG_SMALL, make_arrays
    cfg = dict(CFG_SMALL, n_layers=2)
    a = make_arrays(cfg, seed=9, wide=True)
    for k in ("wq_t", "wk_t", "wv_t", "wo_t", "w1_t", "w2_t", "w3_t"):
        a[k][:] = 0
    r = orc.llama32_int8_forward(a, 3, *_l32_dims(cfg))
    x = a["x_i8"].astype(np.float64)
    assert np.array_equal(a["x_fp32"], a["x_i8"].astype(np.float32))
    xb = x / np.sqrt((x * x).mean() + 1e-5) * a["rms_final_w"]
    lg = a["wcls"].reshape(cfg["vocab_size"], cfg["dim"]).astype(np.float64) @ xb
    np.testing.assert_allclose(a["logits"], lg, rtol=1e-4, atol=1e-4 * np.abs(lg).max())
    assert r == a["logits"][0]
    assert not a["k_cache"].any() and not a["ffn_hb"].any()


def test_llama32_first_layer_cache_rows(orc):
    """Layer 0's K/V rows at pos are (i8)((xb_i8 . W_t row) / 256) with xb_i8 the
    quantized attention RMSNorm of x_i8: recomputed in float64 / int64, equal
    except where xb*127 lies within 1e-4 of an integer (fp32 rounding)."""
    from _llama32 import CFG_SMALL, make_arrays
    cfg = dict(CFG_SMALL, n_layers=1)
    a = make_arrays(cfg, seed=10, wide=True)
    pos = 5
    orc.llama32_int8_forward(a, pos, *_l32_dims(cfg))
    D, kv = cfg["dim"], cfg["n_kv_heads"] * cfg["head_dim"]
    x = a["x_i8"].astype(np.float64)
    v = x / np.sqrt((x * x).mean() + 1e-5) * a["rms_att_w"][:D] * 127.0
    near = (np.abs(v - np.round(v)) < 1e-4) & (v != np.round(v))
    assert not near.any()                                 # no quantization tie in this draw
    xq = np.trunc(np.clip(v, -128, 127)).astype(np.int64)
    for name, w in (("k_cache", "wk_t"), ("v_cache", "wv_t")):
        acc = a[w].reshape(kv, D).astype(np.int64) @ xq
        want = (np.trunc(acc / 256.0).astype(np.int64) & 0xFF).astype(np.uint8).view(np.int8)
        got = a[name].reshape(cfg["max_seq_len"], kv)[pos]
        assert np.array_equal(got, want), name


def test_llama32_attention_is_inert(orc):
    """attn_out = (i32) of a convex combination of int8 values, so |attn_out| <=
    128 and (float)attn_out / 256 truncates to 0: Wo sees a zero vector and
    cannot change the logits (a property of the program's fixed-point scales)."""
    from _llama32 import CFG_SMALL, make_arrays
    cfg = CFG_SMALL
    a = make_arrays(cfg, seed=11, wide=True)
    b = {k: v.copy() for k, v in a.items()}
    b["wo_t"][:] = np.random.default_rng(12).integers(-128, 128, b["wo_t"].size, dtype=np.int8)
    for pos in range(3):
        orc.llama32_int8_forward(a, pos, *_l32_dims(cfg))
        orc.llama32_int8_forward(b, pos, *_l32_dims(cfg))
    assert np.abs(a["attn_out"]).max() <= 128
    assert np.array_equal(a["logits"], b["logits"])


def test_llama32_fptosi_wraps_like_x86(orc):
    """ffn_hb = (i8)(silu(g)*u*127) keeps the low byte of the i32 truncation
    (the program does not clamp there): out-of-range values wrap."""
    from _llama32 import CFG_SMALL, make_arrays
    cfg = dict(CFG_SMALL, n_layers=1)
    a = make_arrays(cfg, seed=13, wide=True)
    a["rms_ffn_w"][:] = 4.0                                # large activations into W1/W3
    orc.llama32_int8_forward(a, 0, *_l32_dims(cfg))
    hb = a["ffn_hb"].astype(np.int64)
    assert np.unique(hb).size > 100                       # wrapped values cover the byte range
    assert np.isin(hb, (-128, 127)).mean() < 0.05         # a clamp would pile them up at the ends


def test_llama32_ffn_composition_closed_form(orc):
    """One layer with the attention matrices zero (Wo sees zeros): the FFN and
    the final norm in float64 / int64 with the program's integer steps
    (llama32_1b_int8_tensor.sl:232-280): xq = trunc(clamp(rmsnorm(x) * 127)),
    G = W1 xq and U = W3 xq exact (i32), ffn_hb = low byte of
    trunc(silu(G / 65536) * (U / 65536) * 127), x += (W2 ffn_hb) / 65536,
    logits = wcls . rmsnorm(x).  ffn_hb is compared except where fp32 and
    float64 may round across an integer (within 1e-3 of one); x and the logits
    are then recomputed from the oracle's own ffn_hb."""
    from _llama32 import CFG_SMALL, make_arrays
    cfg = dict(CFG_SMALL, n_layers=1)
    a = make_arrays(cfg, seed=14, wide=True)
    for k in ("wq_t", "wk_t", "wv_t", "wo_t"):
        a[k][:] = 0
    x0 = a["x_i8"].astype(np.float64)
    orc.llama32_int8_forward(a, 2, *_l32_dims(cfg))
    D, H = cfg["dim"], cfg["hidden_dim"]
    v = x0 / np.sqrt((x0 * x0).mean() + 1e-5) * a["rms_ffn_w"][:D] * 127.0
    assert not ((np.abs(v - np.round(v)) < 1e-4) & (v != np.round(v))).any()
    xq = np.trunc(np.clip(v, -128, 127)).astype(np.int64)
    G = a["w1_t"].reshape(H, D).astype(np.int64) @ xq
    U = a["w3_t"].reshape(H, D).astype(np.int64) @ xq
    g = G / 65536.0
    val = g / (1 + np.exp(-g)) * (U / 65536.0) * 127.0
    want_hb = (np.trunc(val).astype(np.int64) & 0xFF).astype(np.uint8).view(np.int8)
    tie = np.abs(val - np.round(val)) < 1e-3
    assert tie.mean() < 0.05
    assert np.array_equal(a["ffn_hb"][~tie], want_hb[~tie])
    x1 = x0 + (a["w2_t"].reshape(D, H).astype(np.int64) @ a["ffn_hb"].astype(np.int64)) / 65536.0
    np.testing.assert_allclose(a["x_fp32"], x1, rtol=1e-6, atol=1e-6 * np.abs(x1).max())
    xb = x1 / np.sqrt((x1 * x1).mean() + 1e-5) * a["rms_final_w"]
    lg = a["wcls"].reshape(cfg["vocab_size"], D).astype(np.float64) @ xb
    np.testing.assert_allclose(a["logits"], lg, rtol=1e-4, atol=1e-4 * np.abs(lg).max())
    assert not np.array_equal(a["x_fp32"], a["x_i8"].astype(np.float32))  # the FFN acted


def test_llama32_layer_offsets(orc):
    """Per-layer slices (l * dim, l * kv * dim, ... and the cache rows of layer
    l): a two-layer model whose first layer has all-zero int8 weights equals the
    one-layer model made of its second layer (weights and both norms), logits
    and the second layer's cache rows alike."""
    from _llama32 import CFG_SMALL, make_arrays
    cfg2 = dict(CFG_SMALL, n_layers=2)
    cfg1 = dict(CFG_SMALL, n_layers=1)
    a = make_arrays(cfg2, seed=15, wide=True)
    D, H = cfg2["dim"], cfg2["hidden_dim"]
    kv = cfg2["n_kv_heads"] * cfg2["head_dim"]
    per = {"wq_t": D * D, "wk_t": kv * D, "wv_t": kv * D, "wo_t": D * D, "w1_t": H * D,
           "w2_t": D * H, "w3_t": H * D}
    for k, n in per.items():
        a[k][:n] = 0                                        # layer 0 does nothing
    b = make_arrays(cfg1, seed=16, wide=True)
    for k, n in per.items():
        b[k][:] = a[k][n:]
    for k in ("rms_att_w", "rms_ffn_w"):
        b[k][:] = a[k][D:]
    for k in ("x_i8", "rms_final_w", "wcls"):
        b[k][:] = a[k]
    for pos in range(3):
        orc.llama32_int8_forward(a, pos, *_l32_dims(cfg2))
        orc.llama32_int8_forward(b, pos, *_l32_dims(cfg1))
        assert np.array_equal(a["logits"], b["logits"]), pos
    S = cfg2["max_seq_len"]
    for c in ("k_cache", "v_cache"):
        assert np.array_equal(a[c].reshape(2, S, kv)[1], b[c].reshape(1, S, kv)[0])
        assert not a[c].reshape(2, S, kv)[0].any()


# ---------------------------------------------------------------- argmax --
# sample_argmax (generate_stories110M.cpp:73-83) scans from logits[0] with a
# strict '>'. What that scan must return, stated without the scan: 0 when
# logits[0] is NaN, else the first index holding the largest non-NaN value.

def _argmax_closed_form(v):
    v = np.asarray(v, np.float32)
    if np.isnan(v[0]):
        return 0
    ok = ~np.isnan(v)
    return int(np.flatnonzero(ok & (v == v[ok].max()))[0])


def test_argmax_closed_forms(orc):
    nan, inf = np.float32(np.nan), np.float32(np.inf)
    assert orc.argmax([1.0, 3.0, 3.0, 2.0]) == 1            # ties: the first wins
    assert orc.argmax([5.0, 5.0, 5.0]) == 0
    assert orc.argmax([nan, 1.0, 2.0]) == 0                 # NaN at 0: nothing exceeds it
    assert orc.argmax([0.0, nan, 2.0, nan]) == 2            # NaN elsewhere is skipped
    assert orc.argmax([nan] * 7) == 0
    assert orc.argmax([-inf] * 7) == 0
    assert orc.argmax([-inf, nan, -inf]) == 0
    assert orc.argmax([-0.0, 0.0]) == 0                     # -0 == +0: not greater
    assert orc.argmax([-1.0, inf, inf]) == 1
    big = np.zeros(32000, np.float32)
    big[[7, 31999, 20000]] = 4.0
    assert orc.argmax(big) == 7


def test_argmax_brute_force(orc):
    """Every pattern of 5 values from {-inf, -1, 0, -0, 1, NaN} against the
    closed form; a '>=' scan or a seed of -inf with index 0 fails it."""
    import itertools
    vals = np.array([-np.inf, -1.0, 0.0, -0.0, 1.0, np.nan], np.float32)
    for pat in itertools.product(range(len(vals)), repeat=5):
        v = vals[list(pat)]
        assert orc.argmax(v) == _argmax_closed_form(v), v


def test_int8_recipe_inputs_closed_form(orc):
    """bench_int8_matmul_runner.cpp:33-64: val = ((i*N+j) % 127) - 64,
    A[i,j] = B[j,i] = val."""
    for n in (1, 2, 31, 64, 127, 128, 300):
        a, b = orc.recipe_inputs(n)
        i, j = np.meshgrid(np.arange(n), np.arange(n), indexing="ij")
        val = ((i * n + j) % 127 - 64).astype(np.int8)
        assert np.array_equal(a, val), n
        assert np.array_equal(b, val.T), n
