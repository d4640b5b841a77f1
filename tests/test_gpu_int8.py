"""GPU parity of the int8 GEMM entry points against the pinned oracle.

Bit-exact for every shape (integer arithmetic).  Full BASELINE sizes that the
CPU oracle cannot finish in seconds (4096^3, 8192^3) are checked through
size-independent identities: row sums C*1 = A*(B*1), column sums 1^T*C =
(1^T*A)*B (exact in int64), a sample of full rows recomputed exactly, and the
reference's checksum recipe.
"""
import numpy as np
import pytest

import simplang_amd as sa

pytestmark = pytest.mark.gpu

SEED = 42


def _inputs(M, N, K, seed=SEED):
    rng = np.random.default_rng(seed + M * 7 + N * 13 + K)
    a = rng.integers(0, 256, (M, K)).astype(np.uint8)    # config #1: A u8 uniform [0,255]
    b = rng.integers(-128, 128, (K, N)).astype(np.int8)  #            B s8 uniform [-128,127]
    return a, b


def _run(dev, fn, a, b, M, N):
    import torch
    ta = torch.from_numpy(a).to(dev)
    tb = torch.from_numpy(b).to(dev)
    tc = torch.full((M, N), -7, dtype=torch.int32, device=dev)  # poison: C is overwritten
    fn(ta, tb, tc)
    torch.cuda.synchronize()
    return tc.cpu().numpy()


SHAPES = [(256, 256, 256), (512, 512, 512), (768, 768, 768), (1024, 1024, 1024),
          (1, 2048, 768), (8, 2048, 768), (64, 2048, 768),
          (1, 768, 2048), (8, 768, 2048), (64, 768, 2048),
          (1, 8640, 3200), (8, 8640, 3200), (64, 8640, 3200),
          (2048, 2048, 2048),
          # ragged / tails: M, N not multiples of any tile, K not a multiple of 128
          (100, 200, 48), (33, 260, 144), (300, 516, 400), (1, 4, 16)]


@pytest.mark.parametrize("M,N,K", SHAPES)
def test_int8_s8s8_and_u8s8_bit_exact(dev, orc, M, N, K):
    print(f"[int8] M={M} N={N} K={K}", flush=True)
    a, b = _inputs(M, N, K)
    want_u8, _ = orc.matmul_i8_vnni(a, b, a_unsigned=True, nthreads=8)
    got = _run(dev, sa.matmul_u8s8_i32, a, b, M, N)
    assert np.array_equal(got, want_u8)
    a_s8 = a.view(np.int8)                               # same bytes as s8 (SimpLang i8)
    want_s8, _ = orc.matmul_i8_vnni(a_s8, b, nthreads=8)
    got = _run(dev, sa.tensor_matmul_i8, a_s8, b, M, N)
    assert np.array_equal(got, want_s8)


@pytest.mark.parametrize("M,N,K", [(512, 512, 512), (64, 8640, 3200), (1, 2048, 768),
                                   (1024, 1024, 1024), (77, 130, 272)])
def test_int8_nt_variants_bit_exact(dev, orc, M, N, K):
    print(f"[int8-nt] M={M} N={N} K={K}", flush=True)
    a, b = _inputs(M, N, K, seed=7)
    bt = np.ascontiguousarray(b.T)
    want_u8, _ = orc.matmul_i8_vnni(a, b, a_unsigned=True, nthreads=8)
    assert np.array_equal(_run(dev, sa.matmul_nt_u8s8_i32, a, bt, M, N), want_u8)
    want_s8, _ = orc.matmul_i8_vnni(a.view(np.int8), b, nthreads=8)
    assert np.array_equal(_run(dev, sa.tensor_matmul_nt_i8, a.view(np.int8), bt, M, N), want_s8)


@pytest.mark.parametrize("M,N,K", [(1024, 1024, 128), (1024, 1024, 256), (1000, 1040, 1024),
                                   (768, 768, 768), (2048, 2048, 384), (2000, 2064, 1152),
                                   (1536, 1024, 2048), (2048, 2048, 2560), (1000, 1024, 3200),
                                   (96, 8640, 3200), (128, 32000, 3200)])
def test_int8_ring_kernel_bit_exact(dev, orc, M, N, K):
    """Mid sizes with K % 128 == 0 run the ring kernel (64x64 or 128x128 tiles,
    K-stages of 128 through a ring of 2 slots, or of 4 for 64x64 tiles with
    several tiles per workgroup, part of the chip idle or K > 4096, and for
    128x128 tiles whose operands stream from HBM): one stage, fewer stages
    than slots, both slot counts on both tile sizes, several tiles per
    workgroup, 128x128 tiles on part of the chip (M = 96, 68 tiles), ragged M
    and N, B as [K,N] and as B_T, u8 and s8 A."""
    print(f"[int8-ring] M={M} N={N} K={K}", flush=True)
    a, b = _inputs(M, N, K, seed=13)
    bt = np.ascontiguousarray(b.T)
    want_u8, _ = orc.matmul_i8_vnni(a, b, a_unsigned=True, nthreads=8)
    assert np.array_equal(_run(dev, sa.matmul_u8s8_i32, a, b, M, N), want_u8)
    assert np.array_equal(_run(dev, sa.matmul_nt_u8s8_i32, a, bt, M, N), want_u8)
    want_s8, _ = orc.matmul_i8_vnni(a.view(np.int8), b, nthreads=8)
    assert np.array_equal(_run(dev, sa.tensor_matmul_i8, a.view(np.int8), b, M, N), want_s8)
    assert np.array_equal(_run(dev, sa.tensor_matmul_nt_i8, a.view(np.int8), bt, M, N), want_s8)


@pytest.mark.parametrize("M", [1, 2, 3])
@pytest.mark.parametrize("N,K", [(264, 80), (4104, 1040), (4100, 1040), (65536, 64),
                                 (8640, 3200), (2056, 4096)])
def test_int8_skinny_gemv_bit_exact(dev, orc, M, N, K):
    """M = 1 with B of 4 MB or more (M = 2: 8 MB) and B as [K,N] runs the dot4
    GEMV, in one K band (stores, K = 64) or several (atomic sums); N % 8 != 0,
    small B and M = 3 take the MFMA tiles."""
    print(f"[int8-gemv] M={M} N={N} K={K}", flush=True)
    a, b = _inputs(M, N, K, seed=11)
    want_u8, _ = orc.matmul_i8_vnni(a, b, a_unsigned=True, nthreads=8)
    assert np.array_equal(_run(dev, sa.matmul_u8s8_i32, a, b, M, N), want_u8)
    want_s8, _ = orc.matmul_i8_vnni(a.view(np.int8), b, nthreads=8)
    assert np.array_equal(_run(dev, sa.tensor_matmul_i8, a.view(np.int8), b, M, N), want_s8)


def test_int8_skinny_gemv_call_sequence(dev, orc):
    """Consecutive GEMV calls of other widths and depths on one stream (one K
    band and several, so plain stores and atomic sums into the filled C), with
    A, B and C as windows of wider arrays: the columns beside C stay intact."""
    import torch
    for i, (M, N, K) in enumerate([(1, 8640, 3200), (8, 264, 80), (1, 65536, 64),
                                   (1, 264, 80), (2, 8640, 1040), (7, 8640, 3200)]):
        print(f"[int8-gemv-seq] M={M} N={N} K={K}", flush=True)
        a, b = _inputs(M, N, K, seed=20 + i)
        want, _ = orc.matmul_i8_vnni(a, b, a_unsigned=True, nthreads=8)
        ta = torch.zeros((M, K + 48), dtype=torch.uint8, device=dev)
        ta[:, 16:16 + K] = torch.from_numpy(a).to(dev)
        tb = torch.zeros((K, N + 16), dtype=torch.int8, device=dev)
        tb[:, 8:8 + N] = torch.from_numpy(b).to(dev)
        tc = torch.full((M, N + 12), -5, dtype=torch.int32, device=dev)
        sa.matmul_u8s8_i32(ta[:, 16:16 + K], tb[:, 8:8 + N], tc[:, 8:8 + N])
        torch.cuda.synchronize()
        out = tc.cpu().numpy()
        assert np.array_equal(out[:, 8:8 + N], want), (M, N, K)
        assert (out[:, :8] == -5).all() and (out[:, 8 + N:] == -5).all()


@pytest.mark.parametrize("pad", [64, 4])
def test_int8_large_b_window(dev, orc, pad):
    """Large-tile path with B as a column window of a wider [K, N + pad] array:
    16-byte aligned rows (pad 64) are read in place, others (pad 4) are
    transposed first; rows of C are checked in full against the oracle."""
    import torch
    M, N, K = 4096, 4096, 1024
    print(f"[int8-bwin] pad={pad}", flush=True)
    a, b = _inputs(M, N, K, seed=31)
    tb = torch.zeros((K, N + pad), dtype=torch.int8, device=dev)
    tb[:, pad // 2:pad // 2 + N] = torch.from_numpy(b).to(dev)
    ta = torch.from_numpy(a).to(dev)
    tc = torch.empty((M, N), dtype=torch.int32, device=dev)
    sa.matmul_u8s8_i32(ta, tb[:, pad // 2:pad // 2 + N], tc)
    torch.cuda.synchronize()
    rows = np.r_[0:8, 1000:1004, M - 8:M]
    want, _ = orc.matmul_i8_vnni(np.ascontiguousarray(a[rows]), b, a_unsigned=True, nthreads=8)
    assert np.array_equal(tc.cpu().numpy()[rows], want)


@pytest.mark.parametrize("M,N,K", [(5, 9, 13), (3, 130, 100), (17, 6, 24)])
def test_int8_unaligned_shapes_fallback(dev, orc, M, N, K):
    """K % 16 != 0 or N % 4 != 0 take the generic kernel; still bit-exact."""
    a, b = _inputs(M, N, K, seed=3)
    assert np.array_equal(_run(dev, sa.matmul_u8s8_i32, a, b, M, N),
                          orc.matmul_i8(a, b, a_unsigned=True))
    assert np.array_equal(_run(dev, sa.tensor_matmul_i8, a.view(np.int8), b, M, N),
                          orc.matmul_i8(a.view(np.int8), b))


def test_int8_recipe_checksums(dev, orc):
    """The reference benchmark's inputs and checksum (golden fixture)."""
    import json
    import os
    gold = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                       "int8_recipe_checksums.json")))
    for n_str, want in gold["checksums"].items():
        n = int(n_str)
        print(f"[recipe] N={n}", flush=True)
        a, b = orc.recipe_inputs(n)
        got = _run(dev, sa.tensor_matmul_i8, a, b, n, n)
        assert orc.checksum_i32(got) == want, n


@pytest.mark.parametrize("M,N,K", [(4096, 4096, 4096), (8192, 8192, 8192),
                                   (4100, 4112, 4096),    # ragged M, N on the LDS-DMA kernel
                                   (4000, 4112, 4096),    # the same with in-kernel u8 sums
                                   (4100, 4112, 4000)])   # K % 64 != 0: register-staged kernel
@pytest.mark.parametrize("variant", ["u8s8", "s8s8", "nt_u8s8", "nt_s8s8"])
def test_int8_full_size_identities(dev, orc, M, N, K, variant):
    import torch
    print(f"[int8-full] {variant} M={M} N={N} K={K}", flush=True)
    a, b = _inputs(M, N, K)
    if "s8s8" in variant:
        a = a.view(np.int8)
    fn = {"u8s8": sa.matmul_u8s8_i32, "s8s8": sa.tensor_matmul_i8,
          "nt_u8s8": sa.matmul_nt_u8s8_i32, "nt_s8s8": sa.tensor_matmul_nt_i8}[variant]
    bb = np.ascontiguousarray(b.T) if variant.startswith("nt") else b
    got = _run(dev, fn, a, bb, M, N).astype(np.int64)
    a64, b64 = a.astype(np.int64), b.astype(np.int64)
    assert np.array_equal(got.sum(1), a64 @ b64.sum(1))          # C 1 = A (B 1)
    assert np.array_equal(got.sum(0), a64.sum(0) @ b64)          # 1^T C = (1^T A) B
    rng = np.random.default_rng(M + N)
    for r in list(rng.choice(M, 3, replace=False)) + [M - 1]:
        assert np.array_equal(got[r], a64[r] @ b64)              # full rows, exact
    for c in list(rng.choice(N, 2, replace=False)) + [N - 1]:
        assert np.array_equal(got[:, c], a64 @ b64[:, c])        # full columns, exact
    del got
    torch.cuda.empty_cache()


def test_int8_host_pointers_are_staged(orc):
    """numpy operands: the library stages through device memory and blocks."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    a, b = _inputs(96, 160, 224, seed=11)
    c = np.full((96, 160), -1, np.int32)
    sa.set_stream(None)
    sa.matmul_u8s8_i32(a, b, c)
    assert np.array_equal(c, orc.matmul_i8(a, b, a_unsigned=True))
    sa.set_stream(torch.cuda.current_stream())


def test_int8_strided_views(dev, orc):
    """Row strides and offsets of sub-tensor views (descriptor offset/stride0)."""
    import torch
    a, b = _inputs(128, 256, 512, seed=5)
    ta = torch.from_numpy(a).to(dev)[:, 64:320]        # [128, 256], stride0 512
    tb = torch.from_numpy(b).to(dev)[128:384, :]       # [256, 256]
    tc_full = torch.zeros((128, 300), dtype=torch.int32, device=dev)
    tc = tc_full[:, 20:276]
    sa.matmul_u8s8_i32(ta, tb, tc)
    torch.cuda.synchronize()
    want = orc.matmul_i8(np.ascontiguousarray(a[:, 64:320]), np.ascontiguousarray(b[128:384]),
                         a_unsigned=True)
    out = tc_full.cpu().numpy()
    assert np.array_equal(out[:, 20:276], want)
    assert (out[:, :20] == 0).all() and (out[:, 276:] == 0).all()


@pytest.mark.parametrize("M,N,K", [(8192, 8192, 128),     # K-steps < ring stages
                                   (8192, 8192, 512),     # 4 tiles per workgroup
                                   (8192, 4096, 1088),    # odd K-step count
                                   (4100, 4112, 1024),    # ragged last tiles
                                   (4000, 4112, 1024)])   # u8: column sums in the kernel
@pytest.mark.parametrize("variant", ["u8s8", "s8s8", "nt_u8s8"])
def test_int8_persistent_kernel_exact(dev, orc, M, N, K, variant):
    """Every element of the persistent LDS-DMA kernel's output, at sizes where
    workgroups walk several tiles (tile transitions overlap one tile's stores
    with the next tile's loads), against the oracle.  The u8 column sums come
    from the kernel's own MFMAs.  Up to 16 tile rows (M <= 4096) the tiles are
    grouped by rows and each tile forms them; the last shape reaches that with
    ragged tiles and 272 tiles on 256 workgroups (the sums' LDS exchange
    reused by a second tile).  Beyond, the tiles are grouped by columns and a
    workgroup forms the sums once per column tile it visits: at 8192 x 8192
    it keeps them for its four tiles, and at 4100 x 4112 some workgroups
    move to another column tile and form them again."""
    import torch
    print(f"[int8-persistent] {variant} M={M} N={N} K={K}", flush=True)
    a, b = _inputs(M, N, K, seed=9)
    if variant == "s8s8":
        a = a.view(np.int8)
    want, _ = orc.matmul_i8_vnni(a, b, a_unsigned=variant != "s8s8", nthreads=8)
    if variant == "nt_u8s8":
        got = _run(dev, sa.matmul_nt_u8s8_i32, a, np.ascontiguousarray(b.T), M, N)
        assert np.array_equal(got, want)
        return
    fn = sa.matmul_u8s8_i32 if variant == "u8s8" else sa.tensor_matmul_i8
    got = _run(dev, fn, a, b, M, N)
    assert np.array_equal(got, want)
    del got
    torch.cuda.empty_cache()


@pytest.mark.parametrize("variant", ["u8s8", "nt_s8s8"])
def test_int8_large_tile_unaligned_c(dev, orc, variant):
    """Large-tile kernels with a C view that is only 4-byte aligned (scalar stores)."""
    import torch
    M, N, K = 4096, 4096, 192
    print(f"[int8-unaligned-c] {variant}", flush=True)
    a, b = _inputs(M, N, K, seed=3)
    if variant == "nt_s8s8":
        a = a.view(np.int8)
    want, _ = orc.matmul_i8_vnni(a, b, a_unsigned=variant == "u8s8", nthreads=8)
    ta = torch.from_numpy(a).to(dev)
    tb = torch.from_numpy(np.ascontiguousarray(b.T) if variant == "nt_s8s8" else b).to(dev)
    c_full = torch.full((M, N + 4), -7, dtype=torch.int32, device=dev)
    tc = c_full[:, 1:N + 1]
    fn = sa.matmul_u8s8_i32 if variant == "u8s8" else sa.tensor_matmul_nt_i8
    fn(ta, tb, tc)
    torch.cuda.synchronize()
    out = c_full.cpu().numpy()
    assert np.array_equal(out[:, 1:N + 1], want)
    assert (out[:, 0] == -7).all() and (out[:, N + 1:] == -7).all()


@pytest.mark.parametrize("M,N,K", [(0, 64, 32), (48, 0, 32), (48, 64, 0), (0, 0, 0)])
def test_empty_dimensions(dev, M, N, K):
    """Empty operands: M or N = 0 is a no-op that leaves C alone, K = 0 writes
    C = 0 (the empty sum), on the int8 (KN and NT) and fp32 / f64 entry points."""
    import torch
    print(f"[empty] M={M} N={N} K={K}", flush=True)
    cases = [
        (sa.tensor_matmul_i8, torch.int8, torch.int8, False, torch.int32),
        (sa.matmul_u8s8_i32, torch.uint8, torch.int8, False, torch.int32),
        (sa.tensor_matmul_nt_i8, torch.int8, torch.int8, True, torch.int32),
        (sa.tensor_matmul_f32, torch.float32, torch.float32, False, torch.float32),
        (sa.tensor_matmul_f64, torch.float64, torch.float64, False, torch.float64),
    ]
    for fn, ta_t, tb_t, nt, tc_t in cases:
        a = torch.ones((M, K), dtype=ta_t, device=dev)
        b = torch.ones((N, K) if nt else (K, N), dtype=tb_t, device=dev)
        c = torch.full((M, N), 7, dtype=tc_t, device=dev)
        fn(a, b, c)
        torch.cuda.synchronize()
        want = 0 if (K == 0 and M and N) else 7
        assert (c == want).all().item(), (fn.__name__, M, N, K)


def test_int8_strided_views_host_arrays(dev, orc):
    """The same views as numpy host arrays (staged through device memory): the
    result lands in the view, and the bytes between the output rows, which lie
    inside the staged span but outside the view, come back unchanged."""
    a, b = _inputs(128, 256, 512, seed=5)
    c_full = np.full((128, 300), -7, dtype=np.int32)
    c_full[:, 276:] = 12345
    c = c_full[:, 20:276]
    sa.matmul_u8s8_i32(a[:, 64:320], b[128:384, :], c)
    want = orc.matmul_i8(np.ascontiguousarray(a[:, 64:320]), np.ascontiguousarray(b[128:384]),
                         a_unsigned=True)
    assert np.array_equal(c_full[:, 20:276], want)
    assert (c_full[:, :20] == -7).all() and (c_full[:, 276:] == 12345).all()


def _gold_checksums():
    import json
    import os
    return json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                       "int8_recipe_checksums.json")))["checksums"]


def test_benchmark_int8_programs(dev):
    """benchmark_int8_matmul_<N>() (bench_int8_matmul.sl:11-335) returns the
    checksum of the reference's own kernel (golden fixture) at every size the
    program defines, twice (the second call reuses the inputs' workspace)."""
    gold = _gold_checksums()
    for n in sa.host.BENCH_INT8_SIZES:
        print(f"[bench-program] N={n}", flush=True)
        assert sa.benchmark_int8_matmul(n) == gold[str(n)], n
        assert sa.benchmark_int8_matmul(n) == gold[str(n)], n


def test_kernel_main(dev):
    """kernel_main() of bench_int8_matmul.sl:337-339, the runner's entry point
    (kernel_runner.hpp:39-56), bound as the compiled program defines it:
    int32_t (*)(void), returning benchmark_int8_matmul_256()'s checksum."""
    import ctypes as C
    f = C.CFUNCTYPE(C.c_int32)(C.cast(sa.lib.kernel_main, C.c_void_p).value)
    assert f() == _gold_checksums()["256"]
    assert sa.kernel_main() == _gold_checksums()["256"]


@pytest.mark.parametrize("n", [256, 512, 768, 1024, 2048])
def test_int8_chunk_programs(dev, orc, n):
    """int8_chunk_<N> called the way bench_int8_parallel_runner.cpp:38-89 calls
    it: host arrays of the recipe inputs, eight row chunks issued from eight
    host threads at once; C equals the oracle's product bit for bit."""
    from concurrent.futures import ThreadPoolExecutor
    print(f"[chunk-program] N={n}", flush=True)
    a, b = orc.recipe_inputs(n)
    fa, fb = a.reshape(-1).copy(), b.reshape(-1).copy()
    c = np.zeros(n * n, np.int32)
    rows = n // 8
    with ThreadPoolExecutor(8) as ex:
        list(ex.map(lambda i: sa.int8_chunk(n, fa, fb, c, i * rows), range(8)))
    want = orc.matmul_i8(a, b)
    assert np.array_equal(c.reshape(n, n), want)
    if str(n) in _gold_checksums():
        assert orc.checksum_i32(c) == _gold_checksums()[str(n)]
    with pytest.raises(sa.SimpRTError):
        sa.int8_chunk(n, fa, fb, c, n - rows + 1)           # rows past the end
