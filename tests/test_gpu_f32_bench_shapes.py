"""GPU parity of the fp32 tensor_matmul at every shape bench.py's f32_gemm
section times, so each reported rate is backed by a check of the kernels that
produce it: the 256x128-tile ring kernel at 4096^3, the prefill tiles (M = 8, 128,
512 against 2048-wide operands, M = 8 with K split 32 ways and summed by
gemm_f32_sum_parts), and the rank-3 batch on grid z; plus skinny products
whose K split takes each width of gemm_f32_sum_parts' batched part loads.

Reference: float64 products (numpy's BLAS, a library routine; the reference
lowers f32 tensor_matmul to linalg.matmul, ConvertSimpToMemRef.cpp:3280-3291).
4096^3 is checked on 64 whole rows and 64 whole columns chosen at random.
Tolerance: 1e-4 of max|ref| (the f32 bar of the other fp32 tests).
"""
import numpy as np
import pytest

import simplang_amd as sa

pytestmark = pytest.mark.gpu
TOL = 1e-4


def _close(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    err = np.abs(got - want).max()
    assert err <= TOL * np.abs(want).max(), (err, np.abs(want).max())


@pytest.mark.parametrize("M,K,N", [(8, 2048, 2048), (128, 2048, 8192), (512, 2048, 2048)])
def test_f32_prefill_shapes(dev, M, K, N):
    import torch
    print(f"[f32-bench-shape] M={M} K={K} N={N}", flush=True)
    g = torch.Generator(device=dev).manual_seed(7)
    a = torch.randn((M, K), device=dev, generator=g)
    b = torch.randn((K, N), device=dev, generator=g)
    c = torch.full((M, N), float("nan"), device=dev)
    sa.tensor_matmul_f32(a, b, c)
    torch.cuda.synchronize()
    want = a.cpu().double().numpy() @ b.cpu().double().numpy()
    _close(c.cpu().numpy(), want)


@pytest.mark.parametrize("M,K,N,parts", [(8, 512, 65536, 4), (8, 512, 2048, 8),
                                         (12, 1024, 1024, 16), (8, 3200, 2048, 29)])
def test_f32_split_k_part_counts(dev, M, K, N, parts):
    """K split into `parts` slices (M <= 16 tiles of 16 x 256, about four
    blocks per CU, each split at least 64 deep): gemm_f32_sum_parts requests 4,
    8 or 16 parts per round (29: two rounds of 16) and adds them in split
    order."""
    import torch
    print(f"[f32-split-k] M={M} K={K} N={N} parts={parts}", flush=True)
    g = torch.Generator(device=dev).manual_seed(11)
    a = torch.randn((M, K), device=dev, generator=g)
    b = torch.randn((K, N), device=dev, generator=g)
    c = torch.full((M, N), float("nan"), device=dev)
    sa.tensor_matmul_f32(a, b, c)
    torch.cuda.synchronize()
    want = a.cpu().double().numpy() @ b.cpu().double().numpy()
    _close(c.cpu().numpy(), want)


def test_f32_4096_cube_sampled(dev):
    import torch
    n = 4096
    print(f"[f32-bench-shape] {n}^3", flush=True)
    g = torch.Generator(device=dev).manual_seed(7)
    a = torch.randn((n, n), device=dev, generator=g)
    b = torch.randn((n, n), device=dev, generator=g)
    c = torch.full((n, n), float("nan"), device=dev)
    sa.tensor_matmul_f32(a, b, c)
    torch.cuda.synchronize()
    an, bn, cn = a.cpu().double().numpy(), b.cpu().double().numpy(), c.cpu().numpy()
    rng = np.random.default_rng(1)
    rows = np.sort(rng.choice(n, 64, replace=False))
    cols = np.sort(rng.choice(n, 64, replace=False))
    rows[0], cols[-1] = 0, n - 1                      # first and last tile edges
    _close(cn[rows], an[rows] @ bn)
    _close(cn[:, cols], an @ bn[:, cols])
    assert np.isfinite(cn).all()                      # every element written


def test_f32_batch_bench_shape(dev):
    import torch
    bt, M, K, N = 32, 512, 128, 512
    print(f"[f32-bench-shape] batch {bt}x({M}x{K}x{N})", flush=True)
    g = torch.Generator(device=dev).manual_seed(7)
    a = torch.randn((bt, M, K), device=dev, generator=g)
    b = torch.randn((bt, K, N), device=dev, generator=g)
    c = torch.full((bt, M, N), float("nan"), device=dev)
    sa.tensor_batch_matmul(a, b, c)
    torch.cuda.synchronize()
    want = np.matmul(a.cpu().double().numpy(), b.cpu().double().numpy())
    _close(c.cpu().numpy(), want)
