"""GPU parity of gemm_f32_ring, the fp32 MFMA kernel fed by an LDS-DMA ring,
through every entry point that reaches it: tensor_matmul_f32 (B[K,N]),
tensor_matmul_nt_f32 and tensor_matmul_nhwc (B_T rows), and the accumulating
matmul builtin (C += A B at element offsets, ConvertSimpToMemRef.cpp:1794-1920).
The dispatch takes it for products with K % 32 == 0 and 16-byte aligned rows
once the tiles cover the chip: with K <= 256 64x64 tiles four workgroups per
CU, else 256x128 tiles from 512 of them (8 waves of 128x32), else 128x128
tiles from 256 of them, else 64x64 tiles from 256 of them.
Cases cover every form with ragged M and N (rows and columns past the edge load
clamped addresses and must not be stored), one and two K-stages, and several
tiles per workgroup (the persistent loop).

Reference: float64 products (numpy's BLAS).  Tolerance 1e-4 of max|ref|, the
bar of the other fp32 tests; C starts as NaN so an unwritten element fails.
"""
import numpy as np
import pytest

import simplang_amd as sa

pytestmark = pytest.mark.gpu
TOL = 1e-4


def _close(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    assert np.isfinite(got).all()
    err = np.abs(got - want).max()
    assert err <= TOL * np.abs(want).max(), (err, np.abs(want).max())


def _rand(rng, *shape):
    return rng.standard_normal(shape).astype(np.float32)


# (M, K, N): 64x64 tiles (16x17 = 272 tiles, ragged both ways); one and two
# K-stages (short K: 64x64 tiles, up to four workgroups per CU); 64x64 tiles
# two per workgroup (2x510 tiles on 512 workgroups, M ragged); 128x128 tiles
# ragged (16x17 tiles on 256 workgroups); 128x128 tiles two per workgroup;
# 256x128 tiles ragged both ways (16x33 tiles on 256 workgroups, some with three)
SHAPES = [(1000, 2048, 1028), (1024, 32, 1024), (1088, 64, 1024), (120, 320, 32640),
          (2000, 320, 2052), (2048, 512, 4096), (4000, 320, 4100)]


@pytest.mark.parametrize("M,K,N", SHAPES)
def test_ring_tensor_matmul(dev, M, K, N):
    import torch
    print(f"[f32-ring] tensor_matmul M={M} K={K} N={N}", flush=True)
    rng = np.random.default_rng(M + K + N)
    a, b = _rand(rng, M, K), _rand(rng, K, N)
    c = torch.full((M, N), float("nan"), device=dev)
    sa.tensor_matmul_f32(torch.from_numpy(a).to(dev), torch.from_numpy(b).to(dev), c)
    torch.cuda.synchronize()
    _close(c.cpu().numpy(), a.astype(np.float64) @ b)


@pytest.mark.parametrize("M,K,N", SHAPES)
def test_ring_tensor_matmul_nt(dev, M, K, N):
    import torch
    print(f"[f32-ring] tensor_matmul_nt M={M} K={K} N={N}", flush=True)
    rng = np.random.default_rng(M * 3 + K + N)
    a, bt = _rand(rng, M, K), _rand(rng, N, K)
    c = torch.full((M, N), float("nan"), device=dev)
    sa.tensor_matmul_nt_f32(torch.from_numpy(a).to(dev), torch.from_numpy(bt).to(dev), c)
    torch.cuda.synchronize()
    _close(c.cpu().numpy(), a.astype(np.float64) @ bt.astype(np.float64).T)


@pytest.mark.parametrize("m,k,n", [(512, 256, 2048), (2048, 96, 2048)])
def test_ring_matmul_accumulates_at_offsets(dev, m, k, n):
    """matmul builtin: out[m,n] += lhs[m,k] rhs[k,n], offsets of 4/8/12 floats
    (16-byte aligned, so the ring kernel runs with beta = 1); the elements before
    the offsets stay untouched."""
    import torch
    print(f"[f32-ring] matmul m={m} k={k} n={n}", flush=True)
    rng = np.random.default_rng(m + k * n)
    a = _rand(rng, 4 + m * k)
    b = _rand(rng, 8 + k * n)
    c = _rand(rng, 12 + m * n)
    tc = torch.from_numpy(c).to(dev)
    sa.matmul(torch.from_numpy(a).to(dev), torch.from_numpy(b).to(dev), tc, m, k, n, 4, 8, 12)
    torch.cuda.synchronize()
    got = tc.cpu().numpy()
    want = c[12:].reshape(m, n).astype(np.float64) + \
        a[4:].reshape(m, k).astype(np.float64) @ b[8:].reshape(k, n)
    _close(got[12:].reshape(m, n), want)
    assert (got[:12] == c[:12]).all()


def test_ring_nhwc(dev):
    """tensor_matmul_nhwc: (N,H,W) collapse to 4096 rows against W[256, 64]."""
    import torch
    print("[f32-ring] nhwc 4x32x32x64 -> 256", flush=True)
    rng = np.random.default_rng(11)
    x, w = _rand(rng, 4, 32, 32, 64), _rand(rng, 256, 64)
    y = torch.full((4, 32, 32, 256), float("nan"), device=dev)
    sa.tensor_matmul_nhwc(torch.from_numpy(x).to(dev), torch.from_numpy(w).to(dev), y)
    torch.cuda.synchronize()
    want = x.reshape(-1, 64).astype(np.float64) @ w.astype(np.float64).T
    _close(y.cpu().numpy().reshape(-1, 256), want)


@pytest.mark.parametrize("bt,M,K,N", [(16, 200, 64, 260), (24, 300, 320, 400), (32, 512, 128, 512)])
def test_ring_batch(dev, bt, M, K, N):
    """tensor_batch_matmul: the batch's products share one persistent launch
    (16 x 4 x 5 and 32 x 8 x 8 tiles of 64x64 at K <= 256; 24 x 3 x 4 tiles of
    128x128 at K = 320, two per workgroup for some), ragged M and N in the
    first two."""
    import torch
    print(f"[f32-ring] batch {bt} x ({M}x{K}x{N})", flush=True)
    rng = np.random.default_rng(bt * M + K + N)
    a, b = _rand(rng, bt, M, K), _rand(rng, bt, K, N)
    c = torch.full((bt, M, N), float("nan"), device=dev)
    sa.tensor_batch_matmul(torch.from_numpy(a).to(dev), torch.from_numpy(b).to(dev), c)
    torch.cuda.synchronize()
    _close(c.cpu().numpy(), np.matmul(a.astype(np.float64), b.astype(np.float64)))
