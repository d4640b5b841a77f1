"""GPU parity of the W4 GEMV / skinny GEMM entry points against the oracle.

fp32 results are compared with the oracle's double-precision value of the same
dequantised product.  Tolerance (written here, from BASELINE's 1e-4 relative):
normwise  max|gpu - ref| <= 1e-4 * max|ref|  for every output row of x.
"""
import numpy as np
import pytest

import simplang_amd as sa

pytestmark = pytest.mark.gpu

TOL = 1e-4


def _w4s_inputs(M, N, K, gs, seed):
    """q uniform in [-8,7], scale |N(0,0.02)|/7 per group, x ~ N(0,1)."""
    rng = np.random.default_rng(seed)
    q = rng.integers(-8, 8, (N, K))
    nib = (q & 15).astype(np.uint8)
    w = (nib[:, 0::2] | (nib[:, 1::2] << 4)).astype(np.uint8)
    s = (np.abs(rng.standard_normal((N, K // gs))) * 0.02 / 7).astype(np.float32)
    x = rng.standard_normal((M, K)).astype(np.float32)
    return w, s, x


def _close(got, want):
    for m in range(want.shape[0]):
        err = np.abs(got[m].astype(np.float64) - want[m]).max()
        assert err <= TOL * np.abs(want[m]).max(), (m, err, np.abs(want[m]).max())


@pytest.mark.parametrize("K,N", [(3200, 8640), (8640, 3200), (3200, 32000)])
@pytest.mark.parametrize("M", [1, 4, 16])
def test_w4s_baseline_shapes(dev, orc, M, N, K):
    import torch
    print(f"[w4s] M={M} N={N} K={K}", flush=True)
    w, s, x = _w4s_inputs(M, N, K, 32, seed=M * 31 + N + K)
    tw, ts, tx = (torch.from_numpy(a).to(dev) for a in (w, s, x))
    out = torch.full((M, N), float("nan"), device=dev)
    sa.matmul_w4s(tw, ts, tx, out, 32)
    torch.cuda.synchronize()
    _close(out.cpu().numpy(), orc.matmul_w4s(w, s, x, 32).astype(np.float64))


@pytest.mark.parametrize("M,N,K,gs", [(3, 17, 96, 32), (2, 100, 256, 64), (5, 33, 512, 128),
                                      (1, 1, 32, 32), (16, 70, 640, 32),
                                      (2, 9, 40, 8),      # K % 32 != 0: generic kernel
                                      (17, 12, 64, 32),   # M > 16: generic kernel
                                      # M = 1, long rows over few blocks: 8-wave kernel
                                      (1, 1003, 16384, 32), (1, 2000, 12320, 32),
                                      (1, 100, 4128, 96)])
def test_w4s_ragged_and_fallback(dev, orc, M, N, K, gs):
    import torch
    w, s, x = _w4s_inputs(M, N, K, gs, seed=N * 7 + K)
    out = torch.empty((M, N), device=dev)
    sa.matmul_w4s(*(torch.from_numpy(a).to(dev) for a in (w, s, x)), out, gs)
    torch.cuda.synchronize()
    _close(out.cpu().numpy(), orc.matmul_w4s(w, s, x, gs).astype(np.float64))


@pytest.mark.parametrize("M", [2, 3, 4])
@pytest.mark.parametrize("N,K,gs", [(100, 2048, 32), (300, 4096, 64), (257, 6144, 32),
                                    (640, 8640, 32), (96, 16384, 128)])
def test_w4s_few_vectors_views(dev, orc, M, N, K, gs):
    """2 <= M <= 4 runs the dot8 kernel with every vector's limbs in registers;
    x and out as row windows of wider arrays (ldx = K + 4, ldo = N + 3), every
    chunks-per-row configuration, group sizes 32 / 64 / 128."""
    import torch
    print(f"[w4s-mx] M={M} N={N} K={K} gs={gs}", flush=True)
    w, s, x = _w4s_inputs(M, N, K, gs, seed=M * 7 + N + K)
    tx = torch.zeros((M, K + 4), device=dev)
    tx[:, :K] = torch.from_numpy(x).to(dev)
    out = torch.full((M, N + 3), -3.0, device=dev)
    sa.matmul_w4s(torch.from_numpy(w).to(dev), torch.from_numpy(s).to(dev), tx[:, :K],
                  out[:, :N], gs)
    torch.cuda.synchronize()
    o = out.cpu().numpy()
    _close(o[:, :N], orc.matmul_w4s(w, s, x, gs).astype(np.float64))
    assert (o[:, N:] == -3.0).all()


def _f5_model(layers, rows, cols, gs, seed):
    """A concatenated reference-format weight buffer (examples/llama2/llama2_quant.sl
    layout) quantised with the reference's quantizer."""
    rng = np.random.default_rng(seed)
    w = rng.uniform(-0.01, 0.01, layers * rows * cols).astype(np.float32)
    return w


@pytest.mark.parametrize("rows,cols", [(1536, 1536), (6144, 1536), (1536, 6144), (100, 224)])
def test_matmul_quant_reference_format(dev, orc, rows, cols):
    """Reference W4 (u4 + zero, gs 128) on the llama2_quant.sl shapes, at layer 0
    and at a later layer's offset (whose scales the reference itself misreads)."""
    import torch
    gs = 128 if cols % 128 == 0 else 32
    layers = 3
    w = _f5_model(layers, rows, cols, gs, seed=rows + cols)
    qw, sc, ze = orc.quantize_f5(w, gs)
    x = np.random.default_rng(1).standard_normal(cols).astype(np.float32)
    tq, tsc, tze, tx = (torch.from_numpy(a).to(dev) for a in (qw.view(np.int8), sc, ze, x))
    for layer in (0, 2):
        off = layer * rows * cols
        out = torch.full((rows,), float("nan"), device=dev)
        sa.matmul_quant(tq, tsc, tze, tx, out, rows, cols, gs, off)
        torch.cuda.synchronize()
        ref = orc.matmul_quant_f5(qw, sc, ze, x, rows, cols, gs, off).astype(np.float64)
        _close(out.cpu().numpy()[None], ref[None])


def test_matmul_quant_roofline_kat(dev):
    """test_quant_roofline.cpp:71-92 constants: 0x55 bytes, scale 0.01, zero 0 -> w = 0.05."""
    import torch
    rows, cols, gs = 64, 1536, 128
    qw = torch.full((rows * cols // 2,), 0x55, dtype=torch.uint8, device=dev).view(torch.int8)
    sc = torch.full((rows * cols // gs,), 0.01, device=dev)
    ze = torch.zeros(rows * cols // gs, device=dev)
    x = torch.randn(cols, device=dev)
    out = torch.empty(rows, device=dev)
    sa.matmul_quant(qw, sc, ze, x, out, rows, cols, gs, 0)
    want = 0.05 * x.double().sum().item()
    assert np.allclose(out.cpu().numpy(), want, rtol=1e-4, atol=1e-4 * abs(want) + 1e-6)


def test_matmul_quant_unaligned_offset_fallback(dev, orc):
    """An offset that is not a multiple of 32 takes the generic kernel."""
    import torch
    rows, cols, gs = 7, 64, 16
    w = _f5_model(1, rows + 1, cols, gs, seed=3)
    qw, sc, ze = orc.quantize_f5(w, gs)
    x = np.random.default_rng(2).standard_normal(cols).astype(np.float32)
    off = 16
    out = torch.empty(rows, device=dev)
    sa.matmul_quant(*(torch.from_numpy(a).to(dev) for a in (qw.view(np.int8), sc, ze, x)), out,
                    rows, cols, gs, off)
    ref = orc.matmul_quant_f5(qw, sc, ze, x, rows, cols, gs, off).astype(np.float64)
    _close(out.cpu().numpy()[None], ref[None])


@pytest.mark.parametrize("M,nan_row", [(1, 0), (3, 1), (4, 3), (16, 5)])
@pytest.mark.parametrize("K,N", [(3200, 640), (640, 96)])
def test_w4s_nan_in_x_propagates(dev, orc, M, nan_row, K, N):
    """One NaN element of x makes every output of its row NaN, as the reference's
    fp32 multiply-adds do (ConvertSimpToMemRef.cpp:3906-4005); the other rows
    still equal the oracle."""
    import torch
    w, s, x = _w4s_inputs(M, N, K, 32, seed=M + K)
    x[nan_row, K // 3] = np.nan
    out = torch.zeros((M, N), device=dev)
    sa.matmul_w4s(*(torch.from_numpy(a).to(dev) for a in (w, s, x)), out, 32)
    torch.cuda.synchronize()
    o = out.cpu().numpy()
    assert np.isnan(o[nan_row]).all()
    keep = [m for m in range(M) if m != nan_row]
    if keep:
        _close(o[keep], orc.matmul_w4s(w, s, x[keep], 32).astype(np.float64))


def test_matmul_quant_nan_in_x_propagates(dev, orc):
    import torch
    rows, cols, gs = 1536, 1536, 128
    qw, sc, ze = orc.quantize_f5(_f5_model(1, rows, cols, gs, seed=5), gs)
    x = np.random.default_rng(4).standard_normal(cols).astype(np.float32)
    x[777] = np.nan
    out = torch.zeros(rows, device=dev)
    sa.matmul_quant(*(torch.from_numpy(a).to(dev) for a in (qw.view(np.int8), sc, ze, x)), out,
                    rows, cols, gs, 0)
    torch.cuda.synchronize()
    assert np.isnan(out.cpu().numpy()).all()


@pytest.mark.parametrize("idx,count,gs", [(0, 1536 * 64, 128), (37, 1000, 32), (1, 1, 128),
                                          (2 * 1536 * 64 - 5, 5, 128)])
def test_dequant_w4_bit_exact(dev, orc, idx, count, gs):
    """dequant_w4 over a range (ConvertSimpToMemRef.cpp:2367-2429) equals the
    oracle bit for bit, from device arrays and from host arrays (where only the
    range's bytes and groups are staged)."""
    import torch
    w = _f5_model(2, 1536, 64, gs, seed=gs + idx)
    qw, sc, ze = orc.quantize_f5(w, gs)
    want = orc.dequant_w4(qw, sc, ze, idx, count, gs)
    out = torch.full((count,), float("nan"), device=dev)
    sa.dequant_w4(*(torch.from_numpy(a).to(dev) for a in (qw.view(np.int8), sc, ze)), idx, gs, out)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), want)
    host = np.full(count, np.nan, np.float32)
    sa.dequant_w4(qw.view(np.int8), sc, ze, idx, gs, host)
    assert np.array_equal(host, want)
