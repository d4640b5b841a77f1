"""GPU parity of the packed-i4 tensor_matmul against the pinned oracle.

Bit-exact: C = i16(sum_k A*B) with A, B signed nibbles (ConvertSimpToMemRef.cpp:
2953-3133).  Golden checksums of the reference's int4 benchmark recipe, random
shapes with odd K / N (half-used last byte, whose pad nibble must be ignored),
the i16 wraparound, and a full-size shape on the large-tile path checked against
the oracle's exact int8 product of the unpacked values.
"""
import json
import os

import numpy as np
import pytest

import simplang_amd as sa

pytestmark = pytest.mark.gpu


def _run(dev, ap, bp, M, N, c_view=None):
    import torch
    ta = torch.from_numpy(np.ascontiguousarray(ap).view(np.int8)).to(dev)
    tb = torch.from_numpy(np.ascontiguousarray(bp).view(np.int8)).to(dev)
    tc = torch.full((M, N), -7, dtype=torch.int16, device=dev) if c_view is None else c_view
    sa.tensor_matmul_i4(ta, tb, tc)
    torch.cuda.synchronize()
    return tc


def test_i4_recipe_checksums(dev, orc):
    gold = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                       "int4_recipe_checksums.json")))
    for n_str, want in gold["checksums"].items():
        n = int(n_str)
        print(f"[i4-recipe] N={n}", flush=True)
        ap, bp = orc.int4_recipe_inputs(n)
        got = _run(dev, ap, bp, n, n).cpu().numpy()
        assert orc.checksum_i16(got) == want, n


@pytest.mark.parametrize("M,N,K", [(5, 7, 9), (64, 128, 256), (33, 18, 101), (300, 517, 1001),
                                   (1, 8640, 3200), (8, 2048, 768), (1, 1, 1)])
def test_i4_random_vs_oracle(dev, orc, M, N, K):
    print(f"[i4] M={M} N={N} K={K}", flush=True)
    rng = np.random.default_rng(M * 7 + N * 13 + K)
    ap = orc.pack_i4(rng.integers(-8, 8, (M, K)), axis=1)
    bp = orc.pack_i4(rng.integers(-8, 8, (K, N)), axis=1)
    # garbage in the pad nibble of odd-length rows: not an element, must be ignored
    if K % 2:
        ap[:, -1] |= 0xA0
    if N % 2:
        bp[:, -1] |= 0x90
    want = orc.matmul_i4(ap, bp, M, N, K)
    got = _run(dev, ap, bp, M, N).cpu().numpy()
    assert np.array_equal(got, want)


def test_i4_wraps_to_i16(dev, orc):
    K = 1100                                     # 1100 * 64 = 70400 -> 4864
    ap = orc.pack_i4(np.full((3, K), -8), axis=1)
    bp = orc.pack_i4(np.full((K, 5), -8), axis=1)
    got = _run(dev, ap, bp, 3, 5).cpu().numpy()
    assert (got == 4864).all()


def test_i4_large_tile_path_and_strided_c(dev, orc):
    """4096 x 4112 x 1030: the unpacked product runs on the large-tile LDS-DMA
    kernel; C is a strided view.  Checked against the oracle's exact int8 VNNI
    product of the unpacked nibbles, truncated to i16."""
    import torch
    M, N, K = 4096, 4112, 1030
    print(f"[i4-large] M={M} N={N} K={K}", flush=True)
    rng = np.random.default_rng(7)
    a = rng.integers(-8, 8, (M, K)).astype(np.int8)
    b = rng.integers(-8, 8, (K, N)).astype(np.int8)
    want32, _ = orc.matmul_i8_vnni(a, b, nthreads=8)
    want = want32.astype(np.int16)
    c_full = torch.full((M, N + 3), -7, dtype=torch.int16, device=dev)
    tc = c_full[:, 2:N + 2]
    _run(dev, orc.pack_i4(a, 1), orc.pack_i4(b, 1), M, N, c_view=tc)
    out = c_full.cpu().numpy()
    assert np.array_equal(out[:, 2:N + 2], want)
    assert (out[:, :2] == -7).all() and (out[:, N + 2:] == -7).all()


def test_i4_shape_errors(dev):
    import torch
    a = torch.zeros((4, 3), dtype=torch.int8, device=dev)    # K = 5 or 6
    b = torch.zeros((5, 4), dtype=torch.int8, device=dev)    # K = 5, N = 7 or 8
    c = torch.zeros((4, 9), dtype=torch.int16, device=dev)   # N = 9: B would need 5 bytes
    with pytest.raises(sa.SimpRTError):
        sa.tensor_matmul_i4(a, b, c)
    c = torch.zeros((4, 8), dtype=torch.int16, device=dev)
    sa.tensor_matmul_i4(a, b, c)
