"""simp_rt_matmul_u8s8_i32_noalloc (the allocation-free variant of
simp_rt_matmul_u8s8_i32, whose large-shape scratch lives in a static device
array) against simp_rt_matmul_u8s8_i32 itself, bit for bit, through the C ABI:
two calls in a row that transpose B into the scratch (K % 64 != 0: column sums
and B_T in the scratch), the second smaller, so it must clear and refill what
the first left; large-tile calls with B read in place, whose column sums the
GEMM kernel forms itself (no scratch: M = 8192 with tiles grouped by columns,
M = 4096 by rows); a small shape (no scratch); and the documented rejections
(host operands, a scratch need above the maximum)."""
import numpy as np
import pytest

import simplang_amd as sa

pytestmark = pytest.mark.gpu


def _pair(dev, M, N, K, seed):
    import torch
    g = torch.Generator(device=dev).manual_seed(seed)
    a = torch.randint(0, 256, (M, K), dtype=torch.uint8, device=dev, generator=g)
    b = torch.randint(-128, 128, (K, N), dtype=torch.int8, device=dev, generator=g)
    return a, b


def test_noalloc_matches_allocating_entry_point(dev):
    import torch
    for (M, N, K, seed) in ((8192, 4096, 2048, 1), (8192, 2048, 1024, 2),
                            (4096, 4096, 2064, 4), (4096, 4096, 1040, 5),
                            (4096, 4096, 1024, 6), (256, 320, 192, 3)):
        print(f"[noalloc] M={M} N={N} K={K}", flush=True)
        a, b = _pair(dev, M, N, K, seed)
        want = torch.empty((M, N), dtype=torch.int32, device=dev)
        got = torch.full((M, N), -1, dtype=torch.int32, device=dev)
        sa.matmul_u8s8_i32(a, b, want)
        sa.matmul_u8s8_i32_noalloc(a, b, got)
        torch.cuda.synchronize()
        assert torch.equal(got, want), (M, N, K)


@pytest.mark.parametrize("M,N,K", [(8192, 2048, 1024), (2048, 3072, 1040), (4096, 4096, 1024),
                                   (256, 320, 192)])
def test_noalloc_under_graph_capture(dev, M, N, K):
    """The entry point's callers capture it: one call captured in a HIP graph
    (B transposed into the scratch, and three shapes with no scratch: B read in
    place with the column sums formed in the large-tile kernel, by column and
    by row groups of tiles, and a small shape), replayed three times on new
    inputs written into the captured
    buffers, with eager library work between the replays (which uses the same
    scratch-free stream workspace); every replay equals the allocating entry
    point bit for bit."""
    import torch
    print(f"[noalloc-graph] M={M} N={N} K={K}", flush=True)
    a, b = _pair(dev, M, N, K, seed=M + K)
    c = torch.empty((M, N), dtype=torch.int32, device=dev)
    main = torch.cuda.current_stream()
    side = torch.cuda.Stream()
    side.wait_stream(main)
    with torch.cuda.stream(side):          # first use on this stream, outside the capture
        sa.set_stream(side)
        sa.matmul_u8s8_i32_noalloc(a, b, c)
    main.wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        sa.set_stream(side)
        sa.matmul_u8s8_i32_noalloc(a, b, c)
    sa.set_stream(main)
    want = torch.empty_like(c)
    for rep in range(3):
        na, nb = _pair(dev, M, N, K, seed=100 * rep + 7)
        a.copy_(na)
        b.copy_(nb)
        c.fill_(-1)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        sa.matmul_u8s8_i32(a, b, want)       # eager work between the replays
        torch.cuda.synchronize()
        assert torch.equal(c, want), (rep, M, N, K)


def test_noalloc_rejections(dev):
    import torch
    a = np.zeros((64, 64), np.uint8)                       # host memory: would need staging
    b = np.zeros((64, 64), np.int8)
    c = np.zeros((64, 64), np.int32)
    with pytest.raises(sa.SimpRTError):
        sa.matmul_u8s8_i32_noalloc(a, b, c)
    M, N, K = 2048, 16384, 8208                            # K % 64 != 0: B_T of 128 MiB > the maximum
    print(f"[noalloc] rejection M={M} N={N} K={K}", flush=True)
    da = torch.zeros((M, K), dtype=torch.uint8, device=dev)
    db = torch.zeros((K, N), dtype=torch.int8, device=dev)
    dc = torch.zeros((M, N), dtype=torch.int32, device=dev)
    with pytest.raises(sa.SimpRTError, match="allocation-free maximum"):
        sa.matmul_u8s8_i32_noalloc(da, db, dc)
