"""GPU parity of the rank-3 (batched), rank-4 (NHWC) and f64 tensor_matmul
entry points against the pinned oracle and the reference's known answers.

Tolerances: f32 within 1e-4 of max|ref| (ref: the oracle's float64 sums),
f64 within 1e-12; i8 -> i32 bit-exact.
"""
import numpy as np
import pytest

import simplang_amd as sa

pytestmark = pytest.mark.gpu


def _t(dev, a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _close(got, want, tol):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    err = np.abs(got - want).max() if want.size else 0.0
    assert err <= tol * max(np.abs(want).max(), 1e-30), (err, np.abs(want).max())


TOL = {np.float32: 1e-4, np.float64: 1e-12}


def _rand(rng, shape, dt):
    if dt == np.int8:
        return rng.integers(-128, 128, shape, dtype=np.int8)
    return rng.standard_normal(shape).astype(dt)


def _out_dtype(dt):
    import torch
    return {np.float32: torch.float32, np.float64: torch.float64, np.int8: torch.int32}[dt]


def _check(got, want, dt):
    if dt == np.int8:
        assert (np.asarray(got) == want).all()
    else:
        _close(got, want, TOL[dt])


# ---------------------------------------------------------------- known answers --

def test_batch_kats(dev):
    import torch
    a = _t(dev, np.arange(1, 13, dtype=np.float32).reshape(2, 2, 3))
    b = _t(dev, np.tile(np.array([1, 0, 0, 1, 1, 1], np.float32), 2).reshape(2, 3, 2))
    c = torch.full((2, 2, 2), 7.0, device=dev)           # overwritten, not accumulated
    sa.tensor_batch_matmul(a, b, c)
    assert (c[0, 0, 0] + c[1, 0, 0]).item() == 20.0      # test_matmul_dot.sl:135-161
    eye = np.eye(3, dtype=np.float32)
    a = _t(dev, np.stack([eye, 2 * eye, 3 * eye]))
    b = _t(dev, np.stack([5 * eye, 4 * eye, 2 * eye]))
    c = torch.empty(3, 3, 3, device=dev)
    sa.tensor_batch_matmul(a, b, c)
    assert (c[0, 0, 0] + c[1, 1, 1] + c[2, 2, 2]).item() == 19.0  # :164-199
    # tests/test_tensor_matmul.sl:66-117 (f64) and :121-145 (f64 2x2)
    bb, ii, jj = np.meshgrid(np.arange(2), np.arange(3), np.arange(4), indexing="ij")
    A = ((bb + 1) * (ii + jj)).astype(np.float64)
    bb, ii, jj = np.meshgrid(np.arange(2), np.arange(4), np.arange(3), indexing="ij")
    B = ((bb + 1) * (ii + 1)).astype(np.float64)
    c = torch.empty(2, 3, 3, dtype=torch.float64, device=dev)
    sa.tensor_batch_matmul(_t(dev, A), _t(dev, B), c)
    assert c[0, 0, 0].item() == 20.0
    c2 = torch.empty(2, 2, dtype=torch.float64, device=dev)
    sa.tensor_matmul_f64(_t(dev, np.array([[1., 2.], [3., 4.]])), _t(dev, np.eye(2)), c2)
    assert c2[0, 0].item() == 1.0 and c2.cpu().numpy().tolist() == [[1., 2.], [3., 4.]]


def test_nhwc_kats(dev):
    import torch
    x = _t(dev, np.arange(1, 25, dtype=np.float32).reshape(2, 2, 2, 3))
    w = _t(dev, np.array([[1, 0, 0], [0, 1, 0], [0, 0, 1], [.5, .5, .5]], np.float32))
    y = torch.empty(2, 2, 2, 4, device=dev)
    sa.tensor_matmul_nhwc(x, w, y)
    assert (y[0, 0, 0, 0] + y[0, 0, 0, 3]).item() == 4.0  # test_matmul_dot.sl:204-236
    x = _t(dev, np.repeat(np.arange(1, 19, dtype=np.float32), 2).reshape(2, 3, 3, 2))
    w = _t(dev, np.array([[1, 1], [2, 2], [3, 3]], np.float32))
    y = torch.empty(2, 3, 3, 3, device=dev)
    sa.tensor_matmul_nhwc(x, w, y)
    assert (y[0, 0, 0, 0] + y[0, 0, 0, 1] + y[0, 0, 0, 2]).item() == 12.0  # :239-268


# ------------------------------------------------------------------ vs the oracle --

SHAPES = [(1, 1, 1, 1), (3, 7, 13, 5), (2, 64, 64, 64), (5, 65, 129, 63), (32, 17, 64, 100),
          (1, 300, 256, 1), (4, 1, 768, 1), (2, 96, 48, 130), (8, 128, 128, 128),
          (3, 40, 1024, 64), (2, 20, 512, 128)]


@pytest.mark.parametrize("dt", [np.float32, np.float64, np.int8])
@pytest.mark.parametrize("bt,m,k,n", SHAPES)
def test_batch_vs_oracle(dev, orc, dt, bt, m, k, n):
    import torch
    rng = np.random.default_rng(bt * 1000 + m * 7 + k * 3 + n)
    a = _rand(rng, (bt, m, k), dt)
    b = _rand(rng, (bt, k, n), dt)
    c = torch.empty(bt, m, n, dtype=_out_dtype(dt), device=dev)
    print(f"batch {dt.__name__} Bt={bt} M={m} K={k} N={n}", flush=True)
    sa.tensor_batch_matmul(_t(dev, a), _t(dev, b), c)
    torch.cuda.synchronize()
    _check(c.cpu().numpy(), orc.batch_matmul(a, b), dt)


@pytest.mark.parametrize("dt", [np.float32, np.int8])
def test_batch_strided_views(dev, orc, dt):
    """Padded rows and batch gaps: operands are views into larger buffers."""
    import torch
    rng = np.random.default_rng(7)
    bt, m, k, n = 3, 33, 80, 48
    A = _t(dev, _rand(rng, (bt, m + 5, k + 16), dt))
    B = _t(dev, _rand(rng, (bt + 1, k + 3, n + 16), dt))
    C = torch.zeros(bt, m + 2, n + 32, dtype=_out_dtype(dt), device=dev)
    a, b, c = A[:, 2:2 + m, 16:16 + k], B[1:, :k, :n], C[:, 1:1 + m, 16:16 + n]
    sa.tensor_batch_matmul(a, b, c)
    torch.cuda.synchronize()
    want = orc.batch_matmul(a.cpu().numpy(), b.cpu().numpy())
    _check(c.cpu().numpy(), want, dt)
    Cn = C.cpu().numpy()
    assert (Cn[:, 0] == 0).all() and (Cn[:, 1 + m:] == 0).all()  # outside the view untouched
    assert (Cn[:, :, :16] == 0).all() and (Cn[:, :, 16 + n:] == 0).all()


def test_batch_i8_large_products_equal_2d(dev):
    """Products big enough to fill the chip alone run one dispatch each; every
    batch must equal the rank-2 entry point (itself pinned to the oracle)."""
    import torch
    g = torch.Generator(device=dev).manual_seed(3)
    bt, m, k, n = 2, 4096, 256, 4096
    a = torch.randint(-128, 128, (bt, m, k), generator=g, device=dev, dtype=torch.int8)
    b = torch.randint(-128, 128, (bt, k, n), generator=g, device=dev, dtype=torch.int8)
    c = torch.empty(bt, m, n, dtype=torch.int32, device=dev)
    sa.tensor_batch_matmul(a, b, c)
    for i in range(bt):
        ci = torch.empty(m, n, dtype=torch.int32, device=dev)
        sa.tensor_matmul_i8(a[i], b[i], ci)
        assert torch.equal(c[i], ci)


@pytest.mark.parametrize("dt", [np.float32, np.int8])
def test_batch_over_grid_limit(dev, orc, dt):
    """More than 65535 products (grid z is launched in chunks)."""
    import torch
    rng = np.random.default_rng(11)
    bt = 70000
    a = _rand(rng, (bt, 2, 3), dt)
    b = _rand(rng, (bt, 3, 2), dt)
    c = torch.empty(bt, 2, 2, dtype=_out_dtype(dt), device=dev)
    sa.tensor_batch_matmul(_t(dev, a), _t(dev, b), c)
    torch.cuda.synchronize()
    _check(c.cpu().numpy(), orc.batch_matmul(a, b), dt)


def test_batch_host_operands(orc):
    """Plain numpy operands are staged through device memory."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    rng = np.random.default_rng(5)
    a = rng.standard_normal((4, 20, 30)).astype(np.float32)
    b = rng.standard_normal((4, 30, 10)).astype(np.float32)
    c = np.zeros((4, 20, 10), np.float32)
    sa.tensor_batch_matmul(a, b, c)
    _close(c, orc.batch_matmul(a, b), 1e-4)


@pytest.mark.parametrize("dt", [np.float32, np.float64])
@pytest.mark.parametrize("shape,cout", [((2, 5, 7, 33), 17), ((1, 1, 1, 256), 100),
                                        ((4, 8, 8, 64), 128), ((1, 3, 1, 5), 1)])
def test_nhwc_vs_oracle(dev, orc, dt, shape, cout):
    import torch
    rng = np.random.default_rng(sum(shape) + cout)
    x = rng.standard_normal(shape).astype(dt)
    w = rng.standard_normal((cout, shape[3])).astype(dt)
    y = torch.empty(*shape[:3], cout, dtype=_out_dtype(dt), device=dev)
    sa.tensor_matmul_nhwc(_t(dev, x), _t(dev, w), y)
    torch.cuda.synchronize()
    _check(y.cpu().numpy(), orc.matmul_nhwc(x, w), dt)


@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (37, 100, 29), (128, 64, 256), (200, 300, 1)])
def test_matmul_f64_vs_oracle(dev, orc, m, k, n):
    import torch
    rng = np.random.default_rng(m + k + n)
    a = rng.standard_normal((m, k))
    b = rng.standard_normal((k, n))
    c = torch.empty(m, n, dtype=torch.float64, device=dev)
    sa.tensor_matmul_f64(_t(dev, a), _t(dev, b), c)
    torch.cuda.synchronize()
    _close(c.cpu().numpy(), orc.batch_matmul(a[None], b[None])[0], 1e-12)


# --------------------------------------------------------------------- rejects --

def test_rejects(dev):
    import torch
    f = lambda *s: torch.empty(*s, device=dev)
    with pytest.raises(sa.SimpRTError, match="shape mismatch"):
        sa.tensor_batch_matmul(f(2, 3, 4), f(3, 4, 5), f(2, 3, 5))
    with pytest.raises(sa.SimpRTError, match="shape mismatch"):
        sa.tensor_batch_matmul(f(2, 3, 4), f(2, 4, 5), f(2, 3, 6))
    with pytest.raises(sa.SimpRTError, match="inner stride"):
        sa.tensor_batch_matmul(f(2, 4, 3).transpose(1, 2), f(2, 4, 5), f(2, 3, 5))
    with pytest.raises(sa.SimpRTError, match="stride 0"):            # batches overlap
        sa.tensor_batch_matmul(f(1, 3, 4).expand(2, 3, 4), f(2, 4, 5), f(2, 3, 5))
    with pytest.raises(sa.SimpRTError, match="collapse"):
        x = f(2, 3, 8, 4)[:, :, :5, :]                                # W padded: rows not one run
        sa.tensor_matmul_nhwc(x, f(6, 4), f(2, 3, 5, 6))
    with pytest.raises(sa.SimpRTError, match="shape mismatch"):
        sa.tensor_matmul_nhwc(f(2, 3, 5, 4), f(6, 3), f(2, 3, 5, 6))
    with pytest.raises(TypeError):
        sa.tensor_batch_matmul(torch.empty(2, 2, 2, dtype=torch.int32, device=dev),
                               torch.empty(2, 2, 2, dtype=torch.int32, device=dev),
                               torch.empty(2, 2, 2, dtype=torch.int32, device=dev))


@pytest.mark.parametrize("dt", [np.float32, np.int8])
def test_batch_strided_views_host_arrays(dev, orc, dt):
    """Padded rows and batch gaps with numpy host operands (staged): the bytes
    of the output buffer outside the view keep their values."""
    rng = np.random.default_rng(8)
    bt, m, k, n = 3, 33, 80, 48
    A = _rand(rng, (bt, m + 5, k + 16), dt)
    B = _rand(rng, (bt + 1, k + 3, n + 16), dt)
    odt = np.float32 if dt == np.float32 else np.int32
    C = np.full((bt, m + 2, n + 32), 77, dtype=odt)
    a, b, c = A[:, 2:2 + m, 16:16 + k], B[1:, :k, :n], C[:, 1:1 + m, 16:16 + n]
    sa.tensor_batch_matmul(a, b, c)
    want = orc.batch_matmul(np.ascontiguousarray(a), np.ascontiguousarray(b))
    _check(np.ascontiguousarray(c), want, dt)
    assert (C[:, 0] == 77).all() and (C[:, 1 + m:] == 77).all()
    assert (C[:, :, :16] == 77).all() and (C[:, :, 16 + n:] == 77).all()
