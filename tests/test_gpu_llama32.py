"""GPU parity of llama32_forward (the int8 LLaMA-3.2 program,
examples/llama2/llama32_1b_int8_tensor.sl) against the oracle's statement-by-
statement restatement, called as bench_llama32_1b_int8.cpp calls it.

Integer stages (the int8 projections, the int8 KV cache rows) must match
exactly; fp32 outputs (logits, x_fp32, xb_fp32) within 1e-4 of their max
magnitude.  The weights are drawn so that every stage is non-trivial (RMSNorm
weights near 1); the benchmark's own init (RMSNorm weights ~0.01) leaves the
FFN output at zero, and is run too."""
import numpy as np
import pytest

import simplang_amd as sa
from _llama32 import CFG_SMALL, DIMS, make_arrays

pytestmark = pytest.mark.gpu
TOL = 1e-4


def _close(got, want, tol=TOL):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    err = np.abs(got - want).max()
    assert err <= tol * max(np.abs(want).max(), 1e-30), (err, np.abs(want).max())


def _run(orc, cfg, gpu_arrays, ref_arrays, positions, seed):
    import torch
    rng = np.random.default_rng(seed)
    dims = [cfg[k] for k in DIMS]
    kv = cfg["n_kv_heads"] * cfg["head_dim"]
    S, L = cfg["max_seq_len"], cfg["n_layers"]
    for pos in positions:
        x = rng.integers(-64, 64, cfg["dim"], dtype=np.int8)
        ref_arrays["x_i8"][:] = x
        if isinstance(gpu_arrays["x_i8"], np.ndarray):
            gpu_arrays["x_i8"][:] = x
        else:
            gpu_arrays["x_i8"].copy_(torch.from_numpy(x))
        print(f"[llama32] pos={pos}", flush=True)
        r = sa.llama32_forward(gpu_arrays, pos, *dims)
        want = orc.llama32_int8_forward(ref_arrays, pos, *dims)
        host = {k: (v if isinstance(v, np.ndarray) else v.cpu().numpy()) for k, v in gpu_arrays.items()}
        assert r == host["logits"][0]
        _close(host["logits"], ref_arrays["logits"])
        _close(host["x_fp32"], ref_arrays["x_fp32"])
        _close(host["xb_fp32"], ref_arrays["xb_fp32"])
        for name in ("k_cache", "v_cache"):
            got = host[name].reshape(L, S, kv)[:, pos]
            exp = ref_arrays[name].reshape(L, S, kv)[:, pos]
            assert np.array_equal(got, exp), (name, pos, np.argwhere(got != exp)[:5])
        # the last layer's attention, an int32 truncation of an fp32 sum whose
        # order differs from the program's: equal, or 1 apart where the sum
        # sits at an integer
        da = np.abs(host["attn_out"].astype(np.int64) - ref_arrays["attn_out"])
        assert da.max() <= 1 and (da == 0).mean() >= 0.99, (pos, da.max(), (da != 0).sum())
        assert abs(want - r) <= TOL * max(np.abs(ref_arrays["logits"]).max(), 1e-30)


@pytest.mark.parametrize("wide", [True, False])
def test_llama32_host_arrays(dev, orc, wide):
    cfg = CFG_SMALL
    arrays = make_arrays(cfg, seed=3, wide=wide)
    ref = {k: v.copy() for k, v in arrays.items()}
    _run(orc, cfg, arrays, ref, range(12), seed=4)
    sa.forward_cache_clear()


@pytest.mark.parametrize("hs,nh,nkv", [(16, 16, 4), (48, 8, 2), (128, 4, 2), (256, 2, 1)])
def test_llama32_head_sizes(dev, orc, hs, nh, nkv):
    """The attention kernel's lane groupings: 1, 4 (one of them idle), 8 and 16
    lanes per position for the scores and 4, 12, 32 and 64 lanes per V row;
    at head size 256 the scores of positions 128..159 come from a second round
    of four load passes."""
    cfg = dict(CFG_SMALL, dim=hs * nh, n_heads=nh, n_kv_heads=nkv, head_dim=hs, n_layers=1,
               max_seq_len=160)
    arrays = make_arrays(cfg, seed=hs, wide=True)
    ref = {k: v.copy() for k, v in arrays.items()}
    _run(orc, cfg, arrays, ref, range(cfg["max_seq_len"]), seed=hs + 1)
    sa.forward_cache_clear()


def test_llama32_attention_chunks(dev, orc):
    """Contexts of more than 512 positions split the attention over blocks of
    512 and combine them: positions on both sides of every chunk boundary up
    to three chunks, caches filled with random int8 on both sides."""
    cfg = dict(CFG_SMALL, n_layers=1, max_seq_len=1100)
    arrays = make_arrays(cfg, seed=31, wide=True)
    rng = np.random.default_rng(32)
    arrays["k_cache"][:] = rng.integers(-128, 128, arrays["k_cache"].size, dtype=np.int8)
    arrays["v_cache"][:] = rng.integers(-128, 128, arrays["v_cache"].size, dtype=np.int8)
    ref = {k: v.copy() for k, v in arrays.items()}
    _run(orc, cfg, arrays, ref, (0, 510, 511, 512, 513, 1023, 1024, 1025, 1099), seed=33)
    sa.forward_cache_clear()


def test_llama32_device_arrays_long_context(dev, orc):
    """Device-resident arrays used in place; positions up to the last cache row."""
    import torch
    cfg = dict(CFG_SMALL, max_seq_len=300, n_layers=1)
    arrays = make_arrays(cfg, seed=5, wide=True)
    ref = {k: v.copy() for k, v in arrays.items()}
    darr = {k: torch.from_numpy(v).to(dev) for k, v in arrays.items()}
    _run(orc, cfg, darr, ref, range(cfg["max_seq_len"]), seed=6)
    sa.forward_cache_clear()


def test_llama32_bound_program_matches(dev, orc):
    """Llama32Program (descriptors built once) against the oracle, device arrays."""
    import torch
    cfg = CFG_SMALL
    arrays = make_arrays(cfg, seed=8, wide=True)
    ref = {k: v.copy() for k, v in arrays.items()}
    darr = {k: torch.from_numpy(v).to(dev) for k, v in arrays.items()}
    dims = [cfg[k] for k in DIMS]
    fwd = sa.Llama32Program(darr, *dims)
    for pos in range(6):
        r = fwd(pos)
        want = orc.llama32_int8_forward(ref, pos, *dims)
        logits = darr["logits"].cpu().numpy()
        assert r == logits[0]
        _close(logits, ref["logits"])
        assert abs(want - r) <= TOL * max(np.abs(ref["logits"]).max(), 1e-30)
        kv = cfg["n_kv_heads"] * cfg["head_dim"]
        got = darr["k_cache"].cpu().numpy().reshape(cfg["n_layers"], cfg["max_seq_len"], kv)[:, pos]
        exp = ref["k_cache"].reshape(cfg["n_layers"], cfg["max_seq_len"], kv)[:, pos]
        assert np.array_equal(got, exp)
    sa.forward_cache_clear()


@pytest.mark.parametrize("wide", [True, False])
def test_llama32_1b_dims(dev, orc, wide):
    """The kernel instances the bench times at the LLaMA-3.2-1B shape
    (bench_llama32_1b_int8.cpp:17-25: dim 2048, hidden 8192, 32 heads of 64,
    8 KV heads, vocab 128256, 4096 cache rows) with 2 layers. The caller owns
    the int8 caches, so rows below pos are filled with random int8 on both
    sides and single positions up to the last row are checked."""
    import torch
    cfg = dict(dim=2048, hidden_dim=8192, n_layers=2, n_heads=32, n_kv_heads=8,
               vocab_size=128256, max_seq_len=4096, head_dim=64)
    arrays = make_arrays(cfg, seed=21 + wide, wide=wide)
    rng = np.random.default_rng(22)
    arrays["k_cache"][:] = rng.integers(-128, 128, arrays["k_cache"].size, dtype=np.int8)
    arrays["v_cache"][:] = rng.integers(-128, 128, arrays["v_cache"].size, dtype=np.int8)
    ref = {k: v.copy() for k, v in arrays.items()}
    darr = {k: torch.from_numpy(v).to(dev) for k, v in arrays.items()}
    _run(orc, cfg, darr, ref, (0, 1, 127, 511, 2047, 4095), seed=23)
    sa.forward_cache_clear()
    del darr
    torch.cuda.empty_cache()


def test_llama32_rejects(dev):
    cfg = CFG_SMALL
    arrays = make_arrays(cfg, seed=1)
    dims = [cfg[k] for k in DIMS]
    with pytest.raises(sa.SimpRTError, match="dimensions"):
        sa.llama32_forward(arrays, 0, *dims[:-1], 16)          # n_heads * head_dim != dim
    with pytest.raises(sa.SimpRTError, match="pos"):
        sa.llama32_forward(arrays, cfg["max_seq_len"], *dims)
    short = dict(arrays, w2_t=arrays["w2_t"][:100])
    with pytest.raises(sa.SimpRTError, match="w2_t"):
        sa.llama32_forward(short, 0, *dims)
    sa.forward_cache_clear()
