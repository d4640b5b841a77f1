"""The model-level drop-in export stories110M_forward (signature of
examples/llama2/stories110M.sl:5-44 as bound by generate_stories110M.cpp:15-21):
called the way the reference host calls it -- 25 host arrays as rank-1
descriptors plus nine i64 -- and checked against the oracle's restatement of
the program: logits within 1e-4 of max|logit|, the returned logits[0], and the
K/V rows the call writes back into the caller's caches."""
import numpy as np
import pytest

import simplang_amd as sa
from simplang_amd.host import STORIES_ARRAYS

pytestmark = pytest.mark.gpu
TOL = 1e-4
CFG = dict(dim=128, hidden_dim=256, n_layers=2, n_heads=4, n_kv_heads=2, vocab_size=512,
           seq_len=16)


def _host_model(seed):
    rng = np.random.default_rng(seed)
    d, h, L, V, S = (CFG[k] for k in ("dim", "hidden_dim", "n_layers", "vocab_size", "seq_len"))
    kv = d * CFG["n_kv_heads"] // CFG["n_heads"]
    r = lambda *s: (rng.standard_normal(s) * 0.02).astype(np.float32)
    w = {"token_embedding": r(V, d), "rms_att": r(L, d) + 1, "rms_ffn": r(L, d) + 1,
         "rms_final": r(d) + 1, "wq": r(L, d, d), "wk": r(L, kv, d), "wv": r(L, kv, d),
         "wo": r(L, d, d), "w1": r(L, h, d), "w2": r(L, d, h), "w3": r(L, h, d), "wcls": r(V, d)}
    arrays = {"token_embedding_table": w["token_embedding"], "rms_att_w": w["rms_att"],
              "rms_ffn_w": w["rms_ffn"], "rms_final_w": w["rms_final"]}
    for k in ("wq", "wk", "wv", "wo", "w1", "w2", "w3", "wcls"):
        arrays[k] = w[k]
    arrays = {k: np.ascontiguousarray(v).reshape(-1) for k, v in arrays.items()}
    for k, n in (("x", d), ("xb", d), ("xb2", d), ("hb", h), ("hb_silu", h), ("q", d), ("k", kv),
                 ("v", kv), ("att", CFG["n_heads"] * S), ("att_soft", CFG["n_heads"] * S),
                 ("logits", V), ("key_cache", L * S * kv), ("value_cache", L * S * kv)):
        arrays[k] = np.zeros(n, np.float32)
    return w, arrays


def _cfg_args():
    return (CFG["dim"], CFG["hidden_dim"], CFG["n_layers"], CFG["n_heads"], CFG["n_kv_heads"],
            CFG["vocab_size"], CFG["seq_len"])


def test_stories110M_forward_host_arrays(dev, orc):
    w, arrays = _host_model(11)
    o = orc.LlamaOracle(dict(CFG, eps=1e-5, rope_theta=10000.0, weight_format=0), w)
    tokens = [5, 300, 17, 511, 42, 0]
    for pos, t in enumerate(tokens):
        print(f"[forward-export] pos={pos}", flush=True)
        r = sa.stories110M_forward(arrays, t, pos, *_cfg_args())
        want = o.forward(t, pos).astype(np.float64)
        got = arrays["logits"].astype(np.float64)
        assert np.abs(got - want).max() <= TOL * np.abs(want).max(), pos
        assert r == arrays["logits"][0]
    # the caches hold the rows of every position computed so far
    n = len(tokens) * CFG["dim"] * CFG["n_kv_heads"] // CFG["n_heads"]
    kv = CFG["dim"] * CFG["n_kv_heads"] // CFG["n_heads"]
    for name, ref in (("key_cache", o.kc), ("value_cache", o.vc)):
        got = arrays[name].reshape(CFG["n_layers"], CFG["seq_len"], kv)
        want = ref.reshape(CFG["n_layers"], CFG["seq_len"], kv)
        used = slice(0, len(tokens))
        assert np.abs(got[:, used] - want[:, used]).max() <= TOL * np.abs(want[:, used]).max()
        assert (got[:, len(tokens):] == 0).all()
    assert n > 0
    # untouched scratch arrays (the engine keeps its own)
    assert (arrays["x"] == 0).all() and (arrays["att"] == 0).all()
    sa.forward_cache_clear()


def test_stories110M_forward_device_arrays_and_errors(dev, orc):
    import torch
    w, arrays = _host_model(12)
    host_logits = []
    for pos, t in enumerate([1, 2, 3]):
        sa.stories110M_forward(arrays, t, pos, *_cfg_args())
        host_logits.append(arrays["logits"].copy())
    darr = {k: torch.from_numpy(v.copy()).to(dev) for k, v in arrays.items()}
    for k in ("logits", "key_cache", "value_cache"):
        darr[k].zero_()
    for pos, t in enumerate([1, 2, 3]):
        r = sa.stories110M_forward(darr, t, pos, *_cfg_args())
        got = darr["logits"].cpu().numpy()
        assert np.abs(got - host_logits[pos]).max() <= 1e-6 * np.abs(host_logits[pos]).max() + 1e-7
        assert r == got[0]
    with pytest.raises(sa.SimpRTError):
        sa.stories110M_forward(arrays, 0, CFG["seq_len"], *_cfg_args())   # pos out of range
    bad = dict(arrays, wq=arrays["wq"][:10])
    with pytest.raises(sa.SimpRTError):
        sa.stories110M_forward(bad, 0, 0, *_cfg_args())                   # array too short
    sa.forward_cache_clear()


QCFG = dict(dim=128, hidden_dim=256, n_layers=2, n_heads=4, n_kv_heads=4, vocab_size=512,
            seq_len=16)


def _quant_model(orc, seed, gs=128, cfg=None):
    """Arrays of llama2_quant_forward built the way bench_llama_quant.cpp:157-209
    builds them: random fp32 matrices quantized with the reference quantizer
    into one flat qweights array, offsets in elements."""
    cfg = cfg or QCFG
    rng = np.random.default_rng(seed)
    d, h, L, V, S = (cfg[k] for k in ("dim", "hidden_dim", "n_layers", "vocab_size", "seq_len"))
    kv = d * cfg["n_kv_heads"] // cfg["n_heads"]
    r = lambda *s: (rng.standard_normal(s) * 0.05).astype(np.float32)
    mats = [r(L, d, d), r(L, kv, d), r(L, kv, d), r(L, d, d), r(L, h, d), r(L, d, h), r(L, h, d)]
    qs, ss, zs, offs, at = [], [], [], [], 0
    for m in mats:
        q, sc, ze = orc.quantize_f5(m, gs)
        qs.append(q); ss.append(sc); zs.append(ze); offs.append(at)
        at += m.size
    arrays = {"token_emb": r(V, d).ravel(), "rms_att_w": (r(L, d) + 1).ravel(),
              "rms_ffn_w": (r(L, d) + 1).ravel(), "rms_final_w": r(d) + 1, "wcls": r(V, d).ravel(),
              "qweights": np.concatenate(qs).view(np.int8), "scales": np.concatenate(ss),
              "zeros": np.concatenate(zs)}
    for k, n in (("x", d), ("xb", d), ("xb2", d), ("q", d), ("k", kv), ("v", kv),
                 ("att", cfg["n_heads"] * S), ("att_soft", cfg["n_heads"] * S), ("hb", h),
                 ("hb_silu", h), ("hb2", h), ("logits", V), ("key_cache", L * S * kv),
                 ("value_cache", L * S * kv)):
        arrays[k] = np.zeros(n, np.float32)
    return arrays, offs


@pytest.mark.parametrize("gs", [128, 32, 16])
def test_llama2_quant_forward_host_arrays(dev, orc, gs):
    """gs 128 and 32: the fused step (dot8 GEMVs on the unsigned format, graph
    replay); gs 16: the kernel sequence (groups shorter than a 32-weight chunk)."""
    arrays, offs = _quant_model(orc, 21, gs)
    o = orc.LlamaQuantOracle(QCFG, {k: arrays[k] for k in ("token_emb", "rms_att_w", "rms_ffn_w",
                                                           "rms_final_w", "wcls", "scales",
                                                           "zeros")} |
                             {"qweights": arrays["qweights"].view(np.uint8)}, gs, offs)
    dims = tuple(QCFG[k] for k in ("dim", "hidden_dim", "n_layers", "n_heads", "n_kv_heads",
                                   "vocab_size", "seq_len"))
    for pos, t in enumerate([50, 60, 70, 80, 90]):     # bench_llama_quant.cpp:258 tokens
        print(f"[quant-export] gs={gs} pos={pos}", flush=True)
        r = sa.llama2_quant_forward(arrays, t, pos, *dims, gs, offs)
        want = o.forward(t, pos).astype(np.float64)
        got = arrays["logits"].astype(np.float64)
        assert np.abs(got - want).max() <= TOL * np.abs(want).max(), pos
        assert r == arrays["logits"][0] and np.isfinite(r)
    kv = QCFG["dim"] * QCFG["n_kv_heads"] // QCFG["n_heads"]
    for name, ref in (("key_cache", o.kc), ("value_cache", o.vc)):
        got = arrays[name].reshape(QCFG["n_layers"], QCFG["seq_len"], kv)[:, :5]
        want = ref.reshape(QCFG["n_layers"], QCFG["seq_len"], kv)[:, :5]
        assert np.abs(got - want).max() <= TOL * np.abs(want).max()
    bad = dict(arrays, scales=arrays["scales"][:5])
    with pytest.raises(sa.SimpRTError):
        sa.llama2_quant_forward(bad, 0, 0, *dims, gs, offs)
    sa.forward_cache_clear()


@pytest.mark.parametrize("heads", [4, 32])
def test_llama2_quant_forward_long_context(dev, orc, heads):
    """Positions 0..259 through every attention mode of the step: one 64-position
    chunk (pos < 64), then the one-block kernel (4 heads) or the split over
    chunks with the combine kernel (32 heads)."""
    gs = 128
    cfg = dict(QCFG, seq_len=260) if heads == 4 else dict(QCFG, dim=256, n_heads=32,
                                                           n_kv_heads=8, seq_len=260)
    arrays, offs = _quant_model(orc, 23, gs, cfg)
    o = orc.LlamaQuantOracle(cfg, {k: arrays[k] for k in ("token_emb", "rms_att_w", "rms_ffn_w",
                                                          "rms_final_w", "wcls", "scales",
                                                          "zeros")} |
                             {"qweights": arrays["qweights"].view(np.uint8)}, gs, offs)
    dims = tuple(cfg[k] for k in ("dim", "hidden_dim", "n_layers", "n_heads", "n_kv_heads",
                                  "vocab_size", "seq_len"))
    toks = np.random.default_rng(5).integers(0, cfg["vocab_size"], cfg["seq_len"])
    print("[quant-export] long context", flush=True)
    for pos, t in enumerate(toks):
        sa.llama2_quant_forward(arrays, int(t), pos, *dims, gs, offs)
        want = o.forward(int(t), pos).astype(np.float64)
        if pos % 17 == 0 or pos >= 188:
            got = arrays["logits"].astype(np.float64)
            assert np.abs(got - want).max() <= TOL * np.abs(want).max(), pos
    sa.forward_cache_clear()


# ---------------------------------------------------------- caller state --
# The compiled programs read every weight and the caches' rows [0, pos] from the
# caller's arrays on every call.  The exports keep device copies, so they must
# follow changes the caller makes between calls.

def _stories_oracle(orc, w, arrays=None, upto=0):
    o = orc.LlamaOracle(dict(CFG, eps=1e-5, rope_theta=10000.0, weight_format=0), w)
    if arrays is not None:      # start from the caller's cache rows [0, upto)
        kv = CFG["dim"] * CFG["n_kv_heads"] // CFG["n_heads"]
        for name, dst in (("key_cache", o.kc), ("value_cache", o.vc)):
            src = arrays[name].reshape(CFG["n_layers"], CFG["seq_len"], kv)
            dst.reshape(CFG["n_layers"], CFG["seq_len"], kv)[:, :upto] = src[:, :upto]
    return o


def _same(got, want):
    got, want = got.astype(np.float64), want.astype(np.float64)
    assert np.abs(got - want).max() <= TOL * np.abs(want).max()


def test_stories110M_forward_weights_rewritten_in_place(dev, orc):
    """Weights rewritten in place between calls (what a host that frees its
    model and loads another into the same addresses does): the very next call,
    mid-sequence, and a restart at pos 0 use the new values."""
    sa.forward_cache_clear()
    wa, arrays = _host_model(31)
    wb, arrays_b = _host_model(32)
    for pos, t in enumerate([4, 9, 16]):
        sa.stories110M_forward(arrays, t, pos, *_cfg_args())
    for k in ("token_embedding_table", "rms_att_w", "rms_ffn_w", "rms_final_w", "wq", "wk",
              "wv", "wo", "w1", "w2", "w3", "wcls"):
        np.copyto(arrays[k], arrays_b[k])            # same addresses, new contents
    o = _stories_oracle(orc, wb, arrays, upto=3)
    print("[forward-export] rewritten weights, pos=3", flush=True)
    sa.stories110M_forward(arrays, 25, 3, *_cfg_args())
    _same(arrays["logits"], o.forward(25, 3))
    o = _stories_oracle(orc, wb)
    for pos, t in enumerate([7, 3]):
        sa.stories110M_forward(arrays, t, pos, *_cfg_args())
        _same(arrays["logits"], o.forward(t, pos))
    # one edited row of the classifier, then a new sequence (pos 0 re-checks
    # every chunk of every array)
    arrays["wcls"][:CFG["dim"]] *= 3.0
    o = _stories_oracle(orc, {**wb, "wcls": arrays["wcls"].reshape(wb["wcls"].shape)})
    for pos, t in enumerate([7, 3, 8]):
        sa.stories110M_forward(arrays, t, pos, *_cfg_args())
        _same(arrays["logits"], o.forward(t, pos))
    sa.forward_cache_clear()


def test_stories110M_forward_verify_all_sees_every_edit(dev, orc):
    """With simp_rt_export_verify_all(1) a mid-sequence edit of a few rows deep
    inside a host array (chunks the rotation has not reached) is used by the
    very next call, as the compiled program, which reads every weight on every
    call, would use it."""
    sa.forward_cache_clear()
    sa.export_verify_all(True)
    try:
        wa, arrays = _host_model(41)
        o = _stories_oracle(orc, wa)
        for pos, t in enumerate([4, 9]):
            sa.stories110M_forward(arrays, t, pos, *_cfg_args())
            _same(arrays["logits"], o.forward(t, pos))
        d = CFG["dim"]
        rows = slice(CFG["vocab_size"] - 3, CFG["vocab_size"])    # the last chunk of wcls
        arrays["wcls"][rows.start * d:rows.stop * d] *= -2.0
        layer = CFG["n_layers"] - 1                               # the last layer's w2
        w2 = arrays["w2"].reshape(CFG["n_layers"], d, CFG["hidden_dim"])
        w2[layer, d // 2] += 0.5
        wn = {**wa, "wcls": arrays["wcls"].reshape(wa["wcls"].shape),
              "w2": w2.reshape(wa["w2"].shape)}
        o2 = _stories_oracle(orc, wn, arrays, upto=2)
        print("[forward-export] verify_all, edited rows at pos=2", flush=True)
        sa.stories110M_forward(arrays, 16, 2, *_cfg_args())
        _same(arrays["logits"], o2.forward(16, 2))
    finally:
        sa.export_verify_all(False)
        sa.forward_cache_clear()


def test_stories110M_forward_jumps_and_host_filled_caches(dev, orc):
    """A first call at pos 6 on caches the host filled, a jump back to pos 2,
    and a jump forward: each reads the caller's cache rows [0, pos)."""
    sa.forward_cache_clear()
    w, arrays = _host_model(33)
    toks = [11, 22, 33, 44, 55, 66, 77, 88, 99, 101]
    full = _stories_oracle(orc, w)
    for pos in range(6):
        full.forward(toks[pos], pos)
    arrays["key_cache"][:] = full.kc
    arrays["value_cache"][:] = full.vc
    for pos in (6, 2, 7, 9):
        print(f"[forward-export] jump to pos={pos}", flush=True)
        o = _stories_oracle(orc, w, arrays, upto=pos)
        sa.stories110M_forward(arrays, toks[pos], pos, *_cfg_args())
        _same(arrays["logits"], o.forward(toks[pos], pos))
    sa.forward_cache_clear()


def test_stories110M_forward_nan_rows_past_pos_are_not_read(dev, orc):
    """Cache rows past pos never reach the result, whatever they hold: a call
    at pos 8 loads NaN rows [0, 8) into the engine's cache, and a jump back to
    pos 1 (row 0 reloaded) must not see the NaN rows 2..7 that stay behind.
    The split attention loads every row of its chunk before pos is known; a
    row past pos weighted by probability 0 instead of dropped gives 0*NaN."""
    sa.forward_cache_clear()
    w, arrays = _host_model(35)
    toks = [7, 70, 170]
    arrays["key_cache"][:] = np.nan
    arrays["value_cache"][:] = np.nan
    sa.stories110M_forward(arrays, toks[2], 8, *_cfg_args())   # NaN attention: NaN result
    ref = _stories_oracle(orc, w)
    ref.forward(toks[0], 0)
    arrays["key_cache"][:] = ref.kc
    arrays["value_cache"][:] = ref.vc
    kv =CFG["dim"] * CFG["n_kv_heads"] // CFG["n_heads"]
    for name in ("key_cache", "value_cache"):
        arrays[name].reshape(CFG["n_layers"], CFG["seq_len"], kv)[:, 1:] = np.nan
    print("[forward-export] NaN rows past pos 1", flush=True)
    r = sa.stories110M_forward(arrays, toks[1], 1, *_cfg_args())
    assert np.isfinite(arrays["logits"]).all() and r == r
    _same(arrays["logits"], ref.forward(toks[1], 1))
    sa.forward_cache_clear()


def test_stories110M_forward_nan_is_not_an_error(dev, orc):
    """A NaN the arithmetic produces comes back as NaN without an exception,
    even after an earlier failed call left a message behind."""
    sa.forward_cache_clear()
    w, arrays = _host_model(34)
    with pytest.raises(sa.SimpRTError):
        sa.stories110M_forward(arrays, 0, CFG["seq_len"], *_cfg_args())   # pos out of range
    arrays["token_embedding_table"][:CFG["dim"]] = np.nan                # token 0 embeds NaN
    r = sa.stories110M_forward(arrays, 0, 0, *_cfg_args())
    assert r != r and np.isnan(arrays["logits"]).all()
    assert sa.last_error() == ""
    sa.forward_cache_clear()


def test_llama2_quant_forward_caller_state(dev, orc):
    """llama2_quant_forward: rewritten weights and jumps with host-filled caches."""
    sa.forward_cache_clear()
    gs = 128
    arrays, offs = _quant_model(orc, 41, gs)
    arrays_b, _ = _quant_model(orc, 42, gs)
    dims = tuple(QCFG[k] for k in ("dim", "hidden_dim", "n_layers", "n_heads", "n_kv_heads",
                                   "vocab_size", "seq_len"))
    names = ("token_emb", "rms_att_w", "rms_ffn_w", "rms_final_w", "wcls", "scales", "zeros")
    kv = QCFG["dim"] * QCFG["n_kv_heads"] // QCFG["n_heads"]

    def oracle(arr, upto=0):
        o = orc.LlamaQuantOracle(QCFG, {k: arr[k] for k in names} |
                                 {"qweights": arr["qweights"].view(np.uint8)}, gs, offs)
        for name, dst in (("key_cache", o.kc), ("value_cache", o.vc)):
            src = arrays[name].reshape(QCFG["n_layers"], QCFG["seq_len"], kv)
            dst.reshape(QCFG["n_layers"], QCFG["seq_len"], kv)[:, :upto] = src[:, :upto]
        return o

    for pos, t in enumerate([50, 60, 70]):
        sa.llama2_quant_forward(arrays, t, pos, *dims, gs, offs)
    for k in names + ("qweights",):
        np.copyto(arrays[k], arrays_b[k])
    print("[quant-export] rewritten weights, pos=3", flush=True)
    o = oracle(arrays, upto=3)
    sa.llama2_quant_forward(arrays, 80, 3, *dims, gs, offs)
    _same(arrays["logits"], o.forward(80, 3))
    for pos in (1, 5):                                   # jumps: rows [0, pos) from the host
        print(f"[quant-export] jump to pos={pos}", flush=True)
        o = oracle(arrays, upto=pos)
        sa.llama2_quant_forward(arrays, 90 + pos, pos, *dims, gs, offs)
        _same(arrays["logits"], o.forward(90 + pos, pos))
    sa.forward_cache_clear()
