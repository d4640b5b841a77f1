"""Pins of the decode-step oracles against what the mathematics fixes.

orc_llama_forward restates one token of stories110M.sl:44-247 (RoPE :86-112,
KV store :115-121, attention :124-164, SwiGLU FFN :185-228) with the GQA head
map of llama2_quant.sl:98 and the 1/sqrt(head_size) score scale;
orc_llama_quant_forward restates llama2_quant.sl:57-198 (reference W4 format,
no RoPE).  Neither has golden outputs in the reference
(docs/benchmark/llama_results.md:81-95), so they are pinned here by:

* a float64 brute force over tiny models in a different formulation: the
  whole token sequence at once with a causal mask (no KV cache), heads as
  reshapes and whole-matrix products, RoPE as multiplication of (x0 + i x1) by
  exp(i * pos * theta^(-2j/hs)), the GQA map as h // (n_heads / n_kv_heads);
* special cases that reduce the step to closed forms: zero projections
  (logits = wcls . rmsnorm(emb[token])); one score at pos 0 (the logits cannot
  depend on wq, wk or theta); wq = 0 (every head's output is the mean of its V
  rows over 0..pos);
* invariances: GQA equals MHA with its K/V heads duplicated; the symmetric W4
  path equals the fp32 path on the dequantized matrices;
* mutation checks: the brute force with RoPE off, with the wrong GQA map or
  with the attention scale dropped must NOT match, so each pin has teeth.

CPU only (no GPU)."""
import numpy as np
import pytest

CFG = dict(dim=64, hidden_dim=96, n_layers=2, n_heads=4, n_kv_heads=2, vocab_size=50,
           seq_len=12, eps=1e-5, rope_theta=10000.0, weight_format=0, group_size=32)
TOKENS = [3, 17, 42, 8, 8, 29, 0]
REL = 5e-6     # brute force vs oracle (fp32 activations vs float64): observed <= 4e-7


def _weights(cfg, seed, scale=1.0):
    """fp32 weights scaled so that scores have a spread of a few units (peaky
    attention: RoPE and the head map change the logits visibly)."""
    rng = np.random.default_rng(seed)
    d, h, L, V = cfg["dim"], cfg["hidden_dim"], cfg["n_layers"], cfg["vocab_size"]
    kv = d * cfg["n_kv_heads"] // cfg["n_heads"]
    n = lambda *s, fan: (rng.standard_normal(s) * scale * np.sqrt(2.0 / fan)).astype(np.float32)
    return {"token_embedding": rng.standard_normal((V, d)).astype(np.float32),
            "rms_att": (1 + 0.1 * rng.standard_normal((L, d))).astype(np.float32),
            "rms_ffn": (1 + 0.1 * rng.standard_normal((L, d))).astype(np.float32),
            "rms_final": (1 + 0.1 * rng.standard_normal(d)).astype(np.float32),
            "wq": n(L, d, d, fan=d), "wk": n(L, kv, d, fan=d), "wv": n(L, kv, d, fan=d),
            "wo": n(L, d, d, fan=d), "w1": n(L, h, d, fan=d), "w2": n(L, d, h, fan=h),
            "w3": n(L, h, d, fan=d), "wcls": n(V, d, fan=d)}


def _oracle_logits(orc, cfg, w, tokens):
    o = orc.LlamaOracle(cfg, {k: np.ascontiguousarray(v) for k, v in w.items()})
    return np.stack([o.forward(t, p).astype(np.float64) for p, t in enumerate(tokens)])


def _brute_logits(cfg, w, tokens, rope=True, gqa="div", scale_scores=True, mats=None):
    """Logits at every position of `tokens` (fed from pos 0), float64."""
    f = lambda a: np.asarray(a, np.float64)
    d, L, nh, nkv = cfg["dim"], cfg["n_layers"], cfg["n_heads"], cfg["n_kv_heads"]
    hs, eps, theta = d // nh, cfg["eps"], cfg["rope_theta"]
    mats = mats or w
    T = len(tokens)

    def rms(x, g):
        return x / np.sqrt((x * x).mean(-1, keepdims=True) + eps) * f(g)

    def rot(v, heads):       # v [T, heads*hs]
        z = v.reshape(T, heads, hs // 2, 2)
        c = z[..., 0] + 1j * z[..., 1]
        freq = theta ** (-2.0 * np.arange(hs // 2) / hs)
        c = c * np.exp(1j * np.arange(T)[:, None, None] * freq[None, None, :])
        return np.stack([c.real, c.imag], -1).reshape(T, heads * hs)

    x = f(w["token_embedding"])[tokens]
    causal = np.tril(np.ones((T, T), bool))
    for l in range(L):
        xn = rms(x, w["rms_att"][l])
        q, k, v = xn @ f(mats["wq"][l]).T, xn @ f(mats["wk"][l]).T, xn @ f(mats["wv"][l]).T
        if rope:
            q, k = rot(q, nh), rot(k, nkv)
        q, k, v = q.reshape(T, nh, hs), k.reshape(T, nkv, hs), v.reshape(T, nkv, hs)
        out = np.empty((T, nh, hs))
        for h in range(nh):
            kvh = h // (nh // nkv) if gqa == "div" else h % nkv
            s = q[:, h] @ k[:, kvh].T / (np.sqrt(hs) if scale_scores else 1.0)
            s = np.where(causal, s, -np.inf)
            p = np.exp(s - s.max(-1, keepdims=True))
            p /= p.sum(-1, keepdims=True)
            out[:, h] = p @ v[:, kvh]
        x = x + out.reshape(T, d) @ f(mats["wo"][l]).T
        xn = rms(x, w["rms_ffn"][l])
        h1, h3 = xn @ f(mats["w1"][l]).T, xn @ f(mats["w3"][l]).T
        x = x + (h1 / (1 + np.exp(-h1)) * h3) @ f(mats["w2"][l]).T
    return rms(x, w["rms_final"]) @ f(mats["wcls"]).T


def _rel(a, b):
    return np.abs(a - b).max() / np.abs(b).max()


# ------------------------------------------------------- orc_llama_forward --

@pytest.mark.parametrize("n_kv", [4, 2, 1])
def test_forward_matches_brute_force(orc, n_kv):
    cfg = dict(CFG, n_kv_heads=n_kv)
    w = _weights(cfg, 1 + n_kv)
    got = _oracle_logits(orc, cfg, w, TOKENS)
    want = _brute_logits(cfg, w, TOKENS)
    assert _rel(got, want) <= REL, _rel(got, want)


def test_forward_brute_force_has_teeth(orc):
    """Each plausible mistake, planted in the brute force, misses the oracle by
    far more than the tolerance (so the pin above rejects it)."""
    w = _weights(CFG, 7)
    got = _oracle_logits(orc, CFG, w, TOKENS)
    for bad in (dict(rope=False), dict(gqa="mod"), dict(scale_scores=False)):
        assert _rel(got, _brute_logits(CFG, w, TOKENS, **bad)) > 100 * REL, bad
    # RoPE rotating the other way: with S = diag(1, -1) on each pair,
    # S R(a) S = R(-a), so flipping the sign of the odd rows of wq and wk turns
    # the brute force's scores q.R(t-p)k into q.R(p-t)k
    wr = dict(w)
    sign = np.tile([1.0, -1.0], CFG["dim"] // 2).astype(np.float32)
    for m in ("wq", "wk"):
        wr[m] = w[m] * sign[:w[m].shape[1], None]
    assert _rel(got, _brute_logits(CFG, wr, TOKENS)) > 100 * REL


def test_forward_zero_projections_closed_form(orc):
    """All layer matrices zero: attention and FFN contribute nothing, so at every
    position logits = wcls . rmsnorm(emb[token]) * rms_final."""
    w = _weights(CFG, 3)
    for k in ("wq", "wk", "wv", "wo", "w1", "w2", "w3"):
        w[k] = np.zeros_like(w[k])
    got = _oracle_logits(orc, CFG, w, TOKENS)
    e = w["token_embedding"].astype(np.float64)[TOKENS]
    xn = e / np.sqrt((e * e).mean(-1, keepdims=True) + CFG["eps"]) * w["rms_final"]
    want = xn @ w["wcls"].astype(np.float64).T
    assert _rel(got, want) <= 1e-6


def test_forward_residual_only_through_wo_and_w2(orc):
    """wo = w2 = 0 with every other matrix random: the same closed form."""
    w = _weights(CFG, 4)
    w["wo"] = np.zeros_like(w["wo"])
    w["w2"] = np.zeros_like(w["w2"])
    got = _oracle_logits(orc, CFG, w, TOKENS)
    e = w["token_embedding"].astype(np.float64)[TOKENS]
    want = (e / np.sqrt((e * e).mean(-1, keepdims=True) + CFG["eps"]) * w["rms_final"]) \
        @ w["wcls"].astype(np.float64).T
    assert _rel(got, want) <= 1e-6


def test_forward_pos0_independent_of_queries_keys_and_theta(orc):
    """At pos 0 the softmax has one score, exactly 1, so each head outputs its
    own V row: the logits cannot depend on wq, wk or the RoPE base."""
    w = _weights(CFG, 5)
    w2 = dict(w, wq=_weights(CFG, 50)["wq"] * 3, wk=_weights(CFG, 51)["wk"] * 3)
    a = _oracle_logits(orc, CFG, w, TOKENS[:1])
    b = _oracle_logits(orc, dict(CFG, rope_theta=500.0), w2, TOKENS[:1])
    assert np.array_equal(a, b)
    # and at pos 1 they do (the pin is not vacuous)
    a = _oracle_logits(orc, CFG, w, TOKENS[:2])
    b = _oracle_logits(orc, CFG, w2, TOKENS[:2])
    assert not np.allclose(a[1], b[1])


@pytest.mark.parametrize("n_kv", [4, 2])
def test_forward_zero_queries_average_values(orc, n_kv):
    """wq = 0: every score is 0 and the softmax uniform, so head h outputs the
    mean over t <= pos of V_t of its KV head (V_t = wv . rmsnorm(emb[tok_t])).
    One layer, wo = I, FFN off: logits = wcls . rmsnorm(emb[tok_pos] + that)."""
    cfg = dict(CFG, n_layers=1, n_kv_heads=n_kv)
    d, nh, hs = cfg["dim"], cfg["n_heads"], cfg["dim"] // cfg["n_heads"]
    w = _weights(cfg, 6)
    w["wq"] = np.zeros_like(w["wq"])
    w["wo"] = np.eye(d, dtype=np.float32)[None]
    w["w2"] = np.zeros_like(w["w2"])
    got = _oracle_logits(orc, cfg, w, TOKENS)
    e = w["token_embedding"].astype(np.float64)[TOKENS]
    g = w["rms_att"][0].astype(np.float64)
    v = (e / np.sqrt((e * e).mean(-1, keepdims=True) + cfg["eps"]) * g) @ w["wv"][0].astype(np.float64).T
    v = v.reshape(len(TOKENS), n_kv, hs)
    mean = np.cumsum(v, 0) / np.arange(1, len(TOKENS) + 1)[:, None, None]
    heads = mean[:, [h * n_kv // nh for h in range(nh)]].reshape(len(TOKENS), d)
    x = e + heads
    want = (x / np.sqrt((x * x).mean(-1, keepdims=True) + cfg["eps"]) * w["rms_final"]) \
        @ w["wcls"].astype(np.float64).T
    assert _rel(got, want) <= 1e-5


def test_forward_gqa_equals_duplicated_mha(orc):
    """A GQA model (4 query heads over 2 KV heads) equals the MHA model whose
    wk / wv repeat each KV head's rows for the query heads that share it."""
    cfg = dict(CFG, n_kv_heads=2)
    hs = CFG["dim"] // CFG["n_heads"]
    w = _weights(cfg, 8)
    m = dict(w)
    for k in ("wk", "wv"):
        blocks = w[k].reshape(CFG["n_layers"], 2, hs, CFG["dim"])
        m[k] = np.repeat(blocks, 2, axis=1).reshape(CFG["n_layers"], CFG["dim"], CFG["dim"])
    a = _oracle_logits(orc, cfg, w, TOKENS)
    b = _oracle_logits(orc, dict(CFG, n_kv_heads=4), m, TOKENS)
    assert _rel(a, b) <= 1e-6


def _pack_w4s(q):
    """Signed nibbles q[..., K] in [-8, 7] -> bytes [..., K/2], low nibble = even k."""
    u = (q & 15).astype(np.uint8)
    return (u[..., 0::2] | (u[..., 1::2] << 4)).astype(np.uint8)


def test_forward_w4_equals_fp32_on_dequantized_weights(orc):
    """The symmetric W4 path (per-layer slices of packed bytes and scales)
    equals the fp32 path on the dequantized matrices q * scale."""
    cfg = dict(CFG, weight_format=1, group_size=32)
    rng = np.random.default_rng(9)
    w = _weights(CFG, 9)
    wq = {k: w[k] for k in ("token_embedding", "rms_att", "rms_ffn", "rms_final")}
    wf = dict(wq)
    for k in ("wq", "wk", "wv", "wo", "w1", "w2", "w3", "wcls"):
        shp = w[k].shape
        rows, K = int(np.prod(shp[:-1])), shp[-1]
        q = rng.integers(-8, 8, (rows, K))
        s = (np.abs(rng.standard_normal((rows, K // 32))) * np.sqrt(2.0 / K) / 4).astype(np.float32)
        wq["q_" + k] = _pack_w4s(q)
        wq["s_" + k] = s
        wf[k] = (q.astype(np.float32) * np.repeat(s, 32, axis=1)).reshape(shp)
    a = _oracle_logits(orc, cfg, wq, TOKENS)
    b = _oracle_logits(orc, CFG, wf, TOKENS)
    assert _rel(a, b) <= 1e-6
    assert _rel(a, _brute_logits(CFG, wf, TOKENS)) <= REL


@pytest.mark.parametrize("fmt", [0, 1])
def test_cpu_baseline_forward_equals_oracle(orc, fmt):
    """The decode CPU baseline (cpu_decode.c, fp32 accumulation) equals the
    oracle (double accumulation) to 1e-5 of max|logit| at every position, fp32
    (rows of 72 and 84: a remainder past the 16 lanes) and W4, with GQA."""
    cfg = dict(CFG, dim=96 if fmt else 72, hidden_dim=160 if fmt else 84, n_heads=4,
               n_kv_heads=2, weight_format=fmt, group_size=32, seq_len=12)
    rng = np.random.default_rng(40 + fmt)
    w = _weights(cfg, 40 + fmt)
    if fmt:
        for k in ("wq", "wk", "wv", "wo", "w1", "w2", "w3", "wcls"):
            shp = w.pop(k).shape
            rows, K = int(np.prod(shp[:-1])), shp[-1]
            w["q_" + k] = _pack_w4s(rng.integers(-8, 8, (rows, K)))
            w["s_" + k] = (np.abs(rng.standard_normal((rows, K // 32))) * np.sqrt(2.0 / K) / 4
                           ).astype(np.float32)
    a = _oracle_logits(orc, cfg, w, TOKENS)
    cpu = orc.CpuLlama(cfg, {k: np.ascontiguousarray(v) for k, v in w.items()})
    b = np.stack([cpu.forward(t, p).astype(np.float64) for p, t in enumerate(TOKENS)])
    assert _rel(a, b) <= 1e-5


# ------------------------------------------------- orc_llama_quant_forward --

QCFG = dict(dim=128, hidden_dim=256, n_layers=2, n_heads=4, n_kv_heads=4, vocab_size=50,
            seq_len=12, eps=1e-5, rope_theta=10000.0)   # dims multiples of gs = 128


def _quant_arrays(orc, seed, gs=32):
    """The program's arrays built as bench_llama_quant.cpp:157-209 builds them:
    fp32 matrices quantized one after another (reference quantizer) into one
    flat nibble array; returns the arrays, the offsets and the dequantized
    matrices (q * scale + zero per flat group)."""
    w = _weights(QCFG, seed)
    order = ("wq", "wk", "wv", "wo", "w1", "w2", "w3")
    qs, ss, zs, offs, at = [], [], [], [], 0
    for k in order:
        q, s, z = orc.quantize_f5(w[k], gs)
        qs.append(q); ss.append(s); zs.append(z); offs.append(at)
        at += w[k].size
    qw, sc, ze = np.concatenate(qs), np.concatenate(ss), np.concatenate(zs)
    nib = np.empty(2 * qw.size, np.float64)
    nib[0::2], nib[1::2] = qw & 15, qw >> 4
    flat = nib[:at] * np.repeat(sc.astype(np.float64), gs)[:at] + np.repeat(ze, gs)[:at]
    deq = {k: flat[o:o + w[k].size].reshape(w[k].shape) for k, o in zip(order, offs)}
    deq["wcls"] = w["wcls"]
    arrays = {"token_emb": w["token_embedding"].ravel(), "rms_att_w": w["rms_att"].ravel(),
              "rms_ffn_w": w["rms_ffn"].ravel(), "rms_final_w": w["rms_final"],
              "wcls": w["wcls"].ravel(), "qweights": qw, "scales": sc, "zeros": ze}
    return w, arrays, offs, deq


@pytest.mark.parametrize("gs", [32, 128])
def test_quant_forward_matches_brute_force(orc, gs):
    """llama2_quant.sl has no RoPE: the brute force without it, on the matrices
    dequantized from the flat array at the program's per-layer offsets."""
    w, arrays, offs, deq = _quant_arrays(orc, 11, gs)
    o = orc.LlamaQuantOracle(QCFG, arrays, gs, offs)
    got = np.stack([o.forward(t, p).astype(np.float64) for p, t in enumerate(TOKENS)])
    want = _brute_logits(QCFG, w, TOKENS, rope=False, mats=deq)
    assert _rel(got, want) <= REL
    assert _rel(got, _brute_logits(QCFG, w, TOKENS, rope=True, mats=deq)) > 100 * REL


def test_quant_forward_pos0_equals_fp32_forward(orc):
    """At pos 0 RoPE is the identity, so the W4 program equals orc_llama_forward
    on the dequantized matrices there (two restatements, one answer)."""
    w, arrays, offs, deq = _quant_arrays(orc, 12, 32)
    o = orc.LlamaQuantOracle(QCFG, arrays, 32, offs)
    a = o.forward(TOKENS[0], 0).astype(np.float64)
    wf = dict(w, **{k: v.astype(np.float32) for k, v in deq.items()})
    b = _oracle_logits(orc, dict(QCFG, weight_format=0, group_size=32), wf, TOKENS[:1])[0]
    assert _rel(a, b) <= 1e-5


# ------------------------------------- matmul_quant: reference indexing --

def test_matmul_quant_reference_indexing(orc):
    """MatMulQuantOpLowering as emitted (ConvertSimpToMemRef.cpp:3906-4011)
    against the restatement used by the library (group index with the offset,
    gs/16 tiles):
    * offset 0, gs = 128 (the only case the reference is written for): equal
      bit for bit;
    * offset > 0: the reference reads the scales of group (i*cols)/gs + g, i.e.
      the first matrix's -- equal to the fixed form on scales shifted by
      offset/gs groups;
    * gs = 32: the reference's 8 tiles of 16 overlap the next groups, so every
      weight k counts once for each group g with g*gs <= k < g*gs + 128."""
    rng = np.random.default_rng(13)
    rows, cols = 6, 512
    total = 3 * rows * cols
    qw = rng.integers(0, 256, total // 2, dtype=np.uint8)
    x = rng.standard_normal(cols).astype(np.float32)
    gs = 128
    sc = (rng.random(total // gs) + 0.5).astype(np.float32)
    ze = rng.standard_normal(total // gs).astype(np.float32)
    a = orc.matmul_quant_f5(qw, sc, ze, x, rows, cols, gs, 0)
    b = orc.matmul_quant_f5_refidx(qw, sc, ze, x, rows, cols, gs, 0)
    assert np.array_equal(a, b)
    off = rows * cols                                   # the second matrix
    b = orc.matmul_quant_f5_refidx(qw, sc, ze, x, rows, cols, gs, off)
    a = orc.matmul_quant_f5(qw, sc, ze, x, rows, cols, gs, off)
    assert not np.allclose(a, b)
    shift = off // gs                                   # fixed group g + shift reads ref's g
    sc2, ze2 = np.roll(sc, shift), np.roll(ze, shift)
    assert np.array_equal(orc.matmul_quant_f5(qw, sc2, ze2, x, rows, cols, gs, off), b)
    # gs = 32: overlapping tiles, closed form in float64
    gs = 32
    sc = (rng.random(total // gs) + 0.5).astype(np.float32)
    ze = rng.standard_normal(total // gs).astype(np.float32)
    b = orc.matmul_quant_f5_refidx(qw, sc, ze, x, rows, cols, gs, 0)
    nib = np.empty(2 * qw.size, np.float64)
    nib[0::2], nib[1::2] = qw & 15, qw >> 4
    want = np.zeros(rows)
    for i in range(rows):
        for g in range(cols // gs):
            gi = i * cols // gs + g
            k = np.arange(g * gs, min(g * gs + 128, cols))
            want[i] += ((nib[i * cols + k] * sc[gi] + ze[gi]) * x[k]).sum()
    assert np.abs(b - want).max() <= 1e-5 * np.abs(want).max()
    assert not np.allclose(b, orc.matmul_quant_f5(qw, sc, ze, x, rows, cols, gs, 0))
