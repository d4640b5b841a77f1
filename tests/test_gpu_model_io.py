"""GPU side of the model files: the llama2.c checkpoint loaded into device
memory (generate_stories110M.cpp:150-191), the W4 quantizers against the
oracle's restatements bit for bit (reference quantize_w4,
bench_llama_quant.cpp:51-93, and the symmetric BASELINE format), and the packed
W4 files written from a checkpoint and read back, driven through the decode
engine and llama2_quant_forward against the oracle's forward passes."""
import numpy as np
import pytest

import simplang_amd as sa

from _llama2c import random_llama2c, write_checkpoint

pytestmark = pytest.mark.gpu
TOL = 1e-4

CFG = dict(dim=128, hidden_dim=256, n_layers=2, n_heads=4, n_kv_heads=2, vocab_size=96, seq_len=32)
NAMES = ("token_embedding", "rms_att", "wq", "wk", "wv", "wo", "rms_ffn", "w1", "w2", "w3",
         "rms_final", "wcls")


@pytest.mark.parametrize("shared", [True, False])
def test_ckpt_load_f32_arrays_and_logits(dev, orc, tmp_path, shared):
    w = random_llama2c(CFG, seed=3, shared=shared)
    p = tmp_path / "m.bin"
    write_checkpoint(p, CFG, w, shared)
    print(f"[model-io] ckpt shared={shared}", flush=True)
    m = sa.ckpt_load_f32(p)
    for k in NAMES:
        got = m.read(k, w[k].size)
        assert np.array_equal(got, w[k].ravel()), k
    if shared:
        assert m.weights["wcls"] == m.weights["token_embedding"]
    cfg = dict(m.cfg)
    eng = sa.Llama(cfg, m.weights)
    o = orc.LlamaOracle(dict(cfg), {k: w[k].ravel() for k in NAMES})
    lg = np.empty(CFG["vocab_size"], np.float32)
    for pos, t in enumerate([1, 17, 5, 90]):
        eng.forward(t, pos, lg)
        want = o.forward(t, pos).astype(np.float64)
        assert np.abs(lg - want).max() <= TOL * np.abs(want).max(), pos
    eng.close()
    m.close()


def test_ckpt_load_truncated(dev, tmp_path):
    w = random_llama2c(CFG, seed=4)
    p = tmp_path / "m.bin"
    write_checkpoint(p, CFG, w)
    data = p.read_bytes()
    p.write_bytes(data[:-100])
    with pytest.raises(sa.SimpRTError):
        sa.ckpt_load_f32(p)


@pytest.mark.parametrize("n,gs", [(128 * 50, 128), (128 * 50 + 77, 128), (32 * 9 + 1, 32), (6, 4)])
def test_quantize_w4u_matches_oracle(dev, orc, n, gs):
    import torch
    rng = np.random.default_rng(n)
    w = rng.uniform(-0.01, 0.01, n).astype(np.float32)       # bench_llama_quant.cpp:43-49 range
    w[: min(n, gs)] = 0.0                                        # a constant group: scale 1e-8
    tw = torch.from_numpy(w).to(dev)
    q = torch.zeros((n + 1) // 2, dtype=torch.uint8, device=dev)
    ng = (n + gs - 1) // gs
    s, z = (torch.empty(ng, device=dev) for _ in range(2))
    sa.quantize_w4u(tw, gs, q, s, z)
    torch.cuda.synchronize()
    wq, ws, wz = orc.quantize_f5(w, gs)
    assert np.array_equal(q.cpu().numpy(), wq)
    assert np.array_equal(s.cpu().numpy(), ws) and np.array_equal(z.cpu().numpy(), wz)


@pytest.mark.parametrize("rows,cols,gs", [(96, 256, 32), (7, 640, 64), (33, 128, 128)])
def test_quantize_w4s_matches_oracle(dev, orc, rows, cols, gs):
    import torch
    rng = np.random.default_rng(rows * cols)
    w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    w[0, :gs] = 0.0                                              # an all-zero group: scale 1
    tw = torch.from_numpy(w).to(dev)
    q = torch.empty((rows, cols // 2), dtype=torch.uint8, device=dev)
    s = torch.empty((rows, cols // gs), device=dev)
    sa.quantize_w4s(tw, gs, q, s)
    torch.cuda.synchronize()
    wq, ws = orc.quantize_w4s(w, gs)
    assert np.array_equal(q.cpu().numpy(), wq) and np.array_equal(s.cpu().numpy(), ws)


def test_w4s_file_roundtrip_and_engine(dev, orc, tmp_path):
    gs = 32
    w = random_llama2c(CFG, seed=5)
    ck, out = tmp_path / "m.bin", tmp_path / "m.w4s"
    write_checkpoint(ck, CFG, w)
    print("[model-io] w4s file", flush=True)
    sa.w4s_file_write(ck, out, gs)
    m = sa.w4s_file_load(out)
    assert m.cfg["weight_format"] == sa.W_W4S and m.cfg["group_size"] == gs
    L, d, h, V = CFG["n_layers"], CFG["dim"], CFG["hidden_dim"], CFG["vocab_size"]
    wn = {k: w[k].ravel() for k in ("token_embedding", "rms_att", "rms_ffn", "rms_final")}
    for k in wn:
        assert np.array_equal(m.read(k, wn[k].size), wn[k]), k
    for k in ("wq", "wk", "wv", "wo", "w1", "w2", "w3", "wcls"):
        mat = w[k].reshape(-1, w[k].shape[-1])
        wq, ws = orc.quantize_w4s(mat, gs)
        assert np.array_equal(m.read("q_" + k, wq.size, "uint8"), wq.ravel()), k
        assert np.array_equal(m.read("s_" + k, ws.size), ws.ravel()), k
        wn["q_" + k], wn["s_" + k] = wq.ravel(), ws.ravel()
    eng = sa.Llama(m.cfg, m.weights)
    o = orc.LlamaOracle(dict(m.cfg), wn)
    lg = np.empty(V, np.float32)
    for pos, t in enumerate([3, 9, 27, 81]):
        eng.forward(t, pos, lg)
        want = o.forward(t, pos).astype(np.float64)
        assert np.abs(lg - want).max() <= TOL * np.abs(want).max(), pos
    eng.close()
    m.close()


def test_w4u_file_roundtrip_and_quant_forward(dev, orc, tmp_path):
    gs = 64
    w = random_llama2c(CFG, seed=6, shared=False)
    ck, out = tmp_path / "m.bin", tmp_path / "m.w4u"
    write_checkpoint(ck, CFG, w, shared=False)
    print("[model-io] w4u file", flush=True)
    sa.w4u_file_write(ck, out, gs)
    m = sa.w4u_file_load(out)
    c = m.cfg
    qs, ss, zs, offs, at = [], [], [], [], 0
    for k in ("wq", "wk", "wv", "wo", "w1", "w2", "w3"):     # bench_llama_quant.cpp:189-210
        q, s, z = orc.quantize_f5(w[k], gs)
        qs.append(q); ss.append(s); zs.append(z); offs.append(at)
        at += w[k].size
    q, s, z = np.concatenate(qs), np.concatenate(ss), np.concatenate(zs)
    assert c["offsets"] == offs and c["qweights_bytes"] == q.size and c["n_groups"] == s.size
    assert np.array_equal(m.read("qweights", q.size, "uint8"), q)
    assert np.array_equal(m.read("scales", s.size), s) and np.array_equal(m.read("zeros", z.size), z)
    assert np.array_equal(m.read("wcls", w["wcls"].size), w["wcls"].ravel())
    # llama2_quant_forward on the loaded (device) arrays vs the oracle
    import torch
    L, d, h, V, S = (CFG[k] for k in ("n_layers", "dim", "hidden_dim", "vocab_size", "seq_len"))
    kv = d * CFG["n_kv_heads"] // CFG["n_heads"]

    def dev_view(name, n, dtype):
        t = torch.empty(n, dtype=dtype, device=dev)
        sa.lib.simp_rt_memcpy(t.data_ptr(), m.weights[name], t.numel() * t.element_size())
        return t
    arrays = {"token_emb": dev_view("token_embedding", V * d, torch.float32),
              "rms_att_w": dev_view("rms_att", L * d, torch.float32),
              "rms_ffn_w": dev_view("rms_ffn", L * d, torch.float32),
              "rms_final_w": dev_view("rms_final", d, torch.float32),
              "wcls": dev_view("wcls", V * d, torch.float32),
              "qweights": dev_view("qweights", q.size, torch.int8),
              "scales": dev_view("scales", s.size, torch.float32),
              "zeros": dev_view("zeros", z.size, torch.float32)}
    for k, n in (("x", d), ("xb", d), ("xb2", d), ("q", d), ("k", kv), ("v", kv),
                 ("att", CFG["n_heads"] * S), ("att_soft", CFG["n_heads"] * S), ("hb", h),
                 ("hb_silu", h), ("hb2", h), ("logits", V), ("key_cache", L * S * kv),
                 ("value_cache", L * S * kv)):
        arrays[k] = torch.zeros(n, device=dev)
    o = orc.LlamaQuantOracle(CFG, {"token_emb": w["token_embedding"].ravel(),
                                   "rms_att_w": w["rms_att"].ravel(), "rms_ffn_w": w["rms_ffn"].ravel(),
                                   "rms_final_w": w["rms_final"].ravel(), "wcls": w["wcls"].ravel(),
                                   "qweights": q, "scales": s, "zeros": z}, gs, offs)
    dims = tuple(CFG[k] for k in ("dim", "hidden_dim", "n_layers", "n_heads", "n_kv_heads",
                                  "vocab_size", "seq_len"))
    for pos, t in enumerate([50, 60, 70]):
        sa.llama2_quant_forward(arrays, t, pos, *dims, gs, offs)
        torch.cuda.synchronize()
        want = o.forward(t, pos).astype(np.float64)
        got = arrays["logits"].cpu().numpy().astype(np.float64)
        assert np.abs(got - want).max() <= TOL * np.abs(want).max(), pos
    sa.forward_cache_clear()
    m.close()


def test_w4_file_rejects_other_files(dev, tmp_path):
    w = random_llama2c(CFG, seed=8)
    ck = tmp_path / "m.bin"
    write_checkpoint(ck, CFG, w)
    with pytest.raises(sa.SimpRTError):
        sa.w4s_file_load(ck)                  # a checkpoint, not a SIMPW4S1 file
    out = tmp_path / "m.w4s"
    sa.w4s_file_write(ck, out, 32)
    with pytest.raises(sa.SimpRTError):
        sa.w4u_file_load(out)                 # wrong magic
    out.write_bytes(out.read_bytes()[:5000])
    with pytest.raises(sa.SimpRTError):
        sa.w4s_file_load(out)                 # truncated
