"""Random-init LLaMA weights for the decode engine (tests and bench.py) (no checkpoints
exist offline; the reference's own hosts use random weights too:
examples/llama2/test_stories110M.cpp:20-22,122-133, N(0, 0.02) for every array).

fp32 models (the 110M benchmark configuration): every array N(0, 0.02).
W4 models (the 3B W4-g32 configuration): norms and embedding N(0, 0.02) fp32; every linear
weight (classifier included) symmetric int4 uniform in [-8, 7], packed two per
byte along K (low nibble = even k), one fp32 scale |N(0, 0.02)|/7 per group of
32 along K.  Generated on the device with torch (seeded) so that 3B-size models
build in seconds."""
import numpy as np

CFG_110M = dict(dim=768, hidden_dim=2048, n_layers=12, n_heads=12, n_kv_heads=12,
                vocab_size=32000, seq_len=288, eps=1e-5, rope_theta=10000.0,
                weight_format=0, group_size=32)
CFG_3B_W4 = dict(dim=3200, hidden_dim=8640, n_layers=26, n_heads=32, n_kv_heads=32,
                 vocab_size=32000, seq_len=512, eps=1e-5, rope_theta=10000.0,
                 weight_format=1, group_size=32)


def shapes(cfg):
    d, h, L, V = cfg["dim"], cfg["hidden_dim"], cfg["n_layers"], cfg["vocab_size"]
    kv = d * cfg["n_kv_heads"] // cfg["n_heads"]
    mats = {"wq": (L, d, d), "wk": (L, kv, d), "wv": (L, kv, d), "wo": (L, d, d),
            "w1": (L, h, d), "w2": (L, d, h), "w3": (L, h, d), "wcls": (V, d)}
    vecs = {"token_embedding": (V, d), "rms_att": (L, d), "rms_ffn": (L, d), "rms_final": (d,)}
    return mats, vecs


def make_model(cfg, device, seed=42):
    """Returns a dict of device tensors named as simp_rt_llama_weights."""
    import torch
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    mats, vecs = shapes(cfg)
    w = {}
    for name, shp in vecs.items():
        w[name] = torch.randn(shp, generator=g, device=device) * 0.02
    gs = cfg.get("group_size", 32)
    for name, shp in mats.items():
        if cfg.get("weight_format", 0) == 0:
            w[name] = torch.randn(shp, generator=g, device=device) * 0.02
        else:
            rows = int(np.prod(shp[:-1]))
            k = shp[-1]
            w["q_" + name] = torch.randint(0, 256, (rows, k // 2), dtype=torch.uint8,
                                           generator=g, device=device)
            w["s_" + name] = torch.randn((rows, k // gs), generator=g, device=device).abs() * (0.02 / 7)
    return w


def to_numpy(w):
    return {k: v.detach().cpu().numpy() for k, v in w.items()}


def weight_bytes(cfg):
    """Bytes of weights one decode step streams (all matrices, the norms and one
    embedding row), the algorithmic traffic of a step without the KV cache."""
    mats, vecs = shapes(cfg)
    n = sum(int(np.prod(s)) for s in mats.values())
    if cfg.get("weight_format", 0) == 0:
        b = 4 * n
    else:
        b = n // 2 + 4 * n // cfg.get("group_size", 32)
    d, L = cfg["dim"], cfg["n_layers"]
    return b + 4 * (2 * L * d + d) + 4 * d


def kv_bytes(cfg, pos):
    """KV-cache bytes the attention of one step at position pos reads and writes."""
    kv = cfg["dim"] * cfg["n_kv_heads"] // cfg["n_heads"]
    return 2 * cfg["n_layers"] * (pos + 1) * kv * 4
