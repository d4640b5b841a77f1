"""Writers of the llama2.c model files the reference host reads
(examples/llama2/generate_stories110M.cpp:25-70,143-191), for test fixtures.

Checkpoint: 7 int32 (dim, hidden_dim, n_layers, n_heads, n_kv_heads,
vocab_size, seq_len), then fp32 token_embedding, rms_att, wq, wk, wv, wo,
rms_ffn, w1, w2, w3, rms_final, and, for a negative vocab_size, llama2.c's
legacy RoPE tables (seq_len * head_size floats) and the classifier.
Tokenizer: int32 max_token_length, then per token float score, int32 length,
bytes."""
import struct

import numpy as np


def random_llama2c(cfg: dict, seed: int, shared: bool = True) -> dict:
    rng = np.random.default_rng(seed)
    d, h, L, V = cfg["dim"], cfg["hidden_dim"], cfg["n_layers"], cfg["vocab_size"]
    kv = d * cfg["n_kv_heads"] // cfg["n_heads"]
    r = lambda *s: (rng.standard_normal(s) * 0.02).astype(np.float32)
    w = {"token_embedding": r(V, d), "rms_att": (1 + r(L, d)), "wq": r(L, d, d), "wk": r(L, kv, d),
         "wv": r(L, kv, d), "wo": r(L, d, d), "rms_ffn": (1 + r(L, d)), "w1": r(L, h, d),
         "w2": r(L, d, h), "w3": r(L, h, d), "rms_final": (1 + r(d))}
    w["wcls"] = w["token_embedding"] if shared else r(V, d)
    return w


def write_checkpoint(path, cfg: dict, w: dict, shared: bool = True) -> None:
    hs = cfg["dim"] // cfg["n_heads"]
    v = cfg["vocab_size"] if shared else -cfg["vocab_size"]
    with open(path, "wb") as f:
        f.write(struct.pack("<7i", cfg["dim"], cfg["hidden_dim"], cfg["n_layers"], cfg["n_heads"],
                            cfg["n_kv_heads"], v, cfg["seq_len"]))
        for k in ("token_embedding", "rms_att", "wq", "wk", "wv", "wo", "rms_ffn", "w1", "w2", "w3",
                  "rms_final"):
            f.write(np.ascontiguousarray(w[k], np.float32).tobytes())
        if not shared:
            f.write(np.full(cfg["seq_len"] * hs, 7.0, np.float32).tobytes())  # legacy RoPE tables
            f.write(np.ascontiguousarray(w["wcls"], np.float32).tobytes())


def write_tokenizer(path, tokens, scores, max_token_length: int) -> None:
    with open(path, "wb") as f:
        f.write(struct.pack("<i", max_token_length))
        for t, s in zip(tokens, scores):
            f.write(struct.pack("<fi", s, len(t)))
            f.write(t)
