"""Arrays of llama32_forward (examples/llama2/llama32_1b_int8_tensor.sl) for tests:
the host buffers bench_llama32_1b_int8.cpp:136-188 allocates, filled as it fills
them (int8 uniform in [-64, 63], fp32 uniform in [-0.01, 0.01]) or, with
``wide=True``, with RMSNorm weights near 1 so that the quantized activations
span the int8 range and every stage of the program is exercised."""
import numpy as np

CFG_SMALL = dict(dim=256, hidden_dim=512, n_layers=2, n_heads=8, n_kv_heads=2, vocab_size=512,
                 max_seq_len=64, head_dim=32)
DIMS = ("dim", "hidden_dim", "n_layers", "n_heads", "n_kv_heads", "vocab_size", "max_seq_len",
        "head_dim")


def make_arrays(cfg: dict, seed: int, wide: bool = False) -> dict:
    rng = np.random.default_rng(seed)
    D, H, L, V, S = (cfg[k] for k in ("dim", "hidden_dim", "n_layers", "vocab_size", "max_seq_len"))
    kv = cfg["n_kv_heads"] * cfg["head_dim"]
    i8 = lambda n: rng.integers(-64, 64, n, dtype=np.int8)
    f32 = lambda n: rng.uniform(-0.01, 0.01, n).astype(np.float32)
    rms = (lambda n: rng.normal(1.0, 0.1, n).astype(np.float32)) if wide else f32
    return {
        "x_i8": i8(D), "rms_att_w": rms(L * D), "rms_ffn_w": rms(L * D), "rms_final_w": rms(D),
        "wq_t": i8(L * D * D), "wk_t": i8(L * kv * D), "wv_t": i8(L * kv * D),
        "wo_t": i8(L * D * D), "w1_t": i8(L * H * D), "w2_t": i8(L * D * H),
        "w3_t": i8(L * H * D), "wcls": f32(V * D),
        "x_fp32": np.zeros(D, np.float32), "xb_fp32": np.zeros(D, np.float32),
        "logits": np.zeros(V, np.float32), "xb_i8": np.zeros(D, np.int8),
        "k_cache": np.zeros(L * S * kv, np.int8), "v_cache": np.zeros(L * S * kv, np.int8),
        "att_scores": np.zeros(cfg["n_heads"] * S, np.float32),
        "att_probs": np.zeros(cfg["n_heads"] * S, np.float32),
        "attn_out": np.zeros(D, np.int32), "ffn_hb": np.zeros(H, np.int8),
    }
