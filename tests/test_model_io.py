"""Model files and sampling on the host (no GPU): the llama2.c checkpoint
header and tokenizer the reference host reads, and its temperature sampler
(examples/llama2/generate_stories110M.cpp:25-116,143-150), against the files'
definitions and the oracle's restatement of std::mt19937 and
uniform_real_distribution<float>."""
import struct

import numpy as np
import pytest

import simplang_amd as sa

from _llama2c import write_tokenizer

CFG = dict(dim=64, hidden_dim=96, n_layers=2, n_heads=4, n_kv_heads=2, vocab_size=50, seq_len=16)


def _header(path, vals):
    with open(path, "wb") as f:
        f.write(struct.pack("<7i", *vals))


def test_ckpt_read_config(tmp_path):
    p = tmp_path / "m.bin"
    _header(p, [768, 2048, 12, 12, 12, 32000, 1024])          # stories110M's header
    assert sa.ckpt_read_config(p) == dict(dim=768, hidden_dim=2048, n_layers=12, n_heads=12,
                                          n_kv_heads=12, vocab_size=32000, seq_len=1024)
    _header(p, [64, 96, 2, 4, 2, -50, 16])                    # unshared classifier: negative
    assert sa.ckpt_read_config(p)["vocab_size"] == -50


@pytest.mark.parametrize("vals", [[64, 96, 2, 5, 5, 50, 16],   # dim % n_heads
                                  [64, 96, 2, 4, 3, 50, 16],   # n_heads % n_kv_heads
                                  [64, 96, 0, 4, 4, 50, 16],   # no layers
                                  [64, 96, 2, 4, 4, 0, 16]])   # no vocabulary
def test_ckpt_read_config_rejects(tmp_path, vals):
    p = tmp_path / "m.bin"
    _header(p, vals)
    with pytest.raises(sa.SimpRTError):
        sa.ckpt_read_config(p)


def test_ckpt_read_config_short_and_missing(tmp_path):
    p = tmp_path / "m.bin"
    p.write_bytes(b"\0" * 20)
    with pytest.raises(sa.SimpRTError):
        sa.ckpt_read_config(p)
    with pytest.raises(sa.SimpRTError):
        sa.ckpt_read_config(tmp_path / "absent.bin")


def test_tokenizer_decode_and_scores(tmp_path):
    toks = [b"<unk>", b"\n<s>\n", b"", b" the", "été".encode(), b"a\0b", bytes([0xff])]
    toks += [f"tok{i}".encode() for i in range(43)]
    scores = np.linspace(-3, 3, len(toks)).astype(np.float32)
    p = tmp_path / "tok.bin"
    write_tokenizer(p, toks, scores, 27)
    t = sa.Tokenizer(p, len(toks))
    assert t.max_token_length == 27
    for i, b in enumerate(toks):
        assert t.decode(i) == b
        assert t.score(i) == scores[i]
    assert t.decode(-1) == b"?" and t.decode(len(toks)) == b"?"   # generate_stories110M.cpp:64-66
    t.close()


def test_tokenizer_truncated(tmp_path):
    p = tmp_path / "tok.bin"
    write_tokenizer(p, [b"a", b"bb"], [0.0, 1.0], 2)
    with pytest.raises(sa.SimpRTError):
        sa.Tokenizer(p, 3)                     # the file holds two tokens, not three


def test_mt19937_standard_check_value(orc):
    """[rand.predef]: the 10000th draw of a default-constructed std::mt19937 is 4123659995."""
    g = orc.MT19937(5489)
    for _ in range(9999):
        g.next()
    assert g.next() == 4123659995


@pytest.mark.parametrize("seed", [0, 1, 42, 2**31 + 7])
@pytest.mark.parametrize("temperature", [0.0, 0.5, 0.9, 1.0, 1.7])
def test_sampler_matches_oracle(orc, seed, temperature):
    rng = np.random.default_rng(seed % 1000)
    s = sa.Sampler(seed)
    g = orc.MT19937(seed)
    for trial in range(40):
        n = 32000 if trial % 10 == 0 else int(rng.integers(1, 300))
        logits = (rng.standard_normal(n) * rng.uniform(0.1, 6)).astype(np.float32)
        assert s.sample(logits, temperature) == g.sample(logits, temperature), (trial, n)
    s.close()


def test_sampler_argmax_ties_and_uniform(orc):
    s = sa.Sampler(3)
    assert s.sample(np.array([1, 5, 5, 2], np.float32), 0.0) == 1     # first maximum
    # equal logits: the draw r picks floor(r * n) (up to rounding of the cdf)
    g = orc.MT19937(3)
    for _ in range(20):
        want = g.sample(np.zeros(7, np.float32), 1.0)
        assert s.sample(np.zeros(7, np.float32), 1.0) == want
