"""ctypes wrapper of the CPU oracle (oracle/_build/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker.  Nothing on the product path
imports it.  The optional in-place reference build (oracle/_ref/libsimpref.so,
only where the SimpLang sources are mounted in this container) is loaded only on
request, by ``load_ref()`` (None when it is not built).  It is listed in
.gpurunignore: it never travels to the GPU box, and no GPU test, smoke() or
bench.py loads it.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "_build", "liboracle.so")
REF_LIB = os.path.join(HERE, "_ref", "libsimpref.so")
REF_VNNI_TEST = os.path.join(HERE, "_ref", "test_vnni_correctness")

if not os.path.exists(LIB):
    raise ImportError(f"{LIB} not built (make -C oracle)")
_o = C.CDLL(LIB)
_ref = None

_P, _I, _F = C.c_void_p, C.c_int64, C.c_float


def _s(name, args, res=None):
    f = getattr(_o, name)
    f.argtypes = args
    f.restype = res
    return f


_s("orc_vpdpbusd16", [_P, _P, _P, _P])
_s("orc_matmul_i8", [_P, _I, _P, _I, _P, _I, _I, _I, _I, C.c_int, C.c_int])
_s("orc_matmul_i8_vnni", [_P, _P, _P, _I, _I, _I, C.c_int, C.c_int, C.c_int], C.c_int)
_s("orc_int8_recipe_inputs", [_I, _P, _P])
_s("orc_checksum_i32", [_P, _I], C.c_int32)
_s("orc_matmul_i4", [_P, _I, _P, _I, _P, _I, _I, _I, _I])
_s("orc_llama_quant_forward", [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _P, _P, _P, _I, _I, _P])
_s("orc_int4_recipe_inputs", [_I, _P, _P])
_s("orc_checksum_i16", [_P, _I], C.c_int32)
_s("orc_matmul_f32_acc", [_P, _P, _P, _I, _I, _I, _I, _I, _I])
_s("orc_batch_matmul_f32", [_P, _P, _P, _I, _I, _I, _I])
_s("orc_batch_matmul_f64", [_P, _P, _P, _I, _I, _I, _I])
_s("orc_rmsnorm", [_P, _P, _P, _I, _F, _I])
_s("orc_softmax", [_P, _P, _I, _I, _I])
_s("orc_silu", [_P, _P, _I])
_s("orc_matmul_quant_f5", [_P, _P, _P, _P, _P, _I, _I, _I, _I])
_s("orc_dequant_w4", [_P, _P, _P, _I, _I, _I, _P])
_s("orc_matmul_quant_f5_refidx", [_P, _P, _P, _P, _P, _I, _I, _I, _I])
_s("orc_quantize_f5", [_P, _I, _I, _P, _P, _P])
_s("orc_matmul_w4s", [_P, _P, _P, _P, _I, _I, _I, _I])
_s("orc_matmul_w4s_f32", [_P, _P, _P, _P, _I, _I, _I, _I, C.c_int])
_s("orc_matmul_w4s_lowering", [_P, _P, _P, _P, _I, _I, _I, _I, C.c_int])
_s("orc_rope", [_P, _P, _I, _I, _I, _I, _F])
_s("orc_argmax", [_P, _I], C.c_int64)
_s("orc_quantize_w4s", [_P, _I, _I, _I, _P, _P])


class OrcMT(C.Structure):
    _fields_ = [("mt", C.c_uint32 * 624), ("idx", C.c_int)]


_s("orc_mt_seed", [C.POINTER(OrcMT), C.c_uint32])
_s("orc_mt_next", [C.POINTER(OrcMT)], C.c_uint32)
_s("orc_uniform01f", [C.POINTER(OrcMT)], C.c_float)
_s("orc_sample", [_P, _I, C.c_float, C.POINTER(OrcMT)], C.c_int64)


class OrcLlamaCfg(C.Structure):
    _fields_ = [(n, C.c_int64) for n in ("dim", "hidden", "n_layers", "n_heads", "n_kv_heads",
                                         "vocab", "seq_len")] + [
        ("eps", C.c_float), ("theta", C.c_float), ("w4", C.c_int64), ("gs", C.c_int64)]


_ORC_W = ("emb", "rms_att", "rms_ffn", "rms_final", "wq", "wk", "wv", "wo", "w1", "w2", "w3",
          "wcls", "q_wq", "q_wk", "q_wv", "q_wo", "q_w1", "q_w2", "q_w3", "q_wcls",
          "s_wq", "s_wk", "s_wv", "s_wo", "s_w1", "s_w2", "s_w3", "s_wcls")


class OrcLlamaWeights(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in _ORC_W]


_s("orc_llama_forward", [_P, _P, _P, _P, _I, _I, _P])


class LlamaOracle:
    """orc_llama_forward over numpy weights (names as simp_rt_llama_weights;
    token_embedding -> emb).  Keeps its own KV cache."""

    def __init__(self, cfg: dict, weights: dict):
        self.cfg = cfg
        self._w = {k: np.ascontiguousarray(v) for k, v in weights.items()}
        kv_dim = cfg["dim"] * cfg["n_kv_heads"] // cfg["n_heads"]
        self.c = OrcLlamaCfg(dim=cfg["dim"], hidden=cfg["hidden_dim"], n_layers=cfg["n_layers"],
                             n_heads=cfg["n_heads"], n_kv_heads=cfg["n_kv_heads"],
                             vocab=cfg["vocab_size"], seq_len=cfg["seq_len"],
                             eps=cfg.get("eps", 1e-5), theta=cfg.get("rope_theta", 10000.0),
                             w4=int(cfg.get("weight_format", 0) == 1), gs=cfg.get("group_size", 32))
        ptrs = {("emb" if k == "token_embedding" else k): v.ctypes.data for k, v in self._w.items()}
        self.w = OrcLlamaWeights(**ptrs)
        n = cfg["n_layers"] * cfg["seq_len"] * kv_dim
        self.kc = np.zeros(n, np.float32)
        self.vc = np.zeros(n, np.float32)

    def forward(self, token: int, pos: int):
        logits = np.empty(self.cfg["vocab_size"], np.float32)
        _o.orc_llama_forward(C.byref(self.c), C.byref(self.w), self.kc.ctypes.data,
                             self.vc.ctypes.data, token, pos, logits.ctypes.data)
        return logits

_s("cpu_llama_forward", [_P, _P, _P, _P, _I, _I, _P])
_s("cpu_llama_supported", [_P], C.c_int)


class CpuLlama(LlamaOracle):
    """The decode CPU baseline (cpu_decode.c: fp32, OpenMP GEMVs in 16 fp32
    lanes) with the same weights and cache layout as LlamaOracle."""

    def __init__(self, cfg: dict, weights: dict):
        super().__init__(cfg, weights)
        if not _o.cpu_llama_supported(C.byref(self.c)):
            raise ValueError("cpu_llama_forward: W4 needs gs a multiple of 32 dividing dim and hidden")

    def forward(self, token: int, pos: int):
        logits = np.empty(self.cfg["vocab_size"], np.float32)
        _o.cpu_llama_forward(C.byref(self.c), C.byref(self.w), self.kc.ctypes.data,
                             self.vc.ctypes.data, token, pos, logits.ctypes.data)
        return logits


_s("orc_llama32_int8_forward", [_P, _I] + [_P] * 22 + [_I], C.c_float)

LLAMA32_ARRAYS = ("x_i8", "rms_att_w", "rms_ffn_w", "rms_final_w", "wq_t", "wk_t", "wv_t",
                  "wo_t", "w1_t", "w2_t", "w3_t", "wcls", "x_fp32", "xb_fp32", "logits", "xb_i8",
                  "k_cache", "v_cache", "att_scores", "att_probs", "attn_out", "ffn_hb")


def llama32_int8_forward(arrays: dict, pos, dim, hidden_dim, n_layers, n_heads, n_kv_heads,
                         vocab_size, max_seq_len, head_dim) -> float:
    """orc_llama32_int8_forward over numpy arrays named as llama32_forward's
    parameters (contiguous, the program's dtypes); writes them as the program
    does and returns logits[0]."""
    c = OrcLlamaCfg(dim=dim, hidden=hidden_dim, n_layers=n_layers, n_heads=n_heads,
                    n_kv_heads=n_kv_heads, vocab=vocab_size, seq_len=max_seq_len, eps=1e-5,
                    theta=0.0, w4=0, gs=32)
    for name in LLAMA32_ARRAYS:
        a = arrays[name]
        if not (isinstance(a, np.ndarray) and a.flags["C_CONTIGUOUS"]):
            raise ValueError(f"{name} must be a contiguous numpy array")
    return _o.orc_llama32_int8_forward(C.byref(c), head_dim,
                                       *[arrays[n].ctypes.data for n in LLAMA32_ARRAYS], pos)


class LlamaQuantOracle:
    """orc_llama_quant_forward (llama2_quant.sl) over numpy arrays named as the
    program's parameters; keeps its own KV cache."""

    def __init__(self, cfg: dict, arrays: dict, group_size: int, offsets):
        self.cfg = cfg
        self.a = {k: np.ascontiguousarray(v) for k, v in arrays.items()}
        self.gs = group_size
        self.off = (C.c_int64 * 7)(*offsets)
        kv_dim = cfg["dim"] * cfg["n_kv_heads"] // cfg["n_heads"]
        self.c = OrcLlamaCfg(dim=cfg["dim"], hidden=cfg["hidden_dim"], n_layers=cfg["n_layers"],
                             n_heads=cfg["n_heads"], n_kv_heads=cfg["n_kv_heads"],
                             vocab=cfg["vocab_size"], seq_len=cfg["seq_len"], eps=1e-5, theta=0.0,
                             w4=0, gs=group_size)
        n = cfg["n_layers"] * cfg["seq_len"] * kv_dim
        self.kc = np.zeros(n, np.float32)
        self.vc = np.zeros(n, np.float32)

    def forward(self, token: int, pos: int):
        a = self.a
        logits = np.empty(self.cfg["vocab_size"], np.float32)
        _o.orc_llama_quant_forward(C.byref(self.c), a["token_emb"].ctypes.data,
                                   a["rms_att_w"].ctypes.data, a["rms_ffn_w"].ctypes.data,
                                   a["rms_final_w"].ctypes.data, a["wcls"].ctypes.data,
                                   a["qweights"].ctypes.data, a["scales"].ctypes.data,
                                   a["zeros"].ctypes.data, self.gs, self.off, self.kc.ctypes.data,
                                   self.vc.ctypes.data, token, pos, logits.ctypes.data)
        return logits


def load_ref():
    """The reference's own kernels compiled in place (oracle/Makefile target
    ``ref``), or None where they are not built.  Loaded on first use only."""
    global _ref
    if _ref is None and os.path.exists(REF_LIB):
        r = C.CDLL(REF_LIB)
        for n in ("ref_scalar_vpdpbusd", "ref_hw_vpdpbusd"):
            getattr(r, n).argtypes = [_P, _P, _P, _P]
        for n in (64, 128, 256, 512, 1024, 2048):
            getattr(r, f"ref_vnni_matmul_{n}").argtypes = [_P, _P, _P]
        for n in (32, 64, 128):
            getattr(r, f"ref_scalar_int4_{n}").restype = C.c_int32
            getattr(r, f"ref_packed_int4_{n}").restype = C.c_int32
        _ref = r
    return _ref


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def vpdpbusd16(a, b, acc):
    a = np.ascontiguousarray(a, np.uint8)
    b = np.ascontiguousarray(b, np.int8)
    acc = np.ascontiguousarray(acc, np.int32)
    out = np.empty(16, np.int32)
    _o.orc_vpdpbusd16(_p(a), _p(b), _p(acc), _p(out))
    return out


def matmul_i8(a, b, *, a_unsigned=False, b_nk=False):
    """Textbook int8 GEMM (i32 wraparound).  b is [K,N], or [N,K] if b_nk."""
    a = np.ascontiguousarray(a, np.uint8 if a_unsigned else np.int8)
    b = np.ascontiguousarray(b, np.int8)
    M, K = a.shape
    N = b.shape[0] if b_nk else b.shape[1]
    c = np.empty((M, N), np.int32)
    _o.orc_matmul_i8(_p(a), K, _p(b), b.shape[1], _p(c), N, M, N, K,
                     int(a_unsigned), int(b_nk))
    return c


def matmul_i8_vnni(a, b, *, a_unsigned=False, b_nk=False, nthreads=1):
    """The VNNI-pass algorithm (CPU baseline).  Returns (C, used_avx512_vnni)."""
    a = np.ascontiguousarray(a, np.uint8 if a_unsigned else np.int8)
    b = np.ascontiguousarray(b, np.int8)
    M, K = a.shape
    N = b.shape[0] if b_nk else b.shape[1]
    c = np.empty((M, N), np.int32)
    hw = _o.orc_matmul_i8_vnni(_p(a), _p(b), _p(c), M, N, K, int(a_unsigned),
                               int(b_nk), int(nthreads))
    return c, bool(hw)


def recipe_inputs(n: int):
    a = np.empty((n, n), np.int8)
    b = np.empty((n, n), np.int8)
    _o.orc_int8_recipe_inputs(n, _p(a), _p(b))
    return a, b


def matmul_i4(ap, bp, m: int, n: int, k: int):
    """Packed signed-nibble product: ap [M, >=(K+1)/2] u8 packed along K, bp
    [K, >=(N+1)/2] u8 packed along N; returns C [M, N] i16 (i32 sum truncated)."""
    ap = np.ascontiguousarray(ap, np.uint8)
    bp = np.ascontiguousarray(bp, np.uint8)
    c = np.zeros((m, n), np.int16)
    _o.orc_matmul_i4(_p(ap), ap.shape[1] if ap.ndim == 2 else 0, _p(bp),
                     bp.shape[1] if bp.ndim == 2 else 0, _p(c), n, m, n, k)
    return c


def int4_recipe_inputs(n: int):
    pd = (n + 1) // 2
    ap = np.zeros((n, pd), np.uint8)
    bp = np.zeros((n, pd), np.uint8)
    _o.orc_int4_recipe_inputs(n, _p(ap), _p(bp))
    return ap, bp


def checksum_i16(c) -> int:
    c = np.ascontiguousarray(c, np.int16)
    return int(_o.orc_checksum_i16(_p(c), c.size))


def pack_i4(v, axis=-1):
    """Pack signed values in [-8, 7] two per byte along `axis` (low nibble = even)."""
    v = np.asarray(v)
    v = np.moveaxis(v, axis, -1)
    if v.shape[-1] % 2:
        v = np.concatenate([v, np.zeros(v.shape[:-1] + (1,), v.dtype)], -1)
    u = (v.astype(np.int16) & 15).astype(np.uint8)
    p = u[..., 0::2] | (u[..., 1::2] << 4)
    return np.ascontiguousarray(np.moveaxis(p, -1, axis))


def checksum_i32(c) -> int:
    c = np.ascontiguousarray(c, np.int32)
    return int(_o.orc_checksum_i32(_p(c), c.size))


def matmul_f32_acc(lhs, rhs, out, m, k, n, lhs_off=0, rhs_off=0, out_off=0):
    _o.orc_matmul_f32_acc(_p(lhs), _p(rhs), _p(out), m, k, n, lhs_off, rhs_off, out_off)
    return out


def batch_matmul(a, b):
    """Rank-3 ``tensor_matmul``: C[b] = A[b] B[b] (ConvertSimpToMemRef.cpp:3286-3291).

    f32 and f64 go to orc_batch_matmul_*; i8 (s8 x s8 -> i32, linalg's sign
    extension) runs orc_matmul_i8 on each batch."""
    if a.ndim != 3 or b.ndim != 3 or a.shape[0] != b.shape[0] or a.shape[2] != b.shape[1]:
        raise ValueError("batch_matmul: A[Bt,M,K] x B[Bt,K,N] expected")
    bt, m, k = a.shape
    n = b.shape[2]
    if a.dtype == np.int8:
        c = np.empty((bt, m, n), np.int32)
        for i in range(bt):
            c[i] = matmul_i8(np.ascontiguousarray(a[i]), np.ascontiguousarray(b[i]))
        return c
    dt = np.float64 if a.dtype == np.float64 else np.float32
    a = np.ascontiguousarray(a, dt)
    b = np.ascontiguousarray(b, dt)
    c = np.empty((bt, m, n), dt)
    fn = _o.orc_batch_matmul_f64 if dt == np.float64 else _o.orc_batch_matmul_f32
    fn(_p(a), _p(b), _p(c), bt, m, k, n)
    return c


def matmul_nhwc(x, w):
    """4-D x 2-D ``tensor_matmul`` (ConvertSimpToMemRef.cpp:3293-3361), in the
    reference's steps: collapse (N,H,W) to rows, transpose the [C_out, C_in]
    weights to [C_in, C_out], multiply, expand back."""
    nb, h, wd, cin = x.shape
    cout = w.shape[0]
    if w.shape[1] != cin:
        raise ValueError("matmul_nhwc: weights must be [C_out, C_in]")
    rows = np.ascontiguousarray(x).reshape(1, nb * h * wd, cin)
    wt = np.ascontiguousarray(np.asarray(w).T).reshape(1, cin, cout)
    return batch_matmul(rows, wt).reshape(nb, h, wd, cout)


def rmsnorm(x, w, eps=1e-5, w_off=0, size=None):
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    size = x.size if size is None else size
    out = np.empty(size, np.float32)
    _o.orc_rmsnorm(_p(x), _p(w), _p(out), size, eps, w_off)
    return out


def softmax(x, out=None, size=None, in_off=0, out_off=0):
    x = np.ascontiguousarray(x, np.float32)
    size = x.size - in_off if size is None else size
    if out is None:
        out = np.zeros(out_off + size, np.float32)
    _o.orc_softmax(_p(x), _p(out), size, in_off, out_off)
    return out


def silu(x):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    _o.orc_silu(_p(x), _p(out), x.size)
    return out


def matmul_quant_f5(qw, scales, zeros, x, rows, cols, gs, off=0):
    out = np.empty(rows, np.float32)
    _o.orc_matmul_quant_f5(_p(qw), _p(scales), _p(zeros), _p(x), _p(out), rows, cols, gs, off)
    return out


def dequant_w4(qw, scales, zeros, idx, count, gs):
    out = np.empty(count, np.float32)
    _o.orc_dequant_w4(_p(qw), _p(scales), _p(zeros), idx, count, gs, _p(out))
    return out


def matmul_quant_f5_refidx(qw, scales, zeros, x, rows, cols, gs, off=0):
    """MatMulQuantOpLowering exactly as the reference emits it (scale index
    without the offset, a fixed 8 tiles of 16 per group)."""
    out = np.empty(rows, np.float32)
    _o.orc_matmul_quant_f5_refidx(_p(qw), _p(scales), _p(zeros), _p(x), _p(out), rows, cols, gs,
                                  off)
    return out


def quantize_f5(w, gs):
    w = np.ascontiguousarray(w, np.float32).ravel()
    ng = (w.size + gs - 1) // gs
    qw = np.empty((w.size + 1) // 2, np.uint8)
    sc = np.empty(ng, np.float32)
    ze = np.empty(ng, np.float32)
    _o.orc_quantize_f5(_p(w), w.size, gs, _p(qw), _p(sc), _p(ze))
    return qw, sc, ze


def quantize_w4s(w, gs):
    """Symmetric W4 of w [rows, cols]: (q [rows, cols/2] u8, scales [rows, cols/gs])."""
    w = np.ascontiguousarray(w, np.float32)
    rows, cols = w.shape
    qw = np.empty((rows, cols // 2), np.uint8)
    sc = np.empty((rows, cols // gs), np.float32)
    _o.orc_quantize_w4s(_p(w), rows, cols, gs, _p(qw), _p(sc))
    return qw, sc


class MT19937:
    """std::mt19937 restated (orc_mt_*)."""

    def __init__(self, seed: int):
        self._g = OrcMT()
        _o.orc_mt_seed(C.byref(self._g), seed & 0xFFFFFFFF)

    def next(self) -> int:
        return int(_o.orc_mt_next(C.byref(self._g)))

    def uniform01f(self) -> float:
        return float(_o.orc_uniform01f(C.byref(self._g)))

    def sample(self, logits, temperature: float) -> int:
        lg = np.ascontiguousarray(logits, np.float32)
        return int(_o.orc_sample(_p(lg), lg.size, C.c_float(temperature), C.byref(self._g)))


def matmul_w4s(qw, scales, x, gs=32):
    """F6 W4: qw [N, K/2] u8, scales [N, K/gs] f32, x [M, K] f32 -> [M, N] (f64 accumulate)."""
    x = np.ascontiguousarray(x, np.float32)
    M, K = x.shape
    N = qw.shape[0]
    out = np.empty((M, N), np.float32)
    _o.orc_matmul_w4s(_p(np.ascontiguousarray(qw)), _p(np.ascontiguousarray(scales)), _p(x),
                      _p(out), M, N, K, gs)
    return out


def matmul_w4s_f32(qw, scales, x, gs=32, nthreads=1):
    x = np.ascontiguousarray(x, np.float32)
    M, K = x.shape
    N = qw.shape[0]
    out = np.empty((M, N), np.float32)
    _o.orc_matmul_w4s_f32(_p(qw), _p(scales), _p(x), _p(out), M, N, K, gs, nthreads)
    return out


def matmul_w4s_lowering(qw, scales, x, gs=32, nthreads=1):
    """The symmetric W4 product through MatMulQuantOpLowering's loop structure
    (the W4 GEMV CPU baseline)."""
    x = np.ascontiguousarray(x, np.float32)
    M, K = x.shape
    N = qw.shape[0]
    out = np.empty((M, N), np.float32)
    _o.orc_matmul_w4s_lowering(_p(qw), _p(scales), _p(x), _p(out), M, N, K, gs, nthreads)
    return out


def rope(q, k, dim, kv_dim, hs, pos, theta=10000.0):
    _o.orc_rope(_p(q), _p(k), dim, kv_dim, hs, pos, theta)
    return q, k


def argmax(logits) -> int:
    logits = np.ascontiguousarray(logits, np.float32)
    return int(_o.orc_argmax(_p(logits), logits.size))
