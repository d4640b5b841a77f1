"""ctypes binding of libsimp_hip.so and the host-side operator mirror.

Operands are torch tensors on the GPU (used in place, asynchronous on the
stream given to :func:`set_stream`) or numpy arrays (staged by the library,
synchronous).  Descriptor expansion follows the reference host ABI
(``examples/llama2/bench_llama_quant.cpp:10-28``): rank-1 arrays as
``(alloc, aligned, offset, size, stride)``, rank-2 tensors as
``(alloc, aligned, offset, size0, size1, stride0, stride1)``.
"""
from __future__ import annotations

import ctypes as C
import os
import re

_HERE = os.path.dirname(os.path.abspath(__file__))
# SIMP_HIP_LIB selects another build of the library (the host-sanitized
# libsimp_hip_san.so, loaded with the compiler's ASan runtime preloaded)
lib_path = os.environ.get("SIMP_HIP_LIB") or os.path.join(_HERE, "libsimp_hip.so")
HEADER = os.path.join(os.path.dirname(_HERE), "include", "simp_rt.h")


class SimpRTError(RuntimeError):
    """A libsimp_hip.so entry point returned a negative status."""

    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} -> {code}: {msg}")
        self.code = code


def _load():
    if not os.path.exists(lib_path):
        raise ImportError(
            f"{lib_path} is not built; run __graft_entry__.build() "
            "(the HIP runtime has no CPU fallback)")
    return C.CDLL(lib_path, mode=C.RTLD_GLOBAL)


lib = _load()
lib.simp_rt_last_error.restype = C.c_char_p
lib.simp_rt_error_count.restype = C.c_int64
lib.simp_rt_error_count.argtypes = []
lib.simp_rt_get_stream.restype = C.c_void_p

_P, _I = C.c_void_p, C.c_int64
_D1 = [_P, _P, _I, _I, _I]
_D2 = [_P, _P, _I, _I, _I, _I, _I]


def _sig(name, argtypes):
    f = getattr(lib, name)
    f.argtypes = argtypes
    f.restype = C.c_int32
    return f


for _n in ("simp_rt_tensor_matmul_i8", "simp_rt_tensor_matmul_nt_i8",
           "simp_rt_matmul_u8s8_i32", "simp_rt_matmul_nt_u8s8_i32", "simp_rt_tensor_matmul_i4",
           "simp_rt_tensor_matvecmul_i8", "simp_rt_matmul_u8s8_i32_noalloc"):
    _sig(_n, _D2 * 3)
_sig("simp_rt_matmul_quant", _D1 * 5 + [_I, _I, _I, _I])
_sig("simp_rt_matmul_w4s", _D2 * 4 + [_I])
_sig("simp_rt_dequant_w4", _D1 * 3 + [_I, _I] + _D1 + [_I])
_sig("simp_rt_matmul_f32", _D1 * 3 + [_I] * 6)
_sig("simp_rt_tensor_matmul_f32", _D2 * 3)
_sig("simp_rt_tensor_matmul_nt_f32", _D2 * 3)
_sig("simp_rt_tensor_matvecmul_f32", _D2 * 3)
_sig("simp_rt_tensor_matmul_f64", _D2 * 3)
_D3 = [_P, _P, _I] + [_I] * 6
_D4 = [_P, _P, _I] + [_I] * 8
for _n in ("simp_rt_tensor_batch_matmul_f32", "simp_rt_tensor_batch_matmul_f64",
           "simp_rt_tensor_batch_matmul_i8"):
    _sig(_n, _D3 * 3)
for _n in ("simp_rt_tensor_matmul_nhwc_f32", "simp_rt_tensor_matmul_nhwc_f64"):
    _sig(_n, _D4 + _D2 + _D4)
_sig("simp_rt_rmsnorm", _D1 * 3 + [_I, C.c_double, _I])
_sig("simp_rt_softmax", _D1 * 2 + [_I, _I, _I])
_sig("simp_rt_silu", _D1 * 2 + [_I])
_sig("simp_rt_swiglu", _D1 * 3 + [_I])
_sig("simp_rt_rope", _D1 * 2 + [_I, _I, _I, _I, C.c_double])
_sig("simp_rt_llama_create", [_P, _P, _P])
_sig("simp_rt_llama_destroy", [_P])
_sig("simp_rt_llama_forward", [_P, _I, _I, _P])
_sig("simp_rt_llama_generate", [_P, _P, _I, _I, _P, C.c_int32])
_sig("simp_rt_set_stream", [_P])
_sig("simp_rt_register", [_P, _I, C.c_int32])
_sig("simp_rt_unregister", [_P])
_sig("simp_rt_timing", [C.c_int32])
_sig("simp_rt_forward_cache_clear", [])
lib.stories110M_forward.argtypes = [_P, _P, _I, _I, _I] * 25 + [_I] * 9
lib.stories110M_forward.restype = C.c_float
lib.llama2_quant_forward.argtypes = [_P, _P, _I, _I, _I] * 22 + [_I] * 17
lib.llama2_quant_forward.restype = C.c_float
lib.llama32_forward.argtypes = [_P, _P, _I, _I, _I] * 22 + [_I] * 9
lib.llama32_forward.restype = C.c_float
_sig("simp_rt_timing_query", [C.c_char_p, C.POINTER(C.c_double), C.POINTER(C.c_int64)])


def declared_symbols(header: str = HEADER) -> list[str]:
    """Names of the entry points include/simp_rt.h declares."""
    text = open(header).read()
    names = set(re.findall(r"\b(simp_rt_\w+)\s*\(", text))
    # model-level exports keep the reference program's names
    names |= set(re.findall(r"^float\s+(\w+_forward)\s*\(", text, re.M))
    # the int8 benchmark programs keep theirs too
    names |= set(re.findall(r"^int32_t\s+(benchmark_int8_matmul_\d+|kernel_main)\s*\(", text, re.M))
    names |= {f"int8_chunk_{n}" for n in re.findall(r"^SIMP_RT_INT8_CHUNK\((\d+)\);", text, re.M)}
    return sorted(names)


def _check(fn: str, rc: int):
    if rc != 0:
        raise SimpRTError(fn, rc, lib.simp_rt_last_error().decode())


def last_error() -> str:
    """The calling thread's last error message ('' after a model-level export
    that succeeded)."""
    return lib.simp_rt_last_error().decode()


def _check_float(fn: str, errors_before: int, r: float) -> float:
    """Model-level exports return a float (NaN on error): an error is told from
    a NaN of the arithmetic by the thread's error count."""
    if lib.simp_rt_error_count() != errors_before:
        raise SimpRTError(fn, -1, lib.simp_rt_last_error().decode())
    return r


# ------------------------------------------------------------------ operands

def _is_torch(x) -> bool:
    return type(x).__module__.startswith("torch")


def _ptr_stride(x):
    """(data pointer, row stride in elements, shape) of a 1-D/2-D operand."""
    if _is_torch(x):
        if x.dim() == 2:
            if x.stride(1) != 1:
                raise ValueError("rank-2 operand must be row-major (stride1 == 1)")
            return x.data_ptr(), x.stride(0), tuple(x.shape)
        if x.dim() == 1:
            if x.stride(0) != 1:
                raise ValueError("rank-1 operand must be contiguous")
            return x.data_ptr(), 1, tuple(x.shape)
        raise ValueError("operand must be rank 1 or 2")
    import numpy as np
    if not isinstance(x, np.ndarray):
        raise TypeError(f"unsupported operand type {type(x)}")
    isz = x.itemsize
    if x.ndim == 2:
        if x.strides[1] != isz:
            raise ValueError("rank-2 operand must be row-major (stride1 == 1)")
        return x.ctypes.data, x.strides[0] // isz, x.shape
    if x.ndim == 1:
        if x.strides[0] != isz:
            raise ValueError("rank-1 operand must be contiguous")
        return x.ctypes.data, 1, x.shape
    raise ValueError("operand must be rank 1 or 2")


def desc2(x):
    p, st0, shape = _ptr_stride(x)
    if len(shape) != 2:
        raise ValueError("expected a rank-2 tensor")
    return [p, p, 0, shape[0], shape[1], st0, 1]


def descn(x, rank: int):
    """Rank-``rank`` memref descriptor (alloc, aligned, offset, sizes..., strides...)
    of a torch tensor or numpy array; strides in elements, the innermost must be 1."""
    if _is_torch(x):
        p, shape, strides = x.data_ptr(), tuple(x.shape), tuple(x.stride())
    else:
        import numpy as np
        if not isinstance(x, np.ndarray):
            raise TypeError(f"unsupported operand type {type(x)}")
        p, shape = x.ctypes.data, x.shape
        if any(st % x.itemsize for st in x.strides):
            raise ValueError("strides must be whole elements")
        strides = tuple(st // x.itemsize for st in x.strides)
    if len(shape) != rank:
        raise ValueError(f"expected a rank-{rank} tensor, got shape {tuple(shape)}")
    return [p, p, 0, *shape, *strides]


def desc1(x):
    p, _, shape = _ptr_stride(x)
    n = 1
    for s in shape:
        n *= s
    return [p, p, 0, n, 1]


# --------------------------------------------------------------------- ops

def set_stream(stream) -> None:
    """Make the calling thread's launches go to ``stream`` (torch stream, int or None)."""
    if stream is None:
        h = None
    elif hasattr(stream, "cuda_stream"):
        h = stream.cuda_stream
    else:
        h = int(stream)
    _check("simp_rt_set_stream", lib.simp_rt_set_stream(h))


def sync() -> None:
    _check("simp_rt_sync", lib.simp_rt_sync())


def timing(on: bool) -> None:
    """Start (clearing earlier records) or stop per-kernel HIP-event timing."""
    _check("simp_rt_timing", lib.simp_rt_timing(1 if on else 0))


def timing_query(kernel: str):
    """(total ms, launches) recorded for ``kernel`` since timing(True)."""
    ms, n = C.c_double(), C.c_int64()
    _check("simp_rt_timing_query", lib.simp_rt_timing_query(kernel.encode(), C.byref(ms), C.byref(n)))
    return ms.value, n.value


def _gemm(fn_name, a, b, c):
    f = getattr(lib, fn_name)
    _check(fn_name, f(*desc2(a), *desc2(b), *desc2(c)))
    return c


def tensor_matmul_i8(a, b, c):
    """C[M,N] = A[M,K] x B[K,N], s8 x s8 -> i32 (SimpLang ``tensor_matmul`` on i8)."""
    return _gemm("simp_rt_tensor_matmul_i8", a, b, c)


def tensor_matmul_nt_i8(a, bt, c):
    """C[M,N] = A[M,K] x B_T[N,K]^T, s8 x s8 -> i32 (``tensor_matmul_nt``)."""
    return _gemm("simp_rt_tensor_matmul_nt_i8", a, bt, c)


STORIES_ARRAYS = ("token_embedding_table", "rms_att_w", "wq", "wk", "wv", "wo", "rms_ffn_w",
                  "w1", "w2", "w3", "rms_final_w", "wcls", "x", "xb", "xb2", "hb", "hb_silu",
                  "q", "k", "v", "att", "att_soft", "logits", "key_cache", "value_cache")


def stories110M_forward(arrays: dict, token, pos, dim, hidden_dim, n_layers, n_heads,
                        n_kv_heads, vocab_size, seq_len) -> float:
    """The compiled program's entry point (examples/llama2/stories110M.sl:5-44):
    ``arrays`` maps the 25 f32[] parameter names to 1-D numpy arrays or torch
    tensors; returns logits[0].  Raises on a NaN return with the library's
    error message."""
    args = []
    for name in STORIES_ARRAYS:
        args += desc1(arrays[name])
    n0 = lib.simp_rt_error_count()
    r = lib.stories110M_forward(*args, token, pos, dim, hidden_dim, n_layers, n_heads,
                                n_kv_heads, vocab_size, seq_len)
    return _check_float("stories110M_forward", n0, r)


QUANT_ARRAYS = ("token_emb", "rms_att_w", "rms_ffn_w", "rms_final_w", "wcls", "qweights",
                "scales", "zeros", "x", "xb", "xb2", "q", "k", "v", "att", "att_soft", "hb",
                "hb_silu", "hb2", "logits", "key_cache", "value_cache")


def llama2_quant_forward(arrays: dict, token, pos, dim, hidden_dim, n_layers, n_heads, n_kv_heads,
                         vocab_size, seq_len, group_size, offsets) -> float:
    """The reference W4 program's entry point (examples/llama2/llama2_quant.sl:7-56):
    ``arrays`` maps its 22 array parameters to 1-D arrays (``qweights`` int8),
    ``offsets`` = (wq, wk, wv, wo, w1, w2, w3) element offsets; returns logits[0]."""
    args = []
    for name in QUANT_ARRAYS:
        args += desc1(arrays[name])
    n0 = lib.simp_rt_error_count()
    r = lib.llama2_quant_forward(*args, token, pos, dim, hidden_dim, n_layers, n_heads, n_kv_heads,
                                 vocab_size, seq_len, group_size, *offsets)
    return _check_float("llama2_quant_forward", n0, r)


LLAMA32_ARRAYS = ("x_i8", "rms_att_w", "rms_ffn_w", "rms_final_w", "wq_t", "wk_t", "wv_t",
                  "wo_t", "w1_t", "w2_t", "w3_t", "wcls", "x_fp32", "xb_fp32", "logits", "xb_i8",
                  "k_cache", "v_cache", "att_scores", "att_probs", "attn_out", "ffn_hb")


def llama32_forward(arrays: dict, pos, dim, hidden_dim, n_layers, n_heads, n_kv_heads,
                    vocab_size, max_seq_len, head_dim) -> float:
    """``llama32_forward`` of examples/llama2/llama32_1b_int8_tensor.sl, called as
    bench_llama32_1b_int8.cpp calls it: ``arrays`` maps the program's parameter
    names (LLAMA32_ARRAYS) to 1-D arrays (i8 / f32 / i32).  Returns logits[0]
    (raises SimpRTError when the call reports an error)."""
    args = []
    for name in LLAMA32_ARRAYS:
        args += desc1(arrays[name])
    n0 = lib.simp_rt_error_count()
    r = lib.llama32_forward(*args, pos, dim, hidden_dim, n_layers, n_heads, n_kv_heads,
                            vocab_size, max_seq_len, head_dim)
    return _check_float("llama32_forward", n0, r)


class Llama32Program:
    """``llama32_forward`` bound to one set of arrays, as a C++ host binds it:
    the 22 descriptors are built once, and each call passes only the position
    (the arrays must stay alive and in place while the object is used)."""

    def __init__(self, arrays: dict, dim, hidden_dim, n_layers, n_heads, n_kv_heads,
                 vocab_size, max_seq_len, head_dim):
        args = []
        for name in LLAMA32_ARRAYS:
            args += desc1(arrays[name])
        self._arrays = arrays
        self._args = args
        self._dims = (dim, hidden_dim, n_layers, n_heads, n_kv_heads, vocab_size, max_seq_len,
                      head_dim)

    def __call__(self, pos) -> float:
        n0 = lib.simp_rt_error_count()
        r = lib.llama32_forward(*self._args, pos, *self._dims)
        return _check_float("llama32_forward", n0, r)


BENCH_INT8_SIZES = (32, 64, 128, 256, 384, 512, 768, 1024, 2048, 4096)
CHUNK_INT8_SIZES = (256, 512, 768, 1024, 2048)
for _n in BENCH_INT8_SIZES:
    _sig(f"benchmark_int8_matmul_{_n}", [])
_sig("kernel_main", [])
_sig("simp_rt_export_verify_all", [C.c_int32])
for _n in CHUNK_INT8_SIZES:
    _sig(f"int8_chunk_{_n}", [C.c_void_p, C.c_void_p, C.c_int64, C.c_int64, C.c_int64] * 3
         + [C.c_int64])


def benchmark_int8_matmul(n: int) -> int:
    """``benchmark_int8_matmul_<n>()`` of bench_int8_matmul.sl: the recipe
    inputs' s8 x s8 product, returned as the i32 wraparound checksum of C."""
    n0 = lib.simp_rt_error_count()
    r = getattr(lib, f"benchmark_int8_matmul_{n}")()
    if lib.simp_rt_error_count() != n0:
        raise SimpRTError(f"benchmark_int8_matmul_{n}", -1, last_error())
    return r


def kernel_main() -> int:
    """``kernel_main()`` of bench_int8_matmul.sl:337-339 (the runner's entry
    point): ``benchmark_int8_matmul_256()``."""
    n0 = lib.simp_rt_error_count()
    r = lib.kernel_main()
    if lib.simp_rt_error_count() != n0:
        raise SimpRTError("kernel_main", -1, last_error())
    return r


def int8_chunk(n: int, a, b, c, row_start: int) -> None:
    """``int8_chunk_<n>(A, B, C, row_start)`` of bench_int8_matmul_parallel.sl:
    rows [row_start, row_start + n/8) of C = A x B for flat n*n arrays."""
    fn = f"int8_chunk_{n}"
    _check(fn, getattr(lib, fn)(*desc1(a), *desc1(b), *desc1(c), row_start))


def forward_cache_clear() -> None:
    _check("simp_rt_forward_cache_clear", lib.simp_rt_forward_cache_clear())


def export_verify_all(on: bool) -> None:
    """Model-level exports: re-check every chunk of host weights on every call
    (True) or sample one chunk per array mid-sequence (False, the default)."""
    _check("simp_rt_export_verify_all", lib.simp_rt_export_verify_all(1 if on else 0))


def tensor_matvecmul_i8(a, b, c):
    """``tensor_matvecmul`` on i8: the same C = A x B, s8 x s8 -> i32."""
    return _gemm("simp_rt_tensor_matvecmul_i8", a, b, c)


def tensor_matmul_i4(a_packed, b_packed, c):
    """C[M,N] (int16) = A[M,K] x B[K,N] on packed signed nibbles: a_packed is
    [M,(K+1)/2] bytes packed along K, b_packed [K,(N+1)/2] packed along N (low
    nibble = even index); each sum is truncated to i16 (``tensor_matmul`` on i4)."""
    return _gemm("simp_rt_tensor_matmul_i4", a_packed, b_packed, c)


def matmul_u8s8_i32(a, b, c):
    """C = A(u8) x B(s8) -> i32, vpdpbusd semantics, B as [K,N]."""
    return _gemm("simp_rt_matmul_u8s8_i32", a, b, c)


def matmul_u8s8_i32_noalloc(a, b, c):
    """simp_rt_matmul_u8s8_i32_noalloc: the u8 x s8 -> i32 product with no
    device allocation (operands must be device-resident)."""
    return _gemm("simp_rt_matmul_u8s8_i32_noalloc", a, b, c)


def matmul_nt_u8s8_i32(a, bt, c):
    """C = A(u8) x B_T(s8)^T -> i32, vpdpbusd semantics, B as B_T[N,K]."""
    return _gemm("simp_rt_matmul_nt_u8s8_i32", a, bt, c)


def matmul_quant(qweights, scales, zeros, inp, out, rows, cols, group_size, offset=0):
    """``matmul_quant`` builtin (reference W4: unsigned nibbles, scale + zero per flat group)."""
    _check("simp_rt_matmul_quant",
           lib.simp_rt_matmul_quant(*desc1(qweights), *desc1(scales), *desc1(zeros),
                                    *desc1(inp), *desc1(out), rows, cols, group_size, offset))
    return out


def dequant_w4(qweights, scales, zeros, idx, group_size, out, count=None):
    """``dequant_w4`` builtin over a range: out[i] = the reference-format weight
    of flat element idx + i (unsigned nibble * scale + zero), i < count."""
    count = out.shape[0] if count is None else count
    _check("simp_rt_dequant_w4",
           lib.simp_rt_dequant_w4(*desc1(qweights), *desc1(scales), *desc1(zeros), idx,
                                  group_size, *desc1(out), count))
    return out


def matmul_w4s(w, scales, x, out, group_size=32):
    """out[M,N] = x[M,K] W^T, W[N,K/2] signed-nibble W4 with scales[N,K/gs]."""
    _check("simp_rt_matmul_w4s",
           lib.simp_rt_matmul_w4s(*desc2(w), *desc2(scales), *desc2(x), *desc2(out), group_size))
    return out


def matmul(lhs, rhs, out, m, k, n, lhs_offset=0, rhs_offset=0, output_offset=0):
    """``matmul`` builtin: out[m,n] += lhs[m,k] rhs[k,n] on 1-D arrays at element offsets."""
    _check("simp_rt_matmul_f32",
           lib.simp_rt_matmul_f32(*desc1(lhs), *desc1(rhs), *desc1(out), m, k, n,
                                  lhs_offset, rhs_offset, output_offset))
    return out


def tensor_matmul_f32(a, b, c):
    """``tensor_matmul`` on f32 tensors: C = A B."""
    _check("simp_rt_tensor_matmul_f32",
           lib.simp_rt_tensor_matmul_f32(*desc2(a), *desc2(b), *desc2(c)))
    return c


def tensor_matmul_nt_f32(a, bt, c):
    """C[M,N] = A[M,K] x B_T[N,K]^T in fp32 (``tensor_matmul_nt``), C overwritten."""
    _check("simp_rt_tensor_matmul_nt_f32",
           lib.simp_rt_tensor_matmul_nt_f32(*desc2(a), *desc2(bt), *desc2(c)))
    return c


def tensor_matvecmul_f32(a, b, c):
    """``tensor_matvecmul`` on f32: the same C = A x B as tensor_matmul_f32."""
    _check("simp_rt_tensor_matvecmul_f32",
           lib.simp_rt_tensor_matvecmul_f32(*desc2(a), *desc2(b), *desc2(c)))
    return c


def tensor_matmul_f64(a, b, c):
    """``tensor_matmul`` on f64 tensors: C = A B, C overwritten."""
    _check("simp_rt_tensor_matmul_f64",
           lib.simp_rt_tensor_matmul_f64(*desc2(a), *desc2(b), *desc2(c)))
    return c


_BATCH = {"float32": "f32", "float64": "f64", "int8": "i8"}


def tensor_batch_matmul(a, b, c):
    """Rank-3 ``tensor_matmul``: C[b] = A[b] x B[b] for A[Bt,M,K], B[Bt,K,N]
    (f32, f64, or s8 x s8 -> i32), C overwritten."""
    kind = _BATCH.get(str(a.dtype).replace("torch.", ""))
    if kind is None:
        raise TypeError(f"tensor_batch_matmul: unsupported dtype {a.dtype}")
    fn = f"simp_rt_tensor_batch_matmul_{kind}"
    _check(fn, getattr(lib, fn)(*descn(a, 3), *descn(b, 3), *descn(c, 3)))
    return c


def tensor_matmul_nhwc(x, w, y):
    """4-D x 2-D ``tensor_matmul``: y[n,h,w,o] = sum_i x[n,h,w,i] w[o,i] (f32 or f64)."""
    kind = _BATCH.get(str(x.dtype).replace("torch.", ""))
    if kind not in ("f32", "f64"):
        raise TypeError(f"tensor_matmul_nhwc: unsupported dtype {x.dtype}")
    fn = f"simp_rt_tensor_matmul_nhwc_{kind}"
    _check(fn, getattr(lib, fn)(*descn(x, 4), *desc2(w), *descn(y, 4)))
    return y


def rmsnorm(inp, weight, out, size, epsilon=1e-5, weight_offset=0):
    """``rmsnorm`` builtin."""
    _check("simp_rt_rmsnorm", lib.simp_rt_rmsnorm(*desc1(inp), *desc1(weight), *desc1(out),
                                                  size, epsilon, weight_offset))
    return out


def softmax(inp, out, size, input_offset=0, output_offset=0):
    """``softmax`` builtin."""
    _check("simp_rt_softmax", lib.simp_rt_softmax(*desc1(inp), *desc1(out), size,
                                                  input_offset, output_offset))
    return out


def silu(inp, out, size):
    """``silu`` builtin."""
    _check("simp_rt_silu", lib.simp_rt_silu(*desc1(inp), *desc1(out), size))
    return out


def swiglu(gate, up, out, size):
    """out = silu(gate) * up."""
    _check("simp_rt_swiglu", lib.simp_rt_swiglu(*desc1(gate), *desc1(up), *desc1(out), size))
    return out


def rope(q, k, dim, kv_dim, head_size, pos, theta=10000.0):
    """RoPE in place on q and k."""
    _check("simp_rt_rope", lib.simp_rt_rope(*desc1(q), *desc1(k), dim, kv_dim, head_size, pos,
                                            theta))
    return q, k


# ------------------------------------------------------------------ decode

W_F32, W_W4S = 0, 1
_CFG_INTS = ("dim", "hidden_dim", "n_layers", "n_heads", "n_kv_heads", "vocab_size", "seq_len")
_W_NAMES = ("token_embedding", "rms_att", "rms_ffn", "rms_final",
            "wq", "wk", "wv", "wo", "w1", "w2", "w3", "wcls",
            "q_wq", "q_wk", "q_wv", "q_wo", "q_w1", "q_w2", "q_w3", "q_wcls",
            "s_wq", "s_wk", "s_wv", "s_wo", "s_w1", "s_w2", "s_w3", "s_wcls")


class LlamaConfig(C.Structure):
    _fields_ = [(n, C.c_int64) for n in _CFG_INTS] + [
        ("eps", C.c_float), ("rope_theta", C.c_float),
        ("weight_format", C.c_int32), ("group_size", C.c_int32)]


class LlamaWeights(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in _W_NAMES]


class Llama:
    """Decode-step engine (simp_rt_llama_*) over device-resident weights.

    ``cfg``: dict with the keys of simp_rt_llama_config; ``weights``: dict of
    device tensors named as simp_rt_llama_weights (kept alive here)."""

    def __init__(self, cfg: dict, weights: dict):
        self.cfg = dict(cfg)
        self._w = dict(weights)
        c = LlamaConfig(**{k: int(cfg[k]) for k in _CFG_INTS},
                        eps=float(cfg.get("eps", 1e-5)),
                        rope_theta=float(cfg.get("rope_theta", 10000.0)),
                        weight_format=int(cfg.get("weight_format", W_F32)),
                        group_size=int(cfg.get("group_size", 32)))
        w = LlamaWeights(**{k: (v.data_ptr() if hasattr(v, "data_ptr") else v)
                            for k, v in weights.items()})
        h = C.c_void_p()
        _check("simp_rt_llama_create", lib.simp_rt_llama_create(C.byref(c), C.byref(w), C.byref(h)))
        self._h = h

    def forward(self, token: int, pos: int, logits):
        """One step; logits (device tensor or numpy float32[vocab]) receives the output."""
        p = logits.data_ptr() if hasattr(logits, "data_ptr") else logits.ctypes.data
        _check("simp_rt_llama_forward", lib.simp_rt_llama_forward(self._h, token, pos, p))
        return logits

    def generate(self, prompt, n_new: int, use_graph: bool = True):
        import numpy as np
        pr = np.ascontiguousarray(prompt, np.int32)
        out = np.zeros(len(pr) + n_new, np.int32)
        _check("simp_rt_llama_generate",
               lib.simp_rt_llama_generate(self._h, pr.ctypes.data, len(pr), n_new,
                                          out.ctypes.data, int(use_graph)))
        return out

    def close(self):
        if getattr(self, "_h", None):
            lib.simp_rt_llama_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ------------------------------------------------------------- model files

class CkptConfig(C.Structure):
    _fields_ = [(n, C.c_int32) for n in _CFG_INTS]


class W4UModel(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("token_embedding", "rms_att", "rms_ffn", "rms_final",
                                          "wcls", "scales", "zeros", "qweights")] + [
        (n, C.c_int64) for n in _CFG_INTS + ("group_size", "qweights_bytes", "n_groups")] + [
        ("offsets", C.c_int64 * 7)]


_sig("simp_rt_ckpt_read_config", [C.c_char_p, C.POINTER(CkptConfig)])
_sig("simp_rt_ckpt_load_f32", [C.c_char_p, C.POINTER(CkptConfig), C.POINTER(LlamaWeights),
                               C.POINTER(C.c_void_p)])
_sig("simp_rt_tokenizer_load", [C.c_char_p, C.c_int32, C.POINTER(C.c_void_p)])
lib.simp_rt_tokenizer_decode.argtypes = [C.c_void_p, C.c_int32, C.POINTER(C.c_int32)]
lib.simp_rt_tokenizer_decode.restype = C.POINTER(C.c_char)
lib.simp_rt_tokenizer_score.argtypes = [C.c_void_p, C.c_int32]
lib.simp_rt_tokenizer_score.restype = C.c_float
_sig("simp_rt_tokenizer_max_token_length", [C.c_void_p])
_sig("simp_rt_tokenizer_free", [C.c_void_p])
_sig("simp_rt_sampler_create", [C.c_uint32, C.POINTER(C.c_void_p)])
_sig("simp_rt_sampler_sample", [C.c_void_p, _P, C.c_int32, C.c_float])
_sig("simp_rt_sampler_free", [C.c_void_p])
_sig("simp_rt_quantize_w4u", [_P, _I, C.c_int32, _P, _P, _P])
_sig("simp_rt_quantize_w4s", [_P, _I, _I, C.c_int32, _P, _P])
_sig("simp_rt_w4s_file_write", [C.c_char_p, C.c_char_p, C.c_int32])
_sig("simp_rt_w4s_file_load", [C.c_char_p, C.POINTER(LlamaConfig), C.POINTER(LlamaWeights),
                               C.POINTER(C.c_void_p)])
_sig("simp_rt_w4u_file_write", [C.c_char_p, C.c_char_p, C.c_int32])
_sig("simp_rt_w4u_file_load", [C.c_char_p, C.POINTER(W4UModel), C.POINTER(C.c_void_p)])
_sig("simp_rt_free", [_P])
_sig("simp_rt_memcpy", [_P, _P, _I])


def _b(path) -> bytes:
    return os.fsencode(path)


def ckpt_read_config(path) -> dict:
    """llama2.c checkpoint header (generate_stories110M.cpp:143-150)."""
    c = CkptConfig()
    _check("simp_rt_ckpt_read_config", lib.simp_rt_ckpt_read_config(_b(path), C.byref(c)))
    return {k: int(getattr(c, k)) for k in _CFG_INTS}


class DeviceModel:
    """Weights loaded into one device allocation (freed by close()).

    ``cfg`` is the engine configuration (keys of simp_rt_llama_config) and
    ``weights`` maps simp_rt_llama_weights field names to device addresses,
    so ``Llama(m.cfg, m.weights)`` builds an engine over them."""

    def __init__(self, cfg: dict, weights: dict, blob):
        self.cfg, self.weights, self._blob = cfg, weights, blob

    def read(self, name: str, count: int, dtype="float32"):
        """Copies `count` elements of a loaded array to a numpy array."""
        import numpy as np
        out = np.empty(count, dtype)
        if count:
            _check("simp_rt_memcpy", lib.simp_rt_memcpy(out.ctypes.data, self.weights[name], out.nbytes))
        return out

    def close(self):
        if getattr(self, "_blob", None):
            lib.simp_rt_free(self._blob)
            self._blob = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def ckpt_load_f32(path) -> DeviceModel:
    """The whole fp32 checkpoint on the device (generate_stories110M.cpp:150-191)."""
    c, w, blob = CkptConfig(), LlamaWeights(), C.c_void_p()
    _check("simp_rt_ckpt_load_f32", lib.simp_rt_ckpt_load_f32(_b(path), C.byref(c), C.byref(w),
                                                              C.byref(blob)))
    cfg = {k: abs(int(getattr(c, k))) for k in _CFG_INTS}
    cfg.update(eps=1e-5, rope_theta=10000.0, weight_format=W_F32, group_size=32)
    weights = {k: getattr(w, k) for k in _W_NAMES[:12]}
    return DeviceModel(cfg, weights, blob)


def w4s_file_write(ckpt_path, out_path, group_size: int = 32) -> None:
    _check("simp_rt_w4s_file_write", lib.simp_rt_w4s_file_write(_b(ckpt_path), _b(out_path), group_size))


def w4s_file_load(path) -> DeviceModel:
    c, w, blob = LlamaConfig(), LlamaWeights(), C.c_void_p()
    _check("simp_rt_w4s_file_load", lib.simp_rt_w4s_file_load(_b(path), C.byref(c), C.byref(w),
                                                              C.byref(blob)))
    cfg = {k: int(getattr(c, k)) for k in _CFG_INTS}
    cfg.update(eps=float(c.eps), rope_theta=float(c.rope_theta),
               weight_format=int(c.weight_format), group_size=int(c.group_size))
    weights = {k: getattr(w, k) for k in ("token_embedding", "rms_att", "rms_ffn", "rms_final")
               + _W_NAMES[12:]}
    return DeviceModel(cfg, weights, blob)


def w4u_file_write(ckpt_path, out_path, group_size: int = 128) -> None:
    _check("simp_rt_w4u_file_write", lib.simp_rt_w4u_file_write(_b(ckpt_path), _b(out_path), group_size))


def w4u_file_load(path) -> DeviceModel:
    """Arrays of llama2_quant_forward on the device; cfg also holds the sizes
    and the seven element offsets."""
    m, blob = W4UModel(), C.c_void_p()
    _check("simp_rt_w4u_file_load", lib.simp_rt_w4u_file_load(_b(path), C.byref(m), C.byref(blob)))
    cfg = {k: int(getattr(m, k)) for k in _CFG_INTS + ("group_size", "qweights_bytes", "n_groups")}
    cfg["offsets"] = [int(v) for v in m.offsets]
    weights = {k: getattr(m, k) for k in ("token_embedding", "rms_att", "rms_ffn", "rms_final", "wcls",
                                          "scales", "zeros", "qweights")}
    return DeviceModel(cfg, weights, blob)


class Tokenizer:
    """Tokenizer file of generate_stories110M.cpp:36-70."""

    def __init__(self, path, vocab_size: int):
        h = C.c_void_p()
        _check("simp_rt_tokenizer_load", lib.simp_rt_tokenizer_load(_b(path), vocab_size, C.byref(h)))
        self._h = h

    def decode(self, token: int) -> bytes:
        n = C.c_int32()
        p = lib.simp_rt_tokenizer_decode(self._h, token, C.byref(n))
        return C.string_at(p, n.value)

    def score(self, token: int) -> float:
        return float(lib.simp_rt_tokenizer_score(self._h, token))

    @property
    def max_token_length(self) -> int:
        return int(lib.simp_rt_tokenizer_max_token_length(self._h))

    def close(self):
        if getattr(self, "_h", None):
            lib.simp_rt_tokenizer_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Sampler:
    """Token sampling of generate_stories110M.cpp:73-116 with a seeded std::mt19937."""

    def __init__(self, seed: int):
        h = C.c_void_p()
        _check("simp_rt_sampler_create", lib.simp_rt_sampler_create(seed & 0xFFFFFFFF, C.byref(h)))
        self._h = h

    def sample(self, logits, temperature: float) -> int:
        import numpy as np
        lg = np.ascontiguousarray(logits, np.float32)
        r = lib.simp_rt_sampler_sample(self._h, lg.ctypes.data, lg.size, C.c_float(temperature))
        if r < 0:
            _check("simp_rt_sampler_sample", r)
        return int(r)

    def close(self):
        if getattr(self, "_h", None):
            lib.simp_rt_sampler_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def quantize_w4u(w, group_size, q, scales, zeros) -> None:
    """Reference quantize_w4 (bench_llama_quant.cpp:51-93) of a device tensor."""
    _check("simp_rt_quantize_w4u", lib.simp_rt_quantize_w4u(w.data_ptr(), w.numel(), group_size,
                                                            q.data_ptr(), scales.data_ptr(),
                                                            zeros.data_ptr()))


def quantize_w4s(w, group_size, q, scales) -> None:
    """Symmetric W4 of a device matrix w [rows, cols]."""
    rows, cols = w.shape
    _check("simp_rt_quantize_w4s", lib.simp_rt_quantize_w4s(w.data_ptr(), rows, cols, group_size,
                                                            q.data_ptr(), scales.data_ptr()))
