"""simplang_amd -- MI355X (gfx950) runtime for the tensor ops SimpLang lowers into.

The product is ``libsimp_hip.so`` (C ABI declared in ``include/simp_rt.h``).
This package is the host-side mirror of the reference's operator interface:
each function takes the same operands, in the same order, as the SimpLang
builtin it replaces (``src/mlir/mlir_codegen.cpp:1388-1531,2068-2292``) and
calls the C ABI with expanded memref descriptors.  There is no CPU fallback:
if the library is missing or fails, these functions raise.
"""
from .host import (  # noqa: F401
    SimpRTError,
    lib,
    lib_path,
    set_stream,
    sync,
    timing,
    timing_query,
    tensor_matmul_i8,
    tensor_matmul_nt_i8,
    tensor_matmul_i4,
    tensor_matvecmul_i8,
    matmul_u8s8_i32,
    matmul_nt_u8s8_i32,
    matmul_quant,
    matmul_w4s,
    matmul,
    tensor_matmul_f32,
    tensor_matmul_nt_f32,
    tensor_matvecmul_f32,
    tensor_matmul_f64,
    tensor_batch_matmul,
    tensor_matmul_nhwc,
    rmsnorm,
    softmax,
    silu,
    swiglu,
    rope,
    Llama,
    stories110M_forward,
    llama2_quant_forward,
    llama32_forward,
    Llama32Program,
    forward_cache_clear,
    W_F32,
    W_W4S,
    ckpt_read_config,
    ckpt_load_f32,
    DeviceModel,
    Tokenizer,
    Sampler,
    quantize_w4u,
    quantize_w4s,
    w4s_file_write,
    w4s_file_load,
    w4u_file_write,
    w4u_file_load,
)
