"""ctypes binding of ``libecdecode.so`` (the C ABI declared in ``include/ecdecode.h``).

The library is built in-tree by ``estudiocanciones_amd.build``; if it is missing, every
call fails loudly -- there is no CPU or eager-PyTorch fallback for the decode path.
"""
from __future__ import annotations

import ctypes
from ctypes import c_double, c_float, c_int, c_long, c_void_p
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libecdecode.so"

ECD_OK = 0
ECD_EINVAL = -22
ECD_ENOTSUP = -95
ECD_ENOMEM = -12

_P = c_void_p
# name -> argtypes, in the order of include/ecdecode.h
SIGNATURES = {
    "ecd_gemv_i8": [_P, c_long, _P, _P, _P, c_long, _P, c_long, c_int, c_int, c_int, c_int, _P],
    "ecd_gemv_i8_tuned": [_P, c_long, _P, _P, _P, c_long, _P, c_long, c_int, c_int, c_int, c_int,
                          c_int, c_int, _P],
    "ecd_rmsnorm": [_P, c_long, _P, _P, c_long, c_int, c_int, c_float, _P],
    "ecd_rope_kv_write": [_P, _P, _P, _P, _P, _P, c_int, c_int, c_int, c_int, c_int, c_int, _P],
    "ecd_decode_attn": [_P, _P, _P, _P, _P, _P, _P, _P, c_int, c_int, c_int, c_int, c_int, c_int,
                        c_int, c_float, _P],
    "ecd_attn_combine": [_P, _P, _P, _P, c_int, c_int, c_int, _P],
    "ecd_decode_attn_noalloc": [_P, _P, _P, _P, _P, c_int, c_int, c_int, c_int, c_int, c_int, c_int,
                                c_float, _P],
    "ecd_decode_attn_merged": [_P, _P, _P, _P, _P, _P, _P, c_int, c_int, c_int, c_int, c_int,
                               c_int, c_int, c_float, _P],
    "ecd_silu_mul": [_P, _P, c_int, c_int, _P],
    "ecd_embed_sum_i8": [_P, _P, _P, c_long, _P, c_int, c_int, c_int, c_int, _P],
    "ecd_embed_i8": [_P, c_long, _P, _P, c_long, c_int, c_int, _P, _P, c_int, c_int, _P],
    "ecd_quantize_rows_i8": [_P, _P, _P, _P, c_int, c_int, _P],
    "ecd_rope_table": [_P, c_int, c_int, c_double, c_double, c_double, c_double, c_double, _P],
    "ecd_sample_topk": [_P, c_long, c_int, c_int, c_float, c_float, c_int, c_int, _P, _P, _P, c_int,
                        _P, c_long, _P],
    "ecd_sample_topk_next": [_P, c_long, c_int, c_int, c_float, c_float, c_int, c_int, _P, _P, _P,
                             c_int, _P, c_long, _P, c_long, c_int, _P, c_long, c_int, _P, c_long,
                             c_int, _P, _P, c_int, c_int, _P, c_long, c_int, c_int, c_int, _P,
                             c_long, _P, c_long, _P],
    "ecd_frame_advance": [_P, c_long, _P, c_long, _P, c_long, _P, _P, c_int, c_int, c_int, c_int,
                          c_long, _P],
    "ecd_copy_bytes": [_P, _P, c_long, _P],
    "ecd_codec_rope_table": [_P, c_int, c_int, _P],
    "ecd_codec_rope_heads": [_P, c_long, _P, _P, _P, _P, c_int, c_int, c_int, c_int, _P],
    "ecd_gemm_f16p_rope": [_P, c_long, _P, _P, _P, _P, _P, _P, c_int, c_int, c_int, c_int, c_int,
                           _P],
    "ecd_codec_norm_mod": [_P, _P, _P, _P, c_long, _P, _P, _P, _P, _P, c_long, _P, c_int, c_int,
                           c_int, c_int, c_float, _P],
    "ecd_codec_cols3": [_P, _P, _P, _P, _P, _P, c_int, _P, c_int, c_int, _P],
    "ecd_codec_vq_embed": [_P, c_long, c_long, _P, _P, c_int, c_int, c_int, c_int, c_int, c_int,
                           c_int, _P],
    "ecd_codec_cols_taps": [_P, c_long, _P, c_int, _P, c_int, c_int, c_int, c_int, c_int, c_long,
                            c_long, _P],
    "ecd_codec_weight_norm": [_P, _P, _P, c_int, c_int, _P],
    "ecd_codec_latent_split": [_P, _P, c_int, c_int, c_int, _P],
    "ecd_codec_timestep": [_P, _P, c_int, _P],
    "ecd_codec_silu": [_P, _P, c_long, _P],
    "ecd_codec_euler": [_P, _P, _P, _P, c_int, c_int, c_int, c_int, c_int, c_float, c_float,
                        c_float, c_int, _P],
    "ecd_gemv_i8p_splitk": [_P, c_long, _P, _P, _P, c_long, _P, c_long, c_int, c_int, c_int, c_int,
                            _P, c_int, _P],
    "ecd_gemm_i8p": [_P, c_long, _P, _P, _P, c_long, _P, c_long, c_int, c_int, c_int, _P],
    "ecd_gemm_i8p_silu": [_P, c_long, _P, _P, _P, c_long, c_int, c_int, c_int, _P],
    "ecd_gemm_i8p_rope": [_P, c_long, _P, _P, _P, _P, _P, _P, _P, c_int, c_int, c_int, c_int,
                          c_int, c_int, c_int, _P],
    "ecd_prefill_attn": [_P, _P, _P, _P, _P, c_int, c_int, c_int, c_int, c_int, c_int, c_float, _P],
    "ecd_pack_f16": [_P, c_int, c_int, c_int, _P, _P],
    "ecd_gemm_f16p": [_P, c_long, _P, _P, c_float, _P, c_long, _P, c_long, c_int, c_int, c_int, _P],
    "ecd_gemm_f16p_silu": [_P, c_long, _P, _P, c_long, c_int, c_int, c_int, _P],
    "ecd_gemm_f16p_prelu": [_P, c_long, _P, _P, c_float, _P, c_long, _P, c_long, c_int, c_int,
                            c_int, _P],
    "ecd_gemm_f16p_conv": [_P, c_long, _P, _P, c_float, _P, c_long, _P, c_long, c_int, c_int,
                           c_int, c_int, c_int, c_int, _P, c_int, c_int, c_int, _P],
    "ecd_gemm_f16p_conv_tuned": [_P, c_long, _P, _P, c_float, _P, c_long, _P, c_long, c_int, c_int,
                                 c_int, c_int, c_int, c_int, _P, c_int, c_int, c_int, c_int, _P],
    "ecd_gemm_f16p_tuned": [_P, c_long, _P, _P, c_float, _P, c_long, _P, c_long, c_int, c_int,
                            c_int, c_int, c_int, _P],
    "ecd_packed_bytes": [c_int, c_int],
    "ecd_packed_bytes_f16": [c_int, c_int],
    "ecd_pack_i8": [_P, c_int, c_int, c_int, _P, _P],
    "ecd_gemv_i8p": [_P, c_long, _P, _P, _P, c_long, _P, c_long, c_int, c_int, c_int, c_int, c_int,
                     c_int, _P],
    "ecd_rms_gemv_i8p": [_P, c_long, _P, c_float, _P, _P, _P, c_long, c_int, c_int, c_int, c_int, _P],
    "ecd_rms_qkv_rope": [_P, c_long, _P, c_float, _P, _P, _P, _P, _P, _P, _P, c_int, c_int, c_int,
                         c_int, c_int, c_int, c_int, c_int, _P],
    "ecd_rms_w13_silu": [_P, c_long, _P, c_float, _P, _P, _P, c_int, c_int, c_int, c_int, _P],
    "ecd_embed_gemv_i8p": [_P, c_long, _P, _P, c_long, c_int, c_int, _P, _P, _P, _P, c_long, c_int,
                           c_int, c_int, c_int, _P],
    "ecd_layer_tail": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                       _P, _P, _P, _P, _P, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int,
                       c_float, c_int, _P],
    "ecd_layer_head": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, c_int, c_int, c_int,
                       c_int, c_int, c_int, c_int, c_int, c_float, c_int, _P],
    "ecd_layer_tail_supported": [c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int],
    "ecd_layer_tail_ws_bytes": [c_int, c_int, c_int, c_int],
    "ecd_layer_stack_plan": [_P, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int, _P, _P],
    "ecd_layer_stack_plan_bytes": [c_int],
    "ecd_layer_stack_supported": [c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int],
    "ecd_layer_stack_layers_per_launch": [c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int,
                                          c_int],
    "ecd_layer_stack": [_P, c_int, _P, _P, _P, _P, _P, _P, _P, _P, c_int, c_int, c_int, c_int,
                        c_int, c_int, c_int, c_int, c_int, c_int, c_float, c_int, _P],
}

_lib = None


class ECDError(RuntimeError):
    pass


def lib() -> ctypes.CDLL:
    """Load the library once and declare every entry point's signature."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ECDError(
                f"{LIB_PATH} is not built; run `python -m estudiocanciones_amd.build` "
                "(the decode path has no fallback)")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, argtypes in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = argtypes
            fn.restype = c_long if name.startswith("ecd_packed_bytes") or \
                name in ("ecd_layer_tail_ws_bytes", "ecd_layer_stack_plan_bytes") else c_int
        handle.ecd_version.argtypes = []
        handle.ecd_version.restype = ctypes.c_char_p
        _lib = handle
    return _lib


def check(rc: int, name: str) -> None:
    if rc == ECD_OK:
        return
    if rc == ECD_EINVAL:
        raise ValueError(f"{name}: invalid argument")
    if rc == ECD_ENOTSUP:
        raise NotImplementedError(f"{name}: shape not supported by the gfx950 kernels")
    if rc == ECD_ENOMEM:
        raise MemoryError(f"{name}: the call needs more than the library's static workspace")
    raise ECDError(f"{name}: HIP launch failed (hipError_t {rc})")


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args), name)
