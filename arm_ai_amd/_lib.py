"""ctypes binding of libarm_ai_amd.so (the extern "C" ABI in include/aq.h).

The library is loaded from the package directory (built in-tree by
``python -m arm_ai_amd.build``).  There is no CPU fallback: if the library is
missing, every entry point raises.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libarm_ai_amd.so")

AQ_OK = 0
AQ_ERR_INVALID_ARG = -1
AQ_ERR_UNSUPPORTED_TYPE = -2
AQ_ERR_SHAPE = -3
AQ_ERR_NO_DEVICE = -4
AQ_ERR_HIP = -5
AQ_ERR_OOM = -6

STATUS_NAMES = {
    AQ_OK: "AQ_OK",
    AQ_ERR_INVALID_ARG: "AQ_ERR_INVALID_ARG",
    AQ_ERR_UNSUPPORTED_TYPE: "AQ_ERR_UNSUPPORTED_TYPE",
    AQ_ERR_SHAPE: "AQ_ERR_SHAPE",
    AQ_ERR_NO_DEVICE: "AQ_ERR_NO_DEVICE",
    AQ_ERR_HIP: "AQ_ERR_HIP",
    AQ_ERR_OOM: "AQ_ERR_OOM",
}

P = ctypes.c_void_p
I64 = ctypes.c_int64
INT = ctypes.c_int
SZ = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/aq.h exactly
SIGNATURES = {
    "aq_abi_version": (INT, []),
    "aq_last_error": (ctypes.c_char_p, []),
    "aq_device_count": (INT, [ctypes.POINTER(INT)]),
    "aq_ctx_create": (INT, [INT, ctypes.POINTER(P)]),
    "aq_ctx_destroy": (INT, [P]),
    "aq_ctx_synchronize": (INT, [P]),
    "aq_ctx_stream": (INT, [P, ctypes.POINTER(P)]),
    "aq_qweight_upload": (INT, [P, INT, P, SZ, I64, I64, ctypes.POINTER(P)]),
    "aq_qweight_upload_device": (INT, [P, INT, P, SZ, I64, I64, ctypes.POINTER(P)]),
    "aq_qweight_free": (INT, [P]),
    "aq_qweight_info": (INT, [P, ctypes.POINTER(INT), ctypes.POINTER(I64), ctypes.POINTER(I64), ctypes.POINTER(SZ)]),
    "aq_qmatmul_f32": (INT, [P, P, P, I64, I64, P]),
    "aq_qmatmul_f32_device": (INT, [P, P, P, I64, I64, P]),
    "aq_qmatmul_f32_device_noalloc": (INT, [P, P, P, I64, I64, P]),
    "aq_fixed_scratch_bytes": (SZ, []),
    "aq_act_bytes": (SZ, [INT, I64, I64]),
    "aq_quantize_act_device": (INT, [P, INT, P, I64, I64, P]),
    "aq_qmatmul_preq_device": (INT, [P, P, P, I64, I64, P]),
    "aq_qmatmul2_preq_device": (INT, [P, P, P, P, I64, I64, P, P]),
    "aq_quantize_q8k": (INT, [P, P, I64, I64, P]),
    "aq_quantize_q8_0": (INT, [P, P, I64, I64, P]),
    "aq_qmatmul_block_sums": (INT, [P, P, P, I64, I64, P, P]),
    # crate kernels (shape_ops.rs)
    "aq_int8_matmul_f32": (INT, [P, P, P, P, ctypes.c_float, I64, I64, I64, P]),
    "aq_int8_matmul_f32_per_token": (INT, [P, P, P, P, P, I64, I64, I64, P]),
    "aq_int8_matmul_f32_device": (INT, [P, P, P, P, ctypes.c_float, P, I64, I64, I64, P]),
    "aq_quantize_int8_per_token": (INT, [P, P, I64, I64, P, P]),
    "aq_quantize_int8_per_token_device": (INT, [P, P, I64, I64, P, P]),
    "aq_dequant_matmul_int8_f32": (INT, [P, P, P, P, I64, I64, I64, I64, P]),
    "aq_dequant_matmul_f16_f32": (INT, [P, P, P, I64, I64, I64, I64, P]),
    "aq_int4_matmul_f32": (INT, [P, P, P, P, I64, I64, I64, P]),
    "aq_int4_matmul_gemv": (INT, [P, P, P, P, I64, I64, P]),
    "aq_weight_only_matmul_device": (INT, [P, INT, P, P, P, I64, I64, I64, P]),
    "aq_int4_matmul_gemv_q4_x_q8": (INT, [P, P, P, P, I64, I64, P]),
    "aq_q4_x_q8_act_bytes": (SZ, [I64]),
    "aq_int4_matmul_gemv_q4_x_q8_device": (INT, [P, P, P, P, I64, I64, P, P, P, P]),
    "aq_quantize_int4_q4_0": (INT, [P, P, I64, I64, P, P]),
    "aq_dequantize_q6_k": (INT, [P, P, SZ, I64, P]),
    "aq_dequantize_q6_k_device": (INT, [P, P, I64, P]),
    "aq_q4_0_dequant_row": (INT, [P, P, P, I64, I64, I64, P]),
    "aq_q8_0_dequant_row": (INT, [P, P, P, I64, I64, I64, P]),
    "aq_dequant_rows_device": (INT, [P, INT, P, P, I64, P, I64, I64, P]),
    # decode-step glue (k_decode.hip)
    "aq_llama_embed": (INT, [P, P, I64, P, I64, P]),
    "aq_llama_rmsnorm": (INT, [P, P, P, P, I64, I64, ctypes.c_float, P]),
    "aq_llama_silu_mul": (INT, [P, P, I64, P]),
    "aq_llama_embed_rows": (INT, [P, P, I64, P, I64, I64, P]),
    "aq_llama_silu_mul_rows": (INT, [P, P, P, I64, I64, I64, P]),
    "aq_llama_attn_decode": (INT, [P, P, P, P, P, P, P, P, I64, I64, I64, I64, P]),
    "aq_llama_attn_prefill": (INT, [P, P, I64, P, I64, P, I64, P, P, I64, I64, P, P, I64, I64, I64, I64, P]),
    "aq_llama_argmax": (INT, [P, P, I64, P, P, P, I64]),
    "aq_qmatmul_rmsnorm_f32_device": (INT, [P, P, P, P, P, ctypes.c_float, I64, P, P]),
    "aq_qmatmul_silu_mul_f32_device": (INT, [P, P, P, I64, P]),
    "aq_qmatmul2_rmsnorm_f32_device": (INT, [P, P, P, P, P, P, ctypes.c_float, I64, P, P, P]),
    "aq_llama_swiglu_pairs": (INT, [P, P, I64, I64, I64, P]),
    "aq_llama_rmsnorm_act": (INT, [P, P, P, P, I64, I64, ctypes.c_float, P, P]),
    "aq_llama_swiglu_pairs_act": (INT, [P, P, I64, I64, I64, P, P]),
    "aq_swiglu_fused": (INT, [INT, I64, I64]),
    "aq_llama_head_argmax_embed": (INT, [P, P, P, P, P, ctypes.c_float, I64, P, P, P, P, I64, P, I64, P]),
    "aq_qmatmul_rmsnorm_swiglu_f32_device": (INT, [P, P, P, P, P, ctypes.c_float, I64, P, P]),
}


class AqError(RuntimeError):
    """A non-zero aq_status, with the library's message."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"{STATUS_NAMES.get(code, code)}: {msg}")
        self.code = code


_lib = None


def load() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is not built; run `python -m arm_ai_amd.build` (there is no CPU fallback)"
            )
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def check(rc: int) -> None:
    if rc != AQ_OK:
        msg = load().aq_last_error()
        raise AqError(rc, msg.decode() if msg else "")
