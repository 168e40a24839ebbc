"""ctypes binding of libovfq.so (include/ovfq.h).

The library is the only compute path: there is no CPU fallback. Loading fails loudly when the built library
is missing (build it with ``python -c "import __graft_entry__ as g; g.build()"``).
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libovfq.so")

OVFQ_OK = 0
OVFQ_ERR_NULL = -1
OVFQ_ERR_SIZE = -2
OVFQ_ERR_RANGE = -3
OVFQ_ERR_TYPE = -4
OVFQ_ERR_STATE = -5
OVFQ_ERR_HIP = -10
OVFQ_FFN_SWIGLU = 3
OVFQ_FFN_GEGLU = 4

TYPE_Q8_0 = 8
TYPE_Q4_K = 12
TYPE_Q6_K = 14
TYPE_Q5_0 = 6
TYPE_Q5_K = 13

vp = ctypes.c_void_p
ci = ctypes.c_int
sz = ctypes.c_size_t
PP = ctypes.POINTER(ctypes.c_void_p)

# name -> (restype, argtypes). Every symbol include/ovfq.h declares.
SIGNATURES = {
    "ovfq_ctx_create": (ci, [ci, PP]),
    "ovfq_ctx_destroy": (ci, [vp]),
    "ovfq_ctx_set_stream": (ci, [vp, vp]),
    "ovfq_ctx_reset_stream": (ci, [vp]),
    "ovfq_ctx_synchronize": (ci, [vp]),
    "ovfq_ctx_release_retired": (ci, [vp]),
    "ovfq_ctx_scratch_bytes": (ci, [vp, ctypes.POINTER(sz), ctypes.POINTER(sz)]),
    "ovfq_ctx_set_batched_kernel": (ci, [vp, ci]),
    "ovfq_last_error": (ctypes.c_char_p, []),
    "ovfq_version": (ctypes.c_char_p, []),
    "ovfq_weight_create": (ci, [vp, ci, vp, sz, vp, ci, ci, PP]),
    "ovfq_weight_create_from_device": (ci, [vp, ci, vp, sz, vp, ci, ci, PP]),
    "ovfq_weight_destroy": (ci, [vp]),
    "ovfq_weight_prepare_mfma": (ci, [vp, vp]),
    "ovfq_weight_info": (ci, [vp, ctypes.POINTER(ci), ctypes.POINTER(ci), ctypes.POINTER(ci),
                              ctypes.POINTER(sz), PP]),
    "ovfq_weight_decode_row": (ci, [vp, vp, ci, vp]),
    "ovfq_weight_decode_row_dev": (ci, [vp, vp, ci, vp]),
    "ovfq_quantize_q8k": (ci, [vp, vp, ci, ci, vp, vp, vp]),
    "ovfq_quantize_q8k_dev": (ci, [vp, vp, ci, ci, vp, vp, vp]),
    "ovfq_quantize_q8_0": (ci, [vp, vp, ci, ci, vp, vp]),
    "ovfq_quantize_q8_0_dev": (ci, [vp, vp, ci, ci, vp, vp]),
    "ovfq_project": (ci, [vp, vp, vp, ci, vp, vp]),
    "ovfq_project_dev": (ci, [vp, vp, vp, ci, vp, vp]),
    "ovfq_project_noalloc_dev": (ci, [vp, vp, vp, ci, vp, vp]),
    "ovfq_project_prequantized": (ci, [vp, vp, vp, vp, vp, ci, vp, vp]),
    "ovfq_project_prequantized_dev": (ci, [vp, vp, vp, vp, vp, ci, vp, vp]),
    "ovfq_project_gate_up": (ci, [vp, vp, vp, vp, vp, vp]),
    "ovfq_weight_create_gguf": (ci, [vp, ci, vp, ctypes.c_size_t, ci, ci, ctypes.POINTER(vp)]),
    "ovfq_weight_create_gguf_dev": (ci, [vp, ci, vp, ctypes.c_size_t, ci, ci, ctypes.POINTER(vp)]),
    "ovfq_weight_create_experts_gguf": (ci, [vp, ci, vp, ctypes.c_size_t, ci, ci, ci, ctypes.POINTER(vp)]),
    "ovfq_weight_create_experts_gguf_dev": (ci, [vp, ci, vp, ctypes.c_size_t, ci, ci, ci, ctypes.POINTER(vp)]),
    "ovfq_ffn_swiglu": (ci, [vp, vp, vp, vp, vp, ci, vp]),
    "ovfq_ffn_swiglu_dev": (ci, [vp, vp, vp, vp, vp, ci, vp]),
    "ovfq_ffn_gated": (ci, [vp, vp, vp, vp, vp, ci, ci, vp]),
    "ovfq_ffn_gated_dev": (ci, [vp, vp, vp, vp, vp, ci, ci, vp]),
    "ovfq_moe_select_topk": (ci, [vp, vp, ci, ci, ci, ci, vp, vp]),
    "ovfq_moe_select_topk_dev": (ci, [vp, vp, ci, ci, ci, ci, vp, vp]),
    "ovfq_moe_ffn": (ci, [vp, ci, PP, PP, PP, vp, ci, ci, vp, vp, vp]),
    "ovfq_moe_ffn_dev": (ci, [vp, ci, PP, PP, PP, vp, ci, ci, vp, vp, vp]),
    "ovfq_moe_ffn_routed": (ci, [vp, ci, PP, PP, PP, vp, ci, vp, ci, ci, vp, vp, vp]),
    "ovfq_moe_ffn_routed_dev": (ci, [vp, ci, PP, PP, PP, vp, ci, vp, ci, ci, vp, vp, vp]),
    "ovfq_project_gate_up_dev": (ci, [vp, vp, vp, vp, vp, vp]),
    "ovfq_project_multi": (ci, [vp, ci, PP, vp, ci, PP, PP]),
    "ovfq_project_multi_dev": (ci, [vp, ci, PP, vp, ci, PP, PP]),
    "ovfq_project_heads_q8_0": (ci, [vp, ci, PP, vp, ci, vp, vp]),
    "ovfq_project_heads_q8_0_dev": (ci, [vp, ci, PP, vp, ci, vp, vp]),
    "ovfq_project_multi_prequantized_dev": (ci, [vp, ci, PP, vp, vp, vp, ci, PP, PP]),
    "ovfq_quantize_weight_q4k_dev": (ci, [vp, vp, ci, ci, vp]),
    "ovfq_quantize_weight_q6k_dev": (ci, [vp, vp, ci, ci, vp]),
    "ovfq_quantize_weight_q8_0_dev": (ci, [vp, vp, ci, ci, vp, vp]),
}

_lib = None


def load():
    """Load libovfq.so and declare its signatures. Raises if the library has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"libovfq.so not found at {LIB_PATH}: the HIP library must be built "
                "(python -c 'import __graft_entry__ as g; g.build()'); there is no CPU fallback")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def declared_symbols(header_path=None):
    """Names of the functions include/ovfq.h declares (parsed from the header)."""
    import re

    if header_path is None:
        header_path = os.path.join(os.path.dirname(HERE), "include", "ovfq.h")
    text = open(header_path).read()
    return sorted(set(re.findall(r"OVFQ_API\s+[\w\s\*]+?\b(ovfq_\w+)\s*\(", text)))
