"""overfit_amd — MI355X (gfx950) GGUF quantized-linear path for Overfit.

Q4_K / Q6_K / Q8_0 block-dequantize-and-dot projections as hand-written HIP kernels behind a C ABI
(include/ovfq.h, libovfq.so), with a host-side mirror of the reference's kernel classes.
"""
from . import _lib
from .errors import (OverfitArgumentError, OverfitArgumentNullError, OverfitArgumentOutOfRangeError,
                     OverfitHipError, OverfitInvalidOperationError, OverfitUnsupportedTypeError)
from .kernels import (BatchedQuantProjection, FeedForwardActivation, MoeRouter, Q4KDotKernel, Q6KDotKernel,
                      Q8DotKernel, ffn_gated, ffn_swiglu, moe_ffn, moe_ffn_routed, project, project_gate_up, project_heads_q8_0,
                      project_multi, quantize_weight)
from .runtime import Context, default_context
from .weights import DecodeWeight, Q4KWeight, Q6KWeight, Q8Weight, load_gguf_experts, load_gguf_tensor

TYPE_Q8_0 = _lib.TYPE_Q8_0
TYPE_Q4_K = _lib.TYPE_Q4_K
TYPE_Q6_K = _lib.TYPE_Q6_K

__all__ = [
    "BatchedQuantProjection", "Context", "DecodeWeight", "FeedForwardActivation", "MoeRouter", "OverfitArgumentError",
    "OverfitArgumentNullError", "OverfitArgumentOutOfRangeError", "OverfitHipError", "OverfitInvalidOperationError",
    "OverfitUnsupportedTypeError",
    "Q4KDotKernel", "Q4KWeight", "Q6KDotKernel", "Q6KWeight", "Q8DotKernel", "Q8Weight", "TYPE_Q4_K", "TYPE_Q6_K",
    "TYPE_Q8_0", "default_context", "ffn_gated", "ffn_swiglu", "load_gguf_experts", "load_gguf_tensor", "moe_ffn", "moe_ffn_routed", "project",
    "project_gate_up", "project_heads_q8_0", "project_multi", "quantize_weight",
]
