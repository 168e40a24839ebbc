"""Host-side mirror of Overfit's quantized-projection kernels, backed by the HIP library.

Same class and method names, argument meaning and argument checks as the reference's static kernels:
  Q4KDotKernel  RT/Q4KDotKernel.cs   (QuantizeActivationQ8K, Dot, Project, ProjectPreQuantized,
                                      ProjectParallel, ProjectGateUpParallel, ProjectBatched,
                                      ProjectBatchedWeightStationary)
  Q6KDotKernel  RT/Q6KDotKernel.cs   (the same minus gate/up and weight-stationary)
  Q8DotKernel   RT/Q8DotKernel.cs    (Quantize, Dot, Project, ProjectParallel, ProjectBatched)
  BatchedQuantProjection.Dispatch    RT/BatchedQuantProjection.cs:26-87
  MoeRouter.SelectTopK               RT/MoeRouter.cs:40-128 (plus moe_ffn: MoeFeedForwardBlock.DecodeBatched
                                     after routing, RT/MoeFeedForwardBlock.cs:140-241)

Spans become numpy arrays (host memory, synchronous) or torch GPU tensors (device memory, asynchronous on
the context stream). An empty or None bias means "no bias". Outputs and the caller-owned activation scratch
are overwritten exactly as the reference overwrites them. On the GPU there is one projection path, so
ProjectParallel == Project and ProjectBatchedWeightStationary == ProjectBatched (bit-identical, as the
reference requires of its variants).
"""
import ctypes

import enum

import numpy as np

from . import _lib
from .errors import (OverfitArgumentError, OverfitArgumentNullError, OverfitArgumentOutOfRangeError,
                     OverfitUnsupportedTypeError, raise_for_status)
from .runtime import as_buf, default_context, is_empty, same_side
from .weights import DecodeWeight, Q4KWeight, Q6KWeight, Q8Weight


def _validate_project_arguments(inp, bias, out, input_size, output_size):
    # RT/Q4KDotKernel.cs:957-976
    if inp.size < input_size:
        raise OverfitArgumentError("Input span is smaller than the weight's input size.")
    if out.size < output_size:
        raise OverfitArgumentError("Output span is smaller than the weight's output size.")
    if not is_empty(bias) and bias.size < output_size:
        raise OverfitArgumentError("Bias span is smaller than outputSize.")


def _quantize_q8k(ctx, src, q, s, b, rows, k):
    lib = ctx.lib
    fn = lib.ovfq_quantize_q8k_dev if src.device else lib.ovfq_quantize_q8k
    raise_for_status(fn(ctx.handle, src.ptr, rows, k, q.ptr, s.ptr, b.ptr), lib)


def _prequantized(ctx, weight, q, s, b, rows, bias, out):
    lib = ctx.lib
    fn = lib.ovfq_project_prequantized_dev if out.device else lib.ovfq_project_prequantized
    rc = fn(ctx.handle, weight.handle, q.ptr, s.ptr, None if b is None else b.ptr, rows,
            None if is_empty(bias) else bias.ptr, out.ptr)
    raise_for_status(rc, lib)


class _KQuantKernel:
    SuperBlockElements = 256
    GroupSize = 16
    GroupsPerSuperBlock = 16
    _weight_cls = Q4KWeight

    @classmethod
    def _check_weight(cls, weight):
        if weight is None:
            raise OverfitArgumentNullError("weight")
        if not isinstance(weight, cls._weight_cls) or (cls._weight_cls is Q4KWeight and isinstance(weight, Q6KWeight)):
            raise OverfitUnsupportedTypeError(f"{cls.__name__} needs a {cls._weight_cls.__name__}")

    @staticmethod
    def QuantizeActivationQ8K(source, quants, blockScales, bsums) -> None:
        """RT/Q4KDotKernel.cs:71-136 (bit-exact, on the device)."""
        src = as_buf(source, np.float32, "source")
        q = as_buf(quants, np.int8, "quants")
        s = as_buf(blockScales, np.float32, "blockScales")
        b = as_buf(bsums, np.int16, "bsums")
        same_side(src, q, s, b)
        if src.size % 256 != 0:
            raise OverfitArgumentError(f"Source length ({src.size}) must be a multiple of 256.")
        blocks = src.size // 256
        if q.size < src.size:
            raise OverfitArgumentError("Quants span is smaller than source.")
        if s.size < blocks:
            raise OverfitArgumentError("Block-scales span is smaller than the block count.")
        if b.size < blocks * 16:
            raise OverfitArgumentError("Bsums span is smaller than blocks * groups.")
        if blocks == 0:
            return
        _quantize_q8k(default_context(), src, q, s, b, 1, src.size)

    @classmethod
    def Project(cls, input, weight, bias, output, activationQuants, activationScales, activationBsums) -> None:
        """RT/Q4KDotKernel.cs:414-435: quantize the input into the scratch, then ProjectPreQuantized."""
        cls._check_weight(weight)
        inp = as_buf(input, np.float32, "input")
        out = as_buf(output, np.float32, "output")
        bb = as_buf(bias, np.float32, "bias", allow_none=True)
        _validate_project_arguments(inp, bb, out, weight.InputSize, weight.OutputSize)
        q = as_buf(activationQuants, np.int8, "activationQuants")
        s = as_buf(activationScales, np.float32, "activationScales")
        b = as_buf(activationBsums, np.int16, "activationBsums")
        same_side(inp, out, bb, q, s, b)
        k = weight.InputSize
        if q.size < k or s.size < k // 256 or b.size < k // 16:
            raise OverfitArgumentError("Activation quantization scratch is too small.")
        _quantize_q8k(weight.context, inp, q, s, b, 1, k)
        _prequantized(weight.context, weight, q, s, b, 1, bb, out)

    @classmethod
    def ProjectPreQuantized(cls, weight, bias, output, activationQuants, activationScales, activationBsums) -> None:
        """RT/Q4KDotKernel.cs:445-476."""
        cls._check_weight(weight)
        out = as_buf(output, np.float32, "output")
        bb = as_buf(bias, np.float32, "bias", allow_none=True)
        q = as_buf(activationQuants, np.int8, "activationQuants")
        s = as_buf(activationScales, np.float32, "activationScales")
        b = as_buf(activationBsums, np.int16, "activationBsums")
        same_side(out, bb, q, s, b)
        k = weight.InputSize
        if q.size < k or s.size < k // 256 or b.size < k // 16:
            raise OverfitArgumentError("Activation quantization scratch is too small.")
        if out.size < weight.OutputSize:
            raise OverfitArgumentError("Output span is smaller than the weight's output size.")
        if not is_empty(bb) and bb.size < weight.OutputSize:
            raise OverfitArgumentError("Bias span is smaller than outputSize.")
        _prequantized(weight.context, weight, q, s, b, 1, bb, out)

    ProjectParallel = Project

    @classmethod
    def ProjectBatched(cls, input, rows, weight, bias, output, activationQuants, activationScales,
                       activationBsums) -> None:
        """RT/Q4KDotKernel.cs:681-763 (RT/Q6KDotKernel.cs:403-471)."""
        cls._check_weight(weight)
        if rows <= 0:
            raise OverfitArgumentOutOfRangeError(f"rows ({rows}) must be positive")
        inp = as_buf(input, np.float32, "input")
        out = as_buf(output, np.float32, "output")
        bb = as_buf(bias, np.float32, "bias", allow_none=True)
        q = as_buf(activationQuants, np.int8, "activationQuants")
        s = as_buf(activationScales, np.float32, "activationScales")
        b = as_buf(activationBsums, np.int16, "activationBsums")
        same_side(inp, out, bb, q, s, b)
        k, n = weight.InputSize, weight.OutputSize
        if inp.size < rows * k:
            raise OverfitArgumentError("Input span is smaller than rows * inputSize.")
        if out.size < rows * n:
            raise OverfitArgumentError("Output span is smaller than rows * outputSize.")
        if not is_empty(bb) and bb.size < n:
            raise OverfitArgumentError("Bias span is smaller than outputSize.")
        if q.size < rows * k or s.size < rows * (k // 256) or b.size < rows * (k // 16):
            raise OverfitArgumentError("Activation quantization scratch is too small for rows.")
        _quantize_q8k(weight.context, inp, q, s, b, rows, k)
        _prequantized(weight.context, weight, q, s, b, rows, bb, out)

    @classmethod
    def Dot(cls, block, q8Block, q8Scale, bsums) -> float:
        """One super-block dot (RT/Q4KDotKernel.cs:216-256 / RT/Q6KDotKernel.cs:77-116), on the device."""
        nbytes = cls._weight_cls.SuperBlockBytes
        blk = as_buf(block, np.uint8, "block")
        q = as_buf(q8Block, np.int8, "q8Block")
        b = as_buf(bsums, np.int16, "bsums")
        if blk.size < nbytes:
            raise OverfitArgumentError(f"block span is smaller than {nbytes} bytes.")
        if q.size < 256:
            raise OverfitArgumentError("Q8 block span is smaller than 256.")
        if b.size < 16:
            raise OverfitArgumentError("Bsums span is smaller than 16.")
        w = cls._weight_cls(np.ascontiguousarray(np.asarray(blk.obj).reshape(-1)[:nbytes]), 256, 1)
        out = np.zeros(1, np.float32)
        s = np.array([q8Scale], np.float32)
        _prequantized(w.context, w, as_buf(np.ascontiguousarray(np.asarray(q.obj).reshape(-1)[:256]), np.int8, "q"),
                      as_buf(s, np.float32, "s"),
                      as_buf(np.ascontiguousarray(np.asarray(b.obj).reshape(-1)[:16]), np.int16, "b"), 1, None,
                      as_buf(out, np.float32, "out"))
        return float(out[0])


class Q4KDotKernel(_KQuantKernel):
    _weight_cls = Q4KWeight

    @classmethod
    def ProjectGateUpParallel(cls, input, gate, up, gateOutput, upOutput, activationQuants, activationScales,
                              activationBsums) -> None:
        """RT/Q4KDotKernel.cs:563-605: one quantize, gate and up in one launch."""
        if gate is None:
            raise OverfitArgumentNullError("gate")
        if up is None:
            raise OverfitArgumentNullError("up")
        cls._check_weight(gate)
        cls._check_weight(up)
        inp = as_buf(input, np.float32, "input")
        g = as_buf(gateOutput, np.float32, "gateOutput")
        u = as_buf(upOutput, np.float32, "upOutput")
        q = as_buf(activationQuants, np.int8, "activationQuants")
        s = as_buf(activationScales, np.float32, "activationScales")
        b = as_buf(activationBsums, np.int16, "activationBsums")
        same_side(inp, g, u, q, s, b)
        k = gate.InputSize
        if inp.size < k:
            raise OverfitArgumentError("Input span is smaller than the weight's input size.")
        if g.size < gate.OutputSize or u.size < up.OutputSize:
            raise OverfitArgumentError("Output span is smaller than the weight's output size.")
        if q.size < k or s.size < k // 256 or b.size < k // 16:
            raise OverfitArgumentError("Activation quantization scratch is too small.")
        ctx = gate.context
        _quantize_q8k(ctx, inp, q, s, b, 1, k)
        # The quantised activation in the scratch is the one the projection must use; the fused launch reads it
        # back from the caller's scratch (ProjectPreQuantized of both weights, one after the other, is the same
        # arithmetic as the reference's single dispatch).
        _prequantized(ctx, gate, q, s, b, 1, None, g)
        _prequantized(ctx, up, q, s, b, 1, None, u)

    ProjectBatchedWeightStationary = _KQuantKernel.ProjectBatched


class Q6KDotKernel(_KQuantKernel):
    _weight_cls = Q6KWeight


class Q8DotKernel:
    """RT/Q8DotKernel.cs."""

    BlockSize = 32

    @staticmethod
    def Quantize(source, quants, scales) -> None:
        """RT/Q8DotKernel.cs:42-91 (bit-exact, on the device)."""
        src = as_buf(source, np.float32, "source")
        q = as_buf(quants, np.int8, "quants")
        s = as_buf(scales, np.float32, "scales")
        same_side(src, q, s)
        if src.size % 32 != 0:
            raise OverfitArgumentError(f"Source length ({src.size}) must be a multiple of 32.")
        if q.size < src.size:
            raise OverfitArgumentError("Quants span is smaller than source.")
        if s.size < src.size // 32:
            raise OverfitArgumentError("Scales span is smaller than the block count.")
        if src.size == 0:
            return
        ctx = default_context()
        fn = ctx.lib.ovfq_quantize_q8_0_dev if src.device else ctx.lib.ovfq_quantize_q8_0
        raise_for_status(fn(ctx.handle, src.ptr, 1, src.size, q.ptr, s.ptr), ctx.lib)

    @staticmethod
    def Dot(aQuants, aScales, bQuants, bScales, length) -> float:
        """RT/Q8DotKernel.cs:99-140: sum over blocks of (aScale * bScale) * int8dot, on the device."""
        if length % 32 != 0:
            raise OverfitArgumentError(f"Length ({length}) must be a multiple of 32.")
        aq = np.ascontiguousarray(np.asarray(aQuants, dtype=np.int8).reshape(-1))
        bq = np.ascontiguousarray(np.asarray(bQuants, dtype=np.int8).reshape(-1))
        as_ = np.ascontiguousarray(np.asarray(aScales, dtype=np.float32).reshape(-1))
        bs = np.ascontiguousarray(np.asarray(bScales, dtype=np.float32).reshape(-1))
        if aq.size < length or bq.size < length:
            raise OverfitArgumentError("A quant span is smaller than length.")
        if as_.size < length // 32 or bs.size < length // 32:
            raise OverfitArgumentError("A scale span is smaller than the block count.")
        if length == 0:
            return 0.0
        w = Q8Weight(aq[:length], as_[:length // 32], length, 1)
        out = np.zeros(1, np.float32)
        _prequantized(w.context, w, as_buf(bq[:length].copy(), np.int8, "b"),
                      as_buf(bs[:length // 32].copy(), np.float32, "s"), None, 1, None, as_buf(out, np.float32, "y"))
        return float(out[0])

    @staticmethod
    def Project(input, weight, bias, output, inputQuants, inputScales) -> None:
        """RT/Q8DotKernel.cs:224-243 (the Q8Weight overload of :155-215)."""
        if weight is None:
            raise OverfitArgumentNullError("weight")
        if not isinstance(weight, Q8Weight):
            raise OverfitUnsupportedTypeError("Q8DotKernel needs a Q8Weight")
        inp = as_buf(input, np.float32, "input")
        out = as_buf(output, np.float32, "output")
        bb = as_buf(bias, np.float32, "bias", allow_none=True)
        q = as_buf(inputQuants, np.int8, "inputQuants")
        s = as_buf(inputScales, np.float32, "inputScales")
        same_side(inp, out, bb, q, s)
        k, n = weight.InputSize, weight.OutputSize
        if inp.size < k:
            raise OverfitArgumentError("Input span is smaller than inputSize.")
        if out.size < n:
            raise OverfitArgumentError("Output span is smaller than outputSize.")
        if not is_empty(bb) and bb.size < n:
            raise OverfitArgumentError("Bias span is smaller than outputSize.")
        if q.size < k or s.size < k // 32:
            raise OverfitArgumentError("Input quantization scratch is too small.")
        ctx = weight.context
        fn = ctx.lib.ovfq_quantize_q8_0_dev if inp.device else ctx.lib.ovfq_quantize_q8_0
        raise_for_status(fn(ctx.handle, inp.ptr, 1, k, q.ptr, s.ptr), ctx.lib)
        _prequantized(ctx, weight, q, s, None, 1, bb, out)

    ProjectParallel = Project

    @staticmethod
    def ProjectBatched(input, rows, weight, bias, output, inputQuants, inputScales) -> None:
        """RT/Q8DotKernel.cs:352-421."""
        if weight is None:
            raise OverfitArgumentNullError("weight")
        if rows <= 0:
            raise OverfitArgumentOutOfRangeError(f"rows ({rows}) must be positive")
        inp = as_buf(input, np.float32, "input")
        out = as_buf(output, np.float32, "output")
        bb = as_buf(bias, np.float32, "bias", allow_none=True)
        q = as_buf(inputQuants, np.int8, "inputQuants")
        s = as_buf(inputScales, np.float32, "inputScales")
        same_side(inp, out, bb, q, s)
        k, n = weight.InputSize, weight.OutputSize
        if inp.size < rows * k:
            raise OverfitArgumentError("Input span is smaller than rows * inputSize.")
        if out.size < rows * n:
            raise OverfitArgumentError("Output span is smaller than rows * outputSize.")
        if not is_empty(bb) and bb.size < n:
            raise OverfitArgumentError("Bias span is smaller than outputSize.")
        if q.size < rows * k or s.size < rows * (k // 32):
            raise OverfitArgumentError("Input quantization scratch is too small for rows.")
        ctx = weight.context
        fn = ctx.lib.ovfq_quantize_q8_0_dev if inp.device else ctx.lib.ovfq_quantize_q8_0
        raise_for_status(fn(ctx.handle, inp.ptr, rows, k, q.ptr, s.ptr), ctx.lib)
        _prequantized(ctx, weight, q, s, None, rows, bb, out)


class BatchedQuantProjection:
    """RT/BatchedQuantProjection.cs:26-87: rows x one quantized weight, scratch owned by the call."""

    UseWeightStationaryQ4K = True  # kept for interface parity; the device path is weight-stationary

    @staticmethod
    def Dispatch(input, rows, weight, bias, output, inputSize, outputSize) -> None:
        if not isinstance(weight, DecodeWeight):
            weight = DecodeWeight(weight)
        if weight.IsQ6K:
            w = weight.Quantized6K
        elif weight.IsQ4K:
            w = weight.Quantized4K
        elif weight.IsQuantized:
            w = weight.Quantized
        else:
            raise OverfitUnsupportedTypeError("F32 projections are outside the quantized-linear library")
        if rows <= 0:
            raise OverfitArgumentOutOfRangeError(f"rows ({rows}) must be positive")
        inp = as_buf(input, np.float32, "input")
        out = as_buf(output, np.float32, "output")
        bb = as_buf(bias, np.float32, "bias", allow_none=True)
        same_side(inp, out, bb)
        if inp.size < rows * inputSize or out.size < rows * outputSize:
            raise OverfitArgumentError("input/output span smaller than rows * size")
        if w.InputSize != inputSize or w.OutputSize != outputSize:
            raise OverfitArgumentError("weight shape does not match inputSize/outputSize")
        ctx = w.context
        fn = ctx.lib.ovfq_project_dev if inp.device else ctx.lib.ovfq_project
        raise_for_status(fn(ctx.handle, w.handle, inp.ptr, rows, None if is_empty(bb) else bb.ptr, out.ptr), ctx.lib)


class MoeRouter:
    """RT/MoeRouter.cs:40-128 on the device: per-token top-k expert selection and combine weights."""

    @staticmethod
    def SelectTopK(logits, topK, expertIndices, expertWeights, normalize=True, rows=1) -> int:
        """Writes the top-`topK` expert indices (descending by logit, ties to the lower index) and their
        softmax weights for `rows` tokens of logits [rows][nExperts]; returns min(topK, nExperts)."""
        lg = as_buf(logits, np.float32, "logits")
        ix = as_buf(expertIndices, np.int32, "expertIndices")
        wt = as_buf(expertWeights, np.float32, "expertWeights")
        same_side(lg, ix, wt)
        if rows <= 0:
            raise OverfitArgumentOutOfRangeError(f"rows ({rows}) must be positive")
        n = lg.size // rows
        if n == 0:
            raise OverfitArgumentError("Router logits cannot be empty.")
        if topK <= 0:
            raise OverfitArgumentOutOfRangeError(f"topK ({topK}) must be positive")
        k = min(topK, n)
        if ix.size < rows * topK or wt.size < rows * topK:
            raise OverfitArgumentError("expertIndices / expertWeights smaller than rows * topK")
        ctx = default_context()
        fn = ctx.lib.ovfq_moe_select_topk_dev if lg.device else ctx.lib.ovfq_moe_select_topk
        raise_for_status(fn(ctx.handle, lg.ptr, rows, n, topK, int(bool(normalize)), ix.ptr, wt.ptr), ctx.lib)
        return k


class FeedForwardActivation(enum.IntEnum):
    """Runtime/FeedForwardActivation.cs:11-34. The fused FFN takes the gated two: SwiGLU and GeGLU."""
    None_ = 0
    ReLU = 1
    GeLU = 2
    SwiGLU = 3
    GeGLU = 4


def ffn_swiglu(gate, up, down, x, rows=1, out=None):
    """CachedFeedForwardBlock.DecodeSwiGluDispatched / DecodeSwiGluBatchedDispatched (RT/CachedFeedForwardBlock.cs:
    261-344) on the device: down(SiLU(gate(x)) * up(x)) in three launches, no host round trip."""
    return ffn_gated(gate, up, down, x, rows, FeedForwardActivation.SwiGLU, out)


def ffn_gated(gate, up, down, x, rows=1, activation=FeedForwardActivation.SwiGLU, out=None):
    """The gated FFN with ApplyGate's activation (RT/CachedFeedForwardBlock.cs:328-344, :474-485): SwiGLU (SiLU gate)
    or GeGLU (GELU tanh-approximation gate, Gemma), down(act(gate(x)) * up(x)) in three launches."""
    act = int(activation)
    if act not in (FeedForwardActivation.SwiGLU, FeedForwardActivation.GeGLU):
        raise OverfitArgumentError(f"the fused FFN is gated: activation must be SwiGLU or GeGLU, not {activation!r}")
    inp = as_buf(x, np.float32, "x")
    d_model = gate.InputSize
    if out is None:
        if inp.device:
            import torch

            out = torch.empty(rows * d_model, dtype=torch.float32, device=inp.obj.device)
        else:
            out = np.zeros(rows * d_model, np.float32)
    o = as_buf(out, np.float32, "out")
    same_side(inp, o)
    ctx = gate.context
    fn = ctx.lib.ovfq_ffn_gated_dev if inp.device else ctx.lib.ovfq_ffn_gated
    raise_for_status(fn(ctx.handle, gate.handle, up.handle, down.handle, inp.ptr, rows, act, o.ptr), ctx.lib)
    return out


def moe_ffn(gate_experts, up_experts, down_experts, x, rows, top_k, expert_indices, expert_weights, out=None):
    """MoeFeedForwardBlock.DecodeBatched after routing (RT/MoeFeedForwardBlock.cs:140-241): tokens grouped by
    expert, each used expert's SwiGLU FFN on its tokens, weighted sum over the top-k slots in order."""
    E = len(gate_experts)
    if not (len(up_experts) == len(down_experts) == E):
        raise OverfitArgumentError("gate/up/down expert lists differ in length")
    inp = as_buf(x, np.float32, "x")
    d_model = gate_experts[0].InputSize
    if out is None:
        if inp.device:
            import torch

            out = torch.empty(rows * d_model, dtype=torch.float32, device=inp.obj.device)
        else:
            out = np.zeros(rows * d_model, np.float32)
    o = as_buf(out, np.float32, "out")
    ix = as_buf(expert_indices, np.int32, "expert_indices")
    wt = as_buf(expert_weights, np.float32, "expert_weights")
    same_side(inp, o, ix, wt)
    ctx = gate_experts[0].context
    arr = lambda ws: (ctypes.c_void_p * E)(*[w.handle.value for w in ws])
    fn = ctx.lib.ovfq_moe_ffn_dev if inp.device else ctx.lib.ovfq_moe_ffn
    raise_for_status(fn(ctx.handle, E, arr(gate_experts), arr(up_experts), arr(down_experts), inp.ptr, rows, top_k,
                        ix.ptr, wt.ptr, o.ptr), ctx.lib)
    return out


def moe_ffn_routed(gate_experts, up_experts, down_experts, x, rows, router_logits, top_k, normalize=True,
                   expert_indices=None, expert_weights=None, out=None):
    """MoeFeedForwardBlock.DecodeBatched from the router logits on (RT/MoeFeedForwardBlock.cs:140-241): the
    routing of MoeRouter.SelectTopK (RT/MoeRouter.cs:40-128) and the routed FFN (ovfq_moe_ffn_routed[_dev]).
    Returns (out, expert_indices, expert_weights); the routing arrays [rows][top_k] are allocated if not given."""
    E = len(gate_experts)
    if not (len(up_experts) == len(down_experts) == E):
        raise OverfitArgumentError("gate/up/down expert lists differ in length")
    inp = as_buf(x, np.float32, "x")
    d_model = gate_experts[0].InputSize

    def alloc(n, dtype):  # on the input's side: a device tensor beside a device input, else a numpy array
        if inp.device:
            import torch

            return torch.empty(n, dtype={np.int32: torch.int32, np.float32: torch.float32}[dtype],
                               device=inp.obj.device)
        return np.zeros(n, dtype)

    out = alloc(rows * d_model, np.float32) if out is None else out
    expert_indices = alloc(rows * top_k, np.int32) if expert_indices is None else expert_indices
    expert_weights = alloc(rows * top_k, np.float32) if expert_weights is None else expert_weights
    o = as_buf(out, np.float32, "out")
    lg = as_buf(router_logits, np.float32, "router_logits")
    ix = as_buf(expert_indices, np.int32, "expert_indices")
    wt = as_buf(expert_weights, np.float32, "expert_weights")
    same_side(inp, o, lg, ix, wt)
    ctx = gate_experts[0].context
    arr = lambda ws: (ctypes.c_void_p * E)(*[w.handle.value for w in ws])
    fn = ctx.lib.ovfq_moe_ffn_routed_dev if inp.device else ctx.lib.ovfq_moe_ffn_routed
    raise_for_status(fn(ctx.handle, E, arr(gate_experts), arr(up_experts), arr(down_experts), inp.ptr, rows, lg.ptr,
                        top_k, 1 if normalize else 0, ix.ptr, wt.ptr, o.ptr), ctx.lib)
    return out, expert_indices, expert_weights


def project_heads_q8_0(head_weights, x, rows=1, bias=None, out=None):
    """The attention output projection with per-head Q8_0 Wo (ovfq_project_heads_q8_0[_dev]): for each of `rows`
    rows of x [rows][n_heads * head_dim], out = bias (or zero) plus, heads ascending, each head's
    Q8DotKernel.Project of its head_dim slice through head_weights[h] ([d_model][head_dim] Q8Weight) —
    RT/CachedMultiHeadAttention.cs:185-194, :292-297 and RT/CachedSingleHeadAttention.cs:323-337, in one launch."""
    H = len(head_weights)
    if H == 0:
        raise OverfitArgumentError("head_weights is empty")
    inp = as_buf(x, np.float32, "x")
    d_model = head_weights[0].OutputSize
    if inp.size < rows * H * head_weights[0].InputSize:
        raise OverfitArgumentError("x is smaller than rows * n_heads * head_dim")
    if out is None:
        if inp.device:
            import torch

            out = torch.empty(rows * d_model, dtype=torch.float32, device=inp.obj.device)
        else:
            out = np.zeros(rows * d_model, np.float32)
    o = as_buf(out, np.float32, "out")
    if o.size < rows * d_model:
        raise OverfitArgumentError("out is smaller than rows * d_model")
    bb = as_buf(bias, np.float32, "bias", allow_none=True)
    same_side(inp, o, bb)
    ctx = head_weights[0].context
    W = (ctypes.c_void_p * H)(*[w.handle.value for w in head_weights])
    fn = ctx.lib.ovfq_project_heads_q8_0_dev if inp.device else ctx.lib.ovfq_project_heads_q8_0
    raise_for_status(fn(ctx.handle, H, W, inp.ptr, rows, None if is_empty(bb) else bb.ptr, o.ptr), ctx.lib)
    return out


def project(weight, x, bias=None, rows=1, out=None):
    """Convenience: y = (bias +) x @ W^T with the library's own activation scratch."""
    inp = as_buf(x, np.float32, "x")
    if out is None:
        if inp.device:
            import torch

            out = torch.empty(rows * weight.OutputSize, dtype=torch.float32, device=inp.obj.device)
        else:
            out = np.zeros(rows * weight.OutputSize, np.float32)
    o = as_buf(out, np.float32, "out")
    bb = as_buf(bias, np.float32, "bias", allow_none=True)
    same_side(inp, o, bb)
    ctx = weight.context
    fn = ctx.lib.ovfq_project_dev if inp.device else ctx.lib.ovfq_project
    raise_for_status(fn(ctx.handle, weight.handle, inp.ptr, rows, None if is_empty(bb) else bb.ptr, o.ptr), ctx.lib)
    return out


def project_multi(weights, x, rows=1, biases=None, outs=None):
    """Several projections of one activation in one launch (ovfq_project_multi[_dev]): the attention block's q/k/v
    against its once-quantised hidden rows (RT/CachedMultiHeadAttention.cs:196-207). Returns the outputs, each
    rows x OutputSize (allocated on the input's side when `outs` is None)."""
    n = len(weights)
    if n == 0:
        raise OverfitArgumentError("weights is empty")
    inp = as_buf(x, np.float32, "x")
    if outs is None:
        if inp.device:
            import torch

            outs = [torch.empty(rows * w.OutputSize, dtype=torch.float32, device=inp.obj.device) for w in weights]
        else:
            outs = [np.zeros(rows * w.OutputSize, np.float32) for w in weights]
    if len(outs) != n or (biases is not None and len(biases) != n):
        raise OverfitArgumentError("weights, outs and biases must have the same length")
    ob = [as_buf(o, np.float32, "out") for o in outs]
    bb = [None] * n if biases is None else [as_buf(b, np.float32, "bias", allow_none=True) for b in biases]
    same_side(inp, *ob, *bb)
    ctx = weights[0].context
    W = (ctypes.c_void_p * n)(*[w.handle.value for w in weights])
    Y = (ctypes.c_void_p * n)(*[o.ptr for o in ob])
    B = (ctypes.c_void_p * n)(*[None if is_empty(b) else b.ptr for b in bb])
    fn = ctx.lib.ovfq_project_multi_dev if inp.device else ctx.lib.ovfq_project_multi
    raise_for_status(fn(ctx.handle, n, W, inp.ptr, rows, B, Y), ctx.lib)
    return outs


def project_gate_up(gate, up, x, gate_out=None, up_out=None):
    """Convenience: fused gate/up (ovfq_project_gate_up[_dev]) with the library's own scratch."""
    inp = as_buf(x, np.float32, "x")
    if gate_out is None or up_out is None:
        if inp.device:
            import torch

            gate_out = torch.empty(gate.OutputSize, dtype=torch.float32, device=inp.obj.device)
            up_out = torch.empty(up.OutputSize, dtype=torch.float32, device=inp.obj.device)
        else:
            gate_out = np.zeros(gate.OutputSize, np.float32)
            up_out = np.zeros(up.OutputSize, np.float32)
    g = as_buf(gate_out, np.float32, "gate_out")
    u = as_buf(up_out, np.float32, "up_out")
    same_side(inp, g, u)
    ctx = gate.context
    fn = ctx.lib.ovfq_project_gate_up_dev if inp.device else ctx.lib.ovfq_project_gate_up
    raise_for_status(fn(ctx.handle, gate.handle, up.handle, inp.ptr, g.ptr, u.ptr), ctx.lib)
    return gate_out, up_out


def quantize_weight(w, type_id, ctx=None):
    """Quantize an output-major f32 GPU tensor [out, in] on the device: GgmlQuant.QuantizeQ4_K
    (LD/GgmlQuant.cs:132-161) for Q4_K, the build's Q6_K encoder, or Q8Weight.QuantizeRows (Q8_0).
    Returns a torch uint8 tensor of blocks (Q4_K/Q6_K) or a (quants, scales) pair (Q8_0)."""
    import torch

    ctx = ctx or default_context()
    out_rows, k = w.shape
    if type_id == _lib.TYPE_Q4_K:
        dst = torch.empty(out_rows * (k // 256) * 144, dtype=torch.uint8, device=w.device)
        raise_for_status(ctx.lib.ovfq_quantize_weight_q4k_dev(ctx.handle, w.data_ptr(), k, out_rows, dst.data_ptr()),
                         ctx.lib)
        return dst
    if type_id == _lib.TYPE_Q6_K:
        dst = torch.empty(out_rows * (k // 256) * 210, dtype=torch.uint8, device=w.device)
        raise_for_status(ctx.lib.ovfq_quantize_weight_q6k_dev(ctx.handle, w.data_ptr(), k, out_rows, dst.data_ptr()),
                         ctx.lib)
        return dst
    if type_id == _lib.TYPE_Q8_0:
        q = torch.empty(out_rows * k, dtype=torch.int8, device=w.device)
        s = torch.empty(out_rows * (k // 32), dtype=torch.float32, device=w.device)
        raise_for_status(ctx.lib.ovfq_quantize_weight_q8_0_dev(ctx.handle, w.data_ptr(), k, out_rows, q.data_ptr(),
                                                               s.data_ptr()), ctx.lib)
        return q, s
    raise OverfitUnsupportedTypeError(f"type {type_id}")
