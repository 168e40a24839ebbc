"""Resident quantized weights: the device-backed counterparts of Overfit's Q4KWeight, Q6KWeight, Q8Weight
and the DecodeWeight tagged union (RT/Q4KWeight.cs, RT/Q6KWeight.cs, RT/Q8Weight.cs, RT/DecodeWeight.cs).

A weight is uploaded to HBM once, in its native GGUF layout (output-major rows of super-blocks), and is
immutable afterwards. Member names follow the reference.
"""
import ctypes

import numpy as np

from . import _lib
from .errors import (OverfitArgumentError, OverfitArgumentNullError, OverfitArgumentOutOfRangeError,
                     OverfitUnsupportedTypeError, raise_for_status)
from .runtime import as_buf, default_context


class _ResidentWeight:
    _type = None
    SuperBlockElements = 256

    def _upload(self, blocks, nbytes, scales, input_size, output_size, ctx):
        self._ctx = ctx or default_context()
        lib = self._ctx.lib
        h = ctypes.c_void_p()
        on_device = blocks.device
        if scales is not None and scales.device != on_device:
            raise OverfitArgumentError("quants and scales must both be host or both be device buffers")
        fn = lib.ovfq_weight_create_from_device if on_device else lib.ovfq_weight_create
        rc = fn(self._ctx.handle, self._type, blocks.ptr, nbytes, None if scales is None else scales.ptr,
                input_size, output_size, ctypes.byref(h))
        raise_for_status(rc, lib)
        self.handle = h
        self._input_size = input_size
        self._output_size = output_size

    def __del__(self):
        h = getattr(self, "handle", None)
        if h is not None and h.value:
            try:
                self._ctx.lib.ovfq_weight_destroy(h)
            except Exception:
                pass
            self.handle = None

    @property
    def InputSize(self) -> int:
        return self._input_size

    @property
    def OutputSize(self) -> int:
        return self._output_size

    @property
    def context(self):
        return self._ctx

    @property
    def ByteCount(self) -> int:
        n = ctypes.c_size_t()
        raise_for_status(self._ctx.lib.ovfq_weight_info(self.handle, None, None, None, ctypes.byref(n), None),
                         self._ctx.lib)
        return n.value

    def prepare_mfma(self):
        """Adds the opt-in MFMA-ready copy of a Q6_K weight (ovfq_weight_prepare_mfma): batched projections
        (M >= 32) then skip the per-block operand build, bit-identically, for ~2.5x the weight's bytes. A no-op for
        Q4_K weights. Returns self."""
        raise_for_status(self._ctx.lib.ovfq_weight_prepare_mfma(self._ctx.handle, self.handle), self._ctx.lib)
        return self

    def DecodeRow(self, row: int, dst) -> None:
        """Dequantises output row `row` into dst[InputSize] (numpy host array or torch GPU tensor)."""
        if row < 0 or row >= self.OutputSize:
            raise OverfitArgumentOutOfRangeError(f"row {row} out of range [0, {self.OutputSize})")
        d = as_buf(dst, np.float32, "dst")
        if d.size < self.InputSize:
            raise OverfitArgumentError(f"Destination span too small: {d.size} < {self.InputSize}.")
        lib = self._ctx.lib
        fn = lib.ovfq_weight_decode_row_dev if d.device else lib.ovfq_weight_decode_row
        raise_for_status(fn(self._ctx.handle, self.handle, row, d.ptr), lib)


def _check_dims(input_size, output_size, multiple):
    if input_size <= 0:
        raise OverfitArgumentOutOfRangeError(f"inputSize ({input_size}) must be positive")
    if output_size <= 0:
        raise OverfitArgumentOutOfRangeError(f"outputSize ({output_size}) must be positive")
    if input_size % multiple:
        raise OverfitArgumentError(f"inputSize ({input_size}) must be a multiple of {multiple}.")


class Q4KWeight(_ResidentWeight):
    """Q4KWeight(blocks, inputSize, outputSize) — RT/Q4KWeight.cs:44-66."""

    _type = _lib.TYPE_Q4_K
    SuperBlockBytes = 144

    def __init__(self, blocks, input_size: int, output_size: int, ctx=None):
        if blocks is None:
            raise OverfitArgumentNullError("blocks")
        _check_dims(input_size, output_size, self.SuperBlockElements)
        b = as_buf(blocks, np.uint8, "blocks")
        expected = output_size * (input_size // 256) * self.SuperBlockBytes
        if b.size < expected:
            raise OverfitArgumentError(
                f"blocks region ({b.size} B) is smaller than outputSize * superBlocksPerRow * "
                f"{self.SuperBlockBytes} ({expected} B).")
        self._upload(b, b.size, None, input_size, output_size, ctx)

    @property
    def SuperBlocksPerRow(self) -> int:
        return self.InputSize // self.SuperBlockElements


class Q6KWeight(Q4KWeight):
    """Q6KWeight(blocks, inputSize, outputSize) — RT/Q6KWeight.cs:47."""

    _type = _lib.TYPE_Q6_K
    SuperBlockBytes = 210


class Q8Weight(_ResidentWeight):
    """Q8Weight(quants, scales, inputSize, outputSize) — RT/Q8Weight.cs:23-50 (resident int8 + f32 planes)."""

    _type = _lib.TYPE_Q8_0
    BlockSize = 32

    def __init__(self, quants, scales, input_size: int, output_size: int, ctx=None):
        if quants is None:
            raise OverfitArgumentNullError("quants")
        if scales is None:
            raise OverfitArgumentNullError("scales")
        _check_dims(input_size, output_size, self.BlockSize)
        q = as_buf(quants, np.int8, "quants")
        s = as_buf(scales, np.float32, "scales")
        if q.size < output_size * input_size:
            raise OverfitArgumentError("Quants array is smaller than outputSize * inputSize.")
        if s.size < output_size * (input_size // self.BlockSize):
            raise OverfitArgumentError("Scales array is smaller than outputSize * blocksPerRow.")
        self._upload(q, q.size, s, input_size, output_size, ctx)


# GGUF tensor type -> the resident weight class it becomes (the 5-bit types are kept as Q8_0).
_GGUF_CLASS = {_lib.TYPE_Q4_K: Q4KWeight, _lib.TYPE_Q6_K: Q6KWeight, _lib.TYPE_Q8_0: Q8Weight,
               _lib.TYPE_Q5_0: Q8Weight, _lib.TYPE_Q5_K: Q8Weight}


def load_gguf_tensor(type_id, data, input_size: int, output_size: int, ctx=None):
    """A quantized tensor exactly as a GGUF file stores it -> the matching resident weight (GgufReader's
    LoadTensorQ4_KRaw / LoadTensorQ6_KRaw / LoadTensorQ8_0Raw, LD/GgufReader.cs:198-344): Q4_K/Q6_K bytes verbatim,
    Q8_0's 34-byte blocks de-interleaved on the device into the int8 + f32 planes, Q5_0 / Q5_K decoded and requantised
    to a Q8_0 weight on the device (the loader's path for 5-bit tensors, LD/GgufLlamaLoader.cs:665-680)."""
    cls = _GGUF_CLASS.get(type_id)
    if cls is None:
        raise OverfitUnsupportedTypeError(f"type {type_id}")
    buf = as_buf(data, np.uint8, "data")
    w = cls.__new__(cls)
    w._ctx = ctx or default_context()
    lib = w._ctx.lib
    h = ctypes.c_void_p()
    fn = lib.ovfq_weight_create_gguf_dev if buf.device else lib.ovfq_weight_create_gguf
    raise_for_status(fn(w._ctx.handle, type_id, buf.ptr, buf.size, input_size, output_size, ctypes.byref(h)), lib)
    w.handle = h
    w._input_size = input_size
    w._output_size = output_size
    return w


def load_gguf_experts(type_id, data, input_size: int, output_size: int, n_experts: int, ctx=None):
    """GgufLlamaLoader.LoadExperts (LD/GgufLlamaLoader.cs:600-690): a 3-D GGUF expert tensor [input_size,
    output_size, n_experts] (expert axis slowest) -> one resident weight per expert, the experts sharing one device
    allocation (freed with the last of them). Q4_K/Q6_K slices verbatim, Q8_0 de-interleaved per expert, Q5_0 / Q5_K
    requantised to Q8_0 per expert."""
    cls = _GGUF_CLASS.get(type_id)
    if cls is None:
        raise OverfitUnsupportedTypeError(f"type {type_id}")
    buf = as_buf(data, np.uint8, "data")
    ctx = ctx or default_context()
    lib = ctx.lib
    hs = (ctypes.c_void_p * max(int(n_experts), 1))()
    fn = lib.ovfq_weight_create_experts_gguf_dev if buf.device else lib.ovfq_weight_create_experts_gguf
    raise_for_status(fn(ctx.handle, type_id, buf.ptr, buf.size, input_size, output_size, n_experts, hs), lib)
    experts = []
    for h in hs[:n_experts]:
        w = cls.__new__(cls)
        w._ctx = ctx
        w.handle = ctypes.c_void_p(h)
        w._input_size = input_size
        w._output_size = output_size
        experts.append(w)
    return experts


class DecodeWeight:
    """The 4-way tagged union {F32 | Q8_0 | Q4_K | Q6_K} of RT/DecodeWeight.cs:28-177.

    The F32 arm is kept for interface parity (row lookup only); projections of F32 weights are outside this
    library (it implements the GGUF-quantized path only).
    """

    def __init__(self, backing):
        if backing is None:
            raise OverfitArgumentNullError("backing")
        self._b = backing

    @property
    def IsQuantized(self) -> bool:
        return isinstance(self._b, Q8Weight)

    @property
    def IsQ4K(self) -> bool:
        return type(self._b) is Q4KWeight

    @property
    def IsQ6K(self) -> bool:
        return isinstance(self._b, Q6KWeight)

    @property
    def IsEmpty(self) -> bool:
        return isinstance(self._b, np.ndarray) and self._b.size == 0

    @property
    def ElementCount(self) -> int:
        if isinstance(self._b, _ResidentWeight):
            return self._b.OutputSize * self._b.InputSize
        return int(np.asarray(self._b).size)

    @property
    def Quantized(self) -> Q8Weight:
        return self._b

    @property
    def Quantized4K(self) -> Q4KWeight:
        return self._b

    @property
    def Quantized6K(self) -> Q6KWeight:
        return self._b

    @property
    def F32(self):
        return self._b

    def DequantizeRow(self, row: int, dst) -> None:
        if isinstance(self._b, _ResidentWeight):
            self._b.DecodeRow(row, dst)
            return
        f32 = np.asarray(self._b, dtype=np.float32).reshape(-1)
        n = len(dst)
        dst[:] = f32[row * n:(row + 1) * n]
