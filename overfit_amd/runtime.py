"""Device context and buffer plumbing for the ctypes binding.

Buffers may be numpy arrays / bytes (host memory: the synchronous C entry points are used) or torch tensors
on the GPU (device memory: the asynchronous ``_dev`` entry points are used, on the context's stream, which
is bound to torch's default stream so that torch work and library work are ordered). One call never mixes
host and device buffers.
"""
import ctypes
import threading

import numpy as np

from . import _lib
from .errors import OverfitArgumentError, OverfitArgumentNullError, raise_for_status

try:  # torch is plumbing for device memory only
    import torch
except Exception:  # pragma: no cover - torch is present in this image
    torch = None

_NP_OF_TORCH = {}
if torch is not None:
    _NP_OF_TORCH = {
        torch.int8: np.int8,
        torch.uint8: np.uint8,
        torch.int16: np.int16,
        torch.float32: np.float32,
        torch.int32: np.int32,
    }


class Buf:
    """A validated view of a caller buffer: address, element count, and where it lives."""

    __slots__ = ("ptr", "size", "device", "obj")

    def __init__(self, ptr, size, device, obj):
        self.ptr = ptr
        self.size = size
        self.device = device
        self.obj = obj


def as_buf(x, dtype, name, allow_none=False):
    """Wrap `x` (numpy / bytes / torch tensor) as a Buf of element type `dtype`. None -> None if allowed."""
    if x is None:
        if allow_none:
            return None
        raise OverfitArgumentNullError(f"{name} is None")
    dtype = np.dtype(dtype)
    if torch is not None and isinstance(x, torch.Tensor):
        if _NP_OF_TORCH.get(x.dtype) is not dtype.type:
            raise OverfitArgumentError(f"{name} must have dtype {dtype}, got {x.dtype}")
        if not x.is_contiguous():
            raise OverfitArgumentError(f"{name} must be contiguous")
        return Buf(x.data_ptr(), x.numel(), x.is_cuda, x)
    if isinstance(x, (bytes, bytearray, memoryview)):
        x = np.frombuffer(x, dtype=np.uint8)
        if dtype != np.uint8:
            x = x.view(dtype)
    if not isinstance(x, np.ndarray):
        raise OverfitArgumentError(f"{name} must be a numpy array or a torch tensor")
    if x.dtype != dtype:
        raise OverfitArgumentError(f"{name} must have dtype {dtype}, got {x.dtype}")
    if not x.flags["C_CONTIGUOUS"]:
        raise OverfitArgumentError(f"{name} must be C-contiguous")
    return Buf(x.ctypes.data, x.size, False, x)


def same_side(*bufs):
    """True if every non-None buffer is on the device, False if all are host; raises on a mix."""
    sides = {b.device for b in bufs if b is not None}
    if len(sides) > 1:
        raise OverfitArgumentError("host and device buffers cannot be mixed in one call")
    return sides.pop() if sides else False


def is_empty(b):
    return b is None or b.size == 0


class Context:
    """One libovfq context (a device plus the stream its work runs on)."""

    def __init__(self, device: int = 0, bind_torch_stream: bool = True):
        self.lib = _lib.load()
        h = ctypes.c_void_p()
        raise_for_status(self.lib.ovfq_ctx_create(device, ctypes.byref(h)), self.lib)
        self.handle = h
        self.device = device
        if bind_torch_stream and torch is not None:
            self.set_stream(torch.cuda.current_stream(device).cuda_stream)

    def check(self, rc):
        raise_for_status(rc, self.lib)

    def set_stream(self, stream_handle):
        self.check(self.lib.ovfq_ctx_set_stream(self.handle, ctypes.c_void_p(stream_handle or None)))

    def synchronize(self):
        self.check(self.lib.ovfq_ctx_synchronize(self.handle))

    def release_retired(self):
        """Frees scratch buffers that later, larger calls superseded (kept so that captured HIP graphs stay valid).
        Only when no graph captured from this context's calls will be replayed again."""
        self.check(self.lib.ovfq_ctx_release_retired(self.handle))

    def scratch_bytes(self):
        """(live, retired): device scratch bytes in the context's growable buffers and in superseded ones."""
        live, retired = ctypes.c_size_t(), ctypes.c_size_t()
        self.check(self.lib.ovfq_ctx_scratch_bytes(self.handle, ctypes.byref(live), ctypes.byref(retired)))
        return live.value, retired.value

    BATCHED_KERNELS = {"auto": 0, "small": 1, "tiled": 2, "rows": 3}

    def set_batched_kernel(self, kind: str):
        """Kernel for batched K-quant work of 2+ rows: "auto" (by shape), "small" (small-M MFMA kernel), "tiled"
        (64-row-tiled MFMA kernel) or "rows" (multi-row decode kernel), each where it takes the shape; outputs are
        bit-identical. The
        reference's test-only BatchedQuantProjection.UseWeightStationaryQ4K toggle
        (RT/BatchedQuantProjection.cs:21-24) plays this part there."""
        if kind not in self.BATCHED_KERNELS:
            raise ValueError(f"batched kernel must be one of {sorted(self.BATCHED_KERNELS)}, not {kind!r}")
        self.check(self.lib.ovfq_ctx_set_batched_kernel(self.handle, self.BATCHED_KERNELS[kind]))

    def close(self):
        """Destroys the context. Every weight created on it must have been destroyed first (the library refuses
        otherwise, and the context stays usable)."""
        if self.handle:
            self.check(self.lib.ovfq_ctx_destroy(self.handle))
            self.handle = None

    # ---------------------------------------------------------------- device-pointer conveniences

    def quantize_q8k_dev(self, x, rows, k, q, s, b):
        self.check(self.lib.ovfq_quantize_q8k_dev(self.handle, x.data_ptr(), rows, k, q.data_ptr(), s.data_ptr(),
                                                  b.data_ptr()))

    def project_dev(self, weight, x, y, bias=None, rows=1):
        self.check(self.lib.ovfq_project_dev(self.handle, weight.handle, x.data_ptr(), rows,
                                             None if bias is None else bias.data_ptr(), y.data_ptr()))

    def project_multi_dev(self, weights, x, ys, biases=None, rows=1):
        n = len(weights)
        W = (ctypes.c_void_p * n)(*[w.handle.value for w in weights])
        Y = (ctypes.c_void_p * n)(*[y.data_ptr() for y in ys])
        B = None
        if biases is not None:
            B = (ctypes.c_void_p * n)(*[None if b is None else b.data_ptr() for b in biases])
        self.check(self.lib.ovfq_project_multi_dev(self.handle, n, W, x.data_ptr(), rows, B, Y))

    def bind_multi_dev(self, weights, x, ys, biases=None, rows=1):
        """`project_multi_dev` with its arguments converted once: returns a callable that issues exactly
        ovfq_project_multi_dev(ctx, n, weights, x, rows, biases, ys) on every call. For hot decode loops, where
        rebuilding the pointer arrays each call costs more host time than the launch itself; the tensors are
        held until the callable is dropped."""
        return BoundMulti(self, weights, x, ys, biases, rows)

    def project_multi_prequantized_dev(self, weights, q, s, b, ys, biases=None, rows=1):
        n = len(weights)
        W = (ctypes.c_void_p * n)(*[w.handle.value for w in weights])
        Y = (ctypes.c_void_p * n)(*[y.data_ptr() for y in ys])
        B = None
        if biases is not None:
            B = (ctypes.c_void_p * n)(*[None if x is None else x.data_ptr() for x in biases])
        self.check(self.lib.ovfq_project_multi_prequantized_dev(self.handle, n, W, q.data_ptr(), s.data_ptr(),
                                                                b.data_ptr(), rows, B, Y))

    def project_prequantized_dev(self, weight, q, s, b, y, rows=1, bias=None):
        self.check(self.lib.ovfq_project_prequantized_dev(
            self.handle, weight.handle, q.data_ptr(), s.data_ptr(), None if b is None else b.data_ptr(), rows,
            None if bias is None else bias.data_ptr(), y.data_ptr()))


class BoundMulti:
    """A prepared ovfq_project_multi_dev call (see Context.bind_multi_dev)."""

    __slots__ = ("_fn", "_args", "_ctx", "_keep")

    def __init__(self, ctx, weights, x, ys, biases, rows):
        n = len(weights)
        if len(ys) != n or (biases is not None and len(biases) != n):
            raise ValueError("weights, ys and biases must have the same length")
        W = (ctypes.c_void_p * n)(*[w.handle.value for w in weights])
        Y = (ctypes.c_void_p * n)(*[y.data_ptr() for y in ys])
        B = None
        if biases is not None:
            B = (ctypes.c_void_p * n)(*[None if b is None else b.data_ptr() for b in biases])
        self._ctx = ctx
        self._fn = ctx.lib.ovfq_project_multi_dev
        self._args = (ctx.handle, n, W, ctypes.c_void_p(x.data_ptr()), rows, B, Y)
        self._keep = (list(weights), x, list(ys), None if biases is None else list(biases))

    def __call__(self):
        rc = self._fn(*self._args)
        if rc:
            self._ctx.check(rc)


_default = {}
_default_lock = threading.Lock()


def default_context(device: int = 0) -> Context:
    """The process-wide context for `device` (created on first use, bound to torch's default stream)."""
    with _default_lock:
        ctx = _default.get(device)
        if ctx is None:
            ctx = Context(device)
            _default[device] = ctx
        return ctx
