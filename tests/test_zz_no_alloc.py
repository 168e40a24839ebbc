"""ovfq_project_noalloc_dev: the allocation-free projection entry point against ovfq_project_dev.

Both are called through the C ABI on identical device buffers, two calls in a row on each case, the second with
a smaller input than the first (the fixed scratch keeps the first call's contents); outputs must be bit-identical
to ovfq_project_dev's, and to the oracle's. Sizes past the fixed scratch are refused before any work.
"""
import ctypes
import sys

import numpy as np
import pytest

from qdata import normal, random_q4k_blocks, random_q6k_blocks

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
ov = pytest.importorskip("overfit_amd")
from overfit_amd import _lib  # noqa: E402

DEV = "cuda:0"


def case(*what):
    print("[case]", *what, flush=True, file=sys.stderr)


def t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _weight(orc, rng, fmt, n, k):
    """The resident weight and its oracle: (x, rows, bias) -> y[rows][n] (the reference's batched loop, whose
    outputs equal the single-row Project's)."""
    if fmt == "q4k":
        blocks = random_q4k_blocks(rng, n * k // 256).reshape(n, -1)
        return ov.Q4KWeight(blocks, k, n), lambda x, rows, b: orc.q4k_project_batched(x, rows, blocks, k, n, b)
    if fmt == "q6k":
        blocks = random_q6k_blocks(rng, n * k // 256).reshape(n, -1)
        return ov.Q6KWeight(blocks, k, n), lambda x, rows, b: orc.q6k_project_batched(x, rows, blocks, k, n, b)
    wq, ws = orc.q8_quantize_rows(normal(rng, (n, k), 0.05))
    return ov.Q8Weight(wq, ws, k, n), lambda x, rows, b: orc.q8_project_batched(x, rows, wq, ws, k, n, b)


def _call(lib, ctx, fn, w, x, rows, bias, y):
    return fn(ctx.handle, w.handle, ctypes.c_void_p(x.data_ptr()), rows,
              None if bias is None else ctypes.c_void_p(bias.data_ptr()), ctypes.c_void_p(y.data_ptr()))


# (format, outputs, input size, rows of the first call, rows of the second call)
CASES = [
    ("q4k", 512, 4096, 40, 3),     # batched MFMA kernel, then the multi-row kernel (quantised in its launch)
    ("q4k", 256, 4096, 512, 17),   # full scratch (512 x 4096 = 2^21 elements), then a smaller batch
    ("q6k", 256, 14336, 1, 1),     # decode of a long row: quantised into the scratch before the GEMV
    ("q6k", 128, 14336, 9, 2),
    ("q8_0", 512, 4096, 16, 5),
    ("q8_0", 300, 14336, 3, 1),
]


@pytest.mark.parametrize("fmt,n,k,rows1,rows2", CASES)
def test_noalloc_matches_project_dev(orc, fmt, n, k, rows1, rows2):
    ctx = ov.default_context()
    lib = ctx.lib
    rng = np.random.default_rng(n + k + rows1)
    w, ref_fn = _weight(orc, rng, fmt, n, k)
    bias = normal(rng, n)
    for call, rows in enumerate((rows1, rows2)):
        case("noalloc", fmt, n, k, "call", call, "rows", rows)
        x = normal(rng, (rows, k))
        b_host = bias if call == 0 else None
        xd, bd = t(x), None if b_host is None else t(b_host)
        y_ref = torch.full((rows * n,), float("nan"), device=DEV)
        y_new = torch.full((rows * n,), float("nan"), device=DEV)
        assert _call(lib, ctx, lib.ovfq_project_dev, w, xd, rows, bd, y_ref) == 0, lib.ovfq_last_error()
        assert _call(lib, ctx, lib.ovfq_project_noalloc_dev, w, xd, rows, bd, y_new) == 0, lib.ovfq_last_error()
        torch.cuda.synchronize()
        a, b = y_new.cpu().numpy(), y_ref.cpu().numpy()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"call {call}: differs from ovfq_project_dev"
        oracle = ref_fn(x, rows, b_host).reshape(-1)
        assert np.array_equal(a.view(np.uint32), oracle.view(np.uint32)), f"call {call}: differs from the oracle"


def test_noalloc_refuses_past_the_fixed_scratch(orc):
    ctx = ov.default_context()
    lib = ctx.lib
    rng = np.random.default_rng(3)
    k, n = 4096, 64
    w = ov.Q4KWeight(random_q4k_blocks(rng, n * k // 256).reshape(n, -1), k, n)
    rows = (1 << 21) // k + 1
    case("noalloc refuse", rows)
    x = torch.zeros(rows * k, device=DEV)
    y = torch.zeros(rows * n, device=DEV)
    assert _call(lib, ctx, lib.ovfq_project_noalloc_dev, w, x, rows, None, y) == _lib.OVFQ_ERR_SIZE
    assert b"fixed scratch" in lib.ovfq_last_error()


def test_noalloc_allocates_no_device_memory(orc):
    """On a fresh context that has never grown its scratch, calls of ovfq_project_noalloc_dev up to the fixed
    scratch's full size leave the device's free memory unchanged (every tensor is allocated beforehand; the first,
    small call loads the kernels). A path that fell back to the context's growable scratch would allocate at least
    the 2 MiB quant plane here."""
    ctx = ov.Context(0)
    lib = ctx.lib
    rng = np.random.default_rng(8)
    k, n, rows = 4096, 256, (1 << 21) // 4096
    blocks = random_q4k_blocks(rng, n * k // 256).reshape(n, -1)
    w = ov.Q4KWeight(blocks, k, n, ctx=ctx)
    x_small, x_big = t(normal(rng, (40, k))), t(normal(rng, (rows, k)))
    y_small = torch.empty(40 * n, device=DEV)
    y_big = torch.empty(rows * n, device=DEV)
    case("noalloc fresh context", rows)
    assert ctx.scratch_bytes() == (0, 0)
    assert _call(lib, ctx, lib.ovfq_project_noalloc_dev, w, x_small, 40, None, y_small) == 0, lib.ovfq_last_error()
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    assert _call(lib, ctx, lib.ovfq_project_noalloc_dev, w, x_big, rows, None, y_big) == 0, lib.ovfq_last_error()
    torch.cuda.synchronize()
    free1 = torch.cuda.mem_get_info()[0]
    assert free1 == free0, f"device free memory changed by {free0 - free1} bytes"
    assert ctx.scratch_bytes() == (0, 0), "the allocation-free entry point grew the context's scratch"
    ref = orc.q4k_project_batched(x_big.cpu().numpy(), rows, blocks, k, n, None).reshape(-1)
    assert np.array_equal(y_big.cpu().numpy().view(np.uint32), ref.view(np.uint32))
    del w
    import gc
    gc.collect()
    ctx.close()
