"""The per-head Q8_0 attention output projection (ovfq_project_heads_q8_0[_dev]) against the oracle.

Up to 31 rows run on the decode kernel (one launch per 8 rows); from 32 rows the int8-MFMA kernel walks the
contraction head by head (prefill rows, RT/CachedMultiHeadAttention.cs:689-710). Both are covered, also forced.

The reference's default Llama decode o-path: Wo requantised per head to Q8_0 (LD/GgufLlamaLoader.cs:977-995), each
head's Q8DotKernel.Project of its head_dim slice, and output = bias (or zero) + the head outputs in ascending head
order (RT/CachedMultiHeadAttention.cs:185-194, :292-297; prefill rows :600-614, :703-711). Bit-exact everywhere:
the in-launch and the separate Q8_0 quantisation, one launch and several (more than 8 rows), partial output
tiles, head_dim 32 .. 256, the full Llama-3-8B shape, raw int8 planes holding -128.
"""
import ctypes
import sys

import numpy as np
import pytest

from qdata import normal

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
ov = pytest.importorskip("overfit_amd")
from overfit_amd import _lib  # noqa: E402

DEV = "cuda:0"


def case(*what):
    print("[case]", *what, flush=True, file=sys.stderr)


def t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _heads(orc, rng, H, hd, dm, raw=False):
    """H per-head Wo planes [dm][hd]: quantised from N(0, 0.05) floats, or (raw) random int8 including -128 with
    random positive scales."""
    qs, ss = [], []
    for _ in range(H):
        if raw:
            q = rng.integers(-128, 128, size=(dm, hd), dtype=np.int8)
            s = rng.uniform(1e-4, 2e-3, size=(dm, hd // 32)).astype(np.float32)
        else:
            q, s = orc.q8_quantize_rows(normal(rng, (dm, hd), 0.05))
        qs.append(q)
        ss.append(s)
    return qs, ss, [ov.Q8Weight(q, s, hd, dm) for q, s in zip(qs, ss)]


def _check(y, ref, what):
    y = np.asarray(y, np.float32).reshape(ref.shape)
    bad = int(np.count_nonzero(y.view(np.uint32) != ref.view(np.uint32)))
    assert bad == 0, f"{what}: {bad}/{y.size} outputs differ from the oracle"


@pytest.mark.parametrize("H,hd,dm,rows", [
    (32, 128, 4096, 1),   # Llama-3-8B decode: quantised inside the launch
    (32, 128, 4096, 2),   # 8192 inputs: still inside
    (32, 128, 4096, 3),   # separate Q8_0 quantisation, one launch
    (32, 128, 512, 8),    # eight rows in one launch
    (32, 128, 300, 20),   # three launches (8 + 8 + 4 rows), partial last tile
    (8, 96, 100, 3),      # three blocks per head, partial tile
    (16, 256, 272, 1),    # head_dim 256: two blocks per lane
    (16, 256, 272, 5),
    (64, 128, 96, 8),     # two launches of four rows (LDS limit)
    (128, 256, 48, 2),    # 32768 inputs per row: one row per launch
    (3, 32, 17, 4),       # one block per head; five of the eight waves have no head
    (1, 128, 64, 2),      # a single head
    (33, 64, 80, 3),      # wave 0 takes five heads: two ring batches
    (12, 160, 40, 2),     # five blocks per head, two per lane: block values gathered through LDS
    (10, 192, 24, 6),     # six blocks per head
])
def test_heads_bit_exact(orc, H, hd, dm, rows):
    case("heads", H, hd, dm, rows)
    rng = np.random.default_rng(H * 7 + hd + dm + rows)
    qs, ss, ws = _heads(orc, rng, H, hd, dm)
    x = normal(rng, (rows, H * hd))
    x[0, :32] = 0.0  # an all-zero block: scale 0, quants 0
    bias = normal(rng, dm)
    for b in (None, bias):
        y = ov.project_heads_q8_0(ws, t(x), rows=rows, bias=None if b is None else t(b))
        torch.cuda.synchronize()
        ref = orc.q8_project_heads(x, rows, qs, ss, hd, dm, b)
        _check(y.cpu().numpy(), ref, f"bias={b is not None}")


@pytest.mark.parametrize("H,hd,dm,rows", [
    (32, 128, 4096, 512),  # Llama-3-8B prefill: 512 rows, 64-row MFMA tiles
    (32, 128, 4096, 32),   # the first automatic MFMA row count: 32-row tiles
    (32, 128, 1000, 33),   # 64-row tiles with a partial last tile, partial output tile
    (8, 64, 200, 40),      # two blocks per head: every group partial
    (6, 96, 72, 37),       # three blocks per head
    (4, 256, 136, 70),     # eight blocks per head: two groups per head
    (3, 160, 24, 100),     # five blocks per head: a full group and a partial one
    (1, 32, 16, 64),       # one head of one block
])
def test_heads_batched_mfma_bit_exact(orc, H, hd, dm, rows):
    case("heads mfma", H, hd, dm, rows)
    rng = np.random.default_rng(H * 11 + hd + dm + rows)
    qs, ss, ws = _heads(orc, rng, H, hd, dm)
    x = normal(rng, (rows, H * hd))
    x[rows - 1, -32:] = 0.0  # an all-zero block
    bias = normal(rng, dm)
    for b in (None, bias):
        y = ov.project_heads_q8_0(ws, t(x), rows=rows, bias=None if b is None else t(b))
        torch.cuda.synchronize()
        ref = orc.q8_project_heads(x, rows, qs, ss, hd, dm, b)
        _check(y.cpu().numpy(), ref, f"bias={b is not None}")


@pytest.mark.parametrize("kernel,rows", [("tiled", 2), ("tiled", 9), ("tiled", 17), ("rows", 20), ("small", 40)])
def test_heads_forced_kernel_bit_exact(orc, kernel, rows):
    """OVFQ_BATCHED_TILED forces the MFMA kernel down to small batches, the other choices the decode kernel's
    per-8-row launches for any batch; both stay exact."""
    case("heads forced", kernel, rows)
    ctx = ov.default_context()
    rng = np.random.default_rng(rows + len(kernel))
    H, hd, dm = 32, 128, 512
    qs, ss, ws = _heads(orc, rng, H, hd, dm)
    x = normal(rng, (rows, H * hd))
    bias = normal(rng, dm)
    ctx.set_batched_kernel(kernel)
    try:
        y = ov.project_heads_q8_0(ws, t(x), rows=rows, bias=t(bias))
        torch.cuda.synchronize()
    finally:
        ctx.set_batched_kernel("auto")
    _check(y.cpu().numpy(), orc.q8_project_heads(x, rows, qs, ss, hd, dm, bias), kernel)


def test_heads_host_entry_and_raw_planes(orc):
    """The host-pointer entry point (synchronous, staged) and int8 planes holding -128 (a GGUF Q8_0 tensor's full
    range; the reference's own quantiser stops at -127)."""
    case("heads host/raw")
    rng = np.random.default_rng(77)
    H, hd, dm, rows = 32, 128, 1024, 4
    qs, ss, ws = _heads(orc, rng, H, hd, dm, raw=True)
    x = normal(rng, (rows, H * hd))
    bias = normal(rng, dm)
    y = ov.project_heads_q8_0(ws, x, rows=rows, bias=bias)
    _check(y, orc.q8_project_heads(x, rows, qs, ss, hd, dm, bias), "host")


def test_heads_rejects_bad_arguments(orc):
    case("heads arguments")
    ctx = ov.default_context()
    lib = ctx.lib
    rng = np.random.default_rng(5)
    _, _, ws = _heads(orc, rng, 2, 128, 64)
    _, _, other = _heads(orc, rng, 1, 64, 64)
    k4 = ov.Q4KWeight(np.zeros((64, 144), np.uint8), 256, 64)
    _, _, wide = _heads(orc, rng, 1, 512, 8)
    x = torch.zeros(8 * 1024, device=DEV)
    y = torch.zeros(8 * 1024, device=DEV)

    def call(weights, n_heads=None, rows=1):
        n = len(weights) if n_heads is None else n_heads
        W = (ctypes.c_void_p * max(n, 1))(*[w.handle.value for w in weights][:max(n, 1)])
        return lib.ovfq_project_heads_q8_0_dev(ctx.handle, n, W, ctypes.c_void_p(x.data_ptr()), rows, None,
                                               ctypes.c_void_p(y.data_ptr()))

    assert call(ws, n_heads=0) == _lib.OVFQ_ERR_RANGE
    assert call(ws * 65, n_heads=129) == _lib.OVFQ_ERR_RANGE
    assert call([ws[0], other[0]]) == _lib.OVFQ_ERR_SIZE        # heads of different shapes
    assert call([ws[0], k4]) == _lib.OVFQ_ERR_TYPE              # not Q8_0
    assert call(wide) == _lib.OVFQ_ERR_SIZE                     # head_dim 512
    assert call(ws, rows=0) == _lib.OVFQ_ERR_RANGE
    assert call(ws, rows=2) == 0
    torch.cuda.synchronize()
