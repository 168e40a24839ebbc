"""Experts sliced from one 3-D GGUF expert tensor (ovfq_weight_create_experts_gguf[_dev]) against the oracle.

GgufLlamaLoader.LoadExperts (LD/GgufLlamaLoader.cs:600-690) reads ffn_{gate,up,down}_exps as [ne0 = in, ne1 = out,
ne2 = n_experts] with the expert axis slowest, so expert e is the contiguous slice e: Q4_K / Q6_K bytes verbatim,
Q8_0 de-interleaved per expert. Every sliced expert must project bit-identically to the oracle on that slice, the
routed MoE FFN over sliced experts must match the oracle's, and the shared allocation must outlive every slice but
the last (destroy order free; the context refuses to go while any slice lives).
"""
import ctypes
import gc
import sys

import numpy as np
import pytest

from qdata import (normal, q8_0_gguf_blocks, random_q4k_blocks, random_q5_blocks, random_q6k_blocks,
                   set_subnormal_scales)

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
ov = pytest.importorskip("overfit_amd")
from overfit_amd import _lib  # noqa: E402

DEV = "cuda:0"


def case(*what):
    print("[case]", *what, flush=True, file=sys.stderr)


def t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _expert_tensor(orc, rng, fmt, E, k, n):
    """E experts of [n][k] in one GGUF byte tensor (expert axis slowest) plus, per expert, what the oracle projects
    with: the K-quant blocks, or Q8_0's (quant, scale) planes after the oracle's own de-interleave."""
    slices, ref = [], []
    for _ in range(E):
        if fmt == "q4k":
            b = set_subnormal_scales(random_q4k_blocks(rng, n * (k // 256))).reshape(n, -1)
            slices.append(b.ravel())
            ref.append(b)
        elif fmt == "q6k":
            b = set_subnormal_scales(random_q6k_blocks(rng, n * (k // 256)), q6=True).reshape(n, -1)
            slices.append(b.ravel())
            ref.append(b)
        elif fmt in ("q5_0", "q5_k"):
            tid = TYPE[fmt]
            b = random_q5_blocks(rng, tid, n, k)
            slices.append(b.ravel())
            ref.append(orc.q5_requantize_q8_0(tid, b, n, k))
        else:
            q = rng.integers(-128, 128, size=(n * k // 32, 32), dtype=np.int8)
            s = rng.uniform(1e-4, 2e-2, size=n * k // 32).astype(np.float16).astype(np.float32)
            g = q8_0_gguf_blocks(s, q)
            slices.append(g.ravel())
            ref.append(orc.q8_0_deinterleave(g.reshape(-1, 34)))
    return np.concatenate(slices), ref


def _project_ref(orc, fmt, r, x, k, n):
    if fmt == "q4k":
        return orc.q4k_project(x, r, k, n)
    if fmt == "q6k":
        return orc.q6k_project(x, r, k, n)
    return orc.q8_project_batched(x, 1, r[0], r[1], k, n).ravel()


TYPE = {"q4k": 12, "q6k": 14, "q8_0": 8, "q5_0": 6, "q5_k": 13}


@pytest.mark.parametrize("fmt,E,k,n", [("q4k", 4, 512, 96), ("q6k", 5, 768, 33), ("q8_0", 3, 96, 40),
                                       ("q6k", 2, 256, 7), ("q4k", 1, 256, 1), ("q5_0", 3, 96, 40),
                                       ("q5_0", 2, 4096, 65), ("q5_k", 4, 512, 33), ("q5_k", 1, 256, 1)])
@pytest.mark.parametrize("on_device", [False, True])
def test_experts_slice_bit_exact(orc, fmt, E, k, n, on_device):
    """Each sliced expert projects exactly like the oracle on its slice (Q6_K rows of 3 super-blocks: 630-byte
    rows, slices 256-byte aligned on the device); DecodeRow reads the right slice."""
    case("experts slice", fmt, E, k, n, on_device)
    rng = np.random.default_rng(E * 100 + k + n + on_device)
    data, ref = _expert_tensor(orc, rng, fmt, E, k, n)
    ws = ov.load_gguf_experts(TYPE[fmt], t(data) if on_device else data, k, n, E)
    assert len(ws) == E
    x = normal(rng, k)
    for e, (w, r) in enumerate(zip(ws, ref)):
        y = ov.project(w, x)
        expect = _project_ref(orc, fmt, r, x, k, n)
        bad = int(np.count_nonzero(np.asarray(y, np.float32).view(np.uint32) != expect.view(np.uint32)))
        assert bad == 0, f"expert {e}: {bad}/{n} outputs differ"
    row = np.zeros(k, np.float32)
    ws[-1].DecodeRow(n - 1, row)
    if fmt in ("q8_0", "q5_0", "q5_k"):
        info = ctypes.c_int()
        assert ws[-1].context.lib.ovfq_weight_info(ws[-1].handle, ctypes.byref(info), None, None, None, None) == 0
        assert info.value == 8, "a 5-bit GGUF tensor is resident as Q8_0"
    if fmt in ("q8_0", "q5_0", "q5_k"):
        q, s = ref[-1]
        expect = q.reshape(n, k)[n - 1].astype(np.float32) * np.repeat(s.reshape(n, -1)[n - 1], 32)
    else:
        expect = (orc.q4k_decode_row if fmt == "q4k" else orc.q6k_decode_row)(ref[-1], k, n, n - 1)
    assert np.array_equal(row.view(np.uint32), np.asarray(expect, np.float32).view(np.uint32))


def test_experts_moe_ffn_and_lifetime(orc):
    """The routed MoE FFN over experts sliced from 3-D tensors equals the oracle's over the same bytes; destroying
    slices in any order keeps the survivors valid, and the context refuses to close while one lives."""
    case("experts moe + lifetime")
    rng = np.random.default_rng(404)
    E, dm, dff, rows, k = 4, 512, 768, 6, 2
    ctx = ov.Context(0)
    g_all, g_ref = _expert_tensor(orc, rng, "q4k", E, dm, dff)
    u_all, u_ref = _expert_tensor(orc, rng, "q4k", E, dm, dff)
    d_all, d_ref = _expert_tensor(orc, rng, "q6k", E, dff, dm)
    gw = ov.load_gguf_experts(12, g_all, dm, dff, E, ctx=ctx)
    uw = ov.load_gguf_experts(12, t(u_all), dm, dff, E, ctx=ctx)
    dw = ov.load_gguf_experts(14, d_all, dff, dm, E, ctx=ctx)
    x = normal(rng, (rows, dm))
    idx = np.stack([rng.permutation(E)[:k] for _ in range(rows)]).astype(np.int32)
    w = rng.uniform(0.1, 1.0, size=(rows, k)).astype(np.float32)
    ref = orc.moe_ffn_batched([b.ravel() for b in g_ref], [b.ravel() for b in u_ref], [b.ravel() for b in d_ref],
                              12, 14, x, rows, dm, dff, k, idx, w)
    y = ov.moe_ffn(gw, uw, dw, x, rows, k, idx, w)
    y = np.asarray(y, np.float32).reshape(ref.shape)
    scale = float(np.max(np.abs(ref)))
    assert float(np.max(np.abs(y.astype(np.float64) - ref))) <= 1e-3 * scale
    # destroy all but one gate slice, out of order; the survivor still projects from the shared allocation
    xv = normal(rng, dm)
    keep = gw[2]
    for i in (3, 0, 1):
        gw[i] = None
    gc.collect()
    assert np.array_equal(np.asarray(ov.project(keep, xv), np.float32).view(np.uint32),
                          orc.q4k_project(xv, g_ref[2], dm, dff).view(np.uint32))
    rc = ctx.lib.ovfq_ctx_destroy(ctx.handle)
    assert rc == _lib.OVFQ_ERR_STATE and b"destroy them first" in ctx.lib.ovfq_last_error()
    del gw, uw, dw, keep
    gc.collect()
    ctx.close()
    assert ctx.handle is None


def test_experts_rejects_bad_arguments():
    case("experts arguments")
    ctx = ov.default_context()
    lib = ctx.lib
    buf = np.zeros(4 * 144, np.uint8)
    hs = (ctypes.c_void_p * 8)()
    p = buf.ctypes.data_as(ctypes.c_void_p)
    f = lib.ovfq_weight_create_experts_gguf
    assert f(ctx.handle, 12, p, buf.size, 256, 1, 0, hs) == _lib.OVFQ_ERR_RANGE
    assert f(ctx.handle, 12, p, buf.size, 256, 1, 4097, hs) == _lib.OVFQ_ERR_RANGE
    assert f(ctx.handle, 12, p, buf.size, 256, 1, 5, hs) == _lib.OVFQ_ERR_SIZE   # 5 slices need 720 bytes
    assert f(ctx.handle, 12, p, buf.size, 255, 1, 1, hs) == _lib.OVFQ_ERR_SIZE
    assert f(ctx.handle, 2, p, buf.size, 256, 1, 1, hs) == _lib.OVFQ_ERR_TYPE    # Q4_0: not in this library
    assert f(ctx.handle, 12, None, buf.size, 256, 1, 1, hs) == _lib.OVFQ_ERR_NULL
    assert f(ctx.handle, 12, p, buf.size, 256, 1, 4, hs) == 0
    for h in hs[:4]:
        assert lib.ovfq_weight_destroy(ctypes.c_void_p(h)) == 0
