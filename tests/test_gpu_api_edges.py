"""API edges of libovfq on the device: lifetime rules, span-size bounds, the router's register top-k over many
list sizes, and HIP-graph replay after the context's scratch has grown.

Every refusal here happens in the host-side validation, before any device work (the reference throws before
work, RT/Q4KDotKernel.cs:77-97); the buffers passed with them are small and never read.
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


def vp(x):
    return ctypes.c_void_p(x.data_ptr())


def test_context_outlives_its_weights(orc):
    """ovfq_ctx_destroy refuses while a weight made on the context is alive (a weight locks its context when it is
    destroyed), and succeeds once the weights are gone."""
    case("ctx lifetime")
    ctx = ov.Context(0)
    rng = np.random.default_rng(1)
    blocks = random_q4k_blocks(rng, 4).reshape(2, -1)
    w = ov.Q4KWeight(blocks, 512, 2, ctx=ctx)
    rc = ctx.lib.ovfq_ctx_destroy(ctx.handle)
    assert rc == _lib.OVFQ_ERR_STATE and b"destroy them first" in ctx.lib.ovfq_last_error()
    x = normal(rng, 512)
    y = ov.project(w, x)  # the context is still usable
    assert np.array_equal(y.view(np.uint32), orc.q4k_project(x, blocks, 512, 2).view(np.uint32))
    del w
    import gc
    gc.collect()
    ctx.close()
    assert ctx.handle is None


def test_plane_bounds_are_refused_before_work():
    """Activation / output planes of 2^31 elements or more (the reference's Span<T> limit) are refused with
    OVFQ_ERR_SIZE by every projection entry point; the kernels' 32-bit offsets never see them."""
    ctx = ov.default_context()
    lib = ctx.lib
    rng = np.random.default_rng(2)
    k = 32768
    w = ov.Q4KWeight(random_q4k_blocks(rng, k // 256).reshape(1, -1), k, 1)
    w8 = ov.Q8Weight(np.zeros(k, np.int8), np.zeros(k // 32, np.float32), k, 1)
    buf = torch.zeros(1024, device=DEV)
    q = torch.zeros(1024, dtype=torch.int8, device=DEV)
    b = torch.zeros(1024, dtype=torch.int16, device=DEV)
    rows = 65536  # rows x 32768 = 2^31
    case("plane bounds", rows, k)
    assert lib.ovfq_project_dev(ctx.handle, w.handle, vp(buf), rows, None, vp(buf)) == _lib.OVFQ_ERR_SIZE
    assert b"exceeds 2^31" in lib.ovfq_last_error()
    assert lib.ovfq_project_dev(ctx.handle, w8.handle, vp(buf), rows, None, vp(buf)) == _lib.OVFQ_ERR_SIZE
    assert lib.ovfq_project_prequantized_dev(ctx.handle, w.handle, vp(q), vp(buf), vp(b), rows, None,
                                             vp(buf)) == _lib.OVFQ_ERR_SIZE
    assert lib.ovfq_quantize_q8k_dev(ctx.handle, vp(buf), rows, k, vp(q), vp(buf), vp(b)) == _lib.OVFQ_ERR_SIZE
    assert lib.ovfq_quantize_q8_0_dev(ctx.handle, vp(buf), rows, k, vp(q), vp(buf)) == _lib.OVFQ_ERR_SIZE
    W = (ctypes.c_void_p * 1)(w.handle.value)
    Y = (ctypes.c_void_p * 1)(buf.data_ptr())
    assert lib.ovfq_project_multi_prequantized_dev(ctx.handle, 1, W, vp(q), vp(buf), vp(b), rows, None,
                                                   Y) == _lib.OVFQ_ERR_SIZE
    # one row below the bound passes validation (not run: rows - 1 rows of 32768 would need 8 GB of input)


def test_moe_rows_and_pair_planes_are_refused_before_work():
    """ovfq_moe_ffn_dev validates rows like every other entry point (1 .. 65536) and keeps the (token, slot) pair
    planes (pairs x d_ff of gate/up outputs and of the Q8_K intermediate) below 2^31 elements."""
    ctx = ov.default_context()
    lib = ctx.lib
    rng = np.random.default_rng(3)
    E, dm, dff = 2, 256, 16384
    gate = [ov.Q4KWeight(random_q4k_blocks(rng, dff).reshape(dff, -1), dm, dff) for _ in range(E)]
    up = [ov.Q4KWeight(random_q4k_blocks(rng, dff).reshape(dff, -1), dm, dff) for _ in range(E)]
    down = [ov.Q6KWeight(random_q6k_blocks(rng, dm * dff // 256).reshape(dm, -1), dff, dm) for _ in range(E)]
    G, U, D = [(ctypes.c_void_p * E)(*[x.handle.value for x in ws]) for ws in (gate, up, down)]
    buf = torch.zeros(1024, device=DEV)
    idx = torch.zeros(1024, dtype=torch.int32, device=DEV)
    for rows, k, want in [(0, 1, _lib.OVFQ_ERR_RANGE), (65537, 1, _lib.OVFQ_ERR_RANGE),
                          (65536, 2, _lib.OVFQ_ERR_SIZE)]:
        case("moe bounds", rows, k)
        rc = lib.ovfq_moe_ffn_dev(ctx.handle, E, G, U, D, vp(buf), rows, k, vp(idx), vp(buf), vp(buf))
        assert rc == want, (rows, k, rc, lib.ovfq_last_error())


@pytest.mark.parametrize("E,k", [(8, 1), (8, 2), (8, 3), (16, 4), (16, 5), (60, 8), (64, 9), (64, 16), (64, 17),
                                 (40, 33), (64, 64)])
@pytest.mark.parametrize("normalize", [True, False])
def test_topk_register_list_every_size(orc, E, k, normalize):
    """MoeRouter.SelectTopK for list sizes across every compiled bucket (2, 4, 8, 16 and the 64-entry list), with
    ties (the lower index wins) and -inf logits: indices exact, weights within a few ULP (expf)."""
    case("topk", E, k, normalize)
    rng = np.random.default_rng(E * 100 + k)
    rows = 70
    logits = (rng.integers(0, 12, size=(rows, E)) / 4.0).astype(np.float32)  # many ties
    logits[5, :] = -np.inf
    logits[6, : E // 2] = -np.inf
    logits[7] = rng.standard_normal(E).astype(np.float32)
    idx = torch.full((rows * k,), -9, dtype=torch.int32, device=DEV)
    w = torch.zeros(rows * k, dtype=torch.float32, device=DEV)
    assert ov.MoeRouter.SelectTopK(t(logits), k, idx, w, normalize, rows=rows) == min(k, E)
    torch.cuda.synchronize()
    gi, gw = idx.cpu().numpy(), w.cpu().numpy()
    for n in range(rows):
        ri, rw = orc.moe_select_topk(logits[n], k, normalize)
        assert np.array_equal(gi[n * k:(n + 1) * k], ri), n
        np.testing.assert_allclose(gw[n * k:(n + 1) * k], rw, rtol=4e-7, atol=0, err_msg=str(n))


def test_graph_replay_after_scratch_growth(orc):
    """A graph captured from _dev calls at one size keeps the scratch addresses it was recorded with. A larger eager
    call afterwards grows the context's scratch; the superseded buffers stay allocated, so later replays still
    reproduce the eager outputs bit-for-bit (and the larger call is itself exact)."""
    case("graph replay after growth")
    ctx = ov.Context(0)
    rng = np.random.default_rng(21)
    k, n, k2 = 4096, 256, 14336
    bq = random_q4k_blocks(rng, n * k // 256).reshape(n, -1)
    bd = random_q6k_blocks(rng, n * k2 // 256).reshape(n, -1)
    wq = ov.Q4KWeight(bq, k, n, ctx=ctx)
    wd = ov.Q6KWeight(bd, k2, n, ctx=ctx)
    x1 = t(normal(rng, (40, k)))   # batched: quantised into the context scratch
    x2 = t(normal(rng, (1, k2)))   # long decode row: quantised into the context scratch
    ys = [torch.empty(40 * n, device=DEV), torch.empty(n, device=DEV)]

    def step():
        ctx.project_dev(wq, x1, ys[0], rows=40)
        ctx.project_dev(wd, x2, ys[1], rows=1)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        ctx.set_stream(side.cuda_stream)
        step()
        side.synchronize()
        eager = [y.cpu().numpy().copy() for y in ys]
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=side):
            step()
    ctx.set_stream(torch.cuda.current_stream().cuda_stream)
    big_rows = 300
    xb = normal(rng, (big_rows, k2))
    yb = torch.empty(big_rows * n, device=DEV)
    for rep in range(3):
        # a larger eager call each time: grows the activation scratch past what the graph was captured with
        rows = big_rows if rep == 0 else big_rows // (rep + 1)
        ctx.project_dev(wd, t(xb[:rows]), yb, rows=rows)
        torch.cuda.synchronize()
        if rep == 0:
            ref = orc.q6k_project_batched(xb[:rows], rows, bd, k2, n, None)
            got = yb[: rows * n].cpu().numpy()
            assert np.array_equal(got.view(np.uint32), ref.reshape(-1).view(np.uint32)), "large eager call"
        for y in ys:
            y.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        for y, e in zip(ys, eager):
            assert np.array_equal(y.cpu().numpy().view(np.uint32), e.view(np.uint32)), f"replay {rep}"
    del g
    # With the graph gone the superseded scratch can be given back: device memory is freed, and the context's
    # calls stay exact on the buffers it keeps.
    torch.cuda.synchronize()
    live0, retired0 = ctx.scratch_bytes()
    assert retired0 > 0 and live0 > 0
    free0 = torch.cuda.mem_get_info()[0]
    ctx.release_retired()
    free1 = torch.cuda.mem_get_info()[0]
    assert ctx.scratch_bytes() == (live0, 0), "release_retired left superseded scratch"
    assert free1 >= free0  # the runtime may keep small freed blocks in its own pool
    ctx.release_retired()  # nothing left to free
    rows = big_rows // 3
    ctx.project_dev(wd, t(xb[:rows]), yb, rows=rows)
    ref = orc.q6k_project_batched(xb[:rows], rows, bd, k2, n, None)
    assert np.array_equal(yb[: rows * n].cpu().numpy().view(np.uint32), ref.reshape(-1).view(np.uint32))
    del wq, wd
    import gc
    gc.collect()
    ctx.close()


def test_moe_ffn_dev_into_host_mapped_output(orc):
    """ovfq_moe_ffn_dev with top-2 routing folds the combine into float atomics on y only when y is device
    memory; a y in pinned (host-mapped) memory takes the combine launch. Both give the same bits."""
    case("moe dev host-mapped y")
    rng = np.random.default_rng(33)
    E, dm, dff, rows, k = 4, 256, 512, 6, 2
    ctx = ov.default_context()
    mk = lambda n, kk: ov.Q4KWeight(random_q4k_blocks(rng, n * kk // 256).reshape(n, -1), kk, n)
    gate = [mk(dff, dm) for _ in range(E)]
    up = [mk(dff, dm) for _ in range(E)]
    down = [mk(dm, dff) for _ in range(E)]
    x = t(normal(rng, (rows, dm)))
    idx = t(np.stack([rng.permutation(E)[:k] for _ in range(rows)]).astype(np.int32))
    wts = t(rng.random((rows, k)).astype(np.float32))
    y_dev = torch.full((rows * dm,), float("nan"), device=DEV)
    y_host = torch.full((rows * dm,), float("nan")).pin_memory()
    arr = lambda ws: (ctypes.c_void_p * E)(*[w.handle.value for w in ws])
    for y in (y_dev, y_host):
        rc = ctx.lib.ovfq_moe_ffn_dev(ctx.handle, E, arr(gate), arr(up), arr(down), vp(x), rows, k, vp(idx), vp(wts),
                                      ctypes.c_void_p(y.data_ptr()))
        assert rc == 0, ctx.lib.ovfq_last_error()
    torch.cuda.synchronize()
    a = y_dev.cpu().numpy().view(np.uint32)
    b = y_host.numpy().view(np.uint32)
    assert np.array_equal(a, b), "host-mapped output differs from the device output"
    assert not np.isnan(y_host.numpy()).any()


def test_reset_stream_and_swiglu_dev(orc):
    """ovfq_ffn_swiglu_dev equals ovfq_ffn_gated_dev with OVFQ_FFN_SWIGLU bit for bit, on a stream bound with
    ovfq_ctx_set_stream and again after ovfq_ctx_reset_stream returns the context to its own stream (whose work
    ovfq_ctx_synchronize then waits for)."""
    case("reset stream + swiglu dev")
    rng = np.random.default_rng(71)
    dm, dff, rows = 256, 512, 3
    ctx = ov.Context(0)
    gate = ov.Q4KWeight(random_q4k_blocks(rng, dff * dm // 256).reshape(dff, -1), dm, dff, ctx=ctx)
    up = ov.Q4KWeight(random_q4k_blocks(rng, dff * dm // 256).reshape(dff, -1), dm, dff, ctx=ctx)
    down = ov.Q6KWeight(random_q6k_blocks(rng, dm * dff // 256).reshape(dm, -1), dff, dm, ctx=ctx)
    x = t(normal(rng, (rows, dm)))
    lib = ctx.lib
    ys = [torch.empty(rows * dm, device=DEV) for _ in range(3)]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        ctx.set_stream(side.cuda_stream)
        assert lib.ovfq_ffn_swiglu_dev(ctx.handle, gate.handle, up.handle, down.handle, vp(x), rows, vp(ys[0])) == 0
        assert lib.ovfq_ffn_gated_dev(ctx.handle, gate.handle, up.handle, down.handle, vp(x), rows,
                                      _lib.OVFQ_FFN_SWIGLU, vp(ys[1])) == 0
        side.synchronize()
    assert lib.ovfq_ctx_reset_stream(ctx.handle) == 0
    torch.cuda.synchronize()
    assert lib.ovfq_ffn_swiglu_dev(ctx.handle, gate.handle, up.handle, down.handle, vp(x), rows, vp(ys[2])) == 0
    assert lib.ovfq_ctx_synchronize(ctx.handle) == 0
    a, b, c = (y.cpu().numpy().view(np.uint32) for y in ys)
    assert np.array_equal(a, b), "swiglu_dev differs from gated_dev(SWIGLU)"
    assert np.array_equal(a, c), "result on the context's own stream differs"
    del gate, up, down
    import gc
    gc.collect()
    ctx.close()
