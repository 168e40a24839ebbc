"""Parity of the device path (libovfq through its C ABI) with the oracle on identical seeded inputs.

The bar is bit-exactness everywhere: integer dequant and block integer dots are exact by construction, and
the fp32 tail and the per-row super-block sum are evaluated in the reference's order, so every output float
must equal the oracle's. The north-star tolerance (max relative error 1e-3, cosine >= 0.99999) is reported
alongside as the outer bound.
"""
import ctypes
import sys

import numpy as np
import pytest

from qdata import (Q8_0_KATS, normal, q8_0_gguf_blocks, random_q4k_blocks, random_q5_blocks, random_q6k_blocks,
                   set_subnormal_scales)

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
ov = pytest.importorskip("overfit_amd")
from overfit_amd import _lib  # noqa: E402

DEV = "cuda:0"


def case(*what):
    print("[case]", *what, flush=True, file=sys.stderr)


def north_star(y, ref):
    y64, r64 = y.astype(np.float64).ravel(), ref.astype(np.float64).ravel()
    denom = np.maximum(np.abs(r64), 1e-30)
    rel = float(np.max(np.abs(y64 - r64) / denom)) if r64.size else 0.0
    cos = float(np.dot(y64, r64) / (np.linalg.norm(y64) * np.linalg.norm(r64) + 1e-300))
    return rel, cos


def assert_bit_exact(y, ref, what):
    y = np.asarray(y, np.float32).reshape(ref.shape)
    if not np.array_equal(y.view(np.uint32), ref.astype(np.float32).view(np.uint32)):
        rel, cos = north_star(y, ref)
        bad = int(np.count_nonzero(y.view(np.uint32) != ref.astype(np.float32).view(np.uint32)))
        pytest.fail(f"{what}: {bad}/{y.size} outputs differ from the oracle (max rel {rel:.3e}, cos {cos:.8f})")


def t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


@pytest.fixture(scope="module")
def ctx():
    return ov.default_context()


@pytest.fixture
def batched(ctx):
    """Forces the batched K-quant kernel ("small" / "tiled") for one test; automatic again afterwards."""
    yield ctx.set_batched_kernel
    ctx.set_batched_kernel("auto")


def test_batched_kernel_choice_rejects_unknown(ctx):
    with pytest.raises(ValueError):
        ctx.set_batched_kernel("fast")
    assert ctx.lib.ovfq_ctx_set_batched_kernel(ctx.handle, 4) == _lib.OVFQ_ERR_RANGE


# ------------------------------------------------------------------------------------------------ quantizers

@pytest.mark.parametrize("rows,k", [(1, 256), (3, 4096), (2, 14336), (7, 512), (5, 256), (512, 4096)])
def test_quantize_q8k_bit_exact(orc, ctx, rows, k):
    case("quantize_q8k", rows, k)
    rng = np.random.default_rng(rows * 1000 + k)
    x = normal(rng, (rows, k))
    x[0, :256] = 0.0                                    # all-zero block -> scale 0, quants 0
    if k >= 512:
        x[0, 256:512] = 0.0
        x[0, 256] = 127.0
        x[0, 257:265] = [2.5, 3.5, -2.5, -3.5, 0.5, -0.5, 1.5, 126.5]  # ties to even
    if rows > 1:
        x[1] *= 1e-30                                   # tiny values
    q, s, b = (torch.empty(rows * k, dtype=torch.int8, device=DEV),
               torch.empty(rows * k // 256, dtype=torch.float32, device=DEV),
               torch.empty(rows * k // 16, dtype=torch.int16, device=DEV))
    ctx.quantize_q8k_dev(t(x), rows, k, q, s, b)
    rq, rd, rb = orc.quantize_q8k(x)
    torch.cuda.synchronize()
    assert np.array_equal(q.cpu().numpy(), rq.reshape(-1))
    assert np.array_equal(s.cpu().numpy().view(np.uint32), rd.reshape(-1).view(np.uint32))
    assert np.array_equal(b.cpu().numpy(), rb.reshape(-1))


def test_quantize_q8k_host_api_and_mirror(orc):
    case("QuantizeActivationQ8K host")
    rng = np.random.default_rng(5)
    x = normal(rng, 1024)
    q, s, b = np.zeros(1024, np.int8), np.zeros(4, np.float32), np.zeros(64, np.int16)
    ov.Q4KDotKernel.QuantizeActivationQ8K(x, q, s, b)
    rq, rd, rb = orc.quantize_q8k(x)
    assert np.array_equal(q, rq[0]) and np.array_equal(s, rd[0]) and np.array_equal(b, rb[0])


@pytest.mark.parametrize("k", [32, 128, 4096])
def test_quantize_q8_0_bit_exact(orc, k):
    case("quantize_q8_0", k)
    rng = np.random.default_rng(k)
    x = normal(rng, (3, k))
    x[1, :32] = 0.0
    q, s = np.zeros(3 * k, np.int8), np.zeros(3 * k // 32, np.float32)
    for r in range(3):
        ov.Q8DotKernel.Quantize(x[r], q[r * k:(r + 1) * k], s[r * k // 32:(r + 1) * k // 32])
    rq, rs = orc.quantize_q8_0(x)
    assert np.array_equal(q, rq.reshape(-1)) and np.array_equal(s, rs.reshape(-1))


# ------------------------------------------------------------------------------------------------ encoders

@pytest.mark.parametrize("fmt", ["q4k", "q6k"])
@pytest.mark.parametrize("n,k", [(8, 512), (64, 4096), (3, 14336)])
def test_weight_encoder_bit_exact(orc, fmt, n, k):
    case("encode", fmt, n, k)
    rng = np.random.default_rng(n * 7 + k)
    w = normal(rng, (n, k), 0.02)
    w[0, :256] = 0.37                    # constant block (GgmlQuantTests.cs:88-108)
    w[1, :256] = 0.0                     # zero block
    w[2 % n, 256:512] = -np.abs(w[2 % n, 256:512])  # all-negative block (lo < 0, hi < 0)
    ref = orc.quantize_q4k(w) if fmt == "q4k" else orc.quantize_q6k(w)
    got = ov.quantize_weight(t(w), ov.TYPE_Q4_K if fmt == "q4k" else ov.TYPE_Q6_K)
    torch.cuda.synchronize()
    assert np.array_equal(got.cpu().numpy(), ref.reshape(-1))


def test_q8_0_weight_quantize_rows(orc):
    case("Q8Weight.QuantizeRows")
    rng = np.random.default_rng(3)
    w = normal(rng, (50, 256), 0.05)
    q, s = ov.quantize_weight(t(w), ov.TYPE_Q8_0)
    rq, rs = orc.q8_quantize_rows(w)
    torch.cuda.synchronize()
    assert np.array_equal(q.cpu().numpy(), rq.reshape(-1)) and np.array_equal(s.cpu().numpy(), rs.reshape(-1))


# ------------------------------------------------------------------------------------------------ projections

# Rows of 7, 21, 24 and 56 super-blocks: 16-block decode chunks that do not fill the row (the last one partial).
KQ_SHAPES = [(256, 1), (256, 7), (512, 96), (1024, 33), (4096, 129), (4096, 1024), (14336, 65), (3072, 4099),
             (1792, 5), (5376, 9), (6144, 31)]


def _kq_blocks(rng, fmt, n, k):
    if fmt == "q4k":
        return set_subnormal_scales(random_q4k_blocks(rng, n * (k // 256))).reshape(n, -1)
    return set_subnormal_scales(random_q6k_blocks(rng, n * (k // 256)), q6=True).reshape(n, -1)


@pytest.mark.parametrize("fmt", ["q4k", "q6k"])
@pytest.mark.parametrize("k,n", KQ_SHAPES)
@pytest.mark.parametrize("with_bias", [False, True])
def test_kquant_project_bit_exact(orc, ctx, fmt, k, n, with_bias):
    case("project", fmt, k, n, with_bias)
    rng = np.random.default_rng(k * 31 + n + with_bias)
    blocks = _kq_blocks(rng, fmt, n, k)
    x = normal(rng, k)
    bias = normal(rng, n) if with_bias else None
    W = ov.Q4KWeight if fmt == "q4k" else ov.Q6KWeight
    w = W(blocks, k, n)
    ref = (orc.q4k_project if fmt == "q4k" else orc.q6k_project)(x, blocks, k, n, bias)
    # device pointers
    yd = ov.project(w, t(x), None if bias is None else t(bias))
    torch.cuda.synchronize()
    assert_bit_exact(yd.cpu().numpy(), ref, f"{fmt} {k}x{n} device")
    # host pointers (synchronous entry point)
    assert_bit_exact(ov.project(w, x, bias), ref, f"{fmt} {k}x{n} host")


# "auto" at 97 and 512 rows over 96 outputs: the automatic choice takes the tiled kernel for its small grid once the
# small-M kernel would make 6 (Q4_K) / 7 (Q6_K) passes of 16 rows.
@pytest.mark.parametrize("kernel", ["small", "tiled", "rows", "auto"])
@pytest.mark.parametrize("fmt", ["q4k", "q6k"])
@pytest.mark.parametrize("rows", [2, 3, 8, 16, 17, 70, 97, 512])
def test_kquant_batched_bit_exact(orc, batched, kernel, fmt, rows):
    case("batched", kernel, fmt, rows)
    batched(kernel)
    rng = np.random.default_rng(rows * 13)
    k, n = 1024, 96
    blocks = _kq_blocks(rng, fmt, n, k)
    x = normal(rng, (rows, k))
    bias = normal(rng, n)
    w = (ov.Q4KWeight if fmt == "q4k" else ov.Q6KWeight)(blocks, k, n)
    ref = (orc.q4k_project_batched if fmt == "q4k" else orc.q6k_project_batched)(x, rows, blocks, k, n, bias)
    if fmt == "q4k":
        assert np.array_equal(ref, orc.q4k_project_batched_ws(x, rows, blocks, k, n, bias))
    y = ov.project(w, x, bias, rows=rows).reshape(rows, n)
    assert_bit_exact(y, ref, f"{fmt} batched rows={rows}")


# ------------------------------------------------------------------------------------------------ prefill (MFMA)

# Both batched int8-MFMA kernels on every shape (the 64-row-tiled one and the small-M one, forced): partial
# activation tiles (17, 24, 33, 70, 200), partial 64-row weight tiles (n = 130, 200, 1000), an odd super-block
# count (k = 2304: Q6_K rows only 2-byte aligned), one super-block.
PREFILL_SHAPES = [(17, 512, 200), (24, 1024, 64), (32, 256, 64), (33, 768, 1000), (64, 1024, 96), (70, 512, 200),
                  (128, 4096, 130), (200, 2304, 64)]


@pytest.mark.parametrize("kernel", ["tiled", "small"])
@pytest.mark.parametrize("fmt", ["q4k", "q6k"])
@pytest.mark.parametrize("rows,k,n", PREFILL_SHAPES)
def test_kquant_prefill_bit_exact(orc, ctx, batched, kernel, fmt, rows, k, n):
    case("prefill", kernel, fmt, rows, k, n)
    batched(kernel)
    rng = np.random.default_rng(rows * 7 + k + n)
    blocks = _kq_blocks(rng, fmt, n, k)
    x = normal(rng, (rows, k))
    bias = normal(rng, n)
    w = (ov.Q4KWeight if fmt == "q4k" else ov.Q6KWeight)(blocks, k, n)
    batched = orc.q4k_project_batched if fmt == "q4k" else orc.q6k_project_batched
    ref = batched(x, rows, blocks, k, n, bias)
    yd = ov.project(w, t(x), t(bias), rows=rows)
    torch.cuda.synchronize()
    assert_bit_exact(yd.cpu().numpy().reshape(rows, n), ref, f"{fmt} prefill {rows}x{k}x{n} device")
    ref0 = batched(x, rows, blocks, k, n, None)
    assert_bit_exact(ov.project(w, x, None, rows=rows).reshape(rows, n), ref0, f"{fmt} prefill host, no bias")


@pytest.mark.parametrize("fmt", ["q4k", "q6k"])
def test_kquant_prefill_128_row_tiles(orc, ctx, fmt):
    """From 1024 rows the tiled kernel stages 128 activation rows per workgroup: 1100 rows (a partial last tile),
    130 outputs (a partial 64-row weight tile), with a bias, before and after the MFMA-ready copy (Q6_K)."""
    case("prefill 128-row tiles", fmt)
    rows, k, n = 1100, 512, 130
    rng = np.random.default_rng(1100)
    blocks = _kq_blocks(rng, fmt, n, k)
    x = normal(rng, (rows, k))
    bias = normal(rng, n)
    w = (ov.Q4KWeight if fmt == "q4k" else ov.Q6KWeight)(blocks, k, n)
    ref = (orc.q4k_project_batched if fmt == "q4k" else orc.q6k_project_batched)(x, rows, blocks, k, n, bias)
    for prepared in (False, True):
        if prepared:
            w.prepare_mfma()
        yd = ov.project(w, t(x), t(bias), rows=rows)
        torch.cuda.synchronize()
        assert_bit_exact(yd.cpu().numpy().reshape(rows, n), ref, f"{fmt} 1100 rows prepared={prepared}")


@pytest.mark.parametrize("rows,k,shapes", [(200, 512, [14300]), (129, 256, [14336]), (300, 256, [9000, 9000])])
def test_kquant_prefill_wide_tiles(orc, ctx, rows, k, shapes):
    """Q4_K launches whose 128-row grid reaches 448 workgroups take the wide tiled kernel (128 activation rows per
    workgroup in two 64-row LDS halves): ragged last activation tiles (200, 129 and 300 rows), a partial last 64-row
    weight tile, a fused pair, a bias; from the fp32 input (the quantiser's fp16 bsums) and from a prequantised
    activation whose bsums are not the group sums (the caller's int16 bsums read as the reference's Dot does)."""
    case("prefill wide tiles", rows, k, shapes)
    rng = np.random.default_rng(rows * 13 + k + sum(shapes))
    blocks = [_kq_blocks(rng, "q4k", n, k) for n in shapes]
    ws = [ov.Q4KWeight(b, k, n) for b, n in zip(blocks, shapes)]
    x = normal(rng, (rows, k))
    bias = normal(rng, shapes[-1])
    biases = [None] * (len(shapes) - 1) + [bias]
    refs = [orc.q4k_project_batched(x, rows, b, k, n, bb) for b, n, bb in zip(blocks, shapes, biases)]
    ys = [torch.empty(rows * n, device=DEV) for n in shapes]
    ctx.project_multi_dev(ws, t(x), ys, [None if bb is None else t(bb) for bb in biases], rows=rows)
    torch.cuda.synchronize()
    for i, (y, ref) in enumerate(zip(ys, refs)):
        assert_bit_exact(y.cpu().numpy().reshape(rows, -1), ref, f"wide tiles rows={rows} job {i}")
    q, s, b = orc.quantize_q8k(x)
    b = (b.astype(np.int32) + rng.integers(-9, 10, b.shape)).clip(-2048, 2048).astype(np.int16)
    L = orc.lib()
    ref = np.zeros((rows, shapes[0]), np.float32)
    rc = L.orc_q4k_project_batched_prequantized(rows, orc.P(np.ascontiguousarray(blocks[0], np.uint8)), k,
                                                 shapes[0], None, orc.P(ref), orc.P(q), orc.P(s), orc.P(b))
    assert rc == 0
    y = torch.empty(rows * shapes[0], device=DEV)
    ctx.project_prequantized_dev(ws[0], t(q), t(s), t(b), y, rows=rows)
    torch.cuda.synchronize()
    assert_bit_exact(y.cpu().numpy().reshape(rows, -1), ref, f"wide tiles prequantized shifted bsums rows={rows}")


@pytest.mark.parametrize("fmt,rows,k,shapes", [("q6k", 200, 768, [260]), ("q6k", 130, 3328, [250]),
                                               ("q4k", 256, 768, [4096, 1024, 1000]), ("q4k", 500, 1280, [4000])])
def test_kquant_prefill_pair_kernel(orc, ctx, fmt, rows, k, shapes):
    """Launches whose 64-row grid leaves each CU one or two tiles take the pair kernel (two waves per 16 weight rows
    on alternate super-blocks, the odd wave's block values added by the even one in ascending order): an odd number of
    super-blocks (3, 5: the last has no partner), partial weight and activation tiles, a multi-job launch, a bias; from
    the fp32 input and, for Q4_K, a prequantised activation whose bsums are not the group sums."""
    case("prefill pair kernel", fmt, rows, k, shapes)
    rng = np.random.default_rng(rows * 17 + k + sum(shapes))
    blocks = [_kq_blocks(rng, fmt, n, k) for n in shapes]
    Wt = ov.Q4KWeight if fmt == "q4k" else ov.Q6KWeight
    ws = [Wt(b, k, n) for b, n in zip(blocks, shapes)]
    x = normal(rng, (rows, k))
    bias = normal(rng, shapes[-1])
    biases = [None] * (len(shapes) - 1) + [bias]
    proj = orc.q4k_project_batched if fmt == "q4k" else orc.q6k_project_batched
    refs = [proj(x, rows, b, k, n, bb) for b, n, bb in zip(blocks, shapes, biases)]
    ys = [torch.empty(rows * n, device=DEV) for n in shapes]
    ctx.project_multi_dev(ws, t(x), ys, [None if bb is None else t(bb) for bb in biases], rows=rows)
    torch.cuda.synchronize()
    for i, (y, ref) in enumerate(zip(ys, refs)):
        assert_bit_exact(y.cpu().numpy().reshape(rows, -1), ref, f"pair kernel {fmt} rows={rows} job {i}")
    if fmt != "q4k":
        return
    q, s, b = orc.quantize_q8k(x)
    b = (b.astype(np.int32) + rng.integers(-9, 10, b.shape)).clip(-2048, 2048).astype(np.int16)
    ref = np.zeros((rows, shapes[0]), np.float32)
    rc = orc.lib().orc_q4k_project_batched_prequantized(rows, orc.P(np.ascontiguousarray(blocks[0], np.uint8)), k,
                                                         shapes[0], None, orc.P(ref), orc.P(q), orc.P(s), orc.P(b))
    assert rc == 0
    y = torch.empty(rows * shapes[0], device=DEV)
    ctx.project_prequantized_dev(ws[0], t(q), t(s), t(b), y, rows=rows)
    torch.cuda.synchronize()
    assert_bit_exact(y.cpu().numpy().reshape(rows, -1), ref, f"pair kernel prequantized shifted bsums rows={rows}")


@pytest.mark.parametrize("rows,k,shapes", [(512, 768, [4096]), (400, 1280, [3000, 1000]), (420, 512, [4000])])
def test_kquant_prefill_pairwide_kernel(orc, ctx, rows, k, shapes):
    """Q6_K launches whose 128-row grid gives about one workgroup per CU take the pair-wide kernel (8-wave workgroups
    on 64 weight rows x 128 activation rows, alternate super-blocks per wave pair, each wave over both 64-row
    halves, the odd values handed over per half): an odd number of super-blocks (3, 5), ragged activation and weight
    tiles, a two-job launch, a bias."""
    case("prefill pair-wide kernel", rows, k, shapes)
    rng = np.random.default_rng(rows * 19 + k + sum(shapes))
    blocks = [_kq_blocks(rng, "q6k", n, k) for n in shapes]
    ws = [ov.Q6KWeight(b, k, n) for b, n in zip(blocks, shapes)]
    x = normal(rng, (rows, k))
    bias = normal(rng, shapes[-1])
    biases = [None] * (len(shapes) - 1) + [bias]
    refs = [orc.q6k_project_batched(x, rows, b, k, n, bb) for b, n, bb in zip(blocks, shapes, biases)]
    ys = [torch.empty(rows * n, device=DEV) for n in shapes]
    ctx.project_multi_dev(ws, t(x), ys, [None if bb is None else t(bb) for bb in biases], rows=rows)
    torch.cuda.synchronize()
    for i, (y, ref) in enumerate(zip(ys, refs)):
        assert_bit_exact(y.cpu().numpy().reshape(rows, -1), ref, f"pair-wide kernel rows={rows} job {i}")


@pytest.mark.parametrize("fmt", ["q4k", "q6k"])
@pytest.mark.parametrize("rows,k,n", [(32, 256, 64), (70, 512, 200), (128, 4096, 130), (200, 2304, 64)])
def test_prepared_mfma_prefill_bit_exact(orc, ctx, batched, fmt, rows, k, n):
    """The opt-in MFMA-ready copy (ovfq_weight_prepare_mfma; Q6_K, a no-op for Q4_K): batched projections on the
    tiled kernel read the prepared operands and stay bit-exact (n not a multiple of 64: the last tile's absent
    rows), before and after preparing, repeatedly."""
    case("prepared prefill", fmt, rows, k, n)
    batched("tiled")
    rng = np.random.default_rng(rows * 11 + k + n)
    blocks = _kq_blocks(rng, fmt, n, k)
    x = normal(rng, (rows, k))
    bias = normal(rng, n)
    w = (ov.Q4KWeight if fmt == "q4k" else ov.Q6KWeight)(blocks, k, n)
    batched = orc.q4k_project_batched if fmt == "q4k" else orc.q6k_project_batched
    ref = batched(x, rows, blocks, k, n, bias)
    assert_bit_exact(ov.project(w, x, bias, rows=rows).reshape(rows, n), ref, f"{fmt} {rows}x{k}x{n} unprepared")
    assert w.prepare_mfma() is w
    w.prepare_mfma()  # idempotent
    for rep in range(2):
        yd = ov.project(w, t(x), t(bias), rows=rows)
        torch.cuda.synchronize()
        assert_bit_exact(yd.cpu().numpy().reshape(rows, n), ref, f"{fmt} {rows}x{k}x{n} prepared rep {rep}")


def test_prepared_mfma_multi_job_and_mixed(orc, ctx, batched):
    """A fused q/k/v-style launch of Q6_K weights over M = 48 rows on the tiled kernel with every weight prepared
    (the prepared kernel variant), with one weight unprepared (the GGUF-operand variant for the whole launch), and
    Q8_0 rejected."""
    case("prepared multi", 48)
    batched("tiled")
    rng = np.random.default_rng(48)
    rows, k, shapes = 48, 1024, [192, 64, 80]
    blocks = [_kq_blocks(rng, "q6k", n, k) for n in shapes]
    x = normal(rng, (rows, k))
    refs = [orc.q6k_project_batched(x, rows, b, k, n, None) for b, n in zip(blocks, shapes)]
    for prepared in ([0, 1, 2], [0, 2]):
        ws = [ov.Q6KWeight(b, k, n) for b, n in zip(blocks, shapes)]
        for i in prepared:
            ws[i].prepare_mfma()
        ys = [torch.empty(rows * n, device=DEV) for n in shapes]
        ctx.project_multi_dev(ws, t(x), ys, rows=rows)
        torch.cuda.synchronize()
        for i, (y, ref) in enumerate(zip(ys, refs)):
            assert_bit_exact(y.cpu().numpy().reshape(rows, -1), ref, f"prepared {prepared} job {i}")
    wq, wsc = orc.q8_quantize_rows(normal(rng, (8, 64), 0.05))
    with pytest.raises(ov.OverfitArgumentError):
        ov.Q8Weight(wq, wsc, 64, 8).prepare_mfma()


@pytest.mark.parametrize("rows,kernel", [(5, "auto"), (40, "tiled"), (40, "small")])
def test_multi_projection_rows_bit_exact(orc, ctx, batched, rows, kernel):
    """Fused q/k/v-style launch over `rows` activation rows (the tiled kernel's multi-job grid, or the small-M
    kernel per weight), from the fp32 input and from a shared prequantised activation."""
    case("multi rows", rows, kernel)
    batched(kernel)
    rng = np.random.default_rng(400 + rows)
    k, shapes = 1024, [192, 64, 80]
    blocks = [_kq_blocks(rng, "q4k", n, k) for n in shapes]
    ws = [ov.Q4KWeight(b, k, n) for b, n in zip(blocks, shapes)]
    x = normal(rng, (rows, k))
    bias = normal(rng, shapes[2])
    refs = [orc.q4k_project_batched(x, rows, b, k, n, bias if i == 2 else None)
            for i, (b, n) in enumerate(zip(blocks, shapes))]
    ys = [torch.empty(rows * n, device=DEV) for n in shapes]
    ctx.project_multi_dev(ws, t(x), ys, [None, None, t(bias)], rows=rows)
    torch.cuda.synchronize()
    for i, (y, ref) in enumerate(zip(ys, refs)):
        assert_bit_exact(y.cpu().numpy().reshape(rows, -1), ref, f"multi rows={rows} job {i}")
    q = torch.empty(rows * k, dtype=torch.int8, device=DEV)
    s = torch.empty(rows * k // 256, dtype=torch.float32, device=DEV)
    b = torch.empty(rows * k // 16, dtype=torch.int16, device=DEV)
    ctx.quantize_q8k_dev(t(x), rows, k, q, s, b)
    ys2 = [torch.empty(rows * n, device=DEV) for n in shapes]
    ctx.project_multi_prequantized_dev(ws, q, s, b, ys2, [None, None, t(bias)], rows=rows)
    torch.cuda.synchronize()
    for i, (y, ref) in enumerate(zip(ys2, refs)):
        assert_bit_exact(y.cpu().numpy().reshape(rows, -1), ref, f"multi prequantized rows={rows} job {i}")


@pytest.mark.parametrize("rows,kernel", [(4, "auto"), (40, "tiled")])
def test_prequantized_bsums_read_as_reference(orc, ctx, batched, rows, kernel):
    """The decode kernel (up to 8 rows) and the tiled Q4_K MFMA kernel take the min term from the caller's bsums, as
    the reference's Dot does (RT/Q4KDotKernel.cs:249-253): with bsums that are not the group sums (every group
    shifted, within the fp16-exact range |b| <= 2048), both match the oracle's prequantised batched projection
    bit for bit."""
    case("prequantized bsums", rows, kernel)
    batched(kernel)
    rng = np.random.default_rng(700 + rows)
    k, n = 1024, 128
    blocks = _kq_blocks(rng, "q4k", n, k)
    w = ov.Q4KWeight(blocks, k, n)
    x = normal(rng, (rows, k))
    q, s, b = orc.quantize_q8k(x)
    b = (b.astype(np.int32) + rng.integers(-9, 10, b.shape)).clip(-2048, 2048).astype(np.int16)
    ref = np.zeros((rows, n), np.float32)
    L = orc.lib()
    rc = L.orc_q4k_project_batched_prequantized(rows, orc.P(np.ascontiguousarray(blocks, np.uint8)), k, n, None,
                                                 orc.P(ref), orc.P(q), orc.P(s), orc.P(b))
    assert rc == 0
    y = torch.empty(rows * n, device=DEV)
    ctx.project_prequantized_dev(w, t(q), t(s), t(b), y, rows=rows)
    torch.cuda.synchronize()
    assert_bit_exact(y.cpu().numpy().reshape(rows, n), ref, f"prequantized shifted bsums rows={rows} {kernel}")


@pytest.mark.parametrize("rows,kernel", [(1, "auto"), (5, "auto"), (5, "tiled"), (70, "auto")])
def test_q8_0_multi_projection_rows_bit_exact(orc, ctx, batched, rows, kernel):
    """Fused Q8_0 q/k/v-style call over `rows` activation rows (the decode kernel up to 8 rows with rows x K <= 32768,
    the int8-MFMA kernel beyond that or when forced, one launch per weight): every output bit-exact, with a bias on
    the last weight."""
    case("q8_0 multi rows", rows, kernel)
    batched(kernel)
    rng = np.random.default_rng(500 + rows)
    k, shapes = 1024, [192, 64, 80]
    planes = [orc.q8_quantize_rows(normal(rng, (n, k), 0.05)) for n in shapes]
    ws = [ov.Q8Weight(wq, wsc, k, n) for (wq, wsc), n in zip(planes, shapes)]
    x = normal(rng, (rows, k))
    bias = normal(rng, shapes[2])
    refs = [orc.q8_project_batched(x, rows, wq, wsc, k, n, bias if i == 2 else None)
            for i, ((wq, wsc), n) in enumerate(zip(planes, shapes))]
    ys = [torch.empty(rows * n, device=DEV) for n in shapes]
    ctx.project_multi_dev(ws, t(x), ys, [None, None, t(bias)], rows=rows)
    torch.cuda.synchronize()
    for i, (y, ref) in enumerate(zip(ys, refs)):
        assert_bit_exact(y.cpu().numpy().reshape(rows, -1), ref, f"q8_0 multi rows={rows} job {i}")


def test_bound_multi_call_matches_oracle(orc, ctx):
    """A prepared multi-projection call (pointer arrays built once) replayed over new inputs: every call reads the
    bound tensors' current contents and is bit-exact, with and without a bias, M = 1 (decode GEMV) and M = 3."""
    case("bound multi", 0)
    rng = np.random.default_rng(77)
    k, shapes = 4096, [256, 64]
    blocks = [_kq_blocks(rng, "q4k", n, k) for n in shapes]
    ws = [ov.Q4KWeight(b, k, n) for b, n in zip(blocks, shapes)]
    bias = normal(rng, shapes[1])
    for rows in (1, 3):
        xd = torch.empty(rows * k, device=DEV)
        ys = [torch.empty(rows * n, device=DEV) for n in shapes]
        call = ctx.bind_multi_dev(ws, xd, ys, [None, t(bias)], rows=rows)
        for rep in range(3):
            x = normal(rng, (rows, k))
            xd.copy_(t(x).reshape(-1))
            call()
            torch.cuda.synchronize()
            for i, (y, b, n) in enumerate(zip(ys, blocks, shapes)):
                ref = orc.q4k_project_batched(x, rows, b, k, n, bias if i == 1 else None)
                assert_bit_exact(y.cpu().numpy().reshape(rows, n), ref, f"bound rows={rows} rep={rep} job {i}")


# ------------------------------------------------------------------------------------------------ GGUF upload

@pytest.mark.parametrize("on_device", [False, True])
def test_gguf_q8_0_known_answer_blocks(orc, on_device):
    """The reference's Q8_0 dequant KATs (TL/Loading/GgmlDequantTests.cs:20-94) through the GGUF upload and
    DecodeRow: scale * quant for a block with -128 and 127 at scale 2 and for three blocks with their own scales;
    an input size that is not a multiple of 32 is rejected before any device work."""
    case("gguf q8_0 kats", on_device)
    for scales, quants in Q8_0_KATS:
        k = 32 * len(scales)
        blocks = q8_0_gguf_blocks(scales, quants)
        w = ov.load_gguf_tensor(ov.TYPE_Q8_0, t(blocks) if on_device else blocks, k, 1)
        dst = np.zeros(k, np.float32)
        w.DecodeRow(0, dst)
        expected = np.repeat(np.asarray(scales, np.float32), 32) * quants.astype(np.float32)
        assert_bit_exact(dst, expected, f"q8_0 kat k={k}")
    with pytest.raises(ov.OverfitArgumentError, match="32"):
        ov.load_gguf_tensor(ov.TYPE_Q8_0, np.zeros(34, np.uint8), 31, 1)


@pytest.mark.parametrize("on_device", [False, True])
def test_gguf_upload_q8_0_q4k_q6k(orc, on_device):
    """Tensors in their GGUF bytes: Q8_0's 34-byte blocks de-interleaved on the device must project exactly like the
    oracle's LoadTensorQ8_0Raw planes; Q4_K / Q6_K bytes go up verbatim."""
    case("gguf upload", on_device)
    rng = np.random.default_rng(31 + on_device)
    k, n = 1024, 96
    wq, ws = orc.q8_quantize_rows(normal(rng, (n, k), 0.05))
    blocks = np.zeros((n * k // 32, 34), np.uint8)
    half = ws.astype(np.float16)  # a GGUF file stores fp16 scales
    blocks[:, 0:2] = half.view(np.uint8).reshape(-1, 2)
    blocks[:, 2:] = wq.reshape(-1, 32).view(np.uint8)
    rq, rs = orc.q8_0_deinterleave(blocks)
    src = t(blocks.ravel()) if on_device else blocks.ravel()
    w8 = ov.load_gguf_tensor(ov.TYPE_Q8_0, src, k, n)
    x = normal(rng, k)
    assert_bit_exact(ov.project(w8, x), orc.q8_project_batched(x, 1, rq, rs, k, n).ravel(), "gguf Q8_0")
    dec = np.zeros(k, np.float32)
    w8.DecodeRow(5, dec)
    assert np.array_equal(dec, rq.reshape(n, k)[5].astype(np.float32) * np.repeat(rs.reshape(n, -1)[5], 32))
    for fmt in ("q4k", "q6k"):
        b = _kq_blocks(rng, fmt, n, k)
        w = ov.load_gguf_tensor(ov.TYPE_Q4_K if fmt == "q4k" else ov.TYPE_Q6_K, t(b.ravel()) if on_device else b.ravel(),
                                k, n)
        ref = (orc.q4k_project if fmt == "q4k" else orc.q6k_project)(x, b, k, n)
        assert_bit_exact(ov.project(w, x), ref, f"gguf {fmt}")


@pytest.mark.parametrize("type_id,k,n", [(6, 4096, 1024), (6, 96, 7), (13, 4096, 300), (13, 14336, 33), (13, 256, 1)])
@pytest.mark.parametrize("on_device", [False, True])
def test_gguf_upload_q5_requantised_to_q8_0(orc, type_id, k, n, on_device):
    """Q5_0 / Q5_K tensors (a Q4_K_M file's attn_v or ffn_down) become resident Q8_0 weights on the device: the
    planes equal the oracle's decode-then-QuantizeRows bit for bit (LD/GgufLlamaLoader.cs:665-680), and the weight
    projects (one row and a batch) and decodes its rows like the oracle's Q8Weight."""
    case("gguf upload q5", type_id, k, n, on_device)
    rng = np.random.default_rng(type_id * 7 + k + n + on_device)
    data = random_q5_blocks(rng, type_id, n, k)
    rq, rs = orc.q5_requantize_q8_0(type_id, data, n, k)
    w = ov.load_gguf_tensor(type_id, t(data.ravel()) if on_device else data.ravel(), k, n)
    typ, nbytes, dptr = ctypes.c_int(), ctypes.c_size_t(), ctypes.c_void_p()
    lib = w.context.lib
    assert lib.ovfq_weight_info(w.handle, ctypes.byref(typ), None, None, ctypes.byref(nbytes), ctypes.byref(dptr)) == 0
    assert typ.value == ov.TYPE_Q8_0 and nbytes.value == n * k + n * (k // 32) * 4
    for rows in (1, 9):
        x = normal(rng, (rows, k))
        assert_bit_exact(ov.project(w, x, rows=rows), orc.q8_project_batched(x, rows, rq, rs, k, n).ravel(),
                         f"projection rows {rows}")
    dec = np.zeros(k, np.float32)
    for r in sorted({0, n // 2, n - 1}):  # Q8Weight.DecodeRow: quant x scale, so the planes themselves
        w.DecodeRow(r, dec)
        assert np.array_equal(dec.view(np.uint32), (rq[r].astype(np.float32) * np.repeat(rs[r], 32)).view(np.uint32))


# ------------------------------------------------------------------------------------------------ small batch

# Small batches on the automatic kernel choice: long rows, the largest K (64 super-blocks), an odd super-block
# count with 2-byte-aligned Q6_K rows, few output rows.
SMALL_SHAPES = [("q4k", 4, 14336, 300), ("q6k", 7, 2304, 130), ("q4k", 31, 4096, 64), ("q6k", 9, 16384, 70),
                ("q4k", 2, 256, 3)]

# The multi-row decode kernel, forced: 2..8 activation rows staged in LDS (one and two staging rounds), two rows
# per wave (K <= 4096) and one (longer rows), partial 16-block chunks (K = 2304, 4352), odd output counts.
ROWS_SHAPES = [("q6k", 2, 16384, 70), ("q4k", 3, 4352, 129), ("q6k", 5, 2304, 33), ("q4k", 8, 4096, 130),
               ("q6k", 8, 4096, 97), ("q4k", 4, 8192, 64), ("q4k", 7, 256, 5)]


@pytest.mark.parametrize("fmt,rows,k,n", ROWS_SHAPES)
def test_multi_row_decode_bit_exact(orc, batched, fmt, rows, k, n):
    case("multi-row decode", fmt, rows, k, n)
    batched("rows")
    rng = np.random.default_rng(rows * 17 + n)
    blocks = _kq_blocks(rng, fmt, n, k)
    x = normal(rng, (rows, k))
    bias = normal(rng, n)
    w = (ov.Q4KWeight if fmt == "q4k" else ov.Q6KWeight)(blocks, k, n)
    batched_ref = orc.q4k_project_batched if fmt == "q4k" else orc.q6k_project_batched
    y = ov.project(w, t(x), t(bias), rows=rows)
    torch.cuda.synchronize()
    assert_bit_exact(y.cpu().numpy().reshape(rows, n), batched_ref(x, rows, blocks, k, n, bias), f"{fmt} rows {rows}")
    assert_bit_exact(ov.project(w, x, None, rows=rows).reshape(rows, n), batched_ref(x, rows, blocks, k, n, None),
                     f"{fmt} rows {rows} no bias")


@pytest.mark.parametrize("rows", [2, 6])
def test_multi_row_decode_fused_jobs(orc, ctx, rows):
    """A q/k/v-shaped launch of three Q4_K weights over 2 and 6 rows on the automatic choice (the multi-row decode
    kernel runs fused launches of three or more weights up to 8 rows), with a bias on one weight."""
    case("multi-row fused", rows)
    rng = np.random.default_rng(900 + rows)
    k, shapes = 2048, [256, 64, 70]
    blocks = [_kq_blocks(rng, "q4k", n, k) for n in shapes]
    ws = [ov.Q4KWeight(b, k, n) for b, n in zip(blocks, shapes)]
    x = normal(rng, (rows, k))
    bias = normal(rng, shapes[1])
    refs = [orc.q4k_project_batched(x, rows, b, k, n, bias if i == 1 else None)
            for i, (b, n) in enumerate(zip(blocks, shapes))]
    ys = [torch.empty(rows * n, device=DEV) for n in shapes]
    ctx.project_multi_dev(ws, t(x), ys, [None, t(bias), None], rows=rows)
    torch.cuda.synchronize()
    for i, (y, ref) in enumerate(zip(ys, refs)):
        assert_bit_exact(y.cpu().numpy().reshape(rows, -1), ref, f"fused rows={rows} job {i}")


@pytest.mark.parametrize("fmt,rows,k,n", SMALL_SHAPES)
def test_small_batch_bit_exact(orc, fmt, rows, k, n):
    case("small batch", fmt, rows, k, n)
    rng = np.random.default_rng(rows * 31 + n)
    blocks = _kq_blocks(rng, fmt, n, k)
    x = normal(rng, (rows, k))
    bias = normal(rng, n)
    w = (ov.Q4KWeight if fmt == "q4k" else ov.Q6KWeight)(blocks, k, n)
    ref = (orc.q4k_project_batched if fmt == "q4k" else orc.q6k_project_batched)(x, rows, blocks, k, n, bias)
    y = ov.project(w, t(x), t(bias), rows=rows)
    torch.cuda.synchronize()
    assert_bit_exact(y.cpu().numpy().reshape(rows, n), ref, f"{fmt} small batch {rows}x{k}x{n}")


# Tall Q4_K matrices (768 16-row tiles or more) on the small-M path run on the expert-stream kernel: one wave per
# 16-row tile walking every super-block in order, weights by LDS DMA. Shapes: 1, 9 and 16 rows (one pair chunk), 37
# rows (three chunks, the last partial), a row count past the last full tile, gate/up pairs, a bias.
STREAM_SHAPES = [(1, 256, 12288), (9, 512, 12290), (16, 256, 13000), (37, 256, 12300), (5, 768, 12304)]


@pytest.mark.parametrize("rows,k,n", STREAM_SHAPES)
def test_stream_kernel_dense_bit_exact(orc, batched, rows, k, n):
    case("stream dense", rows, k, n)
    batched("small")
    rng = np.random.default_rng(rows * 13 + n)
    blocks = _kq_blocks(rng, "q4k", n, k)
    x = normal(rng, (rows, k))
    bias = normal(rng, n)
    w = ov.Q4KWeight(blocks, k, n)
    y = ov.project(w, t(x), t(bias), rows=rows)
    torch.cuda.synchronize()
    assert_bit_exact(y.cpu().numpy().reshape(rows, n), orc.q4k_project_batched(x, rows, blocks, k, n, bias),
                     f"stream {rows}x{k}x{n}")
    if rows > 1:
        # gate/up: two matrices in one launch (the units of both interleave on the persistent grid)
        b2 = _kq_blocks(rng, "q4k", n, k)
        w2 = ov.Q4KWeight(b2, k, n)
        g = torch.empty(rows * n, device=DEV)
        u = torch.empty(rows * n, device=DEV)
        ov.default_context().project_multi_dev([w, w2], t(x), [g, u], rows=rows)
        torch.cuda.synchronize()
        assert_bit_exact(g.cpu().numpy().reshape(rows, n), orc.q4k_project_batched(x, rows, blocks, k, n, None),
                         "stream gate")
        assert_bit_exact(u.cpu().numpy().reshape(rows, n), orc.q4k_project_batched(x, rows, b2, k, n, None),
                         "stream up")


# Tall Q6_K matrices with rows of a multiple of 8 super-blocks take the stream kernel's Q6_K form: every block DMA'd
# as the 224 aligned bytes around it (2 (sb % 8) bytes of lead-in), the lo/hi operands built from LDS. Row lengths of 8
# and 16 super-blocks (every lead-in), 3 .. 37 rows, partial weight groups and pair chunks.
STREAM_Q6K_SHAPES = [(3, 2048, 12288), (9, 4096, 12290), (16, 2048, 12300), (37, 2048, 12304)]


@pytest.mark.parametrize("rows,k,n", STREAM_Q6K_SHAPES)
def test_stream_kernel_dense_q6k_bit_exact(orc, batched, rows, k, n):
    case("stream dense q6k", rows, k, n)
    batched("small")
    rng = np.random.default_rng(rows * 17 + n)
    blocks = _kq_blocks(rng, "q6k", n, k)
    x = normal(rng, (rows, k))
    bias = normal(rng, n)
    w = ov.Q6KWeight(blocks, k, n)
    y = ov.project(w, t(x), t(bias), rows=rows)
    torch.cuda.synchronize()
    assert_bit_exact(y.cpu().numpy().reshape(rows, n), orc.q6k_project_batched(x, rows, blocks, k, n, bias),
                     f"stream q6k {rows}x{k}x{n}")


@pytest.mark.parametrize("rows", [2, 3, 4, 5])
def test_gate_up_pair_rows_boundary_bit_exact(orc, ctx, rows):
    """A gate/up-shaped Q4_K pair tall enough for the expert-stream kernel (6144 rows each: 768 16-row tiles) under
    the automatic choice: 2 rows on the multi-row decode kernel, from 3 rows on the stream kernel; each output
    bit-exact against the oracle, both through the fp32 entry point and the prequantised one."""
    case("gate/up pair boundary", rows)
    n, k = 6144, 256
    rng = np.random.default_rng(600 + rows)
    bg, bu = _kq_blocks(rng, "q4k", n, k), _kq_blocks(rng, "q4k", n, k)
    wg, wu = ov.Q4KWeight(bg, k, n), ov.Q4KWeight(bu, k, n)
    x = normal(rng, (rows, k))
    g = torch.empty(rows * n, device=DEV)
    u = torch.empty(rows * n, device=DEV)
    ctx.project_multi_dev([wg, wu], t(x), [g, u], rows=rows)
    torch.cuda.synchronize()
    assert_bit_exact(g.cpu().numpy().reshape(rows, n), orc.q4k_project_batched(x, rows, bg, k, n, None), "pair gate")
    assert_bit_exact(u.cpu().numpy().reshape(rows, n), orc.q4k_project_batched(x, rows, bu, k, n, None), "pair up")


def test_moe_ffn_skewed_routing(orc):
    """Few pairs in all (the expert-stream kernel) but one expert with 21 of them (two 16-pair chunks of its units),
    one with a single pair, one with none: against the oracle at the FFN tolerance."""
    case("moe skewed")
    rng = np.random.default_rng(515)
    E, dm, dff, rows, k = 8, 512, 768, 30, 1
    gb = [orc.quantize_q4k(normal(rng, (dff, dm), 0.05)) for _ in range(E)]
    ub = [orc.quantize_q4k(normal(rng, (dff, dm), 0.05)) for _ in range(E)]
    db = [orc.quantize_q4k(normal(rng, (dm, dff), 0.05)) for _ in range(E)]
    gw = [ov.Q4KWeight(b, dm, dff) for b in gb]
    uw = [ov.Q4KWeight(b, dm, dff) for b in ub]
    dw = [ov.Q4KWeight(b, dff, dm) for b in db]
    x = normal(rng, (rows, dm))
    idx = np.array([5] * 21 + [1] + [0, 2, 3, 4, 6, 0, 2, 3], np.int32).reshape(rows, k)  # expert 7: no pair
    rng.shuffle(idx)
    w = rng.random((rows, k)).astype(np.float32)
    ref = orc.moe_ffn_batched(gb, ub, db, ov.TYPE_Q4_K, ov.TYPE_Q4_K, x, rows, dm, dff, k, idx, w)
    y = ov.moe_ffn(gw, uw, dw, t(x), rows, k, t(idx), t(w))
    torch.cuda.synchronize()
    _moe_check(y.cpu().numpy(), ref, "skewed routing")


# ------------------------------------------------------------------------------------------------ routed MoE

@pytest.mark.parametrize("normalize", [True, False])
def test_moe_select_topk_matches_oracle(orc, normalize):
    case("moe topk", normalize)
    rng = np.random.default_rng(8 + normalize)
    rows, E, k = 37, 8, 2
    logits = rng.random((rows, E)).astype(np.float32)
    logits[3, 5] = logits[3, 2]  # a tie: the lower index wins
    idx = torch.zeros(rows * k, dtype=torch.int32, device=DEV)
    w = torch.zeros(rows * k, dtype=torch.float32, device=DEV)
    assert ov.MoeRouter.SelectTopK(t(logits), k, idx, w, normalize, rows=rows) == k
    torch.cuda.synchronize()
    hi, hw = np.zeros(rows * k, np.int32), np.zeros(rows * k, np.float32)
    ov.MoeRouter.SelectTopK(logits, k, hi, hw, normalize, rows=rows)
    for n in range(rows):
        ri, rw = orc.moe_select_topk(logits[n], k, normalize)
        for gi, gw in ((idx.cpu().numpy(), w.cpu().numpy()), (hi, hw)):
            assert np.array_equal(gi[n * k:(n + 1) * k], ri), n
            np.testing.assert_allclose(gw[n * k:(n + 1) * k], rw, rtol=4e-7, atol=0)
    # top_k above the expert count: min(top_k, n) slots written, the rest untouched
    li, lw = np.full(2 * 5, 99, np.int32), np.full(2 * 5, 7.0, np.float32)
    assert ov.MoeRouter.SelectTopK(logits[:2, :3].copy(), 5, li, lw, True, rows=2) == 3
    for n in range(2):
        ri, _ = orc.moe_select_topk(logits[n, :3], 5)
        assert np.array_equal(li[n * 5:n * 5 + 3], ri) and np.all(li[n * 5 + 3:(n + 1) * 5] == 99)


@pytest.mark.parametrize("normalize", [True, False])
def test_moe_select_topk_non_finite_logits(orc, normalize):
    """Router logits with +inf, -inf and NaN entries (and a row of all -inf): the selection follows the reference's
    comparisons (RT/MoeRouter.cs:66-91, where a NaN never compares greater or less-or-equal), on the standalone top-k
    launch and inside the routed MoE launch, against the oracle; weights NaN where the reference's are."""
    case("moe topk non-finite", normalize)
    rng = np.random.default_rng(90 + normalize)
    rows, E, k = 6, 8, 3
    logits = rng.random((rows, E)).astype(np.float32)
    logits[0, 4] = np.inf
    logits[1, 2] = -np.inf
    logits[2, 5] = np.nan
    logits[3, 0] = np.nan
    logits[3, 7] = np.inf
    logits[4, :] = -np.inf
    logits[5, 1] = np.nan
    logits[5, 6] = -np.inf
    idx = torch.zeros(rows * k, dtype=torch.int32, device=DEV)
    w = torch.zeros(rows * k, dtype=torch.float32, device=DEV)
    assert ov.MoeRouter.SelectTopK(t(logits), k, idx, w, normalize, rows=rows) == k
    torch.cuda.synchronize()
    gi, gw = idx.cpu().numpy().reshape(rows, k), w.cpu().numpy().reshape(rows, k)
    for n in range(rows):
        ri, rw = orc.moe_select_topk(logits[n], k, normalize)
        assert np.array_equal(gi[n], ri), (n, gi[n], ri)
        np.testing.assert_allclose(gw[n], rw, rtol=4e-7, atol=0, equal_nan=True)
    # the same selection inside the routed launch (routing fused into the grouping launch at rows * k <= 64)
    dm, dff = 256, 256
    gb = [orc.quantize_q4k(normal(rng, (dff, dm), 0.05)) for _ in range(E)]
    db = [orc.quantize_q4k(normal(rng, (dm, dff), 0.05)) for _ in range(E)]
    gws = [ov.Q4KWeight(b, dm, dff) for b in gb]
    dws = [ov.Q4KWeight(b, dff, dm) for b in db]
    x = normal(rng, (rows, dm))
    _, ri, rw = ov.moe_ffn_routed(gws, gws, dws, t(x), rows, t(logits), k, normalize)
    torch.cuda.synchronize()
    assert np.array_equal(ri.cpu().numpy().reshape(rows, k), gi)
    assert np.array_equal(rw.cpu().numpy().view(np.int32), w.cpu().numpy().view(np.int32))


def _moe_check(y, ref, what):
    y = np.asarray(y, np.float32).reshape(ref.shape)
    rel, cos = north_star(y, ref)
    scale = float(np.max(np.abs(ref)))
    err = float(np.max(np.abs(y.astype(np.float64) - ref)))
    exact = float(np.mean(y.view(np.uint32) == ref.astype(np.float32).view(np.uint32)))
    print(f"[moe] {what}: max abs err / max|ref| = {err / scale:.2e}, cos = {cos:.9f}, bit-exact {exact:.3f}",
          file=sys.stderr)
    # SiLU goes through expf on both sides (a few ULP apart); one ULP can move a Q8_K quant of the down
    # projection's input by one step, so the FFN output is held to the north-star tolerance, not bit-exactness.
    assert cos >= 0.99999 and err <= 1e-3 * scale, what


@pytest.mark.parametrize("rows,kernel", [(1, "auto"), (3, "auto"), (5, "auto"), (40, "tiled"), (40, "small")])
def test_ffn_swiglu_matches_oracle(orc, batched, rows, kernel):
    """The fused decode/prefill FFN (gate/up -> SiLU*up + Q8_K -> down) against the oracle's
    DecodeSwiGluBatchedDispatched restatement: rows 1 (GEMV), 3 (multi-row decode kernel), 5 (small-M MFMA), 40 (both
    batched MFMA kernels)."""
    case("ffn swiglu", rows, kernel)
    batched(kernel)
    rng = np.random.default_rng(70 + rows)
    dm, dff = 1024, 2048
    gb, ub = orc.quantize_q4k(normal(rng, (dff, dm), 0.05)), orc.quantize_q4k(normal(rng, (dff, dm), 0.05))
    db = orc.quantize_q6k(normal(rng, (dm, dff), 0.05))
    g, u, d = ov.Q4KWeight(gb, dm, dff), ov.Q4KWeight(ub, dm, dff), ov.Q6KWeight(db, dff, dm)
    x = normal(rng, (rows, dm))
    ref = orc.swiglu_batched(x, rows, gb, ub, db, 12, 14, dm, dff)
    y = ov.ffn_swiglu(g, u, d, t(x), rows)
    torch.cuda.synchronize()
    _moe_check(y.cpu().numpy(), ref, f"ffn rows={rows} device")
    _moe_check(ov.ffn_swiglu(g, u, d, x, rows), ref, f"ffn rows={rows} host")


@pytest.mark.parametrize("rows,kernel,gtype", [(1, "auto", 12), (3, "auto", 12), (40, "tiled", 12), (2, "auto", 14)])
def test_ffn_geglu_matches_oracle(orc, batched, rows, kernel, gtype):
    """The GeGLU FFN (Gemma: GELU tanh-approximation gate, ApplyGeLU RT/CachedFeedForwardBlock.cs:498-517) against
    the oracle at the FFN tolerance (tanhf on the device and on the host may differ by an ULP); the SwiGLU value of
    the same entry point is bit-identical to ovfq_ffn_swiglu; non-gated activations are refused."""
    case("ffn geglu", rows, kernel, gtype)
    batched(kernel)
    rng = np.random.default_rng(170 + rows)
    dm, dff = 512, 1536
    quant, W = (orc.quantize_q4k, ov.Q4KWeight) if gtype == 12 else (orc.quantize_q6k, ov.Q6KWeight)
    gb, ub = quant(normal(rng, (dff, dm), 0.08)), quant(normal(rng, (dff, dm), 0.08))
    db = orc.quantize_q6k(normal(rng, (dm, dff), 0.05))
    g, u, d = W(gb, dm, dff), W(ub, dm, dff), ov.Q6KWeight(db, dff, dm)
    x = normal(rng, (rows, dm))
    ref = orc.gated_ffn_batched(x, rows, gb, ub, db, gtype, 14, dm, dff, 4)
    y = ov.ffn_gated(g, u, d, t(x), rows, ov.FeedForwardActivation.GeGLU)
    torch.cuda.synchronize()
    _moe_check(y.cpu().numpy(), ref, f"geglu rows={rows} device")
    _moe_check(ov.ffn_gated(g, u, d, x, rows, ov.FeedForwardActivation.GeGLU), ref, f"geglu rows={rows} host")
    silu = orc.gated_ffn_batched(x, rows, gb, ub, db, gtype, 14, dm, dff, 3)
    assert np.linalg.norm(y.cpu().numpy().reshape(ref.shape) - silu) > 10 * np.linalg.norm(
        y.cpu().numpy().reshape(ref.shape) - ref)
    a = ov.ffn_gated(g, u, d, t(x), rows, ov.FeedForwardActivation.SwiGLU)
    b = ov.ffn_swiglu(g, u, d, t(x), rows)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int32), b.view(torch.int32))
    with pytest.raises(ov.OverfitArgumentError):
        ov.ffn_gated(g, u, d, t(x), rows, ov.FeedForwardActivation.GeLU)
    ctx = g.context
    out = torch.empty(rows * dm, device=DEV)
    for bad in (0, 1, 2, 5, -1):
        assert ctx.lib.ovfq_ffn_gated_dev(ctx.handle, g.handle, u.handle, d.handle, ctypes.c_void_p(t(x).data_ptr()),
                                          rows, bad, ctypes.c_void_p(out.data_ptr())) == _lib.OVFQ_ERR_RANGE


def test_ffn_swiglu_llama3_full_size(orc):
    """The Llama-3-8B FFN (gate/up 14336x4096 Q4_K, down 4096x14336 Q6_K) for one decode token."""
    case("ffn llama3 full size")
    gen = torch.Generator(device=DEV).manual_seed(90)
    mats = {}
    for name, (n, k, typ) in {"gate": (14336, 4096, ov.TYPE_Q4_K), "up": (14336, 4096, ov.TYPE_Q4_K),
                              "down": (4096, 14336, ov.TYPE_Q6_K)}.items():
        wf = torch.randn(n, k, generator=gen, device=DEV) * 0.02
        b = ov.quantize_weight(wf, typ)
        del wf
        mats[name] = ((ov.Q6KWeight if typ == ov.TYPE_Q6_K else ov.Q4KWeight)(b, k, n), b.cpu().numpy())
    x = normal(np.random.default_rng(91), (1, 4096))
    y = ov.ffn_swiglu(mats["gate"][0], mats["up"][0], mats["down"][0], t(x), 1)
    torch.cuda.synchronize()
    ref = orc.swiglu_batched(x, 1, mats["gate"][1], mats["up"][1], mats["down"][1], 12, 14, 4096, 14336)
    _moe_check(y.cpu().numpy(), ref, "ffn llama3")


@pytest.mark.parametrize("gfmt,dfmt", [("q4k", "q6k"), ("q4k", "q4k"), ("q6k", "q6k")])
def test_moe_ffn_matches_oracle(orc, gfmt, dfmt):
    case("moe ffn", gfmt, dfmt)
    rng = np.random.default_rng(21)
    E, dm, dff, rows, k = 8, 512, 1024, 16, 2
    T = {"q4k": ov.TYPE_Q4_K, "q6k": ov.TYPE_Q6_K}
    W = {"q4k": ov.Q4KWeight, "q6k": ov.Q6KWeight}
    enc = {"q4k": orc.quantize_q4k, "q6k": orc.quantize_q6k}
    gb = [enc[gfmt](normal(rng, (dff, dm), 0.05)) for _ in range(E)]
    ub = [enc[gfmt](normal(rng, (dff, dm), 0.05)) for _ in range(E)]
    db = [enc[dfmt](normal(rng, (dm, dff), 0.05)) for _ in range(E)]
    gw = [W[gfmt](b, dm, dff) for b in gb]
    uw = [W[gfmt](b, dm, dff) for b in ub]
    dw = [W[dfmt](b, dff, dm) for b in db]
    x = normal(rng, (rows, dm))
    idx = np.stack([rng.choice(E, k, replace=False) for _ in range(rows)]).astype(np.int32)
    idx[:5, 0] = 3  # one expert with many tokens (more than one pass of rows)
    idx[:5, 1] = np.where(idx[:5, 1] == 3, 4, idx[:5, 1])
    w = rng.random((rows, k)).astype(np.float32)
    ref = orc.moe_ffn_batched(gb, ub, db, T[gfmt], T[dfmt], x, rows, dm, dff, k, idx, w)
    y = ov.moe_ffn(gw, uw, dw, t(x), rows, k, t(idx), t(w))
    torch.cuda.synchronize()
    _moe_check(y.cpu().numpy(), ref, f"{gfmt}/{dfmt} device")
    _moe_check(ov.moe_ffn(gw, uw, dw, x, rows, k, idx, w), ref, f"{gfmt}/{dfmt} host")
    # an expert with no tokens, and an unclaimed slot
    idx2 = idx.copy()
    idx2[idx2 == 6] = 7
    idx2[2, 1] = E + 1
    ref2 = orc.moe_ffn_batched(gb, ub, db, T[gfmt], T[dfmt], x, rows, dm, dff, k, idx2, w)
    _moe_check(ov.moe_ffn(gw, uw, dw, x, rows, k, idx2, w), ref2, f"{gfmt}/{dfmt} sparse routing")


@pytest.mark.parametrize("rows,E,k,dfmt,dff", [(16, 8, 1, "q4k", 512), (16, 8, 2, "q4k", 512),
                                                (300, 64, 2, "q4k", 512), (16, 8, 2, "q6k", 512), (40, 8, 1, "q6k", 512),
                                                (16, 8, 2, "q6k", 2048), (40, 8, 1, "q6k", 2048),
                                                (300, 64, 2, "q6k", 2048)])
def test_moe_ffn_top2_combine_bit_exact(orc, rows, E, k, dfmt, dff):
    """Top-1 / top-2 with few pairs per expert: the down launch (the expert-stream kernel for Q4_K and for Q6_K rows of
    a multiple of 8 super-blocks, else the small-M kernel) adds weight * expert output into y with float atomics
    instead of a combine launch. y must equal, bit for bit, the reference's in-order combine
    (0 + w0 o0) + w1 o1 (RT/MoeFeedForwardBlock.cs:225-239) of each expert's output, taken here from the one-token
    SwiGLU FFN on the same expert (the same projections and SiLU launch, bit-identical per pair), with an unclaimed
    slot and a repeated index adding nothing, y first filled with NaN (every element written), and a second call
    with fewer tokens into the same buffer (no stale sums). 300 tokens over 64 experts: 600 pairs in the stream
    kernel's pair map, one expert with more than 40 pairs (several 16-pair chunks)."""
    case("moe top-k combine fold", rows, E, k, dfmt, dff)
    rng = np.random.default_rng(400 + rows + k)
    dm = 256
    gw, uw = ([ov.Q4KWeight(orc.quantize_q4k(normal(rng, shp, 0.05)), shp[1], shp[0]) for _ in range(E)]
              for shp in ((dff, dm), (dff, dm)))
    if dfmt == "q6k":
        dw = [ov.Q6KWeight(orc.quantize_q6k(normal(rng, (dm, dff), 0.05)), dff, dm) for _ in range(E)]
    else:
        dw = [ov.Q4KWeight(orc.quantize_q4k(normal(rng, (dm, dff), 0.05)), dff, dm) for _ in range(E)]
    x = normal(rng, (rows, dm))
    idx = np.stack([rng.choice(E, k, replace=False) for _ in range(rows)]).astype(np.int32)
    w = (rng.random((rows, k)) - 0.3).astype(np.float32)  # signed weights
    idx[3, 0] = E + 1  # unclaimed slot
    if k == 2:
        idx[5] = [4, 4]  # the repeat contributes nothing
    if rows > 64:
        idx[64:110, 1] = 5  # expert 5: over 40 pairs
        idx[64:110, 0] = np.where(idx[64:110, 0] == 5, 6, idx[64:110, 0])
    y = torch.full((rows * dm,), float("nan"), device=DEV)
    expert_out = {}
    for n in (rows, 5):
        out = ov.moe_ffn(gw, uw, dw, t(x[:n]), n, k, t(idx[:n]), t(w[:n]), out=y[: n * dm])
        torch.cuda.synchronize()
        got = out.cpu().numpy().reshape(n, dm)
        want = np.zeros((n, dm), np.float32)
        for tok in range(n):
            seen = set()
            for j in range(k):
                e = int(idx[tok, j])
                if e < 0 or e >= E or e in seen:
                    continue
                seen.add(e)
                if (tok, e) not in expert_out:
                    expert_out[tok, e] = ov.ffn_swiglu(gw[e], uw[e], dw[e], t(x[tok:tok + 1]), 1).cpu().numpy()
                o = expert_out[tok, e]
                want[tok] = want[tok] + np.float32(w[tok, j]) * o
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"top-{k}, {n} tokens: combine differs"


@pytest.mark.parametrize("rows,E,k,normalize", [(16, 8, 2, True), (30, 8, 1, False), (4, 16, 4, True),
                                                 (40, 8, 2, True), (64, 4, 1, True), (3, 32, 16, False),
                                                 (1, 64, 20, True)])
def test_moe_ffn_routed_equals_two_calls(orc, rows, E, k, normalize):
    """ovfq_moe_ffn_routed[_dev] (routing inside the grouping launch up to 64 (token, slot) entries, else the
    router launch first) gives the indices, weights and output of ovfq_moe_select_topk + ovfq_moe_ffn bit for bit,
    on the device and from host buffers; the routing itself against the oracle's SelectTopK."""
    case("moe routed", rows, E, k, normalize)
    rng = np.random.default_rng(1000 + rows * E + k)
    dm, dff = 256, 512
    gb = [orc.quantize_q4k(normal(rng, (dff, dm), 0.05)) for _ in range(E)]
    ub = [orc.quantize_q4k(normal(rng, (dff, dm), 0.05)) for _ in range(E)]
    db = [orc.quantize_q4k(normal(rng, (dm, dff), 0.05)) for _ in range(E)]
    gw = [ov.Q4KWeight(b, dm, dff) for b in gb]
    uw = [ov.Q4KWeight(b, dm, dff) for b in ub]
    dw = [ov.Q4KWeight(b, dff, dm) for b in db]
    x = normal(rng, (rows, dm))
    logits = rng.random((rows, E)).astype(np.float32)
    logits[min(1, rows - 1), :] = 0.25  # all tied: the lowest indices win
    ctx = ov.default_context()
    i2 = torch.empty(rows * k, dtype=torch.int32, device=DEV)
    w2 = torch.empty(rows * k, device=DEV)
    assert ctx.lib.ovfq_moe_select_topk_dev(ctx.handle, ctypes.c_void_p(t(logits).data_ptr()), rows, E, k,
                                            1 if normalize else 0, ctypes.c_void_p(i2.data_ptr()),
                                            ctypes.c_void_p(w2.data_ptr())) == 0
    y2 = ov.moe_ffn(gw, uw, dw, t(x), rows, k, i2, w2)
    y1, i1, w1 = ov.moe_ffn_routed(gw, uw, dw, t(x), rows, t(logits), k, normalize)
    torch.cuda.synchronize()
    assert torch.equal(i1, i2), "indices differ from ovfq_moe_select_topk"
    assert torch.equal(w1.view(torch.int32), w2.view(torch.int32)), "weights differ from ovfq_moe_select_topk"
    assert torch.equal(y1.view(torch.int32), y2.view(torch.int32)), "output differs from the two-call path"
    ref_idx = np.stack([orc.moe_select_topk(logits[n], k, normalize)[0] for n in range(rows)])
    assert np.array_equal(i1.cpu().numpy().reshape(rows, k), ref_idx)
    yh, ih, wh = ov.moe_ffn_routed(gw, uw, dw, x, rows, logits, k, normalize)
    assert np.array_equal(np.asarray(yh).view(np.int32), y1.cpu().numpy().view(np.int32))
    assert np.array_equal(np.asarray(ih), i1.cpu().numpy())
    assert np.array_equal(np.asarray(wh).view(np.int32), w1.cpu().numpy().view(np.int32))


def test_moe_ffn_routed_rejects_bad_arguments():
    """NULL router logits, and top_k above n_experts, are refused before any work."""
    case("moe routed arguments")
    ctx = ov.default_context()
    rng = np.random.default_rng(7)
    E, dm, dff = 2, 256, 256
    ws = [[ov.Q4KWeight(random_q4k_blocks(rng, n * (kk // 256)).reshape(n, -1), kk, n) for _ in range(E)]
          for n, kk in ((dff, dm), (dff, dm), (dm, dff))]
    arr = lambda w: (ctypes.c_void_p * E)(*[v.handle.value for v in w])
    x = np.zeros(dm, np.float32)
    y = np.zeros(dm, np.float32)
    lg = np.zeros(E, np.float32)
    ix = np.zeros(4, np.int32)
    wt = np.zeros(4, np.float32)
    P = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    f = ctx.lib.ovfq_moe_ffn_routed
    assert f(ctx.handle, E, arr(ws[0]), arr(ws[1]), arr(ws[2]), P(x), 1, None, 1, 1, P(ix), P(wt),
             P(y)) == _lib.OVFQ_ERR_NULL
    assert f(ctx.handle, E, arr(ws[0]), arr(ws[1]), arr(ws[2]), P(x), 1, P(lg), 3, 1, P(ix), P(wt),
             P(y)) == _lib.OVFQ_ERR_RANGE


def test_moe_ffn_many_tokens(orc):
    """A prefill-sized MoE batch: 300 tokens (more than one 256-token grouping chunk), top-3 of 8 experts, with a
    repeated expert in one token's slots, an out-of-range expert id and an expert no token chose."""
    case("moe ffn many tokens", 300)
    rng = np.random.default_rng(300)
    E, dm, dff, rows, k = 8, 256, 512, 300, 3
    gb = [orc.quantize_q4k(normal(rng, (dff, dm), 0.05)) for _ in range(E)]
    ub = [orc.quantize_q4k(normal(rng, (dff, dm), 0.05)) for _ in range(E)]
    db = [orc.quantize_q6k(normal(rng, (dm, dff), 0.05)) for _ in range(E)]
    gw = [ov.Q4KWeight(b, dm, dff) for b in gb]
    uw = [ov.Q4KWeight(b, dm, dff) for b in ub]
    dw = [ov.Q6KWeight(b, dff, dm) for b in db]
    x = normal(rng, (rows, dm))
    idx = np.stack([rng.choice(E - 1, k, replace=False) for _ in range(rows)]).astype(np.int32)  # expert 7 unused
    idx[10, 2] = idx[10, 0]  # a repeated expert: only the first slot is a pair
    idx[299, 1] = -1         # an out-of-range id: no pair
    w = rng.random((rows, k)).astype(np.float32)
    ref = orc.moe_ffn_batched(gb, ub, db, ov.TYPE_Q4_K, ov.TYPE_Q6_K, x, rows, dm, dff, k, idx, w)
    y = ov.moe_ffn(gw, uw, dw, t(x), rows, k, t(idx), t(w))
    torch.cuda.synchronize()
    _moe_check(y.cpu().numpy(), ref, "300 tokens top-3")


def test_moe_ffn_grouped_tile_boundaries(orc):
    """Many pairs per expert take the batched MFMA kernel over 64-row expert tiles: an expert with exactly 64 pairs
    (one full tile), one with 66 (a full tile and a 2-row tile), one with none."""
    case("moe grouped tiles", 130)
    rng = np.random.default_rng(130)
    E, dm, dff, rows, k = 3, 256, 256, 130, 1
    gb = [orc.quantize_q4k(normal(rng, (dff, dm), 0.05)) for _ in range(E)]
    ub = [orc.quantize_q4k(normal(rng, (dff, dm), 0.05)) for _ in range(E)]
    db = [orc.quantize_q4k(normal(rng, (dm, dff), 0.05)) for _ in range(E)]
    gw = [ov.Q4KWeight(b, dm, dff) for b in gb]
    uw = [ov.Q4KWeight(b, dm, dff) for b in ub]
    dw = [ov.Q4KWeight(b, dff, dm) for b in db]
    x = normal(rng, (rows, dm))
    idx = np.array([2] * 64 + [0] * 66, np.int32).reshape(rows, k)
    rng.shuffle(idx)
    w = rng.random((rows, k)).astype(np.float32)
    ref = orc.moe_ffn_batched(gb, ub, db, ov.TYPE_Q4_K, ov.TYPE_Q4_K, x, rows, dm, dff, k, idx, w)
    y = ov.moe_ffn(gw, uw, dw, t(x), rows, k, t(idx), t(w))
    torch.cuda.synchronize()
    _moe_check(y.cpu().numpy(), ref, "grouped tiles 64/66/0")


def test_moe_ffn_wide_intermediate(orc):
    """d_ff = 16640 (65 super-blocks, past the small-M kernel's limit) with few tokens: the grouped batched kernel
    takes it."""
    case("moe wide d_ff", 16640)
    rng = np.random.default_rng(65)
    E, dm, dff, rows, k = 2, 256, 16640, 3, 1
    gb = [orc.quantize_q4k(normal(rng, (dff, dm), 0.05)) for _ in range(E)]
    ub = [orc.quantize_q4k(normal(rng, (dff, dm), 0.05)) for _ in range(E)]
    db = [orc.quantize_q6k(normal(rng, (dm, dff), 0.05)) for _ in range(E)]
    gw = [ov.Q4KWeight(b, dm, dff) for b in gb]
    uw = [ov.Q4KWeight(b, dm, dff) for b in ub]
    dw = [ov.Q6KWeight(b, dff, dm) for b in db]
    x = normal(rng, (rows, dm))
    idx = np.array([[1], [0], [1]], np.int32)
    w = rng.random((rows, k)).astype(np.float32)
    ref = orc.moe_ffn_batched(gb, ub, db, ov.TYPE_Q4_K, ov.TYPE_Q6_K, x, rows, dm, dff, k, idx, w)
    _moe_check(ov.moe_ffn(gw, uw, dw, x, rows, k, idx, w), ref, "d_ff 16640")


def test_moe_config5_full_size(orc):
    """benchmark config 5: 8 Mixtral-shaped experts (gate/up 14336x4096, down 4096x14336, Q4_K), 16 tokens, top-2 of
    seeded uniform router logits, routed on the device; checked against the oracle's DecodeBatched restatement."""
    case("config5 full size")
    gen = torch.Generator(device=DEV).manual_seed(55)
    E, dm, dff, rows, k = 8, 4096, 14336, 16, 2
    mats = {"gate": [], "up": [], "down": []}
    host = {"gate": [], "up": [], "down": []}
    for name in ("gate", "up", "down"):
        n, kk = (dm, dff) if name == "down" else (dff, dm)
        for _ in range(E):
            wf = torch.randn(n, kk, generator=gen, device=DEV) * 0.02
            b = ov.quantize_weight(wf, ov.TYPE_Q4_K)
            del wf
            mats[name].append(ov.Q4KWeight(b, kk, n))
            host[name].append(b.cpu().numpy().reshape(n, -1))
    rng = np.random.default_rng(56)
    x = normal(rng, (rows, dm))
    logits = rng.random((rows, E)).astype(np.float32)
    idx = torch.empty(rows * k, dtype=torch.int32, device=DEV)
    w = torch.empty(rows * k, dtype=torch.float32, device=DEV)
    ov.MoeRouter.SelectTopK(t(logits), k, idx, w, rows=rows)
    y = ov.moe_ffn(mats["gate"], mats["up"], mats["down"], t(x), rows, k, idx, w)
    torch.cuda.synchronize()
    hi, hw = idx.cpu().numpy().reshape(rows, k), w.cpu().numpy().reshape(rows, k)
    for n in range(rows):
        assert np.array_equal(hi[n], orc.moe_select_topk(logits[n], k)[0])
    ref = orc.moe_ffn_batched(host["gate"], host["up"], host["down"], 12, 12, x, rows, dm, dff, k, hi, hw)
    _moe_check(y.cpu().numpy(), ref, "config5")


def _extreme_blocks(fmt, n, k):
    """Blocks at the ends of the integer ranges the MFMA operand split must hold: Q4_K sc = m = 63 with nibble 15
    (sc*nib = 945) and nibble 0; Q6_K scale -128 with q = 0 (sc*(q-32) = +4096), scale 127 with q = 63 and q = 0
    (3937, -4064), scale -128 with q = 63 (-3968)."""
    spr = k // 256
    if fmt == "q4k":
        b = np.zeros((n * spr, 144), np.uint8)
        b[:, 0:2] = np.frombuffer(np.float16(0.25).tobytes(), np.uint8)
        b[:, 2:4] = np.frombuffer(np.float16(0.125).tobytes(), np.uint8)
        b[:, 4:16] = 0xFF
        b[:, 16:] = np.where((np.arange(n * spr) % 2 == 0)[:, None], 0xFF, 0x00)
        return b.reshape(n, -1)
    b = np.zeros((n * spr, 210), np.uint8)
    kind = np.arange(n * spr) % 4
    b[:, 192:208] = np.where((kind % 2 == 0)[:, None], 0x80, 0x7F)
    q63 = (kind == 1) | (kind == 3)
    b[q63, :192] = 0xFF
    b[:, 208:210] = np.frombuffer(np.float16(0.01).tobytes(), np.uint8)
    return b.reshape(n, -1)


@pytest.mark.parametrize("fmt", ["q4k", "q6k"])
@pytest.mark.parametrize("rows", [1, 3, 40])
def test_kquant_long_rows_bit_exact(orc, fmt, rows):
    """K = 28672 (a Llama-3-70B down projection row: 112 super-blocks, past the decode GEMV's LDS-staged activation
    and the small-M kernel's limit): every row count takes its path and stays bit-exact, with a bias."""
    case("long rows", fmt, rows)
    rng = np.random.default_rng(rows + (7 if fmt == "q6k" else 0))
    k, n = 28672, 40
    blocks = _kq_blocks(rng, fmt, n, k)
    w = (ov.Q4KWeight if fmt == "q4k" else ov.Q6KWeight)(blocks, k, n)
    x = normal(rng, (rows, k))
    bias = normal(rng, n)
    batched = orc.q4k_project_batched if fmt == "q4k" else orc.q6k_project_batched
    ref = batched(x, rows, blocks, k, n, bias)
    y = ov.project(w, x, bias, rows=rows).reshape(rows, n)
    assert_bit_exact(y, ref, f"{fmt} K={k} rows={rows}")


# Row counts on both sides of every threshold of the automatic kernel choice: one-row GEMV, multi-row decode kernel
# (up to 4 rows; 8 for fused launches), small-M MFMA kernel, tiled MFMA kernel (grid >= 96 workgroups, or from 81 /
# 97 rows), and past K = 16384 the general kernel below 32 rows.
DISPATCH_ROWS = {2304: [1, 2, 3, 4, 5, 8, 9, 15, 16, 17, 31, 32, 33, 64, 65, 80, 81, 96, 97, 112, 113, 129],
                 16640: [1, 2, 4, 9, 31, 32, 33, 70]}


@pytest.mark.parametrize("fmt", ["q4k", "q6k"])
@pytest.mark.parametrize("k", sorted(DISPATCH_ROWS))
def test_automatic_choice_boundaries_bit_exact(orc, ctx, fmt, k):
    """Every row count of DISPATCH_ROWS through the automatic choice, 70 outputs (a partial 64-row tile), a bias:
    bit-exact against the oracle's batched restatement."""
    n = 70
    rng = np.random.default_rng(k + (1 if fmt == "q6k" else 0))
    blocks = _kq_blocks(rng, fmt, n, k)
    w = (ov.Q4KWeight if fmt == "q4k" else ov.Q6KWeight)(blocks, k, n)
    bias = normal(rng, n)
    batched = orc.q4k_project_batched if fmt == "q4k" else orc.q6k_project_batched
    for rows in DISPATCH_ROWS[k]:
        case("automatic choice", fmt, k, rows)
        x = normal(rng, (rows, k))
        ref = batched(x, rows, blocks, k, n, bias)
        y = ov.project(w, x, bias, rows=rows).reshape(rows, n)
        assert_bit_exact(y, ref, f"{fmt} K={k} rows={rows} automatic")


@pytest.mark.parametrize("kernel,rows,k", [("tiled", 48, 1024), ("small", 48, 1024), ("rows", 8, 1024),
                                           ("auto", 1, 28672)])
@pytest.mark.parametrize("fmt", ["q4k", "q6k"])
def test_kquant_prefill_range_extremes(orc, batched, kernel, rows, k, fmt):
    """Operand range extremes (every quant +-127, the largest scales and mins) on both MFMA kernels, the multi-row
    decode kernel (8 rows) and its one-row use for long rows (K = 28672)."""
    case("prefill extremes", kernel, rows, k, fmt)
    batched(kernel)
    n = 64
    blocks = _extreme_blocks(fmt, n, k)
    rng = np.random.default_rng(5)
    x = np.sign(normal(rng, (rows, k))).astype(np.float32)  # every quant +-127
    x[1::2] = normal(rng, (rows // 2, k))
    x[0] = 1.0                 # every group sum +2032 (the tiled Q4_K kernel's fp16 bsums at their largest)
    x[-1, : k // 2] = -1.0     # and -2032
    x[-1, k // 2:] = 1.0
    w = (ov.Q4KWeight if fmt == "q4k" else ov.Q6KWeight)(blocks, k, n)
    ref = (orc.q4k_project_batched if fmt == "q4k" else orc.q6k_project_batched)(x, rows, blocks, k, n)
    assert_bit_exact(ov.project(w, x, None, rows=rows).reshape(rows, n), ref, f"{fmt} extremes")


def test_llama3_8b_layer_prefill_sampled_rows(orc):
    """benchmark config 3 shapes at M = 512 (q 4096x4096, gate 14336x4096 Q4_K; down 4096x14336 Q6_K) at full size
    on the device; 40 sampled weight rows (all 512 activation rows each) are checked against the oracle: output
    rows of a projection are independent, so the sample is exact evidence for the rows it covers."""
    m = 512
    gen = torch.Generator(device=DEV).manual_seed(3)
    rng = np.random.default_rng(33)
    for name, (n, k, fmt) in {"q": (4096, 4096, "q4k"), "gate": (14336, 4096, "q4k"),
                              "down": (4096, 14336, "q6k")}.items():
        case("config3", name, m, n, k)
        wf = torch.randn(n, k, generator=gen, device=DEV) * 0.02
        blocks = ov.quantize_weight(wf, ov.TYPE_Q6_K if fmt == "q6k" else ov.TYPE_Q4_K)
        del wf
        w = (ov.Q6KWeight if fmt == "q6k" else ov.Q4KWeight)(blocks, k, n)
        x = normal(rng, (m, k))
        y = ov.project(w, t(x), rows=m)
        torch.cuda.synchronize()
        sel = np.sort(rng.choice(n, 40, replace=False))
        hb = blocks.cpu().numpy().reshape(n, -1)[sel]
        ref = (orc.q6k_project_batched if fmt == "q6k" else orc.q4k_project_batched)(x, m, hb, k, len(sel))
        got = y.cpu().numpy().reshape(m, n)[:, sel]
        assert_bit_exact(got, ref, f"config3 {name}")
        rel, cos = north_star(got, ref)
        assert rel <= 1e-3 and cos >= 0.99999


# One row on the decode GEMV (activation in LDS up to K = 32768; 32800 takes the row kernel). More rows: automatic
# choice (the decode kernel over up to 8 rows where rows x K <= 32768, else the int8-MFMA kernel from 8 rows, or from
# 4-6 rows for inputs up to 8192, else the row kernel), and each kernel forced ("tiled": the MFMA kernel from 2 rows,
# "rows": the multi-row decode kernel where it takes the shape, "small": the row kernel): partial 16/32/64-row
# activation tiles (2 .. 16, 24, 65, 130), a partial 64-output tile (70), 129 blocks per row (four-block groups with a
# short last one; a partial 64-block GEMV item), one block per row.
@pytest.mark.parametrize("kernel", ["auto", "tiled", "rows", "small"])
@pytest.mark.parametrize("k,n", [(32, 5), (128, 4096), (4096, 300), (14336, 40), (4128, 70), (32768, 24),
                                 (32800, 9)])
@pytest.mark.parametrize("rows", [1, 2, 3, 7, 16, 24, 65, 130])
def test_q8_0_project_bit_exact(orc, batched, kernel, k, n, rows):
    case("q8_0 project", kernel, k, n, rows)
    batched(kernel)
    rng = np.random.default_rng(k + n + rows)
    wq, ws = orc.q8_quantize_rows(normal(rng, (n, k), 0.05))
    wq[0, :32] = -128                               # GGUF Q8_0 weights may hold -128
    x = normal(rng, (rows, k))
    bias = normal(rng, n)
    w = ov.Q8Weight(wq, ws, k, n)
    ref = orc.q8_project_batched(x, rows, wq, ws, k, n, bias)
    if rows == 1:
        assert np.array_equal(ref[0], orc.q8_project(x[0], wq, ws, k, n, bias))
    y = ov.project(w, x, bias, rows=rows).reshape(rows, n)
    assert_bit_exact(y, ref, f"q8_0 {k}x{n} rows={rows}")


# The decode kernel's LDS copy of the activation exactly full (rows x K = 32768) at 4 and 8 rows, and 8 rows on
# every kernel choice.
@pytest.mark.parametrize("kernel", ["auto", "tiled", "rows", "small"])
@pytest.mark.parametrize("k,n,rows", [(4096, 300, 8), (8192, 48, 4), (128, 4096, 8), (2048, 70, 8)])
def test_q8_0_project_full_lds_and_eight_rows(orc, batched, kernel, k, n, rows):
    case("q8_0 project full LDS", kernel, k, n, rows)
    batched(kernel)
    rng = np.random.default_rng(3 * k + n + rows)
    wq, ws = orc.q8_quantize_rows(normal(rng, (n, k), 0.05))
    wq[-1, -32:] = -128
    x = normal(rng, (rows, k))
    bias = normal(rng, n)
    w = ov.Q8Weight(wq, ws, k, n)
    ref = orc.q8_project_batched(x, rows, wq, ws, k, n, bias)
    y = ov.project(w, x, bias, rows=rows).reshape(rows, n)
    assert_bit_exact(y, ref, f"q8_0 {k}x{n} rows={rows}")


def test_gate_up_and_multi_projection(orc, ctx):
    case("gate_up / multi")
    rng = np.random.default_rng(77)
    k, n = 2048, 300
    g = _kq_blocks(rng, "q4k", n, k)
    u = _kq_blocks(rng, "q4k", n, k)
    x = normal(rng, k)
    wg, wu = ov.Q4KWeight(g, k, n), ov.Q4KWeight(u, k, n)
    rg, ru = orc.q4k_project_gate_up(x, g, u, k, n)
    go, uo = ov.project_gate_up(wg, wu, x)
    assert_bit_exact(go, rg, "gate (host)")
    assert_bit_exact(uo, ru, "up (host)")
    go, uo = ov.project_gate_up(wg, wu, t(x))
    torch.cuda.synchronize()
    assert_bit_exact(go.cpu().numpy(), rg, "gate (device)")
    assert_bit_exact(uo.cpu().numpy(), ru, "up (device)")
    # q/k/v-style fused launch with different row counts and a bias on one of them
    n2 = 77
    v = _kq_blocks(rng, "q4k", n2, k)
    wv = ov.Q4KWeight(v, k, n2)
    bias_v = normal(rng, n2)
    ys = [torch.empty(n, device=DEV), torch.empty(n, device=DEV), torch.empty(n2, device=DEV)]
    ctx.project_multi_dev([wg, wu, wv], t(x), ys, [None, None, t(bias_v)])
    torch.cuda.synchronize()
    assert_bit_exact(ys[0].cpu().numpy(), rg, "multi gate")
    assert_bit_exact(ys[1].cpu().numpy(), ru, "multi up")
    assert_bit_exact(ys[2].cpu().numpy(), orc.q4k_project(x, v, k, n2, bias_v), "multi v")


@pytest.mark.parametrize("fmt,rows", [("q4k", 1), ("q4k", 5), ("q6k", 1), ("q6k", 40), ("q8_0", 1), ("q8_0", 9)])
def test_project_multi_host_pointers(orc, ctx, fmt, rows):
    """ovfq_project_multi (host pointers, synchronous; the attention block's q/k/v against one quantised hidden row,
    RT/CachedMultiHeadAttention.cs:196-207) equals the oracle's separate projections bit for bit, through the
    context's page-locked staging; a second call with fewer rows reuses it."""
    case("project_multi host", fmt, rows)
    rng = np.random.default_rng(4242 + rows)
    k = 4096 if fmt != "q6k" else 2048
    ns = [512, 128, 128]
    if fmt == "q8_0":
        planes = [orc.q8_quantize_rows(normal(rng, (n, k), 0.05)) for n in ns]
        ws = [ov.Q8Weight(q, s_, k, n) for (q, s_), n in zip(planes, ns)]
        ref = lambda i, x, r, b: orc.q8_project_batched(x, r, planes[i][0], planes[i][1], k, ns[i], b)
    else:
        blocks = [_kq_blocks(rng, fmt, n, k) for n in ns]
        W = ov.Q4KWeight if fmt == "q4k" else ov.Q6KWeight
        ws = [W(b, k, n) for b, n in zip(blocks, ns)]
        pb = orc.q4k_project_batched if fmt == "q4k" else orc.q6k_project_batched
        ref = lambda i, x, r, b: pb(x, r, blocks[i], k, ns[i], b)
    bias = normal(rng, ns[1])
    for r in (rows, max(1, rows // 2)):
        x = normal(rng, (r, k))
        outs = ov.project_multi(ws, x, rows=r, biases=[None, bias, None])
        for i in range(3):
            assert_bit_exact(outs[i], ref(i, x, r, bias if i == 1 else None).reshape(-1), f"{fmt} job {i} rows {r}")


@pytest.mark.parametrize("fmt", ["q4k", "q6k"])
def test_partial_chunk_decode_multi_and_prequantized(orc, ctx, fmt):
    """Decode kernel on rows of 21 super-blocks (a partial last 16-block chunk): a fused three-job launch with odd row
    counts and one bias, and the prequantised entry point, against the oracle's sequential per-row sums."""
    case("decode 21-block rows multi/prequantized", fmt)
    rng = np.random.default_rng(2121)
    k = 5376
    ns = [33, 7, 130]
    blocks = [_kq_blocks(rng, fmt, n, k) for n in ns]
    W = ov.Q4KWeight if fmt == "q4k" else ov.Q6KWeight
    ws = [W(b, k, n) for b, n in zip(blocks, ns)]
    proj = orc.q4k_project if fmt == "q4k" else orc.q6k_project
    x = normal(rng, k)
    bias = normal(rng, ns[2])
    refs = [proj(x, blocks[0], k, ns[0]), proj(x, blocks[1], k, ns[1]), proj(x, blocks[2], k, ns[2], bias)]
    ys = [torch.empty(n, device=DEV) for n in ns]
    ctx.project_multi_dev(ws, t(x), ys, [None, None, t(bias)])
    torch.cuda.synchronize()
    for i in range(3):
        assert_bit_exact(ys[i].cpu().numpy(), refs[i], f"{fmt} multi job {i}")
    q, s, b = orc.quantize_q8k(x)
    y = torch.empty(ns[2], device=DEV)
    ctx.project_prequantized_dev(ws[2], t(q.ravel()), t(s.ravel()), t(b.ravel()), y, bias=t(bias))
    torch.cuda.synchronize()
    assert_bit_exact(y.cpu().numpy(), refs[2], f"{fmt} prequantized")


def test_reference_mirror_api_host_and_device(orc):
    case("Q4KDotKernel / Q6KDotKernel / Q8DotKernel mirror")
    rng = np.random.default_rng(9)
    k, n = 512, 96
    blocks = _kq_blocks(rng, "q4k", n, k)
    w = ov.Q4KWeight(blocks, k, n)
    x = (rng.random(k) * 2 - 1).astype(np.float32)
    bias = normal(rng, n)
    y = np.zeros(n, np.float32)
    q, s, b = np.zeros(k, np.int8), np.zeros(2, np.float32), np.zeros(32, np.int16)
    ov.Q4KDotKernel.Project(x, w, bias, y, q, s, b)
    ref = orc.q4k_project(x, blocks, k, n, bias)
    assert_bit_exact(y, ref, "Q4KDotKernel.Project")
    rq, rd, rb = orc.quantize_q8k(x)
    assert np.array_equal(q, rq[0]) and np.array_equal(b, rb[0])  # caller scratch holds the Q8_K form
    y2 = np.zeros(n, np.float32)
    ov.Q4KDotKernel.ProjectPreQuantized(w, bias, y2, q, s, b)
    assert_bit_exact(y2, ref, "ProjectPreQuantized")
    yd = torch.zeros(n, device=DEV)
    ov.Q4KDotKernel.ProjectParallel(t(x), w, t(bias), yd, torch.zeros(k, dtype=torch.int8, device=DEV),
                                    torch.zeros(2, device=DEV), torch.zeros(32, dtype=torch.int16, device=DEV))
    torch.cuda.synchronize()
    assert_bit_exact(yd.cpu().numpy(), ref, "ProjectParallel (device)")
    # Dot of one block
    blk = blocks[0, :144].copy()
    got = ov.Q4KDotKernel.Dot(blk, rq[0, :256], float(rd[0, 0]), rb[0, :16])
    assert np.float32(got) == np.float32(orc.lib().orc_q4k_dot(orc.P(blk), orc.P(rq[0]), float(rd[0, 0]), orc.P(rb[0])))
    # errors raised before work, like the reference's argument exceptions
    with pytest.raises(ov.OverfitArgumentError):
        ov.Q4KDotKernel.Project(x, w, bias[:5], y, q, s, b)
    with pytest.raises(ov.OverfitArgumentError):
        ov.Q4KDotKernel.Project(x[:100], w, None, y, q, s, b)
    with pytest.raises(ov.OverfitArgumentOutOfRangeError):
        ov.Q4KDotKernel.ProjectBatched(x, 0, w, None, y, q, s, b)
    with pytest.raises(ov.OverfitArgumentNullError):
        ov.Q4KDotKernel.Project(x, None, None, y, q, s, b)
    # Q6_K and Q8 mirrors
    b6 = _kq_blocks(rng, "q6k", n, k)
    w6 = ov.Q6KWeight(b6, k, n)
    ov.Q6KDotKernel.Project(x, w6, None, y, q, s, b)
    assert_bit_exact(y, orc.q6k_project(x, b6, k, n), "Q6KDotKernel.Project")
    rows = 4
    xb = normal(rng, (rows, k))
    yb = np.zeros(rows * n, np.float32)
    ov.Q6KDotKernel.ProjectBatched(xb, rows, w6, bias, yb, np.zeros(rows * k, np.int8), np.zeros(rows * 2, np.float32),
                                   np.zeros(rows * 32, np.int16))
    assert_bit_exact(yb, orc.q6k_project_batched(xb, rows, b6, k, n, bias), "Q6KDotKernel.ProjectBatched")
    wq, ws = orc.q8_quantize_rows(normal(rng, (n, 128), 0.05))
    w8 = ov.Q8Weight(wq, ws, 128, n)
    x8 = normal(rng, 128)
    y8 = np.zeros(n, np.float32)
    ov.Q8DotKernel.Project(x8, w8, bias, y8, np.zeros(128, np.int8), np.zeros(4, np.float32))
    assert_bit_exact(y8, orc.q8_project(x8, wq, ws, 128, n, bias), "Q8DotKernel.Project")
    dw = ov.DecodeWeight(w)
    assert dw.IsQ4K and not dw.IsQ6K and not dw.IsQuantized
    yb4 = np.zeros(rows * n, np.float32)
    ov.BatchedQuantProjection.Dispatch(xb, rows, dw, bias, yb4, k, n)
    assert_bit_exact(yb4, orc.q4k_project_batched(xb, rows, blocks, k, n, bias), "BatchedQuantProjection")


@pytest.mark.parametrize("fmt", ["q4k", "q6k", "q8"])
def test_decode_row_bit_exact(orc, fmt):
    case("DecodeRow", fmt)
    rng = np.random.default_rng(4)
    k, n = 1024, 9
    if fmt == "q8":
        wq, ws = orc.q8_quantize_rows(normal(rng, (n, k), 0.05))
        w = ov.Q8Weight(wq, ws, k, n)
        ref = lambda r: np.repeat(ws[r], 32) * wq[r].astype(np.float32)  # noqa: E731  RT/Q8Weight.cs:81-106
    else:
        blocks = _kq_blocks(rng, fmt, n, k)
        w = (ov.Q4KWeight if fmt == "q4k" else ov.Q6KWeight)(blocks, k, n)
        dec = orc.q4k_decode_row if fmt == "q4k" else orc.q6k_decode_row
        ref = lambda r: dec(blocks, k, n, r)  # noqa: E731
    for r in (0, 4, n - 1):
        dst = np.zeros(k, np.float32)
        w.DecodeRow(r, dst)
        assert_bit_exact(dst, ref(r), f"{fmt} row {r}")
    with pytest.raises(ov.OverfitArgumentOutOfRangeError):
        w.DecodeRow(n, np.zeros(k, np.float32))


# ------------------------------------------------------------------------------------------------ full sizes

def test_llama3_8b_layer_decode_projections_bit_exact(orc, ctx):
    """benchmark config 2 at full size: q 4096x4096, k/v 1024x4096, o 4096x4096, gate/up 14336x4096 (Q4_K),
    down 4096x14336 (Q6_K); weights N(0, 0.02) quantized on the device, activations N(0, 1)."""
    case("config2 full-size layer")
    gen = torch.Generator(device=DEV).manual_seed(20260519)
    shapes = {"q": (4096, 4096), "k": (1024, 4096), "v": (1024, 4096), "o": (4096, 4096),
              "gate": (14336, 4096), "up": (14336, 4096), "down": (4096, 14336)}
    rng = np.random.default_rng(8)
    for name, (n, k) in shapes.items():
        case("config2", name, n, k)
        wf = torch.randn(n, k, generator=gen, device=DEV) * 0.02
        fmt = ov.TYPE_Q6_K if name == "down" else ov.TYPE_Q4_K
        blocks = ov.quantize_weight(wf, fmt)
        del wf
        w = (ov.Q6KWeight if name == "down" else ov.Q4KWeight)(blocks, k, n)
        x = normal(rng, k)
        y = ov.project(w, t(x))
        torch.cuda.synchronize()
        hb = blocks.cpu().numpy().reshape(n, -1)
        ref = (orc.q6k_project if name == "down" else orc.q4k_project)(x, hb, k, n)
        assert_bit_exact(y.cpu().numpy(), ref, f"config2 {name}")
        rel, cos = north_star(y.cpu().numpy(), ref)
        assert rel <= 1e-3 and cos >= 0.99999


def test_q6k_lm_head_full_size_bit_exact(orc):
    """The Llama-3-8B Q6_K output head (128256 x 4096) of benchmark config 4."""
    case("LM head 128256x4096 Q6_K")
    gen = torch.Generator(device=DEV).manual_seed(7)
    n, k = 128256, 4096
    wf = torch.randn(n, k, generator=gen, device=DEV) * 0.02
    blocks = ov.quantize_weight(wf, ov.TYPE_Q6_K)
    del wf
    w = ov.Q6KWeight(blocks, k, n)
    x = normal(np.random.default_rng(1), k)
    y = ov.project(w, t(x))
    torch.cuda.synchronize()
    ref = orc.q6k_project(x, blocks.cpu().numpy().reshape(n, -1), k, n)
    assert_bit_exact(y.cpu().numpy(), ref, "LM head")


def test_graph_replay_moe_and_ffn(orc, ctx):
    """Captured MoE steps (router, grouping, grouped experts, SwiGLU, combine) and fused FFNs, as the bench replays
    them: every replay reproduces the eager outputs bit-for-bit, with eager work and synchronisations between the
    replays (the grouping kernel clears its own tables: nothing in the graph is a memset node)."""
    case("graph replay moe/ffn")
    rng = np.random.default_rng(44)
    E, dm, dff, rows, k = 8, 256, 512, 16, 2
    gw = [ov.Q4KWeight(orc.quantize_q4k(normal(rng, (dff, dm), 0.05)), dm, dff) for _ in range(E)]
    uw = [ov.Q4KWeight(orc.quantize_q4k(normal(rng, (dff, dm), 0.05)), dm, dff) for _ in range(E)]
    dw = [ov.Q4KWeight(orc.quantize_q4k(normal(rng, (dm, dff), 0.05)), dff, dm) for _ in range(E)]
    fd = ov.Q6KWeight(orc.quantize_q6k(normal(rng, (dm, dff), 0.05)), dff, dm)
    logits = t(rng.random((rows, E)).astype(np.float32))
    x = t(normal(rng, (rows, dm)))
    idx = torch.empty(rows * k, dtype=torch.int32, device=DEV)
    wt = torch.empty(rows * k, dtype=torch.float32, device=DEV)
    ys = [torch.empty(rows * dm, device=DEV), torch.empty(dm, device=DEV)]

    def step():
        ov.MoeRouter.SelectTopK(logits, k, idx, wt, True, rows=rows)
        ov.moe_ffn(gw, uw, dw, x, rows, k, idx, wt, out=ys[0])
        ov.ffn_swiglu(gw[0], uw[0], fd, x[:1].reshape(-1), 1, out=ys[1])

    step()
    torch.cuda.synchronize()
    eager = [y.cpu().numpy().copy() for y in ys]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        ctx.set_stream(side.cuda_stream)
        step()
        side.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=side):
            step()
    ctx.set_stream(torch.cuda.current_stream().cuda_stream)
    for rep in range(4):
        for y in ys:
            y.fill_(float("nan"))
        idx.fill_(-7)
        g.replay()
        torch.cuda.synchronize()
        for y, e in zip(ys, eager):
            assert np.array_equal(y.cpu().numpy().view(np.uint32), e.view(np.uint32)), f"replay {rep}"
        step()  # eager work between replays
        torch.cuda.synchronize()


def test_graph_replay_matches_eager(orc, ctx):
    """The bench replays captured decode steps; every replay must reproduce the eager outputs bit-for-bit
    (replays interleaved with eager work and synchronisations): one-row launches, a 3-row launch on the multi-row
    kernel (quantised inside the launch) and a 3-row Q6_K launch of long rows (separate quantise launch)."""
    case("graph replay")
    rng = np.random.default_rng(12)
    k, n, k2 = 4096, 512, 14336
    wq = ov.Q4KWeight(_kq_blocks(rng, "q4k", n, k), k, n)
    wu = ov.Q4KWeight(_kq_blocks(rng, "q4k", n, k), k, n)
    wd = ov.Q6KWeight(_kq_blocks(rng, "q6k", 256, k2), k2, 256)
    x, xd = t(normal(rng, k)), t(normal(rng, k2))
    x3, xd3 = t(normal(rng, (3, k))), t(normal(rng, (3, k2)))
    ys = [torch.empty(n, device=DEV), torch.empty(n, device=DEV), torch.empty(256, device=DEV),
          torch.empty(3 * n, device=DEV), torch.empty(3 * n, device=DEV), torch.empty(3 * 256, device=DEV)]

    def step():
        ctx.project_multi_dev([wq, wu], x, ys[:2])
        ctx.project_multi_dev([wd], xd, ys[2:3])
        ctx.project_multi_dev([wq, wu], x3, ys[3:5], rows=3)
        ctx.project_multi_dev([wd], xd3, ys[5:], rows=3)

    step()
    torch.cuda.synchronize()
    eager = [y.cpu().numpy().copy() for y in ys]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        ctx.set_stream(side.cuda_stream)
        step()
        side.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=side):
            step()
    ctx.set_stream(torch.cuda.current_stream().cuda_stream)
    for rep in range(4):
        for y in ys:
            y.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        for y, e in zip(ys, eager):
            assert np.array_equal(y.cpu().numpy().view(np.uint32), e.view(np.uint32)), f"replay {rep}"
        step()  # eager work between replays
        torch.cuda.synchronize()


def test_concurrent_calls_on_one_context(orc, ctx):
    """The reference calls Project / ProjectPreQuantized from several worker threads at once
    (RT/CachedMultiHeadAttention.cs:280, :876-907), each with its own activation. Four threads share one context
    (host-pointer calls: staging, launch, copy back and wait happen under the context's lock), over one-row,
    multi-row and prefill shapes, and every output stays bit-exact."""
    import threading
    case("concurrent calls")
    rng = np.random.default_rng(31)
    k, n = 1024, 160
    blocks = {fmt: _kq_blocks(rng, fmt, n, k) for fmt in ("q4k", "q6k")}
    ws = {"q4k": ov.Q4KWeight(blocks["q4k"], k, n), "q6k": ov.Q6KWeight(blocks["q6k"], k, n)}
    jobs = []
    for i, (fmt, rows) in enumerate([("q4k", 1), ("q6k", 3), ("q4k", 40), ("q6k", 1), ("q4k", 2), ("q6k", 17)]):
        x = normal(rng, (rows, k))
        ref = (orc.q4k_project_batched if fmt == "q4k" else orc.q6k_project_batched)(x, rows, blocks[fmt], k, n, None)
        jobs.append((fmt, rows, x, ref))
    errors = []

    def worker(tid):
        try:
            for it in range(6):
                fmt, rows, x, ref = jobs[(tid + it) % len(jobs)]
                y = ov.project(ws[fmt], x, None, rows=rows).reshape(rows, n)
                if not np.array_equal(y.view(np.uint32), ref.view(np.uint32)):
                    errors.append(f"thread {tid} iteration {it}: {fmt} rows={rows} differs")
        except Exception as e:  # noqa: BLE001 - reported below
            errors.append(f"thread {tid}: {e!r}")

    threads = [threading.Thread(target=worker, args=(tid,)) for tid in range(4)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=60)
    assert not any(th.is_alive() for th in threads), "a worker did not finish"
    assert not errors, errors

