"""Pins the oracle (oracle/ovfq_oracle.c) before it is trusted as the GPU checker.

Each function of the oracle is checked against the reference's own known-answer tests and invariants
(cited per test), against library routines where the mathematics reduces to one (numpy float16 for the
fp16 conversions), by brute force on small inputs, and by identities chosen so that a plausible mistake
(a dropped min term, a wrong sign, a swapped nibble, a transposed index) fails.
"""
import numpy as np
import pytest

from qdata import Q8_0_KATS, half_bits, normal, q8_0_gguf_blocks, random_q4k_blocks, random_q6k_blocks


# ------------------------------------------------------------------------------------------------ fp16

def test_half_to_float_all_65536_patterns_match_numpy(orc):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = bits.view(np.float16).astype(np.float32).view(np.uint32)
    got = np.array([orc.lib().orc_half_to_float(int(b)) for b in bits], dtype=np.float32).view(np.uint32)
    finite = ~np.isnan(bits.view(np.float16))
    assert np.array_equal(got[finite], ref[finite])
    assert np.all(np.isnan(got[~finite].view(np.float32)))


def test_float_to_half_matches_numpy_rne(orc):
    rng = np.random.default_rng(1)
    pats = rng.integers(0, 2**32, size=200_000, dtype=np.uint64).astype(np.uint32)
    f = pats.view(np.float32)
    # add ties / boundaries: halfway cases between fp16 neighbours, subnormal range, overflow edge
    edge = np.array([65504.0, 65519.996, 65520.0, 6.0975552e-05, 5.9604645e-08, 2.9802322e-08, 2.9802326e-08,
                     1.0 + 2**-11, 1.0 + 3 * 2**-11, -0.0, 0.0, np.inf, -np.inf], dtype=np.float32)
    halfway = (np.arange(1, 2048, dtype=np.float32) + 0.5) * np.float32(2.0**-24)
    f = np.concatenate([f, edge, halfway]).astype(np.float32)
    f = f[~np.isnan(f)]
    with np.errstate(over="ignore"):
        ref = f.astype(np.float16).view(np.uint16)
    L = orc.lib()
    got = np.array([L.orc_float_to_half(float(x)) for x in f], dtype=np.uint16)
    assert np.array_equal(got, ref)


# ------------------------------------------------------------------------------------------------ a1 unpack

def test_unpack_lower_branch_kat(orc):
    # TL/Loading/GgmlDequantTests.cs:98-130
    p = np.zeros(12, np.uint8)
    p[:8] = [10, 20, 30, 40, 5, 15, 21, 27]
    sc, m = orc.unpack_q4k_scales_mins(p)
    assert list(sc) == [10, 20, 30, 40, 0, 0, 0, 0]
    assert list(m) == [5, 15, 21, 27, 0, 0, 0, 0]


def test_unpack_upper_branch_kat(orc):
    # TL/Loading/GgmlDequantTests.cs:132-170
    p = np.array([0xC0] * 4 + [0x80] * 4 + [0x35] * 4, np.uint8)
    sc, m = orc.unpack_q4k_scales_mins(p)
    assert list(sc) == [0] * 4 + [0x35] * 4
    assert list(m) == [0] * 4 + [0x23] * 4


def test_unpack_is_a_bijection_with_pack(orc):
    # 96 bits <-> 16 six-bit fields: pack(unpack(p)) == p for every 12-byte p, and the inverse.
    rng = np.random.default_rng(2)
    for _ in range(3000):
        p = rng.integers(0, 256, 12, dtype=np.uint8)
        sc, m = orc.unpack_q4k_scales_mins(p)
        assert sc.max() < 64 and m.max() < 64
        assert np.array_equal(orc.pack_q4k_scales_mins(sc, m), p)
        sc2 = rng.integers(0, 64, 8, dtype=np.uint8)
        m2 = rng.integers(0, 64, 8, dtype=np.uint8)
        s3, m3 = orc.unpack_q4k_scales_mins(orc.pack_q4k_scales_mins(sc2, m2))
        assert np.array_equal(s3, sc2) and np.array_equal(m3, m2)


def test_unpack_each_field_depends_on_the_documented_bits(orc):
    # Brute force: flipping one input bit changes exactly the one 6-bit field the ggml layout assigns it.
    def owner(byte, bit):
        if byte < 4:
            return ("sc", byte) if bit < 6 else ("sc", byte + 4)
        if byte < 8:
            return ("m", byte - 4) if bit < 6 else ("m", byte)
        return ("sc", byte - 4) if bit < 4 else ("m", byte - 4)

    base = np.zeros(12, np.uint8)
    s0, m0 = orc.unpack_q4k_scales_mins(base)
    for byte in range(12):
        for bit in range(8):
            p = base.copy()
            p[byte] ^= 1 << bit
            s1, m1 = orc.unpack_q4k_scales_mins(p)
            changed = [("sc", j) for j in range(8) if s1[j] != s0[j]] + [("m", j) for j in range(8) if m1[j] != m0[j]]
            assert changed == [owner(byte, bit)], (byte, bit, changed)


# ------------------------------------------------------------------------------------------------ a19 decode

def _q4k_block(d, dmin, packed, fill):
    b = np.zeros(144, np.uint8)
    b[0:2] = np.frombuffer(np.float16(d).tobytes(), np.uint8)
    b[2:4] = np.frombuffer(np.float16(dmin).tobytes(), np.uint8)
    b[4:16] = packed
    b[16:] = fill
    return b


def test_decode_q4k_kat_unit_scales(orc):
    # TL/Loading/GgmlDequantTests.cs:188-208: d=1, dmin=0, scales 1, mins 0, nibbles 0x21
    packed = np.zeros(12, np.uint8)
    packed[:4] = 1
    packed[8:12] = 1  # scales[4..7] low nibble = 1
    dst = orc.decode_q4k_block(_q4k_block(1.0, 0.0, packed, 0x21))
    for p in range(4):
        assert np.all(dst[64 * p:64 * p + 32] == 1.0)
        assert np.all(dst[64 * p + 32:64 * p + 64] == 2.0)


def test_decode_q4k_kat_scale_and_min_per_sub_block(orc):
    # TL/Loading/GgmlDequantTests.cs:210-249
    packed = np.zeros(12, np.uint8)
    packed[:4] = [1, 2, 3, 4]
    packed[4:8] = [0, 1, 2, 3]
    for j in range(4, 8):
        packed[j + 4] = ((j << 4) | ((j + 1) & 0x0F)) & 0xFF
    dst = orc.decode_q4k_block(_q4k_block(2.0, 1.0, packed, 0x53))
    for p in range(4):
        lo = 2.0 * (2 * p + 1) * 3 - 1.0 * (2 * p)
        hi = 2.0 * (2 * p + 2) * 5 - 1.0 * (2 * p + 1)
        assert np.all(dst[64 * p:64 * p + 32] == lo)
        assert np.all(dst[64 * p + 32:64 * p + 64] == hi)


def _q5_0_block(d, qh, qs_fill):
    b = np.zeros(22, np.uint8)
    b[0:2] = np.frombuffer(np.float16(d).tobytes(), np.uint8)
    b[2:6] = np.frombuffer(np.uint32(qh).tobytes(), np.uint8)
    b[6:] = qs_fill
    return b


def test_decode_q5_0_kats(orc):
    # TL/Loading/GgmlDequantTests.cs:330-380: zero quants give the -16 bias; low nibble -> element j, high -> j + 16;
    # qh bit k -> element k.
    assert np.all(orc.decode_q5_0_block(_q5_0_block(1.0, 0, 0x00)) == -16.0)
    dst = orc.decode_q5_0_block(_q5_0_block(2.0, 0, 0x21))
    assert np.all(dst[:16] == -30.0) and np.all(dst[16:] == -28.0)
    for k in (0, 16, 31):
        dst = orc.decode_q5_0_block(_q5_0_block(1.0, 1 << k, 0x00))
        assert dst[k] == 0.0 and np.all(np.delete(dst, k) == -16.0)


def test_decode_q5_0_every_bit_owns_one_element(orc):
    # Brute force over all 32 qh bits and all 32 nibbles (d = 1, so every value is the integer q - 16): each bit
    # moves exactly the element the block format gives it, by its weight (16 for qh, 1..8 for a nibble bit).
    base = orc.decode_q5_0_block(_q5_0_block(1.0, 0, 0x00))
    for k in range(32):
        diff = orc.decode_q5_0_block(_q5_0_block(1.0, 1 << k, 0x00)) - base
        assert np.flatnonzero(diff).tolist() == [k] and diff[k] == 16.0
    for j in range(16):
        for bit in range(8):
            b = _q5_0_block(1.0, 0, 0x00)
            b[6 + j] = 1 << bit
            diff = orc.decode_q5_0_block(b) - base
            elem = j if bit < 4 else j + 16
            assert np.flatnonzero(diff).tolist() == [elem] and diff[elem] == float(1 << (bit % 4))


def test_decode_q5_0_scale_is_exact_multiplication(orc):
    # Random blocks: every element is (q - 16) * d with q the 5-bit code (exact products, so float64 agrees).
    rng = np.random.default_rng(50)
    for _ in range(200):
        b = rng.integers(0, 256, 22, dtype=np.uint8)
        b[0:2] = np.frombuffer(np.float16(rng.uniform(-0.05, 0.05)).tobytes(), np.uint8)
        d = np.float64(np.frombuffer(b[0:2].tobytes(), np.float16)[0])
        qh = int(np.frombuffer(b[2:6].tobytes(), np.uint32)[0])
        q = np.array([((int(b[6 + (i % 16)]) >> (4 * (i // 16))) & 15) | (((qh >> i) & 1) << 4) for i in range(32)])
        assert np.array_equal(orc.decode_q5_0_block(b).astype(np.float64), (q - 16) * d)


def _q5k_block(d, dmin, packed, qh_fill, qs_fill):
    b = np.zeros(176, np.uint8)
    b[0:2] = np.frombuffer(np.float16(d).tobytes(), np.uint8)
    b[2:4] = np.frombuffer(np.float16(dmin).tobytes(), np.uint8)
    b[4:16] = packed
    b[16:48] = qh_fill
    b[48:] = qs_fill
    return b


def test_decode_q5k_kats(orc):
    # TL/Loading/GgmlDequantTests.cs:392-436: scales 1, mins 0, nibbles 0x21 -> 1 / 2 per 32-element half; every qh
    # bit set adds 16 -> 17 / 18.
    packed = np.zeros(12, np.uint8)
    packed[:4] = 1
    packed[8:12] = 1
    for qh, lo, hi in ((0x00, 1.0, 2.0), (0xFF, 17.0, 18.0)):
        dst = orc.decode_q5k_block(_q5k_block(1.0, 0.0, packed, qh, 0x21))
        for g in range(4):
            assert np.all(dst[64 * g:64 * g + 32] == lo) and np.all(dst[64 * g + 32:64 * g + 64] == hi)


def test_decode_q5k_without_fifth_bits_is_the_q4k_decode(orc):
    # With qh = 0 a Q5_K block is the Q4_K block with the same d, dmin, packed scales/mins and nibbles (the formats
    # share the element map and the float operations), so it decodes bit-identically to the pinned Q4_K decoder.
    rng = np.random.default_rng(51)
    for b4 in random_q4k_blocks(rng, 300):
        b5 = np.zeros(176, np.uint8)
        b5[:16] = b4[:16]
        b5[48:] = b4[16:]
        assert np.array_equal(orc.decode_q5k_block(b5).view(np.uint32), orc.decode_q4k_block(b4).view(np.uint32))


def test_decode_q5k_every_fifth_bit_owns_one_element(orc):
    # d = 1, dmin = 0, all scales 1: qh byte l bit b lifts exactly element 64 (b // 2) + 32 (b % 2) + l by 16.
    packed = np.zeros(12, np.uint8)
    packed[:4] = 1
    packed[8:12] = 1
    base = orc.decode_q5k_block(_q5k_block(1.0, 0.0, packed, 0x00, 0x00))
    for l in range(32):
        for bit in range(8):
            b = _q5k_block(1.0, 0.0, packed, 0x00, 0x00)
            b[16 + l] = 1 << bit
            diff = orc.decode_q5k_block(b) - base
            elem = 64 * (bit // 2) + 32 * (bit % 2) + l
            assert np.flatnonzero(diff).tolist() == [elem] and diff[elem] == 16.0


@pytest.mark.parametrize("type_id,k", [(6, 96), (6, 4096), (13, 256), (13, 1024)])
def test_q5_requantize_is_decode_then_quantize_rows(orc, type_id, k):
    # The loader's Q5 -> Q8_0 path: the resident planes are Q8Weight.QuantizeRows of the decoded F32 rows; their
    # dequantised values stay within half a Q8_0 step of the decoded weights (ties of a 5-bit grid against the
    # 127-step grid reach exactly half a step, so the bound allows the float error of scale and 1 / scale).
    rng = np.random.default_rng(type_id * 1000 + k)
    rows = 7
    bb, blk = (22, 32) if type_id == 6 else (176, 256)
    data = rng.integers(0, 256, (rows, k // blk, bb), dtype=np.uint8)
    data[..., 0:2] = np.frombuffer(rng.uniform(0.001, 0.05, rows * (k // blk)).astype(np.float16).tobytes(),
                                   np.uint8).reshape(rows, k // blk, 2)
    if type_id == 13:
        data[..., 2:4] = np.frombuffer(rng.uniform(0.001, 0.03, rows * (k // blk)).astype(np.float16).tobytes(),
                                       np.uint8).reshape(rows, k // blk, 2)
    dec = orc.decode_q5_0_block if type_id == 6 else orc.decode_q5k_block
    f32 = np.stack([np.concatenate([dec(data[r, b]) for b in range(k // blk)]) for r in range(rows)])
    q, s = orc.q5_requantize_q8_0(type_id, data, rows, k)
    q_ref, s_ref = orc.q8_quantize_rows(f32)
    assert np.array_equal(q, q_ref) and np.array_equal(s.view(np.uint32), s_ref.view(np.uint32))
    back = q.astype(np.float64).reshape(rows, -1, 32) * s.astype(np.float64)[..., None]
    step = s.astype(np.float64)[..., None]
    assert np.all(np.abs(back - f32.reshape(rows, -1, 32)) <= 0.5 * step * (1 + 1e-5))


def _q6k_block(d, scales, ql=None, ql_fill=0, qh_fill=0):
    b = np.zeros(210, np.uint8)
    b[:128] = ql_fill if ql is None else ql
    b[128:192] = qh_fill
    b[192:208] = np.array(scales, np.int8).view(np.uint8)
    b[208:210] = np.frombuffer(np.float16(d).tobytes(), np.uint8)
    return b


def test_decode_q6k_kats(orc):
    # TL/Loading/GgmlDequantTests.cs:262-319
    assert np.all(orc.decode_q6k_block(_q6k_block(1.0, [1] * 16)) == -32.0)
    assert np.all(orc.decode_q6k_block(_q6k_block(0.5, [-1] * 16, ql_fill=0xFF, qh_fill=0xFF)) == -15.5)
    ql = np.zeros(128, np.uint8)
    ql[0] = 0x10
    dst = orc.decode_q6k_block(_q6k_block(1.0, [1] * 16, ql=ql))
    assert dst[64] == -31.0
    assert dst[0] == dst[32] == dst[96] == dst[128] == dst[255] == -32.0


def test_decode_q6k_element_map_codes(orc):
    # Every element position probed alone (d=1, only its sub-block's scale = 1, its 6-bit code = 63): the
    # decoded vector is 31 there, -32 on the other members of that sub-block and 0 elsewhere. Pins the
    # ql/qh/scale index map of LD/GgmlDequant.cs:184-206. Elements of the lit sub-block decode to -32 except the
    # probed one (31); all other sub-blocks have scale 0 and decode to 0.
    for h in range(2):
        for grp in range(4):
            for l in (0, 7, 16, 31):
                i = 128 * h + 32 * grp + l
                ql = np.zeros(128, np.uint8)
                qh = np.zeros(64, np.uint8)
                ql[64 * h + l + (32 if grp & 1 else 0)] = 0xF0 if grp >= 2 else 0x0F
                qh[32 * h + l] = 3 << (2 * grp)
                s = 8 * h + l // 16 + 2 * grp
                sc = [0] * 16
                sc[s] = 1
                b = _q6k_block(1.0, sc, ql=ql)
                b[128:192] = qh
                dst = orc.decode_q6k_block(b)
                members = [128 * h + 32 * g + ll for g in range(4) for ll in range(32)
                           if 8 * h + ll // 16 + 2 * g == s]
                exp = np.zeros(256, np.float32)
                exp[members] = -32.0
                exp[i] = 31.0
                assert np.array_equal(dst, exp), (h, grp, l)


# ------------------------------------------------------------------------------------------------ a3 / a11

def _np_quantize_q8(x, block):
    # numpy restatement of the published formula (vectorised, independent code path)
    xb = x.reshape(-1, block)
    am = np.abs(xb).max(axis=1).astype(np.float32)
    scale = (am / np.float32(127.0)).astype(np.float32)
    inv = np.where(scale > 0, np.float32(1.0) / np.where(scale > 0, scale, 1), 0).astype(np.float32)
    q = np.clip(np.rint((xb * inv[:, None]).astype(np.float32)), -127, 127).astype(np.int8)
    return q.reshape(-1), scale


def test_quantize_q8k_reference_invariants(orc):
    # TL/Runtime/Q4KDotKernelTests.cs:166-216
    rng = np.random.default_rng(7)
    x = (rng.random(256) * 2 - 1).astype(np.float32)
    q, d, b = orc.quantize_q8k(x)
    assert np.all(np.abs(d[0, 0] * q[0].astype(np.float32) - x) <= d[0, 0])
    assert np.array_equal(b[0], q[0].reshape(16, 16).astype(np.int32).sum(1))
    q, d, b = orc.quantize_q8k(np.zeros(256, np.float32))
    assert d[0, 0] == 0 and not q.any() and not b.any()


def test_quantize_q8k_closed_form_and_ties(orc):
    # absmax 127 => scale 1, inverse 1: quants are rint(x) — ties go to even (MathF.Round, not away from zero)
    x = np.zeros(256, np.float32)
    x[0] = 127.0
    x[1:9] = [2.5, 3.5, -2.5, -3.5, 0.5, -0.5, 1.5, 126.5]
    q, d, b = orc.quantize_q8k(x)
    assert d[0, 0] == 1.0
    assert list(q[0, :9]) == [127, 2, 4, -2, -4, 0, 0, 2, 126]
    assert b[0, 0] == 127 + 2 + 4 - 2 - 4 + 0 + 0 + 2 + 126


def test_quantize_q8k_matches_numpy_restatement(orc):
    rng = np.random.default_rng(11)
    x = normal(rng, (5, 1024))
    x[2, :256] = 0.0
    q, d, b = orc.quantize_q8k(x)
    for r in range(5):
        qn, sn = _np_quantize_q8(x[r], 256)
        assert np.array_equal(q[r], qn)
        assert np.array_equal(d[r], sn)
        assert np.array_equal(b[r], qn.reshape(-1, 16).astype(np.int32).sum(1))


def test_quantize_q8_0_matches_numpy_and_reference_invariants(orc):
    # TL/Runtime/Q8DotKernelTests.cs:94-123 (error <= half step) + numpy restatement
    rng = np.random.default_rng(12)
    x = normal(rng, (3, 4096))
    q, s = orc.quantize_q8_0(x)
    for r in range(3):
        qn, sn = _np_quantize_q8(x[r], 32)
        assert np.array_equal(q[r], qn) and np.array_equal(s[r], sn)
        rec = np.repeat(s[r], 32) * q[r].astype(np.float32)
        assert np.all(np.abs(rec - x[r]) <= np.repeat(s[r], 32) * 0.5 + 1e-7)


# ------------------------------------------------------------------------------------------------ dots

def _blk_with(block, d_bits=None, dmin_bits=None, q6=False):
    b = block.copy()
    if q6:
        b[208], b[209] = d_bits & 0xFF, d_bits >> 8
    else:
        if d_bits is not None:
            b[0], b[1] = d_bits & 0xFF, d_bits >> 8
        if dmin_bits is not None:
            b[2], b[3] = dmin_bits & 0xFF, dmin_bits >> 8
    return b


def test_q4k_int_dots_equal_decoded_integer_weights(orc):
    # With d=1, dmin=0 the decode of a block is the integer weight sc[s]*nib; with d=0, dmin=1 it is -m[s].
    # MainDot and the min term must equal the exact integer dots of those decoded weights with q8.
    rng = np.random.default_rng(21)
    L = orc.lib()
    one, zero = int(half_bits(1.0)), int(half_bits(0.0))
    for blk in random_q4k_blocks(rng, 300):
        x = normal(rng, 256)
        q, d, b = orc.quantize_q8k(x)
        w_sc = orc.decode_q4k_block(_blk_with(blk, one, zero)).astype(np.int64)
        w_m = -orc.decode_q4k_block(_blk_with(blk, zero, one)).astype(np.int64)
        sc, m = orc.unpack_q4k_scales_mins(blk[4:16])
        main = L.orc_q4k_main_dot(orc.P(blk[16:].copy()), orc.P(q[0]), orc.P(sc))
        mn = L.orc_q4k_min_acc(orc.P(m), orc.P(b[0]))
        assert main == int((w_sc * q[0].astype(np.int64)).sum())
        assert mn == int((w_m * q[0].astype(np.int64)).sum())


def test_q4k_dot_matches_float64_decode_dot(orc):
    rng = np.random.default_rng(22)
    L = orc.lib()
    for blk in random_q4k_blocks(rng, 200):
        x = normal(rng, 256)
        q, d, b = orc.quantize_q8k(x)
        got = L.orc_q4k_dot(orc.P(blk), orc.P(q[0]), float(d[0, 0]), orc.P(b[0]))
        ref = float((orc.decode_q4k_block(blk).astype(np.float64) * q[0] * float(d[0, 0])).sum())
        scale = float((np.abs(orc.decode_q4k_block(blk).astype(np.float64) * q[0] * float(d[0, 0]))).sum())
        assert abs(got - ref) <= 1e-5 * scale + 1e-30


def test_q6k_int_dot_equals_decoded_integer_weights(orc):
    rng = np.random.default_rng(23)
    L = orc.lib()
    one = int(half_bits(1.0))
    for blk in random_q6k_blocks(rng, 300):
        x = normal(rng, 256)
        q, d, b = orc.quantize_q8k(x)
        w_int = orc.decode_q6k_block(_blk_with(blk, one, q6=True)).astype(np.int64)  # sc*(q-32), exact
        u = L.orc_q6k_unsigned_dot(orc.P(blk), orc.P(q[0]))
        bt = L.orc_q6k_bsum_term(orc.P(blk), orc.P(b[0]))
        assert u - 32 * bt == int((w_int * q[0].astype(np.int64)).sum())


def test_q6k_dot_matches_float64_decode_dot(orc):
    rng = np.random.default_rng(24)
    L = orc.lib()
    for blk in random_q6k_blocks(rng, 200):
        x = normal(rng, 256)
        q, d, b = orc.quantize_q8k(x)
        got = L.orc_q6k_dot(orc.P(blk), orc.P(q[0]), float(d[0, 0]), orc.P(b[0]))
        t = orc.decode_q6k_block(blk).astype(np.float64) * q[0] * float(d[0, 0])
        assert abs(got - t.sum()) <= 1e-5 * np.abs(t).sum() + 1e-30


def test_q8_dot_reference_cases(orc):
    # TL/Runtime/Q8DotKernelTests.cs:34-92
    L = orc.lib()
    rng = np.random.default_rng(25)
    for n in (32, 320, 2048, 11008):
        a = (rng.random(n) * 2 - 1).astype(np.float32)
        bvec = (rng.random(n) * 2 - 1).astype(np.float32)
        qa, sa = orc.quantize_q8_0(a)
        qb, sb = orc.quantize_q8_0(bvec)
        got = L.orc_q8_dot(orc.P(qa[0]), orc.P(sa[0]), orc.P(qb[0]), orc.P(sb[0]), n)
        ref = float(np.dot(a.astype(np.float64), bvec.astype(np.float64)))
        assert abs(got - ref) < 0.03 * abs(ref) or abs(got - ref) < 0.5
    z = np.zeros(64, np.float32)
    qz, sz = orc.quantize_q8_0(z)
    assert L.orc_q8_dot(orc.P(qz[0]), orc.P(sz[0]), orc.P(qz[0]), orc.P(sz[0]), 64) == 0.0
    ones = np.ones(256, np.float32)
    qo, so = orc.quantize_q8_0(ones)
    assert abs(L.orc_q8_dot(orc.P(qo[0]), orc.P(so[0]), orc.P(qo[0]), orc.P(so[0]), 256) - 256.0) < 1e-3


# ------------------------------------------------------------------------------------------------ projections

def _f32_reference_project(decode, blocks, k, n, x, bpb):
    spr = k // 256
    out = np.zeros(n, np.float64)
    for o in range(n):
        row = np.concatenate([decode(blocks[o, sb * bpb:(sb + 1) * bpb]) for sb in range(spr)])
        out[o] = np.dot(row.astype(np.float64), x.astype(np.float64))
    return out


@pytest.mark.parametrize("fmt", ["q4k", "q6k"])
def test_project_matches_f32_decode_within_q8_noise(orc, fmt):
    # TL/Runtime/Q4KDotKernelTests.cs:31-65, Q6KDotKernelTests.cs:31-65: L2-relative < 3%
    rng = np.random.default_rng(20260519)
    k, n = 512, 96
    x = (rng.random(k) * 2 - 1).astype(np.float32)
    if fmt == "q4k":
        blocks = random_q4k_blocks(rng, n * 2).reshape(n, -1)
        y = orc.q4k_project(x, blocks, k, n)
        ref = _f32_reference_project(orc.decode_q4k_block, blocks, k, n, x, 144)
    else:
        blocks = random_q6k_blocks(rng, n * 2).reshape(n, -1)
        y = orc.q6k_project(x, blocks, k, n)
        ref = _f32_reference_project(orc.decode_q6k_block, blocks, k, n, x, 210)
    l2 = np.sqrt(((y - ref) ** 2).sum() / (ref ** 2).sum())
    assert l2 < 0.03


def test_q8_project_matches_f32(orc):
    # TL/Runtime/Q8DotKernelTests.cs:125-201
    rng = np.random.default_rng(26)
    for k, n in ((64, 16), (256, 96), (512, 33), (256, 11008)):
        w = normal(rng, (n, k), 0.05)
        wq, ws = orc.q8_quantize_rows(w)
        x = normal(rng, k)
        y = orc.q8_project(x, wq, ws, k, n)
        ref = w.astype(np.float64) @ x.astype(np.float64)
        l2 = np.sqrt(((y - ref) ** 2).sum() / (ref ** 2).sum())
        assert l2 < 0.03


def _heads(orc, rng, H, hd, dm):
    planes = [orc.q8_quantize_rows(normal(rng, (dm, hd), 0.05)) for _ in range(H)]
    return [p[0] for p in planes], [p[1] for p in planes]


@pytest.mark.parametrize("H,hd,dm,rows", [(1, 128, 96, 1), (32, 128, 256, 2), (8, 96, 64, 3), (4, 256, 40, 1)])
def test_q8_project_heads_is_the_ascending_sum_of_head_projections(orc, H, hd, dm, rows):
    """The per-head o-path (RT/CachedMultiHeadAttention.cs:185-194, :292-297, :600-614, :703-711): output starts as
    the bias (or zero) and each head's Q8DotKernel.Project (already pinned) is added in ascending head order, one
    float32 add per output and head. Restated here from the pinned single-head projection and numpy float32 adds;
    the plausible mistakes (descending order, or one fused Q8 dot over all heads as a single [d_model][H*hd]
    matrix) are shown to differ, so the check can tell them apart."""
    rng = np.random.default_rng(H * 1000 + hd + rows)
    wqs, wss = _heads(orc, rng, H, hd, dm)
    x = normal(rng, (rows, H * hd))
    bias = normal(rng, dm)
    for b in (None, bias):
        y = orc.q8_project_heads(x, rows, wqs, wss, hd, dm, b)
        for n in range(rows):
            ref = np.zeros(dm, np.float32) if b is None else b.copy()
            for h in range(H):
                ref = (ref + orc.q8_project(x[n, h * hd:(h + 1) * hd], wqs[h], wss[h], hd, dm)).astype(np.float32)
            assert np.array_equal(y[n].view(np.uint32), ref.view(np.uint32)), (b is None, n)
    if H == 1:  # one head and no bias is exactly the single projection
        y = orc.q8_project_heads(x, rows, wqs, wss, hd, dm)
        assert np.array_equal(y[0].view(np.uint32), orc.q8_project(x[0], wqs[0], wss[0], hd, dm).view(np.uint32))
        return
    y = orc.q8_project_heads(x, rows, wqs, wss, hd, dm, bias)
    rev = bias.copy()
    for h in reversed(range(H)):
        rev = (rev + orc.q8_project(x[0, h * hd:(h + 1) * hd], wqs[h], wss[h], hd, dm)).astype(np.float32)
    assert not np.array_equal(y[0].view(np.uint32), rev.view(np.uint32)), "order not distinguished"
    whole_q = np.concatenate(wqs, axis=1)  # [dm][H*hd]: the heads as one Q8 matrix
    whole_s = np.concatenate(wss, axis=1)
    fused = orc.q8_project(x[0], whole_q, whole_s, H * hd, dm, bias)
    assert not np.array_equal(y[0].view(np.uint32), fused.view(np.uint32)), "fused dot not distinguished"
    # and the value itself: within Q8 noise of the float64 product with the dequantised weights
    w64 = np.concatenate([q.astype(np.float64) * np.repeat(s, 32, axis=1) for q, s in zip(wqs, wss)], axis=1)
    ref64 = w64 @ x[0].astype(np.float64) + bias
    assert np.max(np.abs(y[0] - ref64)) <= 0.03 * np.max(np.abs(ref64))


@pytest.mark.parametrize("rows", [1, 3, 16, 70])
def test_batched_is_bit_identical_to_per_row_project(orc, rows):
    # TL/Runtime/Q4KDotKernelTests.cs:98-136, Parity/Q4KWeightStationaryParityTests.cs:19-71,
    # Q6KDotKernelTests.cs, Q8DotKernelTests.cs:203-289
    rng = np.random.default_rng(rows * 17 + 5)
    k, n = 512, 96
    x = (rng.random((rows, k)) * 2 - 1).astype(np.float32)
    bias = (rng.random(n) - 0.5).astype(np.float32)
    b4 = random_q4k_blocks(rng, n * 2).reshape(n, -1)
    per_row = np.stack([orc.q4k_project(x[r], b4, k, n, bias) for r in range(rows)])
    assert np.array_equal(orc.q4k_project_batched(x, rows, b4, k, n, bias), per_row)
    assert np.array_equal(orc.q4k_project_batched_ws(x, rows, b4, k, n, bias), per_row)
    b6 = random_q6k_blocks(rng, n * 2).reshape(n, -1)
    per_row6 = np.stack([orc.q6k_project(x[r], b6, k, n, bias) for r in range(rows)])
    assert np.array_equal(orc.q6k_project_batched(x, rows, b6, k, n, bias), per_row6)
    wq, ws = orc.q8_quantize_rows(normal(rng, (n, k), 0.05))
    per_row8 = np.stack([orc.q8_project(x[r], wq, ws, k, n, bias) for r in range(rows)])
    assert np.array_equal(orc.q8_project_batched(x, rows, wq, ws, k, n, bias), per_row8)


def test_gate_up_is_two_projects_and_bias_adds(orc):
    # RT/Q4KDotKernel.cs:563-605 ("bit-identical to two ProjectParallel calls"); Q4KDotKernelTests.cs:138-164
    rng = np.random.default_rng(27)
    k, n = 768, 40
    x = normal(rng, k)
    g = random_q4k_blocks(rng, n * 3).reshape(n, -1)
    u = random_q4k_blocks(rng, n * 3).reshape(n, -1)
    go, uo = orc.q4k_project_gate_up(x, g, u, k, n)
    assert np.array_equal(go, orc.q4k_project(x, g, k, n))
    assert np.array_equal(uo, orc.q4k_project(x, u, k, n))
    bias = normal(rng, n)
    yb = orc.q4k_project(x, g, k, n, bias)
    assert np.array_equal(yb, bias + orc.q4k_project(x, g, k, n))


# ------------------------------------------------------------------------------------------------ a18 encoder

@pytest.mark.parametrize("seed", [1, 2, 3])
def test_quantize_q4k_round_trips_within_precision(orc, seed):
    # TL/Loading/GgmlQuantTests.cs:23-86
    rng = np.random.default_rng(seed)
    k, n = 512, 8
    i = np.arange(n * k)
    f32 = ((rng.random(n * k) * 2 - 1) * (0.2 + (i % 7) * 0.1)).astype(np.float32).reshape(n, k)
    blocks = orc.quantize_q4k(f32)
    dec = np.stack([orc.q4k_decode_row(blocks, k, n, o) for o in range(n)]).astype(np.float64)
    a = f32.astype(np.float64)
    cos = (a * dec).sum() / np.sqrt((a * a).sum() * (dec * dec).sum())
    rmse = np.sqrt(((a - dec) ** 2).mean())
    avg_range = np.mean(f32.max(1) - f32.min(1))
    assert cos > 0.995
    assert rmse < 0.02 * avg_range


def test_quantize_q4k_constant_row(orc):
    # TL/Loading/GgmlQuantTests.cs:88-108, plus the bytes derived by hand: lo clamps to 0, so every
    # sub-scale is 0.37/15, sc = 63, m = 0, dmin = 0, nibbles round to 15.
    f32 = np.full((1, 256), 0.37, np.float32)
    blk = orc.quantize_q4k(f32)[0]
    dec = orc.decode_q4k_block(blk)
    assert np.max(np.abs(dec - 0.37)) < 1e-3
    d = np.float32(np.float32(0.37) / np.float32(15.0)) / np.float32(63.0)
    assert int(blk[0]) | (int(blk[1]) << 8) == int(half_bits(d))
    assert blk[2] == 0 and blk[3] == 0
    assert list(blk[4:16]) == [0xFF] * 4 + [0x00] * 4 + [0x0F] * 4
    assert np.all(blk[16:] == 0xFF)


# ------------------------------------------------------------------------------------------------ Q6_K encoder

def test_quantize_q6k_round_trip_and_step_bound(orc):
    rng = np.random.default_rng(31)
    k, n = 512, 16
    f32 = normal(rng, (n, k), 0.02)
    blocks = orc.quantize_q6k(f32)
    for o in range(n):
        dec = orc.q6k_decode_row(blocks, k, n, o)
        for sb in range(k // 256):
            blk = blocks[o, sb * 210:(sb + 1) * 210]
            dh = np.frombuffer(blk[208:210].tobytes(), np.float16)[0].astype(np.float32)
            sc = blk[192:208].view(np.int8).astype(np.float32)
            step = np.abs(np.repeat(dh * sc, 16))
            err = np.abs(dec[sb * 256:(sb + 1) * 256] - f32[o, sb * 256:(sb + 1) * 256])
            # rounding: half a step; only codes clamped at +31 (x/step in (31.5, 32.x]) may reach 1.5 steps
            code = f32[o, sb * 256:(sb + 1) * 256] / np.repeat(dh * sc, 16)
            inside = np.abs(code) <= 31.5
            assert np.all(err[inside] <= step[inside] * 0.5 * (1 + 1e-6) + 1e-12)
            assert np.all(err <= step * 1.5 + 1e-12)
    dec = np.stack([orc.q6k_decode_row(blocks, k, n, o) for o in range(n)]).astype(np.float64)
    a = f32.astype(np.float64)
    assert (a * dec).sum() / np.sqrt((a * a).sum() * (dec * dec).sum()) > 0.999


def test_quantize_q6k_zero_and_constant_blocks(orc):
    z = orc.quantize_q6k(np.zeros((1, 256), np.float32))
    assert not z.any()
    c = orc.quantize_q6k(np.full((1, 256), -0.5, np.float32))
    assert np.max(np.abs(orc.decode_q6k_block(c[0]) + 0.5)) < 1e-3


# ------------------------------------------------------------------------------------------------ MoE router

def test_moe_router_kats(orc):
    # TL/Runtime/MoeRouterTests.cs:18-151
    idx, w = orc.moe_select_topk([0.1, 2.0, -1.0, 0.5], 1)
    assert list(idx) == [1] and abs(w[0] - 1.0) < 1e-5
    idx, w = orc.moe_select_topk([0.1, 2.0, -1.0, 1.5], 2)
    assert list(idx) == [1, 3] and w[0] > w[1]
    idx, w = orc.moe_select_topk([0.3, 1.1, 0.7, -0.4, 2.2], 3)
    assert abs(w.sum() - 1.0) < 1e-5
    logits = np.array([0.5, 2.0, 1.0, 1.8], np.float32)
    full = np.exp(logits - logits.max())
    full /= full.sum()
    idx, w = orc.moe_select_topk(logits, 2)
    assert list(idx) == [1, 3]
    assert abs(w[0] - full[1] / (full[1] + full[3])) < 1e-5 and abs(w[1] - full[3] / (full[1] + full[3])) < 1e-5
    idx, w = orc.moe_select_topk(logits, 2, normalize=False)
    assert abs(w[0] - full[1]) < 1e-5 and abs(w[1] - full[3]) < 1e-5 and w.sum() < 1
    idx, w = orc.moe_select_topk([1.0, 0.0], 5)
    assert len(idx) == 2 and idx[0] == 0 and abs(w.sum() - 1) < 1e-5
    idx, w = orc.moe_select_topk([1.0, 1.0, 0.5], 1)
    assert list(idx) == [0]  # ties keep the lower index


# ------------------------------------------------------------------------------------------------ GGUF Q8_0

def test_q8_0_deinterleave_round_trip(orc):
    """LoadTensorQ8_0Raw: interleaving (quants, fp16 scale bits) into 34-byte blocks and back returns the quants and
    the scale widened exactly (numpy float16 -> float32), for every fp16 pattern class (subnormal, inf, -0)."""
    rng = np.random.default_rng(9)
    nb = 4096
    q = rng.integers(-128, 128, size=(nb, 32), dtype=np.int8)
    bits = rng.integers(0, 65536, size=nb, dtype=np.uint32).astype(np.uint16)
    bits[:4] = [0x0001, 0x8000, 0x7C00, 0x3C00]
    blocks = np.zeros((nb, 34), np.uint8)
    blocks[:, 0] = bits & 0xFF
    blocks[:, 1] = bits >> 8
    blocks[:, 2:] = q.view(np.uint8)
    gq, gs = orc.q8_0_deinterleave(blocks)
    assert np.array_equal(gq, q.ravel())
    ref = bits.view(np.float16).astype(np.float32)
    finite = ~np.isnan(ref)
    assert np.array_equal(gs[finite].view(np.uint32), ref[finite].view(np.uint32))


def test_q8_0_gguf_dequant_kats(orc):
    """LoadTensorQ8_0Raw on the reference's two Q8_0 known-answer blocks: the planes hold the quants and the exactly
    widened scales, so dequantised values are scale * quant: -256 and 254 for -128 and 127 at scale 2."""
    for scales, quants in Q8_0_KATS:
        q, s = orc.q8_0_deinterleave(q8_0_gguf_blocks(scales, quants))
        assert np.array_equal(q, quants)
        assert s.tolist() == scales
        deq = np.repeat(s, 32) * q.astype(np.float32)
        for b, sc in enumerate(scales):
            for i in (0, 1, 4, 31):
                assert deq[32 * b + i] == sc * int(quants[32 * b + i])
    q, s = orc.q8_0_deinterleave(q8_0_gguf_blocks(*Q8_0_KATS[0]))
    assert (np.repeat(s, 32) * q.astype(np.float32))[[0, 1, 2, 3, 4]].tolist() == [-256.0, -2.0, 0.0, 2.0, 254.0]


# ------------------------------------------------------------------------------------------------ MoE FFN

def _small_experts(orc, rng, E, dm, dff, gate_fmt="q4k", down_fmt="q6k"):
    """E experts of N(0, 0.05) weights quantised by the oracle's own (pinned) encoders."""
    enc = {"q4k": orc.quantize_q4k, "q6k": orc.quantize_q6k}
    mk = lambda fmt, n, k: enc[fmt](normal(rng, (n, k), 0.05))
    return ([mk(gate_fmt, dff, dm) for _ in range(E)], [mk(gate_fmt, dff, dm) for _ in range(E)],
            [mk(down_fmt, dm, dff) for _ in range(E)])


def test_swiglu_batched_matches_f64_dequantised_ffn(orc):
    """orc_swiglu_batched against W_down (silu(W_gate x) * (W_up x)) in float64 on the dequantised weights: only
    the Q8_K activation quantisation separates them (~1%); swapping gate and up, dropping SiLU or feeding the
    down projection the wrong operand fails by far more."""
    rng = np.random.default_rng(77)
    dm, dff, rows = 512, 768, 3
    (g,), (u,), (d,) = _small_experts(orc, rng, 1, dm, dff)
    x = normal(rng, (rows, dm))
    y = orc.swiglu_batched(x, rows, g, u, d, 12, 14, dm, dff)
    dq = lambda blocks, k, n, fn: np.stack([fn(blocks, k, n, r) for r in range(n)]).astype(np.float64)
    Wg, Wu = dq(g, dm, dff, orc.q4k_decode_row), dq(u, dm, dff, orc.q4k_decode_row)
    Wd = dq(d, dff, dm, orc.q6k_decode_row)
    a = x.astype(np.float64) @ Wg.T
    ref = ((a / (1 + np.exp(-a))) * (x.astype(np.float64) @ Wu.T)) @ Wd.T
    err = np.linalg.norm(y - ref) / np.linalg.norm(ref)
    assert err < 0.02, err
    bad = ((a * (x.astype(np.float64) @ Wu.T)) / (1 + np.exp(-(x.astype(np.float64) @ Wu.T)))) @ Wd.T  # gate<->up
    assert np.linalg.norm(y - bad) / np.linalg.norm(ref) > 5 * err


def test_geglu_batched_matches_f64_dequantised_ffn(orc):
    """The GeGLU gate (ApplyGeLU, RT/CachedFeedForwardBlock.cs:498-517: 0.5 x (1 + tanh(sqrt(2/pi)(x + 0.044715
    x^3)))) against the float64 FFN on the dequantised weights with numpy's tanh: only the Q8_K quantisation separates
    them; the SiLU FFN on the same weights is far away, and activation 3 (SwiGLU) is exactly orc_swiglu_batched."""
    rng = np.random.default_rng(78)
    dm, dff, rows = 512, 768, 3
    (g,), (u,), (d,) = _small_experts(orc, rng, 1, dm, dff)
    x = normal(rng, (rows, dm))
    y = orc.gated_ffn_batched(x, rows, g, u, d, 12, 14, dm, dff, 4)
    assert np.array_equal(orc.gated_ffn_batched(x, rows, g, u, d, 12, 14, dm, dff, 3).view(np.uint32),
                          orc.swiglu_batched(x, rows, g, u, d, 12, 14, dm, dff).view(np.uint32))
    dq = lambda blocks, k, n, fn: np.stack([fn(blocks, k, n, r) for r in range(n)]).astype(np.float64)  # noqa: E731
    Wg, Wu = dq(g, dm, dff, orc.q4k_decode_row), dq(u, dm, dff, orc.q4k_decode_row)
    Wd = dq(d, dff, dm, orc.q6k_decode_row)
    a = x.astype(np.float64) @ Wg.T
    gelu = 0.5 * a * (1 + np.tanh(np.sqrt(2 / np.pi) * (a + 0.044715 * a ** 3)))
    ref = (gelu * (x.astype(np.float64) @ Wu.T)) @ Wd.T
    err = np.linalg.norm(y - ref) / np.linalg.norm(ref)
    assert err < 0.02, err
    silu = ((a / (1 + np.exp(-a))) * (x.astype(np.float64) @ Wu.T)) @ Wd.T
    assert np.linalg.norm(y - silu) / np.linalg.norm(ref) > 5 * err
    # the elementwise GELU itself: float32 restatement vs float64 (tanh approximation) on a grid incl. large |x|
    t = np.linspace(-12, 12, 4097).astype(np.float32)
    g64 = 0.5 * t.astype(np.float64) * (1 + np.tanh(np.sqrt(2 / np.pi) * (t + 0.044715 * t.astype(np.float64) ** 3)))
    assert np.max(np.abs(_gelu32(t) - g64)) < 2e-6 * max(1.0, np.max(np.abs(g64)))


def _gelu32(t):
    t = t.astype(np.float32)
    x3 = t * t * t
    inner = np.float32(0.7978845608028654) * (t + np.float32(0.044715) * x3)
    return np.float32(0.5) * t * (np.float32(1.0) + np.tanh(inner).astype(np.float32))


def test_moe_ffn_single_expert_is_the_swiglu_ffn(orc):
    rng = np.random.default_rng(5)
    dm, dff, rows = 256, 512, 4
    g, u, d = _small_experts(orc, rng, 1, dm, dff)
    x = normal(rng, (rows, dm))
    y = orc.moe_ffn_batched(g, u, d, 12, 14, x, rows, dm, dff, 1, np.zeros((rows, 1)), np.ones((rows, 1)))
    assert np.array_equal(y, orc.swiglu_batched(x, rows, g[0], u[0], d[0], 12, 14, dm, dff))


def test_moe_ffn_grouping_and_combine_invariants(orc):
    """Relabelling experts and permuting tokens change nothing but the labels (each token's FFN is row-local);
    two identical experts combine to (0 + w0*o) + w1*o in float32, slot order; an unclaimed slot (index out of
    range, or a repeat of an earlier slot's expert) contributes nothing."""
    rng = np.random.default_rng(6)
    E, dm, dff, rows, k = 4, 256, 512, 7, 2
    g, u, d = _small_experts(orc, rng, E, dm, dff)
    x = normal(rng, (rows, dm))
    idx = np.stack([rng.choice(E, k, replace=False) for _ in range(rows)]).astype(np.int32)
    w = rng.random((rows, k)).astype(np.float32)
    y = orc.moe_ffn_batched(g, u, d, 12, 14, x, rows, dm, dff, k, idx, w)
    perm = rng.permutation(E)  # new label of expert e is perm[e]
    inv = np.argsort(perm)
    y2 = orc.moe_ffn_batched([g[i] for i in inv], [u[i] for i in inv], [d[i] for i in inv], 12, 14, x, rows, dm,
                             dff, k, perm[idx], w)
    assert np.array_equal(y, y2)
    tp = rng.permutation(rows)
    y3 = orc.moe_ffn_batched(g, u, d, 12, 14, x[tp], rows, dm, dff, k, idx[tp], w[tp])
    assert np.array_equal(y3, y[tp])
    # two identical experts
    o = orc.swiglu_batched(x, rows, g[0], u[0], d[0], 12, 14, dm, dff)
    twin = orc.moe_ffn_batched([g[0], g[0]], [u[0], u[0]], [d[0], d[0]], 12, 14, x, rows, dm, dff, 2,
                               np.tile([0, 1], (rows, 1)), w)
    ref = (np.float32(0) + w[:, :1] * o) + w[:, 1:] * o
    assert np.array_equal(twin, ref.astype(np.float32))
    # unclaimed slots
    idx_bad = idx.copy()
    idx_bad[:, 1] = E + 3
    idx_bad[0, 1] = idx_bad[0, 0]
    y4 = orc.moe_ffn_batched(g, u, d, 12, 14, x, rows, dm, dff, k, idx_bad, w)
    only0 = orc.moe_ffn_batched(g, u, d, 12, 14, x, rows, dm, dff, 1, idx[:, :1], w[:, :1])
    assert np.array_equal(y4, only0)


# ------------------------------------------------------------------------------------------------ CPU baseline

def test_cpu_baseline_is_bit_identical_to_oracle(orc):
    L = orc.lib()
    if not L.cpub_has_avx2():
        pytest.skip("no AVX2 on this CPU")
    L.cpub_set_workers(4)
    rng = np.random.default_rng(41)
    k, n = 1024, 203
    x = normal(rng, k)
    q = np.zeros(k, np.int8)
    s = np.zeros(k // 256, np.float32)
    b = np.zeros(k // 16, np.int16)
    q2, s2, b2 = orc.quantize_q8k(x)
    assert L.cpub_quantize_q8k(orc.P(x), k, orc.P(q), orc.P(s), orc.P(b)) == 0
    assert np.array_equal(q, q2[0]) and np.array_equal(s, s2[0]) and np.array_equal(b, b2[0])
    bias = normal(rng, n)
    b4 = random_q4k_blocks(rng, n * 4).reshape(n, -1)
    y = np.zeros(n, np.float32)
    L.cpub_q4k_project_parallel(orc.P(x), orc.P(b4), k, n, orc.P(bias), orc.P(y), orc.P(q), orc.P(s), orc.P(b))
    assert np.array_equal(y, orc.q4k_project(x, b4, k, n, bias))
    b6 = random_q6k_blocks(rng, n * 4).reshape(n, -1)
    L.cpub_q6k_project_parallel(orc.P(x), orc.P(b6), k, n, None, orc.P(y), orc.P(q), orc.P(s), orc.P(b))
    assert np.array_equal(y, orc.q6k_project(x, b6, k, n))
    g = random_q4k_blocks(rng, n * 4).reshape(n, -1)
    yg = np.zeros(n, np.float32)
    yu = np.zeros(n, np.float32)
    L.cpub_q4k_project_gate_up(orc.P(x), orc.P(g), orc.P(b4), k, n, orc.P(yg), orc.P(yu), orc.P(q), orc.P(s),
                               orc.P(b))
    go, uo = orc.q4k_project_gate_up(x, g, b4, k, n)
    assert np.array_equal(yg, go) and np.array_equal(yu, uo)
    wq, ws = orc.q8_quantize_rows(normal(rng, (n, k), 0.05))
    q8 = np.zeros(k, np.int8)
    s8 = np.zeros(k // 32, np.float32)
    L.cpub_q8_project_parallel(orc.P(x), orc.P(wq), orc.P(ws), k, n, orc.P(bias), orc.P(y), orc.P(q8), orc.P(s8))
    assert np.array_equal(y, orc.q8_project(x, wq, ws, k, n, bias))


@pytest.mark.parametrize("workers", [1, 3, 8])
def test_cpu_baseline_batched_paths_are_bit_identical_to_oracle(orc, workers):
    """The batched CPU baseline (OverfitParallel.For over every worker, the caller on the last chunk; the Q4_K
    weight-stationary 64-row tile; Q6_K ProjectBatched; the routed-MoE DecodeBatched) gives the oracle's bits for
    any worker count, for row counts across the tile boundary and output counts not divisible by the chunks."""
    L = orc.lib()
    if not L.cpub_has_avx2():
        pytest.skip("no AVX2 on this CPU")
    L.cpub_set_workers(workers)
    rng = np.random.default_rng(43 + workers)
    k, n = 512, 37
    b4 = random_q4k_blocks(rng, n * k // 256).reshape(n, -1)
    b6 = random_q6k_blocks(rng, n * k // 256).reshape(n, -1)
    bias = normal(rng, n)
    for rows in (1, 5, 64, 131):
        x = normal(rng, (rows, k))
        q = np.zeros(rows * k, np.int8)
        s = np.zeros(rows * k // 256, np.float32)
        b = np.zeros(rows * k // 16, np.int16)
        y = np.full((rows, n), np.nan, np.float32)
        for bb in (None, bias):
            assert L.cpub_q4k_project_batched_ws(orc.P(x), rows, orc.P(b4), k, n, orc.P(bb), orc.P(y), orc.P(q),
                                                 orc.P(s), orc.P(b)) == 0
            ref = orc.q4k_project_batched_ws(x, rows, b4, k, n, bb)
            assert np.array_equal(y.view(np.uint32), ref.view(np.uint32)), ("q4k ws", rows)
            assert L.cpub_q6k_project_batched(orc.P(x), rows, orc.P(b6), k, n, orc.P(bb), orc.P(y), orc.P(q),
                                              orc.P(s), orc.P(b)) == 0
            ref = orc.q6k_project_batched(x, rows, b6, k, n, bb)
            assert np.array_equal(y.view(np.uint32), ref.view(np.uint32)), ("q6k", rows)
    # routed MoE: 5 experts, 9 tokens, top-2 (Q4_K gate/up, Q6_K down)
    import ctypes
    E, dm, dff, rows, top_k = 5, 256, 512, 9, 2
    gate = [orc.quantize_q4k(normal(rng, (dff, dm), 0.05)) for _ in range(E)]
    up = [orc.quantize_q4k(normal(rng, (dff, dm), 0.05)) for _ in range(E)]
    down = [orc.quantize_q6k(normal(rng, (dm, dff), 0.05)) for _ in range(E)]
    x = normal(rng, (rows, dm))
    idx = np.stack([rng.choice(E, top_k, replace=False) for _ in range(rows)]).astype(np.int32)
    w = rng.random((rows, top_k)).astype(np.float32)
    arr = lambda ms: (ctypes.c_void_p * E)(*[m.ctypes.data for m in ms])  # noqa: E731
    y = np.zeros((rows, dm), np.float32)
    assert L.cpub_moe_ffn_batched(E, arr(gate), arr(up), arr(down), 12, 14, orc.P(x), rows, dm, dff, top_k,
                                  orc.P(idx), orc.P(w), orc.P(y)) == 0
    ref = orc.moe_ffn_batched(gate, up, down, 12, 14, x, rows, dm, dff, top_k, idx, w)
    assert np.array_equal(y.view(np.uint32), np.asarray(ref, np.float32).view(np.uint32))
    L.cpub_set_workers(4)
