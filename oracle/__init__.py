"""Python view of the oracle (ovfq_oracle.c) and the CPU baseline (cpu_baseline.c).

TEST INFRASTRUCTURE ONLY: the checker the GPU path is compared against. Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg import this package; the product package
(overfit_amd) never does.
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libovfq_oracle.so")

_lib = None

c_i8p = ctypes.POINTER(ctypes.c_int8)
c_u8p = ctypes.POINTER(ctypes.c_uint8)
c_i16p = ctypes.POINTER(ctypes.c_int16)
c_f32p = ctypes.POINTER(ctypes.c_float)
c_i32p = ctypes.POINTER(ctypes.c_int32)
c_int = ctypes.c_int

_SIGS = {
    "orc_half_to_float": (ctypes.c_float, [ctypes.c_uint16]),
    "orc_float_to_half": (ctypes.c_uint16, [ctypes.c_float]),
    "orc_unpack_q4k_scales_mins": (None, [c_u8p, c_u8p, c_u8p]),
    "orc_pack_q4k_scales_mins": (None, [c_u8p, c_u8p, c_u8p]),
    "orc_decode_q4k_block": (None, [c_u8p, c_f32p]),
    "orc_decode_q5_0_block": (None, [c_u8p, c_f32p]),
    "orc_decode_q5k_block": (None, [c_u8p, c_f32p]),
    "orc_q5_requantize_q8_0": (c_int, [c_int, c_u8p, c_int, c_int, c_i8p, c_f32p]),
    "orc_decode_q6k_block": (None, [c_u8p, c_f32p]),
    "orc_q4k_decode_row": (c_int, [c_u8p, c_int, c_int, c_int, c_f32p]),
    "orc_q6k_decode_row": (c_int, [c_u8p, c_int, c_int, c_int, c_f32p]),
    "orc_q8_decode_row": (c_int, [c_i8p, c_f32p, c_int, c_int, c_int, c_f32p]),
    "orc_quantize_q8k": (c_int, [c_f32p, c_int, c_i8p, c_f32p, c_i16p]),
    "orc_quantize_q8_0": (c_int, [c_f32p, c_int, c_i8p, c_f32p]),
    "orc_q4k_main_dot": (ctypes.c_int32, [c_u8p, c_i8p, c_u8p]),
    "orc_q4k_min_acc": (ctypes.c_int32, [c_u8p, c_i16p]),
    "orc_q4k_dot": (ctypes.c_float, [c_u8p, c_i8p, ctypes.c_float, c_i16p]),
    "orc_q6k_unsigned_dot": (ctypes.c_int32, [c_u8p, c_i8p]),
    "orc_q6k_bsum_term": (ctypes.c_int32, [c_u8p, c_i16p]),
    "orc_q6k_dot": (ctypes.c_float, [c_u8p, c_i8p, ctypes.c_float, c_i16p]),
    "orc_q8_dot": (ctypes.c_float, [c_i8p, c_f32p, c_i8p, c_f32p, c_int]),
    "orc_q8_block_int_dot": (ctypes.c_int32, [c_i8p, c_i8p]),
    "orc_q4k_project_prequantized": (c_int, [c_u8p, c_int, c_int, c_f32p, c_f32p, c_i8p, c_f32p, c_i16p]),
    "orc_q4k_project": (c_int, [c_f32p, c_u8p, c_int, c_int, c_f32p, c_f32p, c_i8p, c_f32p, c_i16p]),
    "orc_q4k_project_gate_up": (c_int, [c_f32p, c_u8p, c_u8p, c_int, c_int, c_f32p, c_f32p, c_i8p, c_f32p,
                                        c_i16p]),
    "orc_q4k_project_batched": (c_int, [c_f32p, c_int, c_u8p, c_int, c_int, c_f32p, c_f32p, c_i8p, c_f32p,
                                        c_i16p]),
    "orc_q4k_project_batched_ws": (c_int, [c_f32p, c_int, c_u8p, c_int, c_int, c_f32p, c_f32p, c_i8p,
                                           c_f32p, c_i16p]),
    "orc_q4k_project_batched_prequantized": (c_int, [c_int, c_u8p, c_int, c_int, c_f32p, c_f32p, c_i8p,
                                                     c_f32p, c_i16p]),
    "orc_q6k_project_prequantized": (c_int, [c_u8p, c_int, c_int, c_f32p, c_f32p, c_i8p, c_f32p, c_i16p]),
    "orc_q6k_project": (c_int, [c_f32p, c_u8p, c_int, c_int, c_f32p, c_f32p, c_i8p, c_f32p, c_i16p]),
    "orc_q6k_project_batched": (c_int, [c_f32p, c_int, c_u8p, c_int, c_int, c_f32p, c_f32p, c_i8p, c_f32p,
                                        c_i16p]),
    "orc_q6k_project_batched_prequantized": (c_int, [c_int, c_u8p, c_int, c_int, c_f32p, c_f32p, c_i8p,
                                                     c_f32p, c_i16p]),
    "orc_q8_project": (c_int, [c_f32p, c_i8p, c_f32p, c_int, c_int, c_f32p, c_f32p, c_i8p, c_f32p]),
    "orc_q8_project_batched": (c_int, [c_f32p, c_int, c_i8p, c_f32p, c_int, c_int, c_f32p, c_f32p, c_i8p,
                                       c_f32p]),
    "orc_q8_project_batched_prequantized": (c_int, [c_int, c_i8p, c_f32p, c_int, c_int, c_f32p, c_f32p, c_i8p,
                                                    c_f32p]),
    "orc_q8_project_heads": (c_int, [c_f32p, c_int, c_int, c_int, c_int, ctypes.c_void_p, ctypes.c_void_p, c_f32p,
                                     c_f32p]),
    "orc_encode_q4k_block": (None, [c_f32p, c_u8p]),
    "orc_quantize_q4k": (c_int, [c_f32p, c_int, c_int, c_u8p]),
    "orc_encode_q6k_block": (None, [c_f32p, c_u8p]),
    "orc_quantize_q6k": (c_int, [c_f32p, c_int, c_int, c_u8p]),
    "orc_q8_quantize_rows": (c_int, [c_f32p, c_int, c_int, c_i8p, c_f32p]),
    "orc_moe_select_topk": (c_int, [c_f32p, c_int, c_int, c_i32p, c_f32p, c_int]),
    "orc_q8_0_deinterleave": (c_int, [c_u8p, ctypes.c_long, c_i8p, c_f32p]),
    "orc_swiglu_batched": (c_int, [c_f32p, c_int, c_u8p, c_u8p, c_u8p, c_int, c_int, c_int, c_int, c_f32p]),
    "orc_gated_ffn_batched": (c_int, [c_f32p, c_int, c_u8p, c_u8p, c_u8p, c_int, c_int, c_int, c_int, c_int, c_f32p]),
    "orc_moe_ffn_batched": (c_int, [c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, c_int, c_int, c_f32p,
                                    c_int, c_int, c_int, c_int, c_i32p, c_f32p, c_f32p]),
    # CPU baseline (cpu_baseline.c)
    "cpub_set_workers": (c_int, [c_int]),
    "cpub_has_avx2": (c_int, []),
    "cpub_quantize_q8k": (c_int, [c_f32p, c_int, c_i8p, c_f32p, c_i16p]),
    "cpub_q4k_project_parallel": (c_int, [c_f32p, c_u8p, c_int, c_int, c_f32p, c_f32p, c_i8p, c_f32p, c_i16p]),
    "cpub_q4k_project_prequantized_parallel": (c_int, [c_u8p, c_int, c_int, c_f32p, c_f32p, c_i8p, c_f32p,
                                                       c_i16p]),
    "cpub_q4k_project_gate_up": (c_int, [c_f32p, c_u8p, c_u8p, c_int, c_int, c_f32p, c_f32p, c_i8p, c_f32p,
                                         c_i16p]),
    "cpub_q6k_project_parallel": (c_int, [c_f32p, c_u8p, c_int, c_int, c_f32p, c_f32p, c_i8p, c_f32p, c_i16p]),
    "cpub_q8_project_parallel": (c_int, [c_f32p, c_i8p, c_f32p, c_int, c_int, c_f32p, c_f32p, c_i8p, c_f32p]),
    "cpub_set_decode_cap": (c_int, [c_int]),
    "cpub_q4k_project_batched_ws": (c_int, [c_f32p, c_int, c_u8p, c_int, c_int, c_f32p, c_f32p, c_i8p, c_f32p,
                                            c_i16p]),
    "cpub_q6k_project_batched": (c_int, [c_f32p, c_int, c_u8p, c_int, c_int, c_f32p, c_f32p, c_i8p, c_f32p,
                                         c_i16p]),
    "cpub_moe_ffn_batched": (c_int, [c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, c_int, c_int, c_f32p,
                                     c_int, c_int, c_int, c_int, c_i32p, c_f32p, c_f32p]),
    "cpub_build_info": (ctypes.c_char_p, []),
}

_NP_CTYPE = {
    np.dtype(np.int8): c_i8p,
    np.dtype(np.uint8): c_u8p,
    np.dtype(np.int16): c_i16p,
    np.dtype(np.float32): c_f32p,
    np.dtype(np.int32): c_i32p,
}


def lib():
    """Load (building first if absent) the oracle shared library."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            from . import build as _build

            _build.build()
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def P(a):
    """ctypes pointer to a C-contiguous numpy array (None -> NULL)."""
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(_NP_CTYPE[a.dtype])


def _check(rc):
    if rc < 0:
        raise ValueError(f"oracle returned status {rc}")
    return rc


# ------------------------------------------------------------------ numpy conveniences

def half_to_float(bits: int) -> float:
    return lib().orc_half_to_float(bits)


def float_to_half(x: float) -> int:
    return lib().orc_float_to_half(x)


def unpack_q4k_scales_mins(packed12):
    p = np.ascontiguousarray(packed12, dtype=np.uint8)
    sc = np.zeros(8, np.uint8)
    m = np.zeros(8, np.uint8)
    lib().orc_unpack_q4k_scales_mins(P(p), P(sc), P(m))
    return sc, m


def pack_q4k_scales_mins(sc, m):
    sc = np.ascontiguousarray(sc, dtype=np.uint8)
    m = np.ascontiguousarray(m, dtype=np.uint8)
    out = np.zeros(12, np.uint8)
    lib().orc_pack_q4k_scales_mins(P(sc), P(m), P(out))
    return out


def decode_q4k_block(block):
    b = np.ascontiguousarray(block, dtype=np.uint8)
    dst = np.zeros(256, np.float32)
    lib().orc_decode_q4k_block(P(b), P(dst))
    return dst


def decode_q5_0_block(block):
    b = np.ascontiguousarray(block, dtype=np.uint8)
    dst = np.zeros(32, np.float32)
    lib().orc_decode_q5_0_block(P(b), P(dst))
    return dst


def decode_q5k_block(block):
    b = np.ascontiguousarray(block, dtype=np.uint8)
    dst = np.zeros(256, np.float32)
    lib().orc_decode_q5k_block(P(b), P(dst))
    return dst


def q5_requantize_q8_0(type_id, data, rows, k):
    """Q5_0 / Q5_K rows -> the loader's resident Q8_0 planes (decode to F32, Q8Weight.QuantizeRows)."""
    d = np.ascontiguousarray(data, np.uint8).ravel()
    q = np.zeros((rows, k), np.int8)
    s = np.zeros((rows, k // 32), np.float32)
    _check(lib().orc_q5_requantize_q8_0(type_id, P(d), rows, k, P(q), P(s)))
    return q, s


def decode_q6k_block(block):
    b = np.ascontiguousarray(block, dtype=np.uint8)
    dst = np.zeros(256, np.float32)
    lib().orc_decode_q6k_block(P(b), P(dst))
    return dst


def quantize_q8k(x):
    """Q8_K of a [rows, K] (or [K]) fp32 array -> (q int8 [rows,K], d f32 [rows,K/256], bsums i16 [rows,K/16])."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    x2 = x.reshape(-1, x.shape[-1])
    rows, k = x2.shape
    q = np.zeros((rows, k), np.int8)
    d = np.zeros((rows, k // 256), np.float32)
    b = np.zeros((rows, k // 16), np.int16)
    for r in range(rows):
        _check(lib().orc_quantize_q8k(P(x2[r]), k, P(q[r]), P(d[r]), P(b[r])))
    return q, d, b


def quantize_q8_0(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    x2 = x.reshape(-1, x.shape[-1])
    rows, k = x2.shape
    q = np.zeros((rows, k), np.int8)
    s = np.zeros((rows, k // 32), np.float32)
    for r in range(rows):
        _check(lib().orc_quantize_q8_0(P(x2[r]), k, P(q[r]), P(s[r])))
    return q, s


def quantize_q4k(w):
    """GgmlQuant.QuantizeQ4_K of an output-major [out, in] fp32 matrix -> uint8 bytes [out, in/256*144]."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    out, k = w.shape
    dst = np.zeros((out, k // 256 * 144), np.uint8)
    _check(lib().orc_quantize_q4k(P(w), k, out, P(dst)))
    return dst


def quantize_q6k(w):
    w = np.ascontiguousarray(w, dtype=np.float32)
    out, k = w.shape
    dst = np.zeros((out, k // 256 * 210), np.uint8)
    _check(lib().orc_quantize_q6k(P(w), k, out, P(dst)))
    return dst


def q8_quantize_rows(w):
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, k = w.shape
    q = np.zeros((rows, k), np.int8)
    s = np.zeros((rows, k // 32), np.float32)
    _check(lib().orc_q8_quantize_rows(P(w), rows, k, P(q), P(s)))
    return q, s


def _proj_q8k(fn_pre, blocks, k, n, q, d, b, bias):
    rows = q.shape[0]
    y = np.zeros((rows, n), np.float32)
    bias = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    if rows == 1:
        _check(fn_pre(P(blocks), k, n, P(bias), P(y[0]), P(q[0]), P(d[0]), P(b[0])))
    else:
        raise AssertionError("use the batched wrappers for rows > 1")
    return y


def q4k_project(x, blocks, k, n, bias=None):
    """Q4KDotKernel.Project for a single row x[K] -> y[N] (oracle)."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    bias = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    q = np.zeros(k, np.int8)
    d = np.zeros(k // 256, np.float32)
    b = np.zeros(k // 16, np.int16)
    y = np.zeros(n, np.float32)
    _check(lib().orc_q4k_project(P(x), P(blocks), k, n, P(bias), P(y), P(q), P(d), P(b)))
    return y


def q6k_project(x, blocks, k, n, bias=None):
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    bias = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    q = np.zeros(k, np.int8)
    d = np.zeros(k // 256, np.float32)
    b = np.zeros(k // 16, np.int16)
    y = np.zeros(n, np.float32)
    _check(lib().orc_q6k_project(P(x), P(blocks), k, n, P(bias), P(y), P(q), P(d), P(b)))
    return y


def q8_project(x, wq, ws, k, n, bias=None):
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    wq = np.ascontiguousarray(wq, dtype=np.int8)
    ws = np.ascontiguousarray(ws, dtype=np.float32)
    bias = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    q = np.zeros(k, np.int8)
    s = np.zeros(k // 32, np.float32)
    y = np.zeros(n, np.float32)
    _check(lib().orc_q8_project(P(x), P(wq), P(ws), k, n, P(bias), P(y), P(q), P(s)))
    return y


def q4k_project_gate_up(x, gate, up, k, n):
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    gate = np.ascontiguousarray(gate, dtype=np.uint8)
    up = np.ascontiguousarray(up, dtype=np.uint8)
    q = np.zeros(k, np.int8)
    d = np.zeros(k // 256, np.float32)
    b = np.zeros(k // 16, np.int16)
    g = np.zeros(n, np.float32)
    u = np.zeros(n, np.float32)
    _check(lib().orc_q4k_project_gate_up(P(x), P(gate), P(up), k, n, P(g), P(u), P(q), P(d), P(b)))
    return g, u


def _batched(fn, x, rows, blocks, k, n, bias, qdt_cols):
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(rows, k)
    bias = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    q = np.zeros(rows * k, np.int8)
    d = np.zeros(rows * (k // 256), np.float32)
    b = np.zeros(rows * (k // 16), np.int16)
    y = np.zeros((rows, n), np.float32)
    _check(fn(P(x), rows, P(blocks), k, n, P(bias), P(y), P(q), P(d), P(b)))
    return y


def q4k_project_batched(x, rows, blocks, k, n, bias=None):
    return _batched(lib().orc_q4k_project_batched, x, rows, np.ascontiguousarray(blocks, np.uint8), k, n, bias, 0)


def q4k_project_batched_ws(x, rows, blocks, k, n, bias=None):
    return _batched(lib().orc_q4k_project_batched_ws, x, rows, np.ascontiguousarray(blocks, np.uint8), k, n,
                    bias, 0)


def q6k_project_batched(x, rows, blocks, k, n, bias=None):
    return _batched(lib().orc_q6k_project_batched, x, rows, np.ascontiguousarray(blocks, np.uint8), k, n, bias, 0)


def q8_project_batched(x, rows, wq, ws, k, n, bias=None):
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(rows, k)
    bias = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    wq = np.ascontiguousarray(wq, dtype=np.int8)
    ws = np.ascontiguousarray(ws, dtype=np.float32)
    q = np.zeros(rows * k, np.int8)
    s = np.zeros(rows * (k // 32), np.float32)
    y = np.zeros((rows, n), np.float32)
    _check(lib().orc_q8_project_batched(P(x), rows, P(wq), P(ws), k, n, P(bias), P(y), P(q), P(s)))
    return y


def q8_project_heads(x, rows, wqs, wss, head_dim, d_model, bias=None):
    """Per-head Q8_0 attention output projection: y[rows][d_model] = (bias or 0) + sum over heads, ascending, of
    Q8DotKernel.Project(x[n][h*head_dim : (h+1)*head_dim], Wo_h) (RT/CachedMultiHeadAttention.cs:185-194, :292-297).
    wqs[h] int8 [d_model][head_dim], wss[h] f32 [d_model][head_dim/32]."""
    H = len(wqs)
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(rows, H * head_dim)
    wqs = [np.ascontiguousarray(w, dtype=np.int8) for w in wqs]
    wss = [np.ascontiguousarray(w, dtype=np.float32) for w in wss]
    QP = (ctypes.c_void_p * H)(*[w.ctypes.data for w in wqs])
    SP = (ctypes.c_void_p * H)(*[w.ctypes.data for w in wss])
    bias = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    y = np.zeros((rows, d_model), np.float32)
    _check(lib().orc_q8_project_heads(P(x), rows, H, head_dim, d_model, QP, SP, P(bias), P(y)))
    return y


def q4k_decode_row(blocks, k, n, row):
    dst = np.zeros(k, np.float32)
    _check(lib().orc_q4k_decode_row(P(np.ascontiguousarray(blocks, np.uint8)), k, n, row, P(dst)))
    return dst


def q6k_decode_row(blocks, k, n, row):
    dst = np.zeros(k, np.float32)
    _check(lib().orc_q6k_decode_row(P(np.ascontiguousarray(blocks, np.uint8)), k, n, row, P(dst)))
    return dst


def q8_0_deinterleave(gguf):
    """GgufReader.LoadTensorQ8_0Raw (oracle): 34-byte blocks -> (int8 quants, f32 scales)."""
    g = np.ascontiguousarray(gguf, np.uint8).ravel()
    nb = g.size // 34
    q = np.zeros(nb * 32, np.int8)
    s = np.zeros(nb, np.float32)
    _check(lib().orc_q8_0_deinterleave(P(g), nb, P(q), P(s)))
    return q, s


def swiglu_batched(x, rows, gate, up, down, gate_type, down_type, d_model, d_ff):
    """CachedFeedForwardBlock.DecodeSwiGluBatchedDispatched (oracle): y[rows][d_model]."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(rows, d_model)
    y = np.zeros((rows, d_model), np.float32)
    g, u, d = (np.ascontiguousarray(a, np.uint8) for a in (gate, up, down))
    _check(lib().orc_swiglu_batched(P(x), rows, P(g), P(u), P(d), gate_type, down_type, d_model, d_ff, P(y)))
    return y


def gated_ffn_batched(x, rows, gate, up, down, gate_type, down_type, d_model, d_ff, activation):
    """The batched gated FFN with ApplyGate's activation (3 SwiGLU, 4 GeGLU: FeedForwardActivation's values)
    (oracle): y[rows][d_model]."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(rows, d_model)
    y = np.zeros((rows, d_model), np.float32)
    g, u, d = (np.ascontiguousarray(a, np.uint8) for a in (gate, up, down))
    _check(lib().orc_gated_ffn_batched(P(x), rows, P(g), P(u), P(d), gate_type, down_type, d_model, d_ff, activation,
                                       P(y)))
    return y


def moe_ffn_batched(gates, ups, downs, gate_type, down_type, x, rows, d_model, d_ff, top_k, idx, w):
    """MoeFeedForwardBlock.DecodeBatched after routing (oracle): idx/w [rows][top_k] -> y[rows][d_model]."""
    E = len(gates)
    keep = [np.ascontiguousarray(a, np.uint8) for a in list(gates) + list(ups) + list(downs)]
    ptrs = [ctypes.c_void_p(a.ctypes.data) for a in keep]
    arr = lambda ps: (ctypes.c_void_p * E)(*[p.value for p in ps])
    G, U, D = arr(ptrs[:E]), arr(ptrs[E:2 * E]), arr(ptrs[2 * E:])
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(rows, d_model)
    idx = np.ascontiguousarray(idx, dtype=np.int32).reshape(rows, top_k)
    w = np.ascontiguousarray(w, dtype=np.float32).reshape(rows, top_k)
    y = np.zeros((rows, d_model), np.float32)
    _check(lib().orc_moe_ffn_batched(E, G, U, D, gate_type, down_type, P(x), rows, d_model, d_ff, top_k, P(idx),
                                     P(w), P(y)))
    return y


def moe_select_topk(logits, top_k, normalize=True):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    k = min(top_k, logits.size)
    idx = np.zeros(max(k, 1), np.int32)
    w = np.zeros(max(k, 1), np.float32)
    rc = _check(lib().orc_moe_select_topk(P(logits), logits.size, top_k, P(idx), P(w), int(normalize)))
    return idx[:rc], w[:rc]
