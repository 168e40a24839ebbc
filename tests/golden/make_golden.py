"""Writes tests/golden/golden_small.npz: small seeded inputs and the oracle's outputs for them.

The reference holds no golden vectors for this path (its quant tests are relations and known answers), so
these fixtures are generated from the pinned oracle. They freeze the oracle's outputs: test_golden.py
checks that the oracle still reproduces them and the GPU tests check the device path against them.
Run: python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
sys.path.insert(0, os.path.dirname(HERE))

import oracle  # noqa: E402
from qdata import normal, random_q4k_blocks, random_q6k_blocks, set_subnormal_scales  # noqa: E402

OUT = os.path.join(HERE, "golden_small.npz")


def make():
    rng = np.random.default_rng(20260519)
    k, n, rows = 512, 24, 3
    x = normal(rng, (rows, k))
    bias = normal(rng, n, 0.1)
    q4 = set_subnormal_scales(random_q4k_blocks(rng, n * 2)).reshape(n, -1)
    q6 = set_subnormal_scales(random_q6k_blocks(rng, n * 2), q6=True).reshape(n, -1)
    w8 = normal(rng, (n, 128), 0.05)
    w8q, w8s = oracle.q8_quantize_rows(w8)
    x8 = normal(rng, (rows, 128))
    wf = normal(rng, (4, 512), 0.02)
    wf[3] = 0.37
    q, d, b = oracle.quantize_q8k(x)
    out = dict(
        k=np.int32(k), n=np.int32(n), rows=np.int32(rows), x=x, bias=bias,
        q8k_q=q, q8k_d=d, q8k_b=b,
        q4k_blocks=q4, q4k_y=oracle.q4k_project(x[0], q4, k, n, bias),
        q4k_y_batched=oracle.q4k_project_batched(x, rows, q4, k, n, bias),
        q6k_blocks=q6, q6k_y=oracle.q6k_project(x[0], q6, k, n),
        q6k_y_batched=oracle.q6k_project_batched(x, rows, q6, k, n, bias),
        q8_wq=w8q, q8_ws=w8s, q8_x=x8, q8_y=oracle.q8_project(x8[0], w8q, w8s, 128, n, bias),
        q8_y_batched=oracle.q8_project_batched(x8, rows, w8q, w8s, 128, n, None),
        enc_w=wf, enc_q4k=oracle.quantize_q4k(wf), enc_q6k=oracle.quantize_q6k(wf),
    )
    np.savez_compressed(OUT, **out)
    return OUT


if __name__ == "__main__":
    print(make())
