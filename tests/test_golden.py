"""The committed golden fixtures (tests/golden/golden_small.npz) against the oracle (CPU) and the device."""
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden_small.npz")


@pytest.fixture(scope="module")
def g():
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def test_oracle_reproduces_golden(orc, g):
    k, n, rows = int(g["k"]), int(g["n"]), int(g["rows"])
    q, d, b = orc.quantize_q8k(g["x"])
    assert np.array_equal(q, g["q8k_q"]) and np.array_equal(d, g["q8k_d"]) and np.array_equal(b, g["q8k_b"])
    assert np.array_equal(orc.q4k_project(g["x"][0], g["q4k_blocks"], k, n, g["bias"]), g["q4k_y"])
    assert np.array_equal(orc.q4k_project_batched(g["x"], rows, g["q4k_blocks"], k, n, g["bias"]), g["q4k_y_batched"])
    assert np.array_equal(orc.q6k_project(g["x"][0], g["q6k_blocks"], k, n), g["q6k_y"])
    assert np.array_equal(orc.q6k_project_batched(g["x"], rows, g["q6k_blocks"], k, n, g["bias"]), g["q6k_y_batched"])
    assert np.array_equal(orc.q8_project(g["q8_x"][0], g["q8_wq"], g["q8_ws"], 128, n, g["bias"]), g["q8_y"])
    assert np.array_equal(orc.q8_project_batched(g["q8_x"], rows, g["q8_wq"], g["q8_ws"], 128, n), g["q8_y_batched"])
    assert np.array_equal(orc.quantize_q4k(g["enc_w"]), g["enc_q4k"])
    assert np.array_equal(orc.quantize_q6k(g["enc_w"]), g["enc_q6k"])


@pytest.mark.gpu
def test_device_reproduces_golden(g):
    import torch

    import overfit_amd as ov

    k, n, rows = int(g["k"]), int(g["n"]), int(g["rows"])
    dev = torch.device("cuda:0")
    x = torch.from_numpy(g["x"]).to(dev)
    q = torch.empty(rows * k, dtype=torch.int8, device=dev)
    s = torch.empty(rows * k // 256, dtype=torch.float32, device=dev)
    b = torch.empty(rows * k // 16, dtype=torch.int16, device=dev)
    ov.default_context().quantize_q8k_dev(x, rows, k, q, s, b)
    torch.cuda.synchronize()
    assert np.array_equal(q.cpu().numpy(), g["q8k_q"].reshape(-1))
    assert np.array_equal(s.cpu().numpy(), g["q8k_d"].reshape(-1))
    assert np.array_equal(b.cpu().numpy(), g["q8k_b"].reshape(-1))
    w4 = ov.Q4KWeight(g["q4k_blocks"], k, n)
    w6 = ov.Q6KWeight(g["q6k_blocks"], k, n)
    w8 = ov.Q8Weight(g["q8_wq"], g["q8_ws"], 128, n)
    assert np.array_equal(ov.project(w4, g["x"][0].copy(), g["bias"]), g["q4k_y"])
    assert np.array_equal(ov.project(w4, g["x"], g["bias"], rows=rows).reshape(rows, n), g["q4k_y_batched"])
    assert np.array_equal(ov.project(w6, g["x"][0].copy()), g["q6k_y"])
    assert np.array_equal(ov.project(w6, g["x"], g["bias"], rows=rows).reshape(rows, n), g["q6k_y_batched"])
    assert np.array_equal(ov.project(w8, g["q8_x"][0].copy(), g["bias"]), g["q8_y"])
    assert np.array_equal(ov.project(w8, g["q8_x"], rows=rows).reshape(rows, n), g["q8_y_batched"])
    wf = torch.from_numpy(g["enc_w"]).to(dev)
    assert np.array_equal(ov.quantize_weight(wf, ov.TYPE_Q4_K).cpu().numpy(), g["enc_q4k"].reshape(-1))
    assert np.array_equal(ov.quantize_weight(wf, ov.TYPE_Q6_K).cpu().numpy(), g["enc_q6k"].reshape(-1))
