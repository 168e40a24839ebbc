"""Seeded synthetic inputs shared by the tests (same bytes go to the oracle and to the GPU)."""
import numpy as np


def half_bits(x):
    return np.array([x], dtype=np.float16).view(np.uint16)[0]


def random_q4k_blocks(rng, n_blocks, d_range=(0.001, 0.051), dmin_range=(0.001, 0.031)):
    """Reference-style synthetic Q4_K blocks: random bytes with sane fp16 d/dmin
    (TL/Runtime/Q4KDotKernelTests.cs:225-247)."""
    b = rng.integers(0, 256, size=(n_blocks, 144), dtype=np.uint8)
    d = rng.uniform(*d_range, size=n_blocks).astype(np.float16).view(np.uint16)
    dm = rng.uniform(*dmin_range, size=n_blocks).astype(np.float16).view(np.uint16)
    b[:, 0] = d & 0xFF
    b[:, 1] = d >> 8
    b[:, 2] = dm & 0xFF
    b[:, 3] = dm >> 8
    return b


def random_q6k_blocks(rng, n_blocks, d_range=(0.0005, 0.01)):
    """Synthetic Q6_K blocks: random quant/scale bytes with a sane fp16 d
    (TL/Runtime/Q6KDotKernelTests.cs:173-194)."""
    b = rng.integers(0, 256, size=(n_blocks, 210), dtype=np.uint8)
    d = rng.uniform(*d_range, size=n_blocks).astype(np.float16).view(np.uint16)
    b[:, 208] = d & 0xFF
    b[:, 209] = d >> 8
    return b


def set_subnormal_scales(blocks, every=7, q6=False):
    """Give every `every`-th block a subnormal fp16 scale (exercises exact fp16 widening)."""
    for i in range(0, blocks.shape[0], every):
        sub = 0x0001 + (i * 37) % 0x3FF  # 0x0001..0x03FF are the fp16 subnormals
        if q6:
            blocks[i, 208] = sub & 0xFF
            blocks[i, 209] = sub >> 8
        else:
            blocks[i, 0] = sub & 0xFF
            blocks[i, 1] = sub >> 8
    return blocks


def normal(rng, shape, sigma=1.0):
    return (rng.standard_normal(shape) * sigma).astype(np.float32)
