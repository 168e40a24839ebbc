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


def q8_0_gguf_blocks(scales, quants):
    """GGUF Q8_0 blocks as a file stores them: fp16 scale, then 32 int8 quants."""
    nb = len(scales)
    blocks = np.zeros((nb, 34), np.uint8)
    blocks[:, 0:2] = np.asarray(scales, np.float16).view(np.uint8).reshape(nb, 2)
    blocks[:, 2:] = np.asarray(quants, np.int8).reshape(nb, 32).view(np.uint8)
    return blocks


# GgmlDequantTests.Q8_0_DequantizesSingleBlock_RoundTrip (TL/Loading/GgmlDequantTests.cs:20-46): scale 2.0, quants
# -128, -1, 0, 1, 127, then i - 16; Q8_0_DequantizesMultipleBlocks_DifferentScales (:48-78): scales 0.5, 1, 0.125,
# quant b * 10 + i - 5 for element i of block b.
Q8_0_KATS = [
    ([2.0], np.array([-128, -1, 0, 1, 127] + [i - 16 for i in range(5, 32)], np.int8)),
    ([0.5, 1.0, 0.125], np.array([b * 10 + i - 5 for b in range(3) for i in range(32)], np.int8)),
]


def random_q5_blocks(rng, type_id, n_rows, k):
    """GGUF Q5_0 (type 6: 22-byte blocks of 32) or Q5_K (type 13: 176-byte super-blocks) rows: random bytes with
    sane fp16 scales (d, and dmin for Q5_K), as a [n_rows][bytes per row] uint8 array."""
    bb, blk = (22, 32) if type_id == 6 else (176, 256)
    b = rng.integers(0, 256, size=(n_rows, k // blk, bb), dtype=np.uint8)
    nb = n_rows * (k // blk)
    b[..., 0:2] = np.frombuffer(rng.uniform(0.001, 0.05, nb).astype(np.float16).tobytes(), np.uint8).reshape(
        n_rows, k // blk, 2)
    if type_id == 13:
        b[..., 2:4] = np.frombuffer(rng.uniform(0.001, 0.03, nb).astype(np.float16).tobytes(), np.uint8).reshape(
            n_rows, k // blk, 2)
    return b.reshape(n_rows, -1)
