"""Seeded inputs shared by the tests."""
import numpy as np


def q4_blocks(rng, rows, cols, scale_std=0.02):
    """rows x cols Q4_0 weights as GGUF blocks: d = fp16(|N(0, std)|), codes
    uniform in 0..15."""
    n = rows * cols // 32
    out = np.empty((n, 18), dtype=np.uint8)
    d = np.abs(rng.normal(0.0, scale_std, n)).astype(np.float16)
    out[:, 0:2] = d.view(np.uint8).reshape(n, 2)
    out[:, 2:] = rng.integers(0, 256, size=(n, 16), dtype=np.uint8)
    return out.reshape(-1)


def dequant(blocks, rows, cols):
    """Q4_0 blocks to float64 weights, by the format's definition
    (q4_0.h:21-23): weight j = ((qs[j] & 15) - 8) d, weight j+16 =
    ((qs[j] >> 4) - 8) d."""
    b = np.asarray(blocks, dtype=np.uint8).reshape(-1, 18)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float64).reshape(-1, 1)
    qs = b[:, 2:].astype(np.int64)
    lo = (qs & 15) - 8
    hi = (qs >> 4) - 8
    w = np.concatenate([lo, hi], axis=1) * d
    return w.reshape(rows, cols)


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def assert_same_bits(got, want, what=""):
    g, w = bits(got), bits(want)
    assert g.shape == w.shape, (g.shape, w.shape)
    diff = np.nonzero(g.ravel() != w.ravel())[0]
    if diff.size:
        i = diff[0]
        raise AssertionError(
            f"{what}: {diff.size} of {g.size} values differ; first at {i}: "
            f"got {np.float32(got.ravel()[i])!r} want {np.float32(want.ravel()[i])!r}")
