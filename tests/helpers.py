"""Seeded inputs and small readers shared by the tests."""
import struct
from pathlib import Path

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


def q4_1_blocks(rng, rows, cols, scale_std=0.02):
    """rows x cols Q4_1 weights as GGUF blocks: d = fp16(|N(0, std)|), a
    block minimum m = fp16(-u d) with u uniform in [6, 10] (so weights lie
    about zero, as a quantizer's minimum puts them), codes uniform in 0..15."""
    n = rows * cols // 32
    out = np.empty((n, 20), dtype=np.uint8)
    d = np.abs(rng.normal(0.0, scale_std, n)).astype(np.float16)
    m = (-d.astype(np.float32) * rng.uniform(6.0, 10.0, n)).astype(np.float16)
    out[:, 0:2] = d.view(np.uint8).reshape(n, 2)
    out[:, 2:4] = m.view(np.uint8).reshape(n, 2)
    out[:, 4:] = rng.integers(0, 256, size=(n, 16), dtype=np.uint8)
    return out.reshape(-1)


def q8_0_blocks(rng, rows, cols, scale_std=0.002):
    """rows x cols Q8_0 weights as GGUF blocks: d = fp16(|N(0, std)|), codes
    uniform signed bytes."""
    n = rows * cols // 32
    out = np.empty((n, 34), dtype=np.uint8)
    d = np.abs(rng.normal(0.0, scale_std, n)).astype(np.float16)
    out[:, 0:2] = d.view(np.uint8).reshape(n, 2)
    out[:, 2:] = rng.integers(0, 256, size=(n, 32), dtype=np.uint8)
    return out.reshape(-1)


def format_blocks(rng, fmt, rows, cols):
    """Seeded GGUF blocks of format fmt (2 Q4_0, 3 Q4_1, 8 Q8_0)."""
    return {2: q4_blocks, 3: q4_1_blocks, 8: q8_0_blocks}[fmt](rng, rows, cols)


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


def read_gguf(path):
    """The tensors of a GGUF v3 file: {name: (dims, type, bytes)}."""
    data = Path(path).read_bytes()
    at = 0

    def take(fmt):
        nonlocal at
        v = struct.unpack_from(fmt, data, at)
        at += struct.calcsize(fmt)
        return v if len(v) > 1 else v[0]

    def string():
        nonlocal at
        n = take("<Q")
        s = data[at:at + n]
        at += n
        return s

    sizes = {0: 1, 1: 1, 2: 2, 3: 2, 4: 4, 5: 4, 6: 4, 7: 1, 10: 8, 11: 8, 12: 8}

    def value(t):
        nonlocal at
        if t == 8:
            return string()
        if t == 9:
            et, n = take("<I"), take("<Q")
            return [value(et) for _ in range(n)]
        v = data[at:at + sizes[t]]
        at += sizes[t]
        return v

    assert data[:4] == b"GGUF"
    at = 4
    version, tensors, kvs = take("<I"), take("<Q"), take("<Q")
    assert version == 3
    meta = {}
    for _ in range(kvs):
        key = string()
        meta[key] = value(take("<I"))
    infos = []
    for _ in range(tensors):
        name = string()
        dims = [take("<q") for _ in range(take("<I"))]
        infos.append((name, dims, take("<I"), take("<Q")))
    align = struct.unpack("<I", meta[b"general.alignment"])[0]
    base = (at + align - 1) // align * align
    out = {}
    for name, dims, ttype, off in infos:
        n = int(np.prod(dims))
        size = n // 32 * 18 if ttype == 2 else n * 4
        out[name] = (dims, ttype, data[base + off:base + off + size])
    return out
