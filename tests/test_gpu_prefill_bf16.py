"""The fast prefill mode (FRZ_PREFILL_BF16): products on the bf16 matrix
cores over split operands, checked against f64 within their stated bound,
and a model's prompt-end logits against the oracle's within 1e-3 relative
(the north star's tolerance for logits, which fp32-order parity does not
need).

The bound of one product y = sum_k w_k x_k: each operand is split into a
pair of bf16 (w exactly for Q4_0, x to 2^-17), the dropped lo x lo term is
below 2^-16 |w x|, and the fp32 accumulation adds at most K 2^-24 sum |w x|,
so |y - y_exact| <= (2^-15 + K 2^-24) sum_k |w_k x_k|.
"""
import numpy as np
import pytest

import _oracle as orc
import frizzle_amd as fz
from helpers import dequant, format_blocks, q4_blocks
from test_gpu_bench_regimes import wandering_pair
from test_gpu_model import MIXED, _mixed_tensors, _set_all, oracle_run, small_config

pytestmark = pytest.mark.gpu


def _dev_blocks(device, fmt, blocks):
    codes, scales = fz.block_split(fmt, blocks)
    return device.array(codes), device.array(scales)


def _f64_rows(fmt, blocks, rows, cols):
    """The matrix in f64 by each format's definition: Q4_0 (q - 8) d and
    Q8_0 q d exactly; Q4_1 q d + m rounded once to f32, as the reference
    unpacks it (q4_1.wgsl:12-25; q d + m is exact in f64)."""
    if fmt == fz.Q4_0:
        return dequant(blocks, rows, cols).astype(np.float64)
    if fmt == fz.Q8_0:
        b = np.asarray(blocks, np.uint8).reshape(-1, 34)
        d = b[:, 0:2].copy().view(np.float16).astype(np.float64).reshape(-1, 1)
        return (b[:, 2:].view(np.int8).astype(np.float64) * d).reshape(rows, cols)
    b = np.asarray(blocks, np.uint8).reshape(-1, 20)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float64).reshape(-1, 1)
    m = b[:, 2:4].copy().view(np.float16).astype(np.float64).reshape(-1, 1)
    qs = b[:, 4:].astype(np.int64)
    q = np.concatenate([qs & 15, qs >> 4], axis=1)
    return (q * d + m).astype(np.float32).astype(np.float64).reshape(rows, cols)


def _bound(w64, x64):
    k = w64.shape[1]
    return (2.0 ** -15 + k * 2.0 ** -24) * (np.abs(x64) @ np.abs(w64).T)


@pytest.mark.parametrize("rows,cols,tokens,splits,fmt", [
    (1536, 1152, 512, 1, fz.Q4_0),   # Q/K/V
    (1152, 1024, 512, 8, fz.Q4_0),   # O, K split 8
    (1152, 6912, 512, 8, fz.Q4_0),   # down, K split 8
    (1152, 6912, 300, 0, fz.Q4_1),   # a Q4_1 down, ragged tokens, the model's split
    (1152, 6912, 77, 3, fz.Q8_0),    # a Q8_0 down, an uneven split
    (200, 64, 5, 1, fz.Q4_0),        # a partial row tile, few tokens
])
def test_gemm_bf16_within_bound(device, rows, cols, tokens, splits, fmt):
    rng = np.random.default_rng(rows + cols + tokens + splits + fmt)
    blocks = format_blocks(rng, fmt, rows, cols)
    x = rng.normal(0, 1, (tokens, cols)).astype(np.float32)
    codes, scales = _dev_blocks(device, fmt, blocks)
    dx = device.array(x)
    dy = device.empty((tokens, rows), np.float32)
    fz._lib.check(fz.load().frz_op_gemm_bf16(device.handle, fmt, codes.ptr, scales.ptr, rows, cols,
                                             dx.ptr, cols, dy.ptr, rows, tokens, splits))
    w64 = _f64_rows(fmt, blocks, rows, cols)
    want = x.astype(np.float64) @ w64.T
    err = np.abs(dy.numpy().astype(np.float64) - want)
    bound = _bound(w64, x.astype(np.float64))
    worst = float(np.max(err / bound))
    assert worst <= 1.0, worst
    # and typically far inside it: the median error is below 2^-16 of the
    # sum of magnitudes
    assert float(np.median(err / (np.abs(x.astype(np.float64)) @ np.abs(w64).T))) < 2.0 ** -16


def test_gated_bf16_within_bound_with_pins(device):
    rows, cols, tokens, position = 6912, 1152, 200, 40
    rng = np.random.default_rng(7)
    g, u = q4_blocks(rng, rows, cols), q4_blocks(rng, rows, cols)
    x = rng.normal(0, 1, (tokens, cols)).astype(np.float32)
    gc, gs = _dev_blocks(device, fz.Q4_0, g)
    uc, us = _dev_blocks(device, fz.Q4_0, u)
    # layer 1's pins: a set over every position, a scale from position 100,
    # a zero over positions 50..60
    edits = [fz.Edit(1, 11, fz.EditKind.SET, -7.5), fz.Edit(1, 4000, fz.EditKind.SCALE, 3.0, 100),
             fz.Edit(1, 6911, fz.EditKind.ZERO, 0.0, 50, 61)]
    table = fz.edit_table(edits, 2, 0)
    dt = device.array(table)
    dx = device.array(x)
    da = device.empty((tokens, rows), np.float32)
    fz._lib.check(fz.load().frz_op_gated_bf16(device.handle, gc.ptr, gs.ptr, uc.ptr, us.ptr, rows,
                                              cols, dx.ptr, da.ptr, tokens, position, dt.ptr, 1))
    got = da.numpy().astype(np.float64)
    x64 = x.astype(np.float64)
    wg, wu = dequant(g, rows, cols).astype(np.float64), dequant(u, rows, cols).astype(np.float64)
    gv, uv = x64 @ wg.T, x64 @ wu.T
    eg, eu = _bound(wg, x64), _bound(wu, x64)
    z = np.sqrt(2 / np.pi) * (gv + 0.044715 * gv ** 3)
    gelu = 0.5 * gv * (1 + np.tanh(z))
    want = gelu * uv
    # gelu's slope is below 1.13; its own fp32 steps (the reference's exp
    # form) within 2^-20 of it
    tol = 1.13 * eg * np.abs(uv) + (np.abs(gelu) + 1.13 * eg) * eu + 2.0 ** -19 * np.abs(want) + 1e-30
    pos = position + np.arange(tokens)
    want[:, 11] = -7.5
    tol[:, 11] = 0.0
    late = pos >= 100
    want[late, 4000] *= 3.0
    tol[late, 4000] *= 3.0
    mid = (pos >= 50) & (pos < 61)
    want[mid, 6911] = 0.0
    tol[mid, 6911] = 0.0
    assert float(np.max(np.abs(got - want) / np.maximum(tol, 1e-30))) <= 1.0


def test_gated_bf16_partial_tile(device):
    # 80 neurons: one whole 64-neuron tile and a tile of 16 whose rows past
    # the end are read clamped and not stored; 40 tokens (a partial
    # 32-token block); no pins.
    rows, cols, tokens = 80, 128, 40
    rng = np.random.default_rng(8)
    g, u = q4_blocks(rng, rows, cols), q4_blocks(rng, rows, cols)
    x = rng.normal(0, 1, (tokens, cols)).astype(np.float32)
    gc, gs = _dev_blocks(device, fz.Q4_0, g)
    uc, us = _dev_blocks(device, fz.Q4_0, u)
    dx = device.array(x)
    da = device.empty((tokens, rows), np.float32)
    fz._lib.check(fz.load().frz_op_gated_bf16(device.handle, gc.ptr, gs.ptr, uc.ptr, us.ptr, rows,
                                              cols, dx.ptr, da.ptr, tokens, 0, None, 0))
    x64 = x.astype(np.float64)
    wg, wu = dequant(g, rows, cols).astype(np.float64), dequant(u, rows, cols).astype(np.float64)
    gv, uv = x64 @ wg.T, x64 @ wu.T
    eg, eu = _bound(wg, x64), _bound(wu, x64)
    z = np.sqrt(2 / np.pi) * (gv + 0.044715 * gv ** 3)
    gelu = 0.5 * gv * (1 + np.tanh(z))
    want = gelu * uv
    tol = 1.13 * eg * np.abs(uv) + (np.abs(gelu) + 1.13 * eg) * eu + 2.0 ** -19 * np.abs(want) + 1e-30
    assert float(np.max(np.abs(da.numpy().astype(np.float64) - want) / tol)) <= 1.0


def _rel_err(got, want):
    return float(np.max(np.abs(got.astype(np.float64) - want)) / np.max(np.abs(want)))


def test_fast_prefill_small_model_logits(device):
    # Three layers (the third global) at the 512-key window: a 1,100-token
    # prompt in steps of 512, 512 and 76, with a pin. The fast mode's
    # prompt-end logits are within 1e-3 of the oracle's (max-norm relative);
    # the exact mode, switched back, is the oracle's bit for bit.
    cfg = fz.gemma3_1b_config(layers=3, vocab=4096, window=512, pattern=3, context=2048,
                              local_slots=1024)
    model, oracle = wandering_pair(device, cfg, seed=101)
    prompt = np.random.default_rng(102).integers(0, cfg.vocab, 1100).astype(np.uint32)
    table = fz.edit_table([fz.Edit(1, 300, fz.EditKind.SET, 9.0)], cfg.layers, 0)
    model.set_edits(table)
    oracle.set_edits(table)
    want = oracle.prompt(prompt)
    model.set_prefill(fz.PREFILL_BF16)
    for p0 in range(0, len(prompt), 512):
        model.step(p0, prompt[p0:p0 + 512], logits=p0 + 512 >= len(prompt))
    err = _rel_err(model.logits(), want)
    print(f"fast prefill, 3 layers, 1,100 tokens: max |logit error| / max |logit| = {err:.2e}")
    assert err < 1e-3
    model.set_prefill(fz.PREFILL_EXACT)
    for p0 in range(0, len(prompt), 512):
        model.step(p0, prompt[p0:p0 + 512], logits=p0 + 512 >= len(prompt))
    assert np.array_equal(model.logits().view(np.uint32), want.view(np.uint32))
    model.close()
    oracle.close()


def test_fast_prefill_full_size_2048(device):
    # The prefill workload: 2,048 seeded ids through all 26 layers of the
    # full Gemma-3-1B shape in four steps of 512, logits at the last
    # position, within 1e-3 relative of the oracle's.
    cfg = fz.gemma3_1b_config(context=4096)
    model, oracle = wandering_pair(device, cfg, seed=103)
    prompt = np.random.default_rng(104).integers(0, cfg.vocab, 2048).astype(np.uint32)
    zeros = np.zeros(2 * cfg.layers, dtype=np.uint32)
    model.set_edits(zeros)
    oracle.set_edits(zeros)
    model.set_prefill(fz.PREFILL_BF16)
    for p0 in range(0, len(prompt), 512):
        model.step(p0, prompt[p0:p0 + 512], logits=p0 + 512 >= len(prompt))
    got = model.logits()
    want = oracle.prompt(prompt)
    err = _rel_err(got, want)
    print(f"fast prefill, 26 layers, 2,048 tokens: max |logit error| / max |logit| = {err:.2e}")
    assert err < 1e-3
    model.close()
    oracle.close()


def test_fast_prefill_mixed_formats(device):
    # The pinned file's formats in the fast mode: a Q8_0 embedding (and so
    # tied head) and Q4_1 / Q8_0 downs, whose weight planes keep their own
    # unpack. A 600-token prompt in steps of 512 and 88: the prompt-end
    # logits within 1e-3 (max-norm relative) of the oracle's over the same
    # formats.
    cfg = small_config()
    t = _mixed_tensors(cfg, 43)
    oracle = orc.OracleModel(cfg.as_dict(), t, formats=MIXED)
    model = fz.Model(device, cfg)
    _set_all(model, t, MIXED)
    zeros = np.zeros(2 * cfg.layers, dtype=np.uint32)
    model.set_edits(zeros)
    prompt = np.random.default_rng(44).integers(0, cfg.vocab, 600).astype(np.uint32)
    _, want = oracle_run(oracle, prompt, 0, cfg)
    model.set_prefill(fz.PREFILL_BF16)
    for p0 in range(0, len(prompt), 512):
        model.step(p0, prompt[p0:p0 + 512], logits=p0 + 512 >= len(prompt))
    err = _rel_err(model.logits(), want)
    print(f"fast prefill, mixed formats, 600 tokens: max |logit error| / max |logit| = {err:.2e}")
    assert err < 1e-3
    model.close()
    oracle.close()
