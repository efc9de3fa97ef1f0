"""Each HIP kernel alone on the GPU against the CPU oracle, bit for bit, at
Gemma-3-1B's shapes (the reference's kernel contract tests run one launch
over scratch buffers the same way: tests/support/scratch_program.h:62-80)."""
import numpy as np
import pytest

import _oracle as orc
import frizzle_amd as fz
from helpers import assert_same_bits, bits, format_blocks, q4_blocks

pytestmark = pytest.mark.gpu


def _q4_dev(device, blocks):
    codes, scales = fz.q4_0_split(blocks)
    return device.array(codes), device.array(scales)


# ---- shared numerics ------------------------------------------------------

def _numerics(device, which, x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    din = device.array(x)
    dout = device.empty(x.shape, np.float32)
    fz.load().frz_op_numerics(device.handle, which, din.ptr, dout.ptr, x.size)
    return dout.numpy()


def test_numerics_match_oracle(device):
    rng = np.random.default_rng(1)
    L = orc.lib()
    cases = {
        0: (rng.uniform(-130, 1, 20000), L.orc_exp2),
        1: (rng.uniform(-np.pi, np.pi, 20000), L.orc_cos),
        2: (rng.uniform(-np.pi, np.pi, 20000), L.orc_sin),
        3: (np.abs(rng.normal(0, 50, 20000)) + 1e-6, L.orc_inverse_sqrt),
        4: (rng.normal(0, 4, 20000), L.orc_gelu_tanh),
        5: (rng.uniform(-120, 0, 20000), L.orc_exp_nonpositive),
    }
    for which, (x, ref) in cases.items():
        x = x.astype(np.float32)
        got = _numerics(device, which, x)
        want = np.array([ref(float(v)) for v in x], dtype=np.float32)
        assert_same_bits(got, want, f"numerics {which}")


def test_f16_pack_matches_oracle(device):
    rng = np.random.default_rng(2)
    x = np.concatenate([
        rng.normal(0, 1, 20000), rng.normal(0, 1e-5, 5000),
        rng.normal(0, 3e4, 5000), [65504, 65520, 1e9, -1e9, 0.0, -0.0]]).astype(np.float32)
    got = _numerics(device, 6, x).view(np.uint32) & 0xFFFF
    want = np.array([orc.lib().orc_f16_pack(float(v)) for v in x], dtype=np.uint32)
    assert np.array_equal(got, want)


def test_sqrt_and_division_correctly_rounded(device):
    # The norm's inverse sqrt is built from IEEE sqrt and division; both must
    # round correctly on the device as on the host.
    rng = np.random.default_rng(3)
    x = np.abs(rng.normal(0, 100, 50000)).astype(np.float32) + np.float32(1e-30)
    got = _numerics(device, 7, x)
    assert_same_bits(got, np.sqrt(x), "sqrt")
    pairs = rng.normal(0, 10, 50000).astype(np.float32)
    pairs[1::2] += np.float32(0.1)
    got = _numerics(device, 8, pairs)
    want = np.repeat(pairs[0::2] / pairs[1::2], 2)
    assert_same_bits(got, want, "division")


# ---- products ---------------------------------------------------------------

SHAPES = [(1536, 1152), (1152, 1024), (6912, 1152), (1152, 6912), (100, 64),
          (16384 + 40, 1152)]


@pytest.mark.parametrize("rows,cols", SHAPES)
def test_gemv_decode_bit_exact(device, rows, cols):
    rng = np.random.default_rng(rows * 7 + cols)
    w = q4_blocks(rng, rows, cols)
    x = rng.normal(0, 1, cols).astype(np.float32)
    codes, scales = _q4_dev(device, w)
    dx = device.array(x)
    dy = device.empty((rows,), np.float32)
    fz._lib.check(fz.load().frz_op_gemv(device.handle, codes.ptr, scales.ptr, rows, cols,
                                        dx.ptr, cols, dy.ptr, rows, 1, 0))
    assert_same_bits(dy.numpy(), orc.gemv(w, rows, cols, x), f"gemv {rows}x{cols}")


def _every_scale_blocks(rng, rows, cols):
    """rows x cols Q4_0 blocks whose scales run through every finite f16
    (subnormals, zeros and negatives included; repeated to fill), codes
    uniform."""
    finite = np.concatenate([np.arange(0x0000, 0x7C00), np.arange(0x8000, 0xFC00)]).astype(np.uint16)
    n = rows * cols // 32
    out = np.empty((n, 18), dtype=np.uint8)
    out[:, 0:2] = np.resize(finite, n).view(np.uint8).reshape(n, 2)
    out[:, 2:] = rng.integers(0, 256, size=(n, 16), dtype=np.uint8)
    return out.reshape(-1)


# The decode forms of the weight (low nibble 1024 + q with d, high nibble
# 1024 + 16 q with d / 16) against the oracle's (q - 8) d, over every finite
# scale: the two-groups-a-lane layout (7 and 14 rows a workgroup) and the
# lane-a-range layout.
@pytest.mark.parametrize("rows,cols", [(1764, 1152), (4200, 1152), (1984, 1024)])
def test_gemv_decode_every_scale_bit_exact(device, rows, cols):
    rng = np.random.default_rng(rows + cols)
    w = _every_scale_blocks(rng, rows, cols)
    x = rng.normal(0, 1, cols).astype(np.float32)
    codes, scales = _q4_dev(device, w)
    dx = device.array(x)
    dy = device.empty((rows,), np.float32)
    fz._lib.check(fz.load().frz_op_gemv(device.handle, codes.ptr, scales.ptr, rows, cols,
                                        dx.ptr, cols, dy.ptr, rows, 1, 0))
    assert_same_bits(dy.numpy(), orc.gemv(w, rows, cols, x), f"gemv {rows}x{cols}")


def test_gated_every_scale_bit_exact(device):
    rng = np.random.default_rng(77)
    rows, cols = 1764, 1152
    g = _every_scale_blocks(rng, rows, cols)
    u = np.roll(_every_scale_blocks(rng, rows, cols).reshape(-1, 18), 1000, axis=0).reshape(-1)
    x = rng.normal(0, 1, cols).astype(np.float32)
    gc, gs = _q4_dev(device, g)
    uc, us = _q4_dev(device, u)
    dx = device.array(x)
    da = device.empty((1, rows), np.float32)
    fz._lib.check(fz.load().frz_op_gated(device.handle, gc.ptr, gs.ptr, uc.ptr, us.ptr, rows,
                                         cols, dx.ptr, da.ptr, 1, 0, None, 0))
    assert_same_bits(da.numpy()[0], orc.gated(g, u, rows, cols, x), "gated")


# Neuron counts whose tiles of 7 do not fill the last workgroup's two: its
# second tile is the last one again, recomputed to the same bits.
@pytest.mark.parametrize("rows", [100, 21, 7])
def test_gated_ragged_tiles_bit_exact(device, rows):
    rng = np.random.default_rng(300 + rows)
    cols, layers, layer, position = 1152, 2, 1, 9
    g = q4_blocks(rng, rows, cols)
    u = q4_blocks(rng, rows, cols)
    x = rng.normal(0, 1, (1, cols)).astype(np.float32)
    edits = [fz.Edit(layer, n, fz.EditKind.SET, 0.25 * n) for n in range(0, rows, 5)]
    table = fz.edit_table(edits, layers, origin=position)
    gc, gs = _q4_dev(device, g)
    uc, us = _q4_dev(device, u)
    dx, dt = device.array(x), device.array(table)
    da = device.empty((1, rows), np.float32)
    fz._lib.check(fz.load().frz_op_gated(device.handle, gc.ptr, gs.ptr, uc.ptr, us.ptr, rows,
                                         cols, dx.ptr, da.ptr, 1, position, dt.ptr, layer))
    want = orc.gated(g, u, rows, cols, x[0])
    orc.lib().orc_edit_row(table.ctypes.data, layer, position, rows, want.ctypes.data)
    assert_same_bits(da.numpy()[0], want, f"gated {rows} neurons")


@pytest.mark.parametrize("rows,cols,tokens", [(1536, 1152, 5), (1152, 6912, 37),
                                               (1152, 1024, 64), (200, 96, 3)])
def test_gemv_tiled_is_decode_bits(device, rows, cols, tokens):
    # Batch invariance (matmul.h:63-72): each token's outputs in a tiled step
    # are the bits it gets decoded alone.
    rng = np.random.default_rng(rows + tokens)
    w = q4_blocks(rng, rows, cols)
    x = rng.normal(0, 1, (tokens, cols)).astype(np.float32)
    codes, scales = _q4_dev(device, w)
    dx = device.array(x)
    dy = device.empty((tokens, rows), np.float32)
    fz._lib.check(fz.load().frz_op_gemv(device.handle, codes.ptr, scales.ptr, rows, cols,
                                        dx.ptr, cols, dy.ptr, rows, tokens, 0))
    got = dy.numpy()
    for t in range(tokens):
        assert_same_bits(got[t], orc.gemv(w, rows, cols, x[t]), f"token {t}")


@pytest.mark.parametrize("rows,cols,tokens", [(1152, 6912, 16), (1152, 1024, 2), (100, 1152, 1),
                                               (16384 + 40, 1152, 16), (1536, 1152, 9),
                                               (32768 + 40, 1152, 16), (32768 + 8, 1152, 3)])
def test_gemv_split_passes_bit_exact(device, rows, cols, tokens):
    # Steps of at most 16 rows split each tile's passes over a workgroup's
    # waves; the range sums meet in LDS and are added in range order. The
    # tokens = 1 case is the decode form (last_token). From 32,768 rows a
    # wave chains two tiles over the same inputs (the last pair ragged or
    # past the end).
    rng = np.random.default_rng(rows + 3 * tokens)
    w = q4_blocks(rng, rows, cols)
    x = rng.normal(0, 1, (tokens, cols)).astype(np.float32)
    codes, scales = _q4_dev(device, w)
    dx = device.array(x)
    dy = device.empty((tokens, rows), np.float32)
    fz._lib.check(fz.load().frz_op_gemv(device.handle, codes.ptr, scales.ptr, rows, cols,
                                        dx.ptr, cols, dy.ptr, rows, tokens, 0))
    got = dy.numpy()
    for t in range(tokens):
        assert_same_bits(got[t], orc.gemv(w, rows, cols, x[t]), f"token {t}")


def test_gemv_tiled_subnormal_products(device):
    # Products and sums below f32's normal range: the prefill's chains keep
    # subnormals exactly as the reference's fma does.
    rng = np.random.default_rng(5)
    rows, cols, tokens = 80, 128, 17
    w = q4_blocks(rng, rows, cols)
    x = (rng.normal(0, 1, (tokens, cols)) * 1e-37).astype(np.float32)
    codes, scales = _q4_dev(device, w)
    dx = device.array(x)
    dy = device.empty((tokens, rows), np.float32)
    fz._lib.check(fz.load().frz_op_gemv(device.handle, codes.ptr, scales.ptr, rows, cols,
                                        dx.ptr, cols, dy.ptr, rows, tokens, 0))
    got = dy.numpy()
    assert np.count_nonzero((got != 0) & (np.abs(got) < np.float32(1.1754944e-38))) > 0
    for t in range(tokens):
        assert_same_bits(got[t], orc.gemv(w, rows, cols, x[t]), f"token {t}")


def test_gemv_last_token(device):
    rng = np.random.default_rng(9)
    rows, cols, tokens = 40000, 1152, 7
    w = q4_blocks(rng, rows, cols)
    x = rng.normal(0, 1, (tokens, cols)).astype(np.float32)
    codes, scales = _q4_dev(device, w)
    dx = device.array(x)
    dy = device.empty((rows,), np.float32)
    fz._lib.check(fz.load().frz_op_gemv(device.handle, codes.ptr, scales.ptr, rows, cols,
                                        dx.ptr, cols, dy.ptr, rows, tokens, 1))
    assert_same_bits(dy.numpy(), orc.gemv(w, rows, cols, x[-1]), "head")


# ---- Q4_1 and Q8_0 weights (the pinned file's first downs and its embedding,
#      which is also the tied head) -------------------------------------------

def _format_dev(device, fmt, blocks):
    codes, scales = fz.block_split(fmt, blocks)
    return device.array(codes), device.array(scales)


def _gemv_format(device, fmt, w, rows, cols, x, tokens, last_token=0):
    codes, scales = _format_dev(device, fmt, w)
    dx = device.array(x)
    n_out = 1 if (tokens == 1 or last_token) else tokens
    dy = device.empty((n_out, rows), np.float32)
    fz._lib.check(fz.load().frz_op_gemv_format(device.handle, fmt, codes.ptr, scales.ptr, rows,
                                               cols, dx.ptr, cols, dy.ptr, rows, tokens,
                                               last_token))
    return dy.numpy()


@pytest.mark.parametrize("fmt,rows,cols", [(3, 1152, 6912), (8, 1152, 6912), (3, 1536, 1152),
                                           (8, 16384 + 40, 1152), (3, 100, 64), (8, 100, 64)])
def test_gemv_format_decode_bit_exact(device, fmt, rows, cols):
    rng = np.random.default_rng(fmt * 1000 + rows + cols)
    w = format_blocks(rng, fmt, rows, cols)
    x = rng.normal(0, 1, cols).astype(np.float32)
    got = _gemv_format(device, fmt, w, rows, cols, x, 1)[0]
    assert_same_bits(got, orc.gemv_format(fmt, w, rows, cols, x), f"format {fmt} {rows}x{cols}")


@pytest.mark.parametrize("fmt,rows,cols,tokens", [(3, 1152, 6912, 37), (8, 1152, 6912, 37),
                                                  (3, 1152, 6912, 16), (8, 4096, 1152, 16),
                                                  (3, 200, 96, 3), (8, 200, 96, 3),
                                                  (3, 1600, 1152, 512), (8, 1600, 1152, 512)])
def test_gemv_format_tiled_bit_exact(device, fmt, rows, cols, tokens):
    # 1600 x 512 outputs take the 32 x 32 tiles, the others the 16 x 16 ones.
    rng = np.random.default_rng(fmt + rows + tokens)
    w = format_blocks(rng, fmt, rows, cols)
    x = rng.normal(0, 1, (tokens, cols)).astype(np.float32)
    got = _gemv_format(device, fmt, w, rows, cols, x, tokens)
    for t in range(tokens):
        assert_same_bits(got[t], orc.gemv_format(fmt, w, rows, cols, x[t]), f"token {t}")


def test_gemv_q8_0_head_last_token(device):
    rng = np.random.default_rng(19)
    rows, cols, tokens = 40000, 1152, 7
    w = format_blocks(rng, 8, rows, cols)
    x = rng.normal(0, 1, (tokens, cols)).astype(np.float32)
    got = _gemv_format(device, 8, w, rows, cols, x, tokens, last_token=1)[0]
    assert_same_bits(got, orc.gemv_format(8, w, rows, cols, x[-1]), "Q8_0 head")


def test_gemv_format_refusals(device):
    codes = device.empty((64,), np.uint8)
    x = device.empty((64,), np.float32)
    y = device.empty((2,), np.float32)
    for fmt in (0, 1, 6):
        with pytest.raises(fz.FrzError, match="format"):
            fz._lib.check(fz.load().frz_op_gemv_format(device.handle, fmt, codes.ptr, codes.ptr,
                                                       2, 32, x.ptr, 32, y.ptr, 2, 1, 0))


def test_gather_q8_0_bit_exact(device):
    rng = np.random.default_rng(37)
    rows, cols = 5000, 1152
    table = format_blocks(rng, 8, rows, cols)
    ids = np.array([0, 4999, 17, 17, 2500], dtype=np.uint32)
    codes, scales = _format_dev(device, 8, table)
    dh = device.empty((ids.size, cols), np.float32)
    scale = np.float32(np.sqrt(np.float32(cols)))
    fz._lib.check(fz.load().frz_op_gather_format(device.handle, 8, codes.ptr, scales.ptr, rows,
                                                 cols, ids.ctypes.data, ids.size, scale, dh.ptr))
    got = dh.numpy()
    for i, tok in enumerate(ids):
        assert_same_bits(got[i], orc.gather_row_format(8, table, cols, int(tok), scale),
                         f"row {i}")


@pytest.mark.parametrize("tokens", [1, 6, 16, 37])
def test_gated_with_pins_bit_exact(device, tokens):
    rng = np.random.default_rng(11 + tokens)
    rows, cols, layers, layer = 6912, 1152, 3, 1
    g = q4_blocks(rng, rows, cols)
    u = q4_blocks(rng, rows, cols)
    x = rng.normal(0, 1, (tokens, cols)).astype(np.float32)
    position = 40
    edits = [fz.Edit(layer, n, fz.EditKind(n % 3), float(n) * 0.5 if n % 3 == 0 else
                     (-1.75 if n % 3 == 1 else 0.0), 2, fz.TO_THE_END)
             for n in range(10, 160)]
    edits += [fz.Edit(layer, 7, fz.EditKind.SCALE, 1.0), fz.Edit(0, 3, fz.EditKind.SET, 99.0),
              fz.Edit(layer, 6911, fz.EditKind.SET, -20.0, 0, 1)]
    table = fz.edit_table(edits, layers, origin=position - 2)
    gc, gs = _q4_dev(device, g)
    uc, us = _q4_dev(device, u)
    dx = device.array(x)
    dt = device.array(table)
    da = device.empty((tokens, rows), np.float32)
    fz._lib.check(fz.load().frz_op_gated(device.handle, gc.ptr, gs.ptr, uc.ptr, us.ptr, rows,
                                         cols, dx.ptr, da.ptr, tokens, position, dt.ptr, layer))
    got = da.numpy()
    for t in range(tokens):
        want = orc.gated(g, u, rows, cols, x[t])
        orc.lib().orc_edit_row(table.ctypes.data, layer, position + t, rows, want.ctypes.data)
        assert_same_bits(got[t], want, f"gated token {t}")


# ---- per-row kernels ----------------------------------------------------------

@pytest.mark.parametrize("add", [False, True])
def test_norm_bit_exact(device, add):
    rng = np.random.default_rng(21)
    tokens, width = 9, 1152
    hidden = rng.normal(0, 3, (tokens, width)).astype(np.float32)
    output = rng.normal(0, 2, (tokens, width)).astype(np.float32)
    gain = (1 + 0.1 * rng.normal(0, 1, width)).astype(np.float32)
    post = (1 + 0.1 * rng.normal(0, 1, width)).astype(np.float32)
    dh, dn = device.array(hidden), device.empty((tokens, width), np.float32)
    dg, dp, do = device.array(gain), device.array(post), device.array(output)
    fz._lib.check(fz.load().frz_op_norm(device.handle, dg.ptr, dp.ptr if add else None,
                                        do.ptr, dh.ptr, dn.ptr, width, 1e-6, tokens, 0))
    gh, gn = dh.numpy(), dn.numpy()
    for t in range(tokens):
        wh, wn = orc.norm_row(gain, hidden[t], output[t] if add else None,
                              post if add else None)
        assert_same_bits(gh[t], wh, "hidden")
        assert_same_bits(gn[t], wn, "normed")


@pytest.mark.parametrize("base,position", [(10000.0, 0), (10000.0, 700), (1e6, 4099)])
def test_rope_bit_exact(device, base, position):
    rng = np.random.default_rng(int(position) + 5)
    tokens, qh, kvh, d, slots = 3, 4, 1, 256, 640
    qkv = rng.normal(0, 2, (tokens, (qh + 2 * kvh) * d)).astype(np.float32)
    qg = (1 + 0.1 * rng.normal(0, 1, d)).astype(np.float32)
    kg = (1 + 0.1 * rng.normal(0, 1, d)).astype(np.float32)
    turns = fz.rope_turns(base, d)
    assert np.array_equal(turns, orc.rope_turns(base, d))
    dq = device.array(qkv)
    kc = device.empty((slots * d,), np.uint16).zero()
    vc = device.empty((slots * d,), np.uint16).zero()
    dt, dqg, dkg = device.array(turns), device.array(qg), device.array(kg)
    stride = (qh + 2 * kvh) * d
    fz._lib.check(fz.load().frz_op_rope(
        device.handle, dt.ptr, dqg.ptr, dkg.ptr, dq.ptr, dq.ptr + qh * d * 4,
        dq.ptr + (qh + kvh) * d * 4, stride, stride, kc.ptr, vc.ptr, slots, d, qh, kvh,
        1e-6, position, tokens))
    got_q = dq.numpy()
    want_k = np.zeros(slots * d, dtype=np.uint16)
    want_v = np.zeros(slots * d, dtype=np.uint16)
    for t in range(tokens):
        q = qkv[t, :qh * d].copy()
        k = qkv[t, qh * d:(qh + kvh) * d].copy()
        v = qkv[t, (qh + kvh) * d:].copy()
        orc.lib().orc_rope_row(position + t, slots, d, qh, kvh, 1e-6, turns.ctypes.data,
                               qg.ctypes.data, kg.ctypes.data, q.ctypes.data, k.ctypes.data,
                               v.ctypes.data, want_k.ctypes.data, want_v.ctypes.data)
        assert_same_bits(got_q[t, :qh * d], q, f"query {t}")
    assert np.array_equal(kc.numpy(), want_k)
    assert np.array_equal(vc.numpy(), want_v)


@pytest.mark.parametrize("position,tokens,window,slots", [
    (0, 1, 512, 5120), (700, 1, 512, 640), (5000, 1, 512, 5120), (100, 4, 512, 5120),
    (1000, 1, 4096, 4096), (4095, 1, 32768, 8192), (63, 2, 512, 5120),
    # past the 224 chunk states one fold stage holds: folded in segments
    (20000, 3, 32768, 32768), (32767, 1, 32768, 32768), (14400, 1, 14400, 16384)])
def test_attention_bit_exact(device, position, tokens, window, slots):
    rng = np.random.default_rng(position + tokens)
    qh, kvh, d = 4, 1, 256
    q = rng.normal(0, 1, (tokens, qh * d)).astype(np.float32)
    # F16-exact cache values (multiples of 1/32), as the reference's
    # attention contract test chooses them.
    kc = (rng.integers(-96, 97, slots * d) / 32.0).astype(np.float16).view(np.uint16)
    vc = (rng.integers(-96, 97, slots * d) / 32.0).astype(np.float16).view(np.uint16)
    dq, dk, dv = device.array(q), device.array(kc), device.array(vc)
    do = device.empty((tokens, qh * d), np.float32)
    fz._lib.check(fz.load().frz_op_attention(device.handle, dq.ptr, qh * d, dk.ptr, dv.ptr,
                                             do.ptr, slots, window, d, qh, kvh, 0.0625,
                                             position, tokens))
    got = do.numpy()
    scale_log2e = np.float32(np.float64(np.float32(0.0625)) * 1.4426950408889634)
    for t in range(tokens):
        want = np.empty(qh * d, dtype=np.float32)
        orc.lib().orc_attention_row(position + t, window, slots, d, qh, kvh, scale_log2e,
                                    q[t].ctypes.data, kc.ctypes.data, vc.ctypes.data,
                                    want.ctypes.data)
        assert_same_bits(got[t], want, f"attention row {t}")


def test_gather_bit_exact(device):
    rng = np.random.default_rng(31)
    rows, cols = 5000, 1152
    table = q4_blocks(rng, rows, cols)
    ids = np.array([0, 4999, 17, 17, 2500], dtype=np.uint32)
    codes, scales = _q4_dev(device, table)
    dids = device.array(ids)
    dh = device.empty((ids.size, cols), np.float32)
    scale = np.float32(np.sqrt(np.float32(cols)))
    fz._lib.check(fz.load().frz_op_gather(device.handle, codes.ptr, scales.ptr, rows, cols,
                                          ids.ctypes.data, ids.size, scale, dh.ptr))
    got = dh.numpy()
    for i, tok in enumerate(ids):
        want = np.empty(cols, dtype=np.float32)
        orc.lib().orc_gather_row(table.ctypes.data, cols, int(tok), scale, want.ctypes.data)
        assert_same_bits(got[i], want, f"row {i}")


def test_edit_kernel_matches_apply(device):
    # The reference's edit kernel contract (tests/contracts/kernels/
    # edit_kernel_test.cpp): 5 rows of 200, >64 edits of every kind, Scale x 1
    # on a subnormal and on -0 keeps their bits; other layers' edits ignored.
    rows, width, layers, layer, origin = 5, 200, 3, 1, 40
    act = ((np.arange(rows * width) % 97) * 0.375 - 13.0).astype(np.float32).reshape(rows, width)
    act[:, 7] = np.array([0x00000123], dtype=np.uint32).view(np.float32)[0]
    act[:, 8] = np.float32(-0.0)
    edits = []
    for n in range(10, 160):
        kind = fz.EditKind(n % 3)
        value = n * 0.5 if kind == fz.EditKind.SET else (-1.75 if kind == fz.EditKind.SCALE else 0.0)
        edits.append(fz.Edit(layer, n, kind, value, 2))
    edits += [fz.Edit(layer, 7, fz.EditKind.SCALE, 1.0, 2), fz.Edit(layer, 8, fz.EditKind.SCALE, 1.0, 2),
              fz.Edit(0, 3, fz.EditKind.SET, 999.0), fz.Edit(2, 4, fz.EditKind.SET, -999.0)]
    assert fz.edit_check(edits, layers, width)[0] == fz.EditError.OK
    table = fz.edit_table(edits, layers, origin)
    da, dt = device.array(act), device.array(table)
    fz._lib.check(fz.load().frz_op_edit(device.handle, dt.ptr, layer, da.ptr, width, origin, rows))
    want = act.copy()
    for r in range(rows):
        orc.lib().orc_edit_row(table.ctypes.data, layer, origin + r, width, want[r].ctypes.data)
    assert_same_bits(da.numpy(), want, "edited")
    # rows at positions 40, 41 untouched; from position 42 on, edited
    assert_same_bits(da.numpy()[:2], act[:2], "before the range")


@pytest.mark.parametrize("count,case", [
    (262144, "normal"), (64, "normal"), (1000, "ties"), (1025, "specials"),
    (16385, "normal"), (300000, "specials"), (50000, "ties")])
def test_topk_matches_oracle(device, count, case):
    # One tile, a ragged last tile, one merge level and two (300,000 logits
    # make 293 lists, then 19, then 2); equal keys order by lower token.
    rng = np.random.default_rng(41 + count)
    logits = rng.normal(0, 3, count).astype(np.float32)
    logits[[5 % count, (70000 % count), count - 1]] = logits.max()
    logits[9 % count] = np.float32(-0.0)
    if case == "ties":
        logits = np.round(logits).astype(np.float32)  # a handful of values, many ties
    if case == "specials":
        specials = np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, np.float32(3.4e38),
                             -np.float32(3.4e38), np.float32(1e-45), -np.float32(1e-45)],
                            dtype=np.float32)
        where = rng.choice(count, 200, replace=False)
        logits[where] = specials[rng.integers(0, specials.size, where.size)]
        logits.view(np.uint32)[where[:5]] = np.array([0x7FC00001, 0xFFC00000, 0x7F800001,
                                                      0xFF812345, 0x7FFFFFFF], dtype=np.uint32)
    dl = device.array(logits)
    dc = device.empty((128,), np.uint32)
    fz._lib.check(fz.load().frz_op_topk(device.handle, dl.ptr, logits.size, dc.ptr))
    got = dc.numpy()
    wb, wi = orc.topk(logits)
    assert np.array_equal(got[0::2], wb)
    assert np.array_equal(got[1::2], wi)


@pytest.mark.parametrize("temperature,top_k,top_p,min_p", [
    (0.0, 1, 1.0, 0.0), (0.8, 40, 0.95, 0.05), (1.0, 64, 1.0, 0.0), (1.5, 10, 0.5, 0.0)])
def test_draw_matches_oracle(device, temperature, top_k, top_p, min_p):
    rng = np.random.default_rng(51)
    for trial in range(20):
        logits = np.sort(rng.normal(0, 2, 64).astype(np.float32))[::-1]
        cand_bits = bits(logits)
        cand_ids = rng.permutation(262144)[:64].astype(np.uint32)
        cand = np.empty(128, dtype=np.uint32)
        cand[0::2], cand[1::2] = cand_bits, cand_ids
        dc = device.array(cand)
        dr = device.empty((4,), np.uint32)
        seed = 0x123456789 + trial
        s = fz.sampling(temperature, top_k, top_p, min_p, seed)
        fz._lib.check(fz.load().frz_op_draw(device.handle, dc.ptr, s, 100 + trial, 1, dr.ptr))
        want = orc.draw(cand_bits, cand_ids, top_k, temperature, top_p, min_p,
                        counter=101 + trial, seed=seed)
        assert np.array_equal(dr.numpy(), want), (trial, dr.numpy(), want)


def _rope_attention_case(device, position, window, slots, base, kc, vc, rng):
    """The fused decode kernel at one position over caches kc, vc (f16
    bits): its cache slot and its output against the oracle's, the output
    as (got, want)."""
    qh, d = 4, 256
    qkv = rng.normal(0, 2, 6 * d).astype(np.float32)
    qg = (1 + 0.1 * rng.normal(0, 1, d)).astype(np.float32)
    kg = (1 + 0.1 * rng.normal(0, 1, d)).astype(np.float32)
    turns = fz.rope_turns(base, d)
    dqkv, dk, dv = device.array(qkv), device.array(kc), device.array(vc)
    dt, dqg, dkg = device.array(turns), device.array(qg), device.array(kg)
    do = device.empty((qh * d,), np.float32)
    fz._lib.check(fz.load().frz_op_rope_attention(
        device.handle, dqkv.ptr, dt.ptr, dqg.ptr, dkg.ptr, dk.ptr, dv.ptr, do.ptr, slots,
        window, 1e-6, 0.0625, position))
    q = qkv[:qh * d].copy()
    k = qkv[qh * d:(qh + 1) * d].copy()
    v = qkv[(qh + 1) * d:].copy()
    want_k, want_v = kc.copy(), vc.copy()
    orc.lib().orc_rope_row(position, slots, d, qh, 1, 1e-6, turns.ctypes.data, qg.ctypes.data,
                           kg.ctypes.data, q.ctypes.data, k.ctypes.data, v.ctypes.data,
                           want_k.ctypes.data, want_v.ctypes.data)
    assert np.array_equal(dk.numpy(), want_k)
    assert np.array_equal(dv.numpy(), want_v)
    want = np.empty(qh * d, dtype=np.float32)
    scale_log2e = np.float32(np.float64(np.float32(0.0625)) * 1.4426950408889634)
    orc.lib().orc_attention_row(position, window, slots, d, qh, 1, scale_log2e, q.ctypes.data,
                                want_k.ctypes.data, want_v.ctypes.data, want.ctypes.data)
    return do.numpy(), want


@pytest.mark.parametrize("position,window,slots,base", [
    (0, 512, 5120, 1e4), (63, 512, 5120, 1e4), (64, 512, 5120, 1e4), (700, 512, 640, 1e4),
    (5000, 512, 5120, 1e4), (4100, 8192, 8192, 1e6), (1000, 64, 640, 1e4),
    (30000, 32768, 32768, 1e6), (14336, 32768, 32768, 1e6), (4360, 512, 4672, 1e4),
    (4391, 512, 4672, 1e4), (100, 64, 96, 1e4), (40, 512, 48, 1e4)])
def test_rope_attention_decode_bit_exact(device, position, window, slots, base):
    # The decode kernel fuses QK-norm, rope, the KV append and attention; its
    # query, cache slot and output are the separate kernels' bits. Cases with
    # a partial first chunk, the step's key first or last in its chunk, a
    # ring that wraps inside a chunk, and rings under a chunk long.
    rng = np.random.default_rng(position + window)
    kc = (rng.integers(-96, 97, slots * 256) / 32.0).astype(np.float16).view(np.uint16)
    vc = (rng.integers(-96, 97, slots * 256) / 32.0).astype(np.float16).view(np.uint16)
    got, want = _rope_attention_case(device, position, window, slots, base, kc, vc, rng)
    assert_same_bits(got, want, "decode attention")


def test_rope_attention_decode_subnormal_and_nonfinite_rows(device):
    # f16 subnormals in the cache enter the products exactly; a value row the
    # token does not see but whose tile it scores (the first tile's keys
    # before the window) still multiplies its weight 0: an infinity there
    # makes its dimension NaN, as in the reference.
    position, window, slots = 5000, 512, 5120
    rng = np.random.default_rng(7)
    kc = (rng.integers(-96, 97, slots * 256) / 32.0).astype(np.float16)
    vc = (rng.integers(-96, 97, slots * 256) / 32.0).astype(np.float16)
    sub = rng.integers(1, 1024, slots * 256).astype(np.uint16)  # subnormal bit patterns
    pick = rng.random(slots * 256) < 0.3
    kc = kc.view(np.uint16).copy()
    vc = vc.view(np.uint16).copy()
    kc[pick] = sub[pick] | (rng.integers(0, 2, pick.sum()).astype(np.uint16) << 15)
    vc[pick] = sub[pick]
    got, want = _rope_attention_case(device, position, window, slots, 1e4, kc, vc, rng)
    assert_same_bits(got, want, "decode attention, subnormal cache")
    earliest = position + 1 - window
    first = earliest // 8 * 8
    assert first < earliest  # a key the token does not see, in a scored tile
    vc[first * 256 + 17] = 0x7C00  # +inf
    got, want = _rope_attention_case(device, position, window, slots, 1e4, kc, vc,
                                     np.random.default_rng(8))
    assert np.isnan(want[17::256]).all() and np.isnan(got[17::256]).all()
    keep = ~np.isnan(want)
    assert np.array_equal(np.isnan(got), ~keep)
    assert_same_bits(got[keep], want[keep], "decode attention, other dimensions")


@pytest.mark.parametrize("position,window,slots", [(100, 512, 96), (100, 16, 32)])
def test_rope_attention_decode_refuses_short_rings(device, position, window, slots):
    # A ring with fewer slots than the window's keys would have the step's
    # key appended over a key the step reads; under 64 slots, a chunk's rows
    # could wrap it twice. Both are refused before any launch.
    rng = np.random.default_rng(3)
    kc = np.zeros(slots * 256, np.uint16)
    with pytest.raises(fz.FrzError, match="fewer slots than the window"):
        _rope_attention_case(device, position, window, slots, 1e4, kc, kc.copy(), rng)
