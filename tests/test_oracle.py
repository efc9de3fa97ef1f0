"""Pins the CPU oracle itself (no GPU): against the reference's own fixture,
closed forms, brute force, an independent IEEE library (numpy) and f64
mathematics, each check chosen so that a plausible slip in the restatement (a
dropped term, a wrong sign or index, a transposed operand, another order of
addition, an unfused fma) fails it.

What these cannot pin is the exact bits the reference's WGSL built-ins give
on its own GPUs (inverseSqrt, cos, sin, exp2, exp): the oracle fixes each to a
stated definition and these tests bound its accuracy; the bits themselves
stay "parity unpinned".
"""
import math
from pathlib import Path

import numpy as np
import pytest

import _oracle as orc
from helpers import bits, dequant, q4_blocks, read_gguf

GOLDEN = Path(__file__).resolve().parent / "golden"
U = 2.0 ** -24  # unit roundoff of f32


def f32(x):
    return np.float32(x)


def ulps(a, b):
    """Distance in f32 units in the last place (same sign assumed)."""
    ia = np.asarray(a, dtype=np.float32).view(np.int32).astype(np.int64)
    ib = np.asarray(b, dtype=np.float32).view(np.int32).astype(np.int64)
    return np.abs(ia - ib)


# ---- the reference's own fixture -------------------------------------------------

def test_q4_0_matches_reference_fixture():
    # tests/fixtures/gguf/valid.gguf (made by make_gguf_fixtures.py:65-73):
    # token_embd.weight is Q4_0 [64, 2], four blocks of scale 0x3C00 (1.0)
    # and code byte 0x10, so each block is sixteen -8s then sixteen -7s.
    t = read_gguf(GOLDEN / "gguf" / "valid.gguf")
    dims, ttype, raw = t[b"token_embd.weight"]
    assert dims == [64, 2] and ttype == 2 and len(raw) == 4 * 18
    blocks = np.frombuffer(raw, dtype=np.uint8).reshape(4, 18)
    for b in blocks:
        w = orc.q4_0_unpack(b)
        assert np.array_equal(w, np.array([-8.0] * 16 + [-7.0] * 16, dtype=np.float32))
    # the same bytes through the product: row o of the [64 x 2] matrix
    w = np.frombuffer(raw, dtype=np.uint8)
    y = orc.gemv(w, 2, 64, np.ones(64, dtype=np.float32))
    assert np.array_equal(y, np.array([-480.0, -480.0], dtype=np.float32))  # 2 blocks a row
    dims, ttype, raw = t[b"output_norm.weight"]
    assert np.array_equal(np.frombuffer(raw, dtype=np.float32), [1, 2, 3, 4])


# ---- formats -----------------------------------------------------------------------

def test_q4_0_exact_for_every_code_and_finite_scale():
    # Weight = (code - 8) d is exact in f32 for every finite f16 d
    # (format.h:94-100): compare with the product taken in f64.
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    d = h.view(np.float16)
    finite = h[np.isfinite(d)]
    codes = np.arange(256, dtype=np.uint8)[:16] | (np.arange(16, dtype=np.uint8) << 4)[::-1]
    block = np.empty(18, dtype=np.uint8)
    block[2:] = codes
    lo = (codes & 15).astype(np.float64) - 8
    hi = (codes >> 4).astype(np.float64) - 8
    for s in finite[::7]:
        block[0:2] = np.array([s], dtype=np.uint16).view(np.uint8)
        w = orc.q4_0_unpack(block)
        dv = np.float64(np.array([s], dtype=np.uint16).view(np.float16)[0])
        want = np.concatenate([lo, hi]) * dv
        assert np.array_equal(w.astype(np.float64), want), hex(s)


def test_f16_unpack_is_exact_for_all_bits():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = np.array([orc.lib().orc_f16_unpack(int(v)) for v in h[::3]], dtype=np.float32)
    want = h[::3].view(np.float16).astype(np.float32)
    same = (bits(got) == bits(want)) | (np.isnan(got) & np.isnan(want))
    assert same.all()


def test_f16_pack_saturates_then_rounds_to_nearest_even():
    # f16_pack.wgsl:16-25: clamp to +-65504, then one round to nearest even;
    # numpy's float16 conversion is IEEE round to nearest even.
    rng = np.random.default_rng(1)
    h = np.arange(0, 0x7C00, dtype=np.uint32).astype(np.uint16)
    f = h.view(np.float16).astype(np.float64)
    nxt = np.append(f[1:], 65520.0)
    halfway = ((f + nxt) / 2).astype(np.float32)  # exact ties, both directions
    vals = np.concatenate([
        halfway, np.nextafter(halfway, np.float32(0)), np.nextafter(halfway, np.float32(1e9)),
        rng.normal(0, 1, 20000).astype(np.float32), rng.normal(0, 3e4, 5000).astype(np.float32),
        (rng.random(5000) * 1e-5).astype(np.float32),
        np.array([0.0, 65504.0, 65519.99, 65520.0, 1e6, 3.4e38, np.inf], dtype=np.float32)])
    vals = np.concatenate([vals, -vals])
    got = np.array([orc.lib().orc_f16_pack(float(v)) for v in vals], dtype=np.uint16)
    want = np.clip(vals, -65504, 65504).astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


# ---- the rounding points the reference leaves to built-ins ---------------------------

def test_inverse_sqrt_is_two_correctly_rounded_operations():
    rng = np.random.default_rng(2)
    x = np.concatenate([np.abs(rng.normal(0, 1, 20000)), rng.random(2000) * 1e-30,
                        rng.random(2000) * 1e30]).astype(np.float32) + np.float32(1e-38)
    got = np.array([orc.lib().orc_inverse_sqrt(float(v)) for v in x], dtype=np.float32)
    want = np.float32(1.0) / np.sqrt(x)
    assert np.array_equal(bits(got), bits(want))


def test_dot4_adds_in_order():
    # ((a0 b0 + a1 b1) + a2 b2) + a3 b3, each rounded: 2^24 + 1 + 1 stays
    # 2^24 this way; any other association gives 2^24 + 2.
    a = np.array([2.0 ** 24, 1.0, 1.0, 0.0], dtype=np.float32)
    b = np.ones(4, dtype=np.float32)
    assert orc.lib().orc_dot4(a.ctypes.data, b.ctypes.data) == 2.0 ** 24
    a = np.array([1.0, 1.0, 2.0 ** 24, 0.0], dtype=np.float32)
    assert orc.lib().orc_dot4(a.ctypes.data, b.ctypes.data) == 2.0 ** 24 + 2


def test_exp2_accuracy_and_exact_powers():
    L = orc.lib()
    for k in range(-125, 128):
        assert L.orc_exp2(float(k)) == 2.0 ** k
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.uniform(-125, 127, 20000), rng.uniform(-1, 1, 5000)]).astype(np.float32)
    got = np.array([L.orc_exp2(float(v)) for v in x], dtype=np.float32)
    want = np.exp2(x.astype(np.float64)).astype(np.float32)
    assert ulps(got, want).max() <= 2
    assert L.orc_exp2(-200.0) == 0.0


def test_exp_nonpositive_accuracy():
    # attention/matmul's exp(x) for x <= 0 (matmul.wgsl:122-150): Cody-Waite
    # split and a degree-6 Taylor polynomial; bounded against f64 exp.
    L = orc.lib()
    assert L.orc_exp_nonpositive(0.0) == 1.0
    rng = np.random.default_rng(4)
    x = -np.concatenate([rng.random(20000) * 80, rng.random(5000) * 1e-3]).astype(np.float32)
    got = np.array([L.orc_exp_nonpositive(float(v)) for v in x], dtype=np.float64)
    want = np.exp(x.astype(np.float64))
    rel = np.abs(got - want) / want
    assert rel.max() < 2.0 ** -20


def test_gelu_tanh_accuracy():
    L = orc.lib()
    rng = np.random.default_rng(5)
    g = np.concatenate([rng.normal(0, 3, 20000), [0.0, -0.0, 1e-20, -30, 30]]).astype(np.float32)
    got = np.array([L.orc_gelu_tanh(float(v)) for v in g], dtype=np.float64)
    gd = g.astype(np.float64)
    want = 0.5 * gd * (1 + np.tanh(math.sqrt(2 / math.pi) * (gd + 0.044715 * gd ** 3)))
    err = np.abs(got - want) / np.maximum(1.0, np.abs(want))
    assert err.max() < 2.0 ** -20
    assert L.orc_gelu_tanh(0.0) == 0.0


@pytest.mark.parametrize("which", ["sin", "cos"])
def test_sin_cos_accuracy_over_rope_angles(which):
    # rope.wgsl reduces every angle to 2 pi (t - round(t)), within [-pi, pi].
    L = orc.lib()
    fn = L.orc_sin if which == "sin" else L.orc_cos
    rng = np.random.default_rng(6)
    a = np.concatenate([rng.uniform(-math.pi, math.pi, 30000), [0.0, math.pi / 2, -math.pi]])
    a = a.astype(np.float32)
    got = np.array([fn(float(v)) for v in a], dtype=np.float64)
    want = (np.sin if which == "sin" else np.cos)(a.astype(np.float64))
    assert np.abs(got - want).max() < 2.0 ** -22
    assert L.orc_sin(0.0) == 0.0 and L.orc_cos(0.0) == 1.0


# ---- products ------------------------------------------------------------------------

def blocks_from(weights_int, scale=1.0):
    """GGUF Q4_0 blocks holding integer weights in -8..7 at scale `scale`."""
    rows, cols = weights_int.shape
    q = (np.asarray(weights_int) + 8).astype(np.uint8).reshape(-1, 32)
    out = np.empty((q.shape[0], 18), dtype=np.uint8)
    out[:, 0:2] = np.full(q.shape[0], scale, dtype=np.float16).view(np.uint8).reshape(-1, 2)
    out[:, 2:] = (q[:, :16] & 15) | ((q[:, 16:] & 15) << 4)
    return out.reshape(-1)


@pytest.mark.parametrize("rows,cols", [(40, 1152), (8, 6912), (16, 1024), (3, 64)])
def test_gemv_exact_on_integers(rows, cols):
    # Small integers keep every product and sum exact, whatever the order:
    # the result must be the integer dot product (no dropped or doubled
    # term, no sign slip, rows and columns not transposed).
    rng = np.random.default_rng(rows + cols)
    w = rng.integers(-8, 8, (rows, cols))
    x = rng.integers(-50, 51, cols)
    y = orc.gemv(blocks_from(w), rows, cols, x.astype(np.float32))
    assert np.array_equal(y, (w @ x).astype(np.float32))


def range_of(group, groups):
    return next(r for r in range(32) if r * groups // 32 <= group < (r + 1) * groups // 32)


@pytest.mark.parametrize("cols", [1152, 6912, 1024])
def test_gemv_ranges_and_their_order(cols):
    # matmul.h:88-97: range r is groups floor(rG/32)..floor((r+1)G/32),
    # chained from zero; the 32 range sums add in order. 2^24 in group 0 and
    # +1 in groups a and b: when a and b share a range its sum is 2 and the
    # total 2^24 + 2; in two ranges, each +1 rounds away against 2^24.
    G = cols // 32
    checked = 0
    for a in range(1, G - 1):
        b = a + 1
        w = np.zeros((1, cols), dtype=np.int64)
        x = np.zeros(cols, dtype=np.float32)
        w[0, 0], x[0] = 1, 2.0 ** 24  # range 0 holds 2^24
        w[0, 32 * a], x[32 * a] = 1, 1.0
        w[0, 32 * b], x[32 * b] = 1, 1.0
        if range_of(0, G) in (range_of(a, G), range_of(b, G)):
            continue
        y = orc.gemv(blocks_from(w), 1, cols, x)[0]
        same = range_of(a, G) == range_of(b, G)
        assert y == (2.0 ** 24 + 2 if same else 2.0 ** 24), (cols, a, b)
        checked += 1
    assert checked > 20


def test_gemv_chains_by_fused_multiply_add():
    # Within a range each product enters by fma. Integer weights and random
    # x make products that f32 cannot hold, so fused and unfused chains part
    # ways; the fused chain is computed here in f64 (where each w x is exact)
    # rounded once per step.
    cols = 1024  # one group a range
    rng = np.random.default_rng(18)
    w = rng.integers(-8, 8, (1, cols))
    x = rng.normal(0, 1, cols).astype(np.float32)
    y = orc.gemv(blocks_from(w), 1, cols, x)[0]

    def chain(fused):
        total = np.float32(0.0)
        for r in range(32):
            s = np.float32(0.0)
            for k in range(32 * r, 32 * r + 32):
                if fused:
                    s = np.float32(np.float64(s) + np.float64(w[0, k]) * np.float64(x[k]))
                else:
                    s = np.float32(s + np.float32(np.float32(w[0, k]) * x[k]))
            total = np.float32(total + s)
        return total

    assert chain(True) != chain(False)  # the inputs tell the two apart
    assert y == chain(True)


@pytest.mark.parametrize("rows,cols", [(64, 1152), (32, 6912)])
def test_gemv_within_error_bound_of_f64(rows, cols):
    # |y - y64| <= gamma(2K) sum |w x| (matmul.h:71-78).
    rng = np.random.default_rng(7)
    wb = q4_blocks(rng, rows, cols)
    x = rng.normal(0, 1, cols).astype(np.float32)
    y = orc.gemv(wb, rows, cols, x).astype(np.float64)
    w = dequant(wb, rows, cols)
    exact = w @ x.astype(np.float64)
    n = 2 * cols
    gamma = n * U / (1 - n * U)
    assert np.all(np.abs(y - exact) <= gamma * (np.abs(w) @ np.abs(x.astype(np.float64))))


def test_gated_is_gelu_of_gate_times_up():
    rng = np.random.default_rng(8)
    rows, cols = 64, 1152
    g, u = q4_blocks(rng, rows, cols), q4_blocks(rng, rows, cols)
    x = rng.normal(0, 1, cols).astype(np.float32)
    act = orc.gated(g, u, rows, cols, x)
    gv, uv = orc.gemv(g, rows, cols, x), orc.gemv(u, rows, cols, x)
    L = orc.lib()
    want = np.array([np.float32(L.orc_gelu_tanh(float(a))) * b for a, b in zip(gv, uv)],
                    dtype=np.float32)
    assert np.array_equal(bits(act), bits(want))


# ---- per-row kernels -------------------------------------------------------------------

def test_norm_against_f64():
    # normed = (X r) g with r = 1/sqrt(mean X^2 + eps); the add path first
    # adds the post-normed block output. Bounded by the design margin 2^-18
    # (norm.h:53-63).
    rng = np.random.default_rng(9)
    n = 1152
    for trial in range(20):
        hidden = rng.normal(0, 3, n).astype(np.float32)
        out = rng.normal(0, 10, n).astype(np.float32)
        gain = (1 + 0.1 * rng.normal(0, 1, n)).astype(np.float32)
        pg = (1 + 0.1 * rng.normal(0, 1, n)).astype(np.float32)
        h2, normed = orc.norm_row(gain, hidden, out, pg)
        h, o = hidden.astype(np.float64), out.astype(np.float64)
        ry = 1 / np.sqrt(np.mean(o * o) + 1e-6)
        x = h + o * ry * pg
        assert np.max(np.abs(h2 - x) / (np.abs(h) + np.abs(o * ry * pg))) < 2.0 ** -18
        # the norm of the row the oracle holds (its rounding of X is checked above)
        x2 = h2.astype(np.float64)
        r = 1 / np.sqrt(np.mean(x2 * x2) + 1e-6)
        want = x2 * r * gain
        assert np.max(np.abs(normed - want) / np.abs(want)) < 2.0 ** -18
    # without the add, hidden is untouched
    h3, _ = orc.norm_row(gain, hidden)
    assert np.array_equal(bits(h3), bits(hidden))


@pytest.mark.parametrize("base", [1e4, 1e6])
def test_rope_turns_closed_form(base):
    # rope.cpp:95-106: turns_k = f32(base^(-2k/d) / (2 pi)) taken in f64.
    d = 256
    got = orc.rope_turns(base, d)
    want = np.array([np.float32(base ** (-2.0 * k / d) / (2 * math.pi)) for k in range(d // 2)])
    assert np.array_equal(bits(got), bits(want))


def test_rope_row_against_f64_and_the_cache_encoding():
    rng = np.random.default_rng(10)
    d, qh, slots, pos = 256, 4, 640, 700
    turns = orc.rope_turns(1e4, d)
    qg = (1 + 0.1 * rng.normal(0, 1, d)).astype(np.float32)
    kg = (1 + 0.1 * rng.normal(0, 1, d)).astype(np.float32)
    q = rng.normal(0, 2, qh * d).astype(np.float32)
    k = rng.normal(0, 2, d).astype(np.float32)
    v = rng.normal(0, 300, d).astype(np.float32)
    v[:3] = [1e5, -1e5, 65519.0]  # saturate, then round
    kc = np.zeros(slots * d, dtype=np.uint16)
    vc = np.zeros(slots * d, dtype=np.uint16)
    qo = q.copy()
    orc.lib().orc_rope_row(pos, slots, d, qh, 1, 1e-6, turns.ctypes.data, qg.ctypes.data,
                           kg.ctypes.data, qo.ctypes.data, k.ctypes.data, v.ctypes.data,
                           kc.ctypes.data, vc.ctypes.data)

    def rotate(x, g):
        x = x.astype(np.float64)
        y = x / np.sqrt(np.mean(x * x) + 1e-6) * g
        t = np.float32(pos) * turns.astype(np.float64)
        ang = 2 * math.pi * (t - np.round(t))
        c, s = np.cos(ang), np.sin(ang)
        a, b = y[:d // 2], y[d // 2:]
        return np.concatenate([a * c - b * s, a * s + b * c])

    for h in range(qh):
        want = rotate(q[h * d:(h + 1) * d], qg)
        assert np.max(np.abs(qo[h * d:(h + 1) * d] - want)) < 2.0 ** -16 * np.max(np.abs(want))
    slot = pos % slots
    k_want = rotate(k, kg)
    k_got = kc[slot * d:(slot + 1) * d].view(np.float16).astype(np.float64)
    assert np.max(np.abs(k_got - k_want) / np.maximum(np.abs(k_want), 1e-2)) < 2.0 ** -10
    assert np.array_equal(vc[slot * d:(slot + 1) * d],
                          np.clip(v, -65504, 65504).astype(np.float16).view(np.uint16))
    assert not kc[:slot * d].any() and not kc[(slot + 1) * d:].any()


@pytest.mark.parametrize("pos,window,slots", [(0, 512, 640), (700, 512, 640), (100, 64, 640),
                                              (1000, 4096, 4096), (63, 512, 640)])
def test_attention_against_f64_softmax(pos, window, slots):
    rng = np.random.default_rng(pos + window)
    d, qh = 256, 4
    kc = (rng.integers(-96, 97, slots * d) / 32.0).astype(np.float16)
    vc = (rng.integers(-96, 97, slots * d) / 32.0).astype(np.float16)
    q = rng.normal(0, 0.5, qh * d).astype(np.float32)
    scale_log2e = np.float32(0.0625 * 1.4426950408889634)
    out = np.empty(qh * d, dtype=np.float32)
    orc.lib().orc_attention_row(pos, window, slots, d, qh, 1, float(scale_log2e), q.ctypes.data,
                                kc.view(np.uint16).ctypes.data, vc.view(np.uint16).ctypes.data,
                                out.ctypes.data)
    keys = [j for j in range(max(0, pos - window + 1), pos + 1)]
    K = np.stack([kc[(j % slots) * d:(j % slots + 1) * d] for j in keys]).astype(np.float64)
    V = np.stack([vc[(j % slots) * d:(j % slots + 1) * d] for j in keys]).astype(np.float64)
    for h in range(qh):
        s = K @ (q[h * d:(h + 1) * d].astype(np.float64) * np.float64(scale_log2e))
        p = np.exp2(s - s.max())
        want = (p / p.sum()) @ V
        assert np.max(np.abs(out[h * d:(h + 1) * d] - want)) < 2.0 ** -14 * (1 + np.abs(V).max())


def test_norm_added_is_what_the_add_added():
    # The capture store's addition is the vector the norm adds: hidden after
    # equals hidden before plus it, each element one f32 add, and it is the
    # post-normed block output (f64 within the 2^-18 margin).
    rng = np.random.default_rng(19)
    n = 1152
    for trial in range(10):
        hidden = rng.normal(0, 3, n).astype(np.float32)
        out = rng.normal(0, 10, n).astype(np.float32)
        gain = (1 + 0.1 * rng.normal(0, 1, n)).astype(np.float32)
        pg = (1 + 0.1 * rng.normal(0, 1, n)).astype(np.float32)
        h = hidden.copy()
        normed = np.empty(n, np.float32)
        added = np.empty(n, np.float32)
        orc.lib().orc_norm_row_added(gain.ctypes.data, pg.ctypes.data, 1, 1, 1.0, 1e-6, n,
                                     h.ctypes.data, out.ctypes.data, normed.ctypes.data,
                                     added.ctypes.data)
        assert np.array_equal(bits(h), bits(hidden + added))
        h2, normed2 = orc.norm_row(gain, hidden, out, pg)
        assert np.array_equal(bits(h), bits(h2)) and np.array_equal(bits(normed), bits(normed2))
        o = out.astype(np.float64)
        want = o / np.sqrt(np.mean(o * o) + 1e-6) * pg
        assert np.max(np.abs(added - want) / (np.abs(want) + 1e-30)) < 2.0 ** -18


@pytest.mark.parametrize("pos,window,slots", [(700, 512, 640), (40, 512, 640), (300, 64, 640)])
def test_attention_scores_and_statistics(pos, window, slots):
    # The capture store's scores are the query's dots with the keys it reads
    # (log2 units), m their maximum and l the sum of exp2(s - m); the output
    # is orc_attention_row's, bit for bit; slots past the keys read stay.
    rng = np.random.default_rng(pos + slots)
    d, qh = 256, 4
    kc = (rng.integers(-96, 97, slots * d) / 32.0).astype(np.float16)
    vc = (rng.integers(-96, 97, slots * d) / 32.0).astype(np.float16)
    q = rng.normal(0, 0.5, qh * d).astype(np.float32)
    sc = np.float32(0.0625 * 1.4426950408889634)
    keys = window
    out, out2 = np.empty(qh * d, np.float32), np.empty(qh * d, np.float32)
    scores = np.full(qh * keys, -7.0, np.float32)
    stats = np.empty(2 * qh, np.float32)
    args = (pos, window, slots, d, qh, 1, float(sc), q.ctypes.data, kc.view(np.uint16).ctypes.data,
            vc.view(np.uint16).ctypes.data)
    orc.lib().orc_attention_row_scores(*args, out.ctypes.data, scores.ctypes.data, keys,
                                       stats.ctypes.data)
    orc.lib().orc_attention_row(*args, out2.ctypes.data)
    assert np.array_equal(bits(out), bits(out2))
    earliest = pos + 1 - min(pos + 1, keys)
    read = pos - earliest + 1
    K = np.stack([kc[(j % slots) * d:(j % slots + 1) * d] for j in range(earliest, pos + 1)])
    for h in range(qh):
        s = scores[h * keys:h * keys + read]
        want = K.astype(np.float64) @ (q[h * d:(h + 1) * d] * sc).astype(np.float64)
        assert np.max(np.abs(s - want)) < 2.0 ** -18 * (1 + np.abs(want).max())
        assert (scores[h * keys + read:(h + 1) * keys] == -7.0).all()
        assert stats[2 * h] == s.max()
        l64 = np.exp2(s.astype(np.float64) - np.float64(s.max())).sum()
        assert abs(stats[2 * h + 1] - l64) < 2.0 ** -18 * l64


def test_attention_ignores_keys_outside_the_window():
    # Keys at or before p - W, and slots not yet written, never count: make
    # them huge and the output must not move.
    rng = np.random.default_rng(12)
    d, qh, slots, window, pos = 256, 4, 640, 64, 300
    kc = (rng.integers(-96, 97, slots * d) / 32.0).astype(np.float16)
    vc = (rng.integers(-96, 97, slots * d) / 32.0).astype(np.float16)
    q = rng.normal(0, 0.5, qh * d).astype(np.float32)
    outs = []
    for poison in (False, True):
        k2, v2 = kc.copy(), vc.copy()
        if poison:
            for j in list(range(pos - window - 100, pos - window + 1)) + list(range(pos + 1, pos + 50)):
                k2[(j % slots) * d:(j % slots + 1) * d] = np.float16(300.0)
                v2[(j % slots) * d:(j % slots + 1) * d] = np.float16(6e4)
        out = np.empty(qh * d, dtype=np.float32)
        orc.lib().orc_attention_row(pos, window, slots, d, qh, 1, 0.09, q.ctypes.data,
                                    k2.view(np.uint16).ctypes.data,
                                    v2.view(np.uint16).ctypes.data, out.ctypes.data)
        outs.append(out)
    assert np.array_equal(bits(outs[0]), bits(outs[1]))


def test_gather_is_the_row_times_the_scale():
    rng = np.random.default_rng(13)
    vocab, width = 50, 1152
    table = q4_blocks(rng, vocab, width)
    scale = np.float32(math.sqrt(1152.0))
    for tok in (0, 17, 49):
        out = np.empty(width, dtype=np.float32)
        orc.lib().orc_gather_row(table.ctypes.data, width, tok, float(scale), out.ctypes.data)
        want = dequant(table, vocab, width)[tok].astype(np.float32) * scale
        assert np.array_equal(bits(out), bits(want))


# ---- edits -----------------------------------------------------------------------------

def edit_table(entries, layers):
    """The reference's table (edit.h:50-60): per layer [first, count], then
    [neuron, kind, value bits, first, end] sorted by (layer, neuron, first)."""
    entries = sorted(entries, key=lambda e: (e[0], e[1], e[4]))
    words = [0] * (2 * layers)
    body = []
    for l in range(layers):
        mine = [e for e in entries if e[0] == l]
        words[2 * l] = 2 * layers + len(body)
        words[2 * l + 1] = len(mine)
        for _, n, kind, value, first, end in mine:
            body += [n, kind, int(np.array([value], dtype=np.float32).view(np.uint32)[0]), first, end]
    return np.array(words + body, dtype=np.uint32)


def test_edit_row_contract():
    # edit_kernel_test.cpp:1-21: Set / Zero / Scale on the listed neurons in
    # the positions their range holds; other layers' edits and other neurons
    # untouched; Scale x 1 keeps a subnormal's bits.
    SET, SCALE, ZERO = 0, 1, 2
    width, layers = 200, 3
    entries = [(1, 5, SET, 2.5, 10, 20), (1, 6, SCALE, -3.0, 0, 0xFFFFFFFF),
               (1, 7, ZERO, 0.0, 15, 16), (1, 8, SCALE, 1.0, 0, 0xFFFFFFFF),
               (0, 5, SET, 99.0, 0, 0xFFFFFFFF), (1, 150, SET, -1.0, 12, 13),
               (1, 150, SET, -2.0, 13, 14)]
    table = edit_table(entries, layers)
    rng = np.random.default_rng(14)
    for position in (9, 10, 12, 13, 15, 19, 20):
        act = rng.normal(0, 1, width).astype(np.float32)
        act[8] = np.float32(1e-40)  # subnormal
        before = act.copy()
        orc.lib().orc_edit_row(table.ctypes.data, 1, position, width, act.ctypes.data)
        want = before.copy()
        if 10 <= position < 20:
            want[5] = 2.5
        want[6] = before[6] * np.float32(-3.0)
        if position == 15:
            want[7] = 0.0
        if position == 12:
            want[150] = -1.0
        if position == 13:
            want[150] = -2.0
        assert np.array_equal(bits(act), bits(want)), position


# ---- selection and the draw ------------------------------------------------------------

def order_key(b):
    b = np.where(b == 0x80000000, 0, b).astype(np.uint64)
    nan = ((b & 0x7F800000) == 0x7F800000) & ((b & 0x7FFFFF) != 0)
    key = np.where(b & 0x80000000, (~b) & 0xFFFFFFFF, b | 0x80000000)
    return np.where(nan, 0xFFFFFFFF, key)


@pytest.mark.parametrize("count", [64, 1000, 5000])
def test_topk_is_the_sorted_head_of_the_total_order(count):
    # topk.wgsl:57-61: larger key first (NaN largest, -0 as +0), ties by the
    # lower token; brute force by a stable sort.
    rng = np.random.default_rng(count)
    logits = np.round(rng.normal(0, 3, count)).astype(np.float32)
    logits[rng.choice(count, 10, replace=False)] = [np.nan, np.inf, -np.inf, -0.0, 0.0,
                                                   1e-45, -1e-45, 3e38, -3e38, np.nan]
    b, ids = orc.topk(logits)
    key = order_key(logits.view(np.uint32))
    order = np.lexsort((np.arange(count), -key.astype(np.float64)))[:64]
    assert np.array_equal(ids, order.astype(np.uint32))
    want_bits = logits.view(np.uint32)[order].copy()
    want_bits[np.isnan(logits[order])] = 0x7FC00000
    want_bits[want_bits == 0x80000000] = 0
    assert np.array_equal(b, want_bits)


def test_philox_known_answers():
    # Philox4x32-10 known-answer vectors (Salmon et al., Random123 kat_vectors).
    cases = [
        ([0, 0, 0, 0], [0, 0], [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]),
        ([0xFFFFFFFF] * 4, [0xFFFFFFFF] * 2, [0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]),
        ([0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344], [0xA4093822, 0x299F31D0],
         [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]),
    ]
    for counter, key, want in cases:
        assert list(orc.philox(counter, key)) == want


def test_mulhi_is_the_high_word_of_the_product():
    rng = np.random.default_rng(15)
    a = rng.integers(0, 2 ** 32, 20000, dtype=np.uint64)
    b = rng.integers(0, 2 ** 32, 20000, dtype=np.uint64)
    L = orc.lib()
    for x, y in list(zip(a, b)) + [(0xFFFFFFFF, 0xFFFFFFFF), (0, 5), (0x10000, 0x10000)]:
        assert L.orc_mulhi(int(x), int(y)) == (int(x) * int(y)) >> 32


def test_draw_greedy_and_the_uniform():
    # T = 0 takes the first candidate; u = (w >> 9) 2^-23 + 2^-24 with w the
    # first Philox word at counter (position + tokens, 0, 0, 0), key = seed.
    rng = np.random.default_rng(16)
    cand = np.sort(rng.normal(0, 2, 64).astype(np.float32))[::-1]
    ids = rng.permutation(1000)[:64].astype(np.uint32)
    for counter, seed in ((5, 0), (1000, 0x123456789ABC)):
        rec = orc.draw(bits(cand), ids, 1, 0.0, 1.0, 0.0, counter, seed)
        w = orc.philox([counter, 0, 0, 0], [seed & 0xFFFFFFFF, seed >> 32])[0]
        u = np.float32(np.float32(w >> 9) * np.float32(2.0 ** -23) + np.float32(2.0 ** -24))
        assert rec[0] == ids[0] and rec[1] == 0 and rec[2] == bits(u) and rec[3] == 0


def test_draw_inverse_transform_against_f64():
    # T > 0, no top-p / min-p: the chosen candidate is where the running sum
    # of exp((x_i - x_0) / T) first exceeds u times the total.
    rng = np.random.default_rng(17)
    for trial in range(200):
        cand = np.sort(rng.normal(0, 1, 64).astype(np.float32))[::-1]
        ids = np.arange(64, dtype=np.uint32)
        rec = orc.draw(bits(cand), ids, 64, 1.0, 1.0, 0.0, trial, 7)
        u = np.float64(np.array([rec[2]], dtype=np.uint32).view(np.float32)[0])
        w = np.exp(cand.astype(np.float64) - np.float64(cand[0]))
        run = np.cumsum(w)
        want = int(np.searchsorted(run, u * run[-1], side="right"))
        near = np.min(np.abs(run - u * run[-1])) < 1e-5 * run[-1]
        assert rec[0] == want or near


# ---- Q8_0 and Q4_1 (the pinned file's head and downs) ----------------------------

def _round_f32(v):
    """The f32 nearest the exact rational v, ties to even."""
    from fractions import Fraction
    a = np.float32(float(v))
    best = a
    for c in (np.nextafter(a, np.float32(-np.inf)), np.nextafter(a, np.float32(np.inf))):
        da, dc = abs(Fraction(float(best)) - v), abs(Fraction(float(c)) - v)
        if dc < da or (dc == da and (int(np.array(c).view(np.uint32)) & 1) == 0):
            best = c
    return best


def test_q8_0_exact_for_every_code_and_sampled_scale():
    # weight j = qs[j] d (q8_0.wgsl:12-24), exact in f32: compare with f64.
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    finite = h[np.isfinite(h.view(np.float16))]
    codes = np.arange(256, dtype=np.uint8)
    for s in finite[::53]:
        for half in range(8):
            block = np.empty(34, dtype=np.uint8)
            block[0:2] = np.array([s], dtype=np.uint16).view(np.uint8)
            block[2:] = codes[32 * half:32 * half + 32]
            w = orc.unpack_format(8, block)
            dv = np.float64(np.array([s], dtype=np.uint16).view(np.float16)[0])
            want = codes[32 * half:32 * half + 32].view(np.int8).astype(np.float64) * dv
            assert np.array_equal(w.astype(np.float64), want), hex(s)


def test_q4_1_rounds_once_for_every_code():
    # weight = q d + m (q4_1.wgsl:12-25): q d is exact, so the value is the
    # exact q d + m rounded once to f32.
    from fractions import Fraction
    rng = np.random.default_rng(13)
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    finite = h[np.isfinite(h.view(np.float16))]
    for _ in range(300):
        d_bits, m_bits = rng.choice(finite, 2)
        block = np.empty(20, dtype=np.uint8)
        block[0:2] = np.array([d_bits], dtype=np.uint16).view(np.uint8)
        block[2:4] = np.array([m_bits], dtype=np.uint16).view(np.uint8)
        block[4:] = (np.arange(16, dtype=np.uint8) | (np.arange(16, dtype=np.uint8)[::-1] << 4))
        w = orc.unpack_format(3, block)
        d = Fraction(float(np.array([d_bits], dtype=np.uint16).view(np.float16)[0]))
        m = Fraction(float(np.array([m_bits], dtype=np.uint16).view(np.float16)[0]))
        lo = np.arange(16)
        qs = np.concatenate([lo, lo[::-1]])
        want = np.array([_round_f32(int(q) * d + m) for q in qs], dtype=np.float32)
        assert np.array_equal(bits(w), bits(want)), (hex(d_bits), hex(m_bits))


def _blocks_exact(rng, fmt, rows, cols):
    """Blocks whose weights are small integers (d = 1, m small), so that
    every product and sum of a short row is exact in f32."""
    n = rows * cols // 32
    bb = {2: 18, 3: 20, 8: 34}[fmt]
    out = np.zeros((n, bb), dtype=np.uint8)
    out[:, 0:2] = np.array([0x3C00], dtype=np.uint16).view(np.uint8)  # d = 1
    if fmt == 3:
        m = rng.integers(-3, 4, n).astype(np.float16)
        out[:, 2:4] = m.view(np.uint8).reshape(n, 2)
        out[:, 4:] = rng.integers(0, 256, (n, 16), dtype=np.uint8)
    elif fmt == 8:
        out[:, 2:] = rng.integers(-20, 21, (n, 32)).astype(np.int8).view(np.uint8)
    else:
        out[:, 2:] = rng.integers(0, 256, (n, 16), dtype=np.uint8)
    return out.reshape(-1)


def _dequant_format(fmt, blocks, rows, cols):
    b = blocks.reshape(-1, {2: 18, 3: 20, 8: 34}[fmt])
    return np.stack([orc.unpack_format(fmt, blk) for blk in b]).reshape(rows, cols)


@pytest.mark.parametrize("fmt", [3, 8])
def test_gemv_format_exact_integers(fmt):
    rng = np.random.default_rng(fmt)
    rows, cols = 24, 256
    w = _blocks_exact(rng, fmt, rows, cols)
    x = rng.integers(-4, 5, cols).astype(np.float32)
    y = orc.gemv_format(fmt, w, rows, cols, x)
    want = _dequant_format(fmt, w, rows, cols).astype(np.float64) @ x.astype(np.float64)
    assert np.array_equal(y.astype(np.float64), want)
    # and the rows' blocks by an independent unpack of the layout
    b = w.reshape(rows, cols // 32, -1)
    if fmt == 8:
        q = b[:, :, 2:].view(np.int8).astype(np.float64).reshape(rows, cols)
        assert np.array_equal(q @ x.astype(np.float64), want)


def test_gemv_format_q4_0_is_gemv():
    rng = np.random.default_rng(4)
    rows, cols = 40, 1152
    w = q4_blocks(rng, rows, cols)
    x = rng.normal(0, 1, cols).astype(np.float32)
    assert np.array_equal(bits(orc.gemv_format(2, w, rows, cols, x)), bits(orc.gemv(w, rows, cols, x)))


@pytest.mark.parametrize("fmt", [2, 8])
def test_gather_format_is_row_times_scale(fmt):
    rng = np.random.default_rng(6 + fmt)
    rows, cols = 7, 128
    w = _blocks_exact(rng, fmt, rows, cols)
    w.reshape(-1, {2: 18, 8: 34}[fmt])[:, 0:2] = np.abs(rng.normal(0, 0.02, rows * cols // 32)).astype(
        np.float16).view(np.uint8).reshape(-1, 2)
    scale = np.float32(np.sqrt(np.float32(cols)))
    got = orc.gather_row_format(fmt, w, cols, 5, scale)
    want = (_dequant_format(fmt, w, rows, cols)[5].astype(np.float32) * scale).astype(np.float32)
    assert np.array_equal(bits(got), bits(want))
