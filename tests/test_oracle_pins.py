"""Pins the oracle's remaining functions with constructions whose answer is
fixed by exact arithmetic (no GPU):

- the norm's halving tree over 256 partial sums and its epsilon
  (norm.wgsl:75-86, 138-198);
- the QK-norm's halving tree over a head's 32 lanes (rope.wgsl:51-61);
- attention's order of addition inside a tile, across tiles and across
  chunks (attention.wgsl:135-163, 304-340);
- the draw's top-p and min-p prefixes against f64 (draw.wgsl:77-170);
- the model's composition (graph.cpp:290-470): closed-form special cases
  in which most matrices are zero, so that the logits reduce to a few
  already-pinned primitives in a known order.

Each construction is chosen so that a plausible slip fails it: another tree
shape (serial, adjacent pairs), a dropped or wrong epsilon, another fold
order, a block output added with the wrong gain or at the wrong norm.
"""
import numpy as np
import pytest

import _oracle as orc
import frizzle_amd as fz
from helpers import bits, dequant

F = np.float32


def _r_of(total, n, eps=1e-6):
    """inverseSqrt(total / n + eps) in f32, each operation rounded once, as
    the reference writes it (norm.wgsl:192, rope.wgsl)."""
    t = F(F(total) / F(n)) + F(eps)
    return F(F(1.0) / np.sqrt(F(t)))


# ---- the norm -------------------------------------------------------------------

def _norm(x, gain):
    h, normed = orc.norm_row(gain, x)
    return normed


def test_norm_tree_halves_the_256_partials():
    # Width 1,152: invocation i holds vec4s i and i + 256 (i < 32), each
    # summed by dot from zero, then partial[i] += partial[i + stride] for
    # stride 128, 64, ..., 1. Vec4 0 carries 4096^2 = 2^24 and every odd
    # vec4 below 256 a 1. The odd partials meet among themselves first (128
    # ones, exact) and join 2^24 at stride 1: 2^24 + 128. A serial sum
    # loses every 1 to rounding (2^24).
    n = 1152
    x = np.zeros(n, F)
    x[0] = 4096.0
    x[4 * np.arange(1, 256, 2)] = 1.0
    got = _norm(x, np.ones(n, F))
    want_r = _r_of(2.0 ** 24 + 128, n)
    assert bits(got[0]) == bits(F(4096.0) * want_r)
    assert bits(got[4]) == bits(want_r)
    # the construction tells the shapes apart
    assert _r_of(2.0 ** 24 + 128, n) != _r_of(2.0 ** 24, n)


def test_norm_tree_second_vec4_joins_its_own_invocation():
    # As above, plus a 1 in the second vec4 (i + 256) of every odd
    # invocation below 32: those invocations hold 2 before the tree, so the
    # total is 2^24 + 144. A norm that read one vec4 an invocation gives
    # 2^24 + 128; one that gave vec4 i + 256 to invocation i + 256 mod 256's
    # neighbour would still meet 2^24 first on the even side.
    n = 1152
    x = np.zeros(n, F)
    x[0] = 4096.0
    x[4 * np.arange(1, 256, 2)] = 1.0
    x[4 * (256 + np.arange(1, 32, 2))] = 1.0
    got = _norm(x, np.ones(n, F))
    assert bits(got[0]) == bits(F(4096.0) * _r_of(2.0 ** 24 + 144, n))
    assert _r_of(2.0 ** 24 + 144, n) != _r_of(2.0 ** 24 + 128, n)


@pytest.mark.parametrize("scale", [1e-3, 3e-4, 1e-2])
def test_norm_epsilon_is_one_millionth(scale):
    # Rows whose mean square is near epsilon: with x = s everywhere, normed
    # = s / sqrt(s^2 + 1e-6) g. Dropping epsilon gives g; 1e-5 gives a
    # different value well past the bound.
    n = 1152
    rng = np.random.default_rng(3)
    x = np.full(n, scale, F)
    g = (1 + 0.1 * rng.normal(0, 1, n)).astype(F)
    got = _norm(x, g).astype(np.float64)
    s = np.float64(F(scale))
    want = s / np.sqrt(s * s + np.float64(F(1e-6))) * g.astype(np.float64)
    assert np.max(np.abs(got - want) / np.abs(want)) < 2.0 ** -20
    for wrong in (0.0, 1e-5):
        alt = s / np.sqrt(s * s + wrong) * g.astype(np.float64)
        assert np.max(np.abs(alt - want) / np.abs(want)) > 1e-3


def test_post_norm_add_uses_the_post_gain_then_adds():
    # hidden' = hidden + ((y r_y) post_gain) 1: with y = c e_k, r_y is
    # 1 / sqrt(c^2 / n + eps); the added element is (c r_y) pg_k, and
    # every other element of hidden is unchanged.
    n = 1152
    rng = np.random.default_rng(4)
    hidden = rng.normal(0, 1, n).astype(F)
    y = np.zeros(n, F)
    y[7] = 48.0  # 48^2 = 2304 = 2n: mean square 2, exact
    pg = (1 + 0.1 * rng.normal(0, 1, n)).astype(F)
    g = np.ones(n, F)
    h2, _ = orc.norm_row(g, hidden, y, pg)
    r_y = _r_of(2304.0, n)
    added = F(F(F(48.0) * r_y) * pg[7]) * F(1.0)
    assert bits(h2[7]) == bits(F(hidden[7] + added))
    others = np.arange(n) != 7
    assert np.array_equal(bits(h2[others]), bits(hidden[others] + F(0.0)))


# ---- the QK-norm ----------------------------------------------------------------

def test_qk_norm_tree_halves_a_heads_32_lanes():
    # A head's lane i holds dimensions 4i..4i+3 and 4i+128..4i+131; its 32
    # lane sums meet in a halving tree (stride 16, 8, 4, 2, 1). Dimension 0
    # carries 4096 (2^24 squared) and dimension 4i a 1 for every odd lane i:
    # the odd lanes meet among themselves first (16 ones, exact) and join
    # 2^24 last: 2^24 + 16. A serial sum gives 2^24; lanes of 8 adjacent
    # dimensions give 2^24 + 14. At position 0 the rotation is the identity
    # (cos 0 = 1, sin 0 = 0), so the query row out is (x r) g.
    L = orc.lib()
    assert L.orc_cos(0.0) == 1.0 and L.orc_sin(0.0) == 0.0
    d, qh, slots = 256, 4, 64
    q = np.zeros(qh * d, F)
    for h in range(qh):
        q[h * d] = 4096.0
        for i in range(1, 32, 2):
            q[h * d + 4 * i] = 1.0
    k = np.zeros(d, F)
    k[3] = 2.0
    v = np.zeros(d, F)
    qg = np.ones(d, F)
    kg = np.ones(d, F)
    turns = orc.rope_turns(1e4, d)
    kc = np.zeros(slots * d, np.uint16)
    vc = np.zeros(slots * d, np.uint16)
    qo = q.copy()
    L.orc_rope_row(0, slots, d, qh, 1, 1e-6, turns.ctypes.data, qg.ctypes.data, kg.ctypes.data,
                   qo.ctypes.data, k.ctypes.data, v.ctypes.data, kc.ctypes.data, vc.ctypes.data)
    r = _r_of(2.0 ** 24 + 16, d)
    for h in range(qh):
        assert bits(qo[h * d]) == bits(F(4096.0) * r)
        assert bits(qo[h * d + 4]) == bits(r)
    assert _r_of(2.0 ** 24 + 16, d) != _r_of(2.0 ** 24, d)
    assert _r_of(2.0 ** 24 + 16, d) != _r_of(2.0 ** 24 + 14, d)


def test_qk_norm_epsilon_on_a_small_key():
    # A key of one element c: normed = c / sqrt(c^2 / 256 + 1e-6); at c =
    # 0.016 the epsilon is 1% of the mean square. The key is packed to F16.
    L = orc.lib()
    d, slots = 256, 64
    q = np.zeros(4 * d, F)
    k = np.zeros(d, F)
    k[5] = 0.016
    v = np.zeros(d, F)
    ones = np.ones(d, F)
    turns = orc.rope_turns(1e4, d)
    kc = np.zeros(slots * d, np.uint16)
    vc = np.zeros(slots * d, np.uint16)
    L.orc_rope_row(0, slots, d, 4, 1, 1e-6, turns.ctypes.data, ones.ctypes.data,
                   ones.ctypes.data, q.ctypes.data, k.ctypes.data, v.ctypes.data,
                   kc.ctypes.data, vc.ctypes.data)
    c = np.float64(F(0.016))
    want = c / np.sqrt(c * c / 256 + np.float64(F(1e-6)))
    got = np.float64(kc[5:6].view(np.float16)[0])
    assert abs(got - want) <= 2.0 ** -11 * abs(want)
    assert abs(c / np.sqrt(c * c / 256) - want) > 2.0 ** -7 * abs(want)


# ---- attention's order of addition ------------------------------------------------

def _attend(pos, window, slots, kc, vc, q, scale_log2e=1.0):
    out = np.empty(q.size, F)
    orc.lib().orc_attention_row(pos, window, slots, 256, 4, 1, float(scale_log2e),
                                q.ctypes.data, kc.view(np.uint16).ctypes.data,
                                vc.view(np.uint16).ctypes.data, out.ctypes.data)
    return out


def _unit_query():
    q = np.zeros(4 * 256, F)
    q[0::256] = 1.0  # every head reads dimension 0 of the keys
    return q


def test_attention_folds_chunks_in_chunk_order():
    # Every score 0, so every weight is 1 and l counts the keys (256, four
    # chunks of 64). Dimension 0 of the values: 32 in chunk 0 (its state
    # 2048), 2^-19 in chunks 1 and 2 (2^-13 each: half an ulp of 2048), 0 in
    # chunk 3. Folding in chunk order rounds 2048 + 2^-13 to 2048 twice; any
    # order that meets chunks 1 and 2 first keeps 2^-12. out = o / 256.
    d, slots, pos = 256, 512, 255
    kc = np.zeros(slots * d, np.float16)
    vc = np.zeros(slots * d, np.float16)
    for j in range(256):
        vc[j * d] = 32.0 if j < 64 else (2.0 ** -19 if j < 192 else 0.0)
    out = _attend(pos, 1024, slots, kc, vc, _unit_query())
    assert np.all(out[0::256] == F(8.0)), out[0::256]
    assert F((2048.0 + 2.0 ** -12) / 256) != F(8.0)


def test_attention_tile_adds_each_key_into_the_running_output():
    # One chunk (position 63): key 0's value 2048, keys 8 and 9 (the second
    # tile) 2^-13 each, every score 0. O = O a + p v key by key: 2048 +
    # 2^-13 rounds to 2048 twice. A tile that summed its own keys first and
    # then added would keep 2^-12.
    d, slots, pos = 256, 128, 63
    kc = np.zeros(slots * d, np.float16)
    vc = np.zeros(slots * d, np.float16)
    vc[0] = 2048.0
    vc[8 * d] = 2.0 ** -13
    vc[9 * d] = 2.0 ** -13
    out = _attend(pos, 512, slots, kc, vc, _unit_query())
    assert np.all(out[0::256] == F(32.0)), out[0::256]


def test_attention_rescales_by_the_side_without_the_maximum():
    # Scores are k[0] exactly (q = e_0, scale 1): chunk 0's keys score 0,
    # chunk 1's score 3. Chunk 0's state (l = 64, o = 64 v) is scaled by
    # exp2(0 - 3) = 1/8 and chunk 1's kept: l = 8 + 64, o = 8 v0 + 64 v1.
    d, slots, pos = 256, 256, 127
    kc = np.zeros(slots * d, np.float16)
    vc = np.zeros(slots * d, np.float16)
    for j in range(128):
        kc[j * d] = 0.0 if j < 64 else 3.0
        vc[j * d] = 1.0 if j < 64 else 2.0
    out = _attend(pos, 512, slots, kc, vc, _unit_query())
    assert np.all(out[0::256] == F(F(8.0 + 128.0) / F(72.0)))
    # the scores within a chunk rise tile by tile: chunk 0's tiles score 0,
    # 1, ..., 7 (a rescale at every tile); the result is exp2-exact sums.
    kc[:] = 0
    vc[:] = 0
    for j in range(64):
        kc[j * d] = float(j // 8)
        vc[j * d] = 1.0
    out = _attend(63, 512, slots, kc, vc, _unit_query())
    assert np.all(out[0::256] == F(1.0))


def test_attention_window_starts_at_the_earliest_keys_tile():
    # Window 100 at position 199: keys 100..199 are read. A key just before
    # the window (99), and one at the window's first position (100), tell a
    # mask off by one either way.
    d, slots, pos = 256, 512, 199
    kc = np.zeros(slots * d, np.float16)
    vc = np.zeros(slots * d, np.float16)
    vc[99 * d] = 1000.0
    vc[100 * d] = 100.0
    out = _attend(pos, 100, slots, kc, vc, _unit_query())
    assert np.all(out[0::256] == F(F(100.0) / F(100.0)))


# ---- the draw's top-p and min-p ---------------------------------------------------

def _draw_f64(cand, top_k, temperature, top_p, min_p, u):
    """draw.wgsl:77-170 in f64: top-p keeps the shortest prefix whose
    temperature-1 softmax reaches top_p; min-p keeps the prefix above
    first + ln(min_p); the inverse transform picks the first running sum of
    exp((x - x0) / T) above u times the survivors' total. Returns the
    chosen index and whether any comparison was within rounding of its
    boundary."""
    x = cand[:min(top_k, cand.size)].astype(np.float64)
    k = x.size
    near = False
    kept = k
    if top_p < 1.0:
        w = np.exp(x - x[0])
        c = np.cumsum(w / w.sum())
        hit = np.nonzero(c >= top_p)[0]
        near |= bool(np.any(np.abs(c - top_p) < 1e-5))
        if hit.size:
            kept = int(hit[0]) + 1
    survivors = 1
    thr = x[0] + np.log(np.float64(F(min_p))) if min_p > 0 else -np.inf
    if min_p > 0:
        near |= bool(np.any(np.abs(x[:kept] - thr) < 1e-5 * (1 + abs(thr))))
    while survivors < kept and (min_p == 0 or x[survivors] >= thr):
        survivors += 1
    if temperature <= 0:
        return 0, near
    t = np.exp((x[:survivors] - x[0]) / np.float64(F(temperature)))
    run = np.cumsum(t)
    goal = u * run[-1]
    near |= bool(np.any(np.abs(run - goal) < 1e-5 * run[-1]))
    above = np.nonzero(run > goal)[0]
    return (int(above[0]) if above.size else survivors - 1), near


@pytest.mark.parametrize("top_p,min_p,temperature,top_k", [
    (0.9, 0.0, 1.0, 64), (0.5, 0.0, 0.7, 64), (1.0, 0.05, 1.0, 64), (1.0, 0.3, 1.3, 40),
    (0.95, 0.05, 0.8, 40), (0.3, 0.2, 2.0, 64)])
def test_draw_top_p_and_min_p_against_f64(top_p, min_p, temperature, top_k):
    rng = np.random.default_rng(int(top_p * 100 + min_p * 1000 + top_k))
    checked = 0
    for trial in range(300):
        spread = rng.choice([0.3, 1.0, 3.0])
        cand = np.sort(rng.normal(0, spread, 64).astype(F))[::-1]
        ids = rng.permutation(5000)[:64].astype(np.uint32)
        rec = orc.draw(bits(cand), ids, top_k, temperature, top_p, min_p, 100 + trial, 0xABCDEF)
        u = np.float64(np.array([rec[2]], np.uint32).view(F)[0])
        want, near = _draw_f64(cand, top_k, temperature, top_p, min_p, u)
        if near:
            continue
        checked += 1
        assert rec[0] == ids[want], (trial, rec[0], ids[want])
        assert rec[1] == 0
    assert checked > 250


def test_draw_top_p_keeps_at_least_the_first():
    # A top_p below the first candidate's share keeps it alone: the draw is
    # the first candidate whatever u is.
    cand = np.array([5.0] + [0.0] * 63, F)
    ids = np.arange(64, dtype=np.uint32) + 7
    for counter in range(50):
        rec = orc.draw(bits(cand), ids, 64, 1.0, 0.01, 0.0, counter, 3)
        assert rec[0] == 7


def test_draw_top_p_prefix_ends_where_the_sum_reaches_top_p():
    # Two equal candidates, the rest -inf (weight 0): the softmax is exactly
    # (1/2, 1/2, 0, ...), so the cumulative sum meets top_p = 1/2 at the
    # first candidate and the prefix is that one alone ("reaching", >=).
    # With top_p just above 1/2 both are kept and both get drawn.
    cand = np.array([1.5, 1.5] + [-np.inf] * 62, F)
    ids = np.arange(64, dtype=np.uint32) + 100
    at_half = {int(orc.draw(bits(cand), ids, 64, 1.0, 0.5, 0.0, c, 9)[0]) for c in range(64)}
    above = {int(orc.draw(bits(cand), ids, 64, 1.0, 0.5001, 0.0, c, 9)[0]) for c in range(64)}
    assert at_half == {100}
    assert above == {100, 101}


def test_draw_failed_on_a_non_finite_first():
    ids = np.arange(64, dtype=np.uint32)
    for first in (np.inf, np.nan):
        cand = np.array([first] + [0.0] * 63, F)
        rec = orc.draw(bits(cand), ids, 64, 1.0, 0.9, 0.05, 5, 1)
        assert rec[0] == 0 and rec[1] == 1


# ---- the model's composition --------------------------------------------------------

ROLES = ["q", "k", "v", "o", "gate", "up", "down", "attn_norm", "q_norm", "k_norm",
         "post_attn_norm", "ffn_norm", "post_ffn_norm"]
MATRICES = ("q", "k", "v", "o", "gate", "up", "down")


def _cfg():
    return fz.gemma3_1b_config(layers=2, vocab=512, window=64, pattern=2, context=512,
                               local_slots=640)


def _tensors(cfg, seed, live=()):
    """Synthetic tensors with every matrix's scales zeroed except those in
    `live` ((layer, role) pairs): a zero matrix's product is exactly zero."""
    t = {(l, r): fz.synth_tensor(cfg, seed, l, r) for l in range(cfg.layers) for r in ROLES}
    t[(-1, "embedding")] = fz.synth_tensor(cfg, seed, -1, "embedding")
    t[(-1, "output_norm")] = fz.synth_tensor(cfg, seed, -1, "output_norm")
    for l in range(cfg.layers):
        for r in MATRICES:
            if (l, r) not in live:
                b = t[(l, r)].reshape(-1, 18).copy()
                b[:, 0:2] = 0
                t[(l, r)] = b.reshape(-1)
    return t


def _embed(cfg, t, token):
    row = dequant(t[(-1, "embedding")], cfg.vocab, cfg.hidden)[token].astype(F)
    return F(row * F(np.sqrt(F(cfg.hidden))))


def _head(cfg, t, hidden, pending_output=None, pending_gain=None):
    """The final norm (adding the last block's post-normed output) and the
    tied head, from pinned primitives."""
    g = t[(-1, "output_norm")]
    if pending_gain is None:
        _, normed = orc.norm_row(g, hidden)
    else:
        _, normed = orc.norm_row(g, hidden, pending_output, pending_gain)
    return orc.gemv(t[(-1, "embedding")], cfg.vocab, cfg.hidden, normed)


def test_model_with_zero_blocks_is_the_head_of_the_scaled_embedding():
    # Every layer's matrices zero: the blocks add nothing, so the residual
    # stays the embedding row times sqrt(1152) (in f32) and the logits are
    # the head of its final norm. Layer 0's residual is that row exactly.
    cfg = _cfg()
    t = _tensors(cfg, 51)
    m = orc.OracleModel(cfg.as_dict(), t)
    m.set_edits(np.zeros(2 * cfg.layers, np.uint32))
    for p, tok in enumerate([3, 500, 77]):
        got = m.token(tok, p)
        x = _embed(cfg, t, tok)
        assert np.array_equal(bits(m.residuals()[0]), bits(x))
        assert np.array_equal(bits(m.residuals()[1]), bits(x))
        assert np.array_equal(bits(got), bits(_head(cfg, t, x, np.zeros(cfg.hidden, F),
                                                    t[(1, "post_ffn_norm")])))
    m.close()


def _attention_block(cfg, t, x, layer, values):
    """One layer with only V and O live: Q and K are zero, so every score is
    0 and attention averages the F16 values read; O of that goes through the
    post-attention norm into the residual at the feed-forward norm."""
    avg = values[0].astype(F)
    if len(values) == 2:
        avg = F(F(values[0] + values[1]) / F(2.0))
    attn = np.tile(avg, cfg.query_heads)
    o = orc.gemv(t[(layer, "o")], cfg.hidden, cfg.query_heads * cfg.head_dim, attn)
    h1, _ = orc.norm_row(t[(layer, "ffn_norm")], x, o, t[(layer, "post_attn_norm")])
    return h1


def test_model_attention_block_plumbing():
    # Layer 0 has V and O, everything else is zero. At position 0 attention
    # returns the one value (its F16 rounding); at position 1 the mean of
    # two. The block's output, post-normed with post_attn_norm, joins the
    # residual at the feed-forward norm; layer 1 and the MLPs add nothing.
    cfg = _cfg()
    t = _tensors(cfg, 52, live={(0, "v"), (0, "o")})
    m = orc.OracleModel(cfg.as_dict(), t)
    m.set_edits(np.zeros(2 * cfg.layers, np.uint32))
    values = []
    for p, tok in enumerate([11, 400]):
        got = m.token(tok, p)
        x = _embed(cfg, t, tok)
        _, n0 = orc.norm_row(t[(0, "attn_norm")], x)
        v = orc.gemv(t[(0, "v")], cfg.head_dim, cfg.hidden, n0)
        values.append(np.clip(v, -65504, 65504).astype(np.float16).astype(F))
        h1 = _attention_block(cfg, t, x, 0, values)
        assert np.array_equal(bits(m.residuals()[1]), bits(h1))
        want = _head(cfg, t, h1, np.zeros(cfg.hidden, F), t[(1, "post_ffn_norm")])
        assert np.array_equal(bits(got), bits(want)), p
    m.close()


@pytest.mark.parametrize("layer", [0, 1])
def test_model_pin_reaches_the_residual_through_down(layer):
    # Only `layer`'s down is live; gate and up are zero, so the activation
    # is gelu(0) * 0 = 0 but for one pinned neuron. down of that one-hot row
    # is a column times the value; post-normed with that layer's
    # post_ffn_norm it joins the residual at the next norm: the next layer's
    # attention norm, or the final norm after the last layer.
    cfg = _cfg()
    t = _tensors(cfg, 53, live={(layer, "down")})
    m = orc.OracleModel(cfg.as_dict(), t)
    neuron, value = 4321, -7.25
    table = fz.edit_table([fz.Edit(layer, neuron, fz.EditKind.SET, value)], cfg.layers, 0)
    m.set_edits(table)
    tok = 99
    got = m.token(tok, 0)
    x = _embed(cfg, t, tok)
    act = np.zeros(cfg.ffn, F)
    act[neuron] = value
    down = orc.gemv(t[(layer, "down")], cfg.hidden, cfg.ffn, act)
    if layer == 0:
        h1, _ = orc.norm_row(t[(1, "attn_norm")], x, down, t[(0, "post_ffn_norm")])
        assert np.array_equal(bits(m.residuals()[1]), bits(h1))
        want = _head(cfg, t, h1, np.zeros(cfg.hidden, F), t[(1, "post_ffn_norm")])
    else:
        assert np.array_equal(bits(m.residuals()[1]), bits(x))
        want = _head(cfg, t, x, down, t[(1, "post_ffn_norm")])
    assert np.array_equal(bits(got), bits(want))
    # and no pin, no change: the zero activation leaves the embedding's head
    m2 = orc.OracleModel(cfg.as_dict(), t)
    m2.set_edits(np.zeros(2 * cfg.layers, np.uint32))
    base = m2.token(tok, 0)
    assert np.array_equal(bits(base), bits(_head(cfg, t, x, np.zeros(cfg.hidden, F),
                                                 t[(1, "post_ffn_norm")])))
    m.close()
    m2.close()


# ---- the prefill block ----------------------------------------------------------------

@pytest.mark.parametrize("window,slots,pattern,blocks", [
    (64, 640, 3, [37, 63, 100]),     # a ring of 640 wrapped by the third block
    (512, 1024, 2, [300, 212, 40]),  # the real window, a global layer each second
])
def test_model_block_is_token_by_token(window, slots, pattern, blocks):
    # A prefill block runs each row through the same arithmetic as a token
    # alone: the last row's logits, every layer's caches and the residuals
    # equal orc_model_token's run over the same positions, bit for bit,
    # with a pin acting on some rows.
    cfg = fz.gemma3_1b_config(layers=3, vocab=512, window=window, pattern=pattern,
                              context=1024, local_slots=slots)
    t = _tensors(cfg, 61, live={(l, r) for l in range(3) for r in MATRICES})
    table = fz.edit_table([fz.Edit(1, 17, fz.EditKind.SET, 3.5, 0, 0xFFFFFFFF),
                           fz.Edit(2, 900, fz.EditKind.SCALE, -2.0, 50, 120)], cfg.layers, 0)
    a = orc.OracleModel(cfg.as_dict(), t)
    b = orc.OracleModel(cfg.as_dict(), t)
    a.set_edits(table)
    b.set_edits(table)
    ids = np.random.default_rng(62).integers(0, cfg.vocab, sum(blocks)).astype(np.uint32)
    at = 0
    for n in blocks:
        got = a.block(ids[at:at + n], at)
        for p in range(at, at + n):
            want = b.token(int(ids[p]), p, want_logits=(p == at + n - 1))
        assert np.array_equal(bits(got), bits(want)), (at, n)
        assert np.array_equal(bits(a.residuals()), bits(b.residuals()))
        for l in range(cfg.layers):
            assert np.array_equal(a.key_cache(l), b.key_cache(l)), l
            assert np.array_equal(a.value_cache(l), b.value_cache(l)), l
        at += n
    a.close()
    b.close()


# ---- which layers are global, their windows and rope bases ----------------------------
#
# gemma3.cpp:79-85: layer l attends to the whole context, with rope base 1e6,
# when l % pattern == pattern - 1; every other layer attends to the last
# `window` keys with base 1e4. The cases below recompute a layer's attention
# in f64 from already pinned primitives (the product, the norm, F16
# rounding) and the closed forms of QK-norm, rope and softmax, and require
# the oracle to agree within a tolerance far below what the other window or
# base would change.

def _f16(x):
    return np.clip(np.asarray(x, np.float64), -65504, 65504).astype(np.float16).astype(np.float64)


def _qk_norm_rope(x, gain, position, base, eps=1e-6):
    """One head's QK-norm and rope in f64: pairs (k, k + d/2) turned by
    position * base^(-2k/d)."""
    x = np.asarray(x, np.float64)
    d = x.size
    y = x / np.sqrt(np.mean(x * x) + eps) * np.asarray(gain, np.float64)
    ang = position * np.power(float(base), -2.0 * np.arange(d // 2) / d)
    c, s = np.cos(ang), np.sin(ang)
    a, b = y[:d // 2], y[d // 2:]
    return np.concatenate([a * c - b * s, a * s + b * c])


def _attention_f64(cfg, t, layer, xs, position, base, window):
    """Layer `layer`'s attention output (before O) at `position`, in f64,
    from the residuals `xs[j]` entering it at positions 0..position: the
    keys read are j in (position - window, position]."""
    d, H = cfg.head_dim, cfg.query_heads
    qs, ks, vs = [], [], []
    for j in range(position + 1):
        _, n = orc.norm_row(t[(layer, "attn_norm")], xs[j])
        q = orc.gemv(t[(layer, "q")], H * d, cfg.hidden, n)
        k = orc.gemv(t[(layer, "k")], d, cfg.hidden, n)
        v = orc.gemv(t[(layer, "v")], d, cfg.hidden, n)
        ks.append(_f16(_qk_norm_rope(k, t[(layer, "k_norm")], j, base)))
        vs.append(_f16(v))
        qs.append(q)
    lo = max(0, position - window + 1)
    K, V = np.array(ks[lo:]), np.array(vs[lo:])
    out = []
    for h in range(H):
        q = _qk_norm_rope(qs[position][h * d:(h + 1) * d], t[(layer, "q_norm")], position, base)
        s = K @ q / 16.0
        w = np.exp(s - s.max())
        out.append((w / w.sum()) @ V)
    return np.concatenate(out).astype(F)


def _block_residual(cfg, t, layer, x, attn):
    """The residual after `layer`'s attention block: O of `attn`,
    post-normed, added at the feed-forward norm."""
    o = orc.gemv(t[(layer, "o")], cfg.hidden, cfg.query_heads * cfg.head_dim, attn)
    h, _ = orc.norm_row(t[(layer, "ffn_norm")], x, o, t[(layer, "post_attn_norm")])
    return h


def _close(a, b):
    return float(np.max(np.abs(a.astype(np.float64) - b)) / np.max(np.abs(b)))


def test_model_local_window_and_global_context():
    # Pattern 2: layer 0 slides over 64 keys, layer 1 (l % 2 == 1) reads the
    # whole context. V and O live in both, Q and K zero, so each attention
    # averages the F16 values it reads. At position 100 the local layer must
    # average the last 64 values and the global layer all 101.
    cfg = _cfg()
    t = _tensors(cfg, 54, live={(0, "v"), (0, "o"), (1, "v"), (1, "o")})
    # the last block's output seen through the logits, not hidden under the
    # residual's own embedding row
    t[(1, "post_attn_norm")] = (t[(1, "post_attn_norm")] * F(32.0)).astype(F)
    m = orc.OracleModel(cfg.as_dict(), t)
    m.set_edits(np.zeros(2 * cfg.layers, np.uint32))
    ids = np.random.default_rng(55).integers(0, cfg.vocab, 101)
    xs, h1s = [], []
    for p, tok in enumerate(ids):
        got = m.token(int(tok), p)
        xs.append(_embed(cfg, t, int(tok)))
        h1s.append(m.residuals()[1])
    P = 100

    def layer0(window):
        return _block_residual(cfg, t, 0, xs[P], _attention_f64(cfg, t, 0, xs, P, 1e4, window))

    want, other = layer0(64), layer0(101)
    assert _close(h1s[P], want) < 1e-5
    assert _close(other, want) > 1e-2  # the window is visible
    # the global layer over the oracle's own residuals entering it

    def logits(window):
        h2 = _block_residual(cfg, t, 1, h1s[P], _attention_f64(cfg, t, 1, h1s, P, 1e6, window))
        return _head(cfg, t, h2, np.zeros(cfg.hidden, F), t[(1, "post_ffn_norm")])

    want, other = logits(101), logits(64)
    assert _close(got, want) < 1e-4
    assert _close(other, want) > 1e-2
    m.close()


@pytest.mark.parametrize("layer,base,wrong", [(0, 1e4, 1e6), (1, 1e6, 1e4)])
def test_model_rope_base_by_layer(layer, base, wrong):
    # Only `layer`'s Q, K, V and O are live (every score depends on the
    # positions through rope): the local layer turns by base 1e4, the global
    # one by 1e6, and the other base moves the output far past the
    # tolerance.
    cfg = _cfg()
    t = _tensors(cfg, 56, live={(layer, r) for r in ("q", "k", "v", "o")})
    t[(1, "post_attn_norm")] = (t[(1, "post_attn_norm")] * F(32.0)).astype(F)
    m = orc.OracleModel(cfg.as_dict(), t)
    m.set_edits(np.zeros(2 * cfg.layers, np.uint32))
    ids = np.random.default_rng(57).integers(0, cfg.vocab, 41)
    xs = []
    for p, tok in enumerate(ids):
        got = m.token(int(tok), p)
        xs.append(_embed(cfg, t, int(tok)))
    P = 40
    if layer == 0:
        res = m.residuals()[1]

        def check(b):
            return _block_residual(cfg, t, 0, xs[P], _attention_f64(cfg, t, 0, xs, P, b, 64))
    else:
        res = got

        def check(b):
            h2 = _block_residual(cfg, t, 1, xs[P], _attention_f64(cfg, t, 1, xs, P, b, 512))
            return _head(cfg, t, h2, np.zeros(cfg.hidden, F), t[(1, "post_ffn_norm")])
    want = check(base)
    assert _close(res, want) < 1e-4
    assert _close(check(wrong), want) > 1e-2
    m.close()
