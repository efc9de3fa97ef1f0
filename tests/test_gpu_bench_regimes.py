"""The configurations the benchmark times, at their real batch, length and
context, against the oracle bit for bit:

- the steered batch: an original and 15 steered variants of one prompt past
  the 512-key window, each pinning 1 to 32 seeded neurons to values in
  [-20, 20], drawn at temperature 1 from one seed, decoded as one batch of
  16 rows; every variant's tokens and the residual entering every layer at
  every step;
- the north star's 256 steps on the full Gemma-3-1B shape, greedy
  unsteered and with 8 pins, and drawn at temperature 1 with those pins;
- a global layer past 4,096 keys inside the model: a 4,160-token prompt in
  512-token steps, then decode, so the global layer folds 66 and more
  chunks with its fold kernel before the O product.
"""
import numpy as np
import pytest

import _oracle as orc
import frizzle_amd as fz
from helpers import assert_same_bits
from test_gpu_model import ROLES, placed

pytestmark = pytest.mark.gpu


def wandering_pair(device, cfg, seed):
    """build_pair's weights with the blocks' post-norm gains 32 times
    larger: a random model's residual is otherwise dominated by its input
    token's own embedding row, so that its tied head echoes the input, and
    neither sampling nor pins move the reply."""
    t = {(l, r): fz.synth_tensor(cfg, seed, l, r) for l in range(cfg.layers) for r in ROLES}
    t[(-1, "embedding")] = fz.synth_tensor(cfg, seed, -1, "embedding")
    t[(-1, "output_norm")] = fz.synth_tensor(cfg, seed, -1, "output_norm")
    for l in range(cfg.layers):
        for r in ("post_attn_norm", "post_ffn_norm"):
            t[(l, r)] = (t[(l, r)] * np.float32(32.0)).astype(np.float32)
    model = fz.Model(device, cfg)
    for (l, r), a in t.items():
        model.set_tensor(l, r, a)
    return model, orc.OracleModel(cfg.as_dict(), t)


def pinned_variants(cfg, rng, count, lo=-20.0, hi=20.0, most=32):
    """The original (no edits) and count - 1 variants, each setting 1 to
    `most` seeded neurons of seeded layers to seeded values in [lo, hi] for
    the whole reply."""
    out = [[]]
    for _ in range(1, count):
        n = int(rng.integers(1, most + 1))
        edits = {}
        while len(edits) < n:
            layer, neuron = int(rng.integers(0, cfg.layers)), int(rng.integers(0, cfg.ffn))
            edits[(layer, neuron)] = fz.Edit(layer, neuron, fz.EditKind.SET,
                                             float(rng.uniform(lo, hi)))
        out.append(list(edits.values()))
    return out


def test_sixteen_steered_variants_sampled_with_residuals(device):
    # The steered batch's regime on three layers (the third global): window
    # 512 over a ring of 1,024 slots, a 1,030-token prompt (prefill steps of
    # 512, 512 and 5 tokens, then every variant from the prompt's last
    # token), 16 rows a variants step. Each variant is the oracle's reply to
    # the prompt under its own pins, drawing from the same seed.
    cfg = fz.gemma3_1b_config(layers=3, vocab=4096, window=512, pattern=3, context=2048,
                              local_slots=1024)
    model, oracle = wandering_pair(device, cfg, seed=71)
    rng = np.random.default_rng(72)
    prompt = rng.integers(0, cfg.vocab, 1030).astype(np.uint32)
    variants = pinned_variants(cfg, rng, 16)
    assert max(len(v) for v in variants) > 16
    samp = fz.sampling(temperature=1.0, top_k=64, top_p=1.0, min_p=0.0, seed=0xC0FFEE)
    steps = 12
    got, res = model.generate_variants(prompt, variants, samp=samp, max_tokens=steps,
                                       residuals=True)
    assert res.shape == (steps, cfg.layers, 16, cfg.hidden)
    # The prompt but its last token, once (no pin acts before the reply).
    oracle.set_edits(np.zeros(2 * cfg.layers, dtype=np.uint32))
    oracle.prompt(prompt[:-1])
    for v, edits in enumerate(variants):
        o = oracle.clone()
        o.set_edits(placed(cfg, edits, len(prompt) - 1))
        tok = int(prompt[-1])
        want = []
        for t in range(steps):
            pos = len(prompt) - 1 + t
            lg = o.token(tok, pos)
            r = o.residuals()
            for layer in range(cfg.layers):
                assert_same_bits(res[t, layer, v], r[layer], f"variant {v} step {t} layer {layer}")
            bits, ids = orc.topk(lg)
            rec = orc.draw(bits, ids, samp.top_k, samp.temperature, samp.top_p, samp.min_p,
                           counter=pos + 1, seed=samp.seed)
            tok = int(rec[0])
            want.append(tok)
        assert np.array_equal(got[v], np.array(want, dtype=np.uint32)), (v, got[v], want)
        o.close()
    # The pins act: a variant pinning a neuron below the last layer enters
    # the last layer with another residual than the original's. (They need
    # not change the drawn tokens: every row draws with the same seed.)
    for v, edits in enumerate(variants[1:], 1):
        if any(e.layer < cfg.layers - 1 for e in edits):
            assert not np.array_equal(res[0, -1, v], res[0, -1, 0]), v
    model.close()
    oracle.close()


@pytest.mark.parametrize("pins,temperature", [(0, 0.0), (8, 0.0), (8, 1.0)])
def test_full_size_256_steps(device, pins, temperature):
    # Gemma-3-1B's full shape (26 layers, 5 sliding to 1 global, the
    # 262,144-row tied Q4_0 head): a 16-token prompt, then 256 steps,
    # greedy unsteered and with 8 seeded pins in [-20, 20] over seeded
    # layers, and drawn at temperature 1 from a seed with those pins. Every
    # token and the last step's logits equal the oracle's. (A random model's
    # greedy reply settles on one token; the drawn reply wanders, so every
    # step's top 64 decide a varied token.)
    cfg = fz.gemma3_1b_config(context=1024)
    model, oracle = wandering_pair(device, cfg, seed=0)
    rng = np.random.default_rng(81 + pins)
    prompt = rng.integers(0, cfg.vocab, 16).astype(np.uint32)
    edits = []
    while len(edits) < pins:
        e = fz.Edit(int(rng.integers(0, cfg.layers)), int(rng.integers(0, cfg.ffn)),
                    fz.EditKind.SET, float(rng.uniform(-20, 20)))
        if all((e.layer, e.neuron) != (x.layer, x.neuron) for x in edits):
            edits.append(e)
    samp = fz.sampling(temperature=temperature, top_k=64, top_p=1.0, min_p=0.0, seed=0xC0FFEE)
    steps = 256
    got = model.generate(prompt, edits, samp=samp, max_tokens=steps)
    got_logits = model.logits()
    oracle.set_edits(placed(cfg, edits, len(prompt) - 1))
    lg = oracle.prompt(prompt)
    want = []
    for i in range(steps):
        bits, ids = orc.topk(lg)
        rec = orc.draw(bits, ids, samp.top_k, samp.temperature, samp.top_p, samp.min_p,
                       counter=len(prompt) + i, seed=samp.seed)
        want.append(int(rec[0]))
        if i + 1 < steps:
            lg = oracle.token(want[-1], len(prompt) + i)
    assert np.array_equal(got, np.array(want, dtype=np.uint32)), (got, want)
    assert_same_bits(got_logits, lg, "the 256th step's logits")
    if temperature > 0:
        assert len(set(want)) > 32
    model.close()
    oracle.close()


def test_global_layer_past_4096_keys(device):
    # Three layers (the third global) with an 8,192-token context: a
    # 4,160-token prompt in eight steps of 512 and one of 64, then 24 greedy
    # decode steps to position 4,183. The global layer reads 66 chunks
    # of 64 keys (4,161 to 4,184 keys) each step, folded in chunk order by
    # the fold kernel ahead of the O product; the sliding layers read their
    # 512-key windows from a ring of 1,024 slots that has wrapped four times.
    cfg = fz.gemma3_1b_config(layers=3, vocab=4096, window=512, pattern=3, context=8192,
                              local_slots=1024)
    model, oracle = wandering_pair(device, cfg, seed=91)
    prompt = np.random.default_rng(92).integers(0, cfg.vocab, 4160).astype(np.uint32)
    model.set_edits(np.zeros(2 * cfg.layers, dtype=np.uint32))
    oracle.set_edits(np.zeros(2 * cfg.layers, dtype=np.uint32))
    for p0 in range(0, len(prompt), 512):
        model.step(p0, prompt[p0:p0 + 512], logits=p0 + 512 >= len(prompt))
    want_end = oracle.prompt(prompt)
    assert_same_bits(model.logits(), want_end, "prompt-end logits")
    steps = 24
    want = []
    lg = want_end
    for i in range(steps):
        tok = int(orc.topk(lg)[1][0])
        want.append(tok)
        if i + 1 < steps:
            lg = oracle.token(tok, len(prompt) + i)
    first = int(model.record()[0])
    rest, failed = model.decode(len(prompt), steps - 1)
    got = np.concatenate([[first], rest]).astype(np.uint32)
    assert not failed.any()
    assert np.array_equal(got, np.array(want, dtype=np.uint32)), (got, want)
    assert_same_bits(model.logits(), lg, "last decode logits")
    for l in range(cfg.layers):
        n = oracle.key_cache(l).size
        assert np.array_equal(model.cache(l, False, n), oracle.key_cache(l)), f"keys {l}"
        assert np.array_equal(model.cache(l, True, n), oracle.value_cache(l)), f"values {l}"
    model.close()
    oracle.close()
