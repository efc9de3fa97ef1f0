"""Many steered replies to one prompt decoded as one batch
(frz_generate_variants): each variant's tokens are the ones the reply gets
alone, through frz_generate and through the oracle, and the residual capture
is the oracle's residual entering each layer, bit for bit."""
import numpy as np
import pytest

import _oracle as orc
import frizzle_amd as fz
from helpers import assert_same_bits
from test_gpu_model import (MIXED, _mixed_tensors, _set_all, build_pair, oracle_run, placed,
                            small_config)

pytestmark = pytest.mark.gpu


def seeded_variants(cfg, rng, count):
    """The original (no edits) and count - 1 variants, each pinning 1 to 8
    seeded neurons of seeded layers to values in [-20, 20], some over a
    bounded range of steps, one scaling and one zeroing."""
    out = [[]]
    for v in range(1, count):
        n = int(rng.integers(1, 9))
        edits = {}
        for _ in range(n):
            layer, neuron = int(rng.integers(0, cfg.layers)), int(rng.integers(0, cfg.ffn))
            start = int(rng.integers(0, 3)) if v % 3 == 0 else 0
            until = start + int(rng.integers(2, 6)) if v % 4 == 0 else fz.TO_THE_END
            edits[(layer, neuron)] = fz.Edit(layer, neuron, fz.EditKind.SET,
                                             float(rng.uniform(-20, 20)), start, until)
        if v % 5 == 0:
            edits[(0, 7)] = fz.Edit(0, 7, fz.EditKind.SCALE, 2.5)
        if v % 5 == 1:
            edits[(1, 9)] = fz.Edit(1, 9, fz.EditKind.ZERO, 0.0)
        out.append(list(edits.values()))
    return out


def test_variants_are_the_replies_alone(device):
    cfg = small_config()
    model, _ = build_pair(device, cfg, seed=51)
    rng = np.random.default_rng(52)
    prompt = rng.integers(0, cfg.vocab, 45).astype(np.uint32)
    variants = seeded_variants(cfg, rng, 8)
    samp = fz.sampling(temperature=1.0, top_k=64, top_p=1.0, min_p=0.0, seed=0x5EED)
    steps = 20
    got, res = model.generate_variants(prompt, variants, samp=samp, max_tokens=steps,
                                       residuals=True)
    for v, edits in enumerate(variants):
        alone = model.generate(prompt, edits, samp=samp, max_tokens=steps)
        assert np.array_equal(got[v], alone), (v, got[v], alone)
    # The pins act: at the prompt's last token the residual leaving the model
    # differs from the original's for the variants pinned from step 0 (a
    # random-init model may keep its tokens, so they alone need not differ).
    last = res[0, -1]
    assert sum(not np.array_equal(last[0], last[v]) for v in range(1, len(variants))) >= 3
    model.close()


def test_variants_over_the_pinned_files_formats(device):
    # A Q8_0 embedding and tied head, Q4_1 and Q8_0 downs: the 16-row
    # products of those formats (the down split over two workgroups, the
    # Q8_0 head) give each variant the tokens its reply gets alone, greedy
    # and sampled.
    cfg = small_config()
    model = fz.Model(device, cfg)
    _set_all(model, _mixed_tensors(cfg, 61), MIXED)
    rng = np.random.default_rng(62)
    prompt = rng.integers(0, cfg.vocab, 70).astype(np.uint32)
    variants = seeded_variants(cfg, rng, 16)
    for samp in (fz.sampling(), fz.sampling(temperature=1.0, top_k=64, seed=0x61)):
        got = model.generate_variants(prompt, variants, samp=samp, max_tokens=12)
        for v, edits in enumerate(variants):
            alone = model.generate(prompt, edits, samp=samp, max_tokens=12)
            assert np.array_equal(got[v], alone), (v, got[v], alone)
    model.close()


def test_variants_greedy_and_the_oracle_with_residuals(device):
    cfg = small_config()
    model, oracle = build_pair(device, cfg, seed=53)
    rng = np.random.default_rng(54)
    prompt = rng.integers(0, cfg.vocab, 33).astype(np.uint32)
    variants = seeded_variants(cfg, rng, 3)
    steps = 10
    got, res = model.generate_variants(prompt, variants, max_tokens=steps, residuals=True)
    assert res.shape == (steps, cfg.layers, 3, cfg.hidden)
    for v in (0, 2):
        o = orc.OracleModel(cfg.as_dict(), oracle.tensors)
        o.set_edits(placed(cfg, variants[v], len(prompt) - 1))
        want, _ = oracle_run(o, prompt, steps, cfg)
        assert np.array_equal(got[v], want), (v, got[v], want)
        # The residuals of every step: the prompt's last token, then each fed
        # token, token by token through the oracle again.
        o2 = orc.OracleModel(cfg.as_dict(), oracle.tensors)
        o2.set_edits(placed(cfg, variants[v], len(prompt) - 1))
        for p, tok in enumerate(prompt[:-1]):
            o2.token(tok, p, want_logits=False)
        fed = [int(prompt[-1])] + [int(t) for t in want[:-1]]
        for t, tok in enumerate(fed):
            o2.token(tok, len(prompt) - 1 + t, want_logits=False)
            r = o2.residuals()
            for layer in range(cfg.layers):
                assert_same_bits(res[t, layer, v], r[layer], f"variant {v} step {t} layer {layer}")
        o.close()
        o2.close()
    model.close()


def test_variants_stop_and_leave_the_prompt_cached(device):
    cfg = small_config()
    model, _ = build_pair(device, cfg, seed=55)
    rng = np.random.default_rng(56)
    prompt = rng.integers(0, cfg.vocab, 28).astype(np.uint32)
    variants = seeded_variants(cfg, rng, 4)
    full = model.generate_variants(prompt, variants, max_tokens=12)
    # A stop token ends a variant's reply where generate() would end it.
    stop = int(full[1][4])
    cut = model.generate_variants(prompt, variants, max_tokens=12, stop_ids=[stop])
    for v in range(4):
        alone = model.generate(prompt, variants[v], max_tokens=12, stop_ids=[stop])
        assert np.array_equal(cut[v], alone), (v, cut[v], alone)
    assert len(cut[1]) <= 5
    # The model's own caches hold the prompt afterwards: a plain reply equals
    # a fresh model's.
    again = model.generate(prompt, (), max_tokens=12)
    fresh, _ = build_pair(device, cfg, seed=55)
    assert np.array_equal(again, fresh.generate(prompt, (), max_tokens=12))
    assert np.array_equal(again, full[0])
    fresh.close()
    model.close()


def test_variants_refusals(device):
    cfg = small_config()
    model, _ = build_pair(device, cfg, seed=57)
    prompt = np.arange(10, dtype=np.uint32)
    with pytest.raises(fz.FrzError, match="1 to 64 variants"):
        model.generate_variants(prompt, [[]] * 65, max_tokens=2)
    with pytest.raises(fz.FrzError, match="within the context"):
        model.generate_variants(prompt, [[]], max_tokens=cfg.context)
    bad = np.zeros(2 * cfg.layers + 5, dtype=np.uint32)
    bad[0], bad[1] = 2 * cfg.layers, 1
    bad[2 * cfg.layers] = cfg.ffn  # a neuron past the width
    lib = fz.load()
    out = np.zeros(4, dtype=np.uint32)
    drawn = np.zeros(1, dtype=np.uint32)
    s = fz.sampling()
    import ctypes
    with pytest.raises(fz.FrzError, match="neuron or kind out of range"):
        fz._lib.check(lib.frz_generate_variants(
            model.handle, prompt.ctypes.data, prompt.size, 1, bad.ctypes.data, bad.size,
            ctypes.byref(s), 4, None, 0, out.ctypes.data, drawn.ctypes.data, None))
    model.close()
