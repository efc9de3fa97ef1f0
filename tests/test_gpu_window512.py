"""The forward path in the regimes the timed workloads run, against the
oracle bit for bit:

- the real 512-key window with a prompt in 512-token prefill steps (the
  32 x 32 product tiles, 512-row chunk attention) and decode steps past the
  window, where each sliding layer folds 9 chunks in the O product's
  prologue and the ring of window + 512 slots wraps;
- the full Gemma-3-1B shape (26 layers, 262,144-token vocabulary) decoding
  past position 512;
- prompt reuse across runs that wrap a sliding layer's ring (the cache's
  high-water mark, cache/kv.h:30-35).
"""
import numpy as np
import pytest

import _oracle as orc
import frizzle_amd as fz
from helpers import assert_same_bits
from test_gpu_model import ROLES, build_pair, oracle_run

pytestmark = pytest.mark.gpu


def _oracle_prompt(oracle, prompt):
    """The prompt in the oracle's prefill blocks of 512 (each row's
    arithmetic is its token-by-token path's)."""
    return oracle.prompt(prompt)


def _oracle_greedy(oracle, logits, position, steps):
    """`steps` greedy draws from the prompt-end logits, each fed back."""
    out = []
    lg = logits
    for i in range(steps):
        tok = int(orc.topk(lg)[1][0])
        out.append(tok)
        if i + 1 < steps:
            lg = oracle.token(tok, position + i)
    return np.array(out, dtype=np.uint32), lg


def _check_caches(model, oracle, layers, what):
    for l in range(layers):
        n = oracle.key_cache(l).size
        assert np.array_equal(model.cache(l, False, n), oracle.key_cache(l)), f"{what}: keys {l}"
        assert np.array_equal(model.cache(l, True, n), oracle.value_cache(l)), f"{what}: values {l}"


def test_window_512_prefill_blocks_then_decode_bit_exact(device):
    # Three layers (the third global), window 512 and the smallest ring the
    # model takes (window + 512 = 1,024 slots). A 1,100-token prompt runs as
    # steps of 512, 512 and 76 tokens; 40 greedy decode steps follow, to
    # position 1,139, so the ring wraps during decode.
    cfg = fz.gemma3_1b_config(layers=3, vocab=4096, window=512, pattern=3, context=2048,
                              local_slots=1024)
    model, oracle = build_pair(device, cfg, seed=23)
    prompt = np.random.default_rng(24).integers(0, cfg.vocab, 1100).astype(np.uint32)
    model.set_edits(np.zeros(2 * cfg.layers, dtype=np.uint32))
    oracle.set_edits(np.zeros(2 * cfg.layers, dtype=np.uint32))
    model.step(0, prompt[:512], logits=False)
    model.step(512, prompt[512:1024], logits=False)
    model.step(1024, prompt[1024:], logits=True)
    want_end = _oracle_prompt(oracle, prompt)
    assert_same_bits(model.logits(), want_end, "prompt-end logits")
    _check_caches(model, oracle, cfg.layers, "after the prompt")
    steps = 40
    want, want_last = _oracle_greedy(oracle, want_end, len(prompt), steps)
    first = int(model.record()[0])
    rest, failed = model.decode(len(prompt), steps - 1)
    got = np.concatenate([[first], rest]).astype(np.uint32)
    assert not failed.any()
    assert np.array_equal(got, want), (got, want)
    assert_same_bits(model.logits(), want_last, "last decode logits")
    _check_caches(model, oracle, cfg.layers, "after decode")
    model.close()
    oracle.close()


def test_window_512_generate_matches_steps(device):
    # The same regime through generate(): prefill blocks planned by the turn
    # loop (turn.cpp:22-40), the decode graph replayed, and a second run of
    # the same prompt reusing all of it but its last token.
    cfg = fz.gemma3_1b_config(layers=3, vocab=4096, window=512, pattern=3, context=2048,
                              local_slots=1024)
    model, oracle = build_pair(device, cfg, seed=29)
    prompt = np.random.default_rng(30).integers(0, cfg.vocab, 700).astype(np.uint32)
    want, _ = oracle_run(oracle, prompt, 48, cfg, np.zeros(2 * cfg.layers, dtype=np.uint32))
    got = model.generate(prompt, max_tokens=48)
    assert np.array_equal(got, want), (got, want)
    again = model.generate(prompt, max_tokens=48)
    assert model.reused == len(prompt) - 1
    assert np.array_equal(again, want)
    model.close()
    oracle.close()


def test_full_size_decode_past_the_window(device):
    # Gemma-3-1B's full shape: 26 layers (5 sliding to 1 global), the
    # 262,144-row tied head. A 530-token prompt (steps of 512 and 18), then
    # 20 greedy decode steps to position 549, where every sliding layer's
    # window has left position 0 behind.
    cfg = fz.gemma3_1b_config(context=1024)
    model, oracle = build_pair(device, cfg, seed=0x5EED)
    prompt = np.random.default_rng(31).integers(0, cfg.vocab, 530).astype(np.uint32)
    model.set_edits(np.zeros(2 * cfg.layers, dtype=np.uint32))
    oracle.set_edits(np.zeros(2 * cfg.layers, dtype=np.uint32))
    model.step(0, prompt[:512], logits=False)
    model.step(512, prompt[512:], logits=True)
    want_end = _oracle_prompt(oracle, prompt)
    assert_same_bits(model.logits(), want_end, "prompt-end logits")
    steps = 20
    want, want_last = _oracle_greedy(oracle, want_end, len(prompt), steps)
    first = int(model.record()[0])
    rest, _ = model.decode(len(prompt), steps - 1)
    got = np.concatenate([[first], rest]).astype(np.uint32)
    assert np.array_equal(got, want), (got, want)
    assert_same_bits(model.logits(), want_last, "last decode logits")
    _check_caches(model, oracle, cfg.layers, "after decode")
    model.close()
    oracle.close()


def _fresh_pair(device, cfg, tensors):
    m = fz.Model(device, cfg)
    for (l, r), a in tensors.items():
        m.set_tensor(l, r, a)
    return m


def test_reuse_keeps_the_ring_high_water_mark(device):
    # Window 64, ring of 640 slots. Run A writes positions 0..999; run B
    # reuses 990 of them; run C repeats only A's first 420 tokens. B wrote
    # no further than A, so A's positions 997..999 still sit in the slots of
    # positions 357..359, inside C's window at 420: C must not reuse, and its
    # reply and logits are a fresh model's.
    cfg = fz.gemma3_1b_config(layers=3, vocab=4096, window=64, pattern=3, context=1024,
                              local_slots=640)
    model, oracle = build_pair(device, cfg, seed=37)
    rng = np.random.default_rng(38)
    a = rng.integers(0, cfg.vocab, 1000).astype(np.uint32)
    b = np.concatenate([a[:990], rng.integers(0, cfg.vocab, 5).astype(np.uint32)])
    c = np.concatenate([a[:420], rng.integers(0, cfg.vocab, 30).astype(np.uint32)])
    model.generate(a, max_tokens=1)
    model.generate(b, max_tokens=1)
    assert model.reused == 990
    got = model.generate(c, max_tokens=6)
    assert model.reused == 0
    got_logits = model.logits()
    fresh = _fresh_pair(device, cfg, oracle.tensors)
    want = fresh.generate(c, max_tokens=6)
    assert np.array_equal(got, want), (got, want)
    assert_same_bits(got_logits, fresh.logits(), "C's last logits")
    # And a run that the mark allows to reuse still does: C's prompt again.
    again = model.generate(c, max_tokens=6)
    assert model.reused == len(c) - 1
    assert np.array_equal(again, want)
    fresh.close()
    model.close()
    oracle.close()


def test_timed_decode_forgets_the_prompt(device):
    # Timing decode steps rewrites the caches after the prompt; a repeated
    # prompt is then computed afresh, and its reply is the oracle's.
    cfg = fz.gemma3_1b_config(layers=3, vocab=4096, window=64, pattern=3, context=1024,
                              local_slots=640)
    model, oracle = build_pair(device, cfg, seed=41)
    prompt = np.random.default_rng(42).integers(0, cfg.vocab, 60).astype(np.uint32)
    model.generate(prompt, max_tokens=4)
    assert model.time_decode(len(prompt) - 20, 30) > 0
    got = model.generate(prompt, max_tokens=8)
    assert model.reused == 0
    want, _ = oracle_run(oracle, prompt, 8, cfg, np.zeros(2 * cfg.layers, dtype=np.uint32))
    assert np.array_equal(got, want), (got, want)
    model.close()
    oracle.close()


def test_window_512_variants_bit_exact(device):
    # Variants steps at the real window: every sliding layer reads 9 chunks
    # (the workgroup-per-(chunk, row) attention and the 16-row products),
    # and the ring of window + 512 slots wraps during the replies. The
    # original and a steered variant equal the oracle's greedy runs.
    from test_gpu_variants import seeded_variants
    from test_gpu_model import placed
    cfg = fz.gemma3_1b_config(layers=3, vocab=4096, window=512, pattern=3, context=2048,
                              local_slots=1024)
    model, oracle = build_pair(device, cfg, seed=31)
    rng = np.random.default_rng(32)
    prompt = rng.integers(0, cfg.vocab, 1030).astype(np.uint32)
    variants = seeded_variants(cfg, rng, 4)
    steps = 16
    got = model.generate_variants(prompt, variants, max_tokens=steps)
    for v in (0, 1):
        o = orc.OracleModel(cfg.as_dict(), oracle.tensors)
        o.set_edits(placed(cfg, variants[v], len(prompt) - 1))
        end = _oracle_prompt(o, prompt)
        want, _ = _oracle_greedy(o, end, len(prompt), steps)
        assert np.array_equal(got[v], want), (v, got[v], want)
        o.close()
    model.close()
    oracle.close()
