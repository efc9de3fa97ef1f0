"""The reference's replay scenario (tests/integration/replay/replay_test.cpp,
contracts 1-5 and 8) on seeded synthetic weights: edits that change nothing,
the cache rewound exactly where edits first differ, edit order, a
conversation after an edited reply, bit-for-bit branch continuation, and a
token past the vocabulary refused before anything runs."""
import numpy as np
import pytest

import frizzle_amd as fz
from helpers import assert_same_bits
from test_gpu_model import build_pair, small_config

pytestmark = pytest.mark.gpu

SAMP = dict(temperature=1.0, top_k=64, top_p=0.95, min_p=0.0, seed=7)


def strong(cfg):
    return [fz.Edit(l, n, fz.EditKind.SET, 20.0 if n % 2 else -20.0)
            for l in range(cfg.layers) for n in range(0, 64, 5)]


def test_scale_by_one_is_the_reply_without_edits(device):
    cfg = small_config()
    model, _ = build_pair(device, cfg, seed=71)
    prompt = np.random.default_rng(72).integers(0, cfg.vocab, 40).astype(np.uint32)
    s = fz.sampling(**SAMP)
    plain = model.generate(prompt, (), samp=s, max_tokens=20)
    logits = model.logits()
    ones = [fz.Edit(l, n, fz.EditKind.SCALE, 1.0) for l in range(cfg.layers) for n in (3, 99, 500)]
    scaled = model.generate(prompt, ones, samp=s, max_tokens=20)
    assert np.array_equal(plain, scaled)
    assert_same_bits(model.logits(), logits, "logits after Scale x 1")
    model.close()


def test_edits_rewind_the_cache_where_they_first_differ(device):
    cfg = small_config()
    model, _ = build_pair(device, cfg, seed=73)
    prompt = np.random.default_rng(74).integers(0, cfg.vocab, 45).astype(np.uint32)
    s = fz.sampling(**SAMP)
    first = model.generate(prompt, (), samp=s, max_tokens=16)
    model.generate(prompt, strong(cfg), samp=s, max_tokens=16)
    assert model.reused == len(prompt) - 1
    third = model.generate(prompt, (), samp=s, max_tokens=16)
    assert model.reused == len(prompt) - 1
    assert np.array_equal(first, third)
    model.close()


def test_one_edit_set_in_two_orders_is_one_reply(device):
    cfg = small_config()
    model, _ = build_pair(device, cfg, seed=75)
    prompt = np.random.default_rng(76).integers(0, cfg.vocab, 30).astype(np.uint32)
    s = fz.sampling(**SAMP)
    edits = strong(cfg)[::3] + [fz.Edit(1, 700, fz.EditKind.ZERO, 0.0, 2, 9)]
    a = model.generate(prompt, edits, samp=s, max_tokens=16)
    la = model.logits()
    b = model.generate(prompt, edits[::-1], samp=s, max_tokens=16)
    assert np.array_equal(a, b)
    assert_same_bits(model.logits(), la, "logits, edits reversed")
    model.generate(prompt, (), samp=s, max_tokens=16)
    assert not np.array_equal(model.logits(), la)
    model.close()


def test_a_conversation_after_an_edited_reply(device):
    # Its cached positions from the edited run's first edited one on are not
    # reused; its reply equals a fresh model's.
    cfg = small_config()
    model, _ = build_pair(device, cfg, seed=77)
    rng = np.random.default_rng(78)
    prompt = rng.integers(0, cfg.vocab, 35).astype(np.uint32)
    s = fz.sampling(**SAMP)
    steered = model.generate(prompt, strong(cfg), samp=s, max_tokens=12)
    turn = np.concatenate([prompt, steered, rng.integers(0, cfg.vocab, 9)]).astype(np.uint32)
    reply = model.generate(turn, (), samp=s, max_tokens=12)
    assert model.reused == len(prompt) - 1
    fresh, _ = build_pair(device, cfg, seed=77)
    assert np.array_equal(reply, fresh.generate(turn, (), samp=s, max_tokens=12))
    fresh.close()
    model.close()


@pytest.mark.parametrize("k", [0, 7, 17])
def test_a_branch_continues_the_reply_bit_for_bit(device, k):
    # Keeping the first k tokens of a reply and asking for what its limit
    # leaves gives the reply's tokens from k on; the kept tokens' cache
    # entries, written by decode steps in the original, come from a prefill
    # step here (batch invariance).
    cfg = small_config()
    model, _ = build_pair(device, cfg, seed=79)
    prompt = np.random.default_rng(80).integers(0, cfg.vocab, 33).astype(np.uint32)
    s = fz.sampling(**SAMP)
    n = 18
    original = model.generate(prompt, (), samp=s, max_tokens=n)
    fresh, _ = build_pair(device, cfg, seed=79)
    branch = fresh.generate(np.concatenate([prompt, original[:k]]).astype(np.uint32), (), samp=s,
                            max_tokens=n - k)
    assert np.array_equal(branch, original[k:])
    # From the same model, reusing its cache, too.
    again = model.generate(np.concatenate([prompt, original[:k]]).astype(np.uint32), (), samp=s,
                           max_tokens=n - k)
    assert model.reused == len(prompt) + k - 1
    assert np.array_equal(again, original[k:])
    fresh.close()
    model.close()


def test_a_token_past_the_vocabulary_is_refused_first(device):
    cfg = small_config()
    model, _ = build_pair(device, cfg, seed=81)
    prompt = np.arange(12, dtype=np.uint32)
    model.generate(prompt, (), max_tokens=2)
    bad = prompt.copy()
    bad[5] = cfg.vocab
    with pytest.raises(fz.FrzError, match="prompt token 5"):
        model.generate(bad, (), max_tokens=2)
    # Nothing ran: the cached prompt is still reused whole.
    model.generate(prompt, (), max_tokens=2)
    assert model.reused == len(prompt) - 1
    model.close()
