"""The capture store on the GPU against the oracle's captures, every word of
every slot, bit for bit, at the step that ends a prompt; and the store's
contract from the reference's replay scenario
(tests/integration/replay/replay_test.cpp: 7, every word written; 9, the
readouts)."""
import numpy as np
import pytest

import _oracle as orc
import frizzle_amd as fz
from test_gpu_model import build_pair, placed, small_config

pytestmark = pytest.mark.gpu


def oracle_capture(oracle, cfg, prompt, table):
    o = orc.OracleModel(cfg.as_dict(), oracle.tensors)
    o.set_edits(table)
    o.set_capture(True)
    for p, tok in enumerate(prompt):
        o.token(tok, p, want_logits=(p == len(prompt) - 1))
    return o


def assert_store_is_oracles(store, layout, o, what):
    for layer, slots in enumerate(layout):
        for name in fz.CAPTURE_SLOTS:
            first, width = slots[name]
            want = o.capture(layer, name)
            assert want.size == width, (what, layer, name, want.size, width)
            got = store[first:first + width]
            bad = np.nonzero(got != want)[0]
            assert bad.size == 0, (f"{what}: layer {layer} {name}: {bad.size} words differ, "
                                   f"first at {bad[0]}: {got[bad[0]]:#x} vs {want[bad[0]]:#x}")


def test_capture_store_is_the_oracles(device):
    cfg = small_config()
    model, oracle = build_pair(device, cfg, seed=61)
    rng = np.random.default_rng(62)
    prompt = rng.integers(0, cfg.vocab, 90).astype(np.uint32)  # past the 64-key window
    edits = [fz.Edit(1, 17, fz.EditKind.SET, 12.5), fz.Edit(2, 300, fz.EditKind.SCALE, -3.0)]
    model.set_capture(True)
    reply = model.generate(prompt, edits, max_tokens=4)
    store, layout = model.capture()
    o = oracle_capture(oracle, cfg, prompt, placed(cfg, edits, len(prompt) - 1))
    assert_store_is_oracles(store, layout, o, "prompt end")
    # The pinned neuron holds its pin; the last layer's readout begins with
    # the reply's first token; every readout is 64 distinct tokens.
    neurons = store[layout[1]["neurons"][0]:][:cfg.ffn].view(np.float32)
    assert neurons[17] == np.float32(12.5)
    for layer in range(cfg.layers):
        first, width = layout[layer]["readout"]
        ids = store[first + 1:first + width:2]
        assert len(set(ids.tolist())) == 64
    assert store[layout[-1]["readout"][0] + 1] == reply[0]
    o.close()
    model.close()


def test_capture_at_a_one_token_prompt_end_and_every_word_rewritten(device):
    # The second run reuses the whole cached prompt but its last token, so
    # its prompt-end step holds one token; a different, shorter prompt
    # before it leaves nothing of its own in the store.
    cfg = small_config()
    model, oracle = build_pair(device, cfg, seed=63)
    rng = np.random.default_rng(64)
    long_prompt = rng.integers(0, cfg.vocab, 120).astype(np.uint32)
    prompt = rng.integers(0, cfg.vocab, 30).astype(np.uint32)
    model.set_capture(True)
    model.generate(long_prompt, (), max_tokens=2)
    model.generate(prompt, (), max_tokens=2)
    model.generate(prompt, (), max_tokens=2)  # one-token prompt end
    store, layout = model.capture()
    o = oracle_capture(oracle, cfg, prompt, placed(cfg, [], len(prompt) - 1))
    assert_store_is_oracles(store, layout, o, "one-token prompt end")
    o.close()
    # With capture off, later runs leave the store as it was.
    model.set_capture(False)
    model.generate(long_prompt, (), max_tokens=2)
    again, _ = model.capture()
    assert np.array_equal(again, store)
    model.close()


def test_inspection_captures_what_a_run_does(device):
    # An inspection (max_tokens 0) draws nothing and captures the whole
    # store, equal to a run's from the same prompt and edits
    # (replay_test.cpp, 7).
    cfg = small_config()
    model, _ = build_pair(device, cfg, seed=67)
    prompt = np.random.default_rng(68).integers(0, cfg.vocab, 50).astype(np.uint32)
    edits = [fz.Edit(0, 9, fz.EditKind.ZERO, 0.0)]
    model.set_capture(True)
    assert model.generate(prompt, edits, max_tokens=0).size == 0
    inspected, _ = model.capture()
    fresh, _ = build_pair(device, cfg, seed=67)
    fresh.set_capture(True)
    fresh.generate(prompt, edits, max_tokens=6)
    ran, _ = fresh.capture()
    assert np.array_equal(inspected, ran)
    fresh.close()
    model.close()


def test_readouts_see_the_residual_where_each_layer_leaves_it(device):
    # A pin at layer 1 leaves the readouts below it bit for bit and changes
    # its own (replay_test.cpp, 9).
    cfg = small_config()
    model, _ = build_pair(device, cfg, seed=65)
    prompt = np.random.default_rng(66).integers(0, cfg.vocab, 40).astype(np.uint32)
    model.set_capture(True)
    model.generate(prompt, (), max_tokens=1)
    plain, layout = model.capture()
    model.generate(prompt, [fz.Edit(1, 5, fz.EditKind.SET, 20.0)], max_tokens=1)
    pinned, _ = model.capture()

    def readout(store, layer):
        first, width = layout[layer]["readout"]
        return store[first:first + width]

    assert np.array_equal(readout(plain, 0), readout(pinned, 0))
    assert not np.array_equal(readout(plain, 1), readout(pinned, 1))
    model.close()
