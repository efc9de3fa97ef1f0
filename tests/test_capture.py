"""The capture store's layout (frz_capture_words, frz_capture_layer) against
the reference's own counts for Gemma 3 1B (src/core/capture/capture.h:67-75)
and its stated order. Pure host functions: no GPU."""
import ctypes

import numpy as np
import pytest

import frizzle_amd as fz

GLOBAL = {5, 11, 17, 23}


def test_layout_matches_the_reference_counts():
    # The reference sizes the global layers' weights by the trained context,
    # 32,768, the context this model is shaped with here.
    cfg = fz.gemma3_1b_config(context=32768)
    layout = fz.capture_layout(cfg)
    assert fz.capture_words(cfg) == 869_072
    total = {k: sum(s[k][1] for s in layout) for k in fz.CAPTURE_SLOTS}
    assert total["neurons"] == 179_712
    assert total["residual"] + total["attention_added"] + total["mlp_added"] == 89_856
    assert total["query"] == 26_624
    assert total["weights"] == 569_344
    assert total["stats"] == 208
    assert total["readout"] == 3_328
    for layer, s in enumerate(layout):
        assert s["full_attention"] == (layer in GLOBAL)
        assert s["keys"] == (32768 if layer in GLOBAL else 512)
        assert s["window"] == s["keys"]
        assert s["weights"][1] == 4 * s["keys"]


@pytest.mark.parametrize("context", [1024, 8192, 32768])
def test_layout_is_two_contiguous_regions_in_order(context):
    cfg = fz.gemma3_1b_config(context=context)
    layout = fz.capture_layout(cfg)
    # Region 1: every layer's neurons, layer after layer, from word 0.
    at = 0
    for s in layout:
        assert s["neurons"] == (at, cfg.ffn)
        at += cfg.ffn
    # Region 2: per layer the residual, the two additions, the query, the
    # weights, the statistics and the readout, each after the last.
    for s in layout:
        for name, width in [("residual", cfg.hidden), ("attention_added", cfg.hidden),
                            ("mlp_added", cfg.hidden), ("query", 4 * 256),
                            ("weights", 4 * s["keys"]), ("stats", 8), ("readout", 128)]:
            assert s[name] == (at, width), name
            at += width
    assert at == fz.capture_words(cfg)
    words = np.zeros(at, dtype=np.int64)
    for s in layout:
        for name in fz.CAPTURE_SLOTS:
            first, width = s[name]
            words[first:first + width] += 1
    assert (words == 1).all()  # every word in exactly one slot


def test_layout_refusals():
    cfg = fz.gemma3_1b_config()
    cfg.layers = 0
    assert fz.capture_words(cfg) == 0
    good = fz.gemma3_1b_config()
    slots = fz._lib.CaptureSlots()
    for layer in (-1, 26):
        assert fz.load().frz_capture_layer(ctypes.byref(good), layer, ctypes.byref(slots)) != 0
