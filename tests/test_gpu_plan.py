"""A model created from a residency plan (frz_model_create_planned) is the
model its tensors make when created directly: the same prefill logits,
caches, tokens and capture store, bit for bit, over the plan's buffers
(Q, K and V read as one product over the members the plan placed apart),
with the formats of the pinned file, and at the limits a WebGPU device
grants as well as this device's. Refusals name what they refuse."""
import numpy as np
import pytest

import frizzle_amd as fz
from frizzle_amd import gguf
from frizzle_amd import plan as fp
from helpers import assert_same_bits, q4_1_blocks, q8_0_blocks
from test_gpu_model import ROLES

pytestmark = pytest.mark.gpu


def _cfg():
    return fz.gemma3_1b_config(layers=3, vocab=4096, window=64, pattern=3, context=1024,
                               local_slots=64 + 512 + 4096)


def _tensors(cfg, seed, mixed=False):
    t = {(l, r): fz.synth_tensor(cfg, seed, l, r) for l in range(cfg.layers) for r in ROLES}
    t[(-1, "embedding")] = fz.synth_tensor(cfg, seed, -1, "embedding")
    t[(-1, "output_norm")] = fz.synth_tensor(cfg, seed, -1, "output_norm")
    formats = {}
    if mixed:
        rng = np.random.default_rng(seed)
        t[(-1, "embedding")] = q8_0_blocks(rng, cfg.vocab, cfg.hidden, scale_std=0.004)
        t[(0, "down")] = q4_1_blocks(rng, cfg.hidden, cfg.ffn, scale_std=0.01)
        t[(2, "down")] = q8_0_blocks(rng, cfg.hidden, cfg.ffn, scale_std=0.0006)
        formats = {(-1, "embedding"): fz.Q8_0, (0, "down"): fz.Q4_1, (2, "down"): fz.Q8_0}
    return t, formats


def _file(tmp_path, cfg, t, formats):
    names = {(-1, "embedding"): "token_embd.weight"}
    for l in range(cfg.layers):
        names[(l, "down")] = f"blk.{l}.ffn_down.weight"
    return gguf.write_gemma3(tmp_path / "m.gguf", cfg, lambda l, r: t[(l, r)].tobytes(),
                             formats={names[k]: f for k, f in formats.items()})


def _direct(device, cfg, t, formats):
    m = fz.Model(device, cfg)
    for (l, r), a in t.items():
        m.set_tensor(l, r, a, formats.get((l, r)))
    return m


def _same_run(a, b, cfg, prompt, steps=16):
    a.set_edits(np.zeros(2 * cfg.layers, dtype=np.uint32))
    b.set_edits(np.zeros(2 * cfg.layers, dtype=np.uint32))
    a.step(0, prompt, logits=True)
    b.step(0, prompt, logits=True)
    assert_same_bits(a.logits(), b.logits(), "prompt-end logits")
    for l in range(cfg.layers):
        n = cfg.context * 256 if l % cfg.pattern == cfg.pattern - 1 else cfg.local_slots * 256
        assert np.array_equal(a.cache(l, False, n), b.cache(l, False, n)), f"keys {l}"
        assert np.array_equal(a.cache(l, True, n), b.cache(l, True, n)), f"values {l}"
    ta = a.generate(prompt, max_tokens=steps)
    tb = b.generate(prompt, max_tokens=steps)
    assert np.array_equal(ta, tb), (ta, tb)
    assert_same_bits(a.logits(), b.logits(), "last logits")


@pytest.mark.parametrize("limits", ["device", "webgpu"])
@pytest.mark.parametrize("mixed", [False, True])
def test_planned_model_is_the_direct_model(device, tmp_path, limits, mixed):
    cfg = _cfg()
    t, formats = _tensors(cfg, 71, mixed)
    path = _file(tmp_path, cfg, t, formats)
    lim = fp.device_limits(device) if limits == "device" else fp.limits(*fp.WEBGPU_DEFAULT_LIMITS)
    p = fp.Plan(gguf.Index.open(path), lim)
    assert p.context_offered == cfg.context
    planned = fz.Model.planned(device, p)
    # the plan's rings: window + 512 + reserve, cut to the context offered
    assert planned.cfg.context == cfg.context and planned.cfg.local_slots == cfg.context
    planned.load_gguf(path)
    direct = _direct(device, planned.cfg, t, formats)
    prompt = np.random.default_rng(72).integers(0, cfg.vocab, 150).astype(np.uint32)
    _same_run(planned, direct, planned.cfg, prompt)
    planned.close()
    direct.close()


def test_planned_capture_store_is_the_plans(device, tmp_path):
    # The capture store lives in the plan's "captures" buffer; its words are
    # the direct model's.
    cfg = _cfg()
    t, formats = _tensors(cfg, 73)
    path = _file(tmp_path, cfg, t, formats)
    p = fp.Plan(gguf.Index.open(path), fp.device_limits(device))
    planned = fz.Model.planned(device, p)
    planned.load_gguf(path)
    direct = _direct(device, planned.cfg, t, formats)
    prompt = np.random.default_rng(74).integers(0, cfg.vocab, 90).astype(np.uint32)
    for m in (planned, direct):
        m.set_capture(True)
        m.generate(prompt, max_tokens=1)
    a, _ = planned.capture()
    b, _ = direct.capture()
    assert np.array_equal(a, b)
    planned.close()
    direct.close()


def test_planned_context_follows_the_budget(device, tmp_path):
    # A smaller budget offers a shorter context; the model runs at it, its
    # global layer's cache that many slots.
    cfg = _cfg()
    t, formats = _tensors(cfg, 75)
    path = _file(tmp_path, cfg, t, formats)
    ix = gguf.Index.open(path)
    full = fp.Plan(ix, fp.device_limits(device))
    s = full.summary
    fixed = s["weight_bytes"] + s["scratch_bytes"] + 2 * cfg.layers * (256 + 4)
    budget = fixed + 2 * 512 * (2 * 700 + 700)  # two sliding layers and one global at 700
    p = fp.Plan(ix, fp.device_limits(device), fp.policy(memory_budget=budget))
    assert p.context_offered == 700
    m = fz.Model.planned(device, p)
    m.load_gguf(path)
    assert m.cfg.context == 700
    prompt = np.random.default_rng(76).integers(0, cfg.vocab, 600).astype(np.uint32)
    got = m.generate(prompt, max_tokens=20)
    direct = _direct(device, fz.gemma3_1b_config(layers=3, vocab=4096, window=64, pattern=3,
                                                 context=700, local_slots=700), t, formats)
    want = direct.generate(prompt, max_tokens=20)
    assert np.array_equal(got, want)
    with pytest.raises(fz.FrzError, match="past the context"):
        m.step(700, np.zeros(1, np.uint32))
    m.close()
    direct.close()


def test_planned_model_refusals(device, tmp_path):
    # A 16 MiB binding holds every working buffer (the largest, the
    # activation, is 14.2 MB) but cuts a 32,768-row embedding (21.2 MB) in
    # two pieces.
    wide = fz.gemma3_1b_config(layers=3, vocab=32768, window=64, pattern=3, context=1024)
    tw, fw = _tensors(wide, 78)
    p = fp.Plan(gguf.Index.open(_file(tmp_path, wide, tw, fw)), fp.limits(256 << 20, 16 << 20, 256))
    assert p.summary["pieces"] == p.summary["tensors"] + 1
    with pytest.raises(fz.FrzError, match="pieces; this backend runs each weight as one"):
        fz.Model.planned(device, p)
    # A tensor in another format than the plan placed it in.
    cfg = _cfg()
    t, formats = _tensors(cfg, 77)
    (tmp_path / "small").mkdir()
    ix = gguf.Index.open(_file(tmp_path / "small", cfg, t, formats))
    p = fp.Plan(ix, fp.device_limits(device))
    m = fz.Model.planned(device, p)
    rng = np.random.default_rng(1)
    with pytest.raises(fz.FrzError, match="the plan placed this tensor in format 2"):
        m.set_tensor(0, "down", q8_0_blocks(rng, cfg.hidden, cfg.ffn), fz.Q8_0)
    m.close()
