"""The whole forward path on the GPU against the oracle: prefill in one or
several steps, greedy and seeded decode, pins, the KV caches, bit for bit."""
import numpy as np
import pytest

import _oracle as orc
import frizzle_amd as fz
from helpers import assert_same_bits, q4_1_blocks, q8_0_blocks

pytestmark = pytest.mark.gpu

ROLES = ["q", "k", "v", "o", "gate", "up", "down", "attn_norm", "q_norm", "k_norm",
         "post_attn_norm", "ffn_norm", "post_ffn_norm"]


def small_config(**kw):
    """Gemma-3-1B's layer shapes with 3 layers (the third global), a 4,096
    vocabulary and a 64-token window, so short runs cross the window."""
    base = dict(layers=3, vocab=4096, window=64, pattern=3, context=1024,
                local_slots=64 + 512 + 64)
    base.update(kw)
    return fz.gemma3_1b_config(**base)


def build_pair(device, cfg, seed):
    """The same synthetic weights on the GPU and in the oracle."""
    tensors = {}
    for l in range(cfg.layers):
        for r in ROLES:
            tensors[(l, r)] = fz.synth_tensor(cfg, seed, l, r)
    tensors[(-1, "embedding")] = fz.synth_tensor(cfg, seed, -1, "embedding")
    tensors[(-1, "output_norm")] = fz.synth_tensor(cfg, seed, -1, "output_norm")
    model = fz.Model(device, cfg)
    for (l, r), a in tensors.items():
        model.set_tensor(l, r, a)
    oracle = orc.OracleModel(cfg.as_dict(), tensors)
    return model, oracle


def oracle_run(oracle, prompt, steps, cfg, edits_table=None, greedy=True, samp=None):
    """Token by token: the prompt, then `steps` draws fed back. Returns the
    drawn tokens and the logits at the prompt's end."""
    if edits_table is not None:
        oracle.set_edits(edits_table)
    end_logits = None
    for p, tok in enumerate(prompt):
        lg = oracle.token(tok, p, want_logits=(p == len(prompt) - 1))
        if p == len(prompt) - 1:
            end_logits = lg
    out = []
    lg = end_logits
    pos = len(prompt)
    for i in range(steps):
        bits, ids = orc.topk(lg)
        if greedy:
            tok = int(ids[0])
        else:
            rec = orc.draw(bits, ids, samp.top_k, samp.temperature, samp.top_p, samp.min_p,
                           counter=pos, seed=samp.seed)
            tok = int(rec[0])
        out.append(tok)
        if i + 1 < steps:
            lg = oracle.token(tok, pos)
            pos += 1
    return np.array(out, dtype=np.uint32), end_logits


def placed(cfg, edits, origin):
    return fz.edit_table(edits, cfg.layers, origin)


def test_prefill_logits_and_cache_bit_exact(device):
    cfg = small_config()
    model, oracle = build_pair(device, cfg, seed=7)
    rng = np.random.default_rng(3)
    prompt = rng.integers(0, cfg.vocab, 100).astype(np.uint32)
    model.set_edits(np.zeros(2 * cfg.layers, dtype=np.uint32))
    model.step(0, prompt[:37], logits=False)
    model.step(37, prompt[37:], logits=True)
    got = model.logits()
    _, want = oracle_run(oracle, prompt, 0, cfg)
    assert_same_bits(got, want, "prompt-end logits")
    for l in range(cfg.layers):
        n = oracle.key_cache(l).size
        assert np.array_equal(model.cache(l, False, n), oracle.key_cache(l)), f"keys {l}"
        assert np.array_equal(model.cache(l, True, n), oracle.value_cache(l)), f"values {l}"
    model.close()


@pytest.mark.parametrize("split", [None, 1])
def test_greedy_decode_token_identical(device, split):
    cfg = small_config()
    model, oracle = build_pair(device, cfg, seed=11)
    rng = np.random.default_rng(5)
    prompt = rng.integers(0, cfg.vocab, 70).astype(np.uint32)
    steps = 40
    want, _ = oracle_run(oracle, prompt, steps, cfg)
    if split is None:
        got = model.generate(prompt, max_tokens=steps)
    else:
        model.set_edits(np.zeros(2 * cfg.layers, dtype=np.uint32))
        for p, tok in enumerate(prompt):  # every position decoded alone
            model.step(p, [tok], logits=(p == len(prompt) - 1))
        first = model.record()[0]
        rest, _ = model.decode(len(prompt), steps - 1)
        got = np.concatenate([[first], rest]).astype(np.uint32)
    assert np.array_equal(got, want), (got, want)
    # The logits the last token was drawn from, bit for bit.
    lg = oracle.token(int(want[-2]), len(prompt) + steps - 2)
    assert_same_bits(model.logits(), lg, "last decode logits")
    model.close()


def test_steered_and_original_token_identical(device):
    cfg = small_config()
    model, oracle = build_pair(device, cfg, seed=13)
    rng = np.random.default_rng(8)
    prompt = rng.integers(0, cfg.vocab, 50).astype(np.uint32)
    steps = 24
    edits = [fz.Edit(int(l), int(n), fz.EditKind.SET, float(v))
             for l, n, v in zip(rng.integers(0, cfg.layers, 8), rng.integers(0, cfg.ffn, 8),
                                rng.uniform(-10, 10, 8))]
    edits = list({(e.layer, e.neuron): e for e in edits}.values())
    edits.append(fz.Edit(0, 5, fz.EditKind.SCALE, 3.0, 4, 9))
    original = model.generate(prompt, (), max_tokens=steps)
    cand_o = model.candidates()
    steered = model.generate(prompt, edits, max_tokens=steps)
    cand_s = model.candidates()
    want_o, _ = oracle_run(oracle, prompt, steps, cfg,
                           np.zeros(2 * cfg.layers, dtype=np.uint32))
    oracle2 = orc.OracleModel(cfg.as_dict(), oracle.tensors)
    want_s, _ = oracle_run(oracle2, prompt, steps, cfg, placed(cfg, edits, len(prompt) - 1))
    assert np.array_equal(original, want_o)
    assert np.array_equal(steered, want_s)
    # The pins act: the last step's candidate logits differ (a random-init
    # model may keep its argmax, so the tokens alone need not).
    assert not np.array_equal(cand_o[0::2], cand_s[0::2])
    # And the original reply again, after the steered run, from the cached
    # prompt: the same tokens (the cache is rewound where the edits act).
    again = model.generate(prompt, (), max_tokens=steps)
    assert np.array_equal(again, original)
    model.close()


def test_seeded_sampling_token_identical(device):
    cfg = small_config()
    model, oracle = build_pair(device, cfg, seed=17)
    rng = np.random.default_rng(9)
    prompt = rng.integers(0, cfg.vocab, 30).astype(np.uint32)
    samp = fz.sampling(temperature=1.0, top_k=64, top_p=1.0, min_p=0.0, seed=0xC0FFEE)
    steps = 20
    want, _ = oracle_run(oracle, prompt, steps, cfg, greedy=False, samp=samp)
    got = model.generate(prompt, samp=samp, max_tokens=steps)
    assert np.array_equal(got, want)
    model.close()


def test_prompt_reuse_forgotten_after_direct_steps(device):
    # generate() reuses the cached prefix of a repeated prompt; a step made
    # outside it rewrites the caches, so the next generate() starts over.
    cfg = small_config()
    model, oracle = build_pair(device, cfg, seed=13)
    rng = np.random.default_rng(6)
    prompt = rng.integers(0, cfg.vocab, 30).astype(np.uint32)
    first = model.generate(prompt, max_tokens=6)
    model.set_edits(np.zeros(2 * cfg.layers, dtype=np.uint32))
    model.step(0, rng.integers(0, cfg.vocab, 20).astype(np.uint32), logits=False)
    again = model.generate(prompt, max_tokens=6)
    want, _ = oracle_run(oracle, prompt, 6, cfg)
    assert np.array_equal(first, want) and np.array_equal(again, want), (first, again, want)
    model.close()


def test_layer_timing_leaves_generation_exact(device):
    # Timing a layer replays its launches at one position; the next
    # generation starts over and is exact.
    cfg = small_config()
    model, oracle = build_pair(device, cfg, seed=19)
    prompt = np.random.default_rng(20).integers(0, cfg.vocab, 70).astype(np.uint32)
    model.generate(prompt, max_tokens=4)
    for layer in range(cfg.layers):
        assert model.time_layer(layer, len(prompt) + 2, iters=20) > 0
    want, _ = oracle_run(oracle, prompt, 6, cfg)
    assert np.array_equal(model.generate(prompt, max_tokens=6), want)
    model.close()


# ---- GGUF files -------------------------------------------------------------------

def _synth_all(cfg, seed):
    t = {(l, r): fz.synth_tensor(cfg, seed, l, r) for l in range(cfg.layers) for r in ROLES}
    t[(-1, "embedding")] = fz.synth_tensor(cfg, seed, -1, "embedding")
    t[(-1, "output_norm")] = fz.synth_tensor(cfg, seed, -1, "output_norm")
    return t


def test_gguf_file_loads_the_same_model(device, tmp_path):
    # A model read from a GGUF file (frz_model_load_gguf) is the model its
    # tensors make when uploaded one by one: same logits, same tokens.
    from frizzle_amd import gguf
    cfg = small_config()
    t = _synth_all(cfg, 31)
    path = gguf.write_gemma3(tmp_path / "m.gguf", cfg, lambda l, r: t[(l, r)].tobytes())
    fc = gguf.Index.open(path).gemma3_config(context=cfg.context)
    for name in ("hidden", "ffn", "head_dim", "query_heads", "kv_heads", "layers", "vocab",
                 "window", "pattern"):
        assert getattr(fc, name) == getattr(cfg, name), name
    a, _ = build_pair(device, cfg, 31)
    b = fz.Model(device, cfg)
    b.load_gguf(path)
    prompt = np.random.default_rng(3).integers(0, cfg.vocab, 40).astype(np.uint32)
    ta = a.generate(prompt, max_tokens=12)
    la = a.logits()
    tb = b.generate(prompt, max_tokens=12)
    lb = b.logits()
    assert np.array_equal(ta, tb)
    assert_same_bits(lb, la, "logits after 12 tokens")
    a.close()
    b.close()


def test_gguf_load_refusals(device, tmp_path):
    from frizzle_amd import gguf
    cfg = small_config()
    t = _synth_all(cfg, 32)
    model = fz.Model(device, cfg)
    # a format this backend does not run for the role, named with its tensor
    q8 = lambda l, r: (np.zeros(cfg.ffn * cfg.hidden // 32 * 34, np.uint8).tobytes()
                       if (l, r) == (1, "gate") else t[(l, r)].tobytes())
    p = gguf.write_gemma3(tmp_path / "q8.gguf", cfg, q8,
                          formats={"blk.1.ffn_gate.weight": gguf.T_Q8_0})
    with pytest.raises(fz.FrzError, match="blk.1.ffn_gate.weight: format Q8_0"):
        model.load_gguf(p)
    # another model's shapes
    other = small_config(layers=2)
    t2 = _synth_all(other, 32)
    p = gguf.write_gemma3(tmp_path / "two.gguf", other, lambda l, r: t2[(l, r)].tobytes())
    with pytest.raises(fz.FrzError, match="shapes are not the model's"):
        model.load_gguf(p)
    # a missing tensor
    ts = [(n, d, f, b) for n, d, f, b in _gemma3_tensors(cfg, t) if n != "blk.2.ffn_up.weight"]
    p = gguf.write(tmp_path / "missing.gguf", ts, _gemma3_meta(cfg))
    with pytest.raises(fz.FrzError, match="missing tensor blk.2.ffn_up.weight"):
        model.load_gguf(p)
    # a malformed file, named by its rule
    whole = (tmp_path / "two.gguf").read_bytes()
    first = min(d["offset"] for d in gguf.Index.open(tmp_path / "two.gguf").tensors)
    p = tmp_path / "cut.gguf"
    p.write_bytes(whole[:first + 100])  # the index whole, the data cut
    with pytest.raises(fz.FrzError, match="tensor data lies outside the file"):
        model.load_gguf(p)
    model.close()


# ---- the pinned file's formats: a Q8_0 embedding (and so head), Q4_1 downs ----

MIXED = {(-1, "embedding"): fz.Q8_0, (0, "down"): fz.Q4_1, (1, "down"): fz.Q4_1,
         (2, "down"): fz.Q8_0}


def _mixed_tensors(cfg, seed):
    t = _synth_all(cfg, seed)
    rng = np.random.default_rng(seed)
    t[(-1, "embedding")] = q8_0_blocks(rng, cfg.vocab, cfg.hidden, scale_std=0.004)
    t[(0, "down")] = q4_1_blocks(rng, cfg.hidden, cfg.ffn, scale_std=0.01)
    t[(1, "down")] = q4_1_blocks(rng, cfg.hidden, cfg.ffn, scale_std=0.01)
    t[(2, "down")] = q8_0_blocks(rng, cfg.hidden, cfg.ffn, scale_std=0.0006)
    return t


def _set_all(model, t, formats):
    for (l, r), a in t.items():
        model.set_tensor(l, r, a, formats.get((l, r)))


def test_mixed_formats_prefill_and_decode_bit_exact(device):
    cfg = small_config()
    t = _mixed_tensors(cfg, 41)
    oracle = orc.OracleModel(cfg.as_dict(), t, formats=MIXED)
    model = fz.Model(device, cfg)
    # First Q4_0 everywhere, decoded once (its graph captured), then the
    # mixed formats: the matrices change format and the graph is captured
    # again over the new buffers.
    _set_all(model, _synth_all(cfg, 41), {})
    model.generate(np.arange(5, dtype=np.uint32), max_tokens=3)
    _set_all(model, t, MIXED)
    rng = np.random.default_rng(8)
    prompt = rng.integers(0, cfg.vocab, 90).astype(np.uint32)
    model.set_edits(np.zeros(2 * cfg.layers, dtype=np.uint32))
    model.step(0, prompt[:41], logits=False)
    model.step(41, prompt[41:], logits=True)
    _, want_logits = oracle_run(oracle, prompt, 0, cfg)
    assert_same_bits(model.logits(), want_logits, "prompt-end logits")
    for l in range(cfg.layers):
        n = oracle.key_cache(l).size
        assert np.array_equal(model.cache(l, False, n), oracle.key_cache(l)), f"keys {l}"
    oracle.close()
    oracle = orc.OracleModel(cfg.as_dict(), t, formats=MIXED)
    steps = 24
    want, _ = oracle_run(oracle, prompt, steps, cfg)
    got = model.generate(prompt, max_tokens=steps)
    assert np.array_equal(got, want), (got, want)
    lg = oracle.token(int(want[-2]), len(prompt) + steps - 2)
    assert_same_bits(model.logits(), lg, "last decode logits")
    model.close()


def test_mixed_formats_gguf_load(device, tmp_path):
    # The file's formats reach the model as they are: a GGUF file with a Q8_0
    # embedding and Q4_1 / Q8_0 downs loads to the model set tensor by tensor;
    # then Q4_0 tensors put the matrices back in Q4_0.
    from frizzle_amd import gguf
    cfg = small_config()
    t = _mixed_tensors(cfg, 43)
    names = {(-1, "embedding"): "token_embd.weight", (0, "down"): "blk.0.ffn_down.weight",
             (1, "down"): "blk.1.ffn_down.weight", (2, "down"): "blk.2.ffn_down.weight"}
    path = gguf.write_gemma3(tmp_path / "mixed.gguf", cfg, lambda l, r: t[(l, r)].tobytes(),
                             formats={names[k]: f for k, f in MIXED.items()})
    a = fz.Model(device, cfg)
    _set_all(a, t, MIXED)
    b = fz.Model(device, cfg)
    b.load_gguf(path)
    prompt = np.random.default_rng(4).integers(0, cfg.vocab, 30).astype(np.uint32)
    ta, tb = a.generate(prompt, max_tokens=10), b.generate(prompt, max_tokens=10)
    assert np.array_equal(ta, tb)
    assert_same_bits(b.logits(), a.logits(), "logits after 10 tokens")
    q = _synth_all(cfg, 44)
    _set_all(b, q, {})
    c, _ = build_pair(device, cfg, 44)
    assert np.array_equal(b.generate(prompt, max_tokens=10), c.generate(prompt, max_tokens=10))
    assert_same_bits(b.logits(), c.logits(), "back in Q4_0")
    for m in (a, b, c):
        m.close()


def test_set_tensor_format_refusals(device):
    cfg = small_config()
    model = fz.Model(device, cfg)
    rng = np.random.default_rng(2)
    q8 = q8_0_blocks(rng, cfg.ffn, cfg.hidden)
    with pytest.raises(fz.FrzError, match="format 8 is not run for this role"):
        model.set_tensor(0, "gate", q8, fz.Q8_0)
    with pytest.raises(fz.FrzError, match="format 3 is not run for this role"):
        model.set_tensor(-1, "embedding", q4_1_blocks(rng, cfg.vocab, cfg.hidden), fz.Q4_1)
    with pytest.raises(fz.FrzError, match="wrong size"):
        model.set_tensor(0, "down", q8[:-34], fz.Q8_0)
    model.close()


def _gemma3_tensors(cfg, t):
    from frizzle_amd import gguf
    out = [("token_embd.weight", [cfg.hidden, cfg.vocab], gguf.T_Q4_0,
            t[(-1, "embedding")].tobytes())]
    for l in range(cfg.layers):
        for role, leaf in gguf.LAYER_NAMES.items():
            fmt = gguf.T_F32 if "norm" in role else gguf.T_Q4_0
            out.append((f"blk.{l}.{leaf}", gguf._extents(cfg, role), fmt, t[(l, role)].tobytes()))
    out.append(("output_norm.weight", [cfg.hidden], gguf.T_F32, t[(-1, "output_norm")].tobytes()))
    return out


def _gemma3_meta(cfg):
    from frizzle_amd import gguf
    return [("general.architecture", gguf.STRING, "gemma3"),
            ("gemma3.block_count", gguf.U32, cfg.layers),
            ("gemma3.embedding_length", gguf.U32, cfg.hidden),
            ("gemma3.feed_forward_length", gguf.U32, cfg.ffn),
            ("gemma3.attention.head_count", gguf.U32, cfg.query_heads),
            ("gemma3.attention.head_count_kv", gguf.U32, cfg.kv_heads),
            ("gemma3.attention.key_length", gguf.U32, cfg.head_dim),
            ("gemma3.attention.layer_norm_rms_epsilon", gguf.F32, cfg.epsilon),
            ("gemma3.rope.freq_base", gguf.F32, cfg.rope_global),
            ("gemma3.attention.sliding_window", gguf.U32, cfg.window),
            ("gemma3.attention.sliding_window_pattern", gguf.U32, cfg.pattern)]
