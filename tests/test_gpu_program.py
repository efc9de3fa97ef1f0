"""Steps through the program boundary (frz_program_build / run / poll) give
the bits frz_generate gives: the graph's launch list (graph::Builder's for
Gemma 3) built over a model created from the plan, a prompt in 512-token
steps, then fed decode steps two in flight, each reported in run order with
the draw's record; an edit table written as a run input into the plan's
edit_table buffer steers as generate's edits do; the capture store is
written at the prompt's end. Refusals, cancellation and a lost device
(marked from the host; nothing faults) report as the reference's
ProgramError does (program.h:264-278)."""
import numpy as np
import pytest

import frizzle_amd as fz
from frizzle_amd import gguf
from frizzle_amd import plan as fp
from frizzle_amd import program as fprog
from helpers import assert_same_bits
from test_gpu_model import ROLES

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def setup(device, tmp_path_factory):
    cfg = fz.gemma3_1b_config(layers=3, vocab=4096, window=64, pattern=3, context=1024)
    t = {(l, r): fz.synth_tensor(cfg, 81, l, r) for l in range(cfg.layers) for r in ROLES}
    t[(-1, "embedding")] = fz.synth_tensor(cfg, 81, -1, "embedding")
    t[(-1, "output_norm")] = fz.synth_tensor(cfg, 81, -1, "output_norm")
    path = gguf.write_gemma3(tmp_path_factory.mktemp("prog") / "m.gguf", cfg,
                             lambda l, r: t[(l, r)].tobytes())
    plan = fp.Plan(gguf.Index.open(path), fp.device_limits(device))
    return cfg, path, plan


def _model(device, plan, path):
    m = fz.Model.planned(device, plan)
    m.load_gguf(path)
    return m


def _run_turn(prog, prompt, steps, samp=None, inputs=()):
    """The turn loop over the program (turn.cpp:22-40): prompt blocks of
    512, logits on the last, then fed decode steps, at most two
    outstanding; the tokens the reports carry, in order."""
    base = len(prog.reports)
    for at in range(0, len(prompt), 512):
        part = prompt[at:at + 512]
        last = at + len(part) == len(prompt)
        assert prog.run(fprog.step_record(at, part, logits=last, samp=samp),
                        inputs if at == 0 else ()) == 0
        while prog.outstanding >= 2:
            prog.poll(wait=True)
    issued, pos = 0, len(prompt)
    while issued < steps - 1:
        while prog.outstanding < 2 and issued < steps - 1:
            assert prog.run(fprog.step_record(pos, fed=True, logits=True, samp=samp)) == 0
            pos += 1
            issued += 1
        prog.poll(wait=True)
    while prog.outstanding:
        prog.poll(wait=True)
    reports = prog.reports[base:]
    assert all(r[0] == fprog.OK for r in reports), reports
    return np.array([r[2][0] for r in reports if r[2] is not None], dtype=np.uint32)


def test_program_steps_are_generate(device, setup):
    cfg, path, plan = setup
    a, b = _model(device, plan, path), _model(device, plan, path)
    prog = fprog.Program(a, plan)
    prompt = np.random.default_rng(82).integers(0, cfg.vocab, 700).astype(np.uint32)
    got = _run_turn(prog, prompt, 40)
    want = b.generate(prompt, max_tokens=40)
    assert np.array_equal(got, want), (got, want)
    assert_same_bits(a.logits(), b.logits(), "last logits")
    # seeded sampling, from one seed, as generate draws
    samp = fz.sampling(temperature=1.0, top_k=64, top_p=0.95, min_p=0.05, seed=0xABC)
    got = _run_turn(prog, prompt, 24, samp)
    want = b.generate(prompt, samp=samp, max_tokens=24)
    assert np.array_equal(got, want), (got, want)
    prog.close()
    a.close()
    b.close()


def test_program_steps_in_the_fast_prefill_mode(device, setup):
    """A model in the fast prefill mode runs the program's prompt steps on
    the bf16 matrix cores, as its own generate does: the same tokens and
    last logits, bit for bit (the decode steps are exact in both). The
    program writes the capture store at the prompt's end, and a step that
    captures takes the exact attention (the store's per-key weights come
    from it), so generate's model captures too."""
    cfg, path, plan = setup
    a, b = _model(device, plan, path), _model(device, plan, path)
    a.set_prefill(fz.PREFILL_BF16)
    b.set_prefill(fz.PREFILL_BF16)
    b.set_capture(True)
    prog = fprog.Program(a, plan)
    prompt = np.random.default_rng(83).integers(0, cfg.vocab, 700).astype(np.uint32)
    got = _run_turn(prog, prompt, 16)
    want = b.generate(prompt, max_tokens=16)
    assert np.array_equal(got, want), (got, want)
    assert_same_bits(a.logits(), b.logits(), "last logits")
    prog.close()
    a.close()
    b.close()


def test_program_edit_table_as_a_run_input(device, setup):
    cfg, path, plan = setup
    a, b = _model(device, plan, path), _model(device, plan, path)
    prog = fprog.Program(a, plan)
    prompt = np.random.default_rng(83).integers(0, cfg.vocab, 120).astype(np.uint32)
    edits = [fz.Edit(1, 77, fz.EditKind.SET, 9.5), fz.Edit(2, 3000, fz.EditKind.SCALE, -4.0, 2)]
    placed = fz.edit_table(edits, cfg.layers, len(prompt) - 1)
    et = plan.scratch("edit_table")
    got = _run_turn(prog, prompt, 20, inputs=[((et[0], et[1], placed.nbytes), placed.tobytes())])
    want = b.generate(prompt, edits, max_tokens=20)
    assert np.array_equal(got, want), (got, want)
    steered = b.logits()
    assert_same_bits(a.logits(), steered, "steered last logits")
    # the pins act: the plain run's logits differ (a random-init model may
    # keep its argmax, so the tokens need not)
    b.generate(prompt, max_tokens=20)
    assert not np.array_equal(b.logits().view(np.uint32), steered.view(np.uint32))
    prog.close()
    a.close()
    b.close()


def test_program_writes_the_capture_store(device, setup):
    cfg, path, plan = setup
    a, b = _model(device, plan, path), _model(device, plan, path)
    prog = fprog.Program(a, plan)
    prompt = np.random.default_rng(84).integers(0, cfg.vocab, 90).astype(np.uint32)
    _run_turn(prog, prompt, 1)
    b.set_capture(True)
    b.generate(prompt, max_tokens=1)
    assert np.array_equal(a.capture()[0], b.capture()[0])
    prog.close()
    a.close()
    b.close()


def test_program_refusals_and_order(device, setup):
    cfg, path, plan = setup
    a = _model(device, plan, path)
    prog = fprog.Program(a, plan)
    ids = np.arange(10, 20, dtype=np.uint32)
    # two outstanding: a third is refused at once, unnumbered
    assert prog.run(fprog.step_record(0, ids, logits=False), tag=1) == 0
    assert prog.run(fprog.step_record(10, ids, logits=True), tag=2) == 0
    assert prog.run(fprog.step_record(20, ids, logits=True), tag=3) == fprog.STEP
    assert prog.reports[-1][0] == fprog.STEP and "two steps are outstanding" in prog.reports[-1][1]
    while prog.outstanding:
        prog.poll(wait=True)
    assert [r[0] for r in prog.reports[-2:]] == [0, 0]
    assert [r[3] for r in prog.reports[-2:]] == [1, 2]  # in run order
    assert prog.reports[-1][2] is not None and prog.reports[-2][2] is None
    # steps of 0 or 513 tokens: refused at once
    rec = fprog.step_record(0, ids)
    rec.tokens = 513
    assert prog.run(rec) == fprog.STEP and "513 tokens" in prog.reports[-1][1]
    # past the context, and an input outside its buffer: failed, reported in order
    n = len(prog.reports)
    assert prog.run(fprog.step_record(1020, ids, logits=True), tag=4) == 0
    et = plan.scratch("edit_table")
    assert prog.run(fprog.step_record(0, ids), [((et[0], et[1] + et[2] - 4, 8), b"\0" * 8)],
                    tag=5) == 0
    while prog.outstanding:
        prog.poll(wait=True)
    assert [(r[0], r[3]) for r in prog.reports[n:]] == [(fprog.STEP, 4), (fprog.STEP, 5)]
    assert "past the context" in prog.reports[n][1]
    assert "outside its buffer" in prog.reports[n + 1][1]
    # a fed step is one token, the last step's draw: a fed step of 3 tokens
    # fails, reported in order, nothing run
    n = len(prog.reports)
    rec = fprog.step_record(20, fed=True, logits=True)
    rec.tokens = 3
    assert prog.run(rec, tag=6) == 0
    prog.poll(wait=True)
    assert [(r[0], r[3]) for r in prog.reports[n:]] == [(fprog.STEP, 6)]
    assert "a fed step of 3 tokens" in prog.reports[n][1]
    prog.close()
    a.close()


def test_program_cancel_and_lost_device(device, setup):
    cfg, path, plan = setup
    a = _model(device, plan, path)
    prog = fprog.Program(a, plan)
    prompt = np.random.default_rng(85).integers(0, cfg.vocab, 512).astype(np.uint32)
    prog.run(fprog.step_record(0, prompt[:256]), tag=1)
    prog.run(fprog.step_record(256, prompt[256:], logits=True), tag=2)
    n = len(prog.reports)
    prog.cancel()
    assert [(r[0], r[3]) for r in prog.reports[n:]] == [(fprog.CANCELLED, 1),
                                                        (fprog.CANCELLED, 2)]
    # still usable after a cancel
    prog.run(fprog.step_record(0, prompt[:100], logits=True), tag=3)
    prog.poll(wait=True)
    assert prog.reports[-1][0] == fprog.OK and prog.reports[-1][2] is not None
    # a device marked lost: the outstanding step reports DEVICE_LOST, new
    # steps are refused so
    prog.run(fprog.step_record(100, prompt[100:200], logits=True), tag=4)
    prog.mark_lost()
    prog.poll(wait=True)
    assert prog.reports[-1][0] == fprog.DEVICE_LOST and prog.reports[-1][2] is None
    assert prog.run(fprog.step_record(200, prompt[200:300])) == fprog.DEVICE_LOST
    assert prog.reports[-1][0] == fprog.DEVICE_LOST
    prog.close()
    # destroying with steps in flight reports them cancelled
    prog2 = fprog.Program(a, plan)
    prog2.run(fprog.step_record(0, prompt[:300], logits=True), tag=6)
    reports = prog2.reports
    prog2.close()
    assert [(r[0], r[3]) for r in reports] == [(fprog.CANCELLED, 6)]
    a.close()


def test_program_refuses_another_models_buffers(device, setup, tmp_path):
    cfg, path, plan = setup
    other = fz.Model(device, cfg)
    with pytest.raises(fprog.BuildRefused, match="not created from this plan"):
        fprog.Program(other, plan)
    other.close()
