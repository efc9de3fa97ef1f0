"""Profiled steps: frz_model_profile_step and frz_model_profile_decode, and
Program::run_profiled through frz_program_run_profiled (program.h:343-372).
Every launch is named by the graph's roles and layer (interface.h:356-362,
graph.h:99-106): the roles of a step's launches, taken in order and split
at "+", are the graph's roles of that step in the graph's order, each
once. A profiled step's results are an unprofiled one's, bit for bit. A
program's profile maps each launch to the graph's last launch it runs, in
the graph's order but for the capture store's readouts; a prefix of a
step, and a profiled step beside an unprofiled one, are refused as the
reference refuses them."""
import numpy as np
import pytest

import frizzle_amd as fz
from frizzle_amd import program as fprog
from helpers import assert_same_bits
from test_gpu_program import _model, setup  # noqa: F401  (the fixture)

pytestmark = pytest.mark.gpu

LAYER_ROLES = ["attention.norm", "attention.qkv", "attention.rope", "attention.scores",
               "attention.combine", "attention.output", "ffn.norm", "ffn.gate_up", "ffn.edit",
               "ffn.down"]
OUTPUT_ROLES = ["output.norm", "output.head", "output.select", "output.draw"]


def _graph_order(layers):
    want = [("embed", 0)]
    for l in range(layers):
        want += [(r, l) for r in LAYER_ROLES]
    return want + [(r, None) for r in OUTPUT_ROLES]


def _flat(launches):
    """The roles of the launches in order, a fused launch's one by one, each
    with its layer (the embedding counted in layer 0, where the decode step
    fuses it)."""
    out = []
    for roles, layer, us in launches:
        assert us > 0.0, (roles, layer, us)
        for r in roles.split("+"):
            out.append((r, 0 if r == "embed" else layer))
    return out


def test_profiled_decode_names_each_launch(device, setup):
    cfg, path, plan = setup
    a, b = _model(device, plan, path), _model(device, plan, path)
    prompt = np.random.default_rng(301).integers(0, cfg.vocab, 100).astype(np.uint32)
    a.step(0, prompt, logits=True)
    b.step(0, prompt, logits=True)
    toks, _ = a.decode(len(prompt), 1)
    launches, tok = b.profile_decode(len(prompt))
    assert tok == int(toks[0])
    assert_same_bits(b.logits(), a.logits(), "logits of a profiled decode step")
    assert _flat(launches) == _graph_order(cfg.layers), launches
    # a decode step fuses every norm into a product: 5 or 6 launches a layer
    assert len(launches) <= 6 * cfg.layers + 2
    a.close()
    b.close()


@pytest.mark.parametrize("mode", [fz.PREFILL_EXACT, fz.PREFILL_BF16])
def test_profiled_prefill_step(device, setup, mode):
    cfg, path, plan = setup
    a, b = _model(device, plan, path), _model(device, plan, path)
    a.set_prefill(mode)
    b.set_prefill(mode)
    prompt = np.random.default_rng(302).integers(0, cfg.vocab, 300).astype(np.uint32)
    a.step(0, prompt, logits=True)
    launches = b.profile_step(0, prompt, logits=True)
    assert_same_bits(b.logits(), a.logits(), "logits of a profiled prefill step")
    assert _flat(launches) == _graph_order(cfg.layers), launches
    a.close()
    b.close()


def test_program_run_profiled(device, setup):
    cfg, path, plan = setup
    a, b = _model(device, plan, path), _model(device, plan, path)
    pa, pb = fprog.Program(a, plan), fprog.Program(b, plan)
    assert pa.can_profile and pa.launch_count > 0
    prompt = np.random.default_rng(303).integers(0, cfg.vocab, 300).astype(np.uint32)
    recs = [fprog.step_record(0, prompt, logits=True)]
    recs += [fprog.step_record(len(prompt) + i, fed=True, logits=True) for i in range(3)]
    for rec in recs:
        assert pa.run_profiled(rec) == 0
        assert pb.run(rec) == 0
        pa.poll(wait=True)
        pb.poll(wait=True)
    assert [r[:3] for r in pa.reports] == [r[:3] for r in pb.reports]
    assert len(pa.profiles) == len(recs)
    for status, begin, end, launches in pa.profiles:
        assert status == fprog.OK and begin == 0 and launches
        ends = [t["end_ns"] for t in launches]
        assert ends == sorted(ends) and end == ends[-1]
        index = [t["graph_index"] for t in launches]
        assert all(0 <= i < pa.launch_count for i in index), index
        # In the graph's order, but for the capture store's readouts, which
        # run after the step's own output here (the graph interleaves layer
        # l's after layer l + 1's Q/K/V); they read the store, nothing the
        # model reads.
        kept = [t["graph_index"] for t in launches if "readout" not in t["roles"]]
        assert kept == sorted(kept), kept
    # the prompt's step captures (the program turns the store on): its
    # capture launches are named too
    roles = {r for t in pa.profiles[0][3] for r in t["roles"].split("+")}
    assert {"attention.capture", "ffn.capture", "readout", "output.readout"} <= roles
    # refused at once: a prefix of the graph's launches, and a profiled step
    # beside an unprofiled one
    rec = fprog.step_record(len(prompt) + 3, fed=True, logits=True)
    assert pa.run_profiled(rec, launches=pa.launch_count - 1) == fprog.STEP
    assert pa.profiles[-1][0] == fprog.STEP and pa.profiles[-1][3] == []
    assert pa.run(rec) == 0
    assert pa.run_profiled(fprog.step_record(len(prompt) + 4, fed=True, logits=True)) == fprog.STEP
    while pa.outstanding:
        pa.poll(wait=True)
    pa.close()
    pb.close()
    a.close()
    b.close()
