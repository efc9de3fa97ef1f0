"""The program's build checks on the CPU (frz_program_check): the launch
list graph::Builder emits for Gemma 3 over a plan is accepted, and each of
Program::build's refusals (program.h:29-41) and each departure from the
graph (a missing or misplaced stage, a stage bound to another layer's
weights, a launch past the end) is refused with a message naming the
launch."""
import copy

import pytest

from frizzle_amd import graph
from frizzle_amd import plan as fp
from frizzle_amd import program as fprog
from test_plan import pinned_index


@pytest.fixture(scope="module")
def plan():
    return fp.Plan(pinned_index(), fp.limits(1 << 40, 1 << 40, 256))


@pytest.fixture(scope="module")
def launches(plan):
    return graph.gemma3_launches(plan)


def _refused(plan, launches, readback, match):
    rc, msg = fprog.check_launches(plan, launches, readback)
    assert rc == fprog.BUILD, msg
    assert match in msg, msg
    return msg


def _index(ls, role, layer=graph.NO_LAYER):
    return next(i for i, l in enumerate(ls) if l.role == role and l.layer == layer)


def test_the_gemma3_graph_is_accepted(plan, launches):
    ls, rb = launches
    assert fprog.check_launches(plan, ls, rb) == (0, "")
    # the split attention's combine is optional (a step that never splits)
    assert fprog.check_launches(plan, [l for l in ls if l.role != "attention.combine"], rb)[0] == 0
    # at the WebGPU limits, the embedding in three pieces, bound piece by piece
    p2 = fp.Plan(pinned_index(), fp.limits(*fp.WEBGPU_DEFAULT_LIMITS))
    l2, r2 = graph.gemma3_launches(p2)
    assert fprog.check_launches(p2, l2, r2) == (0, "")


@pytest.mark.parametrize("change,match", [
    (lambda l: setattr(l, "constants", b"\0" * 769), "constants over 768 bytes"),
    (lambda l: setattr(l, "workgroup_size", 0), "no invocations"),
    (lambda l: setattr(l, "invocations_per_row", 0), "no invocations"),
    (lambda l: (setattr(l, "rows_per_tile", 8), setattr(l, "rows", graph.LAST)),
     "a tiled launch over the last token"),
    (lambda l: (setattr(l, "rows_per_tile", 3), setattr(l, "invocations_per_row", 8),
                setattr(l, "workgroup_size", 256)), "not a whole number of workgroups"),
    (lambda l: (setattr(l, "key_split", graph.PER_CHUNK), setattr(l, "window", 0)),
     "a key split with no window"),
    (lambda l: l.bindings.append((10_000, 0, 4)), "not within a buffer the upload created"),
    (lambda l: l.bindings.append((0, 1 << 41, 4)), "not within a buffer the upload created"),
])
def test_program_build_refusals(plan, launches, change, match):
    ls, rb = copy.deepcopy(launches)
    i = _index(ls, "ffn.edit", 3)
    change(ls[i])
    msg = _refused(plan, ls, rb, match)
    assert msg.startswith(f"launch {i}")


def test_readback_must_be_the_draws_record(plan, launches):
    ls, rb = launches
    _refused(plan, ls, (rb[0], rb[1], 8), "the draw's 16-byte record")
    _refused(plan, ls, (rb[0], rb[1], 20), "4 to 16 bytes")
    _refused(plan, ls, (rb[0], rb[1] + 2, 16), "4 to 16 bytes")
    _refused(plan, ls, None, "no readback range")


def test_a_missing_stage_is_named(plan, launches):
    ls, rb = copy.deepcopy(launches)
    i = _index(ls, "attention.rope", 3)
    del ls[i]
    _refused(plan, ls, rb, f"launch {i}: expected attention.rope of layer 3, found "
                           "attention.capture of layer 3")


def test_stages_out_of_order_are_refused(plan, launches):
    ls, rb = copy.deepcopy(launches)
    i, j = _index(ls, "ffn.norm", 5), _index(ls, "ffn.edit", 5)
    ls[i], ls[j] = ls[j], ls[i]
    _refused(plan, ls, rb, f"launch {i}: expected ffn.norm of layer 5")


def test_a_stage_bound_to_another_layers_weights_is_refused(plan, launches):
    ls, rb = copy.deepcopy(launches)
    i = _index(ls, "attention.output", 2)
    j = _index(ls, "attention.output", 3)
    ls[i].bindings = copy.deepcopy(ls[j].bindings)
    _refused(plan, ls, rb, f"launch {i} (attention.output of layer 2): binds none of")
    # the cache a layer's attention reads
    ls, rb = copy.deepcopy(launches)
    i = _index(ls, "attention.scores", 4)
    ls[i].bindings = [b for b in ls[i].bindings if b != plan.cache(4)[0]]
    _refused(plan, ls, rb, f"launch {i} (attention.scores of layer 4): binds none of")


def test_a_wrong_kernel_and_trailing_launches_are_refused(plan, launches):
    ls, rb = copy.deepcopy(launches)
    i = _index(ls, "ffn.edit", 1)
    ls[i].kernel = graph.NORM
    _refused(plan, ls, rb, f"launch {i} (ffn.edit of layer 1): kernel 1 is not one this stage runs")
    ls, rb = copy.deepcopy(launches)
    ls.append(copy.deepcopy(ls[-1]))
    ls[-1].role = "output.extra"
    _refused(plan, ls, rb, f"launch {len(ls) - 1} (output.extra): after the graph's last stage")


def test_an_ungrouped_plan_is_refused(launches):
    # A Q8_0 attn_q leaves Q, K and V ungrouped: graph::Builder refuses such
    # a model (UngroupedQueryKeyValue), and so does the program.
    p = fp.Plan(pinned_index(q_format=8), fp.limits(1 << 40, 1 << 40, 256))
    ls, rb = launches
    _refused(p, ls, rb, "did not group Q, K and V of layer 0")


def test_overrides_are_accepted_and_checked(plan, launches):
    # kernels::Launch::overrides (interface.h:310-338): the graph's
    # launches carry the launchers' shape and tile overrides, which this
    # backend accepts and ignores by name; Program::build's refusals
    # (program.cpp:432-444) hold: the program's own names, a name twice.
    ls, rb = copy.deepcopy(launches)
    assert sum(len(l.overrides) for l in ls) > 0
    assert fprog.check_launches(plan, ls, rb) == (0, "")
    i = _index(ls, "ffn.down", 2)
    ls[i].overrides = [("columns", 6912.0), ("anything_else", 1.5)]
    assert fprog.check_launches(plan, ls, rb) == (0, "")
    for bad, match in (([("workgroup_size", 64.0)], "override workgroup_size is the program's to set"),
                       ([("last_token", 1.0)], "override last_token is the program's to set"),
                       ([("columns", 1.0), ("tile_tokens", 8.0), ("columns", 2.0)],
                        "override columns given twice"),
                       ([(None, 1.0)], "override 0 has no name")):
        ls2 = copy.deepcopy(ls)
        ls2[i].overrides = bad
        msg = _refused(plan, ls2, rb, match)
        assert msg.startswith(f"launch {i}")
