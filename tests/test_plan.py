"""The residency plan (frz_plan_gemma3) against the reference's contract
(src/core/residency/plan.h:14-121, 305-326) and load policy
(src/core/policy/policy.h:23-76), on the CPU.

The reference holds no fixture of its own for the plan; its header states
the counts for the pinned Gemma-3-1B file (plan.h:103-118, 153-158), and
those pin the restatement here: the pinned file's index is rebuilt from its
published shapes and formats (a Q8_0 embedding, Q4_1 downs in layers 0-2,
Q4_0 matrices elsewhere, F32 norms, tensors in name order within a layer), as
a front of header and index alone, read with the whole file's size declared.
The context offered is checked against the cost's closed form at budgets
between its steps.
"""
import numpy as np
import pytest

from frizzle_amd import gguf
from frizzle_amd import plan as fp

MIB = 1 << 20
Q4_0, Q4_1, Q8_0, F32 = gguf.T_Q4_0, gguf.T_Q4_1, gguf.T_Q8_0, gguf.T_F32
BLOCK = {Q4_0: (32, 18), Q4_1: (32, 20), Q8_0: (32, 34), F32: (1, 4)}
H, F, D, QH, V, L = 1152, 6912, 256, 4, 262144, 26


def _bytes(fmt, dims):
    n = int(np.prod(dims))
    per, size = BLOCK[fmt]
    return n // per * size


def pinned_tensors(down_formats=None, q_format=Q4_0, layers=L):
    """The pinned file's tensors as (name, extents, format, bytes): the
    embedding first, each layer's in name order, the output norm last."""
    down_formats = down_formats or {0: Q4_1, 1: Q4_1, 2: Q4_1}
    out = [("token_embd.weight", [H, V], Q8_0)]
    for l in range(layers):
        leaves = {
            "attn_k.weight": ([H, D], Q4_0), "attn_k_norm.weight": ([D], F32),
            "attn_norm.weight": ([H], F32), "attn_output.weight": ([QH * D, H], Q4_0),
            "attn_q.weight": ([H, QH * D], q_format), "attn_q_norm.weight": ([D], F32),
            "attn_v.weight": ([H, D], Q4_0), "ffn_down.weight": ([F, H], down_formats.get(l, Q4_0)),
            "ffn_gate.weight": ([H, F], Q4_0), "ffn_norm.weight": ([H], F32),
            "ffn_up.weight": ([H, F], Q4_0), "post_attention_norm.weight": ([H], F32),
            "post_ffw_norm.weight": ([H], F32)}
        for leaf in sorted(leaves):
            dims, fmt = leaves[leaf]
            out.append((f"blk.{l}.{leaf}", dims, fmt))
    out.append(("output_norm.weight", [H], F32))
    return [(n, d, f, _bytes(f, d)) for n, d, f in out]


def metadata(trained=32768, layers=L):
    return [("general.architecture", gguf.STRING, "gemma3"),
            ("gemma3.block_count", gguf.U32, layers),
            ("gemma3.context_length", gguf.U32, trained),
            ("gemma3.embedding_length", gguf.U32, H),
            ("gemma3.feed_forward_length", gguf.U32, F),
            ("gemma3.attention.head_count", gguf.U32, QH),
            ("gemma3.attention.head_count_kv", gguf.U32, 1),
            ("gemma3.attention.key_length", gguf.U32, D),
            ("gemma3.attention.layer_norm_rms_epsilon", gguf.F32, 1e-6),
            ("gemma3.rope.freq_base", gguf.F32, 1e6),
            ("gemma3.attention.sliding_window", gguf.U32, 512),
            ("gemma3.attention.sliding_window_pattern", gguf.U32, 6)]


def pinned_index(**kw):
    trained = kw.pop("trained", 32768)
    layers = kw.get("layers", L)
    front, size = gguf.index_only(pinned_tensors(**kw), metadata(trained, layers))
    return gguf.Index.read(front, size)


def webgpu(binding=128 * MIB, buffer=256 * MIB, align=256):
    return fp.limits(buffer, binding, align)


@pytest.fixture(scope="module")
def index():
    return pinned_index()


@pytest.fixture(scope="module")
def plan(index):
    return fp.Plan(index, webgpu())


def test_policy_defaults():
    # policy.h: 2 GiB, a 4,096-token rollback reserve.
    p = fp.default_policy()
    assert p.memory_budget == 2 << 30 and p.rollback_reserve == 4096


def test_pinned_file_counts(index, plan):
    # plan.h:103-111: 340 tensors, 715,385,344 bytes before padding; 342
    # pieces, the Q8_0 embedding's 320,864,256 bytes in three of at most
    # 109,655 rows; 52 groups.
    ts = index.tensors
    assert len(ts) == 340 == plan.summary["tensors"]
    assert sum(t["bytes"] for t in ts) == 715_385_344
    assert plan.summary["pieces"] == 342
    emb = plan.pieces(plan.role(-1, "embedding"))
    assert [rows for _, _, rows in emb] == [109_655, 109_655, 262_144 - 2 * 109_655]
    assert sum(r[2] for r, _, _ in emb) >= 320_864_256
    assert plan.summary["groups"] == 52


def test_pinned_group_spans(index, plan):
    # plan.h:110-111: a QKV span runs from attn_k to attn_v and holds
    # attn_output and three norms between, 1,665,536 bytes before padding;
    # gate and up hold ffn_norm between, 8,962,560.
    ts = index.tensors
    groups = plan.groups()
    for l in range(L):
        q, k, v = (plan.role(l, r) for r in ("q", "k", "v"))
        gate, up = plan.role(l, "gate"), plan.role(l, "up")
        qkv = [g for g in groups if g.members == (q, k, v)]
        gu = [g for g in groups if g.members == (gate, up)]
        assert len(qkv) == 1 and len(gu) == 1
        lo, hi = min(q, k, v), max(q, k, v)
        assert ts[lo]["name"].endswith("attn_k.weight") and ts[hi]["name"].endswith("attn_v.weight")
        assert sum(t["bytes"] for t in ts[lo:hi + 1]) == 1_665_536
        assert sum(t["bytes"] for t in ts[gate:up + 1]) == 8_962_560
        # the span is the members' pieces, first byte to last, in one buffer
        for g in qkv + gu:
            pieces = [plan.pieces(m)[0][0] for m in g.members]
            assert {p[0] for p in pieces} == {g.span[0]}
            assert g.span[1] == min(p[1] for p in pieces)
            assert g.span[1] + g.span[2] == max(p[1] + p[2] for p in pieces)
            assert g.span[2] <= 128 * MIB


def test_pinned_cache_and_context(plan):
    # plan.h:153-158: at the trained 32,768 tokens, F16, reserve 4,096: 22
    # sliding layers of 5,120 slots and 4 global of 32,768, 1 KiB a slot for
    # keys and values, 238 MiB; within 2 GiB the whole trained context.
    assert plan.context_offered == 32768 == plan.summary["trained_context"]
    slots = [plan.cache(l)[2] for l in range(L)]
    assert slots == [32768 if l % 6 == 5 else 5120 for l in range(L)]
    assert plan.summary["cache_bytes"] == (22 * 5120 + 4 * 32768) * 1024 == 249_561_088
    for l in range(L):
        keys, values, n = plan.cache(l)
        assert keys[2] == values[2] == n * D * 2


def test_ranges_obey_the_limits(index, plan):
    # Every range aligned, a multiple of 4 long, within one binding and its
    # buffer; ranges of a buffer disjoint; pools never share a buffer.
    bufs = plan.buffers()
    limit = 128 * MIB
    owners = {}

    def take(r, pool, what):
        b, off, n = r
        assert off % 256 == 0 and n % 4 == 0 and n <= limit, what
        assert off + n <= bufs[b][1] <= 256 * MIB, what
        assert bufs[b][0] == pool, what
        owners.setdefault(b, []).append((off, off + n, what))

    for i, t in enumerate(index.tensors):
        for r, first, rows in plan.pieces(i):
            take(r, fp.WEIGHTS, t["name"])
    for l in range(L):
        k, v, _ = plan.cache(l)
        take(k, fp.CACHE, f"keys {l}")
        take(v, fp.CACHE, f"values {l}")
    names = ["hidden", "normed", "query", "key", "value", "attention", "partials",
             "partial_stats", "output", "activation", "logits", "partials_a", "partials_b",
             "candidates", "sampled", "range_sums", "edit_table", "captures"]
    for n in names:
        r = plan.scratch(n)
        take(r, fp.SCRATCH, n)
        assert r[1] == 0 and bufs[r[0]][1] == r[2]  # alone in its buffer
    for b, spans in owners.items():
        spans.sort()
        for (a0, a1, wa), (b0, b1, wb) in zip(spans, spans[1:]):
            assert a1 <= b0, (wa, wb)
    assert plan.summary["scratch"] == 18
    assert sum(size for _, size in bufs) == plan.summary["total_bytes"]


def test_working_set_sizes(plan):
    # graph.cpp:132-198 for Gemma-3-1B: 512 rows of each activation, one
    # row of logits, the selection's two passes over 1,024-entry tiles, the
    # split products' range sums (13.5 MiB, the output and down
    # projections at 96 tokens: matmul.h:255-257), the edit table.
    want = {"hidden": 512 * H, "normed": 512 * H, "query": 512 * 1024, "key": 512 * D,
            "value": 512 * D, "attention": 512 * 1024, "partials": 512 * 1024,
            "partial_stats": 512 * 8, "output": 512 * H, "activation": 512 * F,
            "logits": V, "partials_a": 2 * 64 * 256, "partials_b": 2 * 64 * 16,
            "candidates": 128, "sampled": 4, "range_sums": 96 * H * 32,
            "edit_table": 2 * L + 5 * 4096}
    for name, floats in want.items():
        assert plan.scratch(name)[2] == floats * 4, name
    assert plan.scratch("range_sums")[2] == int(13.5 * MIB)
    assert plan.summary["partial_rows"] == 512


def _fixed(plan):
    """Weights, working buffers and the cache's most padding (plan.h:86-90)."""
    s = plan.summary
    return s["weight_bytes"] + s["scratch_bytes"] + 2 * L * (256 + 4)


def _context_for(fixed, budget, trained=32768, ring=5120):
    """The largest context whose cost fits the budget (None if 512 does not):
    22 sliding layers of min(c, ring) slots and 4 global of c, keys and
    values of 512 bytes a slot."""
    best = None
    for c in range(512, trained + 1):
        if fixed + 2 * 512 * (22 * min(c, ring) + 4 * c) <= budget:
            best = c
    return best


def test_context_offered_is_the_largest_that_fits(index, plan):
    fixed = _fixed(plan)
    for budget in (fixed + 20 * MIB, fixed + 60 * MIB, fixed + 111 * MIB, fixed + 150 * MIB,
                   fixed + 237 * MIB):
        want = _context_for(fixed, budget)
        got = fp.Plan(index, webgpu(), fp.policy(memory_budget=budget))
        assert got.context_offered == want, budget
        assert got.summary["total_bytes"] <= budget
        global_slots = got.cache(5)[2]
        assert global_slots == want and got.cache(0)[2] == min(want, 5120)


def test_exceeds_budget_states_what_512_needs(index, plan):
    needed = _fixed(plan) + 2 * 512 * 26 * 512
    ok = fp.Plan(index, webgpu(), fp.policy(memory_budget=needed))
    assert ok.context_offered == 512
    with pytest.raises(fp.PlanRefused) as e:
        fp.Plan(index, webgpu(), fp.policy(memory_budget=needed - 1))
    assert e.value.error == "ExceedsBudget"
    assert e.value.summary["total_bytes"] == needed


def test_rollback_reserve_sizes_the_sliding_rings(index):
    p = fp.Plan(index, webgpu(), fp.policy(rollback_reserve=0))
    assert [p.cache(l)[2] for l in range(6)] == [1024] * 5 + [32768]
    cfg = p.config()
    assert cfg.local_slots == 1024 and cfg.context == 32768 and cfg.window == 512


def test_rings_are_cut_to_a_shorter_context():
    p = fp.Plan(pinned_index(trained=2048), webgpu())
    assert p.config().local_slots == 2048 == p.cache(0)[2]


def test_row_wider_than_a_binding_is_refused_by_name(index):
    # The embedding's Q8_0 row is 1,224 bytes: a 1,024-byte binding cannot
    # hold it, and it comes first in file order.
    with pytest.raises(fp.PlanRefused) as e:
        fp.Plan(index, webgpu(binding=1024))
    assert e.value.error == "RowExceedsBinding" and e.value.subject == "token_embd.weight"


def test_working_buffer_wider_than_a_binding_is_refused_by_name(index):
    # 4 MiB holds every weight row and the first nine working buffers; the
    # activation (512 x 6,912 floats) does not fit.
    with pytest.raises(fp.PlanRefused) as e:
        fp.Plan(index, webgpu(binding=4 * MIB, buffer=4 * MIB))
    assert e.value.error == "ScratchExceedsBinding" and e.value.subject == "activation"


def test_groups_need_one_format_and_width():
    # A Q8_0 attn_q cannot join its layer's Q4_0 K and V: 26 QKV groups
    # fewer, the gate/up groups kept.
    ix = pinned_index(q_format=Q8_0)
    p = fp.Plan(ix, webgpu())
    assert p.summary["groups"] == 26
    assert all(len(g.members) == 2 for g in p.groups())


def test_large_limits_keep_every_tensor_whole(index):
    # A device granting large buffers (this backend's own limits) keeps
    # every tensor in one piece, in one weights buffer.
    p = fp.Plan(index, fp.limits(1 << 40, 1 << 40, 256))
    assert p.summary["pieces"] == 340
    weights = [b for b in p.buffers() if b[0] == fp.WEIGHTS]
    assert len(weights) == 1


def test_shorter_trained_context():
    ix = pinned_index(trained=2048)
    p = fp.Plan(ix, webgpu())
    assert p.context_offered == 2048
    assert [p.cache(l)[2] for l in range(6)] == [2048] * 6


def test_file_that_is_no_gemma3_is_refused():
    ts = pinned_tensors()
    md = [m for m in metadata() if m[0] != "gemma3.context_length"]
    front, size = gguf.index_only(ts, md)
    with pytest.raises(fp.PlanRefused) as e:
        fp.Plan(gguf.Index.read(front, size), webgpu())
    assert e.value.error == "NotDescribed" and "context_length" in e.value.subject


def test_context_at_the_rings_edges(index, plan):
    # The cost bends where the context reaches the sliding rings' 5,120
    # slots: budgets a byte either side of each side of the bend, and of the
    # trained context's whole cost.
    fixed = _fixed(plan)
    for c in (5119, 5120, 5121, 32767, 32768):
        cost = fixed + 2 * 512 * (22 * min(c, 5120) + 4 * c)
        for budget in (cost - 1, cost, cost + 1):
            got = fp.Plan(index, webgpu(), fp.policy(memory_budget=budget))
            assert got.context_offered == _context_for(fixed, budget), (c, budget)


def test_context_held_to_what_a_binding_holds(index):
    # With 15 MiB bindings a global layer's keys (512 bytes a slot) hold at
    # most 30,720 slots, whatever the budget allows; the sliding rings' 5,120
    # slots (2.5 MiB) are unaffected.
    p = fp.Plan(index, fp.limits(300 * MIB, 15 * MIB, 16), fp.policy(memory_budget=8 << 30))
    assert p.context_offered == 30720
    assert p.cache(5)[2] == 30720 and p.cache(5)[0][2] == 15 * MIB
    assert p.cache(0)[2] == 5120
