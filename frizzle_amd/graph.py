"""The launch list graph::Builder emits for a Gemma 3 model over a residency
plan (src/core/graph/graph.cpp:290-470), as frz_launch records: each
launch's kernel, rows, geometry, the plan ranges it binds, and the role and
layer graph.h names it by. It is what a reference-side shim hands
frz_program_build (kernels::Launch with its WGSL named by a kernel number);
the program recognises the graph in it and runs its fused schedule.

The geometry follows the reference's launchers (SURVEY's kernel table):
products as a decode form (one token) and prefill tiles (two tokens on),
attention split by key chunks with its combine, selection in three passes.
"""
import ctypes
from dataclasses import dataclass, field

from ._lib import ROLE

GATHER, NORM, MATMUL, ROPE, ATTENTION, COMBINE, EDIT, TOPK, DRAW, CAPTURE, WEIGHTS = range(11)
EVERY, LAST, PROMPT_END = 0, 1, 2
NO_SPLIT, PER_CHUNK, WHEN_SPLIT = 0, 1, 2
NO_LAYER = 0xFFFFFFFF
F16 = 1


class CBinding(ctypes.Structure):
    _fields_ = [("buffer", ctypes.c_uint32), ("offset", ctypes.c_uint64),
                ("size", ctypes.c_uint64)]


class COverride(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("value", ctypes.c_double)]


class CLaunch(ctypes.Structure):
    _fields_ = [("kernel", ctypes.c_int), ("entry_point", ctypes.c_char_p),
                ("format", ctypes.c_int), ("pack_format", ctypes.c_int),
                ("constants", ctypes.c_void_p), ("constants_bytes", ctypes.c_uint32),
                ("bindings", ctypes.POINTER(CBinding)), ("binding_count", ctypes.c_uint32),
                ("invocations_per_row", ctypes.c_uint32), ("workgroup_size", ctypes.c_uint32),
                ("rows", ctypes.c_int), ("rows_per_tile", ctypes.c_uint32),
                ("key_split", ctypes.c_int), ("window", ctypes.c_uint32),
                ("partial_rows", ctypes.c_uint32), ("tokens_least", ctypes.c_uint32),
                ("tokens_most", ctypes.c_uint32), ("role", ctypes.c_char_p),
                ("layer", ctypes.c_uint32), ("overrides", ctypes.POINTER(COverride)),
                ("override_count", ctypes.c_uint32)]


@dataclass
class Launch:
    kernel: int
    bindings: list
    role: str
    layer: int = NO_LAYER
    entry: str = "main"
    fmt: int = -1
    pack: int = -1
    invocations_per_row: int = 64
    workgroup_size: int = 64
    rows: int = EVERY
    rows_per_tile: int = 0
    key_split: int = NO_SPLIT
    window: int = 0
    partial_rows: int = 0
    tokens: tuple = (1, 0xFFFFFFFF)
    constants: bytes = field(default=b"")
    overrides: list = field(default_factory=list)  # (name, value): WGSL override constants


def gemma3_launches(plan):
    """(launches, readback): the graph's launches in order, and the draw's
    record, the range each step reads back."""
    cfg = plan.config()
    S = {n: plan.scratch(n) for n in (
        "hidden", "normed", "query", "key", "value", "attention", "partials", "partial_stats",
        "output", "activation", "logits", "partials_a", "partials_b", "candidates", "sampled",
        "range_sums", "edit_table", "captures")}

    def tensor(layer, role):
        t = plan.role(layer, role)
        return [r for r, _, _ in plan.pieces(t)], plan.format(t)

    def group(layer, roles):
        want = tuple(plan.role(layer, r) for r in roles)
        for g in plan.groups():
            if g.members == want:
                return g.span
        raise ValueError(f"layer {layer}: {roles} not grouped")

    emb, emb_fmt = tensor(-1, "embedding")
    onorm, _ = tensor(-1, "output_norm")
    out = []

    def norm(gain, post, rows, role, layer):
        b = gain + (post or []) + [S["output"], S["hidden"], S["normed"], S["captures"]]
        out.append(Launch(NORM, b, role, layer, invocations_per_row=256, workgroup_size=256,
                          rows=rows))

    def product(weights, fmt, inp, outputs, rows, role, layer, epilogue, columns, width):
        # the decode form, then the prefill tiles (matmul.cpp:106-231), with
        # the shape and tile overrides the launcher sets
        b = weights + [inp] + outputs + [S["range_sums"]]
        shape = [("columns", columns), ("out_width", width)]
        decode = shape + [("set_rows", 4 if epilogue == "gated" else 1), ("x_tile_vec4s", 256)]
        if rows == EVERY:
            out.append(Launch(MATMUL, b, role, layer, entry=f"decode_{epilogue}", fmt=fmt,
                              tokens=(1, 1), overrides=decode))
            out.append(Launch(MATMUL, b, role, layer, entry=f"prefill_{epilogue}", fmt=fmt,
                              rows_per_tile=32, invocations_per_row=8, workgroup_size=256,
                              tokens=(2, 0xFFFFFFFF),
                              overrides=shape + [("tile_tokens", 32), ("x_tile_vec4s", 256)]))
        else:
            out.append(Launch(MATMUL, b, role, layer, entry=f"decode_{epilogue}", fmt=fmt,
                              rows=rows, invocations_per_row=4 * 64, workgroup_size=64,
                              overrides=decode))

    def select(rows, role, layer):
        for entry in ("first", "merge", "merge"):
            out.append(Launch(TOPK, [S["logits"], S["partials_a"], S["partials_b"],
                                     S["candidates"]], role, layer, entry=entry,
                              invocations_per_row=256, workgroup_size=256, rows=rows))

    def readout(layer):
        norm(onorm, None, PROMPT_END, "readout", layer)
        product(emb, emb_fmt, S["normed"], [S["logits"]], PROMPT_END, "readout", layer, "write",
                cfg.hidden, cfg.vocab)
        select(PROMPT_END, "readout", layer)
        out.append(Launch(CAPTURE, [S["candidates"], S["captures"]], "readout", layer,
                          rows=PROMPT_END))

    out.append(Launch(GATHER, emb + [S["sampled"], S["hidden"]], "embed", fmt=emb_fmt,
                      invocations_per_row=cfg.hidden // 32))
    pending = None
    q_width = cfg.query_heads * cfg.head_dim
    heads = [("head_dimension", cfg.head_dim), ("query_heads", cfg.query_heads),
             ("key_value_heads", cfg.kv_heads)]
    for l in range(cfg.layers):
        global_layer = l % cfg.pattern == cfg.pattern - 1
        window = cfg.context if global_layer else cfg.window
        keys, values, _ = plan.cache(l)
        gain, _ = tensor(l, "attn_norm")
        norm(gain, pending, EVERY, "attention.norm", l)
        product([group(l, ("q", "k", "v"))], 2, S["normed"], [S["query"], S["key"], S["value"]],
                EVERY, "attention.qkv", l, "qkv", cfg.hidden, q_width)
        if l > 0:
            readout(l - 1)
        qn, _ = tensor(l, "q_norm")
        kn, _ = tensor(l, "k_norm")
        out.append(Launch(ROPE, qn + kn + [S["query"], S["key"], S["value"], keys, values],
                          "attention.rope", l, pack=F16, invocations_per_row=6 * 32,
                          workgroup_size=32,
                          overrides=heads + [("pairs_per_head", cfg.head_dim // 2)]))
        out.append(Launch(CAPTURE, [S["query"], S["captures"]], "attention.capture", l,
                          rows=PROMPT_END))
        ab = [S["query"], keys, values, S["attention"], S["partials"], S["partial_stats"],
              S["captures"]]
        attn = heads + [("partial_rows", 512)]
        out.append(Launch(ATTENTION, ab, "attention.scores", l, key_split=PER_CHUNK,
                          window=window, partial_rows=512, invocations_per_row=64 * 4,
                          workgroup_size=64, overrides=attn))
        out.append(Launch(COMBINE, ab, "attention.combine", l, entry="combine",
                          key_split=WHEN_SPLIT, window=window, partial_rows=512,
                          invocations_per_row=256, workgroup_size=64, overrides=attn))
        out.append(Launch(WEIGHTS, [S["captures"]], "attention.weights", l, rows=PROMPT_END))
        o, _ = tensor(l, "o")
        product(o, 2, S["attention"], [S["output"]], EVERY, "attention.output", l, "write",
                q_width, cfg.hidden)
        fg, _ = tensor(l, "ffn_norm")
        pa, _ = tensor(l, "post_attn_norm")
        norm(fg, pa, EVERY, "ffn.norm", l)
        product([group(l, ("gate", "up"))], 2, S["normed"], [S["activation"]], EVERY,
                "ffn.gate_up", l, "gated", cfg.hidden, cfg.ffn)
        out.append(Launch(EDIT, [S["activation"], S["edit_table"]], "ffn.edit", l))
        out.append(Launch(CAPTURE, [S["activation"], S["captures"]], "ffn.capture", l,
                          rows=PROMPT_END))
        down, down_fmt = tensor(l, "down")
        product(down, down_fmt, S["activation"], [S["output"]], EVERY, "ffn.down", l, "write",
                cfg.ffn, cfg.hidden)
        pending, _ = tensor(l, "post_ffn_norm")
    norm(onorm, pending, LAST, "output.norm", NO_LAYER)
    product(emb, emb_fmt, S["normed"], [S["logits"]], LAST, "output.head", NO_LAYER, "write",
            cfg.hidden, cfg.vocab)
    select(LAST, "output.select", NO_LAYER)
    out.append(Launch(CAPTURE, [S["candidates"], S["captures"]], "output.readout",
                      rows=PROMPT_END))
    out.append(Launch(DRAW, [S["candidates"], S["sampled"]], "output.draw", rows=LAST))
    rb = S["sampled"]
    return out, (rb[0], rb[1], 16)


class CLaunches:
    """A launch list as the C ABI takes it (kept alive with its strings and
    binding arrays)."""

    def __init__(self, launches):
        self._keep = []
        self.array = (CLaunch * len(launches))()
        for i, l in enumerate(launches):
            binds = (CBinding * max(1, len(l.bindings)))(*[CBinding(*b) for b in l.bindings])
            role = l.role.encode()
            entry = l.entry.encode()
            consts = ctypes.create_string_buffer(l.constants, max(1, len(l.constants)))
            names = [None if n is None else n.encode() for n, _ in l.overrides]
            ovr = (COverride * max(1, len(l.overrides)))(
                *[COverride(n, v) for n, (_, v) in zip(names, l.overrides)])
            self._keep += [binds, role, entry, consts, names, ovr]
            self.array[i] = CLaunch(l.kernel, entry, l.fmt, l.pack,
                                    ctypes.cast(consts, ctypes.c_void_p), len(l.constants),
                                    binds, len(l.bindings), l.invocations_per_row,
                                    l.workgroup_size, l.rows, l.rows_per_tile, l.key_split,
                                    l.window, l.partial_rows, l.tokens[0], l.tokens[1], role,
                                    l.layer, ovr, len(l.overrides))
        self.count = len(launches)


__all__ = ["Launch", "gemma3_launches", "CLaunches", "ROLE"]
