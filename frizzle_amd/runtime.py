"""Python face of the backend: a device, device arrays, the model, and the
engine's operations (load a model, generate, paired original/steered runs),
each a thin call across the C ABI. The host logic lives in the C++ library;
this module only moves numpy arrays and reports errors.
"""
import ctypes
from ctypes import POINTER, byref, c_double, c_uint32, c_void_p
from dataclasses import dataclass
from enum import IntEnum

import numpy as np

from . import _lib
from ._lib import Edit as _CEdit
from ._lib import Limits, ModelConfig, Sampling, check, load


class EditKind(IntEnum):
    """edit::EditKind (src/core/edit/edit.h:118)."""
    SET = 0
    SCALE = 1
    ZERO = 2


TO_THE_END = 0xFFFFFFFF


@dataclass(frozen=True)
class Edit:
    """edit::Edit (src/core/edit/edit.h:123-130): a pin of one neuron over the
    steps [start, until) of a run."""
    layer: int
    neuron: int
    kind: EditKind
    value: float
    start: int = 0
    until: int = TO_THE_END


class EditError(IntEnum):
    """edit::EditError (src/core/edit/edit.h:131-141)."""
    OK = 0
    KIND = 1
    LAYER = 2
    NEURON = 3
    NOT_FINITE = 4
    ZERO_VALUE = 5
    RANGE = 6
    OVERLAP = 7
    TOO_MANY = 8


def _c_edits(edits):
    arr = (_CEdit * max(1, len(edits)))()
    for i, e in enumerate(edits):
        arr[i] = _CEdit(e.layer, e.neuron, int(e.kind), e.value, e.start, e.until)
    return arr


def edit_check(edits, layers, ffn):
    """edit::check: (EditError, index of the first offending edit)."""
    lib = load()
    off = c_uint32(0)
    err = lib.frz_edit_check(_c_edits(edits), len(edits), layers, ffn, byref(off))
    return EditError(err), off.value


def edit_table(edits, layers, origin=0):
    """edit::table as u32 words; origin 0 keeps the ranges in steps."""
    lib = load()
    words = lib.frz_edit_table_words(len(edits), layers)
    out = np.zeros(words, dtype=np.uint32)
    check(lib.frz_edit_table(_c_edits(edits), len(edits), layers, origin,
                             out.ctypes.data))
    return out


def edit_apply(kind, value, neuron):
    return load().frz_edit_apply(int(kind), value, neuron)


def sampling(temperature=0.0, top_k=1, top_p=1.0, min_p=0.0, seed=0):
    """Sampling settings; the defaults are greedy."""
    return Sampling(top_k, temperature, top_p, min_p, seed)


def gemma3_1b_config(context=8192, **overrides):
    cfg = ModelConfig()
    load().frz_gemma3_1b_config(byref(cfg), context)
    for k, v in overrides.items():
        setattr(cfg, k, v)
    return cfg


def tensor_bytes(cfg, role):
    return load().frz_tensor_bytes(byref(cfg), _lib.ROLE[role])


def synth_tensor(cfg, seed, layer, role):
    """The seeded synthetic weights of one tensor, as a GGUF file holds them
    (uint8 Q4_0 blocks, or float32 gains)."""
    lib = load()
    n = lib.frz_tensor_bytes(byref(cfg), _lib.ROLE[role])
    out = np.empty(n, dtype=np.uint8)
    check(lib.frz_synth_tensor(byref(cfg), seed, layer, _lib.ROLE[role],
                               out.ctypes.data, n))
    if _lib.ROLE[role] >= _lib.ROLE["attn_norm"] and role != "embedding":
        return out.view(np.float32)
    return out


def q4_0_split(blocks):
    """GGUF Q4_0 blocks (uint8, 18 a block) to (codes, scales) streams."""
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    n = blocks.size // 18
    codes = np.empty(n * 16, dtype=np.uint8)
    scales = np.empty(n * 2, dtype=np.uint8)
    check(load().frz_q4_0_split(blocks.ctypes.data, n, codes.ctypes.data,
                                scales.ctypes.data))
    return codes, scales


# GGUF format numbers of the weight formats the library computes in.
Q4_0, Q4_1, Q8_0 = 2, 3, 8
# How steps of several rows compute their products (frz_prefill_mode).
PREFILL_EXACT, PREFILL_BF16 = 0, 1
_BLOCK = {Q4_0: (18, 16, 2), Q4_1: (20, 16, 4), Q8_0: (34, 32, 2)}  # bytes, codes, scales


def block_split(fmt, blocks):
    """GGUF blocks of a weight format to its (codes, scales) streams."""
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    bb, cb, sb = _BLOCK.get(fmt, (1, 0, 0))  # another format: the library refuses it
    n = blocks.size // bb
    codes = np.empty(n * cb, dtype=np.uint8)
    scales = np.empty(n * sb, dtype=np.uint8)
    check(load().frz_block_split(fmt, blocks.ctypes.data, n, codes.ctypes.data,
                                 scales.ctypes.data))
    return codes, scales


CAPTURE_SLOTS = ("neurons", "residual", "attention_added", "mlp_added", "query", "weights",
                 "stats", "readout")


def capture_words(cfg):
    """The capture store's size in words (0 for shapes it cannot hold)."""
    return int(load().frz_capture_words(byref(cfg), None))


def capture_layout(cfg):
    """Each layer's slots of the capture store: {name: (first word, width)},
    plus keys, query_heads, window and full_attention."""
    out = []
    for layer in range(cfg.layers):
        s = _lib.CaptureSlots()
        check(load().frz_capture_layer(byref(cfg), layer, byref(s)))
        d = {n: (getattr(s, n).first, getattr(s, n).width) for n in CAPTURE_SLOTS}
        d.update(keys=s.keys, query_heads=s.query_heads, window=s.window,
                 full_attention=bool(s.full_attention))
        out.append(d)
    return out


def rope_turns(base, head_dim):
    out = (ctypes.c_float * (head_dim // 2))()
    load().frz_rope_turns(base, head_dim, out)
    return np.frombuffer(out, dtype=np.float32).copy()


class DeviceArray:
    """A device allocation holding a numpy array's bytes."""

    def __init__(self, device, nbytes, dtype, shape):
        self.device = device
        self.nbytes = int(nbytes)
        self.dtype = np.dtype(dtype)
        self.shape = tuple(shape)
        ptr = c_void_p()
        check(device.lib.frz_alloc(device.handle, self.nbytes, byref(ptr)))
        self.ptr = ptr.value

    def upload(self, array):
        a = np.ascontiguousarray(array)
        assert a.nbytes <= self.nbytes
        check(self.device.lib.frz_write(self.device.handle, self.ptr,
                                        a.ctypes.data, a.nbytes))
        return self

    def numpy(self):
        out = np.empty(self.shape, dtype=self.dtype)
        check(self.device.lib.frz_read(self.device.handle, out.ctypes.data,
                                       self.ptr, out.nbytes))
        return out

    def zero(self):
        check(self.device.lib.frz_fill_zero(self.device.handle, self.ptr, self.nbytes))
        return self

    def free(self):
        if self.ptr:
            self.device.lib.frz_free(self.device.handle, self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def _launches(out, count):
    return [(out[i].role.decode(), None if out[i].layer == 0xFFFFFFFF else int(out[i].layer),
             float(out[i].microseconds)) for i in range(count)]


class Device:
    """One GPU (frz_open). Raises when there is none."""

    def __init__(self, ordinal=0):
        self.lib = load()
        h = c_void_p()
        self.limits = Limits()
        check(self.lib.frz_open(ordinal, byref(h), byref(self.limits)))
        self.handle = h.value

    def array(self, array):
        a = np.ascontiguousarray(array)
        return DeviceArray(self, max(1, a.nbytes), a.dtype, a.shape).upload(a)

    def empty(self, shape, dtype):
        dt = np.dtype(dtype)
        n = int(np.prod(shape)) * dt.itemsize
        return DeviceArray(self, max(1, n), dt, shape)

    def sync(self):
        check(self.lib.frz_sync(self.handle))

    def close(self):
        if self.handle:
            self.lib.frz_close(self.handle)
            self.handle = None


class Model:
    """A Gemma-3 model resident on the device (frz_model_create)."""

    def __init__(self, device, cfg):
        self.device = device
        self.lib = device.lib
        self.cfg = cfg
        h = c_void_p()
        check(self.lib.frz_model_create(device.handle, byref(cfg), byref(h)))
        self.handle = h.value

    @classmethod
    def planned(cls, device, plan):
        """A model created from a residency plan (frz_model_create_planned):
        its buffers the plan's, its context the one the plan offered."""
        self = cls.__new__(cls)
        self.device = device
        self.lib = device.lib
        self.cfg = plan.config()
        h = c_void_p()
        check(self.lib.frz_model_create_planned(device.handle, plan._h, byref(h)))
        self.handle = h.value
        return self

    def set_tensor(self, layer, role, data, fmt=None):
        """A role's tensor as GGUF bytes; fmt a GGUF format number (Q4_1 or
        Q8_0 where the role takes one), else the role's Q4_0 or F32."""
        a = np.ascontiguousarray(data)
        if fmt is None:
            check(self.lib.frz_model_set_tensor(self.handle, layer, _lib.ROLE[role],
                                                a.ctypes.data, a.nbytes))
        else:
            check(self.lib.frz_model_set_tensor_format(self.handle, layer, _lib.ROLE[role], fmt,
                                                       a.ctypes.data, a.nbytes))

    def time_layer(self, layer, position, iters=200):
        """µs of one layer's one-token decode launches, replayed as a graph."""
        us = ctypes.c_double()
        check(self.lib.frz_model_time_layer(self.handle, layer, position, iters, byref(us)))
        return us.value

    @property
    def reused(self):
        """Prompt tokens the last generate() took from the caches."""
        return int(self.lib.frz_model_reused(self.handle))

    def set_capture(self, on=True):
        """The capture store on or off: while on, the step that ends a
        prompt writes it."""
        check(self.lib.frz_model_set_capture(self.handle, int(on)))

    def capture(self):
        """The capture store as uint32 words, and its per-layer slots
        ({slot: (first, width)} a layer, with keys and window)."""
        layout = capture_layout(self.cfg)
        words = capture_words(self.cfg)
        out = np.empty(words, dtype=np.uint32)
        check(self.lib.frz_model_read_capture(self.handle, out.ctypes.data, words))
        return out, layout

    def load_gguf(self, path):
        """Every tensor of a Gemma 3 GGUF file of this model's shapes."""
        check(self.lib.frz_model_load_gguf(self.handle, str(path).encode()))

    def synthesize(self, seed):
        check(self.lib.frz_model_synthesize(self.handle, seed))

    def set_graphs(self, enabled):
        check(self.lib.frz_model_set_graphs(self.handle, int(enabled)))

    def set_prefill(self, mode):
        """PREFILL_EXACT (the reference's order, bit for bit) or PREFILL_BF16
        (products on the bf16 matrix cores over split operands, logits
        within 1e-3 relative) for steps of several rows."""
        check(self.lib.frz_model_set_prefill(self.handle, int(mode)))

    def set_edits(self, table):
        t = np.ascontiguousarray(table, dtype=np.uint32)
        check(self.lib.frz_model_set_edits(self.handle, t.ctypes.data, t.size))

    def step(self, position, ids, logits=False, samp=None):
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        s = samp or sampling()
        check(self.lib.frz_model_step(self.handle, position, ids.size,
                                      ids.ctypes.data, int(logits), byref(s)))

    def decode(self, position, steps, samp=None):
        s = samp or sampling()
        toks = np.zeros(steps, dtype=np.uint32)
        failed = np.zeros(steps, dtype=np.uint32)
        check(self.lib.frz_model_decode(self.handle, position, steps, byref(s),
                                        toks.ctypes.data, failed.ctypes.data))
        return toks, failed

    # A step's launches fit in this many entries (a prompt's last step with
    # the capture store's readouts makes about 420 for Gemma-3-1B).
    PROFILE_CAP = 2048

    def profile_step(self, position, ids, logits=False, samp=None):
        """frz_model_step, profiled: [(roles, layer, microseconds)] a launch,
        roles the graph's names ('+' between a fused launch's), layer None for
        the embedding and the output."""
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        s = samp or sampling()
        n = c_uint32()
        out = (_lib.LaunchTime * self.PROFILE_CAP)()
        check(self.lib.frz_model_profile_step(self.handle, position, ids.size, ids.ctypes.data,
                                              int(logits), byref(s), out, self.PROFILE_CAP,
                                              byref(n)))
        return _launches(out, min(n.value, self.PROFILE_CAP))

    def profile_decode(self, position, samp=None):
        """One fed decode step at `position` (the last step's draw), profiled:
        (launches as profile_step gives them, the step's draw)."""
        s = samp or sampling()
        n, tok = c_uint32(), c_uint32()
        out = (_lib.LaunchTime * self.PROFILE_CAP)()
        check(self.lib.frz_model_profile_decode(self.handle, position, byref(s), out,
                                                self.PROFILE_CAP, byref(n), byref(tok)))
        return _launches(out, min(n.value, self.PROFILE_CAP)), int(tok.value)

    def time_decode(self, position, steps, samp=None):
        s = samp or sampling()
        us = c_double()
        check(self.lib.frz_model_time_decode(self.handle, position, steps,
                                             byref(s), byref(us)))
        return us.value

    def logits(self):
        out = np.empty(self.cfg.vocab, dtype=np.float32)
        check(self.lib.frz_model_read_logits(self.handle, out.ctypes.data, out.size))
        return out

    def record(self):
        out = np.empty(4, dtype=np.uint32)
        check(self.lib.frz_model_read_record(self.handle, out.ctypes.data))
        return out

    def candidates(self):
        out = np.empty(128, dtype=np.uint32)
        check(self.lib.frz_model_read_candidates(self.handle, out.ctypes.data))
        return out

    def normed(self, rows=1):
        out = np.empty((rows, self.cfg.hidden), dtype=np.float32)
        check(self.lib.frz_model_read_hidden(self.handle, out.ctypes.data, rows))
        return out

    def cache(self, layer, values, count):
        out = np.empty(count, dtype=np.uint16)
        check(self.lib.frz_model_read_cache(self.handle, layer, int(values),
                                            out.ctypes.data, count))
        return out

    def generate(self, prompt, edits=(), samp=None, max_tokens=16, stop_ids=()):
        """Engine::generate at the token level: the prompt, then up to
        max_tokens drawn tokens under `edits` (Edit list, ranges in steps)."""
        prompt = np.ascontiguousarray(prompt, dtype=np.uint32)
        edits = list(edits)
        if edits:
            err, idx = edit_check(edits, self.cfg.layers, self.cfg.ffn)
            if err != EditError.OK:
                raise ValueError(f"edit {idx} refused: {err.name}")
            table = edit_table(edits, self.cfg.layers, 0)
        else:
            table = np.zeros(2 * self.cfg.layers, dtype=np.uint32)
        stops = np.ascontiguousarray(list(stop_ids) or [0], dtype=np.uint32)
        out = np.zeros(max(1, max_tokens), dtype=np.uint32)
        drawn = c_uint32()
        s = samp or sampling()
        check(self.lib.frz_generate(self.handle, prompt.ctypes.data, prompt.size,
                                    table.ctypes.data, table.size, byref(s),
                                    max_tokens, stops.ctypes.data,
                                    len(stop_ids), out.ctypes.data, byref(drawn)))
        return out[:drawn.value].copy()

    def generate_variants(self, prompt, variants, samp=None, max_tokens=16, stop_ids=(),
                          residuals=False):
        """Many replies to one prompt decoded together: variants is a list of
        Edit lists (ranges in steps), one a variant. Returns a list of token
        arrays (each what generate() gives for that variant's edits) and,
        with residuals, a [max_tokens, layers, variants, hidden] array of the
        residual entering each layer at each step."""
        prompt = np.ascontiguousarray(prompt, dtype=np.uint32)
        tables = []
        for edits in variants:
            edits = list(edits)
            if edits:
                err, idx = edit_check(edits, self.cfg.layers, self.cfg.ffn)
                if err != EditError.OK:
                    raise ValueError(f"edit {idx} refused: {err.name}")
                tables.append(edit_table(edits, self.cfg.layers, 0))
            else:
                tables.append(np.zeros(2 * self.cfg.layers, dtype=np.uint32))
        words = max(t.size for t in tables)
        packed = np.zeros((len(tables), words), dtype=np.uint32)
        for i, t in enumerate(tables):
            packed[i, :t.size] = t
        n = len(tables)
        stops = np.ascontiguousarray(list(stop_ids) or [0], dtype=np.uint32)
        out = np.zeros((n, max_tokens), dtype=np.uint32)
        drawn = np.zeros(n, dtype=np.uint32)
        res = (np.empty((max_tokens, self.cfg.layers, n, self.cfg.hidden), dtype=np.float32)
               if residuals else None)
        s = samp or sampling()
        check(self.lib.frz_generate_variants(
            self.handle, prompt.ctypes.data, prompt.size, n, packed.ctypes.data, words, byref(s),
            max_tokens, stops.ctypes.data, len(stop_ids), out.ctypes.data, drawn.ctypes.data,
            res.ctypes.data if residuals else None))
        replies = [out[v, :drawn[v]].copy() for v in range(n)]
        return (replies, res) if residuals else replies

    def paired(self, prompt, edits, samp=None, max_tokens=16, stop_ids=()):
        """The native tool's paired runs (tools/frizzle/main.cpp:53-55): the
        original reply, then the steered one from the same seed, sharing the
        cached prompt."""
        original = self.generate(prompt, (), samp, max_tokens, stop_ids)
        steered = self.generate(prompt, edits, samp, max_tokens, stop_ids)
        return original, steered

    def close(self):
        if self.handle:
            self.lib.frz_model_destroy(self.handle)
            self.handle = None
