"""ctypes access to the CPU oracle (oracle/liboracle.so) for the tests.

The oracle is the checker: tests compare the HIP backend against it, and pin
the oracle itself against closed forms, brute force and the reference's own
fixtures. Nothing in the product imports this module.
"""
import ctypes
import subprocess
from ctypes import POINTER, c_float, c_int, c_uint16, c_uint32, c_void_p
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent.parent
ORACLE_DIR = ROOT / "oracle"
ORACLE_LIB = ORACLE_DIR / "liboracle.so"


class OrcConfig(ctypes.Structure):
    _fields_ = [(n, c_int) for n in (
        "hidden", "ffn", "head_dim", "query_heads", "kv_heads", "layers",
        "vocab", "window", "pattern", "context", "local_slots")] + [
        ("rope_local", c_float), ("rope_global", c_float), ("epsilon", c_float),
        ("embedding_format", c_int)]


class OrcLayer(ctypes.Structure):
    _fields_ = [(n, c_void_p) for n in (
        "q", "k", "v", "o", "gate", "up", "down", "attn_norm", "q_norm",
        "k_norm", "post_attn_norm", "ffn_norm", "post_ffn_norm")] + [("down_format", c_int)]


_P = c_void_p
_SIGS = {
    "orc_exp_nonpositive": (c_float, [c_float]),
    "orc_gelu_tanh": (c_float, [c_float]),
    "orc_exp2": (c_float, [c_float]),
    "orc_cos": (c_float, [c_float]),
    "orc_sin": (c_float, [c_float]),
    "orc_inverse_sqrt": (c_float, [c_float]),
    "orc_f16_pack": (c_uint16, [c_float]),
    "orc_f16_unpack": (c_float, [c_uint16]),
    "orc_dot4": (c_float, [_P, _P]),
    "orc_q4_0_unpack": (None, [_P, _P]),
    "orc_gemv": (None, [_P, c_int, c_int, _P, _P]),
    "orc_gemv_format": (None, [c_int, _P, c_int, c_int, _P, _P]),
    "orc_q4_1_unpack": (None, [_P, _P]),
    "orc_q8_0_unpack": (None, [_P, _P]),
    "orc_block_bytes": (c_int, [c_int]),
    "orc_gated": (None, [_P, _P, c_int, c_int, _P, _P]),
    "orc_norm_row": (None, [_P, _P, c_int, c_int, c_float, c_float, c_int, _P,
                            _P, _P]),
    "orc_rope_turns": (None, [c_float, c_int, _P]),
    "orc_rope_row": (None, [c_int, c_int, c_int, c_int, c_int, c_float, _P, _P,
                            _P, _P, _P, _P, _P, _P]),
    "orc_norm_row_added": (None, [_P, _P, c_int, c_int, c_float, c_float, c_int, _P,
                                  _P, _P, _P]),
    "orc_attention_row_scores": (None, [c_int, c_int, c_int, c_int, c_int, c_int, c_float,
                                        _P, _P, _P, _P, _P, c_int, _P]),
    "orc_attention_row": (None, [c_int, c_int, c_int, c_int, c_int, c_int,
                                 c_float, _P, _P, _P, _P]),
    "orc_gather_row": (None, [_P, c_int, c_uint32, c_float, _P]),
    "orc_gather_row_format": (None, [c_int, _P, c_int, c_uint32, c_float, _P]),
    "orc_edit_row": (None, [_P, c_int, c_uint32, c_int, _P]),
    "orc_topk": (None, [_P, c_int, _P, _P]),
    "orc_philox": (None, [_P, _P, _P]),
    "orc_mulhi": (c_uint32, [c_uint32, c_uint32]),
    "orc_draw": (None, [_P, _P, c_uint32, c_uint32, c_float, c_float, c_float,
                        c_float, c_uint32, c_uint32, c_uint32, _P]),
    "orc_model_create": (c_void_p, [POINTER(OrcConfig), POINTER(OrcLayer), _P,
                                    _P]),
    "orc_model_destroy": (None, [_P]),
    "orc_model_clone": (c_void_p, [_P]),
    "orc_model_set_edits": (None, [_P, _P, c_int]),
    "orc_model_token": (None, [_P, c_uint32, c_int, _P]),
    "orc_model_block": (None, [_P, _P, c_int, c_int, _P]),
    "orc_model_normed": (c_void_p, [_P]),
    "orc_model_residuals": (c_void_p, [_P]),
    "orc_model_set_capture": (None, [_P, c_int]),
    "orc_model_capture": (c_void_p, [_P, c_int, c_int, POINTER(c_int)]),
    "orc_model_key_cache": (c_void_p, [_P, c_int]),
    "orc_model_value_cache": (c_void_p, [_P, c_int]),
    "orc_model_slots": (c_int, [_P, c_int]),
}

_lib = None
_libm = ctypes.CDLL("libm.so.6")
_libm.logf.restype = c_float
_libm.logf.argtypes = [c_float]


def _logf(x):
    return _libm.logf(x)


def build():
    subprocess.run(["make", "-s", "-C", str(ORACLE_DIR)], check=True)


def lib():
    global _lib
    if _lib is None:
        if not ORACLE_LIB.exists():
            build()
        L = ctypes.CDLL(str(ORACLE_LIB))
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a):
    return a.ctypes.data


def f32(x):
    return np.ascontiguousarray(x, dtype=np.float32)


def gemv(w_blocks, rows, cols, x):
    y = np.empty(rows, dtype=np.float32)
    x = f32(x)
    lib().orc_gemv(_p(w_blocks), rows, cols, _p(x), _p(y))
    return y


def gated(gate_blocks, up_blocks, rows, cols, x):
    y = np.empty(rows, dtype=np.float32)
    x = f32(x)
    lib().orc_gated(_p(gate_blocks), _p(up_blocks), rows, cols, _p(x), _p(y))
    return y


def gemv_format(fmt, w_blocks, rows, cols, x):
    y = np.empty(rows, dtype=np.float32)
    w = np.ascontiguousarray(w_blocks, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    lib().orc_gemv_format(fmt, _p(w), rows, cols, _p(x), _p(y))
    return y


def unpack_format(fmt, block):
    out = np.empty(32, dtype=np.float32)
    b = np.ascontiguousarray(block, dtype=np.uint8)
    {2: lib().orc_q4_0_unpack, 3: lib().orc_q4_1_unpack, 8: lib().orc_q8_0_unpack}[fmt](
        _p(b), _p(out))
    return out


def gather_row_format(fmt, table, width, token, scale):
    out = np.empty(width, dtype=np.float32)
    t = np.ascontiguousarray(table, dtype=np.uint8)
    lib().orc_gather_row_format(fmt, _p(t), width, token, scale, _p(out))
    return out


def q4_0_unpack(block):
    out = np.empty(32, dtype=np.float32)
    b = np.ascontiguousarray(block, dtype=np.uint8)
    lib().orc_q4_0_unpack(_p(b), _p(out))
    return out


def norm_row(gain, hidden, output=None, post_gain=None, epsilon=1e-6):
    hidden = f32(hidden).copy()
    normed = np.empty_like(hidden)
    add = post_gain is not None
    out = f32(output) if add else hidden
    pg = f32(post_gain) if add else f32(gain)
    lib().orc_norm_row(_p(f32(gain)), _p(pg), int(add), int(add), 1.0, epsilon,
                       hidden.size, _p(hidden), _p(out), _p(normed))
    return hidden, normed


def rope_turns(base, head_dim):
    t = np.empty(head_dim // 2, dtype=np.float32)
    lib().orc_rope_turns(base, head_dim, _p(t))
    return t


def topk(logits):
    bits = np.empty(64, dtype=np.uint32)
    ids = np.empty(64, dtype=np.uint32)
    lg = f32(logits)
    lib().orc_topk(_p(lg), lg.size, _p(bits), _p(ids))
    return bits, ids


def philox(counter, key):
    c = np.ascontiguousarray(counter, dtype=np.uint32)
    k = np.ascontiguousarray(key, dtype=np.uint32)
    out = np.empty(4, dtype=np.uint32)
    lib().orc_philox(_p(c), _p(k), _p(out))
    return out


def draw(cand_bits, cand_ids, top_k=1, temperature=0.0, top_p=1.0, min_p=0.0,
         counter=0, seed=0):
    b = np.ascontiguousarray(cand_bits, dtype=np.uint32)
    i = np.ascontiguousarray(cand_ids, dtype=np.uint32)
    rec = np.empty(4, dtype=np.uint32)
    # ln min_p in f32 by the C library, as sampler::apply takes it
    # (src/core/sampler/sampler.cpp:61) and as the backend does.
    log_min_p = _logf(min_p) if min_p > 0 else 0.0
    lib().orc_draw(_p(b), _p(i), 64, top_k, temperature, top_p, min_p,
                   np.float32(log_min_p), counter, seed & 0xFFFFFFFF,
                   (seed >> 32) & 0xFFFFFFFF, _p(rec))
    return rec


class OracleModel:
    """The oracle's model over host weight arrays (kept alive here)."""

    def __init__(self, cfg_dict, tensors, formats=None):
        """formats: {(layer, "down") or (-1, "embedding"): GGUF format
        number}; every other matrix is Q4_0."""
        formats = formats or {}
        self.cfg = OrcConfig(**cfg_dict, embedding_format=formats.get((-1, "embedding"), 2))
        self.tensors = tensors  # {(layer, role): array}
        n = self.cfg.layers
        self.layers = (OrcLayer * n)()
        for l in range(n):
            fields = {}
            for role in ("q", "k", "v", "o", "gate", "up", "down", "attn_norm",
                         "q_norm", "k_norm", "post_attn_norm", "ffn_norm",
                         "post_ffn_norm"):
                fields[role] = tensors[(l, role)].ctypes.data
            self.layers[l] = OrcLayer(**fields, down_format=formats.get((l, "down"), 2))
        self.handle = lib().orc_model_create(
            ctypes.byref(self.cfg), self.layers,
            tensors[(-1, "embedding")].ctypes.data,
            tensors[(-1, "output_norm")].ctypes.data)

    def clone(self):
        """A second model in this one's state over the same weights."""
        other = OracleModel.__new__(OracleModel)
        other.cfg, other.tensors, other.layers = self.cfg, self.tensors, self.layers
        other.handle = lib().orc_model_clone(self.handle)
        return other

    def set_edits(self, table):
        self._edits = np.ascontiguousarray(table, dtype=np.uint32)
        lib().orc_model_set_edits(self.handle, _p(self._edits), self._edits.size)

    def token(self, token, position, want_logits=True):
        logits = np.empty(self.cfg.vocab, dtype=np.float32) if want_logits else None
        lib().orc_model_token(self.handle, int(token), int(position),
                              _p(logits) if want_logits else None)
        return logits

    def block(self, tokens, position, want_logits=True):
        """A prefill block of up to 512 tokens from `position`; the last
        row's logits."""
        ids = np.ascontiguousarray(tokens, dtype=np.uint32)
        logits = np.empty(self.cfg.vocab, dtype=np.float32) if want_logits else None
        lib().orc_model_block(self.handle, _p(ids), ids.size, int(position),
                              _p(logits) if want_logits else None)
        return logits

    def prompt(self, tokens, position=0, block=512):
        """A prompt in prefill blocks of `block` tokens; the last row's
        logits."""
        tokens = np.ascontiguousarray(tokens, dtype=np.uint32)
        lg = None
        for at in range(0, tokens.size, block):
            part = tokens[at:at + block]
            lg = self.block(part, position + at, want_logits=at + block >= tokens.size)
        return lg

    def key_cache(self, layer):
        slots = lib().orc_model_slots(self.handle, layer)
        n = slots * self.cfg.kv_heads * self.cfg.head_dim
        ptr = lib().orc_model_key_cache(self.handle, layer)
        return np.ctypeslib.as_array((c_uint16 * n).from_address(ptr)).copy()

    def value_cache(self, layer):
        slots = lib().orc_model_slots(self.handle, layer)
        n = slots * self.cfg.kv_heads * self.cfg.head_dim
        ptr = lib().orc_model_value_cache(self.handle, layer)
        return np.ctypeslib.as_array((c_uint16 * n).from_address(ptr)).copy()

    def normed(self):
        ptr = lib().orc_model_normed(self.handle)
        return np.ctypeslib.as_array((c_float * self.cfg.hidden).from_address(ptr)).copy()

    SLOTS = ("neurons", "residual", "attention_added", "mlp_added", "query", "weights",
             "stats", "readout")

    def set_capture(self, on=True):
        lib().orc_model_set_capture(self.handle, int(on))

    def capture(self, layer, slot):
        """The last token's captured words (uint32) of one layer's slot."""
        n = c_int()
        ptr = lib().orc_model_capture(self.handle, layer, self.SLOTS.index(slot), ctypes.byref(n))
        if n.value == 0:
            return np.zeros(0, dtype=np.uint32)
        return np.ctypeslib.as_array((c_uint32 * n.value).from_address(ptr)).copy()

    def residuals(self):
        """[layers][hidden]: the last token's residual entering each layer."""
        ptr = lib().orc_model_residuals(self.handle)
        n = self.cfg.layers * self.cfg.hidden
        return np.ctypeslib.as_array((c_float * n).from_address(ptr)).copy().reshape(
            self.cfg.layers, self.cfg.hidden)

    def close(self):
        if self.handle:
            lib().orc_model_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
