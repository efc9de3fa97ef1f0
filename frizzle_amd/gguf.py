"""GGUF files through the library's reader (frz_gguf_*, include/frizzle_hip.h)
and a GGUF v3 writer.

Index.read(front, file_size) and Index.open(path) give a file's tensors and
metadata, every claim in the file checked by the library; a malformed file
raises GgufError naming the rule it breaks (the reference's ReadError,
src/core/gguf/types.h:237-265). write_gemma3() writes a Gemma 3 model's
tensors, as the library's roles hold them, into a GGUF v3 file that
Model.load_gguf() reads back.
"""
import ctypes
import struct
from pathlib import Path

from ._lib import GgufTensor, ModelConfig, check, load

ERRORS = [
    "OK", "NEED_MORE_BYTES", "SHORT_READ", "BAD_MAGIC", "UNSUPPORTED_VERSION",
    "COUNT_TOO_LARGE", "STRING_TOO_LONG", "ARRAY_TOO_LONG", "UNKNOWN_VALUE_TYPE",
    "UNKNOWN_TENSOR_TYPE", "ROW_NOT_WHOLE_BLOCKS", "TOO_MANY_DIMENSIONS",
    "NEGATIVE_DIMENSION", "ELEMENT_COUNT_OVERFLOW", "OFFSET_OVERFLOW",
    "TENSOR_DATA_OUT_OF_BOUNDS", "DUPLICATE_TENSOR_NAME", "TENSOR_NAME_TOO_LONG",
    "MISALIGNED_TENSOR_DATA", "OVERLAPPING_TENSOR_DATA", "BAD_ALIGNMENT", "EMPTY_KEY",
    "DUPLICATE_METADATA_KEY", "NESTED_ARRAY",
]

# GGUF's metadata value types and the tensor formats used here.
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
T_F32, T_F16, T_Q4_0, T_Q4_1, T_Q8_0 = 0, 1, 2, 3, 8


class GgufError(ValueError):
    """The file breaks a named rule (or, with code NEED_MORE_BYTES, more of
    its front is needed: `needed` bytes from its start)."""

    def __init__(self, code, needed=0):
        name = ERRORS[code] if 0 <= code < len(ERRORS) else str(code)
        text = load().frz_gguf_error_text(code).decode() if code >= 0 else "cannot read the file"
        super().__init__(f"{name}: {text}")
        self.code = code
        self.name = name
        self.needed = needed


class Index:
    """A file's index, held by the library."""

    def __init__(self, handle):
        self._h = handle
        self._lib = load()

    @classmethod
    def read(cls, front, file_size=None):
        """The index from the first len(front) bytes of a file of file_size
        bytes (default: front is the whole file)."""
        front = bytes(front)
        size = len(front) if file_size is None else file_size
        h = ctypes.c_void_p()
        needed = ctypes.c_uint64(0)
        buf = ctypes.create_string_buffer(front, len(front)) if front else None
        rc = load().frz_gguf_read(buf, len(front), size, ctypes.byref(h), ctypes.byref(needed))
        if rc != 0:
            raise GgufError(rc, needed.value)
        return cls(h)

    @classmethod
    def open(cls, path):
        h = ctypes.c_void_p()
        rc = load().frz_gguf_open(str(path).encode(), ctypes.byref(h))
        if rc != 0:
            raise GgufError(rc)
        return cls(h)

    def close(self):
        if self._h:
            self._lib.frz_gguf_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @staticmethod
    def _info(t):
        n = t.dimensions
        return {"name": t.name.decode(), "type": t.type, "shape": list(t.shape[:max(n, 1)])
                if n else [], "elements": t.elements, "offset": t.offset, "bytes": t.bytes}

    @property
    def tensors(self):
        out = []
        for i in range(self._lib.frz_gguf_tensor_count(self._h)):
            t = GgufTensor()
            check(self._lib.frz_gguf_tensor_at(self._h, i, ctypes.byref(t)))
            out.append(self._info(t))
        return out

    def find(self, name):
        t = GgufTensor()
        check(self._lib.frz_gguf_find(self._h, name.encode(), ctypes.byref(t)))
        return self._info(t)

    @property
    def metadata_count(self):
        return self._lib.frz_gguf_metadata_count(self._h)

    def u32(self, key):
        v = ctypes.c_uint32()
        check(self._lib.frz_gguf_get_u32(self._h, key.encode(), ctypes.byref(v)))
        return v.value

    def f32(self, key):
        v = ctypes.c_float()
        check(self._lib.frz_gguf_get_f32(self._h, key.encode(), ctypes.byref(v)))
        return v.value

    def string(self, key):
        n = ctypes.c_uint64()
        check(self._lib.frz_gguf_get_string(self._h, key.encode(), None, 0, ctypes.byref(n)))
        buf = ctypes.create_string_buffer(n.value + 1)
        check(self._lib.frz_gguf_get_string(self._h, key.encode(), buf, n.value + 1, None))
        return buf.raw[:n.value].decode()

    def array(self, key):
        """(element type, count) of an array entry."""
        t, n = ctypes.c_uint32(), ctypes.c_uint64()
        check(self._lib.frz_gguf_get_array(self._h, key.encode(), ctypes.byref(t),
                                           ctypes.byref(n)))
        return t.value, n.value

    def gemma3_config(self, context=0):
        cfg = ModelConfig()
        check(self._lib.frz_gemma3_config_from_gguf(self._h, context, ctypes.byref(cfg)))
        return cfg


def format_layout(ttype):
    """(name, block elements, block bytes) of a GGUF format number."""
    name, el, by = ctypes.c_char_p(), ctypes.c_uint32(), ctypes.c_uint32()
    check(load().frz_gguf_format(ttype, ctypes.byref(name), ctypes.byref(el), ctypes.byref(by)))
    return name.value.decode(), el.value, by.value


# ---- writing ------------------------------------------------------------------

def _gstr(b):
    return struct.pack("<Q", len(b)) + b


_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f",
           BOOL: "<?", U64: "<Q", I64: "<q", F64: "<d"}


def _value(vtype, value):
    if vtype == STRING:
        return _gstr(value.encode() if isinstance(value, str) else value)
    if vtype == ARRAY:
        etype, items = value
        body = b"".join(_value(etype, v) for v in items)
        return struct.pack("<IQ", etype, len(items)) + body
    return struct.pack(_SCALAR[vtype], value)


def _encode(tensors, metadata, alignment):
    """The header and index of a GGUF v3 file (tensors as (name, extents,
    format, bytes)), padded to the data's alignment, and each tensor's data
    offset and padded length."""
    md = [(k, t, v) for k, t, v in metadata]
    if alignment != 32 and not any(k == "general.alignment" for k, _, _ in md):
        md.append(("general.alignment", U32, alignment))
    out = bytearray(b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(md)))
    for key, vtype, value in md:
        out += _gstr(key.encode()) + struct.pack("<I", vtype) + _value(vtype, value)
    offset, spans = 0, []
    for name, dims, ttype, nbytes in tensors:
        out += _gstr(name.encode()) + struct.pack("<I", len(dims))
        out += b"".join(struct.pack("<q", d) for d in dims)
        out += struct.pack("<IQ", ttype, offset)
        pad = (-nbytes) % alignment
        spans.append(nbytes + pad)
        offset += nbytes + pad
    out += b"\0" * ((-len(out)) % alignment)
    return bytes(out), spans


def write(path, tensors, metadata=(), alignment=32):
    """A GGUF v3 file: tensors as (name, extents ne0 first, format, bytes),
    metadata as (key, value type, value); data aligned to `alignment`."""
    head, spans = _encode([(n, d, t, len(b)) for n, d, t, b in tensors], metadata, alignment)
    with open(path, "wb") as f:
        f.write(head)
        for (_, _, _, data), span in zip(tensors, spans):
            f.write(bytes(data) + b"\0" * (span - len(data)))
    return Path(path)


def index_only(tensors, metadata=(), alignment=32):
    """The front of a GGUF v3 file holding only its header and index
    (tensors as (name, extents, format, data bytes)), and the size the whole
    file would have: read with Index.read(front, size), whose index reads no
    tensor data."""
    head, spans = _encode(tensors, metadata, alignment)
    return head, len(head) + sum(spans)


LAYER_NAMES = {
    "q": "attn_q.weight", "k": "attn_k.weight", "v": "attn_v.weight",
    "o": "attn_output.weight", "gate": "ffn_gate.weight", "up": "ffn_up.weight",
    "down": "ffn_down.weight", "attn_norm": "attn_norm.weight",
    "q_norm": "attn_q_norm.weight", "k_norm": "attn_k_norm.weight",
    "post_attn_norm": "post_attention_norm.weight", "ffn_norm": "ffn_norm.weight",
    "post_ffn_norm": "post_ffw_norm.weight",
}


def _extents(cfg, role):
    """(ne0, ne1) of a role's tensor in a file: a matrix of rows over cols
    inputs is [cols, rows]; a norm gain is [n]."""
    qw, kvw = cfg.query_heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
    return {
        "q": [cfg.hidden, qw], "k": [cfg.hidden, kvw], "v": [cfg.hidden, kvw],
        "o": [qw, cfg.hidden], "gate": [cfg.hidden, cfg.ffn], "up": [cfg.hidden, cfg.ffn],
        "down": [cfg.ffn, cfg.hidden], "q_norm": [cfg.head_dim], "k_norm": [cfg.head_dim],
        "embedding": [cfg.hidden, cfg.vocab],
    }.get(role, [cfg.hidden])


def write_gemma3(path, cfg, tensor, name="synthetic gemma3", formats=None, metadata=()):
    """A Gemma 3 GGUF file of cfg's shapes. tensor(layer, role) gives a
    role's bytes as the library's roles hold them (Q4_0 matrices, F32
    gains); layer -1 for "embedding" and "output_norm". `formats` may give a
    tensor name another format number (to write files this backend refuses);
    `metadata` adds entries (key, value type, value), such as a tokenizer's."""
    formats = formats or {}
    md = [
        ("general.architecture", STRING, "gemma3"),
        ("general.name", STRING, name),
        ("general.alignment", U32, 32),
        ("gemma3.block_count", U32, cfg.layers),
        ("gemma3.context_length", U32, cfg.context),
        ("gemma3.embedding_length", U32, cfg.hidden),
        ("gemma3.feed_forward_length", U32, cfg.ffn),
        ("gemma3.attention.head_count", U32, cfg.query_heads),
        ("gemma3.attention.head_count_kv", U32, cfg.kv_heads),
        ("gemma3.attention.key_length", U32, cfg.head_dim),
        ("gemma3.attention.value_length", U32, cfg.head_dim),
        ("gemma3.attention.layer_norm_rms_epsilon", F32, cfg.epsilon),
        ("gemma3.rope.freq_base", F32, cfg.rope_global),
        ("gemma3.rope.freq_base_swa", F32, cfg.rope_local),
        ("gemma3.attention.sliding_window", U32, cfg.window),
        ("gemma3.attention.sliding_window_pattern", U32, cfg.pattern),
    ] + list(metadata)

    def fmt(tname, role):
        return formats.get(tname, T_F32 if "norm" in role else T_Q4_0)

    ts = [("token_embd.weight", _extents(cfg, "embedding"), fmt("token_embd.weight", "embedding"),
           tensor(-1, "embedding"))]
    for layer in range(cfg.layers):
        for role, leaf in LAYER_NAMES.items():
            tname = f"blk.{layer}.{leaf}"
            ts.append((tname, _extents(cfg, role), fmt(tname, role), tensor(layer, role)))
    ts.append(("output_norm.weight", [cfg.hidden], T_F32, tensor(-1, "output_norm")))
    return write(path, ts, md)

