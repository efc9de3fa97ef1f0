"""Gemma 3's SentencePiece BPE tokenizer through the library (frz_tokenizer_*,
include/frizzle_hip.h): Tokenizer.open(gguf_path), encode(text), decode(ids)
and texts(ids), the reference's Tokenizer::encode / decode and a turn's input
as text (src/core/tokenizer/tokenizer.h, detokenizer.h). Host only."""
import ctypes

import numpy as np

from ._lib import check, load

NO_TOKEN_LIMIT = 0xFFFFFFFF
ENCODE_ERRORS = ["OK", "INVALID_UTF8", "TOO_MANY_TOKENS", "TOO_LONG"]
NORMAL, UNKNOWN, CONTROL, USER_DEFINED, UNUSED, BYTE = 1, 2, 3, 4, 5, 6


class EncodeResult(ctypes.Structure):
    _fields_ = [("error", ctypes.c_int), ("least_tokens", ctypes.c_uint64),
                ("normalized_bytes", ctypes.c_uint64), ("raw_bytes", ctypes.c_uint64)]


class EncodeError(ValueError):
    def __init__(self, result):
        super().__init__(f"{ENCODE_ERRORS[result.error]}: at least {result.least_tokens} tokens, "
                         f"{result.normalized_bytes} normalized bytes, {result.raw_bytes} raw")
        self.name = ENCODE_ERRORS[result.error]
        self.least_tokens = result.least_tokens
        self.normalized_bytes = result.normalized_bytes


class Tokenizer:
    def __init__(self, handle):
        self._h = handle
        self._lib = load()

    @classmethod
    def open(cls, path):
        h = ctypes.c_void_p()
        check(load().frz_tokenizer_open(str(path).encode(), ctypes.byref(h)))
        return cls(h)

    def close(self):
        if self._h:
            self._lib.frz_tokenizer_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __len__(self):
        return self._lib.frz_tokenizer_size(self._h)

    @property
    def longest_cover(self):
        return self._lib.frz_tokenizer_longest_cover(self._h)

    def token(self, token_id):
        """(text bytes as the file spells it, type, score)."""
        text, n = ctypes.c_char_p(), ctypes.c_uint32()
        ty, sc = ctypes.c_int32(), ctypes.c_float()
        check(self._lib.frz_tokenizer_token(self._h, token_id, ctypes.byref(text),
                                            ctypes.byref(n), ctypes.byref(ty), ctypes.byref(sc)))
        return ctypes.string_at(text, n.value), ty.value, sc.value

    def encode(self, text, max_tokens=NO_TOKEN_LIMIT):
        """Token ids of `text` (str or bytes); raises EncodeError on a
        refusal."""
        raw = text.encode() if isinstance(text, str) else bytes(text)
        count, res = ctypes.c_uint64(), EncodeResult()
        check(self._lib.frz_tokenizer_encode(self._h, raw, len(raw), max_tokens, None, 0,
                                             ctypes.byref(count), ctypes.byref(res)))
        if res.error:
            raise EncodeError(res)
        ids = np.zeros(count.value, dtype=np.uint32)
        check(self._lib.frz_tokenizer_encode(self._h, raw, len(raw), max_tokens,
                                             ids.ctypes.data, ids.size, ctypes.byref(count),
                                             ctypes.byref(res)))
        return ids

    def decode(self, ids):
        """The bytes the ids stand for, joined."""
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        n = ctypes.c_uint64()
        check(self._lib.frz_tokenizer_decode(self._h, ids.ctypes.data, ids.size, None, 0,
                                             ctypes.byref(n)))
        buf = ctypes.create_string_buffer(max(n.value, 1))
        check(self._lib.frz_tokenizer_decode(self._h, ids.ctypes.data, ids.size, buf, n.value,
                                             ctypes.byref(n)))
        return buf.raw[:n.value]

    def texts(self, ids):
        """Each id's text as a fresh UTF-8 stream gives it (whole characters;
        the last with what ending the stream gives): a list of str."""
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        n = ctypes.c_uint64()
        offsets = np.zeros(ids.size + 1, dtype=np.uint64)
        check(self._lib.frz_tokenizer_texts(self._h, ids.ctypes.data, ids.size, None, 0,
                                            ctypes.byref(n), offsets.ctypes.data))
        buf = ctypes.create_string_buffer(max(n.value, 1))
        check(self._lib.frz_tokenizer_texts(self._h, ids.ctypes.data, ids.size, buf, n.value,
                                            ctypes.byref(n), offsets.ctypes.data))
        pool = buf.raw[:n.value]
        return [pool[offsets[i]:offsets[i + 1]].decode("utf-8") for i in range(ids.size)]
