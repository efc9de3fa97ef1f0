"""The library's GGUF reader against the reference's model-file contract
(tests/contracts/gguf/model_file_test.cpp:52-156), on the reference's own
fixture files (tests/fixtures/gguf/, copied to tests/golden/gguf/), and the
Gemma 3 shapes read from a file's metadata. Host code only: no GPU.

What a fixture holds is stated by the script that wrote it
(scripts/make_gguf_fixtures.py:56-170); the valid file's contents are also
read by an independent parser here (helpers.read_gguf)."""
import struct
from pathlib import Path

import numpy as np
import pytest

import frizzle_amd as fz
from frizzle_amd import gguf
from helpers import read_gguf

FIX = Path(__file__).resolve().parent / "golden" / "gguf"


def error_of(data, file_size=None):
    try:
        gguf.Index.read(data, file_size).close()
        return "OK"
    except gguf.GgufError as e:
        return e.name


def fixture(name):
    return (FIX / f"{name}.gguf").read_bytes()


# model_file_test.cpp:52-73, 75-85
@pytest.mark.parametrize("name,error", [
    ("bad_magic", "BAD_MAGIC"),
    ("bad_version", "UNSUPPORTED_VERSION"),
    ("truncated_header", "SHORT_READ"),
    ("tensor_count_too_large", "COUNT_TOO_LARGE"),
    # claims five keys; the zero padding after the header reads as an empty key
    ("metadata_count_lies", "EMPTY_KEY"),
    ("negative_dimension", "NEGATIVE_DIMENSION"),
    ("unknown_tensor_type", "UNKNOWN_TENSOR_TYPE"),
    ("not_block_aligned", "ROW_NOT_WHOLE_BLOCKS"),
    ("duplicate_tensor_name", "DUPLICATE_TENSOR_NAME"),
    ("duplicate_tensor_name_apart", "DUPLICATE_TENSOR_NAME"),
    ("nested_array", "NESTED_ARRAY"),
    ("unknown_value_type", "UNKNOWN_VALUE_TYPE"),
    ("offset_past_eof", "TENSOR_DATA_OUT_OF_BOUNDS"),
    ("data_truncated", "TENSOR_DATA_OUT_OF_BOUNDS"),
    ("offset_overflow", "OFFSET_OVERFLOW"),
    ("alignment_wrong_type", "BAD_ALIGNMENT"),
    ("alignment_not_power_of_two", "BAD_ALIGNMENT"),
    ("misaligned_tensor_offset", "MISALIGNED_TENSOR_DATA"),
    ("overlapping_tensor_data", "OVERLAPPING_TENSOR_DATA"),
    ("empty_metadata_key", "EMPTY_KEY"),
    ("duplicate_metadata_key", "DUPLICATE_METADATA_KEY"),
    ("tensor_name_65_bytes", "TENSOR_NAME_TOO_LONG"),
    ("valid", "OK"),
])
def test_each_fixture_refused_by_name(name, error):
    assert error_of(fixture(name)) == error


def test_every_fixture_is_covered():
    names = {p.stem for p in FIX.glob("*.gguf")}
    assert len(names) == 23


def test_empty_file_is_short_read():  # model_file_test.cpp:87-90
    assert error_of(b"") == "SHORT_READ"


def test_valid_file_contents():
    # make_gguf_fixtures.py:65-82: token_embd.weight Q4_0 [64, 2] (4 blocks),
    # output_norm.weight F32 [4] = 1, 2, 3, 4; five metadata entries.
    data = fixture("valid")
    ix = gguf.Index.read(data)
    t = {d["name"]: d for d in ix.tensors}
    assert list(t) == ["token_embd.weight", "output_norm.weight"]
    e, n = t["token_embd.weight"], t["output_norm.weight"]
    assert (e["type"], e["shape"], e["elements"], e["bytes"]) == (2, [64, 2], 128, 72)
    assert (n["type"], n["shape"], n["elements"], n["bytes"]) == (0, [4], 4, 16)
    assert ix.metadata_count == 5
    assert ix.string("general.architecture") == "qwen3"
    assert ix.u32("general.alignment") == 32
    assert ix.u32("qwen3.block_count") == 28
    assert ix.u32("qwen3.attention.head_count") == 16
    assert ix.array("tokenizer.ggml.tokens") == (gguf.STRING, 3)
    # the absolute ranges hold exactly the bytes an independent parse finds
    ref = read_gguf(FIX / "valid.gguf")
    for name, d in t.items():
        raw = data[d["offset"]:d["offset"] + d["bytes"]]
        assert raw == ref[name.encode()][2]
        assert d["offset"] % 32 == 0
    assert np.array_equal(np.frombuffer(data[n["offset"]:n["offset"] + 16], np.float32),
                          [1, 2, 3, 4])
    with pytest.raises(fz.FrzError):
        ix.find("missing.weight")
    with pytest.raises(fz.FrzError):
        ix.u32("general.architecture")  # a string, not a number


def test_every_truncation_is_refused():  # model_file_test.cpp:92-116
    full = fixture("valid")
    ix = gguf.Index.read(full)
    last = max(d["offset"] + d["bytes"] for d in ix.tensors)
    assert last < len(full)
    accepted = [cut for cut in range(last) if error_of(full[:cut]) == "OK"]
    assert accepted == []


def test_front_asks_for_bytes_it_lacks():  # model_file_test.cpp:118-134
    full = fixture("valid")
    for cut in range(len(full) + 1):
        try:
            gguf.Index.read(full[:cut], len(full)).close()
        except gguf.GgufError as e:
            assert e.name == "NEED_MORE_BYTES", (cut, e.name)
            assert cut < e.needed <= len(full), (cut, e.needed)


def test_supplying_asked_bytes_converges():  # model_file_test.cpp:136-156
    full = fixture("valid")
    resident = 0
    for _ in range(1000):
        try:
            ix = gguf.Index.read(full[:resident], len(full))
            break
        except gguf.GgufError as e:
            assert e.name == "NEED_MORE_BYTES"
            resident = e.needed
    else:
        pytest.fail("did not converge")
    tensors = ix.tensors
    assert len(tensors) == 2
    assert resident <= tensors[0]["offset"]  # the index is whole with no data resident


def test_format_table():
    # GGUF's block layouts (ggml's own numbers) for the formats a Gemma 3
    # file carries, and a number GGUF leaves undefined.
    assert gguf.format_layout(0) == ("F32", 1, 4)
    assert gguf.format_layout(1) == ("F16", 1, 2)
    assert gguf.format_layout(2) == ("Q4_0", 32, 18)
    assert gguf.format_layout(3) == ("Q4_1", 32, 20)
    assert gguf.format_layout(8) == ("Q8_0", 32, 34)
    assert gguf.format_layout(12) == ("Q4_K", 256, 144)
    for undefined in (4, 5, 31, 999):
        with pytest.raises(fz.FrzError):
            gguf.format_layout(undefined)


# ---- larger and hostile inputs, made by the writer ------------------------------

def test_bounds_refuse_before_reading():
    base = b"GGUF" + struct.pack("<IQQ", 3, 0, 1)
    # a key longer than the reader's bound
    assert error_of(base + struct.pack("<Q", (1 << 20) + 1)) == "STRING_TOO_LONG"
    # an array longer than the reader's bound
    arr = base + struct.pack("<Q", 1) + b"a" + struct.pack("<IIQ", gguf.ARRAY, gguf.U8, (1 << 24) + 1)
    assert error_of(arr) == "ARRAY_TOO_LONG"
    # five dimensions
    t = b"GGUF" + struct.pack("<IQQ", 3, 1, 0) + struct.pack("<Q", 1) + b"t" + struct.pack("<I", 5)
    assert error_of(t + b"\0" * 64) == "TOO_MANY_DIMENSIONS"
    # extents whose product overflows 64 bits
    t = (b"GGUF" + struct.pack("<IQQ", 3, 1, 0) + struct.pack("<Q", 1) + b"t" +
         struct.pack("<Iqq", 2, 1 << 40, 1 << 40))
    assert error_of(t + b"\0" * 64) == "ELEMENT_COUNT_OVERFLOW"


def test_writer_round_trip(tmp_path):
    cfg = fz.gemma3_1b_config(context=4096)
    cfg.layers, cfg.vocab = 2, 512
    rng = np.random.default_rng(5)

    def tensor(layer, role):
        n = fz.tensor_bytes(cfg, role)
        return rng.integers(0, 256, n, dtype=np.uint8).tobytes()

    path = gguf.write_gemma3(tmp_path / "m.gguf", cfg, tensor)
    data = path.read_bytes()
    ix = gguf.Index.open(path)
    got = ix.gemma3_config(context=4096)
    for name, _ in cfg._fields_:
        assert getattr(got, name) == pytest.approx(getattr(cfg, name)), name
    ts = ix.tensors
    assert len(ts) == 2 + 13 * cfg.layers
    ref = read_gguf(path)
    for d in ts:
        assert data[d["offset"]:d["offset"] + d["bytes"]] == ref[d["name"].encode()][2]
    q = ix.find("blk.1.attn_q.weight")
    assert q["shape"] == [cfg.hidden, cfg.query_heads * cfg.head_dim] and q["type"] == 2
    assert ix.find("blk.0.attn_k_norm.weight")["shape"] == [cfg.head_dim]
    assert ix.find("token_embd.weight")["shape"] == [cfg.hidden, cfg.vocab]
    # the same index from its front, as the reader asks for it
    resident = 0
    while True:
        try:
            front = gguf.Index.read(data[:resident], len(data))
            break
        except gguf.GgufError as e:
            assert e.name == "NEED_MORE_BYTES"
            resident = e.needed
    assert resident <= min(d["offset"] for d in ts)
    assert front.tensors == ts


def test_gemma3_config_needs_its_keys(tmp_path):
    cfg = fz.gemma3_1b_config()
    p = gguf.write(tmp_path / "x.gguf", [], [("general.architecture", gguf.STRING, "llama")])
    with pytest.raises(fz.FrzError, match="gemma3"):
        gguf.Index.open(p).gemma3_config()
    p = gguf.write(tmp_path / "y.gguf", [], [("general.architecture", gguf.STRING, "gemma3"),
                                             ("gemma3.block_count", gguf.U32, 26)])
    with pytest.raises(fz.FrzError, match="embedding_length"):
        gguf.Index.open(p).gemma3_config()
    assert cfg.layers == 26


def test_open_missing_file(tmp_path):
    with pytest.raises(gguf.GgufError):
        gguf.Index.open(tmp_path / "absent.gguf")
