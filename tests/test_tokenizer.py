"""Gemma 3's tokenizer against the reference's own fixtures
(tests/contracts/tokenizer/tokenizer_test.cpp): every frozen case encodes to
its ids and decodes back to its text, whole and a token at a time; the
vocabulary's counts as sentencepiece_bpe.h:84-88 and special.h:52-55 state
them; the merge order on a small vocabulary; refusals. Host only."""
import json
from pathlib import Path

import numpy as np
import pytest

from frizzle_amd import gguf
from frizzle_amd.tokenizer import BYTE, CONTROL, NORMAL, USER_DEFINED, EncodeError, Tokenizer

GOLDEN = Path(__file__).parent / "golden" / "tokenizer"
CASES = json.loads((GOLDEN / "cases.json").read_text(encoding="utf-8"))
SPACE = "▁"


@pytest.fixture(scope="module")
def gemma():
    t = Tokenizer.open(GOLDEN / "gemma-3-1b-it-q4_0.gguf")
    yield t
    t.close()


def decoded_text(text):
    # A typed U+2581 reads back as a space: the vocabulary spells both alike.
    return text.replace(SPACE, " ")


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_every_reference_text_encodes_to_its_ids(gemma, case):
    assert gemma.encode(case["text"]).tolist() == case["ids"]


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_every_reference_case_decodes_back(gemma, case):
    ids = case["ids"]
    assert gemma.decode(ids).decode("utf-8") == decoded_text(case["text"])
    # A token at a time through the stream: each token's text is whole
    # characters (some tokens are single bytes of one), joined the text.
    texts = gemma.texts(ids)
    assert len(texts) == len(ids)
    assert "".join(texts) == decoded_text(case["text"])
    assert "�" not in "".join(texts)


def test_an_empty_input_gives_no_text(gemma):
    assert gemma.texts([]) == []
    assert gemma.encode("").size == 0


def test_the_vocabulary_as_the_reference_counts_it(gemma):
    assert len(gemma) == 262_144
    assert gemma.longest_cover == 48
    types = np.array([gemma.token(i)[1] for i in range(len(gemma))])
    assert (types == BYTE).sum() == 256
    assert (types == CONTROL).sum() == 6_251
    assert (types == USER_DEFINED).sum() == 163
    special = [gemma.token(i)[0].decode("utf-8").replace(" ", SPACE)
               for i in np.nonzero((types == CONTROL) | (types == USER_DEFINED))[0]]
    special = [s for s in special if s]
    assert len(special) == 6_414
    assert max(len(s.encode()) for s in special) == 93
    # One normal token holds a U+2581 after its first character.
    straddles = [i for i in np.nonzero(types == NORMAL)[0]
                 if SPACE in gemma.token(i)[0].decode("utf-8", "replace")[1:]]
    assert [gemma.token(i)[0].decode() for i in straddles] == [">" + SPACE + "</"]


def test_control_tokens_written_as_text_are_single_ids(gemma):
    ids = gemma.encode("<start_of_turn>user\n")
    assert ids.tolist()[0] == 105
    assert gemma.token(105)[1] == CONTROL


def test_refusals(gemma):
    with pytest.raises(EncodeError) as e:
        gemma.encode(b"ok \xff bad")
    assert e.value.name == "INVALID_UTF8"
    with pytest.raises(EncodeError) as e:
        gemma.encode("<start_of_turn>" * 5, max_tokens=4)
    assert e.value.name == "TOO_MANY_TOKENS"
    # 200 bytes of ordinary text make at least ceil(200 / 48) = 5 tokens.
    with pytest.raises(EncodeError) as e:
        gemma.encode("x" * 200, max_tokens=4)
    assert e.value.name == "TOO_MANY_TOKENS" and e.value.least_tokens == 5
    assert gemma.encode("x" * 200, max_tokens=5).size >= 5
    with pytest.raises(EncodeError) as e:
        gemma.encode("y" * (512 * 1024 + 1))
    assert e.value.name == "TOO_LONG"


# ---- a small vocabulary: the merge order -------------------------------------------------

def small_vocab(tmp_path, extra, add_space_prefix=False, model="llama"):
    tokens = ["<unk>", "<bos>"] + [f"<0x{b:02X}>" for b in range(256)]
    types = [2, 3] + [BYTE] * 256
    scores = [0.0, 0.0] + [0.0] * 256
    for text, score in extra:
        tokens.append(text)
        types.append(NORMAL)
        scores.append(score)
    md = [("tokenizer.ggml.model", gguf.STRING, model),
          ("tokenizer.ggml.tokens", gguf.ARRAY, (gguf.STRING, tokens)),
          ("tokenizer.ggml.scores", gguf.ARRAY, (gguf.F32, scores)),
          ("tokenizer.ggml.token_type", gguf.ARRAY, (gguf.I32, types))]
    if add_space_prefix is not None:
        md.append(("tokenizer.ggml.add_space_prefix", gguf.BOOL, add_space_prefix))
    path = tmp_path / "vocab.gguf"
    gguf.write(path, [], md)
    return path, {t: i for i, t in enumerate(tokens)}


def test_highest_score_merges_first_and_the_leftmost_on_a_tie(tmp_path):
    path, ids = small_vocab(tmp_path, [("a", 0), ("b", 0), ("c", 0), ("ab", 1.0), ("bc", 2.0),
                                       ("abc", 0.5), ("aa", 3.0)])
    t = Tokenizer.open(path)
    # "bc" outscores "ab"; then a + bc make "abc".
    assert t.encode("abc").tolist() == [ids["abc"]]
    # "aaa": two "aa" candidates tie, the leftmost merges.
    assert t.encode("aaa").tolist() == [ids["aa"], ids["a"]]
    # A character without a normal token is its UTF-8 bytes.
    assert t.encode("é").tolist() == [ids["<0xC3>"], ids["<0xA9>"]]
    assert t.decode(t.encode("é")) == "é".encode()
    # A space is U+2581, with no token here: its three bytes; nothing added.
    assert t.encode(" a").tolist() == [ids["<0xE2>"], ids["<0x96>"], ids["<0x81>"], ids["a"]]
    t.close()


@pytest.mark.parametrize("prefix,why", [(True, "true is not supported"),
                                        (None, "not declared")])
def test_a_space_prefix_is_refused_unless_declared_false(tmp_path, prefix, why):
    path, _ = small_vocab(tmp_path, [("a", 0)], add_space_prefix=prefix)
    with pytest.raises(Exception, match=why):
        Tokenizer.open(path)


def test_other_tokenizers_are_refused(tmp_path):
    path, _ = small_vocab(tmp_path, [("a", 0)], model="gpt2")
    with pytest.raises(Exception, match="not SentencePiece BPE"):
        Tokenizer.open(path)
    with pytest.raises(Exception, match="tokenizer.ggml.model"):
        Tokenizer.open(Path(__file__).parent / "golden" / "gguf" / "valid.gguf")
