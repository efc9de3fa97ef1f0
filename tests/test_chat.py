"""The chat tool's host parts (frizzle_amd/chat.py, after
tools/frizzle/main.cpp:1-60): the template, the --pin syntax, the stop set
from the file, and bad arguments. Host only."""
from pathlib import Path

import pytest

import frizzle_amd as fz
from frizzle_amd import chat, gguf
from frizzle_amd.tokenizer import Tokenizer

TOKENIZER = Path(__file__).parent / "golden" / "tokenizer" / "gemma-3-1b-it-q4_0.gguf"


def test_one_user_turn_as_the_template_renders_it():
    assert chat.render_user_turn(" \tHello\r\n") == (
        "<bos><start_of_turn>user\nHello<end_of_turn>\n<start_of_turn>model\n")
    # Only ASCII whitespace is trimmed.
    assert chat.render_user_turn(" hi ").startswith("<bos><start_of_turn>user\n hi ")
    # It encodes as the reference's "one user turn" case does.
    tok = Tokenizer.open(TOKENIZER)
    assert tok.encode(chat.render_user_turn("Hello")).tolist() == [
        2, 105, 2364, 107, 9259, 106, 107, 105, 4368, 107]


@pytest.mark.parametrize("text,kind,value", [("3:17=2.5", fz.EditKind.SET, 2.5),
                                             ("0:6911*-1.5", fz.EditKind.SCALE, -1.5),
                                             ("25:0=zero", fz.EditKind.ZERO, 0.0),
                                             ("1:2=-20", fz.EditKind.SET, -20.0)])
def test_pins(text, kind, value):
    e = chat.parse_pin(text, fz)
    assert (e.kind, e.value, e.start, e.until) == (kind, value, 0, fz.TO_THE_END)


@pytest.mark.parametrize("text", ["3:17", "a:1=2", "3:17=x", "3-17=2", "3:17=2=3", ":1=2"])
def test_pin_syntax_refused(text):
    with pytest.raises(ValueError, match="--pin"):
        chat.parse_pin(text, fz)


def test_the_stop_set_is_the_files():
    # Gemma 3's pinned file: eos is 106, <end_of_turn>; no eot or eom key.
    assert chat.stop_ids(gguf.Index.open(TOKENIZER)) == [106]


@pytest.mark.parametrize("argv", [[], ["--pin", "x", "hi"], ["--seed", "-1", "hi"],
                                  ["--message-file", "f", "hi"]])
def test_bad_arguments_exit_2(argv, capsys):
    assert chat.run(argv) == 2
