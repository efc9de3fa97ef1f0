"""Writes the tokenizer's golden vectors from the reference's own fixtures:
tests/fixtures/tokenizer/gemma-3-1b-it-q4_0.gguf (the pinned model's
tokenizer entries alone) copied as it is, and the frozen encode cases of
tests/fixtures/tokenizer/gemma-3-1b-it-q4_0.inc (name, text, the ids Hugging
Face tokenizers and llama.cpp both give it) rewritten as cases.json, each
text's C string literal decoded to its bytes. Run in a tree that holds the
reference at /root/reference; the outputs are committed."""
import json
import shutil
from pathlib import Path

SRC = Path("/root/reference/tests/fixtures/tokenizer")
HERE = Path(__file__).resolve().parent


def c_string(s, i):
    """The C string literal starting at s[i] == '"': (its bytes, the index
    after its closing quote)."""
    assert s[i] == '"'
    i += 1
    out = bytearray()
    simple = {"n": 10, "t": 9, "r": 13, "\\": 92, '"': 34, "'": 39, "a": 7, "b": 8, "f": 12,
              "v": 11, "?": 63}
    while s[i] != '"':
        ch = s[i]
        if ch != "\\":
            out += ch.encode()
            i += 1
            continue
        nxt = s[i + 1]
        if nxt in simple:
            out.append(simple[nxt])
            i += 2
        elif nxt == "x":
            j = i + 2
            while j < len(s) and s[j] in "0123456789abcdefABCDEF":
                j += 1
            out.append(int(s[i + 2:j], 16) & 0xFF)
            i = j
        elif nxt in "01234567":
            j = i + 1
            while j < i + 4 and s[j] in "01234567":
                j += 1
            out.append(int(s[i + 1:j], 8) & 0xFF)
            i = j
        else:
            raise ValueError(f"escape \\{nxt}")
    return bytes(out), i + 1


def parse(text):
    cases = []
    for line in text.splitlines():
        line = line.strip()
        if not line.startswith('{"'):
            continue
        name, i = c_string(line, 1)
        while line[i] in ", ":
            i += 1
        body, i = c_string(line, i)
        while line[i] in ", ":
            i += 1
        assert line[i] == "{"
        j = line.index("}", i)
        ids = [int(x) for x in line[i + 1:j].replace(" ", "").split(",") if x]
        cases.append({"name": name.decode(), "text": body.decode("utf-8"), "ids": ids})
    return cases


def main():
    cases = parse((SRC / "gemma-3-1b-it-q4_0.inc").read_text(encoding="utf-8"))
    (HERE / "cases.json").write_text(json.dumps(cases, ensure_ascii=False, indent=1) + "\n",
                                     encoding="utf-8")
    shutil.copyfile(SRC / "gemma-3-1b-it-q4_0.gguf", HERE / "gemma-3-1b-it-q4_0.gguf")
    print(f"{len(cases)} cases")


if __name__ == "__main__":
    main()
