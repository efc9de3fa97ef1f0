"""The chat tool end to end on the GPU (frizzle_amd/chat.py, after
tools/frizzle/main.cpp): a GGUF file holding the pinned model's tokenizer and
seeded synthetic weights of Gemma 3's shapes (3 layers); the message
templated, encoded, the reply sampled and decoded, then the pinned reply from
the same seed reusing the prompt but its last token. The printed replies are
the library's own generate() for the same ids, decoded."""
import io
import re
from pathlib import Path

import numpy as np
import pytest

import frizzle_amd as fz
from frizzle_amd import chat, gguf
from frizzle_amd.tokenizer import Tokenizer
from test_gpu_model import ROLES

pytestmark = pytest.mark.gpu

TOKENIZER = Path(__file__).parent / "golden" / "tokenizer" / "gemma-3-1b-it-q4_0.gguf"


def model_file(path, cfg, seed):
    tok = Tokenizer.open(TOKENIZER)
    entries = [tok.token(i) for i in range(len(tok))]
    md = [("tokenizer.ggml.model", gguf.STRING, "llama"),
          ("tokenizer.ggml.add_space_prefix", gguf.BOOL, False),
          ("tokenizer.ggml.eos_token_id", gguf.U32, 106),
          ("tokenizer.ggml.tokens", gguf.ARRAY, (gguf.STRING, [e[0] for e in entries])),
          ("tokenizer.ggml.scores", gguf.ARRAY, (gguf.F32, [e[2] for e in entries])),
          ("tokenizer.ggml.token_type", gguf.ARRAY, (gguf.I32, [e[1] for e in entries]))]
    t = {(l, r): fz.synth_tensor(cfg, seed, l, r) for l in range(cfg.layers) for r in ROLES}
    t[(-1, "embedding")] = fz.synth_tensor(cfg, seed, -1, "embedding")
    t[(-1, "output_norm")] = fz.synth_tensor(cfg, seed, -1, "output_norm")
    gguf.write_gemma3(path, cfg, lambda l, r: t[(l, r)].tobytes(), metadata=md)
    return tok


def test_the_chat_tool_prints_the_replies_the_library_gives(device, tmp_path):
    cfg = fz.gemma3_1b_config(context=1024, layers=3, pattern=3, window=64,
                              local_slots=64 + 512 + 64)
    path = tmp_path / "chat.gguf"
    tok = model_file(path, cfg, seed=91)
    out, err = io.StringIO(), io.StringIO()
    rc = chat.run(["--model", str(path), "--seed", "5", "--max-tokens", "7", "--context", "1024",
                   "--pin", "0:5=20", "--pin", "2:77*-3", "Why is the sky blue?"],
                  out=out, err=err)
    assert rc == 0, err.getvalue()
    # A reply's text may hold newlines: each runs from its label to the
    # "end: " line after it.
    runs = re.findall(r"(?:^|\n)(?:edited )?reply: (.*?)\nend: ([^\n]*)", out.getvalue(), re.S)
    assert len(runs) == 2, out.getvalue()
    replies = [r[0] for r in runs]
    ends = ["end: " + r[1] for r in runs]
    prompt = tok.encode(chat.render_user_turn("Why is the sky blue?"))
    # The edited run reuses the prompt but its last token.
    assert ends[1].endswith(f"prompt {prompt.size} tokens, {prompt.size - 1} reused from the cache")
    model = fz.Model(device, cfg)
    model.load_gguf(path)
    samp = fz.sampling(temperature=0.8, top_k=40, top_p=0.95, min_p=0.05, seed=5)
    pins = [chat.parse_pin("0:5=20", fz), chat.parse_pin("2:77*-3", fz)]
    for edits, printed in zip([(), pins], replies):
        ids = model.generate(prompt, edits, samp=samp, max_tokens=7, stop_ids=[106])
        assert printed == "".join(tok.texts(ids))
    model.close()
