"""One message through a Gemma 3 GGUF file, as the reference's native tool
runs it (tools/frizzle/main.cpp:1-60): the reply, then with pins the edited
reply from the same seed, sharing the cached prompt.

    python -m frizzle_amd.chat [--model PATH] [--seed N] [--max-tokens N]
                               [--pin PIN]... [--context N] MESSAGE
    python -m frizzle_amd.chat [options] --message-file FILE

The message is wrapped as Gemma 3's chat template renders one user turn with
no system prompt, ASCII whitespace trimmed at both ends:
    <bos><start_of_turn>user\\n{message}<end_of_turn>\\n<start_of_turn>model\\n
A PIN is LAYER:NEURON=VALUE (set), LAYER:NEURON*FACTOR (scale) or
LAYER:NEURON=zero, over every step of the reply. Sampling is the reference's
default policy (temperature 0.8, top-k 40, top-p 0.95, min-p 0.05;
policy/policy.h:30-33) from --seed; a reply ends at a stop token (the file's
tokenizer.ggml.eos_token_id, eot and eom ids; runtime/stops.h:26-29) or at
--max-tokens. Exit status 0 when every reply completed, 1 with the refusal
on stderr, 2 for bad arguments.
"""
import argparse
import re
import sys

ASCII_SPACE = " \t\r\n\v\f"
TEMPLATE = "<bos><start_of_turn>user\n{}<end_of_turn>\n<start_of_turn>model\n"
PIN = re.compile(r"^(\d+):(\d+)(?:=(zero|[-+0-9.eE]+)|\*([-+0-9.eE]+))$")


def render_user_turn(message):
    """The prompt text for one user message (main.cpp:11-20)."""
    return TEMPLATE.format(message.strip(ASCII_SPACE))


def parse_pin(text, fz):
    """One --pin as an Edit over every step, or ValueError naming it."""
    m = PIN.match(text)
    if not m:
        raise ValueError(f"--pin {text}: write LAYER:NEURON=VALUE, LAYER:NEURON*FACTOR or "
                         "LAYER:NEURON=zero")
    layer, neuron = int(m.group(1)), int(m.group(2))
    try:
        if m.group(3) == "zero":
            return fz.Edit(layer, neuron, fz.EditKind.ZERO, 0.0)
        if m.group(3) is not None:
            return fz.Edit(layer, neuron, fz.EditKind.SET, float(m.group(3)))
        return fz.Edit(layer, neuron, fz.EditKind.SCALE, float(m.group(4)))
    except ValueError:
        raise ValueError(f"--pin {text}: not a number") from None


def stop_ids(index):
    """The file's stop tokens: eos, then eot and eom when it names them."""
    out = []
    for key in ("tokenizer.ggml.eos_token_id", "tokenizer.ggml.eot_token_id",
                "tokenizer.ggml.eom_token_id"):
        try:
            v = index.u32(key)
        except Exception:
            continue
        if v not in out:
            out.append(v)
    return out


def parse_args(argv):
    p = argparse.ArgumentParser(prog="python -m frizzle_amd.chat", add_help=True)
    p.add_argument("--model", default=".cache/models/gemma-3-1b-it-q4_0.gguf")
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--max-tokens", type=int, default=256)
    p.add_argument("--context", type=int, default=8192)
    p.add_argument("--pin", action="append", default=[])
    p.add_argument("--message-file")
    p.add_argument("message", nargs="?")
    a = p.parse_args(argv)
    if (a.message is None) == (a.message_file is None):
        p.error("give MESSAGE or --message-file, one of them")
    if a.seed < 0 or a.max_tokens < 0 or a.context < 1:
        p.error("--seed, --max-tokens and --context are not negative")
    return a


def run(argv, out=sys.stdout, err=sys.stderr):
    try:
        a = parse_args(argv)
    except SystemExit as e:
        return 2 if e.code else 0
    import frizzle_amd as fz
    from frizzle_amd import gguf
    from frizzle_amd.tokenizer import Tokenizer
    try:
        pins = [parse_pin(t, fz) for t in a.pin]
    except ValueError as e:
        print(e, file=err)
        return 2
    message = (open(a.message_file, encoding="utf-8").read() if a.message_file else a.message)
    try:
        index = gguf.Index.open(a.model)
        cfg = index.gemma3_config(context=a.context)
        tok = Tokenizer.open(a.model)
        stops = stop_ids(index)
        dev = fz.Device(0)
        print(f"device {dev.limits.name.decode()}, {dev.limits.compute_units} compute units",
              file=out)
        model = fz.Model(dev, cfg)
        model.load_gguf(a.model)
        prompt = tok.encode(render_user_turn(message), max_tokens=cfg.context)
        samp = fz.sampling(temperature=0.8, top_k=40, top_p=0.95, min_p=0.05, seed=a.seed)
        print(f"load: {a.model}; turn: seed {a.seed}, max tokens {a.max_tokens}, "
              f"temperature 0.8, top-k 40, top-p 0.95, min-p 0.05", file=out)
        runs = [((), "reply")] + ([(pins, "edited reply")] if pins else [])
        for edits, label in runs:
            if edits:
                print("pins: " + ", ".join(a.pin), file=out)
            reply = model.generate(prompt, edits, samp=samp, max_tokens=a.max_tokens,
                                   stop_ids=stops)
            text = "".join(tok.texts(reply)) if reply.size else ""
            print(f"{label}: {text}", file=out)
            stopped = reply.size and int(reply[-1]) in stops
            ended = f"stop (token {int(reply[-1])})" if stopped else "limit"
            print(f"end: {ended}, {reply.size} tokens; prompt {prompt.size} tokens, "
                  f"{model.reused} reused from the cache", file=out)
        model.close()
        dev.close()
    except Exception as e:  # the library's named refusal
        print(f"frizzle_amd.chat: {e}", file=err)
        return 1
    return 0


if __name__ == "__main__":
    sys.exit(run(sys.argv[1:]))
