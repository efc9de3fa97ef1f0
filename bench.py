"""Benchmark: Gemma-3-1B Q4_0 greedy decode on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

A step is one fed decode token through all 26 layers, the tied 262,144-row
head, top-64 selection and the draw, on the full Gemma-3-1B shape with
seeded random-init Q4_0 weights, after a 4,096-token seeded random prompt
(prefilled untimed). The timed region replays K captured decode steps.

Also measured, for the JSON line:
  roofline     the Q4_0 dequant-GEMV of 6,912 x 1,152 (the MLP gate's shape):
               64 launches over 64 distinct weight copies captured in a HIP
               graph and replayed, timed with HIP events on the launching
               stream, so the weights stream from HBM; algorithmic bytes
               W 4,478,976 + x 4,608 + y 27,648 a launch. Its HBM traffic a
               launch comes from the committed rocprofv3 counter summary
               (profiles/q4_0_gemv_6912x1152_traffic.md), when present.
  cpu_baseline the CPU oracle (the reference's arithmetic restated in C++,
               OpenMP over output rows) decoding the same model on the host,
               a bounded sample of tokens after a 16-token prompt.
  parity       that sample's tokens against the GPU's from the same prompt.
  prefill      a 2,048-token prefill of seeded ids (four 512-token steps,
               logits at the last position) timed on the wall clock, with
               its rate against the fp32 matrix-core peak: the products
               run on fp32 MFMA in the reference's order of addition.
"""
import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
MFMA_FP32_PEAK_TFLOPS = 157.3
MFMA_BF16_PEAK_TFLOPS = 2500.0
# Gemma-3-1B's weight planes for the fast prefill mode: per layer Q/K/V
# (1,536 x 1,152), O (1,152 x 1,024), gate and up (2 x 6,912 x 1,152) and
# down (1,152 x 6,912), 4 bytes a weight (a bf16 pair).
WEIGHT_PLANE_BYTES = 26 * 4 * (1536 * 1152 + 1152 * 1024 + 2 * 6912 * 1152 + 1152 * 6912)  # dense
# 2 x 697,761,792 weights x 2,048 tokens + local and global attention + the
# last position's head product.
PREFILL_TOKENS = 2048
PREFILL_FLOP = 2.98e12
GEMV_ROWS, GEMV_COLS = 6912, 1152
GEMV_BYTES = GEMV_ROWS * GEMV_COLS // 32 * 18 + GEMV_COLS * 4 + GEMV_ROWS * 4
ROLES = ["q", "k", "v", "o", "gate", "up", "down", "attn_norm", "q_norm", "k_norm",
         "post_attn_norm", "ffn_norm", "post_ffn_norm"]

LAYER_WEIGHT_BYTES = 15_095_808
LAYER_GAIN_BYTES = 4 * (4 * 1152 + 2 * 256)
LAYER_KV_BYTES = 512 * 2 * 256 * 2
LAYER_ACT_BYTES = 4 * (3 * 1152 + 1536 + 1024 + 3 * 1152 + 2 * 6912 + 1152)


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=256)
    p.add_argument("--warmup", type=int, default=8)
    p.add_argument("--prompt", type=int, default=4096)
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--gemv-copies", type=int, default=64)
    p.add_argument("--gemv-iters", type=int, default=3000)
    p.add_argument("--cpu-seconds", type=float, default=15.0)
    p.add_argument("--parity-tokens", type=int, default=256)
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--no-steered", action="store_true",
                   help="skip the batch of 16 steered variants")
    p.add_argument("--steered-only", action="store_true",
                   help="only the batch of 16 steered variants (one JSON line)")
    p.add_argument("--no-pinned", action="store_true",
                   help="skip the decode over the pinned file's Q8_0/Q4_1 formats")
    p.add_argument("--eager", action="store_true",
                   help="launch decode kernels one by one instead of replaying a graph")
    p.add_argument("--roofline-only", action="store_true",
                   help="only the GEMV roofline and a 256 MiB device copy (for counter runs)")
    p.add_argument("--gguf-load", action="store_true",
                   help="only: write the synthetic full-size model as a GGUF file, load it "
                        "with frz_model_load_gguf, check its tokens, print one JSON line")
    p.add_argument("--prefill-only", action="store_true",
                   help="only the 2,048-token prefill, printed as one JSON line (for profiles)")
    p.add_argument("--probes", action="store_true",
                   help="only the floors: an empty kernel's launch (on the stream and "
                        "graph-replayed) and streaming reads of each decode product's "
                        "weight bytes (one JSON line)")
    p.add_argument("--profile-roles", action="store_true",
                   help="only: a decode step after the --prompt tokens and a 512-token "
                        "prefill step, each profiled launch by launch "
                        "(frz_model_profile_decode / _step), the launches named by the "
                        "graph's roles and timed (one JSON line)")
    p.add_argument("--library-gemm", action="store_true",
                   help="only: the vendor bf16 GEMM (torch matmul, hipBLASLt) at the fast "
                        "prefill's product shapes, one product each, for scale (one JSON "
                        "line)")
    p.add_argument("--gemv-stream", action="store_true",
                   help="with --roofline-only, time the GEMV launches back to back on the "
                        "stream (not each between its own events); with --probes, the "
                        "floors on the stream (not graph-replayed)")
    return p.parse_args()


TRAFFIC_FILE = ROOT / "profiles" / "q4_0_gemv_6912x1152_traffic.md"


def committed_traffic():
    """HBM bytes a GEMV launch moves, from the committed counter summary."""
    if not TRAFFIC_FILE.exists():
        return None
    for line in TRAFFIC_FILE.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


def calibration_copy(fz, dev, mib=256):
    """A plain device copy of known size: the counters' scale."""
    import ctypes
    n = mib << 20
    src, dst = dev.empty((n,), np.uint8), dev.empty((n,), np.uint8)
    for _ in range(3):
        fz._lib.check(fz.load().frz_copy(dev.handle, dst.ptr, src.ptr, ctypes.c_uint64(n)))
    src.free()
    dst.free()


def synth_all(fz, cfg, seed):
    t = {}
    for l in range(cfg.layers):
        for r in ROLES:
            t[(l, r)] = fz.synth_tensor(cfg, seed, l, r)
    t[(-1, "embedding")] = fz.synth_tensor(cfg, seed, -1, "embedding")
    t[(-1, "output_norm")] = fz.synth_tensor(cfg, seed, -1, "output_norm")
    return t


# frz_bench_gemv's timing modes: launches replayed from a graph, or launched
# on the stream, back to back either way.
GRAPH, STREAM = 1, 0


def gemv_roofline(fz, dev, copies, iters, seed, mode=STREAM):
    import ctypes
    rng = np.random.default_rng(seed + 1)
    blocks = GEMV_ROWS * GEMV_COLS // 32
    codes, scales = [], []
    for _ in range(copies):
        codes.append(dev.array(rng.integers(0, 256, blocks * 16, dtype=np.uint8)))
        d = np.abs(rng.normal(0, 0.02, blocks)).astype(np.float16)
        scales.append(dev.array(d.view(np.uint8)))
    x = dev.array(rng.normal(0, 1, GEMV_COLS).astype(np.float32))
    y = dev.empty((GEMV_ROWS,), np.float32)
    cp = (ctypes.c_void_p * copies)(*[c.ptr for c in codes])
    sp = (ctypes.c_void_p * copies)(*[s.ptr for s in scales])
    us = ctypes.c_double()
    fz._lib.check(fz.load().frz_bench_gemv(dev.handle, cp, sp, copies, GEMV_ROWS, GEMV_COLS,
                                          x.ptr, y.ptr, iters, mode, ctypes.byref(us)))
    for a in codes + scales + [x, y]:
        a.free()
    return us.value


# Weight bytes of each decode product of one layer (Q4_0: 18 bytes a block
# of 32), and the layer's.
PRODUCT_BYTES = {
    "qkv 1536x1152": 1536 * 1152 // 32 * 18,
    "o 1152x1024": 1152 * 1024 // 32 * 18,
    "gate+up 2x6912x1152": 2 * 6912 * 1152 // 32 * 18,
    "down 1152x6912": 1152 * 6912 // 32 * 18,
    "layer": LAYER_WEIGHT_BYTES,
}
STREAM_SPAN = 768 << 20  # bytes walked per size: past the 256 MB last-level cache


def floors(fz, dev, iters=6400, graph=True):
    """The launch floor (an empty kernel, on the stream and graph-replayed)
    and the streaming floor of each product's weight bytes (reads of
    distinct copies, so they come from HBM; graph-replayed unless `graph` is
    false, for the profiler)."""
    import ctypes
    lib = fz.load()
    us = ctypes.c_double()
    launch = {}
    for graph, name in ((0, "stream"), (1, "graph")):
        fz._lib.check(lib.frz_bench_launch_floor(dev.handle, iters, graph, ctypes.byref(us)))
        launch[name] = us.value
    sink = dev.empty((1024,), np.uint32)
    big = dev.empty((STREAM_SPAN,), np.uint8)
    streams = []
    for what, nbytes in PRODUCT_BYTES.items():
        nbytes = (nbytes + 255) // 256 * 256
        copies = max(1, STREAM_SPAN // nbytes)
        ptrs = (ctypes.c_void_p * copies)(*[big.ptr + c * nbytes for c in range(copies)])
        fz._lib.check(lib.frz_bench_stream(dev.handle, ptrs, copies, ctypes.c_uint64(nbytes),
                                           sink.ptr, max(iters // 10, copies),
                                           1 if graph else 0, ctypes.byref(us)))
        streams.append({"what": what, "bytes": nbytes, "copies": copies, "us": us.value,
                        "gbs": nbytes / (us.value * 1e-6) / 1e9,
                        "us_at_peak": nbytes / (HBM_PEAK_GBS * 1e9) * 1e6})
    big.free()
    sink.free()
    return {"launch_floor_us": launch, "stream_floor": streams,
            "how": "empty kernel (1 workgroup of 64 threads) launched back to back; "
                   "streaming reads by 1,024 workgroups x 256 threads, 4 uint4 loads in "
                   "flight a thread, over distinct copies spanning 768 MiB, "
                   + ("graph-replayed" if graph else "launched on the stream")
                   + "; HIP events on the launching stream"}


def host_cpu():
    """The host CPU's model name, from /proc/cpuinfo."""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def cpu_sample(orc, cfg, tensors, prompt, budget_s, max_tokens):
    """The oracle's greedy decode on the host, until `budget_s` seconds of
    decode or max_tokens; returns the tokens, the logits the last was drawn
    from, the decode seconds and the tokens decoded."""
    oracle = orc.OracleModel(cfg.as_dict(), tensors)
    oracle.set_edits(np.zeros(2 * cfg.layers, dtype=np.uint32))
    lg = None
    for p, t in enumerate(prompt):
        lg = oracle.token(t, p, want_logits=(p == len(prompt) - 1))
    tokens = [int(orc.topk(lg)[1][0])]
    pos = len(prompt)
    t0 = time.perf_counter()
    while len(tokens) < max_tokens:
        lg = oracle.token(tokens[-1], pos)
        pos += 1
        tokens.append(int(orc.topk(lg)[1][0]))
        if time.perf_counter() - t0 > budget_s and len(tokens) >= 3:
            break
    elapsed = time.perf_counter() - t0
    oracle.close()
    return tokens, lg, elapsed, len(tokens) - 1


def gguf_load(fz, seed):
    """The full-size synthetic model through a GGUF file: write, then time
    frz_model_load_gguf (index read, shape checks, file reads, uploads); its
    tokens must equal those of the same weights set directly."""
    import tempfile
    from frizzle_amd import gguf
    cfg = fz.gemma3_1b_config(context=4096)
    tensors = synth_all(fz, cfg, seed)
    dev = fz.Device(0)
    with tempfile.TemporaryDirectory() as tmp:
        path = Path(tmp) / "gemma3-1b-synthetic-q4_0.gguf"
        t0 = time.perf_counter()
        gguf.write_gemma3(path, cfg, lambda l, r: tensors[(l, r)].tobytes())
        write_s = time.perf_counter() - t0
        size = path.stat().st_size
        del tensors
        a = fz.Model(dev, cfg)
        dev.sync()
        t0 = time.perf_counter()
        a.load_gguf(path)
        dev.sync()
        load_s = time.perf_counter() - t0
    b = fz.Model(dev, cfg)
    b.synthesize(seed)
    prompt = np.random.default_rng(seed + 5).integers(0, cfg.vocab, 32).astype(np.uint32)
    same = bool(np.array_equal(a.generate(prompt, max_tokens=16), b.generate(prompt, max_tokens=16)))
    a.close()
    b.close()
    dev.close()
    log(f"gguf: wrote {size / 1e6:.0f} MB in {write_s:.1f}s, loaded in {load_s:.2f}s")
    print(json.dumps({"gguf_load": True, "file_bytes": size, "load_seconds": load_s,
                      "load_gbs": size / load_s / 1e9, "tokens_identical_to_direct_upload": same,
                      "model": "full 26-layer Gemma-3-1B shape, synthetic Q4_0"}))


def pinned_formats(fz, model, cfg, seed):
    """Gives the model the pinned file's formats (device_layout.h:64-66): the
    embedding, and so the tied head, in Q8_0 and the first three downs in
    Q4_1, as seeded blocks of the same scales as the Q4_0 ones."""
    rng = np.random.default_rng(seed + 5)

    def blocks(rows, cols, fmt):
        n = rows * cols // 32
        d = np.abs(rng.normal(0.0, 0.02, n)).astype(np.float16)
        if fmt == fz.Q8_0:
            d = (d.astype(np.float32) / 16).astype(np.float16)  # codes 16 times wider
            out = np.empty((n, 34), dtype=np.uint8)
            out[:, 2:] = rng.integers(0, 256, size=(n, 32), dtype=np.uint8)
        else:
            m = (-d.astype(np.float32) * 8).astype(np.float16)
            out = np.empty((n, 20), dtype=np.uint8)
            out[:, 2:4] = m.view(np.uint8).reshape(n, 2)
            out[:, 4:] = rng.integers(0, 256, size=(n, 16), dtype=np.uint8)
        out[:, 0:2] = d.view(np.uint8).reshape(n, 2)
        return out.reshape(-1)

    model.set_tensor(-1, "embedding", blocks(cfg.vocab, cfg.hidden, fz.Q8_0), fz.Q8_0)
    for layer in range(3):
        model.set_tensor(layer, "down", blocks(cfg.hidden, cfg.ffn, fz.Q4_1), fz.Q4_1)


def steered_batch(fz, model, dev, cfg, seed, prompt_len=1024, variants=16, tokens=128):
    """One original and variants - 1 steered replies to one seeded prompt,
    decoded as one batch at temperature 1 from one seed; each steered variant
    pins 1 to 32 seeded neurons of seeded layers to values in [-20, 20]. The
    second run reuses the cached prompt, so it times the cache copies and
    the batched decode; the residual capture ([tokens][layers][variants]
    [hidden] floats) is written in one run and copied to the host."""
    rng = np.random.default_rng(seed + 9)
    prompt = rng.integers(0, cfg.vocab, prompt_len).astype(np.uint32)
    sets = [[]]
    for _ in range(variants - 1):
        pins = {}
        for _ in range(int(rng.integers(1, 33))):
            layer, neuron = int(rng.integers(0, cfg.layers)), int(rng.integers(0, cfg.ffn))
            pins[(layer, neuron)] = fz.Edit(layer, neuron, fz.EditKind.SET,
                                            float(rng.uniform(-20, 20)))
        sets.append(list(pins.values()))
    samp = fz.sampling(temperature=1.0, top_k=64, top_p=1.0, min_p=0.0, seed=0x5EED)
    model.generate_variants(prompt, sets, samp=samp, max_tokens=tokens)  # prompt, warm-up
    dev.sync()
    t0 = time.perf_counter()
    replies = model.generate_variants(prompt, sets, samp=samp, max_tokens=tokens)
    dev.sync()
    plain = time.perf_counter() - t0
    t0 = time.perf_counter()
    replies_r, res = model.generate_variants(prompt, sets, samp=samp, max_tokens=tokens,
                                             residuals=True)
    dev.sync()
    captured = time.perf_counter() - t0
    same = all(np.array_equal(a, b) for a, b in zip(replies, replies_r))
    drawn = sum(len(r) for r in replies)
    return {"workload": f"1 original + {variants - 1} steered variants of one {prompt_len}-token "
                        f"seeded prompt, {tokens} tokens each at temperature 1.0 from one seed, "
                        "decoded as one batch (1-32 seeded pins in [-20, 20] a variant)",
            "tok_per_s": drawn / plain, "ms_per_step": plain * 1e3 / tokens,
            "tok_per_s_with_residuals": drawn / captured,
            "residual_bytes": int(res.nbytes), "tokens": drawn,
            "replies_identical_with_capture": bool(same)}


# One local layer's single-token decode (its five launches): algorithmic bytes
# = its Q4_0 weights, its gains, its 512 keys and values read (F16), and the
# activation rows its launches read and write.


def one_layer(fz, model, cfg, seed, position, iters=500):
    """Config 2: layer 0 (a sliding layer) decoding one token at `position`
    over its 512-key window, with 8 seeded pins in [-10, 10]."""
    rng = np.random.default_rng(seed + 11)
    neurons = sorted(rng.choice(cfg.ffn, 8, replace=False).tolist())
    pins = [fz.Edit(0, n, fz.EditKind.SET, float(rng.uniform(-10, 10))) for n in neurons]
    model.set_edits(fz.edit_table(pins, cfg.layers, 0))
    us = model.time_layer(0, position, iters)
    total = LAYER_WEIGHT_BYTES + LAYER_GAIN_BYTES + LAYER_KV_BYTES + LAYER_ACT_BYTES
    return {"workload": f"layer 0 (sliding, window 512) of the 26-layer model, one token at "
                        f"position {position}, 8 seeded pins in [-10, 10], its 5 launches "
                        "replayed as a graph",
            "us_per_layer": us, "algorithmic_bytes": total,
            "achieved_gbs": total / (us * 1e-6) / 1e9,
            "frac": total / (us * 1e-6) / 1e9 / HBM_PEAK_GBS}


def timed_decode(model, dev, prompt, warmup, steps, greedy):
    """The prompt in 512-token steps, `warmup` decode steps, then `steps`
    timed ones: (prefill seconds, wall seconds, µs/step by HIP events)."""
    model.set_edits(np.zeros(2 * model.cfg.layers, dtype=np.uint32))
    t0 = time.perf_counter()
    for p0 in range(0, len(prompt), 512):
        ids = prompt[p0:p0 + 512]
        model.step(p0, ids, logits=(p0 + len(ids) == len(prompt)), samp=greedy)
    dev.sync()
    prefill_s = time.perf_counter() - t0
    pos = len(prompt)
    if warmup:
        model.decode(pos, warmup, greedy)
        pos += warmup
    dev.sync()
    t0 = time.perf_counter()
    us_events = model.time_decode(pos, steps, greedy)
    dev.sync()
    return prefill_s, time.perf_counter() - t0, us_events


def profile_roles(fz, model, dev, cfg, prompt_len, seed, reps=20):
    """A fed decode step after a `prompt_len`-token prompt and a 512-token
    prefill step, each profiled: every launch's time (HIP events either side
    of it, launched one by one), grouped by its roles (the graph's names) and
    by local and global layers, averaged over `reps` steps."""
    rng = np.random.default_rng(seed + 7)
    prompt = rng.integers(0, cfg.vocab, prompt_len).astype(np.uint32)
    for p0 in range(0, prompt_len, 512):
        model.step(p0, prompt[p0:p0 + 512], logits=p0 + 512 >= prompt_len)

    def group(runs):
        by = {}
        for launches in runs:
            for roles, layer, us in launches:
                kind = ("output" if layer is None and roles.startswith("output") else
                        "embed" if layer is None else
                        "global" if (layer + 1) % cfg.pattern == 0 else "local")
                key = f"{kind}: {roles}"
                by.setdefault(key, []).append(us)
        n = len(runs)
        return {k: {"us_each": sum(v) / len(v), "launches_a_step": len(v) / n,
                    "us_a_step": sum(v) / n} for k, v in by.items()}

    decode_runs = []
    for i in range(reps + 2):
        launches, _ = model.profile_decode(prompt_len + i)
        if i >= 2:
            decode_runs.append(launches)
    ids = rng.integers(0, cfg.vocab, 512).astype(np.uint32)
    prefill_runs = [model.profile_step(0, ids, logits=True) for _ in range(3)][1:]
    dec = group(decode_runs)
    pre = group(prefill_runs)
    return {"workload": f"Gemma-3-1B Q4_0 decode step after a {prompt_len}-token prompt, and a "
                        "512-token prefill step (exact mode), launched one by one with HIP "
                        "events either side of each launch",
            "decode_us_a_step": sum(v["us_a_step"] for v in dec.values()),
            "decode": dec,
            "prefill_512_us_a_step": sum(v["us_a_step"] for v in pre.values()),
            "prefill_512": pre}


def library_gemm():
    """The vendor bf16 GEMM (torch.matmul over hipBLASLt) at the fast prefill's
    product shapes, one product each: tokens x rows x K, HIP events over 50
    calls after 5 warm-up calls."""
    import torch
    out = []
    for tokens, rows, k, name in [(512, 13824, 1152, "gate+up"), (512, 1152, 6912, "down"),
                                  (512, 1536, 1152, "qkv"), (512, 1152, 1024, "o"),
                                  (2048, 13824, 1152, "gate+up at 2,048 tokens")]:
        a = torch.randn(tokens, k, device="cuda", dtype=torch.bfloat16)
        b = torch.randn(rows, k, device="cuda", dtype=torch.bfloat16)
        for _ in range(5):
            c = a @ b.t()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(50):
            c = a @ b.t()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / 50
        out.append({"product": name, "tokens": tokens, "rows": rows, "k": k, "us": us,
                    "tflops": 2 * tokens * rows * k / (us * 1e-6) / 1e12})
        del c
    return out


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported "
              "(this build runs the forward path on a single MI355X).", file=sys.stderr)
        sys.exit(2)
    import frizzle_amd as fz
    sys.path.insert(0, str(ROOT / "tests"))
    if args.roofline_only:
        dev = fz.Device(0)
        us = gemv_roofline(fz, dev, args.gemv_copies, args.gemv_iters, args.seed,
                           STREAM if args.gemv_stream else GRAPH)
        calibration_copy(fz, dev)
        dev.close()
        achieved = GEMV_BYTES / (us * 1e-6) / 1e9
        print(json.dumps({"roofline_only": True, "us_per_launch": us, "achieved_gbs": achieved,
                          "frac": achieved / HBM_PEAK_GBS,
                          "timing": "back to back on the stream" if args.gemv_stream
                                    else "graph-replayed back to back"}))
        return

    if args.gguf_load:
        gguf_load(fz, args.seed)
        return

    if args.library_gemm:
        print(json.dumps({"library_gemm": True, "products": library_gemm()}))
        return

    if args.probes:
        dev = fz.Device(0)
        out = floors(fz, dev, graph=not args.gemv_stream)
        dev.close()
        print(json.dumps({"probes": True, **out}))
        return

    context = 8192
    assert args.prompt + args.warmup + args.steps + 1 <= context
    cfg = fz.gemma3_1b_config(context=context)
    dev = fz.Device(0)
    log(f"device {dev.limits.name.decode()} CUs {dev.limits.compute_units}")
    t0 = time.perf_counter()
    tensors = synth_all(fz, cfg, args.seed)
    model = fz.Model(dev, cfg)
    for (l, r), a in tensors.items():
        model.set_tensor(l, r, a)
    log(f"weights synthesized and uploaded in {time.perf_counter() - t0:.1f}s")
    if args.eager:
        model.set_graphs(False)
    greedy = fz.sampling()

    if args.profile_roles:
        out = profile_roles(fz, model, dev, cfg, args.prompt, args.seed)
        model.close()
        dev.close()
        print(json.dumps({"profile_roles": True, **out}))
        return
    if args.steered_only:
        out = steered_batch(fz, model, dev, cfg, args.seed)
        model.close()
        dev.close()
        print(json.dumps({"steered_only": True, **out}))
        return
    if args.prefill_only:
        args.no_cpu = True
    # Full-size parity sample: the oracle decodes from a short prompt on the
    # host (also the CPU baseline), then the GPU from the same prompt; the
    # tokens and the last step's logits must agree bit for bit.
    rng = np.random.default_rng(args.seed + 2)
    short = rng.integers(0, cfg.vocab, 16).astype(np.uint32)
    parity = None
    cpu_baseline = None
    if not args.no_cpu:
        import _oracle as orc
        threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
        cpu_tokens, cpu_logits, secs, decoded = cpu_sample(
            orc, cfg, tensors, short, args.cpu_seconds, args.parity_tokens)
        gpu_tokens = model.generate(short, max_tokens=len(cpu_tokens))
        gpu_logits = model.logits()
        differ = int(np.count_nonzero(gpu_logits.view(np.uint32) != cpu_logits.view(np.uint32)))
        parity = {"tokens_compared": len(cpu_tokens),
                  "tokens_identical": bool(np.array_equal(np.array(cpu_tokens), gpu_tokens)),
                  "last_logits_differing_bits": differ,
                  "prompt": "16 seeded ids", "model": "full 26-layer Gemma-3-1B shape"}
        cpu_baseline = {
            "value": decoded / secs, "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"{decoded} greedy decode tokens of the full 26-layer model after a "
                      f"16-token prompt (positions 17..{16 + decoded}), CPU oracle, "
                      f"OpenMP over output rows, {secs:.1f}s",
            "context": f"positions 17..{16 + decoded}: attention over at most "
                       f"{16 + decoded} keys, where the GPU's value is timed at positions "
                       f"{args.prompt + args.warmup + 1}..{args.prompt + args.warmup + args.steps} "
                       "(a 512-key window and up to 4,360 keys); the products, which "
                       "dominate a step, are the same"}
        log(f"parity {parity}; cpu {cpu_baseline['value']:.3f} tok/s")

    # A 2,048-token prefill (its positions are written again by the prompt
    # below).
    ids = rng.integers(0, cfg.vocab, PREFILL_TOKENS).astype(np.uint32)
    model.set_edits(np.zeros(2 * cfg.layers, dtype=np.uint32))
    prefill_runs = []
    for _ in range(2):
        dev.sync()
        t0 = time.perf_counter()
        for p0 in range(0, PREFILL_TOKENS, 512):
            model.step(p0, ids[p0:p0 + 512], logits=(p0 + 512 == PREFILL_TOKENS), samp=greedy)
        dev.sync()
        prefill_runs.append(time.perf_counter() - t0)
    prefill_2048 = min(prefill_runs)
    log(f"prefill {PREFILL_TOKENS} tokens: {prefill_2048 * 1e3:.2f} ms, "
        f"{PREFILL_FLOP / prefill_2048 / 1e12:.1f} TFLOP/s")
    # The same prefill in the fast mode: products on the bf16 matrix cores
    # over split operands (logits within 1e-3 relative, not bit for bit).
    # Setting the mode unpacks every layer's weights once into bf16 pair
    # planes (timed here, outside the prefill).
    dev.sync()
    t0 = time.perf_counter()
    model.set_prefill(fz.PREFILL_BF16)
    dev.sync()
    unpack_s = time.perf_counter() - t0
    fast_runs = []
    for _ in range(3):
        dev.sync()
        t0 = time.perf_counter()
        for p0 in range(0, PREFILL_TOKENS, 512):
            model.step(p0, ids[p0:p0 + 512], logits=(p0 + 512 == PREFILL_TOKENS), samp=greedy)
        dev.sync()
        fast_runs.append(time.perf_counter() - t0)
    model.set_prefill(fz.PREFILL_EXACT)
    prefill_fast = min(fast_runs)
    log(f"prefill {PREFILL_TOKENS} tokens, bf16 mode: {prefill_fast * 1e3:.2f} ms, "
        f"{PREFILL_FLOP / prefill_fast / 1e12:.1f} TFLOP/s")
    prefill_out = {
        "workload": f"Gemma-3-1B Q4_0 prefill of {PREFILL_TOKENS} seeded ids in 512-token "
                    "steps, logits at the last position",
        "flop": PREFILL_FLOP,
        "bf16": {"seconds": prefill_fast, "tflops": PREFILL_FLOP / prefill_fast / 1e12,
                 "peak_tflops": MFMA_BF16_PEAK_TFLOPS,
                 "frac": PREFILL_FLOP / prefill_fast / 1e12 / MFMA_BF16_PEAK_TFLOPS,
                 "arithmetic": "bf16 matrix cores over split operands (each weight and "
                               "activation a pair hi + lo of bf16, three products a pair), "
                               "fp32 accumulation; logits within 1e-3 relative of the "
                               "reference's",
                 "weight_planes": {"bytes": WEIGHT_PLANE_BYTES, "unpack_seconds": unpack_s,
                                   "note": "every layer's weights unpacked once, when the "
                                           "mode is set, into bf16 pair planes in the "
                                           "matrix instruction's operand order"}},
        "exact": {"seconds": prefill_2048, "tflops": PREFILL_FLOP / prefill_2048 / 1e12,
                  "peak_tflops": MFMA_FP32_PEAK_TFLOPS,
                  "frac": PREFILL_FLOP / prefill_2048 / 1e12 / MFMA_FP32_PEAK_TFLOPS,
                  "arithmetic": "f32 matrix cores, K=1 fma chains in the reference's order "
                                "(bit-exact)"}}
    if args.prefill_only:
        model.close()
        dev.close()
        print(json.dumps({"prefill_only": True, "tokens": PREFILL_TOKENS, **prefill_out}))
        return

    # The workload: a 4,096-token prompt, then greedy decode.
    prompt = rng.integers(0, cfg.vocab, args.prompt).astype(np.uint32)
    prefill_s, wall, us_events = timed_decode(model, dev, prompt, args.warmup, args.steps,
                                              greedy)
    log(f"prefill {args.prompt} tokens in {prefill_s:.3f}s")
    ms_per_step = wall * 1000.0 / args.steps
    log(f"decode {args.steps} steps: {ms_per_step * 1000:.1f} us/step wall, "
        f"{us_events:.1f} us/step events")

    # Config 2: one local layer's decode, at the position the decode reached.
    layer = one_layer(fz, model, cfg, args.seed, args.prompt + args.warmup + args.steps)
    log(f"one layer: {layer['us_per_layer']:.2f} us, {layer['achieved_gbs']:.0f} GB/s")

    # Config 5: the batch of steered variants.
    steered = None
    if not args.no_steered:
        steered = steered_batch(fz, model, dev, cfg, args.seed)
        log(f"steered batch: {steered['tok_per_s']:.0f} tok/s, "
            f"{steered['ms_per_step']:.2f} ms a step; with residuals "
            f"{steered['tok_per_s_with_residuals']:.0f} tok/s")

    # The same workload over the pinned file's formats (reported beside the
    # Q4_0 figure, which is the metric's).
    pinned = None
    if not args.no_pinned:
        pinned_formats(fz, model, cfg, args.seed)
        _, pwall, pus = timed_decode(model, dev, prompt, args.warmup, args.steps, greedy)
        pinned = {"workload": "the same decode with the pinned file's formats: Q8_0 "
                              "embedding and tied head (320,864,256 B), Q4_1 downs in "
                              "layers 0-2, Q4_0 elsewhere",
                  "tok_per_s": args.steps / pwall, "us_per_step_hip_events": pus}
        log(f"pinned formats: {args.steps / pwall:.1f} tok/s, {pus:.1f} us/step events")

    # The roofline's time: the launches back to back on the stream, timed
    # with HIP events there (the launches the profiler's trace of
    # --roofline-only --gemv-stream sees); beside it the graph-replayed rate.
    us = gemv_roofline(fz, dev, args.gemv_copies, args.gemv_iters, args.seed, STREAM)
    us_graph = gemv_roofline(fz, dev, args.gemv_copies, args.gemv_iters, args.seed, GRAPH)
    achieved = GEMV_BYTES / (us * 1e-6) / 1e9
    log(f"gemv 6912x1152: {us:.3f} us a launch on the stream, {achieved:.0f} GB/s "
        f"({us_graph:.3f} us graph-replayed)")
    model.close()
    dev.close()
    if cpu_baseline is not None:
        cpu_baseline["host_cpu"] = host_cpu()

    out = {
        "metric": "decode tok/s + Q4_0 GEMV achieved HBM GB/s (% of 8 TB/s), Gemma-3-1B",
        "value": args.steps / wall,
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32 (Q4_0 weights, F16 KV cache)",
        "data": "synthetic: seeded random-init Q4_0 weights, seeded random token ids",
        "config": {"workload": "Gemma-3-1B Q4_0 greedy decode after a 4096-token prompt "
                               "(26 layers, 262144-row tied head), batch 1",
                   "prompt_tokens": args.prompt, "decode_tokens": args.steps,
                   "prefill_seconds": prefill_s, "us_per_step_hip_events": us_events},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
                     "traffic": committed_traffic(),
                     "traffic_source": "committed counter summary "
                                       "profiles/q4_0_gemv_6912x1152_traffic.md (FETCH_SIZE "
                                       "+ WRITE_SIZE a dispatch, scaled by a 256 MiB copy's "
                                       "counters), not measured in this run",
                     "kernel": "Q4_0 decode GEMV 6912x1152 (gemv_pair_kernel<0, 4>: 18 lanes a row, 14 rows a workgroup)",
                     "launch_mode": "launches over 64 weight copies in turn (288 MiB), back "
                                    "to back on the stream, HIP events on that stream",
                     "us_per_launch": us,
                     "us_per_launch_graph": us_graph,
                     "profile": "profiles/q4_0_gemv_6912x1152_kernel_stats.md (rocprofv3 "
                                "per-dispatch durations of the same launches, which the "
                                "profiler runs apart)",
                     "algorithmic_bytes": GEMV_BYTES},
        "cpu_baseline": cpu_baseline,
        "parity": parity,
        "one_layer": layer,
        "pinned_formats": pinned,
        "steered_batch": steered,
        "prefill": prefill_out,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
