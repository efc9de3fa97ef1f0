"""The decode attention entry point that allocates nothing
(frz_op_rope_attention_noalloc) against the one that allocates its chunk
states (frz_op_rope_attention), through the C ABI: two calls in a row, the
second over fewer chunks, each bit for bit the allocating call's output and
cache append; and a window past the static workspace refused by name."""
import numpy as np
import pytest

import frizzle_amd as fz

pytestmark = pytest.mark.gpu


def _inputs(device, rng, slots):
    d = 256
    qkv = rng.normal(0, 2, 6 * d).astype(np.float32)
    qg = (1 + 0.1 * rng.normal(0, 1, d)).astype(np.float32)
    kg = (1 + 0.1 * rng.normal(0, 1, d)).astype(np.float32)
    kc = (rng.integers(-96, 97, slots * d) / 32.0).astype(np.float16).view(np.uint16)
    vc = (rng.integers(-96, 97, slots * d) / 32.0).astype(np.float16).view(np.uint16)
    return qkv, qg, kg, kc, vc


def _call(device, name, qkv, qg, kg, kc, vc, turns, slots, window, position):
    dq, dt, dqg, dkg = (device.array(a) for a in (qkv, turns, qg, kg))
    dk, dv = device.array(kc), device.array(vc)
    do = device.empty((4 * 256,), np.float32)
    fz._lib.check(getattr(fz.load(), name)(device.handle, dq.ptr, dt.ptr, dqg.ptr, dkg.ptr,
                                           dk.ptr, dv.ptr, do.ptr, slots, window, 1e-6, 0.0625,
                                           position))
    return do.numpy(), dk.numpy(), dv.numpy()


@pytest.mark.parametrize("cases", [
    [(5000, 4096, 8192, 1e6), (700, 512, 640, 1e4)],     # 65 chunks, then 9
    [(14000, 14272, 14272, 1e6), (63, 512, 5120, 1e4)],  # the most the workspace holds, then 1
])
def test_no_alloc_attention_equals_the_allocating_call(device, cases):
    for position, window, slots, base in cases:
        rng = np.random.default_rng(position + window)
        qkv, qg, kg, kc, vc = _inputs(device, rng, slots)
        turns = fz.rope_turns(base, 256)
        want = _call(device, "frz_op_rope_attention", qkv, qg, kg, kc, vc, turns, slots,
                     window, position)
        got = _call(device, "frz_op_rope_attention_noalloc", qkv, qg, kg, kc, vc, turns, slots,
                    window, position)
        for g, w, what in zip(got, want, ("output", "keys", "values")):
            assert np.array_equal(g.view(np.uint32) if g.dtype == np.float32 else g,
                                  w.view(np.uint32) if w.dtype == np.float32 else w), (what, position)


def test_no_alloc_attention_refuses_past_its_workspace(device):
    rng = np.random.default_rng(1)
    slots = 16384
    qkv, qg, kg, kc, vc = _inputs(device, rng, slots)
    turns = fz.rope_turns(1e6, 256)
    with pytest.raises(fz.FrzError, match="static workspace holds 224"):
        _call(device, "frz_op_rope_attention_noalloc", qkv, qg, kg, kc, vc, turns, slots,
              slots, 15000)
