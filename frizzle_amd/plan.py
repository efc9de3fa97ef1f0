"""The residency plan through the C ABI (frz_plan_gemma3): where a Gemma 3
file's weights, each layer's KV cache and the working buffers lie, and the
context offered, for given device limits and a load policy
(src/core/residency/plan.h:14-326, src/core/policy/policy.h:23-76). Pure:
no device is opened."""
import ctypes
from dataclasses import dataclass

from ._lib import (LoadPolicy, ModelConfig, Piece, PlanLimits, PlanSummary, Range, check,
                   load)

OK, EXCEEDS_BUDGET, ROW_EXCEEDS_BINDING, SCRATCH_EXCEEDS_BINDING, OVERFLOW, NOT_DESCRIBED = range(6)
ERRORS = ["Ok", "ExceedsBudget", "RowExceedsBinding", "ScratchExceedsBinding", "Overflow",
          "NotDescribed"]
WEIGHTS, CACHE, SCRATCH = 0, 1, 2

# WebGPU's default limits, which the reference's device is granted
# (gpu/device_requirements.h): 256 MiB a buffer, 128 MiB a binding, 256.
WEBGPU_DEFAULT_LIMITS = (256 << 20, 128 << 20, 256)


class PlanRefused(ValueError):
    """frz_plan_gemma3 refused: the PlanError, its subject and the summary
    (total_bytes holds what a 512-token context needs on ExceedsBudget)."""

    def __init__(self, code, subject, summary):
        super().__init__(f"plan refused: {ERRORS[code]} {subject}".strip())
        self.code = code
        self.error = ERRORS[code]
        self.subject = subject
        self.summary = summary


def default_policy():
    p = LoadPolicy()
    load().frz_load_policy_default(ctypes.byref(p))
    return p


def policy(memory_budget=None, rollback_reserve=None):
    p = default_policy()
    if memory_budget is not None:
        p.memory_budget = memory_budget
    if rollback_reserve is not None:
        p.rollback_reserve = rollback_reserve
    return p


def limits(max_buffer_size, max_storage_binding_size, storage_offset_alignment=256):
    return PlanLimits(max_buffer_size, max_storage_binding_size, storage_offset_alignment)


def device_limits(device):
    """The limits this device grants a plan (frz_device_plan_limits)."""
    lim = PlanLimits()
    check(load().frz_device_plan_limits(device.handle, ctypes.byref(lim)))
    return lim


def _summary(s):
    return {n: getattr(s, n) for n, _ in s._fields_}


@dataclass
class Group:
    members: tuple
    span: tuple  # (buffer, offset, length)


class Plan:
    """A plan held by the library (frz_plan_free on close)."""

    def __init__(self, index, lim=None, pol=None):
        lib = load()
        lim = lim or limits(*WEBGPU_DEFAULT_LIMITS)
        pol = pol or default_policy()
        h = ctypes.c_void_p()
        s = PlanSummary()
        subject = ctypes.create_string_buffer(256)
        rc = lib.frz_plan_gemma3(index._h, ctypes.byref(lim), ctypes.byref(pol), ctypes.byref(h),
                                 ctypes.byref(s), subject, 256)
        if rc != OK:
            raise PlanRefused(rc, subject.value.decode(), _summary(s))
        self._h = h
        self._lib = lib
        self.summary = _summary(s)

    def close(self):
        if getattr(self, "_h", None):
            self._lib.frz_plan_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def context_offered(self):
        return self.summary["context_offered"]

    def config(self):
        c = ModelConfig()
        check(self._lib.frz_plan_config(self._h, ctypes.byref(c)))
        return c

    def buffers(self):
        out = []
        for i in range(self.summary["buffers"]):
            pool, size = ctypes.c_int(), ctypes.c_uint64()
            check(self._lib.frz_plan_buffer(self._h, i, ctypes.byref(pool), ctypes.byref(size)))
            out.append((pool.value, size.value))
        return out

    def pieces(self, tensor):
        n = ctypes.c_uint32()
        check(self._lib.frz_plan_tensor(self._h, tensor, 0, None, ctypes.byref(n)))
        out = []
        for i in range(n.value):
            p = Piece()
            check(self._lib.frz_plan_tensor(self._h, tensor, i, ctypes.byref(p), None))
            out.append(((p.range.buffer, p.range.offset, p.range.length), p.first_row, p.rows))
        return out

    def groups(self):
        out = []
        for i in range(self.summary["groups"]):
            m = (ctypes.c_uint64 * 3)()
            n = ctypes.c_uint32()
            r = Range()
            check(self._lib.frz_plan_group(self._h, i, m, ctypes.byref(n), ctypes.byref(r)))
            out.append(Group(tuple(m[:n.value]), (r.buffer, r.offset, r.length)))
        return out

    def cache(self, layer):
        k, v, slots = Range(), Range(), ctypes.c_uint32()
        check(self._lib.frz_plan_cache(self._h, layer, ctypes.byref(k), ctypes.byref(v),
                                       ctypes.byref(slots)))
        return ((k.buffer, k.offset, k.length), (v.buffer, v.offset, v.length), slots.value)

    def scratch(self, purpose):
        r = Range()
        check(self._lib.frz_plan_scratch(self._h, purpose.encode(), ctypes.byref(r)))
        return (r.buffer, r.offset, r.length)

    def format(self, tensor):
        f = ctypes.c_uint32()
        check(self._lib.frz_plan_format(self._h, tensor, ctypes.byref(f)))
        return f.value

    def role(self, layer, role):
        from ._lib import ROLE
        t = ctypes.c_uint64()
        check(self._lib.frz_plan_role(self._h, layer, ROLE[role], ctypes.byref(t)))
        return t.value
