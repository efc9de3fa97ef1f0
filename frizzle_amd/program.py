"""The program boundary through the C ABI (frz_program_*): a graph's launch
list built over a model created from a plan, steps run at most two deep and
reported in run order by poll (kernels::Program, program.h:264-402;
kernels::Order, order.h:68-104)."""
import ctypes
from ctypes import POINTER, byref, c_char_p, c_float, c_int, c_uint32, c_void_p

from . import _lib, graph
from ._lib import check as _check
from ._lib import load

OK, STEP, DEVICE_LOST, CANCELLED, BUILD = 0, 4, 5, 6, 3

_libm = ctypes.CDLL("libm.so.6")
_libm.logf.restype = c_float
_libm.logf.argtypes = [c_float]


class StepRecord(ctypes.Structure):
    _fields_ = [("position", c_uint32), ("tokens", c_uint32), ("logits", c_uint32),
                ("fed", c_uint32), ("seed", c_uint32 * 2), ("top_k", c_uint32),
                ("temperature", c_float), ("top_p", c_float), ("min_p", c_float),
                ("log_min_p", c_float), ("padding", c_uint32 * 5), ("ids", c_uint32 * 512)]


class RunInput(ctypes.Structure):
    _fields_ = [("to", graph.CBinding), ("bytes", c_void_p)]


CALLBACK = ctypes.CFUNCTYPE(None, c_int, c_char_p, c_void_p, c_uint32, c_void_p)


class BuildRefused(ValueError):
    pass


def step_record(position, ids=(), logits=False, fed=False, samp=None):
    """kernels::Step with sampler::apply's settings (sampler.cpp:51-62)."""
    s = StepRecord()
    s.position = position
    ids = list(ids)
    s.tokens = 1 if fed else len(ids)
    s.logits = int(logits)
    s.fed = int(fed)
    if samp is None:
        s.top_k, s.temperature, s.top_p, s.min_p = 1, 0.0, 1.0, 0.0
        seed = 0
    else:
        s.top_k, s.temperature, s.top_p, s.min_p = (samp.top_k, samp.temperature, samp.top_p,
                                                    samp.min_p)
        seed = samp.seed
    s.log_min_p = _libm.logf(s.min_p) if s.min_p > 0 else 0.0
    s.seed[0], s.seed[1] = seed & 0xFFFFFFFF, (seed >> 32) & 0xFFFFFFFF
    for i, t in enumerate(ids):
        s.ids[i] = t
    return s


def check_launches(plan, launches, readback):
    """frz_program_check: (status, message) for a launch list over a plan."""
    cl = graph.CLaunches(launches)
    rb = graph.CBinding(*readback) if readback is not None else None
    msg = ctypes.create_string_buffer(1024)
    rc = load().frz_program_check(plan._h, cl.array, cl.count, byref(rb) if rb else None,
                                  msg, 1024)
    return rc, msg.value.decode()


class Program:
    """A program over `model` (created from `plan`)."""

    def __init__(self, model, plan, launches=None, readback=None):
        if launches is None:
            launches, readback = graph.gemma3_launches(plan)
        self._lib = load()
        self._cl = graph.CLaunches(launches)
        rb = graph.CBinding(*readback)
        msg = ctypes.create_string_buffer(1024)
        h = c_void_p()
        rc = self._lib.frz_program_build(model.handle, plan._h, self._cl.array, self._cl.count,
                                         byref(rb), byref(h), msg, 1024)
        if rc != OK:
            raise BuildRefused(msg.value.decode())
        self._h = h
        self.reports = []  # (status, message, record) in the order they came
        self._cb = CALLBACK(self._on_done)
        self._pcb = _lib.PROFILE_CALLBACK(self._on_profiled)
        self.profiles = []  # a profiled step's (status, begin_ns, end_ns, launches)
        self._inputs = []

    def _on_done(self, status, message, readback, nbytes, userdata):
        rec = None
        if readback and nbytes:
            rec = list((c_uint32 * 4).from_address(readback))
        self.reports.append((status, message.decode() if message else "", rec, userdata))
        if self.on_report:
            self.on_report(status, rec, userdata)

    def _on_profiled(self, status, message, readback, nbytes, times, userdata):
        t = times.contents
        launches = []
        for i in range(t.launch_count):
            lt = t.launches[i]
            launches.append({"roles": lt.role.decode(),
                             "layer": None if lt.layer == 0xFFFFFFFF else int(lt.layer),
                             "us": float(lt.microseconds),
                             "graph_index": int(t.launch_index[i]),
                             "end_ns": int(t.launch_end_ns[i])})
        self.profiles.append((status, int(t.begin_ns), int(t.end_ns), launches))
        self._on_done(status, message, readback, nbytes, userdata)

    on_report = None

    @staticmethod
    def _inputs_of(inputs):
        ins = (RunInput * max(1, len(inputs)))()
        keep = []
        for i, (binding, data) in enumerate(inputs):
            buf = ctypes.create_string_buffer(bytes(data), len(data))
            keep.append(buf)
            ins[i] = RunInput(graph.CBinding(*binding), ctypes.cast(buf, c_void_p))
        return ins, keep

    def run(self, record, inputs=(), tag=0):
        ins, keep = self._inputs_of(inputs)
        return self._lib.frz_program_run(self._h, byref(record), ins, len(inputs), self._cb,
                                         c_void_p(tag))

    def run_profiled(self, record, inputs=(), tag=0, launches=None):
        """Program::run_profiled: the step timed launch by launch; its report
        also lands in `profiles`. `launches` defaults to the whole graph."""
        ins, keep = self._inputs_of(inputs)
        n = self.launch_count if launches is None else launches
        return self._lib.frz_program_run_profiled(self._h, byref(record), ins, len(inputs), n,
                                                  self._pcb, c_void_p(tag))

    @property
    def launch_count(self):
        return self._lib.frz_program_launch_count(self._h)

    @property
    def can_profile(self):
        return bool(self._lib.frz_program_can_profile(self._h))

    def poll(self, wait=False):
        return self._lib.frz_poll(self._h, int(wait))

    @property
    def outstanding(self):
        return self._lib.frz_program_outstanding(self._h)

    def cancel(self):
        _check(self._lib.frz_program_cancel(self._h))

    def mark_lost(self):
        _check(self._lib.frz_program_mark_lost(self._h))

    def close(self):
        if getattr(self, "_h", None):
            self._lib.frz_program_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
