"""ctypes bindings of the HIP backend's C ABI (include/frizzle_hip.h).

The library is libfrizzle_hip.so next to this file, built by
``python -m frizzle_amd.build``. There is no fallback: if the library is
missing, loading raises, naming how to build it.
"""
import ctypes
import os
from ctypes import (POINTER, c_char, c_double, c_float, c_int, c_uint16,
                    c_uint32, c_uint64, c_void_p)
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libfrizzle_hip.so"

FRZ_OK = 0
ROLE = {
    "q": 0, "k": 1, "v": 2, "o": 3, "gate": 4, "up": 5, "down": 6,
    "attn_norm": 7, "q_norm": 8, "k_norm": 9, "post_attn_norm": 10,
    "ffn_norm": 11, "post_ffn_norm": 12, "embedding": 13, "output_norm": 14,
}
LAYER_ROLES = [r for r, i in ROLE.items() if i <= 12]


class FrzError(RuntimeError):
    """A call across the C ABI returned a non-zero status."""

    def __init__(self, status, message):
        super().__init__(f"frizzle_hip status {status}: {message}")
        self.status = status


class Limits(ctypes.Structure):
    _fields_ = [("name", c_char * 64), ("memory_bytes", c_uint64),
                ("compute_units", c_int), ("lds_bytes_per_block", c_int)]


class Sampling(ctypes.Structure):
    _fields_ = [("top_k", c_uint32), ("temperature", c_float),
                ("top_p", c_float), ("min_p", c_float), ("seed", c_uint64)]


class ModelConfig(ctypes.Structure):
    _fields_ = [(n, c_int) for n in (
        "hidden", "ffn", "head_dim", "query_heads", "kv_heads", "layers",
        "vocab", "window", "pattern", "context", "local_slots")] + [
        ("rope_local", c_float), ("rope_global", c_float), ("epsilon", c_float)]

    def as_dict(self):
        return {n: getattr(self, n) for n, _ in self._fields_}


class Edit(ctypes.Structure):
    _fields_ = [("layer", c_uint32), ("neuron", c_uint32), ("kind", c_uint32),
                ("value", c_float), ("from_", c_uint32), ("until", c_uint32)]


class PlanLimits(ctypes.Structure):
    _fields_ = [("max_buffer_size", c_uint64), ("max_storage_binding_size", c_uint64),
                ("storage_offset_alignment", c_uint32)]


class LoadPolicy(ctypes.Structure):
    _fields_ = [("memory_budget", c_uint64), ("rollback_reserve", c_uint32)]


class Range(ctypes.Structure):
    _fields_ = [("buffer", c_uint32), ("offset", c_uint64), ("length", c_uint64)]


class Piece(ctypes.Structure):
    _fields_ = [("range", Range), ("first_row", c_uint64), ("rows", c_uint64)]


class PlanSummary(ctypes.Structure):
    _fields_ = [(n, c_uint32) for n in ("buffers", "tensors", "pieces", "groups", "layers",
                                        "scratch", "partial_rows", "context_offered",
                                        "trained_context")] + [
        (n, c_uint64) for n in ("weight_bytes", "cache_bytes", "scratch_bytes", "total_bytes")]


class GgufTensor(ctypes.Structure):
    _fields_ = [("name", c_char * 65), ("type", c_uint32), ("dimensions", c_uint32),
                ("shape", c_uint64 * 4), ("elements", c_uint64), ("offset", c_uint64),
                ("bytes", c_uint64)]


class CaptureSlot(ctypes.Structure):
    _fields_ = [("first", c_uint32), ("width", c_uint32)]


class CaptureSlots(ctypes.Structure):
    _fields_ = [(n, CaptureSlot) for n in (
        "neurons", "residual", "attention_added", "mlp_added", "query", "weights", "stats",
        "readout")] + [(n, c_uint32) for n in ("keys", "query_heads", "window",
                                                 "full_attention")]


class LaunchTime(ctypes.Structure):
    _fields_ = [("role", ctypes.c_char * 96), ("layer", c_uint32), ("graph_index", c_uint32),
                ("microseconds", c_double)]


class ProfileTimes(ctypes.Structure):
    _fields_ = [("begin_ns", c_uint64), ("end_ns", c_uint64),
                ("launch_index", POINTER(c_uint32)), ("launch_end_ns", POINTER(c_uint64)),
                ("launches", POINTER(LaunchTime)), ("launch_count", c_uint32)]


PROFILE_CALLBACK = ctypes.CFUNCTYPE(None, c_int, ctypes.c_char_p, c_void_p, c_uint32,
                                    POINTER(ProfileTimes), c_void_p)

_P = c_void_p
_S = ctypes.c_char_p
_SIGS = {
    "frz_last_error": (ctypes.c_char_p, []),
    "frz_open": (c_int, [c_int, POINTER(c_void_p), POINTER(Limits)]),
    "frz_close": (None, [_P]),
    "frz_sync": (c_int, [_P]),
    "frz_alloc": (c_int, [_P, c_uint64, POINTER(c_void_p)]),
    "frz_free": (c_int, [_P, _P]),
    "frz_write": (c_int, [_P, _P, _P, c_uint64]),
    "frz_read": (c_int, [_P, _P, _P, c_uint64]),
    "frz_fill_zero": (c_int, [_P, _P, c_uint64]),
    "frz_copy": (c_int, [_P, _P, _P, c_uint64]),
    "frz_q4_0_split": (c_int, [_P, c_uint64, _P, _P]),
    "frz_block_split": (c_int, [c_int, _P, c_uint64, _P, _P]),
    "frz_op_gemv_format": (c_int, [_P, c_int, _P, _P, c_int, c_int, _P, c_int, _P, c_int,
                                   c_uint32, c_int]),
    "frz_op_gather_format": (c_int, [_P, c_int, _P, _P, c_int, c_int, _P, c_uint32, c_float,
                                     _P]),
    "frz_op_gemv": (c_int, [_P, _P, _P, c_int, c_int, _P, c_int, _P, c_int,
                            c_uint32, c_int]),
    "frz_op_gated": (c_int, [_P, _P, _P, _P, _P, c_int, c_int, _P, _P,
                             c_uint32, c_uint32, _P, c_int]),
    "frz_op_gemm_bf16": (c_int, [_P, c_int, _P, _P, c_int, c_int, _P, c_int, _P, c_int,
                                 c_uint32, c_int]),
    "frz_op_gated_bf16": (c_int, [_P, _P, _P, _P, _P, c_int, c_int, _P, _P, c_uint32,
                                  c_uint32, _P, c_int]),
    "frz_op_norm": (c_int, [_P, _P, _P, _P, _P, _P, c_int, c_float, c_uint32,
                            c_int]),
    "frz_op_rope": (c_int, [_P, _P, _P, _P, _P, _P, _P, c_int, c_int, _P, _P,
                            c_int, c_int, c_int, c_int, c_float, c_uint32,
                            c_uint32]),
    "frz_op_attention": (c_int, [_P, _P, c_int, _P, _P, _P, c_int, c_int,
                                 c_int, c_int, c_int, c_float, c_uint32,
                                 c_uint32]),
    "frz_op_rope_attention": (c_int, [_P, _P, _P, _P, _P, _P, _P, _P, c_int,
                                      c_int, c_float, c_float, c_uint32]),
    "frz_op_rope_attention_noalloc": (c_int, [_P, _P, _P, _P, _P, _P, _P, _P, c_int,
                                              c_int, c_float, c_float, c_uint32]),
    "frz_op_gather": (c_int, [_P, _P, _P, c_int, c_int, _P, c_uint32, c_float,
                              _P]),
    "frz_op_edit": (c_int, [_P, _P, c_int, _P, c_int, c_uint32, c_uint32]),
    "frz_op_topk": (c_int, [_P, _P, c_int, _P]),
    "frz_op_draw": (c_int, [_P, _P, POINTER(Sampling), c_uint32, c_uint32,
                            _P]),
    "frz_op_numerics": (c_int, [_P, c_int, _P, _P, c_int]),
    "frz_bench_launch_floor": (c_int, [_P, c_int, c_int, POINTER(c_double)]),
    "frz_bench_stream": (c_int, [_P, POINTER(c_void_p), c_int, c_uint64, _P, c_int, c_int,
                                 POINTER(c_double)]),
    "frz_bench_gemv": (c_int, [_P, POINTER(c_void_p), POINTER(c_void_p), c_int,
                               c_int, c_int, _P, _P, c_int, c_int, POINTER(c_double)]),
    "frz_bench_gated": (c_int, [_P, POINTER(c_void_p), POINTER(c_void_p),
                                POINTER(c_void_p), POINTER(c_void_p), c_int,
                                c_int, c_int, _P, _P, c_int, c_int,
                                POINTER(c_double)]),
    "frz_rope_turns": (None, [c_float, c_int, POINTER(c_float)]),
    "frz_edit_check": (c_int, [_P, c_uint32, c_uint32, c_uint32,
                               POINTER(c_uint32)]),
    "frz_edit_table_words": (c_uint32, [c_uint32, c_uint32]),
    "frz_edit_table": (c_int, [_P, c_uint32, c_uint32, c_uint32, _P]),
    "frz_edit_apply": (c_float, [c_uint32, c_float, c_float]),
    "frz_gemma3_1b_config": (None, [POINTER(ModelConfig), c_int]),
    "frz_tensor_bytes": (c_uint64, [POINTER(ModelConfig), c_int]),
    "frz_synth_tensor": (c_int, [POINTER(ModelConfig), c_uint64, c_int, c_int,
                                 _P, c_uint64]),
    "frz_model_create": (c_int, [_P, POINTER(ModelConfig), POINTER(c_void_p)]),
    "frz_model_destroy": (None, [_P]),
    "frz_model_set_tensor": (c_int, [_P, c_int, c_int, _P, c_uint64]),
    "frz_model_set_tensor_format": (c_int, [_P, c_int, c_int, c_int, _P, c_uint64]),
    "frz_model_synthesize": (c_int, [_P, c_uint64]),
    "frz_model_set_edits": (c_int, [_P, _P, c_uint32]),
    "frz_model_set_graphs": (c_int, [_P, c_int]),
    "frz_model_set_prefill": (c_int, [_P, c_int]),
    "frz_model_step": (c_int, [_P, c_uint32, c_uint32, _P, c_int,
                               POINTER(Sampling)]),
    "frz_model_decode": (c_int, [_P, c_uint32, c_uint32, POINTER(Sampling),
                                 _P, _P]),
    "frz_model_read_logits": (c_int, [_P, _P, c_uint32]),
    "frz_model_read_record": (c_int, [_P, _P]),
    "frz_model_read_candidates": (c_int, [_P, _P]),
    "frz_model_read_hidden": (c_int, [_P, _P, c_uint32]),
    "frz_model_read_cache": (c_int, [_P, c_int, c_int, _P, c_uint64]),
    "frz_model_time_decode": (c_int, [_P, c_uint32, c_uint32,
                                      POINTER(Sampling), POINTER(c_double)]),
    "frz_generate": (c_int, [_P, _P, c_uint32, _P, c_uint32, POINTER(Sampling),
                             c_uint32, _P, c_uint32, _P, POINTER(c_uint32)]),
    "frz_model_get_config": (c_int, [_P, POINTER(ModelConfig)]),
    "frz_capture_words": (c_uint64, [POINTER(ModelConfig), POINTER(c_uint64)]),
    "frz_model_set_capture": (c_int, [_P, c_int]),
    "frz_tokenizer_open": (c_int, [_S, POINTER(c_void_p)]),
    "frz_tokenizer_free": (None, [_P]),
    "frz_tokenizer_size": (c_uint32, [_P]),
    "frz_tokenizer_longest_cover": (c_uint32, [_P]),
    "frz_tokenizer_token": (c_int, [_P, c_uint32, POINTER(_S), POINTER(c_uint32),
                                    POINTER(ctypes.c_int32), POINTER(c_float)]),
    "frz_tokenizer_encode": (c_int, [_P, _S, c_uint64, c_uint32, _P, c_uint64, POINTER(c_uint64),
                                     _P]),
    "frz_tokenizer_decode": (c_int, [_P, _P, c_uint32, _P, c_uint64, POINTER(c_uint64)]),
    "frz_tokenizer_texts": (c_int, [_P, _P, c_uint32, _P, c_uint64, POINTER(c_uint64), _P]),
    "frz_model_reused": (c_uint32, [_P]),
    "frz_model_time_layer": (c_int, [_P, c_int, c_uint32, c_uint32, POINTER(c_double)]),
    "frz_model_read_capture": (c_int, [_P, _P, c_uint64]),
    "frz_capture_layer": (c_int, [POINTER(ModelConfig), c_int, POINTER(CaptureSlots)]),
    "frz_generate_variants": (c_int, [_P, _P, c_uint32, c_uint32, _P, c_uint32,
                                      POINTER(Sampling), c_uint32, _P, c_uint32, _P, _P, _P]),
    "frz_gguf_read": (c_int, [_P, c_uint64, c_uint64, POINTER(c_void_p), POINTER(c_uint64)]),
    "frz_gguf_open": (c_int, [_S, POINTER(c_void_p)]),
    "frz_gguf_free": (None, [_P]),
    "frz_gguf_error_text": (_S, [c_int]),
    "frz_gguf_format": (c_int, [c_uint32, POINTER(_S), POINTER(c_uint32), POINTER(c_uint32)]),
    "frz_gguf_tensor_count": (c_uint64, [_P]),
    "frz_gguf_tensor_at": (c_int, [_P, c_uint64, POINTER(GgufTensor)]),
    "frz_gguf_find": (c_int, [_P, _S, POINTER(GgufTensor)]),
    "frz_gguf_metadata_count": (c_uint64, [_P]),
    "frz_gguf_get_u32": (c_int, [_P, _S, POINTER(c_uint32)]),
    "frz_gguf_get_f32": (c_int, [_P, _S, POINTER(c_float)]),
    "frz_gguf_get_string": (c_int, [_P, _S, _P, c_uint64, POINTER(c_uint64)]),
    "frz_gguf_get_array": (c_int, [_P, _S, POINTER(c_uint32), POINTER(c_uint64)]),
    "frz_gemma3_config_from_gguf": (c_int, [_P, c_int, POINTER(ModelConfig)]),
    "frz_model_load_gguf": (c_int, [_P, _S]),
    "frz_load_policy_default": (None, [POINTER(LoadPolicy)]),
    "frz_plan_gemma3": (c_int, [_P, POINTER(PlanLimits), POINTER(LoadPolicy), POINTER(c_void_p),
                                POINTER(PlanSummary), _P, ctypes.c_size_t]),
    "frz_plan_free": (None, [_P]),
    "frz_plan_error_text": (_S, [c_int]),
    "frz_plan_config": (c_int, [_P, POINTER(ModelConfig)]),
    "frz_plan_buffer": (c_int, [_P, c_uint32, POINTER(c_int), POINTER(c_uint64)]),
    "frz_plan_tensor": (c_int, [_P, c_uint64, c_uint32, POINTER(Piece), POINTER(c_uint32)]),
    "frz_plan_group": (c_int, [_P, c_uint32, POINTER(c_uint64), POINTER(c_uint32),
                               POINTER(Range)]),
    "frz_plan_cache": (c_int, [_P, c_uint32, POINTER(Range), POINTER(Range), POINTER(c_uint32)]),
    "frz_plan_scratch": (c_int, [_P, _S, POINTER(Range)]),
    "frz_plan_role": (c_int, [_P, c_int, c_int, POINTER(c_uint64)]),
    "frz_plan_summarize": (c_int, [_P, POINTER(PlanSummary)]),
    "frz_plan_format": (c_int, [_P, c_uint64, POINTER(c_uint32)]),
    "frz_device_plan_limits": (c_int, [_P, POINTER(PlanLimits)]),
    "frz_model_create_planned": (c_int, [_P, _P, POINTER(c_void_p)]),
    "frz_model_planned_buffer": (c_int, [_P, c_uint32, POINTER(c_void_p), POINTER(c_uint64)]),
    "frz_program_check": (c_int, [_P, _P, c_uint32, _P, _P, ctypes.c_size_t]),
    "frz_program_build": (c_int, [_P, _P, _P, c_uint32, _P, POINTER(c_void_p), _P,
                                  ctypes.c_size_t]),
    "frz_program_run": (c_int, [_P, _P, _P, c_uint32, _P, _P]),
    "frz_poll": (c_int, [_P, c_int]),
    "frz_program_outstanding": (c_uint32, [_P]),
    "frz_program_cancel": (c_int, [_P]),
    "frz_program_destroy": (None, [_P]),
    "frz_program_mark_lost": (c_int, [_P]),
    "frz_model_profile_step": (c_int, [_P, c_uint32, c_uint32, _P, c_int, _P, _P, c_uint32,
                                       POINTER(c_uint32)]),
    "frz_model_profile_decode": (c_int, [_P, c_uint32, _P, _P, c_uint32, POINTER(c_uint32),
                                         POINTER(c_uint32)]),
    "frz_program_run_profiled": (c_int, [_P, _P, _P, c_uint32, c_uint32, PROFILE_CALLBACK, _P]),
    "frz_program_launch_count": (c_uint32, [_P]),
    "frz_program_can_profile": (c_int, [_P]),
}

_lib = None


def load():
    """The loaded library, with every entry point's signature set."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise OSError(
            f"{LIB_PATH} is missing: build it with `python -m frizzle_amd.build` "
            "(there is no CPU fallback)")
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def exported_symbols():
    """Every entry point this binding declares (all must exist in the .so)."""
    return sorted(_SIGS)


def check(status):
    if status != FRZ_OK:
        raise FrzError(status, load().frz_last_error().decode(errors="replace"))
    return status
