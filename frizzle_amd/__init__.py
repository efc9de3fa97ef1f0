"""MI355X-native (gfx950) Gemma-3-1B Q4_0 forward path.

The compute runs in libfrizzle_hip.so, a HIP library with a C ABI
(include/frizzle_hip.h); this package loads it with ctypes. Importing the
package does not load the library; the first call that needs it does, and
raises if it has not been built.
"""
from ._lib import FrzError, exported_symbols, load
from .runtime import (CAPTURE_SLOTS, PREFILL_BF16, PREFILL_EXACT, Q4_0, Q4_1, Q8_0,
                      TO_THE_END, Device,
                      DeviceArray, Edit, EditError, EditKind, Model, block_split,
                      capture_layout, capture_words,
                      edit_apply, edit_check, edit_table, gemma3_1b_config,
                      q4_0_split, rope_turns, sampling, synth_tensor,
                      tensor_bytes)

__all__ = [
    "FrzError", "exported_symbols", "load", "CAPTURE_SLOTS", "PREFILL_BF16", "PREFILL_EXACT",
    "Q4_0", "Q4_1", "Q8_0",
    "capture_layout", "capture_words",
    "TO_THE_END", "Device", "block_split",
    "DeviceArray", "Edit", "EditError", "EditKind", "Model", "edit_apply",
    "edit_check", "edit_table", "gemma3_1b_config", "q4_0_split",
    "rope_turns", "sampling", "synth_tensor", "tensor_bytes",
]
