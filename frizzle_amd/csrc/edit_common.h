// A layer's pins applied to one neuron's activation, shared by the products
// whose epilogue applies them (the reference's edit kernel, edit.wgsl:55-76,
// fused into the gated product).
#pragma once

#include <stdint.h>

#include "numerics.h"

namespace frz {

// A layer's pins on neuron n at `position` (edit.wgsl:55-76): the layer's
// edits are sorted by neuron then first position (edit.cpp:20-31), so a
// binary search finds the neuron's; its ranges never overlap. `first` and
// `count` are the table's words for the layer.
__device__ __forceinline__ float apply_pin_words(const uint32_t* __restrict__ t, uint32_t first,
                                                 uint32_t count, uint32_t n, uint32_t position,
                                                 float value) {
  uint32_t lo = 0, hi = count;
  while (lo < hi) {
    const uint32_t mid = (lo + hi) >> 1;
    if (t[first + 5 * mid] < n) lo = mid + 1; else hi = mid;
  }
  for (uint32_t i = lo; i < count; ++i) {
    const uint32_t* e = t + first + 5 * i;
    if (e[0] != n) break;
    if (position < e[3] || position >= e[4]) continue;
    const float v = bits_to_float(e[2]);
    if (e[1] == 1u) {
      if (v != 1.0f) value = value * v;
    } else {
      value = v;
    }
  }
  return value;
}

__device__ __forceinline__ float apply_edits(const uint32_t* __restrict__ t, int layer, uint32_t n,
                                             uint32_t position, float value) {
  return apply_pin_words(t, t[2 * layer], t[2 * layer + 1], n, position, value);
}

}  // namespace frz
