// Neuron pins as the reference defines them (src/core/edit/edit.h:10-167,
// edit.cpp:93-181): what a valid edit set is, and the u32 table the pin
// kernel reads. Host code only.

#include <algorithm>
#include <cmath>
#include <cstring>
#include <map>
#include <tuple>
#include <vector>

#include "../../include/frizzle_hip.h"
#include "backend.h"

namespace {

constexpr uint32_t kMaxEdits = 4096;
constexpr uint32_t kToTheEnd = 0xFFFFFFFFu;

// Step s at position origin + s, saturating at the end (edit.cpp:35-38).
uint32_t place(uint32_t step, uint32_t origin) {
  if (step == kToTheEnd || step > kToTheEnd - origin) return kToTheEnd;
  return step + origin;
}

// The fault in one edit on its own (edit.cpp:59-91).
int check_one(const frz_edit& e, uint32_t layers, uint32_t ffn) {
  if (e.kind > FRZ_EDIT_ZERO) return FRZ_EDIT_ERR_KIND;
  if (e.layer >= layers) return FRZ_EDIT_ERR_LAYER;
  if (e.neuron >= ffn) return FRZ_EDIT_ERR_NEURON;
  if (!std::isfinite(e.value)) return FRZ_EDIT_ERR_NOT_FINITE;
  if (e.kind == FRZ_EDIT_ZERO && e.value != 0.0f) return FRZ_EDIT_ERR_ZERO_VALUE;
  if (e.from >= e.until) return FRZ_EDIT_ERR_RANGE;
  return FRZ_EDIT_OK;
}

}  // namespace

extern "C" {

int frz_edit_check(const frz_edit* edits, uint32_t count, uint32_t layers, uint32_t ffn,
                   uint32_t* offending) {
  if (offending) *offending = 0;
  if (count > kMaxEdits) {
    if (offending) *offending = kMaxEdits;
    return FRZ_EDIT_ERR_TOO_MANY;
  }
  for (uint32_t i = 0; i < count; ++i) {
    if (int err = check_one(edits[i], layers, ffn)) {
      if (offending) *offending = i;
      return err;
    }
  }
  // Ranges held so far never overlap one another, so an edit overlaps one
  // of them exactly when it overlaps its neighbour before or after its key
  // (edit.cpp:111-133).
  using Key = std::tuple<uint32_t, uint32_t, uint32_t>;
  std::map<Key, uint32_t> held;
  for (uint32_t i = 0; i < count; ++i) {
    const frz_edit& e = edits[i];
    const Key key{e.layer, e.neuron, e.from};
    auto after = held.lower_bound(key);
    bool overlaps = false;
    if (after != held.end()) {
      const frz_edit& o = edits[after->second];
      overlaps = o.layer == e.layer && o.neuron == e.neuron && o.from < e.until;
    }
    if (!overlaps && after != held.begin()) {
      const frz_edit& o = edits[std::prev(after)->second];
      overlaps = o.layer == e.layer && o.neuron == e.neuron && e.from < o.until;
    }
    if (overlaps) {
      if (offending) *offending = i;
      return FRZ_EDIT_ERR_OVERLAP;
    }
    held.emplace(key, i);
  }
  return FRZ_EDIT_OK;
}

uint32_t frz_edit_table_words(uint32_t count, uint32_t layers) { return 2 * layers + 5 * count; }

// The table (edit.cpp:136-161): [first, count] a layer, then each edit by
// (layer, neuron, from, index) as [neuron, kind, value bits, first, end],
// its range placed at origin.
int frz_edit_table(const frz_edit* edits, uint32_t count, uint32_t layers, uint32_t origin,
                   uint32_t* out) {
  if (!out || (count && !edits)) return frz::fail(FRZ_ERR_ARGUMENT, "frz_edit_table: null");
  std::vector<uint32_t> order(count);
  for (uint32_t i = 0; i < count; ++i) order[i] = i;
  std::sort(order.begin(), order.end(), [edits](uint32_t a, uint32_t b) {
    const frz_edit& x = edits[a];
    const frz_edit& y = edits[b];
    return std::tie(x.layer, x.neuron, x.from, a) < std::tie(y.layer, y.neuron, y.from, b);
  });
  std::memset(out, 0, sizeof(uint32_t) * frz_edit_table_words(count, layers));
  uint32_t at = 2 * layers;
  for (uint32_t i : order) {
    const frz_edit& e = edits[i];
    if (e.layer >= layers) return frz::fail(FRZ_ERR_ARGUMENT, "frz_edit_table: layer");
    const uint32_t head = 2 * e.layer;
    if (out[head + 1] == 0) out[head] = at;
    ++out[head + 1];
    uint32_t bits;
    std::memcpy(&bits, &e.value, 4);
    out[at] = e.neuron;
    out[at + 1] = e.kind;
    out[at + 2] = bits;
    out[at + 3] = place(e.from, origin);
    out[at + 4] = place(e.until, origin);
    at += 5;
  }
  return FRZ_OK;
}

float frz_edit_apply(uint32_t kind, float value, float neuron) {
  switch (kind) {
    case FRZ_EDIT_SET: return value;
    case FRZ_EDIT_SCALE: return neuron * value;
    case FRZ_EDIT_ZERO: return 0.0f;
    default: return neuron;
  }
}

}  // extern "C"
