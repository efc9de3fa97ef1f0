// The capture store's layout (src/core/capture/capture.h:43-75): where every
// layer's captured values lie, in 32-bit words. Pure host code.
//
// Region 1 is every layer's neurons, in layer order, the feed-forward width
// each. Region 2 then holds, layer by layer, the residual, the attention
// block's and the MLP block's additions (the embedding width each), the
// query (query heads x head dimension), the attention weights (query heads
// x keys), the statistics (query heads x 2: m then l) and the readout
// (64 pairs of logit bits and token). keys = min(window, context): a global
// layer's window is the context the model was shaped with, so the store
// depends on the model's shapes alone.

#include <algorithm>
#include <cstdint>

#include "../../include/frizzle_hip.h"

namespace {

constexpr uint32_t kReadoutWords = 2 * 64;

bool shapes_ok(const frz_model_config* c) {
  return c && c->layers > 0 && c->hidden > 0 && c->ffn > 0 && c->head_dim > 0 &&
         c->query_heads > 0 && c->window > 0 && c->pattern > 0 && c->context > 0;
}

struct Widths {
  uint32_t keys, window, full;
};

Widths widths_of(const frz_model_config* c, int layer) {
  const bool global = layer % c->pattern == c->pattern - 1;
  const uint32_t window = (uint32_t)(global ? c->context : c->window);
  return {std::min(window, (uint32_t)c->context), window, window >= (uint32_t)c->context ? 1u : 0u};
}

// Words of one layer's region-2 slots.
uint64_t layer_words(const frz_model_config* c, int layer) {
  const uint64_t qh = (uint64_t)c->query_heads;
  return 3ull * c->hidden + qh * c->head_dim + qh * widths_of(c, layer).keys + 2 * qh +
         kReadoutWords;
}

}  // namespace

extern "C" {

uint64_t frz_capture_words(const frz_model_config* c, uint64_t* neuron_words) {
  if (!shapes_ok(c)) return 0;
  const uint64_t neurons = (uint64_t)c->layers * (uint64_t)c->ffn;
  uint64_t words = neurons;
  for (int l = 0; l < c->layers; ++l) words += layer_words(c, l);
  if (neuron_words) *neuron_words = neurons;
  // A slot's first word is a u32 (a launch constant in the reference).
  return words >= (1ull << 32) ? 0 : words;
}

int frz_capture_layer(const frz_model_config* c, int layer, frz_capture_slots* out) {
  if (!out || !shapes_ok(c) || layer < 0 || layer >= c->layers || frz_capture_words(c, nullptr) == 0)
    return FRZ_ERR_ARGUMENT;
  uint64_t at = (uint64_t)c->layers * (uint64_t)c->ffn;
  for (int l = 0; l < layer; ++l) at += layer_words(c, l);
  const Widths w = widths_of(c, layer);
  const uint32_t qh = (uint32_t)c->query_heads;
  auto take = [&at](uint32_t width) {
    const frz_capture_slot s{(uint32_t)at, width};
    at += width;
    return s;
  };
  out->neurons = frz_capture_slot{(uint32_t)((uint64_t)layer * c->ffn), (uint32_t)c->ffn};
  out->residual = take((uint32_t)c->hidden);
  out->attention_added = take((uint32_t)c->hidden);
  out->mlp_added = take((uint32_t)c->hidden);
  out->query = take(qh * (uint32_t)c->head_dim);
  out->weights = take(qh * w.keys);
  out->stats = take(2 * qh);
  out->readout = take(kReadoutWords);
  out->keys = w.keys;
  out->query_heads = qh;
  out->window = w.window;
  out->full_attention = w.full;
  return FRZ_OK;
}

}  // extern "C"
