// The tokenizer's C ABI (include/frizzle_hip.h, the tokenizer section):
// Tokenizer::encode / decode (src/core/tokenizer/tokenizer.h:193-247), the
// capability table's load for "llama" (capability.h, sentencepiece_bpe.h),
// and a turn's input as text (detokenizer.h: texts). Host code only.

#include <cstring>
#include <string>
#include <vector>

#include "../../include/frizzle_hip.h"
#include "tokenizer.h"

namespace frz {
int fail(int status, const std::string& message);
}  // namespace frz

struct frz_tokenizer {
  frz::tok::Tokenizer t;
};

extern "C" {

int frz_tokenizer_open(const char* path, frz_tokenizer** out) {
  if (!path || !out) return frz::fail(FRZ_ERR_ARGUMENT, "frz_tokenizer_open: null argument");
  auto* t = new frz_tokenizer();
  std::string why;
  if (!t->t.load(path, &why)) {
    delete t;
    return frz::fail(FRZ_ERR_ARGUMENT, std::string("tokenizer: ") + why);
  }
  *out = t;
  return FRZ_OK;
}

void frz_tokenizer_free(frz_tokenizer* t) { delete t; }

uint32_t frz_tokenizer_size(const frz_tokenizer* t) { return t ? t->t.size() : 0; }

uint32_t frz_tokenizer_longest_cover(const frz_tokenizer* t) {
  return t ? (uint32_t)t->t.longest_cover() : 0;
}

int frz_tokenizer_token(const frz_tokenizer* t, uint32_t id, const char** text, uint32_t* bytes,
                        int32_t* type, float* score) {
  if (!t || id >= t->t.size()) return frz::fail(FRZ_ERR_ARGUMENT, "frz_tokenizer_token: id");
  if (text) *text = t->t.text(id).data();
  if (bytes) *bytes = (uint32_t)t->t.text(id).size();
  if (type) *type = t->t.type(id);
  if (score) *score = t->t.score(id);
  return FRZ_OK;
}

int frz_tokenizer_encode(const frz_tokenizer* t, const char* text, uint64_t bytes,
                         uint32_t max_tokens, uint32_t* ids, uint64_t cap, uint64_t* count,
                         frz_encode_result* result) {
  if (!t || (!text && bytes) || !count)
    return frz::fail(FRZ_ERR_ARGUMENT, "frz_tokenizer_encode: null argument");
  std::vector<uint32_t> out;
  const frz::tok::EncodeResult r =
      t->t.encode(std::string_view(text ? text : "", bytes), max_tokens, out);
  if (result) *result = frz_encode_result{r.error, r.least_tokens, r.normalized_bytes, r.raw_bytes};
  *count = out.size();
  if (ids) std::memcpy(ids, out.data(), std::min<uint64_t>(cap, out.size()) * 4);
  return FRZ_OK;
}

int frz_tokenizer_decode(const frz_tokenizer* t, const uint32_t* ids, uint32_t n, char* out,
                         uint64_t cap, uint64_t* bytes) {
  if (!t || (!ids && n) || !bytes)
    return frz::fail(FRZ_ERR_ARGUMENT, "frz_tokenizer_decode: null argument");
  std::string s;
  for (uint32_t i = 0; i < n; ++i) {
    if (ids[i] >= t->t.size()) return frz::fail(FRZ_ERR_ARGUMENT, "frz_tokenizer_decode: id");
    t->t.decode(ids[i], s);
  }
  *bytes = s.size();
  if (out) std::memcpy(out, s.data(), std::min<uint64_t>(cap, s.size()));
  return FRZ_OK;
}

int frz_tokenizer_texts(const frz_tokenizer* t, const uint32_t* ids, uint32_t n, char* pool,
                        uint64_t cap, uint64_t* pool_bytes, uint64_t* offsets) {
  if (!t || (!ids && n) || !pool_bytes || !offsets)
    return frz::fail(FRZ_ERR_ARGUMENT, "frz_tokenizer_texts: null argument");
  std::string all, bytes;
  frz::tok::Utf8Stream stream;
  offsets[0] = 0;
  for (uint32_t i = 0; i < n; ++i) {
    if (ids[i] >= t->t.size()) return frz::fail(FRZ_ERR_ARGUMENT, "frz_tokenizer_texts: id");
    bytes.clear();
    t->t.decode(ids[i], bytes);
    stream.push(bytes, all);
    if (i + 1 == n) (void)stream.finish(all);
    offsets[i + 1] = all.size();
  }
  *pool_bytes = all.size();
  if (pool) std::memcpy(pool, all.data(), std::min<uint64_t>(cap, all.size()));
  return FRZ_OK;
}

}  // extern "C"
