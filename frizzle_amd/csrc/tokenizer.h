// Gemma 3's tokenizer, SentencePiece BPE as GGUF names it "llama"
// (src/core/tokenizer/tokenizer.h, bpe/sentencepiece_bpe.h): text to token
// identifiers and identifiers back to bytes, loaded from a GGUF file's
// tokenizer.ggml.* entries. Host code only.
//
// Encode (sentencepiece_bpe.h:64-92): each space becomes U+2581; the control
// and user-defined tokens, spelled the same way, are split out of the text
// by the longest match from the left (special.h); in each ordinary run each
// character becomes its normal token, or one byte token a byte where it has
// none; then any two adjacent normal symbols whose joined text is a normal
// token merge, the token of highest score first and the leftmost on a tie,
// until none can. No space is added before the text, and BOS is never
// added: the chat template writes it as text.
//
// Decode: a normal token's text with each U+2581 a space, a byte token's
// byte, any other token's text as written.
#pragma once

#include <cstdint>
#include <string>
#include <string_view>
#include <unordered_map>
#include <vector>

namespace frz::tok {

// Token types, as tokenizer.ggml.token_type numbers them.
enum Type : int32_t {
  kNormal = 1,
  kUnknown = 2,
  kControl = 3,
  kUserDefined = 4,
  kUnused = 5,
  kByte = 6,
};

// The encode's refusals (tokenizer.h:186-191).
enum EncodeError : int {
  kEncodeOk = 0,
  kInvalidUtf8 = 1,
  kTooManyTokens = 2,  // more tokens, at least, than the caller's limit
  kTooLong = 3,        // past kMaxEncodeBytes of normalized text
};

// The most normalized bytes one encode takes (tokenizer.h:180).
constexpr uint64_t kMaxEncodeBytes = 512ull * 1024;
constexpr uint32_t kNoTokenLimit = UINT32_MAX;

struct EncodeResult {
  int error = kEncodeOk;
  uint64_t least_tokens = 0;
  uint64_t normalized_bytes = 0;
  uint64_t raw_bytes = 0;
};

// Longest-match search over the special tokens' texts: a byte trie, each
// node's edges sorted by byte.
class SpecialTrie {
 public:
  void build(const std::vector<std::pair<std::string, uint32_t>>& entries);
  // The longest special token starting at text[at]: its length in bytes (0
  // for none) and identifier.
  size_t match(std::string_view text, size_t at, uint32_t* id) const;
  size_t longest() const { return longest_; }

 private:
  struct Node {
    std::vector<std::pair<uint8_t, uint32_t>> edges;  // byte, child
    int64_t token = -1;
  };
  std::vector<Node> nodes_;
  size_t longest_ = 0;
};

class Tokenizer {
 public:
  // Loads from a GGUF file; on failure returns false with `error` naming the
  // refusal.
  bool load(const char* path, std::string* error);

  uint32_t size() const { return (uint32_t)text_.size(); }
  size_t longest_cover() const { return cover_; }
  const std::string& text(uint32_t id) const { return text_[id]; }
  int32_t type(uint32_t id) const { return type_[id]; }
  float score(uint32_t id) const { return score_[id]; }

  // Appends the tokens `raw` makes, or refuses with `out` untouched.
  EncodeResult encode(std::string_view raw, uint32_t max_tokens,
                      std::vector<uint32_t>& out) const;
  // Appends the bytes `id` stands for. Precondition: id < size().
  void decode(uint32_t id, std::string& out) const;

 private:
  bool merge_run(std::string_view run, std::vector<uint32_t>& out) const;

  std::vector<std::string> text_;
  std::vector<float> score_;
  std::vector<int32_t> type_;
  std::unordered_map<std::string, uint32_t> normal_;  // normal tokens by text
  uint32_t byte_token_[256] = {};
  SpecialTrie special_;
  size_t cover_ = 0;
};

// Text from bytes a piece at a time, passing only whole UTF-8 characters
// (utf8_stream.cpp): a character's first bytes are held until it completes;
// a byte that cannot begin or continue a character becomes U+FFFD.
class Utf8Stream {
 public:
  void push(std::string_view bytes, std::string& out);
  // Ends the text: U+FFFD where bytes were pending. True when none were.
  bool finish(std::string& out);

 private:
  std::string pending_;
};

// One well-formed UTF-8 character at s[at]: its length (1-4), or 0 when the
// bytes there are not one.
size_t utf8_length(std::string_view s, size_t at);

}  // namespace frz::tok
