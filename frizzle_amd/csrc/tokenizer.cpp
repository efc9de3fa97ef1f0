// Gemma 3's SentencePiece BPE tokenizer: loading, encoding, decoding and the
// UTF-8 stream (src/core/tokenizer/bpe/sentencepiece_bpe.h:21-92,
// special.h:10-57, unicode.h:11-36, utf8_stream.cpp:5-35). Host code only.

#include "tokenizer.h"

#include <algorithm>
#include <cstring>
#include <queue>

#include "gguf.h"

namespace frz::tok {
namespace {

const std::string kSpace = "\xE2\x96\x81";  // U+2581, as the vocabulary spells a space
const std::string kReplacement = "\xEF\xBF\xBD";  // U+FFFD

// The second byte's range for a lead byte (the Unicode Standard's Table 3-7,
// well-formed byte sequences), and the character's length; length 0 for a
// byte that begins none.
struct Lead {
  uint8_t length, lo, hi;
};

Lead lead_of(uint8_t b) {
  if (b < 0x80) return {1, 0, 0};
  if (b >= 0xC2 && b <= 0xDF) return {2, 0x80, 0xBF};
  if (b == 0xE0) return {3, 0xA0, 0xBF};
  if ((b >= 0xE1 && b <= 0xEC) || b == 0xEE || b == 0xEF) return {3, 0x80, 0xBF};
  if (b == 0xED) return {3, 0x80, 0x9F};
  if (b == 0xF0) return {4, 0x90, 0xBF};
  if (b >= 0xF1 && b <= 0xF3) return {4, 0x80, 0xBF};
  if (b == 0xF4) return {4, 0x80, 0x8F};
  return {0, 0, 0};
}

// Whether byte b may stand at place k (1-based after the lead) of a
// character led by `lead`.
bool continues(const Lead& lead, size_t k, uint8_t b) {
  return k == 1 ? (b >= lead.lo && b <= lead.hi) : (b >= 0x80 && b <= 0xBF);
}

// Each space of `raw` as U+2581: the one normalization (step 2).
std::string escape_spaces(std::string_view raw) {
  std::string out;
  out.reserve(raw.size() + raw.size() / 2);
  for (char ch : raw) {
    if (ch == ' ') {
      out += kSpace;
    } else {
      out.push_back(ch);
    }
  }
  return out;
}

// Reads an array of metadata `key` from the file: strings, or 4-byte values.
bool read_strings(gguf::File& file, const gguf::Meta& m, std::vector<std::string>& out) {
  out.clear();
  out.reserve(m.array_count);
  uint64_t at = m.array_offset;
  for (uint64_t i = 0; i < m.array_count; ++i) {
    uint64_t n = 0;
    if (!file.read(at, &n, 8) || n > (1u << 20)) return false;
    std::string s(n, '\0');
    if (n && !file.read(at + 8, s.data(), n)) return false;
    out.push_back(std::move(s));
    at += 8 + n;
  }
  return true;
}

template <typename T>
bool read_words(gguf::File& file, const gguf::Meta& m, std::vector<T>& out) {
  out.resize(m.array_count);
  return m.array_count == 0 || file.read(m.array_offset, out.data(), m.array_count * 4);
}

}  // namespace

size_t utf8_length(std::string_view s, size_t at) {
  const Lead lead = lead_of((uint8_t)s[at]);
  if (lead.length == 0 || at + lead.length > s.size()) return 0;
  for (size_t k = 1; k < lead.length; ++k) {
    if (!continues(lead, k, (uint8_t)s[at + k])) return 0;
  }
  return lead.length;
}

// ---- special tokens (special.h) ----------------------------------------------

void SpecialTrie::build(const std::vector<std::pair<std::string, uint32_t>>& entries) {
  nodes_.assign(1, Node{});
  longest_ = 0;
  for (const auto& [text, id] : entries) {
    uint32_t node = 0;
    for (char ch : text) {
      const uint8_t b = (uint8_t)ch;
      auto& edges = nodes_[node].edges;
      auto it = std::lower_bound(edges.begin(), edges.end(), std::make_pair(b, 0u),
                                 [](const auto& x, const auto& y) { return x.first < y.first; });
      if (it != edges.end() && it->first == b) {
        node = it->second;
      } else {
        const uint32_t child = (uint32_t)nodes_.size();
        edges.insert(it, {b, child});
        nodes_.push_back(Node{});
        node = child;
      }
    }
    nodes_[node].token = id;
    longest_ = std::max(longest_, text.size());
  }
}

size_t SpecialTrie::match(std::string_view text, size_t at, uint32_t* id) const {
  size_t best = 0;
  uint32_t node = 0;
  for (size_t i = at; i < text.size(); ++i) {
    const uint8_t b = (uint8_t)text[i];
    const auto& edges = nodes_[node].edges;
    auto it = std::lower_bound(edges.begin(), edges.end(), std::make_pair(b, 0u),
                               [](const auto& x, const auto& y) { return x.first < y.first; });
    if (it == edges.end() || it->first != b) break;
    node = it->second;
    if (nodes_[node].token >= 0) {
      best = i + 1 - at;
      *id = (uint32_t)nodes_[node].token;
    }
  }
  return best;
}

// ---- load (sentencepiece_bpe.h:28-52) ------------------------------------------

bool Tokenizer::load(const char* path, std::string* error) {
  auto refuse = [error](const std::string& why) {
    if (error) *error = why;
    return false;
  };
  gguf::File file;
  if (!file.open(path)) return refuse(std::string("cannot open ") + path);
  gguf::Index index;
  if (int e = gguf::read_file(file, index)) {
    return refuse(e < 0 ? "cannot read the file" : gguf::error_text(e));
  }
  const gguf::Meta* model = index.meta("tokenizer.ggml.model");
  if (!model || model->type != gguf::kString) return refuse("tokenizer.ggml.model: missing");
  if (model->s != "llama") {
    return refuse("tokenizer.ggml.model: \"" + model->s + "\" is not SentencePiece BPE");
  }
  // A space prefix must be declared, and false: where one would go, the file
  // does not say.
  const gguf::Meta* prefix = index.meta("tokenizer.ggml.add_space_prefix");
  if (!prefix) return refuse("tokenizer.ggml.add_space_prefix: not declared");
  if (prefix->type != gguf::kBool) return refuse("tokenizer.ggml.add_space_prefix: not a bool");
  if (prefix->u != 0) return refuse("tokenizer.ggml.add_space_prefix: true is not supported");
  const gguf::Meta* tokens = index.meta("tokenizer.ggml.tokens");
  const gguf::Meta* scores = index.meta("tokenizer.ggml.scores");
  const gguf::Meta* types = index.meta("tokenizer.ggml.token_type");
  if (!tokens || tokens->type != gguf::kArray || tokens->array_type != gguf::kString)
    return refuse("tokenizer.ggml.tokens: missing or not an array of strings");
  if (!scores || scores->type != gguf::kArray || scores->array_type != gguf::kF32)
    return refuse("tokenizer.ggml.scores: missing or not an array of f32");
  if (!types || types->type != gguf::kArray || types->array_type != gguf::kI32)
    return refuse("tokenizer.ggml.token_type: missing or not an array of i32");
  if (tokens->array_count == 0 || tokens->array_count >= (1ull << 31))
    return refuse("tokenizer.ggml.tokens: count");
  if (scores->array_count != tokens->array_count || types->array_count != tokens->array_count)
    return refuse("tokenizer.ggml.scores / token_type: counts differ from the tokens'");
  std::vector<std::string> text;
  std::vector<float> score;
  std::vector<int32_t> type;
  if (!read_strings(file, *tokens, text) || !read_words(file, *scores, score) ||
      !read_words(file, *types, type)) {
    return refuse("cannot read the vocabulary");
  }
  std::unordered_map<std::string, uint32_t> normal;
  std::vector<std::pair<std::string, uint32_t>> specials;
  uint32_t bytes[256];
  bool have_byte[256] = {};
  size_t cover = 0;
  for (uint32_t id = 0; id < (uint32_t)text.size(); ++id) {
    const std::string& t = text[id];
    const int32_t ty = type[id];
    if (ty < kNormal || ty > kByte) return refuse("token " + std::to_string(id) + ": type");
    cover = std::max(cover, t.size());
    if (ty == kNormal) {
      normal.emplace(t, id);
    } else if (ty == kByte) {
      // "<0xXX>": the byte it stands for.
      unsigned v = 0;
      if (t.size() != 6 || t.compare(0, 3, "<0x") != 0 || t[5] != '>' ||
          std::sscanf(t.c_str() + 3, "%2x", &v) != 1) {
        return refuse("token " + std::to_string(id) + ": a byte token other than <0x00>..<0xFF>");
      }
      bytes[v] = id;
      have_byte[v] = true;
    } else if ((ty == kControl || ty == kUserDefined) && !t.empty()) {
      specials.push_back({escape_spaces(t), id});
    }
    // A one-character token must be one the encode can produce.
    if (!t.empty() && utf8_length(t, 0) == t.size() && ty != kNormal && ty != kControl &&
        ty != kUserDefined && ty != kByte) {
      return refuse("token " + std::to_string(id) + ": a one-character token of type " +
                    std::to_string(ty));
    }
  }
  for (int b = 0; b < 256; ++b) {
    if (!have_byte[b]) return refuse("no byte token for <0x" + std::to_string(b) + ">");
  }
  std::sort(specials.begin(), specials.end());
  for (size_t i = 1; i < specials.size(); ++i) {
    if (specials[i].first == specials[i - 1].first)
      return refuse("two special tokens spelled \"" + specials[i].first + "\"");
  }
  text_ = std::move(text);
  score_ = std::move(score);
  type_ = std::move(type);
  normal_ = std::move(normal);
  std::memcpy(byte_token_, bytes, sizeof bytes);
  special_.build(specials);
  cover_ = cover;
  return true;
}

// ---- encode (sentencepiece_bpe.h:64-82, tokenizer.h:41-66) ----------------------

// One run of ordinary text: its characters as normal tokens or bytes, then
// merged, the highest-scoring token first, the leftmost on a tie.
bool Tokenizer::merge_run(std::string_view run, std::vector<uint32_t>& out) const {
  struct Symbol {
    uint32_t start, length, id;
    bool normal;
    int prev, next;
  };
  std::vector<Symbol> sym;
  for (size_t at = 0; at < run.size();) {
    const size_t n = utf8_length(run, at);
    if (n == 0) return false;
    auto it = normal_.find(std::string(run.substr(at, n)));
    if (it != normal_.end()) {
      sym.push_back({(uint32_t)at, (uint32_t)n, it->second, true, 0, 0});
    } else {
      for (size_t k = 0; k < n; ++k)
        sym.push_back({(uint32_t)(at + k), 1, byte_token_[(uint8_t)run[at + k]], false, 0, 0});
    }
    at += n;
  }
  const int count = (int)sym.size();
  for (int i = 0; i < count; ++i) {
    sym[i].prev = i - 1;
    sym[i].next = i + 1 < count ? i + 1 : -1;
  }
  struct Candidate {
    float score;
    uint32_t start;  // the left symbol's first byte: leftmost wins a tie
    int left, right;
    uint32_t length;  // the joined text's, to tell a stale candidate
    uint32_t id;
  };
  auto worse = [](const Candidate& a, const Candidate& b) {
    return a.score != b.score ? a.score < b.score : a.start > b.start;
  };
  std::priority_queue<Candidate, std::vector<Candidate>, decltype(worse)> heap(worse);
  std::string joined;
  auto offer = [&](int l, int r) {
    if (l < 0 || r < 0 || !sym[l].normal || !sym[r].normal) return;
    joined.assign(run.substr(sym[l].start, sym[l].length + sym[r].length));
    auto it = normal_.find(joined);
    if (it == normal_.end()) return;
    heap.push({score_[it->second], sym[l].start, l, r, sym[l].length + sym[r].length,
               it->second});
  };
  for (int i = 0; i + 1 < count; ++i) offer(i, i + 1);
  while (!heap.empty()) {
    const Candidate c = heap.top();
    heap.pop();
    Symbol& l = sym[c.left];
    if (l.length == 0 || l.next != c.right || l.length + sym[c.right].length != c.length)
      continue;  // one side merged since
    Symbol& r = sym[c.right];
    l.length += r.length;
    l.id = c.id;
    r.length = 0;
    l.next = r.next;
    if (r.next >= 0) sym[r.next].prev = c.left;
    offer(l.prev, c.left);
    offer(c.left, l.next);
  }
  for (int i = 0; i >= 0 && i < count; i = sym[i].next) out.push_back(sym[i].id);
  return true;
}

EncodeResult Tokenizer::encode(std::string_view raw, uint32_t max_tokens,
                               std::vector<uint32_t>& out) const {
  EncodeResult res;
  res.raw_bytes = raw.size();
  // 1. Raw text past what any admitted text could be is refused unread.
  const uint64_t raw_cap =
      kMaxEncodeBytes * 7 / 2 +
      (max_tokens == kNoTokenLimit ? 0 : (uint64_t)max_tokens * special_.longest());
  if (max_tokens != kNoTokenLimit && raw.size() > raw_cap) {
    res.error = kTooLong;
    return res;
  }
  // 2. Spaces as U+2581; 3. the special tokens split out.
  const std::string text = escape_spaces(raw);
  struct Segment {
    size_t start, length;
    int64_t token;  // a special token's id, -1 for ordinary text
  };
  std::vector<Segment> segs;
  uint64_t specials = 0;
  size_t run = 0;
  for (size_t at = 0; at < text.size();) {
    uint32_t id = 0;
    const size_t n = special_.match(text, at, &id);
    if (n == 0) {
      ++at;
      continue;
    }
    if (at > run) segs.push_back({run, at - run, -1});
    segs.push_back({at, n, (int64_t)id});
    if (++specials > max_tokens) {
      res.error = kTooManyTokens;
      res.least_tokens = specials;
      return res;
    }
    at += n;
    run = at;
  }
  if (text.size() > run) segs.push_back({run, text.size() - run, -1});
  // 4. The least tokens the text makes, then its normalized bytes.
  uint64_t least = 0, normalized = 0;
  for (const Segment& s : segs) {
    if (s.token >= 0) {
      least += 1;
    } else {
      least += (s.length + cover_ - 1) / cover_;
      normalized += s.length;
    }
  }
  res.least_tokens = least;
  res.normalized_bytes = normalized;
  if (max_tokens != kNoTokenLimit && least > max_tokens) {
    res.error = kTooManyTokens;
    return res;
  }
  if (normalized > kMaxEncodeBytes) {
    res.error = kTooLong;
    return res;
  }
  // 5. Each run merged; 6. all appended together.
  std::vector<uint32_t> ids;
  for (const Segment& s : segs) {
    if (s.token >= 0) {
      ids.push_back((uint32_t)s.token);
    } else if (!merge_run(std::string_view(text).substr(s.start, s.length), ids)) {
      res.error = kInvalidUtf8;
      return res;
    }
  }
  out.insert(out.end(), ids.begin(), ids.end());
  return res;
}

// ---- decode --------------------------------------------------------------------

void Tokenizer::decode(uint32_t id, std::string& out) const {
  const std::string& t = text_[id];
  if (type_[id] == kByte) {
    unsigned v = 0;
    std::sscanf(t.c_str() + 3, "%2x", &v);
    out.push_back((char)v);
    return;
  }
  if (type_[id] != kNormal) {
    out += t;
    return;
  }
  for (size_t at = 0; at < t.size();) {
    if (t.compare(at, kSpace.size(), kSpace) == 0) {
      out.push_back(' ');
      at += kSpace.size();
    } else {
      out.push_back(t[at++]);
    }
  }
}

// ---- the UTF-8 stream (utf8_stream.cpp:5-35) -------------------------------------

void Utf8Stream::push(std::string_view bytes, std::string& out) {
  for (char ch : bytes) {
    const uint8_t b = (uint8_t)ch;
    if (!pending_.empty()) {
      const Lead lead = lead_of((uint8_t)pending_[0]);
      if (continues(lead, pending_.size(), b)) {
        pending_.push_back(ch);
        if (pending_.size() == lead.length) {
          out += pending_;
          pending_.clear();
        }
        continue;
      }
      // A character begun well but broken off: one U+FFFD; b read afresh.
      out += kReplacement;
      pending_.clear();
    }
    const Lead lead = lead_of(b);
    if (lead.length == 1) {
      out.push_back(ch);
    } else if (lead.length >= 2) {
      pending_.push_back(ch);
    } else {
      out += kReplacement;
    }
  }
}

bool Utf8Stream::finish(std::string& out) {
  if (pending_.empty()) return true;
  out += kReplacement;
  pending_.clear();
  return false;
}

}  // namespace frz::tok
