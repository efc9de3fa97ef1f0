// GGUF v3 index reader (contract in gguf.h). The order of checks follows
// the reference's reader (reader.h:64-107): header, metadata and its
// duplicate keys, alignment, tensor infos and their duplicate names, then
// the placement of every tensor's data, so that each malformed file is
// refused with the same named error.

#include "gguf.h"

#include <algorithm>
#include <cstring>
#include <string_view>

namespace frz::gguf {
namespace {

constexpr Layout kLayouts[] = {
    {0, "F32", 1, 4},        {1, "F16", 1, 2},        {2, "Q4_0", 32, 18},
    {3, "Q4_1", 32, 20},     {6, "Q5_0", 32, 22},     {7, "Q5_1", 32, 24},
    {8, "Q8_0", 32, 34},     {9, "Q8_1", 32, 36},     {10, "Q2_K", 256, 84},
    {11, "Q3_K", 256, 110},  {12, "Q4_K", 256, 144},  {13, "Q5_K", 256, 176},
    {14, "Q6_K", 256, 210},  {15, "Q8_K", 256, 292},  {16, "IQ2_XXS", 256, 66},
    {17, "IQ2_XS", 256, 74}, {18, "IQ3_XXS", 256, 98}, {19, "IQ1_S", 256, 50},
    {20, "IQ4_NL", 32, 18},  {21, "IQ3_S", 256, 110}, {22, "IQ2_S", 256, 82},
    {23, "IQ4_XS", 256, 136}, {24, "I8", 1, 1},       {25, "I16", 1, 2},
    {26, "I32", 1, 4},       {27, "I64", 1, 8},       {28, "F64", 1, 8},
    {29, "IQ1_M", 256, 56},  {30, "BF16", 1, 2},      {34, "TQ1_0", 256, 54},
    {35, "TQ2_0", 256, 66},  {39, "MXFP4", 32, 17},   {40, "NVFP4", 64, 36},
    {41, "Q1_0", 128, 18},   {42, "Q2_0", 64, 18},
};

constexpr const char* kErrorText[kErrorCount] = {
    "ok",
    "more of the file is needed to read its index",
    "the file ends before this field",
    "not a GGUF file (magic)",
    "unsupported GGUF version",
    "a declared count exceeds the reader's bound",
    "a string is longer than the reader's bound",
    "an array is longer than the reader's bound",
    "unknown metadata value type",
    "tensor format not defined by GGUF",
    "a tensor row is not a whole number of its format's blocks",
    "a tensor has more than 4 dimensions",
    "a tensor dimension is negative",
    "a tensor's element count overflows",
    "an offset or length overflows",
    "tensor data lies outside the file",
    "two tensors share a name",
    "a tensor name is longer than 64 bytes",
    "tensor data is not at a multiple of the alignment",
    "two tensors claim the same bytes",
    "general.alignment is not a power-of-two uint32",
    "a metadata key is empty",
    "two metadata entries share a key",
    "arrays of arrays are not supported",
};

uint64_t scalar_bytes(uint32_t t) {
  switch (t) {
    case kU8: case kI8: case kBool: return 1;
    case kU16: case kI16: return 2;
    case kU32: case kI32: case kF32: return 4;
    case kU64: case kI64: case kF64: return 8;
    default: return 0;
  }
}

bool add_ok(uint64_t a, uint64_t b, uint64_t* sum) { return !__builtin_add_overflow(a, b, sum); }
bool mul_ok(uint64_t a, uint64_t b, uint64_t* prod) { return !__builtin_mul_overflow(a, b, prod); }

// A cursor over the file's front. take() needs its bytes resident; skip()
// only needs them inside the file.
class Cursor {
 public:
  Cursor(const uint8_t* front, uint64_t resident, uint64_t size)
      : front_(front), resident_(std::min(resident, size)), size_(size) {}

  uint64_t at() const { return at_; }
  uint64_t needed() const { return needed_; }

  int take(void* out, uint64_t n) {
    if (n > size_ - at_) return kShortRead;
    if (at_ + n > resident_) {
      needed_ = at_ + n;
      return kNeedMoreBytes;
    }
    std::memcpy(out, front_ + at_, n);
    at_ += n;
    return kOk;
  }
  int skip(uint64_t n) {
    if (n > size_ - at_) return kShortRead;
    at_ += n;
    return kOk;
  }
  // Little-endian unsigned of `n` bytes.
  int uint(uint64_t n, uint64_t& v) {
    uint8_t b[8] = {};
    if (int e = take(b, n)) return e;
    v = 0;
    for (uint64_t k = n; k-- > 0;) v = (v << 8) | b[k];
    return kOk;
  }
  int u32(uint32_t& v) {
    uint64_t w;
    if (int e = uint(4, w)) return e;
    v = (uint32_t)w;
    return kOk;
  }
  int u64(uint64_t& v) { return uint(8, v); }
  // A string: kStringTooLong past kMaxString, then `too_long` past `limit`,
  // both before its bytes are read.
  int string(std::string& s, uint64_t limit = kMaxString, int too_long = kStringTooLong) {
    uint64_t n;
    if (int e = u64(n)) return e;
    if (n > kMaxString) return kStringTooLong;
    if (n > limit) return too_long;
    s.resize(n);
    return n ? take(s.data(), n) : kOk;
  }
  int skip_string() {
    uint64_t n;
    if (int e = u64(n)) return e;
    if (n > kMaxString) return kStringTooLong;
    return skip(n);
  }

 private:
  const uint8_t* front_;
  uint64_t resident_, size_;
  uint64_t at_ = 0, needed_ = 0;
};

int read_value(Cursor& c, Meta& m) {
  if (m.type == kString) return c.string(m.s);
  if (m.type == kArray) {
    if (int e = c.u32(m.array_type)) return e;
    if (m.array_type > kF64) return kUnknownValueType;
    if (m.array_type == kArray) return kNestedArray;
    if (int e = c.u64(m.array_count)) return e;
    if (m.array_count > kMaxArray) return kArrayTooLong;
    m.array_offset = c.at();
    if (m.array_type == kString) {
      for (uint64_t k = 0; k < m.array_count; ++k) {
        if (int e = c.skip_string()) return e;
      }
      return kOk;
    }
    uint64_t n;
    if (!mul_ok(m.array_count, scalar_bytes(m.array_type), &n)) return kOffsetOverflow;
    return c.skip(n);
  }
  uint64_t raw;
  if (int e = c.uint(scalar_bytes(m.type), raw)) return e;
  switch (m.type) {
    case kI8: m.i = (int8_t)raw; break;
    case kI16: m.i = (int16_t)raw; break;
    case kI32: m.i = (int32_t)raw; break;
    case kI64: m.i = (int64_t)raw; break;
    case kF32: {
      float f;
      const uint32_t r32 = (uint32_t)raw;
      std::memcpy(&f, &r32, 4);
      m.f = f;
      break;
    }
    case kF64: std::memcpy(&m.f, &raw, 8); break;
    case kBool: m.u = raw != 0; break;
    default: m.u = raw; break;
  }
  return kOk;
}

template <typename T, typename Key>
bool has_duplicate(const std::vector<T>& items, Key key) {
  std::vector<std::string_view> keys;
  keys.reserve(items.size());
  for (const T& t : items) keys.push_back(key(t));
  std::sort(keys.begin(), keys.end());
  return std::adjacent_find(keys.begin(), keys.end()) != keys.end();
}

int read_tensor(Cursor& c, Tensor& t) {
  if (int e = c.string(t.name, kMaxName, kTensorNameTooLong)) return e;
  if (int e = c.u32(t.dims)) return e;
  if (t.dims > kMaxDims) return kTooManyDimensions;
  t.elements = 1;
  for (uint32_t d = 0; d < t.dims; ++d) {
    uint64_t raw;
    if (int e = c.u64(raw)) return e;
    if ((int64_t)raw < 0) return kNegativeDimension;
    t.shape[d] = raw;
    if (!mul_ok(t.elements, raw, &t.elements)) return kElementCountOverflow;
  }
  if (int e = c.u32(t.type)) return e;
  const Layout* l = layout_of(t.type);
  if (!l) return kUnknownTensorType;
  if (t.shape[0] % l->elements != 0) return kRowNotWholeBlocks;
  if (int e = c.u64(t.offset)) return e;
  if (!mul_ok(t.elements / l->elements, l->bytes, &t.bytes)) return kOffsetOverflow;
  return kOk;
}

}  // namespace

const char* error_text(int e) {
  return e >= 0 && e < kErrorCount ? kErrorText[e] : "unrecognised error";
}

const Layout* layout_of(uint32_t type) {
  for (const Layout& l : kLayouts) {
    if (l.type == type) return &l;
  }
  return nullptr;
}

const Tensor* Index::tensor(const std::string& name) const {
  auto it = tensor_at.find(name);
  return it == tensor_at.end() ? nullptr : &tensors[it->second];
}

const Meta* Index::meta(const std::string& key) const {
  auto it = meta_at.find(key);
  return it == meta_at.end() ? nullptr : &metadata[it->second];
}

int read_index(const uint8_t* front, uint64_t resident, uint64_t size, Index& out,
               uint64_t* needed) {
  Cursor c(front, resident, size);
  Index ix;
  auto fail = [&](int e) {
    if (e == kNeedMoreBytes && needed) *needed = c.needed();
    return e;
  };
  // 1. header
  char magic[4];
  if (int e = c.take(magic, 4)) return fail(e);
  if (std::memcmp(magic, "GGUF", 4) != 0) return kBadMagic;
  uint32_t version;
  if (int e = c.u32(version)) return fail(e);
  if (version != 3) return kUnsupportedVersion;
  uint64_t n_tensors, n_meta;
  if (int e = c.u64(n_tensors)) return fail(e);
  if (int e = c.u64(n_meta)) return fail(e);
  if (n_tensors > kMaxTensors || n_meta > kMaxMetadata) return kCountTooLarge;
  // 2. metadata (entries grow as they are read: a count is only a claim)
  for (uint64_t k = 0; k < n_meta; ++k) {
    Meta m;
    if (int e = c.string(m.key)) return fail(e);
    if (m.key.empty()) return kEmptyKey;
    if (int e = c.u32(m.type)) return fail(e);
    if (m.type > kF64) return kUnknownValueType;
    if (int e = read_value(c, m)) return fail(e);
    ix.metadata.push_back(std::move(m));
  }
  if (has_duplicate(ix.metadata, [](const Meta& m) { return std::string_view(m.key); }))
    return kDuplicateMetadataKey;
  // 3. alignment
  for (const Meta& m : ix.metadata) {
    if (m.key != "general.alignment") continue;
    if (m.type != kU32 || m.u == 0 || (m.u & (m.u - 1)) != 0) return kBadAlignment;
    ix.alignment = m.u;
  }
  // 4. tensor infos
  for (uint64_t k = 0; k < n_tensors; ++k) {
    Tensor t;
    if (int e = read_tensor(c, t)) return fail(e);
    ix.tensors.push_back(std::move(t));
  }
  if (has_duplicate(ix.tensors, [](const Tensor& t) { return std::string_view(t.name); }))
    return kDuplicateTensorName;
  // 5. data placement
  uint64_t start;
  if (!add_ok(c.at(), ix.alignment - 1, &start)) return kOffsetOverflow;
  start -= start % ix.alignment;
  if (start > size) return kTensorDataOutOfBounds;
  ix.data_start = start;
  for (Tensor& t : ix.tensors) {
    if (t.offset % ix.alignment != 0) return kMisalignedTensorData;
    uint64_t abs, end;
    if (!add_ok(start, t.offset, &abs) || !add_ok(abs, t.bytes, &end)) return kOffsetOverflow;
    if (end > size) return kTensorDataOutOfBounds;
    t.offset = abs;
  }
  std::vector<std::pair<uint64_t, uint64_t>> ranges;
  ranges.reserve(ix.tensors.size());
  for (const Tensor& t : ix.tensors) ranges.emplace_back(t.offset, t.bytes);
  std::sort(ranges.begin(), ranges.end());
  for (size_t k = 1; k < ranges.size(); ++k) {
    if (ranges[k].first < ranges[k - 1].first + ranges[k - 1].second)
      return kOverlappingTensorData;
  }
  // 6. lookups, then the whole index replaces `out`
  for (size_t k = 0; k < ix.tensors.size(); ++k) ix.tensor_at[ix.tensors[k].name] = k;
  for (size_t k = 0; k < ix.metadata.size(); ++k) ix.meta_at[ix.metadata[k].key] = k;
  out = std::move(ix);
  return kOk;
}

File::~File() {
  if (f) std::fclose(f);
}

bool File::open(const char* path) {
  f = std::fopen(path, "rb");
  if (!f || fseeko(f, 0, SEEK_END) != 0) return false;
  const off_t end = ftello(f);
  if (end < 0) return false;
  size = (uint64_t)end;
  return true;
}

bool File::read(uint64_t offset, void* out, uint64_t bytes) {
  return fseeko(f, (off_t)offset, SEEK_SET) == 0 && std::fread(out, 1, bytes, f) == bytes;
}

int read_file(File& file, Index& out) {
  std::vector<uint8_t> front;
  uint64_t resident = 0;
  uint64_t want = std::min<uint64_t>(file.size, 16ull << 20);
  for (;;) {
    if (want > resident) {
      front.resize(want);
      if (!file.read(resident, front.data() + resident, want - resident)) return -1;
      resident = want;
    }
    uint64_t needed = 0;
    const int e = read_index(front.data(), resident, file.size, out, &needed);
    if (e != kNeedMoreBytes) return e;
    want = std::min<uint64_t>(file.size, std::max<uint64_t>(needed, 2 * resident));
  }
}

}  // namespace frz::gguf
