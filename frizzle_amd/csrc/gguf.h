// GGUF v3 index reader: the header, metadata and tensor infos of an
// untrusted file, every claim checked before use (reader.h:12-107 states the
// same contract for the reference's reader). Host code only.
//
// The source is the front of the file: `resident` bytes held, of a file of
// `size` bytes. A field that lies inside the file but past the resident front
// gives kNeedMoreBytes with `needed`, the length of front the read needed; a
// field past the end of the file gives kShortRead. Tensor data is never read:
// each tensor's range is only checked against the file's size.
//
// Format facts kept as GGUF defines them (the same numbers any reader uses):
// magic "GGUF", version 3, little-endian fields, value types 0..12, tensor
// formats by ggml number with their block sizes, data aligned to 32 bytes
// unless general.alignment (a power-of-two uint32) says otherwise, at most 4
// dimensions, a tensor name at most 64 bytes.
#pragma once

#include <cstdint>
#include <cstdio>
#include <string>
#include <unordered_map>
#include <vector>

namespace frz::gguf {

// The ways reading can fail, in the order the reader checks them. The
// numbers are this library's (frizzle_hip.h, FRZ_GGUF_*).
enum Error : int {
  kOk = 0,
  kNeedMoreBytes,
  kShortRead,
  kBadMagic,
  kUnsupportedVersion,
  kCountTooLarge,
  kStringTooLong,
  kArrayTooLong,
  kUnknownValueType,
  kUnknownTensorType,
  kRowNotWholeBlocks,
  kTooManyDimensions,
  kNegativeDimension,
  kElementCountOverflow,
  kOffsetOverflow,
  kTensorDataOutOfBounds,
  kDuplicateTensorName,
  kTensorNameTooLong,
  kMisalignedTensorData,
  kOverlappingTensorData,
  kBadAlignment,
  kEmptyKey,
  kDuplicateMetadataKey,
  kNestedArray,
  kErrorCount,
};

const char* error_text(int e);

// Metadata value types, GGUF's numbering.
enum ValueType : uint32_t {
  kU8 = 0, kI8, kU16, kI16, kU32, kI32, kF32, kBool, kString, kArray, kU64, kI64, kF64,
};

// A tensor format's block: `elements` consecutive values of a row in
// `bytes` bytes (an unquantized format is a block of one value).
struct Layout {
  uint32_t type;
  const char* name;
  uint32_t elements;
  uint32_t bytes;
};
const Layout* layout_of(uint32_t type);

// This reader's own bounds: a hostile count cannot make it allocate much.
constexpr uint64_t kMaxTensors = 1ull << 20;
constexpr uint64_t kMaxMetadata = 1ull << 20;
constexpr uint64_t kMaxString = 1ull << 20;
constexpr uint64_t kMaxArray = 1ull << 24;
constexpr uint64_t kMaxName = 64;
constexpr uint32_t kMaxDims = 4;

struct Tensor {
  std::string name;
  uint32_t type = 0;
  uint32_t dims = 0;
  uint64_t shape[kMaxDims] = {1, 1, 1, 1};
  uint64_t elements = 0;
  uint64_t offset = 0;  // absolute, in the file
  uint64_t bytes = 0;
};

struct Meta {
  std::string key;
  uint32_t type = 0;
  uint64_t u = 0;     // unsigned integers and bool
  int64_t i = 0;      // signed integers
  double f = 0.0;     // floats
  std::string s;      // strings
  uint32_t array_type = 0;  // arrays: located, not read
  uint64_t array_count = 0;
  uint64_t array_offset = 0;
};

struct Index {
  std::vector<Tensor> tensors;
  std::vector<Meta> metadata;
  uint64_t alignment = 32;
  uint64_t data_start = 0;
  std::unordered_map<std::string, size_t> tensor_at, meta_at;

  const Tensor* tensor(const std::string& name) const;
  const Meta* meta(const std::string& key) const;
};

// Reads the index of a file of `size` bytes whose first `resident` bytes are
// at `front`. On kOk `out` is replaced; otherwise it is untouched.
// `needed` is set with kNeedMoreBytes.
int read_index(const uint8_t* front, uint64_t resident, uint64_t size, Index& out,
               uint64_t* needed);

// A file read by offset.
struct File {
  std::FILE* f = nullptr;
  uint64_t size = 0;
  File() = default;
  File(const File&) = delete;
  File& operator=(const File&) = delete;
  ~File();
  bool open(const char* path);
  bool read(uint64_t offset, void* out, uint64_t bytes);
};

// The index of a whole file, its front read as the reader asks for it (at
// least doubling a round). -1 when the file cannot be read, else read_index's
// result.
int read_file(File& file, Index& out);

}  // namespace frz::gguf

// The C ABI's index handle (frizzle_hip.h, frz_gguf).
struct frz_gguf {
  frz::gguf::Index index;
};
