// Host-side launchers of the forward path's HIP kernels, and the device
// structures they share. Every launcher enqueues on the given stream and
// returns the launch's hipError_t; none allocates or synchronizes.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace frz {

constexpr int kRanges = 32;        // a row's K-ranges (matmul.h:88-97)
constexpr int kSplitParts = kRanges / 2;  // range sums a split product leaves apart
constexpr int kSplitRows = 16;            // most rows a split product takes
constexpr int kChunkKeys = 64;     // attention chunk (attention.wgsl:60)
constexpr int kTileKeys = 8;       // attention tile at d = 256
constexpr int kCandidates = 64;    // top-k kept (residency/plan.h:195)
constexpr int kSelectionTile = 1024;
constexpr int kPrefillBlock = 512; // most tokens a step holds
constexpr int kMaxHeadDim = 256;

// The step's parameters, read by kernels from device memory, as the
// reference's Step uniform (kernels/interface.h:163-188, step.wgsl). A
// decode graph advances it on the device, so replays need no host write.
struct DevStep {
  uint32_t position;
  uint32_t tokens;
  uint32_t logits;
  uint32_t fed;
  uint32_t seed[2];
  uint32_t top_k;
  float temperature;
  float top_p;
  float min_p;
  float log_min_p;
  uint32_t drawn;     // draws recorded so far (index into the token log)
  // Nonzero: the rows are `tokens` sequences (variants) at one position,
  // row r with its own caches and edit table, fed from its own draw
  // (record r); zero: the rows are one sequence's positions position + r.
  uint32_t variants;
  uint32_t pad[3];
  uint32_t ids[kPrefillBlock];
};

// Block formats, by GGUF's numbers (the reference's formats/*: q4_0, q4_1,
// q8_0).
constexpr int kQ4_0 = 2;  // 32 weights: f16 d, 16 bytes of 4-bit codes
constexpr int kQ4_1 = 3;  // f16 d, f16 minimum m, 16 bytes of 4-bit codes
constexpr int kQ8_0 = 8;  // f16 d, 32 signed 8-bit codes
constexpr int code_bytes(int format) { return format == kQ8_0 ? 32 : 16; }
// Halves of scale a block has on the device: d (Q4_0, Q8_0) or d then m.
constexpr int scale_halves(int format) { return format == kQ4_1 ? 2 : 1; }
constexpr int gguf_block_bytes(int format) {
  return format == kQ8_0 ? 34 : format == kQ4_1 ? 20 : 18;
}

// A quantized matrix on the device: `rows` rows of `cols` weights as two
// streams, every block's code bytes in row-major block order, then every
// block's scale halves (the reference's device layout,
// device_layout.h:114-115).
//
// A fused product over members placed apart (a plan's Q, K, V group, each
// member in its own device layout at its own offset, residency/plan.h): rows
// from split[0] on are member 1's, rows from split[1] on member 2's, each
// counted from its member's first row; 0 ends the list. Splits are
// multiples of 32 rows (a prefill tile never straddles two members), and
// only Q4_0 products over K = 1,152 take members.
struct QMatrix {
  const uint8_t* codes;    // rows * cols / 32 blocks of code_bytes(format)
  const uint16_t* scales;  // rows * cols / 32 blocks of scale_halves(format)
  int rows;
  int cols;
  int format = kQ4_0;
  int split[2] = {0, 0};
  const uint8_t* member_codes[2] = {nullptr, nullptr};
  const uint16_t* member_scales[2] = {nullptr, nullptr};
};

// Row `row`'s member: its streams and the row within them.
struct MemberRow {
  const uint8_t* codes;
  const uint16_t* scales;
  int row;
};
__host__ __device__ inline MemberRow member_row(const QMatrix& w, int row) {
  if (w.split[1] != 0 && row >= w.split[1])
    return {w.member_codes[1], w.member_scales[1], row - w.split[1]};
  if (w.split[0] != 0 && row >= w.split[0])
    return {w.member_codes[0], w.member_scales[0], row - w.split[0]};
  return {w.codes, w.scales, row};
}
inline bool has_members(const QMatrix& w) { return w.split[0] != 0; }

// ---- products ----------------------------------------------------------
// y[t][o] = sum_k W[o][k] x[t][k] for t < step.tokens (or only the last
// token when last_token), in the reference's order. Decode form when the
// step holds one token; matrix-core form otherwise.
hipError_t launch_gemv(hipStream_t s, const DevStep* step, QMatrix w,
                       const float* x, int x_stride, float* y, int y_stride,
                       int max_tokens, bool last_token);
// A step of at most 16 rows over a long K may split each output's 32 ranges
// over two workgroups: y then holds the in-order prefix of ranges 0..15 and
// parts + j * parts_stride (y's row layout) range 16 + j's sum, for the
// consumer to add in order (NormArgs::parts). gemv_splits says whether
// launch_gemv_split takes that form; when it does not, it writes y whole.
bool gemv_splits(const QMatrix& w, int max_tokens);
hipError_t launch_gemv_split(hipStream_t s, const DevStep* step, QMatrix w, const float* x,
                             int x_stride, float* y, int y_stride, int max_tokens, float* parts,
                             size_t parts_stride);
// act[t][j] = gelu_tanh(gate_j) * up_j, then layer `layer`'s pins at the
// row's position (edit table in the reference's layout; null for none).
// A variants step gives row r the table at edits + r * edit_stride words;
// edit_stride is 0 for every other step.
hipError_t launch_gated(hipStream_t s, const DevStep* step, QMatrix gate,
                        QMatrix up, const float* x, float* act,
                        int max_tokens, const uint32_t* edits, int layer,
                        uint32_t edit_stride = 0);

// The input row of a decode product, made in the product's prologue.
// mode 0: x as given. mode 1: hidden + post-norm(output) (written to
// hidden_out by the first workgroup when not null), then RMSNorm with gain.
// mode 2: the step's token's embedding row times scale (written to
// hidden_out likewise), then RMSNorm with gain. mode 3: the attention
// output, folded from the decode attention's chunk states (partials, stats;
// at most kFoldPrologueChunks chunks at this window).
struct GemvInput {
  const float* x;
  const float* hidden;
  const float* output;
  const float* post_gain;
  const float* gain;
  float* hidden_out;
  QMatrix table;
  const uint32_t* sampled;
  float scale;
  float epsilon;
  const float* partials;
  const float* stats;
  int window;
  float* normed_out;  // modes 1 and 2: workgroup 0 also writes the normed row here
};
constexpr int kFoldPrologueChunks = 10;
hipError_t launch_gemv_decode(hipStream_t s, const DevStep* step, const QMatrix& w,
                              const GemvInput& in, int mode, float* y);
// The gated decode product (prologue mode 0 or 1): act = gelu(gate) * up,
// then layer `layer`'s pins.
hipError_t launch_gated_decode(hipStream_t s, const DevStep* step, const QMatrix& gate,
                               const QMatrix& up, const GemvInput& in, int mode, float* act,
                               const uint32_t* edits, int layer);

// ---- the fast prefill mode: products on the bf16 matrix cores ------------
// A product over bf16 pair operands (prefill_bf16.hip): each weight and each
// activation as hi + lo bf16, y within about 2^-16 of each product of the
// exact sum (not the reference's order of addition). The weights come as
// fragment planes made once by launch_unpack_planes, activations as the
// planes below, x_hi and x_lo, ldx wide. Gated (the planes of a gate and an up
// matrix): act = gelu(gate) * up, then layer `layer`'s pins, written as
// fp32 to y (when not null) and as pair planes to y_hi, y_lo. Otherwise
// y[t][ldy] fp32; with K split over `splits`, split z's partial sums at
// y + z * part_stride.
// Its activation planes (hi and lo, each a block of rows [t][width]) hold
// element (t, k) in the instruction's fragment order: for each 32-token
// block and each step of 16 k, 64 lanes x 8 values, lane 32 (k % 16 / 8) +
// t % 32, so that a wave loads a fragment as one contiguous 1 KB run.
// width is a multiple of 16; rows are allocated in whole 32-token blocks.
__host__ __device__ inline size_t plane_index(int t, int k, int width) {
  return ((((size_t)(t >> 5) * (width >> 4) + (k >> 4)) * 64 + ((k >> 3) & 1) * 32 + (t & 31))
          << 3) +
         (k & 7);
}
// Four values of row t from k (k % 4 == 0) as bf16 pairs, hi = bf16(v) and
// lo = bf16(v - hi), both rounded to nearest even.
__device__ inline void store_pairs4(uint16_t* hi, uint16_t* lo, int t, int k, int width,
                                    const float (&v)[4]) {
  uint32_t hw[2], lw[2];
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const __bf16 a = (__bf16)v[2 * e], b = (__bf16)v[2 * e + 1];
    const __bf16 c = (__bf16)(v[2 * e] - (float)a), d = (__bf16)(v[2 * e + 1] - (float)b);
    hw[e] = (uint32_t)__builtin_bit_cast(uint16_t, a) |
            ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
    lw[e] = (uint32_t)__builtin_bit_cast(uint16_t, c) |
            ((uint32_t)__builtin_bit_cast(uint16_t, d) << 16);
  }
  const size_t at = plane_index(t, k, width);
  *reinterpret_cast<uint2*>(hi + at) = make_uint2(hw[0], hw[1]);
  *reinterpret_cast<uint2*>(lo + at) = make_uint2(lw[0], lw[1]);
}
struct Bf16Gemm {
  const uint4* w = nullptr;  // fragment planes
  int rows = 0;              // output rows (neurons, gated)
  int cols = 0;              // K
  bool gated = false;
  const uint16_t* x_hi = nullptr;
  const uint16_t* x_lo = nullptr;
  int ldx = 0;
  float* y = nullptr;
  int ldy = 0;
  size_t part_stride = 0;
  uint16_t* y_hi = nullptr;
  uint16_t* y_lo = nullptr;
  const uint32_t* edits = nullptr;
  int layer = 0;
  int k_blocks = 0, token_tiles = 0, splits = 1;  // set by the launcher
};
constexpr int kMaxBf16Splits = 16;  // K splits a bf16 product may take
bool bf16_gemm_shape_ok(const QMatrix& w, int ldx, int ldy);
// Bytes of a matrix's fragment planes (gated: a gate and an up matrix of
// `rows` rows each).
size_t bf16_planes_bytes(int rows, int cols, bool gated);
// w's (with `up`, the gate w's and up's) weights as fragment planes at out.
hipError_t launch_unpack_planes(hipStream_t s, const QMatrix& w, const QMatrix* up, uint4* out);
// The K splits a product of this shape takes to fill the device.
int bf16_splits_for(int rows, int cols, int max_tokens, bool gated);
hipError_t launch_gemm_bf16(hipStream_t s, const DevStep* step, Bf16Gemm g, int max_tokens,
                            int splits);
// y[t][o] = the `count` splits' partial sums (stride floats apart) in order.
hipError_t launch_sum_parts(hipStream_t s, const DevStep* step, const float* parts,
                            size_t stride, int count, int width, int ld, float* y,
                            int max_tokens);
// Rows of fp32 values into bf16 pair planes (hi = bf16(x), lo = bf16(x - hi)),
// plane_index order, width wide.
hipError_t launch_split_rows(hipStream_t s, const DevStep* step, const float* x, int ldx,
                             int width, uint16_t* hi, uint16_t* lo, int max_tokens);

// The fast prefill mode's attention (attention_fast.hip): each (32-row
// block, 64-key chunk) of a step's rows as chunk states on the f16 matrix
// cores, in the layout attention_fold reads (partials, stats; a row's chunk
// index from its earliest key's chunk), within a stated tolerance of the
// reference's tile recursion.
struct FastAttentionArgs {
  const float* query;  // token t's roped heads at query + t * q_stride
  int q_stride;
  const uint16_t* key_cache;
  const uint16_t* value_cache;
  float* partials;
  float* stats;
  int slots;
  int window;
  int head_dim;
  int query_heads;
  int kv_heads;
  int max_chunks;
  float scale_log2e;
};
// Chunks the grid spans for a step whose rows sit at positions first..last.
int fast_attention_chunks(uint32_t first, uint32_t last, int window);
hipError_t launch_attention_fast(hipStream_t s, const DevStep* step, const FastAttentionArgs& a,
                                 int max_tokens, int grid_chunks);

// ---- per-row kernels ---------------------------------------------------
struct NormArgs {
  const float* gain;
  const float* post_gain;  // null: no add
  const float* output;     // the block's output y, added when post_gain
  float* hidden;
  float* normed;
  float epsilon;
  int width;
  bool last_token;         // only the step's last row
  // Not null: hidden after the add (the residual entering the layer) is also
  // written to capture + step.drawn * capture_step + row * width.
  float* capture = nullptr;
  size_t capture_step = 0;
  // Not null: the last row's hidden after the add, and what was added
  // (the block's output after its post-norm), written there too.
  float* store_x = nullptr;
  float* store_added = nullptr;
  // Not null: `output` holds a split product's prefix, to which the
  // part_count range sums (or K-split partial sums) at
  // parts + j * parts_stride (same row layout) are added in order.
  const float* parts = nullptr;
  size_t parts_stride = 0;
  int part_count = kSplitParts;
  // Not null: the normed row is also written as bf16 pair planes (the fast
  // prefill products' inputs, plane_index order).
  uint16_t* normed_hi = nullptr;
  uint16_t* normed_lo = nullptr;
};
hipError_t launch_norm(hipStream_t s, const DevStep* step, const NormArgs& a,
                       int max_tokens);

struct RopeArgs {
  const float* turns;       // head_dim / 2
  const float* query_gain;  // head_dim
  const float* key_gain;
  float* query;             // token t's heads at query + t * q_stride, in place
  const float* key;         // token t's at key + t * kv_stride
  const float* value;       // token t's at value + t * kv_stride
  int q_stride;
  int kv_stride;
  uint16_t* key_cache;      // [slots][kv_heads][head_dim] F16
  uint16_t* value_cache;
  int slots;
  int head_dim;
  int query_heads;
  int kv_heads;
  float epsilon;
  size_t cache_stride = 0;  // elements from one variant's cache to the next
  // Not null: the queries are read from here (same layout), roped into
  // `query`. With part_count > 1, query_in, key and value hold a K-split
  // product's first partial sums, the rest part_stride floats apart each,
  // added in split order.
  const float* query_in = nullptr;
  size_t part_stride = 0;
  int part_count = 1;
};
hipError_t launch_rope(hipStream_t s, const DevStep* step, const RopeArgs& a,
                       int max_tokens);

struct AttentionArgs {
  const float* query;         // token t's roped heads at query + t * q_stride
  int q_stride;
  const uint16_t* key_cache;
  const uint16_t* value_cache;
  float* out;                 // [tokens][query_heads * head_dim]
  float* partials;            // [tokens][max_chunks][query_heads][head_dim]
  float* stats;               // [tokens][max_chunks][query_heads][4]
  int slots;
  int window;
  int head_dim;
  int query_heads;
  int kv_heads;
  int max_chunks;             // chunks a row may reach: the grid's width
  float scale_log2e;
  size_t cache_stride = 0;    // elements from one variant's cache to the next
  // Not null: the last row's scores (log2 units) of the keys it reads, head h
  // key earliest + i at store_scores[h * keys + i]; and each head's final
  // (m, l) at store_stats[2 h], [2 h + 1].
  float* store_scores = nullptr;
  float* store_stats = nullptr;
  int keys = 0;
  // Chunks the grid covers, when the caller knows the step's positions (0:
  // max_chunks); rows reading more would be left out, so it must be at
  // least live_chunks_over of the step's positions.
  int grid_chunks = 0;
};
hipError_t launch_attention(hipStream_t s, const DevStep* step,
                            const AttentionArgs& a, int max_tokens);

// One decode token's QK-norm, rope and KV append fused with its attention:
// one workgroup a (chunk, head), each writing its chunk state.
struct DecodeAttentionArgs {
  const float* qkv;           // the token's q (query_heads * d), k, v
  const float* turns;
  const float* query_gain;
  const float* key_gain;
  uint16_t* key_cache;
  uint16_t* value_cache;
  float* partials;            // [max_chunks][query_heads][d]
  float* stats;               // [max_chunks][query_heads][4]
  int slots;
  int window;
  int head_dim;
  int query_heads;
  int kv_heads;
  int max_chunks;
  float epsilon;
  float scale_log2e;
  // A variants step's rows (grid z): row r's q, k, v at qkv + r * qkv_stride,
  // its caches cache_stride elements on, its chunk states after row r - 1's
  // max_chunks (the fold's layout).
  int qkv_stride = 0;
  size_t cache_stride = 0;
  // Chunk slots launched, when the host knows the step's position (at least
  // the chunks live there; 0: max_chunks). The states keep max_chunks' layout.
  int grid_chunks = 0;
};
// The chunks a query at position p reads under `window` (chunk_range's count).
inline int live_chunks(uint32_t p, int window) {
  const uint32_t earliest = p + 1 > (uint32_t)window ? p + 1 - (uint32_t)window : 0;
  return (int)(p / kChunkKeys - earliest / kChunkKeys + 1);
}
// The most chunks a query at any of positions first..last reads: a window's
// chunk count never falls from p to p + 64 (the chunk of p + 64 is one
// further, its earliest key's at most one), so the last 64 positions decide.
inline int live_chunks_over(uint32_t first, uint32_t last, int window) {
  int most = 0;
  for (uint32_t p = last >= first + 63 ? last - 63 : first; p <= last; ++p) {
    const int n = live_chunks(p, window);
    most = n > most ? n : most;
  }
  return most;
}
hipError_t launch_attention_decode(hipStream_t s, const DevStep* step,
                                   const DecodeAttentionArgs& a, int rows = 1);

// Each row's chunk states folded in chunk order into out[row][heads * d].
struct FoldArgs {
  const float* partials;      // [tokens][max_chunks][query_heads][d]
  const float* stats;         // [tokens][max_chunks][query_heads][4]
  float* out;
  int window;
  int max_chunks;
  float* store_stats = nullptr;  // the last row's (m, l) a head, when not null
  // Not null (steps of several rows): the output also as bf16 pair planes
  // (plane_index order).
  uint16_t* out_hi = nullptr;
  uint16_t* out_lo = nullptr;
};
hipError_t launch_attention_fold(hipStream_t s, const DevStep* step, const FoldArgs& f,
                                 int max_tokens);
constexpr int kMaxFoldChunks = 224;  // chunk states of the static decode workspace: 14,272 keys
// Chunks a context may reach: Gemma 3 1B's trained 32,768 tokens, plus the
// partial chunk a window straddles (the fold stages them in segments).
constexpr int kMaxContextChunks = 32768 / kChunkKeys + 1;

// The capture store's copies at the step that ends the prompt: the last row
// of src (rows row_stride words apart) into dst, word for word
// (capture.wgsl); and the last row's scores turned into attention weights
// exp2(s - m) / l in place, zeros past the keys read (weights.wgsl).
hipError_t launch_capture_copy(hipStream_t s, const DevStep* step, const void* src,
                               size_t row_stride, int width, void* dst);
hipError_t launch_capture_weights(hipStream_t s, const DevStep* step, float* weights,
                                  const float* stats, int keys, int query_heads);

hipError_t launch_gather(hipStream_t s, const DevStep* step, QMatrix table,
                         const uint32_t* sampled, float* hidden, float scale,
                         int max_tokens);
hipError_t launch_edit(hipStream_t s, const DevStep* step,
                       const uint32_t* edits, int layer, float* act,
                       int width, int max_tokens);

// ---- output ------------------------------------------------------------
// Top-64 of `count` logits into candidates (64 x {bits, token}), sorted;
// `scratch` holds topk_scratch_words(count) words.
size_t topk_scratch_words(int count);
hipError_t launch_topk(hipStream_t s, const float* logits, int count,
                       uint32_t* scratch, uint32_t* candidates);
// The top-64 as above, then the draw (as launch_draw) and, when `advance`,
// the fed step's advance (as launch_advance), the last two in the final
// selection kernel.
hipError_t launch_select(hipStream_t s, DevStep* step, const float* logits, int count,
                         uint32_t* scratch, uint32_t* candidates, uint32_t* sampled,
                         uint32_t* token_log, bool advance);
// A variants step's selection: for each of `rows` rows of logits (count
// apart), its top-64 into candidates + 128 r and its draw into record r of
// sampled (token_log entry drawn * rows + r); then the step's advance to
// the next position, every row fed from its own record.
hipError_t launch_select_rows(hipStream_t s, DevStep* step, const float* logits, int count,
                              int rows, uint32_t* scratch, uint32_t* candidates,
                              uint32_t* sampled, uint32_t* token_log);
// The draw: record {token, failed, u bits, 0} into sampled; also appends
// the token to token_log[step.drawn] when token_log is not null.
hipError_t launch_draw(hipStream_t s, const DevStep* step,
                       const uint32_t* candidates, uint32_t* sampled,
                       uint32_t* token_log);
// A fed step's advance: position += tokens, tokens = 1, fed = 1,
// drawn += 1.
hipError_t launch_advance(hipStream_t s, DevStep* step);

}  // namespace frz
