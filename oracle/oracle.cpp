// CPU oracle for the Gemma-3-1B Q4_0 forward path: a restatement of the
// reference's WGSL arithmetic, rounding point for rounding point.
//
// TEST INFRASTRUCTURE ONLY (see oracle.h): loaded by tests/, smoke() and the
// CPU-baseline leg of bench.py, never by the product library.
//
// Built with -ffp-contract=off: every multiply and add written below rounds
// on its own, and every fused multiply-add is an explicit std::fma, as the
// reference's WGSL writes them.

#include "oracle.h"

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

namespace {

inline float as_float(uint32_t u) {
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}
inline uint32_t as_bits(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  return u;
}

constexpr int kRanges = 32;      // matmul.wgsl:45
constexpr int kChunkKeys = 64;   // attention.wgsl:60
constexpr int kTileKeys = 8;     // attention.cpp:54, B = 2048 / d at d = 256
constexpr int kCandidates = 64;  // residency/plan.h:195

// Range r's first group of a row of `groups` groups (matmul.wgsl:88-90).
inline int range_lo(int r, int groups) { return r * groups / kRanges; }

}  // namespace

extern "C" {

// ---- numerics ------------------------------------------------------------

// The reference's explicit e^x for x <= 0 (matmul.wgsl:122-135): Cody-Waite
// with ln 2 in two parts, Taylor to r^6 in Horner form, then ldexp.
float orc_exp_nonpositive(float x) {
  const float xc = std::max(x, -100.0f);
  const float k = std::floor(std::fma(xc, 1.4426950408889634f, 0.5f));
  float r = std::fma(k, -0.693145751953125f, xc);
  r = std::fma(k, -1.4286068203094172e-06f, r);
  float p = static_cast<float>(1.0 / 720.0);
  p = std::fma(p, r, static_cast<float>(1.0 / 120.0));
  p = std::fma(p, r, static_cast<float>(1.0 / 24.0));
  p = std::fma(p, r, static_cast<float>(1.0 / 6.0));
  p = std::fma(p, r, 0.5f);
  p = std::fma(p, r, 1.0f);
  p = std::fma(p, r, 1.0f);
  return std::ldexp(p, static_cast<int>(k));
}

// GELU, tanh form (matmul.wgsl:141-147).
float orc_gelu_tanh(float g) {
  const float z = 0.7978845608028654f * std::fma(0.044715f * g * g, g, g);
  const float e = orc_exp_nonpositive(-2.0f * std::fabs(z));
  const float sign = z > 0.0f ? 1.0f : (z < 0.0f ? -1.0f : 0.0f);
  const float t = sign * ((1.0f - e) * (1.0f / (1.0f + e)));
  const float half_g = 0.5f * g;
  return std::fma(half_g, t, half_g);
}

// 2^x, the definition this build gives WGSL's exp2 built-in (used by
// attention.wgsl:148-150, 322, 327 with x <= 0): k = rint(x), r = x - k
// exact in [-0.5, 0.5]; 2^r = e^(r ln 2) by its Taylor series to r^7 in
// Horner form with fma (truncation under 2^-27); times 2^k built from its
// exponent bits. Below -125.5 the result is 0, so every result is 0 or a
// normal number and no step depends on subnormal handling.
float orc_exp2(float x) {
  if (x < -125.5f) return 0.0f;
  if (x > 127.0f) x = 127.0f;
  const float k = std::nearbyint(x);
  const float r = x - k;
  float p = 1.525273380405984e-05f;
  p = std::fma(p, r, 1.5403530393381608e-04f);
  p = std::fma(p, r, 1.3333558146428443e-03f);
  p = std::fma(p, r, 9.618129107628477e-03f);
  p = std::fma(p, r, 5.550410866482158e-02f);
  p = std::fma(p, r, 2.402265069591007e-01f);
  p = std::fma(p, r, 6.931471805599453e-01f);
  p = std::fma(p, r, 1.0f);
  const uint32_t e = static_cast<uint32_t>(static_cast<int>(k) + 127) << 23;
  return p * as_float(e);
}

namespace {
// sin and cos of r in [-pi/4, pi/4] by their Taylor series (to r^11 and
// r^12), Horner form with fma in r^2.
inline float sin_kernel(float r) {
  const float z = r * r;
  float p = static_cast<float>(-1.0 / 39916800.0);
  p = std::fma(p, z, static_cast<float>(1.0 / 362880.0));
  p = std::fma(p, z, static_cast<float>(-1.0 / 5040.0));
  p = std::fma(p, z, static_cast<float>(1.0 / 120.0));
  p = std::fma(p, z, static_cast<float>(-1.0 / 6.0));
  return std::fma(r * z, p, r);
}
inline float cos_kernel(float r) {
  const float z = r * r;
  float p = static_cast<float>(1.0 / 479001600.0);
  p = std::fma(p, z, static_cast<float>(-1.0 / 3628800.0));
  p = std::fma(p, z, static_cast<float>(1.0 / 40320.0));
  p = std::fma(p, z, static_cast<float>(-1.0 / 720.0));
  p = std::fma(p, z, static_cast<float>(1.0 / 24.0));
  p = std::fma(p, z, -0.5f);
  return std::fma(z, p, 1.0f);
}
// The angle less k quarter turns, k = rint(angle * 2 / pi), pi/2 in three
// parts (Cody-Waite); the quadrant k mod 4.
inline float reduce_quadrant(float angle, int* quadrant) {
  const float k = std::nearbyint(angle * 0.63661977236758134f);
  float r = std::fma(-k, 1.5707963705062866f, angle);
  r = std::fma(-k, -4.3711388286737929e-08f, r);
  r = std::fma(-k, -1.7151245100059026e-15f, r);
  *quadrant = static_cast<int>(k) & 3;
  return r;
}
}  // namespace

// cos and sin of an angle in [-pi, pi], the definition this build gives
// WGSL's built-ins for rope's angles (rope.wgsl:122-129).
float orc_cos(float angle) {
  int q;
  const float r = reduce_quadrant(angle, &q);
  switch (q) {
    case 0: return cos_kernel(r);
    case 1: return -sin_kernel(r);
    case 2: return -cos_kernel(r);
    default: return sin_kernel(r);
  }
}
float orc_sin(float angle) {
  int q;
  const float r = reduce_quadrant(angle, &q);
  switch (q) {
    case 0: return sin_kernel(r);
    case 1: return cos_kernel(r);
    case 2: return -sin_kernel(r);
    default: return -cos_kernel(r);
  }
}

// WGSL's inverseSqrt as this build defines it: two correctly rounded ops.
float orc_inverse_sqrt(float x) { return 1.0f / std::sqrt(x); }

// F16 pack of one value (f16_pack.wgsl:16-20): saturate to +-65504, then
// round once to nearest, ties to even, subnormals kept.
uint16_t orc_f16_pack(float x) {
  if (std::isnan(x)) return 0x7E00;
  x = std::min(std::max(x, -65504.0f), 65504.0f);
  const uint32_t bits = as_bits(x);
  const uint32_t sign = (bits >> 16) & 0x8000u;
  const uint32_t mag = bits & 0x7FFFFFFFu;
  const uint32_t exp = mag >> 23;
  uint32_t h;
  if (exp >= 113) {
    const uint32_t mant = mag & 0x7FFFFFu;
    h = ((exp - 112) << 10) | (mant >> 13);
    const uint32_t rem = mant & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
  } else if (exp >= 102) {
    const uint32_t mant = (mag & 0x7FFFFFu) | 0x800000u;
    const uint32_t shift = 126 - exp;
    h = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (h & 1u))) ++h;
  } else {
    h = 0;
  }
  return static_cast<uint16_t>(sign | h);
}

// F16 to f32, exact (f16_pack.wgsl:24-25's unpack4).
float orc_f16_unpack(uint16_t h) {
  const uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1Fu;
  const uint32_t mant = h & 0x3FFu;
  if (exp == 0) {
    const float v = static_cast<float>(mant) * 5.9604644775390625e-08f;  // 2^-24
    return sign ? -v : v;
  }
  if (exp == 31) return as_float(sign | 0x7F800000u | (mant << 13));
  return as_float(sign | ((exp + 112) << 23) | (mant << 13));
}

// WGSL's dot of two vec4s as this build defines it: products and sums in
// component order, each rounded.
float orc_dot4(const float* a, const float* b) {
  return ((a[0] * b[0] + a[1] * b[1]) + a[2] * b[2]) + a[3] * b[3];
}

// ---- formats and products -------------------------------------------------

// A Q4_0 block's 32 weights, exact (q4_0.wgsl:71-83; q4_0.h:21-23): weight
// j = ((qs[j] & 0xF) - 8) * d, weight j + 16 = ((qs[j] >> 4) - 8) * d.
void orc_q4_0_unpack(const uint8_t* block, float out[32]) {
  const uint16_t d_bits = static_cast<uint16_t>(block[0] | (block[1] << 8));
  const float d = orc_f16_unpack(d_bits);
  for (int j = 0; j < 16; ++j) {
    const uint8_t q = block[2 + j];
    out[j] = (static_cast<float>(q & 0xF) - 8.0f) * d;
    out[j + 16] = (static_cast<float>(q >> 4) - 8.0f) * d;
  }
}

// A Q4_1 block's 32 weights (q4_1.wgsl:12-25): weight j = (qs[j] & 0xF) * d
// + m, weight j + 16 = (qs[j] >> 4) * d + m. The product of a 4-bit code and
// an f16 scale is exact in f32, so the one rounding is the addition's.
void orc_q4_1_unpack(const uint8_t* block, float out[32]) {
  const float d = orc_f16_unpack(static_cast<uint16_t>(block[0] | (block[1] << 8)));
  const float m = orc_f16_unpack(static_cast<uint16_t>(block[2] | (block[3] << 8)));
  for (int j = 0; j < 16; ++j) {
    const uint8_t q = block[4 + j];
    out[j] = static_cast<float>(q & 0xF) * d + m;
    out[j + 16] = static_cast<float>(q >> 4) * d + m;
  }
}

// A Q8_0 block's 32 weights (q8_0.wgsl:12-24): weight j = qs[j] * d, qs
// signed bytes; exact in f32.
void orc_q8_0_unpack(const uint8_t* block, float out[32]) {
  const float d = orc_f16_unpack(static_cast<uint16_t>(block[0] | (block[1] << 8)));
  for (int j = 0; j < 32; ++j) out[j] = static_cast<float>(static_cast<int8_t>(block[2 + j])) * d;
}

int orc_block_bytes(int format) {
  switch (format) {
    case 0: case 2: return 18;
    case 3: return 20;
    case 8: return 34;
    default: return 0;
  }
}

namespace {
void unpack_format(int format, const uint8_t* block, float out[32]) {
  if (format == 3) {
    orc_q4_1_unpack(block, out);
  } else if (format == 8) {
    orc_q8_0_unpack(block, out);
  } else {
    orc_q4_0_unpack(block, out);
  }
}

// One output of a product in the reference's order (matmul.h:88-97,
// matmul.wgsl:154-185): range r's products chained by fma from zero, k in
// order; then the 32 range sums added in order to a total from zero. The
// order is the same whatever the weights' format (format.h: each format
// only supplies its unpack).
float format_row_total(int format, const uint8_t* row, int cols, const float* x) {
  const int groups = cols / 32;
  const int bb = orc_block_bytes(format);
  float total = 0.0f;
  float w[32];
  for (int r = 0; r < kRanges; ++r) {
    float s = 0.0f;
    for (int g = range_lo(r, groups); g < range_lo(r + 1, groups); ++g) {
      unpack_format(format, row + static_cast<size_t>(g) * bb, w);
      const float* xg = x + g * 32;
      for (int i = 0; i < 32; ++i) s = std::fma(w[i], xg[i], s);
    }
    total = total + s;
  }
  return total;
}

float row_total(const uint8_t* row, int cols, const float* x) {
  return format_row_total(2, row, cols, x);
}
}  // namespace

void orc_gemv(const uint8_t* w, int rows, int cols, const float* x,
              float* y) {
  orc_gemv_format(2, w, rows, cols, x, y);
}

void orc_gemv_format(int format, const uint8_t* w, int rows, int cols, const float* x,
                     float* y) {
  const size_t row_bytes = static_cast<size_t>(cols) / 32 * orc_block_bytes(format);
#pragma omp parallel for schedule(static)
  for (int o = 0; o < rows; ++o) y[o] = format_row_total(format, w + o * row_bytes, cols, x);
}

// gelu_tanh(gate) * up, gate and up each in the order above
// (matmul.wgsl:247-271).
void orc_gated(const uint8_t* gate, const uint8_t* up, int rows, int cols,
               const float* x, float* act) {
  const size_t row_bytes = static_cast<size_t>(cols) / 32 * 18;
#pragma omp parallel for schedule(static)
  for (int o = 0; o < rows; ++o) {
    const float g = row_total(gate + o * row_bytes, cols, x);
    const float u = row_total(up + o * row_bytes, cols, x);
    act[o] = orc_gelu_tanh(g) * u;
  }
}

// ---- per-row kernels --------------------------------------------------------

namespace {
constexpr int kNormInvocations = 256;  // norm.cpp: one workgroup of 256

// The norm's sum of squares (norm.wgsl:75-85, 138-144, 182-190): invocation
// i sums its vec4s i, i + 256, ... by dot, from zero; then the halving tree
// over the 256 partial sums.
float norm_squares(const float* v, int width) {
  const int vec4s = width / 4;
  float partial[kNormInvocations];
  for (int i = 0; i < kNormInvocations; ++i) {
    float s = 0.0f;
    for (int q = i; q < vec4s; q += kNormInvocations) {
      s = s + orc_dot4(v + 4 * q, v + 4 * q);
    }
    partial[i] = s;
  }
  for (int stride = kNormInvocations / 2; stride > 0; stride /= 2) {
    for (int i = 0; i < stride; ++i) partial[i] = partial[i] + partial[i + stride];
  }
  return partial[0];
}
}  // namespace

// RMSNorm with the residual add and Gemma's post-norm fused in
// (norm.wgsl:96-198): where `add`, y (the block's output) is first normed
// with its own gain and times post_scale when `post_norm`, then added into
// the hidden row, which is written back; normed = (x * r) * gain.
void orc_norm_row(const float* gain, const float* post_gain, int add,
                  int post_norm, float post_scale, float epsilon, int width,
                  float* hidden, const float* output, float* normed) {
  orc_norm_row_added(gain, post_gain, add, post_norm, post_scale, epsilon, width, hidden, output,
                     normed, nullptr);
}

// The same, also giving the vector the add added (the block's output after
// its post-norm) when `added` is not null: the capture store's additions
// (capture.h:18-21).
void orc_norm_row_added(const float* gain, const float* post_gain, int add,
                        int post_norm, float post_scale, float epsilon, int width,
                        float* hidden, const float* output, float* normed, float* added) {
  const float n = static_cast<float>(width);
  if (add) {
    std::vector<float> y(output, output + width);
    if (post_norm) {
      const float r =
          orc_inverse_sqrt(norm_squares(y.data(), width) / n + epsilon);
      for (int i = 0; i < width; ++i) y[i] = ((y[i] * r) * post_gain[i]) * post_scale;
    }
    for (int i = 0; i < width; ++i) hidden[i] = hidden[i] + y[i];
    if (added) std::copy(y.begin(), y.end(), added);
  }
  const float r = orc_inverse_sqrt(norm_squares(hidden, width) / n + epsilon);
  for (int i = 0; i < width; ++i) normed[i] = (hidden[i] * r) * gain[i];
}

// Each pair's turns a position, theta_k / 2 pi with theta_k =
// base^(-2k/d), in f64, rounded once to f32 (rope.cpp:95-106).
void orc_rope_turns(float base, int head_dim, float* turns) {
  const double pi = 3.14159265358979323846;
  for (int k = 0; k < head_dim / 2; ++k) {
    const double theta =
        std::pow(static_cast<double>(base), -2.0 * k / head_dim);
    turns[k] = static_cast<float>(theta / (2 * pi));
  }
}

// QK-norm, rope and the KV-cache append for one token (rope.wgsl:51-138,
// rope_cache.wgsl:153-229). A head's lane i holds dimensions 4i..4i+3 and
// 4i+d/2..4i+d/2+3; the head's squares meet in a halving tree over its d/8
// lanes; pairs (k, k + d/2) rotate by angle 2 pi (t - round(t)), t =
// f32(p) * turns_k. Keys and values are packed to F16 at slot p mod slots.
void orc_rope_row(int position, int slots, int head_dim, int query_heads,
                  int kv_heads, float epsilon, const float* turns,
                  const float* query_gain, const float* key_gain,
                  float* query, const float* key, const float* value,
                  uint16_t* key_cache, uint16_t* value_cache) {
  const int lanes = head_dim / 8;
  const int half = head_dim / 2;
  std::vector<float> cosines(half), sines(half);
  for (int k = 0; k < half; ++k) {
    const float t = static_cast<float>(position) * turns[k];
    const float angle = 6.283185307179586f * (t - std::nearbyint(t));
    cosines[k] = orc_cos(angle);
    sines[k] = orc_sin(angle);
  }
  const int slot = position % slots;
  std::vector<float> lane_sum(lanes);
  for (int h = 0; h < query_heads + 2 * kv_heads; ++h) {
    const bool is_query = h < query_heads;
    const bool is_value = h >= query_heads + kv_heads;
    const int kv = is_value ? h - query_heads - kv_heads : h - query_heads;
    float* row;
    std::vector<float> scratch(head_dim);
    if (is_query) {
      row = query + h * head_dim;
    } else {
      const float* src = (is_value ? value : key) + kv * head_dim;
      std::copy(src, src + head_dim, scratch.begin());
      row = scratch.data();
    }
    if (!is_value) {
      for (int i = 0; i < lanes; ++i) {
        lane_sum[i] = orc_dot4(row + 4 * i, row + 4 * i) +
                      orc_dot4(row + half + 4 * i, row + half + 4 * i);
      }
      for (int stride = lanes / 2; stride > 0; stride /= 2) {
        for (int i = 0; i < stride; ++i) lane_sum[i] = lane_sum[i] + lane_sum[i + stride];
      }
      const float r = orc_inverse_sqrt(lane_sum[0] / static_cast<float>(head_dim) + epsilon);
      const float* g = is_query ? query_gain : key_gain;
      for (int i = 0; i < head_dim; ++i) row[i] = (row[i] * r) * g[i];
      for (int k = 0; k < half; ++k) {
        const float a = row[k], b = row[k + half];
        row[k] = a * cosines[k] - b * sines[k];
        row[k + half] = a * sines[k] + b * cosines[k];
      }
    }
    if (!is_query) {
      uint16_t* cache = (is_value ? value_cache : key_cache) +
                        (static_cast<size_t>(slot) * kv_heads + kv) * head_dim;
      for (int i = 0; i < head_dim; ++i) cache[i] = orc_f16_pack(row[i]);
    }
  }
}

namespace {
struct Fold {
  float a, b, m;
};
// attention.wgsl:135-151.
Fold fold_factors(bool live, float m, bool chunk_is_live, float chunk_max) {
  if (!chunk_is_live) return {1.0f, 0.0f, m};
  if (!live) return {0.0f, 1.0f, chunk_max};
  if (m == chunk_max) return {1.0f, 1.0f, m};
  if (m > chunk_max) return {1.0f, orc_exp2(chunk_max - m), m};
  return {orc_exp2(m - chunk_max), 1.0f, chunk_max};
}
}  // namespace

// Attention for one token at `position` (attention.wgsl:166-398): per query
// head, chunks of 64 keys from the one holding the earliest key the window
// admits, each from an empty state over 8-key tiles from the tile holding
// the earliest key (an online softmax in base 2, q scaled by scale * log2 e);
// chunks folded in order; then o / l.
void orc_attention_row(int position, int window, int slots, int head_dim,
                       int query_heads, int kv_heads, float scale_log2e,
                       const float* query, const uint16_t* key_cache,
                       const uint16_t* value_cache, float* out) {
  orc_attention_row_scores(position, window, slots, head_dim, query_heads, kv_heads, scale_log2e,
                           query, key_cache, value_cache, out, nullptr, 0, nullptr);
}

// The same, also giving each head's scores of the keys it reads (key
// earliest + i at scores[h * keys + i], earliest = p + 1 - min(p + 1, keys))
// and its final (m, l) at stats[2 h], stats[2 h + 1], when not null: the
// capture store's scores and statistics (weights.h:12-21).
void orc_attention_row_scores(int position, int window, int slots, int head_dim,
                              int query_heads, int kv_heads, float scale_log2e,
                              const float* query, const uint16_t* key_cache,
                              const uint16_t* value_cache, float* out, float* scores,
                              int keys, float* stats) {
  const int p = position;
  const int score0 = p + 1 - std::min(p + 1, keys);
  const int group = query_heads / kv_heads;
  const int earliest = p + 1 > window ? p + 1 - window : 0;
  std::vector<float> q(head_dim), o_run(head_dim), o_chunk(head_dim),
      kf(head_dim);
  for (int h = 0; h < query_heads; ++h) {
    const int kv = h / group;
    for (int i = 0; i < head_dim; ++i) q[i] = query[h * head_dim + i] * scale_log2e;
    bool run_live = false;
    float run_m = 0.0f, run_l = 0.0f;
    std::fill(o_run.begin(), o_run.end(), 0.0f);
    for (int c = earliest / kChunkKeys; c <= p / kChunkKeys; ++c) {
      bool chunk_live = false;
      float cm = 0.0f, cl = 0.0f;
      std::fill(o_chunk.begin(), o_chunk.end(), 0.0f);
      const int k_begin = std::max(c * kChunkKeys, earliest / kTileKeys * kTileKeys);
      const int k_end = std::min((c + 1) * kChunkKeys, p + 1);
      for (int j0 = k_begin; j0 < k_end; j0 += kTileKeys) {
        float s[kTileKeys], e[kTileKeys];
        bool live[kTileKeys];
        float top_tile = 0.0f;
        bool seen = false;
        for (int b = 0; b < kTileKeys; ++b) {
          const int j = j0 + b;
          live[b] = j < k_end && j <= p && j + window > p;
          s[b] = 0.0f;
          if (live[b]) {
            const uint16_t* kr =
                key_cache + (static_cast<size_t>(j % slots) * kv_heads + kv) * head_dim;
            for (int i = 0; i < head_dim; ++i) kf[i] = orc_f16_unpack(kr[i]);
            float acc = 0.0f;
            for (int w = 0; w < head_dim / 4; ++w) acc += orc_dot4(q.data() + 4 * w, kf.data() + 4 * w);
            s[b] = acc;
            if (scores) scores[static_cast<size_t>(h) * keys + (j - score0)] = acc;
            top_tile = seen ? std::max(top_tile, acc) : acc;
            seen = true;
          }
        }
        float a = 1.0f;
        if (seen) {
          const float old = chunk_live ? cm : top_tile;
          chunk_live = true;
          const float top = std::max(old, top_tile);
          a = old == top ? 1.0f : orc_exp2(old - top);
          float sum = 0.0f;
          for (int b = 0; b < kTileKeys; ++b) {
            e[b] = live[b] ? orc_exp2(s[b] - top) : 0.0f;
            sum += e[b];
          }
          cl = cl * a + sum;
          cm = top;
        } else {
          for (int b = 0; b < kTileKeys; ++b) e[b] = 0.0f;
        }
        for (int i = 0; i < head_dim; ++i) o_chunk[i] = o_chunk[i] * a;
        for (int b = 0; b < kTileKeys; ++b) {
          const int j = j0 + b;
          if (j >= k_end) {
            // The tile's rows past the chunk are staged as zeros
            // (attention.wgsl:259-273): each adds e * 0 = +0.
            for (int i = 0; i < head_dim; ++i) o_chunk[i] = o_chunk[i] + e[b] * 0.0f;
            continue;
          }
          const uint16_t* vr =
              value_cache + (static_cast<size_t>(j % slots) * kv_heads + kv) * head_dim;
          for (int i = 0; i < head_dim; ++i) o_chunk[i] = o_chunk[i] + e[b] * orc_f16_unpack(vr[i]);
        }
      }
      const Fold f = fold_factors(run_live, run_m, chunk_live, cm);
      run_l = run_l * f.a + cl * f.b;
      for (int i = 0; i < head_dim; ++i) o_run[i] = o_run[i] * f.a + o_chunk[i] * f.b;
      run_m = f.m;
      run_live = run_live || chunk_live;
    }
    for (int i = 0; i < head_dim; ++i) out[h * head_dim + i] = run_live ? o_run[i] / run_l : 0.0f;
    if (stats) {
      stats[2 * h] = run_m;
      stats[2 * h + 1] = run_l;
    }
  }
}

// Token embedding row times the scale (gather.wgsl:25-48).
void orc_gather_row(const uint8_t* table, int width, uint32_t token,
                    float scale, float* hidden) {
  orc_gather_row_format(2, table, width, token, scale, hidden);
}

void orc_gather_row_format(int format, const uint8_t* table, int width, uint32_t token,
                           float scale, float* hidden) {
  const int bb = orc_block_bytes(format);
  const size_t row_bytes = static_cast<size_t>(width) / 32 * bb;
  float w[32];
  for (int g = 0; g < width / 32; ++g) {
    unpack_format(format, table + token * row_bytes + static_cast<size_t>(g) * bb, w);
    for (int i = 0; i < 32; ++i) hidden[g * 32 + i] = w[i] * scale;
  }
}

// One layer's pins on one activation row (edit.wgsl:55-76; edit.cpp:93-103).
void orc_edit_row(const uint32_t* table, int layer, uint32_t position,
                  int width, float* activation) {
  (void)width;
  const uint32_t first = table[2 * layer];
  const uint32_t count = table[2 * layer + 1];
  for (uint32_t i = 0; i < count; ++i) {
    const uint32_t* e = table + first + 5 * i;
    if (position < e[3] || position >= e[4]) continue;
    const float value = as_float(e[2]);
    float& neuron = activation[e[0]];
    if (e[1] == 1u) {
      if (value != 1.0f) neuron = neuron * value;
    } else {
      neuron = value;
    }
  }
}

namespace {
// topk.wgsl:32-55.
uint32_t key_of(uint32_t b) {
  if (b == 0x80000000u) b = 0;
  if ((b & 0x7F800000u) == 0x7F800000u && (b & 0x007FFFFFu) != 0) return 0xFFFFFFFFu;
  if (b & 0x80000000u) return ~b;
  return b | 0x80000000u;
}
uint32_t bits_of(uint32_t key) {
  if (key == 0xFFFFFFFFu) return 0x7FC00000u;
  if (key & 0x80000000u) return key & 0x7FFFFFFFu;
  return ~key;
}
}  // namespace

// The 64 largest logits in the reference's total order (topk.wgsl:57-61):
// larger key first, equal keys by lower token; as (logit bits, token).
void orc_topk(const float* logits, int count, uint32_t* bits, uint32_t* ids) {
  std::vector<std::pair<uint32_t, uint32_t>> e(count);
  for (int i = 0; i < count; ++i) e[i] = {key_of(as_bits(logits[i])), static_cast<uint32_t>(i)};
  const int k = std::min(count, kCandidates);
  std::partial_sort(e.begin(), e.begin() + k, e.end(), [](const auto& x, const auto& y) {
    return x.first > y.first || (x.first == y.first && x.second < y.second);
  });
  for (int i = 0; i < kCandidates; ++i) {
    if (i < k) {
      bits[i] = bits_of(e[i].first);
      ids[i] = e[i].second;
    } else {
      bits[i] = bits_of(0);
      ids[i] = 0xFFFFFFFFu;
    }
  }
}

// The high word of a * b from 16-bit halves (draw.wgsl:34-45).
uint32_t orc_mulhi(uint32_t a, uint32_t b) {
  const uint32_t a0 = a & 0xFFFFu, a1 = a >> 16, b0 = b & 0xFFFFu, b1 = b >> 16;
  const uint32_t p00 = a0 * b0, p01 = a0 * b1, p10 = a1 * b0, p11 = a1 * b1;
  const uint32_t mid = (p00 >> 16) + (p01 & 0xFFFFu) + (p10 & 0xFFFFu);
  return p11 + (p01 >> 16) + (p10 >> 16) + (mid >> 16);
}

// Philox4x32-10 (draw.wgsl:48-60).
void orc_philox(const uint32_t counter[4], const uint32_t key[2],
                uint32_t out[4]) {
  uint32_t c0 = counter[0], c1 = counter[1], c2 = counter[2], c3 = counter[3];
  uint32_t k0 = key[0], k1 = key[1];
  for (int r = 0; r < 10; ++r) {
    const uint32_t hi0 = orc_mulhi(0xD2511F53u, c0), lo0 = 0xD2511F53u * c0;
    const uint32_t hi1 = orc_mulhi(0xCD9E8D57u, c2), lo1 = 0xCD9E8D57u * c2;
    const uint32_t n0 = hi1 ^ c1 ^ k0, n1 = lo1, n2 = hi0 ^ c3 ^ k1, n3 = lo0;
    c0 = n0; c1 = n1; c2 = n2; c3 = n3;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

// The draw (draw.wgsl:77-170): top-k, top-p, min-p and temperature over the
// sorted candidates, then an inverse transform of one Philox uniform at
// counter (position + tokens, 0, 0, 0). Writes {token, failed, u bits, 0}.
void orc_draw(const uint32_t* cand_bits, const uint32_t* cand_ids,
              uint32_t count, uint32_t top_k, float temperature, float top_p,
              float min_p, float log_min_p, uint32_t counter,
              uint32_t seed_lo, uint32_t seed_hi, uint32_t record[4]) {
  const uint32_t k = std::min(top_k, count);
  const bool use_top_p = top_p < 1.0f;
  const bool failed = (cand_bits[0] & 0x7F800000u) == 0x7F800000u;
  float weight[kCandidates] = {}, tempered[kCandidates] = {}, running[kCandidates] = {};
  uint32_t above[kCandidates] = {};
  for (uint32_t t = 0; t < k; ++t) {
    if (!failed && cand_bits[t] != 0xFF800000u) {
      const float first = as_float(cand_bits[0]);
      const float mine = as_float(cand_bits[t]);
      if (use_top_p) weight[t] = orc_exp_nonpositive(mine - first);
      if (temperature > 0.0f) tempered[t] = orc_exp_nonpositive((mine - first) / temperature);
      above[t] = (min_p == 0.0f || mine >= first + log_min_p) ? 1u : 0u;
    }
  }
  const uint32_t ctr[4] = {counter, 0, 0, 0};
  const uint32_t key[2] = {seed_lo, seed_hi};
  uint32_t ph[4];
  orc_philox(ctr, key, ph);
  const float u = static_cast<float>(ph[0] >> 9) * (1.0f / 8388608.0f) + (1.0f / 16777216.0f);
  if (use_top_p) {
    float sum = 0.0f;
    for (uint32_t i = 0; i < k; ++i) sum = sum + weight[i];
    if (!failed) {
      for (uint32_t t = 0; t < k; ++t) weight[t] = weight[t] / sum;
    }
  }
  uint32_t kept = k;
  float cumulative = 0.0f, tempered_sum = 0.0f;
  for (uint32_t i = 0; i < k; ++i) {
    tempered_sum = tempered_sum + tempered[i];
    running[i] = tempered_sum;
    if (use_top_p) {
      cumulative = cumulative + weight[i];
      if (cumulative >= top_p) {
        kept = i + 1;
        break;
      }
    }
  }
  uint32_t survivors = 1;
  while (survivors < kept && above[survivors] == 1u) ++survivors;
  uint32_t chosen = 0;
  if (temperature > 0.0f) {
    const float goal = u * running[survivors - 1];
    chosen = survivors - 1;
    for (uint32_t i = 0; i < survivors; ++i) {
      if (running[i] > goal) {
        chosen = i;
        break;
      }
    }
  }
  record[0] = failed ? 0u : cand_ids[chosen];
  record[1] = failed ? 1u : 0u;
  record[2] = as_bits(u);
  record[3] = 0;
}

// ---- the model -----------------------------------------------------------------

struct orc_model {
  orc_config c;
  std::vector<orc_layer_weights> w;
  const uint8_t* embedding;
  const float* output_norm;
  std::vector<std::vector<uint16_t>> kcache, vcache;
  std::vector<int> slots, windows;
  std::vector<std::vector<float>> turns;
  std::vector<uint32_t> edits;
  std::vector<float> hidden, normed, output, q, k, v, attn, act;
  std::vector<float> residuals;  // [layers][hidden]: the last token's
  bool capture = false;
  std::vector<std::vector<uint32_t>> cap;  // [layer * 8 + slot]: the last token's
};

namespace {
// A captured value's words (floats as their bits), for layer l's slot.
void put_words(orc_model* m, int layer, int slot, const float* v, int n) {
  std::vector<uint32_t>& out = m->cap[static_cast<size_t>(layer) * 8 + slot];
  out.resize(n);
  std::memcpy(out.data(), v, static_cast<size_t>(n) * 4);
}
}  // namespace

orc_model* orc_model_create(const orc_config* config,
                            const orc_layer_weights* layers,
                            const uint8_t* embedding,
                            const float* output_norm) {
  orc_model* m = new orc_model();
  m->c = *config;
  const orc_config& c = m->c;
  m->w.assign(layers, layers + c.layers);
  m->embedding = embedding;
  m->output_norm = output_norm;
  const int kvw = c.kv_heads * c.head_dim;
  for (int l = 0; l < c.layers; ++l) {
    const bool global = l % c.pattern == c.pattern - 1;
    const int slots = global ? c.context : c.local_slots;
    m->slots.push_back(slots);
    m->windows.push_back(global ? c.context : c.window);
    m->kcache.emplace_back(static_cast<size_t>(slots) * kvw, 0);
    m->vcache.emplace_back(static_cast<size_t>(slots) * kvw, 0);
    std::vector<float> t(c.head_dim / 2);
    orc_rope_turns(global ? c.rope_global : c.rope_local, c.head_dim, t.data());
    m->turns.push_back(t);
  }
  m->edits.assign(2 * c.layers, 0);
  m->hidden.resize(c.hidden);
  m->normed.resize(c.hidden);
  m->output.resize(c.hidden);
  m->q.resize(c.query_heads * c.head_dim);
  m->k.resize(kvw);
  m->v.resize(kvw);
  m->attn.resize(c.query_heads * c.head_dim);
  m->act.resize(c.ffn);
  m->residuals.resize(static_cast<size_t>(c.layers) * c.hidden);
  return m;
}

void orc_model_destroy(orc_model* m) { delete m; }

orc_model* orc_model_clone(const orc_model* m) { return new orc_model(*m); }

void orc_model_set_edits(orc_model* m, const uint32_t* table, int words) {
  m->edits.assign(table, table + words);
}

// One token through the graph (graph.cpp:290-470; gemma3.cpp:100-111): the
// embedding times sqrt(width) in f32; per layer the attention norm (adding
// the last block's post-normed output), Q/K/V, rope, attention, O; the
// feed-forward norm, gate-up with GELU, the pins, down; then the final norm
// and the tied head.
void orc_model_token(orc_model* m, uint32_t token, int position,
                     float* logits) {
  const orc_config& c = m->c;
  const int H = c.hidden;
  const int qw = c.query_heads * c.head_dim;
  const int kvw = c.kv_heads * c.head_dim;
  orc_gather_row_format(c.embedding_format, m->embedding, H, token,
                        std::sqrt(static_cast<float>(H)),
                 m->hidden.data());
  const float* pending = nullptr;
  const float scale_log2e = static_cast<float>(
      static_cast<double>(1.0f / std::sqrt(static_cast<float>(c.head_dim))) *
      1.4426950408889634);
  for (int l = 0; l < c.layers; ++l) {
    const orc_layer_weights& w = m->w[l];
    std::vector<float> added(H);
    orc_norm_row_added(w.attn_norm, pending, pending != nullptr, pending != nullptr,
                       1.0f, c.epsilon, H, m->hidden.data(), m->output.data(),
                       m->normed.data(), added.data());
    // The residual entering layer l: X after the add its first norm makes
    // (capture.h:15-17), layer 0's the embedding row.
    std::copy(m->hidden.begin(), m->hidden.end(),
              m->residuals.begin() + static_cast<size_t>(l) * H);
    if (m->capture) {
      put_words(m, l, 1, m->hidden.data(), H);
      if (l > 0) put_words(m, l - 1, 3, added.data(), H);
    }
    orc_gemv(w.q, qw, H, m->normed.data(), m->q.data());
    orc_gemv(w.k, kvw, H, m->normed.data(), m->k.data());
    orc_gemv(w.v, kvw, H, m->normed.data(), m->v.data());
    orc_rope_row(position, m->slots[l], c.head_dim, c.query_heads, c.kv_heads,
                 c.epsilon, m->turns[l].data(), w.q_norm, w.k_norm,
                 m->q.data(), m->k.data(), m->v.data(), m->kcache[l].data(),
                 m->vcache[l].data());
    if (m->capture) {
      // Q after rope; each head's scores turned into weights by the fold's
      // (m, l), zeros past the keys read (weights.h:29-40).
      put_words(m, l, 4, m->q.data(), qw);
      const int keys = std::min(m->windows[l], c.context);
      std::vector<float> wts(static_cast<size_t>(c.query_heads) * keys, 0.0f);
      std::vector<float> st(2 * c.query_heads);
      orc_attention_row_scores(position, m->windows[l], m->slots[l], c.head_dim, c.query_heads,
                               c.kv_heads, scale_log2e, m->q.data(), m->kcache[l].data(),
                               m->vcache[l].data(), m->attn.data(), wts.data(), keys, st.data());
      const int read = std::min(position + 1, keys);
      for (int h = 0; h < c.query_heads; ++h) {
        for (int i = 0; i < keys; ++i) {
          float& x = wts[static_cast<size_t>(h) * keys + i];
          x = i < read ? orc_exp2(x - st[2 * h]) / st[2 * h + 1] : 0.0f;
        }
      }
      put_words(m, l, 5, wts.data(), static_cast<int>(wts.size()));
      put_words(m, l, 6, st.data(), 2 * c.query_heads);
    } else {
      orc_attention_row(position, m->windows[l], m->slots[l], c.head_dim,
                        c.query_heads, c.kv_heads, scale_log2e, m->q.data(),
                        m->kcache[l].data(), m->vcache[l].data(),
                        m->attn.data());
    }
    orc_gemv(w.o, H, qw, m->attn.data(), m->output.data());
    orc_norm_row_added(w.ffn_norm, w.post_attn_norm, 1, 1, 1.0f, c.epsilon, H,
                       m->hidden.data(), m->output.data(), m->normed.data(), added.data());
    if (m->capture) put_words(m, l, 2, added.data(), H);
    orc_gated(w.gate, w.up, c.ffn, H, m->normed.data(), m->act.data());
    orc_edit_row(m->edits.data(), l, static_cast<uint32_t>(position), c.ffn,
                 m->act.data());
    if (m->capture) put_words(m, l, 0, m->act.data(), c.ffn);
    orc_gemv_format(w.down_format, w.down, H, c.ffn, m->act.data(), m->output.data());
    pending = w.post_ffn_norm;
  }
  std::vector<float> added(H);
  orc_norm_row_added(m->output_norm, pending, 1, 1, 1.0f, c.epsilon, H,
                     m->hidden.data(), m->output.data(), m->normed.data(), added.data());
  if (m->capture) put_words(m, c.layers - 1, 3, added.data(), H);
  if (logits) orc_gemv_format(c.embedding_format, m->embedding, c.vocab, H, m->normed.data(), logits);
  if (m->capture) {
    // Readouts (capture.h:28-34): the residual entering layer l + 1 through
    // the final norm, the head and the selection; the last layer's is the
    // token's own selection.
    std::vector<float> x(H), nrm(H), lg(c.vocab);
    std::vector<uint32_t> bits(kCandidates), ids(kCandidates), pairs(2 * kCandidates);
    for (int l = 0; l < c.layers; ++l) {
      if (l + 1 < c.layers) {
        std::copy(m->residuals.begin() + static_cast<size_t>(l + 1) * H,
                  m->residuals.begin() + static_cast<size_t>(l + 2) * H, x.begin());
        orc_norm_row(m->output_norm, nullptr, 0, 0, 1.0f, c.epsilon, H, x.data(), nullptr,
                     nrm.data());
      } else {
        nrm = m->normed;
      }
      orc_gemv_format(c.embedding_format, m->embedding, c.vocab, H, nrm.data(), lg.data());
      orc_topk(lg.data(), c.vocab, bits.data(), ids.data());
      for (int i = 0; i < kCandidates; ++i) {
        pairs[2 * i] = bits[i];
        pairs[2 * i + 1] = ids[i];
      }
      m->cap[static_cast<size_t>(l) * 8 + 7] = pairs;
    }
  }
}

namespace {
// n rows of a product at once: y[t][o] = format_row_total(W_o, x_t) for each
// row t, bit for bit (the same fma chain a range, k in order, and the same
// ordered totals), with each weight row decoded once for all n rows. The
// chains of the n rows are independent, so they step together over k.
void gemm_rows(int format, const uint8_t* w, int rows, int cols, const float* x, int n,
               float* y) {
  const int groups = cols / 32;
  const int bb = orc_block_bytes(format);
  const size_t row_bytes = static_cast<size_t>(groups) * bb;
  std::vector<float> xt(static_cast<size_t>(cols) * n);  // [k][t]
  for (int t = 0; t < n; ++t)
    for (int k = 0; k < cols; ++k) xt[static_cast<size_t>(k) * n + t] = x[static_cast<size_t>(t) * cols + k];
#pragma omp parallel
  {
    std::vector<float> wrow(cols), s(n), total(n);
#pragma omp for schedule(static)
    for (int o = 0; o < rows; ++o) {
      for (int g = 0; g < groups; ++g)
        unpack_format(format, w + o * row_bytes + static_cast<size_t>(g) * bb, &wrow[g * 32]);
      std::fill(total.begin(), total.end(), 0.0f);
      for (int r = 0; r < kRanges; ++r) {
        std::fill(s.begin(), s.end(), 0.0f);
        for (int k = range_lo(r, groups) * 32; k < range_lo(r + 1, groups) * 32; ++k) {
          const float wk = wrow[k];
          const float* xk = &xt[static_cast<size_t>(k) * n];
#pragma omp simd
          for (int t = 0; t < n; ++t) s[t] = std::fma(wk, xk[t], s[t]);
        }
        for (int t = 0; t < n; ++t) total[t] = total[t] + s[t];
      }
      for (int t = 0; t < n; ++t) y[static_cast<size_t>(t) * rows + o] = total[t];
    }
  }
}
}  // namespace

void orc_model_block(orc_model* m, const uint32_t* tokens, int n, int position,
                     float* logits) {
  const orc_config& c = m->c;
  const int H = c.hidden;
  const int qw = c.query_heads * c.head_dim;
  const int kvw = c.kv_heads * c.head_dim;
  const size_t N = static_cast<size_t>(n);
  std::vector<float> hidden(N * H), normed(N * H), output(N * H, 0.0f), q(N * qw),
      k(N * kvw), v(N * kvw), attn(N * qw), gate(N * c.ffn), up(N * c.ffn), act(N * c.ffn);
  for (int t = 0; t < n; ++t) {
    orc_gather_row_format(c.embedding_format, m->embedding, H, tokens[t],
                          std::sqrt(static_cast<float>(H)), &hidden[static_cast<size_t>(t) * H]);
  }
  const float* pending = nullptr;
  const float scale_log2e = static_cast<float>(
      static_cast<double>(1.0f / std::sqrt(static_cast<float>(c.head_dim))) *
      1.4426950408889634);
  for (int l = 0; l < c.layers; ++l) {
    const orc_layer_weights& w = m->w[l];
    for (int t = 0; t < n; ++t) {
      orc_norm_row(w.attn_norm, pending, pending != nullptr, pending != nullptr, 1.0f, c.epsilon,
                   H, &hidden[t * static_cast<size_t>(H)], &output[t * static_cast<size_t>(H)],
                   &normed[t * static_cast<size_t>(H)]);
    }
    std::copy(hidden.end() - H, hidden.end(), m->residuals.begin() + static_cast<size_t>(l) * H);
    gemm_rows(2, w.q, qw, H, normed.data(), n, q.data());
    gemm_rows(2, w.k, kvw, H, normed.data(), n, k.data());
    gemm_rows(2, w.v, kvw, H, normed.data(), n, v.data());
    for (int t = 0; t < n; ++t) {
      orc_rope_row(position + t, m->slots[l], c.head_dim, c.query_heads, c.kv_heads, c.epsilon,
                   m->turns[l].data(), w.q_norm, w.k_norm, &q[t * static_cast<size_t>(qw)],
                   &k[t * static_cast<size_t>(kvw)], &v[t * static_cast<size_t>(kvw)],
                   m->kcache[l].data(), m->vcache[l].data());
    }
#pragma omp parallel for schedule(dynamic)
    for (int t = 0; t < n; ++t) {
      orc_attention_row(position + t, m->windows[l], m->slots[l], c.head_dim, c.query_heads,
                        c.kv_heads, scale_log2e, &q[t * static_cast<size_t>(qw)],
                        m->kcache[l].data(), m->vcache[l].data(),
                        &attn[t * static_cast<size_t>(qw)]);
    }
    gemm_rows(2, w.o, H, qw, attn.data(), n, output.data());
    for (int t = 0; t < n; ++t) {
      orc_norm_row(w.ffn_norm, w.post_attn_norm, 1, 1, 1.0f, c.epsilon, H,
                   &hidden[t * static_cast<size_t>(H)], &output[t * static_cast<size_t>(H)],
                   &normed[t * static_cast<size_t>(H)]);
    }
    gemm_rows(2, w.gate, c.ffn, H, normed.data(), n, gate.data());
    gemm_rows(2, w.up, c.ffn, H, normed.data(), n, up.data());
    for (size_t i = 0; i < N * c.ffn; ++i) act[i] = orc_gelu_tanh(gate[i]) * up[i];
    for (int t = 0; t < n; ++t) {
      orc_edit_row(m->edits.data(), l, static_cast<uint32_t>(position + t), c.ffn,
                   &act[t * static_cast<size_t>(c.ffn)]);
    }
    gemm_rows(w.down_format, w.down, H, c.ffn, act.data(), n, output.data());
    pending = w.post_ffn_norm;
  }
  // The final norm and the head on the last row (Rows::LastToken).
  const size_t last = static_cast<size_t>(n - 1) * H;
  orc_norm_row(m->output_norm, pending, 1, 1, 1.0f, c.epsilon, H, &hidden[last], &output[last],
               m->normed.data());
  if (logits) orc_gemv_format(c.embedding_format, m->embedding, c.vocab, H, m->normed.data(), logits);
}

void orc_model_set_capture(orc_model* m, int on) {
  m->capture = on != 0;
  m->cap.assign(static_cast<size_t>(m->c.layers) * 8, {});
}

const uint32_t* orc_model_capture(const orc_model* m, int layer, int slot, int* words) {
  const std::vector<uint32_t>& v = m->cap[static_cast<size_t>(layer) * 8 + slot];
  *words = static_cast<int>(v.size());
  return v.data();
}

const float* orc_model_normed(const orc_model* m) { return m->normed.data(); }
const float* orc_model_residuals(const orc_model* m) { return m->residuals.data(); }
const uint16_t* orc_model_key_cache(const orc_model* m, int layer) {
  return m->kcache[layer].data();
}
const uint16_t* orc_model_value_cache(const orc_model* m, int layer) {
  return m->vcache[layer].data();
}
int orc_model_slots(const orc_model* m, int layer) { return m->slots[layer]; }

}  // extern "C"
