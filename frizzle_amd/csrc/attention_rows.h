// Attention over one chunk with the chunk's key and value rows staged once in
// LDS for all four query heads (one key-value head): a wave per head, a lane
// per key for the scores and the weights, four output dimensions a lane for
// the value sums. The chunk state (m, l, O) of each head has the bits of the
// one-head kernels': each key's score is the chain s += dot(q_w, k_w) over
// the head's 64 vec4s in order, the tile maxima, running maxima and rescale
// factors follow the reference's recursion (attention.wgsl:277-340), and each
// output dimension's chain runs over the chunk's keys in order.
//
// Also the cache-reading helpers shared by the decode and row kernels.

#pragma once

#include "attention_common.h"

namespace frz {
namespace attn {

// Key and value rows are read through buffer resources over the cache: a
// row not taken from the cache (past the chunk's end, or the step's own) is
// read at an offset past the resource's end, which the hardware's range
// check returns as zeros. Such keys are never live, and such values stage
// as the zero rows the reference stages past the end.
constexpr int kPastEnd = 0x40000000;
constexpr int kBufferWord3 = 0x00020000;  // raw (untyped) 32-bit data

__device__ __forceinline__ __amdgpu_buffer_rsrc_t cache_resource(const uint16_t* cache,
                                                                 int slots) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(cache), 0, slots * D * 2,
                                           kBufferWord3);
}

// x mod slots for 0 <= x < 2^24: the float quotient is within 1 of the
// true one there (the reciprocal's error is under 2^-22 relative), so one
// correction each way ends exact.
__device__ __forceinline__ int ring_slot(int x, int slots) {
  const int q = (int)((float)x * __builtin_amdgcn_rcpf((float)slots));
  int r = x - q * slots;
  r = r < 0 ? r + slots : r;
  return r >= slots ? r - slots : r;
}

__device__ __forceinline__ float2 ld2f(const float* p) {
  return *reinterpret_cast<const float2*>(p);
}

// The maximum over each 8-lane group: lanes xor 1, xor 2 (quad
// permutations), then the mirrored lane of the 8 (DPP row_half_mirror); the
// order of a maximum's operands does not change it.
__device__ __forceinline__ float max8(float x) {
  x = __builtin_fmaxf(x, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(
                                                       __builtin_bit_cast(int, x), 0xB1, 0xF, 0xF, true)));
  x = __builtin_fmaxf(x, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(
                                                       __builtin_bit_cast(int, x), 0x4E, 0xF, 0xF, true)));
  x = __builtin_fmaxf(x, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(
                                                       __builtin_bit_cast(int, x), 0x141, 0xF, 0xF, true)));
  return x;
}

// DPP with control kCtrl over the rows in kRows; lanes it does not write
// (rows left out, or no source lane) get `fill`.
template <int kCtrl, int kRows>
__device__ __forceinline__ float dpp_or(float x, float fill) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                       __builtin_bit_cast(int, fill), __builtin_bit_cast(int, x),
                                       kCtrl, kRows, 0xF, false));
}

// exp2f_fixed's value, as selects instead of branches.
__device__ __forceinline__ float exp2_select(float x) {
  const float xc = x > 127.0f ? 127.0f : x;
  const float k = rint_(xc);
  const float r = xc - k;
  float p = 1.525273380405984e-05f;
  p = fmaf_(p, r, 1.5403530393381608e-04f);
  p = fmaf_(p, r, 1.3333558146428443e-03f);
  p = fmaf_(p, r, 9.618129107628477e-03f);
  p = fmaf_(p, r, 5.550410866482158e-02f);
  p = fmaf_(p, r, 2.402265069591007e-01f);
  p = fmaf_(p, r, 6.931471805599453e-01f);
  p = fmaf_(p, r, 1.0f);
  const float v = p * bits_to_float((uint32_t)((int)k + 127) << 23);
  return x < -125.5f ? 0.0f : v;
}

__device__ __forceinline__ float lane_value(float x, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), lane));
}

namespace rows {
constexpr int kRowBytes = D * 2;            // an F16 row
constexpr int kGranules = kRowBytes / 16;   // its 16-byte granules
typedef __attribute__((address_space(3))) void* LdsPtr;

__device__ __forceinline__ void load_to_lds(__amdgpu_buffer_rsrc_t r, void* lds, int voffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (LdsPtr)lds, 16, voffset, 0, 0, 0);
}

// Requests the chunk's first `cached` rows from k_begin's slot on, straight
// to LDS (a workgroup of 4 waves): key row r's granule g at r * kRowBytes +
// 16 (g ^ (r % 32)), so that the lanes' reads of one granule fall in
// distinct banks; value rows plain. Instruction i writes rows 2 i and
// 2 i + 1, lane l row 2 i + l / 32's granule l % 32; each wave issues 8 for
// keys and 8 for values. Rows at or past `cached` land as zeros. The caller
// waits (vmcnt 0) and synchronizes before reading them.
__device__ __forceinline__ void stage(const uint16_t* key_cache, const uint16_t* value_cache,
                                      int slots, int k_begin, int cached, uint16_t* keys,
                                      uint16_t* values) {
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int base = ring_slot(k_begin, slots);
  const __amdgpu_buffer_rsrc_t kres = cache_resource(key_cache, slots);
  const __amdgpu_buffer_rsrc_t vres = cache_resource(value_cache, slots);
  int at[8];
#pragma unroll
  for (int n = 0; n < 8; ++n) {
    const int rr = 2 * (8 * w + n) + (lane >> 5);
    int slot = base + rr;
    slot = slot >= slots ? slot - slots : slot;
    at[n] = rr < cached ? slot * kRowBytes : kPastEnd;
  }
#pragma unroll
  for (int n = 0; n < 8; ++n) {
    const int i = 8 * w + n, rr = 2 * i + (lane >> 5);
    load_to_lds(kres, reinterpret_cast<char*>(keys) + 1024 * i, at[n] + 16 * ((lane & 31) ^ (rr & 31)));
  }
#pragma unroll
  for (int n = 0; n < 8; ++n) {
    const int i = 8 * w + n;
    load_to_lds(vres, reinterpret_cast<char*>(values) + 1024 * i, at[n] + 16 * (lane & 31));
  }
}

// One head's chunk state, by one wave (lane = key of the chunk): q is the
// head's query in LDS (roped, times scale * log2(e)); keys and values are
// the staged rows, with the key and value of chunk key `own` (or none, -1)
// in row kChunkKeys instead. The chunk's keys are k_begin .. k_begin +
// valid - 1; key j is live when j + window > p. Writes (m, l, live, 0) to
// stats[0..3] and the unnormalized output to partial[0..D-1]; with
// `scores`, each live key's score (log2 units) at scores[lane].
__device__ __forceinline__ void head_state(const uint16_t* keys, const uint16_t* values,
                                           const float* q, int own, int valid, int k_begin, int p,
                                           int window, float* __restrict__ stats,
                                           float* __restrict__ partial,
                                           float* __restrict__ scores) {
  const int lane = threadIdx.x & 63;
  // Key `lane`'s score (attention.wgsl:277-297): s = sum over vec4s j in
  // order of dot(q_j, k_j).
  const float nz = negative_zero();
  const int krow = lane == own ? kChunkKeys : lane;
  const char* kline = reinterpret_cast<const char*>(keys) + krow * kRowBytes;
  // Eight granules' reads at a time, then their dots.
  float sl = 0.0f;
#pragma unroll
  for (int g8 = 0; g8 < kGranules; g8 += 8) {
    uint4 kk[8];
    float4 qq[16];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int gi = g8 + i;
      kk[i] = *reinterpret_cast<const uint4*>(kline + 16 * (gi ^ (krow & 31)));
      qq[2 * i] = ld4f(q + 8 * gi);
      qq[2 * i + 1] = ld4f(q + 8 * gi + 4);
    }
    __builtin_amdgcn_sched_barrier(0);
    float dd[16];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      dd[2 * i] = dot4_halves(qq[2 * i], kk[i].x, kk[i].y, nz);
      dd[2 * i + 1] = dot4_halves(qq[2 * i + 1], kk[i].z, kk[i].w, nz);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) sl = sl + dd[i];
  }
  // The weights, tile factors and l (attention.wgsl:304-340): tile maxima by
  // DPP within each 8 lanes, running maxima across the tiles, each weight
  // against its tile's running maximum, the factor between consecutive
  // running maxima, the tile sums in order, and l over the seen tiles.
  const bool live = lane < valid && k_begin + lane + window > p;
  if (scores && live) scores[lane] = sl;
  const uint64_t live_bits = __ballot(live);
  const int tile = lane >> 3;
  uint64_t any = live_bits | (live_bits >> 4);
  any |= any >> 2;
  any |= any >> 1;
  const uint32_t seen_tiles =
      (uint32_t)(((any & 0x0101010101010101ull) * 0x0102040810204080ull) >> 56);
  const bool tile_seen = (seen_tiles >> tile) & 1u;
  const bool seen_before = (seen_tiles & ((1u << tile) - 1u)) != 0;
  const float none = __builtin_bit_cast(float, 0x7FC00000u);
  const float top = max8(live ? sl : none);
  float run = tile_seen ? top : none;
  run = __builtin_fmaxf(run, dpp_or<0x118, 0xF>(run, none));
  run = __builtin_fmaxf(run, dpp_or<0x142, 0xA>(run, none));
  run = __builtin_fmaxf(run, dpp_or<0x143, 0xC>(run, none));
  const float back8 = dpp_or<0x118, 0xF>(run, none), back_row = dpp_or<0x142, 0xE>(run, none);
  __asm__ volatile("" ::"v"(back8), "v"(back_row));
  const float prev = (lane & 8) ? back8 : back_row;
  const float my_top = run;
  const float my_old = seen_before ? prev : top;
  const bool chunk_live = seen_tiles != 0;
  const float cm = chunk_live ? lane_value(run, 63) : 0.0f;
  const float e = exp2_select(live ? sl - my_top : -200.0f);
  const float fa = exp2_select(tile_seen && my_old != my_top ? my_old - my_top : 0.0f);
  float tsum = 0.0f;
  tsum = tsum + e;
  tsum = tsum + row_shl<1>(e);
  tsum = tsum + row_shl<2>(e);
  tsum = tsum + row_shl<3>(e);
  tsum = tsum + row_shl<4>(e);
  tsum = tsum + row_shl<5>(e);
  tsum = tsum + row_shl<6>(e);
  tsum = tsum + row_shl<7>(e);
  float cl = 0.0f;
#pragma unroll
  for (int tt = 0; tt < kTiles; ++tt) {
    const float next = cl * lane_value(fa, 8 * tt) + lane_value(tsum, 8 * tt);
    cl = (seen_tiles >> tt) & 1u ? next : cl;
  }
  if (lane == 0) {
    *reinterpret_cast<float4*>(stats) = make_float4(cm, cl, chunk_live ? 1.0f : 0.0f, 0.0f);
  }
  // Output dimensions 4 lane .. 4 lane + 3: o = o a + sum_b e_b v_b per tile
  // over all 8 tiles (keys past the chunk's end have zero weights and rows).
  float o[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int tt = 0; tt < kTiles; ++tt) {
    // The tile's eight value rows read at once.
    uint2 hvs[kTileKeys];
#pragma unroll
    for (int b = 0; b < kTileKeys; ++b) {
      const int key = tt * kTileKeys + b;
      const int vrow = key == own ? kChunkKeys : key;
      hvs[b] = *reinterpret_cast<const uint2*>(values + vrow * D + 4 * lane);
    }
    const float at = lane_value(fa, 8 * tt);
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = o[j] * at;
#pragma unroll
    for (int b = 0; b < kTileKeys; ++b) {
      const int key = tt * kTileKeys + b;
      const float ek = lane_value(e, key);
      const uint2 hv = hvs[b];
      const _Float16 h[4] = {__builtin_bit_cast(_Float16, (uint16_t)(hv.x & 0xFFFFu)),
                             __builtin_bit_cast(_Float16, (uint16_t)(hv.x >> 16)),
                             __builtin_bit_cast(_Float16, (uint16_t)(hv.y & 0xFFFFu)),
                             __builtin_bit_cast(_Float16, (uint16_t)(hv.y >> 16))};
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = o[j] + __builtin_fmaf(ek, (float)h[j], nz);
    }
  }
  *reinterpret_cast<float4*>(partial + 4 * lane) = make_float4(o[0], o[1], o[2], o[3]);
}
}  // namespace rows

}  // namespace attn
}  // namespace frz
