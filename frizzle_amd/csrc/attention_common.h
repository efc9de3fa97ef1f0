// Attention over the F16 KV cache in 64-key chunks fixed by position
// (attention.wgsl:95-438), for Gemma-3's shape: d = 256, 4 query heads on
// one key-value head. A chunk's state (m, l, O) is computed from empty over
// its 8-key tiles in order; a row's chunk states are folded in chunk order
// and O divided by l. The same bits come out whether a step's chunks run in
// one workgroup or many (the reference's split): every chunk starts empty and
// the fold is one sequential pass.
//
// A workgroup computes one head over one chunk. Within it the reference's
// tile recursion is kept exactly, but its independent parts run in
// parallel: each key's score is the chain s += dot(q_w, k_w) over the head's
// 64 vec4s, its 64 dots formed by the key's four lanes (16 each) and added in
// order by each of them, reading the others' through DPP; a tile's maximum
// is a max (order-free); each tile's running maximum, rescale factor and
// every exponential follow from those maxima; only the tile sums (8 ordered
// adds each), the running sum l over the tiles, and each output dimension's
// chain over the chunk's keys stay sequential.

#pragma once

#include "kernels.h"
#include "numerics.h"
#include "rope_common.h"

namespace frz {
namespace attn {

constexpr int D = 256;
constexpr int QH = 4;
constexpr int kThreads = 256;                             // one head over one chunk
constexpr int kTiles = kChunkKeys / kTileKeys;            // 8
constexpr int kKeyLanes = kThreads / kChunkKeys;          // 4 lanes a key
constexpr int kKeyLoads = D / kKeyLanes / 8;              // uint4s of its key row a lane holds
constexpr int kValueLoads = kChunkKeys * D / 8 / kThreads;  // uint4s of value rows a thread stages

struct ChunkShared {
  alignas(16) float q[D];              // the head's query, roped, times scale * log2(e)
  alignas(16) uint16_t v[kChunkKeys * D];  // value rows as stored
  alignas(16) uint16_t knew[D];        // the step's own key row, when the chunk holds it
  alignas(16) float e[kChunkKeys];     // weights
  alignas(16) float tile_top[kTiles];
  alignas(16) int tile_seen[kTiles];
  alignas(16) float tile_a[kTiles];
};

__device__ __forceinline__ float h2f(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

// -0 in a register the compiler does not see into. fma(x, h, -0) is the
// product x h rounded once, the sign of a zero product kept (x h + -0 is
// x h for every x h, zeros included), and with h a half it stays one mixed
// fma instead of a conversion and a multiply.
__device__ __forceinline__ float negative_zero() {
  float z;
  asm("v_mov_b32 %0, 0x80000000" : "=v"(z));
  return z;
}

// dot4 of q with the four halves of words w0 (low, high) and w1: each
// product rounded, added ((p0 + p1) + p2) + p3.
__device__ __forceinline__ float dot4_halves(float4 q, uint32_t w0, uint32_t w1, float nz) {
  const half2v a = __builtin_bit_cast(half2v, w0), b = __builtin_bit_cast(half2v, w1);
  const float p0 = __builtin_fmaf(q.x, (float)a.x, nz);
  const float p1 = __builtin_fmaf(q.y, (float)a.y, nz);
  const float p2 = __builtin_fmaf(q.z, (float)b.x, nz);
  const float p3 = __builtin_fmaf(q.w, (float)b.y, nz);
  return ((p0 + p1) + p2) + p3;
}

// Orders a wave's LDS accesses around it: a wave's LDS instructions execute
// in program order; this keeps the compiler from moving them.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

struct Fold {
  float a, b, m;
};
// attention.wgsl:135-151.
__device__ __forceinline__ Fold fold_factors(bool live, float m, bool chunk_live,
                                             float chunk_max) {
  if (!chunk_live) return {1.0f, 0.0f, m};
  if (!live) return {0.0f, 1.0f, chunk_max};
  if (m == chunk_max) return {1.0f, 1.0f, m};
  if (m > chunk_max) return {1.0f, exp2f_fixed(chunk_max - m), m};
  return {exp2f_fixed(m - chunk_max), 1.0f, chunk_max};
}

struct ChunkRange {
  int earliest, count, c, k_begin, k_end, n_tiles;
};
__device__ __forceinline__ ChunkRange chunk_range(int p, int window, int cs) {
  ChunkRange r;
  r.earliest = p + 1 > window ? p + 1 - window : 0;
  r.count = p / kChunkKeys - r.earliest / kChunkKeys + 1;
  r.c = r.earliest / kChunkKeys + cs;
  r.k_begin = max(r.c * kChunkKeys, r.earliest / kTileKeys * kTileKeys);
  r.k_end = min((r.c + 1) * kChunkKeys, p + 1);
  r.n_tiles = (r.k_end - r.k_begin + kTileKeys - 1) / kTileKeys;
  return r;
}

// The cache slot of the chunk's key k_begin + jj, from k_begin's slot `base`
// (slots is at least a chunk).
__device__ __forceinline__ int chunk_slot(int base, int jj, int slots) {
  const int s = base + jj;
  return s < slots ? s : s - slots;
}

// Loads are issued for every lane, whatever its row (rows at or past k_end
// and the row `own`, supplied later, read row k_begin instead), and nothing
// overwrites their registers until they are used: the code stays
// straight-line, and a wait for earlier loads does not wait for these.

// Lane t's part of a key row: key k_begin + t / 4, halves 64 (t % 4) .. +63.
// A row past k_end only feeds scores that are never used.
__device__ __forceinline__ void key_load(uint4 (&k)[kKeyLoads], const uint16_t* __restrict__ kc,
                                         int slots, const ChunkRange& r, int own) {
  const int jj = threadIdx.x >> 2, u = threadIdx.x & 3, j = r.k_begin + jj;
  const bool keep = jj < r.n_tiles * kTileKeys && j < r.k_end && j != own;
  const int base = r.k_begin % slots;
  const uint4* src = reinterpret_cast<const uint4*>(
      kc + (size_t)(keep ? chunk_slot(base, jj, slots) : base) * D + 64 * u);
#pragma unroll
  for (int m = 0; m < kKeyLoads; ++m) k[m] = src[m];
}

// Thread t's share of the value rows: uint4 i = t + 256 n of the chunk is
// row i / 32, halves 8 (i % 32) .. +7.
__device__ __forceinline__ void value_load(uint4 (&v)[kValueLoads], const uint16_t* __restrict__ vc,
                                           int slots, const ChunkRange& r, int own) {
  const int base = r.k_begin % slots;
#pragma unroll
  for (int n = 0; n < kValueLoads; ++n) {
    const int i = threadIdx.x + n * kThreads;
    const int jj = i / (D / 8), w8 = i % (D / 8), j = r.k_begin + jj;
    const bool keep = jj < r.n_tiles * kTileKeys && j < r.k_end && j != own;
    v[n] = *reinterpret_cast<const uint4*>(
        vc + (size_t)(keep ? chunk_slot(base, jj, slots) : base) * D + 8 * w8);
  }
}
// Stages the value rows into LDS: rows past k_end as zeros, every row but
// `own`.
__device__ __forceinline__ void value_store(ChunkShared& S, const uint4 (&v)[kValueLoads],
                                            const ChunkRange& r, int own) {
#pragma unroll
  for (int n = 0; n < kValueLoads; ++n) {
    const int i = threadIdx.x + n * kThreads;
    const int jj = i / (D / 8), w8 = i % (D / 8), j = r.k_begin + jj;
    if (jj < r.n_tiles * kTileKeys && j != own) {
      *reinterpret_cast<uint4*>(S.v + jj * D + 8 * w8) = j < r.k_end ? v[n] : make_uint4(0, 0, 0, 0);
    }
  }
}

// Lane (l + N) mod 16 of the calling lane l's 16-lane row (DPP row_ror).
template <int N>
__device__ __forceinline__ int row_rotate_int(int x) {
  return __builtin_amdgcn_mov_dpp(x, 0x120 + N, 0xF, 0xF, false);
}
template <int N>
__device__ __forceinline__ float row_rotate(float x) {
  return __builtin_bit_cast(float, row_rotate_int<N>(__builtin_bit_cast(int, x)));
}

// Lane l ^ 16 of the calling lane l's 32-lane group (ds_swizzle bit mode:
// and-mask 31, or-mask 0, xor-mask 16).
__device__ __forceinline__ int other_row(int x) {
  return __builtin_amdgcn_ds_swizzle(x, (16 << 10) | 31);
}

// Lane UU of the calling lane's quad.
template <int UU>
__device__ __forceinline__ float quad_lane(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), UU * 0x55,
                                                            0xF, 0xF, true));
}
template <int UU>
__device__ __forceinline__ float add_quad_dots(float s, const float (&d)[2 * kKeyLoads]) {
#pragma unroll
  for (int w = 0; w < 2 * kKeyLoads; ++w) s = s + quad_lane<UU>(d[w]);
  return s;
}

// The chunk's unnormalized output (D values) and (m, l, live, 0) for one
// head, from its staged query and values in S and each lane's key part in
// k (rows past k_end zeros). Every thread of the workgroup calls it. With
// `scores`, each live key j's score is also written at scores[j - earliest].
template <bool kQueryFirst = false>
__device__ __forceinline__ void chunk_state(ChunkShared& S, const uint4 (&k)[kKeyLoads], int p,
                                            int window, const ChunkRange& r,
                                            float* __restrict__ partial,
                                            float* __restrict__ stats,
                                            float* __restrict__ scores = nullptr,
                                            int earliest = 0) {
  const int t = threadIdx.x, jj = t >> 2, u = t & 3, j = r.k_begin + jj;
  const bool live = jj < r.n_tiles * kTileKeys && j < r.k_end && j <= p && j + window > p;
  // Dimension t of every staged value row, read now so the reads complete
  // under the scores and the softmax and the output chain finds them in
  // registers (rows past the chunk's tiles read as staged; their weight is 0).
  // With kQueryFirst (a latency-bound launch of few workgroups) the 64 query
  // values the lane's dots take are read before them: LDS reads complete in
  // order, so the dots then do not wait for the 64 value reads. It costs 16
  // registers, which a launch of many workgroups pays in occupancy.
  float4 qv[2 * kKeyLoads];
  if constexpr (kQueryFirst) {
#pragma unroll
    for (int m = 0; m < kKeyLoads; ++m) {
      qv[2 * m] = ld4f(S.q + 64 * u + 8 * m);
      qv[2 * m + 1] = ld4f(S.q + 64 * u + 8 * m + 4);
    }
    __asm__ volatile("" ::: "memory");
  }
  uint16_t vt[kChunkKeys];
#pragma unroll
  for (int key = 0; key < kChunkKeys; ++key) vt[key] = S.v[key * D + t];
  // Scores (attention.wgsl:277-297).
  float d[2 * kKeyLoads];
#pragma unroll
  for (int m = 0; m < kKeyLoads; ++m) {
    const float4 qa = kQueryFirst ? qv[2 * m] : ld4f(S.q + 64 * u + 8 * m);
    const float4 qb = kQueryFirst ? qv[2 * m + 1] : ld4f(S.q + 64 * u + 8 * m + 4);
    const uint4 w = k[m];
    d[2 * m] = dot4(qa.x, qa.y, qa.z, qa.w, h2f(w.x & 0xFFFFu), h2f(w.x >> 16),
                    h2f(w.y & 0xFFFFu), h2f(w.y >> 16));
    d[2 * m + 1] = dot4(qb.x, qb.y, qb.z, qb.w, h2f(w.z & 0xFFFFu), h2f(w.z >> 16),
                        h2f(w.w & 0xFFFFu), h2f(w.w >> 16));
  }
  float s = 0.0f;
  s = add_quad_dots<0>(s, d);
  s = add_quad_dots<1>(s, d);
  s = add_quad_dots<2>(s, d);
  s = add_quad_dots<3>(s, d);
  if (scores && live && u == 0) scores[j - earliest] = s;
  // A tile is 8 keys, 32 lanes: two DPP rows of 4 keys. Its maximum and
  // whether any key is live, in every lane: within a row by rotations, then
  // across the two rows by a swizzle (xor 16); a max is order-free.
  float top = live ? s : -__builtin_inff();
  int seen = live ? 1 : 0;
  top = __builtin_fmaxf(top, row_rotate<4>(top));
  seen |= row_rotate_int<4>(seen);
  top = __builtin_fmaxf(top, row_rotate<8>(top));
  seen |= row_rotate_int<8>(seen);
  top = __builtin_fmaxf(top, __builtin_bit_cast(float, other_row(__builtin_bit_cast(int, top))));
  seen |= other_row(seen);
  if ((t & 31) == 0) {
    S.tile_top[jj >> 3] = top;
    S.tile_seen[jj >> 3] = seen;
  }
  __syncthreads();
  // Each tile's running maximum and rescale factor, and each weight
  // (attention.wgsl:304-340), from all tiles' maxima read at once.
  float tops[kTiles];
  int seens[kTiles];
#pragma unroll
  for (int q4 = 0; q4 < kTiles / 4; ++q4) {
    const float4 tv = ld4f(S.tile_top + 4 * q4);
    const int4 sv = *reinterpret_cast<const int4*>(S.tile_seen + 4 * q4);
    tops[4 * q4] = tv.x; tops[4 * q4 + 1] = tv.y; tops[4 * q4 + 2] = tv.z; tops[4 * q4 + 3] = tv.w;
    seens[4 * q4] = sv.x; seens[4 * q4 + 1] = sv.y; seens[4 * q4 + 2] = sv.z; seens[4 * q4 + 3] = sv.w;
  }
  const int tile = jj >> 3;
  bool chunk_live = false;
  float cm = 0.0f, my_old = 0.0f, my_top = 0.0f;
#pragma unroll
  for (int tt = 0; tt < kTiles; ++tt) {
    if (tt < r.n_tiles && seens[tt]) {
      const float top_tile = tops[tt];
      const float old = chunk_live ? cm : top_tile;
      chunk_live = true;
      const float next = __builtin_fmaxf(old, top_tile);
      if (tt == tile) {
        my_old = old;
        my_top = next;
      }
      cm = next;
    }
  }
  // The weight by lane 0 of the key, the tile's factor by lane 1 of its
  // first key: the two exponentials run side by side.
  if (u == 0) S.e[jj] = live ? exp2f_fixed(s - my_top) : 0.0f;
  if (u == 1 && (jj & 7) == 0 && tile < r.n_tiles) {
    S.tile_a[tile] = (seens[tile] != 0 && my_old != my_top) ? exp2f_fixed(my_old - my_top) : 1.0f;
  }
  __syncthreads();
  // Each tile's weights summed in order, then l = l a + sum over the seen
  // tiles in order (wave 0).
  if (t < 64) {
    float sum = 0.0f;
    if (t < kTiles) {
#pragma unroll
      for (int b = 0; b < kTileKeys; ++b) sum += S.e[t * kTileKeys + b];
    }
    float sums[kTiles], as[kTiles];
#pragma unroll
    for (int tt = 0; tt < kTiles; ++tt) {
      sums[tt] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sum), tt));
    }
#pragma unroll
    for (int q4 = 0; q4 < kTiles / 4; ++q4) {
      const float4 av = ld4f(S.tile_a + 4 * q4);
      as[4 * q4] = av.x; as[4 * q4 + 1] = av.y; as[4 * q4 + 2] = av.z; as[4 * q4 + 3] = av.w;
    }
    if (t == 0) {
      float cl = 0.0f;
#pragma unroll
      for (int tt = 0; tt < kTiles; ++tt) {
        if (tt < r.n_tiles && seens[tt]) cl = cl * as[tt] + sums[tt];
      }
      *reinterpret_cast<float4*>(stats) = make_float4(cm, cl, chunk_live ? 1.0f : 0.0f, 0.0f);
    }
  }
  // O = O a + sum_b e_b v_b per tile: thread t is dimension t.
  float o = 0.0f;
#pragma unroll
  for (int tt = 0; tt < kTiles; ++tt) {
    if (tt < r.n_tiles) {
      o = o * S.tile_a[tt];
      const float4 ea = ld4f(S.e + tt * kTileKeys), eb = ld4f(S.e + tt * kTileKeys + 4);
      const float e[kTileKeys] = {ea.x, ea.y, ea.z, ea.w, eb.x, eb.y, eb.z, eb.w};
#pragma unroll
      for (int b = 0; b < kTileKeys; ++b) o = o + e[b] * h2f(vt[tt * kTileKeys + b]);
    }
  }
  partial[t] = o;
}

}  // namespace attn
}  // namespace frz
