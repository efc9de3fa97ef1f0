// Attention over the F16 KV cache in 64-key chunks fixed by position
// (attention.wgsl:95-438), for Gemma-3's shape: d = 256, 4 query heads on
// one key-value head. A chunk's state (m, l, O) is computed from empty over
// its 8-key tiles in order; a row's chunk states are folded in chunk order
// and O divided by l. The same bits come out whether a step's chunks run in
// one workgroup or many (the reference's split): every chunk starts empty and
// the fold is one sequential pass.
//
// Within a chunk the reference's tile recursion is kept exactly, but its
// independent parts run in parallel: each key's score is one lane's chain of
// vec4 dots; a tile's maximum is a max (order-free); each tile's running
// maximum, rescale factor and every exponential follow from those maxima;
// only the tile sums (8 ordered adds each), the running sum l over the
// tiles, and each output dimension's chain over the chunk's keys stay
// sequential.
//
// Decode (one token): the kernel also does that token's QK-norm, rope and
// KV append (rope.wgsl) - only the chunk holding the token's own position
// needs its key and value, and that workgroup computes and stores them - and
// the workgroup that finishes last folds the chunks. The chunk results it
// reads are published with agent-coherent stores (written through to the
// device's coherence point) before a relaxed arrival count, and read back
// with agent-coherent loads, so no cache-wide writeback or invalidate runs.

#pragma once

#include "kernels.h"
#include "numerics.h"
#include "rope_common.h"

namespace frz {
namespace attn {

constexpr int D = 256;
constexpr int QH = 4;
constexpr int kThreads = 1024;
constexpr int kTiles = kChunkKeys / kTileKeys;  // 8
constexpr int kKStride = 260;                   // floats a staged key row, padded
constexpr int kStageLoads = kChunkKeys * (D / 8) / kThreads;  // uint4s a thread stages

struct ChunkShared {
  float q[QH * D];                    // queries, roped and scaled by scale * log2(e)
  float k[kChunkKeys * kKStride];     // keys, converted from F16 (exact)
  uint16_t v[kChunkKeys * D];         // values as stored
  float e[QH * kChunkKeys];           // weights
  float tile_top[QH * kTiles];
  int tile_seen[QH * kTiles];
  float tile_a[QH * kTiles];
  float tile_sum[QH * kTiles];
  float stats[QH * 4];                // m, l, live
};

__device__ __forceinline__ float h2f(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

template <bool COHERENT>
__device__ __forceinline__ void put(float* p, float v) {
  if (COHERENT) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else {
    *p = v;
  }
}
template <bool COHERENT>
__device__ __forceinline__ float get(const float* p) {
  if (COHERENT) return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
  return *p;
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

// A thread's share of the chunk's key and value rows, loaded from the cache
// into registers (so the loads can run while other work proceeds): uint4 i
// of the chunk is row i / 32, halves 8 (i % 32) .. +7; rows at or past
// k_end, and the row `own` (supplied later), load nothing.
struct StageRegs {
  uint4 k[kStageLoads], v[kStageLoads];
};
__device__ __forceinline__ void stage_load(StageRegs& R, const uint16_t* __restrict__ kc,
                                           const uint16_t* __restrict__ vc, int slots,
                                           const ChunkRange& r, int own) {
#pragma unroll
  for (int u = 0; u < kStageLoads; ++u) {
    const int i = threadIdx.x + u * kThreads;
    const int jj = i / (D / 8), w8 = i % (D / 8);
    const int j = r.k_begin + jj;
    R.k[u] = make_uint4(0, 0, 0, 0);
    R.v[u] = R.k[u];
    if (jj < r.n_tiles * kTileKeys && j < r.k_end && j != own) {
      const size_t at = (size_t)(j % slots) * D + 8 * w8;
      R.k[u] = *reinterpret_cast<const uint4*>(kc + at);
      R.v[u] = *reinterpret_cast<const uint4*>(vc + at);
    }
  }
}
// One uint4 of a key row and one of its value row into LDS, keys as f32.
__device__ __forceinline__ void stage_put(ChunkShared& S, int jj, int w8, uint4 kw, uint4 vw) {
  float* kd = S.k + jj * kKStride + 8 * w8;
  *reinterpret_cast<float4*>(kd) = make_float4(h2f(kw.x & 0xFFFFu), h2f(kw.x >> 16),
                                               h2f(kw.y & 0xFFFFu), h2f(kw.y >> 16));
  *reinterpret_cast<float4*>(kd + 4) = make_float4(h2f(kw.z & 0xFFFFu), h2f(kw.z >> 16),
                                                   h2f(kw.w & 0xFFFFu), h2f(kw.w >> 16));
  *reinterpret_cast<uint4*>(S.v + jj * D + 8 * w8) = vw;
}
// Writes the staged rows into LDS, every row but `own`.
__device__ __forceinline__ void stage_store(ChunkShared& S, const StageRegs& R,
                                            const ChunkRange& r, int own) {
#pragma unroll
  for (int u = 0; u < kStageLoads; ++u) {
    const int i = threadIdx.x + u * kThreads;
    const int jj = i / (D / 8), w8 = i % (D / 8);
    if (jj < r.n_tiles * kTileKeys && r.k_begin + jj != own) stage_put(S, jj, w8, R.k[u], R.v[u]);
  }
}

// The chunk's unnormalized output and (m, l, live), from the staged queries
// and key/value rows [k_begin, k_begin + 8 n_tiles) of S (rows past k_end
// staged as zeros). Every thread of the workgroup calls it.
template <bool COHERENT>
__device__ void chunk_state(ChunkShared& S, int p, int window, const ChunkRange& r,
                            float* __restrict__ partial, float* __restrict__ stats) {
  const int t = threadIdx.x;
  const int span = r.n_tiles * kTileKeys;
  float s = 0.0f;
  bool live = false;
  // Scores: wave h is head h, lane jj key k_begin + jj (attention.wgsl:277-297).
  if (t < QH * kChunkKeys) {
    const int h = t >> 6, jj = t & 63, j = r.k_begin + jj;
    live = jj < span && j < r.k_end && j <= p && j + window > p;
    if (live) {
      const float* q = S.q + h * D;
      const float* kr = S.k + jj * kKStride;
#pragma unroll 8
      for (int w = 0; w < D / 4; ++w) {
        const float4 q4 = *reinterpret_cast<const float4*>(q + 4 * w);
        const float4 k4 = *reinterpret_cast<const float4*>(kr + 4 * w);
        s += dot4(q4.x, q4.y, q4.z, q4.w, k4.x, k4.y, k4.z, k4.w);
      }
    }
    float m = live ? s : -__builtin_inff();
    int seen = live ? 1 : 0;
#pragma unroll
    for (int off = 1; off < kTileKeys; off <<= 1) {
      m = __builtin_fmaxf(m, __shfl_xor(m, off, 64));
      seen |= __shfl_xor(seen, off, 64);
    }
    if ((jj & 7) == 0) {
      S.tile_top[h * kTiles + (jj >> 3)] = m;
      S.tile_seen[h * kTiles + (jj >> 3)] = seen;
    }
  }
  __syncthreads();
  // Each tile's running maximum and rescale factor, and each weight
  // (attention.wgsl:304-340).
  if (t < QH * kChunkKeys) {
    const int h = t >> 6, jj = t & 63, tile = jj >> 3;
    bool chunk_live = false;
    float cm = 0.0f, my_old = 0.0f, my_top = 0.0f;
    for (int tt = 0; tt < r.n_tiles; ++tt) {
      if (S.tile_seen[h * kTiles + tt]) {
        const float top_tile = S.tile_top[h * kTiles + tt];
        const float old = chunk_live ? cm : top_tile;
        chunk_live = true;
        const float top = __builtin_fmaxf(old, top_tile);
        if (tt == tile) {
          my_old = old;
          my_top = top;
        }
        cm = top;
      }
    }
    S.e[h * kChunkKeys + jj] = live ? exp2f_fixed(s - my_top) : 0.0f;
    if ((jj & 7) == 0 && tile < r.n_tiles) {
      const bool seen = S.tile_seen[h * kTiles + tile] != 0;
      S.tile_a[h * kTiles + tile] =
          (seen && my_old != my_top) ? exp2f_fixed(my_old - my_top) : 1.0f;
    }
    if (jj == 0) {
      S.stats[h * 4 + 0] = cm;
      S.stats[h * 4 + 2] = chunk_live ? 1.0f : 0.0f;
      S.stats[h * 4 + 3] = 0.0f;
    }
  }
  __syncthreads();
  // Each tile's weights summed in order, one lane a (head, tile).
  if (t < QH * kTiles) {
    const int h = t >> 3, tt = t & 7;
    float sum = 0.0f;
    for (int b = 0; b < kTileKeys; ++b) sum += S.e[h * kChunkKeys + tt * kTileKeys + b];
    S.tile_sum[t] = sum;
  }
  __syncthreads();
  // l = l * a + sum over the seen tiles in order.
  if (t < QH) {
    float cl = 0.0f;
    for (int tt = 0; tt < r.n_tiles; ++tt) {
      if (S.tile_seen[t * kTiles + tt]) cl = cl * S.tile_a[t * kTiles + tt] + S.tile_sum[t * kTiles + tt];
    }
    S.stats[t * 4 + 1] = cl;
  }
  // O = O * a + sum_b e_b v_b per tile: lane (head, dimension).
  {
    const int h = t >> 8, i = t & 255;
    float o = 0.0f;
    for (int tt = 0; tt < r.n_tiles; ++tt) {
      o = o * S.tile_a[h * kTiles + tt];
#pragma unroll
      for (int b = 0; b < kTileKeys; ++b) {
        const int jj = tt * kTileKeys + b;
        o = o + S.e[h * kChunkKeys + jj] * h2f(S.v[jj * D + i]);
      }
    }
    put<COHERENT>(partial + h * D + i, o);
  }
  __syncthreads();
  if (t < QH * 4) put<COHERENT>(stats + t, S.stats[t]);
}

// The row's chunk states folded in chunk order, then o / l
// (attention.wgsl:403-438). Thread (head, dimension); loads run ahead.
template <bool COHERENT>
__device__ __forceinline__ float fold_chunks(const float* __restrict__ partials,
                                             const float* __restrict__ stats, int count) {
  const int h = threadIdx.x >> 8, i = threadIdx.x & 255;
  bool live = false;
  float m = 0.0f, l = 0.0f, o = 0.0f;
  constexpr int kBatch = 8;
  for (int c0 = 0; c0 < count; c0 += kBatch) {
    float sm[kBatch], sl[kBatch], sv[kBatch], po[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      if (c0 + u < count) {
        const float* st = stats + ((size_t)(c0 + u) * QH + h) * 4;
        sm[u] = get<COHERENT>(st);
        sl[u] = get<COHERENT>(st + 1);
        sv[u] = get<COHERENT>(st + 2);
        po[u] = get<COHERENT>(partials + ((size_t)(c0 + u) * QH + h) * D + i);
      }
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      if (c0 + u < count) {
        const bool chunk_live = sv[u] != 0.0f;
        const Fold f = fold_factors(live, m, chunk_live, sm[u]);
        l = l * f.a + sl[u] * f.b;
        o = o * f.a + po[u] * f.b;
        m = f.m;
        live = live || chunk_live;
      }
    }
  }
  return live ? o / l : 0.0f;
}

}  // namespace attn
}  // namespace frz
