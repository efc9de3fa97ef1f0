// The step's chunk states for every row (a workgroup per chunk and row, a
// wave per query head over the chunk's rows staged once in LDS), and the
// fold of each row's chunk states in chunk order (attention.wgsl:403-438),
// which also serves the decode path when a row has more chunks than the O
// product's prologue folds.

#include "attention_rows.h"

namespace frz {
namespace {
using namespace attn;

// Row `row` of the step (attention.wgsl:95-438 for one query): its query
// heads were roped by the rope launch, and its own key and value appended,
// so every key it reads comes from the cache. The chunk's key and value rows
// go straight to LDS; wave w computes head w's chunk state.
__global__ __launch_bounds__(kThreads) void attention_prefill_kernel(
    const DevStep* __restrict__ step, AttentionArgs a) {
  __shared__ __align__(16) float q[QH * D];  // the row's queries, times scale * log2(e)
  __shared__ __align__(16) uint16_t keys[kChunkKeys * D];
  __shared__ __align__(16) uint16_t values[kChunkKeys * D];
  const int cs = blockIdx.x, row = blockIdx.y;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int tokens = (int)step->tokens;
  if (row >= tokens) return;
  // A variants step: every row at the step's position, over its own caches.
  const bool variants = step->variants != 0;
  const int p = (int)step->position + (variants ? 0 : row);
  const ChunkRange r = chunk_range(p, a.window, cs);
  if (cs >= r.count) return;
  const size_t cache_at = variants ? (size_t)row * a.cache_stride : 0;
  const float4 qv = ld4f(a.query + (size_t)row * a.q_stride + w * D + 4 * lane);
  const int valid = r.k_end - r.k_begin;
  rows::stage(a.key_cache + cache_at, a.value_cache + cache_at, a.slots, r.k_begin, valid, keys,
              values);
  const float sc = a.scale_log2e;
  *reinterpret_cast<float4*>(q + w * D + 4 * lane) =
      make_float4(qv.x * sc, qv.y * sc, qv.z * sc, qv.w * sc);
  __builtin_amdgcn_s_waitcnt(0x0F70);  // this wave's rows landed (vmcnt 0)
  __syncthreads();                     // every wave's rows and queries
  const size_t slot = ((size_t)row * a.max_chunks + cs) * QH + w;
  // The last row's scores, for the capture store: keys earliest .. p.
  float* scores = nullptr;
  if (a.store_scores && row == tokens - 1) {
    const int earliest = p + 1 - min(p + 1, a.keys);
    scores = a.store_scores + (size_t)w * a.keys + (r.k_begin - earliest);
  }
  rows::head_state(keys, values, q + w * D, -1, valid, r.k_begin, p, a.window,
                   a.stats + slot * 4, a.partials + slot * D, scores);
}

// ---- fold ------------------------------------------------------------------
// For one row (a decode token's global layers, many chunks): a workgroup
// folds its chunks for kFoldDims dimensions of one head. The
// chunk states are staged into LDS; the running maximum and liveness before
// each chunk come from a wave-wide prefix scan (a maximum and an or, exact
// in any order while no chunk maximum is NaN; with one, lane 0 replays the
// recursion itself); each chunk's factors (a, b) follow in parallel; then
// each dimension's chain o = o a + po b, and l's, run in chunk order. The
// chains read a chunk's (a, b, l term, liveness) as one record, 8 chunks at
// a time; the chunk count is padded to 8 with records (1, 0, 0, 0) and zero
// outputs, which leave o, l and liveness as they are (o and l are never -0,
// so adding 0 * 0 changes no bits).
constexpr int kFoldBatch = 8;  // staging loads a thread keeps in flight; chunks a chain step reads
// Chunk states staged in LDS at once: a row's chunks are folded in segments
// of this many, the running state carried between them, so any context folds.
constexpr int kFoldSegment = 224;

__host__ __device__ constexpr int fold_padded(int chunks) {
  return (chunks + kFoldBatch - 1) / kFoldBatch * kFoldBatch;
}

// Inclusive prefix maximum and or over the wave's 64 lanes: shifts within
// each 16-lane row, then row 0's and 2's last lanes into the next row, then
// lane 31 into rows 2 and 3 (DPP row_shr, row_bcast:15, row_bcast:31).
template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ int dpp_or_old(int old, int v) {
  return __builtin_amdgcn_update_dpp(old, v, CTRL, ROWS, 0xF, false);
}
__device__ __forceinline__ float wave_prefix_max(float v) {
  const int ninf = __builtin_bit_cast(int, -__builtin_inff());
  auto step = [&](int got) { v = __builtin_fmaxf(v, __builtin_bit_cast(float, got)); };
  step(dpp_or_old<0x111>(ninf, __builtin_bit_cast(int, v)));
  step(dpp_or_old<0x112>(ninf, __builtin_bit_cast(int, v)));
  step(dpp_or_old<0x114>(ninf, __builtin_bit_cast(int, v)));
  step(dpp_or_old<0x118>(ninf, __builtin_bit_cast(int, v)));
  step(dpp_or_old<0x142, 0xA>(ninf, __builtin_bit_cast(int, v)));
  step(dpp_or_old<0x143, 0xC>(ninf, __builtin_bit_cast(int, v)));
  return v;
}
__device__ __forceinline__ int wave_prefix_or(int v) {
  v |= dpp_or_old<0x111>(0, v);
  v |= dpp_or_old<0x112>(0, v);
  v |= dpp_or_old<0x114>(0, v);
  v |= dpp_or_old<0x118>(0, v);
  v |= dpp_or_old<0x142, 0xA>(0, v);
  v |= dpp_or_old<0x143, 0xC>(0, v);
  return v;
}

template <int kFoldDims>
__global__ __launch_bounds__(kThreads) void attention_fold_kernel(const DevStep* __restrict__ step,
                                                                  FoldArgs f) {
  constexpr int kFoldVec4s = kFoldDims / 4;  // vec4s of a chunk's output a workgroup stages
  extern __shared__ __align__(16) float fold_smem[];
  const int row = blockIdx.y;
  if (row >= (int)step->tokens) return;
  const int p = (int)step->position + (step->variants ? 0 : row);
  const int count = chunk_range(p, f.window, 0).count;
  const int cap = fold_padded(min(f.max_chunks, kFoldSegment));
  const int h = blockIdx.x / (D / kFoldDims), dim0 = (blockIdx.x % (D / kFoldDims)) * kFoldDims;
  const int t = threadIdx.x;
  float* po = fold_smem;                                       // [cap][64]
  float4* st = reinterpret_cast<float4*>(po + cap * kFoldDims);  // [cap] (m, l, live, 0)
  float4* rec = st + cap;                                      // [cap] (a, b, l, live)
  float* mb = reinterpret_cast<float*>(rec + cap);             // m before chunk c
  int* lb = reinterpret_cast<int*>(mb + cap);                  // live before chunk c
  const float* part = f.partials + (size_t)row * f.max_chunks * QH * D;
  const float* stats = f.stats + (size_t)row * f.max_chunks * QH * 4;
  // Carried from segment to segment: the scan's maximum and liveness before
  // the segment (wave 0), the serial replay's once a NaN maximum is seen
  // (lane 0), and each dimension's chains (threads below kFoldDims).
  bool carry_live = false, nan_seen = false, replay_live = false;
  float carry_m = 0.0f, replay_m = 0.0f;
  bool live = false;
  float l = 0.0f, o = 0.0f;
  int seg0 = 0;
  for (;;) {
    const int n = min(count - seg0, kFoldSegment);
    const int padded = fold_padded(n);
    // Stage: the segment's chunk states (one a thread: n <= 224), then vec4
    // i of the head's block, chunk seg0 + i / kFoldVec4s, dims
    // 4 (i % kFoldVec4s); the padding's outputs zero.
    float4 sv = make_float4(0.f, 0.f, 0.f, 0.f);
    if (t < n) sv = ld4f(stats + ((size_t)(seg0 + t) * QH + h) * 4);
    const int vec4s = n * (kFoldDims / 4);
    const float* seg_part = part + (size_t)seg0 * QH * D;
    for (int base = 0; base < vec4s; base += kFoldBatch * kThreads) {
      float4 v[kFoldBatch];
#pragma unroll
      for (int k = 0; k < kFoldBatch; ++k) {
        const int i = base + t + k * kThreads;
        if (i < vec4s)
          v[k] = ld4f(seg_part + ((size_t)(i / kFoldVec4s) * QH + h) * D + dim0 + 4 * (i % kFoldVec4s));
      }
#pragma unroll
      for (int k = 0; k < kFoldBatch; ++k) {
        const int i = base + t + k * kThreads;
        if (i < vec4s) reinterpret_cast<float4*>(po)[i] = v[k];
      }
    }
    for (int i = vec4s + t; i < padded * (kFoldDims / 4); i += kThreads)
      reinterpret_cast<float4*>(po)[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (t < n) st[t] = sv;
    __syncthreads();
    if (t < 64) {
      bool nan = false;
      for (int base = 0; base < n; base += 64) {
        const int c = base + t;
        const float4 s4 = c < n ? st[c] : make_float4(0.f, 0.f, 0.f, 0.f);
        const bool cl = c < n && s4.z != 0.0f;
        nan = nan || (cl && s4.x != s4.x);
        const float v = wave_prefix_max(cl ? s4.x : -__builtin_inff());
        const int lv = wave_prefix_or(cl ? 1 : 0);
        // Exclusive: lane c - 1's (lane 0: nothing before).
        const float ev = __builtin_bit_cast(
            float, dpp_or_old<0x138>(__builtin_bit_cast(int, -__builtin_inff()), __builtin_bit_cast(int, v)));
        const int el = dpp_or_old<0x138>(0, lv);
        if (c < n) {
          lb[c] = carry_live || el;
          mb[c] = carry_live ? (el ? __builtin_fmaxf(carry_m, ev) : carry_m) : ev;
        }
        const float last_v = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
        const int last_l = __builtin_amdgcn_readlane(lv, 63);
        carry_m = carry_live ? (last_l ? __builtin_fmaxf(carry_m, last_v) : carry_m) : last_v;
        carry_live = carry_live || last_l;
      }
      // Until a chunk maximum is NaN the scan is exact and the serial
      // recursion's state is the scan's; from then on lane 0 replays it.
      const bool replay = nan_seen || __any(nan);
      if (replay && t == 0) {
        for (int c = 0; c < n; ++c) {
          lb[c] = replay_live;
          mb[c] = replay_m;
          const Fold g = fold_factors(replay_live, replay_m, st[c].z != 0.0f, st[c].x);
          replay_m = g.m;
          replay_live = replay_live || st[c].z != 0.0f;
        }
      }
      nan_seen = replay;
      if (!replay) {
        replay_m = carry_m;
        replay_live = carry_live;
      }
    }
    __syncthreads();
    for (int c = t; c < padded; c += kThreads) {
      if (c < n) {
        const float4 s4 = st[c];
        const Fold g = fold_factors(lb[c] != 0, mb[c], s4.z != 0.0f, s4.x);
        rec[c] = make_float4(g.a, g.b, s4.y, s4.z);
      } else {
        rec[c] = make_float4(1.0f, 0.0f, 0.0f, 0.0f);
      }
    }
    __syncthreads();
    if (t < kFoldDims) {
      for (int base = 0; base < padded; base += kFoldBatch) {
        float4 r[kFoldBatch];
        float v[kFoldBatch];
#pragma unroll
        for (int k = 0; k < kFoldBatch; ++k) {
          r[k] = rec[base + k];
          v[k] = po[(base + k) * kFoldDims + t];
        }
#pragma unroll
        for (int k = 0; k < kFoldBatch; ++k) {
          l = l * r[k].x + r[k].z * r[k].y;
          o = o * r[k].x + v[k] * r[k].y;
          live = live || r[k].w != 0.0f;
        }
      }
    }
    if (seg0 + n >= count) break;
    seg0 += n;
    __syncthreads();  // every thread is done with this segment's staging
  }
  if (t < kFoldDims) {
    f.out[(size_t)row * QH * D + h * D + dim0 + t] = live ? o / l : 0.0f;
    // The last row's (m, l), for the capture store: m as the last chunk's
    // fold leaves it.
    const int c = count - 1 - seg0;
    if (f.store_stats && t == 0 && dim0 == 0 && row == (int)step->tokens - 1) {
      const Fold g = fold_factors(lb[c] != 0, mb[c], st[c].z != 0.0f, st[c].x);
      f.store_stats[2 * h] = g.m;
      f.store_stats[2 * h + 1] = l;
    }
  }
}

// A row's chunk states for head h folded in chunk order by one wave (lane l
// dimensions 4 l .. 4 l + 3), the recursion replayed as written:
// chunk c's factors (a, b) from the maximum and liveness before it
// (fold_factors), then l = l a + l_c b and o = o a + o_c b; the output is
// o / l, or 0 when no key was live (attention.wgsl:403-438). Steps of
// several rows fill the chip with their rows; each lane reads its chunks'
// states kRowBatch at a time (a 512-key window's 9 chunks in one batch).
constexpr int kRowBatch = 16;
__global__ __launch_bounds__(64) void attention_fold_rows_kernel(const DevStep* __restrict__ step,
                                                                 FoldArgs f) {
  const int row = blockIdx.x;
  const int tokens = (int)step->tokens;
  if (row >= tokens) return;
  const int p = (int)step->position + (step->variants ? 0 : row);
  const int count = chunk_range(p, f.window, 0).count;
  const int w = blockIdx.y, lane = threadIdx.x;
  const float* part = f.partials + (size_t)row * f.max_chunks * QH * D + w * D + 4 * lane;
  const float* stats = f.stats + (size_t)row * f.max_chunks * QH * 4 + w * 4;
  bool live = false;
  float m = 0.0f, l = 0.0f;
  float o[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int c0 = 0; c0 < count; c0 += kRowBatch) {
    float4 st[kRowBatch], po[kRowBatch];
#pragma unroll
    for (int k = 0; k < kRowBatch; ++k) {
      const int c = min(c0 + k, count - 1);
      st[k] = ld4f(stats + (size_t)c * QH * 4);
      po[k] = ld4f(part + (size_t)c * QH * D);
    }
#pragma unroll
    for (int k = 0; k < kRowBatch; ++k) {
      if (c0 + k < count) {
        const bool chunk_live = st[k].z != 0.0f;
        const Fold g = fold_factors(live, m, chunk_live, st[k].x);
        l = l * g.a + st[k].y * g.b;
        o[0] = o[0] * g.a + po[k].x * g.b;
        o[1] = o[1] * g.a + po[k].y * g.b;
        o[2] = o[2] * g.a + po[k].z * g.b;
        o[3] = o[3] * g.a + po[k].w * g.b;
        m = g.m;
        live = live || chunk_live;
      }
    }
  }
  float* out = f.out + (size_t)row * QH * D + w * D + 4 * lane;
  const float4 res = live ? make_float4(o[0] / l, o[1] / l, o[2] / l, o[3] / l)
                          : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  *reinterpret_cast<float4*>(out) = res;
  if (f.out_hi) {
    // The fast prefill mode's O product reads the row as bf16 pairs.
    const float v[4] = {res.x, res.y, res.z, res.w};
    store_pairs4(f.out_hi, f.out_lo, row, w * D + 4 * lane, QH * D, v);
  }
  // The last row's (m, l), for the capture store: m as the last chunk's
  // fold leaves it.
  if (f.store_stats && lane == 0 && row == tokens - 1) {
    f.store_stats[2 * w] = m;
    f.store_stats[2 * w + 1] = l;
  }
}

}  // namespace

template <int kFoldDims>
hipError_t launch_fold(hipStream_t s, const DevStep* step, const FoldArgs& f, int max_tokens) {
  // po, st, rec, mb, lb for the chunk count padded to a batch.
  const size_t lds =
      (size_t)fold_padded(min(f.max_chunks, kFoldSegment)) * (kFoldDims * 4 + 16 + 16 + 4 + 4);
  hipLaunchKernelGGL(attention_fold_kernel<kFoldDims>, dim3(QH * (D / kFoldDims), max_tokens),
                     dim3(kThreads), lds, s, step, f);
  return hipGetLastError();
}

hipError_t launch_attention_fold(hipStream_t s, const DevStep* step, const FoldArgs& f,
                                 int max_tokens) {
  if (f.max_chunks <= 0 || f.max_chunks > kMaxContextChunks) return hipErrorInvalidValue;
  // One row (a decode token's global layers): its chunks' factors by a
  // scan, its dimensions over many workgroups. Several rows: a wave a row
  // and head.
  if (max_tokens > 1) {
    hipLaunchKernelGGL(attention_fold_rows_kernel, dim3(max_tokens, QH), dim3(64), 0, s, step, f);
    return hipGetLastError();
  }
  return launch_fold<16>(s, step, f, max_tokens);
}

hipError_t launch_attention(hipStream_t s, const DevStep* step, const AttentionArgs& a,
                            int max_tokens) {
  if (a.head_dim != D || a.query_heads != QH || a.kv_heads != 1) return hipErrorInvalidValue;
  if (a.grid_chunks < 0 || a.grid_chunks > a.max_chunks) return hipErrorInvalidValue;
  const int chunks = a.grid_chunks > 0 ? a.grid_chunks : a.max_chunks;
  hipLaunchKernelGGL(attention_prefill_kernel, dim3(chunks, max_tokens), dim3(kThreads), 0, s, step,
                     a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return launch_attention_fold(
      s, step, FoldArgs{a.partials, a.stats, a.out, a.window, a.max_chunks, a.store_stats},
      max_tokens);
}

}  // namespace frz
