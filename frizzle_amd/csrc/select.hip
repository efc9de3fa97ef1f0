// The output block's selection and draw: top-64 of the logits in the
// reference's total order (topk.wgsl), the draw over the candidates
// (draw.wgsl), and the fed step's advance of the step parameters.

#include "kernels.h"
#include "numerics.h"

namespace frz {
namespace {

// Entries are ordered by the order-preserving key of their bits (larger
// first) and, on equal keys, by the lower token (topk.wgsl:57-61); packed as
// key << 32 | ~token, that order is the descending order of one 64-bit
// integer. Slots past the input, and padding (token 0xFFFFFFFF), pack to 0
// and sort last (topk.wgsl:138-166). The top 64 are found by sorted lists
// of 64 held one entry a lane: a wave sorts 64 entries with a bitonic
// network over its lanes, and merges two sorted lists into the top 64 of
// both (the larger half of a bitonic merge), all through lane shuffles.
constexpr int kTileThreads = kSelectionTile / 4;  // four entries a thread
constexpr int kMergeWaves = 4;                    // lists merged by a workgroup: 4 waves x 4
constexpr int kListsPerMerge = 16;

__device__ __forceinline__ uint64_t pack_entry(uint32_t bits, uint32_t id) {
  return id == 0xFFFFFFFFu ? 0ull : ((uint64_t)topk_key(bits) << 32) | (uint32_t)~id;
}

__device__ __forceinline__ uint64_t shfl64(uint64_t v, int src) {
  const uint32_t lo = (uint32_t)__shfl((int)(uint32_t)v, src, 64);
  const uint32_t hi = (uint32_t)__shfl((int)(uint32_t)(v >> 32), src, 64);
  return ((uint64_t)hi << 32) | lo;
}

// Lane l ^ mask's word: masks 1 and 2 by DPP quad permutes, 4 and 8 by DPP
// row shifts (up or down by the lane's bit), 16 by a swizzle within the
// 32-lane group, 32 through LDS. `mask` is a constant after unrolling.
__device__ __forceinline__ int xor_lane(int v, int mask) {
  const int lane = threadIdx.x & 63;
  switch (mask) {
    case 1: return __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);  // [1, 0, 3, 2]
    case 2: return __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);  // [2, 3, 0, 1]
    case 4: {
      const int up = __builtin_amdgcn_update_dpp(0, v, 0x104, 0xF, 0xF, false);
      const int down = __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false);
      return (lane & 4) ? down : up;
    }
    case 8: {
      const int up = __builtin_amdgcn_update_dpp(0, v, 0x108, 0xF, 0xF, false);
      const int down = __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false);
      return (lane & 8) ? down : up;
    }
    case 16: return __builtin_amdgcn_ds_swizzle(v, (16 << 10) | 31);
    default: return __shfl_xor(v, mask, 64);
  }
}

__device__ __forceinline__ uint64_t shfl_xor64(uint64_t v, int mask) {
  const uint32_t lo = (uint32_t)xor_lane((int)(uint32_t)v, mask);
  const uint32_t hi = (uint32_t)xor_lane((int)(uint32_t)(v >> 32), mask);
  return ((uint64_t)hi << 32) | lo;
}

// The wave's 64 entries (one a lane) sorted descending over the lanes.
__device__ __forceinline__ uint64_t wave_sort(uint64_t v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int k = 2; k <= 64; k <<= 1) {
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
      const uint64_t o = shfl_xor64(v, j);
      const bool keep_max = ((lane & j) == 0) == ((lane & k) == 0);
      v = keep_max ? (v > o ? v : o) : (v < o ? v : o);
    }
  }
  return v;
}

// The top 64 of two descending lists, descending: the larger of a[i] and
// b[63 - i] is a bitonic list holding them, which half-cleaners sort.
__device__ __forceinline__ uint64_t wave_merge(uint64_t a, uint64_t b) {
  const int lane = threadIdx.x & 63;
  const uint64_t br = shfl64(b, 63 - lane);
  uint64_t v = a > br ? a : br;
#pragma unroll
  for (int j = 32; j > 0; j >>= 1) {
    const uint64_t o = shfl_xor64(v, j);
    v = (lane & j) == 0 ? (v > o ? v : o) : (v < o ? v : o);
  }
  return v;
}

__device__ __forceinline__ void store_entry(uint32_t* out, int i, uint64_t v) {
  out[2 * i] = topk_bits((uint32_t)(v >> 32));
  out[2 * i + 1] = ~(uint32_t)v;
}

// The workgroup's waves' lists merged into wave 0's (a tree over LDS).
template <int WAVES>
__device__ __forceinline__ uint64_t merge_waves(uint64_t top, uint64_t (*lists)[64]) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int width = WAVES / 2; width >= 1; width >>= 1) {
    if (wave >= width && wave < 2 * width) lists[wave][lane] = top;
    __syncthreads();
    if (wave < width) top = wave_merge(top, lists[wave + width][lane]);
    __syncthreads();
  }
  return top;
}

// Pass one: the top 64 of each tile of 1,024 logits, sorted. Row y of the
// grid reads in + y * in_stride and writes out + y * out_stride (words).
__global__ __launch_bounds__(kTileThreads) void topk_tile_kernel(const uint32_t* __restrict__ in,
                                                                 int count,
                                                                 uint32_t* __restrict__ out,
                                                                 size_t in_stride,
                                                                 size_t out_stride) {
  __shared__ uint64_t lists[kTileThreads / 64][64];
  in += blockIdx.y * in_stride;
  out += blockIdx.y * out_stride;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int base = blockIdx.x * kSelectionTile + wave * 4 * 64 + lane;
  uint64_t v[4];
#pragma unroll
  for (int part = 0; part < 4; ++part) {
    const int e = base + part * 64;
    v[part] = e < count ? pack_entry(in[e], (uint32_t)e) : 0ull;
  }
  uint64_t top = wave_sort(v[0]);
#pragma unroll
  for (int part = 1; part < 4; ++part) top = wave_merge(top, wave_sort(v[part]));
  top = merge_waves<kTileThreads / 64>(top, lists);
  if (wave == 0) store_entry(out, blockIdx.x * kCandidates + lane, top);
}

// Merges sorted lists of 64 (bits, token) pairs, kListsPerMerge a
// workgroup, into one sorted list each.
__device__ __forceinline__ uint64_t merge_lists(const uint32_t* __restrict__ in, int lists,
                                                uint64_t (*shared)[64]) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  uint64_t v[kListsPerMerge / kMergeWaves];
#pragma unroll
  for (int u = 0; u < kListsPerMerge / kMergeWaves; ++u) {
    const int l = blockIdx.x * kListsPerMerge + wave + u * kMergeWaves;
    v[u] = 0ull;
    if (l < lists) {
      const int i = l * kCandidates + lane;
      v[u] = pack_entry(in[2 * i], in[2 * i + 1]);
    }
  }
  uint64_t top = v[0];
#pragma unroll
  for (int u = 1; u < kListsPerMerge / kMergeWaves; ++u) top = wave_merge(top, v[u]);
  return merge_waves<kMergeWaves>(top, shared);
}

__global__ __launch_bounds__(64 * kMergeWaves) void topk_merge_kernel(const uint32_t* __restrict__ in,
                                                                      int lists,
                                                                      uint32_t* __restrict__ out,
                                                                      size_t stride) {
  __shared__ uint64_t shared[kMergeWaves][64];
  in += blockIdx.y * stride;
  out += blockIdx.y * stride;
  const uint64_t top = merge_lists(in, lists, shared);
  if (threadIdx.x < 64) store_entry(out, blockIdx.x * kCandidates + threadIdx.x, top);
}

// The high word of a * b from 16-bit halves (draw.wgsl:34-45).
__device__ __forceinline__ uint32_t mulhi16(uint32_t a, uint32_t b) {
  const uint32_t a0 = a & 0xFFFFu, a1 = a >> 16, b0 = b & 0xFFFFu, b1 = b >> 16;
  const uint32_t p00 = a0 * b0, p01 = a0 * b1, p10 = a1 * b0, p11 = a1 * b1;
  const uint32_t mid = (p00 >> 16) + (p01 & 0xFFFFu) + (p10 & 0xFFFFu);
  return p11 + (p01 >> 16) + (p10 >> 16) + (mid >> 16);
}

// The draw (draw.wgsl:77-170). The per-candidate exponentials are
// independent: candidate i's by thread i, into LDS. Every sum the reference
// takes runs in candidate order on one invocation there too, so thread 0
// takes them in that order and gives the same bits. Every thread of the
// workgroup calls it (it holds a barrier).
// Row `row` of `rows`: a variants step's rows are sequences at one position,
// each drawing as its own one-token step would.
__device__ void draw_one(const DevStep* step, const uint32_t* cand, uint32_t* __restrict__ sampled,
                         uint32_t* __restrict__ token_log, uint32_t row = 0, uint32_t rows = 1) {
  __shared__ float weight[kCandidates], tempered[kCandidates], running[kCandidates];
  __shared__ uint32_t above[kCandidates];
  const uint32_t k = min(step->top_k, (uint32_t)kCandidates);
  const bool use_top_p = step->top_p < 1.0f;
  const float temperature = step->temperature;
  const uint32_t first_bits = cand[0];
  const bool failed = (first_bits & 0x7F800000u) == 0x7F800000u;
  const float first = bits_to_float(first_bits);
  if (threadIdx.x < k) {
    const uint32_t i = threadIdx.x;
    float w = 0.0f, te = 0.0f;
    uint32_t ab = 0u;
    const uint32_t mine_bits = cand[2 * i];
    if (!failed && mine_bits != 0xFF800000u) {
      const float mine = bits_to_float(mine_bits);
      if (use_top_p) w = exp_nonpositive(mine - first);
      if (temperature > 0.0f) te = exp_nonpositive((mine - first) / temperature);
      ab = (step->min_p == 0.0f || mine >= first + step->log_min_p) ? 1u : 0u;
    }
    weight[i] = w;
    tempered[i] = te;
    above[i] = ab;
  }
  __syncthreads();
  if (threadIdx.x != 0) return;
  // Philox4x32-10 at counter (position + tokens, 0, 0, 0), key = seed.
  uint32_t c0 = step->position + (step->variants ? 1u : step->tokens), c1 = 0, c2 = 0, c3 = 0;
  uint32_t k0 = step->seed[0], k1 = step->seed[1];
  for (int r = 0; r < 10; ++r) {
    const uint32_t hi0 = mulhi16(0xD2511F53u, c0), lo0 = 0xD2511F53u * c0;
    const uint32_t hi1 = mulhi16(0xCD9E8D57u, c2), lo1 = 0xCD9E8D57u * c2;
    const uint32_t n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
    c0 = n0; c1 = lo1; c2 = n2; c3 = lo0;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  const float u = (float)(c0 >> 9) * (1.0f / 8388608.0f) + (1.0f / 16777216.0f);
  // The top-p cut, the min-p survivors and the running tempered sums decide
  // only a tempered draw; greedy (temperature 0) takes candidate 0.
  uint32_t chosen = 0;
  if (temperature > 0.0f) {
    if (use_top_p) {
      float sum = 0.0f;
      for (uint32_t i = 0; i < k; ++i) sum = sum + weight[i];
      if (!failed) {
        for (uint32_t i = 0; i < k; ++i) weight[i] = weight[i] / sum;
      }
    }
    uint32_t kept = k;
    float cumulative = 0.0f, tempered_sum = 0.0f;
    for (uint32_t i = 0; i < k; ++i) {
      tempered_sum = tempered_sum + tempered[i];
      running[i] = tempered_sum;
      if (use_top_p) {
        cumulative = cumulative + weight[i];
        if (cumulative >= step->top_p) {
          kept = i + 1;
          break;
        }
      }
    }
    uint32_t survivors = 1;
    while (survivors < kept && above[survivors] == 1u) ++survivors;
    const float goal = u * running[survivors - 1];
    chosen = survivors - 1;
    for (uint32_t i = 0; i < survivors; ++i) {
      if (running[i] > goal) {
        chosen = i;
        break;
      }
    }
  }
  const uint32_t token = failed ? 0u : cand[2 * chosen + 1];
  sampled[0] = token;
  sampled[1] = failed ? 1u : 0u;
  sampled[2] = float_to_bits(u);
  sampled[3] = 0u;
  if (token_log) {
    const size_t at = 2 * ((size_t)step->drawn * rows + row);
    token_log[at] = token;
    token_log[at + 1] = failed ? 1u : 0u;
  }
}

// A fed step's advance of the step parameters.
__device__ void advance_one(DevStep* step) {
  step->position += step->tokens;
  step->tokens = 1;
  step->fed = 1;
  step->logits = 1;
  step->drawn += 1;
}

__global__ __launch_bounds__(64) void draw_kernel(const DevStep* __restrict__ step,
                                                  const uint32_t* __restrict__ cand,
                                                  uint32_t* __restrict__ sampled,
                                                  uint32_t* __restrict__ token_log) {
  draw_one(step, cand, sampled, token_log);
}

__global__ void advance_kernel(DevStep* step) {
  if (threadIdx.x == 0) advance_one(step);
}

// A variants step's advance: the next position, every row fed.
__global__ void advance_rows_kernel(DevStep* step) {
  if (threadIdx.x == 0) {
    step->position += 1;
    step->fed = 1;
    step->logits = 1;
    step->drawn += 1;
  }
}

// The last merge (at most kListsPerMerge lists), the draw from its list and,
// for a fed decode step, the advance.
// Row y of the grid (rows of a variants step) merges in + y * stride and
// draws into record y.
__global__ __launch_bounds__(64 * kMergeWaves) void topk_draw_kernel(
    const uint32_t* __restrict__ in, int lists, uint32_t* __restrict__ cand, DevStep* step,
    uint32_t* __restrict__ sampled, uint32_t* __restrict__ token_log, int advance,
    size_t stride) {
  __shared__ uint64_t shared[kMergeWaves][64];
  __shared__ uint32_t final_list[2 * kCandidates];
  const uint32_t row = blockIdx.y;
  in += row * stride;
  cand += 2 * kCandidates * row;
  const uint64_t top = merge_lists(in, lists, shared);
  if (threadIdx.x < 64) {
    store_entry(cand, threadIdx.x, top);
    store_entry(final_list, threadIdx.x, top);
  }
  __syncthreads();
  draw_one(step, final_list, sampled + 4 * row, token_log, row, gridDim.y);
  // Thread 0 drew (the others left draw_one); its writes to the step come
  // after its own reads of it.
  if (threadIdx.x == 0 && advance) advance_one(step);
}

// Pass one into scratch, then merges of kListsPerMerge lists a workgroup
// until one list is left; `last` launches the final merge.
size_t scratch_words(int count) {
  const int lists = (count + kSelectionTile - 1) / kSelectionTile;
  return (size_t)2 * kCandidates * (lists + (lists + kListsPerMerge - 1) / kListsPerMerge);
}

// `rows` rows of `count` logits, each with its own scratch_words(count)
// words of scratch.
template <typename Last>
hipError_t select_passes(hipStream_t s, const float* logits, int count, int rows,
                         uint32_t* scratch, Last last) {
  if (count < kCandidates || rows < 1) return hipErrorInvalidValue;
  int lists = (count + kSelectionTile - 1) / kSelectionTile;
  const size_t stride = scratch_words(count);
  uint32_t* bufs[2] = {scratch, scratch + 2 * kCandidates * lists};
  hipLaunchKernelGGL(topk_tile_kernel, dim3(lists, rows), dim3(kTileThreads), 0, s,
                     reinterpret_cast<const uint32_t*>(logits), count, bufs[0], (size_t)count,
                     stride);
  hipError_t e = hipGetLastError();
  int at = 0;
  while (e == hipSuccess && lists > kListsPerMerge) {
    const int groups = (lists + kListsPerMerge - 1) / kListsPerMerge;
    hipLaunchKernelGGL(topk_merge_kernel, dim3(groups, rows), dim3(64 * kMergeWaves), 0, s,
                       bufs[at], lists, bufs[at ^ 1], stride);
    e = hipGetLastError();
    lists = groups;
    at ^= 1;
  }
  return e == hipSuccess ? last(bufs[at], lists, stride) : e;
}

}  // namespace

size_t topk_scratch_words(int count) { return scratch_words(count); }

hipError_t launch_topk(hipStream_t s, const float* logits, int count,
                       uint32_t* scratch, uint32_t* candidates) {
  return select_passes(s, logits, count, 1, scratch, [&](const uint32_t* in, int lists, size_t) {
    hipLaunchKernelGGL(topk_merge_kernel, dim3(1), dim3(64 * kMergeWaves), 0, s, in, lists,
                       candidates, (size_t)0);
    return hipGetLastError();
  });
}

hipError_t launch_select(hipStream_t s, DevStep* step, const float* logits, int count,
                         uint32_t* scratch, uint32_t* candidates, uint32_t* sampled,
                         uint32_t* token_log, bool advance) {
  return select_passes(s, logits, count, 1, scratch, [&](const uint32_t* in, int lists, size_t) {
    hipLaunchKernelGGL(topk_draw_kernel, dim3(1), dim3(64 * kMergeWaves), 0, s, in, lists,
                       candidates, step, sampled, token_log, advance ? 1 : 0, (size_t)0);
    return hipGetLastError();
  });
}

hipError_t launch_select_rows(hipStream_t s, DevStep* step, const float* logits, int count,
                              int rows, uint32_t* scratch, uint32_t* candidates,
                              uint32_t* sampled, uint32_t* token_log) {
  hipError_t e = select_passes(
      s, logits, count, rows, scratch, [&](const uint32_t* in, int lists, size_t stride) {
        hipLaunchKernelGGL(topk_draw_kernel, dim3(1, rows), dim3(64 * kMergeWaves), 0, s, in,
                           lists, candidates, step, sampled, token_log, 0, stride);
        return hipGetLastError();
      });
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(advance_rows_kernel, dim3(1), dim3(64), 0, s, step);
  return hipGetLastError();
}

hipError_t launch_draw(hipStream_t s, const DevStep* step, const uint32_t* candidates,
                       uint32_t* sampled, uint32_t* token_log) {
  hipLaunchKernelGGL(draw_kernel, dim3(1), dim3(64), 0, s, step, candidates, sampled,
                     token_log);
  return hipGetLastError();
}

hipError_t launch_advance(hipStream_t s, DevStep* step) {
  hipLaunchKernelGGL(advance_kernel, dim3(1), dim3(64), 0, s, step);
  return hipGetLastError();
}

}  // namespace frz
