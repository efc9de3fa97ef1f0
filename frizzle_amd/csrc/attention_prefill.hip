// The prefill attention kernels: chunk states for every row of a step,
// then each row's in-order fold (the chunk arithmetic is in
// attention_common.h).

#include "attention_common.h"

namespace frz {
namespace {
using namespace attn;

// ---- prefill: chunk states, then the fold per row ------------------------------
__global__ __launch_bounds__(kThreads) void attention_chunk_kernel(
    const DevStep* __restrict__ step, AttentionArgs a) {
  __shared__ ChunkShared S;
  const int row = blockIdx.y;
  if (row >= (int)step->tokens) return;
  const int p = (int)step->position + row;
  const ChunkRange r = chunk_range(p, a.window, blockIdx.x);
  if ((int)blockIdx.x >= r.count) return;
  const int t = threadIdx.x;
  StageRegs R;
  stage_load(R, a.key_cache, a.value_cache, a.slots, r, -1);
  {
    const float* q = a.query + (size_t)row * a.q_stride;
    S.q[t] = q[t] * a.scale_log2e;  // kThreads == QH * D
  }
  stage_store(S, R, r, -1);
  __syncthreads();
  const size_t slot = (size_t)row * a.max_chunks + blockIdx.x;
  chunk_state<false>(S, p, a.window, r, a.partials + slot * QH * D, a.stats + slot * QH * 4);
}

__global__ __launch_bounds__(kThreads) void attention_combine_kernel(
    const DevStep* __restrict__ step, AttentionArgs a) {
  const int row = blockIdx.x;
  if (row >= (int)step->tokens) return;
  const int p = (int)step->position + row;
  const ChunkRange r = chunk_range(p, a.window, 0);
  const size_t slot = (size_t)row * a.max_chunks;
  a.out[(size_t)row * QH * D + threadIdx.x] =
      fold_chunks<false>(a.partials + slot * QH * D, a.stats + slot * QH * 4, r.count);
}

}  // namespace

hipError_t launch_attention(hipStream_t s, const DevStep* step, const AttentionArgs& a,
                            int max_tokens) {
  if (a.head_dim != D || a.query_heads != QH || a.kv_heads != 1) return hipErrorInvalidValue;
  hipLaunchKernelGGL(attention_chunk_kernel, dim3(a.max_chunks, max_tokens), dim3(kThreads), 0,
                     s, step, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(attention_combine_kernel, dim3(max_tokens), dim3(kThreads), 0, s, step, a);
  return hipGetLastError();
}

}  // namespace frz
