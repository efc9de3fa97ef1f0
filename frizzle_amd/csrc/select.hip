// The output block's selection and draw: top-64 of the logits in the
// reference's total order (topk.wgsl), the draw over the candidates
// (draw.wgsl), and the fed step's advance of the step parameters.

#include "kernels.h"
#include "numerics.h"

namespace frz {
namespace {

constexpr int kTopkThreads = 256;

// One pass: each workgroup keeps the top 64 of its tile of 1,024 entries,
// sorted, as (logit bits, token) pairs. Entries are ordered by the
// order-preserving key of their bits (larger first) and, on equal keys, by
// the lower token (topk.wgsl:57-61); packed as key << 32 | ~token, that
// order is the descending order of one 64-bit integer, sorted here by a
// bitonic network. Slots past the input, and slots a pass before padded
// (token 0xFFFFFFFF), pack to 0 and sort last (topk.wgsl:138-166).
template <bool FIRST>
__global__ __launch_bounds__(kTopkThreads) void topk_kernel(const uint32_t* __restrict__ in,
                                                            int count,
                                                            uint32_t* __restrict__ out) {
  __shared__ uint64_t keys[kSelectionTile];
  const int t = threadIdx.x;
  for (int part = 0; part < 4; ++part) {
    const int s = t + part * kTopkThreads;
    const int e = blockIdx.x * kSelectionTile + s;
    uint64_t packed = 0;
    if (e < count) {
      uint32_t bits, id;
      if (FIRST) {
        bits = in[e];
        id = (uint32_t)e;
      } else {
        bits = in[2 * e];
        id = in[2 * e + 1];
      }
      if (id != 0xFFFFFFFFu) packed = ((uint64_t)topk_key(bits) << 32) | (uint32_t)~id;
    }
    keys[s] = packed;
  }
  __syncthreads();
  for (int k = 2; k <= kSelectionTile; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int part = 0; part < 2; ++part) {
        const int i = t + part * kTopkThreads;  // one of 512 pairs
        const int i1 = (i / j) * 2 * j + (i % j);
        const int i2 = i1 + j;
        const bool descending = (i1 & k) == 0;
        const uint64_t x = keys[i1], y = keys[i2];
        if ((x < y) == descending) {
          keys[i1] = y;
          keys[i2] = x;
        }
      }
      __syncthreads();
    }
  }
  if (t < kCandidates) {
    const uint64_t packed = keys[t];
    const uint32_t key = (uint32_t)(packed >> 32);
    const uint32_t id = ~(uint32_t)packed;
    out[2 * (blockIdx.x * kCandidates + t)] = topk_bits(key);
    out[2 * (blockIdx.x * kCandidates + t) + 1] = id;
  }
}

// The high word of a * b from 16-bit halves (draw.wgsl:34-45).
__device__ __forceinline__ uint32_t mulhi16(uint32_t a, uint32_t b) {
  const uint32_t a0 = a & 0xFFFFu, a1 = a >> 16, b0 = b & 0xFFFFu, b1 = b >> 16;
  const uint32_t p00 = a0 * b0, p01 = a0 * b1, p10 = a1 * b0, p11 = a1 * b1;
  const uint32_t mid = (p00 >> 16) + (p01 & 0xFFFFu) + (p10 & 0xFFFFu);
  return p11 + (p01 >> 16) + (p10 >> 16) + (mid >> 16);
}

// The draw (draw.wgsl:77-170), by one lane: every sum the reference takes
// runs in candidate order on one invocation there too, and the per-candidate
// exponentials are independent, so one lane gives the same bits.
__global__ __launch_bounds__(64) void draw_kernel(const DevStep* __restrict__ step,
                                                  const uint32_t* __restrict__ cand,
                                                  uint32_t* __restrict__ sampled,
                                                  uint32_t* __restrict__ token_log) {
  if (threadIdx.x != 0) return;
  const uint32_t k = min(step->top_k, (uint32_t)kCandidates);
  const bool use_top_p = step->top_p < 1.0f;
  const float temperature = step->temperature;
  const uint32_t first_bits = cand[0];
  const bool failed = (first_bits & 0x7F800000u) == 0x7F800000u;
  float weight[kCandidates], tempered[kCandidates], running[kCandidates];
  uint32_t above[kCandidates];
  const float first = bits_to_float(first_bits);
  for (uint32_t i = 0; i < k; ++i) {
    weight[i] = 0.0f;
    tempered[i] = 0.0f;
    above[i] = 0u;
    const uint32_t mine_bits = cand[2 * i];
    if (!failed && mine_bits != 0xFF800000u) {
      const float mine = bits_to_float(mine_bits);
      if (use_top_p) weight[i] = exp_nonpositive(mine - first);
      if (temperature > 0.0f) tempered[i] = exp_nonpositive((mine - first) / temperature);
      above[i] = (step->min_p == 0.0f || mine >= first + step->log_min_p) ? 1u : 0u;
    }
  }
  // Philox4x32-10 at counter (position + tokens, 0, 0, 0), key = seed.
  uint32_t c0 = step->position + step->tokens, c1 = 0, c2 = 0, c3 = 0;
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
  const uint32_t token = failed ? 0u : cand[2 * chosen + 1];
  sampled[0] = token;
  sampled[1] = failed ? 1u : 0u;
  sampled[2] = float_to_bits(u);
  sampled[3] = 0u;
  if (token_log) {
    token_log[2 * step->drawn] = token;
    token_log[2 * step->drawn + 1] = failed ? 1u : 0u;
  }
}

__global__ void advance_kernel(DevStep* step) {
  if (threadIdx.x != 0) return;
  step->position += step->tokens;
  step->tokens = 1;
  step->fed = 1;
  step->logits = 1;
  step->drawn += 1;
}

}  // namespace

hipError_t launch_topk(hipStream_t s, const float* logits, int count,
                       uint32_t* scratch, uint32_t* candidates) {
  if (count < kCandidates) return hipErrorInvalidValue;
  const uint32_t* in = reinterpret_cast<const uint32_t*>(logits);
  int tiles = (count + kSelectionTile - 1) / kSelectionTile;
  uint32_t* bufs[2] = {scratch, scratch + 2 * kCandidates * tiles};
  uint32_t* out = tiles == 1 ? candidates : bufs[0];
  hipLaunchKernelGGL(topk_kernel<true>, dim3(tiles), dim3(kTopkThreads), 0, s, in, count, out);
  hipError_t e = hipGetLastError();
  int pass = 1;
  while (e == hipSuccess && tiles > 1) {
    in = out;
    count = tiles * kCandidates;
    tiles = (count + kSelectionTile - 1) / kSelectionTile;
    out = tiles == 1 ? candidates : bufs[pass % 2];
    hipLaunchKernelGGL(topk_kernel<false>, dim3(tiles), dim3(kTopkThreads), 0, s, in, count,
                       out);
    e = hipGetLastError();
    ++pass;
  }
  return e;
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
