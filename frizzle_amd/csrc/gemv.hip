// Q4_0 matrix products of the forward path, in the reference's order of
// addition (matmul.h:88-97): each output's K weights are cut into 32 ranges
// of whole 32-weight groups at fixed boundaries (range r is groups
// floor(r G / 32) .. floor((r + 1) G / 32)); a range's products chain by fma
// from zero, k in order; the 32 range sums add in order to a total from
// zero. Every form below keeps that order, so a token's outputs are the same
// bits whether it is decoded alone or prefilled in a tile.
//
// Q4_0 weight j of a block is ((code_j) - 8) * d, decoded exactly in f32
// (q4_0.wgsl:71-83) as fma(code, d, -8 d): code * d and 8 d are exact, and
// so is their difference, so the fma's one rounding changes nothing.

#include "kernels.h"
#include "numerics.h"

namespace frz {
namespace {

constexpr int kThreads = 256;
constexpr int kXStride = 36;  // a staged group of x: 32 floats + 4 of padding

__device__ __forceinline__ float half_to_float(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}

// A layer's pins on neuron n at `position` (edit.wgsl:55-76): the layer's
// edits are sorted by neuron then first position (edit.cpp:20-31), so a
// binary search finds the neuron's; its ranges never overlap.
__device__ __forceinline__ float apply_edits(const uint32_t* __restrict__ t,
                                             int layer, uint32_t n,
                                             uint32_t position, float value) {
  const uint32_t first = t[2 * layer];
  const uint32_t count = t[2 * layer + 1];
  uint32_t lo = 0, hi = count;
  while (lo < hi) {
    const uint32_t mid = (lo + hi) >> 1;
    if (t[first + 5 * mid] < n) lo = mid + 1; else hi = mid;
  }
  for (uint32_t i = lo; i < count; ++i) {
    const uint32_t* e = t + first + 5 * i;
    if (e[0] != n) break;
    if (position < e[3] || position >= e[4]) continue;
    const float v = bits_to_float(e[2]);
    if (e[1] == 1u) {
      if (v != 1.0f) value = value * v;
    } else {
      value = v;
    }
  }
  return value;
}

// ---- tiled form ----------------------------------------------------------
// A workgroup computes a tile of 64 rows x 32 tokens. Per group of K: the 64
// rows' weights are decoded into LDS and the 32 tokens' inputs staged; lane
// (slot s = t % 64, token octet t / 64) chains its 8 tokens' products for row
// s. Each range's sums start from zero and are added to the totals at the
// range's end: the order above (matmul.wgsl:320-405).
constexpr int kTileRows = 64;
constexpr int kTileTokens = 32;
constexpr int kWStride = 33;

// Row slot s of the tile: for a gated tile, slots 0..31 are gate rows and
// 32..63 the same up rows.
template <bool GATED>
__global__ __launch_bounds__(kThreads) void gemm_tiled(
    const DevStep* __restrict__ step, Q4Matrix w, Q4Matrix up,
    const float* __restrict__ x, int x_stride, float* __restrict__ y,
    int y_stride, const uint32_t* __restrict__ edits, int layer) {
  __shared__ float ws[kTileRows * kWStride];
  __shared__ float xs[32 * kTileTokens];
  const int tokens = (int)step->tokens;
  const int token0 = blockIdx.y * kTileTokens;
  if (token0 >= tokens) return;
  const int groups = w.cols >> 5;
  const int t = threadIdx.x;
  const int slot = t & 63, octet = t >> 6;
  // Staging roles: thread t decodes word t % 4 of row t / 4's block.
  const int srow = t >> 2, sword = t & 3;
  int stage_row;
  const uint8_t* src_codes = w.codes;
  const uint16_t* src_scales = w.scales;
  if (GATED) {
    const int n = blockIdx.x * 32 + (srow & 31);
    if (srow >= 32) {
      src_codes = up.codes;
      src_scales = up.scales;
    }
    stage_row = n < w.rows ? n : -1;
  } else {
    const int n = blockIdx.x * kTileRows + srow;
    stage_row = n < w.rows ? n : -1;
  }
  // x staging: thread t loads floats 4 (t % 8) .. +3 of token t / 8.
  const int xtok = t >> 3, xpart = t & 7;
  const bool xlive = token0 + xtok < tokens;
  const float* xrow = x + (size_t)(token0 + xtok) * x_stride;

  float s[8], total[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) total[i] = 0.0f;
  for (int r = 0; r < kRanges; ++r) {
#pragma unroll
    for (int i = 0; i < 8; ++i) s[i] = 0.0f;
    const int lo = r * groups / kRanges, hi = (r + 1) * groups / kRanges;
    for (int g = lo; g < hi; ++g) {
      __syncthreads();
      {
        float wv[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        if (stage_row >= 0) {
          const size_t blk = (size_t)stage_row * groups + g;
          const uint32_t word =
              reinterpret_cast<const uint32_t*>(src_codes)[blk * 4 + sword];
          const float d = half_to_float(src_scales[blk]);
          const float m8d = -8.0f * d;
#pragma unroll
          for (int b = 0; b < 4; ++b) {
            wv[b] = fmaf_((float)((word >> (8 * b)) & 0xFu), d, m8d);
            wv[4 + b] = fmaf_((float)((word >> (8 * b + 4)) & 0xFu), d, m8d);
          }
        }
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          ws[srow * kWStride + 4 * sword + b] = wv[b];
          ws[srow * kWStride + 16 + 4 * sword + b] = wv[4 + b];
        }
        float4 xv = make_float4(0.f, 0.f, 0.f, 0.f);
        if (xlive) xv = *reinterpret_cast<const float4*>(xrow + g * 32 + 4 * xpart);
        xs[(4 * xpart + 0) * kTileTokens + xtok] = xv.x;
        xs[(4 * xpart + 1) * kTileTokens + xtok] = xv.y;
        xs[(4 * xpart + 2) * kTileTokens + xtok] = xv.z;
        xs[(4 * xpart + 3) * kTileTokens + xtok] = xv.w;
      }
      __syncthreads();
#pragma unroll 8
      for (int k = 0; k < 32; ++k) {
        const float wk = ws[slot * kWStride + k];
        const float4 x0 = *reinterpret_cast<const float4*>(&xs[k * kTileTokens + octet * 8]);
        const float4 x1 = *reinterpret_cast<const float4*>(&xs[k * kTileTokens + octet * 8 + 4]);
        s[0] = fmaf_(wk, x0.x, s[0]);
        s[1] = fmaf_(wk, x0.y, s[1]);
        s[2] = fmaf_(wk, x0.z, s[2]);
        s[3] = fmaf_(wk, x0.w, s[3]);
        s[4] = fmaf_(wk, x1.x, s[4]);
        s[5] = fmaf_(wk, x1.y, s[5]);
        s[6] = fmaf_(wk, x1.z, s[6]);
        s[7] = fmaf_(wk, x1.w, s[7]);
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) total[i] = total[i] + s[i];
  }
  if (!GATED) {
    const int row = blockIdx.x * kTileRows + slot;
    if (row < w.rows) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int tok = token0 + octet * 8 + i;
        if (tok < tokens) y[(size_t)tok * y_stride + row] = total[i];
      }
    }
  } else {
    // Gate totals meet their up totals in LDS (reusing the weight tile).
    __syncthreads();
    float* meet = ws;  // [32 neurons][32 tokens + 1]
    if (slot >= 32) {
#pragma unroll
      for (int i = 0; i < 8; ++i) meet[(slot - 32) * 33 + octet * 8 + i] = total[i];
    }
    __syncthreads();
    if (slot < 32) {
      const int n = blockIdx.x * 32 + slot;
      if (n < w.rows) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int tok = token0 + octet * 8 + i;
          if (tok < tokens) {
            float v = gelu_tanh(total[i]) * meet[slot * 33 + octet * 8 + i];
            if (edits) v = apply_edits(edits, layer, (uint32_t)n, step->position + tok, v);
            y[(size_t)tok * y_stride + n] = v;
          }
        }
      }
    }
  }
}

}  // namespace

hipError_t launch_gemv(hipStream_t s, const DevStep* step, Q4Matrix w,
                       const float* x, int x_stride, float* y, int y_stride,
                       int max_tokens, bool last_token) {
  if (w.cols % 32 != 0 || w.rows <= 0) return hipErrorInvalidValue;
  if (max_tokens <= 1 || last_token) {
    GemvInput in{};
    in.x = x + (size_t)(last_token ? max_tokens - 1 : 0) * x_stride;
    return launch_gemv_decode(s, step, w, in, 0, y);
  }
  const dim3 grid((w.rows + kTileRows - 1) / kTileRows,
                  (max_tokens + kTileTokens - 1) / kTileTokens);
  hipLaunchKernelGGL(gemm_tiled<false>, grid, dim3(kThreads), 0, s, step, w, w, x,
                     x_stride, y, y_stride, (const uint32_t*)nullptr, 0);
  return hipGetLastError();
}

hipError_t launch_gated(hipStream_t s, const DevStep* step, Q4Matrix gate,
                        Q4Matrix up, const float* x, float* act,
                        int max_tokens, const uint32_t* edits, int layer) {
  if (gate.cols % 32 != 0 || gate.rows != up.rows || gate.cols != up.cols)
    return hipErrorInvalidValue;
  if (max_tokens <= 1) {
    GemvInput in{};
    in.x = x;
    return launch_gated_decode(s, step, gate, up, in, 0, act, edits, layer);
  }
  const dim3 grid((gate.rows + 31) / 32, (max_tokens + kTileTokens - 1) / kTileTokens);
  hipLaunchKernelGGL(gemm_tiled<true>, grid, dim3(kThreads), 0, s, step, gate, up, x,
                     gate.cols, act, gate.rows, edits, layer);
  return hipGetLastError();
}

}  // namespace frz
