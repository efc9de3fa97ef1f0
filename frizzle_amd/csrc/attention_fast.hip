// Prefill attention on the f16 matrix cores (v_mfma_f32_32x32x16_f16), the
// fast prefill mode's attention: chunk states within a stated tolerance of
// the reference's tile recursion instead of bit for bit, folded by the same
// in-order fold (attention_fold_rows_kernel).
//
// A workgroup takes 32 consecutive query rows of the step and one 64-key
// chunk of the cache (the reference's chunks, fixed by position,
// attention.h:40-52), a wave per query head (Gemma 3: four query heads on one
// key-value head, so the chunk's keys and values are staged once for the
// four). Per wave:
//   S^T[key][q] = K q over d = 256 in 16 steps: the key rows as the
//     instruction's A operand straight from LDS, the queries as B, each
//     split into a pair of f16 (hi + lo, to 2^-22 of q; the keys are F16 in
//     the cache, so exact); fp32 accumulation; scaled by 1/16 log2 e;
//   the chunk's maximum m over its live keys (j <= p, j > p - window), each
//     weight exp2(s - m) (v_exp_f32), l their sum, a masked key's weight 0;
//   O^T[d][q] += V^T P over the chunk's keys: V^T from LDS (staged
//     transposed), the weights split into f16 pairs as B.
// The state (m, l, live, O) goes where the fold reads a row's chunk c
// (attention_common.h's layout), so the fold and everything after it are
// the exact path's.

#include "attention_common.h"

namespace frz {
namespace {

using attn::D;
using attn::QH;

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kRows = 32;        // query rows a workgroup
constexpr int kKeyStride = 264;  // halves a staged key row (256 + 8: no bank conflicts)
constexpr int kValStride = 68;   // halves a staged value column (64 + 4)

__device__ __forceinline__ half8 split_hi(const float (&v)[8], half8& lo) {
  half8 hi;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    hi[j] = (_Float16)v[j];
    lo[j] = (_Float16)(v[j] - (float)hi[j]);
  }
  return hi;
}

__global__ __launch_bounds__(256, 2) void chunk_states_mfma_kernel(const DevStep* __restrict__ step,
                                                                   FastAttentionArgs a) {
  __shared__ __attribute__((aligned(16))) _Float16 keys[kChunkKeys * kKeyStride];
  __shared__ __attribute__((aligned(16))) _Float16 vals[D * kValStride];
  const int tokens = (int)step->tokens;
  const int t0 = blockIdx.y * kRows;
  if (t0 >= tokens) return;
  const int p0 = (int)step->position;
  const int t_last = min(t0 + kRows - 1, tokens - 1);
  const int pf = p0 + t0, pl = p0 + t_last;
  const int first_chunk = (pf + 1 > a.window ? pf + 1 - a.window : 0) / kChunkKeys;
  const int c = first_chunk + (int)blockIdx.x;
  if (c > pl / kChunkKeys) return;
  const int tid = threadIdx.x;

  // Stage the chunk's keys (rows) and values (transposed), zeros for keys
  // past the block's last position (never written yet).
  {
    const int key = tid & 63, part = tid >> 6;
    const int j = c * kChunkKeys + key;
    const bool written = j <= pl;
    const size_t slot = (size_t)((uint32_t)j % (uint32_t)a.slots);
    const uint16_t* krow = a.key_cache + slot * D;
    const uint16_t* vrow = a.value_cache + slot * D;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int d0 = 8 * part + 32 * i;
      uint4 kv = make_uint4(0, 0, 0, 0), vv = kv;
      if (written) {
        kv = *reinterpret_cast<const uint4*>(krow + d0);
        vv = *reinterpret_cast<const uint4*>(vrow + d0);
      }
      *reinterpret_cast<uint4*>(keys + key * kKeyStride + d0) = kv;
      const uint32_t w[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        vals[(d0 + 2 * e) * kValStride + key] = __builtin_bit_cast(_Float16, (uint16_t)(w[e] & 0xFFFF));
        vals[(d0 + 2 * e + 1) * kValStride + key] = __builtin_bit_cast(_Float16, (uint16_t)(w[e] >> 16));
      }
    }
  }
  __syncthreads();

  const int h = tid >> 6, lane = tid & 63, half = lane >> 5, q = lane & 31;
  const int t = min(t0 + q, tokens - 1);
  const int p = p0 + t;
  const float* qrow = a.query + (size_t)t * a.q_stride + (size_t)h * D;

  // S^T: two 32-key blocks.
  f32x16 s[2];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int e = 0; e < 16; ++e) s[kb][e] = 0.0f;
#pragma unroll 4
  for (int ds = 0; ds < D / 16; ++ds) {
    const int d = 16 * ds + 8 * half;
    const float4 x0 = *reinterpret_cast<const float4*>(qrow + d);
    const float4 x1 = *reinterpret_cast<const float4*>(qrow + d + 4);
    const float v[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
    half8 ql;
    const half8 qh = split_hi(v, ql);
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const half8 k = *reinterpret_cast<const half8*>(keys + (32 * kb + q) * kKeyStride + d);
      s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(k, qh, s[kb], 0, 0, 0);
      s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(k, ql, s[kb], 0, 0, 0);
    }
  }

  // Register e of block kb: key 32 kb + (e / 4) 8 + half 4 + e % 4 of the
  // chunk, query row q.
  const bool row_live = t0 + q < tokens;
  float m = -__builtin_inff();
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int j = c * kChunkKeys + 32 * kb + (e >> 2) * 8 + half * 4 + (e & 3);
      const bool live = row_live && j <= p && j + a.window > p;
      s[kb][e] = live ? s[kb][e] * a.scale_log2e : -__builtin_inff();
      m = __builtin_fmaxf(m, s[kb][e]);
    }
  m = __builtin_fmaxf(m, __shfl_xor(m, 32));
  const bool chunk_live = m != -__builtin_inff();
  float l = 0.0f;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const float w = s[kb][e] == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(s[kb][e] - m);
      s[kb][e] = w;
      l += w;
    }
  l += __shfl_xor(l, 32);

  // O^T = V^T P, key steps of 16 (k index i of lane half hf is key
  // 16 ks + (i / 4) 8 + hf 4 + i % 4, matching S^T's registers).
  f32x16 o[8];
#pragma unroll
  for (int db = 0; db < 8; ++db)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[db][e] = 0.0f;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    float pv[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) pv[i] = s[ks >> 1][8 * (ks & 1) + i];
    half8 pl_;
    const half8 ph = split_hi(pv, pl_);
    const int k0 = 16 * ks + 4 * half;
#pragma unroll
    for (int db = 0; db < 8; ++db) {
      const _Float16* col = vals + (32 * db + q) * kValStride;
      const uint2 lo4 = *reinterpret_cast<const uint2*>(col + k0);
      const uint2 hi4 = *reinterpret_cast<const uint2*>(col + k0 + 8);
      const half8 v = __builtin_bit_cast(half8, make_uint4(lo4.x, lo4.y, hi4.x, hi4.y));
      o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(v, ph, o[db], 0, 0, 0);
      o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(v, pl_, o[db], 0, 0, 0);
    }
  }

  // The state of row t's chunk (its index among the row's chunks).
  if (!row_live) return;
  const int row_first = (p + 1 > a.window ? p + 1 - a.window : 0) / kChunkKeys;
  if (c < row_first || c > p / kChunkKeys) return;
  const int cs = c - row_first;
  float* out = a.partials + (((size_t)t * a.max_chunks + cs) * QH + h) * D;
#pragma unroll
  for (int db = 0; db < 8; ++db)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const int d = 32 * db + 8 * g4 + 4 * half;
      *reinterpret_cast<float4*>(out + d) =
          make_float4(o[db][4 * g4], o[db][4 * g4 + 1], o[db][4 * g4 + 2], o[db][4 * g4 + 3]);
    }
  if (half == 0) {
    *reinterpret_cast<float4*>(a.stats + (((size_t)t * a.max_chunks + cs) * QH + h) * 4) =
        make_float4(chunk_live ? m : 0.0f, l, chunk_live ? 1.0f : 0.0f, 0.0f);
  }
}

}  // namespace

int fast_attention_chunks(uint32_t first, uint32_t last, int window) {
  int most = 0;
  for (uint32_t pf = first; pf <= last; pf += kRows) {
    const uint32_t pl = pf + kRows - 1 < last ? pf + kRows - 1 : last;
    const uint32_t earliest = pf + 1 > (uint32_t)window ? pf + 1 - (uint32_t)window : 0;
    const int n = (int)(pl / kChunkKeys - earliest / kChunkKeys + 1);
    most = n > most ? n : most;
  }
  return most;
}

hipError_t launch_attention_fast(hipStream_t s, const DevStep* step, const FastAttentionArgs& a,
                                 int max_tokens, int grid_chunks) {
  if (a.head_dim != D || a.query_heads != QH || a.kv_heads != 1 || grid_chunks <= 0)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(chunk_states_mfma_kernel, dim3(grid_chunks, (max_tokens + kRows - 1) / kRows),
                     dim3(256), 0, s, step, a);
  return hipGetLastError();
}

}  // namespace frz
