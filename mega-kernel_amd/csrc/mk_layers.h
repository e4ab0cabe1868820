// Matrix-core and per-head helpers shared by the layer-by-layer engine (layers_kernel.hip) and the
// persistent batched decode kernel (batch_kernel.hip) on MI355X (gfx950).
//
// MFMA operand layout (v_mfma_f32_16x16x32_bf16; lane l, i = l % 16, g = l / 16): A[i][8g + j] and
// B[8g + j][i] for j = 0..7 (8 bf16 = 16 bytes per lane), accumulator C[4g + j][i] for j = 0..3.
// Both operands are read as 16-byte chunks of K-contiguous rows.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mk_device.h"

namespace mkp {
using namespace mk;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned long long u64;

constexpr int D = 128, HQ = 16, HKV = 8;
constexpr float EPS = 1e-6f;
constexpr float ATT_SCALE = 0.08838834764831845f;  // 128 ** -0.5

__device__ __forceinline__ f32x4 mfma(uint4 a, uint4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                 0, 0, 0);
}

// hi = bf16(v), lo = bf16(v - hi) of 8 values, as two 16-byte chunks
__device__ __forceinline__ void split8(const float* v, uint4& hi, uint4& lo) {
  uint32_t h[4], l[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    h[q] = pack_bf16x2(v[2 * q], v[2 * q + 1]);
    l[q] = pack_bf16x2(v[2 * q] - bf16_lo(h[q]), v[2 * q + 1] - bf16_hi(h[q]));
  }
  hi = make_uint4(h[0], h[1], h[2], h[3]);
  lo = make_uint4(l[0], l[1], l[2], l[3]);
}

__device__ __forceinline__ void unpack8(uint4 w, float (&v)[8]) {
  v[0] = bf16_lo(w.x); v[1] = bf16_hi(w.x); v[2] = bf16_lo(w.y); v[3] = bf16_hi(w.y);
  v[4] = bf16_lo(w.z); v[5] = bf16_hi(w.z); v[6] = bf16_lo(w.w); v[7] = bf16_hi(w.w);
}

// Greedy key of a logit: (order-preserving bf16 of the logit) << 32 | ~idx, so that the maximum key
// is the largest bf16-rounded logit and, among equal ones, the lowest index
// (/root/reference/model.py:97 takes torch's argmax of the logits).
__device__ __forceinline__ u64 argmax_key(float logit, int idx) {
  uint32_t u = (uint32_t)f32_to_bf16(logit) << 16;
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((u64)u << 32) | (0xffffffffu - (uint32_t)idx);
}

// Per-head RMSNorm + rotate-half RoPE of 8 dims of one head row held by a 16-lane row (lane t: dims
// 8t..8t+7; the RoPE partner of dim d is d +- 64, in lane t ^ 8), as the decode kernel applies them
// (/root/reference/megakernel.cu:490-630, 548-555).
__device__ __forceinline__ void head_norm_rope(float (&v)[8], const float (&wn)[8], const float (&cs)[8],
                                               const float (&sn)[8], int t) {
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) ss = fmaf(v[i], v[i], ss);
  const float rs = rsqrtf(row16_sum(ss) / (float)D + EPS);
  float u[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) u[i] = v[i] * rs * wn[i];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float pr = dpp<0x128>(u[i]);  // row_ror:8 inside the 16-lane row: lane t ^ 8
    v[i] = t < 8 ? u[i] * cs[i] - pr * sn[i] : u[i] * cs[i] + pr * sn[i];
  }
}

}  // namespace mkp
