// Persistent cooperative decode kernel for Qwen3-shaped models on MI355X (gfx950), plus its C ABI.
//
// One launch = one decode step for batch 1: embedding -> L x {RMSNorm, QKV, per-head norm + RoPE,
// K/V cache write, split-K GQA attention, O-proj + residual, RMSNorm, gate/up + SiLU, down +
// residual} -> final RMSNorm -> tied LM head -> greedy argmax. This is the work of the reference's
// decode_kernel (/root/reference/megakernel.cu:744-893), re-planned for 256 CUs in 8 XCDs.
//
// Work placement (XCD-aware). The grid is one 512-thread workgroup per CU; workgroup b runs on
// XCD x = b % 8 as "local" workgroup j = b / 8 (the dispatcher's round-robin placement, checked
// by the host at initialisation; correctness does not depend on it). XCD x owns K/V head x: the
// 512 Q/K/V rows of that group, its attention and its 256 columns of o_proj, plus a 1/8 slice of
// the MLP intermediate. So per layer only two exchanges cross XCDs:
//
//   A  QKV rows of group x, 16 rows per WG            -> XCD barrier
//   B  q/k norm + RoPE (redundant), K/V cache write,
//      split-K attention over ctx/32 positions per WG -> XCD barrier
//   C  merge 32 partials, o_proj partial over the
//      group's 256 columns                            -> grid barrier
//   D  residual += sum of 8 o_proj partials (every WG,
//      same order), RMSNorm, gate/up rows of slice x  -> XCD barrier
//   E  down_proj partial over slice x's columns       -> grid barrier
//
// The residual stream is kept redundantly in every workgroup's LDS; every workgroup computes it
// from the same inputs in the same order, so all copies are bitwise identical.
//
// Numerics follow the reference kernel's fp32 design: bf16 weights and cache, fp32 activations
// and accumulation, fp32 RMSNorm, exact softmax, new K/V rounded to bf16 as stored. Logits are
// fp32; the greedy token is the argmax of the bf16-rounded logits, lowest index on ties.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <mutex>
#include <string.h>

#include "mk_device.h"
#include "../../include/megakernel_amd.h"

namespace mk {

constexpr int D = 128;        // head_dim
constexpr int HQ = 16;        // query heads
constexpr int HKV = 8;        // K/V heads
constexpr int NXCD = 8;       // XCDs on MI355X
constexpr int WPX = 32;       // workgroups per XCD
constexpr int NWG = NXCD * WPX;
constexpr int NT = 512;       // threads per workgroup
constexpr int NWAVE = NT / 64;
constexpr int NGRP = NT / 16;  // 16-lane row groups per workgroup
constexpr int QKV_ROWS_X = 4 * D;  // q (2 heads) + k + v rows owned by one XCD
constexpr int QKV_ROWS_WG = QKV_ROWS_X / WPX;  // 16
constexpr int APS = 132;      // floats per attention partial: acc[128], m, l, pad
constexpr float EPS = 1e-6f;
constexpr float ATT_SCALE = 0.08838834764831845f;  // 128 ** -0.5
constexpr uint32_t SPIN_LIMIT = 1u << 22;
constexpr uint32_t ERR_TIMEOUT = 1u;

// Workspace layout. Floats first, then 256-byte counter lines.
constexpr int MAX_H = 2048, MAX_I = 6144;
constexpr size_t WS_QKV = 0;
constexpr size_t WS_APART = WS_QKV + NXCD * QKV_ROWS_X;
constexpr size_t WS_OPART = WS_APART + (size_t)NXCD * WPX * 2 * APS;
constexpr size_t WS_MBUF = WS_OPART + (size_t)NXCD * MAX_H;
constexpr size_t WS_DPART = WS_MBUF + MAX_I;
constexpr size_t WS_FLOATS = WS_DPART + (size_t)NXCD * MAX_H;
constexpr int CTR_LINE = 64;  // u32 per counter line (256 B)
enum CtrLine { L_XL = 0, L_XG = 8, L_G = 16, L_XEXIT = 17, L_GEXIT = 25, L_STATUS = 26, L_AMAX = 27, N_LINES = 32 };
constexpr size_t WS_BYTES = WS_FLOATS * 4 + (size_t)N_LINES * CTR_LINE * 4;

struct KArgs {
  const uint16_t* embed;
  const uint16_t* lm_head;
  const uint16_t* final_norm;
  const mk_layer_weights* layers;
  const uint16_t* cos_tab;
  const uint16_t* sin_tab;
  uint16_t* k_cache;
  uint16_t* v_cache;
  float* logits;
  int32_t* out_token;
  float* ws;
  uint32_t* ctr;
  uint64_t* trace;  // optional: per-workgroup phase timestamps (TRACE_N per workgroup)
  int token, position, max_seq, num_layers, vocab;
};

// Phase timestamps (s_memrealtime, 100 MHz): per layer and phase p in A..E, [10*layer + 2p] when the
// phase starts (its barrier released) and [10*layer + 2p + 1] when the workgroup arrives at the
// barrier that ends it; TRACE_TAIL slots for embedding, LM head and exit.
constexpr int TRACE_LAYERS = 64;
constexpr int TRACE_TAIL = 8;
constexpr int TRACE_N = TRACE_LAYERS * 10 + TRACE_TAIL;
__device__ __forceinline__ void mark(const KArgs& a, int idx) {
  if (a.trace != nullptr && threadIdx.x == 0 && idx >= 0 && idx < TRACE_N)
    a.trace[(size_t)blockIdx.x * TRACE_N + idx] = wall_clock64();
}

// ------------------------------------------------------------------------------------------
// Grid synchronisation. Counters only grow during a launch; the last workgroup to leave resets
// them, so every launch starts from zero. Every wait is bounded: on timeout the status word is
// set and all later waits return at once, so a broken launch still drains.
// ------------------------------------------------------------------------------------------
struct Sync {
  uint32_t* xl;     // this XCD's local-barrier counter
  uint32_t* xg;     // this XCD's first-level grid-barrier counter
  uint32_t* g;      // grid-barrier counter
  uint32_t* status;
  uint32_t nl = 0, ng = 0;
  bool failed = false;
};

__device__ __forceinline__ bool wait_ge(const uint32_t* p, uint32_t target, uint32_t* status) {
  for (uint32_t it = 0;; ++it) {
    if ((int32_t)(ld_dev_u32(p) - target) >= 0) return true;
    if ((it & 63u) == 63u && ld_dev_u32(status) != 0) return false;
    if (it > SPIN_LIMIT) {
      st_dev_u32(status, ERR_TIMEOUT);
      return false;
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

__device__ __forceinline__ void xcd_barrier(Sync& s) {
  wait_vmem();
  __syncthreads();
  s.nl++;
  if (threadIdx.x == 0) {
    __hip_atomic_fetch_add(s.xl, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (!s.failed && !wait_ge(s.xl, WPX * s.nl, s.status)) s.failed = true;
  }
  __syncthreads();
}

__device__ __forceinline__ void grid_barrier(Sync& s) {
  wait_vmem();
  __syncthreads();
  s.ng++;
  if (threadIdx.x == 0) {
    uint32_t old = __hip_atomic_fetch_add(s.xg, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (old + 1 == WPX * s.ng) __hip_atomic_fetch_add(s.g, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (!s.failed && !wait_ge(s.g, NXCD * s.ng, s.status)) s.failed = true;
  }
  __syncthreads();
}

// ------------------------------------------------------------------------------------------
// Block helpers
// ------------------------------------------------------------------------------------------
__device__ __forceinline__ float block_sum(float v, float* s_red) {
  v = wave_sum(v);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) s_red[wave] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int w = 0; w < NWAVE; ++w) t += s_red[w];
  __syncthreads();
  return t;
}

// RMSNorm in fp32, the reference's form x * w * rsqrt(mean(x^2) + eps)
// (/root/reference/megakernel.cu:704-739 and :148-182).
template <int H>
__device__ __forceinline__ void rms_norm(const float* s_in, const uint16_t* w, float* s_out, float* s_red) {
  float ss = 0.f;
  for (int i = threadIdx.x; i < H; i += NT) ss += s_in[i] * s_in[i];
  ss = block_sum(ss, s_red);
  const float r = rsqrtf(ss / (float)H + EPS);
  for (int i = threadIdx.x; i < H; i += NT) s_out[i] = s_in[i] * bf16_to_f32(w[i]) * r;
  __syncthreads();
}

// ------------------------------------------------------------------------------------------
// GEMV engine. A workgroup's share of a phase is a list of (row, column-segment) tasks; each
// 16-lane row group takes one task at a time, streams its weight chunks (16 B = 8 bf16 per lane
// per step, 256 contiguous bytes per group per step) and reduces over the 16 lanes with DPP.
// x is the fp32 input in LDS (C floats); emit(r, seg, value) receives each task's sum.
// ------------------------------------------------------------------------------------------
template <int C, int S, typename RowPtr, typename Emit>
__device__ __forceinline__ void gemv(int R, RowPtr rowptr, const float* x, Emit emit) {
  constexpr int CPS = C / 8 / S;  // 16-byte chunks per segment
  constexpr int CPL = CPS / 16;   // chunks per lane per task
  static_assert(CPS % 16 == 0, "segment must be a multiple of 16 chunks");
  const int grp = threadIdx.x >> 4;
  const int t = threadIdx.x & 15;
  for (int task = grp; task < R * S; task += NGRP) {
    const int r = task / S;
    const int sg = task - r * S;
    const uint4* w = reinterpret_cast<const uint4*>(rowptr(r)) + sg * CPS + t;
    const float* xs = x + (sg * CPS + t) * 8;
    uint4 wv[CPL];
#pragma unroll
    for (int k = 0; k < CPL; ++k) wv[k] = ld_stream(w + 16 * k);
    float acc = 0.f;
#pragma unroll
    for (int k = 0; k < CPL; ++k) acc = dot8(wv[k], xs + 128 * k, acc);
    acc = row16_sum(acc);
    if (t == 0) emit(r, sg, acc);
  }
}

// Read n floats published by other workgroups (device scope) into LDS.
__device__ __forceinline__ void fetch_dev(const float* src, float* dst, int n) {
  for (int i = threadIdx.x * 4; i < n; i += NT * 4) {
    float4 v = ld_dev_f32x4(src, i * 4);
    dst[i] = v.x; dst[i + 1] = v.y; dst[i + 2] = v.z; dst[i + 3] = v.w;
  }
}

// s_res[i] += sum over the 8 XCD partials part[x][i], x ascending (identical order everywhere).
template <int H>
__device__ __forceinline__ void add_partials(float* s_res, const float* part) {
  for (int i = threadIdx.x * 4; i < H; i += NT * 4) {
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int x = 0; x < NXCD; ++x) {
      float4 v = ld_dev_f32x4(part, (x * H + i) * 4);
      acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
    }
    s_res[i] += acc.x; s_res[i + 1] += acc.y; s_res[i + 2] += acc.z; s_res[i + 3] += acc.w;
  }
  __syncthreads();
}

__device__ __forceinline__ unsigned long long argmax_key(float logit, int idx) {
  // order-preserving map of the bf16-rounded logit, then the complemented index so that equal
  // values prefer the lower index under an unsigned max
  uint32_t u = (uint32_t)f32_to_bf16(logit) << 16;
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((unsigned long long)u << 32) | (0xffffffffu - (uint32_t)idx);
}

// ------------------------------------------------------------------------------------------
// The kernel
// ------------------------------------------------------------------------------------------
template <int H, int I>
__global__ void __launch_bounds__(NT, 1) decode_kernel(const KArgs a) {
  constexpr int IX = I / NXCD;      // MLP intermediate slice per XCD
  constexpr int IPW = IX / WPX;     // gate (and up) rows per workgroup
  constexpr int HPW = H / WPX;      // o_proj / down_proj rows per workgroup
  // column segments for gate/up: the smallest S with a whole number of task rounds
  constexpr int GU_S = (2 * IPW) % NGRP == 0 ? 1 : (4 * IPW) % NGRP == 0 ? 2 : 4;
  constexpr int XN = (H > IX ? H : IX);
  static_assert(HPW * WPX == H && IPW * WPX == IX && IX * NXCD == I, "shape must split evenly");
  static_assert((2 * IPW * GU_S) % NGRP == 0 && (H / 8 / GU_S) % 16 == 0, "gate/up tasks must tile the groups");

  __shared__ __attribute__((aligned(16))) float s_res[H];
  __shared__ __attribute__((aligned(16))) float s_x[XN];
  __shared__ __attribute__((aligned(16))) float s_part[128];
  __shared__ float s_red[NWAVE];
  __shared__ __attribute__((aligned(16))) float s_q[2][D];
  __shared__ __attribute__((aligned(16))) float s_k[D];
  __shared__ __attribute__((aligned(16))) float s_v[D];
  __shared__ __attribute__((aligned(16))) float s_wpart[NWAVE][2][D + 2];
  __shared__ float s_mw[WPX][2][2];

  const int xcd = blockIdx.x % NXCD;
  const int j = blockIdx.x / NXCD;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;

  float* ws = a.ws;
  float* qkv_x = ws + WS_QKV + xcd * QKV_ROWS_X;
  float* apart_x = ws + WS_APART + (size_t)xcd * WPX * 2 * APS;
  float* opart = ws + WS_OPART;
  float* mbuf_x = ws + WS_MBUF + xcd * IX;
  float* dpart = ws + WS_DPART;

  Sync sync;
  sync.xl = a.ctr + (L_XL + xcd) * CTR_LINE;
  sync.xg = a.ctr + (L_XG + xcd) * CTR_LINE;
  sync.g = a.ctr + L_G * CTR_LINE;
  sync.status = a.ctr + L_STATUS * CTR_LINE;

  const int position = a.position;
  const int ctx = position + 1;

  const int tb = TRACE_LAYERS * 10;
  mark(a, tb + 0);
  // Embedding row -> fp32 residual (every workgroup keeps its own copy).
  {
    const uint16_t* row = a.embed + (size_t)a.token * H;
    for (int i = threadIdx.x; i < H; i += NT) s_res[i] = bf16_to_f32(row[i]);
    __syncthreads();
  }

  for (int layer = 0; layer < a.num_layers; ++layer) {
    const mk_layer_weights lw = a.layers[layer];
    const int tl = layer < TRACE_LAYERS ? layer * 10 : -1000000;
    mark(a, tl + 0);
    if (layer > 0) add_partials<H>(s_res, dpart);

    // ---- A: input RMSNorm, QKV rows of this XCD's K/V group --------------------------------
    rms_norm<H>(s_res, (const uint16_t*)lw.norm_weight, s_x, s_red);
    {
      // local rows [16j, 16j+16) of the XCD's 512: q heads 2x,2x+1 (256), k head x, v head x
      const uint16_t* base;
      int row0;
      if (j < 16) { base = (const uint16_t*)lw.q_weight; row0 = 2 * D * xcd + QKV_ROWS_WG * j; }
      else if (j < 24) { base = (const uint16_t*)lw.k_weight; row0 = D * xcd + QKV_ROWS_WG * (j - 16); }
      else { base = (const uint16_t*)lw.v_weight; row0 = D * xcd + QKV_ROWS_WG * (j - 24); }
      gemv<H, 2>(QKV_ROWS_WG, [&](int r) { return base + (size_t)(row0 + r) * H; }, s_x,
                 [&](int r, int sg, float v) { s_part[r * 2 + sg] = v; });
      __syncthreads();
      if (threadIdx.x < QKV_ROWS_WG)
        st_dev_f32(qkv_x + QKV_ROWS_WG * j + threadIdx.x, s_part[threadIdx.x * 2] + s_part[threadIdx.x * 2 + 1]);
    }
    mark(a, tl + 1);
    xcd_barrier(sync);
    mark(a, tl + 2);

    // ---- B: per-head q/k RMSNorm + RoPE, cache write, split-K attention ------------------------
    {
      fetch_dev(qkv_x, s_x, QKV_ROWS_X);  // s_x[0:256) q (2 heads), [256:384) k, [384:512) v
      __syncthreads();
      const uint16_t* cr = a.cos_tab + (size_t)position * D;
      const uint16_t* sr = a.sin_tab + (size_t)position * D;
      if (wave < 3) {
        // wave 0,1: q heads; wave 2: k head. Lane l handles dims l and l+64.
        const float* src = s_x + (wave < 2 ? wave * D : 2 * D);
        const uint16_t* nw = (const uint16_t*)(wave < 2 ? lw.q_norm_weight : lw.k_norm_weight);
        const float t0 = src[lane], t1 = src[lane + 64];
        const float ss = wave_sum(t0 * t0 + t1 * t1);
        const float rs = rsqrtf(ss / (float)D + EPS);
        const float u0 = t0 * rs * bf16_to_f32(nw[lane]);
        const float u1 = t1 * rs * bf16_to_f32(nw[lane + 64]);
        const float o0 = u0 * bf16_to_f32(cr[lane]) - u1 * bf16_to_f32(sr[lane]);
        const float o1 = u1 * bf16_to_f32(cr[lane + 64]) + u0 * bf16_to_f32(sr[lane + 64]);
        if (wave < 2) { s_q[wave][lane] = o0; s_q[wave][lane + 64] = o1; }
        else { s_k[lane] = round_bf16(o0); s_k[lane + 64] = round_bf16(o1); }
      } else if (wave == 3) {
        s_v[lane] = round_bf16(s_x[3 * D + lane]);
        s_v[lane + 64] = round_bf16(s_x[3 * D + lane + 64]);
      }
      __syncthreads();
      const size_t head_base = ((size_t)layer * HKV + xcd) * a.max_seq * D;
      if (j == 0 && threadIdx.x < D) {
        a.k_cache[head_base + (size_t)position * D + threadIdx.x] = f32_to_bf16(s_k[threadIdx.x]);
        a.v_cache[head_base + (size_t)position * D + threadIdx.x] = f32_to_bf16(s_v[threadIdx.x]);
      }
      // positions [p0, p1) of this workgroup; wave w takes p0+w, p0+w+8, ...
      const int p0 = (int)(((long long)ctx * j) / WPX);
      const int p1 = (int)(((long long)ctx * (j + 1)) / WPX);
      const float q00 = s_q[0][2 * lane], q01 = s_q[0][2 * lane + 1];
      const float q10 = s_q[1][2 * lane], q11 = s_q[1][2 * lane + 1];
      float m0 = -INFINITY, m1 = -INFINITY, l0 = 0.f, l1 = 0.f;
      float a00 = 0.f, a01 = 0.f, a10 = 0.f, a11 = 0.f;
      const uint32_t* kc = reinterpret_cast<const uint32_t*>(a.k_cache + head_base);
      const uint32_t* vc = reinterpret_cast<const uint32_t*>(a.v_cache + head_base);
      for (int p = p0 + wave; p < p1; p += NWAVE) {
        float k0, k1, v0, v1;
        if (p == position) {
          k0 = s_k[2 * lane]; k1 = s_k[2 * lane + 1]; v0 = s_v[2 * lane]; v1 = s_v[2 * lane + 1];
        } else {
          const uint32_t kw = kc[(size_t)p * (D / 2) + lane];
          const uint32_t vw = vc[(size_t)p * (D / 2) + lane];
          k0 = bf16_lo(kw); k1 = bf16_hi(kw); v0 = bf16_lo(vw); v1 = bf16_hi(vw);
        }
        const float s0 = wave_sum(q00 * k0 + q01 * k1) * ATT_SCALE;
        const float s1 = wave_sum(q10 * k0 + q11 * k1) * ATT_SCALE;
        const float n0 = fmaxf(m0, s0), n1 = fmaxf(m1, s1);
        const float c0 = expf(m0 - n0), c1 = expf(m1 - n1);
        const float e0 = expf(s0 - n0), e1 = expf(s1 - n1);
        l0 = l0 * c0 + e0; l1 = l1 * c1 + e1;
        a00 = a00 * c0 + e0 * v0; a01 = a01 * c0 + e0 * v1;
        a10 = a10 * c1 + e1 * v0; a11 = a11 * c1 + e1 * v1;
        m0 = n0; m1 = n1;
      }
      // merge the 8 waves' partials in LDS, then publish this workgroup's partial
      s_wpart[wave][0][2 * lane] = a00; s_wpart[wave][0][2 * lane + 1] = a01;
      s_wpart[wave][1][2 * lane] = a10; s_wpart[wave][1][2 * lane + 1] = a11;
      if (lane == 0) { s_wpart[wave][0][D] = m0; s_wpart[wave][0][D + 1] = l0; s_wpart[wave][1][D] = m1; s_wpart[wave][1][D + 1] = l1; }
      __syncthreads();
      if (threadIdx.x < 2 * D) {
        const int h = threadIdx.x / D, d = threadIdx.x % D;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < NWAVE; ++w) M = fmaxf(M, s_wpart[w][h][D]);
        float acc = 0.f, L = 0.f;
        if (M != -INFINITY) {
#pragma unroll
          for (int w = 0; w < NWAVE; ++w) {
            const float mw = s_wpart[w][h][D];
            if (mw != -INFINITY) {
              const float f = expf(mw - M);
              acc += s_wpart[w][h][d] * f;
              L += s_wpart[w][h][D + 1] * f;
            }
          }
        }
        float* dst = apart_x + ((size_t)j * 2 + h) * APS;
        st_dev_f32(dst + d, acc);
        if (d == 0) { st_dev_f32(dst + D, M); st_dev_f32(dst + D + 1, L); }
      }
    }
    mark(a, tl + 3);
    xcd_barrier(sync);
    mark(a, tl + 4);

    // ---- C: merge 32 attention partials, o_proj partial over this group's 256 columns ----------
    {
      if (threadIdx.x < WPX * 2) {
        const int jj = threadIdx.x >> 1, h = threadIdx.x & 1;
        const float* src = apart_x + ((size_t)jj * 2 + h) * APS;
        s_mw[jj][h][0] = ld_dev_f32(src + D);
        s_mw[jj][h][1] = ld_dev_f32(src + D + 1);
      }
      __syncthreads();
      if (threadIdx.x < 2 * D) {
        const int h = threadIdx.x / D, d = threadIdx.x % D;
        float M = -INFINITY;
        for (int jj = 0; jj < WPX; ++jj) M = fmaxf(M, s_mw[jj][h][0]);
        float acc = 0.f, L = 0.f;
        for (int jj = 0; jj < WPX; ++jj) {
          const float mj = s_mw[jj][h][0];
          if (mj != -INFINITY) {
            const float f = expf(mj - M);
            acc += ld_dev_f32(apart_x + ((size_t)jj * 2 + h) * APS + d) * f;
            L += s_mw[jj][h][1] * f;
          }
        }
        s_x[h * D + d] = acc / L;
      }
      __syncthreads();
      const uint16_t* wo = (const uint16_t*)lw.o_proj_weight;
      const int row0 = HPW * j;
      gemv<2 * D, 1>(HPW, [&](int r) { return wo + (size_t)(row0 + r) * (HQ * D) + 2 * D * xcd; }, s_x,
                     [&](int r, int, float v) { st_dev_f32(opart + (size_t)xcd * H + row0 + r, v); });
    }
    mark(a, tl + 5);
    grid_barrier(sync);
    mark(a, tl + 6);

    // ---- D: residual += o_proj, post-attention RMSNorm, gate/up rows of slice x ---------------
    add_partials<H>(s_res, opart);
    rms_norm<H>(s_res, (const uint16_t*)lw.post_attn_norm_weight, s_x, s_red);
    {
      const uint16_t* wg = (const uint16_t*)lw.gate_proj_weight;
      const uint16_t* wu = (const uint16_t*)lw.up_proj_weight;
      const int row0 = IX * xcd + IPW * j;
      gemv<H, GU_S>(2 * IPW,
                    [&](int r) { return (r < IPW ? wg + (size_t)(row0 + r) * H : wu + (size_t)(row0 + r - IPW) * H); },
                    s_x, [&](int r, int sg, float v) { s_part[r * GU_S + sg] = v; });
      __syncthreads();
      if (threadIdx.x < IPW) {
        float g = 0.f, u = 0.f;
#pragma unroll
        for (int sg = 0; sg < GU_S; ++sg) { g += s_part[threadIdx.x * GU_S + sg]; u += s_part[(threadIdx.x + IPW) * GU_S + sg]; }
        const float m = g / (1.f + expf(-g)) * u;  // silu(g) * u, /root/reference/config.cuh:177-179
        st_dev_f32(mbuf_x + IPW * j + threadIdx.x, m);
      }
    }
    mark(a, tl + 7);
    xcd_barrier(sync);
    mark(a, tl + 8);

    // ---- E: down_proj partial over slice x's columns ------------------------------------------
    {
      fetch_dev(mbuf_x, s_x, IX);
      __syncthreads();
      const uint16_t* wd = (const uint16_t*)lw.down_proj_weight;
      const int row0 = HPW * j;
      gemv<IX, 1>(HPW, [&](int r) { return wd + (size_t)(row0 + r) * I + IX * xcd; }, s_x,
                  [&](int r, int, float v) { st_dev_f32(dpart + (size_t)xcd * H + row0 + r, v); });
    }
    mark(a, tl + 9);
    grid_barrier(sync);
  }

  // ---- final RMSNorm, tied LM head, argmax ------------------------------------------------------
  mark(a, tb + 1);
  add_partials<H>(s_res, dpart);
  rms_norm<H>(s_res, a.final_norm, s_x, s_red);
  mark(a, tb + 2);
  {
    const int r0 = (int)(((long long)a.vocab * blockIdx.x) / NWG);
    const int r1 = (int)(((long long)a.vocab * (blockIdx.x + 1)) / NWG);
    unsigned long long best = 0;
    gemv<H, 1>(r1 - r0, [&](int r) { return a.lm_head + (size_t)(r0 + r) * H; }, s_x, [&](int r, int, float v) {
      a.logits[r0 + r] = v;
      const unsigned long long k = argmax_key(v, r0 + r);
      best = k > best ? k : best;
    });
    // workgroup max of the per-thread keys (only group leaders hold non-zero keys)
    unsigned long long* s_best = reinterpret_cast<unsigned long long*>(s_wpart);
    for (int off = 32; off >= 1; off >>= 1) {
      const unsigned long long o = __shfl_xor(best, off);
      best = o > best ? o : best;
    }
    if (lane == 0) s_best[wave] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
      unsigned long long b = 0;
      for (int w = 0; w < NWAVE; ++w) b = s_best[w] > b ? s_best[w] : b;
      __hip_atomic_fetch_max(reinterpret_cast<unsigned long long*>(a.ctr + L_AMAX * CTR_LINE), b,
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }

  mark(a, tb + 3);
  // ---- exit: the last workgroup out publishes the token and resets the counters ---------------
  wait_vmem();
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t old = __hip_atomic_fetch_add(a.ctr + (L_XEXIT + xcd) * CTR_LINE, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (old == WPX - 1) {
      old = __hip_atomic_fetch_add(a.ctr + L_GEXIT * CTR_LINE, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (old == NXCD - 1) {
        unsigned long long* amax = reinterpret_cast<unsigned long long*>(a.ctr + L_AMAX * CTR_LINE);
        const unsigned long long b = __hip_atomic_load(amax, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (a.out_token) *a.out_token = b ? (int32_t)(0xffffffffu - (uint32_t)(b & 0xffffffffu)) : -1;
        __hip_atomic_store(amax, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        for (int x = 0; x < NXCD; ++x) {
          st_dev_u32(a.ctr + (L_XL + x) * CTR_LINE, 0u);
          st_dev_u32(a.ctr + (L_XG + x) * CTR_LINE, 0u);
          st_dev_u32(a.ctr + (L_XEXIT + x) * CTR_LINE, 0u);
        }
        st_dev_u32(a.ctr + L_G * CTR_LINE, 0u);
        st_dev_u32(a.ctr + L_GEXIT * CTR_LINE, 0u);
      }
    }
  }
}

// ------------------------------------------------------------------------------------------
// Host side: per-device workspace and launch
// ------------------------------------------------------------------------------------------
struct DeviceState {
  bool init = false;
  bool ok = false;
  void* ws = nullptr;
  uint64_t* trace = nullptr;  // set by mk_set_trace; null in normal operation
};
constexpr int MAX_DEVICES = 64;
static DeviceState g_dev[MAX_DEVICES];
static std::mutex g_mu;

template <int H, int I>
static hipError_t check_kernel_fits() {
  int blocks = 0;
  hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, (const void*)decode_kernel<H, I>, NT, 0);
  if (e != hipSuccess) return e;
  return blocks >= 1 ? hipSuccess : hipErrorCooperativeLaunchTooLarge;
}

static hipError_t device_state(DeviceState** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= MAX_DEVICES) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lk(g_mu);
  DeviceState& s = g_dev[dev];
  if (!s.init) {
    s.init = true;
    int cus = 0, coop = 0;
    if ((e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev)) != hipSuccess) return e;
    if ((e = hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev)) != hipSuccess) return e;
    if (cus != NWG || !coop) return hipErrorNotSupported;
    if ((e = check_kernel_fits<1024, 3072>()) != hipSuccess) return e;
    if ((e = check_kernel_fits<2048, 6144>()) != hipSuccess) return e;
    if ((e = hipMalloc(&s.ws, WS_BYTES)) != hipSuccess) return e;
    if ((e = hipMemset(s.ws, 0, WS_BYTES)) != hipSuccess) return e;
    if ((e = hipDeviceSynchronize()) != hipSuccess) return e;
    s.ok = true;
  }
  if (!s.ok) return hipErrorNotSupported;
  *out = &s;
  return hipSuccess;
}

template <int H, int I>
static hipError_t launch(KArgs& k, hipStream_t stream) {
  void* args[] = {(void*)&k};
  return hipLaunchCooperativeKernel((const void*)decode_kernel<H, I>, dim3(NWG), dim3(NT), args, 0, stream);
}

}  // namespace mk

using namespace mk;

extern "C" hipError_t mk_decode(const mk_model_dims* dims, int token_id, const void* embed_weight,
                                const void* lm_head_weight, const void* final_norm_weight,
                                const void* layer_weights, const void* cos_table, const void* sin_table,
                                void* k_cache, void* v_cache, int position, int max_seq_len, float* logits,
                                int32_t* out_token, hipStream_t stream) {
  if (!dims || !embed_weight || !lm_head_weight || !final_norm_weight || !layer_weights || !cos_table ||
      !sin_table || !k_cache || !v_cache || !logits)
    return hipErrorInvalidValue;
  const bool s06 = dims->hidden == 1024 && dims->intermediate == 3072;
  const bool s17 = dims->hidden == 2048 && dims->intermediate == 6144;
  if (!(s06 || s17) || dims->num_layers < 1 || dims->vocab < NWG) return hipErrorInvalidValue;
  if (token_id < 0 || token_id >= dims->vocab) return hipErrorInvalidValue;
  if (max_seq_len < 1 || position < 0 || position >= max_seq_len) return hipErrorInvalidValue;
  DeviceState* st = nullptr;
  hipError_t e = device_state(&st);
  if (e != hipSuccess) return e;
  KArgs k;
  k.embed = (const uint16_t*)embed_weight;
  k.lm_head = (const uint16_t*)lm_head_weight;
  k.final_norm = (const uint16_t*)final_norm_weight;
  k.layers = (const mk_layer_weights*)layer_weights;
  k.cos_tab = (const uint16_t*)cos_table;
  k.sin_tab = (const uint16_t*)sin_table;
  k.k_cache = (uint16_t*)k_cache;
  k.v_cache = (uint16_t*)v_cache;
  k.logits = logits;
  k.out_token = out_token;
  k.ws = (float*)st->ws;
  k.ctr = (uint32_t*)((char*)st->ws + WS_FLOATS * 4);
  k.trace = st->trace;
  k.token = token_id;
  k.position = position;
  k.max_seq = max_seq_len;
  k.num_layers = dims->num_layers;
  k.vocab = dims->vocab;
  return s06 ? launch<1024, 3072>(k, stream) : launch<2048, 6144>(k, stream);
}

extern "C" hipError_t launch_decode_kernel(int token_id, const void* embed_weight, const void* lm_head_weight,
                                           const void* final_norm_weight, const void* layer_weights,
                                           const void* cos_table, const void* sin_table, void* k_cache,
                                           void* v_cache, void* hidden_buffer, void* g_residual,
                                           void* g_activations, void* g_attn_output, void* g_normalized,
                                           void* g_mlp_intermediate, void* g_logits, void* g_q, void* g_k,
                                           void* g_v, int position, int cache_len, int max_seq_len,
                                           hipStream_t stream) {
  (void)hidden_buffer; (void)g_residual; (void)g_activations; (void)g_attn_output; (void)g_normalized;
  (void)g_mlp_intermediate; (void)g_q; (void)g_k; (void)g_v;
  if (cache_len != position + 1) return hipErrorInvalidValue;
  const mk_model_dims dims = {1024, 3072, 28, 151936};
  return mk_decode(&dims, token_id, embed_weight, lm_head_weight, final_norm_weight, layer_weights, cos_table,
                   sin_table, k_cache, v_cache, position, max_seq_len, (float*)g_logits, nullptr, stream);
}

extern "C" hipError_t mk_status(uint32_t* status) {
  if (!status) return hipErrorInvalidValue;
  DeviceState* st = nullptr;
  hipError_t e = device_state(&st);
  if (e != hipSuccess) return e;
  if ((e = hipDeviceSynchronize()) != hipSuccess) return e;
  return hipMemcpy(status, (char*)st->ws + WS_FLOATS * 4 + (size_t)L_STATUS * CTR_LINE * 4, 4, hipMemcpyDeviceToHost);
}

extern "C" hipError_t mk_reset(void) {
  DeviceState* st = nullptr;
  hipError_t e = device_state(&st);
  if (e != hipSuccess) return e;
  if ((e = hipDeviceSynchronize()) != hipSuccess) return e;
  if ((e = hipMemset((char*)st->ws + WS_FLOATS * 4, 0, (size_t)N_LINES * CTR_LINE * 4)) != hipSuccess) return e;
  return hipDeviceSynchronize();
}

extern "C" hipError_t mk_set_trace(uint64_t* device_buffer, size_t bytes) {
  DeviceState* st = nullptr;
  hipError_t e = device_state(&st);
  if (e != hipSuccess) return e;
  if (device_buffer != nullptr && bytes < (size_t)NWG * TRACE_N * sizeof(uint64_t)) return hipErrorInvalidValue;
  st->trace = device_buffer;
  return hipSuccess;
}

extern "C" size_t mk_trace_bytes(void) { return (size_t)NWG * TRACE_N * sizeof(uint64_t); }

extern "C" int mk_grid_size(void) {
  DeviceState* st = nullptr;
  return device_state(&st) == hipSuccess ? NWG : -1;
}

extern "C" const char* mk_version(void) { return "megakernel_amd 0.1 (gfx950, xcd-aware v1)"; }
