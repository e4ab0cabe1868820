// Persistent cooperative decode kernel for Qwen3-shaped models on MI355X (gfx950), plus its C ABI.
//
// One launch = one decode step for batch 1: embedding -> L x {RMSNorm, QKV, per-head norm + RoPE,
// K/V cache write, split-K GQA attention, O-proj + residual, RMSNorm, gate/up + SiLU, down +
// residual} -> final RMSNorm -> tied LM head -> greedy argmax. This is the work of the reference's
// decode_kernel (/root/reference/megakernel.cu:744-893), re-planned for 256 CUs in 8 XCDs.
//
// Placement. One 512-thread workgroup per CU. Workgroup b runs on XCD x = b % 8 as local
// workgroup j = b / 8 (the dispatcher's round-robin placement; every workgroup checks its
// HW_REG_XCC_ID and reports a mismatch in the status word). XCD x owns K/V head x -- the 512
// Q/K/V rows of that group, its attention and its 256 columns of o_proj -- plus a 1/8 slice of
// the MLP intermediate, so within a layer only two exchanges leave the XCD.
//
// Roles. Wave 0 of every workgroup is the communication wave: it waits for other workgroups'
// results, moves exchanged vectors, and does the vector work (RMSNorm, q/k norm + RoPE,
// attention merges, SiLU). Waves 1-7 are math waves: they stream weights and K/V with 16-byte
// loads issued about two phases ahead, and compute dot products from LDS inputs. Splitting the
// roles keeps the math waves' prefetch queue from stalling the polling wave (vector-memory
// completion is counted in order per wave).
//
// Exchanges (no atomics). A producer writes data, waits for its stores, then writes a flag word
// holding the launch epoch; a consumer polls the flags with device-scope loads.
//   * within an XCD (QKV -> attention, attention partials, SiLU(g)*u): plain stores land in the
//     XCD's shared L2 and device-scope loads read them there;
//   * across XCDs (o_proj and down_proj partial sums): workgroup j of XCD y writes its row block
//     j through to memory (device scope); workgroup j of every XCD gathers block j from the 8
//     XCDs, sums it in XCD order and republishes it into its own XCD's L2; then every workgroup
//     reads the full vector from its L2. Two short hops, at most 8 pollers per cross-XCD line.
//
// Numerics follow the reference kernel's fp32 design: bf16 weights and cache, fp32 activations
// and accumulation, fp32 RMSNorm, exact softmax, new K/V rounded to bf16 as stored. Logits are
// fp32; the greedy token is the argmax of the bf16-rounded logits, lowest index on ties. The
// residual stream is kept redundantly in every workgroup's LDS and updated from the same data
// in the same order, so all copies are bitwise identical.
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
constexpr int NMW = 7;        // math waves (1..7)
constexpr int MG = NMW * 4;   // 16-lane math groups
constexpr int QKV_X = 4 * D;  // q (2 heads) + k + v rows owned by one XCD
constexpr int QKV_WG = QKV_X / WPX;  // 16
constexpr int APS = 132;      // floats per head in an attention partial: acc[128], m, l, pad
constexpr int APF = 5;        // K/V positions per math wave loaded ahead of the attention phase
constexpr float EPS = 1e-6f;
constexpr float ATT_SCALE = 0.08838834764831845f;  // 128 ** -0.5
constexpr uint32_t SPIN_LIMIT = 1u << 22;
constexpr uint32_t ERR_TIMEOUT = 1u;
constexpr uint32_t ERR_PLACEMENT = 2u;
constexpr int MAX_LAYERS = 62;  // epoch = seq << 6 | layer; 63 marks the final exchange

// Workspace layout: float buffers, then 256-byte flag lines.
constexpr int MAX_H = 2048, MAX_I = 6144, MAX_IX = MAX_I / NXCD, MAX_HPW = MAX_H / WPX;
constexpr size_t W_QKV = 0;                                       // [8][512]
constexpr size_t W_ATT = W_QKV + NXCD * QKV_X;                    // [8][32][2*APS]
constexpr size_t W_M = W_ATT + (size_t)NXCD * WPX * 2 * APS;      // [8][MAX_IX]
constexpr size_t W_LC = W_M + (size_t)NXCD * MAX_IX;              // [8][MAX_H]
constexpr size_t W_LE = W_LC + (size_t)NXCD * MAX_H;              // [8][MAX_H]
constexpr size_t W_GC = W_LE + (size_t)NXCD * MAX_H;              // [32][8][MAX_HPW]
constexpr size_t W_GE = W_GC + (size_t)WPX * NXCD * MAX_HPW;      // [32][8][MAX_HPW]
constexpr size_t WS_FLOATS = W_GE + (size_t)WPX * NXCD * MAX_HPW;
// Flags, in u32 words after the float buffers. A local flag line (256 B) holds the 32 flags of
// one XCD's workgroups -- all its writers share that XCD's L2. Every flag or value written across
// XCDs gets a 128-byte slot of its own, so no cache line has writers on two XCDs.
constexpr int LINE = 64;  // u32 per local flag line (256 B)
constexpr int SLOT = 32;  // u32 per cross-XCD slot (128 B)
enum LocalFlag { F_QKV = 0, F_ATT = 1, F_M = 2, F_LC = 3, F_LE = 4, N_LOCAL = 5 };
constexpr size_t FL_LOCAL = 0;                                     // [type][x] lines
constexpr size_t FL_CROSS = FL_LOCAL + (size_t)N_LOCAL * NXCD * LINE;  // [kind C/E][j][y] slots
constexpr size_t FL_DONE = FL_CROSS + (size_t)2 * WPX * NXCD * SLOT;  // [wg] slots: flag, pad, key u64
constexpr size_t FL_STATUS = FL_DONE + (size_t)NWG * SLOT;         // own line
constexpr size_t FL_SEQ = FL_STATUS + LINE;                        // own line
constexpr size_t FL_WORDS = FL_SEQ + LINE;
__host__ __device__ constexpr size_t fl_local(int type, int x) { return FL_LOCAL + ((size_t)type * NXCD + x) * LINE; }
__host__ __device__ constexpr size_t fl_cross(int kind, int j, int y) { return FL_CROSS + (((size_t)kind * WPX + j) * NXCD + y) * SLOT; }
__host__ __device__ constexpr size_t fl_done(int wg) { return FL_DONE + (size_t)wg * SLOT; }
constexpr size_t WS_BYTES = WS_FLOATS * 4 + FL_WORDS * 4;

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
  uint32_t* fl;     // flag lines
  uint64_t* trace;  // optional: per-workgroup phase timestamps (TRACE_N per workgroup)
  int token, position, max_seq, num_layers, vocab;
};

// Phase timestamps (s_memrealtime, 100 MHz), TRACE_PER_LAYER slots per layer: for phase p in A..E,
// [2p] when the phase's math starts and [2p + 1] when its outputs are published; [10 + k] when the
// communication wave finishes its k-th wait of the layer (QKV, attention partials, cross o_proj,
// local o_proj, MLP, cross down, local down). TRACE_TAIL slots after the layers: kernel start,
// last exchange done, LM-head start and end.
constexpr int TRACE_LAYERS = 64;
constexpr int TRACE_PER_LAYER = 20;
constexpr int TRACE_TAIL = 8;
constexpr int TRACE_N = TRACE_LAYERS * TRACE_PER_LAYER + TRACE_TAIL;
__device__ __forceinline__ void mark(const KArgs& a, int idx) {
  if (a.trace != nullptr && threadIdx.x == 0 && idx >= 0 && idx < TRACE_N)
    a.trace[(size_t)blockIdx.x * TRACE_N + idx] = wall_clock64();
}

// ------------------------------------------------------------------------------------------
// Communication-wave helpers (called by wave 0 only; every lane participates)
// ------------------------------------------------------------------------------------------
struct Comm {
  uint32_t* status;
  bool failed = false;
};

// Plain store: stays in this XCD's L2 until written back; visible to device-scope loads from the
// same XCD.
__device__ __forceinline__ void st_local_f32(float* p, float v) {
  __hip_atomic_store(reinterpret_cast<uint32_t*>(p), __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void st_local_u32(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
// All earlier stores of this wave are complete before anything after this point is issued.
__device__ __forceinline__ void store_fence() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  wait_vmem();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Wait until flags[0], flags[stride], ... flags[(n-1)*stride] all equal ep (n <= 64). Bounded;
// on timeout sets the status word.
__device__ __forceinline__ void poll_flags(Comm& c, const uint32_t* flags, int n, uint32_t ep, int stride = 1) {
  if (c.failed) return;
  const int lane = threadIdx.x & 63;
  for (uint32_t it = 0;; ++it) {
    const uint32_t v = lane < n ? ld_dev_u32(flags + lane * stride) : ep;
    if (__ballot(v != ep) == 0) return;
    if ((it & 63u) == 63u && ld_dev_u32(c.status) != 0) { c.failed = true; return; }
    if (it > SPIN_LIMIT) {
      if (lane == 0) st_dev_u32(c.status, ERR_TIMEOUT);
      c.failed = true;
      return;
    }
  }
}

// s_res[i] += delta[i] (device-scope reads; delta may be null), then s_x = RMSNorm(s_res) * w in
// fp32, the reference's form x * w * rsqrt(mean(x^2) + eps) (/root/reference/megakernel.cu:704-739).
// Lane l owns the H/64 contiguous elements starting at l*H/64.
template <int H>
__device__ __forceinline__ void comm_residual_norm(float* s_res, const float* delta, const uint16_t* w, float* s_x) {
  constexpr int E = H / 64;
  const int lane = threadIdx.x & 63;
  float v[E];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < E; k += 4) {
    float4 r = *reinterpret_cast<const float4*>(s_res + lane * E + k);
    if (delta != nullptr) {
      const float4 d = ld_dev_f32x4(delta, (lane * E + k) * 4);
      r.x += d.x; r.y += d.y; r.z += d.z; r.w += d.w;
      *reinterpret_cast<float4*>(s_res + lane * E + k) = r;
    }
    v[k] = r.x; v[k + 1] = r.y; v[k + 2] = r.z; v[k + 3] = r.w;
  }
#pragma unroll
  for (int k = 0; k < E; ++k) ss += v[k] * v[k];
  ss = wave_sum(ss);
  const float rs = rsqrtf(ss / (float)H + EPS);
  const uint4* wp = reinterpret_cast<const uint4*>(w + lane * E);
#pragma unroll
  for (int k = 0; k < E; k += 8) {
    const uint4 ww = ld_global16(wp + k / 8);
    const float wv[8] = {bf16_lo(ww.x), bf16_hi(ww.x), bf16_lo(ww.y), bf16_hi(ww.y),
                         bf16_lo(ww.z), bf16_hi(ww.z), bf16_lo(ww.w), bf16_hi(ww.w)};
#pragma unroll
    for (int q = 0; q < 8; ++q) s_x[lane * E + k + q] = v[k + q] * wv[q] * rs;
  }
}

// ------------------------------------------------------------------------------------------
// Math-wave helpers. A phase's weight tile is cut into units of 16 chunks (256 contiguous
// bytes of one row); math group g (16 lanes) owns units g, g+28, g+56, ...; lane t of the group
// loads chunk t of each unit. Unit u covers row u / UPR, column block u % UPR (128 elements).
// ------------------------------------------------------------------------------------------
// Loads are unconditional (a lane past the tile re-reads the tile's last unit): a conditional
// load becomes a branch whose join forces the wave to wait for every outstanding load, which
// would serialize the phase and drain the prefetch of later phases.
template <int NU, int UPR, typename Ptr>
__device__ __forceinline__ void load_units(uint4 (&w)[NU], int k0, int U, int g, int t, Ptr ptr) {
#pragma unroll
  for (int k = 0; k < NU; ++k) {
    int u = g + MG * (k0 + k);
    u = u < U ? u : U - 1;
    w[k] = ld_stream(ptr(u / UPR, u % UPR) + t);
  }
}

template <int NU, int UPR>
__device__ __forceinline__ void dot_units(const uint4 (&w)[NU], int k0, int U, int g, int t, const float* x, float* s_up) {
#pragma unroll
  for (int k = 0; k < NU; ++k) {
    const int u = g + MG * (k0 + k);
    const int uc = u < U ? u : U - 1;
    float acc = dot8(w[k], x + (uc % UPR) * 128 + t * 8, 0.f);
    acc = row16_sum(acc);
    if (t == 0 && u < U) s_up[u] = acc;
  }
}

// A GEMV phase whose first PFN units per lane were loaded ahead (pf); the rest stream here.
template <int NU, int PFN, int UPR, typename Ptr>
__device__ __forceinline__ void gemv_phase(const uint4 (&pf)[PFN], int U, int g, int t, Ptr ptr, const float* x, float* s_up) {
  dot_units<PFN, UPR>(pf, 0, U, g, t, x, s_up);
#pragma unroll
  for (int k0 = PFN; k0 < NU; k0 += PFN) {
    uint4 w[PFN];
    load_units<PFN, UPR>(w, k0, U, g, t, ptr);
    dot_units<PFN, UPR>(w, k0, U, g, t, x, s_up);
  }
}

__device__ __forceinline__ unsigned long long argmax_key(float logit, int idx) {
  // order-preserving map of the bf16-rounded logit, then the complemented index so that equal
  // values prefer the lower index under an unsigned max
  uint32_t u = (uint32_t)f32_to_bf16(logit) << 16;
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((unsigned long long)u << 32) | (0xffffffffu - (uint32_t)idx);
}

__device__ __forceinline__ unsigned long long umax64(unsigned long long a, unsigned long long b) { return a > b ? a : b; }

// Returns v unchanged but hides its origin from the optimizer, so per-unit indices derived from it
// are recomputed inside each phase instead of being hoisted out of the layer loop and held in
// registers for the whole kernel.
__device__ __forceinline__ int opaque(int v) {
  asm volatile("" : "+v"(v));
  return v;
}

// ------------------------------------------------------------------------------------------
// The kernel
// ------------------------------------------------------------------------------------------
template <int H, int I>
__global__ void __launch_bounds__(NT, 1) decode_kernel(const KArgs a) {
  constexpr int IX = I / NXCD;     // MLP intermediate slice per XCD
  constexpr int IPW = IX / WPX;    // gate (and up) rows per workgroup
  constexpr int HPW = H / WPX;     // o_proj / down_proj rows per workgroup
  constexpr int UPR_H = H / 128, UPR_C = 2 * D / 128, UPR_E = IX / 128;
  constexpr int U_A = QKV_WG * UPR_H, U_C = HPW * UPR_C, U_D = 2 * IPW * UPR_H, U_E = HPW * UPR_E;
  constexpr int NU_A = (U_A + MG - 1) / MG, NU_C = (U_C + MG - 1) / MG;
  constexpr int NU_D = (U_D + MG - 1) / MG, NU_E = (U_E + MG - 1) / MG;
  constexpr int PF = H <= 1024 ? 8 : 4;  // max 16-byte chunks per lane loaded ahead of a GEMV phase
  constexpr int PA = NU_A < PF ? NU_A : PF, PC = NU_C < PF ? NU_C : PF;
  constexpr int PD = NU_D < PF ? NU_D : PF, PE = NU_E < PF ? NU_E : PF;
  constexpr int XN = (H > IX ? H : IX);
  constexpr int UMAX = (U_D > U_A ? U_D : U_A) > U_E ? (U_D > U_A ? U_D : U_A) : U_E;
  static_assert(HPW * WPX == H && IPW * WPX == IX && IX * NXCD == I, "shape must split evenly");
  static_assert(IX % 128 == 0 && H % 512 == 0 && HPW <= 64 && IPW <= 64, "unsupported shape");

  __shared__ __attribute__((aligned(16))) float s_res[H];
  __shared__ __attribute__((aligned(16))) float s_x[XN];
  __shared__ __attribute__((aligned(16))) float s_up[UMAX];
  __shared__ __attribute__((aligned(16))) float s_q[2][D];
  __shared__ __attribute__((aligned(16))) float s_k[D];
  __shared__ __attribute__((aligned(16))) float s_v[D];
  __shared__ __attribute__((aligned(16))) float s_wp[NMW][2][D + 2];
  __shared__ unsigned long long s_best[NMW];

  const int xcd = blockIdx.x % NXCD;
  const int j = blockIdx.x / NXCD;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const bool comm = wave == 0;
  const int g = comm ? 0 : (wave - 1) * 4 + (lane >> 4);  // math group
  const int t = lane & 15;

  float* ws = a.ws;
  uint32_t* fl = a.fl;
  Comm c;
  c.status = fl + FL_STATUS;
  const int position = a.position;
  const int ctx = position + 1;
  const int L = a.num_layers;

  // Split-K attention: the context is cut into S = min(32, ceil(ctx / 32)) splits handled by local
  // workgroups 0..S-1; math wave w of a split takes positions p0 + w, p0 + w + 7, ...
  const int S = ctx >= WPX * 32 ? WPX : (ctx + 31) / 32;
  const int p0 = j < S ? (int)(((long long)ctx * j) / S) : 0;
  const int p1 = j < S ? (int)(((long long)ctx * (j + 1)) / S) : 0;
  const int mw = wave - 1;
  const int np_w = (!comm && p1 - p0 > mw) ? (p1 - p0 - mw + NMW - 1) / NMW : 0;

  // ---- per-phase weight tiles (unit (r, b) starts at chunk 16*b of tile row r) -------------
  auto ptr_A = [&](const mk_layer_weights& lw) {
    const uint16_t* base;
    int row0;
    if (j < 16) { base = (const uint16_t*)lw.q_weight; row0 = 2 * D * xcd + QKV_WG * j; }
    else if (j < 24) { base = (const uint16_t*)lw.k_weight; row0 = D * xcd + QKV_WG * (j - 16); }
    else { base = (const uint16_t*)lw.v_weight; row0 = D * xcd + QKV_WG * (j - 24); }
    return [=](int r, int b) { return reinterpret_cast<const uint4*>(base + (size_t)(row0 + r) * H) + 16 * b; };
  };
  auto ptr_C = [&](const mk_layer_weights& lw) {
    const uint16_t* wo = (const uint16_t*)lw.o_proj_weight;
    const int row0 = HPW * j;
    return [=](int r, int b) {
      return reinterpret_cast<const uint4*>(wo + (size_t)(row0 + r) * (HQ * D) + 2 * D * xcd) + 16 * b;
    };
  };
  auto ptr_D = [&](const mk_layer_weights& lw) {
    const uint16_t* wg = (const uint16_t*)lw.gate_proj_weight;
    const uint16_t* wu = (const uint16_t*)lw.up_proj_weight;
    const int row0 = IX * xcd + IPW * j;
    return [=](int r, int b) {
      const uint16_t* row = r < IPW ? wg + (size_t)(row0 + r) * H : wu + (size_t)(row0 + r - IPW) * H;
      return reinterpret_cast<const uint4*>(row) + 16 * b;
    };
  };
  auto ptr_E = [&](const mk_layer_weights& lw) {
    const uint16_t* wd = (const uint16_t*)lw.down_proj_weight;
    const int row0 = HPW * j;
    return [=](int r, int b) { return reinterpret_cast<const uint4*>(wd + (size_t)(row0 + r) * I + IX * xcd) + 16 * b; };
  };

  // K/V of the first APF positions of this math wave, loaded ahead of the attention phase
  uint32_t kv_k[APF], kv_v[APF];
  auto load_kv = [&](int layer) {
    const size_t hb = ((size_t)layer * HKV + xcd) * a.max_seq * D;
    const uint32_t* kc = reinterpret_cast<const uint32_t*>(a.k_cache + hb);
    const uint32_t* vc = reinterpret_cast<const uint32_t*>(a.v_cache + hb);
#pragma unroll
    for (int i = 0; i < APF; ++i) {
      // unconditional (see load_units); positions outside [p0, p1) or the new one are not used
      int p = p0 + mw + NMW * i;
      p = (i < np_w && p != position) ? p : 0;
      kv_k[i] = gp(kc)[(size_t)p * (D / 2) + lane];
      kv_v[i] = gp(vc)[(size_t)p * (D / 2) + lane];
    }
  };

  uint4 wA[PA], wC[PC], wD[PD], wE[PE];
  uint32_t seq = 0;
  float cs_c0 = 0.f, cs_c1 = 0.f, cs_s0 = 0.f, cs_s1 = 0.f;  // comm: cos/sin at dims lane, lane+64

  mark(a, TRACE_LAYERS * TRACE_PER_LAYER + 0);
  if (comm) {
    seq = ld_dev_u32(fl + FL_SEQ);
    if (xcc_id() != (unsigned)xcd && lane == 0) st_dev_u32(c.status, ERR_PLACEMENT);
    const uint16_t* row = a.embed + (size_t)a.token * H;
    for (int i = lane; i < H; i += 64) s_res[i] = bf16_to_f32(gp(row)[i]);
    const uint16_t* cr = a.cos_tab + (size_t)position * D;
    const uint16_t* sr = a.sin_tab + (size_t)position * D;
    cs_c0 = bf16_to_f32(gp(cr)[lane]); cs_c1 = bf16_to_f32(gp(cr)[lane + 64]);
    cs_s0 = bf16_to_f32(gp(sr)[lane]); cs_s1 = bf16_to_f32(gp(sr)[lane + 64]);
    comm_residual_norm<H>(s_res, nullptr, (const uint16_t*)a.layers[0].norm_weight, s_x);
  } else {
    const mk_layer_weights lw0 = a.layers[0];
    load_units<PA, UPR_H>(wA, 0, U_A, g, t, ptr_A(lw0));
  }
  __syncthreads();

  for (int layer = 0; layer < L; ++layer) {
    const mk_layer_weights lw = a.layers[layer];
    const uint32_t ep = (seq << 6) | (uint32_t)layer;
    const int tl = layer < TRACE_LAYERS ? layer * TRACE_PER_LAYER : -1000000;
    float* qkv_x = ws + W_QKV + xcd * QKV_X;
    float* att_x = ws + W_ATT + (size_t)xcd * WPX * 2 * APS;
    float* m_x = ws + W_M + xcd * IX;
    float* lc_x = ws + W_LC + xcd * H;
    float* le_x = ws + W_LE + xcd * H;

    // ---- A: QKV rows of this XCD's group -------------------------------------------------
    mark(a, tl + 0);
    if (!comm) {
      const int gq = opaque(g), tq = opaque(t);
      load_units<PC, UPR_C>(wC, 0, U_C, gq, tq, ptr_C(lw));
      load_kv(layer);
      gemv_phase<NU_A, PA, UPR_H>(wA, U_A, gq, tq, ptr_A(lw), s_x, s_up);
    }
    __syncthreads();
    if (comm) {
      if (lane < QKV_WG) {
        float s = 0.f;
#pragma unroll
        for (int b = 0; b < UPR_H; ++b) s += s_up[lane * UPR_H + b];
        st_local_f32(qkv_x + QKV_WG * j + lane, s);
      }
      store_fence();
      mark(a, tl + 1);
      if (lane == 0) st_local_u32(fl + fl_local(F_QKV, xcd) + j, ep);
      poll_flags(c, fl + fl_local(F_QKV, xcd), WPX, ep);
      mark(a, tl + 10);
      // q heads 2x, 2x+1 at [0, 256), k head x at [256, 384), v head x at [384, 512)
      float t0[3], t1[3];
#pragma unroll
      for (int h = 0; h < 3; ++h) {
        t0[h] = ld_dev_f32(qkv_x + h * D + lane);
        t1[h] = ld_dev_f32(qkv_x + h * D + lane + 64);
      }
      const float v0 = ld_dev_f32(qkv_x + 3 * D + lane), v1 = ld_dev_f32(qkv_x + 3 * D + lane + 64);
      const uint16_t* qn = (const uint16_t*)lw.q_norm_weight;
      const uint16_t* kn = (const uint16_t*)lw.k_norm_weight;
#pragma unroll
      for (int h = 0; h < 3; ++h) {
        // per-head RMSNorm then rotate-half RoPE (/root/reference/megakernel.cu:490-630)
        const uint16_t* nw = h < 2 ? qn : kn;
        const float rs = rsqrtf(wave_sum(t0[h] * t0[h] + t1[h] * t1[h]) / (float)D + EPS);
        const float u0 = t0[h] * rs * bf16_to_f32(gp(nw)[lane]);
        const float u1 = t1[h] * rs * bf16_to_f32(gp(nw)[lane + 64]);
        const float o0 = u0 * cs_c0 - u1 * cs_s0;
        const float o1 = u1 * cs_c1 + u0 * cs_s1;
        if (h < 2) { s_q[h][lane] = o0; s_q[h][lane + 64] = o1; }
        else { s_k[lane] = round_bf16(o0); s_k[lane + 64] = round_bf16(o1); }
      }
      s_v[lane] = round_bf16(v0);
      s_v[lane + 64] = round_bf16(v1);
      if (j == 0) {
        const size_t slot = (((size_t)layer * HKV + xcd) * a.max_seq + position) * D;
        gpw(a.k_cache)[slot + lane] = f32_to_bf16(s_k[lane]);
        gpw(a.k_cache)[slot + lane + 64] = f32_to_bf16(s_k[lane + 64]);
        gpw(a.v_cache)[slot + lane] = f32_to_bf16(v0);
        gpw(a.v_cache)[slot + lane + 64] = f32_to_bf16(v1);
      }
    }
    __syncthreads();

    // ---- B: split-K attention over this workgroup's positions ----------------------------
    mark(a, tl + 2);
    if (!comm) {
      load_units<PD, UPR_H>(wD, 0, U_D, opaque(g), opaque(t), ptr_D(lw));
      const float q00 = s_q[0][2 * lane], q01 = s_q[0][2 * lane + 1];
      const float q10 = s_q[1][2 * lane], q11 = s_q[1][2 * lane + 1];
      float m0 = -INFINITY, m1 = -INFINITY, l0 = 0.f, l1 = 0.f;
      float a00 = 0.f, a01 = 0.f, a10 = 0.f, a11 = 0.f;
      const size_t hb = ((size_t)layer * HKV + xcd) * a.max_seq * D;
      const uint32_t* kc = reinterpret_cast<const uint32_t*>(a.k_cache + hb);
      const uint32_t* vc = reinterpret_cast<const uint32_t*>(a.v_cache + hb);
      for (int i = 0; i < np_w; ++i) {
        const int p = p0 + mw + NMW * i;
        uint32_t kw, vw;
        if (p == position) {
          kw = (uint32_t)f32_to_bf16(s_k[2 * lane]) | ((uint32_t)f32_to_bf16(s_k[2 * lane + 1]) << 16);
          vw = (uint32_t)f32_to_bf16(s_v[2 * lane]) | ((uint32_t)f32_to_bf16(s_v[2 * lane + 1]) << 16);
        } else if (i < APF) {
          kw = kv_k[0]; vw = kv_v[0];
#pragma unroll
          for (int q = 1; q < APF; ++q) if (i == q) { kw = kv_k[q]; vw = kv_v[q]; }
        } else {
          kw = gp(kc)[(size_t)p * (D / 2) + lane];
          vw = gp(vc)[(size_t)p * (D / 2) + lane];
        }
        const float k0 = bf16_lo(kw), k1 = bf16_hi(kw), v0 = bf16_lo(vw), v1 = bf16_hi(vw);
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
      s_wp[mw][0][2 * lane] = a00; s_wp[mw][0][2 * lane + 1] = a01;
      s_wp[mw][1][2 * lane] = a10; s_wp[mw][1][2 * lane + 1] = a11;
      if (lane == 0) { s_wp[mw][0][D] = m0; s_wp[mw][0][D + 1] = l0; s_wp[mw][1][D] = m1; s_wp[mw][1][D + 1] = l1; }
    }
    __syncthreads();
    if (comm) {
      // merge the 7 waves' partials: lane -> head h = lane / 32, dims 4*(lane % 32) .. +3
      const int h = lane >> 5, d0 = (lane & 31) * 4;
      float M = -INFINITY;
#pragma unroll
      for (int w = 0; w < NMW; ++w) M = fmaxf(M, s_wp[w][h][D]);
      float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
      float Lsum = 0.f;
      if (M != -INFINITY) {
#pragma unroll
        for (int w = 0; w < NMW; ++w) {
          const float mw_ = s_wp[w][h][D];
          if (mw_ != -INFINITY) {
            const float f = expf(mw_ - M);
            acc.x += s_wp[w][h][d0] * f; acc.y += s_wp[w][h][d0 + 1] * f;
            acc.z += s_wp[w][h][d0 + 2] * f; acc.w += s_wp[w][h][d0 + 3] * f;
            Lsum += s_wp[w][h][D + 1] * f;
          }
        }
      }
      float* dst = att_x + ((size_t)j * 2 + h) * APS;
      if (j < S) {
        st_local_f32(dst + d0, acc.x); st_local_f32(dst + d0 + 1, acc.y);
        st_local_f32(dst + d0 + 2, acc.z); st_local_f32(dst + d0 + 3, acc.w);
        if ((lane & 31) == 0) { st_local_f32(dst + D, M); st_local_f32(dst + D + 1, Lsum); }
      }
      store_fence();
      mark(a, tl + 3);
      if (lane == 0) st_local_u32(fl + fl_local(F_ATT, xcd) + j, ep);
      poll_flags(c, fl + fl_local(F_ATT, xcd), S, ep);
      mark(a, tl + 11);
      // merge the S split partials of this XCD's two heads -> s_x[0, 256): lane jj < S reads
      // split jj's (m, l) for both heads, the wave reduces them, then every lane accumulates its
      // 4 dims of one head over the splits with the loads of a batch in flight together
      float mj[2], lj[2];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const float* src = att_x + ((size_t)(lane < S ? lane : 0) * 2 + hh) * APS;
        mj[hh] = ld_dev_f32(src + D);
        lj[hh] = ld_dev_f32(src + D + 1);
        if (lane >= S) { mj[hh] = -INFINITY; lj[hh] = 0.f; }
      }
      float Mh[2], Lh[2], fh[2];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        Mh[hh] = wave_max(mj[hh]);
        fh[hh] = mj[hh] == -INFINITY ? 0.f : expf(mj[hh] - Mh[hh]);
        Lh[hh] = wave_sum(lj[hh] * fh[hh]);
      }
      float* s_f = &s_wp[0][0][0];  // merge weights [2][32], reusing the wave-partial buffer
      if (lane < WPX) { s_f[lane] = fh[0]; s_f[WPX + lane] = fh[1]; }
      float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
      for (int j0 = 0; j0 < S; j0 += 8) {
        float4 aj[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const int jj = j0 + q < S ? j0 + q : j0;
          aj[q] = ld_dev_f32x4(att_x + ((size_t)jj * 2 + h) * APS, d0 * 4);
        }
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          if (j0 + q < S) {
            const float f = s_f[h * WPX + j0 + q];
            o.x += aj[q].x * f; o.y += aj[q].y * f; o.z += aj[q].z * f; o.w += aj[q].w * f;
          }
        }
      }
      const float inv = 1.f / Lh[h];
      s_x[h * D + d0] = o.x * inv; s_x[h * D + d0 + 1] = o.y * inv;
      s_x[h * D + d0 + 2] = o.z * inv; s_x[h * D + d0 + 3] = o.w * inv;
    }
    __syncthreads();

    // ---- C: o_proj partial over this group's 256 columns --------------------------------------
    mark(a, tl + 4);
    if (!comm) {
      const int gq = opaque(g), tq = opaque(t);
      load_units<PE, UPR_E>(wE, 0, U_E, gq, tq, ptr_E(lw));
      gemv_phase<NU_C, PC, UPR_C>(wC, U_C, gq, tq, ptr_C(lw), s_x, s_up);
    }
    __syncthreads();
    if (comm) {
      float* gc = ws + W_GC + (size_t)j * NXCD * MAX_HPW;  // [8][MAX_HPW] for row block j
      if (lane < HPW) st_dev_f32(gc + xcd * MAX_HPW + lane, s_up[lane * UPR_C] + s_up[lane * UPR_C + 1]);
      store_fence();
      mark(a, tl + 5);
      if (lane == 0) st_dev_u32(fl + fl_cross(0, j, xcd), ep);
      poll_flags(c, fl + fl_cross(0, j, 0), NXCD, ep, SLOT);
      mark(a, tl + 12);
      if (lane < HPW) {
        float s = 0.f;
#pragma unroll
        for (int y = 0; y < NXCD; ++y) s += ld_dev_f32(gc + y * MAX_HPW + lane);
        st_local_f32(lc_x + HPW * j + lane, s);
      }
      store_fence();
      if (lane == 0) st_local_u32(fl + fl_local(F_LC, xcd) + j, ep);
      poll_flags(c, fl + fl_local(F_LC, xcd), WPX, ep);
      mark(a, tl + 13);
      comm_residual_norm<H>(s_res, lc_x, (const uint16_t*)lw.post_attn_norm_weight, s_x);
    }
    __syncthreads();

    // ---- D: gate/up rows of MLP slice x ------------------------------------------------------
    mark(a, tl + 6);
    if (!comm) {
      const int gq = opaque(g), tq = opaque(t);
      if (layer + 1 < L) load_units<PA, UPR_H>(wA, 0, U_A, gq, tq, ptr_A(a.layers[layer + 1]));
      gemv_phase<NU_D, PD, UPR_H>(wD, U_D, gq, tq, ptr_D(lw), s_x, s_up);
    }
    __syncthreads();
    if (comm) {
      if (lane < IPW) {
        float gs = 0.f, us = 0.f;
#pragma unroll
        for (int b = 0; b < UPR_H; ++b) { gs += s_up[lane * UPR_H + b]; us += s_up[(lane + IPW) * UPR_H + b]; }
        st_local_f32(m_x + IPW * j + lane, gs / (1.f + expf(-gs)) * us);  // silu(g) * u
      }
      store_fence();
      mark(a, tl + 7);
      if (lane == 0) st_local_u32(fl + fl_local(F_M, xcd) + j, ep);
      poll_flags(c, fl + fl_local(F_M, xcd), WPX, ep);
      mark(a, tl + 14);
      for (int i = lane * 4; i < IX; i += 256) {
        const float4 v = ld_dev_f32x4(m_x, i * 4);
        *reinterpret_cast<float4*>(s_x + i) = v;
      }
    }
    __syncthreads();

    // ---- E: down_proj partial over slice x's columns -----------------------------------------
    mark(a, tl + 8);
    if (!comm) gemv_phase<NU_E, PE, UPR_E>(wE, U_E, opaque(g), opaque(t), ptr_E(lw), s_x, s_up);
    __syncthreads();
    if (comm) {
      float* ge = ws + W_GE + (size_t)j * NXCD * MAX_HPW;
      if (lane < HPW) {
        float s = 0.f;
#pragma unroll
        for (int b = 0; b < UPR_E; ++b) s += s_up[lane * UPR_E + b];
        st_dev_f32(ge + xcd * MAX_HPW + lane, s);
      }
      store_fence();
      mark(a, tl + 9);
      if (lane == 0) st_dev_u32(fl + fl_cross(1, j, xcd), ep);
      poll_flags(c, fl + fl_cross(1, j, 0), NXCD, ep, SLOT);
      mark(a, tl + 15);
      if (lane < HPW) {
        float s = 0.f;
#pragma unroll
        for (int y = 0; y < NXCD; ++y) s += ld_dev_f32(ge + y * MAX_HPW + lane);
        st_local_f32(le_x + HPW * j + lane, s);
      }
      store_fence();
      if (lane == 0) st_local_u32(fl + fl_local(F_LE, xcd) + j, ep);
      poll_flags(c, fl + fl_local(F_LE, xcd), WPX, ep);
      mark(a, tl + 16);
      const uint16_t* nw = layer + 1 < L ? (const uint16_t*)a.layers[layer + 1].norm_weight : a.final_norm;
      comm_residual_norm<H>(s_res, le_x, nw, s_x);
    }
    __syncthreads();
  }

  // ---- tied LM head over rows [r0, r1), greedy argmax ------------------------------------------
  mark(a, TRACE_LAYERS * TRACE_PER_LAYER + 1);
  {
    const int r0 = (int)(((long long)a.vocab * blockIdx.x) / NWG);
    const int r1 = (int)(((long long)a.vocab * (blockIdx.x + 1)) / NWG);
    mark(a, TRACE_LAYERS * TRACE_PER_LAYER + 2);
    if (!comm) {
      unsigned long long best = 0;
      // each group takes whole rows r0+g, r0+g+28, ...; a row is SEG segments of 8 chunks per lane;
      // the next segment's loads are issued before the current one is consumed
      constexpr int SEG = UPR_H / 8;
      const int gq = opaque(g), tq = opaque(t);
      int r = r0 + gq;
      int sg = 0;
      uint4 cur[8], nxt[8];
      auto seg_ptr = [&](int row, int seg) {
        return reinterpret_cast<const uint4*>(a.lm_head + (size_t)row * H) + 128 * seg + tq;
      };
      {
        const int rl = r < r1 ? r : r0;
#pragma unroll
        for (int b = 0; b < 8; ++b) cur[b] = ld_stream(seg_ptr(rl, 0) + 16 * b);
      }
      float acc = 0.f;
      while (r < r1) {
        const int sn = sg + 1 == SEG ? 0 : sg + 1;
        const int rn = sg + 1 == SEG ? r + MG : r;
        {
          const int rl = rn < r1 ? rn : r;  // past the end: re-read the current segment, unused
          const int sl = rn < r1 ? sn : sg;
#pragma unroll
          for (int b = 0; b < 8; ++b) nxt[b] = ld_stream(seg_ptr(rl, sl) + 16 * b);
        }
        const float* xs = s_x + 1024 * sg + tq * 8;
#pragma unroll
        for (int b = 0; b < 8; ++b) acc = dot8(cur[b], xs + 128 * b, acc);
        if (sg + 1 == SEG) {
          const float v = row16_sum(acc);
          if (tq == 0) {
            gpw(a.logits)[r] = v;
            best = umax64(best, argmax_key(v, r));
          }
          acc = 0.f;
        }
#pragma unroll
        for (int b = 0; b < 8; ++b) cur[b] = nxt[b];
        r = rn;
        sg = sn;
      }
      for (int off = 32; off >= 1; off >>= 1) best = umax64(best, __shfl_xor(best, off));
      if (lane == 0) s_best[mw] = best;
    }
    __syncthreads();
    mark(a, TRACE_LAYERS * TRACE_PER_LAYER + 3);
    if (comm) {
      const uint32_t ep_end = (seq << 6) | 63u;
      unsigned long long b = 0;
#pragma unroll
      for (int w = 0; w < NMW; ++w) b = umax64(b, s_best[w]);
      // this workgroup's best key and done flag, in its own slot: key first, flag after it
      uint32_t* mine = fl + fl_done(blockIdx.x);
      if (lane == 0) __hip_atomic_store(reinterpret_cast<unsigned long long*>(mine + 2), b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      store_fence();
      if (lane == 0) st_dev_u32(mine, ep_end);
      if (blockIdx.x == 0) {
        // the grid's greedy token: poll all 256 done flags (4 per lane), then reduce the keys
        for (uint32_t it = 0; !c.failed; ++it) {
          bool ok = true;
#pragma unroll
          for (int q = 0; q < 4; ++q) ok &= ld_dev_u32(fl + fl_done(lane * 4 + q)) == ep_end;
          if (__ballot(!ok) == 0) break;
          if ((it & 63u) == 63u && ld_dev_u32(c.status) != 0) c.failed = true;
          if (it > SPIN_LIMIT) { if (lane == 0) st_dev_u32(c.status, ERR_TIMEOUT); c.failed = true; }
        }
        unsigned long long m = 0;
#pragma unroll
        for (int q = 0; q < 4; ++q)
          m = umax64(m, __hip_atomic_load(reinterpret_cast<unsigned long long*>(fl + fl_done(lane * 4 + q) + 2),
                                          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        for (int off = 32; off >= 1; off >>= 1) m = umax64(m, __shfl_xor(m, off));
        if (lane == 0) {
          if (a.out_token) *gpw(a.out_token) = m ? (int32_t)(0xffffffffu - (uint32_t)(m & 0xffffffffu)) : -1;
          st_dev_u32(fl + FL_SEQ, seq + 1);  // every workgroup read seq at its start
        }
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

// Zero every flag and start the launch sequence at 1 (flag value 0 never matches an epoch).
static hipError_t clear_flags(void* ws) {
  char* fl = (char*)ws + WS_FLOATS * 4;
  hipError_t e = hipMemset(fl, 0, FL_WORDS * 4);
  if (e != hipSuccess) return e;
  const uint32_t one = 1;
  e = hipMemcpy(fl + FL_SEQ * 4, &one, 4, hipMemcpyHostToDevice);
  if (e != hipSuccess) return e;
  return hipDeviceSynchronize();
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
    if ((e = clear_flags(s.ws)) != hipSuccess) return e;
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
  if (!(s06 || s17) || dims->num_layers < 1 || dims->num_layers > MAX_LAYERS || dims->vocab < NWG) return hipErrorInvalidValue;
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
  k.fl = (uint32_t*)((char*)st->ws + WS_FLOATS * 4);
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
  return hipMemcpy(status, (char*)st->ws + WS_FLOATS * 4 + FL_STATUS * 4, 4, hipMemcpyDeviceToHost);
}

extern "C" hipError_t mk_reset(void) {
  DeviceState* st = nullptr;
  hipError_t e = device_state(&st);
  if (e != hipSuccess) return e;
  if ((e = hipDeviceSynchronize()) != hipSuccess) return e;
  return clear_flags(st->ws);
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

extern "C" const char* mk_version(void) { return "megakernel_amd 0.2 (gfx950; comm/math waves, flag exchanges)"; }
