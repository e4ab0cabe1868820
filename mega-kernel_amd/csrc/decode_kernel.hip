// Persistent decode kernel for Qwen3-shaped models on MI355X (gfx950), plus its C ABI.
//
// One launch = one decode step for batch 1: embedding -> L x {RMSNorm, QKV, per-head norm + RoPE,
// K/V cache write, split-K GQA attention, O-proj + residual, RMSNorm, gate/up + SiLU, down +
// residual} -> final RMSNorm -> tied LM head -> greedy argmax. This is the work of the reference's
// decode_kernel (/root/reference/megakernel.cu:744-893), re-planned for 256 CUs in 8 XCDs.
//
// Placement. One 576-thread workgroup (9 waves) per CU. The dispatcher deals workgroups to the 8
// XCDs round-robin, so workgroups b and b % 8 share an XCD (which physical XCD a group starts on
// varies with the hardware queue; only the grouping matters). Workgroup b is local workgroup
// j = b / 8 of group x = b % 8, checked from HW_REG_XCC_ID at the end of every launch. Group x owns
// K/V head x -- the 512 Q/K/V rows of that head group, its attention and its 256 columns of o_proj --
// plus a 1/8 slice of the MLP intermediate, so within a layer only two exchanges (the o_proj and
// down_proj partial sums) leave the XCD.
//
// Roles. Wave 0 of every workgroup is the communication wave: it publishes this workgroup's
// results, polls for other workgroups' results and does the vector work (residual, RMSNorm, q/k
// norm + RoPE, attention merges, SiLU). Waves 1-8 are math waves: each phase's weight tile is
// loaded into their registers a fixed number of phases ahead (PF_DIST) and consumed from there with
// bf16 dot instructions; they also run the attention and stream the LM head. Because
// vector-memory completions are counted in issue order per wave, the math waves never poll and the
// comm wave never prefetches.
//
// Exchanges are "LL" words: 32-bit stores of a value rounded to 24 bits (sign, exponent and 15
// stored mantissa bits, relative error <= 2^-16) in bits 8..31 and an 8-bit epoch in bits 0..7,
// epoch = (launch sequence * 64 + layer) mod 255 + 1. A reader polls the words themselves until
// every epoch matches, so one store and one load carry both data and readiness (no flag, no
// store-acknowledge wait), and a poll moves no more bytes than the fp32 values would. Within an XCD the
// words live in that XCD's L2 (plain stores, device-scope loads); across XCDs they are written
// through to memory (device-scope stores). Cross-XCD partial sums go in two hops: workgroup j of
// each XCD gathers row block j from the 8 XCDs, sums it in XCD order and republishes it inside its
// own XCD; then every workgroup reads the whole vector from its L2. Every word is written once
// per layer of every launch (also by workgroups that have nothing to put in it) and read before any
// writer can reach the next layer's write; consecutive writes of a word therefore carry epochs at
// most 127 apart (never 0 mod 255), so no buffer needs clearing and no stale word can pass for a
// fresh one. Each model shape has its own workspace, and each launching stream its own set of them.
//
// Variants chosen per launch on the host: one or two K/V rows per math group held in registers
// (template NKV), a contiguous or a paged K/V cache (block table in LDS), and a token read from
// the arguments or from device memory (the device-side multi-token loop).
//
// Numerics follow the reference kernel's fp32 design: bf16 weights and cache, fp32 activations and
// accumulation, fp32 RMSNorm, exact softmax, new K/V rounded to bf16 as stored. Logits are fp32;
// the greedy token is the argmax of the bf16-rounded logits, lowest index on ties. Every
// workgroup keeps its own copy of the residual stream in the comm wave's registers and updates it
// from the same data in the same order, so all copies are bitwise identical.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <mutex>
#include <type_traits>
#include <string.h>

#include "mk_batch.h"
#include "mk_device.h"
#include "../../include/megakernel_amd.h"

namespace mk {

typedef unsigned long long u64;
typedef unsigned u4v __attribute__((ext_vector_type(4)));

constexpr int D = 128;        // head_dim
constexpr int HQ = 16;        // query heads
constexpr int HKV = 8;        // K/V heads
constexpr int NXCD = 8;       // XCDs on MI355X
constexpr int WPX = 32;       // workgroups per XCD
constexpr int NWG = NXCD * WPX;
constexpr int NMW = 8;        // math waves (1..8); wave 0 is the communication wave
constexpr int NT = 64 * (NMW + 1);  // threads per workgroup
constexpr int MG = NMW * 4;   // 16-lane math groups
constexpr int QKV_X = 4 * D;  // q (2 heads) + k + v rows owned by one XCD
constexpr int QKV_WG = QKV_X / WPX;  // 16
constexpr int D_FREE = 8;            // local workgroups without gate/up rows (see Geo::DPW)
// K/V rows per math group held in registers (loaded a layer ahead) is a kernel template parameter
// NKV: 1 or 2, from split_plan().
constexpr int SPLIT_POS = MG;        // positions per split while the split count is below its cap
// Attention split merge: up to SB0 splits are polled with their (m, l) words in one round; beyond
// that the comm wave polls SB1 splits per round (as many as its registers hold).
template <int H> constexpr int merge_sb0() { return H <= 1024 ? 4 : 2; }
constexpr int SB1 = 8;
// Contexts above this many positions use two merge rounds' worth of splits, which spreads the
// streamed K/V rows over twice as many CUs (measured on MI355X with four streamed rows per round:
// at context 2000 (4000) 16 splits took 525 (593) us per token at 0.6B against 556 (670) with 8).
// At the 1024 width, whose splits stream six rows per round, 8 splits cover up to 2048 positions
// in one round and stay faster up to there (kernel 0.20, prompt 1100 / 1500 / 1900: -6 / -9.5 /
// -1 us per token against switching at 1024).
template <int H> constexpr int s_long_ctx() { return H <= 1024 ? 2048 : 1024; }
constexpr int APW = 264;      // LL words per attention partial: acc[2][128], m0, l0, m1, l1, pad
constexpr float EPS = 1e-6f;
constexpr float ATT_SCALE = 0.08838834764831845f;  // 128 ** -0.5
constexpr uint32_t SPIN_LIMIT = 1u << 22;
// Status word bits (all set with an atomic OR, never cleared by the kernel; mk_reset clears them).
constexpr uint32_t ERR_TIMEOUT = 1u;    // a bounded wait gave up: that launch's results are invalid
constexpr uint32_t ERR_PLACEMENT = 2u;  // workgroups b and b % 8 ran on different XCDs: later launches
                                        // write every exchange word through to memory
constexpr uint32_t ERR_TOKEN = 4u;      // a device-side input token was out of range (token 0 used)
constexpr uint32_t ERR_PAGE = 8u;       // a block-table entry was out of range (page 0 read, no write)
constexpr uint32_t ERR_HOST = 16u;      // set by the host (mk_request_drain)
constexpr uint32_t ERR_DRAIN = ERR_TIMEOUT | ERR_HOST;  // bits that make every launch drain at once
constexpr int MAX_PAGES = 2048;     // block-table entries a paged launch may use (LDS copy)
constexpr int PF_DIST = 2;  // phases of weights each math lane keeps in flight (0..4)
static_assert(PF_DIST >= 0 && PF_DIST <= 4, "prefetch distance");
constexpr int MAX_LAYERS = 62;  // epoch = seq << 6 | layer; 63 marks the final exchange

// Exchange workspace of one model shape. LL regions in 32-bit words (W_*), then the done flags,
// status and sequence in 64-bit words (X_*). Every region and every XCD's part of a region starts
// on a 256-byte boundary, and a cross-XCD slot (one writer) is 256 bytes, so no cache line has
// writers on two XCDs.
constexpr int MAX_H = 2048, MAX_I = 6144, MAX_IX = MAX_I / NXCD, MAX_HPW = MAX_H / WPX;
constexpr size_t W_QKV = 0;                                     // [8][512]
constexpr size_t W_ATT = W_QKV + NXCD * QKV_X;                  // [8][32][APW]
constexpr size_t W_M = W_ATT + (size_t)NXCD * WPX * APW;        // [8][MAX_IX]
constexpr size_t W_OL = W_M + (size_t)NXCD * MAX_IX;            // [8][MAX_H]
constexpr size_t W_EL = W_OL + (size_t)NXCD * MAX_H;            // [8][MAX_H]
constexpr size_t W_OX = W_EL + (size_t)NXCD * MAX_H;            // [32][8][MAX_HPW]
constexpr size_t W_EX = W_OX + (size_t)WPX * NXCD * MAX_HPW;    // [32][8][MAX_HPW]
constexpr size_t W_END = W_EX + (size_t)WPX * NXCD * MAX_HPW;
constexpr size_t X_DONE = W_END / 2;                            // [256][16]: key word, flag word
constexpr size_t X_STATUS = X_DONE + (size_t)NWG * 16;          // u32 status in its own line
constexpr size_t X_SEQ = X_STATUS + 32;                         // u32 launch sequence in its own line
constexpr size_t X_WORDS = X_SEQ + 32;
constexpr size_t WS_BYTES = X_WORDS * 8;
static_assert(W_ATT % 64 == 0 && W_M % 64 == 0 && W_OL % 64 == 0 && W_EL % 64 == 0 && W_OX % 64 == 0 &&
              W_EX % 64 == 0 && W_END % 64 == 0 && (WPX * APW) % 64 == 0 && MAX_IX % 64 == 0 &&
              MAX_HPW % 64 == 0, "exchange regions must be 256-byte aligned");

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
  const int32_t* token_in;  // when set, the input token is read here (written by an earlier launch)
  // Paged K/V cache (block_table set): k_cache/v_cache are [L][num_pages][HKV][page][D] and the
  // rows of positions [i * page, (i + 1) * page) live in page block_table[i]; page = 1 << page_shift.
  const int32_t* block_table;
  int num_pages, page_shift;
  u64* xw;          // exchange workspace
  uint64_t* trace;  // optional: per-workgroup phase timestamps (TRACE_N per workgroup)
  int token, position, max_seq, num_layers, vocab;
  int force_wt;     // write every exchange word through to memory (placement not verified)
};

// Phase timestamps (s_memrealtime, 100 MHz), TRACE_PER_LAYER slots per layer, see TraceSlot.
// TRACE_TAIL slots after the layers: kernel start, LM-head start, LM-head end, exit.
enum TraceSlot {
  T_A_START = 0, T_A_PUB, T_A_POLL, T_B_START, T_B_PUB, T_B_POLL, T_C_START, T_C_PUB, T_C_XPOLL, T_C_LPOLL,
  T_D_START, T_D_PUB, T_D_POLL, T_E_START, T_E_PUB, T_E_XPOLL, T_E_LPOLL,
  T_M_A_END, T_M_B_START, T_M_B_END,  // stamped by math wave 1
  T_B_MAX, T_B_SUM, T_M_A_DOT, T_M_D_ISSUED, T_M_D_DOT, T_M_B_ISSUED, T_M_B_ATT, T_SLOTS
};
constexpr int TRACE_LAYERS = 64;
constexpr int TRACE_PER_LAYER = 32;
constexpr int TRACE_TAIL = 8;
constexpr int TRACE_N = TRACE_LAYERS * TRACE_PER_LAYER + TRACE_TAIL;
static_assert(T_SLOTS <= TRACE_PER_LAYER, "trace slots");
__device__ __forceinline__ void mark(const KArgs& a, int idx, int by_thread = 0) {
  if (a.trace != nullptr && threadIdx.x == by_thread && idx >= 0 && idx < TRACE_N)
    a.trace[(size_t)blockIdx.x * TRACE_N + idx] = wall_clock64();
}

// ------------------------------------------------------------------------------------------
// LL exchange words (comm wave)
// ------------------------------------------------------------------------------------------
__device__ __forceinline__ void unpack8(uint4 w, float (&v)[8]) {
  v[0] = bf16_lo(w.x); v[1] = bf16_hi(w.x); v[2] = bf16_lo(w.y); v[3] = bf16_hi(w.y);
  v[4] = bf16_lo(w.z); v[5] = bf16_hi(w.z); v[6] = bf16_lo(w.w); v[7] = bf16_hi(w.w);
}

// LL word of value v: v rounded to nearest (ties away from zero) at mantissa bit 8, epoch ep in
// [1, 255] in the low byte.
__device__ __forceinline__ uint32_t ll_word(float v, uint32_t ep) {
  return ((__float_as_uint(v) + 0x80u) & 0xFFFFFF00u) | ep;
}
__device__ __forceinline__ float ll_value(uint32_t w) { return __uint_as_float(w & 0xFFFFFF00u); }
// Epoch of a layer's exchanges: nonzero, and 1 to 64 apart (never 0 mod 255) between consecutive
// writes of one word, which are one layer apart or the last layer of one launch and the first of
// the next.
__device__ __forceinline__ uint32_t ll_epoch(uint32_t seq, int layer) {
  return ((seq % 255u) * 64u + (uint32_t)layer) % 255u + 1u;
}

struct Comm {
  uint32_t* status;
  bool failed = false;
  bool wt = false;  // write local exchanges through to memory (fallback when placement is unknown)
};

// W (1, 2 or 4) consecutive LL words at word offset off (a multiple of W) from a wave-uniform
// base, in one store; each 4-byte word is single-copy atomic. Cross-XCD words are written through
// (device scope); local words stay in the XCD's L2.
template <int W>
__device__ __forceinline__ void ll_store(const Comm& c, uint32_t* base, int off, const float* v, uint32_t ep,
                                         bool cross) {
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(base);
  const bool wt = cross || c.wt;
  if constexpr (W == 1) {
    const uint32_t w = ll_word(v[0], ep);
    if (wt) __builtin_amdgcn_raw_buffer_store_b32(w, rs, off * 4, 0, CPOL_SC1);
    else __builtin_amdgcn_raw_buffer_store_b32(w, rs, off * 4, 0, 0);
  } else if constexpr (W == 2) {
    typedef unsigned u2v __attribute__((ext_vector_type(2)));
    const u2v w = {ll_word(v[0], ep), ll_word(v[1], ep)};
    if (wt) __builtin_amdgcn_raw_buffer_store_b64(w, rs, off * 4, 0, CPOL_SC1);
    else __builtin_amdgcn_raw_buffer_store_b64(w, rs, off * 4, 0, 0);
  } else {
    static_assert(W == 4, "LL store width");
    const u4v w = {ll_word(v[0], ep), ll_word(v[1], ep), ll_word(v[2], ep), ll_word(v[3], ep)};
    if (wt) __builtin_amdgcn_raw_buffer_store_b128(w, rs, off * 4, 0, CPOL_SC1);
    else __builtin_amdgcn_raw_buffer_store_b128(w, rs, off * 4, 0, 0);
  }
}

// Polls NL loads of W (2 or 4) LL words at word offsets off[k] from base (device-scope loads)
// until every epoch equals ep; returns the W*NL values. Up to TWO_MAX words per lane, two rounds
// of loads are kept in flight, so a value that lands while one round is out is seen by the next
// one instead of a full round trip later. Bounded: on timeout sets the status word and returns
// zeros.
template <int NL, int W, int TWO_MAX = 32>
__device__ __forceinline__ void ll_poll(Comm& c, const uint32_t* base, const int (&off)[NL], uint32_t ep,
                                        float (&v)[W * NL]) {
  static_assert(W == 2 || W == 4, "LL poll width");
  typedef unsigned uwv __attribute__((ext_vector_type(W)));
  auto zero = [&]() {  // failure paths only, so v holds no registers while the loads are out
#pragma unroll
    for (int k = 0; k < W * NL; ++k) v[k] = 0.f;
  };
  if (c.failed) { zero(); return; }
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(base);
  auto issue = [&](uwv (&r)[NL]) {
#pragma unroll
    for (int k = 0; k < NL; ++k) {
      if constexpr (W == 4)
        r[k] = __builtin_bit_cast(uwv, __builtin_amdgcn_raw_buffer_load_b128(rs, off[k] * 4, 0, CPOL_SC1));
      else
        r[k] = __builtin_bit_cast(uwv, __builtin_amdgcn_raw_buffer_load_b64(rs, off[k] * 4, 0, CPOL_SC1));
    }
  };
  auto ready = [&](const uwv (&r)[NL]) {
    uint32_t bad = 0;
#pragma unroll
    for (int k = 0; k < NL; ++k)
#pragma unroll
      for (int i = 0; i < W; ++i) bad |= (r[k][i] ^ ep) & 0xFFu;
    return __ballot(bad != 0) == 0;
  };
  auto take = [&](const uwv (&r)[NL]) {
#pragma unroll
    for (int k = 0; k < NL; ++k)
#pragma unroll
      for (int i = 0; i < W; ++i) v[W * k + i] = ll_value(r[k][i]);
  };
  auto check = [&](uint32_t it) {
    if ((it & 62u) == 62u && (ld_dev_u32(c.status) & ERR_DRAIN) != 0) { c.failed = true; return true; }
    if (it > SPIN_LIMIT) {
      if ((threadIdx.x & 63) == 0) raise_status(c.status, ERR_TIMEOUT);
      c.failed = true;
      return true;
    }
    return false;
  };
  if constexpr (NL * W <= TWO_MAX) {
    uwv r0[NL], r1[NL];
    issue(r0);
    for (uint32_t it = 0;; it += 2) {
      issue(r1);
      if (ready(r0)) { take(r0); return; }
      issue(r0);
      if (ready(r1)) { take(r1); return; }
      if (check(it)) { zero(); return; }
    }
  } else {  // large polls keep one round in flight (register budget)
    uwv r0[NL];
    for (uint32_t it = 0;; it += 2) {
      issue(r0);
      if (ready(r0)) { take(r0); return; }
      if (check(it)) { zero(); return; }
    }
  }
}

// Activations enter the GEMVs as two bf16 vectors, hi = bf16(x) and lo = bf16(x - hi), so that
// w . x = w . hi + w . lo is computed with bf16 dot instructions (v_dot2_f32_bf16: products exact
// in fp32, fp32 accumulation) to within ~2^-17 relative of the fp32 product, the precision of the
// reference kernel's fp32 activations (/root/reference/megakernel.cu:53-90, :100-142, :191-225).
// xh/xl hold the pairs as uint32 (element 2i in the low half), 16-byte chunks of 8 elements.
__device__ __forceinline__ void split_pair(float a, float b, uint32_t& hi, uint32_t& lo) {
  hi = pack_bf16x2(a, b);
  lo = pack_bf16x2(a - bf16_lo(hi), b - bf16_hi(hi));
}
// Writes n (even) consecutive values starting at element e0 (even) into xh/xl.
template <int N>
__device__ __forceinline__ void store_hilo(uint4* xh, uint4* xl, int e0, const float* v) {
  uint32_t* h = reinterpret_cast<uint32_t*>(xh) + e0 / 2;
  uint32_t* l = reinterpret_cast<uint32_t*>(xl) + e0 / 2;
  if constexpr (N % 8 == 0) {
#pragma unroll
    for (int k = 0; k < N; k += 8) {
      uint32_t hh[4], ll[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) split_pair(v[k + 2 * q], v[k + 2 * q + 1], hh[q], ll[q]);
      *reinterpret_cast<uint4*>(h + k / 2) = make_uint4(hh[0], hh[1], hh[2], hh[3]);
      *reinterpret_cast<uint4*>(l + k / 2) = make_uint4(ll[0], ll[1], ll[2], ll[3]);
    }
  } else {
#pragma unroll
    for (int k = 0; k < N; k += 2) split_pair(v[k], v[k + 1], h[k / 2], l[k / 2]);
  }
}

// x = res * w * rsqrt(mean(res^2) + eps) over the lane's E elements [E*lane, E*lane + E), the
// reference's fp32 RMSNorm (/root/reference/megakernel.cu:704-739, :148-182); w is bf16 in LDS.
template <int H>
__device__ __forceinline__ void comm_norm(const float (&res)[H / 64], const uint16_t* w, uint4* xh, uint4* xl) {
  constexpr int E = H / 64;
  const int lane = threadIdx.x & 63;
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < E; ++k) ss = fmaf(res[k], res[k], ss);
  ss = wave_sum(ss);
  const float rs = rsqrtf(ss / (float)H + EPS);
  float y[E];
#pragma unroll
  for (int k = 0; k < E; k += 8) {
    float wv[8];
    unpack8(*reinterpret_cast<const uint4*>(w + lane * E + k), wv);
#pragma unroll
    for (int q = 0; q < 8; ++q) y[k + q] = res[k + q] * wv[q] * rs;
  }
  store_hilo<E>(xh, xl, E * lane, y);
}

// RMSNorm split in two so that its reduction leaves the critical path: norm_input writes the GEMV
// input x * w (the math waves start on it at once); norm_scale then computes rsqrt(mean(x^2) + eps),
// which the comm wave applies to the GEMV's row sums. A GEMV is linear, so (W . (x*w)) * s equals
// W . (x*w*s) up to rounding.
template <int H>
__device__ __forceinline__ void norm_input(const float (&res)[H / 64], const uint16_t* w, uint4* xh, uint4* xl) {
  constexpr int E = H / 64;
  const int lane = threadIdx.x & 63;
  float y[E];
#pragma unroll
  for (int k = 0; k < E; k += 8) {
    float wv[8];
    unpack8(*reinterpret_cast<const uint4*>(w + lane * E + k), wv);
#pragma unroll
    for (int q = 0; q < 8; ++q) y[k + q] = res[k + q] * wv[q];
  }
  store_hilo<E>(xh, xl, E * lane, y);
}
template <int H>
__device__ __forceinline__ float norm_scale(const float (&res)[H / 64]) {
  constexpr int E = H / 64;
  float s0 = 0.f, s1 = 0.f;
#pragma unroll
  for (int k = 0; k < E; k += 2) { s0 = fmaf(res[k], res[k], s0); s1 = fmaf(res[k + 1], res[k + 1], s1); }
  return rsqrtf(wave_sum(s0 + s1) / (float)H + EPS);
}

// Cross-XCD partial sum of one row block, then republish inside the XCD, then read the whole
// vector and add it to the residual. mine: this workgroup's partial of row HPW*j + lane (lanes <
// HPW). Block j is rows [HPW*j, HPW*j + HPW).
template <int H>
__device__ __forceinline__ void comm_cross_reduce(Comm& c, uint32_t* xl, size_t xbase, size_t lbase, int xcd, int j,
                                                  float mine, uint32_t ep, float (&res)[H / 64], const KArgs& a,
                                                  int tslot_x, int tslot_l) {
  constexpr int HPW = H / WPX, RPL = HPW / 8, E = H / 64;
  static_assert(RPL % 4 == 0 && E % 4 == 0, "LL widths");
  const int lane = threadIdx.x & 63;
  // hop 1: my partial of block j -> slot (j, xcd); written through
  if (lane < HPW) ll_store<1>(c, xl + xbase, (j * NXCD + xcd) * MAX_HPW + lane, &mine, ep, true);
  // gather block j from the 8 XCDs: lane -> XCD y = lane / 8, rows RPL*(lane % 8) ..
  const int y = lane >> 3, r0 = RPL * (lane & 7);
  int off[RPL / 4];
#pragma unroll
  for (int k = 0; k < RPL / 4; ++k) off[k] = (j * NXCD + y) * MAX_HPW + r0 + 4 * k;
  float v[RPL];
  ll_poll<RPL / 4, 4>(c, xl + xbase, off, ep, v);
  mark(a, tslot_x);
  // sum over y in a fixed tree (lanes l, l^8, l^16, l^32 hold the same rows for different y)
#pragma unroll
  for (int k = 0; k < RPL; ++k) {
    v[k] += dpp<0x128>(v[k]);  // row_ror:8 == lane ^ 8 inside a 16-lane row
    v[k] = xsum32(xsum16(v[k]));
  }
  // hop 2: republish block j inside this XCD
  if (lane < 8) {
#pragma unroll
    for (int k = 0; k < RPL; k += 4) ll_store<4>(c, xl + lbase, xcd * MAX_H + HPW * j + r0 + k, v + k, ep, false);
  }
  int offl[E / 4];
#pragma unroll
  for (int k = 0; k < E / 4; ++k) offl[k] = xcd * MAX_H + E * lane + 4 * k;
  float d[E];
  ll_poll<E / 4, 4, (H <= 1024 ? 32 : 16)>(c, xl + lbase, offl, ep, d);
  mark(a, tslot_l);
#pragma unroll
  for (int k = 0; k < E; ++k) res[k] += d[k];
}

// ------------------------------------------------------------------------------------------
// Math-wave GEMV tiles. A phase's weight tile is ROWS rows of C bf16 columns. SPAN lanes share a
// row: lane l holds CPL 16-byte chunks of it, chunk k at column chunk k*SPAN + l % SPAN (so every
// load instruction of a wave reads contiguous bytes), and a wave covers RW = 64 / SPAN rows per
// step. Math wave mw takes rows (s*7 + mw)*RW + l/SPAN at steps s = 0, 1, ...; the first PS steps
// come from registers loaded phases ahead, the rest (large shapes) stream in the phase. A lane's
// activation slice is the same for every row, so it is read from LDS once per phase.
// ------------------------------------------------------------------------------------------
struct NoOp {
  __device__ void operator()() const {}
};

template <int ROWS_, int C_, int SPAN_, int PFS>
struct Tile {
  static constexpr int ROWS = ROWS_, C = C_, SPAN = SPAN_;
  static constexpr int CPL = C / (8 * SPAN);
  static constexpr int RW = 64 / SPAN;
  static constexpr int STEPS = (ROWS + RW * NMW - 1) / (RW * NMW);
  static constexpr int PS = STEPS < PFS ? STEPS : PFS;
  static_assert(C % (8 * SPAN) == 0 && 64 % SPAN == 0 && CPL >= 1, "tile shape");
};

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float dot2(uint32_t w, uint32_t x, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w), __builtin_bit_cast(bf16x2, x), acc, false);
}
template <int CPL>
__device__ __forceinline__ float dot_chunks(const uint4 (&w)[CPL], const uint4 (&xh)[CPL], const uint4 (&xl)[CPL]) {
  float a = 0.f, b = 0.f;
#pragma unroll
  for (int k = 0; k < CPL; ++k) {
    a = dot2(w[k].x, xh[k].x, a); b = dot2(w[k].x, xl[k].x, b);
    a = dot2(w[k].y, xh[k].y, a); b = dot2(w[k].y, xl[k].y, b);
    a = dot2(w[k].z, xh[k].z, a); b = dot2(w[k].z, xl[k].z, b);
    a = dot2(w[k].w, xh[k].w, a); b = dot2(w[k].w, xl[k].w, b);
  }
  return a + b;
}
// Sum over the SPAN lanes of a row; every lane of the row receives it.
template <int SPAN>
__device__ __forceinline__ float span_sum(float v) {
  if constexpr (SPAN == 64) return wave_sum(v);
  else if constexpr (SPAN == 32) return xsum16(row16_sum(v));
  else { static_assert(SPAN == 16, "span"); return row16_sum(v); }
}

template <class T>
__device__ __forceinline__ int tile_row(int s, int mw, int lane) {
  return (s * NMW + mw) * T::RW + lane / T::SPAN;
}
// Loads steps [s0, s0 + NS) of this lane into w (rows past the tile re-read its last row: loads are
// unconditional, see load order note in math_role).
template <class T, int NS, typename RowPtr>
__device__ __forceinline__ void tile_load(uint4 (&w)[NS][T::CPL], int s0, int mw, int lane, RowPtr rp) {
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    int r = tile_row<T>(s0 + s, mw, lane);
    r = r < T::ROWS ? r : T::ROWS - 1;
    const uint4* p = rp(r) + lane % T::SPAN;
#pragma unroll
    for (int k = 0; k < T::CPL; ++k) w[s][k] = ld_stream(p + k * T::SPAN);
  }
}
template <class T>
__device__ __forceinline__ void tile_dot_step(const uint4 (&w)[T::CPL], const uint4 (&xh)[T::CPL], const uint4 (&xl)[T::CPL],
                                              int s, int mw, int lane, float* s_up) {
  const float v = span_sum<T::SPAN>(dot_chunks<T::CPL>(w, xh, xl));
  const int r = tile_row<T>(s, mw, lane);
  if (lane % T::SPAN == 0 && r < T::ROWS) s_up[r] = v;
}
// One phase: row sums of the tile into s_up[row]. pf holds the first PS steps; `after` runs once
// they are consumed (before any streamed step). With NST > 0 the next NST steps come from `stage`,
// this lane's own LDS copy (word ((s - PS) * NMW + mw) * CPL + k of 64, lane-minor); the rest stream.
template <class T, int NST = 0, typename RowPtr, typename After>
__device__ __forceinline__ void tile_consume(const uint4 (&pf)[T::PS][T::CPL], int mw, int lane, const uint4* xh_lds,
                                             const uint4* xl_lds, float* s_up, RowPtr rp, After after,
                                             const uint4* stage = nullptr) {
  static_assert(T::PS + NST <= T::STEPS, "staged steps");
  uint4 xh[T::CPL], xl[T::CPL];
#pragma unroll
  for (int k = 0; k < T::CPL; ++k) {
    xh[k] = xh_lds[k * T::SPAN + lane % T::SPAN];
    xl[k] = xl_lds[k * T::SPAN + lane % T::SPAN];
  }
  if constexpr (T::SPAN == 64 && (T::PS == 2 || T::PS == 4) && T::PS == T::STEPS) {
    // whole-wave rows, all prefetched: reduce the PS row sums together. Each lane-swap step halves
    // the values a lane carries (gfx950 v_permlane32/16_swap: lanes 0-31 keep the first operand's
    // pair sums, lanes 32-63 the second's; likewise per 16-lane row pair), so PS rows cost one
    // 16-lane reduction instead of PS full-wave ones.
    float v[T::PS];
#pragma unroll
    for (int s = 0; s < T::PS; ++s) v[s] = dot_chunks<T::CPL>(pf[s], xh, xl);
    auto swap_add32 = [](float a, float b) {
      const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
      return __uint_as_float(r[0]) + __uint_as_float(r[1]);
    };
    auto swap_add16 = [](float a, float b) {
      const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
      return __uint_as_float(r[0]) + __uint_as_float(r[1]);
    };
    float z;
    int s;
    if constexpr (T::PS == 4) {
      // rows of the 16-lane row groups: step 0 (lanes 0-15), 2 (16-31), 1 (32-47), 3 (48-63)
      z = row16_sum(swap_add16(swap_add32(v[0], v[1]), swap_add32(v[2], v[3])));
      s = ((lane >> 5) & 1) | (((lane >> 4) & 1) << 1);
    } else {
      // step 0 in lanes 0-31, step 1 in lanes 32-63
      z = row16_sum(xsum16(swap_add32(v[0], v[1])));
      s = (lane >> 5) & 1;
    }
    const int r = tile_row<T>(s, mw, 0);
    if ((lane & 15) == 0 && r < T::ROWS) s_up[r] = z;
  } else {
#pragma unroll
    for (int s = 0; s < T::PS; ++s) tile_dot_step<T>(pf[s], xh, xl, s, mw, lane, s_up);
  }
  after();
#pragma unroll
  for (int s = T::PS; s < T::PS + NST; ++s) {
    uint4 w[T::CPL];
#pragma unroll
    for (int k = 0; k < T::CPL; ++k) w[k] = stage[(((s - T::PS) * NMW + mw) * T::CPL + k) * 64 + lane];
    tile_dot_step<T>(w, xh, xl, s, mw, lane, s_up);
  }
#pragma unroll
  for (int s = T::PS + NST; s < T::STEPS; ++s) {
    uint4 w[1][T::CPL];
    tile_load<T, 1>(w, s, mw, lane, rp);
    tile_dot_step<T>(w[0], xh, xl, s, mw, lane, s_up);
  }
}

__device__ __forceinline__ u64 argmax_key(float logit, int idx) {
  // order-preserving map of the bf16-rounded logit, then the complemented index so that equal
  // values prefer the lower index under an unsigned max
  uint32_t u = (uint32_t)f32_to_bf16(logit) << 16;
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((u64)u << 32) | (0xffffffffu - (uint32_t)idx);
}

__device__ __forceinline__ u64 umax64(u64 a, u64 b) { return a > b ? a : b; }

// Returns v unchanged but hides its origin from the optimizer, so per-unit indices derived from it
// are recomputed inside each phase instead of being held in registers for the whole kernel.
__device__ __forceinline__ int opaque(int v) {
  asm volatile("" : "+v"(v));
  return v;
}

// Online-softmax update of one key for one head: (m, l, acc[8]) <- key with score s and values v.
// __expf is the hardware exp2 of x*log2(e) (relative error ~1e-7); exp(-inf) = 0.
__device__ __forceinline__ void softmax_step(float s, const float (&v)[8], float& m, float& l, float (&acc)[8]) {
  const float n = fmaxf(m, s);
  const float cm = __expf(m - n), e = __expf(s - n);
  l = l * cm + e;
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = acc[i] * cm + e * v[i];
  m = n;
}


// ------------------------------------------------------------------------------------------
// The kernel. The comm wave and the math waves run separate loops (so their register live
// ranges never overlap) that meet at the same sequence of workgroup barriers: per layer and
// phase, math work -> barrier -> comm work -> barrier.
// ------------------------------------------------------------------------------------------
template <int H, int I>
struct Geo {
  static constexpr int E = H / 64;        // residual elements per comm lane
  static constexpr int IX = I / NXCD;     // MLP intermediate slice per XCD
  // The MLP slice's gate/up rows go to local workgroups D_FREE..31 only, DPW intermediates (gate and
  // up rows) each: the attention splits run on workgroups 0..S-1, and up to S = D_FREE of them then
  // carry no gate/up weights, whose 48-64 KB of loads would otherwise queue ahead of their exchanges.
  static constexpr int DPW = IX / (WPX - D_FREE);
  static constexpr int HPW = H / WPX;     // o_proj / down_proj rows per workgroup
  static constexpr bool SMALL = H <= 1024;
  // phase tiles: A = QKV rows, C = o_proj partial, D = gate/up rows, E = down_proj partial; the
  // last argument caps the steps held in registers ahead (the rest stream inside the phase). The
  // 1024 width holds every phase. At 2048 the register budget (168 VGPRs, 3 waves on one SIMD)
  // holds QKV and o_proj whole (2 steps each) and 2 of the 4 down steps, whose rows take 32 lanes so
  // that the down phase's activation slice needs 3 chunks per lane instead of 6; gate/up (8 steps,
  // 50 MB chip-wide) streams at bandwidth. Measured on MI355X at config 5: one step each, 843 us
  // per token; o_proj whole, 814; plus QKV whole and the 32-lane down rows, 805.
  typedef Tile<QKV_WG, H, 64, SMALL ? 8 : 2> TA;
  typedef Tile<HPW, 2 * D, 16, SMALL ? 8 : 2> TC;
  typedef Tile<2 * DPW, H, 64, SMALL ? 8 : 1> TD;
  typedef Tile<HPW, IX, SMALL ? 16 : 32, SMALL ? 8 : 2> TE;
  static constexpr int XN = (H > IX ? H : IX);
  // down steps after the register-held ones that go through LDS (see math_role, phase A)
  static constexpr int EST = SMALL ? 0 : TE::STEPS - TE::PS;
  static constexpr int EST_WORDS = EST > 0 ? EST * NMW * TE::CPL * 64 : 1;  // 16-byte words
  static constexpr int UMAX = 2 * DPW > HPW ? 2 * DPW : HPW;
  static constexpr int NSLOT = 2 * H + 2 * D;   // bf16 norm weights per layer: input, post-attention, q, k
  static constexpr int NSL16 = NSLOT / 8;       // ... in 16-byte chunks
  static constexpr int NSL_L = (NSL16 + 64 * NMW - 1) / (64 * NMW);  // chunks per math lane
  static constexpr int IXL = IX / 64;           // MLP words per comm lane
  static_assert(HPW * WPX == H && DPW * (WPX - D_FREE) == IX && IX * NXCD == I, "shape must split evenly");
  static_assert(IX % 128 == 0 && H % 512 == 0 && HPW <= 64 && DPW <= 64 && IXL % 2 == 0, "unsupported shape");
  static_assert(QKV_WG <= UMAX, "s_up too small");
  // past the last layer, tile loads read the final norm (H / 8 chunks): every lane's chunk index fits
  static_assert(TA::CPL * TA::SPAN <= H / 8 && TC::CPL * TC::SPAN <= H / 8 && TD::CPL * TD::SPAN <= H / 8 &&
                TE::CPL * TE::SPAN <= H / 8, "dummy loads stay inside the final norm");
};

template <int H, int I>
struct Smem {
  uint4 xh[Geo<H, I>::XN / 8];       // GEMV input of the current phase, bf16 hi part
  uint4 xl[Geo<H, I>::XN / 8];       // ... and lo part
  float up[Geo<H, I>::UMAX];         // row sums of the current phase
  float q[2][D];                     // normed, rotated queries
  uint16_t kvn[2][D];                // new K (normed, rotated) and V, bf16
  float cs[2][D];                    // cos, sin at position
  uint16_t nw[2][Geo<H, I>::NSLOT];  // per-layer norm weights by layer parity
  float gq[MG][2][D + 4];            // attention partials of the 32 math groups: acc[128], m, l
  u64 best[NMW];
  uint32_t seq, wt;                  // launch sequence and write-through mode, set by the comm wave
  uint32_t failed;                   // the launch drained (set before the LM head): logits are NaN
  mk_layer_weights layers[MAX_LAYERS];  // the layer table, copied once per launch
  int32_t bt[MAX_PAGES];             // block table of a paged launch (entries up to the position)
  uint4 estage[Geo<H, I>::EST_WORDS];  // staged down steps, private to each math lane
};

// Element offset of the K/V row of `head` at position p in layer `layer`: contiguous
// [L][HKV][max_seq][D] cache, or the paged layout through the block table's LDS copy (an invalid
// entry, -1 there, reads page 0).
__device__ __forceinline__ size_t kv_off(const KArgs& a, const int32_t* bt, int layer, int head, int p) {
  if (a.block_table) {
    const size_t page = (size_t)max(bt[p >> a.page_shift], 0);
    return (((((size_t)layer * a.num_pages + page) * HKV + head) << a.page_shift) + (p & ((1 << a.page_shift) - 1))) * D;
  }
  return (((size_t)layer * HKV + head) * a.max_seq + p) * D;
}

// Workgroup barrier for LDS hand-offs only: waits for this wave's LDS operations, not for its
// outstanding global loads (a full __syncthreads fence would also wait for the weight loads that
// run phases ahead). Exchanges through global memory never rely on it.
__device__ __forceinline__ void lds_barrier() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt left alone
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Per-launch constants every role needs.
struct Step {
  int xcd, j, position, ctx, L, S, p0, p1;
  bool att_wg;
};

// Attention split plan of a context: S splits on local workgroups 0..S-1, NKV register K/V rows
// per math group (the kernel's template parameter, chosen by the host from the same plan). One
// split per SPLIT_POS positions, capped at what one merge round takes (two rounds' worth for long
// contexts): a merge round costs more than a longer split. One register row while the splits are
// at most SPLIT_POS long (a second would only re-read a row), two once they are longer, so that
// contexts up to 512 (1024 at two merge rounds) stream no K/V inside the attention phase.
// (Measured on MI355X: packing two rows per group earlier, to keep S within one merge poll up to
// context 256, costs 3-4 us per token at the 0.6B shape and ~4 at 1.7B for short contexts.)
struct SplitPlan {
  int S, nkv;
};
template <int H>
__host__ __device__ constexpr SplitPlan split_plan(int ctx) {
  const int cap = ctx > s_long_ctx<H>() ? 2 * SB1 : SB1;
  const int S = (ctx + SPLIT_POS - 1) / SPLIT_POS;
  return {S < cap ? S : cap, ctx > cap * SPLIT_POS ? 2 : 1};
}

template <int H>
__device__ __forceinline__ Step make_step(const KArgs& a) {
  Step s;
  s.xcd = blockIdx.x % NXCD;
  s.j = blockIdx.x / NXCD;
  s.position = a.position;
  s.ctx = a.position + 1;
  s.L = a.num_layers;
  // Split-K attention (split_plan): up to MG * NKV positions per split come from registers
  // loaded a layer ahead, the rest stream in phase B.
  s.S = split_plan<H>(s.ctx).S;
  s.att_wg = s.j < s.S;
  s.p0 = s.att_wg ? (int)(((long long)s.ctx * s.j) / s.S) : 0;
  s.p1 = s.att_wg ? (int)(((long long)s.ctx * (s.j + 1)) / s.S) : 0;
  return s;
}

// Weight and cache addressing of one workgroup, shared by the math waves and the loader wave: the
// first 16-byte chunk of tile row r of each phase, the K/V row of a position, the norm-weight slots.
template <int H, int I>
struct Addr {
  typedef Geo<H, I> G;
  const KArgs& a;
  const Smem<H, I>& sm;
  const Step& st;
  struct RowsA {
    const uint16_t* base;
    int row0;
    __device__ const uint4* operator()(int r) const { return reinterpret_cast<const uint4*>(base + (size_t)(row0 + r) * H); }
  };
  struct RowsC {
    const uint16_t* base;
    int row0, col0;
    __device__ const uint4* operator()(int r) const {
      return reinterpret_cast<const uint4*>(base + (size_t)(row0 + r) * (HQ * D) + col0);
    }
  };
  struct RowsD {
    const uint16_t* wg;
    const uint16_t* wu;
    int row0;
    const uint16_t* none;  // non-null: this workgroup has no gate/up rows; its loads read this hot row
    __device__ const uint4* operator()(int r) const {
      if (none) return reinterpret_cast<const uint4*>(none);
      return reinterpret_cast<const uint4*>(r < G::DPW ? wg + (size_t)(row0 + r) * H : wu + (size_t)(row0 + r - G::DPW) * H);
    }
  };
  struct RowsE {
    const uint16_t* base;
    int row0, col0;
    __device__ const uint4* operator()(int r) const { return reinterpret_cast<const uint4*>(base + (size_t)(row0 + r) * I + col0); }
  };
  // A: 16 rows of this XCD's q (2 heads), k or v rows; C: o_proj rows x this XCD's 256 columns;
  // D: gate then up rows of this XCD's MLP slice; E: down_proj rows x the slice's columns
  __device__ RowsA A(const mk_layer_weights& lw) const {
    const int j = st.j, xcd = st.xcd;
    if (j < 16) return {(const uint16_t*)lw.q_weight, 2 * D * xcd + QKV_WG * j};
    if (j < 24) return {(const uint16_t*)lw.k_weight, D * xcd + QKV_WG * (j - 16)};
    return {(const uint16_t*)lw.v_weight, D * xcd + QKV_WG * (j - 24)};
  }
  __device__ RowsC C(const mk_layer_weights& lw) const {
    return {(const uint16_t*)lw.o_proj_weight, G::HPW * st.j, 2 * D * st.xcd};
  }
  __device__ RowsD Dm(const mk_layer_weights& lw) const {
    if (st.j < D_FREE) return {nullptr, nullptr, 0, a.final_norm};
    return {(const uint16_t*)lw.gate_proj_weight, (const uint16_t*)lw.up_proj_weight,
            G::IX * st.xcd + G::DPW * (st.j - D_FREE), nullptr};
  }
  __device__ RowsE E(const mk_layer_weights& lw) const {
    return {(const uint16_t*)lw.down_proj_weight, G::HPW * st.j, G::IX * st.xcd};
  }
  // first 16-byte chunk of the K/V row of position p of this XCD's head
  __device__ const uint4* kv_row(const uint16_t* cache, int layer, int p) const {
    return reinterpret_cast<const uint4*>(cache + kv_off(a, sm.bt, layer, st.xcd, p));
  }
  // position math group g attends to from registers, slot r: p0 + g + MG*r; unused slots re-read p0
  __device__ int kv_pos(int g, int r) const {
    const int p = st.p0 + g + MG * r;
    return (p < st.p1 && p != st.position) ? p : st.p0;
  }
  // norm-weight slot: chunk q of [input norm | post norm | q norm | k norm] for layer `layer`, or of
  // the final norm (every piece) when layer == L; q past the end re-reads the last chunk
  __device__ const uint4* slot_chunk(int layer, int q) const {
    q = q < G::NSL16 ? q : G::NSL16 - 1;
    if (layer >= st.L) return reinterpret_cast<const uint4*>(a.final_norm) + (q % (H / 8));
    const mk_layer_weights& lw = sm.layers[layer];
    if (q < H / 8) return reinterpret_cast<const uint4*>(lw.norm_weight) + q;
    if (q < H / 4) return reinterpret_cast<const uint4*>(lw.post_attn_norm_weight) + (q - H / 8);
    if (q < H / 4 + D / 8) return reinterpret_cast<const uint4*>(lw.q_norm_weight) + (q - H / 4);
    return reinterpret_cast<const uint4*>(lw.k_norm_weight) + (q - H / 4 - D / 8);
  }
};

// Split-K attention of this workgroup's split for one math wave (4 groups of 16 lanes, NKV key rows
// per group from registers; longer splits stream the rest). Online softmax per group for both
// query heads of the GQA pair, so each K/V row is read once (/root/reference/megakernel.cu:228-370);
// each group leaves its partial (acc[128], m, l per head) in sm.gq[g] for one merge of all 32
// groups after the next barrier.
template <int H, int I, int NKV>
__device__ __forceinline__ void attention_split(const KArgs& a, Smem<H, I>& sm, const Step& st, const Addr<H, I>& ad,
                                                int layer, int mw, int lane, const uint4 (&kK)[NKV],
                                                const uint4 (&kV)[NKV], int tl) {
  const int g = mw * 4 + (lane >> 4), t = lane & 15;
  float qa[8], qb[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) { qa[i] = sm.q[0][8 * t + i]; qb[i] = sm.q[1][8 * t + i]; }
  const uint4 knew = *reinterpret_cast<const uint4*>(&sm.kvn[0][8 * t]);
  const uint4 vnew = *reinterpret_cast<const uint4*>(&sm.kvn[1][8 * t]);
  float m0 = -INFINITY, m1 = -INFINITY, l0 = 0.f, l1 = 0.f;
  float a0[8], a1[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) { a0[i] = 0.f; a1[i] = 0.f; }
  // scores of both query heads of the group against one key row, then the online-softmax update
  // (the first key of a group initialises m, l, acc directly)
  auto attend = [&](uint4 kw, uint4 vw, bool first) {
    float kf[8], vf[8];
    unpack8(kw, kf);
    unpack8(vw, vf);
    float d0 = 0.f, d1 = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) { d0 = fmaf(qa[i], kf[i], d0); d1 = fmaf(qb[i], kf[i], d1); }
    d0 = row16_sum(d0) * ATT_SCALE;
    d1 = row16_sum(d1) * ATT_SCALE;
    if (first) {
      m0 = d0; m1 = d1; l0 = 1.f; l1 = 1.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) { a0[i] = vf[i]; a1[i] = vf[i]; }
    } else {
      softmax_step(d0, vf, m0, l0, a0);
      softmax_step(d1, vf, m1, l1, a1);
    }
  };
#pragma unroll
  for (int r = 0; r < NKV; ++r) {
    const int p = st.p0 + g + MG * r;
    if (p < st.p1) attend(p == st.position ? knew : kK[r], p == st.position ? vnew : kV[r], r == 0);
  }
  // positions beyond the register-held ones (long contexts) stream here, KV_BATCH keys of the group
  // per round trip (positions past the split re-read its first row and are skipped). At the 1024
  // width six rows fit the register budget and cover the ~5.5 streamed keys per group of a 16-split
  // context near 4K in one round trip (MI355X, prompt 3584: 527 -> 515 us per token); at 2048 the
  // wider batch costs 8 us per token at prompt 512. NKV == 1 never streams (split_plan).
  constexpr int KV_BATCH = (H <= 1024 && NKV == 2) ? 6 : 4;
  for (int p = st.p0 + g + MG * NKV; p < st.p1; p += KV_BATCH * MG) {
    uint4 kw[KV_BATCH], vw[KV_BATCH];
#pragma unroll
    for (int u = 0; u < KV_BATCH; ++u) {
      const int pu = p + u * MG < st.p1 ? p + u * MG : st.p0;
      kw[u] = ld_global16(ad.kv_row(a.k_cache, layer, pu) + t);
      vw[u] = ld_global16(ad.kv_row(a.v_cache, layer, pu) + t);
    }
#pragma unroll
    for (int u = 0; u < KV_BATCH; ++u) {
      const int pu = p + u * MG;
      if (pu < st.p1) attend(pu == st.position ? knew : kw[u], pu == st.position ? vnew : vw[u], false);
    }
  }
  // the group's partial as it stands (lane t holds dims 8t..8t+7); a group without keys leaves
  // m = -inf, l = 0, acc = 0
  mark(a, tl + T_M_B_ATT, 64);
#pragma unroll
  for (int i = 0; i < 8; i += 4) {
    *reinterpret_cast<float4*>(&sm.gq[g][0][8 * t + i]) = make_float4(a0[i], a0[i + 1], a0[i + 2], a0[i + 3]);
    *reinterpret_cast<float4*>(&sm.gq[g][1][8 * t + i]) = make_float4(a1[i], a1[i + 1], a1[i + 2], a1[i + 3]);
  }
  if (t == 0) {
    *reinterpret_cast<float2*>(&sm.gq[g][0][D]) = make_float2(m0, l0);
    *reinterpret_cast<float2*>(&sm.gq[g][1][D]) = make_float2(m1, l1);
  }
}

// Tied LM head over this workgroup's vocabulary rows: wave mw takes row mw of every row group the
// workgroup owns, one row per step (64 lanes x LCPL chunks), LP rows in flight per wave; fused
// greedy argmax key of the wave into sm.best[mw].
template <int H>
struct LmTile {
  static constexpr int LCPL = H / 512;  // 16-byte chunks per lane of one row
  // rows in flight per wave: measured on MI355X (kernel 0.19, config 2), 3 at the 1024 width beats 4
  // by ~1.8 us per token and 2 or 5 by ~1 us; at 2048 (register budget) 2, with 3 no faster
  static constexpr int LP = H <= 1024 ? 3 : 2;
  // row groups of NMW rows interleaved over the workgroups (step s reads group blockIdx.x + NWG*s),
  // so the grid sweeps the table front to back instead of 256 separate streams
  __device__ static int nmine(const KArgs& a) {
    const int ngroups = (a.vocab + NMW - 1) / NMW;
    return ((int)blockIdx.x < ngroups) ? (ngroups - (int)blockIdx.x + NWG - 1) / NWG : 0;
  }
  __device__ static int row_of(int s, int m) { return NMW * ((int)blockIdx.x + NWG * s) + m; }
  // loads row step s of math wave mw into b; past the end it re-reads the last row (unconditional loads)
  __device__ static void load(const KArgs& a, int nm, int s, int mw, int lane, uint4 (&b)[LCPL]) {
    int row = row_of(s, mw);
    row = (s < nm && row <= a.vocab - 1) ? row : a.vocab - 1;
    const uint4* p = reinterpret_cast<const uint4*>(a.lm_head + (size_t)row * H) + lane;
#pragma unroll
    for (int k = 0; k < LCPL; ++k) b[k] = ld_stream(p + 64 * k);
  }
  // the first LP rows: they depend on nothing the layers compute, so they are issued while the
  // last layer's exchanges and the final norm are still running
  __device__ static void first(const KArgs& a, int mw, int lane, uint4 (&buf)[LP][LCPL]) {
    const int nm = nmine(a);
#pragma unroll
    for (int i = 0; i < LP; ++i) load(a, nm, i, opaque(mw), opaque(lane), buf[i]);
  }
};

template <int H, int I>
__device__ __forceinline__ void lm_head(const KArgs& a, Smem<H, I>& sm, int mw, int lane,
                                        uint4 (&buf)[LmTile<H>::LP][LmTile<H>::LCPL]) {
  typedef LmTile<H> T;
  constexpr int LCPL = T::LCPL, LP = T::LP;
  const int nmine = T::nmine(a);
  const int rlast = a.vocab - 1;
  const int lq = opaque(lane), mwq = opaque(mw);
  auto row_of = [&](int s, int m) { return T::row_of(s, m); };
  uint4 xh[LCPL], xl[LCPL];
#pragma unroll
  for (int k = 0; k < LCPL; ++k) { xh[k] = sm.xh[k * 64 + lq]; xl[k] = sm.xl[k * 64 + lq]; }
  auto lm_load = [&](int s, uint4 (&b)[LCPL]) { T::load(a, nmine, s, mwq, lq, b); };
  u64 best = 0;
  const bool failed = __builtin_amdgcn_readfirstlane(sm.failed) != 0;
  for (int s0 = 0; s0 < nmine; s0 += LP) {
#pragma unroll
    for (int i = 0; i < LP; ++i) {
      const float v = wave_sum(dot_chunks<LCPL>(buf[i], xh, xl));
      const int s = s0 + i;
      const int row = row_of(s, mwq);
      if (s < nmine && row <= rlast) {
        if (lq == 0) gpw(a.logits)[row] = failed ? __builtin_nanf("") : v;
        best = umax64(best, argmax_key(v, row));
      }
      lm_load(s + LP, buf[i]);
    }
  }
  if (lane == 0) sm.best[mw] = best;
}

// Copies the layer table, and for a paged launch the block-table entries up to the position, into
// LDS (math waves, before the first barrier). An entry outside [0, num_pages) is kept as -1: reads
// through it take page 0, the new K/V row is not written when its page is such an entry, and the
// status bit ERR_PAGE is set, so no access leaves the page pool and no other sequence's page is
// overwritten.
template <int H, int I>
__device__ __forceinline__ void copy_layer_table(const KArgs& a, Smem<H, I>& sm) {
  constexpr int TW = (int)(sizeof(mk_layer_weights) / 8);
  const int n = a.num_layers * TW;
  for (int i = threadIdx.x - 64; i < n; i += NT - 64)
    reinterpret_cast<u64*>(sm.layers)[i] = reinterpret_cast<const u64*>(a.layers)[i];
  if (a.block_table) {
    const int np = (a.position >> a.page_shift) + 1;
    bool bad = false;
    for (int i = threadIdx.x - 64; i < np; i += NT - 64) {
      const int v = a.block_table[i];
      bad |= v < 0 || v >= a.num_pages;
      sm.bt[i] = (v < 0 || v >= a.num_pages) ? -1 : v;
    }
    if (bad) raise_status(reinterpret_cast<uint32_t*>(a.xw + X_STATUS), ERR_PAGE);
  }
}

// ---- math waves ------------------------------------------------------------------------------
template <int H, int I, int DIST, int NKV>
__device__ __forceinline__ void math_role(const KArgs& a, Smem<H, I>& sm, const Step& st) {
  typedef Geo<H, I> G;
  typedef typename G::TA TA;
  typedef typename G::TC TC;
  typedef typename G::TD TD;
  typedef typename G::TE TE;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int mw = wave - 1;
  const int g = mw * 4 + (lane >> 4);  // 16-lane group (attention: one key row per group)
  const int t = lane & 15;
  const int xcd = st.xcd, j = st.j, L = st.L;
  const bool att = __builtin_amdgcn_readfirstlane((int)st.att_wg) != 0;  // workgroup-uniform branch

  const Addr<H, I> ad{a, sm, st};
  auto rows_A = [&](const mk_layer_weights& lw) { return ad.A(lw); };
  auto rows_C = [&](const mk_layer_weights& lw) { return ad.C(lw); };
  auto rows_D = [&](const mk_layer_weights& lw) { return ad.Dm(lw); };
  auto rows_E = [&](const mk_layer_weights& lw) { return ad.E(lw); };
  auto kv_row = [&](const uint16_t* cache, int layer, int p) { return ad.kv_row(cache, layer, p) + t; };
  auto kv_pos = [&](int r) { return ad.kv_pos(g, r); };
  auto slot_chunk = [&](int layer, int q) { return ad.slot_chunk(layer, q); };

  uint4 wA[TA::PS][TA::CPL], wC[TC::PS][TC::CPL], wD[TD::PS][TD::CPL], wE[TE::PS][TE::CPL];
  constexpr int EST = G::EST;
  uint4 wEs[EST > 0 ? EST : 1][TE::CPL];  // down steps PS .. STEPS - 1, on their way to LDS
  uint4 kK[NKV], kV[NKV];
  uint4 nsl[G::NSL_L];

  // prologue: the layer table into LDS, then layer 0's norm weights (synchronously, wave 1)
  copy_layer_table(a, sm);
  lds_barrier();  // (P0) layer table in LDS
  if (wave == 1)
    for (int q = lane; q < G::NSL16; q += 64) reinterpret_cast<uint4*>(sm.nw[0])[q] = ld_global16(slot_chunk(0, q));

  // Loads of phase Q's registers (A=0: QKV, B=1: K/V rows, C=2: o_proj, D=3: gate/up, E=4: down)
  // for `layer`; past the last layer they re-read the last one. Every path issues the same weight
  // loads in the same order, so the compiler's wait counts stay exact (a load under a
  // data-dependent condition makes later waits count it as possibly absent, i.e. stricter). Phase P of layer l issues the loads
  // of phase P + DIST (of layer l, or of layer l + 1 when it wraps): DIST sets how many phases'
  // weights each CU keeps in flight.
  // Past the last layer the loads still issue (same count, so the wait counts stay exact) but every
  // row reads the final norm's 2-4 KB, which stays in L2: no weight traffic for a layer that never
  // runs.
  // K/V rows: a slot this workgroup's split does not attend to (or a workgroup without a split)
  // skips its load. The compiler then counts these two loads as possibly absent, which makes a few
  // later waits one or two loads stricter; worth it at the 0.6B shape (387 vs 395 us per token at
  // config 2), not at 1.7B (862 vs 848 at config 5, 932 vs 915 from prompt 1800).
  constexpr bool KV_PRED = H <= 1024;
  // QKV register steps issued at phase D (the rest at phase E). A burst of weight loads delays every
  // exchange poll the CU issues after it until the burst has drained (~1.3 us for all QKV rows
  // chip-wide), so the QKV burst is split between the D and E hops, each of which it fits. Measured
  // on MI355X at config 2: 381 -> 365 us per token.
  constexpr int A_FIRST = TA::PS > 1 ? 1 : TA::PS;

  auto load_phase = [&](auto qc, int layer) {
    constexpr int Q = decltype(qc)::value;
    const bool past = layer >= L;
    layer = past ? L - 1 : layer;
    const mk_layer_weights& lw = sm.layers[layer];
    const int mwq = opaque(mw), lq = opaque(lane);
    const uint4* hot = reinterpret_cast<const uint4*>(a.final_norm);
    auto sel = [&](auto rp) { return [=](int r) { return past ? hot : rp(r); }; };
    if constexpr (Q == 0) {  // QKV: the first A_FIRST steps (all of them when A_FIRST == PS)
      typedef uint4 First[A_FIRST][TA::CPL];
      tile_load<TA, A_FIRST>(*reinterpret_cast<First*>(&wA[0]), 0, mwq, lq, sel(rows_A(lw)));
    }
    if constexpr (Q == 6 && A_FIRST < TA::PS) {  // QKV: the remaining steps, issued a phase later
      typedef uint4 Rest[TA::PS - A_FIRST][TA::CPL];
      tile_load<TA, TA::PS - A_FIRST>(*reinterpret_cast<Rest*>(&wA[A_FIRST]), A_FIRST, mwq, lq, sel(rows_A(lw)));
    }
    if constexpr (Q == 1) {
#pragma unroll
      for (int r = 0; r < NKV; ++r) {
        if constexpr (KV_PRED) {
          const int pr = st.p0 + g + MG * r;
          if (opaque(att && pr < st.p1 && pr != st.position ? 1 : 0)) {
            kK[r] = ld_stream(kv_row(a.k_cache, layer, pr));
            kV[r] = ld_stream(kv_row(a.v_cache, layer, pr));
          }
        } else {  // unconditional: a slot outside the split re-reads its first row (never past position)
          kK[r] = ld_stream(kv_row(a.k_cache, layer, kv_pos(r)));
          kV[r] = ld_stream(kv_row(a.v_cache, layer, kv_pos(r)));
        }
      }
    }
    if constexpr (Q == 2) tile_load<TC, TC::PS>(wC, 0, mwq, lq, sel(rows_C(lw)));
    if constexpr (Q == 3) tile_load<TD, TD::PS>(wD, 0, mwq, lq, sel(rows_D(lw)));
    if constexpr (Q == 4) tile_load<TE, TE::PS>(wE, 0, mwq, lq, sel(rows_E(lw)));
  };
  // at the start of phase P. The K/V rows of layer l + 1 are not on this schedule: phase D of
  // layer l issues them (after its own loads), three phases ahead, so that at B they wait on nothing
  // newer than themselves but the rest of the QKV weights. (At phase C they added up to 32 KB per
  // attention workgroup to the down-projection burst in front of the o_proj exchange: measured on
  // MI355X, 1-7 us per token slower with two register rows, at both model widths.)
  auto issue_ahead = [&](auto pc, int layer) {
    constexpr int P = decltype(pc)::value;
    constexpr int Q = P + DIST;
    // At the 1.7B width the o_proj rows are issued after this workgroup's attention partial is
    // published (with the gate/up rows) instead of at phase A start: measured on MI355X, -5.5 us
    // per token at config 5, but +7 to +8.5 at the 0.6B width, where phase A's QKV poll is not
    // held up by them and the later burst lands in front of the split merge.
    constexpr bool C_LATE = H > 1024;
    if constexpr (C_LATE && P == 1) load_phase(std::integral_constant<int, 2>(), layer);
    if constexpr (Q % 5 != 1 && !(C_LATE && Q == 2)) {
      if constexpr (Q < 5) load_phase(std::integral_constant<int, Q>(), layer);
      else load_phase(std::integral_constant<int, Q - 5>(), layer + 1);
    }
    if constexpr (P == 3) load_phase(std::integral_constant<int, 1>(), layer + 1);
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I3 = std::integral_constant<int, 3>;
  using I4 = std::integral_constant<int, 4>;
  auto load_norms = [&](int layer) {
    // the next layer's norm weights (or the final norm), one chunk per math lane
    const int q0 = mw * 64 + lane;
#pragma unroll
    for (int k = 0; k < G::NSL_L; ++k) nsl[k] = ld_global16(slot_chunk(layer + 1, q0 + 64 * NMW * k));
  };
  if constexpr (DIST > 0) load_phase(I0(), 0);
  if constexpr (DIST > 0 && A_FIRST < TA::PS) load_phase(std::integral_constant<int, 6>(), 0);
  load_phase(I1(), 0);
  if constexpr (DIST > 2) load_phase(I2(), 0);
  if constexpr (DIST > 3) load_phase(I3(), 0);
  lds_barrier();  // (P1) norm weights of layer 0 in LDS

  for (int layer = 0; layer < L; ++layer) {
    const mk_layer_weights& lw = sm.layers[layer];
    const int tl = layer < TRACE_LAYERS ? layer * TRACE_PER_LAYER : -1000000;
    // (P2) comm: x = RMSNorm(embedding), for layer 0; (E2) of the previous layer otherwise: x =
    // this layer's normed input. The last layer's E2 follows the loop, after the first LM-head
    // loads, so that no load sits under a condition inside the loop (which would make the
    // compiler's wait counts stricter in every layer).
    lds_barrier();

    // A: QKV rows
    issue_ahead(I0(), layer);
    load_norms(layer);
    tile_consume<TA>(wA, opaque(mw), opaque(lane), sm.xh, sm.xl, sm.up, rows_A(lw), [&]() { mark(a, tl + T_M_A_DOT, 64); });
    mark(a, tl + T_M_A_END, 64);
    if constexpr (EST > 0) tile_load<TE, EST>(wEs, TE::PS, opaque(mw), opaque(lane), rows_E(lw));
    lds_barrier();  // (A1)
    lds_barrier();  // (A2) comm: q, new K/V in LDS
    mark(a, tl + T_M_B_START, 64);

    if (G::SMALL && !att) {
      // B on a workgroup without an attention split (0.6B width): its gate/up rows (phase B + DIST)
      // are issued right away, once its QKV rows are out (A1), so that the burst (48 KB per CU) has
      // mostly drained by the time the split partials it polls for next are published. It publishes
      // zeros into its split slot (every exchange word is written at every layer, see below).
      // Measured on MI355X (mk_bench, against issuing them after B3 as below): config 2 -3 us per
      // token, prompt 3584 -8 us; at the 2048 width +2.4 us, so there every workgroup takes the
      // single path below.
      issue_ahead(I1(), layer);
      mark(a, tl + T_M_B_END, 64);
      lds_barrier();  // (B1)
      {
        Comm c;
        c.wt = sm.wt != 0;
        const uint32_t ep = ll_epoch(sm.seq, layer);
        uint32_t* att_x = reinterpret_cast<uint32_t*>(a.xw) + W_ATT + (size_t)xcd * WPX * APW + (size_t)j * APW;
        const int h = mw >> 2, d0 = 32 * (mw & 3) + 4 * (lane & 7);
        const float zero[4] = {0.f, 0.f, 0.f, 0.f};
        if (lane < 8) ll_store<4>(c, att_x, h * D + d0, zero, ep, false);
        if (lane == 0 && (mw & 3) == 0) ll_store<2>(c, att_x, 2 * D + 2 * h, zero, ep, false);
      }
      lds_barrier();  // (B3)
      mark(a, tl + T_M_B_ISSUED, 64);
      lds_barrier();  // (B2) comm: attention output in x[0, 256)
    } else {
      // B: split-K attention; this phase's loads are issued after it, off the attention's path
      if (att) attention_split<H, I, NKV>(a, sm, st, ad, layer, mw, lane, kK, kV, tl);
      // This phase's loads (phase B + DIST) occupy the CU's memory pipeline for a while, so they are
      // issued only after this workgroup's attention partial is published: neither the attention nor
      // the publish queues behind them.
      mark(a, tl + T_M_B_END, 64);
      lds_barrier();  // (B1) every group's partial in sm.gq
      {
        // Merge the 32 group partials and publish this split's: wave mw takes head mw / 4, dims
        // 32 (mw % 4) .. +32. Lane = (subset sub of 4 groups, dim quad q4): each lane merges its 4
        // groups for 4 dims, then the 8 subsets combine across lanes (xor 8, 16, 32) with a common
        // max. Lanes 0-7 publish the head's 32 dims; lane 0 of waves 0 and 4 its (m, l).
        // A workgroup without a split publishes zeros into its slot: every exchange word is written
        // at every layer, which is what keeps a stale word's epoch from ever matching (the epochs
        // of consecutive writes of a word are then 1 to 64 apart, never equal mod 255).
        const int h = mw >> 2, sub = lane >> 3, d0 = 32 * (mw & 3) + 4 * (lane & 7);
        float M = 0.f, Ls = 0.f;
        float acc[4] = {0.f, 0.f, 0.f, 0.f};
        if (att) {
          float m[4], l[4];
          float4 p[4];
  #pragma unroll
          for (int k = 0; k < 4; ++k) {
            const float2 ml = *reinterpret_cast<const float2*>(&sm.gq[4 * sub + k][h][D]);
            m[k] = ml.x; l[k] = ml.y;
            p[k] = *reinterpret_cast<const float4*>(&sm.gq[4 * sub + k][h][d0]);
          }
          M = fmaxf(fmaxf(m[0], m[1]), fmaxf(m[2], m[3]));
          M = fmaxf(M, dpp<0x128>(M));  // row_ror:8 == lane ^ 8 inside a 16-lane row
          M = xmax32(xmax16(M));        // every split has a key, so M is finite
          mark(a, tl + T_B_MAX, 64);
  #pragma unroll
          for (int k = 0; k < 4; ++k) {
            const float f = __expf(m[k] - M);  // 0 for a group without keys
            Ls = fmaf(l[k], f, Ls);
            acc[0] = fmaf(p[k].x, f, acc[0]); acc[1] = fmaf(p[k].y, f, acc[1]);
            acc[2] = fmaf(p[k].z, f, acc[2]); acc[3] = fmaf(p[k].w, f, acc[3]);
          }
          auto sub_sum = [](float v) { v += dpp<0x128>(v); return xsum32(xsum16(v)); };
          Ls = sub_sum(Ls);
  #pragma unroll
          for (int i = 0; i < 4; ++i) acc[i] = sub_sum(acc[i]);
        }
        Comm c;
        c.wt = sm.wt != 0;
        const uint32_t ep = ll_epoch(sm.seq, layer);
        uint32_t* att_x = reinterpret_cast<uint32_t*>(a.xw) + W_ATT + (size_t)xcd * WPX * APW + (size_t)j * APW;
        const float ml[2] = {M, Ls};
        if (lane < 8) ll_store<4>(c, att_x, h * D + d0, acc, ep, false);
        if (lane == 0 && (mw & 3) == 0) ll_store<2>(c, att_x, 2 * D + 2 * h, ml, ep, false);
        if (att) mark(a, tl + T_B_PUB, 64);
      }
      lds_barrier();  // (B3) every wave's share of the partial is out before the loads below
      issue_ahead(I1(), layer);
      mark(a, tl + T_M_B_ISSUED, 64);
      lds_barrier();  // (B2) comm: attention output in x[0, 256)
    }

    // C: o_proj partial over this group's 256 columns
    issue_ahead(I2(), layer);
    tile_consume<TC>(wC, opaque(mw), opaque(lane), sm.xh, sm.xl, sm.up, rows_C(lw), NoOp());
    if constexpr (EST > 0) {
#pragma unroll
      for (int s2 = 0; s2 < EST; ++s2)
#pragma unroll
        for (int k = 0; k < TE::CPL; ++k) sm.estage[((s2 * NMW + mw) * TE::CPL + k) * 64 + lane] = wEs[s2][k];
    }
    lds_barrier();  // (C1)
    lds_barrier();  // (C2) comm: x = RMSNorm(residual) * post-attention norm

    // D: gate/up rows of MLP slice x
    issue_ahead(I3(), layer);
    mark(a, tl + T_M_D_ISSUED, 64);
    tile_consume<TD>(wD, opaque(mw), opaque(lane), sm.xh, sm.xl, sm.up, rows_D(lw), [&]() { mark(a, tl + T_M_D_DOT, 64); });
    lds_barrier();  // (D1)
    lds_barrier();  // (D2) comm: x[0, IX) = silu(gate) * up of the slice

    // E: down_proj partial over slice x's columns
    issue_ahead(I4(), layer);
    if constexpr (A_FIRST < TA::PS) load_phase(std::integral_constant<int, 6>(), layer + 1);
    tile_consume<TE, EST>(wE, opaque(mw), opaque(lane), sm.xh, sm.xl, sm.up, rows_E(lw), NoOp(), sm.estage);
    {
      // the next layer's norm weights (or the final norm) into the other LDS slot
      uint4* dst = reinterpret_cast<uint4*>(sm.nw[(layer + 1) & 1]);
      const int q0 = mw * 64 + lane;
#pragma unroll
      for (int k = 0; k < G::NSL_L; ++k)
        if (q0 + 64 * NMW * k < G::NSL16) dst[q0 + 64 * NMW * k] = nsl[k];
    }
    lds_barrier();  // (E1)
  }

  uint4 lm_buf[LmTile<H>::LP][LmTile<H>::LCPL];
  LmTile<H>::first(a, mw, lane, lm_buf);
  lds_barrier();  // (E2) of the last layer: comm: x = the final hidden state
  lm_head<H, I>(a, sm, mw, lane, lm_buf);
  lds_barrier();  // (F) per-wave argmax keys in LDS
}

// ---- comm wave -------------------------------------------------------------------------------
template <int H, int I>
__device__ __forceinline__ void comm_role(const KArgs& a, Smem<H, I>& sm, const Step& st) {
  typedef Geo<H, I> G;
  const int lane = threadIdx.x & 63;
  const int xcd = st.xcd, j = st.j, L = st.L, S = st.S;
  u64* xw = a.xw;
  uint32_t* xl = reinterpret_cast<uint32_t*>(xw);
  Comm c;
  c.status = reinterpret_cast<uint32_t*>(xw + X_STATUS);
  float res[G::E];

  lds_barrier();  // (P0)
  const uint32_t seq = ld_dev_u32(reinterpret_cast<const uint32_t*>(xw + X_SEQ));
  const uint32_t st0 = ld_dev_u32(c.status);
  {
    // A launch after a failed one (or after mk_request_drain) drains from the start: every wait
    // gives up at once and the logits come out NaN, until mk_reset.
    c.failed = (st0 & ERR_DRAIN) != 0;
    // Write-through when the host could not verify the placement, or an earlier launch found
    // workgroups b and b % 8 on different XCDs (checked at the end of every launch).
    c.wt = a.force_wt != 0 || (st0 & ERR_PLACEMENT) != 0;
    if (lane == 0) { sm.seq = seq; sm.wt = c.wt ? 1u : 0u; }
  }
  {
    int token = a.token;
    if (a.token_in) {  // every workgroup reads the same word, so all take the same branch below
      token = (int)ld_dev_u32(reinterpret_cast<const uint32_t*>(a.token_in));
      if (token < 0 || token >= a.vocab) {
        if (lane == 0) raise_status(c.status, ERR_TOKEN);
        token = 0;
      }
    }
    const uint16_t* row = a.embed + (size_t)token * H;
#pragma unroll
    for (int k = 0; k < G::E; k += 8) {
      float v[8];
      unpack8(ld_global16(reinterpret_cast<const uint4*>(row + G::E * lane + k)), v);
#pragma unroll
      for (int q = 0; q < 8; ++q) res[k + q] = v[q];
    }
    const uint16_t* cr = a.cos_tab + (size_t)st.position * D;
    const uint16_t* sr = a.sin_tab + (size_t)st.position * D;
    sm.cs[0][lane] = bf16_to_f32(gp(cr)[lane]); sm.cs[0][lane + 64] = bf16_to_f32(gp(cr)[lane + 64]);
    sm.cs[1][lane] = bf16_to_f32(gp(sr)[lane]); sm.cs[1][lane + 64] = bf16_to_f32(gp(sr)[lane + 64]);
  }
  lds_barrier();  // (P1)
  norm_input<H>(res, sm.nw[0], sm.xh, sm.xl);
  lds_barrier();  // (P2)
  float rs_in = norm_scale<H>(res);  // scale of the input norm, applied to the QKV row sums
  float rs_post = 0.f;               // scale of the post-attention norm, applied to gate/up
  // RoPE entries of this lane's 8 dims (d mod 64 of dims 8 (lane % 16) ..), the same at every layer
  float rc[8], rsn[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int d = (8 * (lane & 15) + i) & 63;
    rc[i] = sm.cs[0][d];
    rsn[i] = sm.cs[1][d];
  }

  for (int layer = 0; layer < L; ++layer) {
    const uint32_t ep = ll_epoch(seq, layer);
    const int tl = layer < TRACE_LAYERS ? layer * TRACE_PER_LAYER : -1000000;
    const uint16_t* nw = sm.nw[layer & 1];

    // ---- A: publish QKV rows; attention workgroups gather q, k, v of the group --------------
    mark(a, tl + T_A_START);
    lds_barrier();  // (A1)
    if (lane < QKV_WG) {
      const float qkv = sm.up[lane] * rs_in;
      ll_store<1>(c, xl + W_QKV, xcd * QKV_X + QKV_WG * j + lane, &qkv, ep, false);
    }
    mark(a, tl + T_A_PUB);
    if (st.att_wg) {
      // lane -> 8 values: q head 2x (lanes 0-15), q head 2x+1 (16-31), k head x (32-47), v (48-63)
      const int tt = lane & 15, part = lane >> 4;
      // this lane's 8 q/k-norm weights, read before the poll so that their LDS latency hides in it
      const u4v hwp = *reinterpret_cast<const u4v*>(nw + 2 * H + (part == 2 ? D : 0) + 8 * tt);
      int off[2];
#pragma unroll
      for (int k = 0; k < 2; ++k) off[k] = xcd * QKV_X + 8 * lane + 4 * k;
      float v[8];
      ll_poll<2, 4>(c, xl + W_QKV, off, ep, v);
      mark(a, tl + T_A_POLL);
      // per-head RMSNorm (/root/reference/megakernel.cu:490-630): a head is one 16-lane row
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) ss = fmaf(v[i], v[i], ss);
      ss = row16_sum(ss);
      const float rs = rsqrtf(ss / (float)D + EPS);
      float u[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t wp = hwp[i >> 1];
        u[i] = v[i] * rs * __uint_as_float(i & 1 ? wp & 0xFFFF0000u : wp << 16);
      }
      // rotate-half RoPE with the table entry of dim d mod 64 (/root/reference/megakernel.cu:548-555);
      // dim d's partner d +- 64 sits in lane tt ^ 8 of the same row
      float o[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float pr = dpp<0x128>(u[i]);
        o[i] = tt < 8 ? u[i] * rc[i] - pr * rsn[i] : u[i] * rc[i] + pr * rsn[i];
      }
      if (part < 2) {
#pragma unroll
        for (int i = 0; i < 8; ++i) sm.q[part][8 * tt + i] = o[i];
      } else {
        const float* src = part == 2 ? o : v;
        const u4v pk = {pack_bf16x2(src[0], src[1]), pack_bf16x2(src[2], src[3]), pack_bf16x2(src[4], src[5]),
                        pack_bf16x2(src[6], src[7])};
        *reinterpret_cast<u4v*>(&sm.kvn[part - 2][8 * tt]) = pk;
        // the split that owns `position` stores the new K/V in the cache (not through an invalid
        // block-table entry)
        if (j == S - 1 && (!a.block_table || sm.bt[st.position >> a.page_shift] >= 0)) {
          uint16_t* cache = part == 2 ? a.k_cache : a.v_cache;
          *gpw(reinterpret_cast<u4v*>(cache + kv_off(a, sm.bt, layer, xcd, st.position) + 8 * tt)) = pk;
        }
      }
    }
    lds_barrier();  // (A2)

    // ---- B: merge all split partials of the group (the math waves publish this split's) --------
    mark(a, tl + T_B_START);
    lds_barrier();  // (B1)
    lds_barrier();  // (B3) this workgroup's split partial published
    {
      const int h = lane >> 5, d0 = (lane & 31) * 4;
      uint32_t* att_x = xl + W_ATT + (size_t)xcd * WPX * APW;
      // Merge the S split partials of this XCD's two heads, in split order (lane -> head h, dims
      // d0 .. d0+3, plus each split's (m0, l0, m1, l1)). A poll round under load costs ~0.5 us even
      // when its data is ready, so the splits are taken in as few sequential polls as the registers
      // allow: all of them at once up to SB0 splits, otherwise SB1 splits per poll (at most two).
      // Max first: each poll's split maxima are reduced before any weight exp(m - max) is taken, so
      // the weights are independent and the accumulation is plain FMAs, not a chain of rescales
      // through a running max (which costs ~0.1 us per split on one wave).
      float Ls = 0.f;
      float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
      auto merge_batch = [&](auto nb) {  // all S <= NB splits in one poll
        constexpr int NB = decltype(nb)::value;
        int off[2 * NB];
#pragma unroll
        for (int q = 0; q < NB; ++q) {
          const int s = q < S ? q : 0;
          off[2 * q + 0] = s * APW + h * D + d0;
          off[2 * q + 1] = s * APW + 2 * D;
        }
        float v[8 * NB];
        ll_poll<2 * NB, 4, 32>(c, att_x, off, ep, v);  // two rounds in flight
        float M = -INFINITY;
#pragma unroll
        for (int q = 0; q < NB; ++q)
          if (q < S) M = fmaxf(M, h ? v[8 * q + 6] : v[8 * q + 4]);
#pragma unroll
        for (int q = 0; q < NB; ++q) {
          if (q < S) {
            const float* w = v + 8 * q;
            const float cs = __expf((h ? w[6] : w[4]) - M);
            Ls = fmaf(h ? w[7] : w[5], cs, Ls);
            acc.x = fmaf(w[0], cs, acc.x); acc.y = fmaf(w[1], cs, acc.y);
            acc.z = fmaf(w[2], cs, acc.z); acc.w = fmaf(w[3], cs, acc.w);
          }
        }
      };
      constexpr int SB0 = merge_sb0<H>();
      static_assert(2 * SB1 <= WPX && SB1 == 8, "split count; one 8-lane group holds a round's (m, l)");
      // Rounds of SB1 splits from s0: each lane's accumulator slice of every split, plus one load of
      // the splits' (m0, l0, m1, l1) words on lanes 0..SB1-1 (lane q: split s0 + q). Both heads'
      // running max and sum are kept wave-uniform (M0, M1, L0, L1) across rounds.
      float M0 = -INFINITY, M1 = -INFINITY, L0 = 0.f, L1 = 0.f;
      auto merge_wide = [&](int s0) {
        constexpr int NB = SB1;
        int off[NB + 1];
#pragma unroll
        for (int q = 0; q < NB; ++q) off[q] = (s0 + q < S ? s0 + q : s0) * APW + h * D + d0;
        const bool own = lane < NB && s0 + lane < S;
        off[NB] = (own ? s0 + lane : s0) * APW + 2 * D;
        float v[4 * (NB + 1)];
        // one round in flight (two, at the 0.6B width where they fit without spilling, measured
        // no faster on MI355X: -2 to +3 us per token from context 300 to 3584)
        ll_poll<NB + 1, 4, 16>(c, att_x, off, ep, v);
        auto max8 = [](float x) {  // max over each 8-lane group
          x = fmaxf(x, dpp<0xB1>(x));   // quad_perm [1,0,3,2]
          x = fmaxf(x, dpp<0x4E>(x));   // quad_perm [2,3,0,1]
          return fmaxf(x, dpp<0x141>(x));  // row_half_mirror
        };
        auto sum8 = [](float x) {
          x += dpp<0xB1>(x);
          x += dpp<0x4E>(x);
          return x + dpp<0x141>(x);
        };
        auto lane0 = [](float x) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 0)); };
        const float m0 = own ? v[4 * NB + 0] : -INFINITY, m1 = own ? v[4 * NB + 2] : -INFINITY;
        const float N0 = fmaxf(M0, lane0(max8(m0))), N1 = fmaxf(M1, lane0(max8(m1)));  // finite
        const float f0 = own ? __expf(m0 - N0) : 0.f, f1 = own ? __expf(m1 - N1) : 0.f;
        const float c0 = __expf(M0 - N0), c1 = __expf(M1 - N1);  // 0 on the first round
        L0 = fmaf(L0, c0, lane0(sum8(own ? v[4 * NB + 1] * f0 : 0.f)));
        L1 = fmaf(L1, c1, lane0(sum8(own ? v[4 * NB + 3] * f1 : 0.f)));
        M0 = N0; M1 = N1;
        const float cm = h ? c1 : c0;
        acc.x *= cm; acc.y *= cm; acc.z *= cm; acc.w *= cm;
#pragma unroll
        for (int q = 0; q < NB; ++q) {
          if (s0 + q < S) {
            const float g0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(f0), q));
            const float g1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(f1), q));
            const float cs = h ? g1 : g0;
            const float* w = v + 4 * q;
            acc.x = fmaf(w[0], cs, acc.x); acc.y = fmaf(w[1], cs, acc.y);
            acc.z = fmaf(w[2], cs, acc.z); acc.w = fmaf(w[3], cs, acc.w);
          }
        }
      };
      if (S <= SB0) {
        merge_batch(std::integral_constant<int, SB0>());
      } else {
#pragma unroll 1
        for (int s0 = 0; s0 < S; s0 += SB1) merge_wide(s0);
        Ls = h ? L1 : L0;
      }
      mark(a, tl + T_B_POLL);
      const float inv = 1.f / Ls;
      const float o[4] = {acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv};
      store_hilo<4>(sm.xh, sm.xl, h * D + d0, o);
    }
    lds_barrier();  // (B2)

    // ---- C: o_proj partials -> residual -> post-attention RMSNorm ------------------------------
    mark(a, tl + T_C_START);
    lds_barrier();  // (C1)
    {
      const float mine = lane < G::HPW ? sm.up[lane] : 0.f;
      mark(a, tl + T_C_PUB);
      comm_cross_reduce<H>(c, xl, W_OX, W_OL, xcd, j, mine, ep, res, a, tl + T_C_XPOLL, tl + T_C_LPOLL);
      norm_input<H>(res, nw + H, sm.xh, sm.xl);
    }
    lds_barrier();  // (C2)
    rs_post = norm_scale<H>(res);

    // ---- D: silu(gate) * up of this workgroup's rows; gather the XCD's slice ------------------
    mark(a, tl + T_D_START);
    lds_barrier();  // (D1)
    {
      uint32_t* m_x = xl + W_M + (size_t)xcd * MAX_IX;
      if (j >= D_FREE && lane < G::DPW) {
        const float gs = sm.up[lane] * rs_post, us = sm.up[lane + G::DPW] * rs_post;
        const float m = gs / (1.f + expf(-gs)) * us;  // silu(g) * u
        ll_store<1>(c, m_x, G::DPW * (j - D_FREE) + lane, &m, ep, false);
      }
      mark(a, tl + T_D_PUB);
      constexpr int MW = G::IXL % 4 == 0 ? 4 : 2;
      static_assert(G::IXL % MW == 0, "LL widths");
      int off[G::IXL / MW];
#pragma unroll
      for (int k = 0; k < G::IXL / MW; ++k) off[k] = G::IXL * lane + MW * k;
      float v[G::IXL];
      ll_poll<G::IXL / MW, MW>(c, m_x, off, ep, v);
      mark(a, tl + T_D_POLL);
      store_hilo<G::IXL>(sm.xh, sm.xl, G::IXL * lane, v);
    }
    lds_barrier();  // (D2)

    // ---- E: down_proj partials -> residual -> next layer's input RMSNorm ----------------------
    mark(a, tl + T_E_START);
    lds_barrier();  // (E1)
    {
      const float mine = lane < G::HPW ? sm.up[lane] : 0.f;
      mark(a, tl + T_E_PUB);
      comm_cross_reduce<H>(c, xl, W_EX, W_EL, xcd, j, mine, ep, res, a, tl + T_E_XPOLL, tl + T_E_LPOLL);
      if (layer + 1 < L) {
        norm_input<H>(res, sm.nw[(layer + 1) & 1], sm.xh, sm.xl);  // next layer's input norm
      } else {
        // Every exchange of this launch has been consumed. If this workgroup drained, or any
        // workgroup whose results reached it did (it set a drain bit before publishing them), the
        // LM head writes NaN: a failed launch is visible in its output without a host sync. The
        // status load is issued before the final norm so that its latency overlaps it.
        const uint32_t stw = ld_dev_u32(c.status);
        comm_norm<H>(res, sm.nw[(layer + 1) & 1], sm.xh, sm.xl);  // the final norm, for the LM head
        if (lane == 0) sm.failed = (c.failed || (stw & ERR_DRAIN) != 0) ? 1u : 0u;
      }
    }
    lds_barrier();  // (E2)
    if (layer + 1 < L) rs_in = norm_scale<H>(res);
  }

  mark(a, TRACE_LAYERS * TRACE_PER_LAYER + 1);
  lds_barrier();  // (F)
  mark(a, TRACE_LAYERS * TRACE_PER_LAYER + 2);
  {
    const uint32_t ep_end = (seq << 6) | 63u;
    u64 b = 0;
#pragma unroll
    for (int w = 0; w < NMW; ++w) b = umax64(b, sm.best[w]);
    // this workgroup's best key and done flag, in its own slot: key first, flag after it. The flag
    // carries the epoch in its low 32 bits and the XCD this workgroup ran on above them.
    u64* mine = xw + X_DONE + (size_t)blockIdx.x * 16;
    if (lane == 0) __hip_atomic_store(mine, b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    wait_vmem();
    if (lane == 0)
      __hip_atomic_store(mine + 1, (u64)ep_end | ((u64)xcc_id() << 32), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (blockIdx.x == 0) {
      // the grid's greedy token: poll all 256 done flags (4 per lane), then reduce the keys
      u64 f[4] = {0, 0, 0, 0};
      for (uint32_t it = 0; !c.failed; ++it) {
        bool ok = true;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          f[q] = __hip_atomic_load(xw + X_DONE + (size_t)(lane * 4 + q) * 16 + 1, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
          ok &= (uint32_t)f[q] == ep_end;
        }
        if (__ballot(!ok) == 0) break;
        if ((it & 63u) == 63u && (ld_dev_u32(c.status) & ERR_DRAIN) != 0) c.failed = true;
        if (it > SPIN_LIMIT) { if (lane == 0) raise_status(c.status, ERR_TIMEOUT); c.failed = true; }
      }
      if (!c.failed) {
        // The local exchanges rely on workgroups b and b % 8 sharing an XCD (and so an L2); which
        // physical XCD a group lands on does not matter (the dispatcher may start at any XCD).
        // Lane l holds workgroups 4l..4l+3; workgroup 4l + q's group leader 4(l % 2) + q is slot q
        // of lane l % 2.
        bool bad = false;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int x = (int)(f[q] >> 32);
          bad |= x != __shfl(x, lane & 1);
        }
        if (__ballot(bad) != 0 && lane == 0) raise_status(c.status, ERR_PLACEMENT);
      }
      const bool failed = c.failed || (ld_dev_u32(c.status) & ERR_DRAIN) != 0;
      u64 m = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        m = umax64(m, __hip_atomic_load(xw + X_DONE + (size_t)(lane * 4 + q) * 16, __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT));
      for (int off = 32; off >= 1; off >>= 1) m = umax64(m, __shfl_xor(m, off));
      if (lane == 0) {
        // a failed launch reports token -1 (its logits are NaN)
        if (a.out_token) *gpw(a.out_token) = (m && !failed) ? (int32_t)(0xffffffffu - (uint32_t)(m & 0xffffffffu)) : -1;
        st_dev_u32(reinterpret_cast<uint32_t*>(xw + X_SEQ), seq + 1);  // every workgroup read seq at its start
      }
    }
  }
  mark(a, TRACE_LAYERS * TRACE_PER_LAYER + 3);
}

template <int H, int I, int NKV>
__global__ void __launch_bounds__(NT, 1) decode_kernel(const KArgs a) {
  __shared__ __attribute__((aligned(16))) Smem<H, I> sm;
  const Step st = make_step<H>(a);
  mark(a, TRACE_LAYERS * TRACE_PER_LAYER + 0);
  if (threadIdx.x < 64) comm_role<H, I>(a, sm, st);
  else math_role<H, I, PF_DIST, NKV>(a, sm, st);
}

// ------------------------------------------------------------------------------------------
// Host side: per-device state, exchange workspaces and launch
// ------------------------------------------------------------------------------------------
// A workspace set holds one WS_BYTES workspace per supported model shape, so that every word of a
// workspace is written at every layer of every launch that uses it (the epoch rule above).
constexpr int NSHAPE = 2;
constexpr size_t WS_SET_WORDS = NSHAPE * X_WORDS;
constexpr size_t WS_SET_BYTES = WS_SET_WORDS * 8;

// Zeroes a workspace set and starts each shape's launch sequence at 1 (a zeroed word has epoch 0,
// which never matches). A fill kernel rather than a memset.
__global__ void ws_init_kernel(u64* ws) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < WS_SET_WORDS; i += (size_t)gridDim.x * blockDim.x)
    ws[i] = (i % X_WORDS == X_SEQ) ? 1ull : 0ull;  // the sequence is the low 32 bits of its word
}

// OR status bits into every shape's status word of a workspace set (mk_request_drain).
__global__ void ws_raise_kernel(u64* ws, uint32_t bits) {
  if (threadIdx.x < NSHAPE) raise_status(reinterpret_cast<uint32_t*>(ws + threadIdx.x * X_WORDS + X_STATUS), bits);
}

// Each workgroup of a grid of NWG records the XCD it runs on.
__global__ void placement_probe(uint32_t* out) {
  if (threadIdx.x == 0) out[blockIdx.x] = xcc_id();
}

constexpr int MAX_DEVICES = 64;
// Workspace sets per device, one per stream that launches. A stream beyond this many takes over the
// set used least recently, after a device synchronization (so no launch can still be using it); the
// set's status bits are kept in the device's retired status.
constexpr int MAX_STREAMS = 64;

struct Workspace {
  hipStream_t stream;
  void* ws;
  uint64_t last_use;  // launch counter value at the set's last launch
};
struct DeviceState {
  bool init = false;
  hipError_t err = hipSuccess;  // why the device cannot run the kernel, if it cannot
  bool cooperative = false;     // launch mode, see launch()
  bool force_wt = false;        // placement b % 8 not confirmed: exchanges write through
  bool drain_pending = false;   // mk_request_drain was called and mk_reset has not been since
  uint32_t retired_status = 0;  // status bits of workspace sets handed to another stream
  int nws = 0;
  uint64_t launches = 0;
  Workspace ws[MAX_STREAMS];
  uint64_t* trace = nullptr;    // set by mk_set_trace; null in normal operation
};
static DeviceState g_dev[MAX_DEVICES];

// The no-allocation entry point's workspace set: a file-scope device array (each device that runs
// the library holds its own copy until the process ends). Host code never uses the name `scratch`
// as an address: its per-device address comes from hipGetSymbolAddress, once per device.
static __device__ __align__(256) u64 scratch[WS_SET_WORDS];
struct StaticState {
  bool init = false;
  hipError_t err = hipSuccess;
  bool force_wt = false;
  void* ptr = nullptr;  // this device's address of `scratch`
};
static StaticState g_static[MAX_DEVICES];
static std::mutex g_mu;

template <int H, int I>
static hipError_t check_kernel_fits() {
  for (const void* f : {(const void*)decode_kernel<H, I, 1>, (const void*)decode_kernel<H, I, 2>}) {
    int blocks = 0;
    hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, f, NT, 0);
    if (e != hipSuccess) return e;
    if (blocks < 1) return hipErrorCooperativeLaunchTooLarge;
  }
  return hipSuccess;
}

// Can device `dev` run the kernel: 256 CUs, cooperative launch support, one workgroup per CU.
static hipError_t check_device(int dev) {
  int cus = 0, coop = 0;
  hipError_t e;
  if ((e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev)) != hipSuccess) return e;
  if ((e = hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev)) != hipSuccess) return e;
  if (cus != NWG || !coop) return hipErrorNotSupported;
  if ((e = check_kernel_fits<1024, 3072>()) != hipSuccess) return e;
  return check_kernel_fits<2048, 6144>();
}

// First use of a workspace set: check the workgroup placement the kernel relies on (workgroups b
// and b % 8 on one XCD, the 8 groups on 8 XCDs), using the set's done-key area for the probe's
// output, then zero the set. Synchronizes `stream` once. *placement_ok tells whether the probe's
// grid was placed that way.
static hipError_t init_workspace(void* ws, hipStream_t stream, bool* placement_ok) {
  uint32_t* probe = reinterpret_cast<uint32_t*>(static_cast<u64*>(ws) + X_DONE);
  hipLaunchKernelGGL(placement_probe, dim3(NWG), dim3(64), 0, stream, probe);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  uint32_t ids[NWG];
  if ((e = hipMemcpyAsync(ids, probe, sizeof ids, hipMemcpyDeviceToHost, stream)) != hipSuccess) return e;
  if ((e = hipStreamSynchronize(stream)) != hipSuccess) return e;
  // workgroups b and b % 8 share an XCD, and the 8 groups sit on 8 different XCDs
  bool ok = true;
  for (int b = 0; b < NWG; ++b) ok &= ids[b] == ids[b % NXCD];
  for (int x = 0; x < NXCD; ++x)
    for (int y = 0; y < x; ++y) ok &= ids[x] != ids[y];
  *placement_ok = ok;
  hipLaunchKernelGGL(ws_init_kernel, dim3(64), dim3(256), 0, stream, static_cast<u64*>(ws));
  if ((e = hipGetLastError()) != hipSuccess) return e;
  return hipStreamSynchronize(stream);
}

static hipError_t current_device(int* dev) {
  hipError_t e = hipGetDevice(dev);
  if (e != hipSuccess) return e;
  return (*dev < 0 || *dev >= MAX_DEVICES) ? hipErrorInvalidDevice : hipSuccess;
}

// The current device's state, checked once. Allocates nothing.
static hipError_t device_state(DeviceState** out) {
  int dev = 0;
  hipError_t e = current_device(&dev);
  if (e != hipSuccess) return e;
  std::lock_guard<std::mutex> lk(g_mu);
  DeviceState& s = g_dev[dev];
  if (!s.init) {
    s.init = true;
    s.err = check_device(dev);
  }
  if (s.err != hipSuccess) return s.err;
  *out = &s;
  return hipSuccess;
}

// A newly initialised workspace set starts drained while a drain is pending (mk_request_drain).
static hipError_t mark_if_draining(bool drain_pending, void* ws, hipStream_t stream) {
  if (!drain_pending) return hipSuccess;
  hipLaunchKernelGGL(ws_raise_kernel, dim3(1), dim3(64), 0, stream, static_cast<u64*>(ws), ERR_HOST);
  return hipGetLastError();
}

// The workspace set of `stream` on the current device, allocated and initialised on the stream's
// first launch. Launches on different streams never share exchange words or epochs. With every slot
// taken, the least recently used set is handed over: the device is synchronized first (no launch on
// any stream can still use it), its status bits are kept, and it is initialised again on `stream`.
static hipError_t stream_workspace(DeviceState* st, hipStream_t stream, void** out) {
  std::lock_guard<std::mutex> lk(g_mu);
  const uint64_t now = ++st->launches;
  for (int i = 0; i < st->nws; ++i)
    if (st->ws[i].stream == stream) { st->ws[i].last_use = now; *out = st->ws[i].ws; return hipSuccess; }
  hipError_t e;
  bool placement_ok = false;
  if (st->nws == MAX_STREAMS) {
    int v = 0;
    for (int i = 1; i < st->nws; ++i)
      if (st->ws[i].last_use < st->ws[v].last_use) v = i;
    if ((e = hipDeviceSynchronize()) != hipSuccess) return e;
    for (int i = 0; i < NSHAPE; ++i) {
      uint32_t w = 0;
      if ((e = hipMemcpy(&w, (char*)st->ws[v].ws + i * WS_BYTES + X_STATUS * 8, 4, hipMemcpyDeviceToHost)) != hipSuccess)
        return e;
      st->retired_status |= w;
    }
    if ((e = init_workspace(st->ws[v].ws, stream, &placement_ok)) != hipSuccess) return e;
    if ((e = mark_if_draining(st->drain_pending, st->ws[v].ws, stream)) != hipSuccess) return e;
    if (!placement_ok) st->force_wt = true;
    st->ws[v].stream = stream;
    st->ws[v].last_use = now;
    *out = st->ws[v].ws;
    return hipSuccess;
  }
  void* ws = nullptr;
  if ((e = hipMalloc(&ws, WS_SET_BYTES)) != hipSuccess) return e;
  if ((e = init_workspace(ws, stream, &placement_ok)) != hipSuccess) { (void)hipFree(ws); return e; }
  if ((e = mark_if_draining(st->drain_pending, ws, stream)) != hipSuccess) { (void)hipFree(ws); return e; }
  if (!placement_ok) st->force_wt = true;
  st->ws[st->nws++] = {stream, ws, now};
  *out = ws;
  return hipSuccess;
}

// The static workspace set of the current device: its address via hipGetSymbolAddress and its
// initialisation, once per device. Calls no allocating routine.
static hipError_t static_workspace(hipStream_t stream, void** out, bool* force_wt) {
  int dev = 0;
  hipError_t e = current_device(&dev);
  if (e != hipSuccess) return e;
  std::lock_guard<std::mutex> lk(g_mu);
  StaticState& s = g_static[dev];
  if (!s.init) {
    s.init = true;
    s.err = check_device(dev);
    if (s.err == hipSuccess) s.err = hipGetSymbolAddress(&s.ptr, HIP_SYMBOL(scratch));
    if (s.err == hipSuccess && s.ptr == nullptr) s.err = hipErrorInvalidSymbol;
    bool placement_ok = false;
    if (s.err == hipSuccess) s.err = init_workspace(s.ptr, stream, &placement_ok);
    if (s.err == hipSuccess) s.err = mark_if_draining(g_dev[dev].drain_pending, s.ptr, stream);
    s.force_wt = !placement_ok;
  }
  if (s.err != hipSuccess) return s.err;
  *out = s.ptr;
  *force_wt = s.force_wt;
  return hipSuccess;
}

// The grid's workgroups wait on each other, so all 256 must be resident at once: one per CU, which
// check_kernel_fits() verified, and kernels on one stream never overlap. A plain launch is the
// default: it costs ~16 us less per token than a cooperative one (measured on the MI355X: 423 vs
// 440 us per step). If a kernel from another stream or process holds CUs, the workgroups that did
// start wait for the rest with bounded spins; past the bound the launch ends with the status
// timeout bit set, NaN logits and token -1 instead of hanging. mk_set_launch_mode(1) selects
// hipLaunchCooperativeKernel, whose runtime guarantees co-residency before the grid starts.
template <int H, int I>
static hipError_t launch(KArgs& k, hipStream_t stream, bool cooperative) {
  void* args[] = {(void*)&k};
  const void* f = split_plan<H>(k.position + 1).nkv == 1 ? (const void*)decode_kernel<H, I, 1>
                                                   : (const void*)decode_kernel<H, I, 2>;
  if (cooperative) return hipLaunchCooperativeKernel(f, dim3(NWG), dim3(NT), args, 0, stream);
  return hipLaunchKernel(f, dim3(NWG), dim3(NT), args, 0, stream);
}

// Argument checks shared by the entry points (no HIP call); fills the launch arguments of one step
// at `position` except the token fields.
static hipError_t prepare(const mk_model_dims* dims, const void* embed_weight, const void* lm_head_weight,
                          const void* final_norm_weight, const void* layer_weights, const void* cos_table,
                          const void* sin_table, void* k_cache, void* v_cache, int position, int max_seq_len,
                          float* logits, KArgs& k, bool& s06) {
  if (!dims || !embed_weight || !lm_head_weight || !final_norm_weight || !layer_weights || !cos_table ||
      !sin_table || !k_cache || !v_cache || !logits)
    return hipErrorInvalidValue;
  s06 = dims->hidden == 1024 && dims->intermediate == 3072;
  const bool s17 = dims->hidden == 2048 && dims->intermediate == 6144;
  if (!(s06 || s17) || dims->num_layers < 1 || dims->num_layers > MAX_LAYERS || dims->vocab < NWG) return hipErrorInvalidValue;
  if (max_seq_len < 1 || position < 0 || position >= max_seq_len) return hipErrorInvalidValue;
  k.embed = (const uint16_t*)embed_weight;
  k.lm_head = (const uint16_t*)lm_head_weight;
  k.final_norm = (const uint16_t*)final_norm_weight;
  k.layers = (const mk_layer_weights*)layer_weights;
  k.cos_tab = (const uint16_t*)cos_table;
  k.sin_tab = (const uint16_t*)sin_table;
  k.k_cache = (uint16_t*)k_cache;
  k.v_cache = (uint16_t*)v_cache;
  k.logits = logits;
  k.out_token = nullptr;
  k.token_in = nullptr;
  k.block_table = nullptr;
  k.num_pages = 0;
  k.page_shift = 0;
  k.token = 0;
  k.position = position;
  k.max_seq = max_seq_len;
  k.num_layers = dims->num_layers;
  k.vocab = dims->vocab;
  k.force_wt = 0;
  k.xw = nullptr;
  k.trace = nullptr;
  return hipSuccess;
}

// One launch on workspace set `ws`.
static hipError_t launch_on(const KArgs& k, bool s06, void* ws, bool force_wt, const DeviceState* st,
                            hipStream_t stream) {
  KArgs a = k;
  a.xw = (u64*)((char*)ws + (s06 ? 0 : WS_BYTES));
  a.trace = st->trace;
  a.force_wt = force_wt ? 1 : 0;
  return s06 ? launch<1024, 3072>(a, stream, st->cooperative) : launch<2048, 6144>(a, stream, st->cooperative);
}

// One launch on the stream's own workspace set.
static hipError_t launch_step(const KArgs& k, bool s06, hipStream_t stream) {
  DeviceState* st = nullptr;
  hipError_t e = device_state(&st);
  if (e != hipSuccess) return e;
  void* ws = nullptr;
  if ((e = stream_workspace(st, stream, &ws)) != hipSuccess) return e;
  return launch_on(k, s06, ws, st->force_wt, st, stream);
}

// Every workspace set of the current device (allocated ones, and the static one once initialised).
template <typename F>
static hipError_t for_each_workspace(F f) {
  DeviceState* st = nullptr;
  hipError_t e = device_state(&st);
  if (e != hipSuccess) return e;
  int dev = 0;
  if ((e = current_device(&dev)) != hipSuccess) return e;
  std::lock_guard<std::mutex> lk(g_mu);
  for (int i = 0; i < st->nws; ++i)
    if ((e = f(st->ws[i].ws)) != hipSuccess) return e;
  if (g_static[dev].init && g_static[dev].err == hipSuccess && (e = f(g_static[dev].ptr)) != hipSuccess) return e;
  return hipSuccess;
}

}  // namespace mk

using namespace mk;

extern "C" hipError_t mk_decode(const mk_model_dims* dims, int token_id, const void* embed_weight,
                                const void* lm_head_weight, const void* final_norm_weight,
                                const void* layer_weights, const void* cos_table, const void* sin_table,
                                void* k_cache, void* v_cache, int position, int max_seq_len, float* logits,
                                int32_t* out_token, hipStream_t stream) {
  KArgs k;
  bool s06 = false;
  hipError_t e = prepare(dims, embed_weight, lm_head_weight, final_norm_weight, layer_weights, cos_table, sin_table,
                         k_cache, v_cache, position, max_seq_len, logits, k, s06);
  if (e != hipSuccess) return e;
  if (token_id < 0 || token_id >= dims->vocab) return hipErrorInvalidValue;
  k.token = token_id;
  k.out_token = out_token;
  return launch_step(k, s06, stream);
}

extern "C" hipError_t mk_decode_noalloc(const mk_model_dims* dims, int token_id, const void* embed_weight,
                                        const void* lm_head_weight, const void* final_norm_weight,
                                        const void* layer_weights, const void* cos_table, const void* sin_table,
                                        void* k_cache, void* v_cache, int position, int max_seq_len, float* logits,
                                        int32_t* out_token, hipStream_t stream) {
  KArgs k;
  bool s06 = false;
  hipError_t e = prepare(dims, embed_weight, lm_head_weight, final_norm_weight, layer_weights, cos_table, sin_table,
                         k_cache, v_cache, position, max_seq_len, logits, k, s06);
  if (e != hipSuccess) return e;
  if (token_id < 0 || token_id >= dims->vocab) return hipErrorInvalidValue;
  DeviceState* st = nullptr;
  if ((e = device_state(&st)) != hipSuccess) return e;
  void* ws = nullptr;
  bool force_wt = false;
  if ((e = static_workspace(stream, &ws, &force_wt)) != hipSuccess) return e;
  k.token = token_id;
  k.out_token = out_token;
  return launch_on(k, s06, ws, force_wt, st, stream);
}

// Page-table checks and fields of a paged launch (page size a power of two up to 4096, at most
// MAX_PAGES table entries for max_seq_len positions).
static hipError_t set_paged(KArgs& k, const int32_t* block_table, int num_pages, int page_size, int max_seq_len) {
  int shift = 0;
  while (shift < 12 && (1 << shift) < page_size) ++shift;
  if (!block_table || num_pages < 1 || page_size < 1 || (1 << shift) != page_size ||
      (max_seq_len + page_size - 1) / page_size > MAX_PAGES)
    return hipErrorInvalidValue;
  k.block_table = block_table;
  k.num_pages = num_pages;
  k.page_shift = shift;
  return hipSuccess;
}

// n launches at positions position .. position + n - 1 with device-side tokens (see mk_decode_steps).
static hipError_t run_steps(KArgs& k, bool s06, int32_t* tokens, int n, int generate, int position,
                            int max_seq_len, hipStream_t stream) {
  if (!tokens || n < 1 || (long long)position + n > max_seq_len) return hipErrorInvalidValue;
  for (int i = 0; i < n; ++i) {
    k.position = position + i;
    k.token_in = tokens + i;
    k.out_token = (generate || i == n - 1) ? tokens + i + 1 : nullptr;
    hipError_t e = launch_step(k, s06, stream);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

extern "C" hipError_t mk_decode_paged(const mk_model_dims* dims, int token_id, const void* embed_weight,
                                      const void* lm_head_weight, const void* final_norm_weight,
                                      const void* layer_weights, const void* cos_table, const void* sin_table,
                                      void* k_pages, void* v_pages, const int32_t* block_table, int num_pages,
                                      int page_size, int position, int max_seq_len, float* logits,
                                      int32_t* out_token, hipStream_t stream) {
  KArgs k;
  bool s06 = false;
  hipError_t e = prepare(dims, embed_weight, lm_head_weight, final_norm_weight, layer_weights, cos_table, sin_table,
                         k_pages, v_pages, position, max_seq_len, logits, k, s06);
  if (e != hipSuccess) return e;
  if (token_id < 0 || token_id >= dims->vocab) return hipErrorInvalidValue;
  if ((e = set_paged(k, block_table, num_pages, page_size, max_seq_len)) != hipSuccess) return e;
  k.token = token_id;
  k.out_token = out_token;
  return launch_step(k, s06, stream);
}

extern "C" hipError_t mk_decode_steps(const mk_model_dims* dims, int32_t* tokens, int n, int generate,
                                      const void* embed_weight, const void* lm_head_weight,
                                      const void* final_norm_weight, const void* layer_weights,
                                      const void* cos_table, const void* sin_table, void* k_cache, void* v_cache,
                                      int position, int max_seq_len, float* logits, hipStream_t stream) {
  KArgs k;
  bool s06 = false;
  hipError_t e = prepare(dims, embed_weight, lm_head_weight, final_norm_weight, layer_weights, cos_table, sin_table,
                         k_cache, v_cache, position, max_seq_len, logits, k, s06);
  if (e != hipSuccess) return e;
  return run_steps(k, s06, tokens, n, generate, position, max_seq_len, stream);
}

extern "C" hipError_t mk_decode_steps_paged(const mk_model_dims* dims, int32_t* tokens, int n, int generate,
                                            const void* embed_weight, const void* lm_head_weight,
                                            const void* final_norm_weight, const void* layer_weights,
                                            const void* cos_table, const void* sin_table, void* k_pages,
                                            void* v_pages, const int32_t* block_table, int num_pages, int page_size,
                                            int position, int max_seq_len, float* logits, hipStream_t stream) {
  KArgs k;
  bool s06 = false;
  hipError_t e = prepare(dims, embed_weight, lm_head_weight, final_norm_weight, layer_weights, cos_table, sin_table,
                         k_pages, v_pages, position, max_seq_len, logits, k, s06);
  if (e != hipSuccess) return e;
  if ((e = set_paged(k, block_table, num_pages, page_size, max_seq_len)) != hipSuccess) return e;
  return run_steps(k, s06, tokens, n, generate, position, max_seq_len, stream);
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
  hipError_t e = hipDeviceSynchronize();
  if (e != hipSuccess) return e;
  uint32_t acc = 0;
  e = for_each_workspace([&](void* ws) {
    for (int i = 0; i < NSHAPE; ++i) {
      uint32_t w = 0;
      hipError_t r = hipMemcpy(&w, (char*)ws + i * WS_BYTES + X_STATUS * 8, 4, hipMemcpyDeviceToHost);
      if (r != hipSuccess) return r;
      acc |= w;
    }
    return hipSuccess;
  });
  if (e != hipSuccess) return e;
  DeviceState* st = nullptr;
  if ((e = device_state(&st)) != hipSuccess) return e;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    acc |= st->retired_status;
  }
  *status = acc;
  return hipSuccess;
}

extern "C" hipError_t mk_reset(void) {
  hipError_t e = hipDeviceSynchronize();
  if (e != hipSuccess) return e;
  mkb_set_drain(false);
  DeviceState* st = nullptr;
  if ((e = device_state(&st)) != hipSuccess) return e;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    st->drain_pending = false;
    st->retired_status = 0;
  }
  e = for_each_workspace([](void* ws) {
    hipLaunchKernelGGL(ws_init_kernel, dim3(64), dim3(256), 0, 0, static_cast<u64*>(ws));
    return hipGetLastError();
  });
  if (e != hipSuccess) return e;
  return hipDeviceSynchronize();
}

extern "C" hipError_t mk_request_drain(void) {
  hipError_t e = hipDeviceSynchronize();
  if (e != hipSuccess) return e;
  mkb_set_drain(true);
  DeviceState* st = nullptr;
  if ((e = device_state(&st)) != hipSuccess) return e;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    st->drain_pending = true;  // workspace sets created from now on start drained too
  }
  e = for_each_workspace([](void* ws) {
    hipLaunchKernelGGL(ws_raise_kernel, dim3(1), dim3(64), 0, 0, static_cast<u64*>(ws), ERR_HOST);
    return hipGetLastError();
  });
  if (e != hipSuccess) return e;
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

extern "C" hipError_t mk_set_launch_mode(int cooperative) {
  if (cooperative != 0 && cooperative != 1) return hipErrorInvalidValue;
  DeviceState* st = nullptr;
  hipError_t e = device_state(&st);
  if (e != hipSuccess) return e;
  st->cooperative = cooperative != 0;
  return hipSuccess;
}

extern "C" size_t mk_trace_bytes(void) { return (size_t)NWG * TRACE_N * sizeof(uint64_t); }

extern "C" size_t mk_workspace_bytes(void) { return WS_SET_BYTES; }

extern "C" int mk_grid_size(void) {
  DeviceState* st = nullptr;
  return device_state(&st) == hipSuccess ? NWG : -1;
}

extern "C" const char* mk_version(void) { return "megakernel_amd 0.24 (gfx950; 32-bit LL exchanges, 8 math waves, phase-ahead weight prefetch split across hops, gate/up rows early on split-free workgroups, max-first split merge, early LM-head rows, plain launch, device-side token loop, paged cache, per-stream workspaces, in-band failure; prefill GEMMs on fragment-major activations with K steps in flight in issue order, prefill attention in key-range chunks, skinny products with 4 activation blocks in flight)"; }
