// Persistent batched decode on MI355X (gfx950): up to 16 sequences of the Qwen3-0.6B shape advance
// one token each in one launch of 256 workgroups, one per CU, with no grid barrier and no kernel
// boundary between layers.
//
// The reference decodes one sequence per launch (/root/reference/megakernel.cu:744-994, a cooperative
// grid with grid.sync() between phases). The layer-by-layer engine of this library runs a batch as
// ~220 short kernels per step, and on MI355X every kernel boundary costs a few microseconds (launch,
// cache write-back and invalidation across the 8 XCDs) on top of each kernel's own ramp. Here the
// batch is the columns of the matrix-core tiles instead (sequence b's activations as bf16 hi in
// column 2b and lo in column 2b + 1: one block of 16 columns for up to 8 sequences, two for up to
// 16), and workgroups hand data to each other through 32-bit
// "LL" words (value and epoch in one word) as the single-sequence decode kernel does:
//
//   XCD x owns K/V head x: its 512 q/k/v rows (16 per workgroup), its attention, its 256 input
//   columns of o_proj (32 output rows per workgroup), 1/8 of the MLP (12 intermediates per
//   workgroup) and those intermediates' columns of down_proj (32 rows per workgroup). Per layer:
//     A  input RMSNorm -> QKV rows (MFMA)                       -> publish (local)
//     B  split-K attention of one (sequence, key range) per workgroup, q/k norm + RoPE, cache write
//                                                               -> publish partial (local)
//     C  merge of every sequence's splits -> o_proj partial      -> publish (cross-XCD)
//     D  workgroup j adds row block j over the 8 XCDs to the residual -> republish (local)
//     E  post-attention RMSNorm -> gate/up + SiLU                -> publish (local)
//     F  down_proj partial                                       -> publish (cross-XCD)
//     G  workgroup j adds row block j over the 8 XCDs to the residual -> republish (local)
//   then the final norm and the tied LM head with the greedy keys (finish kernel: tokens).
//
// The fp32 residual of row block j lives in the registers of the lanes that sum that block (each
// XCD's workgroup j holds a bitwise identical copy: same data, same order); every workgroup reads
// the whole residual back from its XCD's republished words before a norm. Waves 0-3 (comm) poll,
// publish and do the vector work; waves 4-11
// (math) hold weights in registers, issued phases ahead, and run the MFMA tiles and the attention.
// Workgroups learn their XCD from the hardware register and their index in it from a ticket counter,
// so the exchange layout never depends on how the dispatcher placed the grid. Every wait is
// bounded; a timeout (or a host drain request) aborts the launch, which then reports NaN logits
// and token -1 for every sequence.
//
// Numerics: fp32 residual, fp32 RMSNorm (scale applied to the product outputs, a linear map), fp32
// softmax, exchanged values (partials, and the residual as read for a norm) rounded to 24 bits, bf16
// new K/V.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
#include <mutex>

#include "mk_device.h"
#include "mk_batch.h"
#include "mk_layers.h"

namespace mkb {
using namespace mk;
using namespace mkp;

constexpr int NXCD = 8, WPX = 32, NWG = NXCD * WPX;
constexpr int NCW = 4, NMW = 8, NWAVE = NCW + NMW, NT = 64 * NWAVE;  // 768 threads
constexpr int CL = 64 * NCW;            // comm lanes
constexpr int BMAX = MKB_MAX;           // sequences per launch: CB column blocks of 8 (hi and lo of 8 fill 16 columns)
constexpr int H = 1024, I = 3072, IX = I / NXCD;
constexpr int QX = 4 * D;               // q (2 heads), k, v rows of one K/V head: 512
constexpr int QR = QX / WPX;            // 16 rows per workgroup
constexpr int OR = H / WPX;             // 32 o_proj rows (and down_proj rows) per workgroup
constexpr int GI = IX / WPX;            // 12 intermediates per workgroup
constexpr int APW = 2 * D + 4;          // attention partial: acc[2][128], m0, l0, m1, l1
constexpr int KST = H + 8;              // LDS row stride of the MFMA B operand (bf16): conflict-free reads
template <int CB> constexpr int rst() { return 16 * CB + 4; }  // reduction tile row stride (floats): conflict-free
constexpr int MAXL = 32;
constexpr int NG = 4 * NMW;             // 16-lane attention groups per workgroup
constexpr int RB = 4;                   // keys per group and round of K/V loads
constexpr uint32_t SPIN_LIMIT = 1u << 22;
static_assert(QR == 16 && OR == 32 && GI == 12, "work split of the 0.6B shape");

// Where the math waves issue each group of weight (and K/V) loads, as points of their layer loop:
//   0 after A1 (before the QKV tile)      1 after A2        2 after B1 (before the attention)
//   3 after the split partial's publish   4 after C1        5 after C2 (before the o_proj tile)
//   6 after C3    7 after E1 (before the gate/up tile)     8 after E2    9 after F1    10 after F2
// (points 2 and 3 are point 1 on a workgroup without a key range). gate/up and down rows are issued
// in the layer that uses them (at most 6 and 8), QKV, o_proj and the first K/V round for the next
// layer (at least 1, 6 and 3). A burst of loads delays any poll of the same CU issued after it, so
// each goes where the comm waves' next poll is furthest away. Measured at 8 sequences of 257 keys
// (0.6B): gate/up+down after the attention publish 797 us per step, gate/up after C1 729, and
// gate/up after C1 and C3 with down after E2 708. Later, at 8 and 16 sequences: down after E1 613
// and 840 us, after E2 618 and 856; the next layer's first K/V round after F1 641 and 875, after F2
// 627 and 857.
// The split merge on all waves (true) or on the comm waves only, the math waves issuing loads meanwhile.
constexpr bool MERGE_ALL = true;
// K steps per load chunk of the LM head (two chunks in flight per wave).
constexpr int LM_CH = 8;
// Polls of up to POLL_TWO_MAX chunks per lane keep two rounds of loads in flight.
constexpr int POLL_TWO_MAX = 4;
constexpr int GU_AT = 4;
constexpr int GU2_AT = 6;  // >= 0: the second half of the gate/up rows at this point (-1: all at GU_AT)
constexpr int DN_AT = 7;
constexpr int QKV_AT = 6;
constexpr int O_AT = 10;
constexpr int KV_AT = 8;
static_assert(GU_AT <= 6 && DN_AT <= 8 && QKV_AT >= 1 && O_AT >= 6 && KV_AT >= 3,
              "load schedule");

// Exchange area (32-bit words) of a launch with up to BM sequences, zeroed before every launch
// (epoch 0 never matches).
template <int BM>
struct WL {
  static constexpr size_t QX_ = 0;                                     // [8][BM][512]    q/k/v sums (local)
  static constexpr size_t AX = QX_ + (size_t)NXCD * BM * QX;           // [8][32][260]    split partials (local)
  static constexpr size_t OX = AX + (size_t)NXCD * WPX * APW;          // [32][8][BM][32] o_proj partials (cross)
  static constexpr size_t OL = OX + (size_t)WPX * NXCD * BM * OR;      // [8][BM][H]      o_proj sums (local)
  static constexpr size_t MX = OL + (size_t)NXCD * BM * H;             // [8][BM][IX]     silu(gate) * up (local)
  static constexpr size_t DX = MX + (size_t)NXCD * BM * IX;            // [32][8][BM][32] down partials (cross)
  static constexpr size_t DL = DX + (size_t)WPX * NXCD * BM * OR;      // [8][BM][H]      down sums (local)
  static constexpr size_t TICK = DL + (size_t)NXCD * BM * H;           // [8] ticket counters, 64 words apart
  static constexpr size_t ABORT = TICK + NXCD * 64;                    // nonzero: the launch gave up
  static constexpr size_t BAD = ABORT + 64;                            // nonzero: a token or position was out of range
  static constexpr size_t ZERO = BAD + 64;                             // words zeroed per launch
  static constexpr size_t KEYS = ZERO;                                 // u64 [NWG][BM] greedy keys per workgroup
  static constexpr size_t END = KEYS + 2 * (size_t)NWG * BM;
  static_assert(AX % 4 == 0 && OX % 4 == 0 && OL % 4 == 0 && MX % 4 == 0 && DX % 4 == 0 && DL % 4 == 0 &&
                    KEYS % 2 == 0,
                "16-byte chunks");
};
constexpr size_t WS_BYTES = WL<BMAX>::END * 4;

struct BArgs {
  const int32_t* tokens;
  const int32_t* positions;
  const uint16_t* embed;
  const uint16_t* lm_head;
  const uint16_t* final_norm;
  const uint16_t* cos_tab;
  const uint16_t* sin_tab;
  uint16_t* k_cache;  // [B][L][8][max_seq][128]
  uint16_t* v_cache;
  float* logits;      // [B][vocab]
  uint32_t* ws;
  int B, L, vocab, max_seq, drain;
  uint64_t* trace;  // optional phase stamps (mk_set_batch_trace), null in normal operation
  mk_layer_weights lw[MAXL];
};

// Phase trace: per workgroup (j * 8 + x) and layer, TRACE_SLOTS s_memrealtime stamps (100 MHz) taken
// by thread 0 (comm wave 0) at fixed points; row MAXL holds kernel start, LM-head start and end.
constexpr int TRACE_SLOTS = 24;
constexpr size_t TRACE_BYTES = (size_t)NWG * (MAXL + 1) * TRACE_SLOTS * 8;
__device__ __forceinline__ void mark(const BArgs& a, int x, int j, int row, int slot, int who = 0) {
  if (a.trace && threadIdx.x == who)
    a.trace[((size_t)(j * NXCD + x) * (MAXL + 1) + row) * TRACE_SLOTS + slot] = __builtin_amdgcn_s_memrealtime();
}

typedef unsigned u4v __attribute__((ext_vector_type(4)));

// LDS of a launch with NCB column blocks of the MFMA operand (up to 8 NCB sequences).
template <int NCB>
struct Smem {
  static constexpr int CB = NCB, BM = 8 * NCB;
  uint16_t act[16 * CB][KST];    // MFMA B operand: column 2b = hi, 2b + 1 = lo of sequence b
  float red[NMW][16][rst<CB>()];  // per-wave MFMA results (columns as in act)
  float gacc[NG][2][D];          // attention group partials
  float gml[NG][4];
  float stg[WPX * APW];          // polled split partials
  alignas(16) float raw[2 * D];  // this workgroup's sequence's q (2 heads, normalised and rotated)
  alignas(16) uint16_t kvn[2][D];  // its new K (normalised, rotated) and V rows, bf16
  float ssw[NCW][BM];            // per comm wave sums of squares
  alignas(16) uint16_t cs[2][D];  // cos, sin at this workgroup's split's position
  u64 wk[NWAVE][BM];             // LM head keys per wave
  int pos[BM], tok[BM], f[BM], ns[BM], sb[WPX];
  int x, j, nsplit, ks, bad;
  uint32_t badseq;  // bit b: sequence b's position or token is out of range
};

// threadIdx.x with its origin hidden from the optimizer: lane offsets derived from it are recomputed
// where they are used instead of being hoisted out of the layer loop and held in registers.
__device__ __forceinline__ int tix() {
  int v = threadIdx.x;
  asm volatile("" : "+v"(v));
  return v;
}

// LL word of v: v rounded at mantissa bit 8, epoch ep (1..255) in the low byte.
__device__ __forceinline__ uint32_t llw(float v, uint32_t ep) { return ((__float_as_uint(v) + 0x80u) & 0xFFFFFF00u) | ep; }
__device__ __forceinline__ float llv(uint32_t w) { return __uint_as_float(w & 0xFFFFFF00u); }

// 4 LL words at word offset `off` (per lane) of the wave-uniform `base`: local words stay in the XCD's
// L2, cross-XCD words are written through (device scope). The buffer descriptor is built from the
// uniform base only; a per-lane base would make the compiler loop over the lanes' descriptors.
template <bool CROSS>
__device__ __forceinline__ void st4(uint32_t* base, int off, const float (&v)[4], uint32_t ep) {
  const u4v w = {llw(v[0], ep), llw(v[1], ep), llw(v[2], ep), llw(v[3], ep)};
  __builtin_amdgcn_raw_buffer_store_b128(w, make_rsrc(base), off * 4, 0, CROSS ? CPOL_SC1 : 0);
}
__device__ __forceinline__ void st1(uint32_t* base, int off, float v, uint32_t ep) {
  __builtin_amdgcn_raw_buffer_store_b32(llw(v, ep), make_rsrc(base), off * 4, 0, 0);
}

struct Ctl {
  uint32_t* abort;  // the launch's abort word
  bool failed;
};

// Polls NK 16-byte chunks of LL words per lane, at byte offsets off[k] from base (device-scope loads),
// until every epoch equals ep; the lanes of a wave wait together. Up to 4 chunks per lane two rounds
// of loads are kept in flight, so data that lands while one round is out is seen by the next one. Bounded: past SPIN_LIMIT rounds, or once another workgroup has given
// up (checked every 32 rounds), it sets the abort word and returns zeros.
template <int NK>
__device__ __forceinline__ void poll(Ctl& c, const uint32_t* base, const int (&off)[NK], uint32_t ep,
                                     float (&v)[NK][4]) {
  auto zero = [&]() {
#pragma unroll
    for (int k = 0; k < NK; ++k) v[k][0] = v[k][1] = v[k][2] = v[k][3] = 0.f;
  };
  if (c.failed) { zero(); return; }
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(base);
  auto issue = [&](u4v (&r)[NK]) {
#pragma unroll
    for (int k = 0; k < NK; ++k) r[k] = __builtin_bit_cast(u4v, __builtin_amdgcn_raw_buffer_load_b128(rs, off[k], 0, CPOL_SC1));
  };
  auto ready = [&](const u4v (&r)[NK]) {
    uint32_t bad = 0;
#pragma unroll
    for (int k = 0; k < NK; ++k)
#pragma unroll
      for (int i = 0; i < 4; ++i) bad |= (r[k][i] ^ ep) & 0xFFu;
    return __ballot(bad != 0) == 0;
  };
  auto take = [&](const u4v (&r)[NK]) {
#pragma unroll
    for (int k = 0; k < NK; ++k)
#pragma unroll
      for (int i = 0; i < 4; ++i) v[k][i] = llv(r[k][i]);
  };
  auto give_up = [&](uint32_t it) {
    if ((it & 63u) == 62u && ld_dev_u32(c.abort) != 0) { c.failed = true; return true; }
    if (it > SPIN_LIMIT) {
      st_dev_u32(c.abort, 1u);
      c.failed = true;
      return true;
    }
    return false;
  };
  if constexpr (NK <= POLL_TWO_MAX) {
    u4v r0[NK], r1[NK];
    issue(r0);
    for (uint32_t it = 0;; it += 2) {
      issue(r1);
      if (ready(r0)) { take(r0); return; }
      issue(r0);
      if (ready(r1)) { take(r1); return; }
      if (give_up(it)) { zero(); return; }
    }
  } else {
    u4v r0[NK];
    for (uint32_t it = 0;; it += 2) {
      issue(r0);
      if (ready(r0)) { take(r0); return; }
      if (give_up(it)) { zero(); return; }
    }
  }
}

__device__ __forceinline__ void lds_barrier() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): LDS operations only, weight loads stay in flight
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// ---- comm-wave vector work ------------------------------------------------------------------------

// x * w (w the RMSNorm weight) of every sequence's residual, polled from `src` (or, at layer 0, the
// embedding rows), into the MFMA operand as bf16 hi/lo, and each comm wave's sums of squares per
// sequence. Comm lane c holds elements 4c..4c+3 of every sequence.
template <bool EMBED, class S>
__device__ __forceinline__ void residual_norm(S& sm, Ctl& c, const BArgs& a, const uint32_t* src, uint32_t ep,
                                              const uint16_t* w) {
  constexpr int BM = S::BM;
  const int cl = tix(), e0 = 4 * cl;
  const uint2 wr = *reinterpret_cast<const uint2*>(w + e0);
  const float wv[4] = {bf16_lo(wr.x), bf16_hi(wr.x), bf16_lo(wr.y), bf16_hi(wr.y)};
  const int wave = cl >> 6, lane = cl & 63;
  float v[BM][4];
  if constexpr (EMBED) {
#pragma unroll
    for (int b = 0; b < BM; ++b) {
      const int tok = sm.tok[b < a.B ? b : 0];
      const uint2 e = *reinterpret_cast<const uint2*>(a.embed + (size_t)tok * H + e0);
      v[b][0] = bf16_lo(e.x); v[b][1] = bf16_hi(e.x); v[b][2] = bf16_lo(e.y); v[b][3] = bf16_hi(e.y);
    }
  } else {
    int off[BM];
#pragma unroll
    for (int b = 0; b < BM; ++b) off[b] = (min(b, a.B - 1) * H + e0) * 4;
    poll<BM>(c, src, off, ep, v);
  }
  float ss[BM];
#pragma unroll
  for (int b = 0; b < BM; ++b) {
    ss[b] = 0.f;
    if (b < a.B) {
      const float y[4] = {v[b][0] * wv[0], v[b][1] * wv[1], v[b][2] * wv[2], v[b][3] * wv[3]};
      uint32_t h0 = pack_bf16x2(y[0], y[1]), h1 = pack_bf16x2(y[2], y[3]);
      uint32_t l0 = pack_bf16x2(y[0] - bf16_lo(h0), y[1] - bf16_hi(h0)), l1 = pack_bf16x2(y[2] - bf16_lo(h1), y[3] - bf16_hi(h1));
      *reinterpret_cast<uint2*>(&sm.act[2 * b][e0]) = make_uint2(h0, h1);
      *reinterpret_cast<uint2*>(&sm.act[2 * b + 1][e0]) = make_uint2(l0, l1);
      ss[b] = v[b][0] * v[b][0] + v[b][1] * v[b][1] + v[b][2] * v[b][2] + v[b][3] * v[b][3];
    }
  }
  // the BM wave reductions side by side
#pragma unroll
  for (int b = 0; b < BM; ++b) ss[b] = row16_sum(ss[b]);
#pragma unroll
  for (int b = 0; b < BM; ++b) ss[b] = xsum16(ss[b]);
#pragma unroll
  for (int b = 0; b < BM; ++b) ss[b] = xsum32(ss[b]);
  if (lane < BM) {
    float mine = ss[0];
#pragma unroll
    for (int b = 1; b < BM; ++b) mine = lane == b ? ss[b] : mine;
    sm.ssw[wave][lane] = mine;
  }
}

template <class S>
__device__ __forceinline__ float norm_scale(const S& sm, int b) {
  return rsqrtf((((sm.ssw[0][b] + sm.ssw[1][b]) + sm.ssw[2][b]) + sm.ssw[3][b]) / (float)H + EPS);
}

// Sum over the waves W0..W0+NW-1 of row r of the MFMA results, hi + lo columns of sequence b (all
// LDS reads issued before the adds).
template <int W0, int NW, class S>
__device__ __forceinline__ float red_sum(const S& sm, int r, int b) {
  float v[NW][2];
#pragma unroll
  for (int m = 0; m < NW; ++m) {
    v[m][0] = sm.red[W0 + m][r][2 * b];
    v[m][1] = sm.red[W0 + m][r][2 * b + 1];
  }
  float s = 0.f;
#pragma unroll
  for (int m = 0; m < NW; ++m) s += v[m][0] + v[m][1];
  return s;
}

// Workgroup j of XCD x sums row block j (OR rows of every sequence) over the 8 XCDs' partials at
// `cross` in a fixed order, adds it to its residual rows xr and republishes them in its XCD at
// `local`. Comm waves 0..BM/8-1, thread t: sequence t / 8, rows 4 (t % 8) .. +3 of the block.
template <int BM>
__device__ __forceinline__ void gather(Ctl& c, const BArgs& a, size_t cross, size_t local, uint32_t ep, int x,
                                       int j, float (&xr)[4]) {
  const int t = tix();
  const int q8 = min(t, 8 * a.B - 1), b = q8 >> 3, q = q8 & 7;
  int off[NXCD];
#pragma unroll
  for (int xs = 0; xs < NXCD; ++xs) off[xs] = ((xs * BM + b) * OR + 4 * q) * 4;
  float v[NXCD][4];
  poll<NXCD>(c, a.ws + cross + (size_t)j * NXCD * BM * OR, off, ep, v);
  if (cross == WL<BM>::OX) mark(a, x, j, ep - 1, 17);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float s = v[0][i];
#pragma unroll
    for (int xs = 1; xs < NXCD; ++xs) s += v[xs][i];
    xr[i] += s;
  }
  if (t < 8 * a.B) st4<false>(a.ws + local + (size_t)x * BM * H + j * OR, b * H + 4 * q, xr, ep);
}

// Publishes the workgroup's OR output rows of every sequence as cross-XCD partials: tile t (computed by
// math waves 4t..4t+3) on math wave t, lane (b, 4 rows). The math waves publish every product (they
// poll nothing): on this GPU one counter tracks a wave's loads and stores, so a wave that polls after
// storing would wait for its store to be acknowledged first.
template <int T, class S>
__device__ __forceinline__ void publish_tile(const S& sm, const BArgs& a, size_t cross, uint32_t ep, int x, int j) {
  const int lane = tix() & 63;
  if (lane >= 4 * a.B) return;
  const int b = lane >> 2, r0 = 4 * (lane & 3);
  float v[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = red_sum<4 * T, 4>(sm, r0 + i, b);
  st4<true>(a.ws + cross + ((size_t)j * NXCD + x) * S::BM * OR, b * OR + 16 * T + r0, v, ep);
}
template <class S>
__device__ __forceinline__ void publish_rows(const S& sm, const BArgs& a, size_t cross, uint32_t ep, int m,
                                             int x, int j) {
  if (m == 0) publish_tile<0>(sm, a, cross, ep, x, j);
  else if (m == 1) publish_tile<1>(sm, a, cross, ep, x, j);
}
// QKV rows (all 8 math waves computed the tile over K): math wave 0, lane (b, 4 rows), scaled by the
// input norm's scale.
template <class S>
__device__ __forceinline__ void publish_qkv(const S& sm, const BArgs& a, uint32_t ep, int x, int j) {
  constexpr int BM = S::BM;
  const int lane = tix() & 63;
  if (lane >= 4 * a.B) return;
  const int b = lane >> 2, r0 = 4 * (lane & 3);
  const float rs = norm_scale(sm, b);
  float v[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = red_sum<0, NMW>(sm, r0 + i, b) * rs;
  st4<false>(a.ws + WL<BM>::QX_ + (size_t)x * BM * QX + QR * j, b * QX + r0, v, ep);
}
// silu(gate) * up of the workgroup's intermediates (gate tile on math waves 0-3, up on 4-7), scaled by
// the post-attention norm's scale: math wave 0, lane (b, 4 intermediates).
template <class S>
__device__ __forceinline__ void publish_silu(const S& sm, const BArgs& a, uint32_t ep, int x, int j) {
  constexpr int BM = S::BM;
  const int lane = tix() & 63;
  if (lane >= 3 * a.B) return;
  const int b = lane / 3, q = lane % 3;
  const float rs = norm_scale(sm, b);
  float v[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int ii = 4 * q + i;
    const float gt = red_sum<0, 4>(sm, ii, b) * rs, up = red_sum<4, 4>(sm, ii, b) * rs;
    v[i] = gt / (1.f + expf(-gt)) * up;
  }
  st4<false>(a.ws + WL<BM>::MX + (size_t)x * BM * IX + GI * j, b * IX + 4 * q, v, ep);
}

// q/k RMSNorm + rotate-half RoPE of one head row held by 32 lanes (lane c % 32: dims 4c..4c+3; the RoPE
// partner of dim d is d +- 64, 16 lanes away), as the single-sequence kernel applies them
// (/root/reference/megakernel.cu:490-630, 548-555); row 3 (v) is only rounded. Writes q as fp32 into
// raw[row][] and the new K/V rows as bf16 into kvn. Both waves' lanes take part in the swaps.
template <class S>
__device__ __forceinline__ void head_norm_rope4(S& sm, const float (&v)[4], uint2 wn, int tid) {
  const int row = tid >> 5, d0 = 4 * (tid & 31);
  float ss = v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + v[3] * v[3];
  ss = xsum16(row16_sum(ss));  // the 32 lanes of this row
  const float rs = rsqrtf(ss / (float)D + EPS);
  const float w[4] = {bf16_lo(wn.x), bf16_hi(wn.x), bf16_lo(wn.y), bf16_hi(wn.y)};
  float u[4], o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) u[i] = v[i] * rs * w[i];
  const uint2 cr = *reinterpret_cast<const uint2*>(&sm.cs[0][d0 & (D / 2 - 1)]);  // dims mod 64
  const uint2 sr = *reinterpret_cast<const uint2*>(&sm.cs[1][d0 & (D / 2 - 1)]);
  const float cs[4] = {bf16_lo(cr.x), bf16_hi(cr.x), bf16_lo(cr.y), bf16_hi(cr.y)};
  const float sn[4] = {bf16_lo(sr.x), bf16_hi(sr.x), bf16_lo(sr.y), bf16_hi(sr.y)};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    // (own, partner) in row order: an even 16-lane row gets its partner second, an odd one first
    const auto pr = __builtin_amdgcn_permlane16_swap(__float_as_uint(u[i]), __float_as_uint(u[i]), false, false);
    const float partner = __uint_as_float((tid & 16) ? pr[0] : pr[1]);
    o[i] = d0 < D / 2 ? u[i] * cs[i] - partner * sn[i] : u[i] * cs[i] + partner * sn[i];
  }
  if (row < 2) {
    *reinterpret_cast<float4*>(&sm.raw[row * D + d0]) = make_float4(o[0], o[1], o[2], o[3]);
  } else {
    const float* src = row == 2 ? o : v;
    *reinterpret_cast<uint2*>(&sm.kvn[row - 2][d0]) =
        make_uint2(pack_bf16x2(src[0], src[1]), pack_bf16x2(src[2], src[3]));
  }
}

// ---- math-wave weight loads (lane: li = row of the tile, g = 8-element K group) -------------------

struct MathLane {
  int m, li, g;  // m: math wave index, wave-uniform (readfirstlane)
};

constexpr int CPOL_NT = 2;  // non-temporal: each weight byte is read once per step
__device__ __forceinline__ uint4 ldnt(__amdgpu_buffer_rsrc_t rs, int off) {
  const u4v v = __builtin_bit_cast(u4v, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, CPOL_NT));
  return make_uint4(v[0], v[1], v[2], v[3]);
}

// Weight rows are read through buffer descriptors with a wave-uniform base and a 32-bit lane offset
// (row li of the tile, K group g): nothing 64-bit per lane stays live across the layer loop.
// QKV: workgroup j's 16 rows of the XCD's 512 (all in one of q, k, v); wave m takes K steps 4m..4m+3.
__device__ __forceinline__ void load_qkv(uint4 (&w)[4], const mk_layer_weights& lw, const MathLane& ml, int x, int j) {
  const uint16_t* base = j < 16   ? (const uint16_t*)lw.q_weight + ((size_t)2 * D * x + QR * j) * H
                         : j < 24 ? (const uint16_t*)lw.k_weight + ((size_t)D * x + QR * (j - 16)) * H
                                  : (const uint16_t*)lw.v_weight + ((size_t)D * x + QR * (j - 24)) * H;
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(base);
  const int off = (ml.li * H + 32 * 4 * ml.m + 8 * ml.g) * 2;
#pragma unroll
  for (int s = 0; s < 4; ++s) w[s] = ldnt(rs, off + 64 * s);
}
// o_proj: rows 32j + 16 (m / 4) + li, the XCD's 256 input columns; K steps 2 (m % 4), +1.
__device__ __forceinline__ void load_o(uint4 (&w)[2], const mk_layer_weights& lw, const MathLane& ml, int x, int j) {
  const __amdgpu_buffer_rsrc_t rs =
      make_rsrc((const uint16_t*)lw.o_proj_weight + (size_t)OR * j * (HQ * D) + 2 * D * x);
  const int off = ((16 * (ml.m >> 2) + ml.li) * (HQ * D) + 64 * (ml.m & 3) + 8 * ml.g) * 2;
#pragma unroll
  for (int s = 0; s < 2; ++s) w[s] = ldnt(rs, off + 64 * s);
}
// gate (waves 0-3) or up (waves 4-7) rows of the workgroup's 12 intermediates; K steps 8 (m % 4) .. +7.
// Rows 12-15 of the tile are empty: their lanes load row 11 again (every lane of the wave issues the
// same loads, so the compiler's count of loads in flight stays exact and later waits need not wait
// for the whole burst) and keep zeros.
template <int S0 = 0, int S1 = 8>
__device__ __forceinline__ void load_gu(uint4 (&w)[8], const mk_layer_weights& lw, const MathLane& ml, int x, int j) {
  const uint16_t* m0 = (const uint16_t*)(ml.m < 4 ? lw.gate_proj_weight : lw.up_proj_weight);
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(m0 + ((size_t)IX * x + GI * j) * H);
  const int off = (min(ml.li, GI - 1) * H + 256 * (ml.m & 3) + 8 * ml.g) * 2;
#pragma unroll
  for (int s = S0; s < S1; ++s) w[s] = ldnt(rs, off + 64 * s);
}
// zeros in the empty rows of the gate/up tile (applied just before the tile's MFMAs)
__device__ __forceinline__ void mask_gu(uint4 (&w)[8], const MathLane& ml) {
  if (ml.li >= GI) {
#pragma unroll
    for (int s = 0; s < 8; ++s) w[s] = make_uint4(0, 0, 0, 0);
  }
}
// down_proj: rows 32j + 16 (m / 4) + li, the XCD's 384 intermediate columns; K steps 3 (m % 4) .. +2.
__device__ __forceinline__ void load_down(uint4 (&w)[3], const mk_layer_weights& lw, const MathLane& ml, int x, int j) {
  const __amdgpu_buffer_rsrc_t rs = make_rsrc((const uint16_t*)lw.down_proj_weight + (size_t)OR * j * I + IX * x);
  const int off = ((16 * (ml.m >> 2) + ml.li) * I + 96 * (ml.m & 3) + 8 * ml.g) * 2;
#pragma unroll
  for (int s = 0; s < 3; ++s) w[s] = ldnt(rs, off + 64 * s);
}

// MFMA over NS K steps starting at step ks0 of the LDS operand, every column block with the same
// weight fragment; result to the wave's reduction tile.
template <int NS, class S>
__device__ __forceinline__ void mma_to_red(S& sm, const uint4 (&w)[NS], int ks0, const MathLane& ml) {
  f32x4 c[S::CB];
#pragma unroll
  for (int cb = 0; cb < S::CB; ++cb) c[cb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < NS; ++s)
#pragma unroll
    for (int cb = 0; cb < S::CB; ++cb) {
      const uint4 b = *reinterpret_cast<const uint4*>(&sm.act[16 * cb + ml.li][32 * (ks0 + s) + 8 * ml.g]);
      c[cb] = mfma(w[s], b, c[cb]);
    }
#pragma unroll
  for (int cb = 0; cb < S::CB; ++cb)
#pragma unroll
    for (int r = 0; r < 4; ++r) sm.red[ml.m][4 * ml.g + r][16 * cb + ml.li] = c[cb][r];
}

// ---- attention ------------------------------------------------------------------------------------

struct Split {
  bool on;
  bool wr;  // the sequence's position and token are valid: its new K/V rows are written
  int b, s, k0, k1, pos;
};

// K/V rows of round `round` of this group's keys (positions k0 + gi + NG (RB round + u)); past the split
// they re-read its last key (every lane issues the same loads, so the compiler's count of loads in
// flight stays exact; the attention skips those keys).
__device__ __forceinline__ void load_kv(uint4 (&kw)[RB], uint4 (&vw)[RB], const BArgs& a, const Split& sp, int layer,
                                        int x, int gi, int t, int round) {
  const size_t head = (((size_t)sp.b * a.L + layer) * HKV + x) * a.max_seq * D;
  const __amdgpu_buffer_rsrc_t rk = make_rsrc(a.k_cache + head), rv = make_rsrc(a.v_cache + head);
#pragma unroll
  for (int u = 0; u < RB; ++u) {
    const int p = min(sp.k0 + gi + NG * (RB * round + u), sp.k1 - 1);
    const int off = (p * D + 8 * t) * 2;
    const u4v k = __builtin_bit_cast(u4v, __builtin_amdgcn_raw_buffer_load_b128(rk, off, 0, 0));
    const u4v v = __builtin_bit_cast(u4v, __builtin_amdgcn_raw_buffer_load_b128(rv, off, 0, 0));
    kw[u] = make_uint4(k[0], k[1], k[2], k[3]);
    vw[u] = make_uint4(v[0], v[1], v[2], v[3]);
  }
}

__device__ __forceinline__ void softmax_step(float sc, const float (&v)[8], float& m, float& l, float (&acc)[8]) {
  const float nm = fmaxf(m, sc);
  const float cm = __expf(m - nm), e = __expf(sc - nm);
  l = l * cm + e;
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = acc[i] * cm + e * v[i];
  m = nm;
}


// Merge of every sequence's split partials (polled into LDS) into the o_proj operand: thread (b, head
// h, 4 dims) for b < B (B * 64 items over the workgroup), max-first over the sequence's splits.
template <class S>
__device__ __forceinline__ void merge_splits(S& sm, const BArgs& a, int o) {
  if (o >= a.B * 64) return;
  const int b = o >> 6, h = (o >> 5) & 1, d0 = 4 * (o & 31);
  const float* p = sm.stg + (size_t)sm.f[b] * APW;
  const int n = sm.ns[b];
  float4 A = make_float4(0.f, 0.f, 0.f, 0.f);
  float Ls = 0.f;
  auto add = [&](float4 acc, float l, float e) {
    A.x = fmaf(acc.x, e, A.x); A.y = fmaf(acc.y, e, A.y); A.z = fmaf(acc.z, e, A.z); A.w = fmaf(acc.w, e, A.w);
    Ls = fmaf(l, e, Ls);
  };
  if (n <= 4) {  // every load first, then the arithmetic
    float2 ml[4];
    float4 acc[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const float* q = p + (s < n ? s : 0) * APW;
      ml[s] = *reinterpret_cast<const float2*>(q + 2 * D + 2 * h);
      acc[s] = *reinterpret_cast<const float4*>(q + h * D + d0);
    }
    float M = ml[0].x;
#pragma unroll
    for (int s = 1; s < 4; ++s) M = s < n ? fmaxf(M, ml[s].x) : M;
#pragma unroll
    for (int s = 0; s < 4; ++s) add(acc[s], ml[s].y, s < n ? __expf(ml[s].x - M) : 0.f);
  } else {  // many key ranges (a long sequence in a small batch): four at a time, loads first
    float M = -INFINITY;
    for (int s0 = 0; s0 < n; s0 += 4) {
      float mm[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) mm[s] = p[min(s0 + s, n - 1) * APW + 2 * D + 2 * h];  // repeats: same max
#pragma unroll
      for (int s = 0; s < 4; ++s) M = fmaxf(M, mm[s]);
    }
    for (int s0 = 0; s0 < n; s0 += 4) {
      float2 ml[4];
      float4 acc[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const float* q = p + min(s0 + s, n - 1) * APW;
        ml[s] = *reinterpret_cast<const float2*>(q + 2 * D + 2 * h);
        acc[s] = *reinterpret_cast<const float4*>(q + h * D + d0);
      }
#pragma unroll
      for (int s = 0; s < 4; ++s) add(acc[s], ml[s].y, s0 + s < n ? __expf(ml[s].x - M) : 0.f);
    }
  }
  const float r = 1.f / Ls;
  const float y[4] = {A.x * r, A.y * r, A.z * r, A.w * r};
  const uint32_t h0 = pack_bf16x2(y[0], y[1]), h1 = pack_bf16x2(y[2], y[3]);
  const uint32_t l0 = pack_bf16x2(y[0] - bf16_lo(h0), y[1] - bf16_hi(h0)), l1 = pack_bf16x2(y[2] - bf16_lo(h1), y[3] - bf16_hi(h1));
  *reinterpret_cast<uint2*>(&sm.act[2 * b][h * D + d0]) = make_uint2(h0, h1);
  *reinterpret_cast<uint2*>(&sm.act[2 * b + 1][h * D + d0]) = make_uint2(l0, l1);
}

// Every split partial of the XCD into LDS (nsplit * 65 chunks of 16 bytes, NK per comm lane).
template <int NK, class S>
__device__ __forceinline__ void poll_splits(S& sm, Ctl& c, const BArgs& a, int x, uint32_t ep) {
  const int tid = tix(), nch = sm.nsplit * (APW / 4);
  int off[NK];
#pragma unroll
  for (int k = 0; k < NK; ++k) off[k] = 16 * min(tid + CL * k, nch - 1);
  float v[NK][4];
  poll<NK>(c, a.ws + WL<S::BM>::AX + (size_t)x * WPX * APW, off, ep, v);
#pragma unroll
  for (int k = 0; k < NK; ++k)
    if (tid + CL * k < nch)
      *reinterpret_cast<float4*>(&sm.stg[4 * (tid + CL * k)]) = make_float4(v[k][0], v[k][1], v[k][2], v[k][3]);
}

// The two roles run separate layer loops that meet at the same sequence of LDS barriers:
// A1 A2 [B1 B2] C1 C2 C3 E1 E2 F1 F2 per layer (B1, B2 on workgroups with an attention split).

// Comm waves (threads 0..255): polls, publishes, norms, reductions of the MFMA tiles; waves 0..BM/8-1
// hold the residual of row block j (thread t: sequence t / 8, rows 4 (t % 8) .. +3).
template <class S>
__device__ __forceinline__ void comm_role(S& sm, Ctl& c, const BArgs& a, const Split& sp, int x, int j) {
  constexpr int BM = S::BM;
  using W = WL<BM>;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  float xr[4];
  {
    const int q8 = min((int)threadIdx.x, 8 * a.B - 1);
    const uint2 e = *reinterpret_cast<const uint2*>(a.embed + (size_t)sm.tok[q8 >> 3] * H + OR * j + 4 * (q8 & 7));
    xr[0] = bf16_lo(e.x); xr[1] = bf16_hi(e.x); xr[2] = bf16_lo(e.y); xr[3] = bf16_hi(e.y);
  }
  for (int l = 0; l < a.L; ++l) {
    const mk_layer_weights& lw = a.lw[l];
    const uint32_t ep = (uint32_t)l + 1;
    const int tid = tix();
    // ---- A: residual + input norm (x * w into the operand; the scale goes on the outputs)
    mark(a, x, j, l, 0);
    if (l == 0) residual_norm<true>(sm, c, a, nullptr, 0, (const uint16_t*)lw.norm_weight);
    else residual_norm<false>(sm, c, a, a.ws + W::DL + (size_t)x * BM * H, ep - 1, (const uint16_t*)lw.norm_weight);
    mark(a, x, j, l, 1);
    uint2 qn = make_uint2(0, 0);  // this layer's q_norm / k_norm weights of lane tid's 4 dims (rows 0-2)
    if (sp.on && tid < 3 * D / 4)
      qn = *reinterpret_cast<const uint2*>((const uint16_t*)(tid < D / 2 ? lw.q_norm_weight : lw.k_norm_weight) +
                                           4 * (tid & 31));
    lds_barrier();  // A1
    lds_barrier();  // A2
    mark(a, x, j, l, 2);
    // ---- B: this workgroup's sequence's q/k/v sums for the attention
    if (sp.on) {
      if (tid < QX / 4) {  // waves 0-1: lane tid holds dims 4 (tid % 32) .. +3 of row tid / 32 (q0, q1, k, v)
        int off[1] = {(int)((((size_t)x * BM + sp.b) * QX + 4 * tid) * 4)};
        float v[1][4];
        poll<1>(c, a.ws + W::QX_, off, ep, v);
        head_norm_rope4(sm, v[0], qn, tid);
      }
      lds_barrier();  // B1
      mark(a, x, j, l, 4);
      lds_barrier();  // B2
      mark(a, x, j, l, 5);
    }
    // ---- C: every split partial of the XCD into LDS
    if (sm.nsplit * (APW / 4) <= 4 * CL) poll_splits<4>(sm, c, a, x, ep);
    else poll_splits<(WPX * APW / 4 + CL - 1) / CL>(sm, c, a, x, ep);
    mark(a, x, j, l, 6);
    lds_barrier();  // C1
    mark(a, x, j, l, 20);
    for (int o = tid; o < a.B * 64; o += MERGE_ALL ? NT : CL) merge_splits(sm, a, o);
    lds_barrier();  // C2
    mark(a, x, j, l, 7);
    lds_barrier();  // C3
    mark(a, x, j, l, 8);
    // ---- D, E: row block j of the o_proj partials summed over the XCDs, residual + post-attention norm
    if (wave < BM / 8) gather<BM>(c, a, W::OX, W::OL, ep, x, j, xr);
    mark(a, x, j, l, 9);
    residual_norm<false>(sm, c, a, a.ws + W::OL + (size_t)x * BM * H, ep, (const uint16_t*)lw.post_attn_norm_weight);
    mark(a, x, j, l, 10);
    lds_barrier();  // E1
    lds_barrier();  // E2
    mark(a, x, j, l, 11);
    // ---- F: the XCD's SiLU outputs into the operand
    {
      constexpr int NK = (BM * IX / 4) / CL;  // 3 per 8 sequences
      const int nch = a.B * (IX / 4);
      int off[NK];
#pragma unroll
      for (int k = 0; k < NK; ++k) off[k] = (int)(((size_t)x * BM * IX + 4 * min(tid + CL * k, nch - 1)) * 4);
      float v[NK][4];
      poll<NK>(c, a.ws + W::MX, off, ep, v);
#pragma unroll
      for (int k = 0; k < NK; ++k) {
        const int ci = tid + CL * k;
        if (ci < nch) {
          const int b = ci / (IX / 4), e0 = 4 * (ci % (IX / 4));
          uint32_t h0 = pack_bf16x2(v[k][0], v[k][1]), h1 = pack_bf16x2(v[k][2], v[k][3]);
          uint32_t l0 = pack_bf16x2(v[k][0] - bf16_lo(h0), v[k][1] - bf16_hi(h0));
          uint32_t l1 = pack_bf16x2(v[k][2] - bf16_lo(h1), v[k][3] - bf16_hi(h1));
          *reinterpret_cast<uint2*>(&sm.act[2 * b][e0]) = make_uint2(h0, h1);
          *reinterpret_cast<uint2*>(&sm.act[2 * b + 1][e0]) = make_uint2(l0, l1);
        }
      }
    }
    mark(a, x, j, l, 12);
    lds_barrier();  // F1
    lds_barrier();  // F2
    mark(a, x, j, l, 13);
    // ---- G: row block j of the down partials summed over the XCDs
    if (wave < BM / 8) gather<BM>(c, a, W::DX, W::DL, ep, x, j, xr);
    mark(a, x, j, l, 14);
  }
  // the last layer's residual, final norm
  residual_norm<false>(sm, c, a, a.ws + W::DL + (size_t)x * BM * H, (uint32_t)a.L, a.final_norm);
  lds_barrier();
}

// Math waves (threads 256..767): weights in registers (issued phases ahead), MFMA tiles, attention.
template <class S>
__device__ __forceinline__ void math_role(S& sm, const BArgs& a, const Split& sp, int x, int j) {
  using W = WL<S::BM>;
  const int tid = threadIdx.x, lane = tid & 63;
  const MathLane ml{__builtin_amdgcn_readfirstlane(tid >> 6) - NCW, lane & 15, lane >> 4};
  const int gi = 4 * ml.m + (lane >> 4), t = lane & 15;
  const int nrounds = (sp.k1 - sp.k0 + NG * RB - 1) / (NG * RB);
  uint4 wq[4], wo[2], wg[8], wd[3], kw[RB], vw[RB];
  load_qkv(wq, a.lw[0], ml, x, j);
  load_o(wo, a.lw[0], ml, x, j);
  if (sp.on) load_kv(kw, vw, a, sp, 0, x, gi, t, 0);
  for (int l = 0; l < a.L; ++l) {
    const mk_layer_weights& lw = a.lw[l];
    const uint32_t ep = (uint32_t)l + 1;
    const bool next = l + 1 < a.L;
    auto issue = [&](int p) {
      if (GU2_AT < 0 && p == GU_AT) load_gu(wg, lw, ml, x, j);
      if (GU2_AT >= 0 && p == GU_AT) load_gu<0, 4>(wg, lw, ml, x, j);
      if (GU2_AT >= 0 && p == GU2_AT) load_gu<4, 8>(wg, lw, ml, x, j);
      if (p == DN_AT) load_down(wd, lw, ml, x, j);
      if (p == QKV_AT && next) load_qkv(wq, a.lw[l + 1], ml, x, j);
      if (p == O_AT && next) load_o(wo, a.lw[l + 1], ml, x, j);
      if (p == KV_AT && next && sp.on) load_kv(kw, vw, a, sp, l + 1, x, gi, t, 0);
    };
    lds_barrier();  // A1
    issue(0);
    mma_to_red<4>(sm, wq, 4 * ml.m, ml);
    lds_barrier();  // A2
    if (ml.m == 0) publish_qkv(sm, a, ep, x, j);
    issue(1);
    if (!sp.on) {
      issue(2);
      issue(3);
    } else {
      lds_barrier();  // B1
      mark(a, x, j, l, 18, 64 * NCW);
      issue(2);
      float qa[8], qb[8];  // normalised, rotated queries of the head pair (lane t: dims 8t..8t+7)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        qa[i] = sm.raw[8 * t + i];
        qb[i] = sm.raw[D + 8 * t + i];
      }
      const uint4 knew = *reinterpret_cast<const uint4*>(&sm.kvn[0][8 * t]);
      const uint4 vnew = *reinterpret_cast<const uint4*>(&sm.kvn[1][8 * t]);
      // the split holding the new position writes its K/V rows, unless the sequence's position or
      // token was out of range: its step reports NaN and -1, and its cache stays as it was
      if (gi == 0 && sp.pos < sp.k1 && sp.wr) {
        const size_t row = ((((size_t)sp.b * a.L + l) * HKV + x) * a.max_seq + sp.pos) * D + 8 * t;
        *reinterpret_cast<uint4*>(a.k_cache + row) = knew;
        *reinterpret_cast<uint4*>(a.v_cache + row) = vnew;
      }
      float m0 = -INFINITY, m1 = -INFINITY, l0 = 0.f, l1 = 0.f, a0[8], a1[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) { a0[i] = 0.f; a1[i] = 0.f; }
      for (int rd = 0; rd < nrounds; ++rd) {
        if (rd > 0) load_kv(kw, vw, a, sp, l, x, gi, t, rd);
#pragma unroll
        for (int u = 0; u < RB; ++u) {
          const int p = sp.k0 + gi + NG * (RB * rd + u);
          const bool own = p == sp.pos;
          float kf[8], vf[8];
          unpack8(own ? knew : kw[u], kf);
          unpack8(own ? vnew : vw[u], vf);
          float d0 = 0.f, d1 = 0.f;
#pragma unroll
          for (int i = 0; i < 8; ++i) { d0 = fmaf(qa[i], kf[i], d0); d1 = fmaf(qb[i], kf[i], d1); }
          d0 = row16_sum(d0) * ATT_SCALE;
          d1 = row16_sum(d1) * ATT_SCALE;
          if (p < sp.k1) {
            softmax_step(d0, vf, m0, l0, a0);
            softmax_step(d1, vf, m1, l1, a1);
          }
        }
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) { sm.gacc[gi][0][8 * t + i] = a0[i]; sm.gacc[gi][1][8 * t + i] = a1[i]; }
      if (t == 0) { sm.gml[gi][0] = m0; sm.gml[gi][1] = l0; sm.gml[gi][2] = m1; sm.gml[gi][3] = l1; }
      mark(a, x, j, l, 19, 64 * NCW);
      lds_barrier();  // B2
      // merge of the 32 group partials: output (head h, dim d) on two adjacent lanes, 16 groups each
      const int lam = tid - 64 * NCW, o = lam >> 1, h = o >> 7, d = o & (D - 1), half = lam & 1;
      float mg[NG / 2], M = -INFINITY;
#pragma unroll
      for (int q = 0; q < NG / 2; ++q) mg[q] = sm.gml[16 * half + q][2 * h];
#pragma unroll
      for (int q = 0; q < NG / 2; ++q) M = fmaxf(M, mg[q]);
      M = fmaxf(M, dpp<0xB1>(M));  // the other half's groups
      float ga[NG / 2], gl[NG / 2];
#pragma unroll
      for (int q = 0; q < NG / 2; ++q) {
        ga[q] = sm.gacc[16 * half + q][h][d];
        gl[q] = sm.gml[16 * half + q][2 * h + 1];
      }
      float A = 0.f, Ls = 0.f;
#pragma unroll
      for (int q = 0; q < NG / 2; ++q) {
        const float e = __expf(mg[q] - M);
        A = fmaf(ga[q], e, A);
        Ls = fmaf(gl[q], e, Ls);
      }
      A += dpp<0xB1>(A);
      Ls += dpp<0xB1>(Ls);
      if (half == 0) {
        uint32_t* base = a.ws + W::AX + ((size_t)x * WPX + j) * APW;
        st1(base, o, A, ep);
        if (d == 0) {
          st1(base, 2 * D + 2 * h, M, ep);
          st1(base, 2 * D + 2 * h + 1, Ls, ep);
        }
      }
      mark(a, x, j, l, 15, 64 * NCW);
      issue(3);
    }
    lds_barrier();  // C1
    issue(4);
    mark(a, x, j, l, 22, 64 * NCW);
    if (MERGE_ALL) merge_splits(sm, a, tid);
    mark(a, x, j, l, 23, 64 * NCW);
    lds_barrier();  // C2
    issue(5);
    mma_to_red<2>(sm, wo, 2 * (ml.m & 3), ml);
    lds_barrier();  // C3
    publish_rows(sm, a, W::OX, ep, ml.m, x, j);
    mark(a, x, j, l, 16, 64 * NCW);
    issue(6);
    lds_barrier();  // E1
    issue(7);
    mask_gu(wg, ml);
    mma_to_red<8>(sm, wg, 8 * (ml.m & 3), ml);
    lds_barrier();  // E2
    if (ml.m == 0) publish_silu(sm, a, ep, x, j);
    issue(8);
    lds_barrier();  // F1
    issue(9);
    mma_to_red<3>(sm, wd, 3 * (ml.m & 3), ml);
    lds_barrier();  // F2
    publish_rows(sm, a, W::DX, ep, ml.m, x, j);
    issue(10);
  }
  lds_barrier();  // the final norm
}

// ------------------------------------------------------------------------------------------------

template <int CB>
__global__ void __launch_bounds__(NT, 1) batch_kernel(const BArgs a) {
  constexpr int BM = 8 * CB;
  using W = WL<BM>;
  __shared__ __attribute__((aligned(16))) Smem<CB> sm;
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const bool comm = wave < NCW;
  Ctl c{a.ws + W::ABORT, a.drain != 0};

  // ---- identity, inputs, split plan
  if (tid == 0) {
    const int x = (int)(xcc_id() & 7u);
    sm.x = x;
    sm.j = (int)__hip_atomic_fetch_add(a.ws + W::TICK + 64 * x, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    sm.bad = 0;
    sm.badseq = 0;
  }
  if (tid >= 64 && tid < 64 + BM) {
    const int b = tid - 64;
    int p = 0, t = 0;
    if (b < a.B) {
      p = a.positions[b];
      t = a.tokens[b];
    }
    bool bad = false;
    if (p < 0 || p >= a.max_seq) { bad = true; p = p < 0 ? 0 : a.max_seq - 1; }
    if (t < 0 || t >= a.vocab) { bad = true; t = 0; }
    sm.pos[b] = p;
    sm.tok[b] = t;
    if (bad && b < a.B) {
      atomicOr(&sm.bad, 1);
      atomicOr(&sm.badseq, 1u << b);
    }
  }
  for (int i = tid; i < 16 * CB * KST / 8; i += NT) reinterpret_cast<uint4*>(&sm.act[0][0])[i] = make_uint4(0, 0, 0, 0);
  __syncthreads();
  if (tid < 64) {
    // Key-range length ks: one range per workgroup of an XCD at most (32), and each range's keys
    // spread over the NG groups as evenly as the batch allows. Lane i tries ks0 + step i (ks0 =
    // 16 ceil(T / 512) for T keys; the last candidate is at least 16 ceil(T / (16 (32 - B))), which
    // always fits); the smallest that fits is rounded up to a multiple of NG (same keys per group,
    // fewer ranges to merge).
    int T = 0;
    for (int b = 0; b < a.B; ++b) T += sm.pos[b] + 1;
    const int ks0 = 16 * ((T + 16 * WPX - 1) / (16 * WPX));
    const int kfit = 16 * ((T + 16 * (WPX - a.B) - 1) / (16 * (WPX - a.B)));
    const int step = 16 * max(1, (kfit - ks0 + 16 * 63 - 1) / (16 * 63));
    const int cand = lane == 63 ? max(kfit, ks0 + step * 63) : ks0 + step * lane;
    int n = 0;
    for (int b = 0; b < a.B; ++b) n += (sm.pos[b] + cand) / cand;
    const int first = __builtin_ctzll(__ballot(n <= WPX));  // lane 63 always fits
    const int kmin = __shfl(cand, first);
    const int ks = NG * ((kmin + NG - 1) / NG);
    if (tid == 0) {
      int f = 0;
      for (int b = 0; b < a.B; ++b) {
        const int nb = (sm.pos[b] + ks) / ks;  // ceil((pos + 1) / ks)
        sm.f[b] = f;
        sm.ns[b] = nb;
        for (int s = 0; s < nb; ++s) sm.sb[f + s] = b;
        f += nb;
      }
      sm.nsplit = f;
      sm.ks = ks;
      if (sm.bad && sm.j == 0 && sm.x == 0) st_dev_u32(a.ws + W::BAD, 1u);
      if (a.drain && sm.j == 0 && sm.x == 0) st_dev_u32(a.ws + W::ABORT, 1u);
      if (sm.j >= WPX) st_dev_u32(a.ws + W::ABORT, 1u);  // more than 32 workgroups on one XCD: no role
    }
  }
  __syncthreads();
  const int x = __builtin_amdgcn_readfirstlane(sm.x), j = __builtin_amdgcn_readfirstlane(sm.j);
  if (j >= WPX) return;
  // the split plan, wave-uniform (read from LDS, so made scalar for the compiler: branches on it are
  // then uniform, and its count of loads in flight stays exact across them)
  Split sp;
  sp.on = __builtin_amdgcn_readfirstlane(j < sm.nsplit ? 1 : 0) != 0;
  sp.b = __builtin_amdgcn_readfirstlane(sp.on ? sm.sb[j] : 0);
  sp.s = __builtin_amdgcn_readfirstlane(sp.on ? j - sm.f[sp.b] : 0);
  sp.pos = __builtin_amdgcn_readfirstlane(sm.pos[sp.b]);
  sp.wr = __builtin_amdgcn_readfirstlane((sm.badseq >> sp.b) & 1u) == 0;
  sp.k0 = sp.s * __builtin_amdgcn_readfirstlane(sm.ks);
  sp.k1 = min(sp.k0 + __builtin_amdgcn_readfirstlane(sm.ks), sp.pos + 1);
  if (tid < 32) {
    const uint16_t* src = (tid < 16 ? a.cos_tab : a.sin_tab) + (size_t)sp.pos * D + 8 * (tid & 15);
    *reinterpret_cast<uint4*>(&sm.cs[tid >> 4][8 * (tid & 15)]) = *reinterpret_cast<const uint4*>(src);
  }
  __syncthreads();

  mark(a, x, j, MAXL, 0);
  if (comm) comm_role(sm, c, a, sp, x, j);
  else math_role(sm, a, sp, x, j);
  mark(a, x, j, MAXL, 1);

  // ---- tied LM head on all waves, greedy keys (lane li of column block cb: sequence 8 cb + li / 2)
  {
    const int li = lane & 15, g = lane >> 4;
    bool out[CB];
    float rs[CB];
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
      out[cb] = !(li & 1) && 8 * cb + (li >> 1) < a.B;
      rs[cb] = out[cb] ? norm_scale(sm, 8 * cb + (li >> 1)) : 0.f;
    }
    const int gw = j * NXCD + x, ntiles = a.vocab / 16;
    u64 best[CB];
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) best[cb] = 0;
    const __amdgpu_buffer_rsrc_t rlm = make_rsrc(a.lm_head);
    // a tile (16 rows x H) in NC chunks of CH K steps, two chunk buffers in flight
    constexpr int CH = LM_CH, NC = H / 32 / CH;
    static_assert(NC >= 2 && NC % 2 == 0, "LM head chunks");
    auto load_chunk = [&](uint4 (&w)[CH], int tile, int ch) {
      const int off = ((16 * tile + li) * H + 32 * CH * ch + 8 * g) * 2;
#pragma unroll
      for (int s = 0; s < CH; ++s) w[s] = ldnt(rlm, off + 64 * s);
    };
    auto mma_chunk = [&](const uint4 (&w)[CH], int ch, f32x4 (&acc)[CB]) {
#pragma unroll
      for (int s = 0; s < CH; ++s)
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
          const uint4 bo = *reinterpret_cast<const uint4*>(&sm.act[16 * cb + li][32 * CH * ch + 32 * s + 8 * g]);
          acc[cb] = mfma(w[s], bo, acc[cb]);
        }
    };
    int tile = gw + NWG * wave;
    uint4 wa[CH], wb[CH];
    if (tile < ntiles) {
      load_chunk(wa, tile, 0);
      load_chunk(wb, tile, 1);
    }
    while (tile < ntiles) {
      // the operand is read from LDS per tile (held in registers it would take 128 of them)
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      const int next = tile + NWG * NWAVE;
      f32x4 acc[CB];
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) acc[cb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ch = 0; ch < NC; ch += 2) {
        mma_chunk(wa, ch, acc);
        if (ch + 2 < NC) load_chunk(wa, tile, ch + 2);
        else if (next < ntiles) load_chunk(wa, next, 0);
        mma_chunk(wb, ch + 1, acc);
        if (ch + 3 < NC) load_chunk(wb, tile, ch + 3);
        else if (next < ntiles) load_chunk(wb, next, 1);
      }
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        float lg[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) lg[r] = (acc[cb][r] + dpp<0xB1>(acc[cb][r])) * rs[cb];  // hi + lo columns
        if (out[cb]) {
          const int v0 = 16 * tile + 4 * g;
          *reinterpret_cast<float4*>(a.logits + (size_t)(8 * cb + (li >> 1)) * a.vocab + v0) =
              make_float4(lg[0], lg[1], lg[2], lg[3]);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const u64 k = argmax_key(lg[r], v0 + r);
            best[cb] = k > best[cb] ? k : best[cb];
          }
        }
      }
      tile = next;
    }
    // reduce over the 4 row groups of the wave, then over the waves
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
#pragma unroll
      for (int sh = 16; sh < 64; sh <<= 1) {
        const u64 o = ((u64)(uint32_t)__shfl_xor((int)(best[cb] >> 32), sh) << 32) |
                      (uint32_t)__shfl_xor((int)best[cb], sh);
        best[cb] = o > best[cb] ? o : best[cb];
      }
      if (g == 0 && out[cb]) sm.wk[wave][8 * cb + (li >> 1)] = best[cb];
    }
    __syncthreads();
    if (tid < a.B) {
      u64 k = 0;
      for (int w = 0; w < NWAVE; ++w) k = sm.wk[w][tid] > k ? sm.wk[w][tid] : k;
      reinterpret_cast<u64*>(a.ws + W::KEYS)[gw * BM + tid] = k;
    }
    mark(a, x, j, MAXL, 2);
  }
}

// Zeroes the exchange words (and the ticket, abort and bad words) before a launch: `words`, a
// multiple of 4.
__global__ void __launch_bounds__(256) batch_zero_kernel(uint32_t* ws, size_t words) {
  uint4* p = reinterpret_cast<uint4*>(ws);
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < words / 4; i += (size_t)gridDim.x * blockDim.x)
    p[i] = make_uint4(0, 0, 0, 0);
}

// Greedy tokens from the workgroups' keys; NaN logits and token -1 for every sequence if the launch
// gave up or an input was out of range.
template <int BM>
__global__ void __launch_bounds__(256) batch_finish_kernel(const uint32_t* ws, int B, int vocab, float* logits,
                                                           int32_t* out_tokens) {
  using W = WL<BM>;
  const bool failed = ws[W::ABORT] != 0 || ws[W::BAD] != 0;
  if (failed) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < (size_t)B * vocab; i += (size_t)gridDim.x * blockDim.x)
      logits[i] = __uint_as_float(0x7fc00000u);
  }
  if (blockIdx.x != 0 || !out_tokens) return;
  const int lane = threadIdx.x & 63, b = threadIdx.x >> 6;  // 4 waves, sequences b, b + 4
  const u64* keys = reinterpret_cast<const u64*>(ws + W::KEYS);
  for (int s = b; s < B; s += 4) {
    u64 k = 0;
    for (int w = lane; w < NWG; w += 64) k = keys[w * BM + s] > k ? keys[w * BM + s] : k;
#pragma unroll
    for (int sh = 1; sh < 64; sh <<= 1) {
      const u64 o = ((u64)(uint32_t)__shfl_xor((int)(k >> 32), sh) << 32) | (uint32_t)__shfl_xor((int)k, sh);
      k = o > k ? o : k;
    }
    if (lane == 0) out_tokens[s] = failed ? -1 : (int32_t)(0xffffffffu - (uint32_t)k);
  }
}

// ---- host ----------------------------------------------------------------------------------------

constexpr int MAX_DEVICES = 64;
struct DevCheck {
  bool done = false;
  bool ok[2] = {false, false};  // one and two column blocks
};
static DevCheck g_check[MAX_DEVICES];
static std::mutex g_mu;
static std::atomic<int> g_engine{0};    // 0 automatic, 1 layer-by-layer engine, 2 this kernel
static std::atomic<bool> g_drain{false};
static std::atomic<uint64_t*> g_trace{nullptr};

// Can the current device run the kernel with cb column blocks: 256 CUs and one 768-thread workgroup
// per CU.
static bool device_ok(int cb) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) return false;
  std::lock_guard<std::mutex> lk(g_mu);
  DevCheck& d = g_check[dev];
  if (!d.done) {
    int cus = 0;
    const bool cus_ok = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && cus == NWG;
    const void* fns[2] = {(const void*)batch_kernel<1>, (const void*)batch_kernel<2>};
    for (int i = 0; i < 2; ++i) {
      int blocks = 0;
      d.ok[i] = cus_ok && hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, fns[i], NT, 0) == hipSuccess && blocks >= 1;
    }
    d.done = true;
  }
  return d.ok[cb - 1];
}

template <int CB>
static hipError_t launch(const BArgs& a, int32_t* out_tokens, hipStream_t stream) {
  using W = WL<8 * CB>;
  hipLaunchKernelGGL(batch_zero_kernel, dim3(128), dim3(256), 0, stream, a.ws, W::ZERO);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(batch_kernel<CB>, dim3(NWG), dim3(NT), 0, stream, a);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  hipLaunchKernelGGL(batch_finish_kernel<8 * CB>, dim3(64), dim3(256), 0, stream, (const uint32_t*)a.ws, a.B, a.vocab,
                     a.logits, out_tokens);
  return hipGetLastError();
}

}  // namespace mkb

bool mkb_applies(const mk_model_dims* dims, int batch, int max_seq_len) {
  using namespace mkb;
  const int e = g_engine.load();
  if (e == 1) return false;
  return dims->hidden == H && dims->intermediate == I && dims->num_layers >= 1 && dims->num_layers <= MAXL &&
         dims->num_layers < 255 && batch >= 1 && batch <= BMAX && max_seq_len >= 1 && device_ok(batch <= 8 ? 1 : 2);
}
size_t mkb_workspace_bytes() { return mkb::WS_BYTES; }
int mkb_engine() { return mkb::g_engine.load(); }
void mkb_set_drain(bool on) { mkb::g_drain.store(on); }

hipError_t mkb_decode_batch(const mk_model_dims* dims, int batch, const int32_t* tokens, const int32_t* positions,
                            const void* embed_weight, const void* lm_head_weight, const void* final_norm_weight,
                            const mk_layer_weights* layers, const void* cos_table, const void* sin_table,
                            void* k_cache, void* v_cache, int max_seq_len, float* logits, int32_t* out_tokens,
                            void* workspace, hipStream_t stream) {
  using namespace mkb;
  BArgs a{};
  a.tokens = tokens;
  a.positions = positions;
  a.embed = (const uint16_t*)embed_weight;
  a.lm_head = (const uint16_t*)lm_head_weight;
  a.final_norm = (const uint16_t*)final_norm_weight;
  a.cos_tab = (const uint16_t*)cos_table;
  a.sin_tab = (const uint16_t*)sin_table;
  a.k_cache = (uint16_t*)k_cache;
  a.v_cache = (uint16_t*)v_cache;
  a.logits = logits;
  a.ws = (uint32_t*)workspace;
  a.B = batch;
  a.L = dims->num_layers;
  a.vocab = dims->vocab;
  a.max_seq = max_seq_len;
  a.drain = g_drain.load() ? 1 : 0;
  a.trace = g_trace.load();
  for (int l = 0; l < a.L; ++l) a.lw[l] = layers[l];
  return batch <= 8 ? launch<1>(a, out_tokens, stream) : launch<2>(a, out_tokens, stream);
}

extern "C" hipError_t mk_set_batch_engine(int engine) {
  if (engine < 0 || engine > 2) return hipErrorInvalidValue;
  mkb::g_engine.store(engine);
  return hipSuccess;
}

extern "C" hipError_t mk_set_batch_trace(uint64_t* device_buffer, size_t bytes) {
  if (device_buffer != nullptr && bytes < mkb::TRACE_BYTES) return hipErrorInvalidValue;
  mkb::g_trace.store(device_buffer);
  return hipSuccess;
}

extern "C" size_t mk_batch_trace_bytes(void) { return mkb::TRACE_BYTES; }
