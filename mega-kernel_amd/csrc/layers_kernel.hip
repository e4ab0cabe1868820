// The layer-by-layer engine of the library on MI355X (gfx950): the batched prefill of a Qwen3-shaped
// model (all prompt tokens at once, layer by layer, writing the decode kernel's K/V cache layout
// [L][8][max_seq][128] -- or its paged layout -- directly) and the batched decode of up to 64
// sequences (second half of this file).
//
// The reference prefills with Transformers on the GPU and copies its cache into the kernel's
// layout (/root/reference/model.py:72-87); the decode kernel of this library could also prefill by
// one decode launch per prompt token. Here the prompt's tokens are the M rows of skinny-to-square
// GEMMs on the matrix cores (v_mfma_f32_16x16x32_bf16), with the elementwise work fused into the
// GEMM epilogues:
//   x = embed[tokens]                                  (fp32 residual rows, workspace)
//   per layer:  a = RMSNorm(x)                         (bnorm_kernel, as bf16 hi/lo pair)
//               q, k, v = a . [Wq; Wk; Wv]^T           (gemm, EPI_QKV: per-head RMSNorm + RoPE on q and k,
//                                                       k and v rounded to bf16 into the cache, q kept)
//               o = causal attention(q, cache)         (attn_kernel: flash-style, online softmax)
//               x += o . Wo^T                          (gemm, EPI_RESID)
//               a = RMSNorm(x)
//               m = silu(a . Wg^T) * (a . Wu^T)        (gemm, EPI_SILU: gate and up rows in one tile)
//               x += m . Wd^T                          (gemm, EPI_RESID)
//   logits of the last row = RMSNorm(x) . E^T, greedy token (lm_head_kernel, fused argmax)
// When the residual products' tile grid is small (below 192 tiles) they are split over K into
// partials that the next norm adds in a fixed order; on grids of at most 128 tiles QKV and gate/up
// are split over K too, into raw sums that qkv_post_kernel / silu_post_kernel finish. The attention
// takes one query block per workgroup, or key-range chunks of the blocks merged by
// attn_merge_kernel where the blocks' key chains are uneven against the grid. Prompts of at most
// small_m(H) tokens run the products on the skinny kernels of the batched decode instead (weights
// as the MFMA A operand, activations in its skinny fragment order).
//
// Numerics are the decode kernel's (the reference kernel's fp32 design, /root/reference/
// megakernel.cu): fp32 residual and accumulation, fp32 RMSNorm, exact softmax, new K/V rounded to
// bf16. The matrix cores take bf16 operands, so every fp32 activation operand is split into
// hi = bf16(x) and lo = bf16(x - hi) and multiplied twice (weights and cache rows are bf16
// already): a product then matches fp32 to ~2^-17 relative.
//
// MFMA operand layout (16x16x32 bf16; lane l, i = l % 16, g = l / 16): A[i][8g + j] and
// B[8g + j][i] for j = 0..7 (8 bf16 = 16 bytes per lane), accumulator C[4g + j][i] for j = 0..3.
// Both A (activation rows) and B (weight rows, C = A . W^T) are read as 16-byte chunks of rows.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mk_device.h"
#include "mk_batch.h"
#include "mk_layers.h"
#include "../../include/megakernel_amd.h"

namespace mkp {
using namespace mk;


// Where the prefill's K/V rows live: the decode layout [L][8][max_seq][128], or (with a block table)
// the paged layout [L][num_pages][8][page_size][128] of mk_decode_paged, position p in page
// bt[p >> shift]. An entry outside [0, num_pages) sets *bad (the call then reports NaN logits and
// token -1), reads page 0 and is never written.
struct KvMap {
  const int32_t* bt;
  int num_pages, shift, max_seq;
};
__device__ __forceinline__ int kv_page(const KvMap& m, int p, int32_t* bad) {
  const int e = m.bt[p >> m.shift];
  if (e < 0 || e >= m.num_pages) {
    if (bad) *bad = 1;
    return -1;
  }
  return e;
}
// element offset of row p of (layer, head) given its page (ignored without a table)
__device__ __forceinline__ size_t kv_row(const KvMap& m, int layer, int head, int p, int page) {
  if (!m.bt) return (((size_t)layer * HKV + head) * m.max_seq + p) * D;
  return (((((size_t)layer * m.num_pages + page) * HKV + head) << m.shift) + (p & ((1 << m.shift) - 1))) * D;
}


// ------------------------------------------------------------------------------------------------
// GEMM C[M][N] = A[M][K] . W[N][K]^T on the matrix cores, A given as a bf16 hi/lo pair in the
// fragment-major layout below, W bf16 row-major (nn.Linear layout, read in place). Tile 128 x 128
// per workgroup of 4 waves, wave w taking rows [32 w, 32 w + 32) and all 128 columns. K in steps of
// 64: the weight tile is staged through LDS (every wave reads all of it), the activation fragments
// go straight from memory into the registers of the one wave that uses them, so only a third of the
// operand bytes are written to LDS. The next step's loads are in flight during the current step's
// MFMAs. The epilogue takes the tile's fp32 sums.
// ------------------------------------------------------------------------------------------------
// KP: padded LDS row of the weight tile, 160 B. A row stride of 32 modulo 128 bytes is what makes the
// fragment reads (16 lanes on 16 rows, 4 lanes on consecutive 16-byte chunks of each) conflict-free
// on MI355X; 144 B (16 mod 128) costs a second LDS cycle per read (SQ_LDS_BANK_CONFLICT, measured
// with an LDS probe: 4 extra cycles per ds_read_b128).
constexpr int MT = 128, NT = 128, KT = 64, KP = KT + 16;
constexpr int CP = NT + 4;                              // padded fp32 row of the epilogue tile

// Fragment-major layout of a bf16 activation matrix with K columns (K a multiple of 32), the A
// operand of gemm_kernel: 16-row x 32-column blocks of 1 KB, block (m / 16, k / 32) at KB offset
// (m / 16) * (K / 32) + k / 32; inside a block, MFMA lane l = (m % 16) + 16 * ((k % 32) / 8) holds
// the 16 bytes of columns [8 ((k % 32) / 8), +8). A wave reads one operand fragment as 1 KB of
// consecutive bytes. Buffers in this layout hold a multiple of MT rows; rows past M are never
// written, and the sums they produce are never stored.
__device__ __forceinline__ size_t frag_off(int m, int k, int K) {
  return ((((size_t)(m >> 4) * (K >> 5) + (k >> 5)) * 64 + ((k >> 3) & 3) * 16 + (m & 15)) << 3) + (k & 7);
}
static size_t frag_rows(int M) { return (size_t)(M + MT - 1) / MT * MT; }

// Activation operand of the skinny products in fragment order ("skinny fragments", used by the
// batched decode): for column block cb (sequences 8 cb .. 8 cb + 7) and K block kb (32 inputs), one
// 1 KB fragment holding, at lane l, MFMA column li = l % 16 (sequence 8 cb + li / 2, bf16 hi part for
// even li, lo for odd) and inputs 32 kb + 8 (l / 16) .. + 8. A wave then loads a whole B operand as
// 1 KB of consecutive bytes. In row order (B rows of ldx elements, hi and lo in two arrays) each lane
// of such a load reads 16 bytes of a different row, and the vector cache takes one access per lane:
// at 64 sequences that was the skinny products' bound (rocprof at 64 sequences: ~64 L1 accesses per
// load instruction, TA address stalls). Rows past the batch are never written; their columns of the
// products are never read.
// Fragment order: with 2 or 4 column blocks (CB, skf_blocks) K-block major (the CB fragments of one
// K block adjacent), with 8 column-block major (the K blocks of one column block adjacent). Every
// workgroup of a product reads the same fragments at about the same time; measured on MI355X at
// context 256 (layer by layer, per step), 16 / 32 / 64 sequences: column-block major 1744 / 2412 /
// 2411 us, K-block major 1513 / 1994 / 2596, row order 1544 / 1979 / 2863.
__host__ __device__ inline int skf_blocks(int B) { return B <= 8 ? 1 : B <= 16 ? 2 : B <= 32 ? 4 : 8; }
__host__ __device__ inline size_t skf_frag(int cb, int kb, int CB, int K) {
  return CB == 8 ? (size_t)cb * (K >> 5) + kb : (size_t)kb * CB + cb;
}
__host__ __device__ inline size_t skf_off(int b, int k, int part, int B, int K) {
  const int cb = b >> 3, li = 2 * (b & 7) + part, kb = k >> 5, lg = (k & 31) >> 3;
  return ((skf_frag(cb, kb, skf_blocks(B), K) * 64 + lg * 16 + li) << 3) + (k & 7);
}
// Elements of the skinny fragments of B rows: whole column blocks of the kernel that reads them (1,
// 2, 4 or 8 blocks of 8 rows), hi and lo.
__host__ __device__ inline size_t skf_elems(int B, int K) { return (size_t)skf_blocks(B) * 8 * K * 2; }

// EPI_QKV_PART / EPI_SILU_PART: the QKV / gate-up products split over K on small grids, each K range's
// raw sums into part[blockIdx.z][M][N] (N = 4096 / 2 I, a tile's columns as in EPI_QKV / EPI_SILU);
// qkv_post_kernel / silu_post_kernel add the ranges in order and finish the epilogue.
enum Epi { EPI_QKV = 0, EPI_RESID = 1, EPI_SILU = 2, EPI_QKV_PART = 3, EPI_SILU_PART = 4 };

struct GemmArgs {
  const uint16_t* ah;  // fragment-major, K columns
  const uint16_t* al;
  int M, N, K;
  // weights: EPI_RESID: w0 [N][K]; EPI_QKV: w0 = Wq, w1 = Wk, w2 = Wv; EPI_SILU: w0 = Wg, w1 = Wu
  const uint16_t* w0;
  const uint16_t* w1;
  const uint16_t* w2;
  // EPI_RESID: x[M][ldx] += C; or, with `part`, the K range of blockIdx.z (K / gridDim.z wide) into
  // part[blockIdx.z][M][N], summed into x by the next norm
  float* x;
  int ldx;
  float* part;
  // EPI_SILU: m = silu(gate) * up into bh/bl, fragment-major with I = N / 2 columns
  uint16_t* bh;
  uint16_t* bl;
  // EPI_QKV
  const uint16_t* q_norm;
  const uint16_t* k_norm;
  const uint16_t* cos_tab;
  const uint16_t* sin_tab;
  uint16_t* qh;  // [M][16 * 128] normed, rotated queries, bf16 hi/lo
  uint16_t* ql;
  uint16_t* k_cache;
  uint16_t* v_cache;
  KvMap kv;
  int32_t* bad;
  int layer, position;
};

// first element of weight row r (0..127) of N-tile t
template <int EPI>
__device__ __forceinline__ const uint16_t* weight_row(const GemmArgs& g, int t, int r) {
  if constexpr (EPI == EPI_QKV || EPI == EPI_QKV_PART) {
    if (t < HQ) return g.w0 + (size_t)(t * D + r) * g.K;
    if (t < HQ + HKV) return g.w1 + (size_t)((t - HQ) * D + r) * g.K;
    return g.w2 + (size_t)((t - HQ - HKV) * D + r) * g.K;
  } else if constexpr (EPI == EPI_SILU || EPI == EPI_SILU_PART) {  // gate rows then up rows of intermediates [64 t, 64 t + 64)
    return r < NT / 2 ? g.w0 + (size_t)(t * (NT / 2) + r) * g.K : g.w1 + (size_t)(t * (NT / 2) + r - NT / 2) * g.K;
  } else {
    return g.w0 + (size_t)(t * NT + r) * g.K;
  }
}

struct GemmSmem {
  union {
    uint16_t w[NT][KP];
    float c[MT][CP];
  };
};

// PF: K steps of operands in flight, loaded ahead in registers. 1: the next step's loads are issued
// as a step's MFMAs start (two workgroups per CU hide each other's load latency). 4: grids of at
// most one workgroup per CU (short prompts), where a lone workgroup otherwise waits out most of each
// load round trip. 2: either. PF 1 and 2 are held to the register budget of two workgroups per CU
// (256 per lane).
template <int EPI, int PF = 1>
__global__ void __launch_bounds__(256, PF == 4 ? 1 : 2) gemm_kernel(const GemmArgs g) {
  __shared__ __attribute__((aligned(16))) GemmSmem sm;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int tn = blockIdx.x, tm = blockIdx.y;
  if (gridDim.x <= 16 && gridDim.y >= 8 && (gridDim.x * gridDim.y) % 8 == 0) {
    // Few column tiles and many row tiles (the residual products of long prompts): consecutive
    // workgroups go to the 8 XCDs in turn, so with the plain order the column tiles of one row tile
    // would sit on different XCDs and each XCD's L2 would fetch that row tile's activations again.
    // XCD b % 8 takes the b % 8-th eighth of the tiles instead, row tile by row tile: the column
    // tiles sharing activations share an L2. (With few row tiles the weights are the larger stream
    // and the plain order, one column tile per XCD, measured faster.)
    const int T = gridDim.x * gridDim.y, b = blockIdx.x + gridDim.x * blockIdx.y;
    const int t = (b & 7) * (T >> 3) + (b >> 3);
    tn = t % gridDim.x;
    tm = t / gridDim.x;
  }
  const int m0 = tm * MT;
  const int li = lane & 15, lg = lane >> 4;
  const int kch = g.K >> 5;  // 1 KB fragments per 16-row block

  // this wave's two 16-row blocks of A: fragment (bm, 32-column chunk kc) at uint4 (bm * kch + kc) * 64
  const size_t abase = (size_t)((m0 >> 4) + 2 * wave) * kch * 64 + lane;
  const uint4* pah = reinterpret_cast<const uint4*>(g.ah) + abase;
  const uint4* pal = reinterpret_cast<const uint4*>(g.al) + abase;
  // one K step of A: [32-column half s][row block bm][hi, lo]
  typedef uint4 AStep[2][2][2];
  auto load_a = [&](int k0, AStep& d) {
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int bm = 0; bm < 2; ++bm) {
        const int f = (bm * kch + (k0 >> 5) + s) * 64;
        d[s][bm][0] = pah[f];
        d[s][bm][1] = pal[f];
      }
  };
  // weights: global -> registers -> LDS, 4 chunks of 16 bytes per thread (row c / 8, chunk c % 8)
  typedef uint4 WStep[4];
  auto load_w = [&](int k0, WStep& rw) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + 256 * i, row = c >> 3, ch = c & 7;
      rw[i] = ld_stream(reinterpret_cast<const uint4*>(weight_row<EPI>(g, tn, row) + k0 + 8 * ch));
    }
  };
  auto store_w = [&](const WStep& rw) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + 256 * i, row = c >> 3, ch = c & 7;
      *reinterpret_cast<uint4*>(&sm.w[row][8 * ch]) = rw[i];
    }
  };

  f32x4 acc[2][8];
#pragma unroll
  for (int bm = 0; bm < 2; ++bm)
#pragma unroll
    for (int bn = 0; bn < 8; ++bn) acc[bm][bn] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int kspan = g.K / gridDim.z, kb = blockIdx.z * kspan, ke = kb + kspan;  // a multiple of KT
  // a wave whose 32 rows all lie past M (a short last row tile: the batched decode's LM head takes 64
  // or fewer rows) still loads its fragments and stages its part of the weight tile -- the same loads
  // in every wave keep the waits exact -- but skips the MFMAs
  const bool act = m0 + 32 * wave < g.M;
  auto step = [&](const AStep& ac) __attribute__((always_inline)) {
#pragma unroll
    for (int s = 0; s < KT / 32; ++s) {
      uint4 fw[8];
#pragma unroll
      for (int bn = 0; bn < 8; ++bn) fw[bn] = *reinterpret_cast<const uint4*>(&sm.w[bn * 16 + li][32 * s + 8 * lg]);
#pragma unroll
      for (int bm = 0; bm < 2; ++bm)
#pragma unroll
        for (int bn = 0; bn < 8; ++bn) {
          acc[bm][bn] = mfma(ac[s][bm][0], fw[bn], acc[bm][bn]);
          acc[bm][bn] = mfma(ac[s][bm][1], fw[bn], acc[bm][bn]);
        }
    }
  };
  if constexpr (PF == 1) {
    AStep an, ac;
    WStep rw;
    load_w(kb, rw);
    load_a(kb, an);
    for (int k0 = kb; k0 < ke; k0 += KT) {
      __syncthreads();  // every wave is done with the previous step's weight tile
      store_w(rw);
      __syncthreads();
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int bm = 0; bm < 2; ++bm) {
          ac[s][bm][0] = an[s][bm][0];
          ac[s][bm][1] = an[s][bm][1];
        }
      if (k0 + KT < ke) {
        load_w(k0 + KT, rw);
        load_a(k0 + KT, an);
      }
      if (act) step(ac);
    }
  } else {
    // The K range is a multiple of PF steps (host). Step i + PF's loads go out as step i starts, the
    // last PF steps issue none. The scheduling barriers keep each step's loads in issue order: the
    // waits before a step then cover that step's loads alone (left free, the scheduler may issue a
    // later step's loads first, and the wait for the earlier ones then drains the whole pipeline).
    AStep aq[PF];
    WStep wq[PF];
#pragma unroll
    for (int p = 0; p < PF; ++p) {
      load_w(kb + p * KT, wq[p]);
      load_a(kb + p * KT, aq[p]);
      __builtin_amdgcn_sched_barrier(0);
    }
    for (int k0 = kb; k0 < ke - PF * KT; k0 += PF * KT) {
#pragma unroll
      for (int p = 0; p < PF; ++p) {
        __syncthreads();  // every wave is done with the previous step's weight tile
        store_w(wq[p]);
        __syncthreads();
        // step i + PF's weights into the registers just stored, its A fragments into the ones the
        // MFMAs just read (no copies: a register copy of a pending load would wait for it)
        const int kn = k0 + (p + PF) * KT;
        load_w(kn, wq[p]);
        if (act) step(aq[p]);
        load_a(kn, aq[p]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
#pragma unroll
    for (int p = 0; p < PF; ++p) {
      __syncthreads();
      store_w(wq[p]);
      __syncthreads();
      if (act) step(aq[p]);
    }
  }

  if constexpr (EPI == EPI_RESID || EPI == EPI_QKV_PART || EPI == EPI_SILU_PART) {
    // x += C (or C into this K range's partial), each element owned by one lane
    auto each = [&](auto&& f) {
#pragma unroll
      for (int bm = 0; bm < 2; ++bm)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int m = m0 + wave * 32 + bm * 16 + 4 * lg + j;
          if (m < g.M) {
#pragma unroll
            for (int bn = 0; bn < 8; ++bn) f(m, tn * NT + bn * 16 + li, acc[bm][bn][j]);
          }
        }
    };
    if (g.part) {
      float* pz = g.part + (size_t)blockIdx.z * g.M * g.N;
      each([&](int m, int n, float v) { pz[(size_t)m * g.N + n] = v; });
    } else {
      each([&](int m, int n, float v) { g.x[(size_t)m * g.ldx + n] += v; });
    }
    return;
  }

  // QKV and SILU need whole rows of the tile: through LDS
  __syncthreads();
#pragma unroll
  for (int bm = 0; bm < 2; ++bm)
#pragma unroll
    for (int bn = 0; bn < 8; ++bn)
#pragma unroll
      for (int j = 0; j < 4; ++j) sm.c[wave * 32 + bm * 16 + 4 * lg + j][bn * 16 + li] = acc[bm][bn][j];
  __syncthreads();
  // The stores are laid out so that a wave's store instruction writes whole 256-byte rows or whole
  // 1 KB fragments: per-thread row segments (two threads per row, each lane of a store on another
  // row) made the stores a third of the QKV GEMM's time at 3,584 tokens.
  auto ld8 = [&](int row, int c, float (&v)[8]) {
    const float4 x0 = *reinterpret_cast<const float4*>(&sm.c[row][c]);
    const float4 x1 = *reinterpret_cast<const float4*>(&sm.c[row][c + 4]);
    v[0] = x0.x; v[1] = x0.y; v[2] = x0.z; v[3] = x0.w; v[4] = x1.x; v[5] = x1.y; v[6] = x1.z; v[7] = x1.w;
  };

  if constexpr (EPI == EPI_SILU) {
    // columns 0..63 gate, 64..127 up of intermediates [64 tn, 64 tn + 64): 8 row blocks x 2 K blocks
    // of 32 = 16 fragments of the down product's A operand; wave w writes fragments 4 w .. 4 w + 3,
    // lane l its row l % 16 and intermediates 8 (l / 16) .. +7 (frag_off's order)
#pragma unroll
    for (int f = 0; f < 4; ++f) {
      const int fr = 4 * wave + f, rb = fr >> 1, kb = fr & 1;
      const int r = 16 * rb + li, m = m0 + r, c = 32 * kb + 8 * lg;
      if (m < g.M) {
        float gt[8], up[8], mv[8];
        ld8(r, c, gt);
        ld8(r, NT / 2 + c, up);
#pragma unroll
        for (int q = 0; q < 8; ++q) mv[q] = gt[q] / (1.f + expf(-gt[q])) * up[q];  // silu(gate) * up (/root/reference/megakernel.cu:659-665)
        uint4 hi, lo;
        split8(mv, hi, lo);
        const size_t o = frag_off(m, tn * (NT / 2) + c, g.N / 2);
        *reinterpret_cast<uint4*>(g.bh + o) = hi;
        *reinterpret_cast<uint4*>(g.bl + o) = lo;
      }
    }
    return;
  }

  if constexpr (EPI == EPI_QKV) {
    // tile tn is one head: q head tn (< 16), k head tn - 16 (< 24) or v head tn - 24. 16 lanes per
    // row (lane t: dims 8t .. 8t + 7), 4 rows per wave and pass, 8 passes
    const int tt = lane & 15, rq = lane >> 4;  // tt: the lane's 8 dims; rq: its row of the pass
    float wn[8];
    if (tn < HQ + HKV) unpack8(*reinterpret_cast<const uint4*>((tn < HQ ? g.q_norm : g.k_norm) + 8 * tt), wn);
#pragma unroll 2
    for (int pass = 0; pass < 8; ++pass) {
      const int r = 32 * wave + 4 * pass + rq, m = m0 + r;
      if (m >= g.M) continue;
      const int pos = g.position + m;
      const int page = tn >= HQ && g.kv.bt ? kv_page(g.kv, pos, g.bad) : 0;
      float v[8];
      ld8(r, 8 * tt, v);
      if (tn >= HQ + HKV) {  // v: rounded to bf16 into the cache as is
        if (page >= 0) {
          uint32_t p[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) p[q] = pack_bf16x2(v[2 * q], v[2 * q + 1]);
          *reinterpret_cast<uint4*>(g.v_cache + kv_row(g.kv, g.layer, tn - HQ - HKV, pos, page) + 8 * tt) =
              make_uint4(p[0], p[1], p[2], p[3]);
        }
        continue;
      }
      // per-head RMSNorm over the 128 dims (/root/reference/megakernel.cu:490-630), then rotate-half
      // RoPE with the table entry of dim d mod 64 (/root/reference/megakernel.cu:548-555)
      float cs[8], sn[8];
      unpack8(*reinterpret_cast<const uint4*>(g.cos_tab + (size_t)pos * D + 8 * (tt & 7)), cs);
      unpack8(*reinterpret_cast<const uint4*>(g.sin_tab + (size_t)pos * D + 8 * (tt & 7)), sn);
      head_norm_rope(v, wn, cs, sn, tt);
      if (tn < HQ) {
        uint4 hi, lo;
        split8(v, hi, lo);
        const size_t off = (size_t)m * (HQ * D) + tn * D + 8 * tt;
        *reinterpret_cast<uint4*>(g.qh + off) = hi;
        *reinterpret_cast<uint4*>(g.ql + off) = lo;
      } else if (page >= 0) {
        uint32_t p[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) p[q] = pack_bf16x2(v[2 * q], v[2 * q + 1]);
        *reinterpret_cast<uint4*>(g.k_cache + kv_row(g.kv, g.layer, tn - HQ, pos, page) + 8 * tt) =
            make_uint4(p[0], p[1], p[2], p[3]);
      }
    }
  }
}

// ------------------------------------------------------------------------------------------------
// Causal attention of the prompt rows (/root/reference/megakernel.cu:228-370 for one query; here
// flash-style over blocks of 64 keys). Query row m sits at position `position + m` and attends keys
// [0, position + m] of the cache, which already holds this layer's new rows (written by the QKV
// epilogue).
//   Work split: a workgroup (8 waves) takes one K/V head and one 64-query block, the blocks with
//   the most keys dispatched first (workgroups 0-7 take the last block of each head), so the CUs
//   that finish short blocks pick up the rest. (Pairs of blocks i and nqb - 1 - i per workgroup balanced the
//   work too, but left 32 of the 256 CUs idle at 3,584 tokens: 224 workgroups.) Where the blocks'
//   key chains are uneven against the grid (attn_plan), a workgroup takes one key-range chunk of a
//   block instead and attn_merge_kernel combines the chunks. Waves 0-3 take
//   query head 2 kvh, waves 4-7 head 2 kvh + 1, 16 queries each: the two heads of a GQA pair share
//   each K/V block staged in LDS.
//   Pipeline: the next K/V block is loaded into registers while the current one is multiplied,
//   then written into the other half of a double-buffered LDS tile; one barrier per block.
//   S^T = K . Q^T on the matrix cores (keys as rows): lane l holds the scores of query i = l % 16
//         against keys 16 mb + 4 g + j -- so each query's row statistics (max, sum) are a
//         reduction over registers and the 4 lanes i, i+16, i+32, i+48;
//   O  += P . V: the A operand (8 keys of query i per lane) is exactly what a lane holds of two
//         consecutive S^T blocks, with key slot 8g + jj meaning key 4g + jj (jj < 4) or
//         16 + 4g + jj - 4; V is staged transposed in LDS ([dim][key]) so that the B operand
//         (those 8 keys at one dim) is two 8-byte reads. The transpose is written as 32-bit words
//         (two consecutive keys of one dim), bank-conflict free.
// Output rows (normalised) as the bf16 hi/lo pair the O-projection GEMM takes, [M][16 * 128],
// staged through LDS so that every global store is 16 bytes.
// ------------------------------------------------------------------------------------------------
constexpr int QB = 64, KB = 64;
constexpr int KSP = D + 16;  // padded K row in LDS (288 B: 32 modulo 128, conflict-free fragment reads)
constexpr int VSP = KB + 4;  // padded V^T row (136 B: the paired 8-byte fragment reads, one ds_read2_b64, conflict-free; 144 B costs 8 cycles each)
constexpr int OSP = D + 8;   // padded output staging row (272 B: its 2-byte writes four rows apart on different banks)

struct AttnArgs {
  const uint16_t* qh;
  const uint16_t* ql;
  const uint16_t* k_cache;
  const uint16_t* v_cache;
  uint16_t* oh;  // output: frag 1 the GEMM's fragment order (frag_off, 16 * 128 columns; hi in oh, lo
  uint16_t* ol;  // in ol), 2 the skinny products' fragments (skf_off, hi and lo both in oh)
  int frag;
  int M, layer, position;
  KvMap kv;
  int32_t* bad;
  // Key-range chunks (attn_plan): chunk > 0 cuts every query block into chunks of `chunk` key blocks,
  // one workgroup each; a block with more than one chunk has its chunks' unnormalised partials
  // written to `part` (slot = workgroup index: [slot][2 heads][qr rows][APS]) and merged by
  // attn_merge_kernel. chunk == 0: one workgroup per query block, no partials.
  float* part;
  int chunk, qr;
};
constexpr int APS = D + 4;  // floats per partial row: acc[128], m, l, pad (16-byte aligned rows)

// Where the 8 output values of row m from column k (k % 8 == 0), part 0 (hi) or 1 (lo), go.
__device__ __forceinline__ uint16_t* attn_out(const AttnArgs& a, int m, int k, int part) {
  if (a.frag == 2) return a.oh + skf_off(m, k, part, a.M, HQ * D);
  return (part ? a.ol : a.oh) + frag_off(m, k, HQ * D);
}

// Key blocks that query block qb attends to: keys [0, position + min(M, (qb + 1) QB)).
__host__ __device__ inline int attn_nkb(int qb, int M, int position) {
  return (position + (M < (qb + 1) * QB ? M : (qb + 1) * QB) - 1) / KB + 1;
}
// Query blocks with more than c * T key blocks, i.e. those with a chunk c: the blocks qb >= the
// first such one (attn_nkb grows with qb). Round c of the grid lists them from qb = nqb - 1 down.
__host__ __device__ inline int attn_round(int c, int T, int M, int position, int nqb) {
  const int need = c * T * KB - position + 1;  // qb qualifies iff min(M, (qb + 1) QB) >= need
  if (need <= 0) return nqb;
  if (need > M) return 0;
  return nqb - ((need + QB - 1) / QB - 1);
}
constexpr int ATT_MAX_PAGES = 2048;  // block-table entries staged in LDS (as mk_decode_paged)

struct AttnSmem {
  union {
    struct {
      uint16_t ks[2][KB][KSP];
      uint16_t vt[2][D][VSP];
    } kv;
    uint16_t o[8][2][16][OSP];  // per wave: hi, lo of its 16 output rows
  };
};
static_assert(sizeof(AttnSmem) >= 8 * 16 * (D + 4) * 4, "a chunk's partial rows staged per wave");

__global__ void __launch_bounds__(512) attn_kernel(const AttnArgs a) {
  __shared__ __attribute__((aligned(16))) AttnSmem sm;
  __shared__ int32_t pages[ATT_MAX_PAGES];  // a paged cache's table entries (-1: out of range)
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li = lane & 15, lg = lane >> 4;
  // workgroup b: K/V head b % 8, query block nqb - 1 - b / 8 (the longest blocks of all heads first);
  // with chunks, round c of the grid (the rounds in order) lists chunk c of every query block that
  // has one, longest blocks first, so the rounds hold full chunks before the shorter last ones
  const int kvh = blockIdx.x % HKV, h = 2 * kvh + (w >> 2), wq = 16 * (w & 3);
  const int nqb = (a.M + QB - 1) / QB;
  int r = (int)blockIdx.x / HKV, c = 0;
  if (a.chunk > 0) {
    for (;; ++c) {  // bounded: the round sizes fall to 0, and the grid is their sum
      const int n = attn_round(c, a.chunk, a.M, a.position, nqb);
      if (n == 0) return;
      if (r < n) break;
      r -= n;
    }
  }
  if (a.kv.bt) {
    const int n = ((a.position + a.M - 1) >> a.kv.shift) + 1;  // entries of keys [0, position + M)
    for (int i = tid; i < n; i += 512) {
      const int e = a.kv.bt[i];
      pages[i] = (e < 0 || e >= a.kv.num_pages) ? -1 : e;
      if (pages[i] < 0) *a.bad = 1;
    }
    __syncthreads();
  }
  // element offset of key kp's row of this K/V head (page 0 for an out-of-range entry)
  auto key_row = [&](int kp) {
    return kv_row(a.kv, a.layer, kvh, kp, a.kv.bt ? max(pages[kp >> a.kv.shift], 0) : 0);
  };
  // staging roles: K chunk c = tid + 512 r (key c / 16, dims 8 (c % 16)); V: keys 2 vp, 2 vp + 1 at
  // dims 8 vc .. +7 (lanes of a wave span 32 key pairs and two chunks: conflict-free 32-bit writes)
  const int vp = lane & 31, vc = 2 * w + (lane >> 5);

  {
    const int qb = nqb - 1 - r;
    const int q0 = qb * QB;
    const int qrow = q0 + wq + li;                       // this lane's query (score layout)
    const int qpos = a.position + qrow;
    const int wlast = a.position + q0 + wq + 15;         // last position any query of this wave has
    const int last = a.position + min(a.M, q0 + QB) - 1;  // last key any query of the block sees
    const int nkb = last / KB + 1;
    // this workgroup's key blocks [kb0, kb1): all of them, or chunk c
    const int kb0 = a.chunk > 0 ? c * a.chunk : 0;
    const int kb1 = a.chunk > 0 ? min(kb0 + a.chunk, nkb) : nkb;
    const bool partial = a.chunk > 0 && nkb > a.chunk;

    // this lane's query fragments (B operand of S^T = K . Q^T): dims 32 s + 8 g .. +7, hi and lo
    uint4 fq[2][4];
    {
      const int qr = min(qrow, a.M - 1);
      const size_t o = (size_t)qr * (HQ * D) + h * D + 8 * lg;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        fq[0][s] = *reinterpret_cast<const uint4*>(a.qh + o + 32 * s);
        fq[1][s] = *reinterpret_cast<const uint4*>(a.ql + o + 32 * s);
      }
    }
    f32x4 acc[8];
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) acc[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
    // running max (of the raw scores) and sum of query qrow, replicated on its 4 lanes; a weight is
    // exp(ATT_SCALE (s - m)) = exp2(s C - m C)
    float mrun = -INFINITY, lrun = 0.f;
    constexpr float C = ATT_SCALE * 1.4426950408889634f;

    // K chunks and V rows of a block, loaded into registers ahead of use. Keys past `last` load key
    // `last` again (finite data; the causal mask gives them probability 0): every lane issues the
    // same loads, so the compiler's count of loads in flight stays exact and each wait below covers
    // only the block it stores.
    struct Blk {
      uint4 k0, k1, v0, v1;
    };
    // Contiguous cache: the (layer, head) rows as a uniform base plus a 32-bit byte offset (one
    // multiply-add per load). Paged: the row through the staged table.
    const size_t hbase = ((size_t)a.layer * HKV + kvh) * a.kv.max_seq * D;
    auto ld = [&](const uint16_t* base, int kp, int e) __attribute__((always_inline)) {
      if (!a.kv.bt)
        return ld_global16(reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(base + hbase) +
                                                          2u * (uint32_t)(kp * D + e)));
      return ld_global16(reinterpret_cast<const uint4*>(base + key_row(kp) + e));  // a value, not a copy
    };
    auto load_block = [&](Blk& b, int kb) __attribute__((always_inline)) {
      const int kp0 = kb * KB;
      b.k0 = ld(a.k_cache, min(kp0 + (tid >> 4), last), 8 * (tid & 15));
      b.k1 = ld(a.k_cache, min(kp0 + 32 + (tid >> 4), last), 8 * (tid & 15));
      b.v0 = ld(a.v_cache, min(kp0 + 2 * vp, last), 8 * vc);
      b.v1 = ld(a.v_cache, min(kp0 + 2 * vp + 1, last), 8 * vc);
    };
    auto store_block = [&](const Blk& b, int buf) __attribute__((always_inline)) {
      uint32_t* k0 = reinterpret_cast<uint32_t*>(&sm.kv.ks[buf][tid >> 4][8 * (tid & 15)]);
      uint32_t* k1 = reinterpret_cast<uint32_t*>(&sm.kv.ks[buf][32 + (tid >> 4)][8 * (tid & 15)]);
      *reinterpret_cast<uint4*>(k0) = make_uint4(b.k0.x, b.k0.y, b.k0.z, b.k0.w);
      *reinterpret_cast<uint4*>(k1) = make_uint4(b.k1.x, b.k1.y, b.k1.z, b.k1.w);
      const uint32_t x0[4] = {b.v0.x, b.v0.y, b.v0.z, b.v0.w};
      const uint32_t x1[4] = {b.v1.x, b.v1.y, b.v1.z, b.v1.w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        uint32_t* lo = reinterpret_cast<uint32_t*>(&sm.kv.vt[buf][8 * vc + 2 * q][2 * vp]);
        uint32_t* hi = reinterpret_cast<uint32_t*>(&sm.kv.vt[buf][8 * vc + 2 * q + 1][2 * vp]);
        *lo = (x0[q] & 0xFFFFu) | (x1[q] << 16);
        *hi = (x0[q] >> 16) | (x1[q] & 0xFFFF0000u);
      }
    };
    // one block of 64 keys from LDS buffer `buf` into the running softmax and output rows
    auto consume = [&](int kb, int buf) __attribute__((always_inline)) {
      const int kp0 = kb * KB;
      if (kp0 > wlast) return;  // a block entirely after this wave's queries adds nothing
      // scores S^T: 4 blocks of 16 keys x this wave's 16 queries. The four key blocks' products are
      // interleaved (a dependent MFMA waits ~45 cycles for its accumulator, an independent one
      // issues every ~17); each block's sum keeps the order dims 0..127, hi before lo.
      f32x4 st[4];
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) st[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        uint4 fk[4];
#pragma unroll
        for (int mb = 0; mb < 4; ++mb)
          fk[mb] = *reinterpret_cast<const uint4*>(&sm.kv.ks[buf][16 * mb + li][32 * s + 8 * lg]);
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) st[mb] = mfma(fk[mb], fq[0][s], st[mb]);
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) st[mb] = mfma(fk[mb], fq[1][s], st[mb]);
      }
      // causal mask (only on blocks that reach past the wave's first query); block maximum of this
      // lane's query over its 4 lanes (gfx950 lane swaps, no LDS round trip), on the raw scores
      if (kp0 + KB - 1 > a.position + q0 + wq) {
#pragma unroll
        for (int mb = 0; mb < 4; ++mb)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (kp0 + 16 * mb + 4 * lg + j > qpos) st[mb][j] = -INFINITY;
      }
      float bmax = -INFINITY;
#pragma unroll
      for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int j = 0; j < 4; ++j) bmax = fmaxf(bmax, st[mb][j]);
      bmax = xmax32(xmax16(bmax));
      // mnew is finite once the query has seen a key: from the first block on (key 0) without
      // chunks; a chunk that starts past some of its block's queries leaves those at -inf, and
      // then mc = 0 keeps their weights exp2(-inf) = 0 instead of NaN
      const float mnew = fmaxf(mrun, bmax);
      const float mc = mnew == -INFINITY ? 0.f : mnew * C;
      const float alpha = __builtin_amdgcn_exp2f(mrun * C - mc);  // exactly 1 when the max holds
      float psum = 0.f;
#pragma unroll
      for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float p = __builtin_amdgcn_exp2f(fmaf(st[mb][j], C, -mc));
          st[mb][j] = p;
          psum += p;
        }
      psum = xsum32(xsum16(psum));
      lrun = lrun * alpha + psum;
      mrun = mnew;
      // rescale the output rows (skipped when no query of the wave has a new maximum): row 4g + j
      // of the accumulator is query 4g + j, whose alpha sits in lane 4g + j (and its copies)
      if (__builtin_amdgcn_ballot_w64(alpha != 1.f) != 0) {
        float ar[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) ar[j] = __shfl(alpha, 4 * lg + j);
#pragma unroll
        for (int nb = 0; nb < 8; ++nb)
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[nb][j] *= ar[j];
      }
      // O += P . V over two 32-key steps
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        float pw[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) { pw[j] = st[2 * t][j]; pw[4 + j] = st[2 * t + 1][j]; }
        uint4 ph, pl;
        split8(pw, ph, pl);
        uint4 fv[8];
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) {
          const uint16_t* vr = &sm.kv.vt[buf][16 * nb + li][32 * t + 4 * lg];
          const uint2 v0 = *reinterpret_cast<const uint2*>(vr);       // keys 32t + 4g .. +3
          const uint2 v1 = *reinterpret_cast<const uint2*>(vr + 16);  // keys 32t + 16 + 4g .. +3
          fv[nb] = make_uint4(v0.x, v0.y, v1.x, v1.y);
        }
        // hi for every dim block, then lo: eight independent accumulators between dependent MFMAs
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) acc[nb] = mfma(ph, fv[nb], acc[nb]);
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) acc[nb] = mfma(pl, fv[nb], acc[nb]);
      }
    };

    // Earlier stores (a paged table's error flag) complete first: with
    // loads alone in flight the compiler's waits below cover single loads (a store in flight with them
    // makes every wait a full one, loads and stores completing out of order relative to each other).
    wait_vmem();
    Blk A;
    load_block(A, kb0);
    store_block(A, 0);
    __syncthreads();
    // the next block in flight while the current one is consumed (a second block in flight, or no
    // streaming at all, times the same: the loop is bound by its MFMA, VALU and LDS work)
    for (int kb = kb0; kb < kb1; ++kb) {
      const int buf = (kb - kb0) & 1;
      if (kb + 1 < kb1) load_block(A, kb + 1);
      consume(kb, buf);
      if (kb + 1 < kb1) store_block(A, buf ^ 1);
      __syncthreads();  // block kb consumed by every wave; block kb + 1 staged
    }
    if (partial) {
      // this chunk's unnormalised rows and their (m ATT_SCALE, l) into the workgroup's slot, staged
      // per wave in LDS as the slot's rows (APS floats; the tiles are free after the loop's last
      // barrier) and stored as 16-byte chunks; rows past qr (queries past a short prompt) are not kept
      float* stg = reinterpret_cast<float*>(&sm) + w * 16 * APS;
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) stg[(4 * lg + j) * APS + 16 * nb + li] = acc[nb][j];
      if (lg == 0) *reinterpret_cast<float2*>(stg + li * APS + D) = make_float2(mrun * ATT_SCALE, lrun);
      float* P = a.part + (((size_t)blockIdx.x * 2 + (w >> 2)) * a.qr + wq) * APS;
      const int nch = (min(16, a.qr - wq) * APS) / 4;  // 16-byte chunks of this wave's kept rows
      for (int k = lane; k < nch; k += 64)
        reinterpret_cast<float4*>(P)[k] = reinterpret_cast<const float4*>(stg)[k];
      return;
    }
    // normalise by each row's sum (query 4g + j's, from lane 4g + j), stage this wave's 16 rows as
    // hi/lo in LDS (the tiles are free after the loop's last barrier), then store 16-byte chunks
    float linv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) linv[j] = 1.f / __shfl(lrun, 4 * lg + j);
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int nb = 0; nb < 8; ++nb) {
        const float o = acc[nb][j] * linv[j];
        const uint16_t hi = f32_to_bf16(o);
        sm.o[w][0][4 * lg + j][16 * nb + li] = hi;
        sm.o[w][1][4 * lg + j][16 * nb + li] = f32_to_bf16(o - bf16_to_f32(hi));
      }
#pragma unroll
    for (int r = 0; r < 8; ++r) {  // 2 x 16 rows x 16 chunks = 512 chunks, 8 per lane
      const int c = lane + 64 * r, part = c >> 8, row = (c >> 4) & 15, ch = c & 15;
      const int m = q0 + wq + row;
      const uint4 v = *reinterpret_cast<const uint4*>(&sm.o[w][part][row][8 * ch]);
      if (m < a.M) *reinterpret_cast<uint4*>(attn_out(a, m, h * D + 8 * ch, part)) = v;
    }
  }
}

// The chunks of the query blocks that attn_kernel split (more than `chunk` key blocks): eight
// workgroups per query block nqb - 1 - r and K/V head kvh, 16 of its 128 rows each, merge them max
// first and in chunk order (so the result does not depend on which chunk finished first), and
// write the normalised rows as the attention's own epilogue does. Chunk c of the block is attention
// workgroup (rounds before c + r) * 8 + kvh.
__global__ void __launch_bounds__(256) attn_merge_kernel(const AttnArgs a) {
  constexpr int MAXC = 32;  // chunks per query block (attn_plan: at most 32)
  __shared__ int slot[MAXC];
  __shared__ float wgt[16][MAXC + 1];  // exp(m_c - max) per row of this workgroup and chunk
  // workgroup b: rows 16 (b % 8) .. +15 of the 128 (2 heads x 64 queries) of query block nqb - 1 - r
  // of K/V head kvh, b / 8 = r * 8 + kvh; thread t: row t / 16, dims 8 (t % 16) .. +7
  const int rg = blockIdx.x & 7, kvh = (blockIdx.x >> 3) % HKV, r = (blockIdx.x >> 3) / HKV;
  const int nqb = (a.M + QB - 1) / QB, qb = nqb - 1 - r, q0 = qb * QB;
  const int nc = min((attn_nkb(qb, a.M, a.position) + a.chunk - 1) / a.chunk, MAXC);
  const int t = threadIdx.x, tr = t >> 4, ch = t & 15;
  const int row = 16 * rg + tr, hh = row >> 6, rq = row & 63, m = q0 + rq;
  if (t == 0) {
    int off = 0;
    for (int c = 0; c < nc; ++c) {
      slot[c] = (off + r) * HKV + kvh;
      off += attn_round(c, a.chunk, a.M, a.position, nqb);
    }
  }
  __syncthreads();
  auto prow = [&](int c, int rr) {  // row rr (of the 128) of chunk c's partial
    return a.part + (((size_t)slot[c] * 2 + (rr >> 6)) * a.qr + (rr & 63)) * APS;
  };
  // every (row, chunk) m of the workgroup's 16 rows, loaded together; then each row's weights
  for (int k = t; k < 16 * nc; k += 256) {
    const int rr = 16 * rg + k / nc, c = k % nc;
    wgt[k / nc][c] = (q0 + (rr & 63) < a.M) ? prow(c, rr)[D] : 0.f;
  }
  __syncthreads();
  if (t < 16) {
    float mx = -INFINITY;
    for (int c = 0; c < nc; ++c) mx = fmaxf(mx, wgt[t][c]);  // finite: chunk 0 holds key 0
    for (int c = 0; c < nc; ++c) wgt[t][c] = __expf(wgt[t][c] - mx);  // 0 for a chunk without keys (m = -inf)
  }
  __syncthreads();
  if (m >= a.M) return;
  float L = 0.f, o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
  for (int c = 0; c < nc; ++c) {
    const float* p = prow(c, row);
    const float f = wgt[tr][c];
    const float4 u = *reinterpret_cast<const float4*>(p + 8 * ch), v = *reinterpret_cast<const float4*>(p + 8 * ch + 4);
    L = fmaf(p[D + 1], f, L);
    o[0] = fmaf(u.x, f, o[0]); o[1] = fmaf(u.y, f, o[1]); o[2] = fmaf(u.z, f, o[2]); o[3] = fmaf(u.w, f, o[3]);
    o[4] = fmaf(v.x, f, o[4]); o[5] = fmaf(v.y, f, o[5]); o[6] = fmaf(v.z, f, o[6]); o[7] = fmaf(v.w, f, o[7]);
  }
  const float inv = 1.f / L;
#pragma unroll
  for (int q = 0; q < 8; ++q) o[q] *= inv;
  uint4 hi, lo;
  split8(o, hi, lo);
  const int h = 2 * kvh + hh;
  *reinterpret_cast<uint4*>(attn_out(a, m, h * D + 8 * ch, 0)) = hi;
  *reinterpret_cast<uint4*>(attn_out(a, m, h * D + 8 * ch, 1)) = lo;
}

// Chunk plan of the attention over a prompt of M tokens at `position`: chunk = ceil(U / 32) key
// blocks, U the key blocks of one head's query blocks summed, i.e. about 256 chunk workgroups over
// the 8 heads (one per CU; a workgroup of attn_kernel fills a CU), when the longest query block has
// at least 1.25 chunks and 2 key blocks more than one chunk; otherwise no chunks (one workgroup per
// query block: the grid then holds the work evenly enough, or the merge's extra launch would cost
// more than the shorter chain saves). Every query block has at most U / chunk + 1 chunks, so the
// grid holds at most 8 (32 + nqb) workgroups, the size of the partials' area. Measured on MI355X
// (0.6B prefill from position 0, same box, against one workgroup per query block): prompt 300 3.11
// -> 3.05 ms, 512 3.47 -> 3.30, 1024 4.76 -> 4.33, 2048 7.05 -> 6.63; 1.7B 512 6.14 -> 5.92, 1500
// 12.96 -> 12.60; prompt 100 (2 key blocks) 2.84 -> 2.93 with chunks, hence the 2-block margin.
struct AttnPlan {
  int chunk, wgs, merge;  // key blocks per chunk (0: none), attn_kernel and attn_merge_kernel workgroups
};
static AttnPlan attn_plan(int M, int position) {
  const int nqb = (M + QB - 1) / QB;
  long long U = 0;
  for (int qb = 0; qb < nqb; ++qb) U += attn_nkb(qb, M, position);
  const int T = (int)((U + 31) / 32), maxn = attn_nkb(nqb - 1, M, position);
  if (4 * maxn < 5 * T || maxn < T + 2) return {0, nqb * HKV, 0};
  int wgs = 0;
  for (int c = 0;; ++c) {
    const int n = attn_round(c, T, M, position, nqb);
    if (n == 0) break;
    wgs += n;
  }
  return {T, wgs * HKV, attn_round(1, T, M, position, nqb) * HKV * 8};
}
static size_t attn_part_slots(int M) { return (size_t)HKV * (32 + (M + QB - 1) / QB); }
static int attn_part_rows(int M) { return M < QB ? M : QB; }

// ------------------------------------------------------------------------------------------------
// Final RMSNorm of row `row` of x (the prompt's last token) and the tied LM head with fused greedy
// argmax (/root/reference/megakernel.cu:876-893 and model.py:97): logits[v] = E[v] . norm(x[row]);
// *key = max over v of (order-preserving bf16 of the logit) << 32 | ~v, so equal bf16 values prefer
// the lowest index. Every workgroup normalises the row into LDS (bf16 hi/lo), then its 8 waves
// stream vocabulary rows (row v to wave v % (8 * grid)), 4 rows in flight per wave.
// ------------------------------------------------------------------------------------------------

template <int H>
__global__ void __launch_bounds__(512) lm_head_kernel(const float* x, int row, const uint16_t* final_norm,
                                                      const uint16_t* lm_head, int vocab, float* logits, u64* key,
                                                      const int32_t* bad) {
  constexpr int C = H / 512;  // 16-byte chunks per lane of one vocabulary row
  __shared__ __attribute__((aligned(16))) uint4 xs[2][H / 8];
  __shared__ u64 best[8];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  if (w == 0) {  // normalise
    constexpr int E = H / 64;
    const float* xr = x + (size_t)row * H + E * lane;
    float v[E];
#pragma unroll
    for (int k = 0; k < E; ++k) v[k] = xr[k];
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < E; ++k) ss = fmaf(v[k], v[k], ss);
    const float rs = rsqrtf(wave_sum(ss) / (float)H + EPS);
#pragma unroll
    for (int k = 0; k < E; k += 8) {
      float wv[8], y[8];
      unpack8(*reinterpret_cast<const uint4*>(final_norm + E * lane + k), wv);
#pragma unroll
      for (int q = 0; q < 8; ++q) y[q] = v[k + q] * wv[q] * rs;
      split8(y, xs[0][(E * lane + k) / 8], xs[1][(E * lane + k) / 8]);
    }
  }
  __syncthreads();
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  auto dot2 = [](uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c, false);
  };
  u64 mine = 0;
  const int stride = 8 * gridDim.x;
  const bool failed = *bad != 0;  // an input token was out of range: NaN logits
  constexpr int LP = 4;
  for (int v0 = blockIdx.x * 8 + w; v0 < vocab; v0 += LP * stride) {
    uint4 wr[LP][C];
#pragma unroll
    for (int p = 0; p < LP; ++p) {
      const int v = min(v0 + p * stride, vocab - 1);
#pragma unroll
      for (int k = 0; k < C; ++k) wr[p][k] = ld_stream(reinterpret_cast<const uint4*>(lm_head + (size_t)v * H) + 64 * k + lane);
    }
#pragma unroll
    for (int p = 0; p < LP; ++p) {
      const int v = v0 + p * stride;
      float s0 = 0.f, s1 = 0.f;
#pragma unroll
      for (int k = 0; k < C; ++k) {
        const uint4 h = xs[0][64 * k + lane], l = xs[1][64 * k + lane];
        s0 = dot2(wr[p][k].x, h.x, s0); s1 = dot2(wr[p][k].x, l.x, s1);
        s0 = dot2(wr[p][k].y, h.y, s0); s1 = dot2(wr[p][k].y, l.y, s1);
        s0 = dot2(wr[p][k].z, h.z, s0); s1 = dot2(wr[p][k].z, l.z, s1);
        s0 = dot2(wr[p][k].w, h.w, s0); s1 = dot2(wr[p][k].w, l.w, s1);
      }
      const float s = wave_sum(s0 + s1);
      if (v < vocab) {
        if (lane == 0) logits[v] = failed ? __builtin_nanf("") : s;
        const u64 kv = argmax_key(s, v);
        mine = mine > kv ? mine : kv;
      }
    }
  }
  if (lane == 0) best[w] = mine;
  __syncthreads();
  if (tid == 0) {
    u64 m = 0;
    for (int q = 0; q < 8; ++q) m = m > best[q] ? m : best[q];
    atomicMax(key, m);
  }
}

// Greedy keys of B rows of logits [B][vocab] (the batched LM head's MFMA output): keys[b] = max over
// v of argmax_key(logits[b][v], v); with *bad set the rows are overwritten with NaN instead (a
// failed call is visible in its output). Grid (ceil(vocab / 4096), B), 16 logits per thread.
__global__ void __launch_bounds__(256) logits_argmax_kernel(float* logits, int vocab, u64* keys, const int32_t* bad) {
  __shared__ u64 best[4];
  const int b = blockIdx.y, tid = threadIdx.x;
  float* row = logits + (size_t)b * vocab;
  const bool failed = *bad != 0;
  u64 k = 0;
  // 16 logits per thread as four 16-byte loads issued together (vocab is a multiple of 16)
  float4 x[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int v = blockIdx.x * 4096 + i * 1024 + 4 * tid;
    x[i] = v < vocab ? *reinterpret_cast<const float4*>(row + v) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int v = blockIdx.x * 4096 + i * 1024 + 4 * tid;
    if (v < vocab) {
      const float e[4] = {x[i].x, x[i].y, x[i].z, x[i].w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const u64 kv = argmax_key(e[q], v + q);
        k = k > kv ? k : kv;
      }
      if (failed) {
        const float n = __builtin_nanf("");
        *reinterpret_cast<float4*>(row + v) = make_float4(n, n, n, n);
      }
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const u64 other = __shfl_xor(k, o);
    k = k > other ? k : other;
  }
  if ((tid & 63) == 0) best[tid >> 6] = k;
  __syncthreads();
  if (tid == 0) {
    u64 m = best[0];
    for (int q = 1; q < 4; ++q) m = m > best[q] ? m : best[q];
    atomicMax(keys + b, m);
  }
}

__global__ void keys_init_kernel(u64* keys, int n, int32_t* bad) {  // n <= 64 keys
  if ((int)threadIdx.x < n) keys[threadIdx.x] = 0;
  if (threadIdx.x == 0) *bad = 0;
}

__global__ void keys_to_tokens_kernel(const u64* keys, int R, const int32_t* bad, int32_t* out) {
  const int r = threadIdx.x;
  if (r < R) out[r] = (keys[r] && *bad == 0) ? (int32_t)(0xffffffffu - (uint32_t)(keys[r] & 0xffffffffu)) : -1;
}

// ------------------------------------------------------------------------------------------------
// Batched decode: BMAX = 64 sequences at most, one token each per step, every sequence with its own
// cache ([B][L][8][max_seq][128]) and position. The layer structure of the prefill, with the
// products as skinny GEMMs: the weights are the MFMA's 16-row operand A and 8 sequences'
// activations, hi and lo, its 16 columns (B operand column 2b + hl), so one
// v_mfma_f32_16x16x32_bf16 multiplies 16 weight rows x 32 inputs by 8 sequences at once, up to 8
// such column blocks per weight fragment, and each weight byte is read once per step. Sums split
// over K are written as partials and added in a fixed order by the next kernel, so results are
// deterministic.
// ------------------------------------------------------------------------------------------------
constexpr int BMAX = 64;
constexpr int KS = 64;  // keys per attention split (one round of 4 keys per 16-lane group)

enum SkEpi { SK_RAW = 0, SK_PART = 1, SK_SILU = 2 };

struct SkArgs {
  const uint16_t* xh;  // activations as skinny fragments (skf_off: K inputs, hi and lo) of B rows
  int B, N, K;
  // SK_RAW: rows [0, n1) of w0, [n1, n2) of w1, [n2, N) of w2 (Q, K, V); SK_PART: w0; SK_SILU: w0 gate, w1 up
  const uint16_t* w0;
  const uint16_t* w1;
  const uint16_t* w2;
  int n1, n2;
  float* out;    // SK_RAW: [B][N]; SK_PART: [gridDim.y][B][N]
  uint16_t* mh;  // SK_SILU: silu(gate) * up as skinny fragments of ldm inputs (the down product's operand)
  int ldm;
};


// A workgroup takes 16 weight rows (rows 16 bx ..). SK_RAW / SK_PART: its K range [by K / gy, ...)
// split over the 4 waves; SK_SILU: 8 intermediates, their 8 gate rows and 8 up rows in one 16-row
// tile, K split over the 4 waves. Each wave's K range is a multiple of 256 (checked on the host).
// The B operand holds CB column blocks of 8 rows of activations (a decode batch, or up to 64 prompt
// tokens): column li of block cb is row 8 cb + li / 2, hi (even li) or lo (odd li), read as skinny
// fragments (skf_off) of the CB column blocks. The weight fragments of a K chunk stay in registers
// across the column blocks; up to 4 blocks' activation fragments are in flight while a block is
// multiplied.
template <int EPI, int CB>
__global__ void __launch_bounds__(256) skinny_kernel(const SkArgs g) {
  constexpr int NC = 8 * CB;
  __shared__ float red[4][16][NC + 1];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const int n0 = 16 * blockIdx.x, n = n0 + li;
  const uint16_t* wrow;
  int kb, ke;
  if constexpr (EPI == SK_SILU) {
    wrow = (li < 8 ? g.w0 : g.w1) + (size_t)(8 * blockIdx.x + (li & 7)) * g.K;
    const int kw = g.K / 4;
    kb = w * kw;
    ke = kb + kw;
  } else {
    if constexpr (EPI == SK_RAW)
      wrow = n < g.n1 ? g.w0 + (size_t)n * g.K
                      : (n < g.n2 ? g.w1 + (size_t)(n - g.n1) * g.K : g.w2 + (size_t)(n - g.n2) * g.K);
    else
      wrow = g.w0 + (size_t)n * g.K;
    const int kc = g.K / gridDim.y, kw = kc / 4;
    kb = blockIdx.y * kc + w * kw;
    ke = kb + kw;
  }
  const int sb = li >> 1;
  f32x4 c[CB];
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) c[cb] = f32x4{0.f, 0.f, 0.f, 0.f};
  const uint4* xf = reinterpret_cast<const uint4*>(g.xh) + lane;  // this lane's 16 bytes of fragment 0
  auto ld_act = [&](int cb, int k) { return xf[skf_frag(cb, k >> 5, CB, g.K) * 64]; };
  // R column blocks' activation fragments in flight: block cb + R's loads go into the registers
  // block cb's MFMAs have just read (no copies: a register copy of a pending load would wait for it)
  constexpr int R = CB < 4 ? CB : 4;
  for (int k0 = kb; k0 < ke; k0 += 256) {
    uint4 wa[8], xq[R][8];
#pragma unroll
    for (int u = 0; u < 8; ++u) wa[u] = ld_stream(reinterpret_cast<const uint4*>(wrow + k0 + 32 * u + 8 * lg));
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
      for (int u = 0; u < 8; ++u) xq[r][u] = ld_act(r, k0 + 32 * u);
      __builtin_amdgcn_sched_barrier(0);  // the blocks' loads in block order: each wait covers one block
    }
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
#pragma unroll
      for (int u = 0; u < 8; ++u) c[cb] = mfma(wa[u], xq[cb % R][u], c[cb]);
      if (cb + R < CB) {
#pragma unroll
        for (int u = 0; u < 8; ++u) xq[cb % R][u] = ld_act(cb + R, k0 + 32 * u);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // C[row 4 lg + j][column li]: activation row 8 cb + li / 2 is the sum of its hi and lo columns
#pragma unroll
  for (int cb = 0; cb < CB; ++cb)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float v = c[cb][j] + __shfl_xor(c[cb][j], 1);
      if (!(li & 1)) red[w][4 * lg + j][8 * cb + sb] = v;
    }
  __syncthreads();
  for (int idx = tid; idx < (EPI == SK_SILU ? 8 : 16) * g.B; idx += 256) {
    const int r = idx / g.B, b = idx % g.B;
    if constexpr (EPI == SK_SILU) {
      const float gt = ((red[0][r][b] + red[1][r][b]) + red[2][r][b]) + red[3][r][b];
      const float up = ((red[0][r + 8][b] + red[1][r + 8][b]) + red[2][r + 8][b]) + red[3][r + 8][b];
      const float m = gt / (1.f + expf(-gt)) * up;
      const uint16_t hi = f32_to_bf16(m), lo = f32_to_bf16(m - bf16_to_f32(hi));
      const int it = 8 * blockIdx.x + r;  // into the down product's skinny fragments (g.ldm inputs)
      g.mh[skf_off(b, it, 0, g.B, g.ldm)] = hi;
      g.mh[skf_off(b, it, 1, g.B, g.ldm)] = lo;
    } else {
      const float v = ((red[0][r][b] + red[1][r][b]) + red[2][r][b]) + red[3][r][b];
      g.out[((size_t)blockIdx.y * g.B + b) * g.N + n0 + r] = v;
    }
  }
}


// The skinny product for up to 8 * cb activation rows (cb: 1, 2, 4 or 8 column blocks).
static hipError_t launch_skinny(int epi, int cb, dim3 grid, const SkArgs& a, hipStream_t st) {
#define MK_SK(E, C) hipLaunchKernelGGL((skinny_kernel<E, C>), grid, dim3(256), 0, st, a)
#define MK_SK_CB(E) \
  if (cb == 1) MK_SK(E, 1); else if (cb == 2) MK_SK(E, 2); else if (cb == 4) MK_SK(E, 4); else MK_SK(E, 8)
  if (epi == SK_RAW) { MK_SK_CB(SK_RAW); } else if (epi == SK_PART) { MK_SK_CB(SK_PART); } else { MK_SK_CB(SK_SILU); }
#undef MK_SK_CB
#undef MK_SK
  return hipGetLastError();
}
static int column_blocks(int rows) { return rows <= 8 ? 1 : rows <= 16 ? 2 : rows <= 32 ? 4 : 8; }

// Rows b < B of the residual: with `tokens`, x[b] = embed[tokens[b]] (a token outside [0, vocab)
// reads row 0 and sets *bad); with `part`, x[b] += sum over s < S of part[s][b] (in order); then,
// with `w`, RMSNorm into the bf16 hi/lo pair in the layout LAYOUT names. One wave per row (any
// number of waves per workgroup).
// LAYOUT 0: row order ah/al [B][lda]; 1: the GEMM's fragment order (frag_off, H columns); 2: skinny
// fragments (skf_off, H inputs, hi and lo both in ah).
template <int H, int LAYOUT = 0>
__global__ void __launch_bounds__(256) bnorm_kernel(float* x, const int32_t* tokens, const uint16_t* embed, int vocab,
                                                    int32_t* bad, const float* part, int S, const uint16_t* w,
                                                    uint16_t* ah, uint16_t* al, int lda, int B) {
  constexpr int E = H / 64;
  const int lane = threadIdx.x & 63;
  const int b = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (b >= B) return;
  // the norm weights first: their loads then overlap the residual's instead of following the
  // reduction (one round trip fewer per call)
  uint4 wr[E / 8];
  if (w) {
#pragma unroll
    for (int k = 0; k < E; k += 8) wr[k / 8] = *reinterpret_cast<const uint4*>(w + E * lane + k);
  }
  float v[E];
  float* xr = x + (size_t)b * H + E * lane;
  if (tokens) {
    int tok = tokens[b];
    if (tok < 0 || tok >= vocab) {
      if (lane == 0) *bad = 1;
      tok = 0;
    }
    const uint16_t* er = embed + (size_t)tok * H + E * lane;
#pragma unroll
    for (int k = 0; k < E; k += 8) {
      float t[8];
      unpack8(*reinterpret_cast<const uint4*>(er + k), t);
#pragma unroll
      for (int q = 0; q < 8; ++q) v[k + q] = t[q];
    }
  } else {
#pragma unroll
    for (int k = 0; k < E; k += 4) {
      const float4 t = *reinterpret_cast<const float4*>(xr + k);
      v[k] = t.x; v[k + 1] = t.y; v[k + 2] = t.z; v[k + 3] = t.w;
    }
    // the partials in order, four at a time: their loads go out together (one round trip per four
    // partials instead of one per partial; up to 16 partials come from the batched decode's products)
    for (int s0 = 0; s0 < S; s0 += 4) {
      float4 t[4][E / 4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float* pr = part + ((size_t)(s0 + i < S ? s0 + i : s0) * B + b) * H + E * lane;
#pragma unroll
        for (int k = 0; k < E; k += 4) t[i][k / 4] = *reinterpret_cast<const float4*>(pr + k);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (s0 + i < S) {
#pragma unroll
          for (int k = 0; k < E; k += 4) {
            v[k] += t[i][k / 4].x; v[k + 1] += t[i][k / 4].y; v[k + 2] += t[i][k / 4].z; v[k + 3] += t[i][k / 4].w;
          }
        }
      }
    }
  }
  if (tokens || S > 0) {  // x changed
#pragma unroll
    for (int k = 0; k < E; k += 4) *reinterpret_cast<float4*>(xr + k) = make_float4(v[k], v[k + 1], v[k + 2], v[k + 3]);
  }
  if (!w) return;
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < E; ++k) ss = fmaf(v[k], v[k], ss);
  const float rs = rsqrtf(wave_sum(ss) / (float)H + EPS);
#pragma unroll
  for (int k = 0; k < E; k += 8) {
    float wv[8], y[8];
    unpack8(wr[k / 8], wv);
#pragma unroll
    for (int q = 0; q < 8; ++q) y[q] = v[k + q] * wv[q] * rs;
    uint4 hi, lo;
    split8(y, hi, lo);
    if constexpr (LAYOUT == 2) {
      *reinterpret_cast<uint4*>(ah + skf_off(b, E * lane + k, 0, B, H)) = hi;
      *reinterpret_cast<uint4*>(ah + skf_off(b, E * lane + k, 1, B, H)) = lo;
    } else {
      const size_t o = LAYOUT == 1 ? frag_off(b, E * lane + k, H) : (size_t)b * lda + E * lane + k;
      *reinterpret_cast<uint4*>(ah + o) = hi;
      *reinterpret_cast<uint4*>(al + o) = lo;
    }
  }
}

// Position of sequence b, clamped into the cache (an out-of-range position sets *bad).
__device__ __forceinline__ int seq_pos(const int32_t* positions, int b, int max_seq, int32_t* bad) {
  const int p = positions[b];
  if (p < 0 || p >= max_seq) {
    if (bad) *bad = 1;
    return p < 0 ? 0 : max_seq - 1;
  }
  return p;
}

// The raw Q/K/V sums of M consecutive prompt tokens of one sequence (fp32 [M][4096], or S such arrays
// of K-range sums added in order; row m at position pos0 + m): per-head RMSNorm + RoPE on q and k,
// q kept as a bf16 hi/lo pair [M][2048], k and v rounded to bf16 into the cache [L][8][max_seq][128].
__global__ void __launch_bounds__(64) qkv_post_kernel(const float* raw, int S, int M, int pos0, const uint16_t* q_norm,
                                                       const uint16_t* k_norm, const uint16_t* cos_tab,
                                                       const uint16_t* sin_tab, uint16_t* qh, uint16_t* ql,
                                                       uint16_t* k_cache, uint16_t* v_cache, int layer, KvMap kv,
                                                       int32_t* bad) {
  // one item (row b, head hd) per 16-lane group, lane t holding dims 8 t .. +7 (head_norm_rope's
  // layout): 16-byte loads and stores
  const int t = threadIdx.x & 15;
  const int item = blockIdx.x * 4 + (threadIdx.x >> 4);  // single-wave workgroups: the items spread over the CUs
  if (item >= M * (HQ + 2 * HKV)) return;  // uniform in the 16-lane group
  const int b = item / (HQ + 2 * HKV), hd = item % (HQ + 2 * HKV);
  const int pos = pos0 + b;
  // the sums of S K ranges (EPI_QKV_PART), added in order
  const size_t rstride = (size_t)M * (HQ + 2 * HKV) * D;
  const float* r = raw + (size_t)b * (HQ + 2 * HKV) * D + hd * D + 8 * t;
  float v[8];
  {
    const float4 x0 = *reinterpret_cast<const float4*>(r), x1 = *reinterpret_cast<const float4*>(r + 4);
    v[0] = x0.x; v[1] = x0.y; v[2] = x0.z; v[3] = x0.w; v[4] = x1.x; v[5] = x1.y; v[6] = x1.z; v[7] = x1.w;
  }
  for (int q = 1; q < S; ++q) {
    const float4 x0 = *reinterpret_cast<const float4*>(r + q * rstride);
    const float4 x1 = *reinterpret_cast<const float4*>(r + q * rstride + 4);
    v[0] += x0.x; v[1] += x0.y; v[2] += x0.z; v[3] += x0.w; v[4] += x1.x; v[5] += x1.y; v[6] += x1.z; v[7] += x1.w;
  }
  const int page = hd >= HQ && kv.bt ? kv_page(kv, pos, t == 0 ? bad : nullptr) : 0;
  auto pack = [&]() {
    return make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                      pack_bf16x2(v[6], v[7]));
  };
  if (hd >= HQ + HKV) {  // v
    if (page >= 0)
      *reinterpret_cast<uint4*>(v_cache + kv_row(kv, layer, hd - HQ - HKV, pos, page) + 8 * t) = pack();
    return;
  }
  // per-head RMSNorm and rotate-half RoPE (/root/reference/megakernel.cu:490-630, 548-555)
  float wn[8], cs[8], sn[8];
  unpack8(*reinterpret_cast<const uint4*>((hd < HQ ? q_norm : k_norm) + 8 * t), wn);
  unpack8(*reinterpret_cast<const uint4*>(cos_tab + (size_t)pos * D + 8 * (t & 7)), cs);
  unpack8(*reinterpret_cast<const uint4*>(sin_tab + (size_t)pos * D + 8 * (t & 7)), sn);
  head_norm_rope(v, wn, cs, sn, t);
  if (hd < HQ) {
    uint4 hi, lo;
    split8(v, hi, lo);
    const size_t o = (size_t)b * HQ * D + hd * D + 8 * t;
    *reinterpret_cast<uint4*>(qh + o) = hi;
    *reinterpret_cast<uint4*>(ql + o) = lo;
  } else if (page >= 0) {
    *reinterpret_cast<uint4*>(k_cache + kv_row(kv, layer, hd - HQ, pos, page) + 8 * t) = pack();
  }
}

// silu(gate) * up of M rows from the S K-range sums of EPI_SILU_PART (part[S][M][2 I]: tile t's
// columns 128 t .. +63 the gate and 128 t + 64 .. +127 the up sums of intermediates 64 t .. +63),
// added in order, into the down product's A operand (bf16 hi/lo, fragment-major, I columns), as
// the EPI_SILU epilogue writes it. One thread per row and 8 intermediates.
__global__ void __launch_bounds__(64) silu_post_kernel(const float* part, int S, int M, int I, uint16_t* bh,
                                                        uint16_t* bl) {
  const int nc = I / 8, idx = blockIdx.x * 64 + threadIdx.x;  // single-wave workgroups: spread over the CUs
  if (idx >= M * nc) return;
  const int m = idx / nc, i0 = 8 * (idx % nc);
  const size_t stride = (size_t)M * 2 * I;
  const float* pg = part + (size_t)m * 2 * I + 128 * (i0 >> 6) + (i0 & 63);
  float gt[8], up[8];
  auto ld8 = [](const float* p, float (&v)[8]) {
    const float4 a = *reinterpret_cast<const float4*>(p), b = *reinterpret_cast<const float4*>(p + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  };
  ld8(pg, gt);
  ld8(pg + 64, up);
  for (int q = 1; q < S; ++q) {
    float g2[8], u2[8];
    ld8(pg + q * stride, g2);
    ld8(pg + q * stride + 64, u2);
#pragma unroll
    for (int k = 0; k < 8; ++k) { gt[k] += g2[k]; up[k] += u2[k]; }
  }
  float mv[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) mv[k] = gt[k] / (1.f + expf(-gt[k])) * up[k];  // silu(gate) * up (/root/reference/megakernel.cu:659-665)
  uint4 hi, lo;
  split8(mv, hi, lo);
  const size_t o = frag_off(m, i0, I);
  *reinterpret_cast<uint4*>(bh + o) = hi;
  *reinterpret_cast<uint4*>(bl + o) = lo;
}

// Split-K attention of one sequence and K/V head over keys [KS s, KS s + KS) of [0, position]: the
// head pair's two queries against each key (16 groups of 16 lanes, lane t holding dims 8t..8t+7,
// keys dealt to the groups in turn, online softmax per group, /root/reference/megakernel.cu:228-370),
// the 16 group partials merged in LDS into this split's (acc[128], m, l) per query head.
// part: [B][8][S][2][D + 2].
constexpr int APW = D + 2;


constexpr int BU = 4;  // keys per 16-lane group and split: one round of loads
static_assert(KS == 16 * BU, "a split is one round of loads");

// Group gi's keys of split s (positions k0 + gi + 16 u; past the split they re-read its last key).
__device__ __forceinline__ void battn_load(const uint16_t* k_cache, const uint16_t* v_cache, int b, int kvh, int s,
                                           int ctx, int L, int layer, int max_seq, uint4 (&kw)[BU],
                                           uint4 (&vw)[BU]) {
  const int lane = threadIdx.x & 63, gi = (threadIdx.x >> 6) * 4 + (lane >> 4), t = lane & 15;
  const int k0 = s * KS, k1 = min(k0 + KS, ctx);
  const size_t base = (((size_t)b * L + layer) * HKV + kvh) * max_seq * D + 8 * t;
#pragma unroll
  for (int u = 0; u < BU; ++u) {
    const int pu = min(k0 + gi + 16 * u, k1 - 1);
    kw[u] = *reinterpret_cast<const uint4*>(k_cache + base + (size_t)pu * D);
    vw[u] = *reinterpret_cast<const uint4*>(v_cache + base + (size_t)pu * D);
  }
}

__device__ __forceinline__ void battn_split(const float (&qa)[8], const float (&qb)[8], uint4 knew, uint4 vnew,
                                            int pos, const uint4 (&kw)[BU], const uint4 (&vw)[BU], int b,
                                            int kvh, int s, int ctx, float* part, int S, float (&gacc)[16][2][D],
                                            float (&gml)[16][2][2]) {
  const int k0 = s * KS;
  const int k1 = min(k0 + KS, ctx);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int gi = w * 4 + (lane >> 4), t = lane & 15;
  float m0 = -INFINITY, m1 = -INFINITY, l0 = 0.f, l1 = 0.f, a0[8], a1[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) { a0[i] = 0.f; a1[i] = 0.f; }
  auto step = [&](float sc, const float (&v)[8], float& m, float& l, float (&acc)[8]) {
    const float nm = fmaxf(m, sc);
    const float cm = __expf(m - nm), e = __expf(sc - nm);
    l = l * cm + e;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = acc[i] * cm + e * v[i];
    m = nm;
  };
#pragma unroll
  for (int u = 0; u < BU; ++u) {
    const int p = k0 + gi + 16 * u;
    const bool own = p == pos;  // the new row, from registers
    float kf[8], vf[8];
    unpack8(own ? knew : kw[u], kf);
    unpack8(own ? vnew : vw[u], vf);
    float d0 = 0.f, d1 = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) { d0 = fmaf(qa[i], kf[i], d0); d1 = fmaf(qb[i], kf[i], d1); }
    d0 = row16_sum(d0) * ATT_SCALE;
    d1 = row16_sum(d1) * ATT_SCALE;
    if (p < k1) {
      step(d0, vf, m0, l0, a0);
      step(d1, vf, m1, l1, a1);
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) { gacc[gi][0][8 * t + i] = a0[i]; gacc[gi][1][8 * t + i] = a1[i]; }
  if (t == 0) { gml[gi][0][0] = m0; gml[gi][0][1] = l0; gml[gi][1][0] = m1; gml[gi][1][1] = l1; }
  __syncthreads();
  const int h = tid >> 7, d = tid & 127;
  float M = -INFINITY;
  for (int q = 0; q < 16; ++q) M = fmaxf(M, gml[q][h][0]);  // finite: the split has a key
  float A = 0.f, Ls = 0.f;
  for (int q = 0; q < 16; ++q) {
    const float f = __expf(gml[q][h][0] - M);  // 0 for a group without keys
    A = fmaf(gacc[q][h][d], f, A);
    Ls = fmaf(gml[q][h][1], f, Ls);
  }
  float* o = part + ((((size_t)b * HKV + kvh) * S + s) * 2 + h) * APW;
  o[d] = A;
  if (d == 0) { o[D] = M; o[D + 1] = Ls; }
}

// The attention of one sequence and K/V head, with the new row's projections finished here (from the
// raw Q/K/V sums, fp32 [B][4096]): every 16-lane group normalises and rotates the pair's two query
// heads itself, and the new K row (normalised, rotated) and V row are rounded to bf16; the workgroup
// whose splits include the sequence's position writes them into the cache and attends to that
// position from registers. Workgroup x takes splits x, x + gridDim.x, ... of [0, position] (the grid
// does not depend on the device-side positions); the merge reads splits below ceil(ctx / KS) only.
__global__ void __launch_bounds__(256) battn_partial_kernel(const float* raw, const int32_t* positions,
                                                            const int32_t* tokens, int vocab,
                                                            const uint16_t* q_norm, const uint16_t* k_norm,
                                                            const uint16_t* cos_tab, const uint16_t* sin_tab,
                                                            uint16_t* k_cache, uint16_t* v_cache, int L, int layer,
                                                            int max_seq, float* part, int S, int32_t* bad) {
  __shared__ float gacc[16][2][D];
  __shared__ float gml[16][2][2];
  const int kvh = blockIdx.y, b = blockIdx.z;
  const int lane = threadIdx.x & 63, t = lane & 15;
  const int pos = seq_pos(positions, b, max_seq, threadIdx.x == 0 && blockIdx.x == 0 && kvh == 0 ? bad : nullptr);
  // a sequence whose position or token is out of range reports NaN and -1 and keeps its cache as it
  // was: its new K/V rows are not written (the clamped position would overwrite a valid row)
  const bool write_ok = positions[b] == pos && tokens[b] >= 0 && tokens[b] < vocab;
  const int ctx = pos + 1;
  if ((int)blockIdx.x * KS >= ctx) return;  // no split for this workgroup (the grid fits the longest cache)
  // the first split's K/V rows are in flight while the new row's projections are finished
  uint4 kw[BU], vw[BU];
  battn_load(k_cache, v_cache, b, kvh, blockIdx.x, ctx, L, layer, max_seq, kw, vw);
  const float* rr = raw + (size_t)b * (HQ + 2 * HKV) * D + 8 * t;
  float qa[8], qb[8], kn[8], vv[8], qw[8], kwn[8], cs[8], sn[8];
  auto ld8 = [](const float* p, float (&v)[8]) {
    const float4 x = *reinterpret_cast<const float4*>(p), y = *reinterpret_cast<const float4*>(p + 4);
    v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w; v[4] = y.x; v[5] = y.y; v[6] = y.z; v[7] = y.w;
  };
  ld8(rr + (2 * kvh) * D, qa);
  ld8(rr + (2 * kvh + 1) * D, qb);
  ld8(rr + (HQ + kvh) * D, kn);
  ld8(rr + (HQ + HKV + kvh) * D, vv);
  unpack8(*reinterpret_cast<const uint4*>(q_norm + 8 * t), qw);
  unpack8(*reinterpret_cast<const uint4*>(k_norm + 8 * t), kwn);
  unpack8(*reinterpret_cast<const uint4*>(cos_tab + (size_t)pos * D + 8 * (t & 7)), cs);  // dims mod 64
  unpack8(*reinterpret_cast<const uint4*>(sin_tab + (size_t)pos * D + 8 * (t & 7)), sn);
  head_norm_rope(qa, qw, cs, sn, t);
  head_norm_rope(qb, qw, cs, sn, t);
  head_norm_rope(kn, kwn, cs, sn, t);
  const uint4 knew = make_uint4(pack_bf16x2(kn[0], kn[1]), pack_bf16x2(kn[2], kn[3]), pack_bf16x2(kn[4], kn[5]),
                                pack_bf16x2(kn[6], kn[7]));
  const uint4 vnew = make_uint4(pack_bf16x2(vv[0], vv[1]), pack_bf16x2(vv[2], vv[3]), pack_bf16x2(vv[4], vv[5]),
                                pack_bf16x2(vv[6], vv[7]));
  if (write_ok && threadIdx.x < 16 && (pos / KS) % gridDim.x == blockIdx.x) {
    const size_t row = ((((size_t)b * L + layer) * HKV + kvh) * max_seq + pos) * D + 8 * t;
    *reinterpret_cast<uint4*>(k_cache + row) = knew;
    *reinterpret_cast<uint4*>(v_cache + row) = vnew;
  }
  for (int s = blockIdx.x; s * KS < ctx; s += gridDim.x) {
    if (s != (int)blockIdx.x) battn_load(k_cache, v_cache, b, kvh, s, ctx, L, layer, max_seq, kw, vw);
    battn_split(qa, qb, knew, vnew, pos, kw, vw, b, kvh, s, ctx, part, S, gacc, gml);
    __syncthreads();  // gacc / gml are reused by the next split
  }
}

// Merge of the splits of each sequence and query head into the O-projection's input row (bf16 hi/lo
// [B][2048]); 128 threads, one per dim.
// ldo == 0: skinny fragments of the 2048 attention outputs in oh (hi and lo).
__global__ void __launch_bounds__(128) battn_merge_kernel(const float* part, int S, const int32_t* positions,
                                                          int max_seq, uint16_t* oh, uint16_t* ol, int ldo) {
  const int b = blockIdx.x, h = blockIdx.y, d = threadIdx.x;
  const int kvh = h >> 1, hh = h & 1;
  const int pos = seq_pos(positions, b, max_seq, nullptr);
  const float* p = part + (((size_t)b * HKV + kvh) * S * 2 + hh) * APW;
  // The first NB splits' words are loaded together with the position (one round trip instead of one
  // per split and pass); those past the sequence's split count are read (inside the S allocated
  // slots) but never used.
  constexpr int NB = 16;
  float mv[NB], lv[NB], av[NB];
  {
    // lane l of each wave loads split l % NB's (m, l) pair (vector loads, issued with the rest), then
    // every lane reads them off lanes 0..NB-1
    const int sl = d & (NB - 1);
    const float2 ml = *reinterpret_cast<const float2*>(p + (size_t)(sl < S ? sl : 0) * 2 * APW + D);
#pragma unroll
    for (int s = 0; s < NB; ++s) av[s] = p[(size_t)(s < S ? s : 0) * 2 * APW + d];
#pragma unroll
    for (int s = 0; s < NB; ++s) {
      mv[s] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ml.x), s));
      lv[s] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ml.y), s));
    }
  }
  const int ns = (pos + KS) / KS;  // ceil((pos + 1) / KS)
  // max first over the first NB splits, then their weighted sums in split order (selects, not
  // branches, so that no loop separates the loads above from their use)
  float M = -INFINITY;
#pragma unroll
  for (int s = 0; s < NB; ++s) M = fmaxf(M, s < ns ? mv[s] : -INFINITY);
  float A = 0.f, Ls = 0.f;
#pragma unroll
  for (int s = 0; s < NB; ++s) {
    const bool in = s < ns;
    const float f = in ? __expf(mv[s] - M) : 0.f;
    A = in ? fmaf(av[s], f, A) : A;
    Ls = in ? fmaf(lv[s], f, Ls) : Ls;
  }
  // splits past NB (caches longer than NB * KS keys): online, rescaling the sums to a new maximum
  for (int s = NB; s < ns; ++s) {
    const float* q = p + (size_t)s * 2 * APW;
    const float m = q[D];
    if (m > M) {
      const float c = __expf(M - m);
      A *= c;
      Ls *= c;
      M = m;
    }
    const float f = __expf(m - M);
    A = fmaf(q[d], f, A);
    Ls = fmaf(q[D + 1], f, Ls);
  }
  const float o = A / Ls;
  const uint16_t hi = f32_to_bf16(o), lo = f32_to_bf16(o - bf16_to_f32(hi));
  if (ldo == 0) {
    oh[skf_off(b, h * D + d, 0, gridDim.x, HQ * D)] = hi;
    oh[skf_off(b, h * D + d, 1, gridDim.x, HQ * D)] = lo;
  } else {
    oh[(size_t)b * ldo + h * D + d] = hi;
    ol[(size_t)b * ldo + h * D + d] = lo;
  }
}

// ------------------------------------------------------------------------------------------------
// Host side
// ------------------------------------------------------------------------------------------------
template <int H, int I>
struct BatchPlan {  // K splits of the skinny O and down products
  static constexpr int SO = H == 1024 ? 2 : 2;  // O: K = 2048
  static constexpr int SD = H == 1024 ? 3 : 2;  // down: K = I
  static constexpr int SP = SO > SD ? SO : SD;
  static_assert((HQ * D / SO / 4) % 256 == 0 && (I / SD / 4) % 256 == 0 && (H / 4) % 256 == 0 && (H / 2) % 256 == 0,
                "wave K ranges must be multiples of 256");
};

struct Work {
  float* x;
  uint16_t *ah, *al, *bh, *bl, *qh, *ql;
  float* raw;   // short prompts: Q/K/V row sums [M][4096]
  float* part;  // split-K partials of the O and down products [splits][M][H]
  float* qpart; // split-K partials of the QKV or gate/up product on small grids [splits][M][4096 or 2 I]
  float* apart; // the attention's key-range chunk partials (attn_plan)
  u64* keys;
  int32_t* bad;
};

// Prompts of at most small_m(H) tokens run their products on the skinny kernels (weights as the
// MFMA A operand, the tokens as up to 4 column blocks); longer ones on 128 x 128 tiles (QKV and
// gate/up split over K on small grids). Measured on MI355X (same box, ms per prefill, skinny /
// tiles): 0.6B 24 tokens 1.51 / 1.81, 32 1.65 / 1.87, 33 1.84 / 1.87, 40 1.93 / 1.91, 64 2.39 / 2.01;
// 1.7B 24 tokens 2.61 / 2.87, 32 2.94 / 2.93, 33 3.29 / 2.94, 48 3.74 / 3.01.
static int small_m(int H) { return H <= 1024 ? 64 : 32; }

static size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

// K splits of a residual product (O or down, N = H columns) on 128 x 128 tiles for M > small_m(H):
// as many as keep the grid within one workgroup per CU (the grid then takes gemm_kernel's deeper
// pipeline), none from 192 tiles on, at most 8, each K range a whole number of 64-wide steps. The
// partials are added to the residual by the next norm, in split order; without a split the
// product adds into the residual itself. Measured on MI355X against grids of up to 512 workgroups
// (two per CU, one step in flight), same box: 0.6B prompt 1,024 / 3,584 4.40 / 12.55 -> 4.29 /
// 12.36 ms, 1.7B prompt 512 / 1,500 5.95 / 13.04 -> 5.47 / 12.77 ms, 2,048 unchanged.
static int resid_splits(int H, int M, int K) {
  const int tiles = (H / NT) * ((M + MT - 1) / MT);
  if (M <= small_m(H) || tiles >= 192) return 1;
  int sp = 256 / tiles;
  sp = sp < 8 ? sp : 8;
  while ((K / KT) % sp != 0) --sp;
  return sp;
}

// K splits of the QKV or gate/up product (`tiles` 128 x 128 tiles, K = H) for M > small_m(H): on a
// grid of at most 128 tiles, as many as keep it within 256 workgroups (one per CU, on gemm_kernel's
// deeper pipeline), at most 8, each K range a whole number of 64-wide steps; qkv_post_kernel /
// silu_post_kernel then add the ranges and do the epilogue the tiles would have fused.
static int small_grid_splits(int tiles, int K) {
  if (tiles > 128) return 1;
  int sp = 256 / tiles;
  sp = sp < 8 ? sp : 8;
  while ((K / KT) % sp != 0) --sp;
  return sp;
}
static int qkv_splits(int H, int M) {
  return M <= small_m(H) ? 1 : small_grid_splits((HQ + 2 * HKV) * D / NT * ((M + MT - 1) / MT), H);
}
static int silu_splits(int H, int I, int M) {
  return M <= small_m(H) ? 1 : small_grid_splits(I / (NT / 2) * ((M + MT - 1) / MT), H);
}

// Workspace layout for M rows: x fp32 [M][H]; a (hi, lo) bf16, max(H, 2048) columns; b (hi, lo)
// bf16, I columns (a and b: row-major for the skinny kernels, fragment-major for gemm_kernel, rows
// rounded up to MT); q (hi, lo) bf16 [M][2048]; for M <= small_m(H) the raw Q/K/V sums; the split-K partials of
// the residual products; the argmax keys. Offsets in bytes, each 256-byte aligned.
struct Layout {
  size_t x, ah, al, bh, bl, qh, ql, raw, part, qpart, apart, keys, bad, bytes;
};
static Layout layout(int H, int I, int M) {
  const size_t A = H > HQ * D ? H : HQ * D;
  Layout L;
  size_t o = 0;
  auto take = [&](size_t n) { const size_t r = o; o += align256(n); return r; };
  const size_t MA = frag_rows(M);  // the GEMMs' activation operands hold whole row tiles
  L.x = take((size_t)M * H * 4);
  L.ah = take(MA * A * 2);
  L.al = take(MA * A * 2);
  L.bh = take(MA * I * 2);
  L.bl = take(MA * I * 2);
  L.qh = take((size_t)M * HQ * D * 2);
  L.ql = take((size_t)M * HQ * D * 2);
  const bool small = M <= small_m(H);
  L.raw = take(small ? (size_t)M * (HQ + 2 * HKV) * D * 4 : 0);
  const int so = resid_splits(H, M, HQ * D), sd = resid_splits(H, M, I);
  const int sp = small ? 3 : (so > sd ? so : sd);
  L.part = take(sp > 1 ? (size_t)sp * M * H * 4 : 0);
  const int sq = qkv_splits(H, M), su = silu_splits(H, I, M);
  size_t qp = sq > 1 ? (size_t)sq * M * (HQ + 2 * HKV) * D : 0;
  if (su > 1 && (size_t)su * M * 2 * I > qp) qp = (size_t)su * M * 2 * I;
  L.qpart = take(qp * 4);
  L.apart = take(attn_part_slots(M) * 2 * attn_part_rows(M) * APS * 4);
  L.keys = take(8);
  L.bad = take(4);
  L.bytes = o;
  return L;
}
static Work carve(void* base, const Layout& L) {
  char* p = static_cast<char*>(base);
  Work w;
  w.x = reinterpret_cast<float*>(p + L.x);
  w.ah = reinterpret_cast<uint16_t*>(p + L.ah);
  w.al = reinterpret_cast<uint16_t*>(p + L.al);
  w.bh = reinterpret_cast<uint16_t*>(p + L.bh);
  w.bl = reinterpret_cast<uint16_t*>(p + L.bl);
  w.qh = reinterpret_cast<uint16_t*>(p + L.qh);
  w.ql = reinterpret_cast<uint16_t*>(p + L.ql);
  w.raw = reinterpret_cast<float*>(p + L.raw);
  w.part = reinterpret_cast<float*>(p + L.part);
  w.qpart = reinterpret_cast<float*>(p + L.qpart);
  w.apart = reinterpret_cast<float*>(p + L.apart);
  w.keys = reinterpret_cast<u64*>(p + L.keys);
  w.bad = reinterpret_cast<int32_t*>(p + L.bad);
  return w;
}

// K steps in flight (gemm_kernel's PF) of a launch. Grids of at most one workgroup per CU: 4, else 2
// (whichever divides the steps). Grids of two or more workgroups per CU: 2, at two workgroups per CU.
// In between (1 to 2 workgroups per CU): 1. Measured on MI355X, per launch, 1 -> 2 steps in flight:
// 0.6B prompt 3,584 QKV (896 workgroups) 80.5 -> 73.3 us, gate/up (1,344) 97.5 -> 96.2 us; prompt
// 2,048 QKV (512) 42.9 -> 40.9 us, gate/up (768) 58.4 -> 54.6 us; 1.7B prompt 1,500 gate/up (1,152)
// 161.9 -> 156.8 us; but 1.7B prompt 512 gate/up (384) 62.5 -> 66.0 us.
static int gemm_pf(dim3 grid, int K) {
  const int steps = K / (int)grid.z / KT, wgs = (int)(grid.x * grid.y * grid.z);
  if (wgs <= 256) return steps % 4 == 0 ? 4 : steps % 2 == 0 ? 2 : 1;
  return wgs >= 512 && steps % 2 == 0 ? 2 : 1;
}
template <int EPI>
static hipError_t launch_gemm(dim3 grid, const GemmArgs& g, hipStream_t st) {
  switch (gemm_pf(grid, g.K)) {
    case 4: hipLaunchKernelGGL((gemm_kernel<EPI, 4>), grid, dim3(256), 0, st, g); break;
    case 2: hipLaunchKernelGGL((gemm_kernel<EPI, 2>), grid, dim3(256), 0, st, g); break;
    default: hipLaunchKernelGGL((gemm_kernel<EPI, 1>), grid, dim3(256), 0, st, g); break;
  }
  return hipGetLastError();
}

template <int H, int I>
static hipError_t run(const mk_model_dims& dims, const int32_t* tokens, int M, int position, const uint16_t* embed,
                      const uint16_t* lm_head, const uint16_t* final_norm, const mk_layer_weights* layers,
                      const uint16_t* cos_tab, const uint16_t* sin_tab, uint16_t* k_cache, uint16_t* v_cache,
                      const KvMap& kv, float* logits, int32_t* out_token, const Work& wk, hipStream_t st) {
  const int A = H > HQ * D ? H : HQ * D;
  const int mtiles = (M + MT - 1) / MT;
  hipError_t e;
#define MKP_LAUNCH(...)                                   \
  do {                                                    \
    hipLaunchKernelGGL(__VA_ARGS__);                      \
    if ((e = hipGetLastError()) != hipSuccess) return e;  \
  } while (0)
  MKP_LAUNCH(keys_init_kernel, dim3(1), dim3(64), 0, st, wk.keys, 1, wk.bad);
  const AttnPlan ap = attn_plan(M, position);
  if ((size_t)ap.wgs > attn_part_slots(M)) return hipErrorInvalidValue;  // cannot happen (see attn_plan)
  const bool small = M <= small_m(H);
  const AttnArgs at0{wk.qh, wk.ql, k_cache, v_cache, wk.ah, wk.al, small ? 2 : 1, M, 0, position, kv, wk.bad,
                     wk.apart, ap.chunk, attn_part_rows(M)};
  const dim3 attn_grid(ap.wgs);
  if (small) {
    // Short prompts: the products are weight-bandwidth bound, so they run on the skinny kernels (16
    // weight rows per workgroup, 256 to 384 workgroups), the O and down products split over K into
    // partials that the next norm adds to the residual in a fixed order.
    typedef BatchPlan<H, I> BP;
    const int cb = column_blocks(M);
    auto skinny = [&](int epi, dim3 grid, const SkArgs& a) { return launch_skinny(epi, cb, grid, a, st); };
    const dim3 rows(M), nthr(64);  // one row per single-wave workgroup: the rows spread over M CUs
    // norms into the products' skinny fragments (hi and lo in ah)
    auto norm = [&](const int32_t* tk, int S, const uint16_t* w) {
      hipLaunchKernelGGL((bnorm_kernel<H, 2>), rows, nthr, 0, st, wk.x, tk, embed, dims.vocab, wk.bad, wk.part, S,
                         w, wk.ah, nullptr, 0, M);
      return hipGetLastError();
    };
    for (int l = 0; l < dims.num_layers; ++l) {
      const mk_layer_weights& lw = layers[l];
      if ((e = norm(l == 0 ? tokens : nullptr, l == 0 ? 0 : BP::SD, (const uint16_t*)lw.norm_weight)) != hipSuccess)
        return e;
      SkArgs q{};
      q.xh = wk.ah; q.B = M; q.N = (HQ + 2 * HKV) * D; q.K = H;
      q.w0 = (const uint16_t*)lw.q_weight; q.w1 = (const uint16_t*)lw.k_weight; q.w2 = (const uint16_t*)lw.v_weight;
      q.n1 = HQ * D; q.n2 = (HQ + HKV) * D; q.out = wk.raw;
      if ((e = skinny(SK_RAW, dim3(q.N / 16, 1), q)) != hipSuccess) return e;
      MKP_LAUNCH(qkv_post_kernel, dim3((M * (HQ + 2 * HKV) + 3) / 4), dim3(64), 0, st, wk.raw, 1, M, position,
                 (const uint16_t*)lw.q_norm_weight, (const uint16_t*)lw.k_norm_weight, cos_tab, sin_tab, wk.qh, wk.ql,
                 k_cache, v_cache, l, kv, wk.bad);
      AttnArgs at = at0;
      at.layer = l;
      MKP_LAUNCH(attn_kernel, attn_grid, dim3(512), 0, st, at);
      if (ap.merge) MKP_LAUNCH(attn_merge_kernel, dim3(ap.merge), dim3(256), 0, st, at);
      SkArgs o{};
      o.xh = wk.ah; o.B = M; o.N = H; o.K = HQ * D;
      o.w0 = (const uint16_t*)lw.o_proj_weight; o.out = wk.part;
      if ((e = skinny(SK_PART, dim3(H / 16, BP::SO), o)) != hipSuccess) return e;
      if ((e = norm(nullptr, BP::SO, (const uint16_t*)lw.post_attn_norm_weight)) != hipSuccess) return e;
      SkArgs u{};
      u.xh = wk.ah; u.B = M; u.N = I; u.K = H;
      u.w0 = (const uint16_t*)lw.gate_proj_weight; u.w1 = (const uint16_t*)lw.up_proj_weight;
      u.mh = wk.bh; u.ldm = I;
      if ((e = skinny(SK_SILU, dim3(I / 8, 1), u)) != hipSuccess) return e;
      SkArgs dn{};
      dn.xh = wk.bh; dn.B = M; dn.N = H; dn.K = I;
      dn.w0 = (const uint16_t*)lw.down_proj_weight; dn.out = wk.part;
      if ((e = skinny(SK_PART, dim3(H / 16, BP::SD), dn)) != hipSuccess) return e;
    }
    // the last layer's down partials into the residual (no norm: the LM head normalises its row)
    MKP_LAUNCH(bnorm_kernel<H>, rows, nthr, 0, st, wk.x, nullptr, embed, dims.vocab, wk.bad, wk.part, BP::SD,
               nullptr, nullptr, nullptr, A, M);
  }
  // Longer prompts: 128 x 128 tiles with the epilogues fused; the residual products split over K
  // into partials when their tile grid is small (the norm after them adds the partials).
  const int so = resid_splits(H, M, HQ * D), sd = resid_splits(H, M, I);
  const int sq = qkv_splits(H, M), su = silu_splits(H, I, M);
  for (int l = 0; !small && l < dims.num_layers; ++l) {
    const mk_layer_weights& lw = layers[l];
    // one row per wave; workgroups of fewer waves on short prompts keep every CU busy. Measured on
    // MI355X (ms per prefill, 4 waves -> this choice): 0.6B 100 tokens 1.97 -> 1.91 (1 wave), 512
    // 2.87 -> 2.88 with 2 waves (so 4 there); 1.7B 64 2.77 -> 2.45, 300 4.35 -> 4.22 (1 wave), 512
    // 4.83 -> 4.72 (2 waves); from 1,024 tokens on no difference
    const int nw = M >= 1024 || (H <= 1024 && M >= 512) ? 4 : M >= 512 ? 2 : 1;
    const dim3 rows((M + nw - 1) / nw), nthr(64 * nw);
    MKP_LAUNCH((bnorm_kernel<H, 1>), rows, nthr, 0, st, wk.x, l == 0 ? tokens : nullptr, embed, dims.vocab,
               wk.bad, wk.part, l > 0 && sd > 1 ? sd : 0, (const uint16_t*)lw.norm_weight, wk.ah, wk.al, A, M);
    GemmArgs g{};
    g.ah = wk.ah; g.al = wk.al; g.M = M; g.K = H;
    g.w0 = (const uint16_t*)lw.q_weight; g.w1 = (const uint16_t*)lw.k_weight; g.w2 = (const uint16_t*)lw.v_weight;
    g.N = (HQ + 2 * HKV) * D;
    g.q_norm = (const uint16_t*)lw.q_norm_weight; g.k_norm = (const uint16_t*)lw.k_norm_weight;
    g.cos_tab = cos_tab; g.sin_tab = sin_tab; g.qh = wk.qh; g.ql = wk.ql; g.k_cache = k_cache; g.v_cache = v_cache;
    g.layer = l; g.position = position; g.kv = kv; g.bad = wk.bad;
    if (sq > 1) {
      GemmArgs gq = g;
      gq.part = wk.qpart;
      if ((e = launch_gemm<EPI_QKV_PART>(dim3(g.N / NT, mtiles, sq), gq, st)) != hipSuccess) return e;
      MKP_LAUNCH(qkv_post_kernel, dim3((M * (HQ + 2 * HKV) + 3) / 4), dim3(64), 0, st, wk.qpart, sq, M, position,
                 (const uint16_t*)lw.q_norm_weight, (const uint16_t*)lw.k_norm_weight, cos_tab, sin_tab, wk.qh, wk.ql,
                 k_cache, v_cache, l, kv, wk.bad);
    } else if ((e = launch_gemm<EPI_QKV>(dim3(g.N / NT, mtiles), g, st)) != hipSuccess) {
      return e;
    }
    AttnArgs at = at0;
    at.layer = l;
    MKP_LAUNCH(attn_kernel, attn_grid, dim3(512), 0, st, at);
    if (ap.merge) MKP_LAUNCH(attn_merge_kernel, dim3(ap.merge), dim3(256), 0, st, at);
    GemmArgs go{};
    go.ah = wk.ah; go.al = wk.al; go.M = M; go.N = H; go.K = HQ * D;
    go.w0 = (const uint16_t*)lw.o_proj_weight; go.x = wk.x; go.ldx = H; go.part = so > 1 ? wk.part : nullptr;
    if ((e = launch_gemm<EPI_RESID>(dim3(H / NT, mtiles, so), go, st)) != hipSuccess) return e;
    MKP_LAUNCH((bnorm_kernel<H, 1>), rows, nthr, 0, st, wk.x, nullptr, embed, dims.vocab, wk.bad, wk.part,
               so > 1 ? so : 0, (const uint16_t*)lw.post_attn_norm_weight, wk.ah, wk.al, A, M);
    GemmArgs gu{};
    gu.ah = wk.ah; gu.al = wk.al; gu.M = M; gu.N = 2 * I; gu.K = H;
    gu.w0 = (const uint16_t*)lw.gate_proj_weight; gu.w1 = (const uint16_t*)lw.up_proj_weight;
    gu.bh = wk.bh; gu.bl = wk.bl;
    if (su > 1) {
      GemmArgs gp = gu;
      gp.part = wk.qpart;
      if ((e = launch_gemm<EPI_SILU_PART>(dim3(I / (NT / 2), mtiles, su), gp, st)) != hipSuccess) return e;
      MKP_LAUNCH(silu_post_kernel, dim3((M * (I / 8) + 63) / 64), dim3(64), 0, st, wk.qpart, su, M, I, wk.bh, wk.bl);
    } else if ((e = launch_gemm<EPI_SILU>(dim3(I / (NT / 2), mtiles), gu, st)) != hipSuccess) {
      return e;
    }
    GemmArgs gd{};
    gd.ah = wk.bh; gd.al = wk.bl; gd.M = M; gd.N = H; gd.K = I;
    gd.w0 = (const uint16_t*)lw.down_proj_weight; gd.x = wk.x; gd.ldx = H; gd.part = sd > 1 ? wk.part : nullptr;
    if ((e = launch_gemm<EPI_RESID>(dim3(H / NT, mtiles, sd), gd, st)) != hipSuccess) return e;
  }
  if (!small && sd > 1)  // the last layer's down partials into the residual
    MKP_LAUNCH(bnorm_kernel<H>, dim3((M + 3) / 4), dim3(256), 0, st, wk.x, nullptr, embed, dims.vocab, wk.bad, wk.part,
               sd, nullptr, nullptr, nullptr, A, M);
  // the last row's logits and greedy token
  MKP_LAUNCH(lm_head_kernel<H>, dim3(256), dim3(512), 0, st, wk.x, M - 1, final_norm, lm_head, dims.vocab, logits,
             wk.keys, wk.bad);
  if (out_token) MKP_LAUNCH(keys_to_tokens_kernel, dim3(1), dim3(64), 0, st, wk.keys, 1, wk.bad, out_token);
#undef MKP_LAUNCH
  return hipSuccess;
}

}  // namespace mkp

using namespace mkp;

extern "C" size_t mk_prefill_workspace_bytes(const mk_model_dims* dims, int num_tokens) {
  if (!dims || num_tokens < 1) return 0;
  return layout(dims->hidden, dims->intermediate, num_tokens).bytes;
}

static hipError_t prefill_impl(const mk_model_dims* dims, const int32_t* tokens, int num_tokens, int position,
                               const void* embed_weight, const void* lm_head_weight, const void* final_norm_weight,
                               const void* layer_weights, const void* cos_table, const void* sin_table,
                               void* k_cache, void* v_cache, const KvMap& kv, int max_seq_len, float* logits,
                               int32_t* out_token, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (!dims || !tokens || !embed_weight || !lm_head_weight || !final_norm_weight || !layer_weights ||
      !cos_table || !sin_table || !k_cache || !v_cache || !logits || !workspace)
    return hipErrorInvalidValue;
  const bool s06 = dims->hidden == 1024 && dims->intermediate == 3072;
  const bool s17 = dims->hidden == 2048 && dims->intermediate == 6144;
  if (!(s06 || s17) || dims->num_layers < 1 || dims->vocab < 1) return hipErrorInvalidValue;
  if (num_tokens < 1 || position < 0 || max_seq_len < 1 || (long long)position + num_tokens > max_seq_len)
    return hipErrorInvalidValue;
  const Layout L = layout(dims->hidden, dims->intermediate, num_tokens);
  if (workspace_bytes < L.bytes) return hipErrorInvalidValue;
  const Work wk = carve(workspace, L);
  if (reinterpret_cast<uintptr_t>(workspace) % 256 != 0) return hipErrorInvalidValue;
  const mk_layer_weights* lw = static_cast<const mk_layer_weights*>(layer_weights);  // host array
  if (s06)
    return run<1024, 3072>(*dims, tokens, num_tokens, position, (const uint16_t*)embed_weight,
                           (const uint16_t*)lm_head_weight, (const uint16_t*)final_norm_weight, lw,
                           (const uint16_t*)cos_table, (const uint16_t*)sin_table, (uint16_t*)k_cache,
                           (uint16_t*)v_cache, kv, logits, out_token, wk, stream);
  return run<2048, 6144>(*dims, tokens, num_tokens, position, (const uint16_t*)embed_weight,
                         (const uint16_t*)lm_head_weight, (const uint16_t*)final_norm_weight, lw,
                         (const uint16_t*)cos_table, (const uint16_t*)sin_table, (uint16_t*)k_cache,
                         (uint16_t*)v_cache, kv, logits, out_token, wk, stream);
}

extern "C" hipError_t mk_prefill(const mk_model_dims* dims, const int32_t* tokens, int num_tokens, int position,
                                 const void* embed_weight, const void* lm_head_weight, const void* final_norm_weight,
                                 const void* layer_weights, const void* cos_table, const void* sin_table,
                                 void* k_cache, void* v_cache, int max_seq_len, float* logits, int32_t* out_token,
                                 void* workspace, size_t workspace_bytes, hipStream_t stream) {
  const KvMap kv{nullptr, 0, 0, max_seq_len};
  return prefill_impl(dims, tokens, num_tokens, position, embed_weight, lm_head_weight, final_norm_weight,
                      layer_weights, cos_table, sin_table, k_cache, v_cache, kv, max_seq_len, logits, out_token,
                      workspace, workspace_bytes, stream);
}

extern "C" hipError_t mk_prefill_paged(const mk_model_dims* dims, const int32_t* tokens, int num_tokens, int position,
                                       const void* embed_weight, const void* lm_head_weight,
                                       const void* final_norm_weight, const void* layer_weights,
                                       const void* cos_table, const void* sin_table, void* k_pages, void* v_pages,
                                       const int32_t* block_table, int num_pages, int page_size, int max_seq_len,
                                       float* logits, int32_t* out_token, void* workspace, size_t workspace_bytes,
                                       hipStream_t stream) {
  if (!block_table || num_pages < 1 || page_size < 1 || page_size > 4096 || (page_size & (page_size - 1)) != 0 ||
      max_seq_len < 1 || (max_seq_len + page_size - 1) / page_size > ATT_MAX_PAGES)
    return hipErrorInvalidValue;
  int shift = 0;
  while ((1 << shift) < page_size) ++shift;
  const KvMap kv{block_table, num_pages, shift, max_seq_len};
  return prefill_impl(dims, tokens, num_tokens, position, embed_weight, lm_head_weight, final_norm_weight,
                      layer_weights, cos_table, sin_table, k_pages, v_pages, kv, max_seq_len, logits, out_token,
                      workspace, workspace_bytes, stream);
}

// ------------------------------------------------------------------------------------------------
// Batched decode, host side
// ------------------------------------------------------------------------------------------------
namespace mkp {

// Split-K factors of the O and down products (each wave's K range a multiple of 256)

struct BLayout {
  size_t x, ah, al, af, bf, raw, part, apart, keys, bad, bytes;
};
static BLayout blayout(int H, int I, int B, int max_seq) {
  const size_t A = H > HQ * D ? H : HQ * D;
  const int S = (max_seq + KS - 1) / KS;
  BLayout L;
  size_t o = 0;
  auto take = [&](size_t n) { const size_t r = o; o += align256(n); return r; };
  L.x = take((size_t)B * H * 4);
  L.ah = take(frag_rows(B) * A * 2);  // whole row tiles for the LM head's gemm_kernel
  L.al = take(frag_rows(B) * A * 2);
  L.af = take(skf_elems(B, (int)A) * 2);  // skinny fragments: the QKV, O and gate/up inputs
  L.bf = take(skf_elems(B, I) * 2);       // ... and the down input
  L.raw = take((size_t)B * (HQ + 2 * HKV) * D * 4);
  L.part = take((size_t)3 * B * H * 4);
  L.apart = take((size_t)B * HKV * S * 2 * APW * 4);
  L.keys = take((size_t)B * 8);
  L.bad = take(4);
  L.bytes = o;
  return L;
}

template <int H, int I>
static hipError_t run_batch(const mk_model_dims& dims, int B, const int32_t* tokens, const int32_t* positions,
                            const uint16_t* embed, const uint16_t* lm_head, const uint16_t* final_norm,
                            const mk_layer_weights* layers, const uint16_t* cos_tab, const uint16_t* sin_tab,
                            uint16_t* k_cache, uint16_t* v_cache, int max_seq, float* logits, int32_t* out_tokens,
                            char* ws, const BLayout& Lo, hipStream_t st) {
  typedef BatchPlan<H, I> BP;
  const int A = H > HQ * D ? H : HQ * D;
  const int S = (max_seq + KS - 1) / KS;
  float* x = reinterpret_cast<float*>(ws + Lo.x);
  uint16_t* ah = reinterpret_cast<uint16_t*>(ws + Lo.ah);
  uint16_t* al = reinterpret_cast<uint16_t*>(ws + Lo.al);
  uint16_t* af = reinterpret_cast<uint16_t*>(ws + Lo.af);
  uint16_t* bf = reinterpret_cast<uint16_t*>(ws + Lo.bf);
  float* raw = reinterpret_cast<float*>(ws + Lo.raw);
  float* part = reinterpret_cast<float*>(ws + Lo.part);
  float* apart = reinterpret_cast<float*>(ws + Lo.apart);
  u64* keys = reinterpret_cast<u64*>(ws + Lo.keys);
  int32_t* bad = reinterpret_cast<int32_t*>(ws + Lo.bad);
  const int L = dims.num_layers;
  hipError_t e;
#define MKB_LAUNCH(...)                                   \
  do {                                                    \
    hipLaunchKernelGGL(__VA_ARGS__);                      \
    if ((e = hipGetLastError()) != hipSuccess) return e;  \
  } while (0)
  MKB_LAUNCH(keys_init_kernel, dim3(1), dim3(64), 0, st, keys, B, bad);
  const int cb = column_blocks(B);
  // attention workgroups per sequence and K/V head (each loops over its splits): about 1024 in all,
  // 16 at most (the grid cannot follow the device-side positions, so it must not be mostly idle)
  const int gx = B <= 8 ? 16 : B <= 16 ? 8 : B <= 32 ? 4 : 2;
  const dim3 rows(B), nthr(64);  // norms: one row per single-wave workgroup
  const int so = BP::SO, sd = BP::SD;
  for (int l = 0; l < L; ++l) {
    const mk_layer_weights& lw = layers[l];
    // x (embedding, or + the previous layer's down partials) -> input norm, as skinny fragments
    MKB_LAUNCH((bnorm_kernel<H, 2>), rows, nthr, 0, st, x, l == 0 ? tokens : nullptr, embed, dims.vocab, bad,
               part, l == 0 ? 0 : sd, (const uint16_t*)lw.norm_weight, af, nullptr, 0, B);
    SkArgs q{};
    q.xh = af; q.B = B; q.N = (HQ + 2 * HKV) * D; q.K = H;
    q.w0 = (const uint16_t*)lw.q_weight; q.w1 = (const uint16_t*)lw.k_weight; q.w2 = (const uint16_t*)lw.v_weight;
    q.n1 = HQ * D; q.n2 = (HQ + HKV) * D; q.out = raw;
    if ((e = launch_skinny(SK_RAW, cb, dim3(q.N / 16, 1), q, st)) != hipSuccess) return e;
    MKB_LAUNCH(battn_partial_kernel, dim3(S < gx ? S : gx, HKV, B), dim3(256), 0, st, raw, positions, tokens,
               dims.vocab, (const uint16_t*)lw.q_norm_weight, (const uint16_t*)lw.k_norm_weight, cos_tab, sin_tab, k_cache,
               v_cache, L, l, max_seq, apart, S, bad);
    MKB_LAUNCH(battn_merge_kernel, dim3(B, HQ), dim3(D), 0, st, apart, S, positions, max_seq, af, nullptr, 0);
    SkArgs o{};
    o.xh = af; o.B = B; o.N = H; o.K = HQ * D; o.w0 = (const uint16_t*)lw.o_proj_weight; o.out = part;
    if ((e = launch_skinny(SK_PART, cb, dim3(H / 16, so), o, st)) != hipSuccess) return e;
    MKB_LAUNCH((bnorm_kernel<H, 2>), rows, nthr, 0, st, x, nullptr, embed, dims.vocab, bad, part, so,
               (const uint16_t*)lw.post_attn_norm_weight, af, nullptr, 0, B);
    SkArgs u{};
    u.xh = af; u.B = B; u.N = I; u.K = H;
    u.w0 = (const uint16_t*)lw.gate_proj_weight; u.w1 = (const uint16_t*)lw.up_proj_weight; u.mh = bf; u.ldm = I;
    if ((e = launch_skinny(SK_SILU, cb, dim3(I / 8, 1), u, st)) != hipSuccess) return e;
    SkArgs dn{};
    dn.xh = bf; dn.B = B; dn.N = H; dn.K = I; dn.w0 = (const uint16_t*)lw.down_proj_weight;
    dn.out = part;
    if ((e = launch_skinny(SK_PART, cb, dim3(H / 16, sd), dn, st)) != hipSuccess) return e;
  }
  // the last layer's down partials and the final norm, then the tied LM head as one more skinny
  // product (vocabulary rows x the B normalised rows: each table byte read once, on the matrix
  // cores) and the greedy keys
  const bool lm_tiles = B > 8 && dims.vocab % NT == 0;
  if (lm_tiles)
    MKB_LAUNCH((bnorm_kernel<H, 1>), rows, nthr, 0, st, x, nullptr, embed, dims.vocab, bad, part, sd,
               final_norm, ah, al, A, B);
  else
    MKB_LAUNCH((bnorm_kernel<H, 2>), rows, nthr, 0, st, x, nullptr, embed, dims.vocab, bad, part, sd,
               final_norm, af, nullptr, 0, B);
  if (!lm_tiles) {
    SkArgs lmh{};
    lmh.xh = af; lmh.B = B; lmh.N = dims.vocab; lmh.K = H;
    lmh.w0 = lm_head; lmh.n1 = dims.vocab; lmh.n2 = dims.vocab; lmh.out = logits;
    if ((e = launch_skinny(SK_RAW, cb, dim3(dims.vocab / 16, 1), lmh, st)) != hipSuccess) return e;
  } else {
    // beyond one column block the skinny product re-reads every row's activations per 16 table
    // rows; a 128-row tile of the table reads them once per 128 (the B rows are one row tile)
    GemmArgs gl{};
    gl.ah = ah; gl.al = al; gl.M = B; gl.N = dims.vocab; gl.K = H;
    gl.w0 = lm_head; gl.part = logits;  // logits[b][v], no residual
    if ((e = launch_gemm<EPI_RESID>(dim3(dims.vocab / NT, 1, 1), gl, st)) != hipSuccess) return e;
  }
  MKB_LAUNCH(logits_argmax_kernel, dim3((dims.vocab + 4095) / 4096, B), dim3(256), 0, st, logits, dims.vocab, keys, bad);
  if (out_tokens) MKB_LAUNCH(keys_to_tokens_kernel, dim3(1), dim3(64), 0, st, keys, B, bad, out_tokens);
#undef MKB_LAUNCH
  return hipSuccess;
}

}  // namespace mkp

// The larger of the two engines' needs, so that the engine can be chosen per call.
extern "C" size_t mk_decode_batch_workspace_bytes(const mk_model_dims* dims, int batch, int max_seq_len) {
  if (!dims || batch < 1 || batch > BMAX || max_seq_len < 1) return 0;
  const size_t n = blayout(dims->hidden, dims->intermediate, batch, max_seq_len).bytes;
  const size_t p = mkb_workspace_bytes();
  return batch <= 2 * MKB_MAX && p > n ? p : n;
}

extern "C" hipError_t mk_decode_batch(const mk_model_dims* dims, int batch, const int32_t* tokens,
                                      const int32_t* positions, const void* embed_weight, const void* lm_head_weight,
                                      const void* final_norm_weight, const void* layer_weights, const void* cos_table,
                                      const void* sin_table, void* k_cache, void* v_cache, int max_seq_len,
                                      float* logits, int32_t* out_tokens, void* workspace, size_t workspace_bytes,
                                      hipStream_t stream) {
  if (!dims || !tokens || !positions || !embed_weight || !lm_head_weight || !final_norm_weight || !layer_weights ||
      !cos_table || !sin_table || !k_cache || !v_cache || !logits || !workspace)
    return hipErrorInvalidValue;
  const bool s06 = dims->hidden == 1024 && dims->intermediate == 3072;
  const bool s17 = dims->hidden == 2048 && dims->intermediate == 6144;
  if (!(s06 || s17) || dims->num_layers < 1 || dims->vocab < 1) return hipErrorInvalidValue;
  if (batch < 1 || batch > BMAX || max_seq_len < 1) return hipErrorInvalidValue;
  if (dims->vocab % 16 != 0) return hipErrorInvalidValue;  // the LM head's skinny product takes 16 rows per workgroup
  const BLayout Lo = blayout(dims->hidden, dims->intermediate, batch, max_seq_len);
  if (workspace_bytes < Lo.bytes || reinterpret_cast<uintptr_t>(workspace) % 256 != 0) return hipErrorInvalidValue;
  const mk_layer_weights* lw = static_cast<const mk_layer_weights*>(layer_weights);  // host array
  if (mkb_applies(dims, batch, max_seq_len)) {
    if (workspace_bytes < mkb_workspace_bytes()) return hipErrorInvalidValue;
    return mkb_decode_batch(dims, batch, tokens, positions, embed_weight, lm_head_weight, final_norm_weight, lw,
                            cos_table, sin_table, k_cache, v_cache, max_seq_len, logits, out_tokens, workspace,
                            stream);
  }
  // 17-24 sequences (17-32 with the persistent engine forced) where the persistent kernel applies
  // to their parts: two persistent launches, MKB_MAX sequences and the rest, one after the other on
  // the stream (each sequence's cache, token, position, logits and greedy token are its own slices,
  // so the parts are independent calls). Measured on MI355X (0.6B, ms per step, two launches /
  // layer by layer), context 256: 17 1.41 / 1.48, 20 1.45 / 1.50, 24 1.49 / 1.52, 28 1.65 / 1.58,
  // 32 1.70 / 1.61; context 1,500: 24 2.10 / 2.19, 28 2.34 / 2.37, 32 2.48 / 2.47.
  const int two_max = mkb_engine() == 2 ? 2 * MKB_MAX : MKB_MAX + 8;
  if (batch > MKB_MAX && batch <= two_max && mkb_applies(dims, MKB_MAX, max_seq_len) &&
      mkb_applies(dims, batch - MKB_MAX, max_seq_len)) {
    if (workspace_bytes < mkb_workspace_bytes()) return hipErrorInvalidValue;
    const size_t seq_cache = (size_t)dims->num_layers * HKV * max_seq_len * D;  // elements per sequence
    for (int b0 = 0; b0 < batch; b0 += MKB_MAX) {
      const int nb = batch - b0 < MKB_MAX ? batch - b0 : MKB_MAX;
      const hipError_t e = mkb_decode_batch(
          dims, nb, tokens + b0, positions + b0, embed_weight, lm_head_weight, final_norm_weight, lw, cos_table,
          sin_table, static_cast<uint16_t*>(k_cache) + b0 * seq_cache, static_cast<uint16_t*>(v_cache) + b0 * seq_cache,
          max_seq_len, logits + (size_t)b0 * dims->vocab, out_tokens ? out_tokens + b0 : nullptr, workspace, stream);
      if (e != hipSuccess) return e;
    }
    return hipSuccess;
  }
  char* ws = static_cast<char*>(workspace);
  if (s06)
    return run_batch<1024, 3072>(*dims, batch, tokens, positions, (const uint16_t*)embed_weight,
                                 (const uint16_t*)lm_head_weight, (const uint16_t*)final_norm_weight, lw,
                                 (const uint16_t*)cos_table, (const uint16_t*)sin_table, (uint16_t*)k_cache,
                                 (uint16_t*)v_cache, max_seq_len, logits, out_tokens, ws, Lo, stream);
  return run_batch<2048, 6144>(*dims, batch, tokens, positions, (const uint16_t*)embed_weight,
                               (const uint16_t*)lm_head_weight, (const uint16_t*)final_norm_weight, lw,
                               (const uint16_t*)cos_table, (const uint16_t*)sin_table, (uint16_t*)k_cache,
                               (uint16_t*)v_cache, max_seq_len, logits, out_tokens, ws, Lo, stream);
}
