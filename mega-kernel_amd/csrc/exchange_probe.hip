// Exchange-latency probe for MI355X: the floors that bound the decode kernel's per-layer chain.
//
// Every measurement here is a bounded spin (a wait gives up after SPIN polls and the run reports a
// failure instead of hanging), every buffer index is checked against its allocation in the
// comments, and every workgroup takes 96 KB of LDS so that no two share a CU.
//
//   exchange_probe pair        1-to-1 ping-pong, one-way latency: same XCD (plain store, device-
//                              scope poll) and across XCDs (device-scope store and poll).
//   exchange_probe allgather   32 -> 32 all-gather inside each XCD (4 KB poll per reader) and
//                              8 -> 8 across XCDs (1 KB poll), the decode kernel's two hop shapes.
//   exchange_probe queue       same-XCD ping-pong while 1, 2, 4 or 8 waves of EVERY CU stream HBM
//                              (8 KB in flight per wave), while every CU but the pair's streams,
//                              and while only the pair's CUs stream.
//   exchange_probe split       per XCD, NS workgroups stream HBM while the others read an
//                              L2-resident 1 MiB region and the pair ping-pongs among them.
//   exchange_probe mall        200 MiB read twice in a row, and again after a 1 GiB read in between:
//                              whether the memory-side cache serves a re-read faster than HBM.
//
// Timestamps are s_memrealtime (100 MHz). Build: hipcc -O3 --offload-arch=gfx950 (megakernel.build).
#include <hip/hip_runtime.h>
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#define CHECK(x)                                                                          \
  do {                                                                                    \
    hipError_t e_ = (x);                                                                  \
    if (e_ != hipSuccess) {                                                               \
      fprintf(stderr, "exchange_probe: %s at line %d\n", hipGetErrorString(e_), __LINE__); \
      exit(1);                                                                            \
    }                                                                                     \
  } while (0)

namespace {

typedef unsigned u4v __attribute__((ext_vector_type(4)));
constexpr int NWG = 256;                  // one workgroup per CU (LDS_PAD forces it)
constexpr int LDS_PAD = 96 * 1024;        // dynamic LDS per workgroup: two cannot share a CU
constexpr int ROUNDS = 1000;              // ping-pong round trips / all-gather rounds
constexpr unsigned SPIN = 1u << 22;       // polls before a wait gives up
constexpr int CPOL_SC1 = 16;              // device-scope cache policy
constexpr int SLOT_WORDS = 64;            // 256-byte slot per writer
constexpr size_t OUT_N = 8192;            // u64 result words (readers: 48 + 3 * 2304 < 8191)

__device__ __forceinline__ unsigned long long now() { return wall_clock64(); }
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, 0x7fffffff, 0x00020000);
}
// One device-scope 4-byte load (the compiler barrier keeps it inside the spin loop).
__device__ __forceinline__ unsigned poll_word(__amdgpu_buffer_rsrc_t rs, int byte_off) {
  asm volatile("" ::: "memory");
  return __builtin_amdgcn_raw_buffer_load_b32(rs, byte_off, 0, CPOL_SC1);
}
template <bool CROSS>
__device__ __forceinline__ void put_word(__amdgpu_buffer_rsrc_t rs, int byte_off, unsigned v) {
  __builtin_amdgcn_raw_buffer_store_b32(v, rs, byte_off, 0, CROSS ? CPOL_SC1 : 0);
}

// Ping-pong between workgroups `a` (starts) and `b`; flags: slot per workgroup (NWG slots).
// out[3 * k + {0,1,2}] = start, end, failed for participant index k.
template <bool CROSS>
__device__ void ping_pong(unsigned* flags, int me, int partner, bool starter, int k, unsigned long long* out,
                          unsigned long long delay) {
  const int lane = threadIdx.x & 63;
  const __amdgpu_buffer_rsrc_t rs = rsrc(flags);
  const int mo = me * SLOT_WORDS * 4, po = partner * SLOT_WORDS * 4;  // < NWG * 256 bytes
  const unsigned long long t0 = now();
  while (now() - t0 < delay) {}
  unsigned fail = 0;
  const unsigned long long ta = now();
  for (int i = 1; i <= ROUNDS && !fail; ++i) {
    if (starter && lane == 0) put_word<CROSS>(rs, mo, (unsigned)i);
    for (unsigned it = 0;; ++it) {
      if (poll_word(rs, po) == (unsigned)i) break;
      if (it > SPIN) { fail = 1; break; }
    }
    if (!starter && lane == 0) put_word<CROSS>(rs, mo, (unsigned)i);
  }
  if (lane == 0) { out[3 * k] = ta; out[3 * k + 1] = now(); out[3 * k + 2] = fail; }
}

// pair: participants 0..15 local (b, b + 8 for b < 8), 16..23 cross (b, b ^ 1 for b < 8) -- run as
// two launches (mode 0 local, mode 1 cross).
__global__ __launch_bounds__(64) void k_pair(unsigned* flags, int cross, unsigned long long* out) {
  const int b = blockIdx.x;
  if (!cross) {
    if (b >= 16) return;
    ping_pong<false>(flags, b, b < 8 ? b + 8 : b - 8, b < 8, b, out, 0);
  } else {
    if (b >= 8) return;
    ping_pong<true>(flags, b, b ^ 1, (b & 1) == 0, b, out, 0);
  }
}

// allgather: local -> the 32 workgroups of each XCD (b % 8 == x) each write a 128-byte block and
// poll all 32 blocks of their XCD (4 KB: lane l reads 64 bytes of block l / 2); cross -> the 8
// workgroups b = 8 j + x (x = 0..7) of each j write their block through and poll the 8 blocks (1 KB:
// lane l reads 16 bytes of block l / 8). A block holds the round number in every word; readers wait
// for >= round (a fast writer may already be one round ahead). data: NWG blocks of 128 bytes.
template <bool CROSS>
__global__ __launch_bounds__(64) void k_allgather(unsigned* data, unsigned long long* out) {
  const int b = blockIdx.x, lane = threadIdx.x, x = b % 8, j = b / 8;
  const __amdgpu_buffer_rsrc_t rs = rsrc(data);
  unsigned fail = 0;
  const unsigned long long ta = now();
  for (int r = 1; r <= ROUNDS && !fail; ++r) {
    // own block: 32 words, lanes 0..31 one word each (b * 128 + lane * 4 < NWG * 128)
    if (lane < 32) put_word<CROSS>(rs, b * 128 + lane * 4, (unsigned)r);
    int off;
    if (!CROSS) off = ((lane >> 1) * 8 + x) * 128 + (lane & 1) * 64;  // block of workgroup 8 (l/2) + x
    else off = (8 * j + (lane >> 3)) * 128 + (lane & 7) * 16;          // block of workgroup 8 j + l/8
    for (unsigned it = 0;; ++it) {
      asm volatile("" ::: "memory");
      const u4v v = __builtin_bit_cast(u4v, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, CPOL_SC1));
      unsigned bad = 0;
      for (int i = 0; i < 4; ++i) bad |= v[i] < (unsigned)r ? 1u : 0u;
      if (!CROSS) {  // the 4 KB poll: 4 loads per lane cover 64 bytes
        for (int q = 1; q < 4; ++q) {
          const u4v w = __builtin_bit_cast(u4v, __builtin_amdgcn_raw_buffer_load_b128(rs, off + 16 * q, 0, CPOL_SC1));
          for (int i = 0; i < 4; ++i) bad |= w[i] < (unsigned)r ? 1u : 0u;
        }
      }
      if (__ballot(bad != 0) == 0) break;
      if (it > SPIN) { fail = 1; break; }
    }
  }
  if (lane == 0) { out[3 * b] = ta; out[3 * b + 1] = now(); out[3 * b + 2] = fail; }
}

// queue / split: wave 0 of workgroups 0..15 ping-pongs (b, b + 8) after a 200 us delay; the other
// waves stream or read. stream_mode: 0 none, 1 every CU, 2 every CU but the pair's, 3 only the
// pair's. nsw streaming waves per CU (1..8), 8 KB in flight per wave (8 x 16 B per lane). ns > 0:
// workgroups j >= 32 - ns of each XCD stream (all 9 waves) and the others read this XCD's 1 MiB of
// l2buf (depth KB per wave in flight). Streams stop when their XCD's pair is done (or after MAXIT).
constexpr int MAXIT = 200000;
__global__ __launch_bounds__(576) void k_queue(unsigned* flags, const u4v* hbm, size_t hchunks, const u4v* l2buf,
                                               int stream_mode, int nsw, int ns, int depth, unsigned long long* out) {
  const int b = blockIdx.x, w = threadIdx.x >> 6, lane = threadIdx.x & 63, x = b % 8, j = b / 8;
  unsigned* done = flags + NWG * SLOT_WORDS;  // 8 slots after the NWG ping-pong slots
  const bool pair = j < 2;
  const bool streamer = ns > 0 && j >= 32 - ns;
  if (w == 0 && pair && !streamer) {
    ping_pong<false>(flags, b, j == 0 ? b + 8 : b - 8, j == 0, b, out, 20000);
    if (j == 0 && lane == 0) __hip_atomic_store(done + x * SLOT_WORDS, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  bool hbm_reader = false, l2_reader = false;
  if (ns > 0) {
    hbm_reader = streamer;
    l2_reader = !streamer && w >= 1;
  } else if (w >= 1 && w <= nsw) {
    hbm_reader = stream_mode == 1 || (stream_mode == 2 && !pair) || (stream_mode == 3 && pair);
  }
  if (!hbm_reader && !l2_reader) return;
  u4v acc = {0, 0, 0, 0};
  unsigned long long bytes = 0;
  const unsigned long long s0 = now();
  const int g = b * 9 + w;  // reader id < NWG * 9
  for (int it = 0; it < MAXIT; ++it) {
    if ((it & 15) == 0 && __hip_atomic_load(done + x * SLOT_WORDS, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) break;
    u4v r[8];
    if (hbm_reader) {  // chunk c < hchunks of 8 KB: index c * 512 + lane + 448 < hchunks * 512
      const size_t c = ((size_t)it * NWG * 9 + g) % hchunks;
      const u4v* p = hbm + c * 512 + lane;
#pragma unroll
      for (int k = 0; k < 8; ++k) r[k] = __builtin_nontemporal_load(p + k * 64);
#pragma unroll
      for (int k = 0; k < 8; ++k) acc ^= r[k];
      bytes += 8192;
    } else {  // XCD x's 1 MiB = 128 chunks: index x * 65536 + c * 512 + lane + 448 < 8 * 65536
      const size_t c = ((size_t)it * 256 + j * 8 + w) % 128;
      const u4v* p = l2buf + (size_t)x * 65536 + c * 512 + lane;
#pragma unroll
      for (int k = 0; k < 8; ++k) if (k < depth) r[k] = p[k * 64];
#pragma unroll
      for (int k = 0; k < 8; ++k) if (k < depth) acc ^= r[k];
      bytes += 1024 * (size_t)depth;
    }
  }
  const unsigned long long s1 = now();
  if ((acc[0] ^ acc[1] ^ acc[2] ^ acc[3]) == 0x9e3779b9u) out[OUT_N - 1] = 1;  // keeps the loads
  if (lane == 0) {  // 48 + 3 g + 2 < 48 + 3 * 2304 < OUT_N
    out[48 + 3 * g] = s0; out[48 + 3 * g + 1] = s1; out[48 + 3 * g + 2] = bytes | (hbm_reader ? 1ull << 62 : 0);
  }
}

template <int CPOL>
__global__ __launch_bounds__(512) void k_read(const u4v* buf, size_t n16, unsigned* sink) {
  u4v acc = {0, 0, 0, 0};
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < n16; e += stride) {
    // 1 GiB windows keep the 32-bit buffer offset in range
    const __amdgpu_buffer_rsrc_t r = rsrc(buf + (e & ~(((size_t)1 << 26) - 1)));
    acc ^= __builtin_bit_cast(u4v, __builtin_amdgcn_raw_buffer_load_b128(r, (int)((e & ((1 << 26) - 1)) * 16), 0, CPOL));
  }
  if ((acc[0] ^ acc[1] ^ acc[2] ^ acc[3]) == 0x9e3779b9u) sink[threadIdx.x] = 1;
}

struct Dev {
  unsigned* flags;
  unsigned long long* out;
  std::vector<unsigned long long> h;
  Dev() : h(OUT_N) {
    CHECK(hipMalloc(&flags, (NWG + 8) * SLOT_WORDS * 4));
    CHECK(hipMalloc(&out, OUT_N * 8));
  }
  void reset() {
    CHECK(hipMemset(flags, 0, (NWG + 8) * SLOT_WORDS * 4));
    CHECK(hipMemset(out, 0, OUT_N * 8));
  }
  void fetch() {
    CHECK(hipDeviceSynchronize());
    CHECK(hipMemcpy(h.data(), out, OUT_N * 8, hipMemcpyDeviceToHost));
  }
  // mean of (end - start) over participants [k0, k1), in microseconds, and the failure count
  double span_us(int k0, int k1, int* fails) const {
    double s = 0;
    *fails = 0;
    for (int k = k0; k < k1; ++k) { s += (double)(h[3 * k + 1] - h[3 * k]) * 0.01; *fails += (int)h[3 * k + 2]; }
    return s / (k1 - k0);
  }
};

void run_pair(Dev& d) {
  for (int cross = 0; cross < 2; ++cross) {
    d.reset();
    hipLaunchKernelGGL(k_pair, dim3(NWG), dim3(64), LDS_PAD, 0, d.flags, cross, d.out);
    CHECK(hipGetLastError());
    d.fetch();
    int f;
    const double us = d.span_us(0, cross ? 8 : 16, &f);
    printf("pair %-9s one-way %.3f us  (%d round trips, failures %d)\n", cross ? "cross-XCD" : "same-XCD", us / (2.0 * ROUNDS),
           ROUNDS, f);
  }
}

void run_allgather(Dev& d) {
  unsigned* data;
  CHECK(hipMalloc(&data, NWG * 128));
  for (int cross = 0; cross < 2; ++cross) {
    CHECK(hipMemset(data, 0, NWG * 128));
    d.reset();
    if (cross) hipLaunchKernelGGL(k_allgather<true>, dim3(NWG), dim3(64), LDS_PAD, 0, data, d.out);
    else hipLaunchKernelGGL(k_allgather<false>, dim3(NWG), dim3(64), LDS_PAD, 0, data, d.out);
    CHECK(hipGetLastError());
    d.fetch();
    int f;
    const double us = d.span_us(0, NWG, &f);
    printf("allgather %-38s %.3f us per round  (%d rounds, failures %d)\n",
           cross ? "8 -> 8 across XCDs, 1 KB poll:" : "32 -> 32 inside an XCD, 4 KB poll:", us / ROUNDS, ROUNDS, f);
  }
  CHECK(hipFree(data));
}

void run_queue(Dev& d, bool split) {
  const size_t HB = (size_t)1 << 30, L2B = (size_t)8 << 20;
  u4v *hbm, *l2;
  CHECK(hipMalloc(&hbm, HB)); CHECK(hipMemset(hbm, 1, HB));
  CHECK(hipMalloc(&l2, L2B)); CHECK(hipMemset(l2, 3, L2B));
  struct Cfg { int mode, nsw, ns, depth; const char* what; };
  std::vector<Cfg> cfgs;
  if (!split) {
    cfgs = {{0, 0, 0, 0, "idle"},
            {1, 1, 0, 0, "every CU streams, 1 wave (8 KB in flight)"},
            {1, 2, 0, 0, "every CU streams, 2 waves (16 KB)"},
            {1, 4, 0, 0, "every CU streams, 4 waves (32 KB)"},
            {1, 8, 0, 0, "every CU streams, 8 waves (64 KB)"},
            {2, 8, 0, 0, "every CU but the pair's streams, 8 waves"},
            {3, 8, 0, 0, "only the pair's CUs stream, 8 waves"}};
  } else {
    cfgs = {{0, 0, 8, 2, "8 streamers/XCD, readers 2 KB/wave"},
            {0, 0, 8, 4, "8 streamers/XCD, readers 4 KB/wave"},
            {0, 0, 8, 8, "8 streamers/XCD, readers 8 KB/wave"},
            {0, 0, 16, 4, "16 streamers/XCD, readers 4 KB/wave"}};
  }
  for (const Cfg& c : cfgs) {
    d.reset();
    hipLaunchKernelGGL(k_queue, dim3(NWG), dim3(576), LDS_PAD, 0, d.flags, hbm, HB / 8192, l2, c.mode, c.nsw, c.ns, c.depth,
                       d.out);
    CHECK(hipGetLastError());
    d.fetch();
    int f;
    const double us = d.span_us(0, 16, &f);
    double hb = 0, lb = 0;
    unsigned long long h0 = ~0ull, h1 = 0, l0 = ~0ull, l1 = 0;
    int nl = 0;
    for (int g = 0; g < NWG * 9; ++g) {
      const unsigned long long* e = &d.h[48 + 3 * g];
      const unsigned long long by = e[2] & ((1ull << 62) - 1);
      if (!by) continue;
      if (e[2] >> 62) { hb += by; h0 = std::min(h0, e[0]); h1 = std::max(h1, e[1]); }
      else { lb += by; l0 = std::min(l0, e[0]); l1 = std::max(l1, e[1]); ++nl; }
    }
    printf("%-46s hop %.3f us (failures %d) | HBM %5.0f GB/s", c.what, us / (2.0 * ROUNDS), f,
           h1 > h0 ? hb / ((h1 - h0) * 1e-8) / 1e9 : 0.0);
    if (split) printf(" | L2 readers %5.1f GB/s per CU", l1 > l0 ? lb / ((l1 - l0) * 1e-8) / 1e9 / (nl / 8.0) : 0.0);
    printf("\n");
  }
  CHECK(hipFree(hbm)); CHECK(hipFree(l2));
}

void run_mall() {
  const size_t BA = (size_t)200 << 20, BB = (size_t)1 << 30;
  u4v *A, *B;
  unsigned* sink;
  CHECK(hipMalloc(&A, BA)); CHECK(hipMalloc(&B, BB)); CHECK(hipMalloc(&sink, 4096));
  CHECK(hipMemset(A, 1, BA)); CHECK(hipMemset(B, 2, BB));
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0)); CHECK(hipEventCreate(&e1));
  auto timed = [&](const u4v* p, size_t bytes, bool nt) {
    CHECK(hipEventRecord(e0));
    if (nt) hipLaunchKernelGGL(k_read<2>, dim3(1024), dim3(512), 0, 0, p, bytes / 16, sink);
    else hipLaunchKernelGGL(k_read<0>, dim3(1024), dim3(512), 0, 0, p, bytes / 16, sink);
    CHECK(hipGetLastError());
    CHECK(hipEventRecord(e1)); CHECK(hipEventSynchronize(e1));
    float ms;
    CHECK(hipEventElapsedTime(&ms, e0, e1));
    return bytes / (ms * 1e-3) / 1e9;
  };
  for (int i = 0; i < 3; ++i) timed(B, BB, false);
  printf("mall: 1 GiB read %.0f GB/s (plain), %.0f GB/s (nt)\n", timed(B, BB, false), timed(B, BB, true));
  const double a1 = timed(A, BA, false), a2 = timed(A, BA, false);
  printf("mall: 200 MiB read twice in a row: %.0f then %.0f GB/s\n", a1, a2);
  timed(B, BB, false);
  printf("mall: 200 MiB again after a 1 GiB nt read: %.0f GB/s\n", (timed(A, BA, false), timed(B, BB, true), timed(A, BA, false)));
  CHECK(hipFree(A)); CHECK(hipFree(B)); CHECK(hipFree(sink));
}

}  // namespace

int main(int argc, char** argv) {
  if (argc != 2) {
    fprintf(stderr, "usage: exchange_probe pair|allgather|queue|split|mall\n");
    return 2;
  }
  int dev = 0, ncu = 0;
  CHECK(hipGetDevice(&dev));
  CHECK(hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev));
  if (ncu != NWG) {
    fprintf(stderr, "exchange_probe: expects %d CUs (MI355X), found %d\n", NWG, ncu);
    return 2;
  }
  const char* m = argv[1];
  Dev d;
  if (!strcmp(m, "pair")) run_pair(d);
  else if (!strcmp(m, "allgather")) run_allgather(d);
  else if (!strcmp(m, "queue")) run_queue(d, false);
  else if (!strcmp(m, "split")) run_queue(d, true);
  else if (!strcmp(m, "mall")) run_mall();
  else { fprintf(stderr, "exchange_probe: unknown mode %s\n", m); return 2; }
  return 0;
}
