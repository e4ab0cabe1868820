// Stand-alone driver of the decode kernel through its C ABI only (no torch): random bf16 weights
// initialised on the device, a K/V cache filled for `prompt` positions, W warm-up and K timed
// decode steps at positions prompt .. prompt+K-1, HIP-event timing per launch. Used for profiling
// (rocprofv3 runs a plain binary) and for phase traces (--trace FILE dumps the last step's
// per-workgroup timestamps, uint64 [grid][TRACE_N]).
//
//   mk_bench [--shape 0.6b|1.7b] [--prompt P] [--max-seq S] [--steps K] [--warmup W] [--trace FILE]
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/megakernel_amd.h"

#define CK(x)                                                                                  \
  do {                                                                                         \
    hipError_t e_ = (x);                                                                       \
    if (e_ != hipSuccess) {                                                                    \
      fprintf(stderr, "mk_bench: %s failed: %s (%s:%d)\n", #x, hipGetErrorString(e_), __FILE__, __LINE__); \
      exit(1);                                                                                 \
    }                                                                                          \
  } while (0)

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

// uniform in [-sqrt(3), sqrt(3)) * std, rounded to bf16; std == 0 writes `fill`
__global__ void init_bf16(uint16_t* p, size_t n, uint64_t seed, float std, float fill) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    float v = fill;
    if (std > 0.f) {
      const uint64_t r = mix64(seed * 0x9e3779b97f4a7c15ull + i);
      v = ((float)(r >> 40) * (1.0f / 16777216.0f) * 2.f - 1.f) * 1.7320508f * std;
    }
    uint32_t u = __float_as_uint(v);
    u += 0x7fffu + ((u >> 16) & 1u);
    p[i] = (uint16_t)(u >> 16);
  }
}

static uint16_t* dev_bf16(size_t n, uint64_t seed, float std, float fill = 0.f) {
  uint16_t* p = nullptr;
  CK(hipMalloc(&p, n * 2));
  hipLaunchKernelGGL(init_bf16, dim3(1024), dim3(256), 0, 0, p, n, seed, std, fill);
  CK(hipGetLastError());
  return p;
}

static uint16_t host_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

int main(int argc, char** argv) {
  std::string shape = "0.6b", trace_path;
  int prompt = 32, max_seq = 512, steps = 256, warmup = 8;
  for (int i = 1; i < argc; ++i) {
    std::string a = argv[i];
    auto next = [&]() { return i + 1 < argc ? std::string(argv[++i]) : std::string(); };
    if (a == "--shape") shape = next();
    else if (a == "--prompt") prompt = atoi(next().c_str());
    else if (a == "--max-seq") max_seq = atoi(next().c_str());
    else if (a == "--steps") steps = atoi(next().c_str());
    else if (a == "--warmup") warmup = atoi(next().c_str());
    else if (a == "--trace") trace_path = next();
    else { fprintf(stderr, "mk_bench: unknown argument %s\n", a.c_str()); return 2; }
  }
  mk_model_dims dims = {1024, 3072, 28, 151936};
  if (shape == "1.7b") dims = {2048, 6144, 28, 151936};
  else if (shape != "0.6b") { fprintf(stderr, "mk_bench: --shape 0.6b|1.7b\n"); return 2; }
  if (prompt < 0 || prompt + std::max(steps, warmup) > max_seq) { fprintf(stderr, "mk_bench: prompt+steps > max-seq\n"); return 2; }
  const size_t H = dims.hidden, I = dims.intermediate, V = dims.vocab, L = dims.num_layers;
  const size_t Q = 16 * 128, KV = 8 * 128;
  printf("mk_bench: %s shape H=%zu I=%zu L=%zu V=%zu prompt=%d max_seq=%d steps=%d warmup=%d grid=%d\n", shape.c_str(), H, I,
         L, V, prompt, max_seq, steps, warmup, mk_grid_size());
  fflush(stdout);
  uint64_t seed = 1;
  const float sd = 0.02f;
  uint16_t* embed = dev_bf16(V * H, seed++, sd);
  uint16_t* fnorm = dev_bf16(H, seed++, 0.f, 1.f);
  std::vector<mk_layer_weights> table(L);
  for (size_t l = 0; l < L; ++l) {
    table[l].norm_weight = dev_bf16(H, seed++, 0.f, 1.f);
    table[l].q_weight = dev_bf16(Q * H, seed++, sd);
    table[l].k_weight = dev_bf16(KV * H, seed++, sd);
    table[l].v_weight = dev_bf16(KV * H, seed++, sd);
    table[l].q_norm_weight = dev_bf16(128, seed++, 0.f, 1.f);
    table[l].k_norm_weight = dev_bf16(128, seed++, 0.f, 1.f);
    table[l].o_proj_weight = dev_bf16(H * Q, seed++, sd);
    table[l].post_attn_norm_weight = dev_bf16(H, seed++, 0.f, 1.f);
    table[l].gate_proj_weight = dev_bf16(I * H, seed++, sd);
    table[l].up_proj_weight = dev_bf16(I * H, seed++, sd);
    table[l].down_proj_weight = dev_bf16(H * I, seed++, sd);
  }
  mk_layer_weights* dtable = nullptr;
  CK(hipMalloc(&dtable, L * sizeof(mk_layer_weights)));
  CK(hipMemcpy(dtable, table.data(), L * sizeof(mk_layer_weights), hipMemcpyHostToDevice));
  const size_t cache_n = L * 8 * (size_t)max_seq * 128;
  uint16_t* kc = dev_bf16(cache_n, seed++, 1.f);
  uint16_t* vc = dev_bf16(cache_n, seed++, 1.f);
  // RoPE tables with theta 1e6 (values do not affect timing)
  std::vector<uint16_t> hc((size_t)max_seq * 128), hs((size_t)max_seq * 128);
  for (int p = 0; p < max_seq; ++p)
    for (int d = 0; d < 128; ++d) {
      const double f = std::pow(1e6, -(double)(2 * (d % 64)) / 128.0);
      hc[(size_t)p * 128 + d] = host_bf16((float)std::cos(p * f));
      hs[(size_t)p * 128 + d] = host_bf16((float)std::sin(p * f));
    }
  uint16_t *cosd = nullptr, *sind = nullptr;
  CK(hipMalloc(&cosd, hc.size() * 2));
  CK(hipMalloc(&sind, hs.size() * 2));
  CK(hipMemcpy(cosd, hc.data(), hc.size() * 2, hipMemcpyHostToDevice));
  CK(hipMemcpy(sind, hs.data(), hs.size() * 2, hipMemcpyHostToDevice));
  float* logits = nullptr;
  int32_t* tok = nullptr;
  CK(hipMalloc(&logits, V * 4));
  CK(hipMalloc(&tok, 4));
  uint64_t* trace = nullptr;
  if (!trace_path.empty()) CK(hipMalloc(&trace, mk_trace_bytes()));
  CK(hipDeviceSynchronize());

  hipStream_t stream;
  CK(hipStreamCreate(&stream));
  int token = 1234;
  for (int w = 0; w < warmup; ++w)
    CK(mk_decode(&dims, token, embed, embed, fnorm, dtable, cosd, sind, kc, vc, prompt + w, max_seq, logits, tok, stream));
  CK(hipStreamSynchronize(stream));
  std::vector<hipEvent_t> ev(2 * steps);
  for (auto& e : ev) CK(hipEventCreate(&e));
  hipEvent_t t0, t1;
  CK(hipEventCreate(&t0));
  CK(hipEventCreate(&t1));
  CK(hipEventRecord(t0, stream));
  for (int s = 0; s < steps; ++s) {
    if (trace && s == steps - 1) {
      CK(hipMemsetAsync(trace, 0, mk_trace_bytes(), stream));
      CK(mk_set_trace(trace, mk_trace_bytes()));
    }
    CK(hipEventRecord(ev[2 * s], stream));
    CK(mk_decode(&dims, (token + 7 * s) % (int)V, embed, embed, fnorm, dtable, cosd, sind, kc, vc, prompt + s, max_seq, logits,
                 tok, stream));
    CK(hipEventRecord(ev[2 * s + 1], stream));
  }
  CK(hipEventRecord(t1, stream));
  CK(hipStreamSynchronize(stream));
  if (trace) CK(mk_set_trace(nullptr, 0));
  uint32_t status = 0;
  CK(mk_status(&status));
  std::vector<float> ms(steps);
  for (int s = 0; s < steps; ++s) CK(hipEventElapsedTime(&ms[s], ev[2 * s], ev[2 * s + 1]));
  float total = 0.f;
  CK(hipEventElapsedTime(&total, t0, t1));
  std::vector<float> sorted = ms;
  std::sort(sorted.begin(), sorted.end());
  double sum = 0;
  for (float m : ms) sum += m;
  int32_t htok = -1;
  CK(hipMemcpy(&htok, tok, 4, hipMemcpyDeviceToHost));
  printf("mk_bench: status=%u steps=%d kernel_us_avg=%.2f kernel_us_median=%.2f kernel_us_min=%.2f stream_us_per_step=%.2f tok/s=%.1f last_token=%d\n",
         status, steps, 1e3 * sum / steps, 1e3 * sorted[steps / 2], 1e3 * sorted[0], 1e3 * total / steps, steps / (total * 1e-3), htok);
  fflush(stdout);  // a profiler's exit-time crash must not lose the result line
  if (trace) {
    std::vector<uint64_t> h(mk_trace_bytes() / 8);
    CK(hipMemcpy(h.data(), trace, mk_trace_bytes(), hipMemcpyDeviceToHost));
    FILE* f = fopen(trace_path.c_str(), "wb");
    if (!f) { fprintf(stderr, "mk_bench: cannot write %s\n", trace_path.c_str()); return 1; }
    fwrite(h.data(), 8, h.size(), f);
    fclose(f);
    printf("mk_bench: trace (%zu bytes) -> %s\n", mk_trace_bytes(), trace_path.c_str());
  }
  return status == 0 ? 0 : 1;
}
