// PyTorch-ROCm operator for the decode mega-kernel: the drop-in for the reference's pybind
// `decode` (/root/reference/pytorch_binding.cu:36-129, registered at :132-134).
//
// Same Python signature and meaning:
//   decode(token_id, embed_weight, lm_head_weight, final_norm_weight, layer_weights,
//          cos_table, sin_table, k_cache, v_cache, position, max_seq_len) -> fp32 logits [V]
// writes the new K/V at `position`, attends over [0, position], returns fresh logits.
//
// Differences by design: every argument is validated before any HIP call (the reference checks
// none); the per-layer weight table is built once per distinct set of weight tensors and kept on
// the device (the reference mallocs, uploads and frees it on every token); the call is fully
// asynchronous on the current stream (the reference's cudaFree synchronizes). `decode_greedy`
// additionally returns the fused device argmax, and the model shape (0.6B or 1.7B) is taken
// from the tensors instead of compile-time constants. A launch that could not complete its grid
// waits returns NaN logits and token -1 (no host synchronization needed to notice); `status()`
// tells why.
#include <torch/extension.h>
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>

#include <mutex>
#include <vector>

#include "../../include/megakernel_amd.h"

namespace {

constexpr int kPerLayer = 11;
constexpr int kHeadDim = 128, kQHeads = 16, kKVHeads = 8;

#define MK_HIP_CHECK(expr)                                                                 \
  do {                                                                                     \
    hipError_t e_ = (expr);                                                                \
    TORCH_CHECK(e_ == hipSuccess, "megakernel: ", #expr, " failed: ", hipGetErrorString(e_)); \
  } while (0)

// Device-resident LayerWeights tables, one per weight set (the 11 * L tensors' data pointers), so
// that sessions alternating between weight sets (e.g. two models) reuse their tables instead of
// rebuilding one on every switch. Each entry holds references to its tensors so the cached pointers
// cannot dangle. Up to kTablesPerDevice sets per device; beyond that the least recently used entry
// is dropped (and its tensors released).
struct TableCache {
  std::vector<torch::Tensor> held;
  std::vector<const void*> ptrs;
  torch::Tensor table;  // uint8 on device, num_layers * sizeof(mk_layer_weights)
  uint64_t last_use = 0;
};
constexpr size_t kTablesPerDevice = 8;
std::mutex g_mu;
std::vector<std::vector<TableCache>> g_tables(64);
uint64_t g_table_clock = 0;
int64_t g_tables_built = 0;

void check_bf16(const torch::Tensor& t, const char* name, at::IntArrayRef shape, const torch::Device& dev) {
  TORCH_CHECK(t.defined(), "megakernel: ", name, " is undefined");
  TORCH_CHECK(t.device() == dev, "megakernel: ", name, " must be on ", dev, ", got ", t.device());
  TORCH_CHECK(t.scalar_type() == torch::kBFloat16, "megakernel: ", name, " must be bfloat16, got ", t.scalar_type());
  TORCH_CHECK(t.is_contiguous(), "megakernel: ", name, " must be contiguous");
  TORCH_CHECK(t.sizes() == shape, "megakernel: ", name, " must have shape ", shape, ", got ", t.sizes());
}

struct Checked {
  mk_model_dims dims;
  torch::Device dev{torch::kCPU};
};

Checked validate(int64_t token_id, const torch::Tensor& embed, const torch::Tensor& lm_head,
                 const torch::Tensor& final_norm, const std::vector<torch::Tensor>& lw,
                 const torch::Tensor& cos, const torch::Tensor& sin, const torch::Tensor& kc,
                 const torch::Tensor& vc, int64_t position, int64_t max_seq_len, bool require_gpu = true,
                 bool paged = false) {
  TORCH_CHECK(embed.defined(), "megakernel: embed_weight is undefined");
  TORCH_CHECK(!require_gpu || embed.is_cuda(), "megakernel: embed_weight must be a GPU tensor");
  TORCH_CHECK(embed.dim() == 2, "megakernel: embed_weight must be [vocab, hidden]");
  const torch::Device dev = embed.device();
  const int64_t V = embed.size(0), H = embed.size(1);
  TORCH_CHECK(lw.size() % kPerLayer == 0 && !lw.empty(),
              "megakernel: layer_weights must hold 11 tensors per layer, got ", lw.size());
  const int64_t L = lw.size() / kPerLayer;
  TORCH_CHECK(lw[8].dim() == 2, "megakernel: gate_proj weight must be 2-D");
  const int64_t I = lw[8].size(0);
  TORCH_CHECK((H == 1024 && I == 3072) || (H == 2048 && I == 6144),
              "megakernel: supported (hidden, intermediate) are (1024, 3072) and (2048, 6144), got (", H, ", ", I, ")");
  check_bf16(embed, "embed_weight", {V, H}, dev);
  check_bf16(lm_head, "lm_head_weight", {V, H}, dev);
  check_bf16(final_norm, "final_norm_weight", {H}, dev);
  const int64_t Q = kQHeads * kHeadDim, KV = kKVHeads * kHeadDim;
  for (int64_t l = 0; l < L; ++l) {
    const torch::Tensor* t = &lw[l * kPerLayer];
    check_bf16(t[0], "input_layernorm", {H}, dev);
    check_bf16(t[1], "q_proj", {Q, H}, dev);
    check_bf16(t[2], "k_proj", {KV, H}, dev);
    check_bf16(t[3], "v_proj", {KV, H}, dev);
    check_bf16(t[4], "q_norm", {kHeadDim}, dev);
    check_bf16(t[5], "k_norm", {kHeadDim}, dev);
    check_bf16(t[6], "o_proj", {H, Q}, dev);
    check_bf16(t[7], "post_attention_layernorm", {H}, dev);
    check_bf16(t[8], "gate_proj", {I, H}, dev);
    check_bf16(t[9], "up_proj", {I, H}, dev);
    check_bf16(t[10], "down_proj", {H, I}, dev);
  }
  TORCH_CHECK(max_seq_len >= 1, "megakernel: max_seq_len must be positive");
  check_bf16(cos, "cos_table", {cos.size(0), kHeadDim}, dev);
  check_bf16(sin, "sin_table", {sin.size(0), kHeadDim}, dev);
  TORCH_CHECK(cos.size(0) >= max_seq_len && sin.size(0) >= max_seq_len,
              "megakernel: cos/sin tables need at least max_seq_len rows");
  if (!paged) {
    check_bf16(kc, "k_cache", {L, kKVHeads, max_seq_len, kHeadDim}, dev);
    check_bf16(vc, "v_cache", {L, kKVHeads, max_seq_len, kHeadDim}, dev);
  }
  TORCH_CHECK(kc.data_ptr() != vc.data_ptr(), "megakernel: k_cache and v_cache must be distinct");
  TORCH_CHECK(position >= 0 && position < max_seq_len, "megakernel: position ", position,
              " out of range [0, ", max_seq_len, ")");
  TORCH_CHECK(token_id >= 0 && token_id < V, "megakernel: token_id ", token_id, " out of range [0, ", V, ")");
  Checked c;
  c.dims = {(int32_t)H, (int32_t)I, (int32_t)L, (int32_t)V};
  c.dev = dev;
  return c;
}

const void* device_table(const std::vector<torch::Tensor>& lw, const torch::Device& dev, hipStream_t stream) {
  std::lock_guard<std::mutex> lk(g_mu);
  const int idx = dev.index() < 0 ? 0 : dev.index();
  TORCH_CHECK(idx < (int)g_tables.size(), "megakernel: device index too large");
  std::vector<TableCache>& cache = g_tables[idx];
  std::vector<const void*> ptrs(lw.size());
  for (size_t i = 0; i < lw.size(); ++i) ptrs[i] = lw[i].data_ptr();
  for (TableCache& tc : cache)
    if (tc.ptrs == ptrs) {
      tc.last_use = ++g_table_clock;
      return tc.table.data_ptr();
    }
  const int64_t L = lw.size() / kPerLayer;
  auto host = torch::empty({L * (int64_t)sizeof(mk_layer_weights)}, torch::dtype(torch::kUInt8).pinned_memory(true));
  auto* h = reinterpret_cast<mk_layer_weights*>(host.data_ptr());
  for (int64_t l = 0; l < L; ++l) {
    const void* const* p = &ptrs[l * kPerLayer];
    h[l] = {p[0], p[1], p[2], p[3], p[4], p[5], p[6], p[7], p[8], p[9], p[10]};
  }
  auto table = torch::empty({host.numel()}, torch::dtype(torch::kUInt8).device(dev));
  MK_HIP_CHECK(hipMemcpyAsync(table.data_ptr(), host.data_ptr(), host.numel(), hipMemcpyHostToDevice, stream));
  MK_HIP_CHECK(hipStreamSynchronize(stream));  // once per new weight set; keeps `host` alive until copied
  TableCache* slot = nullptr;
  if (cache.size() < kTablesPerDevice) {
    cache.emplace_back();
    slot = &cache.back();
  } else {
    // the least recently used set; after a device synchronization no launch on any stream still
    // reads its device table, which can then be released
    MK_HIP_CHECK(hipDeviceSynchronize());
    slot = &cache[0];
    for (TableCache& tc : cache)
      if (tc.last_use < slot->last_use) slot = &tc;
  }
  slot->held = lw;
  slot->ptrs = std::move(ptrs);
  slot->table = table;
  slot->last_use = ++g_table_clock;
  ++g_tables_built;
  return slot->table.data_ptr();
}

// Weight tables built so far by this process (all devices): a test hook showing that alternating
// weight sets reuses their tables.
int64_t weight_tables_built() {
  std::lock_guard<std::mutex> lk(g_mu);
  return g_tables_built;
}

std::tuple<torch::Tensor, torch::Tensor> run(int64_t token_id, torch::Tensor embed, torch::Tensor lm_head,
                                             torch::Tensor final_norm, std::vector<torch::Tensor> lw,
                                             torch::Tensor cos, torch::Tensor sin, torch::Tensor kc,
                                             torch::Tensor vc, int64_t position, int64_t max_seq_len,
                                             bool want_token) {
  Checked c = validate(token_id, embed, lm_head, final_norm, lw, cos, sin, kc, vc, position, max_seq_len);
  c10::hip::HIPGuardMasqueradingAsCUDA guard(c.dev);
  hipStream_t stream = c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(c.dev.index()).stream();
  const void* table = device_table(lw, c.dev, stream);
  auto logits = torch::empty({c.dims.vocab}, embed.options().dtype(torch::kFloat32));
  torch::Tensor tok;
  if (want_token) tok = torch::empty({1}, embed.options().dtype(torch::kInt32));
  MK_HIP_CHECK(mk_decode(&c.dims, (int)token_id, embed.data_ptr(), lm_head.data_ptr(), final_norm.data_ptr(), table,
                         cos.data_ptr(), sin.data_ptr(), kc.data_ptr(), vc.data_ptr(), (int)position,
                         (int)max_seq_len, logits.data_ptr<float>(),
                         want_token ? tok.data_ptr<int32_t>() : nullptr, stream));
  return {logits, tok};
}

torch::Tensor decode(int64_t token_id, torch::Tensor embed, torch::Tensor lm_head, torch::Tensor final_norm,
                     std::vector<torch::Tensor> lw, torch::Tensor cos, torch::Tensor sin, torch::Tensor kc,
                     torch::Tensor vc, int64_t position, int64_t max_seq_len) {
  return std::get<0>(run(token_id, embed, lm_head, final_norm, lw, cos, sin, kc, vc, position, max_seq_len, false));
}

std::tuple<torch::Tensor, torch::Tensor> decode_greedy(int64_t token_id, torch::Tensor embed, torch::Tensor lm_head,
                                                       torch::Tensor final_norm, std::vector<torch::Tensor> lw,
                                                       torch::Tensor cos, torch::Tensor sin, torch::Tensor kc,
                                                       torch::Tensor vc, int64_t position, int64_t max_seq_len) {
  return run(token_id, embed, lm_head, final_norm, lw, cos, sin, kc, vc, position, max_seq_len, true);
}

// Device-side multi-token loop (mk_decode_steps): n steps at position .. position + n - 1, each
// reading its input token from tokens[i] (int32 [n + 1] on the weights' device). generate: step i
// writes its greedy token to tokens[i + 1] for the next step; otherwise tokens[0..n-1] are inputs
// and only tokens[n] is written. Returns the last step's logits; nothing synchronizes the host.
torch::Tensor decode_steps(torch::Tensor tokens, int64_t n, bool generate, torch::Tensor embed, torch::Tensor lm_head,
                           torch::Tensor final_norm, std::vector<torch::Tensor> lw, torch::Tensor cos,
                           torch::Tensor sin, torch::Tensor kc, torch::Tensor vc, int64_t position,
                           int64_t max_seq_len) {
  Checked c = validate(0, embed, lm_head, final_norm, lw, cos, sin, kc, vc, position, max_seq_len);
  TORCH_CHECK(n >= 1, "megakernel: n must be positive");
  TORCH_CHECK(position + n <= max_seq_len, "megakernel: position + n (", position + n, ") exceeds max_seq_len (",
              max_seq_len, ")");
  TORCH_CHECK(tokens.defined() && tokens.device() == c.dev && tokens.scalar_type() == torch::kInt32 &&
                  tokens.is_contiguous() && tokens.dim() == 1 && tokens.size(0) == n + 1,
              "megakernel: tokens must be a contiguous int32 [n + 1] tensor on ", c.dev);
  c10::hip::HIPGuardMasqueradingAsCUDA guard(c.dev);
  hipStream_t stream = c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(c.dev.index()).stream();
  const void* table = device_table(lw, c.dev, stream);
  auto logits = torch::empty({c.dims.vocab}, embed.options().dtype(torch::kFloat32));
  MK_HIP_CHECK(mk_decode_steps(&c.dims, tokens.data_ptr<int32_t>(), (int)n, generate ? 1 : 0, embed.data_ptr(),
                               lm_head.data_ptr(), final_norm.data_ptr(), table, cos.data_ptr(), sin.data_ptr(),
                               kc.data_ptr(), vc.data_ptr(), (int)position, (int)max_seq_len,
                               logits.data_ptr<float>(), stream));
  return logits;
}

struct Paged {
  int num_pages, page_size;
};

// Shapes of a paged cache: k_pages / v_pages bf16 [L, num_pages, 8, page_size, 128] on the weights'
// device, page_size a power of two <= 4096, and an int32 block table of ceil(max_seq_len /
// page_size) <= 2048 entries or more.
Paged check_paged(const Checked& c, const torch::Tensor& kp, const torch::Tensor& vp, const torch::Tensor& block_table,
                  int64_t max_seq_len) {
  TORCH_CHECK(kp.defined() && kp.dim() == 5, "megakernel: k_pages must be [layers, num_pages, 8, page_size, 128]");
  const int64_t L = c.dims.num_layers, NP = kp.size(1), PS = kp.size(3);
  TORCH_CHECK(PS >= 1 && PS <= 4096 && (PS & (PS - 1)) == 0, "megakernel: page_size must be a power of two <= 4096");
  check_bf16(kp, "k_pages", {L, NP, kKVHeads, PS, kHeadDim}, c.dev);
  check_bf16(vp, "v_pages", {L, NP, kKVHeads, PS, kHeadDim}, c.dev);
  TORCH_CHECK(kp.data_ptr() != vp.data_ptr(), "megakernel: k_pages and v_pages must be distinct");
  const int64_t need = (max_seq_len + PS - 1) / PS;
  TORCH_CHECK(need <= 2048, "megakernel: ceil(max_seq_len / page_size) must be at most 2048");
  TORCH_CHECK(block_table.defined() && block_table.device() == c.dev && block_table.scalar_type() == torch::kInt32 &&
                  block_table.is_contiguous() && block_table.dim() == 1 && block_table.size(0) >= need,
              "megakernel: block_table must be a contiguous int32 tensor of >= ", need, " entries on ", c.dev);
  return {(int)NP, (int)PS};
}

// Paged-cache decode (mk_decode_paged): k_pages / v_pages bf16 [L, num_pages, 8, page_size, 128],
// block_table int32 [>= ceil(max_seq_len / page_size)] on the same device; page_size a power of two.
// Returns (fp32 logits [V], int32 greedy token on the device).
std::tuple<torch::Tensor, torch::Tensor> decode_paged(int64_t token_id, torch::Tensor embed, torch::Tensor lm_head,
                                                      torch::Tensor final_norm, std::vector<torch::Tensor> lw,
                                                      torch::Tensor cos, torch::Tensor sin, torch::Tensor kp,
                                                      torch::Tensor vp, torch::Tensor block_table, int64_t position,
                                                      int64_t max_seq_len) {
  Checked c = validate(token_id, embed, lm_head, final_norm, lw, cos, sin, kp, vp, position, max_seq_len, true, true);
  const Paged pg = check_paged(c, kp, vp, block_table, max_seq_len);
  c10::hip::HIPGuardMasqueradingAsCUDA guard(c.dev);
  hipStream_t stream = c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(c.dev.index()).stream();
  const void* table = device_table(lw, c.dev, stream);
  auto logits = torch::empty({c.dims.vocab}, embed.options().dtype(torch::kFloat32));
  auto tok = torch::empty({1}, embed.options().dtype(torch::kInt32));
  MK_HIP_CHECK(mk_decode_paged(&c.dims, (int)token_id, embed.data_ptr(), lm_head.data_ptr(), final_norm.data_ptr(),
                               table, cos.data_ptr(), sin.data_ptr(), kp.data_ptr(), vp.data_ptr(),
                               block_table.data_ptr<int32_t>(), pg.num_pages, pg.page_size, (int)position, (int)max_seq_len,
                               logits.data_ptr<float>(), tok.data_ptr<int32_t>(), stream));
  return {logits, tok};
}

// decode_steps on a paged cache (tensors as decode_paged); returns the last step's fp32 logits.
torch::Tensor decode_steps_paged(torch::Tensor tokens, int64_t n, bool generate, torch::Tensor embed,
                                 torch::Tensor lm_head, torch::Tensor final_norm, std::vector<torch::Tensor> lw,
                                 torch::Tensor cos, torch::Tensor sin, torch::Tensor kp, torch::Tensor vp,
                                 torch::Tensor block_table, int64_t position, int64_t max_seq_len) {
  Checked c = validate(0, embed, lm_head, final_norm, lw, cos, sin, kp, vp, position, max_seq_len, true, true);
  const Paged pg = check_paged(c, kp, vp, block_table, max_seq_len);
  TORCH_CHECK(n >= 1, "megakernel: n must be positive");
  TORCH_CHECK(position + n <= max_seq_len, "megakernel: position + n (", position + n, ") exceeds max_seq_len (",
              max_seq_len, ")");
  TORCH_CHECK(tokens.defined() && tokens.device() == c.dev && tokens.scalar_type() == torch::kInt32 &&
                  tokens.is_contiguous() && tokens.dim() == 1 && tokens.size(0) == n + 1,
              "megakernel: tokens must be a contiguous int32 [n + 1] tensor on ", c.dev);
  c10::hip::HIPGuardMasqueradingAsCUDA guard(c.dev);
  hipStream_t stream = c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(c.dev.index()).stream();
  const void* table = device_table(lw, c.dev, stream);
  auto logits = torch::empty({c.dims.vocab}, embed.options().dtype(torch::kFloat32));
  MK_HIP_CHECK(mk_decode_steps_paged(&c.dims, tokens.data_ptr<int32_t>(), (int)n, generate ? 1 : 0, embed.data_ptr(),
                                     lm_head.data_ptr(), final_norm.data_ptr(), table, cos.data_ptr(), sin.data_ptr(),
                                     kp.data_ptr(), vp.data_ptr(), block_table.data_ptr<int32_t>(), pg.num_pages,
                                     pg.page_size, (int)position, (int)max_seq_len, logits.data_ptr<float>(), stream));
  return logits;
}

// Batched prefill (mk_prefill / mk_prefill_paged): tokens (int32 [n] on the weights' device) at
// positions position .. position + n - 1, K/V rows written into the caches; returns the last token's
// fp32 logits [V] and its greedy token (int32 [1] on the device). The workspace is a tensor from
// torch's caching allocator, held until the call's work is queued.
static std::tuple<torch::Tensor, torch::Tensor> prefill_common(const torch::Tensor& tokens, const Checked& c,
                                                               const torch::Tensor& embed, const torch::Tensor& lm_head,
                                                               const torch::Tensor& final_norm,
                                                               const std::vector<torch::Tensor>& lw,
                                                               const torch::Tensor& cos, const torch::Tensor& sin,
                                                               const torch::Tensor& kc, const torch::Tensor& vc,
                                                               const torch::Tensor* block_table, const Paged* pg,
                                                               int64_t position, int64_t max_seq_len) {
  TORCH_CHECK(tokens.defined() && tokens.device() == c.dev && tokens.scalar_type() == torch::kInt32 &&
                  tokens.is_contiguous() && tokens.dim() == 1 && tokens.size(0) >= 1,
              "megakernel: tokens must be a non-empty contiguous int32 [n] tensor on ", c.dev);
  const int64_t n = tokens.size(0);
  TORCH_CHECK(position + n <= max_seq_len, "megakernel: position + n (", position + n, ") exceeds max_seq_len (",
              max_seq_len, ")");
  c10::hip::HIPGuardMasqueradingAsCUDA guard(c.dev);
  hipStream_t stream = c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(c.dev.index()).stream();
  std::vector<mk_layer_weights> table(c.dims.num_layers);
  for (int64_t l = 0; l < c.dims.num_layers; ++l) {
    const torch::Tensor* t = &lw[l * kPerLayer];
    table[l] = {t[0].data_ptr(), t[1].data_ptr(), t[2].data_ptr(), t[3].data_ptr(), t[4].data_ptr(), t[5].data_ptr(),
                t[6].data_ptr(), t[7].data_ptr(), t[8].data_ptr(), t[9].data_ptr(), t[10].data_ptr()};
  }
  const size_t bytes = mk_prefill_workspace_bytes(&c.dims, (int)n);
  auto ws = torch::empty({(int64_t)bytes}, embed.options().dtype(torch::kUInt8));
  auto logits = torch::empty({c.dims.vocab}, embed.options().dtype(torch::kFloat32));
  auto tok = torch::empty({1}, embed.options().dtype(torch::kInt32));
  if (pg)
    MK_HIP_CHECK(mk_prefill_paged(&c.dims, tokens.data_ptr<int32_t>(), (int)n, (int)position, embed.data_ptr(),
                                  lm_head.data_ptr(), final_norm.data_ptr(), table.data(), cos.data_ptr(),
                                  sin.data_ptr(), kc.data_ptr(), vc.data_ptr(), block_table->data_ptr<int32_t>(),
                                  pg->num_pages, pg->page_size, (int)max_seq_len, logits.data_ptr<float>(),
                                  tok.data_ptr<int32_t>(), ws.data_ptr(), bytes, stream));
  else
    MK_HIP_CHECK(mk_prefill(&c.dims, tokens.data_ptr<int32_t>(), (int)n, (int)position, embed.data_ptr(),
                            lm_head.data_ptr(), final_norm.data_ptr(), table.data(), cos.data_ptr(), sin.data_ptr(),
                            kc.data_ptr(), vc.data_ptr(), (int)max_seq_len, logits.data_ptr<float>(),
                            tok.data_ptr<int32_t>(), ws.data_ptr(), bytes, stream));
  return {logits, tok};
}

// Into the [L, 8, max_seq, 128] caches.
std::tuple<torch::Tensor, torch::Tensor> prefill(torch::Tensor tokens, torch::Tensor embed, torch::Tensor lm_head,
                                                 torch::Tensor final_norm, std::vector<torch::Tensor> lw,
                                                 torch::Tensor cos, torch::Tensor sin, torch::Tensor kc, torch::Tensor vc,
                                                 int64_t position, int64_t max_seq_len) {
  Checked c = validate(0, embed, lm_head, final_norm, lw, cos, sin, kc, vc, position, max_seq_len);
  return prefill_common(tokens, c, embed, lm_head, final_norm, lw, cos, sin, kc, vc, nullptr, nullptr, position,
                        max_seq_len);
}

// Into a paged cache (k_pages / v_pages and block_table as decode_paged).
std::tuple<torch::Tensor, torch::Tensor> prefill_paged(torch::Tensor tokens, torch::Tensor embed,
                                                       torch::Tensor lm_head, torch::Tensor final_norm,
                                                       std::vector<torch::Tensor> lw, torch::Tensor cos,
                                                       torch::Tensor sin, torch::Tensor kp, torch::Tensor vp,
                                                       torch::Tensor block_table, int64_t position, int64_t max_seq_len) {
  Checked c = validate(0, embed, lm_head, final_norm, lw, cos, sin, kp, vp, position, max_seq_len, true, true);
  const Paged pg = check_paged(c, kp, vp, block_table, max_seq_len);
  return prefill_common(tokens, c, embed, lm_head, final_norm, lw, cos, sin, kp, vp, &block_table, &pg, position,
                        max_seq_len);
}

// Batched decode (mk_decode_batch): B sequences, tokens and positions int32 [B] on the weights' device,
// caches bf16 [B, L, 8, max_seq, 128]; returns (fp32 logits [B, V], int32 greedy tokens [B] on the
// device).
std::tuple<torch::Tensor, torch::Tensor> decode_batch(torch::Tensor tokens, torch::Tensor positions, torch::Tensor embed,
                                                      torch::Tensor lm_head, torch::Tensor final_norm,
                                                      std::vector<torch::Tensor> lw, torch::Tensor cos, torch::Tensor sin,
                                                      torch::Tensor kc, torch::Tensor vc, int64_t max_seq_len) {
  Checked c = validate(0, embed, lm_head, final_norm, lw, cos, sin, kc, vc, 0, max_seq_len, true, true);
  TORCH_CHECK(tokens.defined() && tokens.device() == c.dev && tokens.scalar_type() == torch::kInt32 &&
                  tokens.is_contiguous() && tokens.dim() == 1 && tokens.size(0) >= 1 && tokens.size(0) <= 64,
              "megakernel: tokens must be a contiguous int32 [B] tensor (1 <= B <= 64) on ", c.dev);
  const int64_t B = tokens.size(0);
  TORCH_CHECK(positions.defined() && positions.device() == c.dev && positions.scalar_type() == torch::kInt32 &&
                  positions.is_contiguous() && positions.dim() == 1 && positions.size(0) == B,
              "megakernel: positions must be a contiguous int32 [B] tensor on ", c.dev);
  check_bf16(kc, "k_cache", {B, c.dims.num_layers, kKVHeads, max_seq_len, kHeadDim}, c.dev);
  check_bf16(vc, "v_cache", {B, c.dims.num_layers, kKVHeads, max_seq_len, kHeadDim}, c.dev);
  c10::hip::HIPGuardMasqueradingAsCUDA guard(c.dev);
  hipStream_t stream = c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(c.dev.index()).stream();
  std::vector<mk_layer_weights> table(c.dims.num_layers);
  for (int64_t l = 0; l < c.dims.num_layers; ++l) {
    const torch::Tensor* t = &lw[l * kPerLayer];
    table[l] = {t[0].data_ptr(), t[1].data_ptr(), t[2].data_ptr(), t[3].data_ptr(), t[4].data_ptr(), t[5].data_ptr(),
                t[6].data_ptr(), t[7].data_ptr(), t[8].data_ptr(), t[9].data_ptr(), t[10].data_ptr()};
  }
  const size_t bytes = mk_decode_batch_workspace_bytes(&c.dims, (int)B, (int)max_seq_len);
  auto ws = torch::empty({(int64_t)bytes}, embed.options().dtype(torch::kUInt8));
  auto logits = torch::empty({B, c.dims.vocab}, embed.options().dtype(torch::kFloat32));
  auto toks = torch::empty({B}, embed.options().dtype(torch::kInt32));
  MK_HIP_CHECK(mk_decode_batch(&c.dims, (int)B, tokens.data_ptr<int32_t>(), positions.data_ptr<int32_t>(),
                               embed.data_ptr(), lm_head.data_ptr(), final_norm.data_ptr(), table.data(), cos.data_ptr(),
                               sin.data_ptr(), kc.data_ptr(), vc.data_ptr(), (int)max_seq_len, logits.data_ptr<float>(),
                               toks.data_ptr<int32_t>(), ws.data_ptr(), bytes, stream));
  return {logits, toks};
}

int64_t status() {
  uint32_t s = 0;
  MK_HIP_CHECK(mk_status(&s));
  return s;
}

void reset() { MK_HIP_CHECK(mk_reset()); }

void request_drain() { MK_HIP_CHECK(mk_request_drain()); }

// 0 automatic, 1 layer-by-layer engine, 2 persistent kernel (where it applies), for decode_batch
void set_batch_engine(int64_t engine) {
  TORCH_CHECK(engine >= 0 && engine <= 2, "set_batch_engine: expected 0, 1 or 2");
  MK_HIP_CHECK(mk_set_batch_engine((int)engine));
}

// 0 = plain launch (default), 1 = cooperative launch, for the current device
void set_launch_mode(int64_t cooperative) {
  TORCH_CHECK(cooperative == 0 || cooperative == 1, "set_launch_mode: expected 0 or 1");
  MK_HIP_CHECK(mk_set_launch_mode((int)cooperative));
}

// Runs decode's argument validation only (tensors may live on any one device, nothing is
// launched) and returns (hidden, intermediate, num_layers, vocab). For host-side tests.
std::tuple<int64_t, int64_t, int64_t, int64_t> check_args(int64_t token_id, torch::Tensor embed, torch::Tensor lm_head,
                                                           torch::Tensor final_norm, std::vector<torch::Tensor> lw,
                                                           torch::Tensor cos, torch::Tensor sin, torch::Tensor kc,
                                                           torch::Tensor vc, int64_t position, int64_t max_seq_len) {
  Checked c = validate(token_id, embed, lm_head, final_norm, lw, cos, sin, kc, vc, position, max_seq_len, false);
  return {c.dims.hidden, c.dims.intermediate, c.dims.num_layers, c.dims.vocab};
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.def("decode", &decode, "Qwen3 single-token decode (fp32 logits)");
  m.def("decode_greedy", &decode_greedy, "Qwen3 single-token decode; returns (fp32 logits, int32 greedy token on device)");
  m.def("decode_steps", &decode_steps,
        "n decode steps with device-side tokens (int32 [n+1]); generate=True feeds each greedy token to the next "
        "step without host synchronization; returns the last step's fp32 logits");
  m.def("decode_paged", &decode_paged,
        "decode on a paged K/V cache ([L, pages, 8, page_size, 128] + int32 block table); returns (fp32 logits, "
        "int32 greedy token on device)");
  m.def("prefill_paged", &prefill_paged,
        "batched prefill into a paged K/V cache (tensors as decode_paged); returns (fp32 logits of the last token, "
        "int32 greedy token on device)");
  m.def("decode_steps_paged", &decode_steps_paged,
        "decode_steps on a paged K/V cache (tensors as decode_paged); returns the last step's fp32 logits");
  m.def("prefill", &prefill,
        "batched prefill of int32 tokens [n] at positions position..position+n-1 into the [L, 8, max_seq, 128] "
        "caches; returns (fp32 logits of the last token, int32 greedy token on device)");
  m.def("decode_batch", &decode_batch,
        "batched decode of B <= 64 sequences (int32 tokens [B], positions [B], caches [B, L, 8, max_seq, 128]); "
        "returns (fp32 logits [B, V], int32 greedy tokens [B] on device)");
  m.def("set_batch_engine", &set_batch_engine,
        "engine of decode_batch: 0 automatic (the persistent kernel for <= 16 sequences of the 0.6B shape, two launches of it for 17-24), "
        "1 layer by layer, 2 persistent where it applies");
  m.def("status", &status,
        "device status (0 = healthy; bit 0 timeout, 1 placement, 2 token, 3 page, 4 drain requested); synchronizes");
  m.def("reset", &reset, "clear the decode workspaces (exchange words, status words) and restart their launch sequences; synchronizes");
  m.def("request_drain", &request_drain,
        "set status bit 4: every later launch drains at once (NaN logits, token -1) until reset(); synchronizes");
  m.def("set_launch_mode", &set_launch_mode, "0 = plain launch (default), 1 = cooperative launch, on the current device");
  m.def("check_args", &check_args, "validate decode's arguments without launching; returns (hidden, intermediate, layers, vocab)");
  m.def("version", []() { return std::string(mk_version()); });
  m.def("weight_tables_built", &weight_tables_built,
        "LayerWeights tables the operator has built so far (one per distinct weight set while it stays cached)");
}
