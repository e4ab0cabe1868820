/*
 * megakernel_amd.h -- C ABI of the MI355X (gfx950) batch-1 decode mega-kernel.
 *
 * Plain pointers and sizes only; no torch types. Every entry point returns a hipError_t and
 * never throws. Device pointers refer to memory on the current HIP device.
 *
 * Concurrency. A decode launch needs every CU of the device at once (one workgroup per CU,
 * waiting on each other). Each stream that launches gets its own exchange workspace (allocated on
 * the stream's first launch; 64 sets per device, a 65th stream takes over the least recently used
 * set after a device synchronization), so launches on different streams never share exchange
 * words; but launches that overlap in time on one device cannot all be resident:
 * they wait with bounded spins and end as failed launches (see "Failure" below). Serialize decode
 * calls per device.
 *
 * Failure. A launch whose bounded waits give up (its workgroups could not all be resident, or the
 * status word already asked to drain) still completes: it writes NaN logits and greedy token -1,
 * and sets a status bit (mk_status). Every later launch on the device drains the same way until
 * mk_reset, so a device-side token loop cannot continue from a failed step.
 *
 * Reference interface this replaces: the extern "C" launcher of tejeshbhalla/mega-kernel,
 * declared at /root/reference/pytorch_binding.cu:9-33 and defined at
 * /root/reference/megakernel.cu:898-994, bound only by the pybind `decode` operator
 * (/root/reference/pytorch_binding.cu:36-129).
 */
#ifndef MEGAKERNEL_AMD_H_
#define MEGAKERNEL_AMD_H_

#include <hip/hip_runtime_api.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/*
 * Per-layer weight table: 11 device pointers to bf16 tensors in the reference's order.
 * Same layout as the reference's `LayerWeights` (/root/reference/config.cuh:77-89), filled from
 * the flat 11-per-layer list built at /root/reference/model.py:30-44.
 *   norm_weight [H], q_weight [16*128, H], k_weight [8*128, H], v_weight [8*128, H],
 *   q_norm_weight [128], k_norm_weight [128], o_proj_weight [H, 16*128],
 *   post_attn_norm_weight [H], gate_proj_weight [I, H], up_proj_weight [I, H],
 *   down_proj_weight [H, I]
 */
typedef struct mk_layer_weights {
  const void* norm_weight;
  const void* q_weight;
  const void* k_weight;
  const void* v_weight;
  const void* q_norm_weight;
  const void* k_norm_weight;
  const void* o_proj_weight;
  const void* post_attn_norm_weight;
  const void* gate_proj_weight;
  const void* up_proj_weight;
  const void* down_proj_weight;
} mk_layer_weights;

/* Model shape. Head geometry is fixed at 16 query heads, 8 K/V heads, head_dim 128 (Qwen3 0.6B
 * and 1.7B). Supported (hidden, intermediate): (1024, 3072) and (2048, 6144). The reference
 * fixes these as compile-time constants (/root/reference/config.cuh:9-18). */
typedef struct mk_model_dims {
  int32_t hidden;
  int32_t intermediate;
  int32_t num_layers;
  int32_t vocab;
} mk_model_dims;

/*
 * Drop-in for the reference launcher `launch_decode_kernel`
 * (/root/reference/megakernel.cu:898-994; declaration /root/reference/pytorch_binding.cu:9-33).
 * Same arguments, same meaning, Qwen3-0.6B shape (hidden 1024, intermediate 3072, 28 layers,
 * vocab 151936) as in the reference:
 *   layer_weights  device pointer to mk_layer_weights[28]
 *   k_cache/v_cache [28, 8, max_seq_len, 128] bf16; the new K/V are written at `position`
 *   cache_len      must equal position + 1 (the reference always passes that)
 *   g_logits       fp32 [151936] output
 * The remaining scratch pointers (hidden_buffer ... g_v) are accepted for ABI compatibility and
 * not used: the kernel keeps its exchange buffers in a per-stream workspace owned by the library
 * and allocated on the stream's first launch. Returns hipErrorInvalidValue for a null pointer,
 * token/position out of range or cache_len != position + 1, otherwise the status of the launch.
 */
hipError_t launch_decode_kernel(int token_id, const void* embed_weight, const void* lm_head_weight,
                                const void* final_norm_weight, const void* layer_weights,
                                const void* cos_table, const void* sin_table, void* k_cache,
                                void* v_cache, void* hidden_buffer, void* g_residual,
                                void* g_activations, void* g_attn_output, void* g_normalized,
                                void* g_mlp_intermediate, void* g_logits, void* g_q, void* g_k,
                                void* g_v, int position, int cache_len, int max_seq_len,
                                hipStream_t stream);

/*
 * Shape-general form of the same operation (same reference counterpart as above; the reference
 * has one compile-time shape, this takes it at run time). Writes fp32 logits [vocab] and, when
 * out_token is not NULL, the greedy token (argmax over bf16-rounded logits, lowest index on ties)
 * as int32 to device memory, so a caller needs no separate argmax kernel.
 * Argument errors return hipErrorInvalidValue before anything is launched.
 */
hipError_t mk_decode(const mk_model_dims* dims, int token_id, const void* embed_weight,
                     const void* lm_head_weight, const void* final_norm_weight,
                     const void* layer_weights, const void* cos_table, const void* sin_table,
                     void* k_cache, void* v_cache, int position, int max_seq_len, float* logits,
                     int32_t* out_token, hipStream_t stream);

/*
 * mk_decode with no allocation on any call. No counterpart in the reference: it is for callers
 * that cannot call hipMalloc (code under HIP graph capture, tight serving loops, harnesses that
 * forbid allocation). Same arguments, results and errors as mk_decode, and the same kernels; the
 * exchange workspace is a file-scope device array of mk_workspace_bytes() bytes (1.2 MB) that each
 * device running the library holds until the process ends, instead of a per-stream allocation.
 * Limits, rejected with hipErrorInvalidValue before anything is launched: (hidden, intermediate)
 * one of the two supported shapes, 1..62 layers, vocab >= 256, position < max_seq_len.
 * The first call on a device initialises the array (a placement probe and a fill kernel on
 * `stream`, then a synchronization of `stream`), so make it outside graph capture. Every call on
 * one device shares that one array and keeps its state (launch sequence, status word) for the
 * next call: calls on one device must not overlap in time, on any stream, or they race.
 */
hipError_t mk_decode_noalloc(const mk_model_dims* dims, int token_id, const void* embed_weight,
                             const void* lm_head_weight, const void* final_norm_weight,
                             const void* layer_weights, const void* cos_table, const void* sin_table,
                             void* k_cache, void* v_cache, int position, int max_seq_len, float* logits,
                             int32_t* out_token, hipStream_t stream);

/*
 * Batched prefill: tokens[0..num_tokens-1] (int32 device array) at positions position ..
 * position + num_tokens - 1 go through the whole model in one pass -- every layer's products on
 * the matrix cores over all the tokens at once, causal attention over the cache -- writing each
 * token's K/V rows into k_cache/v_cache ([num_layers, 8, max_seq_len, 128] bf16, the decode
 * layout), and the last token's fp32 logits [vocab] to `logits` and, when out_token is not NULL,
 * its greedy token (argmax of the bf16-rounded logits, lowest index on ties). Rows before
 * `position` must already hold the earlier tokens (position 0 for a fresh prompt; larger for a
 * prompt fed in chunks). Numerics are mk_decode's (fp32 activations and accumulation, K/V
 * rounded to bf16), so a decode after the prefill continues exactly as after decode steps.
 *   layer_weights     HOST array of mk_layer_weights[num_layers] (device pointers inside)
 *   workspace         device memory of at least mk_prefill_workspace_bytes(dims, num_tokens)
 *                     bytes, 256-byte aligned, owned by the caller, not used after the call's work
 *                     completes on `stream`
 * A token outside [0, vocab) is embedded as token 0 and the call reports itself as failed in-band
 * (NaN logits, token -1). Asynchronous on `stream`. Argument errors (null pointers, unsupported
 * shape, position + num_tokens > max_seq_len, workspace too small or not 256-byte aligned) return
 * hipErrorInvalidValue before any launch.
 * Replaces the reference's Transformers prefill and the copy of its cache into the kernel layout
 * (/root/reference/model.py:72-87), which the reference runs before its decode loop.
 */
size_t mk_prefill_workspace_bytes(const mk_model_dims* dims, int num_tokens);
hipError_t mk_prefill(const mk_model_dims* dims, const int32_t* tokens, int num_tokens, int position,
                      const void* embed_weight, const void* lm_head_weight, const void* final_norm_weight,
                      const void* layer_weights, const void* cos_table, const void* sin_table,
                      void* k_cache, void* v_cache, int max_seq_len, float* logits, int32_t* out_token,
                      void* workspace, size_t workspace_bytes, hipStream_t stream);

/*
 * mk_prefill into a paged K/V cache: k_pages / v_pages, block_table, num_pages and page_size as
 * mk_decode_paged (bf16 [num_layers][num_pages][8][page_size][128]; position p of every layer and K/V
 * head in page block_table[p / page_size]; page_size a power of two up to 4096, ceil(max_seq_len /
 * page_size) at most 2048). The K/V rows of positions [position, position + num_tokens) are written
 * through the table and the attention reads earlier positions through it, so a prompt can be fed in
 * chunks and the cache handed to mk_decode_paged. A table entry outside [0, num_pages) that the call
 * touches is reported in-band (NaN logits, token -1); its rows are neither read (page 0 is) nor
 * written. Workspace as mk_prefill (mk_prefill_workspace_bytes). No reference counterpart: the
 * reference's cache is contiguous (/root/reference/model.py:79-87).
 */
hipError_t mk_prefill_paged(const mk_model_dims* dims, const int32_t* tokens, int num_tokens, int position,
                            const void* embed_weight, const void* lm_head_weight, const void* final_norm_weight,
                            const void* layer_weights, const void* cos_table, const void* sin_table, void* k_pages,
                            void* v_pages, const int32_t* block_table, int num_pages, int page_size, int max_seq_len,
                            float* logits, int32_t* out_token, void* workspace, size_t workspace_bytes,
                            hipStream_t stream);

/*
 * Batched decode: `batch` (1..64) independent sequences advance by one token each in one call.
 * Two engines: up to 16 sequences of the Qwen3-0.6B shape run as one persistent kernel (256
 * workgroups exchanging data through epoch-tagged words, the batch as the columns of the matrix-core
 * tiles), 17-24 as two such launches (16 and the rest; 17-32 with the persistent engine forced);
 * other batches run layer by layer (a few kernels per layer). mk_set_batch_engine chooses.
 * Sequence b decodes tokens[b] at positions[b] (both int32 device arrays of `batch` entries, so a
 * device-side loop can advance them): it writes its K/V rows at positions[b] of its own cache and
 * attends over [0, positions[b]]. k_cache/v_cache are bf16 [batch][num_layers][8][max_seq_len][128]
 * (sequence b's cache is the decode layout at offset b). Writes fp32 logits [batch][vocab] and,
 * when out_tokens is not NULL, each sequence's greedy token (argmax of the bf16-rounded logits,
 * lowest index on ties). Each layer's products run on the matrix cores with the weights read once
 * for all sequences; numerics are mk_decode's, so each sequence gets what mk_decode gives it up to
 * fp32 summation order.
 *   layer_weights     HOST array of mk_layer_weights[num_layers] (device pointers inside)
 *   workspace         device memory of at least mk_decode_batch_workspace_bytes(dims, batch,
 *                     max_seq_len) bytes, 256-byte aligned, owned by the caller
 * A token or position out of range (checked on the device) makes the call report NaN logits and
 * token -1 for every sequence. The vocabulary size must be a multiple of 16 (Qwen3's 151936 is).
 * Asynchronous on `stream`; argument errors return hipErrorInvalidValue before any launch. No
 * counterpart in the reference, whose operator decodes
 * one token of one sequence (/root/reference/pytorch_binding.cu:36-48).
 */
size_t mk_decode_batch_workspace_bytes(const mk_model_dims* dims, int batch, int max_seq_len);
hipError_t mk_decode_batch(const mk_model_dims* dims, int batch, const int32_t* tokens, const int32_t* positions,
                           const void* embed_weight, const void* lm_head_weight, const void* final_norm_weight,
                           const void* layer_weights, const void* cos_table, const void* sin_table, void* k_cache,
                           void* v_cache, int max_seq_len, float* logits, int32_t* out_tokens, void* workspace,
                           size_t workspace_bytes, hipStream_t stream);

/*
 * Several decode steps in one call, with no host synchronization between them: the device-side
 * multi-token loop. Step i (0 <= i < n) runs at position + i and reads its input token from device
 * memory, tokens[i] (int32, device array of n + 1 entries, tokens[0] set by the caller).
 *   generate != 0: greedy generation. Step i writes its greedy token (as mk_decode's out_token) to
 *                  tokens[i + 1], which step i + 1 then consumes; tokens[1..n] are the output.
 *   generate == 0: teacher forcing, e.g. filling the cache for a prompt through the decode path.
 *                  tokens[0..n-1] are all inputs; only the last step's greedy token is written,
 *                  to tokens[n].
 * logits (fp32 [vocab]) holds the last step's logits when the stream reaches the end of the call;
 * every step writes its K/V row. Requires position + n <= max_seq_len; other argument errors as
 * mk_decode. An input token out of range sets status bit 2 (see mk_status) and decodes token 0.
 * Replaces the reference's host loop of one `decode` call plus `argmax().item()` per token
 * (/root/reference/model.py:95-127), which synchronizes the host on every token.
 */
hipError_t mk_decode_steps(const mk_model_dims* dims, int32_t* tokens, int n, int generate,
                           const void* embed_weight, const void* lm_head_weight,
                           const void* final_norm_weight, const void* layer_weights,
                           const void* cos_table, const void* sin_table, void* k_cache, void* v_cache,
                           int position, int max_seq_len, float* logits, hipStream_t stream);

/*
 * mk_decode on a paged K/V cache. k_pages / v_pages are bf16 [num_layers][num_pages][8][page_size][128]:
 * the rows of positions [i * page_size, (i + 1) * page_size) of every layer and K/V head live in
 * page block_table[i] (int32 device array of ceil(max_seq_len / page_size) entries; only entries up
 * to position are read). page_size is a power of two up to 4096, and ceil(max_seq_len / page_size)
 * at most 2048. The new K/V rows are written at `position`, through the table. An entry outside
 * [0, num_pages) reads page 0 instead and sets status bit 3 (see mk_status); the new K/V rows are
 * not written when the position's own entry is such an entry. Other arguments and
 * errors as mk_decode. No reference counterpart: the reference's cache is contiguous
 * (/root/reference/model.py:79-87); this serves callers whose cache is a shared pool of pages.
 */
hipError_t mk_decode_paged(const mk_model_dims* dims, int token_id, const void* embed_weight,
                           const void* lm_head_weight, const void* final_norm_weight,
                           const void* layer_weights, const void* cos_table, const void* sin_table,
                           void* k_pages, void* v_pages, const int32_t* block_table, int num_pages,
                           int page_size, int position, int max_seq_len, float* logits,
                           int32_t* out_token, hipStream_t stream);

/* mk_decode_steps on a paged K/V cache (layout, table and limits as mk_decode_paged): the
 * device-side multi-token loop for callers that keep their cache in pages. No reference
 * counterpart (see mk_decode_steps and mk_decode_paged). */
hipError_t mk_decode_steps_paged(const mk_model_dims* dims, int32_t* tokens, int n, int generate,
                                 const void* embed_weight, const void* lm_head_weight,
                                 const void* final_norm_weight, const void* layer_weights,
                                 const void* cos_table, const void* sin_table, void* k_pages, void* v_pages,
                                 const int32_t* block_table, int num_pages, int page_size, int position,
                                 int max_seq_len, float* logits, hipStream_t stream);

/* Status of the current device: the OR of the status words of all its workspaces. 0 = healthy.
 *   bit 0  a bounded wait of a launch gave up (its workgroups could not all be resident): that
 *          launch wrote NaN logits and token -1, and every later launch drains until mk_reset;
 *   bit 1  workgroups b and b % 8 ran on different XCDs (the kernel relies on their sharing an L2):
 *          later launches write every exchange word through to memory (slower) until mk_reset;
 *   bit 2  a device-side input token of mk_decode_steps was out of range: token 0 was decoded;
 *   bit 3  a block-table entry was out of range: page 0 was read, and the new K/V rows were not
 *          written when the position's own entry was the bad one;
 *   bit 4  set by mk_request_drain: every later launch drains (NaN logits, token -1).
 * Bits are set with atomic ORs and only mk_reset clears them; bits of a workspace set handed to
 * another stream (more than 64 launching streams on the device) are kept. Synchronizes with the
 * device.
 * No reference counterpart: the reference surfaces errors only through the launch status. */
hipError_t mk_status(uint32_t* status);

/* Engine of mk_decode_batch for the calling process: 0 automatic (the persistent kernel where it
 * applies: the Qwen3-0.6B shape, 1..16 sequences -- one MFMA column block up to 8, two from 9 on --, at
 * most 32 layers, a device with 256 CUs; 17..24 sequences as two launches of it), 1 always
 * the layer-by-layer engine, 2 the persistent kernel where it applies (17..32 sequences as two
 * launches). Both give each sequence
 * mk_decode's numerics. hipErrorInvalidValue for another value. No reference counterpart. */
hipError_t mk_set_batch_engine(int engine);

/* Phase trace of the persistent batched kernel: with a device buffer of at least
 * mk_batch_trace_bytes() bytes, later launches store s_memrealtime stamps (100 MHz) per workgroup
 * (index j * 8 + xcd), layer (33 rows of 24 stamps; row 32: kernel start, LM head start and end) at
 * fixed points of each layer; NULL turns it off. For profiling (megakernel.batch_trace). No
 * reference counterpart. */
hipError_t mk_set_batch_trace(uint64_t* device_buffer, size_t bytes);
size_t mk_batch_trace_bytes(void);

/* Clears the status words and the exchange words of every workspace of the current device and
 * restarts their launch sequences. Synchronizes with the device. No reference counterpart. */
hipError_t mk_reset(void);

/* Waits for all work queued on the current device to finish (a device synchronization), then sets
 * status bit 4 on every workspace of the device, so that every launch enqueued after the call drains
 * at once (all its waits give up, NaN logits, token -1) until mk_reset. Launches queued before the
 * call run to completion first: it does not abandon queued work. Workspace sets created later (a new
 * stream's, or mk_decode_noalloc's first use) start drained too, and batched decodes enqueued after
 * the call on the persistent kernel of mk_decode_batch drain as well (NaN logits, token -1 for every
 * sequence). Its use is to exercise the failure path with every kernel still exiting normally. No
 * reference counterpart. */
hipError_t mk_request_drain(void);

/* Bytes of one exchange workspace set (the static array of mk_decode_noalloc has this size; each
 * stream's allocated workspace too). */
size_t mk_workspace_bytes(void);

/* Phase tracing (profiling builds and tools; no reference counterpart -- the reference has no
 * in-kernel timers). With a non-NULL device buffer of at least mk_trace_bytes() bytes, every later
 * launch on the current device writes, per workgroup, s_memrealtime stamps (100 MHz) at each
 * phase start and barrier arrival: uint64 [grid][TRACE_N], TRACE_N = mk_trace_bytes() / 8 / grid,
 * slot 20*layer + 2*phase (+1 when published) for phases A..E, 20*layer + 10.. for the exchange
 * waits, tail slots 1280.. for kernel start, final
 * norm, LM head and exit. NULL turns tracing off. */
hipError_t mk_set_trace(uint64_t* device_buffer, size_t bytes);
size_t mk_trace_bytes(void);

/* Number of workgroups (one per CU) a launch uses on the current device, or a negative value if
 * the device cannot run the kernel. No reference counterpart (the reference hard-codes 82 blocks,
 * /root/reference/config.cuh:27). */
int mk_grid_size(void);

/* Launch mode on the current device for subsequent calls: 0 = plain launch (default), 1 =
 * cooperative launch (hipLaunchCooperativeKernel: the runtime guarantees that all workgroups are
 * resident before the grid starts, at ~16 us per token). Either way the grid needs every CU; with a
 * plain launch a kernel of another stream or process that holds CUs makes the decode wait and, past
 * its bounded spins, end as a failed launch (status bit 0, NaN logits, token -1). No reference
 * counterpart (the reference always launches cooperatively, /root/reference/megakernel.cu:986-993). */
hipError_t mk_set_launch_mode(int cooperative);

/* Library version string. */
const char* mk_version(void);

#ifdef __cplusplus
}
#endif

#endif /* MEGAKERNEL_AMD_H_ */
