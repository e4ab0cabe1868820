// Internal interface between the C entry points and the persistent batched decode kernel
// (batch_kernel.hip); not part of the exported C header.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/megakernel_amd.h"

// Sequences per launch of the persistent kernel.
constexpr int MKB_MAX = 16;
// Whether mk_decode_batch runs this batch on the persistent kernel: the Qwen3-0.6B shape, at most
// MKB_MAX sequences, at most 32 layers, a device with 256 CUs, and the engine not forced to the
// layer-by-layer one (mk_set_batch_engine). (17-32 sequences run as two such launches.)
bool mkb_applies(const mk_model_dims* dims, int batch, int max_seq_len);
// Workspace bytes the persistent kernel needs (exchange words, tickets, greedy keys).
size_t mkb_workspace_bytes();
// The engine selection (mk_set_batch_engine): 0 automatic, 1 layer by layer, 2 persistent kernel.
int mkb_engine();
// Host drain request (mk_request_drain / mk_reset): later launches give up at once.
void mkb_set_drain(bool on);
// Launches zero fill, the persistent kernel and the finish kernel on `stream`; arguments as
// mk_decode_batch (already validated), `layers` a host array.
hipError_t mkb_decode_batch(const mk_model_dims* dims, int batch, const int32_t* tokens, const int32_t* positions,
                            const void* embed_weight, const void* lm_head_weight, const void* final_norm_weight,
                            const mk_layer_weights* layers, const void* cos_table, const void* sin_table,
                            void* k_cache, void* v_cache, int max_seq_len, float* logits, int32_t* out_tokens,
                            void* workspace, hipStream_t stream);
