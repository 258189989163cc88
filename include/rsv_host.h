/*
 * rsv_host.h -- C-ABI of librsv_host.so, the C++ model driver that sits on
 * top of librsv_hip.so.  It restates the reference's library API
 * (reference: src/gpu_model.rs) for hosts without a Rust toolchain:
 * ModelBuilder/Bundle/State (3685-4105), the decode and prefill drivers
 * (GpuModel, 102-3256) and the batch / self-loop paths (871-1961).
 *
 * Semantics follow the reference: a Bundle owns a model and one session
 * State; logits are [vocab] f32; tokens are u32; every call returns 0 or a
 * non-zero status with the text in rsv_host_last_error().
 */
#ifndef RSV_HOST_H
#define RSV_HOST_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct rsv_bundle rsv_bundle;
typedef struct rsv_state rsv_state;

/* ModelInfo (gpu_model.rs:49) */
typedef struct rsv_model_info {
    uint64_t n_layer, n_embd, n_head, head_size, vocab, ffn;
    uint64_t w_mid, a_mid, v_mid, g_mid;
    int int8_linears; /* every layer linear is int8 */
    int int8_head;
} rsv_model_info;

/* SamplerParams (gpu_model.rs:3873-3911) */
typedef struct rsv_sampler_params {
    float temperature;
    uint32_t top_k;
    float top_p;
    uint32_t seed;
    float repetition_penalty;
    float frequency_penalty;
    float presence_penalty;
} rsv_sampler_params;

const char *rsv_host_last_error(void);

/* ModelBuilder::new(path).build() (gpu_model.rs:3697) on HIP device `device`. */
int rsv_model_build(const char *path, int device, rsv_bundle **out);
/* GpuModel::build_shared (gpu_model.rs:594-628): a second bundle on the same
 * device sharing every weight tensor of `src` (no copy), with its own
 * backend context (stream), work buffers and state.  Either bundle may be
 * freed first; shared memory is released when both are. */
int rsv_bundle_build_shared(rsv_bundle *src, rsv_bundle **out);
int rsv_bundle_free(rsv_bundle *b);
int rsv_bundle_info(rsv_bundle *b, rsv_model_info *info);

/* Bundle API (gpu_model.rs:3723-3860). logits: vocab floats. */
int rsv_infer_tokens(rsv_bundle *b, const uint32_t *tokens, uint64_t n, float *logits);
int rsv_infer_seq(rsv_bundle *b, const uint32_t *tokens, uint64_t n, float *logits);
int rsv_infer_chunked(rsv_bundle *b, const uint32_t *tokens, uint64_t n, uint64_t chunk, float *logits);
/* RnnOption::Full: logits for every position, n*vocab floats (gpu_model.rs:3784-3794). */
int rsv_infer_full(rsv_bundle *b, const uint32_t *tokens, uint64_t n, float *logits);
int rsv_infer_argmax(rsv_bundle *b, const uint32_t *tokens, uint64_t n, uint32_t *token);
int rsv_infer_argmax_selfloop(rsv_bundle *b, uint32_t seed, uint64_t n, uint32_t *out);
int rsv_infer_sample(rsv_bundle *b, const uint32_t *tokens, uint64_t n, const rsv_sampler_params *sp,
                     const uint32_t *history, uint64_t hist_len, uint32_t *token);
int rsv_infer_sample_selfloop(rsv_bundle *b, uint32_t seed, uint64_t n, const rsv_sampler_params *sp,
                              uint32_t *out);
int rsv_state_len(rsv_bundle *b, uint64_t *len); /* floats per session */
int rsv_state_back(rsv_bundle *b, float *out);
int rsv_state_load(rsv_bundle *b, const float *data, uint64_t len);
int rsv_reset(rsv_bundle *b);

/* Batch API (gpu_model.rs:871-1803): a State with `batch` slots. */
int rsv_create_batch_state(rsv_bundle *b, uint64_t batch, rsv_state **out);
int rsv_state_free(rsv_bundle *b, rsv_state *s);
int rsv_state_batch(rsv_state *s, uint64_t *batch);
int rsv_batch_state_back(rsv_bundle *b, rsv_state *s, float *out);               /* batch * state_len */
int rsv_batch_state_load(rsv_bundle *b, rsv_state *s, const float *data, uint64_t len);
int rsv_state_slot_back(rsv_bundle *b, rsv_state *s, uint64_t slot, float *out);
int rsv_state_slot_load(rsv_bundle *b, rsv_state *s, uint64_t slot, const float *data, uint64_t len);
int rsv_batch_state_reset(rsv_bundle *b, rsv_state *s);
/* forward_seq_batch (gpu_model.rs:1001): prompts are ragged (tokens packed,
 * lens[batch]); advances every slot; seeds[b] = last token of prompt b;
 * logits (optional, batch*vocab) = last-token logits of each prompt. */
int rsv_forward_seq_batch(rsv_bundle *b, rsv_state *s, const uint32_t *tokens, const uint64_t *lens,
                          uint32_t *seeds, float *logits);
/* One decode step for every slot: tokens[batch] in, logits[batch*vocab] out. */
int rsv_forward_tokens_batch(rsv_bundle *b, rsv_state *s, const uint32_t *tokens, float *logits);
/* Batch self-loops (gpu_model.rs:1639-1803); out is [batch, n]. */
int rsv_argmax_selfloop_batch(rsv_bundle *b, rsv_state *s, const uint32_t *seeds, uint64_t n,
                              uint32_t *out);
int rsv_sample_selfloop_batch(rsv_bundle *b, rsv_state *s, const uint32_t *seeds, uint64_t n,
                              const rsv_sampler_params *sp, uint32_t *out);

/* Ragged continuous batching (the north star's scheduler; no counterpart
 * in the reference, which pads batch prefill, gpu_model.rs:914-997).  Slot q
 * of s serves prompt q (tokens packed, lens[batch]) and then samples
 * decode_len tokens into out[q*decode_len ...].  Each step is one packed
 * dispatch: a decode token for every generating slot, then prompt chunks
 * (slots in order, split across steps when needed), budget tokens in all
 * (budget >= batch, <= 12288).  The GPU sampler (sp) draws token k of slot q
 * with seed seeds[q] + k.  steps (optional, max_steps entries) receives one
 * record per step; *nsteps the step count. */
typedef struct rsv_serve_step {
    uint64_t prefill_tokens, decode_tokens, sampled;
    double ms; /* host wall time of the step: dispatch, sampling, token download */
} rsv_serve_step;
int rsv_serve_ragged(rsv_bundle *b, rsv_state *s, const uint32_t *tokens, const uint64_t *lens, uint64_t decode_len,
                     const rsv_sampler_params *sp, const uint32_t *seeds, uint64_t budget, uint32_t *out,
                     rsv_serve_step *steps, uint64_t max_steps, uint64_t *nsteps);
/* rsv_serve_ragged that also copies, for each draw, the logits row it was
 * drawn from into sampled_logits[batch][decode_len][vocab] (host memory;
 * for checking the sampler and the batched logits separately). */
int rsv_serve_ragged_logits(rsv_bundle *b, rsv_state *s, const uint32_t *tokens, const uint64_t *lens,
                            uint64_t decode_len, const rsv_sampler_params *sp, const uint32_t *seeds, uint64_t budget,
                            uint32_t *out, rsv_serve_step *steps, uint64_t max_steps, uint64_t *nsteps,
                            float *sampled_logits);

/* Rows per packed prefill chunk of infer_seq / forward_seq_batch (1..12288,
 * default 4096, the reference's packing bound for ragged batches).  Larger
 * chunks fill more GEMM tile rounds per launch; with consecutive chunks
 * overlapped on two streams (rsv_set_prefill_lanes) 4096 is the faster. */
int rsv_set_prefill_chunk(rsv_bundle *b, uint64_t rows);

/* Streams a multi-chunk prefill uses (1 or 2, default 2).  With 2, consecutive
 * packed chunks of infer_seq / forward_seq_batch (without logits) run on two
 * streams of the context, each chunk waiting per layer only for the state its
 * predecessor leaves (token-shift rows, WKV state), so one chunk's scan
 * overlaps the other's GEMMs.  Results are bit-identical to 1.  No
 * counterpart in the reference (one stream). */
int rsv_set_prefill_lanes(rsv_bundle *b, int lanes);

/* Timed variants for benchmarks: run the self-loop with the graph already
 * captured, synchronising before and after, and report device-side elapsed
 * milliseconds through *ms (hipEvent timing on the context stream). */
int rsv_argmax_selfloop_batch_timed(rsv_bundle *b, rsv_state *s, const uint32_t *seeds, uint64_t n,
                                    uint32_t *out, float *ms);
int rsv_sample_selfloop_batch_timed(rsv_bundle *b, rsv_state *s, const uint32_t *seeds, uint64_t n,
                                    const rsv_sampler_params *sp, uint32_t *out, float *ms);

/* Backend context of a bundle (for harnesses that call librsv_hip.so directly). */
void *rsv_bundle_ctx(rsv_bundle *b);

#ifdef __cplusplus
}
#endif
#endif
