/*
 * rsv_hip.h -- C-ABI of librsv_hip.so, the MI355X (gfx950) backend of the
 * rwkv-rsv RWKV-7 forward step.
 *
 * Each entry point replaces one method of the reference's backend trait
 * `ComputeBackend` (reference: src/backend.rs:48-985); the cited line is the
 * trait method it implements.  A Rust `backend_hip.rs` binds these symbols
 * one-to-one: TensorId is a uint32_t, Int8Handle is
 * `rsv_int8`, slices are (pointer, length) pairs, and every call returns 0 on
 * success or a non-zero status whose text is `rsv_last_error()`; the Rust
 * side turns that into `Err(Box<dyn Error>)`.
 *
 * Conventions shared by every op:
 *  - One in-order HIP stream per context; ops are enqueued, downloads
 *    synchronise (backend_cuda.rs:1140-1151 semantics).
 *  - Per-session tensors are [batch, ...] slot-major; weights are shared.
 *  - Linear weights are [out, in] row-major ("A[m,k]"): int8 as the reference
 *    format (idx = u8[m,k] packed 4 per u32 low byte first, sz = u32[m,k/128]
 *    with fp16 scale in the low half and fp16 zero in the high half), fp16 as
 *    F16 tensors.  LoRA matrices are F16 [out, in].
 *  - Token slots hold u32 bit patterns (F32 or U32 tensors).
 */
#ifndef RSV_HIP_H
#define RSV_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct rsv_ctx rsv_ctx;

enum rsv_dtype { RSV_F32 = 0, RSV_F16 = 1, RSV_U32 = 2 };

/* Int8Handle (backend.rs:36-44). */
typedef struct rsv_int8 {
    uint32_t idx; /* U32 tensor, m*k/4 words */
    uint32_t sz;  /* U32 tensor, m*k/128 words */
    uint64_t m;
    uint64_t k;
} rsv_int8;

/* ---- context, errors (create_backend backend.rs:1019; R<T> runtime.rs:18) */
int rsv_create(int device, rsv_ctx **out);
int rsv_destroy(rsv_ctx *ctx);
const char *rsv_last_error(void); /* thread-local text of the last failure */
int rsv_device_name(rsv_ctx *ctx, char *buf, size_t len);

/* ---- tensors (backend.rs:50-60, 671-679) */
int rsv_tensor_create(rsv_ctx *ctx, uint64_t len, int dtype, uint32_t *id);  /* :50 */
int rsv_tensor_free(rsv_ctx *ctx, uint32_t id);                              /* :675 */
int rsv_drop_host(rsv_ctx *ctx, uint32_t id);                                /* :673 (no host copy is kept: no-op) */
int rsv_clear_cache(rsv_ctx *ctx);                                           /* :671 */
int rsv_tensor_len(rsv_ctx *ctx, uint32_t id, uint64_t *len, int *dtype);
/* F16 tensors convert from f32 with round-to-nearest-even. */
int rsv_upload(rsv_ctx *ctx, uint32_t id, const float *data, uint64_t len);                  /* :51 */
int rsv_upload_part(rsv_ctx *ctx, uint32_t id, uint64_t offset, const float *data, uint64_t len); /* :54 */
int rsv_upload_u32(rsv_ctx *ctx, uint32_t id, const uint32_t *data, uint64_t len);           /* :58 */
/* Raw-byte upload (u8 int8_idx payloads, fp16 bit patterns); no conversion. */
int rsv_upload_bytes(rsv_ctx *ctx, uint32_t id, const void *data, uint64_t nbytes);
int rsv_download(rsv_ctx *ctx, uint32_t id, float *out, uint64_t len);                      /* :59 */
int rsv_download_u32(rsv_ctx *ctx, uint32_t id, uint32_t *out, uint64_t len);                /* :60 */
int rsv_copy_device(rsv_ctx *ctx, uint32_t src, uint32_t dst);                              /* :679 */
int rsv_copy_device_f16(rsv_ctx *ctx, uint32_t src, uint32_t dst);                          /* :155 */
/* Share another context's tensors (backend.rs:137-142): every live tensor
 * of `src` appears in `ctx` under the same id and memory.  The destination
 * must hold no tensors yet.  Allocations are shared, not borrowed: each
 * stays valid until every context holding it has freed it (or been
 * destroyed), so either context may go first.  Later tensors of either
 * context get ids of their own table. */
int rsv_import_tensors(rsv_ctx *ctx, rsv_ctx *src);
/* Device ordinal of a context (no reference counterpart: build_shared
 * creates the second context on the source's device). */
int rsv_context_device(rsv_ctx *ctx, int *device);
int rsv_synchronize(rsv_ctx *ctx);

/* ---- batching and graphs (backend.rs:63-109) */
int rsv_begin_batch(rsv_ctx *ctx);        /* :63 */
int rsv_end_batch(rsv_ctx *ctx);          /* :64 (enqueue only; download syncs) */
int rsv_graph_begin(rsv_ctx *ctx);        /* :75 */
int rsv_graph_end(rsv_ctx *ctx);          /* :79 */
int rsv_graph_replay(rsv_ctx *ctx);       /* :83 */
int rsv_supports_graph_capture(rsv_ctx *ctx); /* :88, returns 1 */
int rsv_prefill_graph_valid(rsv_ctx *ctx, uint64_t t, int *valid); /* :95 */
int rsv_prefill_graph_begin(rsv_ctx *ctx, uint64_t t);             /* :99 */
int rsv_prefill_graph_end(rsv_ctx *ctx);                           /* :103 */
int rsv_prefill_graph_replay(rsv_ctx *ctx);                        /* :107 */

/* ---- token / sampler slots (backend.rs:113-135, 634, 954) */
int rsv_store_token(rsv_ctx *ctx, uint32_t tok, uint32_t token);   /* :113, stream-ordered */
int rsv_store_tokens(rsv_ctx *ctx, uint32_t tok, const uint32_t *tokens, uint64_t batch);
int rsv_store_sampler(rsv_ctx *ctx, uint32_t sampler, float temperature, uint32_t top_k, float top_p,
                      uint32_t seed, float repetition_penalty, float frequency_penalty,
                      float presence_penalty, uint32_t hist_len);                      /* :954 */
int rsv_store_sampler_async(rsv_ctx *ctx, uint32_t sampler, uint64_t row, float temperature,
                            uint32_t top_k, float top_p, uint32_t seed, float repetition_penalty,
                            float frequency_penalty, float presence_penalty, uint32_t hist_len); /* :119 */
int rsv_store_sampler_async_batch(rsv_ctx *ctx, uint32_t sampler, uint64_t row, float temperature,
                                  uint32_t top_k, float top_p, const uint32_t *seeds, uint64_t batch,
                                  float repetition_penalty, float frequency_penalty,
                                  float presence_penalty, uint32_t hist_len);            /* :634 */
uint64_t rsv_sampler_async_rows(rsv_ctx *ctx);                                          /* :135 */

/* ---- embedding gather (backend.rs:147, 449).  src may be F16 or F32. */
int rsv_gather_row_device_f16(rsv_ctx *ctx, uint32_t src, uint32_t dst, uint32_t tok, uint64_t c);
int rsv_gather_rows_device_f16(rsv_ctx *ctx, uint32_t src, uint32_t dst, uint32_t tok, uint64_t c,
                               uint64_t batch);

/* ---- normalisation (backend.rs:171, 185, 209, 461, 487) */
int rsv_norm(rsv_ctx *ctx, uint32_t x, uint32_t gamma, uint32_t beta, uint32_t y, uint64_t c,
             uint64_t h, float eps, uint64_t rows);
int rsv_norm_lerp6(rsv_ctx *ctx, uint32_t x, uint32_t state, uint32_t gamma, uint32_t beta,
                   uint32_t x_r, uint32_t x_w, uint32_t x_k, uint32_t x_v, uint32_t x_a, uint32_t x_g,
                   uint32_t o_r, uint32_t o_w, uint32_t o_k, uint32_t o_v, uint32_t o_a, uint32_t o_g,
                   uint64_t c, float eps);
int rsv_norm_lerp6_batch(rsv_ctx *ctx, uint32_t x, uint32_t state, uint32_t gamma, uint32_t beta,
                         uint32_t x_r, uint32_t x_w, uint32_t x_k, uint32_t x_v, uint32_t x_a,
                         uint32_t x_g, uint32_t o_r, uint32_t o_w, uint32_t o_k, uint32_t o_v,
                         uint32_t o_a, uint32_t o_g, uint64_t c, float eps, uint64_t batch);
int rsv_cmix_norm_lerp(rsv_ctx *ctx, uint32_t x, uint32_t state, uint32_t gamma, uint32_t beta,
                       uint32_t x_k, uint32_t out_xb, uint64_t c, float eps);
int rsv_cmix_norm_lerp_batch(rsv_ctx *ctx, uint32_t x, uint32_t state, uint32_t gamma, uint32_t beta,
                             uint32_t x_k, uint32_t out_xb, uint64_t c, float eps, uint64_t batch);

/* ---- WKV7 time-mix state update (backend.rs:223, 566) */
int rsv_fuse_ka_dplr_norm(rsv_ctx *ctx, uint32_t s, uint32_t k, uint32_t k_k, uint32_t a, uint32_t k_a,
                          uint32_t r, uint32_t v, uint32_t w, uint32_t ln_x_w, uint32_t ln_x_b,
                          uint32_t r_k, uint32_t k_mod, uint32_t y, uint32_t y_norm, uint64_t h,
                          uint64_t n, float eps, float gn_eps);
int rsv_fuse_ka_dplr_norm_batch(rsv_ctx *ctx, uint32_t s, uint32_t k, uint32_t k_k, uint32_t a,
                                uint32_t k_a, uint32_t r, uint32_t v, uint32_t w, uint32_t ln_x_w,
                                uint32_t ln_x_b, uint32_t r_k, uint32_t k_mod, uint32_t y,
                                uint32_t y_norm, uint64_t h, uint64_t n, float eps, float gn_eps,
                                uint64_t batch);

/* ---- fused stage-1 projections (backend.rs:247, 278, 503):
 * r,k,v = x{r,k,v} W^T; v_mid = xv V1^T; w_mid = tanh(xw W1^T); a_mid = xa A1^T;
 * g_mid = xg G1^T. */
int rsv_gemv_rkv_stage1(rsv_ctx *ctx, uint32_t rw, uint32_t kw, uint32_t vw, uint32_t v1, uint32_t w1,
                        uint32_t a1, uint32_t g1, uint32_t xr, uint32_t xk, uint32_t xv, uint32_t xw,
                        uint32_t xa, uint32_t xg, uint32_t r, uint32_t k, uint32_t v, uint32_t v_mid,
                        uint32_t w_mid, uint32_t a_mid, uint32_t g_mid, uint64_t c, uint64_t vm,
                        uint64_t wm, uint64_t am, uint64_t gm);
int rsv_gemv_int8_rkv_stage1(rsv_ctx *ctx, const rsv_int8 *rw, const rsv_int8 *kw, const rsv_int8 *vw,
                             uint32_t v1, uint32_t w1, uint32_t a1, uint32_t g1, uint32_t xr,
                             uint32_t xk, uint32_t xv, uint32_t xw, uint32_t xa, uint32_t xg,
                             uint32_t r, uint32_t k, uint32_t v, uint32_t v_mid, uint32_t w_mid,
                             uint32_t a_mid, uint32_t g_mid, uint64_t c, uint64_t vm, uint64_t wm,
                             uint64_t am, uint64_t gm);
int rsv_gemv_int8_rkv_stage1_batch(rsv_ctx *ctx, const rsv_int8 *rw, const rsv_int8 *kw,
                                   const rsv_int8 *vw, uint32_t v1, uint32_t w1, uint32_t a1,
                                   uint32_t g1, uint32_t xr, uint32_t xk, uint32_t xv, uint32_t xw,
                                   uint32_t xa, uint32_t xg, uint32_t r, uint32_t k, uint32_t v,
                                   uint32_t v_mid, uint32_t w_mid, uint32_t a_mid, uint32_t g_mid,
                                   uint64_t c, uint64_t vm, uint64_t wm, uint64_t am, uint64_t gm,
                                   uint64_t batch);
int rsv_gemv_rkv_stage1_batch(rsv_ctx *ctx, uint32_t rw, uint32_t kw, uint32_t vw, uint32_t v1,
                              uint32_t w1, uint32_t a1, uint32_t g1, uint32_t xr, uint32_t xk,
                              uint32_t xv, uint32_t xw, uint32_t xa, uint32_t xg, uint32_t r,
                              uint32_t k, uint32_t v, uint32_t v_mid, uint32_t w_mid, uint32_t a_mid,
                              uint32_t g_mid, uint64_t c, uint64_t vm, uint64_t wm, uint64_t am,
                              uint64_t gm, uint64_t batch);

/* ---- LoRA stage 2 (backend.rs:309, 536):
 * w = exp(scale*sigmoid(w_mid W2^T + w0)); a = sigmoid(a_mid A2^T + a0);
 * v += sigmoid(v_mid V2^T + v0) * (v_first - v); g = sigmoid(g_mid) G2^T.
 * scale_w is a 1-element F32 tensor (-1/sqrt(e)). */
int rsv_gemv_lowrank_chain4(rsv_ctx *ctx, uint32_t w2, uint32_t a2, uint32_t v2, uint32_t g2,
                            uint32_t w_mid, uint32_t a_mid, uint32_t v_mid, uint32_t g_mid,
                            uint32_t w0, uint32_t a0, uint32_t v0, uint32_t scale_w, uint32_t v_first,
                            uint32_t w_out, uint32_t a_out, uint32_t v_inout, uint32_t g_out,
                            uint64_t c, uint64_t wm, uint64_t am, uint64_t vm, uint64_t gm);
int rsv_gemv_lowrank_chain4_batch(rsv_ctx *ctx, uint32_t w2, uint32_t a2, uint32_t v2, uint32_t g2,
                                  uint32_t w_mid, uint32_t a_mid, uint32_t v_mid, uint32_t g_mid,
                                  uint32_t w0, uint32_t a0, uint32_t v0, uint32_t scale_w,
                                  uint32_t v_first, uint32_t w_out, uint32_t a_out, uint32_t v_inout,
                                  uint32_t g_out, uint64_t c, uint64_t wm, uint64_t am, uint64_t vm,
                                  uint64_t gm, uint64_t batch);

/* ---- weight GEMV with fused dequant (backend.rs:160, 337-415).  Shapes:
 * w = [m, k]; x = [n, k]; y = [n, m] (n = batch). */
int rsv_gemv_f16(rsv_ctx *ctx, uint32_t w, uint32_t x, uint32_t y, uint64_t m, uint64_t k, uint64_t n);
int rsv_gemv_f16_relu2(rsv_ctx *ctx, uint32_t w, uint32_t x, uint32_t y, uint64_t m, uint64_t k, uint64_t n);
int rsv_gemv_f16_mul_add(rsv_ctx *ctx, uint32_t w, uint32_t x, uint32_t g, uint32_t y, uint64_t m,
                         uint64_t k, uint64_t n);
int rsv_gemv_f16_add(rsv_ctx *ctx, uint32_t w, uint32_t x, uint32_t y, uint64_t m, uint64_t k, uint64_t n);
int rsv_gemv_int8_relu2(rsv_ctx *ctx, const rsv_int8 *w, uint32_t x, uint32_t y, uint64_t m, uint64_t k,
                        uint64_t n);
int rsv_gemv_int8_mul_add(rsv_ctx *ctx, const rsv_int8 *w, uint32_t x, uint32_t g, uint32_t y, uint64_t m,
                          uint64_t k, uint64_t n);
int rsv_gemv_int8_add(rsv_ctx *ctx, const rsv_int8 *w, uint32_t x, uint32_t y, uint64_t m, uint64_t k,
                      uint64_t n);
int rsv_gemv_int8_plain(rsv_ctx *ctx, const rsv_int8 *w, uint32_t x, uint32_t y, uint64_t m, uint64_t k,
                        uint64_t n);
int rsv_supports_sparse_ffn(rsv_ctx *ctx); /* :439, returns 1 */
/* ffn_value_sparse_add (backend.rs:422-441): x[c] += sum over f with
 * r2[f] != 0 of r2[f] * V[c, f], reading V from value_tiled, the fp16 tiled
 * copy [fh/128][c/256][128][256] made by rsv_tile_ffn_value.  value_w16 is
 * accepted for the trait's signature and not read.  c % 256 == 0,
 * fh % 128 == 0.  Summation order is fixed (no atomics). */
int rsv_ffn_value_sparse_add(rsv_ctx *ctx, uint32_t value_w16, uint32_t value_tiled, uint32_t r2, uint32_t x,
                             uint64_t c, uint64_t fh);
/* ffn_value_sparse_add_batch (backend.rs:592-602): the same for r2 [batch, fh], x [batch, c]. */
int rsv_ffn_value_sparse_add_batch(rsv_ctx *ctx, uint32_t value_tiled, uint32_t r2, uint32_t x, uint64_t c,
                                   uint64_t fh, uint64_t batch);
/* The tiled fp16 copy of ffn.value V [c, fh] for the two ops above (the
 * reference builds it on the host at load, gpu_model.rs:3290-3340): from an
 * int8 handle (dequantised as model.rs:234-252, then rounded to fp16) or an
 * F16 tensor w16 (w8 null).  *out receives a new F16 tensor of fh*c. */
int rsv_tile_ffn_value(rsv_ctx *ctx, uint32_t w16, const rsv_int8 *w8, uint64_t c, uint64_t fh, uint32_t *out);

/* ---- int8 dequant to f32 / f16 (model.rs:234-252; backend.rs:756) */
int rsv_dequant_int8_f32(rsv_ctx *ctx, const rsv_int8 *a, uint32_t out);
int rsv_dequant_int8_to_f16(rsv_ctx *ctx, const rsv_int8 *a, uint32_t out, uint64_t m, uint64_t k);

/* ---- argmax / sampling / token records (backend.rs:606, 621, 651, 654, 969-984) */
int rsv_argmax(rsv_ctx *ctx, uint32_t logits, uint32_t token, uint64_t n);
int rsv_argmax_into_host(rsv_ctx *ctx, uint32_t logits, uint32_t token, uint64_t n);
int rsv_argmax_batch(rsv_ctx *ctx, uint32_t logits, uint32_t token, uint64_t n, uint64_t batch);
/* One greedy self-loop round's tail in one launch: rsv_argmax_batch, then
 * rsv_record_tokens (backend.rs:621) of the chosen tokens, then
 * rsv_gather_rows_device_f16 (backend.rs:449) of their rows of `emb` into x
 * for the next step; the same results as the three calls in that order. */
int rsv_argmax_record_gather_batch(rsv_ctx *ctx, uint32_t logits, uint32_t token, uint64_t n,
                                   uint32_t out_seq, uint32_t cnt, uint64_t stride, uint32_t emb,
                                   uint32_t x, uint64_t c, uint64_t batch);
int rsv_sample(rsv_ctx *ctx, uint32_t logits, uint32_t token, uint64_t n, float temperature,
               uint32_t top_k, float top_p, uint32_t seed, float repetition_penalty,
               float frequency_penalty, float presence_penalty, const uint32_t *history,
               uint64_t hist_len);
int rsv_sample_into_host_seeded(rsv_ctx *ctx, uint32_t logits, uint32_t token, uint64_t n,
                                uint32_t temp, uint32_t mask, uint32_t counter, uint32_t sampler,
                                uint32_t hist);
int rsv_sample_into_host_seeded_batch(rsv_ctx *ctx, uint32_t logits, uint32_t token, uint64_t n,
                                      uint32_t temp, uint32_t mask, uint32_t counter,
                                      uint32_t sampler, uint32_t hist, uint64_t batch);
/* rsv_sample without allocation.  No counterpart in the reference: it is
 * for callers that cannot allocate (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  Same pipeline and result
 * as rsv_sample; the history is a device U32 tensor `hist` holding hist_len
 * token ids (ignored when hist_len is 0) instead of a host array.  The work
 * area (temp, counter, sampler row) is one static device array per GPU of
 * 2*262144+64 words (2 MiB), held until the process ends: n above 262144 is
 * rejected.  The first context on a device to call it owns the array until
 * rsv_destroy; calls from another context on that device fail (their streams
 * could overlap).  Calls from several host threads on the owning context's
 * one stream are ordered by that stream. */
int rsv_sample_noalloc(rsv_ctx *ctx, uint32_t logits, uint32_t token, uint64_t n, float temperature,
                       uint32_t top_k, float top_p, uint32_t seed, float repetition_penalty,
                       float frequency_penalty, float presence_penalty, uint32_t hist, uint64_t hist_len);
int rsv_record_token(rsv_ctx *ctx, uint32_t in_tok, uint32_t out_seq, uint32_t cnt);
int rsv_record_tokens(rsv_ctx *ctx, uint32_t in_tok, uint32_t out_seq, uint32_t cnt, uint64_t stride,
                      uint64_t batch);
/* rsv_record_tokens (backend.rs:621) and rsv_gather_rows_device_f16
 * (backend.rs:449) of the same tokens in one launch: the tail of a sampled
 * self-loop round; the same results as the two calls in that order. */
int rsv_record_gather_batch(rsv_ctx *ctx, uint32_t in_tok, uint32_t out_seq, uint32_t cnt, uint64_t stride,
                            uint32_t emb, uint32_t x, uint64_t c, uint64_t batch);

/* ---- sequence (prefill) ops (backend.rs:681-939) */
int rsv_copy_token(rsv_ctx *ctx, uint32_t x, uint32_t y, uint64_t c, uint64_t stride, uint64_t token);
int rsv_copy_token_batch(rsv_ctx *ctx, uint32_t x, uint32_t state, uint32_t lens, uint64_t c,
                         uint64_t t, uint64_t batch);
/* C[m,n] = A[m,k] B[n,k]^T (+bias[n] | +x[m,n] | relu^2 | tanh); A,B F16, C F32. */
int rsv_gemm(rsv_ctx *ctx, uint32_t a, uint32_t b, uint32_t c, uint64_t m, uint64_t n, uint64_t k);
int rsv_gemm_bias(rsv_ctx *ctx, uint32_t a, uint32_t b, uint32_t bias, uint32_t c, uint64_t m, uint64_t n,
                  uint64_t k);
int rsv_gemm_add(rsv_ctx *ctx, uint32_t a, uint32_t b, uint32_t x, uint32_t y, uint64_t m, uint64_t n,
                 uint64_t k);
int rsv_gemm_relu2(rsv_ctx *ctx, uint32_t a, uint32_t b, uint32_t c, uint64_t m, uint64_t n, uint64_t k);
int rsv_gemm_tanh(rsv_ctx *ctx, uint32_t a, uint32_t b, uint32_t c, uint64_t m, uint64_t n, uint64_t k);
/* C[m,n] (op)= A[m,k] W[n,k]^T with W int8 dequantised in the MFMA tile loader. */
int rsv_gemm_int8(rsv_ctx *ctx, uint32_t a, const rsv_int8 *w, uint32_t c, uint64_t m, int epilogue);
int rsv_to_f16(rsv_ctx *ctx, uint32_t x, uint32_t y, uint64_t c, uint64_t t, uint64_t m_pad,
               uint64_t x_stride, uint64_t y_stride);
int rsv_to_f16_triple(rsv_ctx *ctx, uint32_t xr, uint32_t xk, uint32_t xv, uint32_t yr, uint32_t yk,
                      uint32_t yv, uint64_t c, uint64_t t, uint64_t m_pad, uint64_t x_stride,
                      uint64_t y_stride);
int rsv_elementwise_sigmoid(rsv_ctx *ctx, uint32_t a, uint32_t y, uint64_t c, uint64_t batch);
int rsv_elementwise_sigmoid_inplace(rsv_ctx *ctx, uint32_t y, uint64_t c, uint64_t batch);
int rsv_elementwise_scale_exp(rsv_ctx *ctx, uint32_t a, uint32_t b, uint32_t y, uint64_t c, uint64_t batch);
int rsv_elementwise_mul(rsv_ctx *ctx, uint32_t a, uint32_t b, uint32_t y, uint64_t c, uint64_t batch);
int rsv_v_first_lerp(rsv_ctx *ctx, uint32_t v, uint32_t gate, uint32_t v_first, uint64_t c, uint64_t t,
                     uint64_t stride);
int rsv_fuse_ka(rsv_ctx *ctx, uint32_t k, uint32_t k_k, uint32_t a, uint32_t k_a, uint32_t k_mod,
                uint32_t kk_l2, uint32_t b, uint64_t h, uint64_t n, uint64_t batch);
int rsv_sum_rk_rk(rsv_ctx *ctx, uint32_t r, uint32_t k_mod, uint32_t r_k, uint32_t v, uint32_t y,
                  uint64_t h, uint64_t n, uint64_t batch);
int rsv_seq_shift(rsv_ctx *ctx, uint32_t x, uint32_t state, uint32_t tm, uint32_t y, uint64_t c,
                  uint64_t t, uint64_t stride_x, uint64_t stride_y);
int rsv_seq_shift_batch(rsv_ctx *ctx, uint32_t x, uint32_t state, uint32_t tm, uint32_t y, uint64_t c,
                        uint64_t t, uint64_t stride_x, uint64_t stride_y, uint64_t batch);
/* Sequential WKV over t tokens: s [H,N,N] state; r,w,k(=k_mod),v,a(=kk_l2),b [t, c]; y [t, c]. */
int rsv_dplr_seq(rsv_ctx *ctx, uint32_t s, uint32_t r, uint32_t w, uint32_t k, uint32_t v, uint32_t a,
                 uint32_t b, uint32_t y, uint64_t h, uint64_t n, uint64_t t, uint64_t c);
int rsv_dplr_seq_batch(rsv_ctx *ctx, uint32_t s, uint32_t r, uint32_t w, uint32_t k, uint32_t v,
                       uint32_t a, uint32_t b, uint32_t y, uint32_t lens, uint64_t h, uint64_t n,
                       uint64_t t, uint64_t c, uint64_t batch);
int rsv_segmean(rsv_ctx *ctx, uint32_t x, uint32_t out, uint32_t lens, uint64_t c, uint64_t t_pad,
                uint64_t batch);

/* ---- fused ragged prefill WKV (no reference counterpart as one call; it
 * composes fuse_ka + dplr_seq(_batch) + norm(GN) + sum_rk_rk of
 * backend.rs:765-870 over packed ragged segments).  seg_start/seg_len/seg_slot
 * are U32 [nseg]: token rows [start, start+len) of the packed [T, C] buffers
 * belong to state slot seg_slot. */
int rsv_wkv7_seq_ragged(rsv_ctx *ctx, uint32_t s, uint32_t r, uint32_t w, uint32_t k, uint32_t v,
                        uint32_t a, uint32_t k_k, uint32_t k_a, uint32_t r_k, uint32_t ln_x_w,
                        uint32_t ln_x_b, uint32_t y_norm, uint32_t seg_start, uint32_t seg_len,
                        uint32_t seg_slot, uint64_t nseg, uint64_t h, uint64_t n, float gn_eps);

/* The same scan leaving the att.output operand yg = (GroupNorm(y) + bonus*v)
 * * g as F16 [rows, C] (no reference counterpart as one call: the scan,
 * GroupNorm and the gate multiply of gpu_model.rs's prefill layer,
 * 2280-2320).  Rows [0, t_rows) of the packed buffers are in use.  y_work
 * (F32 [t_rows, C]) and bonus_work (F32 [t_rows, h]) are scratch owned by the
 * caller; their contents on return are unspecified. */
int rsv_wkv7_seq_ragged_gate(rsv_ctx *ctx, uint32_t s, uint32_t r, uint32_t w, uint32_t k, uint32_t v,
                             uint32_t a, uint32_t k_k, uint32_t k_a, uint32_t r_k, uint32_t ln_x_w,
                             uint32_t ln_x_b, uint32_t g, uint32_t y_work, uint32_t bonus_work, uint32_t yg,
                             uint32_t seg_start, uint32_t seg_len, uint32_t seg_slot, uint64_t nseg, uint64_t t_rows,
                             uint64_t h, uint64_t n, float gn_eps);

/* ---- prefill building blocks.  These have no one-to-one trait method: they
 * are the pieces the packed (ragged) prefill is built from, replacing the
 * seq_shift, to_f16, gemm_* and elementwise_* chains of gpu_model.rs:2911-3255 with
 * fewer, fused launches.
 *
 * rsv_seq_norm_mix: per token row t of x [T, C]: ln = LN(x[t]); prev = LN(x[p])
 * when row_prev[t] = p, or state[slot] when row_prev[t] = 0x80000000|slot;
 * out_j[t] = f16(ln + coef_j*(prev - ln)) for j < nout (out_j F16 [T, C]). */
int rsv_seq_norm_mix(rsv_ctx *ctx, uint32_t x, uint32_t state, uint32_t gamma, uint32_t beta,
                     const uint32_t *coef, const uint32_t *out_f16, uint64_t nout, uint32_t row_prev,
                     uint64_t t, uint64_t c, float eps);
/* state[seg_slot[g]] = LN(x[seg_last[g]]) for g < nseg. */
int rsv_seq_state_store(rsv_ctx *ctx, uint32_t x, uint32_t state, uint32_t gamma, uint32_t beta,
                        uint32_t seg_last, uint32_t seg_slot, uint64_t nseg, uint64_t c, float eps);
/* dst[dst_rows[i]] = src[src_rows[i]] for i < n (rows of c f32). */
int rsv_copy_rows(rsv_ctx *ctx, uint32_t src, uint32_t dst, uint32_t src_rows, uint32_t dst_rows,
                  uint64_t n, uint64_t c);
/* y = f16(a * b), n elements. */
int rsv_mul_to_f16(rsv_ctx *ctx, uint32_t a, uint32_t b, uint32_t y, uint64_t n);
/* General prefill GEMM: C[m,n] = epi(A[m,k] W[n,k]^T).  A is F16 [m, k];
 * W is an F16 tensor [n, k] (w8 == NULL) or an int8 handle; C is F32 or F16
 * [m, n].  epilogue: 0 store, 1 +bias[n], 2 +C (in place), 3 relu^2, 4 tanh,
 * 5 exp(scale*sigmoid(acc+bias)), 6 sigmoid(acc+bias),
 * 7 C + sigmoid(acc+bias)*(aux - C), 8 sigmoid(acc).  Unused ids: 0xFFFFFFFF. */
int rsv_gemm_ex(rsv_ctx *ctx, uint32_t a, uint32_t w16, const rsv_int8 *w8, uint32_t c, uint64_t m,
                uint64_t n, uint64_t k, int epilogue, uint32_t bias, uint32_t aux, uint32_t scale);

/* General fused GEMV launch (decode).  One launch runs up to 8 weight
 * matrices ("jobs"); each job is y[batch, m] (epilogue)= x'[batch, k] W^T where
 * x' is x after the prologue:
 *   prologue 0: x;  1: x * xmul;  2: sigmoid(x);
 *   3: LN-mix: ln = LN(x)*gamma + beta (eps 1e-5, over k), x' = ln + coef*(prev - ln);
 *      lnout (optional, [batch, k]) receives ln.
 *   4: GroupNorm-gate, batch 1: x' = ((GN(x)*gamma + beta) + prev) * xmul, GN over each
 *      64 columns (two-pass, gn_eps inside the sqrt): the att.output operand after the
 *      split form of rsv_wkv7_lora_decode (x = y, prev = bonus*v, xmul = gate).
 *   epilogue 0: store; 1: relu^2; 2: y += acc; 3: tanh; 4: exp(scale*sigmoid(acc+p0));
 *      5: sigmoid(acc+p0); 6: y + sigmoid(acc+p0)*(p1 - y); 7: store to y and p1.
 * W is F16 (w16) or int8 (w8).  After the launch, side_dst[b, :side_n] =
 * side_src[b, :side_n] for every batch row (ids 0xFFFFFFFF: no copy).
 * These compose the reference's norm_lerp6 + gemv_*_rkv_stage1,
 * gemv_lowrank_chain4 and cmix_norm_lerp + gemv_*_relu2 pairs
 * (backend.rs:185-415) into single launches. */
typedef struct rsv_gemv_job {
    uint32_t w16;
    const rsv_int8 *w8;
    uint64_t m, k;
    uint32_t x, y;
    int prologue, epilogue;
    uint32_t xmul, p0, p1, scale;
    uint32_t gamma, beta, prev, coef, lnout;
    float gn_eps; /* prologue 4 */
} rsv_gemv_job;
int rsv_gemv_multi(rsv_ctx *ctx, const rsv_gemv_job *jobs, uint64_t njobs, uint32_t side_src,
                   uint32_t side_dst, uint64_t side_n, uint64_t batch);

/* ---- batched decode on matrix cores (sessions B >= 16).  These compose
 * the same per-layer math as the *_batch trait ops (backend.rs:461-648) with
 * fp16 activation operands so the weight products run on MFMA.
 *
 * rsv_gemm_skinny: each job computes y[b, n] (epilogue)= sum_k x[b, k] W[n, k]
 * with x an F16 tensor [batch, k]; W F16 (w16) or int8 (w8); y F32 or F16
 * [batch, n]; y2 (optional F32) receives a copy; epilogue codes as
 * rsv_gemm_ex (0 store .. 8 sigmoid). */
typedef struct rsv_mm_job {
    uint32_t w16;
    const rsv_int8 *w8;
    uint64_t n, k;
    uint32_t x, y, y2;
    int epilogue;
    uint32_t bias, aux, scale;
    int tiled; /* weights (w16, or w8->idx and w8->sz) are the copies made by rsv_tile_weights */
} rsv_mm_job;
/* MFMA-tiled copy of a weight matrix for rsv_gemm_skinny: 32x32 tiles
 * (1 KiB int8 / 2 KiB fp16), lane-ordered, [row tile][k chunk].  src is an
 * int8 idx tensor (esz 1) or an F16 tensor (esz 2) of n x k; *out receives
 * a new tensor (rows padded to a multiple of 32).  esz 4 tiles an int8
 * scale/zero tensor [n, k/128] as [row tile][group][32 rows]; a tiled int8
 * job takes both tiled tensors in its rsv_int8 handle. */
int rsv_tile_weights(rsv_ctx *ctx, uint32_t src, uint64_t n, uint64_t k, int esz, uint32_t *out);
int rsv_gemm_skinny(rsv_ctx *ctx, const rsv_mm_job *jobs, uint64_t njobs, uint64_t batch);
/* rsv_gemm_skinny of one tiled job split into nslice equal k-slices (no
 * reference counterpart: the batched decode's ffn.value, backend.rs:691-725
 * runs it as one GEMM).  Slice s writes its partial product
 * sum_{k in slice s} x[b, k] W[n, k] to y[s, b, n] (y F32 of at least
 * nslice*batch*n; plain store, no epilogue operands), so no partial sums
 * pass through a reduction launch: rsv_ln_mix_f16_acc folds them into the
 * residual row it normalises.  k must be nslice slices of 128-multiples of
 * 288..2560 columns. */
int rsv_gemm_skinny_kslices(rsv_ctx *ctx, const rsv_mm_job *job, uint64_t nslice, uint64_t batch);

/* ---- several prefill GEMMs in one launch (no reference counterpart: the
 * reference issues one cuBLAS GEMM per weight, backend.rs:691-725).  Job i
 * computes y_i[t, n] (epilogue)= sum_k x_i[t, k] W_i[n, k] for t < m, as
 * rsv_gemm_ex does, with the fields of rsv_mm_job: x F16 [m, k]; W
 * row-major F16 (w16) or int8 (w8), tiled = 0; y F32 or F16 [m, n]; y2
 * unused (0xFFFFFFFF); epilogue, bias, aux, scale as rsv_gemm_ex.  Jobs may
 * mix weight formats; each job's results equal its own rsv_gemm_ex launch
 * bit for bit.  At most 8 jobs. */
int rsv_gemm_multi(rsv_ctx *ctx, const rsv_mm_job *jobs, uint64_t njobs, uint64_t m);
/* LN rows of x [batch, c] + nout (1 or 6) token-shift mixes as F16 outputs;
 * coef ids may be 0xFFFFFFFF (plain LN); state (optional) is the token-shift
 * row, read then overwritten with the LN row. */
int rsv_ln_mix_f16(rsv_ctx *ctx, uint32_t x, uint32_t state, uint32_t gamma, uint32_t beta,
                   const uint32_t *coef, const uint32_t *out_f16, uint64_t nout, uint64_t c, float eps,
                   uint64_t batch);
/* rsv_ln_mix_f16 of the row x + ((part[0] + part[1]) + ...) (part F32
 * [nslice, batch, c], nslice 1..4, the k-slice sums of rsv_gemm_skinny_kslices, added in
 * slice order); the summed row is also stored to xout (0xFFFFFFFF: not
 * stored), which must be another tensor than x.  The residual add of
 * ffn.value (model.rs:494-496) joined to the next LayerNorm (model.rs:402, 507). */
int rsv_ln_mix_f16_acc(rsv_ctx *ctx, uint32_t x, uint32_t part, uint64_t nslice, uint32_t xout, uint32_t state,
                       uint32_t gamma, uint32_t beta, const uint32_t *coef, const uint32_t *out_f16, uint64_t nout,
                       uint64_t c, float eps, uint64_t batch);
/* fuse_ka_dplr_norm_batch that also (or only) writes f16(y_norm * g) into
 * yg_f16 (the att.output operand); y_norm may be 0xFFFFFFFF. */
int rsv_wkv7_decode_ex(rsv_ctx *ctx, uint32_t s, uint32_t k, uint32_t k_k, uint32_t a, uint32_t k_a,
                       uint32_t r, uint32_t v, uint32_t w, uint32_t ln_x_w, uint32_t ln_x_b, uint32_t r_k,
                       uint32_t y_norm, uint32_t g, uint32_t yg_f16, uint64_t h, uint64_t n, float eps,
                       float gn_eps, uint64_t batch);

/* ---- fused LoRA-up chain + WKV7 step (no reference
 * counterpart; it composes gemv_lowrank_chain4, backend.rs:309-333, and
 * fuse_ka_dplr_norm, backend.rs:223-243, into one launch per layer).
 * From the stage-1 outputs r, k, v [batch, C] and the LoRA-up inputs
 * w_mid (tanh applied), a_mid, v_mid, g_mid (raw; the sigmoid of g is
 * applied here), F32 [batch, rank]: w = exp(scale_w*sigmoid(w_mid.W2^T + w0)),
 * a = sigmoid(a_mid.A2^T + a0), v += sigmoid(v_mid.V2^T + v0)*(v_first - v),
 * g = sigmoid(g_mid).G2^T; then the WKV7 step on state [batch, H, 64, 64]
 * (updated in place) and yg = (GroupNorm(y) + bonus) * g, the att.output
 * operand.  side_src [batch, C] is copied to side_dst when both are given
 * (ids 0xFFFFFFFF: none).  Each rank must be a multiple of 32 in 32..256.
 * With f16_io, batches of 16 and more, and ranks summing to at most 512,
 * the launch takes 4 sessions per block (the head's LoRA-up rows read once
 * per block, the dots on matrix cores); otherwise one block per (head,
 * session).  Results agree to fp32 rounding. */
typedef struct rsv_wkv_lora {
    uint32_t state, r, k, v, v_first;
    uint32_t w_mid, a_mid, v_mid, g_mid; /* F32 [batch, rank] */
    uint32_t w2, a2, v2, g2;             /* F16 [C, rank] */
    uint32_t w0, a0, v0, scale_w;
    uint32_t k_k, k_a, r_k, ln_x_w, ln_x_b;
    uint32_t yg;                         /* F32 [batch, C] */
    uint32_t side_src, side_dst;
    uint64_t n_head, w_rank, a_rank, v_rank, g_rank;
    float eps, gn_eps;
    int f16_io; /* 1: the four *_mid inputs are F16, g_mid already holds sigmoid(g), and yg is F16 */
    /* Split form (both set, F32 io): the head's
     * rows run on 4 blocks, yg receives the raw y = S r, y_bonus the bonus
     * term times v and y_gate the gate; the GroupNorm and the gate are then
     * applied by the consumer (rsv_gemv_multi prologue 4).  0xFFFFFFFF: the
     * one-launch form with the GroupNorm inside. */
    uint32_t y_bonus, y_gate; /* F32 [batch, C] */
} rsv_wkv_lora;
int rsv_wkv7_lora_decode(rsv_ctx *ctx, const rsv_wkv_lora *op, uint64_t batch);

/* ---- profiling hooks (backend.rs:67-70); kernel timing is done with rocprofv3 */
int rsv_clear_kernel_prof(rsv_ctx *ctx);
int rsv_dump_kernel_prof(rsv_ctx *ctx);

/* ---- prefill lanes.  No counterpart in the reference (its prefill runs on
 * one stream); for the host layer's pipelined prefill, which overlaps
 * consecutive packed chunks.  rsv_lane_select makes lane 0 (the context's
 * own stream) or lane 1 (a second stream of the context, made on first use,
 * default priority) the stream every later launch, copy and synchronisation
 * of ctx uses; refused during graph capture.  rsv_lane_record records event
 * ev (0..255) of the current lane; rsv_lane_wait makes the current lane wait
 * for the last recording of event ev of `lane`.  Work buffers a caller hands
 * to launches on both lanes must not overlap while both are in flight (the
 * batched-decode GEMM and the sampler use context-wide work areas: keep them
 * on one lane at a time). */
int rsv_lane_select(rsv_ctx *ctx, int lane);
int rsv_lane_record(rsv_ctx *ctx, int ev);
int rsv_lane_wait(rsv_ctx *ctx, int lane, int ev);

/* ---- raw access for harnesses: device pointer and stream of a tensor/ctx */
int rsv_tensor_ptr(rsv_ctx *ctx, uint32_t id, void **ptr);
int rsv_stream(rsv_ctx *ctx, void **stream);

#ifdef __cplusplus
}
#endif
#endif
