// Internal header of librsv_hip.so: context, tensor table, error plumbing and
// the launcher prototypes each kernel file provides.  Not part of the C-ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <cstdarg>
#include <cstdio>
#include <map>
#include <string>
#include <memory>
#include <vector>

#include "../../include/rsv_hip.h"

namespace rsv {

// ---------------------------------------------------------------- errors
void set_error(const char *fmt, ...);
#define RSV_FAIL(...) (::rsv::set_error(__VA_ARGS__), -1)
#define RSV_HIP(call)                                                                       \
    do {                                                                                    \
        hipError_t e_ = (call);                                                             \
        if (e_ != hipSuccess) return RSV_FAIL("%s failed: %s", #call, hipGetErrorString(e_)); \
    } while (0)

// ---------------------------------------------------------------- tensors
// A device allocation shared by every context that holds it (the context
// that made it and any that imported it): freed when the last holder lets go.
struct DevMem {
    void *ptr = nullptr;
    int device = 0;
    ~DevMem() {
        if (ptr) {
            hipSetDevice(device);
            hipFree(ptr);
        }
    }
};

struct Tensor {
    void *ptr = nullptr;
    uint64_t len = 0;  // elements
    int dtype = RSV_F32;
    bool live = false;
    bool foreign = false;  // imported from another context (same id and memory as there)
    std::shared_ptr<DevMem> mem;
};

inline size_t dtype_size(int dt) { return dt == RSV_F16 ? 2 : 4; }

// Kernel-side view of a GEMV job (one weight matrix times a batch of inputs
// with a fused prologue on x and a fused epilogue on y).
enum GemvFmt { FMT_I8 = 0, FMT_F16 = 1 };
enum GemvPro {
    PRO_NONE = 0,
    PRO_MUL = 1,      // x * xmul
    PRO_SIGMOID = 2,  // sigmoid(x)
    PRO_LNMIX = 3,    // ln = LN(x)*gamma+beta; ln + coef*(prev - ln)   (LN over the K columns)
    PRO_GNGATE = 4,   // ((GN64(x)*gamma + beta) + prev) * xmul   (GroupNorm over each 64 columns, eps)
};
enum GemvEpi {
    EPI_STORE = 0,    // y = acc
    EPI_RELU2 = 1,    // y = relu(acc)^2
    EPI_ADD = 2,      // y += acc
    EPI_TANH = 3,     // y = tanh(acc)
    EPI_WDECAY = 4,   // y = exp(scale * sigmoid(acc + p0))
    EPI_SIGBIAS = 5,  // y = sigmoid(acc + p0)
    EPI_VLERP = 6,    // y = y + sigmoid(acc + p0) * (p1 - y)
    EPI_STORE2 = 7,   // y = acc and p1 = acc (v_first snapshot)
};

struct GemvJob {
    const void *w;
    const uint32_t *sz;
    const float *x;
    const float *xmul;
    float *y;
    const float *p0;
    const float *p1;
    const float *scale;  // device scalar (EPI_WDECAY)
    // PRO_LNMIX operands: gamma/beta [K], prev [batch, K] (token-shift state),
    // coef [K]; lnout [batch, K] receives the plain LN rows when non-null
    const float *gamma, *beta, *prev, *coef;
    float *lnout;
    float eps;  // PRO_GNGATE
    int M, K;
    int fmt, epi, pro;
    int ldx, ldy;  // batch strides in elements
    int nblk;      // blocks along M (filled by the launcher)
    int ks;        // k-slices per row (register-resident B=1 kernel; filled by the launcher)
    int lpr;       // lanes per row (one-shot B=1 kernel; filled by the launcher)
    int rpb;       // rows per block (batched kernel; filled by the launcher)
    size_t wso;    // offset of the job's k-slice partial sums in the workspace (batched kernel)
};
constexpr int kMaxJobs = 8;
// A side copy done by the first block column of a launch: dst[b, :n] =
// src[b, :n] for the launch's batch rows (moves a token-shift LN row from a
// scratch buffer into the state once no block of the launch reads it).
struct SideCopy {
    const float *src;
    float *dst;
    int n;
};
struct GemvJobs {
    GemvJob j[kMaxJobs];
    int n;
    int blk_start[kMaxJobs + 1];
    SideCopy side;
};

}  // namespace rsv

struct rsv_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    std::vector<rsv::Tensor> tensors;  // TensorId = index
    std::vector<uint32_t> free_ids;
    bool capturing = false;
    hipGraph_t graph = nullptr;
    hipGraphExec_t graph_exec = nullptr;
    // prefill graphs keyed by token count (backend.rs:95-109)
    std::map<uint64_t, hipGraphExec_t> prefill_graphs;
    uint64_t prefill_t = 0;
    bool prefill_capturing = false;
    // device scratch for `sample(...)` (history upload + work rows)
    uint32_t *hist_dev = nullptr;
    uint64_t hist_cap = 0;
    float *sample_work = nullptr;
    uint64_t sample_work_cap = 0;
    int sm_count = 0;
    // split-K workspace of the batched-decode GEMM (fixed size, allocated
    // with the context so that graph capture never allocates)
    float *skinny_ws = nullptr;
    size_t skinny_ws_cap = 0;
    // prefill lanes: lane 0 is the context's own stream, lane 1 a second
    // stream made on first use; `stream` is the lane launches go to
    hipStream_t lane[2] = {nullptr, nullptr};
    std::vector<hipEvent_t> lane_ev[2];
};

namespace rsv {
rsv::Tensor *get_tensor(rsv_ctx *ctx, uint32_t id);

// ------------------------------------------------------------ launchers
// Every launcher validates shapes on the host before enqueuing and returns 0
// or a failure status (text through set_error).
int launch_gemv_jobs(rsv_ctx *ctx, GemvJobs &jobs, int batch);
int launch_dequant_int8(rsv_ctx *ctx, const uint32_t *idx, const uint32_t *sz, uint64_t m, uint64_t k,
                        void *out, int out_f16);

int launch_norm_lerp(rsv_ctx *ctx, const float *x, float *state, const float *gamma, const float *beta,
                     const float *const *coef, float *const *out, int nout, int c, float eps, int batch);
int launch_norm(rsv_ctx *ctx, const float *x, const float *gamma, const float *beta, float *y, int c,
                int h, float eps, int rows);
int launch_wkv7_decode(rsv_ctx *ctx, float *s, const float *k, const float *kk, const float *a,
                       const float *ka, const float *r, const float *v, const float *w,
                       const float *gamma, const float *beta, const float *rk, float *kmod, float *y,
                       float *yn, int h, int n, float eps, float gn_eps, int batch,
                       const float *gmul = nullptr, _Float16 *yg16 = nullptr);
int launch_gather_rows(rsv_ctx *ctx, const void *src, int src_f16, uint64_t src_rows, float *dst,
                       const uint32_t *tok, int c, int batch);
int launch_argmax(rsv_ctx *ctx, const float *logits, uint32_t *tok, int n, int batch);
int launch_record_gather(rsv_ctx *ctx, const uint32_t *in_tok, uint32_t *out_seq, uint32_t *cnt, int stride,
                         const void *emb, int emb_f16, uint64_t emb_rows, float *x, int c, int batch);
int launch_argmax_next(rsv_ctx *ctx, const float *logits, uint32_t *tok, int n, uint32_t *out_seq, uint32_t *cnt,
                       int stride, const void *emb, int emb_f16, uint64_t emb_rows, float *x, int c, int batch);
int launch_record_tokens(rsv_ctx *ctx, const uint32_t *in_tok, uint32_t *out_seq, uint32_t *cnt,
                         int stride, int batch);
int launch_set_u32(rsv_ctx *ctx, uint32_t *dst, const uint32_t *vals, int n);
int launch_store_sampler(rsv_ctx *ctx, float *dst, float temperature, uint32_t top_k, float top_p,
                         const uint32_t *seeds, int batch, float rep, float freq, float pres,
                         uint32_t hist_len);
// allocation-free sampling (k_sample.hip): the static work area's size, its
// per-device set-up (with the device current) and its device address
constexpr uint64_t kNoAllocMaxN = 262144;
constexpr uint64_t kNoAllocWords = 2 * kNoAllocMaxN + 64;
constexpr int kMaxDevices = 64;
int sample_scratch_init(int device);
uint32_t *sample_scratch(int device);
int sample_scratch_claim(int device, const void *ctx);
void sample_scratch_release(int device, const void *ctx);
int launch_sample(rsv_ctx *ctx, const float *logits, uint32_t *token, int n, float *temp,
                  uint32_t *counter, const float *sampler, const uint32_t *hist, int hist_stride,
                  int batch);
int launch_copy(rsv_ctx *ctx, void *dst, const void *src, size_t bytes);
int launch_elementwise(rsv_ctx *ctx, int op, const float *a, const float *b, float *y, int c, int batch);
int launch_to_f16(rsv_ctx *ctx, const float *x, _Float16 *y, int c, int t, int m_pad, int x_stride,
                  int y_stride);
int launch_v_first_lerp(rsv_ctx *ctx, float *v, const float *gate, const float *vf, int c, int t,
                        int stride);
int launch_fuse_ka(rsv_ctx *ctx, const float *k, const float *kk, const float *a, const float *ka,
                   float *kmod, float *kkl2, float *b, int h, int n, int batch);
int launch_sum_rk_rk(rsv_ctx *ctx, const float *r, const float *kmod, const float *rk, const float *v,
                     float *y, int h, int n, int batch);
int launch_seq_shift(rsv_ctx *ctx, const float *x, const float *state, const float *tm, float *y,
                     int c, int t, int sx, int sy, int batch);
int launch_copy_token_batch(rsv_ctx *ctx, const float *x, float *state, const uint32_t *lens, int c,
                            int t, int batch);
int launch_dplr_seq(rsv_ctx *ctx, float *s, const float *r, const float *w, const float *k,
                    const float *v, const float *a, const float *b, float *y, const uint32_t *lens,
                    int h, int n, int t, int c, int batch);
int launch_segmean(rsv_ctx *ctx, const float *x, float *out, const uint32_t *lens, int c, int t_pad,
                   int batch);
int launch_wkv7_seq_ragged_gate(rsv_ctx *ctx, float *s, const float *r, const float *w, const float *k,
                                const float *v, const float *a, const float *kk, const float *ka, const float *rk,
                                const float *gamma, const float *beta, const float *g, float *y_work,
                                float *bonus_work, _Float16 *yg, const uint32_t *seg_start, const uint32_t *seg_len,
                                const uint32_t *seg_slot, int nseg, int h, int n, float gn_eps, uint64_t rows,
                                uint64_t slots);
int launch_wkv7_seq_ragged(rsv_ctx *ctx, float *s, const float *r, const float *w, const float *k,
                           const float *v, const float *a, const float *kk, const float *ka,
                           const float *rk, const float *gamma, const float *beta, float *yn,
                           const uint32_t *seg_start, const uint32_t *seg_len,
                           const uint32_t *seg_slot, int nseg, int h, int n, float gn_eps, uint64_t rows,
                           uint64_t slots);
// Prefill GEMM: C[m,n] = epi(A[m,k] B[n,k]^T), A fp16, B fp16 or int8
// (dequantised in the tile loader), C fp32 or fp16.
enum GemmEpi {
    GE_STORE = 0, GE_BIAS = 1, GE_ADD = 2, GE_RELU2 = 3, GE_TANH = 4,
    GE_WDECAY = 5,   // exp(scale*sigmoid(acc + bias[n]))
    GE_SIGBIAS = 6,  // sigmoid(acc + bias[n])
    GE_VLERP = 7,    // c + sigmoid(acc + bias[n]) * (aux - c)   (c read in place)
    GE_SIGMOID = 8,  // sigmoid(acc)
};
struct GemmArgs {
    const _Float16 *a;
    const void *b;         // fp16 [n,k] or int8 idx
    const uint32_t *sz;    // int8 scale/zero (null for fp16)
    void *c;               // fp32 or fp16 [m,n]
    const float *bias;     // [n]
    const float *aux;      // [m,n] fp32
    const float *scale;    // device scalar
    int m, n, k;
    int lda, ldc;
    int epi, b_i8, c_f16;
};
int launch_gemm(rsv_ctx *ctx, const GemmArgs &g);
// Several prefill GEMMs with the same m in one launch (k_gemm2 tiles; jobs
// may mix int8 and fp16 weights).
struct GemmJobs {
    GemmArgs j[kMaxJobs];
    int n;
    int blk_start[kMaxJobs + 1];
};
int launch_gemm_multi(rsv_ctx *ctx, GemmJobs &jobs);
// Batched-decode GEMM on matrix cores (see k_skinny.hip); epilogue codes are GemmEpi.
struct SkinnyJob {
    const void *w;
    const uint32_t *sz;
    int fmt;
    const _Float16 *x;  // [batch, K] fp16, row stride ldx
    int ldx;
    void *y;            // [batch, N] fp32 or fp16, row stride ldy
    int ldy, y_f16;
    float *y2;          // optional fp32 copy of the result
    const float *bias, *aux, *scale;
    int N, K, epi, nblk;
    int split, ws_slot;  // k-slices per row group; first workspace tile
    int kslice;                    // k-chunks (of 32) per slice
    int tiled;                   // weights are the MFMA-tiled copy
    int wtile_ch;                // k-chunks per row tile of the tiled copy when the job is a k-slice of it (0: K/32)
};
struct SkinnyJobs {
    SkinnyJob j[kMaxJobs];
    int n;
    int blk_start[kMaxJobs + 1];
    int red_start[kMaxJobs + 1];  // blocks of the slice-reduction launch (row-major weights)
};
int launch_skinny(rsv_ctx *ctx, SkinnyJobs &jobs, int MB);
int launch_tile_weights(rsv_ctx *ctx, const void *src, void *dst, int n, int k, int esz);
// LayerNorm rows + up to 6 token-shift mixes, fp16 outputs (state optional).
int launch_ln_mix_f16(rsv_ctx *ctx, const float *x, float *state, const float *gamma, const float *beta,
                      const float *const *coef, _Float16 *const *out, int nout, int c, float eps, int batch,
                      const float *part = nullptr, int nsl = 0, float *xout = nullptr);
int launch_seq_norm_mix(rsv_ctx *ctx, const float *x, const float *state, const float *gamma, const float *beta,
                        const float *const *coef, _Float16 *const *out, int nout, const uint32_t *row_prev, int t,
                        int c, uint64_t slots, float eps);
int launch_seq_state_store(rsv_ctx *ctx, const float *x, float *state, const float *gamma, const float *beta,
                           const uint32_t *seg_last, const uint32_t *seg_slot, int nseg, int c, uint64_t rows,
                           uint64_t slots, float eps);
int launch_copy_rows(rsv_ctx *ctx, const float *src, float *dst, const uint32_t *src_rows, const uint32_t *dst_rows,
                     int n, int c, uint64_t src_n, uint64_t dst_n);
int launch_mul_to_f16(rsv_ctx *ctx, const float *a, const float *b, _Float16 *y, uint64_t n);
// Fused LoRA-up chain + WKV7 decode step of small batches (k_wkv.hip).
struct WkvLoraArgs {
    float *S;                        // [B, H, 64, 64]
    const float *r, *k, *v, *vf;     // [B, C] (vf: v_first)
    const void *mid[4];              // LoRA-up inputs w (tanh applied), a, v, g: [B, mid], F32 (g raw) or,
                                     // with f16_io, F16 (g with its sigmoid applied)
    const _Float16 *up[4];           // LoRA-up weights [C, mid]
    const float *w0, *a0, *v0;       // [C]
    const float *scale;              // device scalar (decay scale)
    const float *kk, *ka, *rk, *gamma, *beta;  // [C]
    void *yg;                        // [B, C] out: (GroupNorm(y) + bonus) * g, F32 or (f16_io) F16;
                                     // with y_bonus/y_gate set, the raw y = S r (split form)
    float *y_bonus, *y_gate;         // [B, C] split form: bonus * v and the gate g (GroupNorm left to the consumer)
    const float *side_src;           // [B, C] copied to side_dst (optional)
    float *side_dst;
    int H, mid_n[4];
    int f16_io;
    float eps, gn_eps;
};
int launch_wkv7_lora(rsv_ctx *ctx, const WkvLoraArgs &a, int batch);
// Sparse ffn.value (k_sparse.hip): tiled fp16 copy and x += r2 V over non-zero r2.
int launch_tile_ffn_value(rsv_ctx *ctx, const uint8_t *idx, const uint32_t *sz, const _Float16 *w16, _Float16 *out,
                          int c, int fh);
int launch_ffn_sparse(rsv_ctx *ctx, const float *r2, const _Float16 *vt, float *x, int c, int fh, int batch);

// s_waitcnt vmcnt(n) for n known at compile time after unrolling (the
// switch folds); other counters left alone.
#define SK_VM(n) case n: __builtin_amdgcn_s_waitcnt((n & 0xF) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8)); break;
__device__ __forceinline__ void sk_wait_vm(int n) {
    switch (n < 63 ? n : 63) {
        SK_VM(0) SK_VM(1) SK_VM(2) SK_VM(3) SK_VM(4) SK_VM(5) SK_VM(6) SK_VM(7) SK_VM(8) SK_VM(9) SK_VM(10) SK_VM(11)
        SK_VM(12) SK_VM(13) SK_VM(14) SK_VM(15) SK_VM(16) SK_VM(17) SK_VM(18) SK_VM(19) SK_VM(20) SK_VM(21) SK_VM(22)
        SK_VM(23) SK_VM(24) SK_VM(25) SK_VM(26) SK_VM(27) SK_VM(28) SK_VM(29) SK_VM(30) SK_VM(31) SK_VM(32) SK_VM(33)
        SK_VM(34) SK_VM(35) SK_VM(36) SK_VM(37) SK_VM(38) SK_VM(39) SK_VM(40) SK_VM(41) SK_VM(42) SK_VM(43) SK_VM(44)
        SK_VM(45) SK_VM(46) SK_VM(47) SK_VM(48) SK_VM(49) SK_VM(50) SK_VM(51) SK_VM(52) SK_VM(53) SK_VM(54) SK_VM(55)
        SK_VM(56) SK_VM(57) SK_VM(58) SK_VM(59) SK_VM(60) SK_VM(61) SK_VM(62)
        default: __builtin_amdgcn_s_waitcnt((15) | (3 << 14) | (0x7 << 4) | (0xF << 8)); break;
    }
}
#undef SK_VM

}  // namespace rsv
