// Elementwise, normalisation, gather, argmax and token-record kernels of the
// decode and prefill paths.  All per-session buffers are [batch, ...].
#include "rsv_common.h"
#include "k_dpp.h"
#include <algorithm>

namespace rsv {

__device__ __forceinline__ float sigmoid_m(float v) { return 1.0f / (1.0f + expf(-v)); }

// Block-wide sum for 256-thread blocks (4 waves).
__device__ __forceinline__ float block_sum256(float v, float *red) {
    v = wave_sum_last(v);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 63) red[w] = v;
    __syncthreads();
    return red[0] + red[1] + red[2] + red[3];
}

// ------------------------------------------------ LayerNorm + token shift
// model.rs:402-411 / 487-490: ln = LN(x); out_j = ln + coef_j*(prev - ln);
// state = ln.  grid (batch), block 256; c <= 256*kMaxPer.
constexpr int kMaxPer = 16;  // prefill rows: c <= 4096
struct Ptr6 { const float *p[6]; };
struct Out6 { float *p[6]; };

template <int NOUT>
__global__ __launch_bounds__(1024) void k_norm_lerp(const float *__restrict__ x, float *__restrict__ state,
                                                    const float *__restrict__ gamma, const float *__restrict__ beta,
                                                    Ptr6 coef, Out6 out, int C, float eps) {
    // every load is issued before the statistics are reduced
    __shared__ float red[16];
    const int b = blockIdx.x, tid = threadIdx.x;
    constexpr int PER = 4;  // C <= 4096
    float xv[PER], gv[PER], bv[PER], pv[PER], cv[NOUT][PER];
#pragma unroll
    for (int m = 0; m < PER; m++) {
        const int i = tid + 1024 * m;
        const bool ok = i < C;
        xv[m] = ok ? x[(size_t)b * C + i] : 0.0f;
        gv[m] = ok ? gamma[i] : 0.0f;
        bv[m] = ok ? beta[i] : 0.0f;
        pv[m] = ok ? state[(size_t)b * C + i] : 0.0f;
#pragma unroll
        for (int j = 0; j < NOUT; j++) cv[j][m] = ok ? coef.p[j][i] : 0.0f;
    }
    float s = 0.0f;
#pragma unroll
    for (int m = 0; m < PER; m++) s += xv[m];
    s = wave_sum_last(s);
    if ((tid & 63) == 63) red[tid >> 6] = s;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int w = 0; w < 16; w++) tot += red[w];
    const float mean = tot / (float)C;
    float q = 0.0f;
#pragma unroll
    for (int m = 0; m < PER; m++) {
        const float d = xv[m] - mean;
        q += (tid + 1024 * m < C) ? d * d : 0.0f;
    }
    q = wave_sum_last(q);
    __syncthreads();
    if ((tid & 63) == 63) red[tid >> 6] = q;
    __syncthreads();
    float qt = 0.0f;
#pragma unroll
    for (int w = 0; w < 16; w++) qt += red[w];
    const float inv_std = 1.0f / sqrtf(qt / (float)C + eps);
#pragma unroll
    for (int m = 0; m < PER; m++) {
        const int i = tid + 1024 * m;
        if (i >= C) continue;
        const float ln = (xv[m] - mean) * inv_std * gv[m] + bv[m];
        const size_t o = (size_t)b * C + i;
        const float dlt = pv[m] - ln;
#pragma unroll
        for (int j = 0; j < NOUT; j++) out.p[j][o] = ln + cv[j][m] * dlt;
        state[o] = ln;
    }
}

int launch_norm_lerp(rsv_ctx *ctx, const float *x, float *state, const float *gamma, const float *beta,
                     const float *const *coef, float *const *out, int nout, int c, float eps, int batch) {
    if (c <= 0 || c > 4096) return RSV_FAIL("norm_lerp: c=%d outside 1..4096", c);
    Ptr6 cp{};
    Out6 op{};
    for (int j = 0; j < nout; j++) { cp.p[j] = coef[j]; op.p[j] = out[j]; }
    switch (nout) {
        case 1: hipLaunchKernelGGL(k_norm_lerp<1>, dim3(batch), dim3(1024), 0, ctx->stream, x, state, gamma, beta, cp, op, c, eps); break;
        case 6: hipLaunchKernelGGL(k_norm_lerp<6>, dim3(batch), dim3(1024), 0, ctx->stream, x, state, gamma, beta, cp, op, c, eps); break;
        default: return RSV_FAIL("norm_lerp: nout must be 1 or 6 (got %d)", nout);
    }
    RSV_HIP(hipGetLastError());
    return 0;
}

// ---------------------------------------------- LayerNorm / GroupNorm rows
// backend.rs:171 semantics: rows*h groups of c elements; gamma/beta indexed
// by (group % h)*c + i.  Two-pass statistics (model.rs:625-635).
__global__ __launch_bounds__(256) void k_norm(const float *__restrict__ x, const float *__restrict__ gamma,
                                              const float *__restrict__ beta, float *__restrict__ y, int c,
                                              int h, float eps) {
    __shared__ float red[4];
    const int g = blockIdx.x, hh = g % h, tid = threadIdx.x;
    const float *xg = x + (size_t)g * c;
    float s = 0.0f;
    for (int i = tid; i < c; i += 256) s += xg[i];
    const float mean = block_sum256(s, red) / (float)c;
    float q = 0.0f;
    for (int i = tid; i < c; i += 256) { const float d = xg[i] - mean; q += d * d; }
    const float var = block_sum256(q, red) / (float)c + eps;
    const float inv_std = 1.0f / sqrtf(var);
    for (int i = tid; i < c; i += 256)
        y[(size_t)g * c + i] = (xg[i] - mean) * inv_std * gamma[hh * c + i] + beta[hh * c + i];
}

// The same for rows of c <= 4096: x, gamma and beta are loaded into
// registers up front (16 per thread), so the two reductions and the output
// wait on one round of loads instead of three.
__global__ __launch_bounds__(256) void k_norm_reg(const float *__restrict__ x, const float *__restrict__ gamma,
                                                  const float *__restrict__ beta, float *__restrict__ y, int c,
                                                  int h, float eps) {
    __shared__ float red[4];
    constexpr int PER = 16;
    const int g = blockIdx.x, hh = g % h, tid = threadIdx.x;
    const float *xg = x + (size_t)g * c;
    float xv[PER], gv[PER], bv[PER];
#pragma unroll
    for (int m = 0; m < PER; m++) {
        const int i = tid + 256 * m;
        const bool ok = i < c;
        xv[m] = ok ? xg[i] : 0.0f;
        gv[m] = ok ? gamma[hh * c + i] : 0.0f;
        bv[m] = ok ? beta[hh * c + i] : 0.0f;
    }
    float s = 0.0f;
#pragma unroll
    for (int m = 0; m < PER; m++) s += xv[m];
    const float mean = block_sum256(s, red) / (float)c;
    float q = 0.0f;
#pragma unroll
    for (int m = 0; m < PER; m++) {
        const float d = xv[m] - mean;
        q += tid + 256 * m < c ? d * d : 0.0f;
    }
    const float var = block_sum256(q, red) / (float)c + eps;
    const float inv_std = 1.0f / sqrtf(var);
#pragma unroll
    for (int m = 0; m < PER; m++) {
        const int i = tid + 256 * m;
        if (i < c) y[(size_t)g * c + i] = (xv[m] - mean) * inv_std * gv[m] + bv[m];
    }
}

int launch_norm(rsv_ctx *ctx, const float *x, const float *gamma, const float *beta, float *y, int c,
                int h, float eps, int rows) {
    if (c <= 0 || h <= 0 || rows <= 0) return RSV_FAIL("norm: bad c=%d h=%d rows=%d", c, h, rows);
    if (c <= 4096)
        hipLaunchKernelGGL(k_norm_reg, dim3(rows * h), dim3(256), 0, ctx->stream, x, gamma, beta, y, c, h, eps);
    else
        hipLaunchKernelGGL(k_norm, dim3(rows * h), dim3(256), 0, ctx->stream, x, gamma, beta, y, c, h, eps);
    RSV_HIP(hipGetLastError());
    return 0;
}

// ------------------------------------------------------------- gather rows
// Token ids at or beyond the table size produce a zero row instead of an
// out-of-bounds read.
__global__ void k_gather_rows(const void *__restrict__ src, int src_f16, uint64_t rows, float *__restrict__ dst,
                              const uint32_t *__restrict__ tok, int c) {
    const int b = blockIdx.y;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= c) return;
    const size_t row = tok[b];
    if (row >= rows) { dst[(size_t)b * c + i] = 0.0f; return; }
    float v;
    if (src_f16)
        v = (float)((const _Float16 *)src)[row * c + i];
    else
        v = ((const float *)src)[row * c + i];
    dst[(size_t)b * c + i] = v;
}

int launch_gather_rows(rsv_ctx *ctx, const void *src, int src_f16, uint64_t src_rows, float *dst,
                       const uint32_t *tok, int c, int batch) {
    if (batch <= 0) return 0;
    hipLaunchKernelGGL(k_gather_rows, dim3((c + 255) / 256, batch), dim3(256), 0, ctx->stream, src, src_f16,
                       src_rows, dst, tok, c);
    RSV_HIP(hipGetLastError());
    return 0;
}

// ------------------------------------------------------------------ argmax
// Ties go to the smaller index (backend_cuda.rs:3640-3680); the scan starts
// from -1e30 at index 0 like the reference.  grid (batch), block 1024.
// Argmax of one row by a 1024-thread block; the index is valid in thread 0.
__device__ __forceinline__ int argmax_block(const float *__restrict__ lg, int n, float *sv, int *si) {
    const int tid = threadIdx.x;
    float bv = -1e30f;
    int bi = 0;
    if ((n & 3) == 0) {
        // float4 quads q = tid + 1024*j, 8 loads in flight per round; each
        // thread still visits its elements in increasing index order, so the
        // strict compare keeps the smallest index of a tie
        const float4 *l4 = (const float4 *)lg;
        const int n4 = n >> 2;
        for (int q0 = tid; q0 < n4; q0 += 8 * 1024) {
            float4 v[8];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int q = q0 + 1024 * j;
                v[j] = q < n4 ? l4[q] : make_float4(-1e30f, -1e30f, -1e30f, -1e30f);
            }
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int e = 4 * (q0 + 1024 * j);
                if (v[j].x > bv) { bv = v[j].x; bi = e; }
                if (v[j].y > bv) { bv = v[j].y; bi = e + 1; }
                if (v[j].z > bv) { bv = v[j].z; bi = e + 2; }
                if (v[j].w > bv) { bv = v[j].w; bi = e + 3; }
            }
        }
    } else {
        for (int i = tid; i < n; i += 1024) {
            const float v = lg[i];
            if (v > bv) { bv = v; bi = i; }
        }
    }
    wave_argmax_last(bv, bi);
    if ((tid & 63) == 63) { sv[tid >> 6] = bv; si[tid >> 6] = bi; }
    __syncthreads();
    int ix = 0;
    if (tid == 0) {
        float v = sv[0];
        ix = si[0];
        for (int w = 1; w < 16; w++)
            if (sv[w] > v || (sv[w] == v && si[w] < ix)) { v = sv[w]; ix = si[w]; }
    }
    return ix;
}

__global__ __launch_bounds__(1024) void k_argmax(const float *__restrict__ logits, uint32_t *__restrict__ tok,
                                                 int n) {
    __shared__ float sv[16];
    __shared__ int si[16];
    const int b = blockIdx.x;
    const int ix = argmax_block(logits + (size_t)b * n, n, sv, si);
    if (threadIdx.x == 0) tok[b] = (uint32_t)ix;
}

// argmax, then the token's record (k_record_tokens) and the gather of its
// embedding row into x for the next step (k_gather_rows), in one launch:
// the three steps of a greedy self-loop round, with the same results.
__global__ __launch_bounds__(1024) void k_argmax_next(const float *__restrict__ logits, uint32_t *__restrict__ tok,
                                                      int n, uint32_t *__restrict__ out_seq,
                                                      uint32_t *__restrict__ cnt, int stride,
                                                      const void *__restrict__ emb, int emb_f16, uint64_t emb_rows,
                                                      float *__restrict__ x, int c) {
    __shared__ float sv[16];
    __shared__ int si[16];
    __shared__ uint32_t stok;
    const int b = blockIdx.x, tid = threadIdx.x;
    const int ix = argmax_block(logits + (size_t)b * n, n, sv, si);
    if (tid == 0) {
        tok[b] = (uint32_t)ix;
        const uint32_t i = cnt[b];
        if (i < (uint32_t)stride) out_seq[(size_t)b * stride + i] = (uint32_t)ix;
        cnt[b] = i + 1u;
        stok = (uint32_t)ix;
    }
    __syncthreads();
    const size_t row = stok;
    for (int i = tid; i < c; i += 1024) {
        float v = 0.0f;
        if (row < emb_rows) v = emb_f16 ? (float)((const _Float16 *)emb)[row * c + i] : ((const float *)emb)[row * c + i];
        x[(size_t)b * c + i] = v;
    }
}

int launch_argmax_next(rsv_ctx *ctx, const float *logits, uint32_t *tok, int n, uint32_t *out_seq, uint32_t *cnt,
                       int stride, const void *emb, int emb_f16, uint64_t emb_rows, float *x, int c, int batch) {
    if (n <= 0 || batch <= 0 || c <= 0) return RSV_FAIL("argmax_next: bad n=%d c=%d batch=%d", n, c, batch);
    hipLaunchKernelGGL(k_argmax_next, dim3(batch), dim3(1024), 0, ctx->stream, logits, tok, n, out_seq, cnt, stride,
                       emb, emb_f16, emb_rows, x, c);
    RSV_HIP(hipGetLastError());
    return 0;
}

int launch_argmax(rsv_ctx *ctx, const float *logits, uint32_t *tok, int n, int batch) {
    if (n <= 0 || batch <= 0) return RSV_FAIL("argmax: bad n=%d batch=%d", n, batch);
    hipLaunchKernelGGL(k_argmax, dim3(batch), dim3(1024), 0, ctx->stream, logits, tok, n);
    RSV_HIP(hipGetLastError());
    return 0;
}

// ------------------------------------------------------------ token record
// out_seq[b*stride + cnt[b]++] = in_tok[b] (backend.rs:621, 981).  The slot
// is bounded by stride so a replay past the buffer end cannot write outside.
__global__ void k_record_tokens(const uint32_t *__restrict__ in_tok, uint32_t *__restrict__ out_seq,
                                uint32_t *__restrict__ cnt, int stride, int batch) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= batch) return;
    const uint32_t i = cnt[b];
    if (i < (uint32_t)stride) out_seq[(size_t)b * stride + i] = in_tok[b];
    cnt[b] = i + 1u;
}

// k_record_tokens and k_gather_rows of the same tokens in one launch (grid
// (ceil(c/256), batch)): the tail of a sampled self-loop round.
__global__ void k_record_gather(const uint32_t *__restrict__ in_tok, uint32_t *__restrict__ out_seq,
                                uint32_t *__restrict__ cnt, int stride, const void *__restrict__ emb, int emb_f16,
                                uint64_t emb_rows, float *__restrict__ x, int c) {
    const int b = blockIdx.y, i = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t t = in_tok[b];
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        const uint32_t k = cnt[b];
        if (k < (uint32_t)stride) out_seq[(size_t)b * stride + k] = t;
        cnt[b] = k + 1u;
    }
    if (i >= c) return;
    const size_t row = t;
    float v = 0.0f;
    if (row < emb_rows) v = emb_f16 ? (float)((const _Float16 *)emb)[row * c + i] : ((const float *)emb)[row * c + i];
    x[(size_t)b * c + i] = v;
}

int launch_record_gather(rsv_ctx *ctx, const uint32_t *in_tok, uint32_t *out_seq, uint32_t *cnt, int stride,
                         const void *emb, int emb_f16, uint64_t emb_rows, float *x, int c, int batch) {
    if (c <= 0 || batch <= 0) return RSV_FAIL("record_gather: bad c=%d batch=%d", c, batch);
    hipLaunchKernelGGL(k_record_gather, dim3((c + 255) / 256, batch), dim3(256), 0, ctx->stream, in_tok, out_seq,
                       cnt, stride, emb, emb_f16, emb_rows, x, c);
    RSV_HIP(hipGetLastError());
    return 0;
}

int launch_record_tokens(rsv_ctx *ctx, const uint32_t *in_tok, uint32_t *out_seq, uint32_t *cnt, int stride,
                         int batch) {
    hipLaunchKernelGGL(k_record_tokens, dim3((batch + 255) / 256), dim3(256), 0, ctx->stream, in_tok, out_seq,
                       cnt, stride, batch);
    RSV_HIP(hipGetLastError());
    return 0;
}

// --------------------------------------------------- stream-ordered stores
constexpr int kMaxVals = 64;
struct Vals { uint32_t v[kMaxVals]; };

__global__ void k_set_u32(uint32_t *dst, Vals vals, int n) {
    const int i = threadIdx.x;
    if (i < n) dst[i] = vals.v[i];
}

int launch_set_u32(rsv_ctx *ctx, uint32_t *dst, const uint32_t *vals, int n) {
    for (int off = 0; off < n; off += kMaxVals) {
        const int cnt = n - off < kMaxVals ? n - off : kMaxVals;
        Vals v{};
        for (int i = 0; i < cnt; i++) v.v[i] = vals[off + i];
        hipLaunchKernelGGL(k_set_u32, dim3(1), dim3(64), 0, ctx->stream, dst + off, v, cnt);
        RSV_HIP(hipGetLastError());
    }
    return 0;
}

// Sampler row layout (backend_cuda.rs:3700-3718): [T, top_k bits, top_p,
// seed bits, rep, freq, pres, hist_len bits], one row of 8 per slot.
struct SamplerRow { float t; uint32_t k; float p; float rep, freq, pres; uint32_t hist; };
__global__ void k_store_sampler(float *dst, SamplerRow row, Vals seeds, int n) {
    const int b = threadIdx.x;
    if (b >= n) return;
    float *d = dst + (size_t)b * 8;
    d[0] = row.t;
    d[1] = __uint_as_float(row.k);
    d[2] = row.p;
    d[3] = __uint_as_float(seeds.v[b]);
    d[4] = row.rep;
    d[5] = row.freq;
    d[6] = row.pres;
    d[7] = __uint_as_float(row.hist);
}

int launch_store_sampler(rsv_ctx *ctx, float *dst, float temperature, uint32_t top_k, float top_p,
                         const uint32_t *seeds, int batch, float rep, float freq, float pres,
                         uint32_t hist_len) {
    SamplerRow row{temperature, top_k, top_p, rep, freq, pres, hist_len};
    for (int off = 0; off < batch; off += kMaxVals) {
        const int cnt = batch - off < kMaxVals ? batch - off : kMaxVals;
        Vals v{};
        for (int i = 0; i < cnt; i++) v.v[i] = seeds[off + i];
        hipLaunchKernelGGL(k_store_sampler, dim3(1), dim3(64), 0, ctx->stream, dst + (size_t)off * 8, row, v, cnt);
        RSV_HIP(hipGetLastError());
    }
    return 0;
}

// Device-to-device copy as a kernel (not a DMA copy node), so that a
// captured graph holds kernel nodes only: 16-byte words when both ends are
// 16-byte aligned, else bytes.
__global__ __launch_bounds__(256) void k_copy16(const uint4 *__restrict__ src, uint4 *__restrict__ dst, size_t n16) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (size_t)gridDim.x * 256) dst[i] = src[i];
}
__global__ __launch_bounds__(256) void k_copy1(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst, size_t n) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) dst[i] = src[i];
}

int launch_copy(rsv_ctx *ctx, void *dst, const void *src, size_t bytes) {
    if (bytes == 0) return 0;
    const bool al = ((uintptr_t)dst % 16 == 0) && ((uintptr_t)src % 16 == 0);
    const size_t n16 = al ? bytes / 16 : 0, tail = bytes - 16 * n16;
    if (n16) {
        const unsigned blocks = (unsigned)std::min<size_t>(2048, (n16 + 255) / 256);
        hipLaunchKernelGGL(k_copy16, dim3(blocks), dim3(256), 0, ctx->stream, (const uint4 *)src, (uint4 *)dst, n16);
        RSV_HIP(hipGetLastError());
    }
    if (tail) {
        const unsigned blocks = (unsigned)std::min<size_t>(2048, (tail + 255) / 256);
        hipLaunchKernelGGL(k_copy1, dim3(blocks), dim3(256), 0, ctx->stream, (const uint8_t *)src + 16 * n16,
                           (uint8_t *)dst + 16 * n16, tail);
        RSV_HIP(hipGetLastError());
    }
    return 0;
}

// -------------------------------------------------------------- elementwise
// op 0: y = sigmoid(a); 1: y = sigmoid(y); 2: y = exp(a * b[row]); 3: y = a*b
__global__ void k_elementwise(int op, const float *__restrict__ a, const float *__restrict__ b, float *y, int c,
                              int batch) {
    const size_t total = (size_t)c * batch;
    for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (size_t)gridDim.x * blockDim.x) {
        switch (op) {
            case 0: y[e] = sigmoid_m(a[e]); break;
            case 1: y[e] = sigmoid_m(y[e]); break;
            case 2: y[e] = expf(a[e] * b[e / c]); break;
            default: y[e] = a[e] * b[e]; break;
        }
    }
}

int launch_elementwise(rsv_ctx *ctx, int op, const float *a, const float *b, float *y, int c, int batch) {
    const size_t total = (size_t)c * batch;
    if (total == 0) return 0;
    size_t blocks = (total + 255) / 256;
    if (blocks > 16384) blocks = 16384;
    hipLaunchKernelGGL(k_elementwise, dim3((unsigned)blocks), dim3(256), 0, ctx->stream, op, a, b, y, c, batch);
    RSV_HIP(hipGetLastError());
    return 0;
}

// f32 -> f16 rows; rows in [t, m_pad) are zeroed (backend.rs:728).
__global__ void k_to_f16(const float *__restrict__ x, _Float16 *__restrict__ y, int c, int t, int m_pad, int sx,
                         int sy) {
    const int row = blockIdx.y;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < c; i += gridDim.x * blockDim.x)
        y[(size_t)row * sy + i] = row < t ? (_Float16)x[(size_t)row * sx + i] : (_Float16)0.0f;
}

int launch_to_f16(rsv_ctx *ctx, const float *x, _Float16 *y, int c, int t, int m_pad, int x_stride,
                  int y_stride) {
    if (m_pad < t) return RSV_FAIL("to_f16: m_pad %d < t %d", m_pad, t);
    if (m_pad == 0) return 0;
    hipLaunchKernelGGL(k_to_f16, dim3((c + 255) / 256, m_pad), dim3(256), 0, ctx->stream, x, y, c, t, m_pad,
                       x_stride, y_stride);
    RSV_HIP(hipGetLastError());
    return 0;
}

// v = v + gate*(v_first - v), v_first is one [c] row shared by all t rows.
__global__ void k_v_first_lerp(float *v, const float *__restrict__ gate, const float *__restrict__ vf, int c,
                               int t, int stride) {
    const int row = blockIdx.y;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < c; i += gridDim.x * blockDim.x) {
        const size_t o = (size_t)row * stride + i;
        const float cur = v[o];
        v[o] = cur + gate[o] * (vf[i] - cur);
    }
}

int launch_v_first_lerp(rsv_ctx *ctx, float *v, const float *gate, const float *vf, int c, int t, int stride) {
    if (t <= 0) return 0;
    hipLaunchKernelGGL(k_v_first_lerp, dim3((c + 255) / 256, t), dim3(256), 0, ctx->stream, v, gate, vf, c, t,
                       stride);
    RSV_HIP(hipGetLastError());
    return 0;
}

// fuse_ka (backend.rs:765): k_mod, kk_l2, b per token row.  grid (h, batch), block 64.
__global__ __launch_bounds__(64) void k_fuse_ka(const float *__restrict__ k, const float *__restrict__ kk,
                                                const float *__restrict__ a, const float *__restrict__ ka,
                                                float *kmod, float *kkl2, float *bo, int H) {
    const int h = blockIdx.x, b = blockIdx.y, i = threadIdx.x;
    const size_t o = (size_t)b * H * 64 + h * 64 + i;
    const float ki = k[o], ai = a[o];
    const float kkv = ki * kk[h * 64 + i];
    float ss = kkv * kkv;
    ss = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wave_sum_last(ss)), 63));
    float nrm = sqrtf(ss);
    nrm = nrm < 1e-12f ? 1e-12f : nrm;
    const float kh = kkv * (1.0f / nrm);
    kmod[o] = ki + ka[h * 64 + i] * (ki * ai - ki);
    kkl2[o] = kh;
    bo[o] = kh * (-ai);
}

int launch_fuse_ka(rsv_ctx *ctx, const float *k, const float *kk, const float *a, const float *ka,
                   float *kmod, float *kkl2, float *b, int h, int n, int batch) {
    if (n != 64) return RSV_FAIL("fuse_ka: head_size must be 64");
    hipLaunchKernelGGL(k_fuse_ka, dim3(h, batch), dim3(64), 0, ctx->stream, k, kk, a, ka, kmod, kkl2, b, h);
    RSV_HIP(hipGetLastError());
    return 0;
}

// y += sum_j(r*k_mod*r_k) * v per head (backend.rs:780).
__global__ __launch_bounds__(64) void k_sum_rk_rk(const float *__restrict__ r, const float *__restrict__ km,
                                                  const float *__restrict__ rk, const float *__restrict__ v,
                                                  float *y, int H) {
    const int h = blockIdx.x, b = blockIdx.y, i = threadIdx.x;
    const size_t o = (size_t)b * H * 64 + h * 64 + i;
    float s = r[o] * km[o] * rk[h * 64 + i];
    s = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wave_sum_last(s)), 63));
    y[o] += s * v[o];
}

int launch_sum_rk_rk(rsv_ctx *ctx, const float *r, const float *kmod, const float *rk, const float *v,
                     float *y, int h, int n, int batch) {
    if (n != 64) return RSV_FAIL("sum_rk_rk: head_size must be 64");
    hipLaunchKernelGGL(k_sum_rk_rk, dim3(h, batch), dim3(64), 0, ctx->stream, r, kmod, rk, v, y, h);
    RSV_HIP(hipGetLastError());
    return 0;
}

// seq_shift (backend.rs:793, 824): y[t] = x[t] + tm*(x[t-1] - x[t]); the
// previous row of t=0 is the slot's state.  Buffers [batch, t, stride].
__global__ void k_seq_shift(const float *__restrict__ x, const float *__restrict__ st, const float *__restrict__ tm,
                            float *__restrict__ y, int c, int t, int sx, int sy) {
    const int row = blockIdx.y, b = blockIdx.z;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < c; i += gridDim.x * blockDim.x) {
        const float cur = x[((size_t)b * t + row) * sx + i];
        const float prev = row == 0 ? st[(size_t)b * c + i] : x[((size_t)b * t + row - 1) * sx + i];
        y[((size_t)b * t + row) * sy + i] = cur + tm[i] * (prev - cur);
    }
}

int launch_seq_shift(rsv_ctx *ctx, const float *x, const float *state, const float *tm, float *y, int c,
                     int t, int sx, int sy, int batch) {
    if (t <= 0 || batch <= 0) return 0;
    hipLaunchKernelGGL(k_seq_shift, dim3((c + 255) / 256, t, batch), dim3(256), 0, ctx->stream, x, state, tm, y,
                       c, t, sx, sy);
    RSV_HIP(hipGetLastError());
    return 0;
}

// state[b] = x[b, lens[b]-1] (backend.rs:839)
__global__ void k_copy_token_batch(const float *__restrict__ x, float *__restrict__ st,
                                   const uint32_t *__restrict__ lens, int c, int t) {
    const int b = blockIdx.y;
    uint32_t l = lens[b];
    if (l == 0) return;
    if (l > (uint32_t)t) l = t;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < c; i += gridDim.x * blockDim.x)
        st[(size_t)b * c + i] = x[((size_t)b * t + l - 1) * c + i];
}

int launch_copy_token_batch(rsv_ctx *ctx, const float *x, float *state, const uint32_t *lens, int c, int t,
                            int batch) {
    if (batch <= 0) return 0;
    hipLaunchKernelGGL(k_copy_token_batch, dim3((c + 255) / 256, batch), dim3(256), 0, ctx->stream, x, state,
                       lens, c, t);
    RSV_HIP(hipGetLastError());
    return 0;
}

// mean over the first lens[b] rows of x[b] (backend.rs:873)
__global__ void k_segmean(const float *__restrict__ x, float *__restrict__ out, const uint32_t *__restrict__ lens,
                          int c, int t) {
    const int b = blockIdx.y;
    uint32_t l = lens[b];
    if (l > (uint32_t)t) l = t;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < c; i += gridDim.x * blockDim.x) {
        float s = 0.0f;
        for (uint32_t r = 0; r < l; r++) s += x[((size_t)b * t + r) * c + i];
        out[(size_t)b * c + i] = l ? s / (float)l : 0.0f;
    }
}

int launch_segmean(rsv_ctx *ctx, const float *x, float *out, const uint32_t *lens, int c, int t_pad,
                   int batch) {
    if (batch <= 0) return 0;
    hipLaunchKernelGGL(k_segmean, dim3((c + 255) / 256, batch), dim3(256), 0, ctx->stream, x, out, lens, c, t_pad);
    RSV_HIP(hipGetLastError());
    return 0;
}

}  // namespace rsv

namespace rsv {

// ------------------------------------------------ packed prefill token mix
// One block per token row, thread t owning the eight consecutive columns
// 8t .. 8t+7 (c % 8 == 0, c <= 8192; blocks of c/8 threads rounded up to a
// whole wave): 32-byte loads and 16-byte fp16 stores.  LN of the row and of
// its predecessor (or the slot's token-shift state for the first row of a
// segment) with the two rows' sums in one pair of block reductions; outputs
// fp16 GEMM operands.  The state itself is written by k_seq_state_store in a
// separate launch (so no block reads a state row another block rewrites),
// with the same arithmetic per row, so a row's LN is the same value whether
// a later row of its chunk recomputes it or a later chunk reads it back.
constexpr int kLnVec = 8;
constexpr int kLnMaxC = 8192;

// Sums of (v.x, v.y) over the block (wave sums, then the waves in order).
__device__ __forceinline__ float2 block_sum2(float2 v, float2 *red) {
    v.x = wave_sum_last(v.x);
    v.y = wave_sum_last(v.y);
    const int nw = blockDim.x >> 6;
    if ((threadIdx.x & 63) == 63) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float2 t = red[0];
    for (int w = 1; w < nw; w++) {
        t.x += red[w].x;
        t.y += red[w].y;
    }
    __syncthreads();  // red is reused by the next call
    return t;
}

__device__ __forceinline__ void ld8(const float *p, float (&v)[kLnVec]) {
    const float4 a = ((const float4 *)p)[0], b = ((const float4 *)p)[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

// LayerNorm of two rows at once (a and b; model.rs:402-411), each row's
// statistics two-pass over its own values; on return a and b hold the
// normalised rows.  Lanes past c hold zeros and take no part.
__device__ __forceinline__ void ln_pair(float (&a)[kLnVec], float (&b)[kLnVec], const float (&gm)[kLnVec],
                                        const float (&bt)[kLnVec], bool live, int C, float eps, float2 *red) {
    float2 s = make_float2(0.0f, 0.0f);
#pragma unroll
    for (int e = 0; e < kLnVec; e++) {
        s.x += a[e];
        s.y += b[e];
    }
    s = block_sum2(s, red);
    const float ma = s.x / (float)C, mb = s.y / (float)C;
    float2 q = make_float2(0.0f, 0.0f);
    if (live) {
#pragma unroll
        for (int e = 0; e < kLnVec; e++) {
            const float da = a[e] - ma, db = b[e] - mb;
            q.x += da * da;
            q.y += db * db;
        }
    }
    q = block_sum2(q, red);
    const float ia = 1.0f / sqrtf(q.x / (float)C + eps), ib = 1.0f / sqrtf(q.y / (float)C + eps);
#pragma unroll
    for (int e = 0; e < kLnVec; e++) {
        a[e] = (a[e] - ma) * ia * gm[e] + bt[e];
        b[e] = (b[e] - mb) * ib * gm[e] + bt[e];
    }
}

struct HOut6 { _Float16 *p[6]; };

__global__ __launch_bounds__(1024) void k_seq_norm_mix(const float *__restrict__ x, const float *__restrict__ state,
                                                       const float *__restrict__ gamma, const float *__restrict__ beta,
                                                       Ptr6 coef, HOut6 out, int nout,
                                                       const uint32_t *__restrict__ row_prev, int C, uint64_t slots,
                                                       float eps) {
    __shared__ float2 red[16];
    const int t = blockIdx.x, c0 = threadIdx.x * kLnVec;
    const bool live = c0 < C;
    const uint32_t p = row_prev[t];
    const bool from_state = (p & 0x80000000u) != 0;
    const uint32_t slot = p & 0x7FFFFFFFu;
    // every load first: this row, its predecessor (raw x, or the LN'd state
    // row), gamma / beta and the mix coefficients
    float xa[kLnVec] = {}, xb[kLnVec] = {}, gm[kLnVec] = {}, bt[kLnVec] = {}, cf[6][kLnVec];
    if (live) {
        ld8(x + (size_t)t * C + c0, xa);
        if (!from_state) ld8(x + (size_t)p * C + c0, xb);
        else if (slot < slots) ld8(state + (size_t)slot * C + c0, xb);
        ld8(gamma + c0, gm);
        ld8(beta + c0, bt);
#pragma unroll
        for (int j = 0; j < 6; j++)
            if (j < nout) ld8(coef.p[j] + c0, cf[j]);
    }
    float pv[kLnVec];
#pragma unroll
    for (int e = 0; e < kLnVec; e++) pv[e] = xb[e];
    ln_pair(xa, xb, gm, bt, live, C, eps, red);  // uniform per block: the barriers inside
    if (!from_state) {
#pragma unroll
        for (int e = 0; e < kLnVec; e++) pv[e] = xb[e];
    }
    if (!live) return;
#pragma unroll
    for (int j = 0; j < 6; j++) {
        if (j >= nout) break;
        typedef _Float16 h8 __attribute__((ext_vector_type(8)));
        h8 o;
#pragma unroll
        for (int e = 0; e < kLnVec; e++) o[e] = (_Float16)(xa[e] + cf[j][e] * (pv[e] - xa[e]));
        *(h8 *)(out.p[j] + (size_t)t * C + c0) = o;
    }
}

static int ln_threads(int c) { return ((c / kLnVec + 63) / 64) * 64; }

int launch_seq_norm_mix(rsv_ctx *ctx, const float *x, const float *state, const float *gamma, const float *beta,
                        const float *const *coef, _Float16 *const *out, int nout, const uint32_t *row_prev, int t,
                        int c, uint64_t slots, float eps) {
    if (c <= 0 || c > kLnMaxC || c % kLnVec) return RSV_FAIL("seq_norm_mix: c=%d must be a multiple of 8 in 8..%d", c, kLnMaxC);
    if (nout < 1 || nout > 6) return RSV_FAIL("seq_norm_mix: nout=%d", nout);
    if (t <= 0) return 0;
    Ptr6 cp{};
    HOut6 op{};
    for (int j = 0; j < nout; j++) { cp.p[j] = coef[j]; op.p[j] = out[j]; }
    hipLaunchKernelGGL(k_seq_norm_mix, dim3(t), dim3(ln_threads(c)), 0, ctx->stream, x, state, gamma, beta, cp, op, nout,
                       row_prev, c, slots, eps);
    RSV_HIP(hipGetLastError());
    return 0;
}

__global__ __launch_bounds__(1024) void k_seq_state_store(const float *__restrict__ x, float *__restrict__ state,
                                                          const float *__restrict__ gamma,
                                                          const float *__restrict__ beta,
                                                          const uint32_t *__restrict__ seg_last,
                                                          const uint32_t *__restrict__ seg_slot, int C, uint64_t rows,
                                                          uint64_t slots, float eps) {
    __shared__ float2 red[16];
    const int g = blockIdx.x, c0 = threadIdx.x * kLnVec;
    const bool live = c0 < C;
    const uint32_t row = seg_last[g], slot = seg_slot[g];
    if (row >= rows || slot >= slots) return;  // uniform per block
    float xa[kLnVec] = {}, xb[kLnVec] = {}, gm[kLnVec] = {}, bt[kLnVec] = {};
    if (live) {
        ld8(x + (size_t)row * C + c0, xa);
        ld8(gamma + c0, gm);
        ld8(beta + c0, bt);
    }
    ln_pair(xa, xb, gm, bt, live, C, eps, red);
    if (!live) return;
    float4 *dst = (float4 *)(state + (size_t)slot * C + c0);
    dst[0] = make_float4(xa[0], xa[1], xa[2], xa[3]);
    dst[1] = make_float4(xa[4], xa[5], xa[6], xa[7]);
}

int launch_seq_state_store(rsv_ctx *ctx, const float *x, float *state, const float *gamma, const float *beta,
                           const uint32_t *seg_last, const uint32_t *seg_slot, int nseg, int c, uint64_t rows,
                           uint64_t slots, float eps) {
    if (c <= 0 || c > kLnMaxC || c % kLnVec) return RSV_FAIL("seq_state_store: c=%d must be a multiple of 8 in 8..%d", c, kLnMaxC);
    if (nseg <= 0) return 0;
    hipLaunchKernelGGL(k_seq_state_store, dim3(nseg), dim3(ln_threads(c)), 0, ctx->stream, x, state, gamma, beta,
                       seg_last, seg_slot, c, rows, slots, eps);
    RSV_HIP(hipGetLastError());
    return 0;
}

__global__ void k_copy_rows(const float *__restrict__ src, float *__restrict__ dst, const uint32_t *__restrict__ sr,
                            const uint32_t *__restrict__ dr, int c, uint64_t src_n, uint64_t dst_n) {
    const int r = blockIdx.y;
    const uint32_t s = sr[r], d = dr[r];
    if (s >= src_n || d >= dst_n) return;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < c; i += gridDim.x * blockDim.x)
        dst[(size_t)d * c + i] = src[(size_t)s * c + i];
}

int launch_copy_rows(rsv_ctx *ctx, const float *src, float *dst, const uint32_t *src_rows, const uint32_t *dst_rows,
                     int n, int c, uint64_t src_n, uint64_t dst_n) {
    if (n <= 0) return 0;
    hipLaunchKernelGGL(k_copy_rows, dim3((c + 255) / 256, n), dim3(256), 0, ctx->stream, src, dst, src_rows,
                       dst_rows, c, src_n, dst_n);
    RSV_HIP(hipGetLastError());
    return 0;
}

__global__ void k_mul_to_f16(const float *__restrict__ a, const float *__restrict__ b, _Float16 *__restrict__ y,
                             uint64_t n) {
    for (uint64_t e = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n; e += (uint64_t)gridDim.x * blockDim.x)
        y[e] = (_Float16)(a[e] * b[e]);
}

int launch_mul_to_f16(rsv_ctx *ctx, const float *a, const float *b, _Float16 *y, uint64_t n) {
    if (n == 0) return 0;
    uint64_t blocks = (n + 255) / 256;
    if (blocks > 16384) blocks = 16384;
    hipLaunchKernelGGL(k_mul_to_f16, dim3((unsigned)blocks), dim3(256), 0, ctx->stream, a, b, y, n);
    RSV_HIP(hipGetLastError());
    return 0;
}

}  // namespace rsv

namespace rsv {

// LayerNorm of each batch row + up to six token-shift mixes written as fp16
// GEMM operands (batched decode on matrix cores).  With coef[j] == null the
// output is the plain LN row.  state (optional) is read as the previous
// token's LN row and overwritten with this row.  c <= 4096.
template <int NOUT>
__global__ __launch_bounds__(1024) void k_ln_mix_f16(const float *__restrict__ x, float *__restrict__ state,
                                                     const float *__restrict__ gamma,
                                                     const float *__restrict__ beta, Ptr6 coef, HOut6 out, int C,
                                                     float eps, const float *__restrict__ part, int nsl,
                                                     size_t pstride, float *__restrict__ xout) {
    // grid (batch, parts): block (b, y) writes elements [y*plen, (y+1)*plen)
    // of row b (plen <= 1024) and takes the row statistics itself.  Every
    // load of the block (the whole row of x, and gamma/beta/state/coef of its
    // share) is issued before the statistics.
    __shared__ float red[16];
    const int b = blockIdx.x, tid = threadIdx.x;
    const int plen = (C + gridDim.y - 1) / gridDim.y;
    const int i = blockIdx.y * plen + tid;
    const bool mine = tid < plen && i < C;
    const size_t o = (size_t)b * C + i;
    constexpr int PER = 4;
    float xv[PER];
#pragma unroll
    for (int m = 0; m < PER; m++) {
        const int e = tid + 1024 * m;
        xv[m] = e < C ? x[(size_t)b * C + e] : 0.0f;
    }
    float xi = mine ? x[o] : 0.0f;
    if (part) {
        // x + the k-slice partial sums of the previous GEMM (at most 4),
        // summed in slice order (missing slices read as 0, which adds
        // nothing); every load is issued before the first sum.  The block
        // owning element i stores the new row to xout (another buffer: the
        // other blocks of the row still read x)
        float pv[PER + 1][4];
#pragma unroll
        for (int m = 0; m <= PER; m++) {
            const int e = m < PER ? tid + 1024 * m : i;
            const bool ok = m < PER ? e < C : mine;
#pragma unroll
            for (int q = 0; q < 4; q++)
                pv[m][q] = ok && q < nsl ? part[(size_t)b * C + e + q * pstride] : 0.0f;
        }
#pragma unroll
        for (int m = 0; m < PER; m++) xv[m] += ((pv[m][0] + pv[m][1]) + pv[m][2]) + pv[m][3];
        xi += ((pv[PER][0] + pv[PER][1]) + pv[PER][2]) + pv[PER][3];
        if (mine && xout) xout[o] = xi;
    }
    const float gi = mine ? gamma[i] : 0.0f, bi = mine ? beta[i] : 0.0f;
    const float pi = (mine && state) ? state[o] : 0.0f;
    float ci[NOUT];
#pragma unroll
    for (int j = 0; j < NOUT; j++) ci[j] = (mine && coef.p[j]) ? coef.p[j][i] : 0.0f;
    float s = 0.0f;
#pragma unroll
    for (int m = 0; m < PER; m++) s += xv[m];
    s = wave_sum_last(s);
    if ((tid & 63) == 63) red[tid >> 6] = s;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int w = 0; w < 16; w++) tot += red[w];
    const float mean = tot / (float)C;
    float q = 0.0f;
#pragma unroll
    for (int m = 0; m < PER; m++) {
        const float d = xv[m] - mean;
        q += (tid + 1024 * m < C) ? d * d : 0.0f;
    }
    q = wave_sum_last(q);
    __syncthreads();
    if ((tid & 63) == 63) red[tid >> 6] = q;
    __syncthreads();
    float qt = 0.0f;
#pragma unroll
    for (int w = 0; w < 16; w++) qt += red[w];
    const float inv = 1.0f / sqrtf(qt / (float)C + eps);
    if (!mine) return;
    const float ln = (xi - mean) * inv * gi + bi;
#pragma unroll
    for (int j = 0; j < NOUT; j++) out.p[j][o] = (_Float16)(coef.p[j] ? ln + ci[j] * (pi - ln) : ln);
    if (state) state[o] = ln;
}

int launch_ln_mix_f16(rsv_ctx *ctx, const float *x, float *state, const float *gamma, const float *beta,
                      const float *const *coef, _Float16 *const *out, int nout, int c, float eps, int batch,
                      const float *part, int nsl, float *xout) {
    if (c <= 0 || c > 4096) return RSV_FAIL("ln_mix_f16: c=%d outside 1..4096", c);
    if (part && (nsl < 1 || nsl > 4)) return RSV_FAIL("ln_mix_f16: %d partial slices outside 1..4", nsl);
    const size_t pstride = (size_t)batch * c;
    if (batch <= 0) return 0;
    Ptr6 cp{};
    HOut6 op{};
    for (int j = 0; j < nout; j++) { cp.p[j] = coef ? coef[j] : nullptr; op.p[j] = out[j]; }
    // a row is split over up to 8 blocks (each takes the row statistics
    // itself and writes its share) so that the launch covers the CUs
    const int cus = ctx->sm_count > 0 ? ctx->sm_count : 256;
    int parts = std::min(8, std::max(1, (cus + batch - 1) / batch));
    while ((c + parts - 1) / parts > 1024) parts++;
    const dim3 grid(batch, parts);
    switch (nout) {
        case 1: hipLaunchKernelGGL(k_ln_mix_f16<1>, grid, dim3(1024), 0, ctx->stream, x, state, gamma, beta, cp, op, c, eps, part, nsl, pstride, xout); break;
        case 6: hipLaunchKernelGGL(k_ln_mix_f16<6>, grid, dim3(1024), 0, ctx->stream, x, state, gamma, beta, cp, op, c, eps, part, nsl, pstride, xout); break;
        default: return RSV_FAIL("ln_mix_f16: nout must be 1 or 6 (got %d)", nout);
    }
    RSV_HIP(hipGetLastError());
    return 0;
}

}  // namespace rsv
