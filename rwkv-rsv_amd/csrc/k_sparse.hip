// Sparse ffn.value projection: x[b, c] += sum over f with r2[b, f] != 0 of
// r2[b, f] * V[c, f] (backend.rs:417-441, backend_cuda.rs:3563-3635).  r2 is
// the relu^2 output, so whole rows f of V^T can be skipped.  V is read from
// the reference's tiled fp16 copy (gpu_model.rs:3290-3340): element (f, c) at
// [f/128][c/256][f%128][c%256], so a non-zero f is one contiguous 512-byte
// row of 256 outputs.
//
// Grid (C/256 column blocks, F-ranges, sessions).  A block loads the r2 of
// its whole F-range, compacts the non-zero f with wave ballots and streams
// those rows with four loads in flight per thread; thread t owns output
// column t of the block.  The F-range partials meet in a workspace and a
// second launch adds them to x in range order, so the result does not depend
// on scheduling (the reference adds with atomics).
#include "rsv_common.h"
#include <algorithm>

namespace rsv {
namespace {

constexpr int kFT = 128;  // f rows per tile
constexpr int kCT = 256;  // output columns per tile

__device__ __forceinline__ float h2f_s(uint32_t b) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(b & 0xFFFFu)); }

// tiled[o] for o = ((f_block * cb + c_block) * 128 + f_local) * 256 + c_local
// from V[c, f] (int8 idx/sz with the dequant of model.rs:234-252, or fp16).
__global__ void k_tile_ffn_value(const uint8_t *__restrict__ idx, const uint32_t *__restrict__ sz,
                                 const _Float16 *__restrict__ w16, _Float16 *__restrict__ out, int c, int fh) {
    const int cb = c / kCT;
    const size_t total = (size_t)c * fh;
    for (size_t o = (size_t)blockIdx.x * blockDim.x + threadIdx.x; o < total; o += (size_t)gridDim.x * blockDim.x) {
        const size_t tile = o / (kFT * kCT);
        const int rem = (int)(o - tile * (kFT * kCT));
        const int f = (int)(tile / cb) * kFT + rem / kCT;
        const int cc = (int)(tile % cb) * kCT + rem % kCT;
        float v;
        if (w16) {
            v = (float)w16[(size_t)cc * fh + f];
        } else {
            const uint32_t s = sz[(size_t)cc * (fh / 128) + f / 128];
            const float q = (float)idx[(size_t)cc * fh + f];
            v = __fadd_rn(__fmul_rn(h2f_s(s), q), h2f_s(s >> 16));
        }
        out[o] = (_Float16)v;
    }
}

constexpr int kSpMaxF = 2048;  // f values one block compacts (its share of fh)

// grid (c/256, S, batch).  Block (cb, s, b) handles f in [s*per, (s+1)*per)
// for output columns cb*256 .. +255 of session b.  With S == 1 the block adds
// its sum to x; with S > 1 it stores its partial to ws[b][s][col] and the
// second launch, k_ffn_sparse_reduce, adds the S partials in s order.  The
// kernel boundary between the two launches orders the partial stores before
// their loads on every XCD (a launch ends with its writes flushed to the
// device-coherent level), so no in-kernel cross-block handshake is needed.
__global__ __launch_bounds__(256) void k_ffn_sparse(const float *__restrict__ r2, const _Float16 *__restrict__ vt,
                                                    float *__restrict__ x, float *__restrict__ ws, int c, int fh,
                                                    int per) {
    __shared__ float rs[kSpMaxF];
    __shared__ short ids[kSpMaxF];
    __shared__ int wcnt[4];
    __shared__ int base_n;
    const int c_block = blockIdx.x, s = blockIdx.y, b = blockIdx.z, S = gridDim.y, cbn = gridDim.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int f0 = s * per, f1 = min(fh, f0 + per);
    const float *r2b = r2 + (size_t)b * fh;
    // 1. r2 of the whole range first, then the compaction of its non-zero f (ascending)
    float rv[kSpMaxF / 256];
#pragma unroll
    for (int i = 0; i < kSpMaxF / 256; i++) {
        const int f = f0 + tid + 256 * i;
        rv[i] = f < f1 ? r2b[f] : 0.0f;
    }
    if (tid == 0) base_n = 0;
    for (int i = 0; i < kSpMaxF / 256; i++) {
        if (f0 + 256 * i >= f1) break;
        const bool nz = rv[i] != 0.0f;
        const unsigned long long m = __ballot(nz);
        __syncthreads();
        if (lane == 0) wcnt[wave] = __popcll(m);
        __syncthreads();
        int pre = base_n;
        for (int w = 0; w < wave; w++) pre += wcnt[w];
        if (nz) {
            const int k = pre + __popcll(m & ((1ull << lane) - 1ull));
            ids[k] = (short)(tid + 256 * i);
            rs[k] = rv[i];
        }
        __syncthreads();
        if (tid == 0) base_n += wcnt[0] + wcnt[1] + wcnt[2] + wcnt[3];
    }
    __syncthreads();
    const int nnz = base_n;
    // 2. the non-zero rows: thread tid reads 16 bytes (8 columns, group tid % 32) of rows
    // tid / 32, tid / 32 + 8, ... with four rows in flight; the 8 row slots meet in LDS
    typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
    const int slot = tid >> 5, cg = tid & 31;
    float a8[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    const _Float16 *colp = vt + (size_t)c_block * kFT * kCT + cg * 8;
    for (int i = slot; i < nnz; i += 32) {
        u32x4_t w[4];
        float a[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int k = i + 8 * u < nnz ? i + 8 * u : slot;
            const int f = f0 + ids[k];
            w[u] = *(const u32x4_t *)(colp + ((size_t)(f / kFT) * cbn * kFT + (f % kFT)) * kCT);
            a[u] = i + 8 * u < nnz ? rs[k] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < 4; u++)
#pragma unroll
            for (int h = 0; h < 4; h++) {
                const uint32_t q = w[u][h];
                a8[2 * h] = fmaf(a[u], (float)__builtin_bit_cast(_Float16, (uint16_t)(q & 0xFFFFu)), a8[2 * h]);
                a8[2 * h + 1] = fmaf(a[u], (float)__builtin_bit_cast(_Float16, (uint16_t)(q >> 16)), a8[2 * h + 1]);
            }
    }
    __syncthreads();  // rs is dead: it holds the slot partials now
#pragma unroll
    for (int e = 0; e < 8; e++) rs[slot * 256 + cg * 8 + e] = a8[e];
    __syncthreads();
    float acc = 0.0f;
#pragma unroll
    for (int q = 0; q < 8; q++) acc += rs[q * 256 + tid];
    const int col = c_block * kCT + tid;
    float *xb = x + (size_t)b * c;
    if (S == 1) {
        xb[col] += acc;
        return;
    }
    ws[((size_t)(b * S + s)) * c + col] = acc;
}

// x[b][col] += ((ws[b][0][col] + ws[b][1][col]) + ...) in s order: the same
// sum for every scheduling of the partial launch.
__global__ __launch_bounds__(256) void k_ffn_sparse_reduce(const float *__restrict__ ws, float *__restrict__ x, int c,
                                                           int S, int batch) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= c * batch) return;
    const int b = i / c, col = i - b * c;
    const float *p = ws + (size_t)b * S * c + col;
    float sum = 0.0f;
    for (int q0 = 0; q0 < S; q0 += 8) {
        float pv[8];
#pragma unroll
        for (int q = 0; q < 8; q++) pv[q] = q0 + q < S ? p[(size_t)(q0 + q) * c] : 0.0f;
#pragma unroll
        for (int q = 0; q < 8; q++)
            if (q0 + q < S) sum += pv[q];
    }
    x[i] += sum;
}

}  // namespace

int launch_tile_ffn_value(rsv_ctx *ctx, const uint8_t *idx, const uint32_t *sz, const _Float16 *w16, _Float16 *out,
                          int c, int fh) {
    if (c % kCT || fh % kFT) return RSV_FAIL("tile_ffn_value: c=%d must be a multiple of 256, fh=%d of 128", c, fh);
    hipLaunchKernelGGL(k_tile_ffn_value, dim3(4096), dim3(256), 0, ctx->stream, idx, sz, w16, out, c, fh);
    RSV_HIP(hipGetLastError());
    return 0;
}

int launch_ffn_sparse(rsv_ctx *ctx, const float *r2, const _Float16 *vt, float *x, int c, int fh, int batch) {
    if (c % kCT || fh % kFT) return RSV_FAIL("ffn_value_sparse_add: c=%d must be a multiple of 256, fh=%d of 128", c, fh);
    if (batch <= 0 || batch > 65535) return RSV_FAIL("ffn_value_sparse_add: batch %d", batch);
    const int cbn = c / kCT;
    // about one block per CU over all sessions, each f-range at most kSpMaxF long
    const int cus = ctx->sm_count > 0 ? ctx->sm_count : 256;
    int S = std::max(1, (cus + cbn * batch - 1) / (cbn * batch));
    S = std::max(S, (fh + kSpMaxF - 1) / kSpMaxF);
    S = std::min(S, fh / kFT);
    const int per = (fh + S - 1) / S;
    S = (fh + per - 1) / per;
    const size_t need = (size_t)S * batch * c;
    if (S > 1 && need > ctx->skinny_ws_cap)
        return RSV_FAIL("ffn_value_sparse_add: workspace too small for batch %d", batch);
    hipLaunchKernelGGL(k_ffn_sparse, dim3(cbn, S, batch), dim3(256), 0, ctx->stream, r2, vt, x, ctx->skinny_ws, c, fh,
                       per);
    RSV_HIP(hipGetLastError());
    if (S > 1) {
        hipLaunchKernelGGL(k_ffn_sparse_reduce, dim3((c * batch + 255) / 256), dim3(256), 0, ctx->stream,
                           (const float *)ctx->skinny_ws, x, c, S, batch);
        RSV_HIP(hipGetLastError());
    }
    return 0;
}

}  // namespace rsv
