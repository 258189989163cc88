// Fused WKV7 time-mix kernels.  One 64-lane wavefront owns one 64x64 fp32
// head state; lane i owns state row i.  Per-token vectors (k_hat, b, w,
// k_mod, r) live in LDS and are read as broadcasts; row reductions are local
// to a lane, head reductions (L2 norm, GroupNorm, bonus term) are
// cross-lane butterflies.
//
// Math (model.rs:445-473, 716-826):
//   kk    = k * k_k;  k_hat = kk / max(||kk||, eps)      (per head)
//   k_mod = k + k_a * (k*a - k);  b = -k_hat * a
//   S     = S diag(w) + (S k_hat) b^T + v k_mod^T
//   y     = S r;  yn = GroupNorm(y) + (sum r*k_mod*r_k) * v
// The L2 norm uses the true per-head sum of squares (the CPU path), not the
// doubled sum of the reference's 2-threads-per-row GPU kernels.
#include "rsv_common.h"

namespace rsv {

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

struct HeadVecs {
    float kh[64], bv[64], wv[64], km[64], rv[64];
};

// Builds the per-token vectors of lane j's channel into LDS and returns
// (k_mod_j, r_j, v_j) for later use.  Caller synchronises.
__device__ __forceinline__ void head_vectors(HeadVecs &hv, int j, float k, float kkc, float a, float ka,
                                             float r, float w, float eps, float &kmod) {
    const float kk = k * kkc;
    const float ss = wave_sum(kk * kk);
    float nrm = sqrtf(ss);
    nrm = nrm < eps ? eps : nrm;
    const float inv = 1.0f / nrm;
    const float kh = kk * inv;
    kmod = k + ka * (k * a - k);
    hv.kh[j] = kh;
    hv.bv[j] = kh * (-a);
    hv.wv[j] = w;
    hv.km[j] = kmod;
    hv.rv[j] = r;
}

// Lane i: row update + y_i = S_i . r (row held in registers).
__device__ __forceinline__ float row_update(float (&s)[64], const HeadVecs &hv, float vi) {
    float sa = 0.0f;
#pragma unroll
    for (int j = 0; j < 64; j++) sa = fmaf(s[j], hv.kh[j], sa);
    float y = 0.0f;
#pragma unroll
    for (int j = 0; j < 64; j++) {
        const float ns = s[j] * hv.wv[j] + sa * hv.bv[j] + vi * hv.km[j];
        s[j] = ns;
        y = fmaf(ns, hv.rv[j], y);
    }
    return y;
}

// GroupNorm over the 64 lanes (two-pass, eps inside sqrt) + bonus term.
__device__ __forceinline__ float head_norm(float y, float gamma, float beta, float bonus_part, float vi,
                                           float gn_eps) {
    const float mean = wave_sum(y) * (1.0f / 64.0f);
    const float d = y - mean;
    const float var = wave_sum(d * d) * (1.0f / 64.0f) + gn_eps;
    const float inv_std = 1.0f / sqrtf(var);
    const float bonus = wave_sum(bonus_part);
    return d * inv_std * gamma + beta + bonus * vi;
}

// ------------------------------------------------------------- decode step
// grid (H, B), block 64.  State [B, H, 64, 64] is read and written with
// coalesced 16-byte accesses through an LDS transpose tile.
__global__ __launch_bounds__(64) void k_wkv7_decode(float *__restrict__ S, const float *__restrict__ k,
                                                    const float *__restrict__ kkc, const float *__restrict__ a,
                                                    const float *__restrict__ ka, const float *__restrict__ r,
                                                    const float *__restrict__ v, const float *__restrict__ w,
                                                    const float *__restrict__ gamma,
                                                    const float *__restrict__ beta,
                                                    const float *__restrict__ rk, float *__restrict__ kmod_out,
                                                    float *__restrict__ y_out, float *__restrict__ yn_out,
                                                    int H, float eps, float gn_eps,
                                                    const float *__restrict__ gmul, _Float16 *__restrict__ yg16) {
    __shared__ float tile[64 * 65];
    __shared__ HeadVecs hv;
    const int h = blockIdx.x, b = blockIdx.y, i = threadIdx.x;
    const size_t C = (size_t)H * 64;
    const size_t vo = (size_t)b * C + (size_t)h * 64;
    float4 *Sg = (float4 *)(S + ((size_t)b * H + h) * 4096);

    // issue the state loads first; they do not depend on the vectors
    float4 st[16];
#pragma unroll
    for (int m = 0; m < 16; m++) st[m] = Sg[m * 64 + i];

    const float ki = k[vo + i], ai = a[vo + i], ri = r[vo + i], vi_own = v[vo + i], wi = w[vo + i];
    float kmod;
    head_vectors(hv, i, ki, kkc[h * 64 + i], ai, ka[h * 64 + i], ri, wi, eps, kmod);
    if (kmod_out) kmod_out[vo + i] = kmod;

#pragma unroll
    for (int m = 0; m < 16; m++) {
        const int e = (m * 64 + i) * 4, row = e >> 6, col = e & 63;
        tile[row * 65 + col + 0] = st[m].x;
        tile[row * 65 + col + 1] = st[m].y;
        tile[row * 65 + col + 2] = st[m].z;
        tile[row * 65 + col + 3] = st[m].w;
    }
    __syncthreads();
    float s[64];
#pragma unroll
    for (int j = 0; j < 64; j++) s[j] = tile[i * 65 + j];
    const float y = row_update(s, hv, vi_own);
    // GroupNorm and the bonus term need every lane's y; the row write-back
    // goes through the tile again.
#pragma unroll
    for (int j = 0; j < 64; j++) tile[i * 65 + j] = s[j];
    const float yn = head_norm(y, gamma[h * 64 + i], beta[h * 64 + i], ri * kmod * rk[h * 64 + i], vi_own, gn_eps);
    if (y_out) y_out[vo + i] = y;
    if (yn_out) yn_out[vo + i] = yn;
    if (yg16) yg16[vo + i] = (_Float16)(yn * gmul[vo + i]);  // att.output operand (y_norm * g)
    __syncthreads();
#pragma unroll
    for (int m = 0; m < 16; m++) {
        const int e = (m * 64 + i) * 4, row = e >> 6, col = e & 63;
        Sg[m * 64 + i] = make_float4(tile[row * 65 + col], tile[row * 65 + col + 1], tile[row * 65 + col + 2],
                                     tile[row * 65 + col + 3]);
    }
}

int launch_wkv7_decode(rsv_ctx *ctx, float *s, const float *k, const float *kk, const float *a,
                       const float *ka, const float *r, const float *v, const float *w,
                       const float *gamma, const float *beta, const float *rk, float *kmod, float *y,
                       float *yn, int h, int n, float eps, float gn_eps, int batch, const float *gmul,
                       _Float16 *yg16) {
    if (n != 64) return RSV_FAIL("wkv7: head_size must be 64 (got %d)", n);
    if (h <= 0 || batch <= 0) return RSV_FAIL("wkv7: bad h=%d batch=%d", h, batch);
    if ((yg16 != nullptr) != (gmul != nullptr)) return RSV_FAIL("wkv7: y*g output needs g");
    if (!yn && !yg16) return RSV_FAIL("wkv7: no output");
    hipLaunchKernelGGL(k_wkv7_decode, dim3(h, batch), dim3(64), 0, ctx->stream, s, k, kk, a, ka, r, v, w,
                       gamma, beta, rk, kmod, y, yn, h, eps, gn_eps, gmul, yg16);
    RSV_HIP(hipGetLastError());
    return 0;
}

// ------------------------------------------------------ ragged prefill scan
// grid (H, nseg), block 64.  Segment g covers packed token rows
// [seg_start[g], seg_start[g]+seg_len[g]) and state slot seg_slot[g]; the
// state row stays in VGPRs for the whole segment.
__global__ __launch_bounds__(64) void k_wkv7_seq_ragged(
    float *__restrict__ S, const float *__restrict__ r, const float *__restrict__ w, const float *__restrict__ k,
    const float *__restrict__ v, const float *__restrict__ a, const float *__restrict__ kkc,
    const float *__restrict__ ka, const float *__restrict__ rk, const float *__restrict__ gamma,
    const float *__restrict__ beta, float *__restrict__ yn_out, const uint32_t *__restrict__ seg_start,
    const uint32_t *__restrict__ seg_len, const uint32_t *__restrict__ seg_slot, int H, float eps,
    float gn_eps, uint64_t rows, uint64_t slots) {
    __shared__ HeadVecs hv;
    const int h = blockIdx.x, g = blockIdx.y, i = threadIdx.x;
    const size_t C = (size_t)H * 64;
    const uint32_t t0 = seg_start[g], len = seg_len[g], slot = seg_slot[g];
    // segments outside the packed buffers or the state are skipped (uniform per block)
    if (slot >= slots || (uint64_t)t0 + len > rows) return;
    float4 *Srow = (float4 *)(S + ((size_t)slot * H + h) * 4096 + (size_t)i * 64);
    float s[64];
#pragma unroll
    for (int m = 0; m < 16; m++) {
        const float4 t = Srow[m];
        s[4 * m] = t.x; s[4 * m + 1] = t.y; s[4 * m + 2] = t.z; s[4 * m + 3] = t.w;
    }
    const float kkc_i = kkc[h * 64 + i], ka_i = ka[h * 64 + i], rk_i = rk[h * 64 + i];
    const float gm_i = gamma[h * 64 + i], bt_i = beta[h * 64 + i];
    for (uint32_t t = 0; t < len; t++) {
        const size_t vo = (size_t)(t0 + t) * C + (size_t)h * 64;
        const float ki = k[vo + i], ai = a[vo + i], ri = r[vo + i], vi = v[vo + i], wi = w[vo + i];
        float kmod;
        __syncthreads();  // previous token's readers are done with hv
        head_vectors(hv, i, ki, kkc_i, ai, ka_i, ri, wi, eps, kmod);
        __syncthreads();
        const float y = row_update(s, hv, vi);
        yn_out[vo + i] = head_norm(y, gm_i, bt_i, ri * kmod * rk_i, vi, gn_eps);
    }
#pragma unroll
    for (int m = 0; m < 16; m++) Srow[m] = make_float4(s[4 * m], s[4 * m + 1], s[4 * m + 2], s[4 * m + 3]);
}

int launch_wkv7_seq_ragged(rsv_ctx *ctx, float *s, const float *r, const float *w, const float *k,
                           const float *v, const float *a, const float *kk, const float *ka,
                           const float *rk, const float *gamma, const float *beta, float *yn,
                           const uint32_t *seg_start, const uint32_t *seg_len,
                           const uint32_t *seg_slot, int nseg, int h, int n, float gn_eps, uint64_t rows,
                           uint64_t slots) {
    if (n != 64) return RSV_FAIL("wkv7_seq: head_size must be 64 (got %d)", n);
    if (nseg <= 0) return 0;
    hipLaunchKernelGGL(k_wkv7_seq_ragged, dim3(h, nseg), dim3(64), 0, ctx->stream, s, r, w, k, v, a, kk, ka,
                       rk, gamma, beta, yn, seg_start, seg_len, seg_slot, h, 1e-12f, gn_eps, rows, slots);
    RSV_HIP(hipGetLastError());
    return 0;
}

// ------------------------------------------- dplr_seq (backend.rs:806, 852)
// Vectors are precomputed per token: k = k_mod, a = k_hat, b = -k_hat*a.
// y[t] = S_t r_t.  lens (optional) truncates each slot's token count; the
// buffers are [batch, t, c].
__global__ __launch_bounds__(64) void k_dplr_seq(float *__restrict__ S, const float *__restrict__ r,
                                                 const float *__restrict__ w, const float *__restrict__ k,
                                                 const float *__restrict__ v, const float *__restrict__ a,
                                                 const float *__restrict__ bb, float *__restrict__ y,
                                                 const uint32_t *__restrict__ lens, int H, int T, int C) {
    __shared__ HeadVecs hv;
    const int h = blockIdx.x, b = blockIdx.y, i = threadIdx.x;
    const int len = lens ? (int)min((uint32_t)T, lens[b]) : T;
    float4 *Srow = (float4 *)(S + ((size_t)b * H + h) * 4096 + (size_t)i * 64);
    float s[64];
#pragma unroll
    for (int m = 0; m < 16; m++) {
        const float4 t = Srow[m];
        s[4 * m] = t.x; s[4 * m + 1] = t.y; s[4 * m + 2] = t.z; s[4 * m + 3] = t.w;
    }
    for (int t = 0; t < len; t++) {
        const size_t vo = ((size_t)b * T + t) * C + (size_t)h * 64;
        __syncthreads();
        hv.kh[i] = a[vo + i];
        hv.bv[i] = bb[vo + i];
        hv.wv[i] = w[vo + i];
        hv.km[i] = k[vo + i];
        hv.rv[i] = r[vo + i];
        const float vi = v[vo + i];
        __syncthreads();
        y[vo + i] = row_update(s, hv, vi);
    }
#pragma unroll
    for (int m = 0; m < 16; m++) Srow[m] = make_float4(s[4 * m], s[4 * m + 1], s[4 * m + 2], s[4 * m + 3]);
}

int launch_dplr_seq(rsv_ctx *ctx, float *s, const float *r, const float *w, const float *k,
                    const float *v, const float *a, const float *b, float *y, const uint32_t *lens,
                    int h, int n, int t, int c, int batch) {
    if (n != 64) return RSV_FAIL("dplr_seq: head_size must be 64 (got %d)", n);
    if (c != h * n) return RSV_FAIL("dplr_seq: c=%d != h*n=%d", c, h * n);
    if (t <= 0 || batch <= 0) return 0;
    hipLaunchKernelGGL(k_dplr_seq, dim3(h, batch), dim3(64), 0, ctx->stream, s, r, w, k, v, a, b, y, lens, h,
                       t, c);
    RSV_HIP(hipGetLastError());
    return 0;
}

}  // namespace rsv
