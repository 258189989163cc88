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
#include <cstdlib>

namespace rsv {

// Sum over the 64 lanes of a wave, returned to every lane.  DPP row
// operations (quad perms, half-row and row mirrors, then row broadcasts 15
// and 31 into the upper rows) leave the total in lane 63, which readlane
// broadcasts: a few cycles per step instead of an LDS round trip per
// butterfly step of __shfl_xor.
template <int CTRL, int RM = 0xF>
__device__ __forceinline__ float wdpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, RM, 0xF, false));
}
__device__ __forceinline__ float wave_sum(float v) {
    v += wdpp<0xB1>(v);        // quad_perm 1,0,3,2
    v += wdpp<0x4E>(v);        // quad_perm 2,3,0,1
    v += wdpp<0x141>(v);       // row_half_mirror
    v += wdpp<0x140>(v);       // row_mirror: each lane holds its 16-lane row sum
    v += wdpp<0x142, 0xA>(v);  // row_bcast:15 into rows 1 and 3
    v += wdpp<0x143, 0xC>(v);  // row_bcast:31 into rows 2 and 3
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
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
    // the transpose goes through a 32-row tile twice (8.3 KB instead of
    // 16.6 KB), so that ten blocks fit a CU and a B=64 launch (2560 blocks)
    // runs in one round
    __shared__ float tile[32 * 65];
    __shared__ HeadVecs hv;
    const int h = blockIdx.x, b = blockIdx.y, i = threadIdx.x;
    const size_t C = (size_t)H * 64;
    const size_t vo = (size_t)b * C + (size_t)h * 64;
    float4 *Sg = (float4 *)(S + ((size_t)b * H + h) * 4096);

    // issue the state loads first; they do not depend on the vectors.  Load m
    // covers rows 4m .. 4m+3, so loads 0..7 are rows 0..31 and 8..15 rows 32..63.
    float4 st[16];
#pragma unroll
    for (int m = 0; m < 16; m++) st[m] = Sg[m * 64 + i];

    const float ki = k[vo + i], ai = a[vo + i], ri = r[vo + i], vi_own = v[vo + i], wi = w[vo + i];
    // the GroupNorm operands too: loads after the barriers below would be a
    // second round trip at the end of the block
    const float gam = gamma[h * 64 + i], bet = beta[h * 64 + i], rki = rk[h * 64 + i];
    const float gmi = yg16 ? gmul[vo + i] : 0.0f;
    float kmod;
    head_vectors(hv, i, ki, kkc[h * 64 + i], ai, ka[h * 64 + i], ri, wi, eps, kmod);
    if (kmod_out) kmod_out[vo + i] = kmod;

    float s[64];
#pragma unroll
    for (int half = 0; half < 2; half++) {
#pragma unroll
        for (int m = 8 * half; m < 8 * half + 8; m++) {
            const int e = (m * 64 + i) * 4, row = (e >> 6) - 32 * half, col = e & 63;
            tile[row * 65 + col + 0] = st[m].x;
            tile[row * 65 + col + 1] = st[m].y;
            tile[row * 65 + col + 2] = st[m].z;
            tile[row * 65 + col + 3] = st[m].w;
        }
        __syncthreads();
        if ((i >> 5) == half) {
#pragma unroll
            for (int j = 0; j < 64; j++) s[j] = tile[(i & 31) * 65 + j];
        }
        __syncthreads();
    }
    const float y = row_update(s, hv, vi_own);
    const float yn = head_norm(y, gam, bet, ri * kmod * rki, vi_own, gn_eps);
    if (y_out) y_out[vo + i] = y;
    if (yn_out) yn_out[vo + i] = yn;
    if (yg16) yg16[vo + i] = (_Float16)(yn * gmi);  // att.output operand (y_norm * g)
    // row write-back through the tile again, 32 rows at a time
#pragma unroll
    for (int half = 0; half < 2; half++) {
        if ((i >> 5) == half) {
#pragma unroll
            for (int j = 0; j < 64; j++) tile[(i & 31) * 65 + j] = s[j];
        }
        __syncthreads();
#pragma unroll
        for (int m = 8 * half; m < 8 * half + 8; m++) {
            const int e = (m * 64 + i) * 4, row = (e >> 6) - 32 * half, col = e & 63;
            Sg[m * 64 + i] = make_float4(tile[row * 65 + col], tile[row * 65 + col + 1], tile[row * 65 + col + 2],
                                         tile[row * 65 + col + 3]);
        }
        __syncthreads();
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

// ------------------------------------------- fused LoRA-up + decode step
// The LoRA-up chain of one head (gpu_model.rs:2206-2262: w decay, a gate,
// v-first lerp, g) and the WKV7 step of that head in one block, for small
// batches: grid (H, B), 256 threads.  Thread (j = tid/4, q = tid%4) owns
// channel 64h+j: it takes quarter q of each LoRA-up dot (the inputs staged in
// LDS, the weights loaded into registers at kernel entry, ranks <= 256) and
// columns 16q..16q+15 of state row j.  Quad sums run on DPP.  The output is
// y_norm * g, the att.output operand.  Each block also copies its head's 64
// channels of side_src -> side_dst for its session (the token-shift state row).
template <int CTRL>
__device__ __forceinline__ float quad_dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float quad_sum(float v) {
    v += quad_dpp<0xB1>(v);  // quad_perm 1,0,3,2
    v += quad_dpp<0x4E>(v);  // quad_perm 2,3,0,1
    return v;
}
__device__ __forceinline__ float sig_f(float v) { return 1.0f / (1.0f + expf(-v)); }
__device__ __forceinline__ float h2f_w(uint32_t b) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(b & 0xFFFFu)); }

template <bool F16IO>
__global__ __launch_bounds__(256) void k_wkv7_lora(WkvLoraArgs A) {
    __shared__ float mids[1024];
    __shared__ float hv[5 * 64];
    __shared__ float red[16];
    const int h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
    const int j = tid >> 2, q = tid & 3, H = A.H, C = H * 64, c = h * 64 + j;
    const size_t vo = (size_t)b * C + c;
    const int m0 = A.mid_n[0], m1 = A.mid_n[1], m2 = A.mid_n[2], m3 = A.mid_n[3];
    const int L4 = m0 + m1 + m2 + m3;
    // every global load of the block first, the LoRA-up weights ahead of the
    // rest: quarter q of row c of each up matrix [C, mid], at most 8 16-byte
    // pieces per matrix (rank <= 256); pieces past a matrix's quarter are not
    // loaded (uniform branches)
    constexpr int kUp = 8;
    uint4 wl[4][kUp];
#pragma unroll
    for (int m = 0; m < 4; m++) {
        const int mid = A.mid_n[m], np = mid >> 5;
        const uint4 *wp = (const uint4 *)(A.up[m] + (size_t)c * mid + q * (mid >> 2));
#pragma unroll
        for (int e = 0; e < kUp; e++)
            if (e < np) wl[m][e] = wp[e];
    }
    // the LoRA inputs (L4 <= 1024: at most 4 per thread) stay in registers
    // until the state and vector loads below are issued: stored to LDS
    // first, they would hold those loads back until the weights had landed
    uint32_t mv[4];  // raw bits, converted when stored (an index past L4 reloads the last input)
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int e = min(tid + 256 * u, L4 - 1);
        const int m = e < m0 ? 0 : e < m0 + m1 ? 1 : e < m0 + m1 + m2 ? 2 : 3;
        const int off = m == 0 ? 0 : m == 1 ? m0 : m == 2 ? m0 + m1 : m0 + m1 + m2;
        // selects, not an indexed kernel-argument array (which is read
        // through memory, one more wait before the loads below)
        const int mid = m == 0 ? m0 : m == 1 ? m1 : m == 2 ? m2 : m3;
        const void *src = m == 0 ? A.mid[0] : m == 1 ? A.mid[1] : m == 2 ? A.mid[2] : A.mid[3];
        const size_t mi = (size_t)b * mid + (e - off);
        if (F16IO) mv[u] = ((const uint16_t *)src)[mi];  // g input already through its sigmoid
        else mv[u] = ((const uint32_t *)src)[mi];
    }
    __builtin_amdgcn_sched_barrier(0);
    const float kc = A.k[vo], rc = A.r[vo], vc = A.v[vo], vfc = A.vf[vo];
    const float w0 = A.w0[c], a0 = A.a0[c], v0 = A.v0[c], kkc = A.kk[c], kac = A.ka[c], rkc = A.rk[c];
    const float gam = A.gamma[c], bet = A.beta[c], sw = A.scale[0];
    float4 *srow = (float4 *)(A.S + (((size_t)b * H + h) * 64 + j) * 64 + 16 * q);
    float4 st4[4];
#pragma unroll
    for (int m = 0; m < 4; m++) st4[m] = srow[m];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int e = tid + 256 * u;
        if (e < L4) {
            const float f = F16IO ? h2f_w(mv[u]) : __uint_as_float(mv[u]);
            mids[e] = (!F16IO && e >= m0 + m1 + m2) ? sig_f(f) : f;
        }
    }
    __syncthreads();
    // LoRA-up dots, reduced over the quad
    float acc[4];
    int mo = 0;
#pragma unroll
    for (int m = 0; m < 4; m++) {
        const int mid = A.mid_n[m], np = mid >> 5;
        const float *xm = mids + mo + q * (mid >> 2);
        float sm = 0.0f;
#pragma unroll
        for (int e = 0; e < kUp; e++) {
            if (e >= np) break;
            const uint4 w = wl[m][e];
            const float4 x0 = *(const float4 *)(xm + 8 * e), x1 = *(const float4 *)(xm + 8 * e + 4);
            sm = fmaf(x0.x, h2f_w(w.x), sm);
            sm = fmaf(x0.y, h2f_w(w.x >> 16), sm);
            sm = fmaf(x0.z, h2f_w(w.y), sm);
            sm = fmaf(x0.w, h2f_w(w.y >> 16), sm);
            sm = fmaf(x1.x, h2f_w(w.z), sm);
            sm = fmaf(x1.y, h2f_w(w.z >> 16), sm);
            sm = fmaf(x1.z, h2f_w(w.w), sm);
            sm = fmaf(x1.w, h2f_w(w.w >> 16), sm);
        }
        acc[m] = quad_sum(sm);
        mo += mid;
    }
    const float wd = expf(sig_f(acc[0] + w0) * sw);
    const float aa = sig_f(acc[1] + a0);
    const float vv = vc + sig_f(acc[2] + v0) * (vfc - vc);
    const float gg = acc[3];
    // WKV7 head vectors (model.rs:445-473, 716-826).  The raw kk and a of
    // each column go to LDS next to the wave partials of |kk|^2 and of the
    // bonus sum, so one barrier serves both reductions; k_hat = kk/|kk| and
    // b = -k_hat*a are formed per column after it, with the same roundings.
    const float kk = kc * kkc;
    const float kmod = kc + kac * (kc * aa - kc);
    const float p_nrm = wave_sum(q == 0 ? kk * kk : 0.0f);
    const float p_bon = wave_sum(q == 0 ? rc * kmod * rkc : 0.0f);
    if (q == 0) {
        hv[j] = kk;
        hv[64 + j] = aa;
        hv[128 + j] = wd;
        hv[192 + j] = kmod;
        hv[256 + j] = rc;
    }
    if ((tid & 63) == 0) {
        red[tid >> 6] = p_nrm;
        red[4 + (tid >> 6)] = p_bon;
    }
    __syncthreads();
    float nrm = sqrtf((red[0] + red[1]) + (red[2] + red[3]));
    nrm = nrm < A.eps ? A.eps : nrm;
    const float inv = 1.0f / nrm;
    const float bonus = (red[4] + red[5]) + (red[6] + red[7]);
    // row j, columns 16q..16q+15: S = S diag(w) + (S k_hat) b^T + v k_mod^T; y = S r
    float sr[16];
#pragma unroll
    for (int m = 0; m < 4; m++) {
        sr[4 * m] = st4[m].x; sr[4 * m + 1] = st4[m].y; sr[4 * m + 2] = st4[m].z; sr[4 * m + 3] = st4[m].w;
    }
    float kh[16];
    float sa = 0.0f;
#pragma unroll
    for (int jj = 0; jj < 16; jj++) {
        kh[jj] = hv[16 * q + jj] * inv;
        sa = fmaf(sr[jj], kh[jj], sa);
    }
    sa = quad_sum(sa);
    float y = 0.0f;
#pragma unroll
    for (int jj = 0; jj < 16; jj++) {
        const int cc = 16 * q + jj;
        const float bb = kh[jj] * (-hv[64 + cc]);
        const float ns = sr[jj] * hv[128 + cc] + sa * bb + vv * hv[192 + cc];
        sr[jj] = ns;
        y = fmaf(ns, hv[256 + cc], y);
    }
    y = quad_sum(y);
#pragma unroll
    for (int m = 0; m < 4; m++) srow[m] = make_float4(sr[4 * m], sr[4 * m + 1], sr[4 * m + 2], sr[4 * m + 3]);
    // GroupNorm over the head (two-pass, eps inside the sqrt) + bonus, times
    // g; each pass one barrier on its own slots
    const float p_mean = wave_sum(q == 0 ? y : 0.0f);
    if ((tid & 63) == 0) red[8 + (tid >> 6)] = p_mean;
    __syncthreads();
    const float mean = ((red[8] + red[9]) + (red[10] + red[11])) * (1.0f / 64.0f);
    const float d = y - mean;
    const float p_var = wave_sum(q == 0 ? d * d : 0.0f);
    if ((tid & 63) == 0) red[12 + (tid >> 6)] = p_var;
    __syncthreads();
    const float var = ((red[12] + red[13]) + (red[14] + red[15])) * (1.0f / 64.0f) + A.gn_eps;
    const float yn = d * (1.0f / sqrtf(var)) * gam + bet + bonus * vv;
    if (q == 0) {
        if (F16IO) ((_Float16 *)A.yg)[vo] = (_Float16)(yn * gg);
        else ((float *)A.yg)[vo] = yn * gg;
    }
    // side copy (the token-shift state row): the head's 64 channels
    if (A.side_dst && tid < 64) {
        const size_t e = (size_t)b * C + (size_t)h * 64 + tid;
        A.side_dst[e] = A.side_src[e];
    }
}

// ------------------------------- fused LoRA-up + decode step, batched
// grid (H, ceil(B/SB)), 256 threads; fp16 LoRA inputs and fp16 output (the
// operands of the batched path).  The head's 64 rows of each LoRA-up matrix
// are read once per block for its SB sessions instead of once per session:
//   1. wave w takes rows 16w..16w+15 of every up matrix on
//      v_mfma_f32_16x16x16_f16 (A = weight rows, B = the sessions' LoRA
//      inputs staged in LDS, fp32 accumulation).  A 16-byte piece of lane
//      (i = l%16, g = l/16) covers k = 32e + 8g .. +7 of both operands and
//      feeds two MFMAs, so A and B pair up on the same k;
//   2. the dots pass through LDS to the WKV7 step, where wave w runs session
//      w on the state as loaded (16 lanes per row, no transpose; its head
//      vectors private to the wave, so the step needs no block barrier).
// Sum over a 16-lane DPP row; every lane of the row gets the same value
// (each step adds a lane's value and its partner's, commutatively).
__device__ __forceinline__ float row16_sum(float v) {
    v += quad_dpp<0xB1>(v);  // quad_perm 1,0,3,2
    v += quad_dpp<0x4E>(v);  // quad_perm 2,3,0,1
    v += quad_dpp<0x141>(v); // row_half_mirror
    v += quad_dpp<0x140>(v); // row_mirror: every lane of the 16-lane row holds its sum
    return v;
}

typedef _Float16 wk_h4 __attribute__((ext_vector_type(4)));
typedef float wk_f4 __attribute__((ext_vector_type(4)));

template <int SB>
__global__ __launch_bounds__(256, SB == 4 ? 3 : 2) void k_wkv7_lora_mb(WkvLoraArgs A, int batch) {
    constexpr int XS = 512 + 8;  // LDS row stride (halves) of one session's inputs (ranks sum <= 512)
    __shared__ __attribute__((aligned(16))) _Float16 xs[SB * XS];
    __shared__ float dots[4][64][SB + 1];
    __shared__ __attribute__((aligned(16))) HeadVecs hvs[4];
    __shared__ __attribute__((aligned(16))) float rowv[4][64];
    static_assert(SB <= 4, "one session per wave");
    const int h = blockIdx.x, b0 = blockIdx.y * SB, tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int li = lane & 15, g = lane >> 4;
    const int H = A.H, C = H * 64;
    int moff[5];
    moff[0] = 0;
#pragma unroll
    for (int m = 0; m < 4; m++) moff[m + 1] = moff[m] + A.mid_n[m];
    const int L4 = moff[4];

    // 1a. weight pieces of the wave's rows (the largest stream) first.  The
    // four matrices' 32-wide k pieces are numbered p = 0 .. L4/32 - 1 in
    // matrix order (piece p covers columns 32p.. of the concatenated
    // inputs); the launcher admits L4 <= 512, so all of them fit the wave's
    // registers at once
    constexpr int kRing = 16;
    const int P = L4 >> 5;
    uint4 wl[kRing];
#pragma unroll
    for (int e = 0; e < kRing; e++) {
        if (e < P) {
            const int k = 32 * e, m = (k >= moff[1]) + (k >= moff[2]) + (k >= moff[3]);
            // selects, not an indexed kernel-argument array (which would go through scratch)
            const _Float16 *up = m == 0 ? A.up[0] : m == 1 ? A.up[1] : m == 2 ? A.up[2] : A.up[3];
            const int mid = m == 0 ? A.mid_n[0] : m == 1 ? A.mid_n[1] : m == 2 ? A.mid_n[2] : A.mid_n[3];
            const int off = m == 0 ? 0 : m == 1 ? moff[1] : m == 2 ? moff[2] : moff[3];
            wl[e] = *((const uint4 *)(up + (size_t)(h * 64 + wave * 16 + li) * mid + (k - off)) + g);
        }
    }
    // 1b. the block's LoRA inputs, session-major, 16-byte pieces (at most
    // NP per thread: SB * L4 / 8 <= SB * 64), held in registers until the
    // state loads below are issued, so that the HBM stream of the state
    // starts at entry
    constexpr int NP = (SB * 64 + 255) / 256;
    const int ppr = L4 >> 3;  // pieces per session
    uint4 xv[NP];
#pragma unroll
    for (int q = 0; q < NP; q++) {
        const int e = tid + 256 * q, sl = e / ppr, k = (e - sl * ppr) * 8;
        xv[q] = make_uint4(0u, 0u, 0u, 0u);
        if (e < SB * ppr && b0 + sl < batch) {
            const int m = (k >= moff[1]) + (k >= moff[2]) + (k >= moff[3]);
            const _Float16 *src = (const _Float16 *)(m == 0 ? A.mid[0] : m == 1 ? A.mid[1] : m == 2 ? A.mid[2] : A.mid[3]);
            const int mid = m == 0 ? A.mid_n[0] : m == 1 ? A.mid_n[1] : m == 2 ? A.mid_n[2] : A.mid_n[3];
            const int off = m == 0 ? 0 : m == 1 ? moff[1] : m == 2 ? moff[2] : moff[3];
            xv[q] = *(const uint4 *)(src + (size_t)(b0 + sl) * mid + (k - off));
        }
    }
    // 1c. the first session's state rows and vectors of this wave
    const int c = h * 64 + lane;
    float4 st[16];
    float nk = 0.0f, nr = 0.0f, nv = 0.0f, nvf = 0.0f;
    // (a session index past the batch reads session b0, which always exists;
    // its values are never used)
#define WKV_MB_LOAD_SESSION(SL)                                                            \
    {                                                                                      \
        const int bq = b0 + (SL) < batch ? b0 + (SL) : b0;                                 \
        const float4 *Sg = (const float4 *)(A.S + ((size_t)bq * H + h) * 4096);            \
        _Pragma("unroll") for (int m = 0; m < 16; m++) st[m] = Sg[m * 64 + lane];          \
        const size_t vq = (size_t)bq * C + c;                                              \
        nk = A.k[vq]; nr = A.r[vq]; nv = A.v[vq]; nvf = A.vf[vq];                          \
    }
    __builtin_amdgcn_sched_barrier(0);
    WKV_MB_LOAD_SESSION(wave)
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int q = 0; q < NP; q++) {
        const int e = tid + 256 * q, sl = e / ppr, k = (e - sl * ppr) * 8;
        if (e < SB * ppr) *(uint4 *)&xs[sl * XS + k] = xv[q];
    }
    __syncthreads();  // (the state loads stay in flight through the dots)

    // 1d. LoRA-up dots: rows 16*wave + 4g + q (q = 0..3) for session li; one
    // accumulator, flushed to LDS where the matrix changes (uniform branch)
    {
        wk_f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
        int mcur = 0;
        auto flush = [&](int m) {
            if (li < SB) {
#pragma unroll
                for (int q = 0; q < 4; q++) dots[m][wave * 16 + 4 * g + q][li] = acc[q];
            }
        };
#pragma unroll
        for (int e = 0; e < kRing; e++) {
            const int k = 32 * e, m = (k >= moff[1]) + (k >= moff[2]) + (k >= moff[3]);
            if (e >= P) continue;
            if (m != mcur) {
                flush(mcur);
                acc = (wk_f4){0.0f, 0.0f, 0.0f, 0.0f};
                mcur = m;
            }
            const uint4 w = wl[e];
            const uint4 x = li < SB ? *(const uint4 *)(xs + li * XS + k + 8 * g) : make_uint4(0u, 0u, 0u, 0u);
            acc = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(wk_h4, make_uint2(w.x, w.y)),
                                                        __builtin_bit_cast(wk_h4, make_uint2(x.x, x.y)), acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(wk_h4, make_uint2(w.z, w.w)),
                                                        __builtin_bit_cast(wk_h4, make_uint2(x.z, x.w)), acc, 0, 0, 0);
        }
        flush(mcur);
    }
    // the channel constants of phase 2, loaded only now: with the weight
    // ring and the state both in registers they would be spilled
    const float w0 = A.w0[c], a0 = A.a0[c], v0 = A.v0[c], kkc = A.kk[c], kac = A.ka[c], rkc = A.rk[c];
    const float gam = A.gamma[c], bet = A.beta[c], sw = A.scale[0];
    // side copy: this block's sessions x the head's 64 channels
    for (int e = tid; e < SB * 64; e += 256) {
        const int b = b0 + (e >> 6);
        if (A.side_dst && b < batch) A.side_dst[(size_t)b * C + c - lane + (e & 63)] = A.side_src[(size_t)b * C + c - lane + (e & 63)];
    }
    __syncthreads();

    // 2. WKV7 step of session wave (model.rs:445-473, 716-826).  The state
    // stays in the layout it was loaded in: lane l holds columns
    // 4(l%16) .. +3 of rows 4m + l/16 (m = 0..15), so each row lies in one
    // 16-lane DPP row and its dot products are 4-column partials summed
    // over that row.  Per-column vectors are formed lane-per-column as in
    // k_wkv7_decode and read back as the lane's four columns.
    HeadVecs &hv = hvs[wave];
    float *vr = rowv[wave];  // v by row group: [l%4][l/4] for row l; then y by row
    if (wave < SB && b0 + wave < batch) {
        const int b = b0 + wave, sl = wave;
        const int rg = lane >> 4, cq = lane & 15;
        const float wd = expf(sig_f(dots[0][lane][sl] + w0) * sw);
        const float aa = sig_f(dots[1][lane][sl] + a0);
        const float vv = nv + sig_f(dots[2][lane][sl] + v0) * (nvf - nv);
        const float gg = dots[3][lane][sl];
        float kmod;
        head_vectors(hv, lane, nk, kkc, aa, kac, nr, wd, A.eps, kmod);
        vr[(lane & 3) * 16 + (lane >> 2)] = vv;
        __builtin_amdgcn_wave_barrier();
        const float4 kh4 = *(const float4 *)&hv.kh[4 * cq], bv4 = *(const float4 *)&hv.bv[4 * cq];
        const float4 wv4 = *(const float4 *)&hv.wv[4 * cq], km4 = *(const float4 *)&hv.km[4 * cq];
        const float4 rv4 = *(const float4 *)&hv.rv[4 * cq];
        float vrow[16];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float4 t = *(const float4 *)&vr[rg * 16 + 4 * q];
            vrow[4 * q] = t.x; vrow[4 * q + 1] = t.y; vrow[4 * q + 2] = t.z; vrow[4 * q + 3] = t.w;
        }
        float ymine = 0.0f;  // y of row 4 cq + rg
#pragma unroll
        for (int m = 0; m < 16; m++) {
            float4 &q = st[m];
            float sa = q.x * kh4.x;
            sa = fmaf(q.y, kh4.y, sa);
            sa = fmaf(q.z, kh4.z, sa);
            sa = fmaf(q.w, kh4.w, sa);
            sa = row16_sum(sa);
            const float vi = vrow[m];
            q.x = q.x * wv4.x + sa * bv4.x + vi * km4.x;
            q.y = q.y * wv4.y + sa * bv4.y + vi * km4.y;
            q.z = q.z * wv4.z + sa * bv4.z + vi * km4.z;
            q.w = q.w * wv4.w + sa * bv4.w + vi * km4.w;
            float y = q.x * rv4.x;
            y = fmaf(q.y, rv4.y, y);
            y = fmaf(q.z, rv4.z, y);
            y = fmaf(q.w, rv4.w, y);
            y = row16_sum(y);
            ymine = cq == m ? y : ymine;
        }
        float4 *Sg = (float4 *)(A.S + ((size_t)b * H + h) * 4096);
#pragma unroll
        for (int m = 0; m < 16; m++) Sg[m * 64 + lane] = st[m];
        __builtin_amdgcn_wave_barrier();
        vr[4 * cq + rg] = ymine;  // (every lane has read its v rows above)
        __builtin_amdgcn_wave_barrier();
        const float y = vr[lane];
        const float yn = head_norm(y, gam, bet, nr * kmod * rkc, vv, A.gn_eps);
        ((_Float16 *)A.yg)[(size_t)b * C + c] = (_Float16)(yn * gg);
    }
#undef WKV_MB_LOAD_SESSION
}

// ------------------------------- fused LoRA-up + decode step, rows split
// One session's head over four blocks (grid 4H x B, 256 threads), block
// part p owning state rows 16p .. 16p+15, so that 4H blocks stream the
// LoRA-up weights and the state instead of H.  Every block forms the head's
// column vectors (k_hat, b = -k_hat*a, w, k_mod, r) and the two column sums
// (|kk|^2, bonus) itself, which needs the w and a LoRA-up rows of all 64
// columns; the v and g rows only for its own 16 rows.  The GroupNorm needs
// the y of all 64 rows, so it is left to the consumer: the block writes
// y = S r (raw), bonus * v and the gate g per row, and the att.output GEMV
// applies ((y - mean) * rstd * gamma + beta + bonus*v) * g in its prologue
// (gemv prologue PRO_GNGATE).  The four blocks of a head sit on one XCD
// (consecutive block ids go to the 8 XCDs in turn) so the w/a rows they all
// read come from one L2.
//   LoRA dots: w and a as in k_wkv7_lora (column j = tid/4, quarter tid%4,
//   quad sums); v and g with 16 threads per row (row 16p + tid/16).
//   State: row 16p + tid/16, columns 4*(tid%16) .. +3; the row sums S k_hat
//   and S r are 16-lane DPP row sums.

__global__ __launch_bounds__(256) void k_wkv7_lora_rows(WkvLoraArgs A) {
    __shared__ float mids[1024];
    __shared__ float hv[5 * 64];
    __shared__ float red[8];
    const int H = A.H, C = H * 64, tid = threadIdx.x, b = blockIdx.y;
    // block -> (head, part): the 4 parts of a head on one XCD when H % 8 == 0
    const int bid = blockIdx.x;
    const int h = (H & 7) == 0 ? (bid & 7) + 8 * (bid >> 5) : bid >> 2;
    const int p = (H & 7) == 0 ? (bid >> 3) & 3 : bid & 3;
    const int j = tid >> 2, q = tid & 3, c = h * 64 + j;          // column role
    const int rr = 16 * p + (tid >> 4), s16 = tid & 15, cr = h * 64 + rr;  // row role
    const int m0 = A.mid_n[0], m1 = A.mid_n[1], m2 = A.mid_n[2], m3 = A.mid_n[3];
    const int L4 = m0 + m1 + m2 + m3;
    // 1. loads: w/a up rows of column j (quarter q), v/g up rows of row rr
    // (part s16 of 16), then mids, vectors and the 16 state rows
    uint4 wl[2][8];
#pragma unroll
    for (int m = 0; m < 2; m++) {
        const int mid = A.mid_n[m], np = mid >> 5;
        const uint4 *wp = (const uint4 *)(A.up[m] + (size_t)c * mid + q * (mid >> 2));
#pragma unroll
        for (int e = 0; e < 8; e++)
            if (e < np) wl[m][e] = wp[e];
    }
    // v and g rows: rank/16 halves per thread (2..16), as 2-half pieces
    uint32_t vl[2][8];
#pragma unroll
    for (int m = 0; m < 2; m++) {
        const int mid = A.mid_n[2 + m], np = mid >> 5;
        const uint32_t *wp = (const uint32_t *)(A.up[2 + m] + (size_t)cr * mid + s16 * (mid >> 4));
#pragma unroll
        for (int e = 0; e < 8; e++)
            if (e < np) vl[m][e] = wp[e];
    }
    // the LoRA inputs (L4 <= 1024: at most 4 per thread; an index past L4
    // reloads the last one) stay in registers until the vector and state
    // loads below are issued; kernel-argument arrays are selected, not
    // indexed (an indexed one is read through memory, one more wait)
    float mv[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int e = min(tid + 256 * u, L4 - 1);
        const int m = e < m0 ? 0 : e < m0 + m1 ? 1 : e < m0 + m1 + m2 ? 2 : 3;
        const int off = m == 0 ? 0 : m == 1 ? m0 : m == 2 ? m0 + m1 : m0 + m1 + m2;
        const int mid = m == 0 ? m0 : m == 1 ? m1 : m == 2 ? m2 : m3;
        const float *src = (const float *)(m == 0 ? A.mid[0] : m == 1 ? A.mid[1] : m == 2 ? A.mid[2] : A.mid[3]);
        mv[u] = src[(size_t)b * mid + (e - off)];
    }
    __builtin_amdgcn_sched_barrier(0);
    const size_t vo = (size_t)b * C + c, ro = (size_t)b * C + cr;
    const float kc = A.k[vo], rc = A.r[vo];
    const float w0 = A.w0[c], a0 = A.a0[c], kkc = A.kk[c], kac = A.ka[c], rkc = A.rk[c];
    const float vrow = A.v[ro], vfrow = A.vf[ro], v0row = A.v0[cr], sw = A.scale[0];
    float4 *srow = (float4 *)(A.S + (((size_t)b * H + h) * 64 + rr) * 64) + s16;
    const float4 st = *srow;
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int e = tid + 256 * u;
        if (e < L4) mids[e] = e >= m0 + m1 + m2 ? sig_f(mv[u]) : mv[u];
    }
    __syncthreads();
    // 2. LoRA dots
    float acc[2];
#pragma unroll
    for (int m = 0; m < 2; m++) {
        const int mid = A.mid_n[m], np = mid >> 5;
        const float *xm = mids + (m == 0 ? 0 : m0) + q * (mid >> 2);
        float sm = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            if (e >= np) break;
            const uint4 w = wl[m][e];
            const float4 x0 = *(const float4 *)(xm + 8 * e), x1 = *(const float4 *)(xm + 8 * e + 4);
            sm = fmaf(x0.x, h2f_w(w.x), sm);
            sm = fmaf(x0.y, h2f_w(w.x >> 16), sm);
            sm = fmaf(x0.z, h2f_w(w.y), sm);
            sm = fmaf(x0.w, h2f_w(w.y >> 16), sm);
            sm = fmaf(x1.x, h2f_w(w.z), sm);
            sm = fmaf(x1.y, h2f_w(w.z >> 16), sm);
            sm = fmaf(x1.z, h2f_w(w.w), sm);
            sm = fmaf(x1.w, h2f_w(w.w >> 16), sm);
        }
        acc[m] = quad_sum(sm);
    }
    float racc[2];
#pragma unroll
    for (int m = 0; m < 2; m++) {
        const int mid = A.mid_n[2 + m], np = mid >> 5;
        const float *xm = mids + (m == 0 ? m0 + m1 : m0 + m1 + m2) + s16 * (mid >> 4);
        float sm = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            if (e >= np) break;
            const uint32_t w = vl[m][e];
            const float2 x0 = *(const float2 *)(xm + 2 * e);
            sm = fmaf(x0.x, h2f_w(w), sm);
            sm = fmaf(x0.y, h2f_w(w >> 16), sm);
        }
        racc[m] = row16_sum(sm);
    }
    const float wd = expf(sig_f(acc[0] + w0) * sw);
    const float aa = sig_f(acc[1] + a0);
    const float vv = vrow + sig_f(racc[0] + v0row) * (vfrow - vrow);
    const float gg = racc[1];
    // 3. column vectors and the two column sums (as k_wkv7_lora)
    const float kk = kc * kkc;
    const float kmod = kc + kac * (kc * aa - kc);
    const float p_nrm = wave_sum(q == 0 ? kk * kk : 0.0f);
    const float p_bon = wave_sum(q == 0 ? rc * kmod * rkc : 0.0f);
    if (q == 0) {
        hv[j] = kk;
        hv[64 + j] = aa;
        hv[128 + j] = wd;
        hv[192 + j] = kmod;
        hv[256 + j] = rc;
    }
    if ((tid & 63) == 0) {
        red[tid >> 6] = p_nrm;
        red[4 + (tid >> 6)] = p_bon;
    }
    __syncthreads();
    float nrm = sqrtf((red[0] + red[1]) + (red[2] + red[3]));
    nrm = nrm < A.eps ? A.eps : nrm;
    const float inv = 1.0f / nrm;
    const float bonus = (red[4] + red[5]) + (red[6] + red[7]);
    // 4. row rr, columns 4*s16 .. +3: S = S diag(w) + (S k_hat) b^T + v k_mod^T; y = S r
    float sr[4] = {st.x, st.y, st.z, st.w}, kh[4];
    float sa = 0.0f;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        kh[e] = hv[4 * s16 + e] * inv;
        sa = fmaf(sr[e], kh[e], sa);
    }
    sa = row16_sum(sa);
    float y = 0.0f;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int cc = 4 * s16 + e;
        const float bb = kh[e] * (-hv[64 + cc]);
        const float ns = sr[e] * hv[128 + cc] + sa * bb + vv * hv[192 + cc];
        sr[e] = ns;
        y = fmaf(ns, hv[256 + cc], y);
    }
    y = row16_sum(y);
    *srow = make_float4(sr[0], sr[1], sr[2], sr[3]);
    if (s16 == 0) {
        ((float *)A.yg)[ro] = y;
        A.y_bonus[ro] = bonus * vv;
        A.y_gate[ro] = gg;
    }
    // side copy (the token-shift state row), 16 elements per block at the
    // end: one block copying the whole row would chain its round trips
    if (A.side_dst && tid < 16) {
        const size_t e = (size_t)b * C + (size_t)(h * 4 + p) * 16 + tid;
        A.side_dst[e] = A.side_src[e];
    }
}

int launch_wkv7_lora(rsv_ctx *ctx, const WkvLoraArgs &a, int batch) {
    if (a.H <= 0 || batch <= 0 || batch > 65535) return RSV_FAIL("wkv7_lora: bad h=%d batch=%d", a.H, batch);
    int L4 = 0;
    for (int m = 0; m < 4; m++) {
        if (a.mid_n[m] <= 0 || a.mid_n[m] % 32 || a.mid_n[m] > 256)
            return RSV_FAIL("wkv7_lora: LoRA rank %d must be a multiple of 32 in 32..256", a.mid_n[m]);
        L4 += a.mid_n[m];
    }
    if (L4 > 1024) return RSV_FAIL("wkv7_lora: LoRA ranks sum to %d (max 1024)", L4);
    // batches of 16 and more with fp16 operands and ranks summing to at most
    // 512: 4 sessions per block (the head's LoRA-up rows read once per block;
    // 8 or 16 sessions per block measured slower: too few blocks to spread
    // the per-CU traffic)
    if (a.y_bonus || a.y_gate) {
        if (!a.y_bonus || !a.y_gate || a.f16_io) return RSV_FAIL("wkv7_lora: the split form needs F32 io and both bonus and gate outputs");
        if ((size_t)4 * a.H > 65535) return RSV_FAIL("wkv7_lora: too many heads for the split form");
        hipLaunchKernelGGL(k_wkv7_lora_rows, dim3(4 * a.H, batch), dim3(256), 0, ctx->stream, a);
    } else if (a.f16_io && batch >= 16 && L4 <= 512) {
        hipLaunchKernelGGL(k_wkv7_lora_mb<4>, dim3(a.H, (batch + 3) / 4), dim3(256), 0, ctx->stream, a, batch);
    } else if (a.f16_io) hipLaunchKernelGGL(k_wkv7_lora<true>, dim3(a.H, batch), dim3(256), 0, ctx->stream, a);
    else hipLaunchKernelGGL(k_wkv7_lora<false>, dim3(a.H, batch), dim3(256), 0, ctx->stream, a);
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
    // the next token's vectors are loaded while the current one is computed
    size_t vn = (size_t)t0 * C + (size_t)h * 64 + i;
    float nk = 0.f, na = 0.f, nr = 0.f, nv = 0.f, nw = 0.f;
    if (len > 0) { nk = k[vn]; na = a[vn]; nr = r[vn]; nv = v[vn]; nw = w[vn]; }
    for (uint32_t t = 0; t < len; t++) {
        const size_t vo = (size_t)(t0 + t) * C + (size_t)h * 64;
        const float ki = nk, ai = na, ri = nr, vi = nv, wi = nw;
        if (t + 1 < len) {  // uniform
            vn += C;
            nk = k[vn]; na = a[vn]; nr = r[vn]; nv = v[vn]; nw = w[vn];
        }
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

// ------------------------------------- ragged prefill scan, gated fp16 out
// The scan of rsv_wkv7_seq_ragged_gate, leaving the att.output operand
// yg = (GroupNorm(y) + bonus*v) * g in fp16: k_wkv7_seq_rows writes the raw
// y = S r and the head's bonus sum per token, then k_gn_gate_f16 applies
// GroupNorm + bonus*v and the gate.  Per (head, segment), 64/RPL lane groups
// of four lanes: a group owns RPL state rows, each lane 16 columns of them.
// The head's column vectors of a batch of tokens (the reductions over the
// head, |k| and the bonus sum, included) are formed four tokens per wave
// into LDS first, so the scan's dependent chain per token is the row-local
// update alone.  Against the one-wave scan with GroupNorm inside
// (k_wkv7_seq_ragged): 560 -> 333 us on 8 segments of 512 tokens (40
// heads), 227 -> 211 us on 64 of 64.
template <int RPL>
__global__ __launch_bounds__(256 / RPL) void k_wkv7_seq_rows(
    float *__restrict__ S, const float *__restrict__ r, const float *__restrict__ w, const float *__restrict__ k,
    const float *__restrict__ v, const float *__restrict__ a, const float *__restrict__ kkc,
    const float *__restrict__ ka, const float *__restrict__ rk, float *__restrict__ y_out,
    float *__restrict__ bonus_out, const uint32_t *__restrict__ seg_start, const uint32_t *__restrict__ seg_len,
    const uint32_t *__restrict__ seg_slot, int H, float eps, uint64_t rows, uint64_t slots) {
    constexpr int NW = 4 / RPL;   // waves per (head, segment)
    constexpr int kRB = 4 * NW;   // tokens per batch: four per wave in the batch phase
    // per batch: [token][k^ | -k^ a | w | k_mod | r | v] x 64 columns, two batches alternating
    __shared__ __attribute__((aligned(16))) float hb[2][kRB][6 * 64];
    // the batch's outputs (y per token and row, the bonus sum per token) are
    // staged in LDS and stored once the batch is done: a global store per
    // token would hold its data register until the write completes
    __shared__ __attribute__((aligned(16))) float yl[2][kRB][64];
    __shared__ float bl[2][kRB];
    const int h = blockIdx.x, gi = blockIdx.y, tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63, q = lane & 3;
    const int row0 = 16 * RPL * wave + RPL * (lane >> 2);  // this lane's rows row0 .. row0 + RPL - 1
    const size_t C = (size_t)H * 64;
    const uint32_t t0 = seg_start[gi], len = seg_len[gi], slot = seg_slot[gi];
    if (slot >= slots || (uint64_t)t0 + len > rows) return;  // uniform per block
    float4 *Sb = (float4 *)(S + ((size_t)slot * H + h) * 4096);
    float s[RPL][16];
#pragma unroll
    for (int i = 0; i < RPL; i++)
#pragma unroll
        for (int m = 0; m < 4; m++) {
            const float4 x = Sb[(row0 + i) * 16 + 4 * q + m];
            s[i][4 * m] = x.x; s[i][4 * m + 1] = x.y; s[i][4 * m + 2] = x.z; s[i][4 * m + 3] = x.w;
        }
    // column role (batch phase): lane j forms column j's vectors of tokens
    // 4*wave .. 4*wave+3 of a batch; every reduction over the head happens
    // here, for four tokens at once, off the scan's dependent chain
    const int j = lane;
    const float kkc_j = kkc[h * 64 + j], ka_j = ka[h * 64 + j], rk_j = rk[h * 64 + j];
    float pk[4], pa[4], pw[4], pr[4], pv[4];
    auto load_batch = [&](uint32_t tb) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t t = tb + 4 * wave + i;
            const size_t vo = (size_t)(t0 + (t < len ? t : 0)) * C + (size_t)h * 64 + j;
            pk[i] = k[vo]; pa[i] = a[vo]; pw[i] = w[vo]; pr[i] = r[vo]; pv[i] = v[vo];
        }
    };
    auto form_batch = [&](int buf, uint32_t tb) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t t = tb + 4 * wave + i;
            if (t >= len) break;  // uniform per wave
            const float kc = pk[i], ac = pa[i], rc = pr[i];
            const float kk = kc * kkc_j;
            float nrm = sqrtf(wave_sum(kk * kk));
            nrm = nrm < eps ? eps : nrm;
            const float kh = kk * (1.0f / nrm);
            const float kmod = kc + ka_j * (kc * ac - kc);
            const float bonus = wave_sum(rc * kmod * rk_j);
            float *hv = hb[buf][4 * wave + i];
            hv[j] = kh; hv[64 + j] = kh * (-ac); hv[128 + j] = pw[i]; hv[192 + j] = kmod; hv[256 + j] = rc; hv[320 + j] = pv[i];
            if (j == 0) bl[buf][4 * wave + i] = bonus;
        }
    };
    auto flush = [&](int buf, uint32_t tb) {
        // kRB tokens x 64 rows = one float4 per thread (non-temporal: acknowledged sooner)
        typedef float f4v __attribute__((ext_vector_type(4)));
        const uint32_t u = tid >> 4, c4 = 4 * (tid & 15);
        if (tb + u < len) {
            const float4 yv = *(const float4 *)&yl[buf][u][c4];
            __builtin_nontemporal_store((f4v){yv.x, yv.y, yv.z, yv.w}, (f4v *)(y_out + (size_t)(t0 + tb + u) * C + (size_t)h * 64 + c4));
        }
        if (tid < kRB && tb + tid < len) __builtin_nontemporal_store(bl[buf][tid], bonus_out + (size_t)(t0 + tb + tid) * H + h);
    };
    if (len > 0) {
        load_batch(0);
        form_batch(0, 0);
    }
    for (uint32_t tb = 0; tb < len; tb += kRB) {
        const int buf = (tb / kRB) & 1;
        // the batch's vectors are in LDS (lgkmcnt(0), then the barrier); the
        // other buffer is free
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_s_barrier();
        if (tb > 0) flush(buf ^ 1, tb - kRB);  // the previous batch's outputs
        const bool more = tb + kRB < len;
        if (more) load_batch(tb + kRB);  // in flight during the scan below
        const uint32_t nt = len - tb < (uint32_t)kRB ? len - tb : (uint32_t)kRB;
        for (uint32_t u = 0; u < nt; u++) {
            const float *hv = hb[buf][u];
            float kv[16], bv[16], wv[16], mv[16], rv[16], vc[RPL];
#pragma unroll
            for (int m = 0; m < 4; m++) {
                const float4 a0 = *(const float4 *)(hv + 16 * q + 4 * m), a1 = *(const float4 *)(hv + 64 + 16 * q + 4 * m),
                             a2 = *(const float4 *)(hv + 128 + 16 * q + 4 * m), a3 = *(const float4 *)(hv + 192 + 16 * q + 4 * m),
                             a4 = *(const float4 *)(hv + 256 + 16 * q + 4 * m);
                kv[4 * m] = a0.x; kv[4 * m + 1] = a0.y; kv[4 * m + 2] = a0.z; kv[4 * m + 3] = a0.w;
                bv[4 * m] = a1.x; bv[4 * m + 1] = a1.y; bv[4 * m + 2] = a1.z; bv[4 * m + 3] = a1.w;
                wv[4 * m] = a2.x; wv[4 * m + 1] = a2.y; wv[4 * m + 2] = a2.z; wv[4 * m + 3] = a2.w;
                mv[4 * m] = a3.x; mv[4 * m + 1] = a3.y; mv[4 * m + 2] = a3.z; mv[4 * m + 3] = a3.w;
                rv[4 * m] = a4.x; rv[4 * m + 1] = a4.y; rv[4 * m + 2] = a4.z; rv[4 * m + 3] = a4.w;
            }
#pragma unroll
            for (int i = 0; i < RPL; i++) vc[i] = hv[320 + row0 + i];
            float sa[RPL], y[RPL];
#pragma unroll
            for (int i = 0; i < RPL; i++) {
                sa[i] = 0.f;
#pragma unroll
                for (int e = 0; e < 16; e++) sa[i] = fmaf(s[i][e], kv[e], sa[i]);
            }
#pragma unroll
            for (int i = 0; i < RPL; i++) sa[i] = quad_sum(sa[i]);
#pragma unroll
            for (int i = 0; i < RPL; i++) {
                y[i] = 0.f;
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    const float ns = s[i][e] * wv[e] + sa[i] * bv[e] + vc[i] * mv[e];
                    s[i][e] = ns;
                    y[i] = fmaf(ns, rv[e], y[i]);
                }
            }
#pragma unroll
            for (int i = 0; i < RPL; i++) y[i] = quad_sum(y[i]);
            if (q == 0)
#pragma unroll
                for (int i = 0; i < RPL; i++) yl[buf][u][row0 + i] = y[i];
        }
        if (more) form_batch(buf ^ 1, tb + kRB);
    }
    if (len > 0) {
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_s_barrier();
        const uint32_t last = (len - 1) / kRB * kRB;
        flush((last / kRB) & 1, last);
    }
#pragma unroll
    for (int i = 0; i < RPL; i++)
#pragma unroll
        for (int m = 0; m < 4; m++)
            Sb[(row0 + i) * 16 + 4 * q + m] = make_float4(s[i][4 * m], s[i][4 * m + 1], s[i][4 * m + 2], s[i][4 * m + 3]);
}

// The scan for latency-bound launches (few segments: a long prompt of one
// session, or a handful): one state row per lane group of G lanes, each lane
// 64/G columns, G waves per (head, segment).  The dependent chain per token
// is 64/G multiply-adds and a log2(G)-step DPP sum instead of 16 and two, at
// G times the threads of k_wkv7_seq_rows<1>.  The head's column vectors of
// a batch of tokens are formed into LDS one token per wave (16 per batch).
template <int G>
__device__ __forceinline__ float group_allsum(float v) {
    v += quad_dpp<0xB1>(v);  // quad_perm 1,0,3,2
    v += quad_dpp<0x4E>(v);  // quad_perm 2,3,0,1
    if (G >= 8) v += quad_dpp<0x141>(v);   // row_half_mirror: the 8-lane sum in every lane of the 8
    if (G >= 16) v += quad_dpp<0x140>(v);  // row_mirror: the 16-lane sum in every lane of the row
    return v;
}

template <int G>
__global__ __launch_bounds__(64 * G) void k_wkv7_seq_cols(
    float *__restrict__ S, const float *__restrict__ r, const float *__restrict__ w, const float *__restrict__ k,
    const float *__restrict__ v, const float *__restrict__ a, const float *__restrict__ kkc,
    const float *__restrict__ ka, const float *__restrict__ rk, float *__restrict__ y_out,
    float *__restrict__ bonus_out, const uint32_t *__restrict__ seg_start, const uint32_t *__restrict__ seg_len,
    const uint32_t *__restrict__ seg_slot, int H, float eps, uint64_t rows, uint64_t slots) {
    constexpr int NW = G;           // waves per (head, segment)
    constexpr int CPL = 64 / G;     // columns per lane
    constexpr int TPW = G >= 4 ? 1 : 4 / G;
    constexpr int kRB = NW * TPW;   // tokens per batch
    __shared__ __attribute__((aligned(16))) float hb[2][kRB][6 * 64];
    __shared__ __attribute__((aligned(16))) float yl[2][kRB][64];
    __shared__ float bl[2][kRB];
    const int h = blockIdx.x, gi = blockIdx.y, tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63, q = lane % G;
    const int row = (64 / G) * wave + lane / G;
    const size_t C = (size_t)H * 64;
    const uint32_t t0 = seg_start[gi], len = seg_len[gi], slot = seg_slot[gi];
    if (slot >= slots || (uint64_t)t0 + len > rows) return;  // uniform per block
    float *Sr = S + ((size_t)slot * H + h) * 4096 + (size_t)row * 64 + q * CPL;
    float s[CPL];
#pragma unroll
    for (int m = 0; m < CPL / 4; m++) {
        const float4 x = ((const float4 *)Sr)[m];
        s[4 * m] = x.x; s[4 * m + 1] = x.y; s[4 * m + 2] = x.z; s[4 * m + 3] = x.w;
    }
    const int j = lane;
    const float kkc_j = kkc[h * 64 + j], ka_j = ka[h * 64 + j], rk_j = rk[h * 64 + j];
    float pk[TPW], pa[TPW], pw[TPW], pr[TPW], pv[TPW];
    auto load_batch = [&](uint32_t tb) {
#pragma unroll
        for (int i = 0; i < TPW; i++) {
            const uint32_t t = tb + TPW * wave + i;
            const size_t vo = (size_t)(t0 + (t < len ? t : 0)) * C + (size_t)h * 64 + j;
            pk[i] = k[vo]; pa[i] = a[vo]; pw[i] = w[vo]; pr[i] = r[vo]; pv[i] = v[vo];
        }
    };
    auto form_batch = [&](int buf, uint32_t tb) {
#pragma unroll
        for (int i = 0; i < TPW; i++) {
            const uint32_t t = tb + TPW * wave + i;
            if (t >= len) break;  // uniform per wave
            const float kc = pk[i], ac = pa[i], rc = pr[i];
            const float kk = kc * kkc_j;
            float nrm = sqrtf(wave_sum(kk * kk));
            nrm = nrm < eps ? eps : nrm;
            const float kh = kk * (1.0f / nrm);
            const float kmod = kc + ka_j * (kc * ac - kc);
            const float bonus = wave_sum(rc * kmod * rk_j);
            float *hv = hb[buf][TPW * wave + i];
            hv[j] = kh; hv[64 + j] = kh * (-ac); hv[128 + j] = pw[i]; hv[192 + j] = kmod; hv[256 + j] = rc; hv[320 + j] = pv[i];
            if (j == 0) bl[buf][TPW * wave + i] = bonus;
        }
    };
    auto flush = [&](int buf, uint32_t tb) {
        for (int e = tid; e < kRB * 64; e += 64 * G) {
            const uint32_t u = e >> 6;
            if (tb + u < len) __builtin_nontemporal_store(yl[buf][u][e & 63], y_out + (size_t)(t0 + tb + u) * C + (size_t)h * 64 + (e & 63));
        }
        if (tid < kRB && tb + tid < len) __builtin_nontemporal_store(bl[buf][tid], bonus_out + (size_t)(t0 + tb + tid) * H + h);
    };
    if (len > 0) {
        load_batch(0);
        form_batch(0, 0);
    }
    for (uint32_t tb = 0; tb < len; tb += kRB) {
        const int buf = (tb / kRB) & 1;
        __syncthreads();
        if (tb > 0) flush(buf ^ 1, tb - kRB);
        const bool more = tb + kRB < len;
        if (more) load_batch(tb + kRB);
        const uint32_t nt = len - tb < (uint32_t)kRB ? len - tb : (uint32_t)kRB;
        for (uint32_t u = 0; u < nt; u++) {
            const float *hv = hb[buf][u] + q * CPL;
            float kv[CPL], bv[CPL], wv[CPL], mv[CPL], rv[CPL];
#pragma unroll
            for (int m = 0; m < CPL / 4; m++) {
                const float4 a0 = *(const float4 *)(hv + 4 * m), a1 = *(const float4 *)(hv + 64 + 4 * m),
                             a2 = *(const float4 *)(hv + 128 + 4 * m), a3 = *(const float4 *)(hv + 192 + 4 * m),
                             a4 = *(const float4 *)(hv + 256 + 4 * m);
                kv[4 * m] = a0.x; kv[4 * m + 1] = a0.y; kv[4 * m + 2] = a0.z; kv[4 * m + 3] = a0.w;
                bv[4 * m] = a1.x; bv[4 * m + 1] = a1.y; bv[4 * m + 2] = a1.z; bv[4 * m + 3] = a1.w;
                wv[4 * m] = a2.x; wv[4 * m + 1] = a2.y; wv[4 * m + 2] = a2.z; wv[4 * m + 3] = a2.w;
                mv[4 * m] = a3.x; mv[4 * m + 1] = a3.y; mv[4 * m + 2] = a3.z; mv[4 * m + 3] = a3.w;
                rv[4 * m] = a4.x; rv[4 * m + 1] = a4.y; rv[4 * m + 2] = a4.z; rv[4 * m + 3] = a4.w;
            }
            const float vc = hb[buf][u][320 + row];
            float sa = 0.f;
#pragma unroll
            for (int e = 0; e < CPL; e++) sa = fmaf(s[e], kv[e], sa);
            sa = group_allsum<G>(sa);
            float y = 0.f;
#pragma unroll
            for (int e = 0; e < CPL; e++) {
                const float ns = s[e] * wv[e] + sa * bv[e] + vc * mv[e];
                s[e] = ns;
                y = fmaf(ns, rv[e], y);
            }
            y = group_allsum<G>(y);
            if (q == 0) yl[buf][u][row] = y;
        }
        if (more) form_batch(buf ^ 1, tb + kRB);
    }
    if (len > 0) {
        __syncthreads();
        const uint32_t last = (len - 1) / kRB * kRB;
        flush((last / kRB) & 1, last);
    }
#pragma unroll
    for (int m = 0; m < CPL / 4; m++)
        ((float4 *)Sr)[m] = make_float4(s[4 * m], s[4 * m + 1], s[4 * m + 2], s[4 * m + 3]);
}

// yg = ((GroupNorm(y) * gamma + beta) + bonus * v) * g in fp16: 16 lanes per
// (token, head), four columns per lane (16-byte loads, 8-byte stores), four
// (token, head) units per wave and 16 per block; the two-pass statistics are
// 16-lane DPP row sums.
__global__ __launch_bounds__(256) void k_gn_gate_f16(const float *__restrict__ y, const float *__restrict__ bonus,
                                                    const float *__restrict__ v, const float *__restrict__ gamma,
                                                    const float *__restrict__ beta, const float *__restrict__ g,
                                                    _Float16 *__restrict__ yg, uint64_t units, int H, float gn_eps) {
    const uint64_t u = (uint64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
    const bool live = u < units;  // the row sums below need every lane of the row
    const int i = 4 * (threadIdx.x & 15), h = live ? (int)(u % H) : 0;
    const size_t o = (live ? (size_t)u : 0) * 64 + i;  // (token, head) units are consecutive 64-column groups
    const float4 yy = *(const float4 *)(y + o), vv = *(const float4 *)(v + o), gg = *(const float4 *)(g + o);
    const float4 gm = *(const float4 *)(gamma + h * 64 + i), bt = *(const float4 *)(beta + h * 64 + i);
    const float bo = bonus[live ? u : 0];
    const float mean = row16_sum((yy.x + yy.y) + (yy.z + yy.w)) * (1.0f / 64.0f);
    const float d0 = yy.x - mean, d1 = yy.y - mean, d2 = yy.z - mean, d3 = yy.w - mean;
    const float var = row16_sum((d0 * d0 + d1 * d1) + (d2 * d2 + d3 * d3)) * (1.0f / 64.0f) + gn_eps;
    const float inv = 1.0f / sqrtf(var);
    if (!live) return;
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    h4 out;
    out[0] = (_Float16)((d0 * inv * gm.x + bt.x + bo * vv.x) * gg.x);
    out[1] = (_Float16)((d1 * inv * gm.y + bt.y + bo * vv.y) * gg.y);
    out[2] = (_Float16)((d2 * inv * gm.z + bt.z + bo * vv.z) * gg.z);
    out[3] = (_Float16)((d3 * inv * gm.w + bt.w + bo * vv.w) * gg.w);
    *(h4 *)(yg + o) = out;
}

int launch_wkv7_seq_ragged_gate(rsv_ctx *ctx, float *s, const float *r, const float *w, const float *k,
                                const float *v, const float *a, const float *kk, const float *ka, const float *rk,
                                const float *gamma, const float *beta, const float *g, float *y_work,
                                float *bonus_work, _Float16 *yg, const uint32_t *seg_start, const uint32_t *seg_len,
                                const uint32_t *seg_slot, int nseg, int h, int n, float gn_eps, uint64_t rows,
                                uint64_t slots) {
    if (n != 64) return RSV_FAIL("wkv7_seq: head_size must be 64 (got %d)", n);
    if (nseg <= 0 || rows == 0) return 0;
    {
        // two rows per lane group (two waves per head and segment, half the
        // LDS vector reads per state element): faster than one row (four
        // waves) at every chunk shape of a 64-session ragged prefill, including
        // chunks of few long segments (115.5k against 114.9k tok/s when one
        // row per group was used below 51 segments)
#define WKV_ROWS_LAUNCH(R)                                                                                            \
    hipLaunchKernelGGL(k_wkv7_seq_rows<R>, dim3(h, nseg), dim3(256 / (R)), 0, ctx->stream, s, r, w, k, v, a, kk, ka, rk, \
                       y_work, bonus_work, seg_start, seg_len, seg_slot, h, 1e-12f, rows, slots)
#define WKV_COLS_LAUNCH(G)                                                                                            \
    hipLaunchKernelGGL(k_wkv7_seq_cols<G>, dim3(h, nseg), dim3(64 * (G)), 0, ctx->stream, s, r, w, k, v, a, kk, ka, rk, \
                       y_work, bonus_work, seg_start, seg_len, seg_slot, h, 1e-12f, rows, slots)
        // (head, segment) blocks: with fewer than one per CU the launch is
        // the longest segment's dependent chain, shortened by more lanes per row
        const int blocks = h * nseg, cus = ctx->sm_count > 0 ? ctx->sm_count : 256;
        const char *e = getenv("RSV_SCAN_G");
        // From 16 blocks per CU (e.g. 256 sessions x 40 heads) four rows per
        // group (one wave per block, half the LDS vector reads per state
        // element again) keeps every SIMD busy: B=256 x T=512 5.09 -> 4.68 ms;
        // below that it leaves SIMDs idle (64 x 64 tokens: 192 -> 208 us)
        const int gsel = e ? atoi(e)
                           : (blocks * 4 <= cus ? 16 : blocks <= cus ? 8 : blocks >= 16 * cus ? -4 : 0);
        if (gsel == 16) WKV_COLS_LAUNCH(16);
        else if (gsel == 8) WKV_COLS_LAUNCH(8);
        else if (gsel == -4) WKV_ROWS_LAUNCH(4);
        else WKV_ROWS_LAUNCH(2);
#undef WKV_COLS_LAUNCH
#undef WKV_ROWS_LAUNCH
        const uint64_t units = rows * (uint64_t)h;
        hipLaunchKernelGGL(k_gn_gate_f16, dim3((unsigned)((units + 15) / 16)), dim3(256), 0, ctx->stream, y_work,
                           bonus_work, v, gamma, beta, g, yg, units, h, gn_eps);
    }
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
