// Weight GEMV with fused dequant for decode (batch <= a few sessions per
// block column).  HBM-bound: each weight byte is streamed exactly once per
// batch tile with 16-byte non-temporal loads; x is staged once per block in
// LDS in a chunk-major layout so that lanes reading consecutive chunks hit
// consecutive LDS addresses.
//
// One launch runs up to kMaxJobs independent matrices ("jobs"), which is how
// the reference's fused stage-1 (r/k/v + four LoRA-down projections,
// backend_cuda.rs:2949-3152) and LoRA stage-2 chain (backend_cuda.rs:
// 3162-3219) become single dispatches here.
//
// int8 format (model.rs:230-252): w[m,k] = s[m,k/128]*q[m,k] + z[m,k/128].
// For a 16-element chunk inside one 128-group the contribution is
// s*sum(x*q) + z*sum(x); sum(x) per chunk is precomputed while staging.
#include "rsv_common.h"
#include <cstdlib>
#include <algorithm>

namespace rsv {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float h2f(uint32_t b) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(b & 0xFFFFu));
}
__device__ __forceinline__ float sigmoid_f(float v) { return 1.0f / (1.0f + expf(-v)); }

// Epilogue of one output element y[b, row] (codes of GemvEpi).
__device__ __forceinline__ void apply_epi(const GemvJob &J, int row, int b, float v) {
    float *yp = J.y + (size_t)b * J.ldy + row;
    switch (J.epi) {
        case EPI_STORE: *yp = v; break;
        case EPI_RELU2: { const float t = v > 0.0f ? v : 0.0f; *yp = t * t; } break;
        case EPI_ADD: *yp = *yp + v; break;
        case EPI_TANH: *yp = tanhf(v); break;
        case EPI_WDECAY: *yp = expf(sigmoid_f(v + J.p0[row]) * J.scale[0]); break;
        case EPI_SIGBIAS: *yp = sigmoid_f(v + J.p0[row]); break;
        case EPI_VLERP: {
            const float g = sigmoid_f(v + J.p0[row]);
            const float cur = *yp;
            const float vf = J.p1[(size_t)b * J.ldy + row];
            *yp = cur + g * (vf - cur);
        } break;
        case EPI_STORE2:
            *yp = v;
            ((float *)J.p1)[(size_t)b * J.ldy + row] = v;
            break;
        default: break;
    }
}

// Sum over each aligned group of G lanes (16, 32 or 64) on DPP row
// operations; the result is valid in the last lane of each group (every lane
// for G = 16, lanes 31 and 63 for G = 32, lane 63 for G = 64).
template <int CTRL, int RM = 0xF>
__device__ __forceinline__ float gdpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, RM, 0xF, false));
}
template <int G>
__device__ __forceinline__ float group_sum_last(float v) {
    v += gdpp<0xB1>(v);        // quad_perm 1,0,3,2
    v += gdpp<0x4E>(v);        // quad_perm 2,3,0,1
    v += gdpp<0x141>(v);       // row_half_mirror
    v += gdpp<0x140>(v);       // row_mirror: 16-lane row sums
    if (G >= 32) v += gdpp<0x142, 0xA>(v);  // row_bcast:15 into rows 1 and 3: 32-lane sums in rows 1, 3
    if (G == 64) v += gdpp<0x143, 0xC>(v);  // row_bcast:31 into rows 2 and 3: total in row 3
    return v;
}

// Read operands of a row's epilogue, loaded at kernel entry by the lane that
// stores the row (a load after the block's barriers would be one more round
// trip at the end of the launch).
struct EpiPre {
    float y, p0, p1;
};
__device__ __forceinline__ EpiPre epi_prefetch(const GemvJob &J, int row, bool live) {
    EpiPre e{0.0f, 0.0f, 0.0f};
    if (!live) return e;
    if (J.epi == EPI_ADD || J.epi == EPI_VLERP) e.y = J.y[row];
    if (J.epi == EPI_WDECAY || J.epi == EPI_SIGBIAS || J.epi == EPI_VLERP) e.p0 = J.p0[row];
    if (J.epi == EPI_VLERP) e.p1 = J.p1[row];
    return e;
}
// apply_epi for batch row 0 with the operands of epi_prefetch.
__device__ __forceinline__ void apply_epi_pre(const GemvJob &J, int row, float v, const EpiPre &e) {
    float *yp = J.y + row;
    switch (J.epi) {
        case EPI_STORE: *yp = v; break;
        case EPI_RELU2: { const float t = v > 0.0f ? v : 0.0f; *yp = t * t; } break;
        case EPI_ADD: *yp = e.y + v; break;
        case EPI_TANH: *yp = tanhf(v); break;
        case EPI_WDECAY: *yp = expf(sigmoid_f(v + e.p0) * J.scale[0]); break;
        case EPI_SIGBIAS: *yp = sigmoid_f(v + e.p0); break;
        case EPI_VLERP: *yp = e.y + sigmoid_f(v + e.p0) * (e.p1 - e.y); break;
        case EPI_STORE2:
            *yp = v;
            ((float *)J.p1)[row] = v;
            break;
        default: break;
    }
}

__device__ __forceinline__ float block_sum_256(float v, float *red) {
    v = group_sum_last<64>(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 63) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return red[0] + red[1] + red[2] + red[3];
}

// Stages the (prologue-transformed) x rows of the block's batch tile into
// LDS, chunk-major: float4 part p of chunk c of row b sits at
// xs[(b*P + p)*NC + c], so lanes reading consecutive chunks read
// consecutive 16-byte LDS words.  For int8 weights the per-chunk sum of x
// (the zero-point term) goes to dxs[b*NC + c].
// LN-mix staging for rows of at most kLnPT*256 elements: every load of the
// block (x, prev, gamma, beta, coef) is issued up front in coalesced
// element order, the two-pass statistics are taken from registers, and the
// mixed row is scattered into the chunk-major LDS layout.  One memory
// latency per batch row instead of one per loop iteration.
constexpr int kLnPT = 16;
template <int FMT, int BT>
__device__ __forceinline__ void stage_x_lnmix(const GemvJob &J, int rb, int b0, int nb, float4 *xs, float *dxs,
                                              float *red) {
    constexpr int CW = FMT == FMT_I8 ? 16 : 8;
    constexpr int P = CW / 4;
    const int K = J.K, NC = K / CW, tid = threadIdx.x;
    float *xsf = (float *)xs;
    float gm[kLnPT], bt[kLnPT], cf[kLnPT];
#pragma unroll
    for (int j = 0; j < kLnPT; j++) {
        const int e = tid + 256 * j;
        const bool in = e < K;
        gm[j] = in ? J.gamma[e] : 0.0f;
        bt[j] = in ? J.beta[e] : 0.0f;
        cf[j] = in ? J.coef[e] : 0.0f;
    }
    const bool wr = J.lnout && rb == 0;
#pragma unroll
    for (int b = 0; b < BT; b++) {
        float xv[kLnPT], pv[kLnPT];
        const bool live = b < nb;
        const size_t ro = (size_t)(b0 + (live ? b : 0)) * J.ldx;
#pragma unroll
        for (int j = 0; j < kLnPT; j++) {
            const int e = tid + 256 * j;
            const bool in = live && e < K;
            xv[j] = in ? J.x[ro + e] : 0.0f;
            pv[j] = in ? J.prev[ro + e] : 0.0f;
        }
        // model.rs:625-635: mean, then the mean of squared deviations
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < kLnPT; j++) s += xv[j];
        const float mu = block_sum_256(s, red) / (float)K;
        float q = 0.0f;
#pragma unroll
        for (int j = 0; j < kLnPT; j++) {
            const int e = tid + 256 * j;
            const float d = xv[j] - mu;
            q += e < K ? d * d : 0.0f;
        }
        const float inv = 1.0f / sqrtf(block_sum_256(q, red) / (float)K + 1.0e-5f);
#pragma unroll
        for (int j = 0; j < kLnPT; j++) {
            const int e = tid + 256 * j;
            if (e >= K) continue;
            float v = 0.0f;
            if (live) {
                const float ln = (xv[j] - mu) * inv * gm[j] + bt[j];
                if (wr) J.lnout[ro + e] = ln;
                v = ln + cf[j] * (pv[j] - ln);
            }
            const int c = e / CW, r = e - c * CW;
            xsf[((b * P + (r >> 2)) * NC + c) * 4 + (r & 3)] = v;
        }
    }
    if (FMT == FMT_I8) {
        __syncthreads();
        for (int e = tid; e < BT * NC; e += 256) {
            const int b = e / NC, c = e - b * NC;
            float s = 0.0f;
#pragma unroll
            for (int p = 0; p < P; p++) {
                const float4 t = xs[(b * P + p) * NC + c];
                s += t.x; s += t.y; s += t.z; s += t.w;
            }
            dxs[b * NC + c] = s;
        }
    }
}

template <int FMT, int BT>
__device__ __forceinline__ void stage_x(const GemvJob &J, int rb, int b0, int nb, float4 *xs, float *dxs,
                                        float *red) {
    constexpr int CW = FMT == FMT_I8 ? 16 : 8;
    constexpr int P = CW / 4;
    const int K = J.K, NC = K / CW, tid = threadIdx.x;
    if (J.pro == PRO_LNMIX && K <= 256 * kLnPT) {
        stage_x_lnmix<FMT, BT>(J, rb, b0, nb, xs, dxs, red);
        return;
    }
    float mean[BT], inv[BT];
    if (J.pro == PRO_LNMIX) {
        // LayerNorm statistics of each batch row, two-pass (model.rs:625-635)
#pragma unroll
        for (int b = 0; b < BT; b++) {
            mean[b] = 0.0f;
            inv[b] = 0.0f;
            if (b >= nb) continue;
            const float *xr = J.x + (size_t)(b0 + b) * J.ldx;
            float s = 0.0f;
            for (int i = tid; i < K; i += 256) s += xr[i];
            const float mu = block_sum_256(s, red) / (float)K;
            float q = 0.0f;
            for (int i = tid; i < K; i += 256) { const float d = xr[i] - mu; q += d * d; }
            const float var = block_sum_256(q, red) / (float)K + 1.0e-5f;
            mean[b] = mu;
            inv[b] = 1.0f / sqrtf(var);
        }
    }
    for (int e = tid; e < BT * NC; e += 256) {
        const int b = e / NC, c = e - (e / NC) * NC;
        float v[CW];
        if (b < nb) {
            const size_t ro = (size_t)(b0 + b) * J.ldx + (size_t)c * CW;
            const float4 *xp = (const float4 *)(J.x + ro);
#pragma unroll
            for (int p = 0; p < P; p++) {
                const float4 t = xp[p];
                v[4 * p] = t.x; v[4 * p + 1] = t.y; v[4 * p + 2] = t.z; v[4 * p + 3] = t.w;
            }
            if (J.pro == PRO_MUL) {
                const float4 *gp = (const float4 *)(J.xmul + ro);
#pragma unroll
                for (int p = 0; p < P; p++) {
                    const float4 t = gp[p];
                    v[4 * p] *= t.x; v[4 * p + 1] *= t.y; v[4 * p + 2] *= t.z; v[4 * p + 3] *= t.w;
                }
            } else if (J.pro == PRO_SIGMOID) {
#pragma unroll
                for (int i = 0; i < CW; i++) v[i] = sigmoid_f(v[i]);
            } else if (J.pro == PRO_LNMIX) {
                const float *gm = J.gamma + (size_t)c * CW, *bt = J.beta + (size_t)c * CW;
                const float *pv = J.prev + ro, *cf = J.coef + (size_t)c * CW;
                float mu = 0.0f, is = 0.0f;
#pragma unroll
                for (int q = 0; q < BT; q++)
                    if (q == b) { mu = mean[q]; is = inv[q]; }
                const bool wr = J.lnout && rb == 0;
#pragma unroll
                for (int i = 0; i < CW; i++) {
                    const float ln = (v[i] - mu) * is * gm[i] + bt[i];
                    if (wr) J.lnout[ro + i] = ln;
                    v[i] = ln + cf[i] * (pv[i] - ln);
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < CW; i++) v[i] = 0.0f;
        }
#pragma unroll
        for (int p = 0; p < P; p++)
            xs[(b * P + p) * NC + c] = make_float4(v[4 * p], v[4 * p + 1], v[4 * p + 2], v[4 * p + 3]);
        if (FMT == FMT_I8) {
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < CW; i++) s += v[i];
            dxs[b * NC + c] = s;
        }
    }
}

// LPR lanes per row, BT batch rows per block, RU rows per lane slot, U
// 16-byte chunks per lane per load round; DB double-buffers load rounds
// (long rows), otherwise every round is loaded before it is used.
template <int FMT, int LPR, int BT, int RU, int U, bool DB>
__device__ __forceinline__ void gemv_body(const GemvJob &J, int rb, int batch, float4 *xs, float *dxs, float *red) {
    constexpr int CW = FMT == FMT_I8 ? 16 : 8;  // weights per 16-byte chunk
    constexpr int P = CW / 4;                   // float4 parts of x per chunk
    constexpr int SLOTS = 64 / LPR;
    const int K = J.K, M = J.M, NC = K / CW;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int slot = lane / LPR, li = lane % LPR;
    const int rows_per_block = 4 * SLOTS * RU;
    const int rbase = rb * rows_per_block + (wave * SLOTS + slot) * RU;
    const int b0 = blockIdx.y * BT;
    const int nb = min(BT, batch - b0);
    const u32x4 *W = (const u32x4 *)J.w;
    const int KG = K / 128;
    const int NJ = (NC + LPR - 1) / LPR;

    u32x4 wa[RU][U], wb[DB ? RU : 1][DB ? U : 1];
    uint32_t sa[RU][U], sb[DB ? RU : 1][DB ? U : 1];
    auto load = [&](u32x4 (&wv)[RU][U], uint32_t (&szv)[RU][U], int j0) {
#pragma unroll
        for (int r = 0; r < RU; r++) {
            const int row = rbase + r;
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int c = li + (j0 + u) * LPR;
                if (c < NC && row < M) {
                    wv[r][u] = __builtin_nontemporal_load(W + (size_t)row * NC + c);
                    if (FMT == FMT_I8) szv[r][u] = J.sz[(size_t)row * KG + (c >> 3)];
                } else {
                    wv[r][u] = (u32x4){0u, 0u, 0u, 0u};
                    if (FMT == FMT_I8) szv[r][u] = 0u;
                }
            }
        }
    };

    float acc[RU][BT];
#pragma unroll
    for (int r = 0; r < RU; r++)
#pragma unroll
        for (int b = 0; b < BT; b++) acc[r][b] = 0.0f;

    auto compute = [&](const u32x4 (&wv)[RU][U], const uint32_t (&szv)[RU][U], int j0) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            int c = li + (j0 + u) * LPR;
            if (c >= NC) c = NC - 1;  // weights are zero there; keep the LDS read in range
#pragma unroll
            for (int b = 0; b < BT; b++) {
                float xv[CW];
#pragma unroll
                for (int p = 0; p < P; p++) {
                    const float4 t = xs[(b * P + p) * NC + c];
                    xv[4 * p] = t.x; xv[4 * p + 1] = t.y; xv[4 * p + 2] = t.z; xv[4 * p + 3] = t.w;
                }
                if (FMT == FMT_I8) {
                    const float dx = dxs[b * NC + c];
#pragma unroll
                    for (int r = 0; r < RU; r++) {
                        float d = 0.0f;
#pragma unroll
                        for (int q = 0; q < 4; q++) {
                            const uint32_t wq = wv[r][u][q];
                            d = fmaf(xv[4 * q + 0], (float)(wq & 0xFFu), d);
                            d = fmaf(xv[4 * q + 1], (float)((wq >> 8) & 0xFFu), d);
                            d = fmaf(xv[4 * q + 2], (float)((wq >> 16) & 0xFFu), d);
                            d = fmaf(xv[4 * q + 3], (float)(wq >> 24), d);
                        }
                        const uint32_t s = szv[r][u];
                        acc[r][b] = fmaf(h2f(s), d, fmaf(h2f(s >> 16), dx, acc[r][b]));
                    }
                } else {
#pragma unroll
                    for (int r = 0; r < RU; r++) {
                        float d = acc[r][b];
#pragma unroll
                        for (int q = 0; q < 4; q++) {
                            const uint32_t wq = wv[r][u][q];
                            d = fmaf(xv[2 * q + 0], h2f(wq), d);
                            d = fmaf(xv[2 * q + 1], h2f(wq >> 16), d);
                        }
                        acc[r][b] = d;
                    }
                }
            }
        }
    };

    // Weight loads go out before x is staged: they do not depend on it.
    load(wa, sa, 0);
    stage_x<FMT, BT>(J, rb, b0, nb, xs, dxs, red);
    __syncthreads();
    if constexpr (DB) {
        for (int j0 = 0; j0 < NJ; j0 += 2 * U) {
            if (j0 + U < NJ) load(wb, sb, j0 + U);
            compute(wa, sa, j0);
            if (j0 + 2 * U < NJ) load(wa, sa, j0 + 2 * U);
            if (j0 + U < NJ) compute(wb, sb, j0 + U);
        }
    } else {
        for (int j0 = 0; j0 < NJ; j0 += U) {
            if (j0) load(wa, sa, j0);
            compute(wa, sa, j0);
        }
    }

    // Reduce each (row, batch) sum across the LPR lanes of the slot.
#pragma unroll
    for (int r = 0; r < RU; r++)
#pragma unroll
        for (int b = 0; b < BT; b++) {
            acc[r][b] = group_sum_last<LPR>(acc[r][b]);
        }

    if (li == LPR - 1) {
#pragma unroll
        for (int r = 0; r < RU; r++) {
            const int row = rbase + r;
            if (row >= M) continue;
#pragma unroll
            for (int b = 0; b < BT; b++) {
                if (b >= nb) continue;
                apply_epi(J, row, b0 + b, acc[r][b]);
            }
        }
    }
}

template <int LPR, int BT, int RU, int U, bool DB>
__global__ __launch_bounds__(256) void k_gemv(GemvJobs jobs, int batch) {
    extern __shared__ float4 smem4[];
    __shared__ float red[4];
    const int bid = blockIdx.x;
    if (jobs.side.src) {
        // side copy of this batch tile's rows, a share per block (one block
        // copying all of it would chain its round trips ahead of its rows)
        const int b0 = blockIdx.y * BT, nb = min(BT, batch - b0);
        const int tot = nb * jobs.side.n, per = (tot + (int)gridDim.x - 1) / (int)gridDim.x;
        const int end = min(tot, (bid + 1) * per);
        for (int i = bid * per + (int)threadIdx.x; i < end; i += 256)
            jobs.side.dst[(size_t)b0 * jobs.side.n + i] = jobs.side.src[(size_t)b0 * jobs.side.n + i];
    }
    int ji = 0;
    while (ji + 1 < jobs.n && bid >= jobs.blk_start[ji + 1]) ji++;
    const GemvJob &J = jobs.j[ji];
    const int rb = bid - jobs.blk_start[ji];
    float4 *xs = smem4;
    float *dxs = (float *)(smem4 + (size_t)BT * J.K / 4);
    if (J.fmt == FMT_I8)
        gemv_body<FMT_I8, LPR, BT, RU, U, DB>(J, rb, batch, xs, dxs, red);
    else
        gemv_body<FMT_F16, LPR, BT, RU, U, DB>(J, rb, batch, xs, dxs, red);
}

template <int LPR, int BT, int RU, int U, bool DB>
static int launch_t(rsv_ctx *ctx, GemvJobs &jobs, int batch) {
    const int rows_per_block = 4 * (64 / LPR) * RU;
    size_t smem = 0;
    int total = 0;
    for (int i = 0; i < jobs.n; i++) {
        GemvJob &J = jobs.j[i];
        J.nblk = (J.M + rows_per_block - 1) / rows_per_block;
        jobs.blk_start[i] = total;
        total += J.nblk;
        const int cw = J.fmt == FMT_I8 ? 16 : 8;
        size_t s = (size_t)BT * J.K * 4 + (J.fmt == FMT_I8 ? (size_t)BT * (J.K / cw) * 4 : 0);
        if (s > smem) smem = s;
    }
    jobs.blk_start[jobs.n] = total;
    dim3 grid(total, (batch + BT - 1) / BT);
    hipLaunchKernelGGL((k_gemv<LPR, BT, RU, U, DB>), grid, dim3(256), smem, ctx->stream, jobs, batch);
    RSV_HIP(hipGetLastError());
    return 0;
}

// ---------------------------------------------------------------- 2 <= B <= 16
// Batched decode GEMV that streams every weight byte once for up to 16
// sessions (the reference's gemv_variant_mb streams it once per 4 sessions,
// backend_cuda.rs:3381-3554).  With B sessions a VALU dot product costs B/2
// v_dot2 per weight pair, about the HBM time of the weights at B = 8; the
// products therefore run on v_mfma_f32_16x16x32_f16 with the sessions as the
// 16 rows of A (x, fp16) and 16 weight rows as the columns of B, and the
// kernel stays bound by the weight stream at every B <= 16.
//
//   - A block owns a range of rows of one job and one k-slice (<= kMfKS
//     columns).  It stages x of all sessions for the slice into LDS as fp16
//     (the job's prologue applied on the way; session-major rows padded by
//     16 bytes so the 16 session rows fall in different banks).
//   - A unit is 16 rows x 64 bytes of weights (64 int8 or 32 fp16 columns),
//     one 16-byte load per lane: lane (n = l%16, g = l/16) loads row n,
//     bytes 16g..16g+15 of the unit.  int8 pairs become the exact fp16
//     values 1024 + q (one v_perm each); the A operand of lane (m = l%16, g)
//     is x of session m at the same columns, so A and B pair up on the same
//     k.  D[session 4g+i][row n] lands in the lane that loaded row n.
//   - int8 (model.rs:234-252): a unit lies inside one 128-column group, so
//     s*sum(x*q) + z*sum(x) = s*D + (z - 1024*s)*dx with D the unit's MFMA
//     sum and dx the sum of the unit's fp16 x of the session (staged).
//   - Each wave streams its units through a kMfRing-deep register ring.
//     With >= 4 row tiles in the block a wave owns whole tiles; with fewer,
//     the four waves split the slice's units and their partial tiles meet in
//     LDS in wave order.
//   - Rows longer than kMfKS split into k-slices whose partial sums go to a
//     workspace; k_gemv_mb_reduce adds them in slice order and applies the
//     epilogue.
constexpr int kMfNT = 512;
constexpr int kMfKS = 2560;
constexpr int kMfXS = kMfKS + 8;  // LDS row stride of one session's x (halves)
constexpr int kMfRing = 8;
constexpr int kMfSlots = 4;  // row tiles one wave may touch (bounds the rows per block)
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));

// int8 bytes 2i, 2i+1 of w -> fp16 pair (1024 + q_lo, 1024 + q_hi)
__device__ __forceinline__ uint32_t q2h(uint32_t w, int pair) {
    return __builtin_amdgcn_perm(0x64646464u, w, pair ? 0x04030402u : 0x04010400u);
}

// Stages x[b, k0 .. k0+KS) for b < nb into LDS rows xs + b*kMfXS as fp16
// after the job's prologue; int8 jobs also get dx[unit*16 + b], the sum of
// the session's fp16 x over each 64-column unit.
template <int BT>
__device__ __forceinline__ void stage_x_mf(const GemvJob &J, int k0, int KS, int nb, bool wr_ln, _Float16 *xs,
                                           float *dx, float (*red)[4]) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const bool i8 = J.fmt == FMT_I8;
    const int NO = KS / 8;  // octets in the slice
    constexpr int UO = (kMfKS / 8 + kMfNT - 1) / kMfNT;
    const bool ln = J.pro == PRO_LNMIX;
    float4 g0[UO], g1[UO], e0[UO], e1[UO], c0[UO], c1[UO];
    if (ln) {
#pragma unroll
        for (int j = 0; j < UO; j++) {
            const int u = min(tid + kMfNT * j, NO - 1);
            const float4 *gp = (const float4 *)(J.gamma + 8 * u), *bp = (const float4 *)(J.beta + 8 * u),
                         *cp = (const float4 *)(J.coef + 8 * u);
            g0[j] = gp[0]; g1[j] = gp[1]; e0[j] = bp[0]; e1[j] = bp[1]; c0[j] = cp[0]; c1[j] = cp[1];
        }
    }
    // sessions in fours: every load of a group first, then its statistics
    constexpr int SG = 4;
    for (int b2 = 0; b2 < nb; b2 += SG) {
        float v[SG][UO][8], pv[SG][UO][8];
#pragma unroll
        for (int q = 0; q < SG; q++) {
            const int b = min(b2 + q, nb - 1);
            const size_t ro = (size_t)b * J.ldx + k0;
#pragma unroll
            for (int j = 0; j < UO; j++) {
                const int uc = min(tid + kMfNT * j, NO - 1);
                const float4 *xp = (const float4 *)(J.x + ro + 8 * uc);
                float4 a0 = xp[0], a1 = xp[1], m0 = make_float4(0.f, 0.f, 0.f, 0.f), m1 = m0;
                if (ln) {
                    const float4 *pp = (const float4 *)(J.prev + ro + 8 * uc);
                    m0 = pp[0]; m1 = pp[1];
                } else if (J.pro == PRO_MUL) {
                    const float4 *pp = (const float4 *)(J.xmul + ro + 8 * uc);
                    m0 = pp[0]; m1 = pp[1];
                }
                v[q][j][0] = a0.x; v[q][j][1] = a0.y; v[q][j][2] = a0.z; v[q][j][3] = a0.w;
                v[q][j][4] = a1.x; v[q][j][5] = a1.y; v[q][j][6] = a1.z; v[q][j][7] = a1.w;
                pv[q][j][0] = m0.x; pv[q][j][1] = m0.y; pv[q][j][2] = m0.z; pv[q][j][3] = m0.w;
                pv[q][j][4] = m1.x; pv[q][j][5] = m1.y; pv[q][j][6] = m1.z; pv[q][j][7] = m1.w;
            }
        }
        if (ln) {
            // LayerNorm of each session row (two-pass, model.rs:625-635)
            float mu[SG], inv[SG];
#pragma unroll
            for (int q = 0; q < SG; q++) {
                float s = 0.0f;
#pragma unroll
                for (int j = 0; j < UO; j++) {
                    if (tid + kMfNT * j >= NO) continue;
#pragma unroll
                    for (int e = 0; e < 8; e++) s += v[q][j][e];
                }
                s = group_sum_last<64>(s);
                if (lane == 63) red[wave][q] = s;
            }
            __syncthreads();
#pragma unroll
            for (int q = 0; q < SG; q++) {
                float t = 0.0f;
#pragma unroll
                for (int w = 0; w < kMfNT / 64; w++) t += red[w][q];
                mu[q] = t / (float)J.K;
            }
            __syncthreads();
#pragma unroll
            for (int q = 0; q < SG; q++) {
                float s = 0.0f;
#pragma unroll
                for (int j = 0; j < UO; j++) {
                    if (tid + kMfNT * j >= NO) continue;
#pragma unroll
                    for (int e = 0; e < 8; e++) { const float d = v[q][j][e] - mu[q]; s += d * d; }
                }
                s = group_sum_last<64>(s);
                if (lane == 63) red[wave][q] = s;
            }
            __syncthreads();
#pragma unroll
            for (int q = 0; q < SG; q++) {
                float t = 0.0f;
#pragma unroll
                for (int w = 0; w < kMfNT / 64; w++) t += red[w][q];
                inv[q] = 1.0f / sqrtf(t / (float)J.K + 1.0e-5f);
            }
            __syncthreads();
#pragma unroll
            for (int q = 0; q < SG; q++) {
                const int b = b2 + q;
#pragma unroll
                for (int j = 0; j < UO; j++) {
                    const int u = tid + kMfNT * j;
                    const float gm[8] = {g0[j].x, g0[j].y, g0[j].z, g0[j].w, g1[j].x, g1[j].y, g1[j].z, g1[j].w};
                    const float bt[8] = {e0[j].x, e0[j].y, e0[j].z, e0[j].w, e1[j].x, e1[j].y, e1[j].z, e1[j].w};
                    const float cf[8] = {c0[j].x, c0[j].y, c0[j].z, c0[j].w, c1[j].x, c1[j].y, c1[j].z, c1[j].w};
                    float l[8];
#pragma unroll
                    for (int e = 0; e < 8; e++) l[e] = (v[q][j][e] - mu[q]) * inv[q] * gm[e] + bt[e];
                    if (wr_ln && b < nb && u < NO) {
                        float4 *lp = (float4 *)(J.lnout + (size_t)b * J.ldx + 8 * u);
                        lp[0] = make_float4(l[0], l[1], l[2], l[3]);
                        lp[1] = make_float4(l[4], l[5], l[6], l[7]);
                    }
#pragma unroll
                    for (int e = 0; e < 8; e++) v[q][j][e] = l[e] + cf[e] * (pv[q][j][e] - l[e]);
                }
            }
        } else if (J.pro == PRO_MUL) {
#pragma unroll
            for (int q = 0; q < SG; q++)
#pragma unroll
                for (int j = 0; j < UO; j++)
#pragma unroll
                    for (int e = 0; e < 8; e++) v[q][j][e] *= pv[q][j][e];
        } else if (J.pro == PRO_SIGMOID) {
#pragma unroll
            for (int q = 0; q < SG; q++)
#pragma unroll
                for (int j = 0; j < UO; j++)
#pragma unroll
                    for (int e = 0; e < 8; e++) v[q][j][e] = sigmoid_f(v[q][j][e]);
        }
        // fp16 rows into LDS; int8 unit sums over the 8 octets of each unit
        // (8 consecutive lanes: quad sums, then the other quad by row_half_mirror)
#pragma unroll
        for (int q = 0; q < SG; q++) {
            const int b = b2 + q;
#pragma unroll
            for (int j = 0; j < UO; j++) {
                const int u = tid + kMfNT * j;
                h8_t h;
                float s = 0.0f;
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    h[e] = (_Float16)v[q][j][e];
                    s += (float)h[e];
                }
                if (b < nb && u < NO) *(h8_t *)(xs + b * kMfXS + 8 * u) = h;
                if (i8) {
                    s += gdpp<0xB1>(s);   // quad_perm 1,0,3,2
                    s += gdpp<0x4E>(s);   // quad_perm 2,3,0,1
                    s += gdpp<0x141>(s);  // row_half_mirror: the other quad of the 8
                    if (b < nb && u < NO && !(u & 7)) dx[(u >> 3) * 16 + b] = s;
                }
            }
        }
    }
}

template <int FMT, int BT>
__device__ __forceinline__ void gemv_mf_body(const GemvJob &J, int q, int batch, float *ws, _Float16 *xs, float *dx,
                                             float *part, float (*red)[4]) {
    constexpr int NW = kMfNT / 64;
    const int nks = J.ks, nbs = J.nblk / nks, ks = q / nbs, rb = q - ks * nbs;
    const int KS = J.K / nks, k0 = ks * KS, NS = KS * (FMT == FMT_I8 ? 1 : 2) / 64;  // units per row tile
    const int rbeg = rb * J.rpb, rend = min(J.M, rbeg + J.rpb), TB = (rend - rbeg + 15) / 16;
    const int tid = threadIdx.x, lane = tid & 63, n = lane & 15, g = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: the loop control stays scalar
    // the wave's units: an even share of the block's TB*NS units, tile-major
    const int U = TB * NS, ua = wave * U / NW, ub = (wave + 1) * U / NW, ta = ua / NS;
    const size_t rowb = (size_t)J.K * (FMT == FMT_I8 ? 1 : 2);  // bytes per weight row
    const unsigned char *W = (const unsigned char *)J.w + (size_t)k0 * (FMT == FMT_I8 ? 1 : 2) + 16 * g;
    const int KG = J.K / 128;
    // issue cursor: rows past the block's end (and units past the wave's end)
    // re-read the last valid ones, so every load is unconditional
    int it = ta, is = ua - ta * NS, iu = ua;
    const unsigned char *wp = W + (size_t)min(rbeg + 16 * it + n, rend - 1) * rowb;
    const uint32_t *sp = J.sz + (size_t)min(rbeg + 16 * it + n, rend - 1) * KG + k0 / 128;
    auto issue = [&](u32x4 &wv, uint32_t &sv) {
        wv = __builtin_nontemporal_load((const u32x4 *)(wp + 64 * is));
        if (FMT == FMT_I8) sv = sp[is >> 1];
        if (iu + 1 < ub) {
            iu++;
            if (++is == NS) {
                is = 0;
                it++;
                const int row = min(rbeg + 16 * it + n, rend - 1);
                wp = W + (size_t)row * rowb;
                if (FMT == FMT_I8) sp = J.sz + (size_t)row * KG + k0 / 128;
            }
        }
    };
    u32x4 ring[kMfRing];
    uint32_t szr[kMfRing];
#pragma unroll
    for (int p = 0; p < kMfRing; p++) issue(ring[p], szr[p]);
    stage_x_mf<BT>(J, k0, KS, batch, J.lnout && q == 0, xs, dx, red);
    __syncthreads();
    const int xm = min(n, batch - 1);  // A row of lane: session n (rows past the batch repeat the last one)
    const _Float16 *xrow = xs + xm * kMfXS + (FMT == FMT_I8 ? 16 : 8) * g;
    int ct = ta, cs = ua - ta * NS, slot = 0;
    f4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int u0 = ua; u0 < ub; u0 += kMfRing) {
#pragma unroll
        for (int p = 0; p < kMfRing; p++) {
            const int u = u0 + p;
            if (u >= ub) break;
            const u32x4 w = ring[p];
            if (FMT == FMT_I8) {
                const h8_t xa = *(const h8_t *)(xrow + 64 * cs), xb = *(const h8_t *)(xrow + 64 * cs + 8);
                const uint32_t s = szr[p];
                const h8_t wa = __builtin_bit_cast(h8_t, (u32x4){q2h(w[0], 0), q2h(w[0], 1), q2h(w[1], 0), q2h(w[1], 1)});
                const h8_t wb = __builtin_bit_cast(h8_t, (u32x4){q2h(w[2], 0), q2h(w[2], 1), q2h(w[3], 0), q2h(w[3], 1)});
                f4_t d = {0.0f, 0.0f, 0.0f, 0.0f};
                d = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa, wa, d, 0, 0, 0);
                d = __builtin_amdgcn_mfma_f32_16x16x32_f16(xb, wb, d, 0, 0, 0);
                const f4_t dxv = *(const f4_t *)(dx + cs * 16 + 4 * g);
                const float sc = h2f(s), zc = h2f(s >> 16) - 1024.0f * sc;
#pragma unroll
                for (int i = 0; i < 4; i++) acc[i] = fmaf(sc, d[i], fmaf(zc, dxv[i], acc[i]));
            } else {
                const h8_t xa = *(const h8_t *)(xrow + 32 * cs);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa, __builtin_bit_cast(h8_t, w), acc, 0, 0, 0);
            }
            issue(ring[p], szr[p]);
            if (++cs == NS || u == ub - 1) {
                // the wave's sum over tile ct (all of it or its share): D[session 4g+i][row n]
                *(f4_t *)(part + ((wave * kMfSlots + slot) * 16 + n) * 16 + 4 * g) = acc;
                acc = (f4_t){0.0f, 0.0f, 0.0f, 0.0f};
                slot++;
                if (cs == NS) { cs = 0; ct++; }
            }
        }
    }
    // every tile: the sums of the waves that cover it, in wave order
    __syncthreads();
    float *wsp = nks > 1 ? ws + J.wso + (size_t)ks * batch * J.M : nullptr;
    for (int e = tid; e < TB * 256; e += kMfNT) {
        const int t = e >> 8, nn = (e >> 4) & 15, b = e & 15, row = rbeg + 16 * t + nn;
        if (b >= batch || row >= rend) continue;
        int w = min(NW - 1, t * NS * NW / U);
        while (w > 0 && (w * U / NW) > t * NS) w--;  // first wave with a unit of tile t
        float v = 0.0f;
        bool any = false;
        for (; w < NW; w++) {
            const int wa = w * U / NW, wb = (w + 1) * U / NW;
            if (wa >= (t + 1) * NS) break;
            if (wb <= t * NS || wa >= wb) continue;
            const float pv = part[((w * kMfSlots + (t - wa / NS)) * 16 + nn) * 16 + b];
            v = any ? v + pv : pv;
            any = true;
        }
        if (wsp) wsp[(size_t)b * J.M + row] = v;
        else apply_epi(J, row, b, v);
    }
}

template <int BT>
__global__ __launch_bounds__(kMfNT) void k_gemv_mb(GemvJobs jobs, int batch, float *ws) {
    __shared__ __attribute__((aligned(16))) _Float16 xs[BT * kMfXS];
    __shared__ __attribute__((aligned(16))) float dx[kMfKS / 64 * 16];
    __shared__ __attribute__((aligned(16))) float part[kMfNT / 64 * kMfSlots * 256];
    __shared__ float red[kMfNT / 64][4];
    const int bid = blockIdx.x;
    if (jobs.side.src) {
        // side copy, a share per block (see k_gemv)
        const int tot = batch * jobs.side.n, per = (tot + (int)gridDim.x - 1) / (int)gridDim.x;
        const int end = min(tot, (bid + 1) * per);
        for (int i = bid * per + (int)threadIdx.x; i < end; i += kMfNT) jobs.side.dst[i] = jobs.side.src[i];
    }
    int ji = 0;
    while (ji + 1 < jobs.n && bid >= jobs.blk_start[ji + 1]) ji++;
    const GemvJob &J = jobs.j[ji];
    const int q = bid - jobs.blk_start[ji];
    if (J.fmt == FMT_I8)
        gemv_mf_body<FMT_I8, BT>(J, q, batch, ws, xs, dx, part, red);
    else
        gemv_mf_body<FMT_F16, BT>(J, q, batch, ws, xs, dx, part, red);
}

// y[b, row] (epilogue) of the k-sliced jobs: the slices' partial sums added
// in slice order.
__global__ __launch_bounds__(256) void k_gemv_mb_reduce(GemvJobs jobs, int batch, const float *ws) {
    int ji = 0;
    while (ji + 1 < jobs.n && (int)blockIdx.x >= jobs.blk_start[ji + 1]) ji++;
    const GemvJob &J = jobs.j[ji];
    const int i = (blockIdx.x - jobs.blk_start[ji]) * 256 + threadIdx.x;
    if (J.ks <= 1 || i >= J.M * batch) return;
    const int b = i / J.M, row = i - b * J.M;
    const float *p = ws + J.wso + i;
    float s = p[0];
    for (int k = 1; k < J.ks; k++) s += p[(size_t)k * batch * J.M];
    apply_epi(J, row, b, s);
}

// 2 <= batch <= 16 on k_gemv_mb.  Returns 1 when a job does not fit it.
static int launch_mb(rsv_ctx *ctx, GemvJobs &jobs, int batch) {
    if (batch > 16) return 1;
    double total = 0.0;
    double bytes[kMaxJobs];
    for (int i = 0; i < jobs.n; i++) {
        GemvJob &J = jobs.j[i];
        const int nks = (J.K + kMfKS - 1) / kMfKS;
        const int KS = J.K / nks;
        if (J.K % nks || KS % (J.fmt == FMT_I8 ? 128 : 32) || J.pro == PRO_GNGATE || (J.pro == PRO_LNMIX && nks > 1))
            return 1;
        J.ks = nks;
        bytes[i] = (double)J.M * J.K * (J.fmt == FMT_I8 ? 1.03125 : 2.0);
        total += bytes[i];
    }
    const int cus = ctx->sm_count > 0 ? ctx->sm_count : 256;
    const int target = cus;
    int nblk = 0;
    size_t wso = 0;
    for (int i = 0; i < jobs.n; i++) {
        GemvJob &J = jobs.j[i];
        int per = (int)(target * bytes[i] / total / J.ks + 0.5);
        per = std::max(1, std::min((J.M + 15) / 16, per));
        // a wave covers TB/8 tiles + 1 boundary tile: at most kMfSlots
        per = std::max(per, (J.M + 16 * 8 * (kMfSlots - 1) - 1) / (16 * 8 * (kMfSlots - 1)));
        J.rpb = (J.M + per - 1) / per;
        per = (J.M + J.rpb - 1) / J.rpb;
        J.nblk = per * J.ks;
        jobs.blk_start[i] = nblk;
        nblk += J.nblk;
        J.wso = wso;
        if (J.ks > 1) wso += (size_t)J.ks * batch * J.M;
    }
    jobs.blk_start[jobs.n] = nblk;
    if (wso > ctx->skinny_ws_cap) return RSV_FAIL("gemv: k-slice workspace too small (%zu floats)", wso);
    const int bt = batch <= 2 ? 2 : batch <= 4 ? 4 : batch <= 8 ? 8 : 16;
#define MB(BT) hipLaunchKernelGGL((k_gemv_mb<BT>), dim3(nblk), dim3(kMfNT), 0, ctx->stream, jobs, batch, ctx->skinny_ws)
    if (bt == 2) MB(2);
    else if (bt == 4) MB(4);
    else if (bt == 8) MB(8);
    else MB(16);
#undef MB
    RSV_HIP(hipGetLastError());
    if (wso) {
        GemvJobs rj = jobs;
        int rb = 0;
        for (int i = 0; i < rj.n; i++) {
            rj.blk_start[i] = rb;
            rb += rj.j[i].ks > 1 ? (rj.j[i].M * batch + 255) / 256 : 0;
        }
        rj.blk_start[rj.n] = rb;
        hipLaunchKernelGGL(k_gemv_mb_reduce, dim3(rb), dim3(256), 0, ctx->stream, rj, batch, (const float *)ctx->skinny_ws);
        RSV_HIP(hipGetLastError());
    }
    return 0;
}

// ---------------------------------------------------------------- B = 1
// One-shot GEMV for one session: NT threads per block (NT/64 waves x 64/LPR
// rows each).  Every vector load of the block (x and, for the LN-mix
// prologue, gamma/beta/coef/prev) goes out before the weight loads and
// returns ahead of them (vector memory returns in order), so the prologue
// runs while the weights stream.  The per-chunk sums of x (zero-point term
// of the int8 dot) are taken once per block into LDS instead of once per
// row.  Wide blocks mean fewer copies of x and of the LN vectors per CU,
// and one LN per 10-20 rows.
template <int NT>
__device__ __forceinline__ float block_sum_nt(float v, float *red) {
    v = group_sum_last<64>(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 63) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float t = red[0];
#pragma unroll
    for (int w = 1; w < NT / 64; w++) t += red[w];
    return t;
}

// PV: vectors the prologue may need (0 x only, 1 x and the gate, 2 the LN-mix set)
template <int FMT, int LPR, int CPL, int Q, int NT, int PV>
__device__ __forceinline__ void gemv_os2_body(const GemvJob &J, int rb, float4 *xs, float *red) {
    constexpr int CW = FMT == FMT_I8 ? 16 : 8;
    constexpr int P = CW / 4;
    constexpr int SLOTS = 64 / LPR, NW = NT / 64;
    const int K = J.K, M = J.M, NC = K / CW, KG = K / 128, K4 = K / 4;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int slot = lane / LPR, li = lane % LPR;
    const int row0 = (rb * NW + wave) * SLOTS + slot;
    const int row = min(row0, M - 1);
    const bool ln = PV == 2 && J.pro == PRO_LNMIX, mul = PV >= 1 && J.pro == PRO_MUL;
    const bool gn = PV == 2 && J.pro == PRO_GNGATE;
    // 1. vectors (clamped addresses; lanes past K are zeroed after the loads)
    const float4 *X4 = (const float4 *)J.x;
    float4 xa[Q], ga[PV >= 1 ? Q : 1], ba[PV == 2 ? Q : 1], ca[PV == 2 ? Q : 1], pa[PV == 2 ? Q : 1];
#pragma unroll
    for (int i = 0; i < Q; i++) {
        const int q = min(tid + NT * i, K4 - 1);
        xa[i] = X4[q];
        if constexpr (PV == 2) {
            if (ln || gn) {
                ga[i] = ((const float4 *)J.gamma)[q];
                ba[i] = ((const float4 *)J.beta)[q];
                ca[i] = ((const float4 *)(ln ? J.coef : J.xmul))[q];
                pa[i] = ((const float4 *)J.prev)[q];
            }
        }
        if constexpr (PV >= 1) {
            if (mul) ga[i] = ((const float4 *)J.xmul)[q];
        }
    }
    // 2. weights of the block's rows, all in flight
    const u32x4 *W = (const u32x4 *)J.w;
    u32x4 wv[CPL];
    uint32_t szv[CPL];
#pragma unroll
    for (int j = 0; j < CPL; j++) {
        const int c = min(li + LPR * j, NC - 1);
        wv[j] = __builtin_nontemporal_load(W + (size_t)row * NC + c);
        if (FMT == FMT_I8) szv[j] = J.sz[(size_t)row * KG + (c >> 3)];
    }
    const EpiPre ep = epi_prefetch(J, row0, li == LPR - 1 && row0 < M);
    // 3. prologue
#pragma unroll
    for (int i = 0; i < Q; i++)
        if (tid + NT * i >= K4) xa[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    if constexpr (PV == 2) {
      if (ln) {
        // LN over the row (two-pass, model.rs:625-635), then the token-shift mix
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < Q; i++) s += (xa[i].x + xa[i].y) + (xa[i].z + xa[i].w);
        const float mu = block_sum_nt<NT>(s, red) / (float)K;
        float v2 = 0.0f;
#pragma unroll
        for (int i = 0; i < Q; i++) {
            if (tid + NT * i >= K4) continue;
            const float d0 = xa[i].x - mu, d1 = xa[i].y - mu, d2 = xa[i].z - mu, d3 = xa[i].w - mu;
            v2 += (d0 * d0 + d1 * d1) + (d2 * d2 + d3 * d3);
        }
        const float inv = 1.0f / sqrtf(block_sum_nt<NT>(v2, red) / (float)K + 1.0e-5f);
        const bool wr = J.lnout && rb == 0;
#pragma unroll
        for (int i = 0; i < Q; i++) {
            const int q = tid + NT * i;
            if (q >= K4) continue;
            float4 l;
            l.x = (xa[i].x - mu) * inv * ga[i].x + ba[i].x;
            l.y = (xa[i].y - mu) * inv * ga[i].y + ba[i].y;
            l.z = (xa[i].z - mu) * inv * ga[i].z + ba[i].z;
            l.w = (xa[i].w - mu) * inv * ga[i].w + ba[i].w;
            if (wr) ((float4 *)J.lnout)[q] = l;
            xa[i].x = l.x + ca[i].x * (pa[i].x - l.x);
            xa[i].y = l.y + ca[i].y * (pa[i].y - l.y);
            xa[i].z = l.z + ca[i].z * (pa[i].z - l.z);
            xa[i].w = l.w + ca[i].w * (pa[i].w - l.w);
        }
      }
    }
    if constexpr (PV == 2) {
      if (gn) {
        // GroupNorm over each 64 columns (two-pass, eps inside the sqrt): the
        // 16 float4 of a group sit in 16 consecutive threads (one DPP row),
        // then ((d * rstd * gamma + beta) + bonus) * gate (model.rs:803-826)
#pragma unroll
        for (int i = 0; i < Q; i++) {
            const float mu = group_sum_last<16>((xa[i].x + xa[i].y) + (xa[i].z + xa[i].w)) * (1.0f / 64.0f);
            const float d0 = xa[i].x - mu, d1 = xa[i].y - mu, d2 = xa[i].z - mu, d3 = xa[i].w - mu;
            const float var = group_sum_last<16>((d0 * d0 + d1 * d1) + (d2 * d2 + d3 * d3)) * (1.0f / 64.0f) + J.eps;
            const float inv = 1.0f / sqrtf(var);
            xa[i].x = (d0 * inv * ga[i].x + ba[i].x + pa[i].x) * ca[i].x;
            xa[i].y = (d1 * inv * ga[i].y + ba[i].y + pa[i].y) * ca[i].y;
            xa[i].z = (d2 * inv * ga[i].z + ba[i].z + pa[i].z) * ca[i].z;
            xa[i].w = (d3 * inv * ga[i].w + ba[i].w + pa[i].w) * ca[i].w;
        }
      }
    }
    if constexpr (PV >= 1) {
        if (mul) {
#pragma unroll
            for (int i = 0; i < Q; i++) {
                xa[i].x *= ga[i].x; xa[i].y *= ga[i].y; xa[i].z *= ga[i].z; xa[i].w *= ga[i].w;
            }
        }
    }
    if (J.pro == PRO_SIGMOID) {
#pragma unroll
        for (int i = 0; i < Q; i++) {
            if (tid + NT * i >= K4) continue;
            xa[i].x = sigmoid_f(xa[i].x); xa[i].y = sigmoid_f(xa[i].y);
            xa[i].z = sigmoid_f(xa[i].z); xa[i].w = sigmoid_f(xa[i].w);
        }
    }
    // 4. x chunk-major into LDS (float4 part p of chunk c at p*NC + c); for
    // int8 the chunk sums of x after it, from the 4 lanes holding the chunk
    float *dxs = reinterpret_cast<float *>(xs + K4);
#pragma unroll
    for (int i = 0; i < Q; i++) {
        const int q = tid + NT * i;
        if (q < K4) xs[((4 * q) % CW >> 2) * NC + (4 * q) / CW] = xa[i];
        if (FMT == FMT_I8) {
            float cs = (xa[i].x + xa[i].y) + (xa[i].z + xa[i].w);
            cs += gdpp<0xB1>(cs);  // quad_perm 1,0,3,2
            cs += gdpp<0x4E>(cs);  // quad_perm 2,3,0,1: the chunk's sum in its 4 lanes
            if (q < K4 && (q & 3) == 0) dxs[q >> 2] = cs;
        }
    }
    __syncthreads();
    // 5. dot products
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < CPL; j++) {
        const int cr = li + LPR * j;
        const bool live = cr < NC;
        const int c = live ? cr : NC - 1;
        float xv[CW];
#pragma unroll
        for (int p = 0; p < P; p++) {
            const float4 t = xs[p * NC + c];
            xv[4 * p] = t.x; xv[4 * p + 1] = t.y; xv[4 * p + 2] = t.z; xv[4 * p + 3] = t.w;
        }
        if (FMT == FMT_I8) {
            // w = s*q + z over one 16-weight chunk of a 128-group (model.rs:234-252)
            const float dx = dxs[c];
            float d = 0.0f;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const uint32_t wq = wv[j][q];
                d = fmaf(xv[4 * q + 0], (float)(wq & 0xFFu), d);
                d = fmaf(xv[4 * q + 1], (float)((wq >> 8) & 0xFFu), d);
                d = fmaf(xv[4 * q + 2], (float)((wq >> 16) & 0xFFu), d);
                d = fmaf(xv[4 * q + 3], (float)(wq >> 24), d);
            }
            const uint32_t sw = live ? szv[j] : 0u;
            acc = fmaf(h2f(sw), d, fmaf(h2f(sw >> 16), dx, acc));
        } else {
            float d = 0.0f;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const uint32_t wq = wv[j][q];
                d = fmaf(xv[2 * q + 0], h2f(wq), d);
                d = fmaf(xv[2 * q + 1], h2f(wq >> 16), d);
            }
            acc += live ? d : 0.0f;
        }
    }
    acc = group_sum_last<LPR>(acc);
    if (li == LPR - 1 && row0 < M) apply_epi_pre(J, row0, acc, ep);
}

template <int CPL, int Q, int NT, int PV>
__global__ __launch_bounds__(NT) void k_gemv_os2(GemvJobs jobs) {
    extern __shared__ float4 xs4[];
    __shared__ float red[NT / 64];
    const int bid = blockIdx.x;
    int ji = 0;
    while (ji + 1 < jobs.n && bid >= jobs.blk_start[ji + 1]) ji++;
    const GemvJob &J = jobs.j[ji];
    const int rb = bid - jobs.blk_start[ji];
    if (J.fmt == FMT_I8) {
        if (J.lpr == 32) gemv_os2_body<FMT_I8, 32, CPL, Q, NT, PV>(J, rb, xs4, red);
        else gemv_os2_body<FMT_I8, 64, CPL, Q, NT, PV>(J, rb, xs4, red);
    } else {
        if (J.lpr == 32) gemv_os2_body<FMT_F16, 32, CPL, Q, NT, PV>(J, rb, xs4, red);
        else gemv_os2_body<FMT_F16, 64, CPL, Q, NT, PV>(J, rb, xs4, red);
    }
    // side copy, a share per block after the block's own rows (one block
    // copying the whole vector up front chained its round trips ahead of
    // that block's weight stream)
    if (jobs.side.src) {
        const int per = (jobs.side.n + (int)gridDim.x - 1) / (int)gridDim.x;
        const int end = min(jobs.side.n, (bid + 1) * per);
        for (int i = bid * per + (int)threadIdx.x; i < end; i += NT) jobs.side.dst[i] = jobs.side.src[i];
    }
}

// B=1 launch on k_gemv_os2 (prologues in the kernel).  640-thread blocks
// for LN-mix launches and rows longer than 2560, 320 otherwise (measured on
// the 3B decode shapes).  Returns 1 when the jobs do not fit.
static int launch_os2(rsv_ctx *ctx, GemvJobs &jobs) {
    int cpl_max = 0, kmax = 0;
    bool lnmix = false, gate = false, gngate = false;
    for (int i = 0; i < jobs.n; i++) {
        GemvJob &J = jobs.j[i];
        const int nc = J.K / (J.fmt == FMT_I8 ? 16 : 8);
        J.lpr = nc <= 32 * 5 ? 32 : 64;
        const int cpl = (nc + J.lpr - 1) / J.lpr;
        if (cpl > 10 || J.K % 16 != 0 || nc < J.lpr / 2) return 1;
        cpl_max = std::max(cpl_max, cpl);
        kmax = std::max(kmax, J.K);
        lnmix |= J.pro == PRO_LNMIX;
        gngate |= J.pro == PRO_GNGATE;
        gate |= J.pro == PRO_MUL;
    }
    const int nt = (lnmix || kmax > 2560) ? 640 : 320;
    const int qn = (kmax / 4 + nt - 1) / nt;
    const int q = qn <= 1 ? 1 : qn <= 2 ? 2 : qn <= 4 ? 4 : 0;
    if (!q || ((lnmix || gngate) && q > 2)) return 1;
    int total = 0;
    for (int i = 0; i < jobs.n; i++) {
        GemvJob &J = jobs.j[i];
        const int rpb = (nt / 64) * (64 / J.lpr);
        J.nblk = (J.M + rpb - 1) / rpb;
        jobs.blk_start[i] = total;
        total += J.nblk;
    }
    jobs.blk_start[jobs.n] = total;
    const size_t lds = (size_t)kmax * 4 + (size_t)kmax / 16 * 4;
#define OS2(C, QQ, N, V) hipLaunchKernelGGL((k_gemv_os2<C, QQ, N, V>), dim3(total), dim3(N), lds, ctx->stream, jobs)
    const bool c5 = cpl_max <= 5;
    if (lnmix || (gngate && nt == 640)) {
        if (q == 1) { if (c5) OS2(5, 1, 640, 2); else OS2(10, 1, 640, 2); }
        else { if (c5) OS2(5, 2, 640, 2); else OS2(10, 2, 640, 2); }
    } else if (gngate) {  // the GroupNorm-gate operand of att.output: 320-thread blocks as plain k <= 2560
        if (q == 1) OS2(5, 1, 320, 2); else OS2(5, 2, 320, 2);
    } else if (nt == 320) {  // k <= 2560: at most 5 chunks per lane
        if (q == 1) { if (gate) OS2(5, 1, 320, 1); else OS2(5, 1, 320, 0); }
        else { if (gate) OS2(5, 2, 320, 1); else OS2(5, 2, 320, 0); }
    } else {
        if (q <= 2) {
            if (gate) { if (c5) OS2(5, 2, 640, 1); else OS2(10, 2, 640, 1); }
            else { if (c5) OS2(5, 2, 640, 0); else OS2(10, 2, 640, 0); }
        } else {
            if (gate) { if (c5) OS2(5, 4, 640, 1); else OS2(10, 4, 640, 1); }
            else { if (c5) OS2(5, 4, 640, 0); else OS2(10, 4, 640, 0); }
        }
    }
#undef OS2
    RSV_HIP(hipGetLastError());
    return 0;
}

int launch_gemv_jobs(rsv_ctx *ctx, GemvJobs &jobs, int batch) {
    if (jobs.n <= 0 || jobs.n > kMaxJobs) return RSV_FAIL("gemv: bad job count %d", jobs.n);
    if (batch <= 0) return RSV_FAIL("gemv: batch must be >= 1 (got %d)", batch);
    int kmax = 0, ncmin = 1 << 30, ncmax = 0;
    for (int i = 0; i < jobs.n; i++) {
        const GemvJob &J = jobs.j[i];
        if (!J.w || !J.x || !J.y) return RSV_FAIL("gemv job %d: null operand", i);
        if (J.M <= 0 || J.K <= 0) return RSV_FAIL("gemv job %d: bad shape m=%d k=%d", i, J.M, J.K);
        if (J.fmt == FMT_I8 && (J.K % 128 != 0 || !J.sz))
            return RSV_FAIL("gemv job %d: int8 needs k %% 128 == 0 (k=%d) and a scale/zero tensor", i, J.K);
        if (J.fmt == FMT_F16 && J.K % 8 != 0) return RSV_FAIL("gemv job %d: fp16 needs k %% 8 == 0 (k=%d)", i, J.K);
        if (J.ldx % 4 != 0) return RSV_FAIL("gemv job %d: x batch stride must be a multiple of 4", i);
        if ((J.epi == EPI_WDECAY || J.epi == EPI_SIGBIAS || J.epi == EPI_VLERP) && !J.p0)
            return RSV_FAIL("gemv job %d: epilogue needs a bias", i);
        if ((J.epi == EPI_VLERP || J.epi == EPI_STORE2) && !J.p1) return RSV_FAIL("gemv job %d: needs v_first", i);
        if (J.epi == EPI_WDECAY && !J.scale) return RSV_FAIL("gemv job %d: decay needs scale", i);
        if (J.pro == PRO_MUL && !J.xmul) return RSV_FAIL("gemv job %d: mul prologue needs g", i);
        if (J.pro == PRO_LNMIX && (!J.gamma || !J.beta || !J.prev || !J.coef))
            return RSV_FAIL("gemv job %d: LN-mix prologue needs gamma/beta/prev/coef", i);
        if (J.K > kmax) kmax = J.K;
        const int nc = J.K / (J.fmt == FMT_I8 ? 16 : 8);
        if (nc < ncmin) ncmin = nc;
        if (nc > ncmax) ncmax = nc;
    }
    if (jobs.side.src && (!jobs.side.dst || jobs.side.n <= 0)) return RSV_FAIL("gemv: bad side copy");
    // B=1: the one-shot kernel (prologues inside it) where the jobs fit it
    if (batch == 1) {
        const int rc = launch_os2(ctx, jobs);
        if (rc <= 0) return rc;
    }
    if (batch >= 2) {
        const int rc = launch_mb(ctx, jobs, batch);
        if (rc <= 0) return rc;
    }
    for (int i = 0; i < jobs.n; i++)
        if (jobs.j[i].pro == PRO_GNGATE) return RSV_FAIL("gemv: the GroupNorm-gate prologue runs on the one-session kernel only (k <= 10240)");
    // Lanes per row: a full wave when rows are long, a quarter wave for the
    // short LoRA-up rows (k = rank).  Long rows (ffn.value) keep fewer rows
    // per wave so more waves are resident.
    const bool wide = ncmin >= 128;
    const bool long_rows = ncmax > 6 * 64;
    auto fits = [&](int bt) { return (size_t)bt * kmax * 4 * 17 / 16 <= 64 * 1024; };
    int bt = batch >= 4 ? 4 : (batch >= 2 ? 2 : 1);
    while (bt > 1 && !fits(bt)) bt >>= 1;
    if (!fits(bt)) return RSV_FAIL("gemv: k=%d too large for the LDS x stage", kmax);
    if (wide) {
        if (long_rows) {
            if (bt == 4) return launch_t<64, 4, 1, 4, true>(ctx, jobs, batch);
            if (bt == 2) return launch_t<64, 2, 1, 4, true>(ctx, jobs, batch);
            return launch_t<64, 1, 1, 4, true>(ctx, jobs, batch);
        }
        if (bt == 4) return launch_t<64, 4, 1, 6, false>(ctx, jobs, batch);
        if (bt == 2) return launch_t<64, 2, 2, 6, false>(ctx, jobs, batch);
        return launch_t<64, 1, 2, 6, false>(ctx, jobs, batch);
    }
    if (bt == 4) return launch_t<16, 4, 2, 2, false>(ctx, jobs, batch);
    if (bt == 2) return launch_t<16, 2, 2, 2, false>(ctx, jobs, batch);
    return launch_t<16, 1, 2, 2, false>(ctx, jobs, batch);
}

// ---------------------------------------------------------------- dequant
// model.rs:234-252, element-exact: p = s*q (rounded) then p + z (rounded);
// no fma, matching the reference's CPU arithmetic bit for bit.
__global__ void k_dequant_int8(const uint32_t *idx, const uint32_t *sz, uint64_t m, uint64_t k, float *out32,
                               _Float16 *out16) {
    const uint64_t words = m * k / 4;
    for (uint64_t wi = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; wi < words;
         wi += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t e = wi * 4, row = e / k, col = e - row * k;
        const uint32_t s = sz[row * (k / 128) + col / 128];
        const float sc = h2f(s), zr = h2f(s >> 16);
        const uint32_t pack = idx[wi];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float q = (float)((pack >> (8 * j)) & 0xFFu);
            const float p = __fmul_rn(sc, q);
            const float w = __fadd_rn(p, zr);
            if (out32) out32[e + j] = w;
            if (out16) out16[e + j] = (_Float16)w;
        }
    }
}

int launch_dequant_int8(rsv_ctx *ctx, const uint32_t *idx, const uint32_t *sz, uint64_t m, uint64_t k,
                        void *out, int out_f16) {
    if (k % 128 != 0) return RSV_FAIL("dequant_int8: k=%llu not a multiple of 128", (unsigned long long)k);
    const uint64_t words = m * k / 4;
    uint64_t blocks = (words + 255) / 256;
    if (blocks > 65535 * 16) blocks = 65535 * 16;
    if (blocks == 0) return 0;
    hipLaunchKernelGGL(k_dequant_int8, dim3((unsigned)blocks), dim3(256), 0, ctx->stream, idx, sz, m, k,
                       out_f16 ? nullptr : (float *)out, out_f16 ? (_Float16 *)out : nullptr);
    RSV_HIP(hipGetLastError());
    return 0;
}

}  // namespace rsv
