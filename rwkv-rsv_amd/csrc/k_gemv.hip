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

namespace rsv {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float h2f(uint32_t b) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(b & 0xFFFFu));
}
__device__ __forceinline__ float sigmoid_f(float v) { return 1.0f / (1.0f + expf(-v)); }

template <int FMT, int LPR, int BT, int RU>
__device__ __forceinline__ void gemv_body(const GemvJob &J, int rb, int batch, float4 *xs, float *dxs) {
    constexpr int CW = FMT == FMT_I8 ? 16 : 8;  // weights per 16-byte chunk
    constexpr int P = CW / 4;                   // float4 parts of x per chunk
    constexpr int SLOTS = 64 / LPR;
    constexpr int U = 4;
    const int K = J.K, M = J.M, NC = K / CW;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int slot = lane / LPR, li = lane % LPR;
    const int rows_per_block = 4 * SLOTS * RU;
    const int rbase = rb * rows_per_block + (wave * SLOTS + slot) * RU;
    const int b0 = blockIdx.y * BT;
    const int nb = min(BT, batch - b0);
    const u32x4 *W = (const u32x4 *)J.w;
    const int KG = K / 128;

    // Stage x (with the prologue applied) into LDS, chunk-major.
    for (int e = tid; e < BT * NC; e += 256) {
        const int b = e / NC, c = e - (e / NC) * NC;
        float v[CW];
        if (b < nb) {
            const float4 *xp = (const float4 *)(J.x + (size_t)(b0 + b) * J.ldx + (size_t)c * CW);
#pragma unroll
            for (int p = 0; p < P; p++) {
                float4 t = xp[p];
                v[4 * p] = t.x; v[4 * p + 1] = t.y; v[4 * p + 2] = t.z; v[4 * p + 3] = t.w;
            }
            if (J.pro == PRO_MUL) {
                const float4 *gp = (const float4 *)(J.xmul + (size_t)(b0 + b) * J.ldx + (size_t)c * CW);
#pragma unroll
                for (int p = 0; p < P; p++) {
                    float4 t = gp[p];
                    v[4 * p] *= t.x; v[4 * p + 1] *= t.y; v[4 * p + 2] *= t.z; v[4 * p + 3] *= t.w;
                }
            } else if (J.pro == PRO_SIGMOID) {
#pragma unroll
                for (int i = 0; i < CW; i++) v[i] = sigmoid_f(v[i]);
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
    __syncthreads();

    float acc[RU][BT];
#pragma unroll
    for (int r = 0; r < RU; r++)
#pragma unroll
        for (int b = 0; b < BT; b++) acc[r][b] = 0.0f;

    const int NJ = (NC + LPR - 1) / LPR;
    for (int j0 = 0; j0 < NJ; j0 += U) {
        u32x4 wv[RU][U];
        uint32_t szv[RU][U];
#pragma unroll
        for (int r = 0; r < RU; r++) {
            const int row = rbase + r;
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int c = li + (j0 + u) * LPR;
                const bool ok = (c < NC) && (row < M);
                if (ok) {
                    wv[r][u] = __builtin_nontemporal_load(W + (size_t)row * NC + c);
                    if (FMT == FMT_I8) szv[r][u] = J.sz[(size_t)row * KG + (c >> 3)];
                } else {
                    wv[r][u] = (u32x4){0u, 0u, 0u, 0u};
                    if (FMT == FMT_I8) szv[r][u] = 0u;
                }
            }
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            int c = li + (j0 + u) * LPR;
            if (c >= NC) c = NC - 1;  // weights are zero there; keep the LDS read in range
#pragma unroll
            for (int b = 0; b < BT; b++) {
                float xv[CW];
#pragma unroll
                for (int p = 0; p < P; p++) {
                    float4 t = xs[(b * P + p) * NC + c];
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
    }

    // Reduce each (row, batch) sum across the LPR lanes of the slot.
#pragma unroll
    for (int r = 0; r < RU; r++)
#pragma unroll
        for (int b = 0; b < BT; b++) {
            float v = acc[r][b];
#pragma unroll
            for (int o = LPR / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
            acc[r][b] = v;
        }

    if (li == 0) {
#pragma unroll
        for (int r = 0; r < RU; r++) {
            const int row = rbase + r;
            if (row >= M) continue;
#pragma unroll
            for (int b = 0; b < BT; b++) {
                if (b >= nb) continue;
                const float v = acc[r][b];
                float *yp = J.y + (size_t)(b0 + b) * J.ldy + row;
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
                        const float vf = J.p1[(size_t)(b0 + b) * J.ldy + row];
                        *yp = cur + g * (vf - cur);
                    } break;
                    default: break;
                }
            }
        }
    }
}

template <int LPR, int BT, int RU>
__global__ __launch_bounds__(256) void k_gemv(GemvJobs jobs, int batch) {
    extern __shared__ float4 smem4[];
    const int bid = blockIdx.x;
    int ji = 0;
    while (ji + 1 < jobs.n && bid >= jobs.blk_start[ji + 1]) ji++;
    const GemvJob &J = jobs.j[ji];
    const int rb = bid - jobs.blk_start[ji];
    const int cw = J.fmt == FMT_I8 ? 16 : 8;
    float4 *xs = smem4;
    float *dxs = (float *)(smem4 + (size_t)BT * J.K / 4);
    (void)cw;
    if (J.fmt == FMT_I8)
        gemv_body<FMT_I8, LPR, BT, RU>(J, rb, batch, xs, dxs);
    else
        gemv_body<FMT_F16, LPR, BT, RU>(J, rb, batch, xs, dxs);
}

template <int LPR, int BT, int RU>
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
    hipLaunchKernelGGL((k_gemv<LPR, BT, RU>), grid, dim3(256), smem, ctx->stream, jobs, batch);
    RSV_HIP(hipGetLastError());
    return 0;
}

int launch_gemv_jobs(rsv_ctx *ctx, GemvJobs &jobs, int batch) {
    if (jobs.n <= 0 || jobs.n > kMaxJobs) return RSV_FAIL("gemv: bad job count %d", jobs.n);
    if (batch <= 0) return RSV_FAIL("gemv: batch must be >= 1 (got %d)", batch);
    int kmax = 0, ncmin = 1 << 30;
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
        if (J.epi == EPI_VLERP && !J.p1) return RSV_FAIL("gemv job %d: v-lerp needs v_first", i);
        if (J.epi == EPI_WDECAY && !J.scale) return RSV_FAIL("gemv job %d: decay needs scale", i);
        if (J.pro == PRO_MUL && !J.xmul) return RSV_FAIL("gemv job %d: mul prologue needs g", i);
        if (J.K > kmax) kmax = J.K;
        const int nc = J.K / (J.fmt == FMT_I8 ? 16 : 8);
        if (nc < ncmin) ncmin = nc;
    }
    // Lanes per row: a full wave when rows are long, a quarter wave for the
    // short LoRA-up rows (k = rank).
    const bool wide = ncmin >= 128;
    auto fits = [&](int bt) { return (size_t)bt * kmax * 4 * 17 / 16 <= 64 * 1024; };
    int bt = batch >= 4 ? 4 : (batch >= 2 ? 2 : 1);
    while (bt > 1 && !fits(bt)) bt >>= 1;
    if (!fits(bt)) return RSV_FAIL("gemv: k=%d too large for the LDS x stage", kmax);
    if (wide) {
        if (bt == 4) return launch_t<64, 4, 2>(ctx, jobs, batch);
        if (bt == 2) return launch_t<64, 2, 4>(ctx, jobs, batch);
        return launch_t<64, 1, 4>(ctx, jobs, batch);
    }
    if (bt == 4) return launch_t<16, 4, 2>(ctx, jobs, batch);
    if (bt == 2) return launch_t<16, 2, 2>(ctx, jobs, batch);
    return launch_t<16, 1, 2>(ctx, jobs, batch);
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
