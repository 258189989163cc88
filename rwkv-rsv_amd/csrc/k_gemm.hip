// Prefill GEMM on CDNA matrix cores: C[m,n] = epi(A[m,k] . B[n,k]^T).
//
// A (token activations) is fp16 row-major; B (weights, [out,in]) is fp16 or
// the reference int8 format, dequantised to fp16 in the tile loader
// (w = s*q + z in fp32, rounded to fp16 -- the same rounding as the
// reference's dequant-to-fp16 prefill scheme, backend_cuda.rs:4195-4227).
// Accumulation is fp32 (v_mfma_f32_32x32x16_f16).
//
// Tile: 128x128 per 256-thread block, BK = 32; each wave owns a 64x64
// quadrant as 2x2 MFMA 32x32 blocks.  The next K-slab is prefetched into
// registers while the current one is multiplied out of LDS.
#include "rsv_common.h"

namespace rsv {

typedef float float16_t __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4g __attribute__((ext_vector_type(4)));

constexpr int BM = 128, BN = 128, BK = 32, LDK = BK + 8;

__device__ __forceinline__ float sigm_g(float v) { return 1.0f / (1.0f + expf(-v)); }
__device__ __forceinline__ float h2f_g(uint32_t b) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(b & 0xFFFFu));
}

__device__ __forceinline__ uint32_t pack2(float a, float b) {
    const uint16_t lo = __builtin_bit_cast(uint16_t, (_Float16)a);
    const uint16_t hi = __builtin_bit_cast(uint16_t, (_Float16)b);
    return (uint32_t)lo | ((uint32_t)hi << 16);
}

// k_gemm2: a 128x128 tile, int8 or fp16 weight loaders, with the LDS
// stage double-buffered (one barrier per k-step: the next slab is written to
// the other buffer while this one is multiplied out) and the gfx950
// v_mfma_f32_32x32x16_f16 (16 k per instruction; lane l holds k 8*(l/32) ..
// +7 of each 16-k half of the 32-k slab, the same mapping for A and B).  The
// epilogue switches once on its kind (a per-element switch unrolled 64 times
// made the kernel body several thousand instructions long).
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));

template <int EPI>
__device__ __forceinline__ float gemm_epi_val(float v, float bias, float aux, float cur, float scale) {
    if constexpr (EPI == GE_BIAS) return v + bias;
    else if constexpr (EPI == GE_ADD) return v + aux;
    else if constexpr (EPI == GE_RELU2) return v > 0.0f ? v * v : 0.0f;
    else if constexpr (EPI == GE_TANH) return tanhf(v);
    else if constexpr (EPI == GE_WDECAY) return expf(sigm_g(v + bias) * scale);
    else if constexpr (EPI == GE_SIGBIAS) return sigm_g(v + bias);
    else if constexpr (EPI == GE_VLERP) return cur + sigm_g(v + bias) * (aux - cur);
    else if constexpr (EPI == GE_SIGMOID) return sigm_g(v);
    else return v;
}

template <int EPI, int MI, int NJ = 2>
__device__ __forceinline__ void gemm2_epilogue(const GemmArgs &g, const float16_t (&acc)[MI][NJ], int m0, int n0, int wm,
                                               int wn, int lane) {
    constexpr bool need_b = EPI == GE_BIAS || EPI == GE_WDECAY || EPI == GE_SIGBIAS || EPI == GE_VLERP;
    constexpr bool need_aux = EPI == GE_ADD || EPI == GE_VLERP;
    constexpr bool need_cur = EPI == GE_VLERP;
    const float scale = EPI == GE_WDECAY ? g.scale[0] : 0.0f;
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const int col = n0 + wn + j * 32 + (lane & 31);
        if (col >= g.n) continue;
        const float bias = need_b ? g.bias[col] : 0.0f;
#pragma unroll
        for (int i = 0; i < MI; i++) {
            // every read operand of the 32 x 32 tile first: the output may be
            // one of them (x += ..., v in place), so a load placed after a
            // store would wait for that store (loads and stores share one
            // counter here)
            float aux[16], cur[16];
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const int row = m0 + wm + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
                const size_t o = (size_t)row * g.ldc + col;
                aux[e] = need_aux && row < g.m ? g.aux[o] : 0.0f;
                cur[e] = need_cur && row < g.m ? ((const float *)g.c)[o] : 0.0f;
            }
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const int row = m0 + wm + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
                if (row >= g.m) continue;
                const size_t o = (size_t)row * g.ldc + col;
                const float v = gemm_epi_val<EPI>(acc[i][j][e], bias, aux[e], cur[e], scale);
                if (g.c_f16)
                    ((_Float16 *)g.c)[o] = (_Float16)v;
                else
                    ((float *)g.c)[o] = v;
            }
        }
    }
}

// BM2 rows (128 or 256) x 128 columns per block of 4 waves in a 2x2 layout:
// each wave owns (BM2/2) x 64 as (BM2/64) x 2 MFMA 32x32 tiles.
template <bool B_I8, int BM2>
__device__ __forceinline__ void gemm2_body(const GemmArgs &g, int m0, int n0, _Float16 (*As)[BM2 * LDK],
                                           _Float16 (*Bs)[BN * LDK]) {
    constexpr int MI = BM2 / 64;
    constexpr int PA = BM2 * BK / 8 / 256;  // 16-byte A pieces per thread
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int wm = (wave >> 1) * (BM2 / 2), wn = (wave & 1) * 64;
    const int lr = tid >> 1, lc = (tid & 1) * 16;  // B loader: row, first k of 16

    float16_t acc[MI][2];
#pragma unroll
    for (int i = 0; i < MI; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[i][j][e] = 0.0f;

    u32x4g ra[PA], rb[2];
    uint32_t rsz = 0;
    const int brow = n0 + lr;
    const bool bok = brow < g.n;
    const int KG = g.k / 128;
    auto load = [&](int k0) {
#pragma unroll
        for (int i = 0; i < PA; i++) {
            const int p = tid + 256 * i, row = m0 + p / (BK / 8), c8 = p % (BK / 8);
            ra[i] = row < g.m ? *(const u32x4g *)(g.a + (size_t)row * g.lda + k0 + 8 * c8) : (u32x4g){0u, 0u, 0u, 0u};
        }
        if (B_I8) {
            if (bok) {
                rb[0] = *(const u32x4g *)((const uint8_t *)g.b + (size_t)brow * g.k + k0 + lc);
                rsz = g.sz[(size_t)brow * KG + (k0 + lc) / 128];
            } else {
                rb[0] = (u32x4g){0u, 0u, 0u, 0u};
                rsz = 0;
            }
        } else {
            if (bok) {
                const u32x4g *p = (const u32x4g *)((const _Float16 *)g.b + (size_t)brow * g.k + k0 + lc);
                rb[0] = p[0];
                rb[1] = p[1];
            } else {
                rb[0] = rb[1] = (u32x4g){0u, 0u, 0u, 0u};
            }
        }
    };
    auto stage = [&](int buf) {
#pragma unroll
        for (int i = 0; i < PA; i++) {
            const int p = tid + 256 * i;
            *(u32x4g *)(As[buf] + (p / (BK / 8)) * LDK + 8 * (p % (BK / 8))) = ra[i];
        }
        u32x4g *bd = (u32x4g *)(Bs[buf] + lr * LDK + lc);
        if (B_I8) {
            // w = s*q + z with the product and the sum each rounded to fp32
            // (model.rs:234-252), then rounded to fp16
            const float s = h2f_g(rsz), z = h2f_g(rsz >> 16);
            uint32_t o[8];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const uint32_t w = rb[0][q];
                const float w0 = __fadd_rn(__fmul_rn(s, (float)(w & 0xFFu)), z);
                const float w1 = __fadd_rn(__fmul_rn(s, (float)((w >> 8) & 0xFFu)), z);
                const float w2 = __fadd_rn(__fmul_rn(s, (float)((w >> 16) & 0xFFu)), z);
                const float w3 = __fadd_rn(__fmul_rn(s, (float)(w >> 24)), z);
                o[2 * q] = pack2(w0, w1);
                o[2 * q + 1] = pack2(w2, w3);
            }
            bd[0] = (u32x4g){o[0], o[1], o[2], o[3]};
            bd[1] = (u32x4g){o[4], o[5], o[6], o[7]};
        } else {
            bd[0] = rb[0];
            bd[1] = rb[1];
        }
    };

    load(0);
    stage(0);
    __syncthreads();
    int cur = 0;
    for (int k0 = 0; k0 < g.k; k0 += BK) {
        const bool more = k0 + BK < g.k;
        if (more) load(k0 + BK);
#pragma unroll
        for (int st = 0; st < 2; st++) {
            half8_t af[MI], bf[2];
#pragma unroll
            for (int i = 0; i < MI; i++)
                af[i] = *(const half8_t *)(As[cur] + (wm + i * 32 + (lane & 31)) * LDK + 16 * st + 8 * (lane >> 5));
#pragma unroll
            for (int j = 0; j < 2; j++)
                bf[j] = *(const half8_t *)(Bs[cur] + (wn + j * 32 + (lane & 31)) * LDK + 16 * st + 8 * (lane >> 5));
#pragma unroll
            for (int i = 0; i < MI; i++)
#pragma unroll
                for (int j = 0; j < 2; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        if (more) stage(cur ^ 1);
        __syncthreads();
        cur ^= 1;
    }
#define GEMM2_EPI(K) gemm2_epilogue<K, MI>(g, acc, m0, n0, wm, wn, lane)
    switch (g.epi) {
        case GE_BIAS: GEMM2_EPI(GE_BIAS); break;
        case GE_ADD: GEMM2_EPI(GE_ADD); break;
        case GE_RELU2: GEMM2_EPI(GE_RELU2); break;
        case GE_TANH: GEMM2_EPI(GE_TANH); break;
        case GE_WDECAY: GEMM2_EPI(GE_WDECAY); break;
        case GE_SIGBIAS: GEMM2_EPI(GE_SIGBIAS); break;
        case GE_VLERP: GEMM2_EPI(GE_VLERP); break;
        case GE_SIGMOID: GEMM2_EPI(GE_SIGMOID); break;
        default: GEMM2_EPI(GE_STORE); break;
    }
#undef GEMM2_EPI
}

template <bool B_I8, int BM2>
__global__ __launch_bounds__(256) void k_gemm2(GemmArgs g) {
    __shared__ __attribute__((aligned(16))) _Float16 As[2][BM2 * LDK];
    __shared__ __attribute__((aligned(16))) _Float16 Bs[2][BN * LDK];
    gemm2_body<B_I8, BM2>(g, blockIdx.y * BM2, blockIdx.x * BN, As, Bs);
}

// A job list in one launch: the block finds its job and tile (row-major over
// the job's n-tiles) and runs that job's body, int8 or fp16.
template <int BM2>
__global__ __launch_bounds__(256) void k_gemm2_multi(GemmJobs jobs) {
    __shared__ __attribute__((aligned(16))) _Float16 As[2][BM2 * LDK];
    __shared__ __attribute__((aligned(16))) _Float16 Bs[2][BN * LDK];
    const int bid = blockIdx.x;
    int ji = 0;
    while (ji + 1 < jobs.n && bid >= jobs.blk_start[ji + 1]) ji++;
    const GemmArgs &g = jobs.j[ji];
    const int local = bid - jobs.blk_start[ji], nt = (g.n + BN - 1) / BN;
    const int m0 = (local / nt) * BM2, n0 = (local % nt) * BN;
    if (g.b_i8)
        gemm2_body<true, BM2>(g, m0, n0, As, Bs);
    else
        gemm2_body<false, BM2>(g, m0, n0, As, Bs);
}

// Third form: the 128x128 tile of k_gemm2 with BKT (64 or 128) k per stage
// and one LDS buffer.  The next stage's loads are issued before the current
// stage is multiplied out, as in k_gemm2, but each stage carries 2x or 4x
// the bytes, so a block keeps 24 or 48 KB in flight instead of 12 KB (the
// stage-to-stage wait is a memory latency, several times a 32-k stage's
// MFMA work).  Two barriers per stage: all waves are done reading the
// buffer before it is overwritten.
template <bool B_I8, int BKT, int NJ, int BMR = 128>
__device__ __forceinline__ void gemm3_body(const GemmArgs &g, int m0, int n0, _Float16 *As, _Float16 *Bs) {
    constexpr int MI = BMR / 64, LD = BKT + 8, BNJ = 64 * NJ;  // block rows BMR, columns BNJ
    constexpr int PA = BMR * BKT / 8 / 256;   // 16-byte A pieces per thread
    constexpr int KH = BKT * BNJ / 256;       // k per thread of the B loader (256 / BNJ threads per row)
    constexpr int PB = B_I8 ? KH / 16 : KH / 8;  // its 16-byte pieces
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int wm = (wave >> 1) * (BMR / 2), wn = (wave & 1) * 32 * NJ;
    const int lr = tid / (256 / BNJ), lc = (tid % (256 / BNJ)) * KH;

    float16_t acc[MI][NJ];
#pragma unroll
    for (int i = 0; i < MI; i++)
#pragma unroll
        for (int j = 0; j < NJ; j++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[i][j][e] = 0.0f;

    u32x4g ra[PA], rb[PB];
    uint32_t rsz = 0;
    const int brow = n0 + lr;
    const bool bok = brow < g.n;
    const int KG = g.k / 128;
    auto load = [&](int k0) {
#pragma unroll
        for (int i = 0; i < PA; i++) {
            const int p = tid + 256 * i, row = m0 + p / (BKT / 8), c8 = p % (BKT / 8);
            ra[i] = row < g.m ? *(const u32x4g *)(g.a + (size_t)row * g.lda + k0 + 8 * c8) : (u32x4g){0u, 0u, 0u, 0u};
        }
        if (bok) {
            const u32x4g *bp = B_I8 ? (const u32x4g *)((const uint8_t *)g.b + (size_t)brow * g.k + k0 + lc)
                                    : (const u32x4g *)((const _Float16 *)g.b + (size_t)brow * g.k + k0 + lc);
#pragma unroll
            for (int e = 0; e < PB; e++) rb[e] = bp[e];
            // KH <= 64 consecutive k from a multiple of KH: one 128-group
            if (B_I8) rsz = g.sz[(size_t)brow * KG + (k0 + lc) / 128];
        } else {
#pragma unroll
            for (int e = 0; e < PB; e++) rb[e] = (u32x4g){0u, 0u, 0u, 0u};
            rsz = 0;
        }
    };
    auto stage = [&]() {
#pragma unroll
        for (int i = 0; i < PA; i++) {
            const int p = tid + 256 * i;
            *(u32x4g *)(As + (p / (BKT / 8)) * LD + 8 * (p % (BKT / 8))) = ra[i];
        }
        u32x4g *bd = (u32x4g *)(Bs + lr * LD + lc);
        if (B_I8) {
            // w = s*q + z with the product and the sum each rounded to fp32
            // (model.rs:234-252), then rounded to fp16
            const float s = h2f_g(rsz), z = h2f_g(rsz >> 16);
#pragma unroll
            for (int e = 0; e < PB; e++) {
                uint32_t o[8];
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const uint32_t w = rb[e][q];
                    const float w0 = __fadd_rn(__fmul_rn(s, (float)(w & 0xFFu)), z);
                    const float w1 = __fadd_rn(__fmul_rn(s, (float)((w >> 8) & 0xFFu)), z);
                    const float w2 = __fadd_rn(__fmul_rn(s, (float)((w >> 16) & 0xFFu)), z);
                    const float w3 = __fadd_rn(__fmul_rn(s, (float)(w >> 24)), z);
                    o[2 * q] = pack2(w0, w1);
                    o[2 * q + 1] = pack2(w2, w3);
                }
                bd[2 * e] = (u32x4g){o[0], o[1], o[2], o[3]};
                bd[2 * e + 1] = (u32x4g){o[4], o[5], o[6], o[7]};
            }
        } else {
#pragma unroll
            for (int e = 0; e < PB; e++) bd[e] = rb[e];
        }
    };

    load(0);
    stage();
    __syncthreads();
    for (int k0 = 0; k0 < g.k; k0 += BKT) {
        const bool more = k0 + BKT < g.k;
        if (more) load(k0 + BKT);
#pragma unroll
        for (int st = 0; st < BKT / 16; st++) {
            half8_t af[MI], bf[NJ];
#pragma unroll
            for (int i = 0; i < MI; i++)
                af[i] = *(const half8_t *)(As + (wm + i * 32 + (lane & 31)) * LD + 16 * st + 8 * (lane >> 5));
#pragma unroll
            for (int j = 0; j < NJ; j++)
                bf[j] = *(const half8_t *)(Bs + (wn + j * 32 + (lane & 31)) * LD + 16 * st + 8 * (lane >> 5));
#pragma unroll
            for (int i = 0; i < MI; i++)
#pragma unroll
                for (int j = 0; j < NJ; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        if (more) {
            __syncthreads();
            stage();
            __syncthreads();
        }
    }
#define GEMM3_EPI(K) gemm2_epilogue<K, MI, NJ>(g, acc, m0, n0, wm, wn, lane)
    switch (g.epi) {
        case GE_BIAS: GEMM3_EPI(GE_BIAS); break;
        case GE_ADD: GEMM3_EPI(GE_ADD); break;
        case GE_RELU2: GEMM3_EPI(GE_RELU2); break;
        case GE_TANH: GEMM3_EPI(GE_TANH); break;
        case GE_WDECAY: GEMM3_EPI(GE_WDECAY); break;
        case GE_SIGBIAS: GEMM3_EPI(GE_SIGBIAS); break;
        case GE_VLERP: GEMM3_EPI(GE_VLERP); break;
        case GE_SIGMOID: GEMM3_EPI(GE_SIGMOID); break;
        default: GEMM3_EPI(GE_STORE); break;
    }
#undef GEMM3_EPI
}

template <bool B_I8, int BKT, int BMR = 128>
__global__ __launch_bounds__(256, BKT == 64 && BMR == 128 ? 3 : 2) void k_gemm3(GemmArgs g) {
    __shared__ __attribute__((aligned(16))) _Float16 As[BMR * (BKT + 8)];
    __shared__ __attribute__((aligned(16))) _Float16 Bs[BN * (BKT + 8)];
    gemm3_body<B_I8, BKT, 2, BMR>(g, blockIdx.y * BMR, blockIdx.x * BN, As, Bs);
}

template <int BKT>
__global__ __launch_bounds__(256, BKT == 64 ? 3 : 2) void k_gemm3_multi(GemmJobs jobs) {
    __shared__ __attribute__((aligned(16))) _Float16 As[128 * (BKT + 8)];
    __shared__ __attribute__((aligned(16))) _Float16 Bs[BN * (BKT + 8)];
    const int bid = blockIdx.x;
    int ji = 0;
    while (ji + 1 < jobs.n && bid >= jobs.blk_start[ji + 1]) ji++;
    const GemmArgs &g = jobs.j[ji];
    const int local = bid - jobs.blk_start[ji], nt = (g.n + BN - 1) / BN;
    const int m0 = (local / nt) * 128, n0 = (local % nt) * BN;
    if (g.b_i8)
        gemm3_body<true, BKT, 2>(g, m0, n0, As, Bs);
    else
        gemm3_body<false, BKT, 2>(g, m0, n0, As, Bs);
}

// k per stage: 64 (k_gemm3) where every job's k is a multiple of 64, else 32
// (k_gemm2, double-buffered: the LoRA-up jobs, k = 96 etc.).
static int gemm_check(const GemmArgs &g) {
    if (g.m <= 0 || g.n <= 0 || g.k <= 0) return RSV_FAIL("gemm: bad shape m=%d n=%d k=%d", g.m, g.n, g.k);
    if (g.k % BK != 0) return RSV_FAIL("gemm: k=%d must be a multiple of %d", g.k, BK);
    if (g.b_i8 && (g.k % 128 != 0 || !g.sz)) return RSV_FAIL("gemm: int8 weights need k %% 128 == 0 and scales");
    if (g.lda < g.k || g.lda % 8 != 0) return RSV_FAIL("gemm: lda=%d must be >= k and a multiple of 8", g.lda);
    if (g.ldc < g.n) return RSV_FAIL("gemm: ldc=%d < n=%d", g.ldc, g.n);
    if ((g.epi == GE_ADD || g.epi == GE_VLERP) && !g.aux) return RSV_FAIL("gemm: epilogue needs aux");
    if ((g.epi == GE_BIAS || g.epi == GE_WDECAY || g.epi == GE_SIGBIAS || g.epi == GE_VLERP) && !g.bias)
        return RSV_FAIL("gemm: epilogue needs bias");
    if (g.epi == GE_WDECAY && !g.scale) return RSV_FAIL("gemm: decay epilogue needs scale");
    if (g.c_f16 && (g.epi == GE_ADD || g.epi == GE_VLERP)) return RSV_FAIL("gemm: in-place epilogues need fp32 C");
    return 0;
}

int launch_gemm_multi(rsv_ctx *ctx, GemmJobs &jobs) {
    if (jobs.n <= 0 || jobs.n > kMaxJobs) return RSV_FAIL("gemm_multi: 1..%d jobs", kMaxJobs);
    int total = 0;
    for (int i = 0; i < jobs.n; i++) {
        const GemmArgs &g = jobs.j[i];
        if (gemm_check(g)) return -1;
        jobs.blk_start[i] = total;
        total += ((g.n + BN - 1) / BN) * ((g.m + BM - 1) / BM);
    }
    jobs.blk_start[jobs.n] = total;
    bool k64 = true;
    for (int i = 0; i < jobs.n; i++) k64 &= jobs.j[i].k % 64 == 0;
    if (k64) hipLaunchKernelGGL((k_gemm3_multi<64>), dim3(total), dim3(256), 0, ctx->stream, jobs);
    else hipLaunchKernelGGL((k_gemm2_multi<128>), dim3(total), dim3(256), 0, ctx->stream, jobs);
    RSV_HIP(hipGetLastError());
    return 0;
}

int launch_gemm(rsv_ctx *ctx, const GemmArgs &g) {
    if (gemm_check(g)) return -1;
    const dim3 grid((g.n + BN - 1) / BN, (g.m + BM - 1) / BM);
    // 128-row tiles: 256-row tiles (one wave per SIMD at 275 registers)
    // measured 1.5x slower on the prefill GEMMs
    if (g.k % 64 == 0) {
        if (g.b_i8) hipLaunchKernelGGL((k_gemm3<true, 64>), grid, dim3(256), 0, ctx->stream, g);
        else hipLaunchKernelGGL((k_gemm3<false, 64>), grid, dim3(256), 0, ctx->stream, g);
    } else if (g.b_i8) hipLaunchKernelGGL((k_gemm2<true, 128>), grid, dim3(256), 0, ctx->stream, g);
    else hipLaunchKernelGGL((k_gemm2<false, 128>), grid, dim3(256), 0, ctx->stream, g);
    RSV_HIP(hipGetLastError());
    return 0;
}

}  // namespace rsv
