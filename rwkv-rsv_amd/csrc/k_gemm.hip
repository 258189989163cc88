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
#include <cstdlib>

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
                // non-temporal stores: acknowledged sooner, so the next
                // tile's reuse of their data registers waits less
                if (g.c_f16)
                    __builtin_nontemporal_store((_Float16)v, (_Float16 *)g.c + o);
                else
                    __builtin_nontemporal_store(v, (float *)g.c + o);
            }
        }
    }
}

// Epilogue of a wave's (32 MI) x (32 NJ) tile (MFMA 32x32 tiles at (r0, c0)) through
// the wave's own 32x36-float LDS tile: each 32x32 tile is written in the
// MFMA layout and read back as rows, so lane l handles row l/8 (+8, +16,
// +24) and columns 4*(l%8) .. +3: one 16-byte access per lane, eight whole
// 128-byte lines per instruction, for the outputs and for the operands an
// epilogue reads (y in place, aux).  Same per-element values as
// gemm2_epilogue.  Needs n % 4 == 0 and ldc % 4 == 0.
template <int EPI, int MI, int NJ>
__device__ __forceinline__ void tile_epilogue(const GemmArgs &g, const float16_t (&acc)[MI][NJ], int r0, int c0,
                                              int lane, float *tl) {
    constexpr bool need_b = EPI == GE_BIAS || EPI == GE_WDECAY || EPI == GE_SIGBIAS || EPI == GE_VLERP;
    constexpr bool need_aux = EPI == GE_ADD || EPI == GE_VLERP;
    constexpr bool need_cur = EPI == GE_VLERP;
    const float scale = EPI == GE_WDECAY ? g.scale[0] : 0.0f;
    const int lr = lane >> 3, lc = 4 * (lane & 7);
    // the read operands of 32x32 tile t = MI*j + i (rows r0 + 32i ..,
    // columns c0 + 32j ..): issued one tile ahead of its use
    constexpr int NT = MI * NJ;
    float4 aux[2][4], cur[2][4];
    auto fetch = [&](int t, int b) {
        const int i = t % MI, j = t / MI;
        const int col = c0 + j * 32 + lc;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int row = r0 + i * 32 + lr + 8 * q;
            const size_t o = (size_t)row * g.ldc + col;
            const bool ok = col < g.n && row < g.m;
            aux[b][q] = (need_aux && ok) ? *(const float4 *)(g.aux + o) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            cur[b][q] = (need_cur && ok) ? *(const float4 *)((const float *)g.c + o) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
    };
    fetch(0, 0);
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const int i = t % MI, j = t / MI, b = t & 1;
        if (t + 1 < NT) fetch(t + 1, b ^ 1);
        const int col = c0 + j * 32 + lc;
        const bool cok = col < g.n;
        float4 bias = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (need_b && cok) bias = *(const float4 *)(g.bias + col);
        // MFMA layout -> LDS rows: element e of lane l is row
        // 8*(e/4) + 4*(l/32) + e%4, column l%32
#pragma unroll
        for (int e = 0; e < 16; e++) tl[(8 * (e >> 2) + 4 * (lane >> 5) + (e & 3)) * 36 + (lane & 31)] = acc[i][j][e];
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int row = r0 + i * 32 + lr + 8 * q;
            const float4 v = *(const float4 *)(tl + (lr + 8 * q) * 36 + lc);
            float4 y;
            y.x = gemm_epi_val<EPI>(v.x, bias.x, aux[b][q].x, cur[b][q].x, scale);
            y.y = gemm_epi_val<EPI>(v.y, bias.y, aux[b][q].y, cur[b][q].y, scale);
            y.z = gemm_epi_val<EPI>(v.z, bias.z, aux[b][q].z, cur[b][q].z, scale);
            y.w = gemm_epi_val<EPI>(v.w, bias.w, aux[b][q].w, cur[b][q].w, scale);
            if (!cok || row >= g.m) continue;
            const size_t o = (size_t)row * g.ldc + col;
            if (g.c_f16) {
                typedef _Float16 h4 __attribute__((ext_vector_type(4)));
                const h4 hv = {(_Float16)y.x, (_Float16)y.y, (_Float16)y.z, (_Float16)y.w};
                __builtin_nontemporal_store(hv, (h4 *)((_Float16 *)g.c + o));
            } else {
                typedef float f4 __attribute__((ext_vector_type(4)));
                const f4 fv = {y.x, y.y, y.z, y.w};
                __builtin_nontemporal_store(fv, (f4 *)((float *)g.c + o));
            }
        }
        __builtin_amdgcn_wave_barrier();  // the LDS tile is rewritten next
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

// Fourth form, for fp16 weights with k a multiple of 64 (the prefill GEMMs
// on the fp16 weight copies): a large tile per block of 4 waves, one wave
// per SIMD, and the operand tiles copied global -> LDS by
// global_load_lds_dwordx4 (no VGPR staging, no LDS stores by the waves).
//   - A stage is 64 k of the block's BMR activation rows and BNC weight
//     rows, 128 bytes per row; NS = 3 stages rotate, the copy of stage s+2
//     in flight while stage s is multiplied out, one barrier per stage.
//   - Copy instruction i of wave w fills 1 KiB: rows 8g .. 8g+7 of the
//     stage (g = w*NI + i; A rows first, then B rows), lane l taking row
//     8g + l/8 and 16-byte piece (l%8) ^ gd_swz(row).  The XOR spreads the
//     operand reads of 8 (or 16) consecutive rows over all the banks.
//   - Each wave owns a (MI*32) x (NJ*32) tile of C as MI x NJ 32x32 MFMA
//     blocks; per 16 k it reads MI + NJ operand pieces (ds_read_b128, in asm:
//     the compiler cannot see which LDS copy a read waits for and would drain
//     every copy in flight before it) and issues MI*NJ MFMAs, the reads of
//     the next 16 k in flight during them.
//   - The MFMA is the one of k_gemm2/3 (v_mfma_f32_32x32x16_f16, lane l
//     holding k 8*(l/32) .. +7 of each 16 k, ascending k): every element's
//     accumulation chain is the same, so the results equal the other forms'
//     bit for bit (the int8 loader's fp16 rounding included).
//   - Blocks are spread XCD-aware: the hardware deals consecutive block ids
//     to the 8 XCDs in turn; block b takes tile (b%8)*(T/8) + b/8 of a
//     grouped order (4 row tiles x all column tiles per group), so the
//     blocks that share an XCD's L2 share operand tiles.
template <int WM, int WN, int MI, int NJ>
struct GdCfg {
    static constexpr int BMR = WM * MI * 32, BNC = WN * NJ * 32;
    static constexpr int ROWS = BMR + BNC;
    static constexpr int SB = ROWS * 128;     // bytes of one stage
    static constexpr int NI = ROWS / 8 / 4;   // copy instructions per wave per stage
    static constexpr int NS = 3;
    static constexpr int LDS = NS * SB;
    static_assert(ROWS % 32 == 0, "stage rows must split evenly over 4 waves");
    static_assert(LDS <= 160 * 1024, "LDS");
};

// block id -> tile order position: XCD-major when the block count allows
__device__ __forceinline__ int gd_xcd_order(int bid, int T) {
    return (T & 7) == 0 ? (bid & 7) * (T >> 3) + (bid >> 3) : bid;
}

// position t of the grouped order over tm x tn tiles -> (row tile, column tile)
__device__ __forceinline__ void gd_tile(int t, int tm, int tn, int &mt, int &nt) {
    constexpr int GM = 4;
    const int gsz = GM * tn, grp = t / gsz, f = grp * GM, gm = min(GM, tm - f), r = t - grp * gsz;
    mt = f + r % gm;
    nt = r / gm;
}

// Stage row r keeps its logical 16-byte piece p in physical piece
// p ^ gd_swz(r): any 8 consecutive rows from a multiple of 8 use 8 distinct
// pieces (8 lanes x 16 bytes meet 32 banks once), and so do the 8 even and
// the 8 odd rows of 16 consecutive rows (16 lanes over 64 banks: rows r and
// r+1 sit 128 bytes apart, in the other half of the banks).
__device__ __forceinline__ int gd_swz(int r) { return (r & 7) ^ ((r >> 3) & 1); }

// One operand piece of a 16-k step: row (l%32) of strip piece p (32 rows
// further per piece), in asm for the reason given at the reads below.
typedef unsigned int gd_u4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void gd_read_piece(gd_u4 &dst, uint32_t va, int p) {
    switch (p) {
        case 0: asm volatile("ds_read_b128 %0, %1 offset:0" : "=v"(dst) : "v"(va)); break;
        case 1: asm volatile("ds_read_b128 %0, %1 offset:4096" : "=v"(dst) : "v"(va)); break;
        case 2: asm volatile("ds_read_b128 %0, %1 offset:8192" : "=v"(dst) : "v"(va)); break;
        case 3: asm volatile("ds_read_b128 %0, %1 offset:12288" : "=v"(dst) : "v"(va)); break;
        case 4: asm volatile("ds_read_b128 %0, %1 offset:16384" : "=v"(dst) : "v"(va)); break;
        case 5: asm volatile("ds_read_b128 %0, %1 offset:20480" : "=v"(dst) : "v"(va)); break;
        case 6: asm volatile("ds_read_b128 %0, %1 offset:24576" : "=v"(dst) : "v"(va)); break;
        default: asm volatile("ds_read_b128 %0, %1 offset:28672" : "=v"(dst) : "v"(va)); break;
    }
}

// MULTI only separates the instantiations of the two kernels: the host
// compilation pass cannot check the VGPR asm constraints, and a body it
// instantiated once (with those errors deferred) is refused to a second
// caller.
template <int WM, int WN, int MI, int NJ, bool MULTI>
__device__ __forceinline__ void gemmd_body(const GemmArgs &g, int m0, int n0, unsigned char *lds) {
    using C = GdCfg<WM, WN, MI, NJ>;
    constexpr int NI = C::NI;
    // the wave index in a scalar register: what derives from it stays scalar
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int wm = (wave / WN) * MI * 32, wn = (wave % WN) * NJ * 32;
    // Copies go through buffer resources over A ([m, lda]) and B ([n, k]):
    // a row past the end reads as zeros (its offset is beyond the resource's
    // size), so partial tiles need no clamping.  Instruction i of this wave
    // copies row group gi = wave*NI + i: A rows 8*gi .. if gi < BMR/8, else
    // B rows 8*gi - BMR ..; lane l takes row 8*gi + l/8 and logical piece
    // (l%8) ^ gd_swz(row).
    const __amdgpu_buffer_rsrc_t rsA = __builtin_amdgcn_make_buffer_rsrc((void *)g.a, (short)0, g.m * g.lda * 2, 0x00020000);
    const __amdgpu_buffer_rsrc_t rsB = __builtin_amdgcn_make_buffer_rsrc((void *)g.b, (short)0, g.n * g.k * 2, 0x00020000);
    const int lr = lane >> 3;
    uint32_t voff[NI];
#pragma unroll
    for (int i = 0; i < NI; i++) {
        const int gi = wave * NI + i, r = 8 * gi;
        const int lp = (lane & 7) ^ gd_swz(r + lr);
        voff[i] = r < C::BMR ? ((uint32_t)(m0 + r + lr) * (uint32_t)g.lda + lp * 8) * 2u
                             : ((uint32_t)(n0 + r - C::BMR + lr) * (uint32_t)g.k + lp * 8) * 2u;
    }
    const int nA = min(max(C::BMR / 8 - wave * NI, 0), NI);  // this wave's A instructions
    auto issue = [&](int s, int buf) {
        unsigned char *dst = lds + buf * C::SB + wave * NI * 1024;
#pragma unroll
        for (int i = 0; i < NI; i++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(i < nA ? rsA : rsB, (__attribute__((address_space(3))) void *)(dst + i * 1024),
                                                     16, voff[i], s * 128, 0, 0);
    };
    float16_t acc[MI][NJ];
#pragma unroll
    for (int i = 0; i < MI; i++)
#pragma unroll
        for (int j = 0; j < NJ; j++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[i][j][e] = 0.0f;
    // operand read addresses: row (l%32) of the wave's A / B strip, piece
    // (2*st + l/32) ^ (l%8) of the 64-k stage for the 16-k step st
    const uint32_t lds0 = (uint32_t)(uintptr_t)lds;
    const uint32_t rowA = lds0 + (wm + (lane & 31)) * 128, rowB = lds0 + (C::BMR + wn + (lane & 31)) * 128;
    uint32_t xo[4];
#pragma unroll
    for (int st = 0; st < 4; st++) xo[st] = ((2 * st + (lane >> 5)) ^ gd_swz(lane & 31)) * 16;
    typedef unsigned int u4 __attribute__((ext_vector_type(4)));
    auto read = [&](u4 (&fa)[MI], u4 (&fb)[NJ], uint32_t boff, int st) {
        const uint32_t va = rowA + boff + xo[st], vb = rowB + boff + xo[st];
#pragma unroll
        for (int i = 0; i < MI; i++) asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(fa[i]) : "v"(va), "i"(i * 4096));
#pragma unroll
        for (int j = 0; j < NJ; j++) asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(fb[j]) : "v"(vb), "i"(j * 4096));
    };
    auto ready = [&](u4 (&fa)[MI], u4 (&fb)[NJ]) {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int i = 0; i < MI; i++) asm volatile("" : "+v"(fa[i]));
#pragma unroll
        for (int j = 0; j < NJ; j++) asm volatile("" : "+v"(fb[j]));
    };
    // Three stage buffers, four operand register sets (one per 16-k step of
    // a stage).  Step st of stage s: wait for its operands (read during step
    // st-1), then its MFMAs with step st+1's reads (into the set step st-3
    // used) issued one after each MFMA.  At the last step every wave has its
    // operands of the stage in registers: after one barrier (which also
    // publishes the next stage's copies, waited for before it) the stage's
    // buffer takes the copy of stage s+3, whose copy instructions go out one
    // after each MFMA too, with the next stage's first reads.  Issued as a
    // burst before the MFMAs, the reads and copies left the matrix pipe idle
    // for their issue time every step: interleaved, att.output at 4096 rows
    // 70 -> 63 us, ffn.value 247 -> 232 us.
    // step(): the MFMAs of operand set (ca, cb), with the LDS reads of set
    // (na, nb) from stage offset boff (when rd) and the copies of stage ds
    // into buffer db (when dm).
    auto step = [&](const u4 (&ca)[MI], const u4 (&cb)[NJ], u4 (&na)[MI], u4 (&nb)[NJ], bool rd, uint32_t boff,
                    int sn, bool dm, int ds, int db) {
        const uint32_t va = rowA + boff + xo[sn], vb = rowB + boff + xo[sn];
        unsigned char *dst = lds + db * C::SB + wave * NI * 1024;
        int r = 0, d = 0;
#pragma unroll
        for (int i = 0; i < MI; i++)
#pragma unroll
            for (int j = 0; j < NJ; j++) {
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8_t, ca[i]),
                                                                 __builtin_bit_cast(half8_t, cb[j]), acc[i][j], 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
                if (rd && r < MI + NJ) {
                    if (r < MI) gd_read_piece(na[r], va, r);
                    else gd_read_piece(nb[r - MI], vb, r - MI);
                }
                r++;
                __builtin_amdgcn_sched_barrier(0);
                if (dm && d < NI)
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(d < nA ? rsA : rsB,
                                                             (__attribute__((address_space(3))) void *)(dst + d * 1024), 16,
                                                             voff[d], ds * 128, 0, 0);
                d++;
                __builtin_amdgcn_sched_barrier(0);
            }
        // whatever did not fit between the MFMAs
#pragma unroll
        for (; r < MI + NJ; r++) {
            if (!rd) break;
            if (r < MI) gd_read_piece(na[r], va, r);
            else gd_read_piece(nb[r - MI], vb, r - MI);
        }
#pragma unroll
        for (; d < NI; d++) {
            if (!dm) break;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(d < nA ? rsA : rsB, (__attribute__((address_space(3))) void *)(dst + d * 1024),
                                                     16, voff[d], ds * 128, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    const int nst = g.k / 64;
    issue(0, 0);
    if (nst > 1) issue(1, 1);
    if (nst > 2) issue(2, 2);
    if (nst > 2) sk_wait_vm(2 * NI);
    else if (nst > 1) sk_wait_vm(NI);
    else sk_wait_vm(0);
    __builtin_amdgcn_s_barrier();
    u4 fa[4][MI], fb[4][NJ];
    read(fa[0], fb[0], 0, 0);
    int buf = 0;
    for (int s = 0; s < nst; s++) {
        const int nbuf = buf == 2 ? 0 : buf + 1;
#pragma unroll
        for (int st = 0; st < 4; st++) {
            __builtin_amdgcn_sched_barrier(0);
            ready(fa[st], fb[st]);
            if (st < 3) {
                step(fa[st], fb[st], fa[st + 1], fb[st + 1], true, buf * C::SB, st + 1, false, 0, 0);
            } else {
                if (s + 2 < nst) sk_wait_vm(NI);
                else sk_wait_vm(0);
                __builtin_amdgcn_s_barrier();
                step(fa[3], fb[3], fa[0], fb[0], s + 1 < nst, nbuf * C::SB, 0, s + 3 < nst, s + 3, buf);
            }
        }
        buf = nbuf;
    }
    // 16-byte epilogue through LDS (the stage buffers are free once every
    // wave is past its last operand reads): each wave takes 32x36 floats
    const bool vec = g.n % 4 == 0 && g.ldc % 4 == 0;
    __syncthreads();
    float *tl = reinterpret_cast<float *>(lds) + wave * (32 * 36);
#define GEMMD_EPI(K) do { if (vec) tile_epilogue<K, MI, NJ>(g, acc, m0 + wm, n0 + wn, lane, tl); \
                          else gemm2_epilogue<K, MI, NJ>(g, acc, m0, n0, wm, wn, lane); } while (0)
    switch (g.epi) {
        case GE_BIAS: GEMMD_EPI(GE_BIAS); break;
        case GE_ADD: GEMMD_EPI(GE_ADD); break;
        case GE_RELU2: GEMMD_EPI(GE_RELU2); break;
        case GE_TANH: GEMMD_EPI(GE_TANH); break;
        case GE_WDECAY: GEMMD_EPI(GE_WDECAY); break;
        case GE_SIGBIAS: GEMMD_EPI(GE_SIGBIAS); break;
        case GE_VLERP: GEMMD_EPI(GE_VLERP); break;
        case GE_SIGMOID: GEMMD_EPI(GE_SIGMOID); break;
        default: GEMMD_EPI(GE_STORE); break;
    }
#undef GEMMD_EPI
}

template <int WM, int WN, int MI, int NJ>
__global__ __launch_bounds__(256, 1) void k_gemmd(GemmArgs g) {
    using C = GdCfg<WM, WN, MI, NJ>;
    __shared__ __attribute__((aligned(1024))) unsigned char lds[C::LDS];
    const int tm = (g.m + C::BMR - 1) / C::BMR, tn = (g.n + C::BNC - 1) / C::BNC;
    int mt, nt;
    gd_tile(gd_xcd_order(blockIdx.x, gridDim.x), tm, tn, mt, nt);
    gemmd_body<WM, WN, MI, NJ, false>(g, mt * C::BMR, nt * C::BNC, lds);
}

template <int WM, int WN, int MI, int NJ>
__global__ __launch_bounds__(256, 1) void k_gemmd_multi(GemmJobs jobs) {
    using C = GdCfg<WM, WN, MI, NJ>;
    __shared__ __attribute__((aligned(1024))) unsigned char lds[C::LDS];
    const int T = gridDim.x, bid = blockIdx.x;
    const int t = gd_xcd_order(bid, T);
    int ji = 0;
    while (ji + 1 < jobs.n && t >= jobs.blk_start[ji + 1]) ji++;
    const GemmArgs &g = jobs.j[ji];
    const int local = t - jobs.blk_start[ji];
    const int tm = (g.m + C::BMR - 1) / C::BMR, tn = (g.n + C::BNC - 1) / C::BNC;
    int mt, nt;
    gd_tile(local, tm, tn, mt, nt);
    gemmd_body<WM, WN, MI, NJ, true>(g, mt * C::BMR, nt * C::BNC, lds);
}

// Short-k job lists on fp16 weights (the prefill LoRA-up products, k = 64..256):
// the product is a few MFMA steps and the launch is bound by its epilogue's
// stores, so the operands skip LDS.  Block = 4 waves on a 128x128 tile as in
// k_gemm2 (waves 2x2, each 64x64 as 2x2 MFMA 32x32 tiles); every wave loads
// its own A and B fragments from global straight into registers in the MFMA
// layout (lane l: row l%32, k 16s + 8*(l/32) .. +7 of step s, one 16-byte
// load per fragment), KB steps in flight, so waves never wait on each other.
// The per-element MFMA chain equals k_gemm2's (same k order and lane
// layout), so the results are bit-identical to it.
template <int KB>
__global__ __launch_bounds__(256, 2) void k_gemm_shortk_multi(GemmJobs jobs) {
    const int bid = blockIdx.x;
    int ji = 0;
    while (ji + 1 < jobs.n && bid >= jobs.blk_start[ji + 1]) ji++;
    const GemmArgs &g = jobs.j[ji];
    const int local = bid - jobs.blk_start[ji], nt = (g.n + BN - 1) / BN;
    const int m0 = (local / nt) * BM, n0 = (local % nt) * BN;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
    const int kq = 8 * (lane >> 5);
    const _Float16 *A = g.a, *B = (const _Float16 *)g.b;
    int ar[2], br[2];
    bool aok[2], bok[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        ar[i] = m0 + wm + i * 32 + (lane & 31);
        aok[i] = ar[i] < g.m;
        br[i] = n0 + wn + i * 32 + (lane & 31);
        bok[i] = br[i] < g.n;
    }
    float16_t acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[i][j][e] = 0.0f;
    const int nsteps = g.k / 16;
    for (int s0 = 0; s0 < nsteps; s0 += KB) {
        u32x4g fa[KB][2], fb[KB][2];
#pragma unroll
        for (int s = 0; s < KB; s++) {
            const int k0 = 16 * (s0 + s) + kq;
            const bool kok = s0 + s < nsteps;
#pragma unroll
            for (int i = 0; i < 2; i++) {
                fa[s][i] = (kok && aok[i]) ? *(const u32x4g *)(A + (size_t)ar[i] * g.lda + k0) : (u32x4g){0u, 0u, 0u, 0u};
                fb[s][i] = (kok && bok[i]) ? *(const u32x4g *)(B + (size_t)br[i] * g.k + k0) : (u32x4g){0u, 0u, 0u, 0u};
            }
        }
#pragma unroll
        for (int s = 0; s < KB; s++) {
            if (s0 + s >= nsteps) break;
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < 2; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8_t, fa[s][i]),
                                                                     __builtin_bit_cast(half8_t, fb[s][j]), acc[i][j], 0, 0, 0);
        }
    }
#define SHORTK_EPI(K) tile_epilogue<K, 2, 2>(g, acc, m0 + wm, n0 + wn, lane, tl)
    __shared__ float tlds[4][32 * 36];
    float *tl = tlds[wave];
    switch (g.epi) {
        case GE_BIAS: SHORTK_EPI(GE_BIAS); break;
        case GE_ADD: SHORTK_EPI(GE_ADD); break;
        case GE_RELU2: SHORTK_EPI(GE_RELU2); break;
        case GE_TANH: SHORTK_EPI(GE_TANH); break;
        case GE_WDECAY: SHORTK_EPI(GE_WDECAY); break;
        case GE_SIGBIAS: SHORTK_EPI(GE_SIGBIAS); break;
        case GE_VLERP: SHORTK_EPI(GE_VLERP); break;
        case GE_SIGMOID: SHORTK_EPI(GE_SIGMOID); break;
        default: SHORTK_EPI(GE_STORE); break;
    }
#undef SHORTK_EPI
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

// The DMA-tile form (fp16 weights, k % 64 == 0, offsets within 31 bits):
// one of three tiles, whichever needs the fewest block rounds (one block per
// CU) times tile area, weighted by the measured per-element cost of each form
// (256x128 is the cheapest per element, 128x128 the dearest).
enum GdKind { GD_NONE = 0, GD_256x160, GD_256x128, GD_128x128 };

static bool gd_fits(const GemmArgs &g) {
    return !g.b_i8 && g.k % 64 == 0 && (uint64_t)(g.m + 256) * g.lda * 2 < (1ull << 31) &&
           (uint64_t)(g.n + 256) * g.k * 2 < (1ull << 31);
}

static int gd_tiles(const GemmArgs &g, int kind) {
    const int bm = kind == GD_128x128 ? 128 : 256, bn = kind == GD_256x160 ? 160 : 128;
    return ((g.m + bm - 1) / bm) * ((g.n + bn - 1) / bn);
}

static GdKind gd_pick(const GemmArgs *gs, int n, int cus) {
    for (int i = 0; i < n; i++)
        if (!gd_fits(gs[i])) return GD_NONE;
    static const double area[4] = {0, 256.0 * 160 * 1.0, 256.0 * 128 * 1.0, 128.0 * 128 * 1.2};
    GdKind best = GD_NONE;
    double best_cost = 0;
    for (int kind = GD_256x160; kind <= GD_128x128; kind++) {
        long tiles = 0;
        for (int i = 0; i < n; i++) tiles += gd_tiles(gs[i], kind);
        const double cost = (double)((tiles + cus - 1) / cus) * area[kind];
        if (best == GD_NONE || cost < best_cost) best = (GdKind)kind, best_cost = cost;
    }
    return best;
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
    const GdKind gk = gd_pick(jobs.j, jobs.n, ctx->sm_count > 0 ? ctx->sm_count : 256);
    if (gk != GD_NONE) {
        total = 0;
        for (int i = 0; i < jobs.n; i++) {
            jobs.blk_start[i] = total;
            total += gd_tiles(jobs.j[i], gk);
        }
        jobs.blk_start[jobs.n] = total;
        if (gk == GD_256x160) hipLaunchKernelGGL((k_gemmd_multi<4, 1, 2, 5>), dim3(total), dim3(256), 0, ctx->stream, jobs);
        else if (gk == GD_256x128) hipLaunchKernelGGL((k_gemmd_multi<2, 2, 4, 2>), dim3(total), dim3(256), 0, ctx->stream, jobs);
        else hipLaunchKernelGGL((k_gemmd_multi<2, 2, 2, 2>), dim3(total), dim3(256), 0, ctx->stream, jobs);
        RSV_HIP(hipGetLastError());
        return 0;
    }
    // RSV_NO_SHORTK=1 forces the LDS-staged form (the test comparing the two)
    bool k64 = true, shortk = !getenv("RSV_NO_SHORTK");
    for (int i = 0; i < jobs.n; i++) {
        const GemmArgs &g = jobs.j[i];
        k64 &= g.k % 64 == 0;
        shortk &= !g.b_i8 && g.k <= 256 && g.k % 16 == 0 && g.lda % 8 == 0 && g.n % 4 == 0 && g.ldc % 4 == 0;
    }
    if (shortk) hipLaunchKernelGGL((k_gemm_shortk_multi<4>), dim3(total), dim3(256), 0, ctx->stream, jobs);
    else if (k64) hipLaunchKernelGGL((k_gemm3_multi<64>), dim3(total), dim3(256), 0, ctx->stream, jobs);
    else hipLaunchKernelGGL((k_gemm2_multi<128>), dim3(total), dim3(256), 0, ctx->stream, jobs);
    RSV_HIP(hipGetLastError());
    return 0;
}

int launch_gemm(rsv_ctx *ctx, const GemmArgs &g) {
    if (gemm_check(g)) return -1;
    const GdKind gk = gd_pick(&g, 1, ctx->sm_count > 0 ? ctx->sm_count : 256);
    if (gk != GD_NONE) {
        const dim3 gd_grid(gd_tiles(g, gk));
        if (gk == GD_256x160) hipLaunchKernelGGL((k_gemmd<4, 1, 2, 5>), gd_grid, dim3(256), 0, ctx->stream, g);
        else if (gk == GD_256x128) hipLaunchKernelGGL((k_gemmd<2, 2, 4, 2>), gd_grid, dim3(256), 0, ctx->stream, g);
        else hipLaunchKernelGGL((k_gemmd<2, 2, 2, 2>), gd_grid, dim3(256), 0, ctx->stream, g);
        RSV_HIP(hipGetLastError());
        return 0;
    }
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
