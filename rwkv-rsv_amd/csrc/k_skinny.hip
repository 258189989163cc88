// Batched decode GEMM on matrix cores ("skinny" M = sessions <= 64):
//   y[b, n] (epilogue)= sum_k x[b, k] W[n, k]
// W is the reference int8 format (dequantised in registers, fp32 s*q+z
// rounded to fp16) or fp16; x is fp16 [batch, k].
//
// Block = 4 waves, tile = 32 weight rows x (32*MT) sessions.  The K
// dimension is split across the 4 waves (chunk c of 32 columns goes to wave
// c % 4) and the partial tiles are summed in LDS in a fixed order, so the
// result is deterministic.  Each wave keeps PF chunks of loads in flight.
//
// v_mfma_f32_32x32x8_f16 operand layout: lane l holds A[i = l%32][4g..4g+3]
// and B[4g..4g+3][j = l%32] with g = l/32.  A lane loads 16 consecutive
// k-values (k0 + 16g .. +15) of its weight row and of its session's x row;
// MFMA step s (0..3) consumes values 4s..4s+3 of both.  A and B use the same
// k permutation, so the products pair up exactly.
#include <algorithm>
#include <cstdlib>

#include "rsv_common.h"

namespace rsv {

typedef _Float16 sk_half4 __attribute__((ext_vector_type(4)));
typedef float sk_f16x __attribute__((ext_vector_type(16)));
typedef unsigned int sk_u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float sk_h2f(uint32_t b) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(b & 0xFFFFu));
}
__device__ __forceinline__ float sk_sig(float v) { return 1.0f / (1.0f + expf(-v)); }

__device__ __forceinline__ void sk_st(float *p, float v) { *p = v; }
__device__ __forceinline__ void sk_st(_Float16 *p, _Float16 v) { *p = v; }
__device__ __forceinline__ void sk_st4(float4 *p, float4 v) { *p = v; }


// fp16 pair (s*q0 + z, s*q1 + z): each an fp32 fma, the pair converted to
// fp16 (round to nearest even) by one v_cvt_pk_f16_f32.  Building the pair
// as a vector keeps the compiler from packing two halves with a shift and an
// or, which is what the scalar-half form lowers to.
typedef _Float16 sk_half2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t sk_deq2(float s, float q0, float q1, float z) {
    const sk_half2 h = {(_Float16)fmaf(s, q0, z), (_Float16)fmaf(s, q1, z)};
    return __builtin_bit_cast(uint32_t, h);
}

// One 32-column k-chunk of a wave's operands: two 32-row weight tiles and
// MT session tiles of x.
template <int MT>
struct SkChunk {
    sk_u32x4 w[2][2];  // [row tile]: int8 uses [rt][0] (16 bytes); fp16 uses both (16 halves)
    uint32_t sz[2];
    sk_u32x4 x[MT][2];  // [session tile][16 halves]
};

template <int MT>
__device__ __forceinline__ void sk_load(const SkinnyJob &J, int n0, int k0, int g, int lane, int MB, bool i8,
                                        SkChunk<MT> &ch) {
    const int kk = k0 + 16 * g;
#pragma unroll
    for (int rt = 0; rt < 2; rt++) {
        const int row = n0 + rt * 32 + (lane & 31);
        if (row < J.N) {
            if (i8) {
                ch.w[rt][0] = __builtin_nontemporal_load((const sk_u32x4 *)((const uint8_t *)J.w + (size_t)row * J.K + kk));
                ch.sz[rt] = J.sz[(size_t)row * (J.K / 128) + kk / 128];
            } else {
                const sk_u32x4 *p = (const sk_u32x4 *)((const _Float16 *)J.w + (size_t)row * J.K + kk);
                ch.w[rt][0] = __builtin_nontemporal_load(p);
                ch.w[rt][1] = __builtin_nontemporal_load(p + 1);
            }
        } else {
            ch.w[rt][0] = ch.w[rt][1] = (sk_u32x4){0u, 0u, 0u, 0u};
            ch.sz[rt] = 0u;
        }
    }
#pragma unroll
    for (int ct = 0; ct < MT; ct++) {
        const int b = ct * 32 + (lane & 31);
        if (b < MB) {
            const sk_u32x4 *p = (const sk_u32x4 *)(J.x + (size_t)b * J.ldx + kk);
            ch.x[ct][0] = p[0];
            ch.x[ct][1] = p[1];
        } else {
            ch.x[ct][0] = ch.x[ct][1] = (sk_u32x4){0u, 0u, 0u, 0u};
        }
    }
}

template <int MT>
__device__ __forceinline__ void sk_mma(const SkChunk<MT> &ch, bool i8, sk_f16x (&acc)[2][MT]) {
#pragma unroll
    for (int rt = 0; rt < 2; rt++) {
        uint32_t wh[8];  // 16 halves
        if (i8) {
            const float s = sk_h2f(ch.sz[rt]), z = sk_h2f(ch.sz[rt] >> 16);
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const uint32_t w = ch.w[rt][0][q];
                wh[2 * q] = sk_deq2(s, (float)(w & 0xFFu), (float)((w >> 8) & 0xFFu), z);
                wh[2 * q + 1] = sk_deq2(s, (float)((w >> 16) & 0xFFu), (float)(w >> 24), z);
            }
        } else {
#pragma unroll
            for (int q = 0; q < 4; q++) {
                wh[q] = ch.w[rt][0][q];
                wh[4 + q] = ch.w[rt][1][q];
            }
        }
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const sk_half4 a = __builtin_bit_cast(sk_half4, (unsigned long long)wh[2 * s] |
                                                                ((unsigned long long)wh[2 * s + 1] << 32));
#pragma unroll
            for (int ct = 0; ct < MT; ct++) {
                const uint32_t lo = ch.x[ct][s >> 1][(s & 1) * 2], hi = ch.x[ct][s >> 1][(s & 1) * 2 + 1];
                const sk_half4 bv =
                    __builtin_bit_cast(sk_half4, (unsigned long long)lo | ((unsigned long long)hi << 32));
                acc[rt][ct] = __builtin_amdgcn_mfma_f32_32x32x8f16(a, bv, acc[rt][ct], 0, 0, 0);
            }
        }
    }
}

__device__ __forceinline__ float sk_epilogue(const SkinnyJob &J, float v, int n, size_t yo) {
    const float bias = J.bias ? J.bias[n] : 0.0f;
    switch (J.epi) {
        case GE_BIAS: v += bias; break;
        case GE_ADD: v += ((const float *)J.y)[yo]; break;
        case GE_RELU2: v = v > 0.0f ? v * v : 0.0f; break;
        case GE_TANH: v = tanhf(v); break;
        case GE_WDECAY: v = expf(sk_sig(v + bias) * J.scale[0]); break;
        case GE_SIGBIAS: v = sk_sig(v + bias); break;
        case GE_VLERP: {
            const float cur = ((const float *)J.y)[yo];
            v = cur + sk_sig(v + bias) * (J.aux[yo] - cur);
        } break;
        case GE_SIGMOID: v = sk_sig(v); break;
        default: break;
    }
    return v;
}

// Epilogue operands of one job held in registers: the job struct lives in
// kernel-argument memory, and the compiler would re-read its fields after
// every store through a generic pointer if the loops used them directly.
struct SkEpi {
    void *y;
    float *y2;
    const float *bias, *aux;
    float scale;
    int ldy, y_f16, epi, N;
};
__device__ __forceinline__ SkEpi sk_epi_of(const SkinnyJob &J) {
    SkEpi e;
    e.y = J.y; e.y2 = J.y2; e.bias = J.bias; e.aux = J.aux;
    e.scale = J.epi == GE_WDECAY ? J.scale[0] : 0.0f;
    e.ldy = J.ldy; e.y_f16 = J.y_f16; e.epi = J.epi; e.N = J.N;
    return e;
}
// y[b, n] (epilogue)= v
__device__ __forceinline__ void sk_store(const SkEpi &E, float v, int n, int b) {
    const size_t yo = (size_t)b * E.ldy + n;
    const float bias = E.bias ? E.bias[n] : 0.0f;
    switch (E.epi) {
        case GE_BIAS: v += bias; break;
        case GE_ADD: v += ((const float *)E.y)[yo]; break;
        case GE_RELU2: v = v > 0.0f ? v * v : 0.0f; break;
        case GE_TANH: v = tanhf(v); break;
        case GE_WDECAY: v = expf(sk_sig(v + bias) * E.scale); break;
        case GE_SIGBIAS: v = sk_sig(v + bias); break;
        case GE_VLERP: {
            const float cur = ((const float *)E.y)[yo];
            v = cur + sk_sig(v + bias) * (E.aux[yo] - cur);
        } break;
        case GE_SIGMOID: v = sk_sig(v); break;
        default: break;
    }
    if (E.y_f16)
        sk_st((_Float16 *)E.y + yo, (_Float16)v);
    else
        sk_st((float *)E.y + yo, v);
    if (E.y2) sk_st(E.y2 + yo, v);
}

// y[b, n] (epilogue)= v with the read operands (y for add / v-lerp, aux,
// bias) already loaded by the caller.
__device__ __forceinline__ void sk_store_v(const SkEpi &E, float v, float yc, float ax, float bias, int n, int b) {
    const size_t yo = (size_t)b * E.ldy + n;
    switch (E.epi) {
        case GE_BIAS: v += bias; break;
        case GE_ADD: v += yc; break;
        case GE_RELU2: v = v > 0.0f ? v * v : 0.0f; break;
        case GE_TANH: v = tanhf(v); break;
        case GE_WDECAY: v = expf(sk_sig(v + bias) * E.scale); break;
        case GE_SIGBIAS: v = sk_sig(v + bias); break;
        case GE_VLERP: v = yc + sk_sig(v + bias) * (ax - yc); break;
        case GE_SIGMOID: v = sk_sig(v); break;
        default: break;
    }
    if (E.y_f16)
        sk_st((_Float16 *)E.y + yo, (_Float16)v);
    else
        sk_st((float *)E.y + yo, v);
    if (E.y2) sk_st(E.y2 + yo, v);
}

// Epilogue value for a compile-time epilogue kind.  The tile epilogues
// switch on the kind once and run a loop instantiated for it: a switch inside
// an unrolled per-element loop put ~10k instructions into one kernel, and
// its waves then spent most of the epilogue waiting on instruction fetch
// (7 us of a 12 us launch, measured with wall-clock marks per phase).
template <int EPI>
__device__ __forceinline__ float sk_epi_val(float v, float yc, float ax, float bias, float scale) {
    if constexpr (EPI == GE_BIAS) return v + bias;
    else if constexpr (EPI == GE_ADD) return v + yc;
    else if constexpr (EPI == GE_RELU2) return v > 0.0f ? v * v : 0.0f;
    else if constexpr (EPI == GE_TANH) return tanhf(v);
    else if constexpr (EPI == GE_WDECAY) return expf(sk_sig(v + bias) * scale);
    else if constexpr (EPI == GE_SIGBIAS) return sk_sig(v + bias);
    else if constexpr (EPI == GE_VLERP) return yc + sk_sig(v + bias) * (ax - yc);
    else if constexpr (EPI == GE_SIGMOID) return sk_sig(v);
    else return v;
}
__device__ __forceinline__ void sk_put(const SkEpi &E, size_t yo, float v) {
    if (E.y_f16)
        sk_st((_Float16 *)E.y + yo, (_Float16)v);
    else
        sk_st((float *)E.y + yo, v);
    if (E.y2) sk_st(E.y2 + yo, v);
}
// Runs f.template operator()<EPI>() for the epilogue kind of E.
#define SK_EPI_DISPATCH(E, CALL)                      \
    switch ((E).epi) {                                \
        case GE_BIAS: CALL(GE_BIAS); break;           \
        case GE_ADD: CALL(GE_ADD); break;             \
        case GE_RELU2: CALL(GE_RELU2); break;         \
        case GE_TANH: CALL(GE_TANH); break;           \
        case GE_WDECAY: CALL(GE_WDECAY); break;       \
        case GE_SIGBIAS: CALL(GE_SIGBIAS); break;     \
        case GE_VLERP: CALL(GE_VLERP); break;         \
        case GE_SIGMOID: CALL(GE_SIGMOID); break;     \
        default: CALL(GE_STORE); break;               \
    }

// Epilogue of a 128-row x TB-session tile held in LDS (tile[row][session]).
// Thread t always handles row t % 128 (coalesced stores along n), so the
// bias is read once; the read-modify-write operands of 8 sessions are
// loaded together before any of them is used.
template <int EPI, int TB>
__device__ __forceinline__ void sk_store_tile_t(const SkEpi &E, const float (*tile)[TB + 1], int n0, int MB) {
    const int r = threadIdx.x & 127, n = n0 + r;
    if (n >= E.N) return;
    constexpr bool need_y = EPI == GE_ADD || EPI == GE_VLERP;
    constexpr bool need_b = EPI == GE_BIAS || EPI == GE_WDECAY || EPI == GE_SIGBIAS || EPI == GE_VLERP;
    const float bias = need_b ? E.bias[n] : 0.0f;
    for (int b0 = threadIdx.x >> 7; b0 < MB; b0 += 16) {
        float yc[8], ax[8];
#pragma unroll
        for (int q = 0; q < 8; q++) {
            const int b = b0 + 2 * q;
            const size_t yo = (size_t)b * E.ldy + n;
            yc[q] = (need_y && b < MB) ? ((const float *)E.y)[yo] : 0.0f;
            ax[q] = (EPI == GE_VLERP && b < MB) ? E.aux[yo] : 0.0f;
        }
#pragma unroll
        for (int q = 0; q < 8; q++) {
            const int b = b0 + 2 * q;
            if (b >= MB) break;
            sk_put(E, (size_t)b * E.ldy + n, sk_epi_val<EPI>(tile[r][b], yc[q], ax[q], bias, E.scale));
        }
    }
}
template <int TB>
__device__ __forceinline__ void sk_store_tile(const SkEpi &E, const float (*tile)[TB + 1], int n0, int MB) {
#define SK_TILE_CALL(K) sk_store_tile_t<K, TB>(E, tile, n0, MB)
    SK_EPI_DISPATCH(E, SK_TILE_CALL)
#undef SK_TILE_CALL
}

// grid: for each job, (rows/64) row groups x J.split k-slices.  Block = 4
// waves on one row group; wave w takes k-chunks w, w+4, ... of the slice.
// The 4 wave tiles are summed in LDS in wave order.  With split == 1 the
// block applies the epilogue; otherwise it stores its tile to the workspace
// and k_skinny_reduce (the next launch) sums the slices in slice order, so
// no cross-block synchronisation is needed inside a launch.
template <int MT>
__global__ __launch_bounds__(256) void k_skinny(SkinnyJobs jobs, int MB, float *__restrict__ ws) {
    constexpr int PF = 4;  // chunks in flight per wave
    constexpr int TB = MT * 32;
    __shared__ float tile[64][TB + 1];
    const int bid = blockIdx.x;
    int ji = 0;
    while (ji + 1 < jobs.n && bid >= jobs.blk_start[ji + 1]) ji++;
    const SkinnyJob &J = jobs.j[ji];
    const int local = bid - jobs.blk_start[ji];
    const int rg = local / J.split, sl = local - (local / J.split) * J.split;
    const int n0 = rg * 64;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 5;
    const bool i8 = J.fmt == FMT_I8;
    const int nchunks = J.K / 32;
    const int per = (nchunks + J.split - 1) / J.split;
    const int c_lo = sl * per, c_hi = min(nchunks, c_lo + per);

    sk_f16x acc[2][MT];
#pragma unroll
    for (int rt = 0; rt < 2; rt++)
#pragma unroll
        for (int ct = 0; ct < MT; ct++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[rt][ct][e] = 0.0f;

    SkChunk<MT> ring[PF];
#pragma unroll
    for (int p = 0; p < PF; p++) {
        const int c = c_lo + wave + 4 * p;
        if (c < c_hi) sk_load<MT>(J, n0, c * 32, g, lane, MB, i8, ring[p]);
    }
    for (int it = 0; c_lo + wave + 4 * it < c_hi; it += PF) {
#pragma unroll
        for (int p = 0; p < PF; p++) {
            const int c = c_lo + wave + 4 * (it + p);
            if (c < c_hi) {
                sk_mma<MT>(ring[p], i8, acc);
                const int cn = c + 4 * PF;
                if (cn < c_hi) sk_load<MT>(J, n0, cn * 32, g, lane, MB, i8, ring[p]);
            }
        }
    }

    // wave tiles -> LDS in wave order; acc[rt][ct][e] is (row rt*32 + 8*(e/4) + 4g + e%4, col ct*32 + lane%32)
    for (int w = 0; w < 4; w++) {
        if (wave == w) {
#pragma unroll
            for (int rt = 0; rt < 2; rt++)
#pragma unroll
                for (int ct = 0; ct < MT; ct++)
#pragma unroll
                    for (int e = 0; e < 16; e++) {
                        float &d = tile[rt * 32 + 8 * (e >> 2) + 4 * g + (e & 3)][ct * 32 + (lane & 31)];
                        d = w == 0 ? acc[rt][ct][e] : d + acc[rt][ct][e];
                    }
        }
        __syncthreads();
    }
    if (J.split > 1) {
        // slice tile, row-group-major then slice: [rg][sl][64 rows][TB sessions]
        float *wsp = ws + ((size_t)J.ws_slot + (size_t)rg * J.split + sl) * 64 * TB;
        for (int o = tid; o < 64 * TB; o += 256) sk_st(wsp + o, tile[o & 63][o >> 6]);
        return;
    }
    for (int o = tid; o < 64 * TB; o += 256) {
        const int r = o & 63, b = o >> 6;  // consecutive threads: consecutive weight rows n
        const int n = n0 + r;
        if (n >= J.N || b >= MB) continue;
        const size_t yo = (size_t)b * J.ldy + n;
        const float v = sk_epilogue(J, tile[r][b], n, yo);
        if (J.y_f16)
            ((_Float16 *)J.y)[yo] = (_Float16)v;
        else
            ((float *)J.y)[yo] = v;
        if (J.y2) J.y2[yo] = v;
    }
}

// Sums the k-slices of every split job in slice order and applies the
// epilogue.  grid: one block per (job, row group); jobs with split == 1
// were finished by k_skinny and have no blocks here.
template <int MT>
__global__ __launch_bounds__(256) void k_skinny_reduce(SkinnyJobs jobs, int MB, const float *__restrict__ ws) {
    constexpr int TB = MT * 32;
    const int bid = blockIdx.x;
    int ji = 0;
    while (ji + 1 < jobs.n && bid >= jobs.red_start[ji + 1]) ji++;
    const SkinnyJob &J = jobs.j[ji];
    constexpr int PB = 64 * TB / 256;  // blocks per row group: one output per thread
    const int rg = (bid - jobs.red_start[ji]) / PB, part = (bid - jobs.red_start[ji]) % PB;
    const float *base = ws + ((size_t)J.ws_slot + (size_t)rg * J.split) * 64 * TB;
    {
        const int o = part * 256 + threadIdx.x;
        const int r = o & 63, b = o >> 6;
        const int n = rg * 64 + r;
        if (n >= J.N || b >= MB) return;
        float v = base[o];
        for (int q = 1; q < J.split; q++) v += base[(size_t)q * 64 * TB + o];
        const size_t yo = (size_t)b * J.ldy + n;
        v = sk_epilogue(J, v, n, yo);
        if (J.y_f16)
            ((_Float16 *)J.y)[yo] = (_Float16)v;
        else
            ((float *)J.y)[yo] = v;
        if (J.y2) J.y2[yo] = v;
    }
}

// ------------------------------------------------------------------ v5
// Batched decode GEMM, weights in the MFMA-tiled copy (see v4).  Block = 4
// waves = 4 row tiles (128 rows) on one k-slice of J.kslice chunks:
//   1. the block's whole x slab (batch x slice columns, fp16) is staged in
//      LDS once, with one barrier, so the weight stream never waits on x;
//   2. each wave streams its row tile's chunks through a PD-deep register
//      ring (no barriers; the prefetch past the slice end re-reads the last
//      chunk instead of branching, so no load waits on a join);
//   3. v_mfma_f32_32x32x16_f16: lane (i = l%32, g = l/32) supplies columns
//      16g + 8s .. +7 of step s for both operands, so A and B pair up;
//   4. split k-slices write partial tiles that k_skinny4_reduce (a second
//      launch over many blocks) adds in slice order, so the result does not
//      depend on timing.
typedef _Float16 sk_half8 __attribute__((ext_vector_type(8)));

template <int MT, bool I8>
__device__ __forceinline__ void skinny5_body(const SkinnyJob &J, int local, int MB, float *__restrict__ ws,
                                             unsigned char *smem5) {
    constexpr int TB = MT * 32;
    constexpr int PD = I8 ? 8 : 6;    // chunks in flight per wave
    constexpr int WV = I8 ? 1 : 2;    // 16-byte loads per lane per chunk
    const int rg = local / J.split, sl = local - (local / J.split) * J.split;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 5;
    const int nchunks = J.K / 32;
    const int c_lo = sl * J.kslice, c_hi = min(nchunks, c_lo + J.kslice);
    const int nloc = c_hi - c_lo;
    const int XS = J.kslice * 32 + 8;  // LDS row stride (halves) of the x slab
    _Float16 *xs = reinterpret_cast<_Float16 *>(smem5);
    float (*tile)[TB + 1] = reinterpret_cast<float (*)[TB + 1]>(smem5);
    const int rt_glob = rg * 4 + wave;
    const int row = rt_glob * 32 + (lane & 31);
    constexpr int tbytes = I8 ? 1024 : 2048;
    const uint8_t *wt = (const uint8_t *)J.w + ((size_t)rt_glob * nchunks) * tbytes + lane * (I8 ? 16 : 32);
    const bool row_ok = row < J.N;
    // tiled scale/zero: [row tile][group][32 rows], one 128-byte line per group
    const uint32_t *szrow = I8 ? J.sz + (size_t)min(rt_glob, (J.N - 1) / 32) * (J.K / 128) * 32 + (lane & 31) : nullptr;

    // 2a. weight chunk loads (the first PD go out right after the x slab's)
    sk_u32x4 wr[PD][WV];
    uint32_t sr[PD];
    // rows past N read row 0 of the tile and chunks past the slice re-read
    // its last chunk; both are masked to zero in compute(), so no load sits
    // behind a branch
    const uint8_t *wt_ok = row_ok ? wt : (const uint8_t *)J.w + (size_t)lane * (I8 ? 16 : 32);
    auto load_w = [&](int p, int c) {
        c = min(c, c_hi - 1);
        const sk_u32x4 *q = (const sk_u32x4 *)(wt_ok + (size_t)c * tbytes);
        // plain (not non-temporal) loads measured faster here
#pragma unroll
        for (int v = 0; v < WV; v++) wr[p][v] = q[v];
        if (I8) sr[p] = szrow[(size_t)(c >> 2) * 32];
    };
    // 1. x slab: TB rows x nloc*32 halves in 16-byte pieces.  Its loads go
    // out first (the main loop waits on the slab), then the first PD weight
    // chunks, then the slab is stored to LDS (kslice <= 16 chunks)
    constexpr int NP = TB * 16 * 4 / 256;  // pieces per thread at the largest slice
    const int pieces_row = nloc * 4;
    const int total = TB * pieces_row;
    // e / pieces_row as a multiply-high: exact for e * pieces_row < 2^32
    const uint32_t rmag = (uint32_t)((0x100000000ull + pieces_row - 1) / pieces_row);
    sk_u32x4 xv[NP];
#pragma unroll
    for (int i = 0; i < NP; i++) {
        const int e = tid + 256 * i;
        const int b = (int)__umulhi((uint32_t)e, rmag), pc = e - b * pieces_row;
        xv[i] = (e < total && b < MB) ? *(const sk_u32x4 *)(J.x + (size_t)b * J.ldx + c_lo * 32 + pc * 8)
                                      : (sk_u32x4){0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int p = 0; p < PD; p++) load_w(p, c_lo + p);
    {
#pragma unroll
        for (int i = 0; i < NP; i++) {
            const int e = tid + 256 * i;
            const int b = (int)__umulhi((uint32_t)e, rmag), pc = e - b * pieces_row;
            if (e < total) *(sk_u32x4 *)&xs[(size_t)b * XS + pc * 8] = xv[i];
        }
    }
    __syncthreads();

    sk_f16x acc[MT];
#pragma unroll
    for (int ct = 0; ct < MT; ct++)
#pragma unroll
        for (int e = 0; e < 16; e++) acc[ct][e] = 0.0f;

    auto compute = [&](int p, int cl) {  // cl: chunk index within the slice
        const bool live = row_ok && cl < nloc;
        cl = min(cl, nloc - 1);
        uint32_t wh[8];
        if (I8) {
            const float s = live ? sk_h2f(sr[p]) : 0.0f, z = live ? sk_h2f(sr[p] >> 16) : 0.0f;
#pragma unroll
            for (int h = 0; h < 4; h++) {
                const uint32_t u = wr[p][0][h];
                wh[2 * h] = sk_deq2(s, (float)(u & 0xFFu), (float)((u >> 8) & 0xFFu), z);
                wh[2 * h + 1] = sk_deq2(s, (float)((u >> 16) & 0xFFu), (float)(u >> 24), z);
            }
        } else {
#pragma unroll
            for (int h = 0; h < 4; h++) {
                wh[h] = live ? wr[p][0][h] : 0u;
                wh[4 + h] = live ? wr[p][WV - 1][h] : 0u;
            }
        }
#pragma unroll
        for (int st = 0; st < 2; st++) {
            const sk_half8 a = __builtin_bit_cast(sk_half8, (sk_u32x4){wh[4 * st], wh[4 * st + 1], wh[4 * st + 2], wh[4 * st + 3]});
#pragma unroll
            for (int ct = 0; ct < MT; ct++) {
                const sk_u32x4 xv = *(const sk_u32x4 *)&xs[(size_t)(ct * 32 + (lane & 31)) * XS + cl * 32 + 16 * g + 8 * st];
                acc[ct] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, __builtin_bit_cast(sk_half8, xv), acc[ct], 0, 0, 0);
            }
        }
    };

    // branch-free body: the trip count is rounded up to PD and the extra
    // chunks contribute zero
    for (int base = 0; base < nloc; base += PD) {
#pragma unroll
        for (int p = 0; p < PD; p++) {
            compute(p, base + p);
            load_w(p, c_lo + base + p + PD);
        }
    }
    __syncthreads();  // x slab dead: the LDS becomes the output tile

    // wave w owns tile rows 32w .. 32w+31: acc[ct][e] -> (row 32w + 8*(e/4) + 4g + e%4, col ct*32 + lane%32)
#pragma unroll
    for (int ct = 0; ct < MT; ct++)
#pragma unroll
        for (int e = 0; e < 16; e++) tile[wave * 32 + 8 * (e >> 2) + 4 * g + (e & 3)][ct * 32 + (lane & 31)] = acc[ct][e];
    __syncthreads();
    const int n0 = rg * 128;
    if (J.split > 1) {
        // slice tile, row-group-major then slice: [rg][sl][128 rows][TB sessions];
        // k_skinny4_reduce (the next launch) sums the slices in slice order
        float4 *wsp = (float4 *)(ws + ((size_t)J.ws_slot + (size_t)rg * J.split + sl) * 128 * TB);
        for (int o4 = tid; o4 < 32 * TB; o4 += 256) {
            const int r = (4 * o4) & 127, b = (4 * o4) >> 7;
            sk_st4(wsp + o4, make_float4(tile[r][b], tile[r + 1][b], tile[r + 2][b], tile[r + 3][b]));
        }
        return;
    }
    sk_store_tile<TB>(sk_epi_of(J), tile, n0, MB);
}

template <int MT, bool I8>
__global__ __launch_bounds__(256) void k_skinny5(SkinnyJobs jobs, int MB, float *__restrict__ ws) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem5[];
    const int bid = blockIdx.x;
    int ji = 0;
    while (ji + 1 < jobs.n && bid >= jobs.blk_start[ji + 1]) ji++;
    skinny5_body<MT, I8>(jobs.j[ji], bid - jobs.blk_start[ji], MB, ws, smem5);
}

// The same for a job list holding both weight formats (stage-1: int8 r/k/v
// next to the fp16 LoRA-down matrices): the block takes its job's body, so
// the two formats share one launch and one slice reduction.
template <int MT>
__global__ __launch_bounds__(256) void k_skinny5_mixed(SkinnyJobs jobs, int MB, float *__restrict__ ws) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem5[];
    const int bid = blockIdx.x;
    int ji = 0;
    while (ji + 1 < jobs.n && bid >= jobs.blk_start[ji + 1]) ji++;
    if (jobs.j[ji].fmt == FMT_I8)
        skinny5_body<MT, true>(jobs.j[ji], bid - jobs.blk_start[ji], MB, ws, smem5);
    else
        skinny5_body<MT, false>(jobs.j[ji], bid - jobs.blk_start[ji], MB, ws, smem5);
}

// One output of a split job: the slices in slice order, then the epilogue.
// The epilogue's read operands (y for add / v-lerp, aux, bias) are loaded
// together with the slices, so the thread waits on one round of loads.
template <int EPI, int TB>
__device__ __forceinline__ void sk_reduce_one(const SkinnyJob &J, const float *base, int o, int n, int b) {
    const SkEpi E = sk_epi_of(J);
    constexpr bool need_y = EPI == GE_ADD || EPI == GE_VLERP;
    constexpr bool need_b = EPI == GE_BIAS || EPI == GE_WDECAY || EPI == GE_SIGBIAS || EPI == GE_VLERP;
    const size_t yo = (size_t)b * E.ldy + n;
    const float yc = need_y ? ((const float *)E.y)[yo] : 0.0f;
    const float ax = EPI == GE_VLERP ? E.aux[yo] : 0.0f;
    const float bias = need_b ? E.bias[n] : 0.0f;
    float v = 0.0f;
    for (int q0 = 0; q0 < J.split; q0 += 8) {
        float part[8];
#pragma unroll
        for (int q = 0; q < 8; q++) part[q] = q0 + q < J.split ? base[(size_t)(q0 + q) * 128 * TB + o] : 0.0f;
#pragma unroll
        for (int q = 0; q < 8; q++)
            if (q0 + q < J.split) v = q0 + q == 0 ? part[q] : v + part[q];
    }
    sk_put(E, yo, sk_epi_val<EPI>(v, yc, ax, bias, E.scale));
}

template <int MT>
__global__ __launch_bounds__(256) void k_skinny4_reduce(SkinnyJobs jobs, int MB, const float *__restrict__ ws) {
    constexpr int TB = MT * 32;
    const int bid = blockIdx.x;
    int ji = 0;
    while (ji + 1 < jobs.n && bid >= jobs.red_start[ji + 1]) ji++;
    const SkinnyJob &J = jobs.j[ji];
    constexpr int PB = 128 * TB / 256;  // blocks per row group: one output per thread
    const int rg = (bid - jobs.red_start[ji]) / PB, part = (bid - jobs.red_start[ji]) % PB;
    const float *base = ws + ((size_t)J.ws_slot + (size_t)rg * J.split) * 128 * TB;
    const int o = part * 256 + threadIdx.x;
    const int r = o & 127, b = o >> 7;
    const int n = rg * 128 + r;
    if (n >= J.N || b >= MB) return;
#define SK_RED_CALL(K) sk_reduce_one<K, TB>(J, base, o, n, b)
    SK_EPI_DISPATCH(J, SK_RED_CALL)
#undef SK_RED_CALL
}


// Epilogue of one 32-row x TB-session tile: thread t owns row t % 32 and
// sessions t/32, t/32 + 8, ...; v[q] holds its TB/8 sums.  Every read
// operand goes out before the first store.
template <int EPI, int TB>
__device__ __forceinline__ void sk8_epilogue(const SkEpi &E, const float (&v)[TB / 8], int n, int b0, int MB) {
    constexpr int NQ = TB / 8;
    constexpr bool need_y = EPI == GE_ADD || EPI == GE_VLERP;
    constexpr bool need_b = EPI == GE_BIAS || EPI == GE_WDECAY || EPI == GE_SIGBIAS || EPI == GE_VLERP;
    float yc[NQ], ax[NQ];
#pragma unroll
    for (int q = 0; q < NQ; q++) {
        const int b = b0 + 8 * q;
        const size_t yo = (size_t)b * E.ldy + n;
        yc[q] = (need_y && b < MB) ? ((const float *)E.y)[yo] : 0.0f;
        ax[q] = (EPI == GE_VLERP && b < MB) ? E.aux[yo] : 0.0f;
    }
    const float bias = need_b ? E.bias[n] : 0.0f;
#pragma unroll
    for (int q = 0; q < NQ; q++) {
        const int b = b0 + 8 * q;
        if (b >= MB) break;
        sk_put(E, (size_t)b * E.ldy + n, sk_epi_val<EPI>(v[q], yc[q], ax[q], bias, E.scale));
    }
}

// Loads this wave issued after its copy of step s, up to the wait of step s,
// in k_skinny8's two-row-tile form: copies of steps 0..NSX-2 then the weights
// of steps 0..DW-1 at entry; in iteration t the copy of step t+NSX-1 and the
// weights of step t+DW.  nx / lw: loads per copy / per weight step.
template <int FIX, int NSX, int DW>
__device__ constexpr int sk8p_younger(int s, int nx, int lw) {
    // position of copy s: entry (s < NSX-1) or iteration s-NSX+1
    int n = 0;
    if (s < NSX - 1) {
        n += (NSX - 2 - s) * nx + DW * lw;  // later entry copies and the entry weights
        for (int t = 0; t < s; t++) n += (t + NSX - 1 < FIX ? nx : 0) + (t + DW < FIX ? lw : 0);
    } else {
        const int t0 = s - NSX + 1;  // iteration that issued copy s
        n += t0 + DW < FIX ? lw : 0;  // its weights
        for (int t = t0 + 1; t < s; t++) n += (t + NSX - 1 < FIX ? nx : 0) + (t + DW < FIX ? lw : 0);
    }
    return n;
}

// ------------------------------------------------------------------ v8
// Batched decode GEMM, one row tile (32 weight rows) per block over the
// whole k, the k range split over the block's 4 waves (each wave its own
// quarter; the four partial tiles are summed in LDS in wave order).  Per
// wave, two 32-column chunks per step:
//   - x of a step (TB sessions x 128 bytes, whole cache lines) is copied
//     global -> LDS by global_load_lds_dwordx4 (no VGPR staging):
//     instruction i fills 1 KiB, lane l taking session 8i + l/8 and 16-byte
//     piece (l%8) ^ (session & 7)
//     (the XOR spreads the MFMA operand reads of 32 sessions over the
//     banks); two wave-private buffers, the next step's copy in flight while
//     this step is multiplied out; the operand reads are one asm block per
//     chunk behind an explicit wait for the step's copy;
//   - the weights of a step (the row tile's next two 1 KiB / 2 KiB tiles, a
//     sequential stream per wave) go to registers DW steps ahead: HBM
//     latency needs many weight bytes in flight;
//   - v_mfma_f32_32x32x16_f16 with the lane mapping of k_skinny5.
// The common k (2560 columns: 10 steps per wave) runs fully unrolled with
// exact wait counts; other k (a multiple of 64) take a two-deep loop.
// With more row tiles than CUs (ffn.key: 320) a block of 8 waves takes two
// row tiles (RT = 2): the two waves of a k quarter each copy half of the
// step's x into shared buffers (four per quarter, three steps ahead), one
// barrier per step, so every x byte read from L2 feeds 64 weight rows.
// Blocks then number fewer than CUs and each CU reads 491 KiB instead of up
// to 2 x 409 KiB (ffn.key at B=64: 18.0 -> 15.8 us).
// x buffers per k quarter: copies NSX-1 steps ahead (one row tile: 3 buffers,
// B=8 4.21k -> 4.26k tok/s against 2; 4 buffers measured no better at B=64)
#ifndef SK8_NS1
#define SK8_NS1 3
#endif
__host__ __device__ constexpr int sk8_nsx(int rt) { return rt == 2 ? 4 : SK8_NS1; }

template <int MT, bool I8, int FIX, int RT, int XC>
__device__ __forceinline__ void skinny8_body(const SkinnyJob &J, int rt0, int MB, unsigned char *xb0) {
    constexpr int TB = MT * 32;
    constexpr int XB = TB * 128;     // bytes of one x buffer
    // 1 KiB copies per step: XC of the TB / 8 (a batch of at most 8 * XC
    // sessions copies only its own; the columns of the sessions not copied
    // hold stale LDS bytes, and an MFMA output column depends on its own
    // input column only, so those columns are computed and never stored)
    static_assert(XC >= 1 && XC <= TB / 8, "copies per step");
    constexpr int NX = XC;
    constexpr int WV = I8 ? 1 : 2;
    constexpr int tbytes = I8 ? 1024 : 2048;
    constexpr int DW = FIX > 0 ? 4 : 2;  // weight steps in flight
    constexpr int LW = 2 * WV + (I8 ? 1 : 0);  // weight loads per step
    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 5;
    // wave -> k quarter (wave % 4) and row tile (wave / 4) of the block
    const int wave = (tid >> 6) & 3, h = tid >> 8;
    const int rt = rt0 + h;
    const bool tile_ok = RT == 1 || rt * 32 < J.N;  // wave-uniform; a masked wave still copies its x share
    const int rt_ld = tile_ok ? rt : rt0;
    const int nchunks = J.K / 32;
    // chunk pairs per wave (k is a multiple of 64)
    const int q4 = ((nchunks + 3) / 4 + 1) & ~1;
    const int cw0 = min(nchunks, wave * q4), cw1 = min(nchunks, cw0 + q4);
    const int nw = (cw1 - cw0) / 2;  // steps of this wave
    // NSX x buffers per k quarter (wave-private with one row tile, shared by
    // the quarter's two waves with two), copies NSX-1 steps ahead
    constexpr int NSX = sk8_nsx(RT);
    unsigned char *xbw[NSX];
#pragma unroll
    for (int i = 0; i < NSX; i++) xbw[i] = xb0 + (i * 4 + wave) * XB;
    // a k-slice job points into a row tile of a wider tiled matrix
    const int tch = J.wtile_ch ? J.wtile_ch : nchunks;
    const uint8_t *wt = (const uint8_t *)J.w + (size_t)rt_ld * tch * tbytes + lane * (I8 ? 16 : 32);
    const uint32_t *szrow = I8 ? J.sz + (size_t)rt_ld * (tch / 4) * 32 + (lane & 31) : nullptr;
    // copy source of lane l in instruction i, relative to the step's column
    // (with two row tiles, this wave's share: instructions h*NX/2 ..)
    // (one copy per step and two row tiles: both halves issue it, the same
    // bytes to the same LDS place)
    constexpr int NXW = NX >= RT ? NX / RT : 1;
    const _Float16 *xsrc[NXW];
#pragma unroll
    for (int j = 0; j < NXW; j++) {
        const int i = NX >= RT ? h * NXW + j : j;
        const int b = 8 * i + (lane >> 3);
        const int piece = (lane & 7) ^ (b & 7);
        xsrc[j] = J.x + (size_t)min(b, MB - 1) * J.ldx + piece * 8;
    }
    sk_u32x4 wr[DW][2][WV];
    uint32_t sr[DW];
    auto issue_x = [&](int slot, int s) {
        const int c = cw0 + 2 * min(s, nw - 1);  // clamped: steps past the end re-read (masked)
        unsigned char *dst = xbw[slot];
        // with two row tiles the quarter's two waves copy half the sessions each
#pragma unroll
        for (int j = 0; j < NXW; j++)
            __builtin_amdgcn_global_load_lds(xsrc[j] + c * 32, (__attribute__((address_space(3))) void *)(dst + (NX >= RT ? h * NXW + j : j) * 1024),
                                             16, 0, 0);
    };
    auto issue_w = [&](int wslot, int s) {
        const int c = cw0 + 2 * min(s, nw - 1);
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const sk_u32x4 *q = (const sk_u32x4 *)(wt + (size_t)(c + h) * tbytes);
#pragma unroll
            for (int v = 0; v < WV; v++) wr[wslot][h][v] = q[v];
        }
        if (I8) sr[wslot] = szrow[(size_t)(c >> 2) * 32];  // c even: both chunks in one 128-group
    };
    sk_f16x acc[MT];
#pragma unroll
    for (int ct = 0; ct < MT; ct++)
#pragma unroll
        for (int e = 0; e < 16; e++) acc[ct][e] = 0.0f;
    // mask = false where every step is a real one: the tiled copy's padding
    // rows are zero (scale and zero too), so only the loop's clamped steps
    // past the end need masking
    auto compute = [&](int slot, int wslot, int s, bool mask) {
        const unsigned char *xb = xbw[slot];
        const bool live = !mask || s < nw;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            uint32_t wh[8];
            if (I8) {
                const float sc = live ? sk_h2f(sr[wslot]) : 0.0f, z = live ? sk_h2f(sr[wslot] >> 16) : 0.0f;
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const uint32_t u = wr[wslot][h][0][q];
                    wh[2 * q] = sk_deq2(sc, (float)(u & 0xFFu), (float)((u >> 8) & 0xFFu), z);
                    wh[2 * q + 1] = sk_deq2(sc, (float)((u >> 16) & 0xFFu), (float)(u >> 24), z);
                }
            } else {
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    wh[q] = live ? wr[wslot][h][0][q] : 0u;
                    wh[4 + q] = live ? wr[wslot][h][WV - 1][q] : 0u;
                }
            }
            // the chunk's x operands: read in one asm block, so that the
            // compiler, which cannot see which LDS copy a read depends on,
            // adds no drain of every copy in flight before them (the explicit
            // wait before the step covers this step's copy)
            sk_u32x4 xv[2][MT];
            const int b_lo = lane & 31;
            const uint32_t a00 = (uint32_t)(uintptr_t)(xb + b_lo * 128 + (((4 * h + 2 * g) ^ (b_lo & 7)) * 16));
            const uint32_t a01 = (uint32_t)(uintptr_t)(xb + b_lo * 128 + (((4 * h + 2 * g + 1) ^ (b_lo & 7)) * 16));
            if constexpr (MT == 1) {
                asm volatile("ds_read_b128 %0, %2\n\tds_read_b128 %1, %3\n\ts_waitcnt lgkmcnt(0)"
                             : "=v"(xv[0][0]), "=v"(xv[1][0])
                             : "v"(a00), "v"(a01)
                             : "memory");
            } else {
                // session tile 1 sits 32 sessions (4096 bytes) further, with
                // the same XOR pattern (b & 7 unchanged)
                asm volatile("ds_read_b128 %0, %4\n\tds_read_b128 %1, %5\n\t"
                             "ds_read_b128 %2, %4 offset:4096\n\tds_read_b128 %3, %5 offset:4096\n\t"
                             "s_waitcnt lgkmcnt(0)"
                             : "=v"(xv[0][0]), "=v"(xv[1][0]), "=v"(xv[0][MT - 1]), "=v"(xv[1][MT - 1])
                             : "v"(a00), "v"(a01)
                             : "memory");
            }
#pragma unroll
            for (int st = 0; st < 2; st++) {
                const sk_half8 a = __builtin_bit_cast(sk_half8, (sk_u32x4){wh[4 * st], wh[4 * st + 1], wh[4 * st + 2], wh[4 * st + 3]});
#pragma unroll
                for (int ct = 0; ct < MT; ct++)
                    acc[ct] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, __builtin_bit_cast(sk_half8, xv[st][ct]), acc[ct], 0, 0, 0);
            }
        }
    };
    if constexpr (RT == 2) {
        // the launcher runs this form with FIX steps only.  x copies go NSX-1
        // steps ahead through NSX buffers per quarter.  Per step: wait for
        // this wave's share of the step's copy, a barrier (every share landed
        // and every wave done with the buffer the next copy refills), the
        // copy NSX-1 steps ahead, the products, the weights DW steps ahead
        // (scheduling barriers keep the issue order the wait counts assume)
#pragma unroll
        for (int d = 0; d < NSX - 1; d++) {
            issue_x(d, d);
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int d = 0; d < DW; d++) issue_w(d, d);
#pragma unroll
        for (int s = 0; s < FIX; s++) {
            __builtin_amdgcn_sched_barrier(0);
            sk_wait_vm(sk8p_younger<FIX, NSX, DW>(s, NXW, LW));
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_sched_barrier(0);
            if (s + NSX - 1 < FIX) issue_x((s + NSX - 1) % NSX, s + NSX - 1);
            compute(s % NSX, s % DW, s, false);  // a masked wave multiplies its stand-in tile, unstored
            __builtin_amdgcn_sched_barrier(0);
            if (s + DW < FIX) issue_w(s % DW, s + DW);
        }
    } else if (FIX > 0 && nw == FIX) {
        // one row tile: the same issue order as above without the barrier
        // (the buffers are the wave's own; the slot a copy refills was last
        // read by the previous step, whose reads completed before its MFMAs)
#pragma unroll
        for (int d = 0; d < NSX - 1; d++) {
            issue_x(d, d);
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int d = 0; d < DW; d++) issue_w(d, d);
#pragma unroll
        for (int s = 0; s < FIX; s++) {
            __builtin_amdgcn_sched_barrier(0);
            sk_wait_vm(sk8p_younger<FIX, NSX, DW>(s, NX, LW));
            __builtin_amdgcn_sched_barrier(0);
            if (s + NSX - 1 < FIX) issue_x((s + NSX - 1) % NSX, s + NSX - 1);
            compute(s % NSX, s % DW, s, false);
            __builtin_amdgcn_sched_barrier(0);
            if (s + DW < FIX) issue_w(s % DW, s + DW);
        }
    } else if (nw > 0) {
        // the x copies are not register results, so the wait before a step
        // is explicit: only the next step's loads may still be outstanding
        constexpr int VM = NX + LW;
        constexpr int WAIT = (VM & 0xF) | ((VM >> 4) << 14) | (0x7 << 4) | (0xF << 8);
        issue_x(0, 0);
        issue_w(0, 0);
        for (int s0 = 0; s0 < nw; s0 += 2) {
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const int s = s0 + u;
                issue_x(u ^ 1, s + 1);
                issue_w(u ^ 1, s + 1);
                __builtin_amdgcn_s_waitcnt(WAIT);
                compute(u, u, s, true);
            }
        }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();  // x buffers dead: the LDS holds the wave tiles now
    float (*part)[32][TB + 1] = reinterpret_cast<float (*)[32][TB + 1]>(xb0) + 4 * h;
#pragma unroll
    for (int ct = 0; ct < MT; ct++)
#pragma unroll
        for (int e = 0; e < 16; e++) part[wave][8 * (e >> 2) + 4 * g + (e & 3)][ct * 32 + (lane & 31)] = acc[ct][e];
    __syncthreads();
    const int r = tid & 31, b0 = (tid >> 5) & 7;
    float v[TB / 8];
#pragma unroll
    for (int q = 0; q < TB / 8; q++) {
        const int b = b0 + 8 * q;
        v[q] = ((part[0][r][b] + part[1][r][b]) + part[2][r][b]) + part[3][r][b];
    }
    if (!tile_ok) return;
    const int n = rt * 32 + r;
    if (n >= J.N) return;
    const SkEpi E = sk_epi_of(J);
#define SK8_CALL(K) sk8_epilogue<K, TB>(E, v, n, b0, MB)
    SK_EPI_DISPATCH(E, SK8_CALL)
#undef SK8_CALL
}

// RT row tiles per block (4 waves each); with RT = 2 the two tiles share
// every x copy, halving the x bytes read from L2 per weight byte.
template <int MT, int RT, int XC>
__global__ __launch_bounds__(256 * RT) void k_skinny8(SkinnyJobs jobs, int MB) {
    // NSX buffers per k quarter of TB sessions x 128 bytes, then the wave
    // tiles of the partial sums in the same bytes
    constexpr int XBYTES = sk8_nsx(RT) * 4 * MT * 32 * 128;
    static_assert(RT * 4 * 32 * (MT * 32 + 1) * 4 <= XBYTES, "partial tiles fit the x buffers");
    __shared__ __attribute__((aligned(16))) unsigned char xb0[XBYTES];
    const int bid = blockIdx.x;
    int ji = 0;
    while (ji + 1 < jobs.n && bid >= jobs.blk_start[ji + 1]) ji++;
    const int rt0 = (bid - jobs.blk_start[ji]) * RT;
    // k = 1280 (a half-k slice) runs its 5 steps per wave unrolled too
    const bool k1280 = RT == 1 && jobs.j[ji].K == 32 * 40;
    if (jobs.j[ji].fmt == FMT_I8) {
        if (k1280) skinny8_body<MT, true, 5, RT, XC>(jobs.j[ji], rt0, MB, xb0);
        else skinny8_body<MT, true, 10, RT, XC>(jobs.j[ji], rt0, MB, xb0);
    } else {
        if (k1280) skinny8_body<MT, false, 5, RT, XC>(jobs.j[ji], rt0, MB, xb0);
        else skinny8_body<MT, false, 10, RT, XC>(jobs.j[ji], rt0, MB, xb0);
    }
}

// Tiled copy of a weight matrix [n, k] (int8 bytes or fp16) for the tiled kernels;
// rows beyond n (up to the next multiple of 32) are zero.  One thread per
// 16-byte lane slice.
__global__ void k_tile_weights(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst, int n, int k, int esz) {
    const int nchunks = k / 32;
    const int lane_bytes = 16 * esz;
    const size_t total = (size_t)((n + 31) / 32) * nchunks * 64;
    for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (size_t)gridDim.x * blockDim.x) {
        const int lane = (int)(e % 64);
        const size_t t = e / 64;
        const int c = (int)(t % nchunks), rt = (int)(t / nchunks);
        const int row = rt * 32 + (lane & 31);
        const int col = c * 32 + 16 * (lane >> 5);
        uint8_t *d = dst + e * lane_bytes;
        if (row < n) {
            const uint8_t *s = src + ((size_t)row * k + col) * esz;
            for (int i = 0; i < lane_bytes; i++) d[i] = s[i];
        } else {
            for (int i = 0; i < lane_bytes; i++) d[i] = 0;
        }
    }
}

// Tiled copy of an int8 scale/zero array [n, k/128] for the tiled kernels:
// [row tile][group][32 rows], so the 32 rows of a tile read one 128-byte
// line per group.  Rows beyond n are zero.
__global__ void k_tile_sz(const uint32_t *__restrict__ src, uint32_t *__restrict__ dst, int n, int groups) {
    const size_t total = (size_t)((n + 31) / 32) * groups * 32;
    for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (size_t)gridDim.x * blockDim.x) {
        const int r = (int)(e % 32);
        const size_t t = e / 32;
        const int gq = (int)(t % groups), rt = (int)(t / groups);
        const int row = rt * 32 + r;
        dst[e] = row < n ? src[(size_t)row * groups + gq] : 0u;
    }
}

int launch_tile_weights(rsv_ctx *ctx, const void *src, void *dst, int n, int k, int esz) {
    if (esz == 4) {
        if (k % 128 != 0) return RSV_FAIL("tile_weights: k=%d must be a multiple of 128 for scale/zero", k);
        const size_t total = (size_t)((n + 31) / 32) * (k / 128) * 32;
        size_t blocks = (total + 255) / 256;
        if (blocks > 65536) blocks = 65536;
        hipLaunchKernelGGL(k_tile_sz, dim3((unsigned)blocks), dim3(256), 0, ctx->stream, (const uint32_t *)src,
                           (uint32_t *)dst, n, k / 128);
        RSV_HIP(hipGetLastError());
        return 0;
    }
    if (k % 32 != 0) return RSV_FAIL("tile_weights: k=%d must be a multiple of 32", k);
    const size_t total = (size_t)((n + 31) / 32) * (k / 32) * 64;
    size_t blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(k_tile_weights, dim3((unsigned)blocks), dim3(256), 0, ctx->stream, (const uint8_t *)src,
                       (uint8_t *)dst, n, k, esz);
    RSV_HIP(hipGetLastError());
    return 0;
}

static int launch_slab(rsv_ctx *ctx, SkinnyJobs &jobs, int MB);

// Batches above 64 run as consecutive 64-row slabs.
constexpr int SK_SMALL_NCH = 8;  // chunks (of 32) of the small-K kernel: K <= 256

int launch_skinny(rsv_ctx *ctx, SkinnyJobs &jobs, int MB) {
    if (MB <= 0) return RSV_FAIL("skinny gemm: batch %d", MB);
    for (int s0 = 0; s0 < MB; s0 += 64) {
        SkinnyJobs sl = jobs;
        for (int i = 0; i < sl.n; i++) {
            SkinnyJob &J = sl.j[i];
            J.x += (size_t)s0 * J.ldx;
            J.y = J.y_f16 ? (void *)((_Float16 *)J.y + (size_t)s0 * J.ldy) : (void *)((float *)J.y + (size_t)s0 * J.ldy);
            if (J.y2) J.y2 += (size_t)s0 * J.ldy;
            if (J.aux) J.aux += (size_t)s0 * J.ldy;
        }
        if (launch_slab(ctx, sl, MB - s0 < 64 ? MB - s0 : 64)) return -1;
    }
    return 0;
}

// k_skinny8: one block per 32-row tile over the whole k (both weight
// formats in one launch).
static int launch_v8(rsv_ctx *ctx, SkinnyJobs &jobs, int MB) {
    int total = 0;
    for (int i = 0; i < jobs.n; i++) {
        SkinnyJob &J = jobs.j[i];
        J.split = 1;
        J.nblk = (J.N + 31) / 32;
        jobs.blk_start[i] = total;
        total += J.nblk;
    }
    jobs.blk_start[jobs.n] = total;
    // more row tiles than CUs and every k = 2560: two tiles per block (every
    // CU one block, each x copy serving 64 rows)
    const int cus = ctx->sm_count > 0 ? ctx->sm_count : 256;
    bool pair = total > cus;
    for (int i = 0; i < jobs.n; i++) pair &= jobs.j[i].K == 32 * 80;
    if (pair) {
        total = 0;
        for (int i = 0; i < jobs.n; i++) {
            SkinnyJob &J = jobs.j[i];
            J.nblk = (J.N + 63) / 64;
            jobs.blk_start[i] = total;
            total += J.nblk;
        }
        jobs.blk_start[jobs.n] = total;
    }
    // the 64-session forms come first in this function so that they lead the
    // code object's kernels: with the narrow forms placed first the B=64
    // decode step measured 0.8% slower with identical machine code
    if (MB > 32) {
        if (pair) hipLaunchKernelGGL((k_skinny8<2, 2, 8>), dim3(total), dim3(512), 0, ctx->stream, jobs, MB);
        else hipLaunchKernelGGL((k_skinny8<2, 1, 8>), dim3(total), dim3(256), 0, ctx->stream, jobs, MB);
    } else if (pair) {
        if (MB <= 8) hipLaunchKernelGGL((k_skinny8<1, 2, 1>), dim3(total), dim3(512), 0, ctx->stream, jobs, MB);
        else if (MB <= 16) hipLaunchKernelGGL((k_skinny8<1, 2, 2>), dim3(total), dim3(512), 0, ctx->stream, jobs, MB);
        else hipLaunchKernelGGL((k_skinny8<1, 2, 4>), dim3(total), dim3(512), 0, ctx->stream, jobs, MB);
    } else if (MB <= 8) {
        hipLaunchKernelGGL((k_skinny8<1, 1, 1>), dim3(total), dim3(256), 0, ctx->stream, jobs, MB);
    } else if (MB <= 16) {
        hipLaunchKernelGGL((k_skinny8<1, 1, 2>), dim3(total), dim3(256), 0, ctx->stream, jobs, MB);
    } else {
        hipLaunchKernelGGL((k_skinny8<1, 1, 4>), dim3(total), dim3(256), 0, ctx->stream, jobs, MB);
    }
    RSV_HIP(hipGetLastError());
    return 0;
}

// v5 launch of tiled jobs.  Each job's k-slice count is set so that the
// launch has about two blocks per CU, with slices of 8..16 chunks when the
// row count allows (16 chunks = the LDS x slab limit, 8 = enough chunks per
// wave to amortise the slab and the partial-tile traffic).
constexpr int SK_KMAX = 16;  // longest k-slice (chunks) of the LDS x slab
static int launch_v5(rsv_ctx *ctx, SkinnyJobs &jobs, int MB) {
    const int TB = MB <= 32 ? 32 : 64;
    const int cus = ctx->sm_count > 0 ? ctx->sm_count : 256;
    const int target = 2 * cus;
    int64_t W = 0;
    for (int i = 0; i < jobs.n; i++) {
        const SkinnyJob &J = jobs.j[i];
        W += (int64_t)((J.N + 127) / 128) * (J.K / 32);
    }
    int total = 0, red_total = 0;
    size_t ws_need = 0, lds = 0;
    for (int i = 0; i < jobs.n; i++) {
        SkinnyJob &J = jobs.j[i];
        const int rgs = (J.N + 127) / 128;
        const int nch = J.K / 32;
        int split = (int)(((int64_t)target * nch + W - 1) / W);
        split = std::min(split, std::max(1, nch / 8));
        split = std::max(split, (nch + SK_KMAX - 1) / SK_KMAX);
        int kslice = (nch + split - 1) / split;
        if (kslice > 8) kslice = std::min(SK_KMAX, (kslice + 7) / 8 * 8);  // whole prefetch rounds
        split = (nch + kslice - 1) / kslice;
        J.split = split;
        J.kslice = kslice;
        J.ws_slot = (int)(ws_need / (128 * (size_t)TB));
        J.nblk = rgs * split;
        jobs.blk_start[i] = total;
        total += J.nblk;
        jobs.red_start[i] = red_total;
        if (split > 1) {
            ws_need += (size_t)rgs * split * 128 * TB;
            red_total += rgs * (128 * TB / 256);
        }
        lds = std::max(lds, std::max((size_t)TB * (kslice * 32 + 8) * 2, (size_t)128 * (TB + 1) * 4));
    }
    jobs.blk_start[jobs.n] = total;
    jobs.red_start[jobs.n] = red_total;
    if (ws_need > ctx->skinny_ws_cap) return RSV_FAIL("skinny gemm: workspace too small (%zu floats)", ws_need);
    const bool i8 = jobs.j[0].fmt == FMT_I8;
    bool mixed = false;
    for (int i = 1; i < jobs.n; i++) mixed |= (jobs.j[i].fmt == FMT_I8) != i8;
    if (mixed) {
        if (MB <= 32) hipLaunchKernelGGL((k_skinny5_mixed<1>), dim3(total), dim3(256), lds, ctx->stream, jobs, MB, ctx->skinny_ws);
        else hipLaunchKernelGGL((k_skinny5_mixed<2>), dim3(total), dim3(256), lds, ctx->stream, jobs, MB, ctx->skinny_ws);
    } else if (MB <= 32) {
        if (i8) hipLaunchKernelGGL((k_skinny5<1, true>), dim3(total), dim3(256), lds, ctx->stream, jobs, MB, ctx->skinny_ws);
        else hipLaunchKernelGGL((k_skinny5<1, false>), dim3(total), dim3(256), lds, ctx->stream, jobs, MB, ctx->skinny_ws);
    } else {
        if (i8) hipLaunchKernelGGL((k_skinny5<2, true>), dim3(total), dim3(256), lds, ctx->stream, jobs, MB, ctx->skinny_ws);
        else hipLaunchKernelGGL((k_skinny5<2, false>), dim3(total), dim3(256), lds, ctx->stream, jobs, MB, ctx->skinny_ws);
    }
    RSV_HIP(hipGetLastError());
    if (red_total) {
        if (MB <= 32)
            hipLaunchKernelGGL(k_skinny4_reduce<1>, dim3(red_total), dim3(256), 0, ctx->stream, jobs, MB, ctx->skinny_ws);
        else
            hipLaunchKernelGGL(k_skinny4_reduce<2>, dim3(red_total), dim3(256), 0, ctx->stream, jobs, MB, ctx->skinny_ws);
        RSV_HIP(hipGetLastError());
    }
    return 0;
}

// Epilogue of k_skinny_sk1 for one epilogue kind: every read operand of the
// thread's sessions is loaded in one round, then the values are stored.
template <int EPI, int TB>
__device__ __forceinline__ void sk1_epilogue(const SkEpi &E, const float (*tile)[TB + 1], int n, int lane, int MB) {
    constexpr int NI = TB / 2;
    constexpr bool need_y = EPI == GE_ADD || EPI == GE_VLERP;
    constexpr bool need_b = EPI == GE_BIAS || EPI == GE_WDECAY || EPI == GE_SIGBIAS || EPI == GE_VLERP;
    const int r = lane & 31, g = lane >> 5;
    float yc[NI], ax[NI];
#pragma unroll
    for (int i = 0; i < NI; i++) {
        const int b = g + 2 * i;
        const size_t yo = (size_t)b * E.ldy + n;
        yc[i] = (need_y && b < MB) ? ((const float *)E.y)[yo] : 0.0f;
        ax[i] = (EPI == GE_VLERP && b < MB) ? E.aux[yo] : 0.0f;
    }
    const float bias = need_b ? E.bias[n] : 0.0f;
#pragma unroll
    for (int i = 0; i < NI; i++) {
        const int b = g + 2 * i;
        if (b >= MB) break;
        sk_put(E, (size_t)b * E.ldy + n, sk_epi_val<EPI>(tile[r][b], yc[i], ax[i], bias, E.scale));
    }
}

// Small-K batched GEMM, one wave per block on one 32-row tile of one job.
// A small-K job moves little data per row, so the launch is bound by what
// each CU can pull: one-wave blocks spread the row tiles of all jobs over
// up to N/32 CUs (four-wave blocks on 128 rows put four copies of x on one
// CU).  Only the job's own chunks are loaded (uniform branches), every load
// of the wave goes out at once, and the epilogue loads all of its
// read-modify-write operands in one round after the MFMAs.
template <int MT, bool I8, int NCH>
__global__ __launch_bounds__(64) void k_skinny_sk1(SkinnyJobs jobs, int MB) {
    constexpr int TB = MT * 32;
    constexpr int WV = I8 ? 1 : 2;
    __shared__ float tile[32][TB + 1];
    const int bid = blockIdx.x;
    int ji = 0;
    while (ji + 1 < jobs.n && bid >= jobs.blk_start[ji + 1]) ji++;
    const SkinnyJob &J = jobs.j[ji];
    const int rt = bid - jobs.blk_start[ji];
    const int lane = threadIdx.x, g = lane >> 5;
    const int nchunks = J.K / 32;
    const int row = rt * 32 + (lane & 31);
    const bool row_ok = row < J.N;
    constexpr int tbytes = I8 ? 1024 : 2048;
    const uint8_t *wt = (const uint8_t *)J.w + (row_ok ? (size_t)rt * nchunks * tbytes : 0) + lane * (I8 ? 16 : 32);
    const uint32_t *szrow = I8 ? J.sz + (size_t)min(rt, (J.N - 1) / 32) * (J.K / 128) * 32 + (lane & 31) : nullptr;
    sk_u32x4 wr[NCH][WV];
    uint32_t sr[NCH];
    sk_u32x4 xv[NCH][MT][2];
#pragma unroll
    for (int c = 0; c < NCH; c++) {
        if (c >= nchunks) break;  // uniform: one job per block
#pragma unroll
        for (int v = 0; v < WV; v++) wr[c][v] = ((const sk_u32x4 *)(wt + (size_t)c * tbytes))[v];
        if (I8) sr[c] = szrow[(size_t)(c >> 2) * 32];
#pragma unroll
        for (int ct = 0; ct < MT; ct++) {
            const int b = min(ct * 32 + (lane & 31), MB - 1);  // sessions past MB are computed, never stored
            const sk_u32x4 *xp = (const sk_u32x4 *)(J.x + (size_t)b * J.ldx + c * 32 + 16 * g);
            xv[c][ct][0] = xp[0];
            xv[c][ct][1] = xp[1];
        }
    }
    sk_f16x acc[MT];
#pragma unroll
    for (int ct = 0; ct < MT; ct++)
#pragma unroll
        for (int e = 0; e < 16; e++) acc[ct][e] = 0.0f;
#pragma unroll
    for (int c = 0; c < NCH; c++) {
        if (c >= nchunks) break;
        uint32_t wh[8];
        if (I8) {
            const float sc = row_ok ? sk_h2f(sr[c]) : 0.0f, z = row_ok ? sk_h2f(sr[c] >> 16) : 0.0f;
#pragma unroll
            for (int h = 0; h < 4; h++) {
                const uint32_t u = wr[c][0][h];
                wh[2 * h] = sk_deq2(sc, (float)(u & 0xFFu), (float)((u >> 8) & 0xFFu), z);
                wh[2 * h + 1] = sk_deq2(sc, (float)((u >> 16) & 0xFFu), (float)(u >> 24), z);
            }
        } else {
#pragma unroll
            for (int h = 0; h < 4; h++) {
                wh[h] = row_ok ? wr[c][0][h] : 0u;
                wh[4 + h] = row_ok ? wr[c][WV - 1][h] : 0u;
            }
        }
#pragma unroll
        for (int st = 0; st < 2; st++) {
            const sk_half8 a = __builtin_bit_cast(sk_half8, (sk_u32x4){wh[4 * st], wh[4 * st + 1], wh[4 * st + 2], wh[4 * st + 3]});
#pragma unroll
            for (int ct = 0; ct < MT; ct++)
                acc[ct] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, __builtin_bit_cast(sk_half8, xv[c][ct][st]), acc[ct], 0, 0, 0);
        }
    }
    // acc[ct][e] -> (row 8*(e/4) + 4g + e%4, session ct*32 + lane%32)
#pragma unroll
    for (int ct = 0; ct < MT; ct++)
#pragma unroll
        for (int e = 0; e < 16; e++) tile[8 * (e >> 2) + 4 * g + (e & 3)][ct * 32 + (lane & 31)] = acc[ct][e];
    __syncthreads();
    // thread: row r = lane % 32, sessions lane/32 + 2i (32 consecutive rows per store)
    const SkEpi E = sk_epi_of(J);
    const int n = rt * 32 + (lane & 31);
    if (n >= E.N) return;
#define SK1_CALL(K) sk1_epilogue<K, TB>(E, tile, n, lane, MB)
    SK_EPI_DISPATCH(E, SK1_CALL)
#undef SK1_CALL
}

// Jobs of K <= 32*SK_SMALL_NCH in one pass each, no k-split: k_skinny_sk1,
// one wave per 32 rows, one launch per weight format.
static int launch_small(rsv_ctx *ctx, SkinnyJobs &jobs, int MB) {
    const bool i8 = jobs.j[0].fmt == FMT_I8;
    bool mixed = false;
    for (int i = 1; i < jobs.n; i++) mixed |= (jobs.j[i].fmt == FMT_I8) != i8;
    if (mixed) {
        SkinnyJobs parts[2]{};
        for (int i = 0; i < jobs.n; i++) {
            SkinnyJobs &p = parts[jobs.j[i].fmt == FMT_I8 ? 0 : 1];
            p.j[p.n++] = jobs.j[i];
        }
        for (auto &p : parts)
            if (launch_small(ctx, p, MB)) return -1;
        return 0;
    }
    int total = 0;
    for (int i = 0; i < jobs.n; i++) {
        SkinnyJob &J = jobs.j[i];
        J.split = 1;
        J.nblk = (J.N + 31) / 32;
        jobs.blk_start[i] = total;
        total += J.nblk;
    }
    jobs.blk_start[jobs.n] = total;
    if (MB <= 32) {
        if (i8) hipLaunchKernelGGL((k_skinny_sk1<1, true, SK_SMALL_NCH>), dim3(total), dim3(64), 0, ctx->stream, jobs, MB);
        else hipLaunchKernelGGL((k_skinny_sk1<1, false, SK_SMALL_NCH>), dim3(total), dim3(64), 0, ctx->stream, jobs, MB);
    } else {
        if (i8) hipLaunchKernelGGL((k_skinny_sk1<2, true, SK_SMALL_NCH>), dim3(total), dim3(64), 0, ctx->stream, jobs, MB);
        else hipLaunchKernelGGL((k_skinny_sk1<2, false, SK_SMALL_NCH>), dim3(total), dim3(64), 0, ctx->stream, jobs, MB);
    }
    RSV_HIP(hipGetLastError());
    return 0;
}

// Tiled jobs: small k -> k_skinny_sk1; k of at most SK8_KMAX chunks, a multiple of 64
// -> k_skinny8 (one block per 32-row tile over the whole k: its x reads
// stay within 4x the weight bytes, and no k-slice partials are needed);
// longer k (ffn.value) -> k_skinny5 with k-slices and the slice reduction.
constexpr int SK8_KMAX = 80;  // chunks (2560 columns)
static int launch_slab(rsv_ctx *ctx, SkinnyJobs &jobs, int MB) {
    if (MB <= 0 || MB > 64) return RSV_FAIL("skinny gemm: batch %d outside 1..64", MB);
    if (jobs.n <= 0 || jobs.n > kMaxJobs) return RSV_FAIL("skinny gemm: bad job count %d", jobs.n);
    for (int i = 0; i < jobs.n; i++) {
        SkinnyJob &J = jobs.j[i];
        if (!J.w || !J.x || !J.y) return RSV_FAIL("skinny job %d: null operand", i);
        if (J.N <= 0 || J.K <= 0 || J.K % 32 != 0) return RSV_FAIL("skinny job %d: k=%d must be a multiple of 32", i, J.K);
        if (J.fmt == FMT_I8 && (J.K % 128 != 0 || !J.sz)) return RSV_FAIL("skinny job %d: int8 needs k %% 128 == 0", i);
        if (J.ldx % 8 != 0 || J.ldx < J.K) return RSV_FAIL("skinny job %d: bad ldx %d", i, J.ldx);
        if ((J.epi == GE_BIAS || J.epi == GE_WDECAY || J.epi == GE_SIGBIAS || J.epi == GE_VLERP) && !J.bias)
            return RSV_FAIL("skinny job %d: epilogue needs bias", i);
        if (J.epi == GE_VLERP && !J.aux) return RSV_FAIL("skinny job %d: v-lerp needs aux", i);
        if (J.epi == GE_WDECAY && !J.scale) return RSV_FAIL("skinny job %d: decay needs scale", i);
        if (J.y_f16 && (J.epi == GE_ADD || J.epi == GE_VLERP)) return RSV_FAIL("skinny job %d: in-place needs fp32 y", i);
        if (J.tiled != jobs.j[0].tiled) return RSV_FAIL("skinny gemm: jobs mix tiled and row-major weights");
    }
    if (jobs.j[0].tiled) {
        // (the head, 65,536 rows, also runs on k_skinny8: B=8 4.31k -> 4.35k
        // tok/s against the 128-row-group kernel it had before)
        bool small = true, v8 = true;
        for (int i = 0; i < jobs.n; i++) {
            const SkinnyJob &J = jobs.j[i];
            small &= J.K <= 32 * SK_SMALL_NCH;
            v8 &= J.K % 64 == 0 && J.K <= 32 * SK8_KMAX;
        }
        bool sliced = false;
        for (int i = 0; i < jobs.n; i++) sliced |= jobs.j[i].wtile_ch != 0;
        if (sliced && (small || !v8)) return RSV_FAIL("skinny gemm: k-slice jobs need 256 < k <= %d, k %% 64 == 0", 32 * SK8_KMAX);
        if (small) return launch_small(ctx, jobs, MB);
        return v8 ? launch_v8(ctx, jobs, MB) : launch_v5(ctx, jobs, MB);
    }
    // row-major weights (the C-ABI's untiled form): k_skinny + slice reduce
    const int TB = MB <= 32 ? 32 : 64;
    int total = 0, red_total = 0;
    size_t ws_need = 0;
    for (int i = 0; i < jobs.n; i++) {
        SkinnyJob &J = jobs.j[i];
        const int rgs = (J.N + 63) / 64;
        const int nchunks = J.K / 32;
        int split = 1;
        // each wave streams at most ~8 chunks (256 columns)
        while (split < 16 && nchunks > split * 4 * 8 && rgs * split * 2 <= 1024) split++;
        J.split = split;
        J.ws_slot = (int)(ws_need / (64 * TB));
        J.nblk = rgs * split;
        jobs.blk_start[i] = total;
        total += J.nblk;
        jobs.red_start[i] = red_total;
        if (split > 1) {
            ws_need += (size_t)rgs * split * 64 * TB;
            red_total += rgs * (64 * TB / 256);
        }
    }
    jobs.blk_start[jobs.n] = total;
    jobs.red_start[jobs.n] = red_total;
    if (ws_need > ctx->skinny_ws_cap) return RSV_FAIL("skinny gemm: workspace too small (%zu floats)", ws_need);
    if (MB <= 32)
        hipLaunchKernelGGL(k_skinny<1>, dim3(total), dim3(256), 0, ctx->stream, jobs, MB, ctx->skinny_ws);
    else
        hipLaunchKernelGGL(k_skinny<2>, dim3(total), dim3(256), 0, ctx->stream, jobs, MB, ctx->skinny_ws);
    RSV_HIP(hipGetLastError());
    if (red_total) {
        if (MB <= 32)
            hipLaunchKernelGGL(k_skinny_reduce<1>, dim3(red_total), dim3(256), 0, ctx->stream, jobs, MB, ctx->skinny_ws);
        else
            hipLaunchKernelGGL(k_skinny_reduce<2>, dim3(red_total), dim3(256), 0, ctx->stream, jobs, MB, ctx->skinny_ws);
        RSV_HIP(hipGetLastError());
    }
    return 0;
}

}  // namespace rsv

