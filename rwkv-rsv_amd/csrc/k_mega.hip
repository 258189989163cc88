// Persistent single-session decode step.  One launch runs a whole token:
// embedding row -> every layer -> ln_out -> head -> argmax, with one
// 256-thread workgroup per CU and grid-wide barriers between the phases of
// a layer.  It replaces the six launches per layer of the B=1 decode path
// (gpu_model.rs:2060-2392 for one session, head and argmax of
// gpu_model.rs:1879-1913 / backend_cuda.rs:3640-3680), whose launch ramps
// and tails cost more than the weight streams themselves at this size.
//
// Phases of layer i (G workgroups, H heads):
//   P1  LN1 + token-shift mixes, int8 r/k/v rows and fp16 LoRA-down rows
//       (w: tanh), split evenly over all workgroups            -> barrier
//   P3  workgroups h < H: LoRA-up (w decay, a gate, v-first lerp, g) for
//       head h, WKV7 state update, GroupNorm + bonus, y*g       -> barrier
//   P4  workgroups >= H: att.output rows, x += o                -> barrier
//   P5  LN2 + mix, ffn.key rows, relu^2                         -> barrier
//   P6  ffn.value rows, x += v                                  -> barrier
// then LN_out, head rows and a two-level argmax.
//
// Every workgroup's weight slice of the next phase is copied HBM -> LDS by
// waves 1-3 (buffer_load ... lds) while wave 0 waits at the grid barrier, so
// the weight stream overlaps the barrier.  Activations pass between
// workgroups through one small buffer that is only touched with sc1 buffer
// loads/stores (coherent across the XCDs' L2s); weights, norms and the
// session state use ordinary loads.  The barrier is a two-level counter
// tree; its spin is bounded and sets an abort flag that makes every
// workgroup leave, so a launch always drains.
#include "rsv_common.h"
#include <algorithm>
#include <cstdlib>

namespace rsv {

typedef unsigned int mu32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void *lds_vp;

namespace {

constexpr unsigned kBufFlags = 0x00020000u;
constexpr int kCoherent = 0x10;       // sc1
constexpr unsigned kSpinLimit = 1u << 22;
constexpr int kGroups = 16;           // barrier tree fan-in
constexpr int kBarStride = 32;        // uints between counters (128 B)
constexpr int kCQ = 16;               // C <= 256 * kCQ
constexpr int kCPL = 5;               // chunks per lane of a row group
constexpr int kPartMax = 512;         // partial-sum slots
constexpr int kOwnMax = 64;           // residual rows per workgroup

__host__ __device__ inline int part_lo(int m, int b, int g) { return (int)((long long)m * b / g); }
__host__ __device__ inline int pad1k(long long x) { return (int)((x + 1023) & ~1023LL); }
__host__ __device__ inline int imin(int a, int b) { return a < b ? a : b; }

// Lanes per row for a row of K elements (16-byte chunks of 16 int8 or 8
// fp16 weights), so that every lane holds at most kCPL chunks of x.
__host__ __device__ inline int lanes_for(int K, bool i8) {
    const int nc = K / (i8 ? 16 : 8);
    for (int lg = 32; lg <= 256; lg *= 2)
        if (nc <= lg * kCPL) return lg;
    return 0;
}

struct RowSeg {
    int mat, r0, n;
};
// P1 work of workgroup b: int8 rows [3C*b/G, 3C*(b+1)/G) of the stacked
// receptance/key/value matrices and the matching share of the stacked
// LoRA-down rows (w1, a1, v1, g1), each cut at matrix boundaries.
struct P1Plan {
    RowSeg s8[2], sl[2];
    int n8, nl;
    int o_idx[2], o_sz[2], o_l[2];
    int bytes;
    bool whole;  // every row landed in at most two segments
};
__host__ __device__ inline void p1_plan(int C, const int *mid, int b, int G, P1Plan &p) {
    // int8 rows: at most two segments when 3C/G <= C
    {
        const int s = part_lo(3 * C, b, G), e = part_lo(3 * C, b + 1, G);
        const int m0 = s / C, e0 = imin(e, (m0 + 1) * C);
        p.s8[0] = RowSeg{m0, s - m0 * C, e0 - s};
        p.s8[1] = RowSeg{m0 + 1, 0, imin(e - e0, C)};
        p.n8 = (e0 > s ? 1 : 0) + (e > e0 ? 1 : 0);
        if (e0 <= s) p.s8[0] = p.s8[1];
        p.whole = e - e0 <= C;
    }
    {
        const int c1 = mid[0], c2 = c1 + mid[1], c3 = c2 + mid[2], c4 = c3 + mid[3];
        const int s = part_lo(c4, b, G), e = part_lo(c4, b + 1, G);
        const int m0 = s < c1 ? 0 : s < c2 ? 1 : s < c3 ? 2 : 3;
        const int lo0 = m0 == 0 ? 0 : m0 == 1 ? c1 : m0 == 2 ? c2 : c3;
        const int hi0 = m0 == 0 ? c1 : m0 == 1 ? c2 : m0 == 2 ? c3 : c4;
        const int e0 = imin(e, hi0);
        const int hi1 = m0 == 0 ? c2 : m0 == 1 ? c3 : c4;
        p.sl[0] = RowSeg{m0, s - lo0, e0 - s};
        p.sl[1] = RowSeg{m0 + 1, 0, e - e0};
        p.nl = (e0 > s ? 1 : 0) + (e > e0 ? 1 : 0);
        if (e0 <= s) p.sl[0] = p.sl[1];
        p.whole = p.whole && e <= hi1;
    }
    int off = 0;
    p.o_idx[0] = off;
    off += p.n8 > 0 ? pad1k((long long)p.s8[0].n * C) : 0;
    p.o_sz[0] = off;
    off += p.n8 > 0 ? pad1k((long long)p.s8[0].n * (C / 32)) : 0;
    p.o_idx[1] = off;
    off += p.n8 > 1 ? pad1k((long long)p.s8[1].n * C) : 0;
    p.o_sz[1] = off;
    off += p.n8 > 1 ? pad1k((long long)p.s8[1].n * (C / 32)) : 0;
    p.o_l[0] = off;
    off += p.nl > 0 ? pad1k((long long)p.sl[0].n * C * 2) : 0;
    p.o_l[1] = off;
    off += p.nl > 1 ? pad1k((long long)p.sl[1].n * C * 2) : 0;
    p.bytes = off;
}
// P3 (workgroup h < H): 64 rows of each LoRA-up matrix and the head state.
struct P3Plan {
    int o_up[4], o_st, bytes;
};
__host__ __device__ inline void p3_plan(const int *mid, P3Plan &p) {
    int off = 0;
    for (int m = 0; m < 4; m++) {
        p.o_up[m] = off;
        off += pad1k(64LL * mid[m] * 2);
    }
    p.o_st = off;
    p.bytes = off + 64 * 64 * 4;
}
// One int8 row range [r0, r0+n) of an [M, K] matrix.
struct I8Plan {
    int r0, n, o_sz, bytes;
};
__host__ __device__ inline void i8_plan(int M, int K, int b, int G, I8Plan &p) {
    p.r0 = part_lo(M, b, G);
    p.n = part_lo(M, b + 1, G) - p.r0;
    p.o_sz = pad1k((long long)p.n * K);
    p.bytes = p.o_sz + pad1k((long long)p.n * (K / 32));
}
// Head rows of workgroup b, streamed in rounds of rr rows through two halves
// of the weight region.
struct HeadPlan {
    int r0, n, rr, o_sz, half;
};
__host__ __device__ inline void head_plan(int V, int C, bool i8, int w_bytes, int b, int G, HeadPlan &p) {
    p.r0 = part_lo(V, b, G);
    p.n = part_lo(V, b + 1, G) - p.r0;
    p.half = (w_bytes / 2) & ~1023;
    const long long rb = i8 ? C : 2LL * C, sb = i8 ? C / 32 : 0;
    int rr = 1;
    while (pad1k((rr + 1) * rb) + pad1k((rr + 1) * sb) <= p.half) rr++;
    p.rr = rr;
    p.o_sz = pad1k(rr * rb);
}

struct MegaArgs {
    MegaModelDev m;
    const MegaLayerDev *layers;
    const uint32_t *token_in;
    uint32_t *token_out;
    float *logits;
    float *act;
    unsigned act_bytes;
    unsigned *bar;  // root at 0, group g at (g+1)*kBarStride, abort flag at (kGroups+1)*kBarStride
    int o_w, o_xv, o_mids, o_part, o_hv, o_misc, w_bytes;
    int lg_c8, lg_f8, lg_c16, lg_head;
    unsigned long long *trace;  // optional phase timestamps (see kTraceLayers)
};
// Phase timestamps for profiling: for layers kTraceLayers[i], workgroup b
// writes wall_clock64() (100 MHz) at 12 points into trace[(i*G + b)*16 + k].
constexpr int kTraceN = 2;
__device__ __forceinline__ void tmark(const MegaArgs &A, int layer, int k) {
    if (!A.trace || threadIdx.x != 0) return;
    const int slot = layer == 1 ? 0 : layer == 17 ? 1 : -1;
    if (slot < 0) return;
    A.trace[((size_t)slot * gridDim.x + blockIdx.x) * 16 + k] = wall_clock64();
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void *p, unsigned bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes, (int)kBufFlags);
}
struct ActIO {
    __amdgpu_buffer_rsrc_t r;
    __device__ __forceinline__ float ld(int i) const {
        return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, i * 4, 0, kCoherent));
    }
    __device__ __forceinline__ void st(int i, float v) const {
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, i * 4, 0, kCoherent);
    }
    __device__ __forceinline__ float4 ld4(int i) const {
        const mu32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, i * 4, 0, kCoherent);
        return make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]), __uint_as_float(v[3]));
    }
    __device__ __forceinline__ void st4(int i, float4 v) const {
        mu32x4 u;
        u[0] = __float_as_uint(v.x); u[1] = __float_as_uint(v.y); u[2] = __float_as_uint(v.z); u[3] = __float_as_uint(v.w);
        __builtin_amdgcn_raw_buffer_store_b128(u, r, i * 4, 0, kCoherent);
    }
};

__device__ __forceinline__ float h2f(uint32_t b) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(b & 0xFFFFu)); }
__device__ __forceinline__ float sigm(float v) { return 1.0f / (1.0f + expf(-v)); }

// Cross-lane sums on the DPP network (no LDS round trips): after
// group_sum<RL> the sum over each aligned group of RL lanes (16, 32 or 64)
// sits in the group's last lane.
template <int CTRL, int RM = 0xF>
__device__ __forceinline__ float dppf(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, RM, 0xF, false));
}
__device__ __forceinline__ float group_sum(float v, int rl) {
    v += dppf<0xB1>(v);   // quad_perm 1,0,3,2
    v += dppf<0x4E>(v);   // quad_perm 2,3,0,1
    v += dppf<0x141>(v);  // row_half_mirror
    v += dppf<0x140>(v);  // row_mirror: every lane holds its 16-lane row sum
    if (rl >= 32) v += dppf<0x142, 0xA>(v);  // row_bcast:15 into rows 1, 3
    if (rl >= 64) v += dppf<0x143, 0xC>(v);  // row_bcast:31 into rows 2, 3
    return v;
}
__device__ __forceinline__ float bsum(float v, float *red) {
    v = group_sum(v, 64);
    __syncthreads();
    if ((threadIdx.x & 63) == 63) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

// Power-of-two factor that brings the workgroup-wide max |x| (mx per lane)
// to at most 2^14 (1 when it already is).
__device__ __forceinline__ float row_scale(float mx, float *red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    const float m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    if (!(m > 16384.0f)) return 1.0f;
    int e;
    frexpf(m, &e);  // m < 2^e
    return ldexpf(1.0f, 14 - e);
}

// ------------------------------------------------------------ LDS copies
struct Dma {
    const void *src;
    int bytes, dst;
};
struct DmaList {
    Dma d[6];  // unused slots have bytes == 0
};
__device__ __forceinline__ void dma_clear(DmaList &L) {
#pragma unroll
    for (int i = 0; i < 6; i++) L.d[i] = Dma{nullptr, 0, 0};
}
// Waves [w0, w0+nw) copy every entry 16 bytes per lane, 1 KiB per wave
// instruction; the destination regions are padded to 1 KiB and reads past
// an entry's end return zeros (buffer range check).
__device__ __forceinline__ void dma_issue(const DmaList &L, char *W, int wv, int nw) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < 6; i++) {
        const Dma d = L.d[i];
        if (d.bytes <= 0) continue;
        const __amdgpu_buffer_rsrc_t r = rsrc(d.src, (unsigned)d.bytes);
        const int units = (d.bytes + 15) >> 4;
        for (int u0 = wv * 64; u0 < units; u0 += nw * 64)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_vp)(W + d.dst + u0 * 16), 16, (u0 + lane) * 16, 0, 0, 0);
    }
}

enum { PH_P1 = 0, PH_P3 = 1, PH_P4 = 2, PH_P5 = 3, PH_P6 = 4, PH_HEAD = 5, PH_NONE = 6 };

__device__ __forceinline__ void build_dma(const MegaArgs &A, int layer, int ph, int b, DmaList &L) {
    const int G = gridDim.x, C = A.m.C, F = A.m.F, H = A.m.H;
    dma_clear(L);
    if (ph == PH_NONE) return;
    if (ph == PH_HEAD) {
        HeadPlan hp;
        head_plan(A.m.V, C, A.m.head_i8, A.w_bytes, b, G, hp);
        const int n = imin(hp.rr, hp.n);
        const long long rb = A.m.head_i8 ? C : 2LL * C;
        L.d[0] = Dma{(const char *)A.m.head + (size_t)hp.r0 * rb, (int)(n * rb), 0};
        if (A.m.head_i8) L.d[1] = Dma{A.m.head_sz + (size_t)hp.r0 * (C / 128), n * (C / 32), hp.o_sz};
        return;
    }
    const MegaLayerDev &Ly = A.layers[layer];
    if (ph == PH_P1) {
        P1Plan p;
        p1_plan(C, A.m.mid, b, G, p);
#pragma unroll
        for (int k = 0; k < 2; k++) {
            if (k < p.n8) {
                const RowSeg s = p.s8[k];
                const uint8_t *ix = s.mat == 0 ? Ly.idx[0] : s.mat == 1 ? Ly.idx[1] : Ly.idx[2];
                const uint32_t *sz = s.mat == 0 ? Ly.sz[0] : s.mat == 1 ? Ly.sz[1] : Ly.sz[2];
                L.d[2 * k] = Dma{ix + (size_t)s.r0 * C, s.n * C, p.o_idx[k]};
                L.d[2 * k + 1] = Dma{sz + (size_t)s.r0 * (C / 128), s.n * (C / 32), p.o_sz[k]};
            }
            if (k < p.nl) {
                const RowSeg s = p.sl[k];
                const _Float16 *dn = s.mat == 0 ? Ly.down[0] : s.mat == 1 ? Ly.down[1] : s.mat == 2 ? Ly.down[2] : Ly.down[3];
                L.d[4 + k] = Dma{dn + (size_t)s.r0 * C, s.n * C * 2, p.o_l[k]};
            }
        }
    } else if (ph == PH_P3) {
        if (b >= H) return;
        P3Plan p;
        p3_plan(A.m.mid, p);
#pragma unroll
        for (int m = 0; m < 4; m++)
            L.d[m] = Dma{Ly.up[m] + (size_t)b * 64 * A.m.mid[m], 64 * A.m.mid[m] * 2, p.o_up[m]};
        L.d[4] = Dma{Ly.rnn + (size_t)b * 4096, 4096 * 4, p.o_st};
    } else {
        int M, K, bb = b, gg = G;
        const uint8_t *ix;
        const uint32_t *sz;
        if (ph == PH_P4) {
            if (b < H) return;
            M = C; K = C; bb = b - H; gg = G - H; ix = Ly.idx[3]; sz = Ly.sz[3];
        } else if (ph == PH_P5) {
            M = F; K = C; ix = Ly.idx[4]; sz = Ly.sz[4];
        } else {
            M = C; K = F; ix = Ly.idx[5]; sz = Ly.sz[5];
        }
        I8Plan p;
        i8_plan(M, K, bb, gg, p);
        L.d[0] = Dma{ix + (size_t)p.r0 * K, p.n * K, 0};
        L.d[1] = Dma{sz + (size_t)p.r0 * (K / 128), p.n * (K / 32), p.o_sz};
    }
}

// Small per-layer vectors of the next phase (norm weights, token-shift
// coefficients and rows, decay/gate biases) are pulled into L2 while the
// barrier waits, so that the phase's plain loads of them hit L2.  Bit i of
// mask < 19 names the i-th vector field of MegaLayerDev (ln1_w .. k_a), bit
// 19 tmix, bit 20 cmix, bit 21 the ln_out weight and bias.  The workgroups
// of one XCD (b mod 8) share the 1 KiB pieces; the copies land in a scratch
// LDS slot (the 1 KiB below the weight region) that nothing reads.
enum : unsigned {
    PF_P1 = (1u << 0) | (1u << 1) | (0x3Fu << 6) | (1u << 19),
    PF_P3 = (1u << 4) | (1u << 5) | (0x3Fu << 13),
    PF_P5 = (1u << 2) | (1u << 3) | (1u << 12) | (1u << 20),
    PF_HEAD = 1u << 21,
};
__device__ __forceinline__ void l2_prefetch(const MegaArgs &A, int layer, unsigned mask, char *junk, int wv, int nw) {
    if (!mask || layer < 0) return;
    const int G = gridDim.x, per = G >= 8 ? G / 8 : 1, slot = (blockIdx.x / 8) % per;
    const int bytes = A.m.C * 4, upv = (bytes + 1023) / 1024;
    const int lane = threadIdx.x & 63;
    int ord = 0;
    for (int i = 0; i < 22; i++) {
        if (!(mask >> i & 1u)) continue;
        for (int h = 0; h < (i == 21 ? 2 : 1); h++) {
            const float *v;
            if (i < 19) v = ((const float *const *)&A.layers[layer])[i];
            else if (i == 19) v = A.layers[layer].tmix;
            else if (i == 20) v = A.layers[layer].cmix;
            else v = h ? A.m.lno_b : A.m.lno_w;
            const __amdgpu_buffer_rsrc_t r = rsrc(v, (unsigned)bytes);
            // pieces g = ord*upv + u of the concatenated list with g % per == slot
            const int g0 = ord * upv;
            int u = ((slot - g0) % per + per) % per;
            for (u += per * wv; u < upv; u += per * nw)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_vp)junk, 16, u * 1024 + lane * 16, 0, 0, 0);
            ord++;
        }
    }
}

// --------------------------------------------------------- grid barrier
// Every wave drains its stores, wave 0's first lane arrives on its group
// counter (the group's last arrival bumps the root) and spins on the root;
// meanwhile waves 1-3 copy the next phase's weights into LDS.  Returns false
// when the launch is aborting.
__device__ __forceinline__ bool grid_sync(const MegaArgs &A, unsigned k, const DmaList &pf, char *W, int *flag,
                                          int l2layer = -1, unsigned l2mask = 0) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (wave == 0) {
        if (threadIdx.x == 0) {
            const unsigned G = gridDim.x, g = blockIdx.x % kGroups;
            const unsigned ng = G < (unsigned)kGroups ? G : (unsigned)kGroups;
            const unsigned gs = (G - g + kGroups - 1) / kGroups;  // workgroups in group g
            unsigned *root = A.bar, *grp = A.bar + (g + 1) * kBarStride, *ab = A.bar + (kGroups + 1) * kBarStride;
            const unsigned old = __hip_atomic_fetch_add(grp, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (old + 1 == k * gs) __hip_atomic_fetch_add(root, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            int ok = 1;
            unsigned spins = 0;
            while (__hip_atomic_load(root, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < k * ng) {
                __builtin_amdgcn_s_sleep(1);
                if ((++spins & 255u) == 0 &&
                    (spins > kSpinLimit || __hip_atomic_load(ab, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))) {
                    __hip_atomic_store(ab, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    ok = 0;
                    break;
                }
            }
            *flag = ok;
        }
    } else {
        l2_prefetch(A, l2layer, l2mask, W - 1024, wave - 1, 3);
        dma_issue(pf, W, wave - 1, 3);
        __builtin_amdgcn_s_waitcnt(0);
    }
    __syncthreads();
    return *flag != 0;
}

// ------------------------------------------------------------ row GEMV
// Rows [0, n) of a weight slice staged in LDS (int8 idx + scale/zero words,
// or fp16), x (K floats) in LDS.  LG lanes own a row; lane li holds x of
// chunks li + LG*j in registers as fp16 pairs for all rows, and the products
// run on v_dot2_f32_f16 (fp32 accumulation).  An int8 byte q becomes the
// fp16 value 1024 + q with one byte permute per two weights, so per 16-weight
// chunk of a 128-group (model.rs:234-252):
//   sum w*x = s*sum(x*q) + z*sum(x) = s*D + (z - 1024 s)*sum(x),
//   D = sum x*(1024 + q),
// with sum(x) taken over the same fp16-rounded x.  x is multiplied by xs (a
// power of two that keeps it inside the fp16 range) and the row sums by 1/xs.
// Branch-free: chunks past the row end read a clamped address and carry
// x = 0.  The next row pass's loads are issued before the current pass is
// reduced (DPP), and epi(row, acc) runs once per row.
typedef _Float16 mh2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float4 f4zero_() { return make_float4(0.f, 0.f, 0.f, 0.f); }
template <bool I8>
struct RowTile {
    mu32x4 w[kCPL];
    uint32_t sz[kCPL];
};
template <bool I8>
__device__ __forceinline__ void row_load(RowTile<I8> &t, const char *wl, const uint32_t *sl, int rr, int rb, int KG,
                                         int li, int LG, int NC) {
    const char *wrow = wl + (size_t)rr * rb;
#pragma unroll
    for (int j = 0; j < kCPL; j++) {
        const int c = imin(li + LG * j, NC - 1);
        t.w[j] = *(const mu32x4 *)(wrow + 16 * c);
        if (I8) t.sz[j] = sl[rr * KG + (c >> 3)];
    }
}
__device__ __forceinline__ uint32_t h2pack(float a, float b) {
    mh2 h;
    h[0] = (_Float16)a;
    h[1] = (_Float16)b;
    return __builtin_bit_cast(uint32_t, h);
}
__device__ __forceinline__ float hsum2(uint32_t u) {
    const mh2 h = __builtin_bit_cast(mh2, u);
    return (float)h[0] + (float)h[1];
}
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(mh2, a), __builtin_bit_cast(mh2, b), c, false);
}
template <bool I8, typename Epi>
__device__ __forceinline__ void gemv_lds(int LG, const char *wl, const uint32_t *sl, int n, int K, const float *xv,
                                         float *part, float xs, Epi epi) {
    constexpr int CW = I8 ? 16 : 8;
    constexpr int P = CW / 4;
    const int NG = 256 / LG;
    const int WPG = LG > 64 ? LG / 64 : 1;
    const int RL = LG < 64 ? LG : 64;
    const int tid = threadIdx.x, grp = tid / LG, li = tid % LG;
    const int NC = K / CW, KG = K / 128;
    const int rb = I8 ? K : 2 * K;
    const float xinv = 1.0f / xs;
    uint32_t xh[kCPL][2 * P];
    float dxr[kCPL];
#pragma unroll
    for (int j = 0; j < kCPL; j++) {
        const int c = li + LG * j;
        const bool ok = c < NC;
        const int cc = ok ? c : 0;
        float sx = 0.0f;
#pragma unroll
        for (int p = 0; p < P; p++) {
            float4 t = ((const float4 *)xv)[cc * P + p];
            if (!ok) t = f4zero_();
            xh[j][2 * p] = h2pack(t.x * xs, t.y * xs);
            xh[j][2 * p + 1] = h2pack(t.z * xs, t.w * xs);
            sx += hsum2(xh[j][2 * p]) + hsum2(xh[j][2 * p + 1]);
        }
        dxr[j] = sx;
    }
    if (n <= 0) return;
    RowTile<I8> cur;
    row_load<I8>(cur, wl, sl, imin(grp, n - 1), rb, KG, li, LG, NC);
    for (int r0 = 0; r0 < n; r0 += NG) {
        const int r = r0 + grp;
        RowTile<I8> nxt;
        if (r0 + NG < n) row_load<I8>(nxt, wl, sl, imin(r + NG, n - 1), rb, KG, li, LG, NC);
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < kCPL; j++) {
            const mu32x4 w = cur.w[j];
            if (I8) {
                float d = 0.0f;
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    d = dot2(__builtin_amdgcn_perm(0x64646464u, w[q], 0x04010400u), xh[j][2 * q], d);
                    d = dot2(__builtin_amdgcn_perm(0x64646464u, w[q], 0x04030402u), xh[j][2 * q + 1], d);
                }
                const uint32_t sw = cur.sz[j];
                const float sc = h2f(sw), zp = h2f(sw >> 16);
                acc = fmaf(sc, d, fmaf(fmaf(-1024.0f, sc, zp), dxr[j], acc));
            } else {
#pragma unroll
                for (int q = 0; q < 4; q++) acc = dot2(w[q], xh[j][q], acc);
            }
        }
        acc = group_sum(acc, RL) * xinv;
        if (WPG == 1) {
            if (li == LG - 1 && r < n) epi(r, acc);
        } else if ((tid & 63) == 63 && r < n) {
            part[r * WPG + (li >> 6)] = acc;
        }
        if (r0 + NG < n) cur = nxt;
    }
    if (WPG > 1) {
        __syncthreads();
        for (int r = tid; r < n; r += 256) {
            float s = 0.0f;
            for (int w = 0; w < WPG; w++) s += part[r * WPG + w];
            epi(r, s);
        }
        __syncthreads();
    }
}

// Whole-row vectors are held four floats per lane: float4 index
// q = tid + 256*j.  Every load of a prologue is issued before the first use
// (branch-free, clamped index), so a phase start costs one memory latency.
constexpr int kQ = kCQ / 4;  // float4 per lane for rows of C elements
constexpr int kQF = 16;      // float4 per lane for rows of F elements (F <= 16384)
__device__ __forceinline__ float4 f4zero() { return make_float4(0.f, 0.f, 0.f, 0.f); }
template <int NQ>
__device__ __forceinline__ void vload(const float *p, int n4, float4 (&v)[NQ]) {
    const float4 *p4 = (const float4 *)p;
#pragma unroll
    for (int j = 0; j < NQ; j++) {
        const int q = threadIdx.x + 256 * j;
        const float4 t = p4[q < n4 ? q : 0];
        v[j] = q < n4 ? t : f4zero();
    }
}
template <int NQ>
__device__ __forceinline__ void aload(const ActIO &io, int base, int n4, float4 (&v)[NQ]) {
#pragma unroll
    for (int j = 0; j < NQ; j++) {
        const int q = threadIdx.x + 256 * j;
        const float4 t = io.ld4(base + 4 * (q < n4 ? q : 0));
        v[j] = q < n4 ? t : f4zero();
    }
}
__device__ __forceinline__ float4 mix4(float4 ln, float4 c, float4 p) {
    return make_float4(ln.x + c.x * (p.x - ln.x), ln.y + c.y * (p.y - ln.y), ln.z + c.z * (p.z - ln.z),
                       ln.w + c.w * (p.w - ln.w));
}
// LayerNorm of a row (two-pass, model.rs:625-635).
__device__ __forceinline__ void ln_rows(const float4 (&x)[kQ], const float4 (&g)[kQ], const float4 (&bt)[kQ], int C,
                                        float eps, float *red, float4 (&ln)[kQ]) {
    const int C4 = C / 4;
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < kQ; j++) s += (x[j].x + x[j].y) + (x[j].z + x[j].w);
    const float mu = bsum(s, red) / (float)C;
    float q = 0.0f;
#pragma unroll
    for (int j = 0; j < kQ; j++) {
        const float d0 = x[j].x - mu, d1 = x[j].y - mu, d2 = x[j].z - mu, d3 = x[j].w - mu;
        q += threadIdx.x + 256 * j < C4 ? (d0 * d0 + d1 * d1) + (d2 * d2 + d3 * d3) : 0.0f;
    }
    const float inv = 1.0f / sqrtf(bsum(q, red) / (float)C + eps);
#pragma unroll
    for (int j = 0; j < kQ; j++) {
        const bool ok = threadIdx.x + 256 * j < C4;
        ln[j] = ok ? make_float4((x[j].x - mu) * inv * g[j].x + bt[j].x, (x[j].y - mu) * inv * g[j].y + bt[j].y,
                                 (x[j].z - mu) * inv * g[j].z + bt[j].z, (x[j].w - mu) * inv * g[j].w + bt[j].w)
                   : f4zero();
    }
}

// act layout (floats)
struct ActOff {
    int x, r, k, v, vf, mid, yg, r2, lnk, cand, total;
};
__host__ __device__ inline ActOff act_off(const MegaModelDev &m) {
    ActOff o;
    const int C = m.C, L = m.mid[0] + m.mid[1] + m.mid[2] + m.mid[3];
    o.x = 0; o.r = C; o.k = 2 * C; o.v = 3 * C; o.vf = 4 * C; o.mid = 5 * C;
    o.yg = 5 * C + L; o.r2 = 6 * C + L; o.lnk = 6 * C + L + m.F; o.cand = 7 * C + L + m.F;
    o.total = o.cand + 2 * 1024;
    return o;
}

__global__ __launch_bounds__(256, 1) void k_mega(MegaArgs A) {
    extern __shared__ __align__(16) char smem[];
    char *W = smem + A.o_w;
    float *XV = (float *)(smem + A.o_xv);
    float4 *XV4 = (float4 *)XV;
    float *MIDS = (float *)(smem + A.o_mids);
    float *part = (float *)(smem + A.o_part);
    float *hv = (float *)(smem + A.o_hv);  // kh, b, w, k_mod, r: 5 x 64
    float *red = (float *)(smem + A.o_misc);
    int *flag = (int *)(smem + A.o_misc + 64);
    float *xo = (float *)(smem + A.o_misc + 128);  // own residual rows
    const int tid = threadIdx.x, b = blockIdx.x, G = gridDim.x;
    const MegaModelDev &M = A.m;
    const int C = M.C, F = M.F, H = M.H, C4 = C / 4, F4 = F / 4;
    const ActOff ao = act_off(M);
    const ActIO io{rsrc(A.act, A.act_bytes)};
    if (__hip_atomic_load(A.bar + (kGroups + 1) * kBarStride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) return;
    unsigned bk = 0;  // barriers passed

    // embedding row (gpu_model.rs:1879-1885); an id past the table gives zeros
    const uint32_t tok = A.token_in[0];
    const bool tok_ok = tok < (uint32_t)M.V;
    const float *erow = M.emb + (tok_ok ? (size_t)tok * C : 0);
    {
        // residual rows owned through ffn.value start as the embedding row
        const int r0 = part_lo(C, b, G), r1 = part_lo(C, b + 1, G);
        if (r0 + tid < r1) io.st(ao.x + r0 + tid, tok_ok ? erow[r0 + tid] : 0.0f);
        DmaList pf;
        build_dma(A, 0, PH_P1, b, pf);
        dma_issue(pf, W, __builtin_amdgcn_readfirstlane(tid >> 6), 4);
    }

    for (int li = 0; li < M.n_layer; li++) {
        const MegaLayerDev &L = A.layers[li];
        tmark(A, li, 0);
        // ---------------------------------------------------------- P1
        {
            float4 x4[kQ], g4[kQ], b4[kQ], p4[kQ], ln[kQ];
            if (li == 0) {
                vload(erow, C4, x4);
                if (!tok_ok)
#pragma unroll
                    for (int j = 0; j < kQ; j++) x4[j] = f4zero();
            } else {
                aload(io, ao.x, C4, x4);
            }
            vload(L.ln1_w, C4, g4);
            vload(L.ln1_b, C4, b4);
            vload(L.tmix, C4, p4);
            P1Plan p;
            p1_plan(C, M.mid, b, G, p);
            // coefficient rows of the (up to four) mixes this workgroup needs
            float4 cf[4][kQ];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const bool i8s = k < 2;
                const int kk = k & 1;
                const bool on = kk < (i8s ? p.n8 : p.nl);
                const int mat = on ? (i8s ? p.s8[kk].mat : p.sl[kk].mat) : 0;
                const float *c = i8s ? (mat == 0 ? L.x_r : mat == 1 ? L.x_k : L.x_v)
                                     : (mat == 0 ? L.x_w : mat == 1 ? L.x_a : mat == 2 ? L.x_v : L.x_g);
                if (on) vload(c, C4, cf[k]);
            }
            ln_rows(x4, g4, b4, C, M.ln_eps, red, ln);
#pragma unroll
            for (int j = 0; j < kQ; j++) {
                const int q = tid + 256 * j;
                if (q >= C4) continue;
                if (b == 0) io.st4(ao.lnk + 4 * q, ln[j]);  // token-shift row, stored once every workgroup has read it
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const bool on = (k & 1) < (k < 2 ? p.n8 : p.nl);
                    if (on) XV4[k * C4 + q] = mix4(ln[j], cf[k][j], p4[j]);
                }
            }
            __builtin_amdgcn_s_waitcnt(0);  // layer 0: this workgroup's own weight copies
            __syncthreads();
            tmark(A, li, 12);
#pragma unroll
            for (int k = 0; k < 2; k++) {
                if (k >= p.n8) continue;
                const RowSeg sg = p.s8[k];
                const bool vf = li == 0 && sg.mat == 2;
                gemv_lds<true>(A.lg_c8, W + p.o_idx[k], (const uint32_t *)(W + p.o_sz[k]), sg.n, C, XV + k * C, part, 1.0f,
                               [&](int r, float acc) {
                                   io.st(ao.r + sg.mat * C + sg.r0 + r, acc);
                                   if (vf) io.st(ao.vf + sg.r0 + r, acc);  // v_first (gpu_model.rs:2200-2204)
                               });
            }
#pragma unroll
            for (int k = 0; k < 2; k++) {
                if (k >= p.nl) continue;
                const RowSeg sg = p.sl[k];
                const int base = ao.mid + sg.r0 + (sg.mat > 0 ? M.mid[0] : 0) + (sg.mat > 1 ? M.mid[1] : 0) +
                                 (sg.mat > 2 ? M.mid[2] : 0);
                const bool th = sg.mat == 0;
                gemv_lds<false>(A.lg_c16, W + p.o_l[k], nullptr, sg.n, C, XV + (2 + k) * C, part, 1.0f,
                                [&](int r, float acc) { io.st(base + r, th ? tanhf(acc) : acc); });
            }
            DmaList pf;
            build_dma(A, li, b < H ? PH_P3 : PH_P4, b, pf);
            tmark(A, li, 1);
            if (!grid_sync(A, ++bk, pf, W, flag, li, PF_P3)) return;
            tmark(A, li, 2);
        }
        // ---------------------------------------------------------- P3
        if (b < H) {
            P3Plan p;
            p3_plan(M.mid, p);
            const int j = tid >> 2, q = tid & 3, c = b * 64 + j;
            const int L4 = M.mid[0] + M.mid[1] + M.mid[2] + M.mid[3], g0 = L4 - M.mid[3];
            // every load of the phase first
            const float kc = io.ld(ao.k + c), rc = io.ld(ao.r + c), vc = io.ld(ao.v + c);
            const float vfc = io.ld((li == 0 ? ao.v : ao.vf) + c);
            const bool mq = tid < L4 / 4;
            const float4 mv = io.ld4(ao.mid + 4 * (mq ? tid : 0));
            const float w0 = L.w0[c], a0 = L.a0[c], v0 = L.v0[c], kkc = L.k_k[c], kac = L.k_a[c], rkc = L.r_k[c];
            const float lw = L.lnx_w[c], lb = L.lnx_b[c], sw = M.scale_w[0];
            float4 lk[kQ];
            if (b == 0) aload(io, ao.lnk, C4, lk);
            if (mq) {
                float4 t = mv;
                if (4 * tid >= g0) t = make_float4(sigm(t.x), sigm(t.y), sigm(t.z), sigm(t.w));  // g input: sigmoid
                ((float4 *)MIDS)[tid] = t;
            }
            if (b == 0)
#pragma unroll
                for (int jj = 0; jj < kQ; jj++) {
                    const int qq = tid + 256 * jj;
                    if (qq < C4) ((float4 *)L.tmix)[qq] = lk[jj];
                }
            if (li == 0 && q == 0) M.v_first[c] = vc;
            __syncthreads();
            float acc[4];
            int mo = 0;
#pragma unroll
            for (int m = 0; m < 4; m++) {
                const int mid = M.mid[m], seg = mid >> 2;
                const char *row = W + p.o_up[m] + (size_t)(j * mid + q * seg) * 2;
                const float *xm = MIDS + mo + q * seg;
                float sm = 0.0f;
                for (int e = 0; e < seg; e += 8) {
                    const mu32x4 w = *(const mu32x4 *)(row + 2 * e);
                    const float4 x0 = *(const float4 *)(xm + e), x1 = *(const float4 *)(xm + e + 4);
                    sm = fmaf(x0.x, h2f(w[0]), sm);
                    sm = fmaf(x0.y, h2f(w[0] >> 16), sm);
                    sm = fmaf(x0.z, h2f(w[1]), sm);
                    sm = fmaf(x0.w, h2f(w[1] >> 16), sm);
                    sm = fmaf(x1.x, h2f(w[2]), sm);
                    sm = fmaf(x1.y, h2f(w[2] >> 16), sm);
                    sm = fmaf(x1.z, h2f(w[3]), sm);
                    sm = fmaf(x1.w, h2f(w[3] >> 16), sm);
                }
                sm += dppf<0xB1>(sm);
                sm += dppf<0x4E>(sm);
                acc[m] = sm;
                mo += mid;
            }
            // LoRA-up epilogues (gpu_model.rs:2206-2262)
            const float wd = expf(sigm(acc[0] + w0) * sw);
            const float aa = sigm(acc[1] + a0);
            const float gv = sigm(acc[2] + v0);
            const float vv = vc + gv * (vfc - vc);
            const float gg = acc[3];
            // WKV7 head vectors (model.rs:445-473, 716-826)
            const float kk = kc * kkc;
            float nrm = sqrtf(bsum(q == 0 ? kk * kk : 0.0f, red));
            nrm = nrm < M.l2_eps ? M.l2_eps : nrm;
            const float inv = 1.0f / nrm;
            const float kh = kk * inv;
            const float kmod = kc + kac * (kc * aa - kc);
            if (q == 0) {
                hv[j] = kh;
                hv[64 + j] = kh * (-aa);
                hv[128 + j] = wd;
                hv[192 + j] = kmod;
                hv[256 + j] = rc;
            }
            const float bonus = bsum(q == 0 ? rc * kmod * rkc : 0.0f, red);
            // state row j, columns 16q..16q+15: S = S diag(w) + (S k_hat) b^T + v k_mod^T; y = S r
            const float *st = (const float *)(W + p.o_st) + j * 64 + 16 * q;
            float sr[16];
#pragma unroll
            for (int m = 0; m < 4; m++) {
                const float4 t = *(const float4 *)(st + 4 * m);
                sr[4 * m] = t.x; sr[4 * m + 1] = t.y; sr[4 * m + 2] = t.z; sr[4 * m + 3] = t.w;
            }
            float sa = 0.0f;
#pragma unroll
            for (int jj = 0; jj < 16; jj++) sa = fmaf(sr[jj], hv[16 * q + jj], sa);
            sa += dppf<0xB1>(sa);
            sa += dppf<0x4E>(sa);
            float y = 0.0f;
#pragma unroll
            for (int jj = 0; jj < 16; jj++) {
                const int cc = 16 * q + jj;
                const float ns = sr[jj] * hv[128 + cc] + sa * hv[64 + cc] + vv * hv[192 + cc];
                sr[jj] = ns;
                y = fmaf(ns, hv[256 + cc], y);
            }
            y += dppf<0xB1>(y);
            y += dppf<0x4E>(y);
            float4 *sg = (float4 *)(L.rnn + (size_t)b * 4096 + j * 64 + 16 * q);
#pragma unroll
            for (int m = 0; m < 4; m++) sg[m] = make_float4(sr[4 * m], sr[4 * m + 1], sr[4 * m + 2], sr[4 * m + 3]);
            // GroupNorm over the head (two-pass) + bonus, then y*g for att.output
            const float mean = bsum(q == 0 ? y : 0.0f, red) * (1.0f / 64.0f);
            const float d = y - mean;
            const float var = bsum(q == 0 ? d * d : 0.0f, red) * (1.0f / 64.0f) + M.gn_eps;
            const float yn = d * (1.0f / sqrtf(var)) * lw + lb + bonus * vv;
            if (q == 0) io.st(ao.yg + c, yn * gg);
        }
        {
            DmaList pf;
            build_dma(A, li, b < H ? PH_P5 : PH_NONE, b, pf);
            tmark(A, li, 3);
            if (!grid_sync(A, ++bk, pf, W, flag)) return;
            tmark(A, li, 4);
        }
        // ---------------------------------------------------------- P4
        if (b >= H) {
            I8Plan p;
            i8_plan(C, C, b - H, G - H, p);
            float4 yv[kQ];
            aload(io, ao.yg, C4, yv);
            const float xr = io.ld(ao.x + p.r0 + (tid < p.n ? tid : 0));
#pragma unroll
            for (int j = 0; j < kQ; j++)
                if (tid + 256 * j < C4) XV4[tid + 256 * j] = yv[j];
            if (tid < p.n) xo[tid] = xr;
            __syncthreads();
            gemv_lds<true>(A.lg_c8, W, (const uint32_t *)(W + p.o_sz), p.n, C, XV, part, 1.0f,
                           [&](int r, float acc) { io.st(ao.x + p.r0 + r, xo[r] + acc); });
        }
        {
            DmaList pf;
            build_dma(A, li, b < H ? PH_NONE : PH_P5, b, pf);
            tmark(A, li, 5);
            if (!grid_sync(A, ++bk, pf, W, flag, li, PF_P5)) return;
            tmark(A, li, 6);
        }
        // ---------------------------------------------------------- P5
        {
            float4 x4[kQ], g4[kQ], b4[kQ], p4[kQ], c4[kQ], ln[kQ];
            aload(io, ao.x, C4, x4);
            vload(L.ln2_w, C4, g4);
            vload(L.ln2_b, C4, b4);
            vload(L.cmix, C4, p4);
            vload(L.ffn_x_k, C4, c4);
            ln_rows(x4, g4, b4, C, M.ln_eps, red, ln);
#pragma unroll
            for (int j = 0; j < kQ; j++) {
                const int q = tid + 256 * j;
                if (q >= C4) continue;
                XV4[q] = mix4(ln[j], c4[j], p4[j]);
                if (b == 0) io.st4(ao.lnk + 4 * q, ln[j]);
            }
            __syncthreads();
            tmark(A, li, 11);
            I8Plan p;
            i8_plan(F, C, b, G, p);
            gemv_lds<true>(A.lg_c8, W, (const uint32_t *)(W + p.o_sz), p.n, C, XV, part, 1.0f, [&](int r, float acc) {
                const float t = acc > 0.0f ? acc : 0.0f;
                io.st(ao.r2 + p.r0 + r, t * t);
            });
            DmaList pf;
            build_dma(A, li, PH_P6, b, pf);
            tmark(A, li, 7);
            if (!grid_sync(A, ++bk, pf, W, flag)) return;
            tmark(A, li, 8);
        }
        // ---------------------------------------------------------- P6
        {
            I8Plan p;
            i8_plan(C, F, b, G, p);
            float4 rv[kQF], lk[kQ];
            aload(io, ao.r2, F4, rv);
            const float xr = io.ld(ao.x + p.r0 + (tid < p.n ? tid : 0));
            if (b == 0) aload(io, ao.lnk, C4, lk);
            // relu^2 rows can exceed the fp16 range: scale by a power of two that
            // maps the largest element to at most 2^14
            float mx = 0.0f;
#pragma unroll
            for (int j = 0; j < kQF; j++) {
                if (tid + 256 * j < F4) XV4[tid + 256 * j] = rv[j];
                mx = fmaxf(mx, fmaxf(fmaxf(fabsf(rv[j].x), fabsf(rv[j].y)), fmaxf(fabsf(rv[j].z), fabsf(rv[j].w))));
            }
            if (tid < p.n) xo[tid] = xr;
            const float xs = row_scale(mx, red);
            if (b == 0)
#pragma unroll
                for (int j = 0; j < kQ; j++) {
                    const int q = tid + 256 * j;
                    if (q < C4) ((float4 *)L.cmix)[q] = lk[j];
                }
            __syncthreads();
            tmark(A, li, 13);
            gemv_lds<true>(A.lg_f8, W, (const uint32_t *)(W + p.o_sz), p.n, F, XV, part, xs,
                           [&](int r, float acc) { io.st(ao.x + p.r0 + r, xo[r] + acc); });
            DmaList pf;
            build_dma(A, li + 1, li + 1 < M.n_layer ? PH_P1 : PH_HEAD, b, pf);
            tmark(A, li, 9);
            if (!grid_sync(A, ++bk, pf, W, flag, li + 1 < M.n_layer ? li + 1 : li, li + 1 < M.n_layer ? PF_P1 : PF_HEAD))
                return;
            tmark(A, li, 10);
        }
    }

    // -------------------------------------------------------------- head
    {
        float4 x4[kQ], g4[kQ], b4[kQ], ln[kQ];
        aload(io, ao.x, C4, x4);
        vload(M.lno_w, C4, g4);
        vload(M.lno_b, C4, b4);
        ln_rows(x4, g4, b4, C, M.ln_eps, red, ln);
#pragma unroll
        for (int j = 0; j < kQ; j++)
            if (tid + 256 * j < C4) XV4[tid + 256 * j] = ln[j];
        HeadPlan hp;
        head_plan(M.V, C, M.head_i8, A.w_bytes, b, G, hp);
        const long long rb = M.head_i8 ? C : 2LL * C;
        float bv = -1e30f;
        int bi = 0;
        const int rounds = (hp.n + hp.rr - 1) / hp.rr;
        for (int rd = 0; rd < rounds; rd++) {
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            if (rd + 1 < rounds) {
                const int rs = hp.r0 + (rd + 1) * hp.rr, n = imin(hp.rr, hp.n - (rd + 1) * hp.rr);
                const int base = ((rd + 1) & 1) * hp.half;
                DmaList L;
                dma_clear(L);
                L.d[0] = Dma{(const char *)M.head + (size_t)rs * rb, (int)(n * rb), base};
                if (M.head_i8) L.d[1] = Dma{M.head_sz + (size_t)rs * (C / 128), n * (C / 32), base + hp.o_sz};
                dma_issue(L, W, __builtin_amdgcn_readfirstlane(tid >> 6), 4);
            }
            const int base = (rd & 1) * hp.half, r0 = hp.r0 + rd * hp.rr, n = imin(hp.rr, hp.n - rd * hp.rr);
            auto epi = [&](int r, float acc) {
                const int row = r0 + r;
                if (A.logits) A.logits[row] = acc;
                if (acc > bv || (acc == bv && row < bi)) { bv = acc; bi = row; }
            };
            if (M.head_i8)
                gemv_lds<true>(A.lg_head, W + base, (const uint32_t *)(W + base + hp.o_sz), n, C, XV, part, 1.0f, epi);
            else
                gemv_lds<false>(A.lg_head, W + base, nullptr, n, C, XV, part, 1.0f, epi);
        }
        // workgroup candidate, smallest index among equal maxima (backend_cuda.rs:3640-3680)
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const float ov = __shfl_xor(bv, o, 64);
            const int oi = __shfl_xor(bi, o, 64);
            if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
        }
        __syncthreads();
        if ((tid & 63) == 0) { red[tid >> 6] = bv; ((int *)red)[4 + (tid >> 6)] = bi; }
        __syncthreads();
        if (tid == 0) {
            float v = red[0];
            int ix = ((int *)red)[4];
            for (int w = 1; w < 4; w++) {
                const float ov = red[w];
                const int oi = ((int *)red)[4 + w];
                if (ov > v || (ov == v && oi < ix)) { v = ov; ix = oi; }
            }
            io.st(ao.cand + 2 * b, v);
            io.st(ao.cand + 2 * b + 1, __int_as_float(ix));
        }
        DmaList none;
        dma_clear(none);
        if (!grid_sync(A, ++bk, none, W, flag)) return;
        if (b == 0) {
            float v = -1e30f;
            int ix = 0;
            for (int g = tid; g < G; g += 256) {
                const float ov = io.ld(ao.cand + 2 * g);
                const int oi = __float_as_int(io.ld(ao.cand + 2 * g + 1));
                if (ov > v || (ov == v && oi < ix)) { v = ov; ix = oi; }
            }
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) {
                const float ov = __shfl_xor(v, o, 64);
                const int oi = __shfl_xor(ix, o, 64);
                if (ov > v || (ov == v && oi < ix)) { v = ov; ix = oi; }
            }
            __syncthreads();
            if ((tid & 63) == 0) { red[tid >> 6] = v; ((int *)red)[4 + (tid >> 6)] = ix; }
            __syncthreads();
            if (tid == 0) {
                for (int w = 1; w < 4; w++) {
                    const float ov = red[w];
                    const int oi = ((int *)red)[4 + w];
                    if (ov > red[0] || (ov == red[0] && oi < ((int *)red)[4])) { red[0] = ov; ((int *)red)[4] = oi; }
                }
                A.token_out[0] = (uint32_t)((int *)red)[4];
            }
        }
    }
}

// Barrier counters back to zero before a launch (an ordinary kernel, so that
// a captured graph holds no memset node).  The abort flag is left alone.
__global__ void k_mega_reset(unsigned *bar) {
    const int i = threadIdx.x;
    if (i <= kGroups) bar[i * kBarStride] = 0u;
}

}  // namespace

struct MegaPlanHost {
    MegaArgs a;
    unsigned long long *trace = nullptr;
    MegaLayerDev *layers_dev = nullptr;
    float *act = nullptr;
    unsigned *bar = nullptr;
    int grid = 0, lds = 0;
};

void mega_free(rsv_ctx *ctx) {
    MegaPlanHost *p = (MegaPlanHost *)ctx->mega;
    if (!p) return;
    if (p->layers_dev) (void)hipFree(p->layers_dev);
    if (p->act) (void)hipFree(p->act);
    if (p->bar) (void)hipFree(p->bar);
    if (p->trace) (void)hipFree(p->trace);
    delete p;
    ctx->mega = nullptr;
}

int mega_build(rsv_ctx *ctx, const MegaModelDev &m, const std::vector<MegaLayerDev> &layers) {
    mega_free(ctx);
    if ((int)layers.size() != m.n_layer || m.n_layer <= 0) return RSV_FAIL("mega: %d layer records for %d layers", (int)layers.size(), m.n_layer);
    const int C = m.C, F = m.F, H = m.H;
    int dev = ctx->device;
    hipDeviceProp_t prop;
    RSV_HIP(hipGetDeviceProperties(&prop, dev));
    const int G = prop.multiProcessorCount;
    if (C % 256 || C > 256 * kCQ || H * 64 != C) return RSV_FAIL("mega: n_embd %d unsupported", C);
    if (F % 256) return RSV_FAIL("mega: ffn %d unsupported", F);
    for (int q = 0; q < 4; q++)
        if (m.mid[q] <= 0 || m.mid[q] % 32) return RSV_FAIL("mega: LoRA rank %d unsupported", m.mid[q]);
    if (G <= H || G > 1024) return RSV_FAIL("mega: %d CUs for %d heads", G, H);
    MegaArgs a{};
    a.m = m;
    a.lg_c8 = lanes_for(C, true);
    a.lg_f8 = lanes_for(F, true);
    a.lg_c16 = lanes_for(C, false);
    a.lg_head = lanes_for(C, m.head_i8 != 0);
    if (!a.lg_c8 || !a.lg_f8 || !a.lg_c16 || !a.lg_head) return RSV_FAIL("mega: rows too long (C %d, F %d)", C, F);
    // weight region: the largest per-workgroup slice of any phase
    int wmax = 0, n_own = 0, n_part = 0;
    for (int b = 0; b < G; b++) {
        P1Plan p1;
        p1_plan(C, m.mid, b, G, p1);
        if (!p1.whole) return RSV_FAIL("mega: stage-1 rows of workgroup %d span three matrices", b);
        wmax = std::max(wmax, p1.bytes);
        I8Plan p;
        i8_plan(F, C, b, G, p);
        wmax = std::max(wmax, p.bytes);
        n_part = std::max(n_part, p.n);
        i8_plan(C, F, b, G, p);
        wmax = std::max(wmax, p.bytes);
        n_own = std::max(n_own, p.n);
        if (b >= H) {
            i8_plan(C, C, b - H, G - H, p);
            wmax = std::max(wmax, p.bytes);
            n_own = std::max(n_own, p.n);
        }
    }
    P3Plan p3;
    p3_plan(m.mid, p3);
    wmax = std::max(wmax, p3.bytes);
    const long long hrb = m.head_i8 ? C : 2LL * C;
    wmax = std::max(wmax, 2 * (pad1k(hrb) + pad1k(m.head_i8 ? C / 32 : 0)));
    wmax = (wmax + 2047) & ~2047;
    if (n_own > kOwnMax || n_part * 4 > kPartMax) return RSV_FAIL("mega: %d rows per workgroup", std::max(n_own, n_part));
    const int Lm = m.mid[0] + m.mid[1] + m.mid[2] + m.mid[3];
    int off = 0;
    a.o_misc = off; off += 128 + kOwnMax * 4;
    a.o_hv = off; off += 5 * 64 * 4;
    a.o_part = off; off += kPartMax * 4;
    a.o_mids = off; off += ((Lm * 4 + 15) & ~15);
    a.o_xv = off; off += std::max(4 * C, F) * 4;
    off = ((off + 1023) & ~1023) + 1024;  // 1 KiB scratch slot for the L2 prefetch copies, then the weights
    a.o_w = off; off += wmax;
    a.w_bytes = wmax;
    if (off > (int)prop.sharedMemPerBlock) return RSV_FAIL("mega: %d bytes of LDS needed, %d available", off, (int)prop.sharedMemPerBlock);
    RSV_HIP(hipFuncSetAttribute((const void *)k_mega, hipFuncAttributeMaxDynamicSharedMemorySize, off));
    int occ = 0;
    RSV_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, k_mega, 256, off));
    if (occ < 1) return RSV_FAIL("mega: kernel does not fit one CU");
    MegaPlanHost *P = new MegaPlanHost();
    const ActOff ao = act_off(m);
    const size_t act_bytes = (size_t)(ao.cand + 2 * G) * 4;
    if (hipMalloc(&P->layers_dev, layers.size() * sizeof(MegaLayerDev)) != hipSuccess ||
        hipMalloc(&P->act, act_bytes) != hipSuccess || hipMalloc(&P->bar, (kGroups + 2) * kBarStride * 4) != hipSuccess) {
        ctx->mega = P;
        mega_free(ctx);
        return RSV_FAIL("mega: device allocation failed");
    }
    ctx->mega = P;
    RSV_HIP(hipMemcpy(P->layers_dev, layers.data(), layers.size() * sizeof(MegaLayerDev), hipMemcpyHostToDevice));
    RSV_HIP(hipMemset(P->act, 0, act_bytes));
    RSV_HIP(hipMemset(P->bar, 0, (kGroups + 2) * kBarStride * 4));
    a.layers = P->layers_dev;
    a.act = P->act;
    a.act_bytes = (unsigned)act_bytes;
    a.bar = P->bar;
    const char *tr = getenv("RSV_MEGA_TRACE");
    if (tr && tr[0]) {
        const size_t tb = (size_t)kTraceN * G * 16 * 8;
        RSV_HIP(hipMalloc(&P->trace, tb));
        RSV_HIP(hipMemset(P->trace, 0, tb));
        a.trace = P->trace;
    }
    P->a = a;
    P->grid = G;
    P->lds = off;
    return 0;
}

int mega_launch(rsv_ctx *ctx, const uint32_t *token_in, uint32_t *token_out, float *logits) {
    MegaPlanHost *P = (MegaPlanHost *)ctx->mega;
    if (!P) return RSV_FAIL("mega: not built");
    MegaArgs a = P->a;
    a.token_in = token_in;
    a.token_out = token_out;
    a.logits = logits;
    hipLaunchKernelGGL(k_mega_reset, dim3(1), dim3(64), 0, ctx->stream, P->bar);
    RSV_HIP(hipGetLastError());
    hipLaunchKernelGGL(k_mega, dim3(P->grid), dim3(256), (size_t)P->lds, ctx->stream, a);
    RSV_HIP(hipGetLastError());
    return 0;
}

int mega_vocab(rsv_ctx *ctx) {
    const MegaPlanHost *P = (const MegaPlanHost *)ctx->mega;
    return P ? P->a.m.V : 0;
}

int mega_status(rsv_ctx *ctx, int *aborted) {
    MegaPlanHost *P = (MegaPlanHost *)ctx->mega;
    if (!P) return RSV_FAIL("mega: not built");
    unsigned v = 0;
    RSV_HIP(hipStreamSynchronize(ctx->stream));
    RSV_HIP(hipMemcpy(&v, P->bar + (kGroups + 1) * kBarStride, 4, hipMemcpyDeviceToHost));
    *aborted = v != 0;
    const char *tr = getenv("RSV_MEGA_TRACE");
    if (P->trace && tr && tr[0]) {
        std::vector<unsigned long long> h((size_t)kTraceN * P->grid * 16);
        RSV_HIP(hipMemcpy(h.data(), P->trace, h.size() * 8, hipMemcpyDeviceToHost));
        if (FILE *f = fopen(tr, "wb")) {
            fwrite(h.data(), 8, h.size(), f);
            fclose(f);
        }
    }
    return 0;
}

}  // namespace rsv
