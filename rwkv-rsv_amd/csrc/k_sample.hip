// On-GPU sampler: penalties -> 1/T -> top-k -> softmax -> top-p -> seeded
// draw.  Rows without top-k and with 0 < top_p < 1 (the serving case) run on
// three launches spread over the chip (k_samp_scale / k_samp_exp /
// k_samp_pick, below); every other row runs the whole pipeline on one
// 1024-thread block.
//
// Observable behaviour follows backend_cuda.rs:3690-4009:
//  - sampler row [T, top_k bits, top_p, seed bits, rep, freq, pres, hist_len bits]
//  - top_k in 1..50: keep values >= K-th largest; candidate list sorted
//    descending; top-p accumulates from the K-th candidate toward the largest;
//    the draw scans that list from the K-th candidate upward
//  - otherwise: top_k > 50 keeps values >= K-th largest; top-p extracts at most
//    512 largest probabilities (ties -> smaller index) until the sum reaches
//    top_p; the draw is a CDF scan over the whole vocabulary in index order
//  - u = u01(seed) * total with u01 = golden-ratio add + MurmurHash3 fmix32.
// Instead of the reference's iterative block-argmax extraction, the R largest
// candidates (R = K or 512) are found with a 4-pass 8-bit radix select on
// order-preserving float keys, gathered in index order, and bitonic-sorted
// in LDS by (value desc, index asc) -- the same sequence the iterative
// extraction produces.
#include "rsv_common.h"
#include "k_dpp.h"

#include <mutex>

namespace rsv {

constexpr int kSampBS = 1024;
constexpr int kCand = 512;

__device__ __forceinline__ float u01_dev(uint32_t s) {
    s += 0x9E3779B9u;
    uint32_t z = s;
    z = (z ^ (z >> 16)) * 0x85EBCA6Bu;
    z = (z ^ (z >> 13)) * 0xC2B2AE35u;
    z ^= z >> 16;
    return (float)z / 4294967296.0f;
}

// Order-preserving key: larger float -> larger key; -0 folded onto +0.
__device__ __forceinline__ uint32_t fkey(float f) {
    if (f == 0.0f) f = 0.0f;
    const uint32_t b = __float_as_uint(f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

struct SampShared {
    uint32_t hist[256];
    uint32_t whist[kSampBS / 64][256];  // per-wave radix histograms
    float cval[kCand];                  // candidate values gathered for the serial scans
    uint32_t cnt_gt[kSampBS];
    uint32_t cnt_eq[kSampBS];
    float part[kSampBS];
    uint32_t ckey[kCand];
    int cidx[kCand];
    float red[16];
    uint32_t sel_bin, sel_rem;
    int chosen;
    float cutoff, u;
};

__device__ float block_max(float v, SampShared &sh) {
    v = wave_max_last(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 63) sh.red[threadIdx.x >> 6] = v;
    __syncthreads();
    float m = sh.red[0];
    for (int w = 1; w < 16; w++) m = fmaxf(m, sh.red[w]);
    return m;
}

__device__ float block_sum(float v, SampShared &sh) {
    v = wave_sum_last(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 63) sh.red[threadIdx.x >> 6] = v;
    __syncthreads();
    float s = 0.0f;
    for (int w = 0; w < 16; w++) s += sh.red[w];
    return s;
}

// The reference's 112-thread block sum (backend_cuda.rs:3880-3921): lane t
// sums t, t+112, ... in order, lanes 64..111 fold into 0..47, then a halving
// tree.  The float result depends on this order, so it is kept exactly.
__device__ float sum112(const float *t, int n, SampShared &sh) {
    __syncthreads();
    if (threadIdx.x < 112) {
        // the lane's elements in order; loads go out 16 at a time so the
        // sequential adds wait for one round trip per 16 instead of per element
        float s = 0.0f;
        int i = threadIdx.x;
        for (; i + 15 * 112 < n; i += 16 * 112) {
            float v[16];
#pragma unroll
            for (int e = 0; e < 16; e++) v[e] = t[i + e * 112];
#pragma unroll
            for (int e = 0; e < 16; e++) s += v[e];
        }
        for (; i < n; i += 112) s += t[i];
        sh.part[threadIdx.x] = s;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int q = 0; q < 48; q++) sh.part[q] += sh.part[q + 64];
        for (int step = 32; step > 0; step >>= 1)
            for (int q = 0; q < step; q++) sh.part[q] += sh.part[q + step];
        sh.u = sh.part[0];
    }
    __syncthreads();
    const float r = sh.u;
    __syncthreads();
    return r;
}

// Exclusive prefix sums of a[0..kSampBS) in place (one entry per thread),
// returning the total; integer, so the order of the additions is free.
__device__ uint32_t block_exscan(uint32_t *a, SampShared &sh) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const uint32_t v = a[tid];
    uint32_t x = v;  // inclusive scan within the wave
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const uint32_t y = __shfl_up(x, d);
        if (lane >= d) x += y;
    }
    __syncthreads();
    if (lane == 63) sh.red[wv] = __uint_as_float(x);
    __syncthreads();
    uint32_t off = 0, tot = 0;
    for (int w = 0; w < kSampBS / 64; w++) {
        const uint32_t s = __float_as_uint(sh.red[w]);
        off += w < wv ? s : 0u;
        tot += s;
    }
    a[tid] = off + x - v;
    __syncthreads();
    return tot;
}

// One radix pass: bin of 8 bits at `shift` of every key under (prefix, mask),
// counted in per-wave histograms (one add of the wave's count where all its
// lanes fall in one bin, the common case of the first pass over near-equal
// values), summed into sh.hist; then wave 0 finds the bin holding the
// remaining-th largest key (suffix sums over the 256 bins, 4 per lane) and
// leaves it in sh.sel_bin / sh.sel_rem.
__device__ __forceinline__ void radix_count(uint32_t k, bool in, int shift, bool first, SampShared &sh) {
    const int wv = threadIdx.x >> 6;
    const uint32_t bin = (k >> shift) & 255u;
    if (!first) {  // later passes: the bins spread, one add per key
        if (in) atomicAdd(&sh.whist[wv][bin], 1u);
        return;
    }
    const uint32_t b0 = __builtin_amdgcn_readfirstlane(bin);
    const uint64_t all = __ballot(1), same = __ballot(!in || bin == b0), cnt = __ballot(in);
    if (same == all) {
        if ((threadIdx.x & 63) == __ffsll((unsigned long long)all) - 1 && cnt)  // the first active lane
            atomicAdd(&sh.whist[wv][b0], (uint32_t)__popcll(cnt));
    } else if (in) {
        atomicAdd(&sh.whist[wv][bin], 1u);
    }
}

__device__ __forceinline__ void radix_clear(SampShared &sh) {
    const int wv = threadIdx.x >> 6;
    for (int i = threadIdx.x & 63; i < 256; i += 64) sh.whist[wv][i] = 0;
    __syncthreads();
}

__device__ __forceinline__ void radix_pick(uint32_t remaining, SampShared &sh) {
    __syncthreads();
    for (int i = threadIdx.x; i < 256; i += kSampBS) {
        uint32_t s = 0;
#pragma unroll
        for (int w = 0; w < kSampBS / 64; w++) s += sh.whist[w][i];
        sh.hist[i] = s;
    }
    __syncthreads();
    if (threadIdx.x < 64) {
        const int l = threadIdx.x;
        uint32_t h[4], s = 0;
#pragma unroll
        for (int e = 0; e < 4; e++) { h[e] = sh.hist[4 * l + e]; s += h[e]; }
        // suffix sum over lanes l..63 of the lane sums
        uint32_t suf = s;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const uint32_t y = __shfl_down(suf, d);
            if (l + d < 64) suf += y;
        }
        uint32_t above = suf - s;  // keys in bins above 4l+3
#pragma unroll
        for (int e = 3; e >= 0; e--) {
            if (above < remaining && above + h[e] >= remaining) {
                sh.sel_bin = (uint32_t)(4 * l + e);
                sh.sel_rem = remaining - above;
            }
            above += h[e];
        }
    }
    __syncthreads();
}

// Key of the R-th largest element (1-based) of t[0..n) (global memory).
__device__ uint32_t radix_select(const float *t, int n, int R, SampShared &sh) {
    uint32_t prefix = 0, mask = 0;
    uint32_t remaining = (uint32_t)R;
    for (int pass = 0; pass < 4; pass++) {
        const int shift = 24 - 8 * pass;
        radix_clear(sh);
        for (int i = threadIdx.x; i < n; i += kSampBS) {
            const uint32_t k = fkey(t[i]);
            radix_count(k, (k & mask) == prefix, shift, pass == 0, sh);
        }
        radix_pick(remaining, sh);
        prefix |= sh.sel_bin << shift;
        mask |= 255u << shift;
        remaining = sh.sel_rem;
        __syncthreads();
    }
    return prefix;
}

// The same over keys held in registers (kr[0..PER) of each thread, all live).
template <int PER>
__device__ uint32_t radix_select_regs(const uint32_t (&kr)[PER], int cnt, int R, SampShared &sh) {
    uint32_t prefix = 0, mask = 0;
    uint32_t remaining = (uint32_t)R;
    for (int pass = 0; pass < 4; pass++) {
        const int shift = 24 - 8 * pass;
        radix_clear(sh);
#pragma unroll
        for (int j = 0; j < PER; j++) radix_count(kr[j], (kr[j] & mask) == prefix, shift, pass == 0, sh);
        radix_pick(remaining, sh);
        prefix |= sh.sel_bin << shift;
        mask |= 255u << shift;
        remaining = sh.sel_rem;
        __syncthreads();
    }
    return prefix;
}

// Bitonic sort of sh.ckey/cidx[0..kCand): descending by key, ascending by index.
// A stage of stride < 64 pairs elements of one wave's 64 (thread i handles
// i and i ^ stride), so it needs only the wave's own LDS order, not a block
// barrier: 6 block barriers for 512 entries instead of 45.
__device__ void cand_sort(SampShared &sh) {
    for (int size = 2; size <= kCand; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            const int i = threadIdx.x;
            if (i < kCand) {
                const int j = i ^ stride;
                if (j > i) {
                    const bool up = (i & size) == 0;  // "up" blocks sort descending
                    const uint32_t ki = sh.ckey[i], kj = sh.ckey[j];
                    const int ii = sh.cidx[i], ij = sh.cidx[j];
                    const bool i_first = ki > kj || (ki == kj && ii < ij);
                    if (up != i_first) {
                        sh.ckey[i] = kj; sh.ckey[j] = ki;
                        sh.cidx[i] = ij; sh.cidx[j] = ii;
                    }
                }
            }
            // the next stage's pairs stay in the wave only if its stride is
            // below 64 too
            if (stride > 64) {
                __syncthreads();
            } else if (stride == 64 || (stride == 1 && size < kCand && 2 * size > 64)) {
                __syncthreads();
            } else {
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                __builtin_amdgcn_wave_barrier();
            }
        }
    }
    __syncthreads();
}

// Gathers the R largest keys (ties at the threshold by ascending index) into
// sh.ckey/cidx sorted by (key desc, index asc), R <= kCand.  Thread t holds
// the keys of its contiguous elements [lo, lo + PER) in kr.
template <int PER>
__device__ void top_r_keys(const uint32_t (&kr)[PER], int lo, int cnt, int R, SampShared &sh) {
    const uint32_t kthr = radix_select_regs<PER>(kr, cnt, R, sh);
    uint32_t gt = 0, eq = 0;
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const uint32_t k = kr[j];
        gt += k > kthr;
        eq += k == kthr;
    }
    sh.cnt_gt[threadIdx.x] = gt;
    sh.cnt_eq[threadIdx.x] = eq;
    const uint32_t G = block_exscan(sh.cnt_gt, sh);  // number strictly greater
    block_exscan(sh.cnt_eq, sh);
    uint32_t og = sh.cnt_gt[threadIdx.x], oe = sh.cnt_eq[threadIdx.x];
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const uint32_t k = kr[j];
        if (k > kthr) {
            sh.ckey[og] = k;
            sh.cidx[og] = lo + j;
            og++;
        } else if (k == kthr) {
            const uint32_t pos = G + oe;
            if (pos < (uint32_t)R) { sh.ckey[pos] = k; sh.cidx[pos] = lo + j; }
            oe++;
        }
    }
    for (int i = R + threadIdx.x; i < kCand; i += kSampBS) { sh.ckey[i] = 0u; sh.cidx[i] = 0x7FFFFFFF; }
    __syncthreads();
    cand_sort(sh);
}

// The same over t[0..n) in global memory (n > 64 x kSampBS: the general kernel).
__device__ void top_r(const float *t, int n, int R, SampShared &sh) {
    const uint32_t kthr = radix_select(t, n, R, sh);
    const int per = (n + kSampBS - 1) / kSampBS;
    const int lo = threadIdx.x * per, hi = min(n, lo + per);
    uint32_t gt = 0, eq = 0;
    for (int i = lo; i < hi; i++) {
        const uint32_t k = fkey(t[i]);
        gt += k > kthr;
        eq += k == kthr;
    }
    sh.cnt_gt[threadIdx.x] = gt;
    sh.cnt_eq[threadIdx.x] = eq;
    const uint32_t G = block_exscan(sh.cnt_gt, sh);
    block_exscan(sh.cnt_eq, sh);
    uint32_t og = sh.cnt_gt[threadIdx.x], oe = sh.cnt_eq[threadIdx.x];
    for (int i = lo; i < hi; i++) {
        const uint32_t k = fkey(t[i]);
        if (k > kthr) {
            sh.ckey[og] = k;
            sh.cidx[og] = i;
            og++;
        } else if (k == kthr) {
            const uint32_t pos = G + oe;
            if (pos < (uint32_t)R) { sh.ckey[pos] = k; sh.cidx[pos] = i; }
            oe++;
        }
    }
    for (int i = R + threadIdx.x; i < kCand; i += kSampBS) { sh.ckey[i] = 0u; sh.cidx[i] = 0x7FFFFFFF; }
    __syncthreads();
    cand_sort(sh);
}

// Inverse of fkey for the keys of non-negative-or-any floats (-0 came in as +0).
__device__ __forceinline__ float fkey_inv(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

// The whole pipeline for row b of any length, on the row in global memory.
__device__ void sample_row_general(int b, const float *__restrict__ logits, uint32_t *__restrict__ token, int n,
                                   float *__restrict__ temp_all, uint32_t *__restrict__ counter_all,
                                   const float *__restrict__ sampler, const uint32_t *__restrict__ hist_all,
                                   int hist_stride, SampShared &sh) {
    const int tid = threadIdx.x;
    const float *lg = logits + (size_t)b * n;
    float *temp = temp_all + (size_t)b * n;
    const float *sp = sampler + (size_t)b * 8;
    const float temperature = sp[0];
    const uint32_t top_k = __float_as_uint(sp[1]);
    const float top_p = sp[2];
    const uint32_t seed = __float_as_uint(sp[3]);
    const float rep = sp[4], freq = sp[5], pres = sp[6];
    // the row's history length, never past the row's own history capacity
    const uint32_t hist_len = min(__float_as_uint(sp[7]), (uint32_t)max(hist_stride, 0));
    const bool do_topk = top_k > 0u && top_k < (uint32_t)n;
    const int K = do_topk ? (int)top_k : 0;
    const bool fast = K > 0 && K <= 50;

    for (int i = tid; i < n; i += kSampBS) temp[i] = lg[i];
    __syncthreads();
    if (hist_len > 0u && hist_all && counter_all && (rep != 1.0f || freq != 0.0f || pres != 0.0f)) {
        uint32_t *counter = counter_all + (size_t)b * n;
        const uint32_t *hist = hist_all + (size_t)b * hist_stride;
        for (int i = tid; i < n; i += kSampBS) counter[i] = 0u;
        __syncthreads();
        for (uint32_t h = tid; h < hist_len; h += kSampBS) {
            const uint32_t tk = hist[h];
            if (tk < (uint32_t)n) atomicAdd(&counter[tk], 1u);
        }
        __syncthreads();
        for (int i = tid; i < n; i += kSampBS) {
            const uint32_t c = counter[i];
            float l = temp[i];
            if (c > 0u) {
                if (rep != 1.0f) l = l > 0.0f ? l / rep : l * rep;
                if (pres != 0.0f) l -= pres;
            }
            if (freq != 0.0f) l -= freq * (float)c;
            temp[i] = l;
        }
    }
    float invT = 1.0f / temperature;
    if (!(temperature > 0.0f)) invT = 1.0f;
    for (int i = tid; i < n; i += kSampBS) temp[i] *= invT;
    __syncthreads();

    if (fast) {
        top_r(temp, n, K, sh);  // sorted top-K list in sh.cidx[0..K)
        const float thr = __uint_as_float(0u);
        (void)thr;
        const float thv = temp[sh.cidx[K - 1]];
        __syncthreads();
        for (int i = tid; i < n; i += kSampBS)
            if (temp[i] < thv) temp[i] = -1e30f;
        __syncthreads();
    } else if (do_topk) {
        const uint32_t kthr = radix_select(temp, n, K, sh);
        for (int i = tid; i < n; i += kSampBS)
            if (fkey(temp[i]) < kthr) temp[i] = -1e30f;
        __syncthreads();
    }

    // softmax
    float lm = -1e30f;
    for (int i = tid; i < n; i += kSampBS) lm = fmaxf(lm, temp[i]);
    const float m = block_max(lm, sh);
    for (int i = tid; i < n; i += kSampBS) temp[i] = expf(temp[i] - m);
    const float total = sum112(temp, n, sh);
    if (total > 0.0f)
        for (int i = tid; i < n; i += kSampBS) temp[i] /= total;
    __syncthreads();

    if (top_p > 0.0f && top_p < 1.0f) {
        if (fast) {
            if (tid == 0) {
                float cum = 0.0f, cut = -1e30f;
                for (int j = K - 1; j >= 0; j--) {
                    const float p = temp[sh.cidx[j]];
                    cum += p;
                    cut = p;
                    if (cum >= top_p) break;
                }
                sh.cutoff = cut;
            }
        } else {
            const int R = n < kCand ? n : kCand;
            top_r(temp, n, R, sh);
            for (int c = tid; c < R; c += kSampBS) sh.cval[c] = temp[sh.cidx[c]];
            __syncthreads();
            if (tid == 0) {
                // the candidates in order until the sum reaches top_p; 16
                // values read per LDS round trip (the adds stay sequential)
                float cum = 0.0f, cut = 0.0f;
                for (int c0 = 0; c0 < R && cum < top_p; c0 += 16) {
                    float v[16];
#pragma unroll
                    for (int e = 0; e < 16; e++) v[e] = sh.cval[c0 + e];
#pragma unroll
                    for (int e = 0; e < 16; e++) {
                        if (c0 + e < R && cum < top_p) {
                            cum += v[e];
                            cut = v[e];
                        }
                    }
                }
                sh.cutoff = cut;
            }
        }
        __syncthreads();
        const float cut = sh.cutoff;
        for (int i = tid; i < n; i += kSampBS)
            if (temp[i] < cut) temp[i] = 0.0f;
        __syncthreads();
    }

    if (fast) {
        if (tid == 0) {
            float tot = 0.0f;
            for (int j = K - 1; j >= 0; j--) {
                const float p = temp[sh.cidx[j]];
                if (p > 0.0f) tot += p;
            }
            const float u = u01_dev(seed) * tot;
            float acc = 0.0f;
            int chosen = sh.cidx[K - 1];
            for (int j = K - 1; j >= 0; j--) {
                const int ix = sh.cidx[j];
                const float p = temp[ix];
                if (p > 0.0f) {
                    acc += p;
                    if (acc > u) { chosen = ix; break; }
                }
            }
            token[b] = (uint32_t)chosen;
        }
        return;
    }
    // CDF draw over the whole vocabulary in index order (backend_cuda.rs:
    // 3978-4007): u = u01(seed) * sum112(temp); the first i whose running
    // sequential sum exceeds u.  Zero entries do not change the running sum,
    // so when few entries are non-zero (top-p kept set) they are compacted in
    // index order and only those are scanned; otherwise one lane scans all n.
    const float tot = sum112(temp, n, sh);
    const int per = (n + kSampBS - 1) / kSampBS;
    const int lo = tid * per, hi = min(n, lo + per);
    // the thread's contiguous elements, in registers when at most 64
    constexpr int PER = 64;
    const int cnt = max(hi - lo, 0);
    const bool regs = per <= PER;
    float pv[PER];
    if (regs) {
#pragma unroll
        for (int j = 0; j < PER; j++) pv[j] = j < cnt ? temp[lo + j] : 0.0f;
    }
    uint32_t nz = 0;
    if (regs) {
#pragma unroll
        for (int j = 0; j < PER; j++) nz += pv[j] != 0.0f;
    } else {
        for (int i = lo; i < hi; i++) nz += temp[i] != 0.0f;
    }
    sh.cnt_gt[tid] = nz;
    const uint32_t NZ = block_exscan(sh.cnt_gt, sh);
    const bool compact = NZ <= (uint32_t)kCand;
    if (compact) {
        uint32_t o = sh.cnt_gt[tid];
        if (regs) {
#pragma unroll
            for (int j = 0; j < PER; j++)
                if (pv[j] != 0.0f) { sh.cidx[o] = lo + j; sh.cval[o] = pv[j]; o++; }
        } else {
            for (int i = lo; i < hi; i++) {
                const float p = temp[i];
                if (p != 0.0f) { sh.cidx[o] = i; sh.cval[o] = p; o++; }
            }
        }
    }
    __syncthreads();
    if (tid == 0) {
        const float u = u01_dev(seed) * tot;
        float acc = 0.0f;
        int chosen = n - 1;
        if (compact) {
            bool found = false;
            for (uint32_t j0 = 0; j0 < NZ && !found; j0 += 16) {
                float v[16];
#pragma unroll
                for (int e = 0; e < 16; e++) v[e] = sh.cval[j0 + e];
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    if (!found && j0 + e < NZ) {
                        acc += v[e];
                        if (acc > u) { chosen = sh.cidx[j0 + e]; found = true; }
                    }
                }
            }
        } else {
            for (int i = 0; i < n; i++) {
                acc += temp[i];
                if (acc > u) { chosen = i; break; }
            }
        }
        token[b] = (uint32_t)chosen;
    }
}

// The same pipeline for rows of exactly PER x kSampBS entries (PER a power of
// two up to 64) with the row in registers: thread t holds the PER contiguous
// entries [PER t, PER t + PER), so the passes (penalties, 1/T, top-k, max, exp, division,
// top-p cut, non-zero compaction) run on registers and the radix select on
// their keys.  Global memory (`temp`) is written only where the
// reference's summation order must be replayed: the two 112-lane sums, and
// the full-row CDF scan when more than 512 entries stay non-zero.  The
// candidates' probabilities are the inverse of their sort keys (exact).
// Every step computes what k_sample computes, in the same order.
template <int PER>
__device__ void sample_row_regs(int b, const float *__restrict__ logits, uint32_t *__restrict__ token, int n,
                                float *__restrict__ temp_all, uint32_t *__restrict__ counter_all,
                                const float *__restrict__ sampler, const uint32_t *__restrict__ hist_all,
                                int hist_stride, SampShared &sh) {
    const int tid = threadIdx.x;
    const float *lg = logits + (size_t)b * n;
    float *temp = temp_all + (size_t)b * n;
    const float *sp = sampler + (size_t)b * 8;
    const float temperature = sp[0];
    const uint32_t top_k = __float_as_uint(sp[1]);
    const float top_p = sp[2];
    const uint32_t seed = __float_as_uint(sp[3]);
    const float rep = sp[4], freq = sp[5], pres = sp[6];
    const uint32_t hist_len = min(__float_as_uint(sp[7]), (uint32_t)max(hist_stride, 0));
    const bool do_topk = top_k > 0u && top_k < (uint32_t)n;
    const int K = do_topk ? (int)top_k : 0;
    const bool fast = K > 0 && K <= 50;
    const int lo = tid * PER, cnt = PER;  // n == PER * kSampBS (launcher)
    float v[PER];
    auto load_row = [&](const float *src) {
        if constexpr (PER >= 4) {
            const float4 *s4 = (const float4 *)(src + lo);
#pragma unroll
            for (int q = 0; q < PER / 4; q++) {
                const float4 x = s4[q];
                v[4 * q] = x.x; v[4 * q + 1] = x.y; v[4 * q + 2] = x.z; v[4 * q + 3] = x.w;
            }
        } else {
#pragma unroll
            for (int j = 0; j < PER; j++) v[j] = src[lo + j];
        }
    };
    auto store_row = [&]() {
        if constexpr (PER >= 4) {
            float4 *d4 = (float4 *)(temp + lo);
#pragma unroll
            for (int q = 0; q < PER / 4; q++) d4[q] = make_float4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
        } else {
#pragma unroll
            for (int j = 0; j < PER; j++) temp[lo + j] = v[j];
        }
    };
    load_row(lg);
    if (hist_len > 0u && hist_all && counter_all && (rep != 1.0f || freq != 0.0f || pres != 0.0f)) {
        uint32_t *counter = counter_all + (size_t)b * n;
        const uint32_t *hist = hist_all + (size_t)b * hist_stride;
        for (int i = tid; i < n; i += kSampBS) counter[i] = 0u;
        __syncthreads();
        for (uint32_t h = tid; h < hist_len; h += kSampBS) {
            const uint32_t tk = hist[h];
            if (tk < (uint32_t)n) atomicAdd(&counter[tk], 1u);
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < PER; j++) {
            const uint32_t c = counter[lo + j];
            float l = v[j];
            if (c > 0u) {
                if (rep != 1.0f) l = l > 0.0f ? l / rep : l * rep;
                if (pres != 0.0f) l -= pres;
            }
            if (freq != 0.0f) l -= freq * (float)c;
            v[j] = l;
        }
    }
    float invT = 1.0f / temperature;
    if (!(temperature > 0.0f)) invT = 1.0f;
#pragma unroll
    for (int j = 0; j < PER; j++) v[j] *= invT;

    // the selections run on the keys of the row, which replace the values
    // in the same registers and are turned back after (fkey is a bijection
    // but for -0, which becomes +0: no comparison or exp sees the difference)
    uint32_t kr[PER];
    if (fast) {
#pragma unroll
        for (int j = 0; j < PER; j++) kr[j] = fkey(v[j]);
        top_r_keys<PER>(kr, lo, cnt, K, sh);  // sorted top-K list in sh.cidx[0..K)
        const uint32_t kth = sh.ckey[K - 1];
#pragma unroll
        for (int j = 0; j < PER; j++) v[j] = kr[j] < kth ? -1e30f : fkey_inv(kr[j]);
    } else if (do_topk) {
#pragma unroll
        for (int j = 0; j < PER; j++) kr[j] = fkey(v[j]);
        const uint32_t kthr = radix_select_regs<PER>(kr, cnt, K, sh);
#pragma unroll
        for (int j = 0; j < PER; j++) v[j] = kr[j] < kthr ? -1e30f : fkey_inv(kr[j]);
    }

    // softmax; the total in the reference's 112-lane order from global memory
    float lm = -1e30f;
#pragma unroll
    for (int j = 0; j < PER; j++) lm = fmaxf(lm, v[j]);
    const float m = block_max(lm, sh);
#pragma unroll
    for (int j = 0; j < PER; j++) v[j] = expf(v[j] - m);
    store_row();
    const float total = sum112(temp, n, sh);
    if (total > 0.0f) {
#pragma unroll
        for (int j = 0; j < PER; j++) v[j] /= total;
    }

    if (top_p > 0.0f && top_p < 1.0f) {
        if (fast) {
            if (tid == 0) {
                float cum = 0.0f, cut = -1e30f;
                for (int j = K - 1; j >= 0; j--) {
                    // the candidate's probability: its logit key -> exp(l - m) / total, as above
                    float p = expf(fkey_inv(sh.ckey[j]) - m);
                    if (total > 0.0f) p /= total;
                    sh.cval[j] = p;
                    cum += p;
                    cut = p;
                    if (cum >= top_p) break;
                }
                sh.cutoff = cut;
            }
        } else {
            const int R = n < kCand ? n : kCand;
#pragma unroll
            for (int j = 0; j < PER; j++) kr[j] = fkey(v[j]);
            top_r_keys<PER>(kr, lo, cnt, R, sh);
#pragma unroll
            for (int j = 0; j < PER; j++) v[j] = fkey_inv(kr[j]);
            for (int c = tid; c < R; c += kSampBS) sh.cval[c] = fkey_inv(sh.ckey[c]);
            __syncthreads();
            if (tid == 0) {
                float cum = 0.0f, cut = 0.0f;
                for (int c0 = 0; c0 < R && cum < top_p; c0 += 16) {
                    float pv[16];
#pragma unroll
                    for (int e = 0; e < 16; e++) pv[e] = sh.cval[c0 + e];
#pragma unroll
                    for (int e = 0; e < 16; e++) {
                        if (c0 + e < R && cum < top_p) {
                            cum += pv[e];
                            cut = pv[e];
                        }
                    }
                }
                sh.cutoff = cut;
            }
        }
        __syncthreads();
        const float cut = sh.cutoff;
#pragma unroll
        for (int j = 0; j < PER; j++)
            if (v[j] < cut) v[j] = 0.0f;
    }

    if (fast) {
        if (tid == 0) {
            // the top-K list in its order from the K-th candidate up, with the
            // cut applied to each probability (recomputed as above)
            const float cut = (top_p > 0.0f && top_p < 1.0f) ? sh.cutoff : -1e30f;
            float tot = 0.0f;
            for (int j = K - 1; j >= 0; j--) {
                float p = expf(fkey_inv(sh.ckey[j]) - m);
                if (total > 0.0f) p /= total;
                if (p < cut) p = 0.0f;
                sh.cval[j] = p;
                if (p > 0.0f) tot += p;
            }
            const float u = u01_dev(seed) * tot;
            float acc = 0.0f;
            int chosen = sh.cidx[K - 1];
            for (int j = K - 1; j >= 0; j--) {
                const float p = sh.cval[j];
                if (p > 0.0f) {
                    acc += p;
                    if (acc > u) { chosen = sh.cidx[j]; break; }
                }
            }
            token[b] = (uint32_t)chosen;
        }
        return;
    }
    // CDF draw in index order (as k_sample): the sum in the 112-lane order,
    // then the compacted non-zero entries (or, past 512 of them, the row)
    __syncthreads();
    store_row();
    const float tot = sum112(temp, n, sh);
    uint32_t nz = 0;
#pragma unroll
    for (int j = 0; j < PER; j++) nz += v[j] != 0.0f;
    sh.cnt_gt[tid] = nz;
    const uint32_t NZ = block_exscan(sh.cnt_gt, sh);
    const bool compact = NZ <= (uint32_t)kCand;
    if (compact) {
        uint32_t o = sh.cnt_gt[tid];
#pragma unroll
        for (int j = 0; j < PER; j++)
            if (v[j] != 0.0f) { sh.cidx[o] = lo + j; sh.cval[o] = v[j]; o++; }
    }
    __syncthreads();
    if (tid == 0) {
        const float u = u01_dev(seed) * tot;
        float acc = 0.0f;
        int chosen = n - 1;
        if (compact) {
            bool found = false;
            for (uint32_t j0 = 0; j0 < NZ && !found; j0 += 16) {
                float pv[16];
#pragma unroll
                for (int e = 0; e < 16; e++) pv[e] = sh.cval[j0 + e];
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    if (!found && j0 + e < NZ) {
                        acc += pv[e];
                        if (acc > u) { chosen = sh.cidx[j0 + e]; found = true; }
                    }
                }
            }
        } else {
            bool found = false;
            for (int i0 = 0; i0 < n && !found; i0 += 16) {
                float pv[16];
#pragma unroll
                for (int e = 0; e < 16; e++) pv[e] = i0 + e < n ? temp[i0 + e] : 0.0f;
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    if (!found && i0 + e < n) {
                        acc += pv[e];
                        if (acc > u) { chosen = i0 + e; found = true; }
                    }
                }
            }
        }
        token[b] = (uint32_t)chosen;
    }
}

__global__ __launch_bounds__(kSampBS) void k_sample(const float *__restrict__ logits, uint32_t *__restrict__ token,
                                                    int n, float *__restrict__ temp_all,
                                                    uint32_t *__restrict__ counter_all,
                                                    const float *__restrict__ sampler,
                                                    const uint32_t *__restrict__ hist_all, int hist_stride) {
    __shared__ SampShared sh;
    sample_row_general(blockIdx.x, logits, token, n, temp_all, counter_all, sampler, hist_all, hist_stride, sh);
}

template <int PER>
__global__ __launch_bounds__(kSampBS) void k_sample_regs(const float *__restrict__ logits, uint32_t *__restrict__ token,
                                                         int n, float *__restrict__ temp_all,
                                                         uint32_t *__restrict__ counter_all,
                                                         const float *__restrict__ sampler,
                                                         const uint32_t *__restrict__ hist_all, int hist_stride) {
    __shared__ SampShared sh;
    sample_row_regs<PER>(blockIdx.x, logits, token, n, temp_all, counter_all, sampler, hist_all, hist_stride, sh);
}

// ------------------------------------------------ multi-CU top-p sampling
// The configs' serving case (no top-k, 0 < top_p < 1) spread over the chip,
// in three launches per batch of rows; the draws are the ones the
// one-block pipeline makes (the same operations in the same order):
//   k_samp_scale (n/1024 blocks per row): penalties, 1/T -> temp; block maxima;
//   k_samp_exp   (n/1024 blocks per row): m = the row maximum, e = exp(l - m)
//                -> temp; a 4096-bin histogram of the keys of e (their top
//                12 bits) in global memory;
//   k_samp_pick  (one block per row): the bin holding the 512-th largest e;
//                one pass over e that takes the softmax total in the
//                112-lane order (backend_cuda.rs:3880-3921) and gathers the
//                elements of that bin and above (and the bin below, which
//                holds any element whose probability can round to a tie
//                with the 512-th); p = e / total for those only; the 512
//                largest p by radix select + rank sort, the sequential top-p
//                accumulation, the kept set in index order, its 112-lane sum
//                (zero entries add nothing) and the CDF draw.
// A row outside this case (top-k, top_p outside (0, 1)), or with more than
// kPickMax gathered candidates, runs the one-block pipeline from its logits
// inside k_samp_pick.
constexpr int kPickMax = 4096;
constexpr int kSampHistBins = 4096;
constexpr int kSampMinN = kSampHistBins + 64 + 1024;  // rows long enough for the work words carved below

// per-row work words inside `counter_all` (n u32 per row): block maxima [64..], histogram [4096]
__device__ __forceinline__ uint32_t *samp_hist(uint32_t *counter_all, int b, int n) { return counter_all + (size_t)b * n; }
__device__ __forceinline__ float *samp_pmax(uint32_t *counter_all, int b, int n) {
    return (float *)(counter_all + (size_t)b * n + kSampHistBins);
}

__device__ __forceinline__ bool samp_multi_case(const float *sp, int n) {
    const uint32_t top_k = __float_as_uint(sp[1]);
    const float top_p = sp[2];
    return (top_k == 0u || top_k >= (uint32_t)n) && top_p > 0.0f && top_p < 1.0f;
}

__global__ __launch_bounds__(1024) void k_samp_scale(const float *__restrict__ logits, int n, float *__restrict__ temp_all,
                                                     uint32_t *__restrict__ counter_all,
                                                     const float *__restrict__ sampler,
                                                     const uint32_t *__restrict__ hist_all, int hist_stride) {
    __shared__ uint32_t cnt[1024];
    __shared__ float red[16];
    const int b = blockIdx.y, blk = blockIdx.x, tid = threadIdx.x;
    const float *sp = sampler + (size_t)b * 8;
    if (!samp_multi_case(sp, n)) return;
    const int base = blk * 1024, i = base + tid;
    const float temperature = sp[0];
    const float rep = sp[4], freq = sp[5], pres = sp[6];
    const uint32_t hist_len = min(__float_as_uint(sp[7]), (uint32_t)max(hist_stride, 0));
    float l = i < n ? logits[(size_t)b * n + i] : -1e30f;
    if (blk == 0) {  // the row's histogram, filled by the next launch
        uint32_t *h = samp_hist(counter_all, b, n);
        for (int q = tid; q < kSampHistBins; q += 1024) h[q] = 0u;
    }
    if (hist_len > 0u && hist_all && (rep != 1.0f || freq != 0.0f || pres != 0.0f)) {
        // occurrences of this block's tokens in the history (the counter of backend_cuda.rs:3700-3720)
        cnt[tid] = 0u;
        __syncthreads();
        const uint32_t *hist = hist_all + (size_t)b * hist_stride;
        for (uint32_t h = tid; h < hist_len; h += 1024) {
            const uint32_t tk = hist[h];
            if (tk >= (uint32_t)base && tk < (uint32_t)min(n, base + 1024)) atomicAdd(&cnt[tk - base], 1u);
        }
        __syncthreads();
        const uint32_t c = cnt[tid];
        if (c > 0u) {
            if (rep != 1.0f) l = l > 0.0f ? l / rep : l * rep;
            if (pres != 0.0f) l -= pres;
        }
        if (freq != 0.0f) l -= freq * (float)c;
    }
    float invT = 1.0f / temperature;
    if (!(temperature > 0.0f)) invT = 1.0f;
    l *= invT;
    if (i < n) temp_all[(size_t)b * n + i] = l;
    float m = wave_max_last(i < n ? l : -1e30f);
    if ((tid & 63) == 63) red[tid >> 6] = m;
    __syncthreads();
    if (tid == 0) {
        float mm = red[0];
        for (int w = 1; w < 16; w++) mm = fmaxf(mm, red[w]);
        samp_pmax(counter_all, b, n)[blk] = mm;
    }
}

__global__ __launch_bounds__(1024) void k_samp_exp(int n, float *__restrict__ temp_all, uint32_t *__restrict__ counter_all,
                                                   const float *__restrict__ sampler) {
    __shared__ uint32_t hb[kSampHistBins];
    __shared__ float mrow;
    const int b = blockIdx.y, blk = blockIdx.x, tid = threadIdx.x, nb = gridDim.x;
    if (!samp_multi_case(sampler + (size_t)b * 8, n)) return;
    for (int q = tid; q < kSampHistBins; q += 1024) hb[q] = 0u;
    if (tid < 64) {
        const float *pm = samp_pmax(counter_all, b, n);
        float m = -1e30f;
        for (int q = tid; q < nb; q += 64) m = fmaxf(m, pm[q]);
        m = wave_max_last(m);
        if (tid == 63) mrow = m;
    }
    __syncthreads();
    const int i = blk * 1024 + tid;
    if (i < n) {
        float *t = temp_all + (size_t)b * n;
        const float e = expf(t[i] - mrow);
        t[i] = e;
        atomicAdd(&hb[fkey(e) >> 20], 1u);
    }
    __syncthreads();
    uint32_t *h = samp_hist(counter_all, b, n);
    for (int q = tid; q < kSampHistBins; q += 1024)
        if (hb[q]) atomicAdd(&h[q], hb[q]);
}

struct PickShared {
    union {
        float chunk[16384];  // one streamed piece of e
        SampShared sh;       // the radix select / fallback pipeline
        struct {
            uint32_t bits[8192];  // kept-set bitmap (rows up to 262,144)
            uint32_t wpre[8192];  // kept entries before each word
        } bm;
    };
    uint64_t comp[kCand];    // the R largest: key << 32 | ~index
    float psort[kCand];      // their p, sorted (p desc, index asc)
    uint32_t sh_scan[1024];
    double dred[1024];
    uint32_t lcnt[112], loff[112], lcur[112];
    double dtot;
    int flat, chosen, cutok;
    float ce[kPickMax];      // gathered candidates: e, then p; at the end the kept set in index order
    int ci[kPickMax];
    union {
        uint32_t fh[8192];   // fine histogram of the boundary bins
        struct {
            float kp[kPickMax];  // the kept set (p >= cut) as found
            int ki[kPickMax];
        };
    };
    float part[112];
    uint32_t bsum[1024];
    uint32_t ncand, ndef, ngt, neq, nsel, nkeep, bin;
    int overflow;
    float total, cut, tot2;
};

template <int PER>
__global__ __launch_bounds__(1024) void k_samp_pick(const float *__restrict__ logits, uint32_t *__restrict__ token,
                                                    int n, float *__restrict__ temp_all,
                                                    uint32_t *__restrict__ counter_all,
                                                    const float *__restrict__ sampler,
                                                    const uint32_t *__restrict__ hist_all, int hist_stride) {
    __shared__ PickShared ps;
    const int b = blockIdx.x, tid = threadIdx.x;
    const float *sp = sampler + (size_t)b * 8;
    auto fallback = [&]() {
        if constexpr (PER > 0)
            sample_row_regs<PER>(b, logits, token, n, temp_all, counter_all, sampler, hist_all, hist_stride, ps.sh);
        else
            sample_row_general(b, logits, token, n, temp_all, counter_all, sampler, hist_all, hist_stride, ps.sh);
    };
    if (!samp_multi_case(sp, n)) {
        fallback();
        return;
    }
    const float top_p = sp[2];
    const uint32_t seed = __float_as_uint(sp[3]);
    const int R = n < kCand ? n : kCand;
    const float *e_row = temp_all + (size_t)b * n;
    // 1. the bin of the R-th largest key: bins from the top, 4 per thread
    {
        const uint32_t *h = samp_hist(counter_all, b, n);
        const int q0 = kSampHistBins - 4 - 4 * tid;  // thread 0 holds the top bins
        uint32_t hv[4], s = 0;
#pragma unroll
        for (int e = 0; e < 4; e++) { hv[e] = h[q0 + e]; s += hv[e]; }
        ps.sh.cnt_gt[tid] = s;
        __syncthreads();
        block_exscan(ps.sh.cnt_gt, ps.sh);
        uint32_t above = ps.sh.cnt_gt[tid];
#pragma unroll
        for (int e = 3; e >= 0; e--) {
            if (above < (uint32_t)R && above + hv[e] >= (uint32_t)R) ps.bin = (uint32_t)(q0 + e);
            above += hv[e];
        }
        if (tid == 0) { ps.ncand = 0u; ps.ndef = 0u; ps.overflow = 0; }
        __syncthreads();
    }
    // 2. pass 1 over e: the 112-lane sums, the elements of the bins above
    // the boundary (fewer than R: all of them are taken), and a histogram of
    // the next 12 key bits of the elements in the boundary bin and the one
    // below it.  Waves 0-1 form the sums (lane t < 112 adds e[t], e[t+112],
    // ... in that order) straight from global memory with 32 loads in flight
    // per lane, while the other 14 waves gather and count: the sums are a
    // dependent chain of n/112 adds, which staged through LDS pieces with the
    // other waves waiting at barriers took most of this kernel's time
    const uint32_t bin = ps.bin, lowbin = bin > 0u ? bin - 1u : 0u;
    const float elo = lowbin > 0u ? fkey_inv(lowbin << 20) : -1.0f;  // the smallest value of bin lowbin
    for (int q = tid; q < 8192; q += 1024) ps.fh[q] = 0u;
    __syncthreads();
    auto take = [&](float ev, int i) {
        const uint32_t slot = atomicAdd(&ps.ncand, 1u);
        if (slot < (uint32_t)kPickMax) { ps.ce[slot] = ev; ps.ci[slot] = i; }
    };
    if (tid < 128) {
        if (PER > 0 && tid < 112) {
            // n = PER * kSampBS is known here: the chain is unrolled whole, so
            // that the load of element j + D goes out right after the add of
            // element j with an exact wait for each add (a loop's back edge
            // makes the compiler wait for every load in flight at its head)
            constexpr int NN = PER * kSampBS, NJ0 = NN / 112, D = 32;
            const float *er = e_row + tid;
            float r[D];
#pragma unroll
            for (int k = 0; k < D; k++) r[k] = er[112 * k];
            float s112 = 0.0f;
#pragma unroll
            for (int j = 0; j < NJ0; j++) {
                s112 += r[j % D];
                if (j + D < NJ0) r[j % D] = er[112 * (j + D)];
            }
            if (tid < NN - 112 * NJ0) s112 += er[112 * NJ0];
            ps.part[tid] = s112;
        } else if (tid < 112) {
            constexpr int D = 32;
            const int nj = (n - tid + 111) / 112;  // this lane's elements: tid + 112 j < n
            const float *er = e_row + tid;
            float r[D];
#pragma unroll
            for (int k = 0; k < D; k++) r[k] = k < nj ? er[112 * k] : 0.0f;
            float s112 = 0.0f;
            int j = 0;
            // (unconditional refills while two windows remain: a conditional
            // load per element becomes a branch, and the waits at the joins
            // drain the loads in flight)
            for (; j + 2 * D <= nj; j += D) {
#pragma unroll
                for (int k = 0; k < D; k++) {
                    s112 += r[k];
                    r[k] = er[(size_t)112 * (j + D + k)];
                }
            }
#pragma unroll
            for (int k = 0; k < D; k++)
                if (j + k < nj) s112 += r[k];
            for (int jj = j + D; jj < nj; jj++) s112 += er[(size_t)112 * jj];
            ps.part[tid] = s112;
        }
    } else if (PER > 0) {
        // the loads of 8 float4 per lane go out before any is used (a loop
        // with one load per trip waits for it at every trip's head)
        constexpr int NN = PER * kSampBS, ITS = (NN + 4 * 896 - 1) / (4 * 896), BT = 8;
#pragma unroll
        for (int i0 = 0; i0 < ITS; i0 += BT) {
            float4 cv[BT];
#pragma unroll
            for (int u = 0; u < BT; u++) {
                const int i = 4 * (tid - 128) + (i0 + u) * 4 * 896;
                cv[u] = i0 + u < ITS && i < NN ? *(const float4 *)(e_row + i) : make_float4(-1.0f, -1.0f, -1.0f, -1.0f);
            }
#pragma unroll
            for (int u = 0; u < BT; u++) {
                const int i = 4 * (tid - 128) + (i0 + u) * 4 * 896;
                const float4 c = cv[u];
                if (i0 + u >= ITS || i >= NN) continue;
                if (fmaxf(fmaxf(c.x, c.y), fmaxf(c.z, c.w)) < elo) continue;
                const float ev[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const uint32_t kk = fkey(ev[e]), cb = kk >> 20;
                    if (cb < lowbin) continue;
                    take(ev[e], i + e);
                    if (cb > bin) atomicAdd(&ps.ndef, 1u);
                    else atomicAdd(&ps.fh[((cb - lowbin) << 12) | ((kk >> 8) & 0xFFFu)], 1u);
                }
            }
        }
    } else {
        for (int i = 4 * (tid - 128); i < n; i += 4 * 896) {
            float4 c;
            if (i + 3 < n) {
                c = *(const float4 *)(e_row + i);
            } else {
                c.x = e_row[i];
                c.y = i + 1 < n ? e_row[i + 1] : 0.0f;
                c.z = i + 2 < n ? e_row[i + 2] : 0.0f;
                c.w = i + 3 < n ? e_row[i + 3] : 0.0f;
            }
            // e >= 0, so key order is float order: one compare rejects the
            // elements below the candidate bins (most of the row)
            if (fmaxf(fmaxf(c.x, c.y), fmaxf(c.z, c.w)) < elo) continue;
            const float ev[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const uint32_t kk = fkey(ev[e]), cb = kk >> 20;
                if (i + e >= n || cb < lowbin) continue;
                take(ev[e], i + e);
                if (cb > bin) atomicAdd(&ps.ndef, 1u);
                else atomicAdd(&ps.fh[((cb - lowbin) << 12) | ((kk >> 8) & 0xFFFu)], 1u);
            }
        }
    }
    __syncthreads();
    if (tid == 0) {
        for (int q = 0; q < 48; q++) ps.part[q] += ps.part[q + 64];
        for (int step = 32; step > 0; step >>= 1)
            for (int q = 0; q < step; q++) ps.part[q] += ps.part[q + step];
        ps.total = ps.part[0];
    }
    // 3. the fine bin of the R-th largest: R - (taken so far) from the top of
    // the 8192 fine bins, 8 per thread
    {
        const uint32_t need = (uint32_t)R - ps.ndef;
        const int q0 = 8192 - 8 - 8 * tid;
        uint32_t hv[8], s = 0;
#pragma unroll
        for (int e = 0; e < 8; e++) { hv[e] = ps.fh[q0 + e]; s += hv[e]; }
        ps.sh.cnt_gt[tid] = s;
        __syncthreads();
        block_exscan(ps.sh.cnt_gt, ps.sh);
        uint32_t above = ps.sh.cnt_gt[tid];
#pragma unroll
        for (int e = 7; e >= 0; e--) {
            if (above < need && above + hv[e] >= need) ps.bin = (uint32_t)(q0 + e);
            above += hv[e];
        }
        __syncthreads();
    }
    // 4. the candidates: the elements above the boundary bin and those of
    // the fine bin of the R-th largest and above (and of the fine bin below,
    // which holds any element whose probability can round to a tie with the
    // R-th).  Pass 1 gathered both boundary bins whole: pruned in place when
    // they fit, else gathered again by a second pass over e.
    const uint32_t k24lo = (lowbin << 12) + (ps.bin > 0u ? ps.bin - 1u : 0u), k24hi = ((bin + 1u) << 12);
    auto wanted = [&](float ev) {
        const uint32_t kk = fkey(ev);
        return (kk >> 20) > bin || ((kk >> 8) >= k24lo && (kk >> 8) < k24hi);
    };
    if (ps.ncand <= (uint32_t)kPickMax) {
        constexpr int KPT = kPickMax / 1024;
        const int C0 = (int)ps.ncand;
        float pe[KPT];
        int pi[KPT];
#pragma unroll
        for (int m = 0; m < KPT; m++) {
            const int c = tid + 1024 * m;
            pe[m] = c < C0 ? ps.ce[c] : 0.0f;
            pi[m] = c < C0 ? ps.ci[c] : -1;
        }
        __syncthreads();
        if (tid == 0) ps.ncand = 0u;
        __syncthreads();
#pragma unroll
        for (int m = 0; m < KPT; m++)
            if (pi[m] >= 0 && wanted(pe[m])) take(pe[m], pi[m]);
    } else {
        __syncthreads();
        if (tid == 0) ps.ncand = 0u;
        __syncthreads();
        for (int i = 4 * tid; i < n; i += 4 * 1024) {
            float4 c;
            if (i + 3 < n) {
                c = *(const float4 *)(e_row + i);
            } else {
                c.x = e_row[i];
                c.y = i + 1 < n ? e_row[i + 1] : 0.0f;
                c.z = i + 2 < n ? e_row[i + 2] : 0.0f;
                c.w = i + 3 < n ? e_row[i + 3] : 0.0f;
            }
            const float ev[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
            for (int e = 0; e < 4; e++)
                if (i + e < n && wanted(ev[e])) take(ev[e], i + e);
        }
    }
    __syncthreads();
    if (tid == 0) ps.overflow = ps.ncand > (uint32_t)kPickMax;
    __syncthreads();
    if (ps.overflow) {
        fallback();
        return;
    }
    const float total = ps.total;
    const int C = (int)ps.ncand;
    // 3. p of the candidates and the key of the R-th largest (radix select)
    for (int c = tid; c < C; c += 1024) {
        float p = ps.ce[c];
        if (total > 0.0f) p /= total;
        ps.ce[c] = p;
    }
    __syncthreads();
    uint32_t prefix = 0, mask = 0, remaining = (uint32_t)R;
    for (int pass = 0; pass < 4; pass++) {
        const int shift = 24 - 8 * pass;
        radix_clear(ps.sh);
        for (int c0 = 0; c0 < C; c0 += 1024) {
            const int c = c0 + tid;
            const uint32_t kk = c < C ? fkey(ps.ce[c]) : 0u;
            radix_count(kk, c < C && (kk & mask) == prefix, shift, pass == 0, ps.sh);
        }
        radix_pick(remaining, ps.sh);
        prefix |= ps.sh.sel_bin << shift;
        mask |= 255u << shift;
        remaining = ps.sh.sel_rem;
        __syncthreads();
    }
    const uint32_t kthr = prefix;
    // 4. top-p's cut.  The sum of the R largest p in double (the ties at
    // the threshold all have its p): when it is below top_p by more than the
    // sequential fp32 rounding can move it, the sequential pass over the
    // sorted list never stops early and its cut is the R-th largest p, with
    // no sort.  Otherwise the R largest are sorted (composite keys key << 32
    // | ~index, ranked) and the pass runs as written.
    {
        double ds = 0.0;
        uint32_t g = 0;
        for (int c = tid; c < C; c += 1024) {
            const uint32_t kk = fkey(ps.ce[c]);
            if (kk > kthr) { ds += (double)ps.ce[c]; g++; }
        }
        ps.dred[tid] = ds;
        ps.sh_scan[tid] = g;
        __syncthreads();
        if (tid < 64) {
            double t = 0.0;
            uint32_t gg = 0;
            for (int q = tid; q < 1024; q += 64) { t += ps.dred[q]; gg += ps.sh_scan[q]; }
            for (int d = 32; d > 0; d >>= 1) {
                t += __shfl_xor(t, d);
                gg += __shfl_xor(gg, d);
            }
            if (tid == 0) {
                const double pr = (double)fkey_inv(kthr);
                ps.dtot = t + (double)(R - (int)gg) * pr;
                ps.flat = ps.dtot < (double)top_p - 1e-4;
                ps.cut = fkey_inv(kthr);
            }
        }
        __syncthreads();
    }
    if (!ps.flat) {
        if (tid == 0) { ps.ngt = 0u; ps.neq = 0u; ps.nsel = 0u; }
        __syncthreads();
        for (int c = tid; c < C; c += 1024) {
            const uint32_t kk = fkey(ps.ce[c]);
            if (kk > kthr) ps.comp[atomicAdd(&ps.ngt, 1u)] = ((uint64_t)kk << 32) | (uint32_t)~ps.ci[c];
            else if (kk == kthr) ps.ki[atomicAdd(&ps.neq, 1u)] = ps.ci[c];
        }
        __syncthreads();
        {
            const int G = (int)ps.ngt, T = (int)ps.neq, take = R - G;
            for (int t = tid; t < T; t += 1024) {
                const int ii = ps.ki[t];
                int before = 0;  // ties with a smaller index
                if (take < T)
                    for (int j = 0; j < T; j++) before += ps.ki[j] < ii;
                if (before < take) ps.comp[G + atomicAdd(&ps.nsel, 1u)] = ((uint64_t)kthr << 32) | (uint32_t)~ii;
            }
        }
        __syncthreads();
        // sorted order: bitonic sort of the R keys (key desc, index asc) in
        // the pipeline's candidate area, free once the radix select is done
        // (a rank count over all keys per thread cost 15-24 us per row)
        for (int r = tid; r < kCand; r += 1024) {
            const uint64_t cv = r < R ? ps.comp[r] : 0ull;
            ps.sh.ckey[r] = r < R ? (uint32_t)(cv >> 32) : 0u;
            ps.sh.cidx[r] = r < R ? (int)~(uint32_t)cv : 0x7FFFFFFF;
        }
        __syncthreads();
        cand_sort(ps.sh);
        for (int r = tid; r < R; r += 1024) ps.psort[r] = fkey_inv(ps.sh.ckey[r]);
        __syncthreads();
        // The sequential fp32 pass adds entry q while the sum of entries
        // 0..q-1 is below top_p and cuts at the last one added.  Its sums
        // differ from the exact ones by at most (q+1) 2^-24 of them, so where
        // the double prefix sums clear top_p by (q+2) 2^-23 max(sum, top_p)
        // on both sides of their crossing, the pass stops at that crossing
        // too; otherwise it runs below as written
        {
            // inclusive double prefix: a scan per wave, then the waves' totals
            double v = tid < R ? (double)ps.psort[tid] : 0.0;
            const int ln = tid & 63;
#pragma unroll
            for (int d = 1; d < 64; d <<= 1) {
                const double t = __shfl_up(v, d);
                if (ln >= d) v += t;
            }
            if (ln == 63) ps.dred[1008 + (tid >> 6)] = v;
            if (tid == 0) ps.cutok = 0;
            __syncthreads();
            double off = 0.0;
            for (int w = 0; w < (tid >> 6); w++) off += ps.dred[1008 + w];
            __syncthreads();
            ps.dred[tid] = v + off;
            __syncthreads();
        }
        if (tid < R) {
            const double tp = (double)top_p, c = ps.dred[tid], cp = tid ? ps.dred[tid - 1] : 0.0;
            const double mc = (tid + 2) * 0x1p-23 * fmax(c, tp), mp = (tid + 1) * 0x1p-23 * fmax(cp, tp);
            if (c >= tp && cp < tp && c >= tp + mc && (tid == 0 || cp < tp - mp)) {
                ps.cut = ps.psort[tid];
                ps.cutok = 1;
            }
            if (tid == R - 1 && c < tp - mc) {
                ps.cut = ps.psort[R - 1];
                ps.cutok = 1;
            }
        }
        __syncthreads();
        // otherwise the sequential pass itself, on one lane (16 values read
        // per batch, then added in order)
        if (!ps.cutok && tid == 0) {
            float cum = 0.0f, cut = 0.0f;
            for (int q0 = 0; q0 < R; q0 += 16) {
                float v[16];
#pragma unroll
                for (int e = 0; e < 16; e++) v[e] = q0 + e < R ? ps.psort[q0 + e] : 0.0f;
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    const bool go = q0 + e < R && cum < top_p;
                    cut = go ? v[e] : cut;
                    cum = go ? cum + v[e] : cum;
                }
            }
            ps.cut = cut;
        }
    }
    // 6. the kept entries (p >= cut; every one is a candidate) in index
    // order: a bitmap over the row, word prefix counts, each entry's place
    const int NWD = (n + 31) / 32;
    for (int w = tid; w < NWD; w += 1024) ps.bm.bits[w] = 0u;
    __syncthreads();
    const float cut = ps.cut;
    for (int c = tid; c < C; c += 1024)
        if (ps.ce[c] >= cut) atomicOr(&ps.bm.bits[ps.ci[c] >> 5], 1u << (ps.ci[c] & 31));
    __syncthreads();
    {
        const int per = (NWD + 1023) / 1024, w0 = tid * per;
        uint32_t s = 0;
        for (int w = w0; w < min(NWD, w0 + per); w++) s += __popc(ps.bm.bits[w]);
        ps.sh_scan[tid] = s;
        __syncthreads();
        if (tid < 64) {
            // exclusive scan of the 1024 thread sums on one wave, 16 per lane
            uint32_t v[16], t = 0;
#pragma unroll
            for (int e = 0; e < 16; e++) { v[e] = ps.sh_scan[16 * tid + e]; t += v[e]; }
            uint32_t x = t;
#pragma unroll
            for (int d = 1; d < 64; d <<= 1) {
                const uint32_t y = __shfl_up(x, d);
                if (tid >= d) x += y;
            }
            uint32_t off = x - t;
#pragma unroll
            for (int e = 0; e < 16; e++) { ps.sh_scan[16 * tid + e] = off; off += v[e]; }
            if (tid == 63) ps.nkeep = x;
        }
        __syncthreads();
        uint32_t o = ps.sh_scan[tid];
        for (int w = w0; w < min(NWD, w0 + per); w++) {
            ps.bm.wpre[w] = o;
            o += __popc(ps.bm.bits[w]);
        }
    }
    __syncthreads();
    for (int c = tid; c < C; c += 1024) {
        const float p = ps.ce[c];
        if (p >= cut) {
            const int i = ps.ci[c];
            const uint32_t pos = ps.bm.wpre[i >> 5] + __popc(ps.bm.bits[i >> 5] & ((1u << (i & 31)) - 1u));
            ps.kp[pos] = p;
            ps.ki[pos] = i;
        }
    }
    if (tid < 112) ps.lcnt[tid] = 0u;
    __syncthreads();
    const int NK = (int)ps.nkeep;
    // 7. the kept probabilities' sum in the 112-lane order: lane t adds the
    // kept entries of index = t mod 112 in ascending index.  The entries go
    // into per-lane lists (counting sort by lane; each list then sorted by
    // its few indices), then each lane adds its list in order.
    for (int j = tid; j < NK; j += 1024) atomicAdd(&ps.lcnt[ps.ki[j] % 112], 1u);
    __syncthreads();
    if (tid == 0) {
        uint32_t o = 0;
        for (int l = 0; l < 112; l++) { ps.loff[l] = o; ps.lcur[l] = o; o += ps.lcnt[l]; }
    }
    __syncthreads();
    uint32_t *lidx = ps.bm.wpre;  // free again after the scatter
    for (int j = tid; j < NK; j += 1024) lidx[atomicAdd(&ps.lcur[ps.ki[j] % 112], 1u)] = (uint32_t)j;
    __syncthreads();
    if (tid < 112) {
        const int o = (int)ps.loff[tid], cnt = (int)ps.lcnt[tid];
        for (int a2 = 1; a2 < cnt; a2++) {  // insertion sort of the lane's list by position (= index order)
            const uint32_t v = lidx[o + a2];
            int q = a2 - 1;
            while (q >= 0 && lidx[o + q] > v) { lidx[o + q + 1] = lidx[o + q]; q--; }
            lidx[o + q + 1] = v;
        }
        float s = 0.0f;
        for (int q = 0; q < cnt; q++) s += ps.kp[lidx[o + q]];
        ps.part[tid] = s;
    }
    __syncthreads();
    if (tid == 0) {
        for (int q = 0; q < 48; q++) ps.part[q] += ps.part[q + 64];
        for (int step = 32; step > 0; step >>= 1)
            for (int q = 0; q < step; q++) ps.part[q] += ps.part[q + step];
        ps.tot2 = ps.part[0];
        ps.chosen = -1;
    }
    __syncthreads();
    // 8. the CDF draw: the first kept entry (index order) whose sequential
    // fp32 running sum exceeds u.  Exact prefix sums (double, in parallel)
    // place the crossing; when u is further from both neighbouring prefix
    // sums than the sequential fp32 sum can stray (each prefix within
    // NK * 2^-24 of the total), the sequential crossing is that entry.
    // Otherwise the sequential scan runs as written.
    const float u = u01_dev(seed) * ps.tot2;
    {
        double *dpre = (double *)ps.bm.bits;  // 4096 doubles (bits is free)
        const int per = (NK + 1023) / 1024, j0 = tid * per, j1 = min(NK, j0 + per);
        double loc = 0.0;
        for (int j = j0; j < j1; j++) loc += (double)ps.kp[j];
        ps.dred[tid] = loc;
        __syncthreads();
        if (tid < 64) {
            double v[16], t = 0.0;
#pragma unroll
            for (int e = 0; e < 16; e++) { v[e] = ps.dred[16 * tid + e]; t += v[e]; }
            double x = t;
#pragma unroll
            for (int d = 1; d < 64; d <<= 1) {
                const double y = __shfl_up(x, d);
                if (tid >= d) x += y;
            }
            double off = x - t;
#pragma unroll
            for (int e = 0; e < 16; e++) { ps.dred[16 * tid + e] = off; off += v[e]; }
        }
        __syncthreads();
        double run = ps.dred[tid];
        for (int j = j0; j < j1; j++) { run += (double)ps.kp[j]; dpre[j] = run; }
        __syncthreads();
        const double bound = (double)(NK + 2) * 1.1920928955078125e-07 * (double)fmaxf(ps.tot2, u) + 1e-30;
        for (int j = j0; j < j1; j++) {
            const double prev = j > 0 ? dpre[j - 1] : 0.0;
            if (dpre[j] > (double)u && prev <= (double)u)
                ps.chosen = (dpre[j] - (double)u > bound && (double)u - prev > bound) ? j : -2;
        }
        if (tid == 0 && NK > 0 && dpre[NK - 1] <= (double)u)
            ps.chosen = (double)u - dpre[NK - 1] > bound ? NK : -2;  // no crossing: the default token
        __syncthreads();
    }
    if (ps.chosen >= 0) {
        if (tid == 0) token[b] = ps.chosen < NK ? (uint32_t)ps.ki[ps.chosen] : (uint32_t)(n - 1);
        return;
    }
    if (tid < 64) {
        float acc = 0.0f;
        int chosen = n - 1;
        bool found = false;
        for (int j0 = 0; j0 < NK && !found; j0 += 64) {
            const float pv = j0 + tid < NK ? ps.kp[j0 + tid] : 0.0f;
            const int cnt = min(64, NK - j0);
            for (int q = 0; q < cnt; q++) {
                acc += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pv), q));
                if (acc > u) {
                    chosen = ps.ki[j0 + q];
                    found = true;
                    break;
                }
            }
        }
        if (tid == 0) token[b] = (uint32_t)chosen;
    }
}

// ------------------------------------------------ allocation-free sampling
// Work area of rsv_sample_noalloc: temp [n] f32, counter [n] u32 and one
// sampler row [8], for n up to kNoAllocMaxN.  One copy per device, held
// until the process ends.  Host code never passes `scratch` itself to a
// kernel (on the host the name is not a device address): each device's
// address comes from hipGetSymbolAddress, taken once per device with that
// device current, and only that address is used.
static __device__ __align__(256) uint32_t scratch[kNoAllocWords];

static std::mutex g_scratch_mu;
static void *g_scratch_ptr[kMaxDevices];

int sample_scratch_init(int device) {
    if (device < 0 || device >= kMaxDevices) return RSV_FAIL("sample scratch: device %d out of range", device);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch_ptr[device]) return 0;
    int cur = -1;
    RSV_HIP(hipGetDevice(&cur));
    if (cur != device) return RSV_FAIL("sample scratch: device %d is not current (%d is)", device, cur);
    void *p = nullptr;
    RSV_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) return RSV_FAIL("sample scratch: no device address");
    g_scratch_ptr[device] = p;
    return 0;
}

uint32_t *sample_scratch(int device) {
    if (device < 0 || device >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    return (uint32_t *)g_scratch_ptr[device];
}

// One context per device may use the work area: the first to call
// rsv_sample_noalloc owns it until it is destroyed, and calls from any other
// context on that device are refused (their streams could overlap).
static const void *g_scratch_owner[kMaxDevices];

int sample_scratch_claim(int device, const void *ctx) {
    if (device < 0 || device >= kMaxDevices) return RSV_FAIL("sample scratch: device %d out of range", device);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_owner[device]) g_scratch_owner[device] = ctx;
    if (g_scratch_owner[device] != ctx)
        return RSV_FAIL("sample_noalloc: the work area of device %d belongs to another context (one context per "
                        "device may use it, until that context is destroyed)", device);
    return 0;
}

void sample_scratch_release(int device, const void *ctx) {
    if (device < 0 || device >= kMaxDevices) return;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch_owner[device] == ctx) g_scratch_owner[device] = nullptr;
}

int launch_sample(rsv_ctx *ctx, const float *logits, uint32_t *token, int n, float *temp, uint32_t *counter,
                  const float *sampler, const uint32_t *hist, int hist_stride, int batch) {
    if (n <= 0 || batch <= 0) return RSV_FAIL("sample: bad n=%d batch=%d", n, batch);
    if (n >= kSampMinN && n <= 262144 && batch <= 65535) {
        // the multi-CU top-p path (each row falls back to the one-block pipeline inside the last launch)
        const dim3 g((n + 1023) / 1024, batch);
        hipLaunchKernelGGL(k_samp_scale, g, dim3(1024), 0, ctx->stream, logits, n, temp, counter, sampler, hist,
                           hist_stride);
        RSV_HIP(hipGetLastError());
        hipLaunchKernelGGL(k_samp_exp, g, dim3(1024), 0, ctx->stream, n, temp, counter, sampler);
        RSV_HIP(hipGetLastError());
#define SAMP_PICK(P)                                                                                          \
    if (P == 0 || n == (P)*kSampBS) {                                                                           \
        hipLaunchKernelGGL(k_samp_pick<P>, dim3(batch), dim3(1024), 0, ctx->stream, logits, token, n, temp, counter, \
                           sampler, hist, hist_stride);                                                          \
        RSV_HIP(hipGetLastError());                                                                             \
        return 0;                                                                                               \
    }
        SAMP_PICK(64) SAMP_PICK(32) SAMP_PICK(16) SAMP_PICK(8) SAMP_PICK(0)
#undef SAMP_PICK
    }
    // rows of 1024 x 2^j entries (j <= 6: vocabularies 1,024 .. 65,536) in
    // registers, others on the general kernel
#define SAMP_REGS(P)                                                                                             \
    if (n == (P)*kSampBS) {                                                                                        \
        hipLaunchKernelGGL(k_sample_regs<P>, dim3(batch), dim3(kSampBS), 0, ctx->stream, logits, token, n, temp, \
                           counter, sampler, hist, hist_stride);                                                  \
        RSV_HIP(hipGetLastError());                                                                                \
        return 0;                                                                                                  \
    }
    SAMP_REGS(64) SAMP_REGS(32) SAMP_REGS(16) SAMP_REGS(8) SAMP_REGS(4) SAMP_REGS(2) SAMP_REGS(1)
#undef SAMP_REGS
    hipLaunchKernelGGL(k_sample, dim3(batch), dim3(kSampBS), 0, ctx->stream, logits, token, n, temp, counter, sampler,
                       hist, hist_stride);
    RSV_HIP(hipGetLastError());
    return 0;
}

}  // namespace rsv
