// On-GPU sampler: penalties -> 1/T -> top-k -> softmax -> top-p -> seeded
// draw, one 1024-thread block per session row.
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
            __syncthreads();
        }
    }
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

__global__ __launch_bounds__(kSampBS) void k_sample(const float *__restrict__ logits, uint32_t *__restrict__ token,
                                                    int n, float *__restrict__ temp_all,
                                                    uint32_t *__restrict__ counter_all,
                                                    const float *__restrict__ sampler,
                                                    const uint32_t *__restrict__ hist_all, int hist_stride) {
    __shared__ SampShared sh;
    const int b = blockIdx.x, tid = threadIdx.x;
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
__global__ __launch_bounds__(kSampBS) void k_sample_regs(const float *__restrict__ logits, uint32_t *__restrict__ token,
                                                         int n, float *__restrict__ temp_all,
                                                         uint32_t *__restrict__ counter_all,
                                                         const float *__restrict__ sampler,
                                                         const uint32_t *__restrict__ hist_all, int hist_stride) {
    __shared__ SampShared sh;
    const int b = blockIdx.x, tid = threadIdx.x;
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

int launch_sample(rsv_ctx *ctx, const float *logits, uint32_t *token, int n, float *temp, uint32_t *counter,
                  const float *sampler, const uint32_t *hist, int hist_stride, int batch) {
    if (n <= 0 || batch <= 0) return RSV_FAIL("sample: bad n=%d batch=%d", n, batch);
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
