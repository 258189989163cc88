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
        float s = 0.0f;
        for (int i = threadIdx.x; i < n; i += 112) s += t[i];
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

// Key of the R-th largest element (1-based) of t[0..n).
__device__ uint32_t radix_select(const float *t, int n, int R, SampShared &sh) {
    uint32_t prefix = 0, mask = 0;
    uint32_t remaining = (uint32_t)R;
    for (int pass = 0; pass < 4; pass++) {
        const int shift = 24 - 8 * pass;
        for (int i = threadIdx.x; i < 256; i += kSampBS) sh.hist[i] = 0;
        __syncthreads();
        for (int i = threadIdx.x; i < n; i += kSampBS) {
            const uint32_t k = fkey(t[i]);
            if ((k & mask) == prefix) atomicAdd(&sh.hist[(k >> shift) & 255u], 1u);
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            uint32_t cum = 0;
            int bin = 0;
            for (int bb = 255; bb >= 0; bb--) {
                const uint32_t c = sh.hist[bb];
                if (cum + c >= remaining) { bin = bb; break; }
                cum += c;
            }
            sh.sel_bin = (uint32_t)bin;
            sh.sel_rem = remaining - cum;
        }
        __syncthreads();
        prefix |= sh.sel_bin << shift;
        mask |= 255u << shift;
        remaining = sh.sel_rem;
        __syncthreads();
    }
    return prefix;
}

// Gathers the R largest elements (ties at the threshold by ascending index)
// into sh.ckey/cidx sorted by (key desc, index asc).  R <= kCand.
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
    __syncthreads();
    if (threadIdx.x == 0) {  // exclusive scans
        uint32_t a = 0, b = 0;
        for (int i = 0; i < kSampBS; i++) {
            const uint32_t g = sh.cnt_gt[i], e = sh.cnt_eq[i];
            sh.cnt_gt[i] = a;
            sh.cnt_eq[i] = b;
            a += g;
            b += e;
        }
        sh.sel_rem = a;  // number strictly greater
    }
    __syncthreads();
    const uint32_t G = sh.sel_rem;
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
    // bitonic sort of kCand entries, descending by key, ascending by index
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
            if (tid == 0) {
                float cum = 0.0f, cut = 0.0f;
                for (int c = 0; c < R && cum < top_p; c++) {
                    const float p = temp[sh.cidx[c]];
                    cum += p;
                    cut = p;
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
    uint32_t nz = 0;
    for (int i = lo; i < hi; i++) nz += temp[i] != 0.0f;
    sh.cnt_gt[tid] = nz;
    __syncthreads();
    if (tid == 0) {
        uint32_t a = 0;
        for (int i = 0; i < kSampBS; i++) { const uint32_t v = sh.cnt_gt[i]; sh.cnt_gt[i] = a; a += v; }
        sh.sel_rem = a;
    }
    __syncthreads();
    const uint32_t NZ = sh.sel_rem;
    const bool compact = NZ <= (uint32_t)kCand;
    if (compact) {
        uint32_t o = sh.cnt_gt[tid];
        for (int i = lo; i < hi; i++)
            if (temp[i] != 0.0f) sh.cidx[o++] = i;
    }
    __syncthreads();
    if (tid == 0) {
        const float u = u01_dev(seed) * tot;
        float acc = 0.0f;
        int chosen = n - 1;
        if (compact) {
            for (uint32_t j = 0; j < NZ; j++) {
                const int ix = sh.cidx[j];
                acc += temp[ix];
                if (acc > u) { chosen = ix; break; }
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
    hipLaunchKernelGGL(k_sample, dim3(batch), dim3(kSampBS), 0, ctx->stream, logits, token, n, temp, counter, sampler,
                       hist, hist_stride);
    RSV_HIP(hipGetLastError());
    return 0;
}

}  // namespace rsv
