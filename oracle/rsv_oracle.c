/*
 * rsv_oracle.c -- CPU fp32 restatement of rwkv-rsv's RWKV-7 forward step.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP
 * path: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * may load it.  The product library never links or calls it.
 *
 * Every function cites the reference code it restates (paths relative to the
 * reference repository root).  Arithmetic follows the reference's CPU path
 * (src/model.rs) operation by operation: two-pass LayerNorm/GroupNorm with
 * eps inside the sqrt, i-outer matvec with the zero skip, separate multiply
 * and add (Rust does not contract a*b+c into an fma; this file is compiled
 * with -ffp-contract=off for the same reason).
 *
 * Pinning (what checks each function independently of this restatement):
 *   f16 <-> f32          exhaustive 65536-pattern round trip + numpy float16
 *   orc_dequant_int8     model.rs:840-876 known answers, backend_cuda.rs:10121-10190 vector
 *   orc_layer_norm/      numpy float64 textbook LayerNorm/GroupNorm
 *   orc_group_norm
 *   orc_matvec           numpy float64 x @ W
 *   orc_dplr_*           numpy float64 matrix form S diag(w) + (S a) b^T + v k^T,
 *                        and the closed-form dplr_seq inputs of backend_cuda.rs:9996-10082
 *   orc_forward          independent numpy float64 RWKV-7 forward on tiny shapes
 *   orc_argmax           backend_cuda.rs:9276-9324 (sin(0.1 i) max, tie {0,999} -> 0)
 *   orc_sample           backend_cuda.rs:9327-9398 known answers; temperature 1e-4 == argmax
 *   orc_u01              MurmurHash3 fmix32 closed form (published finaliser)
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORC_LN_EPS 1.0e-5f   /* model.rs:6 */
#define ORC_GN_EPS 64.0e-5f  /* model.rs:7 */
#define ORC_L2_EPS 1.0e-12f  /* model.rs:8 */

/* ------------------------------------------------------------------ f16 */
/* IEEE binary16 <-> binary32, round-to-nearest-even.  Restates the
 * conversions of the `half` crate 2.7.1 used at model.rs:211-214, 241-242. */
float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal: renormalise */
            int e = -1;
            do { e++; man <<= 1; } while ((man & 0x400u) == 0);
            man &= 0x3FFu;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 0x1F) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xFFu;
    uint32_t man = x & 0x7FFFFFu;
    if (exp == 0xFF) { /* inf / nan (keep a quiet nan payload bit) */
        return (uint16_t)(sign | 0x7C00u | (man ? (0x200u | (man >> 13)) : 0));
    }
    int e = (int)exp - 127 + 15;
    if (e >= 0x1F) return (uint16_t)(sign | 0x7C00u); /* overflow -> inf */
    if (e <= 0) {                                    /* subnormal or zero */
        if (e < -10) return (uint16_t)sign;
        man |= 0x800000u;
        uint32_t shift = (uint32_t)(14 - e);
        uint32_t half_man = man >> shift;
        uint32_t rem = man & ((1u << shift) - 1);
        uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (half_man & 1u))) half_man++;
        return (uint16_t)(sign | half_man);
    }
    uint32_t half_man = man >> 13;
    uint32_t rem = man & 0x1FFFu;
    uint32_t out = sign | ((uint32_t)e << 10) | half_man;
    if (rem > 0x1000u || (rem == 0x1000u && (half_man & 1u))) out++; /* may carry into exp: correct */
    return (uint16_t)out;
}

/* ------------------------------------------------------------- dequant */
/* model.rs:234-252: w[m,k] = scale[m,k/128] * q[m,k] + zero[m,k/128];
 * q packed 4 per u32, low byte first; sz = f16 scale (low 16) | f16 zero (high 16). */
void orc_dequant_int8(const uint32_t *idx, const uint32_t *sz, int64_t m, int64_t k, float *w) {
    int64_t kg = k / 128;
    for (int64_t r = 0; r < m; r++) {
        for (int64_t g = 0; g < kg; g++) {
            uint32_t szv = sz[r * kg + g];
            float scale = orc_f16_to_f32((uint16_t)(szv & 0xFFFFu));
            float zero = orc_f16_to_f32((uint16_t)(szv >> 16));
            for (int64_t j = 0; j < 128; j++) {
                int64_t ki = g * 128 + j;
                uint32_t pack = idx[r * (k / 4) + ki / 4];
                float q = (float)((pack >> ((ki % 4) * 8)) & 0xFFu);
                float p = scale * q;
                w[r * k + ki] = p + zero;
            }
        }
    }
}

/* -------------------------------------------------------------- helpers */
/* model.rs:625-635 (two-pass, eps inside sqrt, recip then multiply) */
void orc_layer_norm(const float *x, const float *w, const float *b, int64_t n, float eps, float *y) {
    float s = 0.0f;
    for (int64_t i = 0; i < n; i++) s += x[i];
    float mean = s / (float)n;
    float v = 0.0f;
    for (int64_t i = 0; i < n; i++) { float d = x[i] - mean; v += d * d; }
    float var = v / (float)n + eps;
    float inv_std = 1.0f / sqrtf(var);
    for (int64_t i = 0; i < n; i++) y[i] = (x[i] - mean) * inv_std * w[i] + b[i];
}

/* model.rs:785-797 */
void orc_group_norm(const float *x, const float *w, const float *b, int64_t h, int64_t n, float eps, float *y) {
    for (int64_t hi = 0; hi < h; hi++) orc_layer_norm(x + hi * n, w + hi * n, b + hi * n, n, eps, y + hi * n);
}

/* model.rs:654-660: x + w*(y-x) */
static void lerp(const float *x, const float *y, const float *w, int64_t n, float *o) {
    for (int64_t i = 0; i < n; i++) o[i] = x[i] + w[i] * (y[i] - x[i]);
}

static float sigmoidf_(float v) { return 1.0f / (1.0f + expf(-v)); } /* model.rs:662-664 */

/* model.rs:700-713: y = x @ W, W [inp, out] row-major, i-outer with zero skip */
static void matvec_cols(const float *x, const float *w, int64_t inp, int64_t out, int64_t j0, int64_t j1,
                        float *y) {
    for (int64_t j = j0; j < j1; j++) y[j] = 0.0f;
    for (int64_t i = 0; i < inp; i++) {
        float xi = x[i];
        if (xi == 0.0f) continue;
        const float *row = w + i * out;
        for (int64_t j = j0; j < j1; j++) y[j] += xi * row[j];
    }
}

/* Checker-side speed-up only: with orc_set_threads(n > 1) the output columns
 * are split over n threads.  Each y[j] is still accumulated over i in the
 * same order with the same zero skip, so results are bit-identical to the
 * single-threaded loop (tests/test_oracle.py checks this).  The CPU baseline
 * keeps the default of 1 thread, the reference's own threading. */
static int orc_threads = 1;
void orc_set_threads(int n) { orc_threads = n < 1 ? 1 : (n > 64 ? 64 : n); }

struct mv_part { const float *x, *w; int64_t inp, out, j0, j1; float *y; };
static void *mv_run(void *p) {
    struct mv_part *a = (struct mv_part *)p;
    matvec_cols(a->x, a->w, a->inp, a->out, a->j0, a->j1, a->y);
    return NULL;
}

void orc_matvec(const float *x, const float *w, int64_t inp, int64_t out, float *y) {
    int nt = orc_threads;
    if (nt <= 1 || out < 1024) { matvec_cols(x, w, inp, out, 0, out, y); return; }
    pthread_t th[64];
    struct mv_part parts[64];
    int64_t per = ((out + nt - 1) / nt + 15) & ~(int64_t)15;
    int n = 0;
    for (int64_t j0 = 0; j0 < out; j0 += per, n++) {
        parts[n] = (struct mv_part){x, w, inp, out, j0, j0 + per < out ? j0 + per : out, y};
    }
    int started[64] = {0};
    for (int t = 1; t < n; t++) started[t] = pthread_create(&th[t], NULL, mv_run, &parts[t]) == 0;
    mv_run(&parts[0]);
    for (int t = 1; t < n; t++) {
        if (started[t]) pthread_join(th[t], NULL);
        else mv_run(&parts[t]);
    }
}

/* model.rs:716-727 */
void orc_l2_norm_groups(const float *x, int64_t h, int64_t n, float *out) {
    for (int64_t hi = 0; hi < h; hi++) {
        float s = 0.0f;
        for (int64_t j = 0; j < n; j++) s += x[hi * n + j] * x[hi * n + j];
        float norm = sqrtf(s);
        if (norm < ORC_L2_EPS) norm = ORC_L2_EPS;
        float inv = 1.0f / norm;
        for (int64_t j = 0; j < n; j++) out[hi * n + j] = x[hi * n + j] * inv;
    }
}

/* model.rs:732-766: S = S*diag(w) + (S a) b^T + v k^T, per head */
void orc_dplr_update(float *s, const float *k, const float *v, const float *w, const float *a,
                     const float *b, int64_t h, int64_t n) {
    float *sa = (float *)malloc(sizeof(float) * (size_t)n);
    for (int64_t hi = 0; hi < h; hi++) {
        float *S = s + hi * n * n;
        const float *wh = w + hi * n, *kh = k + hi * n, *vh = v + hi * n, *ah = a + hi * n, *bh = b + hi * n;
        for (int64_t i = 0; i < n; i++) {
            float acc = 0.0f;
            for (int64_t j = 0; j < n; j++) acc += S[i * n + j] * ah[j];
            sa[i] = acc;
        }
        for (int64_t i = 0; i < n; i++)
            for (int64_t j = 0; j < n; j++)
                S[i * n + j] = S[i * n + j] * wh[j] + sa[i] * bh[j] + vh[i] * kh[j];
    }
    free(sa);
}

/* model.rs:769-782: y = S r per head */
void orc_dplr_matvec(const float *s, const float *r, int64_t h, int64_t n, float *y) {
    for (int64_t hi = 0; hi < h; hi++) {
        const float *S = s + hi * n * n;
        for (int64_t i = 0; i < n; i++) {
            float acc = 0.0f;
            for (int64_t j = 0; j < n; j++) acc += S[i * n + j] * r[hi * n + j];
            y[hi * n + i] = acc;
        }
    }
}

/* model.rs:801-826: out = sum_j(r k r_k) * v per head */
void orc_sum_rk_rk(const float *r, const float *k, const float *rk, const float *v, int64_t h, int64_t n, float *out) {
    for (int64_t hi = 0; hi < h; hi++) {
        float s = 0.0f;
        for (int64_t j = 0; j < n; j++) s += r[hi * n + j] * k[hi * n + j] * rk[hi * n + j];
        for (int64_t j = 0; j < n; j++) out[hi * n + j] = s * v[hi * n + j];
    }
}

/* ---------------------------------------------------------------- model */
/* Weight pointers per layer, in this order; matrices are in the CPU path's
 * [in, out] orientation (model.rs:534-620). */
enum {
    L_LN1_W, L_LN1_B, L_XR, L_XW, L_XK, L_XV, L_XA, L_XG, L_W0, L_A0, L_V0,
    L_W1, L_W2, L_A1, L_A2, L_V1, L_V2, L_G1, L_G2, L_RK, L_KK, L_KA,
    L_RW, L_KW, L_VW, L_OW, L_LNX_W, L_LNX_B, L_LN2_W, L_LN2_B, L_FXK, L_FKW, L_FVW,
    L_NFIELDS
};

typedef struct {
    int64_t n_layer, c, vocab, head_size, n_head, ffn, wm, am, vm, gm;
    const float *emb_ln;   /* [vocab, C]: LN0 already applied (model.rs:385-392) */
    const float *ln_out_w, *ln_out_b;
    const float *head;     /* [C, vocab] */
    const float *const *layer; /* n_layer * L_NFIELDS pointers */
} orc_model;

int orc_nfields(void) { return L_NFIELDS; }

/* LN0 over every embedding row (model.rs:385-392, 637-652). */
void orc_layer_norm_rows(const float *x, const float *w, const float *b, int64_t c, int64_t rows, float eps, float *y) {
    for (int64_t r = 0; r < rows; r++) orc_layer_norm(x + r * c, w, b, c, eps, y + r * c);
}

/* State layout per session (gpu_model.rs:3972-3990): for each layer
 * [tmix_x C][tmix_rnn H*N*N][cmix_x C], then [v_first C]. */
int64_t orc_state_len(const orc_model *m) {
    return m->n_layer * (2 * m->c + m->n_head * m->head_size * m->head_size) + m->c;
}

/* model.rs:374-517.  Advances `state` over `ntok` tokens and writes the last
 * token's logits.  v_first is recomputed per token (model.rs:398); its value
 * for the last token is stored in the state's trailing [C] slot, which is
 * what the GPU State carries there. */
void orc_forward(const orc_model *m, const uint32_t *tokens, int64_t ntok, float *state, float *logits) {
    const int64_t c = m->c, h = m->n_head, n = m->head_size;
    const int64_t wm = m->wm, am = m->am, vm = m->vm, gm = m->gm, fh = m->ffn;
    const int64_t per_layer = 2 * c + h * n * n;
    float *x = malloc(sizeof(float) * c), *ln1 = malloc(sizeof(float) * c);
    float *xr = malloc(sizeof(float) * c), *xw = malloc(sizeof(float) * c), *xk = malloc(sizeof(float) * c);
    float *xv = malloc(sizeof(float) * c), *xa = malloc(sizeof(float) * c), *xg = malloc(sizeof(float) * c);
    float *r = malloc(sizeof(float) * c), *k = malloc(sizeof(float) * c), *v = malloc(sizeof(float) * c);
    float *vf = malloc(sizeof(float) * c), *tmp = malloc(sizeof(float) * c), *full = malloc(sizeof(float) * c);
    float *w = malloc(sizeof(float) * c), *a = malloc(sizeof(float) * c), *kk = malloc(sizeof(float) * c);
    float *kmod = malloc(sizeof(float) * c), *kkl2 = malloc(sizeof(float) * c), *bvec = malloc(sizeof(float) * c);
    float *y = malloc(sizeof(float) * c), *yn = malloc(sizeof(float) * c), *extra = malloc(sizeof(float) * c);
    float *g = malloc(sizeof(float) * c), *yg = malloc(sizeof(float) * c), *ln2 = malloc(sizeof(float) * c);
    float *xb = malloc(sizeof(float) * c), *vout = malloc(sizeof(float) * c);
    int64_t midmax = wm; if (am > midmax) midmax = am; if (vm > midmax) midmax = vm; if (gm > midmax) midmax = gm;
    float *mid = malloc(sizeof(float) * midmax);
    float *r2 = malloc(sizeof(float) * fh);
    const float neg_inv_sqrt_e = -1.0f / sqrtf(2.718281828459045f); /* model.rs:438 */

    for (int64_t t = 0; t < ntok; t++) {
        memcpy(x, m->emb_ln + (int64_t)tokens[t] * c, sizeof(float) * c);
        int have_vf = 0;
        for (int64_t li = 0; li < m->n_layer; li++) {
            const float *const *L = m->layer + li * L_NFIELDS;
            float *st = state + li * per_layer;
            float *tmix_x = st, *rnn = st + c, *cmix_x = st + c + h * n * n;
            /* time mixing */
            orc_layer_norm(x, L[L_LN1_W], L[L_LN1_B], c, ORC_LN_EPS, ln1);
            lerp(ln1, tmix_x, L[L_XR], c, xr);
            lerp(ln1, tmix_x, L[L_XW], c, xw);
            lerp(ln1, tmix_x, L[L_XK], c, xk);
            lerp(ln1, tmix_x, L[L_XV], c, xv);
            lerp(ln1, tmix_x, L[L_XA], c, xa);
            lerp(ln1, tmix_x, L[L_XG], c, xg);
            memcpy(tmix_x, ln1, sizeof(float) * c);
            orc_matvec(xr, L[L_RW], c, c, r);
            orc_matvec(xk, L[L_KW], c, c, k);
            orc_matvec(xv, L[L_VW], c, c, v);
            if (!have_vf) { /* model.rs:419-431 */
                memcpy(vf, v, sizeof(float) * c);
                have_vf = 1;
            } else {
                orc_matvec(xv, L[L_V1], c, vm, mid);
                orc_matvec(mid, L[L_V2], vm, c, full);
                for (int64_t i = 0; i < c; i++) tmp[i] = sigmoidf_(full[i] + L[L_V0][i]);
                lerp(v, vf, tmp, c, vout);
                memcpy(v, vout, sizeof(float) * c);
            }
            /* w = exp(-sigmoid(w0 + tanh(xw@w1)@w2)/sqrt(e)) (model.rs:433-438) */
            orc_matvec(xw, L[L_W1], c, wm, mid);
            for (int64_t i = 0; i < wm; i++) mid[i] = tanhf(mid[i]);
            orc_matvec(mid, L[L_W2], wm, c, full);
            for (int64_t i = 0; i < c; i++) {
                float sg = sigmoidf_(full[i] + L[L_W0][i]);
                w[i] = expf(sg * neg_inv_sqrt_e);
            }
            /* a = sigmoid(a0 + xa@a1@a2) (model.rs:440-443) */
            orc_matvec(xa, L[L_A1], c, am, mid);
            orc_matvec(mid, L[L_A2], am, c, full);
            for (int64_t i = 0; i < c; i++) a[i] = sigmoidf_(full[i] + L[L_A0][i]);
            /* kk, k_mod (model.rs:445-449) */
            for (int64_t i = 0; i < c; i++) kk[i] = k[i] * L[L_KK][i];
            for (int64_t i = 0; i < c; i++) tmp[i] = k[i] * a[i];
            lerp(k, tmp, L[L_KA], c, kmod);
            orc_l2_norm_groups(kk, h, n, kkl2);
            for (int64_t i = 0; i < c; i++) bvec[i] = kkl2[i] * (-a[i]); /* model.rs:460 */
            orc_dplr_update(rnn, kmod, v, w, kkl2, bvec, h, n);
            orc_dplr_matvec(rnn, r, h, n, y);
            orc_group_norm(y, L[L_LNX_W], L[L_LNX_B], h, n, ORC_GN_EPS, yn);
            orc_sum_rk_rk(r, kmod, L[L_RK], v, h, n, extra);
            for (int64_t i = 0; i < c; i++) yn[i] = yn[i] + extra[i];
            /* g = sigmoid(xg@g1)@g2 (model.rs:475-478) */
            orc_matvec(xg, L[L_G1], c, gm, mid);
            for (int64_t i = 0; i < gm; i++) mid[i] = sigmoidf_(mid[i]);
            orc_matvec(mid, L[L_G2], gm, c, g);
            for (int64_t i = 0; i < c; i++) yg[i] = yn[i] * g[i];
            orc_matvec(yg, L[L_OW], c, c, tmp);
            for (int64_t i = 0; i < c; i++) x[i] = x[i] + tmp[i];
            /* channel mixing (model.rs:486-495) */
            orc_layer_norm(x, L[L_LN2_W], L[L_LN2_B], c, ORC_LN_EPS, ln2);
            lerp(ln2, cmix_x, L[L_FXK], c, xb);
            memcpy(cmix_x, ln2, sizeof(float) * c);
            orc_matvec(xb, L[L_FKW], c, fh, r2);
            for (int64_t i = 0; i < fh; i++) { float q = r2[i] > 0.0f ? r2[i] : 0.0f; r2[i] = q * q; }
            orc_matvec(r2, L[L_FVW], fh, c, tmp);
            for (int64_t i = 0; i < c; i++) x[i] = x[i] + tmp[i];
        }
        memcpy(state + m->n_layer * per_layer, vf, sizeof(float) * c);
        orc_layer_norm(x, m->ln_out_w, m->ln_out_b, c, ORC_LN_EPS, tmp);
        orc_matvec(tmp, m->head, c, m->vocab, logits);
    }
    free(x); free(ln1); free(xr); free(xw); free(xk); free(xv); free(xa); free(xg);
    free(r); free(k); free(v); free(vf); free(tmp); free(full); free(w); free(a); free(kk);
    free(kmod); free(kkl2); free(bvec); free(y); free(yn); free(extra); free(g); free(yg);
    free(ln2); free(xb); free(vout); free(mid); free(r2);
}

/* ----------------------------------------------------------- sampling */
/* argmax, ties -> smaller index (backend_cuda.rs:3640-3680: strict > scan,
 * tree reduce preferring the smaller index; initial best -1e30 at index 0). */
uint32_t orc_argmax(const float *x, int64_t n) {
    float best = -1e30f;
    int64_t bi = 0;
    for (int64_t i = 0; i < n; i++)
        if (x[i] > best) { best = x[i]; bi = i; }
    return (uint32_t)bi;
}

/* backend_cuda.rs:3691-3698: golden-ratio increment + MurmurHash3 fmix32. */
float orc_u01(uint32_t s) {
    s += 0x9E3779B9u;
    uint32_t z = s;
    z = (z ^ (z >> 16)) * 0x85EBCA6Bu;
    z = (z ^ (z >> 13)) * 0xC2B2AE35u;
    z ^= z >> 16;
    return (float)z / 4294967296.0f;
}

/* Largest unmasked value, ties -> smaller index (used by the iterative
 * top-k / top-p paths, backend_cuda.rs:3836-3860, 3927-3955). */
static int64_t max_unmasked(const float *t, const unsigned char *mask, int64_t n) {
    float lm = -1e30f;
    int64_t li = 0;
    for (int64_t i = 0; i < n; i++)
        if (!mask[i] && t[i] > lm) { lm = t[i]; li = i; }
    return li;
}

/* Block sum of the reference's 112-thread sampler kernels
 * (backend_cuda.rs:3880-3921, 3978-3990): thread t sums t[i] for i = t,
 * t+112, ... in order; lanes 64..111 fold into 0..47; then a halving tree.
 * The float result depends on this order, so it is restated exactly. */
static float sum112(const float *t, int64_t n) {
    float p[112];
    for (int tid = 0; tid < 112; tid++) {
        float s = 0.0f;
        for (int64_t i = tid; i < n; i += 112) s += t[i];
        p[tid] = s;
    }
    for (int tid = 0; tid < 48; tid++) p[tid] += p[tid + 64];
    for (int step = 32; step > 0; step >>= 1)
        for (int tid = 0; tid < step; tid++) p[tid] += p[tid + step];
    return p[0];
}

/* Sampler pipeline of backend_cuda.rs:3690-4009 restated sequentially:
 * penalties -> 1/T -> top-k (K<=50: K-th largest threshold, sorted
 * candidate list; else iterative) -> softmax -> top-p -> u01(seed) scan.
 * `work` must hold 2*n floats.  Returns the sampled index. */
uint32_t orc_sample(const float *logits, int64_t n, float temperature, uint32_t top_k, float top_p,
                    uint32_t seed, float rep, float freq, float pres, const uint32_t *hist,
                    uint32_t hist_len, float *work) {
    const int MAXK = 50;
    float *temp = work;
    unsigned char *mask = (unsigned char *)calloc((size_t)n, 1);
    uint32_t *cnt = NULL;
    int do_topk = top_k > 0u && top_k < (uint32_t)n;
    int K = do_topk ? (int)top_k : 0;
    int64_t sorted_idx[50];
    for (int64_t i = 0; i < n; i++) temp[i] = logits[i];
    /* penalties (backend_cuda.rs:3750-3768) */
    if (hist_len > 0u && (rep != 1.0f || freq != 0.0f || pres != 0.0f)) {
        cnt = (uint32_t *)calloc((size_t)n, sizeof(uint32_t));
        for (uint32_t i = 0; i < hist_len; i++) cnt[hist[i]]++;
        for (int64_t i = 0; i < n; i++) {
            float l = temp[i];
            if (cnt[i] > 0u) {
                if (rep != 1.0f) l = l > 0.0f ? l / rep : l * rep;
                if (pres != 0.0f) l -= pres;
            }
            if (freq != 0.0f) l -= freq * (float)cnt[i];
            temp[i] = l;
        }
    }
    /* temperature (backend_cuda.rs:3771-3774) */
    float invT = 1.0f / temperature;
    if (!(temperature > 0.0f)) invT = 1.0f;
    for (int64_t i = 0; i < n; i++) temp[i] *= invT;
    /* top-k */
    if (K > 0 && K <= MAXK) {
        /* K largest values, descending; equal values ordered by index. */
        for (int j = 0; j < K; j++) {
            int64_t bi = max_unmasked(temp, mask, n);
            sorted_idx[j] = bi;
            mask[bi] = 1;
        }
        float thr = temp[sorted_idx[K - 1]];
        for (int64_t i = 0; i < n; i++) if (temp[i] < thr) temp[i] = -1e30f;
        memset(mask, 0, (size_t)n);
    } else if (do_topk) {
        float thr = -1e30f;
        for (uint32_t rd = 0; rd < top_k; rd++) {
            int64_t bi = max_unmasked(temp, mask, n);
            thr = temp[bi];
            mask[bi] = 1;
        }
        for (int64_t i = 0; i < n; i++) if (temp[i] < thr) temp[i] = -1e30f;
        memset(mask, 0, (size_t)n);
    }
    /* softmax (backend_cuda.rs:3880-3921) */
    float m = -1e30f;
    for (int64_t i = 0; i < n; i++) m = fmaxf(m, temp[i]);
    for (int64_t i = 0; i < n; i++) temp[i] = expf(temp[i] - m);
    float total = sum112(temp, n);
    if (total > 0.0f) for (int64_t i = 0; i < n; i++) temp[i] /= total;
    /* top-p (backend_cuda.rs:3924-3967) */
    if (top_p > 0.0f && top_p < 1.0f) {
        float cutoff;
        if (K > 0 && K <= MAXK) {
            /* the reference accumulates from the K-th candidate toward the largest */
            float cum = 0.0f;
            cutoff = -1e30f;
            for (int j = K - 1; j >= 0; j--) {
                int64_t idx = sorted_idx[j];
                cum += temp[idx];
                cutoff = temp[idx];
                if (cum >= top_p) break;
            }
        } else {
            float cum = 0.0f;
            cutoff = 0.0f;
            for (int c = 0; c < 512 && cum < top_p; c++) { /* 512-token cap */
                int64_t bi = max_unmasked(temp, mask, n);
                mask[bi] = 1;
                cum += temp[bi];
                cutoff = temp[bi];
            }
        }
        for (int64_t i = 0; i < n; i++) if (temp[i] < cutoff) temp[i] = 0.0f;
    }
    /* draw (backend_cuda.rs:3970-4008) */
    uint32_t chosen;
    if (K > 0 && K <= MAXK) {
        float tot = 0.0f;
        for (int j = K - 1; j >= 0; j--) if (temp[sorted_idx[j]] > 0.0f) tot += temp[sorted_idx[j]];
        float u = orc_u01(seed) * tot;
        float acc = 0.0f;
        chosen = (uint32_t)sorted_idx[K - 1];
        for (int j = K - 1; j >= 0; j--) {
            int64_t idx = sorted_idx[j];
            if (temp[idx] > 0.0f) {
                acc += temp[idx];
                if (acc > u) { chosen = (uint32_t)idx; break; }
            }
        }
    } else {
        float tot = sum112(temp, n);
        float u = orc_u01(seed) * tot;
        float acc = 0.0f;
        chosen = (uint32_t)(n - 1);
        for (int64_t i = 0; i < n; i++) {
            acc += temp[i];
            if (acc > u) { chosen = (uint32_t)i; break; }
        }
    }
    free(mask);
    free(cnt);
    return chosen;
}
