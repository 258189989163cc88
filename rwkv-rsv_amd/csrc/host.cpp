// librsv_host.so: the model driver above the HIP backend C-ABI.
//
// Restates the reference's GpuModel / Bundle / State (src/gpu_model.rs) in
// C++ for hosts without a Rust toolchain.  Talks to the device only through
// include/rsv_hip.h, exactly as a backend_hip.rs-backed GpuModel would.
//
//  - load:    safetensors (mmap) -> config from shapes (gpu_model.rs:401-546),
//             LN0 applied to the embedding on the CPU (gpu_model.rs:450-460),
//             linears int8 when `{key}.int8_idx` exists else fp16
//             (gpu_model.rs:3405-3442), LoRA oriented [out, in] fp16.
//  - decode:  per layer norm_lerp6 -> fused stage-1 -> v_first snapshot
//             (layer 0) -> LoRA stage-2 chain -> WKV7 -> att.output ->
//             cmix_norm_lerp -> ffn.key relu^2 -> ffn.value
//             (gpu_model.rs:2060-2392), batched over B slots.
//  - prefill: packed ragged segments through MFMA GEMMs and one sequential
//             WKV scan per layer (replaces gpu_model.rs:2911-3255 and
//             1041-1350).
//  - self-loops: one step captured as a HIP graph and replayed n times
//             (gpu_model.rs:1824-1874, 732-852, 1639-1803).
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "../../include/rsv_hip.h"
#include "../../include/rsv_host.h"

namespace {

thread_local std::string g_herr;

int herr(const char *fmt, ...) {
    char buf[2048];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_herr = buf;
    return -1;
}

// Propagate a backend failure with its text.
#define CK(call)                                                              \
    do {                                                                      \
        if ((call) != 0) return herr("%s: %s", #call, rsv_last_error());       \
    } while (0)
#define HK(call)                         \
    do {                                 \
        if ((call) != 0) return -1;      \
    } while (0)

constexpr uint32_t NONE = 0xFFFFFFFFu;
constexpr float LN_EPS = 1.0e-5f;  // model.rs:6
constexpr float GN_EPS = 64.0e-5f; // model.rs:7
constexpr float L2_EPS = 1.0e-12f; // model.rs:8

// ------------------------------------------------------------ safetensors
struct StEntry {
    std::string dtype;
    std::vector<uint64_t> shape;
    uint64_t begin = 0, end = 0;
    uint64_t numel() const {
        uint64_t n = 1;
        for (auto s : shape) n *= s;
        return n;
    }
};

struct SafeTensors {
    int fd = -1;
    uint8_t *base = nullptr;
    size_t size = 0;
    const uint8_t *data = nullptr;
    std::map<std::string, StEntry> t;

    ~SafeTensors() {
        if (base) munmap(base, size);
        if (fd >= 0) close(fd);
    }

    // Minimal JSON reader for the safetensors header: an object of objects
    // holding "dtype" (string), "shape" (int array), "data_offsets" (2 ints).
    struct P {
        const char *s, *e;
        void ws() { while (s < e && (*s == ' ' || *s == '\n' || *s == '\r' || *s == '\t')) s++; }
        bool lit(char c) { ws(); if (s < e && *s == c) { s++; return true; } return false; }
        bool str(std::string &out) {
            ws();
            if (s >= e || *s != '"') return false;
            s++;
            out.clear();
            while (s < e && *s != '"') {
                if (*s == '\\' && s + 1 < e) { out.push_back(s[1]); s += 2; continue; }
                out.push_back(*s++);
            }
            if (s >= e) return false;
            s++;
            return true;
        }
        bool num(uint64_t &v) {
            ws();
            if (s >= e || *s < '0' || *s > '9') return false;
            v = 0;
            while (s < e && *s >= '0' && *s <= '9') v = v * 10 + (uint64_t)(*s++ - '0');
            return true;
        }
        bool skip() {  // skip any JSON value
            ws();
            if (s >= e) return false;
            if (*s == '"') { std::string d; return str(d); }
            if (*s == '{' || *s == '[') {
                const char open = *s, close = open == '{' ? '}' : ']';
                int depth = 0;
                bool in_str = false;
                for (; s < e; s++) {
                    if (in_str) { if (*s == '\\') s++; else if (*s == '"') in_str = false; continue; }
                    if (*s == '"') in_str = true;
                    else if (*s == open) depth++;
                    else if (*s == close && --depth == 0) { s++; return true; }
                }
                return false;
            }
            while (s < e && *s != ',' && *s != '}' && *s != ']') s++;
            return true;
        }
    };

    int open_file(const char *path) {
        fd = ::open(path, O_RDONLY);
        if (fd < 0) return herr("cannot open %s", path);
        struct stat st;
        if (fstat(fd, &st) != 0) return herr("cannot stat %s", path);
        size = (size_t)st.st_size;
        if (size < 8) return herr("%s: too small for safetensors", path);
        base = (uint8_t *)mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
        if (base == MAP_FAILED) { base = nullptr; return herr("mmap %s failed", path); }
        uint64_t hl = 0;
        memcpy(&hl, base, 8);
        if (hl > size - 8) return herr("%s: bad header length", path);
        data = base + 8 + hl;
        const uint64_t dsize = size - 8 - hl;
        P p{(const char *)base + 8, (const char *)base + 8 + hl};
        if (!p.lit('{')) return herr("%s: header is not an object", path);
        if (p.lit('}')) return 0;
        do {
            std::string name;
            if (!p.str(name) || !p.lit(':')) return herr("%s: bad header key", path);
            if (name == "__metadata__") { if (!p.skip()) return herr("%s: bad metadata", path); continue; }
            StEntry ent;
            if (!p.lit('{')) return herr("%s: bad entry %s", path, name.c_str());
            if (!p.lit('}')) {
                do {
                    std::string k;
                    if (!p.str(k) || !p.lit(':')) return herr("%s: bad field in %s", path, name.c_str());
                    if (k == "dtype") {
                        if (!p.str(ent.dtype)) return herr("%s: bad dtype", path);
                    } else if (k == "shape" || k == "data_offsets") {
                        std::vector<uint64_t> v;
                        if (!p.lit('[')) return herr("%s: bad array", path);
                        if (!p.lit(']')) {
                            do {
                                uint64_t x;
                                if (!p.num(x)) return herr("%s: bad number", path);
                                v.push_back(x);
                            } while (p.lit(','));
                            if (!p.lit(']')) return herr("%s: unterminated array", path);
                        }
                        if (k == "shape") ent.shape = v;
                        else if (v.size() == 2) { ent.begin = v[0]; ent.end = v[1]; }
                    } else if (!p.skip()) {
                        return herr("%s: bad value", path);
                    }
                } while (p.lit(','));
                if (!p.lit('}')) return herr("%s: unterminated entry", path);
            }
            if (ent.end < ent.begin || ent.end > dsize) return herr("%s: %s out of range", path, name.c_str());
            t[name] = ent;
        } while (p.lit(','));
        return 0;
    }

    const StEntry *get(const std::string &k) const {
        auto it = t.find(k);
        return it == t.end() ? nullptr : &it->second;
    }

    // Tensor as f32 (F32 / F16 / BF16 sources), shape-checked.
    int f32(const std::string &k, std::vector<float> &out, uint64_t expect = 0) const {
        const StEntry *e = get(k);
        if (!e) return herr("missing tensor %s", k.c_str());
        const uint64_t n = e->numel();
        if (expect && n != expect) return herr("%s: %llu elements, expected %llu", k.c_str(), (unsigned long long)n, (unsigned long long)expect);
        out.resize(n);
        const uint8_t *p = data + e->begin;
        if (e->dtype == "F32") {
            if (e->end - e->begin != n * 4) return herr("%s: size mismatch", k.c_str());
            memcpy(out.data(), p, n * 4);
        } else if (e->dtype == "F16") {
            if (e->end - e->begin != n * 2) return herr("%s: size mismatch", k.c_str());
            for (uint64_t i = 0; i < n; i++) {
                uint16_t b;
                memcpy(&b, p + 2 * i, 2);
                _Float16 h;
                memcpy(&h, &b, 2);
                out[i] = (float)h;
            }
        } else if (e->dtype == "BF16") {
            if (e->end - e->begin != n * 2) return herr("%s: size mismatch", k.c_str());
            for (uint64_t i = 0; i < n; i++) {
                uint16_t b;
                memcpy(&b, p + 2 * i, 2);
                const uint32_t w = (uint32_t)b << 16;
                memcpy(&out[i], &w, 4);
            }
        } else {
            return herr("%s: unsupported dtype %s", k.c_str(), e->dtype.c_str());
        }
        return 0;
    }
};

// ------------------------------------------------------------ model types
struct Linear {
    bool i8 = false;
    rsv_int8 h{};      // int8
    uint32_t w16 = NONE; // fp16 [m, k]
    uint64_t m = 0, k = 0;
    // MFMA-tiled copy for the batched path (made on first use)
    bool tiled = false;
    rsv_int8 ht{};
    uint32_t t16 = NONE;
    // fp16 copy of an int8 matrix for the prefill GEMM (made on first use)
    uint32_t p16 = NONE;
};

struct Layer {
    uint32_t ln1_w, ln1_b, ln2_w, ln2_b, lnx_w, lnx_b;
    uint32_t x_r, x_w, x_k, x_v, x_a, x_g, ffn_x_k;
    uint32_t w0, a0, v0, r_k, k_k, k_a;
    uint32_t w1, w2, a1, a2, v1, v2, g1, g2;  // fp16 [out, in]
    Linear rw, kw, vw, ow, fk, fv;
    Linear lw1, lw2, la1, la2, lv1, lv2, lg1, lg2;  // LoRA views (fp16) for the batched path
    uint32_t fv_tiled = NONE;  // sparse ffn.value copy, fp16 [F/128][C/256][128][256] (RSV_FFN_SPARSE=1)
};

struct GpuState {
    uint64_t batch = 1;
    uint64_t serial = 0;  // distinct per state: part of the prefill graph key (graphs hold its tensors)
    std::vector<uint32_t> tmix_x, rnn, cmix_x;  // per layer
    uint32_t v_first = NONE;                    // [batch, C]
};

// An on/off environment switch (unset: def; "0": off).

struct WorkBufs {
    uint64_t batch = 0;
    uint32_t x, xr, xw, xk, xv, xa, xg, r, k, v, vmid, wmid, amid, gmid, w, a, g, yn, xb, r2, xnorm, logits, token;
    uint32_t ln1, ln2;  // LayerNorm rows kept for the token-shift state
    // fp16 operands of the matrix-core path (batch >= kMmBatch)
    bool mm = false;
    uint32_t mix16[6], vmid16, wmid16, amid16, gmid16, yg16, xb16, r216, xn16;
    // ffn.value as k-slices (matrix-core path): partial sums [fv_nsl, B, C]
    // that the next LayerNorm adds to the residual row, written to the other
    // residual buffer (x / xalt); xcur is the buffer holding the row, pend
    // whether partial sums are still to be added.  Set up per decode step.
    int fv_nsl = 0;
    uint32_t fvpart = NONE, xalt = NONE, xcur = NONE;
    int pend = 0;  // k-slices in fvpart still to be added (0: none)
};

constexpr uint64_t kMmBatch = 2;  // sessions from which decode GEMMs run on MFMA
constexpr uint64_t kSmallPrefill = 128;  // packed prefill rows that still take the decode MFMA kernel

struct SeqBufs {
    uint64_t cap = 0, segcap = 0;
    uint32_t tok = NONE, x = NONE, mix[6] = {NONE, NONE, NONE, NONE, NONE, NONE};
    uint32_t r = NONE, k = NONE, v = NONE, w = NONE, a = NONE, g = NONE, vf = NONE, yn = NONE, yg = NONE, xb = NONE,
             r2 = NONE;
    uint32_t vmid = NONE, wmid = NONE, amid = NONE, gmid = NONE;
    uint32_t row_prev = NONE, seg_start = NONE, seg_len = NONE, seg_slot = NONE, seg_last = NONE, seg_iota = NONE;
    uint32_t xlast = NONE, xnorm = NONE, logits = NONE;
    uint32_t bonus = NONE;  // [T, H] scratch of the gated scan
};

}  // namespace

struct rsv_state {
    GpuState s;
};

struct rsv_bundle {
    rsv_ctx *ctx = nullptr;
    uint64_t prefill_chunk = 4096;   // packed prefill rows per chunk (rsv_set_prefill_chunk)
    rsv_model_info info{};
    uint32_t emb_ln = NONE, ln_out_w = NONE, ln_out_b = NONE, scale_w = NONE;
    Linear head;
    std::vector<Layer> layers;
    rsv_state *state = nullptr;  // the bundle's own session
    std::map<uint64_t, WorkBufs> bufs;
    SeqBufs seq;
    SeqBufs seq2;          // the second lane's buffers of the pipelined prefill
    int prefill_lanes = 2; // rsv_set_prefill_lanes
    std::vector<uint32_t> owned;  // every tensor the bundle created
    bool tiled = false;           // MFMA-tiled weight copies made (tile_model)
    bool p16 = false;             // fp16 prefill copies of the int8 linears made (prefill_weights)
    // persistent single-session decode step: the state it is bound to, and
    // whether building it failed for good (shape or format unsupported)

    ~rsv_bundle() {
        if (ctx) rsv_destroy(ctx);
    }
};

namespace {

int new_tensor(rsv_bundle *b, uint64_t len, int dt, uint32_t &id) {
    CK(rsv_tensor_create(b->ctx, len, dt, &id));
    return 0;
}

int upload_vec(rsv_bundle *b, const SafeTensors &st, const std::string &key, uint64_t expect, uint32_t &id) {
    std::vector<float> v;
    HK(st.f32(key, v, expect));
    HK(new_tensor(b, v.size(), RSV_F32, id));
    CK(rsv_upload(b->ctx, id, v.data(), v.size()));
    return 0;
}

// Linear [out=m, in=k]: int8 when `key.int8_idx` exists (gpu_model.rs:3405-3442).
int load_linear(rsv_bundle *b, const SafeTensors &st, const std::string &key, uint64_t m, uint64_t k, Linear &L) {
    L.m = m;
    L.k = k;
    const StEntry *ie = st.get(key + ".int8_idx");
    if (ie) {
        const StEntry *se = st.get(key + ".int8_sz");
        if (!se) return herr("%s.int8_sz missing", key.c_str());
        if (k % 128 != 0) return herr("%s: int8 needs k %% 128 == 0", key.c_str());
        if (ie->end - ie->begin != m * k) return herr("%s.int8_idx: %llu bytes, expected %llu", key.c_str(), (unsigned long long)(ie->end - ie->begin), (unsigned long long)(m * k));
        if (se->end - se->begin != m * k / 128 * 4) return herr("%s.int8_sz size mismatch", key.c_str());
        L.i8 = true;
        HK(new_tensor(b, m * k / 4, RSV_U32, L.h.idx));
        HK(new_tensor(b, m * k / 128, RSV_U32, L.h.sz));
        CK(rsv_upload_bytes(b->ctx, L.h.idx, st.data + ie->begin, m * k));
        CK(rsv_upload_bytes(b->ctx, L.h.sz, st.data + se->begin, m * k / 128 * 4));
        L.h.m = m;
        L.h.k = k;
        return 0;
    }
    std::vector<float> w;
    HK(st.f32(key, w, m * k));
    HK(new_tensor(b, m * k, RSV_F16, L.w16));
    CK(rsv_upload(b->ctx, L.w16, w.data(), w.size()));
    return 0;
}

// LoRA matrix as fp16 [out, in]; the file may hold either orientation
// (model.rs:564-581).
int load_lora(rsv_bundle *b, const SafeTensors &st, const std::string &key, uint64_t in, uint64_t out, uint32_t &id) {
    const StEntry *e = st.get(key);
    if (!e) return herr("missing tensor %s", key.c_str());
    if (e->shape.size() != 2) return herr("%s: expected 2-D", key.c_str());
    std::vector<float> d;
    HK(st.f32(key, d, in * out));
    std::vector<float> o(in * out);
    if (e->shape[0] == out && e->shape[1] == in) {
        o = d;
    } else if (e->shape[0] == in && e->shape[1] == out) {
        for (uint64_t i = 0; i < in; i++)
            for (uint64_t j = 0; j < out; j++) o[j * in + i] = d[i * out + j];
    } else {
        return herr("%s: shape [%llu,%llu] is neither [%llu,%llu] nor its transpose", key.c_str(),
                    (unsigned long long)e->shape[0], (unsigned long long)e->shape[1], (unsigned long long)out, (unsigned long long)in);
    }
    HK(new_tensor(b, in * out, RSV_F16, id));
    CK(rsv_upload(b->ctx, id, o.data(), o.size()));
    return 0;
}

// model.rs:625-635
void layer_norm_cpu(const float *x, const float *w, const float *bb, uint64_t n, float *y) {
    float s = 0.0f;
    for (uint64_t i = 0; i < n; i++) s += x[i];
    const float mean = s / (float)n;
    float v = 0.0f;
    for (uint64_t i = 0; i < n; i++) { const float d = x[i] - mean; v += d * d; }
    const float inv = 1.0f / sqrtf(v / (float)n + LN_EPS);
    for (uint64_t i = 0; i < n; i++) y[i] = (x[i] - mean) * inv * w[i] + bb[i];
}

bool ffn_sparse_requested() {
    const char *e = getenv("RSV_FFN_SPARSE");
    return e && e[0] == '1';
}

int load_model(rsv_bundle *b, const char *path) {
    SafeTensors st;
    HK(st.open_file(path));
    // n_layer from the largest blocks.N index (model.rs:520-532)
    uint64_t n_layer = 0;
    for (auto &kv : st.t) {
        const std::string &k = kv.first;
        if (k.rfind("blocks.", 0) == 0) {
            const uint64_t idx = strtoull(k.c_str() + 7, nullptr, 10);
            if (idx + 1 > n_layer) n_layer = idx + 1;
        }
    }
    const StEntry *emb = st.get("emb.weight");
    const StEntry *rk = st.get("blocks.0.att.r_k");
    if (!emb || emb->shape.size() != 2 || !rk || rk->shape.size() != 2) return herr("%s: not an RWKV-7 model", path);
    rsv_model_info &I = b->info;
    I.n_layer = n_layer;
    I.vocab = emb->shape[0];
    I.n_embd = emb->shape[1];
    I.n_head = rk->shape[0];
    I.head_size = rk->shape[1];
    const uint64_t C = I.n_embd;
    auto mid_of = [&](const char *k, uint64_t &mid) -> int {
        const StEntry *e = st.get(k);
        if (!e || e->shape.size() != 2) return herr("missing %s", k);
        mid = e->shape[0] == C ? e->shape[1] : e->shape[0];
        return 0;
    };
    HK(mid_of("blocks.0.att.w1", I.w_mid));
    HK(mid_of("blocks.0.att.a1", I.a_mid));
    HK(mid_of("blocks.0.att.v1", I.v_mid));
    HK(mid_of("blocks.0.att.g1", I.g_mid));
    if (const StEntry *fk = st.get("blocks.0.ffn.key.weight")) I.ffn = fk->shape[0];
    else if (const StEntry *fk8 = st.get("blocks.0.ffn.key.weight.int8_idx")) I.ffn = fk8->shape[0];
    else return herr("missing blocks.0.ffn.key.weight");
    if (I.n_head * I.head_size != C) return herr("n_head*head_size != n_embd");
    if (I.head_size != 64) return herr("head_size %llu unsupported (64 required)", (unsigned long long)I.head_size);

    // emb_ln = LN0(emb) on the CPU, kept fp32 on the device (the reference
    // stores it fp16, gpu_model.rs:450-460)
    {
        std::vector<float> e, w, bb;
        HK(st.f32("emb.weight", e));
        HK(st.f32("blocks.0.ln0.weight", w, C));
        HK(st.f32("blocks.0.ln0.bias", bb, C));
        std::vector<float> out(e.size());
        for (uint64_t r = 0; r < I.vocab; r++) layer_norm_cpu(&e[r * C], w.data(), bb.data(), C, &out[r * C]);
        HK(new_tensor(b, out.size(), RSV_F32, b->emb_ln));
        CK(rsv_upload(b->ctx, b->emb_ln, out.data(), out.size()));
    }
    HK(upload_vec(b, st, "ln_out.weight", C, b->ln_out_w));
    HK(upload_vec(b, st, "ln_out.bias", C, b->ln_out_b));
    HK(load_linear(b, st, "head.weight", I.vocab, C, b->head));
    I.int8_head = b->head.i8;
    {
        const float sw = -1.0f / sqrtf(2.718281828459045f);  // gpu_model.rs:517-518
        HK(new_tensor(b, 1, RSV_F32, b->scale_w));
        CK(rsv_upload(b->ctx, b->scale_w, &sw, 1));
    }
    b->layers.resize(n_layer);
    bool all_i8 = true;
    for (uint64_t i = 0; i < n_layer; i++) {
        Layer &L = b->layers[i];
        const std::string p = "blocks." + std::to_string(i) + ".";
        HK(upload_vec(b, st, p + "ln1.weight", C, L.ln1_w));
        HK(upload_vec(b, st, p + "ln1.bias", C, L.ln1_b));
        HK(upload_vec(b, st, p + "ln2.weight", C, L.ln2_w));
        HK(upload_vec(b, st, p + "ln2.bias", C, L.ln2_b));
        HK(upload_vec(b, st, p + "att.ln_x.weight", C, L.lnx_w));
        HK(upload_vec(b, st, p + "att.ln_x.bias", C, L.lnx_b));
        HK(upload_vec(b, st, p + "att.x_r", C, L.x_r));
        HK(upload_vec(b, st, p + "att.x_w", C, L.x_w));
        HK(upload_vec(b, st, p + "att.x_k", C, L.x_k));
        HK(upload_vec(b, st, p + "att.x_v", C, L.x_v));
        HK(upload_vec(b, st, p + "att.x_a", C, L.x_a));
        HK(upload_vec(b, st, p + "att.x_g", C, L.x_g));
        HK(upload_vec(b, st, p + "ffn.x_k", C, L.ffn_x_k));
        HK(upload_vec(b, st, p + "att.w0", C, L.w0));
        HK(upload_vec(b, st, p + "att.a0", C, L.a0));
        HK(upload_vec(b, st, p + "att.v0", C, L.v0));
        HK(upload_vec(b, st, p + "att.r_k", C, L.r_k));
        HK(upload_vec(b, st, p + "att.k_k", C, L.k_k));
        HK(upload_vec(b, st, p + "att.k_a", C, L.k_a));
        HK(load_lora(b, st, p + "att.w1", C, I.w_mid, L.w1));
        HK(load_lora(b, st, p + "att.w2", I.w_mid, C, L.w2));
        HK(load_lora(b, st, p + "att.a1", C, I.a_mid, L.a1));
        HK(load_lora(b, st, p + "att.a2", I.a_mid, C, L.a2));
        HK(load_lora(b, st, p + "att.v1", C, I.v_mid, L.v1));
        HK(load_lora(b, st, p + "att.v2", I.v_mid, C, L.v2));
        HK(load_lora(b, st, p + "att.g1", C, I.g_mid, L.g1));
        HK(load_lora(b, st, p + "att.g2", I.g_mid, C, L.g2));
        HK(load_linear(b, st, p + "att.receptance.weight", C, C, L.rw));
        HK(load_linear(b, st, p + "att.key.weight", C, C, L.kw));
        HK(load_linear(b, st, p + "att.value.weight", C, C, L.vw));
        HK(load_linear(b, st, p + "att.output.weight", C, C, L.ow));
        HK(load_linear(b, st, p + "ffn.key.weight", I.ffn, C, L.fk));
        HK(load_linear(b, st, p + "ffn.value.weight", C, I.ffn, L.fv));
        all_i8 = all_i8 && L.rw.i8 && L.kw.i8 && L.vw.i8 && L.ow.i8 && L.fk.i8 && L.fv.i8;
    }
    I.int8_linears = all_i8;
    // sparse ffn.value (gpu_model.rs:2353-2371, 3290-3340): the tiled fp16 copy is made at load when
    // RSV_FFN_SPARSE=1 and the shapes allow it; the B<16 decode layer then reads only the rows of
    // ffn.value whose relu^2 input is non-zero
    if (ffn_sparse_requested() && C % 256 == 0 && I.ffn % 128 == 0) {
        for (auto &L : b->layers) {
            CK(rsv_tile_ffn_value(b->ctx, L.fv.w16, L.fv.i8 ? &L.fv.h : nullptr, C, I.ffn, &L.fv_tiled));
            b->owned.push_back(L.fv_tiled);
        }
    }
    CK(rsv_synchronize(b->ctx));
    return 0;
}

// ------------------------------------------------------------ state
int state_create(rsv_bundle *b, uint64_t batch, GpuState &s) {
    const rsv_model_info &I = b->info;
    const uint64_t C = I.n_embd, HNN = I.n_head * I.head_size * I.head_size;
    static std::atomic<uint64_t> next_serial{1};
    s.batch = batch;
    s.serial = next_serial++;
    s.tmix_x.assign(I.n_layer, NONE);
    s.rnn.assign(I.n_layer, NONE);
    s.cmix_x.assign(I.n_layer, NONE);
    for (uint64_t i = 0; i < I.n_layer; i++) {
        HK(new_tensor(b, C * batch, RSV_F32, s.tmix_x[i]));
        HK(new_tensor(b, HNN * batch, RSV_F32, s.rnn[i]));
        HK(new_tensor(b, C * batch, RSV_F32, s.cmix_x[i]));
    }
    HK(new_tensor(b, C * batch, RSV_F32, s.v_first));  // tensors start zeroed
    return 0;
}

void state_free(rsv_bundle *b, GpuState &s) {
    for (auto id : s.tmix_x) rsv_tensor_free(b->ctx, id);
    for (auto id : s.rnn) rsv_tensor_free(b->ctx, id);
    for (auto id : s.cmix_x) rsv_tensor_free(b->ctx, id);
    rsv_tensor_free(b->ctx, s.v_first);
    s.tmix_x.clear();
    s.rnn.clear();
    s.cmix_x.clear();
}

uint64_t state_len1(const rsv_bundle *b) {
    const rsv_model_info &I = b->info;
    return I.n_layer * (2 * I.n_embd + I.n_head * I.head_size * I.head_size) + I.n_embd;
}

// Slot-major serialisation, gpu_model.rs:3972-3990 / 4038-4095.
int state_back_slots(rsv_bundle *b, GpuState &s, uint64_t slot0, uint64_t nslots, float *out) {
    const rsv_model_info &I = b->info;
    const uint64_t C = I.n_embd, HNN = I.n_head * I.head_size * I.head_size, B = s.batch;
    std::vector<float> tx(C * B), rn(HNN * B), cx(C * B), vf(C * B);
    const uint64_t per = state_len1(b);
    for (uint64_t i = 0; i < I.n_layer; i++) {
        CK(rsv_download(b->ctx, s.tmix_x[i], tx.data(), C * B));
        CK(rsv_download(b->ctx, s.rnn[i], rn.data(), HNN * B));
        CK(rsv_download(b->ctx, s.cmix_x[i], cx.data(), C * B));
        for (uint64_t q = 0; q < nslots; q++) {
            const uint64_t sl = slot0 + q;
            float *o = out + q * per + i * (2 * C + HNN);
            memcpy(o, &tx[sl * C], C * 4);
            memcpy(o + C, &rn[sl * HNN], HNN * 4);
            memcpy(o + C + HNN, &cx[sl * C], C * 4);
        }
    }
    CK(rsv_download(b->ctx, s.v_first, vf.data(), C * B));
    for (uint64_t q = 0; q < nslots; q++) memcpy(out + q * per + I.n_layer * (2 * C + HNN), &vf[(slot0 + q) * C], C * 4);
    return 0;
}

int state_load_slots(rsv_bundle *b, GpuState &s, uint64_t slot0, uint64_t nslots, const float *data) {
    const rsv_model_info &I = b->info;
    const uint64_t C = I.n_embd, HNN = I.n_head * I.head_size * I.head_size;
    const uint64_t per = state_len1(b);
    for (uint64_t q = 0; q < nslots; q++) {
        const uint64_t sl = slot0 + q;
        const float *d = data + q * per;
        for (uint64_t i = 0; i < I.n_layer; i++) {
            const float *o = d + i * (2 * C + HNN);
            CK(rsv_upload_part(b->ctx, s.tmix_x[i], sl * C, o, C));
            CK(rsv_upload_part(b->ctx, s.rnn[i], sl * HNN, o + C, HNN));
            CK(rsv_upload_part(b->ctx, s.cmix_x[i], sl * C, o + C + HNN, C));
        }
        CK(rsv_upload_part(b->ctx, s.v_first, sl * C, d + I.n_layer * (2 * C + HNN), C));
    }
    return 0;
}

int state_reset(rsv_bundle *b, GpuState &s) {
    const uint64_t per = state_len1(b);
    std::vector<float> z(per * s.batch, 0.0f);
    return state_load_slots(b, s, 0, s.batch, z.data());
}

// ------------------------------------------------------------ decode
int tile_model(rsv_bundle *b);

int get_bufs(rsv_bundle *b, uint64_t B, WorkBufs *&out) {
    auto it = b->bufs.find(B);
    if (it != b->bufs.end()) { out = &it->second; return 0; }
    const rsv_model_info &I = b->info;
    const uint64_t C = I.n_embd;
    WorkBufs w;
    w.batch = B;
    uint32_t *c_ids[] = {&w.x, &w.xr, &w.xw, &w.xk, &w.xv, &w.xa, &w.xg, &w.r, &w.k, &w.v, &w.w, &w.a, &w.g, &w.yn, &w.xb, &w.xnorm, &w.ln1, &w.ln2};
    for (auto p : c_ids) HK(new_tensor(b, C * B, RSV_F32, *p));
    HK(new_tensor(b, I.v_mid * B, RSV_F32, w.vmid));
    HK(new_tensor(b, I.w_mid * B, RSV_F32, w.wmid));
    HK(new_tensor(b, I.a_mid * B, RSV_F32, w.amid));
    HK(new_tensor(b, I.g_mid * B, RSV_F32, w.gmid));
    HK(new_tensor(b, I.ffn * B, RSV_F32, w.r2));
    HK(new_tensor(b, I.vocab * B, RSV_F32, w.logits));
    HK(new_tensor(b, B, RSV_U32, w.token));
    w.mm = B >= kMmBatch;
    if (w.mm) {
        HK(tile_model(b));
        for (auto &m : w.mix16) HK(new_tensor(b, C * B, RSV_F16, m));
        HK(new_tensor(b, I.v_mid * B, RSV_F16, w.vmid16));
        HK(new_tensor(b, I.w_mid * B, RSV_F16, w.wmid16));
        HK(new_tensor(b, I.a_mid * B, RSV_F16, w.amid16));
        HK(new_tensor(b, I.g_mid * B, RSV_F16, w.gmid16));
        HK(new_tensor(b, C * B, RSV_F16, w.yg16));
        HK(new_tensor(b, C * B, RSV_F16, w.xb16));
        HK(new_tensor(b, I.ffn * B, RSV_F16, w.r216));
        HK(new_tensor(b, C * B, RSV_F16, w.xn16));
        // ffn.value k-slices of at most 2560 columns, each a 128-multiple
        // above the small-k kernel's 256 (10240 -> 4 x 2560)
        const uint64_t F = I.ffn, nsl = (F + 2559) / 2560;
        if (nsl <= 4 && F % (nsl * 128) == 0 && F / nsl > 256) {
            w.fv_nsl = (int)nsl;
            // also holds att.output's k-slices (atto_nsl: at most 4)
            HK(new_tensor(b, std::max<uint64_t>(nsl, 4) * C * B, RSV_F32, w.fvpart));
            HK(new_tensor(b, C * B, RSV_F32, w.xalt));
        }
    }
    out = &(b->bufs[B] = w);
    return 0;
}

int gemv_lin(rsv_bundle *b, const Linear &L, uint32_t x, uint32_t y, uint64_t B, int op, uint32_t g = NONE) {
    // op: 0 plain, 1 relu2, 2 add, 3 mul_add
    rsv_ctx *c = b->ctx;
    if (L.i8) {
        switch (op) {
            case 0: CK(rsv_gemv_int8_plain(c, &L.h, x, y, L.m, L.k, B)); break;
            case 1: CK(rsv_gemv_int8_relu2(c, &L.h, x, y, L.m, L.k, B)); break;
            case 2: CK(rsv_gemv_int8_add(c, &L.h, x, y, L.m, L.k, B)); break;
            default: CK(rsv_gemv_int8_mul_add(c, &L.h, x, g, y, L.m, L.k, B)); break;
        }
    } else {
        switch (op) {
            case 0: CK(rsv_gemv_f16(c, L.w16, x, y, L.m, L.k, B)); break;
            case 1: CK(rsv_gemv_f16_relu2(c, L.w16, x, y, L.m, L.k, B)); break;
            case 2: CK(rsv_gemv_f16_add(c, L.w16, x, y, L.m, L.k, B)); break;
            default: CK(rsv_gemv_f16_mul_add(c, L.w16, x, g, y, L.m, L.k, B)); break;
        }
    }
    return 0;
}

rsv_gemv_job lin_job(const Linear &L, uint32_t x, uint32_t y, int pro, int epi) {
    rsv_gemv_job j;
    memset(&j, 0xFF, sizeof j);
    j.w16 = L.i8 ? NONE : L.w16;
    j.w8 = L.i8 ? &L.h : nullptr;
    j.m = L.m;
    j.k = L.k;
    j.x = x;
    j.y = y;
    j.prologue = pro;
    j.epilogue = epi;
    return j;
}

rsv_gemv_job lora_job(uint32_t w, uint64_t m, uint64_t k, uint32_t x, uint32_t y, int pro, int epi) {
    Linear L;
    L.w16 = w;
    L.m = m;
    L.k = k;
    return lin_job(L, x, y, pro, epi);
}

void ln_mix(rsv_gemv_job &j, uint32_t gamma, uint32_t beta, uint32_t prev, uint32_t coef, uint32_t lnout) {
    j.gamma = gamma;
    j.beta = beta;
    j.prev = prev;
    j.coef = coef;
    j.lnout = lnout;
}

// The batched layer runs the LoRA-up chain and the WKV7 step as one launch
// (k_wkv7_lora_mb: the head's LoRA-up rows read once per 4 sessions) when
// the LoRA ranks sum to at most 512; RSV_WKV_LORA_MM=0 keeps the two launches (skinny GEMM + k_wkv7_decode).
bool mm_wkv_lora() {
    const char *e = getenv("RSV_WKV_LORA_MM");
    return !(e && e[0] == '0');
}

bool wkv_lora_ok(const rsv_model_info &I) {
    const char *e = getenv("RSV_WKV_LORA");
    if (e && e[0] == '0') return false;
    const uint64_t r[4] = {I.w_mid, I.a_mid, I.v_mid, I.g_mid};
    uint64_t sum = 0;
    for (uint64_t v : r) {
        if (v == 0 || v % 32 || v > 256) return false;
        sum += v;
    }
    return sum <= 1024 && I.head_size == 64;
}

// One layer for B slots with the op sequence of gpu_model.rs:2060-2392 /
// 1373-1566, fused into six launches (five when the LoRA-up chain and the
// WKV7 step share one launch, rsv_wkv7_lora_decode):
//   1. LN1 + token shift + r/k/v (int8) + LoRA-down projections  (state LN row -> ln1)
//   2. LoRA-up chain (w, a, v-first lerp, g)                      (ln1 -> tmix state)
//   3. WKV7 state update + GroupNorm + bonus
//   4. att.output: x += (y_norm * g) W^T
//   5. LN2 + token shift + ffn.key relu^2                          (state LN row -> ln2)
//   6. ffn.value: x += r2 W^T                                      (ln2 -> cmix state)
// The state writes are deferred by one launch so that no block of a launch
// reads a token-shift row another block of the same launch rewrites.
int forward_layer_fused(rsv_bundle *b, uint64_t i, WorkBufs &w, GpuState &s) {
    rsv_ctx *c = b->ctx;
    const rsv_model_info &I = b->info;
    const uint64_t C = I.n_embd, B = w.batch;
    Layer &L = b->layers[i];
    enum { P_NONE = 0, P_MUL = 1, P_SIG = 2, P_LN = 3, P_GN = 4 };
    enum { E_STORE = 0, E_RELU2 = 1, E_ADD = 2, E_TANH = 3, E_WDECAY = 4, E_SIGB = 5, E_VLERP = 6, E_STORE2 = 7 };
    if (L.rw.i8 != L.kw.i8 || L.rw.i8 != L.vw.i8)
        return herr("layer %llu: receptance/key/value must share one format", (unsigned long long)i);
    rsv_gemv_job j1[7] = {
        lin_job(L.rw, w.x, w.r, P_LN, E_STORE),
        lin_job(L.kw, w.x, w.k, P_LN, E_STORE),
        lin_job(L.vw, w.x, w.v, P_LN, i == 0 ? E_STORE2 : E_STORE),
        lora_job(L.v1, I.v_mid, C, w.x, w.vmid, P_LN, E_STORE),
        lora_job(L.w1, I.w_mid, C, w.x, w.wmid, P_LN, E_TANH),
        lora_job(L.a1, I.a_mid, C, w.x, w.amid, P_LN, E_STORE),
        lora_job(L.g1, I.g_mid, C, w.x, w.gmid, P_LN, E_STORE),
    };
    const uint32_t coef1[7] = {L.x_r, L.x_k, L.x_v, L.x_v, L.x_w, L.x_a, L.x_g};
    for (int q = 0; q < 7; q++) ln_mix(j1[q], L.ln1_w, L.ln1_b, s.tmix_x[i], coef1[q], q == 0 ? w.ln1 : NONE);
    if (i == 0) j1[2].p1 = s.v_first;  // v_first snapshot (gpu_model.rs:2200-2204)
    CK(rsv_gemv_multi(c, j1, 7, NONE, NONE, 0, B));

    // LoRA-up chain + WKV7 + GroupNorm in one launch (ranks multiples of 32),
    // its output y_norm*g going straight into att.output; RSV_WKV_LORA=0 keeps
    // the two launches below
    if (wkv_lora_ok(I)) {
        rsv_wkv_lora op;
        op.state = s.rnn[i];
        op.r = w.r; op.k = w.k; op.v = w.v; op.v_first = s.v_first;
        op.w_mid = w.wmid; op.a_mid = w.amid; op.v_mid = w.vmid; op.g_mid = w.gmid;
        op.w2 = L.w2; op.a2 = L.a2; op.v2 = L.v2; op.g2 = L.g2;
        op.w0 = L.w0; op.a0 = L.a0; op.v0 = L.v0; op.scale_w = b->scale_w;
        op.k_k = L.k_k; op.k_a = L.k_a; op.r_k = L.r_k; op.ln_x_w = L.lnx_w; op.ln_x_b = L.lnx_b;
        op.yg = w.yn;
        op.side_src = w.ln1;
        op.side_dst = s.tmix_x[i];
        op.n_head = I.n_head;
        op.w_rank = I.w_mid; op.a_rank = I.a_mid; op.v_rank = I.v_mid; op.g_rank = I.g_mid;
        op.eps = L2_EPS;
        op.gn_eps = GN_EPS;
        op.f16_io = 0;
        // one session: the head's rows over 4 blocks, the GroupNorm and the
        // gate in the att.output prologue (y raw in yn, bonus*v in a, gate in g)
        const bool split = B == 1;
        op.y_bonus = split ? w.a : NONE;
        op.y_gate = split ? w.g : NONE;
        CK(rsv_wkv7_lora_decode(c, &op, B));
        rsv_gemv_job j4 = lin_job(L.ow, w.yn, w.x, split ? P_GN : P_NONE, E_ADD);
        if (split) {
            j4.gamma = L.lnx_w;
            j4.beta = L.lnx_b;
            j4.prev = w.a;
            j4.xmul = w.g;
            j4.gn_eps = GN_EPS;
        }
        CK(rsv_gemv_multi(c, &j4, 1, NONE, NONE, 0, B));
    } else {
        rsv_gemv_job j2[4] = {
            lora_job(L.w2, C, I.w_mid, w.wmid, w.w, P_NONE, E_WDECAY),
            lora_job(L.a2, C, I.a_mid, w.amid, w.a, P_NONE, E_SIGB),
            lora_job(L.v2, C, I.v_mid, w.vmid, w.v, P_NONE, E_VLERP),
            lora_job(L.g2, C, I.g_mid, w.gmid, w.g, P_SIG, E_STORE),
        };
        j2[0].p0 = L.w0;
        j2[0].scale = b->scale_w;
        j2[1].p0 = L.a0;
        j2[2].p0 = L.v0;
        j2[2].p1 = s.v_first;
        CK(rsv_gemv_multi(c, j2, 4, w.ln1, s.tmix_x[i], C, B));

        CK(rsv_fuse_ka_dplr_norm_batch(c, s.rnn[i], w.k, L.k_k, w.a, L.k_a, w.r, w.v, w.w, L.lnx_w, L.lnx_b, L.r_k, NONE,
                                       NONE, w.yn, I.n_head, I.head_size, L2_EPS, GN_EPS, B));

        rsv_gemv_job j4 = lin_job(L.ow, w.yn, w.x, P_MUL, E_ADD);
        j4.xmul = w.g;
        CK(rsv_gemv_multi(c, &j4, 1, NONE, NONE, 0, B));
    }

    rsv_gemv_job j5 = lin_job(L.fk, w.x, w.r2, P_LN, E_RELU2);
    ln_mix(j5, L.ln2_w, L.ln2_b, s.cmix_x[i], L.ffn_x_k, w.ln2);
    CK(rsv_gemv_multi(c, &j5, 1, NONE, NONE, 0, B));

    if (L.fv_tiled != NONE && ffn_sparse_requested()) {
        // x += r2 V over the non-zero r2 rows only, then the token-shift row into the state
        CK(rsv_ffn_value_sparse_add_batch(c, L.fv_tiled, w.r2, w.x, C, I.ffn, B));
        CK(rsv_copy_device(c, w.ln2, s.cmix_x[i]));
        return 0;
    }
    rsv_gemv_job j6 = lin_job(L.fv, w.r2, w.x, P_NONE, E_ADD);
    CK(rsv_gemv_multi(c, &j6, 1, w.ln2, s.cmix_x[i], C, B));
    return 0;
}

// The same layer through the reference's trait-op sequence, one op per
// ComputeBackend method (kept for A/B checks; RSV_DECODE_TRAIT_OPS=1).
int forward_layer_ops(rsv_bundle *b, uint64_t i, WorkBufs &w, GpuState &s) {
    rsv_ctx *c = b->ctx;
    const rsv_model_info &I = b->info;
    const uint64_t C = I.n_embd, B = w.batch;
    Layer &L = b->layers[i];
    CK(rsv_norm_lerp6_batch(c, w.x, s.tmix_x[i], L.ln1_w, L.ln1_b, L.x_r, L.x_w, L.x_k, L.x_v, L.x_a, L.x_g, w.xr,
                            w.xw, w.xk, w.xv, w.xa, w.xg, C, LN_EPS, B));
    if (L.rw.i8 && L.kw.i8 && L.vw.i8) {
        CK(rsv_gemv_int8_rkv_stage1_batch(c, &L.rw.h, &L.kw.h, &L.vw.h, L.v1, L.w1, L.a1, L.g1, w.xr, w.xk, w.xv, w.xw,
                                          w.xa, w.xg, w.r, w.k, w.v, w.vmid, w.wmid, w.amid, w.gmid, C, I.v_mid,
                                          I.w_mid, I.a_mid, I.g_mid, B));
    } else if (!L.rw.i8 && !L.kw.i8 && !L.vw.i8) {
        CK(rsv_gemv_rkv_stage1_batch(c, L.rw.w16, L.kw.w16, L.vw.w16, L.v1, L.w1, L.a1, L.g1, w.xr, w.xk, w.xv, w.xw,
                                     w.xa, w.xg, w.r, w.k, w.v, w.vmid, w.wmid, w.amid, w.gmid, C, I.v_mid, I.w_mid,
                                     I.a_mid, I.g_mid, B));
    } else {
        return herr("layer %llu: receptance/key/value must share one format", (unsigned long long)i);
    }
    if (i == 0) CK(rsv_copy_device(c, w.v, s.v_first));  // v_first snapshot (gpu_model.rs:2200-2204)
    CK(rsv_gemv_lowrank_chain4_batch(c, L.w2, L.a2, L.v2, L.g2, w.wmid, w.amid, w.vmid, w.gmid, L.w0, L.a0, L.v0,
                                     b->scale_w, s.v_first, w.w, w.a, w.v, w.g, C, I.w_mid, I.a_mid, I.v_mid, I.g_mid,
                                     B));
    CK(rsv_fuse_ka_dplr_norm_batch(c, s.rnn[i], w.k, L.k_k, w.a, L.k_a, w.r, w.v, w.w, L.lnx_w, L.lnx_b, L.r_k, NONE,
                                   NONE, w.yn, I.n_head, I.head_size, L2_EPS, GN_EPS, B));
    HK(gemv_lin(b, L.ow, w.yn, w.x, B, 3, w.g));
    CK(rsv_cmix_norm_lerp_batch(c, w.x, s.cmix_x[i], L.ln2_w, L.ln2_b, L.ffn_x_k, w.xb, C, LN_EPS, B));
    HK(gemv_lin(b, L.fk, w.xb, w.r2, B, 1));
    HK(gemv_lin(b, L.fv, w.r2, w.x, B, 2));
    return 0;
}

rsv_mm_job mm_job(const Linear &L, uint32_t x, uint32_t y, int epi) {
    rsv_mm_job j;
    memset(&j, 0xFF, sizeof j);
    j.tiled = L.tiled ? 1 : 0;
    j.w16 = L.i8 ? NONE : (L.tiled ? L.t16 : L.w16);
    j.w8 = L.i8 ? (L.tiled ? &L.ht : &L.h) : nullptr;
    j.n = L.m;
    j.k = L.k;
    j.x = x;
    j.y = y;
    j.epilogue = epi;
    return j;
}

// A prefill GEMM job on the row-major weights (rsv_gemm_multi).
// fp16 prefill copies of the int8 matrices are made and used unless
// RSV_PREFILL_F16=0 (read at each use, so a process can compare both)
bool use_p16() {
    const char *e = getenv("RSV_PREFILL_F16");
    return !(e && e[0] == '0');
}

// Row-major GEMM job of a linear; an int8 matrix with an fp16 prefill copy
// runs on the copy (the same fp16 values the int8 loader would make).
rsv_mm_job gemm_job(const Linear &L, uint32_t x, uint32_t y, int epi) {
    rsv_mm_job j;
    memset(&j, 0xFF, sizeof j);
    j.tiled = 0;
    const bool i8 = L.i8 && (L.p16 == NONE || !use_p16());
    j.w16 = i8 ? NONE : L.i8 ? L.p16 : L.w16;
    j.w8 = i8 ? &L.h : nullptr;
    j.n = L.m;
    j.k = L.k;
    j.x = x;
    j.y = y;
    j.epilogue = epi;
    return j;
}

int tile_linear(rsv_bundle *b, Linear &L) {
    if (L.tiled) return 0;
    if (L.i8) {
        L.ht = L.h;
        CK(rsv_tile_weights(b->ctx, L.h.idx, L.m, L.k, 1, &L.ht.idx));
        CK(rsv_tile_weights(b->ctx, L.h.sz, L.m, L.k, 4, &L.ht.sz));
    } else {
        CK(rsv_tile_weights(b->ctx, L.w16, L.m, L.k, 2, &L.t16));
    }
    L.tiled = true;
    return 0;
}

// MFMA-tiled weight copies for the batched decode path (extra device memory
// of the size of the weights; HBM is not the constraint on this GPU).
int tile_model(rsv_bundle *b) {
    if (b->tiled) return 0;
    const rsv_model_info &I = b->info;
    const uint64_t C = I.n_embd;
    for (auto &L : b->layers) {
        auto lora = [&](Linear &V, uint32_t w, uint64_t m, uint64_t k) { V.w16 = w; V.m = m; V.k = k; return tile_linear(b, V); };
        HK(lora(L.lw1, L.w1, I.w_mid, C));
        HK(lora(L.lw2, L.w2, C, I.w_mid));
        HK(lora(L.la1, L.a1, I.a_mid, C));
        HK(lora(L.la2, L.a2, C, I.a_mid));
        HK(lora(L.lv1, L.v1, I.v_mid, C));
        HK(lora(L.lv2, L.v2, C, I.v_mid));
        HK(lora(L.lg1, L.g1, I.g_mid, C));
        HK(lora(L.lg2, L.g2, C, I.g_mid));
        for (Linear *p : {&L.rw, &L.kw, &L.vw, &L.ow, &L.fk, &L.fv}) HK(tile_linear(b, *p));
    }
    HK(tile_linear(b, b->head));
    CK(rsv_synchronize(b->ctx));
    b->tiled = true;
    return 0;
}

// Batched layer (B >= kMmBatch): the same math with fp16 activation
// operands so every weight product runs on matrix cores, each weight byte
// streamed once per step for all sessions.
// A weight product added to the residual row on the matrix-core path: as
// nsl k-slice partial sums left in fvpart for the next LayerNorm
// (ln_mix_mm), or, with nsl = 0, one GEMM adding into the row.
int resid_gemm_mm(rsv_bundle *b, const Linear &L, uint32_t xin, WorkBufs &w, int nsl) {
    if (nsl) {
        rsv_mm_job j = mm_job(L, xin, w.fvpart, 0);
        CK(rsv_gemm_skinny_kslices(b->ctx, &j, nsl, w.batch));
        w.pend = nsl;
        return 0;
    }
    rsv_mm_job j = mm_job(L, xin, w.xcur, 2);
    CK(rsv_gemm_skinny(b->ctx, &j, 1, w.batch));
    return 0;
}

// rsv_ln_mix_f16 of the residual row, first adding pending k-slice sums
// (the summed row goes to the other residual buffer, which becomes xcur).
int ln_mix_mm(rsv_bundle *b, WorkBufs &w, uint32_t state, uint32_t gamma, uint32_t beta, const uint32_t *coef,
              const uint32_t *out, uint64_t nout, bool keep_row = true) {
    rsv_ctx *c = b->ctx;
    const uint64_t C = b->info.n_embd;
    if (w.pend) {
        const uint32_t dst = !keep_row ? NONE : w.xcur == w.x ? w.xalt : w.x;
        CK(rsv_ln_mix_f16_acc(c, w.xcur, w.fvpart, w.pend, dst, state, gamma, beta, coef, out, nout, C, LN_EPS,
                              w.batch));
        if (keep_row) w.xcur = dst;
        w.pend = 0;
        return 0;
    }
    CK(rsv_ln_mix_f16(c, w.xcur, state, gamma, beta, coef, out, nout, C, LN_EPS, w.batch));
    return 0;
}

// att.output k-slices on the matrix-core path (its 2560 rows are only 80
// row tiles: two slices spread them over twice the CUs, the slice sums
// going to LN2).
int atto_nsl(const Linear &L) {
    const int n = 2;
    if ( L.k % (uint64_t)(n * 128) != 0 || L.k / n <= 256 || L.k / n > 2560 || (L.k / n) % 64) return 0;
    return n;
}

int forward_layer_mm(rsv_bundle *b, uint64_t i, WorkBufs &w, GpuState &s) {
    rsv_ctx *c = b->ctx;
    const rsv_model_info &I = b->info;
    const uint64_t C = I.n_embd, B = w.batch;
    Layer &L = b->layers[i];
    enum { G_STORE = 0, G_BIAS = 1, G_ADD = 2, G_RELU2 = 3, G_TANH = 4, G_WDECAY = 5, G_SIGB = 6, G_VLERP = 7, G_SIG = 8 };
    const uint32_t coef6[6] = {L.x_r, L.x_w, L.x_k, L.x_v, L.x_a, L.x_g};
    HK(ln_mix_mm(b, w, s.tmix_x[i], L.ln1_w, L.ln1_b, coef6, w.mix16, 6));
    const uint32_t xr = w.mix16[0], xw = w.mix16[1], xk = w.mix16[2], xv = w.mix16[3], xa = w.mix16[4], xg = w.mix16[5];
    rsv_mm_job j1[7] = {
        mm_job(L.rw, xr, w.r, G_STORE), mm_job(L.kw, xk, w.k, G_STORE), mm_job(L.vw, xv, w.v, G_STORE),
        mm_job(L.lv1, xv, w.vmid16, G_STORE), mm_job(L.lw1, xw, w.wmid16, G_TANH),
        mm_job(L.la1, xa, w.amid16, G_STORE), mm_job(L.lg1, xg, w.gmid16, G_SIG),
    };
    if (i == 0) j1[2].y2 = s.v_first;  // v_first snapshot (gpu_model.rs:2200-2204)
    CK(rsv_gemm_skinny(c, j1, 7, B));
    if (wkv_lora_ok(I) && mm_wkv_lora() && I.w_mid + I.a_mid + I.v_mid + I.g_mid <= 512) {
        // LoRA-up chain + WKV7 + GroupNorm in one launch, fp16 in and out
        rsv_wkv_lora op;
        op.state = s.rnn[i];
        op.r = w.r; op.k = w.k; op.v = w.v; op.v_first = s.v_first;
        op.w_mid = w.wmid16; op.a_mid = w.amid16; op.v_mid = w.vmid16; op.g_mid = w.gmid16;
        op.w2 = L.w2; op.a2 = L.a2; op.v2 = L.v2; op.g2 = L.g2;
        op.w0 = L.w0; op.a0 = L.a0; op.v0 = L.v0; op.scale_w = b->scale_w;
        op.k_k = L.k_k; op.k_a = L.k_a; op.r_k = L.r_k; op.ln_x_w = L.lnx_w; op.ln_x_b = L.lnx_b;
        op.yg = w.yg16;
        op.side_src = op.side_dst = NONE;
        op.n_head = I.n_head;
        op.w_rank = I.w_mid; op.a_rank = I.a_mid; op.v_rank = I.v_mid; op.g_rank = I.g_mid;
        op.eps = L2_EPS;
        op.gn_eps = GN_EPS;
        op.f16_io = 1;
        op.y_bonus = op.y_gate = NONE;
        CK(rsv_wkv7_lora_decode(c, &op, B));
        HK(resid_gemm_mm(b, L.ow, w.yg16, w, w.fv_nsl ? atto_nsl(L.ow) : 0));
        HK(ln_mix_mm(b, w, s.cmix_x[i], L.ln2_w, L.ln2_b, &L.ffn_x_k, &w.xb16, 1));
        rsv_mm_job j5 = mm_job(L.fk, w.xb16, w.r216, G_RELU2);
        CK(rsv_gemm_skinny(c, &j5, 1, B));
        return resid_gemm_mm(b, L.fv, w.r216, w, w.fv_nsl);
    }
    rsv_mm_job j2[4] = {
        mm_job(L.lw2, w.wmid16, w.w, G_WDECAY), mm_job(L.la2, w.amid16, w.a, G_SIGB),
        mm_job(L.lv2, w.vmid16, w.v, G_VLERP), mm_job(L.lg2, w.gmid16, w.g, G_STORE),
    };
    j2[0].bias = L.w0;
    j2[0].scale = b->scale_w;
    j2[1].bias = L.a0;
    j2[2].bias = L.v0;
    j2[2].aux = s.v_first;
    CK(rsv_gemm_skinny(c, j2, 4, B));
    CK(rsv_wkv7_decode_ex(c, s.rnn[i], w.k, L.k_k, w.a, L.k_a, w.r, w.v, w.w, L.lnx_w, L.lnx_b, L.r_k, NONE, w.g,
                          w.yg16, I.n_head, I.head_size, L2_EPS, GN_EPS, B));
    HK(resid_gemm_mm(b, L.ow, w.yg16, w, w.fv_nsl ? atto_nsl(L.ow) : 0));
    HK(ln_mix_mm(b, w, s.cmix_x[i], L.ln2_w, L.ln2_b, &L.ffn_x_k, &w.xb16, 1));
    rsv_mm_job j5 = mm_job(L.fk, w.xb16, w.r216, G_RELU2);
    CK(rsv_gemm_skinny(c, &j5, 1, B));
    return resid_gemm_mm(b, L.fv, w.r216, w, w.fv_nsl);
}

bool use_trait_ops() {
    const char *e = getenv("RSV_DECODE_TRAIT_OPS");
    return e && e[0] && e[0] != '0';
}

int forward_layer(rsv_bundle *b, uint64_t i, WorkBufs &w, GpuState &s) {
    if (use_trait_ops()) return forward_layer_ops(b, i, w, s);
    if (w.mm) return forward_layer_mm(b, i, w, s);
    return forward_layer_fused(b, i, w, s);
}

// gather -> layers -> ln_out -> head (gpu_model.rs:1879-1913 minus the
// sampler).
// gather = false: x already holds the tokens' embedding rows (the greedy
// self-loop's fused argmax / record / gather launch wrote them).
int decode_step(rsv_bundle *b, WorkBufs &w, GpuState &s, bool gather = true) {
    rsv_ctx *c = b->ctx;
    const rsv_model_info &I = b->info;
    if (gather) CK(rsv_gather_rows_device_f16(c, b->emb_ln, w.x, w.token, I.n_embd, w.batch));
    w.xcur = w.x;
    w.pend = 0;
    for (uint64_t i = 0; i < I.n_layer; i++) HK(forward_layer(b, i, w, s));
    if (w.mm && !use_trait_ops()) {
        HK(ln_mix_mm(b, w, NONE, b->ln_out_w, b->ln_out_b, nullptr, &w.xn16, 1, false));
        rsv_mm_job jh = mm_job(b->head, w.xn16, w.logits, 0);
        CK(rsv_gemm_skinny(c, &jh, 1, w.batch));
        return 0;
    }
    CK(rsv_norm(c, w.x, b->ln_out_w, b->ln_out_b, w.xnorm, I.n_embd, 1, LN_EPS, w.batch));
    HK(gemv_lin(b, b->head, w.xnorm, w.logits, w.batch, 0));
    return 0;
}

// ------------------------------------------------------------ prefill
int get_seq(rsv_bundle *b, uint64_t T, uint64_t nseg, SeqBufs &q) {
    const rsv_model_info &I = b->info;
    const uint64_t C = I.n_embd;
    if (T > q.cap) {
        uint32_t *f32s[] = {&q.x, &q.r, &q.k, &q.v, &q.w, &q.a, &q.g, &q.vf, &q.yn};
        uint32_t *f16s[] = {&q.mix[0], &q.mix[1], &q.mix[2], &q.mix[3], &q.mix[4], &q.mix[5], &q.yg, &q.xb};
        for (auto p : f32s) { if (*p != NONE) rsv_tensor_free(b->ctx, *p); HK(new_tensor(b, T * C, RSV_F32, *p)); }
        for (auto p : f16s) { if (*p != NONE) rsv_tensor_free(b->ctx, *p); HK(new_tensor(b, T * C, RSV_F16, *p)); }
        struct { uint32_t *id; uint64_t n; int dt; } more[] = {
            {&q.r2, T * I.ffn, RSV_F16}, {&q.vmid, T * I.v_mid, RSV_F16}, {&q.wmid, T * I.w_mid, RSV_F16},
            {&q.amid, T * I.a_mid, RSV_F16}, {&q.gmid, T * I.g_mid, RSV_F16}, {&q.tok, T, RSV_U32},
            {&q.row_prev, T, RSV_U32}, {&q.bonus, T * I.n_head, RSV_F32}};
        for (auto &m : more) { if (*m.id != NONE) rsv_tensor_free(b->ctx, *m.id); HK(new_tensor(b, m.n, m.dt, *m.id)); }
        q.cap = T;
    }
    if (nseg > q.segcap) {
        uint32_t *u32s[] = {&q.seg_start, &q.seg_len, &q.seg_slot, &q.seg_last, &q.seg_iota};
        for (auto p : u32s) { if (*p != NONE) rsv_tensor_free(b->ctx, *p); HK(new_tensor(b, nseg, RSV_U32, *p)); }
        uint32_t *f32s[] = {&q.xlast, &q.xnorm};
        for (auto p : f32s) { if (*p != NONE) rsv_tensor_free(b->ctx, *p); HK(new_tensor(b, nseg * C, RSV_F32, *p)); }
        if (q.logits != NONE) rsv_tensor_free(b->ctx, q.logits);
        HK(new_tensor(b, nseg * I.vocab, RSV_F32, q.logits));
        std::vector<uint32_t> iota(nseg);
        for (uint64_t i = 0; i < nseg; i++) iota[i] = (uint32_t)i;
        CK(rsv_upload_u32(b->ctx, q.seg_iota, iota.data(), nseg));
        q.segcap = nseg;
    }
    return 0;
}

struct Seg {
    const uint32_t *tok;
    uint64_t len;
    uint64_t slot;
};

int gemm_lin(rsv_bundle *b, const Linear &L, uint32_t a, uint32_t c, uint64_t m, int epi) {
    const bool i8 = L.i8 && (L.p16 == NONE || !use_p16());
    CK(rsv_gemm_ex(b->ctx, a, i8 ? NONE : L.i8 ? L.p16 : L.w16, i8 ? &L.h : nullptr, c, m, L.m, L.k, epi, NONE, NONE,
                   NONE));
    return 0;
}

// fp16 copies of the int8 layer matrices for the prefill GEMM, dequantised
// with the roundings of the GEMM's own int8 loader (model.rs:234-252: the
// product and the sum each rounded to fp32, then to fp16), so prefill gives
// the same bits with or without them.  The copies take twice the int8 bytes
// (5.2 GB for the 3B shape); RSV_PREFILL_F16=0 keeps the int8 loader.
int prefill_weights(rsv_bundle *b) {
    if (b->p16 || !use_p16()) return 0;
    b->p16 = true;
    for (auto &L : b->layers)
        for (Linear *p : {&L.rw, &L.kw, &L.vw, &L.ow, &L.fk, &L.fv}) {
            if (!p->i8 || p->p16 != NONE) continue;
            uint32_t id;
            CK(rsv_tensor_create(b->ctx, p->m * p->k, RSV_F16, &id));
            CK(rsv_dequant_int8_to_f16(b->ctx, &p->h, id, p->m, p->k));
            p->p16 = id;
        }
    return 0;
}

// PREFILL_GRAPH=1: prefill chunks replay a HIP graph captured for their
// shape (the reference's CUDA prefill graph, gpu_model.rs:2440-2450).
bool prefill_graph_on() {
    const char *e = getenv("PREFILL_GRAPH");
    return e && e[0] == '1' && e[1] == 0;
}

// Packed prefill of non-empty segments into state slots; logits (optional)
// receives nseg*vocab floats (last token of each segment).  With head set
// and no host buffer the logits stay on the device in b->seq.logits.
// Pipelined prefill (prefill_chunks): consecutive packed chunks on
// alternating lanes (streams) of the context, each lane with its own
// buffers.  Chunk c depends on chunk c-1 only through the state it carries:
// per layer i, the LN1 token-shift rows (tmix_x), the WKV state (rnn) and the
// LN2 token-shift rows (cmix_x).  So chunk c waits, per layer, for the
// previous chunk's event after the op that leaves each of them (events 3i,
// 3i+1, 3i+2), and everything else of the two chunks overlaps: the scan of
// one chunk (VALU and LDS bound) runs beside the LN, LoRA-up and GEMM
// launches of the other.  Event kLaneTail closes a chunk.
struct LaneHooks {
    int lane = 0;             // lane this chunk runs on
    int prev_lane = 0;        // lane of the previous chunk
    bool prev_layers = false; // wait for the previous chunk's per-layer events
    bool other_tail = false;  // first wait for the other lane's last chunk to end
};
constexpr int kLaneTail = 255;

int prefill(rsv_bundle *b, GpuState &s, const std::vector<Seg> &segs, float *logits, bool head = false,
            const LaneHooks *lh = nullptr) {
    rsv_ctx *c = b->ctx;
    const rsv_model_info &I = b->info;
    const uint64_t C = I.n_embd, H = I.n_head, N = I.head_size;
    uint64_t T = 0;
    for (auto &g : segs) {
        if (g.len == 0) return herr("prefill: empty segment");
        if (g.slot >= s.batch) return herr("prefill: slot %llu >= batch %llu", (unsigned long long)g.slot, (unsigned long long)s.batch);
        T += g.len;
    }
    const uint64_t S = segs.size();
    if (S == 0) return 0;
    // Short packed batches (decode tokens of ragged serving, small prompt
    // chunks) run their weight products on the batched-decode matrix-core
    // kernel, which streams each weight once per 64 rows; longer ones on the
    // prefill GEMM.
    const bool small = T <= kSmallPrefill;
    // the LoRA matrices' descriptors (and the batched path's tiled copies,
    // which decode needs next) come from tile_model on both paths
    HK(tile_model(b));
    if (!small) HK(prefill_weights(b));
    SeqBufs &q = lh && lh->lane == 1 ? b->seq2 : b->seq;
    HK(get_seq(b, T, S, q));
    std::vector<uint32_t> tok(T), prev(T), st(S), ln(S), sl(S), last(S);
    uint64_t pos = 0;
    for (uint64_t g = 0; g < S; g++) {
        st[g] = (uint32_t)pos;
        ln[g] = (uint32_t)segs[g].len;
        sl[g] = (uint32_t)segs[g].slot;
        for (uint64_t t = 0; t < segs[g].len; t++) {
            if (segs[g].tok[t] >= I.vocab) return herr("prefill: token %u >= vocab", segs[g].tok[t]);
            tok[pos + t] = segs[g].tok[t];
            prev[pos + t] = t == 0 ? (0x80000000u | (uint32_t)segs[g].slot) : (uint32_t)(pos + t - 1);
        }
        pos += segs[g].len;
        last[g] = (uint32_t)(pos - 1);
    }
    CK(rsv_upload_u32(c, q.tok, tok.data(), T));
    CK(rsv_upload_u32(c, q.row_prev, prev.data(), T));
    CK(rsv_upload_u32(c, q.seg_start, st.data(), S));
    CK(rsv_upload_u32(c, q.seg_len, ln.data(), S));
    CK(rsv_upload_u32(c, q.seg_slot, sl.data(), S));
    CK(rsv_upload_u32(c, q.seg_last, last.data(), S));

    // Everything from the embedding gather to the head is enqueue-only, so
    // with PREFILL_GRAPH=1 it is captured once per (rows, segments, state,
    // head) and replayed for later chunks of the same shape
    // (gpu_model.rs:2440-2507); the uploads above and the logits download
    // below stay outside the graph.
    const bool want_head = logits || head;
    // the lane hooks: wait for the previous chunk's event k, record ours
    auto wait_prev = [&](int k) -> int {
        if (lh && lh->prev_layers) CK(rsv_lane_wait(c, lh->prev_lane, k));
        return 0;
    };
    auto record = [&](int k) -> int {
        if (lh) CK(rsv_lane_record(c, k));
        return 0;
    };
    auto enqueue = [&]() -> int {
        if (lh && lh->other_tail) CK(rsv_lane_wait(c, 1 - lh->lane, kLaneTail));
        CK(rsv_gather_rows_device_f16(c, b->emb_ln, q.x, q.tok, C, T));
        for (uint64_t i = 0; i < I.n_layer; i++) {
            Layer &L = b->layers[i];
            const uint32_t coef6[6] = {L.x_r, L.x_w, L.x_k, L.x_v, L.x_a, L.x_g};
            HK(wait_prev((int)(3 * i)));
            CK(rsv_seq_norm_mix(c, q.x, s.tmix_x[i], L.ln1_w, L.ln1_b, coef6, q.mix, 6, q.row_prev, T, C, LN_EPS));
            CK(rsv_seq_state_store(c, q.x, s.tmix_x[i], L.ln1_w, L.ln1_b, q.seg_last, q.seg_slot, S, C, LN_EPS));
            HK(record((int)(3 * i)));
            const uint32_t xr = q.mix[0], xw = q.mix[1], xk = q.mix[2], xv = q.mix[3], xa = q.mix[4], xg = q.mix[5];
            if (small) {
                rsv_mm_job j1[7] = {
                    mm_job(L.rw, xr, q.r, 0), mm_job(L.kw, xk, q.k, 0), mm_job(L.vw, xv, q.v, 0),
                    mm_job(L.lv1, xv, q.vmid, 0), mm_job(L.lw1, xw, q.wmid, 4),
                    mm_job(L.la1, xa, q.amid, 0), mm_job(L.lg1, xg, q.gmid, 8),
                };
                CK(rsv_gemm_skinny(c, j1, 7, T));
            } else {
                // r/k/v and the four LoRA-down products in one launch
                rsv_mm_job j1[7] = {
                    gemm_job(L.rw, xr, q.r, 0), gemm_job(L.kw, xk, q.k, 0), gemm_job(L.vw, xv, q.v, 0),
                    gemm_job(L.lv1, xv, q.vmid, 0), gemm_job(L.lw1, xw, q.wmid, 4),
                    gemm_job(L.la1, xa, q.amid, 0), gemm_job(L.lg1, xg, q.gmid, 8),
                };
                CK(rsv_gemm_multi(c, j1, 7, T));
            }
            if (i == 0) CK(rsv_copy_device(c, q.v, q.vf));
            if (small) {
                rsv_mm_job j2[4] = {mm_job(L.lw2, q.wmid, q.w, 5), mm_job(L.la2, q.amid, q.a, 6),
                                    mm_job(L.lv2, q.vmid, q.v, 7), mm_job(L.lg2, q.gmid, q.g, 0)};
                j2[0].bias = L.w0;
                j2[0].scale = b->scale_w;
                j2[1].bias = L.a0;
                j2[2].bias = L.v0;
                j2[2].aux = q.vf;
                CK(rsv_gemm_skinny(c, j2, 4, T));
            } else {
                // the LoRA-up chain in one launch
                rsv_mm_job j2[4] = {gemm_job(L.lw2, q.wmid, q.w, 5), gemm_job(L.la2, q.amid, q.a, 6),
                                    gemm_job(L.lv2, q.vmid, q.v, 7), gemm_job(L.lg2, q.gmid, q.g, 0)};
                j2[0].bias = L.w0;
                j2[0].scale = b->scale_w;
                j2[1].bias = L.a0;
                j2[2].bias = L.v0;
                j2[2].aux = q.vf;
                CK(rsv_gemm_multi(c, j2, 4, T));
            }
            HK(wait_prev((int)(3 * i + 1)));
            // each segment's layer-0 v of its last token is the slot's v_first
            // (written here, after the previous chunk's write to the same slot)
            if (i == 0) CK(rsv_copy_rows(c, q.vf, s.v_first, q.seg_last, q.seg_slot, S, C));
            CK(rsv_wkv7_seq_ragged_gate(c, s.rnn[i], q.r, q.w, q.k, q.v, q.a, L.k_k, L.k_a, L.r_k, L.lnx_w, L.lnx_b,
                                        q.g, q.yn, q.bonus, q.yg, q.seg_start, q.seg_len, q.seg_slot, S, T, H, N,
                                        GN_EPS));
            HK(record((int)(3 * i + 1)));
            if (small) {
                rsv_mm_job j4 = mm_job(L.ow, q.yg, q.x, 2);
                CK(rsv_gemm_skinny(c, &j4, 1, T));
            } else {
                HK(gemm_lin(b, L.ow, q.yg, q.x, T, 2));
            }
            const uint32_t coef1[1] = {L.ffn_x_k};
            HK(wait_prev((int)(3 * i + 2)));
            CK(rsv_seq_norm_mix(c, q.x, s.cmix_x[i], L.ln2_w, L.ln2_b, coef1, &q.xb, 1, q.row_prev, T, C, LN_EPS));
            CK(rsv_seq_state_store(c, q.x, s.cmix_x[i], L.ln2_w, L.ln2_b, q.seg_last, q.seg_slot, S, C, LN_EPS));
            HK(record((int)(3 * i + 2)));
            if (small) {
                rsv_mm_job j5 = mm_job(L.fk, q.xb, q.r2, 3);
                CK(rsv_gemm_skinny(c, &j5, 1, T));
                rsv_mm_job j6 = mm_job(L.fv, q.r2, q.x, 2);
                CK(rsv_gemm_skinny(c, &j6, 1, T));
            } else {
                HK(gemm_lin(b, L.fk, q.xb, q.r2, T, 3));
                HK(gemm_lin(b, L.fv, q.r2, q.x, T, 2));
            }
        }

        if (want_head) {
            CK(rsv_copy_rows(c, q.x, q.xlast, q.seg_last, q.seg_iota, S, C));
            CK(rsv_norm(c, q.xlast, b->ln_out_w, b->ln_out_b, q.xnorm, C, 1, LN_EPS, S));
            HK(gemv_lin(b, b->head, q.xnorm, q.logits, S, 0));
        }
        HK(record(kLaneTail));
        return 0;
    };
    if (prefill_graph_on() && !lh) {
        const uint64_t key = T | (S << 24) | ((uint64_t)want_head << 47) | ((s.serial & 0xFFFF) << 48);
        int valid = 0;
        CK(rsv_prefill_graph_valid(c, key, &valid));
        if (!valid) {
            CK(rsv_prefill_graph_begin(c, key));
            const int rc = enqueue();
            const int end_rc = rsv_prefill_graph_end(c);
            if (rc || end_rc) {
                rsv_clear_cache(c);  // no partial graph stays behind
                return rc ? rc : herr("prefill graph: %s", rsv_last_error());
            }
        }
        CK(rsv_prefill_graph_replay(c));
    } else {
        HK(enqueue());
    }
    if (logits) CK(rsv_download(c, q.logits, logits, S * I.vocab));
    else if (!head && !lh) CK(rsv_synchronize(c));
    return 0;
}

// Runs packed chunks in order (the state carried from each to the next),
// pipelined over two lanes when there are several; logits (optional) gets
// the head's rows of the last chunk's segments.  Chunks of at most
// kSmallPrefill rows, and the head's GEMV, run kernels that share one
// context-wide split-K work area: such a chunk stays on its predecessor's
// lane and first waits for the other lane's last chunk to end, so that no
// two of them are ever in flight.
int prefill_chunks(rsv_bundle *b, GpuState &s, const std::vector<std::vector<Seg>> &chunks, float *logits) {
    rsv_ctx *c = b->ctx;
    const bool lanes = b->prefill_lanes > 1 && chunks.size() > 1 && !prefill_graph_on() &&
                       3 * b->info.n_layer <= (uint64_t)kLaneTail;
    if (!lanes) {
        for (size_t k = 0; k < chunks.size(); k++) HK(prefill(b, s, chunks[k], k + 1 == chunks.size() ? logits : nullptr));
        return 0;
    }
    // every buffer at its final size before anything is in flight (a
    // reallocation would free memory the other lane still uses)
    uint64_t maxT = 0, maxS = 0;
    for (auto &ch : chunks) {
        uint64_t T = 0;
        for (auto &g : ch) T += g.len;
        maxT = std::max(maxT, T);
        maxS = std::max<uint64_t>(maxS, ch.size());
    }
    HK(tile_model(b));
    if (maxT > kSmallPrefill) HK(prefill_weights(b));
    HK(get_seq(b, maxT, maxS, b->seq));
    HK(get_seq(b, maxT, maxS, b->seq2));
    bool used[2] = {false, false};
    int rc = 0, prev_lane = -1;
    for (size_t k = 0; k < chunks.size() && !rc; k++) {
        uint64_t T = 0;
        for (auto &g : chunks[k]) T += g.len;
        const bool last = k + 1 == chunks.size();
        const bool shared_ws = T <= kSmallPrefill || (last && logits);
        LaneHooks h;
        h.lane = prev_lane < 0 ? 0 : T <= kSmallPrefill ? prev_lane : 1 - prev_lane;
        h.prev_lane = prev_lane < 0 ? 0 : prev_lane;
        h.prev_layers = prev_lane >= 0 && prev_lane != h.lane;
        h.other_tail = shared_ws && used[1 - h.lane];
        if (rsv_lane_select(c, h.lane)) {
            rc = herr("prefill lanes: %s", rsv_last_error());
            break;
        }
        used[h.lane] = true;
        rc = prefill(b, s, chunks[k], last ? logits : nullptr, false, &h);
        prev_lane = h.lane;
    }
    // join: launches go to lane 0 again, after lane 1's last chunk (also after
    // a failure, so that nothing of this call is left in flight)
    // (rc set: the host error text is already set by the failing call)
    int rb = rsv_lane_select(c, 0);
    if (!rb && used[1]) rb = rsv_lane_wait(c, 1, kLaneTail);
    if (!rb) rb = rsv_synchronize(c);
    if (rc) return -1;
    if (rb) return herr("prefill lanes: %s", rsv_last_error());
    return 0;
}

// Rows of one packed prefill dispatch.  Larger chunks fill the GEMM tile
// rounds better (at 12,288 rows att.output and ffn.value take 768 256x160
// tiles, 3 whole rounds of 256 CUs) and halve the launches per token; the
// configs[4] ragged prefill measured 98.2k tok/s at 4096, 99.9k at 8192,
// 101.9k at 12,288 and 100.2k at 16,384.
constexpr uint64_t kMaxChunk = 12288;

// Water filling: the largest piece length L with sum_i min(rem_i, L) <= cap
// (every remaining length when they all fit).  Packing one piece of at most
// L tokens per unfinished prompt keeps a chunk's longest piece, and so its
// sequential WKV scan, as short as the chunk size allows.
static uint64_t water_fill(const std::vector<uint64_t> &rem, uint64_t cap) {
    uint64_t hi = 0, all = 0;
    for (uint64_t r : rem) {
        hi = std::max(hi, r);
        all += r;
    }
    if (all <= cap || hi == 0) return hi;
    uint64_t lo = 0;
    while (lo < hi) {
        const uint64_t mid = (lo + hi + 1) / 2;
        uint64_t sum = 0;
        for (uint64_t r : rem) sum += std::min(r, mid);
        if (sum <= cap) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}

// Single-session prefill in chunks of at most prefill_chunk tokens.
int seq_single(rsv_bundle *b, GpuState &s, uint64_t slot, const uint32_t *tokens, uint64_t n, float *logits) {
    if (n == 0) return herr("infer_seq: empty token list");
    const uint64_t ch = b->prefill_chunk;
    std::vector<std::vector<Seg>> chunks;
    for (uint64_t off = 0; off < n; off += ch) {
        const uint64_t len = n - off < ch ? n - off : ch;
        chunks.push_back({{tokens + off, len, slot}});
    }
    return prefill_chunks(b, s, chunks, logits);
}

// ------------------------------------------------------------ ragged serving
// Continuous batching over the B slots of a State (the scheduler of the
// north star; the reference has only padded batch prefill,
// gpu_model.rs:914-997, and a batch decode self-loop, 1639-1781).  A step is
// one packed dispatch through the layers: one decode token for every slot
// that is generating, then chunks of the prompts still being prefilled (slots
// in order, a prompt split over steps when it does not fit), `budget` tokens
// in all.  A decode token is a segment of length 1, so prefill and decode
// share every launch.  After the dispatch the GPU sampler draws the next
// token of every slot whose prompt or previous token ended in the step; the
// k-th token of slot q is drawn with seed seeds[q] + k.
struct ServeSlot {
    const uint32_t *prompt = nullptr;
    uint64_t plen = 0, done = 0;  // prompt tokens consumed
    uint64_t gen = 0;             // tokens sampled
    uint32_t last = 0;            // last sampled token (next decode input)
};

int serve_ragged(rsv_bundle *b, GpuState &s, const uint32_t *tokens, const uint64_t *lens, uint64_t decode_len,
                 const rsv_sampler_params *sp, const uint32_t *seeds, uint64_t budget, uint32_t *out,
                 rsv_serve_step *steps, uint64_t max_steps, uint64_t *nsteps, float *sampled_logits) {
    rsv_ctx *c = b->ctx;
    const rsv_model_info &I = b->info;
    const uint64_t B = s.batch, V = I.vocab;
    if (budget == 0 || budget > kMaxChunk) return herr("serve_ragged: budget must be 1..%llu", (unsigned long long)kMaxChunk);
    if (decode_len == 0) return herr("serve_ragged: decode_len must be >= 1");
    if (budget < B) return herr("serve_ragged: budget %llu below the slot count %llu", (unsigned long long)budget, (unsigned long long)B);
    std::vector<ServeSlot> sl(B);
    uint64_t off = 0;
    for (uint64_t q = 0; q < B; q++) {
        if (lens[q] == 0) return herr("serve_ragged: prompt %llu is empty", (unsigned long long)q);
        sl[q].prompt = tokens + off;
        sl[q].plen = lens[q];
        off += lens[q];
    }
    for (uint64_t i = 0; i < off; i++)
        if (tokens[i] >= V) return herr("serve_ragged: token %u >= vocab %llu", tokens[i], (unsigned long long)V);
    uint32_t temp = NONE, counter = NONE, sampler = NONE, hist = NONE, tok = NONE;
    auto cleanup = [&]() {
        for (uint32_t id : {temp, counter, sampler, hist, tok})
            if (id != NONE) rsv_tensor_free(c, id);
    };
    int rc = 0;
    uint64_t nst = 0;
    // Steps in which every slot decodes one token run the batched decode step
    // (the kernels of the B-session self-loop) instead of the packed prefill,
    // captured once as a HIP graph and replayed (RSV_NO_GRAPH=1: enqueued
    // eagerly); steps with prompt pieces, or with finished slots, take the
    // packed path.
    WorkBufs *dw = nullptr;
    bool dgraph = false;
    const bool deager = getenv("RSV_NO_GRAPH") && getenv("RSV_NO_GRAPH")[0] && getenv("RSV_NO_GRAPH")[0] != '0';
    do {
        // sampler work rows for up to B segments
        if ((rc = new_tensor(b, V * B, RSV_F32, temp))) break;
        if ((rc = new_tensor(b, V * B, RSV_U32, counter))) break;
        if ((rc = new_tensor(b, 8 * B, RSV_F32, sampler))) break;
        if ((rc = new_tensor(b, B, RSV_U32, hist))) break;
        if ((rc = new_tensor(b, B, RSV_U32, tok))) break;
        std::vector<uint32_t> drawn(B), seed_row(B);
        while (true) {
            std::vector<Seg> segs;
            std::vector<uint64_t> seg_slot;
            std::vector<bool> samples;
            std::vector<uint32_t> one(B);
            uint64_t used = 0, npre = 0, ndec = 0;
            for (uint64_t q = 0; q < B; q++) {  // decode tokens first
                ServeSlot &z = sl[q];
                if (z.done == z.plen && z.gen > 0 && z.gen < decode_len) {
                    one[q] = z.last;
                    segs.push_back({&one[q], 1, q});
                    seg_slot.push_back(q);
                    samples.push_back(true);
                    used++;
                    ndec++;
                }
            }
            // then one prompt piece per prompting slot, water-filled into the
            // rest of the budget
            std::vector<uint64_t> rem(B);
            for (uint64_t q = 0; q < B; q++) rem[q] = sl[q].plen - sl[q].done;
            const uint64_t L = std::max<uint64_t>(1, water_fill(rem, budget - used));
            for (uint64_t q = 0; q < B && used < budget; q++) {
                ServeSlot &z = sl[q];
                if (z.done >= z.plen) continue;
                const uint64_t take = std::min({z.plen - z.done, budget - used, L});
                segs.push_back({z.prompt + z.done, take, q});
                seg_slot.push_back(q);
                samples.push_back(z.done + take == z.plen);
                z.done += take;
                used += take;
                npre += take;
            }
            if (segs.empty()) break;
            if (nst >= max_steps) { rc = herr("serve_ragged: more than %llu steps", (unsigned long long)max_steps); break; }
            const auto t0 = std::chrono::steady_clock::now();
            const bool all_decode = npre == 0 && ndec == B;
            if (all_decode) {
                if (!dw && (rc = get_bufs(b, B, dw))) break;
                if (rsv_store_tokens(c, dw->token, one.data(), B)) { rc = herr("store_tokens: %s", rsv_last_error()); break; }
                if (deager) {
                    if ((rc = decode_step(b, *dw, s))) break;
                } else {
                    if (!dgraph) {
                        if (rsv_graph_begin(c)) { rc = herr("graph_begin: %s", rsv_last_error()); break; }
                        const int cap = decode_step(b, *dw, s);
                        const int end_rc = rsv_graph_end(c);
                        if (cap) { rc = cap; break; }
                        if (end_rc) { rc = herr("graph_end: %s", rsv_last_error()); break; }
                        dgraph = true;
                    }
                    if (rsv_graph_replay(c)) { rc = herr("graph_replay: %s", rsv_last_error()); break; }
                }
            } else if ((rc = prefill(b, s, segs, nullptr, true))) {
                break;
            }
            const uint32_t logits = all_decode ? dw->logits : b->seq.logits;  // prefill may reallocate its rows
            const uint64_t S = segs.size();
            for (uint64_t g = 0; g < S; g++) seed_row[g] = seeds[seg_slot[g]] + (uint32_t)sl[seg_slot[g]].gen;
            if (rsv_store_sampler_async_batch(c, sampler, 0, sp->temperature, sp->top_k, sp->top_p, seed_row.data(), S,
                                              sp->repetition_penalty, sp->frequency_penalty, sp->presence_penalty, 0) ||
                rsv_sample_into_host_seeded_batch(c, logits, tok, V, temp, NONE, counter, sampler, hist, S) ||
                rsv_download_u32(c, tok, drawn.data(), S)) {
                rc = herr("serve_ragged sampler: %s", rsv_last_error());
                break;
            }
            const auto t1 = std::chrono::steady_clock::now();
            if (sampled_logits) {  // the logits row each draw was made from (checks)
                std::vector<float> rows(S * V);
                if (rsv_download(c, logits, rows.data(), S * V)) { rc = herr("serve_ragged logits: %s", rsv_last_error()); break; }
                for (uint64_t g = 0; g < S; g++)
                    if (samples[g])
                        memcpy(sampled_logits + (seg_slot[g] * decode_len + sl[seg_slot[g]].gen) * V, rows.data() + g * V,
                               V * sizeof(float));
            }
            for (uint64_t g = 0; g < S; g++) {
                if (!samples[g]) continue;
                ServeSlot &z = sl[seg_slot[g]];
                out[seg_slot[g] * decode_len + z.gen] = drawn[g];
                z.last = drawn[g];
                z.gen++;
            }
            if (steps) {
                steps[nst].prefill_tokens = npre;
                steps[nst].decode_tokens = ndec;
                steps[nst].sampled = 0;
                for (uint64_t g = 0; g < S; g++) steps[nst].sampled += samples[g] ? 1 : 0;
                steps[nst].ms = std::chrono::duration<double, std::milli>(t1 - t0).count();
            }
            nst++;
            bool busy = false;
            for (auto &z : sl) busy |= z.done < z.plen || z.gen < decode_len;
            if (!busy) break;
        }
    } while (0);
    if (nsteps) *nsteps = nst;
    cleanup();
    return rc;
}

// ------------------------------------------------------------ self-loops
int selfloop(rsv_bundle *b, GpuState &s, const uint32_t *seeds, uint64_t n, const rsv_sampler_params *sp,
             uint32_t *out, float *ms) {
    rsv_ctx *c = b->ctx;
    const rsv_model_info &I = b->info;
    const uint64_t B = s.batch;
    if (n == 0) return 0;
    WorkBufs *w;
    HK(get_bufs(b, B, w));
    uint32_t seq = NONE, cnt = NONE, temp = NONE, counter = NONE, sampler = NONE;
    auto cleanup = [&]() {
        for (uint32_t id : {seq, cnt, temp, counter, sampler})
            if (id != NONE) rsv_tensor_free(c, id);
    };
    int rc = 0;
    do {
        if ((rc = new_tensor(b, n * B, RSV_U32, seq))) break;
        if ((rc = new_tensor(b, B, RSV_U32, cnt))) break;
        if (sp) {
            if ((rc = new_tensor(b, I.vocab * B, RSV_F32, temp))) break;
            if ((rc = new_tensor(b, I.vocab * B, RSV_U32, counter))) break;
            if ((rc = new_tensor(b, 8 * B, RSV_F32, sampler))) break;
        }
        if (rsv_store_tokens(c, w->token, seeds, B)) { rc = herr("store_tokens: %s", rsv_last_error()); break; }
        if (rsv_synchronize(c)) { rc = herr("%s", rsv_last_error()); break; }
        // One step = gather -> layers -> head -> sampler -> record.  It is
        // captured once as a HIP graph and replayed n times; RSV_NO_GRAPH=1
        // enqueues the same kernels eagerly every round instead (the
        // reference's SKIP_GRAPH debugging path, gpu_model.rs:1698-1721).
        const bool eager = getenv("RSV_NO_GRAPH") && getenv("RSV_NO_GRAPH")[0] && getenv("RSV_NO_GRAPH")[0] != '0';
        // A round ends with the token's record and the gather of its
        // embedding row for the next round (one launch with the argmax when
        // greedy, one after the sampler otherwise), so a round starts at the
        // layers; the first round's rows are gathered here.
        if (rsv_gather_rows_device_f16(c, b->emb_ln, w->x, w->token, I.n_embd, B)) {
            rc = herr("gather: %s", rsv_last_error());
            break;
        }
        auto step = [&]() -> int {
            int e = decode_step(b, *w, s, false);
            if (!e && sp) {
                if (rsv_sample_into_host_seeded_batch(c, w->logits, w->token, I.vocab, temp, NONE, counter, sampler,
                                                      seq, B))
                    e = herr("sampler: %s", rsv_last_error());
                else if (rsv_record_gather_batch(c, w->token, seq, cnt, n, b->emb_ln, w->x, I.n_embd, B))
                    e = herr("record: %s", rsv_last_error());
            } else if (!e) {
                if (rsv_argmax_record_gather_batch(c, w->logits, w->token, I.vocab, seq, cnt, n, b->emb_ln, w->x,
                                                   I.n_embd, B))
                    e = herr("argmax: %s", rsv_last_error());
            }
            return e;
        };
        if (!eager) {
            if (rsv_graph_begin(c)) { rc = herr("graph_begin: %s", rsv_last_error()); break; }
            const int cap = step();
            const int end_rc = rsv_graph_end(c);
            if (cap) { rc = cap; break; }
            if (end_rc) { rc = herr("graph_end: %s", rsv_last_error()); break; }
        }
        hipEvent_t e0 = nullptr, e1 = nullptr;
        void *stream = nullptr;
        rsv_stream(c, &stream);
        if (ms) {
            hipEventCreate(&e0);
            hipEventCreate(&e1);
            hipEventRecord(e0, (hipStream_t)stream);
        }
        std::vector<uint32_t> seeds_r(B);
        for (uint64_t r = 0; r < n && !rc; r++) {
            if (sp) {
                // per-round seed = seed + round, hist_len = round (gpu_model.rs:799-812, 1712-1731)
                for (uint64_t q = 0; q < B; q++) seeds_r[q] = seeds[q] + (uint32_t)r;
                if (rsv_store_sampler_async_batch(c, sampler, r, sp->temperature, sp->top_k, sp->top_p, seeds_r.data(),
                                                  B, sp->repetition_penalty, sp->frequency_penalty,
                                                  sp->presence_penalty, (uint32_t)r))
                    rc = herr("store_sampler: %s", rsv_last_error());
            }
            if (!rc) {
                if (eager) rc = step();
                else if (rsv_graph_replay(c)) rc = herr("graph_replay: %s", rsv_last_error());
            }
        }
        if (ms) {
            hipEventRecord(e1, (hipStream_t)stream);
            hipEventSynchronize(e1);
            hipEventElapsedTime(ms, e0, e1);
            hipEventDestroy(e0);
            hipEventDestroy(e1);
        }
        if (rc) break;
        if (rsv_download_u32(c, seq, out, n * B)) { rc = herr("download: %s", rsv_last_error()); break; }
    } while (0);
    cleanup();
    return rc;
}

}  // namespace

// ================================================================ C-ABI
extern "C" {

const char *rsv_host_last_error(void) { return g_herr.c_str(); }

int rsv_model_build(const char *path, int device, rsv_bundle **out) {
    if (!path || !out) return herr("rsv_model_build: null argument");
    auto b = std::make_unique<rsv_bundle>();
    if (rsv_create(device, &b->ctx)) return herr("rsv_create: %s", rsv_last_error());
    HK(load_model(b.get(), path));
    b->state = new rsv_state();
    if (state_create(b.get(), 1, b->state->s)) { delete b->state; b->state = nullptr; return -1; }
    *out = b.release();
    return 0;
}

// GpuModel::build_shared (gpu_model.rs:594-628): a second instance on the
// same device whose context imports every tensor of the source (weights are
// not copied), with its own stream, work buffers and session state.  The
// shared allocations live until both instances have freed them, so either
// may be freed first.  Weight copies made lazily after this call (the
// MFMA-tiled copies of the batched path, the fp16 prefill copies) are made
// per instance.
int rsv_bundle_build_shared(rsv_bundle *src, rsv_bundle **out) {
    if (!src || !out) return herr("rsv_bundle_build_shared: null argument");
    int dev = 0;
    CK(rsv_context_device(src->ctx, &dev));
    auto b = std::make_unique<rsv_bundle>();
    if (rsv_create(dev, &b->ctx)) return herr("rsv_create: %s", rsv_last_error());
    CK(rsv_synchronize(src->ctx));
    CK(rsv_import_tensors(b->ctx, src->ctx));
    b->info = src->info;
    b->emb_ln = src->emb_ln;
    b->ln_out_w = src->ln_out_w;
    b->ln_out_b = src->ln_out_b;
    b->scale_w = src->scale_w;
    b->head = src->head;
    b->layers = src->layers;
    b->tiled = src->tiled;
    b->p16 = src->p16;
    b->state = new rsv_state();
    if (state_create(b.get(), 1, b->state->s)) { delete b->state; b->state = nullptr; return -1; }
    *out = b.release();
    return 0;
}

int rsv_bundle_free(rsv_bundle *b) {
    if (!b) return 0;
    delete b->state;
    delete b;
    return 0;
}

int rsv_bundle_info(rsv_bundle *b, rsv_model_info *info) {
    if (!b || !info) return herr("null argument");
    *info = b->info;
    return 0;
}

void *rsv_bundle_ctx(rsv_bundle *b) { return b ? (void *)b->ctx : nullptr; }

static int tokens_ok(rsv_bundle *b, const uint32_t *t, uint64_t n) {
    if (!b) return herr("null bundle");
    if (n == 0) return herr("empty token list");
    if (!t) return herr("null tokens");
    for (uint64_t i = 0; i < n; i++)
        if (t[i] >= b->info.vocab) return herr("token %u at %llu >= vocab %llu", t[i], (unsigned long long)i, (unsigned long long)b->info.vocab);
    return 0;
}

// forward_with_state (gpu_model.rs:668): token-by-token decode path.
static int run_tokens(rsv_bundle *b, GpuState &s, const uint32_t *tokens, uint64_t n) {
    WorkBufs *w;
    HK(get_bufs(b, 1, w));
    for (uint64_t t = 0; t < n; t++) {
        CK(rsv_store_token(b->ctx, w->token, tokens[t]));
        HK(decode_step(b, *w, s));
    }
    return 0;
}

int rsv_infer_tokens(rsv_bundle *b, const uint32_t *tokens, uint64_t n, float *logits) {
    HK(tokens_ok(b, tokens, n));
    HK(run_tokens(b, b->state->s, tokens, n));
    CK(rsv_download(b->ctx, b->bufs[1].logits, logits, b->info.vocab));
    return 0;
}

int rsv_infer_seq(rsv_bundle *b, const uint32_t *tokens, uint64_t n, float *logits) {
    HK(tokens_ok(b, tokens, n));
    return seq_single(b, b->state->s, 0, tokens, n, logits);
}

int rsv_infer_chunked(rsv_bundle *b, const uint32_t *tokens, uint64_t n, uint64_t chunk, float *logits) {
    HK(tokens_ok(b, tokens, n));
    if (chunk == 0) chunk = 1;
    for (uint64_t off = 0; off < n; off += chunk) {
        const uint64_t len = n - off < chunk ? n - off : chunk;
        HK(seq_single(b, b->state->s, 0, tokens + off, len, off + len == n ? logits : nullptr));
    }
    return 0;
}

int rsv_infer_full(rsv_bundle *b, const uint32_t *tokens, uint64_t n, float *logits) {
    HK(tokens_ok(b, tokens, n));
    for (uint64_t t = 0; t < n; t++) HK(seq_single(b, b->state->s, 0, tokens + t, 1, logits + t * b->info.vocab));
    return 0;
}

int rsv_infer_argmax(rsv_bundle *b, const uint32_t *tokens, uint64_t n, uint32_t *token) {
    HK(tokens_ok(b, tokens, n));
    HK(run_tokens(b, b->state->s, tokens, n));
    WorkBufs &w = b->bufs[1];
    CK(rsv_argmax(b->ctx, w.logits, w.token, b->info.vocab));
    CK(rsv_download_u32(b->ctx, w.token, token, 1));
    return 0;
}

int rsv_infer_argmax_selfloop(rsv_bundle *b, uint32_t seed, uint64_t n, uint32_t *out) {
    if (!b) return herr("null bundle");
    if (seed >= b->info.vocab) return herr("seed token %u >= vocab", seed);
    return selfloop(b, b->state->s, &seed, n, nullptr, out, nullptr);
}

int rsv_infer_sample(rsv_bundle *b, const uint32_t *tokens, uint64_t n, const rsv_sampler_params *sp,
                     const uint32_t *history, uint64_t hist_len, uint32_t *token) {
    HK(tokens_ok(b, tokens, n));
    if (!sp) return herr("null sampler params");
    HK(run_tokens(b, b->state->s, tokens, n));
    WorkBufs &w = b->bufs[1];
    CK(rsv_sample(b->ctx, w.logits, w.token, b->info.vocab, sp->temperature, sp->top_k, sp->top_p, sp->seed,
                  sp->repetition_penalty, sp->frequency_penalty, sp->presence_penalty, history, hist_len));
    CK(rsv_download_u32(b->ctx, w.token, token, 1));
    return 0;
}

int rsv_infer_sample_selfloop(rsv_bundle *b, uint32_t seed, uint64_t n, const rsv_sampler_params *sp,
                              uint32_t *out) {
    if (!b || !sp) return herr("null argument");
    if (seed >= b->info.vocab) return herr("seed token %u >= vocab", seed);
    return selfloop(b, b->state->s, &seed, n, sp, out, nullptr);
}

int rsv_state_len(rsv_bundle *b, uint64_t *len) {
    if (!b || !len) return herr("null argument");
    *len = state_len1(b);
    return 0;
}

int rsv_state_back(rsv_bundle *b, float *out) {
    if (!b || !out) return herr("null argument");
    return state_back_slots(b, b->state->s, 0, 1, out);
}

int rsv_state_load(rsv_bundle *b, const float *data, uint64_t len) {
    if (!b || !data) return herr("null argument");
    if (len != state_len1(b))
        return herr("State::load length mismatch: got %llu, expected %llu", (unsigned long long)len, (unsigned long long)state_len1(b));
    return state_load_slots(b, b->state->s, 0, 1, data);
}

int rsv_reset(rsv_bundle *b) {
    if (!b) return herr("null bundle");
    return state_reset(b, b->state->s);
}

int rsv_create_batch_state(rsv_bundle *b, uint64_t batch, rsv_state **out) {
    if (!b || !out) return herr("null argument");
    if (batch == 0) return herr("batch must be >= 1");
    auto s = std::make_unique<rsv_state>();
    if (state_create(b, batch, s->s)) { state_free(b, s->s); return -1; }
    *out = s.release();
    return 0;
}

int rsv_state_free(rsv_bundle *b, rsv_state *s) {
    if (!b || !s) return 0;
    state_free(b, s->s);
    delete s;
    return 0;
}

int rsv_state_batch(rsv_state *s, uint64_t *batch) {
    if (!s || !batch) return herr("null argument");
    *batch = s->s.batch;
    return 0;
}

int rsv_batch_state_back(rsv_bundle *b, rsv_state *s, float *out) {
    if (!b || !s || !out) return herr("null argument");
    return state_back_slots(b, s->s, 0, s->s.batch, out);
}

int rsv_batch_state_load(rsv_bundle *b, rsv_state *s, const float *data, uint64_t len) {
    if (!b || !s || !data) return herr("null argument");
    if (len != state_len1(b) * s->s.batch)
        return herr("State::load length mismatch: got %llu, expected %llu", (unsigned long long)len, (unsigned long long)(state_len1(b) * s->s.batch));
    return state_load_slots(b, s->s, 0, s->s.batch, data);
}

int rsv_state_slot_back(rsv_bundle *b, rsv_state *s, uint64_t slot, float *out) {
    if (!b || !s || !out) return herr("null argument");
    if (slot >= s->s.batch) return herr("slot_back: slot %llu >= batch %llu", (unsigned long long)slot, (unsigned long long)s->s.batch);
    return state_back_slots(b, s->s, slot, 1, out);
}

int rsv_state_slot_load(rsv_bundle *b, rsv_state *s, uint64_t slot, const float *data, uint64_t len) {
    if (!b || !s || !data) return herr("null argument");
    if (slot >= s->s.batch) return herr("slot_load: slot %llu >= batch %llu", (unsigned long long)slot, (unsigned long long)s->s.batch);
    if (len != state_len1(b))
        return herr("State::slot_load length mismatch: got %llu, expected %llu", (unsigned long long)len, (unsigned long long)state_len1(b));
    return state_load_slots(b, s->s, slot, 1, data);
}

int rsv_batch_state_reset(rsv_bundle *b, rsv_state *s) {
    if (!b || !s) return herr("null argument");
    return state_reset(b, s->s);
}

int rsv_forward_seq_batch(rsv_bundle *b, rsv_state *s, const uint32_t *tokens, const uint64_t *lens, uint32_t *seeds,
                          float *logits) {
    if (!b || !s || !tokens || !lens) return herr("null argument");
    const uint64_t B = s->s.batch;
    std::vector<Seg> segs;
    uint64_t off = 0, T = 0;
    for (uint64_t q = 0; q < B; q++) {
        if (lens[q] == 0) return herr("forward_seq_batch: prompt %llu is empty", (unsigned long long)q);
        HK(tokens_ok(b, tokens + off, lens[q]));
        segs.push_back({tokens + off, lens[q], q});
        if (seeds) seeds[q] = tokens[off + lens[q] - 1];
        off += lens[q];
        T += lens[q];
    }
    // Packed chunks of at most prefill_chunk tokens, filled breadth-first: every
    // unfinished prompt contributes its next piece of at most L tokens, with
    // L the largest length whose pieces still fit one chunk (water filling).
    // A prompt's pieces go through consecutive chunks in order, its state
    // carried between them.  The WKV scan of a chunk is sequential over its
    // longest piece, so many short pieces per chunk keep that scan short;
    // per-token arithmetic does not depend on the packing.
    std::vector<Seg> pending;
    auto flush = [&]() -> int {
        if (pending.empty()) return 0;
        std::vector<float> tmp;
        if (logits) tmp.resize(pending.size() * b->info.vocab);
        HK(prefill(b, s->s, pending, logits ? tmp.data() : nullptr));
        if (logits)
            for (size_t i = 0; i < pending.size(); i++)
                memcpy(logits + pending[i].slot * b->info.vocab, &tmp[i * b->info.vocab], b->info.vocab * 4);
        pending.clear();
        return 0;
    };
    std::vector<uint64_t> done(segs.size(), 0);
    std::vector<std::vector<Seg>> chunks;
    for (;;) {
        std::vector<uint64_t> rem(segs.size());
        for (size_t i = 0; i < segs.size(); i++) rem[i] = segs[i].len - done[i];
        if (rem.empty() || *std::max_element(rem.begin(), rem.end()) == 0) break;
        const uint64_t ch = b->prefill_chunk;
        const uint64_t L = std::max<uint64_t>(1, water_fill(rem, ch));
        uint64_t used = 0;
        for (size_t i = 0; i < segs.size(); i++) {
            const uint64_t take = std::min({segs[i].len - done[i], L, ch - used});
            if (take == 0) continue;
            pending.push_back({segs[i].tok + done[i], take, segs[i].slot});
            done[i] += take;
            used += take;
        }
        if (logits) {
            HK(flush());  // every chunk's last rows feed the logits
        } else {
            chunks.push_back(std::move(pending));
            pending.clear();
        }
    }
    if (!logits) return prefill_chunks(b, s->s, chunks, nullptr);
    HK(flush());
    return 0;
}

int rsv_forward_tokens_batch(rsv_bundle *b, rsv_state *s, const uint32_t *tokens, float *logits) {
    if (!b || !s || !tokens) return herr("null argument");
    const uint64_t B = s->s.batch;
    HK(tokens_ok(b, tokens, B));
    WorkBufs *w;
    HK(get_bufs(b, B, w));
    CK(rsv_store_tokens(b->ctx, w->token, tokens, B));
    HK(decode_step(b, *w, s->s));
    if (logits) CK(rsv_download(b->ctx, w->logits, logits, B * b->info.vocab));
    else CK(rsv_synchronize(b->ctx));
    return 0;
}

int rsv_argmax_selfloop_batch(rsv_bundle *b, rsv_state *s, const uint32_t *seeds, uint64_t n, uint32_t *out) {
    if (!b || !s || !seeds || !out) return herr("null argument");
    HK(tokens_ok(b, seeds, s->s.batch));
    return selfloop(b, s->s, seeds, n, nullptr, out, nullptr);
}

int rsv_argmax_selfloop_batch_timed(rsv_bundle *b, rsv_state *s, const uint32_t *seeds, uint64_t n, uint32_t *out,
                                    float *ms) {
    if (!b || !s || !seeds || !out || !ms) return herr("null argument");
    HK(tokens_ok(b, seeds, s->s.batch));
    return selfloop(b, s->s, seeds, n, nullptr, out, ms);
}

int rsv_set_prefill_lanes(rsv_bundle *b, int lanes) {
    if (!b) return herr("null argument");
    if (lanes != 1 && lanes != 2) return herr("set_prefill_lanes: lanes must be 1 or 2");
    b->prefill_lanes = lanes;
    return 0;
}

int rsv_set_prefill_chunk(rsv_bundle *b, uint64_t rows) {
    if (!b) return herr("null argument");
    if (rows == 0 || rows > kMaxChunk) return herr("set_prefill_chunk: rows must be 1..%llu", (unsigned long long)kMaxChunk);
    b->prefill_chunk = rows;
    return 0;
}

int rsv_serve_ragged(rsv_bundle *b, rsv_state *s, const uint32_t *tokens, const uint64_t *lens, uint64_t decode_len,
                     const rsv_sampler_params *sp, const uint32_t *seeds, uint64_t budget, uint32_t *out,
                     rsv_serve_step *steps, uint64_t max_steps, uint64_t *nsteps) {
    if (!b || !s || !tokens || !lens || !sp || !seeds || !out) return herr("null argument");
    return serve_ragged(b, s->s, tokens, lens, decode_len, sp, seeds, budget, out, steps, max_steps, nsteps, nullptr);
}

int rsv_serve_ragged_logits(rsv_bundle *b, rsv_state *s, const uint32_t *tokens, const uint64_t *lens,
                            uint64_t decode_len, const rsv_sampler_params *sp, const uint32_t *seeds, uint64_t budget,
                            uint32_t *out, rsv_serve_step *steps, uint64_t max_steps, uint64_t *nsteps,
                            float *sampled_logits) {
    if (!b || !s || !tokens || !lens || !sp || !seeds || !out) return herr("null argument");
    return serve_ragged(b, s->s, tokens, lens, decode_len, sp, seeds, budget, out, steps, max_steps, nsteps, sampled_logits);
}

int rsv_sample_selfloop_batch(rsv_bundle *b, rsv_state *s, const uint32_t *seeds, uint64_t n,
                              const rsv_sampler_params *sp, uint32_t *out) {
    if (!b || !s || !seeds || !out || !sp) return herr("null argument");
    HK(tokens_ok(b, seeds, s->s.batch));
    return selfloop(b, s->s, seeds, n, sp, out, nullptr);
}

int rsv_sample_selfloop_batch_timed(rsv_bundle *b, rsv_state *s, const uint32_t *seeds, uint64_t n,
                                    const rsv_sampler_params *sp, uint32_t *out, float *ms) {
    if (!b || !s || !seeds || !out || !sp || !ms) return herr("null argument");
    HK(tokens_ok(b, seeds, s->s.batch));
    return selfloop(b, s->s, seeds, n, sp, out, ms);
}

}  // extern "C"
