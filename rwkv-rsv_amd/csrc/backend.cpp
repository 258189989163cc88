// librsv_hip.so: context, tensor table, stream/graph management and the
// extern "C" entry points of include/rsv_hip.h.  Every op validates its
// operands on the host (existence, dtype, minimum length) before enqueuing,
// so a shape mismatch is an error status, never an out-of-bounds kernel.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "rsv_common.h"

namespace rsv {

static thread_local std::string g_err;

void set_error(const char *fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
}

Tensor *get_tensor(rsv_ctx *ctx, uint32_t id) {
    if (!ctx || id >= ctx->tensors.size() || !ctx->tensors[id].live) return nullptr;
    return &ctx->tensors[id];
}

// f32 -> f16 bits, round to nearest even (IEEE binary16).
static uint16_t f32_to_f16(float f) {
    _Float16 h = (_Float16)f;  // host conversion is RNE
    uint16_t b;
    memcpy(&b, &h, 2);
    return b;
}
static float f16_to_f32(uint16_t b) {
    _Float16 h;
    memcpy(&h, &b, 2);
    return (float)h;
}

}  // namespace rsv

using namespace rsv;

// Operand fetch with validation.  dtype -1 accepts any dtype.
static int opnd(rsv_ctx *ctx, uint32_t id, int dtype, uint64_t min_len, void **p, const char *what) {
    Tensor *t = get_tensor(ctx, id);
    if (!t) return RSV_FAIL("%s: unknown tensor id %u", what, id);
    if (dtype >= 0 && t->dtype != dtype) {
        // U32 and F32 share 4-byte slots (token and counter buffers hold bit patterns)
        const bool word_ok = (dtype == RSV_U32 || dtype == RSV_F32) && (t->dtype == RSV_U32 || t->dtype == RSV_F32);
        if (!word_ok) return RSV_FAIL("%s: tensor %u has dtype %d, expected %d", what, id, t->dtype, dtype);
    }
    if (t->len < min_len)
        return RSV_FAIL("%s: tensor %u holds %llu elements, needs %llu", what, id, (unsigned long long)t->len,
                        (unsigned long long)min_len);
    *p = t->ptr;
    return 0;
}
#define OPND(var, id, dt, n, what)                                          \
    void *var##_v = nullptr;                                                \
    if (opnd(ctx, (id), (dt), (uint64_t)(n), &var##_v, (what)) != 0) return -1;

#define F32P(var) ((float *)var##_v)
#define U32P(var) ((uint32_t *)var##_v)

#define CHECK_CTX()                                     \
    do {                                                \
        if (!ctx) return RSV_FAIL("null context");      \
        if (hipSetDevice(ctx->device) != hipSuccess)    \
            return RSV_FAIL("hipSetDevice(%d) failed", ctx->device); \
    } while (0)

static int no_capture(rsv_ctx *ctx, const char *what) {
    if (ctx->capturing || ctx->prefill_capturing)
        return RSV_FAIL("%s: synchronous host transfer is not allowed during graph capture", what);
    return 0;
}

static int int8_operands(rsv_ctx *ctx, const rsv_int8 *w, uint64_t m, uint64_t k, const uint32_t **idx,
                         const uint32_t **sz, const char *what) {
    if (!w) return RSV_FAIL("%s: null int8 handle", what);
    if (w->m != m || w->k != k)
        return RSV_FAIL("%s: int8 handle is %llux%llu, op asks %llux%llu", what, (unsigned long long)w->m,
                        (unsigned long long)w->k, (unsigned long long)m, (unsigned long long)k);
    if (k % 128 != 0) return RSV_FAIL("%s: k=%llu not a multiple of 128", what, (unsigned long long)k);
    void *a = nullptr, *b = nullptr;
    if (opnd(ctx, w->idx, RSV_U32, m * k / 4, &a, what) || opnd(ctx, w->sz, RSV_U32, m * k / 128, &b, what)) return -1;
    *idx = (const uint32_t *)a;
    *sz = (const uint32_t *)b;
    return 0;
}

extern "C" {

const char *rsv_last_error(void) { return g_err.c_str(); }

int rsv_create(int device, rsv_ctx **out) {
    if (!out) return RSV_FAIL("rsv_create: null out");
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0) return RSV_FAIL("rsv_create: no HIP device");
    if (device < 0 || device >= n) return RSV_FAIL("rsv_create: device %d out of range (%d devices)", device, n);
    RSV_HIP(hipSetDevice(device));
    rsv_ctx *ctx = new rsv_ctx();
    ctx->device = device;
    if (hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking) != hipSuccess) {
        delete ctx;
        return RSV_FAIL("rsv_create: hipStreamCreate failed");
    }
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) == hipSuccess) ctx->sm_count = prop.multiProcessorCount;
    // 32 Mi floats (128 MiB) of split-K partial tiles
    ctx->skinny_ws_cap = (size_t)32 << 20;
    if (hipMalloc(&ctx->skinny_ws, ctx->skinny_ws_cap * 4) != hipSuccess) {
        hipStreamDestroy(ctx->stream);
        delete ctx;
        return RSV_FAIL("rsv_create: workspace allocation failed");
    }
    if (sample_scratch_init(device)) {
        const std::string why = rsv_last_error();
        hipFree(ctx->skinny_ws);
        hipStreamDestroy(ctx->stream);
        delete ctx;
        return RSV_FAIL("rsv_create: %s", why.c_str());
    }
    *out = ctx;
    return 0;
}

int rsv_destroy(rsv_ctx *ctx) {
    if (!ctx) return 0;
    hipSetDevice(ctx->device);
    if (ctx->lane[0]) ctx->stream = ctx->lane[0];
    if (ctx->lane[1]) {
        hipStreamSynchronize(ctx->lane[1]);
        hipStreamDestroy(ctx->lane[1]);
    }
    for (auto &v : ctx->lane_ev)
        for (hipEvent_t e : v) hipEventDestroy(e);
    hipStreamSynchronize(ctx->stream);
    if (ctx->graph_exec) hipGraphExecDestroy(ctx->graph_exec);
    if (ctx->graph) hipGraphDestroy(ctx->graph);
    for (auto &kv : ctx->prefill_graphs) hipGraphExecDestroy(kv.second);
    ctx->tensors.clear();  // drops this context's hold on each allocation
    if (ctx->hist_dev) hipFree(ctx->hist_dev);
    if (ctx->sample_work) hipFree(ctx->sample_work);
    if (ctx->skinny_ws) hipFree(ctx->skinny_ws);
    sample_scratch_release(ctx->device, ctx);
    hipStreamDestroy(ctx->stream);
    delete ctx;
    return 0;
}

int rsv_device_name(rsv_ctx *ctx, char *buf, size_t len) {
    CHECK_CTX();
    hipDeviceProp_t prop;
    RSV_HIP(hipGetDeviceProperties(&prop, ctx->device));
    snprintf(buf, len, "%s (%s, %d CUs)", prop.name, prop.gcnArchName, prop.multiProcessorCount);
    return 0;
}

int rsv_synchronize(rsv_ctx *ctx) {
    CHECK_CTX();
    RSV_HIP(hipStreamSynchronize(ctx->stream));
    return 0;
}

// ------------------------------------------------------------ prefill lanes
constexpr int kLaneEvents = 256;

static int lane_make(rsv_ctx *ctx, int lane) {
    if (!ctx->lane[0]) ctx->lane[0] = ctx->stream;
    if (lane == 1 && !ctx->lane[1]) {
        RSV_HIP(hipSetDevice(ctx->device));
        RSV_HIP(hipStreamCreateWithFlags(&ctx->lane[1], hipStreamNonBlocking));  // default priority
    }
    if (ctx->lane_ev[lane].empty()) {
        ctx->lane_ev[lane].assign(kLaneEvents, nullptr);
        for (auto &e : ctx->lane_ev[lane]) RSV_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    }
    return 0;
}

int rsv_lane_select(rsv_ctx *ctx, int lane) {
    CHECK_CTX();
    if (lane < 0 || lane > 1) return RSV_FAIL("lane_select: lane %d is not 0 or 1", lane);
    if (ctx->capturing || ctx->prefill_capturing) return RSV_FAIL("lane_select: not during graph capture");
    if (lane_make(ctx, lane)) return -1;
    ctx->stream = ctx->lane[lane];
    return 0;
}

int rsv_lane_record(rsv_ctx *ctx, int ev) {
    CHECK_CTX();
    if (ev < 0 || ev >= kLaneEvents) return RSV_FAIL("lane_record: event %d out of 0..%d", ev, kLaneEvents - 1);
    const int lane = ctx->lane[1] && ctx->stream == ctx->lane[1] ? 1 : 0;
    if (lane_make(ctx, lane)) return -1;
    RSV_HIP(hipEventRecord(ctx->lane_ev[lane][ev], ctx->stream));
    return 0;
}

int rsv_lane_wait(rsv_ctx *ctx, int lane, int ev) {
    CHECK_CTX();
    if (lane < 0 || lane > 1) return RSV_FAIL("lane_wait: lane %d is not 0 or 1", lane);
    if (ev < 0 || ev >= kLaneEvents) return RSV_FAIL("lane_wait: event %d out of 0..%d", ev, kLaneEvents - 1);
    if (lane_make(ctx, lane)) return -1;
    RSV_HIP(hipStreamWaitEvent(ctx->stream, ctx->lane_ev[lane][ev], 0));
    return 0;
}

// ------------------------------------------------------------------ tensors
int rsv_tensor_create(rsv_ctx *ctx, uint64_t len, int dtype, uint32_t *id) {
    CHECK_CTX();
    if (!id) return RSV_FAIL("tensor_create: null id");
    if (dtype != RSV_F32 && dtype != RSV_F16 && dtype != RSV_U32) return RSV_FAIL("tensor_create: bad dtype %d", dtype);
    if (no_capture(ctx, "tensor_create")) return -1;
    Tensor t;
    t.len = len;
    t.dtype = dtype;
    const size_t bytes = (size_t)(len ? len : 1) * dtype_size(dtype);
    // pad to 64 bytes so 16-byte vector tails never cross the allocation
    RSV_HIP(hipMalloc(&t.ptr, (bytes + 63) & ~(size_t)63));
    t.mem = std::make_shared<DevMem>();
    t.mem->ptr = t.ptr;
    t.mem->device = ctx->device;
    RSV_HIP(hipMemsetAsync(t.ptr, 0, (bytes + 63) & ~(size_t)63, ctx->stream));
    t.live = true;
    if (!ctx->free_ids.empty()) {
        *id = ctx->free_ids.back();
        ctx->free_ids.pop_back();
        ctx->tensors[*id] = t;
    } else {
        *id = (uint32_t)ctx->tensors.size();
        ctx->tensors.push_back(t);
    }
    return 0;
}

int rsv_tensor_free(rsv_ctx *ctx, uint32_t id) {
    CHECK_CTX();
    Tensor *t = get_tensor(ctx, id);
    if (!t) return 0;  // freeing an unknown id is a no-op, like the reference
    if (ctx->capturing || ctx->prefill_capturing) return RSV_FAIL("tensor_free: not allowed during graph capture");
    // this context's work on the tensor finishes before its hold is dropped;
    // the memory itself goes when no context holds it any more
    hipStreamSynchronize(ctx->stream);
    // captured prefill graphs hold device pointers: one of them may point
    // at this memory, so every such graph is dropped (recaptured on next use)
    for (auto &kv : ctx->prefill_graphs) hipGraphExecDestroy(kv.second);
    ctx->prefill_graphs.clear();
    *t = Tensor();
    ctx->free_ids.push_back(id);
    return 0;
}

int rsv_drop_host(rsv_ctx *ctx, uint32_t id) {
    (void)ctx;
    (void)id;
    return 0;
}

int rsv_clear_cache(rsv_ctx *ctx) {
    CHECK_CTX();
    for (auto &kv : ctx->prefill_graphs) hipGraphExecDestroy(kv.second);
    ctx->prefill_graphs.clear();
    return 0;
}

int rsv_tensor_len(rsv_ctx *ctx, uint32_t id, uint64_t *len, int *dtype) {
    Tensor *t = get_tensor(ctx, id);
    if (!t) return RSV_FAIL("tensor_len: unknown tensor id %u", id);
    if (len) *len = t->len;
    if (dtype) *dtype = t->dtype;
    return 0;
}

int rsv_tensor_ptr(rsv_ctx *ctx, uint32_t id, void **ptr) {
    Tensor *t = get_tensor(ctx, id);
    if (!t) return RSV_FAIL("tensor_ptr: unknown tensor id %u", id);
    *ptr = t->ptr;
    return 0;
}

int rsv_stream(rsv_ctx *ctx, void **stream) {
    if (!ctx) return RSV_FAIL("null context");
    *stream = (void *)ctx->stream;
    return 0;
}

static int upload_impl(rsv_ctx *ctx, uint32_t id, uint64_t offset, const void *data, uint64_t len, bool is_u32) {
    CHECK_CTX();
    if (no_capture(ctx, "upload")) return -1;
    Tensor *t = get_tensor(ctx, id);
    if (!t) return RSV_FAIL("upload: unknown tensor id %u", id);
    if (offset + len > t->len)
        return RSV_FAIL("upload: %llu+%llu elements exceed tensor %u of %llu", (unsigned long long)offset,
                        (unsigned long long)len, id, (unsigned long long)t->len);
    if (len == 0) return 0;
    RSV_HIP(hipStreamSynchronize(ctx->stream));
    if (t->dtype == RSV_F16) {
        if (is_u32) return RSV_FAIL("upload_u32: tensor %u is F16", id);
        std::vector<uint16_t> h(len);
        const float *f = (const float *)data;
        for (uint64_t i = 0; i < len; i++) h[i] = f32_to_f16(f[i]);
        RSV_HIP(hipMemcpy((uint16_t *)t->ptr + offset, h.data(), len * 2, hipMemcpyHostToDevice));
    } else {
        RSV_HIP(hipMemcpy((uint32_t *)t->ptr + offset, data, len * 4, hipMemcpyHostToDevice));
    }
    return 0;
}

int rsv_upload(rsv_ctx *ctx, uint32_t id, const float *data, uint64_t len) {
    return upload_impl(ctx, id, 0, data, len, false);
}
int rsv_upload_part(rsv_ctx *ctx, uint32_t id, uint64_t offset, const float *data, uint64_t len) {
    return upload_impl(ctx, id, offset, data, len, false);
}
int rsv_upload_u32(rsv_ctx *ctx, uint32_t id, const uint32_t *data, uint64_t len) {
    return upload_impl(ctx, id, 0, data, len, true);
}

int rsv_upload_bytes(rsv_ctx *ctx, uint32_t id, const void *data, uint64_t nbytes) {
    CHECK_CTX();
    if (no_capture(ctx, "upload_bytes")) return -1;
    Tensor *t = get_tensor(ctx, id);
    if (!t) return RSV_FAIL("upload_bytes: unknown tensor id %u", id);
    if (nbytes > t->len * dtype_size(t->dtype)) return RSV_FAIL("upload_bytes: %llu bytes exceed tensor %u", (unsigned long long)nbytes, id);
    RSV_HIP(hipStreamSynchronize(ctx->stream));
    RSV_HIP(hipMemcpy(t->ptr, data, nbytes, hipMemcpyHostToDevice));
    return 0;
}

int rsv_download(rsv_ctx *ctx, uint32_t id, float *out, uint64_t len) {
    CHECK_CTX();
    if (no_capture(ctx, "download")) return -1;
    Tensor *t = get_tensor(ctx, id);
    if (!t) return RSV_FAIL("download: unknown tensor id %u", id);
    if (len > t->len) return RSV_FAIL("download: %llu elements exceed tensor %u", (unsigned long long)len, id);
    RSV_HIP(hipStreamSynchronize(ctx->stream));
    if (t->dtype == RSV_F16) {
        std::vector<uint16_t> h(len);
        RSV_HIP(hipMemcpy(h.data(), t->ptr, len * 2, hipMemcpyDeviceToHost));
        for (uint64_t i = 0; i < len; i++) out[i] = f16_to_f32(h[i]);
    } else {
        RSV_HIP(hipMemcpy(out, t->ptr, len * 4, hipMemcpyDeviceToHost));
    }
    return 0;
}

int rsv_download_u32(rsv_ctx *ctx, uint32_t id, uint32_t *out, uint64_t len) {
    CHECK_CTX();
    Tensor *t = get_tensor(ctx, id);
    if (!t) return RSV_FAIL("download_u32: unknown tensor id %u", id);
    if (t->dtype == RSV_F16) return RSV_FAIL("download_u32: tensor %u is F16", id);
    return rsv_download(ctx, id, (float *)out, len);
}

int rsv_copy_device(rsv_ctx *ctx, uint32_t src, uint32_t dst) {
    CHECK_CTX();
    Tensor *a = get_tensor(ctx, src), *b = get_tensor(ctx, dst);
    if (!a || !b) return RSV_FAIL("copy_device: unknown tensor");
    if (a->dtype != b->dtype) return RSV_FAIL("copy_device: dtype mismatch");
    const uint64_t n = a->len < b->len ? a->len : b->len;
    return launch_copy(ctx, b->ptr, a->ptr, n * dtype_size(a->dtype));
}

int rsv_copy_device_f16(rsv_ctx *ctx, uint32_t src, uint32_t dst) { return rsv_copy_device(ctx, src, dst); }

int rsv_context_device(rsv_ctx *ctx, int *device) {
    if (!ctx || !device) return RSV_FAIL("context_device: null argument");
    *device = ctx->device;
    return 0;
}

int rsv_import_tensors(rsv_ctx *ctx, rsv_ctx *src) {
    CHECK_CTX();
    if (!src) return RSV_FAIL("import_tensors: null source");
    if (src->device != ctx->device) return RSV_FAIL("import_tensors: source is on device %d", src->device);
    if (src == ctx) return RSV_FAIL("import_tensors: source is the destination");
    for (auto &t : ctx->tensors)
        if (t.live) return RSV_FAIL("import_tensors: destination already holds tensors");
    // Every live tensor of the source keeps its id and its memory here (the
    // allocation is shared: it stays valid until every holder has freed it,
    // so freeing in either context never leaves the other with a dangling
    // pointer).  Ids that are dead in the source are free here, and later
    // tensors of this context take those or ids past the source's table;
    // ids are per context, so the two tables may diverge from then on.
    ctx->tensors.clear();
    ctx->free_ids.clear();
    ctx->tensors.reserve(src->tensors.size());
    for (size_t i = 0; i < src->tensors.size(); i++) {
        Tensor t = src->tensors[i];
        if (t.live) t.foreign = true;
        else {
            t = Tensor();
            ctx->free_ids.push_back((uint32_t)i);
        }
        ctx->tensors.push_back(t);
    }
    std::reverse(ctx->free_ids.begin(), ctx->free_ids.end());
    return 0;
}

// ------------------------------------------------------- batching / graphs
int rsv_begin_batch(rsv_ctx *ctx) { CHECK_CTX(); return 0; }
int rsv_end_batch(rsv_ctx *ctx) { CHECK_CTX(); return 0; }
int rsv_supports_graph_capture(rsv_ctx *ctx) { (void)ctx; return 1; }
// ---------------------------------------------- fused LoRA-up + WKV7 step
int rsv_wkv7_lora_decode(rsv_ctx *ctx, const rsv_wkv_lora *op, uint64_t batch) {
    CHECK_CTX();
    if (!op) return RSV_FAIL("wkv7_lora_decode: null op");
    const uint64_t H = op->n_head, C = H * 64, B = batch;
    if (H == 0 || H > 4096 || B == 0 || B > 65535) return RSV_FAIL("wkv7_lora_decode: bad n_head %llu / batch %llu", (unsigned long long)H, (unsigned long long)B);
    const uint64_t rk[4] = {op->w_rank, op->a_rank, op->v_rank, op->g_rank};
    WkvLoraArgs a{};
    a.H = (int)H;
    for (int m = 0; m < 4; m++) {
        if (rk[m] == 0 || rk[m] > 256) return RSV_FAIL("wkv7_lora_decode: rank %llu", (unsigned long long)rk[m]);
        a.mid_n[m] = (int)rk[m];
    }
    a.eps = op->eps;
    a.gn_eps = op->gn_eps;
    void *p = nullptr;
#define WL_F32(field, id, n, what)                                   \
    if (opnd(ctx, (id), RSV_F32, (n), &p, (what))) return -1;        \
    field = (decltype(field))p;
    WL_F32(a.S, op->state, B * H * 4096, "wkv7_lora state");
    WL_F32(a.r, op->r, B * C, "wkv7_lora r");
    WL_F32(a.k, op->k, B * C, "wkv7_lora k");
    WL_F32(a.v, op->v, B * C, "wkv7_lora v");
    WL_F32(a.vf, op->v_first, B * C, "wkv7_lora v_first");
    a.f16_io = op->f16_io ? 1 : 0;
    const uint32_t mid_ids[4] = {op->w_mid, op->a_mid, op->v_mid, op->g_mid};
    for (int m = 0; m < 4; m++) {
        if (opnd(ctx, mid_ids[m], a.f16_io ? RSV_F16 : RSV_F32, B * rk[m], &p, "wkv7_lora mid")) return -1;
        a.mid[m] = p;
    }
    WL_F32(a.w0, op->w0, C, "wkv7_lora w0");
    WL_F32(a.a0, op->a0, C, "wkv7_lora a0");
    WL_F32(a.v0, op->v0, C, "wkv7_lora v0");
    WL_F32(a.scale, op->scale_w, 1, "wkv7_lora scale_w");
    WL_F32(a.kk, op->k_k, C, "wkv7_lora k_k");
    WL_F32(a.ka, op->k_a, C, "wkv7_lora k_a");
    WL_F32(a.rk, op->r_k, C, "wkv7_lora r_k");
    WL_F32(a.gamma, op->ln_x_w, C, "wkv7_lora ln_x_w");
    WL_F32(a.beta, op->ln_x_b, C, "wkv7_lora ln_x_b");
    if (opnd(ctx, op->yg, a.f16_io ? RSV_F16 : RSV_F32, B * C, &p, "wkv7_lora yg")) return -1;
    a.yg = p;
#undef WL_F32
    const uint32_t up[4] = {op->w2, op->a2, op->v2, op->g2};
    for (int m = 0; m < 4; m++) {
        if (opnd(ctx, up[m], RSV_F16, C * rk[m], &p, "wkv7_lora up")) return -1;
        a.up[m] = (const _Float16 *)p;
    }
    if (op->y_bonus != 0xFFFFFFFFu || op->y_gate != 0xFFFFFFFFu) {
        if (opnd(ctx, op->y_bonus, RSV_F32, B * C, &p, "wkv7_lora y_bonus")) return -1;
        a.y_bonus = (float *)p;
        if (opnd(ctx, op->y_gate, RSV_F32, B * C, &p, "wkv7_lora y_gate")) return -1;
        a.y_gate = (float *)p;
    }
    if (op->side_src != 0xFFFFFFFFu && op->side_dst != 0xFFFFFFFFu) {
        if (opnd(ctx, op->side_src, RSV_F32, B * C, &p, "wkv7_lora side_src")) return -1;
        a.side_src = (const float *)p;
        if (opnd(ctx, op->side_dst, RSV_F32, B * C, &p, "wkv7_lora side_dst")) return -1;
        a.side_dst = (float *)p;
    }
    return launch_wkv7_lora(ctx, a, (int)B);
}

int rsv_clear_kernel_prof(rsv_ctx *ctx) { (void)ctx; return 0; }
int rsv_dump_kernel_prof(rsv_ctx *ctx) { (void)ctx; return 0; }

int rsv_graph_begin(rsv_ctx *ctx) {
    CHECK_CTX();
    if (ctx->capturing || ctx->prefill_capturing) return RSV_FAIL("graph_begin: capture already active");
    RSV_HIP(hipStreamSynchronize(ctx->stream));
    if (ctx->graph_exec) { hipGraphExecDestroy(ctx->graph_exec); ctx->graph_exec = nullptr; }
    if (ctx->graph) { hipGraphDestroy(ctx->graph); ctx->graph = nullptr; }
    RSV_HIP(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
    ctx->capturing = true;
    return 0;
}

int rsv_graph_end(rsv_ctx *ctx) {
    CHECK_CTX();
    if (!ctx->capturing) return RSV_FAIL("graph_end: no capture active");
    ctx->capturing = false;
    RSV_HIP(hipStreamEndCapture(ctx->stream, &ctx->graph));
    RSV_HIP(hipGraphInstantiate(&ctx->graph_exec, ctx->graph, nullptr, nullptr, 0));
    return 0;
}

int rsv_graph_replay(rsv_ctx *ctx) {
    CHECK_CTX();
    if (!ctx->graph_exec) return RSV_FAIL("graph_replay: no captured graph");
    RSV_HIP(hipGraphLaunch(ctx->graph_exec, ctx->stream));
    return 0;
}

int rsv_prefill_graph_valid(rsv_ctx *ctx, uint64_t t, int *valid) {
    CHECK_CTX();
    if (!valid) return RSV_FAIL("prefill_graph_valid: null out");
    *valid = ctx->prefill_graphs.count(t) ? 1 : 0;
    // a valid graph becomes the one rsv_prefill_graph_replay runs (the
    // reference replays the last captured T, which is the wrong graph when
    // chunk sizes alternate)
    if (*valid) ctx->prefill_t = t;
    return 0;
}

int rsv_prefill_graph_begin(rsv_ctx *ctx, uint64_t t) {
    CHECK_CTX();
    if (ctx->capturing || ctx->prefill_capturing) return RSV_FAIL("prefill_graph_begin: capture already active");
    RSV_HIP(hipStreamSynchronize(ctx->stream));
    RSV_HIP(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
    ctx->prefill_capturing = true;
    ctx->prefill_t = t;
    return 0;
}

int rsv_prefill_graph_end(rsv_ctx *ctx) {
    CHECK_CTX();
    if (!ctx->prefill_capturing) return RSV_FAIL("prefill_graph_end: no capture active");
    ctx->prefill_capturing = false;
    hipGraph_t g = nullptr;
    RSV_HIP(hipStreamEndCapture(ctx->stream, &g));
    hipGraphExec_t ex = nullptr;
    hipError_t e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
    hipGraphDestroy(g);
    if (e != hipSuccess) return RSV_FAIL("prefill graph instantiate: %s", hipGetErrorString(e));
    auto it = ctx->prefill_graphs.find(ctx->prefill_t);
    if (it != ctx->prefill_graphs.end()) hipGraphExecDestroy(it->second);
    ctx->prefill_graphs[ctx->prefill_t] = ex;
    return 0;
}

int rsv_prefill_graph_replay(rsv_ctx *ctx) {
    CHECK_CTX();
    auto it = ctx->prefill_graphs.find(ctx->prefill_t);
    if (it == ctx->prefill_graphs.end()) return RSV_FAIL("prefill_graph_replay: no graph for t=%llu", (unsigned long long)ctx->prefill_t);
    RSV_HIP(hipGraphLaunch(it->second, ctx->stream));
    return 0;
}

// ------------------------------------------------------ token / sampler
int rsv_store_token(rsv_ctx *ctx, uint32_t tok, uint32_t token) {
    CHECK_CTX();
    OPND(t, tok, RSV_U32, 1, "store_token");
    return launch_set_u32(ctx, U32P(t), &token, 1);
}

int rsv_store_tokens(rsv_ctx *ctx, uint32_t tok, const uint32_t *tokens, uint64_t batch) {
    CHECK_CTX();
    OPND(t, tok, RSV_U32, batch, "store_tokens");
    return launch_set_u32(ctx, U32P(t), tokens, (int)batch);
}

int rsv_store_sampler(rsv_ctx *ctx, uint32_t sampler, float temperature, uint32_t top_k, float top_p,
                      uint32_t seed, float rep, float freq, float pres, uint32_t hist_len) {
    CHECK_CTX();
    OPND(s, sampler, RSV_F32, 8, "store_sampler");
    return launch_store_sampler(ctx, F32P(s), temperature, top_k, top_p, &seed, 1, rep, freq, pres, hist_len);
}

int rsv_store_sampler_async(rsv_ctx *ctx, uint32_t sampler, uint64_t row, float temperature, uint32_t top_k,
                            float top_p, uint32_t seed, float rep, float freq, float pres, uint32_t hist_len) {
    (void)row;  // stream-ordered kernel stores need no staging rows
    return rsv_store_sampler(ctx, sampler, temperature, top_k, top_p, seed, rep, freq, pres, hist_len);
}

int rsv_store_sampler_async_batch(rsv_ctx *ctx, uint32_t sampler, uint64_t row, float temperature, uint32_t top_k,
                                  float top_p, const uint32_t *seeds, uint64_t batch, float rep, float freq,
                                  float pres, uint32_t hist_len) {
    CHECK_CTX();
    (void)row;
    OPND(s, sampler, RSV_F32, 8 * batch, "store_sampler_async_batch");
    return launch_store_sampler(ctx, F32P(s), temperature, top_k, top_p, seeds, (int)batch, rep, freq, pres,
                                hist_len);
}

uint64_t rsv_sampler_async_rows(rsv_ctx *ctx) {
    (void)ctx;
    return (uint64_t)1 << 32;  // unbounded: rows are kernel arguments, not staging slots
}

// ------------------------------------------------------------- gather
int rsv_gather_rows_device_f16(rsv_ctx *ctx, uint32_t src, uint32_t dst, uint32_t tok, uint64_t c,
                               uint64_t batch) {
    CHECK_CTX();
    Tensor *s = get_tensor(ctx, src);
    if (!s) return RSV_FAIL("gather_rows: unknown src");
    if (s->dtype == RSV_U32) return RSV_FAIL("gather_rows: src must be F16 or F32");
    OPND(d, dst, RSV_F32, c * batch, "gather_rows dst");
    OPND(t, tok, RSV_U32, batch, "gather_rows tok");
    if (c == 0) return RSV_FAIL("gather_rows: c must be > 0");
    return launch_gather_rows(ctx, s->ptr, s->dtype == RSV_F16, s->len / c, F32P(d), U32P(t), (int)c, (int)batch);
}

int rsv_gather_row_device_f16(rsv_ctx *ctx, uint32_t src, uint32_t dst, uint32_t tok, uint64_t c) {
    return rsv_gather_rows_device_f16(ctx, src, dst, tok, c, 1);
}

// ------------------------------------------------------------- norms
int rsv_norm(rsv_ctx *ctx, uint32_t x, uint32_t gamma, uint32_t beta, uint32_t y, uint64_t c, uint64_t h,
             float eps, uint64_t rows) {
    CHECK_CTX();
    OPND(xx, x, RSV_F32, c * h * rows, "norm x");
    OPND(g, gamma, RSV_F32, c * h, "norm gamma");
    OPND(b, beta, RSV_F32, c * h, "norm beta");
    OPND(yy, y, RSV_F32, c * h * rows, "norm y");
    return launch_norm(ctx, F32P(xx), F32P(g), F32P(b), F32P(yy), (int)c, (int)h, eps, (int)rows);
}

int rsv_norm_lerp6_batch(rsv_ctx *ctx, uint32_t x, uint32_t state, uint32_t gamma, uint32_t beta, uint32_t x_r,
                         uint32_t x_w, uint32_t x_k, uint32_t x_v, uint32_t x_a, uint32_t x_g, uint32_t o_r,
                         uint32_t o_w, uint32_t o_k, uint32_t o_v, uint32_t o_a, uint32_t o_g, uint64_t c, float eps,
                         uint64_t batch) {
    CHECK_CTX();
    OPND(xx, x, RSV_F32, c * batch, "norm_lerp6 x");
    OPND(st, state, RSV_F32, c * batch, "norm_lerp6 state");
    OPND(g, gamma, RSV_F32, c, "norm_lerp6 gamma");
    OPND(b, beta, RSV_F32, c, "norm_lerp6 beta");
    const uint32_t cid[6] = {x_r, x_w, x_k, x_v, x_a, x_g}, oid[6] = {o_r, o_w, o_k, o_v, o_a, o_g};
    const float *cp[6];
    float *op[6];
    for (int j = 0; j < 6; j++) {
        void *p = nullptr;
        if (opnd(ctx, cid[j], RSV_F32, c, &p, "norm_lerp6 coef")) return -1;
        cp[j] = (const float *)p;
        if (opnd(ctx, oid[j], RSV_F32, c * batch, &p, "norm_lerp6 out")) return -1;
        op[j] = (float *)p;
    }
    return launch_norm_lerp(ctx, F32P(xx), F32P(st), F32P(g), F32P(b), cp, op, 6, (int)c, eps, (int)batch);
}

int rsv_norm_lerp6(rsv_ctx *ctx, uint32_t x, uint32_t state, uint32_t gamma, uint32_t beta, uint32_t x_r,
                   uint32_t x_w, uint32_t x_k, uint32_t x_v, uint32_t x_a, uint32_t x_g, uint32_t o_r, uint32_t o_w,
                   uint32_t o_k, uint32_t o_v, uint32_t o_a, uint32_t o_g, uint64_t c, float eps) {
    return rsv_norm_lerp6_batch(ctx, x, state, gamma, beta, x_r, x_w, x_k, x_v, x_a, x_g, o_r, o_w, o_k, o_v, o_a,
                                o_g, c, eps, 1);
}

int rsv_cmix_norm_lerp_batch(rsv_ctx *ctx, uint32_t x, uint32_t state, uint32_t gamma, uint32_t beta,
                             uint32_t x_k, uint32_t out_xb, uint64_t c, float eps, uint64_t batch) {
    CHECK_CTX();
    OPND(xx, x, RSV_F32, c * batch, "cmix x");
    OPND(st, state, RSV_F32, c * batch, "cmix state");
    OPND(g, gamma, RSV_F32, c, "cmix gamma");
    OPND(b, beta, RSV_F32, c, "cmix beta");
    OPND(k, x_k, RSV_F32, c, "cmix coef");
    OPND(o, out_xb, RSV_F32, c * batch, "cmix out");
    const float *cp[1] = {F32P(k)};
    float *op[1] = {F32P(o)};
    return launch_norm_lerp(ctx, F32P(xx), F32P(st), F32P(g), F32P(b), cp, op, 1, (int)c, eps, (int)batch);
}

int rsv_cmix_norm_lerp(rsv_ctx *ctx, uint32_t x, uint32_t state, uint32_t gamma, uint32_t beta, uint32_t x_k,
                       uint32_t out_xb, uint64_t c, float eps) {
    return rsv_cmix_norm_lerp_batch(ctx, x, state, gamma, beta, x_k, out_xb, c, eps, 1);
}

// ------------------------------------------------------------- WKV7
int rsv_fuse_ka_dplr_norm_batch(rsv_ctx *ctx, uint32_t s, uint32_t k, uint32_t k_k, uint32_t a, uint32_t k_a,
                                uint32_t r, uint32_t v, uint32_t w, uint32_t ln_x_w, uint32_t ln_x_b, uint32_t r_k,
                                uint32_t k_mod, uint32_t y, uint32_t y_norm, uint64_t h, uint64_t n, float eps,
                                float gn_eps, uint64_t batch) {
    CHECK_CTX();
    const uint64_t c = h * n;
    OPND(ss, s, RSV_F32, batch * h * n * n, "wkv state");
    OPND(kk, k, RSV_F32, c * batch, "wkv k");
    OPND(kc, k_k, RSV_F32, c, "wkv k_k");
    OPND(aa, a, RSV_F32, c * batch, "wkv a");
    OPND(kac, k_a, RSV_F32, c, "wkv k_a");
    OPND(rr, r, RSV_F32, c * batch, "wkv r");
    OPND(vv, v, RSV_F32, c * batch, "wkv v");
    OPND(ww, w, RSV_F32, c * batch, "wkv w");
    OPND(gw, ln_x_w, RSV_F32, c, "wkv ln_x_w");
    OPND(gb, ln_x_b, RSV_F32, c, "wkv ln_x_b");
    OPND(rkc, r_k, RSV_F32, c, "wkv r_k");
    OPND(yn, y_norm, RSV_F32, c * batch, "wkv y_norm");
    float *km = nullptr, *yy = nullptr;
    if (get_tensor(ctx, k_mod)) { OPND(kmv, k_mod, RSV_F32, c * batch, "wkv k_mod"); km = F32P(kmv); }
    if (get_tensor(ctx, y)) { OPND(yv, y, RSV_F32, c * batch, "wkv y"); yy = F32P(yv); }
    return launch_wkv7_decode(ctx, F32P(ss), F32P(kk), F32P(kc), F32P(aa), F32P(kac), F32P(rr), F32P(vv), F32P(ww),
                              F32P(gw), F32P(gb), F32P(rkc), km, yy, F32P(yn), (int)h, (int)n, eps, gn_eps,
                              (int)batch);
}

int rsv_fuse_ka_dplr_norm(rsv_ctx *ctx, uint32_t s, uint32_t k, uint32_t k_k, uint32_t a, uint32_t k_a, uint32_t r,
                          uint32_t v, uint32_t w, uint32_t ln_x_w, uint32_t ln_x_b, uint32_t r_k, uint32_t k_mod,
                          uint32_t y, uint32_t y_norm, uint64_t h, uint64_t n, float eps, float gn_eps) {
    return rsv_fuse_ka_dplr_norm_batch(ctx, s, k, k_k, a, k_a, r, v, w, ln_x_w, ln_x_b, r_k, k_mod, y, y_norm, h, n,
                                       eps, gn_eps, 1);
}

// ------------------------------------------------------------- GEMV jobs
static int job_f16(rsv_ctx *ctx, GemvJob &J, uint32_t w, uint64_t m, uint64_t k, const char *what) {
    void *p = nullptr;
    if (opnd(ctx, w, RSV_F16, m * k, &p, what)) return -1;
    J.w = p;
    J.sz = nullptr;
    J.fmt = FMT_F16;
    J.M = (int)m;
    J.K = (int)k;
    return 0;
}

static int job_i8(rsv_ctx *ctx, GemvJob &J, const rsv_int8 *w, uint64_t m, uint64_t k, const char *what) {
    const uint32_t *idx, *sz;
    if (int8_operands(ctx, w, m, k, &idx, &sz, what)) return -1;
    J.w = idx;
    J.sz = sz;
    J.fmt = FMT_I8;
    J.M = (int)m;
    J.K = (int)k;
    return 0;
}

static int job_xy(rsv_ctx *ctx, GemvJob &J, uint32_t x, uint32_t y, uint64_t batch, const char *what) {
    void *px = nullptr, *py = nullptr;
    if (opnd(ctx, x, RSV_F32, (uint64_t)J.K * batch, &px, what) || opnd(ctx, y, RSV_F32, (uint64_t)J.M * batch, &py, what))
        return -1;
    J.x = (const float *)px;
    J.y = (float *)py;
    J.ldx = J.K;
    J.ldy = J.M;
    return 0;
}

static int gemv_single(rsv_ctx *ctx, bool i8, uint32_t w16, const rsv_int8 *w8, uint32_t x, uint32_t g, uint32_t y,
                       uint64_t m, uint64_t k, uint64_t n, int epi, const char *what) {
    CHECK_CTX();
    GemvJobs jobs{};
    jobs.n = 1;
    GemvJob &J = jobs.j[0];
    if (i8 ? job_i8(ctx, J, w8, m, k, what) : job_f16(ctx, J, w16, m, k, what)) return -1;
    if (job_xy(ctx, J, x, y, n, what)) return -1;
    J.epi = epi;
    J.pro = PRO_NONE;
    if (g != 0xFFFFFFFFu) {
        void *pg = nullptr;
        if (opnd(ctx, g, RSV_F32, k * n, &pg, what)) return -1;
        J.xmul = (const float *)pg;
        J.pro = PRO_MUL;
    }
    return launch_gemv_jobs(ctx, jobs, (int)n);
}

int rsv_gemv_f16(rsv_ctx *ctx, uint32_t w, uint32_t x, uint32_t y, uint64_t m, uint64_t k, uint64_t n) {
    return gemv_single(ctx, false, w, nullptr, x, 0xFFFFFFFFu, y, m, k, n, EPI_STORE, "gemv_f16");
}
int rsv_gemv_f16_relu2(rsv_ctx *ctx, uint32_t w, uint32_t x, uint32_t y, uint64_t m, uint64_t k, uint64_t n) {
    return gemv_single(ctx, false, w, nullptr, x, 0xFFFFFFFFu, y, m, k, n, EPI_RELU2, "gemv_f16_relu2");
}
int rsv_gemv_f16_mul_add(rsv_ctx *ctx, uint32_t w, uint32_t x, uint32_t g, uint32_t y, uint64_t m, uint64_t k,
                         uint64_t n) {
    return gemv_single(ctx, false, w, nullptr, x, g, y, m, k, n, EPI_ADD, "gemv_f16_mul_add");
}
int rsv_gemv_f16_add(rsv_ctx *ctx, uint32_t w, uint32_t x, uint32_t y, uint64_t m, uint64_t k, uint64_t n) {
    return gemv_single(ctx, false, w, nullptr, x, 0xFFFFFFFFu, y, m, k, n, EPI_ADD, "gemv_f16_add");
}
int rsv_gemv_int8_relu2(rsv_ctx *ctx, const rsv_int8 *w, uint32_t x, uint32_t y, uint64_t m, uint64_t k, uint64_t n) {
    return gemv_single(ctx, true, 0, w, x, 0xFFFFFFFFu, y, m, k, n, EPI_RELU2, "gemv_int8_relu2");
}
int rsv_gemv_int8_mul_add(rsv_ctx *ctx, const rsv_int8 *w, uint32_t x, uint32_t g, uint32_t y, uint64_t m,
                          uint64_t k, uint64_t n) {
    return gemv_single(ctx, true, 0, w, x, g, y, m, k, n, EPI_ADD, "gemv_int8_mul_add");
}
int rsv_gemv_int8_add(rsv_ctx *ctx, const rsv_int8 *w, uint32_t x, uint32_t y, uint64_t m, uint64_t k, uint64_t n) {
    return gemv_single(ctx, true, 0, w, x, 0xFFFFFFFFu, y, m, k, n, EPI_ADD, "gemv_int8_add");
}
int rsv_gemv_int8_plain(rsv_ctx *ctx, const rsv_int8 *w, uint32_t x, uint32_t y, uint64_t m, uint64_t k, uint64_t n) {
    return gemv_single(ctx, true, 0, w, x, 0xFFFFFFFFu, y, m, k, n, EPI_STORE, "gemv_int8_plain");
}
int rsv_supports_sparse_ffn(rsv_ctx *ctx) { (void)ctx; return 1; }

int rsv_ffn_value_sparse_add_batch(rsv_ctx *ctx, uint32_t value_tiled, uint32_t r2, uint32_t x, uint64_t c,
                                   uint64_t fh, uint64_t batch) {
    CHECK_CTX();
    if (c == 0 || fh == 0 || batch == 0 || c > (1u << 20) || fh > (1u << 22) || batch > 65535)
        return RSV_FAIL("ffn_value_sparse_add: bad shape c=%llu fh=%llu batch=%llu", (unsigned long long)c,
                        (unsigned long long)fh, (unsigned long long)batch);
    OPND(vt, value_tiled, RSV_F16, c * fh, "ffn_value_sparse_add value_tiled");
    OPND(rr, r2, RSV_F32, fh * batch, "ffn_value_sparse_add r2");
    OPND(xx, x, RSV_F32, c * batch, "ffn_value_sparse_add x");
    return launch_ffn_sparse(ctx, F32P(rr), (const _Float16 *)vt_v, F32P(xx), (int)c, (int)fh, (int)batch);
}

int rsv_ffn_value_sparse_add(rsv_ctx *ctx, uint32_t value_w16, uint32_t value_tiled, uint32_t r2, uint32_t x,
                             uint64_t c, uint64_t fh) {
    (void)value_w16;
    return rsv_ffn_value_sparse_add_batch(ctx, value_tiled, r2, x, c, fh, 1);
}

int rsv_tile_ffn_value(rsv_ctx *ctx, uint32_t w16, const rsv_int8 *w8, uint64_t c, uint64_t fh, uint32_t *out) {
    CHECK_CTX();
    if (!out) return RSV_FAIL("tile_ffn_value: null out");
    if (c % 256 || fh % 128 || c == 0 || fh == 0) return RSV_FAIL("tile_ffn_value: c=%llu fh=%llu", (unsigned long long)c, (unsigned long long)fh);
    const uint32_t *idx = nullptr, *sz = nullptr;
    const _Float16 *h = nullptr;
    if (w8) {
        if (int8_operands(ctx, w8, c, fh, &idx, &sz, "tile_ffn_value")) return -1;
    } else {
        void *p = nullptr;
        if (opnd(ctx, w16, RSV_F16, c * fh, &p, "tile_ffn_value w16")) return -1;
        h = (const _Float16 *)p;
    }
    uint32_t id;
    if (rsv_tensor_create(ctx, c * fh, RSV_F16, &id)) return -1;
    Tensor *t = get_tensor(ctx, id);
    if (launch_tile_ffn_value(ctx, (const uint8_t *)idx, sz, h, (_Float16 *)t->ptr, (int)c, (int)fh)) {
        rsv_tensor_free(ctx, id);
        return -1;
    }
    *out = id;
    return 0;
}

static int stage1(rsv_ctx *ctx, bool i8, uint32_t rw16, uint32_t kw16, uint32_t vw16, const rsv_int8 *rw8,
                  const rsv_int8 *kw8, const rsv_int8 *vw8, uint32_t v1, uint32_t w1, uint32_t a1, uint32_t g1,
                  uint32_t xr, uint32_t xk, uint32_t xv, uint32_t xw, uint32_t xa, uint32_t xg, uint32_t r,
                  uint32_t k, uint32_t v, uint32_t v_mid, uint32_t w_mid, uint32_t a_mid, uint32_t g_mid,
                  uint64_t c, uint64_t vm, uint64_t wm, uint64_t am, uint64_t gm, uint64_t batch) {
    CHECK_CTX();
    GemvJobs jobs{};
    jobs.n = 7;
    const char *nm = "gemv_rkv_stage1";
    if (i8) {
        if (job_i8(ctx, jobs.j[0], rw8, c, c, nm) || job_i8(ctx, jobs.j[1], kw8, c, c, nm) ||
            job_i8(ctx, jobs.j[2], vw8, c, c, nm))
            return -1;
    } else {
        if (job_f16(ctx, jobs.j[0], rw16, c, c, nm) || job_f16(ctx, jobs.j[1], kw16, c, c, nm) ||
            job_f16(ctx, jobs.j[2], vw16, c, c, nm))
            return -1;
    }
    if (job_f16(ctx, jobs.j[3], v1, vm, c, nm) || job_f16(ctx, jobs.j[4], w1, wm, c, nm) ||
        job_f16(ctx, jobs.j[5], a1, am, c, nm) || job_f16(ctx, jobs.j[6], g1, gm, c, nm))
        return -1;
    const uint32_t xs[7] = {xr, xk, xv, xv, xw, xa, xg};
    const uint32_t ys[7] = {r, k, v, v_mid, w_mid, a_mid, g_mid};
    for (int i = 0; i < 7; i++) {
        if (job_xy(ctx, jobs.j[i], xs[i], ys[i], batch, nm)) return -1;
        jobs.j[i].epi = i == 4 ? EPI_TANH : EPI_STORE;
        jobs.j[i].pro = PRO_NONE;
    }
    return launch_gemv_jobs(ctx, jobs, (int)batch);
}

int rsv_gemv_rkv_stage1_batch(rsv_ctx *ctx, uint32_t rw, uint32_t kw, uint32_t vw, uint32_t v1, uint32_t w1,
                              uint32_t a1, uint32_t g1, uint32_t xr, uint32_t xk, uint32_t xv, uint32_t xw, uint32_t xa,
                              uint32_t xg, uint32_t r, uint32_t k, uint32_t v, uint32_t v_mid, uint32_t w_mid,
                              uint32_t a_mid, uint32_t g_mid, uint64_t c, uint64_t vm, uint64_t wm, uint64_t am,
                              uint64_t gm, uint64_t batch) {
    return stage1(ctx, false, rw, kw, vw, nullptr, nullptr, nullptr, v1, w1, a1, g1, xr, xk, xv, xw, xa, xg, r, k, v,
                  v_mid, w_mid, a_mid, g_mid, c, vm, wm, am, gm, batch);
}
int rsv_gemv_rkv_stage1(rsv_ctx *ctx, uint32_t rw, uint32_t kw, uint32_t vw, uint32_t v1, uint32_t w1, uint32_t a1,
                        uint32_t g1, uint32_t xr, uint32_t xk, uint32_t xv, uint32_t xw, uint32_t xa, uint32_t xg,
                        uint32_t r, uint32_t k, uint32_t v, uint32_t v_mid, uint32_t w_mid, uint32_t a_mid,
                        uint32_t g_mid, uint64_t c, uint64_t vm, uint64_t wm, uint64_t am, uint64_t gm) {
    return rsv_gemv_rkv_stage1_batch(ctx, rw, kw, vw, v1, w1, a1, g1, xr, xk, xv, xw, xa, xg, r, k, v, v_mid, w_mid,
                                     a_mid, g_mid, c, vm, wm, am, gm, 1);
}
int rsv_gemv_int8_rkv_stage1_batch(rsv_ctx *ctx, const rsv_int8 *rw, const rsv_int8 *kw, const rsv_int8 *vw,
                                   uint32_t v1, uint32_t w1, uint32_t a1, uint32_t g1, uint32_t xr, uint32_t xk,
                                   uint32_t xv, uint32_t xw, uint32_t xa, uint32_t xg, uint32_t r, uint32_t k,
                                   uint32_t v, uint32_t v_mid, uint32_t w_mid, uint32_t a_mid, uint32_t g_mid,
                                   uint64_t c, uint64_t vm, uint64_t wm, uint64_t am, uint64_t gm, uint64_t batch) {
    return stage1(ctx, true, 0, 0, 0, rw, kw, vw, v1, w1, a1, g1, xr, xk, xv, xw, xa, xg, r, k, v, v_mid, w_mid,
                  a_mid, g_mid, c, vm, wm, am, gm, batch);
}
int rsv_gemv_int8_rkv_stage1(rsv_ctx *ctx, const rsv_int8 *rw, const rsv_int8 *kw, const rsv_int8 *vw, uint32_t v1,
                             uint32_t w1, uint32_t a1, uint32_t g1, uint32_t xr, uint32_t xk, uint32_t xv, uint32_t xw,
                             uint32_t xa, uint32_t xg, uint32_t r, uint32_t k, uint32_t v, uint32_t v_mid,
                             uint32_t w_mid, uint32_t a_mid, uint32_t g_mid, uint64_t c, uint64_t vm, uint64_t wm,
                             uint64_t am, uint64_t gm) {
    return rsv_gemv_int8_rkv_stage1_batch(ctx, rw, kw, vw, v1, w1, a1, g1, xr, xk, xv, xw, xa, xg, r, k, v, v_mid,
                                          w_mid, a_mid, g_mid, c, vm, wm, am, gm, 1);
}

int rsv_gemv_lowrank_chain4_batch(rsv_ctx *ctx, uint32_t w2, uint32_t a2, uint32_t v2, uint32_t g2, uint32_t w_mid,
                                  uint32_t a_mid, uint32_t v_mid, uint32_t g_mid, uint32_t w0, uint32_t a0,
                                  uint32_t v0, uint32_t scale_w, uint32_t v_first, uint32_t w_out, uint32_t a_out,
                                  uint32_t v_inout, uint32_t g_out, uint64_t c, uint64_t wm, uint64_t am, uint64_t vm,
                                  uint64_t gm, uint64_t batch) {
    CHECK_CTX();
    const char *nm = "gemv_lowrank_chain4";
    GemvJobs jobs{};
    jobs.n = 4;
    if (job_f16(ctx, jobs.j[0], w2, c, wm, nm) || job_f16(ctx, jobs.j[1], a2, c, am, nm) ||
        job_f16(ctx, jobs.j[2], v2, c, vm, nm) || job_f16(ctx, jobs.j[3], g2, c, gm, nm))
        return -1;
    const uint32_t xs[4] = {w_mid, a_mid, v_mid, g_mid}, ys[4] = {w_out, a_out, v_inout, g_out};
    for (int i = 0; i < 4; i++) {
        if (job_xy(ctx, jobs.j[i], xs[i], ys[i], batch, nm)) return -1;
        jobs.j[i].pro = PRO_NONE;
    }
    OPND(pw0, w0, RSV_F32, c, nm);
    OPND(pa0, a0, RSV_F32, c, nm);
    OPND(pv0, v0, RSV_F32, c, nm);
    OPND(psc, scale_w, RSV_F32, 1, nm);
    OPND(pvf, v_first, RSV_F32, c * batch, nm);
    jobs.j[0].epi = EPI_WDECAY;
    jobs.j[0].p0 = F32P(pw0);
    jobs.j[0].scale = F32P(psc);
    jobs.j[1].epi = EPI_SIGBIAS;
    jobs.j[1].p0 = F32P(pa0);
    jobs.j[2].epi = EPI_VLERP;
    jobs.j[2].p0 = F32P(pv0);
    jobs.j[2].p1 = F32P(pvf);
    jobs.j[3].epi = EPI_STORE;
    jobs.j[3].pro = PRO_SIGMOID;
    return launch_gemv_jobs(ctx, jobs, (int)batch);
}

int rsv_gemv_lowrank_chain4(rsv_ctx *ctx, uint32_t w2, uint32_t a2, uint32_t v2, uint32_t g2, uint32_t w_mid,
                            uint32_t a_mid, uint32_t v_mid, uint32_t g_mid, uint32_t w0, uint32_t a0, uint32_t v0,
                            uint32_t scale_w, uint32_t v_first, uint32_t w_out, uint32_t a_out, uint32_t v_inout,
                            uint32_t g_out, uint64_t c, uint64_t wm, uint64_t am, uint64_t vm, uint64_t gm) {
    return rsv_gemv_lowrank_chain4_batch(ctx, w2, a2, v2, g2, w_mid, a_mid, v_mid, g_mid, w0, a0, v0, scale_w, v_first,
                                         w_out, a_out, v_inout, g_out, c, wm, am, vm, gm, 1);
}

// ------------------------------------------------------------- dequant
int rsv_dequant_int8_f32(rsv_ctx *ctx, const rsv_int8 *a, uint32_t out) {
    CHECK_CTX();
    if (!a) return RSV_FAIL("dequant: null handle");
    const uint32_t *idx, *sz;
    if (int8_operands(ctx, a, a->m, a->k, &idx, &sz, "dequant_int8_f32")) return -1;
    OPND(o, out, RSV_F32, a->m * a->k, "dequant_int8_f32 out");
    return launch_dequant_int8(ctx, idx, sz, a->m, a->k, o_v, 0);
}

int rsv_dequant_int8_to_f16(rsv_ctx *ctx, const rsv_int8 *a, uint32_t out, uint64_t m, uint64_t k) {
    CHECK_CTX();
    const uint32_t *idx, *sz;
    if (int8_operands(ctx, a, m, k, &idx, &sz, "dequant_int8_to_f16")) return -1;
    OPND(o, out, RSV_F16, m * k, "dequant_int8_to_f16 out");
    return launch_dequant_int8(ctx, idx, sz, m, k, o_v, 1);
}

// ------------------------------------------------------- argmax / sampling
int rsv_argmax_batch(rsv_ctx *ctx, uint32_t logits, uint32_t token, uint64_t n, uint64_t batch) {
    CHECK_CTX();
    OPND(l, logits, RSV_F32, n * batch, "argmax logits");
    OPND(t, token, RSV_U32, batch, "argmax token");
    return launch_argmax(ctx, F32P(l), U32P(t), (int)n, (int)batch);
}
int rsv_argmax_record_gather_batch(rsv_ctx *ctx, uint32_t logits, uint32_t token, uint64_t n, uint32_t out_seq,
                                   uint32_t cnt, uint64_t stride, uint32_t emb, uint32_t x, uint64_t c,
                                   uint64_t batch) {
    CHECK_CTX();
    OPND(l, logits, RSV_F32, n * batch, "argmax_record_gather logits");
    OPND(t, token, RSV_U32, batch, "argmax_record_gather token");
    OPND(os, out_seq, RSV_U32, stride * batch, "argmax_record_gather out_seq");
    OPND(cn, cnt, RSV_U32, batch, "argmax_record_gather cnt");
    OPND(xd, x, RSV_F32, c * batch, "argmax_record_gather x");
    Tensor *e = get_tensor(ctx, emb);
    if (!e) return RSV_FAIL("argmax_record_gather: unknown emb");
    if (e->dtype == RSV_U32) return RSV_FAIL("argmax_record_gather: emb must be F16 or F32");
    if (c == 0 || stride == 0) return RSV_FAIL("argmax_record_gather: c and stride must be > 0");
    return launch_argmax_next(ctx, F32P(l), U32P(t), (int)n, U32P(os), U32P(cn), (int)stride, e->ptr,
                              e->dtype == RSV_F16, e->len / c, F32P(xd), (int)c, (int)batch);
}
int rsv_argmax(rsv_ctx *ctx, uint32_t logits, uint32_t token, uint64_t n) {
    return rsv_argmax_batch(ctx, logits, token, n, 1);
}
int rsv_argmax_into_host(rsv_ctx *ctx, uint32_t logits, uint32_t token, uint64_t n) {
    return rsv_argmax_batch(ctx, logits, token, n, 1);
}

int rsv_sample_into_host_seeded_batch(rsv_ctx *ctx, uint32_t logits, uint32_t token, uint64_t n, uint32_t temp,
                                      uint32_t mask, uint32_t counter, uint32_t sampler, uint32_t hist,
                                      uint64_t batch) {
    CHECK_CTX();
    (void)mask;
    OPND(l, logits, RSV_F32, n * batch, "sample logits");
    OPND(t, token, RSV_U32, batch, "sample token");
    OPND(tp, temp, RSV_F32, n * batch, "sample temp");
    OPND(ct, counter, RSV_U32, n * batch, "sample counter");
    OPND(sp, sampler, RSV_F32, 8 * batch, "sample sampler");
    if (batch == 0) return RSV_FAIL("sample: batch must be >= 1");
    Tensor *h = get_tensor(ctx, hist);
    if (!h) return RSV_FAIL("sample: unknown hist tensor %u", hist);
    // each row's history capacity; the kernel reads no further than this
    const int stride = (int)(h->len / batch);
    return launch_sample(ctx, F32P(l), U32P(t), (int)n, F32P(tp), U32P(ct), F32P(sp), (const uint32_t *)h->ptr,
                         stride, (int)batch);
}

int rsv_sample_into_host_seeded(rsv_ctx *ctx, uint32_t logits, uint32_t token, uint64_t n, uint32_t temp,
                                uint32_t mask, uint32_t counter, uint32_t sampler, uint32_t hist) {
    return rsv_sample_into_host_seeded_batch(ctx, logits, token, n, temp, mask, counter, sampler, hist, 1);
}

int rsv_sample(rsv_ctx *ctx, uint32_t logits, uint32_t token, uint64_t n, float temperature, uint32_t top_k,
               float top_p, uint32_t seed, float rep, float freq, float pres, const uint32_t *history,
               uint64_t hist_len) {
    CHECK_CTX();
    if (no_capture(ctx, "sample")) return -1;
    OPND(l, logits, RSV_F32, n, "sample logits");
    OPND(t, token, RSV_U32, 1, "sample token");
    // work: temp [n] f32 + counter [n] u32 + sampler row [8]
    const uint64_t need = 2 * n + 8;
    if (ctx->sample_work_cap < need) {
        RSV_HIP(hipStreamSynchronize(ctx->stream));
        if (ctx->sample_work) hipFree(ctx->sample_work);
        RSV_HIP(hipMalloc(&ctx->sample_work, need * 4));
        ctx->sample_work_cap = need;
    }
    if (hist_len > 0) {
        if (ctx->hist_cap < hist_len) {
            RSV_HIP(hipStreamSynchronize(ctx->stream));
            if (ctx->hist_dev) hipFree(ctx->hist_dev);
            RSV_HIP(hipMalloc(&ctx->hist_dev, hist_len * 4));
            ctx->hist_cap = hist_len;
        }
        RSV_HIP(hipStreamSynchronize(ctx->stream));
        RSV_HIP(hipMemcpy(ctx->hist_dev, history, hist_len * 4, hipMemcpyHostToDevice));
    }
    float *temp = ctx->sample_work;
    uint32_t *counter = (uint32_t *)(ctx->sample_work + n);
    float *srow = ctx->sample_work + 2 * n;
    if (launch_store_sampler(ctx, srow, temperature, top_k, top_p, &seed, 1, rep, freq, pres, (uint32_t)hist_len))
        return -1;
    return launch_sample(ctx, F32P(l), U32P(t), (int)n, temp, counter, srow, hist_len ? ctx->hist_dev : nullptr,
                         (int)hist_len, 1);
}

int rsv_sample_noalloc(rsv_ctx *ctx, uint32_t logits, uint32_t token, uint64_t n, float temperature, uint32_t top_k,
                       float top_p, uint32_t seed, float rep, float freq, float pres, uint32_t hist,
                       uint64_t hist_len) {
    CHECK_CTX();
    if (n == 0 || n > kNoAllocMaxN)
        return RSV_FAIL("sample_noalloc: n=%llu outside 1..%llu (the static work area's limit)",
                        (unsigned long long)n, (unsigned long long)kNoAllocMaxN);
    OPND(l, logits, RSV_F32, n, "sample_noalloc logits");
    OPND(t, token, RSV_U32, 1, "sample_noalloc token");
    const uint32_t *hp = nullptr;
    if (hist_len > 0) {
        if (hist_len > 0xFFFFFFFFull) return RSV_FAIL("sample_noalloc: hist_len too large");
        OPND(hh, hist, RSV_U32, hist_len, "sample_noalloc history");
        hp = U32P(hh);
    }
    if (sample_scratch_claim(ctx->device, ctx)) return -1;
    uint32_t *work = sample_scratch(ctx->device);
    if (!work) return RSV_FAIL("sample_noalloc: no work area on device %d", ctx->device);
    // temp [n] f32, counter [n] u32, sampler row [8]: every word the kernel
    // reads is written first in this call (the row here, temp and counter in
    // the kernel), so the previous call's contents do not matter
    float *temp = (float *)work;
    uint32_t *counter = work + n;
    float *srow = (float *)(work + 2 * n);
    if (launch_store_sampler(ctx, srow, temperature, top_k, top_p, &seed, 1, rep, freq, pres, (uint32_t)hist_len))
        return -1;
    return launch_sample(ctx, F32P(l), U32P(t), (int)n, temp, counter, srow, hp, (int)hist_len, 1);
}

int rsv_record_tokens(rsv_ctx *ctx, uint32_t in_tok, uint32_t out_seq, uint32_t cnt, uint64_t stride, uint64_t batch) {
    CHECK_CTX();
    OPND(it, in_tok, RSV_U32, batch, "record in_tok");
    OPND(os, out_seq, RSV_U32, stride * batch, "record out_seq");
    OPND(cn, cnt, RSV_U32, batch, "record cnt");
    return launch_record_tokens(ctx, U32P(it), U32P(os), U32P(cn), (int)stride, (int)batch);
}

int rsv_record_gather_batch(rsv_ctx *ctx, uint32_t in_tok, uint32_t out_seq, uint32_t cnt, uint64_t stride,
                            uint32_t emb, uint32_t x, uint64_t c, uint64_t batch) {
    CHECK_CTX();
    OPND(it, in_tok, RSV_U32, batch, "record_gather in_tok");
    OPND(os, out_seq, RSV_U32, stride * batch, "record_gather out_seq");
    OPND(cn, cnt, RSV_U32, batch, "record_gather cnt");
    OPND(xd, x, RSV_F32, c * batch, "record_gather x");
    Tensor *e = get_tensor(ctx, emb);
    if (!e) return RSV_FAIL("record_gather: unknown emb");
    if (e->dtype == RSV_U32) return RSV_FAIL("record_gather: emb must be F16 or F32");
    if (c == 0 || stride == 0) return RSV_FAIL("record_gather: c and stride must be > 0");
    return launch_record_gather(ctx, U32P(it), U32P(os), U32P(cn), (int)stride, e->ptr, e->dtype == RSV_F16,
                                e->len / c, F32P(xd), (int)c, (int)batch);
}

int rsv_record_token(rsv_ctx *ctx, uint32_t in_tok, uint32_t out_seq, uint32_t cnt) {
    CHECK_CTX();
    Tensor *o = get_tensor(ctx, out_seq);
    if (!o) return RSV_FAIL("record_token: unknown out_seq");
    return rsv_record_tokens(ctx, in_tok, out_seq, cnt, o->len, 1);
}

// ------------------------------------------------------------- prefill ops
int rsv_copy_token(rsv_ctx *ctx, uint32_t x, uint32_t y, uint64_t c, uint64_t stride, uint64_t token) {
    CHECK_CTX();
    OPND(xx, x, RSV_F32, token * stride + c, "copy_token x");
    OPND(yy, y, RSV_F32, c, "copy_token y");
    return launch_copy(ctx, F32P(yy), F32P(xx) + token * stride, c * 4);
}

int rsv_copy_token_batch(rsv_ctx *ctx, uint32_t x, uint32_t state, uint32_t lens, uint64_t c, uint64_t t,
                         uint64_t batch) {
    CHECK_CTX();
    OPND(xx, x, RSV_F32, c * t * batch, "copy_token_batch x");
    OPND(st, state, RSV_F32, c * batch, "copy_token_batch state");
    OPND(ln, lens, RSV_U32, batch, "copy_token_batch lens");
    return launch_copy_token_batch(ctx, F32P(xx), F32P(st), U32P(ln), (int)c, (int)t, (int)batch);
}

static int gemm_common(rsv_ctx *ctx, uint32_t a, uint32_t b, uint32_t aux, uint32_t c, uint64_t m, uint64_t n,
                       uint64_t k, int epi, const char *what) {
    CHECK_CTX();
    OPND(pa, a, RSV_F16, m * k, what);
    OPND(pb, b, RSV_F16, n * k, what);
    OPND(pc, c, RSV_F32, m * n, what);
    GemmArgs g{};
    if (epi == GE_BIAS) { OPND(px, aux, RSV_F32, n, what); g.bias = F32P(px); }
    if (epi == GE_ADD) { OPND(px, aux, RSV_F32, m * n, what); g.aux = F32P(px); }
    g.a = (const _Float16 *)pa_v;
    g.b = pb_v;
    g.c = pc_v;
    g.m = (int)m; g.n = (int)n; g.k = (int)k;
    g.lda = (int)k; g.ldc = (int)n;
    g.epi = epi;
    return launch_gemm(ctx, g);
}

int rsv_gemm(rsv_ctx *ctx, uint32_t a, uint32_t b, uint32_t c, uint64_t m, uint64_t n, uint64_t k) {
    return gemm_common(ctx, a, b, 0, c, m, n, k, GE_STORE, "gemm");
}
int rsv_gemm_bias(rsv_ctx *ctx, uint32_t a, uint32_t b, uint32_t bias, uint32_t c, uint64_t m, uint64_t n, uint64_t k) {
    return gemm_common(ctx, a, b, bias, c, m, n, k, GE_BIAS, "gemm_bias");
}
int rsv_gemm_add(rsv_ctx *ctx, uint32_t a, uint32_t b, uint32_t x, uint32_t y, uint64_t m, uint64_t n, uint64_t k) {
    // y = A B^T + x
    if (x != y) {
        if (rsv_copy_device(ctx, x, y)) return -1;
    }
    return gemm_common(ctx, a, b, y, y, m, n, k, GE_ADD, "gemm_add");
}
int rsv_gemm_relu2(rsv_ctx *ctx, uint32_t a, uint32_t b, uint32_t c, uint64_t m, uint64_t n, uint64_t k) {
    return gemm_common(ctx, a, b, 0, c, m, n, k, GE_RELU2, "gemm_relu2");
}
int rsv_gemm_tanh(rsv_ctx *ctx, uint32_t a, uint32_t b, uint32_t c, uint64_t m, uint64_t n, uint64_t k) {
    return gemm_common(ctx, a, b, 0, c, m, n, k, GE_TANH, "gemm_tanh");
}

int rsv_gemm_int8(rsv_ctx *ctx, uint32_t a, const rsv_int8 *w, uint32_t c, uint64_t m, int epilogue) {
    CHECK_CTX();
    if (!w) return RSV_FAIL("gemm_int8: null handle");
    const uint32_t *idx, *sz;
    if (int8_operands(ctx, w, w->m, w->k, &idx, &sz, "gemm_int8")) return -1;
    OPND(pa, a, RSV_F16, m * w->k, "gemm_int8 a");
    OPND(pc, c, RSV_F32, m * w->m, "gemm_int8 c");
    if (epilogue != GE_STORE && epilogue != GE_ADD && epilogue != GE_RELU2)
        return RSV_FAIL("gemm_int8: epilogue %d not supported", epilogue);
    GemmArgs g{};
    g.a = (const _Float16 *)pa_v;
    g.b = idx;
    g.sz = sz;
    g.c = pc_v;
    g.aux = epilogue == GE_ADD ? F32P(pc) : nullptr;
    g.m = (int)m; g.n = (int)w->m; g.k = (int)w->k;
    g.lda = (int)w->k; g.ldc = (int)w->m;
    g.epi = epilogue;
    g.b_i8 = 1;
    return launch_gemm(ctx, g);
}

int rsv_to_f16(rsv_ctx *ctx, uint32_t x, uint32_t y, uint64_t c, uint64_t t, uint64_t m_pad, uint64_t x_stride,
               uint64_t y_stride) {
    CHECK_CTX();
    OPND(xx, x, RSV_F32, t ? (t - 1) * x_stride + c : 0, "to_f16 x");
    OPND(yy, y, RSV_F16, m_pad ? (m_pad - 1) * y_stride + c : 0, "to_f16 y");
    return launch_to_f16(ctx, F32P(xx), (_Float16 *)yy_v, (int)c, (int)t, (int)m_pad, (int)x_stride, (int)y_stride);
}

int rsv_to_f16_triple(rsv_ctx *ctx, uint32_t xr, uint32_t xk, uint32_t xv, uint32_t yr, uint32_t yk, uint32_t yv,
                      uint64_t c, uint64_t t, uint64_t m_pad, uint64_t x_stride, uint64_t y_stride) {
    if (rsv_to_f16(ctx, xr, yr, c, t, m_pad, x_stride, y_stride)) return -1;
    if (rsv_to_f16(ctx, xk, yk, c, t, m_pad, x_stride, y_stride)) return -1;
    return rsv_to_f16(ctx, xv, yv, c, t, m_pad, x_stride, y_stride);
}

int rsv_elementwise_sigmoid(rsv_ctx *ctx, uint32_t a, uint32_t y, uint64_t c, uint64_t batch) {
    CHECK_CTX();
    OPND(pa, a, RSV_F32, c * batch, "sigmoid a");
    OPND(py, y, RSV_F32, c * batch, "sigmoid y");
    return launch_elementwise(ctx, 0, F32P(pa), nullptr, F32P(py), (int)c, (int)batch);
}
int rsv_elementwise_sigmoid_inplace(rsv_ctx *ctx, uint32_t y, uint64_t c, uint64_t batch) {
    CHECK_CTX();
    OPND(py, y, RSV_F32, c * batch, "sigmoid_inplace y");
    return launch_elementwise(ctx, 1, nullptr, nullptr, F32P(py), (int)c, (int)batch);
}
int rsv_elementwise_scale_exp(rsv_ctx *ctx, uint32_t a, uint32_t b, uint32_t y, uint64_t c, uint64_t batch) {
    CHECK_CTX();
    OPND(pa, a, RSV_F32, c * batch, "scale_exp a");
    OPND(pb, b, RSV_F32, 1, "scale_exp b");
    OPND(py, y, RSV_F32, c * batch, "scale_exp y");
    Tensor *tb = get_tensor(ctx, b);
    if (tb->len < batch) {
        // one scalar shared by every row: expand by launching per row block
        for (uint64_t r = 0; r < batch; r++)
            if (launch_elementwise(ctx, 2, F32P(pa) + r * c, F32P(pb), F32P(py) + r * c, (int)c, 1)) return -1;
        return 0;
    }
    return launch_elementwise(ctx, 2, F32P(pa), F32P(pb), F32P(py), (int)c, (int)batch);
}
int rsv_elementwise_mul(rsv_ctx *ctx, uint32_t a, uint32_t b, uint32_t y, uint64_t c, uint64_t batch) {
    CHECK_CTX();
    OPND(pa, a, RSV_F32, c * batch, "mul a");
    OPND(pb, b, RSV_F32, c * batch, "mul b");
    OPND(py, y, RSV_F32, c * batch, "mul y");
    return launch_elementwise(ctx, 3, F32P(pa), F32P(pb), F32P(py), (int)c, (int)batch);
}
int rsv_v_first_lerp(rsv_ctx *ctx, uint32_t v, uint32_t gate, uint32_t v_first, uint64_t c, uint64_t t,
                     uint64_t stride) {
    CHECK_CTX();
    OPND(pv, v, RSV_F32, t ? (t - 1) * stride + c : 0, "v_first_lerp v");
    OPND(pg, gate, RSV_F32, t ? (t - 1) * stride + c : 0, "v_first_lerp gate");
    OPND(pf, v_first, RSV_F32, c, "v_first_lerp v_first");
    return launch_v_first_lerp(ctx, F32P(pv), F32P(pg), F32P(pf), (int)c, (int)t, (int)stride);
}
int rsv_fuse_ka(rsv_ctx *ctx, uint32_t k, uint32_t k_k, uint32_t a, uint32_t k_a, uint32_t k_mod, uint32_t kk_l2,
                uint32_t b, uint64_t h, uint64_t n, uint64_t batch) {
    CHECK_CTX();
    const uint64_t c = h * n;
    OPND(pk, k, RSV_F32, c * batch, "fuse_ka k");
    OPND(pkk, k_k, RSV_F32, c, "fuse_ka k_k");
    OPND(pa, a, RSV_F32, c * batch, "fuse_ka a");
    OPND(pka, k_a, RSV_F32, c, "fuse_ka k_a");
    OPND(pkm, k_mod, RSV_F32, c * batch, "fuse_ka k_mod");
    OPND(pl2, kk_l2, RSV_F32, c * batch, "fuse_ka kk_l2");
    OPND(pb, b, RSV_F32, c * batch, "fuse_ka b");
    return launch_fuse_ka(ctx, F32P(pk), F32P(pkk), F32P(pa), F32P(pka), F32P(pkm), F32P(pl2), F32P(pb), (int)h,
                          (int)n, (int)batch);
}
int rsv_sum_rk_rk(rsv_ctx *ctx, uint32_t r, uint32_t k_mod, uint32_t r_k, uint32_t v, uint32_t y, uint64_t h,
                  uint64_t n, uint64_t batch) {
    CHECK_CTX();
    const uint64_t c = h * n;
    OPND(pr, r, RSV_F32, c * batch, "sum_rk_rk r");
    OPND(pk, k_mod, RSV_F32, c * batch, "sum_rk_rk k_mod");
    OPND(prk, r_k, RSV_F32, c, "sum_rk_rk r_k");
    OPND(pv, v, RSV_F32, c * batch, "sum_rk_rk v");
    OPND(py, y, RSV_F32, c * batch, "sum_rk_rk y");
    return launch_sum_rk_rk(ctx, F32P(pr), F32P(pk), F32P(prk), F32P(pv), F32P(py), (int)h, (int)n, (int)batch);
}
int rsv_seq_shift_batch(rsv_ctx *ctx, uint32_t x, uint32_t state, uint32_t tm, uint32_t y, uint64_t c, uint64_t t,
                        uint64_t stride_x, uint64_t stride_y, uint64_t batch) {
    CHECK_CTX();
    OPND(px, x, RSV_F32, t ? (batch * t - 1) * stride_x + c : 0, "seq_shift x");
    OPND(ps, state, RSV_F32, c * batch, "seq_shift state");
    OPND(pt, tm, RSV_F32, c, "seq_shift tm");
    OPND(py, y, RSV_F32, t ? (batch * t - 1) * stride_y + c : 0, "seq_shift y");
    return launch_seq_shift(ctx, F32P(px), F32P(ps), F32P(pt), F32P(py), (int)c, (int)t, (int)stride_x,
                            (int)stride_y, (int)batch);
}
int rsv_seq_shift(rsv_ctx *ctx, uint32_t x, uint32_t state, uint32_t tm, uint32_t y, uint64_t c, uint64_t t,
                  uint64_t stride_x, uint64_t stride_y) {
    return rsv_seq_shift_batch(ctx, x, state, tm, y, c, t, stride_x, stride_y, 1);
}
int rsv_dplr_seq_batch(rsv_ctx *ctx, uint32_t s, uint32_t r, uint32_t w, uint32_t k, uint32_t v, uint32_t a,
                       uint32_t b, uint32_t y, uint32_t lens, uint64_t h, uint64_t n, uint64_t t, uint64_t c,
                       uint64_t batch) {
    CHECK_CTX();
    const uint64_t tot = c * t * batch;
    OPND(ps, s, RSV_F32, batch * h * n * n, "dplr_seq s");
    OPND(pr, r, RSV_F32, tot, "dplr_seq r");
    OPND(pw, w, RSV_F32, tot, "dplr_seq w");
    OPND(pk, k, RSV_F32, tot, "dplr_seq k");
    OPND(pv, v, RSV_F32, tot, "dplr_seq v");
    OPND(pa, a, RSV_F32, tot, "dplr_seq a");
    OPND(pb, b, RSV_F32, tot, "dplr_seq b");
    OPND(py, y, RSV_F32, tot, "dplr_seq y");
    const uint32_t *pl = nullptr;
    if (lens != 0xFFFFFFFFu) { OPND(plv, lens, RSV_U32, batch, "dplr_seq lens"); pl = U32P(plv); }
    return launch_dplr_seq(ctx, F32P(ps), F32P(pr), F32P(pw), F32P(pk), F32P(pv), F32P(pa), F32P(pb), F32P(py), pl,
                           (int)h, (int)n, (int)t, (int)c, (int)batch);
}
int rsv_dplr_seq(rsv_ctx *ctx, uint32_t s, uint32_t r, uint32_t w, uint32_t k, uint32_t v, uint32_t a, uint32_t b,
                 uint32_t y, uint64_t h, uint64_t n, uint64_t t, uint64_t c) {
    return rsv_dplr_seq_batch(ctx, s, r, w, k, v, a, b, y, 0xFFFFFFFFu, h, n, t, c, 1);
}
int rsv_segmean(rsv_ctx *ctx, uint32_t x, uint32_t out, uint32_t lens, uint64_t c, uint64_t t_pad, uint64_t batch) {
    CHECK_CTX();
    OPND(px, x, RSV_F32, c * t_pad * batch, "segmean x");
    OPND(po, out, RSV_F32, c * batch, "segmean out");
    OPND(pl, lens, RSV_U32, batch, "segmean lens");
    return launch_segmean(ctx, F32P(px), F32P(po), U32P(pl), (int)c, (int)t_pad, (int)batch);
}

int rsv_wkv7_seq_ragged(rsv_ctx *ctx, uint32_t s, uint32_t r, uint32_t w, uint32_t k, uint32_t v, uint32_t a,
                        uint32_t k_k, uint32_t k_a, uint32_t r_k, uint32_t ln_x_w, uint32_t ln_x_b, uint32_t y_norm,
                        uint32_t seg_start, uint32_t seg_len, uint32_t seg_slot, uint64_t nseg, uint64_t h,
                        uint64_t n, float gn_eps) {
    CHECK_CTX();
    const uint64_t c = h * n;
    Tensor *tr = get_tensor(ctx, r), *ts = get_tensor(ctx, s);
    if (!tr || !ts) return RSV_FAIL("wkv7_seq_ragged: unknown tensor");
    const uint64_t rows = tr->len / c, slots = ts->len / (h * n * n);
    OPND(ps, s, RSV_F32, slots * h * n * n, "wkv7_seq s");
    OPND(pr, r, RSV_F32, rows * c, "wkv7_seq r");
    OPND(pw, w, RSV_F32, rows * c, "wkv7_seq w");
    OPND(pk, k, RSV_F32, rows * c, "wkv7_seq k");
    OPND(pv, v, RSV_F32, rows * c, "wkv7_seq v");
    OPND(pa, a, RSV_F32, rows * c, "wkv7_seq a");
    OPND(pkk, k_k, RSV_F32, c, "wkv7_seq k_k");
    OPND(pka, k_a, RSV_F32, c, "wkv7_seq k_a");
    OPND(prk, r_k, RSV_F32, c, "wkv7_seq r_k");
    OPND(pgw, ln_x_w, RSV_F32, c, "wkv7_seq ln_x_w");
    OPND(pgb, ln_x_b, RSV_F32, c, "wkv7_seq ln_x_b");
    OPND(pyn, y_norm, RSV_F32, rows * c, "wkv7_seq y_norm");
    OPND(pst, seg_start, RSV_U32, nseg, "wkv7_seq seg_start");
    OPND(pln, seg_len, RSV_U32, nseg, "wkv7_seq seg_len");
    OPND(psl, seg_slot, RSV_U32, nseg, "wkv7_seq seg_slot");
    return launch_wkv7_seq_ragged(ctx, F32P(ps), F32P(pr), F32P(pw), F32P(pk), F32P(pv), F32P(pa), F32P(pkk),
                                  F32P(pka), F32P(prk), F32P(pgw), F32P(pgb), F32P(pyn), U32P(pst), U32P(pln),
                                  U32P(psl), (int)nseg, (int)h, (int)n, gn_eps, rows, slots);
}

}  // extern "C"

extern "C" int rsv_wkv7_seq_ragged_gate(rsv_ctx *ctx, uint32_t s, uint32_t r, uint32_t w, uint32_t k, uint32_t v,
                                        uint32_t a, uint32_t k_k, uint32_t k_a, uint32_t r_k, uint32_t ln_x_w,
                                        uint32_t ln_x_b, uint32_t g, uint32_t y_work, uint32_t bonus_work, uint32_t yg,
                                        uint32_t seg_start, uint32_t seg_len, uint32_t seg_slot, uint64_t nseg,
                                        uint64_t t_rows, uint64_t h, uint64_t n, float gn_eps) {
    CHECK_CTX();
    const uint64_t c = h * n;
    Tensor *ts = get_tensor(ctx, s);
    if (!ts || c == 0) return RSV_FAIL("wkv7_seq_ragged_gate: unknown tensor");
    const uint64_t rows = t_rows, slots = ts->len / (h * n * n);
    OPND(ps, s, RSV_F32, slots * h * n * n, "wkv7_seq s");
    OPND(pr, r, RSV_F32, rows * c, "wkv7_seq r");
    OPND(pw, w, RSV_F32, rows * c, "wkv7_seq w");
    OPND(pk, k, RSV_F32, rows * c, "wkv7_seq k");
    OPND(pv, v, RSV_F32, rows * c, "wkv7_seq v");
    OPND(pa, a, RSV_F32, rows * c, "wkv7_seq a");
    OPND(pkk, k_k, RSV_F32, c, "wkv7_seq k_k");
    OPND(pka, k_a, RSV_F32, c, "wkv7_seq k_a");
    OPND(prk, r_k, RSV_F32, c, "wkv7_seq r_k");
    OPND(pgw, ln_x_w, RSV_F32, c, "wkv7_seq ln_x_w");
    OPND(pgb, ln_x_b, RSV_F32, c, "wkv7_seq ln_x_b");
    OPND(pg, g, RSV_F32, rows * c, "wkv7_seq g");
    OPND(pyw, y_work, RSV_F32, rows * c, "wkv7_seq y_work");
    OPND(pbw, bonus_work, RSV_F32, rows * h, "wkv7_seq bonus_work");
    OPND(pyg, yg, RSV_F16, rows * c, "wkv7_seq yg");
    OPND(pst, seg_start, RSV_U32, nseg, "wkv7_seq seg_start");
    OPND(pln, seg_len, RSV_U32, nseg, "wkv7_seq seg_len");
    OPND(psl, seg_slot, RSV_U32, nseg, "wkv7_seq seg_slot");
    return launch_wkv7_seq_ragged_gate(ctx, F32P(ps), F32P(pr), F32P(pw), F32P(pk), F32P(pv), F32P(pa), F32P(pkk),
                                       F32P(pka), F32P(prk), F32P(pgw), F32P(pgb), F32P(pg), F32P(pyw), F32P(pbw),
                                       (_Float16 *)pyg_v, U32P(pst), U32P(pln), U32P(psl), (int)nseg, (int)h, (int)n,
                                       gn_eps, rows, slots);
}

// ------------------------------------------------ prefill building blocks
extern "C" {

int rsv_seq_norm_mix(rsv_ctx *ctx, uint32_t x, uint32_t state, uint32_t gamma, uint32_t beta, const uint32_t *coef,
                     const uint32_t *out_f16, uint64_t nout, uint32_t row_prev, uint64_t t, uint64_t c, float eps) {
    CHECK_CTX();
    if (nout < 1 || nout > 6 || !coef || !out_f16) return RSV_FAIL("seq_norm_mix: bad nout=%llu", (unsigned long long)nout);
    OPND(px, x, RSV_F32, t * c, "seq_norm_mix x");
    Tensor *ts = get_tensor(ctx, state);
    if (!ts || ts->dtype != RSV_F32) return RSV_FAIL("seq_norm_mix: bad state tensor");
    OPND(pg, gamma, RSV_F32, c, "seq_norm_mix gamma");
    OPND(pb, beta, RSV_F32, c, "seq_norm_mix beta");
    OPND(pp, row_prev, RSV_U32, t, "seq_norm_mix row_prev");
    const float *cp[6];
    _Float16 *op[6];
    for (uint64_t j = 0; j < nout; j++) {
        void *p = nullptr;
        if (opnd(ctx, coef[j], RSV_F32, c, &p, "seq_norm_mix coef")) return -1;
        cp[j] = (const float *)p;
        if (opnd(ctx, out_f16[j], RSV_F16, t * c, &p, "seq_norm_mix out")) return -1;
        op[j] = (_Float16 *)p;
    }
    // row_prev values index rows of x (< t) or slots; out-of-range slots read zeros
    return launch_seq_norm_mix(ctx, F32P(px), (const float *)ts->ptr, F32P(pg), F32P(pb), cp, op, (int)nout, U32P(pp),
                               (int)t, (int)c, ts->len / c, eps);
}

int rsv_seq_state_store(rsv_ctx *ctx, uint32_t x, uint32_t state, uint32_t gamma, uint32_t beta, uint32_t seg_last,
                        uint32_t seg_slot, uint64_t nseg, uint64_t c, float eps) {
    CHECK_CTX();
    Tensor *tx = get_tensor(ctx, x), *ts = get_tensor(ctx, state);
    if (!tx || !ts || tx->dtype != RSV_F32 || ts->dtype != RSV_F32) return RSV_FAIL("seq_state_store: bad x/state");
    OPND(pg, gamma, RSV_F32, c, "seq_state_store gamma");
    OPND(pb, beta, RSV_F32, c, "seq_state_store beta");
    OPND(pl, seg_last, RSV_U32, nseg, "seq_state_store seg_last");
    OPND(ps, seg_slot, RSV_U32, nseg, "seq_state_store seg_slot");
    return launch_seq_state_store(ctx, (const float *)tx->ptr, (float *)ts->ptr, F32P(pg), F32P(pb), U32P(pl), U32P(ps),
                                  (int)nseg, (int)c, tx->len / c, ts->len / c, eps);
}

int rsv_copy_rows(rsv_ctx *ctx, uint32_t src, uint32_t dst, uint32_t src_rows, uint32_t dst_rows, uint64_t n,
                  uint64_t c) {
    CHECK_CTX();
    Tensor *ts = get_tensor(ctx, src), *td = get_tensor(ctx, dst);
    if (!ts || !td || ts->dtype != RSV_F32 || td->dtype != RSV_F32) return RSV_FAIL("copy_rows: bad src/dst");
    if (c == 0) return RSV_FAIL("copy_rows: c must be > 0");
    OPND(psr, src_rows, RSV_U32, n, "copy_rows src_rows");
    OPND(pdr, dst_rows, RSV_U32, n, "copy_rows dst_rows");
    return launch_copy_rows(ctx, (const float *)ts->ptr, (float *)td->ptr, U32P(psr), U32P(pdr), (int)n, (int)c,
                            ts->len / c, td->len / c);
}

int rsv_mul_to_f16(rsv_ctx *ctx, uint32_t a, uint32_t b, uint32_t y, uint64_t n) {
    CHECK_CTX();
    OPND(pa, a, RSV_F32, n, "mul_to_f16 a");
    OPND(pb, b, RSV_F32, n, "mul_to_f16 b");
    OPND(py, y, RSV_F16, n, "mul_to_f16 y");
    return launch_mul_to_f16(ctx, F32P(pa), F32P(pb), (_Float16 *)py_v, n);
}

int rsv_gemm_ex(rsv_ctx *ctx, uint32_t a, uint32_t w16, const rsv_int8 *w8, uint32_t c, uint64_t m, uint64_t n,
                uint64_t k, int epilogue, uint32_t bias, uint32_t aux, uint32_t scale) {
    CHECK_CTX();
    if (epilogue < GE_STORE || epilogue > GE_SIGMOID) return RSV_FAIL("gemm_ex: bad epilogue %d", epilogue);
    GemmArgs g{};
    OPND(pa, a, RSV_F16, m * k, "gemm_ex a");
    g.a = (const _Float16 *)pa_v;
    if (w8) {
        const uint32_t *idx, *sz;
        if (int8_operands(ctx, w8, n, k, &idx, &sz, "gemm_ex w8")) return -1;
        g.b = idx;
        g.sz = sz;
        g.b_i8 = 1;
    } else {
        OPND(pw, w16, RSV_F16, n * k, "gemm_ex w16");
        g.b = pw_v;
    }
    Tensor *tc = get_tensor(ctx, c);
    if (!tc || tc->dtype == RSV_U32) return RSV_FAIL("gemm_ex: bad output tensor");
    if (tc->len < m * n) return RSV_FAIL("gemm_ex: output holds %llu < %llu", (unsigned long long)tc->len, (unsigned long long)(m * n));
    g.c = tc->ptr;
    g.c_f16 = tc->dtype == RSV_F16;
    if (epilogue == GE_ADD) g.aux = (const float *)tc->ptr;
    if (bias != 0xFFFFFFFFu) { OPND(pb, bias, RSV_F32, n, "gemm_ex bias"); g.bias = F32P(pb); }
    if (aux != 0xFFFFFFFFu) { OPND(px, aux, RSV_F32, m * n, "gemm_ex aux"); g.aux = F32P(px); }
    if (scale != 0xFFFFFFFFu) { OPND(ps, scale, RSV_F32, 1, "gemm_ex scale"); g.scale = F32P(ps); }
    g.m = (int)m; g.n = (int)n; g.k = (int)k;
    g.lda = (int)k; g.ldc = (int)n;
    g.epi = epilogue;
    return launch_gemm(ctx, g);
}

}  // extern "C"

extern "C" int rsv_gemv_multi(rsv_ctx *ctx, const rsv_gemv_job *jobs, uint64_t njobs, uint32_t side_src,
                              uint32_t side_dst, uint64_t side_n, uint64_t batch) {
    CHECK_CTX();
    if (!jobs || njobs == 0 || njobs > (uint64_t)kMaxJobs) return RSV_FAIL("gemv_multi: 1..%d jobs", kMaxJobs);
    GemvJobs J{};
    J.n = (int)njobs;
    for (uint64_t i = 0; i < njobs; i++) {
        const rsv_gemv_job &q = jobs[i];
        GemvJob &g = J.j[i];
        if (q.w8 ? job_i8(ctx, g, q.w8, q.m, q.k, "gemv_multi") : job_f16(ctx, g, q.w16, q.m, q.k, "gemv_multi"))
            return -1;
        if (job_xy(ctx, g, q.x, q.y, batch, "gemv_multi")) return -1;
        if (q.prologue < PRO_NONE || q.prologue > PRO_GNGATE) return RSV_FAIL("gemv_multi: bad prologue %d", q.prologue);
        if (q.prologue == PRO_GNGATE &&
            (batch != 1 || q.k % 64 != 0 || q.gamma == 0xFFFFFFFFu || q.beta == 0xFFFFFFFFu ||
             q.prev == 0xFFFFFFFFu || q.xmul == 0xFFFFFFFFu))
            return RSV_FAIL("gemv_multi: the GroupNorm-gate prologue needs batch 1, k %% 64 == 0, gamma, beta, prev and xmul");
        g.eps = q.gn_eps;
        if (q.epilogue < EPI_STORE || q.epilogue > EPI_STORE2) return RSV_FAIL("gemv_multi: bad epilogue %d", q.epilogue);
        g.pro = q.prologue;
        g.epi = q.epilogue;
        void *p = nullptr;
        if (q.xmul != 0xFFFFFFFFu) { if (opnd(ctx, q.xmul, RSV_F32, q.k * batch, &p, "gemv_multi xmul")) return -1; g.xmul = (const float *)p; }
        if (q.p0 != 0xFFFFFFFFu) { if (opnd(ctx, q.p0, RSV_F32, q.m, &p, "gemv_multi p0")) return -1; g.p0 = (const float *)p; }
        if (q.p1 != 0xFFFFFFFFu) { if (opnd(ctx, q.p1, RSV_F32, q.m * batch, &p, "gemv_multi p1")) return -1; g.p1 = (const float *)p; }
        if (q.scale != 0xFFFFFFFFu) { if (opnd(ctx, q.scale, RSV_F32, 1, &p, "gemv_multi scale")) return -1; g.scale = (const float *)p; }
        if (q.gamma != 0xFFFFFFFFu) { if (opnd(ctx, q.gamma, RSV_F32, q.k, &p, "gemv_multi gamma")) return -1; g.gamma = (const float *)p; }
        if (q.beta != 0xFFFFFFFFu) { if (opnd(ctx, q.beta, RSV_F32, q.k, &p, "gemv_multi beta")) return -1; g.beta = (const float *)p; }
        if (q.prev != 0xFFFFFFFFu) { if (opnd(ctx, q.prev, RSV_F32, q.k * batch, &p, "gemv_multi prev")) return -1; g.prev = (const float *)p; }
        if (q.coef != 0xFFFFFFFFu) { if (opnd(ctx, q.coef, RSV_F32, q.k, &p, "gemv_multi coef")) return -1; g.coef = (const float *)p; }
        if (q.lnout != 0xFFFFFFFFu) { if (opnd(ctx, q.lnout, RSV_F32, q.k * batch, &p, "gemv_multi lnout")) return -1; g.lnout = (float *)p; }
    }
    if (side_src != 0xFFFFFFFFu || side_dst != 0xFFFFFFFFu) {
        void *a = nullptr, *b = nullptr;
        if (opnd(ctx, side_src, RSV_F32, side_n * batch, &a, "gemv_multi side_src") ||
            opnd(ctx, side_dst, RSV_F32, side_n * batch, &b, "gemv_multi side_dst"))
            return -1;
        J.side.src = (const float *)a;
        J.side.dst = (float *)b;
        J.side.n = (int)side_n;
    }
    return launch_gemv_jobs(ctx, J, (int)batch);
}

// One rsv_mm_job of rsv_gemm_skinny -> its kernel job (operands checked).
static int skinny_job_of(rsv_ctx *ctx, const rsv_mm_job &q, uint64_t batch, SkinnyJob &J) {
    {
        if (q.w8) {
            const uint32_t *idx, *sz;
            if (int8_operands(ctx, q.w8, q.n, q.k, &idx, &sz, "gemm_skinny")) return -1;
            J.w = idx;
            J.sz = sz;
            J.fmt = FMT_I8;
        } else {
            void *p = nullptr;
            if (opnd(ctx, q.w16, RSV_F16, q.n * q.k, &p, "gemm_skinny w16")) return -1;
            J.w = p;
            J.fmt = FMT_F16;
        }
        void *px = nullptr;
        if (opnd(ctx, q.x, RSV_F16, q.k * batch, &px, "gemm_skinny x")) return -1;
        J.x = (const _Float16 *)px;
        J.ldx = (int)q.k;
        Tensor *ty = get_tensor(ctx, q.y);
        if (!ty || ty->dtype == RSV_U32 || ty->len < q.n * batch) return RSV_FAIL("gemm_skinny: bad y tensor %u", q.y);
        J.y = ty->ptr;
        J.y_f16 = ty->dtype == RSV_F16;
        J.ldy = (int)q.n;
        void *p = nullptr;
        if (q.y2 != 0xFFFFFFFFu) { if (opnd(ctx, q.y2, RSV_F32, q.n * batch, &p, "gemm_skinny y2")) return -1; J.y2 = (float *)p; }
        if (q.bias != 0xFFFFFFFFu) { if (opnd(ctx, q.bias, RSV_F32, q.n, &p, "gemm_skinny bias")) return -1; J.bias = (const float *)p; }
        if (q.aux != 0xFFFFFFFFu) { if (opnd(ctx, q.aux, RSV_F32, q.n * batch, &p, "gemm_skinny aux")) return -1; J.aux = (const float *)p; }
        if (q.scale != 0xFFFFFFFFu) { if (opnd(ctx, q.scale, RSV_F32, 1, &p, "gemm_skinny scale")) return -1; J.scale = (const float *)p; }
        if (q.epilogue < GE_STORE || q.epilogue > GE_SIGMOID) return RSV_FAIL("gemm_skinny: bad epilogue %d", q.epilogue);
        J.epi = q.epilogue;
        J.tiled = q.tiled ? 1 : 0;
        if (J.tiled) {  // the tiled copy holds ceil(n/32)*32 rows
            Tensor *tw = get_tensor(ctx, q.w8 ? q.w8->idx : q.w16);
            const uint64_t need = (q.n + 31) / 32 * 32 * q.k * (q.w8 ? 1 : 2);
            if (!tw || tw->len * dtype_size(tw->dtype) < need) return RSV_FAIL("gemm_skinny: tiled weight too small");
            if (q.w8) {
                Tensor *ts = get_tensor(ctx, q.w8->sz);
                if (!ts || ts->len < (q.n + 31) / 32 * 32 * (q.k / 128))
                    return RSV_FAIL("gemm_skinny: tiled scale/zero tensor too small (tile it with esz 4)");
            }
        }
        J.N = (int)q.n;
        J.K = (int)q.k;
    }
    return 0;
}

extern "C" int rsv_gemm_skinny(rsv_ctx *ctx, const rsv_mm_job *jobs, uint64_t njobs, uint64_t batch) {
    CHECK_CTX();
    if (!jobs || njobs == 0 || njobs > (uint64_t)kMaxJobs) return RSV_FAIL("gemm_skinny: 1..%d jobs", kMaxJobs);
    SkinnyJobs S{};
    S.n = (int)njobs;
    for (uint64_t i = 0; i < njobs; i++)
        if (skinny_job_of(ctx, jobs[i], batch, S.j[i])) return -1;
    return launch_skinny(ctx, S, (int)batch);
}

extern "C" int rsv_gemm_skinny_kslices(rsv_ctx *ctx, const rsv_mm_job *job, uint64_t nslice, uint64_t batch) {
    CHECK_CTX();
    if (!job) return RSV_FAIL("gemm_skinny_kslices: null job");
    if (nslice == 0 || nslice > (uint64_t)kMaxJobs) return RSV_FAIL("gemm_skinny_kslices: 1..%d slices", kMaxJobs);
    const rsv_mm_job &q = *job;
    if (!q.tiled) return RSV_FAIL("gemm_skinny_kslices: takes the tiled weight copy");
    if (q.epilogue != GE_STORE || q.y2 != 0xFFFFFFFFu || q.bias != 0xFFFFFFFFu || q.aux != 0xFFFFFFFFu ||
        q.scale != 0xFFFFFFFFu)
        return RSV_FAIL("gemm_skinny_kslices: partial sums take the plain store (no epilogue operands)");
    if (q.k % (nslice * 128) != 0) return RSV_FAIL("gemm_skinny_kslices: k=%llu is not %llu slices of 128-multiples",
                                                   (unsigned long long)q.k, (unsigned long long)nslice);
    Tensor *ty = get_tensor(ctx, q.y);
    if (!ty || ty->dtype != RSV_F32 || ty->len < nslice * batch * q.n)
        return RSV_FAIL("gemm_skinny_kslices: y must be F32 of nslice*batch*n");
    SkinnyJob J0{};
    if (skinny_job_of(ctx, q, batch, J0)) return -1;
    const int ks = (int)(q.k / nslice);
    const size_t tbytes = J0.fmt == FMT_I8 ? 1024 : 2048;
    SkinnyJobs S{};
    S.n = (int)nslice;
    for (int sl = 0; sl < S.n; sl++) {
        SkinnyJob &J = S.j[sl];
        J = J0;
        J.K = ks;
        J.wtile_ch = (int)(q.k / 32);
        J.w = (const uint8_t *)J0.w + (size_t)sl * (ks / 32) * tbytes;
        if (J0.fmt == FMT_I8) J.sz = J0.sz + (size_t)sl * (ks / 128) * 32;
        J.x = J0.x + (size_t)sl * ks;
        J.y = (float *)J0.y + (size_t)sl * batch * q.n;
    }
    return launch_skinny(ctx, S, (int)batch);
}

extern "C" int rsv_gemm_multi(rsv_ctx *ctx, const rsv_mm_job *jobs, uint64_t njobs, uint64_t m) {
    CHECK_CTX();
    if (!jobs || njobs == 0 || njobs > (uint64_t)kMaxJobs) return RSV_FAIL("gemm_multi: 1..%d jobs", kMaxJobs);
    if (m == 0 || m > 0x7FFFFFFF) return RSV_FAIL("gemm_multi: bad m %llu", (unsigned long long)m);
    GemmJobs G{};
    G.n = (int)njobs;
    for (uint64_t i = 0; i < njobs; i++) {
        const rsv_mm_job &q = jobs[i];
        GemmArgs &g = G.j[i];
        if (q.tiled) return RSV_FAIL("gemm_multi job %llu: takes row-major weights (tiled = 0)", (unsigned long long)i);
        if (q.y2 != 0xFFFFFFFFu) return RSV_FAIL("gemm_multi job %llu: y2 is not supported", (unsigned long long)i);
        if (q.epilogue < GE_STORE || q.epilogue > GE_SIGMOID) return RSV_FAIL("gemm_multi: bad epilogue %d", q.epilogue);
        void *p = nullptr;
        if (opnd(ctx, q.x, RSV_F16, m * q.k, &p, "gemm_multi x")) return -1;
        g.a = (const _Float16 *)p;
        if (q.w8) {
            const uint32_t *idx, *sz;
            if (int8_operands(ctx, q.w8, q.n, q.k, &idx, &sz, "gemm_multi w8")) return -1;
            g.b = idx;
            g.sz = sz;
            g.b_i8 = 1;
        } else {
            if (opnd(ctx, q.w16, RSV_F16, q.n * q.k, &p, "gemm_multi w16")) return -1;
            g.b = p;
        }
        Tensor *tc = get_tensor(ctx, q.y);
        if (!tc || tc->dtype == RSV_U32 || tc->len < m * q.n) return RSV_FAIL("gemm_multi: bad y tensor %u", q.y);
        g.c = tc->ptr;
        g.c_f16 = tc->dtype == RSV_F16;
        if (q.epilogue == GE_ADD) g.aux = (const float *)tc->ptr;
        if (q.bias != 0xFFFFFFFFu) { if (opnd(ctx, q.bias, RSV_F32, q.n, &p, "gemm_multi bias")) return -1; g.bias = (const float *)p; }
        if (q.aux != 0xFFFFFFFFu) { if (opnd(ctx, q.aux, RSV_F32, m * q.n, &p, "gemm_multi aux")) return -1; g.aux = (const float *)p; }
        if (q.scale != 0xFFFFFFFFu) { if (opnd(ctx, q.scale, RSV_F32, 1, &p, "gemm_multi scale")) return -1; g.scale = (const float *)p; }
        g.m = (int)m; g.n = (int)q.n; g.k = (int)q.k;
        g.lda = (int)q.k; g.ldc = (int)q.n;
        g.epi = q.epilogue;
    }
    return launch_gemm_multi(ctx, G);
}

extern "C" int rsv_ln_mix_f16(rsv_ctx *ctx, uint32_t x, uint32_t state, uint32_t gamma, uint32_t beta,
                              const uint32_t *coef, const uint32_t *out_f16, uint64_t nout, uint64_t c, float eps,
                              uint64_t batch) {
    CHECK_CTX();
    if ((nout != 1 && nout != 6) || !out_f16) return RSV_FAIL("ln_mix_f16: nout must be 1 or 6");
    OPND(px, x, RSV_F32, c * batch, "ln_mix_f16 x");
    OPND(pg, gamma, RSV_F32, c, "ln_mix_f16 gamma");
    OPND(pb, beta, RSV_F32, c, "ln_mix_f16 beta");
    float *pst = nullptr;
    if (state != 0xFFFFFFFFu) { OPND(ps, state, RSV_F32, c * batch, "ln_mix_f16 state"); pst = F32P(ps); }
    const float *cp[6] = {nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};
    _Float16 *op[6];
    for (uint64_t j = 0; j < nout; j++) {
        void *p = nullptr;
        if (coef && coef[j] != 0xFFFFFFFFu) {
            if (!pst) return RSV_FAIL("ln_mix_f16: a token-shift mix needs the state row");
            if (opnd(ctx, coef[j], RSV_F32, c, &p, "ln_mix_f16 coef")) return -1;
            cp[j] = (const float *)p;
        }
        if (opnd(ctx, out_f16[j], RSV_F16, c * batch, &p, "ln_mix_f16 out")) return -1;
        op[j] = (_Float16 *)p;
    }
    return launch_ln_mix_f16(ctx, F32P(px), pst, F32P(pg), F32P(pb), cp, op, (int)nout, (int)c, eps, (int)batch);
}

extern "C" int rsv_ln_mix_f16_acc(rsv_ctx *ctx, uint32_t x, uint32_t part, uint64_t nslice, uint32_t xout,
                                  uint32_t state, uint32_t gamma, uint32_t beta, const uint32_t *coef,
                                  const uint32_t *out_f16, uint64_t nout, uint64_t c, float eps, uint64_t batch) {
    CHECK_CTX();
    if ((nout != 1 && nout != 6) || !out_f16) return RSV_FAIL("ln_mix_f16_acc: nout must be 1 or 6");
    if (nslice == 0 || nslice > 4) return RSV_FAIL("ln_mix_f16_acc: 1..4 slices");
    OPND(px, x, RSV_F32, c * batch, "ln_mix_f16_acc x");
    OPND(pp, part, RSV_F32, nslice * c * batch, "ln_mix_f16_acc part");
    float *pxo = nullptr;
    if (xout != 0xFFFFFFFFu) {
        if (xout == x) return RSV_FAIL("ln_mix_f16_acc: xout must not be x (other blocks of a row still read it)");
        OPND(po, xout, RSV_F32, c * batch, "ln_mix_f16_acc xout");
        pxo = F32P(po);
    }
    OPND(pg, gamma, RSV_F32, c, "ln_mix_f16_acc gamma");
    OPND(pb, beta, RSV_F32, c, "ln_mix_f16_acc beta");
    float *pst = nullptr;
    if (state != 0xFFFFFFFFu) { OPND(ps, state, RSV_F32, c * batch, "ln_mix_f16_acc state"); pst = F32P(ps); }
    const float *cp[6] = {nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};
    _Float16 *op[6];
    for (uint64_t j = 0; j < nout; j++) {
        void *p = nullptr;
        if (coef && coef[j] != 0xFFFFFFFFu) {
            if (!pst) return RSV_FAIL("ln_mix_f16_acc: a token-shift mix needs the state row");
            if (opnd(ctx, coef[j], RSV_F32, c, &p, "ln_mix_f16_acc coef")) return -1;
            cp[j] = (const float *)p;
        }
        if (opnd(ctx, out_f16[j], RSV_F16, c * batch, &p, "ln_mix_f16_acc out")) return -1;
        op[j] = (_Float16 *)p;
    }
    return launch_ln_mix_f16(ctx, F32P(px), pst, F32P(pg), F32P(pb), cp, op, (int)nout, (int)c, eps, (int)batch,
                             F32P(pp), (int)nslice, pxo);
}

extern "C" int rsv_wkv7_decode_ex(rsv_ctx *ctx, uint32_t s, uint32_t k, uint32_t k_k, uint32_t a, uint32_t k_a,
                                  uint32_t r, uint32_t v, uint32_t w, uint32_t ln_x_w, uint32_t ln_x_b, uint32_t r_k,
                                  uint32_t y_norm, uint32_t g, uint32_t yg_f16, uint64_t h, uint64_t n, float eps,
                                  float gn_eps, uint64_t batch) {
    CHECK_CTX();
    const uint64_t c = h * n;
    OPND(ss, s, RSV_F32, batch * h * n * n, "wkv state");
    OPND(kk, k, RSV_F32, c * batch, "wkv k");
    OPND(kc, k_k, RSV_F32, c, "wkv k_k");
    OPND(aa, a, RSV_F32, c * batch, "wkv a");
    OPND(kac, k_a, RSV_F32, c, "wkv k_a");
    OPND(rr, r, RSV_F32, c * batch, "wkv r");
    OPND(vv, v, RSV_F32, c * batch, "wkv v");
    OPND(ww, w, RSV_F32, c * batch, "wkv w");
    OPND(gw, ln_x_w, RSV_F32, c, "wkv ln_x_w");
    OPND(gb, ln_x_b, RSV_F32, c, "wkv ln_x_b");
    OPND(rkc, r_k, RSV_F32, c, "wkv r_k");
    float *yn = nullptr, *gm = nullptr;
    _Float16 *yg = nullptr;
    if (y_norm != 0xFFFFFFFFu) { OPND(p, y_norm, RSV_F32, c * batch, "wkv y_norm"); yn = F32P(p); }
    if (g != 0xFFFFFFFFu) { OPND(p, g, RSV_F32, c * batch, "wkv g"); gm = F32P(p); }
    if (yg_f16 != 0xFFFFFFFFu) { OPND(p, yg_f16, RSV_F16, c * batch, "wkv yg"); yg = (_Float16 *)p_v; }
    return launch_wkv7_decode(ctx, F32P(ss), F32P(kk), F32P(kc), F32P(aa), F32P(kac), F32P(rr), F32P(vv), F32P(ww),
                              F32P(gw), F32P(gb), F32P(rkc), nullptr, nullptr, yn, (int)h, (int)n, eps, gn_eps,
                              (int)batch, gm, yg);
}

extern "C" int rsv_tile_weights(rsv_ctx *ctx, uint32_t src, uint64_t n, uint64_t k, int esz, uint32_t *out) {
    CHECK_CTX();
    if (!out || (esz != 1 && esz != 2 && esz != 4)) return RSV_FAIL("tile_weights: bad arguments");
    if (k % 32 != 0) return RSV_FAIL("tile_weights: k=%llu must be a multiple of 32", (unsigned long long)k);
    if (esz == 4 && k % 128 != 0) return RSV_FAIL("tile_weights: k=%llu must be a multiple of 128", (unsigned long long)k);
    void *ps = nullptr;
    const uint64_t src_len = esz == 1 ? n * k / 4 : esz == 2 ? n * k : n * (k / 128);
    if (opnd(ctx, src, esz == 2 ? RSV_F16 : RSV_U32, src_len, &ps, "tile_weights src")) return -1;
    const uint64_t rows = (n + 31) / 32 * 32;
    uint32_t id;
    if (esz == 4) {
        if (rsv_tensor_create(ctx, rows * (k / 128), RSV_U32, &id)) return -1;
    } else if (esz == 1) {
        if (rsv_tensor_create(ctx, rows * k / 4, RSV_U32, &id)) return -1;
    } else {
        if (rsv_tensor_create(ctx, rows * k, RSV_F16, &id)) return -1;
    }
    Tensor *t = get_tensor(ctx, id);
    if (launch_tile_weights(ctx, ps, t->ptr, (int)n, (int)k, esz)) return -1;
    *out = id;
    return 0;
}
