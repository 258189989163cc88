"""Benchmark of the rwkv-rsv hot path on one MI355X.

Workload (the metric's configuration): 3B-shape
RWKV-7 (32 layers, d_model 2560, 40 heads x 64, FFN 10240, vocab 65536,
LoRA 96/96/64/256), random-init seed 1, int8 per-row-scale linears + int8
head in the reference's int8 format.  Each session is seeded with a 32-token
uniform random prompt (prefilled untimed), then the argmax decode self-loop
runs:
  - B=1:  `--steps` tokens (one step = one decoded token)      -> `value`
  - B=8 and B=64: `--steps-b64` steps of 8 / 64 concurrent sessions -> extra
and the ragged prefill of configs[4] (64 prompts, lengths U[16, 2048] seed 2,
packed into ragged chunks of <= 4096 tokens as configs[4] says; also timed
with 12,288-row chunks and labelled as such)                       -> extra.

Prints ONE JSON line (rank 0).  Inputs are resident in HBM when each timed
region starts; timings bracket the region with device synchronisation.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [os.path.join(ROOT, "rwkv-rsv_amd"), os.path.join(ROOT, "oracle")]

HBM_PEAK_GBS = 8000.0
# HBM bytes per launch of the dominant kernel, from the two rocprofv3 --pmc
# passes (FETCH_SIZE, WRITE_SIZE) of `bench.py --kernel-only`, scaled by the
# same counters of a plain 64 MiB copy; profiles/ffn_key_gemv_b1.md
FFN_KEY_TRAFFIC = 27671041
NONE = 0xFFFFFFFF


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def model_path(cache_dir, kind="i8"):
    """The configs[3] model file (seed 1), generated once per cache dir:
    "i8" int8 linears + int8 head, "i8_f16" int8 linears + fp16 embedding
    and head (the same files the 3B parity tests use)."""
    import synth
    name, kw = {"i8": ("rsv_3b_i8_seed1.st", dict(linear="i8", head="i8")),
                "i8_f16": ("rsv_3b_i8_f16head_seed1.st", dict(linear="i8", head="f16", emb="f16"))}[kind]
    path = os.path.join(cache_dir, name)
    if not os.path.exists(path):
        t = time.time()
        tmp = path + ".tmp%d" % os.getpid()
        synth.write_model(tmp, synth.THREE_B, seed=1, **kw)
        os.replace(tmp, path)
        log(f"generated {path} in {time.time() - t:.1f}s")
    return path


def decode_bytes_per_step(cfg, batch, head_f16=False):
    """Algorithmic HBM bytes of one decode step (int8 linears + int8 head or
    fp16 head, fp16 LoRA, fp32 state and activations)."""
    C, L, F, V = cfg["c"], cfg["n_layer"], cfg["ffn"], cfg["vocab"]
    H, N = cfg["n_head"], cfg["head_size"]
    lin = L * (4 * C * C + 2 * C * F) * (1 + 1 / 32)
    head = V * C * 2 if head_f16 else V * C * (1 + 1 / 32)
    lora = L * 2 * C * (cfg["wm"] + cfg["am"] + cfg["vm"] + cfg["gm"]) * 2
    vec = L * 14 * C * 4
    per_session = L * (2 * H * N * N * 4 + 4 * C * 4) + V * 4
    return lin + head + lora + vec + batch * per_session


def ffn_key_bytes(C, F):
    """Algorithmic HBM bytes of one ffn.key GEMV launch at B=1: int8 weight
    bytes + packed scale/zero words + the five [C] f32 prologue vectors
    (x, token-shift row, gamma, beta, mix coefficient) + the [F] f32 output."""
    return F * C + F * (C // 128) * 4 + 5 * C * 4 + F * 4


def kernel_leg(reps=200):
    """Times the dominant decode kernel on its own: the fused ffn.key launch
    (LN2 + token-shift mix prologue, int8 10240x2560 fused-dequant GEMV,
    relu^2 epilogue) exactly as one decode layer issues it, `reps` launches
    bracketed by HIP events recorded on the backend's own stream."""
    import ctypes
    import torch
    import rsv
    C, F = 2560, 10240
    rng = np.random.default_rng(3)
    be = rsv.Backend(0)
    idx = rng.integers(0, 256, size=(F, C), dtype=np.uint8)
    s = (np.abs(rng.standard_normal(F)) * 0.02 / 127 + 1e-5).astype(np.float16)
    z = (-128.0 * s.astype(np.float32)).astype(np.float16)
    sz = (s.view(np.uint16).astype(np.uint32) | (z.view(np.uint16).astype(np.uint32) << 16))
    sz = np.repeat(sz[:, None], C // 128, axis=1)
    # 12 weight copies (324 MB, more than the 256 MB MALL) rotated launch by
    # launch, so each launch streams its weights from HBM as in a decode step
    ncopy = 12
    hs = [be.int8(idx, sz) for _ in range(ncopy)]
    ids = dict(x=be.tensor(rng.standard_normal(C).astype(np.float32)),
               prev=be.tensor(rng.standard_normal(C).astype(np.float32)),
               g=be.tensor(np.ones(C, np.float32)), b=be.tensor(np.zeros(C, np.float32)),
               c=be.tensor(rng.random(C).astype(np.float32)), y=be.tensor(n=F))
    js = []
    for h in hs:
        j = rsv.GemvJob()
        ctypes.memset(ctypes.byref(j), 0xFF, ctypes.sizeof(j))
        j.w8 = ctypes.pointer(h)
        j.m, j.k, j.x, j.y = F, C, ids["x"], ids["y"]
        j.prologue, j.epilogue = 3, 1
        j.gamma, j.beta, j.prev, j.coef = ids["g"], ids["b"], ids["prev"], ids["c"]
        js.append(j)
    sp = ctypes.c_void_p()
    rsv.hip_lib().rsv_stream(be.ctx, ctypes.byref(sp))
    stream = torch.cuda.ExternalStream(sp.value, device=torch.device("cuda", 0))
    for i in range(2 * ncopy):
        be.call("rsv_gemv_multi", ctypes.byref(js[i % ncopy]), 1, NONE, NONE, 0, 1)
    be.sync()
    # the launches are captured into one HIP graph so that host enqueue time
    # does not leak into the measurement; the graph is replayed once untimed
    be.call("rsv_graph_begin")
    for i in range(reps):
        be.call("rsv_gemv_multi", ctypes.byref(js[i % ncopy]), 1, NONE, NONE, 0, 1)
    be.call("rsv_graph_end")
    be.call("rsv_graph_replay")
    be.sync()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    be.call("rsv_graph_replay")
    e1.record(stream)
    e1.synchronize()
    us = e0.elapsed_time(e1) * 1000.0 / reps
    be.close()
    # a plain device copy of known size: the reference point that scales the
    # rocprofv3 FETCH_SIZE / WRITE_SIZE counters of this run to bytes
    src = torch.empty(16 << 20, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(4):
        dst.copy_(src)
    torch.cuda.synchronize()
    nbytes = ffn_key_bytes(C, F)
    return dict(kernel="k_gemv_os2<5,1,640,2> (B=1 ffn.key: LN2 + token-shift mix prologue, int8 10240x2560, relu^2)",
                avg_us=us, bytes=nbytes, gbs=nbytes / us / 1e3, launches=reps,
                timing="HIP events around one replay of a graph of the launches, on the backend stream")



MFMA_F16_PEAK_TFLOPS = 2500.0   # dense fp16 matrix-core peak of one MI355X
FP32_PEAK_TFLOPS = 157.3        # fp32 peak of one MI355X (the figure WKV7 T=512 is held to)


class _Timer:
    """Times `reps` enqueues of fn(i) captured as one HIP graph, replayed
    once untimed, then once between HIP events on the backend's stream."""

    def __init__(self, be):
        import ctypes
        import torch
        import rsv
        sp = ctypes.c_void_p()
        rsv.hip_lib().rsv_stream(be.ctx, ctypes.byref(sp))
        self.stream = torch.cuda.ExternalStream(sp.value, device=torch.device("cuda", 0))
        self.be = be
        self.torch = torch
        # --legs-eager: plain enqueues instead of a graph (for per-kernel
        # traces, where the tracer times every dispatch itself)
        self.eager = os.environ.get("RSV_BENCH_EAGER") == "1"

    def us(self, fn, reps):
        be, torch = self.be, self.torch
        for i in range(min(reps, 4)):
            fn(i)
        be.sync()
        if self.eager:
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(self.stream)
            for i in range(reps):
                fn(i)
            e1.record(self.stream)
            e1.synchronize()
            return e0.elapsed_time(e1) * 1000.0 / reps
        be.call("rsv_graph_begin")
        for i in range(reps):
            fn(i)
        be.call("rsv_graph_end")
        be.call("rsv_graph_replay")
        be.sync()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(self.stream)
        be.call("rsv_graph_replay")
        e1.record(self.stream)
        e1.synchronize()
        return e0.elapsed_time(e1) * 1000.0 / reps


def linear_leg():
    """the four 3B weight shapes (out x in) in both weight forms
    (int8 symmetric per-row scale in the reference format from N(0, 0.02^2)
    masters; fp16 N(0, 0.02^2)) times activations of M rows, fp16 N(0, 1)
    (the row-major GEMVs take them as f32 of the same values).  Each call
    is timed over enough weight copies to exceed the 256 MB MALL.  M = 1 is
    the B=1 GEMV; M = 8 .. 128 the batched-decode MFMA form on the tiled
    weight copy (what the model runs for 2 <= B < prefill chunks), with the
    trait-op GEMV on the row-major weights beside it at M = 8; M = 2048 the
    prefill GEMM.  M <= 8 is held to HBM bandwidth; M >= 32 also reports
    MFMA utilisation against dense fp16."""
    import ctypes
    import rsv
    import synth
    NONE = 0xFFFFFFFF
    be = rsv.Backend(0)
    tm = _Timer(be)
    rng = np.random.default_rng(11)
    rows = []
    for (n, k, name) in ((2560, 2560, "2560->2560 (att.*)"), (10240, 2560, "2560->10240 (ffn.key)"),
                         (2560, 10240, "10240->2560 (ffn.value)"), (65536, 2560, "2560->65536 (head)")):
        master = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02))
        idx, sz = synth.quantize_rows(master)
        w16_host = master.astype(np.float16).astype(np.float32)
        del master
        for fmt in ("int8", "fp16"):
            wbytes = n * k * (1 + 4 / 128) if fmt == "int8" else 2 * n * k
            ncopy = max(1, int(np.ceil(300e6 / wbytes)))
            base = be.int8(idx, sz) if fmt == "int8" else be.tensor(w16_host, dtype=rsv.F16)
            copies = [base]
            for _ in range(ncopy - 1):
                if fmt == "int8":
                    h = rsv.Int8Handle(be.tensor(n=n * k // 4, dtype=rsv.U32), be.tensor(n=n * k // 128, dtype=rsv.U32), n, k)
                    be.call("rsv_copy_device", base.idx, h.idx)
                    be.call("rsv_copy_device", base.sz, h.sz)
                    copies.append(h)
                else:
                    t = be.tensor(n=n * k, dtype=rsv.F16)
                    be.call("rsv_copy_device", base, t)
                    copies.append(t)
            tiled = None
            for M in (1, 8, 32, 128, 2048):
                xh = rng.standard_normal((M, k)).astype(np.float16).astype(np.float32)
                y = be.tensor(n=M * n)
                rowmajor_us = None
                if M <= 8:
                    # the trait-op GEMV on the row-major weights (B=1: k_gemv_os2, 2..16: k_gemv_mb)
                    x = be.tensor(xh)
                    if fmt == "int8":
                        fn = lambda i, x=x, y=y, M=M: be.call("rsv_gemv_int8_plain", ctypes.byref(copies[i % ncopy]), x, y, n, k, M)
                    else:
                        fn = lambda i, x=x, y=y, M=M: be.call("rsv_gemv_f16", copies[i % ncopy], x, y, n, k, M)
                    kern = "k_gemv_os2" if M == 1 else "k_gemv_mb"
                    if M > 1:
                        rowmajor_us = tm.us(fn, max(8, min(200, int(3e-3 / (wbytes / 5e12)))))
                if 1 < M <= 128:
                    # the model's batched-decode form: MFMA on the tiled weight copy
                    if tiled is None:
                        tiled = []
                        out = ctypes.c_uint32()
                        for c in copies:
                            if fmt == "int8":
                                ht = rsv.Int8Handle(c.idx, c.sz, n, k)
                                be.call("rsv_tile_weights", c.idx, n, k, 1, ctypes.byref(out))
                                ht.idx = out.value
                                be.call("rsv_tile_weights", c.sz, n, k, 4, ctypes.byref(out))
                                ht.sz = out.value
                                tiled.append(ht)
                            else:
                                be.call("rsv_tile_weights", c, n, k, 2, ctypes.byref(out))
                                tiled.append(out.value)
                    x = be.tensor(xh, dtype=rsv.F16)
                    jobs = [rsv.MmJob(NONE if fmt == "int8" else t, ctypes.pointer(t) if fmt == "int8" else None,
                                      n, k, x, y, NONE, 0, NONE, NONE, NONE, 1) for t in tiled]
                    fn = lambda i, jobs=jobs, M=M: be.call("rsv_gemm_skinny", ctypes.byref(jobs[i % ncopy]), 1, M)
                    kern = "k_skinny8" if k <= 2560 else "k_skinny5"
                elif M > 128:
                    x = be.tensor(xh, dtype=rsv.F16)
                    if fmt == "int8":
                        fn = lambda i, x=x, y=y: be.call("rsv_gemm_ex", x, NONE, ctypes.byref(copies[i % ncopy]), y, 2048, n, k, 0, NONE, NONE, NONE)
                    else:
                        fn = lambda i, x=x, y=y: be.call("rsv_gemm_ex", x, copies[i % ncopy], None, y, 2048, n, k, 0, NONE, NONE, NONE)
                    kern = "k_gemm3" if fmt == "int8" else "k_gemmd"
                reps = max(8, min(200, int(3e-3 / max(wbytes / 5e12, 2 * M * n * k / 1.2e15))))
                us = tm.us(fn, reps)
                byts = wbytes + 2 * M * k + 4 * M * n
                row = dict(shape=name, weights=fmt, M=M, kernel=kern, us=round(us, 3), bytes=int(byts),
                           gbs=round(byts / us / 1e3, 1), hbm_frac=round(byts / us / 1e3 / HBM_PEAK_GBS, 4))
                if rowmajor_us is not None:
                    row.update(rowmajor_kernel="k_gemv_mb", rowmajor_us=round(rowmajor_us, 3),
                               rowmajor_hbm_frac=round(byts / rowmajor_us / 1e3 / HBM_PEAK_GBS, 4))
                if M >= 32:
                    tf = 2.0 * M * n * k / us / 1e6
                    row.update(tflops=round(tf, 1), mfma_frac=round(tf / MFMA_F16_PEAK_TFLOPS, 4))
                rows.append(row)
                log(f"linear {name:24s} {fmt:4s} M={M:5d} {kern:10s} {us:9.2f} us {row['gbs']:8.0f} GB/s"
                    + (f" {row['tflops']:7.1f} TFLOP/s" if M >= 32 else "")
                    + (f"  (row-major k_gemv_mb {rowmajor_us:.2f} us)" if rowmajor_us is not None else ""))
            del copies, tiled
        del idx, sz, w16_host
    be.close()
    return rows


def wkv_leg():
    """the fused WKV7 state update (L2-normalised k, DPLR update,
    y = S r, GroupNorm + bonus) at H=40, N=64, fp32 state, B sessions x T
    tokens.  T=1 is the decode op (fuse_ka_dplr_norm_batch); T=512 the
    ragged prefill scan over B segments of 512 tokens.  Inputs as configs[2]
    (r, v ~ N(0,1); k ~ N(0,1) normalised in the op; w = exp(-0.6065
    sigmoid(x)); a = sigmoid(N(0,1)); S0 ~ N(0, 0.1^2)), fp32 in HBM.
    Algorithmic bytes per (session, head): the state read and written once
    (2 x 16384 B) + T x (5 inputs + 1 output) x 64 x 4 B; flops 36,864 per
    (session, head, token)."""
    import rsv
    NONE = 0xFFFFFFFF
    be = rsv.Backend(0)
    tm = _Timer(be)
    rng = np.random.default_rng(12)
    H, N = 40, 64
    C = H * N
    sig = lambda t: 1.0 / (1.0 + np.exp(-t))
    consts = dict(kk=be.tensor(np.ones(C, np.float32)), ka=be.tensor(rng.random(C).astype(np.float32)),
                  rk=be.tensor(rng.standard_normal(C).astype(np.float32) * 0.1),
                  g=be.tensor(np.ones(C, np.float32)), b=be.tensor(np.zeros(C, np.float32)))
    rows = []
    for B in (1, 32, 256):
        S = be.tensor((rng.standard_normal(B * H * N * N) * 0.1).astype(np.float32))
        for T in (1, 512):
            rowsn = B * T
            vec = lambda: be.tensor(rng.standard_normal(rowsn * C).astype(np.float32))
            r, k, v = vec(), vec(), vec()
            w = be.tensor(np.exp(-0.6065 * sig(rng.standard_normal(rowsn * C))).astype(np.float32))
            a = be.tensor(sig(rng.standard_normal(rowsn * C)).astype(np.float32))
            yn = be.tensor(n=rowsn * C)
            if T == 1:
                fn = lambda i: be.call("rsv_fuse_ka_dplr_norm_batch", S, k, consts["kk"], a, consts["ka"], r, v, w,
                                       consts["g"], consts["b"], consts["rk"], NONE, NONE, yn, H, N, 1e-12, 64e-5, B)
                kern = "k_wkv7_decode"
            else:
                st = be.tensor(np.arange(B, dtype=np.uint32) * T, dtype=rsv.U32)
                ln = be.tensor(np.full(B, T, np.uint32), dtype=rsv.U32)
                sl = be.tensor(np.arange(B, dtype=np.uint32), dtype=rsv.U32)
                # the prefill's form of the scan (rsv_wkv7_seq_ragged_gate: the
                # row-split scan, then GroupNorm + bonus + gate into fp16), with
                # `a` standing in for the gate
                bw = be.tensor(n=rowsn * H)
                yg = be.tensor(n=rowsn * C, dtype=rsv.F16)
                fn = lambda i: be.call("rsv_wkv7_seq_ragged_gate", S, r, w, k, v, a, consts["kk"], consts["ka"],
                                       consts["rk"], consts["g"], consts["b"], a, yn, bw, yg, st, ln, sl, B, B * T, H,
                                       N, 64e-5)
                # the scan form follows the block count (H x B): 16 lanes per
                # state row below a quarter of the CUs, two rows per group of
                # four lanes from one block per CU up, four rows from 16 per CU
                kern = ("k_wkv7_seq_cols<16>" if H * B * 4 <= 256 else "k_wkv7_seq_cols<8>" if H * B <= 256
                        else "k_wkv7_seq_rows<4>" if H * B >= 16 * 256 else "k_wkv7_seq_rows<2>") + "+k_gn_gate_f16"
            reps = 50 if T == 1 else max(2, min(20, 256 // B))
            us = tm.us(fn, reps)
            byts = B * H * (2 * 16384 + T * 6 * 64 * 4)
            fl = 36864.0 * B * H * T
            gbs, tf = byts / us / 1e3, fl / us / 1e6
            row = dict(B=B, T=T, kernel=kern, us=round(us, 2), bytes=int(byts), gbs=round(gbs, 1),
                       hbm_frac=round(gbs / HBM_PEAK_GBS, 4), tflops=round(tf, 2),
                       fp32_frac=round(tf / FP32_PEAK_TFLOPS, 4),
                       bound="hbm" if T == 1 else "max(hbm, fp32)")
            rows.append(row)
            log(f"wkv7 B={B:3d} T={T:3d} {kern:18s} {us:10.2f} us {gbs:8.0f} GB/s {tf:7.2f} TFLOP/s")
    be.close()
    return rows

def gemm_compare_leg(reps=20):
    """The prefill GEMMs of a 4096-row chunk (fp16 weight copies, fp32
    out) on `k_gemmd` (rsv_gemm_ex) and on hipBLASLt through torch.matmul
    (fp16 out), same shapes, HIP events around `reps` launches each on the
    stream each is enqueued on.  Operands: N(0,1) activations, N(0, 0.02^2)
    weights; the weights rotate over copies so that they are not L2-resident."""
    import torch
    import rsv
    be = rsv.Backend(0)
    tm = _Timer(be)
    rng = np.random.default_rng(1)
    rows = []
    for (M, N, K, nm) in ((4096, 10240, 2560, "ffn.key"), (4096, 2560, 10240, "ffn.value"),
                          (4096, 2560, 2560, "att.output"), (4096, 7680, 2560, "r/k/v")):
        ncopy = max(1, int(np.ceil(300e6 / (2 * N * K))))
        w = [be.tensor((rng.standard_normal(N * K) * 0.02).astype(np.float32), dtype=rsv.F16) for _ in range(ncopy)]
        x = be.tensor(rng.standard_normal(M * K).astype(np.float32), dtype=rsv.F16)
        y = be.tensor(n=M * N)
        us = tm.us(lambda i: be.call("rsv_gemm_ex", x, w[i % ncopy], None, y, M, N, K, 0, NONE, NONE, NONE), reps)
        a = torch.randn(M, K, device="cuda", dtype=torch.float16)
        bt = [torch.randn(N, K, device="cuda", dtype=torch.float16) * 0.02 for _ in range(ncopy)]
        for i in range(4):
            c = a @ bt[i % ncopy].t()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(reps):
            c = a @ bt[i % ncopy].t()
        e1.record()
        e1.synchronize()
        ub = e0.elapsed_time(e1) * 1000.0 / reps
        fl = 2.0 * M * N * K
        rows.append(dict(gemm=nm, m=M, n=N, k=K, k_gemmd_us=round(us, 1), hipblaslt_us=round(ub, 1),
                         k_gemmd_tflops=round(fl / us / 1e6, 1), hipblaslt_tflops=round(fl / ub / 1e6, 1)))
        log(f"gemm {nm:10s} {M}x{N}x{K}: k_gemmd {us:7.1f} us ({fl / us / 1e6:6.1f} TFLOP/s), "
            f"hipBLASLt {ub:7.1f} us ({fl / ub / 1e6:6.1f} TFLOP/s)")
        del w, x, y, bt, a, c
    be.close()
    return rows


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=32)
    ap.add_argument("--steps-b64", type=int, default=200)
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-serve", action="store_true")
    ap.add_argument("--serve-decode", type=int, default=256,
                    help="tokens sampled per session in the configs[4] ragged-serving leg")
    ap.add_argument("--cpu-tokens", type=int, default=24,
                    help="decode tokens of the CPU-baseline sample (about 14 s of one core; at most 28)")
    ap.add_argument("--no-legs", action="store_true",
                    help="skip the configs[1] linear and configs[2] WKV7 microbenchmarks and the fp16 variant")
    ap.add_argument("--cache", default=os.environ.get("RSV_BENCH_CACHE", "/tmp"))
    ap.add_argument("--legs-only", action="store_true",
                    help="run only the configs[1] linear and configs[2] WKV7 microbenchmarks")
    ap.add_argument("--legs-eager", action="store_true",
                    help="time the microbenchmarks with plain enqueues instead of graph replays (for traces)")
    ap.add_argument("--kernel-only", action="store_true",
                    help="run only the dominant-kernel leg (for rocprofv3 summaries of that kernel)")
    ap.add_argument("--no-graph", action="store_true",
                    help="enqueue self-loop steps eagerly instead of replaying a HIP graph (profiling)")
    ap.add_argument("--gemm-compare", action="store_true",
                    help="run only the prefill GEMM shapes on k_gemmd and on hipBLASLt (torch.matmul)")
    args = ap.parse_args()
    if args.no_graph:
        os.environ["RSV_NO_GRAPH"] = "1"
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}).",
              file=sys.stderr)
        sys.exit(2)

    if args.legs_eager:
        os.environ["RSV_BENCH_EAGER"] = "1"
    if args.legs_only:
        lin, wk = linear_leg(), wkv_leg()
        print(json.dumps({"linear_configs1": lin, "wkv7_configs2": wk}))
        return

    if args.gemm_compare:
        print(json.dumps({"gemm_compare": gemm_compare_leg()}))
        return

    if args.kernel_only:
        kl = kernel_leg()
        log(f"kernel: {kl['kernel']}: {kl['avg_us']:.2f} us/launch over {kl['launches']} launches, {kl['gbs']:.0f} GB/s")
        print(json.dumps({"kernel_leg": kl}))
        return

    import rsv
    import synth
    cfg = synth.THREE_B
    path = model_path(args.cache)
    t = time.time()
    bundle = rsv.ModelBuilder(path).build()
    log(f"model loaded in {time.time() - t:.1f}s")
    prompt = synth.prompt(cfg, 32, seed=1)

    # ---------------- B = 1 argmax self-loop
    bundle.infer_seq(prompt[:-1])
    if args.warmup:
        bundle.infer_argmax_selfloop(int(prompt[-1]), args.warmup)
    bundle.reset()
    bundle.infer_seq(prompt[:-1])
    S1 = bundle.create_batch_state(1)
    snap1 = bundle.state_back()
    S1.load(snap1)
    toks, ms = bundle.argmax_selfloop_batch_timed(S1, [int(prompt[-1])], args.steps)
    t0 = time.perf_counter()
    bundle.reset()
    bundle.infer_seq(prompt[:-1])
    t1 = time.perf_counter()
    wall = bundle.infer_argmax_selfloop(int(prompt[-1]), args.steps)
    t2 = time.perf_counter()
    assert np.array_equal(wall, toks[0]), "self-loop is not deterministic"
    b1_tps = args.steps / (ms / 1000.0)
    b1_wall_tps = args.steps / (t2 - t1)
    bytes1 = decode_bytes_per_step(cfg, 1)
    log(f"B=1: {b1_tps:.1f} tok/s (device), {b1_wall_tps:.1f} tok/s (wall incl. capture), "
        f"{ms / args.steps * 1000:.1f} us/token, {bytes1 / (ms / args.steps / 1000) / 1e9:.0f} GB/s")
    # ---------------- B = 1 sampling self-loop (configs[4]'s sampler)
    sp1 = rsv.SamplerParams(temperature=1.0, top_k=0, top_p=0.9)
    S1.load(snap1)
    bundle.sample_selfloop_batch(S1, [int(prompt[-1])], 8, sp1)  # warm-up (captures the graph)
    S1.load(snap1)
    _, ms_s = bundle.sample_selfloop_batch_timed(S1, [int(prompt[-1])], args.steps, sp1)
    b1_sample_tps = args.steps / (ms_s / 1000.0)
    log(f"B=1 sample self-loop (T=1, top_p=0.9): {b1_sample_tps:.1f} tok/s")
    S1.free()

    # ---------------- B = 8 argmax self-loop (small-batch decode, HBM-bound)
    B8 = 8
    S8 = bundle.create_batch_state(B8)
    prompts8 = [synth.prompt(cfg, 32, seed=200 + i) for i in range(B8)]
    bundle.forward_seq_batch(S8, [p[:-1] for p in prompts8])
    seeds8 = np.array([int(p[-1]) for p in prompts8], np.uint32)
    snap8 = S8.back()
    bundle.argmax_selfloop_batch(S8, seeds8, 4)
    S8.load(snap8)
    _, ms8 = bundle.argmax_selfloop_batch_timed(S8, seeds8, args.steps_b64)
    b8_tps = B8 * args.steps_b64 / (ms8 / 1000.0)
    bytes8 = decode_bytes_per_step(cfg, B8)
    log(f"B=8: {b8_tps:.0f} tok/s, {ms8 / args.steps_b64:.3f} ms/step, "
        f"{bytes8 / (ms8 / args.steps_b64 / 1000) / 1e9:.0f} GB/s, {b8_tps / b1_tps:.2f}x B=1")
    S8.free()

    # ---------------- B = 64 argmax self-loop
    B = 64
    S = bundle.create_batch_state(B)
    prompts = [synth.prompt(cfg, 32, seed=100 + i) for i in range(B)]
    bundle.forward_seq_batch(S, [p[:-1] for p in prompts])
    seeds64 = np.array([int(p[-1]) for p in prompts], np.uint32)
    snap = S.back()
    bundle.argmax_selfloop_batch(S, seeds64, 4)
    S.load(snap)
    _, ms64 = bundle.argmax_selfloop_batch_timed(S, seeds64, args.steps_b64)
    b64_tps = B * args.steps_b64 / (ms64 / 1000.0)
    bytes64 = decode_bytes_per_step(cfg, B)
    log(f"B=64: {b64_tps:.0f} tok/s, {ms64 / args.steps_b64:.2f} ms/step, "
        f"{bytes64 / (ms64 / args.steps_b64 / 1000) / 1e9:.0f} GB/s")
    S.free()

    # ---------------- ragged prefill
    prefill = None
    if not args.no_prefill:
        rng = np.random.Generator(np.random.PCG64(2))
        lens = rng.integers(16, 2049, size=64)
        pr = [synth.prompt(cfg, int(n), seed=1000 + i) for i, n in enumerate(lens)]
        SP = bundle.create_batch_state(64)

        def timed_prefill(chunk):
            bundle.set_prefill_chunk(chunk)
            # warm-up: the same pass once, so that the timed pass finds its work
            # buffers (sized by the largest chunk) allocated, as a serving process does
            bundle.forward_seq_batch(SP, pr)
            SP.reset()
            rsv.hip_lib().rsv_synchronize(bundle.ctx())
            t0 = time.perf_counter()
            bundle.forward_seq_batch(SP, pr)
            rsv.hip_lib().rsv_synchronize(bundle.ctx())
            dt = time.perf_counter() - t0
            SP.reset()
            return dt

        # configs[4] packs ragged batches of <= 4096 tokens: the headline; the
        # 12,288-row chunks (fuller GEMM tile rounds) are reported beside it
        dt = timed_prefill(4096)
        dt12 = timed_prefill(12288)
        bundle.set_prefill_chunk(4096)
        prefill = dict(tokens=int(lens.sum()), chunk_rows=4096, seconds=dt, tok_s=float(lens.sum() / dt),
                       tok_s_12288_row_chunks=float(lens.sum() / dt12),
                       note="tok_s packs <= 4096-token ragged batches as configs[4]; the 12,288-row figure "
                            "is a larger packing than configs[4] names")
        log(f"prefill (configs[4], <= 4096-token chunks): {lens.sum()} tokens in {dt:.3f}s -> {prefill['tok_s']:.0f} tok/s; "
            f"12,288-row chunks: {prefill['tok_s_12288_row_chunks']:.0f} tok/s")
        SP.free()

    # ---------------- ragged continuous batching
    serve = None
    if not args.no_serve:
        rng = np.random.Generator(np.random.PCG64(2))
        lens = rng.integers(16, 2049, size=64)
        pr = [synth.prompt(cfg, int(n), seed=1000 + i) for i, n in enumerate(lens)]
        SV = bundle.create_batch_state(64)
        sp = rsv.SamplerParams(temperature=1.0, top_k=0, top_p=0.9)
        seeds = np.arange(64, dtype=np.uint32) * 7919 + 2
        # warm-up: 64 x 64 prompt tokens fill a whole 4096-row step, so the
        # timed run finds its work buffers allocated
        bundle.serve_ragged(SV, [p[:64] for p in pr], 2, sp, seeds, budget=4096)
        SV.reset()
        t0 = time.perf_counter()
        toks, steps = bundle.serve_ragged(SV, pr, args.serve_decode, sp, seeds, budget=4096)
        wall = time.perf_counter() - t0
        sms = np.array([st["ms"] for st in steps])
        pre = np.array([st["prefill_tokens"] for st in steps])
        dec = np.array([st["decode_tokens"] for st in steps])
        only_dec = pre == 0
        serve = dict(sessions=64, prompt_tokens=int(lens.sum()), decode_per_session=args.serve_decode,
                     steps=len(steps), wall_s=round(wall, 3),
                     prefill_tok_s=round(float(pre.sum() / (sms[pre > 0].sum() / 1e3)), 1),
                     decode_tok_s=round(float(dec[only_dec].sum() / (sms[only_dec].sum() / 1e3)), 1)
                     if only_dec.any() else None,
                     total_tok_s=round(float((pre.sum() + dec.sum() + 64) / wall), 1),
                     p50_step_ms=round(float(np.percentile(sms, 50)), 3),
                     p99_step_ms=round(float(np.percentile(sms, 99)), 3),
                     sampler="GPU top-p 0.9, T=1.0, seed of token k of session q = seeds[q] + k")
        log(f"serve: {serve}")
        SV.free()

    # ---------------- dominant kernel (roofline)
    kl = kernel_leg()
    log(f"kernel: {kl['kernel']}: {kl['avg_us']:.2f} us/launch, {kl['gbs']:.0f} GB/s")

    # ---------------- configs[3] fp16 embedding/head variant, configs[1], configs[2]
    variant = linear = wkv = None
    if not args.no_legs:
        path16 = model_path(args.cache, kind="i8_f16")
        b16 = rsv.ModelBuilder(path16).build()
        b16.infer_seq(prompt[:-1])
        Sv = b16.create_batch_state(1)
        Sv.load(b16.state_back())
        snapv = Sv.back()
        b16.argmax_selfloop_batch(Sv, [int(prompt[-1])], 8)
        Sv.load(snapv)
        _, msv = b16.argmax_selfloop_batch_timed(Sv, [int(prompt[-1])], args.steps)
        Sv.free()
        Sv = b16.create_batch_state(B)
        b16.forward_seq_batch(Sv, [p[:-1] for p in prompts])
        snapv = Sv.back()
        b16.argmax_selfloop_batch(Sv, seeds64, 4)
        Sv.load(snapv)
        _, msv64 = b16.argmax_selfloop_batch_timed(Sv, seeds64, args.steps_b64)
        Sv.free()
        b16.close()
        bytes1v = decode_bytes_per_step(cfg, 1, head_f16=True)
        variant = dict(model="int8 linears, fp16 embedding and fp16 head (seed 1)",
                       b1_tok_s=round(args.steps / (msv / 1000.0), 1),
                       b1_hbm_frac=round(bytes1v / (msv / args.steps / 1000) / 1e9 / HBM_PEAK_GBS, 4),
                       b64_tok_s=round(B * args.steps_b64 / (msv64 / 1000.0), 1))
        log(f"fp16 variant: {variant}")
        linear = linear_leg()
        wkv = wkv_leg()

    # ---------------- CPU baseline (reference CPU fp32 path, restated)
    cpu = None
    if not args.no_cpu:
        import oracle
        t = time.time()
        m = oracle.Model(path)
        log(f"oracle model built in {time.time() - t:.1f}s")
        st = m.init_state()
        m.forward(prompt[:4], st)
        tt = time.perf_counter()
        if args.cpu_tokens > len(prompt) - 4:
            sys.exit(f"--cpu-tokens {args.cpu_tokens}: the sample prompt has {len(prompt) - 4} tokens after its prefix")
        for i in range(args.cpu_tokens):
            m.forward([int(prompt[4 + i])], st)
        cdt = time.perf_counter() - tt
        cpu = {"value": args.cpu_tokens / cdt, "unit": "tok/s", "cores": 1, "kind": "port",
               "sample": f"oracle (C restatement of model.rs::forward, -O2, 1 thread) on the same 3B int8 model "
                         f"(dequantised to fp32), {args.cpu_tokens} decode tokens after a 4-token prefix; "
                         f"host has {os.cpu_count()} logical cores"}
        log(f"cpu: {cpu['value']:.3f} tok/s")
        del m

    out = {
        "metric": "3B-int8 decode tok/s at B=1 (argmax self-loop)",
        "value": round(b1_tps, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 weights (per-row scale), fp32 accumulate/state",
        "data": "synthetic: random-init seed 1, uniform random prompt ids",
        "config": {"workload": "BASELINE configs[3]: 3B-shape RWKV-7 int8 argmax decode self-loop, B=1 "
                               "(B=64 and configs[4] ragged prefill in extra)",
                   "n_layer": 32, "d_model": 2560, "heads": 40, "ffn": 10240, "vocab": 65536,
                   "batch": 1, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(kl["gbs"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(kl["gbs"] / HBM_PEAK_GBS, 4), "traffic": FFN_KEY_TRAFFIC,
                     "kernel": kl["kernel"], "avg_us": round(kl["avg_us"], 3), "bytes_per_launch": kl["bytes"],
                     "step_achieved_gbs": round(bytes1 / (ms / args.steps / 1000) / 1e9, 1),
                     "step_frac": round(bytes1 / (ms / args.steps / 1000) / 1e9 / HBM_PEAK_GBS, 4)},
        "cpu_baseline": cpu,
        "extra": {"b1_wall_tok_s": round(b1_wall_tps, 2),
                  "b8_tok_s": round(b8_tps, 1), "b8_ms_per_step": round(ms8 / args.steps_b64, 4),
                  "b8_hbm_frac": round(bytes8 / (ms8 / args.steps_b64 / 1000) / 1e9 / HBM_PEAK_GBS, 4),
                  "b8_over_b1": round(b8_tps / b1_tps, 3),
                  "b64_tok_s": round(b64_tps, 1), "b64_ms_per_step": round(ms64 / args.steps_b64, 4),
                  "b64_hbm_frac": round(bytes64 / (ms64 / args.steps_b64 / 1000) / 1e9 / HBM_PEAK_GBS, 4),
                  "b1_sample_selfloop_tok_s": round(b1_sample_tps, 2),
                  "fp16_variant": variant,
                  "prefill": prefill, "serve_ragged": serve,
                  "linear_configs1": linear, "wkv7_configs2": wkv},
    }
    print(json.dumps(out))
    bundle.close()


if __name__ == "__main__":
    main()
