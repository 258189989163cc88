"""Benchmark of the rwkv-rsv hot path on one MI355X.

Workload (the metric's configuration): 3B-shape
RWKV-7 (32 layers, d_model 2560, 40 heads x 64, FFN 10240, vocab 65536,
LoRA 96/96/64/256), random-init seed 1, int8 per-row-scale linears + int8
head in the reference's int8 format.  Each session is seeded with a 32-token
uniform random prompt (prefilled untimed), then the argmax decode self-loop
runs:
  - B=1:  `--steps` tokens (one step = one decoded token)      -> `value`
  - B=64: `--steps-b64` steps of 64 concurrent sessions         -> extra
and the ragged prefill of configs[4] (64 prompts, lengths U[16, 2048] seed 2,
packed into chunks of <= 4096 tokens) is timed once               -> extra.

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


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def model_path(cache_dir):
    import synth
    path = os.path.join(cache_dir, "rsv_3b_i8_seed1.st")
    if not os.path.exists(path):
        t = time.time()
        tmp = path + ".tmp"
        synth.write_model(tmp, synth.THREE_B, seed=1, linear="i8", head="i8")
        os.replace(tmp, path)
        log(f"generated {path} in {time.time() - t:.1f}s")
    return path


def decode_bytes_per_step(cfg, batch):
    """Algorithmic HBM bytes of one decode step (int8 linears + int8 head,
    fp16 LoRA, fp32 state and activations)."""
    C, L, F, V = cfg["c"], cfg["n_layer"], cfg["ffn"], cfg["vocab"]
    H, N = cfg["n_head"], cfg["head_size"]
    lin = L * (4 * C * C + 2 * C * F) * (1 + 1 / 32)
    head = V * C * (1 + 1 / 32)
    lora = L * 2 * C * (cfg["wm"] + cfg["am"] + cfg["vm"] + cfg["gm"]) * 2
    vec = L * 14 * C * 4
    per_session = L * (2 * H * N * N * 4 + 4 * C * 4) + V * 4
    return lin + head + lora + vec + batch * per_session


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=32)
    ap.add_argument("--steps-b64", type=int, default=200)
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-tokens", type=int, default=4)
    ap.add_argument("--cache", default=os.environ.get("RSV_BENCH_CACHE", "/tmp"))
    ap.add_argument("--no-graph", action="store_true",
                    help="enqueue self-loop steps eagerly instead of replaying a HIP graph (profiling)")
    args = ap.parse_args()
    if args.no_graph:
        os.environ["RSV_NO_GRAPH"] = "1"
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}).",
              file=sys.stderr)
        sys.exit(2)

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
    S1.load(bundle.state_back())
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
    S1.free()

    # ---------------- B = 64 argmax self-loop
    B = 64
    S = bundle.create_batch_state(B)
    prompts = [synth.prompt(cfg, 32, seed=100 + i) for i in range(B)]
    seeds = bundle.forward_seq_batch(S, [p[:-1] for p in prompts])
    seeds = np.array([int(p[-1]) for p in prompts], np.uint32)
    snap = S.back()
    bundle.argmax_selfloop_batch(S, seeds, 4)
    S.load(snap)
    _, ms64 = bundle.argmax_selfloop_batch_timed(S, seeds, args.steps_b64)
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
        bundle.forward_seq_batch(SP, [p[:16] for p in pr])  # warm-up
        SP.reset()
        rsv.hip_lib().rsv_synchronize(bundle.ctx())
        t0 = time.perf_counter()
        bundle.forward_seq_batch(SP, pr)
        rsv.hip_lib().rsv_synchronize(bundle.ctx())
        dt = time.perf_counter() - t0
        prefill = dict(tokens=int(lens.sum()), seconds=dt, tok_s=float(lens.sum() / dt))
        log(f"prefill: {lens.sum()} tokens in {dt:.3f}s -> {prefill['tok_s']:.0f} tok/s")
        SP.free()

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
        "roofline": {"bound": "hbm", "achieved": round(bytes1 / (ms / args.steps / 1000) / 1e9, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(bytes1 / (ms / args.steps / 1000) / 1e9 / HBM_PEAK_GBS, 4),
                     "traffic": None, "scope": "whole decode step (all kernels)"},
        "cpu_baseline": cpu,
        "extra": {"b1_wall_tok_s": round(b1_wall_tps, 2),
                  "b64_tok_s": round(b64_tps, 1), "b64_ms_per_step": round(ms64 / args.steps_b64, 4),
                  "b64_hbm_frac": round(bytes64 / (ms64 / args.steps_b64 / 1000) / 1e9 / HBM_PEAK_GBS, 4),
                  "prefill": prefill},
    }
    print(json.dumps(out))
    bundle.close()


if __name__ == "__main__":
    main()
