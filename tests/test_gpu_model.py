"""Whole-model parity of the HIP path (librsv_host.so over librsv_hip.so)
against the CPU fp32 oracle, plus the Bundle/State API contract.

Accuracy bar: logits RMSE <= 1e-2 x logit std; teacher-forced top-1
agreement >= 99% (fp16 / fp32 files) or >= 98% (int8); argmax indices and
state serialisation bit-exact where the arithmetic is (round trips)."""
import numpy as np
import pytest

import oracle as orc
from conftest import SMALL, rel_rmse

pytestmark = pytest.mark.gpu

RMSE_BOUND = 1e-2


def _rsv():
    import rsv
    return rsv


@pytest.fixture(scope="module")
def bundles(small_f32, small_f16, small_i8, small_i8_group):
    rsv = _rsv()
    out = {}
    for name, path in (("f32", small_f32), ("f16", small_f16), ("i8", small_i8), ("i8g", small_i8_group)):
        out[name] = (rsv.ModelBuilder(path).build(), orc.Model(path))
    yield out
    for b, _ in out.values():
        b.close()


def _prompt(n, seed):
    import synth
    return synth.prompt(SMALL, n, seed=seed)


@pytest.mark.parametrize("kind", ["f32", "f16", "i8", "i8g"])
def test_infer_tokens_matches_oracle(bundles, kind):
    b, m = bundles[kind]
    b.reset()
    st = m.init_state()
    for t in _prompt(24, 1):
        got = b.infer_tokens([t])
        want = m.forward([t], st)
        assert rel_rmse(got, want) <= RMSE_BOUND
    # state after the same tokens
    assert rel_rmse(b.state_back(), st) <= RMSE_BOUND


@pytest.mark.parametrize("kind", ["f32", "i8"])
def test_infer_seq_matches_oracle_and_decode(bundles, kind):
    b, m = bundles[kind]
    p = _prompt(77, 2)
    b.reset()
    lg_seq = b.infer_seq(p)
    st_seq = b.state_back()
    st = m.init_state()
    want = m.forward(p, st)
    assert rel_rmse(lg_seq, want) <= RMSE_BOUND
    assert rel_rmse(st_seq, st) <= RMSE_BOUND
    b.reset()
    lg_tok = b.infer_tokens(p)
    assert rel_rmse(lg_tok, lg_seq) <= RMSE_BOUND
    # chunked prefill carries state across chunks
    b.reset()
    lg_ch = b.infer_chunked(p, 10)
    assert rel_rmse(lg_ch, lg_seq) <= 1e-4


@pytest.mark.parametrize("kind,bar", [("f32", 0.99), ("f16", 0.99), ("i8", 0.98)])
def test_argmax_selfloop_teacher_forced(bundles, kind, bar):
    b, m = bundles[kind]
    p = _prompt(16, 3)
    b.reset()
    b.infer_seq(p[:-1])
    n = 48
    toks = b.infer_argmax_selfloop(int(p[-1]), n)
    st = m.init_state()
    m.forward(p[:-1], st)
    agree = 0
    prev = int(p[-1])
    for i in range(n):
        lg = m.forward([prev], st)
        agree += orc.argmax(lg) == toks[i]
        prev = int(toks[i])  # teacher forcing along the GPU's path
    assert agree / n >= bar, f"top-1 agreement {agree}/{n}"


def test_argmax_selfloop_equals_per_token_argmax(bundles):
    """ARGMAX_VERIFY / SELFLOOP_VERIFY (main.rs:1056-1088): the graph-replayed
    self-loop equals per-token infer_argmax on the same device path."""
    b, _ = bundles["i8"]
    b.reset()
    loop = b.infer_argmax_selfloop(17, 20)
    b.reset()
    tok = 17
    for i in range(20):
        tok = b.infer_argmax([tok])
        assert tok == loop[i], i


def test_state_roundtrip_bit_exact(bundles):
    """examples/state_persist.rs:38-69: back -> load -> back is lossless and
    generation continues identically."""
    b, _ = bundles["f16"]
    b.reset()
    b.infer_seq(_prompt(30, 4))
    s1 = b.state_back()
    cont1 = b.infer_tokens([5, 6, 7])
    b.reset()
    assert np.all(b.state_back() == 0)
    b.state_load(s1)
    s2 = b.state_back()
    assert np.array_equal(s1.view(np.uint32), s2.view(np.uint32))
    cont2 = b.infer_tokens([5, 6, 7])
    assert np.array_equal(cont1.view(np.uint32), cont2.view(np.uint32))
    rsv = _rsv()
    with pytest.raises(rsv.RsvError, match="length mismatch"):
        b.state_load(s1[:-1])


def test_batch_prefill_and_decode_match_single(bundles):
    """forward_seq_batch over ragged prompts against per-session infer_seq
    (the batch's last-token rows run on the fp16-activation MFMA path, the
    single session's on the fp32 GEMVs: 1e-3 apart), the batched argmax
    self-loop against the oracle teacher-forced along it, slot back/load."""
    b, m = bundles["i8"]
    lens = [5, 17, 1, 33]
    prompts = [_prompt(l, 10 + i) for i, l in enumerate(lens)]
    S = b.create_batch_state(len(lens))
    seeds, lg = b.forward_seq_batch(S, prompts, want_logits=True)
    assert list(seeds) == [int(p[-1]) for p in prompts]
    for i, p in enumerate(prompts):
        b.reset()
        lg1 = b.infer_seq(p)
        assert rel_rmse(lg[i], lg1) <= 1e-3
        assert rel_rmse(S.slot_back(i), b.state_back()) <= 1e-3
    n = 40
    out = b.argmax_selfloop_batch(S, seeds, n)
    agree = 0
    for i, p in enumerate(prompts):
        st = m.init_state()
        m.forward(p[:-1], st)
        prev = int(seeds[i])
        for t in range(n):
            agree += orc.argmax(m.forward([prev], st)) == out[i, t]
            prev = int(out[i, t])
    assert agree / (n * len(prompts)) >= 0.98
    # slot round trip and bounds
    data = S.slot_back(2)
    S.slot_load(0, data)
    assert np.array_equal(S.slot_back(0).view(np.uint32), data.view(np.uint32))
    rsv = _rsv()
    with pytest.raises(rsv.RsvError, match="slot"):
        S.slot_back(9)
    S.free()


@pytest.mark.parametrize("chunk", [200, 96])
def test_prefill_lanes_bit_identical(bundles, chunk):
    """The pipelined prefill (consecutive packed chunks on two streams, each
    waiting per layer only for the state its predecessor leaves) against the
    one-stream prefill: every slot's state bit for bit, for batch prefill
    over many chunks (chunk 200: large chunks and a small last one; 96: all
    chunks on the batched-decode kernels) and for one long single-session
    prompt, then the next decode step's logits bit for bit."""
    b, m = bundles["i8"]
    lens = [300, 17, 1, 233, 90]
    prompts = [_prompt(l, 40 + i) for i, l in enumerate(lens)]
    b.set_prefill_chunk(chunk)
    try:
        got = {}
        for lanes in (1, 2):
            b.set_prefill_lanes(lanes)
            S = b.create_batch_state(len(lens))
            seeds = b.forward_seq_batch(S, prompts)
            states = [S.slot_back(i).view(np.uint32).copy() for i in range(len(lens))]
            lg = b.forward_tokens_batch(S, np.asarray(seeds, np.uint32))
            S.free()
            b.reset()
            lg1 = b.infer_seq(_prompt(700, 77))
            got[lanes] = (states, np.asarray(lg).view(np.uint32).copy(), lg1.view(np.uint32).copy(),
                          b.state_back().view(np.uint32).copy())
        for i in range(len(lens)):
            assert np.array_equal(got[1][0][i], got[2][0][i]), f"slot {i} state"
        for k in (1, 2, 3):
            assert np.array_equal(got[1][k], got[2][k])
    finally:
        b.set_prefill_lanes(2)
        b.set_prefill_chunk(4096)
        b.reset()


def test_forward_tokens_batch_matches_single(bundles):
    b, m = bundles["f32"]
    S = b.create_batch_state(3)
    toks = np.array([[1, 2, 3], [500, 7, 1023], [9, 9, 9]], np.uint32)
    for t in range(3):
        lg = b.forward_tokens_batch(S, toks[:, t])
    for i in range(3):
        st = m.init_state()
        want = m.forward(toks[i], st)
        assert rel_rmse(lg[i], want) <= RMSE_BOUND
        assert rel_rmse(S.slot_back(i), st) <= RMSE_BOUND
    S.free()


def test_sample_selfloop_teacher_forced(bundles):
    """Sampling self-loop: per round seed = seed_token + round, history = the
    tokens generated so far (gpu_model.rs:799-812); each draw agrees with the
    oracle sampler on the oracle's logits along the GPU path."""
    rsv = _rsv()
    b, m = bundles["f32"]
    sp = rsv.SamplerParams(temperature=1.0, top_k=0, top_p=0.9, repetition_penalty=1.1, frequency_penalty=0.1)
    p = _prompt(8, 5)
    b.reset()
    b.infer_seq(p[:-1])
    n = 24
    seed = int(p[-1])
    toks = b.infer_sample_selfloop(seed, n, sp)
    st = m.init_state()
    m.forward(p[:-1], st)
    prev = seed
    agree = 0
    for r in range(n):
        lg = m.forward([prev], st)
        want = orc.sample(lg, sp.temperature, sp.top_k, sp.top_p, seed + r, sp.repetition_penalty,
                          sp.frequency_penalty, sp.presence_penalty, toks[:r].tolist())
        agree += want == toks[r]
        prev = int(toks[r])
    assert agree >= n - 1, f"{agree}/{n}"


def test_sample_selfloop_batch_low_temperature_is_argmax(bundles):
    rsv = _rsv()
    b, _ = bundles["i8"]
    S = b.create_batch_state(2)
    seeds = b.forward_seq_batch(S, [_prompt(4, 20), _prompt(9, 21)])
    snap = S.back()
    got = b.sample_selfloop_batch(S, seeds, 10, rsv.SamplerParams(temperature=1e-4, top_k=50))
    S.load(snap)
    ref = b.argmax_selfloop_batch(S, seeds, 10)
    assert np.array_equal(got, ref)
    S.free()


def test_api_errors(bundles):
    rsv = _rsv()
    b, _ = bundles["f32"]
    with pytest.raises(rsv.RsvError, match="vocab"):
        b.infer_tokens([SMALL["vocab"] + 5])
    with pytest.raises(rsv.RsvError, match="empty"):
        b.infer_seq([])
    with pytest.raises(rsv.RsvError):
        rsv.ModelBuilder("/nonexistent/model.st").build()


def test_config1_golden(tiny_cfg1):
    """Config 1: tiny model seed 0, 64-token prompt + 32 greedy tokens; the GPU
    tokens must equal the committed golden tokens (teacher-forced >= 99%) and
    the final logits meet the RMSE bound."""
    import json
    import os
    rsv = _rsv()
    gdir = os.path.join(os.path.dirname(__file__), "golden")
    meta = json.load(open(os.path.join(gdir, "config1.json")))
    prompt = np.array(meta["prompt"], np.uint32)
    gold = np.array(meta["greedy"], np.uint32)
    b = rsv.ModelBuilder(tiny_cfg1).build()
    b.infer_seq(prompt[:-1])
    toks = b.infer_argmax_selfloop(int(prompt[-1]), 32)
    agree = int((toks == gold).sum())
    first_div = int(np.argmax(toks != gold)) if agree < 32 else 32
    assert first_div >= 31 or agree >= 31, f"golden mismatch at {first_div}: {toks} vs {gold}"
    # last-prompt-token logits against the committed fixture
    b.reset()
    lg = b.infer_seq(prompt)
    ref = np.load(os.path.join(gdir, "config1_prompt_logits.npy")).astype(np.float32)
    assert rel_rmse(lg, ref) <= RMSE_BOUND
    b.close()


@pytest.mark.parametrize("kind", ["f32", "i8"])
def test_fused_decode_matches_trait_op_sequence(bundles, kind, monkeypatch):
    """The six-launch fused layer equals the reference's one-op-per-method
    sequence (norm_lerp6, stage1, chain4, fuse_ka_dplr_norm, ...)."""
    b, _ = bundles[kind]
    p = _prompt(10, 30)
    b.reset()
    fused = [b.infer_tokens([t]) for t in p]
    s_fused = b.state_back()
    monkeypatch.setenv("RSV_DECODE_TRAIT_OPS", "1")
    b.reset()
    ops = [b.infer_tokens([t]) for t in p]
    s_ops = b.state_back()
    monkeypatch.delenv("RSV_DECODE_TRAIT_OPS")
    for a, c in zip(fused, ops):
        assert rel_rmse(a, c) <= 1e-5
    assert rel_rmse(s_fused, s_ops) <= 1e-5


@pytest.mark.parametrize("kind,bar,B", [("f32", 0.98, 20), ("i8", 0.98, 20), ("i8", 0.98, 2), ("f32", 0.98, 5),
                                        ("i8", 0.98, 8), ("i8", 0.98, 15)])
def test_batch_matrix_core_decode(bundles, kind, bar, B):
    """B >= 2 runs the decode GEMMs on MFMA with fp16 activations: logits and
    states meet the RMSE bound against the oracle, and the batched argmax
    self-loop agrees teacher-forced with the oracle."""
    b, m = bundles[kind]
    S = b.create_batch_state(B)
    prompts = [_prompt(3 + (i % 5), 40 + i) for i in range(B)]
    seeds = b.forward_seq_batch(S, prompts)
    snap = S.back()
    toks = np.array([(7 * i + 3) % SMALL["vocab"] for i in range(B)], np.uint32)
    lg = b.forward_tokens_batch(S, toks)
    for i in sorted(set(range(0, B, 7)) | {B - 1}):
        st = m.init_state()
        m.forward(prompts[i], st)
        want = m.forward([int(toks[i])], st)
        assert rel_rmse(lg[i], want) <= RMSE_BOUND
        assert rel_rmse(S.slot_back(i), st) <= RMSE_BOUND
    S.load(snap)
    n = max(12, 240 // B)  # about 240 teacher-forced tokens per case
    out = b.argmax_selfloop_batch(S, seeds, n)
    agree = total = 0
    for i in range(B):
        st = m.init_state()
        m.forward(prompts[i][:-1], st)
        prev = int(seeds[i])
        for t in range(n):
            agree += orc.argmax(m.forward([prev], st)) == out[i, t]
            total += 1
            prev = int(out[i, t])
    assert agree / total >= bar
    S.free()


def test_serve_ragged_matches_per_session_runs(bundles):
    """Ragged continuous batching: prompts of mixed lengths, split across
    steps by a small token budget and interleaved with other slots' decode
    tokens.  Two separate checks per draw: the served token is exactly the
    oracle sampler's draw (seed rule: token k of slot q takes seeds[q] + k) on
    the logits row it was drawn from, and that row (packed prefill, or the
    batched decode step when every slot decodes) is within 1e-3 of the same
    session served alone along the same tokens."""
    rsv = _rsv()
    b, _ = bundles["i8"]
    lens = [1, 7, 19, 3, 30]
    prompts = [_prompt(n, 40 + i) for i, n in enumerate(lens)]
    seeds = [11, 22, 33, 44, 55]
    sp = rsv.SamplerParams(temperature=1.0, top_k=0, top_p=0.9)
    D, budget = 6, 16
    S = b.create_batch_state(len(lens))
    toks, steps, slg = b.serve_ragged(S, prompts, D, sp, seeds, budget=budget, want_logits=True)
    S.free()
    # schedule accounting
    assert sum(s["prefill_tokens"] for s in steps) == sum(lens)
    assert sum(s["decode_tokens"] for s in steps) == len(lens) * (D - 1)
    assert sum(s["sampled"] for s in steps) == len(lens) * D
    assert all(s["prefill_tokens"] + s["decode_tokens"] <= budget for s in steps)
    assert any(s["prefill_tokens"] and s["decode_tokens"] for s in steps), "no step mixed prefill and decode"
    assert any(s["prefill_tokens"] == 0 and s["decode_tokens"] == len(lens) for s in steps), "no all-decode step"
    for q, p in enumerate(prompts):
        b.reset()
        lg = b.infer_seq(p)
        for k in range(D):
            if k:
                lg = b.infer_seq([int(toks[q, k - 1])])
            assert rel_rmse(slg[q, k], lg) <= 1e-3, (q, k)
            want = orc.sample(slg[q, k], sp.temperature, sp.top_k, sp.top_p, seeds[q] + k)
            assert int(toks[q, k]) == want, (q, k)


def test_serve_ragged_errors(bundles):
    rsv = _rsv()
    b, _ = bundles["i8"]
    sp = rsv.SamplerParams()
    S = b.create_batch_state(3)
    with pytest.raises(rsv.RsvError):
        b.serve_ragged(S, [_prompt(4, 1), _prompt(4, 2), _prompt(4, 3)], 2, sp, [1, 2, 3], budget=2)
    with pytest.raises(rsv.RsvError):
        b.serve_ragged(S, [_prompt(4, 1), [], _prompt(4, 3)], 2, sp, [1, 2, 3], budget=8)
    with pytest.raises(rsv.RsvError):
        b.serve_ragged(S, [_prompt(4, 1), _prompt(4, 2)], 2, sp, [1, 2], budget=8)
    S.free()


def test_sparse_ffn_value_decode(small_i8, monkeypatch):
    """RSV_FFN_SPARSE=1 (gpu_model.rs:2353-2371): the decode layer reads only the
    ffn.value rows whose relu^2 input is non-zero, from the tiled fp16 copy.
    Logits stay within the oracle bound and close to the dense int8 path (the
    copy rounds the dequantised weights to fp16)."""
    import rsv
    monkeypatch.setenv("RSV_FFN_SPARSE", "1")
    bs = rsv.ModelBuilder(small_i8).build()
    monkeypatch.delenv("RSV_FFN_SPARSE")
    bd = rsv.ModelBuilder(small_i8).build()
    m = orc.Model(small_i8)
    try:
        p = _prompt(16, 41)
        monkeypatch.setenv("RSV_FFN_SPARSE", "1")
        got = [bs.infer_tokens([t]) for t in p]
        monkeypatch.delenv("RSV_FFN_SPARSE")
        dense = [bd.infer_tokens([t]) for t in p]
        st = m.init_state()
        want = m.forward(list(p), st)
        assert rel_rmse(got[-1], want) <= RMSE_BOUND
        for g, d in zip(got, dense):
            assert rel_rmse(g, d) <= 2e-3
    finally:
        bs.close()
        bd.close()


@pytest.mark.parametrize("kind", ["f32", "f16", "i8", "i8g"])
def test_fused_lora_wkv_matches_two_launches(bundles, kind, monkeypatch):
    """rsv_wkv7_lora_decode (LoRA-up chain + WKV7 + GroupNorm in one launch)
    equals the two-launch form (gemv_lowrank_chain4 then fuse_ka_dplr_norm)
    on logits and state, fp32 throughout."""
    b, _ = bundles[kind]
    p = _prompt(12, 52)
    monkeypatch.setenv("RSV_WKV_LORA", "0")
    b.reset()
    two = [b.infer_tokens([t]) for t in p]
    s_two = b.state_back()
    monkeypatch.setenv("RSV_WKV_LORA", "1")
    b.reset()
    one = [b.infer_tokens([t]) for t in p]
    s_one = b.state_back()
    for a, c in zip(one, two):
        assert rel_rmse(a, c) <= 1e-5
    assert rel_rmse(s_one, s_two) <= 1e-5


@pytest.mark.parametrize("kind,B", [("f16", 20), ("i8", 20), ("i8", 37)])
def test_batched_fused_lora_wkv(bundles, kind, B, monkeypatch):
    """The batched layer's fused LoRA-up + WKV7 launch (RSV_WKV_LORA_MM=1,
    fp16 operands in and out, 4 sessions per block) equals its two-launch
    form to fp32 rounding, also on batches that leave the last block partly
    empty."""
    b, _ = bundles[kind]
    prompts = [_prompt(3 + (i % 5), 60 + i) for i in range(B)]
    toks = np.array([(11 * i + 5) % SMALL["vocab"] for i in range(B)], np.uint32)
    out = {}
    for flag in ("0", "1"):
        monkeypatch.setenv("RSV_WKV_LORA_MM", flag)
        S = b.create_batch_state(B)
        b.forward_seq_batch(S, prompts)
        lg = b.forward_tokens_batch(S, toks)
        out[flag] = (lg.copy(), S.back().copy())
        S.free()
    assert rel_rmse(out["1"][0], out["0"][0]) <= 1e-4
    assert rel_rmse(out["1"][1], out["0"][1]) <= 1e-4


@pytest.mark.parametrize("kind", ["i8", "i8g"])
def test_prefill_f16_weight_copies_bit_identical(bundles, kind, monkeypatch):
    """Prefill of more than 128 packed rows runs its int8 layer matrices on
    fp16 copies made with the int8 loader's roundings; logits and state equal those of the int8 loader bit for bit."""
    b, _ = bundles[kind]
    prompts = [_prompt(90 + 17 * i, 300 + i) for i in range(3)]
    out = {}
    for flag in ("0", "1"):
        monkeypatch.setenv("RSV_PREFILL_F16", flag)
        S = b.create_batch_state(3)
        _, lg = b.forward_seq_batch(S, prompts, want_logits=True)
        out[flag] = (lg.copy(), S.back().copy())
        S.free()
    assert np.array_equal(out["1"][0], out["0"][0])
    assert np.array_equal(out["1"][1], out["0"][1])


@pytest.mark.parametrize("env", ["RSV_WKV_LORA_MM=0"])
def test_batched_alternative_kernels_agree(bundles, env, monkeypatch):
    """Each selectable alternative of the batched paths (the two-launch
    LoRA-up + WKV7) gives the default's logits and state to fp32 rounding, on a
    prefill of more than 128 packed rows and batched decode steps."""
    b, _ = bundles["i8"]
    B = 20
    prompts = [_prompt(4 + 9 * (i % 4), 500 + i) for i in range(B)]
    toks = np.array([(7 * i + 3) % SMALL["vocab"] for i in range(B)], np.uint32)
    out = {}
    for flag in ("default", env):
        if flag != "default":
            name, val = flag.split("=")
            monkeypatch.setenv(name, val)
        S = b.create_batch_state(B)
        _, lp = b.forward_seq_batch(S, prompts, want_logits=True)
        lg = b.forward_tokens_batch(S, toks)
        lg2 = b.forward_tokens_batch(S, toks[::-1].copy())
        out[flag] = (lp.copy(), lg.copy(), lg2.copy(), S.back().copy())
        S.free()
    for got, want in zip(out[env], out["default"]):
        assert rel_rmse(got, want) <= 1e-4


@pytest.mark.parametrize("kind", ["i8", "f16"])
def test_prefill_graph_replay_bit_exact(bundles, kind, monkeypatch):
    """PREFILL_GRAPH=1 (gpu_model.rs:2440-2507): a prefill chunk is captured
    as a HIP graph per (rows, segments, state, head) and replayed for later
    chunks of the same shape.  Replays with other tokens, shapes that
    alternate (small and large packed chunks), and a multi-session packed
    prefill give the eager path's logits and state bit for bit."""
    b, _ = bundles[kind]
    prompts = [_prompt(40, 700), _prompt(40, 701), _prompt(200, 702), _prompt(40, 703)]

    def run_all():
        out = []
        for p in prompts:
            b.reset()
            lg = b.infer_seq(p)
            out.append((lg.copy(), b.state_back().copy()))
        S = b.create_batch_state(3)
        _, lg = b.forward_seq_batch(S, [prompts[0][:7], prompts[2][:150], prompts[1][:33]], want_logits=True)
        _, lg2 = b.forward_seq_batch(S, [prompts[3][:7], prompts[1][:150], prompts[0][:33]], want_logits=True)
        out.append((lg.copy(), lg2.copy(), S.back().copy()))
        S.free()
        return out

    monkeypatch.delenv("PREFILL_GRAPH", raising=False)
    eager = run_all()
    monkeypatch.setenv("PREFILL_GRAPH", "1")
    graph = run_all()
    graph2 = run_all()  # graphs captured by the previous pass, replayed
    monkeypatch.delenv("PREFILL_GRAPH")
    for e, g, g2 in zip(eager, graph, graph2):
        for a, c, d in zip(e, g, g2):
            assert np.array_equal(a.view(np.uint32), c.view(np.uint32))
            assert np.array_equal(a.view(np.uint32), d.view(np.uint32))


def test_build_shared_weights(small_i8):
    """GpuModel::build_shared (gpu_model.rs:594-628): instances on shared
    weights give the source's logits bit for bit, each with its own state;
    freeing the source leaves the importer valid, and an instance imported
    from an importer works after its parent is freed."""
    rsv = _rsv()
    src = rsv.ModelBuilder(small_i8).build()
    p = _prompt(33, 900)
    want = src.infer_seq(p)
    st_want = src.state_back()
    a = src.build_shared()
    got = a.infer_seq(p)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # the source's own session is untouched by the importer's run
    assert np.array_equal(src.state_back().view(np.uint32), st_want.view(np.uint32))
    # batched path on the importer (its own tiled weight copies)
    S = a.create_batch_state(17)
    lg_b = a.forward_seq_batch(S, [p] * 17, want_logits=True)[1]
    S.free()
    assert rel_rmse(lg_b[5], want) <= 1e-3
    src.close()
    a.reset()
    got2 = a.infer_seq(p)
    assert np.array_equal(got2.view(np.uint32), want.view(np.uint32))
    c = a.build_shared()
    a.close()
    got3 = c.infer_seq(p)
    assert np.array_equal(got3.view(np.uint32), want.view(np.uint32))
    toks = c.infer_argmax_selfloop(int(p[-1]), 4)
    assert len(toks) == 4
    c.close()
