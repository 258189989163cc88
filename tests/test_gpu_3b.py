"""Accuracy at the benchmarked shape: the configs[3] 3B-shape model (32
layers, d_model 2560, 40 heads x 64, FFN 10240, vocab 65536, LoRA
96/96/64/256, seed 1) through the HIP path against the CPU fp32 oracle.

These run exactly the kernels the bench times at B=1 and B=64 (the one-shot
B=1 GEMVs, the fused LoRA-up + WKV7 launches, the batched MFMA GEMMs with
3B K-slices, the prefill GEMM on 4096-row chunks) and hold them to the
north_star bounds, the same criteria as the reference's TOP1_REF /
COMPARE_LOGITS checks (main.rs):

- logits RMSE <= 1e-2 x logit std, at every checked step;
- teacher-forced top-1 agreement >= 98% for int8 linears + int8 head, and
  >= 99% for the fp16 embedding/head variant.  Teacher forcing: the oracle
  is fed the tokens the GPU chose, and its argmax at every step is compared
  with the GPU's choice.  In the B=64 check a differing token counts as
  agreeing when the oracle's gap between its argmax and the GPU's token is
  below the logits tolerance (a near tie), with strict agreement >= 95%.

The oracle splits its matvec columns over threads (bit-identical to one
thread) so that the 3B checks take seconds per token, not half a second.
"""
import os
import time

import numpy as np
import pytest

import oracle as orc
from conftest import rel_rmse, three_b_model

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(900)]

RMSE_BOUND = 1e-2
BAR = {"i8": 0.98, "i8_f16": 0.99}


def log(*a):
    print("[3b]", *a, flush=True)


def _prompt(n, seed):
    import synth
    return synth.prompt(synth.THREE_B, n, seed=seed)


@pytest.fixture(scope="module", params=["i8", "i8_f16"])
def model3b(request):
    import rsv
    kind = request.param
    t = time.time()
    path = three_b_model(kind)
    log(kind, "model file ready", f"{time.time() - t:.1f}s")
    b = rsv.ModelBuilder(path).build()
    orc.set_threads(min(16, os.cpu_count() or 1))
    t = time.time()
    m = orc.Model(path)
    log(kind, "oracle built", f"{time.time() - t:.1f}s")
    yield kind, b, m
    b.close()
    orc.set_threads(1)
    del m


def _teacher_forced(m, st, first, toks):
    """Feeds `first` then toks[:-1] to the oracle; returns its per-step logits."""
    out = []
    prev = int(first)
    for t in toks:
        out.append(m.forward([prev], st))
        prev = int(t)
    return out


def test_3b_b1_prefill_and_selfloop(model3b):
    """B=1: prompt logits and state after infer_seq, then a 64-token argmax
    self-loop (the graph-replayed step the bench times) teacher-forced
    against the oracle, with the GPU's per-token logits along the same path
    held to the RMSE bound at every step."""
    kind, b, m = model3b
    p = _prompt(16, 1)
    b.reset()
    lg = b.infer_seq(p[:-1])
    st = m.init_state()
    want = m.forward(p[:-1], st)
    e = rel_rmse(lg, want)
    es = rel_rmse(b.state_back(), st)
    log(kind, f"prefill logits rel rmse {e:.2e}, state {es:.2e}")
    assert e <= RMSE_BOUND and es <= RMSE_BOUND
    st_pre = st.copy()
    n = 64
    toks = b.infer_argmax_selfloop(int(p[-1]), n)
    t = time.time()
    olg = _teacher_forced(m, st, p[-1], toks)
    log(kind, f"oracle {n} tokens in {time.time() - t:.1f}s")
    agree = sum(int(orc.argmax(o) == toks[i]) for i, o in enumerate(olg))
    log(kind, f"B=1 teacher-forced top-1 {agree}/{n}")
    assert agree / n >= BAR[kind], f"top-1 agreement {agree}/{n}"
    # the per-token path (one decode step per call) along the same tokens:
    # logits within the bound at every step, argmax equal to the self-loop's
    b.reset()
    b.infer_seq(p[:-1])
    prev = int(p[-1])
    worst = 0.0
    for i in range(n):
        g = b.infer_tokens([prev])
        worst = max(worst, rel_rmse(g, olg[i]))
        assert int(np.argmax(g)) == int(toks[i]) or g[int(toks[i])] == g.max(), i
        prev = int(toks[i])
    log(kind, f"B=1 worst per-step logits rel rmse {worst:.2e}")
    assert worst <= RMSE_BOUND
    assert rel_rmse(b.state_back(), st) <= RMSE_BOUND
    del st_pre


def test_3b_b64_prefill_and_selfloop(model3b):
    """B=64: 64 sessions prefilled as one packed batch (512 rows: the prefill
    GEMM path), then a 24-step batched argmax self-loop (the B>=16 MFMA
    decode the bench times, graph-replayed).  The same 24 steps are replayed
    eagerly from the saved state with forward_tokens_batch, which returns
    every step's logits: its argmax must equal the self-loop's token.
    Sessions 0, 15, 31, 47 and 63 are checked against the oracle along the
    same tokens: prompt logits and every decode step's logits within the
    RMSE bound, and teacher-forced top-1 over the 120 steps.  A step whose
    token differs from the oracle's argmax counts as agreeing only when the
    oracle's own gap between the two is below the logits tolerance
    (1e-2 x its logit std: a near tie that the logits bound cannot order);
    each such step is logged, and strict agreement must still be >= 95%."""
    kind, b, m = model3b
    B, plen, n = 64, 8, 24
    prompts = [_prompt(plen, 100 + i) for i in range(B)]
    S = b.create_batch_state(B)
    try:
        seeds, lg = b.forward_seq_batch(S, [q[:-1] for q in prompts], want_logits=True)
        seeds = np.array([int(q[-1]) for q in prompts], np.uint32)
        snap = S.back()
        out = b.argmax_selfloop_batch(S, seeds, n)
        S.load(snap)
        glog = {}
        prev = seeds
        for i in range(n):
            L = b.forward_tokens_batch(S, prev)
            for s in range(B):
                t = int(out[s][i])
                assert int(np.argmax(L[s])) == t or L[s][t] == L[s].max(), (s, i)
            for s in (0, 15, 31, 47, 63):
                glog[(s, i)] = L[s].copy()
            prev = np.ascontiguousarray(out[:, i])
    finally:
        S.free()
    agree = strict = total = 0
    worst = 0.0
    for s in (0, 15, 31, 47, 63):
        st = m.init_state()
        want = m.forward(prompts[s][:-1], st)
        e = rel_rmse(lg[s], want)
        log(kind, f"B=64 session {s}: prompt logits rel rmse {e:.2e}")
        assert e <= RMSE_BOUND, s
        olg = _teacher_forced(m, st, seeds[s], out[s])
        for i, o in enumerate(olg):
            o = np.asarray(o)
            e = rel_rmse(glog[(s, i)], o)
            worst = max(worst, e)
            assert e <= RMSE_BOUND, (s, i, e)
            t, top = int(out[s][i]), int(orc.argmax(o))
            total += 1
            if top == t:
                strict += 1
                agree += 1
            elif o[top] - o[t] <= RMSE_BOUND * o.std():
                agree += 1
                log(kind, f"  session {s} step {i}: near tie, oracle top {top} at {o[top]:.4f}, GPU token {t} at "
                          f"{o[t]:.4f} (oracle logit std {o.std():.3f})")
            else:
                log(kind, f"  session {s} step {i}: oracle top {top} at {o[top]:.4f}, GPU token {t} at {o[t]:.4f}")
    log(kind, f"B=64 decode: worst per-step logits rel rmse {worst:.2e}; top-1 {strict}/{total} strict, "
              f"{agree}/{total} with near ties")
    assert strict / total >= 0.95, f"strict top-1 agreement {strict}/{total}"
    assert agree / total >= BAR[kind], f"top-1 agreement {agree}/{total}"


def _serve_vs_single(b, m, kind, sp, oracle_draw):
    """Serves six sessions; returns, per draw, whether the oracle sampler on
    the served logits row gives the served token.  Each served row is held
    to the logits bound against the session run alone along the same tokens
    (B=1 prefill, then one token at a time)."""
    lens = [5, 300, 37, 700, 64, 129]
    prompts = [_prompt(L, 200 + i) for i, L in enumerate(lens)]
    seeds = [3, 5, 7, 11, 13, 17]
    D = 6
    S = b.create_batch_state(len(lens))
    try:
        toks, steps, slg = b.serve_ragged(S, prompts, D, sp, seeds, budget=512, want_logits=True)
    finally:
        S.free()
    assert sum(s["prefill_tokens"] for s in steps) == sum(lens)
    assert sum(s["sampled"] for s in steps) == len(lens) * D
    assert any(s["prefill_tokens"] and s["decode_tokens"] for s in steps)
    assert any(s["prefill_tokens"] == 0 and s["decode_tokens"] == len(lens) for s in steps), "no all-decode step"
    res = []
    for q, p in enumerate(prompts):
        b.reset()
        lg = b.infer_seq(p)
        if q == 0:
            st = m.init_state()
            e = rel_rmse(lg, m.forward(p, st))
            log(kind, f"serve: session 0 prompt logits rel rmse {e:.2e}")
            assert e <= RMSE_BOUND
        for k in range(D):
            if k:
                lg = b.infer_seq([int(toks[q, k - 1])])
            e = rel_rmse(slg[q, k], lg)
            assert e <= RMSE_BOUND, (q, k, e)
            got, want = int(toks[q, k]), int(oracle_draw(slg[q, k], seeds[q] + k))
            if got != want:
                log(kind, f"serve q={q} k={k}: served {got}, oracle on the served row {want}")
            res.append(got == want)
    return res


def test_3b_serve_ragged_greedy_matches_per_session(model3b):
    """configs[4] at the 3B shape, scaled down: six sessions with prompts of
    5..700 tokens served by the ragged scheduler with a 512-token budget
    (prompts split across steps and sharing steps with decode tokens),
    drawn by the GPU sampler with top_k = 1.  Two separate checks per draw:
    the draw is exactly the argmax of the logits row it was drawn from, and
    that row (packed prefill or batched decode) is within the logits bound of
    the same session run alone along the same tokens.  Session 0's prompt
    logits are also checked against the oracle."""
    import rsv
    kind, b, m = model3b
    sp = rsv.SamplerParams(temperature=1.0, top_k=1, top_p=1.0)
    res = _serve_vs_single(b, m, kind, sp, lambda lg, seed: int(orc.argmax(lg)))
    log(kind, f"serve greedy: exact draws {sum(res)}/{len(res)}")
    assert all(res), res


def test_3b_serve_ragged_top_p_matches_per_session(model3b):
    """The same schedule with the configs[4] sampler (T = 1, top_p = 0.9,
    seeded): every draw is exactly the oracle sampler's draw on the logits
    row it was drawn from, and every row meets the logits bound against the
    session run alone."""
    import rsv
    kind, b, m = model3b
    sp = rsv.SamplerParams(temperature=1.0, top_k=0, top_p=0.9)
    res = _serve_vs_single(b, m, kind, sp, lambda lg, seed: orc.sample(lg, sp.temperature, sp.top_k, sp.top_p, seed))
    log(kind, f"serve top-p: exact draws {sum(res)}/{len(res)}")
    assert all(res), res
