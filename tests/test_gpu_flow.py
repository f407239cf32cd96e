"""GPU parity for GEMV flows (rt_hip_flow_*): a decode step's chain of
dependent GEMV stages in one persistent launch.

The chain is two Llama layers and an lm_head (LlamaBlock::forward_cached,
src/transformer5.cpp:198-212, with the attention between q/k/v and o left
out: o reads q) at small widths:
    q, k, v = W . rmsnorm(h)        o: h1 = h + Wo . q
    gate, up = W . rmsnorm(h1)      down: h2 = h1 + Wd . (silu(gate) * up)
    logits = Wlm . rmsnorm(h2_last)
layer 0 all Q4_K, layer 1 widened as Q4_K_M does (BF16 v in a stage of its
own, BF16 down), and an lm_head of 2500 tiles (more than one round of tiles
per workgroup).

* Every stage against the oracle applied to the flow's own inputs (its
  plain output copies): normwise 1e-5, the stand-alone GEMVs' bar.  The
  gate/up stage also stores silu(gate) * up, which down reads.
* The whole chain against the oracle's composition from h: normwise 1e-5.
* Runs are deterministic and repeatable (the tags advance every run); a
  captured graph replays with the external input read afresh each time.
* Malformed flows are refused at create.
"""
import numpy as np
import pytest

from helpers import from_dev, normwise_err, say, to_dev

pytestmark = pytest.mark.gpu
TOL = 1e-5
H, F, NKV, V = 512, 1024, 256, 40000
EPS = 1e-5


def build(rt, orc, rng):
    import torch

    def q4(n, k):
        blocks = orc.q4k_quantize((rng.standard_normal((n, k)) * 0.05).astype(np.float32))
        return blocks, rt.q4k_tile(to_dev(blocks), n, k)

    def bf(n, k):
        w = orc.f32_to_bf16_n((rng.standard_normal((n, k)) * 0.05).astype(np.float32))
        return w, to_dev(w.view(np.int16))

    def gam(n):
        return (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)

    h0 = rng.standard_normal(H).astype(np.float32)
    vecs = [(H, to_dev(h0))]
    names = {"h0": 0}

    def vec(name, n):
        names[name] = len(vecs)
        vecs.append((n, None))
        return names[name]

    plains, W, stages = {}, {}, []

    def job(fmt, w, n, out, add=-1):
        plains[out] = torch.empty(n, device="cuda")
        return {"format": fmt, "w": w, "n": n, "out": names[out], "add": names[add] if add != -1 else -1,
                "plain": plains[out]}

    h_in = "h0"
    for layer, widened in ((0, False), (1, True)):
        p = f"L{layer}."
        for nm, n in (("q", H), ("k", NKV), ("v", NKV), ("h1", H), ("gate", F), ("up", F), ("act", F), ("h2", H)):
            vec(p + nm, n)
        W[p + "q"], tq = q4(H, H)
        W[p + "k"], tk = q4(NKV, H)
        W[p + "v"], tv = bf(NKV, H) if widened else q4(NKV, H)
        W[p + "o"], to = q4(H, H)
        W[p + "gate"], tg = q4(F, H)
        W[p + "up"], tu = q4(F, H)
        W[p + "down"], td = bf(H, F) if widened else q4(H, F)
        W[p + "g1"], W[p + "g2"] = gam(H), gam(H)
        g1, g2 = to_dev(W[p + "g1"]), to_dev(W[p + "g2"])
        qk = [job(rt.Q4K, tq, H, p + "q"), job(rt.Q4K, tk, NKV, p + "k")]
        if widened:
            stages.append({"k": H, "xop": rt.XOP_RMSNORM, "in0": names[h_in], "gamma": g1, "eps": EPS, "jobs": qk})
            stages.append({"k": H, "xop": rt.XOP_RMSNORM, "in0": names[h_in], "gamma": g1, "eps": EPS,
                           "jobs": [job(rt.BF16, tv, NKV, p + "v")]})
        else:
            stages.append({"k": H, "xop": rt.XOP_RMSNORM, "in0": names[h_in], "gamma": g1, "eps": EPS,
                           "jobs": qk + [job(rt.Q4K, tv, NKV, p + "v")]})
        stages.append({"k": H, "in0": names[p + "q"], "jobs": [job(rt.Q4K, to, H, p + "h1", add=h_in)]})
        stages.append({"k": H, "xop": rt.XOP_RMSNORM, "in0": names[p + "h1"], "gamma": g2, "eps": EPS,
                       "act": names[p + "act"],
                       "jobs": [job(rt.Q4K, tg, F, p + "gate"), job(rt.Q4K, tu, F, p + "up")]})
        stages.append({"k": F, "in0": names[p + "act"],
                       "jobs": [job(rt.BF16 if widened else rt.Q4K, td, H, p + "h2", add=p + "h1")]})
        h_in = p + "h2"
    vec("logits", V)
    W["lm"], tl = q4(V, H)
    W["gf"] = gam(H)
    stages.append({"k": H, "xop": rt.XOP_RMSNORM, "in0": names[h_in], "gamma": to_dev(W["gf"]), "eps": EPS,
                   "jobs": [job(rt.Q4K, tl, V, "logits")]})
    return vecs, stages, plains, W, h0


def mm(orc, w, n, k, x, widened_bf16=False):
    a = np.ascontiguousarray(x, np.float32).reshape(1, k)
    return (orc.bf16_matmul_t(w, a) if widened_bf16 else orc.q4k_matmul_t(w, n, k, a)).reshape(-1)


def check_stages(orc, W, h0, got):
    """Each stage from the flow's own inputs; returns the worst error."""
    worst = 0.0
    h_in = h0
    for layer, widened in ((0, False), (1, True)):
        p = f"L{layer}."
        n1 = orc.rmsnorm(h_in, W[p + "g1"], EPS)
        for nm, n in (("q", H), ("k", NKV), ("v", NKV)):
            ref = mm(orc, W[p + nm], n, H, n1, widened and nm == "v")
            worst = max(worst, normwise_err(got[p + nm], ref))
        ref = h_in + mm(orc, W[p + "o"], H, H, got[p + "q"])
        worst = max(worst, normwise_err(got[p + "h1"], ref))
        n2 = orc.rmsnorm(got[p + "h1"], W[p + "g2"], EPS)
        for nm in ("gate", "up"):
            worst = max(worst, normwise_err(got[p + nm], mm(orc, W[p + nm], F, H, n2)))
        act = orc.swiglu(got[p + "gate"], got[p + "up"])
        ref = got[p + "h1"] + mm(orc, W[p + "down"], H, F, act, widened)
        worst = max(worst, normwise_err(got[p + "h2"], ref))
        h_in = got[p + "h2"]
    ref = mm(orc, W["lm"], V, H, orc.rmsnorm(h_in, W["gf"], EPS))
    worst = max(worst, normwise_err(got["logits"], ref))
    return worst


def chain(orc, W, h0):
    h = h0
    for layer, widened in ((0, False), (1, True)):
        p = f"L{layer}."
        q = mm(orc, W[p + "q"], H, H, orc.rmsnorm(h, W[p + "g1"], EPS))
        h1 = h + mm(orc, W[p + "o"], H, H, q)
        n2 = orc.rmsnorm(h1, W[p + "g2"], EPS)
        act = orc.swiglu(mm(orc, W[p + "gate"], F, H, n2), mm(orc, W[p + "up"], F, H, n2))
        h = h1 + mm(orc, W[p + "down"], H, F, act, widened)
    return mm(orc, W["lm"], V, H, orc.rmsnorm(h, W["gf"], EPS))


def test_flow_chain_parity_and_repeats(rt, orc):
    import torch
    rng = np.random.default_rng(5)
    vecs, stages, plains, W, h0 = build(rt, orc, rng)
    say(f"[flow] {len(stages)} stages, {len(vecs)} vectors")
    flow = rt.Flow(vecs, stages)
    runs = []
    for i in range(3):
        for t in plains.values():
            t.fill_(float("nan"))
        flow.run()
        flow.status()
        runs.append({nm: from_dev(t).copy() for nm, t in plains.items()})
        say(f"[flow] run {i} done")
    for r in runs[1:]:
        for nm in r:
            assert np.array_equal(r[nm].view(np.uint32), runs[0][nm].view(np.uint32)), nm
    got = runs[0]
    worst = check_stages(orc, W, h0, got)
    say(f"[flow] worst stage error {worst:.2e}")
    assert worst <= TOL
    e2e = normwise_err(got["logits"], chain(orc, W, h0))
    say(f"[flow] chain error {e2e:.2e}")
    assert e2e <= TOL
    flow.close()
    torch.cuda.synchronize()


def test_flow_graph_replay_reads_input_afresh(rt, orc):
    import torch
    rng = np.random.default_rng(6)
    vecs, stages, plains, W, h0 = build(rt, orc, rng)
    flow = rt.Flow(vecs, stages)
    h_dev = vecs[0][1]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        flow.run(stream=s)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        flow.run()
    for i in range(3):
        hx = rng.standard_normal(H).astype(np.float32)
        h_dev.copy_(torch.from_numpy(hx).cuda())
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        flow.status()
        graph_logits = from_dev(plains["logits"]).copy()
        flow.run()
        flow.status()
        eager_logits = from_dev(plains["logits"]).copy()
        assert np.array_equal(graph_logits.view(np.uint32), eager_logits.view(np.uint32)), i
        assert normwise_err(graph_logits, chain(orc, W, hx)) <= TOL, i
        say(f"[flow] replay {i} matches")
    del g
    flow.close()


def test_flow_create_errors(rt):
    import torch
    lib = rt.library()
    w = torch.zeros(1 << 20, dtype=torch.uint8, device="cuda")
    x = torch.zeros(512, device="cuda")
    vecs = [(512, x), (512, None), (512, None)]

    def stage(**kw):
        st = {"k": 512, "in0": 0, "jobs": [{"format": rt.Q4K, "w": w, "n": 512, "out": 1}]}
        st.update(kw)
        return st

    def code(vs, sts):
        try:
            rt.Flow(vs, sts).close()
            return 0
        except rt.RtHipError as e:
            return e.code

    assert code(vecs, [stage()]) == 0
    assert code(vecs, [stage(in0=2)]) == 1          # reads a vector no earlier stage wrote
    assert code(vecs, [stage(k=768)]) == 1          # in0 length differs from k
    assert code([(300, x), (512, None)], [stage(k=300)]) == 3  # Q4_K k % 256
    assert code(vecs, [stage(), stage()]) == 1      # vector 1 written twice
    assert code(vecs, [stage(jobs=[{"format": rt.BF16, "w": w, "n": 512, "out": 1},
                                   {"format": rt.BF16, "w": w, "n": 512, "out": 2}])]) == 1
    assert code(vecs, [stage(xop=rt.XOP_RMSNORM)]) == 1  # RMSNorm without gamma
    assert code(vecs, [stage(xop=3)]) == 1              # no such x operation
    assert code(vecs, [stage(act=2)]) == 1              # act needs a gate/up pair
    assert code(vecs, [stage(jobs=[{"format": rt.Q4K, "w": w, "n": 512, "out": 0}])]) == 1  # external out
    del lib
