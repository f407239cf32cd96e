"""Decode chain (rt_hip_chain_*): a sequence of dependent tiled-Q4_K GEMV
stages in one persistent launch.

Pinned by: every stage's output against the oracle's Q4KMat::matmul_t on
the same blocks and the same input (GEMV_TOL, as every M = 1 GEMV); stages
that read an earlier stage's output (the input the oracle gets is the
chain's own stored output, so a stale or partially written activation shows
up as a mismatch); a second run with a new first input; hipGraph replays
with eager work between them; and the argument checks.
"""
import numpy as np
import pytest

from helpers import GEMV_TOL, from_dev, normwise_err, say, to_dev


def _weights(orc, rng, n, k):
    return orc.q4k_quantize((rng.standard_normal((n, k)) * 0.02).astype(np.float32))


def _check(orc, blocks, n, k, x, y, what):
    ref = orc.q4k_matmul_t(blocks, n, k, np.asarray(x, np.float32).reshape(1, k))
    err = normwise_err(from_dev(y).reshape(1, n), ref)
    assert err <= GEMV_TOL, f"{what}: normwise error {err:.3e}"


@pytest.mark.gpu
def test_chain_independent_stages(rt, orc):
    """Stages with their own inputs: decode shapes, a ragged 4-job stage, and
    an output long enough to take two rounds per wave."""
    import torch
    rng = np.random.default_rng(5)
    specs = [([3072, 1024, 1024], 3072), ([3072], 3072), ([8192, 8192], 3072), ([3072], 8192),
             ([37, 130, 5, 16], 512), ([66000], 3072), ([100], 256)]
    stages, keep = [], []
    for ns, k in specs:
        x = rng.standard_normal((1, k)).astype(np.float32)
        bl = [_weights(orc, rng, n, k) for n in ns]
        tl = [rt.q4k_tile(to_dev(b), n, k) for b, n in zip(bl, ns)]
        ys = [torch.full((1, n), float("nan"), device="cuda") for n in ns]
        stages.append((to_dev(x), tl, ys, ns, k))
        keep.append((x, bl))
    say(f"[chain] {len(stages)} independent stages")
    ch = rt.Chain(stages)
    ch.run()
    torch.cuda.synchronize()
    assert ch.status() == 0
    for (x, bl), (_, _, ys, ns, k) in zip(keep, stages):
        for b, y, n in zip(bl, ys, ns):
            _check(orc, b, n, k, x, y, f"n={n} k={k}")
    # Same tile arithmetic as the per-launch kernel: agreement to f32 rounding.
    for (_, tl, ys, ns, k), (x, _) in zip(stages, keep):
        ref = rt.gemv_q4k_tiled_multi(tl, to_dev(x), ns, k)
        for a, b in zip(ys, ref):
            assert normwise_err(from_dev(a), from_dev(b)) <= 1e-6
    ch.close()


def _dataflow(rt, orc, rng):
    """x0 -> o-like (3072) -> gate/up (2 x 8192) -> down (3072, K = 8192) ->
    q/k/v (3 jobs) -> a 4-job stage on q's output: each stage reads the
    output of the one before."""
    import torch
    H, F = 3072, 8192
    x0 = torch.zeros((1, H), device="cuda")
    W = {}

    def tiles(name, n, k):
        b = _weights(orc, rng, n, k)
        W[name] = (b, n, k)
        return rt.q4k_tile(to_dev(b), n, k)

    out = {nm: torch.full((1, n), float("nan"), device="cuda")
           for nm, n in (("o", H), ("g", F), ("u", F), ("d", H), ("q", H), ("k", 1024), ("v", 1024),
                         ("a", 512), ("b", 256), ("c", 16), ("e", 2048))}
    stages = [
        (x0, [tiles("o", H, H)], [out["o"]], [H], H),
        (out["o"], [tiles("g", F, H), tiles("u", F, H)], [out["g"], out["u"]], [F, F], H),
        (out["g"], [tiles("d", H, F)], [out["d"]], [H], F),
        (out["d"], [tiles("q", H, H), tiles("k", 1024, H), tiles("v", 1024, H)],
         [out["q"], out["k"], out["v"]], [H, 1024, 1024], H),
        (out["q"], [tiles("a", 512, H), tiles("b", 256, H), tiles("c", 16, H), tiles("e", 2048, H)],
         [out["a"], out["b"], out["c"], out["e"]], [512, 256, 16, 2048], H),
    ]
    inputs = {"o": x0, "g": out["o"], "u": out["o"], "d": out["g"], "q": out["d"], "k": out["d"],
              "v": out["d"], "a": out["q"], "b": out["q"], "c": out["q"], "e": out["q"]}
    return rt.Chain(stages), x0, out, inputs, W


def _check_dataflow(orc, out, inputs, W, label):
    for nm, (b, n, k) in W.items():
        _check(orc, b, n, k, from_dev(inputs[nm]), out[nm], f"{label} stage {nm}")


@pytest.mark.gpu
def test_chain_dataflow_and_rerun(rt, orc):
    import torch
    rng = np.random.default_rng(9)
    ch, x0, out, inputs, W = _dataflow(rt, orc, rng)
    for run in range(2):
        say(f"[chain dataflow] run {run}")
        x0.copy_(to_dev(rng.standard_normal((1, 3072)).astype(np.float32)))
        for t in out.values():
            t.fill_(float("nan"))
        ch.run()
        torch.cuda.synchronize()
        assert ch.status() == 0
        _check_dataflow(orc, out, inputs, W, f"run {run}")
    ch.close()


@pytest.mark.gpu
def test_chain_graph_replays(rt, orc):
    """Captured once, replayed with a new first input each time (the barrier
    epochs advance on the device, so replays need no host update)."""
    import torch
    rng = np.random.default_rng(13)
    ch, x0, out, inputs, W = _dataflow(rt, orc, rng)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ch.run()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ch.run()
    for rep in range(3):
        say(f"[chain graph] replay {rep}")
        x0.copy_(to_dev(rng.standard_normal((1, 3072)).astype(np.float32)))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert ch.status() == 0
        _check_dataflow(orc, out, inputs, W, f"replay {rep}")
    ch.close()


@pytest.mark.gpu
def test_chain_rejects_bad_stages(rt):
    import ctypes as C

    import torch
    lib = rt.library()
    buf = torch.zeros(1 << 20, dtype=torch.uint8, device="cuda")
    x = torch.zeros(8192 * 2, device="cuda")
    y = torch.zeros(4096, device="cuda")

    def status(k=3072, count=1, n=16, xp=None):
        st = (rt.ChainStage * 1)()
        st[0].x = x.data_ptr() if xp is None else xp
        st[0].k, st[0].count = k, count
        for j in range(4):
            st[0].w[j], st[0].y[j], st[0].n[j] = buf.data_ptr(), y.data_ptr(), n
        h = C.c_void_p()
        rc = lib.lib.rt_hip_chain_create(st, 1, C.byref(h))
        if rc == 0:
            lib.call("rt_hip_chain_destroy", h)
        return rc

    assert status() == 0
    assert status(k=300) == 3          # RT_HIP_E_ALIGN
    assert status(k=8192 + 256) == 2   # RT_HIP_E_SHAPE
    assert status(count=5) == 1        # RT_HIP_E_ARG
    assert status(count=0) == 1
    assert status(n=0) == 2
    assert status(xp=x.data_ptr() + 4) == 3
