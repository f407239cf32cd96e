#!/usr/bin/env python3
"""bench.py -- rich-triplet's quantized-linear path on one MI355X.

Default workload: one Llama-3.2-3B decode step's linear
layers at batch 1 -- 28 layers x {q, k, v, o, gate, up, down} + lm_head =
197 GEMVs, in the model's order, captured once as a hipGraph and replayed
(the MI355X analogue of the reference's one-command-buffer decode step,
include/rt/metal_decode.hpp:10-20).  Weights follow the reference's Q4_K_M
semantics: Q4_K everywhere except v and down in layers
{0,1,2,5,8,11,14,17,20,23,24,25,26,27}, which are BF16 (Q6_K widened at
load, src/transformer4_load.cpp:141-143); the lm_head is Q4_K (requantized,
src/main.cpp:1047-1061).  Weights are random N(0, 0.02), quantized on the GPU
by the library's quantizer (byte-identical to Q4KMat::quantize); inputs are
N(0, 1).  Everything is resident in HBM before timing starts.

One JSON line on stdout; diagnostics on stderr.  Other BASELINE configs are
available with --workload (parity cases, not the headline line).
"""
from __future__ import annotations

import argparse
import importlib.util
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
F32_PEAK_TFLOPS = 157.3
WIDENED_LAYERS = {0, 1, 2, 5, 8, 11, 14, 17, 20, 23, 24, 25, 26, 27}
# --mix q4km_q6k: the widened layers' down projection kept as native Q6_K
# (rt_hip_gemv_q6k_tiled) instead of its BF16-widened copy
Q6K_NATIVE = "q6k"
HIDDEN, KV, FFN, VOCAB, LAYERS = 3072, 1024, 8192, 128256, 28
# HBM bytes per launch of the dominant kernel (fused gate+up, tiled layout)
# come from the committed counter profile of this build (rocprofv3
# FETCH_SIZE / WRITE_SIZE scaled by a 1 GiB device copy; the command is in
# the file): the table row marked "(dominant)".
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "decode_kernels_hbm_traffic.md")


def dominant_traffic_bytes(layout: str):
    """The '(dominant)' row's scaled HBM bytes in TRAFFIC_PROFILE (tiled
    layout only; the row-major layout has no measured figure)."""
    if layout != "tiled" or not os.path.exists(TRAFFIC_PROFILE):
        return None
    col = None
    with open(TRAFFIC_PROFILE) as f:
        for row in f:
            if not row.startswith("|"):
                continue
            cells = [c.strip() for c in row.strip().strip("|").split("|")]
            if col is None and "HBM bytes (scaled)" in cells:
                col = cells.index("HBM bytes (scaled)")
            elif col is not None and "(dominant)" in row:
                return int(cells[col].replace(",", ""))
    return None


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def load_rt():
    name = "rich_triplet_cpp_amd"
    path = os.path.join(ROOT, "rich-triplet-cpp_amd", "__init__.py")
    spec = importlib.util.spec_from_file_location(name, path,
                                                  submodule_search_locations=[os.path.dirname(path)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod.rt_hip


def q4k_bytes(n, k):
    return n * (k // 256) * 144


def weight_bytes(fmt, n, k, rt):
    if fmt == Q6K_NATIVE:
        return n * (k // 256) * 210
    if fmt == rt.Q4K:
        return q4k_bytes(n, k)
    if fmt == rt.Q4_0:
        return n * (k // 32) * 18
    return n * k * 2


def q4_0_blocks(torch, w):
    """GGUF Q4_0 blocks of w [n, k] on the GPU: per 32 values d = absmax/7
    (rounded to f16), q = clamp(round(v/d), -8, 7) + 8, value j < 16 in the
    low nibble of qs[j] and value j + 16 in its high nibble (the layout
    decoded at src/gguf.cpp:495-529).  Synthetic data only."""
    n, k = w.shape
    b = w.reshape(n, k // 32, 32)
    d = (b.abs().amax(dim=-1) / 7.0).half()
    df = d.float()
    q = torch.where(df[..., None] > 0, torch.round(b / df[..., None].clamp_min(1e-30)),
                    torch.zeros_like(b)).clamp(-8, 7).to(torch.int32) + 8
    qs = (q[..., :16] | (q[..., 16:] << 4)).to(torch.uint8)
    out = torch.empty((n, k // 32, 18), dtype=torch.uint8, device=w.device)
    out[..., 0:2] = d.view(torch.uint8).reshape(n, k // 32, 2)
    out[..., 2:] = qs
    return out.reshape(-1)


# --------------------------------------------------------------- config 3 --

def q6k_tiled_synthetic(rt, torch, g, n, k):
    """Synthetic Q6_K blocks (random quants and scales, d = 2^-7), tiled once
    at load as the native GEMV reads them."""
    b = torch.randint(0, 256, (n * (k // 256), 210), dtype=torch.uint8, device="cuda", generator=g)
    b[:, 208] = 0x00
    b[:, 209] = 0x20
    return rt.q6k_tile(b.reshape(-1), n, k)


class DecodeModel:
    """Synthetic Llama-3.2-3B linear weights and per-GEMV inputs on the GPU."""

    def __init__(self, rt, torch, mix: str, layout: str = "tiled", seed: int = 0):
        self.rt, self.torch = rt, torch
        self.layout = layout
        g = torch.Generator(device="cuda").manual_seed(seed)
        self.gemvs = []  # (name, fmt, w, x, y, n, k)
        dev = "cuda"

        def make(n, k, fmt):
            if fmt == Q6K_NATIVE:
                return q6k_tiled_synthetic(rt, torch, g, n, k)
            w = torch.randn((n, k), generator=g, device=dev) * 0.02
            if fmt == rt.Q4K:
                out = rt.quantize_q4k(w)
            else:
                out = w.to(torch.bfloat16).view(torch.int16)  # RNE, as f32_to_bf16
            del w
            return out

        for layer in range(LAYERS):
            wide = mix in ("q4km", "q4km_q6k") and layer in WIDENED_LAYERS
            x_attn = torch.randn((1, HIDDEN), generator=g, device=dev)
            x_o = torch.randn((1, HIDDEN), generator=g, device=dev)
            x_mlp = torch.randn((1, HIDDEN), generator=g, device=dev)
            x_down = torch.randn((1, FFN), generator=g, device=dev)
            specs = [("q", HIDDEN, HIDDEN, rt.Q4K, x_attn),
                     ("k", KV, HIDDEN, rt.Q4K, x_attn),
                     ("v", KV, HIDDEN, rt.BF16 if wide else rt.Q4K, x_attn),
                     ("o", HIDDEN, HIDDEN, rt.Q4K, x_o),
                     ("gate", FFN, HIDDEN, rt.Q4K, x_mlp),
                     ("up", FFN, HIDDEN, rt.Q4K, x_mlp),
                     ("down", HIDDEN, FFN, (Q6K_NATIVE if mix == "q4km_q6k" else rt.BF16) if wide else rt.Q4K,
                      x_down)]
            for name, n, k, fmt, x in specs:
                w = make(n, k, fmt)
                y = torch.empty((1, n), device=dev)
                self.gemvs.append((f"L{layer}.{name}", fmt, w, x, y, n, k))
        x_f = torch.randn((1, HIDDEN), generator=g, device=dev)
        self.gemvs.append(("lm_head", rt.Q4K, make(VOCAB, HIDDEN, rt.Q4K), x_f,
                           torch.empty((1, VOCAB), device=dev), VOCAB, HIDDEN))
        # Tiled copies of the Q4_K weights (a one-time load-time repack; the
        # row-major blocks stay for the CPU baseline, which needs the
        # reference's layout).  Only the copies the plan uses are read per token.
        self.tiled = {}
        if layout == "tiled":
            for name, fmt, w, _, _, n, k in self.gemvs:
                if fmt == rt.Q4K:
                    self.tiled[name] = rt.q4k_tile(w, n, k)
        self.plan = self.launches()
        torch.cuda.synchronize()

    def q4k_multi(self, item):
        if self.layout == "tiled":
            self.rt.gemv_q4k_tiled_multi([self.tiled[gv[0]] for gv in item], item[0][3],
                                         [gv[5] for gv in item], item[0][6], ys=[gv[4] for gv in item])
        else:
            self.rt.gemv_q4k_multi([gv[2] for gv in item], item[0][3], [gv[5] for gv in item],
                                   item[0][6], ys=[gv[4] for gv in item])

    def one(self, gv):
        name, fmt, w, x, y, n, k = gv
        if fmt == Q6K_NATIVE:
            self.rt.gemv_q6k_tiled(w, x, n, k, y=y)
        elif fmt == self.rt.Q4K and self.layout == "tiled":
            self.rt.gemv_q4k_tiled(self.tiled[name], x, n, k, y=y)
        else:
            self.rt.gemv(fmt, w, x, n, k, y=y)

    def bytes_per_token(self) -> int:
        return sum(weight_bytes(f, n, k, self.rt) + 4 * k + 4 * n
                   for _, f, _, _, _, n, k in self.gemvs)

    def launches(self):
        """The step as launches in model order.  GEMVs that read the same
        activation run as one launch: the Q4_K ones as one multi-job launch
        (q/k/v, gate/up), and with the tiled layout a BF16-widened v joins
        its layer's q/k launch (rt_hip_gemv_q4k_tiled_bf16)."""
        out = []
        by = {gv[0]: gv for gv in self.gemvs}
        for layer in range(LAYERS):
            groups = [["q", "k", "v"], ["o"], ["gate", "up"], ["down"]]
            for grp in groups:
                gvs = [by[f"L{layer}.{nm}"] for nm in grp]
                q4 = [gv for gv in gvs if gv[1] == self.rt.Q4K]
                rest = [gv for gv in gvs if gv[1] != self.rt.Q4K]
                if self.layout == "tiled" and q4 and len(rest) == 1 and rest[0][1] == self.rt.BF16:
                    out.append(("fused", (q4, rest[0])))
                    continue
                if len(q4) > 1:
                    out.append(("multi", q4))
                elif q4:
                    out.append(("one", q4[0]))
                for gv in rest:
                    out.append(("one", gv))
        out.append(("one", by["lm_head"]))
        return out

    def fused(self, item):
        q4, (_, _, wb, x, yb, nb, k) = item
        self.rt.gemv_q4k_tiled_bf16([self.tiled[gv[0]] for gv in q4], [gv[5] for gv in q4], wb, nb, x, k,
                                    ys=[gv[4] for gv in q4], yb=yb)

    def step(self):
        for kind, item in self.plan:
            if kind == "multi":
                self.q4k_multi(item)
            elif kind == "fused":
                self.fused(item)
            else:
                self.one(item)

    def step_unfused(self):
        for gv in self.gemvs:
            self.one(gv)


def time_graph(torch, fn, warmup: int, steps: int):
    """Capture fn once as a graph; replay `warmup` times, then time `steps`."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()  # eager warm-up outside capture (first-call setup)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn()
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps, graph


def dominant_kernel_roofline(rt, torch, model, reps: int = 5):
    """The launch that moves the most bytes per token: the fused gate+up
    Q4_K GEMV (2 x 8192 x 3072, one multi-job launch per layer).  All 28 of
    the token's gate+up launches (795 MB of distinct weights, beyond the
    256 MB MALL) are replayed back to back on one stream, bracketed by HIP
    events recorded on that stream; the figure is their average duration."""
    sel = [item for kind, item in model.plan
           if kind == "multi" and item[0][0].endswith(".gate")]

    def run():
        for item in sel:
            model.q4k_multi(item)

    ms, _ = time_graph(torch, run, 2, reps)
    per_launch_us = ms * 1e3 / len(sel)
    algo = 2 * q4k_bytes(FFN, HIDDEN) + 4 * HIDDEN + 4 * 2 * FFN
    achieved = algo / (per_launch_us * 1e-6) / 1e9
    return {"kernel": f"k_gemv_q4k_mfma (fused gate+up Q4_K GEMV, 2 x 8192 x 3072, {model.layout})",
            "bytes_per_launch": algo, "us_per_launch": per_launch_us,
            "achieved_gbs": achieved}


def cpu_baseline(rt, torch, model, budget_s: float = 12.0):
    """The reference's own CPU GEMVs (oracle/_ref: Q4KMat::matmul_q4k_t ->
    gemv_mt, MatBf16::matmul_by_t -> gemv_mt, x86 scalar dot_row) over the
    whole decode step: all 197 GEMVs of the token, in order, timed in full
    (median of at least 5 reps after one warm-up, more until ~budget_s)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np
    from oracle import Oracle, Reference, reference_available  # noqa: PLC0415

    kind = "reference" if reference_available() else "port"
    sample = list(model.gemvs)
    host = []
    for name, fmt, w, x, y, n, k in sample:
        wh = w.cpu().numpy()
        xh = x.cpu().numpy().astype(np.float32)
        host.append((name, fmt, wh if fmt == rt.Q4K else wh.view(np.uint16).reshape(n, k), xh, n, k))
    nbytes = sum(weight_bytes(f, n, k, rt) + 4 * k + 4 * n for _, f, _, _, n, k in host)
    if kind == "reference":
        ref = Reference()
        threads = ref.hardware_threads()
        handles = []
        for name, fmt, wh, xh, n, k in host:
            h = ref.q4k_new(wh, n, k) if fmt == rt.Q4K else ref.bf16_new(wh, n, k)
            handles.append((fmt, h, xh, n))

        def once():
            for fmt, h, xh, n in handles:
                y = np.empty((1, n), np.float32)
                (ref.q4k_handle_matmul_t if fmt == rt.Q4K else ref.bf16_handle_matmul_t)(h, xh, 1, y)
    else:
        orc = Oracle()
        threads = orc.hardware_threads()

        def once():
            for name, fmt, wh, xh, n, k in host:
                if fmt == rt.Q4K:
                    orc.q4k_matmul_t(wh, n, k, xh)
                else:
                    orc.bf16_matmul_t(wh, xh)
    once()  # warm-up
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < 5 or (time.perf_counter() < t_end and len(times) < 50):
        t0 = time.perf_counter()
        once()
        times.append(time.perf_counter() - t0)
    if kind == "reference":
        for fmt, h, _, _ in handles:
            (ref.q4k_delete if fmt == rt.Q4K else ref.bf16_delete)(h)
    med = sorted(times)[len(times) // 2]
    gbs = nbytes / med / 1e9
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": threads, "kind": kind,
            "sample": (f"the whole decode step, timed in full: all {len(host)} GEMVs, "
                       f"{nbytes / 1e6:.1f} MB, median of {len(times)} reps ({med * 1e3:.1f} ms per token); "
                       f"x86 scalar dot_row, gemv_mt threads = min(hw={threads}, N/128)"),
            "us_per_token": round(med * 1e6, 1)}


def bench_decode(args, rt, torch):
    model = DecodeModel(rt, torch, args.mix, args.layout)
    nbytes = model.bytes_per_token()
    log(f"[bench] {len(model.gemvs)} GEMVs in {len(model.plan)} launches, "
        f"{nbytes / 1e9:.3f} GB/token ({args.mix})")
    if args.unfused:
        ms_u, _ = time_graph(torch, model.step_unfused, args.warmup, args.steps)
        log(f"[bench] unfused (one launch per GEMV): {ms_u * 1e3:.1f} us/token")
    ms, _ = time_graph(torch, model.step, args.warmup, args.steps)
    us = ms * 1e3
    gbs = nbytes / (us * 1e-6) / 1e9
    log(f"[bench] {us:.1f} us/token, {gbs:.1f} GB/s ({100 * gbs / HBM_PEAK_GBS:.1f}% of 8 TB/s)")
    dom = dominant_kernel_roofline(rt, torch, model)
    log(f"[bench] dominant kernel: {dom}")
    roof = {"bound": "hbm", "achieved": round(dom["achieved_gbs"], 1), "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": round(dom["achieved_gbs"] / HBM_PEAK_GBS, 4),
            "traffic": (args.traffic_bytes if args.traffic_bytes is not None
                        else dominant_traffic_bytes(args.layout)), "kernel": dom["kernel"],
            "us_per_launch": round(dom["us_per_launch"], 3),
            "bytes_per_launch": dom["bytes_per_launch"]}
    # the native-Q6_K variant has the headline's CPU path (the reference
    # widens Q6_K to BF16 at load): its baseline is the q4km line's
    cpu = None if args.no_cpu_baseline or args.mix == "q4km_q6k" else cpu_baseline(rt, torch, model)
    if cpu:
        log(f"[bench] cpu baseline: {cpu}")
    return {
        "metric": "Q4_K GEMV achieved HBM GB/s (% peak) + us/token all-layer GEMVs @ Llama-3.2-3B",
        "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "q4_k/bf16 weights, f32 activations",
        "data": "synthetic: random N(0,0.02) weights quantized on GPU, N(0,1) inputs",
        "config": {"workload": "llama-3.2-3b decode step, all 28 layers' GEMVs + lm_head, batch 1",
                   "weights": {"q4km": "Q4_K_M mix",
                               "q4km_q6k": "Q4_K_M mix, Q6_K down projections kept native (not widened)",
                               "q4k": "pure Q4_K"}[args.mix],
                   "gemvs_per_token": len(model.gemvs), "bytes_per_token": nbytes,
                   "us_per_token": round(us, 2), "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
                   "launches_per_token": len(model.plan),
                   "launch": "one hipGraph per token; q/k/v (BF16 v included) and gate/up fused per layer",
                   "q4k_layout": ("tiled (rt_hip_q4k_tile once at load; bit-identical results)"
                                  if args.layout == "tiled" else "reference row-major blocks")},
        "roofline": roof, "cpu_baseline": cpu,
    }


# ------------------------------------- layer operations fused into the GEMVs --

def bench_layer_ops(args, rt, torch):
    """28 Llama-3.2-3B layers' linear work with the operations that feed the
    projections: RMSNorm before q/k/v and before gate/up, SwiGLU before
    down, a final RMSNorm before the lm_head.  Weights follow --mix (the
    Q4_K_M mix widens v and down to BF16 in the same 14 layers as the decode
    bench).  Fused: the norms and the SwiGLU run inside the GEMV launches (4
    launches per layer).  Separate: the same operations as torch kernels
    between the same GEMVs (rms_norm, silu, mul).  Attention and the residual
    adds are outside both.  Synthetic weights and inputs; the gate/up
    outputs feed down."""
    g = torch.Generator(device="cuda").manual_seed(0)
    dev = "cuda"

    def tiled(n, k):
        w = torch.randn((n, k), generator=g, device=dev) * 0.02
        return rt.q4k_tile(rt.quantize_q4k(w), n, k)

    def bf16(n, k):
        return (torch.randn((n, k), generator=g, device=dev) * 0.02).to(torch.bfloat16).view(torch.int16)

    layers = []
    for layer in range(LAYERS):
        wide = args.mix in ("q4km", "q4km_q6k") and layer in WIDENED_LAYERS
        q6 = wide and args.mix == "q4km_q6k"
        L = {"wide": wide, "q6": q6, "qk": [tiled(HIDDEN, HIDDEN), tiled(KV, HIDDEN)],
             "v": bf16(KV, HIDDEN) if wide else tiled(KV, HIDDEN), "o": tiled(HIDDEN, HIDDEN),
             "gu": [tiled(FFN, HIDDEN), tiled(FFN, HIDDEN)],
             "down": (q6k_tiled_synthetic(rt, torch, g, HIDDEN, FFN) if q6 else bf16(HIDDEN, FFN)) if wide
             else tiled(HIDDEN, FFN),
             "x": torch.randn((1, HIDDEN), generator=g, device=dev),
             "x_o": torch.randn((1, HIDDEN), generator=g, device=dev),
             "g1": 1.0 + 0.1 * torch.randn((HIDDEN,), generator=g, device=dev),
             "g2": 1.0 + 0.1 * torch.randn((HIDDEN,), generator=g, device=dev)}
        L["y_qkv"] = [torch.empty((1, n), device=dev) for n in (HIDDEN, KV, KV)]
        L["y_o"] = torch.empty((1, HIDDEN), device=dev)
        L["y_gu"] = [torch.empty((1, FFN), device=dev) for _ in range(2)]
        L["y_d"] = torch.empty((1, HIDDEN), device=dev)
        layers.append(L)
    head = {"w": tiled(VOCAB, HIDDEN), "x": torch.randn((1, HIDDEN), generator=g, device=dev),
            "g": 1.0 + 0.1 * torch.randn((HIDDEN,), generator=g, device=dev),
            "y": torch.empty((1, VOCAB), device=dev)}
    eps = 1e-5
    F = torch.nn.functional

    def fused():
        for L in layers:
            if L["wide"]:
                rt.gemv_q4k_tiled_bf16_rmsnorm(L["qk"], [HIDDEN, KV], L["v"], KV, L["x"], L["g1"], eps, HIDDEN,
                                               ys=L["y_qkv"][:2], yb=L["y_qkv"][2])
            else:
                rt.gemv_q4k_tiled_rmsnorm_multi(L["qk"] + [L["v"]], L["x"], L["g1"], eps, [HIDDEN, KV, KV],
                                                HIDDEN, ys=L["y_qkv"])
            rt.gemv_q4k_tiled(L["o"], L["x_o"], HIDDEN, HIDDEN, y=L["y_o"])
            rt.gemv_q4k_tiled_rmsnorm_multi(L["gu"], L["x"], L["g2"], eps, [FFN, FFN], HIDDEN, ys=L["y_gu"])
            if L["q6"]:  # the native Q6_K down with its residual add (y_d is the residual here)
                rt.gemv_swiglu_residual(None, L["down"], L["y_gu"][0], L["y_gu"][1], L["y_d"], HIDDEN, FFN,
                                        q6k=True)
            elif L["wide"]:
                rt.gemv_bf16_swiglu(L["down"], L["y_gu"][0], L["y_gu"][1], HIDDEN, FFN, y=L["y_d"])
            else:
                rt.gemv_q4k_tiled_swiglu(L["down"], L["y_gu"][0], L["y_gu"][1], HIDDEN, FFN, y=L["y_d"])
        rt.gemv_q4k_tiled_rmsnorm_multi([head["w"]], head["x"], head["g"], eps, [VOCAB], HIDDEN, ys=[head["y"]])

    def separate():
        for L in layers:
            xn = F.rms_norm(L["x"], (HIDDEN,), L["g1"], eps)
            if L["wide"]:
                rt.gemv_q4k_tiled_bf16(L["qk"], [HIDDEN, KV], L["v"], KV, xn, HIDDEN, ys=L["y_qkv"][:2],
                                       yb=L["y_qkv"][2])
            else:
                rt.gemv_q4k_tiled_multi(L["qk"] + [L["v"]], xn, [HIDDEN, KV, KV], HIDDEN, ys=L["y_qkv"])
            rt.gemv_q4k_tiled(L["o"], L["x_o"], HIDDEN, HIDDEN, y=L["y_o"])
            xn = F.rms_norm(L["x"], (HIDDEN,), L["g2"], eps)
            rt.gemv_q4k_tiled_multi(L["gu"], xn, [FFN, FFN], HIDDEN, ys=L["y_gu"])
            act = F.silu(L["y_gu"][0]) * L["y_gu"][1]
            if L["q6"]:
                rt.gemv_q6k_tiled(L["down"], act, HIDDEN, FFN, y=L["y_d"])
            elif L["wide"]:
                rt.gemv(rt.BF16, L["down"], act, HIDDEN, FFN, y=L["y_d"])
            else:
                rt.gemv_q4k_tiled(L["down"], act, HIDDEN, FFN, y=L["y_d"])
        xn = F.rms_norm(head["x"], (HIDDEN,), head["g"], eps)
        rt.gemv_q4k_tiled(head["w"], xn, VOCAB, HIDDEN, y=head["y"])

    ms_f, _ = time_graph(torch, fused, args.warmup, args.steps)
    ms_s, _ = time_graph(torch, separate, args.warmup, args.steps)
    log(f"[bench] layer ops fused ({args.mix}): {ms_f * 1e3:.1f} us/token; "
        f"separate torch kernels: {ms_s * 1e3:.1f} us/token")
    return {"metric": "Llama-3.2-3B linear work + RMSNorm/SwiGLU per token, fused into the GEMVs",
            "value": round(ms_f * 1e3, 2), "unit": "us/token", "higher_is_better": False,
            "separate_us_per_token": round(ms_s * 1e3, 2), "steps": args.steps, "warmup": args.warmup,
            "weights": {"q4km": "Q4_K_M mix",
                        "q4km_q6k": "Q4_K_M mix, Q6_K down projections kept native (fused SwiGLU + residual add)",
                        "q4k": "pure Q4_K"}[args.mix],
            "launches_per_token_fused": 4 * LAYERS + 1,
            "separate": "the same GEMVs with torch's rms_norm, silu and mul kernels between them",
            "data": "synthetic"}


# ------------------------------------------------- one decode token, fused --

def bench_decode_layers(args, rt, torch):
    """One Llama-3.2-3B decode token through every operation of the layers
    except the embedding lookup, pure Q4_K weights, at --context cached
    positions: per layer RMSNorm + q/k/v + RoPE + KV append (one launch),
    attention over the cache (two), o + residual (one), RMSNorm + gate/up
    (one), SwiGLU + down + residual (one); then the final RMSNorm + lm_head.
    The KV caches hold random keys and values for positions < context; the
    token is written at position context.  Synthetic weights and inputs."""
    g = torch.Generator(device="cuda").manual_seed(0)
    dev = "cuda"
    ctx = args.context
    nq, nkv, hd = 24, 8, 128

    def tiled(n, k):
        w = torch.randn((n, k), generator=g, device=dev) * 0.02
        return rt.q4k_tile(rt.quantize_q4k(w), n, k)

    layers = []
    for _ in range(LAYERS):
        L = {"qkv": [tiled(HIDDEN, HIDDEN), tiled(KV, HIDDEN), tiled(KV, HIDDEN)], "o": tiled(HIDDEN, HIDDEN),
             "gu": [tiled(FFN, HIDDEN), tiled(FFN, HIDDEN)], "down": tiled(HIDDEN, FFN),
             "g1": 1.0 + 0.1 * torch.randn((HIDDEN,), generator=g, device=dev),
             "g2": 1.0 + 0.1 * torch.randn((HIDDEN,), generator=g, device=dev),
             "kc": torch.randn((ctx + 1, KV), generator=g, device=dev),
             "vc": torch.randn((ctx + 1, KV), generator=g, device=dev)}
        layers.append(L)
    head = tiled(VOCAB, HIDDEN)
    gf = 1.0 + 0.1 * torch.randn((HIDDEN,), generator=g, device=dev)
    resid = torch.randn((1, HIDDEN), generator=g, device=dev)
    q = torch.empty((1, HIDDEN), device=dev)
    attn = torch.empty((1, HIDDEN), device=dev)
    gate, up = torch.empty((1, FFN), device=dev), torch.empty((1, FFN), device=dev)
    logits = torch.empty((1, VOCAB), device=dev)
    # Config5::inv_freq (transformer5.cpp:36-52), rope_theta 500000
    inv = torch.tensor([1.0 / (500000.0 ** (2.0 * i / hd)) for i in range(hd // 2)], dtype=torch.float32, device=dev)
    eps, scale = 1e-5, float(1.0 / (hd ** 0.5))

    def step():
        for L in layers:
            rt.gemv_q4k_tiled_rmsnorm_rope(L["qkv"], resid, L["g1"], eps, [HIDDEN, KV, KV], HIDDEN, inv, ctx, hd, 0x3,
                                           ys=[q, L["kc"][ctx:ctx + 1], L["vc"][ctx:ctx + 1]])
            rt.attention_decode(q, L["kc"], L["vc"], ctx + 1, nq, nkv, scale, out=attn)
            rt.gemv_q4k_tiled_residual(L["o"], attn, resid, HIDDEN, HIDDEN)
            rt.gemv_q4k_tiled_rmsnorm_multi(L["gu"], resid, L["g2"], eps, [FFN, FFN], HIDDEN, ys=[gate, up])
            rt.gemv_swiglu_residual(rt.Q4K, L["down"], gate, up, resid, HIDDEN, FFN)
        rt.gemv_q4k_tiled_rmsnorm_multi([head], resid, gf, eps, [VOCAB], HIDDEN, ys=[logits])

    def attention_only():
        for L in layers:
            rt.attention_decode(q, L["kc"], L["vc"], ctx + 1, nq, nkv, scale, out=attn)

    ms, _ = time_graph(torch, step, args.warmup, args.steps)
    ms_a, _ = time_graph(torch, attention_only, args.warmup, args.steps)
    kv_bytes = LAYERS * 2 * (ctx + 1) * KV * 4
    log(f"[bench] decode token (fused layers, context {ctx}): {ms * 1e3:.1f} us/token; "
        f"attention alone {ms_a * 1e3:.1f} us ({kv_bytes / (ms_a * 1e-3) / 1e9:.0f} GB/s of KV cache)")
    return {"metric": "Llama-3.2-3B decode token through every layer operation (pure Q4_K), fused engine path",
            "value": round(ms * 1e3, 2), "unit": "us/token", "higher_is_better": False, "context": ctx,
            "attention_us_per_token": round(ms_a * 1e3, 2),
            "attention_kv_gbs": round(kv_bytes / (ms_a * 1e-3) / 1e9, 1),
            "launches_per_token": 6 * LAYERS + 1, "steps": args.steps, "warmup": args.warmup,
            "data": "synthetic"}


# ------------------------------------------------------------ decode engine --

ENGINE_MODELS = {
    # Llama-3.2-3B: the headline shapes, Q4_K_M mix (v and down BF16 in the
    # widened layers), Q4_K lm_head, f32 KV cache
    "llama3b": dict(arch=0, n_layers=LAYERS, hidden=HIDDEN, n_heads=24, n_kv_heads=8, head_dim=128, ffn=FFN,
                    vocab=VOCAB, norm_eps=1e-5, rope_theta=500000.0, rope_theta_local=0.0, rope_freq_scale=1.0,
                    rope_freq_scale_local=1.0, rope_half=0, sliding_window=0, global_every=0, attn_scale=0.0,
                    embed_scale=0.0, kv_f16=0, max_batch=0),
    # Gemma-3-4B shapes (Config4::gemma3_4b): 34 layers, hidden 2560, 8 q / 4 kv
    # heads of 256, ffn 10240, vocab 262144, window 1024 on 5 of every 6
    # layers, f16 KV cache, tied bf16 lm_head; projections Q4_K
    "gemma3_4b": dict(arch=1, n_layers=34, hidden=2560, n_heads=8, n_kv_heads=4, head_dim=256, ffn=10240,
                      vocab=262144, norm_eps=1e-6, rope_theta=1e6, rope_theta_local=1e4, rope_freq_scale=0.125,
                      rope_freq_scale_local=1.0, rope_half=1, sliding_window=1024, global_every=6,
                      attn_scale=1.0 / 16.0, embed_scale=float(2560 ** 0.5), kv_f16=1, max_batch=0),
}


def bench_engine(args, rt, torch, model: str):
    """A whole decode token through the decode engine (rt_hip_decoder_step):
    embedding, every layer, final norm, lm_head and the argmax, replayed as
    one captured graph per token; the context is filled with random keys and
    values up to --context, and the timed steps run at positions
    context, context + 1, ...  Synthetic weights (quantized on the GPU by the
    library's quantizer).  Value: GEMV weight bytes per token / time."""
    import numpy as np
    cfg = dict(ENGINE_MODELS[model])
    ctx = args.context
    cfg["max_seq"] = ctx + args.warmup + args.steps + 1
    q6_down = args.mix == "q4km_q6k" and cfg["arch"] != 1
    if q6_down:
        cfg["max_batch"] = 0  # a Q6_K down is single-token only
    dec = rt.Decoder(**cfg)
    g = torch.Generator(device="cuda").manual_seed(0)
    H, F, nq, nkv, d, V, L = (cfg[k] for k in ("hidden", "ffn", "n_heads", "n_kv_heads", "head_dim", "vocab",
                                             "n_layers"))
    gemma = cfg["arch"] == 1
    wbytes = 0

    def q4(n, k):
        w = torch.randn((n, k), generator=g, device="cuda") * 0.02
        return rt.quantize_q4k(w).cpu().numpy()

    def bf(n, k, std=0.02):
        return (torch.randn((n, k), generator=g, device="cuda") * std).to(torch.bfloat16).view(torch.int16).cpu().numpy()

    def norm(n):
        base = 0.0 if gemma else 1.0
        return (base + 0.1 * torch.randn((n,), generator=g, device="cuda")).cpu().numpy()

    for li in range(L):
        wide = (not gemma) and li in WIDENED_LAYERS
        for name, t, n, k, use_bf in [("q", rt.T_Q, nq * d, H, False), ("k", rt.T_K, nkv * d, H, False),
                                      ("v", rt.T_V, nkv * d, H, wide), ("o", rt.T_O, H, nq * d, False),
                                      ("gate", rt.T_GATE, F, H, False), ("up", rt.T_UP, F, H, False),
                                      ("down", rt.T_DOWN, H, F, wide)]:
            if use_bf and q6_down and name == "down":
                # GGUF Q6_K bytes kept native: random quants and scales, d = 2^-14
                arr = torch.randint(0, 256, (n * (k // 256), 210), dtype=torch.uint8, generator=g,
                                    device="cuda").cpu().numpy()
                arr[:, 208], arr[:, 209] = 0x00, 0x04
                dec.set(li, t, rt.Q6K, arr)
            else:
                arr = bf(n, k) if use_bf else q4(n, k)
                dec.set(li, t, rt.BF16 if use_bf else rt.Q4K, arr)
            wbytes += arr.nbytes
        dec.set(li, rt.T_ATTN_NORM, rt.F32, norm(H))
        dec.set(li, rt.T_FFN_NORM, rt.F32, norm(H))
        if gemma:
            for t in (rt.T_POST_ATTN_NORM, rt.T_POST_FFN_NORM):
                dec.set(li, t, rt.F32, norm(H))
            dec.set(li, rt.T_Q_NORM, rt.F32, norm(d))
            dec.set(li, rt.T_K_NORM, rt.F32, norm(d))
        if ctx:
            kv = torch.randn((2, ctx, nkv * d), generator=g, device="cuda").cpu().numpy()
            dec.set_kv(li, kv[0], kv[1], ctx)
    emb = bf(V, H, 0.5)
    dec.set(-1, rt.T_EMBED, rt.BF16, emb)
    dec.set(-1, rt.T_OUTPUT_NORM, rt.F32, norm(H))
    head = emb if gemma else q4(V, H)
    dec.set(-1, rt.T_LM_HEAD, rt.BF16 if gemma else rt.Q4K, head)
    wbytes += head.nbytes
    del emb, head
    log(f"[bench] engine {model}: {L} layers, {wbytes / 1e9:.3f} GB of GEMV weights per token, context {ctx}")
    tokens = np.random.default_rng(0).integers(0, V, args.warmup + args.steps)
    pos = ctx
    for i in range(args.warmup):
        dec.step(int(tokens[i]), pos, argmax=True)
        pos += 1
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        dec.step(int(tokens[args.warmup + i]), pos, argmax=True)
        pos += 1
    wall = (time.perf_counter() - t0) / args.steps
    us = wall * 1e6
    gbs = wbytes / wall / 1e9
    log(f"[bench] engine {model}: {us:.1f} us/token (synchronous steps, logits and argmax to the host), "
        f"{gbs:.1f} GB/s of weights")
    dec.close()
    return line(args, f"decode engine whole-token latency, {model}", round(us, 2), "us/token", wall * 1e3, False,
                "q4_k/bf16 weights, f32 activations, " + ("f16" if cfg["kv_f16"] else "f32") + " KV cache",
                {"workload": f"decode engine (rt_hip_decoder_step), {model}, context {ctx}"
                             + (", Q6_K down projections kept native" if q6_down else ""),
                 "gemv_weight_bytes_per_token": wbytes, "weight_gbs": round(gbs, 1),
                 "includes": "embedding, all layers (norms, q/k/v, RoPE, KV append, attention, o, MLP), final "
                             "norm, lm_head, argmax, the position upload and the host synchronisation"},
                None, None)


# ------------------------------------------------------ other BASELINE configs --

def _cpu_timed(fn, budget_s: float, min_reps: int = 3, max_reps: int = 50):
    """Median wall time of fn() after one warm-up, repeated until budget_s."""
    fn()
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < min_reps or (time.perf_counter() < t_end and len(times) < max_reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return sorted(times)[len(times) // 2], len(times)


def _cpu_handles():
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    from oracle import Oracle, Reference, reference_available  # noqa: PLC0415
    if reference_available():
        ref = Reference()
        return "reference", ref, ref.hardware_threads(), Oracle()
    orc = Oracle()
    return "port", orc, orc.hardware_threads(), orc


def line(args, metric, value, unit, ms, higher, dtype, config, roofline, cpu, data=None):
    return {"metric": metric, "value": value, "unit": unit, "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(ms, 5), "higher_is_better": higher, "scaling": "weak",
            "vs_baseline": None, "dtype": dtype,
            "data": data or "synthetic: random N(0,0.02) weights quantized on GPU, N(0,1) inputs",
            "config": config, "roofline": roofline, "cpu_baseline": cpu}


def bench_single_gemv(args, rt, torch, fmt, n, k, label, workload, copies_bytes=768 << 20, argmax=False):
    """One GEMV shape (2a, 2b), rotating through enough
    distinct weight copies to exceed the 256 MB MALL, so each launch streams
    from HBM.  The launch is the whole product (and with argmax=True the
    fused first-max of the logits), so it is also the roofline kernel; its
    duration is the HIP-event time of the timed replays over the launches."""
    import numpy as np
    wb = weight_bytes(fmt, n, k, rt)
    copies = max(2, copies_bytes // wb)
    g = torch.Generator(device="cuda").manual_seed(0)
    ws = []
    for _ in range(copies):
        w = torch.randn((n, k), generator=g, device="cuda") * 0.02
        if fmt == rt.Q4K:
            ws.append(rt.quantize_q4k(w))
        elif fmt == rt.BF16:
            ws.append(w.to(torch.bfloat16).view(torch.int16))
        elif fmt == rt.Q4_0:
            ws.append(q4_0_blocks(torch, w))
        else:
            raise ValueError(fmt)
        del w
    x = torch.randn((1, k), generator=g, device="cuda")
    y = torch.empty((1, n), device="cuda")

    def run():
        for w in ws:
            if argmax:
                rt.gemv_bf16_argmax(w, x, n, k, y=y)
            else:
                rt.gemv(fmt, w, x, n, k, y=y)

    ms, _ = time_graph(torch, run, args.warmup, args.steps)
    us = ms * 1e3 / copies
    nbytes = wb + 4 * k + 4 * n
    gbs = nbytes / (us * 1e-6) / 1e9
    roof = {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None, "us_per_launch": round(us, 3),
            "bytes_per_launch": nbytes}
    cpu = None
    if not args.no_cpu_baseline:
        kind, cref, threads, orc = _cpu_handles()
        wh = ws[0].cpu().numpy()
        xh = x.cpu().numpy()
        if fmt == rt.Q4K:
            desc = f"Q4KMat::matmul_q4k_t -> gemv_mt, threads = min(hw={threads}, N/128), x86 dot_row"
            if kind == "reference":
                h = cref.q4k_new(wh, n, k)
                out = np.empty((1, n), np.float32)
                med, reps = _cpu_timed(lambda: cref.q4k_handle_matmul_t(h, xh, 1, out), 10.0)
                cref.q4k_delete(h)
            else:
                med, reps = _cpu_timed(lambda: orc.q4k_matmul_t(wh, n, k, xh), 10.0)
        elif fmt == rt.BF16:
            wh = wh.view(np.uint16).reshape(n, k)
            desc = (f"MatBf16::matmul_by_t -> gemv_mt, threads = min(hw={threads}, N/128), x86 dot_row"
                    + (", then the first-max argmax (transformer5.cpp:382-391)" if argmax else ""))
            if kind == "reference":
                h = cref.bf16_new(wh, n, k)
                out = np.empty((1, n), np.float32)

                def once():
                    cref.bf16_handle_matmul_t(h, xh, 1, out)
                    if argmax:
                        orc.argmax_first(out.reshape(-1))
                med, reps = _cpu_timed(once, 10.0)
                cref.bf16_delete(h)
            else:
                med, reps = _cpu_timed(lambda: orc.bf16_matmul_t(wh, xh), 10.0)
        else:  # Q4_0: Q4Mat::matmul_q4_t on decode_q4_0_to_q4mat of the same bytes (single-threaded)
            packed, scales = orc.q4_0_to_q4mat(wh, n * k)
            desc = "Q4Mat::matmul_q4_t (single-threaded) on decode_q4_0_to_q4mat of the same blocks"
            if kind == "reference":
                med, reps = _cpu_timed(lambda: cref.q4mat_matmul_t(packed, scales, n, k, xh), 10.0)
            else:
                med, reps = _cpu_timed(lambda: orc.q4mat_matmul_t(packed, scales, n, k, xh), 10.0)
            threads = 1
        cpu = {"value": round(nbytes / med / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": kind,
               "sample": f"the whole GEMV, median of {reps} reps ({med * 1e3:.2f} ms each); {desc}",
               "us_per_launch": round(med * 1e6, 1)}
    return line(args, f"{label} achieved HBM GB/s", round(gbs, 1), "GB/s", ms / copies, True,
                "q4_k weights, f32 activations (3 exact int8 limbs per value, power-of-two scale per 32)"
                if fmt == rt.Q4K else ("bf16 weights, f32 activations" if fmt == rt.BF16
                                       else "q4_0 weights, f32 activations"),
                {"workload": workload, "n": n, "k": k, "bytes_per_launch": nbytes, "weight_copies": int(copies),
                 "us_per_launch": round(us, 3), "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2)},
                roof, cpu)


def bench_path_gemv(args, rt, torch, kind: str):
    """The GEMV paths beside the headline, each measured like configs 1-2b
    (one product per launch, rotating through weight copies that exceed the
    256 MB MALL, HIP events over graph replays) with the reference's CPU
    path for the same product timed beside it:
      q8_gemv     Q4_K x Q8 activations (the reference's aarch64 gemv_mt,
                  dot_row_q8), 8192 x 3072 tiled;
      q6k_gemv    native GGUF Q6_K, the Llama-3.2-3B down 3072 x 8192 tiled;
      q4mat_gemv  Q4Mat (Linear2::quantize's storage), 4096 x 4096;
      batch_gemv  Q4_K 8192 x 3072 at M = 8 (speculative verify)."""
    import numpy as np
    g = torch.Generator(device="cuda").manual_seed(0)
    m = 1
    if kind == "q8_gemv":
        n, k = 8192, 3072
        wbytes = n * k // 256 * 144
    elif kind == "q6k_gemv":
        n, k = 3072, 8192
        wbytes = n * k // 256 * 210
    elif kind == "q4mat_gemv":
        n, k = 4096, 4096
        wbytes = rt.q4mat_bytes(n, k)
    elif kind == "batch_gemv":
        n, k, m = 8192, 3072, 8
        wbytes = n * k // 256 * 144
    else:
        raise ValueError(kind)
    copies = max(2, (768 << 20) // wbytes)
    ws, host = [], None
    for i in range(copies):
        if kind == "q6k_gemv":
            b = torch.randint(0, 256, (n * (k // 256), 210), dtype=torch.uint8, device="cuda", generator=g)
            b[:, 208] = 0x00
            b[:, 209] = 0x20  # d = 2^-7 (f16 0x2000): finite, typical magnitude
            b = b.reshape(-1)
            if i == 0:
                host = rt.dequant_q6k_bf16(b, n, k).cpu().numpy().view(np.uint16)
            ws.append(rt.q6k_tile(b, n, k))
        elif kind == "q4mat_gemv":
            # synthetic Q4Mat storage: random nibbles (-8..7), scales of the
            # magnitude absmax / 7 gives N(0, 0.02) weights
            packed = torch.randint(0, 256, (n * k // 2,), dtype=torch.uint8, device="cuda",
                                   generator=g).cpu().numpy()
            scales = (0.006 + 0.004 * torch.rand((n * k // 32,), generator=g, device="cuda")).cpu().numpy()
            if i == 0:
                host = (packed, scales)
            ws.append(rt.q4mat_upload(packed, scales, n, k))
        else:
            w = torch.randn((n, k), generator=g, device="cuda") * 0.02
            blocks = rt.quantize_q4k(w)
            del w
            if i == 0:
                host = blocks.cpu().numpy()
            ws.append(rt.q4k_tile(blocks, n, k) if kind == "q8_gemv" else blocks)
    x = torch.randn((m, k), generator=g, device="cuda")
    y = torch.empty((m, n), device="cuda")

    def run():
        for w in ws:
            if kind == "q8_gemv":
                rt.gemv_q4k_q8(w, x, n, k, tiled=True, y=y)
            elif kind == "q6k_gemv":
                rt.gemv_q6k_tiled(w, x, n, k, y=y)
            elif kind == "q4mat_gemv":
                rt.gemv(rt.Q4MAT, w, x, n, k, y=y)
            else:
                rt.gemv(rt.Q4K, w, x, n, k, y=y)

    ms, _ = time_graph(torch, run, args.warmup, args.steps)
    us = ms * 1e3 / copies
    nbytes = wbytes + 4 * m * k + 4 * m * n
    gbs = nbytes / (us * 1e-6) / 1e9
    roof = {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None, "us_per_launch": round(us, 3),
            "bytes_per_launch": nbytes}
    cpu = None
    if not args.no_cpu_baseline:
        ckind, cref, threads, orc = _cpu_handles()
        xh = x.cpu().numpy()
        if kind == "q8_gemv":
            # dot_row_q8 is NEON-only: the oracle's restatement, one thread.
            ckind, threads = "port", 1
            med, reps = _cpu_timed(lambda: orc.q4k_gemv_q8(host, n, k, xh), 10.0)
            desc = ("the oracle's restatement of gemv_mt's aarch64 branch (quantize_activation_q8, then "
                    "dot_row_q8 per row; the reference's NEON code does not build on x86), one thread")
        elif kind == "q6k_gemv":
            if ckind == "reference":
                h = cref.bf16_new(host, n, k)
                out = np.empty((1, n), np.float32)
                med, reps = _cpu_timed(lambda: cref.bf16_handle_matmul_t(h, xh, 1, out), 10.0)
                cref.bf16_delete(h)
            else:
                med, reps = _cpu_timed(lambda: orc.bf16_matmul_t(host, xh), 10.0)
            desc = (f"the reference's path for a Q6_K weight: widened to BF16 at load (not timed), then "
                    f"MatBf16 gemv_mt with threads = min(hw={threads}, N/128); GB/s over the Q6_K bytes")
        elif kind == "q4mat_gemv":
            packed, scales = host
            fn = cref.q4mat_matmul_t if ckind == "reference" else orc.q4mat_matmul_t
            med, reps = _cpu_timed(lambda: fn(packed, scales, n, k, xh), 10.0)
            threads = 1
            desc = "Q4Mat::matmul_q4_t (single-threaded, quant_q4.cpp:92-114)"
        else:
            rows = 256
            bh = host.reshape(n, -1)[:rows].reshape(-1)
            fn = cref.q4k_matmul_t if ckind == "reference" else orc.q4k_matmul_t
            med_rows, reps = _cpu_timed(lambda: fn(bh, rows, k, xh), 10.0)
            med = med_rows * n / rows
            threads = 1
            desc = (f"Q4KMat::matmul_q4k_t's M > 1 loop (single-threaded, quant_q4k.cpp:611-623) on the first "
                    f"{rows} output rows, extrapolated linearly to all {n} rows")
        cpu = {"value": round(nbytes / med / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": ckind,
               "sample": f"the whole product, median of {reps} reps ({med * 1e3:.2f} ms each); {desc}",
               "us_per_launch": round(med * 1e6, 1)}
    label = {"q8_gemv": "Q4_K x Q8-activation GEMV 8192x3072 (aarch64 gemv_mt semantics)",
             "q6k_gemv": "native Q6_K GEMV 3072x8192 (Llama-3.2-3B down)",
             "q4mat_gemv": "Q4Mat GEMV 4096x4096",
             "batch_gemv": "batched Q4_K GEMV 8192x3072, M=8"}[kind]
    dtype = {"q8_gemv": "q4_k weights, int8 activations (per-32 absmax/127 scale), i32 dots, f32 combine",
             "q6k_gemv": "q6_k weights widened in registers to the reference's bf16 values, f32 activations "
                         "(3 exact bf16 limbs)",
             "q4mat_gemv": "q4mat weights (signed nibbles, f32 scale per 32), f32 activations",
             "batch_gemv": "q4_k weights, f32 activations (3 exact int8 limbs per value)"}[kind]
    return line(args, f"{label} achieved HBM GB/s", round(gbs, 1), "GB/s", ms / copies, True, dtype,
                {"workload": kind, "n": n, "k": k, "m": m, "bytes_per_launch": nbytes,
                 "weight_copies": int(copies), "us_per_launch": round(us, 3),
                 "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2)}, roof, cpu)


def bench_gemm(args, rt, torch, shapes, label, a_bf16, workload):
    """BASELINE configs 4 and 5: Q4_K GEMMs (bf16 MFMA, f32 accumulate), one
    graph of the config's GEMMs per step.  The roofline kernel is the GEMM
    kernel that the largest shape runs, alone: where the plan decodes the
    Q4_K weight inside the GEMM (producer waves, config 4's gate), the Q4_K
    GEMM on the bf16 copy of A; where it dequantizes the weight once first
    (config 5), the bf16 GEMM on a BF16 weight of the same shape."""
    import numpy as np
    g = torch.Generator(device="cuda").manual_seed(0)
    items = []
    flops = 0
    for m, n, k in shapes:
        w = torch.randn((n, k), generator=g, device="cuda") * 0.02
        blocks = rt.quantize_q4k(w)
        del w
        a = torch.randn((m, k), generator=g, device="cuda")
        if a_bf16:
            a = a.to(torch.bfloat16)
        c = torch.empty((m, n), device="cuda")
        items.append((a, blocks, c, m, n, k))
        flops += 2 * m * n * k
    need = max(rt.library().lib.rt_hip_gemm_workspace_bytes(rt.Q4K, rt.BF16 if a_bf16 else rt.F32, m, n, k)
               for _, _, _, m, n, k in items)
    rt.reserve_workspace(need)

    def run():
        for a, blocks, c, _, n, k in items:
            rt.gemm(rt.Q4K, a, blocks, n, k, c=c)

    ms, _ = time_graph(torch, run, args.warmup, args.steps)
    tflops = flops / (ms * 1e-3) / 1e12
    # roofline kernel: the largest shape's bf16 GEMM, repeated
    a, blocks, c, m, n, k = max(items, key=lambda it: it[3] * it[4] * it[5])
    ab = a if a_bf16 else a.to(torch.bfloat16)
    # the plan keeps no bf16 copy of the weight: decoded inside the GEMM
    in_gemm = rt.library().lib.rt_hip_gemm_workspace_bytes(rt.Q4K, rt.BF16, m, n, k) < n * k * 2
    wk, fk = (blocks, rt.Q4K) if in_gemm else (rt.dequant_q4k(blocks, n, k, bf16=True), rt.BF16)
    reps = 10

    def run_k():
        for _ in range(reps):
            rt.gemm(fk, ab, wk, n, k, c=c)

    ms_k, _ = time_graph(torch, run_k, 2, max(3, args.steps // 5))
    us_k = ms_k * 1e3 / reps
    kt = 2 * m * n * k / (us_k * 1e-6) / 1e12
    roof = {"bound": "mfma", "achieved": round(kt, 1), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(kt / BF16_PEAK_TFLOPS, 4), "traffic": None,
            "kernel": (f"Q4_K GEMM {m}x{n}x{k}, weight decoded to bf16 in producer waves (k_gemm_ws), bf16 A, "
                       "f32 accumulate") if in_gemm else
                      f"bf16 MFMA GEMM {m}x{n}x{k} (bf16 operands, f32 accumulate)",
            "us_per_launch": round(us_k, 2), "flops_per_launch": 2 * m * n * k}
    cpu = None
    if not args.no_cpu_baseline:
        kind, cref, threads, orc = _cpu_handles()
        total = 0.0
        parts = []
        rows = 64
        for a, blocks, _, m, n, k in items:
            bh = blocks.cpu().numpy().reshape(n, -1)[:rows].reshape(-1)
            ah = a.float().cpu().numpy()
            fn = (lambda bh=bh, ah=ah, k=k: cref.q4k_matmul_t(bh, rows, k, ah)) if kind == "reference" else \
                (lambda bh=bh, ah=ah, k=k: orc.q4k_matmul_t(bh, rows, k, ah))
            med, _ = _cpu_timed(fn, 2.0, min_reps=1, max_reps=3)
            total += med * n / rows
            parts.append(f"{m}x{n}x{k}: {med * 1e3:.0f} ms per {rows} rows")
        cpu = {"value": round(flops / total / 1e9, 3), "unit": "GFLOP/s", "cores": 1, "kind": kind,
               "sample": ("the reference's Linux M>1 path, Q4KMat::matmul_q4k_t's single-threaded loop "
                          f"(quant_q4k.cpp:611-623), timed on the first {rows} output rows of each GEMM and "
                          f"extrapolated linearly to all rows (labelled extrapolation): " + "; ".join(parts)),
               "ms_per_step_extrapolated": round(total * 1e3, 1)}
    return line(args, f"{label} bf16-MFMA TFLOP/s", round(tflops, 1), "TFLOP/s", ms, True,
                "q4_k weights dequantized to bf16, " + ("bf16" if a_bf16 else "f32->bf16") +
                " activations, f32 accumulate",
                {"workload": workload, "shapes": [list(s) for s in shapes], "flops": flops,
                 "pct_bf16_peak": round(100 * tflops / BF16_PEAK_TFLOPS, 2)}, roof, cpu)


def bench_flux_attention(args, rt, torch):
    """FLUX.1 attention at 1024x1024 (metal_flux.mm:254-272 over
    flux.cpp:287-321): t = 4352 tokens (4096 image + 256 text), 24 heads of
    128, f32 throughout.  One launch per step, captured in a graph; it is
    the roofline kernel (f32 matrix cores).  Algorithmic flops: 2 t^2 d per
    head for the scores and 2 t^2 d for the weighted sum of v."""
    import numpy as np
    t, h, d = 4352, 24, 128
    g = torch.Generator(device="cuda").manual_seed(0)
    q, k, v = (torch.randn((t, h * d), generator=g, device="cuda") for _ in range(3))
    out = torch.empty_like(q)

    def run():
        rt.flux_attention(q, k, v, h, d, out=out)

    ms, _ = time_graph(torch, run, args.warmup, args.steps)
    flops = 4 * t * t * d * h
    tf = flops / (ms * 1e-3) / 1e12
    log(f"[bench] flux attention {ms * 1e3:.1f} us, {tf:.1f} TFLOP/s f32")
    roof = {"bound": "mfma", "achieved": round(tf, 2), "peak": F32_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(tf / F32_PEAK_TFLOPS, 4), "traffic": None,
            "kernel": "k_flux_attn<128> (f32 MFMA 16x16x4, online softmax, 128 queries x 32-key tiles)",
            "us_per_launch": round(ms * 1e3, 2), "flops_per_launch": flops}
    cpu = None
    if not args.no_cpu_baseline:
        _, _, _, orc = _cpu_handles()
        qh, kh, vh = (a.cpu().numpy() for a in (q, k, v))
        rows = np.linspace(0, t - 1, 32).astype(np.int64)
        med, reps = _cpu_timed(lambda: orc.flux_attention(qh, kh, vh, h, d, rows=rows), 12.0, min_reps=1,
                               max_reps=5)
        per_row = med / rows.size
        cpu = {"value": round(flops / (per_row * t) / 1e9, 3), "unit": "GFLOP/s", "cores": 1, "kind": "port",
               "sample": (f"the oracle's restatement of flux.cpp:287-321 (single-threaded, -O3 "
                          f"-ffp-contract=off, the reference's loop order) on {rows.size} output rows of all "
                          f"24 heads, median of {reps}, extrapolated linearly to all {t} rows: "
                          f"{per_row * t:.1f} s per call; flux.cpp's attention is file-local to a "
                          f"translation unit that needs the whole model, so it is not built into oracle/_ref")}
    return line(args, "FLUX.1 attention f32 TFLOP/s (t=4352, 24 heads x 128)", round(tf, 2), "TFLOP/s", ms, True,
                "f32", {"workload": "FLUX.1 1024x1024 attention: 4096 image + 256 text tokens, 24 heads of 128, "
                                    "no mask", "t": t, "heads": h, "head_dim": d, "flops": flops,
                        "pct_f32_peak": round(100 * tf / F32_PEAK_TFLOPS, 2)},
                roof, cpu, data="synthetic: N(0,1) q, k, v")


# ------------------------------------------------- launch-ceiling calibration --

def token_launch_bytes(mix: str):
    """Algorithmic bytes of each launch of the headline token, in order: per
    layer q/k/v (one launch; a BF16-widened v included), o, gate+up, down,
    then the lm_head -- the byte counts DecodeModel.launches() reads, with
    the activation counted once per GEMV as DecodeModel.bytes_per_token
    counts it -- and the bytes each launch writes."""
    def q4(n, k):
        return n * (k // 256) * 144

    out = []
    for layer in range(LAYERS):
        wide = mix in ("q4km", "q4km_q6k") and layer in WIDENED_LAYERS
        v = KV * HIDDEN * 2 if wide else q4(KV, HIDDEN)
        if wide and mix == "q4km_q6k":
            down = HIDDEN * (FFN // 256) * 210
        else:
            down = HIDDEN * FFN * 2 if wide else q4(HIDDEN, FFN)
        out.append(("qkv_bf16v" if wide else "qkv",
                    q4(HIDDEN, HIDDEN) + q4(KV, HIDDEN) + v + 3 * 4 * HIDDEN + 4 * (HIDDEN + 2 * KV),
                    4 * (HIDDEN + 2 * KV)))
        out.append(("o", q4(HIDDEN, HIDDEN) + 8 * HIDDEN, 4 * HIDDEN))
        out.append(("gate_up", 2 * q4(FFN, HIDDEN) + 2 * 4 * HIDDEN + 8 * FFN, 8 * FFN))
        out.append(("down_bf16" if wide else "down", down + 4 * FFN + 4 * HIDDEN, 4 * HIDDEN))
    out.append(("lm_head", q4(VOCAB, HIDDEN) + 4 * HIDDEN + 4 * VOCAB, 4 * VOCAB))
    return out


def bench_ceiling(args, rt, torch):
    """What the headline's launch structure allows with no GEMV arithmetic at
    all.  The token's 113 launches keep their order, their byte counts and
    their dependencies (one stream, one hipGraph), but each launch is a plain
    streaming read of its bytes from a buffer of its own
    (rt_hip_probe_read), so nothing is reused across launches and the whole
    token (2.38 GB) exceeds the 256 MB MALL.  Read shapes: several workgroup
    counts; per-launch figures: a graph of the token's launches of one kind
    alone.  Also N dependent empty launches in one graph (the fixed cost of a
    launch) and one read of all the token's bytes in a single launch (the
    bandwidth the device gives with no launch boundaries)."""
    plan = token_launch_bytes(args.mix)
    align = 4096
    offs, total = [], 0
    for _, b, _ in plan:
        offs.append(total)
        total += (b + align - 1) // align * align
    buf = torch.randint(-2**31, 2**31 - 1, (total // 4,), dtype=torch.int32, device="cuda")
    sink = torch.zeros(max(65536, VOCAB), dtype=torch.int32, device="cuda")
    nbytes = sum(b for _, b, _ in plan)
    log(f"[bench] ceiling: {len(plan)} launches, {nbytes / 1e9:.3f} GB/token ({args.mix})")

    def reads(sel, wgs, write=True):
        # each launch reads its bytes, then writes its output rows (a GEMV's
        # y); write=False: reads alone
        def run():
            for i in sel:
                b = plan[i][1] // 16 * 16
                rt.probe_read(buf[offs[i] // 4:], b, wgs(b), sink, plan[i][2] if write else 0)
        return run

    read_shapes = {"256 workgroups": lambda b: 256, "512 workgroups": lambda b: 512,
                   "1024 workgroups": lambda b: 1024, "2048 workgroups": lambda b: 2048,
                   "one workgroup per 16 KB": lambda b: max(256, min(65536, b // 16384)),
                   "one workgroup per 64 KB": lambda b: max(256, min(65536, b // 65536))}
    shapes = {}
    for name, wgs in read_shapes.items():
        ms, _ = time_graph(torch, reads(range(len(plan)), wgs), args.warmup, args.steps)
        shapes[name] = round(ms * 1e3, 2)
        log(f"[bench] token as plain reads, {name}: {ms * 1e3:.1f} us/token "
            f"({nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS * 100:.1f}% of 8 TB/s)")
    best_name = min(shapes, key=shapes.get)
    best_us = shapes[best_name]
    ms, _ = time_graph(torch, reads(range(len(plan)), read_shapes[best_name], write=False), args.warmup, args.steps)
    reads_only_us = round(ms * 1e3, 2)
    log(f"[bench] token as plain reads with no output writes ({best_name}): {reads_only_us} us/token")
    # per kind: the token's launches of one kind alone, back to back, best shape per kind
    per_kind = {}
    for kind in dict.fromkeys(k for k, _, _ in plan):
        sel = [i for i, (k, _, _) in enumerate(plan) if k == kind]
        best = None
        for name, fn in read_shapes.items():
            ms, _ = time_graph(torch, reads(sel, fn), args.warmup, args.steps)
            us = ms * 1e3 / len(sel)
            if best is None or us < best[0]:
                best = (us, name)
        b = plan[sel[0]][1]
        per_kind[kind] = {"bytes": b, "launches": len(sel), "us_per_launch": round(best[0], 3),
                          "gbs": round(b / (best[0] * 1e-6) / 1e9, 1), "shape": best[1]}
        log(f"[bench] {kind}: {b / 1e6:.2f} MB per launch, {best[0]:.2f} us ({best[1]})")
    # fixed cost of a dependent launch
    empty = {}
    for wg, th in [(1, 64), (256, 256), (1024, 256)]:
        def run(wg=wg, th=th):
            for _ in range(len(plan)):
                rt.probe_empty(wg, th)
        ms, _ = time_graph(torch, run, args.warmup, args.steps)
        empty[f"{wg}x{th}"] = round(ms * 1e3 / len(plan), 3)
        log(f"[bench] empty launch {wg}x{th}: {ms * 1e3 / len(plan):.3f} us per dependent launch")
    # the whole token's bytes in one read
    one = {}
    for wg in (1024, 4096, 16384):
        ms, _ = time_graph(torch, lambda wg=wg: rt.probe_read(buf, total, wg, sink, 0), args.warmup, args.steps)
        one[str(wg)] = round(ms * 1e3, 2)
    one_us = min(one.values())
    log(f"[bench] all {total / 1e9:.3f} GB in one launch: {one_us:.1f} us "
        f"({total / (one_us * 1e-6) / 1e9:.0f} GB/s)")
    gbs = nbytes / (best_us * 1e-6) / 1e9
    return line(args, "decode-step launch ceiling: us/token of the headline's 113 launches as plain reads",
                best_us, "us/token", best_us / 1e3, False, "u8 (reads only)",
                {"workload": "the headline token's launch sequence (Llama-3.2-3B, " + args.mix +
                             "), each launch a plain read of its byte count, one hipGraph",
                 "launches_per_token": len(plan), "bytes_per_token": nbytes,
                 "gbs": round(gbs, 1), "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
                 "best_shape": best_name, "us_per_token_by_shape": shapes,
                 "us_per_token_reads_only": reads_only_us, "per_kind": per_kind,
                 "empty_launch_us": empty,
                 "one_launch_read": {"bytes": total, "us_by_workgroups": one,
                                     "gbs": round(total / (one_us * 1e-6) / 1e9, 1)}},
                None, None, data="synthetic: random bytes, read only")


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[1])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="llama_decode",
                    choices=["llama_decode", "q4k_gemv", "q4_0_gemv", "bf16_lm_head", "prefill",
                             "flux", "flux_attention", "layer_ops", "decode_layers", "engine_llama3b", "engine_gemma3_4b",
                             "q8_gemv", "q6k_gemv", "q4mat_gemv", "batch_gemv", "ceiling"])
    ap.add_argument("--mix", default="q4km", choices=["q4km", "q4k", "q4km_q6k"])
    ap.add_argument("--context", type=int, default=1024,
                    help="cached positions for --workload decode_layers")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--calibration-copy-mb", type=int, default=0,
                    help="before the workload, copy a buffer of this many MiB once with a plain "
                         "device copy (the known-size kernel that HBM traffic counters are "
                         "scaled by); untimed")
    ap.add_argument("--layout", default="tiled", choices=["tiled", "rows"],
                    help="Q4_K weights tiled once at load (default) or the reference's row-major "
                         "blocks through rt_hip_gemv_q4k*")
    ap.add_argument("--unfused", action="store_true",
                    help="also time the one-launch-per-GEMV step (stderr)")
    ap.add_argument("--traffic-bytes", type=float, default=None,
                    help="HBM bytes per launch of the dominant kernel from rocprofv3 counters")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this build measures one GPU; the path's multi-GPU sharding is "
              "a design that is not run here. Use --gpus 1.", file=sys.stderr)
        return 2

    import torch
    rt = load_rt()
    rt.init(0)
    log(f"[bench] {rt.library().version()} on {torch.cuda.get_device_name(0)}")
    if args.calibration_copy_mb:
        nel = args.calibration_copy_mb * (1 << 20) // 4
        src = torch.ones(nel, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"[bench] calibration copy: {nel * 4} bytes read, {nel * 4} bytes written")
        del src, dst
    if args.workload == "llama_decode":
        out = bench_decode(args, rt, torch)
    elif args.workload == "q4k_gemv":
        out = bench_single_gemv(args, rt, torch, rt.Q4K, 6912, 1024,
                                "config 1 Q4_K GEMV 6912x1152 (Release semantics: K=1024)",
                                "config 1: Q4_K GEMV 6912x1152, 4 super-blocks per row (reference Release "
                                "semantics), batch 1")
    elif args.workload == "q4_0_gemv":
        out = bench_single_gemv(args, rt, torch, rt.Q4_0, 4096, 4096, "config 2a GGUF Q4_0 GEMV 4096x4096",
                                "config 2a: GGUF Q4_0 GEMV 4096x4096, batch 1")
    elif args.workload == "bf16_lm_head":
        out = bench_single_gemv(args, rt, torch, rt.BF16, 262144, 1152,
                                "config 2b BF16 GEMV 262144x1152 + argmax",
                                "config 2b: BF16 lm_head GEMV 262144x1152 with the fused first-max argmax, "
                                "batch 1", argmax=True)
    elif args.workload == "prefill":
        out = bench_gemm(args, rt, torch, [(512, FFN, HIDDEN), (512, FFN, HIDDEN), (512, HIDDEN, FFN)],
                         "config 4 prefill Q4_K GEMM M=512 (gate, up, down)", False,
                         "config 4: Llama-3.2-3B prefill gate/up/down Q4_K GEMMs, M=512, f32 activations")
    elif args.workload == "flux_attention":
        out = bench_flux_attention(args, rt, torch)
    elif args.workload == "layer_ops":
        out = bench_layer_ops(args, rt, torch)
    elif args.workload == "decode_layers":
        out = bench_decode_layers(args, rt, torch)
    elif args.workload.startswith("engine_"):
        out = bench_engine(args, rt, torch, args.workload[len("engine_"):])
    elif args.workload in ("q8_gemv", "q6k_gemv", "q4mat_gemv", "batch_gemv"):
        out = bench_path_gemv(args, rt, torch, args.workload)
    elif args.workload == "ceiling":
        out = bench_ceiling(args, rt, torch)
    elif args.workload == "flux":
        out = bench_gemm(args, rt, torch, [(4608, 9216, 3072), (4608, 12288, 3072), (4608, 3072, 12288)],
                         "config 5 FLUX linears M=4608 (QKV, MLP-in, MLP-out)", True,
                         "config 5: FLUX.1-schnell MMDiT QKV / MLP-in / MLP-out Q4_K GEMMs, M=4608, bf16 "
                         "activations")
    else:
        raise SystemExit(f"workload {args.workload} not available yet")
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
