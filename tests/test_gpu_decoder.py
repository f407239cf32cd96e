"""The decode engine (rt_hip_decoder_*) against the oracle, token by token.

Small models of the two architectures with the real layer structure:

* Llama 3.2 (LlamaBlock::forward_cached, src/transformer5.cpp:198-212):
  RMSNorm, q/k/v, RoPE (interleaved or half-split), f32 KV cache, attention,
  o + residual, RMSNorm, gate/up, SwiGLU, down + residual; a Q4_K_M-style mix
  (v and down BF16 in layer 0).
* Gemma 3 (the Metal engine, src/metal_decode.mm:436-482 with
  src/shaders/decode_gemma3.msl): bf16 embedding x sqrt(hidden), RMSNorm
  (1 + gamma), per-head q/k RMSNorm, NeoX RoPE with per-layer theta and
  scale, f16 KV cache, a sliding window on the local layer, head_dim 256,
  post-attention and post-FFN norms, GELU-tanh.

The expected logits are the oracle's composition of the reference's
operations (every product in the reference's sequential f32 order, the f16
cache rounded by the same RNE), step after step, so errors would accumulate
in the cache exactly as they would in the engine.  Bar: 1e-5 normwise per
step's logits; the argmax index exact.  Batch steps (up to max_batch tokens
in one graph, each weight byte read once for all rows) must agree with the
single-token steps to the same bar.
"""
import numpy as np
import pytest

from helpers import GEMV_TOL, normwise_err, say

pytestmark = pytest.mark.gpu
STEP_TOL = 1e-5


class Model:
    """Weights on the host and the oracle's decode step."""

    def __init__(self, orc, arch, rng, q6k_down=False, wide_layers=None, randn=None, **cfg):
        self.orc, self.arch, self.cfg = orc, arch, cfg
        self.gemma = arch == "gemma3"
        H, F, nq, nkv, d, V = (cfg[k] for k in ("hidden", "ffn", "n_heads", "n_kv_heads", "head_dim", "vocab"))
        self.fmt = {}
        self.w = {}
        # N(0, 1) draws (float32 arrays of `shape`): numpy's by default
        randn = randn or (lambda shape: rng.standard_normal(shape))

        def proj(name, n, k, bf16):
            if bf16 == "q6k":  # GGUF Q6_K bytes; the oracle multiplies their bf16 widening
                from test_gpu_q6k import random_q6k
                self.w[name] = random_q6k(rng, n, k)
                self.fmt[name] = "q6k"
                self.wide_q6k = getattr(self, "wide_q6k", {})
                self.wide_q6k[name] = orc.f32_to_bf16_n(orc.q6k_decode(self.w[name], n * k)).reshape(n, k)
                return
            w32 = (randn((n, k)) * 0.02).astype(np.float32)
            if bf16:
                self.w[name] = orc.f32_to_bf16_n(w32).reshape(n, k)
                self.fmt[name] = "bf16"
            else:
                self.w[name] = orc.q4k_quantize(w32)
                self.fmt[name] = "q4k"

        def norm(name, n):
            # Gemma 3 norms apply 1 + gamma, Llama's gamma itself
            base = 0.0 if self.gemma else 1.0
            self.w[name] = (base + 0.1 * randn((n,))).astype(np.float32)

        for li in range(cfg["n_layers"]):
            wide = li in wide_layers if wide_layers is not None else (li == 0 and not self.gemma)
            proj(f"{li}.q", nq * d, H, False)
            proj(f"{li}.k", nkv * d, H, False)
            proj(f"{li}.v", nkv * d, H, wide)
            proj(f"{li}.o", H, nq * d, False)
            proj(f"{li}.gate", F, H, False)
            proj(f"{li}.up", F, H, False)
            proj(f"{li}.down", H, F, "q6k" if wide and q6k_down else wide)
            for nm in ("attn_norm", "ffn_norm") + (("post_attn_norm", "post_ffn_norm") if self.gemma else ()):
                norm(f"{li}.{nm}", H)
            if self.gemma:
                norm(f"{li}.q_norm", d)
                norm(f"{li}.k_norm", d)
        self.w["embed"] = orc.f32_to_bf16_n((randn((V, H)) * 0.5).astype(np.float32)).reshape(V, H)
        norm("out_norm", H)
        proj("lm_head", V, H, self.gemma)
        self.kc = [np.zeros((cfg["max_seq"], nkv * d), np.float32) for _ in range(cfg["n_layers"])]
        self.vc = [np.zeros((cfg["max_seq"], nkv * d), np.float32) for _ in range(cfg["n_layers"])]
        if not self.gemma:
            self.inv = orc.llama_inv_freq(cfg["rope_theta"], d)

    def load(self, rt):
        c = dict(self.cfg)
        c["arch"] = rt.ARCH_GEMMA3 if self.gemma else rt.ARCH_LLAMA
        dec = rt.Decoder(**c)
        F = {"q4k": rt.Q4K, "bf16": rt.BF16, "q6k": rt.Q6K}
        T = {"q": rt.T_Q, "k": rt.T_K, "v": rt.T_V, "o": rt.T_O, "gate": rt.T_GATE, "up": rt.T_UP,
             "down": rt.T_DOWN, "attn_norm": rt.T_ATTN_NORM, "ffn_norm": rt.T_FFN_NORM,
             "post_attn_norm": rt.T_POST_ATTN_NORM, "post_ffn_norm": rt.T_POST_FFN_NORM,
             "q_norm": rt.T_Q_NORM, "k_norm": rt.T_K_NORM}
        for name, arr in self.w.items():
            if name == "embed":
                dec.set(-1, rt.T_EMBED, rt.BF16, arr)
            elif name == "out_norm":
                dec.set(-1, rt.T_OUTPUT_NORM, rt.F32, arr)
            elif name == "lm_head":
                dec.set(-1, rt.T_LM_HEAD, F[self.fmt[name]], arr)
            else:
                li, nm = name.split(".")
                dec.set(int(li), T[nm], F.get(self.fmt.get(name), rt.F32), arr)
        return dec

    def mm(self, name, x, n, k):
        if self.fmt[name] == "q4k":
            return self.orc.q4k_matmul_t(self.w[name], n, k, x.reshape(1, k)).reshape(-1)
        if self.fmt[name] == "q6k":
            return self.orc.bf16_matmul_t(self.wide_q6k[name], x.reshape(1, k)).reshape(-1)
        return self.orc.bf16_matmul_t(self.w[name], x.reshape(1, k)).reshape(-1)

    def step(self, token, pos):
        """The oracle's decode step; updates the oracle's caches."""
        o, c = self.orc, self.cfg
        H, F, nq, nkv, d = (c[k] for k in ("hidden", "ffn", "n_heads", "n_kv_heads", "head_dim"))
        eps = c["norm_eps"]
        g = self.gemma
        x = (self.w["embed"][token].astype(np.uint32) << 16).view(np.float32) * np.float32(c.get("embed_scale") or 1.0)
        x = x.astype(np.float32)
        for li in range(c["n_layers"]):
            n1 = o.rmsnorm(x, self.w[f"{li}.attn_norm"], eps, gemma3=g)
            q = self.mm(f"{li}.q", n1, nq * d, H)
            k = self.mm(f"{li}.k", n1, nkv * d, H)
            v = self.mm(f"{li}.v", n1, nkv * d, H)
            window = 0
            if g:
                glob = li % c["global_every"] == c["global_every"] - 1
                theta = c["rope_theta"] if glob else c["rope_theta_local"]
                fs = c["rope_freq_scale"] if glob else c["rope_freq_scale_local"]
                window = 0 if glob else c["sliding_window"]
                q = o.rmsnorm_per_head(q, self.w[f"{li}.q_norm"], nq, d, eps)
                k = o.rmsnorm_per_head(k, self.w[f"{li}.k_norm"], nkv, d, eps)
                q = o.rope_neox(q, nq, d, theta, fs, pos)
                k = o.rope_neox(k, nkv, d, theta, fs, pos)
            else:
                half = bool(c.get("rope_half"))
                q = o.llama_rope(q, nq, d, pos, self.inv, half=half)
                k = o.llama_rope(k, nkv, d, pos, self.inv, half=half)
            if c.get("kv_f16"):  # the cache keeps half(x), RNE
                k = o.f32_to_f16_rne_n(k).view(np.float16).astype(np.float32)
                v = o.f32_to_f16_rne_n(v).view(np.float16).astype(np.float32)
            self.kc[li][pos] = k
            self.vc[li][pos] = v
            k_end = pos + 1
            k_start = max(0, k_end - window) if window else 0
            scale = c.get("attn_scale") or float(1.0 / np.sqrt(np.float32(d)))
            attn = o.gqa_attention_decode(q, self.kc[li], self.vc[li], k_end, nq, nkv, d, scale, k_start=k_start)
            ao = self.mm(f"{li}.o", attn, H, nq * d)
            h = (x + o.rmsnorm(ao, self.w[f"{li}.post_attn_norm"], eps, gemma3=True)) if g else x + ao
            n2 = o.rmsnorm(h, self.w[f"{li}.ffn_norm"], eps, gemma3=g)
            gt = self.mm(f"{li}.gate", n2, F, H)
            up = self.mm(f"{li}.up", n2, F, H)
            act = (o.gelu_tanh(gt) * up).astype(np.float32) if g else o.swiglu(gt, up)
            dn = self.mm(f"{li}.down", act, H, F)
            x = (h + o.rmsnorm(dn, self.w[f"{li}.post_ffn_norm"], eps, gemma3=True)) if g else h + dn
            x = x.astype(np.float32)
        xn = o.rmsnorm(x, self.w["out_norm"], eps, gemma3=g)
        return self.mm("lm_head", xn, c["vocab"], H)


LLAMA = dict(n_layers=2, hidden=512, n_heads=8, n_kv_heads=2, head_dim=64, ffn=1024, vocab=1000, max_seq=64,
             norm_eps=1e-5, rope_theta=500000.0, rope_theta_local=0.0, rope_freq_scale=1.0,
             rope_freq_scale_local=1.0, rope_half=0, sliding_window=0, global_every=0, attn_scale=0.0,
             embed_scale=0.0, kv_f16=0, max_batch=4)
GEMMA = dict(n_layers=2, hidden=512, n_heads=4, n_kv_heads=2, head_dim=256, ffn=1024, vocab=1000, max_seq=32,
             norm_eps=1e-6, rope_theta=1e6, rope_theta_local=1e4, rope_freq_scale=0.125, rope_freq_scale_local=1.0,
             rope_half=1, sliding_window=4, global_every=2, attn_scale=1.0 / 16.0,
             embed_scale=float(np.sqrt(np.float32(512))), kv_f16=1, max_batch=3)


@pytest.mark.parametrize("arch,cfg", [("llama", LLAMA), ("llama_half", dict(LLAMA, rope_half=1)),
                                      ("gemma3", GEMMA)])
def test_decoder_steps_match_oracle(rt, orc, arch, cfg):
    rng = np.random.default_rng(len(arch))
    m = Model(orc, "gemma3" if arch == "gemma3" else "llama", rng, **cfg)
    dec = m.load(rt)
    tokens = rng.integers(0, cfg["vocab"], 10)
    worst = 0.0
    for pos, tok in enumerate(tokens):
        say(f"[decoder {arch}] step pos={pos} token={tok}")
        got, idx = dec.step(int(tok), pos, argmax=True)
        want = m.step(int(tok), pos)
        e = normwise_err(got, want)
        worst = max(worst, e)
        assert e <= STEP_TOL, (pos, e)
        assert idx == orc.argmax_first(got) and idx == orc.argmax_first(want), pos
    say(f"[decoder {arch}] worst step normwise error {worst:.2e}")
    dec.close()


def test_decoder_gemma_mixed_formats_match_oracle(rt, orc):
    """Gemma 3 with BF16 v and down in the middle layer (a Q4_K_M-style mix):
    that layer's q/k/v launch cannot take the previous layer's post-FFN norm
    (the separate norm runs there), the next layer's can (after a BF16 GELU
    down), and every gate/up launch takes its post-attention norm."""
    cfg = dict(GEMMA, n_layers=3)
    rng = np.random.default_rng(23)
    m = Model(orc, "gemma3", rng, wide_layers={1}, **cfg)
    dec = m.load(rt)
    try:
        worst = 0.0
        for pos, tok in enumerate(rng.integers(0, cfg["vocab"], 8)):
            got, idx = dec.step(int(tok), pos, argmax=True)
            want = m.step(int(tok), pos)
            e = normwise_err(got, want)
            worst = max(worst, e)
            assert e <= STEP_TOL, (pos, e)
            assert idx == orc.argmax_first(got), pos
        say(f"[decoder gemma3 mixed] worst step normwise error {worst:.2e}")
    finally:
        dec.close()


@pytest.mark.parametrize("arch,cfg", [("llama", LLAMA), ("gemma3", GEMMA)])
def test_decoder_batch_matches_single_steps(rt, orc, arch, cfg):
    """decode_step_batch: tokens 2..(2 + max_batch) in one graph give the
    single-token steps' logits (and the oracle's)."""
    rng = np.random.default_rng(7 + len(arch))
    m = Model(orc, "gemma3" if arch == "gemma3" else "llama", rng, **cfg)
    a, b = m.load(rt), m.load(rt)
    nb = cfg["max_batch"]
    tokens = rng.integers(0, cfg["vocab"], 2 + nb)
    single = []
    for pos, tok in enumerate(tokens):
        single.append(a.step(int(tok), pos))
        want = m.step(int(tok), pos)
        assert normwise_err(single[-1], want) <= STEP_TOL
    for pos in range(2):
        b.step(int(tokens[pos]), pos)
    say(f"[decoder {arch}] batch of {nb} at position 2")
    batch = b.step_batch(tokens[2:], 2)
    for i in range(nb):
        e = normwise_err(batch[i], single[2 + i])
        assert e <= STEP_TOL, (i, e)
    a.close()
    b.close()


def test_decoder_q6k_down_matches_oracle(rt, orc):
    """A Llama down projection kept as GGUF Q6_K (layer 0; the reference
    widens it to BF16 at load) through rt_hip_gemv_q6k_tiled_swiglu_residual
    inside the token's graph: logits against the oracle's step on the widened
    weights, token by token.  Batch graphs take no Q6_K down: refused."""
    cfg = dict(LLAMA, max_batch=0)
    say("[decoder q6k down] llama, 6 tokens")
    m = Model(orc, "llama", np.random.default_rng(77), q6k_down=True, **cfg)
    assert m.fmt["0.down"] == "q6k" and m.fmt["1.down"] == "q4k"
    dec = m.load(rt)
    try:
        for pos, tok in enumerate([5, 17, 999, 0, 42, 7]):
            got = dec.step(tok, pos)
            want = m.step(tok, pos)
            err = normwise_err(got, want)
            assert err <= STEP_TOL, (pos, err)
    finally:
        dec.close()
    bad = rt.Decoder(**dict(LLAMA, arch=rt.ARCH_LLAMA))  # max_batch 4
    try:
        with pytest.raises(RuntimeError):
            bad.set(0, rt.T_DOWN, rt.Q6K, m.w["0.down"])
    finally:
        bad.close()


def test_decoder_rejects_bad_use(rt, orc):
    import ctypes as C
    lib = rt.library()
    bad = dict(LLAMA, head_dim=96)
    with pytest.raises(rt.RtHipError):
        rt.Decoder(arch=rt.ARCH_LLAMA, **bad)
    dec = rt.Decoder(arch=rt.ARCH_LLAMA, **LLAMA)
    # weights missing: the step is refused with a message
    out = np.zeros(LLAMA["vocab"], np.float32)
    rc = lib.lib.rt_hip_decoder_step(dec.h, 1, 0, out.ctypes.data, None, None)
    assert rc == 1 and b"weights not set" in lib.lib.rt_hip_last_error()
    # wrong byte count for a projection
    with pytest.raises(rt.RtHipError, match="bytes given"):
        dec.set(0, rt.T_Q, rt.BF16, np.zeros(10, np.uint16))
    with pytest.raises(rt.RtHipError):
        dec.set(0, rt.T_EMBED, rt.BF16, np.zeros(10, np.uint16))  # model tensor with a layer
    dec.close()
    del C


# ---- the attention the engine benchmarks: real head geometry, long caches ----
# attention2_splits and the split fold (decoder_ops.hip) only take more than
# one split once the cache is longer than one 64-position chunk per split;
# the toy models above never get there.  These cases keep hidden, ffn and
# vocab small but use the Llama-3.2-3B attention geometry (24 query heads
# over 8 KV heads, head_dim 128: k_attn2_partial<128, 3>) and the Gemma 3
# local/global geometry (8 over 4, head_dim 256, f16 cache) with caches
# pre-filled through rt_hip_decoder_set_kv, so several splits are busy and,
# where the cache is shorter than max_seq, some are idle.

def split_rule(n_kv, m, max_len, cus, head_dim):
    """attention2_splits (decoder_ops.hip): enough (kv head, split) work-
    groups for every CU, at least one round of the partial kernel's positions
    per split (64 at head_dim 128, 32 at 256)."""
    want = -(-cus // (n_kv * m))
    by_len = -(-max_len // (64 if head_dim <= 128 else 32))
    return max(1, min(want, by_len))


def busy_rule(length, S, head_dim):
    """Splits holding positions: chunks of ceil(len / S) positions rounded up
    to whole rounds of the partial kernel (64 positions at head_dim 128, 32 at
    256: 16 or 8 position groups x 4 loaded ahead)."""
    batch = 64 if head_dim <= 128 else 32
    chunk = -(-(-(-length // S)) // batch) * batch
    return min(S, -(-length // chunk))


def cu_count():
    import torch
    return torch.cuda.get_device_properties(0).multi_processor_count


def prefill(m, dec, rng, rows):
    """Random N(0,1) K/V rows 0..rows-1 in every layer, in the engine (set_kv)
    and the oracle's cache (f16-rounded when the cache is f16, as set_kv's
    conversion rounds them)."""
    c = m.cfg
    width = c["n_kv_heads"] * c["head_dim"]
    for li in range(c["n_layers"]):
        k = rng.standard_normal((rows, width)).astype(np.float32)
        v = rng.standard_normal((rows, width)).astype(np.float32)
        dec.set_kv(li, k, v, rows)
        if c.get("kv_f16"):
            k = m.orc.f32_to_f16_rne_n(k.reshape(-1)).view(np.float16).astype(np.float32).reshape(rows, width)
            v = m.orc.f32_to_f16_rne_n(v.reshape(-1)).view(np.float16).astype(np.float32).reshape(rows, width)
        m.kc[li][:rows] = k
        m.vc[li][:rows] = v


LLAMA_3B_ATTN = dict(LLAMA, n_heads=24, n_kv_heads=8, head_dim=128, ffn=512, max_seq=2048, max_batch=0)
GEMMA_4B_ATTN = dict(GEMMA, n_heads=8, n_kv_heads=4, head_dim=256, ffn=512, max_seq=512, sliding_window=200,
                     max_batch=0)


@pytest.mark.parametrize("arch,cfg,rows", [
    # S = 32 splits, 16 busy at 1001 positions
    ("llama3b", LLAMA_3B_ATTN, 1000),
    # S = 32, 2 busy
    ("llama3b", LLAMA_3B_ATTN, 100),
    # the bench's cache: S = 16, all busy
    ("llama3b", dict(LLAMA_3B_ATTN, max_seq=1024), 1000),
    # local layer: window 200 > one chunk, S = 7 (5 busy); global: S = 16 (5 busy)
    ("gemma3_4b", GEMMA_4B_ATTN, 150),
    # local: the window slides past position 0 (all 7 busy); global 13 of 16
    ("gemma3_4b", GEMMA_4B_ATTN, 400),
    # splits of two rounds (S capped by the CUs), the new position in the
    # second round of the last busy split: global layer S = 64, 48 busy;
    # the half-split Llama form (q/k prepared inside the attention launch):
    # S = 32, 24 busy
    ("gemma3_4b", dict(GEMMA_4B_ATTN, max_seq=4096), 3050),
    ("llama3b_half", dict(LLAMA_3B_ATTN, max_seq=4096, rope_half=1), 3050),
    # caches that are not whole rounds long: with no window and S splits of
    # one round covering the cache, every split's loads leave before the
    # position is read, and the last split's rows past the cache (1000..1023,
    # 500..511) are clamped to its last row before being masked: S = 16
    # (Llama), global S = 16 (Gemma; its local layers read the position
    # first)
    ("llama3b", dict(LLAMA_3B_ATTN, max_seq=1000), 990),
    ("gemma3_4b", dict(GEMMA_4B_ATTN, max_seq=500), 480),
])
def test_decoder_long_cache_matches_oracle(rt, orc, arch, cfg, rows):
    gemma = arch.startswith("gemma")
    rng = np.random.default_rng(rows + len(arch))
    m = Model(orc, "gemma3" if gemma else "llama", rng, **cfg)
    dec = m.load(rt)
    cus = cu_count()
    try:
        prefill(m, dec, rng, rows)
        n_kv, hd = cfg["n_kv_heads"], cfg["head_dim"]
        windows = [cfg["sliding_window"] if gemma and li % cfg["global_every"] != cfg["global_every"] - 1 else 0
                   for li in range(cfg["n_layers"])]
        worst = 0.0
        for i, tok in enumerate(rng.integers(0, cfg["vocab"], 4)):
            pos = rows + i
            for li, win in enumerate(windows):
                S = split_rule(n_kv, 1, win if win else cfg["max_seq"], cus, hd)
                length = min(pos + 1, win) if win else pos + 1
                busy = busy_rule(length, S, hd)
                say(f"[decoder {arch}] pos={pos} layer {li}: window {win}, S={S} splits, {busy} busy")
                assert S > 1 and busy >= 1
            got, idx = dec.step(int(tok), pos, argmax=True)
            want = m.step(int(tok), pos)
            e = normwise_err(got, want)
            worst = max(worst, e)
            assert e <= STEP_TOL, (pos, e)
            assert idx == orc.argmax_first(got), pos
        say(f"[decoder {arch}] {rows} cached positions: worst step normwise error {worst:.2e}")
        if arch == "llama3b" and cfg["max_seq"] == 2048:
            # the cases meant to hold idle splits do
            S = split_rule(n_kv, 1, cfg["max_seq"], cus, hd)
            assert busy_rule(rows + 1, S, hd) < S
    finally:
        dec.close()


# The benchmarked models' layer dimensions (hidden, ffn, heads), two layers
# and a 32768-token vocabulary (the weights drawn on the GPU for speed).
LLAMA_3B_FULL = dict(LLAMA, hidden=3072, n_heads=24, n_kv_heads=8, head_dim=128, ffn=8192, vocab=32768,
                     max_seq=1024, max_batch=0)
GEMMA_4B_FULL = dict(GEMMA, hidden=2560, n_heads=8, n_kv_heads=4, head_dim=256, ffn=10240, vocab=32768,
                     max_seq=1024, sliding_window=512, max_batch=0, embed_scale=float(np.sqrt(np.float32(2560))))


@pytest.mark.parametrize("arch,cfg", [("llama3b", LLAMA_3B_FULL), ("gemma3_4b", GEMMA_4B_FULL)])
def test_decoder_full_dimensions_match_oracle(rt, orc, arch, cfg):
    """The engine at Llama-3.2-3B / Gemma-3-4B layer dimensions, 600 cached
    positions, four steps against the oracle.  Llama: layer 0 in the
    Q4_K_M-style mix (BF16 v in the fused q/k/v + RoPE + KV append launch,
    BF16 SwiGLU down), layer 1 all Q4_K.  Gemma: a local layer whose window
    has slid past position 0 and a global one, the post-norms folded into
    gate/up and into layer 1's q/k/v at K = 2560, the GELU down split 10
    ways at K = 10240, the BF16 lm_head's argmax epilogue."""
    import torch
    say(f"[decoder {arch} full dimensions]")
    g = torch.Generator(device="cuda").manual_seed(11 + len(arch))

    def randn(shape):
        return torch.randn(shape, generator=g, device="cuda").cpu().numpy()

    rng = np.random.default_rng(11 + len(arch))
    gemma = arch.startswith("gemma")
    m = Model(orc, "gemma3" if gemma else "llama", rng, randn=randn, **cfg)
    dec = m.load(rt)
    try:
        prefill(m, dec, rng, 600)
        worst = 0.0
        for i, tok in enumerate(rng.integers(0, cfg["vocab"], 4)):
            pos = 600 + i
            got, idx = dec.step(int(tok), pos, argmax=True)
            want = m.step(int(tok), pos)
            e = normwise_err(got, want)
            worst = max(worst, e)
            assert e <= STEP_TOL, (pos, e)
            assert idx == orc.argmax_first(got), pos
        say(f"[decoder {arch} full dimensions] worst step normwise error {worst:.2e}")
    finally:
        dec.close()


def test_decoder_long_cache_batch_matches_single(rt, orc):
    """A batch step of 4 tokens after 1000 cached positions at the
    Llama-3.2-3B attention geometry (S = 8 splits for 4 rows) gives the
    single-token steps' logits."""
    cfg = dict(LLAMA_3B_ATTN, max_seq=1024, max_batch=4)
    rng = np.random.default_rng(31)
    m = Model(orc, "llama", rng, **cfg)
    a, b = m.load(rt), m.load(rt)
    try:
        state = np.random.default_rng(5)
        prefill(m, a, state, 1000)
        state = np.random.default_rng(5)
        prefill(m, b, state, 1000)
        tokens = rng.integers(0, cfg["vocab"], 4)
        S = split_rule(cfg["n_kv_heads"], 4, cfg["max_seq"], cu_count(), cfg["head_dim"])
        say(f"[decoder llama3b batch] 4 tokens at position 1000, S={S}")
        assert S > 1
        single = []
        for i, tok in enumerate(tokens):
            single.append(a.step(int(tok), 1000 + i))
            want = m.step(int(tok), 1000 + i)
            assert normwise_err(single[-1], want) <= STEP_TOL, i
        batch = b.step_batch(tokens, 1000)
        for i in range(4):
            e = normwise_err(batch[i], single[i])
            assert e <= STEP_TOL, (i, e)
    finally:
        a.close()
        b.close()


def test_decoder_window_beyond_cache_matches_oracle(rt, orc):
    """A sliding window longer than the cache (1024 > max_seq 512) covers every
    position a step reaches: the engine treats it as no window, so its split
    count (and the partials it stores) follow max_seq, never the window."""
    cfg = dict(GEMMA_4B_ATTN, sliding_window=1024, max_batch=0)
    rng = np.random.default_rng(1024)
    m = Model(orc, "gemma3", rng, **cfg)
    dec = m.load(rt)
    try:
        prefill(m, dec, rng, 300)
        for i, tok in enumerate([3, 999, 0]):
            say(f"[decoder gemma3 window 1024 > max_seq 512] pos={300 + i}")
            got = dec.step(tok, 300 + i)
            want = m.step(tok, 300 + i)
            e = normwise_err(got, want)
            assert e <= STEP_TOL, (i, e)
    finally:
        dec.close()
