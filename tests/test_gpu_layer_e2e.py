"""One whole Llama decode layer through the fused launches, end to end.

The launch sequence is the decode token's (bench.py --workload decode_layers,
one layer of it): RMSNorm + q/k/v + RoPE + KV append, attention over the
cache, o + residual, RMSNorm + gate/up, SwiGLU + down + residual.  The
expected value is the oracle's composition of the reference's operations
(LlamaBlock::forward_cached, src/transformer5.cpp:198-212):
    h   = x + o(attn(rope(q(n1)), rope(k(n1)) -> cache, v(n1) -> cache))
    out = h + down(silu(gate(n2)) * up(n2)),  n1 = rmsnorm(x), n2 = rmsnorm(h)
with every product in the reference's sequential f32 order.

Tolerance: the layer output is held to the per-GEMV bar itself, 1e-5
normwise, although it passes each stage's rounding on through four dependent
products, the softmax and the residual adds (measured: 1.2e-6 to 2.7e-6; the
figures are printed).  The widened form (Q4_K_M: BF16 v and down) runs
through the BF16 q/k/v and SwiGLU launches instead.
"""
import numpy as np
import pytest

from helpers import from_dev, normwise_err, say, to_dev

pytestmark = pytest.mark.gpu
LAYER_TOL = 1e-5

HIDDEN, FFN, NQ, NKV, HD = 3072, 8192, 24, 8, 128


def oracle_layer(orc, W, x, kc, vc, pos, inv, eps, widened):
    """The reference layer on the CPU; kc / vc [>= pos + 1, NKV * HD] are
    updated at row pos as LlamaLayerKvCache::append does."""
    k = HIDDEN
    n1 = orc.rmsnorm(x, W["g1"], eps).reshape(1, k)
    q = orc.q4k_matmul_t(W["q"], NQ * HD, k, n1).reshape(-1)
    kk = orc.q4k_matmul_t(W["k"], NKV * HD, k, n1).reshape(-1)
    if widened:
        v = orc.bf16_matmul_t(W["v"], n1).reshape(-1)
    else:
        v = orc.q4k_matmul_t(W["v"], NKV * HD, k, n1).reshape(-1)
    q = orc.llama_rope(q, NQ, HD, pos, inv)
    kk = orc.llama_rope(kk, NKV, HD, pos, inv)
    kc = kc.copy()
    vc = vc.copy()
    kc[pos] = kk
    vc[pos] = v
    scale = float(1.0 / np.sqrt(np.float32(HD)))
    attn = orc.gqa_attention_decode(q, kc, vc, pos + 1, NQ, NKV, HD, scale).reshape(1, k)
    h = x + orc.q4k_matmul_t(W["o"], k, k, attn).reshape(-1)
    n2 = orc.rmsnorm(h, W["g2"], eps).reshape(1, k)
    gate = orc.q4k_matmul_t(W["gate"], FFN, k, n2).reshape(-1)
    up = orc.q4k_matmul_t(W["up"], FFN, k, n2).reshape(-1)
    act = orc.swiglu(gate, up).reshape(1, FFN)
    if widened:
        d = orc.bf16_matmul_t(W["down"], act).reshape(-1)
    else:
        d = orc.q4k_matmul_t(W["down"], k, FFN, act).reshape(-1)
    return h + d, kc, vc, h


def make_layer(orc, rng, widened):
    def q4(n, k):
        return orc.q4k_quantize((rng.standard_normal((n, k)) * 0.02).astype(np.float32))

    def bf(n, k):
        return orc.f32_to_bf16_n((rng.standard_normal((n, k)) * 0.02).astype(np.float32))

    W = {"q": q4(NQ * HD, HIDDEN), "k": q4(NKV * HD, HIDDEN),
         "v": bf(NKV * HD, HIDDEN) if widened else q4(NKV * HD, HIDDEN),
         "o": q4(HIDDEN, HIDDEN), "gate": q4(FFN, HIDDEN), "up": q4(FFN, HIDDEN),
         "down": bf(HIDDEN, FFN) if widened else q4(HIDDEN, FFN),
         "g1": (1.0 + 0.1 * rng.standard_normal(HIDDEN)).astype(np.float32),
         "g2": (1.0 + 0.1 * rng.standard_normal(HIDDEN)).astype(np.float32)}
    return W


@pytest.mark.parametrize("widened,pos", [(False, 0), (False, 37), (True, 37), (True, 300)])
def test_llama_layer_end_to_end(rt, orc, widened, pos):
    import torch
    say(f"[layer e2e] widened={widened} pos={pos}")
    rng = np.random.default_rng(1000 + pos + (7 if widened else 0))
    W = make_layer(orc, rng, widened)
    x = rng.standard_normal(HIDDEN).astype(np.float32)
    cap = pos + 3
    kc = rng.standard_normal((cap, NKV * HD)).astype(np.float32)
    vc = rng.standard_normal((cap, NKV * HD)).astype(np.float32)
    kc[pos:] = 0.0
    vc[pos:] = 0.0
    inv = orc.llama_inv_freq(500000.0, HD)
    eps = 1e-5
    want, kc_want, vc_want, h_want = oracle_layer(orc, W, x, kc, vc, pos, inv, eps, widened)

    # device: the fused launch sequence of one decode layer
    tq = rt.q4k_tile(to_dev(W["q"]), NQ * HD, HIDDEN)
    tk = rt.q4k_tile(to_dev(W["k"]), NKV * HD, HIDDEN)
    to = rt.q4k_tile(to_dev(W["o"]), HIDDEN, HIDDEN)
    tg = rt.q4k_tile(to_dev(W["gate"]), FFN, HIDDEN)
    tu = rt.q4k_tile(to_dev(W["up"]), FFN, HIDDEN)
    d_kc, d_vc = to_dev(kc), to_dev(vc)
    resid = to_dev(x).reshape(1, HIDDEN)
    d_g1, d_g2, d_inv = to_dev(W["g1"]), to_dev(W["g2"]), to_dev(inv)
    q = torch.empty((1, NQ * HD), device="cuda")
    attn = torch.empty((1, HIDDEN), device="cuda")
    gate = torch.empty((1, FFN), device="cuda")
    up = torch.empty((1, FFN), device="cuda")
    krow, vrow = d_kc[pos:pos + 1], d_vc[pos:pos + 1]
    if widened:
        rt.gemv_q4k_tiled_bf16_rmsnorm([tq, tk], [NQ * HD, NKV * HD], to_dev(W["v"].view(np.int16)), NKV * HD,
                                       resid, d_g1, eps, HIDDEN, ys=[q, krow], yb=vrow,
                                       rope=(d_inv, pos, HD, 0x3))
    else:
        tv = rt.q4k_tile(to_dev(W["v"]), NKV * HD, HIDDEN)
        rt.gemv_q4k_tiled_rmsnorm_rope([tq, tk, tv], resid, d_g1, eps, [NQ * HD, NKV * HD, NKV * HD], HIDDEN,
                                       d_inv, pos, HD, 0x3, ys=[q, krow, vrow])
    scale = float(1.0 / np.sqrt(np.float32(HD)))
    rt.attention_decode(q, d_kc, d_vc, pos + 1, NQ, NKV, scale, out=attn)
    rt.gemv_q4k_tiled_residual(to, attn, resid, HIDDEN, HIDDEN)
    h = from_dev(resid).reshape(-1).copy()
    rt.gemv_q4k_tiled_rmsnorm_multi([tg, tu], resid, d_g2, eps, [FFN, FFN], HIDDEN, ys=[gate, up])
    if widened:
        rt.gemv_swiglu_residual(rt.BF16, to_dev(W["down"].view(np.int16)), gate, up, resid, HIDDEN, FFN)
    else:
        td = rt.q4k_tile(to_dev(W["down"]), HIDDEN, FFN)
        rt.gemv_swiglu_residual(rt.Q4K, td, gate, up, resid, HIDDEN, FFN)
    got = from_dev(resid).reshape(-1)

    e_h = normwise_err(h, h_want)
    e_out = normwise_err(got, want)
    e_k = normwise_err(from_dev(d_kc)[pos], kc_want[pos])
    e_v = normwise_err(from_dev(d_vc)[pos], vc_want[pos])
    say(f"[layer e2e] errors: h {e_h:.2e}, out {e_out:.2e}, k row {e_k:.2e}, v row {e_v:.2e}")
    assert e_k <= 1e-5 and e_v <= 1e-5
    assert e_h <= LAYER_TOL and e_out <= LAYER_TOL
    # rows other than pos are untouched
    others = [r for r in range(cap) if r != pos]
    assert np.array_equal(from_dev(d_kc)[others], kc[others])
    assert np.array_equal(from_dev(d_vc)[others], vc[others])
