"""GPU parity at the BASELINE configurations' full sizes.

* The Llama-3.2-3B lm_head, 128256 x 3072 Q4_K (the decode step's largest
  launch: 8016 tiles), tiled and RMSNorm-fused, against the oracle's
  reference-order f32 product over every row (1e-5 normwise).  The weight is
  quantized on the GPU by the library's quantizer, which is byte-identical to
  Q4KMat::quantize (test_gpu_quant.py); its bytes come back for the oracle.
* The GEMMs of configs 4 and 5 at full size: prefill down (M=512, N=3072,
  K=8192), FLUX QKV (4608 x 9216 x 3072) and MLP-out (4608 x 3072 x 12288),
  against (i) the product of the same bf16-rounded operands in float64 on
  64 sampled output columns (normwise 1e-5, GEMM_TOL_SAME_OPERANDS), and
  (ii) the reference's f32 CPU loop (Q4KMat::matmul_q4k_t,
  src/quant_q4k.cpp:602-624) on 64 sampled output columns, relative RMS
  within GEMM_TOL_VS_F32_RMS.
"""
import numpy as np
import pytest

from helpers import (GEMM_TOL_SAME_OPERANDS, GEMM_TOL_VS_F32_RMS, GEMV_TOL, from_dev, normwise_err, rel_rms,
                     same_operand_err, say, to_dev)

pytestmark = pytest.mark.gpu
VOCAB, HIDDEN = 128256, 3072


@pytest.fixture(scope="module")
def lm_head(rt):
    import torch
    g = torch.Generator(device="cuda").manual_seed(11)
    w = torch.randn((VOCAB, HIDDEN), generator=g, device="cuda") * 0.02
    blocks = rt.quantize_q4k(w)
    del w
    torch.cuda.synchronize()
    return blocks, from_dev(blocks)


def test_lm_head_full_tiled(rt, orc, lm_head):
    say("[full size] lm_head 128256x3072 tiled")
    d_blocks, blocks = lm_head
    rng = np.random.default_rng(5)
    x = rng.standard_normal((1, HIDDEN)).astype(np.float32)
    t = rt.q4k_tile(d_blocks, VOCAB, HIDDEN)
    got = from_dev(rt.gemv_q4k_tiled(t, to_dev(x), VOCAB, HIDDEN))
    want = orc.q4k_matmul_t(blocks, VOCAB, HIDDEN, x)
    err = normwise_err(got, want)
    say(f"[full size] lm_head tiled normwise {err:.2e}")
    assert err <= GEMV_TOL
    assert orc.argmax_first(got.reshape(-1)) == orc.argmax_first(want.reshape(-1))
    rows = from_dev(rt.gemv(rt.Q4K, d_blocks, to_dev(x), VOCAB, HIDDEN))
    assert np.array_equal(rows.view(np.uint32), got.view(np.uint32))


def test_lm_head_full_rmsnorm_fused(rt, orc, lm_head):
    say("[full size] lm_head 128256x3072 RMSNorm-fused")
    d_blocks, blocks = lm_head
    rng = np.random.default_rng(6)
    x = (rng.standard_normal(HIDDEN) * 3).astype(np.float32)
    gamma = (1.0 + 0.1 * rng.standard_normal(HIDDEN)).astype(np.float32)
    t = rt.q4k_tile(d_blocks, VOCAB, HIDDEN)
    (y,) = rt.gemv_q4k_tiled_rmsnorm_multi([t], to_dev(x), to_dev(gamma), 1e-5, [VOCAB], HIDDEN)
    xn = orc.rmsnorm(x, gamma, 1e-5).reshape(1, HIDDEN)
    want = orc.q4k_matmul_t(blocks, VOCAB, HIDDEN, xn)
    err = normwise_err(from_dev(y), want)
    say(f"[full size] lm_head rmsnorm-fused normwise {err:.2e}")
    assert err <= GEMV_TOL


GEMM_FULL = [
    (512, 3072, 8192, False, "config 4 prefill down"),
    (4608, 9216, 3072, True, "config 5 FLUX QKV"),
    (4608, 3072, 12288, True, "config 5 FLUX MLP-out"),
]


@pytest.mark.parametrize("m,n,k,a_bf16,note", GEMM_FULL)
def test_gemm_full_size(rt, orc, m, n, k, a_bf16, note):
    import torch
    say(f"[full size] GEMM M={m} N={n} K={k} ({note})")
    g = torch.Generator(device="cuda").manual_seed(m + n + k)
    w = torch.randn((n, k), generator=g, device="cuda") * 0.02
    a = torch.randn((m, k), generator=g, device="cuda")
    if a_bf16:
        a = a.bfloat16()
    blocks = rt.quantize_q4k(w)
    del w
    c = rt.gemm(rt.Q4K, a, blocks, n, k)
    # (i) same bf16 operands, float64 product on 64 sampled output columns
    wd = rt.dequant_q4k(blocks, n, k, bf16=True).view(torch.bfloat16)
    err = same_operand_err(c, a, wd, seed=n)
    say(f"[full size] (i) same-operand normwise {err:.2e} (float64, 64 columns)")
    assert err <= GEMM_TOL_SAME_OPERANDS
    del wd
    # (ii) the reference's f32 CPU loop on 64 sampled output columns
    cols = np.sort(np.random.default_rng(n).choice(n, 64, replace=False))
    hb = from_dev(blocks).reshape(n, -1)[cols].reshape(-1)
    ah = from_dev(a.float())
    want = orc.q4k_matmul_t(hb, 64, k, ah)
    got = from_dev(c)[:, cols]
    rr = rel_rms(got, want)
    say(f"[full size] (ii) vs f32 CPU loop rel RMS {rr:.2e}")
    assert rr <= GEMM_TOL_VS_F32_RMS
