"""GPU parity for the bf16-MFMA GEMM (prefill / FLUX linears).

Two stated tolerances:
 (i)  against the f32-accumulated product of the same bf16-rounded operands
      (fp64 reference): normwise <= 1e-5;
 (ii) against the reference's f32 CPU path (Q4KMat::matmul_q4k_t's scalar
      loop / MatBf16::matmul_by_t): relative RMS <= 4e-3 -- the bf16 operand
      rounding, the same philosophy as the reference's Metal GEMM test bound
      (tests/test_metal_flux.cpp:140-145).
"""
import numpy as np
import pytest

from helpers import (GEMM_TOL_SAME_OPERANDS, GEMM_TOL_VS_F32_RMS, bf16_bits_to_f32, f32_to_bf16_rne, from_dev,
                     normwise_err, rel_rms, same_operand_err, say, to_dev)

pytestmark = pytest.mark.gpu

CASES = [
    # (M, N, K, a_bf16)
    (128, 128, 256, False),
    (200, 300, 512, False),
    (64, 1000, 768, True),
    (513, 260, 1024, False),
    (9, 64, 256, False),
    (4100, 4000, 512, True),   # enough 256 x 256 tiles for the large-tile kernel, ragged edges
    (32, 3072, 8192, False),   # one M tile: W dequantized by producer waves, K split 8 ways
    (96, 3072, 3072, True),    # K split 6 ways, bf16 A
]


@pytest.mark.parametrize("m,n,k,a_bf16", CASES)
def test_gemm_q4k(rt, orc, m, n, k, a_bf16):
    say(f"[gemm q4k] M={m} N={n} K={k} a_bf16={a_bf16}")
    import torch
    rng = np.random.default_rng(m + n + k)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    a = rng.standard_normal((m, k)).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    blocks = orc.q4k_quantize(w)
    deq = orc.q4k_dequant(blocks, n, k)
    a_bits = f32_to_bf16_rne(a)
    a_r = bf16_bits_to_f32(a_bits).astype(np.float64)
    w_r = bf16_bits_to_f32(f32_to_bf16_rne(deq)).astype(np.float64)
    same = a_r @ w_r.T + bias
    d_a = to_dev(a_bits).view(torch.bfloat16) if a_bf16 else to_dev(a)
    c = from_dev(rt.gemm(rt.Q4K, d_a, to_dev(blocks), n, k, bias=to_dev(bias)))
    assert normwise_err(c, same) <= GEMM_TOL_SAME_OPERANDS
    if m * n * k <= 64 * 1024 * 1024:
        ref = orc.q4k_matmul_t(blocks, n, k, a if not a_bf16 else bf16_bits_to_f32(a_bits)) + bias
        assert rel_rms(c, ref) <= GEMM_TOL_VS_F32_RMS


@pytest.mark.parametrize("m,n,k,a_bf16", [(128, 128, 128, False), (300, 200, 576, True),
                                         (17, 520, 192, False), (4133, 4044, 256, True)])
def test_gemm_bf16(rt, orc, m, n, k, a_bf16):
    say(f"[gemm bf16] M={m} N={n} K={k}")
    import torch
    rng = np.random.default_rng(m * n + k)
    wb = orc.f32_to_bf16_n((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    a = rng.standard_normal((m, k)).astype(np.float32)
    a_bits = f32_to_bf16_rne(a)
    same = bf16_bits_to_f32(a_bits).astype(np.float64) @ bf16_bits_to_f32(wb).astype(np.float64).T
    d_a = to_dev(a_bits).view(torch.bfloat16) if a_bf16 else to_dev(a)
    c = from_dev(rt.gemm(rt.BF16, d_a, to_dev(wb), n, k))
    assert normwise_err(c, same) <= GEMM_TOL_SAME_OPERANDS
    ref = orc.bf16_matmul_t(wb, a)
    assert rel_rms(c, ref) <= GEMM_TOL_VS_F32_RMS


def test_gemm_prefill_shape_properties(rt):
    """BASELINE config 4 gate shape (M=512, N=8192, K=3072) at full size:
    GEMM of the GPU-quantized weight equals the product with its bf16
    dequantization, computed in float64 on sampled columns (tolerance (i))."""
    import torch
    m, n, k = 512, 8192, 3072
    g = torch.Generator(device="cuda").manual_seed(1)
    w = torch.randn((n, k), generator=g, device="cuda") * 0.02
    a = torch.randn((m, k), generator=g, device="cuda")
    blocks = rt.quantize_q4k(w)
    wd = rt.dequant_q4k(blocks, n, k, bf16=True).view(torch.bfloat16)
    c = rt.gemm(rt.Q4K, a, blocks, n, k)
    err = same_operand_err(c, a, wd, seed=1)
    say(f"[gemm prefill gate shape] same-operand normwise {err:.2e} (float64, 64 columns)")
    assert err <= GEMM_TOL_SAME_OPERANDS


def test_gemm_flux_shape_properties(rt):
    """BASELINE config 5 MLP-in shape (M=4608, N=12288, K=3072, bf16 A) at
    full size, through the large-tile kernel: equals the product of the
    same bf16 operands (float64 on sampled columns, tolerance (i))."""
    import torch
    m, n, k = 4608, 12288, 3072
    g = torch.Generator(device="cuda").manual_seed(2)
    w = torch.randn((n, k), generator=g, device="cuda") * 0.02
    a = torch.randn((m, k), generator=g, device="cuda").bfloat16()
    blocks = rt.quantize_q4k(w)
    wd = rt.dequant_q4k(blocks, n, k, bf16=True).view(torch.bfloat16)
    c = rt.gemm(rt.Q4K, a, blocks, n, k)
    err = same_operand_err(c, a, wd, seed=2)
    say(f"[gemm flux MLP-in shape] same-operand normwise {err:.2e} (float64, 64 columns)")
    assert err <= GEMM_TOL_SAME_OPERANDS


@pytest.mark.parametrize("m,n,k", [(2304, 6400, 1024), (2304, 6400, 12288)])
def test_gemm_large_tile_partial_round(rt, m, n, k):
    """225 tiles of 256 x 256 (fewer than the CUs), short and long K, N not a
    multiple of the tile: equals the product of the same bf16 operands
    (float64 on sampled columns, tolerance (i)), and two runs agree bit for
    bit."""
    import torch
    g = torch.Generator(device="cuda").manual_seed(m + k)
    a = torch.randn((m, k), generator=g, device="cuda").bfloat16()
    wb = (torch.randn((n, k), generator=g, device="cuda") * 0.02).bfloat16()
    c1 = rt.gemm(rt.BF16, a, wb.view(torch.int16), n, k)
    c2 = rt.gemm(rt.BF16, a, wb.view(torch.int16), n, k)
    err = same_operand_err(c1, a, wb, seed=k)
    say(f"[gemm large tile] {m}x{n}x{k} same-operand normwise {err:.2e} (float64, 64 columns)")
    assert err <= GEMM_TOL_SAME_OPERANDS
    assert torch.equal(c1.view(torch.int32), c2.view(torch.int32))


@pytest.mark.parametrize("m,n,k", [(3000, 5000, 1024), (4100, 4000, 512), (4608, 3072, 2048)])
def test_gemm_large_tile_bias(rt, m, n, k):
    """The large-tile kernel with a bias: 240 tiles (ragged M and N), 272
    tiles (a second round of 16) and 216 tiles (the FLUX MLP-out tile grid):
    the output equals the float64 product of the same bf16 operands plus the
    bias (tolerance (i)), and a second run agrees bit for bit."""
    import torch
    say(f"[gemm large tile + bias] {m}x{n}x{k}")
    g = torch.Generator(device="cuda").manual_seed(m + n + k)
    a = torch.randn((m, k), generator=g, device="cuda").bfloat16()
    wb = (torch.randn((n, k), generator=g, device="cuda") * 0.02).bfloat16()
    bias = torch.randn(n, generator=g, device="cuda")
    c1 = rt.gemm(rt.BF16, a, wb.view(torch.int16), n, k, bias=bias)
    c2 = rt.gemm(rt.BF16, a, wb.view(torch.int16), n, k, bias=bias)
    err = same_operand_err(c1 - bias, a, wb, seed=n)
    say(f"[gemm large tile + bias] {m}x{n}x{k} same-operand normwise {err:.2e} (float64, 64 columns)")
    assert err <= GEMM_TOL_SAME_OPERANDS
    assert torch.equal(c1.view(torch.int32), c2.view(torch.int32))


@pytest.mark.parametrize("m,n,k,a_bf16", [(256, 8192, 3072, False), (200, 1000, 1024, True),
                                         (160, 3072, 8192, False), (512, 3072, 8192, False),
                                         (512, 8192, 3072, False), (1000, 4096, 4096, False),
                                         (700, 2048, 1024, False), (384, 3072, 3072, True)])
def test_gemm_q4k_bit_identical_to_bf16_path(rt, m, n, k, a_bf16):
    """Up to two 128-row M tiles (eight when N >= K), a Q4_K weight is
    dequantized inside the GEMM by producer waves (w = (d*sv)*q - dmin*mv,
    RNE bf16) beside the MFMA waves; otherwise once into the workspace.
    Either way, with the same K split, every output equals, bit for bit, the
    bf16 GEMM on the dequantized weight (the same MFMA order), bias
    included: gate and down shapes at 160, 200 and 256 rows (the in-GEMM
    path, K split 2 and 4, ragged M and N, bf16 A), config 4's down (the
    workspace path), gate and N = 2K shapes at 512 and 700 rows (in-GEMM
    with A converted to bf16 first, K split 2 at 700), a square one at 1000
    rows (workspace) and at 384 rows with bf16 A (in-GEMM, K split 3)."""
    import torch
    say(f"[gemm q4k vs bf16 path] M={m} N={n} K={k} a_bf16={a_bf16}")
    g = torch.Generator(device="cuda").manual_seed(m + n + k)
    blocks = rt.quantize_q4k(torch.randn((n, k), generator=g, device="cuda") * 0.02)
    wbf = rt.dequant_q4k(blocks, n, k, bf16=True)
    a = torch.randn((m, k), generator=g, device="cuda")
    if a_bf16:
        a = a.bfloat16()
    bias = torch.randn(n, generator=g, device="cuda")
    c1 = rt.gemm(rt.Q4K, a, blocks, n, k, bias=bias)
    c2 = rt.gemm(rt.BF16, a, wbf, n, k, bias=bias)
    assert torch.equal(c1.view(torch.int32), c2.view(torch.int32))
    c3 = rt.gemm(rt.Q4K, a, blocks, n, k, bias=bias)
    assert torch.equal(c1.view(torch.int32), c3.view(torch.int32))
