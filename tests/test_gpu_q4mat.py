"""GPU parity for the reference's Q4Mat format and the 4-bit formats at any M.

* Q4Mat dequantization: bit-exact against the oracle's Q4Mat::dequantize
  restatement (quant_q4.cpp:67-74), and its bf16 form is the RNE of that.
* Q4Mat GEMV (M <= 8) against the oracle's Q4Mat::matmul_q4_t restatement
  (quant_q4.cpp:92-114): normwise 1e-5.
* GEMM for Q4Mat and GGUF Q4_0 at M > 8 (decoded to bf16 inside the GEMM
  up to two 128-row M tiles, else once into the workspace, then the bf16
  MFMA kernels): (i) normwise 1e-5 against the f32 product of the same
  bf16-rounded operands, (ii) relative RMS within GEMM_TOL_VS_F32_RMS against
  the reference's f32 loop; and bit-identical to the bf16 GEMM on the
  dequantized weight where both split K alike.
* rt_hip_linear_forward over every storage Linear2::fused_linear holds
  (nn2.cpp:143-203: Q4Mat, Q4_K, BF16, and GGUF Q4_0) at M in {1, 8, 64, 512},
  with a bias (qlinear.cpp:42-53).
"""
import numpy as np
import pytest

from helpers import (GEMM_TOL_SAME_OPERANDS, GEMM_TOL_VS_F32_RMS, GEMV_TOL, bf16_bits_to_f32, f32_to_bf16_rne,
                     from_dev, normwise_err, rel_rms, say, to_dev)

pytestmark = pytest.mark.gpu


def q4mat(orc, rng, n, k):
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    packed, scales = orc.q4mat_quantize(w)
    return packed, scales


@pytest.mark.parametrize("n,k", [(300, 1024), (4096, 4096), (37, 32), (1000, 3072)])
def test_q4mat_dequant_bit_exact(rt, orc, n, k):
    say(f"[q4mat dequant] N={n} K={k}")
    rng = np.random.default_rng(n + k)
    packed, scales = q4mat(orc, rng, n, k)
    # every nibble value, including -8 which the quantizer never writes
    packed[: 64] = np.arange(64, dtype=np.uint8) * 17
    want = orc.q4mat_dequant(packed, scales, n * k).reshape(n, k)
    w = rt.q4mat_upload(packed, scales, n, k)
    got = from_dev(rt.dequant(rt.Q4MAT, w, n, k))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    got16 = from_dev(rt.dequant(rt.Q4MAT, w, n, k, bf16=True)).view(np.uint16)
    assert np.array_equal(got16, orc.f32_to_bf16_n(want))


@pytest.mark.parametrize("n,k", [(256, 1024), (4096, 4096)])
def test_q4_0_dequant_bit_exact(rt, orc, n, k):
    say(f"[q4_0 dequant] N={n} K={k}")
    rng = np.random.default_rng(2 * n + k)
    blocks = orc.q4_0_quantize((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    want = orc.q4_0_decode(blocks, n * k).reshape(n, k)
    got = from_dev(rt.dequant(rt.Q4_0, to_dev(blocks), n, k))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("n,k,m", [(4096, 4096, 1), (1000, 3072, 1), (37, 32, 1), (513, 1024, 3),
                                   (4096, 4096, 8), (300, 2048, 8), (64, 15872, 1)])
def test_q4mat_gemv(rt, orc, n, k, m):
    say(f"[q4mat gemv] N={n} K={k} M={m}")
    rng = np.random.default_rng(n * 7 + k + m)
    packed, scales = q4mat(orc, rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    want = orc.q4mat_matmul_t(packed, scales, n, k, x)
    got = from_dev(rt.gemv(rt.Q4MAT, rt.q4mat_upload(packed, scales, n, k), to_dev(x), n, k))
    for r in range(m):
        assert normwise_err(got[r], want[r]) <= GEMV_TOL, (r, normwise_err(got[r], want[r]))


def test_q4mat_gemv_one_hot_is_exact(rt, orc):
    """x = e_j: every partial sum is exact, so y is column j of the
    dequantized weight, bit for bit."""
    n, k = 200, 1024
    rng = np.random.default_rng(3)
    packed, scales = q4mat(orc, rng, n, k)
    deq = orc.q4mat_dequant(packed, scales, n * k).reshape(n, k)
    w = rt.q4mat_upload(packed, scales, n, k)
    for col in (0, 1, 31, 32, 511, 1023):
        x = np.zeros((1, k), np.float32)
        x[0, col] = 1.0
        y = from_dev(rt.gemv(rt.Q4MAT, w, to_dev(x), n, k))[0]
        assert np.array_equal(y.view(np.uint32), deq[:, col].view(np.uint32)), col


@pytest.mark.parametrize("fmt_name,m,n,k", [("q4mat", 64, 1024, 1024), ("q4mat", 512, 4096, 4096),
                                            ("q4_0", 64, 512, 2048), ("q4_0", 512, 4096, 4096),
                                            ("q4mat", 300, 1000, 3072), ("q4mat", 16, 4096, 4096),
                                            ("q4_0", 32, 3072, 8192), ("q4_0", 200, 1000, 1024)])
def test_4bit_gemm(rt, orc, fmt_name, m, n, k):
    say(f"[4-bit gemm] {fmt_name} M={m} N={n} K={k}")
    rng = np.random.default_rng(m + n + k)
    w32 = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    if fmt_name == "q4mat":
        packed, scales = orc.q4mat_quantize(w32)
        dw = rt.q4mat_upload(packed, scales, n, k)
        fmt = rt.Q4MAT
    else:
        blocks = orc.q4_0_quantize(w32)
        packed, scales = orc.q4_0_to_q4mat(blocks, n * k)
        dw = to_dev(blocks)
        fmt = rt.Q4_0
    deq = orc.q4mat_dequant(packed, scales, n * k).reshape(n, k)
    a = rng.standard_normal((m, k)).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    c = from_dev(rt.gemm(fmt, to_dev(a), dw, n, k, bias=to_dev(bias)))
    same = (bf16_bits_to_f32(f32_to_bf16_rne(a)).astype(np.float64)
            @ bf16_bits_to_f32(f32_to_bf16_rne(deq)).astype(np.float64).T) + bias
    assert normwise_err(c, same) <= GEMM_TOL_SAME_OPERANDS
    rows = slice(0, min(m, 64))
    ref = orc.q4mat_matmul_t(packed, scales, n, k, a[rows]) + bias
    rr = rel_rms(c[rows], ref)
    say(f"[4-bit gemm] rel RMS vs f32 loop {rr:.2e}")
    assert rr <= GEMM_TOL_VS_F32_RMS


@pytest.mark.parametrize("m", [1, 8, 64, 512])
def test_linear_forward_every_format(rt, orc, m):
    """Linear2::fused_linear's storages through one entry point, with a bias."""
    n, k = 1024, 2048
    say(f"[linear_forward] every format M={m}")
    rng = np.random.default_rng(40 + m)
    w32 = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    tol_gemv = GEMV_TOL
    packed, scales = orc.q4mat_quantize(w32)
    q4kb = orc.q4k_quantize(w32)
    q40 = orc.q4_0_quantize(w32)
    p0, s0 = orc.q4_0_to_q4mat(q40, n * k)
    wbf = orc.f32_to_bf16_n(w32)
    cases = [
        (rt.Q4MAT, rt.q4mat_upload(packed, scales, n, k), lambda a: orc.q4mat_matmul_t(packed, scales, n, k, a)),
        (rt.Q4K, to_dev(q4kb), lambda a: orc.q4k_matmul_t(q4kb, n, k, a)),
        (rt.Q4_0, to_dev(q40), lambda a: orc.q4mat_matmul_t(p0, s0, n, k, a)),
        (rt.BF16, to_dev(wbf.view(np.int16)), lambda a: orc.bf16_matmul_t(wbf, a)),
    ]
    for fmt, dw, ref_fn in cases:
        y = from_dev(rt.linear_forward(fmt, dw, to_dev(x), n, k, bias=to_dev(bias)))
        rows = slice(0, min(m, 16))
        want = ref_fn(x[rows]) + bias
        if m <= 8:
            for r in range(m):
                assert normwise_err(y[r], want[r]) <= tol_gemv, (fmt, r)
        else:
            assert rel_rms(y[rows], want) <= GEMM_TOL_VS_F32_RMS, fmt


@pytest.mark.parametrize("fmt_name", ["q4mat", "q4_0"])
@pytest.mark.parametrize("m,n,k,a_bf16", [(200, 1000, 1024, False), (160, 3072, 8192, True),
                                         (600, 8192, 3072, False), (512, 4096, 4096, True),
                                         (384, 2048, 1024, False)])
def test_4bit_gemm_in_kernel_decode_bit_identical(rt, orc, fmt_name, m, n, k, a_bf16):
    """Up to two M tiles (eight when N >= 2K, four when N >= K with bf16 A;
    beyond two an f32 A is converted to bf16 first) the 4-bit weight is
    decoded inside the GEMM (signed
    nibble x f32 scale, or (q - 8) x d, then RNE bf16); with the same K split
    every output equals, bit for bit, the bf16 GEMM on the dequantized
    weight.  Every Q4Mat nibble value (-8 included) appears."""
    import torch
    say(f"[4-bit gemm in-kernel] {fmt_name} M={m} N={n} K={k} a_bf16={a_bf16}")
    rng = np.random.default_rng(m * 3 + n + k)
    w32 = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    if fmt_name == "q4mat":
        packed, scales = orc.q4mat_quantize(w32)
        packed[: 256] = np.arange(256, dtype=np.uint8)
        dw = rt.q4mat_upload(packed, scales, n, k)
        fmt = rt.Q4MAT
    else:
        dw = to_dev(orc.q4_0_quantize(w32))
        fmt = rt.Q4_0
    wbf = rt.dequant(fmt, dw, n, k, bf16=True)
    a = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).cuda()
    if a_bf16:
        a = a.bfloat16()
    bias = torch.from_numpy(rng.standard_normal(n).astype(np.float32)).cuda()
    c1 = rt.gemm(fmt, a, dw, n, k, bias=bias)
    c2 = rt.gemm(rt.BF16, a, wbf, n, k, bias=bias)
    assert torch.equal(c1.view(torch.int32), c2.view(torch.int32))
