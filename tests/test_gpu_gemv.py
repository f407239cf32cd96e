"""GPU parity: the gfx950 GEMV kernels (through the C ABI) against the oracle.

Tolerance (BASELINE: max relative error <= 1e-5 vs f32 accumulation),
stated normwise because the kernels sum in a different order than the
reference's sequential dot_row:
    max_i |y_gpu - y_ref| <= 1e-5 * max_i |y_ref|
checked against the oracle's reference-order f32 output and an fp64
brute-force product of the same dequantized weights.
"""
import numpy as np
import pytest

from helpers import GEMV_TOL, from_dev, normwise_err, say, to_dev

pytestmark = pytest.mark.gpu

Q4K_CASES = [
    # (N, K, M, note)
    (6912, 1024, 1, "config 1, reference Release semantics (K=1152 -> 4 super-blocks)"),
    (6912, 1280, 1, "config 1, zero-padded to K=1280"),
    (3072, 3072, 1, "llama q/o"),
    (1024, 3072, 1, "llama k/v"),
    (8192, 3072, 1, "llama gate/up"),
    (3072, 8192, 1, "llama down"),
    (130, 256, 1, "ragged N, one super-block"),
    (33, 2304, 1, "K=9 super-blocks (8 lanes per row)"),
    (513, 768, 2, "K=3 super-blocks, M=2"),
    (100, 3072, 8, "speculative batch M=8"),
    (8192, 3072, 8, "llama gate/up, M=8: K-slices summed in order"),
    (3072, 8192, 5, "llama down, M=5: a part-filled row group"),
    (1000, 768, 4, "ragged N, M=4"),
    (3072, 3072, 2, "llama q/o, M=2"),
    (7, 512, 3, "tiny N"),
    (1, 12288, 1, "single row, K=12288"),
    (2560, 10240, 1, "gemma-3-4b down: K split 10 ways"),
]


@pytest.mark.parametrize("n,k,m,note", Q4K_CASES)
def test_q4k_gemv_matches_oracle(rt, orc, n, k, m, note):
    say(f"[q4k gemv] N={n} K={k} M={m} ({note})")
    rng = np.random.default_rng(n * 31 + k + m)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    blocks = orc.q4k_quantize(w)
    y_ref = orc.q4k_matmul_t(blocks, n, k, x)
    y = from_dev(rt.gemv(rt.Q4K, to_dev(blocks), to_dev(x), n, k))
    assert normwise_err(y, y_ref) <= GEMV_TOL, normwise_err(y, y_ref)
    if n * k <= 4 * 1024 * 1024:
        exact = x.astype(np.float64) @ orc.q4k_dequant(blocks, n, k).astype(np.float64).T
        assert normwise_err(y, exact) <= GEMV_TOL


def test_q4k_gemv_config1_release_semantics(rt, orc):
    """W 6912x1152 quantized by the reference's Release
    quantizer keeps 4 super-blocks per row.  The boundary rejects K=1152;
    the reference's result is the K=1024 product of the same bytes."""
    say("[q4k gemv] config 1 6912x1152 via InitRng seed 0")
    w = orc.initrng_normal(0, 6912 * 1152, 0.02).reshape(6912, 1152)
    x = orc.initrng_normal(1, 1152, 1.0)
    blocks = orc.q4k_quantize(w)                 # Release: 4 blocks per row
    assert blocks.size == 6912 * 4 * 144
    y_ref = orc.q4k_matmul_t(blocks, 6912, 1152, x)  # reference semantics
    lib = rt.library()
    d_blocks, d_x = to_dev(blocks), to_dev(x)
    import torch
    d_y = torch.empty(6912, dtype=torch.float32, device="cuda")
    assert lib.status("rt_hip_gemv_q4k", d_blocks.data_ptr(), d_x.data_ptr(), d_y.data_ptr(),
                      6912, 1152, 1, None) == 3
    y = from_dev(rt.gemv(rt.Q4K, d_blocks, to_dev(x[:1024]), 6912, 1024))
    assert normwise_err(y, y_ref) <= GEMV_TOL


def test_q4k_gemv_one_hot_is_exact(rt, orc):
    """x = e_k: every partial sum is exact, so y must be column k of the
    dequantized weight bit-for-bit, whatever the summation order."""
    rng = np.random.default_rng(4)
    n, k = 300, 1024
    blocks = orc.q4k_quantize((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    deq = orc.q4k_dequant(blocks, n, k)
    d_blocks = to_dev(blocks)
    for col in (0, 15, 16, 31, 32, 47, 63, 64, 255, 256, 777, 1023):
        x = np.zeros(k, np.float32)
        x[col] = 1.0
        y = from_dev(rt.gemv(rt.Q4K, d_blocks, to_dev(x), n, k))[0]
        assert np.array_equal(y.view(np.uint32), deq[:, col].view(np.uint32)), col


def test_q4k_gemv_linearity_full_size(rt, orc):
    """Full Llama gate shape: y(a*x1 + x2) == a*y(x1) + y(x2) to f32 rounding."""
    import torch
    n, k = 8192, 3072
    g = torch.Generator(device="cuda").manual_seed(0)
    w = torch.randn((n, k), generator=g, device="cuda") * 0.02
    blocks = rt.quantize_q4k(w)
    x1 = torch.randn((1, k), generator=g, device="cuda")
    x2 = torch.randn((1, k), generator=g, device="cuda")
    y1 = rt.gemv(rt.Q4K, blocks, x1, n, k)
    y2 = rt.gemv(rt.Q4K, blocks, x2, n, k)
    y12 = rt.gemv(rt.Q4K, blocks, 0.5 * x1 + x2, n, k)
    assert normwise_err(from_dev(y12), from_dev(0.5 * y1 + y2)) <= 2 * GEMV_TOL


def test_q4k_gemv_multi_matches_single(rt, orc):
    """q/k/v-style fused launch: each job bit-identical to its single launch
    (same kernel arithmetic per row) and within tolerance of the oracle."""
    rng = np.random.default_rng(21)
    k = 3072
    ns = [3072, 1024, 1024, 8]
    blocks = [orc.q4k_quantize((rng.standard_normal((n, k)) * 0.02).astype(np.float32)) for n in ns]
    x = rng.standard_normal((1, k)).astype(np.float32)
    dw = [to_dev(b) for b in blocks]
    dx = to_dev(x)
    ys = rt.gemv_q4k_multi(dw, dx, ns, k)
    for j, n in enumerate(ns):
        y = from_dev(ys[j])
        y_ref = orc.q4k_matmul_t(blocks[j], n, k, x)
        assert normwise_err(y, y_ref) <= GEMV_TOL, j
    ys2 = rt.gemv_q4k_multi(dw[:2], dx, ns[:2], k)
    for j in range(2):
        single = from_dev(rt.gemv(rt.Q4K, dw[j], dx, ns[j], k))
        assert normwise_err(from_dev(ys2[j]), single) <= GEMV_TOL


BF16_CASES = [
    (4096, 1152, 1, "lm_head slice (K=1152, 16 lanes per row)"),
    (1024, 3072, 1, "llama v widened to BF16"),
    (3072, 8192, 1, "llama down widened to BF16"),
    (131, 200, 1, "K=200 (K/8 = 25: 1 lane per row)"),
    (64, 96, 4, "M=4"),
    (257, 1152, 8, "M=8"),
    (3072, 8192, 8, "llama down widened, M=8: K-slices"),
    (1024, 3072, 6, "llama v widened, M=6"),
    (300, 1000, 2, "K=1000: a part-filled last 128-value slot, M=2"),
    (33, 8, 3, "K=8, M=3"),
]


@pytest.mark.parametrize("n,k,m,note", BF16_CASES)
def test_bf16_gemv_matches_oracle(rt, orc, n, k, m, note):
    say(f"[bf16 gemv] N={n} K={k} M={m} ({note})")
    rng = np.random.default_rng(n + 7 * k + m)
    w = orc.f32_to_bf16_n((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    x = rng.standard_normal((m, k)).astype(np.float32)
    y_ref = orc.bf16_matmul_t(w, x)
    y = from_dev(rt.gemv(rt.BF16, to_dev(w), to_dev(x), n, k))
    assert normwise_err(y, y_ref) <= GEMV_TOL


def test_bf16_lm_head_config2_with_argmax(rt, orc):
    """BASELINE config 2b: 262144 x 1152 bf16 lm_head, x ~ N(0,1), plus the
    top-1 index.  The index must be the oracle's whenever the oracle's top-2
    gap exceeds the output tolerance, and must always be exactly the first
    maximum of the GPU's own logits."""
    say("[bf16 gemv+argmax] 262144x1152")
    n, k = 262144, 1152
    rng = np.random.default_rng(2)
    w = orc.f32_to_bf16_n((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    x = rng.standard_normal(k).astype(np.float32)
    y_ref = orc.bf16_matmul_t(w, x)[0]
    y, idx, val = rt.gemv_bf16_argmax(to_dev(w), to_dev(x), n, k)
    y = from_dev(y)[0]
    assert normwise_err(y, y_ref) <= GEMV_TOL
    idx, val = int(from_dev(idx)[0]), float(from_dev(val)[0])
    assert idx == orc.argmax_first(y) and val == y[idx]
    top2 = np.sort(y_ref)[-2:]
    if top2[1] - top2[0] > 2 * GEMV_TOL * np.max(np.abs(y_ref)):
        assert idx == orc.argmax_first(y_ref)


def test_bf16_argmax_ties_pick_lowest_row(rt, orc):
    """Identical weight rows give bit-identical logits: the first wins."""
    n, k = 5000, 256
    rng = np.random.default_rng(9)
    w = orc.f32_to_bf16_n((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    x = rng.standard_normal(k).astype(np.float32)
    y_ref = orc.bf16_matmul_t(w, x)[0]
    best = orc.argmax_first(y_ref)
    w[[17, 4000, 4999]] = w[best]
    _, idx, _ = rt.gemv_bf16_argmax(to_dev(w), to_dev(x), n, k)
    assert int(from_dev(idx)[0]) == min(17, best)


def test_argmax_rules_on_gpu(rt, orc):
    import math
    rows = [
        [1.0, 3.0, 3.0, 2.0],
        [math.nan, 1.0, math.nan, 5.0],
        [-math.inf, -math.inf, -math.inf, -math.inf],
        [math.nan, math.nan, math.nan, math.nan],
        [-1.0, -0.0, 0.0, -2.0],
        [-5.0, math.inf, math.inf, 0.0],
    ]
    logits = np.array(rows, np.float32)
    idx, _ = rt.argmax(to_dev(logits))
    assert from_dev(idx).tolist() == [orc.argmax_first(r) for r in logits]
    big = np.random.default_rng(1).standard_normal((3, 300000)).astype(np.float32)
    big[1, 123456] = big[1, 200000] = 99.0
    idx, val = rt.argmax(to_dev(big))
    assert from_dev(idx).tolist() == [orc.argmax_first(r) for r in big]
    assert from_dev(val)[1] == np.float32(99.0)


Q40_CASES = [
    (4096, 4096, 1, "config 2a"),
    (129, 256, 1, "ragged, one 8-block group per row"),
    (200, 1280, 3, "5 groups per row, M=3"),
    (64, 768, 8, "M=8"),
]


@pytest.mark.parametrize("n,k,m,note", Q40_CASES)
def test_q4_0_gemv_matches_oracle(rt, orc, n, k, m, note):
    """GGUF Q4_0 bytes streamed natively; CPU side is the reference's path
    for them: decode_q4_0_to_q4mat then Q4Mat::matmul_q4_t (exact dequant)."""
    say(f"[q4_0 gemv] N={n} K={k} M={m} ({note})")
    rng = np.random.default_rng(n + k + m)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    blocks = orc.q4_0_quantize(w)
    packed, scales = orc.q4_0_to_q4mat(blocks, n * k)
    y_ref = orc.q4mat_matmul_t(packed, scales, n, k, x)
    y = from_dev(rt.gemv(rt.Q4_0, to_dev(blocks), to_dev(x), n, k))
    assert normwise_err(y, y_ref) <= GEMV_TOL


@pytest.mark.parametrize("fmt_name,n,k,m", [("Q4K", 8192, 3072, 8), ("BF16", 3072, 8192, 3), ("Q4K", 1024, 3072, 2)])
def test_batched_gemv_is_deterministic(rt, orc, fmt_name, n, k, m):
    """Batched GEMVs whose K is cut into slices add the slices' partial
    products in slice order, whichever workgroup finishes last: repeated
    calls give the same bits."""
    say(f"[batched gemv determinism] {fmt_name} N={n} K={k} M={m}")
    rng = np.random.default_rng(n + k + m)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    fmt = getattr(rt, fmt_name)
    wb = orc.q4k_quantize(w) if fmt_name == "Q4K" else orc.f32_to_bf16_n(w)
    dw, dx = to_dev(wb), to_dev(x)
    first = from_dev(rt.gemv(fmt, dw, dx, n, k))
    for _ in range(5):
        assert np.array_equal(from_dev(rt.gemv(fmt, dw, dx, n, k)).view(np.uint32), first.view(np.uint32))
    ref = orc.q4k_matmul_t(wb, n, k, x) if fmt_name == "Q4K" else orc.bf16_matmul_t(wb, x)
    assert normwise_err(first, ref) <= GEMV_TOL


def test_linear_forward_dispatch_with_bias(rt, orc):
    """QLinear::forward semantics: product plus bias on every row."""
    rng = np.random.default_rng(12)
    n, k, m = 300, 512, 3
    blocks = orc.q4k_quantize((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    x = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    y_ref = orc.q4k_matmul_t(blocks, n, k, x) + b
    y = from_dev(rt.linear_forward(rt.Q4K, to_dev(blocks), to_dev(x), n, k, bias=to_dev(b)))
    assert normwise_err(y, y_ref) <= GEMV_TOL
