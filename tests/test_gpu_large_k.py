"""GPU parity at K beyond 64 KB of staged activation: every decode GEMV takes
any K whose staged activation fits one workgroup's LDS (160 KB on gfx950),
as the reference's gemv_mt / matmul_by_t / matmul_q4_t stride over K with
no limit (src/quant_q4k.cpp:564-600, src/mat.cpp:318-349,
src/quant_q4.cpp:92-114).

K = 21504 is the Gemma-3-27B down projection's (ffn 21504); K = 16384 the
Q4Mat case.  Expected values come from the oracle's restatement of the
reference's sequential f32 loops, under the GEMV bar (normwise 1e-5); the
fused SwiGLU and RMSNorm entries are compared with the oracle's operation
followed by its product.  The x operations' staging of values past the
register batch (K / 4 above what the threads' registers hold) is exercised
here and nowhere else.
"""
import numpy as np
import pytest

from helpers import GEMV_TOL, from_dev, normwise_err, say, to_dev

pytestmark = pytest.mark.gpu
GEMMA27_DOWN_K = 21504


def q4k_weight(orc, rng, n, k):
    return orc.q4k_quantize((rng.standard_normal((n, k)) * 0.02).astype(np.float32))


@pytest.mark.parametrize("n,k,m", [(512, GEMMA27_DOWN_K, 1), (5376, GEMMA27_DOWN_K, 1), (300, GEMMA27_DOWN_K, 8),
                                   (257, 16384, 1), (64, 40960, 1)])
def test_q4k_rows_large_k(rt, orc, n, k, m):
    say(f"[large k] Q4_K row-major N={n} K={k} M={m}")
    rng = np.random.default_rng(n + k + m)
    blocks = q4k_weight(orc, rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    want = orc.q4k_matmul_t(blocks, n, k, x)
    got = from_dev(rt.gemv(rt.Q4K, to_dev(blocks), to_dev(x), n, k))
    for r in range(m):
        assert normwise_err(got[r], want[r]) <= GEMV_TOL, (r, normwise_err(got[r], want[r]))


@pytest.mark.parametrize("n,k", [(5376, GEMMA27_DOWN_K), (100, 16640)])
def test_q4k_tiled_large_k(rt, orc, n, k):
    say(f"[large k] Q4_K tiled N={n} K={k}")
    rng = np.random.default_rng(3 * n + k)
    blocks = q4k_weight(orc, rng, n, k)
    x = rng.standard_normal((1, k)).astype(np.float32)
    want = orc.q4k_matmul_t(blocks, n, k, x).reshape(-1)
    tiled = rt.q4k_tile(to_dev(blocks), n, k)
    got = from_dev(rt.gemv_q4k_tiled(tiled, to_dev(x), n, k)).reshape(-1)
    assert normwise_err(got, want) <= GEMV_TOL
    # the multi-weight launch at the same K
    blocks2 = q4k_weight(orc, rng, 64, k)
    want2 = orc.q4k_matmul_t(blocks2, 64, k, x).reshape(-1)
    y1, y2 = rt.gemv_q4k_tiled_multi([tiled, rt.q4k_tile(to_dev(blocks2), 64, k)], to_dev(x), [n, 64], k)
    assert normwise_err(from_dev(y1).reshape(-1), want) <= GEMV_TOL
    assert normwise_err(from_dev(y2).reshape(-1), want2) <= GEMV_TOL


def test_q4k_tiled_swiglu_residual_gemma27_down(rt, orc):
    """The MLP's down projection and its residual add at Gemma-3-27B's ffn:
    resid += W . (silu(gate) * up)."""
    n, k = 5376, GEMMA27_DOWN_K
    say(f"[large k] Q4_K tiled SwiGLU + residual N={n} K={k}")
    rng = np.random.default_rng(27)
    blocks = q4k_weight(orc, rng, n, k)
    gate = rng.standard_normal(k).astype(np.float32)
    up = rng.standard_normal(k).astype(np.float32)
    resid = rng.standard_normal(n).astype(np.float32)
    act = orc.swiglu(gate, up)
    want = resid + orc.q4k_matmul_t(blocks, n, k, act.reshape(1, k)).reshape(-1)
    d_resid = to_dev(resid)
    rt.gemv_swiglu_residual(rt.Q4K, rt.q4k_tile(to_dev(blocks), n, k), to_dev(gate), to_dev(up), d_resid, n, k)
    assert normwise_err(from_dev(d_resid), want) <= GEMV_TOL


@pytest.mark.parametrize("gemma3", [False, True])
def test_q4k_tiled_rmsnorm_large_k(rt, orc, gemma3):
    n, k = 1024, GEMMA27_DOWN_K
    say(f"[large k] Q4_K tiled RMSNorm N={n} K={k} gemma3={gemma3}")
    rng = np.random.default_rng(11 + gemma3)
    blocks = q4k_weight(orc, rng, n, k)
    x = rng.standard_normal(k).astype(np.float32)
    gamma = ((0.0 if gemma3 else 1.0) + 0.1 * rng.standard_normal(k)).astype(np.float32)
    xn = orc.rmsnorm(x, gamma, 1e-6, gemma3=gemma3)
    want = orc.q4k_matmul_t(blocks, n, k, xn.reshape(1, k)).reshape(-1)
    (got,) = rt.gemv_q4k_tiled_rmsnorm_multi([rt.q4k_tile(to_dev(blocks), n, k)], to_dev(x), to_dev(gamma), 1e-6,
                                             [n], k, gemma3=gemma3)
    assert normwise_err(from_dev(got).reshape(-1), want) <= GEMV_TOL


@pytest.mark.parametrize("n,k,m", [(5376, GEMMA27_DOWN_K, 1), (700, GEMMA27_DOWN_K, 8), (64, 36864, 1)])
def test_bf16_large_k(rt, orc, n, k, m):
    say(f"[large k] BF16 N={n} K={k} M={m}")
    rng = np.random.default_rng(5 * n + k + m)
    w = orc.f32_to_bf16_n((rng.standard_normal((n, k)) * 0.02).astype(np.float32)).reshape(n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    want = orc.bf16_matmul_t(w, x)
    got = from_dev(rt.gemv(rt.BF16, to_dev(w), to_dev(x), n, k))
    for r in range(m):
        assert normwise_err(got[r], want[r]) <= GEMV_TOL, (r, normwise_err(got[r], want[r]))


def test_bf16_swiglu_residual_gemma27_down(rt, orc):
    n, k = 5376, GEMMA27_DOWN_K
    say(f"[large k] BF16 SwiGLU + residual N={n} K={k}")
    rng = np.random.default_rng(270)
    w = orc.f32_to_bf16_n((rng.standard_normal((n, k)) * 0.02).astype(np.float32)).reshape(n, k)
    gate = rng.standard_normal(k).astype(np.float32)
    up = rng.standard_normal(k).astype(np.float32)
    resid = rng.standard_normal(n).astype(np.float32)
    want = resid + orc.bf16_matmul_t(w, orc.swiglu(gate, up).reshape(1, k)).reshape(-1)
    d_resid = to_dev(resid)
    rt.gemv_swiglu_residual(rt.BF16, to_dev(w), to_dev(gate), to_dev(up), d_resid, n, k)
    assert normwise_err(from_dev(d_resid), want) <= GEMV_TOL


@pytest.mark.parametrize("n,k,m", [(5376, GEMMA27_DOWN_K, 1), (256, GEMMA27_DOWN_K, 8)])
def test_q4_0_large_k(rt, orc, n, k, m):
    """GGUF Q4_0 bytes; the CPU side is decode_q4_0_to_q4mat then
    Q4Mat::matmul_q4_t (src/gguf.cpp:495-529, src/quant_q4.cpp:92-114)."""
    say(f"[large k] Q4_0 N={n} K={k} M={m}")
    rng = np.random.default_rng(n + 2 * k + m)
    blocks = orc.q4_0_quantize((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    packed, scales = orc.q4_0_to_q4mat(blocks, n * k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    want = orc.q4mat_matmul_t(packed, scales, n, k, x)
    got = from_dev(rt.gemv(rt.Q4_0, to_dev(blocks), to_dev(x), n, k))
    for r in range(m):
        assert normwise_err(got[r], want[r]) <= GEMV_TOL, (r, normwise_err(got[r], want[r]))


@pytest.mark.parametrize("n,k,m", [(4096, 16384, 1), (4096, 16384, 8), (300, GEMMA27_DOWN_K, 3)])
def test_q4mat_large_k(rt, orc, n, k, m):
    say(f"[large k] Q4Mat N={n} K={k} M={m}")
    rng = np.random.default_rng(n + k + 7 * m)
    packed, scales = orc.q4mat_quantize((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    x = rng.standard_normal((m, k)).astype(np.float32)
    want = orc.q4mat_matmul_t(packed, scales, n, k, x)
    got = from_dev(rt.gemv(rt.Q4MAT, rt.q4mat_upload(packed, scales, n, k), to_dev(x), n, k))
    for r in range(m):
        assert normwise_err(got[r], want[r]) <= GEMV_TOL, (r, normwise_err(got[r], want[r]))


def test_beyond_lds_is_refused(rt, orc):
    """K whose staged activation exceeds the LDS is an error, not a fault."""
    import torch
    k = 65536  # Q4_K limbs: 3.5 bytes per value, 224 KB
    lib = rt.library()
    w = torch.zeros(16 * (k // 256) * 144, dtype=torch.uint8, device="cuda")
    x = torch.zeros(k, dtype=torch.float32, device="cuda")
    y = torch.empty(16, dtype=torch.float32, device="cuda")
    rc = lib.status("rt_hip_gemv_q4k_tiled", w.data_ptr(), x.data_ptr(), y.data_ptr(), 16, k, None)
    assert rc == 2, rc
