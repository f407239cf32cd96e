"""GPU parity on activations with a wide dynamic range.

The Q4_K GEMV kernels do not contract f32 activations directly: each value
becomes three int8 limbs with a power-of-two scale per 32-value sub-block
(error <= 2^-22 * the sub-block's absmax), contracted on int8 MFMA.  These
tests put that representation where it departs most from f32: an outlier
1000x the rest inside one sub-block, magnitudes spread over 2^-30 .. 2^10,
and a near-subnormal sub-block next to a normal one.

Two bars:
  * normwise 1e-5 against the oracle's reference-order f32 product
    (quant_q4k.cpp:482-523) for every kernel family: row-major and tiled
    M = 1, the RMSNorm-fused launch, batched M = 2..8;
  * per element, bit for bit, where the reference's f32 result is exact:
    hand-built Q4_K blocks (d, dmin powers of two, 3-bit scales) and
    activations that are 3-bit integers times a per-sub-block power of two
    spread over 10 binades.  Every product and partial sum is then exactly
    representable, so the reference's sequential f32 order, an fp64 product
    and any correct kernel must give the same bits.
"""
import numpy as np
import pytest

from helpers import GEMV_TOL, from_dev, normwise_err, say, to_dev

pytestmark = pytest.mark.gpu


def wide_activation(rng, m, k, kind):
    """m x k activations of the named shape."""
    if kind == "outlier":
        x = rng.standard_normal((m, k)).astype(np.float32)
        for r in range(m):
            for sb in rng.choice(k // 32, size=max(1, k // 256), replace=False):
                x[r, 32 * sb + rng.integers(32)] *= 1000.0
        return x
    if kind == "spread":  # |x| = 2^U(-30, 10), random signs
        e = rng.uniform(-30.0, 10.0, (m, k))
        return (np.exp2(e) * rng.choice([-1.0, 1.0], (m, k))).astype(np.float32)
    if kind == "tiny_next_to_normal":  # alternate sub-blocks ~1e-37 and ~1
        x = rng.standard_normal((m, k)).astype(np.float32)
        x.reshape(m, k // 32, 32)[:, ::2, :] *= np.float32(1e-37)
        return x
    if kind == "subblock_scales":  # every sub-block its own scale, 2^-20 .. 2^8
        s = np.exp2(rng.integers(-20, 9, (m, k // 32))).astype(np.float32)
        return (rng.standard_normal((m, k // 32, 32)) * s[..., None]).astype(np.float32).reshape(m, k)
    raise ValueError(kind)


KINDS = ["outlier", "spread", "tiny_next_to_normal", "subblock_scales"]


def _weights(orc, rng, n, k):
    return orc.q4k_quantize((rng.standard_normal((n, k)) * 0.02).astype(np.float32))


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("n,k", [(3072, 3072), (3072, 8192), (200, 768)])
def test_m1_rowmajor_and_tiled(rt, orc, kind, n, k):
    say(f"[wide x] M=1 N={n} K={k} kind={kind}")
    rng = np.random.default_rng(n + k + len(kind))
    blocks = _weights(orc, rng, n, k)
    x = wide_activation(rng, 1, k, kind)
    want = orc.q4k_matmul_t(blocks, n, k, x)
    d_b, d_x = to_dev(blocks), to_dev(x)
    rows = from_dev(rt.gemv(rt.Q4K, d_b, d_x, n, k))
    tiled = from_dev(rt.gemv_q4k_tiled(rt.q4k_tile(d_b, n, k), d_x, n, k))
    assert normwise_err(rows, want) <= GEMV_TOL, normwise_err(rows, want)
    assert normwise_err(tiled, want) <= GEMV_TOL, normwise_err(tiled, want)
    exact = x.astype(np.float64) @ orc.q4k_dequant(blocks, n, k).astype(np.float64).T
    assert normwise_err(tiled, exact) <= GEMV_TOL


@pytest.mark.parametrize("kind", KINDS)
def test_rmsnorm_fused(rt, orc, kind):
    k, ns = 3072, [3072, 1024]
    say(f"[wide x] rmsnorm q/k kind={kind}")
    rng = np.random.default_rng(77 + len(kind))
    blocks = [_weights(orc, rng, n, k) for n in ns]
    x = wide_activation(rng, 1, k, kind).reshape(-1)
    gamma = (1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    tiled = [rt.q4k_tile(to_dev(b), n, k) for b, n in zip(blocks, ns)]
    ys = rt.gemv_q4k_tiled_rmsnorm_multi(tiled, to_dev(x), to_dev(gamma), 1e-5, ns, k)
    xn = orc.rmsnorm(x, gamma, 1e-5).reshape(1, k)
    for b, n, y in zip(blocks, ns, ys):
        got, want = from_dev(y), orc.q4k_matmul_t(b, n, k, xn)
        assert normwise_err(got, want) <= GEMV_TOL, normwise_err(got, want)


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("m", [2, 5, 8])
def test_batched(rt, orc, kind, m):
    n, k = 1024, 3072
    say(f"[wide x] batched M={m} kind={kind}")
    rng = np.random.default_rng(m * 13 + len(kind))
    blocks = _weights(orc, rng, n, k)
    x = wide_activation(rng, m, k, kind)
    got = from_dev(rt.gemv(rt.Q4K, to_dev(blocks), to_dev(x), n, k))
    want = orc.q4k_matmul_t(blocks, n, k, x)
    for r in range(m):
        assert normwise_err(got[r], want[r]) <= GEMV_TOL, (r, normwise_err(got[r], want[r]))


# ---- exactly representable case ---------------------------------------------

def exact_blocks(orc, rng, n, k):
    """Q4_K bytes with d = 2^-8, dmin = 2^-9 (exact f16) and 6-bit scale and
    min codes below 8: every weight (d*sv)*q - dmin*mv has few bits."""
    nb = k // 256
    out = np.empty((n, nb, 144), np.uint8)
    out[..., 0:2] = np.frombuffer(np.float16(2.0 ** -8).tobytes(), np.uint8)
    out[..., 2:4] = np.frombuffer(np.float16(2.0 ** -9).tobytes(), np.uint8)
    for r in range(n):
        for b in range(nb):
            sv = rng.integers(0, 8, 8).astype(np.uint8)
            mv = rng.integers(0, 8, 8).astype(np.uint8)
            out[r, b, 4:16] = orc.q4k_pack_scales(sv, mv)
    out[..., 16:] = rng.integers(0, 256, (n, nb, 128), dtype=np.uint8)
    return out.reshape(-1)


def exact_activation(rng, m, k, spread=10):
    ints = rng.integers(-7, 8, (m, k)).astype(np.float64)
    e = rng.integers(-spread // 2, spread - spread // 2, (m, k // 32)).astype(np.float64)
    return (ints.reshape(m, k // 32, 32) * np.exp2(e)[..., None]).reshape(m, k).astype(np.float32)


@pytest.mark.parametrize("n,k,m", [(512, 3072, 1), (300, 8192, 1), (64, 1024, 1), (256, 3072, 4),
                                   (100, 2048, 8)])
def test_exact_inputs_bit_for_bit(rt, orc, n, k, m):
    say(f"[exact x] N={n} K={k} M={m}")
    rng = np.random.default_rng(n * 3 + k + m)
    blocks = exact_blocks(orc, rng, n, k)
    x = exact_activation(rng, m, k)
    want = orc.q4k_matmul_t(blocks, n, k, x)
    # premise: the reference's f32 order is exact here (equals fp64)
    exact = x.astype(np.float64) @ orc.q4k_dequant(blocks, n, k).astype(np.float64).T
    assert np.array_equal(want.astype(np.float64), exact)
    d_b, d_x = to_dev(blocks), to_dev(x)
    got = from_dev(rt.gemv(rt.Q4K, d_b, d_x, n, k))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    if m == 1:
        t = rt.q4k_tile(d_b, n, k)
        got_t = from_dev(rt.gemv_q4k_tiled(t, d_x, n, k))
        assert np.array_equal(got_t.view(np.uint32), want.view(np.uint32))
        (got_multi,) = rt.gemv_q4k_tiled_multi([t], d_x, [n], k)
        assert np.array_equal(from_dev(got_multi).view(np.uint32), want.view(np.uint32))
