"""GPU parity: GGUF Q6_K on the device (gguf.cpp:531-580; transformer4_load.cpp:33-41, 141-143).

The reference widens a Q6_K projection to bf16 at load and runs the BF16
GEMV.  The checks here:
  * rt_hip_dequant_q6k_bf16 equals that widening bit for bit (the oracle's
    restated decode, itself pinned by the reference's known-block test, then
    the reference's f32 -> bf16 RNE);
  * rt_hip_gemv_q6k_tiled equals the reference's BF16 product on the widened
    weights (normwise 1e-5, the GEMV bar) and this library's BF16 GEMV on
    them; a one-hot x returns the widened column bit for bit (exact limbs,
    exact products).
"""
import numpy as np
import pytest

from helpers import GEMV_TOL, from_dev, normwise_err, say, to_dev

pytestmark = pytest.mark.gpu


def random_q6k(rng, n, k):
    """Random Q6_K rows: random ql/qh, int8 scales, d in [1e-5, 5e-5)
    (weights of a few hundredths), as the oracle's f16 encoder stores it."""
    nb = k // 256
    blk = rng.integers(0, 256, size=(n * nb, 210), dtype=np.uint8)
    blk[:, 192:208] = rng.integers(-128, 128, size=(n * nb, 16)).astype(np.int8).view(np.uint8)
    d = rng.uniform(1e-5, 5e-5, size=n * nb).astype(np.float32).astype(np.float16)
    blk[:, 208:210] = d.view(np.uint8).reshape(-1, 2)
    return blk.reshape(-1)


def widened(orc, blocks, n, k):
    return orc.f32_to_bf16_n(orc.q6k_decode(blocks, n * k)).reshape(n, k)


CASES = [
    (3072, 8192, "llama down (Q6_K in a Q4_K_M model)"),
    (1024, 3072, "llama v"),
    (100, 256, "ragged N, one block"),
    (33, 2304, "K = 9 blocks (no K split)"),
    (17, 512, "two blocks"),
]


@pytest.mark.parametrize("n,k,note", CASES)
def test_q6k_widening_is_bit_exact(rt, orc, n, k, note):
    say(f"[q6k widen] N={n} K={k} ({note})")
    rng = np.random.default_rng(n + k)
    blocks = random_q6k(rng, n, k)
    want = widened(orc, blocks, n, k)
    got = from_dev(rt.dequant_q6k_bf16(to_dev(blocks), n, k)).view(np.uint16)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("n,k,note", CASES)
def test_q6k_gemv_matches_widened_bf16(rt, orc, n, k, note):
    say(f"[q6k gemv] N={n} K={k} ({note})")
    rng = np.random.default_rng(7 * n + k)
    blocks = random_q6k(rng, n, k)
    w = widened(orc, blocks, n, k)
    x = rng.standard_normal((1, k)).astype(np.float32)
    y_ref = orc.bf16_matmul_t(w, x)
    d_blocks = to_dev(blocks)
    tiled = rt.q6k_tile(d_blocks, n, k)
    assert tiled.numel() == ((n + 15) // 16) * (k // 256) * 3360
    y = from_dev(rt.gemv_q6k_tiled(tiled, to_dev(x), n, k))
    assert normwise_err(y, y_ref) <= GEMV_TOL, normwise_err(y, y_ref)
    y_bf16 = from_dev(rt.gemv(rt.BF16, to_dev(w.view(np.int16)), to_dev(x), n, k))
    assert normwise_err(y, y_bf16) <= GEMV_TOL


@pytest.mark.parametrize("n,k", [(3072, 8192), (1000, 2304), (16, 256)])
def test_q6k_swiglu_residual(rt, orc, n, k):
    """resid += W . (silu(gate) * up) on the Q6_K bytes (the down projection
    and residual add of transformer5.cpp:186-190, 205-212) against the
    oracle's composition (swiglu, then the BF16 product on the widened
    weights, plus resid) at the GEMV bar, and against this library's BF16
    swiglu-residual on the widened copy.  K splits 8 (3072 x 8192), 1
    (16 x 256, a single tile) and 9 blocks unsplit (1000 x 2304)."""
    say(f"[q6k swiglu residual] N={n} K={k}")
    rng = np.random.default_rng(3 * n + k)
    blocks = random_q6k(rng, n, k)
    w = widened(orc, blocks, n, k)
    gate = (rng.standard_normal(k) * 2).astype(np.float32)
    up = rng.standard_normal(k).astype(np.float32)
    r0 = rng.standard_normal(n).astype(np.float32)
    want = r0 + orc.bf16_matmul_t(w, orc.swiglu(gate, up).reshape(1, k)).reshape(-1)
    tiled = rt.q6k_tile(to_dev(blocks), n, k)
    resid = to_dev(r0)
    rt.gemv_swiglu_residual(None, tiled, to_dev(gate), to_dev(up), resid, n, k, q6k=True)
    got = from_dev(resid)
    assert normwise_err(got, want) <= GEMV_TOL, normwise_err(got, want)
    rb = to_dev(r0)
    rt.gemv_swiglu_residual(rt.BF16, to_dev(w.view(np.int16)), to_dev(gate), to_dev(up), rb, n, k)
    assert normwise_err(got, from_dev(rb)) <= GEMV_TOL
    # gate = 0 makes silu(gate) * up zero: resid comes back unchanged, bit for bit
    rz = to_dev(r0)
    rt.gemv_swiglu_residual(None, tiled, to_dev(np.zeros(k, np.float32)), to_dev(up), rz, n, k, q6k=True)
    assert np.array_equal(from_dev(rz).view(np.uint32), r0.view(np.uint32))
    # an aliased residual is refused
    lib = rt.library()
    g = to_dev(gate)
    assert lib.status("rt_hip_gemv_q6k_tiled_swiglu_residual", tiled.data_ptr(), g.data_ptr(), g.data_ptr(),
                      g.data_ptr(), n, k, None) != 0


def test_q6k_gemv_one_hot_is_exact(rt, orc):
    """x = e_c gives y = W[:, c], the widened bf16 weight exactly (a -0
    weight gives +0, as the reference's sum that starts from 0.0f does)."""
    n, k = 300, 2048
    say(f"[q6k gemv one-hot] N={n} K={k}")
    rng = np.random.default_rng(5)
    blocks = random_q6k(rng, n, k)
    w = widened(orc, blocks, n, k)
    tiled = rt.q6k_tile(to_dev(blocks), n, k)
    for c in (0, 1, 255, 256, 1000, k - 1):
        x = np.zeros((1, k), np.float32)
        x[0, c] = 1.0
        y = from_dev(rt.gemv_q6k_tiled(tiled, to_dev(x), n, k))[0]
        col = (w[:, c].astype(np.uint32) << 16).view(np.float32) + np.float32(0.0)
        assert np.array_equal(y.view(np.uint32), col.view(np.uint32)), c


def test_q6k_reference_known_block_on_gpu(rt, orc):
    """The reference's Q6_K known block (tests/test_gguf.cpp:292-335: ql/qh
    from mt19937(1234), scales (i*7)%61-30, d = 0.0125) widened on the GPU."""
    from test_oracle import MT19937
    g = MT19937(1234)
    blk = np.zeros(210, np.uint8)
    for i in range(192):
        blk[i] = g() & 0xff
    for i in range(16):
        blk[192 + i] = np.uint8(np.int8((i * 7) % 61 - 30).view(np.uint8))
    h = orc.f32_to_f16(0.0125)
    blk[208], blk[209] = h & 0xff, h >> 8
    want = orc.f32_to_bf16_n(orc.q6k_decode(blk, 256))
    got = from_dev(rt.dequant_q6k_bf16(to_dev(blk), 1, 256)).view(np.uint16).reshape(-1)
    assert np.array_equal(got, want)
    x = np.random.default_rng(1).standard_normal((1, 256)).astype(np.float32)
    y = from_dev(rt.gemv_q6k_tiled(rt.q6k_tile(to_dev(blk), 1, 256), to_dev(x), 1, 256))
    assert normwise_err(y, orc.bf16_matmul_t(want.reshape(1, 256), x)) <= GEMV_TOL


def test_q6k_rejects_bad_shapes(rt):
    lib = rt.library()
    assert lib.lib.rt_hip_q6k_tiled_bytes(16, 100) == -1
    assert lib.lib.rt_hip_q6k_tiled_bytes(16, 256) == 3360
    t = to_dev(np.zeros(3360, np.uint8))
    x = to_dev(np.zeros(256 * 64, np.float32))
    y = to_dev(np.zeros(16, np.float32))
    assert lib.status("rt_hip_gemv_q6k_tiled", t.data_ptr(), x.data_ptr(), y.data_ptr(), 16, 100, None) != 0
    assert lib.status("rt_hip_gemv_q6k_tiled", t.data_ptr(), x.data_ptr(), y.data_ptr(), 16, 16384, None) != 0
