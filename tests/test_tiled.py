"""Tiled Q4_K layout: the device tiling and the GEMV on tiled weights.

The layout is this build's own (no reference counterpart), so it is pinned
by what must hold rather than by reference vectors: untile(tile(b)) == b for
any bytes, dequantizing straight from the tiled bytes gives the oracle's
dequantized weights bit-for-bit, the device tiling equals the numpy one
byte-for-byte, and the GEMV on tiled weights returns exactly the bits of the
GEMV on the row-major blocks (same arithmetic on the same values).
"""
import numpy as np
import pytest

from helpers import (GEMV_TOL, bf16_bits_to_f32, f32_to_bf16_rne, from_dev, normwise_err,
                     q4k_dequant_tiled_np, q4k_tile_np,
                     q4k_untile_np, say, to_dev)

SHAPES = [(37, 256), (130, 1024), (1, 512), (16, 2304), (300, 3072)]


@pytest.mark.parametrize("n,k", SHAPES)
def test_tile_untile_roundtrip_any_bytes(n, k):
    rng = np.random.default_rng(n + k)
    b = rng.integers(0, 256, n * (k // 256) * 144, dtype=np.uint8)
    t = q4k_tile_np(b, n, k)
    assert t.size == (n + 15) // 16 * 16 * (k // 256) * 144
    assert np.array_equal(q4k_untile_np(t, n, k), b)


@pytest.mark.parametrize("n,k", SHAPES)
def test_tiled_dequant_matches_oracle(orc, n, k):
    rng = np.random.default_rng(7 * n + k)
    w = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)
    blocks = orc.q4k_quantize(w)
    ref = orc.q4k_dequant(blocks, n, k)
    got = q4k_dequant_tiled_np(q4k_tile_np(blocks, n, k), n, k)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_tiled_rows_past_n_are_zero():
    n, k = 20, 512
    b = np.full(n * 2 * 144, 0xAB, np.uint8)
    t = q4k_tile_np(b, n, k).reshape(2, 2, 2304)   # tiles, blocks, bytes
    last = t[1]                                   # rows 16..31, of which 16..19 real
    hdr = last[:, :256].copy().view("<u4").reshape(2, 4, 16)
    assert np.all(hdr[:, :, 4:] == 0) and np.all(hdr[:, :, :4] != 0)
    qa = last[:, 256:1280].reshape(2, 4, 16, 16)
    assert np.all(qa[:, :, 4:] == 0) and np.all(qa[:, :, :4] == 0xAB)


@pytest.mark.gpu
@pytest.mark.parametrize("n,k", SHAPES)
def test_device_tiling_matches_numpy(rt, orc, n, k):
    say(f"[q4k tile] N={n} K={k}")
    rng = np.random.default_rng(n * 3 + k)
    b = rng.integers(0, 256, n * (k // 256) * 144, dtype=np.uint8)
    got = from_dev(rt.q4k_tile(to_dev(b), n, k))
    assert np.array_equal(got, q4k_tile_np(b, n, k))


TILED_GEMV = [(3072, 3072), (1024, 3072), (8192, 3072), (3072, 8192), (130, 256), (37, 2304),
              (1, 12288), (128256 // 8, 3072)]


@pytest.mark.gpu
@pytest.mark.parametrize("n,k", TILED_GEMV)
def test_tiled_gemv_equals_rowmajor_gemv(rt, orc, n, k):
    say(f"[q4k tiled gemv] N={n} K={k}")
    rng = np.random.default_rng(n + 5 * k)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((1, k)).astype(np.float32)
    blocks = orc.q4k_quantize(w)
    d_b, d_x = to_dev(blocks), to_dev(x)
    y_rows = from_dev(rt.gemv(rt.Q4K, d_b, d_x, n, k))
    y_tiled = from_dev(rt.gemv_q4k_tiled(rt.q4k_tile(d_b, n, k), d_x, n, k))
    assert np.array_equal(y_tiled.view(np.uint32), y_rows.view(np.uint32))
    y_ref = orc.q4k_matmul_t(blocks, n, k, x)
    assert normwise_err(y_tiled, y_ref) <= GEMV_TOL


@pytest.mark.gpu
def test_tiled_gemv_one_hot_is_exact(rt, orc):
    rng = np.random.default_rng(11)
    n, k = 70, 1024
    blocks = orc.q4k_quantize((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    deq = orc.q4k_dequant(blocks, n, k)
    tiled = rt.q4k_tile(to_dev(blocks), n, k)
    for col in (0, 31, 32, 63, 64, 200, 255, 256, 600, 1023):
        x = np.zeros((1, k), np.float32)
        x[0, col] = 1.0
        y = from_dev(rt.gemv_q4k_tiled(tiled, to_dev(x), n, k))[0]
        assert np.array_equal(y.view(np.uint32), deq[:, col].view(np.uint32)), col


@pytest.mark.gpu
def test_tiled_multi_equals_rowmajor_multi(rt, orc):
    say("[q4k tiled multi] q/k/v 3072+1024+1024 x 3072 and ragged 3-job")
    rng = np.random.default_rng(21)
    for ns, k in (([3072, 1024, 1024], 3072), ([8192, 8192], 3072), ([37, 130, 5, 16], 512)):
        bl = [orc.q4k_quantize((rng.standard_normal((n, k)) * 0.02).astype(np.float32)) for n in ns]
        x = to_dev(rng.standard_normal((1, k)).astype(np.float32))
        dbl = [to_dev(b) for b in bl]
        ys_rows = rt.gemv_q4k_multi(dbl, x, ns, k)
        ys_tiled = rt.gemv_q4k_tiled_multi([rt.q4k_tile(b, n, k) for b, n in zip(dbl, ns)], x, ns, k)
        for a, b in zip(ys_rows, ys_tiled):
            assert np.array_equal(from_dev(a).view(np.uint32), from_dev(b).view(np.uint32))


@pytest.mark.gpu
def test_tile_rejects_bad_shapes(rt):
    import torch
    lib = rt.library()
    buf = torch.empty(4096, dtype=torch.uint8, device="cuda")
    out = torch.empty(4096, dtype=torch.uint8, device="cuda")
    assert lib.status("rt_hip_q4k_tile", buf.data_ptr(), out.data_ptr(), 1, 300, None) == 2
    assert lib.status("rt_hip_q4k_tile", buf.data_ptr(), buf.data_ptr(), 1, 256, None) == 1
    assert rt.q4k_tiled_bytes(17, 256) == 32 * 144
    assert rt.q4k_tiled_bytes(17, 255) == -1


FUSED = [([3072, 1024], 1024, 3072), ([3072], 3072, 8192), ([37, 130, 5, 16], 37, 512),
         ([8192, 8192], 100, 3072)]


@pytest.mark.gpu
@pytest.mark.parametrize("ns,nb,k", FUSED)
def test_fused_q4k_bf16_equals_separate(rt, orc, ns, nb, k):
    """q/k (tiled Q4_K) + BF16 v in one launch: the BF16 rows are the bits of
    rt_hip_gemv_bf16, the Q4_K rows those of the separate multi launch to f32
    rounding, and both meet the oracle."""
    say(f"[fused q4k+bf16] ns={ns} bf16 rows={nb} K={k}")
    rng = np.random.default_rng(sum(ns) + nb + k)
    x = rng.standard_normal((1, k)).astype(np.float32)
    bl = [orc.q4k_quantize((rng.standard_normal((n, k)) * 0.02).astype(np.float32)) for n in ns]
    wb32 = (rng.standard_normal((nb, k)) * 0.02).astype(np.float32)
    wbits = f32_to_bf16_rne(wb32)
    dx = to_dev(x)
    tl = [rt.q4k_tile(to_dev(b), n, k) for b, n in zip(bl, ns)]
    dwb = to_dev(wbits.view(np.int16))
    ys, yb = rt.gemv_q4k_tiled_bf16(tl, ns, dwb, nb, dx, k)
    yb_sep = from_dev(rt.gemv(rt.BF16, dwb, dx, nb, k))
    assert np.array_equal(from_dev(yb).view(np.uint32), yb_sep.view(np.uint32))
    ref_b = bf16_bits_to_f32(wbits).astype(np.float64) @ x[0].astype(np.float64)
    assert normwise_err(from_dev(yb)[0], ref_b) <= GEMV_TOL
    sep = rt.gemv_q4k_tiled_multi(tl, dx, ns, k)
    for b, n, y, y2 in zip(bl, ns, ys, sep):
        assert normwise_err(from_dev(y), from_dev(y2)) <= 1e-6
        assert normwise_err(from_dev(y), orc.q4k_matmul_t(b, n, k, x)) <= GEMV_TOL
