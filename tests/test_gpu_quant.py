"""GPU parity, bit-exact: Q4_K dequantization and quantization against the oracle."""
import os

import numpy as np
import pytest

from helpers import f32_to_bf16_rne, from_dev, say, to_dev

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "ref_vectors.npz")


@pytest.mark.parametrize("n,k", [(1, 256), (37, 512), (300, 3072), (64, 12288)])
def test_dequant_q4k_f32_bit_exact(rt, orc, n, k):
    say(f"[dequant f32] {n}x{k}")
    rng = np.random.default_rng(n + k)
    blocks = orc.q4k_quantize((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    got = from_dev(rt.dequant_q4k(to_dev(blocks), n, k))
    want = orc.q4k_dequant(blocks, n, k)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_dequant_q4k_adversarial_and_random_bytes_bit_exact(rt, orc):
    """Golden adversarial blocks (zero, constant, tiny -> f16-subnormal d,
    huge -> f16 overflow) plus uniformly random block bytes (every header
    and nibble pattern; d/dmin restricted to finite f16)."""
    with np.load(GOLDEN, allow_pickle=False) as z:
        adv = z["q4k_adv_blocks"]
        adv_deq = z["q4k_adv_deq"]
    got = from_dev(rt.dequant_q4k(to_dev(adv), adv_deq.shape[0], 256))
    # NaN/Inf payloads aside (none in the finite rows), bit-equal
    assert np.array_equal(got.view(np.uint32), adv_deq.view(np.uint32))
    rng = np.random.default_rng(77)
    rnd = rng.integers(0, 256, (512, 144), dtype=np.uint8)
    for o in (1, 3):  # clear the f16 exponent top bit -> finite d, dmin
        rnd[:, o] &= 0x7b
    rnd = rnd.reshape(-1)
    got = from_dev(rt.dequant_q4k(to_dev(rnd), 512, 256))
    want = orc.q4k_dequant(rnd, 512, 256)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_dequant_q4k_bf16_adversarial_and_random_bytes(rt, orc):
    """bf16 output on the golden adversarial blocks and on random block
    bytes: the oracle's exact dequant, then the reference's f32 -> bf16
    (orc.f32_to_bf16_n, RNE with NaN quieting), bit for bit."""
    with np.load(GOLDEN, allow_pickle=False) as z:
        adv = z["q4k_adv_blocks"]
        adv_deq = z["q4k_adv_deq"]
    got = from_dev(rt.dequant_q4k(to_dev(adv), adv_deq.shape[0], 256, bf16=True)).view(np.uint16)
    assert np.array_equal(got.reshape(-1), orc.f32_to_bf16_n(adv_deq).reshape(-1))
    rng = np.random.default_rng(78)
    rnd = rng.integers(0, 256, (777, 144), dtype=np.uint8)
    for o in (1, 3):  # finite d, dmin
        rnd[:, o] &= 0x7b
    rnd = rnd.reshape(-1)
    got = from_dev(rt.dequant_q4k(to_dev(rnd), 777, 256, bf16=True)).view(np.uint16)
    want = orc.f32_to_bf16_n(orc.q4k_dequant(rnd, 777, 256))
    assert np.array_equal(got.reshape(-1), want.reshape(-1))


def test_dequant_q4k_bf16_is_rne_of_exact(rt, orc):
    rng = np.random.default_rng(3)
    n, k = 200, 768
    blocks = orc.q4k_quantize((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    got = from_dev(rt.dequant_q4k(to_dev(blocks), n, k, bf16=True)).view(np.uint16)
    want = f32_to_bf16_rne(orc.q4k_dequant(blocks, n, k))
    assert np.array_equal(got, want)


@pytest.mark.parametrize("n,k,scale", [(64, 256, 0.02), (257, 3072, 0.02), (16, 1024, 1e-7),
                                       (16, 512, 3e4)])
def test_quantize_q4k_byte_identical(rt, orc, n, k, scale):
    say(f"[quantize] {n}x{k} scale {scale}")
    rng = np.random.default_rng(n * k)
    w = (rng.standard_normal((n, k)) * scale).astype(np.float32)
    w[0, :64] = 0.0
    w[min(1, n - 1), :128] = np.abs(w[min(1, n - 1), :128])
    got = from_dev(rt.quantize_q4k(to_dev(w)))
    assert np.array_equal(got, orc.q4k_quantize(w))


def test_quantize_q4k_adversarial_golden(rt):
    """The reference's own bytes for rows hitting every branch of
    quantize_block (tests/golden/ref_vectors.npz)."""
    with np.load(GOLDEN, allow_pickle=False) as z:
        w, blocks = z["q4k_adv_w"], z["q4k_adv_blocks"]
    assert np.array_equal(from_dev(rt.quantize_q4k(to_dev(w))), blocks)


def test_quantize_q4k_full_size_roundtrip(rt, orc):
    """Full lm_head-sized quantization (128256 x 3072) on the GPU: a sampled
    set of rows is byte-identical to the oracle, and dequant(quant(W)) stays
    within the Q4_K error bound (<= 0.5 * per-sub-block step + min rounding)."""
    import torch
    n, k = 128256, 3072
    g = torch.Generator(device="cuda").manual_seed(5)
    w = torch.randn((n, k), generator=g, device="cuda") * 0.02
    blocks = rt.quantize_q4k(w)
    rows = np.random.default_rng(0).choice(n, 64, replace=False)
    rb = 12 * 144
    got = from_dev(blocks).reshape(n, rb)
    wh = from_dev(w)
    for r in rows:
        assert np.array_equal(got[r], orc.q4k_quantize(wh[r:r + 1]))
    deq = rt.dequant_q4k(blocks, n, k)
    err = (deq - w).abs().max().item()
    assert err < 0.02 * 6 / 15
