"""GPU parity for the Q8-activation path (the reference's aarch64 gemv_mt:
quantize_activation_q8, quant_q4k.cpp:525-562, then dot_row_q8, :425-478)
against the oracle's restatement (pinned in tests/test_oracle_q8.py and, for
the quantizer, by the reference's golden vectors in tests/test_oracle.py).

Bit-exact on every output: the integer chunk dots are exact on the int8
matrix cores, and the f32 combination and the ordered chunk sum are the
reference's operations in the reference's order.
"""
import numpy as np
import pytest

from helpers import from_dev, say, to_dev

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def activation(rng, k, kind):
    if kind == "normal":
        return rng.standard_normal(k).astype(np.float32)
    if kind == "wide":
        # magnitudes 2^-30 .. 2^10, one outlier per block, zero blocks
        a = (rng.standard_normal(k) * np.exp2(rng.integers(-30, 11, k))).astype(np.float32)
        a[5::32] *= np.float32(1000.0)
        a[64:96] = 0.0
        if k > 130:
            a[130] = -0.0
        return a
    if kind == "ties":
        # a * (1 / scale) lands on .5 often: integers and halves of a 2^-k grid
        a = (rng.integers(-254, 255, k) * 0.5).astype(np.float32)
        a[::32] = np.float32(127.0)
        return a
    raise ValueError(kind)


@pytest.mark.parametrize("k", [1, 31, 32, 33, 256, 1000, 3072, 8192, 16384, 100003])
@pytest.mark.parametrize("kind", ["normal", "wide", "ties"])
def test_quantize_activation_q8_bit_exact(rt, orc, k, kind):
    say(f"[q8 quantize] k={k} {kind}")
    a = activation(np.random.default_rng(k + len(kind)), k, kind)
    q8, sc, su = rt.quantize_activation_q8(to_dev(a))
    rq8, rsc, rsu = orc.q4k_quantize_activation_q8(a)
    assert np.array_equal(from_dev(q8), rq8)
    assert np.array_equal(bits(from_dev(sc)), bits(rsc))
    assert np.array_equal(bits(from_dev(su)), bits(rsu))


CASES = [
    # (N, K, note)
    (3072, 3072, "llama q/o"),
    (1024, 3072, "llama k/v"),
    (8192, 3072, "llama gate/up"),
    (3072, 8192, "llama down"),
    (130, 256, "ragged N, one super-block"),
    (33, 2304, "9 super-blocks: 8 waves, 2 idle"),
    (7, 512, "tiny N"),
    (17, 16384, "K = 16384: 8 super-blocks per wave"),
    (1000, 1280, "5 super-blocks"),
]


@pytest.mark.parametrize("n,k,note", CASES)
@pytest.mark.parametrize("tiled", [False, True])
def test_gemv_q4k_q8_bit_exact(rt, orc, n, k, note, tiled):
    say(f"[q8 gemv] N={n} K={k} tiled={tiled} ({note})")
    rng = np.random.default_rng(n * 7 + k)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    blocks = orc.q4k_quantize(w)
    d_blocks = to_dev(blocks)
    d_w = rt.q4k_tile(d_blocks, n, k) if tiled else d_blocks
    for kind in ("normal", "wide", "ties"):
        x = activation(rng, k, kind)
        y = from_dev(rt.gemv_q4k_q8(d_w, to_dev(x), n, k, tiled=tiled)).reshape(-1)
        want = orc.q4k_gemv_q8(blocks, n, k, x)
        bad = np.flatnonzero(bits(y) != bits(want))
        assert bad.size == 0, (kind, bad[:8], y[bad[:4]], want[bad[:4]])


@pytest.mark.parametrize("n,k", [(40000, 3072), (33000, 8192), (32784, 16384)])
def test_gemv_q4k_q8_many_tiles_bit_exact(rt, orc, n, k):
    """More than 8 tiles per CU: several tiles share a workgroup (and its
    quantized x); random block bytes with finite d and dmin."""
    say(f"[q8 gemv many tiles] N={n} K={k}")
    rng = np.random.default_rng(n + k)
    blocks = rng.integers(0, 256, n * (k // 256) * 144, dtype=np.uint8)
    hdr = blocks.reshape(-1, 144)
    hdr[:, 1] &= 0x3B
    hdr[:, 3] &= 0x3B
    d_blocks = to_dev(blocks)
    x = activation(rng, k, "normal")
    want = orc.q4k_gemv_q8(blocks, n, k, x)
    for tiled in (False, True):
        d_w = rt.q4k_tile(d_blocks, n, k) if tiled else d_blocks
        y = from_dev(rt.gemv_q4k_q8(d_w, to_dev(x), n, k, tiled=tiled)).reshape(-1)
        bad = np.flatnonzero(bits(y) != bits(want))
        assert bad.size == 0, (tiled, bad[:8])


def test_gemv_q4k_q8_zero_and_one_hot(rt, orc):
    n, k = 64, 1024
    blocks = orc.q4k_quantize((np.random.default_rng(3).standard_normal((n, k)) * 0.02).astype(np.float32))
    d_blocks = to_dev(blocks)
    y = from_dev(rt.gemv_q4k_q8(d_blocks, to_dev(np.zeros(k, np.float32)), n, k)).reshape(-1)
    assert np.all(bits(y) == 0)  # every term is +0 - +0: +0
    for kk in (0, 255, 777):
        x = np.zeros(k, np.float32)
        x[kk] = 1.0
        y = from_dev(rt.gemv_q4k_q8(d_blocks, to_dev(x), n, k)).reshape(-1)
        assert np.array_equal(bits(y), bits(orc.q4k_gemv_q8(blocks, n, k, x)))


def test_gemv_q4k_q8_deterministic_and_near_f32(rt, orc):
    """Two runs agree bit for bit, and the result is within the activation
    quantization's error (~0.4%, quant.hpp:160-170) of the f32 GEMV."""
    n, k = 3072, 3072
    rng = np.random.default_rng(9)
    blocks = orc.q4k_quantize((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    x = rng.standard_normal(k).astype(np.float32)
    d_blocks, d_x = to_dev(blocks), to_dev(x)
    a = from_dev(rt.gemv_q4k_q8(d_blocks, d_x, n, k)).reshape(-1)
    b = from_dev(rt.gemv_q4k_q8(d_blocks, d_x, n, k)).reshape(-1)
    assert np.array_equal(bits(a), bits(b))
    y32 = orc.q4k_matmul_t(blocks, n, k, x)[0]
    rel = np.linalg.norm(a - y32) / np.linalg.norm(y32)
    say(f"[q8 gemv] relative distance to the f32 path {rel:.2e}")
    assert 1e-4 < rel < 2e-2


def test_q8_errors(rt):
    import torch
    lib = rt.library()
    x = torch.zeros(4096, device="cuda")
    w = torch.zeros(64 * 16 * 144, dtype=torch.uint8, device="cuda")
    y = torch.empty(64, device="cuda")
    p = lambda t, off=0: t.data_ptr() + off  # noqa: E731
    assert lib.status("rt_hip_gemv_q4k_q8", p(w), p(x), p(y), 64, 4096, None) == 0
    assert lib.status("rt_hip_gemv_q4k_q8", p(w), p(x), p(y), 64, 1000, None) == 3    # k % 256
    assert lib.status("rt_hip_gemv_q4k_q8", p(w), p(x), p(x), 64, 256, None) == 1     # y overlaps x
    assert lib.status("rt_hip_gemv_q4k_q8", None, p(x), p(y), 64, 256, None) == 1     # null
    big = torch.zeros(16640, device="cuda")
    assert lib.status("rt_hip_gemv_q4k_tiled_q8", p(w), p(big), p(y), 1, 16640, None) == 2  # k > 16384
    q8 = torch.empty(4096, dtype=torch.int8, device="cuda")
    sc = torch.empty(128, device="cuda")
    assert lib.status("rt_hip_q4k_quantize_activation_q8", p(x), 4096, p(q8), p(sc), p(sc), None) == 1  # overlap
    assert lib.status("rt_hip_q4k_quantize_activation_q8", p(x, 2), 100, p(q8), p(sc), p(y), None) == 3  # align
    assert lib.status("rt_hip_q4k_quantize_activation_q8", p(x), 0, p(q8), p(sc), p(y), None) == 1
    torch.cuda.synchronize()
