"""Pins the CPU oracle (oracle/rt_oracle.c) before it is trusted as the checker.

Three independent sources pin it:
  * golden vectors written by the reference's own compiled code
    (tests/golden/ref_vectors.npz, from tests/golden/make_golden.py);
  * the live compiled reference (oracle/_ref), on fresh random and
    adversarial inputs, when it was built;
  * what the mathematics fixes: the reference tests' known-answer vectors,
    one-hot activations, fp64 brute force, special values of the conversions.
"""
import math
import os
import struct

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "ref_vectors.npz")


@pytest.fixture(scope="module")
def gold():
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


# ------------------------------------------------------------ golden vectors --

@pytest.mark.parametrize("tag", ["a", "b", "c"])
def test_q4k_golden(orc, gold, tag):
    w, x = gold[f"q4k_{tag}_w"], gold[f"q4k_{tag}_x"]
    rows, cols = w.shape
    blocks = orc.q4k_quantize(w)
    assert np.array_equal(blocks, gold[f"q4k_{tag}_blocks"])
    deq = orc.q4k_dequant(blocks, rows, cols)
    assert np.array_equal(bits(deq[:2]), bits(gold[f"q4k_{tag}_deq"]))
    y = orc.q4k_matmul_t(blocks, rows, cols, x)
    assert np.array_equal(bits(y), bits(gold[f"q4k_{tag}_y"]))


def test_q4k_golden_k1152_release_semantics(orc, gold):
    """K=1152: the reference's Release build keeps
    floor(1152/256) = 4 super-blocks per row and ignores x[1024:]."""
    w, x = gold["q4k_c_w"], gold["q4k_c_x"]
    rows = w.shape[0]
    blocks = gold["q4k_c_blocks"]
    assert blocks.size == rows * 4 * 144
    # Same bytes as quantizing the first 1024 columns as a K=1024 matrix ...
    assert np.array_equal(orc.q4k_quantize(w[:, :1024]), blocks)
    # ... and the same product as K=1024 with the first 1024 activations.
    y1024 = orc.q4k_matmul_t(blocks, rows, 1024, x[:, :1024])
    assert np.array_equal(bits(y1024), bits(gold["q4k_c_y"]))


def test_q4k_adversarial_golden(orc, gold):
    w = gold["q4k_adv_w"]
    blocks = orc.q4k_quantize(w)
    assert np.array_equal(blocks, gold["q4k_adv_blocks"])
    deq = orc.q4k_dequant(blocks, w.shape[0], 256)
    assert np.array_equal(bits(deq), bits(gold["q4k_adv_deq"]))


def test_q4k_from_bf16_golden(orc, gold):
    assert np.array_equal(orc.q4k_quantize_from_bf16(gold["q4k_bf16_bits"]),
                          gold["q4k_bf16_blocks"])


@pytest.mark.parametrize("tag", ["a", "b"])
def test_bf16_golden(orc, gold, tag):
    y = orc.bf16_matmul_t(gold[f"bf16_{tag}_w"], gold[f"bf16_{tag}_x"])
    assert np.array_equal(bits(y), bits(gold[f"bf16_{tag}_y"]))


def test_q4mat_golden(orc, gold):
    packed, scales = orc.q4mat_quantize(gold["q4mat_w"])
    assert np.array_equal(packed, gold["q4mat_packed"])
    assert np.array_equal(bits(scales), bits(gold["q4mat_scales"]))
    y = orc.q4mat_matmul_t(packed, scales, 20, 256, gold["q4mat_x"])
    assert np.array_equal(bits(y), bits(gold["q4mat_y"]))


def test_q8_activation_golden(orc, gold):
    q8, sc, su = orc.q4k_quantize_activation_q8(gold["q8_a"])
    assert np.array_equal(q8, gold["q8_q"])
    assert np.array_equal(bits(sc), bits(gold["q8_scales"]))
    assert np.array_equal(bits(su), bits(gold["q8_sums"]))


def test_conversions_golden(orc, gold):
    vals = gold["conv_vals"]
    assert [orc.f32_to_f16(float(v)) for v in vals] == gold["conv_f16"].tolist()
    assert [orc.f32_to_bf16(float(v)) for v in vals] == gold["conv_bf16"].tolist()


def test_initrng_golden(orc, gold):
    # libm log/cos: identical on this image's glibc; a different libm could
    # round differently, so compare to one ulp.
    a, b = orc.initrng_normal(0, 64), gold["initrng_seed0"]
    assert np.max(np.abs(a - b)) <= 1e-6 * np.max(np.abs(b))


# ------------------------------------------------- live compiled reference --

@pytest.mark.parametrize("rows,cols,m", [(7, 256, 1), (130, 512, 1), (257, 768, 1), (33, 1280, 2)])
def test_q4k_vs_reference(orc, ref, rows, cols, m):
    rng = np.random.default_rng(rows * 7919 + cols)
    w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    w[0, :32] = 0.0
    w[1 % rows, 32:64] = np.abs(w[1 % rows, 32:64])
    x = rng.standard_normal((m, cols)).astype(np.float32)
    qa, qb = orc.q4k_quantize(w), ref.q4k_quantize(w)
    assert np.array_equal(qa, qb)
    assert np.array_equal(bits(orc.q4k_dequant(qa, rows, cols)), bits(ref.q4k_dequant(qb, rows, cols)))
    assert np.array_equal(bits(orc.q4k_matmul_t(qa, rows, cols, x)),
                          bits(ref.q4k_matmul_t(qb, rows, cols, x)))
    for r in (0, rows - 1):
        assert struct.pack("f", orc.q4k_dot_row(qa, cols, r, x[0])) == \
            struct.pack("f", ref.q4k_dot_row(qb, rows, cols, r, x[0]))


def test_q4k_quantize_block_vs_reference_scaled(orc, ref):
    """Blocks across 12 decades of magnitude (f16 subnormal / overflow d)."""
    rng = np.random.default_rng(5)
    for e in range(-9, 4):
        x = (rng.standard_normal(256) * 10.0 ** e).astype(np.float32)
        assert np.array_equal(orc.q4k_quantize_block(x), ref.q4k_quantize_block(x)), e


@pytest.mark.parametrize("rows,cols,m", [(129, 200, 1), (40, 96, 3)])
def test_bf16_vs_reference(orc, ref, rows, cols, m):
    rng = np.random.default_rng(rows + cols)
    w = orc.f32_to_bf16_n((rng.standard_normal((rows, cols)) * 0.02).astype(np.float32))
    x = rng.standard_normal((m, cols)).astype(np.float32)
    assert np.array_equal(bits(orc.bf16_matmul_t(w, x)), bits(ref.bf16_matmul_t(w, x)))


def test_q4mat_vs_reference(orc, ref):
    rng = np.random.default_rng(11)
    w = (rng.standard_normal((33, 320)) * 0.5).astype(np.float32)
    w[3, :40] = 0.0
    pa, sa = orc.q4mat_quantize(w)
    pb, sb = ref.q4mat_quantize(w)
    assert np.array_equal(pa, pb) and np.array_equal(bits(sa), bits(sb))
    x = rng.standard_normal((3, 320)).astype(np.float32)
    assert np.array_equal(bits(orc.q4mat_matmul_t(pa, sa, 33, 320, x)),
                          bits(ref.q4mat_matmul_t(pb, sb, 33, 320, x)))


def test_conversions_exhaustive_vs_reference(orc, ref):
    for b in range(0, 65536, 7):
        assert struct.pack("f", orc.f16_to_f32(b)) == struct.pack("f", ref.f16_to_f32(b))
    rng = np.random.default_rng(3)
    for u in rng.integers(0, 2**32, 20000, dtype=np.uint64):
        v = struct.unpack("f", struct.pack("I", int(u)))[0]
        assert orc.f32_to_f16(v) == ref.f32_to_f16(v)
        assert orc.f32_to_bf16(v) == ref.f32_to_bf16(v)


def test_initrng_vs_reference(orc, ref):
    assert np.array_equal(bits(orc.initrng_normal(7, 5000, 0.02)), bits(ref.initrng_normal(7, 5000, 0.02)))


# ------------------------------------------------- what the mathematics fixes --

def test_scale_min_pack_roundtrip(orc):
    """tests/test_gguf.cpp:379-404: pack known 6-bit values, unpack them."""
    sv = [5, 17, 33, 62, 9, 40, 55, 63]
    mv = [1, 22, 44, 60, 3, 31, 50, 61]
    sc = orc.q4k_pack_scales(sv, mv)
    for j in range(8):
        assert orc.q4k_scale_min(sc, j) == (float(sv[j]), float(mv[j]))


def test_scale_min_exhaustive_roundtrip(orc):
    rng = np.random.default_rng(0)
    for _ in range(300):
        sv, mv = rng.integers(0, 64, 8), rng.integers(0, 64, 8)
        sc = orc.q4k_pack_scales(sv, mv)
        assert [orc.q4k_scale_min(sc, j) for j in range(8)] == \
            [(float(a), float(b)) for a, b in zip(sv, mv)]


def _f16(v: float) -> int:
    return int(np.array([v], np.float16).view(np.uint16)[0])


def test_q4k_dequant_hand_built_block(orc):
    """A block with chosen d, dmin, scales and nibbles against the closed form
    w = (d*sv)*q - dmin*mv, value 64c+l <- low nibble of qs[32c+l] (sub-block
    2c), value 64c+32+l <- high nibble (sub-block 2c+1)."""
    d, dmin = 0.5, 0.25
    sv = [1, 2, 3, 4, 5, 6, 7, 63]
    mv = [0, 1, 2, 3, 60, 5, 6, 7]
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.frombuffer(struct.pack("<H", _f16(d)), np.uint8)
    blk[2:4] = np.frombuffer(struct.pack("<H", _f16(dmin)), np.uint8)
    blk[4:16] = orc.q4k_pack_scales(sv, mv)
    qs = np.array([(i * 7 + 3) & 0xff for i in range(128)], np.uint8)
    blk[16:] = qs
    got = orc.q4k_dequant(blk, 1, 256)[0]
    for c in range(4):
        for l in range(32):
            q = int(qs[32 * c + l])
            want_lo = np.float32(d * sv[2 * c]) * np.float32(q & 15) - np.float32(dmin * mv[2 * c])
            want_hi = np.float32(d * sv[2 * c + 1]) * np.float32(q >> 4) - np.float32(dmin * mv[2 * c + 1])
            assert got[64 * c + l] == np.float32(want_lo)
            assert got[64 * c + 32 + l] == np.float32(want_hi)


def test_q4k_one_hot_reproduces_dequant_columns(orc):
    """x = e_k makes every factorized dot collapse to the dequant expression,
    so y must equal column k of the dequantized weight bit-for-bit."""
    rng = np.random.default_rng(1)
    rows, cols = 9, 512
    blocks = orc.q4k_quantize((rng.standard_normal((rows, cols)) * 0.02).astype(np.float32))
    deq = orc.q4k_dequant(blocks, rows, cols)
    for k in (0, 1, 31, 32, 63, 64, 100, 255, 256, 300, 511):
        x = np.zeros(cols, np.float32)
        x[k] = 1.0
        y = orc.q4k_matmul_t(blocks, rows, cols, x, n_threads=1)[0]
        assert np.array_equal(bits(y), bits(deq[:, k])), k


def test_q4k_gemv_fp64_brute_force(orc):
    rng = np.random.default_rng(2)
    rows, cols = 150, 768
    blocks = orc.q4k_quantize((rng.standard_normal((rows, cols)) * 0.02).astype(np.float32))
    x = rng.standard_normal(cols).astype(np.float32)
    y = orc.q4k_matmul_t(blocks, rows, cols, x)[0].astype(np.float64)
    exact = orc.q4k_dequant(blocks, rows, cols).astype(np.float64) @ x.astype(np.float64)
    assert np.max(np.abs(y - exact)) <= 1e-5 * np.max(np.abs(exact))


def test_q4k_quantizer_properties(orc):
    """tests/test_quant.cpp:138-204: zeros stay zero; the sin matrix
    round-trips within 0.15; quantize_from_bf16 == quantize(to_f32)."""
    z = orc.q4k_quantize(np.zeros((2, 256), np.float32))
    assert not z.any()
    r, c = np.meshgrid(np.arange(4), np.arange(256), indexing="ij")
    src = (np.sin((r * 256 + c).astype(np.float32) * np.float32(0.01)) * np.float32(0.8)).astype(np.float32)
    deq = orc.q4k_dequant(orc.q4k_quantize(src), 4, 256)
    assert np.max(np.abs(deq - src)) < 0.15
    b = orc.f32_to_bf16_n(src)
    f = (b.astype(np.uint32) << 16).view(np.float32)
    assert np.array_equal(orc.q4k_quantize_from_bf16(b), orc.q4k_quantize(f))


def test_q4_0_hand_built_block(orc):
    """tests/test_gguf.cpp:175-218: one block, scale 0.25, values (i-8)*0.25
    clamped to [-8, 7]*scale; flat decode within scale/2; Q4Mat decode equal."""
    scale = 0.25
    vals = np.clip((np.arange(32, dtype=np.float32) - 8.0) * scale, -8 * scale, 7 * scale).astype(np.float32)
    blk = orc.q4_0_encode_block(vals, scale)
    flat = orc.q4_0_decode(blk, 32)
    assert np.all(np.abs(flat - vals) <= scale * 0.5 + 1e-5)
    packed, scales = orc.q4_0_to_q4mat(blk, 32)
    assert np.all(np.abs(orc.q4mat_dequant(packed, scales, 32) - flat) < 1e-6)
    # closed form of the split layout: qs[k] low -> k, high -> k+16
    for k in range(16):
        q = int(blk[2 + k])
        assert flat[k] == np.float32(((q & 15) - 8) * scale)
        assert flat[k + 16] == np.float32(((q >> 4) - 8) * scale)


class MT19937:
    """std::mt19937 (Matsumoto & Nishimura 1998), for the reference's Q6_K block."""

    def __init__(self, seed: int):
        self.mt = [0] * 624
        self.mt[0] = seed & 0xffffffff
        for i in range(1, 624):
            self.mt[i] = (1812433253 * (self.mt[i - 1] ^ (self.mt[i - 1] >> 30)) + i) & 0xffffffff
        self.i = 624

    def __call__(self) -> int:
        if self.i >= 624:
            for k in range(624):
                y = (self.mt[k] & 0x80000000) | (self.mt[(k + 1) % 624] & 0x7fffffff)
                self.mt[k] = self.mt[(k + 397) % 624] ^ (y >> 1) ^ (0x9908b0df if y & 1 else 0)
            self.i = 0
        y = self.mt[self.i]
        self.i += 1
        y ^= y >> 11
        y ^= (y << 7) & 0x9d2c5680
        y ^= (y << 15) & 0xefc60000
        y ^= y >> 18
        return y & 0xffffffff


def test_mt19937_known_answer():
    # The 10000th output of a default-seeded std::mt19937 is 4123659995 (C++11 [rand.predef]).
    g = MT19937(5489)
    for _ in range(9999):
        g()
    assert g() == 4123659995


def test_q6k_known_block(orc):
    """tests/test_gguf.cpp:292-335: random ql/qh from mt19937(1234), int8
    scales (i*7)%61-30, d=0.0125; values l and l+64 of each half follow
    q = (ql nibble | 2 bits of qh << 4) - 32, w = d*sc*q."""
    g = MT19937(1234)
    blk = np.zeros(210, np.uint8)
    for i in range(192):
        blk[i] = g() & 0xff
    for i in range(16):
        blk[192 + i] = np.uint8(np.int8((i * 7) % 61 - 30).view(np.uint8))
    h = orc.f32_to_f16(0.0125)
    blk[208], blk[209] = h & 0xff, h >> 8
    out = orc.q6k_decode(blk, 256)
    dd = orc.f16_to_f32(h)
    sc = blk[192:208].view(np.int8)
    for j in range(2):
        ql = [int(v) for v in blk[j * 64:j * 64 + 64]]
        qh = [int(v) for v in blk[128 + j * 32:128 + j * 32 + 32]]
        for l in range(32):
            is_ = l // 16
            q1 = ((ql[l] & 15) | (((qh[l] >> 0) & 3) << 4)) - 32
            q2 = ((ql[l + 32] & 15) | (((qh[l] >> 2) & 3) << 4)) - 32
            q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32
            q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32
            base = j * 128
            for off, q, s in ((0, q1, sc[8 * j + is_]), (32, q2, sc[8 * j + is_ + 2]),
                              (64, q3, sc[8 * j + is_ + 4]), (96, q4, sc[8 * j + is_ + 6])):
                want = np.float32(np.float32(dd) * np.float32(s)) * np.float32(q)
                assert out[base + l + off] == want


def test_argmax_rules(orc):
    """transformer5.cpp:382-391: first index of the strict maximum; NaN never
    wins; nothing above -inf gives 0; -0 does not beat +0 nor vice versa."""
    assert orc.argmax_first([1.0, 3.0, 3.0, 2.0]) == 1
    assert orc.argmax_first([math.nan, 1.0, math.nan, 5.0, 5.0]) == 3
    assert orc.argmax_first([-math.inf, -math.inf]) == 0
    assert orc.argmax_first([math.nan, math.nan]) == 0
    assert orc.argmax_first([-1.0, -0.0, 0.0]) == 1
    assert orc.argmax_first([-5.0, math.inf, math.inf]) == 1


def test_f16_special_values(orc):
    assert orc.f32_to_f16(65504.0) == 0x7bff
    assert orc.f32_to_f16(65536.0) == 0x7c00           # overflow -> inf
    assert orc.f32_to_f16(1.0 + 2 ** -11) == 0x3c00    # truncates (RNE would too: tie)
    assert orc.f32_to_f16(1.0 + 3 * 2 ** -12) == 0x3c00  # truncation, RNE gives 0x3c01
    assert orc.f32_to_f16(2 ** -24) == 0x0001          # smallest subnormal
    assert orc.f32_to_f16(2 ** -25) == 0x0000          # below: flushed
    for b in range(0, 0x7c00, 37):                     # f16 -> f32 -> f16 is the identity
        assert orc.f32_to_f16(orc.f16_to_f32(b)) == b
        assert orc.f16_to_f32(b) == float(np.array([b], np.uint16).view(np.float16)[0])


def test_bf16_rne(orc):
    one = 0x3f800000
    f = lambda u: struct.unpack("f", struct.pack("I", u))[0]  # noqa: E731
    assert orc.f32_to_bf16(f(one | 0x8000)) == 0x3f80        # tie -> even
    assert orc.f32_to_bf16(f(one | 0x18000)) == 0x3f82       # tie -> even (up)
    assert orc.f32_to_bf16(f(one | 0x8001)) == 0x3f81        # above half
    assert orc.f32_to_bf16(math.nan) & 0x7fc0 == 0x7fc0
