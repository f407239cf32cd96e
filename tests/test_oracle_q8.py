"""Pins the oracle's Q4_K x Q8-activation product (dot_row_q8,
quant_q4k.cpp:425-478, and gemv_mt's aarch64 branch, :564-600) before the
GPU's Q8 GEMV is checked against it.

dot_row_q8 is NEON-only, so the reference cannot be compiled here for it;
its quantizer half (quantize_activation_q8) is pinned by the reference's own
golden vectors in test_oracle.py.  What pins the product:

* a per-element float64 evaluation of what the reference's formula means,
      sum_k (d*sv)_k * q4_k * (q8_k * scale_k)  -  (dmin*mv)_k * a_k,
  built from the block bytes element by element (not chunk by chunk), within
  an f32 rounding bound of the oracle's result -- and the same check rejects
  planted mistakes (the min term dropped, the two sub-blocks of a chunk
  swapped, the quantized activation used in the min term);
* activations that Q8 represents exactly: the product then equals the f64
  dot of the dequantized weights with the activation;
* one-hot activations in closed form;
* the error bound of the activation quantization against the f32 path.
"""
import numpy as np
import pytest


def q4k_weights(orc, rows, cols, seed, std=0.02):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((rows, cols)) * std).astype(np.float32)
    return orc.q4k_quantize(w)


def element_terms(orc, blocks, cols, row):
    """Per element k of row `row`: (d*sv)_k, (dmin*mv)_k and the nibble q4_k,
    read from the 144-byte blocks (d, dmin f16 at 0 and 2, scales at 4..15,
    qs at 16..143; chunk c: low nibbles of qs[32c..32c+32) are values
    64c..64c+31, high nibbles 64c+32..64c+63)."""
    nb = cols // 256
    blk = np.asarray(blocks, np.uint8).reshape(-1, 144)[row * nb:(row + 1) * nb]
    ds = np.zeros(cols)
    dm = np.zeros(cols)
    q4 = np.zeros(cols)
    for b in range(nb):
        bp = blk[b]
        d = orc.f16_to_f32(int(bp[0]) | (int(bp[1]) << 8))
        dmin = orc.f16_to_f32(int(bp[2]) | (int(bp[3]) << 8))
        sc = np.ascontiguousarray(bp[4:16])
        qs = bp[16:144]
        for j in range(8):
            sv, mv = orc.q4k_scale_min(sc, j)
            c, hi = j // 2, j % 2
            sl = slice(b * 256 + 32 * j, b * 256 + 32 * j + 32)
            ds[sl] = float(d) * float(sv)
            dm[sl] = float(dmin) * float(mv)
            q = qs[32 * c:32 * c + 32]
            q4[sl] = (q >> 4) if hi else (q & 0x0F)
    return ds, dm, q4


def f64_q8_dot(ds, dm, q4, q8, scales, a):
    k = a.size
    ahat = q8[:k].astype(np.float64) * np.repeat(scales.astype(np.float64), 32)[:k]
    terms = ds * q4 * ahat - dm * a.astype(np.float64)
    return float(np.sum(terms)), float(np.sum(np.abs(ds * q4 * ahat)) + np.sum(np.abs(dm * a)))


def within(got, want, mag, cols):
    # f32 rounding of 4 products and 4 sums per 64-value chunk plus the
    # running total: a generous 8 * (chunks + 8) ulps of the magnitude.
    return abs(got - want) <= 8.0 * (cols / 64 + 8) * 2.0 ** -24 * mag


@pytest.mark.parametrize("rows,cols,seed,std", [(4, 256, 1, 1.0), (3, 1024, 2, 0.3), (2, 3072, 3, 5.0)])
def test_q8_dot_matches_f64_meaning(orc, rows, cols, seed, std):
    blocks = q4k_weights(orc, rows, cols, seed)
    rng = np.random.default_rng(seed + 100)
    a = (rng.standard_normal(cols) * std).astype(np.float32)
    q8, sc, su = orc.q4k_quantize_activation_q8(a)
    for r in range(rows):
        got = orc.q4k_dot_row_q8(blocks, cols, r, q8, sc, su)
        ds, dm, q4 = element_terms(orc, blocks, cols, r)
        want, mag = f64_q8_dot(ds, dm, q4, q8, sc, a)
        assert within(got, want, mag, cols), (r, got, want)


def test_q8_dot_check_rejects_planted_mistakes(orc):
    """The f64 check above is sharp enough to see each plausible slip."""
    rows, cols = 2, 1024
    blocks = q4k_weights(orc, rows, cols, 7)
    a = (np.random.default_rng(8).standard_normal(cols) + 0.7).astype(np.float32)
    q8, sc, su = orc.q4k_quantize_activation_q8(a)
    ds, dm, q4 = element_terms(orc, blocks, cols, 0)
    want, mag = f64_q8_dot(ds, dm, q4, q8, sc, a)
    got = orc.q4k_dot_row_q8(blocks, cols, 0, q8, sc, su)
    assert within(got, want, mag, cols)
    ahat = q8.astype(np.float64) * np.repeat(sc.astype(np.float64), 32)
    # 1. the min term dropped
    assert not within(got + float(np.sum(dm * a)), want, mag, cols)
    # 2. the quantized activation in the min term instead of the sum of a
    wrong = float(np.sum(ds * q4 * ahat - dm * ahat))
    assert not within(wrong, want, mag, cols)
    # 3. the two sub-blocks of every chunk exchanged (nibble halves swapped)
    perm = np.arange(cols).reshape(-1, 2, 32)[:, ::-1, :].reshape(-1)
    wrong = float(np.sum(ds[perm] * q4[perm] * ahat - dm[perm] * a))
    assert not within(wrong, want, mag, cols)


def test_q8_dot_exact_activations_equal_f32_product(orc):
    """a = q * 2^-7 with |q| <= 127 and a +-127 in every 32-block: scale is
    2^-7 exactly, q8 = q, and the product is the f64 dot of the dequantized
    weights with a, to f32 rounding."""
    rows, cols = 3, 2048
    blocks = q4k_weights(orc, rows, cols, 11)
    rng = np.random.default_rng(12)
    q = rng.integers(-127, 128, cols)
    q[::32] = 127 * np.where(rng.integers(0, 2, cols // 32) > 0, 1, -1)
    a = (q * 2.0 ** -7).astype(np.float32)
    q8, sc, su = orc.q4k_quantize_activation_q8(a)
    assert np.array_equal(q8[:cols], q.astype(np.int8))
    assert np.all(sc == np.float32(2.0 ** -7))
    wdq = orc.q4k_dequant(blocks, rows, cols).astype(np.float64)
    for r in range(rows):
        got = orc.q4k_dot_row_q8(blocks, cols, r, q8, sc, su)
        want = float(wdq[r] @ a.astype(np.float64))
        mag = float(np.abs(wdq[r]) @ np.abs(a.astype(np.float64)))
        assert within(got, want, mag, cols), (r, got, want)


def test_q8_dot_one_hot_closed_form(orc):
    """x = e_k: only k's 32-block is live (scale 1/127, q8 = 127, sum 1), so
    the product is ((d*sv) * (1/127)) * (127 * q4) - dmin*mv, and every other
    block contributes exact zeros."""
    rows, cols = 2, 512
    blocks = q4k_weights(orc, rows, cols, 21)
    f32 = np.float32
    for k in (0, 31, 32, 100, 255, 256, 300, 511):
        a = np.zeros(cols, np.float32)
        a[k] = 1.0
        q8, sc, su = orc.q4k_quantize_activation_q8(a)
        assert q8[k] == 127 and sc[k // 32] == f32(1.0) / f32(127.0) and su[k // 32] == 1.0
        for r in range(rows):
            ds, dm, q4 = element_terms(orc, blocks, cols, r)
            want = f32(f32(f32(ds[k]) * sc[k // 32]) * f32(127 * q4[k])) - f32(dm[k])
            got = orc.q4k_dot_row_q8(blocks, cols, r, q8, sc, su)
            assert np.float32(got) == want, (k, r)


def test_q8_error_bound_against_f32_path(orc):
    """|q8 product - f32 product| <= sum_k |(d*sv)_k q4_k| * |a_k - q8_k scale_k|
    (+ rounding): the quantization error of the activation, nothing else."""
    rows, cols = 4, 3072
    blocks = q4k_weights(orc, rows, cols, 31)
    a = np.random.default_rng(32).standard_normal(cols).astype(np.float32)
    q8, sc, su = orc.q4k_quantize_activation_q8(a)
    ahat = q8.astype(np.float64) * np.repeat(sc.astype(np.float64), 32)
    y8 = orc.q4k_gemv_q8(blocks, rows, cols, a)
    y32 = orc.q4k_matmul_t(blocks, rows, cols, a)[0]
    for r in range(rows):
        ds, dm, q4 = element_terms(orc, blocks, cols, r)
        bound = float(np.sum(np.abs(ds * q4) * np.abs(ahat - a))) + 1e-5 * float(np.sum(np.abs(ds * q4 * a)))
        assert abs(float(y8[r]) - float(y32[r])) <= bound
        # and the quantization did move the result (the path is not the f32 one)
        assert y8[r] != y32[r]


def test_q8_gemv_is_dot_row_q8_per_row(orc):
    rows, cols = 5, 768
    blocks = q4k_weights(orc, rows, cols, 41)
    a = np.random.default_rng(42).standard_normal(cols).astype(np.float32)
    q8, sc, su = orc.q4k_quantize_activation_q8(a)
    y = orc.q4k_gemv_q8(blocks, rows, cols, a)
    for r in range(rows):
        assert np.float32(orc.q4k_dot_row_q8(blocks, cols, r, q8, sc, su)) == y[r]
