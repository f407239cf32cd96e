"""The oracle's restatement of the Gemma 3 decode operations of the Metal
engine (src/shaders/decode_gemma3.msl) pinned without the reference (its
Metal code cannot run here): closed forms, invariants and float64.

* half() of the KV-cache append: IEEE round-to-nearest-even, checked against
  numpy's float16 conversion (itself RNE) on every half value, every midpoint
  between neighbouring halves (ties go to even), overflow and subnormal
  boundaries and 2 M random floats over the half range.
* gelu_tanh: float64 of the same formula; gelu(x) - gelu(-x) = x and
  gelu(0) = 0 (tanh is odd); the clamp of tanh's argument at +-10.
* rope_neox: position 0 is the identity bit for bit; each pair's length is
  kept; a float64 rotation by the same angles; the (i, i + d/2) pairing.
* rmsnorm_per_head: a constant head gives 1 + gamma; heads are independent;
  with eps = 0 a power-of-two scaling of a head does not change it; float64.
"""
import ctypes
import ctypes.util

import numpy as np
import pytest

_libm = ctypes.CDLL(ctypes.util.find_library("m"))
_libm.powf.restype = ctypes.c_float
_libm.powf.argtypes = [ctypes.c_float, ctypes.c_float]


def _powf(a: float, b: float) -> np.float32:
    return np.float32(_libm.powf(a, b))


def test_f16_rne_matches_ieee_everywhere(orc):
    halves = np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16)
    finite = halves[(halves & 0x7C00) != 0x7C00]
    vals = finite.view(np.float16).astype(np.float32)
    assert np.array_equal(orc.f32_to_f16_rne_n(vals), finite)          # exact halves round-trip
    # midpoints between consecutive finite halves of one sign: ties to even
    pos = np.sort(vals[vals > 0].astype(np.float64))
    mids = ((pos[:-1] + pos[1:]) / 2).astype(np.float32)
    assert np.array_equal(orc.f32_to_f16_rne_n(mids), mids.astype(np.float16).view(np.uint16))
    assert np.array_equal(orc.f32_to_f16_rne_n(-mids), (-mids).astype(np.float16).view(np.uint16))
    rng = np.random.default_rng(0)
    r = (rng.standard_normal(2_000_000) * np.exp2(rng.uniform(-26, 17, 2_000_000))).astype(np.float32)
    with np.errstate(over="ignore"):
        want = r.astype(np.float16).view(np.uint16)
    assert np.array_equal(orc.f32_to_f16_rne_n(r), want)
    edge = np.array([65504, 65519.99, 65520, 1e30, -65520, 2.0 ** -24, 2.0 ** -25, 2.0 ** -25 * 1.0001,
                     2.0 ** -14, 2.0 ** -14 * (1 - 2.0 ** -12), 0.0, -0.0, np.inf, -np.inf], np.float32)
    with np.errstate(over="ignore"):
        assert np.array_equal(orc.f32_to_f16_rne_n(edge), edge.astype(np.float16).view(np.uint16))


def test_gelu_tanh_closed_forms(orc):
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(100_000) * 4).astype(np.float32)
    g = orc.gelu_tanh(x).astype(np.float64)
    xd = x.astype(np.float64)
    inner = np.clip(0.7978845608 * (xd + 0.044715 * xd ** 3), -10, 10)
    ref = 0.5 * xd * (1 + np.tanh(inner))
    # f32 rounding of 0.5 v (1 + t): absolute error a few ulp of |v|
    scale = np.maximum(np.abs(ref), np.abs(xd))
    assert np.max(np.abs(g - ref) / np.maximum(scale, 1e-30)) < 1e-6
    # odd tanh: gelu(x) - gelu(-x) = x
    gm = orc.gelu_tanh(-x).astype(np.float64)
    assert np.max(np.abs((g - gm) - xd) / np.maximum(np.abs(xd), 1e-30)) < 1e-6
    assert orc.gelu_tanh(np.zeros(4, np.float32)).tolist() == [0.0] * 4
    # the clamp: for large |x| tanh saturates to +-1 (x or 0)
    big = np.array([30.0, -30.0], np.float32)
    assert orc.gelu_tanh(big).tolist() == [30.0, 0.0]


@pytest.mark.parametrize("head_dim", [64, 128, 256])
def test_rope_neox(orc, head_dim):
    rng = np.random.default_rng(head_dim)
    nh = 3
    x = rng.standard_normal(nh * head_dim).astype(np.float32)
    assert np.array_equal(orc.rope_neox(x, nh, head_dim, 10000.0, 1.0, 0).view(np.uint32), x.view(np.uint32))
    for pos, theta, fs in [(7, 10000.0, 1.0), (1234, 1e6, 0.125)]:
        y = orc.rope_neox(x, nh, head_dim, theta, fs, pos).reshape(nh, head_dim).astype(np.float64)
        xr = x.reshape(nh, head_dim).astype(np.float64)
        half = head_dim // 2
        i = np.arange(half)
        # the angle as f32 arithmetic forms it, with the C library's powf
        # (numpy's float32 power differs from it by an ulp at many points)
        expo = (np.float32(2.0) * i.astype(np.float32)) / np.float32(head_dim)
        den = np.array([_powf(theta, float(e)) for e in expo], np.float32)
        ang = (np.float32(pos) * np.float32(fs)) / den
        assert ang.dtype == np.float32
        c, s = np.cos(ang.astype(np.float64)), np.sin(ang.astype(np.float64))
        want0 = xr[:, :half] * c - xr[:, half:] * s
        want1 = xr[:, :half] * s + xr[:, half:] * c
        tol = 2e-6
        assert np.max(np.abs(y[:, :half] - want0)) < tol and np.max(np.abs(y[:, half:] - want1)) < tol
        n0 = xr[:, :half] ** 2 + xr[:, half:] ** 2
        n1 = y[:, :half] ** 2 + y[:, half:] ** 2
        assert np.max(np.abs(n1 - n0) / n0) < 1e-5


def test_rmsnorm_per_head(orc):
    rng = np.random.default_rng(5)
    nh, d = 4, 256
    g = (rng.standard_normal(d) * 0.1).astype(np.float32)
    const = np.full(nh * d, 3.0, np.float32)
    out = orc.rmsnorm_per_head(const, g, nh, d, 0.0).reshape(nh, d)
    assert np.allclose(out, np.broadcast_to(1.0 + g, (nh, d)), rtol=1e-6, atol=0)
    x = rng.standard_normal(nh * d).astype(np.float32)
    y = orc.rmsnorm_per_head(x, g, nh, d, 1e-6).reshape(nh, d)
    x2 = x.copy().reshape(nh, d)
    x2[1] *= 7.0
    y2 = orc.rmsnorm_per_head(x2.reshape(-1), g, nh, d, 1e-6).reshape(nh, d)
    assert np.array_equal(y[0], y2[0]) and np.array_equal(y[2:], y2[2:])  # heads independent
    x3 = x.copy().reshape(nh, d)
    x3[2] *= 8.0  # power of two, eps = 0: unchanged
    a = orc.rmsnorm_per_head(x, g, nh, d, 0.0).reshape(nh, d)
    b = orc.rmsnorm_per_head(x3.reshape(-1), g, nh, d, 0.0).reshape(nh, d)
    assert np.array_equal(a[2], b[2])
    xd = x.reshape(nh, d).astype(np.float64)
    ref = xd / np.sqrt((xd ** 2).mean(axis=1, keepdims=True) + 1e-6) * (1 + g.astype(np.float64))
    assert np.max(np.abs(y - ref)) < 1e-5
