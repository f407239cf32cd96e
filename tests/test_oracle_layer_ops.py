"""Pins the oracle's RMSNorm and SwiGLU (orc_rmsnorm / orc_swiglu, restating
tensor_node.cpp:320-344, 383-402 and transformer5.cpp:186-190) by what the
mathematics fixes: closed forms, exact invariances and float64 evaluations of
the same formulas.  CPU only."""
import numpy as np


def test_rmsnorm_constant_row_closed_form(orc):
    d = 3072
    rng = np.random.default_rng(0)
    gamma = rng.standard_normal(d).astype(np.float32)
    for c, eps in ((0.5, 1e-5), (3.0, 1e-6), (-2.0, 0.0), (1e-3, 1e-5)):
        x = np.full(d, c, np.float32)
        got = orc.rmsnorm(x, gamma, eps).astype(np.float64)
        want = c / np.sqrt(c * c + eps) * gamma.astype(np.float64)
        assert np.allclose(got, want, rtol=2e-6, atol=0), (c, eps)


def test_rmsnorm_gemma3_is_the_plain_form_on_one_plus_gamma(orc):
    rng = np.random.default_rng(1)
    x = rng.standard_normal((3, 1024)).astype(np.float32)
    gamma = (rng.standard_normal(1024) * 0.1).astype(np.float32)
    one_plus = (np.float32(1.0) + gamma).astype(np.float32)
    assert np.array_equal(orc.rmsnorm(x, gamma, 1e-6, gemma3=True), orc.rmsnorm(x, one_plus, 1e-6))


def test_rmsnorm_power_of_two_scale_invariance(orc):
    """With eps = 0 every step commutes with scaling x by 2^s: the outputs
    are identical bit for bit (a missing sqrt or a wrong divisor breaks it)."""
    rng = np.random.default_rng(2)
    x = rng.standard_normal(2048).astype(np.float32)
    gamma = rng.standard_normal(2048).astype(np.float32)
    base = orc.rmsnorm(x, gamma, 0.0)
    for s in (-6, -1, 3, 9):
        assert np.array_equal(orc.rmsnorm(x * np.float32(2.0 ** s), gamma, 0.0), base), s


def test_rmsnorm_random_rows_against_float64(orc):
    rng = np.random.default_rng(3)
    for d in (256, 3072, 8192):
        x = (rng.standard_normal(d) * rng.uniform(0.01, 10)).astype(np.float32)
        gamma = rng.standard_normal(d).astype(np.float32)
        x64 = x.astype(np.float64)
        want = x64 / np.sqrt(np.mean(x64 * x64) + 1e-5) * gamma
        got = orc.rmsnorm(x, gamma, 1e-5)
        assert np.max(np.abs(got - want)) <= 4e-6 * np.max(np.abs(want)), d


def test_silu_fixed_points_and_odd_identity(orc):
    ones = np.ones(7, np.float32)
    g = np.array([0.0, 30.0, 100.0, -30.0, -100.0, 1.0, -1.0], np.float32)
    s = orc.swiglu(g, ones)
    assert s[0] == 0.0
    assert s[1] == np.float32(30.0) and s[2] == np.float32(100.0)  # sigmoid rounds to 1
    assert -1e-11 < s[3] < 0.0  # -30 * sigmoid(-30)
    assert abs(s[4]) < 1e-40
    rng = np.random.default_rng(4)
    x = (rng.standard_normal(4096) * 4).astype(np.float32)
    one = np.ones_like(x)
    # silu(x) - silu(-x) = x (sigmoid(x) + sigmoid(-x) = 1)
    diff = orc.swiglu(x, one).astype(np.float64) - orc.swiglu(-x, one).astype(np.float64)
    assert np.allclose(diff, x.astype(np.float64), rtol=0, atol=4e-6 * (1 + np.abs(x)).max())


def test_swiglu_against_float64(orc):
    rng = np.random.default_rng(5)
    g = (rng.standard_normal(8192) * 3).astype(np.float32)
    u = rng.standard_normal(8192).astype(np.float32)
    g64 = g.astype(np.float64)
    want = g64 / (1.0 + np.exp(-g64)) * u.astype(np.float64)
    got = orc.swiglu(g, u).astype(np.float64)
    assert np.allclose(got, want, rtol=1e-6, atol=1e-30)


def test_llama_inv_freq_against_float64(orc):
    theta, hd = 500000.0, 128
    got = orc.llama_inv_freq(theta, hd).astype(np.float64)
    want = 1.0 / theta ** (2.0 * np.arange(hd // 2) / hd)
    assert np.allclose(got, want, rtol=2e-6, atol=0)
    div = np.array([1.0, 2.0, 0.0, 32.0], np.float32)
    got_d = orc.llama_inv_freq(theta, hd, div).astype(np.float64)
    want_d = want.copy()
    for i, d in enumerate(div):
        if d > 0:
            want_d[i] /= d
    assert np.allclose(got_d, want_d, rtol=3e-6, atol=0)


def test_llama_rope_interleaved(orc):
    rng = np.random.default_rng(6)
    n_heads, hd = 8, 128
    inv = orc.llama_inv_freq(500000.0, hd)
    x = rng.standard_normal(n_heads * hd).astype(np.float32)
    assert np.array_equal(orc.llama_rope(x, n_heads, hd, 0, inv), x)  # pos 0: identity
    for pos in (1, 17, 1000, 100000):
        got = orc.llama_rope(x, n_heads, hd, pos, inv).astype(np.float64)
        ang = (np.float32(pos) * inv).astype(np.float32).astype(np.float64)  # the f32 angle
        c, s = np.cos(ang), np.sin(ang)
        x2 = x.astype(np.float64).reshape(n_heads, hd // 2, 2)
        want = np.stack([x2[..., 0] * c - x2[..., 1] * s, x2[..., 0] * s + x2[..., 1] * c], axis=-1).reshape(-1)
        assert np.allclose(got, want, rtol=0, atol=1e-5 * np.abs(x).max()), pos
        # each pair keeps its length
        g2 = got.reshape(n_heads, hd // 2, 2)
        assert np.allclose(np.hypot(g2[..., 0], g2[..., 1]), np.hypot(x2[..., 0], x2[..., 1]), rtol=1e-5)


def test_llama_rope_half_split(orc):
    """Half-split pairing (i, i + head_dim/2): pos 0 is the identity; a float64
    rotation by the same f32 angles; and, bit for bit, the interleaved
    rotation of the head-wise permuted row (2j <- j, 2j+1 <- j + half),
    permuted back -- the identity the GPU path's row permutation uses."""
    rng = np.random.default_rng(8)
    n_heads, hd = 8, 128
    half = hd // 2
    inv = orc.llama_inv_freq(500000.0, hd)
    x = rng.standard_normal(n_heads * hd).astype(np.float32)
    assert np.array_equal(orc.llama_rope(x, n_heads, hd, 0, inv, half=True), x)
    perm = np.concatenate([h * hd + np.stack([np.arange(half), np.arange(half) + half], axis=1).reshape(-1)
                           for h in range(n_heads)])  # interleaved slot -> half-split index
    for pos in (1, 17, 1000, 100000):
        got = orc.llama_rope(x, n_heads, hd, pos, inv, half=True)
        ang = (np.float32(pos) * inv).astype(np.float32).astype(np.float64)
        c, s = np.cos(ang), np.sin(ang)
        x3 = x.astype(np.float64).reshape(n_heads, 2, half)
        want = np.stack([x3[:, 0] * c - x3[:, 1] * s, x3[:, 0] * s + x3[:, 1] * c], axis=1).reshape(-1)
        assert np.allclose(got, want, rtol=0, atol=1e-5 * np.abs(x).max()), pos
        inter = orc.llama_rope(x[perm], n_heads, hd, pos, inv)
        back = np.empty_like(inter)
        back[perm] = inter
        assert np.array_equal(back, got), pos
        assert not np.array_equal(got, orc.llama_rope(x, n_heads, hd, pos, inv)), pos  # the pairings differ


def test_gqa_attention_decode(orc):
    rng = np.random.default_rng(7)
    nq, nkv, d = 6, 2, 128
    scale = 1.0 / np.sqrt(d)
    q = rng.standard_normal(nq * d).astype(np.float32)
    # one cached position: out = v exactly
    k1 = rng.standard_normal((1, nkv * d)).astype(np.float32)
    v1 = rng.standard_normal((1, nkv * d)).astype(np.float32)
    out = orc.gqa_attention_decode(q, k1, v1, 1, nq, nkv, d, scale).reshape(nq, d)
    for h in range(nq):
        assert np.array_equal(out[h], v1[0, (h // 3) * d:(h // 3 + 1) * d]), h
    # equal keys: the mean of the values (per KV head)
    L = 10
    kc = np.tile(rng.standard_normal((1, nkv * d)).astype(np.float32), (L, 1))
    vc = rng.standard_normal((L, nkv * d)).astype(np.float32)
    out = orc.gqa_attention_decode(q, kc, vc, L, nq, nkv, d, scale).reshape(nq, d)
    for h in range(nq):
        want = vc[:, (h // 3) * d:(h // 3 + 1) * d].astype(np.float64).mean(axis=0)
        assert np.allclose(out[h], want, rtol=1e-5, atol=1e-6), h
    # random: float64 softmax of the same scores
    L = 37
    kc = rng.standard_normal((L, nkv * d)).astype(np.float32)
    vc = rng.standard_normal((L, nkv * d)).astype(np.float32)
    out = orc.gqa_attention_decode(q, kc, vc, L, nq, nkv, d, scale).reshape(nq, d)
    for h in range(nq):
        kh = kc[:, (h // 3) * d:(h // 3 + 1) * d].astype(np.float64)
        vh = vc[:, (h // 3) * d:(h // 3 + 1) * d].astype(np.float64)
        s = kh @ q[h * d:(h + 1) * d].astype(np.float64) * scale
        p = np.exp(s - s.max())
        p /= p.sum()
        assert np.allclose(out[h], p @ vh, rtol=0, atol=2e-6), h
