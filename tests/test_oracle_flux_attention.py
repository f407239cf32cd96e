"""The oracle's restatement of FLUX's CPU attention (flux.cpp:287-321) pinned
without the reference (flux.cpp's attention sits in an anonymous namespace of
a translation unit that needs the whole FLUX model to link, so it is not
built into oracle/_ref):

* one key: the output row is v bit for bit (weight exp(0) / 1 = 1);
* a dominant key whose score leads every other by more than 104 (exp of the
  gap underflows to 0 in f32): the output row is that key's v bit for bit;
* q = 0: every weight is 1/t, so the output is the mean of v (float64);
* float64 softmax attention on random inputs, plain and peaky scores;
* permuting the keys (k and v together) leaves the output unchanged to
  rounding; a head's output ignores every other head's inputs;
* a subset of output rows equals the same rows of the full computation bit
  for bit.
A wrong scale, a transposed operand, a wrong head offset or a v row taken
from the wrong key fails one of these.
"""
import numpy as np

from helpers import normwise_err


def attn64(q, k, v, h, d):
    """float64 softmax attention, per head."""
    t = q.shape[0]
    out = np.zeros((t, h * d))
    for i in range(h):
        sl = slice(i * d, (i + 1) * d)
        s = q[:, sl].astype(np.float64) @ k[:, sl].astype(np.float64).T / np.sqrt(d)
        p = np.exp(s - s.max(axis=1, keepdims=True))
        p /= p.sum(axis=1, keepdims=True)
        out[:, sl] = p @ v[:, sl].astype(np.float64)
    return out


def rand(rng, t, h, d, std=1.0):
    return [(rng.standard_normal((t, h * d)) * std).astype(np.float32) for _ in range(3)]


def test_one_key_gives_v(orc):
    rng = np.random.default_rng(0)
    q, k, v = rand(rng, 1, 3, 64)
    out = orc.flux_attention(q, k, v, 3, 64)
    assert np.array_equal(out.view(np.uint32), v.view(np.uint32))


def test_dominant_key_gives_its_v(orc):
    rng = np.random.default_rng(1)
    t, h, d = 37, 2, 32
    q, k, v = rand(rng, t, h, d, 0.05)
    star = 23
    # q . k_star / sqrt(d) ~ 200 against |q . k_j| / sqrt(d) < 1 elsewhere
    k[star] = q[5] * np.float32(200.0 * np.sqrt(d) / np.mean(np.square(q[5])) / d)
    out = orc.flux_attention(q, k, v, h, d, rows=[5])
    assert np.array_equal(out[0].view(np.uint32), v[star].view(np.uint32))


def test_zero_query_averages_v(orc):
    rng = np.random.default_rng(2)
    t, h, d = 300, 2, 64
    _, k, v = rand(rng, t, h, d)
    q = np.zeros_like(k)
    out = orc.flux_attention(q, k, v, h, d)
    want = np.broadcast_to(v.astype(np.float64).mean(axis=0), out.shape)
    # 300 sequential f32 additions of (1/t) v: a few hundred ulp at most
    assert np.max(np.abs(out - want)) <= 300 * 2.0 ** -24 * np.max(np.abs(v))


def test_float64_attention(orc):
    rng = np.random.default_rng(3)
    for t, h, d, std in ((50, 3, 128, 1.0), (129, 2, 64, 1.0), (64, 1, 16, 3.0), (200, 4, 72, 2.0)):
        q, k, v = rand(rng, t, h, d, std)
        out = orc.flux_attention(q, k, v, h, d)
        ref = attn64(q, k, v, h, d)
        assert normwise_err(out, ref) <= 2e-6, (t, h, d, std, normwise_err(out, ref))


def test_key_permutation_and_head_independence(orc):
    rng = np.random.default_rng(4)
    t, h, d = 96, 3, 32
    q, k, v = rand(rng, t, h, d)
    out = orc.flux_attention(q, k, v, h, d)
    perm = rng.permutation(t)
    outp = orc.flux_attention(q, k[perm], v[perm], h, d)
    assert normwise_err(outp, out) <= 2e-6
    k2, v2, q2 = k.copy(), v.copy(), q.copy()
    for a in (q2, k2, v2):
        a[:, d:2 * d] = rng.standard_normal((t, d))  # head 1 only
    out2 = orc.flux_attention(q2, k2, v2, h, d)
    for hh in (0, 2):
        sl = slice(hh * d, (hh + 1) * d)
        assert np.array_equal(out2[:, sl], out[:, sl])
    assert not np.allclose(out2[:, d:2 * d], out[:, d:2 * d])


def test_row_subset_matches_full(orc):
    rng = np.random.default_rng(5)
    t, h, d = 77, 2, 64
    q, k, v = rand(rng, t, h, d)
    full = orc.flux_attention(q, k, v, h, d)
    rows = [76, 0, 31, 32, 5]
    sub = orc.flux_attention(q, k, v, h, d, rows=rows)
    assert np.array_equal(sub, full[rows])
