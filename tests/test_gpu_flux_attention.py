"""GPU parity for FLUX's attention (rt_hip_flux_attention) against the
oracle's restatement of flux.cpp:287-321.

* Normwise 1e-5 (FLUX_ATTN_TOL) against the oracle on every output row for
  small and ragged shapes (t not a multiple of the 64-key tile or the
  128-query block, head_dim 8..128 including ones padded inside the kernel),
  plain and peaky scores; at the FLUX.1 shape (t = 4352 = 4096 image + 256
  text tokens, 24 heads of 128) on a sample of rows that covers both ends of
  every block boundary it crosses.
* Closed forms bit for bit: one key gives v; a key that dominates every
  other by more than 104 in score gives its v; and q = 0 gives the mean of v
  (to f32 rounding).
* Shapes with more 128-query blocks than workgroup slots (two per CU),
  where the blocks cut between two workgroups merge two partial states:
  every row against the oracle, a dominant key still gives exactly its v,
  and two runs agree bit for bit.
* Deterministic (two runs agree bit for bit); argument errors; the
  workspace query.
"""
import numpy as np
import pytest

from helpers import from_dev, normwise_err, say, to_dev

pytestmark = pytest.mark.gpu

# |out_gpu - out_ref|_max <= FLUX_ATTN_TOL * |out_ref|_max: f32 products and
# sums in a different order (matrix-core dot products, tiled online softmax);
# measured errors are around 1e-6.
FLUX_ATTN_TOL = 1e-5


def rand(rng, t, h, d, std=1.0):
    return [(rng.standard_normal((t, h * d)) * std).astype(np.float32) for _ in range(3)]


def run(rt, q, k, v, h, d):
    return from_dev(rt.flux_attention(to_dev(q), to_dev(k), to_dev(v), h, d))


@pytest.mark.parametrize("t,h,d,std", [(1, 1, 128, 1.0), (5, 3, 128, 1.0), (64, 2, 64, 1.0), (65, 2, 64, 1.0),
                                       (127, 4, 128, 1.0), (128, 24, 128, 1.0), (129, 2, 128, 2.0),
                                       (200, 2, 72, 1.0), (333, 3, 8, 1.0), (300, 5, 32, 1.0),
                                       (1000, 2, 16, 1.0), (700, 1, 96, 3.0), (517, 2, 128, 0.2)])
def test_flux_attention_vs_oracle(rt, orc, t, h, d, std):
    say(f"[flux attention] t={t} heads={h} head_dim={d} std={std}")
    rng = np.random.default_rng(t * 131 + h * 7 + d)
    q, k, v = rand(rng, t, h, d, std)
    got = run(rt, q, k, v, h, d)
    want = orc.flux_attention(q, k, v, h, d)
    err = normwise_err(got, want)
    say(f"[flux attention] normwise {err:.2e}")
    assert err <= FLUX_ATTN_TOL


@pytest.mark.parametrize("std", [1.0, 2.5])
def test_flux_attention_full_shape_rows(rt, orc, std):
    t, h, d = 4352, 24, 128
    say(f"[flux attention] FLUX.1 shape t={t} heads={h} head_dim={d} std={std}")
    rng = np.random.default_rng(int(std * 10))
    q, k, v = rand(rng, t, h, d, std)
    got = run(rt, q, k, v, h, d)
    rows = sorted(set([0, 1, 15, 16, 63, 64, 127, 128, 129, 2047, 2048, 4095, 4096, 4223, 4224, 4351]
                      + list(rng.integers(0, t, 16))))
    want = orc.flux_attention(q, k, v, h, d, rows=rows)
    err = normwise_err(got[rows], want)
    say(f"[flux attention] {len(rows)} rows, normwise {err:.2e}")
    assert err <= FLUX_ATTN_TOL
    assert np.all(np.isfinite(got))


def test_flux_attention_closed_forms(rt, orc):
    rng = np.random.default_rng(9)
    # one key: exactly v
    q, k, v = rand(rng, 1, 4, 128)
    got = run(rt, q, k, v, 4, 128)
    assert np.array_equal(got.view(np.uint32), v.view(np.uint32))
    # a key that dominates query row 5: exactly that key's v
    t, h, d = 200, 2, 64
    q, k, v = rand(rng, t, h, d, 0.05)
    star = 137
    k[star] = q[5] * np.float32(200.0 * np.sqrt(d) / np.mean(np.square(q[5])) / d)
    got = run(rt, q, k, v, h, d)
    assert np.array_equal(got[5].view(np.uint32), v[star].view(np.uint32))
    # q = 0: the mean of v
    t = 1000
    _, k, v = rand(rng, t, h, d)
    got = run(rt, np.zeros_like(k), k, v, h, d)
    want = np.broadcast_to(v.astype(np.float64).mean(axis=0), got.shape)
    assert np.max(np.abs(got - want)) <= 64 * 2.0 ** -24 * np.max(np.abs(v))


def test_flux_attention_deterministic(rt):
    rng = np.random.default_rng(11)
    q, k, v = rand(rng, 777, 3, 128)
    a = run(rt, q, k, v, 3, 128)
    b = run(rt, q, k, v, 3, 128)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_flux_attention_errors(rt):
    import torch
    lib = rt.library()
    x = torch.zeros((64, 2 * 128), device="cuda")
    o = torch.empty_like(x)
    p = lambda t, off=0: t.data_ptr() + off  # noqa: E731
    name = "rt_hip_flux_attention"
    assert lib.status(name, p(x), p(x), p(x), p(o), 64, 2, 12, None) == 2    # head_dim % 8
    assert lib.status(name, p(x), p(x), p(x), p(o), 64, 1, 136, None) == 2   # head_dim > 128
    assert lib.status(name, p(x), p(x), p(x), p(o), 64, 2, 128, None) == 0
    assert lib.status(name, p(x, 4), p(x), p(x), p(o), 32, 2, 128, None) == 3  # alignment
    assert lib.status(name, p(x), p(x), p(x), p(x), 64, 2, 128, None) == 1   # out overlaps q
    assert lib.status(name, None, p(x), p(x), p(o), 64, 2, 128, None) == 1   # null
    assert lib.status(name, p(x), p(x), p(x), p(o), 0, 2, 128, None) == 0    # t = 0: nothing
    torch.cuda.synchronize()


def slots():
    import torch
    return 2 * torch.cuda.get_device_properties(0).multi_processor_count


@pytest.mark.parametrize("t,h,d", [(512, 130, 8), (300, 260, 16)])
def test_flux_attention_split_blocks_every_row(rt, orc, t, h, d):
    assert h * ((t + 127) // 128) > slots()  # the split path
    say(f"[flux attention split] t={t} heads={h} head_dim={d}")
    rng = np.random.default_rng(t + h + d)
    q, k, v = rand(rng, t, h, d)
    got = run(rt, q, k, v, h, d)
    want = orc.flux_attention(q, k, v, h, d)
    err = normwise_err(got, want)
    say(f"[flux attention split] normwise {err:.2e}")
    assert err <= FLUX_ATTN_TOL
    # per head as well: a wrong merge of one block would hide in the whole
    for hh in range(0, h, 7):
        sl = slice(hh * d, (hh + 1) * d)
        assert normwise_err(got[:, sl], want[:, sl]) <= FLUX_ATTN_TOL, hh


def test_flux_attention_split_blocks_closed_form_and_determinism(rt, orc):
    t, h, d = 600, 120, 8
    assert h * ((t + 127) // 128) > slots()
    rng = np.random.default_rng(5)
    q, k, v = rand(rng, t, h, d, 0.05)
    # key 333 dominates query row 100 in every head by more than 104 in score
    for hh in range(h):
        sl = slice(hh * d, (hh + 1) * d)
        k[333, sl] = q[100, sl] * np.float32(200.0 * np.sqrt(d) / np.sum(np.square(q[100, sl])))
    a = run(rt, q, k, v, h, d)
    b = run(rt, q, k, v, h, d)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert np.array_equal(a[100].view(np.uint32), v[333].view(np.uint32))


def test_flux_attention_workspace_bytes(rt):
    lib = rt.library().lib
    f = lib.rt_hip_flux_attention_workspace_bytes
    assert f(4352, 24, 128) == slots() * 2 * (128 * 128 + 256) * 4
    assert f(1000, 2, 128) == 0
    assert f(512, 130, 8) == slots() * 2 * (128 * 32 + 256) * 4
    assert f(10, 1, 12) == -1
