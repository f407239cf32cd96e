"""GPU parity: layer operations fused into the decode GEMV's activation
staging (rt_hip_gemv_q4k_tiled_rmsnorm_multi / _swiglu).

Expected values: the oracle's RMSNorm / SwiGLU (tensor_node.cpp:320-402,
transformer5.cpp:186-190, pinned in test_oracle_layer_ops.py), then the
oracle's Q4_K product, normwise within the GEMV bar (1e-5); and the product's
own unfused path on the same normalized activation, to the same bar."""
import numpy as np
import pytest

from helpers import GEMV_TOL, from_dev, normwise_err, say, to_dev

pytestmark = pytest.mark.gpu
E_ARG, E_SHAPE = 1, 2


def _weights(orc, rng, ns, k):
    return [orc.q4k_quantize((rng.standard_normal((n, k)) * 0.02).astype(np.float32)) for n in ns]


@pytest.mark.parametrize("ns,k,gemma3,note", [
    ([3072, 1024, 1024], 3072, False, "llama q/k/v"),
    ([8192, 8192], 3072, False, "llama gate/up"),
    ([1152, 256, 256], 1152 // 256 * 256, True, "gemma3 form"),
    ([40], 512, False, "short output"),
])
def test_rmsnorm_fused_gemv(rt, orc, ns, k, gemma3, note):
    say(f"[rmsnorm gemv] ns={ns} K={k} gemma3={gemma3} ({note})")
    rng = np.random.default_rng(sum(ns) + k)
    blocks = _weights(orc, rng, ns, k)
    x = (rng.standard_normal(k) * 3).astype(np.float32)
    gamma = (rng.standard_normal(k) * (0.1 if gemma3 else 1.0)).astype(np.float32)
    eps = 1e-6 if gemma3 else 1e-5
    tiled = [rt.q4k_tile(to_dev(b), n, k) for b, n in zip(blocks, ns)]
    ys = rt.gemv_q4k_tiled_rmsnorm_multi(tiled, to_dev(x), to_dev(gamma), eps, ns, k, gemma3=gemma3)
    xn = orc.rmsnorm(x, gamma, eps, gemma3=gemma3).reshape(1, k)
    unfused = rt.gemv_q4k_tiled_multi(tiled, to_dev(xn), ns, k)
    for b, n, y, u in zip(blocks, ns, ys, unfused):
        want = orc.q4k_matmul_t(b, n, k, xn)
        got = from_dev(y)
        assert normwise_err(got, want) <= GEMV_TOL, normwise_err(got, want)
        assert normwise_err(got, from_dev(u)) <= GEMV_TOL


def test_rmsnorm_zero_activation_gives_zero(rt, orc):
    k, n = 1024, 64
    rng = np.random.default_rng(9)
    (b,) = _weights(orc, rng, [n], k)
    t = rt.q4k_tile(to_dev(b), n, k)
    (y,) = rt.gemv_q4k_tiled_rmsnorm_multi([t], to_dev(np.zeros(k, np.float32)),
                                           to_dev(np.ones(k, np.float32)), 1e-5, [n], k)
    assert not np.any(from_dev(y))


@pytest.mark.parametrize("n,k,note", [(3072, 8192, "llama down"), (2560, 10240, "gemma-3-4b down shape, K split 10"),
                                      (100, 512, "ragged N"), (16, 256, "one block")])
def test_swiglu_fused_gemv(rt, orc, n, k, note):
    say(f"[swiglu gemv] N={n} K={k} ({note})")
    rng = np.random.default_rng(n + 3 * k)
    (b,) = _weights(orc, rng, [n], k)
    gate = (rng.standard_normal(k) * 2).astype(np.float32)
    up = rng.standard_normal(k).astype(np.float32)
    t = rt.q4k_tile(to_dev(b), n, k)
    got = from_dev(rt.gemv_q4k_tiled_swiglu(t, to_dev(gate), to_dev(up), n, k))
    act = orc.swiglu(gate, up).reshape(1, k)
    want = orc.q4k_matmul_t(b, n, k, act)
    assert normwise_err(got, want) <= GEMV_TOL, normwise_err(got, want)
    unfused = from_dev(rt.gemv_q4k_tiled(t, to_dev(act), n, k))
    assert normwise_err(got, unfused) <= GEMV_TOL


def test_layer_ops_reject_bad_arguments(rt):
    import ctypes as C
    lib = rt.library()
    t = to_dev(np.zeros(2304, np.uint8))
    x = to_dev(np.zeros(65536, np.float32))
    y = to_dev(np.zeros(16, np.float32))
    wp = (C.c_void_p * 1)(t.data_ptr())
    yp = (C.c_void_p * 1)(y.data_ptr())
    npp = (C.c_int64 * 1)(16)
    assert lib.status("rt_hip_gemv_q4k_tiled_rmsnorm_multi", 1, wp, yp, npp, x.data_ptr(), None,
                      C.c_float(1e-5), 0, 256, None) == E_ARG
    assert lib.status("rt_hip_gemv_q4k_tiled_rmsnorm_multi", 1, wp, yp, npp, x.data_ptr(), x.data_ptr(),
                      C.c_float(-1.0), 0, 256, None) == E_ARG
    # K whose staged limbs (3.5 bytes per value) exceed one workgroup's LDS:
    # refused before any launch
    assert lib.status("rt_hip_gemv_q4k_tiled_swiglu", t.data_ptr(), x.data_ptr(), x.data_ptr(), y.data_ptr(),
                      16, 65536, None) == E_SHAPE
    assert lib.status("rt_hip_gemv_q4k_tiled_swiglu", t.data_ptr(), x.data_ptr(), None, y.data_ptr(),
                      16, 256, None) == E_ARG


def test_rmsnorm_fused_qk_plus_bf16_v(rt, orc):
    """A widened layer's q/k (Q4_K) and BF16 v on RMSNorm(x), one launch."""
    k, ns, nb = 3072, [3072, 1024], 1024
    say(f"[rmsnorm q/k + bf16 v] K={k}")
    rng = np.random.default_rng(21)
    blocks = _weights(orc, rng, ns, k)
    wv = orc.f32_to_bf16_n((rng.standard_normal((nb, k)) * 0.02).astype(np.float32))
    x = (rng.standard_normal(k) * 2).astype(np.float32)
    gamma = (1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    tiled = [rt.q4k_tile(to_dev(b), n, k) for b, n in zip(blocks, ns)]
    ys, yb = rt.gemv_q4k_tiled_bf16_rmsnorm(tiled, ns, to_dev(wv.view(np.int16)), nb, to_dev(x), to_dev(gamma),
                                            1e-5, k)
    xn = orc.rmsnorm(x, gamma, 1e-5).reshape(1, k)
    for b, n, y in zip(blocks, ns, ys):
        assert normwise_err(from_dev(y), orc.q4k_matmul_t(b, n, k, xn)) <= GEMV_TOL
    assert normwise_err(from_dev(yb), orc.bf16_matmul_t(wv, xn)) <= GEMV_TOL


@pytest.mark.parametrize("pos,half", [(0, False), (7, False), (1000, True), (70000, True)])
def test_rmsnorm_rope_qk_plus_bf16_v_into_kv_cache(rt, orc, pos, half):
    """The q/k/v launch of a widened (Q4_K_M) layer: Q4_K q and k rotated at
    `pos` (interleaved, or half-split with rows interleaved at tiling), the
    BF16 v beside them, k and v written into their KV-cache rows."""
    import torch
    k, hd, nq, nkv = 3072, 128, 24, 8
    ns, nb = [nq * hd, nkv * hd], nkv * hd
    say(f"[rmsnorm+rope q/k + bf16 v] pos={pos} half={half}")
    rng = np.random.default_rng(pos + 41)
    blocks = _weights(orc, rng, ns, k)
    wv = orc.f32_to_bf16_n((rng.standard_normal((nb, k)) * 0.02).astype(np.float32))
    x = (rng.standard_normal(k) * 2).astype(np.float32)
    gamma = (1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    inv = orc.llama_inv_freq(500000.0, hd)
    tiled = [rt.q4k_tile(to_dev(b), n, k, rope_half_head_dim=hd if half else 0) for b, n in zip(blocks, ns)]
    max_tok = 4
    row = pos % max_tok
    kc = torch.zeros((max_tok, nkv * hd), device="cuda")
    vc = torch.zeros((max_tok, nkv * hd), device="cuda")
    q = torch.empty((1, ns[0]), device="cuda")
    jobs = 0x3 | (rt.ROPE_HALF if half else 0)
    rt.gemv_q4k_tiled_bf16_rmsnorm(tiled, ns, to_dev(wv.view(np.int16)), nb, to_dev(x), to_dev(gamma), 1e-5, k,
                                   ys=[q, kc[row:row + 1]], yb=vc[row:row + 1], rope=(to_dev(inv), pos, hd, jobs))
    xn = orc.rmsnorm(x, gamma, 1e-5).reshape(1, k)
    lin = [orc.q4k_matmul_t(b, n, k, xn).reshape(-1) for b, n in zip(blocks, ns)]
    assert normwise_err(from_dev(q).reshape(-1), orc.llama_rope(lin[0], nq, hd, pos, inv, half=half)) <= GEMV_TOL
    assert normwise_err(from_dev(kc)[row], orc.llama_rope(lin[1], nkv, hd, pos, inv, half=half)) <= GEMV_TOL
    assert normwise_err(from_dev(vc)[row], orc.bf16_matmul_t(wv, xn).reshape(-1)) <= GEMV_TOL
    others = [r for r in range(max_tok) if r != row]
    assert not np.any(from_dev(kc)[others]) and not np.any(from_dev(vc)[others])


@pytest.mark.parametrize("n,k", [(3072, 8192), (100, 512)])
def test_bf16_swiglu(rt, orc, n, k):
    say(f"[bf16 swiglu] N={n} K={k}")
    rng = np.random.default_rng(n + k + 5)
    w = orc.f32_to_bf16_n((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    gate = (rng.standard_normal(k) * 2).astype(np.float32)
    up = rng.standard_normal(k).astype(np.float32)
    got = from_dev(rt.gemv_bf16_swiglu(to_dev(w.view(np.int16)), to_dev(gate), to_dev(up), n, k))
    act = orc.swiglu(gate, up).reshape(1, k)
    assert normwise_err(got, orc.bf16_matmul_t(w, act)) <= GEMV_TOL


# (n_q, n_kv, head_dim): Llama-3.2-3B; 640 tiles, which the launch runs at
# one wave per tile (KS = 1: the partner row comes from the lane swap of the
# same wave, no K-split reduction); head_dim 64.
ROPE_SHAPES = [(24, 8, 128), (48, 16, 128), (48, 16, 64)]


@pytest.mark.parametrize("pos", [0, 5, 1000, 70000])
@pytest.mark.parametrize("nq,nkv,hd", ROPE_SHAPES)
def test_rmsnorm_rope_qkv_into_kv_cache(rt, orc, pos, nq, nkv, hd):
    """q/k/v of a Llama layer on RMSNorm(x), q and k rotated at `pos`
    (interleaved pairing), k and v written straight into their KV-cache rows."""
    import torch
    k = 3072
    ns = [nq * hd, nkv * hd, nkv * hd]
    say(f"[rmsnorm+rope qkv] pos={pos} n_q={nq} n_kv={nkv} head_dim={hd}")
    rng = np.random.default_rng(pos + 1)
    blocks = _weights(orc, rng, ns, k)
    x = (rng.standard_normal(k) * 2).astype(np.float32)
    gamma = (1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    inv = orc.llama_inv_freq(500000.0, hd)
    tiled = [rt.q4k_tile(to_dev(b), n, k) for b, n in zip(blocks, ns)]
    max_tok = 8
    row = min(pos, max_tok - 1)
    kc = torch.zeros((max_tok, nkv * hd), device="cuda")
    vc = torch.zeros((max_tok, nkv * hd), device="cuda")
    q = torch.empty((1, ns[0]), device="cuda")
    rt.gemv_q4k_tiled_rmsnorm_rope(tiled, to_dev(x), to_dev(gamma), 1e-5, ns, k, to_dev(inv), pos, hd, 0x3,
                                   ys=[q, kc[row:row + 1], vc[row:row + 1]])
    xn = orc.rmsnorm(x, gamma, 1e-5).reshape(1, k)
    lin = [orc.q4k_matmul_t(b, n, k, xn).reshape(-1) for b, n in zip(blocks, ns)]
    want_q = orc.llama_rope(lin[0], nq, hd, pos, inv)
    want_k = orc.llama_rope(lin[1], nkv, hd, pos, inv)
    assert normwise_err(from_dev(q).reshape(-1), want_q) <= GEMV_TOL
    assert normwise_err(from_dev(kc)[row], want_k) <= GEMV_TOL
    assert normwise_err(from_dev(vc)[row], lin[2]) <= GEMV_TOL
    others = [r for r in range(max_tok) if r != row]
    assert not np.any(from_dev(kc)[others]) and not np.any(from_dev(vc)[others])


@pytest.mark.parametrize("pos", [0, 3, 1000, 70000])
@pytest.mark.parametrize("nq,nkv,hd", ROPE_SHAPES)
def test_rmsnorm_rope_half_split_qkv(rt, orc, pos, nq, nkv, hd):
    """The half-split pairing (HuggingFace weights): q and k tiled with their
    head rows interleaved (rt_hip_q4k_tile_rope_half), v tiled plainly, one
    launch with rope_jobs 0x3 | ROPE_HALF; outputs back in their places."""
    import torch
    k = 3072
    ns = [nq * hd, nkv * hd, nkv * hd]
    say(f"[rmsnorm+rope half qkv] pos={pos} n_q={nq} n_kv={nkv} head_dim={hd}")
    rng = np.random.default_rng(pos + 11)
    blocks = _weights(orc, rng, ns, k)
    x = (rng.standard_normal(k) * 2).astype(np.float32)
    gamma = (1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    inv = orc.llama_inv_freq(500000.0, hd)
    tiled = [rt.q4k_tile(to_dev(b), n, k, rope_half_head_dim=(hd if i < 2 else 0))
             for i, (b, n) in enumerate(zip(blocks, ns))]
    ys = [torch.full((1, n), float("nan"), device="cuda") for n in ns]
    rt.gemv_q4k_tiled_rmsnorm_rope(tiled, to_dev(x), to_dev(gamma), 1e-5, ns, k, to_dev(inv), pos, hd,
                                   0x3 | rt.ROPE_HALF, ys=ys)
    xn = orc.rmsnorm(x, gamma, 1e-5).reshape(1, k)
    lin = [orc.q4k_matmul_t(b, n, k, xn).reshape(-1) for b, n in zip(blocks, ns)]
    got = [from_dev(y).reshape(-1) for y in ys]
    assert all(np.all(np.isfinite(g)) for g in got)  # every element stored
    assert normwise_err(got[0], orc.llama_rope(lin[0], nq, hd, pos, inv, half=True)) <= GEMV_TOL
    assert normwise_err(got[1], orc.llama_rope(lin[1], nkv, hd, pos, inv, half=True)) <= GEMV_TOL
    assert normwise_err(got[2], lin[2]) <= GEMV_TOL
    lib = rt.library()
    b0 = to_dev(blocks[1])
    out = torch.empty(rt.q4k_tiled_bytes(ns[1], k), dtype=torch.uint8, device="cuda")
    assert lib.status("rt_hip_q4k_tile_rope_half", b0.data_ptr(), out.data_ptr(), ns[1], k, 127, None) == 1
    assert lib.status("rt_hip_q4k_tile_rope_half", b0.data_ptr(), out.data_ptr(), 1000, k, 128, None) == E_SHAPE


@pytest.mark.parametrize("nq,nkv,seq_len", [(24, 8, 1), (24, 8, 7), (24, 8, 300), (24, 8, 4096), (32, 8, 1000),
                                            (8, 8, 129), (16, 8, 50)])
def test_attention_decode(rt, orc, nq, nkv, seq_len):
    """rt_hip_attention_decode against the oracle's gqa_attention_cached
    (decode path), positions [0, seq_len) of a longer cache."""
    say(f"[attention decode] n_q={nq} n_kv={nkv} L={seq_len}")
    d = 128
    rng = np.random.default_rng(nq * 7 + seq_len)
    cap = seq_len + 5
    kc = rng.standard_normal((cap, nkv * d)).astype(np.float32)
    vc = rng.standard_normal((cap, nkv * d)).astype(np.float32)
    q = (rng.standard_normal(nq * d) * 0.5).astype(np.float32)
    scale = float(1.0 / np.sqrt(np.float32(d)))
    got = from_dev(rt.attention_decode(to_dev(q), to_dev(kc), to_dev(vc), seq_len, nq, nkv, scale)).reshape(-1)
    want = orc.gqa_attention_decode(q, kc, vc, seq_len, nq, nkv, d, scale)
    assert normwise_err(got, want) <= GEMV_TOL, normwise_err(got, want)
    if seq_len == 1:  # one position: the value row itself, to rounding
        g = nq // nkv
        for h in range(nq):
            assert np.allclose(got[h * d:(h + 1) * d], vc[0, (h // g) * d:(h // g + 1) * d], rtol=1e-6, atol=1e-6)


def test_attention_decode_is_deterministic_and_rejects_bad_shapes(rt):
    import ctypes as C
    rng = np.random.default_rng(3)
    kc = to_dev(rng.standard_normal((2048, 1024)).astype(np.float32))
    vc = to_dev(rng.standard_normal((2048, 1024)).astype(np.float32))
    q = to_dev(rng.standard_normal(3072).astype(np.float32))
    a = from_dev(rt.attention_decode(q, kc, vc, 2048, 24, 8, 0.088))
    b = from_dev(rt.attention_decode(q, kc, vc, 2048, 24, 8, 0.088))
    assert np.array_equal(a, b)
    lib = rt.library()
    p = q.data_ptr()
    assert lib.status("rt_hip_attention_decode", p, kc.data_ptr(), vc.data_ptr(), p, 24, 8, 64, 10,
                      C.c_float(0.1), None) == 6  # head_dim 64: unsupported
    assert lib.status("rt_hip_attention_decode", p, kc.data_ptr(), vc.data_ptr(), p, 24, 7, 128, 10,
                      C.c_float(0.1), None) == E_SHAPE
    assert lib.status("rt_hip_attention_decode", p, kc.data_ptr(), vc.data_ptr(), p, 24, 8, 128, 0,
                      C.c_float(0.1), None) == E_SHAPE


def test_attention_decode_back_to_back_shapes(rt, orc):
    """Calls in a row whose split counts and KV-head counts differ (1 KV head
    and 79 splits, past the one-batch merge; 64 KV heads; 1 split): every
    call matches the oracle."""
    d = 128
    scale = float(1.0 / np.sqrt(np.float32(d)))
    for i, (nq, nkv, seq_len) in enumerate([(4, 1, 5000), (24, 8, 300), (64, 64, 700), (24, 8, 4096),
                                            (4, 1, 5000), (3, 1, 64)]):
        say(f"[attention back-to-back] call {i}: n_q={nq} n_kv={nkv} L={seq_len}")
        rng = np.random.default_rng(100 + i)
        kc = rng.standard_normal((seq_len, nkv * d)).astype(np.float32)
        vc = rng.standard_normal((seq_len, nkv * d)).astype(np.float32)
        q = (rng.standard_normal(nq * d) * 0.5).astype(np.float32)
        got = from_dev(rt.attention_decode(to_dev(q), to_dev(kc), to_dev(vc), seq_len, nq, nkv, scale)).reshape(-1)
        want = orc.gqa_attention_decode(q, kc, vc, seq_len, nq, nkv, d, scale)
        assert normwise_err(got, want) <= GEMV_TOL, (i, normwise_err(got, want))


def test_residual_adds(rt, orc):
    """resid += W . x and resid += W . (silu(gate) * up), Q4_K and BF16."""
    rng = np.random.default_rng(31)
    k, n = 3072, 3072
    (b,) = _weights(orc, rng, [n], k)
    t = rt.q4k_tile(to_dev(b), n, k)
    x = rng.standard_normal(k).astype(np.float32)
    r0 = rng.standard_normal(n).astype(np.float32)
    resid = to_dev(r0)
    rt.gemv_q4k_tiled_residual(t, to_dev(x), resid, n, k)
    want = r0 + orc.q4k_matmul_t(b, n, k, x.reshape(1, k)).reshape(-1)
    assert normwise_err(from_dev(resid), want) <= GEMV_TOL
    kf = 8192
    (bd,) = _weights(orc, rng, [n], kf)
    td = rt.q4k_tile(to_dev(bd), n, kf)
    gate = (rng.standard_normal(kf) * 2).astype(np.float32)
    up = rng.standard_normal(kf).astype(np.float32)
    act = orc.swiglu(gate, up).reshape(1, kf)
    resid = to_dev(r0)
    rt.gemv_swiglu_residual(rt.Q4K, td, to_dev(gate), to_dev(up), resid, n, kf)
    assert normwise_err(from_dev(resid), r0 + orc.q4k_matmul_t(bd, n, kf, act).reshape(-1)) <= GEMV_TOL
    wb = orc.f32_to_bf16_n((rng.standard_normal((n, kf)) * 0.02).astype(np.float32))
    resid = to_dev(r0)
    rt.gemv_swiglu_residual(rt.BF16, to_dev(wb.view(np.int16)), to_dev(gate), to_dev(up), resid, n, kf)
    assert normwise_err(from_dev(resid), r0 + orc.bf16_matmul_t(wb, act).reshape(-1)) <= GEMV_TOL
    # an aliased residual is refused
    lib = rt.library()
    xd = to_dev(x)
    assert lib.status("rt_hip_gemv_q4k_tiled_residual", t.data_ptr(), xd.data_ptr(), xd.data_ptr(), n, k,
                      None) == E_ARG
