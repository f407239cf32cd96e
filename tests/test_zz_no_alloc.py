"""rt_hip_attention_decode_noalloc (no allocation: split partials in a
library-owned device array) against rt_hip_attention_decode, which takes
them from the library workspace.  Same kernels, so the outputs must be equal
bit for bit; checked on two calls in a row, the second smaller, so stale
partials of the first call would show.  Both are also checked against the
oracle's gqa_attention_cached restatement."""
import ctypes as C

import numpy as np
import pytest

from helpers import GEMV_TOL, from_dev, normwise_err, say, to_dev

pytestmark = pytest.mark.gpu


def _call(rt, name, q, kc, vc, out, nq, nkv, L, scale):
    import torch
    rt.library().call(name, q.data_ptr(), kc.data_ptr(), vc.data_ptr(), out.data_ptr(), nq, nkv, 128, L,
                      C.c_float(scale), torch.cuda.current_stream().cuda_stream)


def test_noalloc_attention_matches_workspace_attention(rt, orc):
    import torch
    d = 128
    scale = float(1.0 / np.sqrt(np.float32(d)))
    for i, (nq, nkv, L) in enumerate([(24, 8, 3000), (32, 8, 200)]):
        say(f"[noalloc attention] call {i}: n_q={nq} n_kv={nkv} L={L}")
        rng = np.random.default_rng(500 + i)
        kc = rng.standard_normal((L, nkv * d)).astype(np.float32)
        vc = rng.standard_normal((L, nkv * d)).astype(np.float32)
        q = (rng.standard_normal(nq * d) * 0.5).astype(np.float32)
        dq, dk, dv = to_dev(q), to_dev(kc), to_dev(vc)
        a = torch.full((nq * d,), float("nan"), device="cuda")
        b = torch.full((nq * d,), float("nan"), device="cuda")
        _call(rt, "rt_hip_attention_decode_noalloc", dq, dk, dv, a, nq, nkv, L, scale)
        _call(rt, "rt_hip_attention_decode", dq, dk, dv, b, nq, nkv, L, scale)
        torch.cuda.synchronize()
        ga, gb = from_dev(a), from_dev(b)
        assert np.array_equal(ga.view(np.uint32), gb.view(np.uint32))
        want = orc.gqa_attention_decode(q, kc, vc, L, nq, nkv, d, scale)
        assert normwise_err(ga, want) <= GEMV_TOL


def test_noalloc_attention_rejects_oversized_scratch(rt):
    import torch
    lib = rt.library()
    nkv = 1024
    q = torch.zeros(4 * nkv * 128, device="cuda")
    kc = torch.zeros(64 * nkv * 128, device="cuda")
    out = torch.zeros_like(q)
    rc = lib.status("rt_hip_attention_decode_noalloc", q.data_ptr(), kc.data_ptr(), kc.data_ptr(), out.data_ptr(),
                    4 * nkv, nkv, 128, 64, C.c_float(0.1), None)
    assert rc == 2
    assert b"scratch maximum" in lib.lib.rt_hip_last_error()
