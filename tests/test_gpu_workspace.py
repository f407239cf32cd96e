"""The library workspace under hipGraph capture (regression test).

A graph that captured decode attention (split partials in the workspace)
and the fused BF16 GEMV + argmax (its key in the workspace) keeps writing
the buffers those calls used on every replay.  A later eager GEMM that needs
more workspace replaces the buffer; the old one must stay valid (retired,
not freed), so replays after the growth still match the oracle.  Growth
during capture is refused with an error instead of allocating.
"""
import numpy as np
import pytest

from helpers import GEMV_TOL, from_dev, normwise_err, say, to_dev

pytestmark = pytest.mark.gpu


def test_graph_replays_survive_workspace_growth(rt, orc):
    import torch
    rng = np.random.default_rng(17)
    nq, nkv, d, L = 24, 8, 128, 1500
    kc = rng.standard_normal((L, nkv * d)).astype(np.float32)
    vc = rng.standard_normal((L, nkv * d)).astype(np.float32)
    q = (rng.standard_normal(nq * d) * 0.5).astype(np.float32)
    scale = float(1.0 / np.sqrt(np.float32(d)))
    n, k = 4096, 1152
    wb = orc.f32_to_bf16_n((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    x = rng.standard_normal((1, k)).astype(np.float32)
    want_attn = orc.gqa_attention_decode(q, kc, vc, L, nq, nkv, d, scale)
    want_y = orc.bf16_matmul_t(wb, x).reshape(-1)
    want_idx = orc.argmax_first(want_y)

    d_q, d_kc, d_vc = to_dev(q), to_dev(kc), to_dev(vc)
    d_w, d_x = to_dev(wb.view(np.int16)), to_dev(x)
    out = torch.empty((1, nq * d), device="cuda")
    y = torch.empty((1, n), device="cuda")
    lib = rt.library()
    need = lib.lib.rt_hip_attention_workspace_bytes(nq, nkv, L)
    assert need > 0
    rt.reserve_workspace(need)
    before = rt.workspace_bytes()
    idx = torch.empty(1, dtype=torch.int64, device="cuda")
    val = torch.empty(1, dtype=torch.float32, device="cuda")

    def body():
        rt.attention_decode(d_q, d_kc, d_vc, L, nq, nkv, scale, out=out)
        lib.call("rt_hip_gemv_bf16_argmax", d_w.data_ptr(), d_x.data_ptr(), y.data_ptr(), n, k, idx.data_ptr(),
                 val.data_ptr(), torch.cuda.current_stream().cuda_stream)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        body()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        body()

    def check(tag):
        out.zero_()
        y.zero_()
        idx.fill_(-1)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        e = normwise_err(from_dev(out).reshape(-1), want_attn)
        say(f"[workspace] {tag}: attention {e:.2e}, argmax {int(idx.item())} (want {want_idx})")
        assert e <= GEMV_TOL
        assert normwise_err(from_dev(y).reshape(-1), want_y) <= GEMV_TOL
        assert int(idx.item()) == want_idx

    check("replay 1")
    # an eager GEMM whose bf16 copies need more workspace than the device has
    # now (earlier tests in the process may have grown it): it grows
    gn, gk = 8192, 3072
    m = 512
    while lib.lib.rt_hip_gemm_workspace_bytes(rt.Q4K, rt.F32, m, gn, gk) <= before:
        m += 512
    gw = rng.standard_normal((gn, gk)).astype(np.float32) * 0.02
    blocks = rt.quantize_q4k(to_dev(gw))
    a = to_dev(rng.standard_normal((m, gk)).astype(np.float32))
    c = rt.gemm(rt.Q4K, a, blocks, gn, gk)
    torch.cuda.synchronize()
    assert rt.workspace_bytes() > before
    check("replay 2, after growth")
    del c
    check("replay 3")

    # growth inside a capture is refused with an error, and nothing breaks
    m2 = m
    while lib.lib.rt_hip_gemm_workspace_bytes(rt.Q4K, rt.F32, m2, gn, gk) <= rt.workspace_bytes():
        m2 += 512
    a2 = to_dev(rng.standard_normal((m2, gk)).astype(np.float32))
    c2 = torch.empty((m2, gn), device="cuda")
    g2 = torch.cuda.CUDAGraph()
    with pytest.raises(rt.RtHipError, match="before capture"):
        with torch.cuda.graph(g2):
            rt.gemm(rt.Q4K, a2, blocks, gn, gk, c=c2)
    torch.cuda.synchronize()
    check("replay 4, after a refused capture")
