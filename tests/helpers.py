"""Helpers shared by the GPU parity tests (inputs, uploads, tolerances)."""
import sys

import numpy as np

# Normwise tolerance for f32-accumulated GEMV outputs (the BASELINE bar):
#   max_i |y_gpu - y_ref| <= GEMV_TOL * max_i |y_ref|
GEMV_TOL = 1e-5
# bf16-MFMA GEMM, against the f32 product of the same bf16-rounded operands.
GEMM_TOL_SAME_OPERANDS = 1e-5
# bf16-MFMA GEMM against the reference's f32 CPU output (operand rounding):
# relative RMS error.  RNE to bf16 leaves a relative error of RMS
# 2^-9/sqrt(3) = 1.1e-3 per operand, about 1.6e-3 for a product of two
# rounded operands; measured 1.65e-3 (bf16 A) to 2.33e-3 (f32 A, prefill) at
# the full config-4/5 shapes.  The bar is 4e-3.
GEMM_TOL_VS_F32_RMS = 4e-3


def say(*a):
    """Progress line naming the case, flushed before the GPU step runs."""
    print(*a, file=sys.stderr, flush=True)


def normwise_err(y, ref) -> float:
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(y - ref)) / max(np.max(np.abs(ref)), 1e-30))


def rel_rms(y, ref) -> float:
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.sqrt(np.mean((y - ref) ** 2)) / max(np.sqrt(np.mean(ref ** 2)), 1e-30))


def same_operand_err(c, a, wd, n_cols=64, seed=0):
    """Normwise error of a bf16-MFMA GEMM output c [M, N] (device) against
    the float64 product of the same bf16-rounded operands on n_cols sampled
    output columns: a [M, K] (device f32 or bf16; rounded to bf16 RNE as the
    GEMM rounds it) and wd [N, K] (device bf16 or f32 holding bf16 values).
    float64 makes the reference's own rounding negligible, so the bar is the
    stated GEMM_TOL_SAME_OPERANDS."""
    import torch
    n = wd.shape[0]
    cols = np.sort(np.random.default_rng(seed).choice(n, min(n_cols, n), replace=False))
    idx = torch.from_numpy(cols).to(wd.device)
    ah = a.bfloat16().float().cpu().numpy().astype(np.float64)
    wh = wd.index_select(0, idx).float().cpu().numpy().astype(np.float64)
    ref = ah @ wh.T
    got = c.index_select(1, idx).cpu().numpy().astype(np.float64)
    return float(np.max(np.abs(got - ref)) / max(np.max(np.abs(ref)), 1e-30))


def to_dev(arr):
    import torch
    return torch.from_numpy(np.ascontiguousarray(arr)).cuda()


def from_dev(t):
    return t.detach().cpu().numpy()


def bf16_bits_to_f32(bits):
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_rne(x):
    """numpy RNE f32 -> bf16 bits (NaN not expected in test data)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return r.astype(np.uint16)


# ---- tiled Q4_K layout (the GEMV's load order; include/rt_hip.h) ----------
# Per 16-row tile t and super-block b, 2304 bytes in lane order l = n + 16 g:
#   [0, 256)     u32 per lane: sv(2g) | sv(2g+1) << 6 | mv(2g) << 12 |
#                mv(2g+1) << 18 | byte g of (d | dmin << 16) << 24
#   [256, 1280)  qs[32g, 32g+16) of row n;  [1280, 2304) qs[32g+16, 32g+32)
# Rows past N are zero.  A numpy restatement used to check the device tiling.

def _scale_min_all(sc):
    """sc[..., 12] uint32 -> sv, mv [..., 8] (Q4KMat::scale_min rules)."""
    sv = np.empty(sc.shape[:-1] + (8,), np.uint32)
    mv = np.empty_like(sv)
    for j in range(4):
        sv[..., j] = sc[..., j] & 63
        mv[..., j] = sc[..., j + 4] & 63
    for j in range(4, 8):
        sv[..., j] = (sc[..., j + 4] & 15) | ((sc[..., j - 4] >> 6) << 4)
        mv[..., j] = (sc[..., j + 4] >> 4) | ((sc[..., j] >> 6) << 4)
    return sv, mv


def q4k_tile_np(blocks, n, k):
    nb = k // 256
    t = (n + 15) // 16
    src = np.zeros((t * 16, nb, 144), np.uint8)
    src[:n] = np.frombuffer(np.ascontiguousarray(blocks), np.uint8).reshape(n, nb, 144)
    src = src.reshape(t, 16, nb, 144).transpose(0, 2, 1, 3)   # [t, b, row, 144]
    dd = np.ascontiguousarray(src[..., 0:4]).view("<u4")[..., 0].astype(np.uint32)
    sv, mv = _scale_min_all(src[..., 4:16].astype(np.uint32))
    hdr = np.empty((t, nb, 4, 16), np.uint32)                  # [g][row]
    for g in range(4):
        hdr[:, :, g, :] = (sv[..., 2 * g] | (sv[..., 2 * g + 1] << 6) | (mv[..., 2 * g] << 12)
                           | (mv[..., 2 * g + 1] << 18) | (((dd >> (8 * g)) & 0xFF) << 24))
    qs = src[..., 16:144].reshape(t, nb, 16, 4, 32).transpose(0, 1, 3, 2, 4)  # [t,b,g,row,32]
    out = np.empty((t, nb, 2304), np.uint8)
    out[..., 0:256] = hdr.reshape(t, nb, 64).astype("<u4").view(np.uint8).reshape(t, nb, 256)
    out[..., 256:1280] = qs[..., :16].reshape(t, nb, 1024)
    out[..., 1280:2304] = qs[..., 16:].reshape(t, nb, 1024)
    return out.reshape(-1)


def q4k_untile_np(tiled, n, k):
    """Inverse of q4k_tile_np (the 12 scale bytes are a bijection of the
    eight 6-bit (sv, mv) pairs, so any bytes round-trip)."""
    nb = k // 256
    t = (n + 15) // 16
    src = np.frombuffer(np.ascontiguousarray(tiled), np.uint8).reshape(t, nb, 2304)
    hdr = np.ascontiguousarray(src[..., 0:256]).view("<u4").reshape(t, nb, 4, 16).astype(np.uint32)
    sv = np.empty((t, nb, 16, 8), np.uint32)
    mv = np.empty_like(sv)
    dd = np.zeros((t, nb, 16), np.uint32)
    for g in range(4):
        h = hdr[:, :, g, :]
        sv[..., 2 * g] = h & 63
        sv[..., 2 * g + 1] = (h >> 6) & 63
        mv[..., 2 * g] = (h >> 12) & 63
        mv[..., 2 * g + 1] = (h >> 18) & 63
        dd |= ((h >> 24) & 0xFF) << (8 * g)
    sc = np.empty((t, nb, 16, 12), np.uint32)
    for j in range(4):
        sc[..., j] = sv[..., j] | ((sv[..., j + 4] >> 4) << 6)
        sc[..., j + 4] = mv[..., j] | ((mv[..., j + 4] >> 4) << 6)
        sc[..., j + 8] = (sv[..., j + 4] & 15) | ((mv[..., j + 4] & 15) << 4)
    out = np.empty((t, nb, 16, 144), np.uint8)
    out[..., 0:4] = dd.astype("<u4").view(np.uint8).reshape(t, nb, 16, 4)
    out[..., 4:16] = sc.astype(np.uint8)
    qa = src[..., 256:1280].reshape(t, nb, 4, 16, 16)
    qb = src[..., 1280:2304].reshape(t, nb, 4, 16, 16)
    qs = np.concatenate([qa, qb], axis=-1).transpose(0, 1, 3, 2, 4)  # [t, b, row, g, 32]
    out[..., 16:144] = qs.reshape(t, nb, 16, 128)
    return out.transpose(0, 2, 1, 3).reshape(t * 16, nb, 144)[:n].reshape(-1)


def q4k_dequant_tiled_np(tiled, n, k):
    """w = (d*sv)*q - (dmin*mv) in f32 straight from the tiled bytes."""
    nb = k // 256
    t = (n + 15) // 16
    src = np.frombuffer(np.ascontiguousarray(tiled), np.uint8).reshape(t, nb, 2304)
    hdr = np.ascontiguousarray(src[..., 0:256]).view("<u4").reshape(t, nb, 4, 16).astype(np.uint32)
    dd = np.zeros((t, nb, 16), np.uint32)
    for g in range(4):
        dd |= ((hdr[:, :, g, :] >> 24) & 0xFF) << (8 * g)
    d = (dd & 0xFFFF).astype(np.uint16).view(np.float16).astype(np.float32)
    dm = (dd >> 16).astype(np.uint16).view(np.float16).astype(np.float32)
    qa = src[..., 256:1280].reshape(t, nb, 4, 16, 16)
    qb = src[..., 1280:2304].reshape(t, nb, 4, 16, 16)
    qs = np.concatenate([qa, qb], axis=-1).transpose(0, 1, 3, 2, 4)   # [t, b, row, g, 32]
    w = np.empty((t, nb, 16, 4, 64), np.float32)
    for g in range(4):
        h = hdr[:, :, g, :]
        for half, shift in ((0, 0), (1, 4)):
            sv = ((h >> (6 * half)) & 63).astype(np.float32)
            mv = ((h >> (12 + 6 * half)) & 63).astype(np.float32)
            q = ((qs[:, :, :, g, :] >> shift) & 15).astype(np.float32)
            a = (d * sv).astype(np.float32)[..., None]
            m = (dm * mv).astype(np.float32)[..., None]
            w[:, :, :, g, 32 * half:32 * half + 32] = (a * q).astype(np.float32) - m
    w = w.reshape(t, nb, 16, 256).transpose(0, 2, 1, 3).reshape(t * 16, k)
    return w[:n]
