"""Helpers shared by the GPU parity tests (inputs, uploads, tolerances)."""
import sys

import numpy as np

# Normwise tolerance for f32-accumulated GEMV outputs (the BASELINE bar):
#   max_i |y_gpu - y_ref| <= GEMV_TOL * max_i |y_ref|
GEMV_TOL = 1e-5
# bf16-MFMA GEMM, against the f32 product of the same bf16-rounded operands.
GEMM_TOL_SAME_OPERANDS = 1e-5
# bf16-MFMA GEMM against the reference's f32 CPU output (operand rounding):
# relative RMS error.
GEMM_TOL_VS_F32_RMS = 1e-2


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
