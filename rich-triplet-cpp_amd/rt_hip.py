"""ctypes binding of the C ABI in include/rt_hip.h (lib/librt_hip.so).

torch is only the device-memory and stream plumbing here: every call passes
``tensor.data_ptr()`` and the current HIP stream to the native library, which
runs the gfx950 kernels.  There is no fallback: if the library is missing or
a call fails, an exception is raised.
"""
from __future__ import annotations

import ctypes as C
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
# RT_HIP_LIB_PATH selects another build of the same ABI (the host-sanitizer
# build that tests/test_sanitizers.py runs the host-code tests against).
LIB_PATH = os.environ.get("RT_HIP_LIB_PATH", os.path.join(HERE, "lib", "librt_hip.so"))
HEADER_PATH = os.path.join(ROOT, "include", "rt_hip.h")

F32, BF16, Q4K, Q4_0, Q4MAT, Q6K = 0, 1, 2, 3, 4, 5
GEMV_MAX_M = 8

_vp, _i64, _i32 = C.c_void_p, C.c_int64, C.c_int32

# name -> argtypes (restype is int unless noted)
_SIGNATURES = {
    "rt_hip_init": [C.c_int],
    "rt_hip_gemv_q4k": [_vp, _vp, _vp, _i64, _i64, _i32, _vp],
    "rt_hip_gemv_bf16": [_vp, _vp, _vp, _i64, _i64, _i32, _vp],
    "rt_hip_gemv_q4k_multi": [_i32, C.POINTER(_vp), C.POINTER(_vp), C.POINTER(_i64), _vp, _i64, _vp],
    "rt_hip_q4k_tile": [_vp, _vp, _i64, _i64, _vp],
    "rt_hip_q4k_tile_rope_half": [_vp, _vp, _i64, _i64, _i32, _vp],
    "rt_hip_gemv_q4k_tiled": [_vp, _vp, _vp, _i64, _i64, _vp],
    "rt_hip_gemv_q4k_tiled_multi": [_i32, C.POINTER(_vp), C.POINTER(_vp), C.POINTER(_i64), _vp, _i64, _vp],
    "rt_hip_q4k_quantize_activation_q8": [_vp, _i64, _vp, _vp, _vp, _vp],
    "rt_hip_gemv_q4k_q8": [_vp, _vp, _vp, _i64, _i64, _vp],
    "rt_hip_gemv_q4k_tiled_q8": [_vp, _vp, _vp, _i64, _i64, _vp],
    "rt_hip_gemv_q4_0": [_vp, _vp, _vp, _i64, _i64, _i32, _vp],
    "rt_hip_argmax": [_vp, _i64, _i64, _vp, _vp, _vp],
    "rt_hip_gemv_bf16_argmax": [_vp, _vp, _vp, _i64, _i64, _vp, _vp, _vp],
    "rt_hip_dequant_q4k_f32": [_vp, _vp, _i64, _i64, _vp],
    "rt_hip_dequant_q4k_bf16": [_vp, _vp, _i64, _i64, _vp],
    "rt_hip_quantize_q4k": [_vp, _vp, _i64, _i64, _vp],
    "rt_hip_gemm_q4k": [_vp, _i32, _vp, _vp, _vp, _i64, _i64, _i64, _vp],
    "rt_hip_gemm_bf16": [_vp, _i32, _vp, _vp, _vp, _i64, _i64, _i64, _vp],
    "rt_hip_linear_forward": [_i32, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp],
    "rt_hip_probe_read": [_vp, _i64, _i32, _vp, _i64, _vp],
    "rt_hip_probe_empty": [_i32, _i32, _vp],
    "rt_hip_gemv_q4k_tiled_bf16": [_i32, C.POINTER(_vp), C.POINTER(_vp), C.POINTER(_i64), _vp, _vp, _i64,
                                   _vp, _i64, _vp],
    "rt_hip_gemv_q4k_tiled_rmsnorm_multi": [_i32, C.POINTER(_vp), C.POINTER(_vp), C.POINTER(_i64), _vp, _vp,
                                            C.c_float, _i32, _i64, _vp],
    "rt_hip_gemv_q4k_tiled_swiglu": [_vp, _vp, _vp, _vp, _i64, _i64, _vp],
    "rt_hip_attention_decode": [_vp, _vp, _vp, _vp, _i32, _i32, _i32, _i64, C.c_float, _vp],
    "rt_hip_attention_decode_noalloc": [_vp, _vp, _vp, _vp, _i32, _i32, _i32, _i64, C.c_float, _vp],
    "rt_hip_flux_attention": [_vp, _vp, _vp, _vp, _i64, _i32, _i32, _vp],
    "rt_hip_gemv_q4k_tiled_residual": [_vp, _vp, _vp, _i64, _i64, _vp],
    "rt_hip_gemv_q4k_tiled_swiglu_residual": [_vp, _vp, _vp, _vp, _i64, _i64, _vp],
    "rt_hip_gemv_bf16_swiglu_residual": [_vp, _vp, _vp, _vp, _i64, _i64, _vp],
    "rt_hip_gemv_q6k_tiled_swiglu_residual": [_vp, _vp, _vp, _vp, _i64, _i64, _vp],
    "rt_hip_gemv_q4k_tiled_rmsnorm_rope": [_i32, C.POINTER(_vp), C.POINTER(_vp), C.POINTER(_i64), _vp, _vp,
                                           C.c_float, _i32, _vp, _i32, _i32, _i32, _i64, _vp],
    "rt_hip_gemv_q4k_tiled_bf16_rmsnorm": [_i32, C.POINTER(_vp), C.POINTER(_vp), C.POINTER(_i64), _vp, _vp, _i64,
                                           _vp, _vp, C.c_float, _i32, _i64, _vp],
    "rt_hip_gemv_q4k_tiled_bf16_rmsnorm_rope": [_i32, C.POINTER(_vp), C.POINTER(_vp), C.POINTER(_i64), _vp, _vp,
                                                _i64, _vp, _vp, C.c_float, _i32, _vp, _i32, _i32, _i32, _i64, _vp],
    "rt_hip_gemv_bf16_swiglu": [_vp, _vp, _vp, _vp, _i64, _i64, _vp],
    "rt_hip_dequant_q6k_bf16": [_vp, _vp, _i64, _i64, _vp],
    "rt_hip_q6k_tile": [_vp, _vp, _i64, _i64, _vp],
    "rt_hip_gemv_q6k_tiled": [_vp, _vp, _vp, _i64, _i64, _vp],
    "rt_hip_reserve_workspace": [_i64],
    "rt_hip_gemv_q4mat": [_vp, _vp, _vp, _i64, _i64, _i32, _vp],
    "rt_hip_gemm": [_i32, _vp, _i32, _vp, _vp, _vp, _i64, _i64, _i64, _vp],
    "rt_hip_dequant": [_i32, _vp, _vp, _i32, _i64, _i64, _vp],
}

# name -> argtypes of the int64-returning size queries
_SIZE_SIGNATURES = {
    "rt_hip_q4k_tiled_bytes": [_i64, _i64],
    "rt_hip_q6k_tiled_bytes": [_i64, _i64],
    "rt_hip_workspace_bytes": [],
    "rt_hip_gemm_workspace_bytes": [_i32, _i32, _i64, _i64, _i64],
    "rt_hip_gemv_workspace_bytes": [_i32, _i64, _i64, _i32],
    "rt_hip_attention_workspace_bytes": [_i32, _i32, _i64],
    "rt_hip_flux_attention_workspace_bytes": [_i64, _i32, _i32],
    "rt_hip_q4mat_bytes": [_i64, _i64],
    "rt_hip_q4mat_scales_offset": [_i64, _i64],
}


class GgufTensor(C.Structure):
    """rt_hip_gguf_tensor (include/rt_hip.h)."""
    _fields_ = [("name", C.c_char_p), ("type", _i32), ("n_dims", _i32), ("dims", _i64 * 4), ("n_elements", _i64),
                ("bytes", _i64), ("file_offset", _i64)]


_GGUF_SIGNATURES = [
    ("rt_hip_gguf_type_bytes", _i64, [_i32, _i64]),
    ("rt_hip_gguf_open", C.c_int, [C.c_char_p, C.POINTER(_vp)]),
    ("rt_hip_gguf_close", None, [_vp]),
    ("rt_hip_gguf_tensor_count", _i64, [_vp]),
    ("rt_hip_gguf_find_tensor", _i64, [_vp, C.c_char_p]),
    ("rt_hip_gguf_tensor_info", C.c_int, [_vp, _i64, C.POINTER(GgufTensor)]),
    ("rt_hip_gguf_linear_shape", C.c_int, [_vp, _i64, C.POINTER(_i64), C.POINTER(_i64)]),
    ("rt_hip_gguf_read_tensor", C.c_int, [_vp, _i64, _vp, _i64]),
    ("rt_hip_gguf_upload", C.c_int, [_vp, _i64, _vp, _i64, _vp]),
    ("rt_hip_gguf_meta_u64", C.c_int, [_vp, C.c_char_p, _i64, C.POINTER(C.c_uint64)]),
    ("rt_hip_gguf_meta_f32", C.c_int, [_vp, C.c_char_p, _i64, C.POINTER(C.c_float)]),
    ("rt_hip_gguf_meta_str", C.c_int, [_vp, C.c_char_p, _i64, C.POINTER(C.c_char_p)]),
    ("rt_hip_gguf_meta_array_len", _i64, [_vp, C.c_char_p]),
]


class RtHipError(RuntimeError):
    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed with status {code}: {msg}")
        self.code = code


def header_functions(path: str = HEADER_PATH) -> list[str]:
    """Names of the functions include/rt_hip.h declares."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(rt_hip_\w+)\s*\(", text)))


class Library:
    """The loaded native library (no compute happens at load time)."""

    def __init__(self, path: str = LIB_PATH):
        if not os.path.exists(path):
            raise FileNotFoundError(
                f"{path} is missing: build it with `make -C rich-triplet-cpp_amd` "
                "(or __graft_entry__.build())")
        self.path = path
        self.lib = C.CDLL(path)
        self.lib.rt_hip_last_error.restype = C.c_char_p
        self.lib.rt_hip_version.restype = C.c_char_p
        for name, args in _SIZE_SIGNATURES.items():
            fn = getattr(self.lib, name)
            fn.restype = C.c_int64
            fn.argtypes = args
        for name, res, args in _GGUF_SIGNATURES:
            fn = getattr(self.lib, name)
            fn.restype = res
            fn.argtypes = args
        for name, args in _SIGNATURES.items():
            fn = getattr(self.lib, name)
            fn.restype = C.c_int
            fn.argtypes = args

    def version(self) -> str:
        return self.lib.rt_hip_version().decode()

    def call(self, name: str, *args) -> None:
        rc = getattr(self.lib, name)(*args)
        if rc != 0:
            raise RtHipError(name, rc, self.lib.rt_hip_last_error().decode())

    def status(self, name: str, *args) -> int:
        """Call and return the status code without raising (for error tests)."""
        return getattr(self.lib, name)(*args)


_LIB: Library | None = None


def library() -> Library:
    global _LIB
    if _LIB is None:
        _LIB = Library()
    return _LIB


# ---------------------------------------------------------------- torch API --

def _torch():
    import torch  # noqa: PLC0415  (plumbing only)
    return torch


def _ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(stream=None) -> int:
    torch = _torch()
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


def init(ordinal: int = 0) -> None:
    library().call("rt_hip_init", ordinal)


def reserve_workspace(nbytes: int) -> None:
    """Pre-size the current device's library workspace (before graph capture)."""
    library().call("rt_hip_reserve_workspace", int(nbytes))


def workspace_bytes() -> int:
    return int(library().lib.rt_hip_workspace_bytes())


def _dev_check(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("rt_hip: tensors must live on the GPU")
        if t is not None and not t.is_contiguous():
            raise ValueError("rt_hip: tensors must be contiguous")


def gemv(fmt: int, w, x, n: int, k: int, y=None, stream=None):
    """y[M, N] = x[M, K] @ W^T for M <= 8; W in `fmt` bytes on the device."""
    torch = _torch()
    x = x.reshape(-1, k)
    m = x.shape[0]
    if y is None:
        y = torch.empty((m, n), dtype=torch.float32, device=x.device)
    _dev_check(w, x, y)
    name = {Q4K: "rt_hip_gemv_q4k", BF16: "rt_hip_gemv_bf16", Q4_0: "rt_hip_gemv_q4_0",
            Q4MAT: "rt_hip_gemv_q4mat"}[fmt]
    library().call(name, _ptr(w), _ptr(x), _ptr(y), n, k, m, _stream(stream))
    return y


def gemv_q4k_multi(ws, x, ns, k: int, ys=None, stream=None):
    """y[j] = x @ W[j]^T for up to 4 Q4_K weights sharing x (one launch)."""
    torch = _torch()
    count = len(ws)
    if ys is None:
        ys = [torch.empty((1, n), dtype=torch.float32, device=x.device) for n in ns]
    _dev_check(x, *ws, *ys)
    wp = (_vp * count)(*[w.data_ptr() for w in ws])
    yp = (_vp * count)(*[y.data_ptr() for y in ys])
    npp = (_i64 * count)(*ns)
    library().call("rt_hip_gemv_q4k_multi", count, wp, yp, npp, _ptr(x), k, _stream(stream))
    return ys


def q4k_tiled_bytes(n: int, k: int) -> int:
    return library().lib.rt_hip_q4k_tiled_bytes(n, k)


# rope_jobs flag of gemv_q4k_tiled_rmsnorm_rope: the half-split RoPE pairing.
ROPE_HALF = 0x100


def q4k_tile(blocks, n: int, k: int, stream=None, rope_half_head_dim: int = 0):
    """Tiled copy of row-major Q4_K blocks (for gemv_q4k_tiled*).  With
    rope_half_head_dim, each head's rows are interleaved for a q / k
    projection rotated in the half-split pairing (rope_jobs | ROPE_HALF)."""
    torch = _torch()
    size = q4k_tiled_bytes(n, k)
    if size < 0:
        raise ValueError(f"rt_hip: invalid Q4_K shape n={n} k={k}")
    tiled = torch.empty(size, dtype=torch.uint8, device=blocks.device)
    _dev_check(blocks)
    if rope_half_head_dim:
        library().call("rt_hip_q4k_tile_rope_half", _ptr(blocks), _ptr(tiled), n, k, rope_half_head_dim,
                       _stream(stream))
    else:
        library().call("rt_hip_q4k_tile", _ptr(blocks), _ptr(tiled), n, k, _stream(stream))
    return tiled


def gemv_q4k_tiled(tiled, x, n: int, k: int, y=None, stream=None):
    torch = _torch()
    if y is None:
        y = torch.empty((1, n), dtype=torch.float32, device=x.device)
    _dev_check(tiled, x, y)
    library().call("rt_hip_gemv_q4k_tiled", _ptr(tiled), _ptr(x), _ptr(y), n, k, _stream(stream))
    return y


def quantize_activation_q8(a, stream=None):
    """Q4KMat::quantize_activation_q8 (quant_q4k.cpp:525-562): (q8, scales, sums)."""
    torch = _torch()
    k = a.numel()
    nq = (k + 31) // 32
    q8 = torch.empty(nq * 32, dtype=torch.int8, device=a.device)
    sc = torch.empty(nq, dtype=torch.float32, device=a.device)
    su = torch.empty(nq, dtype=torch.float32, device=a.device)
    _dev_check(a)
    library().call("rt_hip_q4k_quantize_activation_q8", _ptr(a), k, _ptr(q8), _ptr(sc), _ptr(su), _stream(stream))
    return q8, sc, su


def gemv_q4k_q8(w, x, n: int, k: int, tiled: bool = False, y=None, stream=None):
    """gemv_mt's aarch64 branch (quant_q4k.cpp:564-600): Q8 activation, dot_row_q8 per row."""
    torch = _torch()
    if y is None:
        y = torch.empty((1, n), dtype=torch.float32, device=x.device)
    _dev_check(w, x, y)
    library().call("rt_hip_gemv_q4k_tiled_q8" if tiled else "rt_hip_gemv_q4k_q8", _ptr(w), _ptr(x), _ptr(y), n, k,
                   _stream(stream))
    return y


def gemv_q4k_tiled_multi(ws, x, ns, k: int, ys=None, stream=None):
    torch = _torch()
    count = len(ws)
    if ys is None:
        ys = [torch.empty((1, n), dtype=torch.float32, device=x.device) for n in ns]
    _dev_check(x, *ws, *ys)
    wp = (_vp * count)(*[w.data_ptr() for w in ws])
    yp = (_vp * count)(*[y.data_ptr() for y in ys])
    npp = (_i64 * count)(*ns)
    library().call("rt_hip_gemv_q4k_tiled_multi", count, wp, yp, npp, _ptr(x), k, _stream(stream))
    return ys


def gemv_q4k_tiled_bf16(ws, ns, wb, nb: int, x, k: int, ys=None, yb=None, stream=None):
    """Tiled-Q4_K GEMVs ws (out_features ns) and one BF16 GEMV wb [nb, k], all
    on x, in one launch (a layer's q/k and BF16-widened v)."""
    torch = _torch()
    count = len(ws)
    if ys is None:
        ys = [torch.empty((1, n), dtype=torch.float32, device=x.device) for n in ns]
    if yb is None:
        yb = torch.empty((1, nb), dtype=torch.float32, device=x.device)
    _dev_check(x, wb, yb, *ws, *ys)
    wp = (_vp * count)(*[w.data_ptr() for w in ws])
    yp = (_vp * count)(*[y.data_ptr() for y in ys])
    npp = (_i64 * count)(*ns)
    library().call("rt_hip_gemv_q4k_tiled_bf16", count, wp, yp, npp, _ptr(wb), _ptr(yb), nb, _ptr(x), k,
                   _stream(stream))
    return ys, yb


def gemv_q4k_tiled_rmsnorm_multi(ws, x, gamma, eps: float, ns, k: int, gemma3: bool = False, ys=None,
                                 stream=None):
    """y_j = W_j . RMSNorm(x) (gamma, or 1 + gamma for gemma3) for tiled Q4_K
    weights sharing x, the norm applied while x is staged."""
    torch = _torch()
    count = len(ws)
    if ys is None:
        ys = [torch.empty((1, n), dtype=torch.float32, device=x.device) for n in ns]
    _dev_check(x, gamma, *ws, *ys)
    wp = (_vp * count)(*[w.data_ptr() for w in ws])
    yp = (_vp * count)(*[y.data_ptr() for y in ys])
    npp = (_i64 * count)(*ns)
    library().call("rt_hip_gemv_q4k_tiled_rmsnorm_multi", count, wp, yp, npp, _ptr(x), _ptr(gamma),
                   C.c_float(eps), 1 if gemma3 else 0, k, _stream(stream))
    return ys


def gemv_q4k_tiled_rmsnorm_rope(ws, x, gamma, eps: float, ns, k: int, inv_freq, pos: int, head_dim: int,
                                rope_jobs: int, gemma3: bool = False, ys=None, stream=None):
    """gemv_q4k_tiled_rmsnorm_multi, then interleaved RoPE at `pos` on the
    outputs of the jobs in the bit mask rope_jobs (| ROPE_HALF: half-split
    pairing, weights tiled with rope_half_head_dim); ys may point into a KV
    cache (the append)."""
    torch = _torch()
    count = len(ws)
    if ys is None:
        ys = [torch.empty((1, n), dtype=torch.float32, device=x.device) for n in ns]
    _dev_check(x, gamma, inv_freq, *ws, *ys)
    wp = (_vp * count)(*[w.data_ptr() for w in ws])
    yp = (_vp * count)(*[y.data_ptr() for y in ys])
    npp = (_i64 * count)(*ns)
    library().call("rt_hip_gemv_q4k_tiled_rmsnorm_rope", count, wp, yp, npp, _ptr(x), _ptr(gamma), C.c_float(eps),
                   1 if gemma3 else 0, _ptr(inv_freq), pos, head_dim, rope_jobs, k, _stream(stream))
    return ys


def gemv_q4k_tiled_residual(w, x, resid, n: int, k: int, stream=None):
    """resid += W . x (tiled Q4_K)."""
    _dev_check(w, x, resid)
    library().call("rt_hip_gemv_q4k_tiled_residual", _ptr(w), _ptr(x), _ptr(resid), n, k, _stream(stream))
    return resid


def gemv_swiglu_residual(fmt: int, w, gate, up, resid, n: int, k: int, stream=None, q6k: bool = False):
    """resid += W . (silu(gate) * up), W tiled Q4_K (fmt Q4K), BF16 bits, or
    a tiled Q6_K copy (q6k=True)."""
    _dev_check(w, gate, up, resid)
    name = ("rt_hip_gemv_q6k_tiled_swiglu_residual" if q6k else
            "rt_hip_gemv_q4k_tiled_swiglu_residual" if fmt == Q4K else "rt_hip_gemv_bf16_swiglu_residual")
    library().call(name, _ptr(w), _ptr(gate), _ptr(up), _ptr(resid), n, k, _stream(stream))
    return resid


def attention_decode(q, k_cache, v_cache, seq_len: int, n_q: int, n_kv: int, scale: float, head_dim: int = 128,
                     out=None, stream=None):
    """One query token's GQA attention over KV-cache positions [0, seq_len)."""
    torch = _torch()
    if out is None:
        out = torch.empty((1, n_q * head_dim), dtype=torch.float32, device=q.device)
    _dev_check(q, k_cache, v_cache, out)
    library().call("rt_hip_attention_decode", _ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(out), n_q, n_kv, head_dim,
                   seq_len, C.c_float(scale), _stream(stream))
    return out


def flux_attention(q, k, v, n_heads: int, head_dim: int, out=None, stream=None):
    """FLUX's unmasked multi-head attention (flux.cpp:287-321) over
    [t, n_heads * head_dim] f32 q, k, v."""
    torch = _torch()
    t = q.shape[0]
    if out is None:
        out = torch.empty((t, n_heads * head_dim), dtype=torch.float32, device=q.device)
    _dev_check(q, k, v, out)
    library().call("rt_hip_flux_attention", _ptr(q), _ptr(k), _ptr(v), _ptr(out), t, n_heads, head_dim,
                   _stream(stream))
    return out


def gemv_q4k_tiled_swiglu(w, gate, up, n: int, k: int, y=None, stream=None):
    """y = W . (silu(gate) * up) for a tiled Q4_K weight (the down projection)."""
    torch = _torch()
    if y is None:
        y = torch.empty((1, n), dtype=torch.float32, device=gate.device)
    _dev_check(w, gate, up, y)
    library().call("rt_hip_gemv_q4k_tiled_swiglu", _ptr(w), _ptr(gate), _ptr(up), _ptr(y), n, k, _stream(stream))
    return y


def gemv_q4k_tiled_bf16_rmsnorm(ws, ns, wb, nb: int, x, gamma, eps: float, k: int, gemma3: bool = False,
                                ys=None, yb=None, stream=None, rope=None):
    """gemv_q4k_tiled_bf16 on RMSNorm(x) (gamma, or 1 + gamma for gemma3).
    rope = (inv_freq, pos, head_dim, rope_jobs) also rotates the Q4_K jobs in
    rope_jobs (| ROPE_HALF: half-split pairing)."""
    torch = _torch()
    count = len(ws)
    if ys is None:
        ys = [torch.empty((1, n), dtype=torch.float32, device=x.device) for n in ns]
    if yb is None:
        yb = torch.empty((1, nb), dtype=torch.float32, device=x.device)
    _dev_check(x, gamma, wb, yb, *ws, *ys)
    wp = (_vp * count)(*[w.data_ptr() for w in ws])
    yp = (_vp * count)(*[y.data_ptr() for y in ys])
    npp = (_i64 * count)(*ns)
    if rope is not None:
        inv_freq, pos, head_dim, rope_jobs = rope
        _dev_check(inv_freq)
        library().call("rt_hip_gemv_q4k_tiled_bf16_rmsnorm_rope", count, wp, yp, npp, _ptr(wb), _ptr(yb), nb,
                       _ptr(x), _ptr(gamma), C.c_float(eps), 1 if gemma3 else 0, _ptr(inv_freq), pos, head_dim,
                       rope_jobs, k, _stream(stream))
        return ys, yb
    library().call("rt_hip_gemv_q4k_tiled_bf16_rmsnorm", count, wp, yp, npp, _ptr(wb), _ptr(yb), nb, _ptr(x),
                   _ptr(gamma), C.c_float(eps), 1 if gemma3 else 0, k, _stream(stream))
    return ys, yb


def gemv_bf16_swiglu(w, gate, up, n: int, k: int, y=None, stream=None):
    """y = W . (silu(gate) * up) for a BF16 weight [n, k] (int16 bits)."""
    torch = _torch()
    if y is None:
        y = torch.empty((1, n), dtype=torch.float32, device=gate.device)
    _dev_check(w, gate, up, y)
    library().call("rt_hip_gemv_bf16_swiglu", _ptr(w), _ptr(gate), _ptr(up), _ptr(y), n, k, _stream(stream))
    return y


def dequant_q6k_bf16(blocks, n: int, k: int, stream=None):
    """GGUF Q6_K blocks -> bf16 [n, k] (as int16 bits), the reference's widening."""
    torch = _torch()
    out = torch.empty((n, k), dtype=torch.int16, device=blocks.device)
    _dev_check(blocks, out)
    library().call("rt_hip_dequant_q6k_bf16", _ptr(blocks), _ptr(out), n, k, _stream(stream))
    return out


def q6k_tiled_bytes(n: int, k: int) -> int:
    return library().lib.rt_hip_q6k_tiled_bytes(n, k)


def q6k_tile(blocks, n: int, k: int, stream=None):
    torch = _torch()
    out = torch.empty(q6k_tiled_bytes(n, k), dtype=torch.uint8, device=blocks.device)
    _dev_check(blocks, out)
    library().call("rt_hip_q6k_tile", _ptr(blocks), _ptr(out), n, k, _stream(stream))
    return out


def gemv_q6k_tiled(tiled, x, n: int, k: int, y=None, stream=None):
    torch = _torch()
    if y is None:
        y = torch.empty((1, n), dtype=torch.float32, device=x.device)
    _dev_check(tiled, x, y)
    library().call("rt_hip_gemv_q6k_tiled", _ptr(tiled), _ptr(x), _ptr(y), n, k, _stream(stream))
    return y


class GgufFile:
    """A GGUF file opened through rt_hip_gguf_* (the reference's GgufFile)."""

    def __init__(self, path: str):
        self._lib = library()
        h = _vp()
        self._lib.call("rt_hip_gguf_open", os.fsencode(path), C.byref(h))
        self.h = h

    def close(self) -> None:
        if self.h:
            self._lib.lib.rt_hip_gguf_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __len__(self) -> int:
        return self._lib.lib.rt_hip_gguf_tensor_count(self.h)

    def find(self, name: str) -> int:
        return self._lib.lib.rt_hip_gguf_find_tensor(self.h, name.encode())

    def info(self, idx: int) -> dict:
        t = GgufTensor()
        self._lib.call("rt_hip_gguf_tensor_info", self.h, idx, C.byref(t))
        return {"name": t.name.decode(), "type": t.type, "dims": [t.dims[d] for d in range(t.n_dims)],
                "n_elements": t.n_elements, "bytes": t.bytes, "file_offset": t.file_offset}

    def linear_shape(self, idx: int):
        r, c = _i64(), _i64()
        self._lib.call("rt_hip_gguf_linear_shape", self.h, idx, C.byref(r), C.byref(c))
        return r.value, c.value

    def read(self, idx: int):
        import numpy as np
        out = np.empty(self.info(idx)["bytes"], np.uint8)
        self._lib.call("rt_hip_gguf_read_tensor", self.h, idx, out.ctypes.data, out.size)
        return out

    def upload(self, idx: int, device=None, stream=None):
        torch = _torch()
        out = torch.empty(self.info(idx)["bytes"], dtype=torch.uint8, device=device or "cuda")
        self._lib.call("rt_hip_gguf_upload", self.h, idx, _ptr(out), out.numel(), _stream(stream))
        return out

    def meta_u64(self, key: str, index: int = -1) -> int:
        v = C.c_uint64()
        self._lib.call("rt_hip_gguf_meta_u64", self.h, key.encode(), index, C.byref(v))
        return v.value

    def meta_f32(self, key: str, index: int = -1) -> float:
        v = C.c_float()
        self._lib.call("rt_hip_gguf_meta_f32", self.h, key.encode(), index, C.byref(v))
        return v.value

    def meta_str(self, key: str, index: int = -1) -> str:
        v = C.c_char_p()
        self._lib.call("rt_hip_gguf_meta_str", self.h, key.encode(), index, C.byref(v))
        return v.value.decode()

    def meta_array_len(self, key: str) -> int:
        return self._lib.lib.rt_hip_gguf_meta_array_len(self.h, key.encode())


def gemv_bf16_argmax(w, x, n: int, k: int, y=None, stream=None):
    torch = _torch()
    if y is None:
        y = torch.empty((1, n), dtype=torch.float32, device=x.device)
    idx = torch.empty(1, dtype=torch.int64, device=x.device)
    val = torch.empty(1, dtype=torch.float32, device=x.device)
    _dev_check(w, x, y)
    library().call("rt_hip_gemv_bf16_argmax", _ptr(w), _ptr(x), _ptr(y), n, k, _ptr(idx),
                   _ptr(val), _stream(stream))
    return y, idx, val


def argmax(logits, stream=None):
    torch = _torch()
    rows, cols = logits.shape
    idx = torch.empty(rows, dtype=torch.int64, device=logits.device)
    val = torch.empty(rows, dtype=torch.float32, device=logits.device)
    _dev_check(logits)
    library().call("rt_hip_argmax", _ptr(logits), rows, cols, _ptr(idx), _ptr(val),
                   _stream(stream))
    return idx, val


def dequant_q4k(blocks, n: int, k: int, bf16: bool = False, stream=None):
    torch = _torch()
    out = torch.empty((n, k), dtype=torch.int16 if bf16 else torch.float32, device=blocks.device)
    _dev_check(blocks)
    name = "rt_hip_dequant_q4k_bf16" if bf16 else "rt_hip_dequant_q4k_f32"
    library().call(name, _ptr(blocks), _ptr(out), n, k, _stream(stream))
    return out


def quantize_q4k(w, stream=None):
    torch = _torch()
    n, k = w.shape
    blocks = torch.empty(n * (k // 256) * 144, dtype=torch.uint8, device=w.device)
    _dev_check(w)
    library().call("rt_hip_quantize_q4k", _ptr(w), _ptr(blocks), n, k, _stream(stream))
    return blocks


def gemm(fmt: int, a, w, n: int, k: int, bias=None, c=None, stream=None):
    """C[M, N] = A[M, K] @ W^T (+ bias); A f32 or bf16 (torch.bfloat16)."""
    torch = _torch()
    m = a.shape[0]
    if c is None:
        c = torch.empty((m, n), dtype=torch.float32, device=a.device)
    a_dtype = BF16 if a.dtype == torch.bfloat16 else F32
    _dev_check(a, w, c, bias)
    library().call("rt_hip_gemm", fmt, _ptr(a), a_dtype, _ptr(w), _ptr(bias), _ptr(c), m, n, k, _stream(stream))
    return c


def q4mat_bytes(n: int, k: int) -> int:
    v = int(library().lib.rt_hip_q4mat_bytes(n, k))
    if v < 0:
        raise ValueError("q4mat: need n > 0, k % 32 == 0")
    return v


def q4mat_upload(packed, scales, n: int, k: int):
    """The RT_HIP_Q4MAT buffer (uint8 device tensor) from a Q4Mat's host
    `packed` bytes and f32 `scales` (numpy arrays)."""
    import numpy as np  # noqa: PLC0415
    torch = _torch()
    off = int(library().lib.rt_hip_q4mat_scales_offset(n, k))
    buf = np.zeros(q4mat_bytes(n, k), np.uint8)
    buf[:packed.size] = np.asarray(packed, np.uint8).reshape(-1)
    buf[off:off + 4 * scales.size] = np.ascontiguousarray(scales, np.float32).view(np.uint8).reshape(-1)
    return torch.from_numpy(buf).cuda()


def dequant(fmt: int, w, n: int, k: int, bf16: bool = False, stream=None):
    """Weight bytes -> [n, k] f32 (or bf16 bits as int16)."""
    torch = _torch()
    out = torch.empty((n, k), dtype=torch.int16 if bf16 else torch.float32, device=w.device)
    _dev_check(w, out)
    library().call("rt_hip_dequant", fmt, _ptr(w), _ptr(out), BF16 if bf16 else F32, n, k, _stream(stream))
    return out


def linear_forward(fmt: int, w, x, n: int, k: int, bias=None, y=None, stream=None):
    torch = _torch()
    m = x.shape[0]
    if y is None:
        y = torch.empty((m, n), dtype=torch.float32, device=x.device)
    _dev_check(w, x, y, bias)
    library().call("rt_hip_linear_forward", fmt, _ptr(w), _ptr(bias), _ptr(x), _ptr(y), m, n, k,
                   _stream(stream))
    return y


def probe_read(buf, nbytes: int, workgroups: int, out, out_bytes: int = 0, stream=None) -> None:
    """rt_hip_probe_read: a plain streaming read of nbytes of buf, then
    out_bytes of out written (calibration)."""
    library().call("rt_hip_probe_read", _ptr(buf), nbytes, workgroups, _ptr(out), out_bytes, _stream(stream))


def probe_empty(workgroups: int = 1, threads: int = 64, stream=None) -> None:
    """rt_hip_probe_empty: an empty kernel launch (calibration)."""
    library().call("rt_hip_probe_empty", workgroups, threads, _stream(stream))


# ---------------------------------------------------------------- decoder --

ARCH_LLAMA, ARCH_GEMMA3 = 0, 1
(T_EMBED, T_OUTPUT_NORM, T_LM_HEAD, T_ATTN_NORM, T_Q, T_K, T_V, T_O, T_Q_NORM, T_K_NORM, T_POST_ATTN_NORM,
 T_FFN_NORM, T_GATE, T_UP, T_DOWN, T_POST_FFN_NORM) = range(16)


class DecoderConfig(C.Structure):
    """rt_hip_decoder_config (include/rt_hip.h)."""
    _fields_ = [("arch", _i32), ("n_layers", _i32), ("hidden", _i32), ("n_heads", _i32), ("n_kv_heads", _i32),
                ("head_dim", _i32), ("ffn", _i32), ("vocab", _i32), ("max_seq", _i32), ("norm_eps", C.c_float),
                ("rope_theta", C.c_float), ("rope_theta_local", C.c_float), ("rope_freq_scale", C.c_float),
                ("rope_freq_scale_local", C.c_float), ("rope_half", _i32), ("sliding_window", _i32),
                ("global_every", _i32), ("attn_scale", C.c_float), ("embed_scale", C.c_float), ("kv_f16", _i32),
                ("max_batch", _i32), ("llama_inv_freq", C.POINTER(C.c_float))]


class Decoder:
    """The decode engine (rt_hip_decoder_*): weights from host numpy arrays,
    steps return host logits."""

    def __init__(self, **cfg):
        import numpy as np  # noqa: PLC0415
        lib = library()
        L = lib.lib
        for name, res, args in [
            ("rt_hip_decoder_create", C.c_int, [C.POINTER(DecoderConfig), C.POINTER(_vp)]),
            ("rt_hip_decoder_set_tensor", C.c_int, [_vp, _i32, _i32, _i32, _vp, _i64]),
            ("rt_hip_decoder_set_kv", C.c_int, [_vp, _i32, _vp, _vp, _i64]),
            ("rt_hip_decoder_step", C.c_int, [_vp, _i32, _i32, _vp, _vp, _vp]),
            ("rt_hip_decoder_step_batch", C.c_int, [_vp, _vp, _i32, _i32, _vp, _vp]),
            ("rt_hip_decoder_vocab", _i64, [_vp]),
            ("rt_hip_decoder_destroy", C.c_int, [_vp])]:
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        inv = cfg.pop("llama_inv_freq", None)
        c = DecoderConfig(**cfg)
        self._inv = None
        if inv is not None:
            self._inv = np.ascontiguousarray(inv, np.float32)
            c.llama_inv_freq = self._inv.ctypes.data_as(C.POINTER(C.c_float))
        self.cfg = cfg
        h = _vp()
        lib.call("rt_hip_decoder_create", C.byref(c), C.byref(h))
        self.h = h

    def set(self, layer: int, tensor: int, fmt: int, arr) -> None:
        import numpy as np  # noqa: PLC0415
        a = np.ascontiguousarray(arr)
        library().call("rt_hip_decoder_set_tensor", self.h, layer, tensor, fmt, a.ctypes.data, a.nbytes)

    def set_kv(self, layer: int, k, v, rows: int) -> None:
        import numpy as np  # noqa: PLC0415
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        library().call("rt_hip_decoder_set_kv", self.h, layer, k.ctypes.data, v.ctypes.data, rows)

    @property
    def vocab(self) -> int:
        return int(library().lib.rt_hip_decoder_vocab(self.h))

    def step(self, token: int, pos: int, argmax: bool = False, stream=None):
        import numpy as np  # noqa: PLC0415
        out = np.empty(self.vocab, np.float32)
        idx = np.zeros(1, np.int64)
        library().call("rt_hip_decoder_step", self.h, token, pos, out.ctypes.data,
                       idx.ctypes.data if argmax else None, None if stream is None else _stream(stream))
        return (out, int(idx[0])) if argmax else out

    def step_batch(self, tokens, start_pos: int, stream=None):
        import numpy as np  # noqa: PLC0415
        t = np.ascontiguousarray(tokens, np.int32)
        out = np.empty((t.size, self.vocab), np.float32)
        library().call("rt_hip_decoder_step_batch", self.h, t.ctypes.data, t.size, start_pos, out.ctypes.data,
                       None if stream is None else _stream(stream))
        return out

    def close(self) -> None:
        if getattr(self, "h", None):
            library().call("rt_hip_decoder_destroy", self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # noqa: BLE001  (interpreter shutdown)
            pass

