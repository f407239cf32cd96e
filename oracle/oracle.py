"""numpy bindings for the CPU checker (test infrastructure, never the product).

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg
import this module.  It loads:

* ``oracle/liboracle.so`` -- the plain-C restatement in ``rt_oracle.c``;
* ``oracle/_ref/libref_oracle.so`` -- the reference's own sources compiled in
  place (``oracle/Makefile``), when it was built.

Each wrapper names the reference function it stands for; see rt_oracle.h for
what pins it.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libref_oracle.so")

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_sz = C.c_size_t


def _bind(lib, name, res, *args):
    fn = getattr(lib, name)
    fn.restype = res
    fn.argtypes = list(args)
    return fn


class Oracle:
    """The C restatement (rt_oracle.c)."""

    def __init__(self, path: str = LIB_PATH):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing: run `make -C oracle` (or __graft_entry__.build())")
        L = self.lib = C.CDLL(path)
        self._f16_to_f32 = _bind(L, "orc_f16_to_f32", C.c_float, C.c_uint16)
        self._f32_to_f16 = _bind(L, "orc_f32_to_f16", C.c_uint16, C.c_float)
        self._bf16_to_f32 = _bind(L, "orc_bf16_to_f32", C.c_float, C.c_uint16)
        self._f32_to_bf16 = _bind(L, "orc_f32_to_bf16", C.c_uint16, C.c_float)
        self._f32_to_bf16_n = _bind(L, "orc_f32_to_bf16_n", None, _f32p, _u16p, _sz)
        self._scale_min = _bind(L, "orc_q4k_scale_min", None, _u8p, _sz,
                                C.POINTER(C.c_float), C.POINTER(C.c_float))
        self._pack = _bind(L, "orc_q4k_pack_scales", None, _u8p, _u8p, _u8p)
        self._qblock = _bind(L, "orc_q4k_quantize_block", None, _f32p, _u8p)
        self._q4k_quant = _bind(L, "orc_q4k_quantize", None, _f32p, _sz, _sz, _u8p, C.c_int)
        self._q4k_quant_bf16 = _bind(L, "orc_q4k_quantize_from_bf16", None, _u16p, _sz, _sz,
                                     _u8p, C.c_int)
        self._q4k_deq = _bind(L, "orc_q4k_dequant_row", None, _u8p, _sz, _sz, _f32p)
        self._q4k_dot = _bind(L, "orc_q4k_dot_row", C.c_float, _u8p, _sz, _sz, _f32p)
        self._q4k_mm = _bind(L, "orc_q4k_matmul_t", None, _u8p, _sz, _sz, _f32p, _sz, _f32p,
                             C.c_int, _sz, _sz)
        self._q8act = _bind(L, "orc_q4k_quantize_activation_q8", None, _f32p, _sz, _i8p,
                            _f32p, _f32p)
        self._q8dot = _bind(L, "orc_q4k_dot_row_q8", C.c_float, _u8p, _sz, _sz, _i8p, _f32p, _f32p)
        self._q8gemv = _bind(L, "orc_q4k_gemv_q8", None, _u8p, _sz, _sz, _f32p, _f32p)
        self._bf16_mm = _bind(L, "orc_bf16_matmul_t", None, _u16p, _sz, _sz, _f32p, _sz,
                              _f32p, C.c_int, _sz, _sz)
        self._q4mat_quant = _bind(L, "orc_q4mat_quantize", None, _f32p, _sz, _u8p, _f32p)
        self._q4mat_deq = _bind(L, "orc_q4mat_dequant", None, _u8p, _f32p, _sz, _f32p)
        self._q4mat_mm = _bind(L, "orc_q4mat_matmul_t", None, _u8p, _f32p, _sz, _sz, _f32p,
                               _sz, _f32p)
        self._q40_dec = _bind(L, "orc_q4_0_decode_f32", None, _u8p, _sz, _f32p)
        self._q40_to_q4mat = _bind(L, "orc_q4_0_to_q4mat", None, _u8p, _sz, _u8p, _f32p)
        self._q40_enc = _bind(L, "orc_q4_0_encode_block", None, _f32p, C.c_float, _u8p)
        self._q40_quant = _bind(L, "orc_q4_0_quantize", None, _f32p, _sz, _u8p)
        self._q6k_dec = _bind(L, "orc_q6k_decode_f32", None, _u8p, _sz, _f32p)
        self._rmsnorm = _bind(L, "orc_rmsnorm", None, _f32p, _f32p, _sz, C.c_float, C.c_int, _f32p)
        self._swiglu = _bind(L, "orc_swiglu", None, _f32p, _f32p, _sz, _f32p)
        self._inv_freq = _bind(L, "orc_llama_inv_freq", None, C.c_float, _sz, _f32p, _sz, _f32p)
        self._rope = _bind(L, "orc_llama_rope_interleaved", None, _f32p, _sz, _sz, _sz, _f32p, _f32p)
        self._rope_half = _bind(L, "orc_llama_rope_half", None, _f32p, _sz, _sz, _sz, _f32p, _f32p)
        self._attn = _bind(L, "orc_gqa_attention_decode", None, _f32p, _f32p, _f32p, _sz, _sz, _sz, _sz, _sz,
                           C.c_float, _f32p)
        self._rms_head = _bind(L, "orc_rmsnorm_per_head", None, _f32p, _f32p, _sz, _sz, C.c_float, _f32p)
        self._rope_neox = _bind(L, "orc_rope_neox", None, _f32p, _sz, _sz, C.c_float, C.c_float, _sz, _f32p)
        self._gelu = _bind(L, "orc_gelu_tanh", None, _f32p, _sz, _f32p)
        self._f16_rne_n = _bind(L, "orc_f32_to_f16_rne_n", None, _f32p, _u16p, _sz)
        self._flux_attn = _bind(L, "orc_flux_attention", None, _f32p, _f32p, _f32p, _sz, _sz, _sz,
                                C.c_void_p, _sz, _f32p)
        self._argmax = _bind(L, "orc_argmax_first", C.c_int64, _f32p, _sz)
        self._normal = _bind(L, "orc_initrng_normal", None, C.c_uint64, _sz, C.c_float, _f32p)
        self._hw = _bind(L, "orc_hardware_threads", C.c_int)

    # layer operations -- tensor_node.cpp:320-344, 383-402; transformer5.cpp:186-190
    def rmsnorm(self, x: np.ndarray, gamma: np.ndarray, eps: float, gemma3: bool = False) -> np.ndarray:
        """Row-wise RMSNorm of x [rows, d] (or [d])."""
        x = np.ascontiguousarray(x, np.float32)
        g = np.ascontiguousarray(gamma, np.float32).reshape(-1)
        rows = x.reshape(-1, g.size)
        out = np.empty_like(rows)
        for r in range(rows.shape[0]):
            self._rmsnorm(np.ascontiguousarray(rows[r]), g, g.size, eps, 1 if gemma3 else 0, out[r])
        return out.reshape(x.shape)

    def llama_inv_freq(self, theta: float, head_dim: int, divisors=None) -> np.ndarray:
        d = np.ascontiguousarray(divisors if divisors is not None else np.zeros(1), np.float32)
        out = np.empty(head_dim // 2, np.float32)
        self._inv_freq(theta, head_dim, d, 0 if divisors is None else d.size, out)
        return out

    def llama_rope(self, x: np.ndarray, n_heads: int, head_dim: int, pos: int, inv_freq: np.ndarray,
                   half: bool = False) -> np.ndarray:
        """RoPE of one row [n_heads * head_dim]: interleaved pairing, or the
        half-split pairing with half=True."""
        xx = np.ascontiguousarray(x, np.float32).reshape(-1)
        out = np.empty_like(xx)
        fn = self._rope_half if half else self._rope
        fn(xx, n_heads, head_dim, pos, np.ascontiguousarray(inv_freq, np.float32), out)
        return out.reshape(np.shape(x))

    def gqa_attention_decode(self, q, k_cache, v_cache, seq_len: int, n_q: int, n_kv: int, d: int,
                             scale: float, k_start: int = 0) -> np.ndarray:
        """Positions [k_start, seq_len) of the cache (k_start > 0: a sliding window)."""
        qq = np.ascontiguousarray(q, np.float32).reshape(-1)
        kc = np.ascontiguousarray(k_cache, np.float32).reshape(-1)
        vc = np.ascontiguousarray(v_cache, np.float32).reshape(-1)
        out = np.empty(n_q * d, np.float32)
        self._attn(qq, kc, vc, k_start, seq_len, n_q, n_kv, d, scale, out)
        return out

    # Gemma 3 decode operations -- shaders/decode_gemma3.msl
    def rmsnorm_per_head(self, x, gamma, n_heads: int, head_dim: int, eps: float) -> np.ndarray:
        xx = np.ascontiguousarray(x, np.float32).reshape(-1)
        out = np.empty_like(xx)
        self._rms_head(xx, np.ascontiguousarray(gamma, np.float32), n_heads, head_dim, eps, out)
        return out.reshape(np.shape(x))

    def rope_neox(self, x, n_heads: int, head_dim: int, theta: float, freq_scale: float, pos: int) -> np.ndarray:
        xx = np.ascontiguousarray(x, np.float32).reshape(-1)
        out = np.empty_like(xx)
        self._rope_neox(xx, n_heads, head_dim, theta, freq_scale, pos, out)
        return out.reshape(np.shape(x))

    def gelu_tanh(self, x) -> np.ndarray:
        xx = np.ascontiguousarray(x, np.float32).reshape(-1)
        out = np.empty_like(xx)
        self._gelu(xx, xx.size, out)
        return out.reshape(np.shape(x))

    def flux_attention(self, q, k, v, n_heads: int, head_dim: int, rows=None) -> np.ndarray:
        """flux.cpp:287-321 on [t, n_heads * head_dim] f32 q, k, v; the output
        rows `rows` (all when None), as [len(rows), n_heads * head_dim]."""
        q, k, v = (np.ascontiguousarray(a, np.float32) for a in (q, k, v))
        t = q.shape[0]
        assert q.shape == k.shape == v.shape == (t, n_heads * head_dim)
        idx = None if rows is None else np.ascontiguousarray(rows, np.int64)
        n_rows = t if idx is None else idx.size
        out = np.empty((n_rows, n_heads * head_dim), np.float32)
        self._flux_attn(q, k, v, t, n_heads, head_dim, None if idx is None else idx.ctypes.data, n_rows, out)
        return out

    def f32_to_f16_rne_n(self, x) -> np.ndarray:
        xx = np.ascontiguousarray(x, np.float32).reshape(-1)
        out = np.empty(xx.size, np.uint16)
        self._f16_rne_n(xx, out, xx.size)
        return out.reshape(np.shape(x))

    def swiglu(self, gate: np.ndarray, up: np.ndarray) -> np.ndarray:
        g = np.ascontiguousarray(gate, np.float32).reshape(-1)
        u = np.ascontiguousarray(up, np.float32).reshape(-1)
        out = np.empty_like(g)
        self._swiglu(g, u, g.size, out)
        return out.reshape(np.shape(gate))

    # conversions -- bf16.hpp:42-126
    def f16_to_f32(self, b: int) -> float:
        return self._f16_to_f32(b)

    def f32_to_f16(self, v: float) -> int:
        return self._f32_to_f16(v)

    def bf16_to_f32(self, b: int) -> float:
        return self._bf16_to_f32(b)

    def f32_to_bf16(self, v: float) -> int:
        return self._f32_to_bf16(v)

    def f32_to_bf16_n(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty(x.shape, np.uint16)
        self._f32_to_bf16_n(x.reshape(-1), out.reshape(-1), x.size)
        return out

    def hardware_threads(self) -> int:
        return self._hw()

    # Q4_K -- quant_q4k.cpp
    def q4k_scale_min(self, sc: np.ndarray, j: int):
        s, m = C.c_float(), C.c_float()
        self._scale_min(np.ascontiguousarray(sc, np.uint8), j, C.byref(s), C.byref(m))
        return s.value, m.value

    def q4k_pack_scales(self, sv, mv) -> np.ndarray:
        out = np.zeros(12, np.uint8)
        self._pack(np.asarray(sv, np.uint8), np.asarray(mv, np.uint8), out)
        return out

    def q4k_quantize_block(self, x: np.ndarray) -> np.ndarray:
        out = np.zeros(144, np.uint8)
        self._qblock(np.ascontiguousarray(x, np.float32), out)
        return out

    def q4k_quantize(self, w: np.ndarray, n_threads: int | None = None) -> np.ndarray:
        w = np.ascontiguousarray(w, np.float32)
        rows, cols = w.shape
        out = np.zeros(rows * (cols // 256) * 144, np.uint8)
        self._q4k_quant(w, rows, cols, out, n_threads or self.hardware_threads())
        return out

    def q4k_quantize_from_bf16(self, w: np.ndarray, n_threads: int | None = None) -> np.ndarray:
        w = np.ascontiguousarray(w, np.uint16)
        rows, cols = w.shape
        out = np.zeros(rows * (cols // 256) * 144, np.uint8)
        self._q4k_quant_bf16(w, rows, cols, out, n_threads or self.hardware_threads())
        return out

    def q4k_dequant(self, blocks: np.ndarray, rows: int, cols: int) -> np.ndarray:
        """Rows via dequantize_row_into; columns past floor(cols/256)*256 stay 0."""
        out = np.zeros((rows, cols), np.float32)
        b = np.ascontiguousarray(blocks, np.uint8)
        for r in range(rows):
            row = np.zeros(cols, np.float32)
            self._q4k_deq(b, cols, r, row)
            out[r] = row
        return out

    def q4k_dot_row(self, blocks, cols, row, a) -> float:
        return self._q4k_dot(np.ascontiguousarray(blocks, np.uint8), cols, row,
                             np.ascontiguousarray(a, np.float32))

    def q4k_matmul_t(self, blocks, rows, cols, a, n_threads=None, r0=0, r1=None) -> np.ndarray:
        a = np.ascontiguousarray(a, np.float32).reshape(-1, cols)
        m = a.shape[0]
        y = np.zeros((m, rows), np.float32)
        self._q4k_mm(np.ascontiguousarray(blocks, np.uint8), rows, cols, a, m, y,
                     n_threads or self.hardware_threads(), r0, rows if r1 is None else r1)
        return y

    def q4k_quantize_activation_q8(self, a: np.ndarray):
        a = np.ascontiguousarray(a, np.float32)
        nb = (a.size + 31) // 32
        q8 = np.zeros(nb * 32, np.int8)
        sc = np.zeros(nb, np.float32)
        su = np.zeros(nb, np.float32)
        self._q8act(a, a.size, q8, sc, su)
        return q8, sc, su

    def q4k_dot_row_q8(self, blocks, cols, row, q8, scales, sums) -> float:
        """dot_row_q8 (quant_q4k.cpp:425-478) on a quantized activation."""
        return float(self._q8dot(np.ascontiguousarray(blocks, np.uint8), cols, row,
                                 np.ascontiguousarray(q8, np.int8), np.ascontiguousarray(scales, np.float32),
                                 np.ascontiguousarray(sums, np.float32)))

    def q4k_gemv_q8(self, blocks, rows, cols, a) -> np.ndarray:
        """gemv_mt's aarch64 branch (quant_q4k.cpp:564-600): Q8 activation, dot_row_q8."""
        y = np.zeros(rows, np.float32)
        self._q8gemv(np.ascontiguousarray(blocks, np.uint8), rows, cols,
                     np.ascontiguousarray(a, np.float32).reshape(-1)[:cols].copy(), y)
        return y

    # BF16 -- mat.cpp
    def bf16_matmul_t(self, w, a, n_threads=None, r0=0, r1=None) -> np.ndarray:
        w = np.ascontiguousarray(w, np.uint16)
        rows, cols = w.shape
        a = np.ascontiguousarray(a, np.float32).reshape(-1, cols)
        m = a.shape[0]
        y = np.zeros((m, rows), np.float32)
        self._bf16_mm(w, rows, cols, a, m, y, n_threads or self.hardware_threads(), r0,
                      rows if r1 is None else r1)
        return y

    # Q4Mat -- quant_q4.cpp
    def q4mat_quantize(self, w: np.ndarray):
        w = np.ascontiguousarray(w, np.float32)
        n = w.size
        packed = np.zeros((n + 1) // 2, np.uint8)
        scales = np.zeros((n + 31) // 32, np.float32)
        self._q4mat_quant(w.reshape(-1), n, packed, scales)
        return packed, scales

    def q4mat_dequant(self, packed, scales, n) -> np.ndarray:
        out = np.zeros(n, np.float32)
        self._q4mat_deq(np.ascontiguousarray(packed, np.uint8),
                        np.ascontiguousarray(scales, np.float32), n, out)
        return out

    def q4mat_matmul_t(self, packed, scales, rows, cols, a) -> np.ndarray:
        a = np.ascontiguousarray(a, np.float32).reshape(-1, cols)
        m = a.shape[0]
        y = np.zeros((m, rows), np.float32)
        self._q4mat_mm(np.ascontiguousarray(packed, np.uint8),
                       np.ascontiguousarray(scales, np.float32), rows, cols, a, m, y)
        return y

    # GGUF -- gguf.cpp
    def q4_0_decode(self, blocks, n_elem) -> np.ndarray:
        out = np.zeros(n_elem, np.float32)
        self._q40_dec(np.ascontiguousarray(blocks, np.uint8), n_elem, out)
        return out

    def q4_0_to_q4mat(self, blocks, n_elem):
        packed = np.zeros((n_elem + 1) // 2, np.uint8)
        scales = np.zeros((n_elem + 31) // 32, np.float32)
        self._q40_to_q4mat(np.ascontiguousarray(blocks, np.uint8), n_elem, packed, scales)
        return packed, scales

    def q4_0_encode_block(self, vals, scale) -> np.ndarray:
        out = np.zeros(18, np.uint8)
        self._q40_enc(np.ascontiguousarray(vals, np.float32), scale, out)
        return out

    def q4_0_quantize(self, w: np.ndarray) -> np.ndarray:
        w = np.ascontiguousarray(w, np.float32)
        out = np.zeros(w.size // 32 * 18, np.uint8)
        self._q40_quant(w.reshape(-1), w.size, out)
        return out

    def q6k_decode(self, blocks, n_elem) -> np.ndarray:
        out = np.zeros(n_elem, np.float32)
        self._q6k_dec(np.ascontiguousarray(blocks, np.uint8), n_elem, out)
        return out

    def argmax_first(self, v) -> int:
        v = np.ascontiguousarray(v, np.float32)
        return int(self._argmax(v, v.size))

    def initrng_normal(self, seed: int, n: int, std: float = 1.0) -> np.ndarray:
        out = np.empty(n, np.float32)
        self._normal(seed, n, std, out)
        return out


class Reference:
    """The reference's own compiled sources (oracle/_ref/libref_oracle.so)."""

    def __init__(self, path: str = REF_PATH):
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        L = self.lib = C.CDLL(path)
        self._f16_to_f32 = _bind(L, "ref_f16_to_f32", C.c_float, C.c_uint16)
        self._f32_to_f16 = _bind(L, "ref_f32_to_f16", C.c_uint16, C.c_float)
        self._bf16_to_f32 = _bind(L, "ref_bf16_to_f32", C.c_float, C.c_uint16)
        self._f32_to_bf16 = _bind(L, "ref_f32_to_bf16", C.c_uint16, C.c_float)
        self._hw = _bind(L, "ref_hardware_threads", C.c_int)
        self._scale_min = _bind(L, "ref_q4k_scale_min", None, _u8p, _sz,
                                C.POINTER(C.c_float), C.POINTER(C.c_float))
        self._qblock = _bind(L, "ref_q4k_quantize_block", None, _f32p, _u8p)
        self._q4k_quant = _bind(L, "ref_q4k_quantize", None, _f32p, _sz, _sz, _u8p)
        self._q4k_quant_bf16 = _bind(L, "ref_q4k_quantize_from_bf16", None, _u16p, _sz, _sz,
                                     _u8p)
        self._q4k_deq = _bind(L, "ref_q4k_dequant_row", None, _u8p, _sz, _sz, _sz, _f32p)
        self._q4k_dot = _bind(L, "ref_q4k_dot_row", C.c_float, _u8p, _sz, _sz, _sz, _f32p)
        self._q4k_mm = _bind(L, "ref_q4k_matmul_t", None, _u8p, _sz, _sz, _f32p, _sz, _f32p)
        self.q4k_new = _bind(L, "ref_q4k_new", C.c_void_p, _u8p, _sz, _sz)
        self.q4k_delete = _bind(L, "ref_q4k_delete", None, C.c_void_p)
        self.q4k_handle_matmul_t = _bind(L, "ref_q4k_handle_matmul_t", None, C.c_void_p,
                                         _f32p, _sz, _f32p)
        self._q8act = _bind(L, "ref_q4k_quantize_activation_q8", None, _f32p, _sz, _i8p,
                            _f32p, _f32p)
        self._bf16_mm = _bind(L, "ref_bf16_matmul_t", None, _u16p, _sz, _sz, _f32p, _sz, _f32p)
        self.bf16_new = _bind(L, "ref_bf16_new", C.c_void_p, _u16p, _sz, _sz)
        self.bf16_delete = _bind(L, "ref_bf16_delete", None, C.c_void_p)
        self.bf16_handle_matmul_t = _bind(L, "ref_bf16_handle_matmul_t", None, C.c_void_p,
                                          _f32p, _sz, _f32p)
        self._q4mat_quant = _bind(L, "ref_q4mat_quantize", None, _f32p, _sz, _sz, _u8p, _f32p)
        self._q4mat_mm = _bind(L, "ref_q4mat_matmul_t", None, _u8p, _f32p, _sz, _sz, _f32p,
                               _sz, _f32p)
        self._normal = _bind(L, "ref_initrng_normal", None, C.c_uint64, _sz, C.c_float, _f32p)

    def f16_to_f32(self, b):
        return self._f16_to_f32(b)

    def f32_to_f16(self, v):
        return self._f32_to_f16(v)

    def bf16_to_f32(self, b):
        return self._bf16_to_f32(b)

    def f32_to_bf16(self, v):
        return self._f32_to_bf16(v)

    def hardware_threads(self):
        return self._hw()

    def q4k_scale_min(self, sc, j):
        s, m = C.c_float(), C.c_float()
        self._scale_min(np.ascontiguousarray(sc, np.uint8), j, C.byref(s), C.byref(m))
        return s.value, m.value

    def q4k_quantize_block(self, x):
        out = np.zeros(144, np.uint8)
        self._qblock(np.ascontiguousarray(x, np.float32), out)
        return out

    def q4k_quantize(self, w):
        w = np.ascontiguousarray(w, np.float32)
        rows, cols = w.shape
        out = np.zeros(rows * (cols // 256) * 144, np.uint8)
        self._q4k_quant(w, rows, cols, out)
        return out

    def q4k_quantize_from_bf16(self, w):
        w = np.ascontiguousarray(w, np.uint16)
        rows, cols = w.shape
        out = np.zeros(rows * (cols // 256) * 144, np.uint8)
        self._q4k_quant_bf16(w, rows, cols, out)
        return out

    def q4k_dequant(self, blocks, rows, cols):
        out = np.zeros((rows, cols), np.float32)
        b = np.ascontiguousarray(blocks, np.uint8)
        for r in range(rows):
            row = np.zeros(cols, np.float32)
            self._q4k_deq(b, rows, cols, r, row)
            out[r] = row
        return out

    def q4k_dot_row(self, blocks, rows, cols, row, a):
        return self._q4k_dot(np.ascontiguousarray(blocks, np.uint8), rows, cols, row,
                             np.ascontiguousarray(a, np.float32))

    def q4k_matmul_t(self, blocks, rows, cols, a):
        a = np.ascontiguousarray(a, np.float32).reshape(-1, cols)
        m = a.shape[0]
        y = np.zeros((m, rows), np.float32)
        self._q4k_mm(np.ascontiguousarray(blocks, np.uint8), rows, cols, a, m, y)
        return y

    def q4k_quantize_activation_q8(self, a):
        a = np.ascontiguousarray(a, np.float32)
        nb = (a.size + 31) // 32
        q8 = np.zeros(nb * 32, np.int8)
        sc = np.zeros(nb, np.float32)
        su = np.zeros(nb, np.float32)
        self._q8act(a, a.size, q8, sc, su)
        return q8, sc, su

    def bf16_matmul_t(self, w, a):
        w = np.ascontiguousarray(w, np.uint16)
        rows, cols = w.shape
        a = np.ascontiguousarray(a, np.float32).reshape(-1, cols)
        m = a.shape[0]
        y = np.zeros((m, rows), np.float32)
        self._bf16_mm(w, rows, cols, a, m, y)
        return y

    def q4mat_quantize(self, w):
        w = np.ascontiguousarray(w, np.float32)
        rows, cols = w.shape
        n = w.size
        packed = np.zeros((n + 1) // 2, np.uint8)
        scales = np.zeros((n + 31) // 32, np.float32)
        self._q4mat_quant(w, rows, cols, packed, scales)
        return packed, scales

    def q4mat_matmul_t(self, packed, scales, rows, cols, a):
        a = np.ascontiguousarray(a, np.float32).reshape(-1, cols)
        m = a.shape[0]
        y = np.zeros((m, rows), np.float32)
        self._q4mat_mm(np.ascontiguousarray(packed, np.uint8),
                       np.ascontiguousarray(scales, np.float32), rows, cols, a, m, y)
        return y

    def initrng_normal(self, seed, n, std=1.0):
        out = np.empty(n, np.float32)
        self._normal(seed, n, std, out)
        return out


def reference_available() -> bool:
    return os.path.exists(REF_PATH)
