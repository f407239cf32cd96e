"""Writes tests/golden/ref_vectors.npz from the reference's own compiled code.

Run in a container that has the reference tree (it builds oracle/_ref first):

    make -C oracle && python tests/golden/make_golden.py

Every expected output here comes from oracle/_ref/libref_oracle.so, i.e. the
reference's src/quant_q4k.cpp, src/quant_q4.cpp and src/mat.cpp compiled with
its Release flags; the inputs are stored next to them.  The file holds plain
numeric arrays only (np.savez, no pickles) and is loaded with
allow_pickle=False.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

from oracle import Reference  # noqa: E402

OUT = os.path.join(HERE, "ref_vectors.npz")


def adversarial_rows(cols: int) -> np.ndarray:
    """Rows that exercise the quantizer's special branches."""
    rows = []
    rows.append(np.zeros(cols, np.float32))                                # all zero
    rows.append(np.full(cols, 0.37, np.float32))                           # constant > 0
    rows.append(np.full(cols, -0.37, np.float32))                          # constant < 0
    rows.append(np.abs(np.sin(np.arange(cols, dtype=np.float32) * 0.01)))  # non-negative
    r = np.sin(np.arange(cols, dtype=np.float32) * 0.01) * 0.8
    rows.append(r.astype(np.float32))                                      # test_quant style
    rows.append((np.arange(cols, dtype=np.float32) % 17 - 8) * 1e-6)       # tiny: f16 subnormal d
    rows.append((np.arange(cols, dtype=np.float32) % 5 - 2) * 1e3)         # large: f16 overflow
    sub = np.zeros(cols, np.float32)
    sub[::32] = 1.0                                                        # one spike per sub-block
    rows.append(sub)
    mixed = np.zeros(cols, np.float32)
    mixed[: cols // 2] = -3.0e-3                                           # half-negative block
    mixed[cols // 2:] = 5.0e-3
    rows.append(mixed)
    return np.stack(rows).astype(np.float32)


def main() -> None:
    ref = Reference()
    rng = np.random.default_rng(20261201)
    out: dict[str, np.ndarray] = {}

    # Q4_K quantizer + dequant + GEMV, random weights (BASELINE scale 0.02).
    for tag, (rows, cols, m) in {"a": (16, 512, 1), "b": (8, 1024, 3), "c": (8, 1152, 1)}.items():
        w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
        x = rng.standard_normal((m, cols)).astype(np.float32)
        blocks = ref.q4k_quantize(w)
        out[f"q4k_{tag}_w"] = w
        out[f"q4k_{tag}_x"] = x
        out[f"q4k_{tag}_blocks"] = blocks
        out[f"q4k_{tag}_deq"] = ref.q4k_dequant(blocks, rows, cols)[:2]
        out[f"q4k_{tag}_y"] = ref.q4k_matmul_t(blocks, rows, cols, x)

    # Quantizer on adversarial rows (every special branch of quantize_block).
    wa = adversarial_rows(256)
    out["q4k_adv_w"] = wa
    out["q4k_adv_blocks"] = ref.q4k_quantize(wa)
    out["q4k_adv_deq"] = ref.q4k_dequant(out["q4k_adv_blocks"], wa.shape[0], 256)

    # quantize_from_bf16 (quant_q4k.cpp:207-218).
    wb = rng.standard_normal((6, 512)).astype(np.float32)
    bits = np.array([ref.f32_to_bf16(float(v)) for v in wb.reshape(-1)], np.uint16).reshape(wb.shape)
    out["q4k_bf16_bits"] = bits
    out["q4k_bf16_blocks"] = ref.q4k_quantize_from_bf16(bits)

    # BF16 GEMV / M>1 (mat.cpp:304-414).
    for tag, (rows, cols, m) in {"a": (260, 256, 1), "b": (32, 256, 4)}.items():
        w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
        bits = np.array([ref.f32_to_bf16(float(v)) for v in w.reshape(-1)], np.uint16).reshape(w.shape)
        x = rng.standard_normal((m, cols)).astype(np.float32)
        out[f"bf16_{tag}_w"] = bits
        out[f"bf16_{tag}_x"] = x
        out[f"bf16_{tag}_y"] = ref.bf16_matmul_t(bits, x)

    # Q4Mat (quant_q4.cpp:17-114).
    w = (rng.standard_normal((20, 256)) * 0.02).astype(np.float32)
    x = rng.standard_normal((2, 256)).astype(np.float32)
    packed, scales = ref.q4mat_quantize(w)
    out["q4mat_w"] = w
    out["q4mat_x"] = x
    out["q4mat_packed"] = packed
    out["q4mat_scales"] = scales
    out["q4mat_y"] = ref.q4mat_matmul_t(packed, scales, 20, 256, x)

    # Q8 activations (quant_q4k.cpp:525-562, portable part).
    a = rng.standard_normal(200).astype(np.float32)
    a[64:96] = 0.0
    q8, sc, su = ref.q4k_quantize_activation_q8(a)
    out["q8_a"], out["q8_q"], out["q8_scales"], out["q8_sums"] = a, q8, sc, su

    # f16 / bf16 conversions on assorted values.
    vals = np.concatenate([
        rng.standard_normal(512).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 512),
        np.array([0.0, -0.0, 65504.0, 65520.0, 1e9, -1e9, 6e-8, 5.96e-8, 2.98e-8, 1e-10,
                  np.inf, -np.inf], np.float32)]).astype(np.float32)
    out["conv_vals"] = vals
    out["conv_f16"] = np.array([ref.f32_to_f16(float(v)) for v in vals], np.uint16)
    out["conv_bf16"] = np.array([ref.f32_to_bf16(float(v)) for v in vals], np.uint16)

    # InitRng (init_rng.hpp) -- same libm in one process; stored for the record.
    out["initrng_seed0"] = ref.initrng_normal(0, 64)

    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT}: {os.path.getsize(OUT)} bytes, {len(out)} arrays")


if __name__ == "__main__":
    main()
