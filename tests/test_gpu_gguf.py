"""GPU: GGUF file -> device weights -> GEMV (the load path of metal_decode.mm:157-176,
transformer4_load.cpp:133-143), against the oracle on the file's own bytes."""
import numpy as np
import pytest

from gguf_writer import STR, T_BF16, T_Q4_0, T_Q4_K, T_Q6_K, GgufWriter
from helpers import GEMV_TOL, from_dev, normwise_err, say, to_dev
from test_gpu_q6k import random_q6k

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def model_file(orc, tmp_path_factory):
    rng = np.random.default_rng(42)
    q4k_w = (rng.standard_normal((48, 512)) * 0.02).astype(np.float32)
    q40_w = (rng.standard_normal((16, 256)) * 0.02).astype(np.float32)
    bf16_w = orc.f32_to_bf16_n((rng.standard_normal((24, 256)) * 0.02).astype(np.float32))
    q6k = random_q6k(rng, 40, 512)
    w = (GgufWriter().add("general.architecture", STR, "llama")
         .add_tensor("blk.0.attn_q.weight", [512, 48], T_Q4_K, orc.q4k_quantize(q4k_w).tobytes())
         .add_tensor("blk.0.ffn_down.weight", [512, 40], T_Q6_K, q6k.tobytes())
         .add_tensor("blk.0.attn_v.weight", [256, 24], T_BF16, bf16_w.tobytes())
         .add_tensor("blk.0.ffn_gate.weight", [256, 16], T_Q4_0, orc.q4_0_quantize(q40_w).tobytes()))
    return w.write(str(tmp_path_factory.mktemp("gguf") / "tiny.gguf"))


def test_q4k_tensor_upload_and_gemv(rt, orc, model_file):
    say("[gguf] Q4_K upload + GEMV")
    f = rt.GgufFile(model_file)
    i = f.find("blk.0.attn_q.weight")
    n, k = f.linear_shape(i)
    assert (n, k) == (48, 512)
    blocks = f.read(i)
    dev = f.upload(i)
    assert np.array_equal(from_dev(dev), blocks)
    x = np.random.default_rng(1).standard_normal((2, k)).astype(np.float32)
    y = from_dev(rt.gemv(rt.Q4K, dev, to_dev(x), n, k))
    assert normwise_err(y, orc.q4k_matmul_t(blocks, n, k, x)) <= GEMV_TOL


def test_q6k_tensor_upload_widen_and_gemv(rt, orc, model_file):
    say("[gguf] Q6_K upload + widen + GEMV")
    f = rt.GgufFile(model_file)
    i = f.find("blk.0.ffn_down.weight")
    n, k = f.linear_shape(i)
    dev = f.upload(i)
    widened = orc.f32_to_bf16_n(orc.q6k_decode(f.read(i), n * k)).reshape(n, k)
    assert np.array_equal(from_dev(rt.dequant_q6k_bf16(dev, n, k)).view(np.uint16), widened)
    x = np.random.default_rng(2).standard_normal((1, k)).astype(np.float32)
    y = from_dev(rt.gemv_q6k_tiled(rt.q6k_tile(dev, n, k), to_dev(x), n, k))
    assert normwise_err(y, orc.bf16_matmul_t(widened, x)) <= GEMV_TOL


def test_bf16_and_q4_0_tensors(rt, orc, model_file):
    say("[gguf] BF16 and Q4_0 upload + GEMV")
    f = rt.GgufFile(model_file)
    i = f.find("blk.0.attn_v.weight")
    n, k = f.linear_shape(i)
    w = f.read(i).view(np.uint16).reshape(n, k)
    x = np.random.default_rng(3).standard_normal((1, k)).astype(np.float32)
    y = from_dev(rt.gemv(rt.BF16, f.upload(i).view(dtype=__import__("torch").int16), to_dev(x), n, k))
    assert normwise_err(y, orc.bf16_matmul_t(w, x)) <= GEMV_TOL
    i = f.find("blk.0.ffn_gate.weight")
    n, k = f.linear_shape(i)
    blocks = f.read(i)
    packed, scales = orc.q4_0_to_q4mat(blocks, n * k)
    y = from_dev(rt.gemv(rt.Q4_0, f.upload(i), to_dev(x), n, k))
    assert normwise_err(y, orc.q4mat_matmul_t(packed, scales, n, k, x)) <= GEMV_TOL


def test_upload_rejects_wrong_size(rt, model_file):
    import torch
    f = rt.GgufFile(model_file)
    dst = torch.empty(10, dtype=torch.uint8, device="cuda")
    lib = rt.library()
    assert lib.status("rt_hip_gguf_upload", f.h, 0, dst.data_ptr(), 10, None) == 1
