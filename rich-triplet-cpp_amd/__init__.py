"""MI355X (gfx950) quantized-linear path of rich-triplet: Q4_K / GGUF Q4_0 / BF16
GEMV and GEMM behind the C ABI of include/rt_hip.h.

The directory name is not a Python identifier; load it with
``importlib`` (see ``load_package`` in __graft_entry__.py), which registers
it as ``rich_triplet_cpp_amd``.
"""
from . import rt_hip  # noqa: F401
