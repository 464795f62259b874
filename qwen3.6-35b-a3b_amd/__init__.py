"""gfx950 (MI355X) MoE block of Qwen3.6-35B-A3B: router, token sort/permute, fused Q4_K/Q6_K
decode GEMV, MFMA grouped GEMM for prefill, shared expert and combine — hand-written HIP kernels
behind the C-ABI in include/moe_gfx950.h, called through ctypes with PyTorch-ROCm tensors.

The directory name is not a Python identifier; load it with
    importlib.util.spec_from_file_location("qwen36_moe", "<repo>/qwen3.6-35b-a3b_amd/__init__.py",
                                           submodule_search_locations=["<repo>/qwen3.6-35b-a3b_amd"])
(`__graft_entry__.load_package()` does exactly this).
"""
from . import _lib, quant, weights, synth, gguf  # noqa: F401
from . import abi, block  # noqa: F401
from .abi import Refused  # noqa: F401
from .weights import LayerWeights, load_geometry  # noqa: F401
