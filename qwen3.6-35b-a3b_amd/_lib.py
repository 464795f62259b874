"""ctypes binding of libmoe_gfx950.so (the C-ABI declared in include/moe_gfx950.h).

The library is built in-tree by build.py. There is no fallback: if the shared object is missing
or fails to load, importing this module raises, so no code path can silently run elsewhere.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libmoe_gfx950.so"

MOE_OK = 0
MOE_E_ARG = -1
MOE_E_FORMAT = -2
MOE_E_HIP = -3
MOE_E_WORKSPACE = -4
MOE_E_UNSUPPORTED = -5
ERROR_NAMES = {MOE_E_ARG: "bad-argument", MOE_E_FORMAT: "unsupported-format",
               MOE_E_HIP: "hip-error", MOE_E_WORKSPACE: "workspace-too-small",
               MOE_E_UNSUPPORTED: "unsupported-geometry"}

MOE_DT_F32 = 0
MOE_DT_BF16 = 1
MOE_FMT_Q8_0 = 8
MOE_FMT_Q4_K = 12
MOE_FMT_Q5_K = 13
MOE_FMT_Q6_K = 14
MOE_FMT_BF16 = 30
MOE_PATH_AUTO = 0
MOE_PATH_GEMV = 1
MOE_PATH_MFMA = 2
MOE_PATH_MFMA_BF16 = 3
MOE_PATH_GEMV_MULTI = 4
# every workspace starts with this many bytes of device-side sync words
SYNC_BYTES = 512 * 1024
# moe_block_forward_w_noalloc's static scratch (include/moe_gfx950.h)
NOALLOC_SCRATCH_BYTES = 16 << 20
NOALLOC_MAX_T = 120
# the workspace's status word and test-hook word (int32 indices), the status bits, and the first
# of the single-launch router's block-arrival counters (int32 index)
STATUS_WORD = 3
TEST_HOOK_WORD = 4
STATUS_SPIN_TIMEOUT = 1
STATUS_SYNC_STATE = 2
ROUTER_CNT_WORD = 120000



class LayerWeightsC(ctypes.Structure):
    """moe_layer_weights: one layer's MoE weights with their formats (include/moe_gfx950.h)."""
    _fields_ = [("w_router", ctypes.c_void_p), ("router_dtype", ctypes.c_int),
                ("logit_bias", ctypes.c_void_p), ("gate_q", ctypes.c_void_p),
                ("up_q", ctypes.c_void_p), ("gate_up_fmt", ctypes.c_int),
                ("down_q", ctypes.c_void_p), ("down_fmt", ctypes.c_int),
                ("ws_gate", ctypes.c_void_p), ("ws_up", ctypes.c_void_p),
                ("ws_down", ctypes.c_void_p), ("shared_fmt", ctypes.c_int),
                ("ws_scalar_gate", ctypes.c_void_p), ("scalar_gate_dtype", ctypes.c_int),
                ("norm_w", ctypes.c_void_p)]


class NextLayer(ctypes.Structure):
    """moe_next_layer: the router rows and norm weight of the layer the stream runs next."""
    _fields_ = [("w_router", ctypes.c_void_p), ("norm_w", ctypes.c_void_p)]


# every symbol include/moe_gfx950.h declares, with its ctypes signature
_VP, _I, _I64, _SZ, _CP = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_size_t, ctypes.c_char_p
SIGNATURES = {
    "moe_abi_version": (_I, []),
    "moe_last_error": (_CP, []),
    "moe_workspace_bytes": (_SZ, [_I, _I, _I, _I, _I, _I]),
    "moe_router_workspace_bytes": (_SZ, [_I, _I, _I]),
    "moe_dequant": (_I, [_VP, _I, _I64, _VP, _I, _VP]),
    "moe_router_topk": (_I, [_VP, _I, _VP, _I, _VP, _I, _I, _I, _I, _VP, _VP, _VP, _VP, _VP, _VP,
                             _SZ, _VP]),
    "moe_sort_permute": (_I, [_VP, _I, _I, _I, _VP, _VP, _VP, _VP, _VP, _SZ, _VP]),
    "moe_experts": (_I, [_VP, _I, _VP, _VP, _I, _VP, _I, _VP, _VP, _VP, _I, _I, _I, _I, _I, _I,
                         _VP, _VP, _SZ, _VP]),
    "moe_shared_expert": (_I, [_VP, _I, _VP, _VP, _VP, _I, _VP, _I, _I, _I, _I, _I, _VP, _VP, _VP,
                               _SZ, _VP]),
    "moe_combine": (_I, [_VP, _VP, _VP, _VP, _VP, _VP, _I, _I, _I, _VP, _VP, _VP, _VP, _VP]),
    "moe_block_forward": (_I, [_VP, _I, _I, _I, _I, _I, _I, _I, _VP, ctypes.c_float,
                               _VP, _VP, _VP, _I, _VP, _I, _VP,
                               _VP, _VP, _VP, _I, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP,
                               _VP, _VP, _SZ, _VP]),
    "moe_block_forward_prefetch": (_I, [_VP, _I, _I, _I, _I, _I, _I, _I, _VP, ctypes.c_float,
                                        _VP, _VP, _VP, _I, _VP, _I, _VP,
                                        _VP, _VP, _VP, _I, _VP, _VP, _VP, _VP, _VP, _VP, _VP,
                                        _VP, _VP, _VP, _VP, _SZ, _VP,
                                        ctypes.POINTER(NextLayer)]),
    "moe_block_forward_w": (_I, [_VP, _I, _I, _I, _I, _I, _I, _I, ctypes.POINTER(LayerWeightsC),
                                 ctypes.c_float, _I, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP,
                                 _VP, _VP, _SZ, _VP, ctypes.POINTER(LayerWeightsC)]),
    "moe_block_forward_w_noalloc": (_I, [_VP, _I, _I, _I, _I, _I, _I, _I,
                                         ctypes.POINTER(LayerWeightsC), ctypes.c_float, _I, _VP,
                                         _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP,
                                         ctypes.POINTER(LayerWeightsC)]),
    "moe_workspace_init": (_I, [_VP, _SZ, _VP]),
    "moe_workspace_status": (_I, [_VP, _SZ, _VP, _VP]),
    "moe_lm_head": (_I, [_VP, _I, _I, _I, _VP, _I, _I64, _VP, _I64, _VP, _VP]),
}


def _load() -> ctypes.CDLL:
    if not LIB_PATH.exists():
        raise ImportError(f"{LIB_PATH} is not built; run __graft_entry__.build() "
                          "(or python qwen3.6-35b-a3b_amd/build.py) first")
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()
