"""ctypes binding of libburnext_moe.so (include/burnext_moe.h, include/burnext_gptoss.h).

The library is the product; this module only marshals arguments.  It fails loudly when the
library has not been built -- there is no fallback path.
"""
from __future__ import annotations

import ctypes
import pathlib

PKG_DIR = pathlib.Path(__file__).resolve().parent.parent
LIB_PATH = PKG_DIR / "lib" / "libburnext_moe.so"

BURNEXT_OK = 0
BURNEXT_INVALID_ARG = 1
BURNEXT_UNSUPPORTED = 2
BURNEXT_OUT_OF_MEMORY = 3
BURNEXT_DEVICE_ERROR = 4
BURNEXT_WORKSPACE_TOO_SMALL = 5
STATUS_NAMES = {0: "OK", 1: "INVALID_ARG", 2: "UNSUPPORTED", 3: "OUT_OF_MEMORY", 4: "DEVICE_ERROR",
                5: "WORKSPACE_TOO_SMALL"}

BURNEXT_F32 = 0
BURNEXT_BF16 = 1
GATE_UP_HALVES = 0
GATE_UP_INTERLEAVED = 1
APPLY_RMSNORM = 1
ADD_RESIDUAL = 2
FORWARD_DEFAULT = APPLY_RMSNORM | ADD_RESIDUAL
FUSED_EXPERTS = 4  # forward only, opt-in: one launch for the experts of a batch of <= 16 tokens
NUM_KERNELS = 8
KERNEL_NAMES = ["router", "topk", "dispatch", "gate_up", "down", "combine", "reserved", "experts"]

# Every symbol include/burnext_moe.h declares.
EXPORTS = ["burnext_moe_layer_create", "burnext_moe_layer_destroy", "burnext_moe_workspace_size",
           "burnext_moe_forward", "burnext_moe_forward_noalloc", "burnext_moe_route", "burnext_moe_dispatch", "burnext_moe_route_dispatch",
           "burnext_mxfp4_dequant",
           "burnext_moe_profile_enable", "burnext_moe_profile_read", "burnext_last_error",
           # include/burnext_gptoss.h
           "burnext_gptoss_create", "burnext_gptoss_destroy", "burnext_gptoss_workspace_size", "burnext_gptoss_reset",
           "burnext_gptoss_cache_load", "burnext_gptoss_decode"]


class MxFp4Desc(ctypes.Structure):
    """Mirror of burnext_mxfp4_desc / QuantLinearMxFp4Desc."""
    _fields_ = [("experts", ctypes.c_uint64), ("rows", ctypes.c_uint64), ("cols", ctypes.c_uint64),
                ("bpr", ctypes.c_uint64), ("gpr", ctypes.c_uint64), ("ue8_offset", ctypes.c_int32)]

    @classmethod
    def for_matrix(cls, experts: int, rows: int, cols: int, ue8_offset: int = 0) -> "MxFp4Desc":
        return cls(experts, rows, cols, (cols + 1) // 2, (cols + 31) // 32, ue8_offset)


class MoeConfigC(ctypes.Structure):
    """Mirror of burnext_moe_config / MoeConfig."""
    _fields_ = [("d_model", ctypes.c_uint32), ("ffn_hidden", ctypes.c_uint32), ("num_experts", ctypes.c_uint32),
                ("experts_per_token", ctypes.c_uint32), ("swiglu_alpha", ctypes.c_float),
                ("swiglu_limit", ctypes.c_float), ("rms_eps", ctypes.c_float), ("disabled", ctypes.c_int32)]


class GptOssConfigC(ctypes.Structure):
    """Mirror of burnext_gptoss_config."""
    _fields_ = [(n, ctypes.c_uint32) for n in ("vocab_size", "d_model", "n_layers", "n_heads", "kv_heads", "head_dim",
                                               "max_batch", "cache_len", "window_policy", "window", "full_on_even",
                                               "rope_head_stride", "max_positions", "kv_bf16")] + \
               [(n, ctypes.c_float) for n in ("rms_eps", "rope_theta", "rope_scaling_factor", "rope_initial_context",
                                              "rope_ntk_alpha", "rope_ntk_beta", "scale_dk")] + \
               [("sink_tokens", ctypes.c_uint32), ("experts_bf16", ctypes.c_uint32)]


class GptOssWeightsC(ctypes.Structure):
    """Mirror of burnext_gptoss_weights (host bf16 bit patterns)."""
    _fields_ = [(n, ctypes.c_void_p) for n in ("tok_emb", "norm_attn", "wq", "bq", "wk", "bk", "wv", "bv", "wo", "bo",
                                               "sinks", "norm_final", "lm_head")]


class BurnextError(RuntimeError):
    def __init__(self, status: int, msg: str):
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {msg}")
        self.status = status


_lib = None
_vp = ctypes.c_void_p
_u64 = ctypes.c_uint64


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built; run __graft_entry__.build() (hipcc, gfx950)")
        L = ctypes.CDLL(str(LIB_PATH))
        L.burnext_last_error.restype = ctypes.c_char_p
        L.burnext_last_error.argtypes = []
        L.burnext_moe_layer_create.restype = ctypes.c_int
        L.burnext_moe_layer_create.argtypes = [ctypes.POINTER(MoeConfigC), ctypes.POINTER(MxFp4Desc), _vp, _vp,
                                               ctypes.POINTER(MxFp4Desc), _vp, _vp, _vp, _vp, ctypes.c_int, _vp, _vp,
                                               ctypes.c_int, _vp, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                               ctypes.POINTER(_vp)]
        L.burnext_moe_layer_destroy.restype = None
        L.burnext_moe_layer_destroy.argtypes = [_vp]
        L.burnext_moe_workspace_size.restype = ctypes.c_int
        L.burnext_moe_workspace_size.argtypes = [_vp, _u64, ctypes.POINTER(_u64)]
        L.burnext_moe_forward.restype = ctypes.c_int
        L.burnext_moe_forward.argtypes = [_vp, _vp, ctypes.c_int, _vp, _u64, ctypes.c_uint32, _vp, _u64, _vp]
        L.burnext_moe_forward_noalloc.restype = ctypes.c_int
        L.burnext_moe_forward_noalloc.argtypes = [_vp, _vp, ctypes.c_int, _vp, _u64, ctypes.c_uint32, _vp]
        L.burnext_moe_route.restype = ctypes.c_int
        L.burnext_moe_route.argtypes = [_vp, _vp, ctypes.c_int, _u64, ctypes.c_uint32, _vp, _vp, _vp, _vp, _u64, _vp]
        L.burnext_moe_dispatch.restype = ctypes.c_int
        L.burnext_moe_dispatch.argtypes = [_vp, _vp, _u64, _vp, _vp, _vp, _u64, _vp]
        L.burnext_moe_route_dispatch.restype = ctypes.c_int
        L.burnext_moe_route_dispatch.argtypes = [_vp, _vp, ctypes.c_int, _u64, ctypes.c_uint32, _vp, _vp, _vp, _vp,
                                                 _vp, _u64, _vp]
        L.burnext_mxfp4_dequant.restype = ctypes.c_int
        L.burnext_mxfp4_dequant.argtypes = [ctypes.POINTER(MxFp4Desc), _vp, _vp, _vp, ctypes.c_int, _vp]
        L.burnext_moe_profile_enable.restype = ctypes.c_int
        L.burnext_moe_profile_enable.argtypes = [_vp, ctypes.c_int]
        L.burnext_moe_profile_read.restype = ctypes.c_int
        L.burnext_moe_profile_read.argtypes = [_vp, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(_u64),
                                               ctypes.c_int]
        L.burnext_gptoss_create.restype = ctypes.c_int
        L.burnext_gptoss_create.argtypes = [ctypes.POINTER(GptOssConfigC), ctypes.POINTER(GptOssWeightsC), _vp,
                                            ctypes.c_int, ctypes.POINTER(_vp)]
        L.burnext_gptoss_destroy.restype = None
        L.burnext_gptoss_destroy.argtypes = [_vp]
        L.burnext_gptoss_workspace_size.restype = ctypes.c_int
        L.burnext_gptoss_workspace_size.argtypes = [_vp, ctypes.c_uint32, ctypes.POINTER(_u64)]
        L.burnext_gptoss_reset.restype = ctypes.c_int
        L.burnext_gptoss_reset.argtypes = [_vp]
        L.burnext_gptoss_cache_load.restype = ctypes.c_int
        L.burnext_gptoss_cache_load.argtypes = [_vp, _vp, _vp, ctypes.c_uint32, ctypes.c_uint32, _vp]
        L.burnext_gptoss_decode.restype = ctypes.c_int
        L.burnext_gptoss_decode.argtypes = [_vp, _vp, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, _vp, _vp, _vp,
                                            _vp, _u64, _vp]
        _lib = L
    return _lib


def last_error() -> str:
    return lib().burnext_last_error().decode()


def check(status: int) -> None:
    if status != BURNEXT_OK:
        raise BurnextError(status, last_error())
