"""ctypes binding of liblatent_hip.so (include/latent_ffn.h).

The library is loaded after `import torch`, so it shares torch's HIP runtime:
`tensor.data_ptr()` and `torch.cuda.current_stream().cuda_stream` are passed
straight through.  There is no fallback: if the library is missing, importing
this module raises.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch  # noqa: F401  (must precede the CDLL load; see module docstring)

# LATENT_HIP_LIB points at another build of the same library (e.g. a debug build).
LIB_PATH = Path(os.environ.get("LATENT_HIP_LIB", Path(__file__).resolve().parent / "liblatent_hip.so"))

LATENT_OK = 0
LATENT_E_INVALID = -1
LATENT_E_UNSUPPORTED = -2
LATENT_E_WORKSPACE = -3
LATENT_E_HIP = -4
LATENT_E_TIMEOUT = -5

LATENT_F32 = 0
LATENT_F16 = 1
LATENT_BF16 = 2

LATENT_OUT_REDUCED = 0
LATENT_OUT_PER_SLOT = 1

LATENT_LAYOUT_ROWS = 0
LATENT_LAYOUT_TILES = 1

# Factor indices of latent_tiles_repack, in the operand order.
LATENT_GATE_A, LATENT_GATE_B, LATENT_UP_A, LATENT_UP_B, LATENT_DOWN_A, LATENT_DOWN_B = range(6)

EXPORTED = (
    "latent_version",
    "latent_status_string",
    "latent_moe_workspace_size",
    "latent_moe_ffn_forward",
    "latent_moe_ffn_forward_noalloc",
    "latent_moe_path",
    "latent_stream_launch",
    "latent_moe_check",
    "latent_unpack",
    "latent_pack_nf4",
    "latent_pack_int8",
    "latent_route_workspace_size",
    "latent_route",
    "latent_expert_workspace_size",
    "latent_expert_forward",
    "latent_tiles_supported",
    "latent_tiles_repack",
)

LATENT_NOALLOC_SCRATCH_BYTES = 64 << 20
LATENT_NOALLOC_CONTROL_BYTES = 256 << 10

LATENT_Q_NF4 = 0
LATENT_Q_INT8 = 1

LATENT_DROP_NONE = 0
LATENT_DROP_BELOW = 1
LATENT_DROP_INCLUSIVE = 2


class LatentFactor(ctypes.Structure):
    _fields_ = [
        ("codes", ctypes.c_void_p),
        ("scales", ctypes.c_void_p),
        ("int8_bitmap", ctypes.c_void_p),
        ("int8_row_offset", ctypes.c_void_p),
        ("int8_data", ctypes.c_void_p),
        ("rows", ctypes.c_int64),
        ("cols", ctypes.c_int64),
    ]


class LatentMoeArgs(ctypes.Structure):
    _fields_ = [
        ("x", ctypes.c_void_p),
        ("x_dtype", ctypes.c_int32),
        ("ids", ctypes.c_void_p),
        ("weights", ctypes.c_void_p),
        ("weights_dtype", ctypes.c_int32),
        ("gate_a", LatentFactor),
        ("gate_b", LatentFactor),
        ("up_a", LatentFactor),
        ("up_b", LatentFactor),
        ("down_a", LatentFactor),
        ("down_b", LatentFactor),
        ("ranks", ctypes.c_void_p),
        ("n_tokens", ctypes.c_int64),
        ("n_embd", ctypes.c_int64),
        ("n_ff", ctypes.c_int64),
        ("n_expert", ctypes.c_int64),
        ("n_expert_used", ctypes.c_int64),
        ("max_rank", ctypes.c_int64),
        ("weight_before_down", ctypes.c_int32),
        ("out_mode", ctypes.c_int32),
        ("out", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
        ("layout", ctypes.c_int32),
    ]


class LatentRouteArgs(ctypes.Structure):
    _fields_ = [
        ("x", ctypes.c_void_p),
        ("x_dtype", ctypes.c_int32),
        ("router", ctypes.c_void_p),
        ("router_dtype", ctypes.c_int32),
        ("logits_in", ctypes.c_void_p),
        ("logits_out", ctypes.c_void_p),
        ("ids", ctypes.c_void_p),
        ("weights", ctypes.c_void_p),
        ("n_tokens", ctypes.c_int64),
        ("n_embd", ctypes.c_int64),
        ("n_expert", ctypes.c_int64),
        ("n_expert_used", ctypes.c_int64),
        ("drop_rule", ctypes.c_int32),
        ("drop_param", ctypes.c_float),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
    ]


class LatentFlatFactor(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("scales", ctypes.c_void_p),
        ("kind", ctypes.c_int32),
        ("group_size", ctypes.c_int32),
        ("rows", ctypes.c_int64),
        ("cols", ctypes.c_int64),
    ]


class LatentExpertArgs(ctypes.Structure):
    _fields_ = [
        ("x", ctypes.c_void_p),
        ("gate_a", LatentFlatFactor),
        ("gate_b", LatentFlatFactor),
        ("up_a", LatentFlatFactor),
        ("up_b", LatentFlatFactor),
        ("down_a", LatentFlatFactor),
        ("down_b", LatentFlatFactor),
        ("n_tokens", ctypes.c_int64),
        ("weight", ctypes.c_float),
        ("weight_before_down", ctypes.c_int32),
        ("out", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
    ]


class LatentError(RuntimeError):
    def __init__(self, status: int, what: str):
        super().__init__(f"{what}: {status_string(status)} ({status})")
        self.status = status


def _load() -> ctypes.CDLL:
    if not LIB_PATH.exists():
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `python latent_amd/build.py` "
            "(there is no CPU fallback)"
        )
    lib = ctypes.CDLL(str(LIB_PATH))
    lib.latent_version.restype = ctypes.c_int
    lib.latent_version.argtypes = []
    lib.latent_status_string.restype = ctypes.c_char_p
    lib.latent_status_string.argtypes = [ctypes.c_int]
    lib.latent_moe_workspace_size.restype = ctypes.c_int
    lib.latent_moe_workspace_size.argtypes = [ctypes.POINTER(LatentMoeArgs), ctypes.POINTER(ctypes.c_size_t)]
    lib.latent_moe_ffn_forward.restype = ctypes.c_int
    lib.latent_moe_ffn_forward.argtypes = [ctypes.POINTER(LatentMoeArgs), ctypes.c_void_p]
    lib.latent_moe_check.restype = ctypes.c_int
    lib.latent_moe_check.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
    lib.latent_moe_ffn_forward_noalloc.restype = ctypes.c_int
    lib.latent_moe_ffn_forward_noalloc.argtypes = [ctypes.POINTER(LatentMoeArgs), ctypes.c_void_p]
    lib.latent_moe_path.restype = ctypes.c_int
    lib.latent_moe_path.argtypes = [ctypes.POINTER(LatentMoeArgs)]
    lib.latent_stream_launch.restype = ctypes.c_int
    lib.latent_stream_launch.argtypes = [ctypes.POINTER(LatentMoeArgs)]
    lib.latent_unpack.restype = ctypes.c_int
    lib.latent_unpack.argtypes = [ctypes.POINTER(LatentFactor), ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p]
    lib.latent_pack_nf4.restype = ctypes.c_int
    lib.latent_pack_nf4.argtypes = [
        ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
    ]
    lib.latent_pack_int8.restype = ctypes.c_int
    lib.latent_pack_int8.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    lib.latent_route_workspace_size.restype = ctypes.c_int
    lib.latent_route_workspace_size.argtypes = [ctypes.POINTER(LatentRouteArgs), ctypes.POINTER(ctypes.c_size_t)]
    lib.latent_route.restype = ctypes.c_int
    lib.latent_route.argtypes = [ctypes.POINTER(LatentRouteArgs), ctypes.c_void_p]
    lib.latent_expert_workspace_size.restype = ctypes.c_int
    lib.latent_expert_workspace_size.argtypes = [ctypes.POINTER(LatentExpertArgs), ctypes.POINTER(ctypes.c_size_t)]
    lib.latent_expert_forward.restype = ctypes.c_int
    lib.latent_expert_forward.argtypes = [ctypes.POINTER(LatentExpertArgs), ctypes.c_void_p]
    lib.latent_tiles_supported.restype = ctypes.c_int
    lib.latent_tiles_supported.argtypes = [ctypes.POINTER(LatentMoeArgs)]
    lib.latent_tiles_repack.restype = ctypes.c_int
    lib.latent_tiles_repack.argtypes = [
        ctypes.c_int32, ctypes.POINTER(LatentFactor), ctypes.POINTER(LatentFactor), ctypes.c_int64, ctypes.c_int32,
        ctypes.c_void_p,
    ]
    return lib


lib = _load()


def status_string(status: int) -> str:
    return lib.latent_status_string(int(status)).decode()


def check(status: int, what: str) -> None:
    if status != LATENT_OK:
        raise LatentError(status, what)
