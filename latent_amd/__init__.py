"""latent_amd: MI355X (gfx950) LATENT fused low-rank expert FFN.

    from latent_amd import StackedLayer, moe_forward        # MoE layer (ggml op)
    from latent_amd.runtime import load_pair, swiglu_expert # loader/latent_runtime.py
    from latent_amd import route, Router, DecodeStack        # GPU routing, stacked decode

The compute runs in `liblatent_hip.so` (hand-written HIP for gfx950, C ABI in
include/latent_ffn.h); torch provides device memory and streams.  Importing
this package without the built library raises ImportError.
"""

from ._lib import (  # noqa: F401
    LATENT_BF16,
    LATENT_F16,
    LATENT_F32,
    LATENT_OUT_PER_SLOT,
    LATENT_OUT_REDUCED,
    LatentError,
    lib,
)
from .moe import (  # noqa: F401
    DeviceFactor,
    StackedLayer,
    moe_forward,
    moe_path,
    pack_int8,
    pack_nf4,
    unpack,
    workspace_error,
    workspace_size,
)
from .router import Router, route  # noqa: F401
from .stack import DecodeStack  # noqa: F401

__version__ = "0.1.0"


def library_version() -> int:
    return int(lib.latent_version())
