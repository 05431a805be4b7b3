"""The C ABI of liblatent_hip.so without a GPU: load, exports, argument checks.

Only calls that return before any HIP runtime call are made here.
"""

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "latent_ffn.h"


@pytest.fixture(scope="module")
def L():
    from latent_amd import _lib

    return _lib


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(latent_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_entry_points():
    names = declared_functions()
    assert {"latent_moe_ffn_forward", "latent_moe_workspace_size", "latent_unpack", "latent_pack_nf4"} <= set(names)


def test_library_exports_every_declared_symbol(L):
    for name in declared_functions():
        assert hasattr(L.lib, name), name
    assert set(declared_functions()) == set(L.EXPORTED)


def test_status_strings_and_version(L):
    assert L.lib.latent_version() >= 100
    for code in (L.LATENT_OK, L.LATENT_E_INVALID, L.LATENT_E_UNSUPPORTED, L.LATENT_E_WORKSPACE, L.LATENT_E_HIP):
        assert L.status_string(code) and L.status_string(code) != "unknown status"
    assert L.status_string(12345) == "unknown status"


def _args(L, d=256, ff=512, E=16, k=4, R=64, T=8):
    bufs = []

    def fac(rows, cols):
        c = np.zeros(E * rows * cols // 2 + 16, np.uint8)
        s = np.zeros(E * rows * cols // 32, np.uint16)
        bufs.extend([c, s])
        off = (-c.ctypes.data) % 16
        return L.LatentFactor(codes=c.ctypes.data + off, scales=s.ctypes.data, rows=rows, cols=cols)

    a = L.LatentMoeArgs()
    a.gate_a, a.gate_b = fac(d, R), fac(R, ff)
    a.up_a, a.up_b = fac(d, R), fac(R, ff)
    a.down_a, a.down_b = fac(ff, R), fac(R, d)
    a.n_tokens, a.n_embd, a.n_ff, a.n_expert, a.n_expert_used, a.max_rank = T, d, ff, E, k, R
    a.x_dtype, a.weights_dtype, a.out_mode = L.LATENT_BF16, L.LATENT_F32, L.LATENT_OUT_REDUCED
    return a, bufs


def _ws(L, a):
    n = ctypes.c_size_t(0)
    st = L.lib.latent_moe_workspace_size(ctypes.byref(a), ctypes.byref(n))
    return st, n.value


def test_workspace_size_scales_with_pairs(L):
    a, keep = _args(L)
    st, small = _ws(L, a)
    assert st == L.LATENT_OK and small > 0
    a.n_tokens = 64
    st, big = _ws(L, a)
    assert st == L.LATENT_OK and big > small
    # pair accumulators: (T*k) * 3R floats at least
    assert big >= 64 * 4 * 3 * 64 * 4


@pytest.mark.parametrize(
    "mutate,status",
    [
        (lambda a: setattr(a, "n_embd", 250), "LATENT_E_INVALID"),
        (lambda a: setattr(a, "max_rank", 48), "LATENT_E_INVALID"),
        (lambda a: setattr(a, "x_dtype", 9), "LATENT_E_INVALID"),
        (lambda a: setattr(a, "out_mode", 2), "LATENT_E_INVALID"),
        (lambda a: setattr(a, "weights_dtype", 2), "LATENT_E_INVALID"),
        (lambda a: setattr(a.gate_b, "cols", 256), "LATENT_E_INVALID"),
        (lambda a: setattr(a.down_a, "codes", None), "LATENT_E_INVALID"),
        (lambda a: setattr(a.up_a, "int8_bitmap", 4096), "LATENT_E_INVALID"),
        (lambda a: setattr(a, "n_expert", 5000), "LATENT_E_UNSUPPORTED"),
        (lambda a: setattr(a, "max_rank", 1024) or setattr(a.gate_a, "cols", 1024) or setattr(a.up_a, "cols", 1024)
         or setattr(a.down_a, "cols", 1024) or setattr(a.gate_b, "rows", 1024) or setattr(a.up_b, "rows", 1024)
         or setattr(a.down_b, "rows", 1024), "LATENT_E_UNSUPPORTED"),
    ],
)
def test_invalid_arguments_are_rejected(L, mutate, status):
    a, keep = _args(L)
    mutate(a)
    st, _ = _ws(L, a)
    assert st == getattr(L, status)
    assert L.lib.latent_moe_ffn_forward(ctypes.byref(a), None) == st


def test_forward_checks_workspace_and_pointers_before_launch(L):
    a, keep = _args(L)
    # no x / ids / weights / out
    assert L.lib.latent_moe_ffn_forward(ctypes.byref(a), None) == L.LATENT_E_INVALID
    x = np.zeros(64, np.float32)
    a.x = a.ids = a.weights = a.out = x.ctypes.data + ((-x.ctypes.data) % 16)
    assert L.lib.latent_moe_ffn_forward(ctypes.byref(a), None) == L.LATENT_E_WORKSPACE
    # zero tokens is a no-op that succeeds without touching the device
    a.n_tokens = 0
    assert L.lib.latent_moe_ffn_forward(ctypes.byref(a), None) == L.LATENT_OK


def test_codec_entry_points_reject_bad_shapes(L):
    f = L.LatentFactor(codes=None, scales=None, rows=4, cols=64)
    out = np.zeros(256, np.float32)
    assert L.lib.latent_unpack(ctypes.byref(f), 0, out.ctypes.data, None) == L.LATENT_E_INVALID
    assert L.lib.latent_pack_nf4(None, 4, 64, None, None, None) == L.LATENT_E_INVALID
    buf = np.zeros(1024, np.float32)
    p = buf.ctypes.data + ((-buf.ctypes.data) % 16)
    assert L.lib.latent_pack_nf4(p, 4, 48, p, p, None) == L.LATENT_E_INVALID
    assert L.lib.latent_pack_int8(p, 0, p, p, None) == L.LATENT_E_INVALID


def test_route_argument_checks(L):
    a = L.LatentRouteArgs()
    a.n_tokens, a.n_embd, a.n_expert, a.n_expert_used = 4, 7168, 256, 8
    a.x_dtype, a.router_dtype = L.LATENT_BF16, L.LATENT_F32
    n = ctypes.c_size_t(0)
    assert L.lib.latent_route_workspace_size(ctypes.byref(a), ctypes.byref(n)) == L.LATENT_OK
    assert n.value == 56 * 4 * 256 * 4  # one f32 [T][E] slice per 128 rows of d
    a.logits_in = 16
    assert L.lib.latent_route_workspace_size(ctypes.byref(a), ctypes.byref(n)) == L.LATENT_OK and n.value == 0
    for field, value, status in [("n_expert_used", 257, L.LATENT_E_INVALID), ("n_expert", 2048, L.LATENT_E_UNSUPPORTED),
                                 ("n_expert_used", 65, L.LATENT_E_UNSUPPORTED), ("drop_rule", 7, L.LATENT_E_INVALID)]:
        b = L.LatentRouteArgs.from_buffer_copy(a)
        setattr(b, field, value)
        assert L.lib.latent_route_workspace_size(ctypes.byref(b), ctypes.byref(n)) == status, field
    b = L.LatentRouteArgs.from_buffer_copy(a)
    b.drop_rule, b.drop_param = L.LATENT_DROP_INCLUSIVE, 1.5
    assert L.lib.latent_route(ctypes.byref(b), None) == L.LATENT_E_INVALID
    b = L.LatentRouteArgs.from_buffer_copy(a)
    b.logits_in = 0
    b.router_dtype = L.LATENT_F16  # f16 router matrices are not supported
    assert L.lib.latent_route(ctypes.byref(b), None) == L.LATENT_E_INVALID
