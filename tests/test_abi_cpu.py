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
        (lambda a: setattr(a, "n_expert_used", 65), "LATENT_E_UNSUPPORTED"),
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
    assert n.value == 112 * 4 * 256 * 4  # one f32 [T][E] slice per 64 rows of d
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


def _expert_args(L, d=16, ff=12, r=(4, 4, 4), T=3, kinds=(0, 0, 0, 0, 0, 0), group=(32, 32, 32, 32, 32, 32)):
    keep = []

    def fac(rows, cols, kind, g):
        data = np.zeros(rows * cols + 64, np.uint8)
        s = np.zeros(rows * cols // g + 2, np.uint16)
        keep.extend([data, s])
        return L.LatentFlatFactor(data=data.ctypes.data, scales=s.ctypes.data, kind=kind, group_size=g,
                                  rows=rows, cols=cols)

    a = L.LatentExpertArgs()
    shapes = [(d, r[0]), (r[0], ff), (d, r[1]), (r[1], ff), (ff, r[2]), (r[2], d)]
    for name, (rows, cols), kind, g in zip(("gate_a", "gate_b", "up_a", "up_b", "down_a", "down_b"), shapes, kinds,
                                           group):
        setattr(a, name, fac(rows, cols, kind, g))
    a.n_tokens = T
    return a, keep


def test_expert_workspace_and_argument_checks(L):
    # the reference test's shapes (tests/test_latent_loader.py:100-127) and an odd rank
    for r in ((4, 4, 4), (37, 33, 5)):
        a, keep = _expert_args(L, r=r)
        n = ctypes.c_size_t(0)
        assert L.lib.latent_expert_workspace_size(ctypes.byref(a), ctypes.byref(n)) == L.LATENT_OK and n.value > 0
    a, keep = _expert_args(L, kinds=(0, 1, 0, 0, 1, 0), group=(32, 64, 32, 32, 64, 32))
    assert L.lib.latent_expert_workspace_size(ctypes.byref(a), ctypes.byref(ctypes.c_size_t())) == L.LATENT_OK
    cases = [
        (lambda a: setattr(a.gate_b, "rows", 5), L.LATENT_E_INVALID),   # rank mismatch with gate_a
        (lambda a: setattr(a.down_b, "cols", 15), L.LATENT_E_INVALID),  # output width != d
        (lambda a: setattr(a.up_a, "kind", 3), L.LATENT_E_INVALID),
        (lambda a: setattr(a.up_a, "data", None), L.LATENT_E_INVALID),
        (lambda a: setattr(a.up_a, "group_size", 48), L.LATENT_E_UNSUPPORTED),
        (lambda a: setattr(a, "n_tokens", -1), L.LATENT_E_INVALID),
    ]
    for mutate, status in cases:
        a, keep = _expert_args(L)
        mutate(a)
        assert L.lib.latent_expert_workspace_size(ctypes.byref(a), ctypes.byref(ctypes.c_size_t())) == status
        assert L.lib.latent_expert_forward(ctypes.byref(a), None) == status
    a, keep = _expert_args(L)
    assert L.lib.latent_expert_forward(ctypes.byref(a), None) == L.LATENT_E_INVALID  # no x / out
    x = np.zeros(64, np.float32)
    a.x = a.out = x.ctypes.data
    assert L.lib.latent_expert_forward(ctypes.byref(a), None) == L.LATENT_E_WORKSPACE
    a.n_tokens = 0
    assert L.lib.latent_expert_forward(ctypes.byref(a), None) == L.LATENT_OK


def test_check_rejects_missing_workspace(L):
    buf = np.zeros(64, np.uint8)
    assert L.lib.latent_moe_check(buf.ctypes.data, 64, None) == L.LATENT_E_WORKSPACE  # below the control block
    assert L.lib.latent_moe_check(None, 64, None) == L.LATENT_E_WORKSPACE  # NULL names the noalloc array: bytes 0
    assert L.status_string(L.LATENT_E_TIMEOUT) != "unknown status"


def test_runtime_load_pair_keeps_artifacts_flat():
    from latent_amd import runtime
    from oracle import synth

    rng = np.random.default_rng(5)
    m = rng.standard_normal((40, 37)).astype(np.float32) @ rng.standard_normal((37, 48)).astype(np.float32)
    arrays, rep = synth.compress_matrix("w", m, energy=1.0, min_rank=37, max_rank=37, error_threshold=1e9)
    pair = runtime.load_pair(arrays, "w")
    assert (pair.n_in, pair.rank, pair.n_out) == (40, 37, 48)
    assert pair.a.kind == 0 and pair.a.group_size == 32 and pair.a.groups == (40 * 37 + 31) // 32
    assert np.array_equal(pair.a.data, arrays["w.a.nf4"])  # no repacking: the artifact's bytes as they are
    with pytest.raises(KeyError):
        runtime.load_pair(arrays, "nope")
    bad = dict(arrays)
    bad["w.a.scales"] = bad["w.a.scales"][:-1]
    with pytest.raises(ValueError):
        runtime.load_pair(bad, "w")


def test_layout_flag_and_tiles_queries(L):
    # a DeepSeek-V3-like shape at rank 256 can take the tile layout; rank 64 cannot
    a, keep = _args(L, d=512, ff=768, R=256)
    assert L.lib.latent_tiles_supported(ctypes.byref(a)) == 1
    b, keep2 = _args(L)
    assert L.lib.latent_tiles_supported(ctypes.byref(b)) == 0
    b.up_a.int8_bitmap = 4096
    assert L.lib.latent_tiles_supported(ctypes.byref(b)) == 0
    # the flag is checked, and a tile-layout call needs a shape the layout exists for
    a.layout = 3
    assert _ws(L, a)[0] == L.LATENT_E_INVALID
    b, keep2 = _args(L)
    b.layout = L.LATENT_LAYOUT_TILES
    assert _ws(L, b)[0] == L.LATENT_E_UNSUPPORTED
    assert L.lib.latent_moe_path(ctypes.byref(b)) == L.LATENT_E_UNSUPPORTED


def test_tiles_repack_argument_checks(L):
    f = L.LatentFactor(codes=16, scales=16, rows=512, cols=256)
    g = L.LatentFactor(codes=32, scales=32, rows=512, cols=256)
    bad = [
        (L.LATENT_GATE_A, L.LatentFactor(codes=16, scales=16, rows=500, cols=256), g, L.LATENT_E_INVALID),  # rows differ
        (L.LATENT_GATE_A, L.LatentFactor(codes=16, scales=16, rows=384, cols=256),
         L.LatentFactor(codes=32, scales=32, rows=384, cols=256), L.LATENT_E_UNSUPPORTED),  # not whole K tiles
        (L.LATENT_GATE_B, f, g, L.LATENT_E_UNSUPPORTED),  # gate_b has 256 rows
        (6, f, g, L.LATENT_E_INVALID),
        (L.LATENT_GATE_A, L.LatentFactor(codes=16, scales=None, rows=512, cols=256), g, L.LATENT_E_INVALID),
        (L.LATENT_GATE_A, f, L.LatentFactor(codes=33, scales=32, rows=512, cols=256), L.LATENT_E_INVALID),  # unaligned
        (L.LATENT_GATE_A, L.LatentFactor(codes=16, scales=16, int8_bitmap=64, rows=512, cols=256), g,
         L.LATENT_E_UNSUPPORTED),
    ]
    for factor, src, dst, status in bad:
        assert L.lib.latent_tiles_repack(factor, ctypes.byref(src), ctypes.byref(dst), 4, 1, None) == status
    assert L.lib.latent_tiles_repack(0, None, ctypes.byref(g), 4, 1, None) == L.LATENT_E_INVALID
