"""The tile layout (latent_tiles_repack) and a layer held only in it.

Pinned by an independent numpy statement of the layout as include/latent_ffn.h
and the stream kernels document it (which tile-layout nibble holds which
(row, column) of the row layout, which scale slot holds which (row, group)),
by round trips, and end to end: the twelve operand tensors of the reference's
op (kernels/latent_fused_expert_ffn.cu:134-149) repacked one by one, as a
ggml repack buffer type would at upload, with the row-layout buffers then
overwritten, drive latent_moe_ffn_forward through the C ABI to the oracle's
result on the decode and the prefill path.
"""

import ctypes

import numpy as np
import pytest

from oracle import latent_ref as ref
from oracle import routing, synth

pytestmark = pytest.mark.gpu

FACTORS = ref.FACTOR_NAMES  # operand order: gate_a, gate_b, up_a, up_b, down_a, down_b


def _kind(name):
    return {"gate_b": "H", "up_b": "H", "down_b": "N"}.get(name, "K")


def _nibble_map(kind, rows, cols):
    """(row, col) of every nibble of one expert's tile-layout codes, in byte
    order, low nibble first."""
    out_r, out_c = [], []
    if kind == "H":
        ntiles, tw = cols // 128, 128
        w, sp, lane, dw, q, h = np.meshgrid(np.arange(4), np.arange(4), np.arange(64), np.arange(4), np.arange(4),
                                            np.arange(2), indexing="ij")
        s = 2 * sp + (dw >> 1)
        rr = 32 * s + 8 * (lane >> 4) + 2 * q + h
        cc = 32 * w + 2 * (lane & 15) + (dw & 1)
    else:
        ntiles, tw = (rows // 256, 0) if kind == "K" else (cols // 256, 256)
        w, s, lane, j, q, h = np.meshgrid(np.arange(4), np.arange(8), np.arange(64), np.arange(4), np.arange(4),
                                          np.arange(2), indexing="ij")
        rr = 32 * s + 8 * (lane >> 4) + 2 * q + h
        cc = 64 * w + 4 * (lane & 15) + j
    for t in range(ntiles):
        out_r.append(rr.ravel() + (256 * t if kind == "K" else 0))
        out_c.append(cc.ravel() + (tw * t if kind != "K" else 0))
    return np.concatenate(out_r), np.concatenate(out_c)


def _scale_map(kind, rows, cols):
    """(row, group) of every fp16 scale of one expert's tile-layout scales."""
    ng = 4 if kind == "H" else 8
    ntiles = rows // 256 if kind == "K" else cols // (128 if kind == "H" else 256)
    G, Pp, half = np.meshgrid(np.arange(ng), np.arange(128), np.arange(2), indexing="ij")
    P = Pp ^ ((G & 1) << 3)
    rr, gg = (2 * P + half).ravel(), G.ravel()
    out_r, out_g = [], []
    for t in range(ntiles):
        out_r.append(rr + (256 * t if kind == "K" else 0))
        out_g.append(gg + (0 if kind == "K" else ng * t))
    return np.concatenate(out_r), np.concatenate(out_g)


def _tiles_numpy(name, codes, scales):
    """The tile layout of row-layout codes u8 [E, rows, cols/2] and scales
    u16 [E, rows, cols/32], by the documented mapping."""
    E, rows, half = codes.shape
    cols = half * 2
    nib = np.empty((E, rows, cols), np.uint8)
    nib[:, :, 0::2] = codes & 15
    nib[:, :, 1::2] = codes >> 4
    r, c = _nibble_map(_kind(name), rows, cols)
    flat = nib[:, r, c]  # [E, rows*cols] in tile nibble order
    tcodes = (flat[:, 0::2] | (flat[:, 1::2] << 4)).astype(np.uint8).reshape(codes.shape)
    sr, sg = _scale_map(_kind(name), rows, cols)
    tscales = scales[:, sr, sg].reshape(scales.shape)
    return tcodes, tscales


def _repack(f, factor, rows_to_tiles, codes=True, scales=True):
    import torch

    from latent_amd import _lib

    dc = torch.empty_like(f.codes) if codes else None
    ds = torch.empty_like(f.scales) if scales else None
    src = _lib.LatentFactor(codes=f.codes.data_ptr() if codes else None, scales=f.scales.data_ptr() if scales else None,
                            rows=f.rows, cols=f.cols)
    dst = _lib.LatentFactor(codes=dc.data_ptr() if codes else None, scales=ds.data_ptr() if scales else None,
                            rows=f.rows, cols=f.cols)
    st = _lib.lib.latent_tiles_repack(factor, ctypes.byref(src), ctypes.byref(dst), f.n_expert,
                                      1 if rows_to_tiles else 0, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    _lib.check(st, "latent_tiles_repack")
    return dc, ds


@pytest.fixture(scope="module")
def small(gpu):
    from latent_amd import synth as gsynth

    # d 512 and ff 768: two K tiles of gate_a / up_a, three of down_a, six H
    # tiles of gate_b / up_b, two N tiles of down_b per expert.
    return gsynth.make_layer(seed=71, n_expert=5, d=512, ff=768, max_rank=256).to_layout("rows")


def test_repack_matches_documented_layout_and_round_trips(gpu, small):
    import torch

    for k, name in enumerate(FACTORS):
        f = getattr(small, name)
        tc, ts = _repack(f, k, True)
        want_c, want_s = _tiles_numpy(name, f.codes.cpu().numpy(), f.scales.cpu().numpy().view(np.uint16))
        assert np.array_equal(tc.cpu().numpy(), want_c), name
        assert np.array_equal(ts.cpu().numpy().view(np.uint16), want_s), name
        # codes and scales on their own (a ggml tensor each) give the same bytes
        c_only, _ = _repack(f, k, True, scales=False)
        _, s_only = _repack(f, k, True, codes=False)
        assert torch.equal(c_only, tc) and torch.equal(s_only.view(torch.int16), ts.view(torch.int16))
        # back to rows: the original bytes
        from latent_amd import DeviceFactor

        back_c, back_s = _repack(DeviceFactor(tc, ts, layout="tiles"), k, False)
        assert torch.equal(back_c, f.codes) and torch.equal(back_s.view(torch.int16), f.scales.view(torch.int16))
        # an expert slice repacks on its own to the same bytes
        sub = f.select([1, 2, 3])
        sc, ss = _repack(sub, k, True)
        assert torch.equal(sc, tc[1:4]) and torch.equal(ss.view(torch.int16), ts[1:4].view(torch.int16))


def test_repack_rejects_bad_shapes(gpu, small):
    import torch

    from latent_amd import _lib

    f = small.gate_a
    dc = torch.empty_like(f.codes)
    src = _lib.LatentFactor(codes=f.codes.data_ptr(), scales=None, rows=f.rows, cols=f.cols)
    dst = _lib.LatentFactor(codes=dc.data_ptr(), scales=None, rows=f.rows, cols=f.cols)
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    # gate_a's shape is not a down_b / gate_b shape
    assert _lib.lib.latent_tiles_repack(_lib.LATENT_DOWN_B, ctypes.byref(src), ctypes.byref(dst), 5, 1, s) == \
        _lib.LATENT_E_UNSUPPORTED
    assert _lib.lib.latent_tiles_repack(_lib.LATENT_UP_B, ctypes.byref(src), ctypes.byref(dst), 5, 1, s) == \
        _lib.LATENT_E_UNSUPPORTED
    dst.scales = f.scales.data_ptr()  # codes on one side only for scales
    assert _lib.lib.latent_tiles_repack(_lib.LATENT_GATE_A, ctypes.byref(src), ctypes.byref(dst), 5, 1, s) == \
        _lib.LATENT_E_INVALID


def _operand_tensors(host):
    """The twelve operand tensors of a host layer in the row layout, on the GPU."""
    import torch

    out = {}
    for name in FACTORS:
        f = host.factors[name]
        out[name] = torch.from_numpy(np.ascontiguousarray(f.codes)).cuda()
        out[name + "_s"] = torch.from_numpy(np.ascontiguousarray(f.scales.astype(np.float16))).cuda()
    return out


@pytest.mark.parametrize("T,k,path", [(8, 8, 3), (2, 8, 3), (640, 8, 2)])
def test_ggml_style_binding_reads_only_the_repacked_tensors(gpu, T, k, path):
    """What a ggml-hip binding of the op does: each of the twelve
    tensors is repacked on its own when it is uploaded (codes or scales,
    row layout -> tile layout), the row-layout upload buffers are then
    overwritten, and the op's 15 operands (x, ids, weights, the twelve tile
    tensors) go to latent_moe_ffn_forward with layout = tiles."""
    import torch

    from latent_amd import _lib

    E, D, FF = 16, 512, 768
    host = synth.make_layer(seed=900 + T, n_expert=E, d=D, ff=FF, max_rank=256)
    staged = _operand_tensors(host)
    tiles = {}
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for idx, name in enumerate(FACTORS):
        rows, cols = host.factors[name].codes.shape[1], host.factors[name].codes.shape[2] * 2
        for key, is_codes in ((name, True), (name + "_s", False)):
            out = torch.empty_like(staged[key])
            src = _lib.LatentFactor(codes=staged[key].data_ptr() if is_codes else None,
                                    scales=None if is_codes else staged[key].data_ptr(), rows=rows, cols=cols)
            dst = _lib.LatentFactor(codes=out.data_ptr() if is_codes else None,
                                    scales=None if is_codes else out.data_ptr(), rows=rows, cols=cols)
            _lib.check(_lib.lib.latent_tiles_repack(idx, ctypes.byref(src), ctypes.byref(dst), E, 1, s), "repack")
            tiles[key] = out
    for t in staged.values():  # the upload buffers: garbage from here on
        t.view(torch.uint8).fill_(0xA5)
    rng = np.random.default_rng(T)
    x = rng.standard_normal((T, D)).astype(np.float32)
    ids, w = routing.softmax_topk(rng.standard_normal((T, E)), k)
    xt = torch.from_numpy(x).cuda().to(torch.float16)
    it, wt = torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda().to(torch.float16)
    out = torch.full((T, k, D), float("nan"), dtype=torch.float32, device="cuda")  # the op's per-slot dst
    a = _lib.LatentMoeArgs()
    a.x, a.x_dtype = xt.data_ptr(), _lib.LATENT_F16
    a.ids, a.weights, a.weights_dtype = it.data_ptr(), wt.data_ptr(), _lib.LATENT_F16
    for name in FACTORS:
        f = host.factors[name]
        setattr(a, name, _lib.LatentFactor(codes=tiles[name].data_ptr(), scales=tiles[name + "_s"].data_ptr(),
                                           rows=f.codes.shape[1], cols=f.codes.shape[2] * 2))
    a.n_tokens, a.n_embd, a.n_ff, a.n_expert, a.n_expert_used, a.max_rank = T, D, FF, E, k, 256
    a.out_mode, a.out = _lib.LATENT_OUT_PER_SLOT, out.data_ptr()
    a.layout = _lib.LATENT_LAYOUT_TILES
    assert _lib.lib.latent_moe_path(ctypes.byref(a)) == path
    need = ctypes.c_size_t(0)
    _lib.check(_lib.lib.latent_moe_workspace_size(ctypes.byref(a), ctypes.byref(need)), "workspace size")
    ws = torch.zeros(need.value, dtype=torch.uint8, device="cuda")
    a.workspace, a.workspace_bytes = ws.data_ptr(), need.value
    _lib.check(_lib.lib.latent_moe_ffn_forward(ctypes.byref(a), s), "latent_moe_ffn_forward")
    torch.cuda.synchronize()
    xq = xt.float().cpu().numpy()
    wq = wt.float().cpu().numpy()
    want = ref.moe_forward(xq, ids, wq, host, out_mode=_lib.LATENT_OUT_PER_SLOT)
    err = ref.rel_l2(want, out.cpu().numpy())
    print(f"ggml-style binding T={T} k={k} path={path} rel_l2={err:.3e}")
    assert err <= 2e-3
    # the same operands in the row layout are refused by these paths' reader
    a.layout = 7
    assert _lib.lib.latent_moe_ffn_forward(ctypes.byref(a), s) == _lib.LATENT_E_INVALID


def test_dsv3_layer_is_held_once(gpu):
    """A DeepSeek-V3-shaped layer (256 experts, d 7168, ff 2048, rank 256)
    holds its 1,019,215,872 packed bytes once: the tile layout replaces the
    row layout rather than sitting beside it."""
    import torch

    from latent_amd import synth as gsynth

    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated()
    layer = gsynth.make_layer(seed=3, n_expert=256, d=7168, ff=2048, max_rank=256)
    torch.cuda.synchronize()
    held = torch.cuda.memory_allocated() - base
    assert layer.layout == "tiles"
    assert layer.nbytes() == 1_019_215_872
    print(f"dsv3 layer: {held} bytes allocated, {layer.nbytes()} in its factor tensors")
    assert held < 1_019_215_872 + (32 << 20)  # the rank table and allocator rounding
