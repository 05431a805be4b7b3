"""latent_moe_ffn_forward_noalloc against latent_moe_ffn_forward, through the C ABI.

The allocation-free entry point takes its scratch from the library's own
per-GPU array; its output must equal the workspace entry point's on the same
inputs (bit for bit on the paths that sum in a fixed order, to rounding on the
multi-kernel path, which adds workgroup partials with float atomics), on two
calls in a row, the second with a smaller input.
"""

import ctypes

import numpy as np
import pytest

from oracle import latent_ref as ref
from oracle import routing, synth
from tests._layers import to_device

pytestmark = pytest.mark.gpu


def _args(layer, x, ids, w, out):
    from latent_amd import _lib
    from latent_amd.moe import _DTYPE_CODE

    a = layer.args()
    a.x, a.x_dtype = x.data_ptr(), _DTYPE_CODE[x.dtype]
    a.ids, a.weights, a.weights_dtype = ids.data_ptr(), w.data_ptr(), _lib.LATENT_F32
    a.n_tokens, a.n_expert_used = ids.shape[0], ids.shape[1]
    a.out_mode = _lib.LATENT_OUT_REDUCED if out.dim() == 2 else _lib.LATENT_OUT_PER_SLOT
    a.out = out.data_ptr()
    return a


def _noalloc(layer, x, ids, w, mode=0):
    import torch

    from latent_amd import _lib

    shape = (x.shape[0], layer.d) if mode == 0 else (x.shape[0], ids.shape[1], layer.d)
    out = torch.full(shape, float("nan"), dtype=torch.float32, device="cuda")
    a = _args(layer, x, ids, w, out)
    a.workspace, a.workspace_bytes = None, 0
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    st = _lib.lib.latent_moe_ffn_forward_noalloc(ctypes.byref(a), s)
    _lib.check(st, "latent_moe_ffn_forward_noalloc")
    return out


def _with_workspace(gpu, layer, x, ids, w, mode=0):
    return gpu.moe_forward(x, ids, w, layer, out_mode=mode)


def _compare(gpu, layer, T, k, seed, mode, exact):
    import torch

    from latent_amd import synth as gsynth

    ids, w = gsynth.route(seed=seed, n_tokens=T, n_expert=layer.n_expert, k=k)
    x = gsynth.bf16_input(seed=seed + 1, n_tokens=T, d=layer.d)
    got = _noalloc(layer, x, ids, w, mode)
    want = _with_workspace(gpu, layer, x, ids, w, mode)
    torch.cuda.synchronize()
    assert not torch.isnan(got).any()
    if exact:
        assert torch.equal(got, want), f"T={T} mode={mode}: differs from latent_moe_ffn_forward"
    else:
        assert ref.rel_l2(want.cpu().numpy(), got.cpu().numpy()) <= 1e-5


def test_noalloc_matches_workspace_entry_dsv3(gpu):
    from latent_amd import synth as gsynth
    from latent_amd.moe import moe_path

    layer = gsynth.make_layer(seed=7, n_expert=256, d=7168, ff=2048, max_rank=256)
    # calls in a row, each with a smaller input (streaming path, fixed-order
    # sums); batch 64 needs about 48 MiB of the 64 MiB array
    for T in (64, 16, 3):
        x = gsynth.bf16_input(seed=1, n_tokens=T, d=7168)
        assert moe_path(layer, x, 8) == "stream"
        for mode in (0, 1):
            _compare(gpu, layer, T, 8, seed=100 + T, mode=mode, exact=True)


def test_noalloc_small_layer_paths(gpu, monkeypatch):
    host = synth.make_layer(seed=100, n_expert=16, d=256, ff=512, max_rank=64)
    layer = to_device(host)
    # persistent kernel (32+ pairs, fixed order) then the multi-kernel path (atomics)
    for T, exact in ((40, True), (5, False)):
        _compare(gpu, layer, T, 4, seed=200 + T, mode=0, exact=exact)


def test_noalloc_rejects_calls_beyond_its_scratch(gpu):
    import torch

    from latent_amd import _lib
    from latent_amd import synth as gsynth

    layer = gsynth.make_layer(seed=8, n_expert=64, d=1024, ff=512, max_rank=128)
    T = 4096
    ids, w = gsynth.route(seed=5, n_tokens=T, n_expert=64, k=8)
    x = gsynth.bf16_input(seed=6, n_tokens=T, d=1024)
    assert gpu.workspace_size(layer, T, 8) > _lib.LATENT_NOALLOC_SCRATCH_BYTES
    out = torch.empty((T, 1024), dtype=torch.float32, device="cuda")
    a = _args(layer, x, ids, w, out)
    st = _lib.lib.latent_moe_ffn_forward_noalloc(ctypes.byref(a), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert st == _lib.LATENT_E_WORKSPACE
    # and a routing check against the oracle on a call that fits
    rng = np.random.default_rng(4)
    hl = synth.make_layer(seed=9, n_expert=8, d=256, ff=256, max_rank=64)
    dl = to_device(hl)
    xs = rng.standard_normal((6, 256)).astype(np.float32)
    i2, w2 = routing.softmax_topk(rng.standard_normal((6, 8)), 2)
    xt = torch.from_numpy(xs).cuda()
    got = _noalloc(dl, xt, torch.from_numpy(i2).cuda(), torch.from_numpy(w2).cuda())
    torch.cuda.synchronize()
    assert ref.rel_l2(ref.moe_forward(xs, i2, w2, hl), got.cpu().numpy()) <= 2e-3


def test_noalloc_small_batch_chain_calls_in_a_row(gpu):
    """Batch 1 at top-8 takes the small-batch chain, whose counters live in the
    noalloc array's control block: several calls in a row with different
    routings (and a per-slot call between) equal the workspace entry bit for bit."""
    import torch

    from latent_amd import synth as gsynth
    from latent_amd.moe import stream_launch

    layer = gsynth.make_layer(seed=17, n_expert=64, d=1024, ff=1024, max_rank=256)
    x = gsynth.bf16_input(seed=3, n_tokens=1, d=1024)
    assert stream_launch(layer, x, 8) == "lite"
    for seed, mode in ((31, 0), (32, 0), (33, 1), (34, 0)):
        _compare(gpu, layer, 1, 8, seed=seed, mode=mode, exact=True)
    torch.cuda.synchronize()


def test_noalloc_graph_capture_replays(gpu):
    """A noalloc call captured in a HIP graph (torch.cuda.CUDAGraph) and
    replayed several times, with eager work and synchronisations between the
    replays, gives the eager result on every replay."""
    import torch

    from latent_amd import synth as gsynth

    layer = gsynth.make_layer(seed=18, n_expert=64, d=1024, ff=1024, max_rank=256)
    T, k = 2, 8
    ids, w = gsynth.route(seed=41, n_tokens=T, n_expert=64, k=k)
    x = gsynth.bf16_input(seed=42, n_tokens=T, d=1024)
    eager = _noalloc(layer, x, ids, w)  # first call on the device: sets up the array outside the capture
    torch.cuda.synchronize()
    out = torch.zeros((T, 1024), dtype=torch.float32, device="cuda")
    a = _args(layer, x, ids, w, out)
    a.workspace, a.workspace_bytes = None, 0
    from latent_amd import _lib

    g = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(cap):
        with torch.cuda.graph(g, stream=cap):
            st = _lib.lib.latent_moe_ffn_forward_noalloc(ctypes.byref(a), ctypes.c_void_p(cap.cuda_stream))
    torch.cuda.current_stream().wait_stream(cap)
    _lib.check(st, "latent_moe_ffn_forward_noalloc (captured)")
    for i in range(3):
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i} differs from the eager call"
        # eager work on the same array between the replays
        other = _noalloc(layer, gsynth.bf16_input(seed=50 + i, n_tokens=1, d=1024), ids[:1], w[:1])
        torch.cuda.synchronize()
        assert not torch.isnan(other).any()


_FIRST_CALL = r'''
import ctypes, sys
sys.path.insert(0, sys.argv[1])
import torch
from latent_amd import _lib
from oracle import synth
from tests._layers import to_device
from tests.test_zz_no_alloc import _args

layer = to_device(synth.make_layer(seed=101, n_expert=16, d=256, ff=512, max_rank=64))
from latent_amd import synth as gsynth
ids, w = gsynth.route(seed=7, n_tokens=40, n_expert=16, k=4)
x = gsynth.bf16_input(seed=8, n_tokens=40, d=256)
import latent_amd
want = latent_amd.moe_forward(x, ids, w, layer)
out = torch.full((40, 256), float("nan"), dtype=torch.float32, device="cuda")
a = _args(layer, x, ids, w, out)
a.workspace, a.workspace_bytes = None, 0
torch.cuda.synchronize()
hip = ctypes.CDLL("libamdhip64.so")
assert hip.hipSetDevice(ctypes.c_int(4096)) != 0  # an unrelated failed call, its error left pending
st = _lib.lib.latent_moe_ffn_forward_noalloc(ctypes.byref(a), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
assert st == _lib.LATENT_OK, _lib.status_string(st)
torch.cuda.synchronize()
assert torch.equal(out, want)
print("first call ok")
'''


def test_noalloc_first_call_after_an_unrelated_hip_error(gpu, tmp_path):
    """The first allocation-free call of a process sets up the device's
    scratch array; a HIP error that earlier, unrelated code left pending must
    not fail it (checked in a fresh process, where that call is the first)."""
    import subprocess
    import sys
    from pathlib import Path

    script = tmp_path / "first_call.py"
    script.write_text(_FIRST_CALL)
    root = str(Path(__file__).resolve().parents[1])
    r = subprocess.run([sys.executable, str(script), root], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0 and "first call ok" in r.stdout, r.stdout + r.stderr
