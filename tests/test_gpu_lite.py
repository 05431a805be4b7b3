"""Small-batch chain (lite_kernel, at most 32 routed pairs) against the oracle.

With LATENT_STREAM_LAUNCH unset, a layer with a tile layout takes this chain
for calls of at most 32 routed pairs; the grouping, the x conversion and the
combine all run inside its one launch.  Bar: rel-L2 <= 2e-3 against the
oracle's fp32 result on the same packed factors, bit-identical results on a
repeated call, exact zeros where no routed slot contributes, and the
workspace's counters left zero (checked by calls in a row with different
routings, other launch styles in between, and the error word).
"""

import numpy as np
import pytest

from oracle import latent_ref as ref
from oracle import routing, synth
from tests._layers import remap_ids, subset_to_host, to_device

pytestmark = pytest.mark.gpu

TOL = 2e-3
E, D, FF = 12, 1024, 1024


@pytest.fixture(autouse=True)
def default_launch(monkeypatch):
    monkeypatch.delenv("LATENT_STREAM_LAUNCH", raising=False)
    monkeypatch.delenv("LATENT_MOE_PATH", raising=False)


@pytest.fixture(scope="module")
def layer():
    return synth.make_layer(seed=610, n_expert=E, d=D, ff=FF, max_rank=256)


@pytest.fixture(scope="module")
def dev(gpu, layer):
    d = to_device(layer)
    assert d.layout == "tiles"
    return d


def _call(gpu, dev, x, ids, w, x_dtype="bf16", wbd=False, mode=0, ws=None, launch="lite"):
    import torch

    tdt = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}[x_dtype]
    xt = torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda().to(tdt)
    it = torch.from_numpy(np.ascontiguousarray(ids, np.int32)).cuda()
    wt = torch.from_numpy(np.ascontiguousarray(w, np.float32)).cuda()
    from latent_amd.moe import stream_launch

    assert gpu.moe_path(dev, xt, ids.shape[1]) == "stream"
    if launch is not None:
        assert stream_launch(dev, xt, ids.shape[1]) == launch
    out = gpu.moe_forward(xt, it, wt, dev, weight_before_down=wbd, out_mode=mode, workspace=ws)
    return out, xt.float().cpu().numpy()


def _check(gpu, layer, dev, x, ids, w, **kw):
    import torch

    out, xq = _call(gpu, dev, x, ids, w, **kw)
    again, _ = _call(gpu, dev, x, ids, w, **kw)
    torch.cuda.synchronize()
    assert torch.equal(out, again), "repeated call is not bit-identical"
    got = out.cpu().numpy()
    mode = kw.get("mode", 0)
    want = ref.moe_forward(xq, np.where(ids >= E, -1, ids), w, layer,
                           weight_before_down=kw.get("wbd", False), out_mode=mode)
    err = ref.rel_l2(want, got)
    print(f"lite T={ids.shape[0]} k={ids.shape[1]} mode={mode} rel_l2={err:.3e}")
    assert err <= TOL
    return got


@pytest.mark.parametrize("T,k", [(1, 1), (1, 8), (2, 8), (4, 4), (16, 1), (4, 8), (32, 1)])
@pytest.mark.parametrize("mode", [0, 1])
def test_lite_shapes(gpu, layer, dev, T, k, mode):
    rng = np.random.default_rng(100 * T + k)
    x = rng.standard_normal((T, D)).astype(np.float32)
    ids, w = routing.softmax_topk(rng.standard_normal((T, E)), k)
    _check(gpu, layer, dev, x, ids, w, mode=mode)


@pytest.mark.parametrize("x_dtype,wbd", [("f32", True), ("f16", False), ("bf16", True)])
def test_lite_dtypes_and_weighting(gpu, layer, dev, x_dtype, wbd):
    rng = np.random.default_rng(7)
    # Rows of very different magnitude: each 256-column slice takes its own exponent.
    x = (rng.standard_normal((2, D)) * np.array([[1e-3], [40.0]])).astype(np.float32)
    x[1, 256:512] *= 1e-4
    ids, w = routing.softmax_topk(rng.standard_normal((2, E)), 6)
    for mode in (0, 1):
        _check(gpu, layer, dev, x, ids, w, x_dtype=x_dtype, wbd=wbd, mode=mode)


def test_lite_dropped_duplicate_invalid(gpu, layer, dev):
    # One expert taking 8 pairs (a unit of 8 rows), a duplicate expert within a
    # token, dropped and out-of-range slots, and a token with every slot dropped.
    rng = np.random.default_rng(11)
    T, k = 4, 4
    x = rng.standard_normal((T, D)).astype(np.float32)
    ids, w = routing.softmax_topk(rng.standard_normal((T, E)), k)
    ids[:, 0] = 5
    ids[0, 1] = 5
    ids[1, 2] = -1
    ids[2, 3] = E + 3
    ids[3, :] = -1
    for mode in (0, 1):
        got = _check(gpu, layer, dev, x, ids, w, mode=mode)
        if mode == 1:
            assert not got[1, 2].any() and not got[2, 3].any() and not got[3].any()
        else:
            assert not got[3].any()


def test_lite_expert_beyond_16_pairs(gpu, layer, dev):
    # 18 of 24 single-slot tokens route to expert 5: its pairs fill a 16-row
    # unit and start a second unit of 2 rows.
    rng = np.random.default_rng(13)
    T, k = 24, 1
    x = rng.standard_normal((T, D)).astype(np.float32)
    ids, w = routing.softmax_topk(rng.standard_normal((T, E)), k)
    ids[:18, 0] = 5
    for mode in (0, 1):
        _check(gpu, layer, dev, x, ids, w, mode=mode)


def test_lite_all_dropped(gpu, dev):
    import torch

    ids = -np.ones((3, 4), np.int32)
    w = np.zeros((3, 4), np.float32)
    for mode in (0, 1):
        out, _ = _call(gpu, dev, np.ones((3, D), np.float32), ids, w, mode=mode)
        torch.cuda.synchronize()
        assert not out.cpu().numpy().any()


def test_lite_counters_reset_across_calls_and_launch_styles(gpu, layer, dev, monkeypatch):
    """Calls in a row on one workspace, with different routings and unit
    counts, per-phase calls in between: every result matches
    the oracle and the first call's result comes back bit-identical."""
    import torch

    rng = np.random.default_rng(21)
    ws = dev.workspace(16, 8)
    cases = []
    for T, k in [(1, 8), (2, 4), (1, 2), (2, 8)]:
        x = rng.standard_normal((T, D)).astype(np.float32)
        ids, w = routing.softmax_topk(rng.standard_normal((T, E)), k)
        cases.append((x, ids, w))
    first = None
    for rep in range(3):
        for j, (x, ids, w) in enumerate(cases):
            launch = "lite"
            if rep == 1:
                launch = "phases"
                monkeypatch.setenv("LATENT_STREAM_LAUNCH", launch)
            else:
                monkeypatch.delenv("LATENT_STREAM_LAUNCH", raising=False)
            out, xq = _call(gpu, dev, x, ids, w, ws=ws, launch=launch)
            torch.cuda.synchronize()
            want = ref.moe_forward(xq, ids, w, layer)
            assert ref.rel_l2(want, out.cpu().numpy()) <= TOL, (rep, j)
            if rep == 0 and j == 0:
                first = out.clone()
            if rep == 2 and j == 0:
                assert torch.equal(first, out)
    from latent_amd.moe import workspace_error

    assert workspace_error(ws) == 0


def test_lite_dsv3_shape(gpu):
    import torch

    from latent_amd import synth as gsynth
    from latent_amd.moe import stream_launch

    layer = gsynth.make_layer(seed=9, n_expert=256, d=7168, ff=2048, max_rank=256)
    # Up to 11 units the chain's 512 workgroups are all resident; two to four
    # tokens at top-8 (up to 32 units) take a larger grid whose roles follow
    # the workgroups' start order.
    for B, k in [(1, 8), (1, 11), (2, 8), (1, 16), (3, 8), (4, 8)]:
        ids_t, w_t = gsynth.route(seed=300 + B, n_tokens=B, n_expert=256, k=k)
        x_t = gsynth.bf16_input(seed=400 + B, n_tokens=B, d=7168)
        assert stream_launch(layer, x_t, k) == "lite"
        out = gpu.moe_forward(x_t, ids_t, w_t, layer, check_timeout=True)
        again = gpu.moe_forward(x_t, ids_t, w_t, layer, check_timeout=True)
        torch.cuda.synchronize()
        assert torch.equal(out, again)
        ids, w, x = ids_t.cpu().numpy(), w_t.cpu().numpy(), x_t.float().cpu().numpy()
        experts, local = remap_ids(ids, 256)
        want = ref.moe_forward(x, local, w, subset_to_host(layer, experts))
        err = ref.rel_l2(want, out.cpu().numpy())
        print(f"lite dsv3 B={B} experts={experts.size} rel_l2={err:.3e}")
        assert err <= TOL


def test_check_after_timeout_rezeros_control_block(gpu, layer, dev):
    """A timed-out chain leaves the error word set and may leave a counter
    non-zero.  Both are seeded here from the host (no kernel is made to time
    out): latent_moe_check reports LATENT_E_TIMEOUT, leaves the whole control
    block zero, and the next call on that workspace matches the oracle."""
    import torch

    from latent_amd import _lib

    rng = np.random.default_rng(77)
    x = rng.standard_normal((1, D)).astype(np.float32)
    ids, w = routing.softmax_topk(rng.standard_normal((1, E)), 8)
    ws = torch.zeros(gpu.workspace_size(dev, 1, 8), dtype=torch.uint8, device="cuda")
    ctrl = _lib.LATENT_NOALLOC_CONTROL_BYTES
    ws[36:40] = torch.tensor([1, 0, 0, 0], dtype=torch.uint8)  # the error word
    ws[192 * 1024 + 4] = 3                                     # a small-batch chain counter
    ws[4096] = 9                                               # a persistent-kernel ticket
    assert gpu.workspace_error(ws) == _lib.LATENT_E_TIMEOUT
    assert int(ws[:ctrl].count_nonzero()) == 0
    assert gpu.workspace_error(ws) == _lib.LATENT_OK
    got, xq = _call(gpu, dev, x, ids, w, ws=ws)
    torch.cuda.synchronize()
    assert int(ws[:ctrl].count_nonzero()) == 0
    err = ref.rel_l2(ref.moe_forward(xq, ids, w, layer), got.cpu().numpy())
    assert err <= TOL


def test_check_noalloc_array(gpu):
    """latent_moe_check with a NULL workspace reads the calling device's
    noalloc array: no call has timed out, so it reports LATENT_OK."""
    import ctypes

    import torch

    from latent_amd import _lib

    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert _lib.lib.latent_moe_check(None, 0, s) == _lib.LATENT_OK
