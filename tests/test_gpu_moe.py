"""GPU MoE-layer parity against the oracle (loader/latent_runtime.py:48-59 per
routed pair; router-weighted reduce of README.md:111-113).

Bar: rel-L2 <= 2e-3 against the oracle's fp32 result on the same packed
factors and inputs (the decode path computes in fp32 and lands near 1e-6).
"""

import numpy as np
import pytest

from oracle import latent_ref as ref
from oracle import routing, synth
from tests._layers import remap_ids, subset_to_host, to_device

pytestmark = pytest.mark.gpu

TOL = 2e-3


def _run(gpu, layer_dev, x, ids, w, wbd=False, mode=0, x_dtype="f32", w_dtype="f32"):
    import torch

    tdt = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}[x_dtype]
    xt = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).cuda().to(tdt)
    it = torch.from_numpy(np.ascontiguousarray(ids, dtype=np.int32)).cuda()
    wt = torch.from_numpy(np.ascontiguousarray(w, dtype=np.float32)).cuda()
    if w_dtype == "f16":
        wt = wt.to(torch.float16)
    out = gpu.moe_forward(xt, it, wt, layer_dev, weight_before_down=wbd, out_mode=mode)
    torch.cuda.synchronize()
    return out.cpu().numpy(), xt.float().cpu().numpy(), wt.float().cpu().numpy()


# --------------------------------------------------------------------------------
# single expert: the reference's expert-forward entry point
# --------------------------------------------------------------------------------
@pytest.mark.parametrize("wbd", [False, True])
def test_swiglu_expert_config0(gpu, wbd):
    from latent_amd import runtime

    arrays, dense, x = synth.config0_expert(seed=0)
    want = ref.swiglu_expert(x, ref.load_pair(arrays, "gate"), ref.load_pair(arrays, "up"),
                             ref.load_pair(arrays, "down"), weight=0.3, weight_before_down=wbd)
    got = runtime.swiglu_expert(x, runtime.load_pair(arrays, "gate"), runtime.load_pair(arrays, "up"),
                                runtime.load_pair(arrays, "down"), weight=0.3, weight_before_down=wbd)
    assert got.shape == want.shape
    err = ref.rel_l2(want, got)
    print(f"config0 wbd={wbd} rel_l2={err:.3e}")
    assert err <= TOL
    one = runtime.swiglu_expert(x[0], runtime.load_pair(arrays, "gate"), runtime.load_pair(arrays, "up"),
                                runtime.load_pair(arrays, "down"))
    assert one.shape == (512,)


def test_swiglu_expert_int8_factor(gpu):
    from latent_amd import runtime

    arrays, dense, x = synth.config0_expert(seed=1)
    a = ref.load_pair(arrays, "down").a
    q, s, shape = ref.quantize_int8(a, group_size=64)
    arrays = dict(arrays)
    del arrays["down.a.nf4"]
    arrays["down.a.int8"], arrays["down.a.scales"] = q, s
    want = ref.swiglu_expert(x, ref.load_pair(arrays, "gate"), ref.load_pair(arrays, "up"), ref.load_pair(arrays, "down"))
    got = runtime.swiglu_expert(x, runtime.load_pair(arrays, "gate"), runtime.load_pair(arrays, "up"),
                                runtime.load_pair(arrays, "down"))
    assert ref.rel_l2(want, got) <= TOL


def test_missing_factor_raises_keyerror(gpu):
    from latent_amd import runtime

    arrays, _, _ = synth.config0_expert(seed=0, d=64, ff=64, rank=32)
    with pytest.raises(KeyError):
        runtime.load_pair(arrays, "nope")


# --------------------------------------------------------------------------------
# small layers: every mode, dtype and routing edge case
# --------------------------------------------------------------------------------
@pytest.fixture(scope="module")
def small_layer():
    return synth.make_layer(seed=100, n_expert=16, d=256, ff=512, max_rank=64)


@pytest.fixture(scope="module")
def small_dev(gpu, small_layer):
    return to_device(small_layer)


@pytest.mark.parametrize("T", [1, 2, 7, 33, 64, 300])
@pytest.mark.parametrize("mode", [0, 1])
def test_small_layer_modes(gpu, small_layer, small_dev, T, mode):
    rng = np.random.default_rng(T)
    x = rng.standard_normal((T, 256)).astype(np.float32)
    ids, w = routing.softmax_topk(rng.standard_normal((T, 16)), 4)
    got, xq, wq = _run(gpu, small_dev, x, ids, w, mode=mode)
    want = ref.moe_forward(xq, ids, wq, small_layer, out_mode=mode)
    err = ref.rel_l2(want, got)
    print(f"T={T} mode={mode} rel_l2={err:.3e}")
    assert err <= TOL


@pytest.mark.parametrize("x_dtype,w_dtype", [("bf16", "f32"), ("f16", "f16"), ("f32", "f16")])
@pytest.mark.parametrize("wbd", [False, True])
def test_small_layer_dtypes_and_weighting(gpu, small_layer, small_dev, x_dtype, w_dtype, wbd):
    rng = np.random.default_rng(11)
    x = rng.standard_normal((9, 256)).astype(np.float32)
    ids, w = routing.softmax_topk(rng.standard_normal((9, 16)), 4)
    for mode in (0, 1):
        got, xq, wq = _run(gpu, small_dev, x, ids, w, wbd=wbd, mode=mode, x_dtype=x_dtype, w_dtype=w_dtype)
        want = ref.moe_forward(xq, ids, wq, small_layer, weight_before_down=wbd, out_mode=mode)
        assert ref.rel_l2(want, got) <= TOL


def test_dropped_invalid_and_duplicate_slots(gpu, small_layer, small_dev):
    rng = np.random.default_rng(12)
    x = rng.standard_normal((6, 256)).astype(np.float32)
    ids, w = routing.softmax_topk(rng.standard_normal((6, 16)), 4)
    ids[0, :] = -1          # every slot dropped
    ids[1, 1] = 16          # out of range -> dropped
    ids[2, 3] = -7
    ids[3, 2] = ids[3, 0]   # the same expert twice for one token
    for mode in (0, 1):
        got, xq, wq = _run(gpu, small_dev, x, ids, w, mode=mode)
        want = ref.moe_forward(xq, ids, wq, small_layer, out_mode=mode)
        assert ref.rel_l2(want, got) <= TOL
        if mode == 1:
            assert not got[0].any() and not got[1, 1].any() and not got[2, 3].any()
        else:
            assert not got[0].any()


def test_zero_tokens_is_noop(gpu, small_dev):
    import torch

    x = torch.zeros((0, 256), dtype=torch.bfloat16, device="cuda")
    ids = torch.zeros((0, 4), dtype=torch.int32, device="cuda")
    w = torch.zeros((0, 4), dtype=torch.float32, device="cuda")
    out = gpu.moe_forward(x, ids, w, small_dev)
    assert out.shape == (0, 256)


def test_per_slot_sum_equals_reduced(gpu, small_dev):
    rng = np.random.default_rng(13)
    x = rng.standard_normal((40, 256)).astype(np.float32)
    ids, w = routing.softmax_topk(rng.standard_normal((40, 16)), 4)
    per, _, _ = _run(gpu, small_dev, x, ids, w, mode=1)
    red, _, _ = _run(gpu, small_dev, x, ids, w, mode=0)
    assert ref.rel_l2((per.astype(np.float64) * w[..., None]).sum(1), red) < 1e-6


# --------------------------------------------------------------------------------
# heterogeneous ranks + per-group INT8 + adaptive drop (config-3 structure, small)
# --------------------------------------------------------------------------------
def test_hetero_ranks_int8_adaptive_drop(gpu):
    rng = np.random.default_rng(14)
    E, R = 12, 128
    ranks = rng.choice([32, 64, 96, 128], E)
    layer = synth.make_layer(seed=200, n_expert=E, d=256, ff=384, max_rank=R, ranks=ranks, int8_fraction=0.1)
    dev = to_device(layer)
    for T in (3, 40):
        x = rng.standard_normal((T, 256)).astype(np.float32)
        ids, w = routing.softmax_topk(rng.standard_normal((T, E)), 6)
        ids, w = routing.adaptive_drop(ids, w, 0.05)
        for mode in (0, 1):
            got, xq, wq = _run(gpu, dev, x, ids, w, mode=mode, x_dtype="bf16")
            want = ref.moe_forward(xq, ids, wq, layer, out_mode=mode)
            err = ref.rel_l2(want, got)
            print(f"hetero T={T} mode={mode} rel_l2={err:.3e}")
            assert err <= TOL


# --------------------------------------------------------------------------------
# DeepSeek-V3-shaped layer (256 experts, d=7168, ff=2048, r=256, top-8)
# --------------------------------------------------------------------------------
@pytest.fixture(scope="module")
def dsv3(gpu):
    from latent_amd import synth as gsynth

    return gsynth.make_layer(seed=7, n_expert=256, d=7168, ff=2048, max_rank=256)


_ROWS = {}


def _dsv3_rows(dsv3):
    """The DSV3 layer in the row layout (one copy, made on first use)."""
    if id(dsv3) not in _ROWS:
        _ROWS.clear()
        _ROWS[id(dsv3)] = dsv3.to_layout("rows")
    return _ROWS[id(dsv3)]


@pytest.mark.parametrize("path", ["default", "fused", "general"])
@pytest.mark.parametrize("B", [1, 8, 32, 64])
def test_dsv3_decode_parity(gpu, dsv3, B, path, monkeypatch):
    import torch

    from latent_amd import synth as gsynth

    layer = dsv3
    if path != "default":
        # The fp32 paths read the row layout: the same layer reordered back.
        monkeypatch.setenv("LATENT_MOE_PATH", path)
        layer = _dsv3_rows(dsv3)

    ids_t, w_t = gsynth.route(seed=1000 + B, n_tokens=B, n_expert=256, k=8)
    x_t = gsynth.bf16_input(seed=2000 + B, n_tokens=B, d=7168)
    out = gpu.moe_forward(x_t, ids_t, w_t, layer)
    torch.cuda.synchronize()
    # A second call must reproduce the first: bit for bit on the persistent
    # decode kernel (fixed summation order, control block left as found) and
    # the streaming path (fixed-order reductions); the multi-kernel path
    # accumulates with float atomics, so only to rounding.
    again = gpu.moe_forward(x_t, ids_t, w_t, layer)
    torch.cuda.synchronize()
    from latent_amd.moe import moe_path, workspace_error

    used = moe_path(layer, x_t, 8)
    if path == "fused":
        assert used == ("fused" if B >= 4 else "general")  # below 32 pairs the row layout's default
    else:
        assert used == ("stream" if path == "default" else "general")
    if used in ("fused", "stream"):
        assert torch.equal(out, again)
    else:
        assert torch.allclose(out, again, rtol=1e-5, atol=1e-6 * out.abs().max().item())

    assert workspace_error(layer.workspace(B, 8)) == 0
    ids, w, x = ids_t.cpu().numpy(), w_t.cpu().numpy(), x_t.float().cpu().numpy()
    experts, local = remap_ids(ids, 256)
    host = subset_to_host(dsv3, experts)
    want = ref.moe_forward(x, local, w, host)
    err = ref.rel_l2(want, out.cpu().numpy())
    print(f"dsv3 decode B={B} path={used} experts={experts.size} rel_l2={err:.3e}")
    assert err <= TOL


# --------------------------------------------------------------------------------
# prefill: grouped fp16 MFMA path (>= 16 routed pairs per active expert)
# --------------------------------------------------------------------------------
@pytest.fixture(scope="module")
def prefill_layer():
    return synth.make_layer(seed=300, n_expert=32, d=1024, ff=512, max_rank=128)


@pytest.fixture(scope="module")
def prefill_dev(gpu, prefill_layer):
    return to_device(prefill_layer)


@pytest.mark.parametrize("x_dtype,wbd", [("bf16", False), ("f32", True), ("f16", False)])
@pytest.mark.parametrize("mode", [0, 1])
def test_prefill_mfma_parity(gpu, prefill_layer, prefill_dev, x_dtype, wbd, mode):
    import torch

    T, E, K = 256, 32, 4
    rng = np.random.default_rng(31)
    x = rng.standard_normal((T, 1024)).astype(np.float32)
    logits = routing.zipf_logits(rng, T, E, gamma=0.5)
    ids, w = routing.softmax_topk(logits, K)
    xt = torch.from_numpy(x).cuda().to({"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}[x_dtype])
    assert gpu.moe_path(prefill_dev, xt, K) == "prefill"
    got, xq, wq = _run(gpu, prefill_dev, x, ids, w, wbd=wbd, mode=mode, x_dtype=x_dtype)
    want = ref.moe_forward(xq, ids, wq, prefill_layer, weight_before_down=wbd, out_mode=mode)
    err = ref.rel_l2(want, got)
    print(f"prefill x={x_dtype} wbd={wbd} mode={mode} rel_l2={err:.3e}")
    assert err <= TOL
    if mode == 1:
        assert not got[ids < 0].any()


def test_prefill_mfma_ragged_tiles(gpu, prefill_layer, prefill_dev):
    # Expert counts that are not multiples of the 128-pair tile, an expert with
    # exactly one tile, dropped slots and an unrouted expert.
    T, E, K = 300, 32, 4
    rng = np.random.default_rng(32)
    x = rng.standard_normal((T, 1024)).astype(np.float32)
    ids, w = routing.softmax_topk(rng.standard_normal((T, E)), K)
    ids[ids == 5] = -1
    ids[:128, 0] = 7
    got, xq, wq = _run(gpu, prefill_dev, x, ids, w, mode=0, x_dtype="bf16")
    want = ref.moe_forward(xq, ids, wq, prefill_layer, out_mode=0)
    assert ref.rel_l2(want, got) <= TOL
