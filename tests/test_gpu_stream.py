"""Streaming MFMA decode path (stream.hip) against the oracle.

The path is selected with LATENT_MOE_PATH=stream for every call here, in both
launch styles (LATENT_STREAM_LAUNCH=auto: the default, which takes the
small-batch chain for at most 32 routed pairs; =phases: one launch per phase).
Bar:
rel-L2 <= 2e-3 against the oracle's fp32 result on the same packed factors
(fp16 operands, fp32 accumulation), bit-identical results on a repeated call.
"""

import numpy as np
import pytest

from oracle import latent_ref as ref
from oracle import routing, synth
from tests._layers import remap_ids, subset_to_host, to_device

pytestmark = pytest.mark.gpu

TOL = 2e-3


@pytest.fixture(params=["auto", "phases"])
def stream_path(monkeypatch, request):
    # The default launch style (the small-batch chain up to 32 routed pairs,
    # per-phase launches above) and per-phase launches throughout.
    monkeypatch.setenv("LATENT_MOE_PATH", "stream")
    monkeypatch.setenv("LATENT_STREAM_LAUNCH", request.param)


@pytest.fixture(scope="module")
def small_layer():
    # Rank 256 with d and ff multiples of 512: the shapes the streaming path takes.
    return synth.make_layer(seed=410, n_expert=12, d=1024, ff=1024, max_rank=256)


@pytest.fixture(scope="module")
def small_dev(gpu, small_layer):
    return to_device(small_layer)


def _run(gpu, dev, x, ids, w, x_dtype="bf16", wbd=False, mode=0):
    import torch

    tdt = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}[x_dtype]
    xt = torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda().to(tdt)
    it = torch.from_numpy(np.ascontiguousarray(ids, np.int32)).cuda()
    wt = torch.from_numpy(np.ascontiguousarray(w, np.float32)).cuda()
    assert gpu.moe_path(dev, xt, ids.shape[1]) == "stream"
    out = gpu.moe_forward(xt, it, wt, dev, weight_before_down=wbd, out_mode=mode)
    again = gpu.moe_forward(xt, it, wt, dev, weight_before_down=wbd, out_mode=mode)
    torch.cuda.synchronize()
    assert torch.equal(out, again), "repeated call is not bit-identical"
    return out.cpu().numpy(), xt.float().cpu().numpy()


@pytest.mark.parametrize("T,k", [(1, 1), (1, 8), (3, 4), (8, 8), (40, 6)])
@pytest.mark.parametrize("mode", [0, 1])
def test_stream_small_layer(gpu, stream_path, small_layer, small_dev, T, k, mode):
    rng = np.random.default_rng(T * 10 + k)
    x = rng.standard_normal((T, 1024)).astype(np.float32)
    ids, w = routing.softmax_topk(rng.standard_normal((T, 12)), k)
    got, xq = _run(gpu, small_dev, x, ids, w, mode=mode)
    want = ref.moe_forward(xq, ids, w, small_layer, out_mode=mode)
    err = ref.rel_l2(want, got)
    print(f"stream T={T} k={k} mode={mode} rel_l2={err:.3e}")
    assert err <= TOL


@pytest.mark.parametrize("x_dtype,wbd", [("f32", True), ("f16", False), ("bf16", True)])
def test_stream_dtypes_and_weighting(gpu, stream_path, small_layer, small_dev, x_dtype, wbd):
    rng = np.random.default_rng(77)
    x = (rng.standard_normal((9, 1024)) * 3.0).astype(np.float32)
    ids, w = routing.softmax_topk(rng.standard_normal((9, 12)), 3)
    for mode in (0, 1):
        got, xq = _run(gpu, small_dev, x, ids, w, x_dtype=x_dtype, wbd=wbd, mode=mode)
        want = ref.moe_forward(xq, ids, w, small_layer, weight_before_down=wbd, out_mode=mode)
        assert ref.rel_l2(want, got) <= TOL


def test_stream_units_dropped_duplicate_and_invalid(gpu, stream_path, small_layer, small_dev):
    # 40 tokens all routed to expert 3 (three units of 16, 16 and 8 pairs),
    # dropped slots, an id beyond E, and a duplicated expert within a token.
    rng = np.random.default_rng(5)
    T = 40
    x = rng.standard_normal((T, 1024)).astype(np.float32)
    ids, w = routing.softmax_topk(rng.standard_normal((T, 12)), 4)
    ids[:, 0] = 3
    ids[0, 1] = -1
    ids[1, 2] = 99
    ids[2, 3] = ids[2, 1]
    for mode in (0, 1):
        got, xq = _run(gpu, small_dev, x, ids, w, mode=mode)
        want = ref.moe_forward(xq, np.where(ids >= 12, -1, ids), w, small_layer, out_mode=mode)
        assert ref.rel_l2(want, got) <= TOL
        if mode == 1:
            assert not got[0, 1].any() and not got[1, 2].any()


def test_stream_all_dropped(gpu, stream_path, small_dev):
    import torch

    ids = -np.ones((4, 2), np.int32)
    w = np.zeros((4, 2), np.float32)
    got, _ = _run(gpu, small_dev, np.ones((4, 1024), np.float32), ids, w)
    assert not got.any()
    torch.cuda.synchronize()


@pytest.fixture(scope="module")
def dsv3(gpu):
    from latent_amd import synth as gsynth

    return gsynth.make_layer(seed=7, n_expert=256, d=7168, ff=2048, max_rank=256)


@pytest.mark.parametrize("B", [1, 8, 32, 64, 128])
def test_stream_dsv3_decode(gpu, stream_path, dsv3, B):
    import torch

    from latent_amd import synth as gsynth

    ids_t, w_t = gsynth.route(seed=1000 + B, n_tokens=B, n_expert=256, k=8)
    x_t = gsynth.bf16_input(seed=2000 + B, n_tokens=B, d=7168)
    assert gpu.moe_path(dsv3, x_t, 8) == "stream"
    out = gpu.moe_forward(x_t, ids_t, w_t, dsv3)
    again = gpu.moe_forward(x_t, ids_t, w_t, dsv3)
    torch.cuda.synchronize()
    assert torch.equal(out, again)
    ids, w, x = ids_t.cpu().numpy(), w_t.cpu().numpy(), x_t.float().cpu().numpy()
    experts, local = remap_ids(ids, 256)
    if B > 64:  # keep the oracle to a few seconds: check the first 16 tokens
        sel = np.unique(local[:16][local[:16] >= 0])
        experts, ids16 = experts[sel], local[:16]
        lut = -np.ones(256, np.int64)
        lut[sel] = np.arange(sel.size)
        local = np.where(ids16 >= 0, lut[np.clip(ids16, 0, 255)], -1).astype(np.int32)
        x, w, out = x[:16], w[:16], out[:16]
    host = subset_to_host(dsv3, experts)
    want = ref.moe_forward(x, local, w, host)
    err = ref.rel_l2(want, out.cpu().numpy())
    print(f"stream dsv3 B={B} experts={experts.size} rel_l2={err:.3e}")
    assert err <= TOL


@pytest.mark.parametrize("path", ["general", "fused"])
def test_reference_rank_table_at_max_rank_256(gpu, tmp_path, monkeypatch, path):
    """A file whose rank table the reference wrote (uint8 as I8, a rank of 256
    stored as 0) beside factors padded to 256 is read without the table, and
    the fp32 paths that honour ranks then match the oracle at max_rank."""
    import torch

    from latent_amd import StackedLayer, gguf

    layer = synth.make_layer(seed=21, n_expert=4, d=256, ff=256, max_rank=256)
    arrays = {}
    for name in ref.FACTOR_NAMES:
        arrays[name] = layer.factors[name].codes
        arrays[name + "_s"] = layer.factors[name].scales.astype(np.float16)
    p = tmp_path / "refranks256.gguf"
    gguf.write_latent_gguf(p, {0: arrays}, max_rank=256)
    g = gguf.read_latent_gguf(p)
    name = "blk.0.ffn_latent_ranks"
    per_expert = np.array([[256, 256, 256], [128, 256, 64], [256, 32, 256], [256, 256, 256]])
    g.tensors[name] = gguf.TensorInfo(name, (4, 3), gguf.GGML_I8, 0)
    g.arrays[name] = np.frombuffer(per_expert.T.astype(np.uint8).tobytes(), np.int8).reshape(4, 3)
    dev = StackedLayer.from_arrays(g.layer_arrays(0), layer=0, layout="rows")
    assert dev.ranks is None
    monkeypatch.setenv("LATENT_MOE_PATH", path)
    rng = np.random.default_rng(5)
    T = 40 if path == "fused" else 5  # the persistent kernel takes 32..512 routed pairs
    x = rng.standard_normal((T, 256)).astype(np.float32)
    ids, w = routing.softmax_topk(rng.standard_normal((T, 4)), 2)
    xt = torch.from_numpy(x).cuda()
    assert gpu.moe_path(dev, xt, 2) == path
    out = gpu.moe_forward(xt, torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda(), dev)
    want = ref.moe_forward(x, ids, w, layer)
    err = ref.rel_l2(want, out.cpu().numpy())
    print(f"reference rank table, path {path}: rel_l2={err:.3e}")
    assert err <= 1e-5


def test_gguf_round_trip_layer_gives_identical_outputs(gpu, small_dev, tmp_path):
    """A device layer written to GGUF and read back computes bit-identical outputs."""
    import torch

    from latent_amd import StackedLayer, gguf

    path = tmp_path / "layer.gguf"
    gguf.write_latent_gguf(path, {5: gguf.layer_to_arrays(small_dev)}, max_rank=256)
    back = StackedLayer.from_arrays(gguf.read_latent_gguf(path).layer_arrays(5), layer=5)
    rng = np.random.default_rng(8)
    x = torch.from_numpy(rng.standard_normal((6, 1024)).astype(np.float32)).cuda().to(torch.bfloat16)
    ids, w = routing.softmax_topk(rng.standard_normal((6, 12)), 6)
    it, wt = torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda()
    a = gpu.moe_forward(x, it, wt, small_dev)
    b = gpu.moe_forward(x, it, wt, back)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
