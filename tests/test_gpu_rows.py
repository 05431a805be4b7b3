"""Row-layout MFMA phases (rows.hip, latent_moe_path 4) against the oracle.

LATENT_MOE_PATH=rows selects them for every call here.  Layers in the row
layout: uniform rank 256 pure NF4; heterogeneous per-expert ranks (multiples
of 32 and not, so chunks of 1 to 16 groups and partial groups) with 10 % INT8
groups; the config-0 expert shape (d 512, ff 1408: partial 256-column items
of ff, one 512-column item of d).  Batches from one token to experts with
more than 16 pairs (several passes), both output modes, weighting before
down, f32 / f16 / bf16 x, dropped and out-of-range slots.  Bar: rel-L2 <= 2e-3
against the oracle's fp32 result on the same packed factors (fp16 operands,
fp32 accumulation).
"""

import numpy as np
import pytest

from oracle import latent_ref as ref
from oracle import routing, synth

pytestmark = pytest.mark.gpu

TOL = 2e-3

LAYERS = {
    "uniform": dict(seed=71, n_expert=12, d=1024, ff=1024, max_rank=256),
    "hetero": dict(seed=72, n_expert=12, d=1024, ff=1536, max_rank=512,
                   ranks=[64, 128, 256, 512, 96, 320, 100, 512, 128, 256, 32, 448], int8_fraction=0.1),
    "config0": dict(seed=73, n_expert=4, d=512, ff=1408, max_rank=64),
}


def _rows_layer(layer):
    import torch

    from latent_amd import DeviceFactor, StackedLayer

    facs = {}
    for name in ref.FACTOR_NAMES:
        f = layer.factors[name]
        ext = None if f.int8 is None else (f.int8.bitmap, f.int8.row_offset, f.int8.data)
        facs[name] = DeviceFactor.from_numpy(f.codes, f.scales, ext)
    ranks = None if layer.ranks is None else torch.from_numpy(layer.ranks.astype(np.int32)).cuda()
    return StackedLayer(**facs, ranks=ranks, layout="rows")


@pytest.fixture(autouse=True)
def rows_path(monkeypatch):
    monkeypatch.setenv("LATENT_MOE_PATH", "rows")


@pytest.fixture(scope="module", params=sorted(LAYERS))
def layers(request, gpu):
    host = synth.make_layer(**LAYERS[request.param])
    return request.param, host, _rows_layer(host)


def _run(gpu, host, dev, x, ids, w, x_dtype="bf16", wbd=False, mode=0):
    import torch

    tdt = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}[x_dtype]
    xt = torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda().to(tdt)
    it = torch.from_numpy(np.ascontiguousarray(ids, np.int32)).cuda()
    wt = torch.from_numpy(np.ascontiguousarray(w, np.float32)).cuda()
    assert gpu.moe_path(dev, xt, ids.shape[1]) == "rows"
    out = gpu.moe_forward(xt, it, wt, dev, weight_before_down=wbd, out_mode=mode, check_timeout=True)
    torch.cuda.synchronize()
    E = host.n_expert
    want = ref.moe_forward(xt.float().cpu().numpy(), np.where(ids >= E, -1, ids), w, host,
                           weight_before_down=wbd, out_mode=mode)
    got = out.cpu().numpy()
    return got, want


@pytest.mark.parametrize("T,k", [(1, 8), (4, 4), (16, 8), (40, 8)])
@pytest.mark.parametrize("mode", [0, 1])
def test_rows_shapes(gpu, layers, T, k, mode):
    name, host, dev = layers
    E = host.n_expert
    k = min(k, E)
    rng = np.random.default_rng(1000 * T + 10 * k + mode)
    x = rng.standard_normal((T, host.d)).astype(np.float32)
    ids, w = routing.softmax_topk(rng.standard_normal((T, E)), k)
    got, want = _run(gpu, host, dev, x, ids, w, mode=mode)
    err = ref.rel_l2(want, got)
    print(f"rows {name} T={T} k={k} mode={mode} rel_l2={err:.3e}")
    assert np.isfinite(got).all() and err <= TOL


@pytest.mark.parametrize("x_dtype,wbd", [("f32", True), ("f16", False), ("bf16", True)])
def test_rows_dtypes_weighting_and_drops(gpu, layers, x_dtype, wbd):
    name, host, dev = layers
    E = host.n_expert
    rng = np.random.default_rng(9)
    T, k = 6, 4
    # Rows of very different magnitude, dropped and out-of-range slots, a
    # token with every slot dropped.
    x = (rng.standard_normal((T, host.d)) * np.array([[1e-3], [40.0], [1.0], [1.0], [3.0], [1.0]])).astype(np.float32)
    ids, w = routing.softmax_topk(rng.standard_normal((T, E)), k)
    ids[1, 2] = -1
    ids[2, 3] = E + 3
    ids[5, :] = -1
    for mode in (0, 1):
        got, want = _run(gpu, host, dev, x, ids, w, x_dtype=x_dtype, wbd=wbd, mode=mode)
        err = ref.rel_l2(want, got)
        print(f"rows {name} {x_dtype} wbd={wbd} mode={mode} rel_l2={err:.3e}")
        assert err <= TOL
        if mode == 1:
            assert not got[1, 2].any() and not got[2, 3].any() and not got[5].any()
        else:
            assert not got[5].any()
