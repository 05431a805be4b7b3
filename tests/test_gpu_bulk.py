"""Prefill on the tile layout (bulk units of up to 64 pairs) against the
oracle.

Rank-256 layers held in the tile layout take this engine for prefill-sized
batches; the same layer in the row layout takes the grouped GEMMs, which the
last test uses as a second, independent implementation.  Bar: rel-L2 <= 2e-3
against the oracle's fp32 result on the same packed factors, bit-identical
results on a repeated call, exact zeros in dropped per-slot rows.
"""

import numpy as np
import pytest

from oracle import latent_ref as ref
from oracle import routing, synth
from tests._layers import to_device

pytestmark = pytest.mark.gpu

TOL = 2e-3
E, D, FF = 12, 1024, 1024


@pytest.fixture(scope="module")
def layer():
    return synth.make_layer(seed=510, n_expert=E, d=D, ff=FF, max_rank=256)


@pytest.fixture(scope="module")
def dev(gpu, layer):
    d = to_device(layer)
    assert d.layout == "tiles"  # the layer is held in the tile layout, so prefill takes the bulk engine
    return d


def _skewed_ids(rng, T, k):
    # Expert 0 takes most tokens (several 128-pair units), expert 11 a handful.
    logits = rng.standard_normal((T, E))
    logits[:, 0] += 3.0
    logits[:, 11] -= 4.0
    return routing.softmax_topk(logits, k)


def _run(gpu, dev, x, ids, w, x_dtype="bf16", wbd=False, mode=0):
    import torch

    tdt = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}[x_dtype]
    xt = torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda().to(tdt)
    it = torch.from_numpy(np.ascontiguousarray(ids, np.int32)).cuda()
    wt = torch.from_numpy(np.ascontiguousarray(w, np.float32)).cuda()
    assert gpu.moe_path(dev, xt, ids.shape[1]) == "prefill"
    out = gpu.moe_forward(xt, it, wt, dev, weight_before_down=wbd, out_mode=mode)
    again = gpu.moe_forward(xt, it, wt, dev, weight_before_down=wbd, out_mode=mode)
    torch.cuda.synchronize()
    assert torch.equal(out, again), "repeated call is not bit-identical"
    return out.cpu().numpy(), xt.float().cpu().numpy()


@pytest.mark.parametrize("mode", [0, 1])
def test_bulk_skewed_units(gpu, layer, dev, mode):
    rng = np.random.default_rng(41)
    T, k = 320, 4
    x = rng.standard_normal((T, D)).astype(np.float32)
    ids, w = _skewed_ids(rng, T, k)
    counts = np.bincount(ids.reshape(-1), minlength=E)
    assert counts.max() > 256 and counts.min() < 16, counts
    got, xq = _run(gpu, dev, x, ids, w, mode=mode)
    want = ref.moe_forward(xq, ids, w, layer, out_mode=mode)
    err = ref.rel_l2(want, got)
    print(f"bulk skewed mode={mode} counts={counts.tolist()} rel_l2={err:.3e}")
    assert err <= TOL


@pytest.mark.parametrize("x_dtype,wbd", [("f32", True), ("f16", False), ("bf16", True)])
def test_bulk_dtypes_and_weighting(gpu, layer, dev, x_dtype, wbd):
    rng = np.random.default_rng(42)
    T, k = 200, 6
    x = (rng.standard_normal((T, D)) * 3.0).astype(np.float32)
    ids, w = routing.softmax_topk(rng.standard_normal((T, E)), k)
    for mode in (0, 1):
        got, xq = _run(gpu, dev, x, ids, w, x_dtype=x_dtype, wbd=wbd, mode=mode)
        want = ref.moe_forward(xq, ids, w, layer, weight_before_down=wbd, out_mode=mode)
        assert ref.rel_l2(want, got) <= TOL


def test_bulk_one_expert_dropped_and_invalid(gpu, layer, dev):
    # 300 tokens on expert 3 (units of 128, 128 and 44 pairs), dropped and
    # out-of-range slots, and a token with every slot dropped.
    rng = np.random.default_rng(43)
    T, k = 300, 3
    x = rng.standard_normal((T, D)).astype(np.float32)
    ids, w = routing.softmax_topk(rng.standard_normal((T, E)), k)
    ids[:, 0] = 3
    ids[::4, 1] = -1
    ids[::9, 2] = E + 5
    ids[7, :] = -1
    for mode in (0, 1):
        got, xq = _run(gpu, dev, x, ids, w, mode=mode)
        want = ref.moe_forward(xq, np.where(ids >= E, -1, ids), w, layer, out_mode=mode)
        assert ref.rel_l2(want, got) <= TOL
        if mode == 1:
            dropped = (ids < 0) | (ids >= E)
            assert (got[dropped] == 0).all()
        else:
            assert not got[7].any()


def test_bulk_matches_gemm_engine(gpu, layer, dev, monkeypatch):
    import torch

    rng = np.random.default_rng(44)
    T, k = 256, 4
    x = rng.standard_normal((T, D)).astype(np.float32)
    ids, w = _skewed_ids(rng, T, k)
    xt = torch.from_numpy(x).cuda().to(torch.bfloat16)
    it, wt = torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda()
    bulk = gpu.moe_forward(xt, it, wt, dev)
    rows = dev.to_layout("rows")
    assert gpu.moe_path(rows, xt, k) == "prefill"
    gemm = gpu.moe_forward(xt, it, wt, rows)
    torch.cuda.synchronize()
    assert not torch.equal(bulk, gemm), "both calls ran the same engine"
    assert ref.rel_l2(gemm.cpu().numpy(), bulk.cpu().numpy()) <= TOL


@pytest.mark.parametrize("mode", [0, 1])
def test_bulk_token_magnitudes(gpu, layer, dev, mode):
    # Tokens scaled from 1e-12 to 1e12 and one all-zero token: every
    # intermediate row (latents, h, y) carries its own power-of-two exponent,
    # so each token keeps its relative accuracy whatever its size, and the
    # zero token's rows (zero norms, the exponents' clamped end) give exact
    # zeros.  Checked token by token against the oracle.
    rng = np.random.default_rng(45)
    T, k = 256, 4
    x = rng.standard_normal((T, D)) * 10.0 ** rng.uniform(-12.0, 12.0, size=(T, 1))
    x[5] = 0.0
    x = x.astype(np.float32)
    ids, w = _skewed_ids(rng, T, k)
    got, xq = _run(gpu, dev, x, ids, w, mode=mode)
    want = ref.moe_forward(xq, ids, w, layer, out_mode=mode)
    got = got.reshape(T, -1)
    want = want.reshape(T, -1)
    assert np.isfinite(got).all()
    assert not got[5].any()
    live = [t for t in range(T) if t != 5]
    errs = np.array([ref.rel_l2(want[t], got[t]) for t in live])
    print(f"bulk magnitudes mode={mode} worst token rel_l2={errs.max():.3e} median={np.median(errs):.3e}")
    assert errs.max() <= 5 * TOL
