"""GPU parity at the DeepSeek-V3-shaped workloads of the prefill, heterogeneous
and stacked configurations (256 experts, d=7168, ff=2048, top-8), checked
against the oracle on the same packed factors and inputs.

The oracle dequantizes every routed expert in numpy, so where a batch routes
to most of the 256 experts the check runs on a subset of the tokens (every
token's output depends only on its own row and routing).  Bar: rel-L2 <= 2e-3.
"""

import numpy as np
import pytest

from oracle import latent_ref as ref
from oracle import routing
from tests._layers import remap_ids, subset_to_host, to_device

pytestmark = pytest.mark.gpu

TOL = 2e-3
E, D, FF, K = 256, 7168, 2048, 8


def _oracle(dev_layer, x, ids, w, tokens, wbd=False):
    """Oracle per-slot rows and reduced rows for `tokens` of a call."""
    sub_ids, sub_w, sub_x = ids[tokens], w[tokens], x[tokens]
    experts, local = remap_ids(sub_ids, dev_layer.n_expert)
    host = subset_to_host(dev_layer, experts)
    per_slot = ref.moe_forward(sub_x, local, sub_w, host, weight_before_down=wbd, out_mode=1)
    wt = np.where(local >= 0, sub_w, 0.0).astype(np.float64)
    reduced = per_slot.sum(1) if wbd else (per_slot.astype(np.float64) * wt[..., None]).sum(1)
    return per_slot, reduced, experts.size


# --------------------------------------------------------------------------------
# prefill: 4096 tokens, skewed popularity (about 0..400 tokens per expert)
# --------------------------------------------------------------------------------
@pytest.fixture(scope="module")
def dsv3(gpu):
    from latent_amd import synth as gsynth

    return gsynth.make_layer(seed=7, n_expert=E, d=D, ff=FF, max_rank=256)


def test_prefill_4096_skewed(gpu, dsv3):
    import torch

    from latent_amd import synth as gsynth

    T = 4096
    ids_t, w_t = gsynth.route(seed=30_000, n_tokens=T, n_expert=E, k=K, rank_beta=1.5)
    x_t = gsynth.bf16_input(seed=30_001, n_tokens=T, d=D)
    counts = np.bincount(ids_t.cpu().numpy().reshape(-1), minlength=E)
    print(f"prefill tokens per expert: min {counts.min()} max {counts.max()} below 16: {(counts < 16).sum()}")
    assert counts.min() < 16 and 300 <= counts.max() <= 600
    assert gpu.moe_path(dsv3, x_t, K) == "prefill"
    red = gpu.moe_forward(x_t, ids_t, w_t, dsv3, out_mode=0)
    slot = gpu.moe_forward(x_t, ids_t, w_t, dsv3, out_mode=1)
    torch.cuda.synchronize()
    ids, w, x = ids_t.cpu().numpy(), w_t.cpu().numpy(), x_t.float().cpu().numpy()
    # tokens that reach the coldest and the hottest experts, and a spread of others
    cold, hot = int(np.argmin(np.where(counts > 0, counts, 1 << 30))), int(np.argmax(counts))
    pick = {int(np.nonzero((ids == cold).any(1))[0][0]), int(np.nonzero((ids == hot).any(1))[0][0])}
    pick |= set(range(0, T, T // 30))
    tokens = np.array(sorted(pick))[:32]
    per_slot, reduced, n_exp = _oracle(dsv3, x, ids, w, tokens)
    err_red = ref.rel_l2(reduced, red.cpu().numpy()[tokens])
    err_slot = ref.rel_l2(per_slot, slot.cpu().numpy()[tokens])
    print(f"prefill 4096: {tokens.size} tokens, {n_exp} experts: reduced {err_red:.3e} per-slot {err_slot:.3e}")
    assert err_red <= TOL and err_slot <= TOL
    # the reduced output is the weighted sum of the per-slot rows
    s = slot.cpu().numpy().astype(np.float64)
    assert ref.rel_l2((s * w[..., None]).sum(1), red.cpu().numpy()) <= 1e-3


def test_prefill_4096_with_empty_experts(gpu, dsv3):
    # The same skewed routing with every 16th expert's slots moved to its
    # neighbour: 16 experts receive no token (no unit, no tile of theirs may
    # run), their neighbours twice the load.
    import torch

    from latent_amd import synth as gsynth

    T = 4096
    ids_t, w_t = gsynth.route(seed=30_000, n_tokens=T, n_expert=E, k=K, rank_beta=1.5)
    ids = ids_t.cpu().numpy()
    ids = np.where(ids % 16 == 0, ids + 1, ids).astype(np.int32)
    counts = np.bincount(ids.reshape(-1), minlength=E)
    assert (counts == 0).sum() == 16
    ids_t = torch.from_numpy(ids).cuda()
    x_t = gsynth.bf16_input(seed=30_002, n_tokens=T, d=D)
    assert gpu.moe_path(dsv3, x_t, K) == "prefill"
    red = gpu.moe_forward(x_t, ids_t, w_t, dsv3, out_mode=0)
    slot = gpu.moe_forward(x_t, ids_t, w_t, dsv3, out_mode=1)
    torch.cuda.synchronize()
    w, x = w_t.cpu().numpy(), x_t.float().cpu().numpy()
    hot = int(np.argmax(counts))
    tokens = np.array(sorted({int(np.nonzero((ids == hot).any(1))[0][0])} | set(range(7, T, T // 24))))[:28]
    per_slot, reduced, n_exp = _oracle(dsv3, x, ids, w, tokens)
    err_red = ref.rel_l2(reduced, red.cpu().numpy()[tokens])
    err_slot = ref.rel_l2(per_slot, slot.cpu().numpy()[tokens])
    print(f"prefill 4096, 16 empty experts: {tokens.size} tokens, {n_exp} experts: reduced {err_red:.3e} "
          f"per-slot {err_slot:.3e}")
    assert err_red <= TOL and err_slot <= TOL
    assert not torch.isnan(red).any()


def _rows_agree(a, b):
    """rel-L2 of b against a over the whole batch, and the worst token's."""
    a, b = a.astype(np.float64), b.astype(np.float64)
    per_token = np.linalg.norm(a - b, axis=1) / np.maximum(np.linalg.norm(a, axis=1), 1e-30)
    return ref.rel_l2(a, b), float(per_token.max())


def test_prefill_4096_engines_agree_on_every_token(gpu, dsv3):
    # Every one of the 4096 tokens (the oracle checks a subset above): the
    # streaming-tile engine on the tile layout against the grouped-GEMM engine
    # on the row layout of the same layer, two independent implementations.
    import torch

    from latent_amd import synth as gsynth

    T = 4096
    ids_t, w_t = gsynth.route(seed=30_000, n_tokens=T, n_expert=E, k=K, rank_beta=1.5)
    x_t = gsynth.bf16_input(seed=30_003, n_tokens=T, d=D)
    rows = dsv3.to_layout("rows")
    assert gpu.moe_path(dsv3, x_t, K) == "prefill" and gpu.moe_path(rows, x_t, K) == "prefill"
    bulk = gpu.moe_forward(x_t, ids_t, w_t, dsv3).cpu().numpy()
    gemm = gpu.moe_forward(x_t, ids_t, w_t, rows).cpu().numpy()
    del rows
    err, worst = _rows_agree(gemm, bulk)
    print(f"prefill 4096, tile engine vs GEMM engine: rel-L2 {err:.3e}, worst token {worst:.3e}")
    assert err <= TOL and worst <= 5 * TOL


def test_prefill_per_slot_zeroes_dropped_slots(gpu):
    # Per-slot output on the prefill path: dropped (-1) and out-of-range ids
    # give exact zero rows, routed rows match the oracle.
    from oracle import synth

    layer = synth.make_layer(seed=300, n_expert=32, d=1024, ff=512, max_rank=128)
    dev = to_device(layer)
    import torch

    T, k = 256, 4
    rng = np.random.default_rng(33)
    x = rng.standard_normal((T, 1024)).astype(np.float32)
    ids, w = routing.softmax_topk(routing.zipf_logits(rng, T, 32, gamma=0.5), k)
    ids[::5, 1] = -1
    ids[::7, 3] = 32
    ids[3, :] = -1
    xt = torch.from_numpy(x).cuda().to(torch.bfloat16)
    it, wt = torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda()
    assert gpu.moe_path(dev, xt, k) == "prefill"
    out = torch.full((T, k, 1024), float("nan"), device="cuda")  # stale contents must not survive
    gpu.moe_forward(xt, it, wt, dev, out_mode=1, out=out)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    dropped = (ids < 0) | (ids >= 32)
    assert dropped.sum() > 50 and not np.isnan(got).any()
    assert (got[dropped] == 0).all()
    want = ref.moe_forward(xt.float().cpu().numpy(), ids, w, layer, out_mode=1)
    assert ref.rel_l2(want, got) <= TOL


# --------------------------------------------------------------------------------
# heterogeneous ranks {64..512} padded to 512, 10% INT8 groups, drop below 0.05
# --------------------------------------------------------------------------------
@pytest.fixture(scope="module")
def hetero(gpu):
    from latent_amd import synth as gsynth

    rng = np.random.default_rng(3)
    ranks = rng.choice([64, 128, 256, 512], E)
    return gsynth.make_layer(seed=11, n_expert=E, d=D, ff=FF, max_rank=512, ranks=ranks, int8_fraction=0.1)


@pytest.mark.parametrize("T,path", [(16, "default"), (16, "fused"), (16, "general"), (256, "default"), (256, "rows")])
def test_hetero_int8_drop(gpu, hetero, T, path, monkeypatch):
    import torch

    from latent_amd import synth as gsynth
    from latent_amd.moe import moe_path

    if path != "default":
        monkeypatch.setenv("LATENT_MOE_PATH", path)
    # N(0,1) logits drop ~0.3% of slots at 0.05; at 16 tokens, scale them by 2
    # (~16% dropped) so every run exercises the drop rule.
    ids_t, w_t = gsynth.route(seed=40_000 + T, n_tokens=T, n_expert=E, k=K, drop_below=0.05,
                              logit_scale=2.0 if T <= 16 else 1.0)
    x_t = gsynth.bf16_input(seed=41_000 + T, n_tokens=T, d=D)
    used = moe_path(hetero, x_t, K)
    red = gpu.moe_forward(x_t, ids_t, w_t, hetero, out_mode=0, check_timeout=True)
    slot = gpu.moe_forward(x_t, ids_t, w_t, hetero, out_mode=1, check_timeout=True)
    torch.cuda.synchronize()
    ids, w, x = ids_t.cpu().numpy(), w_t.cpu().numpy(), x_t.float().cpu().numpy()
    assert (ids < 0).any()  # the drop rule fired
    tokens = np.arange(T) if T <= 16 else np.arange(0, T, T // 24)
    per_slot, reduced, n_exp = _oracle(hetero, x, ids, w, tokens)
    err_red = ref.rel_l2(reduced, red.cpu().numpy()[tokens])
    err_slot = ref.rel_l2(per_slot, slot.cpu().numpy()[tokens])
    print(f"hetero T={T} path={used}: {tokens.size} tokens, {n_exp} experts: reduced {err_red:.3e} "
          f"per-slot {err_slot:.3e}")
    assert err_red <= TOL and err_slot <= TOL
    assert (slot.cpu().numpy()[ids < 0] == 0).all()


def test_hetero_256_paths_agree_on_every_token(gpu, hetero, monkeypatch):
    # All 256 tokens (the oracle checks a subset above): the row-layout MFMA
    # phases against the fp32 GEMV phases, and each path's reduced output
    # against the weighted sum of its per-slot rows.
    import torch

    from latent_amd import synth as gsynth

    T = 256
    ids_t, w_t = gsynth.route(seed=40_000 + T, n_tokens=T, n_expert=E, k=K, drop_below=0.05)
    x_t = gsynth.bf16_input(seed=41_000 + T, n_tokens=T, d=D)
    w = w_t.cpu().numpy().astype(np.float64)
    outs = {}
    for path in ("rows", "general"):
        monkeypatch.setenv("LATENT_MOE_PATH", path)
        red = gpu.moe_forward(x_t, ids_t, w_t, hetero, out_mode=0, check_timeout=True)
        slot = gpu.moe_forward(x_t, ids_t, w_t, hetero, out_mode=1, check_timeout=True)
        torch.cuda.synchronize()
        red, slot = red.cpu().numpy(), slot.cpu().numpy().astype(np.float64)
        err, worst = _rows_agree((slot * w[..., None]).sum(1), red)
        assert err <= 1e-4 and worst <= 1e-3, (path, err, worst)  # fp16 intermediates: ~4e-5 on the MFMA path
        outs[path] = red
    err, worst = _rows_agree(outs["general"], outs["rows"])
    print(f"hetero T=256, row-layout MFMA vs fp32 GEMV: rel-L2 {err:.3e}, worst token {worst:.3e}")
    assert err <= TOL and worst <= 5 * TOL


# --------------------------------------------------------------------------------
# stacked decode: DeepSeek-V3-shaped layers, batch 32, one HIP graph
# --------------------------------------------------------------------------------
def test_stack_dsv3_graph(gpu):
    import torch

    from latent_amd import synth as gsynth

    n_layers, T = 3, 32
    layers = [gsynth.make_layer(seed=500_000 + 7919 * l, n_expert=E, d=D, ff=FF, max_rank=256) for l in range(n_layers)]
    routers = []
    for l in range(n_layers):
        g = torch.Generator(device="cuda")
        g.manual_seed(900_000 + l)
        routers.append(gpu.Router(torch.randn((D, E), generator=g, device="cuda") / np.sqrt(D), K))
    stack = gpu.DecodeStack(layers, routers, T)
    x0 = gsynth.bf16_input(seed=777, n_tokens=T, d=D).float()
    eager = stack.forward(x0).clone()
    xs = [t.clone() for t in stack.x]
    ys = [t.clone() for t in stack.y]
    ids_l = [t.clone() for t in stack.ids]
    ws_l = [t.clone() for t in stack.w]
    torch.cuda.synchronize()
    assert gpu.moe_path(layers[0], xs[0], K) == "stream"
    tokens = np.arange(0, T, 3)
    for l in range(n_layers):
        x_l, ids, w = xs[l].cpu().numpy(), ids_l[l].cpu().numpy(), ws_l[l].cpu().numpy()
        _, reduced, n_exp = _oracle(layers[l], x_l, ids, w, tokens)
        err = ref.rel_l2(reduced, ys[l].cpu().numpy()[tokens])
        print(f"stack layer {l}: {tokens.size} tokens, {n_exp} experts, rel_l2 {err:.3e}")
        assert err <= TOL
        np.testing.assert_array_equal(xs[l + 1].cpu().numpy(), x_l + ys[l].cpu().numpy())
    stack.capture()
    for rep in range(3):
        stack.load(x0)
        out = stack.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {rep} differs from the eager run"
        stack.forward(x0)
        torch.cuda.synchronize()
        assert torch.equal(stack.output, eager), f"eager run after replay {rep} differs"


# --------------------------------------------------------------------------------
# per-group INT8 selection of the GPU factorizer against the oracle
# --------------------------------------------------------------------------------
def test_int8_group_selection_matches_oracle(gpu):
    import torch

    from latent_amd import factorize

    rng = np.random.default_rng(19)
    v = (rng.standard_normal((2, 64, 256)) * np.exp(1.5 * rng.standard_normal((2, 64, 256)))).astype(np.float32)
    v[0, 3, 32:64] = 0.0
    vt = torch.from_numpy(v).cuda()
    codes, scales = gpu.pack_nf4(vt)
    f = gpu.DeviceFactor(codes.contiguous(), scales.contiguous())
    decoded = torch.stack([gpu.unpack(f, e) for e in range(2)])
    for thr in (8.7, 10.2, 12.4):  # about the 10th, 50th and 90th percentile of the NF4 SNR here
        got = factorize.int8_group_mask(vt, decoded, thr).cpu().numpy()
        want = np.stack([ref.int8_group_mask(v[e], thr) for e in range(2)])
        snr = np.stack([ref.quantization_snr_by_group(v[e], decoded[e].cpu().numpy(), 32).reshape(64, 8)
                        for e in range(2)])
        borderline = np.abs(snr - thr) <= 1e-4 * thr  # fp32 norms summed in another order
        print(f"threshold {thr}: {want.sum()} groups selected, {int((got != want).sum())} differ, "
              f"{int(borderline.sum())} borderline")
        assert 0 < want.sum() < want.size
        assert not ((got != want) & ~borderline).any()


def _fake_int8_args(L, d, E=512, R=256, ff=512, T=8, k=8):
    """Arguments whose pointers are never dereferenced (a path query only),
    with INT8 groups on gate_a (d x R per expert)."""
    def fac(rows, cols, int8=False):
        f = L.LatentFactor(codes=1 << 20, scales=2 << 20, rows=rows, cols=cols)
        if int8:
            f.int8_bitmap, f.int8_row_offset, f.int8_data = 3 << 20, 4 << 20, 5 << 20
        return f

    a = L.LatentMoeArgs()
    a.gate_a, a.gate_b = fac(d, R, True), fac(R, ff)
    a.up_a, a.up_b = fac(d, R), fac(R, ff)
    a.down_a, a.down_b = fac(ff, R), fac(R, d)
    a.x, a.ids, a.weights, a.out = 6 << 20, 7 << 20, 8 << 20, 9 << 20
    a.n_tokens, a.n_embd, a.n_ff, a.n_expert, a.n_expert_used, a.max_rank = T, d, ff, E, k, R
    a.x_dtype, a.weights_dtype, a.out_mode = L.LATENT_BF16, L.LATENT_F32, L.LATENT_OUT_REDUCED
    return a


def test_int8_side_buffer_beyond_32_bit_offsets_leaves_the_persistent_kernel(gpu, monkeypatch):
    """The persistent kernel and the row-layout MFMA phases read INT8 groups
    with 32-bit byte offsets: a factor whose side buffer could reach 2^31
    bytes (every group INT8) goes to the multi-kernel fp32 path, one just
    below stays on them (the row-layout MFMA phases by default, the
    persistent kernel when it is asked for)."""
    import ctypes

    from latent_amd import _lib as L

    below = _fake_int8_args(L, d=8192)  # 512 x 8192 x 256 = 2^30 bytes of INT8 at most
    beyond = _fake_int8_args(L, d=16384)  # 2^31 bytes
    assert L.lib.latent_moe_path(ctypes.byref(below)) == 4
    assert L.lib.latent_moe_path(ctypes.byref(beyond)) == 0
    monkeypatch.setenv("LATENT_MOE_PATH", "fused")
    assert L.lib.latent_moe_path(ctypes.byref(below)) == 1
    assert L.lib.latent_moe_path(ctypes.byref(beyond)) == 0
