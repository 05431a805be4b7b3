"""GPU router front end and the graph-captured layer stack against the oracle.

Routing parity: the GPU's logits match float64 x . W_r to 1e-5 relative; top-k
ids are bit-exact and weights match to 1e-6 when the oracle routes the GPU's
own logits (the selection is then decided by the same values); the drop rules
follow oracle/routing.py.  Stack parity: every layer's expert-FFN output
against the oracle on that layer's GPU input (rel-L2 <= 2e-3), and graph
replays equal the eager run bit for bit.
"""

import numpy as np
import pytest

from oracle import latent_ref as ref
from oracle import routing, synth
from tests._layers import to_device

pytestmark = pytest.mark.gpu

TOL = 2e-3


def _cuda(a, dtype=None):
    import torch

    t = torch.from_numpy(np.ascontiguousarray(a)).cuda()
    return t if dtype is None else t.to(dtype)


@pytest.mark.parametrize("T,d,E,k,x_dtype,r_dtype", [
    (1, 7168, 256, 8, "bf16", "f32"),
    (32, 7168, 256, 8, "bf16", "f32"),
    (37, 300, 64, 6, "f32", "bf16"),
    (5, 1000, 1024, 64, "f16", "f32"),
])
def test_route_from_x_matches_oracle(gpu, T, d, E, k, x_dtype, r_dtype):
    import torch

    tdt = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}
    rng = np.random.default_rng(T * 1000 + E)
    x = _cuda(rng.standard_normal((T, d)).astype(np.float32), tdt[x_dtype])
    W = _cuda((rng.standard_normal((d, E)) / np.sqrt(d)).astype(np.float32), tdt[r_dtype])
    logits = torch.empty((T, E), dtype=torch.float32, device="cuda")
    ids, w = gpu.route(k, x=x, router=W, logits_out=logits)
    torch.cuda.synchronize()
    want_lg = routing.router_logits(x.float().cpu().numpy(), W.float().cpu().numpy())
    got_lg = logits.cpu().numpy()
    assert np.abs(got_lg - want_lg).max() <= 1e-5 * max(1.0, np.abs(want_lg).max())
    want_ids, want_w = routing.softmax_topk(got_lg, k)
    assert np.array_equal(ids.cpu().numpy(), want_ids)
    np.testing.assert_allclose(w.cpu().numpy(), want_w, rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("drop,param", [("none", 0.0), ("below", 0.05), ("below", 0.2), ("inclusive", 0.95),
                                        ("inclusive", 0.5)])
def test_route_from_logits_drop_rules(gpu, drop, param):
    rng = np.random.default_rng(11)
    lg = routing.zipf_logits(rng, 257, 256, gamma=0.11)
    ids, w = gpu.route(8, logits=_cuda(lg), drop=drop, drop_param=param)
    want_ids, want_w = routing.route(lg, 8, drop, param)
    assert np.array_equal(ids.cpu().numpy(), want_ids)
    np.testing.assert_allclose(w.cpu().numpy(), want_w, rtol=2e-6, atol=1e-7)


def test_route_ties_go_to_lower_expert(gpu):
    lg = np.zeros((4, 200), np.float32)
    lg[0, [5, 150, 7]] = 1.0          # equal maxima: 5, 7, 150 then zeros from id 0
    lg[1, :] = -np.inf                 # all -inf: lowest ids first
    lg[2, 199] = np.nan                # NaN never wins
    lg[3, :] = -1.0
    lg[3, [64, 3]] = -0.0              # -0 and +0 are equal: lower id first
    lg[3, [130, 9]] = 0.0
    ids, w = gpu.route(4, logits=_cuda(lg))
    got = ids.cpu().numpy()
    assert got[0].tolist() == [5, 7, 150, 0]
    assert got[1].tolist() == [0, 1, 2, 3]
    assert 199 not in got[2].tolist()
    assert got[3].tolist() == [3, 9, 64, 130]


def test_route_rejects_bad_arguments(gpu):
    import torch

    from latent_amd import LatentError

    lg = torch.zeros((2, 8), dtype=torch.float32, device="cuda")
    with pytest.raises(LatentError):
        gpu.route(9, logits=lg)  # k > E
    with pytest.raises(LatentError):
        gpu.route(2, logits=lg, drop="inclusive", drop_param=0.0)
    with pytest.raises(ValueError):
        gpu.route(2, logits=lg, drop="nope")


@pytest.mark.parametrize("T", [2, 8])
def test_graph_stack_matches_eager_and_oracle(gpu, T):
    """Three small layers (8 routed pairs: multi-kernel path; 32: persistent kernel)."""
    import torch

    E, d, ff, R, k, n_layers = 16, 256, 256, 64, 4, 3
    hosts = [synth.make_layer(seed=40 + l, n_expert=E, d=d, ff=ff, max_rank=R) for l in range(n_layers)]
    layers = [to_device(h) for h in hosts]
    rng = np.random.default_rng(5)
    routers = [gpu.Router(_cuda((rng.standard_normal((d, E)) / np.sqrt(d)).astype(np.float32)), k)
               for _ in range(n_layers)]
    stack = gpu.DecodeStack(layers, routers, T)
    x0 = _cuda(rng.standard_normal((T, d)).astype(np.float32))
    eager = stack.forward(x0).clone()
    xs = [t.clone() for t in stack.x]
    ys = [t.clone() for t in stack.y]
    lgs = [t.clone() for t in stack.logits]
    ids_l = [t.clone() for t in stack.ids]
    torch.cuda.synchronize()
    # Per layer: routing and expert FFN against the oracle on the GPU's layer input.
    for l in range(n_layers):
        x_l = xs[l].cpu().numpy()
        lg = lgs[l].cpu().numpy()
        want_lg = routing.router_logits(x_l, routers[l].weight.cpu().numpy())
        assert np.abs(lg - want_lg).max() <= 1e-5 * max(1.0, np.abs(want_lg).max())
        want_ids, want_w = routing.softmax_topk(lg, k)
        assert np.array_equal(ids_l[l].cpu().numpy(), want_ids)
        want_y = ref.moe_forward(x_l, want_ids, want_w, hosts[l])
        err = ref.rel_l2(want_y, ys[l].cpu().numpy())
        print(f"T={T} layer {l}: rel_l2={err:.3e}")
        assert err <= TOL
        np.testing.assert_array_equal(xs[l + 1].cpu().numpy(), x_l + ys[l].cpu().numpy())
    # Graph replays, with eager work and synchronisations between them.
    # The persistent kernel (>= 32 pairs) sums in a fixed order; the multi-kernel
    # path adds workgroup partials with float atomics (order not fixed).
    exact = gpu.moe_path(layers[0], x0, k) == "fused"
    assert exact == (T * k >= 32)
    stack.capture()
    for rep in range(3):
        stack.load(x0)
        out = stack.replay()
        torch.cuda.synchronize()
        _same(out, eager, exact, f"replay {rep}")
        stack.forward(x0)  # eager run between replays
        torch.cuda.synchronize()
        _same(stack.output, eager, exact, f"eager run after replay {rep}")


def _same(got, want, exact, what):
    import torch

    if exact:
        assert torch.equal(got, want), f"{what} differs from the first eager run"
    else:
        err = ref.rel_l2(want.cpu().numpy(), got.cpu().numpy())
        assert err <= 1e-6, f"{what}: rel_l2 {err:.3e} against the first eager run"
