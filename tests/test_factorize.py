"""Load-time factorisation (latent_amd.factorize) against the oracle and the
mathematics of the truncated SVD.

CPU: the oracle's choose_rank against brute force and the reference's
definition (first index where the cumulative energy reaches the target);
randomized SVD on a matrix of known spectrum (Eckart-Young bound, singular
values, orthonormal columns).  GPU: the torch path's ranks equal the oracle's
on the same singular values; its factors reconstruct like the oracle's; the
packed layer decodes to the factors within NF4 error and runs.
"""

import numpy as np
import pytest

from oracle import latent_ref as ref
from oracle import synth


def _spectrum_matrix(m, n, s, seed):
    rng = np.random.default_rng(seed)
    u, _ = np.linalg.qr(rng.standard_normal((m, len(s))))
    v, _ = np.linalg.qr(rng.standard_normal((n, len(s))))
    return ((u * s) @ v.T).astype(np.float32)


def test_choose_rank_matches_brute_force():
    rng = np.random.default_rng(2)
    for _ in range(50):
        s = np.sort(rng.random(40) ** 3)[::-1]
        energy = float(rng.uniform(0.3, 1.0))
        e2 = s.astype(np.float64) ** 2
        frac = np.cumsum(e2) / e2.sum()
        brute = next(i + 1 for i in range(40) if frac[i] >= energy)  # first rank reaching the energy
        for lo, hi in ((1, 40), (8, 20), (16, 64)):
            assert synth.choose_rank(s, energy, lo, hi) == max(lo, min(brute, hi, 40))
    assert synth.choose_rank(np.zeros(5), 0.9, 3, 5) == 3
    with pytest.raises(ValueError):
        synth.choose_rank(np.ones(3), 1.5, 1, 3)


def test_oracle_randomized_svd_on_known_spectrum():
    s = 0.02 * np.arange(1, 65, dtype=np.float64) ** -0.7
    w = _spectrum_matrix(200, 150, s, 1)
    u, sv, vt = synth.randomized_svd(w.astype(np.float64), 16, seed=3)
    # Projection onto range(Q) never raises a singular value (interlacing);
    # the leading ones are recovered closely.
    assert np.all(sv <= s[:16] * (1 + 1e-9))
    np.testing.assert_allclose(sv[:8], s[:8], rtol=5e-3)
    np.testing.assert_allclose(u.T @ u, np.eye(16), atol=1e-10)
    a, b = synth.make_factors(u, sv, vt, 16)
    err = np.linalg.norm(w - a @ b) / np.linalg.norm(w)
    bound = np.sqrt(np.sum(s[16:] ** 2)) / np.linalg.norm(s)  # Eckart-Young optimum
    assert bound <= err <= 1.05 * bound + 1e-6


def _host_layer(arrays, d, ff, max_rank):
    facs = {}
    for name in ref.FACTOR_NAMES:
        ext = None
        if name + "_i8" in arrays:
            ext = ref.Int8Groups(bitmap=arrays[name + "_i8map"], data=arrays[name + "_i8"],
                                 row_offset=arrays[name + "_i8off"])
        facs[name] = ref.StackedFactor(arrays[name], arrays[name + "_s"], ext)
    return ref.StackedLayer(facs, d=d, ff=ff, max_rank=max_rank, ranks=arrays.get("ranks"))


@pytest.mark.gpu
def test_gpu_factorize_matches_oracle_and_runs(gpu):
    import torch

    from latent_amd import factorize, gguf

    E, d, ff, R = 3, 256, 128, 64
    spec = 0.05 * np.exp(-np.arange(128) / 8.0)  # rank 28 keeps 99.9% of the energy
    mats = {k: [_spectrum_matrix(*((d, ff) if k != "down" else (ff, d)), spec, 10 * e + i) for e in range(E)]
            for i, k in enumerate(("gate", "up", "down"))}
    dev = {k: [torch.from_numpy(m).cuda() for m in v] for k, v in mats.items()}
    # ranks: same choose_rank on the same singular values
    for e in range(E):
        sv = torch.linalg.svdvals(dev["gate"][e]).cpu().numpy()
        assert factorize.choose_rank(torch.from_numpy(sv), 0.999, 16, R) == synth.choose_rank(sv, 0.999, 16, R)
    # randomized SVD: same spectrum and reconstruction as the oracle's on the same sketch
    u, s, vt = factorize.randomized_svd(dev["gate"][0], 32, seed=5)
    a, b = factorize.make_factors(u, s, vt, 32)
    ou, os_, ovt = synth.randomized_svd(mats["gate"][0].astype(np.float64), 32, seed=5)
    oa, ob = synth.make_factors(ou, os_, ovt, 32)
    np.testing.assert_allclose(s.cpu().numpy(), os_, rtol=1e-4)
    assert ref.rel_l2(oa @ ob, (a @ b).cpu().numpy()) <= 1e-3  # fp32 on the GPU against the float64 oracle

    x = torch.randn((4, d), device="cuda")
    ids = torch.tensor([[0, 1], [2, 0], [1, 2], [0, 2]], dtype=torch.int32, device="cuda")
    w = torch.full((4, 2), 0.5, device="cuda")
    xs = x.cpu().numpy()
    dense = np.zeros((4, d), np.float32)
    for t in range(4):
        for kk in range(2):
            e = int(ids[t, kk])
            dense[t] += 0.5 * ref.dense_swiglu_expert(xs[t:t + 1], mats["gate"][e], mats["up"][e], mats["down"][e])[0]
    errs = {}
    for thr in (None, 1e9):  # NF4 only; every non-zero group INT8
        layer, ranks = factorize.stack_experts(dev["gate"], dev["up"], dev["down"], max_rank=R, energy=0.999,
                                               min_rank=16, snr_threshold=thr)
        assert all(16 <= r <= R for rr in ranks for r in rr)
        assert layer.ranks.cpu().tolist() == [list(r) for r in ranks]
        assert all(f.has_int8 == (thr is not None) for f in layer.factors().values())
        host = _host_layer(gguf.layer_to_arrays(layer), d, ff, R)
        for k, (name, f) in enumerate(layer.factors().items()):  # the built layout decodes as the oracle reads it
            for e in range(E):
                assert np.array_equal(gpu.unpack(f, e, kind=k).cpu().numpy(), host.factors[name].expert(e))
        out = gpu.moe_forward(x, ids, w, layer)
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        assert ref.rel_l2(ref.moe_forward(xs, ids.cpu().numpy(), w.cpu().numpy(), host), got) <= 2e-3
        errs[thr] = ref.rel_l2(dense, got)
    print(f"factorized layer vs dense rel_l2: nf4={errs[None]:.3e} int8={errs[1e9]:.3e}")
    # CPU emulation of the same pipeline: truncation alone 0.05, with NF4 0.19
    assert errs[1e9] < 0.1 and errs[1e9] < errs[None] < 0.3
