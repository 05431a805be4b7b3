"""GPU swiglu_expert on factor artifacts exactly as the reference writes them.

loader/latent_loader.py quantizes each factor as one flat array
(quantize_nf4 / quantize_int8, :111-158), so groups straddle rows whenever the
column count is not a multiple of the group: the energy-chosen ranks of the
CLI (:292-297, e.g. 37) and the reference's own test shapes
(tests/test_latent_loader.py:100-127: 16 -> 12 -> 16 at rank 4..8) do that.
The GPU path (`latent_expert_forward` through latent_amd.runtime) decodes
them as they are; the bar is rel-L2 <= 2e-3 against the oracle's fp32
swiglu_expert (loader/latent_runtime.py:48-59) on the same artifacts.
"""

import numpy as np
import pytest

from oracle import latent_ref as ref
from oracle import synth

pytestmark = pytest.mark.gpu

TOL = 2e-3


def _low_rank(rows, cols, rank, seed):
    rng = np.random.default_rng(seed)
    return rng.standard_normal((rows, rank), dtype=np.float32) @ rng.standard_normal((rank, cols), dtype=np.float32)


def _artifacts(mats, **kw):
    arrays, reports = {}, {}
    for name, m in mats.items():
        a, r = synth.compress_matrix(name, m, seed=10, **kw)  # the reference test's seed
        arrays.update(a)
        reports[name] = r
    return arrays, reports


def _both(arrays, x, weight=1.0, wbd=False):
    from latent_amd import runtime

    want = ref.swiglu_expert(x, ref.load_pair(arrays, "gate"), ref.load_pair(arrays, "up"),
                             ref.load_pair(arrays, "down"), weight=weight, weight_before_down=wbd)
    got = runtime.swiglu_expert(x, runtime.load_pair(arrays, "gate"), runtime.load_pair(arrays, "up"),
                                runtime.load_pair(arrays, "down"), weight=weight, weight_before_down=wbd)
    return want, got


@pytest.mark.parametrize("wbd", [False, True])
def test_reference_test_shapes(gpu, wbd):
    # tests/test_latent_loader.py:100-127: gate/up 16x12, down 12x16, true rank 4,
    # compress_matrix(energy=0.999, min_rank=4, max_rank=8, ...): A factors of 16x4
    # have one 32-group per 8 rows.
    mats = {"gate": _low_rank(16, 12, 4, 1), "up": _low_rank(16, 12, 4, 2), "down": _low_rank(12, 16, 4, 3)}
    arrays, reports = _artifacts(mats, energy=0.999, min_rank=4, max_rank=8, error_threshold=1.0,
                                 snr_threshold=0.0, low_snr_fraction_threshold=1.0)
    assert all(not r["fallback"] and r["quantization"] == "nf4_g32" for r in reports.values())
    x = np.random.default_rng(99).standard_normal((3, 16), dtype=np.float32)
    want, got = _both(arrays, x, weight=0.25, wbd=wbd)
    err = ref.rel_l2(want, got)
    print(f"reference test shapes wbd={wbd} ranks={[r['rank'] for r in reports.values()]} rel_l2={err:.3e}")
    assert got.shape == (3, 16) and err <= TOL


def test_cli_default_odd_ranks(gpu):
    # The CLI defaults (energy 0.95, ranks in [16, 128]) on matrices whose
    # spectrum puts 95% of the energy at ranks 37, 45 and 21: A is [d, 37],
    # groups straddle rows and the NF4 nibbles of a row start mid-byte.
    rng = np.random.default_rng(3)
    d, ff = 192, 160

    def spectral(rows, cols, knee, seed):
        g = np.random.default_rng(seed)
        u, _ = np.linalg.qr(g.standard_normal((rows, rows)))
        v, _ = np.linalg.qr(g.standard_normal((cols, cols)))
        n = min(rows, cols)
        s = np.where(np.arange(n) < knee, 1.0, 1e-3)
        return ((u[:, :n] * s) @ v[:, :n].T).astype(np.float32)

    # a flat spectrum of K ones reaches 95% of its energy at rank ceil(0.95 K)
    mats = {"gate": spectral(d, ff, 38, 1), "up": spectral(d, ff, 47, 2), "down": spectral(ff, d, 22, 3)}
    arrays, reports = _artifacts(mats, error_threshold=1.0)
    ranks = [reports[k]["rank"] for k in ("gate", "up", "down")]
    assert ranks == [37, 45, 21]
    x = rng.standard_normal((5, d)).astype(np.float32)
    want, got = _both(arrays, x)
    err = ref.rel_l2(want, got)
    print(f"CLI-default ranks {ranks} rel_l2={err:.3e}")
    assert err <= TOL
    # one token given as a 1-D vector, as the reference accepts
    one_want, one_got = _both(arrays, x[2])
    assert one_got.shape == (d,) and ref.rel_l2(one_want, one_got) <= TOL


def test_int8_group64_on_any_column_count(gpu):
    # Whole-factor INT8 at group 64 (loader/latent_runtime.py:26-27) on factors
    # with 30 and 37 columns: every 64-group straddles rows.
    mats = {"gate": _low_rank(40, 30, 37, 4), "up": _low_rank(40, 30, 37, 5), "down": _low_rank(30, 40, 37, 6)}
    arrays, reports = _artifacts(mats, energy=1.0, min_rank=30, max_rank=37, snr_threshold=np.inf,
                                 low_snr_fraction_threshold=0.0, error_threshold=1.0)
    assert all(r["quantization"] == "int8_g64" for r in reports.values())
    assert "gate.a.int8" in arrays and int(arrays["gate.a.shape"][1]) % 64 != 0
    x = np.random.default_rng(5).standard_normal((7, 40)).astype(np.float32)
    want, got = _both(arrays, x)
    err = ref.rel_l2(want, got)
    print(f"int8 g64 rel_l2={err:.3e}")
    assert err <= TOL


def test_mixed_nf4_and_int8_pairs_and_many_tokens(gpu):
    mats = {"gate": _low_rank(256, 96, 37, 7), "up": _low_rank(256, 96, 37, 8), "down": _low_rank(96, 256, 37, 9)}
    arrays, _ = _artifacts({"gate": mats["gate"], "down": mats["down"]}, energy=1.0, min_rank=37, max_rank=37,
                           error_threshold=1.0)
    up, rep = synth.compress_matrix("up", mats["up"], energy=1.0, min_rank=37, max_rank=37, snr_threshold=np.inf,
                                    low_snr_fraction_threshold=0.0, error_threshold=1.0)
    assert rep["quantization"] == "int8_g64"
    arrays.update(up)
    x = np.random.default_rng(6).standard_normal((300, 256)).astype(np.float32)  # several 8-token tiles
    for wbd in (False, True):
        want, got = _both(arrays, x, weight=0.5, wbd=wbd)
        assert ref.rel_l2(want, got) <= TOL


def test_weight_ignored_without_weight_before_down(gpu):
    mats = {"gate": _low_rank(64, 48, 5, 1), "up": _low_rank(64, 48, 5, 2), "down": _low_rank(48, 64, 5, 3)}
    arrays, _ = _artifacts(mats, energy=1.0, min_rank=5, max_rank=5, error_threshold=1.0)
    x = np.random.default_rng(7).standard_normal((2, 64)).astype(np.float32)
    _, g1 = _both(arrays, x, weight=1.0)
    _, g2 = _both(arrays, x, weight=0.1)
    assert np.array_equal(g1, g2)
    _, gw = _both(arrays, x, weight=0.1, wbd=True)
    assert ref.rel_l2(0.1 * g1, gw) <= 1e-5
