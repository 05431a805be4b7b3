"""Pins the oracle's runtime, stacked layout and layer forward.

loader/latent_runtime.py:13-73, loader/write_latent_gguf.py:101-123, 227-257.
Checks: float64 dense algebra on the dequantized factors, the reference tests'
own properties, literal per-row loops of the writer, and brute-force loops
over (token, slot).
"""

import math

import numpy as np
import pytest
from scipy.special import expit

from oracle import latent_ref as ref
from oracle import routing, synth


def test_silu_closed_form():
    x = np.array([-1e4, -100.0, -10.0, -1.0, -1e-6, 0.0, 1e-6, 0.5, 3.0, 80.0, 1e4], np.float32)
    want = (x.astype(np.float64) * expit(x.astype(np.float64))).astype(np.float32)
    np.testing.assert_allclose(ref.silu(x), want, rtol=1e-6, atol=1e-30)
    assert ref.silu(np.array([np.float32(3e38)]))[0] == np.float32(1e30)  # clip at +-1e30


def _pairs(rng, d, ff, r):
    out = []
    for n_in, n_out in ((d, ff), (d, ff), (ff, d)):
        a, b = synth.closed_form_factors(rng, n_in, n_out, r)
        out.append(ref.FactorPair(a, b))
    return out


def test_swiglu_expert_matches_float64_dense():
    rng = np.random.default_rng(1)
    gate, up, down = _pairs(rng, 96, 64, 32)
    x = rng.standard_normal((5, 96)).astype(np.float32)
    y = ref.swiglu_expert(x, gate, up, down)
    x64 = x.astype(np.float64)
    g = x64 @ (gate.a.astype(np.float64) @ gate.b)
    u = x64 @ (up.a.astype(np.float64) @ up.b)
    h = g / (1 + np.exp(-g)) * u
    want = h @ (down.a.astype(np.float64) @ down.b)
    assert ref.rel_l2(want, y) < 1e-5


def test_weight_semantics():
    # tests/test_latent_loader.py:130-141 (before == after * w) and the reference's
    # behaviour of ignoring `weight` when it is applied after down.
    rng = np.random.default_rng(2)
    gate, up, down = _pairs(rng, 64, 32, 32)
    x = rng.standard_normal((2, 64)).astype(np.float32)
    before = ref.swiglu_expert(x, gate, up, down, weight=0.25, weight_before_down=True)
    plain = ref.swiglu_expert(x, gate, up, down)
    np.testing.assert_allclose(before, plain * np.float32(0.25), rtol=1e-5, atol=1e-12)
    np.testing.assert_array_equal(ref.swiglu_expert(x, gate, up, down, weight=7.0), plain)


def test_load_pair_npz_keys_and_missing():
    arrays, dense, x = synth.config0_expert(seed=3, d=128, ff=96, rank=32)
    pair = ref.load_pair(arrays, "gate")
    assert pair.a.shape == (128, 32) and pair.b.shape == (32, 96)
    with pytest.raises(KeyError):
        ref.load_pair(arrays, "missing")
    # INT8 keys (group 64) are decoded too
    q, s, shape = ref.quantize_int8(pair.a, group_size=64)
    arrays2 = dict(arrays)
    del arrays2["gate.a.nf4"]
    arrays2["gate.a.int8"], arrays2["gate.a.scales"] = q, s
    np.testing.assert_array_equal(ref.load_pair(arrays2, "gate").a, ref.dequantize_int8(q, s, shape, 64))


def test_config0_latent_vs_dense_fidelity():
    arrays, dense, x = synth.config0_expert(seed=0)
    latent = ref.swiglu_expert(x, ref.load_pair(arrays, "gate"), ref.load_pair(arrays, "up"), ref.load_pair(arrays, "down"))
    full = ref.dense_swiglu_expert(x, dense["gate"], dense["up"], dense["down"])
    err = ref.relative_frobenius_error(full, latent)
    assert np.isfinite(err) and err < 1.5  # noise norm exceeds the signal's at this config; report item


def test_pack_rows_matches_writer_row_loop():
    # loader/write_latent_gguf.py:227-257: quantize each row on its own, pad the
    # last axis to a group multiple, pad bytes 0x77 and scales 1.0.
    rng = np.random.default_rng(4)
    st = rng.standard_normal((2, 5, 40)).astype(np.float32) * 1e-3
    codes, scales = ref.pack_rows(st)
    assert codes.shape == (2, 5, 32) and scales.shape == (2, 5, 2)
    for e in range(2):
        for r in range(5):
            row = np.pad(st[e, r], (0, 24))
            p, s, _ = ref.quantize_nf4(row, group_size=32)
            np.testing.assert_array_equal(codes[e, r], p)
            np.testing.assert_array_equal(scales[e, r].view(np.uint16), s.view(np.uint16))
    np.testing.assert_array_equal(ref.unpack_rows(codes, scales)[..., :40].reshape(-1),
                                  ref.dequantize_nf4(codes.reshape(-1), scales.reshape(-1), (2 * 5 * 64,))
                                  .reshape(2, 5, 64)[..., :40].reshape(-1))


def test_mixed_int8_groups_decode():
    rng = np.random.default_rng(5)
    st = rng.standard_normal((2, 3, 64)).astype(np.float32)
    mask = np.zeros((2, 3, 2), bool)
    mask[0, 1, 1] = mask[1, 0, 0] = mask[1, 2, 1] = True
    codes, scales, ext = ref.pack_rows_mixed(st, mask)
    plain_c, plain_s = ref.pack_rows(st)
    for e in range(2):
        out = ref.unpack_rows_mixed(codes, scales, ext, e)
        for r in range(3):
            for g in range(2):
                seg = slice(32 * g, 32 * g + 32)
                if mask[e, r, g]:
                    q, s, _ = ref.quantize_int8(st[e, r, seg], group_size=32)
                    np.testing.assert_array_equal(out[r, seg], ref.dequantize_int8(q, s, (32,), 32))
                else:
                    want = ref.dequantize_nf4(plain_c[e, r, 16 * g:16 * g + 16], plain_s[e, r, g:g + 1], (32,))
                    np.testing.assert_array_equal(out[r, seg], want)
    assert ext.row_offset.tolist() == [[0, 0, 1], [1, 2, 2]]


def _brute_force_moe(x, ids, w, layer, wbd, mode):
    T, K = ids.shape
    per = np.zeros((T, K, layer.d), np.float32)
    for t in range(T):
        for k in range(K):
            e = int(ids[t, k])
            if 0 <= e < layer.n_expert:
                gate, up, down = layer.pairs(e)
                per[t, k] = ref.swiglu_expert(x[t:t + 1], gate, up, down, weight=w[t, k], weight_before_down=wbd)[0]
    if mode == 1:
        return per
    scale = np.where((ids >= 0) & (ids < layer.n_expert), 1.0 if wbd else w, 0.0)
    return (per.astype(np.float64) * scale[..., None]).sum(axis=1)


@pytest.mark.parametrize("wbd", [False, True])
@pytest.mark.parametrize("mode", [0, 1])
def test_moe_forward_matches_brute_force(wbd, mode):
    layer = synth.make_layer(seed=10, n_expert=6, d=64, ff=96, max_rank=32, ranks=[32, 32, 17, 32, 9, 32])
    rng = np.random.default_rng(6)
    x = rng.standard_normal((5, 64)).astype(np.float32)
    ids, w = routing.softmax_topk(rng.standard_normal((5, 6)), 3)
    ids[1, 2] = -1
    ids[3, 0] = 99  # out of range -> dropped
    got = ref.moe_forward(x, ids, w, layer, weight_before_down=wbd, out_mode=mode)
    want = _brute_force_moe(x, ids, w, layer, wbd, mode)
    assert ref.rel_l2(want, got) < 1e-5
    if mode == 1:
        assert not got[1, 2].any() and not got[3, 0].any()


def test_padding_beyond_rank_is_exact_zero():
    layer = synth.make_layer(seed=11, n_expert=2, d=64, ff=64, max_rank=64, ranks=[32, 64])
    gate_a = layer.factors["gate_a"].expert(0)
    assert not gate_a[:, 32:].any() and not layer.factors["down_b"].expert(0)[32:].any()


def test_expert_bytes_config1_shape():
    # 3,981,312 packed bytes per expert at d=7168, ff=2048, r=256 (NF4 + fp16 scales)
    d, ff, r = 7168, 2048, 256
    elems = 2 * d * r + 2 * r * ff + ff * r + r * d
    assert elems // 2 + elems // 32 * 2 == 3_981_312
    layer = synth.make_layer(seed=12, n_expert=1, d=64, ff=32, max_rank=32)
    elems = 2 * 64 * 32 + 2 * 32 * 32 + 32 * 32 + 32 * 64
    assert layer.expert_bytes(0) == elems // 2 + elems // 32 * 2


def test_softmax_topk_brute_force():
    rng = np.random.default_rng(7)
    logits = rng.standard_normal((9, 12)).astype(np.float32)
    ids, w = routing.softmax_topk(logits, 4)
    for t in range(9):
        p = np.exp(logits[t].astype(np.float64))
        p /= p.sum()
        order = sorted(range(12), key=lambda e: (-p[e], e))[:4]
        assert ids[t].tolist() == order
        np.testing.assert_allclose(w[t], p[order] / p[order].sum(), rtol=1e-6)


def test_adaptive_topk_reference_cases():
    # tests/test_adaptive_topk.py:14-59
    s = np.array([0.45, 0.22, 0.15, 0.08, 0.05, 0.03], np.float32)
    assert routing.adaptive_topk_inclusive(s, 0.95) == 4
    assert routing.adaptive_topk_inclusive(s, 1.0) == 6
    assert routing.adaptive_topk_inclusive(s, 0.1) == 0
    assert routing.adaptive_topk_inclusive(np.zeros(6, np.float32), 0.95) == 0
    assert routing.adaptive_topk_inclusive(np.array([], np.float32), 0.95) == 0
    ids, w = routing.adaptive_drop(np.array([[3, 1, 2]]), np.array([[0.7, 0.26, 0.04]], np.float32), 0.05)
    assert ids.tolist() == [[3, 1, -1]] and w.tolist()[0][2] == 0.0


def test_inclusive_drop_matches_per_token_rule():
    # adaptive_topk_batch (loader/adaptive_topk.py:58-90) keeps a prefix of the
    # descending scores whose length is adaptive_topk_inclusive of that row.
    w = np.array([[0.45, 0.22, 0.15, 0.08, 0.05, 0.03], [0.9, 0.05, 0.03, 0.01, 0.005, 0.005]], np.float32)
    ids = np.arange(12, dtype=np.int32).reshape(2, 6)
    got_ids, got_w = routing.inclusive_drop(ids, w, 0.95)
    assert got_ids.tolist() == [[0, 1, 2, 3, -1, -1], [6, -1, -1, -1, -1, -1]]
    assert got_w[0, 4] == 0.0 and got_w[1, 1:].sum() == 0.0 and got_w[0, 3] == w[0, 3]


def test_route_drop_rules_and_logits():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((5, 16))
    W = rng.standard_normal((16, 10))
    lg = routing.router_logits(x, W)
    np.testing.assert_allclose(lg[2, 7], sum(x[2, i] * W[i, 7] for i in range(16)), rtol=1e-12)
    ids, w = routing.route(lg, 4, "below", 0.2)
    base_ids, base_w = routing.softmax_topk(lg, 4)
    assert np.all((ids == -1) == (base_w < np.float32(0.2)))
    assert np.all(w[ids >= 0] == base_w[ids >= 0])
    with pytest.raises(ValueError):
        routing.route(lg, 4, "bogus")


# ----------------------------------------------------------------------------
# quantization_snr_by_group / compress_matrix / int8_group_mask
# ----------------------------------------------------------------------------
def test_snr_by_group_known_answers():
    x = np.zeros(70, np.float32)
    x[:32] = 3.0                      # group 0: noise = signal / 2 exactly
    x[32:64] = np.linspace(-1, 1, 32)  # group 1: exact reconstruction
    x[64:] = 4.0                      # group 2: 6 values, zero-padded to 32
    cand = x.copy()
    cand[:32] = 1.5
    cand[64:] = 2.0
    snr = ref.quantization_snr_by_group(x, cand, 32)
    assert snr.shape == (3,)
    assert snr[0] == pytest.approx(2.0, rel=1e-6)
    assert snr[1] == pytest.approx(np.linalg.norm(x[32:64]) / 1e-12, rel=1e-6)  # noise floor 1e-12
    assert snr[2] == pytest.approx(2.0, rel=1e-6)  # ||4|| / ||2|| over the 6 real values; the pad adds zeros
    # scale invariance and shape independence (flat groups cross rows)
    assert np.allclose(ref.quantization_snr_by_group(5 * x, 5 * cand, 32)[[0, 2]], snr[[0, 2]], rtol=1e-6)
    assert np.array_equal(ref.quantization_snr_by_group(x.reshape(7, 10), cand.reshape(7, 10), 32), snr)


def test_snr_by_group_brute_force():
    rng = np.random.default_rng(8)
    x = rng.standard_normal((9, 29)).astype(np.float32)
    q = x + 0.01 * rng.standard_normal(x.shape).astype(np.float32)
    flat, fq = x.reshape(-1).tolist(), q.reshape(-1).tolist()
    want = []
    for g in range(0, len(flat), 32):
        s = math.sqrt(sum(v * v for v in flat[g:g + 32]))
        n = math.sqrt(sum((a - b) ** 2 for a, b in zip(flat[g:g + 32], fq[g:g + 32])))
        want.append(s / max(n, 1e-12))
    assert np.allclose(ref.quantization_snr_by_group(x, q, 32), want, rtol=1e-5)


def _low_rank(rows, cols, rank, seed):
    rng = np.random.default_rng(seed)
    return rng.standard_normal((rows, rank), dtype=np.float32) @ rng.standard_normal((rank, cols), dtype=np.float32)


def test_compress_matrix_matches_the_reference_tests():
    # tests/test_latent_loader.py:41-62
    arrays, rep = synth.compress_matrix("blk.0.ffn_gate.0", _low_rank(64, 48, 8, 123), energy=0.999, min_rank=4,
                                        max_rank=16, group_size=32, int8_group_size=64, error_threshold=0.35,
                                        snr_threshold=0.0, low_snr_fraction_threshold=1.0, seed=7)
    assert rep["rank"] >= 8 and rep["dense_relative_error"] < 1e-4 and rep["quantized_relative_error"] < 0.35
    assert not rep["fallback"] and "blk.0.ffn_gate.0.a.nf4" in arrays
    assert "blk.0.ffn_gate.0.dense_fallback" not in arrays
    # tests/test_latent_loader.py:100-127: the artifact's swiglu stays within 0.35 of the dense one
    rng = np.random.default_rng(99)
    x = rng.standard_normal((3, 16), dtype=np.float32)
    mats = {"gate": _low_rank(16, 12, 4, 1), "up": _low_rank(16, 12, 4, 2), "down": _low_rank(12, 16, 4, 3)}
    arrays = {}
    for name, m in mats.items():
        a, r = synth.compress_matrix(name, m, energy=0.999, min_rank=4, max_rank=8, error_threshold=1.0,
                                     snr_threshold=0.0, low_snr_fraction_threshold=1.0, seed=10)
        assert not r["fallback"]
        arrays.update(a)
    latent = ref.swiglu_expert(x, ref.load_pair(arrays, "gate"), ref.load_pair(arrays, "up"), ref.load_pair(arrays, "down"))
    dense = ref.dense_swiglu_expert(x, mats["gate"], mats["up"], mats["down"])
    assert ref.relative_frobenius_error(dense, latent) < 0.35


def test_compress_matrix_int8_and_dense_fallbacks():
    m = _low_rank(40, 30, 37, 4)
    # every group below an infinite SNR threshold: the pair goes INT8 at group 64 when that is better
    arrays, rep = synth.compress_matrix("w", m, energy=1.0, min_rank=30, max_rank=30, snr_threshold=np.inf,
                                        low_snr_fraction_threshold=0.0, error_threshold=1.0)
    assert rep["quantization"] == "int8_g64" and "w.a.int8" in arrays and "w.a.nf4" not in arrays
    assert arrays["w.a.scales"].size == -(-40 * 30 // 64)
    aq = ref.load_factor(arrays, "w", "a")
    assert aq.shape == (40, 30) and ref.relative_frobenius_error(m, aq @ ref.load_factor(arrays, "w", "b")) < 0.05
    # an error threshold nothing can meet adds the fp16 dense copy
    arrays, rep = synth.compress_matrix("w", m, energy=0.5, min_rank=1, max_rank=2, error_threshold=0.0)
    assert rep["fallback"] and arrays["w.dense_fallback"].dtype == np.float16


def test_int8_group_mask_brute_force():
    rng = np.random.default_rng(21)
    v = (rng.standard_normal((6, 96)) * np.exp(rng.standard_normal((6, 96)))).astype(np.float32)
    v[2, 32:64] = 0.0  # an all-zero group is never selected
    for thr in (5.0, 12.0, 20.0):
        mask = ref.int8_group_mask(v, thr)
        for r in range(6):
            for g in range(3):
                grp = v[r, 32 * g:32 * (g + 1)]
                packed, scales, shape = ref.quantize_nf4(grp, group_size=32)
                dec = ref.dequantize_nf4(packed, scales, shape, group_size=32)
                snr = np.linalg.norm(grp) / max(np.linalg.norm(grp - dec), 1e-12)
                assert mask[r, g] == (snr < thr and np.abs(grp).max() > 0), (thr, r, g)
    assert ref.int8_group_mask(v, 1e9).sum() == 6 * 3 - 1


def test_mixed_decode_matches_a_per_group_walk():
    # 64 groups per row (two bitmap words), random flags: the vectorised decode
    # against a walk over each row's groups that counts flagged groups in order.
    rng = np.random.default_rng(17)
    st = rng.standard_normal((3, 5, 2048)).astype(np.float32)
    mask = rng.random((3, 5, 64)) < 0.3
    codes, scales, ext = ref.pack_rows_mixed(st, mask)
    for e in range(3):
        got = ref.unpack_rows_mixed(codes, scales, ext, e)
        want = ref.unpack_rows(codes[e], scales[e])
        for r in range(5):
            n = 0
            for g in range(64):
                if (int(ext.bitmap[e, r, g // 32]) >> (g % 32)) & 1:
                    q = ext.data[int(ext.row_offset[e, r]) + n].astype(np.float32)
                    want[r, 32 * g:32 * g + 32] = q * np.float32(scales[e, r, g])
                    n += 1
            assert n == mask[e, r].sum()
        np.testing.assert_array_equal(got, want)


def test_int8_subset_rebases_offsets():
    from tests._layers import _int8_subset

    class Dev:  # the fields of a device factor, as host arrays with a .cpu().numpy() chain
        def __init__(self, a):
            self.a = a

        def cpu(self):
            return self

        def numpy(self):
            return self.a

    rng = np.random.default_rng(3)
    st = rng.standard_normal((4, 6, 96)).astype(np.float32)
    mask = rng.random((4, 6, 3)) < 0.4
    codes, scales, ext = ref.pack_rows_mixed(st, mask)
    f = type("F", (), {})()
    f.int8_bitmap, f.int8_row_offset, f.int8_data = Dev(ext.bitmap.view(np.int32)), Dev(ext.row_offset), Dev(ext.data)
    sub = _int8_subset(f, np.array([3, 1]))
    for j, e in enumerate((3, 1)):
        np.testing.assert_array_equal(ref.unpack_rows_mixed(codes[[3, 1]], scales[[3, 1]], sub, j),
                                      ref.unpack_rows_mixed(codes, scales, ext, e))
