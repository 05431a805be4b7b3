"""Pins the oracle's NF4 / INT8 codec (loader/latent_loader.py:28-48, 111-170).

Each check is independent of the oracle's own formula: a published
construction of the NF4 levels, known answers, brute force in pure Python,
and the reference test's own tolerance check.
"""

import math
import struct

import numpy as np
import pytest
from scipy.stats import norm

from oracle import latent_ref as ref


# -- codebook ------------------------------------------------------------------
def test_codebook_matches_normal_float_construction():
    # NF4 (Dettmers et al. 2023): 8 positive and 7 negative N(0,1) quantiles
    # between offset 0.9677083 and 0.5, plus an exact zero, scaled to [-1, 1].
    offset = 0.9677083
    pos = norm.ppf(np.linspace(offset, 0.5, 9)[:-1])
    neg = -norm.ppf(np.linspace(offset, 0.5, 8)[:-1])
    levels = np.sort(np.concatenate([pos, neg, [0.0]]))
    levels = levels / levels.max()
    assert ref.NF4_CODEBOOK.dtype == np.float32 and ref.NF4_CODEBOOK.shape == (16,)
    np.testing.assert_allclose(ref.NF4_CODEBOOK, levels, rtol=0, atol=5e-7)
    assert ref.NF4_CODEBOOK[7] == 0.0 and ref.NF4_CODEBOOK[0] == -1.0 and ref.NF4_CODEBOOK[15] == 1.0


# -- brute force quantizer ---------------------------------------------------------
def _bf_quantize_nf4(values, group_size):
    """Element-by-element restatement in plain Python with np.float32 scalars."""
    flat = [np.float32(v) for v in np.asarray(values, dtype=np.float32).reshape(-1)]
    groups = math.ceil(len(flat) / group_size)
    flat += [np.float32(0.0)] * (groups * group_size - len(flat))
    codes, scales = [], []
    for g in range(groups):
        grp = flat[g * group_size:(g + 1) * group_size]
        s = np.float32(0.0)
        for v in grp:
            s = max(s, np.float32(abs(v)))
        if s == 0:
            s = np.float32(1.0)
        scales.append(s)
        for v in grp:
            n = np.float32(v / s)
            best, bestd = 0, None
            for c in range(16):
                d = np.float32(abs(np.float32(n - ref.NF4_CODEBOOK[c])))
                if bestd is None or d < bestd:
                    best, bestd = c, d
            codes.append(best)
    if len(codes) % 2:
        codes.append(7)
    packed = bytes(codes[i] | (codes[i + 1] << 4) for i in range(0, len(codes), 2))
    return np.frombuffer(packed, dtype=np.uint8), np.array(scales, dtype=np.float32).astype(np.float16)


def _tie_values():
    cb = ref.NF4_CODEBOOK.astype(np.float64)
    mids = (cb[:-1] + cb[1:]) / 2
    vals = np.concatenate([cb, mids, mids + 1e-8, mids - 1e-8, [1.0]])
    return vals.astype(np.float32)


@pytest.mark.parametrize("group_size", [32, 16, 7])
def test_quantize_nf4_matches_brute_force(group_size):
    rng = np.random.default_rng(5)
    vals = np.concatenate([
        _tie_values(),
        rng.standard_normal(301).astype(np.float32) * 1e-3,
        np.zeros(40, np.float32),
        np.array([3e-8, -6e-5, 7e4, -1e-40], np.float32),
    ])
    packed, scales, shape = ref.quantize_nf4(vals, group_size=group_size)
    bp, bs = _bf_quantize_nf4(vals, group_size)
    assert shape == vals.shape
    np.testing.assert_array_equal(packed, bp)
    np.testing.assert_array_equal(scales.view(np.uint16), bs.view(np.uint16))


def test_quantize_nf4_known_answers():
    s = np.float32(0.5)
    codes = np.array([0, 15, 7, 3, 12, 9, 1, 14] * 4)
    vals = ref.NF4_CODEBOOK[codes] * s
    vals[1] = s  # ensure absmax == s
    packed, scales, _ = ref.quantize_nf4(vals)
    assert scales.dtype == np.float16 and float(scales[0]) == 0.5
    unpacked = np.empty(32, np.uint8)
    unpacked[0::2], unpacked[1::2] = packed & 15, packed >> 4
    np.testing.assert_array_equal(unpacked, codes)
    # low nibble holds the even element
    p2, _, _ = ref.quantize_nf4(np.array([-1.0, 1.0], np.float32))
    assert p2.tolist() == [0xF0] + [0x77] * 15  # zero padding of the group quantizes to code 7
    # an all-zero group gets scale 1.0 and code 7; an odd code count pads with code 7
    p3, s3, _ = ref.quantize_nf4(np.zeros(3, np.float32))
    assert s3.tolist() == [1.0] and p3.tolist() == [0x77] * 16
    p4, _, _ = ref.quantize_nf4(np.array([1.0, -1.0, 1.0], np.float32), group_size=3)
    assert p4.tolist() == [0x0F, 0x7F]


def test_fp16_scale_rounding_is_nearest_even():
    def f16_bits(x):
        return struct.unpack("<H", struct.pack("<e", x))[0]  # IEEE binary16, ties to even

    xs = [1.0 + 2.0**-11, 1.0 + 3 * 2.0**-11, 65504.0, 65520.0, 6.1e-5, 5.96e-8, 2.0**-25, 3.0 * 2.0**-25, 1e-3]
    for x in xs:
        _, s, _ = ref.quantize_nf4(np.array([x] + [0.0] * 31, np.float32))
        x32 = float(np.float32(x))
        try:
            want = f16_bits(x32)
        except OverflowError:
            want = 0x7C00
        assert int(s.view(np.uint16)[0]) == want, x


def test_dequantize_nf4_known_answers():
    packed = np.arange(256, dtype=np.uint8)
    for scale in (1.0, 0.5, 2.0**-20, 65504.0):
        scales = np.full(16, scale, dtype=np.float16)
        out = ref.dequantize_nf4(packed, scales, (512,))
        lo, hi = packed & 15, packed >> 4
        want = np.empty(512, np.float32)
        want[0::2] = ref.NF4_CODEBOOK[lo] * np.float32(np.float16(scale))
        want[1::2] = ref.NF4_CODEBOOK[hi] * np.float32(np.float16(scale))
        np.testing.assert_array_equal(out.view(np.uint32), want.view(np.uint32))
    # codes 0..15 at scale 1.0 decode to the codebook itself
    pk = np.array([c | (c << 4) for c in range(16)], np.uint8)
    out = ref.dequantize_nf4(pk, np.ones(1, np.float16), (32,))
    np.testing.assert_array_equal(out[0::2], ref.NF4_CODEBOOK)


def test_nf4_roundtrip_reference_tolerance():
    # tests/test_latent_loader.py:33-38
    values = np.linspace(-2.0, 2.0, 133, dtype=np.float32).reshape(7, 19)
    packed, scales, shape = ref.quantize_nf4(values, group_size=16)
    restored = ref.dequantize_nf4(packed, scales, shape, group_size=16)
    assert restored.shape == values.shape
    assert ref.relative_frobenius_error(values, restored) < 0.12


def test_nf4_roundtrip_error_bound():
    # |x - dq(q(x))| <= half the widest codebook gap times the group scale (+ fp16 scale rounding)
    rng = np.random.default_rng(0)
    x = rng.standard_normal((64, 96)).astype(np.float32)
    packed, scales, shape = ref.quantize_nf4(x)
    y = ref.dequantize_nf4(packed, scales, shape)
    gap = np.max(np.diff(ref.NF4_CODEBOOK.astype(np.float64))) / 2
    s = np.abs(x).reshape(-1, 32).max(axis=1)
    bound = (gap * s * (1 + 2**-10) + s * 2**-11)[:, None]
    assert np.all(np.abs((x - y).reshape(-1, 32)) <= bound)


# -- INT8 ------------------------------------------------------------------------
def test_int8_known_answers():
    s = np.float32(127.0) / np.float32(127.0)
    vals = np.array([127.0, -127.0, 0.0, 0.5, 1.5, 2.5, -0.5, -1.5] + [0.0] * 24, np.float32)
    q, scales, _ = ref.quantize_int8(vals, group_size=32)
    assert float(scales[0]) == float(np.float16(s))
    # np.rint rounds half to even
    assert q[:8].tolist() == [127, -127, 0, 0, 2, 2, 0, -2]
    q0, s0, _ = ref.quantize_int8(np.zeros(32, np.float32), group_size=32)
    assert float(s0[0]) == 1.0 and not q0.any()
    out = ref.dequantize_int8(np.array([-127, 0, 5, 127] * 8, np.int8), np.array([0.25], np.float16), (32,), 32)
    assert out[:4].tolist() == [-31.75, 0.0, 1.25, 31.75]


def test_int8_matches_brute_force():
    rng = np.random.default_rng(3)
    vals = (rng.standard_normal(160) * rng.choice([1e-4, 1.0, 30.0], 160)).astype(np.float32)
    q, scales, _ = ref.quantize_int8(vals, group_size=32)
    for g in range(5):
        grp = vals[g * 32:(g + 1) * 32]
        s = np.float32(max(abs(float(v)) for v in grp)) / np.float32(127.0)
        s = np.float32(1.0) if s == 0 else np.float32(s)
        want = [int(max(-127, min(127, np.rint(np.float32(v / s))))) for v in grp]
        assert q[g * 32:(g + 1) * 32].tolist() == want
        assert scales[g] == np.float16(s)
