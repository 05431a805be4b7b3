"""GPU codec parity: unpack bit-exact, pack byte-exact against the oracle.

loader/latent_loader.py:111-170; per-row layout loader/write_latent_gguf.py:227-257.
"""

import numpy as np
import pytest

from oracle import latent_ref as ref

pytestmark = pytest.mark.gpu


def _rand_scales(rng, shape):
    s = np.abs(rng.standard_normal(shape)) * rng.choice([1e-6, 1e-3, 1.0, 300.0], shape)
    s = s.astype(np.float16)
    s.reshape(-1)[:4] = np.array([6e-8, 6.1e-5, 65504.0, 1.0], np.float16)  # subnormal, min normal, max
    return s


def test_unpack_nf4_bit_exact(gpu):
    import torch

    rng = np.random.default_rng(0)
    E, rows, cols = 3, 48, 256
    codes = rng.integers(0, 256, (E, rows, cols // 2), dtype=np.uint8)
    codes[0, 0, :] = np.arange(128, dtype=np.uint8)  # every byte value appears
    codes[0, 1, :] = np.arange(128, 256, dtype=np.uint8)
    scales = _rand_scales(rng, (E, rows, cols // 32))
    f = gpu.DeviceFactor.from_numpy(codes, scales)
    for e in range(E):
        got = gpu.unpack(f, e).cpu().numpy()
        want = ref.unpack_rows(codes[e], scales[e])
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    torch.cuda.synchronize()


def test_unpack_int8_groups_bit_exact(gpu):
    rng = np.random.default_rng(1)
    st = (rng.standard_normal((2, 40, 128)) * 1e-2).astype(np.float32)
    mask = rng.random((2, 40, 4)) < 0.3
    codes, scales, ext = ref.pack_rows_mixed(st, mask)
    f = gpu.DeviceFactor.from_numpy(codes, scales, (ext.bitmap, ext.row_offset, ext.data))
    for e in range(2):
        got = gpu.unpack(f, e).cpu().numpy()
        want = ref.unpack_rows_mixed(codes, scales, ext, e)
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def _special_rows(rng, rows, cols):
    v = (rng.standard_normal((rows, cols)) * 1e-3).astype(np.float32)
    cb = ref.NF4_CODEBOOK.astype(np.float64)
    mids = ((cb[:-1] + cb[1:]) / 2).astype(np.float32)
    v[0, :15] = mids  # ties between adjacent levels (group absmax set below)
    v[0, 15] = 1.0
    v[0, 16:31] = np.nextafter(mids, np.float32(2.0))
    v[1, :32] = 0.0  # all-zero group -> scale 1, code 7
    v[2, :32] = np.float32(7e4)  # fp16 scale overflow -> inf
    v[3, :32] = np.float32(3e-8)  # fp16 subnormal scale
    v[4, :32] = ref.NF4_CODEBOOK[np.arange(32) % 16] * np.float32(0.37)
    return v


def test_pack_nf4_byte_exact(gpu):
    import torch

    rng = np.random.default_rng(2)
    v = _special_rows(rng, 96, 512)
    codes, scales = gpu.pack_nf4(torch.from_numpy(v).cuda())
    want_c, want_s = ref.pack_rows(v)
    np.testing.assert_array_equal(codes.cpu().numpy(), want_c)
    np.testing.assert_array_equal(scales.cpu().numpy().view(np.uint16), want_s.view(np.uint16))


def test_pack_int8_byte_exact(gpu):
    import torch

    rng = np.random.default_rng(3)
    g = (rng.standard_normal((300, 32)) * rng.choice([1e-5, 1.0, 50.0], (300, 1))).astype(np.float32)
    g[0] = 0.0
    g[1, :] = np.arange(32) - 15.5  # x.5 multiples of the scale: round half to even
    q, s = gpu.pack_int8(torch.from_numpy(g).cuda())
    wq, ws, _ = ref.quantize_int8(g, group_size=32)
    np.testing.assert_array_equal(q.cpu().numpy().reshape(-1), wq)
    np.testing.assert_array_equal(s.cpu().numpy().view(np.uint16), ws.view(np.uint16))


def test_pack_then_unpack_roundtrip_matches_oracle(gpu):
    import torch

    rng = np.random.default_rng(4)
    v = (rng.standard_normal((4, 64, 256)) * 3e-3).astype(np.float32)
    codes, scales = gpu.pack_nf4(torch.from_numpy(v).cuda())
    f = gpu.DeviceFactor(codes, scales)
    want = ref.unpack_rows(*ref.pack_rows(v))
    for e in range(4):
        np.testing.assert_array_equal(gpu.unpack(f, e).cpu().numpy().view(np.uint32), want[e].view(np.uint32))
