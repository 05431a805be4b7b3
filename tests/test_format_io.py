"""Stacked-factor GGUF writer / reader (latent_amd.gguf) without a GPU.

Pinned by: an independent header parse following the GGUF field order that
benchmarks/inspect_gguf_header.py:16-127 reads; the tensor names, recorded
shapes and types asserted by tests/test_write_latent_gguf.py:100-162; the
unpack semantics of tests/test_write_latent_gguf.py:210-252 (low nibble = even
column, codebook x scale per 32-group) checked against the oracle's decode;
byte-identical round trips including INT8 groups and ranks of 256 and 512.
"""

import struct

import numpy as np
import pytest

from oracle import latent_ref as ref
from oracle import synth

gguf = pytest.importorskip("latent_amd.gguf")  # imports torch + the built library (no GPU needed)


def _host_arrays(layer: ref.StackedLayer):
    out = {}
    for name in ref.FACTOR_NAMES:
        f = layer.factors[name]
        out[name] = f.codes
        out[name + "_s"] = f.scales.astype(np.float16)
        if f.int8 is not None:
            out[name + "_i8map"] = f.int8.bitmap
            out[name + "_i8off"] = f.int8.row_offset
            out[name + "_i8"] = f.int8.data.reshape(-1, 32)
    if layer.ranks is not None:
        out["ranks"] = layer.ranks.astype(np.int32)
    return out


@pytest.fixture(scope="module")
def layers():
    a = synth.make_layer(seed=3, n_expert=4, d=64, ff=96, max_rank=32)
    b = synth.make_layer(seed=4, n_expert=4, d=64, ff=96, max_rank=32, ranks=[32, 16, 8, 32], int8_fraction=0.2)
    return {0: a, 7: b}


@pytest.fixture(scope="module")
def written(tmp_path_factory, layers):
    path = tmp_path_factory.mktemp("gguf") / "latent.gguf"
    gguf.write_latent_gguf(path, {L: _host_arrays(l) for L, l in layers.items()}, max_rank=32,
                           metadata={"general.name": "unit-test"})
    return path


def _parse_header(path):
    """Independent header walk (magic, version, counts, KV records, tensor infos)."""
    data = open(path, "rb").read()
    assert data[:4] == b"GGUF"
    version, n_t, n_kv = struct.unpack_from("<IQQ", data, 4)
    pos = 24

    def s():
        nonlocal pos
        (n,) = struct.unpack_from("<Q", data, pos)
        pos += 8
        v = data[pos:pos + n].decode()
        pos += n
        return v

    kv = {}
    for _ in range(n_kv):
        k = s()
        (t,) = struct.unpack_from("<I", data, pos)
        pos += 4
        if t == 8:
            kv[k] = s()
        elif t == 4:
            (kv[k],) = struct.unpack_from("<I", data, pos)
            pos += 4
        else:
            raise AssertionError(f"unexpected KV type {t} for {k}")
    infos = {}
    for _ in range(n_t):
        name = s()
        (nd,) = struct.unpack_from("<I", data, pos)
        pos += 4
        dims = struct.unpack_from(f"<{nd}Q", data, pos)
        pos += 8 * nd
        t, off = struct.unpack_from("<IQ", data, pos)
        pos += 12
        infos[name] = (dims, t, off)
    return version, kv, infos, pos, data


def test_header_names_shapes_types(written, layers):
    version, kv, infos, end, _ = _parse_header(written)
    assert version == 3
    assert kv["latent.max_rank"] == 32 and kv["latent.group_size"] == 32
    assert kv["latent.quantization"] == "nf4_g32" and kv["latent.format_version"] == "1"
    assert kv["general.name"] == "unit-test"
    E, d, ff, R = 4, 64, 96, 32
    want = {"gate_a": (d, R), "gate_b": (R, ff), "up_a": (d, R), "up_b": (R, ff), "down_a": (ff, R), "down_b": (R, d)}
    for L in (0, 7):
        for name, (rows, cols) in want.items():
            dims, t, off = infos[f"blk.{L}.ffn_latent_{name}"]
            assert dims == (E, rows, cols // 2) and t == gguf.GGML_I8 and off % 32 == 0
            dims, t, _ = infos[f"blk.{L}.ffn_latent_{name}_s"]
            assert dims == (E, rows, cols // 32) and t == gguf.GGML_F16
        dims, t, _ = infos[f"blk.{L}.ffn_latent_ranks"]
        assert dims == (E, 3) and t == gguf.GGML_I32
    assert "blk.7.ffn_latent_gate_a_i8map" in infos and "blk.0.ffn_latent_gate_a_i8map" not in infos


def test_round_trip_bytes_and_decode(written, layers):
    g = gguf.read_latent_gguf(written)
    assert list(g.layers()) == [0, 7]
    for L, layer in layers.items():
        arrs = g.layer_arrays(L)
        for name in ref.FACTOR_NAMES:
            f = layer.factors[name]
            key = f"blk.{L}.ffn_latent_{name}"
            assert np.array_equal(arrs[key], f.codes)
            assert np.array_equal(arrs[key + "_s"].view(np.uint16), f.scales.astype(np.float16).view(np.uint16))
            ext = None
            if f.int8 is not None:
                ext = ref.Int8Groups(bitmap=arrs[key + "_i8map"], data=arrs[key + "_i8"].reshape(f.int8.data.shape),
                                     row_offset=arrs[key + "_i8off"])
                assert np.array_equal(ext.bitmap, f.int8.bitmap) and np.array_equal(ext.data, f.int8.data)
            for e in range(layer.n_expert):
                got = ref.unpack_rows_mixed(arrs[key], arrs[key + "_s"], ext, e)
                assert np.array_equal(got, f.expert(e))
        want_ranks = layer.ranks if layer.ranks is not None else None
        if want_ranks is not None:
            assert np.array_equal(arrs[f"blk.{L}.ffn_latent_ranks"], want_ranks)


def test_unpack_semantics_of_the_reference_test(written, layers):
    # tests/test_write_latent_gguf.py:221-245: codes[:, 0::2] = packed & 0x0F,
    # codes[:, 1::2] = packed >> 4, value = NF4_CODEBOOK[code] * scale per group.
    g = gguf.read_latent_gguf(written)
    arrs = g.layer_arrays(0)
    packed = arrs["blk.0.ffn_latent_gate_b"][2]
    scales = arrs["blk.0.ffn_latent_gate_b_s"][2]
    codes = np.empty((packed.shape[0], packed.shape[1] * 2), np.uint8)
    codes[:, 0::2] = packed & 0x0F
    codes[:, 1::2] = packed >> 4
    dec = np.empty(codes.shape, np.float32)
    for row in range(codes.shape[0]):
        for grp in range(scales.shape[1]):
            sl = slice(grp * 32, (grp + 1) * 32)
            dec[row, sl] = ref.NF4_CODEBOOK[codes[row, sl]] * np.float32(scales[row, grp])
    assert np.array_equal(dec, layers[0].factors["gate_b"].expert(2))


def test_reference_uint8_rank_table_and_wide_ranks(tmp_path):
    layer = synth.make_layer(seed=9, n_expert=2, d=64, ff=64, max_rank=32)
    arrays = _host_arrays(layer)
    arrays["ranks"] = np.array([[256, 512, 32], [7, 8, 9]], np.int32)  # uint8 would wrap 256 and 512 to 0
    p = tmp_path / "r.gguf"
    gguf.write_latent_gguf(p, {3: arrays}, max_rank=32)
    assert np.array_equal(gguf.read_latent_gguf(p).layer_arrays(3)["blk.3.ffn_latent_ranks"], arrays["ranks"])



def test_reference_written_rank_table(tmp_path):
    # The reference writes per_expert_ranks.T.astype(uint8) as I8 with recorded
    # dims (E, 3) (loader/write_latent_gguf.py:262-265, 432-436): the file bytes
    # are the C order of the (3, E) transpose, i.e. kind-major.  Build the
    # tensor exactly that way inside a file and read the table back.
    E = 5
    layer = synth.make_layer(seed=9, n_expert=E, d=64, ff=64, max_rank=32)
    arrays = _host_arrays(layer)
    p = tmp_path / "refranks.gguf"
    gguf.write_latent_gguf(p, {0: arrays}, max_rank=32)
    per_expert_ranks = np.array([[1, 2, 3], [4, 5, 6], [7, 8, 9], [10, 11, 12], [200, 16, 32]], np.uint8)
    table = per_expert_ranks.T.astype(np.uint8)  # what the reference hands to add_tensor
    assert table.shape == (3, E)
    file_bytes = table.tobytes(order="C")  # numpy writes a tensor's data in C order
    assert file_bytes[:E] == bytes([1, 4, 7, 10, 200])  # kind-major, not expert-major
    g = gguf.read_latent_gguf(p)
    name = "blk.0.ffn_latent_ranks"
    g.tensors[name] = gguf.TensorInfo(name, (E, 3), gguf.GGML_I8, 0)  # dims recorded reversed: (E, 3)
    g.arrays[name] = np.frombuffer(file_bytes, np.int8).reshape(E, 3)  # the reader's view of those bytes
    got = g.layer_arrays(0)[name]
    assert got.dtype == np.int32 and got.tolist() == per_expert_ranks.astype(np.int32).tolist()
    # and the ranks drive the forward as the oracle's own table does
    host = ref.StackedLayer(factors=layer.factors, d=64, ff=64, max_rank=32,
                            ranks=np.minimum(got, 32).astype(np.int32))
    rng = np.random.default_rng(3)
    x = rng.standard_normal((2, 64)).astype(np.float32)
    ids = np.array([[0, 4], [2, 1]], np.int32)
    w = np.full((2, 2), 0.5, np.float32)
    want = ref.moe_forward(x, ids, w, ref.StackedLayer(factors=layer.factors, d=64, ff=64, max_rank=32,
                                                        ranks=np.minimum(per_expert_ranks, 32).astype(np.int32)))
    assert np.array_equal(ref.moe_forward(x, ids, w, host), want)


def _with_reference_rank_table(g, layer_idx: int, per_expert_ranks: np.ndarray) -> None:
    """Replace a read file's rank table by the bytes the reference's writer
    produces: per_expert_ranks.T as uint8 recorded as I8 with dims (E, 3)."""
    E = per_expert_ranks.shape[0]
    name = f"blk.{layer_idx}.ffn_latent_ranks"
    file_bytes = per_expert_ranks.T.astype(np.uint8).tobytes(order="C")
    g.tensors[name] = gguf.TensorInfo(name, (E, 3), gguf.GGML_I8, 0)
    g.arrays[name] = np.frombuffer(file_bytes, np.int8).reshape(E, 3)


def test_reference_rank_table_dropped_above_255(tmp_path):
    # At max_rank 256 the reference's uint8 table stores a rank of 256 as 0:
    # the table is ambiguous there, so the reader drops it (the factors are
    # zero-padded to max_rank, so max_rank is exact); at max_rank 32 it is kept.
    layer = synth.make_layer(seed=11, n_expert=3, d=256, ff=256, max_rank=256)
    p = tmp_path / "wide.gguf"
    arrays = _host_arrays(layer)
    gguf.write_latent_gguf(p, {0: arrays}, max_rank=256)
    g = gguf.read_latent_gguf(p)
    _with_reference_rank_table(g, 0, np.array([[256, 256, 256], [128, 64, 256], [256, 200, 32]]))
    got = g.layer_arrays(0)
    assert "blk.0.ffn_latent_ranks" not in got
    assert np.array_equal(got["blk.0.ffn_latent_gate_a"], arrays["gate_a"])

    small = synth.make_layer(seed=12, n_expert=2, d=64, ff=64, max_rank=32)
    p2 = tmp_path / "narrow.gguf"
    gguf.write_latent_gguf(p2, {0: _host_arrays(small)}, max_rank=32)
    g2 = gguf.read_latent_gguf(p2)
    _with_reference_rank_table(g2, 0, np.array([[32, 16, 8], [0, 32, 32]]))
    assert g2.layer_arrays(0)["blk.0.ffn_latent_ranks"].tolist() == [[32, 16, 8], [0, 32, 32]]


def test_writer_rejects_bad_operands(tmp_path):
    layer = synth.make_layer(seed=9, n_expert=2, d=64, ff=64, max_rank=32)
    arrays = _host_arrays(layer)
    arrays["gate_a_s"] = arrays["gate_a_s"][:, :-1, :]
    with pytest.raises(ValueError):
        gguf.write_latent_gguf(tmp_path / "bad.gguf", {0: arrays}, max_rank=32)
    arrays = _host_arrays(layer)
    arrays["up_b_i8map"] = np.zeros((2, 32, 1), np.uint32)
    with pytest.raises(ValueError):
        gguf.write_latent_gguf(tmp_path / "bad2.gguf", {0: arrays}, max_rank=32)


def test_truncated_file_is_rejected(written, tmp_path):
    data = open(written, "rb").read()
    p = tmp_path / "trunc.gguf"
    p.write_bytes(data[: len(data) - 100])
    with pytest.raises(ValueError):
        gguf.read_latent_gguf(p)
