"""Stacked LATENT factors in a GGUF container: writer and memory-mapped reader.

The layout is the one loader/write_latent_gguf.py produces (:72-74 names,
:227-257 per-row NF4 packing, :416-436 how tensors are recorded):

* `blk.{L}.ffn_latent_{gate,up,down}_{a,b}`: NF4 codes, GGML type I8, two
  codes per byte (low nibble = even column), bytes in C order of
  `[E][rows][cols/2]`, dims recorded as `(E, rows, cols/2)`
  (tests/test_write_latent_gguf.py:112-154 asserts these shapes);
* `..._{a,b}_s`: fp16 group scales, type F16, `[E][rows][cols/32]`;
* `blk.{L}.ffn_latent_ranks`: true ranks `[E][3]` (gate, up, down).
* KV `latent.max_rank`, `latent.group_size`, `latent.quantization`,
  `latent.format_version` (loader/write_latent_gguf.py:364-368).

Two documented extensions:

* the rank table is written as I32 `[E][3]` (the reference writes uint8 as
  I8, which cannot hold 256 or 512, in the byte order of `ranks.T`, i.e.
  kind-major `[3][E]` under recorded dims `(E, 3)`); the reader accepts both;
* per-group INT8 fallback groups (no reference format): `..._{a,b}_i8map`
  (I32 bitmap `[E][rows][words]`), `..._{a,b}_i8off` (I32 `[E][rows]`) and
  `..._{a,b}_i8` (I8 `[n][32]`), as in include/latent_ffn.h.

The GGUF framing (magic, version 3, KV and tensor-info records, 32-byte
aligned data) follows the published GGUF specification, the same fields
benchmarks/inspect_gguf_header.py:16-127 reads.
"""

from __future__ import annotations

import struct
from dataclasses import dataclass
from pathlib import Path
from typing import Dict, Iterable, Mapping, Optional, Tuple, Union

import numpy as np

GGUF_MAGIC = b"GGUF"
GGUF_VERSION = 3
DEFAULT_ALIGNMENT = 32

# GGUF value types (KV records).
_KV_U8, _KV_I8, _KV_U16, _KV_I16, _KV_U32, _KV_I32, _KV_F32, _KV_BOOL, _KV_STR, _KV_ARR, _KV_U64, _KV_I64, _KV_F64 = range(13)
_KV_SCALAR = {
    _KV_U8: "<B", _KV_I8: "<b", _KV_U16: "<H", _KV_I16: "<h", _KV_U32: "<I", _KV_I32: "<i",
    _KV_F32: "<f", _KV_BOOL: "<?", _KV_U64: "<Q", _KV_I64: "<q", _KV_F64: "<d",
}

# GGML tensor types used here.
GGML_F32, GGML_F16, GGML_I8, GGML_I16, GGML_I32 = 0, 1, 24, 25, 26
_GGML_DTYPE = {GGML_F32: np.float32, GGML_F16: np.float16, GGML_I8: np.int8, GGML_I16: np.int16, GGML_I32: np.int32}

FACTOR_NAMES = ("gate_a", "gate_b", "up_a", "up_b", "down_a", "down_b")
INT8_SUFFIXES = ("_i8map", "_i8off", "_i8")


def tensor_name(layer: int, suffix: str) -> str:
    """`blk.{layer}.ffn_latent_{suffix}` (loader/write_latent_gguf.py:72-74)."""
    return f"blk.{layer}.ffn_latent_{suffix}"


@dataclass
class TensorInfo:
    name: str
    dims: Tuple[int, ...]  # as recorded (ne order of the writer: (E, rows, cols) for factors)
    ggml_type: int
    offset: int            # relative to the start of the data section


@dataclass
class LatentGGUF:
    version: int
    metadata: Dict[str, object]
    tensors: Dict[str, TensorInfo]
    arrays: Dict[str, np.ndarray]  # C-order views shaped by the recorded dims

    def layers(self) -> Iterable[int]:
        out = set()
        for name in self.tensors:
            if name.startswith("blk.") and ".ffn_latent_" in name:
                out.add(int(name.split(".")[1]))
        return sorted(out)

    def layer_arrays(self, layer: int) -> Dict[str, np.ndarray]:
        """Arrays of one layer under the writer's names, codes as uint8 and the
        rank table widened to int32: the input of StackedLayer.from_arrays."""
        out: Dict[str, np.ndarray] = {}
        for name in FACTOR_NAMES:
            key = tensor_name(layer, name)
            if key not in self.arrays:
                raise KeyError(key)
            out[key] = self.arrays[key].view(np.uint8)
            out[key + "_s"] = self.arrays[key + "_s"]
            for suf in INT8_SUFFIXES:
                if key + suf in self.arrays:
                    arr = self.arrays[key + suf]
                    out[key + suf] = arr.view(np.uint32) if suf == "_i8map" else arr
        rk = tensor_name(layer, "ranks")
        if rk in self.arrays:
            r = self.arrays[rk]
            if r.dtype == np.int8:
                # The reference's table: uint8 ranks written as I8 from
                # per_expert_ranks.T (loader/write_latent_gguf.py:262-265,
                # 432-436), so the bytes are kind-major [3][E] under recorded
                # dims (E, 3).  Ranks of 256 or more wrapped modulo 256 when
                # the reference wrote them, so beside factors padded to a
                # max_rank above 255 the table is ambiguous (a stored 0 may be
                # 256 or 512).  The reference never reads it: its factors are
                # zero-padded to max_rank (loader/write_latent_gguf.py:101-123),
                # so computing every expert at max_rank is exact, and such a
                # table is dropped.
                max_rank = 2 * int(self.arrays[tensor_name(layer, "gate_a")].shape[-1])
                if max_rank > 255:
                    return out
                n_expert = int(self.tensors[rk].dims[0])
                r = r.reshape(-1).view(np.uint8).reshape(3, n_expert).T
            out[rk] = np.ascontiguousarray(r, dtype=np.int32)
        return out


# --------------------------------------------------------------------------
# writing
# --------------------------------------------------------------------------
def _pack_str(s: str) -> bytes:
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _pack_kv(key: str, value) -> bytes:
    if isinstance(value, bool):
        return _pack_str(key) + struct.pack("<I", _KV_BOOL) + struct.pack("<?", value)
    if isinstance(value, int):
        if 0 <= value < 2**32:
            return _pack_str(key) + struct.pack("<I", _KV_U32) + struct.pack("<I", value)
        return _pack_str(key) + struct.pack("<I", _KV_I64) + struct.pack("<q", value)
    if isinstance(value, float):
        return _pack_str(key) + struct.pack("<I", _KV_F32) + struct.pack("<f", value)
    if isinstance(value, str):
        return _pack_str(key) + struct.pack("<I", _KV_STR) + _pack_str(value)
    raise TypeError(f"unsupported KV value for {key}: {type(value).__name__}")


def _ggml_type(arr: np.ndarray) -> int:
    dt = arr.dtype
    if dt == np.uint8 or dt == np.int8:
        return GGML_I8
    if dt == np.float16:
        return GGML_F16
    if dt == np.float32:
        return GGML_F32
    if dt == np.int32 or dt == np.uint32:
        return GGML_I32
    if dt == np.int16 or dt == np.uint16:
        return GGML_I16
    raise TypeError(f"no GGML type for {dt}")


def _align(n: int, a: int) -> int:
    return (n + a - 1) // a * a


def write_latent_gguf(
    path: Union[str, Path],
    layers: Mapping[int, Mapping[str, np.ndarray]],
    max_rank: int,
    group_size: int = 32,
    metadata: Optional[Mapping[str, object]] = None,
    alignment: int = DEFAULT_ALIGNMENT,
) -> None:
    """Write stacked LATENT layers.

    layers[L] maps `gate_a` .. `down_b` to codes u8 [E][rows][cols/2] and the
    same names + `_s` to fp16 scales [E][rows][cols/32]; optional `ranks`
    (int [E][3]) and INT8 extensions `<name>_i8map/_i8off/_i8`.
    """
    kv = {
        "general.architecture": "latent",
        "general.alignment": int(alignment),
        "latent.max_rank": int(max_rank),
        "latent.group_size": int(group_size),
        "latent.quantization": f"nf4_g{group_size}",
        "latent.format_version": "1",
        "latent.rank_table": "i32",
    }
    if metadata:
        kv.update(metadata)
    tensors = []
    for L in sorted(layers):
        arrays = layers[L]
        for name in FACTOR_NAMES:
            codes = np.ascontiguousarray(arrays[name])
            scales = np.ascontiguousarray(arrays[name + "_s"])
            if codes.dtype not in (np.uint8, np.int8) or codes.ndim != 3:
                raise ValueError(f"{name}: codes must be uint8 [E][rows][cols/2]")
            if scales.dtype != np.float16 or scales.shape != codes.shape[:2] + (codes.shape[2] * 2 // group_size,):
                raise ValueError(f"{name}: scales must be float16 [E][rows][cols/{group_size}]")
            tensors.append((tensor_name(L, name), codes.view(np.int8)))
            tensors.append((tensor_name(L, name + "_s"), scales))
            ext = [arrays.get(name + suf) for suf in INT8_SUFFIXES]
            if any(t is not None for t in ext):
                if not all(t is not None for t in ext):
                    raise ValueError(f"{name}: INT8 extension needs _i8map, _i8off and _i8 together")
                tensors.append((tensor_name(L, name + "_i8map"), np.ascontiguousarray(ext[0]).view(np.int32)))
                tensors.append((tensor_name(L, name + "_i8off"), np.ascontiguousarray(ext[1], dtype=np.int32)))
                tensors.append((tensor_name(L, name + "_i8"), np.ascontiguousarray(ext[2], dtype=np.int8).reshape(-1, 32)))
        if "ranks" in arrays and arrays["ranks"] is not None:
            tensors.append((tensor_name(L, "ranks"), np.ascontiguousarray(arrays["ranks"], dtype=np.int32)))

    header = bytearray()
    header += GGUF_MAGIC + struct.pack("<I", GGUF_VERSION) + struct.pack("<QQ", len(tensors), len(kv))
    for k, v in kv.items():
        header += _pack_kv(k, v)
    offset = 0
    for name, arr in tensors:
        header += _pack_str(name) + struct.pack("<I", arr.ndim)
        header += struct.pack(f"<{arr.ndim}Q", *arr.shape)  # recorded dims, writer's order
        header += struct.pack("<I", _ggml_type(arr)) + struct.pack("<Q", offset)
        offset = _align(offset + arr.nbytes, alignment)
    with open(path, "wb") as f:
        f.write(header)
        f.write(b"\0" * (_align(len(header), alignment) - len(header)))
        pos = 0
        for _, arr in tensors:
            f.write(arr.tobytes(order="C"))
            pos += arr.nbytes
            pad = _align(pos, alignment) - pos
            f.write(b"\0" * pad)
            pos += pad


# --------------------------------------------------------------------------
# reading
# --------------------------------------------------------------------------
class _Cursor:
    def __init__(self, buf):
        self.buf, self.pos = buf, 0

    def take(self, fmt: str):
        v = struct.unpack_from(fmt, self.buf, self.pos)
        self.pos += struct.calcsize(fmt)
        return v[0] if len(v) == 1 else v

    def string(self) -> str:
        n = self.take("<Q")
        s = bytes(self.buf[self.pos:self.pos + n]).decode("utf-8")
        self.pos += n
        return s

    def value(self, vtype: int):
        if vtype in _KV_SCALAR:
            return self.take(_KV_SCALAR[vtype])
        if vtype == _KV_STR:
            return self.string()
        if vtype == _KV_ARR:
            atype, n = self.take("<I"), self.take("<Q")
            return [self.value(atype) for _ in range(n)]
        raise ValueError(f"unknown GGUF value type {vtype}")


def read_latent_gguf(path: Union[str, Path]) -> LatentGGUF:
    """Parse the header and map every tensor (no copy: numpy memmap views)."""
    mm = np.memmap(path, dtype=np.uint8, mode="r")
    cur = _Cursor(mm)
    if bytes(mm[:4]) != GGUF_MAGIC:
        raise ValueError(f"{path}: not a GGUF file")
    cur.pos = 4
    version = cur.take("<I")
    if version not in (2, 3):
        raise ValueError(f"{path}: unsupported GGUF version {version}")
    n_tensors, n_kv = cur.take("<Q"), cur.take("<Q")
    meta: Dict[str, object] = {}
    for _ in range(n_kv):
        key = cur.string()
        meta[key] = cur.value(cur.take("<I"))
    infos: Dict[str, TensorInfo] = {}
    for _ in range(n_tensors):
        name = cur.string()
        nd = cur.take("<I")
        dims = tuple(int(d) for d in struct.unpack_from(f"<{nd}Q", mm, cur.pos))
        cur.pos += 8 * nd
        gtype, off = cur.take("<I"), cur.take("<Q")
        infos[name] = TensorInfo(name, dims, gtype, off)
    alignment = int(meta.get("general.alignment", DEFAULT_ALIGNMENT))
    data0 = _align(cur.pos, alignment)
    arrays: Dict[str, np.ndarray] = {}
    for name, ti in infos.items():
        if ti.ggml_type not in _GGML_DTYPE:
            continue  # tensors this module does not interpret stay unmapped
        dt = np.dtype(_GGML_DTYPE[ti.ggml_type])
        count = int(np.prod(ti.dims)) if ti.dims else 1
        start = data0 + ti.offset
        if start + count * dt.itemsize > mm.size:
            raise ValueError(f"{path}: tensor {name} runs past the end of the file")
        arrays[name] = mm[start:start + count * dt.itemsize].view(dt).reshape(ti.dims)
    return LatentGGUF(version=version, metadata=meta, tensors=infos, arrays=arrays)


def layer_to_arrays(layer, experts: Optional[Iterable[int]] = None) -> Dict[str, np.ndarray]:
    """Host copies of a device StackedLayer (of `experts` only, when given)
    under the writer's short names, in the row layout (input of
    write_latent_gguf)."""
    out: Dict[str, np.ndarray] = {}
    for name, f in layer.factors().items():
        if f.layout != "rows" or experts is not None:
            if f.has_int8 and experts is not None:
                raise ValueError("an expert subset of a layer with INT8 groups is not exported")
            f = layer.factor_rows(name, None if experts is None else list(experts))
        out[name] = f.codes.cpu().numpy()
        out[name + "_s"] = f.scales.cpu().numpy().view(np.float16)
        if f.has_int8:
            out[name + "_i8map"] = f.int8_bitmap.cpu().numpy().view(np.uint32)
            out[name + "_i8off"] = f.int8_row_offset.cpu().numpy()
            out[name + "_i8"] = f.int8_data.cpu().numpy()
    if layer.ranks is not None:
        ranks = layer.ranks.cpu().numpy()
        out["ranks"] = ranks if experts is None else ranks[np.asarray(list(experts), dtype=np.int64)]
    return out
