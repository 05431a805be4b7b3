"""GPU counterpart of loader/latent_runtime.py (expert-forward entry point).

Same names and argument meaning as the reference:

    gate = load_pair(arrays, "gate"); up = ...; down = ...
    y = swiglu_expert(x, gate, up, down, weight=1.0, weight_before_down=False)

`arrays` uses the NPZ keys of loader/latent_loader.py:253-260
(`<name>.{a,b}.{nf4|int8,scales,shape}`); a missing factor raises KeyError
(loader/latent_runtime.py:28).  The factors are kept packed in HBM and the
chain runs in the HIP library; numpy in, numpy out.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Mapping, Tuple

import numpy as np
import torch

from . import _lib
from .moe import GROUP, DeviceFactor, StackedLayer, moe_forward

NF4_PAD_BYTE = 0x77  # two zero codes (code 7 == 0.0)


@dataclass
class FactorPair:
    """Packed A [n_in, r] and B [r, n_out] factors (loader/latent_runtime.py:13-16).

    Each side is kept as host arrays in the stacked per-row layout:
    codes u8 [rows, cols/2], scales f16 [rows, cols/32], optional INT8 groups.
    """

    a: Tuple[np.ndarray, np.ndarray, object]
    b: Tuple[np.ndarray, np.ndarray, object]
    n_in: int
    rank: int
    n_out: int


def _int8_as_groups(q: np.ndarray, scales: np.ndarray, shape) -> Tuple[np.ndarray, np.ndarray, object]:
    """Whole-factor INT8 at group 64 (loader/latent_runtime.py:26-27) as per-group INT8.

    A 64-group of a row-major matrix whose column count is a multiple of 64 is
    two adjacent 32-groups of one row sharing the scale, so every 32-group is
    flagged INT8 and the scale is repeated; dequant stays f32(q) * f32(s).
    """
    rows, cols = shape
    if cols % 64:
        raise NotImplementedError("INT8 factors need a column count that is a multiple of 64")
    groups = cols // GROUP
    data = np.asarray(q, dtype=np.int8)[: rows * cols].reshape(rows * groups, GROUP)
    s = np.repeat(np.asarray(scales).astype(np.float16)[: rows * cols // 64], 2).reshape(rows, groups)
    words = (groups + 31) // 32
    bitmap = np.zeros((rows, words), dtype=np.uint32)
    for g in range(groups):
        bitmap[:, g // 32] |= np.uint32(1 << (g % 32))
    row_offset = (np.arange(rows, dtype=np.int64) * groups).astype(np.int32)
    codes = np.zeros((rows, cols // 2), dtype=np.uint8)
    return codes, s, (bitmap, row_offset, data)


def _load_side(arrays: Mapping[str, np.ndarray], name: str, side: str):
    """loader/latent_runtime.py:19-28 (NF4 group 32, else INT8 group 64)."""
    shape = tuple(int(v) for v in arrays[f"{name}.{side}.shape"])
    if len(shape) != 2:
        raise ValueError(f"{name}.{side}: expected a 2-D factor, got shape {shape}")
    scales = arrays[f"{name}.{side}.scales"]
    rows, cols = shape
    if f"{name}.{side}.nf4" in arrays:
        if cols % GROUP:
            raise NotImplementedError(
                f"{name}.{side}: NF4 groups straddle rows when cols ({cols}) is not a multiple of 32")
        codes = np.asarray(arrays[f"{name}.{side}.nf4"], dtype=np.uint8)[: rows * cols // 2].reshape(rows, cols // 2)
        s = np.asarray(scales).astype(np.float16)[: rows * cols // GROUP].reshape(rows, cols // GROUP)
        return (codes, s, None), shape
    if f"{name}.{side}.int8" in arrays:
        return _int8_as_groups(arrays[f"{name}.{side}.int8"], scales, shape), shape
    raise KeyError(f"missing {name}.{side} factor")


def load_pair(arrays: Mapping[str, np.ndarray], name: str) -> FactorPair:
    """loader/latent_runtime.py:31-32."""
    a, a_shape = _load_side(arrays, name, "a")
    b, b_shape = _load_side(arrays, name, "b")
    if a_shape[1] != b_shape[0]:
        raise ValueError(f"{name}: rank mismatch {a_shape} x {b_shape}")
    return FactorPair(a=a, b=b, n_in=a_shape[0], rank=a_shape[1], n_out=b_shape[1])


def _pad_a(side, rows: int, rank: int, R: int):
    """Pad A's columns to R with zero groups (pad byte 0x77, scale 1.0), like
    loader/write_latent_gguf.py:101-123, 249-253."""
    codes, s, ext = side
    if rank == R:
        return codes, s, ext
    pc = np.full((rows, R // 2), NF4_PAD_BYTE, dtype=np.uint8)
    pc[:, : rank // 2] = codes
    ps = np.ones((rows, R // GROUP), dtype=np.float16)
    ps[:, : rank // GROUP] = s
    if ext is not None:
        bm, ro, data = ext
        nb = np.zeros((rows, (R // GROUP + 31) // 32), dtype=np.uint32)
        nb[:, : bm.shape[1]] = bm
        ext = (nb, ro, data)
    return pc, ps, ext


def _pad_b(side, rank: int, cols: int, R: int):
    codes, s, ext = side
    if rank == R:
        return codes, s, ext
    pc = np.full((R, cols // 2), NF4_PAD_BYTE, dtype=np.uint8)
    pc[:rank] = codes
    ps = np.ones((R, cols // GROUP), dtype=np.float16)
    ps[:rank] = s
    if ext is not None:
        bm, ro, data = ext
        nb = np.zeros((R, bm.shape[1]), dtype=np.uint32)
        nb[:rank] = bm
        nro = np.full((R,), data.shape[0], dtype=np.int32)
        nro[:rank] = ro
        ext = (nb, nro, data)
    return pc, ps, ext


def expert_layer(gate: FactorPair, up: FactorPair, down: FactorPair, device: str = "cuda") -> StackedLayer:
    """A one-expert StackedLayer from three factor pairs (ranks padded to the largest)."""
    d, ff = gate.n_in, gate.n_out
    if up.n_in != d or up.n_out != ff or down.n_in != ff or down.n_out != d:
        raise ValueError("gate/up must be [d, ff] and down [ff, d]")
    R = max(p.rank for p in (gate, up, down))
    R = (R + GROUP - 1) // GROUP * GROUP
    facs = {}
    for kind, pair in (("gate", gate), ("up", up), ("down", down)):
        a = _pad_a(pair.a, pair.n_in, pair.rank, R)
        b = _pad_b(pair.b, pair.rank, pair.n_out, R)
        facs[f"{kind}_a"] = DeviceFactor.from_numpy(a[0], a[1], a[2], device=device)
        facs[f"{kind}_b"] = DeviceFactor.from_numpy(b[0], b[1], b[2], device=device)
    ranks = torch.tensor([[gate.rank, up.rank, down.rank]], dtype=torch.int32, device=device)
    return StackedLayer(**facs, ranks=ranks)


def swiglu_expert(
    x: np.ndarray,
    gate: FactorPair,
    up: FactorPair,
    down: FactorPair,
    weight: float = 1.0,
    weight_before_down: bool = False,
) -> np.ndarray:
    """loader/latent_runtime.py:48-59 on the GPU.

    `weight` scales the hidden activations only when `weight_before_down`;
    otherwise it is ignored, as in the reference.
    """
    xa = np.asarray(x, dtype=np.float32)
    squeeze = xa.ndim == 1
    x2 = xa.reshape(1, -1) if squeeze else xa
    layer = expert_layer(gate, up, down)
    T = x2.shape[0]
    xt = torch.from_numpy(np.ascontiguousarray(x2)).cuda()
    ids = torch.zeros((T, 1), dtype=torch.int32, device="cuda")
    w = torch.full((T, 1), float(np.float32(weight)), dtype=torch.float32, device="cuda")
    y = moe_forward(xt, ids, w, layer, weight_before_down=weight_before_down, out_mode=_lib.LATENT_OUT_PER_SLOT)
    out = y[:, 0, :].cpu().numpy()
    return out[0] if squeeze else out
