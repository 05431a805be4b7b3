"""GPU counterpart of loader/latent_runtime.py (expert-forward entry point).

Same names and argument meaning as the reference:

    gate = load_pair(arrays, "gate"); up = ...; down = ...
    y = swiglu_expert(x, gate, up, down, weight=1.0, weight_before_down=False)

`arrays` uses the NPZ keys of loader/latent_loader.py:253-260
(`<name>.{a,b}.{nf4|int8,scales,shape}`); a missing factor raises KeyError
(loader/latent_runtime.py:28).  The factors stay in their packed artifact
form (flat row-major quantization groups: NF4 at group 32, INT8 at group 64,
loader/latent_runtime.py:25-27), are uploaded to HBM once per device and
kept there, and the chain runs in the HIP library (`latent_expert_forward`);
numpy in, numpy out.
"""

from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass, field
from typing import Dict, Mapping, Optional, Tuple

import numpy as np
import torch

from . import _lib
from ._lib import LatentExpertArgs, LatentFlatFactor, check, lib

NF4_GROUP = 32  # loader/latent_runtime.py:25
INT8_GROUP = 64  # loader/latent_runtime.py:27


@dataclass
class FlatFactor:
    """One packed factor [rows, cols] exactly as the artifact stores it.

    kind LATENT_Q_NF4: data u8 [ceil(rows*cols/2)] (two codes per byte, low
    nibble first); LATENT_Q_INT8: data i8 [groups*group_size]; scales f16
    [groups], group g covering flat elements [g*G, (g+1)*G).
    """

    kind: int
    data: np.ndarray
    scales: np.ndarray
    rows: int
    cols: int
    group_size: int
    _device: Dict[int, Tuple[torch.Tensor, torch.Tensor]] = field(default_factory=dict, repr=False)

    @property
    def groups(self) -> int:
        return int(math.ceil(self.rows * self.cols / self.group_size))

    def to_device(self, device: torch.device) -> Tuple[torch.Tensor, torch.Tensor]:
        """(data, scales) in HBM; uploaded on first use and cached per device."""
        key = device.index if device.index is not None else torch.cuda.current_device()
        got = self._device.get(key)
        if got is None:
            dev = torch.device("cuda", key)
            data = torch.from_numpy(np.array(self.data, copy=True).view(np.uint8)).to(dev)
            scales = torch.from_numpy(np.array(self.scales, dtype=np.float16, copy=True)).to(dev)
            got = (data, scales)
            self._device[key] = got
        return got

    def c_struct(self, device: torch.device) -> LatentFlatFactor:
        data, scales = self.to_device(device)
        return LatentFlatFactor(data=data.data_ptr(), scales=scales.data_ptr(), kind=self.kind,
                                group_size=self.group_size, rows=self.rows, cols=self.cols)


@dataclass
class FactorPair:
    """Packed A [n_in, r] and B [r, n_out] factors (loader/latent_runtime.py:13-16)."""

    a: FlatFactor
    b: FlatFactor

    @property
    def n_in(self) -> int:
        return self.a.rows

    @property
    def rank(self) -> int:
        return self.a.cols

    @property
    def n_out(self) -> int:
        return self.b.cols


def _load_factor(arrays: Mapping[str, np.ndarray], name: str, side: str) -> FlatFactor:
    """loader/latent_runtime.py:19-28: NF4 at group 32, else INT8 at group 64, else KeyError."""
    shape = tuple(int(v) for v in arrays[f"{name}.{side}.shape"])
    scales = np.asarray(arrays[f"{name}.{side}.scales"]).astype(np.float16).reshape(-1)
    if len(shape) != 2:
        raise ValueError(f"{name}.{side}: expected a 2-D factor, got shape {shape}")
    rows, cols = shape
    n = rows * cols
    nf4_key, int8_key = f"{name}.{side}.nf4", f"{name}.{side}.int8"
    if nf4_key in arrays:
        kind, group = _lib.LATENT_Q_NF4, NF4_GROUP
        data = np.ascontiguousarray(arrays[nf4_key], dtype=np.uint8).reshape(-1)
        need = int(math.ceil(n / group)) * group // 2
    elif int8_key in arrays:
        kind, group = _lib.LATENT_Q_INT8, INT8_GROUP
        data = np.ascontiguousarray(arrays[int8_key], dtype=np.int8).reshape(-1)
        need = int(math.ceil(n / group)) * group
    else:
        raise KeyError(f"missing {name}.{side} factor")
    groups = int(math.ceil(n / group))
    # The reference's reshape / broadcast fail on these (loader/latent_loader.py:139-144, 166-168).
    if data.size < need:
        raise ValueError(f"{name}.{side}: {data.size} packed values, {need} needed for shape {shape}")
    if scales.size != groups:
        raise ValueError(f"{name}.{side}: {scales.size} scales, {groups} groups for shape {shape}")
    return FlatFactor(kind=kind, data=data, scales=scales, rows=rows, cols=cols, group_size=group)


def load_pair(arrays: Mapping[str, np.ndarray], name: str) -> FactorPair:
    """loader/latent_runtime.py:31-32."""
    a = _load_factor(arrays, name, "a")
    b = _load_factor(arrays, name, "b")
    if a.cols != b.rows:
        raise ValueError(f"{name}: rank mismatch [{a.rows}, {a.cols}] x [{b.rows}, {b.cols}]")
    return FactorPair(a=a, b=b)


def swiglu_expert(
    x: np.ndarray,
    gate: FactorPair,
    up: FactorPair,
    down: FactorPair,
    weight: float = 1.0,
    weight_before_down: bool = False,
    device: Optional[torch.device] = None,
) -> np.ndarray:
    """loader/latent_runtime.py:48-59 on the GPU.

    `weight` scales the hidden activations only when `weight_before_down`;
    otherwise it is ignored, as in the reference.
    """
    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    xa = np.asarray(x, dtype=np.float32)
    squeeze = xa.ndim == 1
    x2 = xa.reshape(1, -1) if squeeze else xa
    if x2.ndim != 2:
        raise ValueError(f"x must be 1-D or 2-D, got shape {xa.shape}")
    d, ff = gate.n_in, gate.n_out
    if x2.shape[1] != d:
        raise ValueError(f"x has {x2.shape[1]} features, gate expects {d}")
    if up.n_in != d or up.n_out != ff or down.n_in != ff or down.n_out != d:
        raise ValueError("gate/up must be [d, ff] and down [ff, d]")
    T = x2.shape[0]
    a = LatentExpertArgs()
    for kind, pair in (("gate", gate), ("up", up), ("down", down)):
        setattr(a, f"{kind}_a", pair.a.c_struct(dev))
        setattr(a, f"{kind}_b", pair.b.c_struct(dev))
    a.n_tokens = T
    a.weight = float(np.float32(weight))
    a.weight_before_down = 1 if weight_before_down else 0
    need = ctypes.c_size_t(0)
    check(lib.latent_expert_workspace_size(ctypes.byref(a), ctypes.byref(need)), "latent_expert_workspace_size")
    xt = torch.from_numpy(np.ascontiguousarray(x2)).to(dev)
    out = torch.empty((T, d), dtype=torch.float32, device=dev)
    ws = torch.empty(max(int(need.value), 256), dtype=torch.uint8, device=dev)
    a.x = xt.data_ptr()
    a.out = out.data_ptr()
    a.workspace = ws.data_ptr()
    a.workspace_bytes = ws.numel()
    stream = torch.cuda.current_stream(dev)
    check(lib.latent_expert_forward(ctypes.byref(a), ctypes.c_void_p(stream.cuda_stream)), "latent_expert_forward")
    y = out.cpu().numpy()
    return y[0] if squeeze else y
