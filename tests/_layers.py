"""Test helpers that move layers between the oracle (host) and the product (GPU)."""

from __future__ import annotations

from typing import Sequence

import numpy as np

from oracle import latent_ref as ref


def to_device(layer: ref.StackedLayer):
    """Upload an oracle StackedLayer (incl. INT8 extension and ranks) to the GPU."""
    import torch

    from latent_amd import DeviceFactor, StackedLayer

    facs = {}
    for name in ref.FACTOR_NAMES:
        f = layer.factors[name]
        ext = None
        if f.int8 is not None:
            ext = (f.int8.bitmap, f.int8.row_offset, f.int8.data)
        facs[name] = DeviceFactor.from_numpy(f.codes, f.scales, ext)
    ranks = None if layer.ranks is None else torch.from_numpy(layer.ranks.astype(np.int32)).cuda()
    return StackedLayer(**facs, ranks=ranks)


def _int8_subset(f, experts: np.ndarray) -> ref.Int8Groups:
    """The INT8 groups of `experts` of a device factor, with row offsets rebased.

    The side buffer holds the flagged groups in (expert, row, group) order, so
    expert e's groups are the contiguous run that starts at row_offset[e, 0]
    and holds as many groups as e's bitmap has bits set."""
    bitmap = f.int8_bitmap.cpu().numpy().view(np.uint32)
    row_offset = f.int8_row_offset.cpu().numpy().astype(np.int64)
    data = f.int8_data.cpu().numpy()
    counts = np.array([int(np.unpackbits(bitmap[e].view(np.uint8)).sum()) for e in experts], np.int64)
    parts, offs, base = [], [], 0
    for e, n in zip(experts, counts):
        start = int(row_offset[e, 0])
        parts.append(data[start:start + n])
        offs.append(row_offset[e] - start + base)
        base += int(n)
    data_sub = np.concatenate(parts) if parts else np.zeros((0, 32), np.int8)
    return ref.Int8Groups(bitmap=bitmap[experts], data=data_sub, row_offset=np.stack(offs).astype(np.int32))


def subset_to_host(dev_layer, experts: Sequence[int]) -> ref.StackedLayer:
    """Oracle StackedLayer holding only `experts` of a device layer (INT8
    groups included; a tile-layout layer is read back in the row layout)."""
    import torch

    ex = np.asarray(experts, dtype=np.int64)
    sel = torch.as_tensor(ex, device=dev_layer.gate_a.codes.device)
    facs = {}
    for name, f in dev_layer.factors().items():
        if f.layout == "tiles":
            rows = dev_layer.factor_rows(name, ex)
            codes, scales = rows.codes.cpu().numpy(), rows.scales.cpu().numpy().view(np.float16)
        else:
            codes = f.codes.index_select(0, sel).cpu().numpy()
            scales = f.scales.index_select(0, sel).cpu().numpy().view(np.float16)
        facs[name] = ref.StackedFactor(codes, scales, _int8_subset(f, ex) if f.has_int8 else None)
    ranks = None if dev_layer.ranks is None else dev_layer.ranks.index_select(0, sel).cpu().numpy()
    return ref.StackedLayer(factors=facs, d=dev_layer.d, ff=dev_layer.ff, max_rank=dev_layer.max_rank, ranks=ranks)


def remap_ids(ids: np.ndarray, n_expert: int):
    """(distinct valid experts, ids renumbered into that list; invalid -> -1)."""
    ids = np.asarray(ids)
    valid = (ids >= 0) & (ids < n_expert)
    experts = np.unique(ids[valid])
    lut = -np.ones(n_expert, np.int64)
    lut[experts] = np.arange(experts.size)
    out = np.where(valid, lut[np.clip(ids, 0, n_expert - 1)], -1).astype(np.int32)
    return experts, out
