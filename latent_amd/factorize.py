"""Load-time low-rank factorisation of dense experts on the GPU.

Restates, on torch (rocBLAS / rocSOLVER) in fp32, the reference's offline
path (loader/latent_loader.py:66-108, compress_matrix at 195-249): the rank
from the full spectrum's energy, then a randomized SVD with the same
sketch (numpy Generator(seed).standard_normal((n, rank + oversample), float32),
one power iteration, reduced QR, SVD of the small projection), the energy-based
rank choice, A = U sqrt(S), B = sqrt(S) V^T, then NF4 packing with the
library's byte-exact kernel.  `stack_experts` builds a StackedLayer: factors
padded to max_rank (code 7 / scale 1.0), per-expert true ranks, and
optionally per-group INT8 fallback for the groups whose NF4 SNR is below a
threshold (the reference switches a whole factor to INT8 at group 64 when too
many groups are noisy, loader/latent_loader.py:229-249; the per-group form is
this build's extension, see include/latent_ffn.h).
"""

from __future__ import annotations

from typing import List, Optional, Sequence, Tuple

import numpy as np
import torch

from .moe import GROUP, DeviceFactor, StackedLayer, pack_int8, pack_nf4, unpack


def randomized_svd(matrix: torch.Tensor, target_rank: int, oversample: int = 16, power_iterations: int = 1,
                   seed: int = 0) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Truncated randomized SVD of a 2-D CUDA matrix: (U [m, r], s [r], Vt [r, n])."""
    if matrix.dim() != 2:
        raise ValueError(f"expected a 2-D matrix, got shape {tuple(matrix.shape)}")
    m, n = matrix.shape
    rank = min(target_rank, m, n)
    sketch = min(rank + oversample, m, n)
    omega = np.random.default_rng(seed).standard_normal((n, sketch), dtype=np.float32)
    a = matrix.to(torch.float32)
    y = a @ torch.from_numpy(omega).to(a.device)
    for _ in range(power_iterations):
        y = a @ (a.T @ y)
    q, _ = torch.linalg.qr(y, mode="reduced")
    b = q.T @ a
    u_hat, s, vt = torch.linalg.svd(b, full_matrices=False)
    u = q @ u_hat
    return u[:, :rank], s[:rank], vt[:rank, :]


def choose_rank(singular_values, energy: float, min_rank: int, max_rank: int) -> int:
    """Smallest rank retaining `energy` of sum(s^2), clamped to [min_rank, max_rank]
    (loader/latent_loader.py:89-97)."""
    if not 0 < energy <= 1:
        raise ValueError("energy must be in (0, 1]")
    s = torch.as_tensor(singular_values, dtype=torch.float64)
    total = float((s * s).sum())
    if total == 0:
        return min_rank
    cumulative = torch.cumsum(s * s, 0) / total
    rank = int(torch.searchsorted(cumulative, torch.tensor([energy], dtype=torch.float64, device=s.device)).item()) + 1
    return max(min_rank, min(rank, max_rank, int(s.numel())))


def make_factors(u: torch.Tensor, s: torch.Tensor, vt: torch.Tensor, rank: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """A = U sqrt(S), B = sqrt(S) V^T in fp32 (loader/latent_loader.py:100-104)."""
    root = torch.sqrt(s[:rank]).to(torch.float32)
    return u[:, :rank].to(torch.float32) * root[None, :], root[:, None] * vt[:rank, :].to(torch.float32)


def group_snr(values: torch.Tensor, decoded: torch.Tensor) -> torch.Tensor:
    """Per-32-group signal-to-noise ratio ||x|| / ||x - q(x)|| of [rows, cols]
    (quantization_snr_by_group of loader/latent_loader.py:173-185 per row group)."""
    rows, cols = values.shape
    x = values.reshape(rows, cols // GROUP, GROUP)
    err = (values - decoded).reshape(rows, cols // GROUP, GROUP)
    return x.norm(dim=2) / err.norm(dim=2).clamp_min(1e-12)


def int8_group_mask(values: torch.Tensor, decoded: torch.Tensor, snr_threshold: float) -> torch.Tensor:
    """bool [..., rows, cols/32]: the non-zero row groups whose NF4 decode has SNR
    below `snr_threshold` (the SNR of quantization_snr_by_group,
    loader/latent_loader.py:173-185, which the reference thresholds at :227-229)."""
    rows, cols = values.shape[-2:]
    lead = values.shape[:-2]
    snr = group_snr(values.reshape(-1, cols), decoded.reshape(-1, cols)).reshape(*lead, rows, cols // GROUP)
    nonzero = values.reshape(*lead, rows, cols // GROUP, GROUP).abs().amax(-1) > 0
    return (snr < snr_threshold) & nonzero


def stack_experts(
    gate: Sequence[torch.Tensor],
    up: Sequence[torch.Tensor],
    down: Sequence[torch.Tensor],
    max_rank: int,
    energy: float = 0.95,
    min_rank: int = 16,
    snr_threshold: Optional[float] = None,
    seed: int = 0,
) -> Tuple[StackedLayer, List[Tuple[int, int, int]]]:
    """Factorise dense experts (gate, up: [d, ff]; down: [ff, d]) into a StackedLayer.

    Returns the layer and the chosen (gate, up, down) rank of every expert.
    With snr_threshold set, groups whose NF4 decode has SNR below it are stored
    as INT8 groups.
    """
    E = len(gate)
    if not (len(up) == len(down) == E) or E == 0:
        raise ValueError("need the same number of gate, up and down experts")
    if max_rank % GROUP:
        raise ValueError("max_rank must be a multiple of 32")
    d, ff = gate[0].shape
    dev = gate[0].device
    shapes = {"gate": (d, ff), "up": (d, ff), "down": (ff, d)}
    a_st = {k: torch.zeros((E, shapes[k][0], max_rank), dtype=torch.float32, device=dev) for k in shapes}
    b_st = {k: torch.zeros((E, max_rank, shapes[k][1]), dtype=torch.float32, device=dev) for k in shapes}
    ranks: List[Tuple[int, int, int]] = []
    for e in range(E):
        rk = []
        for ki, (kind, mats) in enumerate((("gate", gate), ("up", up), ("down", down))):
            w = mats[e].to(torch.float32)
            if tuple(w.shape) != shapes[kind]:
                raise ValueError(f"{kind}[{e}] has shape {tuple(w.shape)}, want {shapes[kind]}")
            full_s = torch.linalg.svdvals(w)  # rank from the full spectrum, as compress_matrix does
            r = choose_rank(full_s, energy, min_rank, max_rank)
            u, s, vt = randomized_svd(w, r, seed=seed + 3 * e + ki)
            a, b = make_factors(u, s, vt, r)
            a_st[kind][e, :, :r] = a
            b_st[kind][e, :r, :] = b
            rk.append(r)
        ranks.append(tuple(rk))
    facs = {}
    for kind in shapes:
        for side, st in (("a", a_st[kind]), ("b", b_st[kind])):
            codes, scales = pack_nf4(st)
            f = DeviceFactor(codes.contiguous(), scales.contiguous())
            if snr_threshold is not None:
                f = _int8_fallback(st, f, snr_threshold)
            facs[f"{kind}_{side}"] = f
    rt = torch.tensor(ranks, dtype=torch.int32, device=dev)
    return StackedLayer(**facs, ranks=rt), ranks


def _int8_fallback(values: torch.Tensor, f: DeviceFactor, snr_threshold: float) -> DeviceFactor:
    """Store the groups whose NF4 SNR is below the threshold as INT8 groups:
    bit g of a row's bitmap word set, the group's 16 code bytes zero, its scale
    absmax/127, its values in `data` row-major over (expert, row, group) with
    row_offset the index of the row's first INT8 group."""
    E, rows, cols = values.shape
    decoded = torch.stack([unpack(f, e) for e in range(E)])
    mask = int8_group_mask(values, decoded, snr_threshold)  # [E, rows, groups]
    if not bool(mask.any()):
        return f
    groups = cols // GROUP
    words = (groups + 31) // 32
    bits = torch.zeros((E, rows, words * 32), dtype=torch.int64, device=values.device)
    bits[:, :, :groups] = mask.to(torch.int64)
    bitmap = (bits.view(E, rows, words, 32) * torch.pow(2, torch.arange(32, device=values.device))).sum(-1)
    bitmap = torch.where(bitmap >= 2**31, bitmap - 2**32, bitmap).to(torch.int32).contiguous()
    per_row = mask.reshape(E * rows, groups).sum(1)
    row_offset = (torch.cumsum(per_row, 0) - per_row).to(torch.int32).reshape(E, rows).contiguous()
    q, s = pack_int8(values.reshape(E, rows, groups, GROUP)[mask].contiguous())
    scales = f.scales.clone()
    scales[mask] = s
    codes = f.codes.clone()
    codes.view(E, rows, groups, GROUP // 2)[mask] = 0
    return DeviceFactor(codes, scales.contiguous(), bitmap, row_offset, q.contiguous())
