"""Seeded synthetic LATENT layers generated and packed on the GPU.

Factors follow the rank-r SVD of W = U diag(s) V^T with s_i = 0.02 * i^-0.7:
A = U_r diag(sqrt(s_r)), B = diag(sqrt(s_r)) V_r^T (make_factors of
loader/latent_loader.py:104-108).  U and V are orthonormalised Gaussian
matrices (Cholesky QR in float64).  Packing uses the library's byte-exact
NF4 / INT8 kernels, so a 256-expert DeepSeek-V3-shaped layer (about 1 GB
packed) takes seconds instead of the hours a host pack would.
"""

from __future__ import annotations

from typing import Dict, Optional, Sequence, Tuple

import numpy as np
import torch

from .moe import GROUP, DeviceFactor, StackedLayer, pack_int8, pack_nf4

KIND_DIMS = {"gate": ("d", "ff"), "up": ("d", "ff"), "down": ("ff", "d")}


def spectrum(n: int, device) -> torch.Tensor:
    i = torch.arange(1, n + 1, dtype=torch.float64, device=device)
    return 0.02 * i.pow(-0.7)


def _seed(base: int, e: int, kind: int, side: int) -> int:
    return (base * 1_000_003 + e * 16 + kind * 2 + side) & 0x7FFF_FFFF_FFFF


def orthonormal_batch(n: int, r: int, seeds: Sequence[int], device) -> torch.Tensor:
    """float64 [len(seeds), n, r], each with orthonormal columns (Cholesky QR2 of a
    Gaussian drawn from its own seed)."""
    g = torch.empty((len(seeds), n, r), dtype=torch.float64, device=device)
    gen = torch.Generator(device=device)
    for i, sd in enumerate(seeds):
        gen.manual_seed(int(sd))
        g[i] = torch.randn((n, r), generator=gen, dtype=torch.float64, device=device)
    eye = torch.eye(r, dtype=torch.float64, device=device).expand(len(seeds), r, r)
    for _ in range(2):
        c = torch.bmm(g.transpose(1, 2).contiguous(), g)
        lower = torch.linalg.cholesky(c)
        inv = torch.linalg.solve_triangular(lower, eye, upper=False)
        g = torch.bmm(g, inv.transpose(1, 2).contiguous())
    return g


def stacked_factors(seed: int, experts: Sequence[int], kind: int, n_in: int, n_out: int, R: int,
                    ranks: Sequence[int], device):
    """fp32 A [n, n_in, R], B [n, R, n_out] for a batch of experts, zero beyond each rank."""
    s = spectrum(R, device)
    root = s.sqrt()[None, :].repeat(len(experts), 1)
    for i, e in enumerate(experts):
        root[i, int(ranks[e]):] = 0.0
    u = orthonormal_batch(n_in, R, [_seed(seed, e, kind, 0) for e in experts], device)
    a = (u * root[:, None, :]).to(torch.float32)
    del u
    v = orthonormal_batch(n_out, R, [_seed(seed, e, kind, 1) for e in experts], device)
    b = (root[:, :, None] * v.transpose(1, 2)).to(torch.float32).contiguous()
    return a, b


def _int8_ext(values: torch.Tensor, mask: torch.Tensor):
    """Per-group INT8 extension of a stacked fp32 factor [E, rows, cols] and group mask."""
    E, rows, cols = values.shape
    groups = cols // GROUP
    words = (groups + 31) // 32
    mpad = torch.zeros((E, rows, words * 32), dtype=torch.int64, device=values.device)
    mpad[:, :, :groups] = mask.to(torch.int64)
    weights = torch.pow(2, torch.arange(32, dtype=torch.int64, device=values.device))
    bitmap = (mpad.view(E, rows, words, 32) * weights).sum(-1)
    bitmap = torch.where(bitmap >= 2**31, bitmap - 2**32, bitmap).to(torch.int32).contiguous()
    per_row = mask.reshape(E * rows, groups).sum(1)
    row_offset = (torch.cumsum(per_row, 0) - per_row).to(torch.int32).reshape(E, rows).contiguous()
    sel = values.reshape(E, rows, groups, GROUP)[mask]
    q, s = pack_int8(sel.contiguous())
    if q.shape[0] == 0:
        q = torch.zeros((1, GROUP), dtype=torch.int8, device=values.device)
    return bitmap, row_offset, q.contiguous(), s


def make_layer(
    seed: int,
    n_expert: int,
    d: int,
    ff: int,
    max_rank: int,
    ranks: Optional[Sequence[int]] = None,
    int8_fraction: float = 0.0,
    device: str = "cuda",
) -> StackedLayer:
    """A packed StackedLayer; ranks[e] (<= max_rank) zero-pads expert e's factors."""
    dims = {"d": d, "ff": ff}
    rank_list = [max_rank] * n_expert if ranks is None else [int(r) for r in ranks]
    facs: Dict[str, DeviceFactor] = {}
    mask_gen = torch.Generator(device=device)
    mask_gen.manual_seed(seed + 1_000_003)
    for k, kind in enumerate(("gate", "up", "down")):
        n_in, n_out = dims[KIND_DIMS[kind][0]], dims[KIND_DIMS[kind][1]]
        a_st = torch.empty((n_expert, n_in, max_rank), dtype=torch.float32, device=device)
        b_st = torch.empty((n_expert, max_rank, n_out), dtype=torch.float32, device=device)
        for e0 in range(0, n_expert, 32):
            batch = list(range(e0, min(n_expert, e0 + 32)))
            a_st[e0:e0 + len(batch)], b_st[e0:e0 + len(batch)] = stacked_factors(
                seed, batch, k, n_in, n_out, max_rank, rank_list, device)
        for side, st in (("a", a_st), ("b", b_st)):
            codes, scales = pack_nf4(st)
            ext = (None, None, None)
            if int8_fraction > 0:
                E, rows, cols = st.shape
                m = torch.rand((E, rows, cols // GROUP), generator=mask_gen, device=device) < int8_fraction
                r = torch.tensor(rank_list, device=device)
                if side == "a":
                    gi = torch.arange(cols // GROUP, device=device)
                    m &= (gi[None, None, :] * GROUP < r[:, None, None])
                else:
                    ri = torch.arange(rows, device=device)
                    m &= (ri[None, :, None] < r[:, None, None])
                bitmap, row_offset, q, s = _int8_ext(st, m)
                scales = scales.clone()
                scales[m] = s
                cg = codes.view(E, rows, cols // GROUP, GROUP // 2)
                cg[m] = 0
                ext = (bitmap, row_offset, q)
            facs[f"{kind}_{side}"] = DeviceFactor(codes.contiguous(), scales.contiguous(), *ext)
        del a_st, b_st
    rt = torch.tensor([[r, r, r] for r in rank_list], dtype=torch.int32, device=device)
    return StackedLayer(**facs, ranks=rt)


# ----------------------------------------------------------------------------
# Routing of the synthetic workloads
# ----------------------------------------------------------------------------
def softmax_topk(logits: torch.Tensor, k: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """Softmax over experts (float64), top-k, renormalised -> (ids int32, w f32)."""
    p = torch.softmax(logits.to(torch.float64), dim=1)
    top, idx = torch.topk(p, k, dim=1)
    w = top / top.sum(dim=1, keepdim=True)
    return idx.to(torch.int32).contiguous(), w.to(torch.float32).contiguous()


def route(seed: int, n_tokens: int, n_expert: int, k: int, device: str = "cuda", zipf_gamma: float = 0.0,
          zipf_alpha: float = 1.1, drop_below: float = 0.0, rank_beta: float = 0.0, logit_scale: float = 1.0):
    """Router logits N(0,1) plus an optional per-expert popularity bias, top-k,
    renormalise, optional drop.

    Each expert gets a popularity rank from a seeded permutation.  Bias
    zipf_gamma * (-zipf_alpha * ln rank) is the Zipf-shaped skew; bias
    -rank_beta * (rank - 1) / (E - 1) falls linearly with the rank.  At 4096
    tokens, 256 experts and top-8 (128 pairs per expert on average), the Zipf
    form cannot give both a near-empty tail and a head near 400 (gamma 0.11:
    about 75..390 tokens per expert; gamma 0.45: about 10..2200), while
    rank_beta = 1.5 gives about 5..430 with some 20 experts below 16 tokens.
    logit_scale multiplies the N(0,1) draw: with 256 experts and top-8, about
    0.3% of renormalised weights fall below 0.05 at scale 1 and 16% at scale 2.
    """
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    logits = torch.randn((n_tokens, n_expert), generator=gen, device=device)
    if logit_scale != 1.0:
        logits = logits * logit_scale
    if zipf_gamma or rank_beta:
        perm = torch.randperm(n_expert, generator=gen, device=device).to(torch.float64) + 1.0
        bias = torch.zeros_like(perm)
        if zipf_gamma:
            bias += zipf_gamma * (-zipf_alpha * torch.log(perm))
        if rank_beta:
            bias += -rank_beta * (perm - 1.0) / max(1, n_expert - 1)
        logits = logits + bias.to(torch.float32)[None, :]
    ids, w = softmax_topk(logits, k)
    if drop_below > 0:
        drop = w < drop_below
        ids = torch.where(drop, torch.full_like(ids, -1), ids)
        w = torch.where(drop, torch.zeros_like(w), w)
    return ids.contiguous(), w.contiguous()


def bf16_input(seed: int, n_tokens: int, d: int, device: str = "cuda") -> torch.Tensor:
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    return torch.randn((n_tokens, d), generator=gen, device=device).to(torch.bfloat16)


def layer_to_host(layer: StackedLayer, experts: Optional[Sequence[int]] = None) -> Dict[str, Tuple]:
    """Copy (a subset of experts of) a layer's packed operands to host numpy
    arrays, in the row layout."""
    out = {}
    for name in layer.factors():
        f = layer.factor_rows(name, None if experts is None else list(experts))
        out[name] = (f.codes.cpu().numpy(), f.scales.cpu().numpy().view(np.float16))
    return out
