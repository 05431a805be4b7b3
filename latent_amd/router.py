"""Router front end on the GPU: logits, softmax, top-k, renormalise, drop.

The reference routes inside the llama.cpp graph builder (build_moe_ffn_latent,
README.md:111-113) and restates adaptive expert dropping on the host
(loader/adaptive_topk.py:29-90).  Here one `latent_route` call of the HIP
library produces the ids / weights operands of `moe_forward` on the device,
so a decode layer is stream-ordered device work a HIP graph can hold.
"""

from __future__ import annotations

import ctypes
from typing import Dict, Optional, Tuple

import torch

from . import _lib
from ._lib import LatentRouteArgs, check, lib

DROP_RULES = {
    "none": _lib.LATENT_DROP_NONE,
    "below": _lib.LATENT_DROP_BELOW,  # renormalised weight < param -> dropped
    "inclusive": _lib.LATENT_DROP_INCLUSIVE,  # adaptive_topk_inclusive (cumulative mass)
}
_X_DTYPE = {torch.float32: _lib.LATENT_F32, torch.float16: _lib.LATENT_F16, torch.bfloat16: _lib.LATENT_BF16}
_R_DTYPE = {torch.float32: _lib.LATENT_F32, torch.bfloat16: _lib.LATENT_BF16}


def _args(n_tokens: int, n_embd: int, n_expert: int, k: int, drop: str, drop_param: float) -> LatentRouteArgs:
    if drop not in DROP_RULES:
        raise ValueError(f"drop must be one of {sorted(DROP_RULES)}")
    a = LatentRouteArgs()
    a.n_tokens, a.n_embd, a.n_expert, a.n_expert_used = int(n_tokens), int(n_embd), int(n_expert), int(k)
    a.drop_rule, a.drop_param = DROP_RULES[drop], float(drop_param)
    return a


def route_workspace_size(n_tokens: int, n_embd: int, n_expert: int, k: int, from_logits: bool = False) -> int:
    a = _args(n_tokens, n_embd, n_expert, k, "none", 0.0)
    a.x_dtype, a.router_dtype = _lib.LATENT_F32, _lib.LATENT_F32
    if from_logits:
        a.logits_in = 1  # any non-NULL value: no workspace is needed then
    n = ctypes.c_size_t(0)
    check(lib.latent_route_workspace_size(ctypes.byref(a), ctypes.byref(n)), "latent_route_workspace_size")
    return int(n.value)


def route(
    k: int,
    x: Optional[torch.Tensor] = None,
    router: Optional[torch.Tensor] = None,
    logits: Optional[torch.Tensor] = None,
    drop: str = "none",
    drop_param: float = 0.0,
    logits_out: Optional[torch.Tensor] = None,
    ids: Optional[torch.Tensor] = None,
    weights: Optional[torch.Tensor] = None,
    workspace: Optional[torch.Tensor] = None,
    stream: Optional[torch.cuda.Stream] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Top-k routing on the GPU -> (ids int32 [T, k], weights f32 [T, k]).

    Either `x` [T, d] (f32/f16/bf16) with `router` [d, E] (f32/bf16), or
    precomputed f32 `logits` [T, E].  Slots are in descending weight order;
    a dropped slot has id -1 and weight 0.
    """
    if logits is not None:
        if logits.dtype != torch.float32 or logits.dim() != 2 or not logits.is_cuda:
            raise TypeError("logits must be a CUDA f32 [T, E] tensor")
        logits = logits.contiguous()
        T, E = logits.shape
        d = 0
    else:
        if x is None or router is None:
            raise ValueError("give x and router, or logits")
        if x.dim() != 2 or router.dim() != 2 or x.shape[1] != router.shape[0]:
            raise ValueError("expected x [T, d] and router [d, E]")
        if x.dtype not in _X_DTYPE or router.dtype not in _R_DTYPE or not (x.is_cuda and router.is_cuda):
            raise TypeError("x must be CUDA f32/f16/bf16 and router CUDA f32/bf16")
        x, router = x.contiguous(), router.contiguous()
        T, d = x.shape
        E = router.shape[1]
    dev = (logits if logits is not None else x).device
    a = _args(T, d, E, k, drop, drop_param)
    if ids is None:
        ids = torch.empty((T, k), dtype=torch.int32, device=dev)
    if weights is None:
        weights = torch.empty((T, k), dtype=torch.float32, device=dev)
    if tuple(ids.shape) != (T, k) or ids.dtype != torch.int32 or not ids.is_contiguous():
        raise ValueError(f"ids must be contiguous int32 {(T, k)}")
    if tuple(weights.shape) != (T, k) or weights.dtype != torch.float32 or not weights.is_contiguous():
        raise ValueError(f"weights must be contiguous f32 {(T, k)}")
    if logits_out is not None and (tuple(logits_out.shape) != (T, E) or logits_out.dtype != torch.float32
                                   or not logits_out.is_contiguous()):
        raise ValueError(f"logits_out must be contiguous f32 {(T, E)}")
    if logits is not None:
        a.logits_in = logits.data_ptr()
    else:
        a.x, a.x_dtype = x.data_ptr(), _X_DTYPE[x.dtype]
        a.router, a.router_dtype = router.data_ptr(), _R_DTYPE[router.dtype]
        if workspace is None:
            need = route_workspace_size(T, d, E, k)
            workspace = torch.empty((max(need, 4),), dtype=torch.uint8, device=dev)
        a.workspace, a.workspace_bytes = workspace.data_ptr(), workspace.numel() * workspace.element_size()
    a.logits_out = 0 if logits_out is None else logits_out.data_ptr()
    a.ids, a.weights = ids.data_ptr(), weights.data_ptr()
    s = stream if stream is not None else torch.cuda.current_stream()
    check(lib.latent_route(ctypes.byref(a), ctypes.c_void_p(s.cuda_stream)), "latent_route")
    return ids, weights


class Router:
    """A device router matrix W_r [d, E] with cached workspaces per token count."""

    def __init__(self, weight: torch.Tensor, k: int, drop: str = "none", drop_param: float = 0.0):
        if weight.dim() != 2 or weight.dtype not in _R_DTYPE or not weight.is_cuda:
            raise TypeError("router weight must be a CUDA f32/bf16 [d, E] tensor")
        self.weight = weight.contiguous()
        self.k, self.drop, self.drop_param = int(k), drop, float(drop_param)
        self._ws: Dict[int, torch.Tensor] = {}

    @property
    def n_embd(self) -> int:
        return int(self.weight.shape[0])

    @property
    def n_expert(self) -> int:
        return int(self.weight.shape[1])

    def workspace(self, n_tokens: int) -> torch.Tensor:
        ws = self._ws.get(n_tokens)
        if ws is None:
            need = route_workspace_size(n_tokens, self.n_embd, self.n_expert, self.k)
            ws = torch.empty((max(need, 4),), dtype=torch.uint8, device=self.weight.device)
            self._ws[n_tokens] = ws
        return ws

    def __call__(self, x: torch.Tensor, ids: Optional[torch.Tensor] = None, weights: Optional[torch.Tensor] = None,
                 logits_out: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
        return route(self.k, x=x, router=self.weight, drop=self.drop, drop_param=self.drop_param, ids=ids,
                     weights=weights, logits_out=logits_out, workspace=self.workspace(int(x.shape[0])))
