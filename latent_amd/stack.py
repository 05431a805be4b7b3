"""Consecutive LATENT MoE layers decoded as one HIP graph.

Each layer l routes its tokens with its own router and adds the expert FFN to
the residual stream:

    ids_l, w_l = top-k(softmax(x_l . W_r[l]))
    y_l        = sum_k w_l * LATENT_FFN_l(x_l)          (latent_moe_ffn_forward)
    x_{l+1}    = x_l + y_l

The residual stream stays fp32 on the device; every buffer is allocated once,
so the whole stack (2 router kernels + the expert FFN + one add per layer) can
be captured in a torch.cuda.CUDAGraph (a HIP graph) and replayed.  This is the
stacked decode of a llama.cpp graph built by build_moe_ffn_latent
(README.md:111-113) with the MoE blocks only.
"""

from __future__ import annotations

from typing import List, Optional, Sequence

import torch

from .moe import StackedLayer, moe_forward, workspace_size
from .router import Router


class DecodeStack:
    def __init__(self, layers: Sequence[StackedLayer], routers: Sequence[Router], n_tokens: int):
        if len(layers) != len(routers) or not layers:
            raise ValueError("need one router per layer")
        d, k = layers[0].d, routers[0].k
        for L, r in zip(layers, routers):
            if L.d != d or r.n_embd != d or r.n_expert != L.n_expert or r.k != k:
                raise ValueError("layers and routers must share d, k and match expert counts")
        self.layers, self.routers = list(layers), list(routers)
        self.T, self.d, self.k = int(n_tokens), d, k
        dev = layers[0].gate_a.codes.device
        n = len(layers)
        self.x = [torch.zeros((self.T, d), dtype=torch.float32, device=dev) for _ in range(n + 1)]
        self.y = [torch.empty((self.T, d), dtype=torch.float32, device=dev) for _ in range(n)]
        self.ids = [torch.empty((self.T, k), dtype=torch.int32, device=dev) for _ in range(n)]
        self.w = [torch.empty((self.T, k), dtype=torch.float32, device=dev) for _ in range(n)]
        self.logits = [torch.empty((self.T, r.n_expert), dtype=torch.float32, device=dev) for r in routers]
        # One zero-filled workspace shared by every layer (calls are stream ordered
        # and each call leaves the control block zero).
        need = max(workspace_size(L, self.T, k) for L in layers)
        self.workspace = torch.zeros((max(need, 256),), dtype=torch.uint8, device=dev)
        for r in self.routers:
            r.workspace(self.T)
        self.graph: Optional[torch.cuda.CUDAGraph] = None

    @property
    def output(self) -> torch.Tensor:
        return self.x[-1]

    def _body(self) -> None:
        for l, (L, r) in enumerate(zip(self.layers, self.routers)):
            r(self.x[l], ids=self.ids[l], weights=self.w[l], logits_out=self.logits[l])
            moe_forward(self.x[l], self.ids[l], self.w[l], L, out=self.y[l], workspace=self.workspace)
            torch.add(self.x[l], self.y[l], out=self.x[l + 1])

    def load(self, x0: torch.Tensor) -> None:
        self.x[0].copy_(x0)

    def forward(self, x0: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Eager run on the current stream."""
        if x0 is not None:
            self.load(x0)
        self._body()
        return self.output

    def capture(self, warmup: int = 2) -> torch.cuda.CUDAGraph:
        """Capture the stack in a graph; replays read x[0] and write every buffer."""
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(warmup):
                self._body()
        torch.cuda.current_stream().wait_stream(side)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self._body()
        self.graph = g
        return g

    def replay(self) -> torch.Tensor:
        if self.graph is None:
            raise RuntimeError("capture() first")
        self.graph.replay()
        return self.output

    def resident_bytes(self) -> int:
        return sum(L.nbytes() for L in self.layers)

    def router_bytes(self) -> int:
        return sum(r.weight.numel() * r.weight.element_size() for r in self.routers)

    def layer_ids(self) -> List[torch.Tensor]:
        return self.ids
