"""Device-resident stacked LATENT factors and the MoE-layer expert FFN.

This is the host side of `GGML_OP_LATENT_EXPERT_FFN`
(kernels/latent_fused_expert_ffn.cu:134-292): the 12 stacked factor operands
of patches/002-latent-gguf-tensors.patch:135-148 live in HBM as torch tensors
and every call goes through `latent_moe_ffn_forward` of the HIP library.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
from typing import Dict, Mapping, Optional, Tuple

import numpy as np
import torch

from . import _lib
from ._lib import LatentFactor, LatentMoeArgs, check, lib

GROUP = 32
FACTOR_NAMES = ("gate_a", "gate_b", "up_a", "up_b", "down_a", "down_b")
KINDS = ("gate", "up", "down")

_DTYPE_CODE = {torch.float32: _lib.LATENT_F32, torch.float16: _lib.LATENT_F16, torch.bfloat16: _lib.LATENT_BF16}


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _stream(stream: Optional[torch.cuda.Stream] = None) -> ctypes.c_void_p:
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


LAYOUTS = ("rows", "tiles")


@dataclass
class DeviceFactor:
    """One stacked factor in HBM: codes u8 [E, rows, cols/2], scales f16 [E, rows, cols/32].

    Optional per-group INT8 fallback (see include/latent_ffn.h): int8_bitmap
    int32 [E, rows, words] (bit patterns of u32), int8_row_offset int32
    [E, rows], int8_data int8 [n, 32].

    layout "rows" is the writer's row order; "tiles" is the same tensors
    reordered by latent_tiles_repack for the MFMA paths (each expert's bytes
    stay in its own slice of the tensor, so expert selection works alike).
    """

    codes: torch.Tensor
    scales: torch.Tensor
    int8_bitmap: Optional[torch.Tensor] = None
    int8_row_offset: Optional[torch.Tensor] = None
    int8_data: Optional[torch.Tensor] = None
    layout: str = "rows"

    def __post_init__(self) -> None:
        if self.codes.dtype != torch.uint8 or self.codes.dim() != 3:
            raise ValueError("codes must be uint8 [E, rows, cols/2]")
        if self.scales.dtype not in (torch.float16, torch.int16) or self.scales.dim() != 3:
            raise ValueError("scales must be float16 [E, rows, cols/32]")
        E, rows, half = self.codes.shape
        if tuple(self.scales.shape) != (E, rows, half * 2 // GROUP) or (half * 2) % GROUP:
            raise ValueError(f"scales shape {tuple(self.scales.shape)} does not match codes {tuple(self.codes.shape)}")
        for t in (self.codes, self.scales, self.int8_bitmap, self.int8_row_offset, self.int8_data):
            if t is not None and (not t.is_cuda or not t.is_contiguous()):
                raise ValueError("factor tensors must be contiguous CUDA tensors")
        ext = (self.int8_bitmap, self.int8_row_offset, self.int8_data)
        if any(t is not None for t in ext) and not all(t is not None for t in ext):
            raise ValueError("INT8 extension needs bitmap, row_offset and data together")
        if self.layout not in LAYOUTS:
            raise ValueError(f"layout must be one of {LAYOUTS}")
        if self.layout == "tiles" and self.has_int8:
            raise ValueError("the tile layout is pure NF4")

    @property
    def n_expert(self) -> int:
        return int(self.codes.shape[0])

    @property
    def rows(self) -> int:
        return int(self.codes.shape[1])

    @property
    def cols(self) -> int:
        return int(self.codes.shape[2]) * 2

    @property
    def has_int8(self) -> bool:
        return self.int8_bitmap is not None

    def c_struct(self) -> LatentFactor:
        return LatentFactor(
            codes=_ptr(self.codes),
            scales=_ptr(self.scales),
            int8_bitmap=_ptr(self.int8_bitmap),
            int8_row_offset=_ptr(self.int8_row_offset),
            int8_data=_ptr(self.int8_data),
            rows=self.rows,
            cols=self.cols,
        )

    def nbytes(self) -> int:
        n = self.codes.numel() + self.scales.numel() * 2
        for t in (self.int8_bitmap, self.int8_row_offset, self.int8_data):
            if t is not None:
                n += t.numel() * t.element_size()
        return n

    def select(self, experts) -> "DeviceFactor":
        """The factor of `experts` only (either layout; pure NF4)."""
        if self.has_int8:
            raise ValueError("select() keeps no INT8 side buffer")
        sel = torch.as_tensor(np.asarray(experts, dtype=np.int64), device=self.codes.device)
        return DeviceFactor(self.codes.index_select(0, sel).contiguous(), self.scales.index_select(0, sel).contiguous(),
                            layout=self.layout)

    def repacked(self, factor: int, layout: str, stream: Optional[torch.cuda.Stream] = None) -> "DeviceFactor":
        """This factor in `layout` (a new pair of tensors; latent_tiles_repack).
        `factor` is its operand index, LATENT_GATE_A .. LATENT_DOWN_B."""
        if layout not in LAYOUTS:
            raise ValueError(f"layout must be one of {LAYOUTS}")
        if layout == self.layout:
            return self
        codes = torch.empty_like(self.codes)
        scales = torch.empty_like(self.scales)
        src = self.c_struct()
        dst = LatentFactor(codes=codes.data_ptr(), scales=scales.data_ptr(), rows=self.rows, cols=self.cols)
        check(lib.latent_tiles_repack(int(factor), ctypes.byref(src), ctypes.byref(dst), self.n_expert,
                                      1 if layout == "tiles" else 0, _stream(stream)), "latent_tiles_repack")
        return DeviceFactor(codes, scales, layout=layout)

    @classmethod
    def from_numpy(
        cls,
        codes: np.ndarray,
        scales: np.ndarray,
        int8: Optional[Tuple[np.ndarray, np.ndarray, np.ndarray]] = None,
        device: str = "cuda",
    ) -> "DeviceFactor":
        """From host arrays; `int8` = (bitmap u32, row_offset i32, data i8 [n, 32])."""
        c = torch.from_numpy(np.ascontiguousarray(codes, dtype=np.uint8)).to(device)
        s = torch.from_numpy(np.ascontiguousarray(scales).astype(np.float16)).to(device)
        if c.dim() == 2:
            c, s = c.unsqueeze(0), s.unsqueeze(0)
        ext = (None, None, None)
        if int8 is not None:
            bm, ro, data = int8
            ext = (
                torch.from_numpy(np.ascontiguousarray(bm, dtype=np.uint32).view(np.int32)).to(device),
                torch.from_numpy(np.ascontiguousarray(ro, dtype=np.int32)).to(device),
                torch.from_numpy(np.ascontiguousarray(data, dtype=np.int8).reshape(-1, GROUP)).to(device),
            )
            if ext[2].numel() == 0:  # keep a valid, aligned pointer for an empty side buffer
                ext = (ext[0], ext[1], torch.zeros((1, GROUP), dtype=torch.int8, device=device))
        return cls(c, s, *ext)


@dataclass
class StackedLayer:
    """The six stacked factors of one MoE layer plus per-expert ranks.

    Shapes (patches/002-latent-gguf-tensors.patch:135-148, packed code axis):
      gate_a, up_a [E, d, R/2]; gate_b, up_b [E, R, ff/2];
      down_a [E, ff, R/2]; down_b [E, R, d/2]; scales on a 1/16 axis.

    layout: "tiles" holds the twelve tensors in the tile layout of the MFMA
    paths (reordered in place of the row layout, factor by factor, so the
    layer is held once); "rows" keeps the writer's row layout; None (the
    default) takes "tiles" wherever latent_tiles_supported says the layer
    can (pure NF4, rank 256, d and ff multiples of 256).
    """

    gate_a: DeviceFactor
    gate_b: DeviceFactor
    up_a: DeviceFactor
    up_b: DeviceFactor
    down_a: DeviceFactor
    down_b: DeviceFactor
    ranks: Optional[torch.Tensor] = None  # int32 [E, 3] (gate, up, down)
    layout: Optional[str] = None
    _workspace: Dict[int, torch.Tensor] = field(default_factory=dict, repr=False)

    def __post_init__(self) -> None:
        E, d, R = self.n_expert, self.d, self.max_rank
        ff = self.ff
        want = {
            "gate_a": (d, R), "gate_b": (R, ff), "up_a": (d, R), "up_b": (R, ff), "down_a": (ff, R), "down_b": (R, d),
        }
        for name, (rows, cols) in want.items():
            f = getattr(self, name)
            if f.n_expert != E or f.rows != rows or f.cols != cols:
                raise ValueError(f"{name}: got [E={f.n_expert}, {f.rows}, {f.cols}], want [E={E}, {rows}, {cols}]")
        given = {f.layout for f in self.factors().values()}
        if len(given) != 1:
            raise ValueError("all six factors must be in one layout")
        if self.ranks is not None:
            if self.ranks.dtype != torch.int32 or tuple(self.ranks.shape) != (E, 3) or not self.ranks.is_cuda:
                raise ValueError("ranks must be a CUDA int32 [E, 3] tensor")
            self.ranks = self.ranks.contiguous()
        target = self.layout
        if target is None:
            target = "tiles" if given == {"tiles"} or self.tiles_supported() else "rows"
        if target not in LAYOUTS:
            raise ValueError(f"layout must be one of {LAYOUTS} or None")
        if target == "tiles" and given != {"tiles"} and not self.tiles_supported():
            raise ValueError("this layer has no tile layout (needs pure NF4, rank 256, d and ff % 256 == 0)")
        self.layout = next(iter(given))
        self._convert(target)

    def tiles_supported(self) -> bool:
        """Whether the layer can take the tile layout (latent_tiles_supported)."""
        a = self.args()
        r = lib.latent_tiles_supported(ctypes.byref(a))
        if r < 0:
            check(r, "latent_tiles_supported")
        return r == 1

    def _convert(self, layout: str) -> None:
        # One factor at a time: the old pair is released before the next is
        # repacked, so converting needs one factor's bytes beyond the layer.
        for k, name in enumerate(FACTOR_NAMES):
            setattr(self, name, getattr(self, name).repacked(k, layout))
        self.layout = layout

    def to_layout(self, layout: str) -> "StackedLayer":
        """A copy of this layer in `layout` (this layer is left as it is)."""
        facs = {k: v for k, v in self.factors().items()}
        return StackedLayer(**facs, ranks=self.ranks, layout=layout)

    def factor_rows(self, name: str, experts=None) -> DeviceFactor:
        """Factor `name` (of `experts` only, when given) in the row layout."""
        f = getattr(self, name)
        if experts is not None:
            f = f.select(experts)
        return f.repacked(FACTOR_NAMES.index(name), "rows")

    @property
    def n_expert(self) -> int:
        return self.gate_a.n_expert

    @property
    def d(self) -> int:
        return self.gate_a.rows

    @property
    def max_rank(self) -> int:
        return self.gate_a.cols

    @property
    def ff(self) -> int:
        return self.gate_b.cols

    def factors(self) -> Dict[str, DeviceFactor]:
        return {n: getattr(self, n) for n in FACTOR_NAMES}

    def nbytes(self) -> int:
        """Bytes of the twelve factor tensors (plus INT8 side buffers): all the
        layer holds in HBM, in either layout."""
        return sum(f.nbytes() for f in self.factors().values())

    @classmethod
    def from_arrays(
        cls,
        arrays: Mapping[str, np.ndarray],
        layer: Optional[int] = None,
        device: str = "cuda",
        layout: Optional[str] = None,
    ) -> "StackedLayer":
        """From the writer's tensor names (loader/write_latent_gguf.py:72-74, 256-265).

        Keys `blk.{layer}.ffn_latent_{kind}_{a,b}` (codes) and `..._{a,b}_s`
        (scales), optional `..._{a,b}_i8map / _i8off / _i8` (per-group INT8
        extension), plus optional `blk.{layer}.ffn_latent_ranks`; with layer=None
        the `blk.N.ffn_latent_` prefix is omitted.  Ranks are widened to int32
        (the writer's uint8 table cannot hold 256 or 512).  The arrays are in
        the row layout; `layout` is the layout the layer is held in.
        """
        prefix = "" if layer is None else f"blk.{layer}.ffn_latent_"
        facs = {}
        for name in FACTOR_NAMES:
            key = prefix + name
            ext = None
            if key + "_i8map" in arrays:  # per-group INT8 extension (see latent_amd.gguf)
                ext = (arrays[key + "_i8map"], arrays[key + "_i8off"], arrays[key + "_i8"])
            facs[name] = DeviceFactor.from_numpy(arrays[key], arrays[key + "_s"], ext, device=device)
        ranks = arrays.get(prefix + "ranks")
        rt = None if ranks is None else torch.from_numpy(np.asarray(ranks).astype(np.int32)).to(device)
        return cls(**facs, ranks=rt, layout=layout)

    def args(self) -> LatentMoeArgs:
        a = LatentMoeArgs()
        for name in FACTOR_NAMES:
            setattr(a, name, getattr(self, name).c_struct())
        a.ranks = _ptr(self.ranks)
        a.n_embd, a.n_ff, a.n_expert, a.max_rank = self.d, self.ff, self.n_expert, self.max_rank
        a.layout = _lib.LATENT_LAYOUT_TILES if self.layout == "tiles" else _lib.LATENT_LAYOUT_ROWS
        return a

    def workspace(self, n_tokens: int, n_expert_used: int) -> torch.Tensor:
        """A cached workspace large enough for (n_tokens, n_expert_used)."""
        need = workspace_size(self, n_tokens, n_expert_used)
        dev = self.gate_a.codes.device
        key = dev.index or 0
        ws = self._workspace.get(key)
        if ws is None or ws.numel() < need:
            # Zero-filled: the library keeps its control block zero between calls.
            ws = torch.zeros(max(need, 256), dtype=torch.uint8, device=dev)
            self._workspace[key] = ws
        return ws


def workspace_error(workspace: torch.Tensor, stream: Optional[torch.cuda.Stream] = None) -> int:
    """Read and clear the workspace's error word through latent_moe_check:
    LATENT_E_TIMEOUT when a call since the last check had a bounded wait time
    out (its output is undefined), else 0.  Synchronises the stream."""
    r = lib.latent_moe_check(workspace.data_ptr(), workspace.numel() * workspace.element_size(), _stream(stream))
    if r not in (_lib.LATENT_OK, _lib.LATENT_E_TIMEOUT):
        check(r, "latent_moe_check")
    return int(r)


def workspace_size(layer: StackedLayer, n_tokens: int, n_expert_used: int) -> int:
    a = layer.args()
    a.n_tokens, a.n_expert_used = int(n_tokens), int(n_expert_used)
    a.x_dtype, a.weights_dtype, a.out_mode = _lib.LATENT_F32, _lib.LATENT_F32, _lib.LATENT_OUT_REDUCED
    n = ctypes.c_size_t(0)
    check(lib.latent_moe_workspace_size(ctypes.byref(a), ctypes.byref(n)), "latent_moe_workspace_size")
    return int(n.value)


def moe_path(layer: StackedLayer, x: torch.Tensor, n_expert_used: int) -> str:
    """'fused' (one persistent decode kernel), 'prefill' (grouped MFMA), 'stream'
    (streaming MFMA decode), 'rows' (multi-kernel MFMA on the row layout) or
    'general' (multi-kernel GEMV) for this call shape (LATENT_MOE_PATH in the
    environment selects another supported path)."""
    a = layer.args()
    a.x = x.data_ptr()
    a.n_tokens, a.n_expert_used = int(x.shape[0]), int(n_expert_used)
    a.x_dtype, a.weights_dtype, a.out_mode = _DTYPE_CODE[x.dtype], _lib.LATENT_F32, _lib.LATENT_OUT_REDUCED
    r = lib.latent_moe_path(ctypes.byref(a))
    if r < 0:
        check(r, "latent_moe_path")
    return {1: "fused", 2: "prefill", 3: "stream", 4: "rows"}.get(r, "general")


def stream_launch(layer: StackedLayer, x: torch.Tensor, n_expert_used: int) -> Optional[str]:
    """Launch style of a streaming-path call: 'lite' (small-batch chain in one
    launch) or 'phases' (one launch per phase); None
    when the call does not take the streaming path."""
    a = layer.args()
    a.x = x.data_ptr()
    a.n_tokens, a.n_expert_used = int(x.shape[0]), int(n_expert_used)
    a.x_dtype, a.weights_dtype, a.out_mode = _DTYPE_CODE[x.dtype], _lib.LATENT_F32, _lib.LATENT_OUT_REDUCED
    r = lib.latent_stream_launch(ctypes.byref(a))
    if r == _lib.LATENT_E_UNSUPPORTED:
        return None
    if r < 0:
        check(r, "latent_stream_launch")
    return {0: "phases", 2: "lite"}[r]


def moe_forward(
    x: torch.Tensor,
    ids: torch.Tensor,
    weights: torch.Tensor,
    layer: StackedLayer,
    weight_before_down: bool = False,
    out_mode: int = _lib.LATENT_OUT_REDUCED,
    out: Optional[torch.Tensor] = None,
    workspace: Optional[torch.Tensor] = None,
    stream: Optional[torch.cuda.Stream] = None,
    check_timeout: bool = False,
) -> torch.Tensor:
    """Router-weighted LATENT expert FFN of one MoE layer on the GPU.

    x [T, d] (f32 / f16 / bf16), ids int32 [T, k] (id < 0 = dropped slot),
    weights [T, k] (f32 / f16).  Returns f32 [T, d] (out_mode 0) or the
    per-slot f32 [T, k, d] of the ggml op (out_mode 1).

    check_timeout=True synchronises after the call and raises LatentError
    (LATENT_E_TIMEOUT) if a bounded wait between workgroups expired, in
    which case the output is undefined.
    """
    if x.dim() != 2 or ids.dim() != 2 or weights.shape != ids.shape or x.shape[0] != ids.shape[0]:
        raise ValueError("expected x [T, d], ids [T, k], weights [T, k]")
    if x.dtype not in _DTYPE_CODE or weights.dtype not in (torch.float32, torch.float16) or ids.dtype != torch.int32:
        raise TypeError("x must be f32/f16/bf16, ids int32, weights f32/f16")
    if x.shape[1] != layer.d:
        raise ValueError(f"x has {x.shape[1]} features, layer expects {layer.d}")
    for t in (x, ids, weights):
        if not t.is_cuda:
            raise ValueError("inputs must be CUDA tensors")
    x, ids, weights = x.contiguous(), ids.contiguous(), weights.contiguous()
    T, k = ids.shape
    shape = (T, layer.d) if out_mode == _lib.LATENT_OUT_REDUCED else (T, k, layer.d)
    if out is None:
        out = torch.empty(shape, dtype=torch.float32, device=x.device)
    elif tuple(out.shape) != shape or out.dtype != torch.float32 or not out.is_contiguous():
        raise ValueError(f"out must be contiguous f32 {shape}")
    if workspace is None:
        workspace = layer.workspace(T, k)
    # A caller-provided workspace must be zero-filled before its first use.
    a = layer.args()
    a.x, a.x_dtype = x.data_ptr(), _DTYPE_CODE[x.dtype]
    a.ids = ids.data_ptr()
    a.weights = weights.data_ptr()
    a.weights_dtype = _lib.LATENT_F32 if weights.dtype == torch.float32 else _lib.LATENT_F16
    a.n_tokens, a.n_expert_used = T, k
    a.weight_before_down = 1 if weight_before_down else 0
    a.out_mode = int(out_mode)
    a.out = out.data_ptr()
    a.workspace = workspace.data_ptr()
    a.workspace_bytes = workspace.numel() * workspace.element_size()
    check(lib.latent_moe_ffn_forward(ctypes.byref(a), _stream(stream)), "latent_moe_ffn_forward")
    if check_timeout:
        check(workspace_error(workspace, stream), "latent_moe_ffn_forward")
    return out


def unpack(factor: DeviceFactor, expert: int, stream: Optional[torch.cuda.Stream] = None,
           kind: Optional[int] = None) -> torch.Tensor:
    """Dequantized f32 [rows, cols] of one expert (bit-exact NF4 / INT8 decode).
    A factor in the tile layout needs its operand index `kind`
    (LATENT_GATE_A .. LATENT_DOWN_B): the expert is repacked to rows first."""
    if not 0 <= expert < factor.n_expert:
        raise IndexError(expert)
    if factor.layout == "tiles":
        if kind is None:
            raise ValueError("unpack of a tile-layout factor needs its operand index `kind`")
        factor = factor.select([expert]).repacked(kind, "rows", stream)
        expert = 0
    out = torch.empty((factor.rows, factor.cols), dtype=torch.float32, device=factor.codes.device)
    c = factor.c_struct()
    check(lib.latent_unpack(ctypes.byref(c), int(expert), out.data_ptr(), _stream(stream)), "latent_unpack")
    return out


def pack_nf4(values: torch.Tensor, stream: Optional[torch.cuda.Stream] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Per-row NF4 pack of f32 [..., cols] on the GPU -> (codes u8 [..., cols/2], scales f16 [..., cols/32])."""
    if values.dtype != torch.float32 or not values.is_cuda:
        raise TypeError("values must be a CUDA f32 tensor")
    v = values.contiguous()
    cols = v.shape[-1]
    if cols % GROUP:
        raise ValueError("last axis must be a multiple of 32")
    rows = v.numel() // cols
    codes = torch.empty(v.shape[:-1] + (cols // 2,), dtype=torch.uint8, device=v.device)
    scales = torch.empty(v.shape[:-1] + (cols // GROUP,), dtype=torch.float16, device=v.device)
    check(lib.latent_pack_nf4(v.data_ptr(), rows, cols, codes.data_ptr(), scales.data_ptr(), _stream(stream)),
          "latent_pack_nf4")
    return codes, scales


def pack_int8(groups: torch.Tensor, stream: Optional[torch.cuda.Stream] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """INT8 pack of f32 [n, 32] groups on the GPU -> (q int8 [n, 32], scales f16 [n])."""
    if groups.dtype != torch.float32 or not groups.is_cuda or groups.shape[-1] != GROUP:
        raise TypeError("groups must be a CUDA f32 [n, 32] tensor")
    g = groups.contiguous().reshape(-1, GROUP)
    n = g.shape[0]
    q = torch.empty((max(n, 1), GROUP), dtype=torch.int8, device=g.device)
    s = torch.empty((max(n, 1),), dtype=torch.float16, device=g.device)
    if n:
        check(lib.latent_pack_int8(g.data_ptr(), n, q.data_ptr(), s.data_ptr(), _stream(stream)), "latent_pack_int8")
    return q[:n], s[:n]
