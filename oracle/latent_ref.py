"""numpy restatement of the LATENT codec, CPU runtime and stacked layout.

TEST INFRASTRUCTURE ONLY (see `oracle/__init__.py`): the product never imports
this module.

Every function cites the reference file:line whose behaviour it restates.
The arithmetic is kept in the same precision and order as the reference:

* NF4 quantize: fp32 group absmax, fp32 normalise, fp32 |n - cb| distances,
  first-index argmin, low nibble = even element, fp16 (RNE) stored scale.
* NF4 / INT8 dequantize: one fp32 multiply `code_value * f32(scale_f16)`.
* project: `(x_f32 @ A) @ B` in fp32 (BLAS sgemm, rank-r latent kept fp32).
* silu: float64 `x / (1 + exp(-x))`, clipped to +-1e30, cast to fp32.

Additions that the reference does not have (it leaves them to the caller or
to empty patches) are marked "no reference counterpart" and follow the
operand contract documented in `include/latent_ffn.h`:

* `moe_forward`: routing-weighted sum over the top-k experts (the reduce the
  reference README places after `GGML_OP_LATENT_EXPERT_FFN`).
* per-group INT8 fallback (bitmap + side buffer) for heterogeneous layers.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Dict, Mapping, Optional, Sequence, Tuple

import numpy as np

# loader/latent_loader.py:28-48 -- the 16 NF4 levels as float32 literals.
NF4_CODEBOOK = np.array(
    [
        -1.0,
        -0.6961928,
        -0.52507305,
        -0.3949175,
        -0.28444138,
        -0.18477343,
        -0.09105004,
        0.0,
        0.0795803,
        0.1609302,
        0.2461123,
        0.33791524,
        0.44070983,
        0.562617,
        0.72295684,
        1.0,
    ],
    dtype=np.float32,
)

NF4_ZERO_CODE = 7  # index of 0.0 in the codebook; the pad nibble
GROUP = 32

# Bound on the temporary [groups, group, 16] distance tensor (elements).
_CHUNK_GROUPS = 1 << 15


# ----------------------------------------------------------------------------
# Codec
# ----------------------------------------------------------------------------
def quantize_nf4(values: np.ndarray, group_size: int = 32) -> Tuple[np.ndarray, np.ndarray, Tuple[int, ...]]:
    """Packed NF4 codes + fp16 group scales.  loader/latent_loader.py:111-130.

    Flatten row-major, zero-pad to a multiple of `group_size`, scale = fp32
    max|x| of the group (0 -> 1.0), normalise in fp32, nearest codebook entry
    (first index on ties), two codes per byte (low nibble = even index), an odd
    code count padded with code 7.  The group loop is chunked only to bound the
    temporary; the arithmetic per group is unchanged.
    """
    flat = np.asarray(values, dtype=np.float32).reshape(-1)
    original_shape = tuple(np.shape(values))
    groups = int(math.ceil(flat.size / group_size))
    padded = np.zeros(groups * group_size, dtype=np.float32)
    padded[: flat.size] = flat
    grouped = padded.reshape(groups, group_size)

    scales = np.max(np.abs(grouped), axis=1).astype(np.float32) if groups else np.zeros(0, np.float32)
    scales[scales == 0] = 1.0
    codes = np.empty((groups, group_size), dtype=np.uint8)
    for g0 in range(0, groups, _CHUNK_GROUPS):
        g1 = min(groups, g0 + _CHUNK_GROUPS)
        normalized = grouped[g0:g1] / scales[g0:g1, np.newaxis]
        distances = np.abs(normalized[..., np.newaxis] - NF4_CODEBOOK[np.newaxis, np.newaxis, :])
        codes[g0:g1] = np.argmin(distances, axis=-1).astype(np.uint8)
    codes = codes.reshape(-1)
    if codes.size % 2:
        codes = np.pad(codes, (0, 1), constant_values=NF4_ZERO_CODE)
    packed = (codes[0::2] | (codes[1::2] << 4)).astype(np.uint8)
    return packed, scales.astype(np.float16), original_shape


def dequantize_nf4(
    packed: np.ndarray,
    scales: np.ndarray,
    original_shape: Sequence[int],
    group_size: int = 32,
) -> np.ndarray:
    """fp32 values `cb[code] * f32(scale)`.  loader/latent_loader.py:133-145."""
    packed = np.asarray(packed, dtype=np.uint8).reshape(-1)
    codes = np.empty(packed.size * 2, dtype=np.uint8)
    codes[0::2] = packed & 0x0F
    codes[1::2] = packed >> 4
    n = int(np.prod(original_shape))
    groups = int(math.ceil(n / group_size))
    codes = codes[: groups * group_size].reshape(groups, group_size)
    decoded = NF4_CODEBOOK[codes] * np.asarray(scales).astype(np.float32).reshape(-1)[:groups, np.newaxis]
    return decoded.reshape(-1)[:n].reshape(tuple(original_shape)).astype(np.float32)


def quantize_int8(values: np.ndarray, group_size: int = 64) -> Tuple[np.ndarray, np.ndarray, Tuple[int, ...]]:
    """Symmetric INT8 with fp16 scale absmax/127.  loader/latent_loader.py:148-158."""
    flat = np.asarray(values, dtype=np.float32).reshape(-1)
    original_shape = tuple(np.shape(values))
    groups = int(math.ceil(flat.size / group_size))
    padded = np.zeros(groups * group_size, dtype=np.float32)
    padded[: flat.size] = flat
    grouped = padded.reshape(groups, group_size)
    scales = np.max(np.abs(grouped), axis=1).astype(np.float32) / np.float32(127.0)
    scales[scales == 0] = 1.0
    quantized = np.rint(grouped / scales[:, np.newaxis]).clip(-127, 127).astype(np.int8)
    return quantized.reshape(-1), scales.astype(np.float16), original_shape


def dequantize_int8(
    quantized: np.ndarray,
    scales: np.ndarray,
    original_shape: Sequence[int],
    group_size: int = 64,
) -> np.ndarray:
    """fp32 values `f32(q) * f32(scale)`.  loader/latent_loader.py:161-170."""
    n = int(np.prod(original_shape))
    groups = int(math.ceil(n / group_size))
    grouped = np.asarray(quantized)[: groups * group_size].reshape(groups, group_size).astype(np.float32)
    decoded = grouped * np.asarray(scales).astype(np.float32).reshape(-1)[:groups, np.newaxis]
    return decoded.reshape(-1)[:n].reshape(tuple(original_shape)).astype(np.float32)


# ----------------------------------------------------------------------------
# CPU runtime  (loader/latent_runtime.py)
# ----------------------------------------------------------------------------
@dataclass
class FactorPair:
    """loader/latent_runtime.py:13-16."""

    a: np.ndarray
    b: np.ndarray


def load_factor(arrays: Mapping[str, np.ndarray], name: str, side: str) -> np.ndarray:
    """NF4 (group 32) or whole-factor INT8 (group 64).  loader/latent_runtime.py:19-28."""
    shape = tuple(int(v) for v in arrays[f"{name}.{side}.shape"])
    scales = arrays[f"{name}.{side}.scales"]
    if f"{name}.{side}.nf4" in arrays:
        return dequantize_nf4(arrays[f"{name}.{side}.nf4"], scales, shape, group_size=32)
    if f"{name}.{side}.int8" in arrays:
        return dequantize_int8(arrays[f"{name}.{side}.int8"], scales, shape, group_size=64)
    raise KeyError(f"missing {name}.{side} factor")


def load_pair(arrays: Mapping[str, np.ndarray], name: str) -> FactorPair:
    """loader/latent_runtime.py:31-32."""
    return FactorPair(a=load_factor(arrays, name, "a"), b=load_factor(arrays, name, "b"))


def project(x: np.ndarray, pair: FactorPair) -> np.ndarray:
    """`(x_f32 @ A) @ B`.  loader/latent_runtime.py:35-36."""
    return (np.asarray(x, dtype=np.float32) @ pair.a) @ pair.b


def silu(x: np.ndarray) -> np.ndarray:
    """float64 SiLU, clipped, cast to fp32.  loader/latent_runtime.py:39-45."""
    x64 = np.asarray(x, dtype=np.float32).astype(np.float64)
    with np.errstate(over="ignore"):
        result = x64 / (1.0 + np.exp(-x64))
    return np.clip(result, -1e30, 1e30).astype(np.float32)


def swiglu_expert(
    x: np.ndarray,
    gate: FactorPair,
    up: FactorPair,
    down: FactorPair,
    weight: float = 1.0,
    weight_before_down: bool = False,
) -> np.ndarray:
    """The expert forward.  loader/latent_runtime.py:48-59.

    `weight` is applied (as fp32) to the hidden activations only when
    `weight_before_down`; otherwise it is ignored, as in the reference.
    """
    hidden = silu(project(x, gate)) * project(x, up)
    if weight_before_down:
        hidden = hidden * np.float32(weight)
    return project(hidden, down)


def dense_swiglu_expert(
    x: np.ndarray,
    gate: np.ndarray,
    up: np.ndarray,
    down: np.ndarray,
    weight: float = 1.0,
    weight_before_down: bool = False,
) -> np.ndarray:
    """Dense fp32 SwiGLU.  loader/latent_runtime.py:62-73."""
    xf = np.asarray(x, dtype=np.float32)
    hidden = silu(xf @ gate) * (xf @ up)
    if weight_before_down:
        hidden = hidden * np.float32(weight)
    return hidden @ down


def relative_frobenius_error(reference: np.ndarray, candidate: np.ndarray) -> float:
    """loader/latent_loader.py:188-192."""
    denom = np.linalg.norm(reference)
    if denom == 0:
        return 0.0
    return float(np.linalg.norm(np.asarray(reference) - np.asarray(candidate)) / denom)


def quantization_snr_by_group(reference: np.ndarray, candidate: np.ndarray, group_size: int) -> np.ndarray:
    """Per-group ||x|| / max(||x - q||, 1e-12) over the flattened arrays, each
    zero-padded to whole groups; fp32 norms.  loader/latent_loader.py:173-185."""
    ref = np.asarray(reference, dtype=np.float32).reshape(-1)
    cand = np.asarray(candidate, dtype=np.float32).reshape(-1)
    groups = int(math.ceil(ref.size / group_size))
    padded_ref = np.zeros(groups * group_size, dtype=np.float32)
    padded_cand = np.zeros(groups * group_size, dtype=np.float32)
    padded_ref[: ref.size] = ref
    padded_cand[: cand.size] = cand
    signal = np.linalg.norm(padded_ref.reshape(groups, group_size), axis=1)
    noise = np.linalg.norm((padded_ref - padded_cand).reshape(groups, group_size), axis=1)
    return signal / np.maximum(noise, 1e-12)


def int8_group_mask(values: np.ndarray, snr_threshold: float) -> np.ndarray:
    """bool [rows, cols/32]: the non-zero row groups of [rows, cols] whose NF4
    round trip has SNR below `snr_threshold`.

    No reference counterpart as a per-group selector: the reference computes
    this SNR (quantization_snr_by_group of quantize_nf4 / dequantize_nf4,
    loader/latent_loader.py:173-185, 216-223) and switches a whole factor to
    INT8 when too many groups fall below the threshold (:227-229).  With
    cols % 32 == 0 the per-row groups are the reference's flat groups.
    """
    v = np.asarray(values, dtype=np.float32)
    rows, cols = v.shape
    codes, scales = pack_rows(v)
    decoded = unpack_rows(codes, scales)
    snr = quantization_snr_by_group(v, decoded, GROUP).reshape(rows, cols // GROUP)
    nonzero = np.abs(v.reshape(rows, cols // GROUP, GROUP)).max(axis=2) > 0
    return (snr < np.float32(snr_threshold)) & nonzero


def rel_l2(reference: np.ndarray, candidate: np.ndarray) -> float:
    """Relative L2 error in float64 (the parity metric)."""
    ref = np.asarray(reference, dtype=np.float64)
    cand = np.asarray(candidate, dtype=np.float64)
    denom = np.linalg.norm(ref)
    return float(np.linalg.norm(ref - cand) / denom) if denom else float(np.linalg.norm(cand))


# ----------------------------------------------------------------------------
# Stacked per-expert layout  (loader/write_latent_gguf.py)
# ----------------------------------------------------------------------------
def stack_pad(factors: Sequence[np.ndarray], pad_to: int) -> np.ndarray:
    """(E, max rows, pad_to) fp32, zero padded.  loader/write_latent_gguf.py:101-123."""
    out_rows = max(f.shape[0] for f in factors)
    stacked = np.zeros((len(factors), out_rows, pad_to), dtype=np.float32)
    for i, f in enumerate(factors):
        nr = min(f.shape[0], out_rows)
        nc = min(f.shape[1], pad_to)
        stacked[i, :nr, :nc] = f[:nr, :nc]
    return stacked


def pack_rows(matrix: np.ndarray, group_size: int = GROUP) -> Tuple[np.ndarray, np.ndarray]:
    """Per-row NF4 pack of a [..., rows, cols] array.  loader/write_latent_gguf.py:227-257.

    Each row is quantized on its own (groups never straddle rows); the last
    axis is zero-padded to a multiple of the group size.  Codes come out as
    [..., rows, padded_cols/2] uint8 and scales as [..., rows, groups] fp16.
    With cols a multiple of the group size this equals one flat
    `quantize_nf4` over the whole array, which is how it is computed here.
    """
    m = np.asarray(matrix, dtype=np.float32)
    cols = m.shape[-1]
    n_groups = (cols + group_size - 1) // group_size
    padded_last = n_groups * group_size
    if padded_last != cols:
        pad = [(0, 0)] * (m.ndim - 1) + [(0, padded_last - cols)]
        m = np.pad(m, pad)
    packed, scales, _ = quantize_nf4(m, group_size=group_size)
    lead = m.shape[:-1]
    return packed.reshape(*lead, padded_last // 2), scales.reshape(*lead, n_groups)


def unpack_rows(codes: np.ndarray, scales: np.ndarray, group_size: int = GROUP) -> np.ndarray:
    """fp32 [..., rows, cols] from per-row packed codes.  tests/test_write_latent_gguf.py:222-252."""
    codes = np.asarray(codes, dtype=np.uint8)
    cols = codes.shape[-1] * 2
    vals = np.empty(codes.shape[:-1] + (cols,), dtype=np.uint8)
    vals[..., 0::2] = codes & 0x0F
    vals[..., 1::2] = codes >> 4
    s = np.asarray(scales).astype(np.float32)
    decoded = NF4_CODEBOOK[vals].reshape(codes.shape[:-1] + (cols // group_size, group_size))
    return (decoded * s[..., np.newaxis]).reshape(codes.shape[:-1] + (cols,))


# ----------------------------------------------------------------------------
# Per-group INT8 extension (no reference counterpart)
# ----------------------------------------------------------------------------
@dataclass
class Int8Groups:
    """Per-group INT8 fallback for one stacked factor.

    bitmap     uint32 [E, rows, words]   bit g of the row set => group g is INT8
    data       int8   [n_int8_groups, 32] the INT8 values of every flagged group,
                                           row-major over (e, row, group)
    row_offset int32  [E, rows]           index into `data` of the row's first
                                           flagged group
    The group's fp16 scale lives in the ordinary scale array (absmax/127) and
    its 16 NF4 code bytes are zero.  Dequant = f32(q) * f32(scale), i.e.
    loader/latent_loader.py:161-170 at group 32.
    """

    bitmap: np.ndarray
    data: np.ndarray
    row_offset: np.ndarray


def pack_rows_mixed(matrix: np.ndarray, int8_mask: np.ndarray) -> Tuple[np.ndarray, np.ndarray, Int8Groups]:
    """Per-row NF4 pack with selected groups stored as INT8 instead.

    matrix [E, rows, cols] fp32 (cols a multiple of 32); int8_mask
    [E, rows, cols/32] bool.  NF4 groups follow `pack_rows`; INT8 groups follow
    `quantize_int8(group, group_size=32)`.
    """
    m = np.asarray(matrix, dtype=np.float32)
    E, rows, cols = m.shape
    assert cols % GROUP == 0
    groups = cols // GROUP
    codes, scales = pack_rows(m)
    mask = np.asarray(int8_mask, dtype=bool).reshape(E, rows, groups)
    words = (groups + 31) // 32
    bitmap = np.zeros((E, rows, words), dtype=np.uint32)
    gi, ri, ci = np.nonzero(mask)
    for w in range(words):
        sel = (ci // 32) == w
        np.bitwise_or.at(bitmap[:, :, w], (gi[sel], ri[sel]), (np.uint32(1) << (ci[sel] % 32).astype(np.uint32)))
    per_row = mask.sum(axis=2).reshape(-1)
    row_offset = np.zeros(E * rows, dtype=np.int64)
    row_offset[1:] = np.cumsum(per_row)[:-1]
    if row_offset.size and row_offset[-1] + per_row[-1] >= 2**31:
        raise ValueError("too many INT8 groups for int32 row offsets")
    grouped = m.reshape(E, rows, groups, GROUP)
    sel_vals = grouped[mask]  # (n, 32), row-major order of (e, row, group)
    q, s, _ = quantize_int8(sel_vals, group_size=GROUP)
    data = q.reshape(-1, GROUP)
    scales = scales.copy()
    scales[mask] = s
    codes = codes.reshape(E, rows, groups, GROUP // 2).copy()
    codes[mask] = 0
    return codes.reshape(E, rows, cols // 2), scales, Int8Groups(bitmap, data, row_offset.astype(np.int32).reshape(E, rows))


def unpack_rows_mixed(codes: np.ndarray, scales: np.ndarray, ext: Optional[Int8Groups], e: int) -> np.ndarray:
    """fp32 [rows, cols] of expert `e` from the mixed NF4/INT8 layout."""
    vals = unpack_rows(codes[e], scales[e])
    if ext is None:
        return vals
    rows, cols = vals.shape
    groups = cols // GROUP
    s = np.asarray(scales[e]).astype(np.float32)
    # flagged[r, g]: bit g % 32 of word g // 32 of row r's bitmap.
    words = np.asarray(ext.bitmap[e], dtype=np.uint32)
    g = np.arange(groups)
    flagged = ((words[:, g // 32] >> (g % 32).astype(np.uint32)) & np.uint32(1)).astype(bool)
    # A flagged group's values sit at data[row_offset + (flagged groups before it in the row)].
    before = np.cumsum(flagged, axis=1) - 1
    idx = np.asarray(ext.row_offset[e], dtype=np.int64)[:, None] + before
    q = np.asarray(ext.data)[idx[flagged]].astype(np.float32)  # [n, 32]
    grouped = vals.reshape(rows, groups, GROUP)
    grouped[flagged] = q * s[flagged][:, None]
    return grouped.reshape(rows, cols)


# ----------------------------------------------------------------------------
# Stacked layer and layer-level forward
# ----------------------------------------------------------------------------
FACTOR_NAMES = ("gate_a", "gate_b", "up_a", "up_b", "down_a", "down_b")


@dataclass
class StackedFactor:
    codes: np.ndarray  # uint8 [E, rows, cols/2]
    scales: np.ndarray  # float16 [E, rows, cols/32]
    int8: Optional[Int8Groups] = None

    def expert(self, e: int) -> np.ndarray:
        return unpack_rows_mixed(self.codes, self.scales, self.int8, e)


@dataclass
class StackedLayer:
    """One layer's 12 stacked operands (+ optional INT8 extension).

    Shapes follow patches/002-latent-gguf-tensors.patch:135-148 with the packed
    code axis of tests/test_write_latent_gguf.py:112-154:
      gate_a, up_a : [E, d, R/2]    gate_b, up_b : [E, R, ff/2]
      down_a       : [E, ff, R/2]   down_b       : [E, R, d/2]
    """

    factors: Dict[str, StackedFactor]
    d: int
    ff: int
    max_rank: int
    ranks: Optional[np.ndarray] = None  # int32 [E, 3] true (gate, up, down) ranks

    @property
    def n_expert(self) -> int:
        return int(self.factors["gate_a"].codes.shape[0])

    def pairs(self, e: int) -> Tuple[FactorPair, FactorPair, FactorPair]:
        f = self.factors
        return (
            FactorPair(f["gate_a"].expert(e), f["gate_b"].expert(e)),
            FactorPair(f["up_a"].expert(e), f["up_b"].expert(e)),
            FactorPair(f["down_a"].expert(e), f["down_b"].expert(e)),
        )

    def expert_bytes(self, e: int, true_rank: bool = True) -> int:
        """Packed bytes of expert e (codes + scales + INT8 side data)."""
        total = 0
        for name in FACTOR_NAMES:
            f = self.factors[name]
            rows, half = f.codes.shape[1], f.codes.shape[2]
            cols = half * 2
            kind = ("gate", "up", "down").index(name.split("_")[0])
            r = int(self.ranks[e, kind]) if (true_rank and self.ranks is not None) else self.max_rank
            if name.endswith("_a"):
                used_rows, used_cols = rows, min(cols, ((r + GROUP - 1) // GROUP) * GROUP)
            else:
                used_rows, used_cols = min(rows, r), cols
            groups = used_cols // GROUP
            n_int8 = 0
            if f.int8 is not None:
                for row in range(used_rows):
                    for w in range((groups + 31) // 32):
                        bits = int(f.int8.bitmap[e, row, w])
                        lim = groups - 32 * w
                        if lim < 32:
                            bits &= (1 << lim) - 1
                        n_int8 += bin(bits).count("1")
            n_groups = used_rows * groups
            total += (n_groups - n_int8) * (GROUP // 2) + n_int8 * GROUP + n_groups * 2
        return total


def build_stacked_layer(
    a_factors: Dict[str, Sequence[np.ndarray]],
    b_factors: Dict[str, Sequence[np.ndarray]],
    d: int,
    ff: int,
    max_rank: int,
    int8_masks: Optional[Dict[str, np.ndarray]] = None,
) -> StackedLayer:
    """Stack, pad and pack per-expert factors.  loader/write_latent_gguf.py:212-257.

    a_factors[kind][e] is [n_in, r_e], b_factors[kind][e] is [r_e, n_out].
    A is padded along its columns to max_rank, B along its rows (the writer's
    `_stack_per_expert_factors` pads rows to the largest rank present; here
    the row count is fixed to max_rank so every layer has one shape).
    """
    factors: Dict[str, StackedFactor] = {}
    n_expert = len(a_factors["gate"])
    ranks = np.zeros((n_expert, 3), dtype=np.int32)
    for k, kind in enumerate(("gate", "up", "down")):
        n_out = ff if kind != "down" else d
        n_in = d if kind != "down" else ff
        a_st = np.zeros((n_expert, n_in, max_rank), dtype=np.float32)
        b_st = np.zeros((n_expert, max_rank, n_out), dtype=np.float32)
        for e in range(n_expert):
            a, b = a_factors[kind][e], b_factors[kind][e]
            r = a.shape[1]
            ranks[e, k] = r
            a_st[e, :, :r] = a
            b_st[e, :r, :] = b
        for side, st in (("a", a_st), ("b", b_st)):
            name = f"{kind}_{side}"
            if int8_masks is not None and name in int8_masks:
                codes, scales, ext = pack_rows_mixed(st, int8_masks[name])
                factors[name] = StackedFactor(codes, scales, ext)
            else:
                codes, scales = pack_rows(st)
                factors[name] = StackedFactor(codes, scales)
    return StackedLayer(factors=factors, d=d, ff=ff, max_rank=max_rank, ranks=ranks)


def moe_forward(
    x: np.ndarray,
    ids: np.ndarray,
    weights: np.ndarray,
    layer: StackedLayer,
    weight_before_down: bool = False,
    out_mode: int = 0,
) -> np.ndarray:
    """Layer-level LATENT MoE expert FFN (no reference counterpart as code).

    For each distinct expert referenced by a valid slot (0 <= id < E), dequantize
    its six factors once and run the swiglu_expert chain
    (loader/latent_runtime.py:48-59) on the gathered tokens, with per-slot
    router weights applied before down when `weight_before_down`.

    out_mode 0: f32 [T, d] = sum over slots of w * y  (y if weight_before_down),
                the reduce of README.md:111-113.
    out_mode 1: f32 [T, k, d] per-slot, unweighted unless weight_before_down --
                the dst of kernels/latent_fused_expert_ffn.cu:255-286; dropped
                slots are zero (kernels/latent_fused_expert_ffn.cu:34-40).
    """
    x = np.asarray(x, dtype=np.float32)
    ids = np.asarray(ids, dtype=np.int64)
    w = np.asarray(weights, dtype=np.float32)
    T, K = ids.shape
    E = layer.n_expert
    per_slot = np.zeros((T, K, layer.d), dtype=np.float32)
    valid = (ids >= 0) & (ids < E)
    for e in np.unique(ids[valid]):
        tok, slot = np.nonzero(ids == e)
        gate, up, down = layer.pairs(int(e))
        xs = x[tok]
        hidden = silu(project(xs, gate)) * project(xs, up)
        if weight_before_down:
            hidden = hidden * w[tok, slot][:, np.newaxis]
        per_slot[tok, slot] = project(hidden, down)
    if out_mode == 1:
        return per_slot
    out = np.zeros((T, layer.d), dtype=np.float32)
    for k in range(K):
        scale = np.where(valid[:, k], np.float32(1.0) if weight_before_down else w[:, k], np.float32(0.0))
        out += per_slot[:, k] * scale.astype(np.float32)[:, np.newaxis]
    return out


def distinct_experts(ids: np.ndarray, n_expert: int) -> np.ndarray:
    ids = np.asarray(ids)
    return np.unique(ids[(ids >= 0) & (ids < n_expert)])
