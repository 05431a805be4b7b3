"""Seeded numpy generators for the small parity workloads, and the
load-time factorization restated in numpy.

TEST INFRASTRUCTURE ONLY (see `oracle/__init__.py`).

Spectrum: s_i = 0.02 * i^-0.7.  Singular vectors: Q factors of Gaussian
matrices.  Factors: A = U_r sqrt(S_r), B = sqrt(S_r) V_r^T (the make_factors of
loader/latent_loader.py:104-108).  Per-expert seed = base + expert id, after
loader/write_latent_gguf.py:190.
"""

from __future__ import annotations

from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np

from . import latent_ref as ref


def spectrum(n: int) -> np.ndarray:
    i = np.arange(1, n + 1, dtype=np.float64)
    return 0.02 * i ** -0.7


def orthonormal(rng: np.random.Generator, n: int, r: int) -> np.ndarray:
    q, _ = np.linalg.qr(rng.standard_normal((n, r)))
    return q


def make_factors(u: np.ndarray, s: np.ndarray, vt: np.ndarray, rank: int) -> Tuple[np.ndarray, np.ndarray]:
    """loader/latent_loader.py:104-108."""
    root = np.sqrt(s[:rank]).astype(np.float32)
    a = u[:, :rank].astype(np.float32) * root[np.newaxis, :]
    b = root[:, np.newaxis] * vt[:rank, :].astype(np.float32)
    return a, b


def closed_form_factors(rng: np.random.Generator, n_in: int, n_out: int, rank: int):
    """Rank-r factors of U diag(s) V^T without forming or decomposing W."""
    s = spectrum(rank)
    u = orthonormal(rng, n_in, rank)
    v = orthonormal(rng, n_out, rank)
    return make_factors(u, s, v.T, rank)


def dense_with_noise(rng: np.random.Generator, n_in: int, n_out: int, noise_sigma: float = 1e-4) -> np.ndarray:
    """W = U diag(s) V^T + N(0, sigma^2) noise, sigma read as 1e-4."""
    n = min(n_in, n_out)
    s = spectrum(n)
    u = orthonormal(rng, n_in, n)
    v = orthonormal(rng, n_out, n)
    w = (u * s[np.newaxis, :]) @ v.T
    return (w + noise_sigma * rng.standard_normal((n_in, n_out))).astype(np.float32)


def svd_factors(w: np.ndarray, rank: int) -> Tuple[np.ndarray, np.ndarray]:
    u, s, vt = np.linalg.svd(np.asarray(w, dtype=np.float32), full_matrices=False)
    return make_factors(u, s, vt, rank)


def config0_expert(seed: int = 0, d: int = 512, ff: int = 1408, rank: int = 64):
    """Single-expert CPU plumbing workload: dense W, SVD factors, NPZ-style arrays.

    Returns (arrays, dense, x) where `arrays` uses the NPZ key scheme of
    loader/latent_loader.py:253-260 (`<name>.{a,b}.{nf4,scales,shape}`).
    """
    rng = np.random.default_rng(seed)
    dense = {
        "gate": dense_with_noise(rng, d, ff),
        "up": dense_with_noise(rng, d, ff),
        "down": dense_with_noise(rng, ff, d),
    }
    arrays: Dict[str, np.ndarray] = {}
    for name, w in dense.items():
        a, b = svd_factors(w, rank)
        for side, f in (("a", a), ("b", b)):
            packed, scales, shape = ref.quantize_nf4(f, group_size=32)
            arrays[f"{name}.{side}.nf4"] = packed
            arrays[f"{name}.{side}.scales"] = scales
            arrays[f"{name}.{side}.shape"] = np.array(shape, dtype=np.int32)
    x = rng.standard_normal((4, d)).astype(np.float32)
    return arrays, dense, x


def make_layer(
    seed: int,
    n_expert: int,
    d: int,
    ff: int,
    max_rank: int,
    ranks: Optional[Sequence[int]] = None,
    int8_fraction: float = 0.0,
) -> ref.StackedLayer:
    """A stacked layer with closed-form factors; optional per-expert ranks and INT8 groups."""
    a_f: Dict[str, List[np.ndarray]] = {"gate": [], "up": [], "down": []}
    b_f: Dict[str, List[np.ndarray]] = {"gate": [], "up": [], "down": []}
    for e in range(n_expert):
        rng = np.random.default_rng(seed + e)
        r = int(ranks[e]) if ranks is not None else max_rank
        for kind, (n_in, n_out) in (("gate", (d, ff)), ("up", (d, ff)), ("down", (ff, d))):
            a, b = closed_form_factors(rng, n_in, n_out, r)
            a_f[kind].append(a)
            b_f[kind].append(b)
    masks = None
    if int8_fraction > 0:
        rng = np.random.default_rng(seed + 1_000_003)
        masks = {}
        for name in ref.FACTOR_NAMES:
            kind = name.split("_")[0]
            n_in, n_out = {"gate": (d, ff), "up": (d, ff), "down": (ff, d)}[kind]
            rows, cols = (n_in, max_rank) if name.endswith("_a") else (max_rank, n_out)
            m = rng.random((n_expert, rows, cols // ref.GROUP)) < int8_fraction
            # Only groups inside each expert's true rank are eligible.
            for e in range(n_expert):
                r = int(ranks[e]) if ranks is not None else max_rank
                if name.endswith("_a"):
                    m[e, :, (r + ref.GROUP - 1) // ref.GROUP:] = False
                else:
                    m[e, r:, :] = False
            masks[name] = m
    return ref.build_stacked_layer(a_f, b_f, d, ff, max_rank, int8_masks=masks)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round fp32 to the nearest bfloat16 (ties to even), returned as fp32."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32)


def randomized_svd(matrix: np.ndarray, target_rank: int, oversample: int = 16, power_iterations: int = 1,
                   seed: int = 0):
    """numpy restatement of randomized_svd (loader/latent_loader.py:66-86): same
    sketch draw, power iteration, reduced QR and SVD of the projection."""
    m, n = matrix.shape
    rank = min(target_rank, m, n)
    sketch = min(rank + oversample, m, n)
    omega = np.random.default_rng(seed).standard_normal((n, sketch), dtype=np.float32)
    y = matrix @ omega
    for _ in range(power_iterations):
        y = matrix @ (matrix.T @ y)
    q, _ = np.linalg.qr(y, mode="reduced")
    u_hat, s, vt = np.linalg.svd(q.T @ matrix, full_matrices=False)
    return (q @ u_hat)[:, :rank], s[:rank], vt[:rank, :]


def choose_rank(singular_values: np.ndarray, energy: float, min_rank: int, max_rank: int) -> int:
    """numpy restatement of choose_rank (loader/latent_loader.py:89-97)."""
    if not 0 < energy <= 1:
        raise ValueError("energy must be in (0, 1]")
    s = np.asarray(singular_values, np.float64)
    total = float(np.sum(s ** 2))
    if total == 0:
        return min_rank
    rank = int(np.searchsorted(np.cumsum(s ** 2) / total, energy) + 1)
    return max(min_rank, min(rank, max_rank, s.size))


def compress_matrix(name: str, matrix: np.ndarray, energy: float = 0.95, min_rank: int = 16, max_rank: int = 128,
                    group_size: int = 32, int8_group_size: int = 64, error_threshold: float = 0.02,
                    snr_threshold: float = 3.0, low_snr_fraction_threshold: float = 0.05, seed: int = 0):
    """numpy restatement of compress_matrix (loader/latent_loader.py:195-285);
    defaults are the CLI's (:292-303).

    Rank from the full spectrum's energy, randomized SVD, A = U sqrt(S),
    B = sqrt(S) V^T, flat NF4 of both factors; the whole pair switches to INT8
    (group int8_group_size) when more than low_snr_fraction_threshold of the
    NF4 groups have SNR below snr_threshold and INT8 reconstructs the matrix
    better; a dense fp16 copy is added when the error still exceeds
    error_threshold.  Returns (arrays with the artifact's NPZ keys, report dict).
    """
    matrix = np.asarray(matrix, dtype=np.float32)
    full_s = np.linalg.svd(matrix, compute_uv=False)
    rank = choose_rank(full_s, energy, min_rank, max_rank)
    u, s, vt = randomized_svd(matrix, rank, seed=seed)
    root = np.sqrt(s[:rank]).astype(np.float32)
    a = u[:, :rank].astype(np.float32) * root[np.newaxis, :]
    b = root[:, np.newaxis] * vt[:rank, :].astype(np.float32)
    dense_error = ref.relative_frobenius_error(matrix, a @ b)
    a_packed, a_scales, a_shape = ref.quantize_nf4(a, group_size=group_size)
    b_packed, b_scales, b_shape = ref.quantize_nf4(b, group_size=group_size)
    aq = ref.dequantize_nf4(a_packed, a_scales, a_shape, group_size=group_size)
    bq = ref.dequantize_nf4(b_packed, b_scales, b_shape, group_size=group_size)
    quant_error = ref.relative_frobenius_error(matrix, aq @ bq)
    snr = np.concatenate([ref.quantization_snr_by_group(a, aq, group_size),
                          ref.quantization_snr_by_group(b, bq, group_size)])
    low_snr_fraction = float(np.mean(snr < snr_threshold)) if snr.size else 0.0
    quantization = "nf4_g%d" % group_size
    use_int8 = low_snr_fraction > low_snr_fraction_threshold
    arrays: Dict[str, np.ndarray] = {}
    if use_int8:
        a_i8, a_i8s, _ = ref.quantize_int8(a, group_size=int8_group_size)
        b_i8, b_i8s, _ = ref.quantize_int8(b, group_size=int8_group_size)
        aq8 = ref.dequantize_int8(a_i8, a_i8s, a_shape, group_size=int8_group_size)
        bq8 = ref.dequantize_int8(b_i8, b_i8s, b_shape, group_size=int8_group_size)
        int8_error = ref.relative_frobenius_error(matrix, aq8 @ bq8)
        if int8_error < quant_error:
            quant_error = int8_error
            arrays = {f"{name}.a.int8": a_i8, f"{name}.a.scales": a_i8s,
                      f"{name}.b.int8": b_i8, f"{name}.b.scales": b_i8s}
            quantization = "int8_g%d" % int8_group_size
        else:
            use_int8 = False
    if not use_int8:
        arrays = {f"{name}.a.nf4": a_packed, f"{name}.a.scales": a_scales,
                  f"{name}.b.nf4": b_packed, f"{name}.b.scales": b_scales}
    arrays[f"{name}.a.shape"] = np.array(a_shape, dtype=np.int32)
    arrays[f"{name}.b.shape"] = np.array(b_shape, dtype=np.int32)
    fallback = quant_error > error_threshold
    if fallback:
        arrays[f"{name}.dense_fallback"] = matrix.astype(np.float16)
    report = {"rank": rank, "dense_relative_error": dense_error, "quantized_relative_error": quant_error,
              "low_snr_group_fraction": low_snr_fraction, "quantization": quantization, "fallback": fallback}
    return arrays, report
