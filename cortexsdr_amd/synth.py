"""Seeded synthetic workloads for the configurations the path is measured on.

Generator (fully specified, portable): SplitMix64 in counter form,
    z_i = mix64(seed + (i + 1) * 0x9E3779B97F4A7C15)
    mix64(z): z ^= z >> 30; z *= 0xBF58476D1CE4E5B9; z ^= z >> 27; z *= 0x94D049BB133111EB;
              z ^= z >> 31
    uniform u_i = (z_i >> 11) * 2^-53 in [0, 1)
    normal: Box-Muller on consecutive pairs (u_2i, u_2i+1):
              rho = sqrt(-2 ln(1 - u_2i)), n_2i = rho cos(2 pi u_2i+1), n_2i+1 = rho sin(...)
Each array draws from its own seed stream (a different 64-bit seed), so arrays do not
depend on each other's sizes. "N(0, 0.5)" coefficients use standard deviation 0.5.
"""
from __future__ import annotations

import numpy as np

from . import formats

_GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def _stream_seed(seed: int, stream: int) -> np.uint64:
    return np.uint64((seed * 0x100000001B3 + stream * 0xD1B54A32D192ED03) & 0xFFFFFFFFFFFFFFFF)


def splitmix64(seed: int, n: int, stream: int = 0) -> np.ndarray:
    s = _stream_seed(seed, stream)
    with np.errstate(over="ignore"):
        z = s + (np.arange(1, n + 1, dtype=np.uint64) * _GAMMA)
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        z = z ^ (z >> np.uint64(31))
    return z


def uniform(seed: int, n: int, stream: int = 0) -> np.ndarray:
    return (splitmix64(seed, n, stream) >> np.uint64(11)).astype(np.float64) * (2.0 ** -53)


def normal(seed: int, n: int, stream: int = 0, sigma: float = 1.0) -> np.ndarray:
    m = (n + 1) // 2
    u = uniform(seed, 2 * m, stream).reshape(m, 2)
    rho = np.sqrt(-2.0 * np.log1p(-u[:, 0]))
    th = 2.0 * np.pi * u[:, 1]
    out = np.empty((m, 2))
    out[:, 0] = rho * np.cos(th)
    out[:, 1] = rho * np.sin(th)
    return (out.reshape(-1)[:n] * sigma)


def distinct_indices(seed: int, n_sets: int, k: int, K: int, stream: int = 0) -> np.ndarray:
    """n_sets rows of k distinct values uniform in [0, K) (sequential sampling without
    replacement: draw rank v_j uniform in [0, K - j), map it to the v_j-th unused value)."""
    if k > K:
        raise ValueError("cannot draw more distinct values than K")
    u = uniform(seed, n_sets * k, stream).reshape(n_sets, k)
    sel = np.empty((n_sets, k), np.int64)
    for j in range(k):
        c = np.minimum(np.floor(u[:, j] * (K - j)).astype(np.int64), K - j - 1)
        prev = np.sort(sel[:, :j], axis=1)
        for i in range(j):
            c = c + (prev[:, i] <= c)
        sel[:, j] = c
    return sel


def dictionary(K: int, B: int, seed: int) -> np.ndarray:
    """K unit-norm atoms of length B (Gaussian, normalised)."""
    D = normal(seed, K * B, stream=11).reshape(K, B)
    D /= np.linalg.norm(D, axis=1, keepdims=True)
    return D.astype(np.float32)


def block_codes(R: int, C: int, K: int, s: int, seed: int, sigma: float = 0.5, B: int = 64):
    """idx (R*NB, s) uint16 distinct per block, coef (R*NB, s) fp16 ~ N(0, sigma)."""
    NB = C // B
    n = R * NB
    idx = distinct_indices(seed, n, s, K, stream=21).astype(np.uint16)
    coef = normal(seed, n * s, stream=22, sigma=sigma).astype(np.float16).reshape(n, s)
    return idx, coef


def hsdb_layer(R: int, C: int, K: int, s: int, seed_dict: int = 1, seed_codes: int = 2,
               sigma: float = 0.5, B: int = 64, D: np.ndarray | None = None,
               edge_seed: int = 4) -> bytes:
    """One HSDB-coded R x C matrix (configs 1/2 of the measured workload)."""
    if D is None:
        D = dictionary(K, B, seed_dict)
    idx, coef = block_codes(R, C, K, s, seed_codes, sigma, B)
    ce = C - (C // B) * B
    edge = None
    if ce:
        edge = (normal(edge_seed, R * ce, stream=31, sigma=0.05)
                .astype(np.float32).reshape(R, ce))
    return formats.pack_hsdb(R, C, D, idx, coef, edge=edge)


def activations(C: int, M: int, seed: int = 3, dtype=np.float32) -> np.ndarray:
    """X (C, M) ~ N(0, 1), feature-major."""
    return normal(seed, C * M, stream=41).astype(dtype).reshape(C, M)


def q4k_matrix(R: int, C: int, seed: int, order: str = "ggml") -> bytes:
    """R x C Q4_K matrix: q uniform [0,15], 6-bit scales/mins uniform [0,63],
    d and dmin fp16 ~ U(0.001, 0.05)."""
    if C % 256:
        raise ValueError("C must be a multiple of 256")
    n = R * C // 256
    q = (uniform(seed, n * 256, stream=51) * 16).astype(np.uint8).reshape(n, 256)
    sc = (uniform(seed, n * 8, stream=52) * 64).astype(np.uint8).reshape(n, 8)
    mn = (uniform(seed, n * 8, stream=53) * 64).astype(np.uint8).reshape(n, 8)
    d = (0.001 + 0.049 * uniform(seed, n, stream=54)).astype(np.float16).view(np.uint16)
    dmin = (0.001 + 0.049 * uniform(seed, n, stream=55)).astype(np.float16).view(np.uint16)
    return formats.pack_q4k(d, dmin, sc, mn, q, order)
