"""Seeded synthetic inputs for the quantized-inference configurations.

Every generator is a pure function of its seed (numpy PCG64), so the GPU path
and the CPU checker see identical bytes. Shapes follow the benchmark
configurations: decode GEMV, prefill GEMM, ternary matmul, RotorQuant KV and
the 784-256-128-10 int8 MLP.
"""
from __future__ import annotations

import numpy as np

PREFILL = dict(m=2048, k=4096, n=14336)
GEMV_SHAPES = [(m, 4096, n) for n in (4096, 11008) for m in (1, 8, 16)]
TERNARY = dict(m=512, k=4096, n=4096)
ROTORQUANT = dict(batch=8, heads=32, seq=4096, head_dim=128, bits=4)
MLP_LAYERS = (784, 256, 128, 10)
MLP_BATCH = 32


def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def weights(n: int, k: int, seed: int, std: float = 0.02) -> np.ndarray:
    """W ~ N(0, std) f32 [n, k] (output channels x input features)."""
    return (rng(seed).standard_normal((n, k), dtype=np.float32) * np.float32(std)).astype(np.float32)


def activations(m: int, k: int, seed: int, outlier_frac: float = 0.0,
                outlier_scale: float = 20.0) -> np.ndarray:
    """x ~ N(0, 1) f32 [m, k]; each element is multiplied by outlier_scale
    with probability outlier_frac (seeded Bernoulli)."""
    g = rng(seed)
    x = g.standard_normal((m, k), dtype=np.float32)
    if outlier_frac > 0:
        mask = g.random((m, k), dtype=np.float32) < outlier_frac
        x = np.where(mask, x * np.float32(outlier_scale), x).astype(np.float32)
    return x


def rotors(n_groups: int, seed: int) -> np.ndarray:
    """Unit Cl(3,0) rotors {s, p12, p13, p23} drawn with the formula of
    Rotor::random (src/quant.rs:39-65): a, b, c ~ U(-1,1), theta ~ U(0, pi),
    R = cos(theta/2) + sin(theta/2) * (a e12 + b e13 + c e23)/|(a,b,c)|,
    evaluated in f32."""
    g = rng(seed)
    out = np.empty((n_groups, 4), np.float32)
    for i in range(n_groups):
        a, b, c = (np.float32(g.uniform(-1.0, 1.0)) for _ in range(3))
        theta = np.float32(g.uniform(0.0, np.pi))
        norm = np.sqrt(np.float32(a * a + b * b + c * c), dtype=np.float32)
        if norm < np.float32(1e-8):
            out[i] = (1.0, 0.0, 0.0, 0.0)
            continue
        half = np.float32(theta / np.float32(2.0))
        s, mag = np.cos(half, dtype=np.float32), np.sin(half, dtype=np.float32)
        out[i] = (s, mag * (a / norm), mag * (b / norm), mag * (c / norm))
    return out


def kv_outlier_channels(head_dim: int, seed: int, frac: float = 0.02) -> np.ndarray:
    """Indices of the head_dim channels scaled x10 (round(frac*head_dim) of them)."""
    n = int(round(frac * head_dim))
    return np.sort(rng(seed).choice(head_dim, size=n, replace=False))


def ternary_latent(n: int, k: int, seed: int) -> np.ndarray:
    """Latent ternary weights ~ N(0, 1) f32 [n, k] (absmean rule gives ~31% zeros)."""
    return rng(seed).standard_normal((n, k), dtype=np.float32)
