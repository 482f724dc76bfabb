"""Seeded synthetic operands shared by the tests (generated on the CPU)."""

from __future__ import annotations

import functools

import numpy as np
import torch

from oracle import hif8_oracle as o

HIF8_MAX = 32768.0
# Projection shapes (N, K) of one 9B-class decoder layer: q, fused k+v, o, fused gate+up, down.
LAYER_SHAPES = [(4096, 4096), (2048, 4096), (4096, 4096), (24576, 4096), (4096, 12288)]


def bf16_activation(m: int, k: int, seed: int, heavy_tail: bool = False) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=g, dtype=torch.float32)
    if heavy_tail:
        cols = torch.randperm(k, generator=g)[: max(1, int(np.ceil(0.001 * k)))]
        x[:, cols] *= 50.0
    return x.to(torch.bfloat16)


def input_scale_of(x: torch.Tensor) -> torch.Tensor:
    """Static per-tensor scale mapping absmax to the HiF8 maximum."""
    return torch.tensor([float(x.float().abs().max()) / HIF8_MAX], dtype=torch.float32)


@functools.lru_cache(maxsize=8)
def hif8_weight(n: int, k: int, seed: int) -> tuple[np.ndarray, np.ndarray]:
    """W ~ N(0, 0.02) fp32 -> per-row scale absmax/32768 -> static-encoded bytes."""
    g = torch.Generator().manual_seed(seed)
    w = (torch.randn(n, k, generator=g, dtype=torch.float32) * 0.02).numpy()
    ws = (np.abs(w).max(axis=1) / HIF8_MAX).astype(np.float32)
    data, _ = o.static_quant_rows(w, ws)
    return data, ws


def random_codes(shape, seed: int, high: int = 111) -> np.ndarray:
    """Finite codes 0..110 (no Inf/NaN), as the reference tests draw them."""
    return np.random.default_rng(seed).integers(0, high, shape, dtype=np.uint8)


C1_SEED = 20261201


def c1_operands():
    """BASELINE configs[0] (the CPU-reference GEMV): x bf16 [1, 4096] ~ N(0, 1)
    with input_scale = absmax / 32768; W fp32 [12288, 4096] ~ N(0, 0.02) with
    per-row scale = row absmax / 32768, encoded by the oracle.  One seeded CPU
    generator drives both.  Returns (x bf16, input_scale f32 [1], W fp32,
    W codes u8, W scales f32)."""
    g = torch.Generator().manual_seed(C1_SEED)
    x = torch.randn(1, 4096, generator=g, dtype=torch.float32).to(torch.bfloat16)
    w = (torch.randn(12288, 4096, generator=g, dtype=torch.float32) * 0.02).numpy()
    ws = (np.abs(w).max(axis=1) / HIF8_MAX).astype(np.float32)
    wq, _ = o.static_quant_rows(w, ws)
    return x, input_scale_of(x), w, wq, ws
