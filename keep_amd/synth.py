"""Seeded synthetic inputs for the benchmark configurations (no data files).

Codes are uniform uint16 over [0, 65536); scales fp16 ``exp(N(0, 0.3))`` one
per output row (``group_size = K``); activations fp16 ``FWHT(N(0,1) * s)``
with seeded random signs s; router logits N(0,1) fp32. Large tensors are drawn
on the GPU with a seeded ``torch.Generator``; small ones (and everything a
CPU test compares) with ``numpy.random.default_rng``.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from keep_amd.rht import apply_rht


@dataclass
class Projection:
    codes: torch.Tensor  # int16 view of uint16 codes [E, N, K/8]
    scales: torch.Tensor  # fp16 [E, N, K/group]

    @property
    def code_bytes(self) -> int:
        return self.codes.numel() * 2


def projection(E: int, N: int, K: int, *, group_size: int | None = None, seed: int = 0, device="cuda",
               scale_dtype=torch.float16) -> Projection:
    """Uniform-random E8P codes and log-normal(0, 0.3) scales, drawn on ``device``."""

    gs = K if group_size is None else group_size
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    codes = torch.randint(-32768, 32768, (E, N, K // 8), dtype=torch.int16, device=device, generator=g)
    scales = torch.exp(torch.randn((E, N, K // gs), device=device, generator=g, dtype=torch.float32) * 0.3)
    return Projection(codes, scales.to(scale_dtype))


def projection_np(E: int, N: int, K: int, *, group_size: int | None = None, seed: int = 0):
    """Host (numpy) variant for CPU-checked sizes: ``(codes uint16, scales float16)``."""

    gs = K if group_size is None else group_size
    rng = np.random.default_rng(seed)
    codes = rng.integers(0, 1 << 16, size=(E, N, K // 8), dtype=np.uint16)
    scales = np.exp(rng.normal(0.0, 0.3, size=(E, N, K // gs))).astype(np.float16)
    return codes, scales


def rht_activations(T: int, K: int, *, seed: int = 0, device="cuda", dtype=torch.float16) -> torch.Tensor:
    """N(0,1) activations pre-multiplied by a seeded random-sign Walsh-Hadamard transform."""

    rng = np.random.default_rng(seed)
    x = torch.from_numpy(rng.standard_normal((T, K)).astype(np.float32)).to(device)
    signs = torch.from_numpy(np.where(rng.integers(0, 2, size=K) == 0, -1.0, 1.0).astype(np.float32)).to(device)
    return apply_rht(x, signs).to(dtype)


def router_logits(T: int, E: int, *, seed: int = 0, device="cuda") -> torch.Tensor:
    rng = np.random.default_rng(seed)
    return torch.from_numpy(rng.standard_normal((T, E)).astype(np.float32)).to(device)


def zipf_routes(T: int, E: int, k: int, *, s: float = 1.1, seed: int = 0) -> np.ndarray:
    """Top-k experts per token without replacement by Gumbel-top-k on
    ``log p_e + N(0,1)`` with Zipf(s) popularity under a seeded permutation."""

    rng = np.random.default_rng(seed)
    perm = rng.permutation(E)
    logp = -s * np.log(np.arange(1, E + 1, dtype=np.float64))[np.argsort(perm)]
    keys = logp[None, :] + rng.standard_normal((T, E)) + rng.gumbel(size=(T, E))
    return np.argsort(-keys, axis=1)[:, :k].astype(np.int32)


def resident_mask(E: int, *, frac: float = 0.5, seed: int = 0) -> np.ndarray:
    rng = np.random.default_rng(seed)
    m = np.zeros(E, dtype=bool)
    m[rng.permutation(E)[: int(round(E * frac))]] = True
    return m
