"""Shared helpers for the parity tests: seeded caches, bit views, ulp math."""

from __future__ import annotations

import numpy as np
import torch

from daser_amd.workloads import KVShape
from oracle import oracle

TORCH_DT = {"bf16": torch.bfloat16, "fp16": torch.float16, "e4m3": torch.float8_e4m3fn,
            "e5m2": torch.float8_e5m2}
BITS_NP = {"bf16": np.uint16, "fp16": np.uint16, "e4m3": np.uint8, "e5m2": np.uint8}
BITS_T = {"bf16": torch.int16, "fp16": torch.int16, "e4m3": torch.uint8, "e5m2": torch.uint8}
ORC_DT = {"bf16": 0, "fp16": 1, "e4m3": 2, "e5m2": 3}


def rand_caches(shape: KVShape, num_blocks: int, dt: str, device, seed: int,
                scale: float = 1.0) -> list[torch.Tensor]:
    """One (2, NB, bs, H, D) cache per layer, ~N(0, scale^2), seeded."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    out = []
    for _ in range(shape.num_layers):
        x = torch.randn((2, num_blocks, shape.block_size, shape.num_heads, shape.head_dim),
                        generator=g, dtype=torch.float32) * scale
        out.append(x.to(TORCH_DT[dt]).to(device))
    return out


def to_bits_np(t: torch.Tensor, dt: str) -> np.ndarray:
    return t.detach().cpu().view(BITS_T[dt]).numpy().view(BITS_NP[dt]).copy()


def ordered(bits: np.ndarray, dt: str) -> np.ndarray:
    """Maps sign-magnitude float bits to integers ordered like the values,
    so that |ordered(a) - ordered(b)| counts representable steps (ulps)."""
    b = bits.astype(np.int64)
    sign = 1 << (7 if dt in ("e4m3", "e5m2") else 15)
    mag = b & (sign - 1)
    return np.where(b & sign, -mag, mag)


def ulp_diff(a: np.ndarray, b: np.ndarray, dt: str) -> np.ndarray:
    return np.abs(ordered(a, dt) - ordered(b, dt))


def rotation_within_tolerance(got, ref, dt: str, rel_row: float = 2.0 ** -18):
    return oracle.rotation_within_tolerance(got, ref, ORC_DT[dt], rel_row)
