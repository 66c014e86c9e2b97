"""Writes the golden vectors in this directory (run from the repo root:
``python -m tests.golden.gen_golden``).

The vectors come from the C oracle, which tests/test_oracle.py pins against
a brute-force restatement of the reference loops, torch's dtype conversions
and closed forms of rotation. They freeze seeded inputs and expected outputs
so that later changes to the oracle or the kernels are checked against the
same bytes. Shapes are small (Qwen2-0.5B heads, few layers) to keep the files
small.
"""

from __future__ import annotations

import os

import numpy as np
import torch

from oracle import oracle

HERE = os.path.dirname(os.path.abspath(__file__))


def _bf16_bits(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(x.astype(np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def _e4m3_bits(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(x.astype(np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def _e5m2_bits(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(x.astype(np.float32)).to(torch.float8_e5m2).view(torch.uint8).numpy()


def gather_scatter_case():
    rng = np.random.default_rng(100)
    L, nb, bs, H, D = 2, 8, 16, 2, 64
    caches = np.stack([_bf16_bits(rng.normal(size=(2, nb, bs, H, D))) for _ in range(L)])
    # two requests: tokens 40 (3 pages) and 20 (2 pages), permuted blocks
    page_ids = rng.permutation(nb)[:5].astype(np.int32)
    layer_bytes = 2 * bs * H * D * 2
    slot = layer_bytes * L
    offs = np.arange(5, dtype=np.int64) * slot
    stg = np.zeros(5 * slot, dtype=np.uint8)
    oracle.gather(list(caches), page_ids, offs, stg, layer_bytes)
    dst = [np.zeros_like(c) for c in caches]
    oracle.scatter(dst, page_ids, offs, stg, layer_bytes)
    np.savez_compressed(os.path.join(HERE, "gather_scatter_bf16.npz"), caches=caches,
                        page_ids=page_ids, slot_offsets=offs, layer_bytes=layer_bytes,
                        staging=stg, scattered=np.stack(dst))


def rerotate_case(name, dt, style, rot_dim):
    rng = np.random.default_rng(200 + dt * 10 + style)
    L, nb, bs, H, D = 2, 6, 16, 2, 64
    fp8 = {oracle.E4M3: _e4m3_bits, oracle.E5M2: _e5m2_bits}.get(dt)
    if dt == oracle.BF16:
        src = np.stack([_bf16_bits(rng.normal(size=(2, nb, bs, H, D))) for _ in range(L)])
        k_scale = np.ones(L, np.float32)
    else:
        src = np.stack([fp8(rng.normal(size=(2, nb, bs, H, D)) * 50) for _ in range(L)])
        k_scale = np.float32([0.125, 2.5])
    esz = src.dtype.itemsize
    layer_bytes = 2 * bs * H * D * esz
    slot = layer_bytes * L
    rec_ids = np.arange(4, dtype=np.int32)
    offs = np.arange(4, dtype=np.int64) * slot
    stg = np.zeros(4 * slot, dtype=np.uint8)
    oracle.gather(list(src), rec_ids, offs, stg, layer_bytes)
    dst0 = np.stack([_bf16_bits(rng.normal(size=(2, nb, bs, H, D))) if dt == oracle.BF16
                     else fp8(rng.normal(size=(2, nb, bs, H, D))) for _ in range(L)])
    page_ids = np.array([5, 0, 3, 1], dtype=np.int32)
    deltas = np.array([0, 1, 4097, 32767], dtype=np.int64)
    out = [c.copy() for c in dst0]
    oracle.scatter_rerotate(out, page_ids, offs, stg, layer_bytes, dtype=dt, rot_dim=rot_dim,
                            style=style, stored_pos=np.zeros(4, np.int64), new_pos=deltas,
                            rotate=deltas != 0, theta=500000.0, k_scale=k_scale)
    np.savez_compressed(os.path.join(HERE, name), staging=stg, dst_before=dst0,
                        page_ids=page_ids, slot_offsets=offs, layer_bytes=layer_bytes,
                        deltas=deltas, k_scale=k_scale, rot_dim=rot_dim, style=style,
                        dtype=dt, theta=500000.0, expected=np.stack(out))


if __name__ == "__main__":
    gather_scatter_case()
    rerotate_case("rerotate_bf16_neox.npz", oracle.BF16, oracle.NEOX, 64)
    rerotate_case("rerotate_bf16_gptj_partial.npz", oracle.BF16, oracle.GPTJ, 32)
    rerotate_case("rerotate_e4m3_neox.npz", oracle.E4M3, oracle.NEOX, 64)
    rerotate_case("rerotate_e5m2_gptj.npz", oracle.E5M2, oracle.GPTJ, 64)
    print("golden vectors written to", HERE)
