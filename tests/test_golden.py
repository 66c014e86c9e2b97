"""Golden vectors (tests/golden/*.npz, written by tests/golden/gen_golden.py):
the oracle reproduces them on the CPU; the HIP kernels reproduce them on the
GPU (bit-exact copies, re-rotated K within the rotation tolerance)."""

from __future__ import annotations

import glob
import os

import numpy as np
import pytest
import torch

from oracle import oracle

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
ROT_CASES = sorted(os.path.basename(p) for p in glob.glob(os.path.join(HERE, "rerotate_*.npz")))


def load(name):
    with np.load(os.path.join(HERE, name), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def test_oracle_reproduces_gather_scatter_vectors():
    g = load("gather_scatter_bf16.npz")
    stg = np.zeros_like(g["staging"])
    oracle.gather(list(g["caches"]), g["page_ids"], g["slot_offsets"], stg, int(g["layer_bytes"]))
    assert np.array_equal(stg, g["staging"])
    dst = [np.zeros_like(c) for c in g["caches"]]
    oracle.scatter(dst, g["page_ids"], g["slot_offsets"], stg, int(g["layer_bytes"]))
    assert np.array_equal(np.stack(dst), g["scattered"])


@pytest.mark.parametrize("name", ROT_CASES)
def test_oracle_reproduces_rerotate_vectors(name):
    g = load(name)
    out = [c.copy() for c in g["dst_before"]]
    n = g["page_ids"].size
    oracle.scatter_rerotate(out, g["page_ids"], g["slot_offsets"], g["staging"],
                            int(g["layer_bytes"]), dtype=int(g["dtype"]),
                            rot_dim=int(g["rot_dim"]), style=int(g["style"]),
                            stored_pos=np.zeros(n, np.int64), new_pos=g["deltas"],
                            rotate=g["deltas"] != 0, theta=float(g["theta"]),
                            k_scale=g["k_scale"])
    assert np.array_equal(np.stack(out), g["expected"])


_TDT = {oracle.BF16: torch.bfloat16, oracle.E4M3: torch.float8_e4m3fn,
        oracle.E5M2: torch.float8_e5m2}
_FP8 = (oracle.E4M3, oracle.E5M2)


def _to_device(bits: np.ndarray, tdt, dev):
    t = torch.from_numpy(bits.view(np.int16) if bits.dtype == np.uint16 else bits)
    return t.to(dev).view(tdt)


@pytest.mark.gpu
def test_kernels_reproduce_gather_scatter_vectors(gpu):
    from daser_amd import ops

    print("case: golden gather/scatter", flush=True)
    g = load("gather_scatter_bf16.npz")
    caches = [_to_device(c, torch.bfloat16, gpu) for c in g["caches"]]
    stg = torch.zeros(g["staging"].size, dtype=torch.uint8, device=gpu)
    ops.gather(ops.LayerTable(caches), g["page_ids"], g["slot_offsets"], stg)
    dst = [torch.zeros_like(c) for c in caches]
    ops.scatter(ops.LayerTable(dst), g["page_ids"], g["slot_offsets"], stg)
    torch.cuda.synchronize()
    assert np.array_equal(stg.cpu().numpy(), g["staging"])
    got = np.stack([d.view(torch.int16).cpu().numpy().view(np.uint16) for d in dst])
    assert np.array_equal(got, g["scattered"])


@pytest.mark.gpu
@pytest.mark.parametrize("name", ROT_CASES)
def test_kernel_reproduces_rerotate_vectors(gpu, name):
    from daser_amd import ops, position

    print(f"case: golden {name}", flush=True)
    g = load(name)
    dt = int(g["dtype"])
    tdt = _TDT[dt]
    dst = [_to_device(c.copy(), tdt, gpu) for c in g["dst_before"]]
    stg = torch.from_numpy(g["staging"]).to(gpu)
    ridx, uniq = position.page_rope_index([1] * g["page_ids"].size, g["deltas"])
    tabs = position.delta_tables(uniq, int(g["rot_dim"]), float(g["theta"]), device=gpu)
    ks = torch.from_numpy(g["k_scale"]).to(gpu) if dt in _FP8 else None
    ops.scatter_rerotate(ops.LayerTable(dst), g["page_ids"], g["slot_offsets"], stg, tabs, ridx,
                         rot_dim=int(g["rot_dim"]),
                         style="neox" if int(g["style"]) == oracle.NEOX else "gptj", k_scale=ks)
    torch.cuda.synchronize()
    for l, d in enumerate(dst):
        bits = d.view(torch.uint8 if dt in _FP8 else torch.int16).cpu().numpy()
        bits = bits if dt in _FP8 else bits.view(np.uint16)
        exp = g["expected"][l]
        assert np.array_equal(bits[1], exp[1])
        ok, msg = oracle.rotation_within_tolerance(bits[0], exp[0], dt)
        assert ok, f"layer {l}: {msg}"
