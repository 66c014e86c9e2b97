"""numpy front end of the C oracle (kv_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the daser_amd package.

Arrays are host numpy arrays. A layer cache is a C-contiguous array of shape
(2, num_blocks, block_size, num_heads, head_dim) holding raw element bits
(uint16 for bf16/fp16, uint8 for e4m3 / e5m2); staging is a uint8 array.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from typing import Optional, Sequence

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libkv_oracle.so")

BF16, FP16, E4M3, E5M2 = 0, 1, 2, 3
NEOX, GPTJ = 0, 1

_lib: Optional[ctypes.CDLL] = None


def build() -> str:
    """Compiles libkv_oracle.so with the Makefile beside this file."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        h = ctypes.CDLL(LIB_PATH)
        P, I, I64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64
        copy = [P, I, I64, I64, I64, P, P, I, P, I64, I]
        h.orc_gather.argtypes = copy
        h.orc_scatter.argtypes = copy
        h.orc_scatter_rerotate.argtypes = copy + [
            I, I, I, I, I, P, P, P, P, ctypes.c_double, P,
        ]
        slots = [P, I, I64, I64, I64, I, I64, P, P, I, P, I64, I]
        h.orc_gather_slots.argtypes = slots
        h.orc_scatter_slots.argtypes = slots
        h.orc_scatter_slots_rerotate.argtypes = slots + [
            I, I, I, I, I, P, P, P, P, ctypes.c_double, P,
        ]
        h.orc_decode_array.argtypes = [I, P, P, I64]
        h.orc_encode_array.argtypes = [I, P, P, I64]
        for f in ("orc_gather", "orc_scatter", "orc_scatter_rerotate", "orc_gather_slots",
                  "orc_scatter_slots", "orc_scatter_slots_rerotate",
                  "orc_decode_array", "orc_encode_array"):
            getattr(h, f).restype = None
        _lib = h
    return _lib


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def _layer_table(layers: Sequence[np.ndarray]):
    l0 = layers[0]
    for a in layers:
        if not a.flags["C_CONTIGUOUS"] or a.shape != l0.shape or a.dtype != l0.dtype:
            raise ValueError("layers must be C-contiguous arrays of one shape/dtype")
    tab = np.array([_ptr(a) for a in layers], dtype=np.uint64)
    page_bytes = int(np.prod(l0.shape[2:])) * l0.itemsize
    return tab, l0.strides[0], l0.strides[1], page_bytes


def _tables(page_ids, slot_offsets):
    ids = np.ascontiguousarray(page_ids, dtype=np.int32)
    offs = np.ascontiguousarray(slot_offsets, dtype=np.int64)
    assert ids.shape == offs.shape
    return ids, offs


def gather(layers, page_ids, slot_offsets, staging: np.ndarray, layer_bytes: int,
           layer0: int = 0) -> None:
    tab, kvs, ps, pb = _layer_table(layers)
    ids, offs = _tables(page_ids, slot_offsets)
    assert staging.dtype == np.uint8 and staging.flags["C_CONTIGUOUS"]
    lib().orc_gather(_ptr(tab), len(layers), kvs, ps, pb, _ptr(ids), _ptr(offs),
                     ids.size, _ptr(staging), layer_bytes, layer0)


def scatter(layers, page_ids, slot_offsets, staging: np.ndarray, layer_bytes: int,
            layer0: int = 0) -> None:
    tab, kvs, ps, pb = _layer_table(layers)
    ids, offs = _tables(page_ids, slot_offsets)
    lib().orc_scatter(_ptr(tab), len(layers), kvs, ps, pb, _ptr(ids), _ptr(offs),
                      ids.size, _ptr(np.ascontiguousarray(staging)), layer_bytes, layer0)


def scatter_rerotate(layers, page_ids, slot_offsets, staging: np.ndarray,
                     layer_bytes: int, *, dtype: int, rot_dim: int, style: int,
                     stored_pos, new_pos, rotate, theta: float,
                     inv_freq: Optional[np.ndarray] = None,
                     k_scale: Optional[np.ndarray] = None, layer0: int = 0) -> None:
    tab, kvs, ps, pb = _layer_table(layers)
    ids, offs = _tables(page_ids, slot_offsets)
    _, _, bs, h, d = layers[0].shape
    sp = np.ascontiguousarray(stored_pos, dtype=np.int64)
    npos = np.ascontiguousarray(new_pos, dtype=np.int64)
    rot = np.ascontiguousarray(rotate, dtype=np.int8)
    ks = None if k_scale is None else np.ascontiguousarray(k_scale, dtype=np.float32)
    inv = None if inv_freq is None else np.ascontiguousarray(inv_freq, dtype=np.float64)
    stg = np.ascontiguousarray(staging)
    lib().orc_scatter_rerotate(
        _ptr(tab), len(layers), kvs, ps, pb, _ptr(ids), _ptr(offs), ids.size,
        _ptr(stg), layer_bytes, layer0, h, d, rot_dim, style, dtype,
        None if ks is None else _ptr(ks), _ptr(sp), _ptr(npos), _ptr(rot),
        float(theta), None if inv is None else _ptr(inv))


def kx_to_nhd(pages: np.ndarray, block_size: int, num_heads: int, head_dim: int) -> np.ndarray:
    """K pages of the split-x layout (vLLM's PagedAttention kernels: element
    (t, h, d) at ((h * (D / X) + d / X) * block_size + t) * X + d % X, with
    X = 16 / element bytes) as token-major pages [block_size][H][D]. The
    last axis of ``pages`` is one page of element bits; the result has the
    leading axes plus (block_size, H, D). The layout is vLLM's (external and
    absent here); this function states it and a brute-force index test pins
    it."""
    x = 16 // pages.itemsize
    lead = pages.shape[:-1]
    v = pages.reshape(*lead, num_heads, head_dim // x, block_size, x)
    n = len(lead)
    perm = tuple(range(n)) + (n + 2, n, n + 1, n + 3)  # -> (t, h, d / X, d % X)
    return np.ascontiguousarray(v.transpose(perm)).reshape(*lead, block_size, num_heads,
                                                          head_dim)


def nhd_to_kx(pages: np.ndarray) -> np.ndarray:
    """Inverse of kx_to_nhd: (..., block_size, H, D) -> (..., page elements)."""
    *lead, bs, h, d = pages.shape
    x = 16 // pages.itemsize
    v = pages.reshape(*lead, bs, h, d // x, x)
    n = len(lead)
    perm = tuple(range(n)) + (n + 1, n + 2, n, n + 3)  # -> (h, d / X, t, d % X)
    return np.ascontiguousarray(v.transpose(perm)).reshape(*lead, bs * h * d)


def _slots_call(fn, layers, slot_mapping, row_offsets, staging, layer_bytes, layer0):
    tab, kvs, ps, pb = _layer_table(layers)
    _, _, bs, h, d = layers[0].shape
    row = h * d * layers[0].itemsize
    sm = np.ascontiguousarray(slot_mapping, dtype=np.int64)
    ro = np.ascontiguousarray(row_offsets, dtype=np.int64)
    assert sm.shape == ro.shape
    fn(_ptr(tab), len(layers), kvs, ps, pb, bs, row, _ptr(sm), _ptr(ro), sm.size,
       _ptr(staging), layer_bytes, layer0)


def gather_slots(layers, slot_mapping, row_offsets, staging: np.ndarray, layer_bytes: int,
                 layer0: int = 0) -> None:
    assert staging.dtype == np.uint8 and staging.flags["C_CONTIGUOUS"]
    _slots_call(lib().orc_gather_slots, layers, slot_mapping, row_offsets, staging,
                layer_bytes, layer0)


def scatter_slots(layers, slot_mapping, row_offsets, staging: np.ndarray, layer_bytes: int,
                  layer0: int = 0) -> None:
    _slots_call(lib().orc_scatter_slots, layers, slot_mapping, row_offsets,
                np.ascontiguousarray(staging), layer_bytes, layer0)


def scatter_slots_rerotate(layers, slot_mapping, row_offsets, staging: np.ndarray,
                           layer_bytes: int, *, dtype: int, rot_dim: int, style: int,
                           stored_pos, new_pos, rotate, theta: float,
                           inv_freq: Optional[np.ndarray] = None,
                           k_scale: Optional[np.ndarray] = None, layer0: int = 0) -> None:
    """Token form of :func:`scatter_rerotate`: per-token positions."""
    tab, kvs, ps, pb = _layer_table(layers)
    _, _, bs, h, d = layers[0].shape
    row_bytes = h * d * layers[0].itemsize
    sm = np.ascontiguousarray(slot_mapping, dtype=np.int64)
    ro = np.ascontiguousarray(row_offsets, dtype=np.int64)
    sp = np.ascontiguousarray(stored_pos, dtype=np.int64)
    npos = np.ascontiguousarray(new_pos, dtype=np.int64)
    rot = np.ascontiguousarray(rotate, dtype=np.int8)
    ks = None if k_scale is None else np.ascontiguousarray(k_scale, dtype=np.float32)
    inv = None if inv_freq is None else np.ascontiguousarray(inv_freq, dtype=np.float64)
    stg = np.ascontiguousarray(staging)
    lib().orc_scatter_slots_rerotate(
        _ptr(tab), len(layers), kvs, ps, pb, bs, row_bytes, _ptr(sm), _ptr(ro), sm.size,
        _ptr(stg), layer_bytes, layer0, h, d, rot_dim, style, dtype,
        None if ks is None else _ptr(ks), _ptr(sp), _ptr(npos), _ptr(rot), float(theta),
        None if inv is None else _ptr(inv))


def decode(dtype: int, bits) -> np.ndarray:
    b = np.ascontiguousarray(bits, dtype=np.uint32)
    out = np.empty(b.shape, dtype=np.float64)
    lib().orc_decode_array(dtype, _ptr(b), _ptr(out), b.size)
    return out


def encode(dtype: int, values) -> np.ndarray:
    v = np.ascontiguousarray(values, dtype=np.float64)
    out = np.empty(v.shape, dtype=np.uint32)
    lib().orc_encode_array(dtype, _ptr(v), _ptr(out), v.size)
    return out


def ulp_steps(a: np.ndarray, b: np.ndarray, dtype: int) -> np.ndarray:
    """Representable steps between two sign-magnitude bit patterns."""
    sign = 1 << (7 if dtype in (E4M3, E5M2) else 15)

    def ordered(x):
        x = np.asarray(x).astype(np.int64)
        mag = x & (sign - 1)
        return np.where(x & sign, -mag, mag)

    return np.abs(ordered(a) - ordered(b))


def rotation_within_tolerance(got: np.ndarray, ref: np.ndarray, dtype: int,
                              rel_row: float = 2.0 ** -18) -> tuple[bool, str]:
    """Checks kernel re-rotated K bits against the oracle's correctly rounded
    float64 result: every element within 1 ulp, except where the result
    cancels to far below its inputs' magnitude. There the float32 angle table
    alone (cos/sin rounded to 2^-24) moves the output by ~2^-24 |x|, more than
    one ulp of a near-zero value; such elements must be within
    rel_row x (largest |value| of their row). got/ref: (..., head_dim) bits."""
    d = ulp_steps(got, ref, dtype)
    bad = d > 1
    if not bad.any():
        return True, f"max ulp {int(d.max()) if d.size else 0}"
    g = decode(dtype, got)
    r = decode(dtype, ref)
    rowmax = np.nanmax(np.abs(r), axis=-1, keepdims=True)
    err = np.abs(g - r)
    allowed = rel_row * np.broadcast_to(rowmax, r.shape)
    ok = bool(np.all(err[bad] <= allowed[bad]))
    return ok, (f"{int(bad.sum())} elements > 1 ulp (max {int(d.max())}); "
                f"max abs err there {err[bad].max():.3g}, allowed {allowed[bad].min():.3g}")
