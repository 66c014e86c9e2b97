"""ctypes binding of libdaser_kv.so (declarations in include/daser_kv.h).

torch is imported first on purpose: torch ships its own libamdhip64.so.7 and
the dynamic loader then resolves the library's HIP dependency to that same
runtime, so streams and device pointers handed over from torch are valid in
the library.

There is no fallback: if the library has not been built, ``lib()`` raises.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (must precede loading the HIP library)

LIB_PATH = os.environ.get("DASER_KV_LIB") or os.path.join(
    os.path.dirname(os.path.abspath(__file__)), "libdaser_kv.so"
)

DSR_ABI_VERSION = 11
DSR_OK = 0
DSR_ERR_ARG = -1
DSR_ERR_ALIGN = -2
DSR_ERR_SHAPE = -3
DSR_ERR_IO = -4
DSR_ERR_NOFILE = -5
DSR_ERR_TOO_LARGE = -6
DSR_STATIC_TABLE_BYTES = 4 << 20

DSR_RING_HOST = 1
DSR_RING_DIRECT = 2
DSR_RING_NO_URING = 4
DSR_RING_MMAP = 8

DSR_DTYPE_BF16 = 0
DSR_DTYPE_FP16 = 1
DSR_DTYPE_FP8_E4M3 = 2
DSR_DTYPE_FP8_E5M2 = 3

DSR_ROPE_NEOX = 0
DSR_ROPE_GPTJ = 1

DSR_SHARED_RECORDS = 1
DSR_K_NHD, DSR_K_KX, DSR_K_HND = 0, 1, 2
DSR_REROTATE_SHARED_RECORDS = DSR_SHARED_RECORDS

# dsr_set_tuning knobs (measurements and tests only)
TUNE = {"units_per_group": 0, "max_wg_per_launch": 1, "rot_kernel": 2, "rot_wg_per_cu": 3,
        "rot_grouped_wg_per_cu": 4, "slots_tpw": 5, "slots_kernel": 6, "slots_unroll": 7,
        "copy_wg_per_cu": 8, "scatter_kernel": 9, "gather_split": 10,
        "page_parts": 11, "slots_order": 12, "slots_wg_per_cu": 13,
        "fanout_wg_per_cu": 14, "fanout_parts": 15}
ROT_KERNEL_CODES = {"auto": 0, "pairs": 1, "contig": 2, "grouped": 3}

_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64

# Argument lists, one per exported entry point, in header order.
_COPY_ARGS = [_P, _I, _I64, _I64, _I64, _I64, _P, _P, _I, _P, _I64, _I64, _I, _P]
_SLOT_ARGS = [_P, _I, _I64, _I64, _I64, _I64, _I, _I64, _P, _P, _I, _P, _I64, _I64, _I, _P]
SIGNATURES = {
    "dsr_abi_version": ([], _I),
    "dsr_error_string": ([_I], ctypes.c_char_p),
    "dsr_set_tuning": ([_I, _I64], _I),
    "dsr_gather": (_COPY_ARGS, _I),
    "dsr_scatter": (_COPY_ARGS, _I),
    "dsr_scatter_ex": (_COPY_ARGS[:-1] + [ctypes.c_uint, _P], _I),
    "dsr_gather_slots": (_SLOT_ARGS, _I),
    "dsr_scatter_slots": (_SLOT_ARGS, _I),
    "dsr_scatter_slots_rerotate": (
        _SLOT_ARGS[:-1] + [_P, _P, _I, _P, _I, _I, _I, _I, _I, _P, _P], _I),
    "dsr_ring_open": ([ctypes.c_char_p, _I64, _I, _I, ctypes.POINTER(_P)], _I),
    "dsr_ring_write": ([_P, _P, _I64, _I64, _P], _I),
    "dsr_ring_read": ([_P, _P, _I64, _I64, _P], _I),
    "dsr_ring_uses_io_uring": ([_P], _I),
    "dsr_ring_is_mapped": ([_P], _I),
    "dsr_ring_last_errno": ([_P], _I),
    "dsr_ring_close": ([_P], _I),
    "dsr_scatter_rerotate": (
        _COPY_ARGS[:-1] + [_P, _P, _I, _P, _I, _I, _I, _I, _I, _P, ctypes.c_uint, _P],
        _I,
    ),
    "dsr_scatter_fanout": (
        [_P, _I, _I64, _I64, _I64, _I64, _P, _I, _P, _P, _P, _I, _P, _I64, _I64, _I,
         _P, _I, _P, _I, _I, _I, _I, _I, _P, _I, _I, _I, _P], _I),
    "dsr_scatter_rerotate_static": (
        _COPY_ARGS[:-1] + [_P, _P, _I, _P, _I, _I, _I, _I, _I, _P, ctypes.c_uint, _P],
        _I,
    ),
    "dsr_scatter_rerotate_kx": (
        _COPY_ARGS[:-1] + [_P, _P, _I, _P, _I, _I, _I, _I, _I, _P, _I, ctypes.c_uint, _P],
        _I,
    ),
    "dsr_gather_hnd": (_COPY_ARGS[:-1] + [_I, _I, _P], _I),
    "dsr_scatter_hnd": (_COPY_ARGS[:-1] + [_I, _I, _P], _I),
    "dsr_scatter_rerotate_hnd": (
        _COPY_ARGS[:-1] + [_P, _P, _I, _P, _I, _I, _I, _I, _I, _P, _I, ctypes.c_uint, _P],
        _I,
    ),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class DaserKVError(RuntimeError):
    """A non-zero return code from libdaser_kv."""

    def __init__(self, fn: str, code: int, text: str) -> None:
        super().__init__(f"{fn} failed with code {code}: {text}")
        self.code = code


def lib() -> ctypes.CDLL:
    """Loads (once) and returns the HIP library; raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"{LIB_PATH} is missing: build it with "
                    "`python -m daser_amd._build` (there is no CPU fallback)"
                )
            handle = ctypes.CDLL(LIB_PATH)
            for name, (args, res) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.argtypes = args
                fn.restype = res
            ver = handle.dsr_abi_version()
            if ver != DSR_ABI_VERSION:
                raise RuntimeError(f"libdaser_kv ABI {ver} != expected {DSR_ABI_VERSION}")
            _lib = handle
    return _lib


def check(fn: str, code: int) -> None:
    if code != DSR_OK:
        text = lib().dsr_error_string(code).decode()
        raise DaserKVError(fn, code, text)


def set_tuning(knob: str, value) -> None:
    """Launch-shape override for measurements and tests (``TUNE`` names;
    ``rot_kernel`` also takes "auto" / "pairs" / "contig" / "grouped",
    ``slots_kernel`` "small"); 0 or "auto" restores the default."""
    if knob == "rot_kernel" and isinstance(value, str):
        value = ROT_KERNEL_CODES[value]
    elif knob == "slots_kernel" and isinstance(value, str):
        value = 1 if value == "small" else 0
    check("dsr_set_tuning", lib().dsr_set_tuning(TUNE[knob], int(value)))
