"""Builds libdaser_kv.so (gfx950) in-tree with hipcc.

Run as ``python -m daser_amd._build`` or through ``__graft_entry__.build()``.
The library is written next to this file so that it travels with the source
tree; ``daser_amd._lib`` loads it from there.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SRCS = [os.path.join(HERE, "csrc", "kv_move.hip"), os.path.join(HERE, "csrc", "store_ring.cpp")]
INCLUDE = os.path.join(ROOT, "include")
OUT = os.path.join(HERE, "libdaser_kv.so")
ABI_TEST_SRC = os.path.join(ROOT, "tests", "c", "abi_roundtrip.cpp")
ABI_TEST_OUT = os.path.join(ROOT, "tests", "c", "abi_roundtrip")
RING_SAN_SRC = os.path.join(ROOT, "tests", "c", "ring_sanitize.cpp")
RING_SAN_OUT = os.path.join(ROOT, "tests", "c", "ring_sanitize")
PROBE_SRC = os.path.join(HERE, "csrc", "bw_probe.hip")
PROBE_OUT = os.path.join(HERE, "libdaser_bwprobe.so")

ARCH = "gfx950"

# -packed-fp32-ops keeps v_pk_{add,mul,fma}_f32 out of the generated code.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-shared",
    "-fPIC",
    "-Wall",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found; the HIP library cannot be built")


def build(verbose: bool = False) -> str:
    """Compiles the kernels and C ABI into ``daser_amd/libdaser_kv.so``."""
    tmp = OUT + ".tmp"
    cmd = [hipcc(), *HIPCC_FLAGS, f"-I{INCLUDE}", *SRCS, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{proc.stderr}")
    os.replace(tmp, OUT)
    # a C++ caller of the C ABI (no Python, no torch), run by the GPU tests
    cmd = [hipcc(), "-O2", "-std=c++17", f"-I{INCLUDE}", ABI_TEST_SRC, "-o", ABI_TEST_OUT + ".tmp",
           f"-L{HERE}", "-ldaser_kv", "-Wl,-rpath,$ORIGIN/../../daser_amd"]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{proc.stderr}")
    os.replace(ABI_TEST_OUT + ".tmp", ABI_TEST_OUT)
    # the HBM ceiling probes of bench.py --ceilings (not part of the KV path)
    cmd = [hipcc(), *HIPCC_FLAGS, PROBE_SRC, "-o", PROBE_OUT + ".tmp"]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{proc.stderr}")
    os.replace(PROBE_OUT + ".tmp", PROBE_OUT)
    build_ring_sanitize(verbose)
    return OUT


def build_ring_sanitize(verbose: bool = False) -> None:
    """Best effort: the staging ring's host-mode driver under ASan and UBSan
    (ROCm's clang, host code only), run by a CPU test. Skipped with a note
    where the sanitizer runtimes are missing."""
    clang = "/opt/rocm/llvm/bin/clang++"
    if not os.path.exists(clang):
        return
    cmd = [clang, "-O1", "-g", "-fsanitize=address,undefined", "-fno-omit-frame-pointer",
           "-std=c++17", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include", f"-I{INCLUDE}",
           SRCS[1], RING_SAN_SRC, "-L/opt/rocm/lib", "-lamdhip64", "-Wl,-rpath,/opt/rocm/lib",
           "-o", RING_SAN_OUT + ".tmp"]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        print(f"note: ring sanitizer driver not built ({proc.stderr.strip()[:200]})", flush=True)
        return
    os.replace(RING_SAN_OUT + ".tmp", RING_SAN_OUT)


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
