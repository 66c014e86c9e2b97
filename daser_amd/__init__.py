"""MI355X (gfx950) KV data-movement path for DaseR.

Paged-KV gather (offload), scatter (load) and fused RoPE re-rotation of
reused chunks, as hand-written HIP kernels behind the C ABI of
include/daser_kv.h, with the DaseR connector's worker hooks on top.
"""

__version__ = "0.1.0"
