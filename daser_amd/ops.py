"""Host-side wrappers of the HIP gather / scatter / re-rotate kernels.

The functions take torch tensors (device memory and streams only) and call
the C ABI of libdaser_kv.so on torch's current stream. Index tables given as
host data (lists, numpy arrays, CPU tensors) are validated on the host and
uploaded; tables given as device tensors are used as they are (the kernels
then skip out-of-range entries instead of faulting).

Reference semantics restated here:
  * LAYER_SIZE = kv.nbytes // kv.shape[1], SLOT_SIZE = LAYER_SIZE * L
    (daser/connector/daser_connector.py:404-408);
  * record of (slot i, layer l) at i * SLOT_SIZE + l * LAYER_SIZE, holding
    bytes(kv_l[:, block_id]) = K page then V page (:625-632, :536-551).
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional, Sequence

import numpy as np
import torch

from daser_amd import _lib

_DTYPE_CODES = {
    torch.bfloat16: _lib.DSR_DTYPE_BF16,
    torch.float16: _lib.DSR_DTYPE_FP16,
    torch.float8_e4m3fn: _lib.DSR_DTYPE_FP8_E4M3,
    torch.float8_e5m2: _lib.DSR_DTYPE_FP8_E5M2,
}
FP8_DTYPES = (torch.float8_e4m3fn, torch.float8_e5m2)

ROPE_STYLES = {"neox": _lib.DSR_ROPE_NEOX, "gptj": _lib.DSR_ROPE_GPTJ}


@dataclass(frozen=True)
class PagedKVLayout:
    """Geometry of vLLM's per-layer paged caches ``kv_l[2, NB, ...]``.

    Built from the registered caches (reference ``register_kv_caches``,
    daser/connector/daser_connector.py:383-413): layer order is the dict's
    insertion order, every layer must share shape, dtype and strides, and a
    page (``kv_l[0, b]``) must be contiguous. The reference moves
    ``kv_l[:, b]`` of any cache shape as bytes (:545-550, :625-632), and so
    do the page copies here. Re-rotation also needs the element layout of a
    K page (``k_layout``):

    * ``"nhd"``: ``[block_size][H][D]``, the 5-D caches
      ``(2, NB, block_size, H, D)`` of vLLM's FlashAttention-style backends;
    * ``"kx"``: ``[H][D / X][block_size][X]`` with X = 16 / element bytes,
      the 3-D caches ``(2, NB, block_size * H * D)`` of vLLM's
      PagedAttention kernels (its ROCm paged-attention backend);
    * ``"hnd"``: 5-D caches whose pages are stored head-major,
      ``[H][block_size][D]`` (vLLM's HND layout). Their records still hold
      the page in index order ``[block_size][H][D]``, as the reference's
      ``reshape(-1)`` of ``kv[:, b]`` does, so the copies permute rows.

    A cache that is not 5-D carries no head geometry in its shape: pass
    ``block_size`` and ``head_dim`` (``num_heads`` follows from the page
    size); without them copies work and re-rotation is refused.
    """

    num_layers: int
    num_blocks: int
    block_size: int  # 0: unknown (copies only)
    num_heads: int
    head_dim: int
    dtype: torch.dtype
    elem_bytes: int
    page_bytes: int  # one K (or V) page
    kv_stride: int  # bytes K page -> V page
    page_stride: int  # bytes block b -> b + 1
    layer_bytes: int  # LAYER_SIZE of the slot record
    device: torch.device
    k_layout: str = "nhd"

    @property
    def slot_bytes(self) -> int:
        """SLOT_SIZE: one block's record over all layers."""
        return self.layer_bytes * self.num_layers

    @property
    def has_geometry(self) -> bool:
        return self.head_dim > 0 and self.block_size > 0

    @staticmethod
    def from_caches(kv_caches: Sequence[torch.Tensor], *, block_size: Optional[int] = None,
                    head_dim: Optional[int] = None,
                    k_layout: Optional[str] = None) -> "PagedKVLayout":
        if not kv_caches:
            raise ValueError("no KV caches registered")
        t0 = kv_caches[0]
        if t0.dim() < 3 or t0.shape[0] != 2:
            raise ValueError(
                f"expected per-layer KV cache of shape (2, num_blocks, ...) such as "
                f"(2, num_blocks, block_size, num_heads, head_dim), got {tuple(t0.shape)}"
            )
        for t in kv_caches:
            if t.shape != t0.shape or t.dtype != t0.dtype or t.stride() != t0.stride():
                raise ValueError("all layer caches must share shape, dtype and strides")
            if t.device != t0.device:
                raise ValueError("all layer caches must live on one device")
        nb = t0.shape[1]
        s = t0.stride()
        expect, c_order = 1, True
        for dim in range(t0.dim() - 1, 1, -1):  # is a page kv[0, b] C-contiguous?
            if t0.shape[dim] != 1 and s[dim] != expect:
                c_order = False
            expect *= t0.shape[dim]
        page_elems = expect
        e = t0.element_size()
        head_major = False
        if not c_order:
            # vLLM's HND layout: logical (2, NB, bs, H, D), page stored [H][bs][D]
            head_major = (t0.dim() == 5 and s[4] == 1 and s[2] == t0.shape[4] and
                          s[3] == t0.shape[2] * t0.shape[4])
            if not head_major:
                raise ValueError("a KV page kv[0, b] must be contiguous in memory, in "
                                 "(block_size, heads, head_dim) order or head-major")
        if t0.dim() == 5:
            want = "hnd" if head_major else "nhd"
            if k_layout not in (None, want):
                raise ValueError(f"this 5-D cache's pages have the {want!r} layout")
            _, _, bs, h, d = t0.shape
            if (block_size not in (None, bs)) or (head_dim not in (None, d)):
                raise ValueError(f"cache shape {tuple(t0.shape)} disagrees with "
                                 f"block_size={block_size}, head_dim={head_dim}")
            layout = want
        else:
            layout = k_layout or ("kx" if t0.dim() == 3 else "nhd")
            if layout not in ("nhd", "kx"):
                raise ValueError("k_layout must be 'nhd' or 'kx'")
            bs, d, h = int(block_size or 0), int(head_dim or 0), 0
            if bs and d:
                if page_elems % (bs * d):
                    raise ValueError(f"a page of {page_elems} elements is not block_size "
                                     f"{bs} x heads x head_dim {d}")
                h = page_elems // (bs * d)
                if layout == "kx" and (d * e) % 16:
                    raise ValueError("the 'kx' K layout needs head_dim * element size to be "
                                     "a multiple of 16 bytes")
            else:
                bs = d = 0
        page_bytes = page_elems * e
        # LAYER_SIZE as the reference derives it (kv.nbytes // num_blocks).
        layer_bytes = t0.numel() * e // nb if nb else 2 * page_bytes
        return PagedKVLayout(
            num_layers=len(kv_caches),
            num_blocks=nb,
            block_size=bs,
            num_heads=h,
            head_dim=d,
            dtype=t0.dtype,
            elem_bytes=e,
            page_bytes=page_bytes,
            kv_stride=s[0] * e,
            page_stride=s[1] * e,
            layer_bytes=layer_bytes,
            device=t0.device,
            k_layout=layout,
        )


class LayerTable:
    """Device array of per-layer cache base addresses (uint64)."""

    def __init__(self, kv_caches: Sequence[torch.Tensor], **geometry) -> None:
        """``geometry``: ``block_size``, ``head_dim``, ``k_layout`` for caches
        that are not 5-D (see PagedKVLayout)."""
        self.layout = PagedKVLayout.from_caches(kv_caches, **geometry)
        self._caches = list(kv_caches)  # keep the borrowed tensors alive
        ptrs = np.array([t.data_ptr() for t in kv_caches], dtype=np.uint64)
        self.table = torch.from_numpy(ptrs.view(np.int64)).to(self.layout.device)

    def ptr(self, first: int = 0) -> int:
        return self.table.data_ptr() + 8 * first


def _stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _as_device_table(
    x, dtype: torch.dtype, device: torch.device, name: str
) -> torch.Tensor:
    if isinstance(x, torch.Tensor) and x.device.type != "cpu":
        if x.dtype != dtype or not x.is_contiguous():
            raise ValueError(f"{name} must be a contiguous {dtype} tensor")
        return x
    arr = torch.as_tensor(np.asarray(x), dtype=dtype)
    return _upload(arr, device)


def _upload(arr: torch.Tensor, device: torch.device) -> torch.Tensor:
    """Host table -> device, stream-ordered on the current stream without
    blocking the host: copied into pinned memory (torch's caching host
    allocator keeps it until the copy has run), then an asynchronous copy.
    A pageable copy would wait for the stream's earlier work, e.g. the
    store reads that the load's scatter follows."""
    if device.type != "cuda":
        return arr.to(device)
    if torch.cuda.is_current_stream_capturing():
        # a captured copy would replay from a pinned buffer torch reuses
        raise ValueError("host index tables cannot be used under graph capture: pass "
                         "device tensors")
    return arr.pin_memory().to(device, non_blocking=True)


def _host_array(x, np_dtype) -> Optional[np.ndarray]:
    if isinstance(x, torch.Tensor):
        if x.device.type != "cpu":
            return None
        return x.numpy().astype(np_dtype, copy=False)
    return np.asarray(x, dtype=np_dtype)


def _validate(layout: PagedKVLayout, page_ids, slot_offsets, staging, layer0, n_layers,
              records_written: bool):
    ids = _host_array(page_ids, np.int64)
    offs = _host_array(slot_offsets, np.int64)
    if ids is not None and offs is not None and ids.shape != offs.shape:
        raise ValueError("page_ids and slot_offsets differ in length")
    if ids is not None and ids.size and (ids.min() < 0 or ids.max() >= layout.num_blocks):
        raise IndexError(f"block id out of range [0, {layout.num_blocks})")
    if offs is not None and offs.size:
        end = offs.max() + (layer0 + n_layers - 1) * layout.layer_bytes + 2 * layout.page_bytes
        if offs.min() < 0 or end > staging.numel() * staging.element_size():
            raise IndexError("slot record outside the staging buffer")
        if np.any(offs % 16):
            raise ValueError("slot offsets must be multiples of 16 bytes")
        span = (n_layers - 1) * layout.layer_bytes + 2 * layout.page_bytes
        so = np.sort(offs)
        # a gather writes the records: two pages' records must not overlap
        # (a scatter may read one cached record into several pages)
        if records_written and so.size > 1 and np.any(np.diff(so) < span):
            raise ValueError("slot records of two pages overlap")


def check_tables(table: "LayerTable", page_ids, slot_offsets, staging: torch.Tensor, *,
                 layer0: int = 0, records_written: bool = False) -> None:
    """The checks the copy wrappers run on host tables, for device-resident
    ones (which the wrappers trust: the kernels skip a page whose block id or
    record range is out of bounds instead of faulting, where the reference's
    indexing would raise). Copies the tables to the host, so it synchronises
    the stream: for debugging and for callers that build tables on the
    device and want the reference's errors."""
    def host(x, dt):
        return x.detach().cpu().numpy().astype(dt) if isinstance(x, torch.Tensor) \
            else np.asarray(x, dt)

    _validate(table.layout, host(page_ids, np.int64), host(slot_offsets, np.int64), staging,
              layer0, table.layout.num_layers, records_written)


def dest_order(page_ids, slot_offsets, extra=None):
    """Host tables of a scatter, reordered by destination block (stable).

    Processing order does not change the result (each destination block is
    written once) but near-sequential page writes run faster. A destination
    block listed several times keeps only its last entry: the reference's
    sequential copies (daser_connector.py:536-551) leave the last one's
    bytes, while copies inside one launch would race. Device tables are
    returned unchanged (there, duplicates race)."""
    ids = _host_array(page_ids, np.int64)
    offs = _host_array(slot_offsets, np.int64)
    if ids is None or offs is None or ids.size == 0:
        return page_ids, slot_offsets, extra
    order = np.argsort(ids, kind="stable")
    sids = ids[order]
    if sids.size > 1 and np.any(sids[1:] == sids[:-1]):
        # within a run of equal ids the stable order keeps list order: the
        # run's last element is the list's last entry for that block
        last = np.append(sids[1:] != sids[:-1], True)
        order, sids = order[last], sids[last]
    ex = None
    if extra is not None:
        e = _host_array(extra, np.int64)
        ex = extra if e is None else e[order]
    return sids, offs[order], ex


def _copy_args(table: LayerTable, page_ids, slot_offsets, staging, layer0, layers,
               records_written: bool = False):
    lay = table.layout
    first, count = (0, lay.num_layers) if layers is None else layers
    if first < 0 or count < 0 or first + count > lay.num_layers:
        raise IndexError("layer range outside the registered caches")
    if staging.device != lay.device:
        raise ValueError("staging must live on the KV caches' device")
    if not staging.is_contiguous():
        raise ValueError("staging must be contiguous")
    _validate(lay, page_ids, slot_offsets, staging, layer0 + first, count, records_written)
    ids = _as_device_table(page_ids, torch.int32, lay.device, "page_ids")
    offs = _as_device_table(slot_offsets, torch.int64, lay.device, "slot_offsets")
    if ids.numel() != offs.numel():
        raise ValueError("page_ids and slot_offsets differ in length")
    args = (
        table.ptr(first),
        count,
        lay.kv_stride,
        lay.page_stride,
        lay.page_bytes,
        lay.num_blocks,
        ids.data_ptr(),
        offs.data_ptr(),
        ids.numel(),
        staging.data_ptr(),
        staging.numel() * staging.element_size(),
        lay.layer_bytes,
        layer0 + first,
    )
    return args, (ids, offs)


def gather(
    table: LayerTable,
    page_ids,
    slot_offsets,
    staging: torch.Tensor,
    *,
    layer0: int = 0,
    layers: Optional[tuple[int, int]] = None,
) -> None:
    """Packs pages into slot records (reference save loop, :610-632).

    ``layers=(first, count)`` restricts the launch to a layer range; the
    record index of table layer ``first + i`` is ``layer0 + first + i``.
    """
    args, _tables = _copy_args(table, page_ids, slot_offsets, staging, layer0, layers,
                            records_written=True)
    fn, name, extra = _copy_entry(table.layout, "dsr_gather")
    rc = fn(*args, *extra, _stream_handle(table.layout.device))
    _lib.check(name, rc)


def _copy_entry(lay: PagedKVLayout, base: str):
    """The copy entry point for the layout's pages and its extra arguments:
    head-major pages go through the row-permuting ``*_hnd`` variant."""
    if lay.k_layout == "hnd":
        return getattr(_lib.lib(), base + "_hnd"), base + "_hnd", (lay.block_size,
                                                                   lay.num_heads)
    return getattr(_lib.lib(), base), base, ()


class PreparedGather:
    """A gather of fixed page tables into a fixed staging buffer, checked and
    converted once; each call launches it for a layer range. For callers
    that launch the same gather once per layer (the connector's
    save_kv_layer runs 32-80 times a step), so that a call costs one ctypes
    launch and no table checks or conversions."""

    def __init__(self, table: LayerTable, page_ids, slot_offsets, staging: torch.Tensor,
                 *, layer0: int = 0) -> None:
        args, self._keep = _copy_args(table, page_ids, slot_offsets, staging, layer0, None,
                                      records_written=True)
        self.tables = self._keep  # (page_ids, slot_offsets) as device tensors
        self._table = table
        self._staging = staging
        self._mid = args[2:12]  # strides, page geometry, tables, staging
        self._layer0 = layer0
        self._n_layers = table.layout.num_layers
        self._fn, self._name, self._extra = _copy_entry(table.layout, "dsr_gather")

    def __call__(self, first: int, count: int, stream: int) -> None:
        """Gathers table layers [first, first + count) on ``stream`` (a HIP
        stream handle, e.g. ``torch.cuda.current_stream().cuda_stream``)."""
        if first < 0 or count < 0 or first + count > self._n_layers:
            raise IndexError("layer range outside the registered caches")
        rc = self._fn(self._table.ptr(first), count, *self._mid, self._layer0 + first,
                      *self._extra, stream)
        if rc:
            _lib.check(self._name, rc)


def scatter(
    table: LayerTable,
    page_ids,
    slot_offsets,
    staging: torch.Tensor,
    *,
    layer0: int = 0,
    layers: Optional[tuple[int, int]] = None,
    shared_records: Optional[bool] = None,
) -> None:
    """Unpacks slot records into pages (reference load loop, :536-551).

    ``shared_records``: several pages read the same records. Host tables
    then take the fan-out load (:class:`PreparedFanout`: each record read
    once and written to all of its pages) where the pages allow it, device
    tables a launch shaped for cache-served reads. None: inferred from host
    ``slot_offsets`` (at most half of them distinct), False for device
    tables. Results do not depend on it."""
    if shared_records is None:
        shared_records = _shared_offsets(slot_offsets)
    page_ids, slot_offsets, _ = dest_order(page_ids, slot_offsets)
    if shared_records and _scatter_fanout(table, page_ids, slot_offsets, staging, layer0,
                                          layers):
        return
    args, _tables = _copy_args(table, page_ids, slot_offsets, staging, layer0, layers)
    stream = _stream_handle(table.layout.device)
    if shared_records and table.layout.k_layout != "hnd":
        rc = _lib.lib().dsr_scatter_ex(*args, _lib.DSR_SHARED_RECORDS, stream)
        _lib.check("dsr_scatter_ex", rc)
        return
    fn, name, extra = _copy_entry(table.layout, "dsr_scatter")
    rc = fn(*args, *extra, stream)
    _lib.check(name, rc)


def _shared_offsets(slot_offsets) -> bool:
    """At most half of the host record offsets are distinct."""
    offs_h = _host_array(slot_offsets, np.int64)
    return offs_h is not None and offs_h.size > 1 and 2 * np.unique(offs_h).size <= offs_h.size


def fanout_tables(page_ids: np.ndarray, slot_offsets: np.ndarray,
                  rope_idx: Optional[np.ndarray] = None):
    """Host tables of a scatter (destination order, one entry per block)
    grouped by source record: (src_offsets, dst_start, dst_pages, dst_rope),
    where the destinations of source s are entries dst_start[s] to
    dst_start[s + 1] - 1, in block order."""
    ids = np.asarray(page_ids, np.int64)
    offs = np.asarray(slot_offsets, np.int64)
    order = np.argsort(offs, kind="stable")  # keeps block order inside a source
    so = offs[order]
    first = np.ones(so.size, bool)
    first[1:] = so[1:] != so[:-1]
    starts = np.nonzero(first)[0]
    dst_start = np.append(starts, so.size).astype(np.int32)
    dst_rope = None if rope_idx is None else np.asarray(rope_idx, np.int64)[order]
    return so[starts], dst_start, ids[order], dst_rope


_K_LAYOUTS = {"nhd": _lib.DSR_K_NHD, "kx": _lib.DSR_K_KX, "hnd": _lib.DSR_K_HND}


def fanout_supported(lay: PagedKVLayout, rot_dim: Optional[int] = None,
                     style: str = "neox") -> bool:
    """Whether dsr_scatter_fanout takes these pages (``rot_dim`` None: a
    plain copy), asked of the library itself: a call with no work checks
    the geometry and launches nothing. It takes pages of at most 32 KiB in
    every cache layout; the re-rotation wants whole-vector rotary widths
    and neox partners a power of two of at most 32 vectors apart (split-x
    pages: the split-x kernels' conditions)."""
    rot = rot_dim is not None
    if rot and (not lay.has_geometry or lay.dtype not in _DTYPE_CODES):
        return False
    if lay.k_layout != "nhd" and lay.block_size <= 0:
        return False
    rc = _lib.lib().dsr_scatter_fanout(
        16, lay.num_layers, lay.kv_stride, lay.page_stride, lay.page_bytes, lay.num_blocks,
        None, 0, None, None, 16 if rot else None, 0, 16, 0, lay.layer_bytes, 0, None, 0, None, 0,
        lay.head_dim, rot_dim or 0, ROPE_STYLES[style], _DTYPE_CODES.get(lay.dtype, 0), 16,
        _K_LAYOUTS[lay.k_layout], lay.block_size, lay.num_heads, None)
    return rc == _lib.DSR_OK


class PreparedFanout:
    """A load of host tables whose pages share records (a cached chunk
    placed in several requests), through dsr_scatter_fanout: each record is
    read once and written to all of its pages. The tables are checked,
    grouped by record (:func:`fanout_tables`) and uploaded once; each call
    launches the load on the current stream. ``rope``: None for a plain
    copy, else (rope_idx, cos_sin, rot_dim, style, k_scale, layer_group) as
    for :func:`scatter_rerotate`. Pages must satisfy
    :func:`fanout_supported`; a block listed twice keeps its last entry."""

    def __init__(self, table: LayerTable, page_ids, slot_offsets, staging: torch.Tensor, *,
                 rope=None, layer0: int = 0, layers: Optional[tuple[int, int]] = None) -> None:
        lay = table.layout
        ids = _host_array(page_ids, np.int64)
        offs = _host_array(slot_offsets, np.int64)
        if ids is None or offs is None:
            raise ValueError("PreparedFanout takes host tables")
        first, count = (0, lay.num_layers) if layers is None else layers
        if first < 0 or count < 0 or first + count > lay.num_layers:
            raise IndexError("layer range outside the registered caches")
        if staging.device != lay.device or not staging.is_contiguous():
            raise ValueError("staging must be a contiguous tensor on the KV caches' device")
        tail = (None, 0, None, 0, 0, 0, 0, 0, None)
        ridx = None
        keep = []
        if rope is not None:
            rope_idx, cos_sin, rot_dim, style, k_scale, layer_group = rope
            rot_dim, n_tables, n_groups, lg_d, ks_ptr = _rope_args(
                lay, cos_sin, rope_idx, rot_dim, k_scale, layer0, layer_group)
            ridx = _host_array(rope_idx, np.int64)
            if ridx is None:
                raise ValueError("PreparedFanout takes host tables")
            if ridx.shape != ids.shape:
                raise ValueError("rope_idx and page_ids differ in length")
            if not fanout_supported(lay, rot_dim, style):
                raise ValueError("these pages need the per-page re-rotation kernels")
            tail = (cos_sin.data_ptr(), n_tables, None if lg_d is None else lg_d.data_ptr(),
                    n_groups, lay.head_dim, rot_dim, ROPE_STYLES[style],
                    _DTYPE_CODES[lay.dtype], ks_ptr)
            keep += [cos_sin, lg_d, k_scale]
        elif not fanout_supported(lay):
            raise ValueError("these pages need the per-page scatter kernels")
        ids, offs, ridx = dest_order(ids, offs, ridx)
        _validate(lay, ids, offs, staging, layer0 + first, count, False)
        src, start, dpages, drope = fanout_tables(ids, offs, ridx)
        dev = lay.device
        self._tables = [_upload(torch.from_numpy(src), dev),
                        _upload(torch.from_numpy(start), dev),
                        _upload(torch.from_numpy(dpages.astype(np.int32)), dev),
                        None if drope is None else
                        _upload(torch.from_numpy(drope.astype(np.int32)), dev)]
        self._keep = keep + [table, staging]
        self.n_src, self.n_dst = int(src.size), int(dpages.size)
        src_d, start_d, pages_d, rope_d = self._tables
        self._args = (table.ptr(first), count, lay.kv_stride, lay.page_stride, lay.page_bytes,
                      lay.num_blocks, src_d.data_ptr(), self.n_src, start_d.data_ptr(),
                      pages_d.data_ptr(), None if rope_d is None else rope_d.data_ptr(),
                      self.n_dst, staging.data_ptr(), staging.numel() * staging.element_size(),
                      lay.layer_bytes, layer0 + first, *tail, _K_LAYOUTS[lay.k_layout],
                      lay.block_size, lay.num_heads)
        self._device = dev

    def __call__(self) -> None:
        rc = _lib.lib().dsr_scatter_fanout(*self._args, _stream_handle(self._device))
        _lib.check("dsr_scatter_fanout", rc)


def _scatter_fanout(table: LayerTable, page_ids, slot_offsets, staging: torch.Tensor,
                    layer0: int, layers, rope=None) -> bool:
    """The load of host tables whose pages share records, each record read
    once (:class:`PreparedFanout`, prepared and launched once). Returns
    False, having launched nothing, for device tables and for pages that
    need the per-page kernels (:func:`fanout_supported`)."""
    lay = table.layout
    if _host_array(page_ids, np.int64) is None or _host_array(slot_offsets, np.int64) is None:
        return False
    if rope is not None:
        if _host_array(rope[0], np.int64) is None:
            return False
        rot_dim = lay.head_dim if rope[2] is None else rope[2]
        if not fanout_supported(lay, rot_dim, rope[3]):
            return False
    elif not fanout_supported(lay):
        return False
    PreparedFanout(table, page_ids, slot_offsets, staging, rope=rope, layer0=layer0,
                   layers=layers)()
    return True


def _rope_args(lay: PagedKVLayout, cos_sin: torch.Tensor, rope_idx, rot_dim, k_scale,
               layer0: int, layer_group):
    """Checks the re-rotation inputs shared by the page and token forms;
    returns (rot_dim, n_tables, n_groups or 0, device layer_group or None,
    k_scale pointer or None)."""
    if lay.dtype not in _DTYPE_CODES:
        raise TypeError(f"re-rotation does not support KV dtype {lay.dtype}")
    if not lay.has_geometry:
        raise ValueError("re-rotation needs the K page geometry: register caches that are "
                         "not 5-D with block_size and head_dim")
    rot_dim = lay.head_dim if rot_dim is None else rot_dim
    grouped = layer_group is not None
    if cos_sin.dtype != torch.float32 or cos_sin.dim() != (4 if grouped else 3) or \
            cos_sin.shape[-2:] != (rot_dim // 2, 2):
        shape = "[groups, n, {}, 2]" if grouped else "[n, {}, 2]"
        raise ValueError("cos_sin must be float32 " + shape.format(rot_dim // 2))
    if cos_sin.device != lay.device or not cos_sin.is_contiguous():
        raise ValueError("cos_sin must be a contiguous device tensor")
    n_groups = cos_sin.shape[0] if grouped else 1
    n_tables = cos_sin.shape[-3]
    ridx = _host_array(rope_idx, np.int64)
    if ridx is not None and ridx.size and (ridx.max() >= n_tables or ridx.min() < -1):
        raise IndexError("rope_idx outside [-1, n_tables)")
    lg_d = None
    if grouped:
        lg = _host_array(layer_group, np.int64)
        if lg is not None and (lg.size < layer0 + lay.num_layers or
                               (lg.size and (lg.min() < -1 or lg.max() >= n_groups))):
            raise IndexError("layer_group needs one group in [-1, n_groups) per layer")
        lg_d = _as_device_table(layer_group, torch.int32, lay.device, "layer_group")
    ks_ptr = None
    if lay.dtype in FP8_DTYPES:
        if k_scale is None:
            raise ValueError("fp8 re-rotation needs per-layer k_scale")
        if (
            k_scale.dtype != torch.float32
            or k_scale.device != lay.device
            or k_scale.numel() < layer0 + lay.num_layers
        ):
            raise ValueError("k_scale must be a float32 device tensor with one scale per layer")
        ks_ptr = k_scale.data_ptr()
    return rot_dim, n_tables, n_groups if grouped else 0, lg_d, ks_ptr


def scatter_rerotate(
    table: LayerTable,
    page_ids,
    slot_offsets,
    staging: torch.Tensor,
    cos_sin: torch.Tensor,
    rope_idx,
    *,
    rot_dim: Optional[int] = None,
    style: str = "neox",
    k_scale: Optional[torch.Tensor] = None,
    layer0: int = 0,
    layers: Optional[tuple[int, int]] = None,
    layer_group=None,
    shared_records: Optional[bool] = None,
) -> None:
    """Scatter with K re-rotated by ``cos_sin[rope_idx[p]]`` (-1 = copy).

    ``cos_sin`` is a float32 tensor ``[n_tables, rot_dim/2, 2]`` from
    :func:`daser_amd.position.delta_tables`; ``k_scale`` holds per-layer
    fp32 scales (fp8 caches only). For models whose layers differ in RoPE
    (other frequencies, or none), ``cos_sin`` is ``[n_groups, n_tables,
    rot_dim/2, 2]`` and ``layer_group[layer0 + l]`` picks layer l's group
    (-1: no RoPE, K copied).

    ``shared_records``: several pages read the same records (a cached chunk
    placed in several requests). Host tables then take the fan-out load
    (:class:`PreparedFanout`) where the pages allow it, device tables a
    launch shaped for cache-served reads. None: inferred from host
    ``slot_offsets`` (at most half of them distinct), False for device
    tables. Results do not depend on it.
    """
    lay = table.layout
    rot_dim, n_tables, n_groups, lg_d, ks_ptr = _rope_args(
        lay, cos_sin, rope_idx, rot_dim, k_scale, layer0, layer_group)
    if shared_records is None:
        shared_records = _shared_offsets(slot_offsets)
    page_ids, slot_offsets, rope_idx = dest_order(page_ids, slot_offsets, rope_idx)
    if shared_records and _scatter_fanout(
            table, page_ids, slot_offsets, staging, layer0, layers,
            (rope_idx, cos_sin, rot_dim, style, k_scale, layer_group)):
        return
    args, _tables = _copy_args(table, page_ids, slot_offsets, staging, layer0, layers)
    ridx_d = _as_device_table(rope_idx, torch.int32, lay.device, "rope_idx")
    if ridx_d.numel() != _tables[0].numel():
        raise ValueError("rope_idx and page_ids differ in length")
    common = (*args, cos_sin.data_ptr(), ridx_d.data_ptr(), n_tables,
              None if lg_d is None else lg_d.data_ptr(), n_groups,
              lay.head_dim, rot_dim, ROPE_STYLES[style], _DTYPE_CODES[lay.dtype], ks_ptr)
    flags = _lib.DSR_REROTATE_SHARED_RECORDS if shared_records else 0
    if lay.k_layout in ("kx", "hnd"):
        name = "dsr_scatter_rerotate_" + lay.k_layout
        rc = getattr(_lib.lib(), name)(*common, lay.block_size, flags,
                                       _stream_handle(lay.device))
        _lib.check(name, rc)
    else:
        rc = _lib.lib().dsr_scatter_rerotate(*common, flags, _stream_handle(lay.device))
        _lib.check("dsr_scatter_rerotate", rc)


def _slots_args(table: LayerTable, slot_mapping, row_offsets, staging, layer0, layers,
                records_written: bool):
    lay = table.layout
    if not lay.has_geometry or lay.k_layout != "nhd":
        raise ValueError("the token form needs token-major pages ([block_size][H][D]) of "
                         "known geometry")
    first, count = (0, lay.num_layers) if layers is None else layers
    if first < 0 or count < 0 or first + count > lay.num_layers:
        raise IndexError("layer range outside the registered caches")
    if staging.device != lay.device or not staging.is_contiguous():
        raise ValueError("staging must be a contiguous tensor on the caches' device")
    row_bytes = lay.num_heads * lay.head_dim * lay.elem_bytes
    sm = _host_array(slot_mapping, np.int64)
    ro = _host_array(row_offsets, np.int64)
    if sm is not None and ro is not None:
        if sm.shape != ro.shape:
            raise ValueError("slot_mapping and row_offsets differ in length")
        valid = sm >= 0
        if valid.any():
            if sm[valid].max() >= lay.num_blocks * lay.block_size:
                raise IndexError("slot outside the block pool")
            r = ro[valid]
            end = r.max() + (layer0 + first + count - 1) * lay.layer_bytes + lay.page_bytes \
                + row_bytes
            if r.min() < 0 or end > staging.numel() * staging.element_size():
                raise IndexError("token row outside the staging buffer")
            if np.any(r % 16):
                raise ValueError("row offsets must be multiples of 16 bytes")
            # Two tokens writing the same record row (gather) or the same
            # slot (scatter) would race inside the launch; as the reference's
            # sequential copies leave the last one's bytes, the earlier ones
            # become padding (slot -1) in a copy of the host table.
            if records_written:
                if np.unique(r).size != r.size:
                    idx = np.nonzero(valid)[0]
                    _, last_rev = np.unique(r[::-1], return_index=True)
                    keep = np.zeros(idx.size, bool)
                    keep[idx.size - 1 - last_rev] = True
                    sm = sm.copy()
                    sm[idx[~keep]] = -1
                    slot_mapping = sm
            else:
                slot_mapping = _last_per_slot(sm)
    sm_d = _as_device_table(slot_mapping, torch.int64, lay.device, "slot_mapping")
    ro_d = _as_device_table(row_offsets, torch.int64, lay.device, "row_offsets")
    if sm_d.numel() != ro_d.numel():
        raise ValueError("slot_mapping and row_offsets differ in length")
    return (table.ptr(first), count, lay.kv_stride, lay.page_stride, lay.page_bytes,
            lay.num_blocks, lay.block_size, row_bytes, sm_d.data_ptr(), ro_d.data_ptr(),
            sm_d.numel(), staging.data_ptr(), staging.numel() * staging.element_size(),
            lay.layer_bytes, layer0 + first), (sm_d, ro_d)


def gather_slots(table: LayerTable, slot_mapping, row_offsets, staging: torch.Tensor, *,
                 layer0: int = 0, layers: Optional[tuple[int, int]] = None) -> None:
    """Token-granular gather driven by vLLM's slot_mapping (-1 = padding):
    each valid token's K and V rows of every layer go to its record rows at
    ``row_offsets[t]`` (see :func:`token_row_offsets`)."""
    args, _tables = _slots_args(table, slot_mapping, row_offsets, staging, layer0, layers, True)
    rc = _lib.lib().dsr_gather_slots(*args, _stream_handle(table.layout.device))
    _lib.check("dsr_gather_slots", rc)


def _last_per_slot(sm: np.ndarray) -> np.ndarray:
    """slot_mapping with every entry but the last of a repeated slot turned
    into padding (-1): the reference's sequential copies leave the last
    one's bytes, while copies inside one launch would race."""
    valid = np.nonzero(sm >= 0)[0]
    dest = sm[valid]
    if np.unique(dest).size == dest.size:
        return sm
    _, last_rev = np.unique(dest[::-1], return_index=True)
    keep = np.zeros(valid.size, bool)
    keep[valid.size - 1 - last_rev] = True
    sm = sm.copy()
    sm[valid[~keep]] = -1
    return sm


def whole_pages(slot_mapping: np.ndarray, row_offsets: np.ndarray, block_size: int,
                row_bytes: int, rope_idx: Optional[np.ndarray] = None):
    """Splits the host tables of a token-form scatter into whole pages and
    the rest. The entries must be in slot order with no slot listed twice
    (padding, -1, anywhere). A block is whole when its block_size slots sit
    in consecutive entries, in order, with consecutive record rows
    (row_offsets stepping by row_bytes: the block's K rows form one record
    page, its V rows the page after) and, with rope_idx, one table index.

    Returns (page_ids, page_offsets, page_rope or None, rest): the whole
    blocks, the record offset of each one's first row (its slot record
    offset in the page form), their table indices, and a mask of the entries
    left for the token kernels."""
    sm = np.asarray(slot_mapping, np.int64)
    ro = np.asarray(row_offsets, np.int64)
    n, bs = sm.size, int(block_size)
    rest = np.ones(n, bool)
    empty = np.zeros(0, np.int64)
    if n < bs:
        return empty, empty, None if rope_idx is None else empty, rest
    step = np.zeros(n, bool)  # entry i continues entry i - 1 inside one record page
    step[1:] = (sm[1:] == sm[:-1] + 1) & (ro[1:] == ro[:-1] + row_bytes) & (sm[:-1] >= 0)
    ri = None
    if rope_idx is not None:
        ri = np.asarray(rope_idx, np.int64)
        step[1:] &= ri[1:] == ri[:-1]
    breaks = np.cumsum(~step)
    i = np.arange(n - bs + 1)
    start = (sm[i] >= 0) & (sm[i] % bs == 0) & (breaks[i + bs - 1] == breaks[i])
    starts = i[start]
    rest[(starts[:, None] + np.arange(bs)).ravel()] = False
    return (sm[starts] // bs, ro[starts], None if ri is None else ri[starts], rest)


def slot_order(slot_mapping, row_offsets, rope_idx=None):
    """Host tables in slot order, repeated slots padded but the last; None
    for device tables."""
    sm = _host_array(slot_mapping, np.int64)
    ro = _host_array(row_offsets, np.int64)
    ri = None if rope_idx is None else _host_array(rope_idx, np.int64)
    if sm is None or ro is None or (rope_idx is not None and ri is None) or not sm.size:
        return None
    if sm.shape != ro.shape or (ri is not None and ri.shape != sm.shape):
        raise ValueError("slot_mapping, row_offsets and rope_idx differ in length")
    order = np.argsort(sm, kind="stable")
    # within a run of equal slots the stable order keeps list order
    return _last_per_slot(sm[order]), ro[order], None if ri is None else ri[order]


def scatter_slots(table: LayerTable, slot_mapping, row_offsets, staging: torch.Tensor, *,
                  layer0: int = 0, layers: Optional[tuple[int, int]] = None) -> None:
    """Inverse of :func:`gather_slots`. Host tables are processed in
    destination-slot order (near-sequential writes), like :func:`scatter`,
    and blocks whose every slot is listed with consecutive record rows go
    as whole pages through the page scatter (:func:`whole_pages`); the other
    tokens (the ragged edges of requests) go through the token kernel;
    whole pages that share records load through :class:`PreparedFanout`,
    as in :func:`scatter`. Device tables go to the token kernel as given."""
    host = slot_order(slot_mapping, row_offsets)
    if host is not None:
        sm, ro, _ = host
        lay = table.layout
        if lay.has_geometry and lay.k_layout == "nhd":
            row = lay.num_heads * lay.head_dim * lay.elem_bytes
            pages, offs, _, rest = whole_pages(sm, ro, lay.block_size, row)
            if pages.size:
                scatter(table, pages, offs, staging, layer0=layer0, layers=layers,
                        shared_records=None)
                sm, ro = sm[rest], ro[rest]
                if not np.any(sm >= 0):
                    return
        slot_mapping, row_offsets = sm, ro
    args, _tables = _slots_args(table, slot_mapping, row_offsets, staging, layer0, layers, False)
    rc = _lib.lib().dsr_scatter_slots(*args, _stream_handle(table.layout.device))
    _lib.check("dsr_scatter_slots", rc)


def scatter_slots_rerotate(table: LayerTable, slot_mapping, row_offsets,
                           staging: torch.Tensor, cos_sin: torch.Tensor, rope_idx, *,
                           rot_dim: Optional[int] = None, style: str = "neox",
                           k_scale: Optional[torch.Tensor] = None, layer0: int = 0,
                           layers: Optional[tuple[int, int]] = None,
                           layer_group=None) -> None:
    """:func:`scatter_slots` with each valid token's K rotated by
    ``cos_sin[rope_idx[t]]`` (-1 = copy), as :func:`scatter_rerotate` rotates
    a page row (same tables, scales and layer groups). Host tables are
    processed in destination-slot order, whole pages with one table index
    through :func:`scatter_rerotate` (the fan-out load where they share
    records)."""
    lay = table.layout
    rot_dim, n_tables, n_groups, lg_d, ks_ptr = _rope_args(
        lay, cos_sin, rope_idx, rot_dim, k_scale, layer0, layer_group)
    host = slot_order(slot_mapping, row_offsets, rope_idx)
    if host is not None:
        sm, ro, ri = host
        if lay.has_geometry and lay.k_layout == "nhd":
            row = lay.num_heads * lay.head_dim * lay.elem_bytes
            pages, offs, pri, rest = whole_pages(sm, ro, lay.block_size, row, ri)
            if pages.size:
                scatter_rerotate(table, pages, offs, staging, cos_sin, pri, rot_dim=rot_dim,
                                 style=style, k_scale=k_scale, layer0=layer0, layers=layers,
                                 layer_group=layer_group, shared_records=None)
                sm, ro, ri = sm[rest], ro[rest], ri[rest]
                if not np.any(sm >= 0):
                    return
        slot_mapping, row_offsets, rope_idx = sm, ro, ri
    args, _tables = _slots_args(table, slot_mapping, row_offsets, staging, layer0, layers, False)
    ridx_d = _as_device_table(rope_idx, torch.int32, lay.device, "rope_idx")
    if ridx_d.numel() != _tables[0].numel():
        raise ValueError("rope_idx and slot_mapping differ in length")
    rc = _lib.lib().dsr_scatter_slots_rerotate(
        *args, cos_sin.data_ptr(), ridx_d.data_ptr(), n_tables,
        None if lg_d is None else lg_d.data_ptr(), n_groups, lay.head_dim, rot_dim,
        ROPE_STYLES[style], _DTYPE_CODES[lay.dtype], ks_ptr, _stream_handle(lay.device))
    _lib.check("dsr_scatter_slots_rerotate", rc)


def token_row_offsets(req_tokens: Sequence[int], slot_bytes: int, block_size: int,
                      row_bytes: int, base: int = 0) -> np.ndarray:
    """Record offset of each token's K row for requests whose records are
    packed back to back (request r's slot i at base + (slots before r + i) *
    slot_bytes): token t of a request sits in its slot t // block_size at row
    t % block_size, the position dsr_gather puts it at."""
    out = []
    slot0 = 0
    for n in req_tokens:
        t = np.arange(int(n), dtype=np.int64)
        out.append(base + (slot0 + t // block_size) * slot_bytes + (t % block_size) * row_bytes)
        slot0 += -(-int(n) // block_size)
    return np.concatenate(out) if out else np.zeros(0, np.int64)


def slot_mapping_for(block_tables: Sequence[Sequence[int]], req_tokens: Sequence[int],
                     block_size: int) -> np.ndarray:
    """vLLM's slot_mapping of the requests' tokens:
    slot = block_ids[t // block_size] * block_size + t % block_size."""
    out = []
    for blocks, n in zip(block_tables, req_tokens):
        t = np.arange(int(n), dtype=np.int64)
        b = np.asarray(blocks, dtype=np.int64)
        out.append(b[t // block_size] * block_size + t % block_size)
    return np.concatenate(out) if out else np.zeros(0, np.int64)


def slot_offsets_for(num_pages: Sequence[int], slot_bytes: int, base: int = 0) -> np.ndarray:
    """Record offsets for requests packed back to back in one staging buffer:
    request r's slot i lives at ``base + (pages before r + i) * slot_bytes``."""
    total = int(sum(num_pages))
    return base + np.arange(total, dtype=np.int64) * slot_bytes


def pages_for_tokens(token_count: int, block_size: int) -> int:
    """ceil(tokens / block_size): pages holding token_count tokens
    (daser/connector/daser_connector.py:280, :292)."""
    return math.ceil(token_count / block_size)
