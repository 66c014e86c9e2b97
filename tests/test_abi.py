"""The C-ABI library loads, exports every symbol include/daser_kv.h
declares, and rejects bad arguments before touching the device."""

from __future__ import annotations

import os
import re

from daser_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "daser_kv.h")


def declared_symbols() -> list[str]:
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dsr_\w+)\s*\(", text)))


def test_header_declares_entry_points():
    syms = declared_symbols()
    assert {"dsr_gather", "dsr_scatter", "dsr_scatter_rerotate",
            "dsr_abi_version", "dsr_error_string"} <= set(syms)


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    for s in declared_symbols():
        assert hasattr(lib, s), s
    assert set(_lib.SIGNATURES) == set(declared_symbols())


def test_abi_version_and_error_strings():
    lib = _lib.lib()
    assert lib.dsr_abi_version() == _lib.DSR_ABI_VERSION
    for code in (_lib.DSR_ERR_ARG, _lib.DSR_ERR_ALIGN, _lib.DSR_ERR_SHAPE):
        assert len(lib.dsr_error_string(code)) > 10
    assert lib.dsr_error_string(0) == b"success"


def _gather(**kw):
    args = dict(layer_base=16, n_layers=2, kv_stride=4096, page_stride=4096,
                page_bytes=4096, num_blocks=8, page_ids=32, slot_offsets=48,
                n_pages=1, staging=64, staging_bytes=1 << 20, layer_bytes=8192,
                layer0=0, stream=None)
    args.update(kw)
    return _lib.lib().dsr_gather(*args.values())


def test_argument_errors_return_before_launch():
    # These never reach the device: validation fails first.
    assert _gather(kv_stride=4100) == _lib.DSR_ERR_ALIGN
    assert _gather(staging=72) == _lib.DSR_ERR_ALIGN
    assert _gather(n_pages=-1) == _lib.DSR_ERR_ARG
    assert _gather(page_ids=None) == _lib.DSR_ERR_ARG
    assert _gather(layer_bytes=4096) == _lib.DSR_ERR_SHAPE
    # empty work is a successful no-op with no launch
    assert _gather(n_pages=0) == _lib.DSR_OK
    assert _gather(n_layers=0) == _lib.DSR_OK


def test_rerotate_argument_errors():
    lib = _lib.lib()
    base = [16, 1, 4096, 4096, 4096, 8, 32, 48, 1, 64, 1 << 20, 8192, 0]

    def call(head_dim=128, rot_dim=128, style=0, dtype=0, k_scale=80, n_tables=1,
             layer_group=None, n_groups=0):
        return lib.dsr_scatter_rerotate(*base, 96, 112, n_tables, layer_group, n_groups,
                                        head_dim, rot_dim, style, dtype, k_scale, 0, None)

    assert call(style=7) == _lib.DSR_ERR_ARG
    assert call(dtype=9) == _lib.DSR_ERR_ARG
    assert call(rot_dim=130) == _lib.DSR_ERR_SHAPE
    assert call(rot_dim=127) == _lib.DSR_ERR_SHAPE
    assert call(head_dim=100, rot_dim=100) == _lib.DSR_ERR_SHAPE  # page not whole rows
    assert call(dtype=2, k_scale=None) == _lib.DSR_ERR_ARG
    assert call(layer_group=128, n_groups=0) == _lib.DSR_ERR_ARG  # groups without a count
    # the split-x entry point: a block size is required, and whole-vector widths
    kx = [*base, 96, 112, 1, None, 0, 128, 128, 0, 0, 80]
    assert lib.dsr_scatter_rerotate_kx(*kx, 0, 0, None) == _lib.DSR_ERR_ARG
    kx[19] = 120  # rot_dim 120: half not a whole number of vectors
    assert lib.dsr_scatter_rerotate_kx(*kx, 16, 0, None) == _lib.DSR_ERR_SHAPE


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "nope.so"))
    try:
        _lib.lib()
    except RuntimeError as e:
        assert "no CPU fallback" in str(e)
    else:
        raise AssertionError("expected a RuntimeError")


def test_set_tuning_checks_and_no_environment_reads():
    """Launch-shape overrides come only through dsr_set_tuning: unknown
    knobs and negative values are rejected, and no library source reads the
    environment."""
    lib = _lib.lib()
    assert lib.dsr_set_tuning(-1, 0) == _lib.DSR_ERR_ARG
    assert lib.dsr_set_tuning(len(_lib.TUNE), 0) == _lib.DSR_ERR_ARG
    assert lib.dsr_set_tuning(_lib.TUNE["rot_kernel"], -2) == _lib.DSR_ERR_ARG
    for knob in _lib.TUNE:
        assert lib.dsr_set_tuning(_lib.TUNE[knob], 0) == _lib.DSR_OK
    # the Python names are exactly the header's knobs
    text = open(HEADER).read()
    header = {m.group(1).lower(): int(m.group(2))
              for m in re.finditer(r"#define DSR_TUNE_(\w+) (\d+)", text) if m.group(1) != "COUNT_"}
    assert header == _lib.TUNE
    assert int(re.search(r"#define DSR_TUNE_COUNT_ (\d+)", text).group(1)) == len(_lib.TUNE)
    csrc = os.path.join(ROOT, "daser_amd", "csrc")
    for name in os.listdir(csrc):
        with open(os.path.join(csrc, name)) as f:
            assert "getenv" not in f.read(), name


def test_static_rerotate_argument_errors():
    """dsr_scatter_rerotate_static checks its host tables' sizes against the
    library's fixed table area before any copy or launch."""
    lib = _lib.lib()

    def call(n_pages=1, page_ids=32, rot_dim=128, n_tables=1, layer_group=None, n_groups=0):
        return lib.dsr_scatter_rerotate_static(
            16, 1, 4096, 4096, 4096, 8, page_ids, 48, n_pages, 64, 1 << 20, 8192, 0, 96, 112,
            n_tables, layer_group, n_groups, 128, rot_dim, 0, 0, None, 0, None)

    n_max = _lib.DSR_STATIC_TABLE_BYTES // 16  # 16 table bytes per page
    assert call(n_pages=n_max + 1) == _lib.DSR_ERR_TOO_LARGE
    assert call(n_tables=_lib.DSR_STATIC_TABLE_BYTES // (64 * 8) + 1) == _lib.DSR_ERR_TOO_LARGE
    assert call(n_pages=0) == _lib.DSR_OK
    assert call(page_ids=None) == _lib.DSR_ERR_ARG
    assert call(n_pages=-1) == _lib.DSR_ERR_ARG
    assert call(rot_dim=127) == _lib.DSR_ERR_SHAPE
    assert call(layer_group=128, n_groups=0) == _lib.DSR_ERR_ARG
    assert b"static table" in lib.dsr_error_string(_lib.DSR_ERR_TOO_LARGE)


def test_fanout_refuses_shapes_it_does_not_take():
    """Geometries the fan-out kernel does not take are refused before any
    launch, so that callers fall back to the per-page entry points."""
    lib = _lib.lib()
    base = [16, 1, 1 << 20, 1 << 20, 64 << 10, 8, 32, 1, 48, 64, 80, 1, 96, 1 << 24, 128 << 10,
            0, 112, 1, None, 0]
    # 64 KiB pages: more than 8 vectors per lane
    assert lib.dsr_scatter_fanout(*base, 128, 128, 0, 0, None, 0, 0, 0, None) == _lib.DSR_ERR_SHAPE
    # neox partner 6 vectors away (head_dim 96): not a power of two
    base[4] = 24 << 10
    base[14] = 48 << 10
    assert lib.dsr_scatter_fanout(*base, 96, 96, 0, 0, None, 0, 0, 0, None) == _lib.DSR_ERR_SHAPE
    # an unknown page layout, and split-x pages without a block size
    base[4] = 32 << 10
    base[14] = 64 << 10
    assert lib.dsr_scatter_fanout(*base, 128, 128, 0, 0, None, 7, 16, 8, None) == _lib.DSR_ERR_ARG
    assert lib.dsr_scatter_fanout(*base, 128, 128, 0, 0, None, 1, 0, 8, None) == _lib.DSR_ERR_ARG
    # the capability query: no work, null tables, the geometry's verdict
    assert lib.dsr_scatter_fanout(16, 1, 1 << 20, 1 << 20, 32 << 10, 8, None, 0, None, None, 16, 0,
                                  16, 0, 64 << 10, 0, None, 0, None, 0, 128, 128, 0, 0, None,
                                  0, 16, 8, None) == _lib.DSR_OK
