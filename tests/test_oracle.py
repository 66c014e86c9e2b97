"""Pins the C oracle before it is trusted as the checker of the HIP kernels.

Each oracle function is checked against something independent of its own
formula: a brute-force restatement of the reference loops, the reference's
own constants, torch's dtype conversions, and closed forms of rotation.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from daser_amd import ops, position
from daser_amd.workloads import KVShape
from oracle import oracle

BF16, FP16, E4M3, E5M2 = oracle.BF16, oracle.FP16, oracle.E4M3, oracle.E5M2


# ---------------------------------------------------------------------------
# gather / scatter: brute force following daser/connector/daser_connector.py


def _reference_save(kv_caches, block_ids_per_req, slot_size):
    """Restates DaserConnector.save_kv_layer (:610-632) with numpy: per
    request a staging buffer of num_slots * SLOT bytes; for each layer (dict
    order) and slot i, staging[i*SLOT + layer*LAYER : +nbytes] =
    bytes(kv[:, block_id]), LAYER = SLOT // num_layers (:608)."""
    num_layers = len(kv_caches)
    layer_size = slot_size // num_layers
    out = []
    for block_ids in block_ids_per_req:
        staging = np.zeros(len(block_ids) * slot_size, dtype=np.uint8)
        for layer_idx, kv in enumerate(kv_caches):
            for slot_i, block_id in enumerate(block_ids):
                dst_off = slot_i * slot_size + layer_idx * layer_size
                src = np.ascontiguousarray(kv[:, block_id]).reshape(-1).view(np.uint8)
                staging[dst_off:dst_off + src.nbytes] = src
        out.append(staging)
    return out


def _reference_load(kv_caches, block_ids_per_req, stagings, slot_size):
    """Restates the scatter loop of DaserConnector.start_load_kv (:536-551)."""
    num_layers = len(kv_caches)
    layer_size = slot_size // num_layers
    for staging, block_ids in zip(stagings, block_ids_per_req):
        for slot_i, block_id in enumerate(block_ids):
            slot_base = slot_i * slot_size
            for layer_idx, kv in enumerate(kv_caches):
                dst = kv[:, block_id]
                off = slot_base + layer_idx * layer_size
                kv[:, block_id] = staging[off:off + dst.nbytes].view(kv.dtype).reshape(dst.shape)


def _slot_size(kv_caches):
    # register_kv_caches: layer_size = kv.nbytes // kv.shape[1]; SLOT = layer_size * L
    kv = kv_caches[0]
    return kv.nbytes // kv.shape[1] * len(kv_caches)


@pytest.mark.parametrize("dtype,shape", [(np.uint16, (3, 2, 4, 8)), (np.uint8, (2, 4, 1, 16))])
def test_gather_matches_reference_loop(dtype, shape):
    rng = np.random.default_rng(0)
    L, bs, H, D = shape
    nb = 11
    caches = [rng.integers(0, np.iinfo(dtype).max, size=(2, nb, bs, H, D), dtype=dtype)
              for _ in range(L)]
    reqs = [[5, 2, 9], [0], [7, 3]]
    slot = _slot_size(caches)
    ref = _reference_save(caches, reqs, slot)
    ids = np.concatenate([np.asarray(r) for r in reqs]).astype(np.int32)
    offs = np.arange(ids.size, dtype=np.int64) * slot
    stg = np.zeros(ids.size * slot, dtype=np.uint8)
    oracle.gather(caches, ids, offs, stg, slot // L)
    assert np.array_equal(stg, np.concatenate(ref))


def test_scatter_matches_reference_loop_and_round_trips():
    rng = np.random.default_rng(1)
    L, bs, H, D, nb = 4, 2, 2, 8, 9
    src = [rng.integers(0, 65535, size=(2, nb, bs, H, D), dtype=np.uint16) for _ in range(L)]
    reqs = [[1, 4], [8, 0, 6]]
    slot = _slot_size(src)
    stagings = _reference_save(src, reqs, slot)
    ref_dst = [np.zeros_like(c) for c in src]
    _reference_load(ref_dst, reqs, stagings, slot)
    ids = np.concatenate([np.asarray(r) for r in reqs]).astype(np.int32)
    offs = np.arange(ids.size, dtype=np.int64) * slot
    dst = [np.zeros_like(c) for c in src]
    oracle.scatter(dst, ids, offs, np.concatenate(stagings), slot // L)
    for a, b, s in zip(dst, ref_dst, src):
        assert np.array_equal(a, b)
        assert np.array_equal(a[:, ids], s[:, ids])  # scatter . gather = id on touched
        untouched = np.setdiff1d(np.arange(nb), ids)
        assert not a[:, untouched].any()


def test_per_layer_record_offsets():
    """layer0 places a single-layer launch at its record slot."""
    rng = np.random.default_rng(2)
    caches = [rng.integers(0, 255, size=(2, 3, 2, 1, 16), dtype=np.uint8) for _ in range(3)]
    slot = _slot_size(caches)
    full = np.zeros(2 * slot, dtype=np.uint8)
    oracle.gather(caches, [2, 0], [0, slot], full, slot // 3)
    per = np.zeros_like(full)
    for l in range(3):
        oracle.gather([caches[l]], [2, 0], [0, slot], per, slot // 3, layer0=l)
    assert np.array_equal(full, per)


@pytest.mark.parametrize(
    "layers,expected",
    [
        (28, 8 * 128 * 2 * 28 * 16 * 2),  # reference tests/test_config.py:12-21
        (36, 2_359_296),  # reference tests/integration/conftest.py:26-30
        (32, 2_097_152),  # reference benchmarks/bench_storage_imdb.py:45-48
    ],
)
def test_slot_size_matches_reference_constants(layers, expected):
    caches = [torch.empty((2, 64, 16, 8, 128), dtype=torch.bfloat16, device="meta")
              for _ in range(layers)]
    lay = ops.PagedKVLayout.from_caches(caches)
    assert lay.slot_bytes == expected
    assert lay.layer_bytes == 65_536
    assert KVShape(layers, 8, 128, 16, 2).slot_bytes == expected


# ---------------------------------------------------------------------------
# element codecs against torch's conversions


def test_e4m3_decode_all_codes():
    codes = np.arange(256, dtype=np.uint32)
    ours = oracle.decode(E4M3, codes)
    ref = torch.from_numpy(codes.astype(np.uint8)).view(torch.float8_e4m3fn).double().numpy()
    assert np.array_equal(np.isnan(ours), np.isnan(ref))
    ok = ~np.isnan(ref)
    assert np.array_equal(ours[ok], ref[ok])
    assert np.isnan(ours[[0x7F, 0xFF]]).all() and np.isnan(ours).sum() == 2
    assert ours[0x7E] == 448.0 and ours[0x01] == 2.0 ** -9


def _fp32_sweep(rng, n, lo, hi):
    mags = np.exp(rng.uniform(np.log(lo), np.log(hi), n))
    v = (mags * rng.choice([-1.0, 1.0], n)).astype(np.float32)
    return v


def test_e4m3_encode_matches_torch_rne():
    rng = np.random.default_rng(3)
    v = _fp32_sweep(rng, 20000, 2.0 ** -12, 448.0)
    # exact ties between neighbouring codes (midpoints), incl. subnormals
    codes = np.arange(0, 0x7E, dtype=np.uint32)
    a = oracle.decode(E4M3, codes)
    mid = ((a[:-1] + a[1:]) / 2).astype(np.float32)
    v = np.concatenate([v, mid, -mid, np.float32([0.0, -0.0, 448.0, -448.0])])
    ours = oracle.encode(E4M3, v.astype(np.float64)).astype(np.uint8)
    ref = torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(ours, ref)


def test_e4m3_encode_saturates_and_keeps_nan():
    out = oracle.encode(E4M3, [449.0, 1e30, -500.0, np.inf, -np.inf, np.nan])
    assert list(out) == [0x7E, 0x7E, 0xFE, 0x7E, 0xFE, 0x7F]


def test_e5m2_decode_all_codes():
    codes = np.arange(256, dtype=np.uint32)
    ours = oracle.decode(oracle.E5M2, codes)
    ref = torch.from_numpy(codes.astype(np.uint8)).view(torch.float8_e5m2).double().numpy()
    assert np.array_equal(np.isnan(ours), np.isnan(ref))
    ok = ~np.isnan(ref)
    assert np.array_equal(ours[ok], ref[ok])
    assert np.isnan(ours).sum() == 6 and ours[0x7C] == np.inf and ours[0xFC] == -np.inf
    assert ours[0x7B] == 57344.0 and ours[0x01] == 2.0 ** -16


def test_e5m2_encode_matches_torch_rne():
    rng = np.random.default_rng(13)
    v = _fp32_sweep(rng, 20000, 2.0 ** -18, 57344.0)
    codes = np.arange(0, 0x7C, dtype=np.uint32)  # every finite positive code
    a = oracle.decode(oracle.E5M2, codes)
    mid = ((a[:-1] + a[1:]) / 2).astype(np.float32)  # exact ties, subnormals included
    v = np.concatenate([v, mid, -mid, np.float32([0.0, -0.0, 57344.0, -57344.0, 60000.0])])
    ours = oracle.encode(oracle.E5M2, v.astype(np.float64)).astype(np.uint8)
    ref = torch.from_numpy(v).to(torch.float8_e5m2).view(torch.uint8).numpy()
    assert np.array_equal(ours, ref)


def test_e5m2_encode_saturates_and_keeps_nan():
    """Beyond the largest finite value torch's conversion gives infinity;
    the oracle (and the kernels) saturate, as the 8-bit KV cache writes do,
    and keep NaN as torch's 0x7F."""
    out = oracle.encode(oracle.E5M2, [61440.0, 1e30, -70000.0, np.inf, -np.inf, np.nan])
    assert list(out) == [0x7B, 0x7B, 0xFB, 0x7B, 0xFB, 0x7F]
    assert torch.tensor([np.nan]).to(torch.float8_e5m2).view(torch.uint8).item() == 0x7F


@pytest.mark.parametrize("dt,tdt", [(BF16, torch.bfloat16), (FP16, torch.float16)])
def test_16bit_codecs_match_torch(dt, tdt):
    codes = np.arange(65536, dtype=np.uint32)
    ours = oracle.decode(dt, codes)
    ref = torch.from_numpy(codes.astype(np.uint16).view(np.int16)).view(tdt).double().numpy()
    assert np.array_equal(np.isnan(ours), np.isnan(ref))
    ok = ~np.isnan(ref)
    assert np.array_equal(ours[ok], ref[ok])
    rng = np.random.default_rng(4)
    hi = 3e38 if dt == BF16 else 65000.0
    v = _fp32_sweep(rng, 40000, 1e-9, hi)
    a = ours[ok & np.isfinite(ours)]
    a = np.unique(a[(np.abs(a) < hi)])
    mid = ((a[:-1] + a[1:]) / 2)
    mid = mid[np.abs(mid) < hi].astype(np.float32)
    v = np.concatenate([v, mid[::7]])
    got = oracle.encode(dt, v.astype(np.float64)).astype(np.uint16)
    exp = torch.from_numpy(v).to(tdt).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, exp)


# ---------------------------------------------------------------------------
# rotation: closed forms


def _rot_case(dt, L=2, H=3, D=16, nb=6, scale=1.0, seed=5):
    rng = np.random.default_rng(seed)
    vals = rng.normal(size=(2, nb, 2, H, D)) * scale
    if dt == BF16:
        bits = torch.from_numpy(vals.astype(np.float32)).to(torch.bfloat16).view(torch.int16)
        return [bits.numpy().view(np.uint16).copy() for _ in range(L)]
    if dt == FP16:
        bits = torch.from_numpy(vals.astype(np.float32)).to(torch.float16).view(torch.int16)
        return [bits.numpy().view(np.uint16).copy() for _ in range(L)]
    tdt = torch.float8_e4m3fn if dt == E4M3 else torch.float8_e5m2
    bits = torch.from_numpy(vals.astype(np.float32)).to(tdt).view(torch.uint8)
    return [bits.numpy().copy() for _ in range(L)]


def _records(caches, ids):
    slot = _slot_size(caches)
    stg = np.zeros(len(ids) * slot, dtype=np.uint8)
    offs = np.arange(len(ids), dtype=np.int64) * slot
    oracle.gather(caches, ids, offs, stg, slot // len(caches))
    return stg, offs, slot // len(caches)


def _rerotate(caches, ids, dt, stored, new, rot_dim=None, style=oracle.NEOX,
              theta=10000.0, k_scale=None, inv_freq=None):
    stg, offs, lb = _records(caches, ids)
    D = caches[0].shape[-1]
    out = [np.zeros_like(c) for c in caches]
    n = len(ids)
    oracle.scatter_rerotate(out, ids, offs, stg, lb, dtype=dt, rot_dim=rot_dim or D,
                            style=style, stored_pos=np.full(n, stored), new_pos=np.full(n, new),
                            rotate=np.ones(n), theta=theta, k_scale=k_scale, inv_freq=inv_freq)
    return out


def test_zero_delta_is_bit_exact_copy():
    for dt in (BF16, FP16, E4M3, E5M2):
        c = _rot_case(dt, scale=3.0)
        out = _rerotate(c, [1, 4], dt, stored=777, new=777,
                        k_scale=np.float32([0.7, 1.3]) if dt in (E4M3, E5M2) else None)
        for a, b in zip(out, c):
            assert np.array_equal(a[:, [1, 4]], b[:, [1, 4]])


def test_known_answer_single_pair():
    """(1, 0) rotated by delta with w_0 = 1 is (cos delta, sin delta)."""
    one = np.zeros((2, 1, 1, 1, 2), dtype=np.uint16)
    one[0, 0, 0, 0, 0] = 0x3F80  # bf16 1.0
    for delta in (1, 2, 1000, 32767):
        out = _rerotate([one], [0], BF16, stored=0, new=delta, theta=12345.0)
        got = oracle.decode(BF16, out[0][0, 0, 0, 0])
        exp = torch.tensor([math.cos(delta), math.sin(delta)]).to(torch.bfloat16).double().numpy()
        assert np.array_equal(got, exp)


def test_matches_complex_multiplication():
    """neox pair (x_j, x_{j+R/2}) rotates like x_j + i x_{j+R/2} times
    e^{i delta w_j}, w_j = theta^(-2j/R), evaluated here in complex128."""
    c = _rot_case(BF16, D=32)
    delta, theta = 4097, 500000.0
    out = _rerotate(c, [0, 3], BF16, stored=0, new=delta, theta=theta)
    x = oracle.decode(BF16, c[0][0, [0, 3]])
    z = x[..., :16] + 1j * x[..., 16:]
    w = theta ** (-2.0 * np.arange(16) / 32)
    zr = z * np.exp(1j * delta * w)
    exp_bits = oracle.encode(BF16, np.concatenate([zr.real, zr.imag], axis=-1))
    assert np.array_equal(out[0][0, [0, 3]], exp_bits.astype(np.uint16))
    assert np.array_equal(out[0][1, [0, 3]], c[0][1, [0, 3]])  # V untouched


def test_composition_of_rotations():
    """R(200) after R(300) is R(500) (each step rounded once to bf16), and a
    move from stored position 1000 to 1500 equals one from 0 to 500."""
    c = _rot_case(BF16, D=16, seed=15)
    two = _rerotate(_rerotate(c, [2], BF16, stored=0, new=300, theta=777.0), [2], BF16,
                    stored=300, new=500, theta=777.0)
    one = _rerotate(c, [2], BF16, stored=1000, new=1500, theta=777.0)
    ok, msg = oracle.rotation_within_tolerance(two[0][0, 2], one[0][0, 2], BF16, 2 ** -7)
    assert ok, msg
    assert np.median(oracle.ulp_steps(two[0][0, 2], one[0][0, 2], BF16)) == 0


def test_inverse_and_norm_preservation():
    c = _rot_case(BF16, D=16, seed=9)
    fwd = _rerotate(c, [0, 1, 2], BF16, stored=0, new=12345)
    back = _rerotate(fwd, [0, 1, 2], BF16, stored=12345, new=0)
    d = oracle.ulp_steps(back[0][0, :3], c[0][0, :3], BF16)
    x = oracle.decode(BF16, c[0][0, :3])
    y = oracle.decode(BF16, fwd[0][0, :3])
    n0 = np.hypot(x[..., :8], x[..., 8:])
    n1 = np.hypot(y[..., :8], y[..., 8:])
    assert np.allclose(n0, n1, rtol=2 ** -7, atol=1e-6)
    # two roundings to bf16: within 2 ulps except near-cancelled elements
    ok, msg = oracle.rotation_within_tolerance(back[0][0, :3], c[0][0, :3], BF16, 2 ** -7)
    assert ok, msg
    assert np.median(d) == 0


def test_gptj_is_neox_on_interleaved_layout():
    """Interleaving (x_j, x_{j+R/2}) into (2j, 2j+1) turns the neox rotation
    into the gptj one, bit for bit."""
    c = _rot_case(BF16, D=16, seed=11)
    perm = np.empty(16, dtype=np.int64)
    perm[0::2] = np.arange(8)
    perm[1::2] = np.arange(8, 16)
    ci = [np.ascontiguousarray(x[..., perm]) for x in c]
    neox = _rerotate(c, [0, 5], BF16, stored=0, new=333, style=oracle.NEOX)
    gptj = _rerotate(ci, [0, 5], BF16, stored=0, new=333, style=oracle.GPTJ)
    for a, b in zip(neox, gptj):
        assert np.array_equal(a[..., perm], b)


def test_partial_rotary_copies_tail():
    c = _rot_case(BF16, D=32, seed=12)
    out = _rerotate(c, [1], BF16, stored=0, new=99, rot_dim=16)
    assert np.array_equal(out[0][0, 1, ..., 16:], c[0][0, 1, ..., 16:])
    full = _rerotate([x[..., :16].copy() for x in c], [1], BF16, stored=0, new=99, rot_dim=16)
    assert np.array_equal(out[0][0, 1, ..., :16], full[0][0, 1])


@pytest.mark.parametrize("dt", [E4M3, E5M2])
def test_fp8_dequant_rotate_requant(dt):
    c = _rot_case(dt, D=16, scale=40.0, seed=13)
    ks = np.float32([0.25, 3.0])
    out = _rerotate(c, [0, 2], dt, stored=0, new=2024, k_scale=ks, theta=500000.0)
    for l in range(2):
        x = oracle.decode(dt, c[l][0, [0, 2]]) * float(ks[l])
        z = x[..., :8] + 1j * x[..., 8:]
        w = 500000.0 ** (-2.0 * np.arange(8) / 16)
        zr = z * np.exp(1j * 2024 * w) / float(ks[l])
        exp = oracle.encode(dt, np.concatenate([zr.real, zr.imag], axis=-1))
        assert np.array_equal(out[l][0, [0, 2]], exp.astype(np.uint8))


def test_custom_inv_freq_is_used():
    c = _rot_case(BF16, D=4, seed=14)
    inv = np.array([0.5, 0.125])
    out = _rerotate(c, [0], BF16, stored=0, new=10, inv_freq=inv)
    x = oracle.decode(BF16, c[0][0, 0])
    z = (x[..., :2] + 1j * x[..., 2:]) * np.exp(1j * 10 * inv)
    exp = oracle.encode(BF16, np.concatenate([z.real, z.imag], axis=-1))
    assert np.array_equal(out[0][0, 0], exp.astype(np.uint16))


# ---------------------------------------------------------------------------
# host tables consumed by the kernel


def test_delta_tables_match_direct_evaluation():
    t = position.delta_tables([0, 7, 32767], 128, 500000.0).numpy()
    w = 500000.0 ** (-2.0 * np.arange(64) / 128)
    for r, d in enumerate([0, 7, 32767]):
        assert np.array_equal(t[r, :, 0], np.cos(d * w).astype(np.float32))
        assert np.array_equal(t[r, :, 1], np.sin(d * w).astype(np.float32))
    assert np.all(t[0, :, 0] == 1.0) and np.all(t[0, :, 1] == 0.0)


def test_page_rope_index():
    idx, uniq = position.page_rope_index([2, 1, 3, 2], [5, 0, 5, 9])
    assert uniq == [5, 9]
    assert idx.tolist() == [0, 0, -1, 0, 0, 0, 1, 1]


# ---------------------------------------------------------------------------
# token-granular (slot_mapping) forms


def test_slot_gather_equals_page_gather_on_valid_tokens():
    """With slot = block_ids[t // bs] * bs + t % bs and each token's record
    row at slot t // bs, row t % bs, the token form writes the page form's
    bytes for every valid token and leaves the tail rows of a partial last
    page untouched; padding tokens (slot -1) are skipped."""
    rng = np.random.default_rng(20)
    L, nb, bs, H, D = 3, 10, 4, 2, 8
    caches = [rng.integers(1, 65535, size=(2, nb, bs, H, D), dtype=np.uint16) for _ in range(L)]
    tables = [[7, 1, 4], [9, 0]]
    toks = [10, 8]  # request 0 ends inside its third page
    slot = _slot_size(caches)
    row = H * D * 2
    ids = np.concatenate([np.asarray(t) for t in tables]).astype(np.int32)
    page = np.zeros(ids.size * slot, dtype=np.uint8)
    oracle.gather(caches, ids, np.arange(ids.size) * slot, page, slot // L)
    sm = ops.slot_mapping_for(tables, toks, bs)
    ro = ops.token_row_offsets(toks, slot, bs, row)
    sm = np.concatenate([sm, [-1, -1]])  # padding
    ro = np.concatenate([ro, [0, 0]])
    tok = np.zeros_like(page)
    oracle.gather_slots(caches, sm, ro, tok, slot // L)
    mask = np.zeros_like(page, dtype=bool)
    for r in ro[:-2]:
        for l in range(L):
            o = r + l * (slot // L)
            mask[o:o + row] = True
            mask[o + bs * row:o + bs * row + row] = True
    assert np.array_equal(tok[mask], page[mask])
    assert not tok[~mask].any()
    # the partial page's tail rows (tokens 10, 11 of request 0) stay zero
    back = [np.zeros_like(c) for c in caches]
    oracle.scatter_slots(back, sm, ro, tok, slot // L)
    for b, c in zip(back, caches):
        bt = b[:, :, :, :, :].reshape(2, nb * bs, H, D)
        ct = c.reshape(2, nb * bs, H, D)
        valid = sm[sm >= 0]
        assert np.array_equal(bt[:, valid], ct[:, valid])
        others = np.setdiff1d(np.arange(nb * bs), valid)
        assert not bt[:, others].any()


@pytest.mark.parametrize("dt,style,rot", [(BF16, oracle.NEOX, 16), (E4M3, oracle.GPTJ, 12),
                                          (FP16, oracle.NEOX, 8), (E5M2, oracle.NEOX, 16)])
def test_slot_rerotate_equals_page_rerotate_on_valid_tokens(dt, style, rot):
    """The token form of the re-rotation writes, for every valid token, the
    bytes of the page form (pinned above by closed forms) on the same
    records; padding tokens are skipped, tail rows of a partial page are not
    written, and tokens without rotation are plain copies."""
    rng = np.random.default_rng(21 + dt)
    L, nb, bs, H, D = 2, 10, 4, 3, 16
    c8 = dt in (E4M3, E5M2)
    if c8:
        caches = [_rot_case(dt, L=1, H=H, D=D, nb=nb, scale=30.0, seed=40 + l)[0]
                  for l in range(L)]
        caches = [np.concatenate([c] * 2, axis=2)[:, :, :bs].copy() for c in caches]
    else:
        caches = [_rot_case(dt, L=1, H=H, D=D, nb=nb, seed=40 + l)[0] for l in range(L)]
        caches = [np.concatenate([c] * 2, axis=2)[:, :, :bs].copy() for c in caches]
    ks = np.float32([0.5, 3.0]) if c8 else None
    tables = [[7, 1, 4], [9, 0]]
    toks = [10, 8]
    deltas = [777, 0]  # request 1 unrotated
    slot = _slot_size(caches)
    row = H * D * caches[0].itemsize
    ids = np.concatenate([np.asarray(t) for t in tables]).astype(np.int32)
    recs = np.zeros(ids.size * slot, dtype=np.uint8)
    oracle.gather(caches, ids, np.arange(ids.size) * slot, recs, slot // L)
    # page form: every page of each request rotated by its delta
    pdel = np.repeat(deltas, [len(t) for t in tables])
    page = [np.zeros_like(c) for c in caches]
    oracle.scatter_rerotate(page, ids, np.arange(ids.size) * slot, recs, slot // L, dtype=dt,
                            rot_dim=rot, style=style, stored_pos=np.zeros(ids.size, np.int64),
                            new_pos=pdel, rotate=pdel != 0, theta=500000.0, k_scale=ks)
    # token form: per-token positions of the same requests, plus padding
    sm = np.concatenate([ops.slot_mapping_for(tables, toks, bs), [-1, -1]])
    ro = np.concatenate([ops.token_row_offsets(toks, slot, bs, row), [0, 0]])
    tdel = np.concatenate([np.full(n, d) for n, d in zip(toks, deltas)] + [[5, 5]])
    tok = [np.zeros_like(c) for c in caches]
    oracle.scatter_slots_rerotate(tok, sm, ro, recs, slot // L, dtype=dt, rot_dim=rot,
                                  style=style, stored_pos=np.zeros(sm.size, np.int64),
                                  new_pos=tdel, rotate=tdel != 0, theta=500000.0, k_scale=ks)
    valid = sm[sm >= 0]
    others = np.setdiff1d(np.arange(nb * bs), valid)
    for a, b in zip(tok, page):
        at = a.reshape(2, nb * bs, H, D)
        bt = b.reshape(2, nb * bs, H, D)
        assert np.array_equal(at[:, valid], bt[:, valid])
        assert not at[:, others].any()
    moved = tok[0].reshape(2, nb * bs, H, D)[0, valid[:10]]
    plain = [np.zeros_like(c) for c in caches]
    oracle.scatter_slots(plain, sm, ro, recs, slot // L)
    assert not np.array_equal(moved, plain[0].reshape(2, nb * bs, H, D)[0, valid[:10]])
    assert np.array_equal(tok[0].reshape(2, nb * bs, H, D)[:, valid[10:]],
                          plain[0].reshape(2, nb * bs, H, D)[:, valid[10:]])


@pytest.mark.parametrize("itemsize,bs,h,d", [(2, 16, 2, 64), (1, 8, 3, 32), (2, 4, 1, 16)])
def test_kx_layout_permutation_brute_force(itemsize, bs, h, d):
    """kx_to_nhd / nhd_to_kx against the split-x index formula evaluated
    element by element: (t, h, d) at ((h * (D/X) + d/X) * bs + t) * X + d % X."""
    x = 16 // itemsize
    dt = np.uint16 if itemsize == 2 else np.uint8
    n = bs * h * d
    page = (np.arange(2 * n) % (np.iinfo(dt).max + 1)).astype(dt).reshape(2, n)
    nhd = oracle.kx_to_nhd(page, bs, h, d)
    assert nhd.shape == (2, bs, h, d)
    for p in range(2):
        for t in range(bs):
            for hh in range(h):
                for dd in range(d):
                    pos = ((hh * (d // x) + dd // x) * bs + t) * x + dd % x
                    assert nhd[p, t, hh, dd] == page[p, pos]
    assert np.array_equal(oracle.nhd_to_kx(nhd), page)
