"""Position encoders and RoPE delta tables for reused-chunk re-rotation.

``PositionEncoder`` / ``FixedOffsetEncoder`` keep the reference interface
(daser/position/base.py:10-48, daser/position/fixed_offset.py:11-50): an
integer offset is assigned when a chunk is allocated and returned when it is
loaded. The reference stops there; this module adds what the load path needs
to make a chunk stored at position ``stored`` valid at position ``new``: the
per-chunk angle table of ``R(new) . R(stored)^-1 = R(new - stored)``.

The tables are computed on the host in float64 (angles reach
``32768 * 1 rad`` for theta = 5e5 at head_dim 128, where float32 argument
reduction would lose ~1e-3 rad) and rounded once to float32 for the kernel.
"""

from __future__ import annotations

from abc import ABC, abstractmethod
from typing import Optional, Sequence

import numpy as np
import torch


class PositionEncoder(ABC):
    """Pluggable position strategy (reference daser/position/base.py:10-48)."""

    @abstractmethod
    def assign_offset(self, chunk_key: str, token_count: int) -> int:
        """Position of the chunk's first token when it is stored."""

    @abstractmethod
    def get_offset(self, meta) -> int:
        """Stored position to undo when the chunk is loaded (``meta.pos_offset``)."""


class FixedOffsetEncoder(PositionEncoder):
    """Every chunk is stored at one fixed position (default 0).

    Reference daser/position/fixed_offset.py:11-50; its docstring names the
    case this build implements: RoPE re-applied at load time.
    """

    def __init__(self, fixed_offset: int = 0) -> None:
        self._offset = int(fixed_offset)

    def assign_offset(self, chunk_key: str, token_count: int) -> int:
        return self._offset

    def get_offset(self, meta) -> int:
        return int(meta.pos_offset)


class PrefillOffsetEncoder(PositionEncoder):
    """Stores each chunk at the position it was actually prefilled at.

    The reference's interface anticipates encoders beyond the fixed offset
    (daser/position/base.py:10-20). A chunk cached out of the middle of a
    prompt (a retrieved passage at token 3000) holds K rotated for positions
    3000.., so its stored offset must be 3000 for a later load at another
    position to re-rotate by the right delta. Whoever splits the prompt
    calls :meth:`note_position` before the chunk is allocated;
    :meth:`assign_offset` then returns that position once (and ``default``
    for chunks never noted, e.g. prompt prefixes at 0).
    """

    def __init__(self, default: int = 0) -> None:
        self._default = int(default)
        self._pending: dict[str, int] = {}

    def note_position(self, chunk_key: str, first_position: int) -> None:
        if first_position < 0:
            raise ValueError("positions are non-negative")
        self._pending[chunk_key] = int(first_position)

    def assign_offset(self, chunk_key: str, token_count: int) -> int:
        return self._pending.pop(chunk_key, self._default)

    def get_offset(self, meta) -> int:
        return int(meta.pos_offset)


def rope_inv_freq(rot_dim: int, theta: float) -> np.ndarray:
    """inv_freq_j = theta^(-2j/rot_dim), j < rot_dim/2, in float64
    (RoFormer, Su et al. 2021; the Llama / GPT-NeoX convention)."""
    if rot_dim <= 0 or rot_dim % 2:
        raise ValueError("rot_dim must be a positive even number")
    j = np.arange(rot_dim // 2, dtype=np.float64)
    return np.power(float(theta), -2.0 * j / rot_dim)


def llama3_inv_freq(
    rot_dim: int,
    theta: float,
    factor: float,
    low_freq_factor: float,
    high_freq_factor: float,
    original_max_position: int,
) -> np.ndarray:
    """Frequency-dependent scaling of Llama 3.1 ("rope_type": "llama3")."""
    inv = rope_inv_freq(rot_dim, theta)
    low_wl = original_max_position / low_freq_factor
    high_wl = original_max_position / high_freq_factor
    wl = 2.0 * np.pi / inv
    smooth = (original_max_position / wl - low_freq_factor) / (high_freq_factor - low_freq_factor)
    scaled = np.where(wl > low_wl, inv / factor, inv)
    mid = (wl <= low_wl) & (wl >= high_wl)
    return np.where(mid, (1 - smooth) * inv / factor + smooth * inv, scaled)


def yarn_inv_freq(rot_dim: int, theta: float, factor: float, original_max_position: int,
                  beta_fast: float = 32.0, beta_slow: float = 1.0,
                  truncate: bool = True) -> np.ndarray:
    """YaRN frequencies (Peng et al. 2023, "YaRN: Efficient Context Window
    Extension"): dimensions rotating faster than beta_fast turns over the
    original context keep their frequency, slower than beta_slow are
    interpolated by 1/factor, a linear ramp in between. The attention
    magnitude factor of YaRN scales cos/sin at prefill; a delta rotation is
    pure, so that factor is not part of the re-rotation table."""
    import math

    inv = rope_inv_freq(rot_dim, theta)

    def corr_dim(n_rot: float) -> float:
        return (rot_dim * math.log(original_max_position / (n_rot * 2 * math.pi))) / (
            2 * math.log(theta))

    low, high = corr_dim(beta_fast), corr_dim(beta_slow)
    if truncate:
        low, high = math.floor(low), math.ceil(high)
    low, high = max(low, 0), min(high, rot_dim - 1)
    if low == high:
        high += 0.001
    ramp = np.clip((np.arange(rot_dim // 2, dtype=np.float64) - low) / (high - low), 0.0, 1.0)
    extrapolation = 1.0 - ramp
    return (inv / factor) * (1.0 - extrapolation) + inv * extrapolation


def inv_freq_for(rope_scaling: Optional[dict], rot_dim: int, theta: float) -> np.ndarray:
    """inv_freq of a model's RoPE from its HF-style ``rope_scaling`` entry
    (None / "default", "mrope", "linear", "llama3", "yarn"). Scalings whose
    frequencies depend on the sequence length at prefill ("dynamic",
    "longrope") leave no single rotation between two positions and are
    rejected."""
    if not rope_scaling:
        return rope_inv_freq(rot_dim, theta)
    kind = rope_scaling.get("rope_type", rope_scaling.get("type", "default"))
    if kind in ("default", "mrope"):
        # M-RoPE (Qwen2-VL) splits the rotary dims into temporal / height /
        # width sections driven by three position components, with the
        # plain frequencies. Moving a cached chunk shifts all three by the
        # same delta, so one delta rotation with these frequencies is exact.
        return rope_inv_freq(rot_dim, theta)
    if kind == "linear":
        return rope_inv_freq(rot_dim, theta) / float(rope_scaling["factor"])
    if kind == "llama3":
        return llama3_inv_freq(rot_dim, theta, float(rope_scaling["factor"]),
                               float(rope_scaling["low_freq_factor"]),
                               float(rope_scaling["high_freq_factor"]),
                               int(rope_scaling["original_max_position_embeddings"]))
    if kind == "yarn":
        return yarn_inv_freq(rot_dim, theta, float(rope_scaling["factor"]),
                             int(rope_scaling["original_max_position_embeddings"]),
                             float(rope_scaling.get("beta_fast", 32.0)),
                             float(rope_scaling.get("beta_slow", 1.0)),
                             bool(rope_scaling.get("truncate", True)))
    raise ValueError(f"RoPE scaling {kind!r} depends on the sequence length; a stored chunk "
                     "cannot be re-rotated by a position delta")


def layer_rope_groups(specs: Sequence[Optional[dict]], rot_dim: int,
                      default_theta: float = 10000.0) -> tuple[np.ndarray, list[np.ndarray]]:
    """Per-layer RoPE specs -> (group of each layer, inv_freq of each group).

    ``specs[l]`` is None for a layer without RoPE (group -1), else a dict with
    ``rope_theta`` and optionally ``rope_scaling``; layers with the same
    frequencies share a group.
    """
    groups: list[np.ndarray] = []
    keys: dict[bytes, int] = {}
    out = np.full(len(specs), -1, np.int32)
    for l, spec in enumerate(specs):
        if spec is None:
            continue
        inv = inv_freq_for(spec.get("rope_scaling"), rot_dim,
                           float(spec.get("rope_theta", default_theta)))
        k = inv.tobytes()
        if k not in keys:
            keys[k] = len(groups)
            groups.append(inv)
        out[l] = keys[k]
    return out, groups


def _text_config(hf_config):
    return getattr(hf_config, "text_config", None) or hf_config


def head_dim_from_hf(hf_config) -> Optional[int]:
    """Attention head size of a HF config: ``head_dim`` when set, else
    hidden_size / num_attention_heads; None when neither is there."""
    cfg = _text_config(hf_config)
    d = getattr(cfg, "head_dim", None)
    if isinstance(d, int) and d > 0:
        return d
    hs, nh = getattr(cfg, "hidden_size", None), getattr(cfg, "num_attention_heads", None)
    if isinstance(hs, int) and isinstance(nh, int) and nh > 0 and hs % nh == 0:
        return hs // nh
    return None


def model_rope_from_hf(hf_config) -> tuple[Optional[float], Optional[dict]]:
    """(rope_theta, rope_scaling) of a HF config, in either form
    transformers uses: ``rope_theta`` / ``rope_scaling`` attributes, or one
    ``rope_parameters`` dict (which carries ``rope_theta`` itself). For
    per-layer-type parameters the full-attention entry is returned."""
    cfg = _text_config(hf_config)
    rp = getattr(cfg, "rope_parameters", None)
    if isinstance(rp, dict) and rp:
        if all(isinstance(v, dict) for v in rp.values()):
            rp = rp.get("full_attention") or next(iter(rp.values()))
        theta = rp.get("rope_theta")
        return (None if theta is None else float(theta)), dict(rp)
    theta = getattr(cfg, "rope_theta", None)
    return (None if theta is None else float(theta)), getattr(cfg, "rope_scaling", None)


def layer_rope_from_hf(hf_config) -> Optional[list[Optional[dict]]]:
    """Per-layer RoPE of models whose layers differ, from a HF config; None
    when every layer uses the model's one RoPE.

    * local / global attention layers with their own bases (Gemma 3):
      ``rope_parameters`` keyed by layer type, or ``rope_local_base_freq``
      (unscaled) for "sliding_attention" layers in ``layer_types``;
    * layers without RoPE (Llama 4: ``no_rope_layers[l] == 0``).
    """
    cfg = _text_config(hf_config)
    n = getattr(cfg, "num_hidden_layers", None)
    if not n:
        return None
    theta, scaling = model_rope_from_hf(hf_config)
    base = {"rope_theta": theta if theta is not None else 10000.0, "rope_scaling": scaling}
    specs: list[Optional[dict]] = [dict(base) for _ in range(n)]
    differs = False
    types = getattr(cfg, "layer_types", None)
    rp = getattr(cfg, "rope_parameters", None)
    per_type = isinstance(rp, dict) and rp and all(isinstance(v, dict) for v in rp.values())
    local = getattr(cfg, "rope_local_base_freq", None)
    if types:
        for l, t in enumerate(list(types)[:n]):
            if per_type and t in rp:
                spec = {"rope_theta": float(rp[t].get("rope_theta", base["rope_theta"])),
                        "rope_scaling": dict(rp[t])}
            elif t == "sliding_attention" and local is not None:
                spec = {"rope_theta": float(local), "rope_scaling": None}
            else:
                continue
            if spec != specs[l]:
                specs[l] = spec
                differs = True
    no_rope = getattr(cfg, "no_rope_layers", None)
    if no_rope:
        for l, use in enumerate(list(no_rope)[:n]):
            if not use:
                specs[l] = None
                differs = True
    if differs:
        # compared on 64 dims (a 2-dim probe has the frequency 1 for any base)
        inv = [None if sp is None else inv_freq_for(sp.get("rope_scaling"), 64, sp["rope_theta"])
               for sp in specs]
        if all(x is not None for x in inv) and all(np.array_equal(x, inv[0]) for x in inv):
            return None  # written per layer type, but the same everywhere
    return specs if differs else None


def delta_tables(
    deltas: Sequence[int],
    rot_dim: int,
    theta: float = 10000.0,
    inv_freq: Optional[np.ndarray] = None,
    device: Optional[torch.device] = None,
) -> torch.Tensor:
    """float32 ``[len(deltas), rot_dim/2, 2]`` of (cos, sin)(delta * inv_freq).

    Row r rotates a chunk whose tokens move by ``deltas[r]`` positions.
    """
    inv = rope_inv_freq(rot_dim, theta) if inv_freq is None else np.asarray(inv_freq, np.float64)
    if inv.shape != (rot_dim // 2,):
        raise ValueError("inv_freq must have rot_dim/2 entries")
    d = np.asarray(deltas, dtype=np.float64).reshape(-1, 1)
    ang = d * inv.reshape(1, -1)
    tab = np.stack([np.cos(ang), np.sin(ang)], axis=-1).astype(np.float32)
    t = torch.from_numpy(np.ascontiguousarray(tab))
    if device is None:
        return t
    device = torch.device(device)
    if device.type == "cuda":  # stream-ordered, without blocking the host
        if torch.cuda.is_current_stream_capturing():
            raise ValueError("delta tables cannot be built under graph capture (the copy "
                             "would replay from a reused pinned buffer): build them before")
        return t.pin_memory().to(device, non_blocking=True)
    return t.to(device)


def page_rope_index(
    num_pages_per_chunk: Sequence[int], deltas: Sequence[int]
) -> tuple[np.ndarray, list[int]]:
    """Per-page table index for chunks laid out back to back.

    Chunks with delta 0 map to -1 (bit-exact copy, no table). Returns the
    int32 per-page index and the list of distinct non-zero deltas, whose
    order is the table order.
    """
    uniq: dict[int, int] = {}
    out = []
    for n, dl in zip(num_pages_per_chunk, deltas):
        dl = int(dl)
        if dl == 0:
            idx = -1
        else:
            idx = uniq.setdefault(dl, len(uniq))
        out.extend([idx] * int(n))
    return np.asarray(out, dtype=np.int32), list(uniq.keys())
