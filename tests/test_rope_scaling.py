"""RoPE frequency scalings against transformers' reference implementations
(modeling_rope_utils), and the rejection of sequence-length dependent ones."""

import numpy as np
import pytest

from daser_amd import position

transformers = pytest.importorskip("transformers")
from transformers import LlamaConfig  # noqa: E402
from transformers import modeling_rope_utils as mru  # noqa: E402


def _cfg(theta, scaling, max_pos=131072):
    return LlamaConfig(hidden_size=4096, num_attention_heads=32, num_key_value_heads=8,
                       max_position_embeddings=max_pos, rope_theta=theta, rope_scaling=scaling)


@pytest.mark.parametrize("scaling,fn", [
    ({"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
      "original_max_position_embeddings": 8192}, "_compute_llama3_parameters"),
    ({"rope_type": "yarn", "factor": 4.0, "original_max_position_embeddings": 8192},
     "_compute_yarn_parameters"),
    ({"rope_type": "yarn", "factor": 16.0, "original_max_position_embeddings": 4096,
      "beta_fast": 16.0, "beta_slow": 2.0}, "_compute_yarn_parameters"),
    ({"rope_type": "linear", "factor": 2.0}, "_compute_linear_scaling_rope_parameters"),
])
@pytest.mark.parametrize("theta", [10000.0, 500000.0])
def test_matches_transformers(scaling, fn, theta):
    ref, _ = getattr(mru, fn)(_cfg(theta, dict(scaling)), device="cpu")  # it edits the dict
    ours = position.inv_freq_for(scaling, 128, theta)
    np.testing.assert_allclose(ours, ref.double().numpy(), rtol=2e-6)


def test_default_and_none():
    np.testing.assert_array_equal(position.inv_freq_for(None, 64, 1e4),
                                  position.rope_inv_freq(64, 1e4))
    np.testing.assert_array_equal(position.inv_freq_for({"rope_type": "default"}, 64, 1e4),
                                  position.rope_inv_freq(64, 1e4))


@pytest.mark.parametrize("kind", ["dynamic", "longrope"])
def test_sequence_length_dependent_scalings_rejected(kind):
    with pytest.raises(ValueError, match="sequence length"):
        position.inv_freq_for({"rope_type": kind, "factor": 2.0}, 128, 1e4)


def test_data_plane_takes_scaling(tmp_path):
    from daser_amd.connector import KVDataPlane

    sc = {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0,
          "high_freq_factor": 4.0, "original_max_position_embeddings": 8192}
    p = KVDataPlane(str(tmp_path / "s"), rope_theta=5e5, rotary_dim=128, rope_scaling=sc)
    np.testing.assert_array_equal(p.inv_freq, position.inv_freq_for(sc, 128, 5e5))
    with pytest.raises(ValueError, match="sequence length"):
        KVDataPlane(str(tmp_path / "s"), rope_scaling={"rope_type": "dynamic", "factor": 2.0})


def test_mrope_uses_plain_frequencies():
    """Qwen2-VL's M-RoPE: three position components over sections of the
    rotary dims, plain frequencies; a chunk moved by d shifts every
    component by d, which is one rotation by d on every pair."""
    sc = {"type": "mrope", "mrope_section": [16, 24, 24]}
    np.testing.assert_array_equal(position.inv_freq_for(sc, 128, 1e6),
                                  position.rope_inv_freq(128, 1e6))
    # the composed rotation of the three sections at positions (p+d, p+d, p+d)
    # after (p, p, p) equals the rotation by d
    inv = position.rope_inv_freq(128, 1e6)
    bounds = np.cumsum([0] + sc["mrope_section"])
    p, d = np.array([7, 3, 11]), 250
    ang_before = np.concatenate([p[i] * inv[bounds[i]:bounds[i + 1]] for i in range(3)])
    ang_after = np.concatenate([(p[i] + d) * inv[bounds[i]:bounds[i + 1]] for i in range(3)])
    np.testing.assert_allclose(ang_after - ang_before, d * inv, rtol=1e-12)


def test_per_layer_rope_from_hf_configs():
    """Gemma 3 (local / global bases) and Llama 4 (layers without RoPE) give
    layer groups; a plain Llama config gives none."""
    from transformers import Gemma3TextConfig, Llama4TextConfig

    specs = position.layer_rope_from_hf(Gemma3TextConfig(num_hidden_layers=12))
    groups, invs = position.layer_rope_groups(specs, 256)
    assert groups.tolist() == [0, 0, 0, 0, 0, 1] * 2
    np.testing.assert_allclose(invs[0], position.rope_inv_freq(256, 10000.0))
    np.testing.assert_allclose(invs[1], position.rope_inv_freq(256, 1e6))
    specs = position.layer_rope_from_hf(Llama4TextConfig(num_hidden_layers=8))
    groups, invs = position.layer_rope_groups(specs, 128)
    assert groups.tolist() == [0, 0, 0, -1, 0, 0, 0, -1] and len(invs) == 1
    assert position.layer_rope_from_hf(_cfg(5e5, None, 8192)) is None
    assert position.model_rope_from_hf(_cfg(5e5, None, 8192))[0] == 5e5


def test_data_plane_layer_groups(tmp_path):
    """Registered layers are mapped to model layers by their names; a
    per-layer list with one RoPE collapses to the single-table path."""
    import torch

    from daser_amd.connector import KVDataPlane

    caches = {f"model.layers.{i}.self_attn.attn": torch.zeros(2, 4, 16, 1, 64,
                                                              dtype=torch.bfloat16)
              for i in (0, 1, 2, 3)}
    rope = [{"rope_theta": 1e4}, None, {"rope_theta": 1e6}, {"rope_theta": 1e4}]
    p = KVDataPlane(str(tmp_path / "s"), io_backend="python", layer_rope=rope)
    p.register(caches)
    assert p._layer_group.tolist() == [0, -1, 1, 0]
    p.close()
    same = [{"rope_theta": 5e5}] * 4
    q = KVDataPlane(str(tmp_path / "t"), io_backend="python", layer_rope=same)
    q.register(caches)
    assert q._layer_group is None
    np.testing.assert_array_equal(q.inv_freq, position.rope_inv_freq(64, 5e5))
    q.close()
    r = KVDataPlane(str(tmp_path / "u"), io_backend="python", layer_rope=rope[:2])
    with pytest.raises(ValueError, match="no entry for layer 2"):
        r.register(caches)


def test_connector_reads_rope_from_model_config(tmp_path):
    from types import SimpleNamespace

    from daser_amd import connector as C

    hf = _cfg(5e5, {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0,
                    "high_freq_factor": 4.0, "original_max_position_embeddings": 8192}, 131072)
    cfg = SimpleNamespace(
        model_config=SimpleNamespace(hf_config=hf),
        kv_transfer_config=SimpleNamespace(kv_connector_extra_config=dict(
            store_path=str(tmp_path / "s"), io_backend="python")))
    w = C.DaserConnector(cfg, C.KVConnectorRole.WORKER, ipc_async=object())
    assert w._plane.rope_theta == 5e5
    assert w._plane.rope_scaling["rope_type"] == "llama3"
    w.shutdown()
