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
