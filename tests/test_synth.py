"""Synthetic benchmark geometries: exact sizes (config 1's N and P were
measured independently on the same definition)."""
import numpy as np
import pytest

from bevy_synth_amd import synth


def test_config1_sizes(oracle):
    c = synth.config1_coords()
    assert c.shape == (14648, 4) and c.dtype == np.int32
    nbr = oracle.build_neighbor_rows(oracle.OracleConfig(64, 64), c)
    assert int((nbr >= 0).sum()) == 261416
    # lexicographic, unique
    key = ((c[:, 1].astype(np.int64) * 64 + c[:, 2]) * 64 + c[:, 3])
    assert np.all(np.diff(key) > 0)


def test_config2_size():
    c = synth.config2_coords()
    assert 100_000 <= len(c) <= 140_000
    assert len(np.unique(c, axis=0)) == len(c)


@pytest.mark.slow
def test_config3_size():
    c = synth.config3_coords()
    assert len(c) == 1_040_679
    assert c[:, 1:].max() < 256 and c.min() >= 0


def test_bf16_bits_match_oracle(oracle):
    x = np.random.default_rng(1).standard_normal(4096).astype(np.float32)
    assert np.array_equal(synth.bf16_to_f32(synth.bf16_bits(x)), oracle.bf16_round(x))


def test_config4_mask_selects_near_surface_children():
    g = synth.ShellCubeGeometry()
    parents = g.coords()[:5000]
    m = synth.subdivision_mask_near_surface(parents, g)
    assert m.shape == (5000, 8)
    frac = m.mean()
    assert 0.2 < frac < 0.95
