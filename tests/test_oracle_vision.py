"""Pins of the vision-tower oracle (oracle/svl_oracle_vision.c).

No offline golden exists for the vision tower: the reference's image golden
(fixtures/model/image_golden.json) needs the full released weights, which are
absent. The oracle is therefore pinned by
  * the known-answer tests of src/model/vision.rs:1154-1182 (axial RoPE),
  * closed forms and invariants (rotation norms, identity at the origin, the
    3x3 bin average),
  * an independent float64 numpy restatement of VisionModel::forward
    (tests/ref64.py) on small random models, with a planted axis swap to
    show the comparison can tell the x and y halves apart.
"""
import numpy as np
import pytest

from oracle import oracle
import ref64
import svl_synth


def small_vision_config(layers=2):
    c = svl_synth.config_v(layers)
    c["vision_config"].update(hidden_size=64, intermediate_size=96, num_attention_heads=4,
                              num_key_value_heads=2, head_dim=16, position_embedding_size=16)
    return c


class _Patches:
    def __init__(self, pix, pos, valid, soft, max_patches, grid):
        self.pixel_values, self.positions = pix, pos
        self.valid_patches, self.soft_tokens = valid, soft
        self.max_patches, self.patch_grid = max_patches, grid


def grid_patches(gw, gh, seed=0, max_patches=None):
    rng = np.random.default_rng(seed)
    valid = gw * gh
    mp = max_patches or valid
    pix = np.zeros((mp, 768), np.float32)
    pix[:valid] = rng.integers(0, 256, (valid, 768)).astype(np.float32) * (np.float32(1) / np.float32(255))
    pos = np.full((mp, 2), -1, np.int32)
    ys, xs = np.divmod(np.arange(valid), gw)
    pos[:valid, 0], pos[:valid, 1] = xs, ys
    return _Patches(pix, pos, valid, valid // 9, mp, (gw, gh))


# ---- vision.rs:1154-1182 known answers ------------------------------------------

def test_axial_frequencies_match_the_reference_layout():
    f = oracle.axial_inv_freq(64, 100.0)
    assert len(f) == 16
    assert abs(f[0] - 1.0) <= 1e-6
    assert abs(f[15] - np.float32(1.0) / np.float32(100.0) ** np.float32(30.0 / 32.0)) <= 1e-6


def test_axial_rope_rotates_the_x_and_y_halves():
    f = oracle.axial_inv_freq(4, 100.0)
    assert f.tolist() == [1.0]
    v = oracle.axial_rope(np.array([1, 0, 1, 0], np.float32), 1, 1, 4, [[1, 0]], f)
    assert abs(v[0] - np.cos(np.float32(1.0))) <= 1e-6
    assert abs(v[1] - np.sin(np.float32(1.0))) <= 1e-6
    assert abs(v[2] - 1.0) <= 1e-6
    assert abs(v[3] - 0.0) <= 1e-6


def test_axial_rope_rejects_a_non_divisible_head_dimension():
    with pytest.raises(oracle.OracleError) as e:
        oracle.axial_inv_freq(6, 100.0)
    assert e.value.status == 7
    with pytest.raises(oracle.OracleError) as e:
        oracle.axial_rope(np.zeros(6, np.float32), 1, 1, 6, [[0, 0]], np.ones(1, np.float32))
    assert e.value.status == 7


# ---- closed forms -----------------------------------------------------------------

def test_axial_rope_matches_a_float64_rotation():
    rng = np.random.default_rng(3)
    seq, heads, hd = 11, 3, 24
    x = rng.standard_normal((seq, heads, hd)).astype(np.float32)
    pos = rng.integers(0, 40, (seq, 2)).astype(np.int32)
    inv = oracle.axial_inv_freq(hd, 100.0)
    got = oracle.axial_rope(x, seq, heads, hd, pos, inv).reshape(seq, heads, hd)
    want = ref64.axial_rope64(x, pos, inv)
    np.testing.assert_allclose(got, want, atol=2e-5)
    # each rotated pair keeps its length
    q = hd // 4
    for hf in (0, 1):
        a, b = slice(hf * 2 * q, hf * 2 * q + q), slice(hf * 2 * q + q, (hf + 1) * 2 * q)
        n0 = x[..., a].astype(np.float64) ** 2 + x[..., b].astype(np.float64) ** 2
        n1 = got[..., a].astype(np.float64) ** 2 + got[..., b].astype(np.float64) ** 2
        np.testing.assert_allclose(n1, n0, rtol=1e-5, atol=1e-6)


def test_axial_rope_is_the_identity_at_the_origin_and_axis_local():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((2, 2, 16)).astype(np.float32)
    inv = oracle.axial_inv_freq(16, 100.0)
    same = oracle.axial_rope(x, 2, 2, 16, [[0, 0], [0, 0]], inv).reshape(x.shape)
    np.testing.assert_array_equal(same, x)
    only_x = oracle.axial_rope(x, 2, 2, 16, [[5, 0], [7, 0]], inv).reshape(x.shape)
    np.testing.assert_array_equal(only_x[..., 8:], x[..., 8:])
    assert np.abs(only_x[..., :8] - x[..., :8]).max() > 1e-2
    only_y = oracle.axial_rope(x, 2, 2, 16, [[0, 3], [0, 9]], inv).reshape(x.shape)
    np.testing.assert_array_equal(only_y[..., :8], x[..., :8])


def test_pool_patches_is_the_scaled_bin_average():
    rng = np.random.default_rng(5)
    gw, gh, H = 9, 6, 40
    p = grid_patches(gw, gh)
    h = rng.standard_normal((gw * gh, H)).astype(np.float32)
    got = oracle.pool_patches(h, p.positions[: gw * gh], gw * gh, gw, gh, 6, H).reshape(6, H)
    want = ref64.pool_patches64(h.astype(np.float64), p.positions[: gw * gh], gw, gh, 6)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)
    # bin 0 holds patches (0..2, 0..2)
    idx = [y * gw + x for y in range(3) for x in range(3)]
    np.testing.assert_allclose(got[0], h[idx].astype(np.float64).mean(0) * np.sqrt(H), rtol=1e-5)


@pytest.mark.parametrize("grid,soft", [((8, 6), 4), ((9, 6), 5)])
def test_pool_patches_rejects_an_inconsistent_geometry(grid, soft):
    p = grid_patches(9, 6)
    with pytest.raises(oracle.OracleError) as e:
        oracle.pool_patches(np.zeros((54, 8), np.float32), p.positions, 54, grid[0], grid[1],
                            soft, 8)
    assert e.value.status == 7


# ---- the whole tower vs the float64 restatement ---------------------------------------

@pytest.fixture(scope="module")
def small_tower():
    c = small_vision_config()
    w = svl_synth.vision_weights(c, 48, seed=7)
    return c, w, oracle.OracleVisionModel(c, w, 48)


def test_vision_forward_matches_float64(small_tower):
    c, w, m = small_tower
    p = grid_patches(6, 9, seed=1, max_patches=63)  # 54 real patches + 9 padding rows
    got = m.forward(p, capture_hidden=True)
    want = ref64.vision_forward64(oracle.resolve_vision_config(c), w, p.pixel_values[:54],
                                  p.positions[:54], p.patch_grid, p.soft_tokens)
    assert got["pooled"].shape == (6, 48)
    np.testing.assert_allclose(got["hidden_states"], want["hidden_states"], rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(got["pooled"], want["pooled"], rtol=1e-4, atol=5e-5)


def test_vision_forward_comparison_sees_the_axis_assignment(small_tower):
    c, w, m = small_tower
    p = grid_patches(6, 9, seed=1)
    got = m.forward(p)["pooled"]
    swapped = ref64.vision_forward64(oracle.resolve_vision_config(c), w, p.pixel_values,
                                     p.positions, p.patch_grid, p.soft_tokens, swap_axes=True)
    assert np.abs(got - swapped["pooled"]).max() > 1e-3


def test_vision_forward_error_taxonomy(small_tower):
    c, w, m = small_tower
    p = grid_patches(6, 6)
    zero = _Patches(p.pixel_values, p.positions, 0, 4, 36, (6, 6))
    with pytest.raises(oracle.OracleError) as e:
        m.forward(zero)
    assert e.value.status == 4
    far = grid_patches(6, 6)
    far.positions[3] = [16, 0]  # table has 16 entries per axis
    with pytest.raises(oracle.OracleError) as e:
        m.forward(far)
    assert e.value.status == 4
    neg = grid_patches(6, 6)
    neg.positions[2] = [-1, 0]
    with pytest.raises(oracle.OracleError) as e:
        m.forward(neg)
    assert e.value.status == 7
    odd = grid_patches(6, 6)
    odd.patch_grid = (4, 9)
    with pytest.raises(oracle.OracleError) as e:
        m.forward(odd)
    assert e.value.status == 7
