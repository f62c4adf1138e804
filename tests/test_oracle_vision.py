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


# ---- closed forms of the whole tower (vision.rs:742-959) -----------------------------
#
# Two degenerate weight sets reduce the forward pass to formulas that need no
# attention softmax and no RoPE, so they pin the composition independently of
# any restatement of the layer loop. Each comparison is shown to fail when a
# plausible mistake is planted in the closed form.

L_ = "vision_tower.encoder.layers.{}."
W_IN = "vision_tower.patch_embedder.input_proj.weight"
TABLE = "vision_tower.patch_embedder.position_embedding_table"
W_OUT = "embed_vision.embedding_projection.weight"


def _config(kind):
    return small_vision_config(2) if kind == "small" else svl_synth.config_v(2)


def _soft_closed_form(vc, w, h, pos, grid, soft, mistake=None):
    """pool_patches (vision.rs:980-1040: per 3x3 bin, sum / 9 * sqrt(H)),
    unscaled RMSNorm, embedding projection (vision.rs:937-946), in float64."""
    gw, _ = grid
    H = h.shape[1]
    pooled = np.zeros((soft, H))
    for i in range(h.shape[0]):
        pooled[pos[i, 0] // 3 + (gw // 3) * (pos[i, 1] // 3)] += h[i]
    div = 1.0 if mistake == "pool_no_div9" else 9.0
    mul = 1.0 if mistake == "pool_no_sqrt_h" else np.sqrt(H)
    pooled = pooled / div * mul
    return ref64.rms(pooled, None, vc["rms_norm_eps"]) @ w[W_OUT].astype(np.float64).T


def _embedding_closed_form(w, pix, pos, mistake=None):
    """hidden_0 = 2 (x - 0.5) W_in^T + table[0][x] + table[1][y] (vision.rs:760-809)."""
    x = pix.astype(np.float64)
    x = x if mistake == "no_rescale" else 2.0 * (x - 0.5)
    t = w[TABLE].astype(np.float64)
    xs, ys = (pos[:, 1], pos[:, 0]) if mistake == "xy_swap" else (pos[:, 0], pos[:, 1])
    return x @ w[W_IN].astype(np.float64).T + t[0][xs] + t[1][ys]


def _rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / np.abs(b).max())


@pytest.mark.parametrize("kind", ["small", "config_v"])
def test_zero_projections_reduce_the_tower_to_its_embedding_and_pooling(kind):
    """With every q/k/v/o and gate/up/down weight zero, each layer adds
    RMSNorm(0) = 0 twice, so every hidden state equals the patch embedding bit
    for bit, and the soft tokens are the closed form of the embedding, the
    3x3 pooling, the unscaled norm and the projection. The embedding is scaled
    so the pooled rows' mean square is near eps: the norm then sees the pool's
    1/9 and sqrt(H) factors too."""
    c = _config(kind)
    vc = oracle.resolve_vision_config(c)
    H, L = vc["hidden_size"], vc["num_hidden_layers"]
    w = dict(svl_synth.vision_weights(c, 48, seed=21))
    for l in range(L):
        for n in ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
                  "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj"):
            k = L_.format(l) + n + ".linear.weight"
            w[k] = np.zeros_like(w[k])
    s = np.float32(3e-3 / np.sqrt(H))
    w[W_IN] = (w[W_IN] * s).astype(np.float32)
    w[TABLE] = (w[TABLE] * s).astype(np.float32)
    p = grid_patches(6, 9, seed=3)
    out = oracle.OracleVisionModel(c, w, 48).forward(p, capture_hidden=True)
    hs = out["hidden_states"]
    for l in range(1, L + 1):
        assert np.array_equal(hs[l], hs[0]), f"layer {l} is not the identity"
    h0 = _embedding_closed_form(w, p.pixel_values, p.positions)
    assert _rel(hs[0], h0) <= 1e-5
    want = _soft_closed_form(vc, w, h0, p.positions, p.patch_grid, p.soft_tokens)
    ms = (np.asarray(want) ** 2).mean()
    assert _rel(out["pooled"], want) <= 1e-4, (ms, _rel(out["pooled"], want))
    for mistake in ("xy_swap", "no_rescale"):
        bad = _soft_closed_form(vc, w, _embedding_closed_form(w, p.pixel_values, p.positions,
                                                              mistake),
                                p.positions, p.patch_grid, p.soft_tokens)
        assert _rel(out["pooled"], bad) > 1e-2, mistake
    for mistake in ("pool_no_div9", "pool_no_sqrt_h"):
        bad = _soft_closed_form(vc, w, h0, p.positions, p.patch_grid, p.soft_tokens, mistake)
        assert _rel(out["pooled"], bad) > 1e-2, mistake


def _layer_one_row(vc, w, l, h, mistake=None):
    """One encoder layer (vision.rs:816-935) on a hidden state whose rows are
    all equal: every key's value row is the same, so attention returns it
    whatever the softmax weights (sum_j p_j v = v) and RoPE drops out."""
    NH, NKV, hd, eps = (vc["num_attention_heads"], vc["num_key_value_heads"], vc["head_dim"],
                        vc["rms_norm_eps"])
    p = L_.format(l)
    f64 = lambda n: w[p + n].astype(np.float64)
    n = ref64.rms(h, w[p + "input_layernorm.weight"], eps)
    v = (n @ f64("self_attn.v_proj.linear.weight").T).reshape(NKV, hd)
    v = ref64.rms(v, w[p + "self_attn.k_norm.weight"] if mistake == "scaled_v_norm" else None, eps)
    attn = np.concatenate([v[hh // (NH // NKV)] for hh in range(NH)])
    o = attn @ f64("self_attn.o_proj.linear.weight").T
    h = h + (o if mistake == "no_post_attention_norm" else
             ref64.rms(o, w[p + "post_attention_layernorm.weight"], eps))
    n = ref64.rms(h, w[p + "pre_feedforward_layernorm.weight"], eps)
    g = n @ f64("mlp.gate_proj.linear.weight").T
    u = n @ f64("mlp.up_proj.linear.weight").T
    act = ref64.gelu(u) * g if mistake == "gate_up_swapped" else ref64.gelu(g) * u
    return h + ref64.rms(act @ f64("mlp.down_proj.linear.weight").T,
                         w[p + "post_feedforward_layernorm.weight"], eps)


@pytest.mark.parametrize("kind", ["small", "config_v"])
def test_identical_patches_reduce_attention_to_the_value_row(kind):
    """Identical patches and a zero position table make every row of every
    hidden state equal, so each layer is the closed form of one row: the
    unscaled V norm, the O projection, the sandwich norms, GeGLU and both
    residuals (planted: a weighted V norm, a missing post-attention norm,
    gate and up swapped)."""
    c = _config(kind)
    vc = oracle.resolve_vision_config(c)
    L = vc["num_hidden_layers"]
    w = dict(svl_synth.vision_weights(c, 48, seed=22))
    w[TABLE] = np.zeros_like(w[TABLE])
    p = grid_patches(6, 6, seed=4)
    p.pixel_values[:] = p.pixel_values[0]
    out = oracle.OracleVisionModel(c, w, 48).forward(p, capture_hidden=True)
    hs = out["hidden_states"]
    h = _embedding_closed_form(w, p.pixel_values[:1], p.positions[:1])[0]
    assert _rel(hs[0], np.broadcast_to(h, hs[0].shape)) <= 1e-5
    for l in range(L):
        prev = h
        h = _layer_one_row(vc, w, l, prev)
        e = _rel(hs[l + 1], np.broadcast_to(h, hs[l + 1].shape))
        assert e <= 1e-4, f"layer {l + 1}: {e}"
        for mistake in ("scaled_v_norm", "no_post_attention_norm", "gate_up_swapped"):
            bad = _layer_one_row(vc, w, l, prev, mistake)
            assert _rel(hs[l + 1], np.broadcast_to(bad, hs[l + 1].shape)) > 1e-3, \
                (l, mistake)
    want = _soft_closed_form(vc, w, np.broadcast_to(h, hs[L].shape), p.positions,
                             p.patch_grid, p.soft_tokens)
    assert _rel(out["pooled"], want) <= 1e-4
