"""Pins of the oracle's 1-D parameter wiring by closed forms.

The official fixtures hold constants in every 1-D tensor (all text norms and
layer scalars are 1.0; the audio norms are 1.0, per_dim_scale 0, the output
bias 0 and every clipping bound +-20), so they cannot see which norm weight,
scalar or bound goes where. Here degenerate weight sets reduce the forward
pass to short formulas (tests/closed_forms.py) that need no restatement of
the layer loop, with random 1-D weights, and every comparison is shown to
fail for planted wiring mistakes:

* text (text.rs:182-538): zero projections make each layer the layer_scalar
  multiply (bit for bit); a row of one repeated token makes each layer a
  one-row closed form of every norm, the PLE gate and the scalar's place; two
  tokens make attention a two-way logistic that fixes q_norm / k_norm, RoPE
  and the GQA head map;
* vision (vision.rs:816-935): two patches fix q_norm / k_norm and axial RoPE
  through the oracle's single-layer entry point, which composes to the
  forward pass bit for bit;
* audio (audio.rs:981-1134, 1136-1322): zero projections leave norm_out; one
  live branch at a time, with distinct binding clip bounds per linear and a
  binding gradient clip, fixes each branch's norms and bounds; identical rows
  and two rows fix the attention block; the output bias by the tail's closed
  form; the subsampling LayerNorm weights by their equivalence with scaling
  the next layer's input channels.
"""
import json
import math
import os

import numpy as np
import pytest

import closed_forms as CF
import svl_synth
from oracle import oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
TOL = 1e-4      # closed form (float64) against the float32 oracle, relative
SEEN = 1e-3     # a planted mistake must move the comparison by more than this


# ---- text --------------------------------------------------------------------------

def text_config(kind, layers):
    types = ["sliding_attention"] * (layers - 1) + ["full_attention"]
    if kind == "shape_a":
        return svl_synth.config_a(layers, vocab=512)
    c = json.load(open(os.path.join(HERE, "golden", "tiny_text", "config.json")))
    c.update(num_hidden_layers=layers, layer_types=types)
    if kind == "tiny":
        c["per_layer_config"] = {str(layers - 1): {"head_dim": 16, "num_key_value_heads": 1}}
    else:  # "gqa": 4 query heads over 2 KV heads
        c.update(hidden_size=32, intermediate_size=48, num_attention_heads=4,
                 num_key_value_heads=2, head_dim=8)
        c["per_layer_config"] = {}
    return c


def text_model(kind, layers, seed):
    """Synthetic weights with random norm weights U(0.5, 1.5), layer scalars
    U(0.5, 1.0) and, below head_dim 64, q/k norms U(0.6, 1.4) so the two-key
    scores are of order one."""
    c = text_config(kind, layers)
    w = dict(svl_synth.weights(c, seed=seed))
    rng = np.random.default_rng(seed)
    rc = O.resolve_config(c)
    for k, a in w.items():
        if a.ndim != 1:
            continue
        if k.endswith("layer_scalar"):
            w[k] = rng.uniform(0.5, 1.0, a.shape).astype(np.float32)
        elif k.endswith(("q_norm.weight", "k_norm.weight")):
            if a.size < 64:
                w[k] = rng.uniform(0.6, 1.4, a.shape).astype(np.float32)
        else:
            w[k] = rng.uniform(0.5, 1.5, a.shape).astype(np.float32)
    return c, rc, w


def max_rel(states, want):
    return max(CF.rel(s, np.broadcast_to(x, s.shape)) for s, x in zip(states, want))


@pytest.mark.parametrize("kind", ["tiny", "shape_a"])
def test_text_zero_projections_reduce_each_layer_to_its_scalar(kind):
    """With q/k/v/o, gate/up/down, the PLE gate and the PLE projection zero,
    every branch adds RMSNorm(0) = 0: hidden_l = hidden_{l-1} * layer_scalar_l
    bit for bit, from the gather times sqrt(H); the head is the final norm
    with its own weight, the projection and the pool."""
    c, rc, w = text_model(kind, 4, seed=31)
    L = rc["num_hidden_layers"]
    w = CF.zero_text(w, L)
    ids = np.random.default_rng(1).integers(0, rc["vocab_size"], 9)
    out = O.OracleTextModel(c, w).forward(ids.tolist(), capture_hidden=True)
    hs = out["hidden_states"]
    want = CF.text_zero_projection_states(w, rc, ids)
    for l in range(L + 1):
        assert np.array_equal(hs[l], want[l]), f"hidden state {l}"
    for mistake in ("no_embedding_scale", "no_layer_scalar", "scalars_reversed"):
        assert max_rel(hs, CF.text_zero_projection_states(w, rc, ids, mistake)) > SEEN, mistake
    head = CF.text_head(w, rc, hs[L])
    assert CF.rel(out["projected"], head["projected"]) <= 1e-5
    assert np.abs(out["normalized"] - head["normalized"]).max() <= 1e-6
    for mistake in ("final_norm_is_input_layernorm", "final_norm_reversed", "no_final_norm"):
        assert CF.rel(out["projected"], CF.text_head(w, rc, hs[L], mistake)["projected"]) > SEEN


TEXT_ROW_MISTAKES = ("attention_norms_swapped", "ffn_norms_swapped", "ple_norm_is_post_ffn",
                     "scaled_v_norm", "ple_gate_on_normalised_hidden", "ple_slices_reversed",
                     "scalar_before_ple_residual", "no_ple_scale")


def small_ple_projection(w, rc):
    """Scale the PLE model projection so its output's mean square is near
    eps, and each layer's PLE projection so its output's is too: a factor on
    the per-layer inputs (the 1/sqrt(H) scale) then survives both the segment
    norm and the post-PLE norm instead of cancelling in them."""
    w = dict(w)
    eps = rc["rms_norm_eps"]
    s = math.sqrt(eps * rc["hidden_size"])
    w[CF.PLE_MODEL] = (w[CF.PLE_MODEL] * np.float32(s)).astype(np.float32)
    for l in range(rc["num_hidden_layers"]):
        k = CF.TL.format(l) + "ple_block.per_layer_projection.weight"
        w[k] = (w[k] * np.float32(3.0 * math.sqrt(eps))).astype(np.float32)
    return w


@pytest.mark.parametrize("kind", ["tiny", "gqa", "shape_a"])
def test_text_identical_tokens_reduce_each_layer_to_one_row(kind):
    """A row repeating one token keeps every hidden row equal, so attention
    returns the value row and each layer is a one-row closed form of every
    norm weight, the PLE block and layer_scalar (text.rs:345-513)."""
    c, rc, w = text_model(kind, 4, seed=32)
    w = small_ple_projection(w, rc)
    L = rc["num_hidden_layers"]
    m = O.OracleTextModel(c, w)
    for tok, n in ((7, 6), (rc["vocab_size"] - 3, 5)):
        out = m.forward([tok] * n, capture_hidden=True)
        hs = out["hidden_states"]
        want = CF.text_identical_token_states(w, rc, tok)
        e = max_rel(hs, want)
        assert e <= TOL, e
        head = CF.text_head(w, rc, np.broadcast_to(want[L], hs[L].shape))
        assert np.abs(out["normalized"] - head["normalized"]).max() <= 1e-5
        for mistake in TEXT_ROW_MISTAKES:
            bad = max_rel(hs, CF.text_identical_token_states(w, rc, tok, mistake))
            assert bad > SEEN, (mistake, bad)


@pytest.mark.parametrize("kind", ["tiny", "gqa", "shape_a"])
def test_text_two_token_attention_pins_the_query_key_side(kind):
    """Two tokens through a sliding and a full layer whose feed-forward and
    PLE gate weights are zero: attention is a two-way logistic of the score
    difference, which fixes q_norm / k_norm, rotate-half RoPE at positions 0
    and 1 with each layer type's theta, the GQA head map and scale 1.0
    (text.rs:345-433, kernels.rs:936-1135)."""
    c, rc, w = text_model(kind, 2, seed=33)
    w = CF.zero_text(w, 2, names=("mlp.gate_proj.weight", "mlp.up_proj.weight",
                                  "mlp.down_proj.weight", "ple_block.per_layer_input_gate.weight"))
    m = O.OracleTextModel(c, w)
    mistakes = ["qk_norms_swapped", "no_k_norm_weight", "rope_before_norm", "no_rope",
                "rope_pairs_interleaved", "theta_swapped", "scores_scaled"]
    if kind == "gqa":
        mistakes.append("gqa_heads_interleaved")
    rng = np.random.default_rng(5)
    errs, bad = [], {k: 0.0 for k in mistakes}
    for _ in range(4):
        ids = rng.choice(rc["vocab_size"], 2, replace=False).tolist()
        hs = m.forward(ids, capture_hidden=True)["hidden_states"]
        errs.append(max_rel(hs, CF.text_two_token_states(w, rc, ids)))
        for k in mistakes:
            bad[k] = max(bad[k], max_rel(hs, CF.text_two_token_states(w, rc, ids, k)))
    assert max(errs) <= TOL, errs
    for k, e in bad.items():
        assert e > SEEN, (k, e)


# ---- vision ------------------------------------------------------------------------

def vision_model(kind, layers, seed):
    c = svl_synth.config_v(layers)
    if kind == "small":
        c["vision_config"].update(hidden_size=64, intermediate_size=96, num_attention_heads=4,
                                  num_key_value_heads=2, head_dim=16, position_embedding_size=16)
    w = dict(svl_synth.vision_weights(c, 48, seed=seed))
    rng = np.random.default_rng(seed)
    vc = O.resolve_vision_config(c)
    for k, a in w.items():
        if a.ndim == 1 and k.endswith(("q_norm.weight", "k_norm.weight")):
            if vc["head_dim"] < 64:
                w[k] = rng.uniform(0.6, 1.4, a.shape).astype(np.float32)
        elif a.ndim == 1:
            w[k] = rng.uniform(0.5, 1.5, a.shape).astype(np.float32)
    return c, vc, w


def test_vision_single_layer_path_composes_to_the_forward_pass():
    """OracleVisionModel.layer runs the forward pass's own per-layer code:
    chaining it from the patch embedding reproduces every hidden state bit
    for bit."""
    import test_oracle_vision as TV
    c, vc, w = vision_model("small", 3, seed=41)
    om = O.OracleVisionModel(c, w, 48)
    p = TV.grid_patches(6, 6, seed=8)
    ref = om.forward(p, capture_hidden=True)
    h = ref["hidden_states"][0]
    for l in range(3):
        h = om.layer(l, h, p.positions[:36])
        assert np.array_equal(h, ref["hidden_states"][l + 1]), f"layer {l}"
    with pytest.raises(O.OracleError):
        om.layer(3, h, p.positions[:36])
    with pytest.raises(O.OracleError):
        om.layer(0, h[:2], np.array([[0, -1], [1, 1]]))


@pytest.mark.parametrize("kind", ["small", "config_v"])
def test_vision_two_patch_attention_pins_the_query_key_side(kind):
    """Two patches through a layer whose feed-forward weights are zero: the
    attention is a two-way logistic that fixes q_norm / k_norm, axial RoPE by
    (x, y) and scale 1.0 (vision.rs:816-878, 1073-1148)."""
    c, vc, w = vision_model(kind, 1, seed=42)
    for n in CF.V_FFN:
        w[CF.VL.format(0) + n] = np.zeros_like(w[CF.VL.format(0) + n])
    om = O.OracleVisionModel(c, w, 48)
    rng = np.random.default_rng(6)
    mistakes = ("xy_swapped", "qk_norms_swapped", "rope_before_norm", "text_rope",
                "no_key_rope", "scores_scaled")
    errs, bad = [], {k: 0.0 for k in mistakes}
    for pos in ([[0, 0], [1, 2]], [[3, 1], [5, 7]], [[10, 4], [2, 9]]):
        h = rng.standard_normal((2, vc["hidden_size"])).astype(np.float32)
        got = om.layer(0, h, pos)
        errs.append(CF.rel(got, CF.vision_two_patch_layer(w, vc, 0, h, pos)))
        for k in mistakes:
            bad[k] = max(bad[k], CF.rel(got, CF.vision_two_patch_layer(w, vc, 0, h, pos, k)))
    assert max(errs) <= TOL, errs
    for k, e in bad.items():
        assert e > SEEN, (k, e)


# ---- audio -------------------------------------------------------------------------

def audio_model(kind, layers, seed, clip=1.25):
    """Synthetic weights with random norm weights U(0.5, 1.5), per_dim_scale
    U(-1, 1) and output bias U(-0.5, 0.5); `clip` is the gradient clipping
    (1e10 in the frozen model, binding here so its wiring shows)."""
    if kind == "tiny":
        c = json.load(open(os.path.join(HERE, "golden", "tiny_audio", "config.json")))
        c["audio_config"]["num_hidden_layers"] = layers
        th = c["text_config"]["hidden_size"]
    else:
        c = svl_synth.config_au(layers)
        th = 48
    c["audio_config"]["gradient_clipping"] = clip
    w = dict(svl_synth.audio_weights(c, th, seed=seed))
    rng = np.random.default_rng(seed)
    for k, a in w.items():
        if k.endswith("per_dim_scale"):
            w[k] = rng.uniform(-1.0, 1.0, a.shape).astype(np.float32)
        elif k.endswith("output_proj.bias"):
            w[k] = rng.uniform(-0.5, 0.5, a.shape).astype(np.float32)
        elif a.ndim == 1 and a.size > 1:
            w[k] = rng.uniform(0.5, 1.5, a.shape).astype(np.float32)
    return c, O.resolve_audio_config(c), w, th


def _hidden(rows, H, seed, scale=1.5):
    return (np.random.default_rng(seed).standard_normal((rows, H)) * scale).astype(np.float32)


@pytest.mark.parametrize("kind", ["tiny", "au"])
def test_audio_zero_projections_leave_the_output_norm_and_the_tail(kind):
    """Every clipped linear zero (bounds distinct and binding): each branch
    adds 0, so a layer is RMSNorm(hidden, norm_out) and the tower's soft
    tokens are the tail's closed form with the output bias (audio.rs:1074-1133)."""
    c, ac, w0, th = audio_model(kind, 2, seed=51)
    w = CF.audio_degenerate(w0, 2, keep=(), seed=1)
    om = O.OracleAudioModel(c, w, th)
    h = _hidden(7, ac["hidden_size"], 2)
    got = om.layer(1, h, np.ones(7, bool))
    assert CF.rel(got, CF.audio_norm_out64(h, w, 1, ac)) <= 1e-6
    assert CF.rel(got, CF.audio_norm_out64(h, w, 1, ac, "norm_out_is_pre_attention")) > SEEN
    mel = svl_synth.mel_clips([23], seed=4)[0]
    out = om.forward(mel.features, mel.mask.astype(bool), capture_hidden=True)
    hs = out["hidden_states"]
    assert CF.rel(hs[0], CF.audio_norm_out64(out["sscp_output"], w, 0, ac)) <= 1e-6
    assert CF.rel(hs[1], CF.audio_norm_out64(hs[0], w, 1, ac)) <= 1e-6
    assert CF.rel(out["pooled"], CF.audio_tail64(hs[1], w, ac)) <= 1e-5
    for mistake in ("no_output_bias", "bias_after_norm"):
        assert CF.rel(out["pooled"], CF.audio_tail64(hs[1], w, ac, mistake)) > SEEN, mistake


@pytest.mark.parametrize("kind", ["tiny", "au"])
@pytest.mark.parametrize("branch", ["feed_forward1", "feed_forward2"])
def test_audio_feed_forward_branch_wiring(kind, branch):
    """Only one feed-forward branch live: the layer is
    RMSNorm(h + w_r RMSNorm(clamp(l2(SiLU(l1(RMSNorm(clamp(h), pre)))))), post), norm_out)
    with each linear's own bounds (audio.rs:1374-1433)."""
    c, ac, w0, th = audio_model(kind, 1, seed=52)
    w = CF.audio_degenerate(w0, 1, keep=(branch,), seed=2)
    om = O.OracleAudioModel(c, w, th)
    h = _hidden(6, ac["hidden_size"], 3)
    got = om.layer(0, h, np.ones(6, bool))
    want = lambda m=None: CF.audio_norm_out64(CF.audio_ff64(h, w, 0, ac, branch, m), w, 0, ac)
    assert CF.rel(got, want()) <= TOL
    for mistake in ("ffn_norms_swapped", "ffn_norms_of_the_other_branch", "ffn_bounds_swapped",
                    "no_gradient_clip", "no_residual_weight"):
        assert CF.rel(got, want(mistake)) > SEEN, mistake


@pytest.mark.parametrize("kind", ["tiny", "au"])
def test_audio_attention_block_on_identical_rows(kind):
    """Only the attention branch live and every row equal: attention returns
    the value row, so the block is h + RMSNorm(post(v(RMSNorm(h, pre)))) with
    the v and post bounds (audio.rs:1022-1050)."""
    c, ac, w0, th = audio_model(kind, 1, seed=53)
    w = CF.audio_degenerate(w0, 1, keep=("attention",), seed=3)
    om = O.OracleAudioModel(c, w, th)
    h = np.repeat(_hidden(1, ac["hidden_size"], 4), 9, axis=0)
    got = om.layer(0, h, np.ones(9, bool))
    want = lambda m=None: CF.audio_norm_out64(CF.audio_attention_identical64(h, w, 0, ac, m),
                                             w, 0, ac)
    assert CF.rel(got, want()) <= TOL
    for mistake in ("attention_norms_swapped", "v_bounds_are_k_bounds",
                    "post_bounds_are_q_bounds"):
        assert CF.rel(got, want(mistake)) > SEEN, mistake


@pytest.mark.parametrize("kind", ["tiny", "au"])
def test_audio_attention_block_on_two_rows(kind):
    """Only the attention branch live, two valid rows: the second row's
    attention is a two-way softmax of soft-capped scores with per_dim_scale
    through softplus, the key scale and the relative keys of each key's
    position id (audio.rs:1529-1669)."""
    c, ac, w0, th = audio_model(kind, 1, seed=54)
    w = CF.audio_degenerate(w0, 1, keep=("attention",), seed=4)
    om = O.OracleAudioModel(c, w, th)
    mistakes = ("per_dim_scale_reversed", "no_softplus", "no_key_scale",
                "relative_distance_flipped")
    errs, bad = [], {k: 0.0 for k in mistakes}
    for seed in range(4):
        h = _hidden(2, ac["hidden_size"], 10 + seed)
        got = om.layer(0, h, np.ones(2, bool))
        want = lambda m=None: CF.audio_norm_out64(CF.audio_attention_two_rows64(h, w, 0, ac, m),
                                                 w, 0, ac)
        errs.append(CF.rel(got, want()))
        for k in mistakes:
            bad[k] = max(bad[k], CF.rel(got, want(k)))
    assert max(errs) <= TOL, errs
    for k, e in bad.items():
        assert e > SEEN, (k, e)


@pytest.mark.parametrize("kind", ["tiny", "au"])
def test_audio_light_conv_branch_wiring(kind):
    """Only the light-conv branch live: pre norm, start linear, GLU, causal
    depthwise taps, clamp, conv norm, SiLU, end linear (audio.rs:1448-1527)."""
    c, ac, w0, th = audio_model(kind, 1, seed=55)
    w = CF.audio_degenerate(w0, 1, keep=("light_conv",), seed=5)
    om = O.OracleAudioModel(c, w, th)
    h = _hidden(9, ac["hidden_size"], 6)
    got = om.layer(0, h, np.ones(9, bool))
    want = lambda m=None: CF.audio_norm_out64(CF.audio_lconv64(h, w, 0, ac, m), w, 0, ac)
    assert CF.rel(got, want()) <= TOL
    for mistake in ("lconv_norms_swapped", "lconv_bounds_swapped", "glu_halves_swapped",
                    "taps_reversed"):
        assert CF.rel(got, want(mistake)) > SEEN, mistake


@pytest.mark.parametrize("kind", ["tiny", "au"])
def test_audio_subsampling_norm_weights_act_per_channel(kind):
    """A positive LayerNorm weight commutes with the ReLU after it
    (audio.rs:1290-1322), so scaling layer 0's norm weight by w equals
    scaling layer 1's conv weights along their input channel by w, and
    scaling layer 1's norm weight equals scaling the input projection's
    columns of that channel in the [t, f, c] flattening (audio.rs:1136-1255).
    A reversed w must not."""
    c, ac, w0, th = audio_model(kind, 1, seed=56, clip=1e10)
    pre = "audio_tower.subsample_conv_projection."
    C0, C1, H = ac["conv_channels0"], ac["conv_channels1"], ac["hidden_size"]
    rng = np.random.default_rng(7)
    base = dict(w0)
    base[pre + "layer0.norm.weight"] = np.ones(C0, np.float32)
    base[pre + "layer1.norm.weight"] = np.ones(C1, np.float32)
    mel = svl_synth.mel_clips([21], seed=6)[0]

    def sscp(w):
        return O.OracleAudioModel(c, w, th).forward(mel.features, mel.mask.astype(bool),
                                                    capture_hidden=True)["sscp_output"]

    s0 = rng.uniform(0.5, 1.5, C0).astype(np.float32)
    s1 = rng.uniform(0.5, 1.5, C1).astype(np.float32)
    got = sscp(dict(base, **{pre + "layer0.norm.weight": s0, pre + "layer1.norm.weight": s1}))

    def moved(a0, a1):
        w = dict(base)
        w[pre + "layer1.conv.weight"] = (base[pre + "layer1.conv.weight"] *
                                         a0[None, :, None, None]).astype(np.float32)
        win = base[pre + "input_proj_linear.weight"].reshape(H, -1, C1)
        w[pre + "input_proj_linear.weight"] = (win * a1[None, None, :]).reshape(H, -1).astype(
            np.float32)
        return sscp(w)

    assert CF.rel(got, moved(s0, s1)) <= 1e-5
    assert CF.rel(got, moved(s0[::-1].copy(), s1)) > SEEN
    assert CF.rel(got, moved(s0, s1[::-1].copy())) > SEEN
