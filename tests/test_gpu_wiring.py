"""The closed forms that pin the oracle's 1-D parameter wiring
(tests/test_oracle_wiring.py), met by the GPU path through the C ABI.

* text at full depth (shape A and shape B, 24 layers, vocab 262144): zero
  projections leave hidden_l = hidden_{l-1} * layer_scalar_l bit for bit and
  the head's closed form; rows repeating one token meet the one-row closed
  form of every norm weight, the PLE block and layer_scalar at every layer,
  including a 600-token row that crosses the 512-token window;
* text, two-token rows through a sliding and a full layer: the two-way
  logistic of the q_norm / k_norm / RoPE / GQA side, for head_dim 8, 16 and
  256;
* audio at config AU: zero projections through 12 layers on a 30 s clip
  (norm_out per layer, the tail with its output bias); one live branch at a
  time (both feed-forwards, the light conv) from the GPU's own subsampling
  output, with distinct binding bounds per linear and a binding gradient
  clip; the subsampling norm weights' equivalence with scaled input channels.
"""
import numpy as np
import pytest

import closed_forms as CF
import svl_amd as S
import svl_audio as A
import svl_synth
import test_oracle_wiring as TW

pytestmark = pytest.mark.gpu

TOL = 1e-4
SEEN = 1e-3


def random_1d(w, seed):
    """Norm weights U(0.5, 1.5) and layer scalars U(0.5, 1.0); q/k norms keep
    the synthetic U(0.2, 0.3), which gives order-one scores at head_dim 256."""
    rng = np.random.default_rng(seed)
    w = dict(w)
    for k, a in w.items():
        if a.ndim != 1 or k.endswith(("q_norm.weight", "k_norm.weight")):
            continue
        hi = 1.0 if k.endswith("layer_scalar") else 1.5
        w[k] = rng.uniform(0.5, hi, a.shape).astype(np.float32)
    return w


@pytest.fixture(scope="module")
def shape_a_full():
    c = svl_synth.config_a(24)
    return c, S.TextConfig.from_json_value(c), random_1d(svl_synth.weights(c, seed=0), 61)


def test_zero_projections_at_full_depth(shape_a_full):
    """Shape A, 24 layers, vocab 262144, a 128-token and a 37-token row: the
    gather times sqrt(H), then one layer_scalar multiply per layer, bit for
    bit; then the final norm, projection, pool and L2 (text.rs:209-537)."""
    from oracle import oracle as O
    c, tc, w = shape_a_full
    rc = O.resolve_config(c)
    wz = CF.zero_text(w, 24)
    m = S.TextModel(tc, wz)
    rng = np.random.default_rng(2)
    rows = [rng.integers(0, 262144, 128), rng.integers(0, 262144, 37)]
    outs = m.forward_batch([r.tolist() for r in rows], capture_hidden=True)
    for r, out in zip(rows, outs):
        hs = out.hidden_states()
        want = CF.text_zero_projection_states(wz, rc, r)
        for l in range(25):
            assert np.array_equal(hs[l], want[l]), f"row of {len(r)}, hidden state {l}"
        assert TW.max_rel(hs, CF.text_zero_projection_states(wz, rc, r, "scalars_reversed")) > SEEN
        head = CF.text_head(wz, rc, hs[24])
        e = CF.rel(out.projected(), head["projected"])
        print(f"row of {len(r)}: head relative error {e:.3g}", flush=True)
        assert e <= 1e-5
        assert np.abs(out.normalized() - head["normalized"]).max() <= 1e-6
        bad = CF.text_head(wz, rc, hs[24], "final_norm_reversed")["projected"]
        assert CF.rel(out.projected(), bad) > SEEN
    m.close()


@pytest.mark.parametrize("shape", ["a", "b"])
def test_identical_tokens_at_full_depth(shape, shape_a_full):
    """Rows repeating one token (64 and 600 tokens: the second crosses the
    sliding window) through 24 layers at vocab 262144 meet the one-row closed
    form at every layer. Shape B adds two KV heads on sliding layers and
    head_dim 512 on full layers."""
    from oracle import oracle as O
    if shape == "a":
        c, tc, w = shape_a_full
    else:
        c = svl_synth.config_b(24)
        tc = S.TextConfig.from_json_value(c)
        w = random_1d(svl_synth.weights(c, seed=0), 62)
    rc = O.resolve_config(c)
    w = TW.small_ple_projection(w, rc)
    m = S.TextModel(tc, w)
    toks = (11, 262140)
    outs = m.forward_batch([[toks[0]] * 64, [toks[1]] * 600], capture_hidden=True)
    for tok, out in zip(toks, outs):
        hs = out.hidden_states()
        want = CF.text_identical_token_states(w, rc, tok)
        e = TW.max_rel(hs, want)
        print(f"shape {shape}, token {tok} x {hs.shape[1]}: max relative error {e:.3g}",
              flush=True)
        assert e <= TOL
        head = CF.text_head(w, rc, np.broadcast_to(want[24], hs[24].shape))
        assert np.abs(out.normalized() - head["normalized"]).max() <= 1e-5
        for mistake in ("ffn_norms_swapped", "scalar_before_ple_residual", "no_ple_scale"):
            assert TW.max_rel(hs, CF.text_identical_token_states(w, rc, tok, mistake)) > SEEN
    m.close()


@pytest.mark.parametrize("kind", ["tiny", "gqa", "shape_a"])
def test_two_token_attention(kind):
    """Two-token rows through a sliding and a full layer with zero
    feed-forward and PLE gate weights (four rows in one batch)."""
    c, rc, w = TW.text_model(kind, 2, seed=33)
    w = CF.zero_text(w, 2, names=("mlp.gate_proj.weight", "mlp.up_proj.weight",
                                  "mlp.down_proj.weight", "ple_block.per_layer_input_gate.weight"))
    m = S.TextModel(S.TextConfig.from_json_value(c), w)
    rng = np.random.default_rng(5)
    rows = [rng.choice(rc["vocab_size"], 2, replace=False).tolist() for _ in range(4)]
    errs = []
    for ids, out in zip(rows, m.forward_batch(rows, capture_hidden=True)):
        hs = out.hidden_states()
        errs.append(TW.max_rel(hs, CF.text_two_token_states(w, rc, ids)))
        assert TW.max_rel(hs, CF.text_two_token_states(w, rc, ids, "qk_norms_swapped")) > SEEN
    print(f"{kind}: max relative error {max(errs):.3g}", flush=True)
    assert max(errs) <= TOL
    m.close()


# ---- audio -------------------------------------------------------------------------

def _audio_gpu(c, w, th):
    return A.AudioModel(A.AudioConfig.from_json_value(c), w, th)


def test_audio_zero_projections_at_full_depth():
    """Config AU, 12 layers, a 2999-frame clip: every clipped linear zero, so
    layer l's output is RMSNorm(layer l-1's, norm_out_l), from the GPU's own
    subsampling output, and the soft tokens are the tail with its bias."""
    c, ac, w0, th = TW.audio_model("au", 12, seed=63)
    w = CF.audio_degenerate(w0, 12, keep=(), seed=11)
    am = _audio_gpu(c, w, th)
    mel = svl_synth.mel_clips([2999], seed=7)[0]
    out = am.forward(mel, capture_hidden=True)
    hs = out.hidden_states()
    prev = out.sscp_output()
    for l in range(12):
        e = CF.rel(hs[l], CF.audio_norm_out64(prev, w, l, ac))
        assert e <= 1e-5, (l, e)
        prev = hs[l]
    assert CF.rel(hs[5], CF.audio_norm_out64(hs[4], w, 5, ac, "norm_out_is_pre_attention")) > SEEN
    e = CF.rel(out.pooled(), CF.audio_tail64(hs[11], w, ac))
    print(f"tail relative error {e:.3g}", flush=True)
    assert e <= 1e-5
    assert CF.rel(out.pooled(), CF.audio_tail64(hs[11], w, ac, "no_output_bias")) > SEEN
    am.close()


@pytest.mark.parametrize("branch", ["feed_forward1", "feed_forward2", "light_conv"])
def test_audio_branch_wiring(branch):
    """Config AU, one layer, one live branch, bounds distinct per linear and
    binding, gradient clip 1.25: the layer output against the branch's closed
    form applied to the GPU's own subsampling output."""
    c, ac, w0, th = TW.audio_model("au", 1, seed=64)
    w = CF.audio_degenerate(w0, 1, keep=(branch,), seed=12)
    am = _audio_gpu(c, w, th)
    mel = svl_synth.mel_clips([301], seed=8)[0]
    out = am.forward(mel, capture_hidden=True)
    h = out.sscp_output()
    if branch == "light_conv":
        f = lambda m=None: CF.audio_lconv64(h, w, 0, ac, m)
        mistake = "taps_reversed"
    else:
        f = lambda m=None: CF.audio_ff64(h, w, 0, ac, branch, m)
        mistake = "ffn_bounds_swapped"
    got = out.hidden_states()[0]
    e = CF.rel(got, CF.audio_norm_out64(f(), w, 0, ac))
    print(f"{branch}: relative error {e:.3g}", flush=True)
    assert e <= TOL
    assert CF.rel(got, CF.audio_norm_out64(f(mistake), w, 0, ac)) > SEEN
    am.close()


def test_audio_subsampling_norm_weights_act_per_channel():
    """The GPU's subsampling output with norm weights s0, s1 equals the one
    with unit norms and layer 1's conv input channels scaled by s0 and the
    input projection's channel columns by s1 (audio.rs:1136-1322)."""
    c, ac, w0, th = TW.audio_model("au", 1, seed=65, clip=1e10)
    pre = "audio_tower.subsample_conv_projection."
    C0, C1, H = ac["conv_channels0"], ac["conv_channels1"], ac["hidden_size"]
    rng = np.random.default_rng(9)
    s0 = rng.uniform(0.5, 1.5, C0).astype(np.float32)
    s1 = rng.uniform(0.5, 1.5, C1).astype(np.float32)
    mel = svl_synth.mel_clips([257], seed=9)[0]

    def sscp(w):
        am = _audio_gpu(c, w, th)
        s = am.forward(mel, capture_hidden=True).sscp_output()
        am.close()
        return s

    got = sscp(dict(w0, **{pre + "layer0.norm.weight": s0, pre + "layer1.norm.weight": s1}))
    w = dict(w0, **{pre + "layer0.norm.weight": np.ones(C0, np.float32),
                    pre + "layer1.norm.weight": np.ones(C1, np.float32)})
    w[pre + "layer1.conv.weight"] = (w0[pre + "layer1.conv.weight"] *
                                     s0[None, :, None, None]).astype(np.float32)
    win = w0[pre + "input_proj_linear.weight"].reshape(H, -1, C1)
    w[pre + "input_proj_linear.weight"] = (win * s1[None, None, :]).reshape(H, -1).astype(
        np.float32)
    e = CF.rel(got, sscp(w))
    print(f"subsampling equivalence: relative error {e:.3g}", flush=True)
    assert e <= 1e-5
