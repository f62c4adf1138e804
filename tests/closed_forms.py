"""Closed forms of the encoder towers on degenerate weight sets, in float64.

Each function states one branch or one layer of the reference for inputs
that make it a short formula: zero projections (a branch adds RMSNorm(0) = 0),
rows that are all equal (attention returns the value row whatever the softmax
weights), or two rows (the softmax is a two-way logistic). They are written
from the reference source, independently of the C oracle's loop nests, and
every function takes a `mistake` argument that plants one plausible wiring
error, so a test can show that the comparison it makes would catch it.

References: src/model/text.rs:182-538, src/model/vision.rs:742-959,
src/model/audio.rs:981-1134, 1290-1527, 1529-1669.
"""
import math

import numpy as np

# ---- primitives (kernels.rs:380-388, 727-857; audio.rs:1339-1372) --------------------


def rms(x, w, eps):
    """RMSNorm over the last axis; w None is the unscaled norm."""
    x = np.asarray(x, np.float64)
    y = x / np.sqrt((x * x).mean(-1, keepdims=True) + float(eps))
    return y if w is None else y * np.asarray(w, np.float64)


def gelu(x):
    return 0.5 * x * (1.0 + np.tanh(0.7978846 * (x + 0.044715 * x ** 3)))


def silu(x):
    return x / (1.0 + np.exp(-x))


def sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def softplus(x):
    return np.log1p(np.exp(x))


def f64(a):
    return np.asarray(a, np.float64)


def rel(a, b):
    a, b = f64(a), f64(b)
    return float(np.abs(a - b).max() / np.abs(b).max())


def two_way_softmax(s0, s1):
    """softmax([s0, s1]) as the logistic of the score difference."""
    p0 = 1.0 / (1.0 + np.exp(s1 - s0))
    return p0, 1.0 - p0


# ---- text encoder (text.rs:182-538) ---------------------------------------------------

TL = "language_model.layers.{}."
EMBED = "language_model.embed_tokens.weight"
OUT_PROJ = "language_model.embedding_projection.weight"
FINAL_NORM = "language_model.norm.weight"
PLE_MODEL = "language_model.ple.per_layer_model_projection.weight"
PLE_NORM = "language_model.ple.per_layer_projection_norm.weight"
TEXT_PROJECTIONS = ("self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight",
                    "self_attn.o_proj.weight", "mlp.gate_proj.weight", "mlp.up_proj.weight",
                    "mlp.down_proj.weight", "ple_block.per_layer_input_gate.weight",
                    "ple_block.per_layer_projection.weight")


def zero_text(w, layers, names=TEXT_PROJECTIONS):
    out = dict(w)
    for l in range(layers):
        for n in names:
            k = TL.format(l) + n
            out[k] = np.zeros_like(w[k])
    return out


def embedding_scale(H):
    """config.rs:241: (hidden_size as f32).sqrt()."""
    return np.sqrt(np.float32(H), dtype=np.float32)


def text_zero_projection_states(w, rc, ids, mistake=None):
    """Hidden states of a model whose nine projections per layer are zero:
    every branch adds RMSNorm(0) = 0, so hidden_l = hidden_{l-1} * layer_scalar_l
    exactly (text.rs:505-513), starting from the gather times sqrt(H)
    (text.rs:209-224). float32, the reference's own rounding."""
    H, L = rc["hidden_size"], rc["num_hidden_layers"]
    h = np.asarray(w[EMBED], np.float32)[np.asarray(ids)]
    if mistake != "no_embedding_scale":
        h = h * embedding_scale(H)
    states = [h]
    for l in range(L):
        src = L - 1 - l if mistake == "scalars_reversed" else l
        s = np.float32(np.asarray(w[TL.format(src) + "layer_scalar"]).reshape(-1)[0])
        if mistake != "no_layer_scalar":
            h = (h * s).astype(np.float32)
        states.append(h)
    return states


def text_head(w, rc, h, mistake=None):
    """text.rs:520-537: final norm, embedding projection, mean pool, L2."""
    eps = rc["rms_norm_eps"]
    nw = w[FINAL_NORM]
    if mistake == "final_norm_is_input_layernorm":
        nw = w[TL.format(0) + "input_layernorm.weight"]
    elif mistake == "final_norm_reversed":
        nw = np.asarray(nw)[::-1]
    n = f64(h) if mistake == "no_final_norm" else rms(h, nw, eps)
    proj = n @ f64(w[OUT_PROJ]).T
    pooled = proj.mean(0)
    return dict(projected=proj, pooled=pooled, normalized=pooled / np.linalg.norm(pooled))


def text_per_layer_inputs(w, rc, h0, mistake=None):
    """text.rs:285-306: ((h0 W_ple^T) * 1/sqrt(H)) as [rows, L, p], RMSNorm per
    p-wide segment with the shared projection norm."""
    H, L, P, eps = (rc["hidden_size"], rc["num_hidden_layers"], rc["hidden_size_per_layer_input"],
                    rc["rms_norm_eps"])
    x = f64(h0) @ f64(w[PLE_MODEL]).T
    if mistake != "no_ple_scale":
        x = x * (1.0 / math.sqrt(H))
    return rms(x.reshape(*x.shape[:-1], L, P), w[PLE_NORM], eps)


def text_identical_token_states(w, rc, tok, mistake=None):
    """One-row hidden states of a row that repeats one token id. Every row of
    every hidden state is then equal, so attention returns the unscaled-norm
    value row whatever its weights (sum_j p_j v = v), and each layer is the
    closed form of text.rs:345-513 on one row: input norm, V projection and
    unscaled norm, O projection, post-attention norm, pre/post feed-forward
    norms around GeGLU, the PLE gate on the un-normalised hidden times this
    layer's slice, projection, post-PLE norm, and layer_scalar over the sum."""
    H, L, NH, eps = (rc["hidden_size"], rc["num_hidden_layers"], rc["num_attention_heads"],
                     rc["rms_norm_eps"])
    h = f64(np.asarray(w[EMBED], np.float32)[tok] * embedding_scale(H))
    per_layer = text_per_layer_inputs(w, rc, h, mistake)
    states = [h]
    for l in range(L):
        p = TL.format(l)
        W = lambda n: f64(w[p + n])
        hd, nkv = rc["head_dim"][l], rc["num_kv_heads"][l]
        in_ln, post_attn = w[p + "input_layernorm.weight"], w[p + "post_attention_layernorm.weight"]
        pre_ff, post_ff = w[p + "pre_feedforward_layernorm.weight"], \
            w[p + "post_feedforward_layernorm.weight"]
        post_ple = w[p + "ple_block.post_per_layer_input_norm.weight"]
        if mistake == "attention_norms_swapped":
            in_ln, post_attn = post_attn, in_ln
        if mistake == "ffn_norms_swapped":
            pre_ff, post_ff = post_ff, pre_ff
        if mistake == "ple_norm_is_post_ffn":
            post_ple = post_ff
        n = rms(h, in_ln, eps)
        v = (n @ W("self_attn.v_proj.weight").T).reshape(nkv, hd)
        v = rms(v, w[p + "self_attn.k_norm.weight"] if mistake == "scaled_v_norm" else None, eps)
        attn = np.concatenate([v[hh // (NH // nkv)] for hh in range(NH)])
        h = h + rms(attn @ W("self_attn.o_proj.weight").T, post_attn, eps)
        n = rms(h, pre_ff, eps)
        act = gelu(n @ W("mlp.gate_proj.weight").T) * (n @ W("mlp.up_proj.weight").T)
        h = h + rms(act @ W("mlp.down_proj.weight").T, post_ff, eps)
        gate_in = rms(h, pre_ff, eps) if mistake == "ple_gate_on_normalised_hidden" else h
        slice_ = per_layer[L - 1 - l] if mistake == "ple_slices_reversed" else per_layer[l]
        g = gelu(gate_in @ W("ple_block.per_layer_input_gate.weight").T) * slice_
        proj = rms(g @ W("ple_block.per_layer_projection.weight").T, post_ple, eps)
        s = float(np.asarray(w[p + "layer_scalar"]).reshape(-1)[0])
        h = h * s + proj if mistake == "scalar_before_ple_residual" else (h + proj) * s
        states.append(h)
    return states


def rope_inv_freq64(hd, theta):
    """kernels.rs:991-1010: 1 / theta^(2j / hd), j < hd / 2."""
    return 1.0 / (float(theta) ** (np.arange(0, hd, 2, dtype=np.float64) / hd))


def rope_rotate_half(x, pos, inv):
    """kernels.rs:936-988: element j pairs with j + hd/2;
    (a, b) -> (a cos - b sin, a sin + b cos) at angle pos * inv_freq[j]."""
    half = x.shape[-1] // 2
    ang = np.asarray(pos, np.float64)[:, None] * inv[None, :]
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    a, b = x[..., :half], x[..., half:]
    return np.concatenate([a * c - b * s, a * s + b * c], -1)


def rope_interleaved(x, pos, inv):
    """A wrong pairing (2j with 2j + 1), planted to show the tests see it."""
    ang = np.asarray(pos, np.float64)[:, None] * inv[None, :]
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    a, b = x[..., 0::2], x[..., 1::2]
    out = np.empty_like(x)
    out[..., 0::2], out[..., 1::2] = a * c - b * s, a * s + b * c
    return out


def text_two_token_states(w, rc, ids, mistake=None):
    """Hidden states of a two-token row through a model whose feed-forward
    and PLE gate weights are zero (those branches add RMSNorm(0) = 0), so a
    layer is hidden' = (hidden + RMSNorm(attention W_o^T)) * layer_scalar.
    Attention over two keys is a two-way logistic of the score difference,
    here written out with the per-head q_norm / k_norm, rotate-half RoPE at
    positions 0 and 1 with the layer type's theta, GQA head h -> h / (nh / kv)
    and scale 1.0 (text.rs:345-433, kernels.rs:1013-1135)."""
    H, L, NH, eps = (rc["hidden_size"], rc["num_hidden_layers"], rc["num_attention_heads"],
                     rc["rms_norm_eps"])
    assert len(ids) == 2
    h = f64(np.asarray(w[EMBED], np.float32)[np.asarray(ids)] * embedding_scale(H))
    pos = np.array([0.0, 1.0])
    states = [h]
    for l in range(L):
        p = TL.format(l)
        W = lambda n: f64(w[p + n])
        hd, nkv, full = rc["head_dim"][l], rc["num_kv_heads"][l], rc["layer_type"][l] == 1
        theta = rc["full_rope_theta"] if full else rc["sliding_rope_theta"]
        if mistake == "theta_swapped":
            theta = rc["sliding_rope_theta"] if full else rc["full_rope_theta"]
        qn_w, kn_w = w[p + "self_attn.q_norm.weight"], w[p + "self_attn.k_norm.weight"]
        if mistake == "qk_norms_swapped":
            qn_w, kn_w = kn_w, qn_w
        if mistake == "no_k_norm_weight":
            kn_w = None
        n = rms(h, w[p + "input_layernorm.weight"], eps)
        q = (n @ W("self_attn.q_proj.weight").T).reshape(2, NH, hd)
        k = (n @ W("self_attn.k_proj.weight").T).reshape(2, nkv, hd)
        v = rms((n @ W("self_attn.v_proj.weight").T).reshape(2, nkv, hd), None, eps)
        inv = rope_inv_freq64(hd, theta)
        rope = rope_interleaved if mistake == "rope_pairs_interleaved" else rope_rotate_half
        if mistake == "rope_before_norm":
            q, k = rms(rope(q, pos, inv), qn_w, eps), rms(rope(k, pos, inv), kn_w, eps)
        elif mistake == "no_rope":
            q, k = rms(q, qn_w, eps), rms(k, kn_w, eps)
        else:
            q, k = rope(rms(q, qn_w, eps), pos, inv), rope(rms(k, kn_w, eps), pos, inv)
        scale = 1.0 / math.sqrt(hd) if mistake == "scores_scaled" else 1.0
        out = np.zeros((2, NH, hd))
        for i in range(2):
            for hh in range(NH):
                g = hh % nkv if mistake == "gqa_heads_interleaved" else hh // (NH // nkv)
                p0, p1 = two_way_softmax(scale * (q[i, hh] @ k[0, g]), scale * (q[i, hh] @ k[1, g]))
                out[i, hh] = p0 * v[0, g] + p1 * v[1, g]
        h = h + rms(out.reshape(2, NH * hd) @ W("self_attn.o_proj.weight").T,
                    w[p + "post_attention_layernorm.weight"], eps)
        h = h * float(np.asarray(w[p + "layer_scalar"]).reshape(-1)[0])
        states.append(h)
    return states


# ---- vision tower (vision.rs:742-959) -------------------------------------------------

VL = "vision_tower.encoder.layers.{}."
V_FFN = ("mlp.gate_proj.linear.weight", "mlp.up_proj.linear.weight",
         "mlp.down_proj.linear.weight")


def axial_inv_freq64(hd, theta):
    """vision.rs:1047-1065: hd/4 frequencies 1 / theta^(2i / (hd/2))."""
    spatial = hd // 2
    return 1.0 / (float(theta) ** (np.arange(0, spatial, 2, dtype=np.float64) / spatial))


def axial_rope64(x, pos, inv):
    """vision.rs:1073-1148: the first half of a head rotates by x, the second
    by y; within a half, quarter i pairs with quarter i + hd/4."""
    hd = x.shape[-1]
    half, q = hd // 2, hd // 4
    out = np.array(x, np.float64)
    for hf in (0, 1):
        ang = np.asarray(pos, np.float64)[:, hf][:, None] * inv[None, :]
        c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
        a = x[..., hf * half: hf * half + q]
        b = x[..., hf * half + q: (hf + 1) * half]
        out[..., hf * half: hf * half + q] = a * c - b * s
        out[..., hf * half + q: (hf + 1) * half] = b * c + a * s
    return out


def vision_two_patch_layer(w, vc, l, h, pos, mistake=None):
    """One encoder layer over two patches whose feed-forward weights are zero
    (that branch adds RMSNorm(0) = 0): hidden + RMSNorm(attention W_o^T) with
    the attention a two-way logistic over the per-head q_norm / k_norm
    outputs rotated by axial RoPE at the patches' (x, y), scale 1.0
    (vision.rs:816-878)."""
    NH, NKV, hd, eps = (vc["num_attention_heads"], vc["num_key_value_heads"], vc["head_dim"],
                        vc["rms_norm_eps"])
    p = VL.format(l)
    W = lambda n: f64(w[p + n])
    pos = np.asarray(pos, np.float64)
    if mistake == "xy_swapped":
        pos = pos[:, ::-1]
    qn_w, kn_w = w[p + "self_attn.q_norm.weight"], w[p + "self_attn.k_norm.weight"]
    if mistake == "qk_norms_swapped":
        qn_w, kn_w = kn_w, qn_w
    n = rms(h, w[p + "input_layernorm.weight"], eps)
    q = (n @ W("self_attn.q_proj.linear.weight").T).reshape(2, NH, hd)
    k = (n @ W("self_attn.k_proj.linear.weight").T).reshape(2, NKV, hd)
    v = rms((n @ W("self_attn.v_proj.linear.weight").T).reshape(2, NKV, hd), None, eps)
    inv = axial_inv_freq64(hd, vc["rope_theta"])
    if mistake == "rope_before_norm":
        q, k = rms(axial_rope64(q, pos, inv), qn_w, eps), rms(axial_rope64(k, pos, inv), kn_w, eps)
    elif mistake == "text_rope":
        tinv = rope_inv_freq64(hd, vc["rope_theta"])
        q = rope_rotate_half(rms(q, qn_w, eps), pos[:, 0], tinv)
        k = rope_rotate_half(rms(k, kn_w, eps), pos[:, 0], tinv)
    elif mistake == "no_key_rope":
        q, k = axial_rope64(rms(q, qn_w, eps), pos, inv), rms(k, kn_w, eps)
    else:
        q, k = axial_rope64(rms(q, qn_w, eps), pos, inv), axial_rope64(rms(k, kn_w, eps), pos, inv)
    scale = 1.0 / math.sqrt(hd) if mistake == "scores_scaled" else 1.0
    out = np.zeros((2, NH, hd))
    for i in range(2):
        for hh in range(NH):
            g = hh // (NH // NKV)
            p0, p1 = two_way_softmax(scale * (q[i, hh] @ k[0, g]), scale * (q[i, hh] @ k[1, g]))
            out[i, hh] = p0 * v[0, g] + p1 * v[1, g]
    return h + rms(out.reshape(2, NH * hd) @ W("self_attn.o_proj.linear.weight").T,
                   w[p + "post_attention_layernorm.weight"], eps)


# ---- audio tower (audio.rs:981-1134) --------------------------------------------------

AL = "audio_tower.layers.{}."
BOUNDS = ("input_min", "input_max", "output_min", "output_max")
# Every ClippedLinear of a layer, by its weight prefix.
AUDIO_LINEARS = ("feed_forward1.ffw_layer_1", "feed_forward1.ffw_layer_2",
                 "feed_forward2.ffw_layer_1", "feed_forward2.ffw_layer_2",
                 "self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.post",
                 "lconv1d.linear_start", "lconv1d.linear_end")
AUDIO_BRANCHES = {
    "feed_forward1": ("feed_forward1.ffw_layer_1", "feed_forward1.ffw_layer_2"),
    "feed_forward2": ("feed_forward2.ffw_layer_1", "feed_forward2.ffw_layer_2"),
    "attention": ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.post"),
    "light_conv": ("lconv1d.linear_start", "lconv1d.linear_end"),
}


def audio_degenerate(w, layers, keep=(), seed=0):
    """Copy of audio weights whose clipped linears are zero except those of
    the branches named in `keep`, with distinct bounds per linear drawn so
    that they bind on O(1) activations (inputs in -U(0.5,1.5)..U(0.5,1.5),
    outputs likewise). A zero linear's output 0 stays inside its bounds, so a
    zeroed branch adds RMSNorm(0) = 0 (or 0 for the light conv's end)."""
    rng = np.random.default_rng(seed)
    out = dict(w)
    for l in range(layers):
        p = AL.format(l)
        live = {lin for b in keep for lin in AUDIO_BRANCHES[b]}
        for lin in AUDIO_LINEARS:
            k = p + lin + ".linear.weight"
            if lin not in live:
                out[k] = np.zeros_like(w[k])
            lo_hi = rng.uniform(0.5, 1.5, 4) * np.array([-1, 1, -1, 1])
            for b, v in zip(BOUNDS, lo_hi):
                out[p + lin + "." + b] = np.asarray(v, np.float32).reshape(np.shape(w[p + lin + "." + b]))
    return out


def _bounds(w, prefix):
    return [float(np.asarray(w[prefix + "." + b]).reshape(-1)[0]) for b in BOUNDS]


def clipped(x, w, prefix, bounds_from=None):
    """audio.rs:558-601: clamp the input, multiply, clamp the output."""
    b = _bounds(w, bounds_from or prefix)
    y = np.clip(f64(x), b[0], b[1]) @ f64(w[prefix + ".linear.weight"]).T
    return np.clip(y, b[2], b[3])


def audio_ff64(h, w, l, ac, branch, mistake=None):
    """audio.rs:1374-1433 feed_forward: clamp(+-clip) -> pre norm -> clipped
    linear -> SiLU -> clipped linear -> clamp -> post norm -> residual +
    residual_weight * x."""
    p = AL.format(l) + branch + "."
    eps, clip, rw = ac["rms_norm_eps"], ac["gradient_clipping"], ac["residual_weight"]
    pre, post = w[p + "pre_layer_norm.weight"], w[p + "post_layer_norm.weight"]
    if mistake == "ffn_norms_swapped":
        pre, post = post, pre
    if mistake == "ffn_norms_of_the_other_branch":
        other = AL.format(l) + ("feed_forward2." if branch == "feed_forward1" else "feed_forward1.")
        pre, post = w[other + "pre_layer_norm.weight"], w[other + "post_layer_norm.weight"]
    x = f64(h) if mistake == "no_gradient_clip" else np.clip(f64(h), -clip, clip)
    b1, b2 = p + "ffw_layer_1", p + "ffw_layer_2"
    swap = mistake == "ffn_bounds_swapped"
    a = silu(clipped(rms(x, pre, eps), w, b1, b2 if swap else None))
    y = clipped(a, w, b2, b1 if swap else None)
    y = y if mistake == "no_gradient_clip" else np.clip(y, -clip, clip)
    return f64(h) + (1.0 if mistake == "no_residual_weight" else rw) * rms(y, post, eps)


def audio_attention_identical64(h, w, l, ac, mistake=None):
    """The attention block (audio.rs:1022-1050) on rows that are all equal and
    all valid: every key of a query's window has the same value row, and the
    query's own key is always in its window, so attention returns the value
    row: hidden + RMSNorm(post(v(RMSNorm(hidden, pre)))), post norm."""
    p = AL.format(l)
    eps = ac["rms_norm_eps"]
    pre, post = w[p + "norm_pre_attn.weight"], w[p + "norm_post_attn.weight"]
    if mistake == "attention_norms_swapped":
        pre, post = post, pre
    n = rms(h, pre, eps)
    v = clipped(n, w, p + "self_attn.v_proj", p + "self_attn.k_proj" if mistake == "v_bounds_are_k_bounds" else None)
    o = clipped(v, w, p + "self_attn.post", p + "self_attn.q_proj" if mistake == "post_bounds_are_q_bounds" else None)
    return f64(h) + rms(o, post, eps)


def audio_sinusoid64(hidden, distance):
    """audio.rs:1257-1287 for one relative distance d: [sin(d t_i), cos(d t_i)]
    with t_i = exp(-i ln(10000) / (hidden/2 - 1))."""
    T = hidden // 2
    inv = np.exp(-np.arange(T) * (math.log(10000.0) / (T - 1)))
    return np.concatenate([np.sin(distance * inv), np.cos(distance * inv)])


def audio_attention_two_rows64(h, w, l, ac, mistake=None):
    """The attention block on two valid rows (one chunk; the window reaches one
    row back). Row 0 sees only itself and returns its value row. Row 1 sees
    rows 0 and 1, a two-way softmax of soft-capped scores
    cap * tanh((q . k_j + q . relk(d_j)) / cap), with
    q = q_proj(x) * (hd^-1/2 / ln 2) * softplus(per_dim_scale),
    k = k_proj(x) * ln(1 + e) / ln 2, relk the sinusoid of the key's position
    id projected by relative_k_proj (audio.rs:1529-1669)."""
    p = AL.format(l)
    H, NH, eps, cap = ac["hidden_size"], ac["num_attention_heads"], ac["rms_norm_eps"], \
        ac["attention_logit_cap"]
    hd = H // NH
    n = rms(h, w[p + "norm_pre_attn.weight"], eps)
    pds = f64(w[p + "self_attn.per_dim_scale"]).reshape(-1)
    if mistake == "per_dim_scale_reversed":
        pds = pds[::-1]
    qs = (hd ** -0.5) / math.log(2.0)
    scale = pds if mistake == "no_softplus" else softplus(pds)
    ks = 1.0 if mistake == "no_key_scale" else math.log(1.0 + math.e) / math.log(2.0)
    q = clipped(n, w, p + "self_attn.q_proj").reshape(2, NH, hd) * qs * scale
    k = clipped(n, w, p + "self_attn.k_proj").reshape(2, NH, hd) * ks
    v = clipped(n, w, p + "self_attn.v_proj").reshape(2, NH, hd)
    wrel = f64(w[p + "self_attn.relative_k_proj.weight"])
    # Query 1, key j: context index j + left - 1, relative index j + left - 2,
    # table row of position id P - 1 - relative (audio.rs:1267-1275, 1610-1620).
    left = ac["attention_context_left"]
    P = (ac["attention_chunk_size"] + left - 1 + ac["attention_context_right"]) // 2 + 1
    assert all(0 <= j + left - 2 < P for j in (0, 1))
    d = [P - 1 - (j + left - 2) for j in (0, 1)]
    if mistake == "relative_distance_flipped":
        d = d[::-1]
    relk = [(audio_sinusoid64(H, dd) @ wrel.T).reshape(NH, hd) for dd in d]
    out = np.zeros((2, NH, hd))
    out[0] = v[0]
    for hh in range(NH):
        s = [cap * np.tanh((q[1, hh] @ k[j, hh] + q[1, hh] @ relk[j][hh]) / cap) for j in (0, 1)]
        p0, p1 = two_way_softmax(*s)
        out[1, hh] = p0 * v[0, hh] + p1 * v[1, hh]
    o = clipped(out.reshape(2, H), w, p + "self_attn.post")
    return f64(h) + rms(o, w[p + "norm_post_attn.weight"], eps)


def audio_lconv64(h, w, l, ac, mistake=None):
    """audio.rs:1448-1527 light_conv: pre norm -> clipped linear to 2H -> GLU
    a * sigmoid(b) -> causal depthwise conv (tap t reads row r - (K-1) + t) ->
    clamp -> conv norm -> SiLU -> clipped linear -> residual."""
    p = AL.format(l) + "lconv1d."
    eps, clip = ac["rms_norm_eps"], ac["gradient_clipping"]
    H = ac["hidden_size"]
    pre, cn = w[p + "pre_layer_norm.weight"], w[p + "conv_norm.weight"]
    if mistake == "lconv_norms_swapped":
        pre, cn = cn, pre
    swap = mistake == "lconv_bounds_swapped"
    st = clipped(rms(h, pre, eps), w, p + "linear_start", p + "linear_end" if swap else None)
    a, b = st[:, :H], st[:, H:]
    g = b * sigmoid(a) if mistake == "glu_halves_swapped" else a * sigmoid(b)
    dw = f64(w[p + "depthwise_conv1d.weight"]).reshape(H, -1)
    K = dw.shape[1]
    if mistake == "taps_reversed":
        dw = dw[:, ::-1]
    rows = g.shape[0]
    conv = np.zeros_like(g)
    for r in range(rows):
        for t in range(K):
            src = r - (K - 1) + t
            if 0 <= src < rows:
                conv[r] += g[src] * dw[:, t]
    conv = np.clip(conv, -clip, clip)
    e = clipped(silu(rms(conv, cn, eps)), w, p + "linear_end", p + "linear_start" if swap else None)
    return f64(h) + e


def audio_norm_out64(h, w, l, ac, mistake=None):
    p = AL.format(l)
    nw = w[p + ("norm_pre_attn.weight" if mistake == "norm_out_is_pre_attention"
                else "norm_out.weight")]
    return rms(h, nw, ac["rms_norm_eps"])


def audio_tail64(h_last, w, ac, mistake=None):
    """audio.rs:1085-1133: output projection plus bias, unscaled RMSNorm,
    projection to the text width."""
    y = f64(h_last) @ f64(w["audio_tower.output_proj.weight"]).T
    b = f64(w["audio_tower.output_proj.bias"])
    if mistake not in ("no_output_bias", "bias_after_norm"):
        y = y + b
    n = rms(y, None, ac["rms_norm_eps"])
    if mistake == "bias_after_norm":
        n = n + b
    return n @ f64(w["embed_audio.embedding_projection.weight"]).T
