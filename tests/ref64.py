"""Independent float64 numpy restatement of the reference text forward pass
(src/model/text.rs:182-538), written from the reference source, used as a
brute-force pin of the C oracle on tiny random models whose norm weights and
layer scalars are NOT all ones (the official tiny golden has all-ones 1-D
weights, so it cannot see a skipped layer_scalar or a misaligned weight)."""
import numpy as np


def rms(x, w, eps):
    x = x.astype(np.float64)
    inv = 1.0 / np.sqrt((x * x).mean(-1, keepdims=True) + eps)
    return x * inv * (1.0 if w is None else w.astype(np.float64))


def gelu(x):
    return 0.5 * x * (1.0 + np.tanh(0.7978846 * (x + 0.044715 * x ** 3)))


def rope(x, pos, inv_freq):
    # x [seq, heads, hd]; rotate-half pairs j with j + hd/2 (kernels.rs:936-988)
    half = x.shape[-1] // 2
    ang = pos[:, None].astype(np.float64) * inv_freq[None, :].astype(np.float64)
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    a, b = x[..., :half], x[..., half:]
    return np.concatenate([a * c - b * s, a * s + b * c], -1)


def forward(rc, w, ids, features=None, start=0):
    """rc: oracle.resolve_config(...) dict; w: name -> array."""
    H, P, L = rc["hidden_size"], rc["hidden_size_per_layer_input"], rc["num_hidden_layers"]
    NH, eps = rc["num_attention_heads"], rc["rms_norm_eps"]
    f64 = lambda n: w[n].astype(np.float64)
    seq = len(ids)
    h = f64("language_model.embed_tokens.weight")[np.asarray(ids)] * np.sqrt(np.float32(H))
    if features is not None:
        h[start:start + features.shape[0]] = features
    states = [h.copy()]
    ple = h @ f64("language_model.ple.per_layer_model_projection.weight").T / np.sqrt(H)
    ple = rms(ple.reshape(seq, L, P), w["language_model.ple.per_layer_projection_norm.weight"], eps)
    pos = np.arange(seq)

    def inv_freq(hd, theta):
        return 1.0 / (theta ** (np.arange(0, hd, 2, dtype=np.float64) / hd))

    for l in range(L):
        p = f"language_model.layers.{l}."
        hd, nkv, full = rc["head_dim"][l], rc["num_kv_heads"][l], rc["layer_type"][l] == 1
        theta = rc["full_rope_theta"] if full else rc["sliding_rope_theta"]
        n = rms(h, w[p + "input_layernorm.weight"], eps)
        q = (n @ f64(p + "self_attn.q_proj.weight").T).reshape(seq, NH, hd)
        k = (n @ f64(p + "self_attn.k_proj.weight").T).reshape(seq, nkv, hd)
        v = (n @ f64(p + "self_attn.v_proj.weight").T).reshape(seq, nkv, hd)
        q = rope(rms(q, w[p + "self_attn.q_norm.weight"], eps), pos, inv_freq(hd, theta))
        k = rope(rms(k, w[p + "self_attn.k_norm.weight"], eps), pos, inv_freq(hd, theta))
        v = rms(v, None, eps)
        out = np.zeros((seq, NH, hd))
        r = None if full else rc["sliding_window"]
        for i in range(seq):
            lo, hi = (0, seq - 1) if r is None else (max(0, i - r), min(seq - 1, i + r))
            for hh in range(NH):
                g = hh // (NH // nkv)
                s = k[lo:hi + 1, g] @ q[i, hh]
                pr = np.exp(s - s.max())
                out[i, hh] = (pr / pr.sum()) @ v[lo:hi + 1, g]
        a = out.reshape(seq, NH * hd) @ f64(p + "self_attn.o_proj.weight").T
        h = h + rms(a, w[p + "post_attention_layernorm.weight"], eps)
        n = rms(h, w[p + "pre_feedforward_layernorm.weight"], eps)
        act = gelu(n @ f64(p + "mlp.gate_proj.weight").T) * (n @ f64(p + "mlp.up_proj.weight").T)
        h = h + rms(act @ f64(p + "mlp.down_proj.weight").T, w[p + "post_feedforward_layernorm.weight"], eps)
        gated = gelu(h @ f64(p + "ple_block.per_layer_input_gate.weight").T) * ple[:, l, :]
        pr = gated @ f64(p + "ple_block.per_layer_projection.weight").T
        h = (h + rms(pr, w[p + "ple_block.post_per_layer_input_norm.weight"], eps)) * float(w[p + "layer_scalar"][0])
        states.append(h.copy())
    n = rms(h, w["language_model.norm.weight"], eps)
    proj = n @ f64("language_model.embedding_projection.weight").T
    pooled = proj.mean(0)
    return dict(projected=proj, pooled=pooled, normalized=pooled / np.linalg.norm(pooled),
                hidden_states=np.stack(states))


def randomize_1d(w, seed=0):
    """Copy of w whose 1-D tensors (norm weights, layer scalars) are random."""
    rng = np.random.default_rng(seed)
    out = {}
    for k, a in w.items():
        if a.ndim == 1 and "layer_scalar" in k:
            out[k] = rng.uniform(0.5, 1.0, a.shape).astype(np.float32)
        elif a.ndim == 1:
            out[k] = (1.0 + rng.uniform(-0.3, 0.3, a.shape)).astype(np.float32)
        else:
            out[k] = a
    return out


# ---- vision tower (src/model/vision.rs:742-1148) ---------------------------------

def axial_inv_freq64(hd, theta):
    spatial = hd // 2
    return 1.0 / (float(theta) ** (np.arange(0, spatial, 2, dtype=np.float64) / spatial))


def axial_rope64(x, pos, inv_freq):
    """x [seq, heads, hd]; half 0 rotates by pos[:, 0] (x), half 1 by pos[:, 1]
    (y); within a half, quarter i pairs with quarter i + hd/4."""
    hd = x.shape[-1]
    half, q = hd // 2, hd // 4
    out = np.array(x, dtype=np.float64)
    for hf in (0, 1):
        ang = pos[:, hf].astype(np.float64)[:, None] * np.asarray(inv_freq, np.float64)[None, :]
        c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
        a = x[..., hf * half: hf * half + q].astype(np.float64)
        b = x[..., hf * half + q: (hf + 1) * half].astype(np.float64)
        out[..., hf * half: hf * half + q] = a * c - b * s
        out[..., hf * half + q: (hf + 1) * half] = b * c + a * s
    return out


def pool_patches64(h, pos, grid_w, grid_h, soft):
    pw = grid_w // 3
    out = np.zeros((soft, h.shape[1]))
    for p in range(h.shape[0]):
        out[pos[p, 0] // 3 + pw * (pos[p, 1] // 3)] += h[p]
    return out / 9.0 * np.sqrt(h.shape[1])


def vision_forward64(vc, w, pix, pos, grid, soft, swap_axes=False):
    """vc: oracle.resolve_vision_config(...) dict; w: name -> array;
    pix [valid, 768]; pos [valid, 2]. swap_axes rotates the first half by y
    and the second by x (a planted mistake for the sensitivity test)."""
    H, L = vc["hidden_size"], vc["num_hidden_layers"]
    NH, NKV, hd, eps = vc["num_attention_heads"], vc["num_key_value_heads"], vc["head_dim"], vc["rms_norm_eps"]
    f64 = lambda n: w[n].astype(np.float64)
    valid = pix.shape[0]
    h = (2.0 * (pix.astype(np.float64) - 0.5)) @ f64("vision_tower.patch_embedder.input_proj.weight").T
    table = f64("vision_tower.patch_embedder.position_embedding_table")
    h = h + table[0][pos[:, 0]] + table[1][pos[:, 1]]
    states = [h.copy()]
    inv = axial_inv_freq64(hd, vc["rope_theta"])
    rpos = pos[:, ::-1] if swap_axes else pos
    for l in range(L):
        p = f"vision_tower.encoder.layers.{l}."
        n = rms(h, w[p + "input_layernorm.weight"], eps)
        q = (n @ f64(p + "self_attn.q_proj.linear.weight").T).reshape(valid, NH, hd)
        k = (n @ f64(p + "self_attn.k_proj.linear.weight").T).reshape(valid, NKV, hd)
        v = (n @ f64(p + "self_attn.v_proj.linear.weight").T).reshape(valid, NKV, hd)
        q = axial_rope64(rms(q, w[p + "self_attn.q_norm.weight"], eps), rpos, inv)
        k = axial_rope64(rms(k, w[p + "self_attn.k_norm.weight"], eps), rpos, inv)
        v = rms(v, None, eps)
        out = np.zeros((valid, NH, hd))
        for hh in range(NH):
            g = hh // (NH // NKV)
            s = q[:, hh] @ k[:, g].T
            pr = np.exp(s - s.max(1, keepdims=True))
            out[:, hh] = (pr / pr.sum(1, keepdims=True)) @ v[:, g]
        a = out.reshape(valid, NH * hd) @ f64(p + "self_attn.o_proj.linear.weight").T
        h = h + rms(a, w[p + "post_attention_layernorm.weight"], eps)
        n = rms(h, w[p + "pre_feedforward_layernorm.weight"], eps)
        act = gelu(n @ f64(p + "mlp.gate_proj.linear.weight").T) * (n @ f64(p + "mlp.up_proj.linear.weight").T)
        h = h + rms(act @ f64(p + "mlp.down_proj.linear.weight").T, w[p + "post_feedforward_layernorm.weight"], eps)
        states.append(h.copy())
    pooled = pool_patches64(h, pos, grid[0], grid[1], soft)
    proj = rms(pooled, None, eps) @ f64("embed_vision.embedding_projection.weight").T
    return dict(pooled=proj, hidden_states=np.stack(states))
