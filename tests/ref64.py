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
