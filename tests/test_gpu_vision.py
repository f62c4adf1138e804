"""GPU parity of the vision tower (VisionModel::forward, src/model/vision.rs:
742-959) and of the image prompt glue (ImageEmbedder::embed_impl,
src/model/image.rs:209-253) through the C ABI.

* a small random tower (hidden 64, 4 heads / 2 KV heads of dim 16: the
  generic attention kernel) and config V at 2 layers (12 heads of dim 64: the
  MFMA attention kernel) against the CPU oracle, image by image, over ragged
  batches with padding rows;
* config V at full depth on a full 768 x 768 image (48 x 48 patches): every
  stage checked from the GPU's own input to it (the patch embedding, pooling
  and projection in float64; layers 1 / 8 / 16 by the oracle's single-layer
  path, since the whole oracle tower needs minutes at that size), the
  260-token image prompt through the 24-layer shape-A text encoder against
  the text oracle, and a four-image batch bit-identical to single calls;
* batching and device-resident variants bit-identical to single calls;
* the image embedder (tower + prompt + text encoder with soft tokens)
  against the oracle chain at Matryoshka dims 768 and 128;
* the error taxonomy of vision.rs / image.rs."""
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

import ref64
import svl_amd as S
import svl_synth
import svl_vision as V
from oracle import oracle as O

pytestmark = pytest.mark.gpu

MAX_ABS = 1e-4
MIN_COS = 0.99999


def cosine(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))


def small_config(layers=2):
    c = svl_synth.config_v(layers)
    c["vision_config"].update(hidden_size=64, intermediate_size=96, num_attention_heads=4,
                              num_key_value_heads=2, head_dim=16, position_embedding_size=16)
    return c


def build(c, text_hidden, seed=7):
    w = svl_synth.vision_weights(c, text_hidden, seed=seed)
    gpu = V.VisionModel(V.VisionConfig.from_json_value(c), w, text_hidden)
    return w, gpu, O.OracleVisionModel(c, w, text_hidden)


def oracle_all(om, patches, capture=False):
    with ThreadPoolExecutor(max_workers=min(8, len(patches))) as ex:
        return list(ex.map(lambda p: om.forward(p, capture_hidden=capture), patches))


def check_soft(got, want, label):
    d = float(np.abs(got - want).max())
    c = cosine(got, want)
    print(f"{label}: soft tokens {got.shape} max-abs {d:.3g} cosine {c:.9f}", flush=True)
    assert d <= MAX_ABS and c >= MIN_COS, f"{label}: max-abs {d:.3g} cosine {c:.9f}"


@pytest.fixture(scope="module")
def small():
    return build(small_config(), 48)


@pytest.fixture(scope="module")
def tower_v2():
    return build(svl_synth.config_v(2), 768, seed=11)


def test_small_tower_matches_oracle(small):
    w, gpu, om = small
    patches = [svl_synth.image_patches(1, 6, 9, seed=21, max_patches=63)[0],
               svl_synth.image_patches(1, 9, 6, seed=22)[0]]
    got = gpu.forward_batch(patches, capture_hidden=True)
    want = oracle_all(om, patches, capture=True)
    for i, (g, o) in enumerate(zip(got, want)):
        assert g.soft_tokens() == o["soft_tokens"] == 6
        hs = np.stack(g.hidden_states())
        np.testing.assert_allclose(hs, o["hidden_states"], rtol=1e-4, atol=1e-4)
        check_soft(g.pooled(), o["pooled"], f"small image {i}")


def test_config_v_two_layers_matches_oracle(tower_v2):
    w, gpu, om = tower_v2
    patches = [svl_synth.image_patches(1, 12, 12, seed=31, max_patches=160)[0],
               svl_synth.image_patches(1, 9, 15, seed=32)[0],
               svl_synth.image_patches(1, 6, 6, seed=33)[0]]
    got = gpu.forward_batch(patches, capture_hidden=True)
    want = oracle_all(om, patches, capture=True)
    for i, (g, o) in enumerate(zip(got, want)):
        hs = np.stack(g.hidden_states())
        d = np.abs(hs - o["hidden_states"]).max(axis=(1, 2))
        print(f"image {i}: per-layer hidden max-abs {d}", flush=True)
        np.testing.assert_allclose(hs, o["hidden_states"], rtol=1e-4, atol=2e-4)
        check_soft(g.pooled(), o["pooled"], f"config V image {i}")


def test_batch_is_bit_identical_to_single_calls(tower_v2):
    w, gpu, om = tower_v2
    patches = svl_synth.image_patches(3, 12, 9, seed=41)
    patches.append(svl_synth.image_patches(1, 6, 15, seed=42)[0])
    batch = gpu.forward_batch(patches)
    for i, p in enumerate(patches):
        one = gpu.forward(p).pooled()
        assert np.array_equal(one, batch[i].pooled()), f"image {i}"
    again = gpu.forward_batch(patches[::-1])
    for i, p in enumerate(patches[::-1]):
        assert np.array_equal(again[i].pooled(), batch[len(patches) - 1 - i].pooled())


def test_image_groups_are_bit_identical(tower_v2):
    # Batches of two or more images and 4096 or more patches run the encoder
    # layers as two image groups on two streams: here images 0-1 (2304 + 1296
    # patches) against images 2-3 (2304 + 576).
    w, gpu, om = tower_v2
    patches = [svl_synth.image_patches(1, 48, 48, seed=61)[0],
               svl_synth.image_patches(1, 36, 36, seed=62)[0],
               svl_synth.image_patches(1, 48, 48, seed=63)[0],
               svl_synth.image_patches(1, 24, 24, seed=64)[0]]
    split = gpu.forward_batch(patches)
    gpu.set_stream_split(1)
    try:
        single = gpu.forward_batch(patches)
    finally:
        gpu.set_stream_split(2)
    captured = gpu.forward_batch(patches, capture_hidden=True)  # one group while capturing
    for i in range(4):
        assert np.array_equal(split[i].pooled(), single[i].pooled()), f"image {i}"
        assert np.array_equal(split[i].pooled(), captured[i].pooled()), f"image {i}"
    assert np.array_equal(gpu.forward(patches[2]).pooled(), split[2].pooled())


def test_device_resident_matches_host(tower_v2):
    import torch
    w, gpu, om = tower_v2
    patches = svl_synth.image_patches(2, 12, 12, seed=51)
    host = np.concatenate([p.pooled() for p in gpu.forward_batch(patches)])
    pix = np.concatenate([p.pixel_values[: p.valid_patches] for p in patches])
    d_pix = torch.from_numpy(pix).to("cuda:0")
    d_out = torch.empty((sum(p.soft_tokens for p in patches), 768), device="cuda:0")
    torch.cuda.synchronize()
    gpu.forward_device(d_pix.data_ptr(), patches, d_out.data_ptr())
    assert np.array_equal(d_out.cpu().numpy(), host)


def test_batches_run_in_passes_bit_for_bit(tower_v2, embedder):
    """A batch whose workspace would pass the budget runs as passes of
    consecutive images. At a 300-patch budget the images below (108, 144, 324,
    90 and 108 patches) take three passes, the 324-patch image alone, and with
    a 30-token text budget their prompts (16, 20, 40, 14 and 16 tokens) take
    the text encoder in four passes. The soft tokens, the captured hidden
    states, the device entry point and the image embedder equal the one-pass
    run bit for bit."""
    import torch
    w, gpu, om = tower_v2
    emb, _, _ = embedder
    grids = [(12, 9), (12, 12), (18, 18), (6, 15), (9, 12)]
    patches = [svl_synth.image_patches(1, gw, gh, seed=71 + i)[0] for i, (gw, gh) in enumerate(grids)]
    pix = np.concatenate([p.pixel_values[: p.valid_patches] for p in patches])
    soft = sum(p.soft_tokens for p in patches)
    runs = []
    for budget in (0, 300):
        gpu.set_pass_patches(budget)
        emb.vision.set_pass_patches(budget)
        emb.model.set_pass_tokens(30 if budget else 0)
        try:
            host = gpu.forward_batch(patches, capture_hidden=True)
            d_pix = torch.from_numpy(pix).to("cuda:0")
            d_out = torch.empty((soft, 768), device="cuda:0")
            torch.cuda.synchronize()
            gpu.forward_device(d_pix.data_ptr(), patches, d_out.data_ptr())
            runs.append((host, d_out.cpu().numpy(), emb.embed_batch(patches, 768)))
        finally:
            gpu.set_pass_patches(0)
            emb.vision.set_pass_patches(0)
            emb.model.set_pass_tokens(0)
    (h1, d1, e1), (h2, d2, e2) = runs
    for i in range(len(patches)):
        assert h1[i].pooled().tobytes() == h2[i].pooled().tobytes(), f"image {i}"
        assert (np.stack(h1[i].hidden_states()).tobytes() ==
                np.stack(h2[i].hidden_states()).tobytes()), f"image {i}"
    assert d1.tobytes() == d2.tobytes()
    assert e1.tobytes() == e2.tobytes()
    with pytest.raises(S.SvlError) as e:
        gpu.set_pass_patches(-1)
    assert e.value.kind == "Usage"


@pytest.fixture(scope="module")
def full_v():
    """Config V at 16 layers and one 768 x 768 noise image (2304 patches, 256
    soft tokens), run once on the GPU with every hidden state captured."""
    c = svl_synth.config_v(16)
    w = svl_synth.vision_weights(c, 768, seed=13)
    gpu = V.VisionModel(V.VisionConfig.from_json_value(c), w, 768)
    p = svl_synth.image_patches(1, 48, 48, seed=2)[0]
    out = gpu.forward(p, capture_hidden=True)
    return c, w, gpu, p, out


def test_full_size_image_every_stage(full_v):
    """Config V, 16 layers, one 768 x 768 image (2304 patches, 256 soft
    tokens). Each checked stage is computed from the GPU's own input to that
    stage: the patch embedding in float64, layers 1, 8 and 16 by the oracle's
    single-layer path (the forward pass's own per-layer code; the whole
    oracle tower needs minutes at this size), and the pool, unscaled norm and
    projection in float64."""
    c, w, gpu, p, out = full_v
    hs = out.hidden_states()
    assert len(hs) == 17 and hs[0].shape == (2304, 768)
    assert out.pooled().shape == (256, 768)
    vc = O.resolve_vision_config(c)
    pos = p.positions[:2304]
    om = O.OracleVisionModel(c, w, 768)

    def rel(g, r):
        return float(np.abs(np.asarray(g, np.float64) - r).max() / np.abs(r).max())

    with ThreadPoolExecutor(max_workers=3) as ex:
        layers = {l: ex.submit(om.layer, l - 1, hs[l - 1], pos) for l in (1, 8, 16)}

        # patch embedding + position add
        pe = (2.0 * (p.pixel_values[:2304].astype(np.float64) - 0.5)) @ \
            w["vision_tower.patch_embedder.input_proj.weight"].astype(np.float64).T
        table = w["vision_tower.patch_embedder.position_embedding_table"].astype(np.float64)
        pe += table[0][pos[:, 0]] + table[1][pos[:, 1]]
        e = rel(hs[0], pe)
        print(f"patch embedding: relative max error {e:.3g}", flush=True)
        assert e <= 1e-5

        # pool + unscaled norm + projection from the GPU's last hidden state
        pooled = ref64.pool_patches64(hs[16].astype(np.float64), pos, 48, 48, 256)
        soft = ref64.rms(pooled, None, vc["rms_norm_eps"]) @ \
            w["embed_vision.embedding_projection.weight"].astype(np.float64).T
        d = float(np.abs(out.pooled() - soft).max())
        c_ = cosine(out.pooled(), soft)
        print(f"soft tokens: max-abs {d:.3g} cosine {c_:.9f}", flush=True)
        assert d <= MAX_ABS and c_ >= MIN_COS
        assert np.isfinite(out.pooled()).all()

        for l, f in layers.items():
            e = rel(hs[l], f.result())
            print(f"layer {l} against the oracle layer: relative max error {e:.3g}", flush=True)
            assert e <= 1e-4


def test_full_size_image_prompt_through_the_text_encoder(full_v):
    """The 260-token image prompt of one 768 x 768 image through the 24-layer
    shape-A text encoder (vocab 262144, the reference's special-token ids)
    against the text oracle run on the GPU tower's own soft tokens
    (image.rs:209-253), at Matryoshka dims 768 and 128."""
    c, w, gpu, p, out = full_v
    tc = svl_synth.config_a()
    tw = svl_synth.weights(tc, seed=0)
    tm = S.TextModel(S.TextConfig.from_json_value(tc), tw)
    tokens = V.ImageSpecialTokens()
    emb = V.ImageEmbedder(tm, gpu, tokens)
    got = {d: emb.embed_patches(p, d) for d in (768, 128)}
    ids = [tokens.bos, tokens.boi] + [tokens.image] * 256 + [tokens.eoi, tokens.eos]
    ref = O.OracleTextModel(tc, tw).forward(ids, features=out.pooled(), feature_start=2,
                                            feature_count=256)["normalized"]
    for d in (768, 128):
        r = O.truncate_and_normalize(ref, d)
        diff = float(np.abs(got[d] - r).max())
        c_ = cosine(got[d], r)
        print(f"260-token image prompt dim {d}: max-abs {diff:.3g} cosine {c_:.9f}", flush=True)
        assert diff <= MAX_ABS and c_ >= MIN_COS
    tm.close()


def test_four_full_size_images_equal_single_calls(full_v):
    """A batch of four 768 x 768 images through the 16-layer tower returns,
    image by image, the bits of four single calls."""
    c, w, gpu, p, out = full_v
    patches = [p] + svl_synth.image_patches(3, 48, 48, seed=5)
    batch = gpu.forward_batch(patches)
    assert np.array_equal(batch[0].pooled(), out.pooled())
    for i in (1, 3):
        assert np.array_equal(batch[i].pooled(), gpu.forward(patches[i]).pooled()), i


# ---- image prompt glue ----------------------------------------------------------------

TOKENS = V.ImageSpecialTokens(bos=2, eos=1, pad=0, boi=1000, image=1001, eoi=1002)


@pytest.fixture(scope="module")
def embedder():
    tc = svl_synth.config_a(layers=2, vocab=1024)
    c = svl_synth.config_v(2, text=tc)
    tw = svl_synth.weights(tc, seed=3)
    vw = svl_synth.vision_weights(c, 768, seed=17)
    tm = S.TextModel(S.TextConfig.from_json_value(tc), tw)
    vm = V.VisionModel(V.VisionConfig.from_json_value(c), vw, 768)
    return (V.ImageEmbedder(tm, vm, TOKENS), O.OracleTextModel(tc, tw),
            O.OracleVisionModel(c, vw, 768))


def test_image_embedder_matches_oracle(embedder):
    emb, ot, ov = embedder
    patches = [svl_synth.image_patches(1, 12, 12, seed=61)[0],
               svl_synth.image_patches(1, 9, 6, seed=62)[0]]
    for dim in (768, 128):
        got = emb.embed_batch(patches, dim)
        for i, p in enumerate(patches):
            soft = ov.forward(p)["pooled"]
            ids = [TOKENS.bos, TOKENS.boi] + [TOKENS.image] * p.soft_tokens + [TOKENS.eoi,
                                                                                TOKENS.eos]
            ref = ot.forward(ids, features=soft, feature_start=2,
                             feature_count=p.soft_tokens)["normalized"]
            ref = O.truncate_and_normalize(ref, dim)
            d = float(np.abs(got[i] - ref).max())
            c = cosine(got[i], ref)
            print(f"image {i} dim {dim}: max-abs {d:.3g} cosine {c:.9f}", flush=True)
            assert d <= MAX_ABS and c >= MIN_COS
    one = emb.embed_patches(patches[1], 768)
    batch = emb.embed_batch(patches, 768)
    assert np.array_equal(one, batch[1])
    import torch
    pix = np.concatenate([p.pixel_values[: p.valid_patches] for p in patches])
    d_pix = torch.from_numpy(pix).to("cuda:0")
    torch.cuda.synchronize()
    assert np.array_equal(emb.embed_device(d_pix.data_ptr(), patches, 768), batch)


def test_image_embedder_rejects_bad_dimensions(embedder):
    emb, _, _ = embedder
    p = svl_synth.image_patches(1, 6, 6, seed=63)[0]
    for dim in (0, 769):
        with pytest.raises(S.SvlError) as e:
            emb.embed_patches(p, dim)
        assert e.value.kind == "Internal"


# ---- error taxonomy ---------------------------------------------------------------------

def test_vision_error_taxonomy(small):
    w, gpu, om = small

    def fresh():
        return svl_synth.image_patches(1, 6, 6, seed=71)[0]

    p = fresh()
    p.valid_patches = 0
    with pytest.raises(S.SvlError) as e:
        gpu.forward(p)
    assert e.value.kind == "Corrupt"
    p = fresh()
    p.positions[3] = [16, 0]
    with pytest.raises(S.SvlError) as e:
        gpu.forward(p)
    assert e.value.kind == "Corrupt"
    p = fresh()
    p.positions[2] = [-1, 0]
    with pytest.raises(S.SvlError) as e:
        gpu.forward(p)
    assert e.value.kind == "Internal"
    p = fresh()
    p.patch_grid = (4, 9)
    with pytest.raises(S.SvlError) as e:
        gpu.forward(p)
    assert e.value.kind == "Internal"
    p = fresh()
    p.max_patches = 10
    with pytest.raises(S.SvlError) as e:
        gpu.forward(p)
    assert e.value.kind == "Internal"
    # the model still works after rejected calls
    ok = gpu.forward(fresh()).pooled()
    assert np.isfinite(ok).all()


def test_vision_weight_inventory(small):
    w, gpu, om = small
    c = small_config()
    vc = V.VisionConfig.from_json_value(c)
    missing = dict(w)
    del missing["vision_tower.encoder.layers.1.mlp.up_proj.linear.weight"]
    with pytest.raises(S.SvlError) as e:
        V.VisionModel(vc, missing, 48)
    assert e.value.kind == "Corrupt"
    extra = dict(w)
    extra["vision_tower.encoder.layers.2.input_layernorm.weight"] = np.ones(64, np.float32)
    with pytest.raises(S.SvlError) as e:
        V.VisionModel(vc, extra, 48)
    assert e.value.kind == "Corrupt"
    bad = dict(w)
    bad["embed_vision.embedding_projection.weight"] = np.zeros((47, 64), np.float32)
    with pytest.raises(S.SvlError) as e:
        V.VisionModel(vc, bad, 48)
    assert e.value.kind == "Corrupt"


# ---- the closed forms that pin the oracle, on the GPU ----------------------------------

def test_gpu_tower_meets_the_closed_forms():
    """Config V at 2 layers on the two degenerate weight sets of the oracle's
    closed-form pins: with zero projections every GPU layer is the identity
    (bit for bit) and the soft tokens are the closed form of embedding,
    pooling, unscaled norm and projection; with identical patches and a zero
    position table every layer is the one-row closed form."""
    import test_oracle_vision as TV
    c = svl_synth.config_v(2)
    vc = O.resolve_vision_config(c)
    H = vc["hidden_size"]
    w = dict(svl_synth.vision_weights(c, 768, seed=21))
    for l in range(2):
        for n in ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
                  "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj"):
            k = TV.L_.format(l) + n + ".linear.weight"
            w[k] = np.zeros_like(w[k])
    s = np.float32(3e-3 / np.sqrt(H))
    w[TV.W_IN] = (w[TV.W_IN] * s).astype(np.float32)
    w[TV.TABLE] = (w[TV.TABLE] * s).astype(np.float32)
    gpu = V.VisionModel(V.VisionConfig.from_json_value(c), w, 768)
    p = svl_synth.image_patches(1, 12, 9, seed=31)[0]
    out = gpu.forward(p, capture_hidden=True)
    hs = out.hidden_states()
    for l in (1, 2):
        assert np.array_equal(hs[l], hs[0]), f"layer {l} is not the identity"
    n = p.valid_patches
    h0 = TV._embedding_closed_form(w, p.pixel_values[:n], p.positions[:n])
    assert TV._rel(hs[0], h0) <= 1e-5
    want = TV._soft_closed_form(vc, w, h0, p.positions[:n], p.patch_grid, p.soft_tokens)
    e = TV._rel(out.pooled(), want)
    print(f"zero projections: soft tokens relative max error {e:.3g}", flush=True)
    assert e <= 1e-4
    gpu.close()

    w = dict(svl_synth.vision_weights(c, 768, seed=22))
    w[TV.TABLE] = np.zeros_like(w[TV.TABLE])
    gpu = V.VisionModel(V.VisionConfig.from_json_value(c), w, 768)
    p = svl_synth.image_patches(1, 12, 12, seed=32)[0]
    p.pixel_values[:] = p.pixel_values[0]
    out = gpu.forward(p, capture_hidden=True)
    hs = out.hidden_states()
    h = TV._embedding_closed_form(w, p.pixel_values[:1], p.positions[:1])[0]
    for l in range(2):
        h = TV._layer_one_row(vc, w, l, h)
        e = TV._rel(hs[l + 1], np.broadcast_to(h, hs[l + 1].shape))
        print(f"identical patches: layer {l + 1} relative max error {e:.3g}", flush=True)
        assert e <= 1e-4
    gpu.close()
