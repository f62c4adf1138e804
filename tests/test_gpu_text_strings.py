"""GPU parity of TextEmbedder::embed (src/model/text.rs:610-626) over raw
strings through the C ABI: prompt prefix, the library's tokenizer (the
reduced official tokenizer, whose ids reach 258884), the 8192-token context
check, one batched forward pass, Matryoshka truncation.

* the string path equals the ids path (svl_text_embed_ids on the oracle
  tokenizer's ids of the prefixed text) bit for bit;
* the embeddings match the CPU oracle's forward pass at max-abs 1e-4 and
  cosine 0.99999;
* a batch equals one-by-one calls; the error taxonomy of embed."""
import os

import numpy as np
import pytest

import svl_amd as S
import svl_synth
import svl_tokenizer as T
from oracle import oracle as O
from oracle.tokenizer_oracle import OracleTokenizer

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
MINI = open(os.path.join(HERE, "golden", "tokenizer", "mini_tokenizer.json"),
            encoding="utf-8").read()
TEXTS = ["hello", "Bonjour, le monde !", "The quick brown fox jumps over the lazy dog.",
         "<|image|> a photo", "", "café naïve façade 😀 emoji 日本語のテキスト"]


@pytest.fixture(scope="module")
def setup():
    cfg = svl_synth.config_a(layers=2, vocab=262144)
    w = svl_synth.weights(cfg, seed=21)
    model = S.TextModel(S.TextConfig.from_json_value(cfg), w)
    emb = T.TextEmbedder.from_parts(model, T.Tokenizer.from_json_str(MINI))
    return cfg, w, model, emb


def test_strings_match_ids_path_and_oracle(setup):
    cfg, w, model, emb = setup
    ot, om = OracleTokenizer(MINI), O.OracleTextModel(cfg, w)
    for prompt in (T.Prompt.SearchQuery, T.Prompt.Document):
        got = emb.embed_batch(TEXTS, prompt, 768)
        for i, text in enumerate(TEXTS):
            ids = ot.encode(prompt.prefix() + text, True)
            one = np.empty(768, np.float32)
            a = np.ascontiguousarray(ids, np.uint32)
            S._check(S.lib().svl_text_embed_ids(model.handle, S._ptr(a), a.size, 768,
                                                S._ptr(one)))
            assert np.array_equal(got[i], one), f"{prompt.name} text {i}"
            ref = O.truncate_and_normalize(om.forward(ids)["normalized"], 768)
            d = float(np.abs(got[i] - ref).max())
            c = float(got[i].astype(np.float64) @ ref / np.linalg.norm(ref) /
                      np.linalg.norm(got[i].astype(np.float64)))
            print(f"{prompt.name} text {i} ({len(ids)} ids): max-abs {d:.3g} cosine {c:.9f}",
                  flush=True)
            assert d <= 1e-4 and c >= 0.99999
    for dim in (128, 256):
        small = emb.embed_batch(TEXTS[:2], T.Prompt.SearchQuery, dim)
        for i in range(2):
            assert np.array_equal(small[i], emb.embed(TEXTS[i], T.Prompt.SearchQuery, dim))


def test_embed_errors(setup):
    cfg, w, model, emb = setup
    with pytest.raises(S.SvlError) as e:       # text.rs:619-624
        emb.embed("hello " * 9000, T.Prompt.Document, 768)
    assert e.value.kind == "LimitExceeded"
    for dim in (0, 769):                       # text.rs:546-552
        with pytest.raises(S.SvlError) as e:
            emb.embed("hello", T.Prompt.Document, dim)
        assert e.value.kind == "Internal"
    with pytest.raises(S.SvlError) as e:       # TextEmbedder::from_files vocabulary check
        T.TextEmbedder(model, T.Tokenizer.from_json_str(MINI))
    assert e.value.kind == "Corrupt"
