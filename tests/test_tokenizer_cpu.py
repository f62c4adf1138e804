"""The library's tokenizer (host C++ behind include/svl_hip.h) without a GPU:

* every golden case of fixtures/tokenizer/golden.json through the reduced
  tokenizer, and the unit tests of src/model/tokenizer.rs:852-1078;
* identical ids to the oracle (a literal restatement of the reference's
  quadratic merge loop) on seeded fuzz strings mixing corpus characters,
  spaces, added tokens, byte-fallback scalars and long runs;
* batch encode equal to one-by-one encode; decode(encode(x)) == x at sizes
  the oracle cannot reach (up to the 262144-symbol cap);
* the strict document validation (tokenizer.rs:102-334, json/mod.rs) and the
  error kinds of encode / decode."""
import json
import os
import time

import numpy as np
import pytest

import svl_amd as S
import svl_tokenizer as T
from oracle.tokenizer_oracle import OracleTokenizer

HERE = os.path.dirname(os.path.abspath(__file__))
TOK = os.path.join(HERE, "golden", "tokenizer")
MINI = open(os.path.join(TOK, "mini_tokenizer.json"), encoding="utf-8").read()
GOLDEN = json.load(open(os.path.join(TOK, "golden.json"), encoding="utf-8"))


@pytest.fixture(scope="module")
def tok():
    return T.Tokenizer.from_json_str(MINI)


@pytest.fixture(scope="module")
def oracle():
    return OracleTokenizer(MINI)


@pytest.mark.parametrize("case", GOLDEN["cases"], ids=lambda c: c["name"])
def test_golden_corpus(tok, case):
    assert tok.encode(case["text"], False) == case["ids"]
    assert tok.encode(case["text"], True) == case["ids_with_special"]
    assert tok.decode(case["ids_with_special"], True) == case["decoded"]


def test_reference_unit_cases(tok):
    # tokenizer.rs:862-1078
    assert tok.encode("\U0010FFFF", False) == [482, 381, 429, 429]
    assert tok.encode("<bos>hello<eos>", True) == [2, 2, 23391, 1, 1]
    assert tok.encode("", True) == [2, 1]
    assert tok.decode([2, 23391, 1], True) == "hello"
    assert tok.decode([2, 23391, 1], False) == "<bos>hello<eos>"
    assert tok.decode([258880, 496, 4429], True) == " a photo"
    assert (tok.bos_id(), tok.eos_id(), tok.unk_id(), tok.pad_id()) == (2, 1, 3, 0)
    assert tok.is_special_id(2) and not tok.is_special_id(23391)
    assert tok.token_id("<bos>") == 2 and tok.token(2) == "<bos>"
    assert tok.token_id("no such token") is None and tok.token(7) is None
    assert tok.vocab_size() == 694 and tok.max_token_id() == 258884
    assert tok.decode(tok.encode("\U0010FFFF", False), True) == "\U0010FFFF"


def fuzz_strings(n, seed):
    rng = np.random.default_rng(seed)
    chars = sorted({ch for c in GOLDEN["cases"] for ch in c["text"]})
    pieces = chars + [" ", "  ", "\n", "\t", "<bos>", "<eos>", "<|image|>", "<|tool_call>",
                      "\U0010FFFF", "é", "aaaa", "    ", "▁", "<0x41>", "<", "|"]
    out = []
    for _ in range(n):
        k = int(rng.integers(0, 60))
        out.append("".join(pieces[int(i)] for i in rng.integers(0, len(pieces), k)))
    return out


def test_fuzz_against_the_oracle(tok, oracle):
    texts = fuzz_strings(400, 1)
    for t in texts:
        for special in (False, True):
            assert tok.encode(t, special) == oracle.encode(t, special), repr(t)
        ids = tok.encode(t, False)
        # the decoder maps the space marker back to a space (tokenizer.rs:409-415)
        assert tok.decode(ids, False) == oracle.decode(ids, False) == t.replace("▁", " ")
        assert tok.decode(ids, True) == oracle.decode(ids, True)
    assert tok.encode_batch(texts, True) == [tok.encode(t, True) for t in texts]


def test_long_runs_against_the_oracle(tok, oracle):
    for text in ("a" * 1500, " " * 700, "ab" * 400 + "   " + "b" * 300, "\t\n " * 200):
        assert tok.encode(text, True) == oracle.encode(text, True)


def test_large_inputs_round_trip_quickly(tok):
    """Inputs just under the 262144-symbol cap (checked before merging,
    tokenizer.rs:517-521): the heap merge keeps them fast."""
    big = "".join(fuzz_strings(30000, 3))[:200000]
    t0 = time.perf_counter()
    ids = tok.encode(big, False)
    dt = time.perf_counter() - t0
    assert tok.decode(ids, False) == big.replace("▁", " ")
    run = "a" * 262144
    t0 = time.perf_counter()
    ids_run = tok.encode(run, False)
    dt_run = time.perf_counter() - t0
    assert tok.decode(ids_run, False) == run
    print(f"{len(big)} mixed chars: {len(ids)} ids in {dt * 1e3:.1f} ms; 262144-char run: "
          f"{len(ids_run)} ids in {dt_run * 1e3:.1f} ms")
    assert dt < 5 and dt_run < 5
    with pytest.raises(S.SvlError) as e:
        tok.encode("a" * 262145, False)
    assert e.value.kind == "LimitExceeded"


def test_encode_limits_and_errors(tok):
    with pytest.raises(S.SvlError) as e:
        tok.encode("a" * (1024 * 1024 + 1), False)
    assert e.value.kind == "LimitExceeded"
    with pytest.raises(S.SvlError) as e:   # 270000 byte-fallback symbols > 262144 tokens
        tok.encode("\x01" * 270000, False)
    assert e.value.kind == "LimitExceeded"
    with pytest.raises(S.SvlError) as e:
        tok.encode(b"abc\xff", False)
    assert e.value.kind == "Corrupt"
    with pytest.raises(S.SvlError) as e:
        tok.decode([2**32 - 1], True)
    assert e.value.kind == "Corrupt"
    with pytest.raises(S.SvlError) as e:   # a lone continuation byte
        tok.decode([tok.token_id("<0xBF>")], True)
    assert e.value.kind == "Corrupt"
    with pytest.raises(S.SvlError) as e:
        tok.encode_batch(["fine", "a" * (1024 * 1024 + 1)], False)
    assert e.value.kind == "LimitExceeded" and "text 1" in str(e.value)


def _mutated(**changes):
    doc = json.loads(MINI)
    for path, value in changes.items():
        node = doc
        keys = path.split("__")
        for k in keys[:-1]:
            node = node[int(k)] if isinstance(node, list) else node[k]
        last = int(keys[-1]) if isinstance(node, list) else keys[-1]
        if value is KeyError:
            del node[last]
        else:
            node[last] = value
    return json.dumps(doc, ensure_ascii=False)


@pytest.mark.parametrize("doc,kind", [
    ("{}", "Corrupt"),
    ('{"model":{"type":"Unigram"}}', "Unsupported"),
    (_mutated(model__type="Unigram"), "Unsupported"),
    (_mutated(model__byte_fallback=False), "Unsupported"),
    (_mutated(model__fuse_unk=False), "Unsupported"),
    (_mutated(model__ignore_merges=True), "Unsupported"),
    (_mutated(model__dropout=0.1), "Unsupported"),
    (_mutated(model__continuing_subword_prefix="##"), "Unsupported"),
    (_mutated(model__byte_fallback=KeyError), "Corrupt"),
    (_mutated(model__unk_token="<nope>"), "Corrupt"),
    (_mutated(normalizer__content="_"), "Unsupported"),
    (_mutated(pre_tokenizer__behavior="Isolated"), "Unsupported"),
    (_mutated(pre_tokenizer__invert=True), "Unsupported"),
    (_mutated(post_processor__type="BertProcessing"), "Unsupported"),
    (_mutated(decoder__decoders__1__type="Strip"), "Unsupported"),
    (_mutated(added_tokens__0__id=999999999), "Corrupt"),
    (_mutated(added_tokens__1__id=0), "Corrupt"),
    (_mutated(added_tokens__0__content=""), "Corrupt"),
    (_mutated(model__merges__0=["▁▁▁", "zzzz"]), "Corrupt"),
    (_mutated(model__merges__0=["a"]), "Corrupt"),
    (_mutated(model__vocab___stray=2 ** 33), "LimitExceeded"),  # fits u64, not u32
    (_mutated(model__vocab___stray=5 ** 30), "Corrupt"),        # beyond u64: a float
    (_mutated(model__vocab___stray=-1), "Corrupt"),
    (_mutated(model__vocab___stray=2), "Corrupt"),            # duplicate id
], ids=lambda v: v[:40] if isinstance(v, str) and len(v) > 40 else None)
def test_document_validation(doc, kind):
    with pytest.raises(S.SvlError) as e:
        T.Tokenizer.from_json_str(doc)
    assert e.value.kind == kind, e.value


def test_missing_byte_token_and_space_marker():
    doc = json.loads(MINI)
    del doc["model"]["vocab"]["<0x41>"]
    doc["model"]["merges"] = [m for m in doc["model"]["merges"] if "<0x41>" not in m]
    with pytest.raises(S.SvlError) as e:
        T.Tokenizer.from_json_str(json.dumps(doc))
    assert e.value.kind == "Corrupt" and "0x41" in str(e.value)


@pytest.mark.parametrize("text,kind", [
    ('{"a": 1, "a": 2}', "Corrupt"),          # duplicate key
    ('{"a": [1, 2,]}', "Corrupt"),            # trailing comma
    ('{"a": 01}', "Corrupt"),                 # leading zero
    ('{"a": "\\ud800"}', "Corrupt"),          # lone surrogate
    ('{"a": "x\x01y"}', "Corrupt"),           # unescaped control character
    ('{"a": 1} x', "Corrupt"),                # trailing content
    ('{"a": 1e999}', "Corrupt"),              # non-finite number
    ("[" * 70 + "]" * 70, "LimitExceeded"),   # depth cap 64
    (b'{"a": "\xff"}', "Corrupt"),            # not UTF-8
])
def test_json_strictness(text, kind):
    with pytest.raises(S.SvlError) as e:
        T.Tokenizer.from_json_str(text)
    assert e.value.kind == kind, e.value


def test_json_escapes_reach_the_vocabulary():
    # \u escapes, surrogate pairs and "\/" decode to the same strings
    doc = MINI.replace('"\\t":', '"\\u0009":', 1)
    assert doc != MINI
    t = T.Tokenizer.from_json_str(doc)
    assert t.encode("a\nb\tc", False) == [236746, 107, 236763, 255968, 236755]


def test_prompts():
    # prompt.rs:104-160
    assert T.Prompt.SearchQuery.prefix() == "task: search result | query: "
    assert T.Prompt.Document.prefix() == "title: none | text: "
    assert T.Prompt.from_name("CodeRetrieval") is T.Prompt.CodeRetrieval
    assert T.Prompt.from_name("searchquery") is None
    assert T.Prompt.SearchQuery.is_query() and not T.Prompt.Document.is_query()
