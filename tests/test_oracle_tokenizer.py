"""Pins of the tokenizer oracle (oracle/tokenizer_oracle.py, a restatement of
src/model/tokenizer.rs): every case of fixtures/tokenizer/golden.json (ids
from the official `tokenizers` library) through the reduced tokenizer, and
the unit tests of tokenizer.rs:852-1078."""
import json
import os

import pytest

from oracle.tokenizer_oracle import OracleTokenizer, TokenizerError

HERE = os.path.dirname(os.path.abspath(__file__))
TOK = os.path.join(HERE, "golden", "tokenizer")
MINI = open(os.path.join(TOK, "mini_tokenizer.json"), encoding="utf-8").read()
GOLDEN = json.load(open(os.path.join(TOK, "golden.json"), encoding="utf-8"))


@pytest.fixture(scope="module")
def tok():
    return OracleTokenizer(MINI)


@pytest.mark.parametrize("case", GOLDEN["cases"], ids=lambda c: c["name"])
def test_golden_corpus(tok, case):
    assert tok.encode(case["text"], False) == case["ids"]
    assert tok.encode(case["text"], True) == case["ids_with_special"]
    assert tok.decode(case["ids_with_special"], True) == case["decoded"]


def test_reference_unit_cases(tok):
    # tokenizer.rs:862-889 encodes_reference_texts
    cases = [
        ("hello", [23391]), ("Hello, world!", [9259, 236764, 1902, 236888]),
        ("Bonjour, le monde !", [53406, 236764, 674, 22150, 1717]), ("café", [123125, 236859]),
        ("😀 emoji", [242398, 64334]), ("  leading spaces", [138, 26016, 9952]),
        ("multiple   spaces", [43819, 139, 35220]),
        ("a\nb\tc", [236746, 107, 236763, 255968, 236755]), ("<bos>hello<eos>", [2, 23391, 1]),
        ("<|image|> a photo", [258880, 496, 4429]), ("\U0010FFFF", [482, 381, 429, 429]),
    ]
    for text, ids in cases:
        assert tok.encode(text, False) == ids, text
    # :892-904, :925-944
    assert tok.encode("", True) == [2, 1]
    assert tok.encode("<bos>hello<eos>", True) == [2, 2, 23391, 1, 1]
    assert tok.decode([2, 23391, 1], False) == "<bos>hello<eos>"
    assert tok.decode([258880, 496, 4429], True) == " a photo"
    assert (tok.bos_id, tok.eos_id, tok.unk_id, tok.pad_id) == (2, 1, 3, 0)
    assert len(tok.vocab) == 694 and max(tok.id_to_token) == 258884
    with pytest.raises(TokenizerError) as e:
        tok.decode([2**32 - 1], True)
    assert e.value.kind == "Corrupt"
    with pytest.raises(TokenizerError) as e:
        tok.encode("a" * (1024 * 1024 + 1), False)
    assert e.value.kind == "LimitExceeded"
    assert tok.decode(tok.encode("\U0010FFFF", False), True) == "\U0010FFFF"
