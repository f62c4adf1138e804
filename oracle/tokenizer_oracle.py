"""CPU oracle, tokenizer: a pure-Python restatement of src/model/tokenizer.rs.

TEST INFRASTRUCTURE ONLY: the oracle for the library's C++ tokenizer, never
part of the product. It follows the reference step by step, including its
quadratic merge loop (best_merge scans every adjacent pair, then one
left-to-right pass merges every occurrence; tokenizer.rs:497-552), so it is
meant for the golden corpus and short fuzz strings.

Parity pins (tests/test_oracle_tokenizer.py): all 21 cases of
fixtures/tokenizer/golden.json (ids, ids with <bos>/<eos>, decoded text;
produced by the official `tokenizers` library) through the reduced
fixtures/tokenizer/mini_tokenizer.json, and the unit tests of
tokenizer.rs:852-1078.
"""
from __future__ import annotations

import json

SPACE_MARKER = "▁"
MAX_INPUT_BYTES = 1024 * 1024           # tokenizer.rs:37
MAX_TOKENS = 262_144                    # tokenizer.rs:43


class TokenizerError(Exception):
    def __init__(self, kind, message):
        super().__init__(f"{kind}: {message}")
        self.kind = kind


def _byte_token(token):
    """parse_byte_token (tokenizer.rs:825-832)."""
    if len(token.encode()) != 6 or not token.startswith("<0x") or not token.endswith(">"):
        return None
    digits = token[3:5]
    if digits.startswith("+"):
        digits = digits[1:]
    try:
        if not all(c in "0123456789abcdefABCDEF" for c in digits) or not digits:
            return None
        return int(digits, 16)
    except ValueError:
        return None


class OracleTokenizer:
    """Tokenizer::from_json (tokenizer.rs:102-334) for a well-formed
    document; validation beyond what the fixtures need is the library's."""

    def __init__(self, document: str | dict):
        root = json.loads(document) if isinstance(document, str) else document
        model = root["model"]
        if model["type"] != "BPE":
            raise TokenizerError("Unsupported", "only BPE is implemented")
        self.vocab = dict(model["vocab"])
        self.id_to_token = {i: t for t, i in self.vocab.items()}
        self.char_ids = {t: i for t, i in self.vocab.items() if len(t) == 1}
        self.byte_ids = [self.vocab[f"<0x{b:02X}>"] for b in range(256)]
        self.merges = {}
        for rank, (left, right) in enumerate(model["merges"]):
            self.merges[(self.vocab[left], self.vocab[right])] = (rank, self.vocab[left + right])
        self.unk_id = self.vocab[model["unk_token"]]
        self.added = []
        self.special = set()
        for a in root["added_tokens"]:
            self.added.append((a["content"], a["id"]))
            if a["special"]:
                self.special.add(a["id"])
        self.added.sort(key=lambda a: (-len(a[0].encode()), a[1]))
        self.bos_id, self.eos_id = self.vocab["<bos>"], self.vocab["<eos>"]
        self.pad_id = self.vocab.get("<pad>")

    def encode(self, text: str, add_special_tokens: bool):
        """Tokenizer::encode (tokenizer.rs:339-389)."""
        if len(text.encode()) > MAX_INPUT_BYTES:
            raise TokenizerError("LimitExceeded", "input cap")
        ids = [self.bos_id] if add_special_tokens else []
        segment = []
        i = 0
        while i < len(text):
            rest = text[i:]
            match = next((a for a in self.added if rest.startswith(a[0])), None)
            if match is not None:
                if segment:
                    self._encode_segment("".join(segment), ids)
                    segment = []
                ids.append(match[1])
                self._check(len(ids))
                i += len(match[0])
            else:
                segment.append(text[i])
                i += 1
        if segment:
            self._encode_segment("".join(segment), ids)
        if add_special_tokens:
            ids.append(self.eos_id)
        self._check(len(ids))
        return ids

    def _encode_segment(self, segment, ids):
        """encode_segment + best_merge (tokenizer.rs:497-552)."""
        symbols = []
        for ch in segment:
            n = SPACE_MARKER if ch == " " else ch
            if n in self.char_ids:
                symbols.append(self.char_ids[n])
            else:
                symbols.extend(self.byte_ids[b] for b in n.encode())
        if len(symbols) > MAX_TOKENS:
            raise TokenizerError("LimitExceeded", "token cap")
        while True:
            best = None
            for a, b in zip(symbols, symbols[1:]):
                m = self.merges.get((a, b))
                if m is not None and (best is None or m[0] < best[0]):
                    best = (m[0], a, b, m[1])
            if best is None:
                break
            _, left, right, merged = best
            out, k = [], 0
            while k < len(symbols):
                if k + 1 < len(symbols) and symbols[k] == left and symbols[k + 1] == right:
                    out.append(merged)
                    k += 2
                else:
                    out.append(symbols[k])
                    k += 1
            symbols = out
        ids.extend(symbols)
        self._check(len(ids))

    @staticmethod
    def _check(n):
        if n > MAX_TOKENS:
            raise TokenizerError("LimitExceeded", "token cap")

    def decode(self, ids, skip_special_tokens: bool):
        """Tokenizer::decode (tokenizer.rs:391-425)."""
        out = bytearray()
        for i in ids:
            if i not in self.id_to_token:
                raise TokenizerError("Corrupt", f"cannot decode unknown token id {i}")
            if skip_special_tokens and i in self.special:
                continue
            tok = self.id_to_token[i]
            b = _byte_token(tok)
            if b is not None:
                out.append(b)
            else:
                out.extend(tok.replace(SPACE_MARKER, " ").encode())
        try:
            return out.decode("utf-8")
        except UnicodeDecodeError:
            raise TokenizerError("Corrupt", "decoded token sequence is not valid UTF-8")
