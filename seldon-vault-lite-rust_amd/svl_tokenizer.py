"""The frozen model's BPE tokenizer and the text embedder over strings, shaped
like the reference crate's API:

* ``Tokenizer`` — src/model/tokenizer.rs (``from_json_str``, ``load``,
  ``encode``, ``decode`` and the id accessors), plus ``encode_batch`` (host
  threads)
* ``Prompt`` — the roles of src/model/prompt.rs:38-55 and their prefixes
* ``TextEmbedder`` — src/model/text.rs:556-626 (``embed`` of raw text with a
  prompt), plus ``embed_batch`` (one batched forward pass)

Tokenization is the library's C++ host code; the forward pass runs on the
GPU. There is no Python fallback.
"""
from __future__ import annotations

import ctypes
import enum

import numpy as np

import svl_amd
from svl_amd import SvlError, _check, lib

MAX_TOKENIZER_FILE_BYTES = 64 * 1024 * 1024  # tokenizer.rs:25
MAX_TOKENS = 262_144                         # tokenizer.rs:43


def _load():
    L = lib()
    if not getattr(L, "_tok_ready", False):
        vp, i64, i32, sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_size_t
        L.svl_tokenizer_create.argtypes = [ctypes.c_char_p, sz, ctypes.POINTER(vp)]
        L.svl_tokenizer_destroy.argtypes = [vp]
        L.svl_tokenizer_encode.argtypes = [vp, ctypes.c_char_p, sz, ctypes.c_int, vp, sz,
                                           ctypes.POINTER(sz)]
        L.svl_tokenizer_encode_batch.argtypes = [vp, vp, vp, i32, ctypes.c_int, vp, sz, vp]
        L.svl_tokenizer_decode.argtypes = [vp, vp, sz, ctypes.c_int, vp, sz, ctypes.POINTER(sz)]
        L.svl_tokenizer_token_id.restype = i64
        L.svl_tokenizer_token_id.argtypes = [vp, ctypes.c_char_p, sz]
        L.svl_tokenizer_token.restype = ctypes.POINTER(ctypes.c_char)
        L.svl_tokenizer_token.argtypes = [vp, ctypes.c_uint32, ctypes.POINTER(sz)]
        for name in ("vocab_size", "max_token_id", "bos_id", "eos_id", "unk_id", "pad_id"):
            f = getattr(L, f"svl_tokenizer_{name}")
            f.restype = i64
            f.argtypes = [vp]
        L.svl_tokenizer_is_special_id.restype = ctypes.c_int
        L.svl_tokenizer_is_special_id.argtypes = [vp, ctypes.c_uint32]
        L.svl_text_embed_texts.argtypes = [vp, vp, vp, vp, i32, i32, i64, vp]
        L._tok_ready = True
    return L


def _texts(texts):
    raw = [t.encode("utf-8") if isinstance(t, str) else bytes(t) for t in texts]
    bufs = [ctypes.create_string_buffer(r, len(r) or 1) for r in raw]
    ptrs = (ctypes.c_void_p * max(len(raw), 1))(*[ctypes.addressof(b) for b in bufs])
    lens = (ctypes.c_size_t * max(len(raw), 1))(*[len(r) for r in raw])
    return raw, bufs, ptrs, lens


class Tokenizer:
    """Frozen-model BPE tokenizer (tokenizer.rs:64-334)."""

    def __init__(self, handle):
        self.handle = handle

    @classmethod
    def from_json_str(cls, text: str | bytes) -> "Tokenizer":
        data = text.encode("utf-8") if isinstance(text, str) else bytes(text)
        h = ctypes.c_void_p()
        _check(_load().svl_tokenizer_create(data, len(data), ctypes.byref(h)))
        return cls(h)

    @classmethod
    def load(cls, path: str) -> "Tokenizer":
        """Tokenizer::load (tokenizer.rs:82-87): bounded by the file cap."""
        import os
        if os.path.getsize(path) > MAX_TOKENIZER_FILE_BYTES:
            raise SvlError(5, f"{path} is larger than the {MAX_TOKENIZER_FILE_BYTES}-byte cap")
        with open(path, "rb") as f:
            return cls.from_json_str(f.read())

    def __del__(self):
        if getattr(self, "handle", None):
            _load().svl_tokenizer_destroy(self.handle)
            self.handle = None

    def encode(self, text: str | bytes, add_special_tokens: bool) -> list:
        data = text.encode("utf-8") if isinstance(text, str) else bytes(text)
        out = np.empty(MAX_TOKENS + 2, np.uint32)
        n = ctypes.c_size_t()
        _check(_load().svl_tokenizer_encode(self.handle, data, len(data), int(add_special_tokens),
                                            ctypes.c_void_p(out.ctypes.data), out.size,
                                            ctypes.byref(n)))
        return out[: n.value].tolist()

    def encode_batch(self, texts, add_special_tokens: bool) -> list:
        raw, bufs, ptrs, lens = _texts(texts)
        offsets = np.zeros(len(raw) + 1, np.int64)
        cap = sum(len(r) for r in raw) * 4 + 2 * len(raw) + 1  # one id per byte at most
        out = np.empty(cap, np.uint32)
        _check(_load().svl_tokenizer_encode_batch(self.handle, ptrs, lens, len(raw),
                                                  int(add_special_tokens),
                                                  ctypes.c_void_p(out.ctypes.data), cap,
                                                  ctypes.c_void_p(offsets.ctypes.data)))
        return [out[offsets[i]:offsets[i + 1]].tolist() for i in range(len(raw))]

    def decode(self, ids, skip_special_tokens: bool) -> str:
        a = np.ascontiguousarray(ids, np.uint32)
        n = ctypes.c_size_t()
        L = _load()
        st = L.svl_tokenizer_decode(self.handle, ctypes.c_void_p(a.ctypes.data), a.size,
                                    int(skip_special_tokens), None, 0, ctypes.byref(n))
        if st != 0 and n.value == 0:
            _check(st)
        buf = ctypes.create_string_buffer(max(n.value, 1))
        _check(L.svl_tokenizer_decode(self.handle, ctypes.c_void_p(a.ctypes.data), a.size,
                                      int(skip_special_tokens), buf, n.value, ctypes.byref(n)))
        return buf.raw[: n.value].decode("utf-8")

    def token_id(self, token: str):
        data = token.encode("utf-8")
        v = _load().svl_tokenizer_token_id(self.handle, data, len(data))
        return None if v < 0 else int(v)

    def token(self, id_: int):
        n = ctypes.c_size_t()
        p = _load().svl_tokenizer_token(self.handle, int(id_), ctypes.byref(n))
        return None if not p else ctypes.string_at(p, n.value).decode("utf-8")

    def vocab_size(self):
        return int(_load().svl_tokenizer_vocab_size(self.handle))

    def max_token_id(self):
        return int(_load().svl_tokenizer_max_token_id(self.handle))

    def bos_id(self):
        return int(_load().svl_tokenizer_bos_id(self.handle))

    def eos_id(self):
        return int(_load().svl_tokenizer_eos_id(self.handle))

    def unk_id(self):
        return int(_load().svl_tokenizer_unk_id(self.handle))

    def pad_id(self):
        v = int(_load().svl_tokenizer_pad_id(self.handle))
        return None if v < 0 else v

    def is_special_id(self, id_: int) -> bool:
        return bool(_load().svl_tokenizer_is_special_id(self.handle, int(id_)))


class Prompt(enum.IntEnum):
    """prompt.rs:38-55."""
    SearchQuery = 0
    Document = 1
    Classification = 2
    Clustering = 3
    CodeRetrieval = 4
    FactChecking = 5
    SentenceSimilarity = 6
    QuestionAnswering = 7

    def prefix(self) -> str:
        return PREFIXES[self]

    def is_query(self) -> bool:
        return self is not Prompt.Document

    @classmethod
    def from_name(cls, name: str):
        """prompt.rs:82-94; case-sensitive."""
        return cls.__members__.get(name)


PREFIXES = {
    Prompt.SearchQuery: "task: search result | query: ",
    Prompt.Document: "title: none | text: ",
    Prompt.Classification: "task: classification | query: ",
    Prompt.Clustering: "task: clustering | query: ",
    Prompt.CodeRetrieval: "task: code retrieval | query: ",
    Prompt.FactChecking: "task: fact checking | query: ",
    Prompt.SentenceSimilarity: "task: sentence similarity | query: ",
    Prompt.QuestionAnswering: "task: question answering | query: ",
}


class TextEmbedder:
    """TextEmbedder (text.rs:556-626): a text model plus the tokenizer."""

    def __init__(self, model: svl_amd.TextModel, tokenizer: Tokenizer, check_vocab=True):
        if check_vocab and tokenizer.vocab_size() != model.config.vocab_size:
            raise SvlError(4, f"tokenizer vocabulary has {tokenizer.vocab_size()} entries, "
                              f"model declares {model.config.vocab_size}")
        self.model, self.tokenizer = model, tokenizer

    @classmethod
    def from_parts(cls, model, tokenizer):
        """text.rs:597-600: no vocabulary check."""
        return cls(model, tokenizer, check_vocab=False)

    def embed(self, text: str, prompt: Prompt, dimension: int):
        return self.embed_batch([text], prompt, dimension)[0]

    def embed_batch(self, texts, prompt: Prompt, dimension: int):
        raw, bufs, ptrs, lens = _texts(texts)
        out = np.empty((max(len(raw), 1), int(dimension)), np.float32)
        _check(_load().svl_text_embed_texts(self.model.handle, self.tokenizer.handle, ptrs, lens,
                                            len(raw), int(prompt), int(dimension),
                                            ctypes.c_void_p(out.ctypes.data)))
        return out[: len(raw)]
