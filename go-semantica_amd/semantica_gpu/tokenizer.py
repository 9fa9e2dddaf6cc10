"""The reference tokenizer (internal/tokenizer/tokenizer.go) through the
library's C ABI (sg_tokenizer_*, csrc/sg_tokenizer.cpp): the same token IDs
Model.Tokenizer().Encode produces, from a vocabulary or a GGUF image."""
from __future__ import annotations

import ctypes
import os

import numpy as np

from . import _lib

# tokenizer.TokenType (tokenizer.go:15-23)
TOKEN_NORMAL, TOKEN_UNKNOWN, TOKEN_CONTROL, TOKEN_USER_DEFINED, TOKEN_UNUSED, TOKEN_BYTE = 1, 2, 3, 4, 5, 6


def _ptr(a: np.ndarray):
    return ctypes.c_void_p(a.ctypes.data)


def _packed(items):
    """bytes items -> (data, int64 offsets[n+1])."""
    offs = np.zeros(len(items) + 1, np.int64)
    offs[1:] = np.cumsum([len(b) for b in items]) if items else []
    data = np.frombuffer(b"".join(items) + b"\0", np.uint8)
    return data, offs


def _utf8(s) -> bytes:
    return s if isinstance(s, (bytes, bytearray)) else s.encode("utf-8", "surrogateescape")


class Tokenizer:
    """tokenizer.Tokenizer: new(...) = tokenizer.New, from_gguf = LoadFromGGUF."""

    def __init__(self, handle):
        self.lib = _lib.load()
        self.handle = handle

    @classmethod
    def new(cls, vocab, scores, token_types=None, add_bos=False, add_eos=False, lowercase=False,
            remove_accents=False, nfkc=False, bos_id=-1, eos_id=-1, unk_id=-1, pad_id=-1) -> "Tokenizer":
        """tokenizer.New(vocab, scores, tokenTypes, Config{...}) plus the special
        ids (New leaves them at -1; LoadFromGGUF sets them from metadata)."""
        if len(vocab) != len(scores):
            raise _lib.SemanticaError(_lib.SG_ERR_INVALID,
                                      f"vocab and scores length mismatch: {len(vocab)} != {len(scores)}")
        data, offs = _packed([_utf8(v) for v in vocab])
        sc = np.ascontiguousarray(scores, np.float32)
        ty = None if token_types is None or len(token_types) == 0 else np.ascontiguousarray(token_types, np.int32)
        if ty is not None and ty.size != len(vocab):
            raise _lib.SemanticaError(_lib.SG_ERR_INVALID,
                                      f"vocab and tokenTypes length mismatch: {len(vocab)} != {ty.size}")
        cfg = _lib.TokenizerConfig(int(add_bos), int(add_eos), int(lowercase), int(remove_accents), int(nfkc),
                                   bos_id, eos_id, unk_id, pad_id)
        h = ctypes.c_void_p()
        _lib.check(_lib.load().sg_tokenizer_create(_ptr(data), _ptr(offs), _ptr(sc) if sc.size else None,
                                                   _ptr(ty) if ty is not None else None, len(vocab),
                                                   ctypes.byref(cfg), ctypes.byref(h)))
        return cls(h)

    @classmethod
    def from_gguf(cls, source) -> "Tokenizer":
        """LoadFromGGUF over a GGUF image (bytes) or a file path."""
        lib = _lib.load()
        h = ctypes.c_void_p()
        if isinstance(source, (bytes, bytearray, memoryview)):
            image = bytes(source)
            buf = ctypes.create_string_buffer(image, len(image))
            _lib.check(lib.sg_tokenizer_from_gguf(buf, len(image), ctypes.byref(h)))
        else:
            _lib.check(lib.sg_tokenizer_from_gguf_file(os.fspath(source).encode(), ctypes.byref(h)))
        return cls(h)

    def close(self):
        if self.handle:
            self.lib.sg_tokenizer_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def vocab_size(self) -> int:
        return int(self.lib.sg_tokenizer_vocab_size(self.handle))

    def encode(self, text) -> list:
        """Encode (tokenizer.go:99-133); str or bytes (bytes may be ill-formed UTF-8)."""
        b = _utf8(text)
        n = ctypes.c_int32()
        _lib.check(self.lib.sg_tokenizer_encode(self.handle, b, len(b), None, 0, ctypes.byref(n)))
        ids = np.zeros(max(n.value, 1), np.int32)
        _lib.check(self.lib.sg_tokenizer_encode(self.handle, b, len(b), _ptr(ids), ids.size, ctypes.byref(n)))
        return ids[:n.value].tolist()

    def encode_batch(self, texts):
        """Encode of every text into packed IDs + CSR offsets (sg_forward's input)."""
        data, offs = _packed([_utf8(t) for t in texts])
        id_off = np.zeros(len(texts) + 1, np.int32)
        _lib.check(self.lib.sg_tokenizer_encode_batch(self.handle, _ptr(data), _ptr(offs), len(texts), None, 0,
                                                      _ptr(id_off)))
        ids = np.zeros(max(int(id_off[-1]), 1), np.int32)
        _lib.check(self.lib.sg_tokenizer_encode_batch(self.handle, _ptr(data), _ptr(offs), len(texts), _ptr(ids),
                                                      ids.size, _ptr(id_off)))
        return ids[:int(id_off[-1])], id_off

    def decode(self, ids) -> str:
        """Decode (tokenizer.go:135-159)."""
        a = np.ascontiguousarray(ids, np.int32)
        n = ctypes.c_size_t()
        _lib.check(self.lib.sg_tokenizer_decode(self.handle, _ptr(a) if a.size else None, a.size, None, 0,
                                                ctypes.byref(n)))
        buf = ctypes.create_string_buffer(max(n.value, 1))
        _lib.check(self.lib.sg_tokenizer_decode(self.handle, _ptr(a) if a.size else None, a.size, buf, n.value,
                                                ctypes.byref(n)))
        return buf.raw[:n.value].decode("utf-8", "surrogateescape")
