"""CPU restatement of go-semantica's tokenizer (internal/tokenizer/tokenizer.go)
-- TEST INFRASTRUCTURE ONLY: the checker the library's C++ tokenizer
(csrc/sg_tokenizer.cpp) is compared against.  Plain Python, following the
reference line by line, including its quadratic merge loop (it rescans every
pair after each merge); small inputs only.

Normalization uses Python's unicodedata (Unicode 13); the reference uses
golang.org/x/text (Unicode 15).  Tests keep to characters both versions
treat alike.
"""
from __future__ import annotations

import unicodedata

METASPACE = "▁"


def decode_go(b: bytes) -> list:
    """Go's rune iteration over a string (utf8.DecodeRune): each byte of an
    ill-formed sequence becomes U+FFFD on its own."""
    out, i, n = [], 0, len(b)
    while i < n:
        c = b[i]
        if c < 0x80:
            out.append(chr(c))
            i += 1
            continue
        if 0xC2 <= c <= 0xDF:
            ln, lo, hi = 2, 0x80, 0xBF
        elif 0xE0 <= c <= 0xEF:
            ln, lo, hi = 3, (0xA0 if c == 0xE0 else 0x80), (0x9F if c == 0xED else 0xBF)
        elif 0xF0 <= c <= 0xF4:
            ln, lo, hi = 4, (0x90 if c == 0xF0 else 0x80), (0x8F if c == 0xF4 else 0xBF)
        else:
            ln = 0
        ok = ln > 0 and i + ln <= n
        if ok:
            if not (lo <= b[i + 1] <= hi):
                ok = False
            for k in range(2, ln):
                if not (0x80 <= b[i + k] <= 0xBF):
                    ok = False
        if ok:
            out.append(b[i:i + ln].decode("utf-8"))
            i += ln
        else:
            out.append("�")
            i += 1
    return out


def _lower(c: str) -> str:
    """unicode.ToLower (simple mapping): one rune in, one rune out."""
    if c == "İ":
        return "i"
    low = c.lower()
    return low if len(low) == 1 else c


class Tokenizer:
    """tokenizer.New (tokenizer.go:56-97) + the special ids LoadFromGGUF sets."""

    def __init__(self, vocab, scores, token_types=None, add_bos=False, add_eos=False, lowercase=False,
                 remove_accents=False, nfkc=False, bos_id=-1, eos_id=-1, unk_id=-1, pad_id=-1):
        if len(vocab) != len(scores):
            raise ValueError(f"vocab and scores length mismatch: {len(vocab)} != {len(scores)}")
        if token_types and len(token_types) != len(vocab):
            raise ValueError(f"vocab and tokenTypes length mismatch: {len(vocab)} != {len(token_types)}")
        self.vocab = [v if isinstance(v, bytes) else v.encode("utf-8") for v in vocab]
        self.scores = [float(s) for s in scores]
        self.types = list(token_types) if token_types else [1] * len(vocab)
        self.add_bos, self.add_eos = add_bos, add_eos
        self.lowercase, self.remove_accents, self.nfkc = lowercase, remove_accents, nfkc
        self.bos, self.eos, self.unk, self.pad = bos_id, eos_id, unk_id, pad_id
        self.to_id = {}
        for i, t in enumerate(self.vocab):  # later duplicates win (tokenizer.go:88-91)
            self.to_id[t] = i

    def normalize(self, runes: list) -> list:
        """Normalizer.Normalize (tokenizer.go:459-494)."""
        s = "".join(runes)
        if self.nfkc:
            s = unicodedata.normalize("NFKC", s)
        if self.remove_accents:
            s = "".join(c for c in unicodedata.normalize("NFD", s) if unicodedata.category(c) != "Mn")
        if self.lowercase:
            s = "".join(_lower(c) for c in s)
        return list(s)

    @staticmethod
    def preprocess(runes: list) -> list:
        """preprocessSpaces (tokenizer.go:161-215) -> the runes BPE starts from."""
        out, i = [], 0
        while i < len(runes):
            if runes[i] != " ":
                out.append(runes[i])
                i += 1
                continue
            j = i
            while j < len(runes) and runes[j] == " ":
                j += 1
            out.extend([METASPACE] if j - i == 1 else [" "] * (j - i))
            i = j
        return out

    def bpe(self, runes: list) -> list:
        """tokenizeBPE (tokenizer.go:217-348), symbols as UTF-8 bytes."""
        if not runes:
            return []
        text = [r.encode("utf-8") for r in runes]
        nxt = [i + 1 for i in range(len(text))]
        prv = [i - 1 for i in range(len(text))]
        nxt[-1] = -1
        while True:
            cands = []
            for i in range(len(text)):
                if text[i] != b"" and nxt[i] != -1:
                    t = text[i] + text[nxt[i]]
                    if t in self.to_id:
                        cands.append((i, nxt[i], self.scores[self.to_id[t]], t))
            if not cands:
                break
            best = cands[0]
            for c in cands[1:]:  # highest score; ties to the rightmost (tokenizer.go:284-293)
                if c[2] > best[2] or (c[2] == best[2] and c[0] > best[0]):
                    best = c
            left, right, _, t = best
            text[left] = t
            nxt[left] = nxt[right]
            if nxt[right] != -1:
                prv[nxt[right]] = left
            text[right] = b""
        final = []
        for t in text:
            if t == b"":
                continue
            if t in self.to_id:
                final.append(t)
            elif len(self.vocab) > 493:  # byte tokens 238 + b (tokenizer.go:322-331)
                final.extend(self.vocab[238 + b] for b in t)
            elif 0 <= self.unk < len(self.vocab):
                final.append(self.vocab[self.unk])
        return final

    def encode(self, text) -> list:
        """Encode (tokenizer.go:99-133); text as str or raw bytes."""
        b = text if isinstance(text, bytes) else text.encode("utf-8", "surrogateescape")
        runes = self.normalize(decode_go(b))
        ids = []
        if self.add_bos and self.bos >= 0:
            ids.append(self.bos)
        for t in self.bpe(self.preprocess(runes)):
            if t in self.to_id:
                ids.append(self.to_id[t])
            elif self.unk >= 0:
                ids.append(self.unk)
        if self.add_eos and self.eos >= 0:
            ids.append(self.eos)
        return ids

    def decode(self, ids) -> bytes:
        """Decode (tokenizer.go:135-159)."""
        out = b""
        for i in ids:
            if i < 0 or i >= len(self.vocab):
                continue
            if i in (self.bos, self.eos, self.unk, self.pad) or self.types[i] in (3, 5):
                continue
            out += self.vocab[i].replace(METASPACE.encode("utf-8"), b" ")
        return out
