"""The library's tokenizer (csrc/sg_tokenizer.cpp) against the oracle's
restatement of internal/tokenizer/tokenizer.go (oracle/tokenizer_ref.py),
the oracle against the reference's own tests (tokenizer_test.go) and
hand-derived cases, GGUF tokenizer metadata (LoadFromGGUF) and the task
prompts of pkg/ggufembed (tasks.go).  CPU only: the tokenizer is host code.

Parity with llama.cpp's IDs for real text (testdata/reference_token_ids.json)
needs the real model's vocabulary, a Git-LFS file that is not available
offline: unpinned."""
import numpy as np
import pytest

import tokenizer_ref as ref

CONTROL, NORMAL, BYTE = 3, 1, 6


def lib_tok(**kw):
    from semantica_gpu.tokenizer import Tokenizer
    return Tokenizer.new(**kw)


# ---- the reference's test vocabularies (tokenizer_test.go) -----------------

def basic_vocab():
    """TestTokenizerBasic (tokenizer_test.go:8-45): score = byte length - 10."""
    vocab = ["<unk>", "<s>", "</s>", "▁", "h", "e", "l", "o", "w", "r", "d", "t", "a", "n",
             "he", "ll", "el", "lo", "wo", "or", "rl", "ld", "th", "an",
             "hello", "world", "▁hello", "▁world", "▁the", "▁a", "▁an"]
    scores = [float(len(v.encode())) - 10 for v in vocab]
    types = [CONTROL if i < 3 else NORMAL for i in range(len(vocab))]
    return dict(vocab=vocab, scores=scores, token_types=types)


def byte_vocab():
    """TestBytefallbackTokens (tokenizer_test.go:128-185): 494 tokens, bytes at
    238..493, UNK = 0."""
    vocab = ["<unk>", "<s>", "</s>", "▁", "h", "e", "l", "o", "hello", "▁hello"]
    scores = [float(i) for i in range(10)]
    types = [CONTROL] * 3 + [NORMAL] * 7
    for i in range(10, 238):
        vocab.append(f"<token_{i}>")
        scores.append(0.0)
        types.append(NORMAL)
    for b in range(256):
        vocab.append(f"<0x{b:02X}>")
        scores.append(-10.0)
        types.append(BYTE)
    return dict(vocab=vocab, scores=scores, token_types=types, unk_id=0)


BASIC_CASES = [  # hand-derived from tokenizeBPE (tokenizer.go:217-348), see test docstring
    ("hello world", [4, 16, 17, 3, 8, 19, 21]),
    ("the", [11, 14]),
    ("", []),
]

BYTE_CASES = [  # tokenizer_test.go:188-243, 446-560
    (b"\xff", [477, 429, 427]),
    (b"\x80", [477, 429, 427]),
    (b"\xc0\x80", [477, 429, 427, 477, 429, 427]),
    ("ñ".encode(), [433, 415]),
    ("😀".encode(), [478, 397, 390, 366]),
    (b"z", [360]),
    (b"", []),
    (b"hello", [4, 5, 6, 6, 7]),
    (b"hello\xff", [4, 5, 6, 6, 7, 477, 429, 427]),
] + [(bytes([c]), [238 + c]) for c in (0x00, 0x07, 0x08, 0x09, 0x0A, 0x0D, 0x1B, 0x1F)]


def test_oracle_basic_vocab_hand_derived():
    """"hello world" -> "hello▁world"; every candidate bigram scores -8, so the
    rightmost merges first: ld, or, lo, el; then no pair is in the vocabulary:
    h el lo ▁ w or ld.  "the": he (rightmost of th/he), then "the" is not a
    token.  These pin the tie rule and the byte-length scores."""
    t = ref.Tokenizer(**basic_vocab())
    for text, want in BASIC_CASES:
        assert t.encode(text) == want, text


def test_oracle_reference_byte_fallback_cases():
    t = ref.Tokenizer(**byte_vocab())
    for text, want in BYTE_CASES:
        assert t.encode(text) == want, text
    # ByteFallbackReverseDecode: byte tokens decode to their "<0xXX>" text
    for b in (0x00, 0x20, 0x41, 0x7E, 0xFF):
        assert t.decode([238 + b]) == f"<0x{b:02X}>".encode()
    assert t.decode([0, 1, 2, 3, 8]) == b" hello"  # control tokens skipped, ▁ -> space


def test_oracle_normalizer_cases():
    """TestNormalizer (tokenizer_test.go:83-112) with exact results."""
    t = ref.Tokenizer(["a"], [0.0], nfkc=True)
    assert "".join(t.normalize(list("ﬁ"))) == "fi"
    t = ref.Tokenizer(["a"], [0.0], nfkc=True, lowercase=True)
    assert "".join(t.normalize(list("Ｈｅｌｌｏ"))) == "hello"
    t = ref.Tokenizer(["a"], [0.0], lowercase=True)
    assert "".join(t.normalize(list("Hello"))) == "hello"
    t = ref.Tokenizer(["a"], [0.0], remove_accents=True)
    assert "".join(t.normalize(list("café naïve"))) == "cafe naive"


def test_oracle_space_runs():
    """preprocessSpaces (tokenizer.go:161-215): one space -> ▁, runs stay raw."""
    assert ref.Tokenizer.preprocess(list("a b  c   d ")) == list("a▁b  c   d▁")
    assert ref.Tokenizer.preprocess(list(" ")) == ["▁"]


def test_oracle_go_utf8_decoding():
    """utf8.DecodeRune: every byte of an ill-formed sequence is one U+FFFD
    (Python's own decoder would fold a truncated sequence into one)."""
    assert ref.decode_go(b"\xe2\x82") == ["�", "�"]
    assert ref.decode_go(b"\xe2\x82x") == ["�", "�", "x"]
    assert ref.decode_go(b"\xed\xa0\x80") == ["�"] * 3  # surrogate
    assert ref.decode_go(b"\xf4\x90\x80\x80") == ["�"] * 4  # above U+10FFFF
    assert ref.decode_go("€😀".encode()) == ["€", "😀"]


# ---- library vs oracle ----------------------------------------------------

def test_library_reference_cases():
    t = lib_tok(**basic_vocab())
    for text, want in BASIC_CASES:
        assert t.encode(text) == want, text
    t = lib_tok(**byte_vocab())
    for text, want in BYTE_CASES:
        assert t.encode(text) == want, text
    assert t.vocab_size() == 494
    assert t.decode([0, 1, 2, 3, 8, 238 + 0x41]) == " hello<0x41>"
    from semantica_gpu.tokenizer import Tokenizer
    assert Tokenizer.new(["a", "b", "c"], [1, 2, 3]).vocab_size() == 3  # TestTokenizerVocabSize


ALPHABET = list("abcdeé ") + ["  ", "   ", "ﬁ", "Ｈ", "ñ", "😀", "́", "x", "\t"]


def _random_vocab(rng, n_pieces, with_bytes, dup=False):
    pieces = set()
    base = list("abcdeéñ") + ["▁", " ", "  "]
    while len(pieces) < n_pieces:
        k = int(rng.integers(2, 5))
        pieces.add("".join(rng.choice(base, size=k)))
    vocab = ["<unk>", "<s>", "</s>"] + base + sorted(pieces)
    if dup:
        vocab += vocab[5:25]  # duplicated strings: the later index wins
    scores = rng.choice([-1.0, -2.0, -3.0, -2.5], size=len(vocab)).astype(np.float32).tolist()
    types = [CONTROL] * 3 + [NORMAL] * (len(vocab) - 3)
    if with_bytes:
        while len(vocab) < 238:
            vocab.append(f"<tok{len(vocab)}>")
            scores.append(0.0)
            types.append(NORMAL)
        vocab = vocab[:238] + [f"<0x{b:02X}>" for b in range(256)]
        scores = scores[:238] + [-10.0] * 256
        types = types[:238] + [BYTE] * 256
    return vocab, scores, types


@pytest.mark.parametrize("seed", range(6))
def test_library_matches_oracle_random(seed):
    """Random texts (single and multiple spaces, NFKC-changing and combining
    characters, ill-formed bytes) over random vocabularies with tied scores,
    with and without byte fallback, duplicates, BOS/EOS: identical IDs, and
    identical decodes."""
    rng = np.random.default_rng(seed)
    vocab, scores, types = _random_vocab(rng, 150, with_bytes=seed % 2 == 0, dup=seed % 3 == 0)
    cfg = dict(vocab=vocab, scores=scores, token_types=types, add_bos=seed % 2 == 1, add_eos=seed == 5,
               nfkc=seed < 4, lowercase=seed == 4, remove_accents=seed == 5, bos_id=1, eos_id=2,
               unk_id=0 if seed != 3 else -1)
    o, t = ref.Tokenizer(**cfg), lib_tok(**cfg)
    texts = []
    for _ in range(150):
        k = int(rng.integers(0, 40))
        s = "".join(rng.choice(ALPHABET, size=k)).encode()
        if rng.random() < 0.2:
            s += bytes(rng.choice([0x80, 0xC3, 0xE2, 0xFF], size=int(rng.integers(1, 3))).tolist())
        texts.append(s)
    for s in texts:
        want = o.encode(s)
        assert t.encode(s) == want, s
        assert t.decode(want).encode("utf-8", "surrogateescape") == o.decode(want), s
    ids, off = t.encode_batch(texts)
    for i, s in enumerate(texts):
        assert ids[off[i]:off[i + 1]].tolist() == o.encode(s)


def test_long_text_matches_oracle():
    """A few thousand runes: the heap-based merge order equals the reference's
    rescan-every-pair loop."""
    rng = np.random.default_rng(99)
    vocab, scores, types = _random_vocab(rng, 400, with_bytes=True)
    o, t = ref.Tokenizer(vocab, scores, types, unk_id=0), lib_tok(vocab=vocab, scores=scores, token_types=types,
                                                                   unk_id=0)
    s = "".join(rng.choice(ALPHABET[:7], size=2500))
    assert t.encode(s) == o.encode(s)


# ---- GGUF metadata (LoadFromGGUF) ------------------------------------------

def _gguf(extra):
    from semantica_gpu import synth
    return synth.gguf_image([("general.architecture", "str", "gemma-embedding")] + extra, [])


def test_from_gguf_matches_oracle():
    from semantica_gpu.tokenizer import Tokenizer
    v = byte_vocab()
    md = [("tokenizer.ggml.tokens", "arr:str", v["vocab"]),
          ("tokenizer.ggml.scores", "arr:f32", v["scores"]),
          ("tokenizer.ggml.token_type", "arr:i32", v["token_types"]),
          ("tokenizer.ggml.bos_token_id", "u32", 1), ("tokenizer.ggml.eos_token_id", "u32", 2),
          ("tokenizer.ggml.unknown_token_id", "u32", 0), ("tokenizer.ggml.padding_token_id", "i32", 0)]
    t = Tokenizer.from_gguf(_gguf(md))
    # LoadFromGGUF: add_bos defaults to true, add_eos to false, NFKC on; the
    # padding id is ignored unless stored as uint32.
    o = ref.Tokenizer(v["vocab"], v["scores"], v["token_types"], add_bos=True, nfkc=True, bos_id=1, eos_id=2,
                      unk_id=0)
    for s in ["hello", "ﬁ hello", "Ｈello  x", "z\xff".encode("latin-1"), ""]:
        assert t.encode(s) == o.encode(s), s
    md2 = md + [("tokenizer.ggml.add_bos_token", "bool", False), ("tokenizer.ggml.add_eos_token", "bool", True)]
    t2 = Tokenizer.from_gguf(_gguf(md2))
    assert t2.encode("hello") == [4, 5, 6, 6, 7, 2]
    # float64 scores and uint32 token types are read too; other element types -> normal
    md3 = [("tokenizer.ggml.tokens", "arr:str", ["<s>", "a", "b", "ab"]),
           ("tokenizer.ggml.scores", "arr:f64", [0.0, -1.0, -1.0, -0.5]),
           ("tokenizer.ggml.token_type", "arr:u8", [3, 1, 1, 1])]
    t3 = Tokenizer.from_gguf(_gguf(md3))
    assert t3.encode("ab") == [3] and t3.decode([0, 3]) == "<s>ab"


def test_from_gguf_errors():
    from semantica_gpu import SemanticaError
    from semantica_gpu.tokenizer import Tokenizer

    def err(md):
        with pytest.raises(SemanticaError) as e:
            Tokenizer.from_gguf(_gguf(md))
        return str(e.value)

    assert "tokenizer.ggml.tokens not found" in err([])
    assert "tokenizer.ggml.tokens is not an array" in err([("tokenizer.ggml.tokens", "str", "a")])
    assert "token 1 is not a string" in err([("tokenizer.ggml.tokens", "arr:arr:str", [["a"], ["b"]])]) or \
        "token 0 is not a string" in err([("tokenizer.ggml.tokens", "arr:arr:str", [["a"], ["b"]])])
    toks = [("tokenizer.ggml.tokens", "arr:str", ["a", "b"])]
    assert "tokenizer.ggml.scores not found" in err(toks)
    assert "tokenizer.ggml.scores is not an array" in err(toks + [("tokenizer.ggml.scores", "f32", 1.0)])
    assert "score 0 is not a number" in err(toks + [("tokenizer.ggml.scores", "arr:i32", [1, 2])])
    assert "vocab and scores length mismatch: 2 != 1" in err(toks + [("tokenizer.ggml.scores", "arr:f32", [1.0])])
    assert "vocab and tokenTypes length mismatch: 2 != 3" in err(
        toks + [("tokenizer.ggml.scores", "arr:f32", [1.0, 2.0]), ("tokenizer.ggml.token_type", "arr:i32", [1, 1, 1])])


# ---- prompts (pkg/ggufembed/tasks.go) ---------------------------------------

def test_build_prompt():
    """EmbedInput.prompt (tasks.go:117-147) for every task."""
    from semantica_gpu.embed import EmbedError, EmbedInput, Task, build_prompt
    assert build_prompt(EmbedInput(Task.NONE, "  raw text \n")) == "raw text"
    assert build_prompt(EmbedInput(Task.SEARCH_DOCUMENT, "body", title=" T ")) == "title: T | text: body"
    assert build_prompt(EmbedInput(Task.SEARCH_DOCUMENT, "body")) == "title: none | text: body"
    want = {Task.SEARCH_QUERY: "search result", Task.QUESTION_ANSWERING: "question answering",
            Task.FACT_VERIFICATION: "fact checking", Task.CLASSIFICATION: "classification",
            Task.CLUSTERING: "clustering", Task.SEMANTIC_SIMILARITY: "sentence similarity",
            Task.CODE_RETRIEVAL: "code retrieval"}
    for task, desc in want.items():
        assert build_prompt(EmbedInput(task, "q")) == f"task: {desc} | query: q"
    assert build_prompt(EmbedInput(Task.CLUSTERING, "q", custom_task_description=" mine ")) == \
        "task: mine | query: q"
    with pytest.raises(EmbedError, match="content must not be empty"):
        build_prompt(EmbedInput(Task.SEARCH_QUERY, " \t　 "))
    with pytest.raises(EmbedError, match=r"unsupported task task\(42\) \(missing default description\)"):
        build_prompt(EmbedInput(42, "q"))
    # strings.TrimSpace keeps U+001F (not unicode.IsSpace), unlike str.strip()
    assert build_prompt(EmbedInput(Task.NONE, "\x1fa\x1f")) == "\x1fa\x1f"


def test_embed_cancellation_stops_before_work():
    """A cancelled context (api.go:190-195, :268-273) raises before the next
    tokenize or forward starts; a live one lets the calls through.  Stub
    tokenizer and model record what ran (host logic only, no device)."""
    import threading
    from semantica_gpu.embed import Cancelled, EmbedInput, EmbedRuntime, Task
    calls = []

    class Tok:
        def encode_batch(self, prompts):
            calls.append("tokenize")
            off = np.arange(len(prompts) + 1, dtype=np.int32)
            return np.ones(len(prompts), np.int32), off

    class Mdl:
        max_seq_len = 2048

        def forward_packed(self, toks, off, d):
            calls.append(f"forward {d}")
            if d == 768:  # cancelled during the first dimension's forward
                ev.set()
            return np.zeros((len(off) - 1, d), np.float32)

    rt = EmbedRuntime(None, Mdl(), Tok())
    ev = threading.Event()
    inputs = [EmbedInput(Task.SEARCH_QUERY, "a", dim=768), EmbedInput(Task.SEARCH_QUERY, "b", dim=256)]
    with pytest.raises(Cancelled, match="context canceled"):
        rt.embed_inputs(inputs, ctx=ev)  # dims run largest first: 256's forward never starts
    assert calls == ["tokenize", "forward 768"]
    calls.clear()
    with pytest.raises(Cancelled):
        rt.embed(["x"], ctx=ev)  # already cancelled: nothing runs
    with pytest.raises(Cancelled):
        rt.embed_single_input(EmbedInput(Task.NONE, "x"), ctx=lambda: True)
    assert calls == []
    ev = threading.Event()
    out = rt.embed_inputs([inputs[1]], ctx=ev)
    assert [o.shape[0] for o in out] == [256] and calls == ["tokenize", "forward 256"]
    assert rt.embed_single("x", ctx=None).shape == (512,)
