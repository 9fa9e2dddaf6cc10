"""GGUF v3 images: parseConfig over the C ABI on the CPU (no device call),
built with the synthetic writer in semantica_gpu.synth.  Cases follow
internal/gguf/reader.go:98-178 and internal/runtime/model.go:424-517."""
import numpy as np
import pytest

from conftest import TINY

P = "gemma-embedding."


def _tiny():
    from semantica_gpu import synth
    return synth.make_model(dict(TINY, num_layers=1, vocab_size=64))


def _md(drop=(), replace=None, arch="gemma-embedding"):
    p = arch + "." if arch else ""
    c = dict(TINY, num_layers=1, vocab_size=64)
    md = [("general.architecture", "str", arch)] if arch else []
    md += [(p + "embedding_length", "u32", c["embed_dim"]), (p + "block_count", "u32", c["num_layers"]),
           (p + "attention.head_count", "u32", c["num_heads"]), (p + "attention.head_count_kv", "u32", 1),
           (p + "feed_forward_length", "u32", c["interm_dim"]), (p + "context_length", "u32", 1024),
           (p + "attention.layer_norm_rms_epsilon", "f32", 1e-5), (p + "rope.freq_base", "f32", 5e5),
           ("tokenizer.ggml.tokens", "arr:str", [f"t{i}" for i in range(64)])]
    md = [m for m in md if m[0].split(".", 1)[-1] not in drop and m[0] not in drop]
    if replace:
        md = [(k, *replace[k]) if k in replace else (k, kind, v) for k, kind, v in md]
    return md


def _image(md, tensors=()):
    from semantica_gpu import synth
    return synth.gguf_image(md, list(tensors))


def _err(image):
    from semantica_gpu import SemanticaError, read_gguf_config
    with pytest.raises(SemanticaError) as ei:
        read_gguf_config(image)
    return ei.value


def test_config_round_trip_of_model_image():
    from semantica_gpu import read_gguf_config, synth
    m = _tiny()
    cfg = read_gguf_config(synth.model_gguf(m))
    for k, v in m.config.items():
        assert cfg[k] == pytest.approx(v, rel=1e-7), k


def test_explicit_metadata_and_every_value_kind():
    from semantica_gpu import read_gguf_config
    noise = [("x.u8", "u8", 7), ("x.i8", "i8", -7), ("x.u16", "u16", 65535), ("x.i16", "i16", -3),
             ("x.i32", "i32", -9), ("x.u64", "u64", 2 ** 40), ("x.i64", "i64", -2 ** 40), ("x.f64", "f64", 0.25),
             ("x.bool", "bool", True), ("x.arr", "arr:u32", [1, 2, 3]), ("x.nested", "arr:arr:u8", [[1], [2, 3]]),
             ("x.strs", "arr:str", ["a", "bc", ""])]
    cfg = read_gguf_config(_image(noise + _md()))
    assert cfg == {"embed_dim": 768, "num_layers": 1, "num_heads": 3, "num_kv_heads": 1, "interm_dim": 1152,
                   "max_seq_len": 1024, "vocab_size": 64, "norm_eps": pytest.approx(1e-5, rel=1e-6),
                   "rope_base": 5e5}


def test_defaults():
    """head_count_kv -> head_count; feed_forward_length -> blk.0.ffn_up dims[1];
    context_length -> 2048; eps/rope only when float32; vocab -> tensor count."""
    from semantica_gpu import read_gguf_config, synth
    md = _md(drop=("attention.head_count_kv", "feed_forward_length", "context_length", "tokenizer.ggml.tokens"),
             replace={P + "attention.layer_norm_rms_epsilon": ("f64", 1e-5), P + "rope.freq_base": ("u32", 7)})
    up = synth.q8_0_random(np.random.default_rng(0), 96, 64)
    tensors = [("blk.0.ffn_up.weight", [64, 96], synth.GGUF_DTYPE_Q8_0, up.tobytes()),
               ("other", [4], synth.GGUF_DTYPE_F32, np.zeros(4, np.float32).tobytes())]
    cfg = read_gguf_config(_image(md, tensors))
    assert cfg["num_kv_heads"] == 3 and cfg["interm_dim"] == 96 and cfg["max_seq_len"] == 2048
    assert cfg["norm_eps"] == pytest.approx(1e-6, rel=1e-6) and cfg["rope_base"] == 10000.0
    assert cfg["vocab_size"] == 2
    # without blk.0.ffn_up.weight: 3 x embedding_length
    assert read_gguf_config(_image(md))["interm_dim"] == 3 * 768


def test_no_architecture_uses_unprefixed_keys():
    from semantica_gpu import read_gguf_config
    assert read_gguf_config(_image(_md(arch="")))["embed_dim"] == 768


@pytest.mark.parametrize("case,msg", [
    ("short", "file too small for header"),
    ("magic", "invalid magic: 0x"),
    ("version", "unsupported version: 2"),
    ("missing", "gemma-embedding.embedding_length not found"),
    ("type", "gemma-embedding.block_count has metadata type 10, want uint32"),
    ("truncated", "read metadata"),
])
def test_errors(case, msg):
    from semantica_gpu import _lib, synth
    img = _image(_md())
    if case == "short":
        img = img[:20]
    elif case == "magic":
        img = b"GGUG" + img[4:]
    elif case == "version":
        img = synth.gguf_image(_md(), [], version=2)
    elif case == "missing":
        img = _image(_md(drop=("embedding_length",)))
    elif case == "type":
        img = _image(_md(replace={P + "block_count": ("u64", 1)}))
    elif case == "truncated":
        img = img[:60]
    e = _err(img)
    assert e.code == _lib.SG_ERR_INVALID and msg in e.message, e.message


def _hand_image():
    """A GGUF v3 image assembled field by field in the order reader.go:98-178
    parses it (independent of synth.py): header (magic, version, tensor
    count, metadata count), key/value pairs (u64-length key, u32 value type,
    value), tensor infos (name, u32 n_dims, u64 dims, u32 dtype, u64 offset),
    then the data at the next 32-byte boundary."""
    import struct

    def s(x):
        b = x.encode()
        return struct.pack("<Q", len(b)) + b

    def kv(key, typ, payload):
        return s(key) + struct.pack("<I", typ) + payload

    def arr(typ, items):
        return struct.pack("<IQ", typ, len(items)) + b"".join(items)

    p = "gemma-embedding."
    kvs = [
        kv("general.architecture", 8, s("gemma-embedding")),
        kv("x.u8", 0, struct.pack("<B", 250)), kv("x.i8", 1, struct.pack("<b", -5)),
        kv("x.u16", 2, struct.pack("<H", 65000)), kv("x.i16", 3, struct.pack("<h", -300)),
        kv("x.i32", 5, struct.pack("<i", -70000)), kv("x.u64", 10, struct.pack("<Q", 1 << 40)),
        kv("x.i64", 11, struct.pack("<q", -(1 << 40))), kv("x.f64", 12, struct.pack("<d", 0.5)),
        kv("x.bool", 7, b"\x01"),
        kv("x.nested", 9, arr(9, [arr(0, [b"\x01"]), arr(4, [struct.pack("<I", 2), struct.pack("<I", 3)])])),
        kv(p + "embedding_length", 4, struct.pack("<I", 768)),
        kv(p + "block_count", 4, struct.pack("<I", 2)),
        kv(p + "attention.head_count", 4, struct.pack("<I", 3)),
        kv(p + "attention.head_count_kv", 4, struct.pack("<I", 1)),
        kv(p + "feed_forward_length", 4, struct.pack("<I", 1152)),
        kv(p + "context_length", 4, struct.pack("<I", 512)),
        kv(p + "attention.layer_norm_rms_epsilon", 6, struct.pack("<f", 1e-6)),
        kv(p + "rope.freq_base", 6, struct.pack("<f", 1e6)),
        kv("tokenizer.ggml.tokens", 9, arr(8, [s("<pad>"), s("a"), s("bc")])),
    ]
    tensor = s("output_norm.weight") + struct.pack("<I", 1) + struct.pack("<Q", 4) + struct.pack("<IQ", 0, 0)
    head = b"GGUF" + struct.pack("<IQQ", 3, 1, len(kvs))
    body = head + b"".join(kvs) + tensor
    body += b"\0" * (-len(body) % 32)
    return body + struct.pack("<4f", 1, 2, 3, 4)


def test_hand_assembled_image():
    """parseConfig over an image built byte by byte from the format (not by
    the repository's writer), with every metadata value type and a nested
    array ahead of the model keys."""
    from semantica_gpu import read_gguf_config
    cfg = read_gguf_config(_hand_image())
    assert cfg == {"embed_dim": 768, "num_layers": 2, "num_heads": 3, "num_kv_heads": 1, "interm_dim": 1152,
                   "max_seq_len": 512, "vocab_size": 3, "norm_eps": pytest.approx(1e-6, rel=1e-6),
                   "rope_base": 1e6}


def test_hand_assembled_image_truncations():
    """Every cut inside the header or a key/value pair fails as the reference
    does (header: 'file too small for header'; later: 'read metadata i'),
    never reading past the image."""
    from semantica_gpu import SemanticaError, read_gguf_config
    img = _hand_image()
    for cut in list(range(0, 24, 5)) + list(range(24, 200, 7)):
        with pytest.raises(SemanticaError) as ei:
            read_gguf_config(img[:cut])
        want = "file too small for header" if cut < 24 else "read metadata"
        assert want in ei.value.message, (cut, ei.value.message)


def test_hand_assembled_model_image_config():
    """parseConfig over the full hand-assembled model image (tests/gguf_hand.py:
    every tensor the model reads, at unaligned and out-of-order offsets):
    the configuration its metadata states, with the vocabulary from the
    token list."""
    import gguf_hand
    from semantica_gpu import read_gguf_config
    image, cfg, placed, norms = gguf_hand.hand_model_image()
    assert read_gguf_config(image) == pytest.approx(cfg)
    assert any(a % 32 for a, _ in placed.values())  # some payloads are unaligned
    assert "output_norm.weight" not in placed and "blk.1.attn_k_norm.weight" not in placed
