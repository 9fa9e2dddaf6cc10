"""A GGUF v3 model image assembled field by field from the format as
internal/gguf/reader.go:98-178 parses it, without the repository's writer
(semantica_gpu/synth.py) or loader, plus a record of where every tensor's
bytes were put.

Layout (reader.go): header (u32 magic "GGUF", u32 version 3, u64 tensor
count, u64 metadata count); key/value pairs (u64-length key, u32 value type,
value); tensor infos (u64-length name, u32 n_dims, u64 dims ne0 first, u32
dtype, u64 offset); tensor data from the next 32-byte boundary
(reader.go:175-176), each tensor at data_start + its offset.  Q8_0 tensors
hold 34-byte blocks (fp16 scale + 32 int8, gguf/tensor.go:94-112), rows of
ne0 elements (model_int8.go:54-140 reads [ne1 rows][ne0/32 blocks]).

The tensors are laid out in the data region in the reverse of their info
order, at offsets that are not all 32-byte aligned (the reference's reader
accepts any offset), with an unused tensor between them.  Weights are drawn
here with numpy: Q8_0 int8 U[-127, 127] with fp16 scales |N(0, 1e-3)| (about
5% of them fp16 subnormals, which the token embedding's halving converter
treats differently, gguf/tensor.go:207-240), norms U[0.5, 1.5].  One norm is
stored as Q8_0 (scale 1/64 and values that are multiples of 1/64, so its
dequantized F32 is exact, model.go:621-651), and three optional norms are
left out (the reference skips them: model_int8.go:66-69 for the QK norms,
:203 / :225 / :236 for the post and output norms).
"""
from __future__ import annotations

import struct

import numpy as np

GGUF_F32, GGUF_Q8_0 = 0, 8
MT_U32, MT_F32, MT_STR, MT_ARR = 4, 6, 8, 9

D, H, HKV, FF = 768, 3, 1, 1152
HD = D // H


def _s(x: str) -> bytes:
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


def _kv(key: str, typ: int, payload: bytes) -> bytes:
    return _s(key) + struct.pack("<I", typ) + payload


def _q8(rng, rows: int, cols: int) -> bytes:
    nb = cols // 32
    d = np.abs(rng.normal(0.0, 1e-3, size=(rows, nb))).astype("<f2")
    q = rng.integers(-127, 128, size=(rows, nb, 32), dtype=np.int8)
    blk = np.empty((rows, nb, 34), np.uint8)
    blk[:, :, :2] = d.view(np.uint8).reshape(rows, nb, 2)
    blk[:, :, 2:] = q.view(np.uint8)
    return blk.tobytes()


def hand_model_image(vocab: int = 96, layers: int = 2, ctx_len: int = 512, eps: float = 1e-5,
                     rope_base: float = 1e6, seed: int = 2024):
    """Returns (image, config, placed, norms):
      config  the model configuration the metadata states;
      placed  {tensor name: (absolute byte offset in image, size in bytes)};
      norms   {tensor name: float32 values} for the norms (the Q8_0-stored one
              as its exact dequantized values); absent optional norms are not
              listed."""
    rng = np.random.default_rng(seed)
    cfg = dict(embed_dim=D, num_layers=layers, num_heads=H, num_kv_heads=HKV, interm_dim=FF, max_seq_len=ctx_len,
               vocab_size=vocab, norm_eps=float(np.float32(eps)), rope_base=float(np.float32(rope_base)))
    p = "gemma-embedding."
    kvs = [
        _kv("general.architecture", MT_STR, _s("gemma-embedding")),
        _kv("general.name", MT_STR, _s("hand-assembled test image")),
        _kv(p + "embedding_length", MT_U32, struct.pack("<I", D)),
        _kv(p + "block_count", MT_U32, struct.pack("<I", layers)),
        _kv(p + "attention.head_count", MT_U32, struct.pack("<I", H)),
        _kv(p + "attention.head_count_kv", MT_U32, struct.pack("<I", HKV)),
        _kv(p + "feed_forward_length", MT_U32, struct.pack("<I", FF)),
        _kv(p + "context_length", MT_U32, struct.pack("<I", ctx_len)),
        _kv(p + "attention.layer_norm_rms_epsilon", MT_F32, struct.pack("<f", eps)),
        _kv(p + "rope.freq_base", MT_F32, struct.pack("<f", rope_base)),
        _kv("tokenizer.ggml.tokens", MT_ARR,
            struct.pack("<IQ", MT_STR, vocab) + b"".join(_s(f"tok{i}") for i in range(vocab))),
    ]
    # (name, dims ne0 first, dtype, bytes)
    tensors = [("token_embd.weight", [D, vocab], GGUF_Q8_0, _q8(rng, vocab, D))]
    norms = {}

    def f32_norm(name, n):
        v = rng.uniform(0.5, 1.5, size=n).astype(np.float32)
        norms[name] = v
        tensors.append((name, [n], GGUF_F32, v.astype("<f4").tobytes()))

    def q8_norm(name, n):
        q = rng.integers(32, 97, size=n).astype(np.int8)  # values q/64 in [0.5, 1.5]
        norms[name] = (q.astype(np.float32) / np.float32(64)).astype(np.float32)
        blk = np.empty((n // 32, 34), np.uint8)
        blk[:, :2] = np.full(n // 32, 1 / 64, "<f2").view(np.uint8).reshape(-1, 2)
        blk[:, 2:] = q.reshape(-1, 32).view(np.uint8)
        tensors.append((name, [n], GGUF_Q8_0, blk.tobytes()))

    absent = {"blk.0.post_ffw_norm.weight", "blk.1.attn_k_norm.weight"}
    for l in range(layers):
        b = f"blk.{l}."
        for name, rows, cols in (("attn_q", H * HD, D), ("attn_k", HKV * HD, D), ("attn_v", HKV * HD, D),
                                 ("attn_output", D, H * HD), ("ffn_gate", FF, D), ("ffn_up", FF, D),
                                 ("ffn_down", D, FF)):
            tensors.append((b + name + ".weight", [cols, rows], GGUF_Q8_0, _q8(rng, rows, cols)))
        for name, n in (("attn_norm", D), ("attn_q_norm", HD), ("attn_k_norm", HD), ("post_attention_norm", D),
                        ("ffn_norm", D), ("post_ffw_norm", D)):
            full = b + name + ".weight"
            if full in absent:
                continue
            if full == "blk.1.ffn_norm.weight":
                q8_norm(full, n)
            else:
                f32_norm(full, n)
    tensors.append(("rope_freqs.weight", [HD // 2], GGUF_F32, np.ones(HD // 2, "<f4").tobytes()))  # unused
    # output_norm.weight is left out (optional)

    # Data region: reverse order, gaps of 0 / 4 / 6 / 38 / 64 bytes in turn.
    gaps = (0, 4, 6, 38, 64)
    offsets, pos = {}, 0
    for i, (name, _, _, raw) in enumerate(reversed(tensors)):
        pos += gaps[i % len(gaps)]
        offsets[name] = pos
        pos += len(raw)
    infos = b"".join(_s(name) + struct.pack("<I", len(dims)) + struct.pack(f"<{len(dims)}Q", *dims) +
                     struct.pack("<IQ", dtype, offsets[name]) for name, dims, dtype, _ in tensors)
    head = b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(kvs))
    meta = head + b"".join(kvs) + infos
    data_start = (len(meta) + 31) // 32 * 32
    image = bytearray(meta + b"\xAB" * (data_start - len(meta)) + b"\xCD" * pos)  # filler bytes, never read
    placed = {}
    for name, _, _, raw in tensors:
        a = data_start + offsets[name]
        image[a:a + len(raw)] = raw
        placed[name] = (a, len(raw))
    return bytes(image), cfg, placed, norms


def oracle_model(image: bytes, cfg: dict, placed: dict, norms: dict):
    """The model as the oracle takes it: each Q8_0 matrix read straight out
    of the image at the offset the assembler put it (no GGUF parsing), the
    norms as the assembler drew them."""
    from semantica_gpu.synth import SynthModel

    def q8(name, rows, cols):
        a, n = placed[name]
        assert n == rows * (cols // 32) * 34
        return np.frombuffer(image, np.uint8, count=n, offset=a).reshape(rows, cols // 32, 34)

    layers = []
    for l in range(cfg["num_layers"]):
        b = f"blk.{l}."
        ly = {"attn_q": q8(b + "attn_q.weight", H * HD, D), "attn_k": q8(b + "attn_k.weight", HKV * HD, D),
              "attn_v": q8(b + "attn_v.weight", HKV * HD, D), "attn_output": q8(b + "attn_output.weight", D, H * HD),
              "ffn_gate": q8(b + "ffn_gate.weight", FF, D), "ffn_up": q8(b + "ffn_up.weight", FF, D),
              "ffn_down": q8(b + "ffn_down.weight", D, FF)}
        for name in ("attn_norm", "attn_q_norm", "attn_k_norm", "post_attention_norm", "ffn_norm", "post_ffw_norm"):
            ly[name] = norms.get(b + name + ".weight")
        layers.append(ly)
    return SynthModel(dict(cfg), q8("token_embd.weight", cfg["vocab_size"], D), None, layers)
