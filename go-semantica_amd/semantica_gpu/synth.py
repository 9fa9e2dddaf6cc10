"""Deterministic synthetic EmbeddingGemma-300M Q8_0 weights and inputs.

The real GGUF is not available offline, so benchmarks and tests use random
tensors of the exact shapes and byte format the GGUF holds:
  * Q8_0 matrices: GGUF blocks of 34 bytes (little-endian fp16 scale, then 32
    int8), int8 uniform in [-127, 127], scale = fp16(|N(0, 1e-3)|) (about 5% of
    those scales are fp16 subnormals, which exercises the token-embedding
    converter quirk);
  * F32 norm weights uniform in [0.5, 1.5];
  * token IDs uniform in [2, vocab).
All draws use numpy's PCG64 with fixed seeds, so every process (and the CPU
oracle fed the same arrays) sees identical bytes.
"""
from __future__ import annotations

import dataclasses

import numpy as np

# gemma-embedding.* metadata of embeddinggemma-300m (the keys parseConfig
# reads, internal/runtime/model.go:424-517).
EMBEDDINGGEMMA_300M = dict(
    embed_dim=768, num_layers=24, num_heads=3, num_kv_heads=1, interm_dim=1152,
    max_seq_len=2048, vocab_size=262144, norm_eps=1e-6, rope_base=10000.0)

SEED_WEIGHTS = 5
SEED_NORMS = 2
SEED_TOKENS = 0

LAYER_Q8 = ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down")
LAYER_NORMS = ("attn_norm", "attn_q_norm", "attn_k_norm", "post_attention_norm", "ffn_norm", "post_ffw_norm")


def q8_0_random(rng: np.random.Generator, rows: int, cols: int) -> np.ndarray:
    """Raw Q8_0 bytes, shape [rows, cols/32, 34]."""
    assert cols % 32 == 0
    nb = cols // 32
    out = np.empty((rows, nb, 34), np.uint8)
    d = np.abs(rng.normal(0.0, 1e-3, size=(rows, nb))).astype(np.float16)
    out[:, :, 0:2] = d.astype("<f2").view(np.uint8).reshape(rows, nb, 2)
    out[:, :, 2:] = rng.integers(-127, 128, size=(rows, nb, 32), dtype=np.int8).view(np.uint8)
    return out


def q8_0_from_parts(scales_f16: np.ndarray, qs: np.ndarray) -> np.ndarray:
    """Builds raw Q8_0 bytes from fp16 scales [rows, nb] and int8 values [rows, nb*32]."""
    rows, nb = scales_f16.shape
    out = np.empty((rows, nb, 34), np.uint8)
    out[:, :, 0:2] = scales_f16.astype("<f2").view(np.uint8).reshape(rows, nb, 2)
    out[:, :, 2:] = qs.astype(np.int8).reshape(rows, nb, 32).view(np.uint8)
    return out


@dataclasses.dataclass
class SynthModel:
    config: dict
    token_embd: np.ndarray          # uint8 [vocab, d/32, 34]
    output_norm: np.ndarray         # f32 [d]
    layers: list                    # dicts: name -> array

    def layer_shapes(self):
        c = self.config
        d, ff = c["embed_dim"], c["interm_dim"]
        hd = d // c["num_heads"]
        qd, kvd = c["num_heads"] * hd, c["num_kv_heads"] * hd
        return {"attn_q": (qd, d), "attn_k": (kvd, d), "attn_v": (kvd, d), "attn_output": (d, qd),
                "ffn_gate": (ff, d), "ffn_up": (ff, d), "ffn_down": (d, ff)}


def make_model(config: dict | None = None, seed_weights: int = SEED_WEIGHTS,
               seed_norms: int = SEED_NORMS) -> SynthModel:
    c = dict(EMBEDDINGGEMMA_300M if config is None else config)
    d, ff, L = c["embed_dim"], c["interm_dim"], c["num_layers"]
    hd = d // c["num_heads"]
    qd, kvd = c["num_heads"] * hd, c["num_kv_heads"] * hd
    rw = np.random.default_rng(seed_weights)
    rn = np.random.default_rng(seed_norms)
    shapes = {"attn_q": (qd, d), "attn_k": (kvd, d), "attn_v": (kvd, d), "attn_output": (d, qd),
              "ffn_gate": (ff, d), "ffn_up": (ff, d), "ffn_down": (d, ff)}
    norm_len = {"attn_norm": d, "attn_q_norm": hd, "attn_k_norm": hd, "post_attention_norm": d,
                "ffn_norm": d, "post_ffw_norm": d}
    token_embd = q8_0_random(rw, c["vocab_size"], d)
    layers = []
    for _ in range(L):
        ly = {}
        for name in LAYER_Q8:
            ly[name] = q8_0_random(rw, *shapes[name])
        for name in LAYER_NORMS:
            ly[name] = rn.uniform(0.5, 1.5, size=norm_len[name]).astype(np.float32)
        layers.append(ly)
    output_norm = rn.uniform(0.5, 1.5, size=d).astype(np.float32)
    return SynthModel(c, token_embd, output_norm, layers)


def token_ids(n: int, vocab: int, seed: int = SEED_TOKENS) -> np.ndarray:
    return np.random.default_rng(seed).integers(2, vocab, size=n, dtype=np.int64).astype(np.int32)


def offsets_from_lengths(lengths) -> np.ndarray:
    off = np.zeros(len(lengths) + 1, np.int32)
    off[1:] = np.cumsum(np.asarray(lengths, np.int64))
    return off


def lengths_uniform(n: int, lo: int, hi: int, seed: int) -> np.ndarray:
    """Config 3: S ~ U[lo, hi] per row."""
    return np.random.default_rng(seed).integers(lo, hi + 1, size=n).astype(np.int32)


def lengths_log_uniform(n: int, lo: int, hi: int, seed: int) -> np.ndarray:
    """Config 4: S = round(exp(U[ln lo, ln hi]))."""
    u = np.random.default_rng(seed).uniform(np.log(lo), np.log(hi), size=n)
    return np.clip(np.round(np.exp(u)), lo, hi).astype(np.int32)
