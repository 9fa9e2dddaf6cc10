"""Host-side mirror of the reference's model and runtime API over the C ABI.

  Model.forward_with_dim(token_ids, target_dim)   <- (*Model).ForwardWithDim,
                                                     internal/runtime/model.go:661-667
  Model.forward_batch(sequences, target_dim)      <- embedPrompts' per-sequence fan-out,
                                                     pkg/ggufembed/api.go:237-295, as one
                                                     packed GPU call
  Runtime.embed_tokens(sequences, dim)            <- Runtime.Embed / EmbedInputs
                                                     (api.go:90-112) with token IDs in
                                                     place of texts (the tokenizer is host
                                                     code outside this library)
  Model.from_gguf(ctx, image_or_path)             <- LoadModelFromBytes / LoadModel,
                                                     internal/runtime/model.go:236-262
  read_gguf_config(image)                         <- parseConfig, model.go:424-517
  resolve_dim / supported_dims                    <- ggufembed.ResolveDim / SupportedDims
                                                     (pkg/ggufembed/tasks.go:80-117)

Errors surface as SemanticaError with the reference's messages ("empty
input", "sequence too long: %d > %d", "token ID out of range: %d",
"target dimension %d out of range (1..%d)").
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib
from .synth import SynthModel

DEFAULT_EMBED_DIM = 512
SUPPORTED_DIMS = (768, 512, 256, 128)


def resolve_dim(dim: int) -> int:
    """ResolveDim, pkg/ggufembed/tasks.go:101-110: 0 -> 512; else one of 768/512/256/128."""
    if dim == 0:
        return DEFAULT_EMBED_DIM
    if dim not in SUPPORTED_DIMS:
        raise ValueError(f"unsupported embed dim {dim} (allowed: 768, 512, 256, 128)")
    return dim


def supported_dims():
    return list(SUPPORTED_DIMS)


def _ptr(a: np.ndarray):
    return ctypes.c_void_p(a.ctypes.data)


class Context:
    """One GPU (sg_init)."""

    def __init__(self, device: int = 0):
        self.lib = _lib.load()
        h = ctypes.c_void_p()
        _lib.check(self.lib.sg_init(device, ctypes.byref(h)))
        self.handle = h

    def close(self):
        if self.handle:
            self.lib.sg_shutdown(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


def model_desc(model: SynthModel):
    """Builds an sg_model_desc (plus the arrays it points into, which must stay alive)."""
    c = model.config
    keep = []

    def p(a):
        a = np.ascontiguousarray(a)
        keep.append(a)
        return a.ctypes.data

    L = c["num_layers"]
    layers = (_lib.LayerDesc * L)()
    for i, ly in enumerate(model.layers):
        for name in _lib.LayerDesc._fields_:
            key = name[0]
            arr = ly.get(key)
            setattr(layers[i], key, p(arr) if arr is not None else None)
    cfg = _lib.ModelConfig(c["embed_dim"], c["num_layers"], c["num_heads"], c["num_kv_heads"],
                           c["interm_dim"], c["max_seq_len"], c["vocab_size"], c["norm_eps"],
                           c["rope_base"])
    desc = _lib.ModelDesc(cfg, p(model.token_embd),
                          p(model.output_norm) if model.output_norm is not None else None, layers)
    keep.append(layers)
    return desc, keep


_CONFIG_FIELDS = ("embed_dim", "num_layers", "num_heads", "num_kv_heads", "interm_dim", "max_seq_len",
                  "vocab_size", "norm_eps", "rope_base")


def read_gguf_config(image: bytes) -> dict:
    """parseConfig (internal/runtime/model.go:424-517) over a GGUF v3 image."""
    lib = _lib.load()
    buf = ctypes.create_string_buffer(bytes(image), len(image))
    cfg = _lib.ModelConfig()
    _lib.check(lib.sg_gguf_read_config(buf, len(image), ctypes.byref(cfg)))
    return {k: getattr(cfg, k) for k in _CONFIG_FIELDS}


class Model:
    """Weights resident on one GPU (sg_model_load) and the batched forward."""

    def __init__(self, ctx: Context, model: SynthModel):
        self.ctx = ctx
        self.lib = ctx.lib
        self.config = dict(model.config)
        desc, keep = model_desc(model)
        h = ctypes.c_void_p()
        _lib.check(self.lib.sg_model_load(ctx.handle, ctypes.byref(desc), ctypes.byref(h)))
        del keep
        self.handle = h

    @classmethod
    def from_gguf(cls, ctx: Context, source) -> "Model":
        """LoadModelFromBytes / LoadModel (model.go:236-262): a GGUF image (bytes)
        or a file path (str / os.PathLike)."""
        self = cls.__new__(cls)
        self.ctx = ctx
        self.lib = ctx.lib
        h = ctypes.c_void_p()
        if isinstance(source, (bytes, bytearray, memoryview)):
            image = bytes(source)
            buf = ctypes.create_string_buffer(image, len(image))
            _lib.check(self.lib.sg_model_load_gguf(ctx.handle, buf, len(image), ctypes.byref(h)))
            self.config = read_gguf_config(image)
        else:
            import os
            path = os.fspath(source)
            _lib.check(self.lib.sg_model_load_gguf_file(ctx.handle, path.encode(), ctypes.byref(h)))
            with open(path, "rb") as f:
                self.config = read_gguf_config(f.read())
        self.handle = h
        return self

    def close(self):
        if self.handle:
            self.lib.sg_model_free(self.handle)
            self.handle = None

    @property
    def embed_dim(self):
        return self.config["embed_dim"]

    @property
    def max_seq_len(self):
        return self.config["max_seq_len"]

    def forward_packed(self, tokens: np.ndarray, offsets: np.ndarray, target_dim: int) -> np.ndarray:
        tokens = np.ascontiguousarray(tokens, np.int32)
        offsets = np.ascontiguousarray(offsets, np.int32)
        n = len(offsets) - 1
        out = np.empty((max(n, 0), target_dim), np.float32)
        _lib.check(self.lib.sg_forward(self.handle, _ptr(tokens), _ptr(offsets), n, target_dim, _ptr(out)))
        return out

    def forward_batch(self, sequences, target_dim: int) -> np.ndarray:
        lens = [len(s) for s in sequences]
        off = np.zeros(len(lens) + 1, np.int32)
        off[1:] = np.cumsum(lens)
        toks = np.concatenate([np.asarray(s, np.int32) for s in sequences]) if lens and off[-1] else \
            np.zeros(1, np.int32)
        return self.forward_packed(toks, off, target_dim)

    def forward_with_dim(self, token_ids, target_dim: int) -> np.ndarray:
        return self.forward_batch([token_ids], target_dim)[0]

    def forward_device(self, d_tokens_ptr: int, offsets: np.ndarray, target_dim: int, d_out_ptr: int,
                       stream: int = 0):
        """sg_forward_device with device pointers (e.g. torch tensors' data_ptr())."""
        offsets = np.ascontiguousarray(offsets, np.int32)
        _lib.check(self.lib.sg_forward_device(self.handle, ctypes.c_void_p(d_tokens_ptr), _ptr(offsets),
                                              len(offsets) - 1, target_dim, ctypes.c_void_p(d_out_ptr),
                                              ctypes.c_void_p(stream) if stream else None))


    def forward_hidden(self, d_tokens_ptr: int, offsets: np.ndarray, n_layers: int, d_hidden_ptr: int,
                       stream: int = 0):
        """sg_forward_hidden: residual stream after n_layers layers into a [T, embed_dim] device buffer."""
        offsets = np.ascontiguousarray(offsets, np.int32)
        _lib.check(self.lib.sg_forward_hidden(self.handle, ctypes.c_void_p(d_tokens_ptr), _ptr(offsets),
                                              len(offsets) - 1, n_layers, ctypes.c_void_p(d_hidden_ptr),
                                              ctypes.c_void_p(stream) if stream else None))

    def forward_trace(self, d_tokens_ptr: int, offsets: np.ndarray, n_layers: int, d_qkv_ptr: int = 0,
                      d_att_ptr: int = 0, d_h_ptr: int = 0, stream: int = 0):
        """sg_forward_trace: per-layer Q|K|V, attention output and residual stream
        into [n_layers, T, cols] device buffers (0 skips one)."""
        offsets = np.ascontiguousarray(offsets, np.int32)
        vp = lambda x: ctypes.c_void_p(x) if x else None  # noqa: E731
        _lib.check(self.lib.sg_forward_trace(self.handle, ctypes.c_void_p(d_tokens_ptr), _ptr(offsets),
                                             len(offsets) - 1, n_layers, vp(d_qkv_ptr), vp(d_att_ptr), vp(d_h_ptr),
                                             vp(stream)))

    def set_attention_mode(self, mode: int):
        """sg_model_set_attention_mode: _lib.SG_ATTN_FAST (matrix cores, the
        default) or _lib.SG_ATTN_EXACT (the reference's float32 order: the
        forward then gives the block-serial path's bits)."""
        _lib.check(self.lib.sg_model_set_attention_mode(self.handle, int(mode)))

    def profile_enable(self, on: bool = True):
        _lib.check(self.lib.sg_profile_enable(self.handle, 1 if on else 0))

    def profile_read(self) -> dict:
        """Per kernel class: {"ms", "work", "launches"} accumulated since profile_enable."""
        p = _lib.Profile()
        _lib.check(self.lib.sg_profile_read(self.handle, ctypes.byref(p)))
        return {name: {"ms": p.ms[i], "work": p.work[i], "launches": p.launches[i]}
                for i, name in enumerate(_lib.KERNEL_CLASSES)}


class Runtime:
    """Runtime.Embed surface over token IDs (api.go:90-107)."""

    def __init__(self, model: Model):
        self.model = model

    def embed_dim(self):
        return self.model.embed_dim

    def max_seq_len(self):
        return self.model.max_seq_len

    def embed_tokens(self, sequences, dim: int = 0):
        if len(sequences) == 0:
            return []
        d = resolve_dim(dim)
        return [row for row in self.model.forward_batch(sequences, d)]
