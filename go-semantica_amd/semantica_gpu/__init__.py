"""semantica_gpu: Python host side of the MI355X EmbeddingGemma Q8_0 library.

The compute path is libsemantica_gpu.so (hand-written HIP for gfx950); this
package only binds its C ABI and mirrors the reference's host API.
"""
from ._lib import SemanticaError, load  # noqa: F401
from .runtime import (Context, Model, Runtime, read_gguf_config, resolve_dim, supported_dims,  # noqa: F401
                      DEFAULT_EMBED_DIM, SUPPORTED_DIMS)
from . import embed, search, synth, tokenizer  # noqa: F401
