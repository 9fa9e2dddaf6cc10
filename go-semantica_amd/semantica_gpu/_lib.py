"""ctypes binding of libsemantica_gpu.so (the C ABI in include/semantica_gpu.h).

Loading fails loudly when the library has not been built: there is no CPU
fallback anywhere in this package.
"""
from __future__ import annotations

import ctypes
import os

_PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(_PKG_ROOT, "lib", "libsemantica_gpu.so")
HEADER_PATH = os.path.join(os.path.dirname(_PKG_ROOT), "include", "semantica_gpu.h")

SG_OK = 0
SG_ERR_EMPTY = -1
SG_ERR_TOO_LONG = -2
SG_ERR_TOKEN = -3
SG_ERR_DIM = -4
SG_ERR_INVALID = -5
SG_ERR_DEVICE = -6
SG_ERR_NOMEM = -7

SG_ATTN_FAST, SG_ATTN_EXACT = 0, 1

_ERR_NAMES = {
    SG_ERR_EMPTY: "EMPTY",
    SG_ERR_TOO_LONG: "TOO_LONG",
    SG_ERR_TOKEN: "TOKEN",
    SG_ERR_DIM: "DIM",
    SG_ERR_INVALID: "INVALID",
    SG_ERR_DEVICE: "DEVICE",
    SG_ERR_NOMEM: "NOMEM",
}


class SemanticaError(RuntimeError):
    """A failed library call; `code` is the SG_ERR_* status."""

    def __init__(self, code: int, message: str):
        super().__init__(f"{message} [{_ERR_NAMES.get(code, code)}]")
        self.code = code
        self.message = message


class ModelConfig(ctypes.Structure):
    _fields_ = [
        ("embed_dim", ctypes.c_int32),
        ("num_layers", ctypes.c_int32),
        ("num_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("interm_dim", ctypes.c_int32),
        ("max_seq_len", ctypes.c_int32),
        ("vocab_size", ctypes.c_int32),
        ("norm_eps", ctypes.c_float),
        ("rope_base", ctypes.c_float),
    ]


_vp = ctypes.c_void_p


class LayerDesc(ctypes.Structure):
    _fields_ = [(n, _vp) for n in (
        "attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down",
        "attn_norm", "attn_q_norm", "attn_k_norm", "post_attention_norm", "ffn_norm", "post_ffw_norm")]


class ModelDesc(ctypes.Structure):
    _fields_ = [
        ("config", ModelConfig),
        ("token_embd", _vp),
        ("output_norm", _vp),
        ("layers", ctypes.POINTER(LayerDesc)),
    ]


SG_K_CLASSES = 8
KERNEL_CLASSES = ("gemm", "attention", "quantize", "norm", "gelu", "pool", "other", "gemm_norm")


class TokenizerConfig(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in ("add_bos", "add_eos", "lowercase", "remove_accents", "nfkc",
                                                "bos_id", "eos_id", "unk_id", "pad_id")]


class Profile(ctypes.Structure):
    _fields_ = [("ms", ctypes.c_double * SG_K_CLASSES), ("work", ctypes.c_double * SG_K_CLASSES),
                ("launches", ctypes.c_int64 * SG_K_CLASSES)]


_i32 = ctypes.c_int32
_f32 = ctypes.c_float
_pp = ctypes.POINTER(ctypes.c_void_p)

# name -> (restype, argtypes)
_PROTOS = {
    "sg_init": (ctypes.c_int, [ctypes.c_int, _pp]),
    "sg_shutdown": (None, [_vp]),
    "sg_last_error": (ctypes.c_char_p, []),
    "sg_abi_version": (ctypes.c_int, []),
    "sg_model_load": (ctypes.c_int, [_vp, ctypes.POINTER(ModelDesc), _pp]),
    "sg_model_free": (None, [_vp]),
    "sg_gguf_read_config": (ctypes.c_int, [_vp, ctypes.c_size_t, ctypes.POINTER(ModelConfig)]),
    "sg_model_load_gguf": (ctypes.c_int, [_vp, _vp, ctypes.c_size_t, _pp]),
    "sg_model_load_gguf_file": (ctypes.c_int, [_vp, ctypes.c_char_p, _pp]),
    "sg_forward": (ctypes.c_int, [_vp, _vp, _vp, _i32, _i32, _vp]),
    "sg_forward_device": (ctypes.c_int, [_vp, _vp, _vp, _i32, _i32, _vp, _vp]),
    "sg_forward_hidden": (ctypes.c_int, [_vp, _vp, _vp, _i32, _i32, _vp, _vp]),
    "sg_forward_trace": (ctypes.c_int, [_vp, _vp, _vp, _i32, _i32, _vp, _vp, _vp, _vp]),
    "sg_profile_enable": (ctypes.c_int, [_vp, ctypes.c_int]),
    "sg_profile_read": (ctypes.c_int, [_vp, ctypes.POINTER(Profile)]),
    "sg_q8_weight_create": (ctypes.c_int, [_vp, _vp, _i32, _i32, _pp]),
    "sg_q8_weight_free": (None, [_vp]),
    "sg_quantize_act": (ctypes.c_int, [_vp, _vp, _i32, _i32, _vp, _i32, _vp, _vp, _vp]),
    "sg_matmul_q8_0_int8": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _i32, _vp]),
    "sg_matmul_q8_0_int8_noalloc": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _i32, _vp]),
    "sg_matmul_q8_0_int8_bench": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _i32, _i32, _vp,
                                                 ctypes.POINTER(ctypes.c_float)]),
    "sg_q8_block_sums": (ctypes.c_int, [_vp, _vp, _vp, _vp, _i32, _vp]),
    "sg_hbm_probe": (ctypes.c_int, [_vp, _i32, _vp, _vp, _vp, ctypes.c_int64, _i32, _vp,
                                    ctypes.POINTER(ctypes.c_float)]),
    "sg_issue_probe": (ctypes.c_int, [_vp, _i32, _i32, _i32, _vp, ctypes.POINTER(ctypes.c_float),
                                      ctypes.POINTER(ctypes.c_float)]),
    "sg_ffn_gate_up": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _i32, _vp]),
    "sg_rmsnorm": (ctypes.c_int, [_vp, _vp, _vp, _vp, _i32, _i32, _f32, _vp]),
    "sg_qknorm_rope": (ctypes.c_int, [_vp, _vp, _i32, _vp, _i32, _vp, _vp, _i32, _i32, _i32, _f32, _f32,
                                      _i32, _vp, _i32, _vp]),
    "sg_attention": (ctypes.c_int, [_vp, _vp, _vp, _i32, _vp, _vp, _i32, _i32, _i32, _i32, _vp, _i32, _vp]),
    "sg_attention_exact": (ctypes.c_int, [_vp, _vp, _vp, _i32, _vp, _vp, _i32, _i32, _i32, _i32, _vp, _i32, _vp]),
    "sg_model_set_attention_mode": (ctypes.c_int, [_vp, ctypes.c_int]),
    "sg_gelu_quick_mul": (ctypes.c_int, [_vp, _vp, _i32, _vp, _i32, _vp, _i32, _i32, _i32, _vp]),
    "sg_embed_tokens": (ctypes.c_int, [_vp, _vp, _vp, _i32, _vp]),
    "sg_pool_l2": (ctypes.c_int, [_vp, _vp, _vp, _i32, _i32, _vp, _i32, _vp]),
    "sg_index_build": (ctypes.c_int, [_vp, _i32, _i32, _vp, _vp, _i32, _pp]),
    "sg_index_build_device": (ctypes.c_int, [_vp, _i32, _i32, _vp, _vp, ctypes.c_int64, _i32, _vp, _pp]),
    "sg_index_deserialize": (ctypes.c_int, [_vp, _vp, ctypes.c_size_t, _pp]),
    "sg_index_serialize": (ctypes.c_int, [_vp, _vp, ctypes.c_size_t, ctypes.POINTER(ctypes.c_size_t)]),
    "sg_index_info": (ctypes.c_int, [_vp, ctypes.POINTER(_i32), ctypes.POINTER(_i32), ctypes.POINTER(_i32)]),
    "sg_index_vector": (ctypes.c_int, [_vp, _i32, _vp]),
    "sg_index_search": (ctypes.c_int, [_vp, _vp, _i32, _i32, _i32, _vp, _vp, _vp, _vp]),
    "sg_index_free": (None, [_vp]),
    "sg_tokenizer_create": (ctypes.c_int, [_vp, _vp, _vp, _vp, _i32, _vp, _pp]),
    "sg_tokenizer_from_gguf": (ctypes.c_int, [_vp, ctypes.c_size_t, _pp]),
    "sg_tokenizer_from_gguf_file": (ctypes.c_int, [ctypes.c_char_p, _pp]),
    "sg_tokenizer_encode": (ctypes.c_int, [_vp, _vp, ctypes.c_size_t, _vp, _i32, ctypes.POINTER(_i32)]),
    "sg_tokenizer_encode_batch": (ctypes.c_int, [_vp, _vp, _vp, _i32, _vp, ctypes.c_int64, _vp]),
    "sg_tokenizer_decode": (ctypes.c_int, [_vp, _vp, _i32, _vp, ctypes.c_size_t, ctypes.POINTER(ctypes.c_size_t)]),
    "sg_tokenizer_vocab_size": (_i32, [_vp]),
    "sg_tokenizer_free": (None, [_vp]),
}

_lib = None


def exported_names():
    return sorted(_PROTOS)


def load():
    """Returns the loaded library; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
            "or `make -C go-semantica_amd`")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in _PROTOS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(code: int):
    if code != SG_OK:
        msg = load().sg_last_error()
        raise SemanticaError(code, msg.decode() if msg else "unknown error")
