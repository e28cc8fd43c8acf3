"""MI355X-native attention hot path of the Audio8 streaming TTS engine.

Drop-in operators for the reference's serve/fast_kernels.py attention functions, backed by
hand-written gfx950 HIP kernels behind a C ABI (include/a8attn.h, liba8attn.so in this directory):

    bias_rope_store, DecodeAttention, PrefillPlan, prefill_attention   (fast_kernels)
    rope_tables, permute_qk, ref_nsplit, AttnStack, PrefillMeta         (attn_stack)

The directory name contains dashes, so it is loaded under the module name `audio8_turbo_engine_amd`
(see load_package in __graft_entry__.py at the repository root).
"""
from .fast_kernels import (DecodeAttention, PrefillPlan, bias_rope_store, prefill_attention,  # noqa: F401
                           prefill_attention_qkv, prefix_copy, rmsnorm, silu_mul, conv_cl, conv_cl_ws_bytes, conv_out_tanh, snake_cat, ru_cl, gemm_small,
                           gemm_silu_small, gemm_small_norm, fold_norm, gemm_ws_bytes, GemmDispatch)
from .attn_stack import AttnStack, PrefillMeta, permute_qk, ref_nsplit, rope_tables  # noqa: F401
from .slow_stack import SlowStack  # noqa: F401
from ._lib import LIB_PATH, load as load_library, runtime_path, version  # noqa: F401

__all__ = ["bias_rope_store", "DecodeAttention", "PrefillPlan", "prefill_attention", "prefill_attention_qkv",
           "prefix_copy",
           "rmsnorm", "silu_mul", "conv_cl", "conv_out_tanh", "snake_cat", "ru_cl", "gemm_small", "gemm_silu_small", "gemm_small_norm", "fold_norm", "gemm_ws_bytes", "GemmDispatch", "SlowStack", "AttnStack", "PrefillMeta",
           "permute_qk", "ref_nsplit", "rope_tables", "load_library", "LIB_PATH", "version", "runtime_path"]
