"""frank-models_amd: the MoE FFN hot path of stellaraccident/frank-models,
rebuilt for AMD MI355X (gfx950).

Public API (same signatures as the reference's components/oracles):

* ``moe_ffn_block(input, gate_inp_w, up_exps_w, gate_exps_w, down_exps_w,
  n_expert, n_expert_used, n_embd, n_ff, normalize_weights)``
* ``mul_mat_id(weights, input, ids)``
* ``swiglu(gate, up)``
* ``rms_norm(x, weight, eps)`` (oracles/normalization.py:10)
* ``moe_ffn_sublayer(residual, ffn_norm_w, rms_eps, gate_inp_w, up_exps_w,
  gate_exps_w, down_exps_w, n_expert, n_expert_used, n_embd, n_ff,
  normalize_weights)``: ffn_norm, block and residual add of a transformer
  layer (transformer_layer_moe_prefill.mlir:205-242)

and per-layer loading of GGUF-named MoE parameters (``load_moe_layers``,
``save_packed`` / ``load_packed``, ``quantize_fp8``; see ``params``),

the decode step's attention half (the component after the MoE block on
the decode path): ``attention_block_decode(input, positions, k_cached,
v_cached, wq, wk, wv, wo, bq, bk, bv, bo, use_bias, n_head, n_head_kv,
n_embd, rope_freq_base, rope_freq_scale)``, the paged KV cache
(``kvcache_gather``, ``kvcache_scatter_decode``, ``kvcache_scatter_prefill``)
and ``AttentionBlockDecode`` (packed weights; ``.paged`` reads the paged
cache in place),

plus ``router``, ``permute``, ``pack_expert_weights``,
``quantize_expert_weights``, ``QuantizedExpertWeights``,
``PackedExpertWeights`` and ``MoEFFNBlock`` (packed weights + reusable
workspace for repeated calls).  All arithmetic runs in libfmoe.so; import
fails loudly if it has not been built.

The directory name is not a Python identifier; import it with
``importlib.import_module("frank-models_amd")``.
"""

from ._lib import (  # noqa: F401
    FmoeError,
    NoDeviceError,
    hip_runtimes_loaded,
    lib as _load_lib,
)
from .api import (  # noqa: F401
    MoEFFNBlock,
    PackedExpertWeights,
    QuantizedExpertWeights,
    moe_ffn_block,
    moe_ffn_sublayer,
    mul_mat_id,
    pack_expert_weights,
    permute,
    quantize_expert_weights,
    rms_norm,
    router,
    swiglu,
)
from .attention import (  # noqa: F401
    AttentionBlockDecode,
    PackedLinearWeights,
    attention_block_decode,
    kvcache_gather,
    kvcache_scatter_decode,
    kvcache_scatter_prefill,
    pack_linear_weights,
)
from . import _lib as lowlevel  # noqa: F401
from . import params  # noqa: F401
from .params import (  # noqa: F401
    ATTN_HPARAMS,
    AttentionHParams,
    AttentionLayer,
    load_attention_layers,
    HPARAMS,
    MoEFFNLayer,
    MoEHParams,
    load_moe_layers,
    load_packed,
    quantize_fp8,
    save_packed,
)

_load_lib()

__all__ = [
    "moe_ffn_block",
    "mul_mat_id",
    "swiglu",
    "rms_norm",
    "moe_ffn_sublayer",
    "router",
    "permute",
    "pack_expert_weights",
    "quantize_expert_weights",
    "QuantizedExpertWeights",
    "PackedExpertWeights",
    "MoEFFNBlock",
    "MoEFFNLayer",
    "MoEHParams",
    "HPARAMS",
    "load_moe_layers",
    "save_packed",
    "load_packed",
    "quantize_fp8",
    "FmoeError",
    "NoDeviceError",
    "hip_runtimes_loaded",
    "lowlevel",
    "params",
    "attention_block_decode",
    "AttentionBlockDecode",
    "PackedLinearWeights",
    "pack_linear_weights",
    "kvcache_gather",
    "kvcache_scatter_decode",
    "kvcache_scatter_prefill",
    "ATTN_HPARAMS",
    "AttentionHParams",
    "AttentionLayer",
    "load_attention_layers",
]
