"""CPU restatement of the layer glue around the MoE FFN block -- TEST
INFRASTRUCTURE ONLY (see the package docstring for who may import it).

* ``rms_norm``: components/normalization/rms_norm.mlir:18-85 and
  oracles/normalization.py:10-43 -- per row, sum of squares, mean over the
  hidden size, ``sqrt(mean + eps)``, divide, then scale by the weight.
* ``moe_ffn_sublayer``: the MoE FFN sub-layer of
  architectures/llm/transformer_layer_moe_prefill.mlir:205-242 (and
  transformer_layer_moe_decode.mlir:227-255): ``ffn_norm`` RMSNorm of the
  residual stream, ``moe_ffn_block`` on the normalised rows, residual add.
"""

from __future__ import annotations

import numpy as np

from .moe import moe_ffn_block


def rms_norm(x, weight, eps=1e-6, dtype=np.float64):
    """``(x / sqrt(mean(x^2, -1) + eps)) * weight`` in the order of
    rms_norm.mlir:27-83: reduce, divide by the hidden size, add eps, sqrt,
    divide, multiply."""
    x = np.asarray(x, dtype=dtype)
    w = np.asarray(weight, dtype=dtype)
    sum_sq = np.sum(x * x, axis=-1, keepdims=True)
    mean_sq = sum_sq / x.shape[-1]
    rms = np.sqrt(mean_sq + dtype(eps))
    return (x / rms) * w


def moe_ffn_sublayer(
    residual,
    ffn_norm_w,
    rms_eps,
    gate_inp_w,
    up_exps_w,
    gate_exps_w,
    down_exps_w,
    n_expert,
    n_expert_used,
    n_embd,
    n_ff,
    normalize_weights,
    dtype=np.float64,
    return_routing=False,
):
    """``residual + moe_ffn_block(rms_norm(residual, ffn_norm_w, rms_eps), ...)``
    on the flattened ``[n_tokens, n_embd]`` residual stream
    (transformer_layer_moe_prefill.mlir:207-242)."""
    res = np.asarray(residual, dtype=dtype)
    xn = rms_norm(res, ffn_norm_w, rms_eps, dtype=dtype)
    out = moe_ffn_block(xn, gate_inp_w, up_exps_w, gate_exps_w, down_exps_w, n_expert, n_expert_used,
                        n_embd, n_ff, normalize_weights, dtype=dtype, return_routing=return_routing)
    if return_routing:
        moe_out, ids, w = out
        return res + moe_out, ids, w
    return res + out
