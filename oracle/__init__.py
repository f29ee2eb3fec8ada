"""CPU oracle for the MoE FFN hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, in NumPy, the arithmetic of the reference's
``moe_ffn_block`` / ``mul_mat_id`` / ``swiglu`` path:

* components/moe/moe_ffn_block.mlir:34-209 and oracles/moe.py:51-132
* components/moe/mul_mat_id.mlir:22-120 and oracles/moe.py:9-48
* components/activation/swiglu.mlir:16-51 and oracles/activation.py:6-21
* the layer glue (``layer.py``): components/normalization/rms_norm.mlir:18-85
  and oracles/normalization.py:10-43; the MoE FFN sub-layer of
  architectures/llm/transformer_layer_moe_prefill.mlir:205-242

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only as the checker (or, for the CPU
baseline, as the thing timed on the host).  The product path
(``frank-models_amd``) never imports, links or executes anything here.

Parity pins (each function's checks live in ``tests/test_oracle.py``):

* ``swiglu`` / ``silu``: closed form, known answers (zeros, u=0, large u),
  torch ``F.silu`` cross-check, a planted operand swap that must fail.
* ``router``: float64 closed form, softmax invariants (sum to 1,
  shift-invariance, equal logits -> 1/E), brute-force top-k on tiny inputs,
  hand-built ties resolved toward the lower expert index, renormalisation
  invariants.
* ``permute``: brute-force loops and the ``argsort(kind="stable")`` +
  ``bincount`` closed form, the reference's hand-written id arrays
  (tests/components/test_mul_mat_id.py:23-25, :42-48, :64).
* ``mul_mat_id`` (grouped) vs ``mul_mat_id_literal`` (the reference's
  gather + einsum formula) vs a pure-Python triple loop; identity weights,
  one-hot inputs, all-ids-equal reduces to a dense GEMM.
* ``moe_ffn_block`` (grouped) vs ``moe_ffn_block_literal``; E=k=1 and
  identical-experts reductions to a dense SwiGLU FFN.
* ``bf16_round`` / ``e4m3fn_*``: bit-pattern closed forms cross-checked
  against torch's ``bfloat16`` / ``float8_e4m3fn`` casts.
* ``rms_norm``: constant rows (closed form ``c / sqrt(c^2 + eps)``), one-hot
  rows, scale invariance at eps = 0, unit RMS of the output at unit weight,
  torch ``rms_norm`` cross-check, planted mistakes (sum instead of mean, eps
  outside the square root, weight dropped) that must fail.
* ``moe_ffn_sublayer``: zero expert weights leave the residual unchanged;
  the residual add is linear (sub-layer minus residual equals the pinned
  block on the pinned norm's output).

Parity unpinned: the reference oracle's order for EXACT probability ties
(``np.argsort(-probs, axis=0)`` is not a stable sort, oracles/moe.py:95-97).
This restatement breaks ties toward the lower expert index, the rule the
drop-in implements; the synthetic inputs exclude near-ties.
"""

from .moe import (  # noqa: F401
    silu,
    swiglu,
    router,
    permute,
    mul_mat_id,
    mul_mat_id_literal,
    mul_mat_id_loops,
    moe_ffn_block,
    moe_ffn_block_literal,
    moe_ffn_block_tokens,
)
from .layer import rms_norm, moe_ffn_sublayer  # noqa: F401
from .numerics import (  # noqa: F401
    bf16_round,
    e4m3fn_decode,
    e4m3fn_encode,
    quantize_per_channel_e4m3fn,
)
