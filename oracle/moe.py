"""NumPy restatement of the reference MoE FFN path (test infrastructure only).

Two forms of every projection are kept:

* ``*_literal``: the reference's own decomposition -- transpose the weights,
  gather one whole expert matrix per (slot, token) assignment, batched
  mat-vec, transpose back (components/moe/mul_mat_id.mlir:37-117,
  oracles/moe.py:29-48).  It materialises ``[k, T, n_out, n_in]`` and is
  only usable on small shapes.
* the default (expert-grouped) form: for every expert that is routed to,
  gather its assignments and run one BLAS GEMM.  Arithmetically the same
  sums; it runs at every BASELINE size.

``dtype`` selects the arithmetic type (float64 by default, the tightest
reference; float32 reproduces the reference oracle's precision).
"""

from __future__ import annotations

import numpy as np

from . import numerics as _nm

# The literal gather refuses to materialise more than this many bytes.
LITERAL_BUDGET_BYTES = 2 << 30


def silu(x: np.ndarray) -> np.ndarray:
    """``x / (1 + exp(-x))`` (oracles/activation.py:6-8; swiglu.mlir:40-45)."""
    return x / (1 + np.exp(-x))


def swiglu(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    """``gate * silu(up)`` -- silu acts on ``up`` (oracles/activation.py:11-21;
    components/activation/swiglu.mlir:37-47)."""
    return gate * silu(up)


def router_probs(input: np.ndarray, gate_inp_w: np.ndarray, dtype=np.float64) -> np.ndarray:
    """Softmax over experts of ``gate_inp_w @ input.T`` -> ``[E, T]``.

    moe_ffn_block.mlir:50-75 (transpose + linalg.matmul + softmax dim 0);
    oracles/moe.py:86-91 (max-subtracted softmax).
    """
    x = np.asarray(input, dtype=dtype)
    wr = np.asarray(gate_inp_w, dtype=dtype)
    logits = wr @ x.T
    e = np.exp(logits - logits.max(axis=0, keepdims=True))
    return e / e.sum(axis=0, keepdims=True)


def router(
    input: np.ndarray,
    gate_inp_w: np.ndarray,
    n_expert_used: int,
    normalize_weights: bool,
    dtype=np.float64,
):
    """Router -> ``(ids [k, T] int32, weights [k, T])``.

    Top-k runs on the probabilities, slot 0 holding the largest
    (moe_ffn_block.mlir:77-89, comparator ``ogt``; oracles/moe.py:93-100).
    Exact ties go to the lower expert index: a stable sort of ``-probs``
    keeps equal keys in ascending index order.  Optional renormalisation
    divides by the slot sum (moe_ffn_block.mlir:91-128; oracles/moe.py:102-105).
    """
    probs = router_probs(input, gate_inp_w, dtype)
    k = int(n_expert_used)
    if not 1 <= k <= probs.shape[0]:
        raise ValueError(f"n_expert_used={k} outside [1, {probs.shape[0]}]")
    ids = np.argsort(-probs, axis=0, kind="stable")[:k]
    weights = np.take_along_axis(probs, ids, axis=0)
    if normalize_weights:
        weights = weights / weights.sum(axis=0, keepdims=True)
    return ids.astype(np.int32), weights


def permute(ids: np.ndarray, n_expert: int):
    """Token->expert permutation: ``(order [k*T] int32, offsets [E+1] int32)``.

    The reference has no permutation; its gather walks assignments in the
    slot-major flat order ``f = s*T + t`` of ``collapse_shape ids [[0, 1]]``
    (mul_mat_id.mlir:50-61).  The drop-in groups that same flat order by
    expert, stably: ``order[offsets[e] + r]`` is the r-th smallest ``f``
    routed to expert ``e``.
    """
    flat = np.asarray(ids, dtype=np.int64).reshape(-1)
    if flat.size and (flat.min() < 0 or flat.max() >= n_expert):
        raise ValueError("ids outside [0, n_expert)")
    order = np.argsort(flat, kind="stable").astype(np.int32)
    counts = np.bincount(flat, minlength=n_expert)
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    return order, offsets


def mul_mat_id_literal(weights: np.ndarray, input: np.ndarray, ids: np.ndarray,
                       budget_bytes: int = LITERAL_BUDGET_BYTES) -> np.ndarray:
    """The reference's gather + batched mat-vec, step for step
    (mul_mat_id.mlir:37-117; oracles/moe.py:29-48).  Small shapes only: the
    gathered weights may take at most ``budget_bytes``."""
    n_out, n_in, n_expert = weights.shape
    k, T = ids.shape
    need = k * T * n_out * n_in * weights.dtype.itemsize
    if need > budget_bytes:
        raise MemoryError(f"literal mul_mat_id would materialise {need / 1e9:.1f} GB")
    weights_t = weights.transpose(2, 0, 1)  # [E, n_out, n_in]
    gathered = weights_t[ids]  # [k, T, n_out, n_in]
    input_t = input.transpose(1, 2, 0)  # [k, T, n_in]
    out = np.einsum("etoi,eti->eto", gathered, input_t)
    return out.transpose(2, 0, 1)  # [n_out, k, T]


def mul_mat_id_loops(weights, input, ids):
    """Pure-Python triple loop ``out[o, s, t] = sum_i W[o, i, ids[s, t]] * in[i, s, t]``
    (the definition in mul_mat_id.mlir:8-11).  Tiny inputs only."""
    n_out, n_in, _ = weights.shape
    k, T = ids.shape
    out = np.zeros((n_out, k, T), dtype=np.float64)
    for s in range(k):
        for t in range(T):
            e = int(ids[s, t])
            for o in range(n_out):
                acc = 0.0
                for i in range(n_in):
                    acc += float(weights[o, i, e]) * float(input[i, s, t])
                out[o, s, t] = acc
    return out


def mul_mat_id(weights: np.ndarray, input: np.ndarray, ids: np.ndarray, dtype=np.float64) -> np.ndarray:
    """Expert-grouped ``mul_mat_id``: same sums as the literal form, one GEMM
    per routed expert.  ``weights [n_out, n_in, E]``, ``input [n_in, k, T]``,
    ``ids [k, T]`` -> ``[n_out, k, T]`` (oracles/moe.py:9-28 signature)."""
    n_out, n_in, n_expert = weights.shape
    k, T = ids.shape
    if input.shape != (n_in, k, T):
        raise ValueError(f"input shape {input.shape} != {(n_in, k, T)}")
    x = np.asarray(input, dtype=dtype).reshape(n_in, k * T).T  # row f = s*T + t
    flat = np.asarray(ids).reshape(-1)
    out = np.zeros((k * T, n_out), dtype=dtype)
    for e in np.unique(flat):
        rows = np.nonzero(flat == e)[0]
        w = np.ascontiguousarray(weights[:, :, int(e)], dtype=dtype)  # [n_out, n_in]
        out[rows] = x[rows] @ w.T
    return np.ascontiguousarray(out.T).reshape(n_out, k, T)


def moe_ffn_block_literal(
    input,
    gate_inp_w,
    up_exps_w,
    gate_exps_w,
    down_exps_w,
    n_expert,
    n_expert_used,
    n_embd,
    n_ff,
    normalize_weights,
    dtype=np.float32,
    budget_bytes=LITERAL_BUDGET_BYTES,
):
    """The reference block step for step (moe_ffn_block.mlir:46-208;
    oracles/moe.py:84-132): replicate the input per slot, three literal
    ``mul_mat_id`` calls, SwiGLU, weight, slot-sum, transpose."""
    x = np.asarray(input, dtype=dtype)
    ids, w = router(x, np.asarray(gate_inp_w, dtype), n_expert_used, normalize_weights, dtype)
    T = x.shape[0]
    k = int(n_expert_used)
    xr = np.broadcast_to(x.T[:, None, :], (n_embd, k, T)).copy()
    up = mul_mat_id_literal(np.asarray(up_exps_w, dtype), xr, ids, budget_bytes)
    gate = mul_mat_id_literal(np.asarray(gate_exps_w, dtype), xr, ids, budget_bytes)
    act = swiglu(gate, up)
    y = mul_mat_id_literal(np.asarray(down_exps_w, dtype), act, ids, budget_bytes)
    y = y * w[None, :, :].astype(dtype)
    return y.sum(axis=1).T


def moe_ffn_block(
    input,
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
    act_quant=False,
):
    """Expert-grouped ``moe_ffn_block`` (same positional signature as
    oracles/moe.py:51-62).  Weighted expert outputs are summed in slot order
    s = 0..k-1, as the reduction at moe_ffn_block.mlir:179-193.

    ``act_quant=True`` is the fp8-activation variant (no counterpart in the
    reference): the GEMM inputs -- the token rows, and the SwiGLU rows after
    rounding to bf16 -- are replaced by their per-row e4m3 quantisation
    (``numerics.fake_quantize_rows_e4m3fn``); routing still uses the
    unquantised rows.  ``act_quant="x2"`` replaces them by their two-term
    quantisation instead (``numerics.fake_quantize_rows_e4m3fn_x2``)."""
    if act_quant not in (False, True, "x2"):
        raise ValueError(f"act_quant must be False, True or 'x2', not {act_quant!r}")
    fq = _nm.fake_quantize_rows_e4m3fn_x2 if act_quant == "x2" else _nm.fake_quantize_rows_e4m3fn
    x = np.asarray(input, dtype=dtype)
    T, H = x.shape
    if H != n_embd:
        raise ValueError(f"input hidden {H} != n_embd {n_embd}")
    ids, w = router(x, gate_inp_w, n_expert_used, normalize_weights, dtype)
    xg = fq(x).astype(dtype) if act_quant else x
    k = int(n_expert_used)
    y = np.zeros((k, T, H), dtype=dtype)
    for e in np.unique(ids):
        s_idx, t_idx = np.nonzero(ids == e)
        xe = xg[t_idx]
        # Contiguous per-expert copies keep the products on BLAS (a strided
        # expert slice would send NumPy down its element-wise matmul loop).
        up = xe @ np.ascontiguousarray(up_exps_w[:, :, int(e)], dtype=dtype).T
        gate = xe @ np.ascontiguousarray(gate_exps_w[:, :, int(e)], dtype=dtype).T
        h = swiglu(gate, up)
        if act_quant:
            h = fq(_nm.bf16_round(h)).astype(dtype)
        d = h @ np.ascontiguousarray(down_exps_w[:, :, int(e)], dtype=dtype).T
        y[s_idx, t_idx] = d * w[s_idx, t_idx][:, None]
    out = y[0].copy()
    for s in range(1, k):
        out += y[s]
    if return_routing:
        return out, ids, w
    return out


def moe_ffn_block_tokens(token_idx, input, *args, **kwargs):
    """The block evaluated on a subset of tokens.  Each token routes and
    mixes independently (moe_ffn_block.mlir:21), so these rows equal the
    same rows of the full-batch result."""
    return moe_ffn_block(np.asarray(input)[np.asarray(token_idx)], *args, **kwargs)
