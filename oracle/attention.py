"""CPU restatement of the decode step's attention half -- TEST
INFRASTRUCTURE ONLY (see the package docstring for who may import it).

* ``rope``: components/position/rope.mlir:22-110 and oracles/position.py:6-50.
  Adjacent pairs ``(2i, 2i+1)`` rotate by ``pos * freq_scale /
  freq_base^(2i/head_dim)``.
* ``attention_gqa``: components/attention/attention_gqa.mlir:22-165 and
  oracles/attention.py:8-52.  KV head ``h`` serves query heads
  ``h*r .. h*r+r-1`` (r = n_head / n_head_kv; the broadcast + collapse of
  attention_gqa.mlir:81-117).  Softmax over all keys, no mask.
* ``kv_gather`` / ``kv_scatter_decode`` / ``kv_scatter_prefill``: the paged
  cache of components/kvcache/kvcache.mlir and oracles/kvcache.py:51-185.
  The block pool is ``[n_blocks, block_size, n_head_kv, head_dim]``; gather
  zero-fills positions at or past a sequence's context length.
* ``attention_block_decode``: components/attention/attention_block_decode.mlir:52-244.
  Q/K/V projections (+ optional biases), RoPE on Q and the new K, the new
  K/V appended after the ``ctx_len`` cached positions, ``attention_gqa`` with
  scale ``1/sqrt(head_dim)``, output projection (+ bias).  Returns the
  output and the new K (with RoPE) and V for the cache.
* ``attention_decode_paged``: the decode layer's attention sequence
  (architectures/llm/transformer_layer_moe_decode.mlir:180-209): gather of
  ``max_context_len`` positions, ``attention_block_decode``, then
  ``scatter_decode`` of the new K/V.  Because gather zero-fills and the
  attention has no mask, each position in ``[min(ctx_len, max_ctx),
  max_ctx)`` enters the softmax as a key of zeros (score 0, value 0).
* ``attention_sublayer_decode_paged``: attn_norm RMSNorm (layer.rms_norm),
  the paged decode above, residual add
  (transformer_layer_moe_decode.mlir:174-221).
"""

from __future__ import annotations

import numpy as np


def rope(x, positions, freq_base=10000.0, freq_scale=1.0, dtype=np.float64):
    """``x [B, S, H, D]``, ``positions [B, S]`` -> rotated ``[B, S, H, D]``."""
    x = np.asarray(x, dtype=dtype)
    B, S, H, D = x.shape
    half = D // 2
    i = np.arange(half, dtype=dtype)
    freqs = dtype(freq_scale) / np.power(dtype(freq_base), 2 * i / D)
    ang = np.asarray(positions, dtype=dtype)[:, :, None, None] * freqs[None, None, None, :]
    c, s = np.cos(ang), np.sin(ang)
    pairs = x.reshape(B, S, H, half, 2)
    x0, x1 = pairs[..., 0], pairs[..., 1]
    out = np.stack([x0 * c - x1 * s, x0 * s + x1 * c], axis=-1)
    return out.reshape(B, S, H, D)


def attention_gqa(q, k, v, scale, dtype=np.float64):
    """``q [B, Sq, H, D]``, ``k``/``v`` ``[B, Skv, Hkv, D]`` -> ``[B, Sq, H, D]``."""
    q, k, v = (np.asarray(a, dtype=dtype) for a in (q, k, v))
    r = q.shape[2] // k.shape[2]
    k = np.repeat(k, r, axis=2)  # [h0, h0, h1, h1]: head h uses KV head h // r
    v = np.repeat(v, r, axis=2)
    qt, kt, vt = (a.transpose(0, 2, 1, 3) for a in (q, k, v))
    s = np.matmul(qt, kt.transpose(0, 1, 3, 2)) * dtype(scale)
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p = p / p.sum(axis=-1, keepdims=True)
    return np.matmul(p, vt).transpose(0, 2, 1, 3)


def kv_gather(cache, layer, block_tables, context_lens, max_context_len):
    """``cache [n_blocks, bs, Hkv, D]`` -> ``[B, max_context_len, Hkv, D]``;
    positions at or past ``context_lens[layer, b]`` are zero."""
    bt, cl = np.asarray(block_tables)[layer], np.asarray(context_lens)[layer]
    B, bs = bt.shape[0], cache.shape[1]
    out = np.zeros((B, max_context_len) + cache.shape[2:], dtype=cache.dtype)
    for b in range(B):
        n = min(int(cl[b]), max_context_len)
        pos = np.arange(n)
        out[b, :n] = cache[bt[b, pos // bs], pos % bs]
    return out


def kv_scatter_decode(cache, new_vals, block_indices, pos_in_blocks):
    """One new ``[Hkv, D]`` row per sequence into ``cache[block, pos]``; returns
    an updated copy (later rows win on a repeated slot, as in a sequential loop)."""
    out = np.array(cache, copy=True)
    for b in range(len(block_indices)):
        out[int(block_indices[b]), int(pos_in_blocks[b])] = new_vals[b]
    return out


def kv_scatter_prefill(cache, layer, new_vals, block_tables, start_positions, block_size):
    """``new_vals [B, S, Hkv, D]`` at positions ``start + s`` through the block table."""
    out = np.array(cache, copy=True)
    bt = np.asarray(block_tables)[layer]
    for b in range(new_vals.shape[0]):
        for s in range(new_vals.shape[1]):
            p = int(start_positions[b]) + s
            out[int(bt[b, p // block_size]), p % block_size] = new_vals[b, s]
    return out


def attention_block_decode(x, positions, k_cached, v_cached, wq, wk, wv, wo, bq, bk, bv, bo, use_bias,
                           n_head, n_head_kv, n_embd, freq_base=10000.0, freq_scale=1.0, dtype=np.float64):
    """``x [B, n_embd]``, ``positions [B]``, ``k_cached``/``v_cached [B, ctx, Hkv, D]``,
    ``w* [n_in, n_out]`` (``x @ w``) -> ``(out [B, n_embd], k_new [B, Hkv, D], v_new [B, Hkv, D])``."""
    x = np.asarray(x, dtype=dtype)
    B = x.shape[0]
    D = n_embd // n_head
    q = x @ np.asarray(wq, dtype)
    k = x @ np.asarray(wk, dtype)
    v = x @ np.asarray(wv, dtype)
    if use_bias:
        q, k, v = q + np.asarray(bq, dtype), k + np.asarray(bk, dtype), v + np.asarray(bv, dtype)
    Dkv = k.shape[1] // n_head_kv
    pos = np.asarray(positions).reshape(B, 1)
    q = rope(q.reshape(B, 1, n_head, D), pos, freq_base, freq_scale, dtype)
    k = rope(k.reshape(B, 1, n_head_kv, Dkv), pos, freq_base, freq_scale, dtype)
    v = v.reshape(B, 1, n_head_kv, Dkv)
    k_full = np.concatenate([np.asarray(k_cached, dtype), k], axis=1)
    v_full = np.concatenate([np.asarray(v_cached, dtype), v], axis=1)
    attn = attention_gqa(q, k_full, v_full, 1.0 / np.sqrt(dtype(D)), dtype)
    out = attn.reshape(B, n_embd) @ np.asarray(wo, dtype)
    if use_bias:
        out = out + np.asarray(bo, dtype)
    return out, k[:, 0], v[:, 0]


def attention_decode_paged(x, positions, k_cache, v_cache, layer, block_tables, context_lens, max_context_len,
                           block_indices, pos_in_blocks, wq, wk, wv, wo, bq, bk, bv, bo, use_bias, n_head,
                           n_head_kv, n_embd, freq_base=10000.0, freq_scale=1.0, dtype=np.float64):
    """Gather -> ``attention_block_decode`` -> ``scatter_decode``; returns
    ``(out, k_new, v_new, k_cache', v_cache')``."""
    kc = kv_gather(k_cache, layer, block_tables, context_lens, max_context_len)
    vc = kv_gather(v_cache, layer, block_tables, context_lens, max_context_len)
    out, k_new, v_new = attention_block_decode(x, positions, kc, vc, wq, wk, wv, wo, bq, bk, bv, bo, use_bias,
                                               n_head, n_head_kv, n_embd, freq_base, freq_scale, dtype)
    kc2 = kv_scatter_decode(k_cache, k_new.astype(k_cache.dtype), block_indices, pos_in_blocks)
    vc2 = kv_scatter_decode(v_cache, v_new.astype(v_cache.dtype), block_indices, pos_in_blocks)
    return out, k_new, v_new, kc2, vc2


def attention_sublayer_decode_paged(residual, attn_norm_w, rms_eps, positions, k_cache, v_cache, layer,
                                    block_tables, context_lens, max_context_len, block_indices, pos_in_blocks, wq, wk,
                                    wv, wo, bq, bk, bv, bo, use_bias, n_head, n_head_kv, n_embd,
                                    freq_base=10000.0, freq_scale=1.0, dtype=np.float64):
    """The decode layer's attention sub-layer (transformer_layer_moe_decode.mlir:174-221):
    attn_norm RMSNorm, the paged attention, residual add.  Returns
    ``(out, k_new, v_new, k_cache', v_cache')``."""
    from .layer import rms_norm

    xn = rms_norm(residual, attn_norm_w, rms_eps, dtype=dtype)
    out, k_new, v_new, kc, vc = attention_decode_paged(xn, positions, k_cache, v_cache, layer, block_tables,
                                                       context_lens, max_context_len, block_indices, pos_in_blocks,
                                                       wq, wk, wv, wo, bq, bk, bv, bo, use_bias, n_head, n_head_kv,
                                                       n_embd, freq_base, freq_scale, dtype)
    return np.asarray(residual, dtype) + out, k_new, v_new, kc, vc
