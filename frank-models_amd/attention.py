"""Host mirror of the decode step's attention half: the paged KV cache
(components/kvcache/kvcache.mlir; oracles/kvcache.py) and
``attention_block_decode`` (components/attention/attention_block_decode.mlir:52-244),
running on libfmoe.so's kernels through the C ABI.

Value semantics follow the rest of the package: NumPy inputs are copied to
the device and a NumPy array comes back; device tensors stay on the device
and the call is asynchronous on torch's current stream.  The cache
functions update a device pool in place (the reference's value-semantics
copy is what the NumPy form returns).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import numpy as np
import torch

from . import _lib as L
from .api import _DT_TO_TORCH, _TORCH_TO_DT, _device, _dtype_code, _finish, _ptr, _stream, _to_device, _workspace


def _ints_to_device(a, name: str, dtype=torch.int32) -> torch.Tensor:
    if isinstance(a, np.ndarray):
        if not np.issubdtype(a.dtype, np.integer):
            raise TypeError(f"{name}: integer dtype expected, got {a.dtype}")
        return torch.from_numpy(np.ascontiguousarray(a)).to(_device(), dtype)
    if isinstance(a, torch.Tensor):
        if a.dtype.is_floating_point or a.dtype == torch.bool:
            raise TypeError(f"{name}: integer dtype expected, got {a.dtype}")
        return a.to(_device(), dtype).contiguous()
    raise TypeError(f"{name}: expected numpy.ndarray or torch.Tensor, got {type(a).__name__}")


def _pool(cache, name="cache"):
    t, from_np = _to_device(cache, name)
    if t.dim() != 4:
        raise ValueError(f"{name} must be [n_blocks, block_size, n_head_kv, head_dim], got {tuple(t.shape)}")
    return t, from_np


# ---------------------------------------------------------------- paged cache
def kvcache_gather(cache, layer: int, block_tables, context_lens, max_context_len: int):
    """``[batch, max_context_len, n_head_kv, head_dim]`` rows of the pool for
    one layer (oracles/kvcache.py:57-100); rows at and past the context length
    are zero."""
    c, from_np = _pool(cache)
    bt = _ints_to_device(block_tables, "block_tables")
    cl = _ints_to_device(context_lens, "context_lens")
    if bt.dim() != 3 or cl.dim() != 2 or tuple(cl.shape) != tuple(bt.shape[:2]):
        raise ValueError("block_tables [n_layers, batch, max_blocks] and context_lens [n_layers, batch] expected")
    n_layers, batch, max_blocks = (int(s) for s in bt.shape)
    n_blocks, bs, hkv, d = (int(s) for s in c.shape)
    out = torch.empty((batch, int(max_context_len), hkv, d), dtype=c.dtype, device=c.device)
    L.call("fmoe_kvcache_gather", _ptr(c), _TORCH_TO_DT[c.dtype], n_blocks, bs, hkv, d, int(layer), _ptr(bt),
           _ptr(cl), n_layers, batch, max_blocks, int(max_context_len), _ptr(out), _stream())
    return _finish(out, from_np)


def kvcache_scatter_decode(cache, layer: int, new_vals, block_indices, pos_in_blocks):
    """Writes ``new_vals [batch, n_head_kv, head_dim]`` to
    ``cache[block_indices[b], pos_in_blocks[b]]`` (oracles/kvcache.py:103-139).
    ``layer`` is accepted for the reference's signature and unused, as there.
    A device pool is updated in place and returned; a NumPy pool comes back
    as an updated copy."""
    del layer
    c, from_np = _pool(cache)
    v, _ = _to_device(new_vals, "new_vals")
    v = v.to(c.dtype).contiguous()
    bi = _ints_to_device(block_indices, "block_indices")
    pi = _ints_to_device(pos_in_blocks, "pos_in_blocks")
    n_blocks, bs, hkv, d = (int(s) for s in c.shape)
    batch = int(bi.numel())
    if tuple(v.shape) != (batch, hkv, d) or int(pi.numel()) != batch:
        raise ValueError("new_vals [batch, n_head_kv, head_dim], block_indices and pos_in_blocks [batch] expected")
    L.call("fmoe_kvcache_scatter_decode", _ptr(c), _TORCH_TO_DT[c.dtype], n_blocks, bs, hkv, d, _ptr(v), _ptr(bi),
           _ptr(pi), batch, _stream())
    return _finish(c, from_np)


def kvcache_scatter_prefill(cache, layer: int, new_vals, block_tables, start_positions, block_size: int):
    """Writes ``new_vals [batch, seq_len, n_head_kv, head_dim]`` at positions
    ``start_positions[b] + s`` through the layer's block table
    (oracles/kvcache.py:142-185).  In place for a device pool."""
    c, from_np = _pool(cache)
    n_blocks, bs, hkv, d = (int(s) for s in c.shape)
    if int(block_size) != bs:
        raise ValueError(f"block_size {block_size} != the pool's {bs}")
    v, _ = _to_device(new_vals, "new_vals")
    v = v.to(c.dtype).contiguous()
    bt = _ints_to_device(block_tables, "block_tables")
    sp = _ints_to_device(start_positions, "start_positions")
    if bt.dim() != 3 or v.dim() != 4 or tuple(v.shape[2:]) != (hkv, d) or int(v.shape[0]) != int(bt.shape[1]):
        raise ValueError("new_vals [batch, seq_len, n_head_kv, head_dim] and block_tables [n_layers, batch, max_blocks]")
    n_layers, batch, max_blocks = (int(s) for s in bt.shape)
    L.call("fmoe_kvcache_scatter_prefill", _ptr(c), _TORCH_TO_DT[c.dtype], n_blocks, bs, hkv, d, int(layer), _ptr(v),
           int(v.shape[1]), _ptr(bt), n_layers, batch, max_blocks, _ptr(sp), _stream())
    return _finish(c, from_np)


# ---------------------------------------------------------------- weights
@dataclass
class PackedLinearWeights:
    """A dense projection packed once for the kernels: ``[n_out, n_in]``
    (one-expert packed layout), fp8 packs with float32 ``scales [n_out]``."""

    data: torch.Tensor
    scales: Optional[torch.Tensor]
    dtype: int
    n_out: int
    n_in: int


def pack_linear_weights(parts, dtype=None) -> PackedLinearWeights:
    """Packs ``x @ W`` weights ``W [n_in, n_out_i]`` side by side into one
    ``[sum n_out_i, n_in]`` weight (e.g. wq | wk | wv)."""
    dev = _device()
    srcs = [_to_device(w, "weight")[0] for w in parts]
    n_in = int(srcs[0].shape[0])
    if any(s.dim() != 2 or int(s.shape[0]) != n_in for s in srcs):
        raise ValueError("weights must be [n_in, n_out] with one n_in")
    dst_dt = _TORCH_TO_DT[srcs[0].dtype] if dtype is None else _dtype_code(dtype)
    n_total = sum(int(s.shape[1]) for s in srcs)
    nbytes = L.lib().fmoe_packed_weight_bytes(n_total, n_in, 1, dst_dt)
    data = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
    scales = torch.empty(n_total, dtype=torch.float32, device=dev) if dst_dt == L.F8E4M3FN else None
    row = 0
    for s in srcs:
        L.call("fmoe_pack_linear_weight", _ptr(s), _TORCH_TO_DT[s.dtype], n_in, int(s.shape[1]), row, n_total, dst_dt,
               _ptr(data), _ptr(scales), _stream())
        row += int(s.shape[1])
    return PackedLinearWeights(data, scales, dst_dt, n_total, n_in)


def _bias(b, n, name):
    if b is None:
        return None
    t, _ = _to_device(b, name)
    t = t.float().contiguous()
    if tuple(t.shape) != (n,):
        raise ValueError(f"{name} must be [{n}], got {tuple(t.shape)}")
    return t


class AttentionBlockDecode:
    """``attention_block_decode`` with packed weights and a reusable workspace.

    ``blk(x, positions, k_cached, v_cached)`` -> ``(out, k_new, v_new)`` as
    attention_block_decode.mlir:52-70 defines them; ``blk.paged(...)`` runs
    the decode layer's gather + attention + scatter_decode on a paged pool
    (transformer_layer_moe_decode.mlir:180-209), reading the pool in place.
    """

    def __init__(self, wq, wk, wv, wo, bq=None, bk=None, bv=None, bo=None, use_bias=False, *, n_head, n_head_kv,
                 n_embd, rope_freq_base=10000.0, rope_freq_scale=1.0, act_dtype=torch.bfloat16, weight_dtype=None):
        self.act = _TORCH_TO_DT[act_dtype]
        wdt = self.act if weight_dtype is None else _dtype_code(weight_dtype)
        if self.act == L.F32 and wdt != L.F32:
            raise TypeError("f32 activations need f32 weights")
        self.n_head, self.n_head_kv, self.n_embd = int(n_head), int(n_head_kv), int(n_embd)
        shapes = [tuple(int(s) for s in (w.shape)) for w in (wq, wk, wv, wo)]
        self.n_embd_kv = shapes[1][1]
        if (shapes[0] != (self.n_embd, self.n_embd) or shapes[1] != (self.n_embd, self.n_embd_kv)
                or shapes[2] != shapes[1] or shapes[3] != (self.n_embd, self.n_embd)):
            raise ValueError(f"wq/wk/wv/wo shapes {shapes} do not match n_embd {self.n_embd}")
        self.wqkv = pack_linear_weights([wq, wk, wv], wdt)
        self.wo = pack_linear_weights([wo], wdt)
        self.wdt = wdt
        self.use_bias = bool(use_bias)
        self.bq = _bias(bq, self.n_embd, "bq") if use_bias else None
        self.bk = _bias(bk, self.n_embd_kv, "bk") if use_bias else None
        self.bv = _bias(bv, self.n_embd_kv, "bv") if use_bias else None
        self.bo = _bias(bo, self.n_embd, "bo") if use_bias else None
        self.freq_base, self.freq_scale = float(rope_freq_base), float(rope_freq_scale)
        self.head_dim = self.n_embd // self.n_head
        self._ws = None

    def _get_ws(self, batch, ctx, sublayer=False):
        fn = ("fmoe_attention_sublayer_decode_paged_workspace_bytes" if sublayer
              else "fmoe_attention_block_decode_workspace_bytes")
        nbytes = getattr(L.lib(), fn)(batch, ctx, self.n_head, self.n_head_kv, self.n_embd, self.n_embd_kv, self.act)
        dev = torch.device("cuda", torch.cuda.current_device())
        if self._ws is None or self._ws.numel() < nbytes or self._ws.device != dev:
            self._ws = _workspace(nbytes)
        return self._ws

    def _weights(self):
        return (_ptr(self.wqkv.data), _ptr(self.wqkv.scales), _ptr(self.wo.data), _ptr(self.wo.scales), self.wdt,
                _ptr(self.bq), _ptr(self.bk), _ptr(self.bv), _ptr(self.bo), int(self.use_bias))

    def _x(self, x, positions):
        dt = _DT_TO_TORCH[self.act]
        if not isinstance(x, torch.Tensor) or x.dtype != dt or x.device.type != "cuda":
            raise TypeError(f"x must be a {dt} device tensor")
        if x.dim() != 2 or int(x.shape[1]) != self.n_embd:
            raise ValueError(f"x must be [batch, {self.n_embd}]")
        pos = _ints_to_device(positions, "positions", torch.int64)
        if int(pos.numel()) != int(x.shape[0]):
            raise ValueError("positions must be [batch]")
        return x.contiguous(), pos

    def __call__(self, x, positions, k_cached, v_cached):
        x, pos = self._x(x, positions)
        B = int(x.shape[0])
        dt = x.dtype
        kc = k_cached.to(dt).contiguous()
        vc = v_cached.to(dt).contiguous()
        if kc.dim() != 4 or tuple(kc.shape) != tuple(vc.shape) or int(kc.shape[0]) != B \
                or tuple(kc.shape[2:]) != (self.n_head_kv, self.head_dim):
            raise ValueError(f"k_cached / v_cached must be [{B}, ctx_len, {self.n_head_kv}, {self.head_dim}]")
        ctx = int(kc.shape[1])
        out = torch.empty((B, self.n_embd), dtype=dt, device=x.device)
        k_new = torch.empty((B, self.n_head_kv, self.head_dim), dtype=dt, device=x.device)
        v_new = torch.empty_like(k_new)
        ws = self._get_ws(B, ctx)
        L.call("fmoe_attention_block_decode", _ptr(x), _ptr(pos), _ptr(kc), _ptr(vc), ctx, *self._weights(), B,
               self.n_head, self.n_head_kv, self.n_embd, self.n_embd_kv, self.freq_base, self.freq_scale, self.act,
               _ptr(out), _ptr(k_new), _ptr(v_new), _ptr(ws), ws.numel(), _stream())
        return out, k_new, v_new

    def _paged_args(self, B, dt, k_cache, v_cache, block_tables, context_lens, block_indices, pos_in_blocks):
        """Checks the pools and paging metadata of a paged call; returns the
        device int32 tensors (tables, lens, block indices, positions in block)."""
        for name, p in (("k_cache", k_cache), ("v_cache", v_cache)):
            if not isinstance(p, torch.Tensor) or p.dtype != dt or p.device.type != "cuda" or not p.is_contiguous():
                raise TypeError(f"{name} must be a contiguous {dt} device tensor")
            if p.dim() != 4 or tuple(p.shape[2:]) != (self.n_head_kv, self.head_dim):
                raise ValueError(f"{name} must be [n_blocks, block_size, {self.n_head_kv}, {self.head_dim}]")
        bt = _ints_to_device(block_tables, "block_tables")
        cl = _ints_to_device(context_lens, "context_lens")
        bi = _ints_to_device(block_indices, "block_indices")
        pi = _ints_to_device(pos_in_blocks, "pos_in_blocks")
        if bt.dim() != 3 or int(bt.shape[1]) != B or tuple(cl.shape) != tuple(bt.shape[:2]):
            raise ValueError("block_tables [n_layers, batch, max_blocks] and context_lens [n_layers, batch] expected")
        if int(bi.numel()) != B or int(pi.numel()) != B:
            raise ValueError("block_indices and pos_in_blocks must be [batch]")
        return bt, cl, bi, pi

    def _paging(self, k_cache, v_cache, layer, bt, cl, max_context_len, bi, pi):
        """The C ABI's pool and paging arguments, from k_cache to pos_in_blocks."""
        return (_ptr(k_cache), _ptr(v_cache), int(k_cache.shape[0]), int(k_cache.shape[1]), int(layer), _ptr(bt),
                _ptr(cl), int(bt.shape[0]), int(bt.shape[2]), int(max_context_len), _ptr(bi), _ptr(pi))

    def _tail(self, B, out, k_new, v_new, ws):
        return (B, self.n_head, self.n_head_kv, self.n_embd, self.n_embd_kv, self.freq_base, self.freq_scale,
                self.act, _ptr(out), _ptr(k_new), _ptr(v_new), _ptr(ws), ws.numel(), _stream())

    def paged(self, x, positions, k_cache, v_cache, layer, block_tables, context_lens, max_context_len,
              block_indices, pos_in_blocks):
        """Attention of one new token per sequence over the paged pools
        ``[n_blocks, block_size, n_head_kv, head_dim]`` (updated in place with
        the new K/V) -> ``(out, k_new, v_new)``."""
        x, pos = self._x(x, positions)
        B, dt = int(x.shape[0]), x.dtype
        bt, cl, bi, pi = self._paged_args(B, dt, k_cache, v_cache, block_tables, context_lens, block_indices,
                                          pos_in_blocks)
        out = torch.empty((B, self.n_embd), dtype=dt, device=x.device)
        k_new = torch.empty((B, self.n_head_kv, self.head_dim), dtype=dt, device=x.device)
        v_new = torch.empty_like(k_new)
        ws = self._get_ws(B, int(max_context_len))
        L.call("fmoe_attention_decode_paged", _ptr(x), _ptr(pos),
               *self._paging(k_cache, v_cache, layer, bt, cl, max_context_len, bi, pi), *self._weights(),
               *self._tail(B, out, k_new, v_new, ws))
        return out, k_new, v_new

    def paged_sublayer(self, residual, attn_norm_w, rms_eps, positions, k_cache, v_cache, layer, block_tables,
                       context_lens, max_context_len, block_indices, pos_in_blocks, out=None):
        """The decode layer's attention sub-layer (transformer_layer_moe_decode.mlir:174-221):
        ``residual + paged(rms_norm(residual, attn_norm_w, rms_eps), ...)``.
        ``out=residual`` updates the residual stream in place.  Returns
        ``(out, k_new, v_new)``."""
        x, pos = self._x(residual, positions)
        B, dt = int(x.shape[0]), x.dtype
        nw, _ = _to_device(attn_norm_w, "attn_norm_w")
        nw = nw.to(dt).contiguous()
        if tuple(nw.shape) != (self.n_embd,):
            raise ValueError(f"attn_norm_w must be [{self.n_embd}]")
        bt, cl, bi, pi = self._paged_args(B, dt, k_cache, v_cache, block_tables, context_lens, block_indices,
                                          pos_in_blocks)
        if out is None:
            out = torch.empty((B, self.n_embd), dtype=dt, device=x.device)
        elif out.dtype != dt or tuple(out.shape) != (B, self.n_embd) or not out.is_contiguous():
            raise ValueError(f"out must be a contiguous {dt} [{B}, {self.n_embd}] tensor")
        k_new = torch.empty((B, self.n_head_kv, self.head_dim), dtype=dt, device=x.device)
        v_new = torch.empty_like(k_new)
        ws = self._get_ws(B, int(max_context_len), sublayer=True)
        L.call("fmoe_attention_sublayer_decode_paged", _ptr(x), _ptr(nw), float(rms_eps), _ptr(pos),
               *self._paging(k_cache, v_cache, layer, bt, cl, max_context_len, bi, pi), *self._weights(),
               *self._tail(B, out, k_new, v_new, ws))
        return out, k_new, v_new


def attention_block_decode(input, positions, k_cached, v_cached, wq, wk, wv, wo, bq, bk, bv, bo, use_bias: bool,
                           n_head: int, n_head_kv: int, n_embd: int, rope_freq_base: float = 10000.0,
                           rope_freq_scale: float = 1.0):
    """Positional signature of attention_block_decode.mlir:52-70:
    ``(output [batch, n_embd], k_new [batch, n_head_kv, head_dim], v_new)``.
    NumPy float32 in, NumPy out (fp32 arithmetic); device tensors stay on the
    device in their dtype."""
    x, x_np = _to_device(input, "input")
    kc, _ = _to_device(k_cached, "k_cached")
    vc, _ = _to_device(v_cached, "v_cached")
    blk = AttentionBlockDecode(wq, wk, wv, wo, bq, bk, bv, bo, use_bias, n_head=n_head, n_head_kv=n_head_kv,
                               n_embd=n_embd, rope_freq_base=rope_freq_base, rope_freq_scale=rope_freq_scale,
                               act_dtype=x.dtype)
    out, k_new, v_new = blk(x, positions, kc, vc)
    return _finish(out, x_np), _finish(k_new, x_np), _finish(v_new, x_np)
