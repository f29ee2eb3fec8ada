"""Drop-in host API mirroring the reference's MoE FFN functions.

``moe_ffn_block``, ``mul_mat_id`` and ``swiglu`` take the same positional
arguments, tensor layouts and meaning as the reference
(oracles/moe.py:9-13, :51-62; oracles/activation.py:11-21;
components/moe/moe_ffn_block.mlir:34-45; components/moe/mul_mat_id.mlir:22-26),
and run on the gfx950 kernels of libfmoe.so through its C ABI.

Value semantics follow the reference harness (tests/utils.py:151-169): NumPy
inputs are copied to the device, the call runs synchronously, and a NumPy
float32 array comes back.  torch tensors already on the GPU stay there: the
call is asynchronous on torch's current stream and returns a device tensor.

Errors: ``TypeError`` for unsupported dtypes (the reference raises
``ValueError("Unsupported dtype")`` at its marshalling layer, tests/utils.py:155-156),
``ValueError`` for inconsistent shapes, ``IndexError`` for expert ids outside
``[0, n_expert)`` (the reference's NumPy oracle raises IndexError for ids >= E).
"""

from __future__ import annotations

import ctypes
import threading
import weakref
from dataclasses import dataclass
from typing import Optional

import numpy as np
import torch

from . import _lib as L

_TORCH_TO_DT = {torch.float32: L.F32, torch.bfloat16: L.BF16}
_DT_TO_TORCH = {L.F32: torch.float32, L.BF16: torch.bfloat16}
_DT_NAMES = {"f32": L.F32, "float32": L.F32, "bf16": L.BF16, "bfloat16": L.BF16,
             "fp8": L.F8E4M3FN, "f8e4m3fn": L.F8E4M3FN, "float8_e4m3fn": L.F8E4M3FN}


# ---------------------------------------------------------------- plumbing
def _device() -> torch.device:
    if not torch.cuda.is_available():
        raise L.NoDeviceError("no GPU visible to torch; libfmoe needs a gfx950 device")
    return torch.device("cuda", torch.cuda.current_device())


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _to_device(x, name: str, allowed=(torch.float32, torch.bfloat16)):
    """-> (contiguous device tensor, came_from_numpy)."""
    if isinstance(x, np.ndarray):
        if x.dtype == np.float32:
            t = torch.from_numpy(np.ascontiguousarray(x))
        else:
            raise TypeError(f"{name}: unsupported dtype {x.dtype} (float32 expected)")
        return t.to(_device(), non_blocking=False), True
    if isinstance(x, torch.Tensor):
        if x.dtype not in allowed:
            raise TypeError(f"{name}: unsupported dtype {x.dtype}")
        if x.device.type != "cuda":
            x = x.to(_device())
        return x.contiguous(), False
    raise TypeError(f"{name}: expected numpy.ndarray or torch.Tensor, got {type(x).__name__}")


def _ids_to_device(ids, n_expert: int, name="ids"):
    """Integer ids -> int32 device tensor; host arrays are range-checked here."""
    if isinstance(ids, np.ndarray):
        if not np.issubdtype(ids.dtype, np.integer):
            raise TypeError(f"{name}: integer dtype expected, got {ids.dtype}")
        if ids.size and (ids.min() < 0 or ids.max() >= n_expert):
            raise IndexError(f"{name}: expert id outside [0, {n_expert})")
        return torch.from_numpy(np.ascontiguousarray(ids, dtype=np.int32)).to(_device()), True
    if isinstance(ids, torch.Tensor):
        if ids.dtype.is_floating_point or ids.dtype == torch.bool:
            raise TypeError(f"{name}: integer dtype expected, got {ids.dtype}")
        checked = False
        if ids.device.type != "cuda":
            if ids.numel() and (int(ids.min()) < 0 or int(ids.max()) >= n_expert):
                raise IndexError(f"{name}: expert id outside [0, {n_expert})")
            checked = True
            ids = ids.to(_device())
        return ids.to(torch.int32).contiguous(), checked
    raise TypeError(f"{name}: expected numpy.ndarray or torch.Tensor")


def _shape(x):
    """Shape of a numpy array, torch tensor or (packed / quantised) weights."""
    if isinstance(x, (np.ndarray, torch.Tensor, PackedExpertWeights, QuantizedExpertWeights)):
        return tuple(int(s) for s in x.shape)
    raise TypeError(f"expected numpy.ndarray or torch.Tensor, got {type(x).__name__}")


def _check_float(x, name):
    if isinstance(x, np.ndarray) and x.dtype != np.float32:
        raise TypeError(f"{name}: unsupported dtype {x.dtype} (float32 expected)")
    if isinstance(x, torch.Tensor) and x.dtype not in _TORCH_TO_DT:
        raise TypeError(f"{name}: unsupported dtype {x.dtype}")


def _check_ids_host(ids, n_expert, name="ids"):
    if isinstance(ids, np.ndarray):
        if not np.issubdtype(ids.dtype, np.integer):
            raise TypeError(f"{name}: integer dtype expected, got {ids.dtype}")
        if ids.size and (ids.min() < 0 or ids.max() >= n_expert):
            raise IndexError(f"{name}: expert id outside [0, {n_expert})")
    elif isinstance(ids, torch.Tensor):
        if ids.dtype.is_floating_point or ids.dtype == torch.bool:
            raise TypeError(f"{name}: integer dtype expected, got {ids.dtype}")
    else:
        raise TypeError(f"{name}: expected numpy.ndarray or torch.Tensor")


def _workspace(nbytes: int) -> torch.Tensor:
    # torch's caching allocator returns 512-byte aligned blocks.
    return torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=_device())


def _finish(t: torch.Tensor, to_numpy: bool):
    if to_numpy:
        return t.float().cpu().numpy()
    return t


def _dtype_code(dtype) -> int:
    if dtype is None:
        return -1
    if isinstance(dtype, int):
        return dtype
    if isinstance(dtype, torch.dtype):
        if dtype in _TORCH_TO_DT:
            return _TORCH_TO_DT[dtype]
        if dtype == torch.float8_e4m3fn:
            return L.F8E4M3FN
    if isinstance(dtype, str) and dtype.lower() in _DT_NAMES:
        return _DT_NAMES[dtype.lower()]
    raise TypeError(f"unsupported weight dtype {dtype!r}")


# ---------------------------------------------------------------- weights
@dataclass
class QuantizedExpertWeights:
    """Expert weights already in OCP fp8-e4m3 with per-output-channel scales,
    in the reference layout: ``q [n_out, n_in, n_expert]`` (uint8 codes or
    torch.float8_e4m3fn) and ``scales [n_out, n_expert]`` float32.  The
    weights they stand for are ``decode(q) * scales[:, None, :]``."""

    q: object
    scales: object

    @property
    def shape(self):
        return tuple(self.q.shape)


@dataclass
class PackedExpertWeights:
    """Expert weights packed once for the kernels: per expert ``[n_out, n_in]``
    rows with n_in contiguous, in ``dtype`` (fmoe_dtype code); fp8 packs carry
    float32 scales ``[n_expert, n_out]``.  Accepted in every weight position
    of ``moe_ffn_block`` / ``mul_mat_id`` in place of the reference-layout
    array ``[n_out, n_in, n_expert]``."""

    data: torch.Tensor
    scales: Optional[torch.Tensor]
    dtype: int
    n_out: int
    n_in: int
    n_expert: int

    @property
    def shape(self):
        return (self.n_out, self.n_in, self.n_expert)


def pack_expert_weights(w, dtype=None) -> PackedExpertWeights:
    """Pack reference-layout expert weights ``[n_out, n_in, n_expert]``.

    ``dtype``: target "f32", "bf16" or "fp8" (or a torch dtype); default is
    the source dtype.  fp32/bf16 -> fp8 quantises each output channel with
    scale = absmax/448 on the GPU.  A ``QuantizedExpertWeights`` is packed
    as fp8 as-is.  Replaces the per-call weight transpose of
    mul_mat_id.mlir:37-48.
    """
    if isinstance(w, PackedExpertWeights):
        if dtype is not None and _dtype_code(dtype) != w.dtype:
            raise TypeError("weights are already packed in another dtype")
        return w
    dev = _device()
    src_scales = None
    if isinstance(w, QuantizedExpertWeights):
        q = w.q
        if isinstance(q, np.ndarray):
            if q.dtype != np.uint8:
                raise TypeError("QuantizedExpertWeights.q: uint8 codes expected")
            q = torch.from_numpy(np.ascontiguousarray(q))
        elif isinstance(q, torch.Tensor):
            if q.dtype == torch.float8_e4m3fn:
                q = q.view(torch.uint8)
            elif q.dtype != torch.uint8:
                raise TypeError("QuantizedExpertWeights.q: uint8 or float8_e4m3fn expected")
        src = q.to(dev).contiguous()
        sc = w.scales
        sc = torch.from_numpy(np.ascontiguousarray(sc, dtype=np.float32)) if isinstance(sc, np.ndarray) else sc
        src_scales = sc.to(dev, torch.float32).contiguous()
        src_dt = L.F8E4M3FN
        if src.dim() != 3 or tuple(src_scales.shape) != (src.shape[0], src.shape[2]):
            raise ValueError("QuantizedExpertWeights: q [n_out, n_in, E] and scales [n_out, E] expected")
    else:
        src, _ = _to_device(w, "expert weights")
        src_dt = _TORCH_TO_DT[src.dtype]
    if src.dim() != 3:
        raise ValueError(f"expert weights must be [n_out, n_in, n_expert], got {tuple(src.shape)}")
    dst_dt = src_dt if dtype is None else _dtype_code(dtype)
    n_out, n_in, n_expert = (int(s) for s in src.shape)
    nbytes = L.lib().fmoe_packed_weight_bytes(n_out, n_in, n_expert, dst_dt)
    data = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
    scales = None
    if dst_dt == L.F8E4M3FN:
        scales = torch.empty((n_expert, n_out), dtype=torch.float32, device=dev)
    L.call("fmoe_pack_expert_weights", _ptr(src), src_dt, _ptr(src_scales), n_out, n_in, n_expert,
           dst_dt, _ptr(data), _ptr(scales), _stream())
    return PackedExpertWeights(data, scales, dst_dt, n_out, n_in, n_expert)


def quantize_expert_weights(w) -> PackedExpertWeights:
    """fp8-e4m3 per-output-channel quantisation + packing (on the GPU)."""
    return pack_expert_weights(w, "fp8")


class _PackCache:
    """Packed copies of torch weight tensors, keyed on the tensor object, its
    storage pointer and its in-place version counter."""

    def __init__(self, capacity=16):
        self._lock = threading.Lock()
        self._items = []  # [(weakref, ptr, version, shape, torch dtype, dst dtype, packed)]
        self._capacity = capacity

    def get(self, w, dst_dt) -> PackedExpertWeights:
        if isinstance(w, (PackedExpertWeights, QuantizedExpertWeights)) or not isinstance(w, torch.Tensor):
            return pack_expert_weights(w, None if isinstance(w, (PackedExpertWeights, QuantizedExpertWeights)) else dst_dt)
        key = (w.data_ptr(), w._version, tuple(w.shape), w.dtype, dst_dt)
        with self._lock:
            for ref, *k, packed in self._items:
                if ref() is w and tuple(k) == key:
                    return packed
        packed = pack_expert_weights(w, dst_dt)
        with self._lock:
            self._items = [it for it in self._items if it[0]() is not None and it[0]() is not w]
            self._items.append((weakref.ref(w), *key, packed))
            if len(self._items) > self._capacity:
                self._items.pop(0)
        return packed


_pack_cache = _PackCache()


# ---------------------------------------------------------------- swiglu
def swiglu(gate, up):
    """``gate * silu(up)`` element-wise (components/activation/swiglu.mlir:16-51,
    oracles/activation.py:11-21)."""
    _check_float(gate, "gate")
    _check_float(up, "up")
    if _shape(gate) != _shape(up):
        raise ValueError(f"gate {_shape(gate)} and up {_shape(up)} differ")
    g, g_np = _to_device(gate, "gate")
    u, _ = _to_device(up, "up")
    if g.shape != u.shape:
        raise ValueError(f"gate {tuple(g.shape)} and up {tuple(u.shape)} differ")
    if g.dtype != u.dtype:
        raise TypeError("gate and up dtypes differ")
    out = torch.empty_like(g)
    L.call("fmoe_swiglu", _ptr(g), _ptr(u), _ptr(out), g.numel(), _TORCH_TO_DT[g.dtype], _stream())
    return _finish(out, g_np)


def rms_norm(x, weight, eps: float = 1e-6):
    """``(x / sqrt(mean(x^2, axis=-1) + eps)) * weight`` per row, positional
    signature of oracles/normalization.py:10-14 (components/normalization/
    rms_norm.mlir:18-85).  x ``[..., n_embd]``, weight ``[n_embd]``; fp32
    arithmetic, output in x's dtype."""
    _check_float(x, "x")
    _check_float(weight, "weight")
    xs, ws = _shape(x), _shape(weight)
    if len(xs) < 1 or ws != (xs[-1],):
        raise ValueError(f"weight shape {ws} != [{xs[-1] if xs else '?'}]")
    t, t_np = _to_device(x, "x")
    w, _ = _to_device(weight, "weight")
    w = w.to(t.dtype).contiguous()
    out = torch.empty_like(t)
    H = xs[-1]
    rows = t.numel() // H if H else 0
    L.call("fmoe_rms_norm", _ptr(t), _ptr(w), float(eps), _ptr(out), rows, H, _TORCH_TO_DT[t.dtype], _stream())
    return _finish(out, t_np)


# ---------------------------------------------------------------- router / permutation
def router(input, gate_inp_w, n_expert_used: int, normalize_weights: bool):
    """Steps 1-4 of the block (moe_ffn_block.mlir:50-128): returns
    ``(ids [k, T] int32, weights [k, T] float32)``."""
    x, x_np = _to_device(input, "input")
    wr, _ = _to_device(gate_inp_w, "gate_inp_w")
    wr = wr.to(x.dtype)
    T, H = x.shape
    E = wr.shape[0]
    if wr.shape[1] != H:
        raise ValueError("gate_inp_w and input hidden sizes differ")
    k = int(n_expert_used)
    ids = torch.empty((k, T), dtype=torch.int32, device=x.device)
    w = torch.empty((k, T), dtype=torch.float32, device=x.device)
    L.call("fmoe_router", _ptr(x), _ptr(wr), T, H, E, k, int(bool(normalize_weights)),
           _TORCH_TO_DT[x.dtype], _ptr(ids), _ptr(w), _stream())
    if x_np:
        return ids.cpu().numpy(), w.cpu().numpy()
    return ids, w


def permute(ids, n_expert: int):
    """Stable grouping of the slot-major flat assignments by expert:
    ``(order [k*T] int32, offsets [n_expert+1] int32)``."""
    was_np = isinstance(ids, np.ndarray)
    d, _ = _ids_to_device(ids, n_expert)
    if d.dim() != 2:
        raise ValueError("ids must be [n_expert_used, n_tokens]")
    k, T = d.shape
    order = torch.empty(max(k * T, 1), dtype=torch.int32, device=d.device)[: k * T]
    offsets = torch.empty(n_expert + 1, dtype=torch.int32, device=d.device)
    ws = _workspace(L.lib().fmoe_permute_workspace_bytes(k, T, n_expert))
    L.call("fmoe_permute", _ptr(d), k, T, n_expert, _ptr(order), _ptr(offsets), _ptr(ws),
           ws.numel(), _stream())
    bad = ctypes.c_int64(0)
    L.call("fmoe_workspace_error_count", _ptr(ws), _stream(), ctypes.byref(bad))
    if bad.value:
        raise IndexError(f"ids: {bad.value} expert id(s) outside [0, {n_expert})")
    if was_np:
        return order.cpu().numpy(), offsets.cpu().numpy()
    return order, offsets


# ---------------------------------------------------------------- mul_mat_id
def mul_mat_id(weights, input, ids):
    """``out[:, s, t] = weights[:, :, ids[s, t]] @ input[:, s, t]``.

    weights ``[n_out, n_in, n_expert]`` (or packed), input
    ``[n_in, n_expert_used, n_tokens]``, ids ``[n_expert_used, n_tokens]`` ->
    ``[n_out, n_expert_used, n_tokens]`` (oracles/moe.py:9-48,
    components/moe/mul_mat_id.mlir:22-120).
    """
    _check_float(input, "input")
    if not isinstance(weights, (PackedExpertWeights, QuantizedExpertWeights)):
        _check_float(weights, "weights")
    ws_shape, in_shape, ids_shape = _shape(weights), _shape(input), _shape(ids)
    if len(ws_shape) != 3:
        raise ValueError(f"weights must be [n_out, n_in, n_expert], got {ws_shape}")
    if len(ids_shape) != 2:
        raise ValueError(f"ids must be [n_expert_used, n_tokens], got {ids_shape}")
    if in_shape != (ws_shape[1], *ids_shape):
        raise ValueError(f"input shape {in_shape} != {(ws_shape[1], *ids_shape)}")
    _check_ids_host(ids, ws_shape[2])
    x, x_np = _to_device(input, "input")
    act = _TORCH_TO_DT[x.dtype]
    pw = _pack_cache.get(weights, act)
    if pw.dtype == L.F32 and act != L.F32:
        raise TypeError("f32 weights need f32 input")
    if act == L.F32 and pw.dtype != L.F32:
        raise TypeError("f32 input needs f32 weights")
    n_out, n_in, n_expert = pw.shape
    d_ids, checked = _ids_to_device(ids, n_expert)
    if d_ids.dim() != 2:
        raise ValueError("ids must be [n_expert_used, n_tokens]")
    k, T = (int(s) for s in d_ids.shape)
    if tuple(x.shape) != (n_in, k, T):
        raise ValueError(f"input shape {tuple(x.shape)} != {(n_in, k, T)}")
    out = torch.empty((n_out, k, T), dtype=x.dtype, device=x.device)
    ws = _workspace(L.lib().fmoe_mul_mat_id_workspace_bytes(n_out, n_in, n_expert, k, T, act))
    L.call("fmoe_mul_mat_id", _ptr(pw.data), _ptr(pw.scales), pw.dtype, _ptr(x), _ptr(d_ids),
           _ptr(out), n_out, n_in, n_expert, k, T, act, _ptr(ws), ws.numel(), _stream())
    if not checked and k * T > 0:
        bad = ctypes.c_int64(0)
        L.call("fmoe_workspace_error_count", _ptr(ws), _stream(), ctypes.byref(bad))
        if bad.value:
            raise IndexError(f"ids: {bad.value} expert id(s) outside [0, {n_expert})")
    return _finish(out, x_np)


# ---------------------------------------------------------------- moe_ffn_block
class MoEFFNBlock:
    """A ``moe_ffn_block`` with packed weights and a reusable workspace.

    ``block(x)`` computes the same function as ``moe_ffn_block(x, gate_inp_w,
    up, gate, down, n_expert, n_expert_used, n_embd, n_ff, normalize)`` on a
    device tensor x ``[n_tokens, n_embd]``, asynchronously on the current
    stream, allocating only the output (or writing into ``out=``).
    """

    def __init__(self, gate_inp_w, up_exps_w, gate_exps_w, down_exps_w, n_expert, n_expert_used,
                 n_embd, n_ff, normalize_weights, act_dtype=torch.bfloat16, weight_dtype=None,
                 fp8_activations=False):
        """``fp8_activations=True`` (e4m3 weights, bf16 activations) runs the
        prefill-sized GEMMs on the fp8 MFMA with activations quantised to e4m3
        per row (the C ABI's FMOE_F8E4M3FN_A8); decode-sized batches are
        unchanged.  It adds the activations' e4m3 rounding to the result.
        ``fp8_activations="x2"`` carries each activation as two e4m3 terms
        (hi = e4m3(v), lo = e4m3(v - hi), FMOE_F8E4M3FN_A8X2): the products
        still run on the fp8 MFMA, and the result keeps the bf16-activation
        tolerance."""
        self.act = _TORCH_TO_DT[act_dtype]
        wdt = self.act if weight_dtype is None else _dtype_code(weight_dtype)
        self.up = _pack_cache.get(up_exps_w, wdt)
        self.gate = _pack_cache.get(gate_exps_w, wdt)
        self.down = _pack_cache.get(down_exps_w, wdt)
        if not (self.up.dtype == self.gate.dtype == self.down.dtype):
            raise TypeError("up/gate/down weights must share one dtype")
        self.wdt = self.up.dtype
        if self.act == L.F32 and self.wdt != L.F32:
            raise TypeError("f32 activations need f32 weights")
        if fp8_activations not in (False, True, "x2"):
            raise ValueError(f"fp8_activations must be False, True or 'x2', not {fp8_activations!r}")
        if fp8_activations:
            if self.wdt != L.F8E4M3FN or self.act != L.BF16:
                raise TypeError("fp8 activations need e4m3 weights and bf16 activations")
            # the block's weight dtype code; the packed buffers are unchanged
            self.wdt = L.F8E4M3FN_A8X2 if fp8_activations == "x2" else L.F8E4M3FN_A8
        wr, _ = _to_device(gate_inp_w, "gate_inp_w")
        self.wr = wr.to(_DT_TO_TORCH[self.act]).contiguous()
        self.n_expert = int(n_expert)
        self.k = int(n_expert_used)
        self.n_embd = int(n_embd)
        self.n_ff = int(n_ff)
        self.normalize = bool(normalize_weights)
        _check_block_shapes(tuple(self.wr.shape), self.up.shape, self.gate.shape, self.down.shape,
                            self.n_expert, self.n_embd, self.n_ff)
        self._ws = None
        self._ws_key = None
        self._last = None  # n_tokens of the last call that completed its launches

    def workspace_bytes(self, n_tokens: int, sublayer: bool = False) -> int:
        fn = "fmoe_moe_ffn_sublayer_workspace_bytes" if sublayer else "fmoe_moe_ffn_block_workspace_bytes"
        return getattr(L.lib(), fn)(n_tokens, self.n_expert, self.k, self.n_embd, self.n_ff, self.act, self.wdt)

    def _get_ws(self, n_tokens, sublayer=False):
        nbytes = self.workspace_bytes(n_tokens, sublayer)
        key = (torch.cuda.current_device(), nbytes)
        if self._ws is None or self._ws_key[0] != key[0] or self._ws.numel() < nbytes:
            self._ws = _workspace(nbytes)
            self._ws_key = key
        return self._ws

    def __call__(self, x: torch.Tensor, out: Optional[torch.Tensor] = None, noalloc: bool = False) -> torch.Tensor:
        """``noalloc=True`` runs fmoe_moe_ffn_block_noalloc: no workspace,
        the library's fixed per-GPU scratch instead (at most
        NOALLOC_SCRATCH_BYTES of workspace; calls on one GPU must not
        overlap), and ``routing()`` is not available afterwards."""
        if x.dtype != _DT_TO_TORCH[self.act] or x.device.type != "cuda":
            raise TypeError(f"x must be a {_DT_TO_TORCH[self.act]} device tensor")
        if x.dim() != 2 or x.shape[1] != self.n_embd:
            raise ValueError(f"x must be [n_tokens, {self.n_embd}]")
        x = x.contiguous()
        T = int(x.shape[0])
        out = self._check_out(out, T, x.device)
        self._last = None
        if noalloc:
            L.call("fmoe_moe_ffn_block_noalloc", _ptr(x), _ptr(self.wr), _ptr(self.up.data), _ptr(self.gate.data),
                   _ptr(self.down.data), _ptr(self.up.scales), _ptr(self.gate.scales), _ptr(self.down.scales),
                   self.wdt, _ptr(out), T, self.n_expert, self.k, self.n_embd, self.n_ff,
                   int(self.normalize), self.act, _stream())
            return out
        ws = self._get_ws(T)
        L.call("fmoe_moe_ffn_block", _ptr(x), _ptr(self.wr), _ptr(self.up.data), _ptr(self.gate.data),
               _ptr(self.down.data), _ptr(self.up.scales), _ptr(self.gate.scales), _ptr(self.down.scales),
               self.wdt, _ptr(out), T, self.n_expert, self.k, self.n_embd, self.n_ff,
               int(self.normalize), self.act, _ptr(ws), ws.numel(), _stream())
        self._last = T
        return out

    def _check_out(self, out, T, device):
        """The output tensor: a new one, or the caller's ``out=`` after the
        checks the C ABI cannot make (it writes T * n_embd elements of the
        activation dtype through the raw pointer)."""
        dt = _DT_TO_TORCH[self.act]
        if out is None:
            return torch.empty((T, self.n_embd), dtype=dt, device=device)
        if (not isinstance(out, torch.Tensor) or out.device != device or out.dtype != dt
                or tuple(out.shape) != (T, self.n_embd) or not out.is_contiguous()):
            raise ValueError(f"out must be a contiguous {dt} [{T}, {self.n_embd}] tensor on {device}")
        return out

    def sublayer(self, residual: torch.Tensor, ffn_norm_w, rms_eps: float,
                 out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """The MoE FFN sub-layer of a transformer layer,
        ``residual + block(rms_norm(residual, ffn_norm_w, rms_eps))``
        (transformer_layer_moe_prefill.mlir:205-242), on a device tensor
        ``[n_tokens, n_embd]``.  ``out=residual`` updates in place."""
        dt = _DT_TO_TORCH[self.act]
        if residual.dtype != dt or residual.device.type != "cuda":
            raise TypeError(f"residual must be a {dt} device tensor")
        if residual.dim() != 2 or residual.shape[1] != self.n_embd:
            raise ValueError(f"residual must be [n_tokens, {self.n_embd}]")
        _check_float(ffn_norm_w, "ffn_norm_w")
        if _shape(ffn_norm_w) != (self.n_embd,):
            raise ValueError(f"ffn_norm_w shape {_shape(ffn_norm_w)} != [{self.n_embd}]")
        nw, _ = _to_device(ffn_norm_w, "ffn_norm_w")
        nw = nw.to(dt).contiguous()
        residual = residual.contiguous()
        T = int(residual.shape[0])
        out = self._check_out(out, T, residual.device)
        ws = self._get_ws(T, sublayer=True)
        self._last = None
        L.call("fmoe_moe_ffn_sublayer", _ptr(residual), _ptr(nw), float(rms_eps), _ptr(self.wr),
               _ptr(self.up.data), _ptr(self.gate.data), _ptr(self.down.data), _ptr(self.up.scales),
               _ptr(self.gate.scales), _ptr(self.down.scales), self.wdt, _ptr(out), T, self.n_expert, self.k,
               self.n_embd, self.n_ff, int(self.normalize), self.act, _ptr(ws), ws.numel(), _stream())
        self._last = T
        return out

    def routing(self, n_tokens: Optional[int] = None):
        """Device views of the routing computed by the last call (block or
        sub-layer): ``(ids [k, T], weights [k, T], order [k*T], offsets
        [E+1])``.  ``n_tokens``, when given, must be that call's T."""
        ws = self._ws
        if ws is None or self._last is None:
            raise RuntimeError("no call has completed on this block yet")
        if n_tokens is None:
            n_tokens = self._last
        elif int(n_tokens) != self._last:
            raise ValueError(f"n_tokens={n_tokens}, but the last call ran {self._last} tokens")
        ptrs = [ctypes.c_void_p() for _ in range(4)]
        L.call("fmoe_moe_ffn_block_routing", _ptr(ws), n_tokens, self.n_expert, self.k, self.n_embd,
               self.n_ff, self.act, self.wdt, *[ctypes.byref(p) for p in ptrs])
        base = ws.data_ptr()
        n = self.k * n_tokens

        def view(p, count, dtype):
            off = p.value - base
            itemsize = torch.empty((), dtype=dtype).element_size()
            return ws[off: off + count * itemsize].view(dtype)

        ids = view(ptrs[0], n, torch.int32).view(self.k, n_tokens)
        w = view(ptrs[1], n, torch.float32).view(self.k, n_tokens)
        order = view(ptrs[2], n, torch.int32)
        offsets = view(ptrs[3], self.n_expert + 1, torch.int32)
        return ids, w, order, offsets


def _check_block_shapes(wr, up, gate, down, n_expert, n_embd, n_ff):
    """Shapes of moe_ffn_block.mlir:35-39 against the size arguments (the
    reference does not check them)."""
    if tuple(wr) != (n_expert, n_embd):
        raise ValueError(f"gate_inp_w shape {tuple(wr)} != {(n_expert, n_embd)}")
    if tuple(up) != (n_ff, n_embd, n_expert):
        raise ValueError(f"up_exps_w shape {tuple(up)} != {(n_ff, n_embd, n_expert)}")
    if tuple(gate) != (n_ff, n_embd, n_expert):
        raise ValueError(f"gate_exps_w shape {tuple(gate)} != {(n_ff, n_embd, n_expert)}")
    if tuple(down) != (n_embd, n_ff, n_expert):
        raise ValueError(f"down_exps_w shape {tuple(down)} != {(n_embd, n_ff, n_expert)}")


def moe_ffn_block(input, gate_inp_w, up_exps_w, gate_exps_w, down_exps_w, n_expert: int,
                  n_expert_used: int, n_embd: int, n_ff: int, normalize_weights: bool):
    """Full MoE FFN block, positional signature of oracles/moe.py:51-62.

    input ``[n_tokens, n_embd]``; gate_inp_w ``[n_expert, n_embd]``;
    up/gate ``[n_ff, n_embd, n_expert]``; down ``[n_embd, n_ff, n_expert]``
    (or packed / quantised weights) -> ``[n_tokens, n_embd]``.
    """
    _check_float(input, "input")
    _check_float(gate_inp_w, "gate_inp_w")
    for name, w in (("up_exps_w", up_exps_w), ("gate_exps_w", gate_exps_w), ("down_exps_w", down_exps_w)):
        if not isinstance(w, (PackedExpertWeights, QuantizedExpertWeights)):
            _check_float(w, name)
    xs = _shape(input)
    if len(xs) != 2 or xs[1] != int(n_embd):
        raise ValueError(f"input shape {xs} != [n_tokens, {n_embd}]")
    _check_block_shapes(_shape(gate_inp_w), _shape(up_exps_w), _shape(gate_exps_w), _shape(down_exps_w),
                        int(n_expert), int(n_embd), int(n_ff))
    k = int(n_expert_used)
    if not 1 <= k <= int(n_expert):
        raise ValueError(f"n_expert_used={k} outside [1, {n_expert}]")
    x, x_np = _to_device(input, "input")
    blk = MoEFFNBlock(gate_inp_w, up_exps_w, gate_exps_w, down_exps_w, n_expert, n_expert_used,
                      n_embd, n_ff, normalize_weights, act_dtype=x.dtype)
    out = blk(x)
    return _finish(out, x_np)


def moe_ffn_sublayer(residual, ffn_norm_w, rms_eps: float, gate_inp_w, up_exps_w, gate_exps_w, down_exps_w,
                     n_expert: int, n_expert_used: int, n_embd: int, n_ff: int, normalize_weights: bool):
    """``residual + moe_ffn_block(rms_norm(residual, ffn_norm_w, rms_eps), ...)``:
    the MoE FFN sub-layer of architectures/llm/transformer_layer_moe_prefill.mlir:205-242
    (decode: transformer_layer_moe_decode.mlir:227-255) on the flattened
    residual stream ``[n_tokens, n_embd]``.  NumPy in, NumPy out; device
    tensors stay on the device."""
    _check_float(residual, "residual")
    _check_float(ffn_norm_w, "ffn_norm_w")
    _check_float(gate_inp_w, "gate_inp_w")
    for name, w in (("up_exps_w", up_exps_w), ("gate_exps_w", gate_exps_w), ("down_exps_w", down_exps_w)):
        if not isinstance(w, (PackedExpertWeights, QuantizedExpertWeights)):
            _check_float(w, name)
    rs = _shape(residual)
    if len(rs) != 2 or rs[1] != int(n_embd):
        raise ValueError(f"residual shape {rs} != [n_tokens, {n_embd}]")
    if _shape(ffn_norm_w) != (int(n_embd),):
        raise ValueError(f"ffn_norm_w shape {_shape(ffn_norm_w)} != [{n_embd}]")
    _check_block_shapes(_shape(gate_inp_w), _shape(up_exps_w), _shape(gate_exps_w), _shape(down_exps_w),
                        int(n_expert), int(n_embd), int(n_ff))
    k = int(n_expert_used)
    if not 1 <= k <= int(n_expert):
        raise ValueError(f"n_expert_used={k} outside [1, {n_expert}]")
    r, r_np = _to_device(residual, "residual")
    blk = MoEFFNBlock(gate_inp_w, up_exps_w, gate_exps_w, down_exps_w, n_expert, n_expert_used,
                      n_embd, n_ff, normalize_weights, act_dtype=r.dtype)
    out = blk.sublayer(r, ffn_norm_w, rms_eps)
    return _finish(out, r_np)
