"""MoE layer parameters: GGUF-style names, load-time packing, packed artifacts.

The reference addresses a model's weights by GGUF names in the parameter
scope ``"model"`` (tests/utils.py:340-370 builds the index from a
``dict[str, np.ndarray]``; models/llm/mixtral/params.mlir:361-383 and
tests/models/test_toy_llm.py:111-123 name the MoE tensors), with the
expert dimension innermost:

* ``blk.{i}.ffn_norm.weight``       ``[n_embd]``
* ``blk.{i}.ffn_gate_inp.weight``   ``[n_expert, n_embd]``
* ``blk.{i}.ffn_up_exps.weight``    ``[n_ff, n_embd, n_expert]``
* ``blk.{i}.ffn_gate_exps.weight``  ``[n_ff, n_embd, n_expert]``
* ``blk.{i}.ffn_down_exps.weight``  ``[n_embd, n_ff, n_expert]``

(the reference's accessors take the layer index but always read ``blk.0``,
params.mlir:299-304; here every layer is addressed.)

This module turns such a parameter set -- a mapping of names to NumPy
arrays / torch tensors, or a safetensors file -- into per-layer
``MoEFFNLayer`` objects whose expert weights are already packed for the
kernels, so no packing or quantisation happens on the request path:

* ``load_moe_layers``: pack at load time (bf16, fp32, or fp8-e4m3 quantised
  per output channel on the GPU).  Pre-quantised expert weights are accepted
  as fp8 codes (``torch.float8_e4m3fn`` or uint8) next to a
  ``blk.{i}.ffn_*_exps.scale`` tensor ``[n_out, n_expert]`` float32.
* ``save_packed`` / ``load_packed``: an offline artifact (safetensors) that
  holds the packed buffers themselves, so loading it is a copy.
* ``quantize_fp8``: offline fp8 quantisation = load with ``weight_dtype="fp8"``
  and save the packed result.
* ``load_attention_layers``: the decode attention half's tensors under the
  same scheme (``blk.{i}.attn_norm.weight``, ``blk.{i}.attn_{q,k,v,output}.weight``
  in the ``x @ W`` layout ``[n_in, n_out]``, optional ``.bias``;
  tests/models/test_toy_llm.py:80-109), packed into ``AttentionBlockDecode``.
"""

from __future__ import annotations

import json
from dataclasses import asdict, dataclass
from pathlib import Path
from typing import Iterable, Mapping, Optional, Union

import numpy as np
import torch

from . import _lib as L
from .api import (
    MoEFFNBlock,
    PackedExpertWeights,
    QuantizedExpertWeights,
    _device,
    _dtype_code,
    pack_expert_weights,
)

PACKED_FORMAT = "fmoe-packed-v1"  # WF_MFMA16 / row-major packing of libfmoe ABI 1

_EXPERT_TENSORS = ("ffn_up_exps", "ffn_gate_exps", "ffn_down_exps")


@dataclass(frozen=True)
class MoEHParams:
    """The hyper-parameters the MoE FFN sub-layer reads, under the names of the
    reference's hparams accessors (models/llm/mixtral/hparams.mlir:26-80)."""

    block_count: int
    embedding_length: int  # n_embd
    feed_forward_length: int  # n_ff
    expert_count: int  # n_expert
    expert_used_count: int  # n_expert_used
    layer_norm_rms_epsilon: float
    normalize_expert_weights: bool


HPARAMS = {
    # models/llm/mixtral/hparams.mlir:26-80
    "mixtral": MoEHParams(32, 4096, 14336, 8, 2, 1e-5, False),
    # models/llm/toy/hparams.mlir:27-81
    "toy": MoEHParams(2, 64, 128, 4, 2, 1e-5, False),
}


def param_name(layer: int, tensor: str) -> str:
    """``blk.{layer}.{tensor}.weight`` (tensor: ffn_norm, ffn_gate_inp,
    ffn_up_exps, ffn_gate_exps, ffn_down_exps)."""
    return f"blk.{int(layer)}.{tensor}.weight"


def scale_name(layer: int, tensor: str) -> str:
    """Per-output-channel fp8 scales of an expert tensor: ``blk.{layer}.{tensor}.scale``."""
    return f"blk.{int(layer)}.{tensor}.scale"


def expected_shapes(hp: MoEHParams) -> dict:
    """Shape of each MoE tensor of one layer (reference layouts)."""
    H, F, E = hp.embedding_length, hp.feed_forward_length, hp.expert_count
    return {
        "ffn_norm": (H,),
        "ffn_gate_inp": (E, H),
        "ffn_up_exps": (F, H, E),
        "ffn_gate_exps": (F, H, E),
        "ffn_down_exps": (H, F, E),
    }


class ParamSource:
    """Read-only name -> tensor access over a mapping or a safetensors file.
    Tensors come back as torch tensors on the CPU (a safetensors file is
    memory-mapped and read one tensor at a time)."""

    def __init__(self, source: Union[Mapping, str, Path]):
        self._map = None
        self._path = None
        if isinstance(source, Mapping):
            self._map = source
        elif isinstance(source, (str, Path)):
            self._path = str(source)
            from safetensors import safe_open

            with safe_open(self._path, framework="pt", device="cpu") as f:
                self._keys = set(f.keys())
                self._meta = dict(f.metadata() or {})
        else:
            raise TypeError(f"parameters: expected a mapping or a safetensors path, got {type(source).__name__}")

    def __contains__(self, name: str) -> bool:
        return name in (self._map if self._map is not None else self._keys)

    def metadata(self) -> dict:
        return {} if self._map is not None else dict(self._meta)

    def shape(self, name: str) -> tuple:
        """Shape of a tensor without reading its data."""
        if name not in self:
            raise KeyError(f"parameter {name!r} not found")
        if self._map is not None:
            return tuple(int(s) for s in self._map[name].shape)
        from safetensors import safe_open

        with safe_open(self._path, framework="pt", device="cpu") as f:
            return tuple(int(s) for s in f.get_slice(name).get_shape())

    def get(self, name: str) -> torch.Tensor:
        if name not in self:
            raise KeyError(f"parameter {name!r} not found")
        if self._map is not None:
            v = self._map[name]
            if isinstance(v, np.ndarray):
                return torch.from_numpy(np.ascontiguousarray(v))
            if isinstance(v, torch.Tensor):
                return v
            raise TypeError(f"parameter {name!r}: expected an array, got {type(v).__name__}")
        from safetensors import safe_open

        with safe_open(self._path, framework="pt", device="cpu") as f:
            return f.get_tensor(name)


class MoEFFNLayer:
    """One transformer layer's MoE FFN with packed weights.

    ``layer(residual)`` is the sub-layer ``residual + moe_ffn_block(
    rms_norm(residual))`` (transformer_layer_moe_prefill.mlir:205-242);
    ``layer.block(x)`` is the block alone.  Both run on device tensors
    ``[n_tokens, n_embd]`` asynchronously on the current stream.
    """

    def __init__(self, index: int, hp: MoEHParams, norm_w: torch.Tensor, block: MoEFFNBlock):
        self.index = int(index)
        self.hp = hp
        self.norm_w = norm_w
        self.block = block

    def __call__(self, residual: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
        return self.block.sublayer(residual, self.norm_w, self.hp.layer_norm_rms_epsilon, out=out)

    @property
    def weight_dtype(self) -> int:
        return self.block.wdt


def _as_fp8_codes(q: torch.Tensor, name: str) -> torch.Tensor:
    if q.dtype == torch.float8_e4m3fn:
        return q
    if q.dtype == torch.uint8:
        return q
    raise TypeError(f"{name}: fp8 codes (float8_e4m3fn or uint8) expected with a .scale tensor, got {q.dtype}")


def _check_shape(name: str, t, shape) -> None:
    if tuple(int(s) for s in t.shape) != tuple(shape):
        raise ValueError(f"parameter {name!r} has shape {tuple(t.shape)}, expected {tuple(shape)}")


def load_moe_layers(params, hp: MoEHParams, act_dtype=torch.bfloat16, weight_dtype=None,
                    layers: Optional[Iterable[int]] = None) -> list:
    """Pack every requested layer's MoE tensors for the kernels.

    ``params``: mapping or safetensors path (``ParamSource``).
    ``weight_dtype``: "bf16", "f32" or "fp8" (quantise per output channel on
    the GPU); default: the activation dtype, or fp8 for tensors stored as fp8
    codes with scales.  ``layers``: indices (default all ``block_count``).
    Shapes are checked against ``hp`` and every problem names the parameter.
    """
    src = params if isinstance(params, ParamSource) else ParamSource(params)
    if act_dtype not in (torch.float32, torch.bfloat16):
        raise TypeError(f"act_dtype must be torch.float32 or torch.bfloat16, got {act_dtype}")
    act_dt = L.F32 if act_dtype == torch.float32 else L.BF16
    wdt = None if weight_dtype is None else _dtype_code(weight_dtype)
    shapes = expected_shapes(hp)
    idx = list(range(hp.block_count) if layers is None else layers)
    # Names and shapes of every requested layer first (metadata only), so a
    # bad parameter set fails before any device work.
    for i in idx:
        for t, shape in shapes.items():
            name = param_name(i, t)
            if tuple(src.shape(name)) != tuple(shape):
                raise ValueError(f"parameter {name!r} has shape {src.shape(name)}, expected {tuple(shape)}")
            if t in _EXPERT_TENSORS and scale_name(i, t) in src:
                sname = scale_name(i, t)
                if tuple(src.shape(sname)) != (shape[0], shape[2]):
                    raise ValueError(f"parameter {sname!r} has shape {src.shape(sname)}, "
                                     f"expected {(shape[0], shape[2])}")
    dev = _device()
    out = []
    for i in idx:
        tensors = {t: src.get(param_name(i, t)) for t in shapes}
        packed = {}
        for t in _EXPERT_TENSORS:
            name = param_name(i, t)
            sname = scale_name(i, t)
            if sname in src:
                q = _as_fp8_codes(tensors[t], name)
                sc = src.get(sname)
                if wdt not in (None, L.F8E4M3FN):
                    raise TypeError(f"{name} is stored as fp8; it cannot be loaded as dtype {weight_dtype!r}")
                packed[t] = pack_expert_weights(QuantizedExpertWeights(q.to(dev), sc.to(dev, torch.float32)))
            else:
                w = tensors[t]
                if not w.dtype.is_floating_point or w.dtype == torch.float8_e4m3fn:
                    raise TypeError(f"{name}: float weights expected (fp8 codes need {sname})")
                target = act_dt if wdt is None else wdt
                # the packer reads fp32 or bf16; other float types go through fp32
                keep = w.dtype in (torch.float32, torch.bfloat16) and target != L.F32
                w = w.to(dev, w.dtype if keep else torch.float32)
                packed[t] = pack_expert_weights(w, target)
        dts = {p.dtype for p in packed.values()}
        if len(dts) != 1:
            raise TypeError(f"layer {i}: up/gate/down expert tensors load to different dtypes")
        torch_act = torch.float32 if act_dt == L.F32 else torch.bfloat16
        norm_w = tensors["ffn_norm"].to(dev, torch_act).contiguous()
        wr = tensors["ffn_gate_inp"].to(dev, torch_act).contiguous()
        block = MoEFFNBlock(wr, packed["ffn_up_exps"], packed["ffn_gate_exps"], packed["ffn_down_exps"],
                            hp.expert_count, hp.expert_used_count, hp.embedding_length, hp.feed_forward_length,
                            hp.normalize_expert_weights, act_dtype=torch_act)
        out.append(MoEFFNLayer(i, hp, norm_w, block))
    return out


def save_packed(layers, path: Union[str, Path]) -> None:
    """Write packed layers to a safetensors artifact: per expert tensor the
    packed bytes (``blk.{i}.ffn_*_exps.packed``, uint8) and fp8 scales
    (``.packed_scale``, ``[n_expert, n_out]``), plus the norm and router
    weights in the activation dtype; metadata records the packing format,
    the ABI version and the hyper-parameters."""
    from safetensors.torch import save_file

    if not layers:
        raise ValueError("no layers to save")
    hp = layers[0].hp
    tensors = {}
    shapes = {}
    for lay in layers:
        i = lay.index
        tensors[param_name(i, "ffn_norm")] = lay.norm_w.detach().cpu().contiguous()
        tensors[param_name(i, "ffn_gate_inp")] = lay.block.wr.detach().cpu().contiguous()
        for t, p in zip(_EXPERT_TENSORS, (lay.block.up, lay.block.gate, lay.block.down)):
            base = f"blk.{i}.{t}"
            tensors[base + ".packed"] = p.data.detach().cpu().contiguous()
            if p.scales is not None:
                tensors[base + ".packed_scale"] = p.scales.detach().cpu().contiguous()
            shapes[base] = [p.n_out, p.n_in, p.n_expert, p.dtype]
    meta = {
        "format": PACKED_FORMAT,
        "abi": str(L.lib().fmoe_abi_version()),
        "hparams": json.dumps(asdict(hp)),
        "act_dtype": str(layers[0].block.act),
        "layers": json.dumps([lay.index for lay in layers]),
        "expert_tensors": json.dumps(shapes),
    }
    save_file(tensors, str(path), metadata=meta)


def load_packed(path: Union[str, Path], layers: Optional[Iterable[int]] = None) -> list:
    """Load an artifact written by ``save_packed``: the packed buffers are
    copied to the GPU as they are (no packing, no quantisation).  The packing
    format, ABI version and buffer sizes are checked."""
    src = ParamSource(path)
    meta = src.metadata()
    if meta.get("format") != PACKED_FORMAT:
        raise ValueError(f"{path}: not an fmoe packed artifact (format {meta.get('format')!r})")
    if meta.get("abi") != str(L.lib().fmoe_abi_version()):
        raise ValueError(f"{path}: packed for ABI {meta.get('abi')}, library is ABI {L.lib().fmoe_abi_version()}")
    hp = MoEHParams(**json.loads(meta["hparams"]))
    act_dt = int(meta["act_dtype"])
    torch_act = torch.float32 if act_dt == L.F32 else torch.bfloat16
    shapes = json.loads(meta["expert_tensors"])
    stored = json.loads(meta["layers"])
    want = stored if layers is None else list(layers)
    dev = _device()
    out = []
    for i in want:
        if i not in stored:
            raise KeyError(f"{path}: layer {i} not in the artifact (has {stored})")
        packed = {}
        for t in _EXPERT_TENSORS:
            base = f"blk.{i}.{t}"
            n_out, n_in, n_expert, dt = shapes[base]
            data = src.get(base + ".packed")
            need = L.lib().fmoe_packed_weight_bytes(n_out, n_in, n_expert, dt)
            if data.dtype != torch.uint8 or data.numel() != max(need, 1):
                raise ValueError(f"{path}: {base}.packed holds {data.numel()} bytes, expected {need}")
            scales = None
            if dt == L.F8E4M3FN:
                scales = src.get(base + ".packed_scale").to(dev, torch.float32).contiguous()
                _check_shape(base + ".packed_scale", scales, (n_expert, n_out))
            packed[t] = PackedExpertWeights(data.to(dev).contiguous(), scales, dt, n_out, n_in, n_expert)
        norm_w = src.get(param_name(i, "ffn_norm")).to(dev, torch_act).contiguous()
        wr = src.get(param_name(i, "ffn_gate_inp")).to(dev, torch_act).contiguous()
        block = MoEFFNBlock(wr, packed["ffn_up_exps"], packed["ffn_gate_exps"], packed["ffn_down_exps"],
                            hp.expert_count, hp.expert_used_count, hp.embedding_length, hp.feed_forward_length,
                            hp.normalize_expert_weights, act_dtype=torch_act)
        out.append(MoEFFNLayer(i, hp, norm_w, block))
    return out


def quantize_fp8(params, hp: MoEHParams, path: Optional[Union[str, Path]] = None, act_dtype=torch.bfloat16,
                 layers: Optional[Iterable[int]] = None) -> list:
    """Offline fp8-e4m3 quantisation (per output channel, scale = absmax/448)
    of every layer's expert tensors; writes the packed artifact to ``path``
    when given.  Returns the loaded layers."""
    out = load_moe_layers(params, hp, act_dtype=act_dtype, weight_dtype="fp8", layers=layers)
    if path is not None:
        save_packed(out, path)
    return out


# ---------------------------------------------------------------- attention
_ATTN_PROJ = ("attn_q", "attn_k", "attn_v", "attn_output")


@dataclass(frozen=True)
class AttentionHParams:
    """The hyper-parameters of the decode attention half, under the names of
    the reference's hparams accessors (models/llm/mixtral/hparams.mlir:26-80)."""

    block_count: int
    embedding_length: int  # n_embd
    attention_head_count: int  # n_head
    attention_head_count_kv: int  # n_head_kv
    rope_freq_base: float
    use_attention_bias: bool
    layer_norm_rms_epsilon: float
    rope_freq_scale: float = 1.0


ATTN_HPARAMS = {
    # models/llm/mixtral/hparams.mlir:26-80
    "mixtral": AttentionHParams(32, 4096, 32, 8, 10000.0, False, 1e-5),
    # models/llm/toy/hparams.mlir:27-81
    "toy": AttentionHParams(2, 64, 4, 2, 10000.0, False, 1e-5),
}


def attention_shapes(hp: AttentionHParams) -> dict:
    """``blk.{i}.attn_*`` shapes (tests/models/test_toy_llm.py:80-109): the
    projections in the ``x @ W`` layout ``[n_in, n_out]``."""
    H = hp.embedding_length
    kv = hp.attention_head_count_kv * (H // hp.attention_head_count)
    return {"attn_norm": (H,), "attn_q": (H, H), "attn_k": (H, kv), "attn_v": (H, kv), "attn_output": (H, H)}


class AttentionLayer:
    """One layer's attention half: ``attn_norm`` weight and an
    ``AttentionBlockDecode`` with packed projections."""

    def __init__(self, index: int, hp: AttentionHParams, norm_w: torch.Tensor, attn):
        self.index = index
        self.hp = hp
        self.norm_w = norm_w
        self.attn = attn


def load_attention_layers(params, hp: AttentionHParams, act_dtype=torch.bfloat16, weight_dtype=None,
                          layers: Optional[Iterable[int]] = None) -> list:
    """Pack every requested layer's attention projections
    (``blk.{i}.attn_{q,k,v,output}.weight``, biases ``.bias`` when
    ``hp.use_attention_bias``, ``blk.{i}.attn_norm.weight``) for the decode
    kernels.  ``weight_dtype``: "bf16", "f32" or "fp8"; default: the
    activation dtype.  Shapes are checked before any device work."""
    from .attention import AttentionBlockDecode

    src = params if isinstance(params, ParamSource) else ParamSource(params)
    if act_dtype not in (torch.float32, torch.bfloat16):
        raise TypeError(f"act_dtype must be torch.float32 or torch.bfloat16, got {act_dtype}")
    shapes = attention_shapes(hp)
    idx = list(range(hp.block_count) if layers is None else layers)
    for i in idx:
        for t, shape in shapes.items():
            name = param_name(i, t)
            if tuple(src.shape(name)) != tuple(shape):
                raise ValueError(f"parameter {name!r} has shape {src.shape(name)}, expected {tuple(shape)}")
        if hp.use_attention_bias:
            for t in _ATTN_PROJ:
                name = f"blk.{i}.{t}.bias"
                want = (shapes[t][1],)
                if tuple(src.shape(name)) != want:
                    raise ValueError(f"parameter {name!r} has shape {src.shape(name)}, expected {want}")
    dev = _device()
    out = []
    for i in idx:
        # the packer converts fp32 sources to the weight dtype
        w = [src.get(param_name(i, t)).to(dev, torch.float32) for t in _ATTN_PROJ]
        b = [None] * 4
        if hp.use_attention_bias:
            b = [src.get(f"blk.{i}.{t}.bias").to(dev, torch.float32) for t in _ATTN_PROJ]
        attn = AttentionBlockDecode(*w, *b, use_bias=hp.use_attention_bias, n_head=hp.attention_head_count,
                                    n_head_kv=hp.attention_head_count_kv, n_embd=hp.embedding_length,
                                    rope_freq_base=hp.rope_freq_base, rope_freq_scale=hp.rope_freq_scale,
                                    act_dtype=act_dtype, weight_dtype=weight_dtype)
        norm_w = src.get(param_name(i, "attn_norm")).to(dev, act_dtype).contiguous()
        out.append(AttentionLayer(i, hp, norm_w, attn))
    return out
