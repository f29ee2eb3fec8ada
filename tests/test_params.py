"""Parameter names, shapes and sources of the MoE layer loader, without a
GPU: GGUF names of the reference (tests/models/test_toy_llm.py:111-123,
models/llm/mixtral/params.mlir:361-383), hyper-parameters of its hparams
modules, and errors that name the offending parameter before any device
work."""

import numpy as np
import pytest
import torch


def _params(fm, hp, layers=None, drop=None, bad=None):
    P = fm.params
    out = {}
    for i in range(hp.block_count if layers is None else layers):
        for t, shape in P.expected_shapes(hp).items():
            out[P.param_name(i, t)] = np.zeros(shape, np.float32)
    if drop:
        del out[drop]
    if bad:
        out[bad] = np.zeros((3, 3), np.float32)
    return out


def test_names_and_hparams(fm):
    P = fm.params
    assert P.param_name(3, "ffn_up_exps") == "blk.3.ffn_up_exps.weight"
    assert P.scale_name(0, "ffn_down_exps") == "blk.0.ffn_down_exps.scale"
    mx = fm.HPARAMS["mixtral"]
    assert (mx.embedding_length, mx.feed_forward_length, mx.expert_count, mx.expert_used_count) == (4096, 14336, 8, 2)
    assert mx.block_count == 32 and mx.layer_norm_rms_epsilon == 1e-5 and not mx.normalize_expert_weights
    toy = fm.HPARAMS["toy"]
    assert (toy.embedding_length, toy.feed_forward_length, toy.expert_count, toy.expert_used_count) == (64, 128, 4, 2)
    sh = P.expected_shapes(mx)
    assert sh["ffn_up_exps"] == (14336, 4096, 8) and sh["ffn_down_exps"] == (4096, 14336, 8)
    assert sh["ffn_gate_inp"] == (8, 4096) and sh["ffn_norm"] == (4096,)


def test_missing_and_misshapen_parameters_are_named(fm):
    hp = fm.HPARAMS["toy"]
    with pytest.raises(KeyError, match="blk.1.ffn_gate_exps.weight"):
        fm.load_moe_layers(_params(fm, hp, drop="blk.1.ffn_gate_exps.weight"), hp)
    with pytest.raises(ValueError, match="blk.0.ffn_down_exps.weight"):
        fm.load_moe_layers(_params(fm, hp, bad="blk.0.ffn_down_exps.weight"), hp)
    p = _params(fm, hp)
    p["blk.0.ffn_up_exps.scale"] = np.zeros((128, 3), np.float32)
    with pytest.raises(ValueError, match="blk.0.ffn_up_exps.scale"):
        fm.load_moe_layers(p, hp)
    with pytest.raises(TypeError):
        fm.load_moe_layers(_params(fm, hp), hp, act_dtype=torch.float16)


def test_safetensors_source(fm, tmp_path):
    from safetensors.torch import save_file

    hp = fm.HPARAMS["toy"]
    p = {k: torch.from_numpy(v) for k, v in _params(fm, hp).items()}
    p["blk.0.ffn_norm.weight"] = torch.arange(64, dtype=torch.float32)
    path = tmp_path / "toy.safetensors"
    save_file(p, str(path))
    src = fm.params.ParamSource(path)
    assert "blk.1.ffn_up_exps.weight" in src and "blk.2.ffn_up_exps.weight" not in src
    assert src.shape("blk.0.ffn_down_exps.weight") == (64, 128, 4)
    assert torch.equal(src.get("blk.0.ffn_norm.weight"), torch.arange(64, dtype=torch.float32))
    with pytest.raises(KeyError):
        src.get("blk.0.attn_q.weight")
    with pytest.raises(ValueError, match="not an fmoe packed artifact"):
        fm.load_packed(path)


# ------------------------------------------------------------------ attention tensors
def test_attention_shapes_follow_the_toy_model(fm):
    """tests/models/test_toy_llm.py:80-109: attn_q/attn_output [n_embd, n_embd],
    attn_k/attn_v [n_embd, n_head_kv * head_dim]."""
    hp = fm.ATTN_HPARAMS["toy"]
    s = fm.params.attention_shapes(hp)
    assert s == {"attn_norm": (64,), "attn_q": (64, 64), "attn_k": (64, 32), "attn_v": (64, 32),
                 "attn_output": (64, 64)}
    m = fm.ATTN_HPARAMS["mixtral"]
    assert fm.params.attention_shapes(m)["attn_k"] == (4096, 1024)


def test_attention_loader_checks_shapes_before_device_work(fm):
    hp = fm.ATTN_HPARAMS["toy"]
    params = {f"blk.0.{t}.weight": np.zeros(s, np.float32) for t, s in fm.params.attention_shapes(hp).items()}
    params["blk.0.attn_k.weight"] = np.zeros((64, 16), np.float32)
    with pytest.raises(ValueError, match="attn_k"):
        fm.load_attention_layers(params, hp, layers=[0])
    del params["blk.0.attn_k.weight"]
    with pytest.raises(KeyError, match="attn_k"):
        fm.load_attention_layers(params, hp, layers=[0])
