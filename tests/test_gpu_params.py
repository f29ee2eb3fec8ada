"""MoE layers loaded from GGUF-named parameters, on the GPU.

* Every loaded layer's sub-layer equals the oracle sub-layer on THAT
  layer's tensors (blk.{i}, not blk.0), routing bit-exact, output within the
  configuration tolerance (fp32 1e-4, bf16 2e-2, fp8 5e-2 vs the dequantised
  weights).
* A packed artifact (save_packed -> load_packed) reproduces the loaded
  layers bit for bit, bf16 and fp8.
* Offline fp8 (quantize_fp8) equals quantise-on-load, and pre-quantised
  codes + scales in the parameter set (from the pinned host quantiser)
  equal both, bit for bit.
* A safetensors file and a dict with the same tensors load the same layers.
"""

import numpy as np
import pytest
import torch

from oracle import layer as ol
from oracle import numerics as nm

pytestmark = pytest.mark.gpu


def _model(fm, wl, hp, T, act="bf16", seed=0):
    """GGUF-named parameters for hp.block_count layers plus one residual
    input per layer whose normalised rows meet the router margin."""
    P = fm.params
    cfg = wl.Config("P", hp.embedding_length, hp.feed_forward_length, hp.expert_count, hp.expert_used_count,
                    (T,), act, act, hp.normalize_expert_weights, 1e-3, rtol=1e-4 if act == "f32" else 2e-2,
                    seed=seed)
    std = 0.02 * (4096 / hp.embedding_length) ** 0.5
    params, inputs = {}, []
    for i in range(hp.block_count):
        res, nw, wr, eps, _ = wl.sublayer_inputs(cfg, T, seed=1000 * seed + i, eps=hp.layer_norm_rms_epsilon,
                                                 scale_range=(0.1, 1.5))
        up, gate, down = wl.expert_weights(cfg, "cpu", seed=77 * seed + i, std=std)
        rnd = (lambda a: a) if act == "f32" else (lambda a: a.bfloat16().float())
        params[P.param_name(i, "ffn_norm")] = nw
        params[P.param_name(i, "ffn_gate_inp")] = wr
        params[P.param_name(i, "ffn_up_exps")] = rnd(up).numpy()
        params[P.param_name(i, "ffn_gate_exps")] = rnd(gate).numpy()
        params[P.param_name(i, "ffn_down_exps")] = rnd(down).numpy()
        inputs.append(res)
    return cfg, params, inputs


def _run(layers, inputs, act):
    dt = torch.float32 if act == "f32" else torch.bfloat16
    outs, ids = [], []
    for lay, res in zip(layers, inputs):
        r = torch.from_numpy(res).to("cuda", dt)
        o = lay(r)
        torch.cuda.synchronize()
        outs.append(o.float().cpu().numpy())
        ids.append(lay.block.routing(r.shape[0])[0].cpu().numpy())
    return outs, ids


def _oracle(fm, hp, params, i, res, fp8=False):
    P = fm.params
    w = [params[P.param_name(i, t)] for t in ("ffn_up_exps", "ffn_gate_exps", "ffn_down_exps")]
    if fp8:
        w = [nm.dequantize_e4m3fn(*nm.quantize_per_channel_e4m3fn(np.asarray(a, np.float32))) for a in w]
    return ol.moe_ffn_sublayer(res, params[P.param_name(i, "ffn_norm")], hp.layer_norm_rms_epsilon,
                               params[P.param_name(i, "ffn_gate_inp")], *w, hp.expert_count, hp.expert_used_count,
                               hp.embedding_length, hp.feed_forward_length, hp.normalize_expert_weights,
                               return_routing=True)


def _check(outs, ids, fm, hp, params, inputs, rtol, fp8=False):
    from helpers import assert_close_rms

    for i, res in enumerate(inputs):
        ref, ref_ids, _ = _oracle(fm, hp, params, i, res, fp8)
        np.testing.assert_array_equal(ids[i], ref_ids, err_msg=f"layer {i}")
        assert_close_rms(outs[i], ref, rtol, what=f"layer {i}")


@pytest.mark.parametrize("act", ["f32", "bf16"])
def test_toy_model_layers(fm, wl, act):
    hp = fm.HPARAMS["toy"]
    cfg, params, inputs = _model(fm, wl, hp, 24, act)
    layers = fm.load_moe_layers(params, hp, act_dtype=torch.float32 if act == "f32" else torch.bfloat16)
    assert [lay.index for lay in layers] == [0, 1]
    outs, ids = _run(layers, inputs, act)
    _check(outs, ids, fm, hp, params, inputs, cfg.rtol)
    # each layer reads its own blk.{i} tensors: layer 1 on layer 0's input differs from layer 0
    o10, _ = _run(layers[1:], inputs[:1], act)
    assert not np.allclose(o10[0], outs[0], rtol=1e-2, atol=1e-2)


def test_packed_artifact_round_trip(fm, wl, tmp_path):
    hp = fm.MoEHParams(2, 256, 512, 8, 2, 1e-5, False)
    cfg, params, inputs = _model(fm, wl, hp, 40, "bf16", seed=1)
    layers = fm.load_moe_layers(params, hp)
    outs, ids = _run(layers, inputs, "bf16")
    _check(outs, ids, fm, hp, params, inputs, 2e-2)
    path = tmp_path / "packed.safetensors"
    fm.save_packed(layers, path)
    again = fm.load_packed(path)
    outs2, ids2 = _run(again, inputs, "bf16")
    for a, b in zip(outs, outs2):
        np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))
    # one layer on its own
    only1 = fm.load_packed(path, layers=[1])
    o1, _ = _run(only1, inputs[1:], "bf16")
    np.testing.assert_array_equal(o1[0].view(np.uint32), outs[1].view(np.uint32))


def test_fp8_offline_quantisation(fm, wl, tmp_path):
    hp = fm.MoEHParams(2, 256, 512, 8, 2, 1e-5, False)
    cfg, params, inputs = _model(fm, wl, hp, 40, "bf16", seed=2)
    on_load = fm.load_moe_layers(params, hp, weight_dtype="fp8")
    assert all(lay.weight_dtype == fm.lowlevel.F8E4M3FN for lay in on_load)
    outs, ids = _run(on_load, inputs, "bf16")
    _check(outs, ids, fm, hp, params, inputs, 5e-2, fp8=True)
    path = tmp_path / "fp8.safetensors"
    fm.quantize_fp8(params, hp, path)
    offline, _ = _run(fm.load_packed(path), inputs, "bf16")
    # pre-quantised codes + scales from the host quantiser
    P = fm.params
    pq = dict(params)
    for i in range(hp.block_count):
        for t in ("ffn_up_exps", "ffn_gate_exps", "ffn_down_exps"):
            q, s = nm.quantize_per_channel_e4m3fn(np.asarray(params[P.param_name(i, t)], np.float32))
            pq[P.param_name(i, t)] = torch.from_numpy(q).view(torch.float8_e4m3fn)
            pq[P.scale_name(i, t)] = s.astype(np.float32)
    prequant, _ = _run(fm.load_moe_layers(pq, hp), inputs, "bf16")
    for a, b, c in zip(outs, offline, prequant):
        np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))
        np.testing.assert_array_equal(a.view(np.uint32), c.view(np.uint32))


def test_safetensors_and_dict_sources_agree(fm, wl, tmp_path):
    from safetensors.torch import save_file

    hp = fm.HPARAMS["toy"]
    _, params, inputs = _model(fm, wl, hp, 16, "bf16", seed=3)
    path = tmp_path / "toy.safetensors"
    save_file({k: torch.from_numpy(np.ascontiguousarray(v)) for k, v in params.items()}, str(path))
    a, _ = _run(fm.load_moe_layers(params, hp), inputs, "bf16")
    b, _ = _run(fm.load_moe_layers(path, hp), inputs, "bf16")
    for x, y in zip(a, b):
        np.testing.assert_array_equal(x.view(np.uint32), y.view(np.uint32))


# ------------------------------------------------------------------ attention tensors
@pytest.mark.parametrize("act,bias", [("f32", False), ("f32", True), ("bf16", False)])
def test_attention_layers_from_named_parameters(fm, act, bias):
    """blk.{i}.attn_* tensors (tests/models/test_toy_llm.py:80-109 layout) load
    into AttentionBlockDecode; each layer equals the oracle on its own tensors."""
    from dataclasses import replace

    from oracle import attention as oa
    from helpers import assert_close_rms

    hp = replace(fm.ATTN_HPARAMS["toy"], use_attention_bias=bias)
    shapes = fm.params.attention_shapes(hp)
    rng = np.random.default_rng(3 + bias)
    params = {}
    for i in range(hp.block_count):
        for t, s in shapes.items():
            params[f"blk.{i}.{t}.weight"] = (rng.standard_normal(s) * 0.2).astype(np.float32)
        for t in ("attn_q", "attn_k", "attn_v", "attn_output"):
            params[f"blk.{i}.{t}.bias"] = (rng.standard_normal(shapes[t][1]) * 0.1).astype(np.float32)
    dt = torch.float32 if act == "f32" else torch.bfloat16
    layers = fm.load_attention_layers(params, hp, act_dtype=dt)
    assert [lay.index for lay in layers] == list(range(hp.block_count))
    B, ctx, H, Hkv, n = 3, 20, hp.attention_head_count, hp.attention_head_count_kv, hp.embedding_length
    D = n // H
    rnd = (lambda a: a) if act == "f32" else nm.bf16_round
    for lay in layers:
        i = lay.index
        w = {t: rnd(params[f"blk.{i}.{t}.weight"]) for t in ("attn_q", "attn_k", "attn_v", "attn_output")}
        x = rnd(rng.standard_normal((B, n)).astype(np.float32))
        kc = rnd(rng.standard_normal((B, ctx, Hkv, D)).astype(np.float32))
        vc = rnd(rng.standard_normal((B, ctx, Hkv, D)).astype(np.float32))
        pos = np.array([20, 5, 300], np.int64)
        out, k_new, _ = lay.attn(torch.from_numpy(x).to("cuda", dt), torch.from_numpy(pos).cuda(),
                                 torch.from_numpy(kc).to("cuda", dt), torch.from_numpy(vc).to("cuda", dt))
        b = [params[f"blk.{i}.{t}.bias"] for t in ("attn_q", "attn_k", "attn_v", "attn_output")]
        ref = oa.attention_block_decode(x, pos, kc, vc, w["attn_q"], w["attn_k"], w["attn_v"], w["attn_output"],
                                        *b, bias, H, Hkv, n, hp.rope_freq_base, hp.rope_freq_scale)
        rtol = 1e-4 if act == "f32" else 2e-2
        assert_close_rms(out.float().cpu().numpy(), ref[0], rtol, what=f"layer {i}")
        assert_close_rms(k_new.float().cpu().numpy(), ref[1], rtol, what=f"layer {i} k_new")
        np.testing.assert_array_equal(lay.norm_w.float().cpu().numpy(), rnd(params[f"blk.{i}.attn_norm.weight"]))
