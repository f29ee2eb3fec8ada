"""The layer glue on the GPU vs the oracle: ffn_norm RMSNorm and the MoE FFN
sub-layer (RMSNorm -> moe_ffn_block -> residual add) of
architectures/llm/transformer_layer_moe_prefill.mlir:205-242.

* rms_norm: fp32 rtol 1e-5; bf16 output within one bf16 rounding (rtol 4e-3)
  of the float64 oracle on the same bf16 inputs; vector and scalar kernels
  (hidden sizes with and without a factor of 4); in place.
* Sub-layer: routing on the normalised rows bit-exact with the oracle's;
  output within the configuration's rtol (atol = rtol * RMS(reference)), and
  the block's contribution (output - residual) within rtol as a relative
  Frobenius error, on data where that contribution is a large part of the
  output; the in-place form (out aliases residual) equals the out-of-place one
  bit for bit.
"""

import numpy as np
import pytest
import torch

from oracle import layer as ol
from oracle import moe as om
from oracle import numerics as nm
from helpers import assert_close_rms

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("rows,H", [(1, 64), (7, 67), (33, 4096), (300, 2048), (5, 3)])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_rms_norm(fm, rows, H, dtype):
    rng = np.random.default_rng(rows * 1000 + H)
    x = (rng.standard_normal((rows, H)) * rng.uniform(0.1, 20.0, (rows, 1))).astype(np.float32)
    w = rng.standard_normal(H).astype(np.float32)
    eps = 1e-5
    if dtype == "bf16":
        xt = torch.from_numpy(x).cuda().bfloat16()
        wt = torch.from_numpy(w).cuda().bfloat16()
        out = fm.rms_norm(xt, wt, eps).float().cpu().numpy()
        ref = ol.rms_norm(xt.float().cpu().numpy(), wt.float().cpu().numpy(), eps)
        np.testing.assert_allclose(out, ref, rtol=4e-3, atol=4e-3 * np.abs(w).max() * 1e-3)
    else:
        out = fm.rms_norm(x, w, eps)
        assert isinstance(out, np.ndarray) and out.dtype == np.float32
        ref = ol.rms_norm(x, w, eps)
        np.testing.assert_allclose(out, ref, rtol=1e-5, atol=1e-6)


def test_rms_norm_in_place_and_batched_rows(fm):
    ll = fm.lowlevel
    rng = np.random.default_rng(3)
    x = torch.from_numpy(rng.standard_normal((2, 5, 128)).astype(np.float32)).cuda()
    w = torch.from_numpy(rng.uniform(0.5, 2, 128).astype(np.float32)).cuda()
    ref = fm.rms_norm(x, w, 1e-6)  # [..., H] rows
    assert ref.shape == x.shape
    y = x.clone()
    ll.call("fmoe_rms_norm", y.data_ptr(), w.data_ptr(), 1e-6, y.data_ptr(), 10, 128, ll.F32,
            torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert torch.equal(y, ref)


# Residual scales per configuration: the norm removes them, so they only set
# the residual's size next to the block's output (small for C4, whose 64
# unnormalised top-6 routing weights are ~0.05).
RES_SCALE = {"C1": (0.25, 4.0), "C2": (0.1, 1.5), "C3": (0.25, 4.0), "C4": (0.02, 0.2), "C5": (0.1, 1.5)}


class SubCase:
    def __init__(self, fm, wl, cfg, T, scale_range=None, fp8_activations=False):
        self.cfg, self.T = cfg, T
        res, nw, wr, eps, _ = wl.sublayer_inputs(cfg, T, scale_range=scale_range or RES_SCALE[cfg.name[:2]])
        act = torch.bfloat16 if cfg.act == "bf16" else torch.float32
        self.res_np, self.nw_np, self.wr_np, self.eps = res, nw, wr, eps
        self.res = torch.from_numpy(res).to("cuda", act)
        self.nw = torch.from_numpy(nw).to("cuda", act)
        wr_t = torch.from_numpy(wr).to("cuda", act)
        # std 0.02 at Mixtral's hidden size; scaled so that smaller test shapes
        # keep the block's output on the order of the residual.
        std = 0.02 * (4096 / cfg.n_embd) ** 0.5
        up, gate, down = wl.expert_weights(cfg, "cuda", dtype=torch.float32 if cfg.act == "f32" else torch.bfloat16,
                                           std=std)
        if cfg.weights == "fp8":
            packed = [fm.quantize_expert_weights(w) for w in (up, gate, down)]
            self.host_w = []
            for w in (up, gate, down):
                q, s = nm.quantize_per_channel_e4m3fn(w.float().cpu().numpy())
                self.host_w.append(nm.dequantize_e4m3fn(q, s))
        else:
            packed = [fm.pack_expert_weights(w) for w in (up, gate, down)]
            self.host_w = [w.float().cpu().numpy() for w in (up, gate, down)]
        self.block = fm.MoEFFNBlock(wr_t, *packed, cfg.n_expert, cfg.n_expert_used, cfg.n_embd, cfg.n_ff,
                                    cfg.normalize, act_dtype=act, fp8_activations=fp8_activations)

    def run(self, out=None):
        o = self.block.sublayer(self.res if out is None else out, self.nw, self.eps, out=out)
        torch.cuda.synchronize()
        return o.float().cpu().numpy()

    def oracle(self, tokens=None):
        c = self.cfg
        r = self.res_np if tokens is None else self.res_np[tokens]
        return ol.moe_ffn_sublayer(r, self.nw_np, self.eps, self.wr_np, *self.host_w, c.n_expert,
                                   c.n_expert_used, c.n_embd, c.n_ff, c.normalize, dtype=np.float64,
                                   return_routing=True)

    def check(self, out, tokens=None):
        ref, ids, _ = self.oracle(tokens)
        dev_ids = self.block.routing(self.T)[0].cpu().numpy()
        if tokens is not None:
            dev_ids = dev_ids[:, tokens]
        np.testing.assert_array_equal(dev_ids, ids)
        r = self.res_np if tokens is None else self.res_np[tokens]
        o = out if tokens is None else out[tokens]
        what = f"{self.cfg.name} T={self.T}"
        assert_close_rms(o, ref, self.cfg.rtol, what=what + " output")
        # The block's contribution alone (output - residual) vs the oracle's,
        # as a relative Frobenius error: element-wise it carries the output's
        # rounding at the residual's magnitude.  The data must make the block
        # a large part of the output, or the check above would not see it.
        d_ref = ref - r
        assert np.linalg.norm(d_ref) > 0.2 * np.linalg.norm(ref), what
        rel = np.linalg.norm((o - r) - d_ref) / np.linalg.norm(d_ref)
        assert rel <= self.cfg.rtol, (what, rel)


def test_sublayer_c1_fp32(fm, wl):
    case = SubCase(fm, wl, wl.CONFIGS["C1"], 32)
    case.check(case.run())


@pytest.mark.parametrize("name,H,F,T", [("C2", 256, 512, 16), ("C2", 256, 512, 300), ("C3", 128, 256, 200),
                                        ("C4", 256, 384, 5), ("C5", 256, 512, 64)])
def test_sublayer_scaled(fm, wl, name, H, F, T):
    cfg = wl.scaled(wl.CONFIGS[name], H, F)
    case = SubCase(fm, wl, cfg, T)
    case.check(case.run())


@pytest.mark.parametrize("name,T,sample", [("C2", 16, None), ("C4", 64, None), ("C2", 4096, 128)])
def test_sublayer_full_size(fm, wl, name, T, sample):
    case = SubCase(fm, wl, wl.CONFIGS[name], T)
    out = case.run()
    tok = None if sample is None else np.sort(np.random.default_rng(T).choice(T, sample, replace=False))
    case.check(out, tok)


# One decode token at full size: at most 16 assignments, so the down
# projection, the slot-ordered combine and the residual add run in one launch
# (no combine launch recorded).  Residual scales at the low end of each
# configuration's range keep the block a large part of a single row's output.
@pytest.mark.parametrize("name,scale", [("C4", (0.02, 0.03)), ("C2", (0.1, 0.15)), ("C5", (0.1, 0.15))])
def test_sublayer_one_token_fused(fm, wl, name, scale):
    case = SubCase(fm, wl, wl.CONFIGS[name], 1, scale_range=scale)
    ll = fm.lowlevel
    ll.timing_read()
    ll.timing_enable(True)
    try:
        out = case.run()
        kern = ll.timing_read()
    finally:
        ll.timing_enable(False)
    assert kern["combine"][1] == 0 and kern["down"][1] > 0, kern
    case.check(out)
    buf = case.res.clone()
    again = case.run(out=buf)
    np.testing.assert_array_equal(out.view(np.uint32), again.view(np.uint32))


def test_sublayer_two_term_fp8_activations(fm, wl):
    """The sub-layer with fp8 weights and two-term e4m3 activations at a
    prefill size (both GEMMs on the fp8 MFMA, the residual added in the
    combine): within C5's tolerance of the oracle on the dequantised weights
    with bf16 activations, and in place equal to out of place."""
    cfg = wl.scaled(wl.CONFIGS["C5"], 512, 1024)
    case = SubCase(fm, wl, cfg, 300, fp8_activations="x2")
    assert case.block.wdt == fm.lowlevel.F8E4M3FN_A8X2
    a = case.run()
    case.check(a)
    buf = case.res.clone()
    b = case.run(out=buf)
    np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))


def test_sublayer_in_place_equals_out_of_place(fm, wl):
    cfg = wl.scaled(wl.CONFIGS["C3"], 128, 256)
    case = SubCase(fm, wl, cfg, 100)
    a = case.run()
    buf = case.res.clone()
    b = case.run(out=buf)
    np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))


def test_sublayer_numpy_drop_in(fm, wl):
    cfg = wl.CONFIGS["C1"]
    res, nw, wr, eps, _ = wl.sublayer_inputs(cfg, 32)
    rng = np.random.default_rng(1)
    up = (rng.standard_normal((128, 64, 8)) * 0.02).astype(np.float32)
    gate = (rng.standard_normal((128, 64, 8)) * 0.02).astype(np.float32)
    down = (rng.standard_normal((64, 128, 8)) * 0.02).astype(np.float32)
    out = fm.moe_ffn_sublayer(res, nw, eps, wr, up, gate, down, 8, 2, 64, 128, True)
    assert isinstance(out, np.ndarray) and out.dtype == np.float32 and out.shape == (32, 64)
    xn = ol.rms_norm(res, nw, eps, dtype=np.float32)
    ref = res + om.moe_ffn_block_literal(xn, wr, up, gate, down, 8, 2, 64, 128, True)
    np.testing.assert_allclose(out, ref, rtol=1e-4, atol=1e-5)
