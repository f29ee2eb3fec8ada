"""fmoe_moe_ffn_block_noalloc (the block with the library's fixed per-GPU
scratch instead of a workspace) against fmoe_moe_ffn_block, through the C
ABI: the same kernels run, so the outputs must be bit-identical.  Two calls
in a row on one block, the second with fewer tokens, so the second call
runs on scratch the first one left behind."""

import ctypes
import sys

import pytest
import torch

pytestmark = pytest.mark.gpu


def _p(t):
    return ctypes.c_void_p(t.data_ptr() if t is not None else 0)


def _call(fm, blk, name, x, out, ws=None):
    L = fm.lowlevel
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    args = [_p(x), _p(blk.wr), _p(blk.up.data), _p(blk.gate.data), _p(blk.down.data), _p(blk.up.scales),
            _p(blk.gate.scales), _p(blk.down.scales), blk.wdt, _p(out), x.shape[0], blk.n_expert, blk.k,
            blk.n_embd, blk.n_ff, int(blk.normalize), blk.act]
    if ws is not None:
        args += [_p(ws), ws.numel()]
    L.call(name, *args, stream)


# (config, n_embd, n_ff, weights, token counts): decode-sized batches (the
# split-logits router and the weight-streaming GEMM) and prefill-sized ones
# (the 256x256-tile GEMMs, a K-split down projection), bf16 and fp8 weights.
CASES = [
    ("C4", None, None, "bf16", (64, 5)),
    # 18 assignments, then 6: the second call fuses the down projection and
    # the combine into one launch (batches of at most 16 assignments)
    ("C4", None, None, "bf16", (3, 1)),
    ("C2", 1024, 2048, "bf16", (1200, 300)),
    ("C5", 512, 1024, "fp8", (100, 33)),
    ("C3", 512, 256, "bf16", (700, 64)),
]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_noalloc_matches_workspace_entry(fm, wl, case):
    name, H, F, wdt, tokens = CASES[case]
    cfg = wl.CONFIGS[name]
    if H is not None:
        cfg = wl.scaled(cfg, H, F)
    print(f"[noalloc] {cfg.name} weights {wdt} tokens {tokens}", file=sys.stderr, flush=True)
    torch.cuda.set_device(0)
    up, gate, down = wl.expert_weights(cfg, "cuda", dtype=torch.bfloat16)
    if wdt == "fp8":
        up, gate, down = (fm.quantize_expert_weights(w) for w in (up, gate, down))
    x_np, wr_np, _ = wl.router_inputs(cfg, max(tokens))
    wr = torch.from_numpy(wr_np).to("cuda", torch.bfloat16)
    blk = fm.MoEFFNBlock(wr, up, gate, down, cfg.n_expert, cfg.n_expert_used, cfg.n_embd, cfg.n_ff,
                         cfg.normalize, act_dtype=torch.bfloat16)
    lib = fm.lowlevel.lib()
    for T in tokens:
        need = lib.fmoe_moe_ffn_block_workspace_bytes(T, cfg.n_expert, cfg.n_expert_used, cfg.n_embd, cfg.n_ff,
                                                      blk.act, blk.wdt)
        assert 0 < need <= fm.lowlevel.NOALLOC_SCRATCH_BYTES
        x = torch.from_numpy(x_np[:T]).to("cuda", torch.bfloat16).contiguous()
        ws = torch.empty(need, dtype=torch.uint8, device="cuda")
        want = torch.empty((T, cfg.n_embd), dtype=torch.bfloat16, device="cuda")
        got = torch.full((T, cfg.n_embd), float("nan"), dtype=torch.bfloat16, device="cuda")
        _call(fm, blk, "fmoe_moe_ffn_block_noalloc", x, got)
        _call(fm, blk, "fmoe_moe_ffn_block", x, want, ws)
        torch.cuda.synchronize()
        assert torch.isfinite(got.float()).all()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"T={T}"
        # the Python path reaches the same entry point
        again = blk(x, noalloc=True)
        torch.cuda.synchronize()
        assert torch.equal(again.view(torch.int16), want.view(torch.int16)), f"T={T} (Python)"


# The rejection of a batch beyond the scratch (before any device work) is
# tested on the CPU: tests/test_boundary.py::test_noalloc_block_rejects_oversize_before_device.
