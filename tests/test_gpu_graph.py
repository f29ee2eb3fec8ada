"""The block and the decode attention captured in a HIP graph (through
torch.cuda.graph) and replayed: every replay must equal the eager call on the
same inputs, with new inputs copied into the captured buffers and eager work
on the stream between replays.  The library's launch sequence holds kernels
only (no memsets, no host synchronisation) when its timers are off."""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _replays_match(make_inputs, static_inputs, run, outputs, n=3):
    g = torch.cuda.CUDAGraph()
    # warm up on a side stream (first-use attribute setup, workspace allocation)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        run()
    for i in range(n):
        fresh = make_inputs(i)
        for dst, src in zip(static_inputs, fresh):
            dst.copy_(src)
        g.replay()
        torch.cuda.synchronize()
        got = [o.clone() for o in outputs]
        _ = torch.ones(1 << 20, device="cuda").sum()  # unrelated eager work between replays
        run()  # eager on the same inputs
        torch.cuda.synchronize()
        for a, b in zip(got, outputs):
            assert torch.equal(a, b), f"replay {i} differs from the eager call"


@pytest.mark.parametrize("noalloc", [False, True])
@pytest.mark.parametrize("T", [1, 16, 300])
def test_moe_ffn_block_graph_replay(fm, wl, T, noalloc):
    """Also the allocation-free entry point (the library's fixed scratch in
    place of the block's workspace): its launches hold no allocation, copy or
    memset either."""
    cfg = wl.scaled(wl.CONFIGS["C3"], 256, 384)
    up, gate, down = wl.expert_weights(cfg, "cuda", dtype=torch.bfloat16)
    packed = [fm.pack_expert_weights(w) for w in (up, gate, down)]

    def make(i):
        x, wr, _ = wl.router_inputs(cfg, T, seed=100 + i)
        return [torch.from_numpy(x).to("cuda", torch.bfloat16)]

    x0, wr, _ = wl.router_inputs(cfg, T, seed=99)
    blk = fm.MoEFFNBlock(torch.from_numpy(wr).to("cuda", torch.bfloat16), *packed, cfg.n_expert, cfg.n_expert_used,
                         cfg.n_embd, cfg.n_ff, cfg.normalize)
    x = torch.from_numpy(x0).to("cuda", torch.bfloat16)
    out = torch.empty((T, cfg.n_embd), dtype=torch.bfloat16, device="cuda")
    _replays_match(make, [x], lambda: blk(x, out=out, noalloc=noalloc), [out])


def test_paged_attention_graph_replay(fm):
    rng = np.random.default_rng(5)
    B, n_embd, H, Hkv, bs, n_blocks, max_ctx = 4, 512, 8, 2, 16, 72, 300
    D = n_embd // H
    bf = torch.bfloat16
    f = lambda *s: torch.from_numpy((rng.standard_normal(s) * 0.2).astype(np.float32)).to("cuda", bf)
    blk = fm.AttentionBlockDecode(f(n_embd, n_embd), f(n_embd, Hkv * D), f(n_embd, Hkv * D), f(n_embd, n_embd),
                                  n_head=H, n_head_kv=Hkv, n_embd=n_embd, act_dtype=bf)
    tables = torch.arange(n_blocks, dtype=torch.int32, device="cuda")[: B * 16].view(1, B, 16)
    lens = torch.tensor([[300, 17, 256, 1]], dtype=torch.int32, device="cuda")
    # the new K/V go to blocks no table names, so calls do not change what later calls read
    bi = torch.arange(64, 64 + B, dtype=torch.int32, device="cuda")
    pi = torch.zeros(B, dtype=torch.int32, device="cuda")
    kp, vp = f(n_blocks, bs, Hkv, D), f(n_blocks, bs, Hkv, D)
    x = f(B, n_embd)
    pos = torch.tensor([300, 17, 256, 1], dtype=torch.int64, device="cuda")
    outs = []

    def run():
        o, k, v = blk.paged(x, pos, kp, vp, 0, tables, lens, max_ctx, bi, pi)
        outs[:] = [o, k, v]

    run()
    torch.cuda.synchronize()
    # the graph writes into the tensors the captured call allocated
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run()
    captured = list(outs)
    for i in range(3):
        x.copy_(f(B, n_embd))
        g.replay()
        torch.cuda.synchronize()
        got = [t.clone() for t in captured]
        run()
        torch.cuda.synchronize()
        for a, b in zip(got, outs):
            assert torch.equal(a, b), f"replay {i} differs from the eager call"
