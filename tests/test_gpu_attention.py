"""The decode step's attention half on the GPU against the oracle
(oracle/attention.py).

* Paged cache copies (gather, scatter_decode, scatter_prefill) are compared
  bit-exactly, in f32 and bf16, on the reference's own table layouts
  (tests/components/test_kvcache.py) and on edge cases: contexts longer than
  max_context_len, table entries outside the pool, duplicate slots.
* attention_block_decode and the paged decode: fp32 rtol 1e-4, bf16 2e-2,
  fp8 weights 5e-2 against the oracle on the dequantised weights; atol =
  rtol * RMS(reference) (helpers.assert_close_rms).  bf16 inputs are rounded
  to bf16 before the oracle sees them.
"""

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import numerics as nm
from helpers import assert_close_rms

pytestmark = pytest.mark.gpu

DT = {"f32": torch.float32, "bf16": torch.bfloat16}


def _dev(a, dt):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to("cuda", dt)


def _host(t):
    return t.float().cpu().numpy()


def _round(a, dt):
    return nm.bf16_round(np.asarray(a, np.float32)) if dt == torch.bfloat16 else np.asarray(a, np.float32)


# ------------------------------------------------------------------ paged cache
@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_kvcache_gather_reference_layout(fm, dt):
    """TestGather.test_basic / test_variable_context_lens layouts
    (tests/components/test_kvcache.py:78-100, :183-230)."""
    rng = np.random.default_rng(42)
    cache = _round(rng.standard_normal((8, 4, 2, 8)), DT[dt])
    tables = np.array([[[0, 1, 2, 0], [3, 4, 5, 0]], [[5, 4, 3, 2], [1, 0, 7, 6]]], np.int32)
    lens = np.array([[10, 8], [16, 3]], np.int32)
    c = _dev(cache, DT[dt])
    for layer, max_ctx in ((0, 12), (1, 16), (1, 5), (0, 0)):
        got = fm.kvcache_gather(c, layer, tables, lens, max_ctx)
        np.testing.assert_array_equal(_host(got), oa.kv_gather(cache, layer, tables, lens, max_ctx))


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_kvcache_gather_out_of_pool_entries_read_zero(fm, dt):
    rng = np.random.default_rng(1)
    cache = _round(rng.standard_normal((4, 2, 1, 4)), DT[dt])
    tables = np.array([[[0, -1, 9]]], np.int32)   # entries outside [0, 4): zero rows
    lens = np.array([[6]], np.int32)
    got = _host(fm.kvcache_gather(_dev(cache, DT[dt]), 0, tables, lens, 8))
    np.testing.assert_array_equal(got[0, :2], cache[0])
    np.testing.assert_array_equal(got[0, 2:], 0)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_kvcache_scatter_decode(fm, dt):
    rng = np.random.default_rng(2)
    cache = _round(rng.standard_normal((5, 4, 2, 8)), DT[dt])
    vals = _round(rng.standard_normal((6, 2, 8)), DT[dt])
    bi = np.array([1, 3, 1, 0, 4, 7], np.int32)   # slot (1, 2) twice: the later row wins; block 7 is outside
    pi = np.array([2, 0, 2, 3, 1, 0], np.int32)
    c = _dev(cache, DT[dt])
    fm.kvcache_scatter_decode(c, 0, _dev(vals, DT[dt]), bi, pi)
    want = oa.kv_scatter_decode(cache, vals, bi[:5], pi[:5])
    np.testing.assert_array_equal(_host(c), want)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_kvcache_scatter_prefill_then_gather(fm, dt):
    """TestScatterPrefill / test_scatter_then_gather layouts
    (tests/components/test_kvcache.py:351-560)."""
    rng = np.random.default_rng(3)
    bs = 4
    tables = np.array([[[3, 0, 5, 6], [1, 2, 4, 7]], [[7, 6, 5, 4], [3, 2, 1, 0]]], np.int32)
    vals = _round(rng.standard_normal((2, 9, 2, 8)), DT[dt])
    start = np.array([0, 3], np.int32)
    cache = np.zeros((8, bs, 2, 8), np.float32)
    c = _dev(cache, DT[dt])
    fm.kvcache_scatter_prefill(c, 1, _dev(vals, DT[dt]), tables, start, bs)
    want = oa.kv_scatter_prefill(cache, 1, vals, tables, start, bs)
    np.testing.assert_array_equal(_host(c), want)
    lens = np.array([[0, 0], [9, 12]], np.int32)
    got = _host(fm.kvcache_gather(c, 1, tables, lens, 12))
    np.testing.assert_array_equal(got, oa.kv_gather(want, 1, tables, lens, 12))
    np.testing.assert_array_equal(got[1, 3:12], vals[1])


# ------------------------------------------------------------------ attention_block_decode
def _weights(rng, n_embd, nkv, dt, fp8=False):
    s = 1.0 / np.sqrt(n_embd)
    w = {k: rng.standard_normal(shape).astype(np.float32) * s
         for k, shape in (("wq", (n_embd, n_embd)), ("wk", (n_embd, nkv)), ("wv", (n_embd, nkv)),
                          ("wo", (n_embd, n_embd)))}
    b = {k: (rng.standard_normal(n) * 0.1).astype(np.float32)
         for k, n in (("bq", n_embd), ("bk", nkv), ("bv", nkv), ("bo", n_embd))}
    host = {}
    for k, v in w.items():
        v = _round(v, dt)
        if fp8:
            q, sc = nm.quantize_per_channel_e4m3fn(v.T[:, :, None])
            host[k] = nm.dequantize_e4m3fn(q, sc)[:, :, 0].T
        else:
            host[k] = v
        w[k] = v
    return w, b, host


CASES = [
    # B, ctx, n_embd, n_head, n_head_kv, bias, dtype
    (2, 5, 64, 4, 2, True, "f32"),        # the toy model's heads (head_dim 16, 2 per KV head)
    (3, 0, 64, 4, 2, False, "f32"),       # no cached positions
    (4, 300, 512, 4, 4, True, "f32"),     # head_dim 128, MHA, 2 context splits
    (2, 257, 256, 8, 1, False, "f32"),    # head_dim 32, 8 query heads per KV head
    (5, 1000, 1024, 16, 2, True, "bf16"),  # head_dim 64
    (4, 513, 4096, 32, 8, True, "bf16"),   # Mixtral heads: head_dim 128, 4 per KV head
    (1, 256, 4096, 32, 8, False, "bf16"),  # exactly one split
    (40, 100, 512, 4, 2, True, "bf16"),    # 40 rows: RoPE after a K-split Q/K/V product
    (40, 50, 320, 5, 5, True, "bf16"),     # 40 rows, 960 / 320 outputs: partial 256-column tiles, K split
    # bf16 scores on the matrix cores (head_dim 64 / 128) for every group
    # size, with contexts that end inside an 8-position tile
    (3, 77, 512, 4, 4, False, "bf16"),     # head_dim 128, MHA
    (2, 301, 1024, 8, 1, False, "bf16"),   # head_dim 128, 8 per KV head
    (3, 19, 256, 4, 2, True, "bf16"),      # head_dim 64, 2 per KV head
    (2, 130, 512, 8, 2, False, "bf16"),    # head_dim 64, 4 per KV head
    (2, 45, 256, 8, 4, False, "bf16"),     # head_dim 32: bf16 scores on the vector units
]


@pytest.mark.parametrize("B,ctx,n_embd,H,Hkv,bias,dt", CASES)
def test_attention_block_decode(fm, B, ctx, n_embd, H, Hkv, bias, dt):
    rng = np.random.default_rng(B * 7919 + ctx + n_embd)
    D = n_embd // H
    tdt = DT[dt]
    w, b, hw = _weights(rng, n_embd, Hkv * D, tdt)
    x = _round(rng.standard_normal((B, n_embd)), tdt)
    kc = _round(rng.standard_normal((B, ctx, Hkv, D)), tdt)
    vc = _round(rng.standard_normal((B, ctx, Hkv, D)), tdt)
    pos = rng.integers(0, 4096, B).astype(np.int64)
    blk = fm.AttentionBlockDecode(*(_dev(w[k], tdt) for k in ("wq", "wk", "wv", "wo")),
                                  *(torch.from_numpy(b[k]).cuda() for k in ("bq", "bk", "bv", "bo")),
                                  use_bias=bias, n_head=H, n_head_kv=Hkv, n_embd=n_embd, act_dtype=tdt)
    out, k_new, v_new = blk(_dev(x, tdt), torch.from_numpy(pos).cuda(), _dev(kc, tdt), _dev(vc, tdt))
    torch.cuda.synchronize()
    ref = oa.attention_block_decode(x, pos, kc, vc, hw["wq"], hw["wk"], hw["wv"], hw["wo"], b["bq"], b["bk"], b["bv"],
                                    b["bo"], bias, H, Hkv, n_embd)
    rtol = 1e-4 if dt == "f32" else 2e-2
    what = f"B={B} ctx={ctx} n_embd={n_embd} H={H}/{Hkv} {dt}"
    assert_close_rms(_host(out), ref[0], rtol, what=what)
    assert_close_rms(_host(k_new), ref[1], rtol, what=what + " k_new")
    assert_close_rms(_host(v_new), ref[2], rtol, what=what + " v_new")


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_rope_large_positions(fm, dt):
    """RoPE angles up to 1e6 rad (positions near 1e6, the head's first pair):
    the angles are formed in double precision, so the rotated k_new follows
    the float64 oracle as closely as at small positions (bf16: RoPE in the
    Q/K/V GEMM's epilogue; f32: the separate RoPE kernel)."""
    rng = np.random.default_rng(5)
    tdt = DT[dt]
    B, ctx, n_embd, H, Hkv = 4, 3, 256, 4, 2
    D = n_embd // H
    w, b, hw = _weights(rng, n_embd, Hkv * D, tdt)
    x = _round(rng.standard_normal((B, n_embd)), tdt)
    kc = _round(rng.standard_normal((B, ctx, Hkv, D)), tdt)
    vc = _round(rng.standard_normal((B, ctx, Hkv, D)), tdt)
    pos = np.array([999_983, 524_287, 65_537, 1_000_000], np.int64)
    blk = fm.AttentionBlockDecode(*(_dev(w[k], tdt) for k in ("wq", "wk", "wv", "wo")),
                                  *(torch.from_numpy(b[k]).cuda() for k in ("bq", "bk", "bv", "bo")),
                                  use_bias=True, n_head=H, n_head_kv=Hkv, n_embd=n_embd, act_dtype=tdt)
    out, k_new, _ = blk(_dev(x, tdt), torch.from_numpy(pos).cuda(), _dev(kc, tdt), _dev(vc, tdt))
    torch.cuda.synchronize()
    ref = oa.attention_block_decode(x, pos, kc, vc, hw["wq"], hw["wk"], hw["wv"], hw["wo"], b["bq"], b["bk"], b["bv"],
                                    b["bo"], True, H, Hkv, n_embd)
    rtol = 1e-4 if dt == "f32" else 1e-2
    assert_close_rms(_host(k_new), ref[1], rtol, what=f"k_new at large positions {dt}")
    assert_close_rms(_host(out), ref[0], 1e-4 if dt == "f32" else 2e-2, what=f"output at large positions {dt}")


def test_attention_block_decode_reference_signature(fm):
    """NumPy in / NumPy out through the reference's positional signature."""
    rng = np.random.default_rng(11)
    n_embd, H, Hkv, B, ctx = 64, 4, 2, 2, 7
    w, b, _ = _weights(rng, n_embd, 32, torch.float32)
    x = rng.standard_normal((B, n_embd)).astype(np.float32)
    kc = rng.standard_normal((B, ctx, Hkv, 16)).astype(np.float32)
    vc = rng.standard_normal((B, ctx, Hkv, 16)).astype(np.float32)
    pos = np.array([3, 40], np.int64)
    got = fm.attention_block_decode(x, pos, kc, vc, w["wq"], w["wk"], w["wv"], w["wo"], b["bq"], b["bk"], b["bv"],
                                    b["bo"], True, H, Hkv, n_embd, 10000.0, 1.0)
    ref = oa.attention_block_decode(x, pos, kc, vc, w["wq"], w["wk"], w["wv"], w["wo"], b["bq"], b["bk"], b["bv"],
                                    b["bo"], True, H, Hkv, n_embd, 10000.0, 1.0)
    for g, r in zip(got, ref):
        assert isinstance(g, np.ndarray) and g.dtype == np.float32
        assert_close_rms(g, r, 1e-4)


@pytest.mark.parametrize("B", [3, 20, 48])
def test_attention_block_decode_fp8_weights(fm, B):
    """fp8-e4m3 projection weights: streamed with the fused epilogues (3
    rows), streamed with a K split and the separate RoPE (20 rows), and on
    the 256-row tile kernel with a K split (48 rows)."""
    rng = np.random.default_rng(12 + B)
    ctx, n_embd, H, Hkv = 400, 1024, 8, 2
    D = n_embd // H
    w, b, hw = _weights(rng, n_embd, Hkv * D, torch.bfloat16, fp8=True)
    x = _round(rng.standard_normal((B, n_embd)), torch.bfloat16)
    kc = _round(rng.standard_normal((B, ctx, Hkv, D)), torch.bfloat16)
    vc = _round(rng.standard_normal((B, ctx, Hkv, D)), torch.bfloat16)
    pos = rng.integers(0, 4096, B).astype(np.int64)
    blk = fm.AttentionBlockDecode(*(_dev(w[k], torch.bfloat16) for k in ("wq", "wk", "wv", "wo")), n_head=H,
                                  n_head_kv=Hkv, n_embd=n_embd, act_dtype=torch.bfloat16, weight_dtype="fp8")
    out, _, _ = blk(_dev(x, torch.bfloat16), torch.from_numpy(pos).cuda(), _dev(kc, torch.bfloat16),
                    _dev(vc, torch.bfloat16))
    ref = oa.attention_block_decode(x, pos, kc, vc, hw["wq"], hw["wk"], hw["wv"], hw["wo"], None, None, None, None,
                                    False, H, Hkv, n_embd)
    assert_close_rms(_host(out), ref[0], 5e-2)


# ------------------------------------------------------------------ paged decode
PAGED = [
    # B, n_embd, H, Hkv, block_size, n_blocks, lens, max_ctx, dtype
    (2, 64, 4, 2, 4, 16, [10, 3], 12, "f32"),            # zero rows past both contexts
    (3, 512, 4, 2, 16, 64, [300, 17, 256], 300, "f32"),  # context == max_ctx, one sequence in one split
    (4, 4096, 32, 8, 16, 512, [1000, 999, 1500, 1], 1200, "bf16"),  # one context truncated at max_ctx
]


@pytest.mark.parametrize("B,n_embd,H,Hkv,bs,n_blocks,lens,max_ctx,dt", PAGED)
def test_attention_decode_paged(fm, B, n_embd, H, Hkv, bs, n_blocks, lens, max_ctx, dt):
    rng = np.random.default_rng(n_embd + bs + B)
    tdt = DT[dt]
    D = n_embd // H
    max_blocks = (max(max(lens), max_ctx) + bs - 1) // bs + 1
    perm = rng.permutation(n_blocks)
    tables = np.zeros((2, B, max_blocks), np.int32)
    used = 0
    for bb in range(B):
        for layer in range(2):
            need = (max(lens[bb], max_ctx) + bs - 1) // bs
            tables[layer, bb, :need] = perm[(used + np.arange(need)) % n_blocks]
        used += (max(lens[bb], max_ctx) + bs - 1) // bs
    ctx_lens = np.stack([np.zeros(B, np.int32), np.array(lens, np.int32)])
    kp = _round(rng.standard_normal((n_blocks, bs, Hkv, D)), tdt)
    vp = _round(rng.standard_normal((n_blocks, bs, Hkv, D)), tdt)
    bi = np.array([tables[1, bb, min(lens[bb], max_ctx) // bs] for bb in range(B)], np.int32)
    pi = np.array([min(lens[bb], max_ctx) % bs for bb in range(B)], np.int32)
    w, b, hw = _weights(rng, n_embd, Hkv * D, tdt)
    x = _round(rng.standard_normal((B, n_embd)), tdt)
    pos = np.array(lens, np.int64)
    blk = fm.AttentionBlockDecode(*(_dev(w[k], tdt) for k in ("wq", "wk", "wv", "wo")),
                                  *(torch.from_numpy(b[k]).cuda() for k in ("bq", "bk", "bv", "bo")),
                                  use_bias=True, n_head=H, n_head_kv=Hkv, n_embd=n_embd, act_dtype=tdt)
    kd, vd = _dev(kp, tdt), _dev(vp, tdt)
    out, k_new, v_new = blk.paged(_dev(x, tdt), torch.from_numpy(pos).cuda(), kd, vd, 1, tables, ctx_lens, max_ctx,
                                  bi, pi)
    torch.cuda.synchronize()
    ref = oa.attention_decode_paged(x, pos, kp, vp, 1, tables, ctx_lens, max_ctx, bi, pi, hw["wq"], hw["wk"],
                                    hw["wv"], hw["wo"], b["bq"], b["bk"], b["bv"], b["bo"], True, H, Hkv, n_embd)
    rtol = 1e-4 if dt == "f32" else 2e-2
    what = f"paged B={B} n_embd={n_embd} {dt}"
    assert_close_rms(_host(out), ref[0], rtol, what=what)
    assert_close_rms(_host(k_new), ref[1], rtol, what=what + " k_new")
    # the pools hold exactly the returned new K/V at the written slots and are unchanged elsewhere
    kh, vh = _host(kd), _host(vd)
    np.testing.assert_array_equal(kh[bi, pi], _host(k_new))
    np.testing.assert_array_equal(vh[bi, pi], _host(v_new))
    mask = np.ones((n_blocks, bs), bool)
    mask[bi, pi] = False
    np.testing.assert_array_equal(kh[mask], kp[mask])
    np.testing.assert_array_equal(vh[mask], vp[mask])


def test_paged_equals_gather_then_block(fm):
    """The in-place paged read gives the same numbers as gather + block."""
    rng = np.random.default_rng(21)
    B, n_embd, H, Hkv, bs, n_blocks, max_ctx = 3, 256, 8, 2, 8, 40, 70
    D = n_embd // H
    tables = rng.permutation(n_blocks)[: B * 10].reshape(1, B, 10).astype(np.int32)
    lens = np.array([[70, 33, 5]], np.int32)
    kp = rng.standard_normal((n_blocks, bs, Hkv, D)).astype(np.float32)
    vp = rng.standard_normal((n_blocks, bs, Hkv, D)).astype(np.float32)
    w, b, _ = _weights(rng, n_embd, Hkv * D, torch.float32)
    blk = fm.AttentionBlockDecode(*(_dev(w[k], torch.float32) for k in ("wq", "wk", "wv", "wo")), n_head=H,
                                  n_head_kv=Hkv, n_embd=n_embd, act_dtype=torch.float32)
    x = _dev(rng.standard_normal((B, n_embd)), torch.float32)
    pos = torch.tensor([70, 33, 5], dtype=torch.int64, device="cuda")
    kd, vd = _dev(kp, torch.float32), _dev(vp, torch.float32)
    kc = fm.kvcache_gather(kd, 0, tables, lens, max_ctx)
    vc = fm.kvcache_gather(vd, 0, tables, lens, max_ctx)
    o1, k1, v1 = blk(x, pos, kc, vc)
    o2, k2, v2 = blk.paged(x, pos, kd, vd, 0, tables, lens, max_ctx, np.array([39, 38, 37], np.int32),
                           np.zeros(3, np.int32))
    torch.cuda.synchronize()
    assert torch.equal(k1, k2) and torch.equal(v1, v2)
    assert_close_rms(_host(o2), _host(o1), 1e-5)


def test_paged_scatter_after_read_duplicates_out_of_pool(fm):
    """The paged decode's scatter of the new K/V (written by the combine
    launch) on 130 sequences: a slot named twice keeps the later row, slots
    outside the pool are skipped, and slots inside a sequence's own context
    are written only after the attention has read them (gather-then-scatter
    order of transformer_layer_moe_decode.mlir:180-206)."""
    rng = np.random.default_rng(31)
    B, n_embd, H, Hkv, bs, n_blocks, max_ctx = 130, 64, 4, 2, 4, 80, 16
    D = n_embd // H
    tables = rng.integers(0, n_blocks, (1, B, 5)).astype(np.int32)
    lens = rng.integers(1, 21, (1, B)).astype(np.int32)
    kp = rng.standard_normal((n_blocks, bs, Hkv, D)).astype(np.float32)
    vp = rng.standard_normal((n_blocks, bs, Hkv, D)).astype(np.float32)
    bi = rng.integers(0, n_blocks, B).astype(np.int32)
    pi = rng.integers(0, bs, B).astype(np.int32)
    bi[129], pi[129] = bi[0], pi[0]        # a duplicate slot: row 129 wins
    bi[64], pi[64] = bi[3], pi[3]          # and one where the earlier row is 3
    bi[5], bi[6], pi[7] = n_blocks, -1, bs  # outside the pool: skipped
    bi[8], pi[8] = tables[0, 8, 0], 0      # inside sequence 8's own context
    w, b, hw = _weights(rng, n_embd, Hkv * D, torch.float32)
    blk = fm.AttentionBlockDecode(*(_dev(w[k], torch.float32) for k in ("wq", "wk", "wv", "wo")), n_head=H,
                                  n_head_kv=Hkv, n_embd=n_embd, act_dtype=torch.float32)
    x = rng.standard_normal((B, n_embd)).astype(np.float32)
    pos = lens[0].astype(np.int64)
    kd, vd = _dev(kp, torch.float32), _dev(vp, torch.float32)
    out, k_new, v_new = blk.paged(_dev(x, torch.float32), torch.from_numpy(pos).cuda(), kd, vd, 0, tables, lens,
                                  max_ctx, bi, pi)
    torch.cuda.synchronize()
    kc = oa.kv_gather(kp, 0, tables, lens, max_ctx)
    vc = oa.kv_gather(vp, 0, tables, lens, max_ctx)
    ref = oa.attention_block_decode(x, pos, kc, vc, hw["wq"], hw["wk"], hw["wv"], hw["wo"], None, None, None, None,
                                    False, H, Hkv, n_embd)
    assert_close_rms(_host(out), ref[0], 1e-4, what="paged B=130 output (pools read before the scatter)")
    ok = (bi >= 0) & (bi < n_blocks) & (pi >= 0) & (pi < bs)
    assert ok.sum() == B - 3
    for pool, new, name in ((kp, k_new, "K"), (vp, v_new, "V")):
        want = oa.kv_scatter_decode(pool, _host(new)[ok], bi[ok], pi[ok])
        np.testing.assert_array_equal(_host(kd if name == "K" else vd), want, err_msg=f"{name} pool")


@pytest.mark.parametrize("dt,B", [("f32", 3), ("bf16", 3), ("bf16", 40)])
def test_attention_sublayer_decode_paged(fm, dt, B):
    """attn_norm + paged attention + residual add in one call; in place
    (out=residual) equals out of place bit for bit.  bf16 at 3 rows runs
    bias + RoPE and bias + residual in the projections' epilogues; at 40
    rows RoPE runs as its own launch over a K-split Q/K/V product."""
    rng = np.random.default_rng(31 + B)
    tdt = DT[dt]
    n_embd, H, Hkv, bs, max_ctx = 256, 8, 2, 16, 100
    n_blocks = max(40, B * 8)
    D = n_embd // H
    tables = rng.permutation(n_blocks)[: B * 8].reshape(1, B, 8).astype(np.int32)
    lens = np.array([[100, 37, 64]], np.int32) if B == 3 else rng.integers(1, 101, (1, B)).astype(np.int32)
    kp = _round(rng.standard_normal((n_blocks, bs, Hkv, D)), tdt)
    vp = _round(rng.standard_normal((n_blocks, bs, Hkv, D)), tdt)
    bi = np.array([tables[0, b, 7] for b in range(B)], np.int32)
    pi = np.full(B, 15, np.int32)
    w, b, hw = _weights(rng, n_embd, Hkv * D, tdt)
    res = _round(rng.standard_normal((B, n_embd)), tdt)
    nw = _round(rng.standard_normal(n_embd) * 0.5 + 1.0, tdt)
    pos = lens[0].astype(np.int64)
    blk = fm.AttentionBlockDecode(*(_dev(w[k], tdt) for k in ("wq", "wk", "wv", "wo")),
                                  *(torch.from_numpy(b[k]).cuda() for k in ("bq", "bk", "bv", "bo")),
                                  use_bias=True, n_head=H, n_head_kv=Hkv, n_embd=n_embd, act_dtype=tdt)
    kd, vd = _dev(kp, tdt), _dev(vp, tdt)
    r = _dev(res, tdt)
    out, k_new, _ = blk.paged_sublayer(r, _dev(nw, tdt), 1e-5, torch.from_numpy(pos).cuda(), kd, vd, 0, tables,
                                       lens, max_ctx, bi, pi)
    torch.cuda.synchronize()
    ref = oa.attention_sublayer_decode_paged(res, nw, 1e-5, pos, kp, vp, 0, tables, lens, max_ctx, bi, pi, hw["wq"],
                                             hw["wk"], hw["wv"], hw["wo"], b["bq"], b["bk"], b["bv"], b["bo"], True, H,
                                             Hkv, n_embd)
    rtol = 1e-4 if dt == "f32" else 2e-2
    assert_close_rms(_host(out), ref[0], rtol, what=f"sub-layer {dt}")
    if dt == "f32":
        # the attention part on its own (a bf16 sum's rounding is relative to
        # the residual, so this is checked in fp32 only)
        assert_close_rms(_host(out) - res, ref[0] - res, rtol, what="sub-layer attention part")
    # in place on the same pools (pools restored first: the call wrote the new K/V)
    kd2, vd2 = _dev(kp, tdt), _dev(vp, tdt)
    r2 = _dev(res, tdt)
    out2, _, _ = blk.paged_sublayer(r2, _dev(nw, tdt), 1e-5, torch.from_numpy(pos).cuda(), kd2, vd2, 0, tables, lens,
                                    max_ctx, bi, pi, out=r2)
    torch.cuda.synchronize()
    assert out2.data_ptr() == r2.data_ptr()
    assert torch.equal(out2, out)


# Shapes for the projections' LDS-ring kernel: the Mixtral attention shape,
# and small input axes whose four K quarters are short (n_embd 544: 17 input
# steps, quarters of 4, 4, 4 and 5 steps, each below the 8-step ring) or
# single steps (n_embd 160: 5 steps).
RING = [
    # B, n_embd, H, Hkv
    (16, 4096, 32, 8),
    (1, 4096, 32, 8),
    (7, 544, 17, 17),
    (3, 160, 5, 5),
]


@pytest.mark.parametrize("B,n_embd,H,Hkv", RING)
def test_projection_ring_matches_register_stream(fm, gemm_path, B, n_embd, H, Hkv):
    """Up to 16 rows, bf16 weights: the automatic choice runs the Q/K/V and
    output projections on the LDS-ring streaming kernel with bias + RoPE and
    bias + residual in its epilogue; the forced streaming path runs the same
    products on the register-staged streaming kernel (fp32 out) with the
    bias, RoPE and residual in separate launches.  Same K quarters, MFMA
    chains and epilogue arithmetic: equal bit for bit, out of place (block)
    and with the residual (sub-layer)."""
    rng = np.random.default_rng(B * 1000 + n_embd)
    tdt = torch.bfloat16
    D = n_embd // H
    bs, max_ctx = 16, 40
    n_blocks = B * 4 + 4
    tables = rng.permutation(n_blocks)[: B * 4].reshape(1, B, 4).astype(np.int32)
    lens = rng.integers(1, max_ctx + 1, (1, B)).astype(np.int32)
    kp = _round(rng.standard_normal((n_blocks, bs, Hkv, D)), tdt)
    vp = _round(rng.standard_normal((n_blocks, bs, Hkv, D)), tdt)
    bi = np.array([tables[0, b, 3] for b in range(B)], np.int32)
    pi = np.full(B, 15, np.int32)
    w, b, _ = _weights(rng, n_embd, Hkv * D, tdt)
    x = _round(rng.standard_normal((B, n_embd)), tdt)
    nw = _round(rng.standard_normal(n_embd) * 0.5 + 1.0, tdt)
    pos = torch.from_numpy(lens[0].astype(np.int64)).cuda()
    blk = fm.AttentionBlockDecode(*(_dev(w[k], tdt) for k in ("wq", "wk", "wv", "wo")),
                                  *(torch.from_numpy(b[k]).cuda() for k in ("bq", "bk", "bv", "bo")),
                                  use_bias=True, n_head=H, n_head_kv=Hkv, n_embd=n_embd, act_dtype=tdt)
    ll = gemm_path
    got = {}
    for path in (ll.PATH_AUTO, ll.PATH_STREAM):
        ll.check(ll.lib().fmoe_set_gemm_path(path))
        kd, vd = _dev(kp, tdt), _dev(vp, tdt)
        o = blk.paged(_dev(x, tdt), pos, kd, vd, 0, tables, lens, max_ctx, bi, pi)
        kd2, vd2 = _dev(kp, tdt), _dev(vp, tdt)
        s = blk.paged_sublayer(_dev(x, tdt), _dev(nw, tdt), 1e-5, pos, kd2, vd2, 0, tables, lens, max_ctx, bi, pi)
        torch.cuda.synchronize()
        got[path] = [t.view(torch.int16).cpu().numpy() for t in (*o, *s, kd, vd)]
    for name, a, c in zip(("out", "k_new", "v_new", "sub out", "sub k_new", "sub v_new", "k pool", "v pool"),
                          got[ll.PATH_AUTO], got[ll.PATH_STREAM]):
        np.testing.assert_array_equal(a, c, err_msg=f"B={B} n_embd={n_embd}: {name}")
