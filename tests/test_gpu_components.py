"""GPU parity of the path's components against the oracle: router (ids
bit-exact), permutation (bit-exact), SwiGLU, packing (bf16 / fp8 bits),
and the reference's own mul_mat_id / moe_ffn_block test cases at the
reference's tolerance (rtol 1e-4, atol 1e-5)."""

import numpy as np
import pytest
import torch

import oracle
from oracle import moe as om
from oracle import numerics as nm
from helpers import assert_close, packed_index
from test_oracle import (BLOCK_REFERENCE_CASES, MMID_REFERENCE_CASES, REFERENCE_IDS, _mmid_case, block_inputs,
                         ulp_tie_router_inputs)

pytestmark = pytest.mark.gpu


def test_device_is_gfx950(fm):
    import ctypes

    d = ctypes.c_int(-1)
    buf = ctypes.create_string_buffer(64)
    fm.lowlevel.check(fm.lowlevel.lib().fmoe_device_check(ctypes.byref(d), buf, 64))
    assert buf.value.decode().startswith("gfx950")
    assert len(fm.hip_runtimes_loaded()) == 1, fm.hip_runtimes_loaded()


# ------------------------------------------------------------------ swiglu
@pytest.mark.parametrize("seed,scale,kind", [(42, 1, "rand"), (0, 0, "zeros"), (123, 1, "pos"), (456, 10, "rand")])
def test_swiglu_reference_cases(fm, seed, scale, kind):
    """tests/components/test_swiglu.py:15-59."""
    if kind == "zeros":
        g = np.zeros((2, 4, 8), np.float32)
        u = np.zeros((2, 4, 8), np.float32)
    else:
        np.random.seed(seed)
        g = np.random.randn(2, 4, 8).astype(np.float32) * scale
        u = np.random.randn(2, 4, 8).astype(np.float32) * scale
        if kind == "pos":
            g, u = np.abs(g) + 0.1, np.abs(u) + 0.1
    out = fm.swiglu(g, u)
    tol = dict(rtol=1e-4, atol=1e-5) if scale == 10 else dict(rtol=1e-5, atol=1e-6)
    assert_close(out, oracle.swiglu(g.astype(np.float64), u.astype(np.float64)), **tol)


def test_swiglu_bf16(fm):
    rng = np.random.default_rng(1)
    g = torch.from_numpy(rng.standard_normal(10000).astype(np.float32)).to("cuda", torch.bfloat16)
    u = torch.from_numpy(rng.standard_normal(10000).astype(np.float32) * 3).to("cuda", torch.bfloat16)
    out = fm.swiglu(g, u).float().cpu().numpy()
    ref = oracle.swiglu(g.float().cpu().numpy().astype(np.float64), u.float().cpu().numpy().astype(np.float64))
    np.testing.assert_allclose(out, ref, rtol=2**-8, atol=1e-6)


# ------------------------------------------------------------------ router
def _router_check(fm, x, wr, k, norm, rtol_w=1e-5):
    ids, w = fm.router(x, wr, k, norm)
    rids, rw = om.router(x, wr, k, norm)
    np.testing.assert_array_equal(ids, rids)
    np.testing.assert_allclose(w, rw, rtol=rtol_w, atol=1e-7)


@pytest.mark.parametrize("path", ["tiled", "tiled_large", "stream", "auto"])
@pytest.mark.parametrize("n_out,n_in,k,T", [(304, 512, 2, 300), (256, 256, 4, 700), (208, 96, 2, 40),
                                            (208, 96, 2, 5)])
def test_mul_mat_id_bf16_paths(fm, path, n_out, n_in, k, T):
    """bf16 mul_mat_id (plain scatter epilogue, bf16 output) on each MFMA
    path vs the oracle on the same bf16 values: rtol 2e-2 of the output's RMS.
    300 and 700 tokens over 8 experts give partial row tiles and (n_out 304)
    a partial column tile; n_out 208 (13 blocks of 16 rows) with a 96-input
    axis leaves the streaming kernel's last block of column tiles part-full."""
    ll = fm.lowlevel
    rng = np.random.default_rng(n_out + T)
    w = torch.from_numpy((rng.standard_normal((n_out, n_in, 8)) * 0.05).astype(np.float32)).bfloat16()
    x = torch.from_numpy(rng.standard_normal((n_in, k, T)).astype(np.float32)).bfloat16()
    ids = np.stack([rng.permutation(8)[:k] for _ in range(T)], axis=1).astype(np.int32)
    code = {"tiled": ll.PATH_TILED, "tiled_large": ll.PATH_TILED_LARGE, "stream": ll.PATH_STREAM,
            "auto": ll.PATH_AUTO}[path]
    ll.check(ll.lib().fmoe_set_gemm_path(code))
    try:
        out = fm.mul_mat_id(w.cuda(), x.cuda(), torch.from_numpy(ids).cuda())
        torch.cuda.synchronize()
    finally:
        ll.lib().fmoe_set_gemm_path(ll.PATH_AUTO)
    assert out.shape == (n_out, k, T) and out.dtype == torch.bfloat16
    ref = om.mul_mat_id(w.float().numpy(), x.float().numpy(), ids)
    from helpers import assert_close_rms

    assert_close_rms(out.float().cpu().numpy(), ref, 2e-2, what=f"{path} {n_out}x{n_in} k={k} T={T}")


@pytest.mark.parametrize("case", range(len(BLOCK_REFERENCE_CASES)))
def test_router_reference_cases(fm, case):
    seed, T, H, F, E, k, norm = BLOCK_REFERENCE_CASES[case]
    x, wr, *_ = block_inputs(seed, T, H, F, E)
    _router_check(fm, x, wr, k, norm)


@pytest.mark.parametrize("cfg_name,T", [("C1", 32), ("C2", 16), ("C2", 512), ("C3", 64), ("C3", 2048),
                                        ("C4", 1), ("C4", 64)])
def test_router_configs(fm, wl, cfg_name, T):
    cfg = wl.CONFIGS[cfg_name]
    x, wr, _ = wl.router_inputs(cfg, T)
    if cfg.act == "bf16":
        xt = torch.from_numpy(x).to("cuda", torch.bfloat16)
        wt = torch.from_numpy(wr).to("cuda", torch.bfloat16)
        ids, w = fm.router(xt, wt, cfg.n_expert_used, cfg.normalize)
        ids, w = ids.cpu().numpy(), w.cpu().numpy()
        rids, rw = om.router(x, wr, cfg.n_expert_used, cfg.normalize)
        np.testing.assert_array_equal(ids, rids)
        np.testing.assert_allclose(w, rw, rtol=1e-5, atol=1e-7)
    else:
        _router_check(fm, x, wr, cfg.n_expert_used, cfg.normalize)


# Large batches with 33..256 experts and uneven expert counts (33, 40, 80,
# 200 leave MFMA columns partly unused; above 128 experts the SIMT kernel
# runs).  k <= 16 takes the four-tokens-per-wave top-k.
@pytest.mark.parametrize("E,k,H,T", [(128, 8, 2048, 8192), (64, 6, 2048, 512), (80, 4, 256, 300),
                                     (40, 2, 128, 256), (33, 1, 64, 1000), (256, 8, 512, 512),
                                     (200, 6, 320, 700), (160, 4, 192, 256), (128, 8, 2048, 255)])
def test_router_wide(fm, wl, E, k, H, T):
    cfg = wl.Config("R", H, 64, E, k, (T,), "bf16", "bf16", True, 1e-4, seed=E)
    x, wr, _ = wl.router_inputs(cfg, T)
    xt = torch.from_numpy(x).to("cuda", torch.bfloat16)
    wt = torch.from_numpy(wr).to("cuda", torch.bfloat16)
    ids, w = fm.router(xt, wt, k, True)
    rids, rw = om.router(x, wr, k, True)
    np.testing.assert_array_equal(ids.cpu().numpy(), rids)
    np.testing.assert_allclose(w.cpu().numpy(), rw, rtol=1e-5, atol=1e-7)


# H = 64 takes the 16-token MFMA kernel, H = 128 the 32-token tile kernel.
@pytest.mark.parametrize("H", [64, 128])
def test_router_wide_ties_lower_index(fm, H):
    # one-hot rows over a large batch: token t's logits are router column
    # t % 3, exactly
    E, T = 48, 300
    wr = np.zeros((E, H), np.float32)
    wr[[7, 20, 33], 0] = 5.0   # three-way tie at the top
    wr[[41, 40], 2] = 1.0      # two-way tie; column 1 is all equal
    x = np.zeros((T, H), np.float32)
    x[np.arange(T), np.arange(T) % 3] = 1.0
    ids, _ = fm.router(torch.from_numpy(x).to("cuda", torch.bfloat16), torch.from_numpy(wr).to("cuda", torch.bfloat16),
                       2, False)
    want = {0: [7, 20], 1: [0, 1], 2: [40, 41]}
    got = ids.cpu().numpy()
    for t in range(T):
        assert list(got[:, t]) == want[t % 3], t


def test_router_ties_lower_index(fm):
    # identity inputs make the logits equal to the router columns exactly
    logits = np.array([[1.0, 0.0, 5.0], [2.0, 0.0, 5.0], [2.0, 0.0, 5.0], [0.0, 0.0, 5.0]], np.float32)
    x = np.eye(3, dtype=np.float32)
    for dt in (torch.float32, torch.bfloat16):
        # H = 3 (SIMT path) and a padded H = 128 (MFMA path for bf16)
        for H in (3, 128):
            xx = np.zeros((3, H), np.float32)
            xx[:, :3] = x
            wr = np.zeros((4, H), np.float32)
            wr[:, :3] = logits
            ids, w = fm.router(torch.from_numpy(xx).to("cuda", dt), torch.from_numpy(wr).to("cuda", dt), 2, False)
            np.testing.assert_array_equal(ids.cpu().numpy(), [[1, 0, 0], [2, 1, 1]])


# Logits one ulp apart have one fp32 probability: the selection runs on the
# probabilities (lower expert index first), on every kernel fmoe_router runs:
# the SIMT kernel (fp32), the MFMA kernels (bf16: 16 tokens per block, or 32
# for 33..128 experts with n_embd % 128 == 0), and the one-token-per-wave
# top-k (k > 16).  The block's own routers are covered below.
@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("T", [1, 16, 100])
@pytest.mark.parametrize("E,k,H", [(8, 3, 64), (40, 18, 64), (40, 3, 128), (128, 8, 256)])
def test_router_ulp_apart_logits(fm, dt, T, E, k, H):
    x, wr = ulp_tie_router_inputs(E, H, T)
    want, want_w = om.router(x, wr, k, False, dtype=np.float32)
    assert list(want[:3, 0]) == [2, 5, 0]
    for norm in (False, True):
        ids, w = fm.router(torch.from_numpy(x).to("cuda", dt), torch.from_numpy(wr).to("cuda", dt), k, norm)
        ids, w = ids.cpu().numpy(), w.cpu().numpy()
        np.testing.assert_array_equal(ids, want)
        assert np.array_equal(w[0], w[1])  # the tied pair has one weight


# The same ties through the block, whose routing runs other kernels: the
# decode split-logits router (bf16, T <= 64) with its one-wave finish (up to
# 4 tokens), its one-block finish, and its top-k over blocks (above 64
# experts and 32 tokens); and the split prefill router (33..128 experts,
# n_embd % 128 == 0, T > 64), which sums partial logits over hidden-axis
# ranges.
@pytest.mark.parametrize("E,k,H,T", [(128, 8, 256, 1), (128, 8, 256, 3), (64, 6, 256, 16), (128, 8, 256, 40),
                                     (40, 3, 128, 100)])
def test_block_router_ulp_apart_logits(fm, wl, E, k, H, T):
    F = 64
    cfg = wl.scaled(wl.CONFIGS["C3"], H, F, n_expert=E, n_expert_used=k)
    x, wr = ulp_tie_router_inputs(E, H, T)
    want, _ = om.router(x, wr, k, False, dtype=np.float32)
    up, gate, down = wl.expert_weights(cfg, "cuda", dtype=torch.bfloat16)
    packed = [fm.pack_expert_weights(w) for w in (up, gate, down)]
    for norm in (False, True):
        blk = fm.MoEFFNBlock(torch.from_numpy(wr).to("cuda", torch.bfloat16), *packed, E, k, H, F, norm,
                             act_dtype=torch.bfloat16)
        blk(torch.from_numpy(x).to("cuda", torch.bfloat16))
        torch.cuda.synchronize()
        ids, w, _, _ = blk.routing(T)
        np.testing.assert_array_equal(ids.cpu().numpy(), want, err_msg=f"normalize={norm}")
        w = w.cpu().numpy()
        assert np.array_equal(w[0], w[1])  # the tied pair has one weight


def test_router_many_experts_and_k(fm):
    # N(0,1) router weights give logits of std ~sqrt(H); their fp32
    # accumulation error (~1e-5 absolute) is a relative error of the
    # probabilities, so the weights are held to the reference's fp32 rtol 1e-4.
    rng = np.random.default_rng(11)
    for E, k, H in [(256, 8, 64), (128, 64, 128), (3, 3, 5)]:
        x = rng.standard_normal((37, H)).astype(np.float32)
        wr = rng.standard_normal((E, H)).astype(np.float32)
        _router_check(fm, x, wr, k, True, rtol_w=1e-4)


# ------------------------------------------------------------------ permutation
@pytest.mark.parametrize("case", range(len(REFERENCE_IDS)))
def test_permute_reference_ids(fm, case):
    ids, E = REFERENCE_IDS[case]
    order, offsets = fm.permute(ids, E)
    ro, roff = om.permute(ids, E)
    np.testing.assert_array_equal(order, ro)
    np.testing.assert_array_equal(offsets, roff)


# Batches above 2048 assignments take the chunked two-kernel path; 2048 and
# 2049 sit on either side of the switch.
@pytest.mark.parametrize("E,k,T,skew", [(8, 2, 4096, 0), (128, 8, 8192, 1.1), (64, 6, 64, 0),
                                        (8, 2, 1, 0), (512, 1, 3000, 0), (4, 4, 1500, 0), (2, 1, 70000, 0),
                                        (4, 1, 2048, 0), (4, 1, 2049, 0), (16, 2, 1025, 0)])
def test_permute_random(fm, E, k, T, skew):
    rng = np.random.default_rng(E * 7 + k + T)
    if skew:
        p = 1.0 / np.arange(1, E + 1) ** skew
        p /= p.sum()
        ids = np.stack([rng.choice(E, size=k, replace=False, p=p) for _ in range(T)], axis=1)
    elif k <= E:
        ids = np.argsort(rng.random((E, T)), axis=0)[:k]
    ids = ids.astype(np.int32)
    order, offsets = fm.permute(ids, E)
    ro, roff = om.permute(ids, E)
    np.testing.assert_array_equal(offsets, roff)
    np.testing.assert_array_equal(order, ro)


def test_permute_all_one_expert_and_empty(fm):
    ids = np.full((2, 3000), 5, np.int32)
    order, offsets = fm.permute(ids, 8)
    ro, roff = om.permute(ids, 8)
    np.testing.assert_array_equal(order, ro)
    np.testing.assert_array_equal(offsets, roff)
    order, offsets = fm.permute(np.zeros((2, 0), np.int32), 8)
    assert order.size == 0 and np.all(offsets == 0)


def test_permute_device_ids_out_of_range(fm):
    ids = torch.tensor([[0, 9, 1], [2, -1, 3]], dtype=torch.int32, device="cuda")
    with pytest.raises(IndexError):
        fm.permute(ids, 8)
    # chunked path: invalid ids in two different chunks are counted, the valid
    # ones still grouped stably
    ll = fm.lowlevel
    host = np.random.default_rng(5).integers(0, 8, (2, 3000)).astype(np.int32)
    host[0, 10] = 8
    host[1, 2900] = -3
    host[1, 100] = 513  # one past the largest expert count any kernel takes
    d = torch.from_numpy(host).cuda()
    with pytest.raises(IndexError, match="3 expert id"):
        fm.permute(d, 8)
    order = torch.empty(6000, dtype=torch.int32, device="cuda")
    offsets = torch.empty(9, dtype=torch.int32, device="cuda")
    ws = torch.empty(ll.lib().fmoe_permute_workspace_bytes(2, 3000, 8), dtype=torch.uint8, device="cuda")
    ll.call("fmoe_permute", d.data_ptr(), 2, 3000, 8, order.data_ptr(), offsets.data_ptr(), ws.data_ptr(),
            ws.numel(), torch.cuda.current_stream().cuda_stream)
    flat = host.reshape(-1)
    valid = np.nonzero((flat >= 0) & (flat < 8))[0]
    ref = valid[np.argsort(flat[valid], kind="stable")]
    off = offsets.cpu().numpy()
    assert off[-1] == valid.size
    np.testing.assert_array_equal(order.cpu().numpy()[: valid.size], ref)


# ------------------------------------------------------------------ packing
def _unpack(buf, shape, dt):
    """Packed buffer -> [E, n_out, n_in] through the documented layout."""
    n_out, n_in, E = shape
    idx = packed_index(n_out, n_in, E, dt)
    return buf[idx]


@pytest.mark.parametrize("shape", [(24, 40, 5), (32, 64, 3), (48, 96, 2)])
def test_pack_bf16_bits(fm, shape):
    rng = np.random.default_rng(12)
    w = (rng.standard_normal(shape) * 0.02).astype(np.float32)
    p = fm.pack_expert_weights(w, "bf16")
    buf = p.data.view(torch.int16).cpu().numpy().view(np.uint16)
    np.testing.assert_array_equal(_unpack(buf, shape, "bf16"), nm.bf16_bits(w).transpose(2, 0, 1))


@pytest.mark.parametrize("shape", [(24, 40, 5), (32, 128, 3), (16, 64, 2)])
def test_pack_fp8_codes_and_scales(fm, shape):
    rng = np.random.default_rng(13)
    w = (rng.standard_normal(shape) * 0.02).astype(np.float32)
    w[3, :, 1] = 0.0
    w[4, 7, 1] = 1e-9  # subnormal after scaling
    p = fm.quantize_expert_weights(w)
    q, s = nm.quantize_per_channel_e4m3fn(w)
    np.testing.assert_array_equal(_unpack(p.data.cpu().numpy(), shape, "fp8"), q.transpose(2, 0, 1))
    np.testing.assert_array_equal(p.scales.cpu().numpy(), s.T)


def test_pack_prequantized(fm):
    rng = np.random.default_rng(14)
    shape = (32, 64, 3)
    w = (rng.standard_normal(shape) * 0.02).astype(np.float32)
    q, s = nm.quantize_per_channel_e4m3fn(w)
    p = fm.pack_expert_weights(fm.QuantizedExpertWeights(q, s))
    np.testing.assert_array_equal(_unpack(p.data.cpu().numpy(), shape, "fp8"), q.transpose(2, 0, 1))
    np.testing.assert_array_equal(p.scales.cpu().numpy(), s.T)


# ------------------------------------------------------------------ reference cases, fp32
@pytest.mark.parametrize("case", range(len(MMID_REFERENCE_CASES)))
def test_mul_mat_id_reference_cases(fm, case):
    """tests/components/test_mul_mat_id.py, same seeds/shapes/tolerance."""
    w, x, ids = _mmid_case(*MMID_REFERENCE_CASES[case])
    out = fm.mul_mat_id(w, x, ids)
    assert out.shape == (w.shape[0], *ids.shape) and out.dtype == np.float32
    assert_close(out, om.mul_mat_id_literal(w, x, ids), rtol=1e-4, atol=1e-5)
    assert_close(out, om.mul_mat_id(w, x, ids), rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("case", range(len(BLOCK_REFERENCE_CASES)))
def test_moe_ffn_block_reference_cases(fm, case):
    """tests/components/test_moe_ffn_block.py, same seeds/shapes/tolerance."""
    seed, T, H, F, E, k, norm = BLOCK_REFERENCE_CASES[case]
    x, wr, up, gate, down = block_inputs(seed, T, H, F, E)
    out = fm.moe_ffn_block(x, wr, up, gate, down, E, k, H, F, norm)
    assert out.shape == (T, H) and out.dtype == np.float32
    assert_close(out, om.moe_ffn_block_literal(x, wr, up, gate, down, E, k, H, F, norm), rtol=1e-4, atol=1e-5)


# ------------------------------------------------------------------ e4m3 row quantiser
def _unblock_e4m3(q, n_rows, n_cols):
    """K-blocked 64-input pieces (chunk g: inputs 8g..8g+7, 32+8g..32+8g+7)
    -> [n_rows, n_cols] codes in input order."""
    q = q.reshape(n_cols // 64, n_rows, 4, 2, 8)  # piece, row, chunk g, half, byte
    out = np.empty((n_rows, n_cols // 64, 2, 4, 8), np.uint8)  # row, piece, half, g, byte
    out[:] = q.transpose(1, 0, 3, 2, 4)
    return out.reshape(n_rows, n_cols)


def _quantizer_rows():
    """bf16 rows whose scaled values hit every e4m3 value, every midpoint
    between neighbours (the round-to-nearest-even ties), one bf16 ulp either
    side of each midpoint, and the subnormal range, at several row scales and
    both signs; then random rows of mixed magnitudes and an all-zero row."""
    vals = nm.E4M3FN_VALUES[:127].astype(np.float64)
    mids = (vals[:-1] + vals[1:]) / 2
    b = lambda a: nm.bf16_round(np.asarray(a, np.float32))
    pts = np.concatenate([vals, mids, b(mids) * (1 + 2.0**-7), b(mids) * (1 - 2.0**-8), np.linspace(0, 2.0**-6, 40)])
    pts = b(pts)
    n_cols = 512
    rows = []
    for s in (-20, -3, 0, 5):
        for sign in (1.0, -1.0):
            for off in range(0, len(pts), n_cols - 1):
                r = np.zeros(n_cols, np.float32)
                chunk = pts[off:off + n_cols - 1]
                r[0] = 448.0  # fixes the row scale at 2^s
                r[1:1 + len(chunk)] = sign * chunk
                rows.append(b(r * np.float32(2.0**s)))
    rng = np.random.default_rng(21)
    for _ in range(40):
        rows.append(b(rng.standard_normal(n_cols) * 10.0 ** rng.uniform(-6, 4)))
    rows.append(np.zeros(n_cols, np.float32))
    return np.stack(rows).astype(np.float32)


@pytest.mark.parametrize("two_terms", [False, True])
def test_row_quantizer_codes_match_the_oracle(fm, two_terms):
    a = _quantizer_rows()
    n_rows, n_cols = a.shape
    src = torch.from_numpy(a).to("cuda", torch.bfloat16)
    hi = torch.zeros(n_rows * n_cols, dtype=torch.uint8, device="cuda")
    lo = torch.zeros_like(hi)
    sc = torch.zeros(n_rows, dtype=torch.float32, device="cuda")
    ll = fm.lowlevel
    ll.check(ll.lib().fmoe_quantize_rows_e4m3(src.data_ptr(), n_rows, n_cols, hi.data_ptr(),
                                              lo.data_ptr() if two_terms else None, sc.data_ptr(),
                                              torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    rh, rl, rs = nm.quantize_rows_e4m3fn_x2(src.float().cpu().numpy())
    np.testing.assert_array_equal(sc.cpu().numpy(), rs)
    np.testing.assert_array_equal(_unblock_e4m3(hi.cpu().numpy(), n_rows, n_cols), rh)
    if two_terms:
        np.testing.assert_array_equal(_unblock_e4m3(lo.cpu().numpy(), n_rows, n_cols), rl)
    else:
        assert not lo.any()
