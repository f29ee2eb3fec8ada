"""Pins of the attention-half oracle (oracle/attention.py) against closed
forms, invariants, brute-force loops and hand-built known answers.  Each
check is chosen so that a plausible slip (pairing dims (i, i + D/2) instead
of (2i, 2i+1), a KV head mapping of h % n_head_kv instead of h // r, a
missing scale, a gather that forgets the zero fill, a scatter that lets the
first duplicate win) fails one of them."""

import math

import numpy as np
import pytest

from oracle import attention as oa


# ------------------------------------------------------------------ rope
def test_rope_position_zero_is_identity():
    x = np.random.default_rng(0).standard_normal((2, 3, 4, 16))
    np.testing.assert_array_equal(oa.rope(x, np.zeros((2, 3), np.int64)), x)


def test_rope_known_answer_adjacent_pairs():
    # D = 4: pair 0 = dims (0, 1) at freq 1, pair 1 = dims (2, 3) at freq 1/base^(2/4)
    x = np.array([1.0, 0.0, 0.0, 1.0]).reshape(1, 1, 1, 4)
    base, pos = 100.0, 3
    out = oa.rope(x, np.array([[pos]]), base, 1.0).reshape(4)
    a0, a1 = pos * 1.0, pos / base ** 0.5
    want = [math.cos(a0), math.sin(a0), -math.sin(a1), math.cos(a1)]
    np.testing.assert_allclose(out, want, rtol=0, atol=1e-15)


def test_rope_angles_add_and_norms_are_kept():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((1, 1, 2, 32))
    p1, p2 = 17, 250
    twice = oa.rope(oa.rope(x, np.array([[p1]]), 500.0, 0.5), np.array([[p2]]), 500.0, 0.5)
    once = oa.rope(x, np.array([[p1 + p2]]), 500.0, 0.5)
    np.testing.assert_allclose(twice, once, rtol=0, atol=1e-12)
    pair_norm = lambda a: np.hypot(a[..., 0::2], a[..., 1::2])
    np.testing.assert_allclose(pair_norm(once), pair_norm(x), rtol=1e-13)


def test_rope_freq_scale_scales_the_angle():
    x = np.random.default_rng(2).standard_normal((1, 1, 1, 8))
    np.testing.assert_allclose(oa.rope(x, np.array([[10]]), 10000.0, 0.5), oa.rope(x, np.array([[5]]), 10000.0, 1.0),
                               atol=1e-14)


# ------------------------------------------------------------------ attention_gqa
def _attention_loops(q, k, v, scale):
    B, Sq, H, D = q.shape
    Skv, Hkv = k.shape[1], k.shape[2]
    r = H // Hkv
    out = np.zeros_like(q)
    for b in range(B):
        for h in range(H):
            kh = h // r
            for i in range(Sq):
                s = [scale * sum(q[b, i, h, d] * k[b, j, kh, d] for d in range(D)) for j in range(Skv)]
                m = max(s)
                e = [math.exp(x - m) for x in s]
                z = sum(e)
                for d in range(D):
                    out[b, i, h, d] = sum(e[j] / z * v[b, j, kh, d] for j in range(Skv))
    return out


@pytest.mark.parametrize("H,Hkv", [(4, 4), (4, 2), (6, 1), (8, 2)])
def test_attention_gqa_matches_loops(H, Hkv):
    rng = np.random.default_rng(H * 10 + Hkv)
    q = rng.standard_normal((2, 3, H, 4))
    k = rng.standard_normal((2, 5, Hkv, 4))
    v = rng.standard_normal((2, 5, Hkv, 4))
    np.testing.assert_allclose(oa.attention_gqa(q, k, v, 0.7), _attention_loops(q, k, v, 0.7), rtol=1e-12)


def test_attention_single_key_returns_its_value():
    rng = np.random.default_rng(3)
    q = rng.standard_normal((1, 1, 4, 8))
    k = rng.standard_normal((1, 1, 2, 8))
    v = rng.standard_normal((1, 1, 2, 8))
    out = oa.attention_gqa(q, k, v, 0.25)
    # heads 0, 1 read KV head 0; heads 2, 3 read KV head 1 ([h0, h0, h1, h1])
    np.testing.assert_allclose(out[0, 0], v[0, 0, [0, 0, 1, 1]], rtol=1e-15)


def test_attention_equal_scores_average_the_values():
    v = np.random.default_rng(4).standard_normal((1, 7, 1, 4))
    out = oa.attention_gqa(np.zeros((1, 1, 1, 4)), np.ones((1, 7, 1, 4)), v, 1.0)
    np.testing.assert_allclose(out[0, 0, 0], v[0, :, 0].mean(axis=0), rtol=1e-14)


# ------------------------------------------------------------------ paged cache
def _pool(rng, n_blocks, bs, hkv, d):
    return rng.standard_normal((n_blocks, bs, hkv, d)).astype(np.float32)


def test_gather_known_tables():
    # the layout of the reference's TestGather.test_basic
    # (tests/components/test_kvcache.py:78-100): seq 0 -> blocks 0,1,2, seq 1 -> 3,4,5
    rng = np.random.default_rng(42)
    cache = _pool(rng, 8, 4, 2, 8)
    tables = np.array([[[0, 1, 2, 0], [3, 4, 5, 0]], [[0, 1, 2, 0], [3, 4, 5, 0]]], np.int32)
    lens = np.array([[10, 8], [10, 8]], np.int32)
    out = oa.kv_gather(cache, 0, tables, lens, 12)
    assert out.shape == (2, 12, 2, 8)
    for b, (blocks, n) in enumerate((([0, 1, 2], 10), ([3, 4, 5], 8))):
        for j in range(12):
            want = cache[blocks[j // 4], j % 4] if j < n else np.zeros((2, 8), np.float32)
            np.testing.assert_array_equal(out[b, j], want)


def test_gather_truncates_at_max_context_len_and_uses_the_layer():
    rng = np.random.default_rng(5)
    cache = _pool(rng, 6, 2, 1, 4)
    tables = np.array([[[0, 1, 2]], [[5, 4, 3]]], np.int32)
    lens = np.array([[6], [5]], np.int32)
    np.testing.assert_array_equal(oa.kv_gather(cache, 0, tables, lens, 3)[0], cache[[0, 0, 1], [0, 1, 0]])
    out = oa.kv_gather(cache, 1, tables, lens, 6)[0]
    np.testing.assert_array_equal(out[:5], cache[[5, 5, 4, 4, 3], [0, 1, 0, 1, 0]])
    np.testing.assert_array_equal(out[5], 0)


def test_scatter_decode_last_duplicate_wins_and_copies():
    cache = np.zeros((2, 2, 1, 2), np.float32)
    vals = np.arange(6, dtype=np.float32).reshape(3, 1, 2)
    out = oa.kv_scatter_decode(cache, vals, np.array([1, 0, 1]), np.array([0, 1, 0]))
    np.testing.assert_array_equal(out[1, 0, 0], [4, 5])
    np.testing.assert_array_equal(out[0, 1, 0], [2, 3])
    assert not cache.any()


def test_scatter_prefill_then_gather_round_trip():
    rng = np.random.default_rng(6)
    bs, hkv, d = 4, 2, 4
    tables = np.array([[[3, 0, 5], [1, 2, 4]]], np.int32)
    vals = rng.standard_normal((2, 9, hkv, d)).astype(np.float32)
    cache = oa.kv_scatter_prefill(np.zeros((6, bs, hkv, d), np.float32), 0, vals, tables, np.array([0, 2]), bs)
    got = oa.kv_gather(cache, 0, tables, np.array([[9, 11]], np.int32), 11)
    np.testing.assert_array_equal(got[0, :9], vals[0])
    np.testing.assert_array_equal(got[1, 2:11], vals[1])
    np.testing.assert_array_equal(got[1, :2], 0)   # never written
    np.testing.assert_array_equal(got[0, 9:], 0)   # past the context


# ------------------------------------------------------------------ attention_block_decode
def _block_inputs(rng, B, ctx, n_embd, H, Hkv, bias=True):
    D = n_embd // H
    nkv = Hkv * D
    f = lambda *s: rng.standard_normal(s) * 0.3
    return dict(x=f(B, n_embd), positions=rng.integers(0, 50, B), k_cached=f(B, ctx, Hkv, D),
                v_cached=f(B, ctx, Hkv, D), wq=f(n_embd, n_embd), wk=f(n_embd, nkv), wv=f(n_embd, nkv),
                wo=f(n_embd, n_embd), bq=f(n_embd), bk=f(nkv), bv=f(nkv), bo=f(n_embd), use_bias=bias)


def _block_loops(a, H, Hkv, n_embd, base, scale_f):
    """attention_block_decode.mlir:96-233 step by step with Python loops."""
    x, B = a["x"], a["x"].shape[0]
    D = n_embd // H
    q = x @ a["wq"] + (a["bq"] if a["use_bias"] else 0)
    k = x @ a["wk"] + (a["bk"] if a["use_bias"] else 0)
    v = x @ a["wv"] + (a["bv"] if a["use_bias"] else 0)

    def rot(vec, pos):
        out = vec.copy()
        for hh in range(vec.shape[0] // D):
            for i in range(D // 2):
                ang = pos * scale_f / base ** (2 * i / D)
                x0, x1 = vec[hh * D + 2 * i], vec[hh * D + 2 * i + 1]
                out[hh * D + 2 * i] = x0 * math.cos(ang) - x1 * math.sin(ang)
                out[hh * D + 2 * i + 1] = x0 * math.sin(ang) + x1 * math.cos(ang)
        return out

    outs, knew, vnew = [], [], []
    for b in range(B):
        qb, kb = rot(q[b], a["positions"][b]), rot(k[b], a["positions"][b])
        keys = np.concatenate([a["k_cached"][b], kb.reshape(1, Hkv, D)])
        vals = np.concatenate([a["v_cached"][b], v[b].reshape(1, Hkv, D)])
        att = np.zeros(n_embd)
        for h in range(H):
            kh = h // (H // Hkv)
            s = [qb[h * D:(h + 1) * D] @ keys[j, kh] / math.sqrt(D) for j in range(len(keys))]
            e = np.exp(np.array(s) - max(s))
            att[h * D:(h + 1) * D] = (e / e.sum()) @ vals[:, kh]
        outs.append(att @ a["wo"] + (a["bo"] if a["use_bias"] else 0))
        knew.append(kb.reshape(Hkv, D))
        vnew.append(v[b].reshape(Hkv, D))
    return np.array(outs), np.array(knew), np.array(vnew)


@pytest.mark.parametrize("B,ctx,n_embd,H,Hkv,bias", [(2, 5, 16, 4, 2, True), (1, 0, 8, 2, 2, False),
                                                     (3, 3, 24, 6, 1, True)])
def test_attention_block_decode_matches_loops(B, ctx, n_embd, H, Hkv, bias):
    a = _block_inputs(np.random.default_rng(B * 100 + ctx), B, ctx, n_embd, H, Hkv, bias)
    got = oa.attention_block_decode(a["x"], a["positions"], a["k_cached"], a["v_cached"], a["wq"], a["wk"], a["wv"],
                                    a["wo"], a["bq"], a["bk"], a["bv"], a["bo"], bias, H, Hkv, n_embd, 300.0, 0.5)
    want = _block_loops(a, H, Hkv, n_embd, 300.0, 0.5)
    for g, w in zip(got, want):
        np.testing.assert_allclose(g, w, rtol=1e-10, atol=1e-12)


def test_attention_block_decode_without_cache_returns_projected_value():
    # one key (the token itself): attention output = v_new, so out = v_new @ wo
    a = _block_inputs(np.random.default_rng(8), 2, 0, 16, 2, 2, bias=False)
    out, _, v_new = oa.attention_block_decode(a["x"], a["positions"], a["k_cached"], a["v_cached"], a["wq"], a["wk"],
                                              a["wv"], a["wo"], None, None, None, None, False, 2, 2, 16)
    np.testing.assert_allclose(out, v_new.reshape(2, 16) @ a["wo"], rtol=1e-12)


def test_paged_decode_is_gather_block_scatter_with_zero_rows():
    rng = np.random.default_rng(9)
    n_embd, H, Hkv, bs = 16, 4, 2, 4
    D = n_embd // H
    a = _block_inputs(rng, 2, 0, n_embd, H, Hkv, bias=True)
    kp, vp = _pool(rng, 6, bs, Hkv, D), _pool(rng, 6, bs, Hkv, D)
    tables = np.array([[[2, 5, 0], [1, 3, 4]]], np.int32)
    lens = np.array([[6, 3]], np.int32)
    max_ctx = 7
    out, k_new, v_new, kc2, vc2 = oa.attention_decode_paged(
        a["x"], a["positions"], kp, vp, 0, tables, lens, max_ctx, np.array([5, 3]), np.array([2, 3]),
        a["wq"], a["wk"], a["wv"], a["wo"], a["bq"], a["bk"], a["bv"], a["bo"], True, H, Hkv, n_embd)
    # explicit: cached rows, zero rows up to max_ctx, then the new token
    kc = np.zeros((2, max_ctx, Hkv, D))
    vc = np.zeros((2, max_ctx, Hkv, D))
    for b, blocks in enumerate(([2, 5], [1])):
        for j in range(lens[0, b]):
            kc[b, j], vc[b, j] = kp[blocks[j // bs], j % bs], vp[blocks[j // bs], j % bs]
    want = oa.attention_block_decode(a["x"], a["positions"], kc, vc, a["wq"], a["wk"], a["wv"], a["wo"], a["bq"],
                                     a["bk"], a["bv"], a["bo"], True, H, Hkv, n_embd)
    np.testing.assert_allclose(out, want[0], rtol=1e-12)
    np.testing.assert_array_equal(kc2[5, 2], k_new[0].astype(np.float32))
    np.testing.assert_array_equal(vc2[3, 3], v_new[1].astype(np.float32))
    untouched = np.ones(6 * bs, bool).reshape(6, bs)
    untouched[5, 2] = untouched[3, 3] = False
    np.testing.assert_array_equal(kc2[untouched], kp[untouched])


def test_attention_sublayer_is_norm_then_paged_then_residual():
    from oracle import layer as ol

    rng = np.random.default_rng(10)
    n_embd, H, Hkv, bs = 16, 4, 2, 4
    D = n_embd // H
    a = _block_inputs(rng, 2, 0, n_embd, H, Hkv, bias=False)
    kp, vp = _pool(rng, 6, bs, Hkv, D), _pool(rng, 6, bs, Hkv, D)
    tables = np.array([[[2, 5, 0], [1, 3, 4]]], np.int32)
    lens = np.array([[6, 3]], np.int32)
    nw = rng.standard_normal(n_embd)
    args = (a["positions"], kp, vp, 0, tables, lens, 7, np.array([5, 3]), np.array([2, 3]), a["wq"], a["wk"],
            a["wv"], a["wo"], None, None, None, None, False, H, Hkv, n_embd)
    got = oa.attention_sublayer_decode_paged(a["x"], nw, 1e-5, *args)
    xn = ol.rms_norm(a["x"], nw, 1e-5)
    want = oa.attention_decode_paged(xn, *args)
    np.testing.assert_allclose(got[0], a["x"] + want[0], rtol=1e-14)
    np.testing.assert_array_equal(got[3], want[3])
