"""Pins the CPU oracle (oracle/) before anything is checked against it.

Every oracle function is checked against something other than a retyped copy
of its own formula: brute-force loops, closed forms in another form,
invariants, special cases that reduce to textbook routines, torch's casts,
and the reference's hand-written id arrays.  Each group also plants a
plausible mistake in a copy of the oracle and shows the pin catches it.
"""

import itertools
import math

import numpy as np
import pytest
import torch

import oracle
from oracle import moe as om
from oracle import numerics as nm


# ------------------------------------------------------------------ swiglu
def test_swiglu_known_answers():
    g = np.array([0.0, 1.0, 1.0, 1.0, 2.0, -3.0], np.float64)
    u = np.array([0.0, 0.0, 30.0, -30.0, 1.0, 2.0], np.float64)
    out = oracle.swiglu(g, u)
    assert out[0] == 0.0 and out[1] == 0.0  # u = 0 -> silu 0
    assert abs(out[2] - 30.0) < 1e-9  # silu(30) ~ 30
    assert abs(out[3]) < 1e-10  # silu(-30) ~ -30 e^-30
    assert out[4] == pytest.approx(2.0 / (1.0 + math.exp(-1.0)))  # g * sigmoid(1) * 1
    assert out[5] == pytest.approx(-3.0 * 2.0 / (1.0 + math.exp(-2.0)))


def test_swiglu_matches_torch_silu():
    rng = np.random.default_rng(0)
    g = rng.standard_normal((3, 5, 7)) * 4
    u = rng.standard_normal((3, 5, 7)) * 4
    ref = (torch.nn.functional.silu(torch.from_numpy(u)) * torch.from_numpy(g)).numpy()
    np.testing.assert_allclose(oracle.swiglu(g, u), ref, rtol=1e-12, atol=1e-14)


def test_swiglu_operand_swap_is_caught():
    """silu acts on `up` (swiglu.mlir:37-47): the HF/llama.cpp order would
    fail the known-answer test."""
    swapped = lambda g, u: u * om.silu(g)  # noqa: E731  (planted mistake)
    g, u = np.array([1.0]), np.array([-30.0])
    assert abs(oracle.swiglu(g, u)[0]) < 1e-10
    assert abs(swapped(g, u)[0]) > 1.0


# ------------------------------------------------------------------ router
def _one_hot_router(logits_et):
    """Input/router pair whose logits are exactly `logits_et` [E, T]:
    x = identity rows (T = H), W_router = logits."""
    E, T = logits_et.shape
    return np.eye(T), np.asarray(logits_et, np.float64)


def test_router_softmax_closed_form_and_invariants():
    rng = np.random.default_rng(1)
    logits = rng.standard_normal((8, 16)) * 3
    x, wr = _one_hot_router(logits)
    p = om.router_probs(x, wr)
    # scipy's softmax is an independent restatement
    from scipy.special import softmax

    np.testing.assert_allclose(p, softmax(logits, axis=0), rtol=1e-13)
    np.testing.assert_allclose(p.sum(axis=0), 1.0, rtol=1e-14)
    # shift invariance: adding c to every logit of a token changes nothing
    p2 = om.router_probs(x, wr + 5.0)
    np.testing.assert_allclose(p, p2, rtol=1e-12)
    # equal logits -> 1/E
    x, wr = _one_hot_router(np.zeros((8, 3)))
    np.testing.assert_allclose(om.router_probs(x, wr), 1.0 / 8)


def _topk_brute(probs, k):
    E, T = probs.shape
    ids = np.zeros((k, T), np.int32)
    for t in range(T):
        order = sorted(range(E), key=lambda e: (-probs[e, t], e))
        ids[:, t] = order[:k]
    return ids


@pytest.mark.parametrize("E,k,T", [(4, 2, 5), (8, 2, 16), (8, 8, 3), (16, 6, 9), (5, 1, 7)])
def test_router_topk_brute_force(E, k, T):
    rng = np.random.default_rng(E * 100 + k)
    x = rng.standard_normal((T, 12))
    wr = rng.standard_normal((E, 12))
    ids, w = om.router(x, wr, k, False)
    p = om.router_probs(x, wr)
    np.testing.assert_array_equal(ids, _topk_brute(p, k))
    np.testing.assert_array_equal(w, np.take_along_axis(p, ids.astype(np.int64), axis=0))
    assert np.all(np.diff(w, axis=0) <= 0)  # descending slots


def test_router_ties_go_to_lower_index():
    logits = np.array([[1.0, 0.0, 5.0], [2.0, 0.0, 5.0], [2.0, 0.0, 5.0], [0.0, 0.0, 5.0]])  # [E=4, T=3]
    x, wr = _one_hot_router(logits)
    ids, _ = om.router(x, wr, 2, False)
    np.testing.assert_array_equal(ids[:, 0], [1, 2])  # 2.0 tie between experts 1, 2
    np.testing.assert_array_equal(ids[:, 1], [0, 1])  # all equal
    np.testing.assert_array_equal(ids[:, 2], [0, 1])
    # planted mistake: ties to the higher index
    p = om.router_probs(x, wr)
    bad = (p.shape[0] - 1 - np.argsort(-p[::-1], axis=0, kind="stable"))[:2]
    assert not np.array_equal(bad, ids)


def ulp_tie_router_inputs(E, H, T):
    """Router inputs whose fp32 logits for experts 2 and 5 are one ulp apart
    (c and c + 2**-37 with c = 1.5 * 2**-14, both exact in bf16 and in an
    fp32 sum) while every other expert's logit is -1: exp of a -7.3e-12
    difference rounds to 1 in fp32, so the two probabilities are equal.  The
    larger logit sits at the higher index, so selecting on logits and
    selecting on fp32 probabilities disagree on the slot order."""
    c = 1.5 * 2.0**-14
    x = np.zeros((T, H), np.float32)
    x[:, :2] = 1.0
    wr = np.zeros((E, H), np.float32)
    wr[:, 0] = -1.0
    wr[2, 0] = c
    wr[5, 0] = c
    wr[5, 1] = 2.0**-37
    return x, wr


def test_router_ulp_apart_logits_tie_on_fp32_probabilities():
    E, k = 8, 3
    x, wr = ulp_tie_router_inputs(E, 64, 4)
    logits = (wr @ x.T).astype(np.float32)
    assert logits[5, 0] == np.nextafter(logits[2, 0], np.float32(1))  # one ulp apart
    ids32, w32 = om.router(x, wr, k, False, dtype=np.float32)
    # fp32 probabilities tie: the lower index first, then expert 0 (lowest of
    # the equal -1 logits)
    np.testing.assert_array_equal(ids32[:, 0], [2, 5, 0])
    assert w32[0, 0] == w32[1, 0]
    # in float64 the larger logit wins: exact ties exist only at fp32
    ids64, _ = om.router(x, wr, k, False)
    np.testing.assert_array_equal(ids64[:, 0], [5, 2, 0])


def test_router_renormalisation():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((20, 16))
    wr = rng.standard_normal((8, 16))
    ids, w = om.router(x, wr, 3, True)
    np.testing.assert_allclose(w.sum(axis=0), 1.0, rtol=1e-14)
    ids1, w1 = om.router(x, wr, 1, True)
    assert np.all(w1 == 1.0)
    ids0, w0 = om.router(x, wr, 3, False)
    np.testing.assert_array_equal(ids, ids0)
    np.testing.assert_allclose(w, w0 / w0.sum(axis=0), rtol=1e-15)


# ------------------------------------------------------------------ permutation
def _permute_brute(ids, E):
    flat = [int(v) for v in np.asarray(ids).reshape(-1)]
    order, offsets = [], [0]
    for e in range(E):
        order += [f for f, v in enumerate(flat) if v == e]
        offsets.append(len(order))
    return np.array(order, np.int32), np.array(offsets, np.int32)


REFERENCE_IDS = [  # tests/components/test_mul_mat_id.py:23-25, :42-48, :64
    (np.array([[0, 3]], np.int32), 8),
    (np.array([[0, 1, 2, 3], [4, 5, 6, 7]], np.int32), 8),
    (np.array([[2, 2, 2]], np.int32), 4),
]


@pytest.mark.parametrize("case", range(len(REFERENCE_IDS)))
def test_permute_reference_ids(case):
    ids, E = REFERENCE_IDS[case]
    order, offsets = om.permute(ids, E)
    bo, boff = _permute_brute(ids, E)
    np.testing.assert_array_equal(order, bo)
    np.testing.assert_array_equal(offsets, boff)


def test_permute_known_answer():
    ids = np.array([[0, 1, 2, 3], [4, 5, 6, 7]], np.int32)
    order, offsets = om.permute(ids, 8)
    np.testing.assert_array_equal(order, [0, 1, 2, 3, 4, 5, 6, 7])
    ids = np.array([[2, 0, 2], [0, 1, 1]], np.int32)  # flat [2,0,2,0,1,1]
    order, offsets = om.permute(ids, 3)
    np.testing.assert_array_equal(order, [1, 3, 4, 5, 0, 2])
    np.testing.assert_array_equal(offsets, [0, 2, 4, 6])


@pytest.mark.parametrize("E,k,T", [(8, 2, 50), (64, 6, 33), (128, 8, 17), (3, 3, 1)])
def test_permute_random_vs_brute(E, k, T):
    rng = np.random.default_rng(E + k + T)
    ids = np.stack([rng.permutation(E)[:k] for _ in range(T)], axis=1).astype(np.int32)
    order, offsets = om.permute(ids, E)
    bo, boff = _permute_brute(ids, E)
    np.testing.assert_array_equal(order, bo)
    np.testing.assert_array_equal(offsets, boff)
    # planted mistake: an unstable sort is not the stable grouping
    rng2 = np.random.default_rng(0)
    shuffled = np.concatenate([rng2.permutation(bo[offsets[e]:offsets[e + 1]]) for e in range(E)])
    if not np.array_equal(shuffled, bo):
        assert not np.array_equal(shuffled, order)


def test_permute_rejects_bad_ids():
    with pytest.raises(ValueError):
        om.permute(np.array([[0, 8]], np.int32), 8)
    with pytest.raises(ValueError):
        om.permute(np.array([[-1, 0]], np.int32), 8)


# ------------------------------------------------------------------ mul_mat_id
def _mmid_case(seed, n_out, n_in, E, k, T, ids=None):
    np.random.seed(seed)
    w = np.random.randn(n_out, n_in, E).astype(np.float32) * 0.1
    x = np.random.randn(n_in, k, T).astype(np.float32) * 0.1
    if ids is None:
        ids = np.random.randint(0, E, size=(k, T), dtype=np.int32)
    return w, x, ids


# The reference's four mul_mat_id cases (tests/components/test_mul_mat_id.py).
MMID_REFERENCE_CASES = [
    (42, 4, 3, 8, 1, 2, np.array([[0, 3]], np.int32)),
    (123, 8, 4, 8, 2, 4, np.array([[0, 1, 2, 3], [4, 5, 6, 7]], np.int32)),
    (456, 6, 4, 4, 1, 3, np.array([[2, 2, 2]], np.int32)),
    (789, 64, 32, 8, 2, 16, None),
]


@pytest.mark.parametrize("case", range(len(MMID_REFERENCE_CASES)))
def test_mul_mat_id_three_forms_agree(case):
    w, x, ids = _mmid_case(*MMID_REFERENCE_CASES[case])
    loops = om.mul_mat_id_loops(w, x, ids)
    lit = om.mul_mat_id_literal(w, x, ids)
    grp = om.mul_mat_id(w, x, ids)
    np.testing.assert_allclose(lit, loops, rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(grp, loops, rtol=1e-12, atol=1e-14)
    # planted mistake: the transposed weight operand is caught by the loops
    if w.shape[0] == w.shape[1]:
        bad = om.mul_mat_id(w.transpose(1, 0, 2), x, ids)
        assert not np.allclose(bad, loops)


def test_mul_mat_id_special_cases():
    rng = np.random.default_rng(3)
    E, k, T, n = 4, 2, 5, 6
    # identity weights -> output equals input
    w = np.repeat(np.eye(n)[:, :, None], E, axis=2)
    x = rng.standard_normal((n, k, T))
    ids = rng.integers(0, E, (k, T)).astype(np.int32)
    np.testing.assert_allclose(om.mul_mat_id(w, x, ids), x, rtol=1e-15)
    # all ids equal e -> dense GEMM with W[:, :, e]
    w = rng.standard_normal((7, n, E))
    ids = np.full((k, T), 2, np.int32)
    dense = np.einsum("oi,ist->ost", w[:, :, 2], x)
    np.testing.assert_allclose(om.mul_mat_id(w, x, ids), dense, rtol=1e-12)
    # one-hot input e_j selects column j of the routed expert
    x1 = np.zeros((n, 1, 1))
    x1[3, 0, 0] = 1.0
    out = om.mul_mat_id(w, x1, np.array([[1]], np.int32))
    np.testing.assert_array_equal(out[:, 0, 0], w[:, 3, 1])


# ------------------------------------------------------------------ moe_ffn_block
# The reference's four block cases (tests/components/test_moe_ffn_block.py).
BLOCK_REFERENCE_CASES = [
    # seed, T, H, F, E, k, normalize
    (42, 4, 8, 16, 4, 2, False),
    (123, 3, 8, 12, 4, 2, True),
    (456, 4, 8, 16, 8, 1, False),
    (789, 8, 32, 64, 8, 2, False),
]


def block_inputs(seed, T, H, F, E):
    np.random.seed(seed)
    x = np.random.randn(T, H).astype(np.float32) * 0.1
    wr = np.random.randn(E, H).astype(np.float32) * 0.1
    up = np.random.randn(F, H, E).astype(np.float32) * 0.1
    gate = np.random.randn(F, H, E).astype(np.float32) * 0.1
    down = np.random.randn(H, F, E).astype(np.float32) * 0.1
    return x, wr, up, gate, down


@pytest.mark.parametrize("case", range(len(BLOCK_REFERENCE_CASES)))
def test_block_grouped_equals_literal(case):
    seed, T, H, F, E, k, norm = BLOCK_REFERENCE_CASES[case]
    x, wr, up, gate, down = block_inputs(seed, T, H, F, E)
    lit = om.moe_ffn_block_literal(x, wr, up, gate, down, E, k, H, F, norm)
    lit64 = om.moe_ffn_block_literal(x, wr, up, gate, down, E, k, H, F, norm, dtype=np.float64)
    grp = om.moe_ffn_block(x, wr, up, gate, down, E, k, H, F, norm)
    np.testing.assert_allclose(lit64, grp, rtol=1e-12, atol=1e-15)
    np.testing.assert_allclose(lit, grp, rtol=1e-4, atol=1e-6)


def test_block_single_expert_is_dense_swiglu_ffn():
    rng = np.random.default_rng(5)
    T, H, F = 6, 10, 14
    x = rng.standard_normal((T, H))
    up, gate, down = rng.standard_normal((F, H, 1)), rng.standard_normal((F, H, 1)), rng.standard_normal((H, F, 1))
    wr = rng.standard_normal((1, H))
    out = om.moe_ffn_block(x, wr, up, gate, down, 1, 1, H, F, False)
    u = x @ up[:, :, 0].T
    g = x @ gate[:, :, 0].T
    h = g * (u * (1.0 / (1.0 + np.exp(-u))))  # sigmoid form of swiglu.mlir:40-45
    np.testing.assert_allclose(out, h @ down[:, :, 0].T, rtol=1e-12)


def test_block_identical_experts_normalized_is_dense():
    rng = np.random.default_rng(6)
    T, H, F, E, k = 9, 8, 12, 6, 3
    x = rng.standard_normal((T, H))
    wr = rng.standard_normal((E, H))
    one_up, one_gate, one_down = rng.standard_normal((F, H)), rng.standard_normal((F, H)), rng.standard_normal((H, F))
    up = np.repeat(one_up[:, :, None], E, axis=2)
    gate = np.repeat(one_gate[:, :, None], E, axis=2)
    down = np.repeat(one_down[:, :, None], E, axis=2)
    dense = (x @ one_gate.T) * om.silu(x @ one_up.T) @ one_down.T
    out = om.moe_ffn_block(x, wr, up, gate, down, E, k, H, F, True)
    np.testing.assert_allclose(out, dense, rtol=1e-12, atol=1e-13)
    # planted mistake: dropping the renormalisation scales the output by sum(w) < 1
    unnorm = om.moe_ffn_block(x, wr, up, gate, down, E, k, H, F, False)
    assert not np.allclose(unnorm, dense, rtol=1e-3)


def test_block_token_independence():
    rng = np.random.default_rng(7)
    T, H, F, E, k = 12, 8, 16, 5, 2
    x = rng.standard_normal((T, H)).astype(np.float32)
    wr = rng.standard_normal((E, H)).astype(np.float32)
    up, gate, down = (rng.standard_normal(s).astype(np.float32) for s in ((F, H, E), (F, H, E), (H, F, E)))
    full = om.moe_ffn_block(x, wr, up, gate, down, E, k, H, F, False)
    idx = np.array([11, 0, 5])
    part = om.moe_ffn_block_tokens(idx, x, wr, up, gate, down, E, k, H, F, False)
    np.testing.assert_allclose(part, full[idx], rtol=1e-12)


# ------------------------------------------------------------------ numerics
def test_bf16_round_matches_torch():
    rng = np.random.default_rng(8)
    x = np.concatenate([
        rng.standard_normal(50000).astype(np.float32) * 100,
        np.array([0.0, -0.0, 1.0 + 2**-8, 1.0 + 3 * 2**-8, 3.3895314e38, np.inf, -np.inf], np.float32),
    ])
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(nm.bf16_round(x).view(np.uint32), ref.view(np.uint32))
    # ties to even: 1 + 2^-8 is halfway between 1 and 1 + 2^-7 -> 1
    assert nm.bf16_round(np.float32(1.0 + 2**-8)) == 1.0
    assert nm.bf16_round(np.float32(1.0 + 3 * 2**-8)) == np.float32(1.0 + 2**-6)


def test_e4m3fn_decode_table():
    v = nm.E4M3FN_VALUES
    assert v[0x7E] == 448.0 and v[0xFE] == -448.0
    assert np.isnan(v[0x7F]) and np.isnan(v[0xFF])
    assert v[0x01] == 2.0**-9 and v[0x08] == 2.0**-6 and v[0x38] == 1.0
    codes = np.array([c for c in range(256) if c not in (0x7F, 0xFF)], np.uint8)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    np.testing.assert_array_equal(nm.e4m3fn_decode(codes), ref)


def test_e4m3fn_encode_matches_torch_and_saturates():
    rng = np.random.default_rng(9)
    mids = ((nm.E4M3FN_VALUES[:126] + nm.E4M3FN_VALUES[1:127]) / 2).astype(np.float32)
    x = np.concatenate([rng.standard_normal(100000).astype(np.float32) * 50, mids, -mids,
                        nm.E4M3FN_VALUES[:127].astype(np.float32)])
    x = x[np.abs(x) <= 448]
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(nm.e4m3fn_encode(x), ref)
    sat = nm.e4m3fn_encode(np.array([449.0, 1e6, -500.0, np.nan], np.float32))
    np.testing.assert_array_equal(sat, [0x7E, 0x7E, 0xFE, 0x7F])


def test_per_channel_quantisation():
    rng = np.random.default_rng(10)
    w = (rng.standard_normal((16, 64, 3)) * 0.02).astype(np.float32)
    w[5, :, 1] = 0.0
    q, s = nm.quantize_per_channel_e4m3fn(w)
    assert q.shape == w.shape and s.shape == (16, 3)
    assert s[5, 1] == 1.0 and np.all(q[5, :, 1] == 0)
    # the absmax element of every non-zero channel encodes to +-448
    mags = nm.e4m3fn_decode(q & 0x7F)
    assert np.all(mags.max(axis=1)[s != 1.0] == 448.0)
    deq = nm.dequantize_e4m3fn(q, s)
    # e4m3 has 3 mantissa bits: relative error <= 2^-4 for normals
    big = np.abs(w) > s[:, None, :] * 2.0**-6
    assert np.all(np.abs(deq - w)[big] <= np.abs(w)[big] * 2.0**-4 + 1e-12)


# ------------------------------------------------------------------ rms_norm / sub-layer
def _rms_norm_mistakes():
    """Plausible mistakes in an RMSNorm, each of which the pins below catch."""
    def sum_not_mean(x, w, eps=1e-6):
        return x / np.sqrt(np.sum(x * x, -1, keepdims=True) + eps) * w

    def eps_outside_sqrt(x, w, eps=1e-6):
        return x / (np.sqrt(np.mean(x * x, -1, keepdims=True)) + eps) * w

    def weight_dropped(x, w, eps=1e-6):
        return x / np.sqrt(np.mean(x * x, -1, keepdims=True) + eps)

    return [sum_not_mean, eps_outside_sqrt, weight_dropped]


def _rms_norm_pins(f):
    """Closed forms that an RMSNorm must meet; returns the failures."""
    bad = []
    H = 16
    w = np.linspace(0.5, 2.0, H)
    # a constant row c: mean(x^2) = c^2, so out = c / sqrt(c^2 + eps) * w
    for c, eps in ((3.0, 1e-6), (0.01, 1e-2), (-2.0, 0.5)):
        x = np.full((1, H), c)
        if not np.allclose(f(x, w, eps), c / math.sqrt(c * c + eps) * w, rtol=1e-12, atol=0):
            bad.append(("constant", c, eps))
    # a one-hot row v e_i: mean(x^2) = v^2 / H
    x = np.zeros((1, H))
    x[0, 5] = 4.0
    ref = np.zeros(H)
    ref[5] = 4.0 / math.sqrt(16.0 / H + 1e-3) * w[5]
    if not np.allclose(f(x, w, 1e-3), ref, rtol=1e-12, atol=0):
        bad.append("one-hot")
    return bad


def test_rms_norm_closed_forms():
    assert _rms_norm_pins(oracle.rms_norm) == []
    for mistake in _rms_norm_mistakes():
        assert _rms_norm_pins(mistake), mistake.__name__


def test_rms_norm_invariants_and_torch():
    rng = np.random.default_rng(7)
    x = rng.standard_normal((5, 64)) * rng.uniform(0.1, 10.0, (5, 1))
    w = rng.standard_normal(64)
    # eps = 0: invariant under a positive per-row scale; unit weight gives unit RMS
    np.testing.assert_allclose(oracle.rms_norm(x * 37.0, w, 0.0), oracle.rms_norm(x, w, 0.0), rtol=1e-12)
    y = oracle.rms_norm(x, np.ones(64), 0.0)
    np.testing.assert_allclose(np.sqrt(np.mean(y * y, -1)), 1.0, rtol=1e-12)
    # torch's own RMSNorm
    ref = torch.nn.functional.rms_norm(torch.from_numpy(x), (64,), torch.from_numpy(w), eps=1e-5).numpy()
    np.testing.assert_allclose(oracle.rms_norm(x, w, 1e-5), ref, rtol=1e-12, atol=1e-14)
    # float32 evaluation stays close to float64
    np.testing.assert_allclose(oracle.rms_norm(x, w, 1e-5, dtype=np.float32), ref, rtol=1e-5, atol=1e-6)


def _tiny_layer(rng, T=6, H=16, F=24, E=4, k=2):
    res = rng.standard_normal((T, H)) * 2.0
    nw = rng.uniform(0.5, 1.5, H)
    wr = rng.standard_normal((E, H)) * 0.3
    up = rng.standard_normal((F, H, E)) * 0.2
    gate = rng.standard_normal((F, H, E)) * 0.2
    down = rng.standard_normal((H, F, E)) * 0.2
    return res, nw, wr, up, gate, down, E, k, H, F


def test_sublayer_zero_experts_is_identity():
    rng = np.random.default_rng(8)
    res, nw, wr, up, gate, down, E, k, H, F = _tiny_layer(rng)
    z = np.zeros_like(up)
    out = oracle.moe_ffn_sublayer(res, nw, 1e-6, wr, z, z, np.zeros_like(down), E, k, H, F, True)
    np.testing.assert_array_equal(out, res)


def test_sublayer_is_residual_plus_block_of_norm():
    rng = np.random.default_rng(9)
    res, nw, wr, up, gate, down, E, k, H, F = _tiny_layer(rng)
    out, ids, _ = oracle.moe_ffn_sublayer(res, nw, 1e-5, wr, up, gate, down, E, k, H, F, False,
                                          return_routing=True)
    # the pinned block (literal reference formula) on the pinned norm's output
    xn = oracle.rms_norm(res, nw, 1e-5)
    block = om.moe_ffn_block_literal(xn, wr, up, gate, down, E, k, H, F, False, dtype=np.float64)
    np.testing.assert_allclose(out - res, block, rtol=1e-10, atol=1e-12)
    ref_ids, _ = om.router(xn, wr, k, False)
    np.testing.assert_array_equal(ids, ref_ids)
    # planted mistake: routing on the un-normalised residual changes the output
    wrong = res + om.moe_ffn_block_literal(res, wr, up, gate, down, E, k, H, F, False, dtype=np.float64)
    assert not np.allclose(out, wrong, rtol=1e-6, atol=1e-8)


# ------------------------------------------------------------------ per-row e4m3 activations
def test_quantize_rows_e4m3fn_known_answer_and_bounds():
    rows = np.array([[1.0, -2.0, 0.5, 3.0], [0.0, 0.0, 0.0, 0.0], [448.0, 1.0, -2.0, 0.0],
                     [449.0, 0.0, 0.0, 0.0], [2.0**-130, 0.0, 0.0, 0.0]], np.float32)
    q, s = nm.quantize_rows_e4m3fn(rows)
    # max 3: 3 / 448 lies in (2^-8, 2^-7], so the scale is 2^-7 and the row is exact
    assert s[0] == 2.0**-7
    np.testing.assert_array_equal(nm.e4m3fn_decode(q[0]), [128.0, -256.0, 64.0, 384.0])
    assert s[1] == 1.0 and not q[1].any()  # all-zero row
    assert s[2] == 1.0 and nm.e4m3fn_decode(q[2])[0] == 448.0  # 448 fits exactly: 2^0
    assert s[3] == 2.0  # just above 448: the next power of two
    assert s[4] == 2.0**-126  # a subnormal maximum: the scale is clamped
    rng = np.random.default_rng(3)
    a = (rng.standard_normal((64, 512)) * rng.uniform(0.01, 100, (64, 1))).astype(np.float32)
    q, s = nm.quantize_rows_e4m3fn(a)
    # powers of two; every row's largest magnitude lands in (224, 448]
    np.testing.assert_array_equal(np.frexp(s)[0], 0.5)
    top = np.argmax(np.abs(a), axis=1)
    big = np.abs(a[np.arange(64), top]) / s
    assert np.all((big > 224) & (big <= 448))
    # half an ulp of a 3-bit mantissa: 2^-4 relative, above the subnormal range
    d = nm.fake_quantize_rows_e4m3fn(a)
    normal = np.abs(a) >= 2.0**-6 * s[:, None]
    assert np.all(np.abs(d - a)[normal] <= 2.0**-4 * np.abs(a)[normal] * (1 + 1e-6))
    # scale invariance: a row times a power of two quantises to the same codes
    q2, s2 = nm.quantize_rows_e4m3fn(a * np.float32(8.0))
    np.testing.assert_array_equal(q2, q)
    np.testing.assert_array_equal(s2, s * 8)
    # planted mistake: scale = max/448 (not a power of two) changes some codes
    q_bad = nm.e4m3fn_encode(a / (np.abs(a).max(axis=1, keepdims=True) / 448.0))
    assert not np.array_equal(q_bad, q)


def test_act_quant_block_is_the_block_on_quantised_rows():
    """E = k = 1: the fp8-activation block is the dense SwiGLU FFN of the
    per-row e4m3 token rows, with the SwiGLU rows rounded to bf16 and
    quantised per row before the down projection."""
    rng = np.random.default_rng(4)
    T, H, F = 24, 64, 128
    x = nm.bf16_round(rng.standard_normal((T, H)).astype(np.float32))
    wr = np.zeros((1, H), np.float32)
    up, gate = ((rng.standard_normal((F, H, 1)) * 0.05).astype(np.float32) for _ in range(2))
    down = (rng.standard_normal((H, F, 1)) * 0.05).astype(np.float32)
    out = om.moe_ffn_block(x, wr, up, gate, down, 1, 1, H, F, False, dtype=np.float64, act_quant=True)
    xq = nm.fake_quantize_rows_e4m3fn(x).astype(np.float64)
    g, u = xq @ gate[:, :, 0].T.astype(np.float64), xq @ up[:, :, 0].T.astype(np.float64)
    h = nm.fake_quantize_rows_e4m3fn(nm.bf16_round(g * u / (1 + np.exp(-u)))).astype(np.float64)
    np.testing.assert_allclose(out, h @ down[:, :, 0].T.astype(np.float64), rtol=1e-12, atol=1e-12)
    # and it differs from the unquantised block by the e4m3 rounding only (a few percent)
    plain = om.moe_ffn_block(x, wr, up, gate, down, 1, 1, H, F, False, dtype=np.float64)
    rel = np.linalg.norm(out - plain) / np.linalg.norm(plain)
    assert 1e-3 < rel < 0.1, rel


def test_quantize_rows_e4m3fn_x2_is_exact_on_bf16_rows():
    """Two-term rows (hi = e4m3(v), lo = e4m3(v - hi) under one power-of-two
    row scale).  What the arithmetic fixes: a bf16 value v (8 significant
    bits) scaled into (224, 448] has hi = v rounded to 4 significant bits,
    so v - hi is a multiple of v's last bit of at most 4 bits, which lo holds
    exactly while that bit is at least e4m3's smallest step 2^-9, i.e. for
    |v| >= 2^-2; below, lo rounds to the 2^-9 grid (error at most 2^-10)."""
    rng = np.random.default_rng(11)
    a = nm.bf16_round((rng.standard_normal((64, 512)) * rng.uniform(0.01, 100, (64, 1))).astype(np.float32))
    a[:, :64] *= np.float32(2.0**-12)  # some tiny entries, below the exact range
    hi, lo, s = nm.quantize_rows_e4m3fn_x2(a)
    q1, s1 = nm.quantize_rows_e4m3fn(a)
    np.testing.assert_array_equal(hi, q1)  # hi is the one-term quantisation
    np.testing.assert_array_equal(s, s1)
    v = a / s[:, None]
    d = nm.fake_quantize_rows_e4m3fn_x2(a) / s[:, None]
    big = np.abs(v) >= 2.0**-2
    assert big.mean() > 0.5 and (~big).any()
    np.testing.assert_array_equal(d[big], v[big])
    assert np.all(np.abs(d - v)[~big] <= 2.0**-10)
    # lo is at most half an ulp of hi: 2^-4 of the value
    assert np.all(np.abs(nm.e4m3fn_decode(lo)) <= 2.0**-4 * np.abs(v) * (1 + 1e-6) + 2.0**-10)
    # planted mistakes: lo coded from v (not its remainder), or one term only
    wrong = (nm.e4m3fn_decode(hi) + nm.e4m3fn_decode(nm.e4m3fn_encode(v))) * s[:, None]
    assert not np.allclose(wrong, a, rtol=1e-3)
    assert not np.array_equal(nm.fake_quantize_rows_e4m3fn(a)[big], a[big])


def test_act_quant_x2_block_is_the_block_on_two_term_rows():
    """E = k = 1: the two-term block is the dense SwiGLU FFN on the two-term
    token rows and bf16-rounded SwiGLU rows, and since those rows are bf16
    values represented exactly (above 2^-2 of their scale), it stays within
    bf16-level rounding of the unquantised block, unlike the one-term block."""
    rng = np.random.default_rng(12)
    T, H, F = 24, 64, 128
    x = nm.bf16_round(rng.standard_normal((T, H)).astype(np.float32))
    wr = np.zeros((1, H), np.float32)
    up, gate = ((rng.standard_normal((F, H, 1)) * 0.05).astype(np.float32) for _ in range(2))
    down = (rng.standard_normal((H, F, 1)) * 0.05).astype(np.float32)
    out = om.moe_ffn_block(x, wr, up, gate, down, 1, 1, H, F, False, dtype=np.float64, act_quant="x2")
    xq = nm.fake_quantize_rows_e4m3fn_x2(x).astype(np.float64)
    g, u = xq @ gate[:, :, 0].T.astype(np.float64), xq @ up[:, :, 0].T.astype(np.float64)
    h = nm.fake_quantize_rows_e4m3fn_x2(nm.bf16_round(g * u / (1 + np.exp(-u)))).astype(np.float64)
    np.testing.assert_allclose(out, h @ down[:, :, 0].T.astype(np.float64), rtol=1e-12, atol=1e-12)
    plain = om.moe_ffn_block(x, wr, up, gate, down, 1, 1, H, F, False, dtype=np.float64)
    one = om.moe_ffn_block(x, wr, up, gate, down, 1, 1, H, F, False, dtype=np.float64, act_quant=True)
    rel2 = np.linalg.norm(out - plain) / np.linalg.norm(plain)
    rel1 = np.linalg.norm(one - plain) / np.linalg.norm(plain)
    assert rel2 < 5e-3 and rel2 < rel1 / 5, (rel2, rel1)
    with pytest.raises(ValueError):
        om.moe_ffn_block(x, wr, up, gate, down, 1, 1, H, F, False, act_quant="x3")


def _branchfree_e4m3(x):
    """The kernels' branch-free float -> e4m3fn encoder (common.h
    f32_to_e4m3fn), step for step in NumPy integer arithmetic."""
    x = np.asarray(x, np.float32)
    sign = (x.view(np.uint32) >> 24) & 0x80
    a = np.abs(x)
    ab = a.view(np.uint32).astype(np.uint64)
    r = (ab + 0x7FFFF + ((ab >> 20) & 1)) & 0xFFFFFFFF
    normal = ((((r >> 23) - 120) & 0xFFFFFFFF) << 3) | ((r >> 20) & 7)
    sub = np.rint(a * np.float32(512.0)).astype(np.uint64)
    code = np.where(a < np.float32(2.0**-6), sub, normal)
    code = np.where(a >= np.float32(448.0), 0x7E, code)
    return np.where(np.isnan(a), 0x7F, sign.astype(np.uint64) | code).astype(np.uint8)


def test_branchfree_e4m3_encoder_matches_the_oracle():
    """Every representable value, every midpoint between neighbours and one
    float32 ulp either side of it (the RNE ties), the subnormal range,
    saturation, inf and NaN, and a random sweep: the integer-add rounding the
    kernels use equals the oracle's nearest-value search."""
    vals = nm.E4M3FN_VALUES[:127]
    mids = (vals[:-1] + vals[1:]) / 2
    pts = np.concatenate([vals, mids, np.nextafter(mids.astype(np.float32), np.float32(0)),
                          np.nextafter(mids.astype(np.float32), np.float32(1e9)), [448.0, 460.0, 464.0, 1e6]])
    rng = np.random.default_rng(5)
    pts = np.concatenate([pts, rng.uniform(0, 500, 200000), rng.uniform(0, 2.0**-5, 50000),
                          2.0 ** rng.uniform(-12, 9, 100000)]).astype(np.float32)
    pts = np.concatenate([pts, -pts, [np.inf, -np.inf, np.nan, -0.0]]).astype(np.float32)
    np.testing.assert_array_equal(_branchfree_e4m3(pts), nm.e4m3fn_encode(pts))
