"""Pins the CPU oracle (oracle/attn_oracle.py) before it is trusted.

Every function of the oracle is checked against something it does not
restate: brute-force loops, torch's float64 SDPA + autograd, finite
differences, closed forms and invariants, and golden vectors written by
torch (tests/golden/make_golden.py).  The last group plants mistakes in a copy
of the oracle, on the CPU, and shows that these checks catch them.
"""
import hashlib
import math
import os

import numpy as np
import pytest
import torch

from oracle import attn_oracle as orc

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def rnd(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape).astype(np.float64)


def torch_ref(q, k, v, do, scale, causal):
    tq = torch.tensor(q, dtype=torch.float64, requires_grad=True)
    tk = torch.tensor(k, dtype=torch.float64, requires_grad=True)
    tv = torch.tensor(v, dtype=torch.float64, requires_grad=True)
    o = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, is_causal=causal, scale=scale)
    o.backward(torch.tensor(do, dtype=torch.float64))
    return o.detach().numpy(), tq.grad.numpy(), tk.grad.numpy(), tv.grad.numpy()


# ---------------------------------------------------------------- bf16 helpers

def test_bf16_rne_matches_torch():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(100000).astype(np.float32) * 10,
        np.array([0.0, -0.0, 1.0, -1.0, np.inf, -np.inf, 1e-40, -1e-40, 3.4e38, 1.00390625,
                  1.01171875, 1.0078125 + 2 ** -9], dtype=np.float32),
        # exact ties: bit 15 set, lower bits zero, both parities of bit 16
        (np.arange(0x3F800000, 0x3F800000 + 2 ** 18, 0x8000, dtype=np.uint32) | 0x8000).view(np.float32),
    ])
    ours = orc.bf16_bits(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(ours, ref)
    back = orc.bf16_to_f32(ours)
    np.testing.assert_array_equal(back, torch.from_numpy(x).to(torch.bfloat16).float().numpy())


def test_bf16_nan_stays_nan():
    x = np.array([np.nan, -np.nan], dtype=np.float32)
    assert np.all(np.isnan(orc.bf16_round(x)))


# ---------------------------------------------------------------- seeded inputs

def test_seeded_inputs_shapes_and_bf16_exact():
    for cid in (1, 2, 3):
        cfg = orc.CONFIGS[cid]
        x = orc.seeded_inputs(cfg)
        assert x["q"].shape == (cfg.B, cfg.H, cfg.Lq, cfg.d)
        assert x["k"].shape == (cfg.B, cfg.H, cfg.Lk, cfg.d)
        assert ("do" in x) == cfg.backward
        for a in x.values():
            assert a.dtype == np.float32
            if cfg.dtype == "bf16":
                np.testing.assert_array_equal(a, orc.bf16_round(a))
    x3 = orc.seeded_inputs(orc.CONFIGS[3])
    # c3 scales Q/K/V by 0.5 but not dO
    assert 0.4 < float(np.std(x3["q"])) < 0.6 and 0.9 < float(np.std(x3["do"])) < 1.1


def test_config_flop_formula():
    c5 = orc.CONFIGS[5]
    assert math.isclose(c5.fwd_flops() + c5.bwd_flops(), 1.6493e12, rel_tol=1e-4)
    c2 = orc.CONFIGS[2]
    assert math.isclose(c2.fwd_flops() + c2.bwd_flops(), 3.221e9, rel_tol=1e-3)
    c3 = orc.CONFIGS[3]
    assert math.isclose(c3.fwd_flops() + c3.bwd_flops(), 1.031e11, rel_tol=1e-3)
    assert orc.CONFIGS[1].fwd_flops() == 5.24288e5


# ---------------------------------------------------------------- brute force

def brute_fwd(q, k, v, scale, causal):
    Lq, d = q.shape
    Lk = k.shape[0]
    o = np.zeros((Lq, v.shape[1]))
    lse = np.zeros(Lq)
    for i in range(Lq):
        s = []
        for j in range(Lk):
            if causal and j > i:
                s.append(-math.inf)
                continue
            acc = 0.0
            for t in range(d):
                acc += float(q[i, t]) * float(k[j, t])
            s.append(acc * scale)
        m = max(s)
        e = [math.exp(x - m) for x in s]
        z = sum(e)
        lse[i] = m + math.log(z)
        for j in range(Lk):
            if e[j]:
                o[i] += (e[j] / z) * v[j].astype(np.float64)
    return o, lse


@pytest.mark.parametrize("causal", [False, True])
def test_bruteforce_c1_size(causal):
    cfg = orc.CONFIGS[1]
    x = orc.seeded_inputs(cfg)
    q, k, v = x["q"][0, 0], x["k"][0, 0], x["v"][0, 0]
    o, lse = orc.attn_fwd_f64(q, k, v, cfg.scale, causal)
    ob, lb = brute_fwd(q, k, v, cfg.scale, causal)
    np.testing.assert_allclose(o, ob, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(lse, lb, rtol=1e-12, atol=1e-12)


# ---------------------------------------------------------------- golden vectors

def test_golden_c1_matches_oracle():
    g = np.load(os.path.join(GOLDEN, "c1_fwd.npz"))
    cfg = orc.CONFIGS[1]
    x = orc.seeded_inputs(cfg)
    for n in ("q", "k", "v"):
        np.testing.assert_array_equal(x[n], g[n])
        assert hashlib.sha256(x[n].tobytes()).hexdigest() == str(g["sha_" + n])
    assert float(g["scale"]) == cfg.scale
    o, lse = orc.attn_fwd_f64(g["q"], g["k"], g["v"], cfg.scale, False)
    np.testing.assert_allclose(o, g["o"], rtol=1e-12, atol=1e-13)
    np.testing.assert_allclose(lse, g["lse"], rtol=1e-12, atol=1e-13)


def test_golden_c2_matches_oracle():
    g = np.load(os.path.join(GOLDEN, "c2_fwdbwd.npz"))
    cfg = orc.CONFIGS[2]
    x = orc.seeded_inputs(cfg)
    for n in ("q", "k", "v", "do"):
        assert hashlib.sha256(x[n].tobytes()).hexdigest() == str(g["sha_" + n]), n
    o, lse = orc.attn_fwd_f64(x["q"], x["k"], x["v"], cfg.scale, False)
    dq, dk, dv = orc.attn_bwd_f64(x["q"], x["k"], x["v"], x["do"], cfg.scale, False)
    full = dict(o=o, lse=lse, dq=dq, dk=dk, dv=dv)
    for n, a in full.items():
        heads = np.stack([a[b, h] for b, h in g["heads"]])
        assert orc.max_rel_err(heads, g[n + "_heads"]) < 1e-6, n
        assert math.isclose(float(a.sum()), float(g[n + "_sum"]), rel_tol=1e-9, abs_tol=1e-9), n
        assert math.isclose(float(np.abs(a).sum()), float(g[n + "_abssum"]), rel_tol=1e-11), n


# ---------------------------------------------------------------- library cross-check

@pytest.mark.parametrize("shape,causal", [
    ((2, 3, 37, 32), False), ((2, 3, 37, 32), True), ((1, 2, 64, 64), True),
    ((1, 1, 130, 128), True), ((1, 2, 1, 64), False), ((1, 1, 65, 16), False),
])
def test_oracle_vs_torch_sdpa(shape, causal):
    q, k, v, do = (rnd(shape, s) for s in range(4))
    scale = 1.0 / math.sqrt(shape[-1])
    o, _ = orc.attn_fwd_f64(q, k, v, scale, causal)
    dq, dk, dv = orc.attn_bwd_f64(q, k, v, do, scale, causal)
    to, tdq, tdk, tdv = torch_ref(q, k, v, do, scale, causal)
    for a, b in ((o, to), (dq, tdq), (dk, tdk), (dv, tdv)):
        np.testing.assert_allclose(a, b, rtol=1e-10, atol=1e-11)


# ---------------------------------------------------------------- finite differences

@pytest.mark.parametrize("causal", [False, True])
def test_backward_finite_differences(causal):
    L, d = 6, 4
    q, k, v, do = (rnd((L, d), 10 + s) for s in range(4))
    scale = 0.7

    def loss(q_, k_, v_):
        return float(np.sum(orc.attn_fwd_f64(q_, k_, v_, scale, causal)[0] * do))

    dq, dk, dv = orc.attn_bwd_f64(q, k, v, do, scale, causal)
    h = 1e-6
    for arr, grad in ((q, dq), (k, dk), (v, dv)):
        num = np.zeros_like(arr)
        for idx in np.ndindex(arr.shape):
            old = arr[idx]
            arr[idx] = old + h
            lp = loss(q, k, v)
            arr[idx] = old - h
            lm = loss(q, k, v)
            arr[idx] = old
            num[idx] = (lp - lm) / (2 * h)
        np.testing.assert_allclose(grad, num, rtol=1e-6, atol=1e-8)


# ---------------------------------------------------------------- closed forms

def test_causal_first_row_is_v0():
    q, k, v = (rnd((50, 32), s) for s in range(3))
    o, lse = orc.attn_fwd_f64(q, k, v, 0.3, True)
    np.testing.assert_allclose(o[0], v[0], rtol=0, atol=1e-15)
    assert math.isclose(lse[0], 0.3 * float(q[0] @ k[0]), rel_tol=1e-13)


@pytest.mark.parametrize("causal", [False, True])
def test_constant_scores_mean_of_v(causal):
    L, d = 40, 16
    q = np.zeros((L, d))
    k, v = rnd((L, d), 1), rnd((L, d), 2)
    o, lse = orc.attn_fwd_f64(q, k, v, 0.25, causal)
    for i in range(L):
        n = i + 1 if causal else L
        np.testing.assert_allclose(o[i], v[:n].mean(axis=0), rtol=1e-12, atol=1e-14)
        assert math.isclose(lse[i], math.log(n), rel_tol=1e-13)


@pytest.mark.parametrize("causal", [False, True])
def test_probability_rows_sum_to_one(causal):
    q, k = rnd((33, 8), 3), rnd((33, 8), 4)
    p = orc.attn_probs_f64(q, k, 0.9, causal)
    np.testing.assert_allclose(p.sum(axis=-1), 1.0, rtol=1e-14)
    if causal:
        assert np.all(p[np.triu_indices(33, 1)] == 0)


@pytest.mark.parametrize("causal", [False, True])
def test_shift_invariance_and_sum_of_ds(causal):
    """Adding u to every key row adds q_i.u to row i of S (constant in j):
    O is unchanged, and dQ = s dS K changes by s (sum_j dS_ij) u = 0."""
    L, d = 29, 8
    q, k, v, do = (rnd((L, d), 20 + s) for s in range(4))
    u = rnd((d,), 99)
    o1, _ = orc.attn_fwd_f64(q, k, v, 0.5, causal)
    o2, _ = orc.attn_fwd_f64(q, k + u, v, 0.5, causal)
    np.testing.assert_allclose(o1, o2, rtol=1e-11, atol=1e-12)
    dq1, _, _ = orc.attn_bwd_f64(q, k, v, do, 0.5, causal)
    dq2, _, _ = orc.attn_bwd_f64(q, k + u, v, do, 0.5, causal)
    np.testing.assert_allclose(dq1, dq2, rtol=1e-10, atol=1e-11)


@pytest.mark.parametrize("causal", [False, True])
def test_constant_v_backward(causal):
    L, d = 21, 8
    q, k, do = rnd((L, d), 5), rnd((L, d), 6), rnd((L, d), 7)
    v = np.tile(rnd((d,), 8), (L, 1))
    dq, dk, dv = orc.attn_bwd_f64(q, k, v, do, 0.4, causal)
    np.testing.assert_allclose(dq, 0, atol=1e-13)
    np.testing.assert_allclose(dk, 0, atol=1e-13)
    p = orc.attn_probs_f64(q, k, 0.4, causal)
    np.testing.assert_allclose(dv, p.T @ do, rtol=1e-13, atol=1e-14)


def test_causal_independence_of_future():
    L, d = 24, 8
    q, k, v, do = (rnd((L, d), 30 + s) for s in range(4))
    o1, _ = orc.attn_fwd_f64(q, k, v, 0.5, True)
    dq1, dk1, dv1 = orc.attn_bwd_f64(q, k, v, do, 0.5, True)
    i = 10
    k2, v2 = k.copy(), v.copy()
    k2[i + 1:] += 3.0
    v2[i + 1:] -= 2.0
    o2, _ = orc.attn_fwd_f64(q, k2, v2, 0.5, True)
    np.testing.assert_allclose(o1[:i + 1], o2[:i + 1], rtol=1e-13, atol=1e-14)
    # dK/dV row j only receives contributions from queries >= j
    q3, do3 = q.copy(), do.copy()
    q3[:i] += 1.5
    do3[:i] *= -2.0
    _, dk3, dv3 = orc.attn_bwd_f64(q3, k, v, do3, 0.5, True)
    np.testing.assert_allclose(dk1[i:], dk3[i:], rtol=1e-12, atol=1e-13)
    np.testing.assert_allclose(dv1[i:], dv3[i:], rtol=1e-12, atol=1e-13)


# ---------------------------------------------------------------- decode

def test_decode_equals_forward_and_split_merge():
    q = rnd((2, 3, 1, 64), 40)
    k, v = rnd((2, 3, 300, 64), 41), rnd((2, 3, 300, 64), 42)
    o, lse = orc.attn_decode_f64(q, k, v, 0.125)
    of, lf = orc.attn_fwd_f64(q, k, v, 0.125, False)
    np.testing.assert_array_equal(o, of)
    np.testing.assert_array_equal(lse, lf)
    for splits in (1, 2, 3, 7, 300):
        os_, ls_ = orc.decode_split_merge_f64(q, k, v, 0.125, splits)
        np.testing.assert_allclose(os_, o, rtol=1e-12, atol=1e-13)
        np.testing.assert_allclose(ls_, lse, rtol=1e-13)
    to, _, _, _ = torch_ref(q, k, v, np.zeros_like(q), 0.125, False)
    np.testing.assert_allclose(o, to, rtol=1e-11, atol=1e-12)


# ---------------------------------------------------------------- fp32 composition

@pytest.mark.parametrize("causal", [False, True])
def test_fp32_composition_agrees_with_f64(causal):
    shape = (2, 2, 96, 64)
    q, k, v, do = (rnd(shape, 50 + s).astype(np.float32) for s in range(4))
    scale = float(np.float32(1 / 8))
    o32 = orc.composition_fwd_f32(q, k, v, scale, causal)
    dq32, dk32, dv32 = orc.composition_bwd_f32(q, k, v, do, scale, causal)
    assert o32.dtype == np.float32 and dq32.dtype == np.float32
    o, _ = orc.attn_fwd_f64(q, k, v, scale, causal)
    dq, dk, dv = orc.attn_bwd_f64(q, k, v, do, scale, causal)
    for a, b in ((o32, o), (dq32, dq), (dk32, dk), (dv32, dv)):
        assert orc.max_rel_err(a, b) < 1e-5


def test_error_metrics():
    ref = np.array([1.0, -4.0, 2.0])
    assert orc.max_rel_err(ref + np.array([0, 0.4, 0]), ref) == pytest.approx(0.1)
    assert orc.max_rel_err(np.zeros(0), np.zeros(0)) == 0.0
    assert orc.elem_rel_err(ref * 1.01, ref) == pytest.approx(0.01, rel=1e-5)


# ---------------------------------------------------------------- planted mistakes

def _broken_fwd(kind):
    def f(q, k, v, scale, causal):
        q = np.asarray(q, np.float64)
        k = np.asarray(k, np.float64)
        v = np.asarray(v, np.float64)
        sc = 1.0 if kind == "no_scale" else scale
        kk = k[..., ::-1, :] if kind == "key_order" else k
        s = np.matmul(q, np.swapaxes(kk, -1, -2)) * sc
        if causal:
            diag = 0 if kind == "mask_off_by_one" else 1
            s = np.where(np.triu(np.ones(s.shape[-2:], bool), k=diag), -np.inf, s)
        with np.errstate(invalid="ignore"):  # the off-by-one mask empties row 0: NaN, as it should
            p = np.exp(s - s.max(-1, keepdims=True))
            p /= p.sum(-1, keepdims=True)
        return np.matmul(p, v)
    return f


@pytest.mark.parametrize("kind", ["no_scale", "key_order", "mask_off_by_one"])
def test_planted_forward_mistakes_are_caught(kind):
    g = np.load(os.path.join(GOLDEN, "c1_fwd.npz"))
    cfg = orc.CONFIGS[1]
    causal = kind == "mask_off_by_one"
    f = _broken_fwd(kind)
    if causal:
        q, k, v = (rnd((40, 16), s) for s in range(3))
        o_bad = f(q, k, v, 0.25, True)
        o_good = brute_fwd(q, k, v, 0.25, True)[0]
    else:
        o_bad = f(g["q"], g["k"], g["v"], cfg.scale, False)
        o_good = g["o"]
    assert orc.max_rel_err(o_bad, o_good) > 1e-3


def test_planted_backward_mistakes_are_caught():
    """A transposed operand in dK or a sign error in dS shows in the torch
    cross-check and the finite-difference check."""
    shape = (1, 1, 12, 8)
    q, k, v, do = (rnd(shape, 60 + s) for s in range(4))
    p = orc.attn_probs_f64(q, k, 0.5, False)
    dp = do @ np.swapaxes(v, -1, -2)
    ds = p * (dp - np.sum(p * dp, -1, keepdims=True))
    dk_bad_transpose = 0.5 * (ds @ q)              # dS instead of dS^T
    ds_bad_sign = p * (dp + np.sum(p * dp, -1, keepdims=True))
    dq_bad_sign = 0.5 * (ds_bad_sign @ k)
    _, tdq, tdk, _ = torch_ref(q, k, v, do, 0.5, False)
    assert orc.max_rel_err(dk_bad_transpose, tdk) > 1e-3
    assert orc.max_rel_err(dq_bad_sign, tdq) > 1e-3


# ---------------------------------------------------------------- row softmax

def _brute_softmax(x):
    """Row by row with math.exp: the textbook definition, no max shift."""
    out = np.empty_like(x, dtype=np.float64)
    for idx in np.ndindex(x.shape[:-1]):
        row = [math.exp(float(v)) for v in x[idx]]
        s = sum(row)
        out[idx] = [r / s for r in row]
    return out


def test_softmax_oracle_matches_brute_force_and_torch():
    x = rnd((5, 3, 17), 70)
    ref = orc.softmax_rows_f64(x)
    assert orc.max_rel_err(ref, _brute_softmax(x)) < 1e-14
    t = torch.softmax(torch.tensor(x, dtype=torch.float64), dim=-1).numpy()
    assert orc.max_rel_err(ref, t) < 1e-14


def test_softmax_oracle_closed_forms():
    x = rnd((64, 33), 71)
    p = orc.softmax_rows_f64(x)
    np.testing.assert_allclose(p.sum(-1), 1.0, rtol=0, atol=1e-14)          # rows sum to one
    np.testing.assert_allclose(orc.softmax_rows_f64(x + rnd((64, 1), 72) * 50), p, rtol=1e-12, atol=1e-15)  # shift
    np.testing.assert_array_equal(orc.softmax_rows_f64(np.full((3, 7), 2.5)), np.full((3, 7), 1 / 7))  # constant row
    two = rnd((100, 2), 73)
    np.testing.assert_allclose(orc.softmax_rows_f64(two)[:, 0], 1 / (1 + np.exp(two[:, 1] - two[:, 0])), rtol=1e-13)
    # large magnitudes: the max shift keeps it finite where the textbook form overflows
    big = np.array([[1000.0, 999.0, -1000.0]])
    np.testing.assert_allclose(orc.softmax_rows_f64(big)[0], [1 / (1 + math.exp(-1)), 1 / (1 + math.e), 0.0], rtol=1e-14)
    # -inf entries get exactly 0; a row of -inf is NaN, as the reference's x - max gives
    m = orc.softmax_rows_f64(np.array([[0.0, -np.inf, 0.0], [-np.inf, -np.inf, -np.inf]]))
    np.testing.assert_array_equal(m[0], [0.5, 0.0, 0.5])
    assert np.isnan(m[1]).all()


def test_softmax_reference_order_f32_agrees_with_f64():
    x = (rnd((300, 1000), 74) * 4).astype(np.float32)
    ref = orc.softmax_rows_f64(x)
    r32 = orc.softmax_rows_ref_f32(x)
    assert r32.dtype == np.float32
    assert orc.max_rel_err(r32, ref) < 1e-6


def test_planted_softmax_mistakes_are_caught():
    """Normalising over the wrong axis or dropping the max shift shows."""
    x = rnd((8, 40), 75) * 3
    ref = _brute_softmax(x)
    wrong_axis = np.exp(x - x.max(0, keepdims=True)) / np.exp(x - x.max(0, keepdims=True)).sum(0, keepdims=True)
    assert orc.max_rel_err(wrong_axis, ref) > 1e-3
    with np.errstate(over="ignore", invalid="ignore"):
        no_shift_big = np.exp(x * 300) / np.exp(x * 300).sum(-1, keepdims=True)  # overflows to NaN
    assert not np.isfinite(no_shift_big).all()
    assert np.isfinite(orc.softmax_rows_f64(x * 300)).all()


# ---------------------------------------------------------------- GEMM (cudaGemm contract)

def _brute_gemm(ta, tb, alpha, A, B, beta, C):
    """Element by element from the contract's index formulas (row-major, lda = k or m, ldb = n or k)."""
    m = A.shape[1] if ta else A.shape[0]
    k = A.shape[0] if ta else A.shape[1]
    n = B.shape[0] if tb else B.shape[1]
    out = np.zeros((m, n))
    for i in range(m):
        for j in range(n):
            acc = 0.0
            for p in range(k):
                a = A[p, i] if ta else A[i, p]
                b = B[j, p] if tb else B[p, j]
                acc += a * b
            out[i, j] = alpha * acc + (beta * C[i, j] if beta != 0 else 0.0)
    return out


@pytest.mark.parametrize("ta", [False, True])
@pytest.mark.parametrize("tb", [False, True])
def test_gemm_oracle_matches_brute_force(ta, tb):
    m, n, k = 5, 7, 3
    A = rnd((k, m) if ta else (m, k), 80)
    B = rnd((n, k) if tb else (k, n), 81)
    C = rnd((m, n), 82)
    for alpha, beta in [(1.0, 0.0), (0.5, 2.0), (-1.25, 1.0)]:
        np.testing.assert_allclose(orc.gemm_f64(ta, tb, alpha, A, B, beta, C),
                                   _brute_gemm(ta, tb, alpha, A, B, beta, C), rtol=1e-14, atol=1e-14)


def test_gemm_oracle_identities():
    A, B = rnd((40, 30), 83), rnd((30, 20), 84)
    ab = orc.gemm_f64(False, False, 1.0, A, B, 0.0)
    np.testing.assert_allclose(ab, (torch.tensor(A) @ torch.tensor(B)).numpy(), rtol=1e-13)
    # (A B)^T = B^T A^T through the transpose flags on the stored matrices
    np.testing.assert_allclose(orc.gemm_f64(True, True, 1.0, B, A, 0.0), ab.T, rtol=1e-13)
    # identity, linearity in alpha, beta = 0 ignores a NaN C
    np.testing.assert_allclose(orc.gemm_f64(False, False, 1.0, A, np.eye(30), 0.0), A, rtol=0, atol=0)
    np.testing.assert_allclose(orc.gemm_f64(False, False, 3.0, A, B, 0.0), 3 * ab, rtol=1e-14)
    assert np.isfinite(orc.gemm_f64(False, False, 1.0, A, B, 0.0, np.full((40, 20), np.nan))).all()
    # k = 0: only beta C remains
    C = rnd((4, 6), 85)
    np.testing.assert_allclose(orc.gemm_f64(False, False, 1.0, np.zeros((4, 0)), np.zeros((0, 6)), 2.0, C), 2 * C)


def test_planted_gemm_mistakes_are_caught():
    """Ignoring a transpose flag or swapping the operands shows."""
    A, B = rnd((6, 6), 86), rnd((6, 6), 87)
    good = _brute_gemm(True, False, 1.0, A, B, 0.0, None)
    assert orc.max_rel_err(orc.gemm_f64(False, False, 1.0, A, B, 0.0), good) > 1e-3
    assert orc.max_rel_err(orc.gemm_f64(True, False, 1.0, B, A, 0.0), good) > 1e-3


def test_dq_dk_contraction_identity_and_its_power():
    """sum_i dQ_i . Q_i = sum_j dK_j . K_j per head (both are
    s sum_ij dS_ij q_i . k_j): holds for the oracle, causal or not, and fails
    when dQ of one head is swapped with another's (the mistake the GPU tests
    use this identity to catch on heads the oracle does not sample)."""
    rng = np.random.default_rng(31)
    for causal in (False, True):
        q, k, v, do = (rng.standard_normal((2, 3, 40, 32)) for _ in range(4))
        dq, dk, _ = orc.attn_bwd_f64(q, k, v, do, 0.2, causal)
        lhs = np.einsum("bhld,bhld->bh", dq, q)
        rhs = np.einsum("bhld,bhld->bh", dk, k)
        norm = np.einsum("bhld,bhld->bh", np.abs(dq), np.abs(q)).max()
        assert np.abs(lhs - rhs).max() / norm < 1e-12
        bad = dq.copy()
        bad[0, 1], bad[1, 2] = dq[1, 2], dq[0, 1]
        lhs_bad = np.einsum("bhld,bhld->bh", bad, q)
        assert np.abs(lhs_bad - rhs).max() / norm > 2e-2
