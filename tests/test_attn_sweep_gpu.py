"""Seeded random sweep of the attention entry points (forward, backward,
decode; fp32 and bf16) against the float64 oracle, beyond the fixed shapes of
test_attn_gpu.py: random batch / head counts (16 of the cases over head
counts that are multiples of 8), lengths from 1 to 700 or 1500 (ragged
against every tile size, Lq != Lk when not causal), every head dim, and input
scales from 0.25 to 4, so that the softmax ranges from nearly uniform to
nearly one-hot (score spreads far past the forward's lazy-rescale threshold
of 8 in the log2 domain, which moves the running max mid-row).

Six bf16 d = 128 cases lie around 2048 keys, where causal heads switch between
the two dK/dV kernels.

A few structured inputs pin behaviour a random draw rarely reaches:
identical keys (uniform weights: O = mean of V, LSE = ln(#keys) + s q.k),
dO = 0 (all gradients exactly 0), and one key far larger than the rest.

Bar (normwise max|x - ref| / max|ref|, as test_attn_gpu.py): fp32 <= 1e-4,
bf16 inputs with fp32 accumulation <= 2e-2.
"""
import math
import sys

import numpy as np
import pytest

from oracle import attn_oracle as orc

pytestmark = pytest.mark.gpu

TOL = orc.TOL


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def capi():
    import tt_capi

    assert tt_capi.lib().device_count() >= 1, "no HIP device visible"
    return tt_capi


def _cases(n=24, seed=2024, heads=None, lmax=700, base=5000):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        d = int(rng.choice([32, 64, 128]))
        causal = bool(rng.integers(0, 2))
        Lq = int(rng.integers(1, lmax + 1))
        Lk = Lq if causal else int(rng.integers(1, lmax + 1))
        if heads is None:
            B, H = int(rng.integers(1, 4)), int(rng.integers(1, 4))
        else:
            B, H = heads[int(rng.integers(0, len(heads)))]
        sigma = float(rng.choice([0.25, 1.0, 2.0, 4.0]))
        dtype = "bf16" if i % 2 else "f32"
        out.append((B, H, Lq, Lk, d, causal, sigma, dtype, base + i))
    return out


CASES = _cases()
# head counts that are multiples of 8: the launches' per-XCD head groups and,
# for causal d <= 64, the held-back cheap tiles (attn_tiles.h)
CASES += _cases(16, seed=2025, heads=[(1, 8), (2, 8), (1, 16), (3, 8)], lmax=1500, base=6000)


def _switch_cases(n=6, seed=2026, base=7000):
    """bf16 d = 128 around 2048 keys, where causal heads move from the
    two-waves-per-SIMD dK/dV kernel (Lk <= 2048) to the persistent one."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        causal = i < 4
        Lq = int(rng.integers(1990, 2110))
        Lk = Lq if causal else int(rng.integers(1990, 2110))
        B, H = [(1, 2), (1, 3), (2, 1)][int(rng.integers(0, 3))]
        out.append((B, H, Lq, Lk, 128, causal, float(rng.choice([0.5, 1.0, 2.0])), "bf16", base + i))
    return out


CASES += _switch_cases()


def _inputs(B, H, Lq, Lk, d, sigma, dtype, seed):
    rng = np.random.default_rng(seed)
    x = {
        "q": (sigma * rng.standard_normal((B, H, Lq, d))).astype(np.float32),
        "k": (sigma * rng.standard_normal((B, H, Lk, d))).astype(np.float32),
        "v": rng.standard_normal((B, H, Lk, d)).astype(np.float32),
        "do": rng.standard_normal((B, H, Lq, d)).astype(np.float32),
    }
    if dtype == "bf16":
        x = {n: orc.bf16_round(a) for n, a in x.items()}
    return x


def _fwd_bwd(capi, x, dtype, scale, causal):
    B, H, Lq, d = x["q"].shape
    bq, bk, bv = (capi.DeviceBuffer.from_numpy(x[n], dtype) for n in ("q", "k", "v"))
    bo = capi.DeviceBuffer(x["q"].shape, dtype)
    bl = capi.DeviceBuffer((B, H, Lq), "f32")
    capi.attn_fwd(bq, bk, bv, bo, bl, scale, causal)
    bdo = capi.DeviceBuffer.from_numpy(x["do"], dtype)
    gq = capi.DeviceBuffer(x["q"].shape, dtype)
    gk = capi.DeviceBuffer(x["k"].shape, dtype)
    gv = capi.DeviceBuffer(x["v"].shape, dtype)
    capi.attn_bwd(bq, bk, bv, bo, bl, bdo, gq, gk, gv, scale, causal)
    capi.lib().sync()
    return bo.download(), bl.download(), gq.download(), gk.download(), gv.download()


def _check(name, x, ref, tol):
    err = orc.max_rel_err(x, ref)
    _say(f"  {name}: max-rel-err {err:.3e} (tol {tol:g})")
    assert err <= tol, f"{name}: {err:.3e} > {tol:g}"


@pytest.mark.parametrize("case", CASES, ids=[f"{c[7]}-B{c[0]}H{c[1]}-{c[2]}x{c[3]}-d{c[4]}-{'c' if c[5] else 'n'}-s{c[6]}"
                                             for c in CASES])
def test_random_fwd_bwd(capi, case):
    B, H, Lq, Lk, d, causal, sigma, dtype, seed = case
    _say(f"sweep {case}")
    x = _inputs(B, H, Lq, Lk, d, sigma, dtype, seed)
    scale = float(np.float32(1.0 / math.sqrt(d)))
    tol = TOL[dtype]
    o, lse, dq, dk, dv = _fwd_bwd(capi, x, dtype, scale, causal)
    o_ref, l_ref = orc.attn_fwd_f64(x["q"], x["k"], x["v"], scale, causal)
    rq, rk, rv = orc.attn_bwd_f64(x["q"], x["k"], x["v"], x["do"], scale, causal)
    _check("O", o, o_ref, tol)
    _check("LSE", lse, l_ref, tol)
    _check("dQ", dq, rq, tol)
    _check("dK", dk, rk, tol)
    _check("dV", dv, rv, tol)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("seed", [1, 2, 3])
def test_random_decode(capi, dtype, seed):
    rng = np.random.default_rng(900 + seed)
    d = int(rng.choice([32, 64, 128]))
    B, H, Lkv = int(rng.integers(1, 5)), int(rng.integers(1, 5)), int(rng.integers(1, 3000))
    sigma = float(rng.choice([0.5, 2.0, 4.0]))
    _say(f"decode sweep {dtype} B={B} H={H} Lkv={Lkv} d={d} sigma={sigma}")
    q = (sigma * rng.standard_normal((B, H, 1, d))).astype(np.float32)
    k = (sigma * rng.standard_normal((B, H, Lkv, d))).astype(np.float32)
    v = rng.standard_normal((B, H, Lkv, d)).astype(np.float32)
    if dtype == "bf16":
        q, k, v = orc.bf16_round(q), orc.bf16_round(k), orc.bf16_round(v)
    scale = float(np.float32(1.0 / math.sqrt(d)))
    bq, bk, bv = (capi.DeviceBuffer.from_numpy(a, dtype) for a in (q, k, v))
    bo = capi.DeviceBuffer(q.shape, dtype)
    bl = capi.DeviceBuffer((B, H), "f32")
    capi.attn_decode(bq, bk, bv, bo, bl, scale)
    o_ref, l_ref = orc.attn_decode_f64(q, k, v, scale)
    _check("o", bo.download(), o_ref, TOL[dtype])
    _check("lse", bl.download(), l_ref[..., 0], TOL[dtype])


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("d", [64, 128])
def test_identical_keys_give_uniform_weights(capi, dtype, d):
    """Every key the same: P is uniform over the unmasked keys, so O_i is the
    mean of V over them and LSE_i = ln(n_i) + s q_i . k (closed form)."""
    B, H, L = 1, 2, 300
    x = _inputs(B, H, L, L, d, 1.0, dtype, 77 + d)
    x["k"][:] = x["k"][:, :, :1, :]
    scale = float(np.float32(1.0 / math.sqrt(d)))
    for causal in (False, True):
        o, lse, dq, dk, dv = _fwd_bwd(capi, x, dtype, scale, causal)
        v = x["v"].astype(np.float64)
        if causal:
            mean_v = np.cumsum(v, axis=2) / np.arange(1, L + 1)[None, None, :, None]
            n = np.arange(1, L + 1, dtype=np.float64)[None, None, :]
        else:
            mean_v = np.broadcast_to(v.mean(axis=2, keepdims=True), v.shape)
            n = np.full((1, 1, L), float(L))
        qk = np.einsum("bhid,bhd->bhi", x["q"].astype(np.float64), x["k"][:, :, 0, :].astype(np.float64))
        _check(f"O = mean V (causal={causal})", o, mean_v, TOL[dtype])
        _check(f"LSE = ln n + s q.k (causal={causal})", lse, np.log(n) + scale * qk, TOL[dtype])
        rq, rk, rv = orc.attn_bwd_f64(x["q"], x["k"], x["v"], x["do"], scale, causal)
        _check("dV", dv, rv, TOL[dtype])
        _check("dK", dk, rk, TOL[dtype])


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_zero_grad_out_gives_zero_gradients(capi, dtype):
    x = _inputs(2, 2, 256, 256, 128, 1.0, dtype, 31)
    x["do"][:] = 0
    scale = float(np.float32(1.0 / math.sqrt(128)))
    for causal in (False, True):
        _, _, dq, dk, dv = _fwd_bwd(capi, x, dtype, scale, causal)
        assert not dq.any() and not dk.any() and not dv.any()


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_dominant_key(capi, dtype):
    """Key 0 with entries of +-8 (the rest N(0, 1)): its score has a spread
    of 8 per row against 1 for the others, so each row's weights are nearly
    one-hot on key 0 or nearly ignore it -- the regime where the max
    subtraction and the running-max moves matter most; against the oracle."""
    d, L = 128, 200
    x = _inputs(1, 2, L, L, d, 1.0, dtype, 41)
    x["k"][:, :, 0, :] = 8.0 * np.sign(x["q"].sum(axis=2))
    if dtype == "bf16":
        x = {n: orc.bf16_round(a) for n, a in x.items()}
    scale = float(np.float32(1.0 / math.sqrt(d)))
    o, lse, dq, dk, dv = _fwd_bwd(capi, x, dtype, scale, False)
    o_ref, l_ref = orc.attn_fwd_f64(x["q"], x["k"], x["v"], scale, False)
    rq, rk, rv = orc.attn_bwd_f64(x["q"], x["k"], x["v"], x["do"], scale, False)
    for n, a, r in (("O", o, o_ref), ("LSE", lse, l_ref), ("dQ", dq, rq), ("dK", dk, rk), ("dV", dv, rv)):
        _check(n, a, r, TOL[dtype])


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("causal", [False, True])
def test_huge_logits(capi, dtype, causal):
    """Inputs of scale 10 (scores up to about +-1000, log2-domain jumps of
    hundreds): rows are one-hot up to rounding and the running max moves by
    far more than the forward's lazy-rescale threshold within a row; against
    the oracle.  (At scale 20, scores near +-3200, fp32 rounding of the score
    sums alone perturbs the weights by ~2e-4: the fp32 kernels measured
    1.4e-4 against float64 there, and the reference's own fp32 op chain
    8e-5.)"""
    d, L = 64, 300
    x = _inputs(1, 2, L, L, d, 10.0, dtype, 53 + int(causal))
    scale = float(np.float32(1.0 / math.sqrt(d)))
    o, lse, dq, dk, dv = _fwd_bwd(capi, x, dtype, scale, causal)
    o_ref, l_ref = orc.attn_fwd_f64(x["q"], x["k"], x["v"], scale, causal)
    rq, rk, rv = orc.attn_bwd_f64(x["q"], x["k"], x["v"], x["do"], scale, causal)
    assert np.isfinite(o).all() and np.isfinite(dq).all() and np.isfinite(dk).all() and np.isfinite(dv).all()
    for n, a, r in (("O", o, o_ref), ("LSE", lse, l_ref), ("dQ", dq, rq), ("dK", dk, rk), ("dV", dv, rv)):
        _check(n, a, r, TOL[dtype])


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("d", [64, 128])
def test_nan_in_one_query_row_stays_where_the_oracle_puts_it(capi, dtype, d):
    """A NaN in one query row (no mask): that row's O, LSE and dQ are NaN, so
    are the dK and dV rows of every key (through the row's dS and P), and
    every other value matches the oracle -- the positions the reference's op
    chain gives (NaN propagates through max, exp and the products).  Under a
    causal mask the reference also turns the row's masked weights into NaN
    (exp(-inf - NaN)) and so every key's dK / dV; these kernels never touch
    the key tiles wholly past a row's diagonal, whose dK / dV stay finite."""
    L, bad = 200, 137
    x = _inputs(1, 2, L, L, d, 1.0, dtype, 61 + d)
    x["q"][0, 1, bad, 5] = np.nan
    scale = float(np.float32(1.0 / math.sqrt(d)))
    for causal in (False,):
        o, lse, dq, dk, dv = _fwd_bwd(capi, x, dtype, scale, causal)
        o_ref, l_ref = orc.attn_fwd_f64(x["q"], x["k"], x["v"], scale, causal)
        rq, rk, rv = orc.attn_bwd_f64(x["q"], x["k"], x["v"], x["do"], scale, causal)
        for n, a, r in (("O", o, o_ref), ("LSE", lse, l_ref), ("dQ", dq, rq), ("dK", dk, rk), ("dV", dv, rv)):
            nan_ref = np.isnan(r)
            assert nan_ref.any() and (np.isnan(a) == nan_ref).all(), f"{n}: NaN positions differ (causal={causal})"
            _check(f"{n} (finite part, causal={causal})", np.where(nan_ref, 0, a), np.where(nan_ref, 0, r), TOL[dtype])
