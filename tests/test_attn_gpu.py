"""GPU parity tests: the HIP kernels, called through the C-ABI
(include/tt_attn.h via pku-aiprogramming_amd/tt_capi.py), against the CPU
oracle (oracle/attn_oracle.py, float64 ground truth) on seeded inputs.

Error metric (per output tensor): max|x - ref| / max|ref| with ref the
float64 oracle on the exact (bf16-rounded) inputs.  Tolerances, as stated by
the target: fp32 <= 1e-4, bf16 with fp32 accumulation <= 2e-2.

Full-size configs are checked on sampled heads against the oracle and, over
every head, through size-independent identities of the exact result:
  sum_j dV_j = sum_i dO_i      (rows of P sum to 1)
  sum_j dK_j = 0               (rows of dS sum to 0)
  sum_i dQ_i . Q_i = sum_j dK_j . K_j   (both s sum_ij dS_ij q_i . k_j)
  causal: O[0] = V[0] and LSE[0] = s q_0 . k_0
and every head of the bf16 result against the fp32 kernels on the same inputs.
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

    L = tt_capi.lib()
    assert L.device_count() >= 1, "no HIP device visible"
    return tt_capi


def _run_fwd(capi, x, dtype, scale, causal, want_lse=True):
    q, k, v = x["q"], x["k"], x["v"]
    B, H, Lq, d = q.shape
    dq = capi.DeviceBuffer.from_numpy(q, dtype)
    dk = capi.DeviceBuffer.from_numpy(k, dtype)
    dv = capi.DeviceBuffer.from_numpy(v, dtype)
    do = capi.DeviceBuffer(q.shape, dtype)
    dl = capi.DeviceBuffer((B, H, Lq), "f32") if want_lse else None
    capi.attn_fwd(dq, dk, dv, do, dl, scale, causal)
    capi.lib().sync()
    return dict(q=dq, k=dk, v=dv, o=do, lse=dl)


def _run_bwd(capi, bufs, dout, dtype, scale, causal):
    ddo = capi.DeviceBuffer.from_numpy(dout, dtype)
    gq = capi.DeviceBuffer(bufs["q"].shape, dtype)
    gk = capi.DeviceBuffer(bufs["k"].shape, dtype)
    gv = capi.DeviceBuffer(bufs["v"].shape, dtype)
    capi.attn_bwd(bufs["q"], bufs["k"], bufs["v"], bufs["o"], bufs["lse"], ddo, gq, gk, gv, scale, causal)
    capi.lib().sync()
    return gq.download(), gk.download(), gv.download()


def _check(name, x, ref, tol):
    err = orc.max_rel_err(x, ref)
    _say(f"  {name}: max-rel-err {err:.3e} (tol {tol:g})")
    assert err <= tol, f"{name}: {err:.3e} > {tol:g}"
    return err


# ------------------------------------------------------------------ configs

def test_c1_fp32_forward(capi):
    cfg = orc.CONFIGS[1]
    _say("c1: fp32 fwd B=1 H=1 L=64 d=32")
    g = np.load(orc_golden("c1_fwd.npz"))
    x = {n: g[n] for n in ("q", "k", "v")}
    b = _run_fwd(capi, x, "f32", cfg.scale, False)
    _check("O", b["o"].download(), g["o"], TOL["f32"])
    _check("LSE", b["lse"].download(), g["lse"], TOL["f32"])


def test_c2_fp32_fwd_bwd(capi):
    cfg = orc.CONFIGS[2]
    _say("c2: fp32 fwd+bwd B=8 H=8 L=256 d=64")
    x = orc.seeded_inputs(cfg)
    b = _run_fwd(capi, x, "f32", cfg.scale, False)
    o_ref, lse_ref = orc.attn_fwd_f64(x["q"], x["k"], x["v"], cfg.scale, False)
    _check("O", b["o"].download(), o_ref, TOL["f32"])
    _check("LSE", b["lse"].download(), lse_ref, TOL["f32"])
    dq, dk, dv = _run_bwd(capi, b, x["do"], "f32", cfg.scale, False)
    rq, rk, rv = orc.attn_bwd_f64(x["q"], x["k"], x["v"], x["do"], cfg.scale, False)
    _check("dQ", dq, rq, TOL["f32"])
    _check("dK", dk, rk, TOL["f32"])
    _check("dV", dv, rv, TOL["f32"])
    # the committed torch-written golden heads as a second anchor
    gd = np.load(orc_golden("c2_fwdbwd.npz"))
    for n, a in (("o", b["o"].download()), ("dq", dq), ("dk", dk), ("dv", dv)):
        heads = np.stack([a[i, j] for i, j in gd["heads"]])
        _check(f"golden {n}", heads, gd[n + "_heads"], TOL["f32"])


def _identities(name, x, o, lse, dq, dk, dv, scale, causal, tol):
    """Size-independent properties over every head (see module docstring)."""
    do = x["do"].astype(np.float64)
    sum_dv = dv.astype(np.float64).sum(axis=2)
    _check(f"{name} sum_j dV_j = sum_i dO_i", sum_dv, do.sum(axis=2), tol)
    # sum_j dK_j = 0: compare against the scale of dK itself
    sum_dk = np.abs(dk.astype(np.float64).sum(axis=2)).max()
    ref_scale = np.abs(dk.astype(np.float64)).sum(axis=2).max()
    _say(f"  {name} |sum_j dK_j| / sum_j |dK_j| = {sum_dk / ref_scale:.3e}")
    assert sum_dk <= tol * ref_scale
    # sum_i dQ_i . Q_i = sum_j dK_j . K_j (both are s sum_ij dS_ij q_i . k_j), per
    # head: ties dQ of every head to dK of the same head, so a dQ written to
    # the wrong head or computed from another head's rows fails
    lhs = np.einsum("bhld,bhld->bh", dq.astype(np.float64), x["q"].astype(np.float64))
    rhs = np.einsum("bhld,bhld->bh", dk.astype(np.float64), x["k"].astype(np.float64))
    norm = np.einsum("bhld,bhld->bh", np.abs(dq.astype(np.float64)), np.abs(x["q"].astype(np.float64))).max()
    err = np.abs(lhs - rhs).max() / norm
    _say(f"  {name} |sum dQ.Q - sum dK.K| / sum |dQ.Q| = {err:.3e}")
    assert err <= tol
    if causal:
        _check(f"{name} O[0] = V[0]", o[:, :, 0], x["v"][:, :, 0], tol)
        s00 = scale * np.einsum("bhd,bhd->bh", x["q"][:, :, 0].astype(np.float64), x["k"][:, :, 0].astype(np.float64))
        _check(f"{name} LSE[0] = s q0.k0", lse[:, :, 0], s00, tol)


def _sampled_heads(name, x, o, lse, dq, dk, dv, scale, causal, heads, tol):
    for (bb, hh) in heads:
        q, k, v = x["q"][bb, hh], x["k"][bb, hh], x["v"][bb, hh]
        o_ref, l_ref = orc.attn_fwd_f64(q, k, v, scale, causal)
        rq, rk, rv = orc.attn_bwd_f64(q, k, v, x["do"][bb, hh], scale, causal)
        _say(f" {name} head ({bb},{hh})")
        _check("O", o[bb, hh], o_ref, tol)
        _check("LSE", lse[bb, hh], l_ref, tol)
        _check("dQ", dq[bb, hh], rq, tol)
        _check("dK", dk[bb, hh], rk, tol)
        _check("dV", dv[bb, hh], rv, tol)


def _all_heads_vs_f32(capi, name, x, o, lse, dq, dk, dv, scale, causal, tol):
    """Every head of the bf16 result against the fp32 kernels' result on the
    same (bf16-valued) inputs: a second, independently tiled kernel family
    (128-query / 128-key workgroups on the fp32 MFMA, its own schedules),
    itself held to 1e-4 against the oracle elsewhere.  Per head and tensor,
    max|bf16 - f32| / max|f32| <= the bf16 tolerance, so a head whose rows the
    bf16 kernels mapped, masked or scaled wrongly fails even when it is not
    one of the sampled heads."""
    b32 = _run_fwd(capi, x, "f32", scale, causal)
    o32, l32 = b32["o"].download(), b32["lse"].download()
    q32, k32, v32 = _run_bwd(capi, b32, x["do"], "f32", scale, causal)
    worst = {}
    for n, a, r in (("O", o, o32), ("LSE", lse, l32), ("dQ", dq, q32), ("dK", dk, k32), ("dV", dv, v32)):
        a64, r64 = a.astype(np.float64), r.astype(np.float64)
        ax = tuple(range(2, a64.ndim))
        err = np.abs(a64 - r64).max(axis=ax) / np.maximum(np.abs(r64).max(axis=ax), 1e-30)
        bb, hh = np.unravel_index(int(np.argmax(err)), err.shape)
        worst[n] = (float(err.max()), int(bb), int(hh))
    _say(f"  {name} every head vs fp32 kernels: " + ", ".join(f"{n} {e:.2e} at ({b},{h})" for n, (e, b, h) in worst.items()))
    for n, (e, b, h) in worst.items():
        assert e <= tol, f"{name} {n} head ({b},{h}): {e:.3e} > {tol:g}"


def test_c3_bf16_causal_fwd_bwd(capi):
    cfg = orc.CONFIGS[3]
    _say("c3: bf16 causal fwd+bwd B=16 H=16 L=1024 d=64")
    x = orc.seeded_inputs(cfg)
    b = _run_fwd(capi, x, "bf16", cfg.scale, True)
    o, lse = b["o"].download(), b["lse"].download()
    dq, dk, dv = _run_bwd(capi, b, x["do"], "bf16", cfg.scale, True)
    _sampled_heads("c3", x, o, lse, dq, dk, dv, cfg.scale, True, [(0, 0), (7, 3), (15, 15)], TOL["bf16"])
    _identities("c3", x, o, lse, dq, dk, dv, cfg.scale, True, TOL["bf16"])
    _all_heads_vs_f32(capi, "c3", x, o, lse, dq, dk, dv, cfg.scale, True, TOL["bf16"])


def test_c5_bf16_causal_fwd_bwd(capi):
    cfg = orc.CONFIGS[5]
    _say("c5: bf16 causal fwd+bwd B=4 H=32 L=4096 d=128")
    x = orc.seeded_inputs(cfg)
    b = _run_fwd(capi, x, "bf16", cfg.scale, True)
    o, lse = b["o"].download(), b["lse"].download()
    dq, dk, dv = _run_bwd(capi, b, x["do"], "bf16", cfg.scale, True)
    _sampled_heads("c5", x, o, lse, dq, dk, dv, cfg.scale, True, [(0, 0), (3, 31)], TOL["bf16"])
    _identities("c5", x, o, lse, dq, dk, dv, cfg.scale, True, TOL["bf16"])
    _all_heads_vs_f32(capi, "c5", x, o, lse, dq, dk, dv, cfg.scale, True, TOL["bf16"])


def test_c4_bf16_decode(capi):
    """Full-size decode.  K/V (2^31 elements each) are filled on the device by
    the library's counter-based N(0,1) generator; sampled heads are downloaded
    and checked against the oracle, and every head against the forward kernel
    run with Lq = 1 (same inputs)."""
    cfg = orc.CONFIGS[4]
    B, H, Lkv, d = cfg.B, cfg.H, cfg.Lk, cfg.d
    _say("c4: bf16 decode B=64 H=32 Lkv=8192 d=128")
    q = capi.DeviceBuffer((B, H, 1, d), "bf16")
    k = capi.DeviceBuffer((B, H, Lkv, d), "bf16")
    v = capi.DeviceBuffer((B, H, Lkv, d), "bf16")
    q.fill_normal(40)
    k.fill_normal(41)
    v.fill_normal(42)
    o = capi.DeviceBuffer((B, H, 1, d), "bf16")
    lse = capi.DeviceBuffer((B, H), "f32")
    capi.attn_decode(q, k, v, o, lse, cfg.scale)
    o2 = capi.DeviceBuffer((B, H, 1, d), "bf16")
    lse2 = capi.DeviceBuffer((B, H, 1), "f32")
    capi.attn_fwd(q, k, v, o2, lse2, cfg.scale, False)
    capi.lib().sync()
    od, ld = o.download(), lse.download()
    _check("decode vs forward kernel O", od, o2.download(), TOL["bf16"])
    # The bf16 forward normalises by the sum of the bf16-rounded weights its
    # PV MFMAs apply (relative error <= 2^-9 against an fp32 sum); the decode
    # kernel sums in fp32.  The two LSEs agree to that bound; both are checked
    # against the float64 oracle below.
    _check("decode vs forward kernel LSE", ld, lse2.download()[..., 0], 2.0 ** -9)
    qh = q.download()
    # sampled heads: copy their K/V rows back (bh-contiguous slabs)
    for (bb, hh) in [(0, 0), (33, 17), (63, 31)]:
        bh = bb * H + hh
        slab = Lkv * d
        kb = np.empty(slab, np.uint16)
        vb = np.empty(slab, np.uint16)
        import ctypes as C
        capi.lib().call("tt_memcpy_d2h", kb.ctypes.data, C.c_void_p(k.ptr + 2 * bh * slab), 2 * slab)
        capi.lib().call("tt_memcpy_d2h", vb.ctypes.data, C.c_void_p(v.ptr + 2 * bh * slab), 2 * slab)
        kh = capi.bf16_to_f32(kb).reshape(Lkv, d)
        vh = capi.bf16_to_f32(vb).reshape(Lkv, d)
        o_ref, l_ref = orc.attn_decode_f64(qh[bb, hh], kh, vh, cfg.scale)
        _say(f" c4 head ({bb},{hh})")
        _check("o", od[bb, hh], o_ref, TOL["bf16"])
        _check("lse", ld[bb, hh], l_ref[0], TOL["bf16"])
    assert abs(float(np.std(qh)) - 1.0) < 0.05  # the generator is N(0,1)


def test_long_sequence_few_heads_bf16(capi):
    """L = 8192 with only two heads (B*H not a multiple of 8: no per-XCD head
    grouping; 64 query tiles per head): one
    head against the float64 oracle, both through the identities."""
    B, H, L, d = 1, 2, 8192, 128
    _say("long sequence: bf16 causal B=1 H=2 L=8192 d=128")
    rng = np.random.default_rng(8192)
    x = {n: orc.bf16_round(rng.standard_normal((B, H, L, d), dtype=np.float32)) for n in ("q", "k", "v", "do")}
    scale = float(np.float32(1.0 / math.sqrt(d)))
    b = _run_fwd(capi, x, "bf16", scale, True)
    o, lse = b["o"].download(), b["lse"].download()
    dq, dk, dv = _run_bwd(capi, b, x["do"], "bf16", scale, True)
    _identities("long", x, o, lse, dq, dk, dv, scale, True, TOL["bf16"])
    one = {n: a[:, 1:2] for n, a in x.items()}
    o_ref, l_ref = orc.attn_fwd_f64(one["q"], one["k"], one["v"], scale, True)
    _check("head 1 O", o[:, 1:2], o_ref, TOL["bf16"])
    _check("head 1 LSE", lse[:, 1:2], l_ref, TOL["bf16"])
    rq, rk, rv = orc.attn_bwd_f64(one["q"], one["k"], one["v"], one["do"], scale, True)
    _check("head 1 dQ", dq[:, 1:2], rq, TOL["bf16"])
    _check("head 1 dK", dk[:, 1:2], rk, TOL["bf16"])
    _check("head 1 dV", dv[:, 1:2], rv, TOL["bf16"])


PERSISTENT_SCHEDULES = [
    # (B, H, L): the d = 128 dK/dV kernel runs one workgroup per CU (256 on the
    # MI355X) over (256-key block, head) items.
    # 12 heads x 32 key blocks = 384 items; B*H % 8 != 0, so the items are
    # dealt over all workgroups without the per-XCD head grouping, in two
    # rounds, the second one ragged (128 items for 256 workgroups).
    (1, 12, 8192),
    # 24 heads x 16 key blocks = 384 items; B*H % 8 == 0, so each XCD owns 3
    # heads (48 items for its 32 workgroups): one full round and a ragged one.
    (3, 8, 4096),
]


@pytest.mark.parametrize("B,H,L", PERSISTENT_SCHEDULES)
def test_persistent_dkdv_schedules_bf16(capi, B, H, L):
    """The two regimes of the persistent dK/dV schedule that c5 (2048 items,
    eight full rounds with per-XCD head grouping) does not reach: every head
    against the fp32 kernels and through the identities, one head against the
    float64 oracle."""
    d = 128
    _say(f"persistent dK/dV schedule: bf16 causal B={B} H={H} L={L} d={d}")
    rng = np.random.default_rng(1000 * H + B)
    x = {n: orc.bf16_round(rng.standard_normal((B, H, L, d), dtype=np.float32)) for n in ("q", "k", "v", "do")}
    scale = float(np.float32(1.0 / math.sqrt(d)))
    b = _run_fwd(capi, x, "bf16", scale, True)
    o, lse = b["o"].download(), b["lse"].download()
    dq, dk, dv = _run_bwd(capi, b, x["do"], "bf16", scale, True)
    _identities("sched", x, o, lse, dq, dk, dv, scale, True, TOL["bf16"])
    _all_heads_vs_f32(capi, "sched", x, o, lse, dq, dk, dv, scale, True, TOL["bf16"])
    bb, hh = B - 1, H - 1  # the last head: its items come last in both schedules
    _sampled_heads("sched", x, o, lse, dq, dk, dv, scale, True, [(bb, hh)], TOL["bf16"])


# (B, H, L) of causal d = 128 launches on either side of the dK/dV kernel
# choice: up to 2048 keys the two-waves-per-SIMD kernel (32-query tiles at
# d = 128), beyond it the one-wave-per-SIMD persistent kernel.
D128_CAUSAL_DKDV_PATHS = [
    (2, 16, 2048),  # two-wave kernel, at the boundary
    (4, 8, 1000),   # two-wave kernel, a ragged last key and query tile
    (1, 8, 2056),   # one-wave kernel, just past the boundary (ragged)
]


@pytest.mark.parametrize("B,H,L", D128_CAUSAL_DKDV_PATHS)
def test_d128_causal_dkdv_paths_bf16(capi, B, H, L):
    """Both d = 128 dK/dV kernels near the length where the launcher switches
    between them: every head against the fp32 kernels and through the
    identities, two heads against the float64 oracle."""
    d = 128
    _say(f"d = 128 causal dK/dV path: bf16 B={B} H={H} L={L}")
    rng = np.random.default_rng(7000 + L)
    x = {n: orc.bf16_round(rng.standard_normal((B, H, L, d), dtype=np.float32)) for n in ("q", "k", "v", "do")}
    scale = float(np.float32(1.0 / math.sqrt(d)))
    b = _run_fwd(capi, x, "bf16", scale, True)
    o, lse = b["o"].download(), b["lse"].download()
    dq, dk, dv = _run_bwd(capi, b, x["do"], "bf16", scale, True)
    _identities("d128", x, o, lse, dq, dk, dv, scale, True, TOL["bf16"])
    _all_heads_vs_f32(capi, "d128", x, o, lse, dq, dk, dv, scale, True, TOL["bf16"])
    _sampled_heads("d128", x, o, lse, dq, dk, dv, scale, True, [(0, 0), (B - 1, H - 1)], TOL["bf16"])


DECODE_LONG_SPLITS = [
    # (B, H, Lkv, d): 512 heads -> five 2048-key splits per head, the last one
    # partial (808 keys), merged by the combine kernel
    (8, 64, 9000, 64),
    # 2048 heads -> one 3000-key split per head, written directly (no combine)
    (64, 32, 3000, 64),
]


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("B,H,Lkv,d", DECODE_LONG_SPLITS)
def test_decode_large_grid_ragged_last_split(capi, dtype, B, H, Lkv, d):
    """Grids large enough for splits longer than 1024 keys, ragged in their
    last split: every head against the forward kernel run with Lq = 1, and
    sampled heads against the oracle."""
    scale = float(np.float32(1.0 / math.sqrt(d)))
    _say(f"decode {dtype} B={B} H={H} Lkv={Lkv} d={d} (long splits, ragged last)")
    q = capi.DeviceBuffer((B, H, 1, d), dtype)
    k = capi.DeviceBuffer((B, H, Lkv, d), dtype)
    v = capi.DeviceBuffer((B, H, Lkv, d), dtype)
    q.fill_normal(50)
    k.fill_normal(51)
    v.fill_normal(52)
    o = capi.DeviceBuffer((B, H, 1, d), dtype)
    lse = capi.DeviceBuffer((B, H), "f32")
    capi.attn_decode(q, k, v, o, lse, scale)
    o2 = capi.DeviceBuffer((B, H, 1, d), dtype)
    lse2 = capi.DeviceBuffer((B, H, 1), "f32")
    capi.attn_fwd(q, k, v, o2, lse2, scale, False)
    capi.lib().sync()
    od, ld = o.download(), lse.download()
    _check("decode vs forward kernel O", od, o2.download(), TOL[dtype])
    _check("decode vs forward kernel LSE", ld, lse2.download()[..., 0], 2.0 ** -9)
    qh = q.download()
    esz = 2 if dtype == "bf16" else 4
    import ctypes as C
    for (bb, hh) in [(0, 0), (B // 2 + 1, H // 2 + 5), (B - 1, H - 1)]:
        bh = bb * H + hh
        slab = Lkv * d
        raw = np.empty(slab, np.uint16 if dtype == "bf16" else np.float32)
        heads = []
        for buf in (k, v):
            capi.lib().call("tt_memcpy_d2h", raw.ctypes.data, C.c_void_p(buf.ptr + esz * bh * slab), esz * slab)
            heads.append((capi.bf16_to_f32(raw) if dtype == "bf16" else raw.copy()).reshape(Lkv, d))
        o_ref, l_ref = orc.attn_decode_f64(qh[bb, hh], heads[0], heads[1], scale)
        _check(f"head ({bb},{hh}) o", od[bb, hh], o_ref, TOL[dtype])
        _check(f"head ({bb},{hh}) lse", ld[bb, hh], l_ref[0], TOL[dtype])


# ------------------------------------------------------------------ shapes and edges

SHAPES = [
    # (B, H, Lq, Lk, d, causal)
    (1, 1, 1, 1, 32, False),
    (1, 2, 37, 37, 64, True),
    (2, 1, 130, 130, 128, True),
    (1, 3, 200, 77, 64, False),
    (1, 1, 65, 300, 128, False),
    (2, 2, 257, 257, 32, True),
    (1, 1, 3, 1000, 64, False),
    # d = 128 with Lq, Lk multiples of the 128-row tiles: no masked edge tile
    (1, 2, 256, 256, 128, True),
    (2, 1, 512, 512, 128, True),
    (1, 1, 128, 512, 128, False),
    (2, 1, 384, 256, 128, False),
    # d = 128 bf16 dK / dV: 256-key workgroups (two 32-key halves per wave), 32-query tiles
    (1, 1, 33, 33, 128, True),      # one key block, ragged query tile on the diagonal
    (1, 2, 300, 300, 128, True),    # second key block of 44 keys, ragged last query tile
    (2, 1, 257, 513, 128, False),   # last key block holds one key
    (1, 1, 96, 40, 128, False),     # fewer keys than one wave's first half
    (1, 1, 544, 544, 128, True),    # a last key block of exactly one 32-key half
    (1, 1, 1000, 1000, 128, True),  # four key blocks, each with its diagonal tiles, the last one ragged
]


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("shape", SHAPES, ids=[str(s) for s in SHAPES])
def test_ragged_shapes(capi, dtype, shape):
    B, H, Lq, Lk, d, causal = shape
    _say(f"ragged {dtype} {shape}")
    rng = np.random.default_rng(1000 + Lq + Lk + d)
    x = {
        "q": rng.standard_normal((B, H, Lq, d), dtype=np.float32),
        "k": rng.standard_normal((B, H, Lk, d), dtype=np.float32),
        "v": rng.standard_normal((B, H, Lk, d), dtype=np.float32),
        "do": rng.standard_normal((B, H, Lq, d), dtype=np.float32),
    }
    if dtype == "bf16":
        x = {n: orc.bf16_round(a) for n, a in x.items()}
    scale = float(np.float32(1.0 / math.sqrt(d)))
    tol = TOL["f32" if dtype == "f32" else "bf16"]
    b = _run_fwd(capi, x, dtype, scale, causal)
    o_ref, l_ref = orc.attn_fwd_f64(x["q"], x["k"], x["v"], scale, causal)
    _check("O", b["o"].download(), o_ref, tol)
    _check("LSE", b["lse"].download(), l_ref, tol)
    dq, dk, dv = _run_bwd(capi, b, x["do"], dtype, scale, causal)
    rq, rk, rv = orc.attn_bwd_f64(x["q"], x["k"], x["v"], x["do"], scale, causal)
    _check("dQ", dq, rq, tol)
    _check("dK", dk, rk, tol)
    _check("dV", dv, rv, tol)


# Launches over a head count that is a multiple of 8, where the tile mapping
# keeps every head on one XCD (id % 8) and, for causal launches at d <= 64,
# holds each head's cheapest half of the tiles back to a final phase: odd,
# ragged and single-tile counts per head, both dtypes, every head against the
# oracle; non-causal ones keep the plain head groups.
XCD_SHAPES = [
    # (B, H, Lq, Lk, d, dtype, causal)
    (1, 8, 300, 300, 64, "bf16", True),      # 3 query tiles per head, one held back
    (2, 8, 1000, 1000, 64, "bf16", True),    # 8 query tiles, the last one ragged
    (1, 8, 96, 96, 64, "bf16", True),        # one query tile: nothing held back
    (1, 16, 129, 129, 32, "bf16", True),     # the d = 32 kernels
    (1, 8, 2048, 2048, 64, "bf16", True),    # 16 query tiles
    (1, 8, 513, 513, 64, "f32", True),       # the fp32 kernels
    (3, 8, 700, 700, 128, "bf16", True),     # d = 128: head groups only
    (2, 8, 700, 333, 64, "bf16", False),     # non-causal, Lq != Lk
    (1, 16, 257, 900, 128, "bf16", False),
    (1, 8, 300, 500, 64, "f32", False),
]


@pytest.mark.parametrize("shape", XCD_SHAPES, ids=[str(s) for s in XCD_SHAPES])
def test_xcd_grouped_tile_order(capi, shape):
    B, H, Lq, Lk, d, dtype, causal = shape
    _say(f"xcd-grouped {dtype} B={B} H={H} Lq={Lq} Lk={Lk} d={d} causal={causal}")
    rng = np.random.default_rng(3000 + Lq + Lk + d + B * H)
    x = {n: rng.standard_normal((B, H, L, d), dtype=np.float32)
         for n, L in (("q", Lq), ("k", Lk), ("v", Lk), ("do", Lq))}
    if dtype == "bf16":
        x = {n: orc.bf16_round(a) for n, a in x.items()}
    scale = float(np.float32(1.0 / math.sqrt(d)))
    tol = TOL[dtype]
    b = _run_fwd(capi, x, dtype, scale, causal)
    o_ref, l_ref = orc.attn_fwd_f64(x["q"], x["k"], x["v"], scale, causal)
    _check("O", b["o"].download(), o_ref, tol)
    _check("LSE", b["lse"].download(), l_ref, tol)
    dq, dk, dv = _run_bwd(capi, b, x["do"], dtype, scale, causal)
    rq, rk, rv = orc.attn_bwd_f64(x["q"], x["k"], x["v"], x["do"], scale, causal)
    # per head, so that one wrong head cannot hide behind the others' scale
    for bb in range(B):
        for hh in range(H):
            for name, got, ref in (("dQ", dq, rq), ("dK", dk, rk), ("dV", dv, rv)):
                err = orc.max_rel_err(got[bb, hh], ref[bb, hh])
                assert err <= tol, f"head ({bb},{hh}) {name}: {err:.3e} > {tol:g}"
    _check("dQ", dq, rq, tol)
    _check("dK", dk, rk, tol)
    _check("dV", dv, rv, tol)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("Lkv,d", [(1, 64), (100, 32), (777, 128), (4096, 64), (5000, 128)])
def test_decode_shapes(capi, dtype, Lkv, d):
    _say(f"decode {dtype} Lkv={Lkv} d={d}")
    rng = np.random.default_rng(Lkv + d)
    B, H = 3, 5
    q = rng.standard_normal((B, H, 1, d), dtype=np.float32)
    k = rng.standard_normal((B, H, Lkv, d), dtype=np.float32)
    v = rng.standard_normal((B, H, Lkv, d), dtype=np.float32)
    if dtype == "bf16":
        q, k, v = orc.bf16_round(q), orc.bf16_round(k), orc.bf16_round(v)
    scale = float(np.float32(1.0 / math.sqrt(d)))
    bq = capi.DeviceBuffer.from_numpy(q, dtype)
    bk = capi.DeviceBuffer.from_numpy(k, dtype)
    bv = capi.DeviceBuffer.from_numpy(v, dtype)
    bo = capi.DeviceBuffer(q.shape, dtype)
    bl = capi.DeviceBuffer((B, H), "f32")
    capi.attn_decode(bq, bk, bv, bo, bl, scale)
    o_ref, l_ref = orc.attn_decode_f64(q, k, v, scale)
    tol = TOL["f32" if dtype == "f32" else "bf16"]
    _check("o", bo.download(), o_ref, tol)
    _check("lse", bl.download(), l_ref[..., 0], tol)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_repeated_calls_are_bitwise_identical(capi, dtype):
    """No atomics and a fixed reduction order: the same inputs give the same
    bits on every call (forward, backward and decode), including the fp32
    forward's key split and combine."""
    B, H, L, d = 2, 3, 300, 64
    _say(f"determinism {dtype} [{B},{H},{L},{d}] causal fwd+bwd, decode, 3 calls")
    rng = np.random.default_rng(77)
    x = {n: rng.standard_normal((B, H, L, d), dtype=np.float32) for n in ("q", "k", "v", "do")}
    scale = float(np.float32(1 / math.sqrt(d)))
    runs = []
    for _ in range(3):
        b = _run_fwd(capi, x, dtype, scale, True)
        ddo = capi.DeviceBuffer.from_numpy(x["do"], dtype)
        g = [capi.DeviceBuffer((B, H, L, d), dtype) for _ in range(3)]
        capi.attn_bwd(b["q"], b["k"], b["v"], b["o"], b["lse"], ddo, *g, scale, True)
        q1 = capi.DeviceBuffer.from_numpy(x["q"][:, :, :1].copy(), dtype)
        o1 = capi.DeviceBuffer((B, H, 1, d), dtype)
        l1 = capi.DeviceBuffer((B, H), "f32")
        capi.attn_decode(q1, b["k"], b["v"], o1, l1, scale)
        capi.lib().sync()
        runs.append([t.download_bytes() for t in (b["o"], b["lse"], *g, o1, l1)])
    for later in runs[1:]:
        for name, a, r in zip(("O", "LSE", "dQ", "dK", "dV", "decode o", "decode lse"), later, runs[0]):
            assert np.array_equal(a.view(np.uint8), r.view(np.uint8)), f"{name} differs between calls"


def test_empty_inputs_are_noops(capi):
    z = capi.DeviceBuffer((0, 2, 16, 64), "bf16")
    capi.attn_fwd(z, z, z, z, None, 0.125, True)
    e = capi.DeviceBuffer((1, 1, 0, 64), "f32")
    capi.attn_fwd(e, e, e, e, None, 0.125, True)
    # no queries: dK and dV are defined as zero
    k = capi.DeviceBuffer.from_numpy(np.ones((1, 1, 5, 64), np.float32), "f32")
    dk = capi.DeviceBuffer.from_numpy(np.full((1, 1, 5, 64), 7, np.float32), "f32")
    dv = capi.DeviceBuffer.from_numpy(np.full((1, 1, 5, 64), 7, np.float32), "f32")
    capi.attn_bwd(e, k, k, e, e, e, e, dk, dv, 0.125, False)
    assert not dk.download().any() and not dv.download().any()


def test_errors_are_reported(capi):
    a = capi.DeviceBuffer((1, 1, 8, 96), "f32")
    with pytest.raises(capi.TTError) as ei:
        capi.attn_fwd(a, a, a, a, None, 0.1, False)
    assert ei.value.code == capi.TT_ERR_UNSUPPORTED and "head dim" in str(ei.value)
    q = capi.DeviceBuffer((1, 1, 8, 64), "f32")
    k = capi.DeviceBuffer((1, 1, 9, 64), "f32")
    with pytest.raises(capi.TTError) as ei:
        capi.attn_fwd(q, k, k, q, None, 0.1, True)
    assert ei.value.code == capi.TT_ERR_ARG and "Lq == Lk" in str(ei.value)
    with pytest.raises(capi.TTError):
        capi.lib().call("tt_attn_fwd_f32", None, None, None, None, None, 1, 1, 8, 8, 64, 0.1, 0, None)


def test_overlapping_outputs_are_refused(capi):
    """An output whose bytes overlap an input's or another output's is
    refused before anything is launched; inputs may overlap each other
    (q = k = v).  Every pointer lies inside an allocation of its size."""
    import ctypes as C

    L = capi.lib()
    B, H, Lq, d = 1, 2, 64, 64
    shp = (B, H, Lq, d)
    big = capi.DeviceBuffer((2,) + shp, "bf16")  # room for two tensors
    half = big.nbytes // 2
    k, v, do = (capi.DeviceBuffer(shp, "bf16") for _ in range(3))
    for i, b in enumerate((big, k, v, do)):
        b.fill_normal(90 + i)
    lse = capi.DeviceBuffer(shp[:3], "f32")
    s = C.c_float(0.125)

    def fwd(q, k_, v_, o, l):
        return L.lib.tt_attn_fwd_bf16(q, k_, v_, o, l, B, H, Lq, Lq, d, s, 0, None)

    assert fwd(big.ptr, k.ptr, v.ptr, big.ptr + half // 2, lse.ptr) == capi.TT_ERR_ARG
    assert "output o overlaps input q" in L.last_error()
    assert fwd(big.ptr, k.ptr, v.ptr, big.ptr + half, big.ptr + half + 64) == capi.TT_ERR_ARG
    assert "outputs o and lse overlap" in L.last_error()
    q32 = capi.DeviceBuffer((1, 1, 8, 32), "f32")
    assert L.lib.tt_attn_fwd_f32(q32.ptr, k.ptr, v.ptr, big.ptr, q32.ptr + 64, 1, 1, 8, 8, 32, s, 0, None) \
        == capi.TT_ERR_ARG
    assert "output lse overlaps input q" in L.last_error()
    # q = k = v is a valid self-attention call; o right after q in one block
    assert fwd(big.ptr, big.ptr, big.ptr, big.ptr + half, lse.ptr) == capi.TT_OK, L.last_error()
    L.sync()
    o = big.ptr + half
    assert L.lib.tt_attn_bwd_bf16(big.ptr, k.ptr, v.ptr, o, lse.ptr, do.ptr, k.ptr, v.ptr, do.ptr,
                                  B, H, Lq, Lq, d, s, 0, None) == capi.TT_ERR_ARG
    assert "output dQ overlaps input k" in L.last_error()
    assert L.lib.tt_attn_bwd_bf16(k.ptr, k.ptr, k.ptr, k.ptr, lse.ptr, k.ptr, big.ptr, big.ptr + half - 2, do.ptr,
                                  B, H, Lq, Lq, d, s, 0, None) == capi.TT_ERR_ARG
    assert "outputs dQ and dK overlap" in L.last_error()
    q1 = capi.DeviceBuffer((B, H, 1, d), "bf16")
    assert L.lib.tt_attn_decode_bf16(q1.ptr, k.ptr, v.ptr, v.ptr + 128, None, B, H, Lq, d, s, None) == capi.TT_ERR_ARG
    assert "output o overlaps input v" in L.last_error()


def orc_golden(name):
    import os

    return os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", name)
