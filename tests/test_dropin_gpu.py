"""GPU parity through the drop-in surface: the pybind11 ``myLayer`` entry
points on ``myTensor`` tensors (Tensor_float / Tensor_bf16), and the Python
autograd operator ``operators.attention(...)`` with ``.backward(dO)``, each
against the float64 oracle (oracle/attn_oracle.py).

The reference's calling pattern these follow: a layer function over
TinyTensor references that resizes its outputs (src/bind_Layer.cpp:12-23 ->
src/Layers.cu:9-79), and a TensorOp whose compute uploads with
Tensor_float(..., "gpu") and whose gradient calls the backward layer function
(optimizer/operators.py:498-532, the FC op).

Bars as in test_attn_gpu.py: max|x - ref| / max|ref| <= 1e-4 (fp32), <= 2e-2
(bf16 with fp32 accumulation), on the exact (bf16-rounded) inputs.
"""
import math
import os
import sys

import numpy as np
import pytest

from oracle import attn_oracle as orc

pytestmark = pytest.mark.gpu

TOL = orc.TOL
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _check(name, x, ref, tol):
    err = orc.max_rel_err(np.asarray(x), ref)
    _say(f"  {name}: max-rel-err {err:.3e} (tol {tol:g})")
    assert err <= tol, f"{name}: {err:.3e} > {tol:g}"


@pytest.fixture(scope="module")
def mods():
    import myLayer
    import myTensor

    assert myTensor.device_count() >= 1, "no HIP device visible"
    return myTensor, myLayer


def _cls(mt, dtype):
    return mt.Tensor_bf16 if dtype == "bf16" else mt.Tensor_float


def _layer_fwd_bwd(mods, x, dtype, scale, causal, backward=True):
    """myLayer.AttentionForward (+ Backward) on uploaded tensors; outputs
    start as 1-element tensors that the callee resizes."""
    mt, ml = mods
    T = _cls(mt, dtype)
    q, k, v = (T(np.ascontiguousarray(x[n], np.float32), "gpu") for n in ("q", "k", "v"))
    out, lse = T([1], "gpu"), mt.Tensor_float([1], "gpu")
    ml.AttentionForward(q, k, v, out, lse, scale, causal)
    res = {"o": out.numpy(), "lse": lse.numpy()}
    assert list(out.get_shape()) == list(x["q"].shape)
    assert list(lse.get_shape()) == list(x["q"].shape[:3])
    if backward:
        do = T(np.ascontiguousarray(x["do"], np.float32), "gpu")
        gq, gk, gv = T([1], "gpu"), T([1], "gpu"), T([1], "gpu")
        ml.AttentionBackward(q, k, v, out, lse, do, gq, gk, gv, scale, causal)
        res.update(dq=gq.numpy(), dk=gk.numpy(), dv=gv.numpy())
    return res


def _bf16_inputs(x):
    return {n: orc.bf16_round(a) for n, a in x.items()}


# ------------------------------------------------------------------ myLayer

@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_layer_c1_golden(mods, dtype):
    """c1 (B=1 H=1 L=64 d=32, no mask) through myLayer.AttentionForward
    against the torch-written golden O / LSE (fp32) or the oracle on the
    bf16-rounded inputs."""
    g = np.load(os.path.join(GOLDEN, "c1_fwd.npz"))
    x = {n: g[n] for n in ("q", "k", "v")}
    scale = float(g["scale"])
    _say(f"myLayer c1 {dtype}")
    if dtype == "bf16":
        x = _bf16_inputs(x)
        ro, rl = orc.attn_fwd_f64(x["q"], x["k"], x["v"], scale, False)
    else:
        ro, rl = g["o"], g["lse"]
    r = _layer_fwd_bwd(mods, x, dtype, scale, False, backward=False)
    _check("O", r["o"], ro, TOL[dtype])
    _check("LSE", r["lse"], rl, TOL[dtype])


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_layer_c2_full(mods, dtype):
    """c2 (B=8 H=8 L=256 d=64, no mask) forward + backward, every head."""
    cfg = orc.CONFIGS[2]
    x = orc.seeded_inputs(cfg)
    if dtype == "bf16":
        x = _bf16_inputs(x)
    _say(f"myLayer c2 {dtype}")
    r = _layer_fwd_bwd(mods, x, dtype, cfg.scale, False)
    ro, rl = orc.attn_fwd_f64(x["q"], x["k"], x["v"], cfg.scale, False)
    rq, rk, rv = orc.attn_bwd_f64(x["q"], x["k"], x["v"], x["do"], cfg.scale, False)
    for n, ref in (("o", ro), ("lse", rl), ("dq", rq), ("dk", rk), ("dv", rv)):
        _check(n, r[n], ref, TOL[dtype])


def test_layer_c3_head_subset(mods):
    """c3 (bf16 causal B=16 H=16 L=1024 d=64) through myLayer; three heads
    against the oracle."""
    cfg = orc.CONFIGS[3]
    x = orc.seeded_inputs(cfg)
    _say("myLayer c3 bf16 causal")
    r = _layer_fwd_bwd(mods, x, "bf16", cfg.scale, True)
    for (b, h) in [(0, 0), (9, 4), (15, 15)]:
        one = {n: a[b, h] for n, a in x.items()}
        ro, rl = orc.attn_fwd_f64(one["q"], one["k"], one["v"], cfg.scale, True)
        rq, rk, rv = orc.attn_bwd_f64(one["q"], one["k"], one["v"], one["do"], cfg.scale, True)
        _say(f" head ({b},{h})")
        for n, ref in (("o", ro), ("lse", rl), ("dq", rq), ("dk", rk), ("dv", rv)):
            _check(n, r[n][b, h], ref, TOL["bf16"])


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_layer_decode(mods, dtype):
    mt, ml = mods
    B, H, Lkv, d = 2, 3, 1500, 128
    scale = float(np.float32(1 / math.sqrt(d)))
    rng = np.random.default_rng(77)
    x = {"q": rng.standard_normal((B, H, 1, d), dtype=np.float32),
         "k": rng.standard_normal((B, H, Lkv, d), dtype=np.float32),
         "v": rng.standard_normal((B, H, Lkv, d), dtype=np.float32)}
    if dtype == "bf16":
        x = _bf16_inputs(x)
    _say(f"myLayer decode {dtype} B={B} H={H} Lkv={Lkv} d={d}")
    T = _cls(mt, dtype)
    q, k, v = (T(x[n], "gpu") for n in ("q", "k", "v"))
    out = T([1], "gpu")
    ml.AttentionDecode(q, k, v, out, scale)
    assert list(out.get_shape()) == [B, H, 1, d]
    ro, _ = orc.attn_decode_f64(x["q"], x["k"], x["v"], scale)
    _check("o", out.numpy(), ro, TOL[dtype])


def test_layer_rejects_bad_shapes(mods):
    mt, ml = mods
    q = mt.Tensor_float(np.zeros((1, 1, 8, 48), np.float32), "gpu")  # d = 48 is not supported
    out, lse = mt.Tensor_float([1], "gpu"), mt.Tensor_float([1], "gpu")
    with pytest.raises((ValueError, RuntimeError)):
        ml.AttentionForward(q, q, q, out, lse, 0.1, False)
    q3 = mt.Tensor_float(np.zeros((1, 8, 64), np.float32), "gpu")  # rank 3
    with pytest.raises(ValueError):
        ml.AttentionForward(q3, q3, q3, out, lse, 0.1, False)


@pytest.mark.parametrize("dtype", ["float32", "bf16"])
def test_layer_rejects_outputs_aliasing_inputs(mods, dtype):
    """An output that is one of the inputs (or another output) is refused
    before any resize or launch, and the inputs keep their data."""
    mt, ml = mods
    T = _cls(mt, dtype)
    rng = np.random.default_rng(7)
    x = {n: orc.bf16_round(rng.standard_normal((1, 2, 64, 32), dtype=np.float32)) for n in ("q", "k", "v", "do")}
    q, k, v, do = (T(x[n], "gpu") for n in ("q", "k", "v", "do"))
    kl = T(orc.bf16_round(rng.standard_normal((1, 2, 96, 32), dtype=np.float32)), "gpu")
    out, lse = T([1], "gpu"), mt.Tensor_float([1], "gpu")
    with pytest.raises(ValueError, match="out is the same tensor as input q"):
        ml.AttentionForward(q, k, v, q, lse, 0.1, False)
    with pytest.raises(ValueError, match="out is the same tensor as input k"):
        ml.AttentionForward(q, kl, kl, kl, lse, 0.1, False)  # its resize would free k
    ml.AttentionForward(q, k, v, out, lse, 0.1, True)
    gq, gk = T([1], "gpu"), T([1], "gpu")
    with pytest.raises(ValueError, match="grad_v is the same tensor as input v"):
        ml.AttentionBackward(q, k, v, out, lse, do, gq, gk, v, 0.1, True)
    with pytest.raises(ValueError, match="outputs grad_q and grad_k are the same tensor"):
        ml.AttentionBackward(q, k, v, out, lse, do, gq, gq, gk, 0.1, True)
    q1 = T(x["q"][:, :, :1], "gpu")
    with pytest.raises(ValueError, match="out is the same tensor as input q"):
        ml.AttentionDecode(q1, k, v, q1, 0.1)
    for n, t in (("q", q), ("k", k), ("v", v), ("do", do)):
        np.testing.assert_array_equal(np.asarray(t.numpy(), np.float32).reshape(x[n].shape), x[n], err_msg=n)
    assert kl.numpy().shape == (1, 2, 96, 32)


# ------------------------------------------------------------------ autograd operator

@pytest.fixture(scope="module")
def ops():
    import operators

    return operators


CASES = [
    # (B, H, Lq, Lk, d, causal, dtype)
    (2, 3, 96, 96, 64, True, "float32"),
    (1, 2, 80, 130, 32, False, "float32"),
    (2, 2, 160, 160, 128, True, "bf16"),
    (1, 3, 64, 200, 64, False, "bf16"),
]


@pytest.mark.parametrize("case", CASES, ids=[str(c) for c in CASES])
def test_operator_attention_backward(ops, case):
    """operators.attention(q, k, v, causal, dtype).backward(dO): O and the
    .grad of q, k and v against the oracle."""
    B, H, Lq, Lk, d, causal, dtype = case
    rng = np.random.default_rng(Lq * 7 + Lk + d)
    x = {"q": rng.standard_normal((B, H, Lq, d), dtype=np.float32),
         "k": rng.standard_normal((B, H, Lk, d), dtype=np.float32),
         "v": rng.standard_normal((B, H, Lk, d), dtype=np.float32),
         "do": rng.standard_normal((B, H, Lq, d), dtype=np.float32)}
    if dtype == "bf16":
        x = _bf16_inputs(x)
    tol = TOL["bf16" if dtype == "bf16" else "f32"]
    scale = float(np.float32(1 / math.sqrt(d)))
    _say(f"operators.attention {case}")
    tq, tk, tv = (ops.Tensor(x[n]) for n in ("q", "k", "v"))
    out = ops.attention(tq, tk, tv, causal=causal, dtype=dtype)
    out.backward(ops.Tensor(x["do"], requires_grad=False))
    ro, _ = orc.attn_fwd_f64(x["q"], x["k"], x["v"], scale, causal)
    rq, rk, rv = orc.attn_bwd_f64(x["q"], x["k"], x["v"], x["do"], scale, causal)
    _check("O", out.numpy(), ro, tol)
    _check("q.grad", tq.grad.numpy(), rq, tol)
    _check("k.grad", tk.grad.numpy(), rk, tol)
    _check("v.grad", tv.grad.numpy(), rv, tol)
    assert out.saved is None  # device tensors released after the gradient


def test_operator_instance_reused_for_two_nodes(ops):
    """One Attention object applied to two different inputs: each node's
    backward uses its own inputs (the saved state lives on the node)."""
    rng = np.random.default_rng(5)
    shp = (1, 2, 64, 64)
    xs = [{n: rng.standard_normal(shp, dtype=np.float32) for n in ("q", "k", "v", "do")} for _ in range(2)]
    op = ops.Attention(causal=True, dtype="float32")
    ts = [tuple(ops.Tensor(x[n]) for n in ("q", "k", "v")) for x in xs]
    y1 = op(*ts[0])
    y2 = op(*ts[1])
    y1.backward(ops.Tensor(xs[0]["do"], requires_grad=False))
    scale = float(np.float32(1 / 8))
    for i, (x, t) in enumerate(zip(xs[:1], ts[:1])):
        rq, rk, rv = orc.attn_bwd_f64(x["q"], x["k"], x["v"], x["do"], scale, True)
        _check(f"node {i} q.grad", t[0].grad.numpy(), rq, TOL["f32"])
        _check(f"node {i} k.grad", t[1].grad.numpy(), rk, TOL["f32"])
        _check(f"node {i} v.grad", t[2].grad.numpy(), rv, TOL["f32"])
    y2.backward(ops.Tensor(xs[1]["do"], requires_grad=False))
    rq, _, _ = orc.attn_bwd_f64(xs[1]["q"], xs[1]["k"], xs[1]["v"], xs[1]["do"], scale, True)
    _check("node 1 q.grad", ts[1][0].grad.numpy(), rq, TOL["f32"])


def test_operator_second_backward_recomputes(ops):
    """A second backward through the same node (its saved device tensors were
    released by the first) recomputes the forward and gives the same grads."""
    rng = np.random.default_rng(6)
    shp = (1, 1, 48, 64)
    x = {n: rng.standard_normal(shp, dtype=np.float32) for n in ("q", "k", "v", "do")}
    tq, tk, tv = (ops.Tensor(x[n]) for n in ("q", "k", "v"))
    y = ops.attention(tq, tk, tv, causal=False)
    y.backward(ops.Tensor(x["do"], requires_grad=False))
    g1 = tq.grad.numpy().copy()
    y.backward(ops.Tensor(x["do"], requires_grad=False))
    np.testing.assert_array_equal(tq.grad.numpy(), g1)


def test_operator_inside_a_larger_graph(ops):
    """The fused op composed with host ops: loss = sum((attention(q, k, v) @ W)),
    so the upstream gradient reaching the op is ones @ W^T."""
    rng = np.random.default_rng(8)
    shp = (1, 2, 32, 32)
    q, k, v = (rng.standard_normal(shp, dtype=np.float32) for _ in range(3))
    W = rng.standard_normal((32, 5)).astype(np.float32)
    tq, tk, tv = ops.Tensor(q), ops.Tensor(k), ops.Tensor(v)
    (ops.attention(tq, tk, tv, causal=True) @ ops.Tensor(W, requires_grad=False)).sum().backward()
    do = np.broadcast_to(np.ones((32, 5)) @ W.T, shp)
    scale = float(np.float32(1 / math.sqrt(32)))
    rq, rk, rv = orc.attn_bwd_f64(q, k, v, do, scale, True)
    _check("q.grad", tq.grad.numpy(), rq, TOL["f32"])
    _check("k.grad", tk.grad.numpy(), rk, TOL["f32"])
    _check("v.grad", tv.grad.numpy(), rv, TOL["f32"])


@pytest.mark.parametrize("dtype", ["float32", "bf16"])
def test_operator_attention_decode(ops, dtype):
    rng = np.random.default_rng(9)
    B, H, Lkv, d = 3, 2, 700, 64
    x = {"q": rng.standard_normal((B, H, 1, d), dtype=np.float32),
         "k": rng.standard_normal((B, H, Lkv, d), dtype=np.float32),
         "v": rng.standard_normal((B, H, Lkv, d), dtype=np.float32)}
    if dtype == "bf16":
        x = _bf16_inputs(x)
    y = ops.attention_decode(ops.Tensor(x["q"]), ops.Tensor(x["k"]), ops.Tensor(x["v"]), dtype=dtype)
    ro, _ = orc.attn_decode_f64(x["q"], x["k"], x["v"], float(np.float32(1 / 8)))
    _check(f"decode {dtype}", y.numpy(), ro, TOL["bf16" if dtype == "bf16" else "f32"])
