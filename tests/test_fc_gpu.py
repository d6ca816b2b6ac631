"""GPU tests of the fully connected layer (myLayer.FcForward / FcBackward,
reference src/Layers.cu:9-79, bound at src/bind_Layer.cpp:12-13) and of the
``operators.FC`` op over it (reference optimizer/operators.py:498-533): the
products run on the library GEMM (tt_gemm_*), the bias through a rank-1 GEMM
against a ones column, as in the reference.

Oracle: numpy float64 on the same (for bf16: bf16-rounded) values.  Bar
(normwise max|x - ref| / max|ref|): fp32 <= 1e-5 (fp32 products and sums on
the fp32 MFMA), bf16 <= 2e-2 (bf16 operands and results, fp32 sums; the bias
is added to the bf16-rounded product and rounded again).
"""
import numpy as np
import pytest

from oracle import attn_oracle as orc

pytestmark = pytest.mark.gpu

TOL = {"float": 1e-5, "bf16": 2e-2}


@pytest.fixture(scope="module")
def mods():
    import myLayer
    import myTensor

    assert myTensor.device_count() >= 1, "no HIP device visible"
    return myTensor, myLayer


def _vals(shape, seed, dt):
    x = np.random.default_rng(seed).standard_normal(shape).astype(np.float32)
    return orc.bf16_round(x) if dt == "bf16" else x


def _dev(mt, dt, a):
    return getattr(mt, "Tensor_" + dt)(np.ascontiguousarray(a, np.float32), "gpu")


def _empty(mt, dt):
    return getattr(mt, "Tensor_" + dt)([1], "gpu")


def _fc_ref(x, w, b, scalar):
    x64 = x.reshape(-1, x.shape[-1]).astype(np.float64)
    y = x64 @ w.astype(np.float64) + (b.astype(np.float64)[0] if scalar else b.astype(np.float64))
    return y.reshape(x.shape[:-1] + (w.shape[1],))


# (input shape, fout, scalar bias): ragged sizes on the general GEMM, a 3-D
# input (two batch axes), a [1] bias, and an aligned size on the bf16
# direct-to-LDS kernel (k % 32 == 0)
CASES = [((7, 13), 5, False), ((3, 5, 40), 24, False), ((33, 70), 17, True), ((1, 1), 1, False),
         ((256, 512), 384, False), ((64, 96), 128, True)]


@pytest.mark.parametrize("dt", ["float", "bf16"])
@pytest.mark.parametrize("shape,fout,scalar", CASES)
def test_fc_forward_backward(mods, dt, shape, fout, scalar):
    mt, ml = mods
    fin = shape[-1]
    x, w = _vals(shape, 1, dt), _vals((fin, fout), 2, dt)
    b = _vals((1,) if scalar else (fout,), 3, dt)
    go = _vals(shape[:-1] + (fout,), 4, dt)
    X, W, Bt, GO = (_dev(mt, dt, a) for a in (x, w, b, go))
    out = _empty(mt, dt)
    ml.FcForward(X, out, W, Bt)
    assert out.get_shape() == list(shape[:-1]) + [fout]
    err = orc.max_rel_err(np.asarray(out.numpy()).reshape(out.get_shape()), _fc_ref(x, w, b, scalar))
    assert err <= TOL[dt], f"forward {err:.3e}"

    gx, gw, gb = _empty(mt, dt), _empty(mt, dt), _empty(mt, dt)
    ml.FcBackward(X, out, W, Bt, gx, GO, gw, gb)
    assert gx.get_shape() == list(shape) and gw.get_shape() == [fin, fout] and gb.get_shape() == list(b.shape)
    g64 = go.reshape(-1, fout).astype(np.float64)
    x64 = x.reshape(-1, fin).astype(np.float64)
    ref = {"grad_input": (g64 @ w.astype(np.float64).T).reshape(shape),
           "grad_weight": x64.T @ g64,
           "grad_bias": np.array([g64.sum()]) if scalar else g64.sum(0)}
    got = {"grad_input": gx, "grad_weight": gw, "grad_bias": gb}
    for name, r in ref.items():
        a = np.asarray(got[name].numpy()).reshape(r.shape)
        e = orc.max_rel_err(a, r)
        assert e <= TOL[dt], f"{name} {e:.3e}"


def test_fc_errors(mods):
    mt, ml = mods
    X = _dev(mt, "float", np.ones((4, 8)))
    W = _dev(mt, "float", np.ones((8, 3)))
    out = _empty(mt, "float")
    with pytest.raises(ValueError, match="weight rows"):
        ml.FcForward(X, out, _dev(mt, "float", np.ones((7, 3))), _dev(mt, "float", np.ones(3)))
    with pytest.raises(ValueError, match="bias"):
        ml.FcForward(X, out, W, _dev(mt, "float", np.ones(2)))
    with pytest.raises(ValueError, match="same tensor"):
        ml.FcForward(X, X, W, _dev(mt, "float", np.ones(3)))
    gx, gw, gb = _empty(mt, "float"), _empty(mt, "float"), _empty(mt, "float")
    with pytest.raises(ValueError, match="grad_output"):
        ml.FcBackward(X, out, W, _dev(mt, "float", np.ones(3)), gx, _dev(mt, "float", np.ones((4, 2))), gw, gb)


@pytest.mark.parametrize("use_bias", [True, False])
def test_fc_operator_autograd(use_bias):
    import operators as ops

    rng = np.random.default_rng(7)
    x = rng.standard_normal((6, 20)).astype(np.float32)
    w = rng.standard_normal((20, 9)).astype(np.float32)
    b = rng.standard_normal(9).astype(np.float32)
    g = rng.standard_normal((6, 9)).astype(np.float32)
    X, W, B = ops.Tensor(x), ops.Tensor(w), ops.Tensor(b)
    y = ops.fc(X, W, B, use_bias=use_bias)
    ref = x.astype(np.float64) @ w + (b if use_bias else 0.0)
    assert orc.max_rel_err(np.asarray(y.realize_cached_data()), ref) <= 1e-5
    y.backward(ops.Tensor(g, requires_grad=False))
    g64 = g.astype(np.float64)
    assert orc.max_rel_err(np.asarray(X.grad.realize_cached_data()).reshape(x.shape), g64 @ w.T) <= 1e-5
    assert orc.max_rel_err(np.asarray(W.grad.realize_cached_data()).reshape(w.shape), x.T @ g64) <= 1e-5
    gb = np.asarray(B.grad.realize_cached_data()).reshape(b.shape)
    if use_bias:
        assert orc.max_rel_err(gb, g64.sum(0)) <= 1e-5
    else:
        assert not gb.any()
