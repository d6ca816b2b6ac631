"""GPU tests of the convolution layer on the library GEMM: myLayer.im2col /
col2im (tt_im2col / tt_col2im; reference src/Layers.cu:81-158, kernels
src/Layers_kernels.cu:32-105), ConvForward / ConvBackward (src/Layers.cu:
160-252) and ``operators.Conv`` (optimizer/operators.py:535-569).

Oracle: numpy float64 on the same (for bf16: bf16-rounded) values, the
convolution written as a sum over kernel offsets of shifted, strided slices
of the zero-padded input; im2col checked element by element against its
definition, col2im as its adjoint (<im2col(x), c> = <x, col2im(c)>) and
against a scatter-add.  Bar (normwise): fp32 <= 1e-5, bf16 <= 2e-2;
im2col is a copy and must be exact.
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


def _np(t):
    return np.asarray(t.numpy(), np.float64).reshape(t.get_shape())


def _out_hw(H, W, kh, kw, ph, pw, sh, sw):
    return (H + 2 * ph - kh) // sh + 1, (W + 2 * pw - kw) // sw + 1


def _im2col_ref(x, kh, kw, ph, pw, sh, sw):
    N, C, H, W = x.shape
    oh, ow = _out_hw(H, W, kh, kw, ph, pw, sh, sw)
    xp = np.zeros((N, C, H + 2 * ph, W + 2 * pw))
    xp[:, :, ph:ph + H, pw:pw + W] = x
    col = np.empty((N, oh, ow, C, kh, kw))
    for ky in range(kh):
        for kx in range(kw):
            col[:, :, :, :, ky, kx] = xp[:, :, ky:ky + sh * oh:sh, kx:kx + sw * ow:sw].transpose(0, 2, 3, 1)
    return col.reshape(N, oh * ow, C * kh * kw)


def _col2im_ref(col, shape, kh, kw, ph, pw, sh, sw):
    N, C, H, W = shape
    oh, ow = _out_hw(H, W, kh, kw, ph, pw, sh, sw)
    c6 = col.reshape(N, oh, ow, C, kh, kw)
    xp = np.zeros((N, C, H + 2 * ph, W + 2 * pw))
    for ky in range(kh):
        for kx in range(kw):
            xp[:, :, ky:ky + sh * oh:sh, kx:kx + sw * ow:sw] += c6[:, :, :, :, ky, kx].transpose(0, 3, 1, 2)
    return xp[:, :, ph:ph + H, pw:pw + W]


def _conv_ref(x, w, ph, pw, sh, sw):
    N = x.shape[0]
    Cout, Cin, kh, kw = w.shape
    col = _im2col_ref(x.astype(np.float64), kh, kw, ph, pw, sh, sw)  # [N, P, K]
    oh, ow = _out_hw(x.shape[2], x.shape[3], kh, kw, ph, pw, sh, sw)
    return (w.reshape(Cout, -1).astype(np.float64) @ col.transpose(0, 2, 1)).reshape(N, Cout, oh, ow)


# (N, Cin, H, W, Cout, kh, kw, pad_h, pad_w, stride_h, stride_w)
CASES = [(2, 3, 9, 9, 4, 3, 3, 1, 1, 1, 1), (1, 1, 5, 7, 2, 2, 3, 0, 1, 2, 1), (3, 4, 12, 10, 5, 3, 3, 2, 0, 2, 3),
         (2, 8, 16, 16, 16, 5, 5, 2, 2, 1, 1), (1, 2, 4, 4, 3, 4, 4, 0, 0, 1, 1)]


@pytest.mark.parametrize("dt", ["float", "bf16"])
@pytest.mark.parametrize("case", CASES)
def test_im2col_col2im(mods, dt, case):
    mt, ml = mods
    N, C, H, W, _, kh, kw, ph, pw, sh, sw = case
    x = _vals((N, C, H, W), 1, dt)
    col = _empty(mt, dt)
    ml.im2col(_dev(mt, dt, x), col, [kh, kw], ph, pw, sh, sw)
    ref = _im2col_ref(x.astype(np.float64), kh, kw, ph, pw, sh, sw)
    np.testing.assert_array_equal(_np(col), ref)
    c = _vals(ref.shape, 2, dt)
    im = _empty(mt, dt)
    ml.col2im(_dev(mt, dt, c), im, [kh, kw], [N, C, H, W], ph, pw, sh, sw)
    back = _np(im)
    assert back.shape == (N, C, H, W)
    r = _col2im_ref(c.astype(np.float64), (N, C, H, W), kh, kw, ph, pw, sh, sw)
    assert orc.max_rel_err(back, r) <= TOL[dt]
    # adjointness on the reference operators pins the scatter-add itself
    assert abs((ref * c).sum() - (x.astype(np.float64) * r).sum()) <= 1e-9 * (abs(ref * c).sum() + 1)


def test_im2col_rank3_shape(mods):
    mt, ml = mods
    x = _vals((3, 6, 5), 3, "float")
    col = _empty(mt, "float")
    ml.im2col(_dev(mt, "float", x), col, [3, 3], 1, 1, 1, 1)
    assert col.get_shape() == [30, 27]
    np.testing.assert_array_equal(_np(col), _im2col_ref(x[None].astype(np.float64), 3, 3, 1, 1, 1, 1)[0])


@pytest.mark.parametrize("dt", ["float", "bf16"])
@pytest.mark.parametrize("case", CASES)
def test_conv_forward_backward(mods, dt, case):
    mt, ml = mods
    N, Cin, H, W, Cout, kh, kw, ph, pw, sh, sw = case
    x, w = _vals((N, Cin, H, W), 4, dt), _vals((Cout, Cin, kh, kw), 5, dt)
    X, Wt = _dev(mt, dt, x), _dev(mt, dt, w)
    out = _empty(mt, dt)
    ml.ConvForward(X, out, Wt, ph, pw, sh, sw)
    ref = _conv_ref(x, w, ph, pw, sh, sw)
    assert out.get_shape() == list(ref.shape)
    assert orc.max_rel_err(_np(out), ref) <= TOL[dt], "forward"
    go = _vals(ref.shape, 6, dt)
    gx, gw = _empty(mt, dt), _empty(mt, dt)
    ml.ConvBackward(X, out, Wt, gx, _dev(mt, dt, go), gw, ph, pw, sh, sw)
    g64 = go.reshape(N, Cout, -1).astype(np.float64)
    col = _im2col_ref(x.astype(np.float64), kh, kw, ph, pw, sh, sw)
    ref_gw = np.einsum("nop,npk->ok", g64, col).reshape(w.shape)
    ref_gx = _col2im_ref(np.einsum("nop,ok->npk", g64, w.reshape(Cout, -1).astype(np.float64)),
                         (N, Cin, H, W), kh, kw, ph, pw, sh, sw)
    assert orc.max_rel_err(_np(gw), ref_gw) <= TOL[dt], "grad_weight"
    assert orc.max_rel_err(_np(gx), ref_gx) <= TOL[dt], "grad_input"


def test_conv_errors(mods):
    mt, ml = mods
    X = _dev(mt, "float", np.ones((1, 3, 5, 5)))
    out = _empty(mt, "float")
    with pytest.raises(ValueError, match="Cin"):
        ml.ConvForward(X, out, _dev(mt, "float", np.ones((2, 4, 3, 3))), 0, 0, 1, 1)
    with pytest.raises(ValueError, match="larger than the padded image"):
        ml.ConvForward(X, out, _dev(mt, "float", np.ones((2, 3, 7, 7))), 0, 0, 1, 1)
    with pytest.raises(ValueError, match="strides"):
        ml.ConvForward(X, out, _dev(mt, "float", np.ones((2, 3, 3, 3))), 0, 0, 0, 1)
    with pytest.raises(ValueError, match="col_tensor"):
        ml.col2im(_dev(mt, "float", np.ones((8, 27))), out, [3, 3], [1, 3, 5, 5], 0, 0, 1, 1)


def test_conv_operator_autograd():
    import operators as ops

    rng = np.random.default_rng(9)
    x = rng.standard_normal((2, 3, 8, 8)).astype(np.float32)
    w = rng.standard_normal((4, 3, 3, 3)).astype(np.float32)
    X, Wt = ops.Tensor(x), ops.Tensor(w)
    y = ops.conv(X, Wt, 1, 1, 2, 2)
    ref = _conv_ref(x, w, 1, 1, 2, 2)
    assert orc.max_rel_err(np.asarray(y.realize_cached_data()).reshape(ref.shape), ref) <= 1e-5
    g = rng.standard_normal(ref.shape).astype(np.float32)
    y.backward(ops.Tensor(g, requires_grad=False))
    g64 = g.reshape(2, 4, -1).astype(np.float64)
    col = _im2col_ref(x.astype(np.float64), 3, 3, 1, 1, 2, 2)
    ref_gw = np.einsum("nop,npk->ok", g64, col).reshape(w.shape)
    ref_gx = _col2im_ref(np.einsum("nop,ok->npk", g64, w.reshape(4, -1).astype(np.float64)), x.shape, 3, 3, 1, 1, 2, 2)
    assert orc.max_rel_err(np.asarray(Wt.grad.realize_cached_data()).reshape(w.shape), ref_gw) <= 1e-5
    assert orc.max_rel_err(np.asarray(X.grad.realize_cached_data()).reshape(x.shape), ref_gx) <= 1e-5
