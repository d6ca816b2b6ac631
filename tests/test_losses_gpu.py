"""GPU tests of the softmax cross-entropy that follows SoftmaxForward:
myLayer.CrossEntropyLoss / CrossEntropyLossBackward / SoftmaxLoss (reference
src/Layers.cu:351-423, kernels src/Layers_kernels.cu:260-282; C-ABI
tt_cross_entropy_f32 / tt_cross_entropy_backward_f32) and the
``operators.softmaxcrossentropyloss`` op (optimizer/operators.py:636-665).

Oracle: numpy float64 on the softmax rows the GPU returned.  Bar: the loss
within 1e-6 relative (summed in double), the gradient p - onehot bitwise equal
to numpy's float32 p - 1, the error rate exact.
"""
import numpy as np
import pytest
from scipy.special import logsumexp

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def mods():
    import myLayer
    import myTensor

    assert myTensor.device_count() >= 1, "no HIP device visible"
    return myTensor, myLayer


def _softmax_gpu(mt, ml, z):
    p = mt.Tensor_float([1], "gpu")
    ml.SoftmaxForward(mt.Tensor_float(z, "gpu"), p)
    return p, np.asarray(p.numpy()).reshape(z.shape)


@pytest.mark.parametrize("rows,cols", [(1, 10), (64, 10), (1000, 37), (5000, 1000)])
def test_cross_entropy_loss_and_gradient(mods, rows, cols):
    mt, ml = mods
    rng = np.random.default_rng(rows + cols)
    z = (3 * rng.standard_normal((rows, cols))).astype(np.float32)
    y = rng.integers(0, cols, rows).astype(np.int32)
    p, pn = _softmax_gpu(mt, ml, z)
    labels = mt.Tensor_int(y.reshape(1, -1), "gpu")
    loss = mt.Tensor_float([1], "gpu")
    ml.CrossEntropyLoss(p, labels, loss)
    assert loss.get_shape() == [1]
    ref = -np.log(pn[np.arange(rows), y].astype(np.float64)).sum()
    assert abs(loss.get_data()[0] - ref) <= 1e-6 * abs(ref) + 1e-6
    g = mt.Tensor_float([1], "gpu")
    ml.CrossEntropyLossBackward(p, labels, g)
    want = pn.copy()
    want[np.arange(rows), y] -= np.float32(1)
    np.testing.assert_array_equal(np.asarray(g.numpy()).reshape(rows, cols), want)
    err = ml.SoftmaxLoss(p, labels)
    assert err == pytest.approx(np.count_nonzero(pn.argmax(1) != y) / rows, abs=1e-7)


def test_out_of_range_label_and_errors(mods):
    mt, ml = mods
    z = np.zeros((3, 4), np.float32)
    p, pn = _softmax_gpu(mt, ml, z)
    bad = mt.Tensor_int(np.array([[0, 4, 1]], np.int32), "gpu")
    loss = mt.Tensor_float([1], "gpu")
    ml.CrossEntropyLoss(p, bad, loss)
    assert np.isnan(loss.get_data()[0])
    g = mt.Tensor_float([1], "gpu")
    ml.CrossEntropyLossBackward(p, bad, g)
    gn = np.asarray(g.numpy()).reshape(3, 4)
    np.testing.assert_array_equal(gn[1], pn[1])  # nothing subtracted from the bad row
    assert gn[0, 0] == pn[0, 0] - 1 and gn[2, 1] == pn[2, 1] - 1
    with pytest.raises(ValueError, match="labels"):
        ml.CrossEntropyLoss(p, mt.Tensor_int(np.array([[0, 1]], np.int32), "gpu"), loss)


def test_softmax_cross_entropy_operator():
    import operators as ops

    rng = np.random.default_rng(3)
    z = rng.standard_normal((32, 10)).astype(np.float32)
    y = rng.integers(0, 10, 32)
    X = ops.Tensor(z)
    L = ops.softmaxcrossentropyloss(X, ops.Tensor(y, requires_grad=False))
    loss, err = L.realize_cached_data()
    z64 = z.astype(np.float64)
    lse = logsumexp(z64, axis=1)
    ref_loss = (lse - z64[np.arange(32), y]).sum() / (10 * 32)
    assert loss == pytest.approx(ref_loss, rel=1e-5)
    assert err == pytest.approx(np.count_nonzero(z.argmax(1) != y) / (10 * 32))
    L.backward()
    p = np.exp(z64 - lse[:, None])
    p[np.arange(32), y] -= 1
    np.testing.assert_allclose(np.asarray(X.grad.realize_cached_data()).reshape(32, 10), p / 32, atol=1e-7)
    # the CPU op agrees
    cpu_loss, cpu_err = ops.softmaxloss(ops.Tensor(z), ops.Tensor(y, requires_grad=False)).realize_cached_data()
    assert cpu_loss == pytest.approx(loss, rel=1e-5) and cpu_err == err
