"""CPU tests of ``operators.softmaxloss`` (reference optimizer/operators.py:
604-632): the loss and error rate divided by 10 * batch as the reference
reports them, against scipy's logsumexp, and the gradient (softmax -
onehot) / batch against a central finite difference of the summed loss."""
import numpy as np
import pytest
from scipy.special import logsumexp


@pytest.fixture(scope="module")
def ops():
    import operators

    return operators


def test_softmaxloss_values_and_gradient(ops):
    rng = np.random.default_rng(11)
    z = rng.standard_normal((16, 7))
    y = rng.integers(0, 7, 16)
    X = ops.Tensor(z)
    L = ops.softmaxloss(X, ops.Tensor(y, requires_grad=False))
    loss, err = L.realize_cached_data()
    total = (logsumexp(z, axis=1) - z[np.arange(16), y]).sum()
    assert loss == pytest.approx(total / 160, rel=1e-12)
    assert err == np.count_nonzero(z.argmax(1) != y) / 160
    L.backward()
    g = np.asarray(X.grad.realize_cached_data())
    # d(total / batch) / dz by central differences
    h = 1e-6
    num = np.zeros_like(z)
    for i in range(16):
        for j in range(7):
            zp, zm = z.copy(), z.copy()
            zp[i, j] += h
            zm[i, j] -= h
            fp = (logsumexp(zp, axis=1) - zp[np.arange(16), y]).sum()
            fm = (logsumexp(zm, axis=1) - zm[np.arange(16), y]).sum()
            num[i, j] = (fp - fm) / (2 * h) / 16
    np.testing.assert_allclose(g, num, atol=1e-8)
