"""GPU tests of max pooling: myLayer.MaxPoolingForward / MaxPoolingBackward
(reference src/Layers.cu:254-322, kernels src/Layers_kernels.cu:109-175;
C-ABI tt_maxpool_f32 / tt_maxpool_backward_f32) and ``operators.maxpool``
(optimizer/operators.py:570-602).

Oracle: numpy loops over the windows (clipped to the image, first largest
element in row-major order).  Bar: bitwise (a max and a sum of at most
kh * kw gradients in a fixed order; the test values are small integers
and halves, so every sum is exact).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def mods():
    import myLayer
    import myTensor

    assert myTensor.device_count() >= 1, "no HIP device visible"
    return myTensor, myLayer


def _ref(x, kh, kw, ph, pw, sh, sw, g):
    N, C, H, W = x.shape
    oh, ow = (H + 2 * ph - kh) // sh + 1, (W + 2 * pw - kw) // sw + 1
    out = np.empty((N, C, oh, ow), np.float32)
    mask = np.empty((N, C, oh, ow), np.float32)
    gin = np.zeros_like(x)
    for n in range(N):
        for c in range(C):
            for i in range(oh):
                for j in range(ow):
                    best, arg = -np.float32(3.402823466e38), -1
                    for y in range(max(i * sh - ph, 0), min(i * sh - ph + kh, H)):
                        for xx in range(max(j * sw - pw, 0), min(j * sw - pw + kw, W)):
                            if x[n, c, y, xx] > best:
                                best, arg = x[n, c, y, xx], y * W + xx
                    out[n, c, i, j], mask[n, c, i, j] = best, arg
                    if arg >= 0 and g is not None:
                        gin[n, c, arg // W, arg % W] += g[n, c, i, j]
    return out, mask, gin


# (N, C, H, W, kh, kw, pad_h, pad_w, stride_h, stride_w): the MNIST 2 x 2 / 2,
# ragged edges, padding, and overlapping windows (stride < kernel)
CASES = [(2, 3, 8, 8, 2, 2, 0, 0, 2, 2), (1, 2, 7, 9, 2, 2, 0, 0, 2, 2), (2, 2, 6, 6, 3, 3, 1, 1, 2, 2),
         (1, 3, 7, 7, 3, 3, 0, 0, 1, 1), (2, 1, 5, 8, 2, 3, 1, 0, 1, 2)]


@pytest.mark.parametrize("case", CASES)
def test_maxpool_forward_backward(mods, case):
    mt, ml = mods
    N, C, H, W, kh, kw, ph, pw, sh, sw = case
    rng = np.random.default_rng(sum(case))
    x = rng.integers(-8, 9, (N, C, H, W)).astype(np.float32) / 2  # ties on purpose
    out_ref, mask_ref, _ = _ref(x, kh, kw, ph, pw, sh, sw, None)
    g = (rng.integers(-4, 5, out_ref.shape) / 2).astype(np.float32)
    _, _, gin_ref = _ref(x, kh, kw, ph, pw, sh, sw, g)
    out, mask = mt.Tensor_float([1], "gpu"), mt.Tensor_float([1], "gpu")
    ml.MaxPoolingForward(mt.Tensor_float(x, "gpu"), out, mask, [kh, kw], ph, pw, sh, sw)
    np.testing.assert_array_equal(np.asarray(out.numpy()).reshape(out_ref.shape), out_ref)
    np.testing.assert_array_equal(np.asarray(mask.numpy()).reshape(mask_ref.shape), mask_ref)
    gx = mt.Tensor_float([1], "gpu")
    ml.MaxPoolingBackward(mt.Tensor_float(g, "gpu"), mask, gx, [N, C, H, W], [kh, kw], ph, pw, sh, sw)
    assert gx.get_shape() == [N, C, H, W]
    np.testing.assert_array_equal(np.asarray(gx.numpy()).reshape(x.shape), gin_ref)


def test_maxpool_operator():
    import operators as ops

    rng = np.random.default_rng(5)
    x = rng.integers(-8, 9, (2, 3, 6, 6)).astype(np.float32) / 2
    X = ops.Tensor(x)
    y = ops.maxpool(X)
    out_ref, _, _ = _ref(x, 2, 2, 0, 0, 2, 2, None)
    np.testing.assert_array_equal(np.asarray(y.realize_cached_data()).reshape(out_ref.shape), out_ref)
    g = (rng.integers(-4, 5, out_ref.shape) / 2).astype(np.float32)
    y.backward(ops.Tensor(g, requires_grad=False))
    _, _, gin_ref = _ref(x, 2, 2, 0, 0, 2, 2, g)
    np.testing.assert_array_equal(np.asarray(X.grad.realize_cached_data()).reshape(x.shape), gin_ref)
