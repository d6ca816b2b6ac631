"""GPU tests of the TinyTensor methods (myTensor, reference src/bind_Tensor.cpp:20-45)
on the "gpu" device, for every dtype including bf16: the elementwise kernels
(tt_elementwise, reference src/TinyTensor_kernels.cu:6-85) against numpy on
the same values, device transfers, copies, indexing and resize.

Bar: float and double and int results equal numpy's (bit-exact for the
arithmetic, within a few ulp for sigmoid, whose exp differs); bf16 results
equal numpy's float32 result rounded to bf16 (round to nearest even), except
sigmoid within one bf16 ulp.
"""
import numpy as np
import pytest

from oracle import attn_oracle as orc

pytestmark = pytest.mark.gpu

DTYPES = ["float", "double", "int", "bf16"]
NP = {"float": np.float32, "double": np.float64, "int": np.int32, "bf16": np.float32}


@pytest.fixture(scope="module")
def mt():
    import myTensor

    assert myTensor.device_count() >= 1, "no HIP device visible"
    return myTensor


def _cls(mt, dt):
    return getattr(mt, "Tensor_" + dt)


def _vals(dt, n, seed):
    """n values as a [1, n] array: a 1-D int array would bind to the
    (shape, device) constructor, which pybind11 tries first (the reference's
    constructor order, src/bind_Tensor.cpp:16-19)."""
    rng = np.random.default_rng(seed)
    if dt == "int":
        return rng.integers(-1000, 1000, (1, n)).astype(np.int32)
    x = (rng.standard_normal((1, n)) * 4).astype(NP[dt])
    return orc.bf16_round(x) if dt == "bf16" else x


def _round(dt, x):
    """What the dtype stores for the exact result x."""
    if dt == "bf16":
        return orc.bf16_round(np.asarray(x, np.float32))
    return np.asarray(x).astype(NP[dt])


def _data(t):
    return np.asarray(t.numpy())


@pytest.mark.parametrize("dt", DTYPES)
def test_transfer_copy_index_resize(mt, dt):
    T = _cls(mt, dt)
    a = _vals(dt, 3 * 5 * 7, 1).reshape(3, 5, 7)
    g = T(a, "gpu")
    assert g.get_device() == "gpu" and g.get_shape() == [3, 5, 7] and g.Size() == 105
    np.testing.assert_array_equal(_data(g).reshape(a.shape), a)
    np.testing.assert_array_equal(np.asarray(g.get_data(), NP[dt]), a.ravel())
    c = T(g)  # deep copy on the device
    g.zeros()
    np.testing.assert_array_equal(_data(c).reshape(a.shape), a)
    assert c[1].get_shape() == [5, 7]
    np.testing.assert_array_equal(_data(c[1]).reshape(5, 7), a[1])
    h = T(c).cpu()
    assert h.get_device() == "cpu"
    np.testing.assert_array_equal(_data(h).reshape(a.shape), a)
    back = T(h).gpu()
    assert back.get_device() == "gpu"
    c.resize([2, 4])
    assert c.get_shape() == [2, 4]
    np.testing.assert_array_equal(_data(c).ravel(), a.ravel()[:8])
    f = T(np.zeros((2, 3, 4, 5), NP[dt]), "gpu").flatten()
    assert f.get_shape() == [2, 60]


@pytest.mark.parametrize("dt", DTYPES)
def test_elementwise_arithmetic(mt, dt):
    T = _cls(mt, dt)
    n = 100_003  # not a multiple of any block size
    a, b = _vals(dt, n, 2), _vals(dt, n, 3)
    ga, gb = T(a, "gpu"), T(b, "gpu")
    wide = np.float64 if dt != "int" else np.int64
    np.testing.assert_array_equal(_data(ga + gb), _round(dt, a.astype(wide) + b))
    np.testing.assert_array_equal(_data(ga - gb), _round(dt, a.astype(wide) - b))
    t = T(ga)
    t.negative()
    np.testing.assert_array_equal(_data(t), _round(dt, -a.astype(wide)))
    t = T(ga)
    if dt == "int":
        t.mults(3)
        np.testing.assert_array_equal(_data(t), a * 3)
    else:
        t.mults(0.75)  # exact in every float format
        np.testing.assert_array_equal(_data(t), _round(dt, a.astype(np.float64) * 0.75))
    t.ones()
    np.testing.assert_array_equal(_data(t), np.ones((1, n), NP[dt]))
    t.floatks(2.5)
    np.testing.assert_array_equal(_data(t), _round(dt, np.full((1, n), 2.5 if dt != "int" else 2)))
    t.zeros()
    assert not _data(t).any()


@pytest.mark.parametrize("dt", ["float", "double", "bf16"])
def test_activations(mt, dt):
    T = _cls(mt, dt)
    n = 65_537
    x, g = _vals(dt, n, 4), _vals(dt, n, 5)
    gx, gg = T(x, "gpu"), T(g, "gpu")
    np.testing.assert_array_equal(_data(gx.ReluForward()), _round(dt, np.maximum(x, 0)))
    np.testing.assert_array_equal(_data(gx.ReluBackward(gg)), _round(dt, np.where(x > 0, g, 0)))
    s = 1.0 / (1.0 + np.exp(-x.astype(np.float64)))
    sg = s * (1 - s) * g
    ys, ysg = _data(gx.SigmoidForward()), _data(gx.SigmoidBackward(gg))
    if dt == "bf16":
        # one bf16 ulp (2^-8 relative) of the exact value
        assert np.all(np.abs(ys - s) <= 2.0 ** -8 * np.abs(s) + 1e-30)
        assert np.all(np.abs(ysg - sg) <= 2.0 ** -7 * np.abs(sg) + 1e-6)
    else:
        # s (1 - s) cancels for large x: absolute error ~ eps |g|
        eps = 2.0 ** -23 if dt == "float" else 2.0 ** -52
        np.testing.assert_allclose(ys, s, rtol=40 * eps)
        np.testing.assert_allclose(ysg, sg, rtol=40 * eps, atol=4 * eps * np.abs(g).max())


@pytest.mark.parametrize("dt", DTYPES)
def test_random_fills_the_range(mt, dt):
    T = _cls(mt, dt)
    if dt == "int":
        r = _data(T([20000], "gpu").random(3, 7))
        assert set(np.unique(r)) == {3, 4, 5, 6, 7}
        return
    r = _data(T([20000], "gpu").random(-1.0, 2.0)).astype(np.float64)
    assert r.min() >= -1.0 and r.max() <= 2.0 and abs(r.mean() - 0.5) < 0.05 and r.std() > 0.8
    if dt == "bf16":
        np.testing.assert_array_equal(r.astype(np.float32), orc.bf16_round(r.astype(np.float32)))


def test_bf16_repr_and_shape_errors(mt):
    t = mt.Tensor_bf16(np.array([1.0, 2.0, 3.0], np.float32), "gpu")
    assert "Shape: [3]" in repr(t)
    with pytest.raises(ValueError, match="Shape mismatch"):
        t + mt.Tensor_bf16(np.zeros(4, np.float32), "gpu")


EW_OPS = {"add": 0, "sub": 1, "fill": 2, "neg": 3, "scale": 4, "relu": 5, "relu_bwd": 6, "sigmoid": 7,
          "sigmoid_bwd": 8, "uniform": 9}
CAPI_DT = {"float": ("f32", 0, np.float32), "double": ("f64", 1, np.float64), "int": ("i32", 2, np.int32),
           "bf16": ("bf16", 3, np.uint16)}


@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("n", [1, 7, 13, 4099, 100_003])
def test_elementwise_vector_and_scalar_paths_agree(dt, n):
    """tt_elementwise takes a 16-byte vector kernel when every operand is
    16-byte aligned (the n % (16 / itemsize) tail elements done one by one)
    and a one-element-per-thread kernel otherwise.  Run every op on aligned
    buffers and on the same values one element past the start of a block
    (misaligned for every dtype); the stored bytes must be identical, and the
    aligned result equals numpy's where the op is exact."""
    import tt_capi as capi

    name, code, raw = CAPI_DT[dt]
    item = capi.DeviceBuffer.ITEM[name]
    x, y = _vals(dt, n, 11).ravel(), _vals(dt, n, 12).ravel()
    L = capi.lib()

    def buffers(off):
        bufs = []
        for v in (x, y, None):
            b = capi.DeviceBuffer((n + 1,), name)
            if v is not None:
                host = np.concatenate([np.zeros(1, v.dtype), v]) if off else np.concatenate([v, np.zeros(1, v.dtype)])
                b.upload(host)
            bufs.append(b)
        return bufs

    alpha, beta = (3.0, 9.0) if dt == "int" else (0.75, 2.5)
    for op, k in EW_OPS.items():
        out = []
        for off in (0, 1):
            ba, bb, bc = buffers(off)
            sh = off * item
            L.call("tt_elementwise", k, code, bc.ptr + sh, ba.ptr + sh, bb.ptr + sh, n, alpha, beta, 5, None)
            L.sync()
            got = bc.download_bytes().view(raw)
            out.append(got[off:off + n].copy())
        np.testing.assert_array_equal(out[0], out[1], err_msg=f"{dt} {op} n={n}")
        if op in ("add", "sub", "neg") or (op == "scale" and dt != "int"):
            wide = np.float64 if dt != "int" else np.int64
            ref = {"add": x.astype(wide) + y, "sub": x.astype(wide) - y, "neg": -x.astype(wide),
                   "scale": x.astype(np.float64) * alpha}[op]
            want = _round(dt, ref)
            if dt == "bf16":
                want = want.astype(np.float32).view(np.uint32) >> 16
            np.testing.assert_array_equal(out[0].astype(np.int64), np.asarray(want).astype(np.int64),
                                          err_msg=f"{dt} {op} n={n}")
