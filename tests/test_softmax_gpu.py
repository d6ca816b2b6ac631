"""GPU parity tests of the row softmax (``tt_softmax_rows_f32`` and
``myLayer.SoftmaxForward``) against the float64 oracle
(``oracle.attn_oracle.softmax_rows_f64``).

The kernel exponentiates with v_exp_f32 (2^(x log2 e)), whose relative error
grows with |x - max|; terms far below the row max carry small weights, so the
normwise error max|y - ref| / max|ref| stays near float32 rounding.  Bar:
normwise <= 2e-6 (the fp32 target is 1e-4), row sums within 1e-5 of 1, and
exact zeros / NaNs where the reference's x - max gives them.
"""
import sys

import numpy as np
import pytest

from oracle import attn_oracle as orc

pytestmark = pytest.mark.gpu

TOL = 2e-6


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def capi():
    import tt_capi

    assert tt_capi.lib().device_count() >= 1, "no HIP device visible"
    return tt_capi


def _softmax_gpu(capi, x, inplace=False):
    dx = capi.DeviceBuffer.from_numpy(x, "f32")
    dy = dx if inplace else capi.DeviceBuffer(x.shape, "f32")
    capi.softmax_rows(dx, dy)
    capi.lib().sync()
    return dy.download()


def _check(name, y, x):
    ref = orc.softmax_rows_f64(x)
    err = orc.max_rel_err(y, ref)
    sums = np.abs(y.astype(np.float64).sum(-1) - 1.0).max() if y.size else 0.0
    _say(f"  {name}: max-rel-err {err:.3e}, max |row sum - 1| {sums:.2e}")
    assert err <= TOL, f"{name}: {err:.3e} > {TOL:g}"
    assert sums <= 1e-5


# every kernel shape: lane groups of 1..64, one wave with 2..32 elements per
# lane, workgroups of 4 / 16 waves with 16..64 elements per lane, rows split
# over workgroups (aligned lengths from 8196 on: 16384, 32768, 65536, 200000)
# and the two-pass stream, at the edges of each
COLS = [1, 2, 3, 5, 8, 10, 16, 17, 31, 32, 33, 63, 64, 65, 100, 128, 129, 255, 256, 257, 500, 512, 513, 1000,
        1024, 1025, 2047, 2048, 2049, 4095, 4096, 4097, 8192, 8193, 10000, 16384, 16385, 32768, 32769, 65535,
        65536, 65537, 200000]


@pytest.mark.parametrize("cols", COLS)
def test_rows_of_every_length(capi, cols):
    rows = max(1, min(517, 2_000_000 // cols))
    _say(f"softmax rows={rows} cols={cols}")
    x = (np.random.default_rng(cols).standard_normal((rows, cols)) * 3).astype(np.float32)
    _check(f"[{rows}, {cols}]", _softmax_gpu(capi, x), x)


@pytest.mark.parametrize("cols", [10, 100, 1000, 3000, 40000, 70000])
def test_in_place(capi, cols):
    _say(f"softmax in place cols={cols}")
    x = np.random.default_rng(7 + cols).standard_normal((33, cols)).astype(np.float32)
    _check("in place", _softmax_gpu(capi, x, inplace=True), x)


@pytest.mark.parametrize("rows,cols", [(300_000, 70), (65_600, 2100)])
def test_many_rows_grid_stride(capi, rows, cols):
    # more rows than the launch's 65536 workgroups cover at once (4 rows per
    # workgroup for one wave per row; one row per workgroup of 4 waves)
    x = np.random.default_rng(11).standard_normal((rows, cols)).astype(np.float32)
    _say(f"softmax rows={rows} cols={cols} (grid-stride)")
    _check(f"[{rows}, {cols}]", _softmax_gpu(capi, x), x)


@pytest.mark.parametrize("cols", [7, 300, 5000, 70000])
def test_large_magnitudes_and_infinities(capi, cols):
    _say(f"softmax extremes cols={cols}")
    rng = np.random.default_rng(20 + cols)
    x = (rng.standard_normal((6, cols)) * 60).astype(np.float32)  # exp would overflow without the max shift
    x[1, ::3] = -np.inf          # masked entries -> exactly 0
    x[2, :] = -np.inf            # a fully masked row -> NaN (the reference's -inf - -inf)
    x[3, cols // 2] = np.inf     # +inf -> NaN row
    x[4, :] = 88.0               # constant row -> 1 / cols
    y = _softmax_gpu(capi, x)
    ref = orc.softmax_rows_f64(x)
    assert np.isnan(y[2]).all() and np.isnan(y[3]).all()
    assert (y[1, ::3] == 0).all()
    np.testing.assert_allclose(y[4], 1.0 / cols, rtol=1e-6)
    keep = [0, 1, 4, 5]
    err = orc.max_rel_err(y[keep], ref[keep])
    _say(f"  finite rows: max-rel-err {err:.3e}")
    assert err <= TOL


# Rows split over workgroups that exchange (max, sum) partials through device
# memory (16-byte aligned rows of 8193 .. 2 Mi columns): 3, 16, 32 and 64
# chunks, a ragged last chunk, and the first length past the split range
# (the two-pass stream kernel).
@pytest.mark.parametrize("rows,cols", [(40, 12288), (6, 262144), (3, 1048576), (2, 2097152), (2, 2097156),
                                       (7, 1000004)])
def test_split_rows(capi, rows, cols):
    _say(f"softmax split rows={rows} cols={cols}")
    x = (np.random.default_rng(cols + rows).standard_normal((rows, cols)) * 3).astype(np.float32)
    _check(f"[{rows}, {cols}]", _softmax_gpu(capi, x), x)


def test_split_grid_far_beyond_the_resident_workgroups(capi):
    # 4000 rows x 3 chunks = 12000 workgroups: rows wait for chunks that are
    # dispatched only after earlier rows have finished
    rows, cols = 4000, 12288
    _say(f"softmax split rows={rows} cols={cols} (grid beyond the resident workgroups)")
    x = np.random.default_rng(99).standard_normal((rows, cols)).astype(np.float32)
    _check(f"[{rows}, {cols}]", _softmax_gpu(capi, x), x)


def test_split_chunks_without_a_finite_value_and_nan(capi):
    cols = 65536  # 8 chunks of 8192 columns
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((5, cols)) * 4).astype(np.float32)
    x[0, 8192:3 * 8192] = -np.inf     # two whole chunks masked: exact zeros there, the rest as usual
    x[1, :cols - 8192] = -np.inf      # only the last chunk finite
    x[2, 20000] = np.nan              # NaN in one chunk -> the whole row NaN
    x[3, :] = -np.inf                 # every chunk masked -> NaN row
    y = _softmax_gpu(capi, x)
    ref = orc.softmax_rows_f64(x)
    assert (y[0, 8192:3 * 8192] == 0).all() and (y[1, :cols - 8192] == 0).all()
    assert np.isnan(y[2]).all() and np.isnan(y[3]).all()
    err = orc.max_rel_err(y[[0, 1, 4]], ref[[0, 1, 4]])
    _say(f"  finite rows: max-rel-err {err:.3e}")
    assert err <= TOL


def test_split_repeated_calls_reuse_the_partials_buffer(capi):
    """Consecutive calls on one stream reuse the slot buffer with a new
    generation each: stale partials of an earlier call (other values, another
    chunk layout) must never be taken for the current ones."""
    rng = np.random.default_rng(12)
    for rows, cols in [(64, 65536), (64, 65536), (32, 131072), (200, 16384), (64, 65536)]:
        x = (rng.standard_normal((rows, cols)) * 2 + rng.standard_normal()).astype(np.float32)
        _check(f"repeat [{rows}, {cols}]", _softmax_gpu(capi, x), x)


def test_split_random_shapes(capi):
    """Seeded random aligned lengths, log-uniform over the whole split range
    (4 Ki .. 32 Ki column chunks, ragged last chunks of any multiple of 4
    columns), random row counts, scales and offsets."""
    rng = np.random.default_rng(2024)
    for i in range(12):
        cols = 4 * int(np.exp(rng.uniform(np.log(8196 // 4), np.log(2 * 1024 * 1024 // 4))))
        rows = int(rng.integers(1, max(2, 6_000_000 // cols) + 1))
        scale, shift = float(rng.uniform(0.5, 8)), float(rng.uniform(-50, 50))
        _say(f"softmax split random #{i}: rows={rows} cols={cols} scale={scale:.2f} shift={shift:.1f}")
        x = (rng.standard_normal((rows, cols)) * scale + shift).astype(np.float32)
        _check(f"random [{rows}, {cols}]", _softmax_gpu(capi, x), x)


def test_layer_softmax_forward_matches_oracle():
    """myLayer.SoftmaxForward(input, output) as the reference's cross-entropy
    caller uses it (optimizer/operators.py:642-647): [batch, 10] on "gpu";
    output takes the input's shape; any rank >= 1 softmaxes the last axis."""
    import myLayer
    import myTensor as mt

    assert mt.device_count() >= 1
    rng = np.random.default_rng(5)
    for shape in [(64, 10), (3, 4, 257), (2000,), (2, 3, 4, 5)]:
        x = rng.standard_normal(shape).astype(np.float32)
        t = mt.Tensor_float(x, "gpu")
        out = mt.Tensor_float([1], "gpu")
        myLayer.SoftmaxForward(t, out)
        assert out.get_shape() == list(shape)
        _check(f"SoftmaxForward {shape}", out.numpy().reshape(shape), x)
    # output may be the input tensor itself
    x = rng.standard_normal((5, 40)).astype(np.float32)
    t = mt.Tensor_float(x, "gpu")
    myLayer.SoftmaxForward(t, t)
    _check("SoftmaxForward in place", t.numpy().reshape(5, 40), x)
    # a cpu output tensor moves to the gpu, as the reference's output = input makes it
    out = mt.Tensor_float([2, 2], "cpu")
    myLayer.SoftmaxForward(mt.Tensor_float(x, "gpu"), out)
    assert out.get_device() == "gpu"
    _check("SoftmaxForward cpu output", out.numpy().reshape(5, 40), x)
