"""GPU tests of host <-> device transfers: ``tt_memcpy_h2d`` / ``tt_memcpy_d2h``
(the reference's synchronous cudaMemcpy, src/Tinytensor.cu:40,61,213,238,251),
the converting bf16 copies ``tt_upload_bf16_from_f32`` /
``tt_download_bf16_to_f32``, pinned host memory (``tt_host_malloc``), and the
TinyTensor methods built on them.

Bar: bit-exact.  Sizes straddle the 4 MiB direct-copy threshold and the
16 MiB staging chunks (odd byte counts, unaligned host pointers, a partial
last chunk); bf16 rounding is checked bit for bit against numpy's round to
nearest even on the special values (signed zeros, subnormals, infinities,
NaNs, the overflow edge, ties).
"""
import sys
import threading

import numpy as np
import pytest

from oracle import attn_oracle as orc

pytestmark = pytest.mark.gpu

MIB = 1 << 20
CHUNK = 16 * MIB


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def capi():
    import tt_capi

    assert tt_capi.lib().device_count() >= 1, "no HIP device visible"
    return tt_capi


def _bytes(n, seed):
    return np.random.default_rng(seed).integers(0, 256, n, dtype=np.uint8)


BYTE_SIZES = [1, 3, 4 * MIB - 1, 4 * MIB, 4 * MIB + 1, CHUNK - 1, CHUNK, CHUNK + 7, 2 * CHUNK, 3 * CHUNK + 12345]


@pytest.mark.parametrize("nbytes", BYTE_SIZES)
def test_plain_copies_round_trip(capi, nbytes):
    _say(f"h2d/d2h {nbytes} bytes")
    L = capi.lib()
    host = _bytes(nbytes + 1, nbytes)
    d = capi.DeviceBuffer((nbytes + 64,), "i32")          # room to spare
    src = host[1:]                                           # an odd host address
    L.call("tt_memcpy_h2d", d.ptr + 3, src.ctypes.data, nbytes)   # an odd device address
    back = np.zeros(nbytes + 2, np.uint8)
    L.call("tt_memcpy_d2h", back.ctypes.data + 1, d.ptr + 3, nbytes)
    np.testing.assert_array_equal(back[1:-1], src)
    assert back[0] == 0 and back[-1] == 0                    # nothing written outside the range


def _special_f32():
    bits = np.array([
        0x00000000, 0x80000000,                  # +-0
        0x00000001, 0x807fffff, 0x00008000,      # subnormals
        0x00018000, 0x00028000,                  # ties (to even: down, up)
        0x3f808000, 0x3f818000, 0x3f80ffff, 0x3f807fff,
        0x7f7fffff, 0xff7fffff, 0x7f7f7fff,      # overflow edge: rounds to +-inf / stays finite
        0x7f800000, 0xff800000,                  # +-inf
        0x7f800001, 0x7fc00000, 0xffffffff, 0x7fbfffff,   # NaNs (signalling and quiet)
    ], np.uint32)
    return bits.view(np.float32)


@pytest.mark.parametrize("n", [1, 20, 2 * MIB - 3, 8 * MIB, 8 * MIB + 5, 20 * MIB + 1])
def test_bf16_upload_rounds_like_numpy(capi, n):
    """fp32 -> bf16 in the staging pass equals numpy's round to nearest even,
    bit for bit; the download widens exactly."""
    _say(f"bf16 upload/download n={n}")
    L = capi.lib()
    x = (np.random.default_rng(n).standard_normal(n) * 100).astype(np.float32)
    sp = _special_f32()
    x[: min(n, sp.size)] = sp[: min(n, sp.size)]
    d = capi.DeviceBuffer((n,), "bf16")
    L.call("tt_upload_bf16_from_f32", d.ptr, x.ctypes.data, n)
    bits = d.download_bytes()
    want = capi.bf16_bits(x)
    nan = np.isnan(x)
    np.testing.assert_array_equal(bits[~nan], want[~nan])
    # NaN stays NaN with its sign, quietened
    assert np.all((bits[nan] & 0x7F80) == 0x7F80) and np.all((bits[nan] & 0x0040) != 0)
    assert np.array_equal(bits[nan] >> 15, want[nan] >> 15)
    out = np.full(n, 7.0, np.float32)
    L.call("tt_download_bf16_to_f32", out.ctypes.data, d.ptr, n)
    np.testing.assert_array_equal(out.view(np.uint32), bits.astype(np.uint32) << 16)
    # against the oracle's rounding on the finite values
    fin = np.isfinite(x)
    np.testing.assert_array_equal(out[fin], orc.bf16_round(x[fin]))


def test_pinned_host_memory_copies_directly(capi):
    L = capi.lib()
    import ctypes as C

    n = 24 * MIB + 4
    p = C.c_void_p()
    L.call("tt_host_malloc", C.byref(p), n)
    try:
        view = np.ctypeslib.as_array((C.c_uint8 * n).from_address(p.value))
        view[:] = _bytes(n, 9)
        d = capi.DeviceBuffer((n // 4,), "i32")
        L.call("tt_memcpy_h2d", d.ptr, p.value, n)
        got = d.download_bytes().view(np.uint8)
        np.testing.assert_array_equal(got, view)
        view[:] = 0
        L.call("tt_memcpy_d2h", p.value, d.ptr, n)
        np.testing.assert_array_equal(view, got)
    finally:
        L.call("tt_host_free", p.value)
    L.call("tt_host_free", None)


def test_copies_from_two_threads(capi):
    """Staged copies from several host threads at once (ctypes drops the GIL
    during the calls) keep each transfer whole."""
    L = capi.lib()
    n = 40 * MIB + 12
    errors = []

    def worker(seed):
        try:
            host = _bytes(n, seed)
            d = capi.DeviceBuffer((n // 4,), "i32")
            x = np.random.default_rng(seed).standard_normal(5 * MIB + 3).astype(np.float32)
            db = capi.DeviceBuffer(x.shape, "bf16")
            for _ in range(3):
                L.call("tt_memcpy_h2d", d.ptr, host.ctypes.data, n)
                back = np.empty(n, np.uint8)
                L.call("tt_memcpy_d2h", back.ctypes.data, d.ptr, n)
                assert np.array_equal(back, host)
                db.upload(x)
                assert np.array_equal(db.download(), orc.bf16_round(x))
        except Exception as e:  # pragma: no cover - reported below
            errors.append(repr(e))

    th = [threading.Thread(target=worker, args=(s,)) for s in (1, 2, 3)]
    for t in th:
        t.start()
    for t in th:
        t.join()
    assert not errors, errors


@pytest.mark.parametrize("dt", ["float", "double", "int", "bf16"])
def test_tensor_large_round_trips(dt):
    """TinyTensor upload, numpy(), get_data(), cpu() and gpu() through the
    staged path (sizes above one staging chunk, not a multiple of it)."""
    import myTensor as mt

    assert mt.device_count() >= 1
    T = getattr(mt, "Tensor_" + dt)
    n = 6 * MIB + 7
    rng = np.random.default_rng(3)
    if dt == "int":
        a = rng.integers(-2**31, 2**31 - 1, (1, n), dtype=np.int64).astype(np.int32)
    else:
        a = (rng.standard_normal((1, n)) * 50).astype(np.float64 if dt == "double" else np.float32)
        if dt == "bf16":
            a = orc.bf16_round(a)
    _say(f"Tensor_{dt} round trips n={n}")
    g = T(a, "gpu")
    np.testing.assert_array_equal(np.asarray(g.numpy()), a)
    h = T(g).cpu()
    np.testing.assert_array_equal(np.asarray(h.numpy()), a)
    h.gpu()
    np.testing.assert_array_equal(np.asarray(h.numpy()), a)
    if dt != "bf16":
        return
    # a float32 array that is not on the bf16 grid rounds on upload
    x = rng.standard_normal((3, 1000)).astype(np.float32)
    np.testing.assert_array_equal(np.asarray(T(x, "gpu").numpy()), orc.bf16_round(x))
    # the list constructor pads with zeros past the data
    t = T([2, 3], "gpu", [1.5, 2.0, 3.00390625])
    np.testing.assert_array_equal(np.asarray(t.get_data(), np.float32), [1.5, 2.0, 3.0, 0, 0, 0])


def test_device_pointer_as_host_side_is_an_error(capi):
    """A device pointer passed where host memory belongs is refused before
    any copy (the staged path's host threads could not touch it)."""
    a = capi.DeviceBuffer((8 * MIB,), "i32")
    b = capi.DeviceBuffer((8 * MIB,), "i32")
    L = capi.lib()
    for fn, args in (("tt_memcpy_h2d", (a.ptr, b.ptr, 32 * MIB)), ("tt_memcpy_d2h", (a.ptr, b.ptr, 32 * MIB)),
                     ("tt_memcpy_h2d", (a.ptr, b.ptr, 64)),
                     ("tt_upload_bf16_from_f32", (a.ptr, b.ptr, 1000)),
                     ("tt_download_bf16_to_f32", (a.ptr, b.ptr, 1000))):
        with pytest.raises(capi.TTError) as ei:
            L.call(fn, *args)
        assert ei.value.code == capi.TT_ERR_ARG and "device memory" in str(ei.value)
    # the library still works afterwards
    x = _bytes(4096, 5)
    L.call("tt_memcpy_h2d", a.ptr, x.ctypes.data, 4096)
    np.testing.assert_array_equal(a.download_bytes().view(np.uint8)[:4096], x)
