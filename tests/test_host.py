"""CPU tests of the host side: the C-ABI library loads and exports what
include/tt_attn.h declares, argument errors are reported without a GPU, the
myTensor / myLayer modules keep the reference's Python surface and
semantics on the "cpu" device, and the Python autograd layer
(pku-aiprogramming_amd/optimizer) differentiates the reference's op chain
correctly (checked against the float64 oracle).

No test here launches a kernel; GPU parity lives in test_attn_gpu.py.
"""
import ctypes as C
import math
import os
import subprocess
import sys

import numpy as np
import pytest

from oracle import attn_oracle as orc

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def capi():
    import tt_capi

    return tt_capi


# ------------------------------------------------------------------ C-ABI library

def test_library_exports_every_declared_symbol(capi):
    declared = capi.header_functions()
    assert len(declared) >= 25
    out = subprocess.run(["nm", "-D", "--defined-only", capi.LIB_PATH], capture_output=True, text=True, check=True)
    exported = {line.split()[-1] for line in out.stdout.splitlines() if " T " in line}
    missing = [f for f in declared if f not in exported]
    assert not missing, f"declared but not exported: {missing}"
    # and ctypes binds every one of them with a signature
    assert set(declared) == set(capi._SIGS), set(declared) ^ set(capi._SIGS)
    lib = capi.Lib()
    for f in declared:
        assert getattr(lib.lib, f) is not None


def test_library_exports_nothing_else_but_the_abi(capi):
    out = subprocess.run(["nm", "-D", "--defined-only", capi.LIB_PATH], capture_output=True, text=True, check=True)
    tt = sorted(line.split()[-1] for line in out.stdout.splitlines() if " T tt_" in line)
    assert tt == capi.header_functions()


def _gpu_present():
    return os.path.exists("/dev/kfd")


def test_argument_errors_need_no_gpu(capi):
    L = capi.lib()
    f = L.lib.tt_attn_fwd_f32
    # unsupported head dim
    assert f(None, None, None, None, None, 1, 1, 8, 8, 96, 0.1, 0, None) == capi.TT_ERR_UNSUPPORTED
    assert "head dim" in L.last_error()
    # causal with Lq != Lk
    assert f(None, None, None, None, None, 1, 1, 8, 9, 64, 0.1, 1, None) == capi.TT_ERR_ARG
    assert "Lq == Lk" in L.last_error()
    # softmax over zero keys
    assert f(None, None, None, None, None, 1, 1, 8, 0, 64, 0.1, 0, None) == capi.TT_ERR_ARG
    # negative sizes
    assert L.lib.tt_attn_fwd_bf16(None, None, None, None, None, -1, 1, 8, 8, 64, 0.1, 0, None) == capi.TT_ERR_ARG
    # null pointers with a valid shape
    assert f(None, None, None, None, None, 1, 1, 8, 8, 64, 0.1, 0, None) == capi.TT_ERR_ARG
    assert "null pointer" in L.last_error()
    assert L.lib.tt_attn_decode_bf16(None, None, None, None, None, 2, 2, 16, 48, 0.1, None) == capi.TT_ERR_UNSUPPORTED
    assert L.lib.tt_attn_bwd_bf16(*([None] * 9), 1, 1, 4, 4, 64, 0.1, 0, None) == capi.TT_ERR_ARG
    # empty work is a no-op that succeeds
    assert f(None, None, None, None, None, 0, 4, 8, 8, 64, 0.1, 1, None) == capi.TT_OK
    assert f(None, None, None, None, None, 2, 4, 0, 8, 64, 0.1, 0, None) == capi.TT_OK
    assert L.lib.tt_elementwise(99, 0, None, None, None, 4, 0.0, 0.0, 0, None) == capi.TT_ERR_ARG
    assert L.lib.tt_elementwise(0, 0, None, None, None, 0, 0.0, 0.0, 0, None) == capi.TT_OK
    assert L.lib.tt_free(None) == capi.TT_OK
    # row softmax: negative sizes, null pointers, empty work
    sm = L.lib.tt_softmax_rows_f32
    assert sm(None, None, -1, 4, None) == capi.TT_ERR_ARG
    assert sm(None, None, 2, 4, None) == capi.TT_ERR_ARG and "null pointer" in L.last_error()
    assert sm(None, None, 0, 4, None) == capi.TT_OK
    assert sm(None, None, 3, 0, None) == capi.TT_OK
    # read probe: sizes that are not whole 16-byte words, null / unaligned buffers, empty work
    rp = L.lib.tt_read_probe
    assert rp(None, 24, None, None) == capi.TT_ERR_ARG and "multiple of 16" in L.last_error()
    assert rp(None, 32, None, None) == capi.TT_ERR_ARG and "null" in L.last_error()
    assert rp(C.c_void_p(8), 32, C.c_void_p(64), None) == capi.TT_ERR_ARG and "unaligned" in L.last_error()
    assert rp(None, 0, None, None) == capi.TT_OK


@pytest.mark.skipif(_gpu_present(), reason="checks the no-device path")
def test_no_device_is_reported_not_faked(capi):
    L = capi.lib()
    assert L.device_count() == 0
    p = C.c_void_p()
    rc = L.lib.tt_malloc(C.byref(p), 1024)
    assert rc == capi.TT_ERR_HIP and "no HIP device" in L.last_error()
    with pytest.raises(capi.TTError):
        capi.DeviceBuffer((4,), "f32")


def test_bf16_host_rounding_matches_oracle(capi):
    x = np.random.default_rng(3).standard_normal(50000).astype(np.float32) * 7
    x[:4] = [np.inf, -np.inf, 0.0, -0.0]
    np.testing.assert_array_equal(capi.bf16_bits(x), orc.bf16_bits(x))
    np.testing.assert_array_equal(capi.bf16_to_f32(capi.bf16_bits(x)), orc.bf16_round(x))


# ------------------------------------------------------------------ myTensor on the CPU

@pytest.fixture(scope="module")
def mt():
    import myTensor

    return myTensor


def test_tensor_constructors_and_data(mt):
    a = np.arange(24, dtype=np.float32).reshape(2, 3, 4)
    t = mt.Tensor_float(a, "cpu")
    assert t.get_shape() == [2, 3, 4] and t.get_device() == "cpu" and t.Size() == 24
    assert t.get_data() == list(a.ravel())
    np.testing.assert_array_equal(t.numpy(), a)
    # float64 input is cast (pybind11 forcecast), non-contiguous input is copied correctly
    t2 = mt.Tensor_float(np.asfortranarray(a.astype(np.float64)), "cpu")
    np.testing.assert_array_equal(t2.numpy(), a)
    t3 = mt.Tensor_float([2, 2], "cpu", [1.0, 2.0, 3.0])  # short data: leading values copied
    assert t3.get_data()[:3] == [1.0, 2.0, 3.0]
    t4 = mt.Tensor_float(t)
    assert t4.get_data() == t.get_data()
    ti = mt.Tensor_int(np.array([[1, -2], [3, 4]], dtype=np.int32), "cpu")
    assert ti.get_data() == [1, -2, 3, 4]
    td = mt.Tensor_double(np.array([0.1, 0.2]), "cpu")
    assert td.get_data() == [0.1, 0.2]


def test_tensor_bf16_rounds_on_construction(mt):
    x = np.random.default_rng(5).standard_normal(1000).astype(np.float32)
    b = mt.Tensor_bf16(x, "cpu")
    np.testing.assert_array_equal(np.array(b.get_data(), np.float32), orc.bf16_round(x))
    np.testing.assert_array_equal(b.numpy(), orc.bf16_round(x))


def test_tensor_arithmetic_and_errors(mt):
    a = mt.Tensor_float(np.array([1.0, -2.0, 3.0], np.float32), "cpu")
    b = mt.Tensor_float(np.array([0.5, 0.5, -1.0], np.float32), "cpu")
    assert (a + b).get_data() == [1.5, -1.5, 2.0]
    assert (a - b).get_data() == [0.5, -2.5, 4.0]
    with pytest.raises(ValueError, match="Shape mismatch"):
        a + mt.Tensor_float(np.zeros(4, np.float32), "cpu")
    with pytest.raises(ValueError, match="Invalid device"):
        mt.Tensor_float([2], "tpu")
    t = mt.Tensor_float(np.arange(6, dtype=np.float32).reshape(2, 3), "cpu")
    assert t[1].get_data() == [3.0, 4.0, 5.0] and t[1].get_shape() == [3]
    with pytest.raises(ValueError, match="Index out of range"):
        t[2]


def test_tensor_inplace_methods(mt):
    t = mt.Tensor_float(np.array([1.0, -2.0, 3.0, -4.0], np.float32), "cpu")
    t.negative()
    assert t.get_data() == [-1.0, 2.0, -3.0, 4.0]
    t.mults(2.0)
    assert t.get_data() == [-2.0, 4.0, -6.0, 8.0]
    t.floatks(0.25)
    assert t.get_data() == [0.25] * 4
    t.ones()
    assert t.get_data() == [1.0] * 4
    t.zeros()
    assert t.get_data() == [0.0] * 4
    r = mt.Tensor_float([1000], "cpu").random(-1.0, 2.0)
    d = np.array(r.get_data())
    assert d.min() >= -1.0 and d.max() < 2.0 and d.std() > 0.5
    ri = mt.Tensor_int([1000], "cpu").random(3, 5)
    assert set(ri.get_data()) == {3, 4, 5}
    # resize keeps the leading elements (reference Tinytensor.cu:356-382)
    u = mt.Tensor_float(np.arange(6, dtype=np.float32), "cpu")
    u.resize([2, 2])
    assert u.get_shape() == [2, 2] and u.get_data() == [0.0, 1.0, 2.0, 3.0]
    u.resize([1, 6])
    assert u.get_data()[:4] == [0.0, 1.0, 2.0, 3.0]
    f = mt.Tensor_float(np.zeros((2, 3, 4, 5), np.float32), "cpu").flatten()
    assert f.get_shape() == [2, 60]


def test_activations(mt):
    x = np.array([-1.5, 0.0, 2.0], np.float32)
    g = np.array([10.0, 20.0, 30.0], np.float32)
    t, tg = mt.Tensor_float(x, "cpu"), mt.Tensor_float(g, "cpu")
    assert t.ReluForward().get_data() == [0.0, 0.0, 2.0]
    assert t.ReluBackward(tg).get_data() == [0.0, 0.0, 30.0]
    s = 1 / (1 + np.exp(-x.astype(np.float64)))
    np.testing.assert_allclose(t.SigmoidForward().get_data(), s, rtol=1e-6)
    np.testing.assert_allclose(t.SigmoidBackward(tg).get_data(), s * (1 - s) * g, rtol=1e-6)
    assert "Shape: [3]" in repr(t)


def test_layer_functions_reject_cpu_tensors(mt):
    import myLayer

    q = mt.Tensor_float(np.zeros((1, 1, 4, 32), np.float32), "cpu")
    o = mt.Tensor_float([1], "cpu")
    lse = mt.Tensor_float([1], "cpu")
    with pytest.raises(ValueError, match="gpu"):
        myLayer.AttentionForward(q, q, q, o, lse, 0.1, False)
    qb = mt.Tensor_bf16(np.zeros((1, 1, 1, 32), np.float32), "cpu")
    with pytest.raises(ValueError, match="gpu"):
        myLayer.AttentionDecode(qb, qb, qb, qb, 0.1)
    x = mt.Tensor_float(np.zeros((4, 10), np.float32), "cpu")
    with pytest.raises(ValueError, match="gpu"):
        myLayer.SoftmaxForward(x, o)
    w = mt.Tensor_float(np.zeros((10, 3), np.float32), "cpu")
    bias = mt.Tensor_float(np.zeros(3, np.float32), "cpu")
    with pytest.raises(ValueError, match="gpu"):
        myLayer.FcForward(x, o, w, bias)
    with pytest.raises(ValueError, match="gpu"):
        myLayer.FcBackward(x, o, w, bias, o, o, o, o)


# ------------------------------------------------------------------ autograd layer

@pytest.fixture(scope="module")
def ops():
    import operators

    return operators


def test_topo_sort_and_gradient_accumulation(ops):
    import autodiff

    x = ops.Tensor(np.array([2.0, 3.0]))
    y = x * x          # uses x twice
    z = y + x          # and a third time
    w = z.sum()
    order = autodiff.find_topo_sort([w])
    pos = {id(n): i for i, n in enumerate(order)}
    for n in order:
        for i in n.inputs:
            assert pos[id(i)] < pos[id(n)]
    assert order[-1] is w and len(order) == len({id(n) for n in order})
    w.backward()
    np.testing.assert_allclose(x.grad.numpy(), 2 * np.array([2.0, 3.0]) + 1)


def test_deep_graph_needs_no_recursion_limit(ops):
    x = ops.Tensor(np.ones(3))
    y = x
    for _ in range(5000):
        y = y + 1.0
    y.sum().backward()
    np.testing.assert_array_equal(x.grad.numpy(), np.ones(3))


def test_matmul_broadcast_gradient(ops):
    a = ops.Tensor(np.random.default_rng(0).standard_normal((2, 3, 4, 5)))
    b = ops.Tensor(np.random.default_rng(1).standard_normal((5, 6)))
    (a @ b).sum().backward()
    np.testing.assert_allclose(b.grad.numpy(), a.numpy().reshape(-1, 5).T @ np.ones((24, 6)))


@pytest.mark.parametrize("causal", [False, True])
def test_composed_attention_matches_oracle(ops, causal):
    """The reference's op chain built from the autograd ops (the path the
    fused kernel replaces) reproduces the float64 oracle, forward and
    backward, in float32."""
    rng = np.random.default_rng(11)
    shape = (2, 3, 40, 32)
    q, k, v, do = (rng.standard_normal(shape).astype(np.float32) for _ in range(4))
    tq, tk, tv = ops.Tensor(q), ops.Tensor(k), ops.Tensor(v)
    o = ops.attention_composed(tq, tk, tv, causal=causal)
    o.backward(ops.Tensor(do, requires_grad=False))
    scale = float(np.float32(1 / math.sqrt(32)))
    ro, _ = orc.attn_fwd_f64(q, k, v, scale, causal)
    rq, rk, rv = orc.attn_bwd_f64(q, k, v, do, scale, causal)
    assert orc.max_rel_err(o.numpy(), ro) < 1e-5
    assert orc.max_rel_err(tq.grad.numpy(), rq) < 1e-4
    assert orc.max_rel_err(tk.grad.numpy(), rk) < 1e-4
    assert orc.max_rel_err(tv.grad.numpy(), rv) < 1e-4


def test_attention_op_fails_loudly_without_gpu(ops):
    if _gpu_present():
        pytest.skip("GPU present")
    q = ops.Tensor(np.zeros((1, 1, 4, 32), np.float32))
    with pytest.raises(RuntimeError, match="HIP"):
        ops.attention(q, q, q)
    with pytest.raises(ValueError):
        ops.Attention(dtype="fp8")


# ------------------------------------------------------------------ bench contract

def test_bench_refuses_multi_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "4"], capture_output=True, text=True)
    assert r.returncode == 2 and "one GPU" in r.stderr


def test_bench_flop_accounting():
    sys.path.insert(0, ROOT)
    import bench

    assert bench.fwdbwd_flops(4, 32, 4096, 128) == pytest.approx(1.6493e12, rel=1e-4)
    kf = bench.kernel_flops(4, 32, 4096, 128)
    assert sum(kf.values()) == pytest.approx(bench.fwdbwd_flops(4, 32, 4096, 128))
    assert bench.decode_bytes(64, 32, 8192, 128) == 8590983168
