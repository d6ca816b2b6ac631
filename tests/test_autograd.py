"""CPU tests of the Python autograd layer (optimizer/): graph order, gradient
accumulation, and every operator's gradient rule against central finite
differences of its own forward, so a wrong rule (a dropped factor, a swapped
operand, a missing broadcast reduction) fails here.  No GPU is used.
"""
import numpy as np
import pytest


@pytest.fixture(scope="module")
def ops():
    import operators

    return operators


def _fd_grad(f, arrays, i, eps=1e-6):
    """Central finite-difference gradient of sum(f(*arrays) * W) w.r.t.
    arrays[i], for the fixed random weights W that _check uses."""
    x = arrays[i]
    g = np.zeros_like(x)
    it = np.nditer(x, flags=["multi_index"])
    for _ in it:
        idx = it.multi_index
        old = x[idx]
        x[idx] = old + eps
        up = f(*arrays)
        x[idx] = old - eps
        dn = f(*arrays)
        x[idx] = old
        g[idx] = (up - dn) / (2 * eps)
    return g


def _check(ops, build, arrays, rtol=1e-6, atol=1e-8):
    """build(*tensors) -> Tensor.  Compares .grad of every input against
    finite differences of sum(build(...) * W) evaluated in float64."""
    rng = np.random.default_rng(0)
    arrays = [np.array(a, dtype=np.float64) for a in arrays]
    out = build(*[ops.Tensor(a) for a in arrays])
    W = rng.standard_normal(out.shape)

    def scalar(*xs):
        return float(np.sum(build(*[ops.Tensor(x) for x in xs]).numpy() * W))

    ts = [ops.Tensor(a) for a in arrays]
    y = build(*ts)
    y.backward(ops.Tensor(W, requires_grad=False))
    for i, t in enumerate(ts):
        fd = _fd_grad(scalar, arrays, i)
        np.testing.assert_allclose(t.grad.numpy(), fd, rtol=rtol, atol=atol, err_msg=f"input {i}")


def _fn(name):
    import operators

    return getattr(operators, name)


rng0 = np.random.default_rng(42)
A = rng0.standard_normal((3, 4))
B = rng0.standard_normal((3, 4))
POS = rng0.uniform(0.5, 2.0, (3, 4))


@pytest.mark.parametrize("name,build,arrays", [
    ("add", lambda a, b: a + b, [A, B]),
    ("sub", lambda a, b: a - b, [A, B]),
    ("mul", lambda a, b: a * b, [A, B]),
    ("div", lambda a, b: a / b, [A, POS]),
    ("pow", lambda a, b: a ** b, [POS, B]),
    ("add_scalar", lambda a: a + 1.5, [A]),
    ("rsub", lambda a: 2.0 - a, [A]),
    ("mul_scalar", lambda a: a * -3.0, [A]),
    ("div_scalar", lambda a: a / 4.0, [A]),
    ("rdiv", lambda a: 3.0 / a, [POS]),
    ("power_scalar", lambda a: a ** 3, [A]),
    ("neg", lambda a: -a, [A]),
    ("log", lambda a: _fn("log")(a), [POS]),
    ("exp", lambda a: _fn("exp")(a), [A]),
])
def test_elementwise_rules_match_finite_differences(ops, name, build, arrays):
    _check(ops, build, arrays)


def test_shape_rules_match_finite_differences(ops):
    x = rng0.standard_normal((2, 3, 4))
    _check(ops, lambda a: a.transpose(), [x])
    _check(ops, lambda a: a.transpose((0, 2)), [x])
    _check(ops, lambda a: a.reshape((6, 4)), [x])
    _check(ops, lambda a: a.sum(), [x])
    _check(ops, lambda a: a.sum(1), [x])
    _check(ops, lambda a: a.sum((0, 2)), [x])
    _check(ops, lambda a: a.broadcast_to((5, 2, 3, 4)), [x])
    _check(ops, lambda a: a.broadcast_to((2, 3, 4)), [rng0.standard_normal((1, 3, 1))])


def test_matmul_rules_with_batch_broadcast(ops):
    _check(ops, lambda a, b: a @ b, [rng0.standard_normal((3, 4)), rng0.standard_normal((4, 5))])
    # batch axes: leading extra axes and size-1 axes are summed back
    _check(ops, lambda a, b: a @ b, [rng0.standard_normal((2, 3, 3, 4)), rng0.standard_normal((4, 5))])
    _check(ops, lambda a, b: a @ b, [rng0.standard_normal((1, 3, 4)), rng0.standard_normal((2, 4, 5))])
    # the free function propagates gradients too
    _check(ops, lambda a, b: _fn("matmul")(a, b),
           [rng0.standard_normal((3, 4)), rng0.standard_normal((4, 2))])


def test_topological_order_on_a_diamond_with_repeated_inputs(ops):
    import autodiff

    x = ops.Tensor(np.array([1.0, 2.0]))
    a = x * x                 # x used twice by one node
    b = x + 3.0
    c = a * b                 # diamond: a and b both depend on x
    d = c + a                 # a used by two users
    order = autodiff.find_topo_sort([d])
    pos = {id(n): i for i, n in enumerate(order)}
    assert len(order) == len(pos) == 5
    for n in order:
        for i in n.inputs:
            assert pos[id(i)] < pos[id(n)]
    assert order[-1] is d and order[0] is x
    d.backward()
    xv = np.array([1.0, 2.0])
    # d = x^2 (x + 3) + x^2  ->  dd/dx = 3x^2 + 6x + 2x
    np.testing.assert_allclose(x.grad.numpy(), 3 * xv ** 2 + 8 * xv)


def test_topo_sort_dfs_is_the_post_order_walk(ops):
    import autodiff

    def rec(node, visited, out):  # the definition: recursive post-order DFS
        if node in visited:
            return
        visited.add(node)
        for i in node.inputs:
            rec(i, visited, out)
        out.append(node)

    x = ops.Tensor(np.array([1.0, 2.0]))
    w = ops.Tensor(np.array([3.0, -1.0]))
    a = x * x
    b = x + w
    c = a * b
    d = c + a
    e = d * w
    for roots in ([e], [d, e], [b, e, a]):
        want, got = [], []
        vw, vg = set(), set()
        for r in roots:
            rec(r, vw, want)
            autodiff.topo_sort_dfs(r, vg, got)
        assert [id(n) for n in got] == [id(n) for n in want]
        assert vg == vw
    # a deep chain needs no recursion limit
    y = x
    for _ in range(5000):
        y = y + 1.0
    out = []
    autodiff.topo_sort_dfs(y, set(), out)
    assert len(out) == 5001 and out[0] is x and out[-1] is y


def test_topological_order_of_several_outputs(ops):
    import autodiff

    x = ops.Tensor(np.ones(2))
    y = x * 2.0
    z = y + x
    order = autodiff.find_topo_sort([z, y])
    assert [id(n) for n in order].index(id(y)) < [id(n) for n in order].index(id(z))
    assert len(order) == 3


def test_constant_subgraph_is_cut_and_still_correct(ops):
    c = ops.Tensor(np.array([2.0, 5.0]), requires_grad=False)
    k = c * 3.0 + 1.0                       # no input needs a gradient
    assert k.is_leaf() and not k.requires_grad and k.inputs == []
    x = ops.Tensor(np.array([1.0, -1.0]))
    (x * k).sum().backward()
    np.testing.assert_array_equal(x.grad.numpy(), np.array([7.0, 16.0]))


def test_deep_chain_needs_no_recursion_limit(ops):
    x = ops.Tensor(np.ones(3))
    y = x
    for _ in range(20000):
        y = y + 1.0
    y.sum().backward()
    np.testing.assert_array_equal(x.grad.numpy(), np.ones(3))


def test_second_backward_overwrites_grad(ops):
    x = ops.Tensor(np.array([3.0]))
    y = x * x
    y.backward()
    y.backward(ops.Tensor(np.array([2.0]), requires_grad=False))
    np.testing.assert_array_equal(x.grad.numpy(), [12.0])


def test_tensor_construction_and_data_semantics(ops):
    a = np.arange(6.0).reshape(2, 3)
    t = ops.Tensor(a, dtype="float32")
    assert t.dtype == np.float32 and t.shape == (2, 3) and t.device == ops.cpu()
    a[0, 0] = 99.0
    assert t.numpy()[0, 0] == 0.0           # a Tensor owns a copy of numpy input
    u = ops.Tensor(t)
    assert u.numpy() is t.numpy()           # from a Tensor: shares the data
    t.data = ops.Tensor(np.ones((2, 3), np.float32))
    assert float(t.numpy().sum()) == 6.0
    with pytest.raises(TypeError):
        t.data = ops.Tensor(np.ones((2, 3), np.float64))
    d = t.detach()
    assert d.is_leaf() and not d.requires_grad
    with pytest.raises(ValueError):
        import device

        ops.Tensor(a, device=device.Device("gpu"))


def test_op_arity_and_scalar_are_checked(ops):
    x = ops.Tensor(np.ones(2))
    with pytest.raises(TypeError):
        ops.EWiseAdd()(x)
    with pytest.raises(TypeError):
        ops.MulScalar()
    assert isinstance(x + x, ops.Tensor) and isinstance((x + x).op, ops.EWiseAdd)
    assert isinstance((x * 2.0).op, ops.MulScalar) and (x * 2.0).op.scalar == 2.0


def test_device_handle(ops):
    import device

    assert device.cpu() == device.cpu() and hash(device.cpu()) == hash(device.Device("cpu"))
    assert repr(device.cpu()) == "cpu()" and device.cpu().enabled()
    assert device.Device("gpu") != device.cpu()
    # the rest of the reference's device module (device.py:9-59)
    assert isinstance(device.cpu(), device.CPUDevice) and isinstance(device.cpu(), device.Device)
    assert device.CPUDevice() == device.cpu() and {device.cpu(): 1}[device.CPUDevice()] == 1
    assert device.default_device() == device.cpu() and device.all_devices() == [device.cpu()]


def test_cpu_device_factories(ops):
    import device

    c = device.cpu()
    z = c.zeros(2, 3)
    assert z.shape == (2, 3) and z.dtype == np.float32 and not z.any()
    o = c.ones(4, dtype="float64")
    assert o.dtype == np.float64 and (o == 1).all()
    np.random.seed(5)
    r = c.randn(3, 2)
    np.random.seed(5)
    assert r.shape == (3, 2) and np.array_equal(r, np.random.standard_normal((3, 2)))
    np.random.seed(6)
    u = c.rand(5)
    np.random.seed(6)
    assert np.array_equal(u, np.random.random_sample(5)) and ((u >= 0) & (u < 1)).all()
    h = c.one_hot(4, np.array([2, 0]))
    np.testing.assert_array_equal(h, [[0, 0, 1, 0], [1, 0, 0, 0]])
    assert h.dtype == np.float32
    assert c.empty((2, 2)).shape == (2, 2) and c.empty((1,), dtype="int32").dtype == np.int32
    f = c.full((2, 1), 7.5)
    assert f.dtype == np.float32 and (f == 7.5).all()


def test_make_const_unwraps_a_tensor_and_takes_requires_grad_positionally(ops):
    a = ops.Tensor(np.arange(3.0))
    c = ops.Tensor.make_const(a)
    assert isinstance(c.cached_data, np.ndarray) and c.numpy() is a.numpy()
    assert c.is_leaf() and not c.requires_grad
    g = ops.Tensor.make_const(np.ones(2), True)
    assert g.requires_grad and isinstance(g, ops.Tensor)
    y = ops.summation(g * 3.0)
    y.backward()
    np.testing.assert_array_equal(g.grad.numpy(), [3.0, 3.0])


def test_tensor_counter_counts_live_nodes(ops):
    import gc

    import basic_operator as bo

    gc.collect()
    base = bo.TENSOR_COUNTER
    a = ops.Tensor(np.ones(3))
    b = ops.Tensor.make_const(np.zeros(3))
    c = a + b  # one op node
    assert bo.TENSOR_COUNTER == base + 3
    del a, b, c
    gc.collect()
    assert bo.TENSOR_COUNTER == base


def test_causal_mask_closed_form(ops):
    m = ops.causal_mask(3, 5)
    assert m.dtype == np.float32
    expect = np.array([[0, -np.inf, -np.inf, -np.inf, -np.inf],
                       [0, 0, -np.inf, -np.inf, -np.inf],
                       [0, 0, 0, -np.inf, -np.inf]], np.float32)
    np.testing.assert_array_equal(m, expect)
