"""``Tensor`` and the operators of the TinyTensor Python layer, with the fused
MI355X attention operator.

Drop-in for Task3/Tinytensor/optimizer/operators.py on the attention path:
callers keep ``from operators import *``, build ``Tensor`` from numpy arrays,
other ``Tensor`` objects or ``myTensor`` tensors, compose with ``@ + - * / **``
and the op functions, call ``.backward(out_grad)`` and read ``.grad``
(reference :14-187 for ``Tensor``, :194-475 for the numpy ops, :478-491 for
``ReLU``).

Design:

* the elementwise operators are rows of one rule table (``_RULES``): a
  forward on arrays and a vector-Jacobian product written with graph ops, so
  gradients of gradients stay expressible; ``EWiseAdd``, ``MulScalar``, ... are
  classes generated from it, so ``isinstance`` checks and constructor
  arguments (the scalar of the ``*Scalar`` ops) work as before;
* shape operators (``Transpose``, ``Reshape``, ``BroadcastTo``, ``Summation``)
  and ``MatMul`` reduce a broadcast gradient back to the input's shape by one
  helper, ``_unbroadcast``;
* the GPU operators run through ``myTensor`` / ``myLayer`` (the pybind11 drop-in
  over the HIP C-ABI).  ``Attention`` keeps the device tensors of its forward
  on the output node (``node.saved``), releases them after its gradient, and
  recomputes them from the node's inputs when a second backward needs them.

Deliberate departures from the reference: ``matmul(a, b)`` propagates
gradients (the reference's wraps its arguments in new leaves, :432-433), and
``c - t`` computes c - t (the reference aliases ``__rsub__`` to ``__sub__``,
:187).  Of the reference's MNIST layers, ``FC`` (:498-533) runs on the library
GEMM through ``myLayer.FcForward`` / ``FcBackward`` and ``Conv`` (:535-569)
through ``myLayer.ConvForward`` / ``ConvBackward`` (im2col + the GEMM), and the
softmax losses (:604-665) through ``myLayer.SoftmaxForward`` and the
cross-entropy kernels, and ``MaxPool`` (:570-602) through
``myLayer.MaxPoolingForward`` / ``MaxPoolingBackward``.
"""
from __future__ import annotations

import math
from typing import Callable, Optional, Sequence

import numpy as np

from autodiff import compute_gradient_of_variables
from basic_operator import Op, Value
from device import Device, cpu
import myLayer as ml  # compiled extension: the import fails loudly when it is not built
from myTensor import Tensor_bf16, Tensor_float, Tensor_int

_DEVICE_TENSORS = (Tensor_float, Tensor_int, Tensor_bf16)


def _host_array(obj, dtype=None) -> np.ndarray:
    """A fresh host array for a Tensor's data from numpy-like input, another
    Tensor or a myTensor tensor (downloaded once)."""
    if isinstance(obj, Tensor):
        obj = obj.realize_cached_data()
    elif isinstance(obj, _DEVICE_TENSORS):
        obj = obj.numpy()
    return np.array(obj, dtype=dtype)


class Tensor(Value):
    """A graph node whose data is a host numpy array."""

    grad: "Tensor"

    def __init__(self, array, *, device: Optional[Device] = None, dtype=None, requires_grad=True, **kwargs):
        if device is not None and device != cpu():
            raise ValueError(f"Tensor data lives on the host; device {device!r} is not available")
        if isinstance(array, Tensor) and dtype is None:
            data = array.realize_cached_data()  # shares the array, as the reference does
        else:
            data = _host_array(array, dtype)
        self._setup(None, (), data, requires_grad)

    # ---------------------------------------------------------------- data
    @property
    def data(self) -> "Tensor":
        return self.detach()

    @data.setter
    def data(self, value: "Tensor") -> None:
        if not isinstance(value, Tensor):
            raise TypeError("Tensor.data takes a Tensor")
        if value.dtype != self.dtype:
            raise TypeError(f"Tensor.data: dtype {value.dtype} does not match {self.dtype}")
        self.cached_data = value.realize_cached_data()

    @classmethod
    def make_const(cls, data, requires_grad: bool = False) -> "Tensor":
        """A leaf holding `data` (a Tensor argument gives its realised data,
        not the Tensor itself), as the reference's Tensor.make_const
        (operators.py:70-79)."""
        if isinstance(data, Tensor):
            data = data.realize_cached_data()
        return super().make_const(data, requires_grad=requires_grad)

    def detach(self) -> "Tensor":
        return Tensor.make_const(self.realize_cached_data())

    @property
    def shape(self):
        return self.realize_cached_data().shape

    @property
    def dtype(self):
        return self.realize_cached_data().dtype

    @property
    def device(self) -> Device:
        return cpu()

    def numpy(self) -> np.ndarray:
        return self.realize_cached_data()

    def backward(self, out_grad=None) -> None:
        """Gradients of sum(self * out_grad) into .grad of every node this
        one depends on; out_grad defaults to ones."""
        if out_grad is None:
            out_grad = Tensor(np.ones(self.shape, dtype=self.dtype), requires_grad=False)
        elif not isinstance(out_grad, Tensor):
            out_grad = Tensor(out_grad, requires_grad=False)
        compute_gradient_of_variables(self, out_grad)

    def __repr__(self) -> str:
        return f"Tensor({self.realize_cached_data()})"

    def __str__(self) -> str:
        return str(self.realize_cached_data())

    # ------------------------------------------------------------ operators
    def __add__(self, other):
        return EWiseAdd()(self, other) if isinstance(other, Tensor) else AddScalar(other)(self)

    def __sub__(self, other):
        return EWiseAdd()(self, Negate()(other)) if isinstance(other, Tensor) else AddScalar(-other)(self)

    def __rsub__(self, other):
        return AddScalar(other)(Negate()(self))

    def __mul__(self, other):
        return EWiseMul()(self, other) if isinstance(other, Tensor) else MulScalar(other)(self)

    def __truediv__(self, other):
        return EWiseDiv()(self, other) if isinstance(other, Tensor) else DivScalar(other)(self)

    def __rtruediv__(self, other):
        return MulScalar(other)(PowerScalar(-1)(self))

    def __pow__(self, other):
        return EWisePow()(self, other) if isinstance(other, Tensor) else PowerScalar(other)(self)

    def __neg__(self):
        return Negate()(self)

    def __matmul__(self, other):
        return MatMul()(self, other)

    def __rmatmul__(self, other):
        return MatMul()(other, self)

    __radd__ = __add__
    __rmul__ = __mul__

    def matmul(self, other):
        return MatMul()(self, other)

    def sum(self, axes=None):
        return Summation(axes)(self)

    def broadcast_to(self, shape):
        return BroadcastTo(shape)(self)

    def reshape(self, shape):
        return Reshape(shape)(self)

    def transpose(self, axes=None):
        return Transpose(axes)(self)


class TensorOp(Op):
    """An operator whose nodes are Tensors."""

    def __call__(self, *args):
        return Tensor.make_from_op(self, args)


def _const(array) -> Tensor:
    return Tensor.make_const(array)


# ------------------------------------------------------------------ elementwise rule table
# name -> (number of tensor inputs, takes a scalar, forward(arrays, c), vjp(g, node, c))
# The vjp returns one gradient per tensor input, built from graph ops.
def _inputs(node):
    return node.inputs


_RULES = {
    "EWiseAdd": (2, False, lambda x, c: x[0] + x[1], lambda g, n, c: (g, g)),
    "AddScalar": (1, True, lambda x, c: x[0] + c, lambda g, n, c: (g,)),
    "EWiseMul": (2, False, lambda x, c: x[0] * x[1],
                 lambda g, n, c: (g * _inputs(n)[1], g * _inputs(n)[0])),
    "MulScalar": (1, True, lambda x, c: x[0] * c, lambda g, n, c: (g * c,)),
    "PowerScalar": (1, True, lambda x, c: np.power(x[0], c),
                    lambda g, n, c: (g * (_inputs(n)[0] ** (c - 1)) * c,)),
    "EWisePow": (2, False, lambda x, c: np.power(x[0], x[1]),
                 lambda g, n, c: (g * _inputs(n)[1] * _inputs(n)[0] ** (_inputs(n)[1] - 1),
                                  g * n.detach() * Log()(_inputs(n)[0]))),
    "EWiseDiv": (2, False, lambda x, c: x[0] / x[1],
                 lambda g, n, c: (g / _inputs(n)[1], -(g * _inputs(n)[0]) / (_inputs(n)[1] ** 2))),
    "DivScalar": (1, True, lambda x, c: x[0] / c, lambda g, n, c: (g / c,)),
    "Negate": (1, False, lambda x, c: -x[0], lambda g, n, c: (-g,)),
    "Log": (1, False, lambda x, c: np.log(x[0]), lambda g, n, c: (g / _inputs(n)[0],)),
    # d exp(a) = exp(a) da, with exp(a) the node's own (constant) output
    "Exp": (1, False, lambda x, c: np.exp(x[0]), lambda g, n, c: (g * n.detach(),)),
}


class _Elementwise(TensorOp):
    """Operator defined by a row of the rule table."""

    _arity = 1
    _forward: Callable = None
    _vjp: Callable = None
    _scalar_op = False

    def __init__(self, scalar=None):
        if self._scalar_op and scalar is None:
            raise TypeError(f"{type(self).__name__} needs a scalar")
        self.scalar = scalar

    def __call__(self, *args):
        if len(args) != self._arity:
            raise TypeError(f"{type(self).__name__} takes {self._arity} tensor input(s), got {len(args)}")
        return Tensor.make_from_op(self, args)

    def compute(self, *arrays):
        return type(self)._forward(arrays, self.scalar)

    def gradient(self, out_grad, node):
        return type(self)._vjp(out_grad, node, self.scalar)


def _make_elementwise(name, rule):
    arity, scalar, fwd, vjp = rule
    return type(name, (_Elementwise,), {
        "_arity": arity, "_scalar_op": scalar, "_forward": staticmethod(fwd), "_vjp": staticmethod(vjp),
        "__doc__": f"Elementwise operator {name} (rule table row).", "__module__": __name__,
    })


EWiseAdd = _make_elementwise("EWiseAdd", _RULES["EWiseAdd"])
AddScalar = _make_elementwise("AddScalar", _RULES["AddScalar"])
EWiseMul = _make_elementwise("EWiseMul", _RULES["EWiseMul"])
MulScalar = _make_elementwise("MulScalar", _RULES["MulScalar"])
PowerScalar = _make_elementwise("PowerScalar", _RULES["PowerScalar"])
EWisePow = _make_elementwise("EWisePow", _RULES["EWisePow"])
EWiseDiv = _make_elementwise("EWiseDiv", _RULES["EWiseDiv"])
DivScalar = _make_elementwise("DivScalar", _RULES["DivScalar"])
Negate = _make_elementwise("Negate", _RULES["Negate"])
Log = _make_elementwise("Log", _RULES["Log"])
Exp = _make_elementwise("Exp", _RULES["Exp"])


def add(a, b):
    return EWiseAdd()(a, b)


def add_scalar(a, scalar):
    return AddScalar(scalar)(a)


def multiply(a, b):
    return EWiseMul()(a, b)


def mul_scalar(a, scalar):
    return MulScalar(scalar)(a)


def power_scalar(a, scalar):
    return PowerScalar(scalar)(a)


def power(a, b):
    return EWisePow()(a, b)


def divide(a, b):
    return EWiseDiv()(a, b)


def divide_scalar(a, scalar):
    return DivScalar(scalar)(a)


def negate(a):
    return Negate()(a)


def log(a):
    return Log()(a)


def exp(a):
    return Exp()(a)


# ------------------------------------------------------------------ shapes and products

def _unbroadcast(grad: Tensor, shape: Sequence[int]) -> Tensor:
    """Sum `grad` down to `shape`: over the leading axes it has beyond
    len(shape), and over the axes where `shape` has size 1 and grad does not
    (numpy broadcasting in reverse)."""
    shape = tuple(shape)
    gshape = tuple(grad.shape)
    lead = len(gshape) - len(shape)
    axes = tuple(range(lead)) + tuple(lead + i for i, s in enumerate(shape) if s == 1 and gshape[lead + i] != 1)
    if axes:
        grad = Summation(axes)(grad)
    if tuple(grad.shape) != shape:
        grad = Reshape(shape)(grad)
    return grad


class Transpose(TensorOp):
    """Swap two axes: the given pair, or the last two (reference :323-340)."""

    def __init__(self, axes: Optional[tuple] = None):
        self.axes = axes

    def compute(self, a):
        i, j = self.axes if self.axes is not None else (-2, -1)
        return np.swapaxes(a, i, j)

    def gradient(self, out_grad, node):
        return Transpose(self.axes)(out_grad)


class Reshape(TensorOp):
    def __init__(self, shape):
        self.shape = tuple(shape)

    def compute(self, a):
        return np.reshape(a, self.shape)

    def gradient(self, out_grad, node):
        return Reshape(node.inputs[0].shape)(out_grad)


class BroadcastTo(TensorOp):
    def __init__(self, shape):
        self.shape = tuple(shape)

    def compute(self, a):
        return np.broadcast_to(a, self.shape)

    def gradient(self, out_grad, node):
        return _unbroadcast(out_grad, node.inputs[0].shape)


class Summation(TensorOp):
    """Sum over `axes` (an int, a tuple, or None for all), dropping them."""

    def __init__(self, axes=None):
        self.axes = axes

    def _axes(self, ndim):
        if self.axes is None:
            return tuple(range(ndim))
        ax = self.axes if isinstance(self.axes, (tuple, list)) else (self.axes,)
        return tuple(a % ndim for a in ax)

    def compute(self, a):
        return np.sum(a, axis=self._axes(a.ndim))

    def gradient(self, out_grad, node):
        in_shape = tuple(node.inputs[0].shape)
        axes = self._axes(len(in_shape))
        kept = tuple(1 if i in axes else s for i, s in enumerate(in_shape))
        return BroadcastTo(in_shape)(Reshape(kept)(out_grad))


class MatMul(TensorOp):
    """np.matmul with broadcast batch axes; each gradient is summed back to
    its input's shape (reference :416-429)."""

    def compute(self, a, b):
        return np.matmul(a, b)

    def gradient(self, out_grad, node):
        a, b = node.inputs
        ga = MatMul()(out_grad, Transpose()(b)) if len(b.shape) > 1 else None
        gb = MatMul()(Transpose()(a), out_grad) if len(a.shape) > 1 else None
        if ga is None or gb is None:
            raise NotImplementedError("MatMul gradient needs operands of rank >= 2")
        return _unbroadcast(ga, a.shape), _unbroadcast(gb, b.shape)


def transpose(a, axes=None):
    return Transpose(axes)(a)


def reshape(a, shape):
    return Reshape(shape)(a)


def broadcast_to(a, shape):
    return BroadcastTo(shape)(a)


def summation(a, axes=None):
    return Summation(axes)(a)


def matmul(a, b):
    return MatMul()(a, b)


# ------------------------------------------------------------------ GPU operators

class ReLU(TensorOp):
    """max(x, 0) on the GPU through myTensor (reference :478-491)."""

    def compute(self, a):
        return Tensor_float(np.asarray(a, np.float32), "gpu").ReluForward().numpy()

    def gradient(self, out_grad, node):
        x = Tensor_float(np.asarray(node.inputs[0].realize_cached_data(), np.float32), "gpu")
        g = Tensor_float(np.asarray(out_grad.realize_cached_data(), np.float32), "gpu")
        return Tensor(x.ReluBackward(g))


def relu(a):
    return ReLU()(a)


class FC(TensorOp):
    """Fully connected layer, input @ weight + bias, on the GPU through
    ``myLayer.FcForward`` / ``FcBackward`` (reference :498-529): weight
    [fin, fout], bias [fout] or [1]; ``use_bias=False`` zeroes the bias and
    its gradient as the reference does (:506-507, :527-528).  Every leading
    axis of the input is a batch axis (the layer's reading, Layers.cu:16-20)."""

    def __init__(self, use_bias: bool = True):
        self.use_bias = use_bias

    @staticmethod
    def _dev(a):
        return Tensor_float(np.asarray(a, np.float32), "gpu")

    def compute(self, input, weight, bias):
        x, w, b = self._dev(input), self._dev(weight), self._dev(bias)
        if not self.use_bias:
            b.zeros()
        out = Tensor_float([1], "gpu")
        ml.FcForward(x, out, w, b)
        return out.numpy()

    def gradient(self, out_grad, node):
        x, w, b = (self._dev(t.realize_cached_data()) for t in node.inputs)
        go = self._dev(out_grad.realize_cached_data())
        gx, gw, gb = Tensor_float([1], "gpu"), Tensor_float([1], "gpu"), Tensor_float([1], "gpu")
        ml.FcBackward(x, Tensor_float([1], "gpu"), w, b, gx, go, gw, gb)
        if not self.use_bias:
            gb.zeros()
        return Tensor(gx, requires_grad=False), Tensor(gw, requires_grad=False), Tensor(gb, requires_grad=False)


def fc(input, weight, bias, use_bias=True):
    return FC(use_bias)(input, weight, bias)


class Conv(TensorOp):
    """2-D convolution, no bias, on the GPU through ``myLayer.ConvForward`` /
    ``ConvBackward`` (reference :535-566): input [N, Cin, H, W], weight
    [Cout, Cin, kh, kw] -> [N, Cout, OH, OW], OH = (H + 2 pad_h - kh) //
    stride_h + 1; ``gradient`` returns (grad_input, grad_weight)."""

    def __init__(self, pad_h, pad_w, stride_h, stride_w):
        self.pad_h, self.pad_w, self.stride_h, self.stride_w = pad_h, pad_w, stride_h, stride_w

    def _args(self):
        return self.pad_h, self.pad_w, self.stride_h, self.stride_w

    def compute(self, input, weight):
        x, w = FC._dev(input), FC._dev(weight)
        out = Tensor_float([1], "gpu")
        ml.ConvForward(x, out, w, *self._args())
        return out.numpy()

    def gradient(self, out_grad, node):
        x, w = (FC._dev(t.realize_cached_data()) for t in node.inputs)
        go = FC._dev(out_grad.realize_cached_data())
        gx, gw = Tensor_float([1], "gpu"), Tensor_float([1], "gpu")
        ml.ConvBackward(x, Tensor_float([1], "gpu"), w, gx, go, gw, *self._args())
        return Tensor(gx, requires_grad=False), Tensor(gw, requires_grad=False)


def conv(input, weight, pad_h=0, pad_w=0, stride_h=1, stride_w=1):
    return Conv(pad_h, pad_w, stride_h, stride_w)(input, weight)


class MaxPool(TensorOp):
    """Max pooling over the last two axes on the GPU (reference :570-602):
    the window's first largest element passes; its gradient goes back to that
    element (summed where windows overlap).  Each output node keeps its own
    device mask until its gradient is taken."""

    def __init__(self, kernel_shape=(2, 2), pad_h=0, pad_w=0, stride_h=2, stride_w=2):
        self.kernel_shape = [int(k) for k in kernel_shape]
        self.pad_h, self.pad_w, self.stride_h, self.stride_w = pad_h, pad_w, stride_h, stride_w

    def _args(self):
        return self.kernel_shape, self.pad_h, self.pad_w, self.stride_h, self.stride_w

    def _run(self, x):
        xd = FC._dev(x)
        out, mask = Tensor_float([1], "gpu"), Tensor_float([1], "gpu")
        ml.MaxPoolingForward(xd, out, mask, *self._args())
        return out, mask, list(np.shape(x))

    def compute(self, input):
        return self._run(input)[0].numpy()

    def forward(self, node, input):
        out, mask, shape = self._run(input)
        node.saved = (mask, shape)
        return out.numpy()

    def gradient(self, out_grad, node):
        saved = getattr(node, "saved", None)
        if saved is None:
            _, mask, shape = self._run(node.inputs[0].realize_cached_data())
        else:
            mask, shape = saved
        node.saved = None
        gx = Tensor_float([1], "gpu")
        ml.MaxPoolingBackward(FC._dev(out_grad.realize_cached_data()), mask, gx, shape, *self._args())
        return Tensor(gx, requires_grad=False)


def maxpool(input, kernel_shape=(2, 2), pad_h=0, pad_w=0, stride_h=2, stride_w=2):
    return MaxPool(kernel_shape, pad_h, pad_w, stride_h, stride_w)(input)


def _labels_array(labels) -> np.ndarray:
    data = labels.realize_cached_data() if isinstance(labels, Value) else labels
    return np.asarray(data).astype(np.int32).ravel()


class _SoftmaxLossBase(TensorOp):
    """Softmax over the classes of logits [batch, classes], then (loss, error)
    as the reference reports them (operators.py:604-665): the summed cross
    entropy and the misclassified rows, both divided by 10 * batch (the
    reference's reporting scale), returned as a 2-element float64 array so
    that ``loss, error = node.realize_cached_data()`` unpacks as before and
    ``node.backward()`` works.  The gradient with respect to the logits is
    (softmax - onehot(labels)) / batch, whatever out_grad holds (as in the
    reference)."""

    def __init__(self, labels):
        self.labels = _labels_array(labels)
        self.batchsize = self.labels.shape[0]
        self.softmax = None

    def _report(self, loss_sum):
        wrong = np.count_nonzero(self.softmax.argmax(axis=1) != self.labels)
        scale = 10.0 * self.batchsize
        return np.array([loss_sum / scale, wrong / scale])


class Softmaxloss(_SoftmaxLossBase):
    """The reference's CPU softmax loss (operators.py:604-629), in numpy."""

    def compute(self, z):
        z = np.asarray(z, np.float64)
        shifted = z - z.max(axis=1, keepdims=True)
        e = np.exp(shifted)
        self.softmax = e / e.sum(axis=1, keepdims=True)
        rows = np.arange(self.batchsize)
        # -log softmax[label] = log sum_j exp(z_j - z_label)
        loss_sum = np.log(np.exp(shifted - shifted[rows, self.labels][:, None]).sum(axis=1)).sum()
        return self._report(loss_sum)

    def gradient(self, out_grad, node):
        g = self.softmax.copy()
        g[np.arange(self.batchsize), self.labels] -= 1.0
        return Tensor(g / self.batchsize, requires_grad=False)


class Softmaxcrossentropyloss(_SoftmaxLossBase):
    """The reference's GPU softmax cross entropy (operators.py:636-661):
    ``myLayer.SoftmaxForward``, ``CrossEntropyLoss`` and, for the gradient,
    ``CrossEntropyLossBackward`` scaled by 1 / batch."""

    def _labels_dev(self):
        return Tensor_int(self.labels.reshape(1, -1), "gpu")

    def compute(self, input):
        x = Tensor_float(np.asarray(input, np.float32), "gpu")
        p = Tensor_float([1], "gpu")
        ml.SoftmaxForward(x, p)
        self.softmax = np.asarray(p.numpy()).reshape(x.get_shape())
        loss = Tensor_float([1], "gpu")
        ml.CrossEntropyLoss(p, self._labels_dev(), loss)
        return self._report(float(loss.get_data()[0]))

    def gradient(self, out_grad, node):
        p = Tensor_float(self.softmax.astype(np.float32), "gpu")
        g = Tensor_float([1], "gpu")
        ml.CrossEntropyLossBackward(p, self._labels_dev(), g)
        g.mults(1.0 / self.batchsize)
        return Tensor(g, requires_grad=False)


def softmaxloss(X, y):
    return Softmaxloss(y)(X)


def softmaxcrossentropyloss(X, y):
    return Softmaxcrossentropyloss(y)(X)


_ATTN_DTYPES = {"float32": Tensor_float, "bf16": Tensor_bf16}


def _default_scale(d: int) -> float:
    return float(np.float32(1.0 / math.sqrt(d)))


class Attention(TensorOp):
    """Fused scaled dot-product attention on the MI355X.

    ``softmax(q @ k^T * scale + mask) @ v`` for q [B, H, Lq, d] and k, v
    [B, H, Lk, d], d in {32, 64, 128}; the mask is -inf where key > query when
    ``causal``.  ``scale`` defaults to 1/sqrt(d) rounded to float32.  dtype
    "float32" runs the fp32 kernels; "bf16" rounds the inputs to bfloat16 on
    upload and accumulates in fp32.  The result equals the reference's
    composition ``(q @ k.transpose()) * scale`` -> ``+ mask`` -> exp / sum /
    divide -> ``@ v`` (operators.py:163-164, 234-239, 194-196, 611-612,
    416-419) without forming the L x L scores, and ``gradient`` returns
    (dQ, dK, dV) like that composition's backward.  A ``myLayer`` call runs
    each direction (bind_Layer.cpp:12-23 style, shaped like FC at
    operators.py:498-532).
    """

    def __init__(self, causal: bool = False, scale: Optional[float] = None, dtype: str = "float32"):
        if dtype not in _ATTN_DTYPES:
            raise ValueError(f"Attention dtype must be one of {sorted(_ATTN_DTYPES)}, got {dtype!r}")
        self.causal = bool(causal)
        self.scale = scale
        self.dtype = dtype

    def _run_forward(self, q, k, v):
        """Upload, run the forward kernel; returns the device tensors
        (q, k, v, out, lse) and the scale used."""
        T = _ATTN_DTYPES[self.dtype]
        qd, kd, vd = (T(np.asarray(x, np.float32), "gpu") for x in (q, k, v))
        out, lse = T([1], "gpu"), Tensor_float([1], "gpu")
        scale = _default_scale(qd.get_shape()[-1]) if self.scale is None else float(self.scale)
        ml.AttentionForward(qd, kd, vd, out, lse, scale, self.causal)
        return (qd, kd, vd, out, lse), scale

    def compute(self, q, k, v):
        (_, _, _, out, _), _ = self._run_forward(q, k, v)
        return out.numpy()

    def forward(self, node, q, k, v):
        dev, scale = self._run_forward(q, k, v)
        node.saved = (dev, scale)
        return dev[3].numpy()

    def gradient(self, out_grad, node):
        saved = node.saved
        if saved is None:  # a second backward through this node: recompute the forward
            saved = self._run_forward(*[x.realize_cached_data() for x in node.inputs])
        (qd, kd, vd, out, lse), scale = saved
        node.saved = None  # release the device tensors
        T = _ATTN_DTYPES[self.dtype]
        go = T(np.asarray(out_grad.realize_cached_data(), np.float32), "gpu")
        gq, gk, gv = T([1], "gpu"), T([1], "gpu"), T([1], "gpu")
        ml.AttentionBackward(qd, kd, vd, out, lse, go, gq, gk, gv, scale, self.causal)
        return Tensor(gq, requires_grad=False), Tensor(gk, requires_grad=False), Tensor(gv, requires_grad=False)


def attention(q, k, v, causal: bool = False, scale: Optional[float] = None, dtype: str = "float32"):
    return Attention(causal, scale, dtype)(q, k, v)


class AttentionDecode(TensorOp):
    """Single-query decode (forward only): q [B, H, 1, d] against a K/V cache
    [B, H, Lkv, d], no mask; the memory-bound split-KV kernel."""

    def __init__(self, scale: Optional[float] = None, dtype: str = "bf16"):
        if dtype not in _ATTN_DTYPES:
            raise ValueError(f"AttentionDecode dtype must be one of {sorted(_ATTN_DTYPES)}, got {dtype!r}")
        self.scale = scale
        self.dtype = dtype

    def compute(self, q, k, v):
        T = _ATTN_DTYPES[self.dtype]
        qd, kd, vd = (T(np.asarray(x, np.float32), "gpu") for x in (q, k, v))
        out = T([1], "gpu")
        scale = _default_scale(qd.get_shape()[-1]) if self.scale is None else float(self.scale)
        ml.AttentionDecode(qd, kd, vd, out, scale)
        return out.numpy()

    def gradient(self, out_grad, node):
        raise NotImplementedError("decode attention is forward-only")


def attention_decode(q, k, v, scale: Optional[float] = None, dtype: str = "bf16"):
    return AttentionDecode(scale, dtype)(q, k, v)


# ------------------------------------------------------------------ the composition the fused op replaces

def causal_mask(Lq: int, Lk: int, dtype=np.float32) -> np.ndarray:
    """The constant additive mask: -inf where key > query, 0 elsewhere."""
    return np.where(np.arange(Lk)[None, :] > np.arange(Lq)[:, None], -np.inf, 0.0).astype(dtype)


def attention_composed(q: Tensor, k: Tensor, v: Tensor, causal: bool = False, scale: Optional[float] = None):
    """Attention built from this module's numpy operators in the reference's
    op order: MatMul(Q, Transpose(K)) -> MulScalar -> EWiseAdd(mask) -> shift
    by the (constant) row max -> Exp -> Summation -> Reshape -> BroadcastTo ->
    EWiseDiv -> MatMul(., V).  Runs on the host; used to check the fused
    operator against the composition it replaces."""
    s = _default_scale(q.shape[-1]) if scale is None else float(scale)
    scores = (q @ k.transpose()) * s
    if causal:
        scores = scores + Tensor(causal_mask(q.shape[-2], k.shape[-2], scores.dtype), requires_grad=False)
    shift = _const(np.max(scores.numpy(), axis=-1, keepdims=True))
    e = exp(scores - broadcast_to(shift, scores.shape))
    z = summation(e, axes=(len(e.shape) - 1,))
    zb = broadcast_to(reshape(z, tuple(z.shape) + (1,)), e.shape)
    return (e / zb) @ v
