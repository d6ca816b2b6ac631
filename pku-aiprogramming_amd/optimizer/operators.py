"""Tensor and operators of the TinyTensor Python layer, with the fused
MI355X attention op.

Drop-in for Task3/Tinytensor/optimizer/operators.py on the attention path:

* ``Tensor(Value)`` with the same constructors (numpy array, ``Tensor``, or a
  ``myTensor`` tensor; :17-58), ``backward(out_grad)`` (:115-119) and the
  operator sugar (:133-187);
* the numpy ops the reference composes attention from -- ``EWiseAdd``,
  ``AddScalar``, ``EWiseMul``, ``MulScalar``, ``PowerScalar``, ``EWisePow``,
  ``EWiseDiv``, ``DivScalar``, ``Transpose``, ``Reshape``, ``BroadcastTo``,
  ``Summation``, ``MatMul``, ``Negate``, ``Log``, ``Exp`` (:194-475) -- with
  the same forward semantics and gradient rules;
* ``ReLU`` over ``myTensor`` (:478-491);
* new: ``Attention(TensorOp)`` -- one fused GPU op for
  ``softmax(Q K^T * scale + mask) V`` in fp32 or bf16, shaped like ``FC``
  (:498-532): ``compute`` uploads with ``Tensor_*(..., "gpu")``, calls
  ``myLayer.AttentionForward`` and stashes the device tensors and the
  log-sum-exp; ``gradient`` calls ``myLayer.AttentionBackward``.

GPU ops return float32 numpy arrays through ``numpy()`` (one copy); the
reference returns float64 arrays built from a Python list.

The MNIST layers of the reference (FC, Conv, MaxPool and the softmax losses,
:494-665) are not part of this build.
"""
from __future__ import annotations

import math
from typing import List, Optional, Tuple

import numpy as np

from autodiff import compute_gradient_of_variables
from basic_operator import Op, Value
from device import Device, cpu
import myLayer as ml  # noqa: E402  (compiled extension; import fails loudly if unbuilt)
from myTensor import Tensor_bf16 as tb
from myTensor import Tensor_float as tf
from myTensor import Tensor_int as ti

_MYTENSOR_TYPES = (tf, ti, tb)


class Tensor(Value):
    grad: "Tensor"

    def __init__(self, array, *, device: Optional[Device] = None, dtype=None, requires_grad=True, **kwargs):
        if isinstance(array, Tensor):
            device = device or array.device
            dtype = dtype or array.dtype
            if device == array.device and dtype == array.dtype:
                data = array.realize_cached_data()
            else:
                data = Tensor._array_from_numpy(array.numpy(), device=device, dtype=dtype)
        elif isinstance(array, _MYTENSOR_TYPES):
            data = Tensor._array_from_mytensor(array, device=device or cpu(), dtype=dtype)
        else:
            data = Tensor._array_from_numpy(np.asarray(array), device=device or cpu(), dtype=dtype)
        self._init(None, [], cached_data=data, requires_grad=requires_grad)

    @staticmethod
    def _array_from_numpy(numpy_array, device, dtype):
        return np.array(numpy_array, dtype=dtype)

    @staticmethod
    def _array_from_mytensor(mytensor, device, dtype):
        return np.array(mytensor.numpy(), dtype=dtype)

    @staticmethod
    def make_from_op(op: Op, inputs: List["Value"]):
        t = Tensor.__new__(Tensor)
        t._init(op, inputs)
        if not t.requires_grad:
            return t.detach()
        t.realize_cached_data()
        return t

    @staticmethod
    def make_const(data, requires_grad=False):
        t = Tensor.__new__(Tensor)
        if isinstance(data, Tensor):
            data = data.realize_cached_data()
        t._init(None, [], cached_data=data, requires_grad=requires_grad)
        return t

    @property
    def data(self):
        return self.detach()

    @data.setter
    def data(self, value):
        assert isinstance(value, Tensor)
        assert value.dtype == self.dtype, f"{value.dtype} {self.dtype}"
        self.cached_data = value.realize_cached_data()

    def detach(self):
        return Tensor.make_const(self.realize_cached_data())

    @property
    def shape(self):
        if isinstance(self.cached_data, tuple):
            return [1]
        return self.realize_cached_data().shape

    @property
    def dtype(self):
        if isinstance(self.cached_data, tuple):
            return float
        return self.realize_cached_data().dtype

    @property
    def device(self):
        return cpu()

    def backward(self, out_grad=None):
        if out_grad is None:
            out_grad = Tensor(np.ones(self.shape, dtype=self.dtype), dtype=self.dtype, requires_grad=False)
        elif not isinstance(out_grad, Tensor):
            out_grad = Tensor(out_grad, requires_grad=False)
        compute_gradient_of_variables(self, out_grad)

    def __repr__(self):
        return "Tensor(" + str(self.realize_cached_data()) + ")"

    def __str__(self):
        return str(self.realize_cached_data())

    def numpy(self):
        return self.realize_cached_data()

    def __add__(self, other):
        return EWiseAdd()(self, other) if isinstance(other, Tensor) else AddScalar(other)(self)

    def __mul__(self, other):
        return EWiseMul()(self, other) if isinstance(other, Tensor) else MulScalar(other)(self)

    def __pow__(self, other):
        return EWisePow()(self, other) if isinstance(other, Tensor) else PowerScalar(other)(self)

    def __sub__(self, other):
        return EWiseAdd()(self, Negate()(other)) if isinstance(other, Tensor) else AddScalar(-other)(self)

    def __truediv__(self, other):
        return EWiseDiv()(self, other) if isinstance(other, Tensor) else DivScalar(other)(self)

    def __matmul__(self, other):
        return MatMul()(self, other)

    def matmul(self, other):
        return MatMul()(self, other)

    def sum(self, axes=None):
        return Summation(axes)(self)

    def broadcast_to(self, shape):
        return BroadcastTo(shape)(self)

    def reshape(self, shape):
        return Reshape(shape)(self)

    def __neg__(self):
        return Negate()(self)

    def transpose(self, axes=None):
        return Transpose(axes)(self)

    __radd__ = __add__
    __rmul__ = __mul__
    __rsub__ = __sub__
    __rmatmul__ = __matmul__


class TensorOp(Op):
    def __call__(self, *args):
        return Tensor.make_from_op(self, args)


# --------------------------------------------------------------- elementwise

class EWiseAdd(TensorOp):
    def compute(self, a, b):
        return a + b

    def gradient(self, out_grad, node):
        return out_grad, out_grad


def add(a, b):
    return EWiseAdd()(a, b)


class AddScalar(TensorOp):
    def __init__(self, scalar):
        self.scalar = scalar

    def compute(self, a):
        return a + self.scalar

    def gradient(self, out_grad, node):
        return out_grad


def add_scalar(a, scalar):
    return AddScalar(scalar)(a)


class EWiseMul(TensorOp):
    def compute(self, a, b):
        return a * b

    def gradient(self, out_grad, node):
        a, b = node.inputs
        return out_grad * b, out_grad * a


def multiply(a, b):
    return EWiseMul()(a, b)


class MulScalar(TensorOp):
    def __init__(self, scalar):
        self.scalar = scalar

    def compute(self, a):
        return a * self.scalar

    def gradient(self, out_grad, node):
        return out_grad * self.scalar


def mul_scalar(a, scalar):
    return MulScalar(scalar)(a)


class PowerScalar(TensorOp):
    """a ** scalar, elementwise."""

    def __init__(self, scalar):
        self.scalar = scalar

    def compute(self, a):
        return np.power(a, self.scalar)

    def gradient(self, out_grad, node):
        a = node.inputs[0]
        return out_grad * self.scalar * (a ** (self.scalar - 1))


def power_scalar(a, scalar):
    return PowerScalar(scalar)(a)


class EWisePow(TensorOp):
    """a ** b, elementwise."""

    def compute(self, a, b):
        return a ** b

    def gradient(self, out_grad, node):
        a, b = node.inputs
        if not isinstance(a, Tensor) or not isinstance(b, Tensor):
            raise ValueError("Both inputs must be tensors.")
        return out_grad * b * (a ** (b - 1)), out_grad * (a ** b) * log(a)


def power(a, b):
    return EWisePow()(a, b)


class EWiseDiv(TensorOp):
    """a / b; d/da = 1/b, d/db = -a/b^2 (quotient rule, as the reference)."""

    def compute(self, a, b):
        return a / b

    def gradient(self, out_grad, node):
        a, b = node.inputs
        return out_grad / b, -out_grad * a / (b ** 2)


def divide(a, b):
    return EWiseDiv()(a, b)


class DivScalar(TensorOp):
    def __init__(self, scalar):
        self.scalar = scalar

    def compute(self, a):
        return a / self.scalar

    def gradient(self, out_grad, node):
        return out_grad / self.scalar


def divide_scalar(a, scalar):
    return DivScalar(scalar)(a)


class Negate(TensorOp):
    def compute(self, a):
        return -a

    def gradient(self, out_grad, node):
        return -out_grad


def negate(a):
    return Negate()(a)


class Log(TensorOp):
    def compute(self, a):
        return np.log(a)

    def gradient(self, out_grad, node):
        return out_grad / node.inputs[0]


def log(a):
    return Log()(a)


class Exp(TensorOp):
    def compute(self, a):
        return np.exp(a)

    def gradient(self, out_grad, node):
        # the reference multiplies by a constant exp(input), not by a graph node
        return out_grad * np.exp(node.inputs[0].realize_cached_data())


def exp(a):
    return Exp()(a)


# --------------------------------------------------------------- shape ops

class Transpose(TensorOp):
    """Swap two axes; default: the last two (reference :323-336)."""

    def __init__(self, axes: Optional[tuple] = None):
        self.axes = axes

    def _perm(self, ndim):
        perm = list(range(ndim))
        if self.axes is None:
            perm[-2], perm[-1] = perm[-1], perm[-2]
        else:
            x, y = self.axes
            perm[x], perm[y] = perm[y], perm[x]
        return perm

    def compute(self, a):
        return np.transpose(a, self._perm(a.ndim))

    def gradient(self, out_grad, node):
        return transpose(out_grad, self.axes)


def transpose(a, axes=None):
    return Transpose(axes)(a)


class Reshape(TensorOp):
    def __init__(self, shape):
        self.shape = shape

    def compute(self, a):
        return np.reshape(a, self.shape)

    def gradient(self, out_grad, node):
        return reshape(out_grad, node.inputs[0].shape)


def reshape(a, shape):
    return Reshape(shape)(a)


class BroadcastTo(TensorOp):
    def __init__(self, shape):
        self.shape = shape

    def compute(self, a):
        return np.broadcast_to(a, self.shape)

    def gradient(self, out_grad, node):
        in_shape = tuple(node.inputs[0].shape)
        padded = (1,) * (len(self.shape) - len(in_shape)) + in_shape
        axes = tuple(i for i, (s, p) in enumerate(zip(self.shape, padded)) if s != p)
        return (reshape(summation(out_grad, axes=axes), in_shape),)


def broadcast_to(a, shape):
    return BroadcastTo(shape)(a)


class Summation(TensorOp):
    def __init__(self, axes: Optional[tuple] = None):
        self.axes = axes

    def compute(self, a):
        return np.sum(a) if self.axes is None else np.sum(a, axis=self.axes)

    def gradient(self, out_grad, node):
        in_shape = node.inputs[0].shape
        if self.axes is None:
            axes = tuple(range(len(in_shape)))
        elif isinstance(self.axes, (list, tuple)):
            axes = tuple(self.axes)
        else:
            axes = (self.axes,)
        kept = [1 if i in axes else s for i, s in enumerate(in_shape)]
        return broadcast_to(reshape(out_grad, kept), in_shape)


def summation(a, axes=None):
    return Summation(axes)(a)


class MatMul(TensorOp):
    """np.matmul with batch broadcasting; gradients sum over broadcast
    leading axes (reference :416-429)."""

    def compute(self, a, b):
        return np.matmul(a, b)

    def gradient(self, out_grad, node):
        a, b = node.inputs
        ga = out_grad @ transpose(b)
        gb = transpose(a) @ out_grad
        if len(ga.shape) > len(a.shape):
            ga = summation(ga, axes=tuple(range(len(ga.shape) - len(a.shape))))
        if len(gb.shape) > len(b.shape):
            gb = summation(gb, axes=tuple(range(len(gb.shape) - len(b.shape))))
        return ga, gb


def matmul(a, b):
    # As in the reference (:432-433) this wraps both arguments in new leaf
    # tensors, so it does not propagate gradients; use ``a @ b`` for that.
    return MatMul()(Tensor(a), Tensor(b))


# --------------------------------------------------------------- GPU ops

class ReLU(TensorOp):
    def compute(self, a):
        return tf(np.asarray(a, np.float32), "gpu").ReluForward().numpy()

    def gradient(self, out_grad, node):
        x = tf(np.asarray(node.inputs[0].realize_cached_data(), np.float32), "gpu")
        g = tf(np.asarray(out_grad.realize_cached_data(), np.float32), "gpu")
        return Tensor(x.ReluBackward(g))


def relu(a):
    return ReLU()(a)


class Attention(TensorOp):
    """Fused scaled dot-product attention on the MI355X.

    ``compute(q, k, v)`` -> ``softmax(q @ k^T * scale + mask) @ v`` with
    q [B, H, Lq, d], k/v [B, H, Lk, d], d in {32, 64, 128}; ``mask`` is -inf
    where key > query when ``causal``.  ``scale`` defaults to 1/sqrt(d)
    rounded to float32.  ``dtype`` "float32" runs the fp32 kernels, "bf16"
    rounds the inputs to bfloat16 on upload and accumulates in fp32.

    The same result as composing the reference's ops
    ``(q @ k.transpose()) * scale`` -> ``+ mask`` -> ``exp`` / ``sum`` /
    ``divide`` -> ``@ v`` (operators.py:163-164, 234-239, 194-196, 611-612,
    416-419), without materialising the L x L scores; ``gradient`` returns
    (dQ, dK, dV) for the upstream gradient like that composition's backward.
    """

    def __init__(self, causal: bool = False, scale: Optional[float] = None, dtype: str = "float32"):
        if dtype not in ("float32", "bf16"):
            raise ValueError("Attention dtype must be 'float32' or 'bf16'")
        self.causal = bool(causal)
        self.scale = scale
        self.dtype = dtype
        self._saved = None

    def _cls(self):
        return tb if self.dtype == "bf16" else tf

    def _scale_for(self, d):
        return float(np.float32(1.0 / math.sqrt(d))) if self.scale is None else float(self.scale)

    def compute(self, q, k, v):
        T = self._cls()
        qt = T(np.asarray(q, np.float32), "gpu")
        kt = T(np.asarray(k, np.float32), "gpu")
        vt = T(np.asarray(v, np.float32), "gpu")
        out = T([1], "gpu")
        lse = tf([1], "gpu")
        ml.AttentionForward(qt, kt, vt, out, lse, self._scale_for(qt.get_shape()[-1]), self.causal)
        self._saved = (qt, kt, vt, out, lse)
        return out.numpy()

    def gradient(self, out_grad, node):
        T = self._cls()
        if self._saved is None:
            self.compute(*[x.realize_cached_data() for x in node.inputs])
        qt, kt, vt, out, lse = self._saved
        go = T(np.asarray(out_grad.realize_cached_data(), np.float32), "gpu")
        gq, gk, gv = T([1], "gpu"), T([1], "gpu"), T([1], "gpu")
        ml.AttentionBackward(qt, kt, vt, out, lse, go, gq, gk, gv, self._scale_for(qt.get_shape()[-1]),
                             self.causal)
        return Tensor(gq), Tensor(gk), Tensor(gv)


def attention(q, k, v, causal: bool = False, scale: Optional[float] = None, dtype: str = "float32"):
    return Attention(causal, scale, dtype)(q, k, v)


class AttentionDecode(TensorOp):
    """Single-query decode (forward only): q [B, H, 1, d] against a K/V cache
    [B, H, Lkv, d]; memory-bound split-KV kernel."""

    def __init__(self, scale: Optional[float] = None, dtype: str = "bf16"):
        if dtype not in ("float32", "bf16"):
            raise ValueError("AttentionDecode dtype must be 'float32' or 'bf16'")
        self.scale = scale
        self.dtype = dtype

    def compute(self, q, k, v):
        T = tb if self.dtype == "bf16" else tf
        qt = T(np.asarray(q, np.float32), "gpu")
        kt = T(np.asarray(k, np.float32), "gpu")
        vt = T(np.asarray(v, np.float32), "gpu")
        out = T([1], "gpu")
        d = qt.get_shape()[-1]
        scale = float(np.float32(1.0 / math.sqrt(d))) if self.scale is None else float(self.scale)
        ml.AttentionDecode(qt, kt, vt, out, scale)
        return out.numpy()

    def gradient(self, out_grad, node):
        raise NotImplementedError("decode attention is forward-only")


def attention_decode(q, k, v, scale: Optional[float] = None, dtype: str = "bf16"):
    return AttentionDecode(scale, dtype)(q, k, v)


# --------------------------------------------------------------- reference composition

def causal_mask(Lq: int, Lk: int, dtype=np.float32) -> np.ndarray:
    """The constant additive mask: -inf strictly above the diagonal."""
    m = np.zeros((Lq, Lk), dtype=dtype)
    m[np.triu_indices(Lq, 1, Lk)] = -np.inf
    return m


def attention_composed(q: Tensor, k: Tensor, v: Tensor, causal: bool = False, scale: Optional[float] = None):
    """Attention written with the reference's own autodiff ops, in its op
    order: MatMul(Q, Transpose(K)) -> MulScalar -> EWiseAdd(mask) -> shift by
    the (constant) row max -> Exp -> Summation -> Reshape -> BroadcastTo ->
    EWiseDiv -> MatMul(., V).  Runs on the CPU through numpy; used to check
    the fused op against the composition it replaces."""
    d = q.shape[-1]
    s = float(np.float32(1.0 / math.sqrt(d))) if scale is None else float(scale)
    scores = (q @ k.transpose()) * s
    if causal:
        scores = scores + Tensor(causal_mask(q.shape[-2], k.shape[-2], scores.dtype), requires_grad=False)
    shift = Tensor(np.max(scores.numpy(), axis=-1, keepdims=True), requires_grad=False)
    e = exp(scores - broadcast_to(shift, scores.shape))
    z = summation(e, axes=(len(e.shape) - 1,))
    zb = broadcast_to(reshape(z, tuple(z.shape) + (1,)), e.shape)
    return (e / zb) @ v
