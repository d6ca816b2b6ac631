"""Graph primitives of the TinyTensor autodiff: ``Op`` and ``Value``.

Same contract as the reference (Task3/Tinytensor/optimizer/basic_operator.py):

* ``Op.compute(*arrays)`` runs the forward on realised inputs,
  ``Op.gradient(out_grad, node)`` returns the input gradients, and
  ``Op.gradient_as_tuple`` always hands back a tuple (:11-39);
* ``Value`` is a graph node with ``op``, ``inputs``, ``cached_data`` and
  ``requires_grad``; data is realised eagerly and cached (:43-105);
* ``make_const`` builds a leaf, ``make_from_op`` a node that is realised at
  once and detached when no input requires a gradient.
"""
from __future__ import annotations

from typing import List, Optional, Tuple, Union

import numpy as np

# Number of live graph nodes (kept for parity with the reference's counter).
TENSOR_COUNTER = 0


class Op:
    """An operator of the graph."""

    def __call__(self, *args):
        raise NotImplementedError()

    def compute(self, *args: Tuple[np.ndarray]):
        raise NotImplementedError()

    def gradient(self, out_grad: "Value", node: "Value") -> Union["Value", Tuple["Value", ...]]:
        raise NotImplementedError()

    def gradient_as_tuple(self, out_grad: "Value", node: "Value") -> Tuple["Value", ...]:
        grads = self.gradient(out_grad, node)
        if isinstance(grads, tuple):
            return grads
        if isinstance(grads, list):
            return tuple(grads)
        return (grads,)


class Value:
    """A node: the op that made it, its inputs and its realised data."""

    op: Optional[Op]
    inputs: List["Value"]
    cached_data: object
    requires_grad: bool

    def realize_cached_data(self):
        if self.cached_data is None:
            self.cached_data = self.op.compute(*[x.realize_cached_data() for x in self.inputs])
        return self.cached_data

    def is_leaf(self) -> bool:
        return self.op is None

    def __del__(self):
        global TENSOR_COUNTER
        TENSOR_COUNTER -= 1

    def _init(self, op, inputs, *, num_outputs: int = 1, cached_data=None, requires_grad: Optional[bool] = None):
        global TENSOR_COUNTER
        TENSOR_COUNTER += 1
        if requires_grad is None:
            requires_grad = any(x.requires_grad for x in inputs)
        self.op = op
        self.inputs = list(inputs)
        self.num_outputs = num_outputs
        self.cached_data = cached_data
        self.requires_grad = requires_grad

    @classmethod
    def make_const(cls, data, *, requires_grad: bool = False):
        v = cls.__new__(cls)
        v._init(None, [], cached_data=data, requires_grad=requires_grad)
        return v

    @classmethod
    def make_from_op(cls, op: Op, inputs: List["Value"]):
        v = cls.__new__(cls)
        v._init(op, inputs)
        if not v.requires_grad:
            return v.detach()
        v.realize_cached_data()
        return v
