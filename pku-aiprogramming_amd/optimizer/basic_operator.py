"""Graph nodes and operators of the TinyTensor Python layer.

The protocol callers rely on (reference: Task3/Tinytensor/optimizer/
basic_operator.py:11-39 and :43-105) is kept: an ``Op`` has
``compute(*arrays)`` for the forward on realised data and
``gradient(out_grad, node)`` for the vector-Jacobian product, and
``gradient_as_tuple`` always yields a tuple; a ``Value`` carries ``op``,
``inputs``, ``cached_data`` and ``requires_grad`` and hands out its data by
``realize_cached_data()``; ``make_const`` and ``make_from_op`` build leaves and
op nodes.

How it works here:

* nodes are evaluated eagerly when they are made, and a node none of whose
  inputs needs a gradient is cut from the graph on the spot (it keeps its data
  and becomes a leaf), so no dead subgraph is kept alive;
* the forward runs through ``Op.forward(node, *arrays)``.  By default that is
  ``compute``; an operator that must carry state from its forward to its
  gradient (device buffers, a log-sum-exp) overrides it and keeps the state on
  the node (``node.saved``), never on the operator object, so one operator
  instance can serve any number of nodes.
"""
from __future__ import annotations

from typing import Any, Iterable, Optional, Tuple

# Graph nodes made and not yet collected in this process, as the reference's
# module counter (basic_operator.py:9, 63-65, 76-77).
TENSOR_COUNTER = 0


class Op:
    """An operation of the graph."""

    def __call__(self, *args):
        raise NotImplementedError()

    def compute(self, *arrays):
        """Forward on realised input arrays; returns the output array."""
        raise NotImplementedError()

    def forward(self, node: "Value", *arrays):
        """Forward of `node`; operators with per-node state override this."""
        return self.compute(*arrays)

    def gradient(self, out_grad: "Value", node: "Value"):
        """Gradients of sum(node * out_grad) with respect to node.inputs, as
        graph values (one value, or a tuple / list of them)."""
        raise NotImplementedError()

    def gradient_as_tuple(self, out_grad: "Value", node: "Value") -> Tuple["Value", ...]:
        g = self.gradient(out_grad, node)
        if isinstance(g, (tuple, list)):
            return tuple(g)
        return (g,)


class Value:
    """A node of the graph: the op that made it, its inputs, its data."""

    op: Optional[Op]
    inputs: list
    cached_data: Any
    requires_grad: bool

    _counted = False  # whether TENSOR_COUNTER holds this node

    def _setup(self, op: Optional[Op], inputs: Iterable["Value"], data, requires_grad: Optional[bool]) -> None:
        global TENSOR_COUNTER
        if not self._counted:
            TENSOR_COUNTER += 1
            self._counted = True
        self.op = op
        self.inputs = list(inputs)
        self.cached_data = data
        if requires_grad is None:
            requires_grad = any(x.requires_grad for x in self.inputs)
        self.requires_grad = bool(requires_grad)
        self.saved = None  # per-node state an op keeps between forward and gradient

    def __del__(self):
        global TENSOR_COUNTER
        if self._counted:
            try:
                TENSOR_COUNTER -= 1
            except TypeError:  # interpreter shutdown may have cleared the module
                pass

    def realize_cached_data(self):
        if self.cached_data is None:
            self.cached_data = self.op.forward(self, *[x.realize_cached_data() for x in self.inputs])
        return self.cached_data

    def is_leaf(self) -> bool:
        return self.op is None

    @classmethod
    def make_const(cls, data, *, requires_grad: bool = False):
        node = cls.__new__(cls)
        node._setup(None, (), data, requires_grad)
        return node

    @classmethod
    def make_from_op(cls, op: Op, inputs):
        node = cls.__new__(cls)
        node._setup(op, inputs, None, None)
        node.realize_cached_data()
        if not node.requires_grad:
            # nothing upstream needs a gradient: keep the data, drop the graph
            node.op, node.inputs, node.saved = None, [], None
        return node
