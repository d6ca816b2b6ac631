"""Reverse-mode differentiation over the ``Value`` graph.

Same entry points and results as the reference driver
(Task3/Tinytensor/optimizer/autodiff.py:9-61): ``find_topo_sort`` returns the
nodes inputs-first, ``topo_sort_dfs`` is its post-order walk helper, and
``compute_gradient_of_variables(output, out_grad)`` leaves in every node's
``.grad`` the gradient of sum(output * out_grad).

The order is found by Kahn's algorithm on user counts instead of a recursive
depth-first search, so graphs of any depth need no recursion limit: a node
is processed once every node that uses it has pushed its contribution, and
contributions are added up in the order they arrive.
"""
from __future__ import annotations

from collections import deque
from typing import Dict, List

from basic_operator import Value


def _users_first(outputs: List[Value]) -> List[Value]:
    """Every node reachable from `outputs`, each after all of its users."""
    users: Dict[Value, int] = {}
    stack = []
    for root in outputs:
        if root not in users:
            users[root] = 0
            stack.append(root)
    while stack:  # count the edges into each reachable node
        node = stack.pop()
        for inp in node.inputs:
            if inp in users:
                users[inp] += 1
            else:
                users[inp] = 1
                stack.append(inp)
    ready = deque(n for n in dict.fromkeys(outputs) if users[n] == 0)
    order: List[Value] = []
    while ready:
        node = ready.popleft()
        order.append(node)
        for inp in node.inputs:
            users[inp] -= 1
            if users[inp] == 0:
                ready.append(inp)
    return order


def topo_sort_dfs(node: Value, visited: set, topo_order: List[Value]) -> None:
    """Post-order depth-first walk from `node` (the reference's helper of the
    same name, autodiff.py:24-31): every node reachable from it that is not in
    `visited` yet is added to `visited` and appended to `topo_order` after its
    inputs, which are walked in list order.  Iterative, so a deep graph needs
    no recursion limit."""
    if node in visited:
        return
    visited.add(node)
    stack = [(node, iter(node.inputs))]
    while stack:
        cur, rest = stack[-1]
        for inp in rest:
            if inp not in visited:
                visited.add(inp)
                stack.append((inp, iter(inp.inputs)))
                break
        else:
            stack.pop()
            topo_order.append(cur)


def find_topo_sort(node_list: List[Value]) -> List[Value]:
    """Topological order of the graph ending at `node_list`: every node comes
    after all of its inputs."""
    return _users_first(node_list)[::-1]


def compute_gradient_of_variables(output_tensor: Value, out_grad: Value) -> None:
    """Set ``.grad`` on `output_tensor` and every node it depends on, for the
    upstream gradient `out_grad` (the gradient of sum(output * out_grad))."""
    pending: Dict[Value, Value] = {output_tensor: out_grad}
    for node in _users_first([output_tensor]):
        grad = pending.pop(node, None)
        if grad is None:
            continue
        node.grad = grad
        if node.op is None:
            continue
        for inp, part in zip(node.inputs, node.op.gradient_as_tuple(grad, node)):
            prev = pending.get(inp)
            pending[inp] = part if prev is None else prev + part
