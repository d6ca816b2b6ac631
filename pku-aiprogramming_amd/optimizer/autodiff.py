"""Reverse-mode differentiation over the ``Value`` graph.

Follows the reference driver (Task3/Tinytensor/optimizer/autodiff.py:9-61):
a post-order DFS gives a topological order; the output is seeded with
``out_grad``; nodes are visited in reverse order, each node's gradient
contributions are summed in the order they were produced (first + second +
...), stored in ``node.grad`` and pushed through ``op.gradient_as_tuple`` to
the inputs.

The DFS is iterative here, so deep graphs need no recursion-limit change
(the reference raises the limit to 10**8 at :7 instead).
"""
from __future__ import annotations

from typing import Dict, List

from basic_operator import Value


def find_topo_sort(node_list: List[Value]) -> List[Value]:
    """Topological order (inputs before users) of the graph ending at
    ``node_list``: post-order DFS along input edges."""
    visited = set()
    order: List[Value] = []
    for root in node_list:
        if root in visited:
            continue
        visited.add(root)
        stack = [(root, iter(root.inputs))]
        while stack:
            node, it = stack[-1]
            nxt = next(it, None)
            if nxt is None:
                stack.pop()
                order.append(node)
            elif nxt not in visited:
                visited.add(nxt)
                stack.append((nxt, iter(nxt.inputs)))
    return order


def compute_gradient_of_variables(output_tensor: Value, out_grad: Value) -> None:
    """Set ``.grad`` on every node that ``output_tensor`` depends on, for the
    upstream gradient ``out_grad`` (i.e. the gradient of
    sum(output * out_grad))."""
    contributions: Dict[Value, List[Value]] = {output_tensor: [out_grad]}
    for node in reversed(find_topo_sort([output_tensor])):
        parts = contributions.get(node)
        if not parts:
            continue
        total = parts[0]
        for extra in parts[1:]:
            total = total + extra
        node.grad = total
        if node.op is None:
            continue
        for inp, g in zip(node.inputs, node.op.gradient_as_tuple(total, node)):
            contributions.setdefault(inp, []).append(g)
