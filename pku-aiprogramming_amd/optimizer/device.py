"""Device handle of the TinyTensor Python layer.

Graph data of the Python layer always lives in host numpy arrays; the GPU
operators move it to the MI355X inside their forward / gradient and bring the
result back.  So the only device a graph node reports is the host, and the
only part of the reference's device module its callers use is that handle:
``cpu()``, compared by value and usable as a dict key
(reference: Task3/Tinytensor/optimizer/device.py:9-59, used by
optimizer/operators.py:8,40-58).
"""
from __future__ import annotations


class Device:
    """A named place where a node's data lives; equal when the names are."""

    __slots__ = ("name",)

    def __init__(self, name: str):
        self.name = name

    def __repr__(self) -> str:
        return f"{self.name}()"

    def __eq__(self, other) -> bool:
        return isinstance(other, Device) and other.name == self.name

    def __hash__(self) -> int:
        return hash(("Device", self.name))

    def enabled(self) -> bool:
        """Whether node data can be held here (only the host can)."""
        return self.name == "cpu"


_HOST = Device("cpu")


def cpu() -> Device:
    """The host device: where every node's numpy data lives."""
    return _HOST
