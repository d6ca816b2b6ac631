"""Device handles of the TinyTensor Python layer.

Graph data of the Python layer always lives in host numpy arrays; the GPU
operators move it to the MI355X inside their forward / gradient and bring the
result back.  So the one device a graph node reports is the host.  The module
keeps the reference's public surface (Task3/Tinytensor/optimizer/device.py:
9-59): the ``Device`` base, ``CPUDevice`` with its array factories (``zeros``,
``ones``, ``randn``, ``rand``, ``one_hot``, ``empty``, ``full``), ``cpu()``,
``default_device()`` and ``all_devices()``.  Handles compare by name and can
be dict keys; ``randn`` / ``rand`` draw from numpy's global generator, so a
caller's ``np.random.seed`` fixes them as before.
"""
from __future__ import annotations

import numpy as np


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
        return hash(repr(self))

    def enabled(self) -> bool:
        """Whether node data can be held here (only the host can)."""
        return self.name == "cpu"


class CPUDevice(Device):
    """The host: node data are numpy arrays, made by the factories below."""

    __slots__ = ()

    def __init__(self):
        super().__init__("cpu")

    def zeros(self, *shape, dtype="float32") -> np.ndarray:
        return np.zeros(shape, dtype=dtype)

    def ones(self, *shape, dtype="float32") -> np.ndarray:
        return np.ones(shape, dtype=dtype)

    def randn(self, *shape) -> np.ndarray:
        """Standard normal samples (float64, as numpy draws them)."""
        return np.random.randn(*shape)

    def rand(self, *shape) -> np.ndarray:
        """Uniform [0, 1) samples (float64)."""
        return np.random.rand(*shape)

    def one_hot(self, n, i, dtype="float32") -> np.ndarray:
        """Row(s) i of the n x n identity: one-hot codes of the index or
        index array i."""
        return np.eye(n, dtype=dtype)[i]

    def empty(self, shape, dtype="float32") -> np.ndarray:
        return np.empty(shape, dtype=dtype)

    def full(self, shape, fill_value, dtype="float32") -> np.ndarray:
        return np.full(shape, fill_value, dtype=dtype)


_HOST = CPUDevice()


def cpu() -> CPUDevice:
    """The host device: where every node's numpy data lives."""
    return _HOST


def default_device() -> CPUDevice:
    return _HOST


def all_devices() -> list:
    return [_HOST]
