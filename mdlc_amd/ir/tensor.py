"""Value metadata carried by graph edges: dtype names and static shapes.

Mirrors the reference's ``DType`` / ``TensorInfo`` contract
(mdlc/ir/tensor.py:17-98): dtype names are strings, a dimension is an int, a
symbolic name, or None, and codegen only accepts fully static shapes.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional, Union

import numpy as np

Dim = Union[int, str, None]
Shape = tuple


class DType:
    """String dtype names and their NumPy equivalents (tensor.py:17-53).

    INT8 and INT32 carry the quantized path: int8 activations and weights,
    int32 biases and accumulators.
    """

    FLOAT32 = "float32"
    FLOAT16 = "float16"
    INT64 = "int64"
    INT32 = "int32"
    INT8 = "int8"
    BOOL = "bool"

    _NP = {
        "float32": np.float32,
        "float16": np.float16,
        "int64": np.int64,
        "int32": np.int32,
        "int8": np.int8,
        "bool": np.bool_,
    }

    @classmethod
    def to_numpy(cls, name: str) -> np.dtype:
        try:
            return np.dtype(cls._NP[name])
        except KeyError:
            raise KeyError(f"unsupported dtype: {name!r}") from None

    @classmethod
    def from_numpy(cls, dt) -> str:
        want = np.dtype(dt)
        for name, t in cls._NP.items():
            if np.dtype(t) == want:
                return name
        raise KeyError(f"unsupported numpy dtype: {want!r}")

    @classmethod
    def itemsize(cls, name: str) -> int:
        return cls.to_numpy(name).itemsize


@dataclass
class TensorInfo:
    """Type and shape of one named edge (not its data)."""

    name: str
    dtype: str = DType.FLOAT32
    shape: Shape = field(default_factory=tuple)

    @property
    def is_static(self) -> bool:
        return all(isinstance(d, (int, np.integer)) and d >= 0 for d in self.shape)

    @property
    def rank(self) -> int:
        return len(self.shape)

    def numel(self) -> Optional[int]:
        if not self.is_static:
            return None
        return int(np.prod([int(d) for d in self.shape], dtype=np.int64)) if self.shape else 1

    def nbytes(self) -> Optional[int]:
        n = self.numel()
        return None if n is None else n * DType.itemsize(self.dtype)

    def with_shape(self, shape) -> "TensorInfo":
        return TensorInfo(self.name, self.dtype, tuple(shape))

    def __repr__(self) -> str:
        dims = "x".join(str(d) for d in self.shape) if self.shape else "scalar"
        return f"{self.name}:{self.dtype}[{dims}]"
