"""One operator of the graph IR (contract of mdlc/ir/node.py:10-49)."""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Optional


@dataclass
class Node:
    """An op_type with named input/output edges and decoded attributes.

    An empty string in ``inputs`` marks an omitted optional input (ONNX
    convention). Fused nodes record the op types they replaced in
    ``fused_from``; a ``FusedElementwise`` node keeps its member nodes in
    ``attrs["subgraph"]``.
    """

    op_type: str
    inputs: list = field(default_factory=list)
    outputs: list = field(default_factory=list)
    attrs: dict = field(default_factory=dict)
    name: str = ""
    fused_from: Optional[list] = None

    def attr(self, key: str, default: Any = None) -> Any:
        return self.attrs.get(key, default)

    @property
    def is_fused(self) -> bool:
        return self.fused_from is not None

    def real_inputs(self) -> list:
        return [e for e in self.inputs if e]

    def replace_input(self, old: str, new: str) -> None:
        self.inputs = [new if e == old else e for e in self.inputs]

    def __repr__(self) -> str:
        tag = "" if not self.fused_from else " <-" + "+".join(self.fused_from)
        return f"{self.op_type}({', '.join(self.inputs)}) -> ({', '.join(self.outputs)}){tag}"
