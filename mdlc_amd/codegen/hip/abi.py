"""Launch arguments checked against the kernels' own declarations.

``hipModuleLaunchKernel`` copies each entry of a launch's argument array by
the width the kernel's metadata gives for that position. A launch whose
argument list differs from the kernel's parameter list is therefore not
rejected by HIP: every argument after the first difference lands in the
wrong parameter. An extra pointer in front of the integers, for example,
makes the kernel read the low half of an address as its row count and store
through another tensor's base. The executor runs ``check_launch`` on every
launch before it packs a plan, so such a mismatch raises on the host instead
of reaching the device.

Kinds: ``p`` pointer, ``i`` 32-bit int, ``q`` 64-bit int, ``f`` float,
``d`` an ``mdlc::Dims6`` record (six ints by value).
"""

from __future__ import annotations

import re
from typing import Dict, Sequence

_DECL = re.compile(r'extern "C"\s+__global__\s+(?:__launch_bounds__\(\s*\d+\s*(?:,\s*\d+\s*)?\)\s+)?void\s+'
                   r"(\w+)\s*\(([^)]*)\)")


class LaunchAbiError(ValueError):
    """A launch's argument kinds differ from its kernel's parameter kinds."""


def _kind(param: str) -> str:
    p = " ".join(param.split())
    if "*" in p:
        return "p"
    if "Dims6" in p:
        return "d"
    if re.search(r"\b(long long|int64_t|size_t)\b", p):
        return "q"
    if re.search(r"\bfloat\b", p):
        return "f"
    if re.search(r"\b(int|unsigned)\b", p):
        return "i"
    raise LaunchAbiError(f"kernel parameter {param!r} has no argument kind")


def declared_kinds(source: str) -> Dict[str, str]:
    """{kernel name: parameter kinds as a string} for every ``extern "C"``
    kernel declared in ``source``."""
    out = {}
    for m in _DECL.finditer(source):
        params = [p for p in m.group(2).split(",") if p.strip()]
        out[m.group(1)] = "".join(_kind(p) for p in params)
    return out


def check_launch(kernel: str, declared: Dict[str, str], arg_kinds: Sequence[str]) -> None:
    """Raise ``LaunchAbiError`` unless ``arg_kinds`` equals the declared
    parameter kinds of ``kernel``, position by position."""
    want = declared.get(kernel)
    if want is None:
        raise LaunchAbiError(f"kernel {kernel!r} has no extern \"C\" declaration in its module")
    got = "".join(arg_kinds)
    if got != want:
        at = next((i for i, (a, b) in enumerate(zip(got, want)) if a != b), min(len(got), len(want)))
        raise LaunchAbiError(
            f"launch of {kernel!r} passes argument kinds {got!r} but the kernel declares {want!r} "
            f"(first difference at argument {at})")
