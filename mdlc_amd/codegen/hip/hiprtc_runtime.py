"""hipRTC + HIP runtime for generated kernels, reached over ctypes.

Same surface as the reference's NVRTC/driver module
(mdlc/codegen/cuda/nvrtc_runtime.py:41-225) — an availability probe, a
source -> code-object compiler, a context that allocates, copies, loads,
launches and times — but every call goes through the C ABI of
``libmdlc_hip.so`` (include/mdlc_hip.h), which owns one HIP stream.

There is no fallback: if the library is missing or the device does not
initialise, the functions raise ``HipError``.
"""

from __future__ import annotations

import ctypes
import hashlib
import os
import struct
from typing import Optional

import numpy as np

from mdlc_amd.build import HIP_ARCH, LIB_PATH

CACHE_DIR = os.environ.get(
    "MDLC_CACHE_DIR", os.path.join(os.path.dirname(os.path.dirname(os.path.dirname(
        os.path.abspath(__file__)))), "_cache"))

RTC_OPTIONS = ("-O3", "-std=c++17", "-ffp-contract=off",
               "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops")


class HipError(RuntimeError):
    pass


_LIB: Optional[ctypes.CDLL] = None

_SIGS = {
    "mdlc_last_error": ([], ctypes.c_char_p),
    "mdlc_device_count": ([ctypes.POINTER(ctypes.c_int)], ctypes.c_int),
    "mdlc_init": ([ctypes.c_int, ctypes.c_char_p, ctypes.c_int], ctypes.c_int),
    "mdlc_rtc_compile": ([ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_char_p),
                          ctypes.c_int, ctypes.POINTER(ctypes.c_void_p),
                          ctypes.POINTER(ctypes.c_size_t), ctypes.c_char_p, ctypes.c_size_t],
                         ctypes.c_int),
    "mdlc_rtc_free": ([ctypes.c_void_p], None),
    "mdlc_rtc_version": ([ctypes.POINTER(ctypes.c_int)] * 3, ctypes.c_int),
    "mdlc_module_load": ([ctypes.c_void_p, ctypes.c_size_t, ctypes.POINTER(ctypes.c_void_p)],
                         ctypes.c_int),
    "mdlc_get_function": ([ctypes.c_void_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_void_p)],
                          ctypes.c_int),
    "mdlc_module_unload": ([ctypes.c_void_p], ctypes.c_int),
    "mdlc_malloc": ([ctypes.c_size_t, ctypes.POINTER(ctypes.c_void_p)], ctypes.c_int),
    "mdlc_free": ([ctypes.c_void_p], ctypes.c_int),
    "mdlc_memcpy_htod": ([ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t], ctypes.c_int),
    "mdlc_memcpy_dtoh": ([ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t], ctypes.c_int),
    "mdlc_memcpy_dtod": ([ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t], ctypes.c_int),
    "mdlc_launch": ([ctypes.c_void_p] + [ctypes.c_uint] * 7 + [ctypes.POINTER(ctypes.c_void_p)],
                    ctypes.c_int),
    "mdlc_sync": ([], ctypes.c_int),
    "mdlc_event_create": ([ctypes.POINTER(ctypes.c_void_p)], ctypes.c_int),
    "mdlc_event_destroy": ([ctypes.c_void_p], ctypes.c_int),
    "mdlc_event_record": ([ctypes.c_void_p], ctypes.c_int),
    "mdlc_event_elapsed_ms": ([ctypes.c_void_p, ctypes.c_void_p, ctypes.POINTER(ctypes.c_float)],
                              ctypes.c_int),
    "mdlc_plan_create": ([ctypes.c_void_p, ctypes.c_size_t, ctypes.POINTER(ctypes.c_void_p)],
                         ctypes.c_int),
    "mdlc_plan_destroy": ([ctypes.c_void_p], ctypes.c_int),
    "mdlc_plan_num_launches": ([ctypes.c_void_p, ctypes.POINTER(ctypes.c_int)], ctypes.c_int),
    "mdlc_plan_run": ([ctypes.c_void_p, ctypes.c_int], ctypes.c_int),
    "mdlc_plan_time_ms": ([ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                           ctypes.POINTER(ctypes.c_float)], ctypes.c_int),
    "mdlc_plan_profile": ([ctypes.c_void_p, ctypes.c_int, ctypes.POINTER(ctypes.c_float)],
                          ctypes.c_int),
    "mdlc_plan_use_graph": ([ctypes.c_void_p, ctypes.c_int], ctypes.c_int),
    "mdlc_plan_run_static": ([ctypes.c_void_p, ctypes.c_int], ctypes.c_int),
}

# Size of the library's static scratch array per GPU (mdlc_plan_run_static).
STATIC_SCRATCH_BYTES = 64 << 20


def lib() -> ctypes.CDLL:
    """The loaded ``libmdlc_hip.so`` (raises ``HipError`` if it is not built)."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise HipError(f"{LIB_PATH} is missing; build it with `python -m mdlc_amd.build`")
        try:
            handle = ctypes.CDLL(LIB_PATH)
        except OSError as exc:
            raise HipError(f"cannot load {LIB_PATH}: {exc}") from exc
        for name, (args, res) in _SIGS.items():
            fn = getattr(handle, name)
            fn.argtypes = args
            fn.restype = res
        _LIB = handle
    return _LIB


def _ck(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().mdlc_last_error().decode(errors="replace")
        raise HipError(f"{what} failed with HIP code {rc}: {msg}")


def hip_available() -> bool:
    """True iff the shim loads and at least one HIP device is visible."""
    try:
        n = ctypes.c_int(0)
        return lib().mdlc_device_count(ctypes.byref(n)) == 0 and n.value > 0
    except Exception:
        return False


# ----- hipRTC compile -------------------------------------------------------

_TOOLCHAIN: Optional[str] = None


def toolchain_version() -> str:
    """``"hiprtc-<major>.<minor>/hip-<runtime version>"`` of the loaded
    hipRTC and HIP runtime (no device needed)."""
    global _TOOLCHAIN
    if _TOOLCHAIN is None:
        a, b, r = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        _ck(lib().mdlc_rtc_version(ctypes.byref(a), ctypes.byref(b), ctypes.byref(r)),
            "mdlc_rtc_version")
        _TOOLCHAIN = f"hiprtc-{a.value}.{b.value}/hip-{r.value}"
    return _TOOLCHAIN


def _cache_key(source: str, name: str, arch: str, options: tuple) -> str:
    h = hashlib.sha256()
    for part in (toolchain_version(), source, name, arch, "\0".join(options)):
        h.update(part.encode())
        h.update(b"\x00")
    return h.hexdigest()


def compile_code_object(source: str, name: str = "kernels.hip", arch: str = HIP_ARCH,
                        options: Optional[tuple] = None, *, use_cache: bool = True) -> bytes:
    """Compile HIP source to a gfx950 code object with hipRTC.

    Results are cached on disk keyed by sha256(hipRTC and HIP runtime
    versions, source, name, arch, options), so a toolchain change never
    reloads an object the old compiler built.
    A compile error raises ``HipError`` carrying the full hipRTC log.
    """
    opts = (f"--offload-arch={arch}",) + tuple(options if options is not None else RTC_OPTIONS)
    key = _cache_key(source, name, arch, opts)
    path = os.path.join(CACHE_DIR, key + ".co")
    if use_cache and os.path.exists(path):
        with open(path, "rb") as f:
            blob = f.read()
        try:
            os.utime(path)          # last use, so stale objects can be told apart by age
        except OSError:
            pass
        return blob
    arr = (ctypes.c_char_p * len(opts))(*[o.encode() for o in opts])
    code = ctypes.c_void_p()
    size = ctypes.c_size_t()
    log = ctypes.create_string_buffer(1 << 16)
    rc = lib().mdlc_rtc_compile(source.encode(), name.encode(), arr, len(opts),
                                ctypes.byref(code), ctypes.byref(size), log, len(log))
    if rc != 0:
        msg = lib().mdlc_last_error().decode(errors="replace")
        raise HipError(f"hipRTC compile failed ({msg}):\n{log.value.decode(errors='replace')}")
    try:
        blob = ctypes.string_at(code, size.value)
    finally:
        lib().mdlc_rtc_free(code)
    if use_cache:
        os.makedirs(CACHE_DIR, exist_ok=True)
        tmp = f"{path}.{os.getpid()}.tmp"
        with open(tmp, "wb") as f:
            f.write(blob)
        os.replace(tmp, path)
    return blob


compile = compile_code_object  # noqa: A001 - the reference-facing name


# ----- device context / launching ---------------------------------------------

class HipCodeModule:
    """A loaded code object: resolve and launch its kernels."""

    def __init__(self, ctx: "HipContext", code: bytes) -> None:
        self.ctx = ctx
        self._code = ctypes.create_string_buffer(code, len(code))
        self._mod = ctypes.c_void_p()
        _ck(lib().mdlc_module_load(self._code, len(code), ctypes.byref(self._mod)),
            "hipModuleLoadData")
        self._funcs: dict = {}

    def close(self) -> None:
        """Unload the code object; its function handles become invalid."""
        if self._mod is not None and self._mod.value:
            _ck(lib().mdlc_module_unload(self._mod), "hipModuleUnload")
        self._mod = None
        self._funcs = {}

    def func(self, name: str) -> ctypes.c_void_p:
        if self._mod is None:
            raise HipError("code module is closed")
        if name not in self._funcs:
            f = ctypes.c_void_p()
            _ck(lib().mdlc_get_function(self._mod, name.encode(), ctypes.byref(f)),
                f"hipModuleGetFunction({name})")
            self._funcs[name] = f
        return self._funcs[name]

    def launch(self, name: str, grid, block, args: list, *, shared_bytes: int = 0) -> None:
        """Enqueue ``name``; ``args`` are ctypes values (pointers as
        ``c_void_p``, scalars as ``c_int``/``c_float``/``c_longlong``)."""
        f = self.func(name)
        argv = (ctypes.c_void_p * max(1, len(args)))()
        for i, a in enumerate(args):
            argv[i] = ctypes.cast(ctypes.byref(a), ctypes.c_void_p)
        gx, gy, gz = (list(grid) + [1, 1])[:3]
        bx, by, bz = (list(block) + [1, 1])[:3]
        _ck(lib().mdlc_launch(f, gx, gy, gz, bx, by, bz, shared_bytes, argv),
            f"hipModuleLaunchKernel({name})")


class HipContext:
    """Owns the device selection and the library stream; allocates, copies,
    loads code objects and times launches."""

    def __init__(self, device: int = 0) -> None:
        if not hip_available():
            raise HipError("no HIP device available")
        buf = ctypes.create_string_buffer(64)
        _ck(lib().mdlc_init(device, buf, len(buf)), "mdlc_init")
        self.device = device
        self.arch = buf.value.decode()

    def malloc(self, nbytes: int) -> ctypes.c_void_p:
        p = ctypes.c_void_p()
        _ck(lib().mdlc_malloc(int(nbytes), ctypes.byref(p)), "hipMalloc")
        return p

    def free(self, ptr) -> None:
        _ck(lib().mdlc_free(ptr), "hipFree")

    def htod(self, dst: int, arr: np.ndarray) -> None:
        arr = np.ascontiguousarray(arr)
        _ck(lib().mdlc_memcpy_htod(ctypes.c_void_p(int(dst)), arr.ctypes.data_as(ctypes.c_void_p),
                                   arr.nbytes), "hipMemcpy H2D")

    def dtoh(self, src: int, shape, dtype=np.float32) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        _ck(lib().mdlc_memcpy_dtoh(out.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(int(src)),
                                   out.nbytes), "hipMemcpy D2H")
        return out

    def to_device(self, arr: np.ndarray) -> ctypes.c_void_p:
        arr = np.ascontiguousarray(arr)
        p = self.malloc(arr.nbytes)
        self.htod(p.value, arr)
        return p

    def from_device(self, ptr, shape, dtype=np.float32) -> np.ndarray:
        return self.dtoh(ptr.value if isinstance(ptr, ctypes.c_void_p) else int(ptr), shape, dtype)

    def synchronize(self) -> None:
        _ck(lib().mdlc_sync(), "hipStreamSynchronize")

    def load_code(self, code: bytes) -> HipCodeModule:
        return HipCodeModule(self, code)

    def time_ms(self, fn, iters: int = 50, warmup: int = 10) -> float:
        """Average ms per call of ``fn`` (which enqueues work), by events."""
        a, b = ctypes.c_void_p(), ctypes.c_void_p()
        _ck(lib().mdlc_event_create(ctypes.byref(a)), "hipEventCreate")
        _ck(lib().mdlc_event_create(ctypes.byref(b)), "hipEventCreate")
        try:
            for _ in range(warmup):
                fn()
            self.synchronize()
            _ck(lib().mdlc_event_record(a), "hipEventRecord")
            for _ in range(iters):
                fn()
            _ck(lib().mdlc_event_record(b), "hipEventRecord")
            ms = ctypes.c_float()
            _ck(lib().mdlc_event_elapsed_ms(a, b, ctypes.byref(ms)), "hipEventElapsedTime")
            return ms.value / iters
        finally:
            lib().mdlc_event_destroy(a)
            lib().mdlc_event_destroy(b)


# ----- packed launch plans ------------------------------------------------------

class Arg:
    """A kernel argument for a packed plan: a raw value of a fixed width and
    its kind, which ``abi.check_launch`` matches against the kernel's
    declared parameter: ``p`` pointer, ``i`` 32-bit int, ``q`` 64-bit int,
    ``f`` float, ``d`` an ``mdlc::Dims6`` record."""

    __slots__ = ("data", "workspace", "kind")

    def __init__(self, data: bytes, workspace: bool = False, kind: str = "p") -> None:
        self.data = data
        self.workspace = workspace
        self.kind = kind

    @staticmethod
    def ws(offset: int) -> "Arg":
        """A pointer ``offset`` bytes into the plan's workspace (plan format 2)."""
        return Arg(struct.pack("<Q", int(offset)), workspace=True)

    @staticmethod
    def ptr(v: int) -> "Arg":
        return Arg(struct.pack("<Q", int(v)))

    @staticmethod
    def i32(v: int) -> "Arg":
        return Arg(struct.pack("<i", int(v)), kind="i")

    @staticmethod
    def i64(v: int) -> "Arg":
        return Arg(struct.pack("<q", int(v)), kind="q")

    @staticmethod
    def f32(v: float) -> "Arg":
        return Arg(struct.pack("<f", float(v)), kind="f")

    @staticmethod
    def dims6(vals, fill: int = 1) -> "Arg":
        """``mdlc::Dims6``: up to six ints, left-padded with ``fill`` to six
        (1 for extents, 0 for offsets)."""
        vals = [int(v) for v in vals]
        if len(vals) > 6:
            raise HipError(f"more than six dimensions: {vals}")
        return Arg(struct.pack("<6i", *([fill] * (6 - len(vals)) + vals)), kind="d")


def pack_plan(launches: list, workspace: Optional[tuple] = None) -> bytes:
    """Serialise [(function_handle, grid, block, lds_bytes, [Arg])] in the
    layout mdlc_plan_create expects. ``workspace`` = (base, bytes) writes
    format 2, where ``Arg.ws`` arguments are offsets into that workspace
    (base 0: none of the caller's, the plan runs on the static scratch)."""
    ver = 1 if workspace is None else 2
    out = [b"MDLP", struct.pack("<III", ver, len(launches), 0)]
    if workspace is not None:
        out.append(struct.pack("<QQ", int(workspace[0]), int(workspace[1])))
    for fn, grid, block, lds, args in launches:
        g = (list(grid) + [1, 1])[:3]
        bl = (list(block) + [1, 1])[:3]
        out.append(struct.pack("<Q3I3III", int(fn), *g, *bl, int(lds), len(args)))
        for a in args:
            n = len(a.data)
            if a.workspace and workspace is None:
                raise HipError("a workspace argument needs a format-2 plan")
            tag = (n | 0x80000000) if a.workspace else n
            out.append(struct.pack("<I", tag) + a.data + b"\0" * ((-n) % 8))
    return b"".join(out)


class Plan:
    """A launch plan living in the C++ runtime."""

    def __init__(self, launches: list, workspace: Optional[tuple] = None) -> None:
        blob = pack_plan(launches, workspace)
        self._blob = ctypes.create_string_buffer(blob, len(blob))
        self._h = ctypes.c_void_p()
        _ck(lib().mdlc_plan_create(self._blob, len(blob), ctypes.byref(self._h)),
            "mdlc_plan_create")
        self.n = len(launches)

    def run(self, iters: int = 1) -> None:
        _ck(lib().mdlc_plan_run(self._h, iters), "mdlc_plan_run")

    def run_static(self, iters: int = 1) -> None:
        """Run on the library's static scratch (allocates nothing)."""
        _ck(lib().mdlc_plan_run_static(self._h, iters), "mdlc_plan_run_static")

    def time_ms(self, warmup: int = 3, iters: int = 10) -> float:
        ms = ctypes.c_float()
        _ck(lib().mdlc_plan_time_ms(self._h, warmup, iters, ctypes.byref(ms)), "mdlc_plan_time_ms")
        return ms.value

    def profile(self, iters: int = 3) -> list:
        buf = (ctypes.c_float * max(1, self.n))()
        _ck(lib().mdlc_plan_profile(self._h, iters, buf), "mdlc_plan_profile")
        return [buf[i] for i in range(self.n)]

    def use_graph(self, enable: bool = True) -> None:
        _ck(lib().mdlc_plan_use_graph(self._h, 1 if enable else 0), "mdlc_plan_use_graph")

    def close(self) -> None:
        if self._h:
            lib().mdlc_plan_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self) -> None:  # pragma: no cover - best effort
        try:
            self.close()
        except Exception:
            pass
