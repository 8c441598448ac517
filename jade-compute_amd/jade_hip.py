"""ctypes binding of libjade_runtime_hip.so (include/jade_runtime_hip.h,
include/jade_gemm_hip.h).

`HipRuntime` mirrors the reference's owned-buffer `Runtime` trait
(src/runtime/mod.rs:45-61) the way its CoreX backend drives the C ABI
(src/runtime/corex.rs:206-612): buffers and kernels belong to one runtime,
uploads are exact-length, `execute` validates the whole batch before any work
is enqueued, replays it `repeats` times and returns an `Execution` whose
`gpu_ms` is None when the device timer reads zero (corex.rs:601-608).
`GemmPlan` mirrors the per-shape GEMM plan of src/corex.rs:57-190.

There is no CPU fallback: constructing a runtime without the built library or
without a GPU raises.
"""
from __future__ import annotations

import ctypes
import json
import os
import time
from dataclasses import dataclass
from typing import Iterable, Optional, Sequence

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIBRARY_PATH = os.path.join(_HERE, "libjade_runtime_hip.so")
ERROR_CAPACITY = 1024  # bytes the reference's Rust caller passes (corex.rs:366)

_c = ctypes
_vp = _c.c_void_p
_sz = _c.c_size_t
_cp = _c.c_char_p


class JadeError(RuntimeError):
    """A nonzero status from the C ABI: 1 invalid, 2 runtime, 3 allocation
    (4 allocation for the GEMM-plan ABI)."""

    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code
        self.message = message


class _Job(_c.Structure):
    _fields_ = [("launch", _vp), ("buffers", _c.POINTER(_vp)), ("buffer_count", _sz)]


class _Dispatch(_c.Structure):
    _fields_ = [("kernel", _vp), ("buffers", _c.POINTER(_vp)), ("buffer_count", _sz)]


_lib_cache: dict = {}


def load(path: Optional[str] = None) -> ctypes.CDLL:
    """Loads the library and declares every exported signature."""
    path = path or LIBRARY_PATH
    if path in _lib_cache:
        return _lib_cache[path]
    if not os.path.exists(path):
        raise FileNotFoundError(
            f"{path} is not built; run __graft_entry__.build() (make -C jade-compute_amd)")
    lib = _c.CDLL(path)
    sig = {
        "jr_version": (_c.c_uint32, []),
        "jr_create": (_c.c_int, [_c.c_int, _c.POINTER(_vp), _cp, _sz]),
        "jr_destroy": (None, [_vp]),
        "jr_info": (_c.c_int, [_vp, _cp, _sz, _cp, _sz]),
        "jr_alloc": (_c.c_int, [_vp, _sz, _c.POINTER(_vp), _cp, _sz]),
        "jr_free": (None, [_vp, _vp]),
        "jr_upload": (_c.c_int, [_vp, _vp, _vp, _sz, _cp, _sz]),
        "jr_download": (_c.c_int, [_vp, _vp, _vp, _sz, _cp, _sz]),
        "jr_execute": (_c.c_int, [_vp, _c.POINTER(_Job), _sz, _c.c_uint32, _c.POINTER(_c.c_double), _cp, _sz]),
        "jr_spec_describe": (_c.c_int, [_cp, _sz, _cp, _sz, _cp, _sz]),
        "jr_spec_validate_bindings": (_c.c_int, [_cp, _sz, _c.POINTER(_c.c_uint64), _c.POINTER(_c.c_uint64), _sz,
                                                 _cp, _sz]),
        "jr_compile": (_c.c_int, [_vp, _cp, _sz, _c.POINTER(_vp), _cp, _sz]),
        "jr_kernel_release": (None, [_vp, _vp]),
        "jr_kernel_describe": (_c.c_int, [_vp, _vp, _cp, _sz, _cp, _sz]),
        "jr_execute_dispatches": (_c.c_int, [_vp, _c.POINTER(_Dispatch), _sz, _c.c_uint32,
                                             _c.POINTER(_c.c_double), _cp, _sz]),
        "jr_plan_dispatches": (_c.c_int, [_vp, _c.POINTER(_Dispatch), _sz, _cp, _sz, _cp, _sz]),
        "jr_buffer_elements": (_c.c_int, [_vp, _vp, _c.POINTER(_sz), _cp, _sz]),
        "jr_fill_values": (_c.c_int, [_vp, _sz, _c.c_uint32, _c.c_float]),
        "jr_fill_normal": (_c.c_int, [_vp, _sz, _c.c_uint32, _c.c_float, _c.c_float]),
        "jade_corex_abi_version": (_c.c_uint32, []),
        "jade_corex_create": (_c.c_int, [_c.c_uint32, _c.c_uint32, _c.c_uint32, _c.c_int, _c.c_uint32,
                                         _c.POINTER(_vp), _cp, _sz]),
        "jade_corex_upload": (_c.c_int, [_vp, _vp, _sz, _vp, _sz, _cp, _sz]),
        "jade_corex_run": (_c.c_int, [_vp, _c.c_uint32, _c.POINTER(_c.c_double), _cp, _sz]),
        "jade_corex_download": (_c.c_int, [_vp, _vp, _sz, _cp, _sz]),
        "jade_corex_device_info": (_c.c_int, [_vp, _cp, _sz, _cp, _sz]),
        "jade_corex_destroy": (None, [_vp]),
    }
    for name, (restype, argtypes) in sig.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    _lib_cache[path] = lib
    return lib


def _error_buffer():
    return _c.create_string_buffer(ERROR_CAPACITY)


def _check(code: int, err) -> None:
    if code != 0:
        raise JadeError(code, err.value.decode(errors="replace"))


def _f32(data) -> np.ndarray:
    return np.ascontiguousarray(data, dtype=np.float32)


def spec_json(spec) -> str:
    return spec if isinstance(spec, str) else json.dumps(spec)


def spec_describe(spec, lib: Optional[ctypes.CDLL] = None) -> dict:
    """Validates a KernelSpec without a device and returns its description."""
    lib = lib or load()
    text = spec_json(spec).encode()
    out = _c.create_string_buffer(1 << 16)
    err = _error_buffer()
    _check(lib.jr_spec_describe(text, len(text), out, len(out), err, len(err)), err)
    return json.loads(out.value.decode())


def spec_validate_bindings(spec, lengths: Sequence[int], ids: Sequence[int], lib=None) -> None:
    """KernelSpec::validate_bindings (src/runtime/ir.rs:340-367); raises JadeError."""
    lib = lib or load()
    text = spec_json(spec).encode()
    n = len(lengths)
    lens = (_c.c_uint64 * max(1, n))(*lengths)
    idents = (_c.c_uint64 * max(1, len(ids)))(*ids)
    err = _error_buffer()
    _check(lib.jr_spec_validate_bindings(text, len(text), lens, idents, n, err, len(err)), err)


def fill_values(length: int, seed: int, scale: float = 1.0, lib=None) -> np.ndarray:
    """workloads::values (src/runtime/workloads.rs:17-27)."""
    lib = lib or load()
    out = np.empty(length, dtype=np.float32)
    if lib.jr_fill_values(out.ctypes.data_as(_vp), length, seed & 0xFFFFFFFF, scale) != 0:
        raise JadeError(1, "jr_fill_values rejected its arguments")
    return out


def fill_normal(length: int, seed: int, mean: float = 0.0, sigma: float = 1.0, lib=None) -> np.ndarray:
    """Box-Muller normal inputs over the xorshift32 stream."""
    lib = lib or load()
    out = np.empty(length, dtype=np.float32)
    if lib.jr_fill_normal(out.ctypes.data_as(_vp), length, seed & 0xFFFFFFFF, mean, sigma) != 0:
        raise JadeError(1, "jr_fill_normal rejected its arguments")
    return out


@dataclass
class Execution:
    """src/runtime/mod.rs:23-29."""
    host_ms: float
    gpu_ms: Optional[float]
    dispatches: int
    repeats: int


class Buffer:
    """A device allocation of `len()` f32 elements owned by one runtime."""

    def __init__(self, runtime: "HipRuntime", ptr: int, elements: int):
        self._runtime = runtime
        self.ptr = ptr
        self.elements = elements

    def __len__(self) -> int:
        return self.elements

    @property
    def id(self) -> int:
        return self.ptr

    def free(self) -> None:
        if self.ptr and self._runtime._ctx:
            self._runtime._lib.jr_free(self._runtime._ctx, self.ptr)
        self.ptr = 0


class Kernel:
    """A compiled pipeline handle plus its checked description."""

    def __init__(self, runtime: "HipRuntime", handle: int, description: dict):
        self._runtime = runtime
        self.handle = handle
        self.description = description
        self.spec = description["spec"]
        self.name = description["name"]
        self.bindings = description["bindings"]
        self.launch = description["launch"]

    def release(self) -> None:
        if self.handle and self._runtime._ctx:
            self._runtime._lib.jr_kernel_release(self._runtime._ctx, self.handle)
        self.handle = 0


class HipRuntime:
    """The HIP backend behind the reference's Runtime contract."""

    def __init__(self, device: int = 0, library: Optional[str] = None):
        self._lib = load(library)
        if self._lib.jr_version() < 2:
            raise JadeError(1, "libjade_runtime_hip ABI 2 required")
        ctx = _vp()
        err = _error_buffer()
        _check(self._lib.jr_create(device, _c.byref(ctx), err, len(err)), err)
        self._ctx = ctx.value
        self.device = device
        out = _c.create_string_buffer(1024)
        _check(self._lib.jr_info(self._ctx, out, len(out), err, len(err)), err)
        self.device_info = out.value.decode()

    # -- lifetime ---------------------------------------------------------
    def close(self) -> None:
        if getattr(self, "_ctx", None):
            self._lib.jr_destroy(self._ctx)
            self._ctx = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- Runtime trait ----------------------------------------------------
    def info(self) -> dict:
        """RuntimeInfo (src/runtime/mod.rs:15-21)."""
        return {
            "backend": "HIP native precompiled gfx950 kernels",
            "device": self.device_info,
            "execution": "ordered launches on one persistent non-blocking stream; hipEvent timing over the "
                         "whole replayed sequence",
            "limitations": [
                "FP32 buffers and validated KernelSpec operations only; gemm_mps is an Apple library op",
                "Synchronous API; ordered replay uses host launches, not HIP graphs",
            ],
        }

    def _own(self, buffer: Buffer) -> None:
        if not isinstance(buffer, Buffer) or buffer._runtime is not self or not buffer.ptr:
            raise JadeError(1, "buffer belongs to another runtime/device context")

    def alloc(self, elements: int) -> Buffer:
        if elements <= 0:
            raise JadeError(1, "buffer allocation must be nonempty")
        ptr = _vp()
        err = _error_buffer()
        _check(self._lib.jr_alloc(self._ctx, elements * 4, _c.byref(ptr), err, len(err)), err)
        return Buffer(self, ptr.value, elements)

    def upload(self, buffer: Buffer, data) -> None:
        self._own(buffer)
        host = _f32(data).reshape(-1)
        if host.size != buffer.elements:
            raise JadeError(1, "upload element count must match buffer exactly")
        err = _error_buffer()
        _check(self._lib.jr_upload(self._ctx, buffer.ptr, host.ctypes.data_as(_vp), host.nbytes, err, len(err)),
               err)

    def download(self, buffer: Buffer) -> np.ndarray:
        self._own(buffer)
        out = np.empty(buffer.elements, dtype=np.float32)
        err = _error_buffer()
        _check(self._lib.jr_download(self._ctx, buffer.ptr, out.ctypes.data_as(_vp), out.nbytes, err, len(err)),
               err)
        return out

    def compile(self, spec) -> Kernel:
        text = spec_json(spec).encode()
        handle = _vp()
        err = _error_buffer()
        _check(self._lib.jr_compile(self._ctx, text, len(text), _c.byref(handle), err, len(err)), err)
        out = _c.create_string_buffer(1 << 16)
        _check(self._lib.jr_kernel_describe(self._ctx, handle.value, out, len(out), err, len(err)), err)
        return Kernel(self, handle.value, json.loads(out.value.decode()))

    def _dispatches(self, jobs: Sequence):
        arrays = []
        native = (_Dispatch * len(jobs))()
        for i, (kernel, buffers) in enumerate(jobs):
            if not isinstance(kernel, Kernel) or kernel._runtime is not self or not kernel.handle:
                raise JadeError(1, "kernel belongs to another runtime/device context")
            for b in buffers:
                self._own(b)
            ptrs = (_vp * max(1, len(buffers)))(*[b.ptr for b in buffers])
            arrays.append(ptrs)
            native[i].kernel = kernel.handle
            native[i].buffers = _c.cast(ptrs, _c.POINTER(_vp))
            native[i].buffer_count = len(buffers)
        return native, arrays

    def plan(self, jobs: Sequence) -> list:
        """The launches execute() would make for these jobs, as (form, first
        job) pairs: form "single", "pair", "gate_up_swiglu" or
        "gemm_residual" (jr_plan_dispatches)."""
        if not jobs:
            raise JadeError(1, "a plan needs jobs")
        native, _keep = self._dispatches(jobs)
        out = _c.create_string_buffer(1 << 16)
        err = _error_buffer()
        _check(self._lib.jr_plan_dispatches(self._ctx, native, len(jobs), out, len(out), err, len(err)), err)
        return [(form, int(first)) for form, first in (item.split(":") for item in out.value.decode().split())]

    def execute(self, jobs: Sequence, repeats: int) -> Execution:
        """jobs: sequence of (Kernel, [Buffer, ...]) in dispatch order."""
        if not jobs or repeats <= 0:
            raise JadeError(1, "execution requires jobs and positive repeats")
        native, _keep = self._dispatches(jobs)
        gpu_ms = _c.c_double(0.0)
        err = _error_buffer()
        started = time.perf_counter()
        _check(self._lib.jr_execute_dispatches(self._ctx, native, len(jobs), repeats, _c.byref(gpu_ms), err,
                                               len(err)), err)
        host_ms = (time.perf_counter() - started) * 1000.0
        return Execution(host_ms=host_ms, gpu_ms=gpu_ms.value if gpu_ms.value > 0 else None,
                         dispatches=len(jobs) * repeats, repeats=repeats)

    # -- convenience ------------------------------------------------------
    def resident(self, data) -> Buffer:
        host = _f32(data).reshape(-1)
        buffer = self.alloc(host.size)
        self.upload(buffer, host)
        return buffer


class GemmPlan:
    """The per-shape GEMM plan ABI (native/jade_corex.h) as the reference's
    CorexPlan drives it (src/corex.rs:57-190)."""

    def __init__(self, m: int, n: int, k: int, device: int = 0, precision: int = 0, library: Optional[str] = None):
        self._lib = load(library)
        if self._lib.jade_corex_abi_version() != 1:
            raise JadeError(1, "GEMM plan ABI v1 required")
        ctx = _vp()
        err = _error_buffer()
        _check(self._lib.jade_corex_create(m, n, k, device, precision, _c.byref(ctx), err, len(err)), err)
        self._ctx = ctx.value
        self.m, self.n, self.k = m, n, k

    def device_info(self) -> str:
        out = _c.create_string_buffer(1024)
        err = _error_buffer()
        _check(self._lib.jade_corex_device_info(self._ctx, out, len(out), err, len(err)), err)
        return out.value.decode()

    def upload(self, a, b) -> None:
        a = _f32(a).reshape(-1)
        b = _f32(b).reshape(-1)
        err = _error_buffer()
        _check(self._lib.jade_corex_upload(self._ctx, a.ctypes.data_as(_vp), a.size, b.ctypes.data_as(_vp), b.size,
                                           err, len(err)), err)

    def run(self, iterations: int) -> float:
        ms = _c.c_double(0.0)
        err = _error_buffer()
        _check(self._lib.jade_corex_run(self._ctx, iterations, _c.byref(ms), err, len(err)), err)
        return ms.value

    def download(self) -> np.ndarray:
        out = np.empty(self.m * self.n, dtype=np.float32)
        err = _error_buffer()
        _check(self._lib.jade_corex_download(self._ctx, out.ctypes.data_as(_vp), out.size, err, len(err)), err)
        return out

    def close(self) -> None:
        if getattr(self, "_ctx", None):
            self._lib.jade_corex_destroy(self._ctx)
            self._ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
