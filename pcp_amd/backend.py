"""HipGrpoBackend: the worker-backend face of the library for Python hosts.

Mirrors the interface the GRPO step reaches (src/backends/worker_backend.zig:7-62,
src/backends/iree.zig:38-497): ``init(backend, device_id)``, ``execute(artifact,
function_name, inputs_data, input_shapes, input_dtypes) -> list of output bytes``,
``executeFunction``, ``executeTrainingStep`` (function "main", which this library answers
with PCP_ERR_UNSUPPORTED: it holds the loss head, not the whole step), ``getBackendType``,
``deinit`` and ``asWorkerBackend``. Inputs are borrowed host byte buffers,
outputs are owned by the caller, errors raise PcpError with the library's status
(the Zig error union's analogue). The ``artifact`` argument is accepted for
signature compatibility and ignored: the compiled kernels live in the library,
not in a VMFB.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Callable, Sequence

import numpy as np

from . import _lib
from ._lib import Backend, DType, PcpError, check, lib


def _as_bytes_view(x) -> tuple[int, int, object]:
    """(address, nbytes, keepalive) of a bytes-like or numpy input."""
    if isinstance(x, np.ndarray):
        a = np.ascontiguousarray(x)
        return a.ctypes.data, a.nbytes, a
    mv = memoryview(x).cast("B")
    buf = (ctypes.c_char * len(mv)).from_buffer_copy(mv) if mv.readonly else (ctypes.c_char * len(mv)).from_buffer(mv)
    return ctypes.addressof(buf), len(mv), buf


class HipGrpoBackend:
    """~ IreeBackend for the GRPO loss head on one MI355X."""

    def __init__(self, handle: ctypes.c_void_p, backend: Backend, device_id: int):
        self._h = handle
        self.backend = backend
        self.device_id = device_id

    @classmethod
    def init(cls, backend: Backend | int = Backend.rocm, device_id: int = 0) -> "HipGrpoBackend":
        h = ctypes.c_void_p()
        check(lib().pcp_init(int(backend), int(device_id), ctypes.byref(h)))
        return cls(h, Backend(int(backend)), device_id)

    def deinit(self) -> None:
        if self._h:
            lib().pcp_destroy(self._h)
            self._h = None

    def getBackendType(self) -> Backend:
        return Backend(lib().pcp_get_backend_type(self._h))

    def execute(self, artifact: bytes | None, function_name: str, inputs_data: Sequence,
                input_shapes: Sequence[Sequence[int]], input_dtypes: Sequence[DType | int] | None) -> list[bytes]:
        return execute_raw(self._h, function_name, inputs_data, input_shapes, input_dtypes)

    def executeFunction(self, artifact, function_name, inputs_data, input_shapes, input_dtypes=None):
        return self.execute(artifact, function_name, inputs_data, input_shapes, input_dtypes)

    def executeTrainingStep(self, artifact, inputs_data, input_shapes, input_dtypes=None):
        # iree.zig:463-486 runs the VMFB's "main", the whole training step. The library
        # holds only its loss head, so this raises PcpError (PCP_ERR_UNSUPPORTED) with a
        # message naming the split: forward to logits, "grpo_loss_fwd_bwd", backward.
        return self.execute(artifact, "main", inputs_data, input_shapes, input_dtypes)

    def asWorkerBackend(self) -> "WorkerBackend":
        return WorkerBackend(ptr=self, vtable=WorkerBackend.VTable(
            executeTrainingStep=lambda p, art, d, s, t: p.executeTrainingStep(art, d, s, t),
            executeFunction=lambda p, art, fn, d, s, t: p.executeFunction(art, fn, d, s, t),
            getBackendType=lambda p: p.getBackendType(),
            deinit=lambda p: p.deinit()))

    def __del__(self):
        try:
            self.deinit()
        except Exception:
            pass


@dataclass
class WorkerBackend:
    """~ WorkerBackend {ptr, vtable} (worker_backend.zig:7-62)."""

    @dataclass
    class VTable:
        executeTrainingStep: Callable
        executeFunction: Callable
        getBackendType: Callable
        deinit: Callable

    ptr: object
    vtable: "WorkerBackend.VTable"

    def executeTrainingStep(self, artifact, data, shapes, dtypes=None):
        return self.vtable.executeTrainingStep(self.ptr, artifact, data, shapes, dtypes)

    def executeFunction(self, artifact, function_name, data, shapes, dtypes=None):
        return self.vtable.executeFunction(self.ptr, artifact, function_name, data, shapes, dtypes)

    def getBackendType(self):
        return self.vtable.getBackendType(self.ptr)

    def deinit(self):
        self.vtable.deinit(self.ptr)


def execute_raw(handle, function_name: str, inputs_data: Sequence, input_shapes: Sequence[Sequence[int]],
                input_dtypes: Sequence[DType | int] | None) -> list[bytes]:
    """pcp_execute over host buffers; ``handle`` may be None to exercise argument
    checking without a device (the call then fails with PCP_ERR_INVALID_ARG after
    the checks pass)."""
    m = marshal_inputs(inputs_data, input_shapes, input_dtypes)
    n_out = ctypes.c_int(0)
    out_data = ctypes.POINTER(ctypes.c_void_p)()
    out_nbytes = ctypes.POINTER(ctypes.c_size_t)()
    rc = lib().pcp_execute(handle, function_name.encode(), m.n, m.ptrs, m.nbytes, m.shapes, m.ranks, m.dtypes,
                           ctypes.byref(n_out), ctypes.byref(out_data), ctypes.byref(out_nbytes))
    check(rc, handle)
    try:
        return [ctypes.string_at(out_data[i], out_nbytes[i]) for i in range(n_out.value)]
    finally:
        lib().pcp_free(handle, n_out.value, out_data, out_nbytes)


@dataclass
class MarshalledInputs:
    """pcp_execute's input arrays over borrowed host buffers (``keep`` holds them alive)."""
    n: int
    ptrs: object
    nbytes: object
    shapes: object
    ranks: object
    dtypes: object
    keep: list


def marshal_inputs(inputs_data: Sequence, input_shapes: Sequence[Sequence[int]],
                   input_dtypes: Sequence[DType | int] | None) -> MarshalledInputs:
    n = len(inputs_data)
    if len(input_shapes) != n or (input_dtypes is not None and len(input_dtypes) != n):
        raise PcpError(-8, "inputs, shapes and dtypes differ in length")
    keep = []
    ptrs = (ctypes.c_void_p * max(n, 1))()
    nbytes = (ctypes.c_size_t * max(n, 1))()
    shapes = (ctypes.POINTER(ctypes.c_int64) * max(n, 1))()
    ranks = (ctypes.c_int * max(n, 1))()
    for i, (d, s) in enumerate(zip(inputs_data, input_shapes)):
        addr, nb, k = _as_bytes_view(d)
        keep.append(k)
        ptrs[i] = addr
        nbytes[i] = nb
        arr = (ctypes.c_int64 * max(len(s), 1))(*[int(v) for v in s])
        keep.append(arr)
        shapes[i] = ctypes.cast(arr, ctypes.POINTER(ctypes.c_int64))
        ranks[i] = len(s)
    dts = None
    if input_dtypes is not None:
        dts = (ctypes.c_int * max(n, 1))(*[int(t) for t in input_dtypes])
    return MarshalledInputs(n, ptrs, nbytes, shapes, ranks, dts, keep)
