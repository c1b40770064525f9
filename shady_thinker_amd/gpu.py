"""GpuContext: the reference's device runtime (src/gpu.rs:7-297) over st_context.

Buffers are torch device tensors (torch is plumbing here: device memory and
streams). Every kernel call runs on torch's current stream of the context's
device, so torch ops and HIP kernels stay ordered without extra syncs.
"""
from __future__ import annotations

import contextlib
import ctypes

import numpy as np

from ._lib import TUNE, call, lib


def ptr(t) -> int | None:
    """Device address of a tensor (None passes NULL)."""
    return None if t is None else t.data_ptr()


class GpuContext:
    """Mirror of `GpuContext` (src/gpu.rs:7-14).

    new() -> st_context_create (src/gpu.rs:17-78); create_storage_buffer /
    upload_buffer / read_buffer / write_buffer / copy_buffer / flush keep the
    reference's names and meaning (src/gpu.rs:80-282). dispatch() has no
    counterpart: kernels are called by name through the C ABI
    (shady_thinker_amd.model).
    """

    def __init__(self, device: int = 0):
        import torch

        self.torch = torch
        self.device = torch.device("cuda", device)
        handle = ctypes.c_void_p()
        call("st_context_create", device, ctypes.byref(handle))
        self.handle = handle
        self._stream = None
        self.sync_stream()

    # -- stream -------------------------------------------------------------
    def sync_stream(self) -> None:
        """Follow torch's current stream (called before every kernel)."""
        s = self.torch.cuda.current_stream(self.device).cuda_stream
        if s != self._stream:
            call("st_context_set_stream", self.handle, s)
            self._stream = s

    # -- kernel-path overrides (st_context_set_tune) -------------------------
    def set_tune(self, knob: str, value: int) -> None:
        """Force a kernel-path setting of this context (-1 = automatic), e.g.
        set_tune("DECODE_KERNEL", 1) for the streaming decode kernel."""
        call("st_context_set_tune", self.handle, TUNE[knob], int(value))

    def get_tune(self, knob: str) -> int:
        v = ctypes.c_int()
        call("st_context_get_tune", self.handle, TUNE[knob], ctypes.byref(v))
        return v.value

    @contextlib.contextmanager
    def tuning(self, **knobs):
        """with gpu.tuning(NO_CHUNK=1, ...): the settings hold inside the
        block and the previous values come back after it."""
        old = {k: self.get_tune(k) for k in knobs}
        try:
            for k, v in knobs.items():
                self.set_tune(k, v)
            yield self
        finally:
            for k, v in old.items():
                self.set_tune(k, v)

    def reserve_workspace(self, nbytes: int) -> None:
        call("st_context_reserve_workspace", self.handle, nbytes)

    # -- buffers (src/gpu.rs:80-117) -----------------------------------------
    def create_storage_buffer(self, label: str, size: int):
        aligned = (size + 3) & ~3  # src/gpu.rs:86
        return self.torch.zeros(max(aligned, 4), dtype=self.torch.uint8, device=self.device)

    def upload_buffer(self, label: str, data):
        """Host bytes/array -> new device buffer; returns when uploaded."""
        arr = np.ascontiguousarray(data)
        buf = self.create_storage_buffer(label, arr.nbytes)
        self.sync_stream()
        call("st_upload", self.handle, buf.data_ptr(), arr.ctypes.data, arr.nbytes)
        return buf

    def upload_array(self, data, dtype):
        """Host array -> device tensor of a torch dtype, same shape."""
        arr = np.ascontiguousarray(data)
        t = self.torch.empty(arr.shape, dtype=dtype, device=self.device)
        if t.numel() * t.element_size() != arr.nbytes:
            raise ValueError("upload_array: byte size mismatch")
        self.sync_stream()
        call("st_upload", self.handle, t.data_ptr(), arr.ctypes.data, arr.nbytes)
        return t

    def write_buffer(self, buffer, offset: int, data) -> None:
        arr = np.ascontiguousarray(data)
        self.sync_stream()
        call("st_write", self.handle, buffer.data_ptr(), offset, arr.ctypes.data, arr.nbytes)

    def read_buffer(self, buffer, size: int | None = None) -> bytes:
        """Flush, then copy `size` bytes back (src/gpu.rs:252-276)."""
        n = buffer.numel() * buffer.element_size() if size is None else size
        out = np.empty(n, np.uint8)
        self.sync_stream()
        call("st_read", self.handle, buffer.data_ptr(), out.ctypes.data, n)
        return out.tobytes()

    def copy_buffer(self, src, dst, size: int) -> None:
        self.sync_stream()
        call("st_copy", self.handle, dst.data_ptr(), src.data_ptr(), size)

    def flush(self) -> None:
        self.sync_stream()
        call("st_flush", self.handle)

    def close(self) -> None:
        if self.handle:
            lib().st_context_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
