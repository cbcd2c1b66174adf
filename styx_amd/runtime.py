"""Python mirror of the vk-backend surface (crates/vk-backend/src/lib.rs) over
libstyx_hip.so: Gpu, Buffer, Kernel, Batch, plus numpy helpers and thin
wrappers of the hot-path op entry points.  Device memory is owned by the
library; numpy arrays cross only by copy."""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib as L


class Gpu:
    """Gpu::new (lib.rs:356).  Closes with close() or as a context manager."""

    def __init__(self, device: int = 0):
        self.lib = L.load()
        h = C.c_void_p()
        L.check(self.lib.styx_gpu_new(device, C.byref(h)))
        self.h = h

    @property
    def name(self) -> str:
        return self.lib.styx_gpu_name(self.h).decode()

    @property
    def hbm_bytes(self) -> int:
        return int(self.lib.styx_gpu_hbm_bytes(self.h))

    def sync(self) -> None:
        L.check(self.lib.styx_gpu_sync(self.h))

    def close(self) -> None:
        if self.h:
            self.lib.styx_gpu_free(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    # ------------------------------------------------------------ memory --
    def buffer(self, nbytes: int, kind: int = L.BUF_DEVICE) -> "Buffer":
        return Buffer(self, nbytes, kind)

    def from_numpy(self, a: np.ndarray, kind: int = L.BUF_DEVICE) -> "Buffer":
        a = np.ascontiguousarray(a)
        b = Buffer(self, max(a.nbytes, 16), kind)
        if a.nbytes:
            b.upload(a)
        return b

    def zeros(self, nbytes: int) -> "Buffer":
        b = Buffer(self, max(nbytes, 16))
        b.upload(np.zeros(max(nbytes, 16), np.uint8))
        return b


class Buffer:
    """create_buffer / create_buffer_host (lib.rs:568, 756)."""

    def __init__(self, gpu: Gpu, nbytes: int, kind: int = L.BUF_DEVICE):
        self.gpu, self.lib = gpu, gpu.lib
        h = C.c_void_p()
        L.check(self.lib.styx_buf_new(gpu.h, int(nbytes), kind, C.byref(h)))
        self.h, self.nbytes, self.kind = h, int(nbytes), kind

    @property
    def ptr(self) -> int:
        return int(self.lib.styx_buf_device_ptr(self.h))

    def upload(self, a: np.ndarray, off: int = 0) -> None:
        a = np.ascontiguousarray(a)
        L.check(self.lib.styx_upload(self.gpu.h, self.h, off, a.ctypes.data, a.nbytes))

    def download(self, dtype=np.uint8, count: int | None = None, off: int = 0) -> np.ndarray:
        dtype = np.dtype(dtype)
        if count is None:
            count = (self.nbytes - off) // dtype.itemsize
        out = np.empty(count, dtype)
        L.check(self.lib.styx_download(self.gpu.h, self.h, off, out.ctypes.data, out.nbytes))
        return out

    def copy_to(self, dst: "Buffer", soff: int, doff: int, n: int) -> None:
        L.check(self.lib.styx_copy_region(self.gpu.h, self.h, soff, dst.h, doff, n))

    def free(self) -> None:
        if self.h:
            self.lib.styx_buf_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Kernel:
    """create_pipeline (lib.rs:1222) by reference pipeline name."""

    def __init__(self, gpu: Gpu, name: str, spec: list[tuple[int, int]] = ()):
        self.gpu, self.lib, self.name = gpu, gpu.lib, name
        arr = (C.c_uint32 * (2 * len(spec) or 1))(*[v for p in spec for v in p])
        h = C.c_void_p()
        L.check(self.lib.styx_kernel_get(gpu.h, name.encode(), arr, len(spec), C.byref(h)))
        self.h = h

    def free(self):
        if self.h:
            self.lib.styx_kernel_free(self.h)
            self.h = None


def _bindings(binds):
    arr = (L.Binding * len(binds))()
    for i, b in enumerate(binds):
        buf, off, rng = (b if isinstance(b, tuple) else (b, 0, 2**64 - 1))
        arr[i].buf, arr[i].offset, arr[i].range = buf.h, off, rng
    return arr


def dispatch_sync(gpu: "Gpu", k: "Kernel", binds, push: bytes, groups):
    """Gpu::dispatch_sync (lib.rs:1415-1515): one dispatch, waited for."""
    pb = C.create_string_buffer(push, len(push))
    gx, gy, gz = (tuple(groups) + (1, 1))[:3]
    L.check(gpu.lib.styx_dispatch_sync(gpu.h, k.h, _bindings(binds), len(binds), pb, len(push),
                                       gx, gy, gz))


class Timeline:
    """Timeline semaphore (Gpu::create_timeline_semaphore, lib.rs:700-713)."""

    def __init__(self, gpu: Gpu):
        self.gpu, self.lib = gpu, gpu.lib
        h = C.c_void_p()
        L.check(self.lib.styx_timeline_new(gpu.h, C.byref(h)))
        self.h = h

    def value(self) -> int:
        v = C.c_uint64()
        L.check(self.lib.styx_timeline_value(self.h, C.byref(v)))
        return v.value

    def free(self):
        if self.h:
            self.lib.styx_timeline_free(self.h)
            self.h = None


class Batch:
    """Batch (lib.rs:44-333): begin, dispatch*, submit; an async batch
    (Gpu::create_async_batch) also submit_async / wait_idle."""

    def __init__(self, gpu: Gpu, is_async: bool = False):
        self.gpu, self.lib = gpu, gpu.lib
        h = C.c_void_p()
        new = self.lib.styx_batch_new_async if is_async else self.lib.styx_batch_new
        L.check(new(gpu.h, C.byref(h)))
        self.h = h

    def begin(self):
        L.check(self.lib.styx_batch_begin(self.h))

    def dispatch(self, k: Kernel, binds, push: bytes, groups, barrier: bool = True):
        arr = _bindings(binds)
        pb = C.create_string_buffer(push, len(push))
        gx, gy, gz = (tuple(groups) + (1, 1))[:3]
        L.check(self.lib.styx_batch_dispatch(self.h, k.h, arr, len(binds), pb, len(push),
                                             gx, gy, gz, int(barrier)))

    def submit(self):
        L.check(self.lib.styx_batch_submit(self.h))

    def submit_async(self, t: Timeline, value: int):
        L.check(self.lib.styx_batch_submit_async(self.h, t.h, value))

    def wait_idle(self):
        L.check(self.lib.styx_batch_wait_idle(self.h))

    def submit_wait_sem(self, t: Timeline, value: int):
        L.check(self.lib.styx_batch_submit_wait_sem(self.h, t.h, value))

    def free(self):
        if self.h:
            self.lib.styx_batch_free(self.h)
            self.h = None


def split_nblocks(type_: int, rows: int, cols: int) -> int:
    return rows * (cols // L.BLOCK[type_][0])


def nbytes_of(type_: int, n: int) -> int:
    el, by = L.BLOCK[type_]
    return n // el * by


def to_split(gpu: Gpu, type_: int, gguf: Buffer, rows: int, cols: int, nmat: int = 1) -> Buffer:
    out = gpu.buffer(gguf.nbytes)
    L.check(gpu.lib.styx_op_to_split(gpu.h, type_, gguf.ptr, out.ptr,
                                     split_nblocks(type_, rows, cols), nmat))
    return out


def from_split(gpu: Gpu, type_: int, split: Buffer, rows: int, cols: int, nmat: int = 1) -> Buffer:
    out = gpu.buffer(split.nbytes)
    L.check(gpu.lib.styx_op_from_split(gpu.h, type_, split.ptr, out.ptr,
                                       split_nblocks(type_, rows, cols), nmat))
    return out
