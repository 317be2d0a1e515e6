"""The device, its buffers and typed tensors over libh3hip.so (mirror of engine/h3-core/src/device.rs and dtype.rs).

A ``Device`` owns a library context (``h3s_open`` / ``h3s_open_gpu``) or wraps an existing HIP stream
(``h3s_create``: PyTorch's current stream, so the kernels are ordered with PyTorch's work and PyTorch tensors can be
used in place). ``Buf`` is device memory from ``h3s_alloc``, freed when dropped (device.rs:198-203). ``Tensor`` is a
dtype and a row-major shape over a ``Buf`` or over a PyTorch tensor's storage.
"""
from __future__ import annotations

import enum
from typing import Sequence

import numpy as np

from . import api as _api


class Error(Exception):
    """A failed library call, with the library's message (engine/h3-core/src/lib.rs's Error)."""


class DType(enum.Enum):
    """engine/h3-core/src/dtype.rs:5-15."""

    F32 = "F32"
    F16 = "F16"
    BF16 = "BF16"
    I8 = "I8"
    U8 = "U8"
    I32 = "I32"
    I64 = "I64"
    F64 = "F64"

    def size(self) -> int:
        return {"I8": 1, "U8": 1, "F16": 2, "BF16": 2, "F32": 4, "I32": 4, "I64": 8, "F64": 8}[self.value]

    def kernel_code(self) -> int:
        """The library's code for a floating-point type (dtype.rs:43-50)."""
        codes = {"F32": _api.F32, "F16": _api.F16, "BF16": _api.BF16}
        if self.value not in codes:
            raise Error(f"{self} is not a floating-point tensor type")
        return codes[self.value]

    def numpy(self):
        """The numpy type that carries the bits (16-bit floats as uint16 bit patterns)."""
        return {"F32": np.float32, "F16": np.uint16, "BF16": np.uint16, "I8": np.int8, "U8": np.uint8,
                "I32": np.int32, "I64": np.int64, "F64": np.float64}[self.value]


class Device:
    """A library context on one GPU (device.rs:23-75)."""

    def __init__(self, ctx: int, api: _api.Api, owns: bool = True, keep=None):
        if not ctx:
            raise Error(api.error())
        self.ctx = ctx
        self.api = api
        self._owns = owns
        self._keep = keep

    @staticmethod
    def open(index: int | None = None) -> "Device":
        a = _api.load()
        return Device(a.open() if index is None else a.open_gpu(index), a)

    @staticmethod
    def from_stream(hip_stream: int, keep=None) -> "Device":
        """A context on an existing hipStream_t, e.g. ``torch.cuda.current_stream().cuda_stream``."""
        a = _api.load()
        return Device(a.create(hip_stream), a, keep=keep)

    @staticmethod
    def from_torch() -> "Device":
        import torch

        s = torch.cuda.current_stream()
        return Device.from_stream(s.cuda_stream, keep=s)

    def check(self, rc: int) -> None:
        """rc -1 -> Error with the library's message (device.rs:132-138)."""
        if rc != 0:
            raise Error(self.api.error())

    def name(self) -> str:
        return (self.api.device_name(self.ctx) or b"").decode()

    def stream(self) -> int:
        return self.api.stream(self.ctx) or 0

    def wait(self) -> None:
        self.check(self.api.wait(self.ctx))

    def mem_used(self) -> int:
        return int(self.api.mem_used(self.ctx))

    def mem_cap(self) -> int:
        return int(self.api.mem_cap(self.ctx))

    def close(self) -> None:
        if self.ctx and self._owns:
            self.api.destroy(self.ctx)
        self.ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Buf:
    """Device memory from h3s_alloc, freed on drop (device.rs:185-203)."""

    def __init__(self, dev: Device, nbytes: int):
        p = dev.api.alloc(dev.ctx, nbytes)
        if not p:
            raise Error(dev.api.error())
        self.dev, self.nbytes, self._ptr = dev, nbytes, p

    def ptr(self) -> int:
        return self._ptr

    def __len__(self) -> int:
        return self.nbytes

    def write(self, data: bytes | np.ndarray, offset: int = 0) -> None:
        a = np.ascontiguousarray(data).view(np.uint8)
        if offset + a.nbytes > self.nbytes:
            raise Error(f"write of {a.nbytes} bytes at {offset} into a buffer of {self.nbytes}")
        self.dev.check(self.dev.api.write(self.dev.ctx, self._ptr + offset, a.ctypes.data, a.nbytes))

    def read(self, nbytes: int | None = None, offset: int = 0) -> np.ndarray:
        n = self.nbytes - offset if nbytes is None else nbytes
        out = np.empty(n, dtype=np.uint8)
        self.dev.check(self.dev.api.read(self.dev.ctx, out.ctypes.data, self._ptr + offset, n))
        return out

    def free(self) -> None:
        if self._ptr:
            self.dev.api.free(self.dev.ctx, self._ptr)
            self._ptr = 0

    def __del__(self):
        try:
            if self._ptr and self.dev.ctx:
                self.free()
        except Exception:
            pass


class Tensor:
    """A dtype and a row-major shape over device memory (device.rs:205-320)."""

    def __init__(self, dtype: DType, shape: Sequence[int], ptr: int, owner, dev: Device | None):
        self.dtype, self.shape, self._ptr, self._owner, self.dev = dtype, list(shape), ptr, owner, dev

    def elements(self) -> int:
        n = 1
        for s in self.shape:
            n *= int(s)
        return n

    def nbytes(self) -> int:
        return self.elements() * self.dtype.size()

    def ptr(self) -> int:
        return self._ptr

    @staticmethod
    def new(dev: Device, dtype: DType, shape: Sequence[int]) -> "Tensor":
        n = 1
        for s in shape:
            n *= int(s)
        b = Buf(dev, max(1, n * dtype.size()))
        return Tensor(dtype, shape, b.ptr(), b, dev)

    @staticmethod
    def from_numpy(dev: Device, dtype: DType, shape: Sequence[int], data: np.ndarray) -> "Tensor":
        t = Tensor.new(dev, dtype, shape)
        a = np.ascontiguousarray(data)
        if a.nbytes != t.nbytes():
            raise Error(f"{a.nbytes} bytes for a {dtype} tensor of shape {list(shape)}")
        t._owner.write(a)
        return t

    @staticmethod
    def from_torch(t, dtype: DType | None = None, dev: Device | None = None) -> "Tensor":
        """A view of a contiguous PyTorch tensor's storage (no copy); the tensor is kept alive."""
        import torch

        if not t.is_contiguous():
            raise Error("from_torch: the tensor must be contiguous")
        m = {torch.float32: DType.F32, torch.float16: DType.F16, torch.bfloat16: DType.BF16, torch.int8: DType.I8,
             torch.uint8: DType.U8, torch.int32: DType.I32, torch.int64: DType.I64, torch.float64: DType.F64}
        return Tensor(dtype or m[t.dtype], list(t.shape), t.data_ptr(), t, dev)

    def to_numpy(self) -> np.ndarray:
        """The tensor's bits, read back (waits)."""
        if isinstance(self._owner, Buf):
            raw = self._owner.read(self.nbytes(), self._ptr - self._owner.ptr())
        else:
            import torch

            raw = self._owner.detach().contiguous().reshape(-1).view(torch.uint8).cpu().numpy()[: self.nbytes()]
        return raw.view(self.dtype.numpy()).reshape(self.shape)

    def to_f32(self) -> np.ndarray:
        a = self.to_numpy()
        if self.dtype == DType.BF16:
            return (a.astype(np.uint32) << 16).view(np.float32)
        if self.dtype == DType.F16:
            return a.view(np.float16).astype(np.float32)
        return a.astype(np.float32)
