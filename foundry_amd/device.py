"""HipDevice: the reference's ``Device`` trait (src/nn/primitive.rs:70-120)
implemented over the C-ABI, for the q4 ops.

Method names, argument meaning and error behaviour follow the trait and its
Metal implementation (src/metal/mod.rs:527-725): ``run`` returns a fresh
contiguous output; ``storage_to_bytes`` synchronises first; a device error is
sticky. Storage is device memory owned by one device (``HipStorage``); an
op given storage of another device fails with ``ForeignStorage``, as
src/metal/mod.rs:187-200 does.
"""
from __future__ import annotations

import ctypes
import warnings
from dataclasses import dataclass

import numpy as np

from . import _lib
from .primitive import (Binary, Cat, Copy, DType, IndexSelect, Matmul, QuantizedIndexSelect, QuantizedMatmul,
                        Reduce, SliceScatter, TensorError, ToDtype, Unary, check_shape, output)


class HipStorage:
    """One device allocation. Freed when the last reference drops, as the
    reference's Rc<Storage> is (src/nn/tensor.rs:49-53)."""

    __slots__ = ("device", "ptr", "nbytes", "views", "__weakref__")

    def __init__(self, device: "HipDevice", ptr: int, nbytes: int):
        self.device = device
        self.ptr = ptr
        self.nbytes = nbytes
        self.views = 0  # live Tensor views (Rc::get_mut's uniqueness test)

    def __del__(self):
        dev = self.device
        if dev is not None and dev._handle and self.ptr:
            lib = _lib.load()
            rc = lib.fh_free(dev._handle, ctypes.c_void_p(self.ptr))
            self.ptr = 0
            if rc != _lib.OK:
                # a destructor cannot raise: report the lost allocation
                warnings.warn(f"fh_free failed ({_lib.STATUS_NAMES.get(rc, rc)}): "
                              f"{lib.fh_last_error().decode(errors='replace')}", RuntimeWarning)


@dataclass(frozen=True)
class Layout:
    """src/nn/layout.rs: shape, strides in elements, storage offset."""

    shape: tuple
    strides: tuple
    offset: int = 0

    @staticmethod
    def contiguous(shape) -> "Layout":
        strides, acc = [], 1
        for d in reversed(shape):
            strides.append(acc)
            acc *= int(d)
        return Layout(tuple(int(d) for d in shape), tuple(reversed(strides)), 0)

    def is_contiguous(self) -> bool:
        """Layout::is_contiguous (src/nn/layout.rs:33-40): a dim of size one
        may have any stride."""
        want = Layout.contiguous(self.shape).strides
        return all(n == 1 or st == w for n, st, w in zip(self.shape, self.strides, want))

    @property
    def numel(self) -> int:
        n = 1
        for d in self.shape:
            n *= d
        return n

    def view(self) -> "_lib.View":
        return _lib.View.of(self.shape, self.strides, self.offset)

    def reshape(self, shape) -> "Layout":
        """Layout::reshape (src/nn/layout.rs:42-60)."""
        shape = check_shape(shape)
        if not self.is_contiguous():
            raise TensorError("ReshapeNonContiguous")
        if Layout.contiguous(shape).numel != self.numel:
            raise TensorError("NumelMismatch", f"{self.shape} -> {shape}")
        c = Layout.contiguous(shape)
        return Layout(c.shape, c.strides, self.offset)

    def permute(self, dims) -> "Layout":
        """Layout::permute (src/nn/layout.rs:62-92)."""
        dims = tuple(int(d) for d in dims)
        if sorted(dims) != list(range(len(self.shape))):
            raise TensorError("InvalidPermutation", f"{dims} of rank {len(self.shape)}")
        return Layout(tuple(self.shape[d] for d in dims), tuple(self.strides[d] for d in dims), self.offset)

    def narrow(self, dim: int, start: int, length: int) -> "Layout":
        """Layout::narrow (src/nn/layout.rs:94-130)."""
        if not 0 <= dim < len(self.shape):
            raise TensorError("DimOutOfRange", f"dim {dim}")
        if start < 0 or length < 0 or start + length > self.shape[dim]:
            raise TensorError("NarrowOutOfBounds", f"{start}+{length} of {self.shape[dim]}")
        shape = self.shape[:dim] + (int(length),) + self.shape[dim + 1:]
        return Layout(shape, self.strides, self.offset + start * self.strides[dim])

    def expand(self, shape) -> "Layout":
        """Layout::expand (src/nn/layout.rs:132-170): new leading dims and
        dims of size one take stride 0."""
        shape = check_shape(shape)
        lead = len(shape) - len(self.shape)
        if lead < 0:
            raise TensorError("ExpandIncompatible", f"{self.shape} -> {shape}")
        strides = []
        for d, n in enumerate(shape):
            s = d - lead
            if s < 0:
                strides.append(0)
            elif self.shape[s] == n:
                strides.append(self.strides[s])
            elif self.shape[s] == 1:
                strides.append(0)
            else:
                raise TensorError("ExpandIncompatible", f"{self.shape} -> {shape}")
        return Layout(shape, tuple(strides), self.offset)


@dataclass(frozen=True)
class Operand:
    """src/nn/tensor.rs:21-47: storage, layout and dtype of one op input."""

    storage: HipStorage
    layout: Layout
    dtype: DType

    def address(self) -> int:
        return self.storage.ptr + self.layout.offset * self.dtype.itemsize


class HipDevice:
    """One GPU, one HIP stream."""

    def __init__(self, ordinal: int = 0, profile_mode: int = _lib.PROFILE_OFF):
        lib = _lib.load()
        handle = ctypes.c_void_p()
        if profile_mode == _lib.PROFILE_OFF:
            _lib.check(lib.fh_device_create(ordinal, ctypes.byref(handle)))
        else:
            _lib.check(lib.fh_device_create_profiled(ordinal, profile_mode, ctypes.byref(handle)))
        self._handle = handle.value
        self.ordinal = ordinal

    @classmethod
    def profiled(cls, mode: int, ordinal: int = 0) -> "HipDevice":
        """MetalDevice::profiled (src/metal/mod.rs:142-149)."""
        return cls(ordinal, mode)

    def close(self) -> None:
        if self._handle:
            h, self._handle = self._handle, None
            _lib.check(_lib.load().fh_device_destroy(h))

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def handle(self) -> int:
        if not self._handle:
            raise _lib.HipError(_lib.ERR_INVALID_ARGUMENT, "device is closed")
        return self._handle

    # ---- Device trait ----
    def device_name(self) -> str:
        buf = ctypes.create_string_buffer(256)
        _lib.call("fh_device_name", self.handle, buf, len(buf))
        return buf.value.decode()

    def synchronize(self) -> None:
        _lib.call("fh_synchronize", self.handle)

    def max_memory_allocated(self):
        m = _lib.AllocatedMemory()
        _lib.call("fh_max_memory_allocated", self.handle, ctypes.byref(m))
        return {"bytes": m.bytes, "source": m.source.decode()}

    def reset_run_memory_peak(self) -> None:
        _lib.call("fh_reset_run_memory_peak", self.handle)

    def run_memory_peak(self):
        m = _lib.AllocatedMemory()
        _lib.call("fh_run_memory_peak", self.handle, ctypes.byref(m))
        return {"bytes": m.bytes, "source": m.source.decode()}

    def take_profile(self):
        """Counters since the previous call, or None when profiling is off."""
        p = _lib.Profile()
        rc = _lib.load().fh_take_profile(self.handle, ctypes.byref(p))
        if rc == _lib.ERR_UNSUPPORTED:
            return None
        _lib.check(rc)
        return {
            "dispatches": p.dispatches,
            "allocations": p.allocations,
            "allocated_bytes": p.allocated_bytes,
            "gpu_busy_ns": p.gpu_busy_ns,
        }

    def _alloc(self, nbytes: int, zero: bool) -> HipStorage:
        ptr = ctypes.c_void_p()
        _lib.call("fh_alloc", self.handle, nbytes, 1 if zero else 0, ctypes.byref(ptr))
        return HipStorage(self, ptr.value, nbytes)

    def storage_from_bytes(self, data) -> HipStorage:
        buf = np.ascontiguousarray(np.frombuffer(memoryview(data).cast("B"), dtype=np.uint8))
        st = self._alloc(buf.nbytes, zero=False)
        if buf.nbytes:
            _lib.call("fh_upload", self.handle, ctypes.c_void_p(st.ptr),
                      buf.ctypes.data_as(ctypes.c_void_p), buf.nbytes)
        return st

    def zeros(self, nbytes: int) -> HipStorage:
        return self._alloc(nbytes, zero=True)

    def empty(self, nbytes: int) -> HipStorage:
        """Uninitialised storage (an op's output)."""
        return self._alloc(nbytes, zero=False)

    def storage_to_bytes(self, operand: Operand) -> bytes:
        if not operand.layout.is_contiguous():
            raise TensorError("ToBytesNonContiguous")
        nbytes = operand.layout.numel * operand.dtype.itemsize
        out = np.empty(nbytes, dtype=np.uint8)
        if nbytes:
            _lib.call("fh_download", self.handle, out.ctypes.data_as(ctypes.c_void_p),
                      ctypes.c_void_p(operand.address()), nbytes)
        return out.tobytes()

    def _owns(self, operand: Operand) -> None:
        if operand.storage.device is not self:
            raise _lib.HipError(_lib.ERR_FOREIGN_STORAGE, "storage was produced by another device")

    def run(self, op, inputs, output_shape, dtype) -> HipStorage:
        """Runs an op into fresh contiguous storage (Device::run)."""
        for operand in inputs:
            self._owns(operand)
        shape, out_dtype = output(op, [(o.dtype, o.layout.shape) for o in inputs])
        if tuple(output_shape) != shape or DType(dtype) != out_dtype:
            raise TensorError("OperandCount", f"output {output_shape}/{dtype} does not match {shape}/{out_dtype}")
        numel = 1
        for d in shape:
            numel *= d
        out = self.empty(numel * out_dtype.itemsize)
        if isinstance(op, QuantizedMatmul):
            x, wq, s, b = inputs
            for w in (wq, s, b):
                if not w.layout.is_contiguous():
                    raise TensorError("MatmulIncompatible", "q4 weights must be contiguous")
            rows, k = x.layout.shape
            if x.dtype is not DType.BF16:
                raise _lib.HipError(_lib.ERR_DTYPE, "the q4 kernels take bf16 activations")
            x_ptr, x_ld = x.address(), x.layout.strides[0] if rows > 1 else max(k, x.layout.strides[0])
            if (k > 1 and x.layout.strides[1] != 1) or (rows > 1 and x.layout.strides[0] < k):
                # The operand rule of the reference's matmul (matmul_operand,
                # src/metal/mod.rs:384-401): rows the kernel cannot read in
                # place (a column stride, overlapping or broadcast rows) are
                # copied to a contiguous [rows, k] first.
                staged = self.empty(rows * k * 2)
                _lib.call("fh_copy_strided", self.handle, int(x.dtype), ctypes.c_void_p(x.storage.ptr),
                          ctypes.byref(x.layout.view()), ctypes.c_void_p(staged.ptr))
                x_ptr, x_ld = staged.ptr, k
            _lib.call("fh_q4_matmul", self.handle, ctypes.c_void_p(x_ptr), rows, k, x_ld,
                      ctypes.c_void_p(wq.address()), ctypes.c_void_p(s.address()),
                      ctypes.c_void_p(b.address()), shape[1], op.group, ctypes.c_void_p(out.ptr),
                      _lib.BF16 if out_dtype is DType.BF16 else _lib.F32)
            return out
        if isinstance(op, QuantizedIndexSelect):
            wq, s, b, ids = inputs
            for w in (wq, s, b, ids):
                if not w.layout.is_contiguous():
                    raise TensorError("IndexSelectIncompatible", "operands must be contiguous")
            rows = wq.layout.shape[0]
            _lib.call("fh_q4_embed", self.handle, ctypes.c_void_p(wq.address()),
                      ctypes.c_void_p(s.address()), ctypes.c_void_p(b.address()), rows, shape[1],
                      op.group, ctypes.c_void_p(ids.address()), shape[0], ctypes.c_void_p(out.ptr))
            return out
        self._run_standard(op, inputs, shape, out_dtype, out)
        return out

    def _run_standard(self, op, inputs, shape, dtype, out) -> None:
        """The reference's own Ops through the strided entry points
        (MetalDevice::run, src/metal/mod.rs:639-695)."""
        h, dst = self.handle, ctypes.c_void_p(out.ptr)

        def base(o):
            return ctypes.c_void_p(o.storage.ptr)

        def view(o):
            return ctypes.byref(o.layout.view())

        if isinstance(op, Unary):
            (x,) = inputs
            _lib.call("fh_unary", h, int(op.op), int(x.dtype), base(x), view(x), dst)
        elif isinstance(op, Binary):
            a, b = inputs
            _lib.call("fh_binary", h, int(op.op), int(a.dtype), base(a), view(a), base(b), view(b), dst)
        elif isinstance(op, Reduce):
            (x,) = inputs
            _lib.call("fh_reduce", h, int(op.op), int(x.dtype), base(x), view(x), op.dim, dst)
        elif isinstance(op, Matmul):
            a, b = inputs
            _lib.call("fh_matmul", h, int(a.dtype), base(a), view(a), base(b), view(b), dst)
        elif isinstance(op, Copy):
            (x,) = inputs
            _lib.call("fh_copy_strided", h, int(x.dtype), base(x), view(x), dst)
        elif isinstance(op, ToDtype):
            (x,) = inputs
            _lib.call("fh_to_dtype", h, int(x.dtype), base(x), view(x), int(dtype), dst)
        elif isinstance(op, IndexSelect):
            t, i = inputs
            _lib.call("fh_index_select", h, int(t.dtype), base(t), view(t), base(i), view(i), dst)
        elif isinstance(op, Cat):
            a, b = inputs
            _lib.call("fh_cat", h, int(a.dtype), op.dim, base(a), view(a), base(b), view(b), dst)
        else:
            raise _lib.HipError(_lib.ERR_INVALID_ARGUMENT, f"unsupported op {op!r}")

    def run_in_place(self, op, target: Operand, inputs) -> None:
        """Device::run_in_place (src/metal/mod.rs:697-725): SliceScatter of
        one source into a contiguous target this device owns."""
        if not isinstance(op, SliceScatter) or len(inputs) != 1:
            raise _lib.HipError(_lib.ERR_INVALID_ARGUMENT, f"run_in_place supports SliceScatter only, got {op!r}")
        self._owns(target)
        (src,) = inputs
        self._owns(src)
        _lib.call("fh_slice_scatter", self.handle, int(target.dtype), op.dim, op.start,
                  ctypes.c_void_p(target.storage.ptr), ctypes.byref(target.layout.view()),
                  ctypes.c_void_p(src.storage.ptr), ctypes.byref(src.layout.view()))

    # ---- batching and timing (CommandStream counterpart) ----
    def capture_begin(self) -> None:
        _lib.call("fh_capture_begin", self.handle)

    def capture_end(self) -> "HipGraph":
        g = ctypes.c_void_p()
        _lib.call("fh_capture_end", self.handle, ctypes.byref(g))
        return HipGraph(self, g.value)

    def timer_begin(self) -> None:
        _lib.call("fh_timer_begin", self.handle)

    def timer_end(self) -> float:
        ms = ctypes.c_double()
        _lib.call("fh_timer_end", self.handle, ctypes.byref(ms))
        return ms.value


class HipGraph:
    """A captured sequence of ops, replayed with ``launch``. The library
    keeps every allocation the graph's ops touched alive until the graph is
    destroyed, so storages dropped meanwhile cannot be reused under it."""

    def __init__(self, device: HipDevice, handle: int):
        self.device = device
        self._handle = handle

    def launch(self) -> None:
        _lib.call("fh_graph_launch", self.device.handle, ctypes.c_void_p(self._handle))

    def __del__(self):
        if self._handle:
            _lib.load().fh_graph_destroy(ctypes.c_void_p(self._handle))
            self._handle = None


def device_count() -> int:
    n = ctypes.c_int()
    _lib.call("fh_device_count", ctypes.byref(n))
    return n.value
