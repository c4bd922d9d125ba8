"""Device memory, copies, streams, events and graph capture over the HIP runtime.

A thin ctypes layer over libamdhip64 -- the runtime libpbsample.so itself
links -- so that the sampler's Python host side needs no other framework.
Only what the sampler's callers use is bound: device and pinned host
buffers, synchronous and stream-ordered copies, streams, timing events and
stream capture into HIP graphs.

The runtime is opened by its SONAME (libamdhip64.so.7).  A process that
already mapped a HIP runtime (for instance one bundled with another
framework) gets that same copy, so device pointers and stream handles stay
valid across both; otherwise the dynamic loader finds /opt/rocm's.
"""
from __future__ import annotations

import ctypes

import numpy as np

_vp = ctypes.c_void_p
_sz = ctypes.c_size_t
_int = ctypes.c_int
_uint = ctypes.c_uint

H2D, D2H, D2D = 1, 2, 3  # hipMemcpyKind
_CAPTURE_MODE_THREAD_LOCAL = 1  # hipStreamCaptureModeThreadLocal

_SIGS = {
    "hipGetErrorString": (ctypes.c_char_p, [_int]),
    "hipGetDeviceCount": (_int, [ctypes.POINTER(_int)]),
    "hipSetDevice": (_int, [_int]),
    "hipGetDevice": (_int, [ctypes.POINTER(_int)]),
    "hipDeviceSynchronize": (_int, []),
    "hipMalloc": (_int, [ctypes.POINTER(_vp), _sz]),
    "hipFree": (_int, [_vp]),
    "hipHostMalloc": (_int, [ctypes.POINTER(_vp), _sz, _uint]),
    "hipHostFree": (_int, [_vp]),
    "hipMemcpy": (_int, [_vp, _vp, _sz, _int]),
    "hipMemcpyAsync": (_int, [_vp, _vp, _sz, _int, _vp]),
    "hipStreamCreate": (_int, [ctypes.POINTER(_vp)]),
    "hipStreamDestroy": (_int, [_vp]),
    "hipStreamSynchronize": (_int, [_vp]),
    "hipEventCreate": (_int, [ctypes.POINTER(_vp)]),
    "hipEventDestroy": (_int, [_vp]),
    "hipEventRecord": (_int, [_vp, _vp]),
    "hipEventSynchronize": (_int, [_vp]),
    "hipEventElapsedTime": (_int, [ctypes.POINTER(ctypes.c_float), _vp, _vp]),
    "hipStreamBeginCapture": (_int, [_vp, _int]),
    "hipStreamEndCapture": (_int, [_vp, ctypes.POINTER(_vp)]),
    "hipGraphInstantiate": (_int, [ctypes.POINTER(_vp), _vp, _vp, ctypes.c_char_p, _sz]),
    "hipGraphLaunch": (_int, [_vp, _vp]),
    "hipGraphExecDestroy": (_int, [_vp]),
    "hipGraphDestroy": (_int, [_vp]),
}

_rt = None


class HipError(RuntimeError):
    def __init__(self, call: str, code: int):
        msg = runtime().hipGetErrorString(code)
        super().__init__(f"{call} failed: {code} ({msg.decode() if msg else '?'})")
        self.code = code


def runtime() -> ctypes.CDLL:
    global _rt
    if _rt is None:
        rt = ctypes.CDLL("libamdhip64.so.7")
        for name, (res, args) in _SIGS.items():
            fn = getattr(rt, name)
            fn.restype = res
            fn.argtypes = args
        _rt = rt
    return _rt


def _ok(call: str, code: int) -> None:
    if code != 0:
        raise HipError(call, code)


def device_count() -> int:
    n = _int(0)
    code = runtime().hipGetDeviceCount(ctypes.byref(n))
    return n.value if code == 0 else 0


def set_device(device: int) -> None:
    _ok("hipSetDevice", runtime().hipSetDevice(device))


def synchronize() -> None:
    _ok("hipDeviceSynchronize", runtime().hipDeviceSynchronize())


def stream_handle(stream) -> int | None:
    """A hipStream_t from None (the null stream), an int, a Stream, or any
    object carrying a `cuda_stream` handle."""
    if stream is None:
        return None
    if isinstance(stream, int):
        return stream
    if isinstance(stream, Stream):
        return stream.handle
    return int(stream.cuda_stream)


class Stream:
    """A blocking HIP stream at the default priority."""

    def __init__(self):
        h = _vp()
        _ok("hipStreamCreate", runtime().hipStreamCreate(ctypes.byref(h)))
        self.handle = h.value

    def synchronize(self) -> None:
        _ok("hipStreamSynchronize", runtime().hipStreamSynchronize(self.handle))

    def close(self) -> None:
        if self.handle:
            runtime().hipStreamDestroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Event:
    def __init__(self):
        h = _vp()
        _ok("hipEventCreate", runtime().hipEventCreate(ctypes.byref(h)))
        self.handle = h.value

    def record(self, stream=None) -> None:
        _ok("hipEventRecord", runtime().hipEventRecord(self.handle, stream_handle(stream)))

    def synchronize(self) -> None:
        _ok("hipEventSynchronize", runtime().hipEventSynchronize(self.handle))

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float(0.0)
        _ok("hipEventElapsedTime",
            runtime().hipEventElapsedTime(ctypes.byref(ms), self.handle, end.handle))
        return float(ms.value)

    def __del__(self):
        try:
            if self.handle:
                runtime().hipEventDestroy(self.handle)
        except Exception:
            pass


class DeviceArray:
    """A C-contiguous device buffer with a numpy shape and dtype."""

    def __init__(self, shape, dtype=np.uint32):
        self.shape = tuple(int(x) for x in (shape if np.iterable(shape) else (shape,)))
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        p = _vp()
        if self.nbytes:
            _ok("hipMalloc", runtime().hipMalloc(ctypes.byref(p), self.nbytes))
        self._ptr = p.value or 0

    @classmethod
    def from_numpy(cls, a) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = cls(a.shape, a.dtype)
        d.upload(a)
        return d

    @classmethod
    def zeros(cls, shape, dtype=np.uint32) -> "DeviceArray":
        return cls.from_numpy(np.zeros(shape, dtype))

    def data_ptr(self) -> int:
        return self._ptr

    def numel(self) -> int:
        return self.nbytes // self.dtype.itemsize

    def upload(self, a) -> None:
        """Synchronous host -> device copy of a same-sized array (any dtype)."""
        a = np.ascontiguousarray(a)
        if a.nbytes != self.nbytes:
            raise ValueError(f"upload of {a.nbytes} bytes into a {self.nbytes}-byte buffer")
        if self.nbytes:
            synchronize()
            _ok("hipMemcpy", runtime().hipMemcpy(self._ptr, a.ctypes.data, self.nbytes, H2D))

    def numpy(self, dtype=None) -> np.ndarray:
        """Waits for the device, then copies the buffer to a new host array."""
        out = np.empty(self.shape, self.dtype)
        if self.nbytes:
            synchronize()
            _ok("hipMemcpy", runtime().hipMemcpy(out.ctypes.data, self._ptr, self.nbytes, D2H))
        return out if dtype is None else out.view(dtype)

    def copy_from(self, other: "DeviceArray", stream=None) -> None:
        """Stream-ordered device -> device copy of the whole buffer."""
        if other.nbytes != self.nbytes:
            raise ValueError("device copy between buffers of different sizes")
        if self.nbytes:
            _ok("hipMemcpyAsync", runtime().hipMemcpyAsync(self._ptr, other._ptr, self.nbytes,
                                                            D2D, stream_handle(stream)))

    def free(self) -> None:
        if self._ptr:
            runtime().hipFree(self._ptr)
            self._ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class PinnedArray:
    """Page-locked host memory viewed as a numpy array (for stream-ordered copies)."""

    def __init__(self, shape, dtype=np.uint32):
        self.dtype = np.dtype(dtype)
        shape = tuple(int(x) for x in (shape if np.iterable(shape) else (shape,)))
        self.nbytes = int(np.prod(shape, dtype=np.int64)) * self.dtype.itemsize
        p = _vp()
        _ok("hipHostMalloc", runtime().hipHostMalloc(ctypes.byref(p), max(self.nbytes, 1), 0))
        self._ptr = p.value
        buf = (ctypes.c_char * max(self.nbytes, 1)).from_address(self._ptr)
        self.array = np.frombuffer(buf, dtype=self.dtype, count=self.nbytes // self.dtype.itemsize
                                   ).reshape(shape)

    def data_ptr(self) -> int:
        return self._ptr

    def free(self) -> None:
        if self._ptr:
            self.array = None
            runtime().hipHostFree(self._ptr)
            self._ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def copy_async(dst, src, nbytes: int, kind: int, stream=None) -> None:
    """hipMemcpyAsync between raw pointers (or objects with data_ptr())."""
    d = dst if isinstance(dst, int) else dst.data_ptr()
    s = src if isinstance(src, int) else src.data_ptr()
    _ok("hipMemcpyAsync", runtime().hipMemcpyAsync(d, s, nbytes, kind, stream_handle(stream)))


class Graph:
    """Work enqueued on `stream` between begin() and end(), replayable with
    launch().  Capture is thread-local: other threads' HIP calls are not
    affected."""

    def __init__(self, stream: Stream):
        self.stream = stream
        self._graph = None
        self._exec = None

    def begin(self) -> None:
        _ok("hipStreamBeginCapture",
            runtime().hipStreamBeginCapture(self.stream.handle, _CAPTURE_MODE_THREAD_LOCAL))

    def end(self) -> None:
        g = _vp()
        _ok("hipStreamEndCapture", runtime().hipStreamEndCapture(self.stream.handle,
                                                                 ctypes.byref(g)))
        self._graph = g.value
        e = _vp()
        _ok("hipGraphInstantiate",
            runtime().hipGraphInstantiate(ctypes.byref(e), self._graph, None, None, 0))
        self._exec = e.value

    def launch(self) -> None:
        _ok("hipGraphLaunch", runtime().hipGraphLaunch(self._exec, self.stream.handle))

    def close(self) -> None:
        if self._exec:
            runtime().hipGraphExecDestroy(self._exec)
            self._exec = None
        if self._graph:
            runtime().hipGraphDestroy(self._graph)
            self._graph = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
