"""Device context and buffer plumbing for the C-ABI.

A buffer is any object exposing a device pointer and a size in bytes: a
torch tensor on the GPU (data_ptr(), numel()*element_size()) or a
(pointer, nbytes) pair.  Streams are torch streams, raw hipStream_t handles
(int) or None for torch's current stream.
"""
import ctypes as C
import threading

from . import _lib
from .errors import check

_ctx_lock = threading.Lock()
_contexts = {}


class Context:
    """Loaded gfx950 code objects + split-K scratch on one device
    (the state PagedKvGpu::new / PagedAttention::new build in the reference)."""

    def __init__(self, device=0, code_object_dir=None):
        L = _lib.load()
        h = C.c_void_p()
        check(L.eh_create(int(device), code_object_dir.encode() if code_object_dir else None,
                          C.byref(h)))
        self.handle = h
        self.device = int(device)

    def __del__(self):
        h = getattr(self, "handle", None)
        if h:
            try:
                _lib.load().eh_destroy(h)
            except Exception:
                pass
            self.handle = None


def context(device=0):
    """Process-wide context for `device` (created on first use)."""
    dev = _device_index(device)
    with _ctx_lock:
        ctx = _contexts.get(dev)
        if ctx is None:
            ctx = Context(dev)
            _contexts[dev] = ctx
    return ctx


def _device_index(device):
    if device is None:
        return 0
    if isinstance(device, int):
        return device
    idx = getattr(device, "index", None)
    return 0 if idx is None else int(idx)


def buf(x):
    """(pointer, nbytes) of a device buffer; (None, 0) for None."""
    if x is None:
        return None, 0
    if isinstance(x, tuple):
        return C.c_void_p(int(x[0])), int(x[1])
    if not x.is_cuda:
        raise ValueError("buffer must live in device memory")
    if not x.is_contiguous():
        raise ValueError("buffer must be contiguous")
    return C.c_void_p(x.data_ptr()), x.numel() * x.element_size()


def ptr(x):
    return buf(x)[0]


def stream_handle(stream):
    if stream is None:
        import torch
        return C.c_void_p(torch.cuda.current_stream().cuda_stream)
    if isinstance(stream, int):
        return C.c_void_p(stream)
    return C.c_void_p(stream.cuda_stream)
