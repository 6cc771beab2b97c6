"""Typed errors mirroring engine-cuda's CudaError (engine-cuda/src/error.rs:6-50)
and engine-kvcache's KvCacheError (engine-kvcache/src/error.rs:4-16)."""
import ctypes as C

from . import _lib

STATUS = {
    0: "Ok", 1: "InvalidSize", 2: "KernelLoad", 3: "KernelLaunch", 4: "AllocFailed",
    5: "StreamFailed", 6: "MemcpyFailed", 7: "EventFailed", 8: "GraphFailed", 9: "Driver",
    20: "PoolExhausted", 21: "InvalidArgs", 30: "Unsupported",
}


class HipError(Exception):
    """CudaError counterpart.  `kind` names the variant; InvalidSize carries
    expected/actual like `CudaError::InvalidSize{expected, actual}`."""

    def __init__(self, kind, expected=None, actual=None, site=None, code=None):
        self.kind, self.expected, self.actual, self.site, self.code = kind, expected, actual, site, code
        if kind == "InvalidSize":
            msg = f"Invalid buffer size: expected <= {expected}, got {actual} ({site})"
        else:
            msg = f"{kind} in '{site}' (hip code {code})"
        super().__init__(msg)


class KvCacheError(Exception):
    """KvCacheError counterpart: PoolExhausted{blocks_used, blocks_total} or InvalidArgs(msg)."""

    def __init__(self, kind, msg=None, blocks_used=None, blocks_total=None):
        self.kind, self.msg, self.blocks_used, self.blocks_total = kind, msg, blocks_used, blocks_total
        if kind == "PoolExhausted":
            text = f"KV-cache block pool exhausted: {blocks_used} of {blocks_total} blocks in use"
        else:
            text = f"Invalid KV-cache argument: {msg}"
        super().__init__(text)


def check(status, host=False):
    """Raise the typed error for a non-zero eh_status.  `host` marks calls of
    the host bookkeeping (kv_host.h), whose detail is kept separately."""
    if status == 0:
        return
    L = _lib.load()
    kind = STATUS.get(status, f"Status{status}")
    if host and status in (20, 21):
        used, total = C.c_uint64(), C.c_uint64()
        L.eh_kvcache_last_exhausted(C.byref(used), C.byref(total))
        msg = L.eh_kvcache_last_message()
        raise KvCacheError(kind, msg.decode() if msg else None, used.value, total.value)
    exp, act, site, code = C.c_uint64(), C.c_uint64(), C.c_char_p(), C.c_int()
    L.eh_last_error(C.byref(exp), C.byref(act), C.byref(site), C.byref(code))
    if status == 21:
        raise KvCacheError(kind, site.value.decode() if site.value else None)
    raise HipError(kind, exp.value, act.value, site.value.decode() if site.value else None, code.value)
