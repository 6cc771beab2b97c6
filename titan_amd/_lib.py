"""ctypes binding of libengine_hip.so (include/engine_hip.h, include/kv_host.h).

There is no fallback: if the library or its code objects are missing, every
entry point raises.  Build them with `python -m titan_amd.build` (or
__graft_entry__.build()).
"""
import ctypes as C
import os
import threading

LIB_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib")
LIB_PATH = os.path.join(LIB_DIR, "libengine_hip.so")

_lock = threading.Lock()
_lib = None

vp, u32, u64, i32, i64, f32 = C.c_void_p, C.c_uint32, C.c_uint64, C.c_int, C.c_int64, C.c_float
P = C.POINTER


class eh_kv_layout(C.Structure):
    _fields_ = [("n_blocks", u64), ("block_tokens", u64), ("row_len", u64),
                ("data_type", u32), ("reserved", u32)]


_SIGS = {
    "eh_create": (i32, [i32, C.c_char_p, P(vp)]),
    "eh_destroy": (None, [vp]),
    "eh_last_error": (i32, [P(u64), P(u64), P(C.c_char_p), P(i32)]),
    "eh_status_name": (C.c_char_p, [i32]),
    "eh_kv_element_bytes": (u64, [u32]),
    "eh_kv_layout_bytes_total": (u64, [P(eh_kv_layout)]),
    "eh_append_kv": (i32, [vp, vp, P(eh_kv_layout), vp, u64, vp, u64, vp, u64, vp, u64, u64, u64, vp]),
    "eh_gather_kv": (i32, [vp, vp, P(eh_kv_layout), vp, u64, vp, u64, vp, u64, u64, u64, i32]),
    "eh_append_kv_batched": (i32, [vp, vp, P(eh_kv_layout), vp, u64, vp, u64, vp, u64, vp, u64, u32,
                                   vp, vp, u32, u64]),
    "eh_copy_pages": (i32, [vp, vp, P(eh_kv_layout), vp, u64, vp, vp, u32]),
    "eh_remap_block_tables": (i32, [vp, vp, vp, u64, vp, u32]),
    "eh_page_refcounts": (i32, [vp, vp, vp, u32, vp, u32, vp, u32]),
    "eh_paged_attention": (i32, [vp, vp, u32, vp, u64, vp, u64, vp, u64, vp, u64, u64, u64, u64,
                                 u64, u64, u64, i32, vp]),
    "eh_flash_decoding": (i32, [vp, vp, u32, vp, u64, vp, u64, vp, u64, vp, u64, u64, u64, u64,
                                u64, u64, u64, i32, vp]),
    "eh_decode_plan": (i32, [u32, u32, u32, u32, u32, u32, u32, u32, P(u32), P(u32), P(u64)]),
    "eh_paged_decode_batched": (i32, [vp, vp, u32, vp, u64, vp, u64, vp, u64, u32, vp, u32, vp, u64,
                                      u32, u32, u32, u32, u32, u32, vp, u64]),
    "eh_flash_attention_prefill": (i32, [vp, vp, u32, vp, u64, vp, u64, vp, u64, vp, u64, u64, u64,
                                         u64, u64, u64, u64, vp]),
    "eh_prefill_batched": (i32, [vp, vp, u32, vp, u64, vp, u64, vp, u64, u32, vp, vp, u32, u32, u32,
                                 vp, u64, u32, u32, u32, u32]),
    # host bookkeeping (kv_host.h)
    "eh_kvcache_new": (i32, [u64, u64, u64, u64, u32, P(vp)]),
    "eh_kvcache_destroy": (None, [vp]),
    "eh_kvcache_last_message": (C.c_char_p, []),
    "eh_kvcache_last_exhausted": (i32, [P(u64), P(u64)]),
    "eh_kvcache_seed_free_list": (i32, [vp, vp, u64]),
    "eh_kvcache_blocks_total": (u64, [vp]),
    "eh_kvcache_blocks_used": (u64, [vp]),
    "eh_kvcache_sequences": (u64, [vp]),
    "eh_kvcache_new_sequence": (u64, [vp]),
    "eh_kvcache_free_sequence": (None, [vp, u64]),
    "eh_kvcache_token_count": (u64, [vp, u64]),
    "eh_kvcache_block_table": (i64, [vp, u64, vp, u64]),
    "eh_kvcache_reserve": (i32, [vp, u64, u64, P(u64)]),
    "eh_kvcache_export_tables": (i32, [vp, vp, u64, vp, u64, vp]),
}

EXPORTED = tuple(_SIGS)


def load():
    """Load and type the C-ABI library (raises if it has not been built)."""
    global _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"titan_amd native library missing: {LIB_PATH}; build it with "
                    "`python -m titan_amd.build` -- there is no CPU fallback")
            L = C.CDLL(LIB_PATH)
            for name, (res, args) in _SIGS.items():
                fn = getattr(L, name)
                fn.restype = res
                fn.argtypes = args
            _lib = L
    return _lib
