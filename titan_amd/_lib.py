"""ctypes binding of libengine_hip.so (include/engine_hip.h, include/kv_host.h).

There is no fallback: if the library or its code objects are missing, every
entry point raises.  Build them with `python -m titan_amd.build` (or
__graft_entry__.build()).
"""
import ctypes as C
import os
import threading

LIB_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib")
# TITAN_AMD_HOST_LIB selects another build of the host library (the sanitized
# one of `python -m titan_amd.build --sanitize`); the code objects stay in LIB_DIR.
LIB_PATH = os.environ.get("TITAN_AMD_HOST_LIB") or os.path.join(LIB_DIR, "libengine_hip.so")

_lock = threading.Lock()
_lib = None

vp, u32, u64, i32, i64, f32 = C.c_void_p, C.c_uint32, C.c_uint64, C.c_int, C.c_int64, C.c_float
P = C.POINTER


class eh_kv_layout(C.Structure):
    _fields_ = [("n_blocks", u64), ("block_tokens", u64), ("row_len", u64),
                ("data_type", u32), ("reserved", u32)]


class eh_stream_cfg(C.Structure):
    _fields_ = [("sink_tokens", u64), ("recent_window_tokens", u64), ("max_budget_tokens", u64),
                ("block_tokens", u64)]


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
    "eh_append_kv_e4m3_batched": (i32, [vp, vp, P(eh_kv_layout), vp, u64, vp, u64, vp, u64, vp,
                                        u64, u32, vp, vp, u32, u64, u32, vp, vp]),
    "eh_gather_kv_e4m3": (i32, [vp, vp, P(eh_kv_layout), vp, u64, vp, u64, vp, u64, u64, u64, i32,
                                u32, vp]),
    "eh_kv_e4m3_scales": (i32, [vp, vp, P(eh_kv_layout), vp, u64, vp, u64, u64, u32, vp, u64, vp,
                                u64]),
    "eh_copy_pages": (i32, [vp, vp, P(eh_kv_layout), vp, u64, vp, vp, u32]),
    "eh_remap_block_tables": (i32, [vp, vp, vp, u64, vp, u32]),
    "eh_stream_pages": (i32, [vp, vp, P(eh_kv_layout), vp, u64, vp, u64, u32, u32, u32, vp, u64]),
    "eh_stream_pages_heads": (i32, [vp, vp, P(eh_kv_layout), vp, u64, vp, u64, u32, u32, u32, vp,
                                    u64]),
    "eh_page_refcounts": (i32, [vp, vp, vp, u32, vp, u32, vp, u32]),
    "eh_paged_attention": (i32, [vp, vp, u32, vp, u64, vp, u64, vp, u64, vp, u64, u64, u64, u64,
                                 u64, u64, u64, i32, vp]),
    "eh_flash_decoding": (i32, [vp, vp, u32, vp, u64, vp, u64, vp, u64, vp, u64, u64, u64, u64,
                                u64, u64, u64, i32, vp]),
    "eh_append_flash_decoding": (i32, [vp, vp, u32, vp, u64, vp, u64, vp, u64, vp, u64, vp, u64, vp,
                                       u64, u64, u64, u64, u64, u64, vp]),
    "eh_single_decode_workspace_bytes": (u64, []),
    "eh_paged_attention_ws": (i32, [vp, vp, u32, vp, u64, vp, u64, vp, u64, vp, u64, u64, u64, u64,
                                    u64, u64, u64, i32, vp, vp, u64]),
    "eh_flash_decoding_ws": (i32, [vp, vp, u32, vp, u64, vp, u64, vp, u64, vp, u64, u64, u64, u64,
                                   u64, u64, u64, i32, vp, vp, u64]),
    "eh_append_flash_decoding_ws": (i32, [vp, vp, u32, vp, u64, vp, u64, vp, u64, vp, u64, vp, u64,
                                          vp, u64, u64, u64, u64, u64, u64, vp, vp, u64]),
    "eh_decode_plan": (i32, [u32, u32, u32, u32, u32, u32, u32, u32, P(u32), P(u32), P(u64)]),
    "eh_decode_kernel_name": (i32, [u32, u32, u32, u32, u32, C.c_char_p, u64]),
    "eh_paged_decode_batched": (i32, [vp, vp, u32, vp, u64, vp, u64, vp, u64, u32, vp, u32, vp, u64,
                                      u32, u32, u32, u32, u32, u32, vp, u64]),
    "eh_paged_decode_batched_e4m3": (i32, [vp, vp, vp, u64, vp, u64, vp, u64, u32, vp, u32, vp, u64,
                                           u32, u32, u32, u32, vp, vp, u32, vp, u64]),
    "eh_paged_decode_batched_window": (i32, [vp, vp, u32, vp, u64, vp, u64, vp, u64, u32, vp, u32,
                                             vp, u64, u32, u32, u32, u32, u32, u32, vp, vp, vp, u64,
                                             u32, vp, u64]),
    "eh_decode_mass_workspace_bytes": (u64, [u32, u32, u32, u32]),
    "eh_decode_grid_workspace_bytes": (u64, [u32, u32, u32]),
    "eh_append_decode_batched": (i32, [vp, vp, P(eh_kv_layout), vp, u64, vp, u64, vp, u64, vp, u64,
                                       u32, vp, u32, vp, u64, vp, u64, u32, u32, u32, vp, u64]),
    "eh_decode_schedule_bytes": (u64, [u32, u32, u32, u32]),
    "eh_decode_schedule": (i32, [vp, vp, P(eh_kv_layout), vp, u64, u32, vp, u32, u32, u32, vp, u64]),
    "eh_append_decode_scheduled": (i32, [vp, vp, P(eh_kv_layout), vp, u64, vp, u64, vp, u64, vp, u64,
                                         u32, u32, vp, u64, vp, u64, u32, u32, u32, vp, u64, vp,
                                         vp]),
    "eh_append_decode_batched_noalloc": (i32, [vp, vp, P(eh_kv_layout), vp, u64, vp, u64, vp, u64,
                                               vp, u64, u32, vp, u32, vp, u64, vp, u64, u32, u32,
                                               u32]),
    "eh_append_decode_batched_e4m3": (i32, [vp, vp, P(eh_kv_layout), vp, u64, vp, u64, vp, u64, vp,
                                            u64, u32, vp, u32, vp, u64, vp, u64, u32, u32, u32, vp,
                                            u64, vp, vp]),
    "eh_flash_attention_prefill": (i32, [vp, vp, u32, vp, u64, vp, u64, vp, u64, vp, u64, u64, u64,
                                         u64, u64, u64, u64, vp]),
    "eh_prefill_batched_e4m3": (i32, [vp, vp, vp, u64, vp, u64, vp, u64, u32, vp, vp, u32, u32, u32,
                                      vp, u64, u32, u32, u32, u32, vp, vp]),
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
    "eh_kvcache_reserve_batch": (i32, [vp, vp, u64, vp, vp]),
    "eh_kvcache_truncate": (i32, [vp, u64, u64]),
    "eh_kvcache_export_tables": (i32, [vp, vp, u64, vp, u64, vp]),
    # prefix sharing (kv_share.h)
    "eh_cow_new": (vp, []),
    "eh_cow_fork": (vp, [vp]),
    "eh_cow_destroy": (None, [vp]),
    "eh_cow_append_block": (None, [vp, u32]),
    "eh_cow_is_shared": (i32, [vp, u64]),
    "eh_cow_tail_needs_cow": (i32, [vp]),
    "eh_cow_perform_tail_cow": (None, [vp, u32]),
    "eh_cow_block_ids": (u64, [vp, vp, u64]),
    "eh_cow_len": (u64, [vp]),
    "eh_cow_is_dirty": (i32, [vp, u64]),
    "eh_cow_ref_count": (u64, [vp, u64]),
    "eh_cow_seq_len": (u64, [vp]),
    "eh_cow_set_seq_len": (None, [vp, u64]),
    "eh_radix_new": (vp, [u64]),
    "eh_radix_destroy": (None, [vp]),
    "eh_radix_match_prefix": (u64, [vp, vp, u64, vp, u64, P(u64)]),
    "eh_radix_insert": (None, [vp, vp, u64, vp, u64, i32]),
    "eh_radix_evict_lru": (u64, [vp, u64, vp, u64]),
    "eh_radix_total_cached_blocks": (u64, [vp]),
    "eh_radix_invalidate_physical_blocks": (None, [vp, vp, u64]),
    "eh_radix_set_ref_count": (i32, [vp, vp, u64, u64]),
    "eh_stream_cfg_new": (eh_stream_cfg, [u64, u64, u64, u64]),
    "eh_stream_cfg_default": (eh_stream_cfg, []),
    "eh_stream_sink_blocks": (u64, [eh_stream_cfg]),
    "eh_stream_recent_blocks": (u64, [eh_stream_cfg]),
    "eh_stream_max_active_blocks": (u64, [eh_stream_cfg]),
    "eh_stream_new": (vp, [eh_stream_cfg]),
    "eh_stream_destroy": (None, [vp]),
    "eh_stream_record_attention_mass": (None, [vp, u32, f32]),
    "eh_stream_record_attention_masses": (None, [vp, vp, u64]),
    "eh_stream_scores_len": (u64, [vp]),
    "eh_stream_score": (f32, [vp, u32]),
    "eh_stream_prune_blocks": (None, [vp, vp, u64, vp, P(u64), vp, P(u64)]),
    "eh_compaction_plan": (i64, [vp, u64, vp, u64, u32, vp, vp, vp]),
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
