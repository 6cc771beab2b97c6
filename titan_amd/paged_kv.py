"""Paged KV append / gather on gfx950 -- the engine-cuda `paged_kv` surface.

Mirrors engine-cuda/src/paged_kv.rs: `KvDataType`, `PagedKvLayout` and
`PagedKvGpu` with `append_kv`, `append_kv_with_pos_ptr`, `read_keys` and
`read_values`, same argument meaning and the same InvalidSize checks, plus
batched extensions (ragged append, page copies for copy-on-write and
compaction, block-table remap, page reference counts).
"""
import ctypes as C
from dataclasses import dataclass
from enum import IntEnum

from . import _lib
from .errors import check
from .runtime import buf, context, stream_handle


class KvDataType(IntEnum):
    """engine-cuda/src/paged_kv.rs:36-52 (+ BF16)."""
    F32 = 0
    F16 = 1
    FP8 = 2
    BF16 = 3

    def element_bytes(self):
        return {0: 4, 1: 2, 2: 1, 3: 2}[int(self)]


@dataclass(frozen=True)
class PagedKvLayout:
    """engine-cuda/src/paged_kv.rs:55-102."""
    n_blocks: int
    block_tokens: int
    row_len: int
    data_type: KvDataType = KvDataType.F32

    def floats_per_token(self):
        return 2 * self.row_len

    def floats_per_block(self):
        return self.block_tokens * self.floats_per_token()

    def floats_total(self):
        return self.n_blocks * self.floats_per_block()

    def bytes_total(self):
        return self.floats_total() * KvDataType(self.data_type).element_bytes()

    def total_tokens(self):
        return self.n_blocks * self.block_tokens

    def page_bytes(self):
        return self.floats_per_block() * KvDataType(self.data_type).element_bytes()

    def c(self):
        return _lib.eh_kv_layout(self.n_blocks, self.block_tokens, self.row_len,
                                 int(self.data_type), 0)


class PagedKvGpu:
    """engine-cuda/src/paged_kv.rs:108-491 on HIP code objects."""

    def __init__(self, device=0):
        self._ctx = context(device)
        self._L = _lib.load()

    def append_kv(self, stream, layout, pool, keys, values, block_table, start_token, n_tokens):
        """paged_kv.rs:200-224"""
        return self.append_kv_with_pos_ptr(stream, layout, pool, keys, values, block_table,
                                           start_token, n_tokens, None)

    def append_kv_with_pos_ptr(self, stream, layout, pool, keys, values, block_table,
                               start_token, n_tokens, pos_ptr):
        """paged_kv.rs:227-327; pos_ptr (device u32) overrides start_token."""
        pp, pb = buf(pool)
        kp, kb = buf(keys)
        vp, vb = buf(values)
        bp, bb = buf(block_table)
        check(self._L.eh_append_kv(self._ctx.handle, stream_handle(stream), C.byref(layout.c()),
                                   pp, pb, kp, kb, vp, vb, bp, bb, int(start_token),
                                   int(n_tokens), buf(pos_ptr)[0]))

    def read_keys(self, stream, layout, pool, block_table, out, start_token, n_tokens):
        """paged_kv.rs:331-353"""
        self._gather(stream, layout, pool, block_table, out, start_token, n_tokens, 0)

    def read_values(self, stream, layout, pool, block_table, out, start_token, n_tokens):
        """paged_kv.rs:356-378"""
        self._gather(stream, layout, pool, block_table, out, start_token, n_tokens, 1)

    def _gather(self, stream, layout, pool, block_table, out, start_token, n_tokens, is_value):
        pp, pb = buf(pool)
        bp, bb = buf(block_table)
        op, ob = buf(out)
        check(self._L.eh_gather_kv(self._ctx.handle, stream_handle(stream), C.byref(layout.c()),
                                   pp, pb, bp, bb, op, ob, int(start_token), int(n_tokens),
                                   int(is_value)))

    # ---- batched extensions -------------------------------------------------
    def append_kv_batched(self, stream, layout, pool, keys, values, block_tables, cu_seqlens,
                          start_pos, total_tokens):
        """Ragged batch: block_tables [B, stride] u32, cu_seqlens [B+1], start_pos [B]."""
        pp, pb = buf(pool)
        kp, kb = buf(keys)
        vp, vb = buf(values)
        bp, bb = buf(block_tables)
        batch, stride = block_tables.shape
        check(self._L.eh_append_kv_batched(self._ctx.handle, stream_handle(stream),
                                           C.byref(layout.c()), pp, pb, kp, kb, vp, vb, bp, bb,
                                           int(stride), buf(cu_seqlens)[0], buf(start_pos)[0],
                                           int(batch), int(total_tokens)))

    # ---- FP8 (E4M3) pools with per-kv-head f32 scales ---------------------
    def append_kv_e4m3_batched(self, stream, layout, pool, keys, values, block_tables, cu_seqlens,
                               start_pos, total_tokens, head_dim, k_scale, v_scale):
        """append_kv_batched into an E4M3 pool: keys/values [T, row_len] f32 are
        stored as quantize(x / scale[head]) (round to nearest even, saturating
        at 448); k_scale/v_scale [n_kv] f32 device tensors."""
        pp, pb = buf(pool)
        kp, kb = buf(keys)
        vp, vb = buf(values)
        bp, bb = buf(block_tables)
        batch, stride = block_tables.shape
        check(self._L.eh_append_kv_e4m3_batched(
            self._ctx.handle, stream_handle(stream), C.byref(layout.c()), pp, pb, kp, kb, vp, vb, bp,
            bb, int(stride), buf(cu_seqlens)[0], buf(start_pos)[0], int(batch), int(total_tokens),
            int(head_dim), buf(k_scale)[0], buf(v_scale)[0]))

    def e4m3_scales(self, stream, layout, keys, values, head_dim, k_scale, v_scale):
        """Dynamic per-kv-head scales of an E4M3 pool from f32 rows keys/values
        [n, row_len] (a prompt or a calibration sample): scale = max(amax / 448,
        FLT_MIN) per head over the finite elements, 1 for a head with none
        nonzero; written to the device tensors k_scale / v_scale [n_kv] that
        the E4M3 entry points read (the per-head scales of the FP8 KV design,
        openspec/archive/2026-08-28-fp8-kv-cache-quantization/specs/
        kv-compression/spec.md:9)."""
        kp, kb = buf(keys)
        vp, vb = buf(values)
        ksp, ksb = buf(k_scale)
        vsp, vsb = buf(v_scale)
        check(self._L.eh_kv_e4m3_scales(self._ctx.handle, stream_handle(stream),
                                        C.byref(layout.c()), kp, kb, vp, vb, int(keys.shape[0]),
                                        int(head_dim), ksp, ksb, vsp, vsb))

    def read_e4m3(self, stream, layout, pool, block_table, out, start_token, n_tokens, is_value,
                  head_dim, scale):
        """read_keys / read_values of an E4M3 pool, dequantised: out [n, row_len]
        f32 = decode(code) * scale[head]."""
        pp, pb = buf(pool)
        bp, bb = buf(block_table)
        op, ob = buf(out)
        check(self._L.eh_gather_kv_e4m3(self._ctx.handle, stream_handle(stream), C.byref(layout.c()),
                                        pp, pb, bp, bb, op, ob, int(start_token), int(n_tokens),
                                        int(is_value), int(head_dim), buf(scale)[0]))

    def copy_pages(self, stream, layout, pool, src_ids, dst_ids):
        """Whole-page copies dst_ids[k] <- src_ids[k] (copy-on-write, compaction)."""
        pp, pb = buf(pool)
        n = src_ids.numel()
        if dst_ids.numel() != n:
            raise ValueError("src_ids and dst_ids differ in length")
        check(self._L.eh_copy_pages(self._ctx.handle, stream_handle(stream), C.byref(layout.c()),
                                    pp, pb, buf(src_ids)[0], buf(dst_ids)[0], int(n)))

    def stream_pages(self, stream, layout, pool, ids, out, depth=1, grid=256):
        """Measurement aid (no reference counterpart): reads the pages listed
        in `ids` once (16 KiB items, `depth` in flight per wave, `grid`
        workgroups of 8 waves) and writes one xor of the words read per
        wave into `out` (u32 [grid * 8]): the cold-read floor of a decode
        over the same pages."""
        pp, pb = buf(pool)
        ip, ib = buf(ids)
        op, ob = buf(out)
        check(self._L.eh_stream_pages(self._ctx.handle, stream_handle(stream),
                                      C.byref(layout.c()), pp, pb, ip, ib, int(ids.numel()),
                                      int(depth), int(grid), op, ob))

    def stream_pages_heads(self, stream, layout, pool, ids, out, head_dim, grid=256):
        """Measurement aid (no reference counterpart): reads the pages listed
        in `ids` in the token-balanced decode's pattern, one wave per kv head
        reading only that head's K and V rows, the n_kv waves of a group
        walking the same pages (two in flight); `out` as stream_pages."""
        pp, pb = buf(pool)
        ip, ib = buf(ids)
        op, ob = buf(out)
        check(self._L.eh_stream_pages_heads(self._ctx.handle, stream_handle(stream),
                                            C.byref(layout.c()), pp, pb, ip, ib, int(ids.numel()),
                                            int(head_dim), int(grid), op, ob))

    def remap_block_tables(self, stream, block_tables, remap):
        """entry = remap[entry] for every entry below len(remap)."""
        check(self._L.eh_remap_block_tables(self._ctx.handle, stream_handle(stream),
                                            buf(block_tables)[0], block_tables.numel(),
                                            buf(remap)[0], remap.numel()))

    def page_refcounts(self, stream, block_tables, n_used, counts):
        """counts[p] = number of live table entries equal to p (overwritten)."""
        batch, stride = block_tables.shape
        check(self._L.eh_page_refcounts(self._ctx.handle, stream_handle(stream),
                                        buf(block_tables)[0], int(stride), buf(n_used)[0],
                                        int(batch), buf(counts)[0], counts.numel()))
