"""Paged-attention decode on gfx950 -- the engine-cuda `PagedAttention` surface.

Mirrors engine-cuda/src/paged_attention.rs: `launch`, `launch_with_pos_ptr`
and `launch_flash_decoding` with the reference's argument order and
validation, plus `decode_batched` for B sequences in one launch.  The pool's
element type is an extra keyword (`kv_dtype`, default F32 as in the
reference).  MAX_* constants are kept for API compatibility; the HIP path
itself attends every token (no 32-split cap).
"""
import ctypes as C

import torch

from . import _lib
from .errors import check
from .paged_kv import KvDataType
from .runtime import buf, context, stream_handle

MAX_FLASH_DECODING_SPLITS = 32   # paged_attention.rs:33
MAX_ATTN_HEADS = 64              # paged_attention.rs:35
MAX_HEAD_DIM = 128               # paged_attention.rs:37
SUPPORTED_HEAD_DIMS = (4, 8, 16, 32, 64, 128, 256)


class PagedAttention:
    """engine-cuda/src/paged_attention.rs:40-490 on HIP code objects."""

    def __init__(self, device=0):
        self._ctx = context(device)
        self._L = _lib.load()

    def launch(self, stream, q, pool, block_table, out, n_head, n_head_kv, head_dim,
               block_tokens, seq_tokens, query_pos, causal, kv_dtype=KvDataType.F32):
        """paged_attention.rs:143-174"""
        self.launch_with_pos_ptr(stream, q, pool, block_table, out, n_head, n_head_kv, head_dim,
                                 block_tokens, seq_tokens, query_pos, causal, None, kv_dtype)

    def launch_with_pos_ptr(self, stream, q, pool, block_table, out, n_head, n_head_kv, head_dim,
                            block_tokens, seq_tokens, query_pos, causal, pos_ptr,
                            kv_dtype=KvDataType.F32, workspace=None):
        """paged_attention.rs:177-345 (single pass per kv head).  With a
        workspace tensor the split-K partials go there instead of the
        context's shared scratch (calls on other streams may overlap)."""
        self._call(self._L.eh_paged_attention, stream, q, pool, block_table, out, n_head,
                   n_head_kv, head_dim, block_tokens, seq_tokens, query_pos, causal, pos_ptr,
                   kv_dtype, workspace, self._L.eh_paged_attention_ws)

    def launch_flash_decoding(self, stream, q, pool, block_table, out, n_head, n_head_kv,
                              head_dim, block_tokens, seq_tokens, query_pos, causal, pos_ptr=None,
                              kv_dtype=KvDataType.F32, workspace=None):
        """paged_attention.rs:352-490 (split-K + log-sum-exp merge); workspace
        as launch_with_pos_ptr."""
        self._call(self._L.eh_flash_decoding, stream, q, pool, block_table, out, n_head,
                   n_head_kv, head_dim, block_tokens, seq_tokens, query_pos, causal, pos_ptr,
                   kv_dtype, workspace, self._L.eh_flash_decoding_ws)

    @staticmethod
    def single_workspace_bytes():
        """A workspace size that suffices for every single-sequence call."""
        return int(_lib.load().eh_single_decode_workspace_bytes())

    def append_flash_decoding(self, stream, keys, values, q, pool, block_table, out, n_head,
                              n_head_kv, head_dim, block_tokens, query_pos, pos_ptr=None,
                              kv_dtype=KvDataType.F32, workspace=None):
        """One decode step of one sequence in one launch: keys/values [row_len]
        land at position *pos_ptr (or query_pos), then q attends tokens 0..that
        position (PagedKvGpu.append_kv, paged_kv.rs:200-327, followed by
        launch_flash_decoding, paged_attention.rs:352-490); workspace as
        launch_with_pos_ptr."""
        kp, kb = buf(keys)
        vp_, vb = buf(values)
        qp, qb = buf(q)
        pp, pb = buf(pool)
        bp, bb = buf(block_table)
        op, ob = buf(out)
        args = (self._ctx.handle, stream_handle(stream), int(kv_dtype), kp, kb, vp_, vb, qp, qb, pp,
                pb, bp, bb, op, ob, int(n_head), int(n_head_kv), int(head_dim), int(block_tokens),
                int(query_pos), buf(pos_ptr)[0])
        if workspace is None:
            check(self._L.eh_append_flash_decoding(*args))
        else:
            check(self._L.eh_append_flash_decoding_ws(*args, *buf(workspace)))

    def _call(self, fn, stream, q, pool, block_table, out, n_head, n_head_kv, head_dim,
              block_tokens, seq_tokens, query_pos, causal, pos_ptr, kv_dtype, workspace=None,
              fn_ws=None):
        qp, qb = buf(q)
        pp, pb = buf(pool)
        bp, bb = buf(block_table)
        op, ob = buf(out)
        args = (self._ctx.handle, stream_handle(stream), int(kv_dtype), qp, qb, pp, pb, bp, bb,
                op, ob, int(n_head), int(n_head_kv), int(head_dim), int(block_tokens),
                int(seq_tokens), int(query_pos), 1 if causal else 0, buf(pos_ptr)[0])
        if workspace is None:
            check(fn(*args))
        else:
            check(fn_ws(*args, *buf(workspace)))

    # ---- batched extension ---------------------------------------------------
    @staticmethod
    def plan(batch, n_head, n_head_kv, head_dim, block_tokens, max_ctx, tokens_per_split=0,
             kv_dtype=KvDataType.F16):
        """(tokens_per_split, max_splits, workspace_bytes) for decode_batched."""
        L = _lib.load()
        tps, ms, ws = C.c_uint32(), C.c_uint32(), C.c_uint64()
        check(L.eh_decode_plan(int(kv_dtype), int(batch), int(n_head), int(n_head_kv), int(head_dim),
                               int(block_tokens), int(max_ctx), int(tokens_per_split),
                               C.byref(tps), C.byref(ms), C.byref(ws)))
        return tps.value, ms.value, ws.value

    @staticmethod
    def kernel_name(n_head, n_head_kv, head_dim, block_tokens, kv_dtype=KvDataType.F16):
        """Split kernel decode_batched launches for this shape."""
        buf_ = C.create_string_buffer(64)
        check(_lib.load().eh_decode_kernel_name(int(kv_dtype), int(n_head), int(n_head_kv),
                                                int(head_dim), int(block_tokens), buf_, 64))
        return buf_.value.decode()

    @staticmethod
    def workspace(plan, device="cuda"):
        """Workspace for the split partials of decode_batched."""
        nbytes = max(plan[2], 4)
        return torch.empty(nbytes // 4, dtype=torch.float32, device=device)

    def decode_batched(self, stream, q, pool, block_tables, ctx_lens, out, n_head, n_head_kv,
                       head_dim, block_tokens, kv_dtype, plan, workspace):
        """q/out [B, n_head, head_dim] f32, block_tables [B, stride] u32,
        ctx_lens [B] u32 (each <= plan's max_ctx)."""
        batch, stride = block_tables.shape
        qp, qb = buf(q)
        pp, pb = buf(pool)
        bp, bb = buf(block_tables)
        op, ob = buf(out)
        wp, wb = buf(workspace)
        check(self._L.eh_paged_decode_batched(
            self._ctx.handle, stream_handle(stream), int(kv_dtype), qp, qb, pp, pb, bp, bb,
            int(stride), buf(ctx_lens)[0], int(batch), op, ob, int(n_head), int(n_head_kv),
            int(head_dim), int(block_tokens), int(plan[0]), int(plan[1]), wp, wb))

    def decode_batched_e4m3(self, stream, q, pool, block_tables, ctx_lens, out, n_head,
                            n_head_kv, head_dim, block_tokens, k_scale, v_scale, plan, workspace):
        """decode_batched over an E4M3 pool (per-kv-head f32 scales k_scale /
        v_scale): attention on decode(code) * scale.  `plan` is
        PagedAttention.plan(..., kv_dtype=KvDataType.FP8) (token-balanced)."""
        batch, stride = block_tables.shape
        qp, qb = buf(q)
        pp, pb = buf(pool)
        bp, bb = buf(block_tables)
        op, ob = buf(out)
        wp, wb = buf(workspace)
        check(self._L.eh_paged_decode_batched_e4m3(
            self._ctx.handle, stream_handle(stream), qp, qb, pp, pb, bp, bb, int(stride),
            buf(ctx_lens)[0], int(batch), op, ob, int(n_head), int(n_head_kv), int(head_dim),
            int(block_tokens), buf(k_scale)[0], buf(v_scale)[0], int(plan[1]), wp, wb))

    @staticmethod
    def with_grid(plan, grid, batch, n_head):
        """A token-balanced plan launched with `grid` workgroups instead of its
        own, with the workspace size that grid needs."""
        if plan[0] != 0:
            raise ValueError("a grid applies to token-balanced plans (tokens_per_split 0)")
        return 0, int(grid), int(_lib.load().eh_decode_grid_workspace_bytes(int(grid), int(batch),
                                                                            int(n_head)))

    @staticmethod
    def mass_workspace_bytes(batch, bt_stride, block_tokens, n_head):
        """Extra workspace decode_batched_window needs when it accumulates block_mass."""
        return int(_lib.load().eh_decode_mass_workspace_bytes(int(batch), int(bt_stride),
                                                               int(block_tokens), int(n_head)))

    def decode_batched_window(self, stream, q, pool, block_tables, ctx_lens, out, n_head,
                              n_head_kv, head_dim, block_tokens, kv_dtype, sink_tokens,
                              window_tokens, plan, workspace, k_scale=None, v_scale=None,
                              block_mass=None):
        """decode_batched over the protected-sinks range: the query at
        pos = ctx_lens[b] - 1 attends [0, sink) and [max(sink, pos - window), pos]
        (window 0: every token).  E4M3 pools pass k_scale / v_scale.  With
        block_mass ([pages] f32) each page's attention mass summed over q heads
        is added to it (the H2O score of record_attention_mass); the workspace
        then needs plan[2] + mass_workspace_bytes(...) bytes."""
        batch, stride = block_tables.shape
        qp, qb = buf(q)
        pp, pb = buf(pool)
        bp, bb = buf(block_tables)
        op, ob = buf(out)
        wp, wb = buf(workspace)
        check(self._L.eh_paged_decode_batched_window(
            self._ctx.handle, stream_handle(stream), int(kv_dtype), qp, qb, pp, pb, bp, bb,
            int(stride), buf(ctx_lens)[0], int(batch), op, ob, int(n_head), int(n_head_kv),
            int(head_dim), int(block_tokens), int(sink_tokens), int(window_tokens),
            buf(k_scale)[0], buf(v_scale)[0], *buf(block_mass), int(plan[1]), wp, wb))

    def append_decode_batched(self, stream, layout, pool, keys, values, block_tables, start_pos,
                              q, out, n_head, head_dim, plan, workspace):
        """One decode step in one launch: row b of keys/values [B, row_len]
        lands at logical position start_pos[b] (device u32) through
        block_tables [B, stride], then q [B, n_head, head_dim] attends tokens
        0..start_pos[b] (the batched append_kv of paged_kv.rs:200-327 followed
        by launch_with_pos_ptr, paged_attention.rs:177-345).  `plan` is
        PagedAttention.plan(...) with tokens_per_split 0 on a shape the
        token-balanced kernel serves (plan[0] == 0)."""
        if plan[0] != 0:
            raise ValueError("append_decode_batched needs a token-balanced plan (tokens_per_split 0)")
        batch, stride = block_tables.shape
        pp, pb = buf(pool)
        kp, kb = buf(keys)
        vp_, vb = buf(values)
        bp, bb = buf(block_tables)
        qp, qb = buf(q)
        op, ob = buf(out)
        wp, wb = buf(workspace)
        lay = layout.c()
        check(self._L.eh_append_decode_batched(
            self._ctx.handle, stream_handle(stream), C.byref(lay), pp, pb, kp, kb, vp_, vb, bp, bb,
            int(stride), buf(start_pos)[0], int(batch), qp, qb, op, ob, int(n_head), int(head_dim),
            int(plan[1]), wp, wb))

    # ---- step schedule: the work split computed once per decode step -------
    @staticmethod
    def schedule_bytes(batch, bt_stride, block_tokens, plan):
        """Bytes of the step schedule for `batch` sequences with tables of
        `bt_stride` entries and a token-balanced plan."""
        return int(_lib.load().eh_decode_schedule_bytes(int(batch), int(bt_stride),
                                                         int(block_tokens), int(plan[1])))

    @staticmethod
    def schedule_buffer(batch, bt_stride, block_tokens, plan, device="cuda"):
        n = PagedAttention.schedule_bytes(batch, bt_stride, block_tokens, plan)
        return torch.empty((n + 15) // 16 * 4, dtype=torch.int32, device=device)

    def build_schedule(self, stream, layout, block_tables, lens, lens_add, plan, sched):
        """eh_decode_schedule: the token-balanced split of the step, from
        block_tables [B, stride] and lens [B] (+ lens_add: 1 with the
        positions a fused step appends at)."""
        if plan[0] != 0:
            raise ValueError("a step schedule needs a token-balanced plan (tokens_per_split 0)")
        batch, stride = block_tables.shape
        bp, bb = buf(block_tables)
        sp, sb = buf(sched)
        lay = layout.c()
        check(self._L.eh_decode_schedule(self._ctx.handle, stream_handle(stream), C.byref(lay), bp,
                                         bb, int(stride), buf(lens)[0], int(lens_add), int(batch),
                                         int(plan[1]), sp, sb))

    def append_decode_scheduled(self, stream, layout, pool, keys, values, sched, bt_stride, q,
                                out, n_head, head_dim, plan, workspace, k_scale=None,
                                v_scale=None):
        """One layer's decode step from a step schedule: keys/values [B,
        row_len] appended at the schedule's positions (None: decode only),
        then q [B, n_head, head_dim] attends (append_decode_batched /
        decode_batched with the split read from `sched`).  E4M3 pools pass
        f32 rows and k_scale / v_scale."""
        batch = q.shape[0]
        pp, pb = buf(pool)
        kp, kb = buf(keys)
        vp_, vb = buf(values)
        sp, sb = buf(sched)
        qp, qb = buf(q)
        op, ob = buf(out)
        wp, wb = buf(workspace)
        lay = layout.c()
        check(self._L.eh_append_decode_scheduled(
            self._ctx.handle, stream_handle(stream), C.byref(lay), pp, pb, kp, kb, vp_, vb, sp, sb,
            int(bt_stride), int(batch), qp, qb, op, ob, int(n_head), int(head_dim), int(plan[1]),
            wp, wb, buf(k_scale)[0], buf(v_scale)[0]))

    def append_decode_batched_noalloc(self, stream, layout, pool, keys, values, block_tables,
                                      start_pos, q, out, n_head, head_dim, grid):
        """append_decode_batched with the library's per-GPU static scratch in
        place of a workspace: for callers that cannot allocate device memory.
        `grid` is plan[1] of a token-balanced plan; shapes whose partials
        exceed the 32 MiB scratch raise InvalidSize.  Calls that overlap in
        time on one GPU race on the shared scratch."""
        batch, stride = block_tables.shape
        pp, pb = buf(pool)
        kp, kb = buf(keys)
        vp_, vb = buf(values)
        bp, bb = buf(block_tables)
        qp, qb = buf(q)
        op, ob = buf(out)
        lay = layout.c()
        check(self._L.eh_append_decode_batched_noalloc(
            self._ctx.handle, stream_handle(stream), C.byref(lay), pp, pb, kp, kb, vp_, vb, bp, bb,
            int(stride), buf(start_pos)[0], int(batch), qp, qb, op, ob, int(n_head), int(head_dim),
            int(grid)))

    def append_decode_batched_e4m3(self, stream, layout, pool, keys, values, block_tables,
                                   start_pos, q, out, n_head, head_dim, plan, workspace, k_scale,
                                   v_scale):
        """append_decode_batched over E4M3 pages: keys/values [B, row_len] f32
        are quantised in the launch with k_scale / v_scale [n_head_kv] (as
        PagedKvGpu.append_kv_e4m3_batched), then attended as
        decode_batched_e4m3."""
        if plan[0] != 0:
            raise ValueError("append_decode_batched_e4m3 needs a token-balanced plan "
                             "(tokens_per_split 0)")
        batch, stride = block_tables.shape
        pp, pb = buf(pool)
        kp, kb = buf(keys)
        vp_, vb = buf(values)
        bp, bb = buf(block_tables)
        qp, qb = buf(q)
        op, ob = buf(out)
        wp, wb = buf(workspace)
        lay = layout.c()
        check(self._L.eh_append_decode_batched_e4m3(
            self._ctx.handle, stream_handle(stream), C.byref(lay), pp, pb, kp, kb, vp_, vb, bp, bb,
            int(stride), buf(start_pos)[0], int(batch), qp, qb, op, ob, int(n_head), int(head_dim),
            int(plan[1]), wp, wb, buf(k_scale)[0], buf(v_scale)[0]))
