"""Causal chunked prefill on gfx950 -- the engine-cuda `FlashAttention2` surface.

Mirrors engine-cuda/src/flash_attention.rs:20-225: `launch` (host
pos_offset) and `launch_with_pos_ptr` (device position, for graph replay) with
the reference's argument order and size checks, plus `launch_batched` for a
ragged batch of chunks in one launch.  The pool's element type is an extra
keyword (`kv_dtype`, default F32 as in the reference).  QK^T and PV run on
MFMA tiles.
"""
from . import _lib
from .errors import check
from .paged_kv import KvDataType
from .runtime import buf, context, stream_handle

SUPPORTED_HEAD_DIMS = (64, 128)


class FlashAttention2:
    """engine-cuda/src/flash_attention.rs:20-225 on a HIP code object."""

    def __init__(self, device=0):
        self._ctx = context(device)
        self._L = _lib.load()

    def launch(self, stream, q, pool, block_table, out, n_head, n_head_kv, head_dim,
               block_tokens, q_tokens, pos_offset, kv_dtype=KvDataType.F32):
        """flash_attention.rs:95-125"""
        self.launch_with_pos_ptr(stream, q, pool, block_table, out, n_head, n_head_kv, head_dim,
                                 block_tokens, q_tokens, pos_offset, None, kv_dtype)

    def launch_with_pos_ptr(self, stream, q, pool, block_table, out, n_head, n_head_kv, head_dim,
                            block_tokens, q_tokens, pos_offset, pos_ptr,
                            kv_dtype=KvDataType.F32):
        """flash_attention.rs:128-225: a device u32 at pos_ptr overrides pos_offset."""
        qp, qb = buf(q)
        pp, pb = buf(pool)
        bp, bb = buf(block_table)
        op, ob = buf(out)
        check(self._L.eh_flash_attention_prefill(
            self._ctx.handle, stream_handle(stream), int(kv_dtype), qp, qb, pp, pb, bp, bb, op, ob,
            int(n_head), int(n_head_kv), int(head_dim), int(block_tokens), int(q_tokens),
            int(pos_offset), buf(pos_ptr)[0]))

    def launch_batched(self, stream, q, pool, block_tables, cu_q, start_pos, out, n_head,
                       n_head_kv, head_dim, block_tokens, max_q_tokens, kv_dtype=KvDataType.F32):
        """q/out [total, n_head, head_dim] f32; block_tables [B, stride] u32;
        cu_q [B+1] and start_pos [B] u32 device tensors; max_q_tokens bounds
        every chunk length."""
        batch, stride = block_tables.shape
        total = q.shape[0]
        qp, qb = buf(q)
        pp, pb = buf(pool)
        bp, bb = buf(block_tables)
        op, ob = buf(out)
        check(self._L.eh_prefill_batched(
            self._ctx.handle, stream_handle(stream), int(kv_dtype), qp, qb, pp, pb, bp, bb,
            int(stride), buf(cu_q)[0], buf(start_pos)[0], int(batch), int(max_q_tokens),
            int(total), op, ob, int(n_head), int(n_head_kv), int(head_dim), int(block_tokens)))

    def launch_batched_e4m3(self, stream, q, pool, block_tables, cu_q, start_pos, out, n_head,
                            n_head_kv, head_dim, block_tokens, max_q_tokens, k_scale, v_scale):
        """launch_batched over an E4M3 pool with per-kv-head f32 scales
        (k_scale / v_scale [n_head_kv] device tensors): attention on
        decode(code) * scale."""
        batch, stride = block_tables.shape
        total = q.shape[0]
        qp, qb = buf(q)
        pp, pb = buf(pool)
        bp, bb = buf(block_tables)
        op, ob = buf(out)
        check(self._L.eh_prefill_batched_e4m3(
            self._ctx.handle, stream_handle(stream), qp, qb, pp, pb, bp, bb, int(stride),
            buf(cu_q)[0], buf(start_pos)[0], int(batch), int(max_q_tokens), int(total), op, ob,
            int(n_head), int(n_head_kv), int(head_dim), int(block_tokens), buf(k_scale)[0],
            buf(v_scale)[0]))
