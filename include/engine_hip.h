/*
 * engine_hip.h -- C-ABI of the MI355X (gfx950) paged KV-cache hot path.
 *
 * Drop-in replacement for Titan's engine-cuda paged-KV / paged-attention /
 * flash-attention launchers (NVRTC + cuLaunchKernel) with offline-compiled
 * gfx950 code objects loaded by hipModuleLoad and launched by
 * hipModuleLaunchKernel.  Each entry point names the reference interface it
 * replaces (paths relative to the reference root).
 *
 * Conventions (engine-cuda/src/{paged_kv,paged_attention}.rs):
 *   - the caller owns every device buffer and passes (pointer, size in bytes);
 *     sizes are validated exactly as the reference validates DeviceBuffer
 *     sizes and a short buffer yields EH_INVALID_SIZE with expected/actual;
 *   - launches are asynchronous on the caller's stream (hipStream_t, 0 = null
 *     stream), never synchronise the host and never allocate device memory;
 *   - an optional device `pos_ptr` (uint32) overrides the host position so a
 *     captured graph can be replayed as the position advances;
 *   - n_tokens == 0 is success;
 *   - the failing call's detail is kept per thread (eh_last_error).
 */
#ifndef TITAN_ENGINE_HIP_H
#define TITAN_ENGINE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct eh_context eh_context;
typedef void* eh_stream; /* hipStream_t */

/* One code per CudaError / KvCacheError variant
 * (engine-cuda/src/error.rs:6-50, engine-kvcache/src/error.rs:4-16). */
typedef enum eh_status {
    EH_OK = 0,
    EH_INVALID_SIZE = 1,   /* CudaError::InvalidSize{expected, actual} */
    EH_KERNEL_LOAD = 2,    /* CudaError::KernelLoad(site, code) */
    EH_KERNEL_LAUNCH = 3,  /* CudaError::KernelLaunch(site, code) */
    EH_ALLOC_FAILED = 4,   /* CudaError::AllocFailed */
    EH_STREAM_FAILED = 5,  /* CudaError::StreamFailed */
    EH_MEMCPY_FAILED = 6,  /* CudaError::MemcpyFailed */
    EH_EVENT_FAILED = 7,   /* CudaError::EventFailed */
    EH_GRAPH_FAILED = 8,   /* CudaError::GraphFailed */
    EH_DRIVER = 9,         /* CudaError::Driver (device selection etc.) */
    EH_POOL_EXHAUSTED = 20,/* KvCacheError::PoolExhausted{blocks_used, blocks_total} */
    EH_INVALID_ARGS = 21,  /* KvCacheError::InvalidArgs(msg) */
    EH_UNSUPPORTED = 30    /* shape outside the compiled kernel set (no reference counterpart) */
} eh_status;

/* KvDataType (engine-cuda/src/paged_kv.rs:36-52) plus BF16 (extension). */
typedef enum eh_kv_dtype { EH_KV_F32 = 0, EH_KV_F16 = 1, EH_KV_FP8 = 2, EH_KV_BF16 = 3 } eh_kv_dtype;

/* PagedKvLayout (engine-cuda/src/paged_kv.rs:55-102), 64-bit fields. */
typedef struct eh_kv_layout {
    uint64_t n_blocks;
    uint64_t block_tokens;
    uint64_t row_len;    /* n_kv_heads * head_dim elements */
    uint32_t data_type;  /* eh_kv_dtype */
    uint32_t reserved;
} eh_kv_layout;

/* ---- context: PagedKvGpu::new / PagedAttention::new / FlashAttention2::new
 *      (paged_kv.rs:122-196, paged_attention.rs:58-134, flash_attention.rs:44-93).
 * Loads the gfx950 code objects from code_object_dir (NULL = the directory
 * of this library) and allocates the split-K scratch once. */
eh_status eh_create(int device, const char* code_object_dir, eh_context** out);
/* Drop for all three (paged_kv.rs:478-491): unloads modules, frees scratch.
 * Work launched through ctx must have completed, and no HIP graph captured
 * with its launches may be replayed afterwards: the graph's kernel nodes
 * point into the unloaded code objects. */
void eh_destroy(eh_context* ctx);
/* Detail of this thread's last failure: expected/actual for InvalidSize and
 * PoolExhausted (blocks_used/blocks_total), the site string, the HIP code. */
eh_status eh_last_error(uint64_t* expected, uint64_t* actual, const char** site, int* hip_code);
const char* eh_status_name(eh_status s);
/* PagedKvLayout::{element_bytes, bytes_total} (paged_kv.rs:45-51, 94-96). */
uint64_t eh_kv_element_bytes(uint32_t data_type);
uint64_t eh_kv_layout_bytes_total(const eh_kv_layout* layout);

/* ---- PagedKvGpu::append_kv / append_kv_with_pos_ptr (paged_kv.rs:200-327).
 * keys/values: [n_tokens, row_len] in the pool's element type. */
eh_status eh_append_kv(eh_context* ctx, eh_stream stream, const eh_kv_layout* layout,
                       void* pool, uint64_t pool_bytes, const void* keys, uint64_t keys_bytes,
                       const void* values, uint64_t values_bytes, const uint32_t* block_table,
                       uint64_t bt_bytes, uint64_t start_token, uint64_t n_tokens,
                       const uint32_t* pos_ptr);

/* ---- PagedKvGpu::read_keys / read_values (paged_kv.rs:331-470). */
eh_status eh_gather_kv(eh_context* ctx, eh_stream stream, const eh_kv_layout* layout,
                       const void* pool, uint64_t pool_bytes, const uint32_t* block_table,
                       uint64_t bt_bytes, void* out, uint64_t out_bytes, uint64_t start_token,
                       uint64_t n_tokens, int is_value);

/* ---- Batched append (extension of paged_kv.rs:200 for B sequences):
 * token i of the ragged batch belongs to sequence b with
 * cu_seqlens[b] <= i < cu_seqlens[b+1] and lands at logical position
 * start_pos[b] + i - cu_seqlens[b] through block_tables + b*bt_stride.
 * cu_seqlens [batch+1], start_pos [batch] and block_tables are device arrays. */
eh_status eh_append_kv_batched(eh_context* ctx, eh_stream stream, const eh_kv_layout* layout,
                               void* pool, uint64_t pool_bytes, const void* keys,
                               uint64_t keys_bytes, const void* values, uint64_t values_bytes,
                               const uint32_t* block_tables, uint64_t bt_bytes, uint32_t bt_stride,
                               const uint32_t* cu_seqlens, const uint32_t* start_pos,
                               uint32_t batch, uint64_t total_tokens);

/* ---- FP8 (E4M3) KV storage (extension: the FP8 KV format of
 * openspec/archive/2026-08-28-fp8-kv-cache-quantization/design.md:3-6 and
 * specs/kv-compression/spec.md:8-10, which no reference kernel implements).
 * Codes are OCP E4M3FN (bias 7, no infinities, S.1111.111 = NaN, max 448);
 * each kv head has one f32 scale for K and one for V (device arrays
 * k_scale/v_scale [row_len / head_dim]): element e of a row stores
 * quantize(x / scale[e / head_dim]) -- round to nearest, ties to even,
 * |x| >= 448 and infinities saturate to +-448, NaN stays NaN -- and reads back
 * as decode(code) * scale.  layout->data_type must be EH_KV_FP8; head_dim a
 * multiple of 4.
 *
 * Quantising batched append (PagedKvGpu::append_kv, paged_kv.rs:200-327, for
 * B sequences as eh_append_kv_batched): keys/values [total_tokens, row_len] f32. */
eh_status eh_append_kv_e4m3_batched(eh_context* ctx, eh_stream stream, const eh_kv_layout* layout,
                                    void* pool, uint64_t pool_bytes, const float* keys,
                                    uint64_t keys_bytes, const float* values, uint64_t values_bytes,
                                    const uint32_t* block_tables, uint64_t bt_bytes,
                                    uint32_t bt_stride, const uint32_t* cu_seqlens,
                                    const uint32_t* start_pos, uint32_t batch,
                                    uint64_t total_tokens, uint32_t head_dim,
                                    const float* k_scale, const float* v_scale);
/* Dynamic per-head scales for the E4M3 pool (extension: the "dynamic
 * per-head scaling factors" of specs/kv-compression/spec.md:9, one f32 scale
 * per head as design.md:5 allows), computed on the device from f32 rows
 * keys/values [n_rows, row_len] (a prompt, or a calibration sample):
 * k_scale[h] = max(amax / 448, FLT_MIN), amax = the largest finite |x| of
 * head h's K elements (inf and NaN ignored), 1 for a head with no finite
 * nonzero element; v_scale likewise from values.  448 is E4M3's largest
 * value, so the rows measured use the whole code range; later rows beyond
 * it saturate.  The scales are the device arrays every E4M3 entry point
 * reads; one launch, nothing allocated. */
eh_status eh_kv_e4m3_scales(eh_context* ctx, eh_stream stream, const eh_kv_layout* layout,
                            const float* keys, uint64_t keys_bytes, const float* values,
                            uint64_t values_bytes, uint64_t n_rows, uint32_t head_dim,
                            float* k_scale, uint64_t k_scale_bytes, float* v_scale,
                            uint64_t v_scale_bytes);
/* Dequantising read (PagedKvGpu::read_keys / read_values, paged_kv.rs:331-470,
 * of an FP8 pool): out [n_tokens, row_len] f32; `scale` is k_scale or v_scale. */
eh_status eh_gather_kv_e4m3(eh_context* ctx, eh_stream stream, const eh_kv_layout* layout,
                            const void* pool, uint64_t pool_bytes, const uint32_t* block_table,
                            uint64_t bt_bytes, float* out, uint64_t out_bytes, uint64_t start_token,
                            uint64_t n_tokens, int is_value, uint32_t head_dim, const float* scale);

/* ---- Page copies dst_ids[k] <- src_ids[k] (device arrays): copy-on-write
 * of a shared tail page (the copy_block_gpu step sketched for
 * CowBlockTable::perform_tail_cow, engine-kvcache/src/cow.rs:73-81) and
 * gather-compaction of surviving pages.  Pairs with src == dst are skipped;
 * destinations must not also be sources. */
eh_status eh_copy_pages(eh_context* ctx, eh_stream stream, const eh_kv_layout* layout,
                        void* pool, uint64_t pool_bytes, const uint32_t* src_ids,
                        const uint32_t* dst_ids, uint32_t n_pairs);

/* ---- Block-table rewrite after compaction: e = remap[e] for e < n_remap. */
eh_status eh_remap_block_tables(eh_context* ctx, eh_stream stream, uint32_t* block_tables,
                                uint64_t n_entries, const uint32_t* remap, uint32_t n_remap);

/* ---- Page reference counts (Arc::strong_count of SharedBlock, cow.rs:56-61,
 * counted over device block tables): counts[p] = number of entries j <
 * n_used[b] of rows b equal to p.  counts [n_blocks] is overwritten. */
eh_status eh_page_refcounts(eh_context* ctx, eh_stream stream, const uint32_t* block_tables,
                            uint32_t bt_stride, const uint32_t* n_used, uint32_t batch,
                            uint32_t* counts, uint32_t n_blocks);

/* ---- PagedAttention::launch / launch_with_pos_ptr (paged_attention.rs:143-345):
 * decode for one sequence; q/out [n_head, head_dim] f32, pool in kv_dtype.
 * Validation follows paged_attention.rs:193-257.  One pass per kv head when
 * the context fits one split, otherwise the split-K path of
 * eh_flash_decoding (same result within rounding). */
eh_status eh_paged_attention(eh_context* ctx, eh_stream stream, uint32_t kv_dtype,
                             const float* q, uint64_t q_bytes, const void* pool,
                             uint64_t pool_bytes, const uint32_t* block_table, uint64_t bt_bytes,
                             float* out, uint64_t out_bytes, uint64_t n_head, uint64_t n_head_kv,
                             uint64_t head_dim, uint64_t block_tokens, uint64_t seq_tokens,
                             uint64_t query_pos, int causal, const uint32_t* pos_ptr);

/* ---- PagedAttention::launch_flash_decoding (paged_attention.rs:352-490):
 * split-K decode using the context's scratch.  Unlike the reference, every
 * token is attended (no 32-split cap) and the split count follows the
 * device-side position when pos_ptr is given (grid sized from the block
 * table's capacity).  Calls sharing one context must not overlap in time
 * (eh_flash_decoding_ws takes a workspace of its own instead). */
eh_status eh_flash_decoding(eh_context* ctx, eh_stream stream, uint32_t kv_dtype,
                            const float* q, uint64_t q_bytes, const void* pool,
                            uint64_t pool_bytes, const uint32_t* block_table, uint64_t bt_bytes,
                            float* out, uint64_t out_bytes, uint64_t n_head, uint64_t n_head_kv,
                            uint64_t head_dim, uint64_t block_tokens, uint64_t seq_tokens,
                            uint64_t query_pos, int causal, const uint32_t* pos_ptr);
/* Single-sequence decode step in one launch (extension: PagedKvGpu::append_kv
 * / append_kv_with_pos_ptr, paged_kv.rs:200-327, of one token followed by
 * launch_flash_decoding, paged_attention.rs:352-490): keys/values [row_len]
 * (pool element type) are written at position p = *pos_ptr (device) or
 * query_pos, then q attends tokens 0..p.  Pool bytes after the call equal
 * the append's, the output equals eh_flash_decoding's with seq_tokens = p + 1,
 * query_pos = p, causal.  16-bit and f32 pages; FP8 returns EH_UNSUPPORTED.
 * Masked page: a host query_pos whose page lies past the table is
 * EH_INVALID_SIZE.  With pos_ptr, a position whose table entry lies past the
 * table or whose page id is >= the pool's pages is masked like every other
 * token on such a page: the row is NOT written, the call returns EH_OK and q
 * attends only the tokens on valid pages (the same masking eh_flash_decoding
 * applies). */
eh_status eh_append_flash_decoding(eh_context* ctx, eh_stream stream, uint32_t kv_dtype,
                                   const void* keys, uint64_t keys_bytes, const void* values,
                                   uint64_t values_bytes, const float* q, uint64_t q_bytes,
                                   void* pool, uint64_t pool_bytes, const uint32_t* block_table,
                                   uint64_t bt_bytes, float* out, uint64_t out_bytes,
                                   uint64_t n_head, uint64_t n_head_kv, uint64_t head_dim,
                                   uint64_t block_tokens, uint64_t query_pos,
                                   const uint32_t* pos_ptr);

/* ---- The three single-sequence calls above with a caller-owned workspace
 * (extension): the split-K partials go to `workspace` instead of the
 * context's scratch, so calls on different streams may overlap in time (one
 * workspace per concurrent call).  Arguments and results are those of the
 * call without _ws.  The split grows until its partials fit workspace_bytes;
 * eh_single_decode_workspace_bytes() (the context scratch's size) always
 * suffices, and a context that fits one pass needs none (0 bytes).  A
 * workspace too small for the longest split is EH_INVALID_SIZE (expected =
 * the least that fits).  16-byte aligned. */
uint64_t eh_single_decode_workspace_bytes(void);
eh_status eh_paged_attention_ws(eh_context* ctx, eh_stream stream, uint32_t kv_dtype,
                                const float* q, uint64_t q_bytes, const void* pool,
                                uint64_t pool_bytes, const uint32_t* block_table,
                                uint64_t bt_bytes, float* out, uint64_t out_bytes,
                                uint64_t n_head, uint64_t n_head_kv, uint64_t head_dim,
                                uint64_t block_tokens, uint64_t seq_tokens, uint64_t query_pos,
                                int causal, const uint32_t* pos_ptr, void* workspace,
                                uint64_t workspace_bytes);
eh_status eh_flash_decoding_ws(eh_context* ctx, eh_stream stream, uint32_t kv_dtype,
                               const float* q, uint64_t q_bytes, const void* pool,
                               uint64_t pool_bytes, const uint32_t* block_table, uint64_t bt_bytes,
                               float* out, uint64_t out_bytes, uint64_t n_head, uint64_t n_head_kv,
                               uint64_t head_dim, uint64_t block_tokens, uint64_t seq_tokens,
                               uint64_t query_pos, int causal, const uint32_t* pos_ptr,
                               void* workspace, uint64_t workspace_bytes);
eh_status eh_append_flash_decoding_ws(eh_context* ctx, eh_stream stream, uint32_t kv_dtype,
                                      const void* keys, uint64_t keys_bytes, const void* values,
                                      uint64_t values_bytes, const float* q, uint64_t q_bytes,
                                      void* pool, uint64_t pool_bytes,
                                      const uint32_t* block_table, uint64_t bt_bytes, float* out,
                                      uint64_t out_bytes, uint64_t n_head, uint64_t n_head_kv,
                                      uint64_t head_dim, uint64_t block_tokens, uint64_t query_pos,
                                      const uint32_t* pos_ptr, void* workspace,
                                      uint64_t workspace_bytes);

/* ---- Batched decode (extension: B sequences in one launch).
 * eh_decode_plan picks the kernel and its launch shape for contexts up to
 * max_ctx, and the workspace size the call needs:
 *   - hint 0 on a shape the token-balanced kernel serves (16-bit KV,
 *     head_dim 128, 1/2/4/8 kv heads, at most 8 q heads per kv head,
 *     power-of-two pages of at least 16 tokens, batch <= 2048):
 *     tokens_per_split = 0 and max_splits = the grid (workgroups); the device
 *     cuts the batch's 16-token tiles evenly among them from the live
 *     lengths, so any context lengths are served (max_ctx is not a bound);
 *     q enters its MFMAs as hi + lo 16-bit halves, so over f16 (and E4M3)
 *     pages q's elements must stay below ~5e5 in magnitude (|q| log2(e) /
 *     sqrt(128) within f16's 65504);
 *   - otherwise fixed splits: tokens_per_split (hint rounded up to the
 *     kernel's split granularity -- one round of its four waves, 8 to 256
 *     tokens, for the per-token kernel -- or automatic; at most
 *     1022 * block_tokens) and the split bound max_splits (at most 256). */
eh_status eh_decode_plan(uint32_t kv_dtype, uint32_t batch, uint32_t n_head, uint32_t n_head_kv,
                         uint32_t head_dim, uint32_t block_tokens, uint32_t max_ctx,
                         uint32_t tokens_per_split_hint, uint32_t* tokens_per_split,
                         uint32_t* max_splits, uint64_t* workspace_bytes);
/* Workspace bytes of a token-balanced decode call launched with `grid`
 * workgroups, for callers that pass a grid of their own instead of the
 * plan's to the calls taking one (eh_append_decode_batched[_e4m3],
 * eh_decode_schedule / eh_append_decode_scheduled, and max_splits of the
 * batched decodes): 4 * (grid + batch) * n_head * 130, the partial states of
 * every run plus one per sequence, or UINT64_MAX where that does not fit
 * 64 bits (no reference counterpart). */
uint64_t eh_decode_grid_workspace_bytes(uint32_t grid, uint32_t batch, uint32_t n_head);
/* Name of the split kernel eh_paged_decode_batched launches for a shape
 * (diagnostics and profiling; no reference counterpart). */
eh_status eh_decode_kernel_name(uint32_t kv_dtype, uint32_t n_head, uint32_t n_head_kv,
                                uint32_t head_dim, uint32_t block_tokens, char* buf, uint64_t size);
/* q/out [batch, n_head, head_dim] f32; block_tables [batch, bt_stride] u32;
 * ctx_lens [batch] u32 = tokens each query attends (its own position + 1;
 * with fixed splits each at most tokens_per_split * max_splits).  workspace,
 * tokens_per_split and max_splits come from eh_decode_plan; calls sharing one
 * workspace must not overlap in time.  Runs one split kernel and one
 * log-sum-exp merge kernel (fixed splits: only when max_splits > 1). */
eh_status eh_paged_decode_batched(eh_context* ctx, eh_stream stream, uint32_t kv_dtype,
                                  const float* q, uint64_t q_bytes, const void* pool,
                                  uint64_t pool_bytes, const uint32_t* block_tables,
                                  uint64_t bt_bytes, uint32_t bt_stride, const uint32_t* ctx_lens,
                                  uint32_t batch, float* out, uint64_t out_bytes, uint32_t n_head,
                                  uint32_t n_head_kv, uint32_t head_dim, uint32_t block_tokens,
                                  uint32_t tokens_per_split, uint32_t max_splits, void* workspace,
                                  uint64_t workspace_bytes);

/* ---- Batched decode over an E4M3 pool (extension; format and scales as
 * eh_append_kv_e4m3_batched): eh_paged_decode_batched's semantics on the
 * dequantised pool, decode(code) * scale.  Shapes of the token-balanced kernel
 * only: eh_decode_plan(EH_KV_FP8, ..., hint 0) gives max_splits (the grid) and
 * the workspace size. */
eh_status eh_paged_decode_batched_e4m3(eh_context* ctx, eh_stream stream, const float* q,
                                       uint64_t q_bytes, const void* pool, uint64_t pool_bytes,
                                       const uint32_t* block_tables, uint64_t bt_bytes,
                                       uint32_t bt_stride, const uint32_t* ctx_lens, uint32_t batch,
                                       float* out, uint64_t out_bytes, uint32_t n_head,
                                       uint32_t n_head_kv, uint32_t head_dim, uint32_t block_tokens,
                                       const float* k_scale, const float* v_scale,
                                       uint32_t max_splits, void* workspace, uint64_t workspace_bytes);

/* ---- Batched decode over the protected-sinks range (extension: the
 * attention-sinks + sliding-window rule of openspec/specs/protected-kv-sinks/
 * spec.md:9-15 and openspec/changes/archive/
 * 2026-08-28-agent-runtime-optimizations/design.md:211-216, which the
 * reference's paged_attention.cu does not implement): the query at
 * pos = ctx_lens[b] - 1 attends tokens [0, sink_tokens) and
 * [max(sink_tokens, pos - window_tokens), pos]; window_tokens 0 attends all.
 * Only the tiles holding attended tokens are read and the work split counts
 * only those.  kv_dtype EH_KV_F16 / EH_KV_BF16 (scales NULL) or EH_KV_FP8
 * (k_scale / v_scale as eh_append_kv_e4m3_batched); token-balanced shapes,
 * max_splits and workspace from eh_decode_plan with hint 0.
 * block_mass (optional, [pool pages] f32, block_mass_bytes >= 4 * pages):
 * += each page's attention mass, the softmax weights of its attended tokens
 * summed over the q heads -- the H2O score that
 * StreamingKvManager::record_attention_mass adds per block
 * (engine-kvcache/src/streaming.rs:135-141); pages shared by several
 * sequences get one addition from each, in any order.  It needs
 * eh_decode_mass_workspace_bytes more workspace (after the plan's) and
 * block_tokens a multiple of 16, and adds a third launch. */
eh_status eh_paged_decode_batched_window(eh_context* ctx, eh_stream stream, uint32_t kv_dtype,
                                         const float* q, uint64_t q_bytes, const void* pool,
                                         uint64_t pool_bytes, const uint32_t* block_tables,
                                         uint64_t bt_bytes, uint32_t bt_stride,
                                         const uint32_t* ctx_lens, uint32_t batch, float* out,
                                         uint64_t out_bytes, uint32_t n_head, uint32_t n_head_kv,
                                         uint32_t head_dim, uint32_t block_tokens,
                                         uint32_t sink_tokens, uint32_t window_tokens,
                                         const float* k_scale, const float* v_scale,
                                         float* block_mass, uint64_t block_mass_bytes,
                                         uint32_t max_splits, void* workspace,
                                         uint64_t workspace_bytes);
/* Extra workspace bytes eh_paged_decode_batched_window needs with block_mass
 * (no reference counterpart). */
uint64_t eh_decode_mass_workspace_bytes(uint32_t batch, uint32_t bt_stride, uint32_t block_tokens,
                                        uint32_t n_head);

/* ---- Fused decode-step append + attention (extension: the batched
 * PagedKvGpu::append_kv of paged_kv.rs:200-327 -- in production the decode
 * append slot of NormRope::launch_fused_qk, norm_rope.cu:280-298 -- followed
 * by PagedAttention::launch_with_pos_ptr, paged_attention.rs:177-345, for B
 * sequences in ONE launch of the token-balanced kernel).  Row b of
 * keys/values [batch, row_len] (pool element type) is written at logical
 * position start_pos[b] (device u32) through block_tables + b*bt_stride,
 * then q row b attends tokens 0..start_pos[b] inclusive.  Pool bytes after
 * the call equal eh_append_kv_batched's; the output equals
 * eh_paged_decode_batched's with ctx_lens = start_pos + 1.  Shapes: those of
 * the token-balanced kernel (eh_decode_plan with hint 0 returns
 * tokens_per_split 0; its max_splits is `grid` and its workspace size
 * applies); other shapes return EH_UNSUPPORTED.  The appended page must not
 * be read by another sequence of the same call (copy-on-write first).
 * Masked page: when start_pos[b] / block_tokens >= bt_stride, or the table
 * entry is 0xFFFFFFFF or >= the pool's pages, row b is NOT written and q row
 * b attends only the tokens on valid pages (EH_OK; eh_paged_decode_batched
 * masks such pages the same way). */
eh_status eh_append_decode_batched(eh_context* ctx, eh_stream stream, const eh_kv_layout* layout,
                                   void* pool, uint64_t pool_bytes, const void* keys,
                                   uint64_t keys_bytes, const void* values, uint64_t values_bytes,
                                   const uint32_t* block_tables, uint64_t bt_bytes,
                                   uint32_t bt_stride, const uint32_t* start_pos, uint32_t batch,
                                   const float* q, uint64_t q_bytes, float* out, uint64_t out_bytes,
                                   uint32_t n_head, uint32_t head_dim, uint32_t grid,
                                   void* workspace, uint64_t workspace_bytes);
/* ---- Decode step schedule (extension): the layers of one decode step share
 * one block table and one set of positions (the reference passes one bt_dev
 * to every layer, engine-core/src/forward_driver.rs:2230-2243), so the
 * token-balanced work split -- which pages each run reads, which sequence
 * each tile belongs to, which runs hold each sequence -- is computed once per
 * step by eh_decode_schedule and read by every layer's
 * eh_append_decode_scheduled, instead of each layer's launch deriving it
 * from the lengths and tables again.  The schedule is device-side: a
 * captured graph that rebuilds it each step stays correct as contexts grow.
 *
 * Bytes of a schedule for batch sequences, bt_stride table entries each and
 * grid runs (grid = max_splits of eh_decode_plan with hint 0). */
uint64_t eh_decode_schedule_bytes(uint32_t batch, uint32_t bt_stride, uint32_t block_tokens,
                                  uint32_t grid);
/* Builds the schedule from block_tables [batch, bt_stride] and the lengths
 * lens[b] + lens_add (lens_add = 1 with the positions a fused step appends
 * at) for a pool of layout->n_blocks pages of layout->block_tokens tokens
 * (a power of two, >= 16).  Tiles the table cannot address are dropped
 * (their tokens are masked in every decode form).  One launch. */
eh_status eh_decode_schedule(eh_context* ctx, eh_stream stream, const eh_kv_layout* layout,
                             const uint32_t* block_tables, uint64_t bt_bytes, uint32_t bt_stride,
                             const uint32_t* lens, uint32_t lens_add, uint32_t batch, uint32_t grid,
                             void* sched, uint64_t sched_bytes);
/* One layer's decode step from a schedule (extension: eh_append_decode_batched
 * / eh_append_decode_batched_e4m3 with the work split read from `sched`
 * rather than derived from the lengths): row b of keys/values is written at
 * the position the schedule was built with (lens[b] when lens_add = 1) and q
 * row b attends the schedule's tokens of sequence b.  keys = values = NULL
 * skips the append (a decode over a schedule built with lens_add = 0, as
 * eh_paged_decode_batched / eh_paged_decode_batched_e4m3).  E4M3 pages take
 * f32 rows and both scales.  layout, bt_stride, batch and grid must be those
 * the schedule was built with; the pool may differ per layer (same layout).
 * Outputs equal the self-scheduled forms'; workspace as eh_decode_plan.  The
 * schedule and the workspace must be 16-byte aligned (EH_INVALID_ARGS).
 * keys/values with a schedule built with lens_add = 0 are not appended (the
 * schedule's last tiles hold existing tokens, which the append would
 * overwrite): the pool is left unchanged and q attends the schedule's
 * tokens.  A schedule built for other shapes is not detected: the kernels
 * still stay inside the pool, q, out and the workspace, but the results are
 * unspecified. */
eh_status eh_append_decode_scheduled(eh_context* ctx, eh_stream stream, const eh_kv_layout* layout,
                                     void* pool, uint64_t pool_bytes, const void* keys,
                                     uint64_t keys_bytes, const void* values,
                                     uint64_t values_bytes, const void* sched,
                                     uint64_t sched_bytes, uint32_t bt_stride, uint32_t batch,
                                     const float* q, uint64_t q_bytes, float* out,
                                     uint64_t out_bytes, uint32_t n_head, uint32_t head_dim,
                                     uint32_t grid, void* workspace, uint64_t workspace_bytes,
                                     const float* k_scale, const float* v_scale);

/* ---- Measurement aid (no counterpart in the reference): the read ceiling
 * of a paged decode.  Streams the n_ids pages listed in ids (page ids of the
 * pool described by layout; page bytes a multiple of 16 KiB) once, in list
 * order, with grid workgroups of 8 waves, each wave taking an equal
 * contiguous share of the pages' 16 KiB items and keeping depth (1 or 2)
 * items in flight; every word read is folded into one xor per wave, written
 * to out[grid * 8] (4 bytes per wave, nothing else is written).  Timing it
 * over a decode's page list gives the cold-read floor the decode is
 * measured against.  Ids past the pool are skipped. */
eh_status eh_stream_pages(eh_context* ctx, eh_stream stream, const eh_kv_layout* layout,
                          const void* pool, uint64_t pool_bytes, const uint32_t* ids,
                          uint64_t ids_bytes, uint32_t n_ids, uint32_t depth, uint32_t grid,
                          uint32_t* out, uint64_t out_bytes);
/* Measurement aid (no counterpart in the reference): the same read in the
 * token-balanced decode's access pattern, one wave per kv head.  The page
 * list is cut into equal contiguous ranges, one per group of n_kv waves
 * (n_kv = row_len / head_dim: 1, 2, 4 or 8); wave h of a group reads only kv
 * head h's K and V rows of each page, two pages in flight, as the decode's
 * waves of one run do.  Pages of 16 tokens and kv head rows of 256 bytes
 * (head_dim * element bytes); out as eh_stream_pages (grid * 8 words, the
 * xor of every word each wave read). */
eh_status eh_stream_pages_heads(eh_context* ctx, eh_stream stream, const eh_kv_layout* layout,
                                const void* pool, uint64_t pool_bytes, const uint32_t* ids,
                                uint64_t ids_bytes, uint32_t n_ids, uint32_t head_dim,
                                uint32_t grid, uint32_t* out, uint64_t out_bytes);

/* ---- eh_append_decode_batched without a workspace argument, for callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  No reference counterpart.
 * Same arguments and results as eh_append_decode_batched; the partial states
 * live in a 32 MiB scratch array that the library holds on every GPU it runs
 * on until the process ends.  Shapes whose partials need more
 * (4 * (grid + batch) * n_head * 130 bytes > 32 MiB) return EH_INVALID_SIZE
 * (expected = the limit, actual = the need) before any launch.  The call
 * allocates nothing; all calls on one GPU share its scratch, so calls that
 * overlap in time on one GPU (two streams, two threads) race. */
eh_status eh_append_decode_batched_noalloc(eh_context* ctx, eh_stream stream,
                                          const eh_kv_layout* layout, void* pool,
                                          uint64_t pool_bytes, const void* keys,
                                          uint64_t keys_bytes, const void* values,
                                          uint64_t values_bytes, const uint32_t* block_tables,
                                          uint64_t bt_bytes, uint32_t bt_stride,
                                          const uint32_t* start_pos, uint32_t batch,
                                          const float* q, uint64_t q_bytes, float* out,
                                          uint64_t out_bytes, uint32_t n_head, uint32_t head_dim,
                                          uint32_t grid);
/* The same fused decode step over E4M3 pages (extension: the quantising
 * append of eh_append_kv_e4m3_batched, then eh_paged_decode_batched_e4m3, in
 * one launch): keys/values [batch, row_len] f32 are quantised in the launch
 * (code = quantize(x / scale) with k_scale / v_scale [n_head_kv], as the
 * append); pool bytes after the call equal eh_append_kv_e4m3_batched's and
 * the output equals eh_paged_decode_batched_e4m3's with ctx_lens =
 * start_pos + 1.  layout->data_type must be EH_KV_FP8. */
eh_status eh_append_decode_batched_e4m3(eh_context* ctx, eh_stream stream,
                                        const eh_kv_layout* layout, void* pool, uint64_t pool_bytes,
                                        const float* keys, uint64_t keys_bytes, const float* values,
                                        uint64_t values_bytes, const uint32_t* block_tables,
                                        uint64_t bt_bytes, uint32_t bt_stride,
                                        const uint32_t* start_pos, uint32_t batch, const float* q,
                                        uint64_t q_bytes, float* out, uint64_t out_bytes,
                                        uint32_t n_head, uint32_t head_dim, uint32_t grid,
                                        void* workspace, uint64_t workspace_bytes,
                                        const float* k_scale, const float* v_scale);

/* ---- FlashAttention2::launch / launch_with_pos_ptr (flash_attention.rs:95-225):
 * causal chunked prefill.  q/out [q_tokens, n_head, head_dim] f32; query i
 * sits at position p0 + i (p0 = *pos_ptr when given, else pos_offset) and
 * attends keys 0..=p0+i through the block table (flash_attention_2.cu:44-68);
 * a row with no valid key is zero.  Size checks follow
 * flash_attention.rs:142-164 (q, out, ceil((pos_offset+q_tokens)/block_tokens)
 * table entries).  QK^T and PV run on MFMA: f16 KV with f16 operands (q as
 * hi + lo f16 halves for the scores); bf16 KV widened to f16 as it is staged
 * (exact below 2^16), a tile holding a larger value on bf16 MFMAs with hi + lo
 * bf16 operand pairs; f32 KV with f32 MFMA.  head_dim 64 or 128.  Keys whose
 * block-table entry lies past the table or past the pool are masked.  bf16
 * pages run the ping-pong kernel (the workgroup's halves alternate MFMA and
 * softmax phases), the other types the single-phase kernel; at head_dim 128
 * both give bit-identical outputs.  The environment variable
 * EH_PREFILL_KERNEL=single or =pp, read at each call, overrides that choice
 * for 16-bit and E4M3 pages (a diagnostic). */
eh_status eh_flash_attention_prefill(eh_context* ctx, eh_stream stream, uint32_t kv_dtype,
                                     const float* q, uint64_t q_bytes, const void* pool,
                                     uint64_t pool_bytes, const uint32_t* block_table,
                                     uint64_t bt_bytes, float* out, uint64_t out_bytes,
                                     uint64_t n_head, uint64_t n_head_kv, uint64_t head_dim,
                                     uint64_t block_tokens, uint64_t q_tokens,
                                     uint64_t pos_offset, const uint32_t* pos_ptr);

/* ---- Batched chunked prefill (extension of flash_attention.rs:95 for B
 * sequences in one launch): rows cu_q[b] .. cu_q[b+1] of q/out
 * [total_q_tokens, n_head, head_dim] belong to sequence b, whose first query
 * sits at position start_pos[b], through block_tables + b*bt_stride.
 * cu_q [batch+1] and start_pos [batch] are device arrays; max_q_tokens must
 * be >= every cu_q[b+1]-cu_q[b] (it sizes the grid). */
eh_status eh_prefill_batched(eh_context* ctx, eh_stream stream, uint32_t kv_dtype,
                             const float* q, uint64_t q_bytes, const void* pool,
                             uint64_t pool_bytes, const uint32_t* block_tables, uint64_t bt_bytes,
                             uint32_t bt_stride, const uint32_t* cu_q, const uint32_t* start_pos,
                             uint32_t batch, uint32_t max_q_tokens, uint32_t total_q_tokens,
                             float* out, uint64_t out_bytes, uint32_t n_head, uint32_t n_head_kv,
                             uint32_t head_dim, uint32_t block_tokens);

/* ---- Batched chunked prefill over an E4M3 pool (extension; format and
 * scales as eh_append_kv_e4m3_batched): eh_prefill_batched's semantics on the
 * dequantised pool, decode(code) * scale.  Codes are widened to f16 (exact)
 * as the tiles are staged and take the f16 MFMA path; head_dim 64 or 128. */
eh_status eh_prefill_batched_e4m3(eh_context* ctx, eh_stream stream, const float* q,
                                  uint64_t q_bytes, const void* pool, uint64_t pool_bytes,
                                  const uint32_t* block_tables, uint64_t bt_bytes,
                                  uint32_t bt_stride, const uint32_t* cu_q,
                                  const uint32_t* start_pos, uint32_t batch, uint32_t max_q_tokens,
                                  uint32_t total_q_tokens, float* out, uint64_t out_bytes,
                                  uint32_t n_head, uint32_t n_head_kv, uint32_t head_dim,
                                  uint32_t block_tokens, const float* k_scale,
                                  const float* v_scale);

#ifdef __cplusplus
}
#endif
#endif
