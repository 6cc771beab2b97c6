// paged_kv.hip -- page-row data movement for the paged KV pool on gfx950.
//
// Pool layout (identical to engine-kvcache/src/cache.rs:3-7,181-188 and
// engine-cuda/kernels/paged_kv.cu:3-11, so page bytes compare bit-exactly):
//   page b        at byte  b * page_bytes,  page_bytes = block_tokens * 2 * row_bytes
//   token slot s  at       + s * 2 * row_bytes
//   K row         at       + 0 .. row_bytes
//   V row         at       + row_bytes .. 2 * row_bytes
// row_bytes = n_kv_heads * head_dim * element_bytes.
//
// Because a slot's K row and V row are contiguous, one token's page row is a
// single 2*row_bytes run.  Every kernel here walks a flat index over
// CHUNK-byte pieces of such runs, so consecutive lanes touch consecutive
// bytes: 64 lanes x 16 B = one 1 KiB page row per wave instruction at the
// decode shape (2 kv heads x 128 x f16).  Work is byte copies only: results
// are bit-exact by construction.
//
// All integer kernels bound-check block-table indices and page ids so a bad
// table skips the row instead of touching memory outside the pool.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "e4m3.h"

namespace {

template <int CHUNK> struct chunk_type;
template <> struct chunk_type<16> { using T = uint4; };
template <> struct chunk_type<8> { using T = uint2; };
template <> struct chunk_type<4> { using T = uint32_t; };
template <> struct chunk_type<2> { using T = uint16_t; };

// Sequence lookup for a ragged batch: largest b with cu[b] <= i.
__device__ __forceinline__ uint32_t seq_of(const uint32_t* __restrict__ cu, uint32_t batch,
                                           uint32_t i) {
    uint32_t lo = 0, hi = batch;  // invariant: cu[lo] <= i < cu[hi]
    while (hi - lo > 1) {
        uint32_t mid = (lo + hi) >> 1;
        if (cu[mid] <= i) lo = mid; else hi = mid;
    }
    return lo;
}

// Scatter new K/V rows into their pages.
//   single sequence : cu == nullptr; token i goes to logical position
//                     (pos_ptr ? *pos_ptr : start) + i through `bt`.
//   ragged batch    : token i belongs to b = seq_of(cu, i) and goes to
//                     start_pos[b] + (i - cu[b]) through bt + b*bt_stride.
template <int CHUNK>
__device__ __forceinline__ void append_body(
    const uint8_t* __restrict__ keys, const uint8_t* __restrict__ values,
    const uint32_t* __restrict__ bt, uint32_t bt_stride, uint8_t* __restrict__ pool,
    uint32_t n_tokens, uint32_t start, const uint32_t* __restrict__ pos_ptr,
    const uint32_t* __restrict__ cu, const uint32_t* __restrict__ start_pos, uint32_t batch,
    uint32_t row_bytes, uint32_t block_tokens, uint64_t n_blocks) {
    using T = typename chunk_type<CHUNK>::T;
    const uint32_t cpr = row_bytes / CHUNK;          // chunks per K (or V) row
    const uint32_t cpt = 2 * cpr;                     // chunks per token page row
    const uint32_t total = n_tokens * cpt;           // host guarantees < 2^31
    const uint64_t page_bytes = (uint64_t)block_tokens * 2 * row_bytes;
    const uint32_t base_pos = pos_ptr ? *pos_ptr : start;
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += gridDim.x * blockDim.x) {
        const uint32_t tok = i / cpt;
        const uint32_t c = i - tok * cpt;
        uint32_t pos;
        const uint32_t* row_bt = bt;
        if (cu) {
            const uint32_t b = seq_of(cu, batch, tok);
            pos = start_pos[b] + (tok - cu[b]);
            row_bt = bt + (uint64_t)b * bt_stride;
        } else {
            pos = base_pos + tok;
        }
        const uint32_t page = pos / block_tokens;
        const uint32_t slot = pos - page * block_tokens;
        if (page >= bt_stride) continue;
        const uint32_t phys = row_bt[page];
        if (phys >= n_blocks) continue;
        const bool is_v = c >= cpr;
        const T* src = reinterpret_cast<const T*>((is_v ? values : keys) + (uint64_t)tok * row_bytes) +
                       (is_v ? c - cpr : c);
        T* dst = reinterpret_cast<T*>(pool + (uint64_t)phys * page_bytes +
                                      (uint64_t)slot * 2 * row_bytes) + c;
        *dst = *src;
    }
}

// Gather [n_tokens, row] K (is_value=0) or V rows of one sequence.
template <int CHUNK>
__device__ __forceinline__ void gather_body(
    const uint8_t* __restrict__ pool, const uint32_t* __restrict__ bt, uint32_t bt_len,
    uint8_t* __restrict__ out, uint32_t n_tokens, uint32_t start, uint32_t is_value,
    uint32_t row_bytes, uint32_t block_tokens, uint64_t n_blocks) {
    using T = typename chunk_type<CHUNK>::T;
    const uint32_t cpr = row_bytes / CHUNK;
    const uint32_t total = n_tokens * cpr;           // host guarantees < 2^31
    const uint64_t page_bytes = (uint64_t)block_tokens * 2 * row_bytes;
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += gridDim.x * blockDim.x) {
        const uint32_t tok = i / cpr;
        const uint32_t c = i - tok * cpr;
        const uint32_t pos = start + tok;
        const uint32_t page = pos / block_tokens;
        const uint32_t slot = pos - page * block_tokens;
        if (page >= bt_len) continue;
        const uint32_t phys = bt[page];
        if (phys >= n_blocks) continue;
        const T* src = reinterpret_cast<const T*>(pool + (uint64_t)phys * page_bytes +
                                                  (uint64_t)slot * 2 * row_bytes +
                                                  (is_value ? row_bytes : 0)) + c;
        reinterpret_cast<T*>(out + (uint64_t)tok * row_bytes)[c] = *src;
    }
}

// Whole-page copies dst_ids[k] <- src_ids[k]: copy-on-write of a shared tail
// page and compaction of surviving pages.  One workgroup per page pair.
template <int CHUNK>
__device__ __forceinline__ void copy_pages_body(uint8_t* __restrict__ pool,
                                                const uint32_t* __restrict__ src_ids,
                                                const uint32_t* __restrict__ dst_ids,
                                                uint32_t n_pairs, uint64_t page_bytes,
                                                uint64_t n_blocks) {
    using T = typename chunk_type<CHUNK>::T;
    const uint64_t cpp = page_bytes / CHUNK;
    for (uint32_t k = blockIdx.x; k < n_pairs; k += gridDim.x) {
        const uint32_t s = src_ids[k], d = dst_ids[k];
        if (s >= n_blocks || d >= n_blocks || s == d) continue;
        const T* src = reinterpret_cast<const T*>(pool + (uint64_t)s * page_bytes);
        T* dst = reinterpret_cast<T*>(pool + (uint64_t)d * page_bytes);
        for (uint64_t c = threadIdx.x; c < cpp; c += blockDim.x) dst[c] = src[c];
    }
}

// ---- FP8 E4M3 storage (OCP E4M3FN: bias 7, S.1111.111 = NaN, max 448)
// with one f32 scale per (kv head, K or V): code = quantize(x / scale),
// value = decode(code) * scale.  The format is the one named by the
// reference's FP8 KV design (openspec/archive/2026-08-28-fp8-kv-cache-
// quantization/design.md:3-6); the reference has no kernel for it.

// Token row `tok` of a ragged batch (or single sequence): its page-row byte
// offset in the pool, or ~0 when its block-table entry is missing.
__device__ __forceinline__ uint64_t row_offset(
    uint32_t tok, const uint32_t* __restrict__ bt, uint32_t bt_stride, uint32_t start,
    const uint32_t* __restrict__ pos_ptr, const uint32_t* __restrict__ cu,
    const uint32_t* __restrict__ start_pos, uint32_t batch, uint32_t block_tokens,
    uint64_t n_blocks, uint64_t page_bytes, uint32_t slot_bytes) {
    uint32_t pos;
    const uint32_t* row_bt = bt;
    if (cu) {
        const uint32_t b = seq_of(cu, batch, tok);
        pos = start_pos[b] + (tok - cu[b]);
        row_bt = bt + (uint64_t)b * bt_stride;
    } else {
        pos = (pos_ptr ? *pos_ptr : start) + tok;
    }
    const uint32_t page = pos / block_tokens;
    if (page >= bt_stride) return ~0ull;
    const uint32_t phys = row_bt[page];
    if (phys >= n_blocks) return ~0ull;
    return (uint64_t)phys * page_bytes + (uint64_t)(pos - page * block_tokens) * slot_bytes;
}

}  // namespace

// Quantising append: f32 keys/values [n_tokens, row_len] -> E4M3 page rows,
// 4 elements (one u32 of codes) per thread; addressing as eh_append_kv_c*.
extern "C" __global__ __launch_bounds__(256) void eh_append_kv_e4m3(
    const float* keys, const float* values, const uint32_t* bt, uint32_t bt_stride, uint8_t* pool,
    uint32_t n_tokens, uint32_t start, const uint32_t* pos_ptr, const uint32_t* cu,
    const uint32_t* start_pos, uint32_t batch, uint32_t row_len, uint32_t head_dim,
    uint32_t block_tokens, uint64_t n_blocks, const float* k_scale, const float* v_scale) {
    const uint32_t qpr = row_len / 4;   // quads per K (or V) row
    const uint32_t qpt = 2 * qpr;
    const uint32_t total = n_tokens * qpt;  // host guarantees < 2^31
    const uint64_t page_bytes = (uint64_t)block_tokens * 2 * row_len;
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < total; i += gridDim.x * blockDim.x) {
        const uint32_t tok = i / qpt;
        const uint32_t c = i - tok * qpt;
        const uint64_t off = row_offset(tok, bt, bt_stride, start, pos_ptr, cu, start_pos, batch,
                                        block_tokens, n_blocks, page_bytes, 2 * row_len);
        if (off == ~0ull) continue;
        const bool is_v = c >= qpr;
        const uint32_t e = 4 * (is_v ? c - qpr : c);  // element within the row
        const float4 x = *reinterpret_cast<const float4*>((is_v ? values : keys) +
                                                          (uint64_t)tok * row_len + e);
        const float sc = (is_v ? v_scale : k_scale)[e / head_dim];
        const uint32_t w = e4m3_code(x.x / sc) | (e4m3_code(x.y / sc) << 8) |
                           (e4m3_code(x.z / sc) << 16) | (e4m3_code(x.w / sc) << 24);
        *reinterpret_cast<uint32_t*>(pool + off + (is_v ? row_len : 0u) + e) = w;
    }
}

// Dynamic per-head E4M3 scales from data (the FP8 KV design's per-head f32
// scale): scale[h] = max(amax_h / 448, FLT_MIN), amax_h = the largest finite
// magnitude among head h's elements of rows [n_rows, row_len], so those
// elements span the whole code range (448 is E4M3's largest value); a head
// with no finite nonzero element gets 1.  Grid (n_kv, 2): y = 0 reads keys
// into k_scale, y = 1 values into v_scale; 256 threads; head_dim % 4 == 0.
extern "C" __global__ __launch_bounds__(256) void eh_kv_e4m3_scales(
    const float* keys, const float* values, uint32_t n_rows, uint32_t row_len, uint32_t head_dim,
    float* k_scale, float* v_scale) {
    __shared__ float wmax[4];
    const uint32_t h = blockIdx.x;
    const float* src = (blockIdx.y ? values : keys) + (uint64_t)h * head_dim;
    const uint32_t qph = head_dim / 4;  // float4s per head row
    const uint64_t total = (uint64_t)n_rows * qph;
    float m = 0.0f;
    for (uint64_t i = threadIdx.x; i < total; i += blockDim.x) {
        const uint64_t r = i / qph;
        const float4 x = *reinterpret_cast<const float4*>(src + r * row_len + 4 * (i - r * qph));
        const float a[4] = {__builtin_fabsf(x.x), __builtin_fabsf(x.y), __builtin_fabsf(x.z),
                            __builtin_fabsf(x.w)};
#pragma unroll
        for (int k = 0; k < 4; ++k)
            if (a[k] <= 3.40282347e38f) m = a[k] > m ? a[k] : m;  // finite only: NaN and inf fail
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float y = __shfl_xor(m, o, 64);
        m = y > m ? y : m;
    }
    if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (uint32_t w = 1; w < blockDim.x / 64; ++w) m = wmax[w] > m ? wmax[w] : m;
        const float s = m / 448.0f;
        (blockIdx.y ? v_scale : k_scale)[h] = m > 0.0f ? (s > 1.17549435e-38f ? s : 1.17549435e-38f) : 1.0f;
    }
}

// Dequantising gather of one sequence's K (is_value = 0) or V rows:
// out [n_tokens, row_len] f32 = decode(code) * scale of the element's head;
// rows whose block-table entry is missing are left untouched.
extern "C" __global__ __launch_bounds__(256) void eh_gather_kv_e4m3(
    const uint8_t* pool, const uint32_t* bt, uint32_t bt_len, float* out, uint32_t n_tokens,
    uint32_t start, uint32_t is_value, uint32_t row_len, uint32_t head_dim, uint32_t block_tokens,
    uint64_t n_blocks, const float* scale) {
    const uint32_t qpr = row_len / 4;
    const uint32_t total = n_tokens * qpr;
    const uint64_t page_bytes = (uint64_t)block_tokens * 2 * row_len;
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < total; i += gridDim.x * blockDim.x) {
        const uint32_t tok = i / qpr;
        const uint32_t e = 4 * (i - tok * qpr);
        const uint64_t off = row_offset(tok, bt, bt_len, start, nullptr, nullptr, nullptr, 0,
                                        block_tokens, n_blocks, page_bytes, 2 * row_len);
        if (off == ~0ull) continue;
        const uint32_t w = *reinterpret_cast<const uint32_t*>(pool + off + (is_value ? row_len : 0u) + e);
        const float sc = scale[e / head_dim];
        typedef float f32x2 __attribute__((ext_vector_type(2)));
        const f32x2 lo = __builtin_amdgcn_cvt_pk_f32_fp8(w, false), hi = __builtin_amdgcn_cvt_pk_f32_fp8(w, true);
        *reinterpret_cast<float4*>(out + (uint64_t)tok * row_len + e) =
            make_float4(lo[0] * sc, lo[1] * sc, hi[0] * sc, hi[1] * sc);
    }
}

#define EH_DEFINE_CHUNK(CH)                                                                      \
    extern "C" __global__ __launch_bounds__(256) void eh_append_kv_c##CH(                        \
        const uint8_t* keys, const uint8_t* values, const uint32_t* bt, uint32_t bt_stride,      \
        uint8_t* pool, uint32_t n_tokens, uint32_t start, const uint32_t* pos_ptr,               \
        const uint32_t* cu, const uint32_t* start_pos, uint32_t batch, uint32_t row_bytes,       \
        uint32_t block_tokens, uint64_t n_blocks) {                                              \
        append_body<CH>(keys, values, bt, bt_stride, pool, n_tokens, start, pos_ptr, cu,         \
                        start_pos, batch, row_bytes, block_tokens, n_blocks);                    \
    }                                                                                            \
    extern "C" __global__ __launch_bounds__(256) void eh_gather_kv_c##CH(                        \
        const uint8_t* pool, const uint32_t* bt, uint32_t bt_len, uint8_t* out,                  \
        uint32_t n_tokens, uint32_t start, uint32_t is_value, uint32_t row_bytes,                \
        uint32_t block_tokens, uint64_t n_blocks) {                                              \
        gather_body<CH>(pool, bt, bt_len, out, n_tokens, start, is_value, row_bytes,             \
                        block_tokens, n_blocks);                                                 \
    }                                                                                            \
    extern "C" __global__ __launch_bounds__(256) void eh_copy_pages_c##CH(                       \
        uint8_t* pool, const uint32_t* src_ids, const uint32_t* dst_ids, uint32_t n_pairs,       \
        uint64_t page_bytes, uint64_t n_blocks) {                                                \
        copy_pages_body<CH>(pool, src_ids, dst_ids, n_pairs, page_bytes, n_blocks);              \
    }

EH_DEFINE_CHUNK(16)
EH_DEFINE_CHUNK(8)
EH_DEFINE_CHUNK(4)
EH_DEFINE_CHUNK(2)

// Rewrite block-table entries through a page remap: e = remap[e] for every
// entry below n_remap (padding entries >= n_remap are left alone).
extern "C" __global__ __launch_bounds__(256) void eh_remap_block_tables(
    uint32_t* bt, uint64_t n_entries, const uint32_t* remap, uint32_t n_remap) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n_entries;
         i += (uint64_t)gridDim.x * blockDim.x) {
        const uint32_t e = bt[i];
        if (e < n_remap) bt[i] = remap[e];
    }
}

// Page reference counts: counts[p] += number of (row b, j < n_used[b])
// block-table entries equal to p.  counts must be zeroed by the caller.
extern "C" __global__ __launch_bounds__(256) void eh_page_refcounts(
    const uint32_t* bt, uint32_t bt_stride, const uint32_t* n_used, uint32_t batch,
    uint32_t* counts, uint32_t n_blocks) {
    const uint64_t total = (uint64_t)batch * bt_stride;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (uint64_t)gridDim.x * blockDim.x) {
        const uint32_t b = (uint32_t)(i / bt_stride);
        const uint32_t j = (uint32_t)(i - (uint64_t)b * bt_stride);
        if (j >= n_used[b]) continue;
        const uint32_t p = bt[i];
        if (p < n_blocks) atomicAdd(&counts[p], 1u);
    }
}

// Clear a u32 array with vector stores (graph-capture safe, unlike a memset node).
extern "C" __global__ __launch_bounds__(256) void eh_fill_u32(uint32_t* p, uint64_t n,
                                                              uint32_t v) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x)
        p[i] = v;
}

// ---------------------------------------------------------------------------
// Read ceiling of a paged decode (a measurement aid, not part of the KV
// path): streams the listed pages once, in list order, and folds every word
// read into one xor per wave, so no load is dead and nothing but 4 bytes per
// wave is written.  A page is read as 16 KiB items, one wave per item, 64
// lanes x 16 B per wave instruction (16 instructions per item); the item
// list (page-major) is cut into equal contiguous ranges, one per wave, and
// each wave keeps DEPTH items in flight (the next item is issued as soon as
// its slot is consumed; issues past the range re-read the range's last item,
// never folded).  page_bytes is a multiple of 16 KiB; ids past the pool are
// skipped (read as page 0, not folded).
namespace {
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
constexpr uint32_t kItemBytes = 16384;

template <int DEPTH>
__device__ __forceinline__ void stream_pages_body(const uint8_t* __restrict__ pool,
                                                  const uint32_t* __restrict__ ids,
                                                  uint32_t n_ids, uint64_t page_bytes,
                                                  uint64_t n_blocks, uint32_t* __restrict__ out) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wpb = blockDim.x >> 6;
    const uint32_t W = gridDim.x * wpb;
    const uint32_t w = blockIdx.x * wpb + (uint32_t)__builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const uint32_t ipp = (uint32_t)(page_bytes / kItemBytes);  // items per page
    const uint64_t n_items = (uint64_t)n_ids * ipp;
    const uint64_t i0 = n_items * w / W, i1 = n_items * (w + 1) / W;
    u32x4v acc = {0u, 0u, 0u, 0u};
    if (i0 < i1) {
        u32x4v r[DEPTH][16];
        bool ok[DEPTH];
        auto issue = [&](int d, uint64_t i) {
            const uint64_t ic = i < i1 ? i : i1 - 1;
            const uint32_t p = ids[ic / ipp];
            ok[d] = i < i1 && (uint64_t)p < n_blocks;
            const uint8_t* src = pool + ((uint64_t)p < n_blocks ? p : 0u) * page_bytes +
                                 (ic % ipp) * kItemBytes + lane * 16u;
#pragma unroll
            for (int j = 0; j < 16; ++j) r[d][j] = *reinterpret_cast<const u32x4v*>(src + j * 1024);
        };
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) issue(d, i0 + d);
        for (uint64_t base = i0; base < i1; base += DEPTH) {
#pragma unroll
            for (int d = 0; d < DEPTH; ++d) {
                u32x4v x = r[d][0];
#pragma unroll
                for (int j = 1; j < 16; ++j) x ^= r[d][j];
                acc ^= ok[d] ? x : u32x4v{0u, 0u, 0u, 0u};
                issue(d, base + d + DEPTH);
            }
        }
    }
    uint32_t v = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v ^= (uint32_t)__shfl_xor((int)v, o, 64);
    if (lane == 0) out[w] = v;
}
}  // namespace

#define EH_STREAM_PAGES(D)                                                                       \
    extern "C" __global__ __launch_bounds__(512) void eh_stream_pages_d##D(                      \
        const uint8_t* pool, const uint32_t* ids, uint32_t n_ids, uint64_t page_bytes,           \
        uint64_t n_blocks, uint32_t* out) {                                                      \
        stream_pages_body<D>(pool, ids, n_ids, page_bytes, n_blocks, out);                       \
    }
EH_STREAM_PAGES(1)
EH_STREAM_PAGES(2)

// The same read in the decode's pattern (a measurement aid): the token-balanced
// decode runs one wave per kv head, and the waves of a run walk the same pages
// together, each reading only its kv head's K and V rows.  Here the page list
// is cut into equal contiguous ranges, one per group of n_kv waves (8 / n_kv
// groups per workgroup); wave h of a group reads kv head h's 256-byte slice of
// the K row and of the V row of every token (16 lanes per slice, 4 tokens per
// instruction), two pages in flight.  Pages hold 16 tokens; row_bytes is one
// K (or V) row, n_kv * 256 bytes.  Every word read is folded into one xor per
// wave; ids past the pool are skipped (read as page 0, not folded).
extern "C" __global__ __launch_bounds__(512) void eh_stream_pages_heads(
    const uint8_t* __restrict__ pool, const uint32_t* __restrict__ ids, uint32_t n_ids,
    uint64_t page_bytes, uint64_t n_blocks, uint32_t row_bytes, uint32_t n_kv,
    uint32_t* __restrict__ out) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t w = blockIdx.x * 8u + (uint32_t)__builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const uint32_t G = gridDim.x * 8u / n_kv, g = w / n_kv, h = w % n_kv;
    const uint32_t i0 = (uint32_t)((uint64_t)n_ids * g / G), i1 = (uint32_t)((uint64_t)n_ids * (g + 1) / G);
    uint32_t off[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)  // j < 4: K rows of tokens 4j..4j+3, j >= 4: V rows
        off[j] = (4u * (j & 3) + lane / 16u) * 2u * row_bytes + (j >= 4 ? row_bytes : 0u) +
                 h * 256u + (lane & 15u) * 16u;
    u32x4v acc = {0u, 0u, 0u, 0u};
    for (uint32_t i = i0; i < i1; i += 2) {
        const uint32_t pa = ids[i], pb = ids[i + 1 < i1 ? i + 1 : i];
        const bool oka = (uint64_t)pa < n_blocks, okb = i + 1 < i1 && (uint64_t)pb < n_blocks;
        const uint8_t* a = pool + (oka ? (uint64_t)pa : 0u) * page_bytes;
        const uint8_t* b = pool + ((uint64_t)pb < n_blocks ? (uint64_t)pb : 0u) * page_bytes;
        u32x4v r[16];
#pragma unroll
        for (int j = 0; j < 8; ++j) r[j] = *reinterpret_cast<const u32x4v*>(a + off[j]);
#pragma unroll
        for (int j = 0; j < 8; ++j) r[8 + j] = *reinterpret_cast<const u32x4v*>(b + off[j]);
        u32x4v xa = r[0], xb = r[8];
#pragma unroll
        for (int j = 1; j < 8; ++j) {
            xa ^= r[j];
            xb ^= r[8 + j];
        }
        acc ^= oka ? xa : u32x4v{0u, 0u, 0u, 0u};
        acc ^= okb ? xb : u32x4v{0u, 0u, 0u, 0u};
    }
    uint32_t v = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v ^= (uint32_t)__shfl_xor((int)v, o, 64);
    if (lane == 0) out[w] = v;
}
