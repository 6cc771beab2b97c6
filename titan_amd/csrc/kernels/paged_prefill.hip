// paged_prefill.hip -- causal chunked-prefill attention over paged KV for gfx950.
//
// Semantics follow the reference FlashAttention-2 prefill kernel
// (engine-cuda/kernels/flash_attention_2.cu:22-106, launcher
// engine-cuda/src/flash_attention.rs:95-225): query i of a chunk sits at
// global position p0 + i (p0 = pos_offset, or *pos_ptr when given) and
// attends keys 0..=p0+i of its sequence through the block table, q head qh
// reading kv head qh / (n_head / n_head_kv); scale 1/sqrt(head_dim); a row
// with no attended key yields zeros (flash_attention_2.cu:98).
//
// Work decomposition (MI355X-first; the reference runs one warp per
// (q head, query) and re-reads K/V for each):
//   * one workgroup of 8 waves per (256-row tile, kv head, sequence); the
//     rows of a tile are (query token, q head of the GQA group) pairs, so one
//     K/V tile in LDS serves every q head of the group;
//   * K/V tiles of N keys are gathered through the block table into LDS,
//     K and V both row-major (padded rows), double-buffered: the global loads
//     of the next tile are in flight while MFMAs consume the current one; the
//     V^T operand of P.V is read from the row-major V tile with the gfx950
//     transposed LDS read ds_read_b64_tr_b16;
//   * each wave owns 32 rows: S^T = K Q^T on 32x32 MFMA tiles, online softmax
//     in the log2 domain on the accumulator registers (the S^T layout puts one
//     query row per lane column, so row statistics stay lane-local up to one
//     exchange between the two lane halves), then O^T += V^T P^T with P taken
//     straight from registers (keys permuted consistently between P and V^T);
//   * the accumulators are rescaled only when a row maximum grows by more
//     than 2^8 (exact: every term uses the same stale maximum);
//   * operands: f16 KV -> f16 MFMA with Q split into hi + lo f16 halves
//     for the scores (~22 significant bits) and P one f16; bf16 KV ->
//     widened to f16 as the tiles are staged (exact: a bf16 significand has
//     8 bits, and every finite bf16 below 2^16 in magnitude is an f16, down
//     to 2^-14; below that the f16 subnormals keep the value to 2^-24), then
//     the f16 path; a staged tile holding a finite bf16 of magnitude >= 2^16
//     is re-staged raw and computed on bf16 MFMAs with Q and P each split
//     into hi + lo bf16 parts (two MFMAs per product, ~16 significant bits);
//     E4M3 KV -> widened to f16 (exact), the f16 path; f32 KV -> f32 MFMA
//     (no operand rounding);
//   * workgroups are dispatched longest row block first (causal: a later
//     row block attends more keys), so the second round of workgroups on a
//     CU fills in behind the first; the row blocks of one (sequence, kv
//     head) share one XCD's L2 when the pair count is a multiple of 8.
// Invalid block-table entries (beyond the table or >= n_blocks) mask their
// keys instead of reading outside the pool.

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

enum { DT_F32 = 0, DT_F16 = 1, DT_BF16 = 2, DT_FP8 = 3 };

constexpr int NT = 512;           // threads per workgroup (8 waves)
constexpr int NL = 256;           // threads (waves 0-3) staging f16 / E4M3 / f32 tiles
constexpr uint32_t ROWS = NT / 2;  // query rows per workgroup: 32 per wave
constexpr uint32_t SLICE = 1024;  // block-table entries staged in LDS at once
constexpr float RESCALE_LOG2 = 8.0f;

// Exponent e that puts a row whose largest |element| is amax in
// [2^14, 2^15) once scaled by 2^e (0 for an all-zero or non-finite row).
__device__ __forceinline__ int q_exponent(float amax) {
    if (!(amax > 0.0f) || !(amax < __builtin_inff())) return 0;
    const int e = 15 - __builtin_amdgcn_frexp_expf(amax);
    return e < -100 ? -100 : e > 100 ? 100 : e;
}

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
// Native vectors for staged K/V words: HIP's uint4 / uint2 are structs, whose
// copies the compiler keeps as memory (a private array it then places in
// LDS or scratch) instead of registers.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

template <int DT> struct op_t;
// 16-bit pages (f16, bf16 widened to f16, E4M3 widened to f16): q is split
// into hi + lo f16 halves for S = K Q^T (two MFMAs per step, ~22-bit scores;
// one f16 q would carry an error that grows with |K|: 7e-3 max-abs at K of
// standard deviation 16 against 5e-4 with the split); P stays one f16.
// q is first scaled by a power of two per wave (largest element in
// [2^14, 2^15)): a lo half of ~2^-11 of an element is then a normal f16,
// where unscaled it would often be subnormal and keep only the few bits
// above f16's absolute step of 2^-24 (with E4M3 pages q carries the K scale
// and is ~1e-3); the scores are scaled back, exactly.  The row sums l are
// taken from the same f16-rounded P that feeds the P.V MFMAs, so that
// acc / l stays a weighted mean: with the unrounded sums, a dominant weight
// rounded by up to 2^-11 shifts the output by that much of its V row
// (2.7e-3 measured at K of standard deviation 16).
template <> struct op_t<DT_F16> {
    typedef f16x8 v;
    static constexpr int KS = 16;  // contraction depth of one MFMA
    static constexpr int ELT = 2;
    static constexpr bool SPLIT = true;
    static __device__ __forceinline__ f32x16 mma(v a, v b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
};
template <> struct op_t<DT_BF16> {
    typedef bf16x8 v;
    static constexpr int KS = 16;
    static constexpr int ELT = 2;
    static constexpr bool SPLIT = true;
    static __device__ __forceinline__ f32x16 mma(v a, v b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
};
template <> struct op_t<DT_F32> {
    typedef float v;
    static constexpr int KS = 2;
    static constexpr int ELT = 4;
    static constexpr bool SPLIT = false;
    static __device__ __forceinline__ f32x16 mma(v a, v b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
    }
};

// E4M3 pages are staged into LDS as f16 (exact) and use the f16 operands.
template <> struct op_t<DT_FP8> : op_t<DT_F16> {};

// 8 f32 -> MFMA operand (hi part, and lo = x - hi for split types).  A
// caller whose x are products must pass them through opaque(): fused with
// the product, the backend formed the hi that feeds the MFMA and the hi
// subtracted for lo from two differently rounded products (v_cvt_pk_f16_f32
// of the rounded product, v_fma_mixlo_f16 of the exact one), and where
// they differed hi + lo missed x by one f16 step (1e-3-scale score errors).
template <int DT>
__device__ __forceinline__ void pack8(const float* x, typename op_t<DT>::v& hi,
                                      typename op_t<DT>::v& lo) {
    if constexpr (DT == DT_F16) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const _Float16 h = (_Float16)x[e];
            hi[e] = h;
            lo[e] = (_Float16)(x[e] - (float)h);
        }
    } else if constexpr (DT == DT_BF16) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const __bf16 h = (__bf16)x[e];
            hi[e] = h;
            lo[e] = (__bf16)(x[e] - (float)h);
        }
    }
}

typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

// A value the compiler may not fuse with the operations that made it or
// use it (an empty asm: no instruction is emitted).
__device__ __forceinline__ void opaque(float& v) { asm volatile("" : "+v"(v)); }

// max / sum of x over lanes l and l ^ 32, on every lane, without the LDS
// path of a shuffle: v_permlane32_swap(a, b) leaves the lower halves of a and
// b in the first result and their upper halves in the second.  b is an opaque
// copy of a: with the same value in both operands the compiler took the two
// results for equal and dropped one of them.
__device__ __forceinline__ uint2 halves(float x) {
    uint32_t a = __builtin_bit_cast(uint32_t, x), b = a;
    asm volatile("" : "+v"(b));
    const auto r = __builtin_amdgcn_permlane32_swap(a, b, false, false);
    return make_uint2(r[0], r[1]);
}
__device__ __forceinline__ float max_halves(float x) {
    const uint2 r = halves(x);
    return fmaxf(__builtin_bit_cast(float, r.x), __builtin_bit_cast(float, r.y));
}
__device__ __forceinline__ float sum_halves(float x) {
    const uint2 r = halves(x);
    return __builtin_bit_cast(float, r.x) + __builtin_bit_cast(float, r.y);
}

// Transposed LDS read (ds_read_b64_tr_b16): in each 16-lane group, lane
// 4r + b points at 4 consecutive 16-bit elements of row r (columns 4b..4b+3)
// of a 4 x 16 block; lane c receives column c of rows 0..3.
__device__ __forceinline__ uint64_t lds_read_tr(const uint8_t* p) {
    const i16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(const_cast<uint8_t*>(p)));
    return __builtin_bit_cast(uint64_t, v);
}

__device__ __forceinline__ uint32_t perm(uint32_t hi_src, uint32_t lo_src, uint32_t sel) {
    return __builtin_amdgcn_perm(hi_src, lo_src, sel);
}

// Geometry per (type, head_dim): one load item = KPI consecutive keys x 16
// bytes of a head row; N keys per tile so that the NLOAD staging threads own
// one item each.  bf16 pages: every thread stages 2 keys, so the bf16 -> f16
// widening is spread over all 8 waves (measured 8.5 % faster than waves 0-3
// staging 4 keys each, which stays faster for f16, E4M3 and f32 pages:
// for f32, an item is one 16-byte V^T group of 4 keys).
template <int DT, int HD>
struct geo {
    static constexpr int ELT = op_t<DT>::ELT;
    static constexpr int EPC = 16 / ELT;          // elements per 16-byte chunk
    static constexpr int PARTS = HD / EPC;        // chunks per head row
    static constexpr int KPI = DT == DT_BF16 ? 2 : 4;  // keys per load item
    static constexpr int NLOAD = DT == DT_BF16 ? NT : NL;
    static constexpr int N = KPI * NLOAD / PARTS;  // keys per tile
    static constexpr int SUB = N / 32;            // 32-key sub-blocks per tile
    static constexpr int KPITCH = HD * ELT + 16;  // bytes per K row in LDS
    static constexpr int VPITCH = N * ELT + (ELT == 4 ? 16 : 8);  // bytes per V^T row
    // V^T rows hold N/4 groups of 4 keys; group g of row d is stored at
    // g ^ (row block of d) so that the transposing stores spread over banks.
    static constexpr int GMASK = N / 4 - 1;
    static constexpr int GBYTES = 4 * ELT;
    static constexpr int KBYTES = N * KPITCH;
    // 16-bit operands: V row-major (keys x dims, rows padded by 128 bytes) and
    // read back transposed by ds_read_b64_tr_b16; f32: V^T rows
    static constexpr bool VROWM = ELT == 2;
    static constexpr int VRPITCH = HD * 2 + 128;  // padding measured best for the transposed reads
    static constexpr int VBYTES = VROWM ? N * VRPITCH : HD * VPITCH;
    static constexpr int STAGE = KBYTES + VBYTES;
    static_assert(N % 32 == 0 && N >= 32, "tile must hold whole 32-key sub-blocks");
    static_assert(HD % 32 == 0, "head_dim must be a multiple of 32");
};

template <int HD>
struct geo<DT_FP8, HD> : geo<DT_F16, HD> {};

// Eight E4M3 codes (two dwords, lowest byte first) as eight f16 (four dwords);
// exact: every E4M3 value is an f16.
__device__ __forceinline__ u32x4 e4m3x8_to_f16(uint32_t w0, uint32_t w1) {
    return u32x4{
        __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 1.0f, false)),
        __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 1.0f, true)),
        __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 1.0f, false)),
        __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 1.0f, true))};
}

struct lds_hdr {
    uint32_t tile_bad[2];  // tile index whose keys include an invalid page
    uint32_t slice_base;
    uint32_t tile_big[2];  // bf16 pages: tile index holding a value beyond f16's range
};

// Eight bf16 (four dwords) as eight f16, and the running packed maximum of
// the bf16 exponent fields (finite values of magnitude >= 2^16 -- exponent
// field >= 143 -- do not fit an f16; inf / NaN fields count too, which only
// sends such a tile to the exact bf16 path).  In-range values convert
// exactly; the rounding mode only matters below 2^-14 (f16 subnormals).
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ u32x4 bf16x8_to_f16(u32x4 w, u16x2& emax) {
    uint32_t r[4];
    const uint32_t in[4] = {w[0], w[1], w[2], w[3]};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float lo = __builtin_bit_cast(float, in[i] << 16);
        const float hi = __builtin_bit_cast(float, in[i] & 0xFFFF0000u);
        r[i] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(lo, hi));
        emax = __builtin_elementwise_max(emax, __builtin_bit_cast(u16x2, in[i] & 0x7F807F80u));
    }
    return u32x4{r[0], r[1], r[2], r[3]};
}
constexpr unsigned short BF16_F16_LIMIT = 143u << 7;  // exponent field of 2^16

template <int DT, int HD>
__device__ __forceinline__ void prefill(
    const float* __restrict__ q, const uint8_t* __restrict__ pool,
    const uint32_t* __restrict__ bt_all, uint32_t bt_stride, uint32_t bt_entries,
    const uint32_t* __restrict__ cu_q, const uint32_t* __restrict__ start_pos,
    const uint32_t* __restrict__ pos_ptr, uint32_t q_tokens, uint32_t pos_offset,
    float* __restrict__ out, uint32_t n_head, uint32_t n_head_kv, uint32_t block_tokens,
    int bt_shift, uint32_t row_bytes, float scale_log2, uint64_t n_blocks, uint8_t* smem,
    const float* __restrict__ k_scale, const float* __restrict__ v_scale) {
    // bf16 pages are staged as f16 and take the f16 operands; OB: the exact
    // bf16 path of tiles beyond f16's range
    constexpr bool B2H = DT == DT_BF16;
    typedef op_t<B2H ? DT_F16 : DT> O;
    typedef op_t<DT_BF16> OB;
    typedef typename O::v opv;
    typedef geo<DT, HD> Gm;
    constexpr int N = Gm::N;

    // ---- workgroup order.  Dispatch position d (x fastest) takes row block
    // gx - 1 - d / pairs of (kv head, sequence) pair d % pairs: the longest
    // row blocks go first, so the workgroups of the second round land on the
    // CUs that finished their first one earliest (config 3: 33..40 key tiles
    // per row block, every CU ends near the 73-tile mean; measured 3-4 %
    // faster than a row-block-major order).  Dispatch is round-robin over
    // the 8 XCDs, so with pairs a multiple of 8 every row block of a pair
    // runs on one XCD and shares its L2.
    const uint32_t gx = gridDim.x, gy = gridDim.y;
    const uint32_t pairs = gy * gridDim.z;
    const uint32_t d = blockIdx.x + gx * (blockIdx.y + gy * blockIdx.z);
    const uint32_t tile = gx - 1u - d / pairs;
    const uint32_t hk = (d % pairs) % gy;
    const uint32_t b = (d % pairs) / gy;

    uint32_t qoff, n_q, p0;
    const uint32_t* bt;
    if (cu_q) {  // ragged batch; q_tokens is the total row count of q / out
        qoff = min(cu_q[b], q_tokens);
        const uint32_t end = min(cu_q[b + 1], q_tokens);
        n_q = end > qoff ? end - qoff : 0u;
        p0 = start_pos[b];
        bt = bt_all + (uint64_t)b * bt_stride;
    } else {
        qoff = 0;
        n_q = q_tokens;
        p0 = pos_ptr ? pos_ptr[0] : pos_offset;
        bt = bt_all;
    }
    const uint32_t group = n_head / n_head_kv;
    const uint32_t rows = n_q * group;
    const uint32_t row0 = tile * ROWS;
    if (row0 >= rows) return;  // uniform over the workgroup

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31;
    const int h = lane >> 5;
    // transposed V reads: this lane's byte offset in a row-major V tile
    const uint32_t vtr_off = (4 * h + ((lane & 15) >> 2)) * Gm::VRPITCH +
                             (16 * ((lane >> 4) & 1) + 4 * (lane & 3)) * 2;

    // ---- this lane's query row (column of S^T / O^T)
    const uint32_t row_raw = row0 + wave * 32 + l32;
    const bool row_ok = row_raw < rows;
    const uint32_t row = row_ok ? row_raw : rows - 1u;
    const uint32_t tok = row / group;
    const uint32_t head = hk * group + (row - tok * group);
    // Key positions are capped at the block table's capacity: keys past it
    // have no page (masked), and the cap bounds the loop for any device-side
    // position.
    const uint64_t cap = (uint64_t)bt_entries * block_tokens - 1u;
    auto clamp_pos = [&](uint32_t t) -> uint32_t {
        const uint64_t v = (uint64_t)p0 + t;
        return (uint32_t)(v < cap ? v : cap);
    };
    const uint32_t lim = clamp_pos(tok);  // attends keys <= lim
    // wave / workgroup bounds (rows are ordered by token)
    const uint32_t wr0 = min(row0 + wave * 32u, rows - 1u);
    const uint32_t wr1 = min(row0 + wave * 32u + 31u, rows - 1u);
    const uint32_t wave_min = clamp_pos(wr0 / group);
    const uint32_t wave_max = clamp_pos(wr1 / group);
    const uint32_t kmax = clamp_pos(min(row0 + ROWS - 1u, rows - 1u) / group);  // workgroup bound
    const uint32_t n_tiles = kmax / N + 1u;

    // ---- LDS carve-up
    lds_hdr* hdr = reinterpret_cast<lds_hdr*>(smem);
    uint32_t* slice = reinterpret_cast<uint32_t*>(smem + 64);
    uint8_t* kflag = smem + 64 + SLICE * 4;                 // [2][N] key valid bytes
    uint8_t* stage = smem + 64 + SLICE * 4 + 2 * N;         // [2][STAGE]

    auto entry_of = [&](uint32_t key) -> uint32_t {
        return bt_shift >= 0 ? (key >> bt_shift) : key / block_tokens;
    };
    auto stage_slice = [&](uint32_t base) {
        for (uint32_t i = tid; i < SLICE; i += NT) {
            const uint32_t e = base + i;
            uint32_t v = 0xFFFFFFFFu;
            if (e < bt_entries) {
                const uint32_t p = bt[e];
                if ((uint64_t)p < n_blocks) v = p;
            }
            slice[i] = v;
        }
        if (tid == 0) hdr->slice_base = base;
    };

    // ---- load item of this thread: keys 4*kg .. 4*kg+3 of a tile, chunk `part`
    const int part = tid % Gm::PARTS;
    const int kg = tid / Gm::PARTS;
    const uint64_t page_bytes = (uint64_t)block_tokens * 2u * row_bytes;
    // E4M3 pages: one byte per element, a load item is 8 codes per key
    constexpr bool F8 = DT == DT_FP8;
    constexpr int CT = (F8 || B2H) ? DT_F16 : DT;  // MFMA operand type
    constexpr uint32_t SE = F8 ? 1u : (uint32_t)Gm::ELT;  // stored element bytes
    const uint32_t head_off = hk * HD * SE + part * (16 / Gm::ELT) * SE;
    constexpr int KPI = Gm::KPI;
    u32x4 kr[KPI], vr[KPI];
    uint32_t okbits = 0;  // bit j: key KPI*kg+j loadable; bit KPI+j: key <= kmax with a bad page

    const uint32_t slot_bytes = 2u * row_bytes;
    const bool pagek = block_tokens % KPI == 0u;  // an item's KPI aligned keys share a page
    // page id of table entry e: from the LDS slice, or (direct) from the
    // global table with the slice's bounds checks -- the re-stage of a tile
    // runs after the slice may have moved on to the next tile
    auto page_of = [&](uint32_t e, bool direct) -> uint32_t {
        if (!direct) return slice[e - hdr->slice_base];
        uint32_t v = 0xFFFFFFFFu;
        if (e < bt_entries) {
            const uint32_t p = bt[e];
            if ((uint64_t)p < n_blocks) v = p;
        }
        return v;
    };
    auto issue = [&](uint32_t t, bool direct = false) {
        const uint32_t key0 = t * N + KPI * kg;
        okbits = 0;
        if (pagek) {
            const uint32_t e = entry_of(key0);
            const uint32_t phys = page_of(e, direct);
            const uint32_t slot = key0 - e * block_tokens;
            const bool pv = phys != 0xFFFFFFFFu;
            const uint8_t* p = pool + (uint64_t)(pv ? phys : 0u) * page_bytes +
                               (uint64_t)(pv ? slot * slot_bytes + head_off : 0u);
            const uint32_t step = pv ? slot_bytes : 0u;
#pragma unroll
            for (int j = 0; j < KPI; ++j) {
                const bool live = key0 + j <= kmax;
                okbits |= (live && pv ? 1u : 0u) << j;
                okbits |= (live && !pv ? 1u : 0u) << (KPI + j);
                if constexpr (F8) {
                    const u32x2 a = *reinterpret_cast<const u32x2*>(p + j * step);
                    const u32x2 b = *reinterpret_cast<const u32x2*>(p + j * step + row_bytes);
                    kr[j] = u32x4{a[0], a[1], 0u, 0u};
                    vr[j] = u32x4{b[0], b[1], 0u, 0u};
                } else {
                    kr[j] = *reinterpret_cast<const u32x4*>(p + j * step);
                    vr[j] = *reinterpret_cast<const u32x4*>(p + j * step + row_bytes);
                }
            }
        } else {
            uint32_t phys[KPI];
#pragma unroll
            for (int j = 0; j < KPI; ++j) phys[j] = page_of(entry_of(key0 + j), direct);
#pragma unroll
            for (int j = 0; j < KPI; ++j) {
                const uint32_t key = key0 + j;
                const uint32_t slot = key - entry_of(key) * block_tokens;
                const bool live = key <= kmax;
                const bool pv = phys[j] != 0xFFFFFFFFu;
                okbits |= (live && pv ? 1u : 0u) << j;
                okbits |= (live && !pv ? 1u : 0u) << (KPI + j);
                const uint8_t* p = pool + (uint64_t)(pv ? phys[j] : 0u) * page_bytes +
                                   (uint64_t)(pv ? slot * slot_bytes + head_off : 0u);
                if constexpr (F8) {
                    const u32x2 a = *reinterpret_cast<const u32x2*>(p);
                    const u32x2 b = *reinterpret_cast<const u32x2*>(p + row_bytes);
                    kr[j] = u32x4{a[0], a[1], 0u, 0u};
                    vr[j] = u32x4{b[0], b[1], 0u, 0u};
                } else {
                    kr[j] = *reinterpret_cast<const u32x4*>(p);
                    vr[j] = *reinterpret_cast<const u32x4*>(p + row_bytes);
                }
            }
        }
    };

    auto commit = [&](uint32_t t, int buf, bool raw = false) {
        uint8_t* ks = stage + buf * Gm::STAGE;
        uint8_t* vs = ks + Gm::KBYTES;
        if constexpr (F8) {  // codes -> f16, then the f16 staging below
#pragma unroll
            for (int j = 0; j < KPI; ++j) {
                kr[j] = e4m3x8_to_f16(kr[j][0], kr[j][1]);
                vr[j] = e4m3x8_to_f16(vr[j][0], vr[j][1]);
            }
        }
        if constexpr (B2H) {
            if (!raw) {  // bf16 -> f16; a value beyond f16's range flags the tile
                u16x2 emax = {0, 0};
#pragma unroll
                for (int j = 0; j < KPI; ++j) {
                    kr[j] = bf16x8_to_f16(kr[j], emax);
                    vr[j] = bf16x8_to_f16(vr[j], emax);
                }
                if (emax[0] >= BF16_F16_LIMIT || emax[1] >= BF16_F16_LIMIT) hdr->tile_big[buf] = t;
            }
        }
#pragma unroll
        for (int j = 0; j < KPI; ++j) {
            if (okbits != (1u << KPI) - 1u) {  // rare: keys past the window or on a bad page
                const bool z = !((okbits >> j) & 1u);
                vr[j] = z ? u32x4{0u, 0u, 0u, 0u} : vr[j];
            }
            *reinterpret_cast<u32x4*>(ks + (KPI * kg + j) * Gm::KPITCH + part * 16) = kr[j];
        }
        if constexpr (Gm::VROWM) {  // V rows like K rows
#pragma unroll
            for (int j = 0; j < KPI; ++j)
                *reinterpret_cast<u32x4*>(vs + (KPI * kg + j) * Gm::VRPITCH + part * 16) = vr[j];
        } else {
            static_assert(Gm::VROWM || KPI == 4, "a V^T group is 4 keys of one item");
            const uint32_t w[4][4] = {{vr[0][0], vr[0][1], vr[0][2], vr[0][3]},
                                      {vr[1][0], vr[1][1], vr[1][2], vr[1][3]},
                                      {vr[2][0], vr[2][1], vr[2][2], vr[2][3]},
                                      {vr[3][0], vr[3][1], vr[3][2], vr[3][3]}};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int d = part * 4 + i;
                const int col = (kg ^ (part & Gm::GMASK)) * Gm::GBYTES;  // d >> 2 == part
                *reinterpret_cast<u32x4*>(vs + d * Gm::VPITCH + col) =
                    u32x4{w[0][i], w[1][i], w[2][i], w[3][i]};
            }
        }
        if (part == 0) {
            uint32_t f = 0;
#pragma unroll
            for (int j = 0; j < KPI; ++j) f |= ((okbits >> j) & 1u) << (8 * j);
            if constexpr (KPI == 4)
                *reinterpret_cast<uint32_t*>(kflag + buf * N + 4 * kg) = f;
            else
                *reinterpret_cast<uint16_t*>(kflag + buf * N + 2 * kg) = (uint16_t)f;
        }
        if (okbits >> KPI) hdr->tile_bad[buf] = t;
    };

    // ---- Q operands for this lane's row: contraction index mapping
    //   16-bit: step t, half h -> dims 16t + 8h + e (e < 8)
    //   f32:    step t = 4u + e, half h -> dim 8u + 4h + e
    constexpr int QSTEPS = HD / O::KS;
    const float qscale = scale_log2 * (F8 ? k_scale[hk] : 1.0f);  // E4M3: the K scale folds into q
    opv qa[QSTEPS], qb[O::SPLIT ? QSTEPS : 1];
    // 16-bit operands: the wave's q is scaled by 2^qe before the split and
    // its scores by qdown = 2^-qe after the MFMAs (both exact)
    float qdown = 1.0f;
    {
        const float* qrow = q + ((uint64_t)(qoff + tok) * n_head + head) * HD;
        if constexpr (Gm::ELT == 2) {
            float4 a[QSTEPS], c[QSTEPS];
            float amax = 0.0f;
#pragma unroll
            for (int t = 0; t < QSTEPS; ++t) {
                a[t] = *reinterpret_cast<const float4*>(qrow + 16 * t + 8 * h);
                c[t] = *reinterpret_cast<const float4*>(qrow + 16 * t + 8 * h + 4);
                amax = fmaxf(amax, fmaxf(fmaxf(fabsf(a[t].x), fabsf(a[t].y)),
                                         fmaxf(fabsf(a[t].z), fabsf(a[t].w))));
                amax = fmaxf(amax, fmaxf(fmaxf(fabsf(c[t].x), fabsf(c[t].y)),
                                         fmaxf(fabsf(c[t].z), fabsf(c[t].w))));
            }
            // one exponent for the wave's 32 rows (wave-uniform, so the
            // scale costs no vector register in the tile loop): a row's lo
            // halves stay normal down to 2^17 below the wave's largest element
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
            amax = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(
                                                 __builtin_bit_cast(int, amax))) * qscale;
            const int qe = q_exponent(amax);
            const float up = __builtin_amdgcn_ldexpf(qscale, qe);
            qdown = __builtin_amdgcn_ldexpf(1.0f, -qe);
#pragma unroll
            for (int t = 0; t < QSTEPS; ++t) {
                float x[8] = {a[t].x * up, a[t].y * up, a[t].z * up, a[t].w * up,
                              c[t].x * up, c[t].y * up, c[t].z * up, c[t].w * up};
#pragma unroll
                for (int e = 0; e < 8; ++e) opaque(x[e]);  // rounded once, then split
                pack8<CT>(x, qa[t], qb[O::SPLIT ? t : 0]);
            }
        } else {
#pragma unroll
            for (int u = 0; u < HD / 8; ++u) {
                const float4 a = *reinterpret_cast<const float4*>(qrow + 8 * u + 4 * h);
                qa[4 * u + 0] = a.x * qscale;
                qa[4 * u + 1] = a.y * qscale;
                qa[4 * u + 2] = a.z * qscale;
                qa[4 * u + 3] = a.w * qscale;
            }
        }
    }

    f32x16 acc[HD / 32];
#pragma unroll
    for (int i = 0; i < HD / 32; ++i) acc[i] = f32x16{};
    float m_run = -1e30f, l_run = 0.f;

    // ---- prologue
    if (tid == 0) {
        hdr->tile_bad[0] = 0xFFFFFFFFu;
        hdr->tile_bad[1] = 0xFFFFFFFFu;
        hdr->tile_big[0] = 0xFFFFFFFFu;
        hdr->tile_big[1] = 0xFFFFFFFFu;
    }
    stage_slice(0);
    __syncthreads();
    const bool loader = tid < Gm::NLOAD;  // uniform per wave
    if (loader) issue(0);

    for (uint32_t j = 0; j < n_tiles; ++j) {
        const int buf = j & 1;
        if (loader) commit(j, buf);
        if (j + 1 < n_tiles) {
            const uint32_t e_last = entry_of((j + 1) * N + N - 1);
            if (e_last >= hdr->slice_base + SLICE) {  // uniform
                __syncthreads();
                stage_slice(entry_of((j + 1) * N));
            }
        }
        __syncthreads();
        bool big = false;  // bf16 tile beyond f16's range: re-staged raw, exact bf16 path
        if constexpr (B2H) {
            big = hdr->tile_big[buf] == j;  // uniform: read after the barrier
            if (big) {
                if (loader) {
                    issue(j, true);
                    commit(j, buf, true);
                }
                __syncthreads();
            }
        }
        if (loader && j + 1 < n_tiles) issue(j + 1);

        const uint8_t* ks = stage + buf * Gm::STAGE;
        const uint8_t* vs = ks + Gm::KBYTES;
        const bool bad = hdr->tile_bad[buf] == j;
        // all score blocks of the tile first, one running-max update per tile,
        // then per block the weights and O^T += V^T P^T (one basic block: the
        // next block's weights can interleave with this block's MFMAs)
        f32x16 sv[Gm::SUB];
#pragma unroll
        for (int sb = 0; sb < Gm::SUB; ++sb) {
            const uint32_t kb = j * N + sb * 32;
            // S^T (32 keys x 32 rows) = K Q^T
            f32x16 s = f32x16{};
            const uint8_t* krow = ks + (sb * 32 + l32) * Gm::KPITCH;
            if constexpr (Gm::ELT == 2) {
                if (B2H && big) {  // uniform: raw bf16 keys, q (f16 hi + lo) split hi + lo bf16
#pragma unroll
                    for (int t = 0; t < QSTEPS; ++t) {
                        const typename OB::v a = *reinterpret_cast<const typename OB::v*>(krow + (16 * t + 8 * h) * 2);
                        // recomputed per use (kept out of the loop-invariant set:
                        // hoisted for every step it would hold 64 more registers)
                        opv qt = qa[t], qu = qb[t];
                        asm volatile("" : "+v"(qt), "+v"(qu));
                        float x[8];
#pragma unroll
                        for (int e = 0; e < 8; ++e) x[e] = (float)qt[e] + (float)qu[e];
                        typename OB::v qh, ql;
                        pack8<DT_BF16>(x, qh, ql);
                        s = OB::mma(a, qh, s);
                        s = OB::mma(a, ql, s);
                    }
                } else {
#pragma unroll
                    for (int t = 0; t < QSTEPS; ++t) {
                        const opv a = *reinterpret_cast<const opv*>(krow + (16 * t + 8 * h) * 2);
                        s = O::mma(a, qa[t], s);
                        if constexpr (O::SPLIT) s = O::mma(a, qb[t], s);
                    }
                }
            } else {
#pragma unroll
                for (int u = 0; u < HD / 8; ++u) {
                    const float4 a = *reinterpret_cast<const float4*>(krow + (8 * u + 4 * h) * 4);
                    s = O::mma(a.x, qa[4 * u + 0], s);
                    s = O::mma(a.y, qa[4 * u + 1], s);
                    s = O::mma(a.z, qa[4 * u + 2], s);
                    s = O::mma(a.w, qa[4 * u + 3], s);
                }
            }
            // causal / page mask; key of register r: kb + 8(r/4) + 4h + r%4
            if (bad || kb + 31u > wave_min) {
                const uint8_t* fl = kflag + buf * N + sb * 32;
#pragma unroll
                for (int g4 = 0; g4 < 4; ++g4) {
                    const int ko = 8 * g4 + 4 * h;
                    const uint32_t f = bad ? *reinterpret_cast<const uint32_t*>(fl + ko) : 0x01010101u;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const bool ok = (kb + ko + e <= lim) && ((f >> (8 * e)) & 1u);
                        s[4 * g4 + e] = ok ? s[4 * g4 + e] : -__builtin_inff();
                    }
                }
            }
            sv[sb] = s;
        }
        {
            float mx = sv[0][0];
#pragma unroll
            for (int sb = 0; sb < Gm::SUB; ++sb)
#pragma unroll
                for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sv[sb][r]);
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64)) * qdown;
            if (__builtin_amdgcn_ballot_w64(mx > m_run + RESCALE_LOG2)) {
                const float mn = fmaxf(m_run, mx);
                const float alpha = __builtin_amdgcn_exp2f(m_run - mn);
                l_run *= alpha;
#pragma unroll
                for (int i = 0; i < HD / 32; ++i) acc[i] *= alpha;
                m_run = mn;
            }
        }
#pragma unroll
        for (int sb = 0; sb < Gm::SUB; ++sb) {
            const f32x16 s = sv[sb];
            float p[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) p[r] = __builtin_amdgcn_exp2f(fmaf(s[r], qdown, -m_run));
            // O^T (HD x 32 rows) += V^T P^T
            if constexpr (Gm::ELT == 2) {
                opv pa[2], pb[2];
                pack8<CT>(p, pa[0], pb[0]);
                pack8<CT>(p + 8, pa[1], pb[1]);
                if (B2H && big) {  // uniform: P as hi + lo bf16 pairs (~16 bits), f32 sum
                    float ps = 0.f;
#pragma unroll
                    for (int r = 0; r < 16; ++r) ps += p[r];
                    l_run += ps;
                } else {  // the sum of the f16 weights the MFMAs see
                    // (pairs taken lane by lane: reading them through a u32x4
                    // bit-cast of pa[i] compiled, with ROCm 7.2's hipcc, to
                    // four dot2s of the first dword)
                    typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
                    const f16x2 one2 = {(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
                    for (int i = 0; i < 2; ++i)
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            l_run = __builtin_amdgcn_fdot2(f16x2{pa[i][2 * j], pa[i][2 * j + 1]},
                                                           one2, l_run, false);
                }

                const uint8_t* vtr = vs + vtr_off;
                // A = V^T[dims db*32 + l32][keys]: lane (l32, h) takes keys
                // 16st + 4h + 0..3 and 16st + 8 + 4h + 0..3 (the order P^T holds
                // them in), two transposed reads of 4 keys each; within a
                // 16-lane group c = lane % 16 points at key row 4h + c/4 (+ the
                // step's base) and dims 16 ((lane/16) % 2) + 4 (c % 4) ..
#pragma unroll
                for (int db = 0; db < HD / 32; ++db) {
#pragma unroll
                    for (int st = 0; st < 2; ++st) {
                        const uint8_t* vp = vtr + (sb * 32 + 16 * st) * Gm::VRPITCH + db * 64;
                        const uint64_t r0 = lds_read_tr(vp);
                        const uint64_t r1 = lds_read_tr(vp + 8 * Gm::VRPITCH);
                        const u32x4 w = u32x4{(uint32_t)r0, (uint32_t)(r0 >> 32), (uint32_t)r1,
                                              (uint32_t)(r1 >> 32)};
                        if (B2H && big) {  // uniform; P as hi + lo bf16, packed per step (rare path)
                            typename OB::v pbh, pbl;
                            pack8<DT_BF16>(p + 8 * st, pbh, pbl);
                            const typename OB::v ab = __builtin_bit_cast(typename OB::v, w);
                            acc[db] = OB::mma(ab, pbh, acc[db]);
                            acc[db] = OB::mma(ab, pbl, acc[db]);
                        } else {
                            const opv a = __builtin_bit_cast(opv, w);
                            acc[db] = O::mma(a, pa[st], acc[db]);
                        }
                    }
                }
            } else {
                float ps = 0.f;
#pragma unroll
                for (int r = 0; r < 16; ++r) ps += p[r];
                l_run += ps;
#pragma unroll
                for (int db = 0; db < HD / 32; ++db) {
                    const int d = db * 32 + l32;
                    const uint8_t* vrow = vs + d * Gm::VPITCH;
                    const int sw = (d >> 2) & Gm::GMASK;
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        const int g = sb * 8 + 2 * u + h;  // keys 8u+4h..
                        const float4 a = *reinterpret_cast<const float4*>(vrow + (g ^ sw) * Gm::GBYTES);
                        acc[db] = O::mma(a.x, p[4 * u + 0], acc[db]);
                        acc[db] = O::mma(a.y, p[4 * u + 1], acc[db]);
                        acc[db] = O::mma(a.z, p[4 * u + 2], acc[db]);
                        acc[db] = O::mma(a.w, p[4 * u + 3], acc[db]);
                    }
                }
            }
        }
    }

    // ---- epilogue: combine the two halves' sums, normalise, store
    const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
    const float inv = l_tot > 0.f ? (F8 ? v_scale[hk] : 1.0f) / l_tot : 0.f;
    if (row_ok) {
        float* orow = out + ((uint64_t)(qoff + tok) * n_head + head) * HD;
#pragma unroll
        for (int db = 0; db < HD / 32; ++db) {
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
                const int d = db * 32 + 8 * g4 + 4 * h;
                *reinterpret_cast<float4*>(orow + d) =
                    make_float4(acc[db][4 * g4 + 0] * inv, acc[db][4 * g4 + 1] * inv,
                                acc[db][4 * g4 + 2] * inv, acc[db][4 * g4 + 3] * inv);
            }
        }
    }
}


// ---------------------------------------------------------------------------
// Ping-pong prefill for pages whose tiles are staged as f16 (f16; bf16 below
// 2^16; E4M3), block_tokens a multiple of the staging item's keys.  The host
// library sends bf16 pages here (7-8 % faster than prefill() at config 3; f16
// and E4M3 pages ran 3 % slower here and stay on prefill()).
//
// Per 64-key tile a wave's work is MFMA-bound (S = K Q^T: 32 MFMAs with the q
// split; P.V: 16) or VALU-bound (mask, running max, 32 exponentials, packing,
// row sums).  With one barrier per tile the two waves of a SIMD run the same
// phase at the same time.  Here the halves of the workgroup take turns: waves
// 0-3 (one per SIMD) run their MFMA phase while waves 4-7 run their softmax,
// then they swap, with a workgroup barrier between the phases.  A wave's MFMA
// phase is P.V of the previous tile, then S of the current one, so P stays in
// registers; it ends by staging the next tile (waves 0-3 write K one tile
// ahead, waves 4-7 write V) behind its last MFMAs:
//   interval 2j  : waves 0-3 MFMA [P.V(j-1), S(j)], write K(j+1)  waves 4-7 softmax(j-1)
//   interval 2j+1: waves 0-3 softmax(j)   waves 4-7 MFMA [P.V(j-1), S(j)], write V(j)
// K(j+1) is read at intervals 2j+2 and 2j+3 and its buffer next written at
// 2j+4; V(j) is read at 2j+2 and 2j+3 and its buffer next written at 2j+5:
// two buffers of each.  Tile t's key flags are written at 2t-2 and read by the
// softmaxes at 2t+1 and 2t+2: three buffers.  The barriers wait for LDS only:
// each staging thread's global loads for the next tile (and the page id for
// the one after) stay in flight across them.  Operands, masking and softmax
// are those of prefill(), in the same order per accumulator (bit-identical
// outputs where both walk 64-key tiles, head_dim 128).  A bf16 tile holding a
// value of magnitude >= 2^16 raises a flag that every wave reads after the
// next barrier; the workgroup then restarts on prefill(), which computes such
// tiles exactly.
template <int HD>
struct ppg {
    static constexpr int N = 64;                 // keys per tile
    static constexpr int SUB = N / 32;           // 32-key score blocks per tile
    static constexpr int PARTS = HD / 8;         // 8-element chunks per head row
    static constexpr int KPI = N * PARTS / 256;  // keys per staging item (256 threads per K or V tile)
    static constexpr int KPITCH = HD * 2 + 16;   // bytes per K row in LDS (f16)
    static constexpr int VRPITCH = HD * 2 + 128; // bytes per V row in LDS (f16)
    static constexpr int KBYTES = N * KPITCH;
    static constexpr int VBYTES = N * VRPITCH;
    static constexpr int KFLAG = 64;             // [3][N] key valid bytes
    static constexpr int KB0 = KFLAG + 3 * N;    // two K buffers
    static constexpr int VB0 = KB0 + 2 * KBYTES; // two V buffers
    static constexpr int BYTES = VB0 + 2 * VBYTES;
    static_assert(KPI >= 1 && N * PARTS == 256 * KPI, "one staging item per thread of a half");
};

struct pp_hdr {
    uint32_t tile_bad[2];  // tile index whose keys include an invalid page
    uint32_t big_at;       // bf16 pages: interval that staged a value beyond f16's range
};

// Block-table entries per staging item for the ping-pong kernel (keys of an
// item share one page when block_tokens is a multiple of it).
template <int HD>
constexpr uint32_t pp_item_keys() { return (uint32_t)ppg<HD>::KPI; }

template <int DT, int HD>
__device__ __forceinline__ void prefill_pp(
    const float* __restrict__ q, const uint8_t* __restrict__ pool,
    const uint32_t* __restrict__ bt_all, uint32_t bt_stride, uint32_t bt_entries,
    const uint32_t* __restrict__ cu_q, const uint32_t* __restrict__ start_pos,
    const uint32_t* __restrict__ pos_ptr, uint32_t q_tokens, uint32_t pos_offset,
    float* __restrict__ out, uint32_t n_head, uint32_t n_head_kv, uint32_t block_tokens,
    int bt_shift, uint32_t row_bytes, float scale_log2, uint64_t n_blocks, uint8_t* smem,
    const float* __restrict__ k_scale, const float* __restrict__ v_scale) {
    static_assert(DT == DT_F16 || DT == DT_BF16 || DT == DT_FP8, "f16-staged pages only");
    constexpr bool B2H = DT == DT_BF16;
    constexpr bool F8 = DT == DT_FP8;
    typedef op_t<DT_F16> O;
    typedef f16x8 opv;
    typedef ppg<HD> G;
    constexpr int N = G::N;
    constexpr int SUB = G::SUB;
    constexpr int KPI = G::KPI;
    constexpr uint32_t SE = F8 ? 1u : 2u;  // stored element bytes

    // ---- workgroup order: as prefill() (longest row block first)
    const uint32_t gx = gridDim.x, gy = gridDim.y;
    const uint32_t pairs = gy * gridDim.z;
    const uint32_t d = blockIdx.x + gx * (blockIdx.y + gy * blockIdx.z);
    const uint32_t tile = gx - 1u - d / pairs;
    const uint32_t hk = (d % pairs) % gy;
    const uint32_t b = (d % pairs) / gy;

    uint32_t qoff, n_q, p0;
    const uint32_t* bt;
    if (cu_q) {
        qoff = min(cu_q[b], q_tokens);
        const uint32_t end = min(cu_q[b + 1], q_tokens);
        n_q = end > qoff ? end - qoff : 0u;
        p0 = start_pos[b];
        bt = bt_all + (uint64_t)b * bt_stride;
    } else {
        qoff = 0;
        n_q = q_tokens;
        p0 = pos_ptr ? pos_ptr[0] : pos_offset;
        bt = bt_all;
    }
    const uint32_t group = n_head / n_head_kv;
    const uint32_t rows = n_q * group;
    const uint32_t row0 = tile * ROWS;
    if (row0 >= rows) return;  // uniform over the workgroup

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int grp = wave >> 2;  // 0: waves 0-3 (stage K), 1: waves 4-7 (stage V)
    const int l32 = lane & 31;
    const int h = lane >> 5;
    const uint32_t vtr_off = (4 * h + ((lane & 15) >> 2)) * G::VRPITCH +
                             (16 * ((lane >> 4) & 1) + 4 * (lane & 3)) * 2;

    const uint32_t row_raw = row0 + wave * 32 + l32;
    const bool row_ok = row_raw < rows;
    const uint32_t row = row_ok ? row_raw : rows - 1u;
    const uint32_t tok = row / group;
    const uint32_t head = hk * group + (row - tok * group);
    const uint64_t cap = (uint64_t)bt_entries * block_tokens - 1u;
    auto clamp_pos = [&](uint32_t t) -> uint32_t {
        const uint64_t v = (uint64_t)p0 + t;
        return (uint32_t)(v < cap ? v : cap);
    };
    const uint32_t lim = clamp_pos(tok);
    const uint32_t wr0 = min(row0 + wave * 32u, rows - 1u);
    const uint32_t wave_min = clamp_pos(wr0 / group);
    const uint32_t kmax = clamp_pos(min(row0 + ROWS - 1u, rows - 1u) / group);
    const uint32_t n_tiles = kmax / N + 1u;

    pp_hdr* hdr = reinterpret_cast<pp_hdr*>(smem);
    uint8_t* kflag = smem + G::KFLAG;
    uint8_t* kbuf0 = smem + G::KB0;
    uint8_t* vbuf0 = smem + G::VB0;

    // ---- staging item of this thread: keys KPI*kg .. of a tile, 8-element
    // chunk `part` of the kv head's K row (waves 0-3) or V row (waves 4-7)
    const int sti = tid & 255;
    const int part = sti % G::PARTS;
    const int kg = sti / G::PARTS;
    const uint64_t page_bytes = (uint64_t)block_tokens * 2u * row_bytes;
    const uint32_t slot_bytes = 2u * row_bytes;
    const uint32_t src_off = (grp ? row_bytes : 0u) + hk * HD * SE + part * 8u * SE;
    auto entry_of = [&](uint32_t key) -> uint32_t {
        return bt_shift >= 0 ? (key >> bt_shift) : key / block_tokens;
    };
    // The table entry of this item's keys in the next tile to issue is read
    // one tile ahead and checked only when that tile is issued: a check right
    // after the load would wait for every load in flight.  (bt_entries >= 1.)
    uint32_t ph_e = entry_of(KPI * kg);
    uint32_t ph = bt[min(ph_e, bt_entries - 1u)];
    u32x4 r[KPI];
    uint32_t okb = 0;  // bit j: key KPI*kg+j loadable; bit KPI+j: key <= kmax on a bad page
    // Staging comes in pieces so that an MFMA phase can run them between its
    // MFMAs (issue_addr, issue_key(j), issue_page; commit_key(j), commit_flags).
    const uint8_t* ip = pool;  // address of key 0 of the item being issued
    uint32_t istep = 0;        // bytes between its keys
    auto issue_addr = [&](uint32_t t) {
        const uint32_t key0 = t * N + KPI * kg;
        const uint32_t slot = key0 - ph_e * block_tokens;
        const bool pv = ph_e < bt_entries && (uint64_t)ph < n_blocks;
        // an invalid page reads page 0 (in bounds; its keys are masked)
        ip = pool + (uint64_t)(pv ? ph : 0u) * page_bytes + (pv ? slot * slot_bytes : 0u) + src_off;
        istep = pv ? slot_bytes : 0u;
        okb = 0;
#pragma unroll
        for (int j = 0; j < KPI; ++j) {
            const bool live = key0 + j <= kmax;
            okb |= (live && pv ? 1u : 0u) << j;
            okb |= (live && !pv ? 1u : 0u) << (KPI + j);
        }
    };
    auto issue_key = [&](int j) {
        if constexpr (F8) {
            const u32x2 a = *reinterpret_cast<const u32x2*>(ip + j * istep);
            r[j] = u32x4{a[0], a[1], 0u, 0u};
        } else {
            r[j] = *reinterpret_cast<const u32x4*>(ip + j * istep);
        }
    };
    auto issue_page = [&](uint32_t t) {  // the table entry for tile t + 1
        if (t + 1 < n_tiles) {
            ph_e = entry_of((t + 1) * N + KPI * kg);
            ph = bt[min(ph_e, bt_entries - 1u)];
        }
    };
    auto issue = [&](uint32_t t) {
        issue_addr(t);
#pragma unroll
        for (int j = 0; j < KPI; ++j) issue_key(j);
        issue_page(t);
    };
    // key j of the issued item into its tile buffer (bf16: widened, emax
    // gathering the range check)
    auto commit_key = [&](uint32_t t, int j, u16x2& emax) {
        const int bb = t & 1;
        u32x4 w = r[j];
        if constexpr (F8) w = e4m3x8_to_f16(w[0], w[1]);
        if constexpr (B2H) w = bf16x8_to_f16(w, emax);
        if (grp == 0) {
            *reinterpret_cast<u32x4*>(kbuf0 + bb * G::KBYTES + (KPI * kg + j) * G::KPITCH +
                                      part * 16) = w;
        } else {
            // keys past the window or on a bad page: zero rows (their weights
            // are 0, and 0 * a non-finite pool value would not be)
            const bool z = !((okb >> j) & 1u);
            *reinterpret_cast<u32x4*>(vbuf0 + bb * G::VBYTES + (KPI * kg + j) * G::VRPITCH +
                                      part * 16) = z ? u32x4{0u, 0u, 0u, 0u} : w;
        }
    };
    // the item's key flags (K stagers) and the bf16 range flag (interval `iv`)
    auto commit_flags = [&](uint32_t t, uint32_t iv, u16x2 emax) {
        const int bb = t & 1;
        if constexpr (B2H) {
            if (emax[0] >= BF16_F16_LIMIT || emax[1] >= BF16_F16_LIMIT) hdr->big_at = iv;
        }
        if (grp == 0) {
            if (part == 0) {
                uint32_t f = 0;
#pragma unroll
                for (int j = 0; j < KPI; ++j) f |= ((okb >> j) & 1u) << (8 * j);
                // three flag buffers: tile t's are written during interval 2t-2
                // and read by the softmaxes at 2t+1 and 2t+2
                uint8_t* fl = kflag + (t % 3u) * N;
                if constexpr (KPI == 4)
                    *reinterpret_cast<uint32_t*>(fl + 4 * kg) = f;
                else if constexpr (KPI == 2)
                    *reinterpret_cast<uint16_t*>(fl + 2 * kg) = (uint16_t)f;
                else
                    fl[kg] = (uint8_t)f;
            }
            if (okb >> KPI) hdr->tile_bad[bb] = t;
        }
    };
    auto commit = [&](uint32_t t, uint32_t iv) {
        u16x2 emax = {0, 0};
#pragma unroll
        for (int j = 0; j < KPI; ++j) commit_key(t, j, emax);
        commit_flags(t, iv, emax);
    };

    // ---- q operands (as prefill(): scaled per wave by a power of two, split
    // hi + lo f16 behind opaque())
    constexpr int QSTEPS = HD / O::KS;
    const float qscale = scale_log2 * (F8 ? k_scale[hk] : 1.0f);
    opv qa[QSTEPS], qb[QSTEPS];
    float qdown;
    {
        const float* qrow = q + ((uint64_t)(qoff + tok) * n_head + head) * HD;
        float4 a[QSTEPS], c[QSTEPS];
        float amax = 0.0f;
#pragma unroll
        for (int t = 0; t < QSTEPS; ++t) {
            a[t] = *reinterpret_cast<const float4*>(qrow + 16 * t + 8 * h);
            c[t] = *reinterpret_cast<const float4*>(qrow + 16 * t + 8 * h + 4);
            amax = fmaxf(amax, fmaxf(fmaxf(fabsf(a[t].x), fabsf(a[t].y)),
                                     fmaxf(fabsf(a[t].z), fabsf(a[t].w))));
            amax = fmaxf(amax, fmaxf(fmaxf(fabsf(c[t].x), fabsf(c[t].y)),
                                     fmaxf(fabsf(c[t].z), fabsf(c[t].w))));
        }
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
        amax = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(
                                             __builtin_bit_cast(int, amax))) * qscale;
        const int qe = q_exponent(amax);
        const float up = __builtin_amdgcn_ldexpf(qscale, qe);
        qdown = __builtin_amdgcn_ldexpf(1.0f, -qe);
#pragma unroll
        for (int t = 0; t < QSTEPS; ++t) {
            float x[8] = {a[t].x * up, a[t].y * up, a[t].z * up, a[t].w * up,
                          c[t].x * up, c[t].y * up, c[t].z * up, c[t].w * up};
#pragma unroll
            for (int e = 0; e < 8; ++e) opaque(x[e]);
            pack8<DT_F16>(x, qa[t], qb[t]);
        }
    }

    f32x16 acc[HD / 32];
#pragma unroll
    for (int i = 0; i < HD / 32; ++i) acc[i] = f32x16{};
    float m_run = -1e30f, l_run = 0.f;
    f32x16 sv[SUB];   // scores of the tile between a wave's MFMA phase and its softmax
    opv pf[SUB][2];   // f16 weights of the tile between its softmax and the next MFMA phase

    // a barrier that waits for this wave's LDS traffic only
    auto bar = [&]() {
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
        __builtin_amdgcn_sched_barrier(0);
    };
    // every wave reads the flag after the same barrier: a value set during
    // interval iv is acted on at the start of interval iv + 1
    auto big_seen = [&](uint32_t iv) -> bool {
        if constexpr (B2H) return hdr->big_at < iv;
        else return false;
    };

    // MFMA phase: O^T += V^T P^T for tile j-1 (pv), then S^T = K Q^T for tile j
    // (sc).  In this phase no other wave of the SIMD issues MFMAs, so each
    // operand is read from LDS ahead of its MFMA (P.V: PV_AHEAD MFMAs ahead;
    // S: one step ahead) and the order is pinned with sched_barrier: left to
    // itself the scheduler read each K operand right before its MFMAs and the
    // matrix unit idled through every LDS round trip (a 48-MFMA phase took
    // ~3000 cycles for 1536 of MFMA work).  The two score blocks' chains and
    // the four P.V accumulators interleave; each accumulator sees its MFMAs
    // in the order of prefill().
    static_assert(SUB == 2, "two 32-key score blocks per tile");
    bool bad_nx = false;  // tile of the next softmax holds a key on an invalid page
    constexpr int NPV = SUB * 2 * (HD / 32);  // P.V MFMAs per tile: (sb, st, db)
    constexpr int PV_AHEAD = 4;
    constexpr uint32_t NONE = 0xFFFFFFFFu;
    auto mma_phase = [&](uint32_t j, bool pv, bool sc, uint32_t commit_t = NONE,
                         uint32_t issue_t = NONE, uint32_t iv = 0) {
        // the MFMA phase issues ahead of the other half's softmax on the SIMD
        // (without it the older waves 0-3 won every issue conflict and
        // waves 4-7 ran both of their phases late)
        __builtin_amdgcn_s_setprio(1);
        const uint8_t* vtr = vbuf0 + ((j - 1u) & 1u) * G::VBYTES + vtr_off;
        const uint8_t* kr = kbuf0 + (j & 1u) * G::KBYTES + l32 * G::KPITCH + 16 * h;
        // operand of P.V MFMA i: sub-block i / (2 HD/32), step (i / (HD/32)) % 2, dims block i % (HD/32)
        auto vread = [&](int i) -> opv {
            const int sb = i / (2 * (HD / 32)), st = (i / (HD / 32)) & 1, db = i % (HD / 32);
            const uint8_t* vp = vtr + (sb * 32 + 16 * st) * G::VRPITCH + db * 64;
            const uint64_t r0 = lds_read_tr(vp);
            const uint64_t r1 = lds_read_tr(vp + 8 * G::VRPITCH);
            return __builtin_bit_cast(opv, u32x4{(uint32_t)r0, (uint32_t)(r0 >> 32), (uint32_t)r1,
                                                 (uint32_t)(r1 >> 32)});
        };
        auto kread = [&](int t, int sb) -> opv {
            return *reinterpret_cast<const opv*>(kr + sb * 32 * G::KPITCH + 32 * t);
        };
        opv ka0, ka1;
        if (sc) {
            ka0 = kread(0, 0);
            ka1 = kread(0, 1);
        }
        if (pv) {
            opv vq[PV_AHEAD];
#pragma unroll
            for (int i = 0; i < PV_AHEAD; ++i) vq[i] = vread(i);
#pragma unroll
            for (int i = 0; i < NPV; ++i) {
                __builtin_amdgcn_sched_barrier(0);
                const int db = i % (HD / 32);
                const int sb = i / (2 * (HD / 32)), st = (i / (HD / 32)) & 1;
                acc[db] = O::mma(vq[i % PV_AHEAD], pf[sb][st], acc[db]);
                if (i + PV_AHEAD < NPV) vq[i % PV_AHEAD] = vread(i + PV_AHEAD);
            }
        }
        if (sc) {
            // the next softmax is tile j's: its page flag is read here, where
            // the LDS round trip hides under the MFMAs
            bad_nx = hdr->tile_bad[j & 1u] == j;
            f32x16 s0 = f32x16{}, s1 = f32x16{};
#pragma unroll
            for (int t = 0; t < QSTEPS; ++t) {
                __builtin_amdgcn_sched_barrier(0);
                opv kn0 = ka0, kn1 = ka1;
                if (t + 1 < QSTEPS) {
                    kn0 = kread(t + 1, 0);
                    kn1 = kread(t + 1, 1);
                }
                __builtin_amdgcn_sched_barrier(0);  // step t+1's reads go out before step t's MFMAs
                s0 = O::mma(ka0, qa[t], s0);
                s1 = O::mma(ka1, qa[t], s1);
                s0 = O::mma(ka0, qb[t], s0);
                s1 = O::mma(ka1, qb[t], s1);
                ka0 = kn0;
                ka1 = kn1;
            }
            __builtin_amdgcn_sched_barrier(0);
            sv[0] = s0;
            sv[1] = s1;
        }
        // staging ends the MFMA phase, behind its last MFMAs and operand
        // reads: this thread's item of tile commit_t goes to LDS, then its
        // loads of tile issue_t go out.  (At the start of the phase it
        // measured 1.3 % slower for bf16 pages, after the P.V MFMAs 0.6 %; in
        // the softmax phase it made that phase the longer one, and spread
        // between the MFMAs slower still.)
        __builtin_amdgcn_sched_barrier(0);
        if (commit_t != NONE) {
            commit(commit_t, iv);
            if (issue_t != NONE) issue(issue_t);
        }
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(0);
    };

    // softmax phase for tile j: mask, one running-max update, weights (f16,
    // in the P^T layout of the next MFMA phase) and their row sums
    auto softmax = [&](uint32_t j) {
        const int bb = j & 1;
        const bool bad = bad_nx;
#pragma unroll
        for (int sb = 0; sb < SUB; ++sb) {
            const uint32_t kb = j * N + sb * 32;
            if (bad || kb + 31u > wave_min) {
                const uint8_t* fl = kflag + (j % 3u) * N + sb * 32;
#pragma unroll
                for (int g4 = 0; g4 < 4; ++g4) {
                    const int ko = 8 * g4 + 4 * h;
                    const uint32_t f = bad ? *reinterpret_cast<const uint32_t*>(fl + ko) : 0x01010101u;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const bool ok = (kb + ko + e <= lim) && ((f >> (8 * e)) & 1u);
                        sv[sb][4 * g4 + e] = ok ? sv[sb][4 * g4 + e] : -__builtin_inff();
                    }
                }
            }
        }
        {
            float mx = sv[0][0];
#pragma unroll
            for (int sb = 0; sb < SUB; ++sb)
#pragma unroll
                for (int r2 = 0; r2 < 16; ++r2) mx = fmaxf(mx, sv[sb][r2]);
            mx = max_halves(mx) * qdown;
            if (__builtin_amdgcn_ballot_w64(mx > m_run + RESCALE_LOG2)) {
                const float mn = fmaxf(m_run, mx);
                const float alpha = __builtin_amdgcn_exp2f(m_run - mn);
                l_run *= alpha;
#pragma unroll
                for (int i = 0; i < HD / 32; ++i) acc[i] *= alpha;
                m_run = mn;
            }
        }
        typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
        const f16x2 one2 = {(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
        for (int sb = 0; sb < SUB; ++sb) {
#pragma unroll
            for (int st = 0; st < 2; ++st) {
                opv pv;
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    pv[e] = (_Float16)__builtin_amdgcn_exp2f(fmaf(sv[sb][8 * st + e], qdown, -m_run));
                pf[sb][st] = pv;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    l_run = __builtin_amdgcn_fdot2(f16x2{pv[2 * e], pv[2 * e + 1]}, one2, l_run, false);
            }
        }
        // the weights and sums are made here, before the barrier that ends
        // the phase: the optimiser otherwise sank the exponentials into the
        // MFMA phase that consumes them
#pragma unroll
        for (int sb = 0; sb < SUB; ++sb)
#pragma unroll
            for (int st = 0; st < 2; ++st) asm volatile("" : "+v"(pf[sb][st]));
        asm volatile("" : "+v"(l_run));
    };

    // ---- prologue: page ids and the first tile's loads, q, then K(0)
    if (tid == 0) {
        hdr->tile_bad[0] = 0xFFFFFFFFu;
        hdr->tile_bad[1] = 0xFFFFFFFFu;
        hdr->big_at = 0xFFFFFFFFu;
    }
    issue(0);
    {  // tile -1 (see the main loop): its V buffer (1) holds zeros
        u32x4* z = reinterpret_cast<u32x4*>(vbuf0 + G::VBYTES);
        for (int i = tid; i < G::VBYTES / 16; i += NT) z[i] = u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int sb = 0; sb < SUB; ++sb)
#pragma unroll
        for (int r2 = 0; r2 < 16; ++r2) sv[sb][r2] = -__builtin_inff();
#pragma unroll
    for (int sb = 0; sb < SUB; ++sb) pf[sb][0] = pf[sb][1] = opv{};
    bar();  // header initialised
    if (grp == 0) {
        commit(0, 0);
        if (n_tiles > 1) issue(1);
    }
    bar();

    // ---- main loop: interval 2j has number 2j + 1 (the prologue is 0)
    // Both loops run the same body for every tile, the first one included
    // (with a first iteration of their own the compiler peeled it, and the
    // loads it issued into other registers made it wait for every load in
    // flight at the head of each MFMA phase).  Tile -1 is a zero tile: its
    // scores are -inf, its weights 0 and its V buffer zeroed in the prologue,
    // so its P.V adds exact zeros and its softmax changes nothing.
    bool exact = false;
    if (grp == 0) {
        for (uint32_t j = 0; j < n_tiles; ++j) {
            if (big_seen(2 * j + 1)) { exact = true; break; }
            mma_phase(j, true, true, j + 1 < n_tiles ? j + 1 : NONE, j + 2 < n_tiles ? j + 2 : NONE,
                      2 * j + 1);
            bar();
            if (big_seen(2 * j + 2)) { exact = true; break; }
            softmax(j);
            bar();
        }
        if (!exact) {
            mma_phase(n_tiles, true, false);
            bar();
            bar();
        }
    } else {
        for (uint32_t j = 0; j < n_tiles; ++j) {
            if (big_seen(2 * j + 1)) { exact = true; break; }
            softmax(j - 1u);
            bar();
            if (big_seen(2 * j + 2)) { exact = true; break; }
            mma_phase(j, true, true, j, j + 1 < n_tiles ? j + 1 : NONE, 2 * j + 2);
            bar();
        }
        if (!exact) {
            softmax(n_tiles - 1);
            bar();
            mma_phase(n_tiles, true, false);
            bar();
        }
    }
    if constexpr (B2H) {
        if (exact) {  // uniform over the workgroup: every wave broke at the same interval
            bar();
            // (inlined: with the restart in the kernel the bf16 kernel keeps 3
            // VGPRs of the prologue in scratch across the tile loops, stored once
            // before them and reloaded once after; as a called function the
            // kernel would carry 468 bytes of scratch per lane instead)
            prefill<DT_BF16, HD>(q, pool, bt_all, bt_stride, bt_entries, cu_q, start_pos, pos_ptr,
                                 q_tokens, pos_offset, out, n_head, n_head_kv, block_tokens,
                                 bt_shift, row_bytes, scale_log2, n_blocks, smem, k_scale,
                                 v_scale);
            return;
        }
    }

    // ---- epilogue: combine the two halves' sums, normalise, store
    const float l_tot = sum_halves(l_run);
    const float inv = l_tot > 0.f ? (F8 ? v_scale[hk] : 1.0f) / l_tot : 0.f;
    if (row_ok) {
        float* orow = out + ((uint64_t)(qoff + tok) * n_head + head) * HD;
#pragma unroll
        for (int db = 0; db < HD / 32; ++db) {
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
                const int dd = db * 32 + 8 * g4 + 4 * h;
                *reinterpret_cast<float4*>(orow + dd) =
                    make_float4(acc[db][4 * g4 + 0] * inv, acc[db][4 * g4 + 1] * inv,
                                acc[db][4 * g4 + 2] * inv, acc[db][4 * g4 + 3] * inv);
            }
        }
    }
}

}  // namespace

#define EH_PREFILL(DTN, DT, HD)                                                                   \
    extern "C" __global__ __launch_bounds__(NT, 1) void eh_prefill_##DTN##_hd##HD(              \
        const float* q, const uint8_t* pool, const uint32_t* bt, uint32_t bt_stride,             \
        uint32_t bt_entries, const uint32_t* cu_q, const uint32_t* start_pos,                    \
        const uint32_t* pos_ptr, uint32_t q_tokens, uint32_t pos_offset, float* out,             \
        uint32_t n_head, uint32_t n_head_kv, uint32_t block_tokens, int bt_shift,                \
        uint32_t row_bytes, float scale_log2, uint64_t n_blocks, const float* k_scale,           \
        const float* v_scale) {                                                                  \
        constexpr int BYTES = 64 + SLICE * 4 + 2 * geo<DT, HD>::N + 2 * geo<DT, HD>::STAGE;      \
        __shared__ __attribute__((aligned(16))) uint8_t smem[BYTES];                             \
        prefill<DT, HD>(q, pool, bt, bt_stride, bt_entries, cu_q, start_pos, pos_ptr, q_tokens,  \
                        pos_offset, out, n_head, n_head_kv, block_tokens, bt_shift, row_bytes,   \
                        scale_log2, n_blocks, smem, k_scale, v_scale);                           \
    }

EH_PREFILL(f16, DT_F16, 64)
EH_PREFILL(f16, DT_F16, 128)
EH_PREFILL(bf16, DT_BF16, 64)
EH_PREFILL(bf16, DT_BF16, 128)
EH_PREFILL(f32, DT_F32, 64)
EH_PREFILL(f32, DT_F32, 128)
EH_PREFILL(fp8, DT_FP8, 64)
EH_PREFILL(fp8, DT_FP8, 128)

// Ping-pong kernels (f16-staged pages, block_tokens a multiple of
// pp_item_keys<HD>()); bf16 reserves the LDS of prefill() for its exact restart.
#define EH_PREFILL_PP(DTN, DT, HD)                                                                \
    extern "C" __global__ __launch_bounds__(NT, 1) void eh_prefill_pp_##DTN##_hd##HD(           \
        const float* q, const uint8_t* pool, const uint32_t* bt, uint32_t bt_stride,             \
        uint32_t bt_entries, const uint32_t* cu_q, const uint32_t* start_pos,                    \
        const uint32_t* pos_ptr, uint32_t q_tokens, uint32_t pos_offset, float* out,             \
        uint32_t n_head, uint32_t n_head_kv, uint32_t block_tokens, int bt_shift,                \
        uint32_t row_bytes, float scale_log2, uint64_t n_blocks, const float* k_scale,           \
        const float* v_scale) {                                                                  \
        constexpr int OLD = 64 + SLICE * 4 + 2 * geo<DT, HD>::N + 2 * geo<DT, HD>::STAGE;        \
        constexpr int BYTES = (DT == DT_BF16 && OLD > ppg<HD>::BYTES) ? OLD : ppg<HD>::BYTES;   \
        __shared__ __attribute__((aligned(16))) uint8_t smem[BYTES];                             \
        prefill_pp<DT, HD>(q, pool, bt, bt_stride, bt_entries, cu_q, start_pos, pos_ptr,         \
                           q_tokens, pos_offset, out, n_head, n_head_kv, block_tokens, bt_shift, \
                           row_bytes, scale_log2, n_blocks, smem, k_scale, v_scale);             \
    }

EH_PREFILL_PP(f16, DT_F16, 64)
EH_PREFILL_PP(f16, DT_F16, 128)
EH_PREFILL_PP(bf16, DT_BF16, 64)
EH_PREFILL_PP(bf16, DT_BF16, 128)
EH_PREFILL_PP(fp8, DT_FP8, 64)
EH_PREFILL_PP(fp8, DT_FP8, 128)
