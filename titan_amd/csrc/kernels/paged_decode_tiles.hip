// paged_decode_tiles.hip -- token-balanced paged decode for gfx950 (CDNA4, wave64).
//
// Semantics: the reference decode attention (engine-cuda/kernels/
// paged_attention.cu:6-103, split-K form :200-369) and its CPU authority
// sdpa_decode (engine-core/src/forward_cpu.rs:424-510): q head qh reads kv
// head qh / (n_head / n_head_kv), attends logical tokens t < n_b with
// scores q.k / sqrt(head_dim), out = softmax-weighted V (zeros if n_b == 0).
// With new_k/new_v the launch first appends one token per sequence at
// position n_b - 1 (the scatter of paged_kv.cu:13-45 / the decode-time append
// slot of norm_rope.cu:280-298) and attends it in the same pass.
//
// Work decomposition (MI355X-first):
//   * the ragged batch is cut into 16-token tiles; every workgroup of the
//     grid takes an equal run of consecutive tiles of the flattened
//     (sequence, tile) order, cut on the device from the live lengths, so
//     the load is balanced whatever the context mix and a captured graph
//     stays correct as contexts grow;
//   * a run has one wave per kv head; the waves walk the same tiles, so
//     together they stream whole pages (all kv heads of each token slot),
//     and each wave owns the complete softmax state of its q heads; a
//     workgroup of 8 waves holds 8 / n_kv runs (fewer, larger workgroups
//     dispatch faster) that share one scan of the lengths;
//   * q.k is one MFMA tile per 16 tokens: S[16 tok x 16 heads] =
//     K[16 x 128] . Q^T with v_mfma_f32_16x16x32 (f16 or bf16), q split into
//     hi + lo 16-bit halves (two MFMAs per step) so scores keep ~22 bits
//     (an f16 lo half below 2^-14 is a subnormal: its 2^-24 step still
//     leaves q ~21 bits at the scale of the contract's data);
//   * the score tile leaves lane (g, x) = (lane / 16, lane % 16) with the
//     scores of tokens 4g..4g+3 for head x; the online softmax runs there in
//     the log2 domain with a lazy rescale (the running max only moves when a
//     score exceeds it by 2^8; every weight uses the same stale max, exact);
//   * P.V is MFMA too: O^T[16 dims x 16 heads] += V^T . P^T with
//     v_mfma_f32_16x16x16.  P^T is exactly the score tile each lane holds
//     (f16 P; bf16 P as hi + lo halves); V^T comes from the V tile staged in
//     LDS through the gfx950 transposed read ds_read_b64_tr_b16; with f16 P
//     the weight sums l add the rounded f16 weights the MFMAs see, so acc / l
//     stays a weighted mean (a dominant weight rounded by up to 2^-11 would
//     otherwise shift the output by that much of its V row);
//   * E4M3 pages apply the K scale to the scores after the MFMAs (folded
//     into q, q * scale ~ 1e-3 would leave its lo halves only a few bits);
//   * every wave keeps DEPTH tiles of K/V loads in flight (16-byte lanes,
//     K in the MFMA A layout) and fetches its page ids in batches of 64
//     tiles, read back by v_readlane;
//   * a wave writes its state when its run leaves a sequence: the final
//     rows when the whole sequence lies in the workgroup, else one partial
//     (m, l, acc) that eh_decode_tiles_merge combines.
// E4M3 pages (OCP E4M3FN codes with one f32 scale per kv head for K and for
// V) are converted to f16 in registers -- exact, every E4M3 value is an f16 --
// and take the f16 path: the K scale multiplies the scores, the V scale the
// written rows and partials.
// Pages must be a power of two of at least 16 tokens; head_dim 128;
// at most 8 q heads per kv head; block-table entries past the table or the
// pool mask their tokens.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "e4m3.h"

namespace {

enum { DT_F16 = 1, DT_BF16 = 2, DT_FP8 = 3 };

constexpr int TILE = 16;         // tokens per tile (MFMA rows)
constexpr int QSEG = 2;          // sequences per run whose q is staged in LDS up front
constexpr float RESCALE = 8.0f;  // lazy-rescale threshold, log2 domain
constexpr float NEG_BIG = -1e30f;
constexpr int VROW = 288;        // LDS bytes per V token row (256 + 32: conflict-free transposed reads)


typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

// Transposed LDS read (ds_read_b64_tr_b16): in each 16-lane group, lane
// 4r + b points at 4 consecutive 16-bit elements of row r (columns 4b..4b+3)
// of a 4 x 16 block; lane c receives column c of rows 0..3.
__device__ __forceinline__ uint64_t lds_read_tr(const uint8_t* p) {
    const i16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(const_cast<uint8_t*>(p)));
    return __builtin_bit_cast(uint64_t, v);
}

template <int DT> struct kvt;
template <> struct kvt<DT_F16> {
    typedef f16x8 v8;
    typedef f16x2 v2;
    typedef _Float16 s;
    static __device__ __forceinline__ f32x4 mma(v8 a, v8 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
    // 16x16x16 step on raw 4 x 16-bit operands
    static __device__ __forceinline__ f32x4 mma16(uint64_t a, uint64_t b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a),
                                                     __builtin_bit_cast(f16x4, b), c, 0, 0, 0);
    }
    static __device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
        return __builtin_amdgcn_fdot2(__builtin_bit_cast(v2, a), __builtin_bit_cast(v2, b), c, false);
    }
};
template <> struct kvt<DT_BF16> {
    typedef bf16x8 v8;
    typedef bf16x2 v2;
    typedef __bf16 s;
    static __device__ __forceinline__ f32x4 mma(v8 a, v8 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ f32x4 mma16(uint64_t a, uint64_t b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(bf16x4, a),
                                                         __builtin_bit_cast(bf16x4, b), c, 0, 0, 0);
    }
    static __device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
        return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2, a), __builtin_bit_cast(v2, b),
                                               c, false);
    }
};

template <int N> struct ic { static constexpr int value = N; };
template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (I < N) {
        f(ic<I>{});
        static_for<I + 1, N>(f);
    }
}
// f(ic<I>) for I = 0, 1, ... while it returns true, each call nested inside
// the previous one's branch: no control-flow merge between the steps, so the
// compiler's load counters stay exact along the chain.
template <int I, int N, typename F>
__device__ __forceinline__ void nested_for(F&& f) {
    if constexpr (I < N) {
        if (f(ic<I>{})) nested_for<I + 1, N>(f);
    }
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// A value the compiler may not fuse with the operations that made it or
// use it (an empty asm: no instruction is emitted).
__device__ __forceinline__ void opaque(float& v) { asm volatile("" : "+v"(v)); }

// Workgroup barrier ordering LDS only: global loads and stores still in
// flight (the tile stream, partial writes) are not waited for.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ uint32_t uni(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_readfirstlane((int)v);
}

// Even cut of T tiles over at most P runs.  The largest run holds
// k = ceil(T / P) tiles whatever the cut, so the cut uses the fewest runs
// that keep it at k, P' = ceil(T / k): every used run holds k or k - 1 tiles
// (config 2: 890 runs of 5 and one of 4, instead of 358 of 5 and 666 of 4),
// and fewer runs leave fewer partial states -- measured 2 % faster per call.
// T = q P' + r: run w < r takes q + 1 tiles, the others q; runs P' .. P - 1
// are empty (first() is clamped to T).
struct tile_split {
    uint32_t q, r, T;
    __device__ __forceinline__ uint32_t first(uint32_t w) const {
        const uint64_t f = (uint64_t)w * q + (w < r ? w : r);
        return f < T ? (uint32_t)f : T;
    }
    // run holding tile f < T
    __device__ __forceinline__ uint32_t owner(uint32_t f) const {
        const uint32_t big = r * (q + 1);
        return f < big ? f / (q + 1) : r + (f - big) / q;
    }
};
__device__ __forceinline__ tile_split make_split(uint32_t T, uint32_t P) {
    if (T == 0u || P == 0u) return tile_split{0u, 0u, 0u};
    const uint32_t k = T / P + (T % P != 0u);
    const uint32_t pe = T / k + (T % k != 0u);
    return tile_split{T / pe, T % pe, T};
}

// Tokens a decode query attends out of the n of its sequence: all of them,
// or with a window W > 0 the attention sinks [0, min(sink, n)) and the
// rolling window [lo, n), lo = max(sink, n - 1 - W) (the valid range of the
// reference's protected-sinks design, openspec/changes/archive/
// 2026-08-28-agent-runtime-optimizations/design.md:211-216).  Only tiles
// holding attended tokens are walked: tiles 0 .. st-1, then the window's
// from lo / 16 on; walked tile j is tile j < st ? j : j + gap.
struct span {
    uint32_t n, lo, sink, st, gap, tiles;
    __device__ __forceinline__ uint32_t tile(uint32_t j) const { return j < st ? j : j + gap; }
    __device__ __forceinline__ bool valid(uint32_t t) const { return t < n && (t < sink || t >= lo); }
    // some token of the tile at tok0 is not attended
    __device__ __forceinline__ bool partial(uint32_t tok0) const {
        return tok0 + TILE > n || (lo > sink && tok0 < lo && tok0 + TILE > sink);
    }
};
__device__ __forceinline__ span make_span(uint32_t n, uint32_t sink, uint32_t window) {
    const uint32_t full = n / TILE + (n % TILE != 0u);
    span sp{n, 0u, 0u, full, 0u, full};
    if (window != 0u && n != 0u) {
        const uint32_t back = n - 1u > window ? n - 1u - window : 0u;
        sp.lo = back > sink ? back : sink;
        sp.sink = sink;
        const uint32_t ns = sink < n ? sink : n;
        const uint32_t st = ns / TILE + (ns % TILE != 0u);
        const uint32_t wf = sp.lo / TILE;
        if (sp.lo >= n) {  // the sinks cover the sequence
            sp.st = st;
            sp.tiles = st;
        } else if (wf > st) {  // a gap between sink and window tiles
            sp.st = st;
            sp.gap = wf - st;
            sp.tiles = st + (full - wf);
        }
    }
    return sp;
}

// Two floats as a packed 16-bit pair (RNE), low half first.
template <int DT>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    typedef typename kvt<DT>::s S;
    typedef typename kvt<DT>::v2 V2;
    const V2 v = {(S)a, (S)b};
    return __builtin_bit_cast(uint32_t, v);
}
// The lo half of a hi + lo 16-bit split of a (a = hi + lo to ~2^-22).  An
// `a` that is a product must come through opaque(): fused with the product,
// the backend can form the hi the caller packs and the hi subtracted here
// from differently rounded products (one f16 step apart where they differ).
template <int DT>
__device__ __forceinline__ float lo_part(float a) {
    typedef typename kvt<DT>::s S;
    return a - (float)(S)a;
}

// Four E4M3 codes (one dword, lowest byte first) as four f16 (a dword pair,
// low dword first); exact: every E4M3 value is an f16.
__device__ __forceinline__ uint64_t e4m3x4_to_f16(uint32_t w) {
    const uint32_t lo = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, false));
    const uint32_t hi = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, true));
    return (uint64_t)lo | ((uint64_t)hi << 32);
}
// Eight E4M3 codes (two dwords) as one 16-byte f16 operand.
__device__ __forceinline__ u32x4 e4m3x8_to_f16(uint32_t w0, uint32_t w1) {
    const uint64_t a = e4m3x4_to_f16(w0), b = e4m3x4_to_f16(w1);
    return u32x4{(uint32_t)a, (uint32_t)(a >> 32), (uint32_t)b, (uint32_t)(b >> 32)};
}

}  // namespace

// ---------------------------------------------------------------------------
// Work item descriptors.  Every run walks a list of 16-token tiles; item k
// of a run is one uint32x4 {phys, b, tok0, info}: the physical page (~0 =
// masked), the sequence, the tile's first token and info = nvalid (tokens of
// the tile before the sequence end, 1..16) | HOLDS_LAST << 8 (the tile holds
// the sequence's last token, the appended one in a fused step) | WHOLE << 9
// (the run holds every tile of the sequence: its rows are final, no partial).
// They are built in registers from the live lengths (self-scheduled launch)
// or read from a step schedule built once per decode step
// (eh_decode_tiles_schedule) and shared by every layer.
constexpr uint32_t INFO_LAST = 1u << 8;
constexpr uint32_t INFO_WHOLE = 1u << 9;
constexpr uint32_t NO_PAGE = 0xFFFFFFFFu;

// Step schedule layout (uint32x4 records): P run headers {n_items, b_first,
// b_last, appends} (appends = 1 when the schedule was built with lens_add > 0,
// so that the tile holding a sequence's last token is the appended one); P x
// cap item descriptors (run w's at w * cap); batch sequence records {w0, w1,
// tokens, tiles} (the runs holding the sequence's first and last tile).
struct sched_view {
    const u32x4* hdr;
    const u32x4* items;
    const u32x4* seqs;
};
__device__ __forceinline__ sched_view view_of(const u32x4* s, uint32_t P, uint32_t cap) {
    return sched_view{s, s + P, s + P + (uint64_t)P * cap};
}

// ---------------------------------------------------------------------------
// Split kernel.  Grid: 1-D workgroups of SUB * n_kv waves holding SUB runs
// each (n_runs in all; the surplus runs of the last workgroup are empty);
// wave kv of a run serves kv head kv on every tile of the run.  Dynamic LDS
// (bytes): waves*16*VROW (V tiles) + waves*QSEG*G*128*4 (staged q rows) +
// 4*(2*batch + 1) (tile prefix, token counts; self-scheduled launches only).
// lens[b] + lens_add = tokens sequence b attends (lens_add = 1 when lens are
// the positions of a fused append).  Partials: slot w + b for run w and
// sequence b, part_acc [slots, n_head, 128], part_ml [slots, n_head, 2],
// slots = P + batch.
// EXT: the protected-sinks range and the per-tile attention-mass records are
// compiled in (the plain instantiation keeps the hot loop free of them).
// SCHED: the run's items come from a step schedule (sched, cap) instead of
// the lengths and block tables.
template <int DT, int G, int DEPTH, int CHUNK, bool EXT, bool SCHED>
__device__ __forceinline__ void decode_tiles(
    const float* __restrict__ q, uint8_t* pool, uint64_t n_blocks,
    const uint32_t* __restrict__ bt, uint32_t bt_stride, const uint32_t* __restrict__ lens,
    uint32_t lens_add, const uint8_t* __restrict__ new_k, const uint8_t* __restrict__ new_v,
    uint32_t batch, float* __restrict__ out, float* __restrict__ part_acc,
    float* __restrict__ part_ml, uint32_t n_head, uint32_t n_head_kv,
    uint32_t block_tokens, uint32_t bt_shift, float scale_log2, uint32_t n_runs,
    uint32_t sink, uint32_t window, float* __restrict__ tile_rec, float* __restrict__ fin,
    uint32_t rec_row, const float* __restrict__ k_scale, const float* __restrict__ v_scale,
    const u32x4* __restrict__ sched, uint32_t cap) {
    constexpr int HD = 128;
    constexpr int KSTEPS = HD / 32;  // MFMA steps over head_dim
    // E4M3 pages are converted to f16 in registers (exact) and use the f16 path
    constexpr bool F8 = DT == DT_FP8;
    constexpr int CT = F8 ? DT_F16 : DT;  // MFMA operand type
    constexpr uint32_t ELT = F8 ? 1u : 2u;
    constexpr int KREG = F8 ? 2 : KSTEPS;  // 16-byte K loads per lane and tile
    constexpr int VREG = F8 ? 2 : 4;       // 16-byte V loads per lane and tile
    typedef kvt<CT> K;
    typedef typename K::v8 V8;
    static_assert(G <= 16, "one 16-column score tile per kv head");
    static_assert(!(EXT && SCHED), "the protected-sinks range is self-scheduled");

    extern __shared__ __align__(16) uint8_t smem[];

    // A workgroup holds SUB = waves / n_kv independent runs side by side
    // (one wave per kv head each); run w = blockIdx * SUB + sub of P = n_runs.
    const uint32_t NW = blockDim.x >> 6;
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63;
    const uint32_t wave = uni(tid >> 6);
    const uint32_t kv = wave % n_head_kv;  // this wave's kv head
    const uint32_t SUB = NW / n_head_kv;
    const uint32_t group = n_head / n_head_kv;
    const uint32_t P = n_runs;
    const uint32_t w = blockIdx.x * SUB + wave / n_head_kv;  // runs past n_runs have no tiles
    const uint32_t g = lane >> 4;   // row group: tokens 4g..4g+3 of a tile
    const uint32_t x = lane & 15;   // head of the score tile / dim slice

    uint8_t* vt = smem + wave * (TILE * VROW);                      // this wave's V tile
    uint8_t* qst = smem + NW * TILE * VROW + wave * (QSEG * G * HD * 4);  // staged q rows (f32)
    uint32_t* cum = reinterpret_cast<uint32_t*>(smem + NW * (TILE * VROW + QSEG * G * HD * 4));
    uint32_t* ntok = cum + batch + 1;

    // ---- the run's items: n_items tiles, descriptors of items kb + lane in
    // dsc (current batch of 64) and dsc_next (the following one)
    uint32_t n_items, b0, b_last;
    u32x4 dsc, dsc_next = u32x4{NO_PAGE, 0u, 0u, 0u};
    tile_split ts{0u, 0u, 0u};
    uint32_t F0 = 0;
    auto make_desc = [&](uint32_t kb) -> u32x4 {  // self-scheduled: item kb + lane
        const uint32_t k = kb + lane;
        u32x4 d = {NO_PAGE, 0u, 0u, 1u};
        if (k < n_items) {
            const uint32_t f = F0 + k;
            uint32_t b = b0;
            while (cum[b + 1] <= f) ++b;
            const uint32_t j = f - cum[b];
            const uint32_t n = ntok[b];
            const uint32_t tok0 = (EXT && window ? make_span(n, sink, window).tile(j) : j) * TILE;
            const uint32_t page = tok0 >> bt_shift;
            uint32_t phys = NO_PAGE;
            if (page < bt_stride) {
                const uint32_t p = bt[(uint64_t)b * bt_stride + page];
                phys = (uint64_t)p < n_blocks ? p : NO_PAGE;
            }
            const uint32_t nv = n - tok0 < (uint32_t)TILE ? n - tok0 : (uint32_t)TILE;
            const bool whole = ts.owner(cum[b]) == ts.owner(cum[b + 1] - 1);
            d = u32x4{phys, b, tok0, nv | (tok0 + TILE >= n ? INFO_LAST : 0u) | (whole ? INFO_WHOLE : 0u)};
        }
        return d;
    };
    if constexpr (SCHED) {
        if (w >= P) return;
        const sched_view sv = view_of(sched, P, cap);
        const u32x4 h = sv.hdr[w];
        const u32x4* it = sv.items + (uint64_t)w * cap;
        dsc = lane < cap ? it[lane] : u32x4{NO_PAGE, 0u, 0u, 1u};
        // a schedule is trusted only as far as memory safety needs: counts
        // within the run's item capacity, sequences within the batch
        n_items = uni(h[0]) < cap ? uni(h[0]) : cap;
        b0 = uni(h[1]);
        b_last = uni(h[2]);
        if (n_items == 0 || b0 > b_last || b_last >= batch) return;
        // rows to append with a schedule built for no append (lens_add 0):
        // its last tiles hold existing tokens, which an append would
        // overwrite; the rows are dropped and the pool stays as it is
        if (uni(h[3]) == 0u) {
            new_k = nullptr;
            new_v = nullptr;
        }
        if (n_items > 64) dsc_next = lane + 64 < n_items ? it[lane + 64] : u32x4{NO_PAGE, 0u, 0u, 1u};
    } else {
        // tile prefix over the batch (wave 0), from the live lengths
        if (wave == 0) {
            uint32_t run = 0;
            for (uint32_t base = 0; base < batch; base += 64) {
                const uint32_t j = base + lane;
                const uint32_t n = j < batch ? lens[j] + lens_add : 0u;
                uint32_t t = make_span(n, EXT ? sink : 0u, EXT ? window : 0u).tiles;
#pragma unroll
                for (int o = 1; o < 64; o <<= 1) {
                    const uint32_t y = __shfl_up(t, o, 64);
                    if (lane >= (uint32_t)o) t += y;
                }
                if (j < batch) { cum[j + 1] = run + t; ntok[j] = n; }
                run += __shfl(t, 63, 64);
            }
            if (lane == 0) cum[0] = 0;
        }
        lds_barrier();
        // the runs' cut of the T tiles (make_split; runs past the used ones are empty)
        const uint32_t T = cum[batch];
        ts = make_split(T, P);
        F0 = w < P ? ts.first(w) : T;
        const uint32_t F1 = w < P ? ts.first(w + 1) : T;
        if (F0 >= F1) return;  // uniform over the wave: no tiles for this run (no barrier follows)
        n_items = F1 - F0;
        // sequence holding tile f (f < T)
        auto seq_of = [&](uint32_t f) -> uint32_t {
            uint32_t lo = 0, hi = batch - 1;
            while (lo < hi) {
                const uint32_t mid = (lo + hi) >> 1;
                if (cum[mid + 1] > f) hi = mid; else lo = mid + 1;
            }
            return lo;
        };
        b0 = uni(seq_of(F0));
        b_last = uni(seq_of(F1 - 1));
        dsc = make_desc(0);
        if (n_items > 64) dsc_next = make_desc(64);
    }

    const uint32_t row_bytes = n_head_kv * HD * ELT;
    const uint32_t slot_bytes = 2u * row_bytes;
    const uint64_t page_bytes = (uint64_t)block_tokens * slot_bytes;
    const uint32_t kv_off = kv * HD * ELT;
    const uint32_t slot_mask = block_tokens - 1u;

    // ---- q of this lane's head x (dims 32s + 8g .. +7: the MFMA B operand),
    // scaled into the log2 domain, split into hi + lo 16-bit halves; heads
    // past the group are zero.  The q rows of the run's first QSEG
    // sequences (this wave's heads) are fetched together up front and staged
    // in LDS, so a sequence change inside the run does not wait on global
    // memory; later sequences (runs over many short sequences) load directly.
    V8 qa[KSTEPS], qb[KSTEPS];
    const bool hv = x < group;
    // E4M3 pages: the K scale multiplies the scores after the MFMAs rather
    // than q (q * scale ~ 1e-3 would leave the lo halves a few bits above
    // f16's 2^-24 step).  With f16 operands, |q| * log2(e) / sqrt(128) must
    // stay below 65504 (|q| below ~5e5).
    const float qdown = F8 ? k_scale[kv] : 1.0f;
    auto set_q = [&](const float4* a, const float4* c) {
        typedef typename K::s S;
        const float sc = hv ? scale_log2 : 0.0f;
#pragma unroll
        for (int st = 0; st < KSTEPS; ++st) {
            const float v[8] = {a[st].x, a[st].y, a[st].z, a[st].w, c[st].x, c[st].y, c[st].z, c[st].w};
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                float vv = v[e] * sc;
                opaque(vv);  // rounded once, then split
                qa[st][e] = (S)vv;
                qb[st][e] = (S)lo_part<CT>(vv);
            }
        }
    };
    const uint32_t n_stage = b_last - b0 + 1 < (uint32_t)QSEG ? b_last - b0 + 1 : (uint32_t)QSEG;
    {
        // float4 i of the staged block: sequence i / (G*32), row (i / 32) % G
        constexpr int NQ4 = QSEG * G * (HD / 4);
        constexpr int PER = (NQ4 + 63) / 64;
        float4 v[PER];
#pragma unroll
        for (int u = 0; u < PER; ++u) {
            const uint32_t i = lane + 64 * u;
            const uint32_t sg = i / (G * (HD / 4)), h = (i / (HD / 4)) % G, d4 = i % (HD / 4);
            const bool ok = i < (uint32_t)NQ4 && sg < n_stage && h < group;
            const uint32_t bb = ok ? b0 + sg : b0, hh = ok ? h : 0u;
            v[u] = *reinterpret_cast<const float4*>(q + ((uint64_t)bb * n_head + kv * group + hh) * HD + 4 * d4);
        }
#pragma unroll
        for (int u = 0; u < PER; ++u) {
            const uint32_t i = lane + 64 * u;
            if (i < (uint32_t)NQ4) reinterpret_cast<float4*>(qst)[i] = v[u];
        }
    }
    // q of sequence b: staged (LDS) or, past the staged ones, fetched now.
    // Contraction index of MFMA step st, lane (g, x): dims 32 st + 8 g + e for
    // 16-bit pages; E4M3 lanes hold 32 contiguous dims (32 g ..) of their
    // token, so step st takes dims 32 g + 8 st + e.
    const uint32_t qg = F8 ? 32u * g : 8u * g, qs = F8 ? 8u : 32u;
    auto load_q = [&](uint32_t b) {
        float4 a[KSTEPS], c[KSTEPS];
        const float* src;
        if (b - b0 < n_stage)
            src = reinterpret_cast<const float*>(qst) + ((b - b0) * G + (hv ? x : 0u)) * HD + qg;
        else
            src = q + ((uint64_t)b * n_head + kv * group + (hv ? x : 0u)) * HD + qg;
#pragma unroll
        for (int st = 0; st < KSTEPS; ++st) {
            a[st] = *reinterpret_cast<const float4*>(src + qs * st);
            c[st] = *reinterpret_cast<const float4*>(src + qs * st + 4);
        }
        set_q(a, c);
    };

    // ---- item k of the run (its descriptor, in ring slot D while in flight)
    u32x4 kr[DEPTH][KREG], vr[DEPTH][VREG];
    uint32_t physp[DEPTH], tokp[DEPTH], infop[DEPTH], seqp[DEPTH];
    // Loads of item k into ring slot D.  Tokens past the sequence re-read
    // the tile's first token (masked); with a fused append the appended
    // token is read from new_k / new_v.
    auto issue = [&](auto Dc, uint32_t k) {
        constexpr int D = decltype(Dc)::value;
        const uint32_t li = k & 63u;
        const u32x4& src = dsc;
        const uint32_t praw = uni((uint32_t)__builtin_amdgcn_readlane((int)src[0], (int)li));
        const uint32_t braw = uni((uint32_t)__builtin_amdgcn_readlane((int)src[1], (int)li));
        const uint32_t tok0 = uni((uint32_t)__builtin_amdgcn_readlane((int)src[2], (int)li)) & ~(uint32_t)(TILE - 1);
        const uint32_t iraw = uni((uint32_t)__builtin_amdgcn_readlane((int)src[3], (int)li));
        // memory safety whatever the descriptor holds: pages inside the pool,
        // the sequence inside the run's range, at most TILE tokens at a tile
        // boundary (a well-formed descriptor passes unchanged)
        const bool pok = (uint64_t)praw < n_blocks;
        const uint32_t phys = pok ? praw : NO_PAGE;
        const uint32_t ib = braw < b0 ? b0 : braw > b_last ? b_last : braw;
        const uint32_t info = (iraw & 31u) > (uint32_t)TILE ? (iraw & ~31u) | (uint32_t)TILE : iraw;
        physp[D] = phys;
        tokp[D] = tok0;
        infop[D] = info;
        seqp[D] = ib;
        const uint8_t* base = pool + (uint64_t)(pok ? phys : 0u) * page_bytes +
                              (uint64_t)(tok0 & slot_mask) * slot_bytes + kv_off;
        const uint32_t nvalid = info & 31u;
        const bool last = new_k != nullptr && (info & INFO_LAST) != 0u;  // holds the appended token
        // K: token x of the tile; 16-bit: dims 32 st + 8 g .. (16 B per step),
        // E4M3: dims 32 g .. 32 g + 31 (two 16 B loads).  V (row layout):
        // 16-bit: tokens 4 g + r, dims 8 x ..; E4M3: tokens l / 8 + 8 j, dims
        // 16 (l % 8) ..
        auto k_at = [&](const uint8_t* row, int j) -> const u32x4* {
            return reinterpret_cast<const u32x4*>(row + (F8 ? 32 * g + 16 * j : 64 * j + 16 * g));
        };
        auto v_tok = [&](int j) -> uint32_t { return F8 ? (lane >> 3) + 8 * j : 4 * g + j; };
        const uint32_t v_off = F8 ? 16 * (lane & 7u) : 16 * x;
        if (nvalid == (uint32_t)TILE && !last) {
            static_for<0, KREG>([&](auto Sc) {
                constexpr int j = decltype(Sc)::value;
                kr[D][j] = *k_at(base + x * slot_bytes, j);
            });
            static_for<0, VREG>([&](auto Rc) {
                constexpr int j = decltype(Rc)::value;
                vr[D][j] = *reinterpret_cast<const u32x4*>(base + row_bytes + v_tok(j) * slot_bytes + v_off);
            });
        } else if constexpr (F8) {
            // partial tile; with a fused append the appended token's codes
            // replace its (not yet written) pool row in the registers
            static_for<0, KREG>([&](auto Sc) {
                constexpr int j = decltype(Sc)::value;
                kr[D][j] = *k_at(base + (x < nvalid ? x : 0u) * slot_bytes, j);
            });
            static_for<0, VREG>([&](auto Rc) {
                constexpr int j = decltype(Rc)::value;
                const uint32_t t = v_tok(j);
                vr[D][j] = *reinterpret_cast<const u32x4*>(base + row_bytes +
                                                           (t < nvalid ? t : 0u) * slot_bytes + v_off);
            });
            if (last) {  // uniform
                // The appended f32 row of this kv head, quantised by the whole
                // wave: lane l < 32 codes K dims 4l .. 4l + 3, lane 32 + l V
                // dims 4l .. 4l + 3 (x / scale, as eh_append_kv_e4m3); the
                // codes then move to the lanes of the tile layout by
                // ds_bpermute -- K: lane (g, pos) takes dims 32 g + 16 j + 4 w
                // from lane 8 g + 4 j + w; V: a lane holding token pos takes
                // dims 16 (lane % 8) + 4 w from lane 32 + 4 (lane % 8) + w.
                const uint32_t pos = nvalid - 1u;
                const bool kh = lane < 32u;
                const float* nrow = reinterpret_cast<const float*>(kh ? new_k : new_v) +
                                    (uint64_t)ib * n_head_kv * HD + kv * HD + 4u * (lane & 31u);
                const float4 nv = *reinterpret_cast<const float4*>(nrow);
                const float sc = kh ? k_scale[kv] : v_scale[kv];
                const uint32_t c4 = e4m3_code(nv.x / sc) | (e4m3_code(nv.y / sc) << 8) |
                                    (e4m3_code(nv.z / sc) << 16) | (e4m3_code(nv.w / sc) << 24);
                // Lanes of tokens past pos (masked) take the appended token's
                // codes as well: they re-read the tile's first token, which is
                // the appended one when it opens the tile, and its pool row is
                // not written yet (a zero weight on a non-finite V row would
                // not be zero).
                static_for<0, KREG>([&](auto Sc) {
                    constexpr int j = decltype(Sc)::value;
                    u32x4 c;
#pragma unroll
                    for (int w = 0; w < 4; ++w)
                        c[w] = (uint32_t)__builtin_amdgcn_ds_bpermute((int)((8u * g + 4u * j + w) * 4u), (int)c4);
                    if (x >= pos) kr[D][j] = c;
                });
                u32x4 cv;
#pragma unroll
                for (int w = 0; w < 4; ++w)
                    cv[w] = (uint32_t)__builtin_amdgcn_ds_bpermute((int)((32u + 4u * (lane & 7u) + w) * 4u), (int)c4);
                static_for<0, VREG>([&](auto Rc) {
                    constexpr int j = decltype(Rc)::value;
                    if (v_tok(j) >= pos) vr[D][j] = cv;
                });
            }
        } else {
            // appended token within the tile (when last); lanes of tokens past
            // it (masked) read the appended row too, not the tile's first
            // token, which is the appended one when it opens the tile and is
            // not in the pool yet (a zero weight on a non-finite V row would
            // not be zero)
            const uint32_t pos = nvalid - 1u;
            const uint64_t nrow = (uint64_t)ib * row_bytes + kv_off;
            {
                const bool isnew = last && x >= pos;
                const uint8_t* src = isnew ? new_k + nrow : base + (x < nvalid ? x : 0u) * slot_bytes;
                static_for<0, KREG>([&](auto Sc) {
                    constexpr int j = decltype(Sc)::value;
                    kr[D][j] = *k_at(src, j);
                });
            }
            static_for<0, VREG>([&](auto Rc) {
                constexpr int j = decltype(Rc)::value;
                const uint32_t t = v_tok(j);
                const bool isnew = last && t >= pos;
                const uint8_t* src = isnew ? new_v + nrow
                                           : base + row_bytes + (t < nvalid ? t : 0u) * slot_bytes;
                vr[D][j] = *reinterpret_cast<const u32x4*>(src + v_off);
            });
        }
    };

    // ---- per-lane state of head x (the four lanes of column x of the
    // score tile share m): m_own, l_own: running max and this lane's weight
    // sum; acc[db]: O^T rows (dims) 16 db + 4g .. +3, column (head) x.
    float m_own = NEG_BIG, l_own = 0.0f;
    f32x4 acc[HD / 16];
#pragma unroll
    for (int db = 0; db < HD / 16; ++db) acc[db] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // Write this wave's state for sequence b: the final rows when the whole
    // sequence lies in this run, else the partial for slot w + b; reset.
    // E4M3 pages: the V scale of this kv head multiplies the weighted sum
    const float vsc = F8 ? v_scale[kv] : 1.0f;
    auto flush = [&](uint32_t b, bool whole) {
        float L = l_own;
        L += __shfl_xor(L, 16, 64);
        L += __shfl_xor(L, 32, 64);
        if (hv) {
            const uint32_t qh = kv * group + x;
            if (whole) {
                const float inv = L > 0.0f ? vsc / L : 0.0f;
                if (EXT && fin != nullptr && g == 0)
                    reinterpret_cast<float2*>(fin)[(uint64_t)b * n_head + qh] = make_float2(m_own, L);
                float* dst = out + ((uint64_t)b * n_head + qh) * HD + 4 * g;
#pragma unroll
                for (int db = 0; db < HD / 16; ++db)
                    *reinterpret_cast<f32x4*>(dst + 16 * db) = acc[db] * inv;
            } else {
                const uint64_t slot = (uint64_t)(w + b) * n_head + qh;
                float* dst = part_acc + slot * HD + 4 * g;
#pragma unroll
                for (int db = 0; db < HD / 16; ++db) *reinterpret_cast<f32x4*>(dst + 16 * db) = acc[db] * vsc;
                if (g == 0) *reinterpret_cast<float2*>(part_ml + slot * 2) = make_float2(m_own, L);
            }
        }
        m_own = NEG_BIG;
        l_own = 0.0f;
#pragma unroll
        for (int db = 0; db < HD / 16; ++db) acc[db] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    };

    // transposed-read address of lane (g, r*4+b): token row 4g + r,
    // dims 4b .. 4b+3 of each 16-dim block
    const uint32_t tr_off = (4 * g + (x >> 2)) * VROW + (x & 3u) * 8;

    auto compute = [&](auto Dc) {
        constexpr int D = decltype(Dc)::value;
        const uint32_t phys = physp[D];
        if (phys == NO_PAGE) return;  // masked page: its tokens do not count (uniform)
        const uint32_t tok0 = tokp[D];
        const uint32_t info = infop[D];
        const uint32_t nvalid = info & 31u;
        const uint32_t cb = seqp[D];
        const bool win = EXT && window != 0u;
        // sinks/window: a tile that the attended range cuts (uniform)
        span sp{};
        bool cut = false;
        if constexpr (EXT) {
            if (win) {
                sp = make_span(ntok[cb], sink, window);
                cut = sp.partial(tok0);
            }
        }

        // V tile rows into LDS as f16 (16-bit lane (g, x): tokens 4g..4g+3,
        // dims 8x..8x+7; E4M3 lane l: tokens l/8 and l/8 + 8, dims 16 (l%8)..).
        // In a cut tile the rows of unattended tokens (outside the sinks and
        // the window, on a valid page) are zeroed first: their weight is 0,
        // and 0 times a non-finite row would not be.
        if constexpr (EXT) {
            if (cut) {
                if constexpr (F8) {
                    static_for<0, VREG>([&](auto Rc) {
                        constexpr int j = decltype(Rc)::value;
                        if (!sp.valid(tok0 + (lane >> 3) + 8 * j)) vr[D][j] = u32x4{0u, 0u, 0u, 0u};
                    });
                } else {
                    static_for<0, 4>([&](auto Rc) {
                        constexpr int r = decltype(Rc)::value;
                        if (!sp.valid(tok0 + 4 * g + r)) vr[D][r] = u32x4{0u, 0u, 0u, 0u};
                    });
                }
            }
        }
        if constexpr (F8) {
            static_for<0, VREG>([&](auto Rc) {
                constexpr int j = decltype(Rc)::value;
                const u32x4 h0 = e4m3x8_to_f16(vr[D][j][0], vr[D][j][1]);
                const u32x4 h1 = e4m3x8_to_f16(vr[D][j][2], vr[D][j][3]);
                uint8_t* row = vt + ((lane >> 3) + 8 * j) * VROW + 32 * (lane & 7u);
                *reinterpret_cast<u32x4*>(row) = h0;
                *reinterpret_cast<u32x4*>(row + 16) = h1;
            });
        } else {
            static_for<0, 4>([&](auto Rc) {
                constexpr int r = decltype(Rc)::value;
                *reinterpret_cast<u32x4*>(vt + (4 * g + r) * VROW + 16 * x) = vr[D][r];
            });
        }

        // S = K Q^T: lane (g, x) receives tokens 4g..4g+3 of head x
        f32x4 s = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int st = 0; st < KSTEPS; ++st) {
            V8 a;
            if constexpr (F8) {  // codes 8 st .. 8 st + 7 of the lane's 32
                a = __builtin_bit_cast(V8, e4m3x8_to_f16(kr[D][st >> 1][2 * (st & 1)],
                                                         kr[D][st >> 1][2 * (st & 1) + 1]));
            } else {
                a = __builtin_bit_cast(V8, kr[D][st]);
            }
            s = K::mma(a, qa[st], s);
            s = K::mma(a, qb[st], s);
        }
        if constexpr (F8) s *= qdown;  // the K scale
        if constexpr (EXT) {
            if (win) {  // uniform
                if (cut) {
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        s[r] = sp.valid(tok0 + 4 * g + r) ? s[r] : -__builtin_inff();
                }
            } else if (nvalid < (uint32_t)TILE) {
#pragma unroll
                for (int r = 0; r < 4; ++r) s[r] = 4 * g + r < nvalid ? s[r] : -__builtin_inff();
            }
        } else if (nvalid < (uint32_t)TILE) {  // uniform
#pragma unroll
            for (int r = 0; r < 4; ++r) s[r] = 4 * g + r < nvalid ? s[r] : -__builtin_inff();
        }
        // fused append: store the appended token's K/V slice of this kv
        // head from the registers that already hold it (E4M3: its codes;
        // K lane (g, pos): dims 32 g .. 32 g + 31, V: the lanes holding
        // token pos, dims 16 (lane % 8) ..)
        const bool app = new_k != nullptr && (info & INFO_LAST) != 0u;
        if constexpr (F8) if (app) {
            const uint32_t pos = nvalid - 1u;
            uint8_t* dst = pool + (uint64_t)phys * page_bytes +
                           (uint64_t)((tok0 & slot_mask) + pos) * slot_bytes + kv_off;
            if (x == pos) {
                static_for<0, KREG>([&](auto Sc) {
                    constexpr int j = decltype(Sc)::value;
                    *reinterpret_cast<u32x4*>(dst + 32 * g + 16 * j) = kr[D][j];
                });
            }
            static_for<0, VREG>([&](auto Rc) {
                constexpr int j = decltype(Rc)::value;
                if ((lane >> 3) + 8u * j == pos)
                    *reinterpret_cast<u32x4*>(dst + row_bytes + 16 * (lane & 7u)) = vr[D][j];
            });
        }
        if constexpr (!F8) if (app) {
            const uint32_t pos = nvalid - 1u;
            uint8_t* dst = pool + (uint64_t)phys * page_bytes +
                           (uint64_t)((tok0 & slot_mask) + pos) * slot_bytes + kv_off;
            if (x == pos) {
#pragma unroll
                for (int st = 0; st < KSTEPS; ++st)
                    *reinterpret_cast<u32x4*>(dst + 64 * st + 16 * g) = kr[D][st];
            }
            static_for<0, 4>([&](auto Rc) {
                constexpr int r = decltype(Rc)::value;
                if (4 * g + r == pos) *reinterpret_cast<u32x4*>(dst + row_bytes + 16 * x) = vr[D][r];
            });
        }
        // online softmax of head x; the running max moves (for all four row
        // groups together) only when a score exceeds it by 2^8
        const float mt = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
        if (__builtin_amdgcn_ballot_w64(mt > m_own + RESCALE)) {
            float mg = fmaxf(mt, __shfl_xor(mt, 16, 64));
            mg = fmaxf(mg, __shfl_xor(mg, 32, 64));
            const float mn = fmaxf(m_own, mg);
            const float corr = fast_exp2(m_own - mn);
            l_own *= corr;
#pragma unroll
            for (int db = 0; db < HD / 16; ++db) acc[db] *= corr;
            m_own = mn;
        }
        const float p0 = fast_exp2(s[0] - m_own), p1 = fast_exp2(s[1] - m_own);
        const float p2 = fast_exp2(s[2] - m_own), p3 = fast_exp2(s[3] - m_own);
        // P^T operand (tokens 4g..4g+3 of head x) straight from the scores
        const uint32_t ph0 = pack2<CT>(p0, p1), ph1 = pack2<CT>(p2, p3);
        const uint64_t ph = (uint64_t)ph0 | ((uint64_t)ph1 << 32);
        // the tile's weight sum: of the f16 weights the MFMAs see (f16 P),
        // of the f32 weights (bf16 P as hi + lo, ~16 bits)
        float pl;
        if constexpr (CT == DT_F16) {
            const f16x2 one2 = {(_Float16)1.0f, (_Float16)1.0f};
            pl = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, ph1), one2,
                                        __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, ph0),
                                                               one2, 0.0f, false),
                                        false);
        } else {
            pl = (p0 + p1) + (p2 + p3);
        }
        l_own += pl;
        if (EXT && tile_rec != nullptr) {  // uniform: this tile's weight sum per head, relative to m_own
            float e = pl;
            e += __shfl_xor(e, 16, 64);
            e += __shfl_xor(e, 32, 64);
            const uint32_t a = tok0 / TILE;
            if (g == 0 && hv && a < rec_row)
                reinterpret_cast<float2*>(tile_rec)[((uint64_t)cb * rec_row + a) * n_head +
                                                    kv * group + x] = make_float2(e, m_own);
        }
        uint64_t plo = 0;
        if constexpr (CT == DT_BF16)
            plo = (uint64_t)pack2<CT>(lo_part<CT>(p0), lo_part<CT>(p1)) |
                  ((uint64_t)pack2<CT>(lo_part<CT>(p2), lo_part<CT>(p3)) << 32);
        // O^T += V^T P^T per 16-dim block, V^T by transposed LDS reads
#pragma unroll
        for (int db = 0; db < HD / 16; ++db) {
            const uint64_t va = lds_read_tr(vt + tr_off + 32 * db);
            acc[db] = K::mma16(va, ph, acc[db]);
            if constexpr (DT == DT_BF16) acc[db] = K::mma16(va, plo, acc[db]);
        }
    };

    // ---- main loop: chunks of CHUNK tiles, each fully unrolled so that no
    // in-flight load crosses a loop edge (the register allocator would
    // otherwise copy the ring at the back edge, waiting for it).  Every
    // chunk issues the same load stream -- DEPTH tiles up front, one refill
    // per step while the chunk lasts; refills past the chunk's last tile
    // re-read that tile (a cache hit, never computed) -- and the steps nest,
    // so each step waits for exactly its own tile.  A chunk never straddles
    // a batch of 64 descriptors (CHUNK divides 64).
    static_assert(64 % CHUNK == 0, "chunks stay inside one descriptor batch");
    uint32_t cmp_b = b0;
    bool cmp_whole = (uni((uint32_t)__builtin_amdgcn_readlane((int)dsc[3], 0)) & INFO_WHOLE) != 0u;
    load_q(b0);
    for (uint32_t c0 = 0; c0 < n_items; c0 += CHUNK) {
        const uint32_t cn = n_items - c0 < (uint32_t)CHUNK ? n_items - c0 : (uint32_t)CHUNK;
        if (c0 != 0 && (c0 & 63u) == 0u) {  // next batch of descriptors
            dsc = dsc_next;
            if (c0 + 64 < n_items) {
                if constexpr (SCHED) {
                    const u32x4* it = view_of(sched, P, cap).items + (uint64_t)w * cap;
                    dsc_next = c0 + 64 + lane < n_items ? it[c0 + 64 + lane] : u32x4{NO_PAGE, 0u, 0u, 1u};
                } else {
                    dsc_next = make_desc(c0 + 64);
                }
            }
        }
        const uint32_t klast = c0 + cn - 1;
        static_for<0, DEPTH>([&](auto Dc) {
            const uint32_t k = c0 + decltype(Dc)::value;
            issue(Dc, k < klast ? k : klast);
        });
        nested_for<0, CHUNK>([&](auto Kc) -> bool {
            constexpr int kk = decltype(Kc)::value;
            constexpr int D = kk % DEPTH;
            if ((uint32_t)kk >= cn) return false;  // uniform
            const uint32_t k = c0 + kk;
            if (seqp[D] != cmp_b) {  // uniform: the run moves to the next sequence
                flush(cmp_b, cmp_whole);
                cmp_b = seqp[D];
                cmp_whole = (infop[D] & INFO_WHOLE) != 0u;
                load_q(cmp_b);
            }
            compute(ic<D>{});
            // the refill stays below the slot's last use, so its loads reuse
            // the slot's registers
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (kk + DEPTH < CHUNK) {
                const uint32_t kn = k + DEPTH;
                issue(ic<D>{}, kn < klast ? kn : klast);
            }
            return true;
        });
    }
    flush(cmp_b, cmp_whole);
}

// Log-sum-exp merge of the run partials of every sequence that spans more
// than one run.  Grid (ceil(n_head*128/64), batch), 256 threads: lane =
// output element, the 4 waves split the sequence's partials (each wave
// fetches up to NB of them in one memory round trip) and combine their
// results through LDS.  The runs holding the sequence (every run between
// its first and last holds tiles of it) come from the step schedule (SCHED)
// or are recomputed from the same lengths as the split kernel; writes zeros
// for empty sequences; sequences inside one run were finished by the split
// kernel.
template <bool SCHED>
__device__ __forceinline__ void merge_body(
    const float* __restrict__ part_acc, const float* __restrict__ part_ml, float* __restrict__ out,
    const uint32_t* __restrict__ lens, uint32_t lens_add, uint32_t batch, uint32_t n_head,
    uint32_t head_dim, uint32_t P, uint32_t sink, uint32_t window, float* __restrict__ fin,
    const u32x4* __restrict__ seqs) {
    constexpr int NB = 16;
    __shared__ float sM[4][64], sL[4][64], sA[4][64];
    const uint32_t b = blockIdx.y;
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wave = threadIdx.x >> 6;
    uint32_t w0, w1;
    bool empty;
    if constexpr (SCHED) {
        const u32x4 r = seqs[b];
        w0 = uni(r[0]);
        w1 = uni(r[1]);
        empty = uni(r[3]) == 0u;
        if (w0 > w1 || w1 >= P) w1 = w0;  // a span outside the runs: nothing to merge
    } else {
        uint32_t tot = 0, before = 0, mine = 0;
        for (uint32_t j = lane; j < batch; j += 64) {
            const uint32_t t = make_span(lens[j] + lens_add, sink, window).tiles;
            tot += t;
            before += j < b ? t : 0u;
            mine += j == b ? t : 0u;
        }
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) {
            tot += __shfl_xor(tot, o, 64);
            before += __shfl_xor(before, o, 64);
            mine += __shfl_xor(mine, o, 64);
        }
        empty = mine == 0;
        const tile_split ts = make_split(tot, P);
        w0 = empty ? 0u : ts.owner(before);
        w1 = empty ? 0u : ts.owner(before + mine - 1);
    }
    const uint32_t e = blockIdx.x * 64 + lane;
    const bool live = e < n_head * head_dim;
    const uint64_t orow = (uint64_t)b * n_head * head_dim + e;
    if (empty) {  // uniform
        if (wave == 0 && live) out[orow] = 0.0f;
        return;
    }
    if (w0 == w1) return;  // finished by the split kernel
    const uint32_t ec = live ? e : 0u;
    // the 64 lanes lie in one head (head_dim is a multiple of 64): the slot
    // index is wave-uniform, so (m, l) come by scalar loads and every acc
    // load is one SGPR base plus the lane's dim, all issued before any wait
    const uint32_t qh = uni(blockIdx.x * 64u / head_dim), d = ec - qh * head_dim;
    const uint32_t ns = w1 - w0 + 1;
    float M = NEG_BIG, Ls = 0.0f, A = 0.0f;
    static_assert(NB <= 64, "one (m, l) per lane");
    for (uint32_t s0 = uni(wave); s0 < ns; s0 += 4 * NB) {
        // (m, l) of the wave's NB partials by one vector load (lane i % NB
        // takes partial s0 + 4 i), read back by readlane; acc: NB loads
        const uint32_t li = lane & (NB - 1);
        const uint32_t sl = s0 + 4 * li < ns ? s0 + 4 * li : s0;
        const float2 mlv = reinterpret_cast<const float2*>(part_ml)[(uint64_t)(w0 + sl + b) * n_head + qh];
        float2 v[NB];
        float a[NB];
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            const uint32_t s = s0 + 4 * i < ns ? s0 + 4 * i : s0;
            const uint64_t slot = (uint64_t)(w0 + s + b) * n_head + qh;
            a[i] = (part_acc + slot * head_dim)[d];
        }
        __builtin_amdgcn_sched_barrier(0);  // every load of the batch is issued before any wait
#pragma unroll
        for (int i = 0; i < NB; ++i)
            v[i] = make_float2(__builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, mlv.x), i)),
                               __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, mlv.y), i)));
        float mx = M;
#pragma unroll
        for (int i = 0; i < NB; ++i)
            if (s0 + 4 * i < ns && v[i].y > 0.0f) mx = fmaxf(mx, v[i].x);
        const float c = fast_exp2(M - mx);  // 0 while nothing was folded in
        Ls *= c;
        A *= c;
        M = mx;
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            if (s0 + 4 * i >= ns || !(v[i].y > 0.0f)) continue;
            const float fw = fast_exp2(v[i].x - M);
            Ls = fmaf(v[i].y, fw, Ls);
            A = fmaf(a[i], fw, A);
        }
    }
    sM[wave][lane] = M;
    sL[wave][lane] = Ls;
    sA[wave][lane] = A;
    __syncthreads();
    if (wave != 0 || !live) return;
    float Mx = NEG_BIG;
#pragma unroll
    for (int u = 0; u < 4; ++u)
        if (sL[u][lane] > 0.0f) Mx = fmaxf(Mx, sM[u][lane]);
    float L = 0.0f, Acc = 0.0f;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        if (!(sL[u][lane] > 0.0f)) continue;
        const float fw = fast_exp2(sM[u][lane] - Mx);
        L = fmaf(sL[u][lane], fw, L);
        Acc = fmaf(sA[u][lane], fw, Acc);
    }
    out[orow] = L > 0.0f ? Acc / L : 0.0f;
    if (fin != nullptr && d == 0) reinterpret_cast<float2*>(fin)[(uint64_t)b * n_head + qh] = make_float2(Mx, L);
}


extern "C" __global__ __launch_bounds__(256) void eh_decode_tiles_merge(
    const float* __restrict__ part_acc, const float* __restrict__ part_ml, float* __restrict__ out,
    const uint32_t* __restrict__ lens, uint32_t lens_add, uint32_t batch, uint32_t n_head,
    uint32_t head_dim, uint32_t P, uint32_t sink, uint32_t window, float* __restrict__ fin) {
    merge_body<false>(part_acc, part_ml, out, lens, lens_add, batch, n_head, head_dim, P, sink,
                      window, fin, nullptr);
}

// The merge of a scheduled call: the sequence's runs are the step
// schedule's sequence records.
extern "C" __global__ __launch_bounds__(256) void eh_decode_tiles_merge_sched(
    const float* __restrict__ part_acc, const float* __restrict__ part_ml, float* __restrict__ out,
    const u32x4* __restrict__ sched, uint32_t P, uint32_t cap, uint32_t batch, uint32_t n_head,
    uint32_t head_dim) {
    merge_body<true>(part_acc, part_ml, out, nullptr, 0u, batch, n_head, head_dim, P, 0u, 0u,
                     nullptr, view_of(sched, P, cap).seqs);
}

// Step schedule of the token-balanced decode, built once per decode step
// from the live lengths and block tables and read by every layer's split and
// merge kernels (the layers of a step share one block table and one set of
// positions).  The batch's 16-token tiles -- at most the tiles the block
// table can address per sequence; tokens past the table are masked in any
// case -- are cut into P equal runs as the self-scheduled kernel cuts them,
// and every tile gets its item descriptor.  Grid-stride over
// max(P, batch, batch * bt_stride * block_tokens / 16) indices, 256 threads
// per workgroup; dynamic LDS 4 * (2 * batch + 1) bytes (each workgroup scans
// the lengths itself).
extern "C" __global__ __launch_bounds__(256) void eh_decode_tiles_schedule(
    const uint32_t* __restrict__ lens, uint32_t lens_add, const uint32_t* __restrict__ bt,
    uint32_t bt_stride, uint64_t n_blocks, uint32_t batch, uint32_t block_tokens, uint32_t bt_shift,
    uint32_t P, uint32_t cap, uint32_t n_index, u32x4* __restrict__ sched) {
    extern __shared__ __align__(16) uint32_t sm[];
    uint32_t* cum = sm;
    uint32_t* ntok = sm + batch + 1;
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t max_tiles = bt_stride * (block_tokens / TILE);
    if (threadIdx.x < 64) {
        uint32_t run = 0;
        for (uint32_t base = 0; base < batch; base += 64) {
            const uint32_t j = base + lane;
            const uint32_t n = j < batch ? lens[j] + lens_add : 0u;
            const uint32_t full = n / TILE + (n % TILE != 0u);
            uint32_t t = full < max_tiles ? full : max_tiles;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const uint32_t y = __shfl_up(t, o, 64);
                if (lane >= (uint32_t)o) t += y;
            }
            if (j < batch) { cum[j + 1] = run + t; ntok[j] = n; }
            run += __shfl(t, 63, 64);
        }
        if (lane == 0) cum[0] = 0;
    }
    __syncthreads();
    const uint32_t T = cum[batch];
    const tile_split ts = make_split(T, P);
    auto seq_of = [&](uint32_t f) -> uint32_t {  // sequence holding tile f < T
        uint32_t lo = 0, hi = batch - 1;
        while (lo < hi) {
            const uint32_t mid = (lo + hi) >> 1;
            if (cum[mid + 1] > f) hi = mid; else lo = mid + 1;
        }
        return lo;
    };
    const sched_view sv = view_of(sched, P, cap);
    u32x4* hdr = const_cast<u32x4*>(sv.hdr);
    u32x4* items = const_cast<u32x4*>(sv.items);
    u32x4* seqs = const_cast<u32x4*>(sv.seqs);
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n_index; i += gridDim.x * blockDim.x) {
        if (i < P) {  // run header
            const uint32_t f0 = ts.first(i) < T ? ts.first(i) : T;
            const uint32_t f1 = ts.first(i + 1) < T ? ts.first(i + 1) : T;
            const uint32_t n = f1 > f0 ? f1 - f0 : 0u;
            hdr[i] = u32x4{n, n ? seq_of(f0) : 0u, n ? seq_of(f1 - 1) : 0u, lens_add != 0u ? 1u : 0u};
        }
        if (i < T) {  // item descriptor of tile i
            const uint32_t b = seq_of(i);
            const uint32_t c0 = cum[b], c1 = cum[b + 1];
            const uint32_t tok0 = (i - c0) * TILE;
            const uint32_t n = ntok[b];
            const uint32_t page = tok0 >> bt_shift;
            uint32_t phys = NO_PAGE;
            if (page < bt_stride) {
                const uint32_t p = bt[(uint64_t)b * bt_stride + page];
                phys = (uint64_t)p < n_blocks ? p : NO_PAGE;
            }
            const uint32_t nv = n - tok0 < (uint32_t)TILE ? n - tok0 : (uint32_t)TILE;
            const bool whole = ts.owner(c0) == ts.owner(c1 - 1);
            const uint32_t w = ts.owner(i);
            const uint32_t k = i - ts.first(w);  // < cap: a run holds at most ceil(T / P) tiles
            items[(uint64_t)w * cap + k] =
                u32x4{phys, b, tok0, nv | (tok0 + TILE >= n ? INFO_LAST : 0u) | (whole ? INFO_WHOLE : 0u)};
        }
        if (i < batch) {  // sequence record
            const uint32_t c0 = cum[i], c1 = cum[i + 1];
            seqs[i] = c1 > c0 ? u32x4{ts.owner(c0), ts.owner(c1 - 1), ntok[i], c1 - c0}
                              : u32x4{0u, 0u, ntok[i], 0u};
        }
    }
}

// H2O attention mass of one decode call (the score StreamingKvManager::
// record_attention_mass adds per block, engine-kvcache/src/streaming.rs:
// 135-141): block_mass[page] += the softmax weights of the page's attended
// tokens summed over the q heads, from the decode kernel's per-tile records
// (weight sum e relative to the running max m) and each head's final (M, L):
// e * 2^(m - M) / L.  One thread per (sequence, block-table entry); pages
// shared by several sequences receive one atomic add from each.
extern "C" __global__ __launch_bounds__(256) void eh_decode_tiles_mass(
    const float* __restrict__ tile_rec, const float* __restrict__ fin,
    const uint32_t* __restrict__ lens, uint32_t lens_add, const uint32_t* __restrict__ bt,
    uint32_t bt_stride, uint32_t batch, uint32_t n_head, uint32_t block_tokens, uint64_t n_blocks,
    uint32_t sink, uint32_t window, uint32_t rec_row, float* __restrict__ block_mass) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (uint64_t)batch * bt_stride) return;
    const uint32_t b = (uint32_t)(i / bt_stride), p = (uint32_t)(i % bt_stride);
    const uint32_t phys = bt[i];
    if ((uint64_t)phys >= n_blocks) return;  // masked page: never attended
    const span sp = make_span(lens[b] + lens_add, sink, window);
    const uint32_t full = sp.n / TILE + (sp.n % TILE != 0u);
    const uint32_t tpp = block_tokens / TILE;
    const float2* rec = reinterpret_cast<const float2*>(tile_rec);
    const float2* fl = reinterpret_cast<const float2*>(fin) + (uint64_t)b * n_head;
    float total = 0.0f;
    for (uint32_t a = p * tpp; a < (p + 1) * tpp && a < full && a < rec_row; ++a) {
        if (!(a < sp.st || a >= sp.st + sp.gap)) continue;  // tile outside the attended range
        const float2* r = rec + ((uint64_t)b * rec_row + a) * n_head;
        for (uint32_t h = 0; h < n_head; ++h) {
            const float2 f = fl[h];
            if (f.y > 0.0f) total += r[h].x * exp2f(r[h].y - f.x) / f.y;
        }
    }
    if (total > 0.0f) atomicAdd(block_mass + phys, total);
}

// One wave per kv head; at most 8 waves per workgroup; two waves per SIMD
// (256 VGPRs, no AGPR copies, which would wait for the loads they copy).
// Tiles in flight per wave: 2 for 16-bit pages, 1 for E4M3 pages (half the
// bytes per tile).  Measured at config 2: 16-bit 1 / 2 / 3 tiles 26.0 / 25.0
// / 26.5 us per call; E4M3 1 / 2 / 3 / 4 tiles 18.1 / 19.2 / 19.8 / 20.3 us
// -- deeper queues slow the random page reads.
constexpr int tiles_depth(int dt) { return dt == DT_FP8 ? 1 : 2; }
#define EH_TILES_ONE(NAME, DT, G, EXT, SCHED)                                                       \
    extern "C" __global__ __launch_bounds__(512, 1) void NAME(                                     \
        const float* q, uint8_t* pool, uint64_t n_blocks, const uint32_t* bt, uint32_t bt_stride,  \
        const uint32_t* lens, uint32_t lens_add, const uint8_t* new_k, const uint8_t* new_v,       \
        uint32_t batch, float* out, float* part_acc, float* part_ml, uint32_t n_head,              \
        uint32_t n_head_kv, uint32_t block_tokens, uint32_t bt_shift, float scale_log2,            \
        uint32_t n_runs, uint32_t sink, uint32_t window, float* tile_rec, float* fin,              \
        uint32_t rec_row, const float* k_scale, const float* v_scale, const u32x4* sched,          \
        uint32_t cap) {                                                                            \
        decode_tiles<DT, G, tiles_depth(DT), 16, EXT, SCHED>(q, pool, n_blocks, bt, bt_stride, lens, lens_add,   \
                                               new_k, new_v, batch, out, part_acc, part_ml, n_head, \
                                               n_head_kv, block_tokens, bt_shift, scale_log2,      \
                                               n_runs, sink, window, tile_rec, fin, rec_row,       \
                                               k_scale, v_scale, sched, cap);                      \
    }
// _ext: with the protected-sinks range and attention-mass records;
// _sched: the run's items from a step schedule
#define EH_TILES(DTN, DT, G)                                                         \
    EH_TILES_ONE(eh_decode_tiles_##DTN##_hd128_g##G, DT, G, false, false)           \
    EH_TILES_ONE(eh_decode_tiles_##DTN##_hd128_g##G##_ext, DT, G, true, false)      \
    EH_TILES_ONE(eh_decode_tiles_##DTN##_hd128_g##G##_sched, DT, G, false, true)

#define EH_TILES_ALL(DTN, DT) \
    EH_TILES(DTN, DT, 1)      \
    EH_TILES(DTN, DT, 2)      \
    EH_TILES(DTN, DT, 4)      \
    EH_TILES(DTN, DT, 6)      \
    EH_TILES(DTN, DT, 8)

#if !defined(EH_ONLY_DT) || EH_ONLY_DT == 1
EH_TILES_ALL(f16, DT_F16)
#endif
#if !defined(EH_ONLY_DT) || EH_ONLY_DT == 2
EH_TILES_ALL(bf16, DT_BF16)
#endif
#if !defined(EH_ONLY_DT) || EH_ONLY_DT == 3
EH_TILES_ALL(fp8, DT_FP8)
#endif
