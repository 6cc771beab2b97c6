// paged_decode.hip -- paged-attention decode for gfx950 (CDNA4, wave64).
//
// Semantics follow the reference decode attention
// (engine-cuda/kernels/paged_attention.cu:6-103, split-K form :200-369) and
// its CPU authority sdpa_decode (engine-core/src/forward_cpu.rs:424-510):
// for query head qh, kv head hk = qh / (n_head / n_head_kv); attend logical
// tokens t < n with scores q.k * 1/sqrt(head_dim); out = softmax-weighted V.
//
// Work decomposition (MI355X-first, not the reference's warp-per-q-head):
//   * one workgroup (4 waves) per (context split, kv head [x head chunk], sequence);
//   * the workgroup serves every q head of the GQA group from ONE read of each
//     K/V row, so each KV byte crosses HBM once per kv head, not once per q head;
//   * a token's head row is split over LPT lanes with EPL elements (16 B) each;
//     each wave streams TPW = 64/LPT neighbouring tokens per wave step;
//   * every lane keeps DEPTH token rows in flight in a register pipeline:
//     a slot is refilled with the row DEPTH steps ahead as soon as it has
//     been consumed; the steps of a chunk are fully unrolled so no in-flight
//     load is carried across a loop edge (a loop-carried copy of an in-flight
//     register would drain the pipeline);
//   * the split's block-table slice is staged once in LDS, so page lookups
//     never wait on global memory;
//   * q.k partial sums are reduced inside each LPT-lane group with DPP
//     butterflies (bitwise-identical result in every lane of the group);
//   * online softmax runs in the log2 domain (q pre-scaled by scale*log2 e)
//     and rescales the accumulators only when the running max moves;
//   * split results (m, l, acc) go to a workspace; eh_decode_merge combines
//     them in a second launch (a kernel boundary instead of device-scope
//     fences, which write back the whole L2 per workgroup on this part).
//     A split count of one writes the output directly.
// Sequence lengths are read on the device (pos_ptr or ctx_lens), so a grid
// sized for the capacity bound stays correct under graph replay as the
// context grows: splits past the live length exit at once.
// The file is compiled once per KV element type (EH_ONLY_DT) so the three
// code objects build in parallel.

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

constexpr int NW = 4;  // waves per workgroup

enum { DT_F32 = 0, DT_F16 = 1, DT_BF16 = 2 };

template <int DT> struct dt_info;
template <> struct dt_info<DT_F32> { static constexpr int bytes = 4; };
template <> struct dt_info<DT_F16> { static constexpr int bytes = 2; };
template <> struct dt_info<DT_BF16> { static constexpr int bytes = 2; };

typedef _Float16 half2_v __attribute__((ext_vector_type(2)));

// Raw load of NB bytes (8 or 16) as 32-bit words.
template <int NWORDS> struct raw_t { uint32_t w[NWORDS]; };

template <int NWORDS>
__device__ __forceinline__ raw_t<NWORDS> load_raw(const uint8_t* p) {
    raw_t<NWORDS> r;
    if constexpr (NWORDS > 4) {  // several 16-byte vectors
        static_assert(NWORDS % 4 == 0, "unsupported vector width");
#pragma unroll
        for (int i = 0; i < NWORDS / 4; ++i) {
            const uint4 v = *reinterpret_cast<const uint4*>(p + 16 * i);
            r.w[4 * i] = v.x; r.w[4 * i + 1] = v.y; r.w[4 * i + 2] = v.z; r.w[4 * i + 3] = v.w;
        }
    } else if constexpr (NWORDS == 4) {
        const uint4 v = *reinterpret_cast<const uint4*>(p);
        r.w[0] = v.x; r.w[1] = v.y; r.w[2] = v.z; r.w[3] = v.w;
    } else if constexpr (NWORDS == 2) {
        const uint2 v = *reinterpret_cast<const uint2*>(p);
        r.w[0] = v.x; r.w[1] = v.y;
    } else {
        static_assert(NWORDS == 1, "unsupported vector width");
        r.w[0] = *reinterpret_cast<const uint32_t*>(p);
    }
    return r;
}

// Raw store of a raw vector (the inverse of load_raw).
template <int NWORDS>
__device__ __forceinline__ void store_raw(uint8_t* p, const raw_t<NWORDS>& r) {
    if constexpr (NWORDS >= 4) {
#pragma unroll
        for (int i = 0; i < NWORDS / 4; ++i)
            *reinterpret_cast<uint4*>(p + 16 * i) =
                make_uint4(r.w[4 * i], r.w[4 * i + 1], r.w[4 * i + 2], r.w[4 * i + 3]);
    } else if constexpr (NWORDS == 2) {
        *reinterpret_cast<uint2*>(p) = make_uint2(r.w[0], r.w[1]);
    } else {
        *reinterpret_cast<uint32_t*>(p) = r.w[0];
    }
}

// Element e of a raw vector, widened to f32 (exact for every storage type).
template <int DT, int NWORDS>
__device__ __forceinline__ float elem(const raw_t<NWORDS>& r, int e) {
    if constexpr (DT == DT_F32) {
        return __uint_as_float(r.w[e]);
    } else if constexpr (DT == DT_F16) {
        const half2_v h = __builtin_bit_cast(half2_v, r.w[e >> 1]);
        return (float)((e & 1) ? h.y : h.x);
    } else {
        const uint32_t w = r.w[e >> 1];
        return __uint_as_float((e & 1) ? (w & 0xFFFF0000u) : (w << 16));
    }
}

__device__ __forceinline__ uint32_t perm(uint32_t hi_src, uint32_t lo_src, uint32_t sel) {
    return __builtin_amdgcn_perm(hi_src, lo_src, sel);
}

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Sum over aligned groups of N lanes; every lane of a group gets the same bits.
template <int N>
__device__ __forceinline__ float group_sum(float v) {
    if constexpr (N >= 2) v += dpp_f<0xB1>(v);    // quad_perm [1,0,3,2]
    if constexpr (N >= 4) v += dpp_f<0x4E>(v);    // quad_perm [2,3,0,1]
    if constexpr (N >= 8) v += dpp_f<0x141>(v);   // row_half_mirror
    if constexpr (N >= 16) v += dpp_f<0x140>(v);  // row_mirror
    if constexpr (N >= 32) v += __shfl_xor(v, 16, 64);
    if constexpr (N >= 64) v += __shfl_xor(v, 32, 64);
    return v;
}

struct len_src {
    const uint32_t* ptr;  // device lengths or position
    uint32_t mode;        // 0: host scalars, 1: *ptr is the query position, 2: ptr[b] = tokens
    uint32_t seq_tokens, query_pos, causal;
};

__device__ __forceinline__ uint32_t live_tokens(const len_src& L, uint32_t b) {
    if (L.mode == 2) return L.ptr[b];
    if (L.mode == 1) return L.ptr[0] + 1u;  // paged_attention.cu:21-24
    uint32_t n = L.seq_tokens;
    if (L.causal && L.query_pos + 1u < n) n = L.query_pos + 1u;
    return n;
}

// Splits covering n tokens, capped by the launched grid.  Callers size the
// grid so that n <= max_splits * tps; the cap only keeps a violating length
// inside the workspace.
__device__ __forceinline__ uint32_t split_count(uint32_t n, uint32_t tps, uint32_t max_splits) {
    const uint32_t s = n / tps + (n % tps != 0u);
    return s < max_splits ? s : max_splits;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// The slot kernel's f16 q is scaled by 2^q_exponent(max |q|) before its hi
// + lo split (largest element in [2^14, 2^15)), so that the lo halves are
// normal f16 values rather than subnormals holding a few bits above the
// 2^-24 step, and the scores by the inverse (exact).
__device__ __forceinline__ int q_exponent(float amax) {
    if (!(amax > 0.0f) || !(amax < __builtin_inff())) return 0;
    const int e = 15 - __builtin_amdgcn_frexp_expf(amax);
    return e < -100 ? -100 : e > 100 ? 100 : e;
}

// Block-table entries one workgroup stages in LDS: every page its split
// touches.  The host keeps tokens_per_split <= (BT_SLICE - 2) * block_tokens.
constexpr uint32_t BT_SLICE = 1024;
// Wave steps per chunk: 16, fewer for narrow heads so that a chunk stays at
// most 512 tokens.  tokens_per_split is a multiple of one round of the
// waves, NW * TPW tokens (the host derives the same value).
__host__ __device__ constexpr int chunk_steps(int tpw) {
    return (512 / (NW * tpw)) < 1 ? 1 : ((512 / (NW * tpw)) > 16 ? 16 : 512 / (NW * tpw));
}

template <int DT, int HD, int G>
__device__ __forceinline__ void decode_split(
    const float* __restrict__ q, const uint8_t* pool,  // written only by a fused append
    const uint32_t* __restrict__ bt, uint32_t bt_stride, len_src L, float* __restrict__ out,
    float* __restrict__ part_acc, float* __restrict__ part_ml, uint32_t n_head,
    uint32_t n_head_kv, uint32_t block_tokens, int bt_shift, uint32_t tps, uint32_t max_splits,
    float scale_log2, uint64_t n_blocks, const uint8_t* __restrict__ new_k,
    const uint8_t* __restrict__ new_v) {
    constexpr int ELT = dt_info<DT>::bytes;
    constexpr int EPL = (16 / ELT) < HD ? (16 / ELT) : HD;  // elements per lane
    constexpr int LPT = HD / EPL;                            // lanes per token row
    constexpr int TPW = 64 / LPT;                            // tokens per wave step
    constexpr int NWORDS = EPL * ELT / 4;
    static_assert(LPT >= 1 && LPT <= 64 && (64 % LPT) == 0, "head_dim/lane mapping");
    static_assert(EPL % 4 == 0 || EPL == HD, "query vector loads");
    constexpr int STEPS = chunk_steps(TPW);
    constexpr uint32_t CHUNK = (uint32_t)(NW * TPW * STEPS);
    constexpr int DEPTH = STEPS < 4 ? STEPS : 4;

    __shared__ uint32_t s_bt[BT_SLICE];
    __shared__ float s_m[NW][G], s_l[NW][G];
    __shared__ float s_acc[NW][G][HD];

    const uint32_t split = blockIdx.x;
    const uint32_t group = n_head / n_head_kv;
    const uint32_t n_chunks = (group + G - 1) / G;
    const uint32_t hk = blockIdx.y / n_chunks;
    const uint32_t hc = blockIdx.y - hk * n_chunks;
    const uint32_t b = blockIdx.z;
    const uint32_t qh0 = hk * group + hc * G;

    const uint32_t t0 = split * tps;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int grp = lane / LPT;
    const int sub = lane - grp * LPT;

    const uint32_t row_bytes = n_head_kv * HD * ELT;
    const uint64_t tok_bytes = 2ull * row_bytes;
    const uint64_t page_bytes = (uint64_t)block_tokens * tok_bytes;
    const uint32_t* bt_row = bt + (uint64_t)b * bt_stride;
    const uint8_t* kbase = pool + (uint64_t)hk * HD * ELT + (uint64_t)sub * EPL * ELT;

    auto page_of = [&](uint32_t t) -> uint32_t {
        return bt_shift >= 0 ? (t >> bt_shift) : (t / block_tokens);
    };

    // Stage the block-table slice of this split's whole range (invalid
    // entries -> ~0) and load the query slice before the live length is
    // known: with a device position that length is one more memory round
    // trip.  Entries past the length are staged and never read; the host's
    // bound on tokens per split keeps a whole range's slice inside BT_SLICE.
    const uint32_t pg0 = page_of(t0);
    const uint32_t t_end = t0 > 0xFFFFFFFFu - tps ? 0xFFFFFFFFu : t0 + tps;  // >= every t1
    const uint32_t npg = page_of(t_end - 1) - pg0 + 1;
    for (uint32_t i = threadIdx.x; i < npg && i < BT_SLICE; i += NW * 64) {
        const uint32_t pg = pg0 + i;
        s_bt[i] = pg < bt_stride ? bt_row[pg] : 0xFFFFFFFFu;
    }

    // Query slice of every head in this chunk, pre-scaled into the log2
    // domain.  Loads are unconditional (heads past the group re-read the last
    // valid head and are zeroed), so they issue back to back.
    float qv[G][EPL];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        const uint32_t hh = (hc * G + h < group) ? hc * G + h : group - 1;
        const float sc = (hc * G + h < group) ? scale_log2 : 0.0f;
        const float* qp = q + ((uint64_t)b * n_head + hk * group + hh) * HD + sub * EPL;
        if constexpr (EPL % 4 == 0) {
#pragma unroll
            for (int e = 0; e < EPL; e += 4) {
                const float4 v = *reinterpret_cast<const float4*>(qp + e);
                qv[h][e] = v.x * sc; qv[h][e + 1] = v.y * sc;
                qv[h][e + 2] = v.z * sc; qv[h][e + 3] = v.w * sc;
            }
        } else {
#pragma unroll
            for (int e = 0; e < EPL; ++e) qv[h][e] = qp[e] * sc;
        }
    }

    const uint32_t n = live_tokens(L, b);
    if (t0 >= n) {  // uniform over the workgroup
        // No live tokens at all: the output is zero (forward_cpu.rs:436-439).
        if (n == 0 && split == 0)
            for (int idx = threadIdx.x; idx < G * HD; idx += NW * 64)
                if (hc * G + idx / HD < group)
                    out[((uint64_t)b * n_head + qh0 + idx / HD) * HD + idx % HD] = 0.0f;
        return;
    }
    const uint32_t t1 = (n - t0 < tps) ? n : t0 + tps;
    const uint32_t nsplit = split_count(n, tps, max_splits);

    float m[G], l[G], acc[G][EPL];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        m[h] = -INFINITY; l[h] = 0.0f;
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[h][e] = 0.0f;
    }
    __syncthreads();

    // The split is walked in chunks of NW * TPW * STEPS tokens.  Inside a
    // chunk the waves take turns by TPW neighbouring tokens (one per lane
    // group): wave step k of wave w covers tokens c0 + (k NW + w) TPW ..,
    // so a split shorter than a chunk still spreads over every wave.  Each
    // wave streams its steps through a DEPTH-deep register pipeline; the
    // steps are fully unrolled, so slot indices are compile time constants
    // and no in-flight load crosses a loop back edge.
    for (uint32_t c0 = t0; c0 < t1; c0 += CHUNK) {
        const uint32_t w0 = c0 + (uint32_t)wave * TPW;  // this wave's first token
        if (w0 >= t1) continue;                         // wave-uniform: nothing left
        raw_t<NWORDS> kr[DEPTH], vr[DEPTH];
        bool ok[DEPTH];
        // Loads of wave step k into slot k % DEPTH.  Steps past the end of
        // the range re-read the wave's first row (masked), staying in bounds.
        auto issue = [&](int k) {
            const int j = k % DEPTH;
            const uint32_t t = w0 + (uint32_t)(k * NW * TPW) + grp;
            const bool valid = t < t1;
            const uint32_t tc = valid ? t : w0;
            const uint32_t pg = page_of(tc);
            const uint32_t rel = pg - pg0;
            const uint32_t phys = rel < BT_SLICE ? s_bt[rel] : 0xFFFFFFFFu;
            const bool pv = phys < n_blocks;
            const uint8_t* p = kbase + (uint64_t)(pv ? phys : 0u) * page_bytes +
                               (uint64_t)(tc - pg * block_tokens) * tok_bytes;
            // fused append: the new token's row comes from new_k / new_v
            const bool isnew = new_k != nullptr && valid && t == n - 1u;
            const uint64_t noff = ((uint64_t)hk * HD + (uint64_t)sub * EPL) * ELT;
            kr[j] = load_raw<NWORDS>(isnew ? new_k + noff : p);
            vr[j] = load_raw<NWORDS>(isnew ? new_v + noff : p + row_bytes);
            ok[j] = valid && pv;
        };
#pragma unroll
        for (int k = 0; k < DEPTH; ++k) issue(k);
#pragma unroll
        for (int k = 0; k < STEPS; ++k) {
            const int j = k % DEPTH;
            if (w0 + (uint32_t)(k * NW * TPW) >= t1) break;  // wave-uniform tail exit
            float s[G];
#pragma unroll
            for (int h = 0; h < G; ++h) {
                float p = 0.0f;
#pragma unroll
                for (int e = 0; e < EPL; ++e) p = fmaf(qv[h][e], elem<DT>(kr[j], e), p);
                s[h] = group_sum<LPT>(p);
            }
            const bool okj = ok[j];
            // A masked lane (past the range, or on an invalid page) adds
            // nothing: its V row is a stand-in (the wave's first row, page 0,
            // or an appended row not written yet), and a zero weight on a
            // non-finite row would not be zero.
            if (okj) {
#pragma unroll
                for (int h = 0; h < G; ++h) {
                    if (s[h] > m[h]) {  // rescale only when the running max moves
                        const float corr = fast_exp2(m[h] - s[h]);
                        l[h] *= corr;
#pragma unroll
                        for (int e = 0; e < EPL; ++e) acc[h][e] *= corr;
                        m[h] = s[h];
                    }
                    const float p = fast_exp2(s[h] - m[h]);
                    l[h] += p;
#pragma unroll
                    for (int e = 0; e < EPL; ++e) acc[h][e] = fmaf(p, elem<DT>(vr[j], e), acc[h][e]);
                }
            }
            if (new_k != nullptr && okj) {  // fused append: write the new row to its page
                const uint32_t t = w0 + (uint32_t)(k * NW * TPW) + grp;
                if (t == n - 1u) {
                    const uint32_t pg = page_of(t);
                    uint8_t* p = const_cast<uint8_t*>(kbase) + (uint64_t)s_bt[pg - pg0] * page_bytes +
                                 (uint64_t)(t - pg * block_tokens) * tok_bytes;
                    store_raw<NWORDS>(p, kr[j]);
                    store_raw<NWORDS>(p + row_bytes, vr[j]);
                }
            }
            if (k + DEPTH < STEPS) issue(k + DEPTH);  // refill the slot DEPTH steps ahead
        }
    }

    // Merge the TPW lane groups of this wave (lanes sub, sub+LPT, ...).
#pragma unroll
    for (int off = LPT; off < 64; off <<= 1) {
#pragma unroll
        for (int h = 0; h < G; ++h) {
            const float mo = __shfl_xor(m[h], off, 64);
            const float lo = __shfl_xor(l[h], off, 64);
            const float M = fmaxf(m[h], mo);
            const float fa = (M == -INFINITY) ? 0.0f : fast_exp2(m[h] - M);
            const float fb = (M == -INFINITY) ? 0.0f : fast_exp2(mo - M);
            l[h] = l[h] * fa + lo * fb;
#pragma unroll
            for (int e = 0; e < EPL; ++e) {
                const float ao = __shfl_xor(acc[h][e], off, 64);
                acc[h][e] = acc[h][e] * fa + ao * fb;
            }
            m[h] = M;
        }
    }
    if (grp == 0) {
#pragma unroll
        for (int h = 0; h < G; ++h) {
            if (sub == 0) { s_m[wave][h] = m[h]; s_l[wave][h] = l[h]; }
#pragma unroll
            for (int e = 0; e < EPL; ++e) s_acc[wave][h][sub * EPL + e] = acc[h][e];
        }
    }
    __syncthreads();

    // Merge the NW waves: final output for a single split, else a partial
    // that eh_decode_merge combines.
    for (int idx = threadIdx.x; idx < G * HD; idx += NW * 64) {
        const int h = idx / HD;
        const int d = idx - h * HD;
        if (hc * G + h >= group) continue;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < NW; ++w) M = fmaxf(M, s_m[w][h]);
        float Ls = 0.0f, A = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            const float f = (s_m[w][h] == -INFINITY) ? 0.0f : fast_exp2(s_m[w][h] - M);
            Ls = fmaf(s_l[w][h], f, Ls);
            A = fmaf(s_acc[w][h][d], f, A);
        }
        const uint64_t qrow = (uint64_t)b * n_head + qh0 + h;
        if (nsplit == 1) {
            out[qrow * HD + d] = Ls > 0.0f ? A / Ls : 0.0f;
        } else {
            const uint64_t slot = qrow * max_splits + split;
            part_acc[slot * HD + d] = A;
            if (d == 0) { part_ml[slot * 2] = M; part_ml[slot * 2 + 1] = Ls; }
        }
    }
}

// ---------------------------------------------------------------------------
// Slot-major split (16-bit KV, head_dim 64/128, power-of-two kv-head counts
// and pages): one workgroup per (split, head chunk, sequence) serves every kv
// head, so each wave step reads whole token slots (the K row of all heads,
// then the V row) -- contiguous pages -- rather than one head's slice.
//
// Lane layout: lane = ((tk * n_kv + hk) * HGR + hg) * 8 + sub.  Eight lanes
// cover one head row (16 dims each for head_dim 128, 8 for 64); HGR head
// groups of GH q heads each share that K/V slice (the duplicate lanes load the
// same bytes within one instruction, so HBM traffic is unchanged), which cuts
// the per-lane reduction and softmax work to GH heads.  TPI = 64 / (8 n_kv
// HGR) tokens per wave step; a step never straddles a page, so its page is
// wave-uniform and its block-table entry a scalar load.
//
// Arithmetic: q.k with packed dot2 and q split into hi + lo 16-bit parts (a
// single rounded q is too coarse for large scores; f16: q scaled by a power
// of two first, see q_exponent); f16 P.V pairs two tokens per dot2 (P
// rounded to f16, with the weight sums l taken from the same rounded
// weights, so that acc / l stays a weighted mean); bf16 P.V widens V and
// uses f32 fma.  Invalid tokens enter the softmax as -inf scores.
constexpr int SLOT_STEPS = 16;   // unrolled wave steps per chunk (even, power of two <= 64)
constexpr int SLOT_DEPTH = 4;    // wave steps in flight (even)
constexpr int SLOT_HMAX = 64;    // q heads one workgroup may serve

typedef __bf16 bf16x2_v __attribute__((ext_vector_type(2)));

// Dims of lane `sub` within a head row (8 lanes per row): 8-dim pieces at
// sub*8 and, for head_dim 128, 64 + sub*8, so that every 16-byte load
// instruction covers a contiguous run of the row across the 8 lanes.
template <int HD>
__device__ __forceinline__ uint32_t slot_dim(uint32_t sub, int e) {
    return (uint32_t)(e < 8 ? (int)sub * 8 + e : 64 + (int)sub * 8 + (e - 8));
}

template <int NWD>
__device__ __forceinline__ raw_t<NWD> load_slot_row(const uint8_t* p) {
    raw_t<NWD> r;
#pragma unroll
    for (int i = 0; i < NWD / 4; ++i) {  // 16-byte pieces 128 bytes apart
        const uint4 v = *reinterpret_cast<const uint4*>(p + 128 * i);
        r.w[4 * i] = v.x; r.w[4 * i + 1] = v.y; r.w[4 * i + 2] = v.z; r.w[4 * i + 3] = v.w;
    }
    return r;
}

template <int DT, int HD, int GH>
__device__ __forceinline__ void decode_slots(
    const float* __restrict__ q, const uint8_t* __restrict__ pool,
    const uint32_t* __restrict__ bt, uint32_t bt_stride, len_src L, float* __restrict__ out,
    float* __restrict__ part_acc, float* __restrict__ part_ml, uint32_t n_head,
    uint32_t n_head_kv, uint32_t hgr, uint32_t block_tokens, int bt_shift, uint32_t tps,
    uint32_t max_splits, float scale_log2, uint64_t n_blocks) {
    static_assert(DT == DT_F16 || DT == DT_BF16, "16-bit KV only");
    static_assert(HD == 64 || HD == 128, "head_dim 64 or 128");
    constexpr int EPL = HD / 8;       // dims per lane (8 lanes per head row)
    constexpr int NWD = EPL / 2;      // 32-bit words per lane row
    constexpr int NP = EPL / 2;       // packed pairs per lane row

    // Epilogue staging: one partial state per (wave, token lane tk, head):
    // TPI * n_wg_heads = 8 * GH per wave.
    constexpr int NPART = NW * 8 * GH;
    __shared__ float s_acc[NPART][HD];
    __shared__ float s_m[NPART], s_l[NPART], s_w[NPART];

    // grid (batch, head chunks, splits): dispatch walks split-major, so the
    // splits past the shorter contexts (empty workgroups) come last.
    const uint32_t b = blockIdx.x;
    const uint32_t hc = blockIdx.y;
    const uint32_t split = blockIdx.z;
    const uint32_t group = n_head / n_head_kv;
    const uint32_t lpt = n_head_kv * hgr * 8;  // lanes per token (power of two <= 64)
    const uint32_t tpi = 64u / lpt;            // tokens per wave step
    const int lane = threadIdx.x & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t tk = (uint32_t)lane / lpt;
    const uint32_t r = (uint32_t)lane - tk * lpt;
    const uint32_t hk = r / (hgr * 8);
    const uint32_t hg = (r >> 3) - hk * hgr;
    const uint32_t sub = r & 7u;
    const uint32_t hbase = (hc * hgr + hg) * GH;  // first head of this lane, within the group
    const uint32_t n_wg_heads = n_head_kv * hgr * GH;

    const uint32_t t0 = split * tps;
    const uint32_t row_bytes = n_head_kv * HD * 2;
    const uint32_t slot_bytes = 2u * row_bytes;
    const uint64_t page_bytes = (uint64_t)block_tokens * slot_bytes;
    const uint32_t bsh = (uint32_t)bt_shift;  // power-of-two pages here
    const uint32_t* bt_row = bt + (uint64_t)b * bt_stride;
    const uint32_t lane_off = hk * HD * 2 + sub * 16;

    const uint32_t wtoks = tpi * SLOT_STEPS;  // tokens per wave per chunk
    // Page entry of step `lane` of the chunk starting at w0 (one vector load
    // per chunk; steps read it back with readlane).  Entries past the table
    // read its last entry and are invalidated at use.
    auto load_pages = [&](uint32_t w0) -> uint32_t {
        const uint32_t pg = (w0 + (uint32_t)(lane & (SLOT_STEPS - 1)) * tpi) >> bsh;
        return bt_row[pg < bt_stride ? pg : bt_stride - 1u];
    };
    uint32_t pv_next = load_pages(t0 + wave * wtoks);

    // q of this lane's GH heads and EPL dims, pre-scaled into the log2
    // domain, as hi + lo 16-bit pairs (heads past the group are zero).
    uint32_t qa[GH][NP], qb[GH][NP];
    // f16: one exponent for the wave's q (wave-uniform); scores times qdown
    float qup = scale_log2, qdown = 1.0f;
    if constexpr (DT == DT_F16) {
        float amax = 0.0f;
#pragma unroll
        for (int h = 0; h < GH; ++h) {
            const bool hv = hbase + h < group;
            const float* qp = q + ((uint64_t)b * n_head + hk * group + (hv ? hbase + h : group - 1)) * HD;
#pragma unroll
            for (int e = 0; e < EPL; e += 4) {
                const float4 v = *reinterpret_cast<const float4*>(qp + slot_dim<HD>(sub, e));
                amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
            }
        }
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
        const int qe = q_exponent(__builtin_bit_cast(
            float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, amax))) * scale_log2);
        qup = __builtin_amdgcn_ldexpf(scale_log2, qe);
        qdown = __builtin_amdgcn_ldexpf(1.0f, -qe);
    }
#pragma unroll
    for (int h = 0; h < GH; ++h) {
        const bool hv = hbase + h < group;
        const uint32_t hh = hv ? hbase + h : group - 1;
        const float sc = hv ? qup : 0.0f;
        const float* qp = q + ((uint64_t)b * n_head + hk * group + hh) * HD;
#pragma unroll
        for (int e = 0; e < EPL; e += 4) {
            const float4 v = *reinterpret_cast<const float4*>(qp + slot_dim<HD>(sub, e));
            // each product rounded once, then split (opaque: fused with the
            // product, hi and lo could come from differently rounded values)
            float x[4] = {v.x * sc, v.y * sc, v.z * sc, v.w * sc};
#pragma unroll
            for (int i = 0; i < 4; ++i) asm volatile("" : "+v"(x[i]));
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                if constexpr (DT == DT_F16) {
                    const _Float16 a0 = (_Float16)x[2 * u], a1 = (_Float16)x[2 * u + 1];
                    const half2_v hi = {a0, a1};
                    const half2_v lo = {(_Float16)(x[2 * u] - (float)a0),
                                        (_Float16)(x[2 * u + 1] - (float)a1)};
                    qa[h][e / 2 + u] = __builtin_bit_cast(uint32_t, hi);
                    qb[h][e / 2 + u] = __builtin_bit_cast(uint32_t, lo);
                } else {
                    const __bf16 a0 = (__bf16)x[2 * u], a1 = (__bf16)x[2 * u + 1];
                    const bf16x2_v hi = {a0, a1};
                    const bf16x2_v lo = {(__bf16)(x[2 * u] - (float)a0),
                                         (__bf16)(x[2 * u + 1] - (float)a1)};
                    qa[h][e / 2 + u] = __builtin_bit_cast(uint32_t, hi);
                    qb[h][e / 2 + u] = __builtin_bit_cast(uint32_t, lo);
                }
            }
        }
    }

    const uint32_t n = live_tokens(L, b);
    if (t0 >= n) {
        if (n == 0 && split == 0)
            for (uint32_t idx = threadIdx.x; idx < n_wg_heads * HD; idx += NW * 64) {
                const uint32_t hh = idx / HD;
                const uint32_t kv = hh / (hgr * GH), w = hh - kv * hgr * GH;
                const uint32_t hin = hc * hgr * GH + w;
                if (hin < group) out[((uint64_t)b * n_head + kv * group + hin) * HD + idx % HD] = 0.0f;
            }
        return;
    }
    const uint32_t t1 = (n - t0 < tps) ? n : t0 + tps;
    const uint32_t nsplit = split_count(n, tps, max_splits);

    float m[GH], l[GH], acc[GH][EPL];
#pragma unroll
    for (int h = 0; h < GH; ++h) {
        m[h] = -1e30f; l[h] = 0.0f;
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[h][e] = 0.0f;
    }

    // q.k of one step for every head of the lane, reduced over the 8 lanes
    // of the head row; invalid tokens score -inf.
    auto scores = [&](const raw_t<NWD>& kr, bool ok, float* s) {
#pragma unroll
        for (int h = 0; h < GH; ++h) {
            float d = 0.0f;
#pragma unroll
            for (int u = 0; u < NP; ++u) {
                if constexpr (DT == DT_F16) {
                    const half2_v kk = __builtin_bit_cast(half2_v, kr.w[u]);
                    d = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_v, qa[h][u]), kk, d, false);
                    d = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_v, qb[h][u]), kk, d, false);
                } else {
                    const bf16x2_v kk = __builtin_bit_cast(bf16x2_v, kr.w[u]);
                    d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_v, qa[h][u]), kk, d, false);
                    d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_v, qb[h][u]), kk, d, false);
                }
            }
            d = group_sum<8>(d);
            s[h] = ok ? d * qdown : -INFINITY;
        }
    };
    // Lazy rescale: the running maximum only moves when a score exceeds it by
    // more than 2^8 (wave-uniform branch); otherwise every weight uses the
    // stale maximum, exactly.
    auto rescale_if = [&](const float* s0, const float* s1) {
        bool need = false;
#pragma unroll
        for (int h = 0; h < GH; ++h) need |= fmaxf(s0[h], s1[h]) > m[h] + 8.0f;
        if (__builtin_amdgcn_ballot_w64(need)) {
#pragma unroll
            for (int h = 0; h < GH; ++h) {
                const float mn = fmaxf(m[h], fmaxf(s0[h], s1[h]));
                const float corr = fast_exp2(m[h] - mn);
                l[h] *= corr;
#pragma unroll
                for (int e = 0; e < EPL; ++e) acc[h][e] *= corr;
                m[h] = mn;
            }
        }
    };

    for (uint32_t c0 = t0; c0 < t1; c0 += NW * wtoks) {
        const uint32_t w0 = c0 + wave * wtoks;
        const uint32_t w1 = (w0 + wtoks < t1) ? w0 + wtoks : t1;
        if (w0 >= w1) continue;  // wave-uniform
        const uint32_t pv_cur = pv_next;
        if (c0 + NW * wtoks < t1) pv_next = load_pages(w0 + NW * wtoks);  // next chunk, early
        raw_t<NWD> kr[SLOT_DEPTH], vr[SLOT_DEPTH];
        bool ok[SLOT_DEPTH];
        auto issue = [&](int k) {
            const int j = k % SLOT_DEPTH;
            const uint32_t ts = w0 + (uint32_t)k * tpi;  // first token of the step (uniform)
            const uint32_t tsc = ts < w1 ? ts : w0;
            const uint32_t phys = ((ts >> bsh) < bt_stride)
                                      ? (uint32_t)__builtin_amdgcn_readlane((int)pv_cur, k)
                                      : 0xFFFFFFFFu;
            const bool pv = phys < n_blocks;
            const uint32_t t = ts + tk;
            const bool valid = t < w1;
            const uint32_t tc = valid ? t : tsc;
            const uint8_t* p = pool + (uint64_t)(pv ? phys : 0u) * page_bytes +
                               (uint64_t)((tc & ((1u << bsh) - 1u)) * slot_bytes + lane_off);
            kr[j] = load_slot_row<NWD>(p);
            vr[j] = load_slot_row<NWD>(p + row_bytes);
            ok[j] = valid && pv;
        };
#pragma unroll
        for (int k = 0; k < SLOT_DEPTH; ++k) issue(k);
#pragma unroll
        for (int k = 0; k < SLOT_STEPS; k += 2) {  // steps in pairs: P.V packs two tokens
            const int j0 = k % SLOT_DEPTH, j1 = (k + 1) % SLOT_DEPTH;
            float s0[GH], s1[GH];
            scores(kr[j0], ok[j0], s0);
            scores(kr[j1], ok[j1], s1);
            rescale_if(s0, s1);
            // masked tokens (invalid pages read page 0) carry zero V words:
            // their weights are 0, and 0 times a non-finite word would not be
#pragma unroll
            for (int w = 0; w < NWD; ++w) {
                vr[j0].w[w] = ok[j0] ? vr[j0].w[w] : 0u;
                vr[j1].w[w] = ok[j1] ? vr[j1].w[w] : 0u;
            }
            if constexpr (DT == DT_F16) {
                uint32_t vp[EPL];  // (token k, token k+1) pairs per dim
#pragma unroll
                for (int w = 0; w < NWD; ++w) {
                    vp[2 * w] = perm(vr[j1].w[w], vr[j0].w[w], 0x05040100u);
                    vp[2 * w + 1] = perm(vr[j1].w[w], vr[j0].w[w], 0x07060302u);
                }
#pragma unroll
                for (int h = 0; h < GH; ++h) {
                    const float p0 = fast_exp2(s0[h] - m[h]), p1 = fast_exp2(s1[h] - m[h]);
                    const half2_v pp = {(_Float16)p0, (_Float16)p1};
                    l[h] = __builtin_amdgcn_fdot2(pp, half2_v{(_Float16)1.0f, (_Float16)1.0f},
                                                  l[h], false);
#pragma unroll
                    for (int e = 0; e < EPL; ++e)
                        acc[h][e] = __builtin_amdgcn_fdot2(pp, __builtin_bit_cast(half2_v, vp[e]),
                                                           acc[h][e], false);
                }
            } else {
                float v0[EPL], v1[EPL];
#pragma unroll
                for (int e = 0; e < EPL; ++e) {
                    v0[e] = elem<DT>(vr[j0], e);
                    v1[e] = elem<DT>(vr[j1], e);
                }
#pragma unroll
                for (int h = 0; h < GH; ++h) {
                    const float p0 = fast_exp2(s0[h] - m[h]), p1 = fast_exp2(s1[h] - m[h]);
                    l[h] += p0 + p1;
#pragma unroll
                    for (int e = 0; e < EPL; ++e) acc[h][e] = fmaf(p1, v1[e], fmaf(p0, v0[e], acc[h][e]));
                }
            }
            if (k + SLOT_DEPTH < SLOT_STEPS) issue(k + SLOT_DEPTH);
            if (k + 1 + SLOT_DEPTH < SLOT_STEPS) issue(k + 1 + SLOT_DEPTH);
        }
    }

    // Epilogue.  Every lane group (wave, tk) holds a partial softmax state
    // for its heads; stage them all in LDS, compute one weight per partial,
    // then combine per output element -- no shuffles, no atomics.
    // Partial index: (wave * TPI + tk) * n_wg_heads + hh, hh = (hk*HGR+hg)*GH + h.
    const uint32_t hh0 = (hk * hgr + hg) * GH;
    const uint32_t pbase = (wave * tpi + tk) * n_wg_heads;
#pragma unroll
    for (int h = 0; h < GH; ++h) {
        float* dst = s_acc[pbase + hh0 + h];
#pragma unroll
        for (int e = 0; e < EPL; e += 4)
            *reinterpret_cast<float4*>(dst + slot_dim<HD>(sub, e)) =
                make_float4(acc[h][e], acc[h][e + 1], acc[h][e + 2], acc[h][e + 3]);
        if (sub == 0) { s_m[pbase + hh0 + h] = m[h]; s_l[pbase + hh0 + h] = l[h]; }
    }
    __syncthreads();
    const uint32_t nparts = NW * tpi;  // partials per head
    for (uint32_t i = threadIdx.x; i < nparts * n_wg_heads; i += NW * 64) {
        const uint32_t hh = i % n_wg_heads;
        float M = -1e30f;
        for (uint32_t pp = 0; pp < nparts; ++pp) M = fmaxf(M, s_m[pp * n_wg_heads + hh]);
        s_w[i] = fast_exp2(s_m[i] - M);
    }
    __syncthreads();
    for (uint32_t idx = threadIdx.x; idx < n_wg_heads * HD; idx += NW * 64) {
        const uint32_t hh = idx / HD, d = idx - hh * HD;
        const uint32_t kv = hh / (hgr * GH), w = hh - kv * hgr * GH;
        const uint32_t hin = hc * hgr * GH + w;  // head index within the kv group
        if (hin >= group) continue;
        float M = -1e30f, Ls = 0.0f, A = 0.0f;
        for (uint32_t pp = 0; pp < nparts; ++pp) {
            const uint32_t i = pp * n_wg_heads + hh;
            M = fmaxf(M, s_m[i]);
            Ls = fmaf(s_l[i], s_w[i], Ls);
            A = fmaf(s_acc[i][d], s_w[i], A);
        }
        const uint64_t qrow = (uint64_t)b * n_head + kv * group + hin;
        if (nsplit == 1) {
            out[qrow * HD + d] = Ls > 0.0f ? A / Ls : 0.0f;
        } else {
            const uint64_t slot = qrow * max_splits + split;
            part_acc[slot * HD + d] = A;
            if (d == 0) { part_ml[slot * 2] = M; part_ml[slot * 2 + 1] = Ls; }
        }
    }
}

}  // namespace

// Log-sum-exp merge of split partials: out = sum_s w_s acc_s / sum_s w_s l_s
// with w_s = exp2(m_s - max m), splits with l_s == 0 skipped.  One thread
// per output element (grid (ceil(n_head * head_dim / 256), batch), 256
// threads); the partials of up to 32 splits are fetched together before they
// are folded in (an online max keeps one pass), so a context of S splits
// costs ceil(S / 32) memory round trips, the first beside the length read.
extern "C" __global__ __launch_bounds__(256) void eh_decode_merge(
    const float* __restrict__ part_acc, const float* __restrict__ part_ml, float* __restrict__ out,
    const uint32_t* lens_ptr, uint32_t lens_mode, uint32_t seq_tokens, uint32_t query_pos,
    uint32_t causal, uint32_t n_head, uint32_t head_dim, uint32_t tps, uint32_t max_splits) {
    const len_src L{lens_ptr, lens_mode, seq_tokens, query_pos, causal};
    const uint32_t b = blockIdx.y;
    const uint32_t e = blockIdx.x * 256 + threadIdx.x;
    if (e >= n_head * head_dim) return;
    const uint32_t qh = e / head_dim, d = e - qh * head_dim;
    const uint64_t qrow = (uint64_t)b * n_head + qh;
    const float2* ml = reinterpret_cast<const float2*>(part_ml) + qrow * max_splits;
    const float* pa = part_acc + qrow * max_splits * head_dim + d;
    // Partials in batches of NB: every load of a batch is in flight at once
    // (one memory round trip for up to NB splits).  The first batch goes out
    // before the live length is known (a device position is one more round
    // trip): slots past the length lie inside the row's max_splits slots and
    // are not folded.
    constexpr int NB = 32;
    float2 v[NB];
    float x[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        const uint32_t sidx = (uint32_t)i < max_splits ? (uint32_t)i : 0u;
        v[i] = ml[sidx];
        x[i] = pa[(uint64_t)sidx * head_dim];
    }
    const uint32_t n = live_tokens(L, b);
    const uint32_t nsplit = split_count(n, tps, max_splits);
    if (n == 0 || nsplit <= 1) return;  // the split kernel wrote the output
    float M = -INFINITY, Ls = 0.0f, A = 0.0f;
    for (uint32_t s0 = 0; s0 < nsplit; s0 += NB) {
        if (s0 > 0) {
#pragma unroll
            for (int i = 0; i < NB; ++i) {
                const uint32_t sidx = s0 + i < nsplit ? s0 + i : s0;
                v[i] = ml[sidx];
                x[i] = pa[(uint64_t)sidx * head_dim];
            }
        }
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            if (s0 + i >= nsplit || !(v[i].y > 0.0f)) continue;
            if (v[i].x > M) {
                const float c = fast_exp2(M - v[i].x);  // 0 on the first live split
                Ls *= c;
                A *= c;
                M = v[i].x;
            }
            const float w = fast_exp2(v[i].x - M);
            Ls = fmaf(v[i].y, w, Ls);
            A = fmaf(x[i], w, A);
        }
    }
    out[qrow * head_dim + d] = Ls > 0.0f ? A / Ls : 0.0f;
}

#define EH_DECODE(DTN, DT, HD, G)                                                                \
    extern "C" __global__ __launch_bounds__(NW * 64) void eh_decode_split_##DTN##_hd##HD##_g##G( \
        const float* q, const uint8_t* pool, const uint32_t* bt, uint32_t bt_stride,            \
        const uint32_t* lens_ptr, uint32_t lens_mode, uint32_t seq_tokens, uint32_t query_pos,  \
        uint32_t causal, float* out, float* part_acc, float* part_ml, uint32_t n_head,          \
        uint32_t n_head_kv, uint32_t block_tokens, int bt_shift, uint32_t tps,                  \
        uint32_t max_splits, float scale_log2, uint64_t n_blocks, const uint8_t* new_k,         \
        const uint8_t* new_v) {                                                                 \
        const len_src L{lens_ptr, lens_mode, seq_tokens, query_pos, causal};                    \
        decode_split<DT, HD, G>(q, pool, bt, bt_stride, L, out, part_acc, part_ml, n_head,      \
                                n_head_kv, block_tokens, bt_shift, tps, max_splits, scale_log2, \
                                n_blocks, new_k, new_v);                                        \
    }

#define EH_DECODE_G(DTN, DT, HD) \
    EH_DECODE(DTN, DT, HD, 1)    \
    EH_DECODE(DTN, DT, HD, 2)    \
    EH_DECODE(DTN, DT, HD, 4)    \
    EH_DECODE(DTN, DT, HD, 6)    \
    EH_DECODE(DTN, DT, HD, 7)    \
    EH_DECODE(DTN, DT, HD, 8)

#define EH_DECODE_HD(DTN, DT) \
    EH_DECODE_G(DTN, DT, 4)   \
    EH_DECODE_G(DTN, DT, 8)   \
    EH_DECODE_G(DTN, DT, 16)  \
    EH_DECODE_G(DTN, DT, 32)  \
    EH_DECODE_G(DTN, DT, 64)  \
    EH_DECODE_G(DTN, DT, 128) \
    EH_DECODE_G(DTN, DT, 256)

#define EH_SLOTS(DTN, DT, HD, GH)                                                               \
    extern "C" __global__ __launch_bounds__(NW * 64, 2) void eh_decode_slots_##DTN##_hd##HD##_h##GH( \
        const float* q, const uint8_t* pool, const uint32_t* bt, uint32_t bt_stride,              \
        const uint32_t* lens_ptr, uint32_t lens_mode, uint32_t seq_tokens, uint32_t query_pos,    \
        uint32_t causal, float* out, float* part_acc, float* part_ml, uint32_t n_head,            \
        uint32_t n_head_kv, uint32_t hgr, uint32_t block_tokens, int bt_shift, uint32_t tps,      \
        uint32_t max_splits, float scale_log2, uint64_t n_blocks) {                               \
        const len_src L{lens_ptr, lens_mode, seq_tokens, query_pos, causal};                      \
        decode_slots<DT, HD, GH>(q, pool, bt, bt_stride, L, out, part_acc, part_ml, n_head,       \
                                 n_head_kv, hgr, block_tokens, bt_shift, tps, max_splits,         \
                                 scale_log2, n_blocks);                                           \
    }

#define EH_SLOTS_ALL(DTN, DT) \
    EH_SLOTS(DTN, DT, 64, 1)  \
    EH_SLOTS(DTN, DT, 64, 2)  \
    EH_SLOTS(DTN, DT, 64, 3)  \
    EH_SLOTS(DTN, DT, 64, 4)  \
    EH_SLOTS(DTN, DT, 128, 1) \
    EH_SLOTS(DTN, DT, 128, 2) \
    EH_SLOTS(DTN, DT, 128, 3) \
    EH_SLOTS(DTN, DT, 128, 4)

#if !defined(EH_ONLY_DT) || EH_ONLY_DT == 0
EH_DECODE_HD(f32, DT_F32)
#endif
#if !defined(EH_ONLY_DT) || EH_ONLY_DT == 1
EH_DECODE_HD(f16, DT_F16)
EH_SLOTS_ALL(f16, DT_F16)
#endif
#if !defined(EH_ONLY_DT) || EH_ONLY_DT == 2
EH_DECODE_HD(bf16, DT_BF16)
EH_SLOTS_ALL(bf16, DT_BF16)
#endif
