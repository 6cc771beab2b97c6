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
//     a wave instruction reads TPW = 64/LPT consecutive tokens' rows;
//   * q.k partial sums are reduced inside each LPT-lane group with DPP
//     butterflies (bitwise-identical result in every lane of the group);
//   * online softmax runs in the log2 domain (q pre-scaled by scale*log2 e),
//     rescaling once per U-token chunk, not once per token;
//   * split results (m, l, acc) go to a workspace; eh_decode_merge does the
//     log-sum-exp merge.  A split count of one writes the output directly.
// Sequence lengths are read on the device (pos_ptr or ctx_lens), so a grid
// sized for the capacity bound stays correct under graph replay as the
// context grows: splits past the live length exit at once.

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

constexpr int NW = 4;  // waves per workgroup
constexpr int U = 4;   // tokens per stream per iteration

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
    if constexpr (NWORDS == 4) {
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

template <int DT, int HD, int G>
__device__ __forceinline__ void decode_split(
    const float* __restrict__ q, const uint8_t* __restrict__ pool,
    const uint32_t* __restrict__ bt, uint32_t bt_stride, len_src L, float* __restrict__ out,
    float* __restrict__ part_acc, float* __restrict__ part_ml, uint32_t n_head,
    uint32_t n_head_kv, uint32_t block_tokens, int bt_shift, uint32_t tps,
    uint32_t max_splits, float scale_log2, uint64_t n_blocks) {
    constexpr int ELT = dt_info<DT>::bytes;
    constexpr int EPL = (16 / ELT) < HD ? (16 / ELT) : HD;  // elements per lane
    constexpr int LPT = HD / EPL;                            // lanes per token row
    constexpr int TPW = 64 / LPT;                            // tokens per wave instruction
    constexpr int R = NW * TPW;                              // token streams per workgroup
    constexpr int NWORDS = EPL * ELT / 4;
    static_assert(LPT >= 1 && LPT <= 64 && (64 % LPT) == 0, "head_dim/lane mapping");

    __shared__ float s_m[NW][G], s_l[NW][G];
    __shared__ float s_acc[NW][G][HD];

    const uint32_t split = blockIdx.x;
    const uint32_t group = n_head / n_head_kv;
    const uint32_t n_chunks = (group + G - 1) / G;
    const uint32_t hk = blockIdx.y / n_chunks;
    const uint32_t hc = blockIdx.y - hk * n_chunks;
    const uint32_t b = blockIdx.z;

    const uint32_t n = live_tokens(L, b);
    const uint32_t t0 = split * tps;
    if (t0 >= n) return;
    const uint32_t t1 = (n - t0 < tps) ? n : t0 + tps;
    const uint32_t nsplit = split_count(n, tps, max_splits);

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int grp = lane / LPT;
    const int sub = lane - grp * LPT;
    const int stream = wave * TPW + grp;

    const uint32_t row_bytes = n_head_kv * HD * ELT;
    const uint64_t tok_bytes = 2ull * row_bytes;
    const uint64_t page_bytes = (uint64_t)block_tokens * tok_bytes;
    const uint32_t* bt_row = bt + (uint64_t)b * bt_stride;
    const uint8_t* kbase = pool + (uint64_t)hk * HD * ELT + (uint64_t)sub * EPL * ELT;

    // Query slice for every head of this chunk, pre-scaled into the log2 domain.
    float qv[G][EPL];
    const uint32_t qh0 = hk * group + hc * G;
#pragma unroll
    for (int h = 0; h < G; ++h) {
        const bool hv = hc * G + h < group;
        const float* qp = q + ((uint64_t)b * n_head + qh0 + h) * HD + sub * EPL;
#pragma unroll
        for (int e = 0; e < EPL; ++e) qv[h][e] = hv ? qp[e] * scale_log2 : 0.0f;
    }

    float m[G], l[G], acc[G][EPL];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        m[h] = -INFINITY; l[h] = 0.0f;
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[h][e] = 0.0f;
    }

    for (uint32_t tb = t0 + stream; tb < t1; tb += R * U) {
        raw_t<NWORDS> kr[U], vr[U];
        bool ok[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t t = tb + u * R;
#pragma unroll
            for (int w = 0; w < NWORDS; ++w) { kr[u].w[w] = 0u; vr[u].w[w] = 0u; }
            ok[u] = false;
            if (t < t1) {
                const uint32_t page = bt_shift >= 0 ? (t >> bt_shift) : (t / block_tokens);
                const uint32_t slot = t - page * block_tokens;
                const uint32_t phys = page < bt_stride ? bt_row[page] : 0xFFFFFFFFu;
                if (phys < n_blocks) {
                    const uint8_t* p = kbase + (uint64_t)phys * page_bytes + (uint64_t)slot * tok_bytes;
                    kr[u] = load_raw<NWORDS>(p);
                    vr[u] = load_raw<NWORDS>(p + row_bytes);
                    ok[u] = true;
                }
            }
        }
        float s[U][G];
#pragma unroll
        for (int u = 0; u < U; ++u) {
#pragma unroll
            for (int h = 0; h < G; ++h) {
                float p = 0.0f;
#pragma unroll
                for (int e = 0; e < EPL; ++e) p = fmaf(qv[h][e], elem<DT>(kr[u], e), p);
                p = group_sum<LPT>(p);
                s[u][h] = ok[u] ? p : -INFINITY;
            }
        }
#pragma unroll
        for (int h = 0; h < G; ++h) {
            float mc = m[h];
#pragma unroll
            for (int u = 0; u < U; ++u) mc = fmaxf(mc, s[u][h]);
            if (mc == -INFINITY) continue;
            const float corr = exp2f(m[h] - mc);
            l[h] *= corr;
#pragma unroll
            for (int e = 0; e < EPL; ++e) acc[h][e] *= corr;
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const float p = exp2f(s[u][h] - mc);
                l[h] += p;
#pragma unroll
                for (int e = 0; e < EPL; ++e) acc[h][e] = fmaf(p, elem<DT>(vr[u], e), acc[h][e]);
            }
            m[h] = mc;
        }
    }

    // Merge the TPW token streams of this wave (lanes sub, sub+LPT, ...).
#pragma unroll
    for (int off = LPT; off < 64; off <<= 1) {
#pragma unroll
        for (int h = 0; h < G; ++h) {
            const float mo = __shfl_xor(m[h], off, 64);
            const float lo = __shfl_xor(l[h], off, 64);
            const float M = fmaxf(m[h], mo);
            const float fa = (M == -INFINITY) ? 0.0f : exp2f(m[h] - M);
            const float fb = (M == -INFINITY) ? 0.0f : exp2f(mo - M);
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

    // Merge the NW waves and emit: final output for a single split, else a partial.
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
            const float f = (s_m[w][h] == -INFINITY) ? 0.0f : exp2f(s_m[w][h] - M);
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

}  // namespace

// Log-sum-exp merge of split partials.  grid (n_head, batch), 64 threads.
extern "C" __global__ __launch_bounds__(64) void eh_decode_merge(
    const float* __restrict__ part_acc, const float* __restrict__ part_ml, float* __restrict__ out,
    const uint32_t* lens_ptr, uint32_t lens_mode, uint32_t seq_tokens, uint32_t query_pos,
    uint32_t causal, uint32_t n_head, uint32_t head_dim, uint32_t tps, uint32_t max_splits) {
    const len_src L{lens_ptr, lens_mode, seq_tokens, query_pos, causal};
    const uint32_t qh = blockIdx.x, b = blockIdx.y;
    const uint32_t n = live_tokens(L, b);
    const uint64_t qrow = (uint64_t)b * n_head + qh;
    if (n == 0) {
        for (uint32_t d = threadIdx.x; d < head_dim; d += 64) out[qrow * head_dim + d] = 0.0f;
        return;
    }
    const uint32_t nsplit = split_count(n, tps, max_splits);
    if (nsplit <= 1) return;  // the split kernel wrote the output
    const float* ml = part_ml + qrow * max_splits * 2;
    float M = -INFINITY;
    for (uint32_t s = 0; s < nsplit; ++s)
        if (ml[2 * s + 1] > 0.0f) M = fmaxf(M, ml[2 * s]);
    float Ls = 0.0f;
    for (uint32_t s = 0; s < nsplit; ++s)
        if (ml[2 * s + 1] > 0.0f) Ls = fmaf(ml[2 * s + 1], exp2f(ml[2 * s] - M), Ls);
    const float inv = Ls > 0.0f ? 1.0f / Ls : 0.0f;
    for (uint32_t d = threadIdx.x; d < head_dim; d += 64) {
        float A = 0.0f;
        for (uint32_t s = 0; s < nsplit; ++s)
            if (ml[2 * s + 1] > 0.0f)
                A = fmaf(part_acc[(qrow * max_splits + s) * head_dim + d], exp2f(ml[2 * s] - M), A);
        out[qrow * head_dim + d] = A * inv;
    }
}

#define EH_DECODE(DTN, DT, HD, G)                                                                \
    extern "C" __global__ __launch_bounds__(NW * 64) void eh_decode_split_##DTN##_hd##HD##_g##G( \
        const float* q, const uint8_t* pool, const uint32_t* bt, uint32_t bt_stride,            \
        const uint32_t* lens_ptr, uint32_t lens_mode, uint32_t seq_tokens, uint32_t query_pos,  \
        uint32_t causal, float* out, float* part_acc, float* part_ml, uint32_t n_head,          \
        uint32_t n_head_kv, uint32_t block_tokens, int bt_shift, uint32_t tps,                  \
        uint32_t max_splits, float scale_log2, uint64_t n_blocks) {                             \
        const len_src L{lens_ptr, lens_mode, seq_tokens, query_pos, causal};                    \
        decode_split<DT, HD, G>(q, pool, bt, bt_stride, L, out, part_acc, part_ml, n_head,      \
                                n_head_kv, block_tokens, bt_shift, tps, max_splits, scale_log2, \
                                n_blocks);                                                      \
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

EH_DECODE_HD(f32, DT_F32)
EH_DECODE_HD(f16, DT_F16)
EH_DECODE_HD(bf16, DT_BF16)
