// engine_hip.cpp -- C-ABI launcher for the gfx950 paged KV-cache kernels.
//
// Replaces engine-cuda's NVRTC compile + cuModuleLoadData + cuLaunchKernel
// (engine-cuda/src/paged_kv.rs:122-196, paged_attention.rs:58-134) with
// hipModuleLoad of offline code objects and hipModuleLaunchKernel.  Sizes
// are validated the way the reference validates DeviceBuffer sizes before
// anything is launched; launches never allocate and never synchronise.

#include "../../include/engine_hip.h"

#include <hip/hip_runtime.h>

#include <dlfcn.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>

struct eh_context {
    int device = 0;
    hipModule_t mod_kv = nullptr;
    hipModule_t mod_decode[3] = {nullptr, nullptr, nullptr};  // f32, f16, bf16
    hipModule_t mod_prefill = nullptr;
    hipModule_t mod_tiles[3] = {nullptr, nullptr, nullptr};  // token-balanced decode: f16, bf16, e4m3
    std::mutex mu;
    std::unordered_map<std::string, hipFunction_t> fns;
    // Split-K scratch for eh_flash_decoding, allocated once at creation
    // (the reference does the same at paged_attention.rs:111-123).
    float* scratch = nullptr;
    uint64_t scratch_floats = 0;
    // This device's copy of the library's static scratch array (noalloc.hip),
    // looked up once at creation: the workspace of
    // eh_append_decode_batched_noalloc.
    void* noalloc = nullptr;
    uint64_t noalloc_bytes = 0;
};

// noalloc.hip
extern "C" int eh_noalloc_scratch_setup(void** ptr, uint64_t* bytes);

namespace {

struct err_state {
    uint64_t expected = 0, actual = 0;
    const char* site = "";
    int hip = 0;
};
thread_local err_state g_err;

eh_status fail(eh_status s, const char* site, uint64_t expected = 0, uint64_t actual = 0,
               int hip = 0) {
    g_err.expected = expected;
    g_err.actual = actual;
    g_err.site = site;
    g_err.hip = hip;
    return s;
}

eh_status invalid_size(uint64_t expected, uint64_t actual, const char* site = "InvalidSize") {
    return fail(EH_INVALID_SIZE, site, expected, actual);
}

// Scratch capacity of the single-sequence decode: 64 q heads x 256 splits x
// 256 dims of partials.
constexpr uint64_t kScratchFloats = 64ull * 256 * (256 + 2);
// Splits one merge workgroup combines (LDS-resident weights).
constexpr uint64_t kMaxSplits = 256;
// Block-table entries a decode workgroup stages in LDS.
constexpr uint64_t kBtSlice = 1024;
// Decode workgroup: 4 waves.
constexpr uint32_t kDecodeThreads = 256;

eh_status bind(eh_context* c) {
    int cur = -1;
    if (hipGetDevice(&cur) != hipSuccess || cur != c->device) {
        hipError_t e = hipSetDevice(c->device);
        if (e != hipSuccess) return fail(EH_DRIVER, "hipSetDevice", 0, 0, (int)e);
    }
    return EH_OK;
}

eh_status get_fn(eh_context* c, hipModule_t mod, const char* name, hipFunction_t* f) {
    std::lock_guard<std::mutex> lk(c->mu);
    auto it = c->fns.find(name);
    if (it != c->fns.end()) { *f = it->second; return EH_OK; }
    hipFunction_t fn = nullptr;
    hipError_t e = hipModuleGetFunction(&fn, mod, name);
    if (e != hipSuccess || !fn) return fail(EH_KERNEL_LOAD, "hipModuleGetFunction", 0, 0, (int)e);
    c->fns.emplace(name, fn);
    *f = fn;
    return EH_OK;
}

template <typename... A>
eh_status launch_lds(eh_context* c, hipModule_t mod, const char* name, dim3 grid, dim3 block,
                     uint32_t lds_bytes, eh_stream stream, A... a) {
    hipFunction_t f = nullptr;
    eh_status st = get_fn(c, mod, name, &f);
    if (st != EH_OK) return st;
    void* argv[] = {static_cast<void*>(&a)...};
    hipError_t e = hipModuleLaunchKernel(f, grid.x, grid.y, grid.z, block.x, block.y, block.z,
                                         lds_bytes, (hipStream_t)stream, argv, nullptr);
    if (e != hipSuccess) return fail(EH_KERNEL_LAUNCH, "hipModuleLaunchKernel", 0, 0, (int)e);
    return EH_OK;
}

template <typename... A>
eh_status launch(eh_context* c, hipModule_t mod, const char* name, dim3 grid, dim3 block,
                 eh_stream stream, A... a) {
    return launch_lds(c, mod, name, grid, block, 0, stream, a...);
}

uint64_t elt_bytes(uint32_t dt) {
    switch (dt) {
        case EH_KV_F32: return 4;
        case EH_KV_F16: return 2;
        case EH_KV_BF16: return 2;
        case EH_KV_FP8: return 1;
        default: return 0;
    }
}

uint64_t div_ceil(uint64_t a, uint64_t b) { return a / b + (a % b != 0); }

// Byte counts of the argument checks saturate at UINT64_MAX: a size beyond 64
// bits fits no real buffer, so its check fails instead of passing on a wrapped
// value, and no page size wraps to 0 before a division.
uint64_t smul(uint64_t a, uint64_t b) {
    uint64_t r;
    return __builtin_mul_overflow(a, b, &r) ? UINT64_MAX : r;
}
template <class... T>
uint64_t smul(uint64_t a, uint64_t b, uint64_t c, T... rest) {
    return smul(smul(a, b), c, rest...);
}
uint64_t sadd(uint64_t a, uint64_t b) {
    uint64_t r;
    return __builtin_add_overflow(a, b, &r) ? UINT64_MAX : r;
}

// Largest copy chunk (16/8/4/2 bytes) dividing the row size and every base.
int pick_chunk(uint64_t row_bytes, std::initializer_list<const void*> ptrs) {
    for (int ch : {16, 8, 4, 2}) {
        bool ok = row_bytes % ch == 0;
        for (const void* p : ptrs) ok = ok && ((uintptr_t)p % ch == 0);
        if (ok) return ch;
    }
    return 0;
}

uint32_t grid_for(uint64_t work, uint32_t per_block, uint32_t cap = 16384) {
    uint64_t g = div_ceil(work, per_block);
    if (g < 1) g = 1;
    return (uint32_t)(g > cap ? cap : g);
}

const char* dt_name(uint32_t dt) {
    switch (dt) {
        case EH_KV_F32: return "f32";
        case EH_KV_F16: return "f16";
        case EH_KV_BF16: return "bf16";
        default: return nullptr;
    }
}

// Compiled decode head sizes.
bool supported_hd(uint32_t kv_dtype, uint64_t hd) {
    (void)kv_dtype;
    return hd == 4 || hd == 8 || hd == 16 || hd == 32 || hd == 64 || hd == 128 || hd == 256;
}

// Smallest compiled head-group width covering min(group, 8).
uint32_t pick_g(uint32_t group) {
    const uint32_t want = group < 8 ? group : 8;
    for (uint32_t g : {1u, 2u, 4u, 6u, 7u, 8u})
        if (g >= want) return g;
    return 8;
}

int log2_exact(uint64_t v) {
    if (v == 0 || (v & (v - 1))) return -1;
    int s = 0;
    while ((1ull << s) < v) ++s;
    return s;
}

int dt_index(uint32_t dt) {
    switch (dt) {
        case EH_KV_F32: return 0;
        case EH_KV_F16: return 1;
        case EH_KV_BF16: return 2;
        default: return -1;
    }
}

// Workspace of the split-K decode: partial accumulators then (m, l) pairs.
uint64_t decode_ws_floats(uint64_t rows, uint64_t max_splits, uint64_t head_dim) {
    return max_splits <= 1 ? 0 : smul(rows, max_splits, sadd(head_dim, 2));
}

// Largest split that keeps a workgroup's block-table slice inside LDS.
uint64_t max_tps(uint64_t block_tokens, uint64_t chunk = 1) {
    return std::max<uint64_t>((kBtSlice - 2) * block_tokens / chunk, 1) * chunk;
}

// Split granularity of the fixed-split kernel: one round of its 4 waves, TPW
// tokens each (mirrors the kernel: 16-byte lane vectors, a head row over
// head_dim / (16 / elt) lanes).  The waves take turns by TPW tokens, so any
// multiple of a round keeps every wave busy.
uint64_t chunk_tokens(uint32_t kv_dtype, uint64_t head_dim) {
    const uint64_t elt = elt_bytes(kv_dtype) ? elt_bytes(kv_dtype) : 4;
    const uint64_t epl = std::min<uint64_t>(16 / elt, head_dim);
    const uint64_t tpw = 64 / std::max<uint64_t>(head_dim / epl, 1);
    const uint64_t nw = kDecodeThreads / 64;
    return nw * tpw;
}

// Which split kernel serves a decode shape, and its work granularity.
//   slot-major (eh_decode_slots_*): 16-bit KV, head_dim 64/128, power-of-two
//     pages and at most 8 kv heads (a power of two); one workgroup serves
//     every kv head, lanes split a group's q heads into head groups of gh;
//   head-major (eh_decode_split_*): everything else; one workgroup per kv head.
struct decode_kernel {
    bool slots = false;
    uint32_t gh = 1, hgr = 1, tpi = 1;  // slot-major: heads per lane, head groups, tokens per step
    uint32_t g = 1;                     // head-major: compiled head-group width
    uint32_t chunks = 1;                // workgroups per (split, sequence) along the heads
    uint64_t chunk = 1;                 // tokens one workgroup walks per unrolled chunk
    uint64_t units = 1;                 // workgroups per (split, sequence)
};

constexpr uint32_t kSlotSteps = 16;  // mirrors SLOT_STEPS in paged_decode.hip

decode_kernel pick_decode_kernel(uint32_t kv_dtype, uint64_t head_dim, uint64_t n_head,
                                 uint64_t n_head_kv, uint64_t block_tokens, bool no_slots = false) {
    decode_kernel k;
    const uint32_t group = (uint32_t)(n_head / n_head_kv);
    const bool pow2_kv = n_head_kv && !(n_head_kv & (n_head_kv - 1));
    const bool pow2_bt = block_tokens && !(block_tokens & (block_tokens - 1));
    if (!no_slots && (kv_dtype == EH_KV_F16 || kv_dtype == EH_KV_BF16) &&
        (head_dim == 64 || head_dim == 128) && pow2_kv && pow2_bt && n_head_kv <= 8 && group >= 1) {
        const uint32_t gh = group % 4 == 0 ? 4 : group % 3 == 0 ? 3 : group <= 4 ? group : 4;
        const uint32_t need = (group + gh - 1) / gh;  // head groups per kv head
        uint32_t hgr = 1;
        while (hgr < need && n_head_kv * hgr * 2 <= 8) hgr *= 2;
        const uint32_t tpi = (uint32_t)(64 / (n_head_kv * hgr * 8));
        if (block_tokens % tpi == 0) {
            k.slots = true;
            k.gh = gh;
            k.hgr = hgr;
            k.tpi = tpi;
            k.chunks = (need + hgr - 1) / hgr;
            k.chunk = (uint64_t)(kDecodeThreads / 64) * kSlotSteps * tpi;
            k.units = k.chunks;
            return k;
        }
    }
    k.g = pick_g(group);
    k.chunks = (group + k.g - 1) / k.g;
    k.chunk = chunk_tokens(kv_dtype, head_dim);
    k.units = n_head_kv * k.chunks;
    return k;
}

struct decode_args {
    uint32_t kv_dtype;
    const float* q;
    const void* pool;
    uint64_t n_blocks;
    const uint32_t* bt;
    uint32_t bt_stride;
    const uint32_t* lens_ptr;
    uint32_t lens_mode, seq_tokens, query_pos, causal;
    uint32_t batch;
    float* out;
    uint32_t n_head, n_head_kv, head_dim, block_tokens;
    uint32_t tps, max_splits;
    float* part_acc;
    float* part_ml;
    // fused append (split kernel only): the row written at the last live
    // position, [row_len] of the pool type
    const void* new_k = nullptr;
    const void* new_v = nullptr;
};

eh_status run_decode(eh_context* c, eh_stream stream, const decode_args& a) {
    const char* dn = dt_name(a.kv_dtype);
    if (!dn) return fail(EH_UNSUPPORTED, "kv_dtype");
    if (!supported_hd(a.kv_dtype, a.head_dim)) return fail(EH_UNSUPPORTED, "head_dim", 256, a.head_dim);
    if (a.max_splits > kMaxSplits) return invalid_size(kMaxSplits, a.max_splits, "max_splits");
    const decode_kernel dk =
        pick_decode_kernel(a.kv_dtype, a.head_dim, a.n_head, a.n_head_kv, a.block_tokens,
                           a.new_k != nullptr);
    char name[64];
    if (dk.slots)
        std::snprintf(name, sizeof name, "eh_decode_slots_%s_hd%u_h%u", dn, a.head_dim, dk.gh);
    else
        std::snprintf(name, sizeof name, "eh_decode_split_%s_hd%u_g%u", dn, a.head_dim, dk.g);
    if (a.tps % dk.chunk) return invalid_size(dk.chunk, a.tps, "tokens_per_split % chunk");
    const float scale = 1.0f / std::sqrt((float)a.head_dim);  // paged_attention.rs:286
    const float scale_log2 = scale * 1.4426950408889634f;
    const int bt_shift = log2_exact(a.block_tokens);
    if (a.tps > max_tps(a.block_tokens, dk.chunk))
        return invalid_size(max_tps(a.block_tokens, dk.chunk), a.tps, "tokens_per_split");
    const hipModule_t mod = c->mod_decode[dt_index(a.kv_dtype)];
    eh_status st;
    if (dk.slots)
        st = launch(c, mod, name, dim3(a.batch, dk.chunks, a.max_splits), dim3(kDecodeThreads),
                    stream, a.q, (const uint8_t*)a.pool, a.bt, a.bt_stride, a.lens_ptr, a.lens_mode,
                    a.seq_tokens, a.query_pos, a.causal, a.out, a.part_acc, a.part_ml, a.n_head,
                    a.n_head_kv, dk.hgr, a.block_tokens, bt_shift, a.tps, a.max_splits, scale_log2,
                    a.n_blocks);
    else
        st = launch(c, mod, name, dim3(a.max_splits, a.n_head_kv * dk.chunks, a.batch),
                    dim3(kDecodeThreads), stream, a.q, (const uint8_t*)a.pool, a.bt, a.bt_stride,
                    a.lens_ptr, a.lens_mode, a.seq_tokens, a.query_pos, a.causal, a.out,
                    a.part_acc, a.part_ml, a.n_head, a.n_head_kv, a.block_tokens, bt_shift, a.tps,
                    a.max_splits, scale_log2, a.n_blocks, (const uint8_t*)a.new_k,
                    (const uint8_t*)a.new_v);
    if (st != EH_OK || a.max_splits <= 1) return st;
    return launch(c, mod, "eh_decode_merge",
                  dim3((uint32_t)div_ceil((uint64_t)a.n_head * a.head_dim, 256), a.batch), dim3(256),
                  stream,
                  (const float*)a.part_acc, (const float*)a.part_ml, a.out, a.lens_ptr, a.lens_mode,
                  a.seq_tokens, a.query_pos, a.causal, a.n_head, a.head_dim, a.tps, a.max_splits);
}

// ---- token-balanced decode (eh_decode_tiles_*, paged_decode_tiles.hip)
// Serves 16-bit KV with head_dim 128, 1/2/4/8 kv heads, at most 8 q heads per
// kv head and power-of-two pages of at least 16 tokens.  A workgroup is one
// wave per kv head; the grid fills every CU at two waves per SIMD; the device
// cuts the batch's tiles evenly among the workgroups from the live lengths.
constexpr uint32_t kTilesMaxBatch = 2048;  // lengths + tile prefix staged in LDS
constexpr uint32_t kTilesQSeg = 2;         // mirrors QSEG in paged_decode_tiles.hip
constexpr uint32_t kTilesVRow = 288;       // mirrors VROW in paged_decode_tiles.hip

struct tiles_cfg {
    bool ok = false;
    uint32_t g = 0, nw = 1;  // compiled head-group width, waves (= kv heads) per workgroup
};

tiles_cfg pick_tiles(uint32_t kv_dtype, uint64_t head_dim, uint64_t n_head, uint64_t n_head_kv,
                     uint64_t block_tokens, uint64_t batch) {
    tiles_cfg t;
    if (kv_dtype != EH_KV_F16 && kv_dtype != EH_KV_BF16 && kv_dtype != EH_KV_FP8) return t;
    if (head_dim != 128 || n_head_kv == 0 || n_head % n_head_kv) return t;
    if (!(n_head_kv == 1 || n_head_kv == 2 || n_head_kv == 4 || n_head_kv == 8)) return t;
    const uint64_t group = n_head / n_head_kv;
    if (group < 1 || group > 8) return t;
    if (block_tokens < 16 || (block_tokens & (block_tokens - 1))) return t;
    if (batch > kTilesMaxBatch) return t;
    for (uint32_t g : {1u, 2u, 4u, 6u, 8u})
        if (g >= group) { t.g = g; break; }
    t.nw = (uint32_t)n_head_kv;
    t.ok = true;
    return t;
}

uint32_t device_cus() {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
        return (uint32_t)n;
    return 256;  // MI355X
}

// one 8-wave workgroup per CU (two waves per SIMD) holding 8 / n_kv runs;
// the plan's grid counts runs
uint32_t tiles_grid(const tiles_cfg& t) { return device_cus() * (8u / t.nw); }

uint64_t tiles_ws_bytes(uint64_t grid, uint64_t batch, uint64_t n_head) {
    return smul(4, sadd(grid, batch), n_head, 128 + 2);
}

// Attention-mass scratch: one (weight sum, max) pair per (sequence, 16-token
// tile the block table can address, q head), then the heads' final (M, L).
uint64_t mass_rec_row(uint64_t bt_stride, uint64_t block_tokens) { return smul(bt_stride, block_tokens / 16); }
uint64_t mass_ws_bytes(uint64_t batch, uint64_t bt_stride, uint64_t block_tokens, uint64_t n_head) {
    return smul(8, batch, n_head, sadd(mass_rec_row(bt_stride, block_tokens), 1));
}

// Step schedule (eh_decode_schedule): P run headers, P * cap item
// descriptors and batch sequence records, 16 bytes each; cap = the most
// tiles one run can hold, from the tiles the block tables can address.
uint64_t sched_tile_bound(uint64_t batch, uint64_t bt_stride, uint64_t block_tokens) {
    return smul(batch, bt_stride, block_tokens / 16);
}
uint64_t sched_cap(uint64_t batch, uint64_t bt_stride, uint64_t block_tokens, uint64_t grid) {
    return std::max<uint64_t>(div_ceil(sched_tile_bound(batch, bt_stride, block_tokens), grid), 1);
}
uint64_t sched_bytes(uint64_t batch, uint64_t bt_stride, uint64_t block_tokens, uint64_t grid) {
    return smul(16, sadd(sadd(grid, smul(grid, sched_cap(batch, bt_stride, block_tokens, grid))), batch));
}

struct tiles_args {
    uint32_t kv_dtype;
    const float* q;
    void* pool;
    uint64_t n_blocks;
    const uint32_t* bt;
    uint32_t bt_stride;
    const uint32_t* lens;
    uint32_t lens_add;
    const void* new_k;
    const void* new_v;
    uint32_t batch;
    float* out;
    uint32_t n_head, n_head_kv, block_tokens, grid;
    void* ws;
    const float* k_scale;  // E4M3 pages only
    const float* v_scale;
    uint32_t sink, window;  // protected-sinks range; window 0 attends every token
    float* block_mass;      // optional H2O scores [n_blocks]: += attention mass per page
    void* mass_ws;          // tile records + final (M, L), mass_ws_bytes
    const void* sched;      // step schedule (eh_decode_schedule) or null: self-scheduled
    uint32_t cap;           // items per run in the schedule
};

eh_status run_tiles(eh_context* c, eh_stream stream, const tiles_args& a, const tiles_cfg& t) {
    // partial states are written and read as 16-byte vectors
    if (!a.ws || (uintptr_t)a.ws % 16)
        return fail(EH_INVALID_ARGS, "workspace is null or not 16-byte aligned");
    char name[64];
    const bool f8 = a.kv_dtype == EH_KV_FP8;
    const bool ext = a.window != 0 || a.block_mass != nullptr;  // sinks/window or mass records
    std::snprintf(name, sizeof name, "eh_decode_tiles_%s_hd128_g%u%s", f8 ? "fp8" : dt_name(a.kv_dtype),
                  t.g, ext ? "_ext" : a.sched ? "_sched" : "");
    const hipModule_t mod = c->mod_tiles[f8 ? 2 : a.kv_dtype == EH_KV_F16 ? 0 : 1];
    const float scale_log2 = (1.0f / std::sqrt(128.0f)) * 1.4426950408889634f;  // paged_attention.rs:286
    // per-wave V tiles (16 rows x kTilesVRow bytes) and staged q rows
    // (kTilesQSeg sequences x g heads x 128 f32), the tile prefix and token
    // counts of the batch
    const uint32_t runs_per_wg = 8u / t.nw;
    const uint32_t waves = 8u;
    const uint32_t lds = waves * (16 * kTilesVRow + kTilesQSeg * t.g * 128 * 4) + 4u * (2 * a.batch + 1);
    float* part_acc = (float*)a.ws;
    float* part_ml = part_acc + (uint64_t)(a.grid + a.batch) * a.n_head * 128;
    const uint32_t rec_row = (uint32_t)mass_rec_row(a.bt_stride, a.block_tokens);
    float* tile_rec = a.block_mass ? (float*)a.mass_ws : nullptr;
    float* fin = a.block_mass ? tile_rec + 2ull * a.batch * rec_row * a.n_head : nullptr;
    eh_status st = launch_lds(c, mod, name, dim3((uint32_t)div_ceil(a.grid, runs_per_wg)),
                              dim3(waves * 64), lds, stream, a.q,
                              (uint8_t*)a.pool, a.n_blocks, a.bt, a.bt_stride, a.lens, a.lens_add,
                              (const uint8_t*)a.new_k, (const uint8_t*)a.new_v, a.batch, a.out,
                              part_acc, part_ml, a.n_head, a.n_head_kv, a.block_tokens,
                              (uint32_t)log2_exact(a.block_tokens), scale_log2, a.grid, a.sink,
                              a.window, tile_rec, fin, rec_row, a.k_scale, a.v_scale, a.sched,
                              a.cap);
    if (st != EH_OK) return st;
    const dim3 mgrid((uint32_t)div_ceil((uint64_t)a.n_head * 128, 64), a.batch);
    if (a.sched)
        return launch(c, mod, "eh_decode_tiles_merge_sched", mgrid, dim3(256), stream,
                      (const float*)part_acc, (const float*)part_ml, a.out, a.sched, a.grid, a.cap,
                      a.batch, a.n_head, 128u);
    st = launch(c, mod, "eh_decode_tiles_merge", mgrid, dim3(256), stream,
                  (const float*)part_acc, (const float*)part_ml, a.out, a.lens, a.lens_add, a.batch,
                  a.n_head, 128u, a.grid, a.sink, a.window, fin);
    if (st != EH_OK || !a.block_mass) return st;
    const uint64_t threads = (uint64_t)a.batch * a.bt_stride;
    return launch(c, mod, "eh_decode_tiles_mass", dim3((uint32_t)div_ceil(threads, 256)), dim3(256),
                  stream, (const float*)tile_rec, (const float*)fin, a.lens, a.lens_add, a.bt,
                  a.bt_stride, a.batch, a.n_head, a.block_tokens, a.n_blocks, a.sink, a.window,
                  rec_row, a.block_mass);
}

// Splits: aim for enough workgroups to fill 256 CUs several times over, with
// at most kMaxSplits splits and a block-table slice that fits LDS.
uint64_t auto_tps(uint64_t batch, uint64_t units, uint64_t max_ctx, uint64_t block_tokens,
                  uint64_t chunk, uint64_t target_wgs = 1024) {
    uint64_t tps = div_ceil(batch * units * (max_ctx ? max_ctx : 1), target_wgs);
    tps = std::max<uint64_t>((tps + chunk / 2) / chunk, 1) * chunk;  // nearest chunk multiple
    while (div_ceil(max_ctx ? max_ctx : 1, tps) > kMaxSplits) tps += chunk;
    return std::min(tps, max_tps(block_tokens, chunk));
}

// Checks shared by the single-sequence attention entry points
// (paged_attention.rs:193-257), in the reference's order.
eh_status validate_attention(uint32_t kv_dtype, uint64_t q_bytes, uint64_t pool_bytes,
                             uint64_t bt_bytes, uint64_t out_bytes, uint64_t n_head,
                             uint64_t n_head_kv, uint64_t head_dim, uint64_t block_tokens,
                             uint64_t seq_tokens, uint64_t query_pos) {
    if (n_head < 1) return invalid_size(1, n_head);
    if (n_head_kv < 1) return invalid_size(1, n_head_kv);
    if (n_head % n_head_kv != 0) return invalid_size(n_head_kv, n_head % n_head_kv);
    if (head_dim < 1) return invalid_size(1, head_dim);
    if (block_tokens < 1) return invalid_size(1, block_tokens);
    if (seq_tokens < 1) return invalid_size(1, seq_tokens);
    const uint64_t q_expected = smul(n_head, head_dim, 4);
    if (q_bytes < q_expected) return invalid_size(q_expected, q_bytes);
    if (out_bytes < q_expected) return invalid_size(q_expected, out_bytes);
    if (pool_bytes < 4) return invalid_size(4, pool_bytes);
    const uint64_t bt_expected = smul(div_ceil(seq_tokens, block_tokens), 4);
    if (bt_bytes < bt_expected) return invalid_size(bt_expected, bt_bytes);
    const uint64_t imax = 0x7FFFFFFFull;
    for (uint64_t v : {n_head, n_head_kv, head_dim, block_tokens, seq_tokens, query_pos})
        if (v > imax) return invalid_size(imax, v);
    if (!dt_name(kv_dtype)) return fail(EH_UNSUPPORTED, "kv_dtype");
    if (!supported_hd(kv_dtype, head_dim)) return fail(EH_UNSUPPORTED, "head_dim", 256, head_dim);
    return EH_OK;
}

// Compiled prefill head sizes (MFMA tiles need multiples of 32).
bool prefill_hd(uint64_t hd) { return hd == 64 || hd == 128; }

struct prefill_args {
    uint32_t kv_dtype;
    const float* q;
    const void* pool;
    uint64_t n_blocks;
    const uint32_t* bt;
    uint32_t bt_stride, bt_entries;
    const uint32_t* cu_q;
    const uint32_t* start_pos;
    const uint32_t* pos_ptr;
    uint32_t q_tokens, pos_offset, batch, max_q;
    float* out;
    uint32_t n_head, n_head_kv, head_dim, block_tokens;
    const float* k_scale;  // E4M3 pages only
    const float* v_scale;
};

constexpr uint32_t kPrefillRows = 256;  // query rows per workgroup (8 waves x 32), mirrors ROWS
// One launch: grid (256-row tiles, kv heads, sequences) of 512 threads.
// bf16 pages with whole staging items per page take the ping-pong kernels
// (eh_prefill_pp_*: the workgroup's two halves alternate their MFMA and
// softmax phases), measured 7-8 % faster than the single-phase kernels at
// config 3; f16 and E4M3 pages ran 3 % slower on them and keep the
// single-phase kernels, as do f32 pages and other page sizes.  Both compute
// the same products in the same order per accumulator, so their outputs are
// bit-identical.  EH_PREFILL_KERNEL in the environment overrides the choice
// for the 16-bit and E4M3 types: "single" or "pp" (a diagnostic).
bool prefill_pingpong(const prefill_args& a) {
    if (a.kv_dtype == EH_KV_F32) return false;
    const uint32_t item_keys = a.head_dim == 128 ? 4u : 2u;  // pp_item_keys<HD>() in the kernel
    if (a.block_tokens % item_keys != 0) return false;
    const char* env = std::getenv("EH_PREFILL_KERNEL");
    if (env && std::strcmp(env, "single") == 0) return false;
    if (env && std::strcmp(env, "pp") == 0) return true;
    return a.kv_dtype == EH_KV_BF16;
}

eh_status run_prefill(eh_context* c, eh_stream stream, const prefill_args& a) {
    char name[48];
    std::snprintf(name, sizeof name, "eh_prefill_%s%s_hd%u", prefill_pingpong(a) ? "pp_" : "",
                  a.kv_dtype == EH_KV_FP8 ? "fp8" : dt_name(a.kv_dtype), a.head_dim);
    const uint32_t group = a.n_head / a.n_head_kv;
    const uint64_t tiles = div_ceil((uint64_t)a.max_q * group, kPrefillRows);
    if (tiles > 0x7FFFFFFFull) return invalid_size(0x7FFFFFFFull, tiles, "row tiles");
    const float scale = 1.0f / std::sqrt((float)a.head_dim);  // flash_attention.rs:166
    const float scale_log2 = scale * 1.4426950408889634f;
    const uint32_t row_bytes = a.n_head_kv * a.head_dim * (uint32_t)elt_bytes(a.kv_dtype);
    return launch(c, c->mod_prefill, name, dim3((uint32_t)tiles, a.n_head_kv, a.batch),
                  dim3(2 * kPrefillRows), stream, a.q, (const uint8_t*)a.pool, a.bt, a.bt_stride,
                  a.bt_entries, a.cu_q, a.start_pos, a.pos_ptr, a.q_tokens, a.pos_offset, a.out,
                  a.n_head, a.n_head_kv, a.block_tokens, log2_exact(a.block_tokens), row_bytes,
                  scale_log2, a.n_blocks, a.k_scale, a.v_scale);
}

// Shape checks shared by the prefill entry points (beyond the reference's
// size checks, which come first): the kernel set and a pool of >= 1 page.
eh_status validate_prefill_shape(uint32_t kv_dtype, uint64_t n_head, uint64_t n_head_kv,
                                 uint64_t head_dim, uint64_t block_tokens, uint64_t pool_bytes,
                                 bool e4m3 = false) {
    if (e4m3 ? kv_dtype != EH_KV_FP8 : !dt_name(kv_dtype)) return fail(EH_UNSUPPORTED, "kv_dtype");
    if (!prefill_hd(head_dim)) return fail(EH_UNSUPPORTED, "head_dim", 128, head_dim);
    const uint64_t page_bytes = smul(block_tokens, 2, n_head_kv, head_dim, elt_bytes(kv_dtype));
    if (pool_bytes < page_bytes) return invalid_size(page_bytes, pool_bytes);
    const uint64_t imax = 0x7FFFFFFFull;
    for (uint64_t v : {n_head, n_head_kv, block_tokens})
        if (v > imax) return invalid_size(imax, v);
    return EH_OK;
}

// Shape checks of every call that takes a pool layout, ahead of its own: the
// kernels take the page and row sizes as 32-bit values, and the checks divide
// by block_tokens.
eh_status check_layout(const eh_kv_layout* l) {
    const uint64_t imax = 0x7FFFFFFFull;
    if (l->block_tokens < 1) return invalid_size(1, 0, "block_tokens");
    if (l->block_tokens > imax) return invalid_size(imax, l->block_tokens, "block_tokens");
    if (l->row_len < 1) return invalid_size(1, 0, "row_len");
    const uint64_t row_bytes = smul(l->row_len, std::max<uint64_t>(elt_bytes(l->data_type), 1));
    if (row_bytes > imax) return invalid_size(imax, row_bytes, "row bytes");
    return EH_OK;
}

}  // namespace

extern "C" {

const char* eh_status_name(eh_status s) {
    switch (s) {
        case EH_OK: return "Ok";
        case EH_INVALID_SIZE: return "InvalidSize";
        case EH_KERNEL_LOAD: return "KernelLoad";
        case EH_KERNEL_LAUNCH: return "KernelLaunch";
        case EH_ALLOC_FAILED: return "AllocFailed";
        case EH_STREAM_FAILED: return "StreamFailed";
        case EH_MEMCPY_FAILED: return "MemcpyFailed";
        case EH_EVENT_FAILED: return "EventFailed";
        case EH_GRAPH_FAILED: return "GraphFailed";
        case EH_DRIVER: return "Driver";
        case EH_POOL_EXHAUSTED: return "PoolExhausted";
        case EH_INVALID_ARGS: return "InvalidArgs";
        case EH_UNSUPPORTED: return "Unsupported";
    }
    return "Unknown";
}

eh_status eh_last_error(uint64_t* expected, uint64_t* actual, const char** site, int* hip_code) {
    if (expected) *expected = g_err.expected;
    if (actual) *actual = g_err.actual;
    if (site) *site = g_err.site;
    if (hip_code) *hip_code = g_err.hip;
    return EH_OK;
}

uint64_t eh_kv_element_bytes(uint32_t data_type) { return elt_bytes(data_type); }

uint64_t eh_kv_layout_bytes_total(const eh_kv_layout* l) {
    return smul(l->n_blocks, l->block_tokens, 2, l->row_len, elt_bytes(l->data_type));
}

eh_status eh_create(int device, const char* code_object_dir, eh_context** out) {
    if (!out) return fail(EH_INVALID_ARGS, "out is null");
    *out = nullptr;
    std::string dir;
    if (code_object_dir && *code_object_dir) {
        dir = code_object_dir;
    } else {
        Dl_info info;
        if (dladdr((void*)&eh_create, &info) && info.dli_fname) {
            dir = info.dli_fname;
            size_t slash = dir.rfind('/');
            dir = slash == std::string::npos ? "." : dir.substr(0, slash);
        } else {
            dir = ".";
        }
    }
    eh_context* c = new eh_context();
    c->device = device;
    hipError_t e = hipSetDevice(device);
    if (e != hipSuccess) { delete c; return fail(EH_DRIVER, "hipSetDevice", 0, 0, (int)e); }
    const std::string kv = dir + "/paged_kv.hsaco";
    e = hipModuleLoad(&c->mod_kv, kv.c_str());
    if (e != hipSuccess) { delete c; return fail(EH_KERNEL_LOAD, "hipModuleLoad(paged_kv)", 0, 0, (int)e); }
    const char* dec_names[3] = {"/paged_decode_f32.hsaco", "/paged_decode_f16.hsaco",
                                "/paged_decode_bf16.hsaco"};
    for (int i = 0; i < 3; ++i) {
        const std::string path = dir + dec_names[i];
        e = hipModuleLoad(&c->mod_decode[i], path.c_str());
        if (e != hipSuccess) {
            eh_destroy(c);
            return fail(EH_KERNEL_LOAD, "hipModuleLoad(paged_decode)", 0, 0, (int)e);
        }
    }
    const std::string pf = dir + "/paged_prefill.hsaco";
    e = hipModuleLoad(&c->mod_prefill, pf.c_str());
    if (e != hipSuccess) {
        eh_destroy(c);
        return fail(EH_KERNEL_LOAD, "hipModuleLoad(paged_prefill)", 0, 0, (int)e);
    }
    const char* tile_names[3] = {"/paged_decode_tiles_f16.hsaco", "/paged_decode_tiles_bf16.hsaco",
                                 "/paged_decode_tiles_fp8.hsaco"};
    for (int i = 0; i < 3; ++i) {
        const std::string path = dir + tile_names[i];
        e = hipModuleLoad(&c->mod_tiles[i], path.c_str());
        if (e != hipSuccess) {
            eh_destroy(c);
            return fail(EH_KERNEL_LOAD, "hipModuleLoad(paged_decode_tiles)", 0, 0, (int)e);
        }
    }
    e = hipMalloc((void**)&c->scratch, kScratchFloats * sizeof(float));
    if (e != hipSuccess) {
        eh_destroy(c);
        return fail(EH_ALLOC_FAILED, "hipMalloc(split-K scratch)", 0, 0, (int)e);
    }
    c->scratch_floats = kScratchFloats;
    // device address of the static scratch array on this device (the device
    // is current here)
    const int se = eh_noalloc_scratch_setup(&c->noalloc, &c->noalloc_bytes);
    if (se != 0) {
        eh_destroy(c);
        return fail(EH_KERNEL_LOAD, "hipGetSymbolAddress(scratch)", 0, 0, se);
    }
    *out = c;
    return EH_OK;
}

void eh_destroy(eh_context* c) {
    if (!c) return;
    hipSetDevice(c->device);
    if (c->scratch) hipFree(c->scratch);
    if (c->mod_kv) hipModuleUnload(c->mod_kv);
    for (hipModule_t m : c->mod_decode)
        if (m) hipModuleUnload(m);
    if (c->mod_prefill) hipModuleUnload(c->mod_prefill);
    for (hipModule_t m : c->mod_tiles)
        if (m) hipModuleUnload(m);
    delete c;
}

eh_status eh_append_kv(eh_context* c, eh_stream stream, const eh_kv_layout* l, void* pool,
                       uint64_t pool_bytes, const void* keys, uint64_t keys_bytes,
                       const void* values, uint64_t values_bytes, const uint32_t* bt,
                       uint64_t bt_bytes, uint64_t start_token, uint64_t n_tokens,
                       const uint32_t* pos_ptr) {
    if (!c || !l) return fail(EH_INVALID_ARGS, "null context or layout");
    if (eh_status ls = check_layout(l)) return ls;
    const uint64_t elt = elt_bytes(l->data_type);
    if (!elt) return fail(EH_UNSUPPORTED, "data_type");
    // paged_kv.rs:240-267 (element size taken from the layout, not fixed at 4).
    const uint64_t pool_expected = eh_kv_layout_bytes_total(l);
    if (pool_bytes < pool_expected) return invalid_size(pool_expected, pool_bytes);
    const uint64_t kv_expected = smul(n_tokens, l->row_len, elt);
    if (keys_bytes < kv_expected) return invalid_size(kv_expected, keys_bytes);
    if (values_bytes < kv_expected) return invalid_size(kv_expected, values_bytes);
    if (bt_bytes == 0) return invalid_size(4, 0);
    if (n_tokens == 0) return EH_OK;
    // Added check: the table must cover start+n tokens when the host knows start.
    if (!pos_ptr) {
        const uint64_t need = smul(div_ceil(sadd(start_token, n_tokens), l->block_tokens), 4);
        if (bt_bytes < need) return invalid_size(need, bt_bytes, "block_table");
    }
    const uint64_t row_bytes = smul(l->row_len, elt);
    const int ch = pick_chunk(row_bytes, {pool, keys, values});
    if (!ch) return fail(EH_UNSUPPORTED, "row alignment", 2, row_bytes);
    const uint64_t total = n_tokens * 2 * (row_bytes / ch);
    if (total >= (1ull << 31) || start_token + n_tokens >= (1ull << 32) || l->block_tokens >= (1ull << 32))
        return invalid_size((1ull << 31) - 1, total, "append too large");
    eh_status st = bind(c);
    if (st) return st;
    char name[32];
    std::snprintf(name, sizeof name, "eh_append_kv_c%d", ch);
    return launch(c, c->mod_kv, name, dim3(grid_for(total, 256)), dim3(256), stream,
                  (const uint8_t*)keys, (const uint8_t*)values, bt,
                  (uint32_t)std::min<uint64_t>(bt_bytes / 4, 0xFFFFFFFFull), (uint8_t*)pool,
                  (uint32_t)n_tokens, (uint32_t)start_token, pos_ptr, (const uint32_t*)nullptr,
                  (const uint32_t*)nullptr, (uint32_t)1, (uint32_t)row_bytes,
                  (uint32_t)l->block_tokens, (uint64_t)l->n_blocks);
}

eh_status eh_gather_kv(eh_context* c, eh_stream stream, const eh_kv_layout* l, const void* pool,
                       uint64_t pool_bytes, const uint32_t* bt, uint64_t bt_bytes, void* out,
                       uint64_t out_bytes, uint64_t start_token, uint64_t n_tokens, int is_value) {
    if (!c || !l) return fail(EH_INVALID_ARGS, "null context or layout");
    if (eh_status ls = check_layout(l)) return ls;
    const uint64_t elt = elt_bytes(l->data_type);
    if (!elt) return fail(EH_UNSUPPORTED, "data_type");
    // paged_kv.rs:391-416
    const uint64_t pool_expected = eh_kv_layout_bytes_total(l);
    if (pool_bytes < pool_expected) return invalid_size(pool_expected, pool_bytes);
    const uint64_t out_expected = smul(n_tokens, l->row_len, elt);
    if (out_bytes < out_expected) return invalid_size(out_expected, out_bytes);
    if (bt_bytes == 0) return invalid_size(4, 0);
    if (n_tokens == 0) return EH_OK;
    const uint64_t need = smul(div_ceil(sadd(start_token, n_tokens), l->block_tokens), 4);
    if (bt_bytes < need) return invalid_size(need, bt_bytes, "block_table");
    const uint64_t row_bytes = smul(l->row_len, elt);
    const int ch = pick_chunk(row_bytes, {pool, out});
    if (!ch) return fail(EH_UNSUPPORTED, "row alignment", 2, row_bytes);
    const uint64_t total = n_tokens * (row_bytes / ch);
    if (total >= (1ull << 31) || start_token + n_tokens >= (1ull << 32))
        return invalid_size((1ull << 31) - 1, total, "gather too large");
    eh_status st = bind(c);
    if (st) return st;
    char name[32];
    std::snprintf(name, sizeof name, "eh_gather_kv_c%d", ch);
    return launch(c, c->mod_kv, name, dim3(grid_for(total, 256)), dim3(256), stream,
                  (const uint8_t*)pool, bt, (uint32_t)std::min<uint64_t>(bt_bytes / 4, 0xFFFFFFFFull),
                  (uint8_t*)out, (uint32_t)n_tokens, (uint32_t)start_token, (uint32_t)(is_value != 0),
                  (uint32_t)row_bytes, (uint32_t)l->block_tokens, (uint64_t)l->n_blocks);
}

eh_status eh_append_kv_batched(eh_context* c, eh_stream stream, const eh_kv_layout* l, void* pool,
                               uint64_t pool_bytes, const void* keys, uint64_t keys_bytes,
                               const void* values, uint64_t values_bytes, const uint32_t* bt,
                               uint64_t bt_bytes, uint32_t bt_stride, const uint32_t* cu_seqlens,
                               const uint32_t* start_pos, uint32_t batch, uint64_t total_tokens) {
    if (!c || !l) return fail(EH_INVALID_ARGS, "null context or layout");
    if (eh_status ls = check_layout(l)) return ls;
    const uint64_t elt = elt_bytes(l->data_type);
    if (!elt) return fail(EH_UNSUPPORTED, "data_type");
    const uint64_t pool_expected = eh_kv_layout_bytes_total(l);
    if (pool_bytes < pool_expected) return invalid_size(pool_expected, pool_bytes);
    const uint64_t kv_expected = smul(total_tokens, l->row_len, elt);
    if (keys_bytes < kv_expected) return invalid_size(kv_expected, keys_bytes);
    if (values_bytes < kv_expected) return invalid_size(kv_expected, values_bytes);
    if (total_tokens == 0 || batch == 0) return EH_OK;
    if (!cu_seqlens || !start_pos) return fail(EH_INVALID_ARGS, "cu_seqlens/start_pos are null");
    if (bt_stride == 0) return invalid_size(1, 0, "bt_stride");
    const uint64_t bt_expected = smul(batch, bt_stride, 4);
    if (bt_bytes < bt_expected) return invalid_size(bt_expected, bt_bytes, "block_tables");
    const uint64_t row_bytes = smul(l->row_len, elt);
    const int ch = pick_chunk(row_bytes, {pool, keys, values});
    if (!ch) return fail(EH_UNSUPPORTED, "row alignment", 2, row_bytes);
    const uint64_t total = total_tokens * 2 * (row_bytes / ch);
    if (total >= (1ull << 31)) return invalid_size((1ull << 31) - 1, total, "append too large");
    eh_status st = bind(c);
    if (st) return st;
    char name[32];
    std::snprintf(name, sizeof name, "eh_append_kv_c%d", ch);
    return launch(c, c->mod_kv, name, dim3(grid_for(total, 256)), dim3(256), stream,
                  (const uint8_t*)keys, (const uint8_t*)values, bt, bt_stride, (uint8_t*)pool,
                  (uint32_t)total_tokens, (uint32_t)0, (const uint32_t*)nullptr, cu_seqlens,
                  start_pos, batch, (uint32_t)row_bytes, (uint32_t)l->block_tokens,
                  (uint64_t)l->n_blocks);
}

// ---- FP8 (E4M3) storage: quantising append and dequantising gather
// (paged_kv.hip).  Elements move four at a time (f32x4 <-> one u32 of codes).
static eh_status check_e4m3(const eh_kv_layout* l, uint64_t head_dim, const float* s0,
                            const float* s1) {
    if (l->data_type != EH_KV_FP8) return fail(EH_UNSUPPORTED, "data_type must be EH_KV_FP8");
    if (head_dim == 0 || head_dim % 4 || l->row_len % head_dim)
        return invalid_size(head_dim, l->row_len, "head_dim (multiple of 4 dividing row_len)");
    if (!s0 || !s1) return fail(EH_INVALID_ARGS, "scale arrays are null");
    return EH_OK;
}

eh_status eh_append_kv_e4m3_batched(eh_context* c, eh_stream stream, const eh_kv_layout* l,
                                    void* pool, uint64_t pool_bytes, const float* keys,
                                    uint64_t keys_bytes, const float* values, uint64_t values_bytes,
                                    const uint32_t* bt, uint64_t bt_bytes, uint32_t bt_stride,
                                    const uint32_t* cu_seqlens, const uint32_t* start_pos,
                                    uint32_t batch, uint64_t total_tokens, uint32_t head_dim,
                                    const float* k_scale, const float* v_scale) {
    if (!c || !l) return fail(EH_INVALID_ARGS, "null context or layout");
    if (eh_status ls = check_layout(l)) return ls;
    eh_status st = check_e4m3(l, head_dim, k_scale, v_scale);
    if (st) return st;
    const uint64_t pool_expected = eh_kv_layout_bytes_total(l);
    if (pool_bytes < pool_expected) return invalid_size(pool_expected, pool_bytes);
    const uint64_t kv_expected = smul(total_tokens, l->row_len, 4);
    if (keys_bytes < kv_expected) return invalid_size(kv_expected, keys_bytes);
    if (values_bytes < kv_expected) return invalid_size(kv_expected, values_bytes);
    if (total_tokens == 0 || batch == 0) return EH_OK;
    if (!cu_seqlens || !start_pos) return fail(EH_INVALID_ARGS, "cu_seqlens/start_pos are null");
    if (bt_stride == 0) return invalid_size(1, 0, "bt_stride");
    const uint64_t bt_expected = smul(batch, bt_stride, 4);
    if (bt_bytes < bt_expected) return invalid_size(bt_expected, bt_bytes, "block_tables");
    if (((uintptr_t)keys | (uintptr_t)values) % 16 || (uintptr_t)pool % 4)
        return fail(EH_UNSUPPORTED, "alignment (keys/values 16 B, pool 4 B)");
    const uint64_t total = total_tokens * 2 * (l->row_len / 4);
    if (total >= (1ull << 31)) return invalid_size((1ull << 31) - 1, total, "append too large");
    st = bind(c);
    if (st) return st;
    return launch(c, c->mod_kv, "eh_append_kv_e4m3", dim3(grid_for(total, 256)), dim3(256), stream,
                  keys, values, bt, bt_stride, (uint8_t*)pool, (uint32_t)total_tokens, (uint32_t)0,
                  (const uint32_t*)nullptr, cu_seqlens, start_pos, batch, (uint32_t)l->row_len,
                  head_dim, (uint32_t)l->block_tokens, (uint64_t)l->n_blocks, k_scale, v_scale);
}

eh_status eh_kv_e4m3_scales(eh_context* c, eh_stream stream, const eh_kv_layout* l,
                            const float* keys, uint64_t keys_bytes, const float* values,
                            uint64_t values_bytes, uint64_t n_rows, uint32_t head_dim,
                            float* k_scale, uint64_t k_scale_bytes, float* v_scale,
                            uint64_t v_scale_bytes) {
    if (!c || !l) return fail(EH_INVALID_ARGS, "null context or layout");
    if (eh_status ls = check_layout(l)) return ls;
    eh_status st = check_e4m3(l, head_dim, k_scale, v_scale);
    if (st) return st;
    const uint64_t n_kv = l->row_len / head_dim;
    if (k_scale_bytes < n_kv * 4) return invalid_size(n_kv * 4, k_scale_bytes, "k_scale");
    if (v_scale_bytes < n_kv * 4) return invalid_size(n_kv * 4, v_scale_bytes, "v_scale");
    if (n_kv > 65535) return invalid_size(65535, n_kv, "kv heads");
    const uint64_t kv_expected = smul(n_rows, l->row_len, 4);
    if (keys_bytes < kv_expected) return invalid_size(kv_expected, keys_bytes);
    if (values_bytes < kv_expected) return invalid_size(kv_expected, values_bytes);
    if (n_rows && (!keys || !values)) return fail(EH_INVALID_ARGS, "keys/values are null");
    if (((uintptr_t)keys | (uintptr_t)values) % 16)
        return fail(EH_UNSUPPORTED, "alignment (keys/values 16 B)");
    if (n_rows > 0xFFFFFFFFull) return invalid_size(0xFFFFFFFFull, n_rows, "rows");
    st = bind(c);
    if (st) return st;
    return launch(c, c->mod_kv, "eh_kv_e4m3_scales", dim3((uint32_t)n_kv, 2), dim3(256), stream,
                  keys, values, (uint32_t)n_rows, (uint32_t)l->row_len, head_dim, k_scale, v_scale);
}

eh_status eh_gather_kv_e4m3(eh_context* c, eh_stream stream, const eh_kv_layout* l,
                            const void* pool, uint64_t pool_bytes, const uint32_t* bt,
                            uint64_t bt_bytes, float* out, uint64_t out_bytes, uint64_t start_token,
                            uint64_t n_tokens, int is_value, uint32_t head_dim, const float* scale) {
    if (!c || !l) return fail(EH_INVALID_ARGS, "null context or layout");
    if (eh_status ls = check_layout(l)) return ls;
    eh_status st = check_e4m3(l, head_dim, scale, scale);
    if (st) return st;
    const uint64_t pool_expected = eh_kv_layout_bytes_total(l);
    if (pool_bytes < pool_expected) return invalid_size(pool_expected, pool_bytes);
    const uint64_t out_expected = smul(n_tokens, l->row_len, 4);
    if (out_bytes < out_expected) return invalid_size(out_expected, out_bytes);
    if (bt_bytes == 0) return invalid_size(4, 0);
    if (n_tokens == 0) return EH_OK;
    const uint64_t need = smul(div_ceil(sadd(start_token, n_tokens), l->block_tokens), 4);
    if (bt_bytes < need) return invalid_size(need, bt_bytes, "block_table");
    if ((uintptr_t)out % 16 || (uintptr_t)pool % 4)
        return fail(EH_UNSUPPORTED, "alignment (out 16 B, pool 4 B)");
    const uint64_t total = n_tokens * (l->row_len / 4);
    if (total >= (1ull << 31) || start_token + n_tokens >= (1ull << 32))
        return invalid_size((1ull << 31) - 1, total, "gather too large");
    st = bind(c);
    if (st) return st;
    return launch(c, c->mod_kv, "eh_gather_kv_e4m3", dim3(grid_for(total, 256)), dim3(256), stream,
                  (const uint8_t*)pool, bt, (uint32_t)std::min<uint64_t>(bt_bytes / 4, 0xFFFFFFFFull),
                  out, (uint32_t)n_tokens, (uint32_t)start_token, (uint32_t)(is_value != 0),
                  (uint32_t)l->row_len, head_dim, (uint32_t)l->block_tokens, (uint64_t)l->n_blocks,
                  scale);
}

eh_status eh_copy_pages(eh_context* c, eh_stream stream, const eh_kv_layout* l, void* pool,
                        uint64_t pool_bytes, const uint32_t* src_ids, const uint32_t* dst_ids,
                        uint32_t n_pairs) {
    if (!c || !l) return fail(EH_INVALID_ARGS, "null context or layout");
    if (eh_status ls = check_layout(l)) return ls;
    const uint64_t elt = elt_bytes(l->data_type);
    if (!elt) return fail(EH_UNSUPPORTED, "data_type");
    const uint64_t pool_expected = eh_kv_layout_bytes_total(l);
    if (pool_bytes < pool_expected) return invalid_size(pool_expected, pool_bytes);
    if (n_pairs == 0) return EH_OK;
    if (!src_ids || !dst_ids) return fail(EH_INVALID_ARGS, "page id arrays are null");
    const uint64_t page_bytes = smul(l->block_tokens, 2, l->row_len, elt);
    const int ch = pick_chunk(page_bytes, {pool});
    if (!ch) return fail(EH_UNSUPPORTED, "page alignment", 2, page_bytes);
    eh_status st = bind(c);
    if (st) return st;
    char name[32];
    std::snprintf(name, sizeof name, "eh_copy_pages_c%d", ch);
    return launch(c, c->mod_kv, name, dim3(std::min<uint32_t>(n_pairs, 65535)), dim3(256), stream,
                  (uint8_t*)pool, src_ids, dst_ids, n_pairs, page_bytes, (uint64_t)l->n_blocks);
}

eh_status eh_stream_pages(eh_context* c, eh_stream stream, const eh_kv_layout* l,
                         const void* pool, uint64_t pool_bytes, const uint32_t* ids,
                         uint64_t ids_bytes, uint32_t n_ids, uint32_t depth, uint32_t grid,
                         uint32_t* out, uint64_t out_bytes) {
    if (!c || !l) return fail(EH_INVALID_ARGS, "null context or layout");
    if (eh_status ls = check_layout(l)) return ls;
    const uint64_t elt = elt_bytes(l->data_type);
    if (!elt) return fail(EH_UNSUPPORTED, "data_type");
    const uint64_t page_bytes = smul(l->block_tokens, 2, l->row_len, elt);
    if (page_bytes == 0 || page_bytes % 16384)
        return fail(EH_UNSUPPORTED, "page bytes: a multiple of 16 KiB", 16384, page_bytes);
    const uint64_t pool_expected = eh_kv_layout_bytes_total(l);
    if (pool_bytes < pool_expected) return invalid_size(pool_expected, pool_bytes);
    if (depth != 1 && depth != 2) return fail(EH_UNSUPPORTED, "depth: 1 or 2", 2, depth);
    if (grid < 1) return invalid_size(1, grid, "grid");
    if (n_ids == 0) return EH_OK;
    if (!ids || !out || !pool) return fail(EH_INVALID_ARGS, "null pool, ids or out");
    if (ids_bytes < 4ull * n_ids) return invalid_size(4ull * n_ids, ids_bytes, "ids");
    const uint64_t out_need = smul(4, grid, 8);
    if (out_bytes < out_need) return invalid_size(out_need, out_bytes, "out");
    eh_status st = bind(c);
    if (st) return st;
    return launch(c, c->mod_kv, depth == 1 ? "eh_stream_pages_d1" : "eh_stream_pages_d2",
                  dim3(grid), dim3(512), stream, (const uint8_t*)pool, ids, n_ids, page_bytes,
                  (uint64_t)l->n_blocks, out);
}

eh_status eh_stream_pages_heads(eh_context* c, eh_stream stream, const eh_kv_layout* l,
                               const void* pool, uint64_t pool_bytes, const uint32_t* ids,
                               uint64_t ids_bytes, uint32_t n_ids, uint32_t head_dim, uint32_t grid,
                               uint32_t* out, uint64_t out_bytes) {
    if (!c || !l) return fail(EH_INVALID_ARGS, "null context or layout");
    if (eh_status ls = check_layout(l)) return ls;
    const uint64_t elt = elt_bytes(l->data_type);
    if (!elt) return fail(EH_UNSUPPORTED, "data_type");
    if (l->block_tokens != 16) return fail(EH_UNSUPPORTED, "block_tokens: 16", 16, l->block_tokens);
    if (head_dim == 0 || l->row_len % head_dim)
        return invalid_size(head_dim, l->row_len, "head_dim (dividing row_len)");
    if (head_dim * elt != 256) return fail(EH_UNSUPPORTED, "kv head row: 256 bytes", 256, head_dim * elt);
    const uint64_t n_kv = l->row_len / head_dim;
    if (n_kv != 1 && n_kv != 2 && n_kv != 4 && n_kv != 8)
        return fail(EH_UNSUPPORTED, "kv heads: 1, 2, 4 or 8", 8, n_kv);
    const uint64_t pool_expected = eh_kv_layout_bytes_total(l);
    if (pool_bytes < pool_expected) return invalid_size(pool_expected, pool_bytes);
    if (grid < 1) return invalid_size(1, grid, "grid");
    if (n_ids == 0) return EH_OK;
    if (!ids || !out || !pool) return fail(EH_INVALID_ARGS, "null pool, ids or out");
    if (ids_bytes < 4ull * n_ids) return invalid_size(4ull * n_ids, ids_bytes, "ids");
    const uint64_t out_need = smul(4, grid, 8);
    if (out_bytes < out_need) return invalid_size(out_need, out_bytes, "out");
    eh_status st = bind(c);
    if (st) return st;
    const uint64_t row_bytes = l->row_len * elt;
    return launch(c, c->mod_kv, "eh_stream_pages_heads", dim3(grid), dim3(512), stream,
                  (const uint8_t*)pool, ids, n_ids, smul(16, 2, row_bytes), (uint64_t)l->n_blocks,
                  (uint32_t)row_bytes, (uint32_t)n_kv, out);
}

eh_status eh_remap_block_tables(eh_context* c, eh_stream stream, uint32_t* bt, uint64_t n_entries,
                                const uint32_t* remap, uint32_t n_remap) {
    if (!c) return fail(EH_INVALID_ARGS, "null context");
    if (n_entries == 0) return EH_OK;
    if (!bt || !remap) return fail(EH_INVALID_ARGS, "null block table or remap");
    eh_status st = bind(c);
    if (st) return st;
    return launch(c, c->mod_kv, "eh_remap_block_tables", dim3(grid_for(n_entries, 256)), dim3(256),
                  stream, bt, n_entries, remap, n_remap);
}

eh_status eh_page_refcounts(eh_context* c, eh_stream stream, const uint32_t* bt, uint32_t bt_stride,
                            const uint32_t* n_used, uint32_t batch, uint32_t* counts,
                            uint32_t n_blocks) {
    if (!c) return fail(EH_INVALID_ARGS, "null context");
    if (n_blocks == 0) return EH_OK;
    if (!counts) return fail(EH_INVALID_ARGS, "null counts");
    eh_status st = bind(c);
    if (st) return st;
    st = launch(c, c->mod_kv, "eh_fill_u32", dim3(grid_for(n_blocks, 256)), dim3(256), stream,
                counts, (uint64_t)n_blocks, (uint32_t)0);
    if (st || batch == 0 || bt_stride == 0) return st;
    if (!bt || !n_used) return fail(EH_INVALID_ARGS, "null block tables or n_used");
    return launch(c, c->mod_kv, "eh_page_refcounts",
                  dim3(grid_for((uint64_t)batch * bt_stride, 256)), dim3(256), stream, bt,
                  bt_stride, n_used, batch, counts, n_blocks);
}

static eh_status single_seq_attention(eh_context* c, eh_stream stream, uint32_t kv_dtype,
                                      const float* q, uint64_t q_bytes, const void* pool,
                                      uint64_t pool_bytes, const uint32_t* bt, uint64_t bt_bytes,
                                      float* out, uint64_t out_bytes, uint64_t n_head,
                                      uint64_t n_head_kv, uint64_t head_dim, uint64_t block_tokens,
                                      uint64_t seq_tokens, uint64_t query_pos, int causal,
                                      const uint32_t* pos_ptr, bool single_pass,
                                      const void* new_k = nullptr, const void* new_v = nullptr,
                                      bool own_ws = false, void* ws = nullptr,
                                      uint64_t ws_bytes = 0) {
    if (!c) return fail(EH_INVALID_ARGS, "null context");
    // partials: the caller's workspace (own_ws) or the context's scratch
    if (own_ws && ws_bytes && (!ws || (uintptr_t)ws % 16))
        return fail(EH_INVALID_ARGS, "workspace is null or not 16-byte aligned");
    float* const part = own_ws ? (float*)ws : c->scratch;
    const uint64_t part_floats = own_ws ? ws_bytes / 4 : c->scratch_floats;
    eh_status st = validate_attention(kv_dtype, q_bytes, pool_bytes, bt_bytes, out_bytes, n_head,
                                      n_head_kv, head_dim, block_tokens, seq_tokens, query_pos);
    if (st) return st;
    st = bind(c);
    if (st) return st;
    const uint64_t page_bytes = smul(block_tokens, 2, n_head_kv, head_dim, elt_bytes(kv_dtype));
    decode_args a{};
    a.kv_dtype = kv_dtype;
    a.q = q;
    a.pool = pool;
    a.n_blocks = pool_bytes / page_bytes;
    a.bt = bt;
    a.bt_stride = (uint32_t)std::min<uint64_t>(bt_bytes / 4, 0xFFFFFFFFull);
    a.lens_ptr = pos_ptr;
    a.lens_mode = pos_ptr ? 1u : 0u;
    a.seq_tokens = (uint32_t)seq_tokens;
    a.query_pos = (uint32_t)query_pos;
    a.causal = causal ? 1u : 0u;
    a.batch = 1;
    a.out = out;
    a.n_head = (uint32_t)n_head;
    a.n_head_kv = (uint32_t)n_head_kv;
    a.head_dim = (uint32_t)head_dim;
    a.block_tokens = (uint32_t)block_tokens;
    // Capacity bound: with pos_ptr the live length is only known on the
    // device, so size the grid for everything the block table can address.
    uint64_t cap = seq_tokens;
    if (pos_ptr) cap = std::max<uint64_t>(cap, (uint64_t)a.bt_stride * block_tokens);
    const decode_kernel dk =
        pick_decode_kernel(kv_dtype, head_dim, n_head, n_head_kv, block_tokens, new_k != nullptr);
    const uint64_t chunk = dk.chunk;
    uint64_t tps = auto_tps(1, dk.units, cap, block_tokens, chunk, dk.slots ? 512 : 1024);
    if (single_pass && cap <= max_tps(block_tokens, chunk))
        tps = std::max<uint64_t>(div_ceil(cap, chunk), 1) * chunk;
    // Grow the split until the partials fit the scratch (or workspace).
    while (div_ceil(cap, tps) > 1 &&
           decode_ws_floats(n_head, div_ceil(cap, tps), head_dim) > part_floats)
        tps *= 2;
    if (own_ws && tps > max_tps(block_tokens, chunk)) {
        const uint64_t least = decode_ws_floats(n_head, div_ceil(cap, max_tps(block_tokens, chunk)),
                                                head_dim) * 4;
        return invalid_size(least, ws_bytes, "workspace");
    }
    if (tps > max_tps(block_tokens, chunk) || div_ceil(cap, tps) > kMaxSplits)
        return invalid_size(max_tps(block_tokens, chunk) * kMaxSplits, cap, "context too long");
    a.tps = (uint32_t)tps;
    a.max_splits = (uint32_t)div_ceil(cap, tps);
    a.part_acc = part;
    a.part_ml = part + n_head * a.max_splits * head_dim;
    a.new_k = new_k;
    a.new_v = new_v;
    return run_decode(c, stream, a);
}

eh_status eh_paged_attention(eh_context* c, eh_stream stream, uint32_t kv_dtype, const float* q,
                             uint64_t q_bytes, const void* pool, uint64_t pool_bytes,
                             const uint32_t* bt, uint64_t bt_bytes, float* out, uint64_t out_bytes,
                             uint64_t n_head, uint64_t n_head_kv, uint64_t head_dim,
                             uint64_t block_tokens, uint64_t seq_tokens, uint64_t query_pos,
                             int causal, const uint32_t* pos_ptr) {
    return single_seq_attention(c, stream, kv_dtype, q, q_bytes, pool, pool_bytes, bt, bt_bytes, out,
                                out_bytes, n_head, n_head_kv, head_dim, block_tokens, seq_tokens,
                                query_pos, causal, pos_ptr, true);
}

eh_status eh_flash_decoding(eh_context* c, eh_stream stream, uint32_t kv_dtype, const float* q,
                            uint64_t q_bytes, const void* pool, uint64_t pool_bytes,
                            const uint32_t* bt, uint64_t bt_bytes, float* out, uint64_t out_bytes,
                            uint64_t n_head, uint64_t n_head_kv, uint64_t head_dim,
                            uint64_t block_tokens, uint64_t seq_tokens, uint64_t query_pos,
                            int causal, const uint32_t* pos_ptr) {
    return single_seq_attention(c, stream, kv_dtype, q, q_bytes, pool, pool_bytes, bt, bt_bytes, out,
                                out_bytes, n_head, n_head_kv, head_dim, block_tokens, seq_tokens,
                                query_pos, causal, pos_ptr, false);
}

static eh_status append_flash_decoding(eh_context* c, eh_stream stream, uint32_t kv_dtype,
                                       const void* keys, uint64_t keys_bytes, const void* values,
                                       uint64_t values_bytes, const float* q, uint64_t q_bytes,
                                       void* pool, uint64_t pool_bytes, const uint32_t* bt,
                                       uint64_t bt_bytes, float* out, uint64_t out_bytes,
                                       uint64_t n_head, uint64_t n_head_kv, uint64_t head_dim,
                                       uint64_t block_tokens, uint64_t query_pos,
                                       const uint32_t* pos_ptr, bool own_ws, void* ws,
                                       uint64_t ws_bytes) {
    if (kv_dtype == EH_KV_FP8) return fail(EH_UNSUPPORTED, "FP8 pages: fused single-sequence step");
    if (!keys || !values) return fail(EH_INVALID_ARGS, "keys / values are null");
    const uint64_t row = n_head_kv * head_dim * elt_bytes(kv_dtype);
    if (keys_bytes < row) return invalid_size(row, keys_bytes);
    if (values_bytes < row) return invalid_size(row, values_bytes);
    // A host-known position must have its page in the table.  This is
    // stricter than the reference, whose append only rejects an empty table
    // (paged_kv.rs:262-267); a device position is checked in the kernel,
    // where a page past the table or the pool is masked (row not written).
    if (!pos_ptr && block_tokens && query_pos / block_tokens >= bt_bytes / 4)
        return invalid_size((query_pos / block_tokens + 1) * 4, bt_bytes, "block_table");
    return single_seq_attention(c, stream, kv_dtype, q, q_bytes, pool, pool_bytes, bt, bt_bytes, out,
                                out_bytes, n_head, n_head_kv, head_dim, block_tokens, query_pos + 1,
                                query_pos, 1, pos_ptr, false, keys, values, own_ws, ws, ws_bytes);
}

eh_status eh_append_flash_decoding(eh_context* c, eh_stream stream, uint32_t kv_dtype,
                                   const void* keys, uint64_t keys_bytes, const void* values,
                                   uint64_t values_bytes, const float* q, uint64_t q_bytes,
                                   void* pool, uint64_t pool_bytes, const uint32_t* bt,
                                   uint64_t bt_bytes, float* out, uint64_t out_bytes,
                                   uint64_t n_head, uint64_t n_head_kv, uint64_t head_dim,
                                   uint64_t block_tokens, uint64_t query_pos,
                                   const uint32_t* pos_ptr) {
    return append_flash_decoding(c, stream, kv_dtype, keys, keys_bytes, values, values_bytes, q,
                                 q_bytes, pool, pool_bytes, bt, bt_bytes, out, out_bytes, n_head,
                                 n_head_kv, head_dim, block_tokens, query_pos, pos_ptr, false,
                                 nullptr, 0);
}

// ---- The single-sequence calls with a caller-owned workspace (no shared
// scratch: calls on different streams may overlap).
uint64_t eh_single_decode_workspace_bytes(void) { return kScratchFloats * sizeof(float); }

eh_status eh_paged_attention_ws(eh_context* c, eh_stream stream, uint32_t kv_dtype, const float* q,
                                uint64_t q_bytes, const void* pool, uint64_t pool_bytes,
                                const uint32_t* bt, uint64_t bt_bytes, float* out,
                                uint64_t out_bytes, uint64_t n_head, uint64_t n_head_kv,
                                uint64_t head_dim, uint64_t block_tokens, uint64_t seq_tokens,
                                uint64_t query_pos, int causal, const uint32_t* pos_ptr,
                                void* workspace, uint64_t workspace_bytes) {
    return single_seq_attention(c, stream, kv_dtype, q, q_bytes, pool, pool_bytes, bt, bt_bytes, out,
                                out_bytes, n_head, n_head_kv, head_dim, block_tokens, seq_tokens,
                                query_pos, causal, pos_ptr, true, nullptr, nullptr, true, workspace,
                                workspace_bytes);
}

eh_status eh_flash_decoding_ws(eh_context* c, eh_stream stream, uint32_t kv_dtype, const float* q,
                               uint64_t q_bytes, const void* pool, uint64_t pool_bytes,
                               const uint32_t* bt, uint64_t bt_bytes, float* out, uint64_t out_bytes,
                               uint64_t n_head, uint64_t n_head_kv, uint64_t head_dim,
                               uint64_t block_tokens, uint64_t seq_tokens, uint64_t query_pos,
                               int causal, const uint32_t* pos_ptr, void* workspace,
                               uint64_t workspace_bytes) {
    return single_seq_attention(c, stream, kv_dtype, q, q_bytes, pool, pool_bytes, bt, bt_bytes, out,
                                out_bytes, n_head, n_head_kv, head_dim, block_tokens, seq_tokens,
                                query_pos, causal, pos_ptr, false, nullptr, nullptr, true, workspace,
                                workspace_bytes);
}

eh_status eh_append_flash_decoding_ws(eh_context* c, eh_stream stream, uint32_t kv_dtype,
                                      const void* keys, uint64_t keys_bytes, const void* values,
                                      uint64_t values_bytes, const float* q, uint64_t q_bytes,
                                      void* pool, uint64_t pool_bytes, const uint32_t* bt,
                                      uint64_t bt_bytes, float* out, uint64_t out_bytes,
                                      uint64_t n_head, uint64_t n_head_kv, uint64_t head_dim,
                                      uint64_t block_tokens, uint64_t query_pos,
                                      const uint32_t* pos_ptr, void* workspace,
                                      uint64_t workspace_bytes) {
    return append_flash_decoding(c, stream, kv_dtype, keys, keys_bytes, values, values_bytes, q,
                                 q_bytes, pool, pool_bytes, bt, bt_bytes, out, out_bytes, n_head,
                                 n_head_kv, head_dim, block_tokens, query_pos, pos_ptr, true,
                                 workspace, workspace_bytes);
}

eh_status eh_decode_plan(uint32_t kv_dtype, uint32_t batch, uint32_t n_head, uint32_t n_head_kv,
                         uint32_t head_dim, uint32_t block_tokens, uint32_t max_ctx,
                         uint32_t hint, uint32_t* tokens_per_split, uint32_t* max_splits,
                         uint64_t* workspace_bytes) {
    if (n_head < 1 || n_head_kv < 1 || n_head % n_head_kv) return fail(EH_INVALID_ARGS, "heads");
    if (block_tokens < 1) return fail(EH_INVALID_ARGS, "block_tokens");
    const tiles_cfg tc = pick_tiles(kv_dtype, head_dim, n_head, n_head_kv, block_tokens, batch);
    if (kv_dtype == EH_KV_FP8 && !(hint == 0 && tc.ok))
        return fail(EH_UNSUPPORTED, "E4M3 pages: token-balanced shapes with hint 0 only");
    if (kv_dtype != EH_KV_FP8 && !dt_name(kv_dtype)) return fail(EH_UNSUPPORTED, "kv_dtype");
    if (hint == 0 && tc.ok) {  // token-balanced kernel: tokens_per_split 0, max_splits = grid
        const uint32_t grid = tiles_grid(tc);
        if (tokens_per_split) *tokens_per_split = 0;
        if (max_splits) *max_splits = grid;
        if (workspace_bytes) *workspace_bytes = tiles_ws_bytes(grid, batch, n_head);
        return EH_OK;
    }
    const decode_kernel dk = pick_decode_kernel(kv_dtype, head_dim, n_head, n_head_kv, block_tokens);
    uint64_t tps = hint ? div_ceil(hint, dk.chunk) * dk.chunk
                        : auto_tps(batch, dk.units, max_ctx, block_tokens, dk.chunk,
                                   dk.slots ? 512 : 1024);
    while (div_ceil(max_ctx ? max_ctx : 1, tps) > kMaxSplits) tps *= 2;
    if (tps > max_tps(block_tokens, dk.chunk))
        return invalid_size(max_tps(block_tokens, dk.chunk), tps, "tokens_per_split");
    const uint32_t ms = (uint32_t)div_ceil(max_ctx ? max_ctx : 1, tps);
    if (tokens_per_split) *tokens_per_split = (uint32_t)tps;
    if (max_splits) *max_splits = ms;
    if (workspace_bytes) *workspace_bytes = 4 * decode_ws_floats((uint64_t)batch * n_head, ms, head_dim);
    return EH_OK;
}

eh_status eh_decode_kernel_name(uint32_t kv_dtype, uint32_t n_head, uint32_t n_head_kv,
                                uint32_t head_dim, uint32_t block_tokens, char* buf, uint64_t size) {
    if (n_head < 1 || n_head_kv < 1 || n_head % n_head_kv) return fail(EH_INVALID_ARGS, "heads");
    if (block_tokens < 1) return fail(EH_INVALID_ARGS, "block_tokens");
    const char* dn = kv_dtype == EH_KV_FP8 ? "fp8" : dt_name(kv_dtype);
    if (!dn) return fail(EH_UNSUPPORTED, "kv_dtype");
    const decode_kernel dk = pick_decode_kernel(kv_dtype, head_dim, n_head, n_head_kv, block_tokens);
    const tiles_cfg tc = pick_tiles(kv_dtype, head_dim, n_head, n_head_kv, block_tokens, 1);
    char name[64];
    if (kv_dtype == EH_KV_FP8 && !tc.ok) return fail(EH_UNSUPPORTED, "E4M3 shape");
    if (tc.ok)
        std::snprintf(name, sizeof name, "eh_decode_tiles_%s_hd128_g%u", dn, tc.g);
    else if (dk.slots)
        std::snprintf(name, sizeof name, "eh_decode_slots_%s_hd%u_h%u", dn, head_dim, dk.gh);
    else
        std::snprintf(name, sizeof name, "eh_decode_split_%s_hd%u_g%u", dn, head_dim, dk.g);
    if (!buf || size <= std::strlen(name)) return invalid_size(std::strlen(name) + 1, size, "name buffer");
    std::memcpy(buf, name, std::strlen(name) + 1);
    return EH_OK;
}

eh_status eh_paged_decode_batched(eh_context* c, eh_stream stream, uint32_t kv_dtype,
                                  const float* q, uint64_t q_bytes, const void* pool,
                                  uint64_t pool_bytes, const uint32_t* bt, uint64_t bt_bytes,
                                  uint32_t bt_stride, const uint32_t* ctx_lens, uint32_t batch,
                                  float* out, uint64_t out_bytes, uint32_t n_head,
                                  uint32_t n_head_kv, uint32_t head_dim, uint32_t block_tokens,
                                  uint32_t tps, uint32_t max_splits, void* ws, uint64_t ws_bytes) {
    if (!c) return fail(EH_INVALID_ARGS, "null context");
    if (n_head < 1) return invalid_size(1, n_head);
    if (n_head_kv < 1) return invalid_size(1, n_head_kv);
    if (n_head % n_head_kv != 0) return invalid_size(n_head_kv, n_head % n_head_kv);
    if (head_dim < 1) return invalid_size(1, head_dim);
    if (block_tokens < 1) return invalid_size(1, block_tokens);
    if (batch == 0) return EH_OK;
    if (!ctx_lens) return fail(EH_INVALID_ARGS, "ctx_lens is null");
    if (max_splits < 1) return invalid_size(1, max_splits, "max_splits");
    if (kv_dtype == EH_KV_FP8) return fail(EH_UNSUPPORTED, "E4M3 pages: eh_paged_decode_batched_e4m3");
    if (tps == 0) {  // token-balanced kernel, max_splits workgroups
        const uint64_t q_expected = smul(batch, n_head, head_dim, 4);
        if (q_bytes < q_expected) return invalid_size(q_expected, q_bytes);
        if (out_bytes < q_expected) return invalid_size(q_expected, out_bytes);
        const uint64_t bt_expected = smul(batch, bt_stride, 4);
        if (bt_stride == 0 || bt_bytes < bt_expected)
            return invalid_size(bt_expected, bt_bytes, "block_tables");
        const tiles_cfg tc = pick_tiles(kv_dtype, head_dim, n_head, n_head_kv, block_tokens, batch);
        if (!tc.ok) return fail(EH_UNSUPPORTED, "tokens_per_split 0: shape outside the balanced kernel");
        const uint64_t page_bytes = smul(block_tokens, 2, n_head_kv, head_dim, 2);
        if (pool_bytes < page_bytes) return invalid_size(page_bytes, pool_bytes);
        const uint64_t ws_need = tiles_ws_bytes(max_splits, batch, n_head);
        if (ws_bytes < ws_need) return invalid_size(ws_need, ws_bytes, "workspace");
        eh_status st = bind(c);
        if (st) return st;
        tiles_args a{};
        a.kv_dtype = kv_dtype;
        a.q = q;
        a.pool = const_cast<void*>(pool);
        a.n_blocks = pool_bytes / page_bytes;
        a.bt = bt;
        a.bt_stride = bt_stride;
        a.lens = ctx_lens;
        a.lens_add = 0;
        a.batch = batch;
        a.out = out;
        a.n_head = n_head;
        a.n_head_kv = n_head_kv;
        a.block_tokens = block_tokens;
        a.grid = max_splits;
        a.ws = ws;
        return run_tiles(c, stream, a, tc);
    }
    const uint64_t q_expected = smul(batch, n_head, head_dim, 4);
    if (q_bytes < q_expected) return invalid_size(q_expected, q_bytes);
    if (out_bytes < q_expected) return invalid_size(q_expected, out_bytes);
    const uint64_t bt_expected = smul(batch, bt_stride, 4);
    if (bt_stride == 0 || bt_bytes < bt_expected) return invalid_size(bt_expected, bt_bytes, "block_tables");
    const uint64_t page_bytes = smul(block_tokens, 2, n_head_kv, head_dim, elt_bytes(kv_dtype));
    if (!dt_name(kv_dtype)) return fail(EH_UNSUPPORTED, "kv_dtype");
    if (!supported_hd(kv_dtype, head_dim)) return fail(EH_UNSUPPORTED, "head_dim", 256, head_dim);
    if (pool_bytes < page_bytes) return invalid_size(page_bytes, pool_bytes);
    if (max_splits > kMaxSplits) return invalid_size(kMaxSplits, max_splits, "max_splits");
    const uint64_t ws_need = smul(4, decode_ws_floats(smul(batch, n_head), max_splits, head_dim));
    if (ws_bytes < ws_need) return invalid_size(ws_need, ws_bytes, "workspace");
    eh_status st = bind(c);
    if (st) return st;
    decode_args a{};
    a.kv_dtype = kv_dtype;
    a.q = q;
    a.pool = pool;
    a.n_blocks = pool_bytes / page_bytes;
    a.bt = bt;
    a.bt_stride = bt_stride;
    a.lens_ptr = ctx_lens;
    a.lens_mode = 2;
    a.batch = batch;
    a.out = out;
    a.n_head = n_head;
    a.n_head_kv = n_head_kv;
    a.head_dim = head_dim;
    a.block_tokens = block_tokens;
    a.tps = tps;
    a.max_splits = max_splits;
    a.part_acc = (float*)ws;
    a.part_ml = (float*)ws + (uint64_t)batch * n_head * max_splits * head_dim;
    return run_decode(c, stream, a);
}

// Token-balanced batched decode with every option: E4M3 scales and the
// protected-sinks range.
static eh_status decode_tiles_entry(eh_context* c, eh_stream stream, uint32_t kv_dtype,
                                    const float* q, uint64_t q_bytes, const void* pool,
                                    uint64_t pool_bytes, const uint32_t* bt, uint64_t bt_bytes,
                                    uint32_t bt_stride, const uint32_t* ctx_lens, uint32_t batch,
                                    float* out, uint64_t out_bytes, uint32_t n_head,
                                    uint32_t n_head_kv, uint32_t head_dim, uint32_t block_tokens,
                                    uint32_t sink, uint32_t window, const float* k_scale,
                                    const float* v_scale, float* block_mass,
                                    uint64_t block_mass_bytes, uint32_t max_splits, void* ws,
                                    uint64_t ws_bytes) {
    if (!c) return fail(EH_INVALID_ARGS, "null context");
    if (n_head < 1) return invalid_size(1, n_head);
    if (n_head_kv < 1) return invalid_size(1, n_head_kv);
    if (n_head % n_head_kv != 0) return invalid_size(n_head_kv, n_head % n_head_kv);
    if (block_tokens < 1) return invalid_size(1, block_tokens);
    if (batch == 0) return EH_OK;
    if (!ctx_lens) return fail(EH_INVALID_ARGS, "ctx_lens is null");
    const bool f8 = kv_dtype == EH_KV_FP8;
    if (f8 && (!k_scale || !v_scale)) return fail(EH_INVALID_ARGS, "scale arrays are null");
    if (max_splits < 1) return invalid_size(1, max_splits, "max_splits");
    const tiles_cfg tc = pick_tiles(kv_dtype, head_dim, n_head, n_head_kv, block_tokens, batch);
    if (!tc.ok) return fail(EH_UNSUPPORTED, "shape outside the token-balanced kernel");
    const uint64_t q_expected = smul(batch, n_head, head_dim, 4);
    if (q_bytes < q_expected) return invalid_size(q_expected, q_bytes);
    if (out_bytes < q_expected) return invalid_size(q_expected, out_bytes);
    const uint64_t bt_expected = smul(batch, bt_stride, 4);
    if (bt_stride == 0 || bt_bytes < bt_expected) return invalid_size(bt_expected, bt_bytes, "block_tables");
    const uint64_t page_bytes = smul(block_tokens, 2, n_head_kv, head_dim, f8 ? 1 : 2);
    if (pool_bytes < page_bytes) return invalid_size(page_bytes, pool_bytes);
    const uint64_t ws_tiles = tiles_ws_bytes(max_splits, batch, n_head);
    const uint64_t ws_need =
        ws_tiles + (block_mass ? mass_ws_bytes(batch, bt_stride, block_tokens, n_head) : 0);
    if (ws_bytes < ws_need) return invalid_size(ws_need, ws_bytes, "workspace");
    if (block_mass && block_mass_bytes < smul(pool_bytes / page_bytes, 4))
        return invalid_size(smul(pool_bytes / page_bytes, 4), block_mass_bytes, "block_mass");
    if (block_tokens % 16) return fail(EH_UNSUPPORTED, "block_tokens");
    eh_status st = bind(c);
    if (st) return st;
    tiles_args a{};
    a.kv_dtype = kv_dtype;
    a.q = q;
    a.pool = const_cast<void*>(pool);
    a.n_blocks = pool_bytes / page_bytes;
    a.bt = bt;
    a.bt_stride = bt_stride;
    a.lens = ctx_lens;
    a.lens_add = 0;
    a.batch = batch;
    a.out = out;
    a.n_head = n_head;
    a.n_head_kv = n_head_kv;
    a.block_tokens = block_tokens;
    a.grid = max_splits;
    a.ws = ws;
    a.k_scale = f8 ? k_scale : nullptr;
    a.v_scale = f8 ? v_scale : nullptr;
    a.sink = sink;
    a.window = window;
    a.block_mass = block_mass;
    a.mass_ws = block_mass ? (uint8_t*)ws + ws_tiles : nullptr;
    return run_tiles(c, stream, a, tc);
}

eh_status eh_paged_decode_batched_e4m3(eh_context* c, eh_stream stream, const float* q,
                                       uint64_t q_bytes, const void* pool, uint64_t pool_bytes,
                                       const uint32_t* bt, uint64_t bt_bytes, uint32_t bt_stride,
                                       const uint32_t* ctx_lens, uint32_t batch, float* out,
                                       uint64_t out_bytes, uint32_t n_head, uint32_t n_head_kv,
                                       uint32_t head_dim, uint32_t block_tokens,
                                       const float* k_scale, const float* v_scale,
                                       uint32_t max_splits, void* ws, uint64_t ws_bytes) {
    return decode_tiles_entry(c, stream, EH_KV_FP8, q, q_bytes, pool, pool_bytes, bt, bt_bytes,
                              bt_stride, ctx_lens, batch, out, out_bytes, n_head, n_head_kv,
                              head_dim, block_tokens, 0, 0, k_scale, v_scale, nullptr, 0,
                              max_splits, ws, ws_bytes);
}

eh_status eh_paged_decode_batched_window(eh_context* c, eh_stream stream, uint32_t kv_dtype,
                                         const float* q, uint64_t q_bytes, const void* pool,
                                         uint64_t pool_bytes, const uint32_t* bt, uint64_t bt_bytes,
                                         uint32_t bt_stride, const uint32_t* ctx_lens,
                                         uint32_t batch, float* out, uint64_t out_bytes,
                                         uint32_t n_head, uint32_t n_head_kv, uint32_t head_dim,
                                         uint32_t block_tokens, uint32_t sink_tokens,
                                         uint32_t window_tokens, const float* k_scale,
                                         const float* v_scale, float* block_mass,
                                         uint64_t block_mass_bytes, uint32_t max_splits, void* ws,
                                         uint64_t ws_bytes) {
    return decode_tiles_entry(c, stream, kv_dtype, q, q_bytes, pool, pool_bytes, bt, bt_bytes,
                              bt_stride, ctx_lens, batch, out, out_bytes, n_head, n_head_kv,
                              head_dim, block_tokens, sink_tokens, window_tokens, k_scale, v_scale,
                              block_mass, block_mass_bytes, max_splits, ws, ws_bytes);
}

uint64_t eh_decode_mass_workspace_bytes(uint32_t batch, uint32_t bt_stride, uint32_t block_tokens,
                                        uint32_t n_head) {
    return mass_ws_bytes(batch, bt_stride, block_tokens, n_head);
}

uint64_t eh_decode_grid_workspace_bytes(uint32_t grid, uint32_t batch, uint32_t n_head) {
    // (grid + batch) * n_head < 2^65; the size saturates where 520 times that
    // leaves 64 bits (no call accepts such a shape)
    const unsigned __int128 b = (unsigned __int128)tiles_ws_bytes(1, 0, 1) *
                                ((uint64_t)grid + batch) * n_head;
    return b > UINT64_MAX ? UINT64_MAX : (uint64_t)b;
}

static eh_status append_decode_body(eh_context* c, eh_stream stream, const eh_kv_layout* l,
                                    void* pool, uint64_t pool_bytes, const void* keys,
                                    uint64_t keys_bytes, const void* values, uint64_t values_bytes,
                                    const uint32_t* bt, uint64_t bt_bytes, uint32_t bt_stride,
                                    const uint32_t* start_pos, uint32_t batch, const float* q,
                                    uint64_t q_bytes, float* out, uint64_t out_bytes,
                                    uint32_t n_head, uint32_t head_dim, uint32_t grid, void* ws,
                                    uint64_t ws_bytes, const float* k_scale,
                                    const float* v_scale) {
    const bool e4m3 = k_scale != nullptr;
    if (!c || !l) return fail(EH_INVALID_ARGS, "null context or layout");
    if (eh_status ls = check_layout(l)) return ls;
    if (batch == 0) return EH_OK;
    if (!start_pos) return fail(EH_INVALID_ARGS, "start_pos is null");
    if (head_dim < 1 || l->row_len % head_dim) return invalid_size(head_dim, l->row_len % (head_dim ? head_dim : 1));
    const uint64_t n_head_kv = l->row_len / head_dim;
    if (n_head < 1 || n_head_kv < 1 || n_head % n_head_kv) return invalid_size(n_head_kv, n_head);
    const uint64_t elt = elt_bytes(l->data_type);
    const uint64_t page_bytes = smul(l->block_tokens, 2, l->row_len, elt);
    if (l->n_blocks < 1 || page_bytes == 0) return fail(EH_INVALID_ARGS, "layout");
    if (pool_bytes < l->n_blocks * page_bytes) return invalid_size(l->n_blocks * page_bytes, pool_bytes);
    if (e4m3 && (l->data_type != EH_KV_FP8 || !v_scale))
        return fail(EH_INVALID_ARGS, "E4M3 fused append+decode: FP8 layout and both scales");
    if (!e4m3 && l->data_type == EH_KV_FP8)
        return fail(EH_UNSUPPORTED, "FP8 pages: use eh_append_decode_batched_e4m3");
    // E4M3: the appended rows arrive as f32 and are quantised in the launch
    const uint64_t row_expected = smul(batch, l->row_len, e4m3 ? 4 : elt);
    if (keys_bytes < row_expected) return invalid_size(row_expected, keys_bytes);
    if (values_bytes < row_expected) return invalid_size(row_expected, values_bytes);
    const uint64_t bt_expected = smul(batch, bt_stride, 4);
    if (bt_stride == 0 || bt_bytes < bt_expected) return invalid_size(bt_expected, bt_bytes, "block_tables");
    const uint64_t q_expected = smul(batch, n_head, head_dim, 4);
    if (q_bytes < q_expected) return invalid_size(q_expected, q_bytes);
    if (out_bytes < q_expected) return invalid_size(q_expected, out_bytes);
    const tiles_cfg tc = pick_tiles(l->data_type, head_dim, n_head, n_head_kv, l->block_tokens, batch);
    if (!tc.ok) return fail(EH_UNSUPPORTED, "fused append+decode: shape outside the balanced kernel");
    if (grid < 1) return invalid_size(1, grid, "grid");
    const uint64_t ws_need = tiles_ws_bytes(grid, batch, n_head);
    if (ws_bytes < ws_need) return invalid_size(ws_need, ws_bytes, "workspace");
    eh_status st = bind(c);
    if (st) return st;
    tiles_args a{};
    a.kv_dtype = l->data_type;
    a.q = q;
    a.pool = pool;
    a.n_blocks = l->n_blocks;
    a.bt = bt;
    a.bt_stride = bt_stride;
    a.lens = start_pos;
    a.lens_add = 1;
    a.new_k = keys;
    a.new_v = values;
    a.batch = batch;
    a.out = out;
    a.n_head = n_head;
    a.n_head_kv = (uint32_t)n_head_kv;
    a.block_tokens = (uint32_t)l->block_tokens;
    a.grid = grid;
    a.ws = ws;
    a.k_scale = k_scale;
    a.v_scale = v_scale;
    return run_tiles(c, stream, a, tc);
}

eh_status eh_append_decode_batched(eh_context* c, eh_stream stream, const eh_kv_layout* l,
                                  void* pool, uint64_t pool_bytes, const void* keys,
                                  uint64_t keys_bytes, const void* values, uint64_t values_bytes,
                                  const uint32_t* bt, uint64_t bt_bytes, uint32_t bt_stride,
                                  const uint32_t* start_pos, uint32_t batch, const float* q,
                                  uint64_t q_bytes, float* out, uint64_t out_bytes, uint32_t n_head,
                                  uint32_t head_dim, uint32_t grid, void* ws, uint64_t ws_bytes) {
    return append_decode_body(c, stream, l, pool, pool_bytes, keys, keys_bytes, values,
                              values_bytes, bt, bt_bytes, bt_stride, start_pos, batch, q, q_bytes,
                              out, out_bytes, n_head, head_dim, grid, ws, ws_bytes, nullptr,
                              nullptr);
}

eh_status eh_append_decode_batched_noalloc(eh_context* c, eh_stream stream, const eh_kv_layout* l,
                                          void* pool, uint64_t pool_bytes, const void* keys,
                                          uint64_t keys_bytes, const void* values,
                                          uint64_t values_bytes, const uint32_t* bt,
                                          uint64_t bt_bytes, uint32_t bt_stride,
                                          const uint32_t* start_pos, uint32_t batch,
                                          const float* q, uint64_t q_bytes, float* out,
                                          uint64_t out_bytes, uint32_t n_head, uint32_t head_dim,
                                          uint32_t grid) {
    // eh_append_decode_batched with this device's static scratch array as the
    // workspace: no device allocation anywhere on this path.  The partials
    // are fully written by each call before they are read, so nothing in the
    // scratch needs clearing; calls on one device share it and must not
    // overlap in time.
    if (!c) return fail(EH_INVALID_ARGS, "null context");
    if (!c->noalloc) return fail(EH_KERNEL_LOAD, "no-alloc scratch missing");
    if (grid >= 1 && batch >= 1) {
        const uint64_t need = tiles_ws_bytes(grid, batch, n_head);
        if (need > c->noalloc_bytes)
            return invalid_size(c->noalloc_bytes, need, "no-alloc scratch limit");
    }
    return append_decode_body(c, stream, l, pool, pool_bytes, keys, keys_bytes, values,
                              values_bytes, bt, bt_bytes, bt_stride, start_pos, batch, q, q_bytes,
                              out, out_bytes, n_head, head_dim, grid, c->noalloc, c->noalloc_bytes,
                              nullptr, nullptr);
}

eh_status eh_append_decode_batched_e4m3(eh_context* c, eh_stream stream, const eh_kv_layout* l,
                                       void* pool, uint64_t pool_bytes, const float* keys,
                                       uint64_t keys_bytes, const float* values,
                                       uint64_t values_bytes, const uint32_t* bt, uint64_t bt_bytes,
                                       uint32_t bt_stride, const uint32_t* start_pos, uint32_t batch,
                                       const float* q, uint64_t q_bytes, float* out,
                                       uint64_t out_bytes, uint32_t n_head, uint32_t head_dim,
                                       uint32_t grid, void* ws, uint64_t ws_bytes,
                                       const float* k_scale, const float* v_scale) {
    if (!k_scale) return fail(EH_INVALID_ARGS, "k_scale is null");
    return append_decode_body(c, stream, l, pool, pool_bytes, keys, keys_bytes, values,
                              values_bytes, bt, bt_bytes, bt_stride, start_pos, batch, q, q_bytes,
                              out, out_bytes, n_head, head_dim, grid, ws, ws_bytes, k_scale,
                              v_scale);
}

uint64_t eh_decode_schedule_bytes(uint32_t batch, uint32_t bt_stride, uint32_t block_tokens,
                                  uint32_t grid) {
    if (batch == 0 || bt_stride == 0 || grid == 0 || block_tokens < 16) return 0;
    return sched_bytes(batch, bt_stride, block_tokens, grid);
}

// Shape checks shared by the schedule builder and the scheduled decode.
static eh_status check_sched_shape(const eh_kv_layout* l, uint32_t batch, uint32_t bt_stride,
                                   uint32_t grid, uint64_t sched_bytes_given) {
    if (!l) return fail(EH_INVALID_ARGS, "null layout");
    if (l->block_tokens < 16 || (l->block_tokens & (l->block_tokens - 1)) ||
        l->block_tokens > 0xFFFFFFFFull)
        return fail(EH_UNSUPPORTED, "block_tokens: a power of two of at least 16");
    if (eh_status ls = check_layout(l)) return ls;
    if (batch > kTilesMaxBatch) return invalid_size(kTilesMaxBatch, batch, "batch");
    if (bt_stride == 0) return invalid_size(1, 0, "bt_stride");
    if (grid < 1) return invalid_size(1, grid, "grid");
    const uint64_t tb = sched_tile_bound(batch, bt_stride, l->block_tokens);
    if (tb > 0x7FFFFFFFull) return invalid_size(0x7FFFFFFFull, tb, "schedule tiles");
    const uint64_t need = sched_bytes(batch, bt_stride, l->block_tokens, grid);
    if (sched_bytes_given < need) return invalid_size(need, sched_bytes_given, "schedule");
    return EH_OK;
}

eh_status eh_decode_schedule(eh_context* c, eh_stream stream, const eh_kv_layout* l,
                             const uint32_t* bt, uint64_t bt_bytes, uint32_t bt_stride,
                             const uint32_t* lens, uint32_t lens_add, uint32_t batch, uint32_t grid,
                             void* sched, uint64_t sched_bytes_given) {
    if (!c) return fail(EH_INVALID_ARGS, "null context");
    if (batch == 0) return EH_OK;
    eh_status st = check_sched_shape(l, batch, bt_stride, grid, sched_bytes_given);
    if (st) return st;
    if (!lens || !bt) return fail(EH_INVALID_ARGS, "lens / block_tables is null");
    // the kernels read and write the schedule as 16-byte records
    if (!sched || (uintptr_t)sched % 16)
        return fail(EH_INVALID_ARGS, "schedule is null or not 16-byte aligned");
    const uint64_t bt_expected = smul(batch, bt_stride, 4);
    if (bt_bytes < bt_expected) return invalid_size(bt_expected, bt_bytes, "block_tables");
    if (l->n_blocks < 1) return fail(EH_INVALID_ARGS, "layout");
    st = bind(c);
    if (st) return st;
    const uint64_t cap = sched_cap(batch, bt_stride, l->block_tokens, grid);
    const uint64_t n_index = std::max<uint64_t>(
        std::max<uint64_t>(grid, batch), sched_tile_bound(batch, bt_stride, l->block_tokens));
    const uint32_t wgs = (uint32_t)std::min<uint64_t>(div_ceil(n_index, 256), 1024);
    return launch_lds(c, c->mod_tiles[0], "eh_decode_tiles_schedule", dim3(wgs), dim3(256),
                      4u * (2u * batch + 1u), stream, lens, lens_add, bt, bt_stride,
                      (uint64_t)l->n_blocks, batch, (uint32_t)l->block_tokens,
                      (uint32_t)log2_exact(l->block_tokens), grid, (uint32_t)cap,
                      (uint32_t)n_index, sched);
}

eh_status eh_append_decode_scheduled(eh_context* c, eh_stream stream, const eh_kv_layout* l,
                                     void* pool, uint64_t pool_bytes, const void* keys,
                                     uint64_t keys_bytes, const void* values,
                                     uint64_t values_bytes, const void* sched,
                                     uint64_t sched_bytes_given, uint32_t bt_stride,
                                     uint32_t batch, const float* q, uint64_t q_bytes, float* out,
                                     uint64_t out_bytes, uint32_t n_head, uint32_t head_dim,
                                     uint32_t grid, void* ws, uint64_t ws_bytes,
                                     const float* k_scale, const float* v_scale) {
    if (!c) return fail(EH_INVALID_ARGS, "null context");
    if (batch == 0) return EH_OK;
    eh_status st = check_sched_shape(l, batch, bt_stride, grid, sched_bytes_given);
    if (st) return st;
    if (!sched || (uintptr_t)sched % 16)
        return fail(EH_INVALID_ARGS, "schedule is null or not 16-byte aligned");
    if ((keys == nullptr) != (values == nullptr)) return fail(EH_INVALID_ARGS, "keys / values");
    if (head_dim < 1 || l->row_len % head_dim) return invalid_size(head_dim, l->row_len % (head_dim ? head_dim : 1));
    const uint64_t n_head_kv = l->row_len / head_dim;
    if (n_head < 1 || n_head_kv < 1 || n_head % n_head_kv) return invalid_size(n_head_kv, n_head);
    const bool f8 = l->data_type == EH_KV_FP8;
    if (f8 && (!k_scale || !v_scale)) return fail(EH_INVALID_ARGS, "E4M3 pages: both scales");
    const uint64_t elt = elt_bytes(l->data_type);
    const uint64_t page_bytes = smul(l->block_tokens, 2, l->row_len, elt);
    if (l->n_blocks < 1 || page_bytes == 0) return fail(EH_INVALID_ARGS, "layout");
    if (pool_bytes < l->n_blocks * page_bytes) return invalid_size(l->n_blocks * page_bytes, pool_bytes);
    if (keys) {  // E4M3: the appended rows arrive as f32 and are quantised in the launch
        const uint64_t row_expected = smul(batch, l->row_len, f8 ? 4 : elt);
        if (keys_bytes < row_expected) return invalid_size(row_expected, keys_bytes);
        if (values_bytes < row_expected) return invalid_size(row_expected, values_bytes);
    }
    const uint64_t q_expected = smul(batch, n_head, head_dim, 4);
    if (q_bytes < q_expected) return invalid_size(q_expected, q_bytes);
    if (out_bytes < q_expected) return invalid_size(q_expected, out_bytes);
    const tiles_cfg tc = pick_tiles(l->data_type, head_dim, n_head, n_head_kv, l->block_tokens, batch);
    if (!tc.ok) return fail(EH_UNSUPPORTED, "scheduled decode: shape outside the balanced kernel");
    const uint64_t ws_need = tiles_ws_bytes(grid, batch, n_head);
    if (ws_bytes < ws_need) return invalid_size(ws_need, ws_bytes, "workspace");
    st = bind(c);
    if (st) return st;
    tiles_args a{};
    a.kv_dtype = l->data_type;
    a.q = q;
    a.pool = pool;
    a.n_blocks = l->n_blocks;
    a.bt = nullptr;
    a.bt_stride = bt_stride;
    a.lens = nullptr;
    a.lens_add = 0;
    a.new_k = keys;
    a.new_v = values;
    a.batch = batch;
    a.out = out;
    a.n_head = n_head;
    a.n_head_kv = (uint32_t)n_head_kv;
    a.block_tokens = (uint32_t)l->block_tokens;
    a.grid = grid;
    a.ws = ws;
    a.k_scale = f8 ? k_scale : nullptr;
    a.v_scale = f8 ? v_scale : nullptr;
    a.sched = sched;
    a.cap = (uint32_t)sched_cap(batch, bt_stride, l->block_tokens, grid);
    return run_tiles(c, stream, a, tc);
}

eh_status eh_flash_attention_prefill(eh_context* c, eh_stream stream, uint32_t kv_dtype,
                                     const float* q, uint64_t q_bytes, const void* pool,
                                     uint64_t pool_bytes, const uint32_t* bt, uint64_t bt_bytes,
                                     float* out, uint64_t out_bytes, uint64_t n_head,
                                     uint64_t n_head_kv, uint64_t head_dim, uint64_t block_tokens,
                                     uint64_t q_tokens, uint64_t pos_offset,
                                     const uint32_t* pos_ptr) {
    if (!c) return fail(EH_INVALID_ARGS, "null context");
    if (n_head < 1) return invalid_size(1, n_head);
    if (n_head_kv < 1) return invalid_size(1, n_head_kv);
    if (n_head % n_head_kv != 0) return invalid_size(n_head_kv, n_head % n_head_kv);
    if (head_dim < 1) return invalid_size(1, head_dim);
    if (block_tokens < 1) return invalid_size(1, block_tokens);
    // flash_attention.rs:142-169: q, out, then the block table of
    // ceil((pos_offset + q_tokens) / block_tokens) entries.
    const uint64_t q_expected = smul(q_tokens, n_head, head_dim, 4);
    if (q_bytes < q_expected) return invalid_size(q_expected, q_bytes);
    if (out_bytes < q_expected) return invalid_size(q_expected, out_bytes);
    const uint64_t bt_expected = smul(div_ceil(sadd(pos_offset, q_tokens), block_tokens), 4);
    if (bt_bytes < bt_expected) return invalid_size(bt_expected, bt_bytes);
    eh_status st = validate_prefill_shape(kv_dtype, n_head, n_head_kv, head_dim, block_tokens,
                                          pool_bytes);
    if (st) return st;
    if (q_tokens > 0x7FFFFFFFull) return invalid_size(0x7FFFFFFFull, q_tokens);
    if (pos_offset > 0xFFFFFFFFull) return invalid_size(0xFFFFFFFFull, pos_offset);
    if (q_tokens == 0) return EH_OK;
    st = bind(c);
    if (st) return st;
    prefill_args a{};
    a.kv_dtype = kv_dtype;
    a.q = q;
    a.pool = pool;
    a.n_blocks = pool_bytes / smul(block_tokens, 2, n_head_kv, head_dim, elt_bytes(kv_dtype));
    a.bt = bt;
    a.bt_stride = 0;
    a.bt_entries = (uint32_t)std::min<uint64_t>(bt_bytes / 4, 0xFFFFFFFFull);
    a.pos_ptr = pos_ptr;
    a.q_tokens = (uint32_t)q_tokens;
    a.pos_offset = (uint32_t)pos_offset;
    a.batch = 1;
    a.max_q = (uint32_t)q_tokens;
    a.out = out;
    a.n_head = (uint32_t)n_head;
    a.n_head_kv = (uint32_t)n_head_kv;
    a.head_dim = (uint32_t)head_dim;
    a.block_tokens = (uint32_t)block_tokens;
    return run_prefill(c, stream, a);
}

static eh_status prefill_batched_body(eh_context* c, eh_stream stream, uint32_t kv_dtype,
                                      const float* q, uint64_t q_bytes, const void* pool,
                                      uint64_t pool_bytes, const uint32_t* bt, uint64_t bt_bytes,
                                      uint32_t bt_stride, const uint32_t* cu_q,
                                      const uint32_t* start_pos, uint32_t batch,
                                      uint32_t max_q_tokens, uint32_t total_q_tokens, float* out,
                                      uint64_t out_bytes, uint32_t n_head, uint32_t n_head_kv,
                                      uint32_t head_dim, uint32_t block_tokens,
                                      const float* k_scale, const float* v_scale) {
    const bool e4m3 = k_scale != nullptr;
    if (!c) return fail(EH_INVALID_ARGS, "null context");
    if (n_head < 1) return invalid_size(1, n_head);
    if (n_head_kv < 1) return invalid_size(1, n_head_kv);
    if (n_head % n_head_kv != 0) return invalid_size(n_head_kv, n_head % n_head_kv);
    if (head_dim < 1) return invalid_size(1, head_dim);
    if (block_tokens < 1) return invalid_size(1, block_tokens);
    const uint64_t q_expected = smul(total_q_tokens, n_head, head_dim, 4);
    if (q_bytes < q_expected) return invalid_size(q_expected, q_bytes);
    if (out_bytes < q_expected) return invalid_size(q_expected, out_bytes);
    const uint64_t bt_expected = smul(batch, bt_stride, 4);
    if (bt_stride == 0 || bt_bytes < bt_expected) return invalid_size(bt_expected, bt_bytes, "block_tables");
    eh_status st = validate_prefill_shape(kv_dtype, n_head, n_head_kv, head_dim, block_tokens,
                                          pool_bytes, e4m3);
    if (st) return st;
    if (batch == 0 || total_q_tokens == 0 || max_q_tokens == 0) return EH_OK;
    if (!cu_q || !start_pos) return fail(EH_INVALID_ARGS, "cu_q / start_pos is null");
    st = bind(c);
    if (st) return st;
    prefill_args a{};
    a.kv_dtype = kv_dtype;
    a.q = q;
    a.pool = pool;
    a.n_blocks = pool_bytes / smul(block_tokens, 2, n_head_kv, head_dim, elt_bytes(kv_dtype));
    a.bt = bt;
    a.bt_stride = bt_stride;
    a.bt_entries = bt_stride;
    a.cu_q = cu_q;
    a.start_pos = start_pos;
    a.q_tokens = total_q_tokens;
    a.batch = batch;
    a.max_q = max_q_tokens;
    a.out = out;
    a.n_head = n_head;
    a.n_head_kv = n_head_kv;
    a.head_dim = head_dim;
    a.block_tokens = block_tokens;
    a.k_scale = k_scale;
    a.v_scale = v_scale;
    return run_prefill(c, stream, a);
}

eh_status eh_prefill_batched(eh_context* c, eh_stream stream, uint32_t kv_dtype, const float* q,
                             uint64_t q_bytes, const void* pool, uint64_t pool_bytes,
                             const uint32_t* bt, uint64_t bt_bytes, uint32_t bt_stride,
                             const uint32_t* cu_q, const uint32_t* start_pos, uint32_t batch,
                             uint32_t max_q_tokens, uint32_t total_q_tokens, float* out,
                             uint64_t out_bytes, uint32_t n_head, uint32_t n_head_kv,
                             uint32_t head_dim, uint32_t block_tokens) {
    return prefill_batched_body(c, stream, kv_dtype, q, q_bytes, pool, pool_bytes, bt, bt_bytes,
                                bt_stride, cu_q, start_pos, batch, max_q_tokens, total_q_tokens,
                                out, out_bytes, n_head, n_head_kv, head_dim, block_tokens, nullptr,
                                nullptr);
}

eh_status eh_prefill_batched_e4m3(eh_context* c, eh_stream stream, const float* q,
                                  uint64_t q_bytes, const void* pool, uint64_t pool_bytes,
                                  const uint32_t* bt, uint64_t bt_bytes, uint32_t bt_stride,
                                  const uint32_t* cu_q, const uint32_t* start_pos, uint32_t batch,
                                  uint32_t max_q_tokens, uint32_t total_q_tokens, float* out,
                                  uint64_t out_bytes, uint32_t n_head, uint32_t n_head_kv,
                                  uint32_t head_dim, uint32_t block_tokens, const float* k_scale,
                                  const float* v_scale) {
    if (!k_scale || !v_scale) return fail(EH_INVALID_ARGS, "scale arrays are null");
    return prefill_batched_body(c, stream, EH_KV_FP8, q, q_bytes, pool, pool_bytes, bt, bt_bytes,
                                bt_stride, cu_q, start_pos, batch, max_q_tokens, total_q_tokens,
                                out, out_bytes, n_head, n_head_kv, head_dim, block_tokens, k_scale,
                                v_scale);
}

}  // extern "C"
