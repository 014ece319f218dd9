// The C ABI (include/insitu.h): contexts, caches, validation and launches.
//
// Validation mirrors the reference's raise sites: config.py:45-61 (head_dim a
// power of two, GQA divisibility), config.py:178-207 (code widths, whole
// bytes), quantize.py:150-156 (threshold_frac >= qk_frac), base.py:67-73
// (capacity), ddr_layout.py:126-146 (beat-friendly planes).
#include <cmath>
#include <cstdio>
#include <cstring>
#include <atomic>
#include <mutex>
#include <string>
#include <vector>

#include "insitu_internal.h"

using namespace insitu;

namespace {

thread_local std::string g_last_error;

int fail(int code, const std::string &msg) {
    g_last_error = msg;
    return code;
}

int hip_fail(hipError_t e, const char *what) {
    return fail(INSITU_EHIP, std::string(what) + ": " + hipGetErrorString(e));
}

#define HIP_TRY(expr, what)                        \
    do {                                           \
        hipError_t e_ = (expr);                    \
        if (e_ != hipSuccess) return hip_fail(e_, what); \
    } while (0)

}  // namespace

int insitu::set_last_error(int code, const char *msg) { return fail(code, msg); }

namespace {

__global__ void zero_u64(unsigned long long *p, int n) {
    int i = threadIdx.x;
    if (i < n) p[i] = 0;
}

bool format_supported(const insitu_format &f, std::string &why) {
    char buf[256];
    if (f.head_dim != 64 && f.head_dim != 128) {
        snprintf(buf, sizeof buf, "head_dim=%d: the HIP kernels support 64 and 128", f.head_dim);
        why = buf;
        return false;
    }
    if (f.key_bits < 1 || f.key_bits > 8 || f.value_bits < 1 || f.value_bits > 8) {
        snprintf(buf, sizeof buf, "key_bits=%d value_bits=%d outside 1..8 (config.py:179-181)",
                 f.key_bits, f.value_bits);
        why = buf;
        return false;
    }
    if (f.norm_bits != 16) {
        why = "norm_bits must be 16 (the row stores two int16 norms)";
        return false;
    }
    if (f.norm_frac < 1 || f.norm_frac > 15) {
        why = "norm_frac must be in 1..15: centroid_frac + norm_frac must reach qk_frac "
              "(quantize.py:150-156)";
        return false;
    }
    if (f.qk_frac != QK_FRAC || f.qk_width != QK_WIDTH || f.centroid_frac != CENT_FRAC ||
        f.acc_frac != ACC_FRAC || f.acc_width != ACC_WIDTH || f.score_width != SCORE_WIDTH ||
        f.prob_frac != PROB_FRAC || f.exp_lut_bits != LUT_BITS) {
        why = "only the reference FixedFormat (Q8.16/Q1.15/acc Q16 32b/score 48b/prob Q15/8-bit LUT) "
              "is implemented";
        return false;
    }
    if (f.rot_rounds < 0 || f.rot_rounds > 2) {
        why = "rot_rounds must be 0, 1 or 2";
        return false;
    }
    return true;
}

}  // namespace

struct insitu_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    bool own_stream = false;
    Tables *hook_tables = nullptr;        // exp table for the exp-LUT test hook
    unsigned long long *hook_flags = nullptr;
    int64_t *hook_i64 = nullptr;          // small staging for host arrays (codebooks)
    size_t hook_i64_n = 0;
    // attend kernel timing (insitu_ctx_timing): event pairs, reused across reads
    bool timing = false;
    std::vector<hipEvent_t> ev;           // 2 per attend: start, end
    size_t ev_used = 0;
    void *blas = nullptr;                 // the host half's rocBLAS state (host_half.hip)
};

// The allocation-free prefill (insitu_attend_causal_static) keeps its chunk
// scratch and the virtual batch's lengths in this array: one copy per device,
// held until the process ends, shared by every call on that device. Host code
// never passes the array's name to a kernel or a copy: it is a host-side
// stand-in; the device address comes from hipGetSymbolAddress, once per device,
// in insitu_ctx_create.
constexpr size_t STATIC_SCRATCH_BYTES = (size_t)64 << 20;
constexpr size_t STATIC_LEN_BYTES = 8192;      // PREFILL_QB int64 lengths, rounded up
static __device__ __align__(256) uint8_t scratch[STATIC_SCRATCH_BYTES];

namespace {

constexpr int MAX_DEVICES = 64;
struct StaticScratch {
    // the device's copy of `scratch`: published last (release), after cs and len, so that a
    // reader that sees it (acquire) sees them too
    std::atomic<uint8_t *> ptr{nullptr};
    ChunkScratch cs;            // its chunk-scratch part and attend count
    int64_t *len = nullptr;     // its lengths part
};
StaticScratch g_static[MAX_DEVICES];
std::mutex g_static_mu;

__global__ void clear_bytes_kernel(uint4 *p, int64_t n16) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += (int64_t)gridDim.x * blockDim.x)
        p[i] = make_uint4(0u, 0u, 0u, 0u);
}

// With `device` current: look the array up and clear it, once per device.
hipError_t static_scratch_setup(int device, hipStream_t stream) {
    std::lock_guard<std::mutex> lock(g_static_mu);
    if (device < 0 || device >= MAX_DEVICES) return hipErrorInvalidDevice;
    StaticScratch &ss = g_static[device];
    if (ss.ptr.load(std::memory_order_acquire)) return hipSuccess;
    void *p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    const int64_t n16 = (int64_t)(STATIC_SCRATCH_BYTES / 16);
    hipLaunchKernelGGL(clear_bytes_kernel, dim3(4096), dim3(256), 0, stream, (uint4 *)p, n16);
    e = hipGetLastError();
    if (e == hipSuccess) e = hipStreamSynchronize(stream);
    if (e != hipSuccess) return e;
    ss.cs.p = p;
    ss.cs.bytes = STATIC_SCRATCH_BYTES - STATIC_LEN_BYTES;
    ss.len = (int64_t *)((uint8_t *)p + ss.cs.bytes);
    ss.ptr.store((uint8_t *)p, std::memory_order_release);
    return hipSuccess;
}

}  // namespace

int insitu::ctx_device(insitu_ctx *c) { return c->device; }
hipStream_t insitu::ctx_stream(insitu_ctx *c) { return c->stream; }
void *&insitu::ctx_blas(insitu_ctx *c) { return c->blas; }

// The chunked attend's two builds (attend_chunked.hip): 1,024-token chunks, the default, and
// 512-token chunks (insitu_cache_desc.chunk_tokens = 512).
static const insitu::ChunkedApi k_chunk1024 = {
    1024, insitu::chunked_supported, insitu::chunked_max_chunks, insitu::chunked_pool_slots,
    insitu::chunked_scratch_bytes, insitu::chunked_query_area, insitu::launch_attend_chunked};
static const insitu::ChunkedApi k_chunk512 = {
    512, insitu::c512::chunked_supported, insitu::c512::chunked_max_chunks, insitu::c512::chunked_pool_slots,
    insitu::c512::chunked_scratch_bytes, insitu::c512::chunked_query_area, insitu::c512::launch_attend_chunked};

struct insitu_cache {
    insitu_ctx *ctx = nullptr;
    insitu_cache_desc desc{};
    Geom g{};
    Tables tabs_host{};
    Tables *tabs = nullptr;
    uint8_t *base = nullptr;
    int64_t total_bytes = 0;
    int64_t *len_dev[2] = {nullptr, nullptr};
    int cur = 0;
    std::vector<int64_t> len_host;
    DevStats *stats = nullptr;
    int32_t *wire_scratch = nullptr;      // insitu_step: the rotated queries
    const ChunkedApi *api = nullptr;      // the chunked attend's build: 1,024- or 512-token chunks
    bool chunked = false;                 // the chunked attend handles this format and capacity
    bool vsplit = false;                  // ... seeing each KV head's 8 query heads as two chains of 4
    bool gpad = false;                    // ... computing fewer than 4 query heads a KV head in 4 slots
    bool scan = false;                    // the scan attend does (sequential mode)
    bool step = false;                    // the fused step's own kernel does (sequential mode)
    int64_t step_mc = 0;                  // its layout: chunks per sequence
    ChunkScratch scr;                     // decode attends: run sums and counters, one call's worth
    int64_t max_chunks = 0, pool = 0;     // the chunked attend's layout
    int64_t scan_mc = 0;                  // the scan attend's: chunks per sequence
    // prefill (insitu_attend_causal): scratch for a virtual batch of queries, their lengths
    ChunkScratch prefill_scr;
    int64_t *prefill_len = nullptr;
    int32_t spin_limit = 1 << 20;         // insitu_cache_debug
    int32_t path = 0;                     // insitu_cache_debug: 0 auto, 1 scan, 2 chunked, 3 step kernel
    int32_t append_path = 0;              // insitu_cache_debug: 0 auto, 1 the lane-per-channel kernel
};

namespace {

void fill_exp(Tables &t) {
    for (int i = 0; i < 256; ++i)
        t.exp_table[i] = (int32_t)std::nearbyint(std::exp2(-(double)i / 256.0) * 32768.0);
    // attention.py:145-146: ceil(((span << shift) << acc_frac) / log2e).
    const int64_t num = ((int64_t)LUT_SPAN << (ACC_FRAC - LUT_BITS)) << ACC_FRAC;
    t.delta_max = (num + LOG2E_Q16 - 1) / LOG2E_Q16;
}

int ensure_hook(insitu_ctx *c, size_t n) {
    if (c->hook_i64_n >= n) return INSITU_OK;
    if (c->hook_i64) hipFree(c->hook_i64);
    c->hook_i64 = nullptr;
    HIP_TRY(hipMalloc(&c->hook_i64, n * sizeof(int64_t)), "hipMalloc");
    c->hook_i64_n = n;
    return INSITU_OK;
}

int copy_stats(insitu_cache *c, insitu_stats *out) {
    if (!out) return INSITU_OK;
    DevStats h{};
    HIP_TRY(hipMemcpyAsync(&h, c->stats, sizeof h, hipMemcpyDeviceToHost, c->ctx->stream),
            "stats copy");
    HIP_TRY(hipStreamSynchronize(c->ctx->stream), "stream sync");
    out->n_tokens = (int64_t)h.n_tokens;
    out->rescale_events = (int64_t)h.rescale_events;
    out->score_overflows = (int64_t)h.score_overflows;
    out->acc_overflows = (int64_t)h.acc_overflows;
    out->max_abs_score = (int64_t)h.max_abs_score;
    out->max_abs_acc = (int64_t)h.max_abs_acc;
    out->range_errors = (int64_t)h.range_errors;
    out->serial_fallbacks = (int64_t)h.serial_fallbacks;
    if (h.fault) return fail(INSITU_EFAULT, "a kernel raised its internal fault flag");
    return INSITU_OK;
}

int zero_stats(insitu_cache *c) {
    hipLaunchKernelGGL(zero_u64, dim3(1), dim3(64), 0, c->ctx->stream,
                       (unsigned long long *)c->stats, (int)(sizeof(DevStats) / 8));
    HIP_TRY(hipGetLastError(), "zero stats");
    return INSITU_OK;
}

}  // namespace

// The start/stop events of an attend when timing is on (null events otherwise),
// from the context's pool; the launches record them.
int insitu::timing_events(insitu_ctx *c, LaunchEv *ev) {
    *ev = LaunchEv{};
    if (!c->timing) return INSITU_OK;
    while (c->ev.size() < c->ev_used + 2) {
        hipEvent_t e;
        HIP_TRY(hipEventCreate(&e), "hipEventCreate");
        c->ev.push_back(e);
    }
    ev->start = c->ev[c->ev_used++];
    ev->stop = c->ev[c->ev_used++];
    return INSITU_OK;
}

extern "C" {

const char *insitu_last_error(void) { return g_last_error.c_str(); }

int insitu_ctx_create(int32_t device, void *hip_stream, insitu_ctx **out) {
    if (!out) return fail(INSITU_EINVAL, "out is NULL");
    *out = nullptr;
    int n = 0;
    HIP_TRY(hipGetDeviceCount(&n), "hipGetDeviceCount");
    if (device < 0 || device >= n) return fail(INSITU_EINVAL, "no such device");
    HIP_TRY(hipSetDevice(device), "hipSetDevice");
    auto *c = new insitu_ctx();
    c->device = device;
    // NULL is the device's default stream (what torch uses unless told
    // otherwise), so library kernels and the caller's copies stay ordered.
    c->stream = (hipStream_t)hip_stream;
    Tables t{};
    fill_exp(t);
    hipError_t e = hipMalloc(&c->hook_tables, sizeof(Tables));
    if (e == hipSuccess) e = hipMemcpy(c->hook_tables, &t, sizeof(Tables), hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMalloc(&c->hook_flags, 64);
    if (e == hipSuccess) e = static_scratch_setup(device, c->stream);
    if (e != hipSuccess) {
        insitu_ctx_destroy(c);
        return hip_fail(e, "ctx set-up");
    }
    *out = c;
    return INSITU_OK;
}

int insitu_ctx_destroy(insitu_ctx *c) {
    if (!c) return INSITU_OK;
    hipSetDevice(c->device);
    if (c->stream) hipStreamSynchronize(c->stream);
    for (hipEvent_t e : c->ev) hipEventDestroy(e);
    if (c->hook_tables) hipFree(c->hook_tables);
    if (c->hook_flags) hipFree(c->hook_flags);
    if (c->hook_i64) hipFree(c->hook_i64);
    blas_release(c);
    if (c->own_stream && c->stream) hipStreamDestroy(c->stream);
    delete c;
    return INSITU_OK;
}

int insitu_ctx_sync(insitu_ctx *c) {
    if (!c) return fail(INSITU_EINVAL, "ctx is NULL");
    HIP_TRY(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    return INSITU_OK;
}

void *insitu_ctx_stream(insitu_ctx *c) { return c ? (void *)c->stream : nullptr; }

int insitu_ctx_timing(insitu_ctx *c, int32_t enable) {
    if (!c) return fail(INSITU_EINVAL, "ctx is NULL");
    c->timing = enable != 0;
    c->ev_used = 0;
    return INSITU_OK;
}

int insitu_ctx_timing_read(insitu_ctx *c, double *total_ms, int64_t *n_attends) {
    if (!c || !total_ms || !n_attends) return fail(INSITU_EINVAL, "null argument");
    HIP_TRY(hipSetDevice(c->device), "hipSetDevice");
    double sum = 0.0;
    if (c->ev_used) HIP_TRY(hipEventSynchronize(c->ev[c->ev_used - 1]), "hipEventSynchronize");
    for (size_t i = 0; i + 1 < c->ev_used; i += 2) {
        float ms = 0.0f;
        HIP_TRY(hipEventElapsedTime(&ms, c->ev[i], c->ev[i + 1]), "hipEventElapsedTime");
        sum += ms;
    }
    *total_ms = sum;
    *n_attends = (int64_t)(c->ev_used / 2);
    c->ev_used = 0;
    return INSITU_OK;
}

int insitu_ctx_timing_read_each(insitu_ctx *c, double *ms_each, int64_t cap, int64_t *n_attends) {
    if (!c || !n_attends || (!ms_each && cap)) return fail(INSITU_EINVAL, "null argument");
    HIP_TRY(hipSetDevice(c->device), "hipSetDevice");
    const int64_t n = (int64_t)(c->ev_used / 2);
    if (n > cap) return fail(INSITU_EBADLEN, "more timed attends than the array holds");
    if (c->ev_used) HIP_TRY(hipEventSynchronize(c->ev[c->ev_used - 1]), "hipEventSynchronize");
    for (int64_t i = 0; i < n; ++i) {
        float ms = 0.0f;
        HIP_TRY(hipEventElapsedTime(&ms, c->ev[2 * i], c->ev[2 * i + 1]), "hipEventElapsedTime");
        ms_each[i] = ms;
    }
    *n_attends = n;
    c->ev_used = 0;
    return INSITU_OK;
}

int insitu_rotate(insitu_ctx *c, const int32_t *x, int32_t *y, int64_t n_vec,
                  const insitu_format *fmt) {
    if (!c || !fmt || (!x && n_vec) || (!y && n_vec)) return fail(INSITU_EINVAL, "null argument");
    const int d = fmt->head_dim;
    if (d < 16 || d > 128 || (d & (d - 1)))
        return fail(INSITU_EINVAL, "rotate supports power-of-two d in 16..128 (rotate.py:146-147)");
    if (fmt->rot_rounds < 0 || fmt->rot_rounds > 2) return fail(INSITU_EINVAL, "rot_rounds 0..2");
    if (n_vec < 0 || n_vec > 0x7fffffff) return fail(INSITU_EBADLEN, "n_vec out of range");
    HIP_TRY(hipSetDevice(c->device), "hipSetDevice");
    HIP_TRY(launch_rotate(c->stream, x, y, n_vec, d, fmt->rot_rounds, fmt->rot_signs,
                          c->hook_flags),
            "rotate launch");
    return INSITU_OK;
}

int insitu_encode(insitu_ctx *c, const int32_t *x, int64_t n_vec, const insitu_format *fmt,
                  const int64_t *bounds_host, int32_t bits, int32_t *norm, uint8_t *codes) {
    if (!c || !fmt || !bounds_host) return fail(INSITU_EINVAL, "null argument");
    std::string why;
    if (!format_supported(*fmt, why)) return fail(INSITU_EINVAL, why);
    if (bits < 1 || bits > 8) return fail(INSITU_EINVAL, "bits outside 1..8");
    if (n_vec < 0 || n_vec > 0x7fffffff) return fail(INSITU_EBADLEN, "n_vec out of range");
    HIP_TRY(hipSetDevice(c->device), "hipSetDevice");
    const int nb = (1 << bits) - 1;
    int rc = ensure_hook(c, 256);
    if (rc) return rc;
    HIP_TRY(hipMemcpyAsync(c->hook_i64, bounds_host, nb * sizeof(int64_t), hipMemcpyHostToDevice,
                           c->stream),
            "bounds upload");
    HIP_TRY(launch_encode(c->stream, x, n_vec, fmt->head_dim, fmt->norm_frac, c->hook_i64, nb, norm,
                          codes),
            "encode launch");
    HIP_TRY(hipStreamSynchronize(c->stream), "sync");   // the staging buffer is reused
    return INSITU_OK;
}

int insitu_qtab(insitu_ctx *c, const int32_t *q, int32_t n_heads, int32_t d,
                const int64_t *centroids_host, int32_t n_c, int64_t *table) {
    if (!c || !centroids_host) return fail(INSITU_EINVAL, "null argument");
    if (n_c < 1 || n_c > 256 || n_heads < 0 || d < 1) return fail(INSITU_EBADLEN, "bad shape");
    HIP_TRY(hipSetDevice(c->device), "hipSetDevice");
    int rc = ensure_hook(c, 256);
    if (rc) return rc;
    HIP_TRY(hipMemcpyAsync(c->hook_i64, centroids_host, n_c * sizeof(int64_t),
                           hipMemcpyHostToDevice, c->stream),
            "centroid upload");
    HIP_TRY(launch_qtab(c->stream, q, n_heads, d, c->hook_i64, n_c, table), "qtab launch");
    HIP_TRY(hipStreamSynchronize(c->stream), "sync");
    return INSITU_OK;
}

int insitu_exp_lut(insitu_ctx *c, const int64_t *delta, int64_t n, int32_t *p) {
    if (!c) return fail(INSITU_EINVAL, "null argument");
    HIP_TRY(hipSetDevice(c->device), "hipSetDevice");
    HIP_TRY(launch_exp_lut(c->stream, c->hook_tables, delta, n, p), "exp launch");
    return INSITU_OK;
}

int insitu_finalize(insitu_ctx *c, const int64_t *acc, const int64_t *l, int32_t rows, int32_t d,
                    int64_t *out, int64_t *recip, int32_t *shift) {
    if (!c) return fail(INSITU_EINVAL, "null argument");
    HIP_TRY(hipSetDevice(c->device), "hipSetDevice");
    HIP_TRY(launch_finalize(c->stream, acc, l, rows, d, out, recip, shift), "finalize launch");
    return INSITU_OK;
}

// The geometry the chunked attend sees: the cache's, or with every KV head as two chains of
// 4 query heads (vsplit; planes from KV head h >> 1).
static Geom chunk_geom(const insitu_cache *k, Geom g) {
    if (k->vsplit) {
        g.n_kv *= 2;
        g.G = 4;
        g.kv_shift = 1;
    } else if (k->gpad) {
        // 1 to 3 query heads a KV head: the chain's 4 slots compute head h % G (the slots
        // past G duplicate; their outputs and statistics are dropped)
        g.gq = g.G;
        g.G = 4;
    }
    return g;
}

int insitu_cache_create(insitu_ctx *c, const insitu_cache_desc *desc, insitu_cache **out) {
    if (!c || !desc || !out) return fail(INSITU_EINVAL, "null argument");
    *out = nullptr;
    std::string why;
    if (!format_supported(desc->fmt, why)) return fail(INSITU_EINVAL, why);
    const insitu_format &f = desc->fmt;
    if (desc->n_kv_heads < 1 || desc->n_q_heads < 1 || desc->n_q_heads % desc->n_kv_heads)
        return fail(INSITU_EINVAL, "num_heads must be a multiple of num_kv_heads (config.py:49-53)");
    if (desc->n_q_heads / desc->n_kv_heads > MAX_G)
        return fail(INSITU_EINVAL, "more than 8 query heads per KV head is not supported");
    if (desc->batch < 1 || desc->capacity < 1) return fail(INSITU_EINVAL, "batch and capacity >= 1");
    if (desc->chunk_tokens != 0 && desc->chunk_tokens != 512 && desc->chunk_tokens != 1024)
        return fail(INSITU_EINVAL, "chunk_tokens is 0 (the default, 1,024), 512 or 1,024");
    if (!desc->key_centroids_host || !desc->key_bounds_host || !desc->value_centroids_host ||
        !desc->value_bounds_host)
        return fail(INSITU_EINVAL, "codebooks are required");
    const int nk = 1 << f.key_bits, nv = 1 << f.value_bits;
    for (int i = 1; i < nk; ++i)
        if (desc->key_centroids_host[i] <= desc->key_centroids_host[i - 1])
            return fail(INSITU_EINVAL, "key centroids must be strictly ascending (codebook.py:55-58)");
    for (int i = 1; i < nv; ++i)
        if (desc->value_centroids_host[i] <= desc->value_centroids_host[i - 1])
            return fail(INSITU_EINVAL, "value centroids must be strictly ascending");
    for (int i = 0; i < nk; ++i)
        if (std::llabs(desc->key_centroids_host[i]) >= (1ll << 20))
            return fail(INSITU_ERANGE, "a key centroid does not fit 20 bits (hw/vectors.py:314)");
    for (int i = 0; i < nv; ++i)
        if (std::llabs(desc->value_centroids_host[i]) >= (1ll << 20))
            return fail(INSITU_ERANGE, "a value centroid does not fit 20 bits");

    HIP_TRY(hipSetDevice(c->device), "hipSetDevice");
    auto *k = new insitu_cache();
    k->ctx = c;
    k->desc = *desc;
    k->desc.key_centroids_host = k->desc.key_bounds_host = nullptr;
    k->desc.value_centroids_host = k->desc.value_bounds_host = nullptr;

    Geom &g = k->g;
    g.d = f.head_dim;
    g.kb = f.key_bits;
    g.vb = f.value_bits;
    g.norm_frac = f.norm_frac;
    g.n_kv = desc->n_kv_heads;
    g.n_q = desc->n_q_heads;
    g.G = g.n_q / g.n_kv;
    g.batch = desc->batch;
    g.capacity = desc->capacity;
    g.key_bytes = g.d * g.kb / 8;
    g.value_bytes = g.d * g.vb / 8;
    g.row_bytes = g.key_bytes + g.value_bytes + 4;
    // ddr_layout.py:110-124 + 148-163: fields first, then 16-byte beats.
    const int fields[3][2] = {{0, g.key_bytes},
                              {g.key_bytes, g.key_bytes + g.value_bytes},
                              {g.key_bytes + g.value_bytes, g.row_bytes}};
    g.n_planes = 0;
    int maxw = 0;
    for (auto &fl : fields) {
        for (int a = fl[0]; a < fl[1];) {
            int bnd = a + 16 < fl[1] ? a + 16 : fl[1];
            if (g.n_planes >= MAX_PLANES) {
                delete k;
                return fail(INSITU_EINVAL, "row needs more than 16 planes");
            }
            g.plane_lo[g.n_planes] = a;
            g.plane_w[g.n_planes] = bnd - a;
            if (16 % (bnd - a)) {
                delete k;
                return fail(INSITU_EINVAL, "plane width does not divide the 16-byte beat "
                                           "(ddr_layout.py:140-146)");
            }
            maxw = maxw > bnd - a ? maxw : bnd - a;
            ++g.n_planes;
            a = bnd;
        }
    }
    g.span = (desc->capacity * maxw + 4095) / 4096 * 4096;   // ddr_layout.py:195-196
    g.head_stride = g.n_planes * g.span;
    g.seq_stride = g.n_kv * g.head_stride;
    k->total_bytes = g.seq_stride * g.batch;

    Tables &t = k->tabs_host;
    fill_exp(t);
    for (int i = 0; i < nk; ++i) t.kc[i] = desc->key_centroids_host[i];
    t.kc_absmax = 0.0;
    for (int i = 0; i < nk; ++i) t.kc_absmax = std::fmax(t.kc_absmax, std::fabs((double)t.kc[i]));
    for (int i = 0; i + 1 < nk; ++i) t.kbnd[i] = desc->key_bounds_host[i];
    for (int i = 0; i < nv; ++i) t.vc[i] = desc->value_centroids_host[i];
    for (int i = 0; i + 1 < nv; ++i) t.vbnd[i] = desc->value_bounds_host[i];
    t.bnd_sorted = 1;
    for (int i = 0; i + 2 < nk; ++i) t.bnd_sorted &= t.kbnd[i] <= t.kbnd[i + 1] ? 1 : 0;
    for (int i = 0; i + 2 < nv; ++i) t.bnd_sorted &= t.vbnd[i] <= t.vbnd[i + 1] ? 1 : 0;

    hipError_t e = hipMalloc(&k->base, k->total_bytes);
    if (e == hipSuccess) e = hipMemsetAsync(k->base, 0, k->total_bytes, c->stream);
    if (e == hipSuccess) e = hipMalloc(&k->tabs, sizeof(Tables));
    if (e == hipSuccess)
        e = hipMemcpyAsync(k->tabs, &t, sizeof(Tables), hipMemcpyHostToDevice, c->stream);
    for (int i = 0; i < 2 && e == hipSuccess; ++i) {
        e = hipMalloc(&k->len_dev[i], sizeof(int64_t) * g.batch);
        if (e == hipSuccess) e = hipMemsetAsync(k->len_dev[i], 0, sizeof(int64_t) * g.batch, c->stream);
    }
    if (e == hipSuccess) e = hipMalloc(&k->stats, sizeof(DevStats));
    if (e == hipSuccess) e = hipMemsetAsync(k->stats, 0, sizeof(DevStats), c->stream);
    if (e == hipSuccess)
        e = hipMalloc(&k->wire_scratch,
                      sizeof(int32_t) * (size_t)g.batch * (g.n_q + 2 * g.n_kv) * g.d);
    k->api = desc->chunk_tokens == 512 ? &k_chunk512 : &k_chunk1024;
    k->chunked = k->api->supported(g, desc->capacity);
    k->scan = scan_supported(g, desc->capacity);
    k->step = step_supported(g, desc->capacity);
    if (!k->chunked && !k->scan && g.G == 8) {
        // 8 query heads a KV head, in a format only the chunked attend takes: as two chains of
        // 4 query heads over the same rows (the rows are read twice, the recurrence is each
        // head's own either way)
        k->vsplit = true;
        k->chunked = k->api->supported(chunk_geom(k, g), desc->capacity);
        k->vsplit = k->chunked;
    } else if (!k->chunked && g.G >= 1 && g.G < 4) {
        k->gpad = true;
        k->chunked = k->api->supported(chunk_geom(k, g), desc->capacity);
        k->gpad = k->chunked;
    }
    if (e == hipSuccess && (k->chunked || k->scan || k->step)) {
        size_t nb = 0;
        if (k->step) {
            k->step_mc = step_max_chunks(desc->capacity);
            nb = step_scratch_bytes(g, k->step_mc);
        }
        if (k->chunked) {
            k->max_chunks = k->api->max_chunks(desc->capacity);
            k->pool = k->api->pool_slots(k->max_chunks);
            const size_t nc = k->api->scratch_bytes(chunk_geom(k, g), k->max_chunks, k->pool);
            nb = nc > nb ? nc : nb;
        }
        if (k->scan) {
            k->scan_mc = scan_max_chunks(desc->capacity);
            const size_t ns = scan_scratch_bytes(g, k->scan_mc);
            nb = ns > nb ? ns : nb;
        }
        e = hipMalloc(&k->scr.p, nb);
        k->scr.bytes = nb;
        if (e == hipSuccess) e = hipMemsetAsync(k->scr.p, 0, nb, c->stream);
    }
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) {
        insitu_cache_destroy(k);
        return e == hipErrorOutOfMemory ? fail(INSITU_ENOMEM, "cache allocation")
                                        : hip_fail(e, "cache allocation");
    }
    g.base = k->base;
    k->len_host.assign(g.batch, 0);
    *out = k;
    return INSITU_OK;
}

int insitu_cache_destroy(insitu_cache *k) {
    if (!k) return INSITU_OK;
    hipSetDevice(k->ctx->device);
    hipStreamSynchronize(k->ctx->stream);
    if (k->base) hipFree(k->base);
    if (k->tabs) hipFree(k->tabs);
    for (auto *p : k->len_dev)
        if (p) hipFree(p);
    if (k->stats) hipFree(k->stats);
    if (k->wire_scratch) hipFree(k->wire_scratch);
    if (k->scr.p) hipFree(k->scr.p);
    if (k->prefill_scr.p) hipFree(k->prefill_scr.p);
    if (k->prefill_len) hipFree(k->prefill_len);
    delete k;
    return INSITU_OK;
}

int insitu_cache_reset(insitu_cache *k) {
    if (!k) return fail(INSITU_EINVAL, "cache is NULL");
    HIP_TRY(hipSetDevice(k->ctx->device), "hipSetDevice");
    for (auto *p : k->len_dev)
        HIP_TRY(hipMemsetAsync(p, 0, sizeof(int64_t) * k->g.batch, k->ctx->stream), "reset");
    HIP_TRY(hipStreamSynchronize(k->ctx->stream), "sync");
    k->len_host.assign(k->g.batch, 0);
    return INSITU_OK;
}

int insitu_cache_length(const insitu_cache *k, int32_t seq, int64_t *len) {
    if (!k || !len) return fail(INSITU_EINVAL, "null argument");
    if (seq < 0 || seq >= k->g.batch) return fail(INSITU_EINVAL, "no such sequence");
    *len = k->len_host[seq];
    return INSITU_OK;
}

int insitu_cache_set_length(insitu_cache *k, int32_t seq, int64_t len) {
    if (!k) return fail(INSITU_EINVAL, "cache is NULL");
    if (seq < 0 || seq >= k->g.batch) return fail(INSITU_EINVAL, "no such sequence");
    if (len < 0 || len > k->g.capacity) return fail(INSITU_ECAPACITY, "length beyond capacity");
    HIP_TRY(hipSetDevice(k->ctx->device), "hipSetDevice");
    k->len_host[seq] = len;
    HIP_TRY(hipMemcpyAsync(k->len_dev[k->cur] + seq, &k->len_host[seq], sizeof(int64_t),
                           hipMemcpyHostToDevice, k->ctx->stream),
            "length upload");
    HIP_TRY(hipStreamSynchronize(k->ctx->stream), "sync");
    return INSITU_OK;
}

int insitu_cache_layout(const insitu_cache *k, insitu_layout *o) {
    if (!k || !o) return fail(INSITU_EINVAL, "null argument");
    std::memset(o, 0, sizeof *o);
    o->row_bytes = k->g.row_bytes;
    o->n_planes = k->g.n_planes;
    for (int p = 0; p < k->g.n_planes; ++p) {
        o->plane_lo[p] = k->g.plane_lo[p];
        o->plane_width[p] = k->g.plane_w[p];
    }
    o->plane_span = k->g.span;
    o->head_stride = k->g.head_stride;
    o->seq_stride = k->g.seq_stride;
    o->total_bytes = k->total_bytes;
    o->device_base = (uint64_t)(uintptr_t)k->base;
    return INSITU_OK;
}

static int append_impl(insitu_cache *k, int seq_lo, int seq_hi, const int32_t *kr,
                       const int32_t *vr, int32_t n_tok, bool wire = false) {
    if (!k || !kr || !vr) return fail(INSITU_EINVAL, "null argument");
    if (n_tok < 0) return fail(INSITU_EBADLEN, "n_tok < 0");
    if (n_tok == 0) return INSITU_OK;
    for (int b = seq_lo; b < seq_hi; ++b)
        if (k->len_host[b] + n_tok > k->g.capacity) {
            char buf[200];
            snprintf(buf, sizeof buf,
                     "cache holds %lld of %lld tokens; cannot append %d (base.py:67-73)",
                     (long long)k->len_host[b], (long long)k->g.capacity, n_tok);
            return fail(INSITU_ECAPACITY, buf);
        }
    HIP_TRY(hipSetDevice(k->ctx->device), "hipSetDevice");
    HIP_TRY(launch_append(k->ctx->stream, k->g, k->tabs, kr, vr, n_tok, seq_lo, seq_hi,
                          k->len_dev[k->cur], k->len_dev[k->cur ^ 1], k->stats,
                          wire ? k->desc.fmt.rot_rounds : 0, wire ? k->desc.fmt.rot_signs : nullptr,
                          k->append_path == 0 ? &k->tabs_host : nullptr),
            "append launch");
    k->cur ^= 1;
    for (int b = seq_lo; b < seq_hi; ++b) k->len_host[b] += n_tok;
    return INSITU_OK;
}

int insitu_append(insitu_cache *k, const int32_t *kr, const int32_t *vr, int32_t n_tok) {
    if (!k) return fail(INSITU_EINVAL, "cache is NULL");
    return append_impl(k, 0, k->g.batch, kr, vr, n_tok);
}

int insitu_append_seq(insitu_cache *k, int32_t seq, const int32_t *kr, const int32_t *vr,
                      int32_t n_tok) {
    if (!k) return fail(INSITU_EINVAL, "cache is NULL");
    if (seq < 0 || seq >= k->g.batch) return fail(INSITU_EINVAL, "no such sequence");
    return append_impl(k, seq, seq + 1, kr, vr, n_tok);
}

int insitu_append_wire(insitu_cache *k, int32_t seq, const int32_t *kw, const int32_t *vw, int32_t n_tok) {
    if (!k) return fail(INSITU_EINVAL, "cache is NULL");
    if (seq < -1 || seq >= k->g.batch) return fail(INSITU_EINVAL, "no such sequence");
    if (k->desc.fmt.rot_rounds < 1 || k->desc.fmt.rot_rounds > 2)
        return fail(INSITU_EINVAL, "the cache's format has no rotation of one or two rounds");
    return seq < 0 ? append_impl(k, 0, k->g.batch, kw, vw, n_tok, true)
                   : append_impl(k, seq, seq + 1, kw, vw, n_tok, true);
}


// Sequential (and split) mode: the chunked attend where it handles the format and
// capacity (d = 64 or 128, 4 query heads per KV head, up to 512 chunks), the scan
// attend elsewhere (8 query heads per KV head; longer contexts); a test hook can
// pin either.
static bool use_scan(const insitu_cache *k, int32_t mode) {
    if (mode == INSITU_SERIAL || mode == INSITU_TWO_PASS || !k->scan) return false;
    if (k->path == 1) return true;
    if (k->path == 2 || k->path == 3) return false;
    return !k->chunked;
}

// The fused decode step's own kernel (attend_step.hip), sequential and split mode, wherever
// it handles the format (d = 64, 4 query heads per KV head, 4-bit keys, 2-bit values, up to
// 512 chunks of 1,024 tokens); the test hook can pin the chunked (2) or scan (1) attend.
static bool use_step_kernel(const insitu_cache *k, int32_t mode) {
    if ((mode != INSITU_SEQUENTIAL && mode != INSITU_SPLIT) || !k->step) return false;
    return k->path == 0 || k->path == 3;
}

// q_staged: the chunked path's fp64 query staging already holds q (the step's
// write kernel filled it). step: the whole decode step in the attend launch
// (chunked sequential mode; the lengths are those before the step).
// ep: the attend's epoch from scratch_begin (0: take one here).
static int attend_impl(insitu_cache *k, const int32_t *q, int32_t *out, int32_t mode,
                       bool q_staged, const StepIn *step = nullptr, uint32_t ep = 0) {
    const int64_t *len = k->len_dev[k->cur];
    const int two_pass = mode == INSITU_TWO_PASS ? 1 : 0;
    LaunchEv ev;
    int rc = timing_events(k->ctx, &ev);
    if (rc) return rc;
    if (use_scan(k, mode)) {
        // the scan attend, its grid sized by the longest sequence
        if (!ep) HIP_TRY(scratch_begin(k->ctx->stream, k->scr, &ep), "scratch clear");
        k->scr.spin_limit = k->spin_limit;
        int64_t longest = 0;
        for (int64_t n : k->len_host) longest = n > longest ? n : longest;
        const int64_t chunks = scan_max_chunks(longest + (step ? 1 : 0));
        HIP_TRY(launch_attend_scan(k->ctx->stream, k->g, k->tabs, q, out, len, k->scr, ep, k->scan_mc, chunks,
                                   step, ev, k->stats),
                "scan attend launch");
        return INSITU_OK;
    }
    if (step && use_step_kernel(k, mode)) {
        // the fused step's own kernel, its grid sized by the longest sequence
        if (!ep) HIP_TRY(scratch_begin(k->ctx->stream, k->scr, &ep), "scratch clear");
        k->scr.spin_limit = k->spin_limit;
        int64_t longest = 0;
        for (int64_t n : k->len_host) longest = n > longest ? n : longest;
        HIP_TRY(launch_step(k->ctx->stream, k->g, k->tabs, out, len, k->scr, ep, k->step_mc,
                            step_max_chunks(longest + 1), *step, ev, k->stats),
                "step launch");
        return INSITU_OK;
    }
    if (mode != INSITU_SERIAL && k->chunked) {
        if (!ep) HIP_TRY(scratch_begin(k->ctx->stream, k->scr, &ep), "scratch clear");
        k->scr.spin_limit = k->spin_limit;
        int64_t longest = 0;
        for (int64_t n : k->len_host) longest = n > longest ? n : longest;
        HIP_TRY(k->api->launch(k->ctx->stream, chunk_geom(k, k->g), k->tabs, q, out, len, k->scr, ep,
                               k->max_chunks, k->pool, two_pass, q_staged, step, ev, k->stats, 0,
                               k->api->max_chunks(longest + (step ? 1 : 0))),
                "chunked attend launch");
        return INSITU_OK;
    }
    HIP_TRY(launch_attend_serial(k->ctx->stream, k->g, k->tabs, q, out, len, two_pass, ev, k->stats),
            "attend launch");
    return INSITU_OK;
}

int insitu_attend(insitu_cache *k, const int32_t *q, int32_t *out, int32_t mode,
                  insitu_stats *stats) {
    if (!k || !q || !out) return fail(INSITU_EINVAL, "null argument");
    if (mode < INSITU_SEQUENTIAL || mode > INSITU_SERIAL) return fail(INSITU_EINVAL, "unknown mode");
    HIP_TRY(hipSetDevice(k->ctx->device), "hipSetDevice");
    // Statistics are only gathered (and the device counters only cleared) when
    // the caller asks for them; without them the call never synchronises.
    int rc = stats ? zero_stats(k) : INSITU_OK;
    if (rc) return rc;
    rc = attend_impl(k, q, out, mode, false);
    if (rc) return rc;
    return copy_stats(k, stats);
}

// A prefill attend (attend_causal_batch / attend_online_batch, attention.py:517-871)
// runs as a virtual batch: query i a "sequence" of its own length base + i + 1
// whose planes are those of the real sequence (sequence stride 0). Every query
// then gets exactly the decode path's arithmetic over rows 0 .. base + i.
//
// The chunk scratch of a launch is laid out for its own longest query (its
// chunk count, not the cache's capacity), and a launch takes as many queries as
// fit PREFILL_SCRATCH_BUDGET (at most PREFILL_QB): at ctx 32k and d = 64 about
// 2.2 MB per query, so 116 queries per launch; at d = 128 and ctx 131,072 about
// 17 MB per query, so 15.
constexpr int64_t PREFILL_QB = 1024;
constexpr size_t PREFILL_SCRATCH_BUDGET = (size_t)256 << 20;

__global__ void prefill_lengths_kernel(int64_t *len, int64_t first, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) len[i] = first + i;
}

namespace {

// How many queries one prefill launch takes, and the scratch it needs: the
// launch's chunk count is that of its longest query, base + n_q rows.
struct PrefillPlan {
    int64_t qb, max_chunks, pool;
    size_t bytes;
};
PrefillPlan prefill_plan(const ChunkedApi &api, const Geom &gv, int64_t base, int64_t n_q, size_t budget) {
    // gv: the geometry the chunked attend sees (chunk_geom)
    PrefillPlan pl{};
    pl.max_chunks = api.max_chunks(base + n_q);
    pl.pool = api.pool_slots(pl.max_chunks);
    Geom one = gv;
    one.batch = 1;
    const size_t per_q = api.scratch_bytes(one, pl.max_chunks, pl.pool);
    pl.qb = (int64_t)(budget / (per_q ? per_q : 1));
    if (pl.qb > PREFILL_QB) pl.qb = PREFILL_QB;
    if (pl.qb > n_q) pl.qb = n_q;
    Geom all = gv;
    all.batch = (int32_t)(pl.qb > 0 ? pl.qb : 1);
    pl.bytes = api.scratch_bytes(all, pl.max_chunks, pl.pool);
    return pl;
}

}  // namespace

// The prefill launches over a scratch the caller provides (scr, lengths len_dev for
// PREFILL_QB queries); shared by insitu_attend_causal and its allocation-free variant.
static int prefill_launches(insitu_cache *k, const Geom &gv, const PrefillPlan &pl, ChunkScratch &scr,
                            int64_t *len_dev, int64_t base, int64_t n_q, const int32_t *q, int32_t *out,
                            int32_t mode, bool timed = true) {
    const Geom &g = k->g;
    const bool chunked = mode != INSITU_SERIAL && k->chunked;
    const int64_t row = (int64_t)g.n_q * g.d;
    const int64_t qb = chunked ? pl.qb : PREFILL_QB;
    Geom gb = gv;
    for (int64_t i0 = 0; i0 < n_q; i0 += qb) {
        const int64_t nb = n_q - i0 < qb ? n_q - i0 : qb;
        gb.batch = (int32_t)nb;
        hipLaunchKernelGGL(prefill_lengths_kernel, dim3((unsigned)((nb + 255) / 256)), dim3(256), 0,
                           k->ctx->stream, len_dev, base + i0 + 1, nb);
        HIP_TRY(hipGetLastError(), "prefill lengths");
        LaunchEv ev;
        int rc = timed ? timing_events(k->ctx, &ev) : INSITU_OK;
        if (rc) return rc;
        if (chunked) {
            uint32_t ep = 0;
            HIP_TRY(scratch_begin(k->ctx->stream, scr, &ep), "scratch clear");
            scr.spin_limit = k->spin_limit;
            HIP_TRY(k->api->launch(k->ctx->stream, chunk_geom(k, gb), k->tabs, q + i0 * row, out + i0 * row, len_dev,
                                   scr, ep, pl.max_chunks, pl.pool, mode == INSITU_TWO_PASS ? 1 : 0,
                                   false, nullptr, ev, k->stats, pl.qb, 0),
                    "prefill attend launch");
        } else {
            HIP_TRY(launch_attend_serial(k->ctx->stream, gb, k->tabs, q + i0 * row, out + i0 * row, len_dev,
                                         mode == INSITU_TWO_PASS ? 1 : 0, ev, k->stats),
                    "prefill attend launch");
        }
    }
    return INSITU_OK;
}

static int prefill_check(insitu_cache *k, int32_t seq, int64_t base, int64_t n_q, const int32_t *q,
                         int32_t *out, int32_t mode) {
    if (!k || (n_q > 0 && (!q || !out))) return fail(INSITU_EINVAL, "null argument");
    if (mode < INSITU_SEQUENTIAL || mode > INSITU_SERIAL) return fail(INSITU_EINVAL, "unknown mode");
    const Geom &g = k->g;
    if (seq < 0 || seq >= g.batch) return fail(INSITU_EINVAL, "no such sequence");
    if (base < 0 || n_q < 0 || base + n_q > k->len_host[seq]) {
        char buf[200];
        snprintf(buf, sizeof buf, "queries %lld .. %lld attend rows 0 .. base + i, but the sequence "
                 "holds %lld rows", (long long)base, (long long)(base + n_q - 1),
                 (long long)k->len_host[seq]);
        return fail(INSITU_EBADLEN, buf);
    }
    return INSITU_OK;
}

// The prefill attend over the geometry gv: the whole sequence (every KV head), or
// one KV head of it (n_kv = 1, planes from that head's).
static int causal_impl(insitu_cache *k, const Geom &gv, int64_t base, int64_t n_q, const int32_t *q,
                       int32_t *out, int32_t mode, insitu_stats *stats) {
    HIP_TRY(hipSetDevice(k->ctx->device), "hipSetDevice");
    int rc = stats ? zero_stats(k) : INSITU_OK;
    if (rc) return rc;
    if (n_q == 0) return copy_stats(k, stats);
    const PrefillPlan pl = prefill_plan(*k->api, chunk_geom(k, gv), base, n_q, PREFILL_SCRATCH_BUDGET);
    if (!k->prefill_len) HIP_TRY(hipMalloc(&k->prefill_len, PREFILL_QB * sizeof(int64_t)), "hipMalloc");
    if (mode != INSITU_SERIAL && k->chunked && k->prefill_scr.bytes < pl.bytes) {
        // grow: the old buffer may still be in use by queued launches
        HIP_TRY(hipStreamSynchronize(k->ctx->stream), "sync");
        if (k->prefill_scr.p) HIP_TRY(hipFree(k->prefill_scr.p), "hipFree");
        k->prefill_scr.p = nullptr;
        k->prefill_scr.bytes = 0;
        HIP_TRY(hipMalloc(&k->prefill_scr.p, pl.bytes), "hipMalloc");
        HIP_TRY(hipMemsetAsync(k->prefill_scr.p, 0, pl.bytes, k->ctx->stream), "hipMemsetAsync");
        k->prefill_scr.bytes = pl.bytes;
        k->prefill_scr.calls = 0;
    }
    rc = prefill_launches(k, gv, pl, k->prefill_scr, k->prefill_len, base, n_q, q, out, mode);
    if (rc) return rc;
    return copy_stats(k, stats);
}

int insitu_attend_causal(insitu_cache *k, int32_t seq, int64_t base, int64_t n_q, const int32_t *q,
                         int32_t *out, int32_t mode, insitu_stats *stats) {
    int rc = prefill_check(k, seq, base, n_q, q, out, mode);
    if (rc) return rc;
    const Geom &g = k->g;
    Geom gv = g;
    gv.base = g.base + (int64_t)seq * g.seq_stride;
    gv.seq_stride = 0;
    return causal_impl(k, gv, base, n_q, q, out, mode, stats);
}

int insitu_attend_causal_head(insitu_cache *k, int32_t seq, int32_t kv_head, int64_t base, int64_t n_q,
                              const int32_t *q, int32_t *out, int32_t mode, insitu_stats *stats) {
    int rc = prefill_check(k, seq, base, n_q, q, out, mode);
    if (rc) return rc;
    const Geom &g = k->g;
    if (kv_head < 0 || kv_head >= g.n_kv) return fail(INSITU_EINVAL, "no such KV head");
    Geom gv = g;
    gv.base = g.base + (int64_t)seq * g.seq_stride + (int64_t)kv_head * g.head_stride;
    gv.seq_stride = 0;
    gv.n_kv = 1;
    gv.n_q = g.G;
    return causal_impl(k, gv, base, n_q, q, out, mode, stats);
}

int insitu_attend_causal_static(insitu_cache *k, int32_t seq, int64_t base, int64_t n_q, const int32_t *q,
                                int32_t *out, int32_t mode) {
    int rc = prefill_check(k, seq, base, n_q, q, out, mode);
    if (rc) return rc;
    if (n_q == 0) return INSITU_OK;
    const int dev = k->ctx->device;
    if (dev < 0 || dev >= MAX_DEVICES || !g_static[dev].ptr.load(std::memory_order_acquire))
        return fail(INSITU_EINVAL, "the device's static scratch is not set up (insitu_ctx_create)");
    StaticScratch &ss = g_static[dev];
    HIP_TRY(hipSetDevice(dev), "hipSetDevice");
    const Geom &g = k->g;
    Geom gv = g;
    gv.base = g.base + (int64_t)seq * g.seq_stride;
    gv.seq_stride = 0;
    PrefillPlan pl{};
    if (mode != INSITU_SERIAL && k->chunked) {
        pl = prefill_plan(*k->api, chunk_geom(k, gv), base, n_q, ss.cs.bytes);
        if (pl.qb < 1) {
            Geom one = chunk_geom(k, gv);
            one.batch = 1;
            char buf[240];
            snprintf(buf, sizeof buf, "one query over %lld rows needs %zu B of chunk scratch; the static "
                     "scratch holds %zu B (insitu_attend_causal allocates instead)", (long long)(base + n_q),
                     k->api->scratch_bytes(one, pl.max_chunks, pl.pool), ss.cs.bytes);
            return fail(INSITU_EBADLEN, buf);
        }
    }
    return prefill_launches(k, gv, pl, ss.cs, ss.len, base, n_q, q, out, mode, false);
}

int insitu_step(insitu_cache *k, const int32_t *q, const int32_t *kw, const int32_t *vw,
                int32_t *out, int32_t mode, insitu_stats *stats) {
    if (!k || !q || !kw || !vw || !out) return fail(INSITU_EINVAL, "null argument");
    if (mode < INSITU_SEQUENTIAL || mode > INSITU_SERIAL) return fail(INSITU_EINVAL, "unknown mode");
    const Geom &g = k->g;
    int32_t *qr = k->wire_scratch;
    for (int b = 0; b < g.batch; ++b)
        if (k->len_host[b] + 1 > g.capacity) {
            char buf[200];
            snprintf(buf, sizeof buf, "cache holds %lld of %lld tokens; cannot append (base.py:67-73)",
                     (long long)k->len_host[b], (long long)g.capacity);
            return fail(INSITU_ECAPACITY, buf);
        }
    HIP_TRY(hipSetDevice(k->ctx->device), "hipSetDevice");
    int rc = stats ? zero_stats(k) : INSITU_OK;
    if (rc) return rc;
    // kernel.py:271-284: k, v and q are all rotated, the k/v row appended (the
    // token attends to itself), then the attend (:337-345). In chunked
    // sequential mode at d = 64 that is one launch; otherwise one write kernel
    // (which also stages the rotated queries for a chunked attend) and the attend.
    const bool scan = use_scan(k, mode);
    const bool chunked = !scan && mode != INSITU_SERIAL && k->chunked;
    // (a KV head seen as two chains would write its new row twice, and duplicate query slots
    // would count the rotation's range errors twice: two launches then)
    const bool fused = scan || use_step_kernel(k, mode) ||
                       (mode != INSITU_TWO_PASS && chunked && !k->vsplit && !k->gpad && chunked_fused_step(g));
    if (fused) {
        StepIn si;
        si.qw = q;
        si.kw = kw;
        si.vw = vw;
        si.sg = rot_signs(k->desc.fmt.rot_rounds, k->desc.fmt.rot_signs);
        si.rounds = k->desc.fmt.rot_rounds;
        si.len_out = k->len_dev[k->cur ^ 1];
        rc = attend_impl(k, qr, out, mode, false, &si);
        if (rc) return rc;
        k->cur ^= 1;
        for (int b = 0; b < g.batch; ++b) k->len_host[b] += 1;
        return copy_stats(k, stats);
    }
    double *qd = nullptr;
    int32_t *qok = nullptr;
    uint32_t ep = 0;
    // the chunked attend's query staging (4 query heads a KV head, as the write kernel stages
    // them; a KV head seen as two chains reads the rotated queries instead)
    const bool staged = chunked && !k->vsplit && !k->gpad;
    if (staged) {
        // the epoch (and the wrap's clear) before the write kernel stages the queries
        HIP_TRY(scratch_begin(k->ctx->stream, k->scr, &ep), "scratch clear");
        k->api->query_area(g, k->max_chunks, k->pool, k->scr.p, &qd, &qok);
    }
    HIP_TRY(launch_step_write(k->ctx->stream, g, k->tabs, q, kw, vw, k->desc.fmt.rot_rounds,
                              k->desc.fmt.rot_signs, qr, qd, qok, k->len_dev[k->cur],
                              k->len_dev[k->cur ^ 1], k->stats),
            "step write launch");
    k->cur ^= 1;
    for (int b = 0; b < g.batch; ++b) k->len_host[b] += 1;
    rc = attend_impl(k, qr, out, mode, staged, nullptr, ep);
    if (rc) return rc;
    return copy_stats(k, stats);
}

// Test hook: the invariants of a scratch layout, computed on the host (no GPU call).
int insitu_debug_scratch_layout(int32_t kernel, int64_t capacity, int32_t batch, int32_t n_kv, int32_t d,
                                int64_t *facts, int32_t n) {
    if (!facts || n < 11 || capacity < 1 || batch < 1 || n_kv < 1 || (d != 64 && d != 128))
        return fail(INSITU_EINVAL, "bad argument");
    Geom g{};
    g.batch = batch;
    g.n_kv = n_kv;
    g.d = d;
    g.G = 4;
    g.n_q = 4 * n_kv;
    if (kernel == 0)
        insitu::chunked_layout_facts(g, insitu::chunked_max_chunks(capacity), facts);
    else if (kernel == 1)
        insitu::c512::chunked_layout_facts(g, insitu::c512::chunked_max_chunks(capacity), facts);
    else if (kernel == 2 && d == 64)
        insitu::step_layout_facts(g, insitu::step_max_chunks(capacity), facts);
    else
        return fail(INSITU_EINVAL, "kernel: 0 chunked (1,024-token chunks), 1 chunked (512), 2 step (d = 64)");
    return INSITU_OK;
}

int insitu_cache_debug(insitu_cache *k, int32_t what, int64_t value) {
    if (!k) return fail(INSITU_EINVAL, "cache is NULL");
    switch (what) {
    case INSITU_DEBUG_DECODE_CALLS:
        if (value < 0 || value > 0xFFFFFFFFll) return fail(INSITU_EINVAL, "call count out of range");
        k->scr.calls = (uint32_t)value;
        return INSITU_OK;
    case INSITU_DEBUG_PREFILL_CALLS:
        if (value < 0 || value > 0xFFFFFFFFll) return fail(INSITU_EINVAL, "call count out of range");
        k->prefill_scr.calls = (uint32_t)value;
        return INSITU_OK;
    case INSITU_DEBUG_SPIN_LIMIT:
        if (value < 0 || value > (1 << 30)) return fail(INSITU_EINVAL, "spin limit out of range");
        k->spin_limit = (int32_t)value;
        return INSITU_OK;
    case INSITU_DEBUG_PATH:
        if (value == 1 && !k->scan) return fail(INSITU_EINVAL, "the scan attend does not handle this cache");
        if (value == 2 && !k->chunked) return fail(INSITU_EINVAL, "the chunked attend does not handle this cache");
        if (value == 3 && !k->step) return fail(INSITU_EINVAL, "the step kernel does not handle this cache");
        if (value < 0 || value > 3)
            return fail(INSITU_EINVAL, "path is 0 (auto), 1 (scan), 2 (chunked) or 3 (step kernel)");
        k->path = (int32_t)value;
        return INSITU_OK;
    case INSITU_DEBUG_APPEND:
        if (value < 0 || value > 1) return fail(INSITU_EINVAL, "append kernel is 0 (auto) or 1 (lane per channel)");
        k->append_path = (int32_t)value;
        return INSITU_OK;
    default:
        return fail(INSITU_EINVAL, "unknown debug setting");
    }
}

int insitu_cache_stats(insitu_cache *k, insitu_stats *stats) {
    if (!k || !stats) return fail(INSITU_EINVAL, "null argument");
    HIP_TRY(hipSetDevice(k->ctx->device), "hipSetDevice");
    const int rc = copy_stats(k, stats);
    const int rz = zero_stats(k);
    return rc != INSITU_OK ? rc : rz;
}

int insitu_read_rows(insitu_cache *k, int32_t seq, int32_t head, int64_t t0, int64_t n,
                     uint8_t *rows) {
    if (!k || (!rows && n)) return fail(INSITU_EINVAL, "null argument");
    const Geom &g = k->g;
    if (seq < 0 || seq >= g.batch || head < 0 || head >= g.n_kv)
        return fail(INSITU_EINVAL, "no such sequence/head");
    if (t0 < 0 || n < 0 || t0 + n > g.capacity) return fail(INSITU_EBADLEN, "rows outside capacity");
    if (n == 0) return INSITU_OK;
    HIP_TRY(hipSetDevice(k->ctx->device), "hipSetDevice");
    std::vector<uint8_t> stage((size_t)n * 16);
    for (int p = 0; p < g.n_planes; ++p) {
        const int w = g.plane_w[p];
        const uint8_t *src = g.base + seq * g.seq_stride + head * g.head_stride + p * g.span + t0 * w;
        HIP_TRY(hipMemcpyAsync(stage.data(), src, (size_t)n * w, hipMemcpyDeviceToHost, k->ctx->stream),
                "row read");
        HIP_TRY(hipStreamSynchronize(k->ctx->stream), "sync");
        for (int64_t t = 0; t < n; ++t)
            std::memcpy(rows + t * g.row_bytes + g.plane_lo[p], stage.data() + t * w, w);
    }
    return INSITU_OK;
}

int insitu_load_rows(insitu_cache *k, int32_t seq, int32_t head, int64_t t0, int64_t n,
                     const uint8_t *rows) {
    if (!k || (!rows && n)) return fail(INSITU_EINVAL, "null argument");
    const Geom &g = k->g;
    if (seq < 0 || seq >= g.batch || head < 0 || head >= g.n_kv)
        return fail(INSITU_EINVAL, "no such sequence/head");
    if (t0 < 0 || n < 0 || t0 + n > g.capacity) return fail(INSITU_EBADLEN, "rows outside capacity");
    if (n == 0) return INSITU_OK;
    HIP_TRY(hipSetDevice(k->ctx->device), "hipSetDevice");
    std::vector<uint8_t> stage((size_t)n * 16);
    for (int p = 0; p < g.n_planes; ++p) {
        const int w = g.plane_w[p];
        for (int64_t t = 0; t < n; ++t)
            std::memcpy(stage.data() + t * w, rows + t * g.row_bytes + g.plane_lo[p], w);
        uint8_t *dst = g.base + seq * g.seq_stride + head * g.head_stride + p * g.span + t0 * w;
        HIP_TRY(hipMemcpyAsync(dst, stage.data(), (size_t)n * w, hipMemcpyHostToDevice, k->ctx->stream),
                "row load");
        HIP_TRY(hipStreamSynchronize(k->ctx->stream), "sync");
    }
    return INSITU_OK;
}

int insitu_read_image(insitu_cache *k, int32_t seq, uint8_t *img, int64_t nbytes) {
    if (!k || !img) return fail(INSITU_EINVAL, "null argument");
    if (seq < 0 || seq >= k->g.batch) return fail(INSITU_EINVAL, "no such sequence");
    if (nbytes != k->g.seq_stride) return fail(INSITU_EBADLEN, "image size must be seq_stride");
    HIP_TRY(hipSetDevice(k->ctx->device), "hipSetDevice");
    HIP_TRY(hipMemcpyAsync(img, k->g.base + seq * k->g.seq_stride, nbytes, hipMemcpyDeviceToHost,
                           k->ctx->stream),
            "image read");
    HIP_TRY(hipStreamSynchronize(k->ctx->stream), "sync");
    return INSITU_OK;
}

int insitu_load_image(insitu_cache *k, int32_t seq, const uint8_t *img, int64_t nbytes) {
    if (!k || !img) return fail(INSITU_EINVAL, "null argument");
    if (seq < 0 || seq >= k->g.batch) return fail(INSITU_EINVAL, "no such sequence");
    if (nbytes != k->g.seq_stride) return fail(INSITU_EBADLEN, "image size must be seq_stride");
    HIP_TRY(hipSetDevice(k->ctx->device), "hipSetDevice");
    HIP_TRY(hipMemcpyAsync(k->g.base + seq * k->g.seq_stride, img, nbytes, hipMemcpyHostToDevice,
                           k->ctx->stream),
            "image load");
    HIP_TRY(hipStreamSynchronize(k->ctx->stream), "sync");
    return INSITU_OK;
}

}  // extern "C"
