// Internal definitions shared by the HIP translation units of libinsitu_hip.
//
// Fixed-point constants follow config.py:214-254 of the reference
// (FixedFormat defaults). The kernels are written for that format; the
// cache constructor rejects any other one with INSITU_EINVAL rather than
// computing something subtly different.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/insitu.h"

namespace insitu {

constexpr int QK_FRAC = 16;       // Q8.16 seam values
constexpr int QK_WIDTH = 24;
constexpr int CENT_FRAC = 15;     // Q1.15 centroids
constexpr int ACC_FRAC = 16;
constexpr int ACC_WIDTH = 32;
constexpr int SCORE_WIDTH = 48;
constexpr int PROB_FRAC = 15;
constexpr int LUT_BITS = 8;
constexpr int MAX_INT_PART = PROB_FRAC + 1;                      // attention.py:113
constexpr int LUT_SPAN = (MAX_INT_PART + 1) << LUT_BITS;         // 4352, attention.py:129
constexpr int64_t LOG2E_Q16 = 94548;                             // round(log2(e) * 2^16)
constexpr int64_t SCORE_LO = -(int64_t(1) << (SCORE_WIDTH - 1));
constexpr int64_t SCORE_HI = (int64_t(1) << (SCORE_WIDTH - 1)) - 1;
constexpr int64_t ACC_LO = -(int64_t(1) << (ACC_WIDTH - 1));
constexpr int64_t ACC_HI = (int64_t(1) << (ACC_WIDTH - 1)) - 1;
constexpr int MAX_PLANES = 16;
constexpr int MAX_D = 128;
constexpr int MAX_G = 8;          // query heads per KV head handled by one block
constexpr int64_t Q_ROT_LIMIT = int64_t(1) << 27;  // |q_rot| bound that keeps scores exact

// Plane geometry of a cache: hw/ddr_layout.py:148-214, one region per sequence.
struct Geom {
    uint8_t *base;
    int64_t seq_stride, head_stride, span, capacity;
    int32_t n_planes;
    int32_t plane_lo[MAX_PLANES];
    int32_t plane_w[MAX_PLANES];
    int32_t row_bytes, key_bytes, value_bytes;   // norms follow the value field, 4 B
    int32_t d, kb, vb, norm_frac;
    int32_t n_kv, n_q, G, batch;
    // KV head h's planes are those of h >> kv_shift: an attend may see each KV head as
    // 2^kv_shift chains of G query heads (8 query heads a KV head as two chains of 4)
    int32_t kv_shift;
    // 0, or the query heads a KV head has when fewer than an attend's chains hold: chain
    // slot h then computes query head h % gq (the slots past gq duplicate, and are dropped)
    int32_t gq;
};

// Device-resident constants of a cache: codebooks and the exp table.
struct Tables {
    int64_t kc[256];     // key centroids, Q1.15
    int64_t kbnd[256];   // key boundaries
    int64_t vc[256];
    int64_t vbnd[256];
    int32_t exp_table[256];   // rint(2^(-i/256) * 2^15), attention.py:106-108
    int64_t delta_max;        // attention.py:145-146
    double kc_absmax;         // max |kc[i]|, for the exactness bound of the fp64 scores
    int32_t bnd_sorted;       // 1: both boundary lists non-decreasing (the encoder may bisect)
};

// The sign diagonals of up to two rotation rounds, one 64-bit word per 64 channels.
struct RotSigns {
    uint64_t s0a, s0b, s1a, s1b;
};

inline RotSigns rot_signs(int rounds, const uint64_t (*signs)[2]) {
    RotSigns sg;
    sg.s0a = rounds > 0 ? signs[0][0] : 0;
    sg.s0b = rounds > 0 ? signs[0][1] : 0;
    sg.s1a = rounds > 1 ? signs[1][0] : 0;
    sg.s1b = rounds > 1 ? signs[1][1] : 0;
    return sg;
}

// The fused decode step's inputs to the chunked attend: the wire rows (batch,
// heads, d) in Q8.16, the rotation, and the other half of the length double
// buffer, which receives len + 1.
struct StepIn {
    const int32_t *qw, *kw, *vw;
    RotSigns sg;
    int32_t rounds;
    int64_t *len_out;
};

// Device statistics; merged with atomics (AttentionStats.merge semantics).
struct DevStats {
    unsigned long long n_tokens;          // max
    unsigned long long rescale_events;    // sum
    unsigned long long score_overflows;   // sum
    unsigned long long acc_overflows;     // sum
    unsigned long long max_abs_score;     // max
    unsigned long long max_abs_acc;       // max
    unsigned long long range_errors;      // sum
    unsigned long long serial_fallbacks;  // sum
    unsigned long long fault;             // nonzero = internal error
};

// ---------------------------------------------------------------------------
// device helpers
// ---------------------------------------------------------------------------

__device__ __forceinline__ int64_t wmul(int64_t a, int64_t b) {
    return (int64_t)((uint64_t)a * (uint64_t)b);
}
__device__ __forceinline__ int64_t wadd(int64_t a, int64_t b) {
    return (int64_t)((uint64_t)a + (uint64_t)b);
}

// ExpLut.__call__ (attention.py:153-159) for delta >= 0: the flat index is
// floor(min(delta, delta_max) * log2e / 2^24); past the table it is zero.
// delta_max < 2^20, so after the clamp the product fits a 32x32->64 multiply.
// Branch-free: the table read is unconditional (index & 255 is always in
// range) and a select zeroes the past-the-table case, so the compiler can
// batch the LDS reads of several calls.
__device__ __forceinline__ int32_t exp_lut(int64_t delta, const int32_t *table, int64_t delta_max) {
    const uint32_t d = (uint32_t)(delta < delta_max ? delta : delta_max);
    const uint32_t u = (uint32_t)(((uint64_t)d * (uint64_t)LOG2E_Q16) >> (ACC_FRAC + ACC_FRAC - LUT_BITS));
    const int32_t v = table[u & 255] >> (u >> LUT_BITS);
    return u < (uint32_t)LUT_SPAN ? v : 0;
}

// reciprocal + _finalize for one row (attention.py:177-250, 873-880).
struct Recip {
    int64_t r;
    int32_t shift;
};
__device__ __forceinline__ Recip reciprocal(int64_t l) {
    int64_t s = 0;
    if (l >= 2) {
        s = 63 - __clzll((unsigned long long)l);
        if (s > 47) s = 47;
    }
    int64_t k = s - 31;
    int64_t ln = k >= 0 ? (l >> k) : (int64_t)((uint64_t)l << (-k));
    Recip out;
    out.r = 0;
    if (l > 0) {
        // floor(2^62 / ln) without a 64-bit integer division. ln lies in
        // [2^31, 2^48): it is exact in fp64 and the quotient is at most 2^31, so
        // the correctly rounded fp64 quotient truncates to the floor or to one
        // more (when the true quotient sits just below an integer); the integer
        // check r * ln <= 2^62 (no overflow: r * ln <= 2^62 + ln) settles it.
        const uint64_t n = (uint64_t)ln;
        uint64_t r = (uint64_t)(4611686018427387904.0 / (double)n);
        if (r * n > ((uint64_t)1 << 62)) --r;
        out.r = (int64_t)r;
    }
    out.shift = (int32_t)(62 - PROB_FRAC + k);
    return out;
}

__device__ __forceinline__ uint8_t *plane_ptr(const Geom &g, int b, int h, int p) {
    return g.base + (int64_t)b * g.seq_stride + (int64_t)(h >> g.kv_shift) * g.head_stride + (int64_t)p * g.span;
}

// Code of channel c in an LSB-first bitstream of `bits`-wide codes (quantize.py:271-283).
__device__ __forceinline__ int code_at(const uint8_t *field, int c, int bits) {
    int o = c * bits;
    int j = o >> 3, sh = o & 7;
    uint32_t v = field[j];
    if (sh + bits > 8) v |= (uint32_t)field[j + 1] << 8;
    return (int)((v >> sh) & ((1u << bits) - 1u));
}

__device__ __forceinline__ int64_t sext16(uint32_t v) {
    return (int64_t)(int16_t)(uint16_t)(v & 0xFFFFu);
}

}  // namespace insitu

// Host-side internal API between translation units.
namespace insitu {

struct LaunchErr {
    hipError_t e;
};

// The start/stop timing events of a launch sequence (null: untimed). They are
// attached to the dispatches themselves (hipExtLaunchKernelGGL), so timing
// adds no packets to the stream.
struct LaunchEv {
    hipEvent_t start = nullptr, stop = nullptr;
};

hipError_t launch_rotate(hipStream_t s, const int32_t *x, int32_t *y, int64_t n_vec, int d,
                         int rounds, const uint64_t (*signs)[2], unsigned long long *range_err);
hipError_t launch_encode(hipStream_t s, const int32_t *x, int64_t n_vec, int d, int norm_frac,
                         const int64_t *bounds_dev, int n_bounds, int32_t *norm, uint8_t *codes);
hipError_t launch_qtab(hipStream_t s, const int32_t *q, int n_heads, int d, const int64_t *c_dev,
                       int n_c, int64_t *table);
hipError_t launch_exp_lut(hipStream_t s, const Tables *t, const int64_t *delta, int64_t n,
                          int32_t *p);
hipError_t launch_finalize(hipStream_t s, const int64_t *acc, const int64_t *l, int rows, int d,
                           int64_t *out, int64_t *recip, int32_t *shift);
// Append n_tok rows of k/v ([seq][tok][kv head][d], int32) to sequences [seq_lo, seq_hi);
// rounds > 0 rotates them first (wire rows, rotate.py:170-197, `signs` as launch_rotate's).
hipError_t launch_append(hipStream_t s, const Geom &g, const Tables *t, const int32_t *k,
                         const int32_t *v, int n_tok, int seq_lo, int seq_hi, const int64_t *len_in,
                         int64_t *len_out, DevStats *st, int rounds = 0,
                         const uint64_t (*signs)[2] = nullptr, const Tables *host_tabs = nullptr);
bool chunked_supported(const Geom &g, int64_t capacity);
int64_t chunked_max_chunks(int64_t capacity);
int64_t chunked_pool_slots(int64_t max_chunks);
size_t chunked_scratch_bytes(const Geom &g, int64_t max_chunks, int64_t pool);
// The fp64 query staging in the chunked attend's scratch (query.h): the step's
// write kernel fills it, and the attend is then launched with q_staged;
// otherwise the attend stages the caller's rotated int32 rows itself. With
// step (sequential mode only), the attend is the whole decode step: len holds
// the lengths before it, q is unused and the wire rows come in step.
void chunked_query_area(const Geom &g, int64_t max_chunks, int64_t pool, void *scratch,
                        double **qd, int32_t **qok);
// Whether insitu_step runs as one fused launch in sequential mode (the
// register budget of the fused kernel allows it at d = 64).
bool chunked_fused_step(const Geom &g);
// A chunked attend's scratch: look-back words, chunk headers, run slots, the
// query staging. Its words carry the epoch of the attend that wrote them (the
// attend's number among the buffer's attends, 1 .. 2^14 - 1), so a word from an
// earlier attend reads as unpublished and nothing is reset between attends.
// Each buffer counts its own attends. spin_limit bounds every wait of the
// kernel on another workgroup (0: give up at once, which sends the chain to the
// exact serial path; a test hook).
// The per-chain completion counters are the only words that must read zero
// when an attend starts (its last workgroup puts them back to zero); when a
// launch lays the buffer out differently from the previous one (a prefill's
// chunk count follows its prompt), they are cleared first.
struct ChunkScratch {
    void *p = nullptr;
    size_t bytes = 0;
    uint32_t calls = 0;
    int32_t spin_limit = 1 << 20;
    uint64_t layout = 0;          // the carve of the last launch (0: none yet)
};
// The epoch of the next attend on the buffer. Every 2^14 - 1 attends the epoch
// wraps, and the whole buffer is cleared first (a fill kernel on the stream):
// a word written exactly that many attends ago would otherwise read as current.
// Call it before any work of the attend writes the buffer (the query staging of
// a two-launch step included).
hipError_t scratch_begin(hipStream_t s, ChunkScratch &cs, uint32_t *ep);
// A launch lays the buffer out as `layout` (a signature of its carve) with its
// epoch-checked words (look-back words, headers, completion counters) in the
// first `front` bytes: when the previous launch laid it out differently, those
// bytes are zeroed first (a fill kernel), since stale words of another layout
// could otherwise carry the current epoch by chance.
hipError_t scratch_layout(hipStream_t s, ChunkScratch &cs, uint64_t layout, size_t front);
// The scan attend (attend_scan.hip): sequential mode, 16 waves per 1,024-token
// chunk, queries staged per workgroup and read as scalar operands, the chain's
// last chunk replays. mc: chunks per sequence the scratch is laid out for (the
// capacity's); grid_chunks: chunks of the longest sequence of this launch.
bool scan_supported(const Geom &g, int64_t capacity);
int64_t scan_max_chunks(int64_t tokens);
size_t scan_scratch_bytes(const Geom &g, int64_t mc);
hipError_t launch_attend_scan(hipStream_t s, const Geom &g, const Tables *t, const int32_t *q, int32_t *out,
                              const int64_t *len, ChunkScratch &cs, uint32_t ep, int64_t mc, int64_t grid_chunks,
                              const StepIn *step, LaunchEv ev, DevStats *st);
// carve_batch: the sequences the scratch is laid out for (g.batch when 0); a
// launch over fewer sequences than its scratch holds passes the larger count.
hipError_t launch_attend_chunked(hipStream_t s, const Geom &g, const Tables *t, const int32_t *q,
                                 int32_t *out, const int64_t *len, ChunkScratch &cs,
                                 uint32_t ep, int64_t max_chunks, int64_t pool, int two_pass,
                                 bool q_staged, const StepIn *step, LaunchEv ev, DevStats *st,
                                 int64_t carve_batch = 0,
                                 int64_t grid_chunks = 0);
// The same entry points of the chunked attend built with 512-token chunks
// (attend_chunked.hip with INSITU_CHUNK_TPT=1). A cache uses one build for all
// its attends, so its scratch is laid out by that build's carve.
namespace c512 {
bool chunked_supported(const Geom &g, int64_t capacity);
int64_t chunked_max_chunks(int64_t capacity);
int64_t chunked_pool_slots(int64_t max_chunks);
size_t chunked_scratch_bytes(const Geom &g, int64_t max_chunks, int64_t pool);
void chunked_query_area(const Geom &g, int64_t max_chunks, int64_t pool, void *scratch,
                        double **qd, int32_t **qok);
hipError_t launch_attend_chunked(hipStream_t s, const Geom &g, const Tables *t, const int32_t *q,
                                 int32_t *out, const int64_t *len, ChunkScratch &cs,
                                 uint32_t ep, int64_t max_chunks, int64_t pool, int two_pass,
                                 bool q_staged, const StepIn *step, LaunchEv ev, DevStats *st,
                                 int64_t carve_batch = 0,
                                 int64_t grid_chunks = 0);
}  // namespace c512
// One chunk size's entry points, as a cache holds them.
struct ChunkedApi {
    int32_t tokens;   // tokens per chunk
    bool (*supported)(const Geom &, int64_t);
    int64_t (*max_chunks)(int64_t);
    int64_t (*pool_slots)(int64_t);
    size_t (*scratch_bytes)(const Geom &, int64_t, int64_t);
    void (*query_area)(const Geom &, int64_t, int64_t, void *, double **, int32_t **);
    hipError_t (*launch)(hipStream_t, const Geom &, const Tables *, const int32_t *, int32_t *,
                         const int64_t *, ChunkScratch &, uint32_t, int64_t, int64_t, int, bool,
                         const StepIn *, LaunchEv, DevStats *, int64_t, int64_t);
};
// The fused decode step's own kernel (attend_step.hip): sequential mode at d = 64, 4 query
// heads per KV head, 4-bit keys and 2-bit values, 1,024-token chunks of 16 waves. It lays the
// chunk scratch out its own way (scratch_layout clears the front when the layout changes).
// The scratch layouts' invariants, for a host-side test (insitu_debug_scratch_layout):
// f[0] chunks the layout is for, f[1] run slots per head (pool), f[2] slots per chunk after
// chunk 0, f[3] one past the last chunk's slots, f[4] runs the replay lists per head, f[5]
// most chunks per sequence, f[6] bytes, f[7] bytes of the epoch-checked front, f[8] 1 when
// every area is 256-aligned and ends before the next begins, f[9] tokens per chunk, f[10]
// the slot id limit (15 bits).
void chunked_layout_facts(const Geom &g, int64_t max_chunks, int64_t *f);
namespace c512 {
void chunked_layout_facts(const Geom &g, int64_t max_chunks, int64_t *f);
}
void step_layout_facts(const Geom &g, int64_t mc, int64_t *f);
bool step_supported(const Geom &g, int64_t capacity);
int64_t step_max_chunks(int64_t capacity);
size_t step_scratch_bytes(const Geom &g, int64_t mc);
hipError_t launch_step(hipStream_t s, const Geom &g, const Tables *t, int32_t *out, const int64_t *len,
                       ChunkScratch &cs, uint32_t ep, int64_t mc, int64_t grid_chunks, const StepIn &si,
                       LaunchEv ev, DevStats *st);
hipError_t launch_step_write(hipStream_t s, const Geom &g, const Tables *t, const int32_t *qw,
                             const int32_t *kw, const int32_t *vw, int rounds,
                             const uint64_t (*signs)[2], int32_t *qr, double *qd, int32_t *qok,
                             const int64_t *len_in, int64_t *len_out, DevStats *st);
hipError_t launch_attend_serial(hipStream_t s, const Geom &g, const Tables *t, const int32_t *q,
                                int32_t *out, const int64_t *len, int two_pass, LaunchEv ev,
                                DevStats *st);

// Shared with the files that add entry points beside abi.hip: the error
// message for insitu_last_error, and a context's device and stream.
int set_last_error(int code, const char *msg);
int ctx_device(insitu_ctx *c);
hipStream_t ctx_stream(insitu_ctx *c);
// The host half's rocBLAS handle, staging buffer and counters (host_half.hip): one
// set per context, made on first use on the context's device and stream, and
// released with the context.
void *&ctx_blas(insitu_ctx *c);
void blas_release(insitu_ctx *c);
// The start/stop events of the next timed launch (null events when timing is off).
int timing_events(insitu_ctx *c, LaunchEv *ev);

}  // namespace insitu
