// The fused decode step (kernel.py:271-345): rotate q/k/v, encode and append the
// token's k/v row, then attend_online (ops/attention.py:451-513) and the finalize
// (:873-880) over every cached row, bit-exact, in one launch of 16-wave workgroups,
// one per (1,024-token chunk, sequence, KV head) at d = 64, 4 query heads per KV head.
//
// The arithmetic is the chunked attend's (attend_chunked.hip): a chunk knows the
// running maximum before it (M_in, by a decoupled look-back over its predecessors'
// chunk maxima), so every token's p = LUT(m_t - s_t) and every rescale event
// (s_t > m_{t-1}, factor f = LUT(s_t - m_{t-1})) are known locally; between two
// events the terms floor(v_norm * p * c_v[code] / 2^23) only add, so the chunk
// hands over per query head one int32 sum per run and the factor opening it, and
//     acc = floor(acc * f / 2^15) + S,   l = floor(l * f / 2^15) + L
// replayed over the runs in order is the reference recurrence whenever the
// per-token int32 clamp never fires. That is certified per run from the exact acc
// where the run starts and B, the sum of its |term| bounds; a head that fails is
// recomputed token by token (serial_head.h).
//
// What this kernel does differently, so that the chain of dependent steps inside a
// workgroup stays short:
//   - 16 waves, one token per thread, 4 waves per SIMD to hide the plane loads;
//   - the group's rotated query rows are staged by the workgroup in global memory
//     and read back by scalar loads, entering the fp64 score FMAs as scalar
//     operands: the LDS then carries only the centroid reads;
//   - candidates, p, the factors and each token's term for every value code are
//     computed with lane = token for the 4 heads at once; the run sums are then
//     walked by every wave over its own 64 tokens (lane = channel) and merged by
//     LDS atomics into per-run accumulators (integer adds commute, and their
//     wrapping sum is exact whenever the result fits);
//   - a chunk publishes everything before it counts itself done, so the last
//     workgroup of a sequence's KV head reads all headers in one batch, stages the
//     runs' sums in LDS with all its waves, and walks them in blocks of 8.
// A sequence of one chunk (context <= 1,024) never publishes, counts or replays.
#include "query.h"
#include "row_codec.h"
#include "serial_head.h"
#include "wave.h"

#include <type_traits>

#ifdef INSITU_STEP_STAMPS
// Phase stamps (s_memrealtime) of every wave, for timing studies only, in a build
// that defines INSITU_STEP_STAMPS: [workgroup][wave][stamp], read back by the host.
__device__ unsigned long long insitu_step_stamps[8192 * 16 * 32];
extern "C" int insitu_step_stamps_read(unsigned long long *host, long n) {
    return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(insitu_step_stamps), (size_t)n * 8, 0, hipMemcpyDeviceToHost);
}
extern "C" int insitu_step_stamps_clear() {
    void *p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(insitu_step_stamps)) != hipSuccess) return 1;
    return (int)hipMemset(p, 0, sizeof(unsigned long long) * 8192 * 16 * 32);
}
// Each wave keeps its stamps in LDS (so that no global store enters the memory counters the
// kernel waits on) and writes them out once, where it ends (STAMP_FLUSH).
#define STAMP(k)                                                                                \
    do {                                                                                        \
        const unsigned long long _t = __builtin_amdgcn_s_memrealtime();                         \
        if ((threadIdx.x & 63) == 0) S.stamps[threadIdx.x >> 6][(k)] = _t;                      \
    } while (0)
// a count instead of a time, in slots 24 and up
#define STAMPV(k, v)                                                                            \
    do {                                                                                        \
        if ((threadIdx.x & 63) == 0) S.stamps[threadIdx.x >> 6][(k)] = (unsigned long long)(v); \
    } while (0)
#define STAMP_INIT()                                                                            \
    do {                                                                                        \
        if ((threadIdx.x & 63) < 32) S.stamps[threadIdx.x >> 6][threadIdx.x & 31] = 0;          \
    } while (0)
#define STAMP_FLUSH()                                                                           \
    do {                                                                                        \
        if ((threadIdx.x & 63) < 32 && blockIdx.x < 8192)                                       \
            insitu_step_stamps[((size_t)blockIdx.x * 16 + (threadIdx.x >> 6)) * 32 + (threadIdx.x & 31)] = \
                S.stamps[threadIdx.x >> 6][threadIdx.x & 31];                                   \
    } while (0)
#else
#define STAMPV(k, v) \
    do {             \
    } while (0)
#define STAMP_INIT() \
    do {             \
    } while (0)
#define STAMP_FLUSH() \
    do {              \
    } while (0)
#define STAMP(k) \
    do {         \
    } while (0)
#endif

namespace insitu {
namespace stepk {

constexpr int NT = 1024;          // threads per workgroup: 16 waves, 4 per SIMD
constexpr int NW = NT / 64;
constexpr int CHUNK = NT;         // tokens per workgroup, one per thread
constexpr int D = 64;
constexpr int G = GF;             // query heads per KV head
constexpr int RMAX = 32;          // runs per head a chunk sums in LDS
constexpr int RPB = 64;           // runs per head the replay loads in one round trip (lane = run)
constexpr int SLOTS = 16;         // runs per head a chunk after chunk 0 publishes
constexpr int HMAX = 512;         // chunks per sequence
constexpr int NSEG = 2048;        // runs per head the replay lists
constexpr int LPOOL = 256;        // chunk 0's candidate list (every head): at most this many
constexpr uint16_t RUN_EVENT = 0x8000;
static_assert(1 + (HMAX - 1) * SLOTS + 1 < RUN_EVENT, "run slots fit 15 bits");
// Per-head flags in a chunk header: the head is recomputed serially.
constexpr int FL_POOL = 1;        // more runs than the chunk can hold
constexpr int FL_LB = 2;          // a look-back gave up waiting
constexpr int FL_Q = 4;           // the query rows fail the fp64 exactness bound
constexpr int FL_CERT = 8;        // chunk 0's own clamp certificate failed
// Look-back words: flag (bits 62-63) | call epoch (bits 48-61) | score - SCORE_LO.
constexpr unsigned long long ST_AGG = 1ull << 62, ST_INC = 2ull << 62, ST_FLAGS = 3ull << 62;
constexpr unsigned EPOCH_MASK = (1u << 14) - 1u;
constexpr double MAGIC = 6755399441055744.0;   // 1.5 * 2^52
constexpr int64_t MAGIC_BITS = 0x4338000000000000LL;

__device__ __forceinline__ void pub64(void *p, uint64_t v) {
    __hip_atomic_store((uint64_t *)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void pub32(void *p, uint32_t v) {
    __hip_atomic_store((uint32_t *)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t get64(const void *p) {
    return __hip_atomic_load((uint64_t *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t get32(const void *p) {
    return __hip_atomic_load((uint32_t *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Wait until this thread's stores (the relaxed atomics above, and plain stores) have completed.
__device__ __forceinline__ void stores_done() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_s_waitcnt(0x0F70);          // vmcnt(0)
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
__device__ __forceinline__ unsigned long long st_pack(unsigned long long flag, unsigned ep, int64_t v) {
    return flag | (unsigned long long)ep << 48 | (unsigned long long)(v - SCORE_LO);
}
__device__ __forceinline__ unsigned long long st_flag(unsigned long long w, unsigned ep) {
    return ((unsigned)(w >> 48) & EPOCH_MASK) == ep ? w & ST_FLAGS : 0ull;
}
__device__ __forceinline__ int64_t st_val(unsigned long long w) {
    return (int64_t)(w & ((1ull << 48) - 1)) + SCORE_LO;
}
__device__ __forceinline__ int64_t dbl_to_i64(double x) {
    // x is an integer with |x| <= 2^51: adding 1.5 * 2^52 puts it in the low mantissa bits.
    return (int64_t)__double_as_longlong(x + MAGIC) - MAGIC_BITS;
}
// |acc| + B <= 2^31 - 1: no prefix sum of a run whose |terms| sum to at most B can
// take acc out of int32 (B >= 0).
__device__ __forceinline__ bool fits(int32_t acc, int64_t bound) {
    const int64_t a = acc < 0 ? -(int64_t)acc : (int64_t)acc;
    return a + bound <= ACC_HI;
}
struct OpOr64 {
    __device__ static int64_t f(int64_t a, int64_t b) { return a | b; }
};
__host__ __device__ __forceinline__ int slot_base(int chunk) { return chunk == 0 ? 0 : 1 + (chunk - 1) * SLOTS; }

// Chunk scratch: look-back words, headers, counters and chunk 0's tagged state first (the
// epoch-checked front, zeroed when a launch lays the buffer out differently), then the runs.
struct Sck {
    unsigned long long *status;   // [chain][G][2][mc]: inclusive, aggregate
    uint64_t *hdr;                // [chain][mc][G][2]: w0, w1
    unsigned int *done;           // [chain]: chunks done with their runs
    uint64_t *st0;                // [chain][G][D + 1]: chunk 0's state, each word tagged with the
                                  // epoch (<< 48): acc (lane = channel), then l | events << 26
    uint64_t *meta;               // [chain][G][pool][2]: L | f << 32, B
    int32_t *segS;                // [chain][G][pool][D]
    int32_t mc, pool;
    uint32_t ep;                  // this call's epoch, 1 .. 2^14 - 1
    int32_t spin_limit;
};

template <int KB, int VB>
struct StepLds {
    static constexpr int NV = 1 << VB;
    static constexpr int VWORDS = D * VB / 32;
    static constexpr int RS = (D * KB / 8 + D * VB / 8 + 4 + 3) / 4 * 4;
    // the small tables first: their reads then take the LDS address from an immediate offset
    double kcd[256][2];                     // a key-code byte's two centroids (low nibble first)
    int32_t vc9[8];                         // the value centroids << 9 (|c| < 2^18)
    int32_t expt[256];
    union {
        struct {
            union {
                int4 tt[CHUNK][NV];         // each token's term for every value code, the 4 heads
                // the chunk's list: (score - SCORE_LO) | token << 48 and v_norm, head h at
                // [loff[h], ...); per head its tokens of weight: p | f << 16, the bound of its
                // term | event << 31 (bounds lie below 2^25), its term
                // floor(v_norm * p * c_v[c] / 2^23) for each value code c, and its value codes
                struct {
                    uint64_t e[LPOOL];
                    int32_t vn[LPOOL];
                    uint32_t ipf[G][LPOOL], ib[G][LPOOL];
                    int4 it4[G][LPOOL];
                    uint32_t iw[G][LPOOL][VWORDS];
                } ol;
            } tu;
            uint32_t vw[CHUNK][VWORDS];     // each token's value codes
            uint32_t rix[CHUNK];            // each token's run, a byte per head
            uint16_t clist[CHUNK];          // the chunk's candidates (any head) in token order
        } ph;
        struct {
            uint16_t rl[G][NSEG];           // the runs of chunks 1.. in order: slot | RUN_EVENT
            uint64_t rlf[G][RMAX], rbb[G][RMAX];
            int32_t rs[G][RMAX][D];         // their sums, RMAX runs per head at a time
        } rp;
        struct {
            uint16_t rl_[G][NSEG];          // (the replay's list, left intact: no barrier between)
            SerialLds<RS> fb[G];            // the serial path, per head
        } sr;
    } u;
    int32_t runS[G][RMAX][D];               // run sums; the replay's staged runs
    unsigned long long runB[G][RMAX];
    uint32_t runL[G][RMAX];
    int32_t runf[G][RMAX];
    int32_t qi[G][D];                       // the rotated query rows (the score, the serial path)
    uint8_t codes[2][MAX_D];                // the new token's key and value codes
    uint32_t nk[D * 4 / 32 + 1], nv[D * 2 / 32 + 1], nn;   // the new row: key words, value words, norms
    int64_t wmax[NW][G];
    int64_t wt[G][NW];
    int32_t evc[G][NW];
    int32_t ccnt[NW];                       // candidates per wave
    int32_t lcnt[G][NW];                    // chunk 0's list: candidates per head and wave
    int32_t onseg[G];                       // chunk 0's list: segments per head
    int64_t min_[G], lmax[G];
    int32_t total[G];
    int qbad[G];
    int sbad[G];                            // a replay slot index past the pool (a fault)
    int lbfail, last;
    unsigned long long ovf, mabs;
    unsigned long long sev, samax;          // the chain's merged statistics (replay)
    int32_t sdone;
    int32_t hfin;                           // head waves done with the finalize
#ifdef INSITU_STEP_STAMPS
    unsigned long long stamps[NW][32];      // each wave's phase stamps (timing studies only)
#endif
};

// Applies a chunk's runs 0 .. nr - 1 of head h (its LDS run accumulators; run r > 0 opens
// with a rescale by its factor) to the state (acc, l), lane = channel. A rescale never grows
// |acc| (|floor(acc * f / 2^15)| <= |acc| for 0 <= f <= 2^15), so |acc| + the sum of the runs'
// bounds B certifies every run at once; then only the rescales and adds remain, eight runs'
// sums read at a time. Returns false (nothing applied) when the bound does not certify them,
// and the caller goes run by run.
template <class L>
__device__ __forceinline__ bool fold_runs_certified(const L &S, int h, int nr, int lane, int32_t &acc, int64_t &l) {
    constexpr int RM = sizeof(S.runL[0]) / sizeof(S.runL[0][0]);
    const bool in = lane < nr && lane < RM;
    const uint32_t Lr = in ? S.runL[h][lane] : 0u;
    const int32_t fr = in ? S.runf[h][lane] : 0;
    const int64_t bsum = wave_sum_i64(in ? (int64_t)S.runB[h][lane] : 0);
    const int64_t a = acc < 0 ? -(int64_t)acc : (int64_t)acc;
    if (__ballot(a + bsum > ACC_HI)) return false;
    for (int r0 = 0; r0 < nr; r0 += 8) {
        int32_t v[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = r0 + k < nr ? S.runS[h][r0 + k][lane] : 0;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            if (r0 + k < nr) {
                if (r0 + k > 0) {
                    const int64_t f = __builtin_amdgcn_readlane(fr, r0 + k);
                    acc = (int32_t)(((int64_t)acc * f) >> PROB_FRAC);
                    l = (l * f) >> PROB_FRAC;
                }
                acc += v[k];
                l += (uint32_t)__builtin_amdgcn_readlane((int)Lr, r0 + k);
            }
        }
    }
    return true;
}

template <int KB, int VB>
__global__ void __launch_bounds__(NT, 1) step_kernel(Geom g, const Tables *__restrict__ tabs, int32_t *out,
                                                     const int64_t *__restrict__ len, Sck ck, DevStats *st,
                                                     StepIn si) {
    using L = StepLds<KB, VB>;
    constexpr int NV = 1 << VB, NK = 1 << KB;
    constexpr int KWORDS = D * KB / 32, VWORDS = D * VB / 32;
    constexpr int KBYTES = D * KB / 8;
    constexpr int NFULL = KBYTES / 16, HALF = (KBYTES % 16) / 8;
    constexpr int KPL = NFULL + HALF;         // key planes; the value plane follows, then the norms
    static_assert(VB == 1 || VB == 2, "one value plane of 8 or 16 bytes");
    static_assert(KB == 4, "the score's channel slices take 8 codes a word, 2 planes a row");
    static_assert(32 % KB == 0 && 32 % VB == 0, "the new row's codes never straddle a word");
    static_assert(KWORDS <= D * 4 / 32 && VWORDS <= D * 2 / 32, "new-row staging sizes");
    __shared__ L S;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n_chains = g.batch * g.n_kv;
    // chunk-major: every predecessor of a chunk has a smaller workgroup number
    const int chunk = (int)(blockIdx.x / (unsigned)n_chains);
    const int chain = (int)(blockIdx.x % (unsigned)n_chains);
    const int b = chain / g.n_kv, kvh = chain % g.n_kv;
    const int64_t T = len[b] + 1;
    const int nch = (int)((T + CHUNK - 1) / CHUNK);
    if (chunk >= nch) return;
    STAMP_INIT();
    STAMP(0);
    const bool newrow = chunk == nch - 1;     // this chunk holds the step's new token
    const int64_t t0 = (int64_t)chunk * CHUNK;
    const int tln = (int)(T - 1 - t0);
    const bool live = t0 + tid < T;
    const bool fresh = newrow && tid == tln;
    const bool own = chunk == 0;
    // The score's waves: a chunk of ntw token waves (lane = token) splits its channels over
    // sp = 16 / ntw waves when it has few tokens (sp a power of two): wave wv scores channel
    // slice wv / ntw of token wave wv % ntw; slice 0 is the token wave itself, which adds the
    // other slices' partial sums (exact: integers below 2^51 in fp64).
    const int ntok = (int)(T - t0 < CHUNK ? T - t0 : CHUNK);
    const int ntw = (ntok + 63) >> 6;
    const int sp = ntw > 8 ? 1 : ntw > 4 ? 2 : ntw > 2 ? 4 : ntw > 1 ? 8 : 16;
    const bool scorer = wv < ntw * sp;
    const int slice = wv / ntw, tw = wv - slice * ntw;
    const int cps = D / sp;                   // channels per slice
    const int hidx = 64 * tw + lane;          // a helper's token, within the chunk
    const bool hlive = slice > 0 && scorer && t0 + hidx < T;
    const bool hfresh = hlive && newrow && hidx == tln;
    // A wave with no token of the chunk skips the per-token work (its reductions and scans
    // would only take issue slots from the waves that share its SIMD) and leaves neutral
    // entries in LDS; it still takes every barrier and its share of the walk.
    const bool wlive = t0 + 64 * wv < T;
    if (own && kvh == 0 && tid == 0) si.len_out[b] = T;
    const int score_shift = CENT_FRAC + g.norm_frac;
    const uint8_t *hb = plane_ptr(g, b, kvh, 0);

    // -- P0: loads, rotations, the new row ---------------------------------------
    // The small loads first (wire rows, tables), then the chunk's planes: the vector
    // memory counter drains in order, so the rotations wait only for their rows.
    // The loads of P0 go out in order: the wire row (unconditional: a wave that needs none
    // reads one it ignores), the new row's boundaries (their waves wait for them where the
    // paths join, before their planes go out), the score's table, the planes. A wait for a
    // later load waits for every earlier one.
    const int32_t *xsrc = wv < G ? si.qw + ((int64_t)b * g.n_q + kvh * G + wv) * D
                                 : (wv == G + 1 ? si.vw : si.kw) + ((int64_t)b * g.n_kv + kvh) * D;
    const int32_t xv = xsrc[lane];
    // the new token's encoder: lane i < 2^bits - 1 of wave G (keys) and G + 1 (values) holds
    // boundary i (quantize.py:183-196)
    int64_t bl = 0;
    if (newrow && wv == G && lane < NK - 1)
        bl = tabs->kbnd[lane];
    else if (newrow && wv == G + 1 && lane < NV - 1)
        bl = tabs->vbnd[lane];
    const double kc_absmax = tabs->kc_absmax;
    // The score's table by code byte (two channels' key centroids in one LDS read), loaded by
    // waves past the head waves, whose one load before the rotation is their query row.
    const int64_t kp0 = tabs->kc[tid & 15], kp1 = tabs->kc[(tid >> 4) & 15];   // used by tid 512 .. 767
    __builtin_amdgcn_sched_barrier(0);          // (these before the planes: see above)
    uint32_t kw[KWORDS + 1];
    uint32_t vwd[VWORDS];
    uint32_t nw = 0;
#pragma unroll
    for (int i = 0; i <= KWORDS; ++i) kw[i] = 0;
#pragma unroll
    for (int i = 0; i < VWORDS; ++i) vwd[i] = 0;
    // Wave w's planes (key words, value words, norm word) into (k, v, n): the row of its
    // token wave's token (a helper picks its slice's words after barrier B1).
    auto load_planes = [&](int w, uint32_t(&k)[KWORDS + 1], uint32_t(&v)[VWORDS], uint32_t &n)
        __attribute__((always_inline)) {
        const int tww = w % ntw;
        // Every lane loads, with no branch: a lane past the context reads the chunk's row t0
        // (its values are never used: the score, the list and the walk take live tokens only,
        // a helper's partial sums go to dead lanes), and the step's new token is replaced by
        // its row from LDS after barrier B1. (Lanes that returned early, and a helper path of
        // its own, made the compiler join the paths with copies of the loaded registers, so
        // that every wave waited for its planes before B1.)
        const int lt = 64 * tww + lane;
        const int64_t t = t0 + lt < T ? t0 + lt : t0;
#pragma unroll
        for (int p = 0; p < NFULL; ++p) {
            const uint4 x = *(const uint4 *)(hb + p * g.span + t * 16);
            k[4 * p] = x.x;
            k[4 * p + 1] = x.y;
            k[4 * p + 2] = x.z;
            k[4 * p + 3] = x.w;
        }
        if (HALF) {
            const uint2 x = *(const uint2 *)(hb + NFULL * g.span + t * 8);
            k[4 * NFULL] = x.x;
            k[4 * NFULL + 1] = x.y;
        }
        if (VB == 2) {
            const uint4 x = *(const uint4 *)(hb + KPL * g.span + t * 16);
            v[0] = x.x;
            v[1] = x.y;
            v[2 % VWORDS] = x.z;
            v[3 % VWORDS] = x.w;
        } else {
            const uint2 x = *(const uint2 *)(hb + KPL * g.span + t * 8);
            v[0] = x.x;
            v[1 % VWORDS] = x.y;
        }
        n = *(const uint32_t *)(hb + (KPL + 1) * g.span + t * 4);
    };
    // Every wave's planes, right after its wire row: the loads are unconditional, so that a
    // rotation waits for its row alone (the vector memory counter drains in order), and no
    // wave waits for its planes before barrier B1. (Loaded for the head waves by waves 4-7 and
    // handed over in LDS, or branching per lane, B1 waited for the planes.)
    load_planes(wv, kw, vwd, nw);
    // zero the run accumulators (LDS atomics add into them)
    for (int i = tid; i < G * RMAX * D; i += NT) (&S.runS[0][0][0])[i] = 0;
    if (tid < G * RMAX) {
        (&S.runB[0][0])[tid] = 0;
        (&S.runL[0][0])[tid] = 0;
        (&S.runf[0][0])[tid] = 0;
    }
    if (tid < G) S.sbad[tid] = 0;
    if (tid == 0) {
        S.ovf = S.mabs = 0;
        S.lbfail = 0;
        S.sev = S.samax = 0;
        S.sdone = 0;
        S.hfin = 0;
    }
    if (tid >= 512 && tid < 512 + 256) {
        S.kcd[tid - 512][0] = (double)kp0;          // |centroid| < 2^18: exact
        S.kcd[tid - 512][1] = (double)kp1;
    }
    if (wv < G) {
        // Chunk 0 counts the queries' range errors, once per call: values beyond int32
        // after the rotation, and rotated values beyond the 24-bit seam's +-2^27.
        int32_t r[1];
        const int32_t in[1] = {xv};
        rotate_loaded<1>(in, D, si.rounds, si.sg, r, own ? &st->range_errors : nullptr);
        // The rotated row, for every wave's score (which reads it from LDS after the barrier)
        // and the serial path. Scores stay exact fp64 integers when ||q||_1 * max|c| < 2^51
        // (attention.py:333-359 computes them in int64); rotated values beyond the 24-bit
        // seam's +-2^27 count as range errors.
        S.qi[wv][lane] = r[0];
        const int64_t xq = r[0];
        const uint32_t aq = (uint32_t)(xq < 0 ? -xq : xq);  // <= 2^31
        // ||q||_1 from the sums of |q|'s 16-bit halves (each below 2^22 over 64 lanes)
        const uint32_t halves[2] = {aq >> 16, aq & 0xFFFFu};
        uint32_t hs[2];
        wave_sum_u32_n<2>(halves, hs);
        const int64_t l1 = (int64_t)hs[0] * 65536 + hs[1];   // < 2^38: exact as a double below
        const int bad = __popcll(__ballot(aq >= (uint32_t)Q_ROT_LIMIT));
        if (own && lane == 0 && bad) atomicAdd(&st->range_errors, (unsigned long long)bad);
        const bool okh = (double)l1 * kc_absmax < DOT_LIMIT;
        if (lane == 0) S.qbad[wv] = okh ? 0 : 1;
    } else if (newrow && wv < G + 2) {
        // the new token: rotate, norm, codes (quantize.py:164-212), pack (:237-252), store
        const int f = wv - G;      // 0: key, 1: value
        int32_t r[1];
        const int32_t in[1] = {xv};
        rotate_loaded<1>(in, D, si.rounds, si.sg, r, &st->range_errors);
        const int64_t x[1] = {r[0]};
        const int64_t n = norm_wire<1>(x, D, g.norm_frac);
        // code = #{i : (x << 8) > norm * b_i}, the products norm * b_i broadcast from their lanes
        const int64_t xs = x[0] << (CENT_FRAC + g.norm_frac - QK_FRAC);
        const int64_t thr = n * bl;
        const int nb = f == 0 ? NK - 1 : NV - 1;
        int code = 0;
#pragma unroll
        for (int i = 0; i < NK - 1; ++i)
            if (i < nb) code += xs > readlane64(thr, i) ? 1 : 0;
        // Pack: a word holds 32 / bits consecutive codes, LSB first (quantize.py:271-289): each
        // lane shifts its code into place, an OR over its group of lanes (lane xor 1, 2, ...)
        // gives the word in every lane of the group, and the group's first lane stores it.
        const int bits = f == 0 ? KB : VB;
        const int per = 32 / bits;                                  // codes per word
        uint32_t wword = (uint32_t)code << (bits * (lane & (per - 1)));
        wword |= xor_lane32<1>(wword, lane);
        wword |= xor_lane32<2>(wword, lane);
        if (per > 4) wword |= xor_lane32<4>(wword, lane);
        if (per > 8) wword |= xor_lane32<8>(wword, lane);
        if (per > 16) wword |= xor_lane32<16>(wword, lane);
        const int wi = lane / per;                                  // the word of the field
        uint8_t *const rowb = plane_ptr(g, b, kvh, 0);            // writable
        uint16_t *nword = (uint16_t *)(rowb + (KPL + 1) * g.span + (T - 1) * 4);
        if ((lane & (per - 1)) == 0) {
            if (f == 0) {
                // key word wi: plane wi / 4, word wi % 4 of the token's 16 bytes (8 in a half plane)
                const int pw = wi / 4 < NFULL ? 16 : 8;
                pub32(rowb + (wi / 4) * g.span + (T - 1) * pw + 4 * (wi % 4), wword);
                S.nk[wi] = wword;
            } else {
                pub32(rowb + KPL * g.span + (T - 1) * (VWORDS * 4) + 4 * wi, wword);
                S.nv[wi] = wword;
            }
        }
        if (lane == 0) {
            __hip_atomic_store(nword + f, (uint16_t)(n & 0xFFFF), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            ((uint16_t *)&S.nn)[f] = (uint16_t)(n & 0xFFFF);
        }
    }
    STAMP(1);
    __syncthreads();                                               // B1
    STAMP(2);
    const bool ok = !(S.qbad[0] | S.qbad[1] | S.qbad[2] | S.qbad[3]);
    // the value centroids and the exp table, first read after barrier B2: requested here and
    // stored before B2, so that neither barrier waits for them
    int64_t tab = 0;
    int32_t ex = 0;
    if (tid >= 320 && tid < 320 + NV) tab = tabs->vc[tid - 320];
    if (tid >= 384 && tid < 384 + 256) ex = tabs->exp_table[tid - 384];
    if (slice > 0) {
        // a helper's slice of its token's key words: word w0 on (uniform selects over the row)
        const int w0 = cps >= 8 ? slice * cps / 8 : slice / 2;
        // x[i] = word (w0 + i) mod KWORDS, with constant register indices only (a runtime index
        // into kw would put the array in scratch memory)
        uint32_t x[4] = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int j = 0; j < KWORDS; ++j) {
            const int d = (j - w0) & (KWORDS - 1);
#pragma unroll
            for (int i = 0; i < 4; ++i) x[i] = d == i ? kw[j] : x[i];
        }
        kw[0] = x[0] >> (cps >= 8 ? 0 : 16 * (slice & 1));
#pragma unroll
        for (int i = 1; i < 4; ++i) kw[i] = x[i];
    }
    if (fresh) {
#pragma unroll
        for (int i = 0; i < KWORDS; ++i) kw[i] = S.nk[i];
#pragma unroll
        for (int i = 0; i < VWORDS; ++i) vwd[i] = S.nv[i];
        nw = S.nn;
    }
    if (hfresh) {
        const int w0 = cps >= 8 ? slice * cps / 8 : slice / 2;
        const uint32_t x = S.nk[w0];
        kw[0] = x >> (cps >= 8 ? 0 : 16 * (slice & 1));
#pragma unroll
        for (int i = 1; i < 4; ++i) kw[i] = S.nk[(w0 + i) & (KWORDS - 1)];
    }

    // -- P1: scores (attention.py:333-359), lane = token, the 4 heads at once ------
    // sum_ch q[ch] * c[code_ch] in fp64 FMA is exact: every partial sum is an integer
    // below 2^51 (the query check). Then the int64 norm multiply, >> 24, clamp to 48 bits.
    int64_t s[G];
#pragma unroll
    for (int h = 0; h < G; ++h) s[h] = SCORE_LO;
    unsigned long long ovf = 0;
    int64_t mabs = 0;
    double acc[G];
#pragma unroll
    for (int h = 0; h < G; ++h) acc[h] = 0.0;
    // The loop for NS steps of two channels. The query values come from VGPRs by row broadcast:
    // register j holds, in every row of 16 lanes, channels 4j .. 4j + 3 (of this slice) of the 4
    // heads, lane 4 c + h: channel 4j + c of head h, and the FMA's DPP operand row_newbcast:n
    // hands lane n of the row to all 16 (the same value in every row, so in every lane). The
    // centroids of a step's two channels come from one LDS read, by the token's code byte.
    auto score_steps = [&](auto ns) __attribute__((always_inline)) {
        constexpr int NS = decltype(ns)::value;
        constexpr int NQ = NS / 2;                                  // query registers
        static_assert(KB == 4, "the score reads two 4-bit codes' centroids by code byte");
        double(&ac)[G] = acc;
        int32_t qi[NQ];
        {
            const int qh = lane & 3, qc = (lane >> 2) & 3;
#pragma unroll
            for (int j = 0; j < NQ; ++j) qi[j] = S.qi[qh][slice * cps + 4 * j + qc];
        }
#pragma unroll
        for (int j = 0; j < NQ; ++j) {
            // steps 2j and 2j + 1: channels 4j .. 4j + 3, centroids by code bytes 2j and 2j + 1
            const uint32_t w = kw[j >> 1];
            const uint32_t b0 = __builtin_amdgcn_ubfe(w, (uint32_t)(16 * (j & 1)), 8u);
            const uint32_t b1 = __builtin_amdgcn_ubfe(w, (uint32_t)(16 * (j & 1) + 8), 8u);
            const double c0 = S.kcd[b0][0], c1 = S.kcd[b0][1], c2 = S.kcd[b1][0], c3 = S.kcd[b1][1];
            double qd;
            // The conversion writes the DPP operand: two wait states (s_nop 1) before its first
            // DPP read, which the compiler cannot see inside the asm.
            asm("v_cvt_f64_i32 %4, %5\n\t"
                "s_nop 1\n\t"
                "v_fmac_f64_dpp %0, %4, %6 row_newbcast:0 row_mask:0xf bank_mask:0xf\n\t"
                "v_fmac_f64_dpp %1, %4, %6 row_newbcast:1 row_mask:0xf bank_mask:0xf\n\t"
                "v_fmac_f64_dpp %2, %4, %6 row_newbcast:2 row_mask:0xf bank_mask:0xf\n\t"
                "v_fmac_f64_dpp %3, %4, %6 row_newbcast:3 row_mask:0xf bank_mask:0xf\n\t"
                "v_fmac_f64_dpp %0, %4, %7 row_newbcast:4 row_mask:0xf bank_mask:0xf\n\t"
                "v_fmac_f64_dpp %1, %4, %7 row_newbcast:5 row_mask:0xf bank_mask:0xf\n\t"
                "v_fmac_f64_dpp %2, %4, %7 row_newbcast:6 row_mask:0xf bank_mask:0xf\n\t"
                "v_fmac_f64_dpp %3, %4, %7 row_newbcast:7 row_mask:0xf bank_mask:0xf\n\t"
                "v_fmac_f64_dpp %0, %4, %8 row_newbcast:8 row_mask:0xf bank_mask:0xf\n\t"
                "v_fmac_f64_dpp %1, %4, %8 row_newbcast:9 row_mask:0xf bank_mask:0xf\n\t"
                "v_fmac_f64_dpp %2, %4, %8 row_newbcast:10 row_mask:0xf bank_mask:0xf\n\t"
                "v_fmac_f64_dpp %3, %4, %8 row_newbcast:11 row_mask:0xf bank_mask:0xf\n\t"
                "v_fmac_f64_dpp %0, %4, %9 row_newbcast:12 row_mask:0xf bank_mask:0xf\n\t"
                "v_fmac_f64_dpp %1, %4, %9 row_newbcast:13 row_mask:0xf bank_mask:0xf\n\t"
                "v_fmac_f64_dpp %2, %4, %9 row_newbcast:14 row_mask:0xf bank_mask:0xf\n\t"
                "v_fmac_f64_dpp %3, %4, %9 row_newbcast:15 row_mask:0xf bank_mask:0xf"
                : "+v"(ac[0]), "+v"(ac[1]), "+v"(ac[2]), "+v"(ac[3]), "=&v"(qd)
                : "v"(qi[j]), "v"(c0), "v"(c1), "v"(c2), "v"(c3));
        }
    };
    if (ok && scorer) {
        switch (sp) {
        case 1: score_steps(std::integral_constant<int, 32>{}); break;
        case 2: score_steps(std::integral_constant<int, 16>{}); break;
        case 4: score_steps(std::integral_constant<int, 8>{}); break;
        case 8: score_steps(std::integral_constant<int, 4>{}); break;
        default: score_steps(std::integral_constant<int, 2>{}); break;
        }
    }
    STAMP(22);
    if (sp > 1) {
        // the slices' partial sums to their token wave, through the (not yet used) tt area
        double *part = (double *)&S.u.ph.tu.tt[0][0];
        if (ok && scorer && slice > 0) {
#pragma unroll
            for (int h = 0; h < G; ++h) part[(((slice - 1) * ntw + tw) * G + h) * 64 + lane] = acc[h];
        }
        __syncthreads();
        if (ok && slice == 0 && scorer) {
            for (int j = 1; j < sp; ++j) {
#pragma unroll
                for (int h = 0; h < G; ++h) acc[h] += part[(((j - 1) * ntw + tw) * G + h) * 64 + lane];
            }
        }
    }
    if (ok && slice == 0 && scorer) {
        if (live) {
            const int64_t kn = sext16(nw);
            // (acc kn) >> score_shift in fp64: acc * (kn / 2^shift) is exact while |acc kn| <
            // 2^53, and a computed |product| below 2^(53 - shift) proves it (rounding never
            // crosses the power of two); floor is then the arithmetic shift. A lane past the
            // bound takes the int64 product, which wraps as the reference's does.
            const double kns = (double)kn * __builtin_ldexp(1.0, -score_shift);
            const double lim = __builtin_ldexp(1.0, 53 - score_shift);
            double pr[G];
            bool fast = true;
#pragma unroll
            for (int h = 0; h < G; ++h) {
                pr[h] = acc[h] * kns;
                fast = fast && fabs(pr[h]) < lim;
            }
            if (fast) {
                double am = 0.0;
#pragma unroll
                for (int h = 0; h < G; ++h) {
                    const double f = floor(pr[h]);
                    const double v = fmax(fmin(f, (double)SCORE_HI), (double)SCORE_LO);
                    ovf += f != v ? 1 : 0;
                    am = fmax(am, fabs(v));
                    s[h] = dbl_to_i64(v);                          // |v| <= 2^47
                }
                mabs = dbl_to_i64(am);
            } else {
#pragma unroll
                for (int h = 0; h < G; ++h) {
                    int64_t v = wmul(dbl_to_i64(acc[h]), kn) >> score_shift;
                    if (v < SCORE_LO || v > SCORE_HI) {
                        ++ovf;
                        v = v < SCORE_LO ? SCORE_LO : SCORE_HI;
                    }
                    const int64_t a = v < 0 ? -v : v;
                    mabs = a > mabs ? a : mabs;
                    s[h] = v;
                }
            }
        }
    }
#pragma unroll
    for (int i = 0; i < VWORDS; ++i) S.u.ph.vw[tid][i] = vwd[i];
    // the wave's maxima (scores lie in [SCORE_LO, SCORE_HI], within +-2^47: 32-bit steps),
    // its overflow count (at most 4 a lane: three ballots) and its largest |score|
    // (the 4 heads' maxima and the largest |score| - 2^47 reduced together)
    int64_t wm[G + 1], mv[G + 1];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        wm[h] = SCORE_LO;
        mv[h] = s[h];
    }
    wm[G] = 0;
    mv[G] = mabs - (int64_t(1) << 47);
    static_assert(G + 1 == 5, "the 4 heads' maxima and max |score| reduce as 5 values");
    if (wlive) wave_max_s48_x5(mv, wm);
    if (lane == 0) {
#pragma unroll
        for (int h = 0; h < G; ++h) S.wmax[wv][h] = wm[h];
    }
    if (ok && wlive) {
        ovf = (unsigned long long)(__popcll(__ballot(ovf & 1)) + 2 * __popcll(__ballot(ovf & 2)) +
                                   4 * __popcll(__ballot(ovf & 4)));
        mabs = wm[G] + (int64_t(1) << 47);                      // |score| <= 2^47
        if (lane == 0) {
            if (ovf) atomicAdd(&S.ovf, ovf);
            if (mabs) atomicMax(&S.mabs, (unsigned long long)mabs);
        }
    }
    if (tid >= 320 && tid < 320 + NV) S.vc9[tid - 320] = (int32_t)tab * 512;   // |centroid| < 2^18
    if (tid >= 384 && tid < 384 + 256) S.expt[tid - 384] = ex;
    STAMP(3);
    __syncthreads();                                               // B2
    STAMP(4);

    // This chunk's maxima go out first (wave G + h: head h's aggregate; chunk 0: its inclusive
    // maximum), and wave h issues the look-back's first poll (the nearest 64 predecessors'
    // words), whose round trip the list test's scans below then overlap.
    int64_t local0 = SCORE_LO;
    unsigned long long pw1 = 0, pw2 = 0;
    if (ok && wv < 2 * G && nch > 1) {
        const int h = wv & (G - 1);
        unsigned long long *wi0 = ck.status + ((int64_t)chain * G + h) * 2 * ck.mc;
        if (wv >= G) {
            local0 = wave_max_i64(lane < NW ? S.wmax[lane & (NW - 1)][h] : SCORE_LO);
            if (lane == 0)
                __hip_atomic_store((own ? wi0 : wi0 + ck.mc) + chunk, st_pack(own ? ST_INC : ST_AGG, ck.ep, local0),
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else if (!own && (int64_t)chunk - 1 - lane >= 0) {
            pw1 = __hip_atomic_load(wi0 + chunk - 1 - lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            pw2 = __hip_atomic_load(wi0 + ck.mc + chunk - 1 - lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    // The list test's half that needs no M_in (its 32-bit running maxima), done here so that
    // it overlaps the look-back's wait: k32[h] holds the tokens with floor(s / 2^16) >= hi -
    // ceil(delta_max / 2^16), hi the running maximum of floor(s / 2^16) up to the token.
    const int64_t dmh = (tabs->delta_max + 65535) >> 16;
    uint64_t k32[G];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        uint32_t wmx = lane < NW ? (uint32_t)(int32_t)(S.wmax[lane & (NW - 1)][h] >> 16) : 0x80000000u;
        wmx = (uint32_t)max((int32_t)wmx, (int32_t)dpp32<DPP_ROW_SHR1>(0x80000000u, wmx));
        wmx = (uint32_t)max((int32_t)wmx, (int32_t)dpp32<DPP_ROW_SHR2>(0x80000000u, wmx));
        wmx = (uint32_t)max((int32_t)wmx, (int32_t)dpp32<DPP_ROW_SHR4>(0x80000000u, wmx));
        wmx = (uint32_t)max((int32_t)wmx, (int32_t)dpp32<DPP_ROW_SHR8>(0x80000000u, wmx));
        const int32_t before = wv ? __builtin_amdgcn_readlane((int)wmx, wv - 1) : INT32_MIN;
        const int32_t hs = (int32_t)(s[h] >> 16);         // scores lie in [-2^47, 2^47)
        const int32_t hi = max(wave_scan_max32(hs), before);
        k32[h] = __ballot(ok && live && (int64_t)hs + dmh >= (int64_t)hi);
    }

    // -- P2: the maximum before this chunk, by look-back --------------------------
    // Two words per (chunk, head): the inclusive maximum and this chunk's own
    // (aggregate). Wave G + h publishes head h's aggregate (chunk 0: its inclusive
    // maximum) while wave h looks back, so that the polling wave has no store in
    // flight. A sequence of one chunk needs neither. The query check fails alike in
    // every chunk of a sequence, and then nothing is scored or waited for.
    if (ok && wv < 2 * G) {
        const int h = wv & (G - 1);
        // the chunk's maximum: lanes 0..15 hold the waves' maxima
        const int64_t local = wave_max_i64(lane < NW ? S.wmax[lane & (NW - 1)][h] : SCORE_LO);
        int64_t run = SCORE_LO;
        if (nch > 1) {
            unsigned long long *wi0 = ck.status + ((int64_t)chain * G + h) * 2 * ck.mc;
            unsigned long long *wa0 = wi0 + ck.mc;
            if (wv >= G) {
                // (published above)
            } else if (!own) {
                int64_t base = chunk - 1;       // the predecessor lane 0 reads
                int spins = 0;
                bool fail = ck.spin_limit == 0;
                bool first = true;              // the first poll's words were loaded above
                while (!fail) {
                    const int64_t pc = base - lane;
                    unsigned long long flag = ST_INC;
                    int64_t val = SCORE_LO;
                    if (pc >= 0) {
                        const unsigned long long w1 =
                            first ? pw1 : __hip_atomic_load(wi0 + pc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        const unsigned long long w2 =
                            first ? pw2 : __hip_atomic_load(wa0 + pc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        const bool has_inc = st_flag(w1, ck.ep) == ST_INC;
                        flag = has_inc ? ST_INC : st_flag(w2, ck.ep);
                        val = st_val(has_inc ? w1 : w2);
                    }
                    first = false;
                    const unsigned long long inc = __ballot(flag == ST_INC);
                    const int nearest = inc ? __ffsll((long long)inc) - 1 : 64;
                    const unsigned long long wait = __ballot(flag == 0 && lane <= nearest);
                    if (wait) {
                        if (++spins > ck.spin_limit) {
                            fail = true;
                            break;
                        }
                        __builtin_amdgcn_s_sleep(2);
                        continue;
                    }
                    const int64_t v = wave_max_i64(lane <= nearest ? val : SCORE_LO);
                    run = v > run ? v : run;
                    if (nearest < 64) break;
                    base -= 64;
                }
                const int64_t incl = run > local ? run : local;
                if (lane == 0)
                    __hip_atomic_store(wi0 + chunk, st_pack(ST_INC, ck.ep, incl), __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
                if (fail && lane == 0) S.lbfail = 1;
            }
        }
        if (wv < G && lane == 0) {
            S.min_[h] = run;
            S.lmax[h] = local;
        }
    }
    __syncthreads();                                               // B3
    STAMP(5);
    const bool lbfail = S.lbfail != 0;
    int flags = (ok ? 0 : FL_Q) | (lbfail ? FL_LB : 0);
    int32_t acc0 = 0;
    int64_t l0 = 0;
    int nev0 = 0;
    const int64_t dm = tabs->delta_max;
    // u = floor(min(d, delta_max) * log2e / 2^24) (attention.py:153-159), then the table
    auto lut = [&](int64_t d) __attribute__((always_inline)) {
        const uint32_t dc = (uint32_t)(d < dm ? d : dm);                     // < 2^20
        const uint32_t u = __umulhi(dc << 8, (uint32_t)LOG2E_Q16);
        const int32_t v = S.expt[u & 255] >> (u >> LUT_BITS);
        return u < (uint32_t)LUT_SPAN ? v : 0;
    };

    // -- P3 from a list of the chunk's candidates -------------------------------------
    // A token of weight or an event has s > m_t - delta_max, m_t its running maximum, which is
    // at least M_in and at least the chunk's own running maximum. The chunk lists the tokens
    // that pass both tests (a superset; the second in 32-bit steps: with hi the running
    // maximum of floor(s / 2^16) up to the token, s > m - delta_max implies floor(s / 2^16) >=
    // hi - ceil(delta_max / 2^16)). When they fit LPOOL, per head one pass over the list (lane
    // = entry) gives every listed token its running maximum (the larger of M_in and the listed
    // scores before it: every event is listed), hence its event, p and factor
    // (ops/attention.py:451-513 over the listed tokens is the recurrence over all: the others
    // add nothing), and the head's wave then walks its tokens of weight in order (lane =
    // channel): chunk 0 folds them into its state (a rescale at an event, then the term of this
    // lane's code, certified by one bound: a rescale never grows |acc|), the other chunks cut
    // them into runs at their events. The lane-per-token phases below, which scan every token,
    // remain for a chunk whose list does not fit (a flat softmax).
    uint64_t evb[G], cb[G];
    uint64_t candb = 0;
    int rb[G];
    int nruns[G];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        evb[h] = cb[h] = 0;
        rb[h] = 0;
        nruns[h] = 1;
    }
    const bool replayer = chunk == nch - 1;      // the sequence's last chunk replays the others
    bool olist = false;
    if (ok && !lbfail) {
        uint64_t lb[G];
#pragma unroll
        for (int h = 0; h < G; ++h) {
            lb[h] = k32[h] & __ballot(s[h] > S.min_[h] - dm);
            if (lane == 0) S.lcnt[h][wv] = (int32_t)__popcll(lb[h]);
        }
        STAMP(17);
        __syncthreads();                                           // L1
        STAMP(18);
        int lnum[G], loff[G], lwoff[G], lsum = 0;
#pragma unroll
        for (int h = 0; h < G; ++h) {
            uint32_t c = lane < NW ? (uint32_t)S.lcnt[h][lane & (NW - 1)] : 0u;
            c += dpp32<DPP_ROW_SHR1>(0u, c);
            c += dpp32<DPP_ROW_SHR2>(0u, c);
            c += dpp32<DPP_ROW_SHR4>(0u, c);
            c += dpp32<DPP_ROW_SHR8>(0u, c);
            lnum[h] = __builtin_amdgcn_readlane((int)c, NW - 1);
            lwoff[h] = wv ? __builtin_amdgcn_readlane((int)c, wv - 1) : 0;
            loff[h] = lsum;
            lsum += lnum[h];
        }
        olist = lsum <= LPOOL;
        if (olist) {
            auto &ol = S.u.ph.tu.ol;
#pragma unroll
            for (int h = 0; h < G; ++h) {
                if ((lb[h] >> lane) & 1ull) {
                    const int at = loff[h] + lwoff[h] +
                                   (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(lb[h] >> 32),
                                                                  __builtin_amdgcn_mbcnt_lo((uint32_t)lb[h], 0u));
                    ol.e[at] = (uint64_t)(s[h] - SCORE_LO) | ((uint64_t)tid << 48);
                    ol.vn[at] = (int32_t)(int16_t)(nw >> 16);
                }
            }
            STAMP(19);
            __syncthreads();                                       // L2
            STAMP(21);
            if (wv < G) {
                // Head h's wave alone (the heads' waves sit on the four SIMDs): one pass over the
                // list gives the tokens of weight, their four terms and the bound B, then the
                // fold walks them in order: a rescale at an event, then the term of this lane's
                // code. |acc| + the sum of B certifies every step (a rescale never grows |acc|).
                const int h = wv, n = lnum[h], o = loff[h];
                int32_t vcs[4];
#pragma unroll
                for (int c = 0; c < 4; ++c) vcs[c] = uni32(S.vc9[c < L::NV ? c : 0]);
                uint32_t vcmax9 = 0;
#pragma unroll
                for (int c = 0; c < L::NV; ++c) {
                    const uint32_t a = (uint32_t)(vcs[c] < 0 ? -vcs[c] : vcs[c]);
                    vcmax9 = a > vcmax9 ? a : vcmax9;
                }
                int64_t smax = S.min_[h];                          // M_in
                int nitem = 0, nev = 0;
                uint64_t bsum = 0;
                for (int j0 = 0; j0 < n; j0 += 64) {
                    const int j = j0 + lane;
                    const bool in = j < n;
                    const uint64_t e = in ? ol.e[o + j] : 0ull;
                    const int64_t sc = in ? (int64_t)(e & ((1ull << 48) - 1)) + SCORE_LO : SCORE_LO;
                    const int64_t inc = wave_scan64<OpMax64>(sc, SCORE_LO);
                    int64_t mb = wave_shr1_64(inc, SCORE_LO);
                    mb = mb > smax ? mb : smax;                    // the running maximum before
                    smax = OpMax64::f(smax, readlane64(inc, 63));
                    const bool ev = in && sc > mb;
                    const int32_t p = in ? lut(ev ? 0 : mb - sc) : 0;
                    const int32_t f = ev ? lut(sc - mb) : 0;
                    const bool useful = in && (ev || p > 0);
                    const uint64_t ub = __ballot(useful);
                    const int32_t w = useful ? ol.vn[o + j] * p : 0;          // |w| <= 2^30
                    const uint32_t aw = (uint32_t)(w < 0 ? -w : w);
                    bsum += (uint32_t)__builtin_amdgcn_readlane(
                        (int)wave_scan_add32(w != 0 ? __umulhi(aw, vcmax9) + 1 : 0u), 63);   // < 2^31
                    if (useful) {
                        const int ipos = nitem + (int)__builtin_amdgcn_mbcnt_hi(
                                                     (uint32_t)(ub >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)ub, 0u));
                        const int tk = (int)(e >> 48) & (CHUNK - 1);
                        ol.ipf[h][ipos] = ev ? 0x80000000u | (uint32_t)f : (uint32_t)p;
                        ol.ib[h][ipos] = w != 0 ? __umulhi(aw, vcmax9) + 1 : 0u;
                        ol.it4[h][ipos] = make_int4(__mulhi(w, vcs[0]), __mulhi(w, vcs[1]), __mulhi(w, vcs[2]),
                                                    __mulhi(w, vcs[3]));
#pragma unroll
                        for (int k = 0; k < L::VWORDS; ++k) ol.iw[h][ipos][k] = S.u.ph.vw[tk][k];
                    }
                    nitem += (int)__popcll(ub);
                    nev += (int)__popcll(__ballot(ev));
                }
                // up to a multiple of 8 with tokens that change nothing (no event, p 0, terms and
                // bound 0): the walks below then take whole batches of 8 with no mask
                if (nitem + lane < ((nitem + 7) & ~7)) {
                    ol.ipf[h][nitem + lane] = 0u;
                    ol.ib[h][nitem + lane] = 0u;
                    ol.it4[h][nitem + lane] = make_int4(0, 0, 0, 0);
                }
                STAMP(20);
                STAMPV(24, n);
                STAMPV(25, nitem);
                STAMPV(26, nev);
                const int wsel = (lane * VB) >> 5, wsh = (lane * VB) & 31;
                const uint32_t pev = (uint32_t)uni32(S.expt[0]);   // an event's p: LUT(0)
                // The walk, lane = channel, 8 tokens at a time: every value the 8 need (event | f
                // or p, the bound, the four terms, this lane's value-code word) is read from the
                // list by position, all loads issued before the first is used.
                uint32_t pfv[8], ibv[8], wd[8];
                int4 t4[8];
                auto batch = [&](int i0, bool bounds) __attribute__((always_inline)) {
#pragma unroll
                    for (int q = 0; q < 8; ++q) {
                        const int i = (i0 + q) & (LPOOL - 1);
                        pfv[q] = ol.ipf[h][i];
                        if (bounds) ibv[q] = ol.ib[h][i];
                        t4[q] = ol.it4[h][i];
                        wd[q] = ol.iw[h][i][wsel];
                    }
                    __builtin_amdgcn_sched_barrier(0);     // every load issued before any use
                };
                auto term = [&](int q) __attribute__((always_inline)) {
                    const uint32_t code = __builtin_amdgcn_ubfe(wd[q], (uint32_t)wsh, (uint32_t)VB);
                    const int32_t t01 = code & 1 ? t4[q].y : t4[q].x, t23 = code & 1 ? t4[q].w : t4[q].z;
                    return code & 2 ? t23 : t01;
                };
                if (!own) {
                    // runs: run r holds the tokens from the chunk's r-th event on (run 0: those
                    // before its first), with its sum, L, bound and opening factor
                    int r = 0;
                    int32_t sacc = 0;
                    uint32_t sL = 0;
                    uint64_t sB = 0;
                    for (int i0 = 0; i0 < nitem; i0 += 8) {
                        batch(i0, true);
                        uint32_t any = 0;
#pragma unroll
                        for (int q = 0; q < 8; ++q) any |= pfv[q];
                        if (!((uint32_t)uni32((int32_t)any) >> 31)) {
                            // no event among them: one tree of adds (int32: the same bits in any order)
                            int32_t t[8];
#pragma unroll
                            for (int q = 0; q < 8; ++q) t[q] = term(q);
                            sacc += ((t[0] + t[1]) + (t[2] + t[3])) + ((t[4] + t[5]) + (t[6] + t[7]));
#pragma unroll
                            for (int q = 0; q < 8; ++q) {
                                sL += (uint32_t)uni32((int32_t)pfv[q]);
                                sB += (uint32_t)uni32((int32_t)ibv[q]);
                            }
                            continue;
                        }
#pragma unroll
                        for (int q = 0; q < 8; ++q) {
                            const uint32_t pw = (uint32_t)uni32((int32_t)pfv[q]);
                            const uint32_t bq = (uint32_t)uni32((int32_t)ibv[q]);
                            if (pw >> 31) {
                                if (r < RMAX) {
                                    S.runS[h][r][lane] = sacc;
                                    if (lane == 0) {
                                        S.runL[h][r] = sL;
                                        S.runB[h][r] = sB;
                                    }
                                }
                                ++r;
                                if (r < RMAX && lane == 0) S.runf[h][r] = (int32_t)(pw & 0xFFFF);
                                sacc = 0;
                                sL = 0;
                                sB = 0;
                            }
                            sacc += term(q);
                            sL += pw >> 31 ? pev : pw;
                            sB += bq;
                        }
                    }
                    if (r < RMAX) {
                        S.runS[h][r][lane] = sacc;
                        if (lane == 0) {
                            S.runL[h][r] = sL;
                            S.runB[h][r] = sB;
                        }
                    }
                    nruns[h] = r + 1;
                    if (r + 1 > RMAX || (!replayer && r + 1 > SLOTS)) flags |= FL_POOL;
                } else if (bsum > (uint64_t)ACC_HI) {
                    nev0 = nev;
                    flags |= FL_CERT;
                } else {
                    nev0 = nev;
                    // Chunk 0's events are dense (its running maximum starts low), so every token
                    // takes the same steps, with no branch: a factor of 2^15 where there is no
                    // event (floor(acc * 2^15 / 2^15) = acc). The batch's factors, p and terms
                    // first (none depends on acc), then the chain of rescales and adds alone, so
                    // that the in-order wave does not stall on them token by token.
                    for (int i0 = 0; i0 < nitem; i0 += 8) {
                        batch(i0, false);
                        int64_t fq[8];
                        uint32_t pq[8];
                        int32_t tq[8];
#pragma unroll
                        for (int q = 0; q < 8; ++q) {
                            const uint32_t pw = (uint32_t)uni32((int32_t)pfv[q]);
                            const bool ev = (pw >> 31) != 0;
                            fq[q] = ev ? (int64_t)(pw & 0xFFFF) : (int64_t)1 << PROB_FRAC;
                            pq[q] = ev ? pev : pw;
                            tq[q] = term(q);
                        }
                        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                        for (int q = 0; q < 8; ++q) {
                            acc0 = (int32_t)(((int64_t)acc0 * fq[q]) >> PROB_FRAC) + tq[q];
                            l0 = ((l0 * fq[q]) >> PROB_FRAC) + pq[q];
                        }
                    }
                }
            }
        }
    }
    const bool work = ok && !lbfail && !olist;     // the lane-per-token phases
    if (olist) STAMP(16);

    // -- P3: events, p, factors and terms, lane = token --------------------------
    // A head whose chunk maximum does not exceed M_in has no event here, and then
    // every token's running maximum is M_in. Otherwise the running maximum comes from
    // a block-wide prefix-max scan. A token at or below m - delta_max has p = 0; the
    // others are candidates, and only waves that hold one do the rest: each
    // candidate's terms floor(v_norm * p * c_v[c] / 2^23) for every value code c go to
    // LDS; run r of a head is the tokens from its r-th event of the chunk on (run 0:
    // before the first), and its L = sum p, its bound B = sum ((|w| * max|c_v|) >> 23) + 1
    // over w = v_norm * p != 0, and its opening factor go to the run accumulators.
    // The reference's int64 floors are taken as 32-bit high products: for |a * b| < 2^63,
    // floor(a * b / 2^k) = mulhi(a, b * 2^(32 - k)) whenever b * 2^(32 - k) fits 32 bits.
    if (work) {
        int64_t Min[G], incl[G];
        bool evh[G];
        bool any_ev = false;
#pragma unroll
        for (int h = 0; h < G; ++h) {
            Min[h] = S.min_[h];
            evh[h] = S.lmax[h] > Min[h];
            any_ev = any_ev || evh[h];
            incl[h] = SCORE_LO;
            if (evh[h]) {
                if (wlive) incl[h] = wave_scan64<OpMax64>(s[h], SCORE_LO);
                if (lane == 63) S.wt[h][wv] = incl[h];
            }
        }
        if (any_ev) __syncthreads();                               // B4 (uniform)
        STAMP(11);
        int64_t pm[G], dd[G];
        bool ev[G], cand[G];
#pragma unroll
        for (int h = 0; h < G; ++h) {
            pm[h] = Min[h];
            ev[h] = cand[h] = false;
            dd[h] = 0;
            if (!wlive) continue;
            if (evh[h]) {
                // the maxima of the waves before this one: lanes 0..15 hold the waves' maxima,
                // a 16-lane inclusive max-scan, read at wave - 1
                int64_t wmx = lane < NW ? S.wt[h][lane & (NW - 1)] : SCORE_LO;
                wmx = OpMax64::f(wmx, dpp64<DPP_ROW_SHR1>(SCORE_LO, wmx));
                wmx = OpMax64::f(wmx, dpp64<DPP_ROW_SHR2>(SCORE_LO, wmx));
                wmx = OpMax64::f(wmx, dpp64<DPP_ROW_SHR4>(SCORE_LO, wmx));
                wmx = OpMax64::f(wmx, dpp64<DPP_ROW_SHR8>(SCORE_LO, wmx));
                const int64_t before = wv ? readlane64(wmx, wv - 1) : SCORE_LO;
                pm[h] = before > pm[h] ? before : pm[h];
                const int64_t ex1 = wave_shr1_64(incl[h], SCORE_LO);
                pm[h] = ex1 > pm[h] ? ex1 : pm[h];
            }
            ev[h] = evh[h] && live && s[h] > pm[h];
            dd[h] = (ev[h] ? s[h] : pm[h]) - s[h];                   // m - s >= 0; 0 at an event
            cand[h] = live && dd[h] < dm;
            evb[h] = __ballot(ev[h]);
            cb[h] = __ballot(cand[h]);
            candb |= cb[h];
        }
        int32_t pv[G], fv[G], bw[G];
#pragma unroll
        for (int h = 0; h < G; ++h) pv[h] = fv[h] = bw[h] = 0;
        if (candb) {
            const int32_t vn = (int32_t)(int16_t)(nw >> 16);
            uint32_t vcmax9 = 0;
#pragma unroll
            for (int c = 0; c < NV; ++c) {
                const uint32_t a = (uint32_t)(S.vc9[c] < 0 ? -S.vc9[c] : S.vc9[c]);
                vcmax9 = a > vcmax9 ? a : vcmax9;
            }
            int32_t tv[NV][G];
#pragma unroll
            for (int h = 0; h < G; ++h) {
#pragma unroll
                for (int c = 0; c < NV; ++c) tv[c][h] = 0;
                if (!cb[h]) continue;
                const int32_t p = cand[h] ? lut(dd[h]) : 0;           // LUT(0) = 2^15 at an event
                const int32_t w = vn * p;                              // |w| <= 2^30
                const uint32_t aw = (uint32_t)(w < 0 ? -w : w);
                pv[h] = p;
                // (|w| * max|c_v|) >> 23 < 2^25; the term floor(w * c / 2^23) < 2^25 in magnitude
                bw[h] = w != 0 ? (int32_t)__umulhi(aw, vcmax9) + 1 : 0;
#pragma unroll
                for (int c = 0; c < NV; ++c) tv[c][h] = __mulhi(w, S.vc9[c]);
                if (evb[h]) fv[h] = ev[h] ? lut(s[h] - pm[h]) : 0;
            }
            if ((candb >> lane) & 1ull) {
#pragma unroll
                for (int c = 0; c < NV; ++c) S.u.ph.tu.tt[tid][c] = make_int4(tv[c][0], tv[c][1], tv[c][2], tv[c][3]);
            }
        }
        if (any_ev) {
            if (lane == 0) {
#pragma unroll
                for (int h = 0; h < G; ++h) S.evc[h][wv] = (int32_t)__popcll(evb[h]);
            }
            __syncthreads();                                       // B5 (uniform)
            STAMP(13);
            // the events of the waves before this one, and of all: lanes 0..15 hold the waves'
            // counts, a 16-lane prefix sum read at wave - 1 and at 15
#pragma unroll
            for (int h = 0; h < G; ++h) {
                if (!evh[h]) continue;
                uint32_t c = lane < NW ? (uint32_t)S.evc[h][lane & (NW - 1)] : 0u;
                c += dpp32<DPP_ROW_SHR1>(0u, c);
                c += dpp32<DPP_ROW_SHR2>(0u, c);
                c += dpp32<DPP_ROW_SHR4>(0u, c);
                c += dpp32<DPP_ROW_SHR8>(0u, c);
                rb[h] = wv ? __builtin_amdgcn_readlane((int)c, wv - 1) : 0;
                nruns[h] = 1 + __builtin_amdgcn_readlane((int)c, NW - 1);
            }
        }
        // Per-run L and B: the wave's tokens lie in run rb[h] up to its first event, then in
        // one run per event. Lane prefix sums (p <= 2^15 and a term bound < 2^25, so 64 of
        // them fit 32 bits) give every segment's sums: the segment's last lane adds its
        // inclusive sum less the one before the segment's first lane into its run. Each
        // candidate also records its run for the walk, a byte per head (runs < RMAX count).
        const uint64_t le = lane == 63 ? ~0ull : (2ull << lane) - 1ull;       // lanes 0 .. lane
        uint32_t rix = 0;
#pragma unroll
        for (int h = 0; h < G; ++h) {
            const uint64_t mine = evb[h] & le;                     // events at or before this lane
            const int ri = rb[h] + (int)__popcll(mine);           // this lane's run
            rix |= (uint32_t)(ri < 255 ? ri : 255) << (8 * h);
            if (!cb[h]) continue;
            const uint32_t sl = wave_scan_add32((uint32_t)pv[h]);
            const uint32_t sb = wave_scan_add32((uint32_t)bw[h]);
            const int first = mine ? 63 - __clzll((long long)mine) : 0;   // the first lane of its segment
            const bool last = lane == 63 || ((evb[h] >> (lane + 1)) & 1ull);
            const uint32_t pl = (uint32_t)__builtin_amdgcn_ds_bpermute(4 * (first - 1), (int)sl);
            const uint32_t pb = (uint32_t)__builtin_amdgcn_ds_bpermute(4 * (first - 1), (int)sb);
            const uint32_t L = sl - (first ? pl : 0u), B = sb - (first ? pb : 0u);
            if (last && ri < RMAX && (L || B)) {
                atomicAdd(&S.runL[h][ri], L);
                atomicAdd(&S.runB[h][ri], (unsigned long long)B);
            }
            if (((evb[h] >> lane) & 1ull) && ri < RMAX) S.runf[h][ri] = fv[h];   // the factor opening run ri
        }
        if ((candb >> lane) & 1ull) S.u.ph.rix[tid] = rix;
    }
    // The chunk's candidates listed in token order (16-lane prefix sum of the waves' counts):
    // the walk then gives every wave an equal share, wherever the candidates crowd. (work is
    // uniform in the workgroup: a chunk that took the list path passes none of these barriers.)
    int n_all = 0;
    if (work) {
        if (lane == 0) S.ccnt[wv] = (int32_t)__popcll(candb);
        __syncthreads();                                           // B6 (uniform)
        uint32_t c = lane < NW ? (uint32_t)S.ccnt[lane & (NW - 1)] : 0u;
        c += dpp32<DPP_ROW_SHR1>(0u, c);
        c += dpp32<DPP_ROW_SHR2>(0u, c);
        c += dpp32<DPP_ROW_SHR4>(0u, c);
        c += dpp32<DPP_ROW_SHR8>(0u, c);
        n_all = __builtin_amdgcn_readlane((int)c, NW - 1);
        const int off = wv ? __builtin_amdgcn_readlane((int)c, wv - 1) : 0;
        if ((candb >> lane) & 1ull) {
            const int at = off + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(candb >> 32),
                                                                __builtin_amdgcn_mbcnt_lo((uint32_t)candb, 0u));
            S.u.ph.clist[at] = (uint16_t)tid;
        }
        __syncthreads();                                           // B6b (uniform)
    }
    STAMP(6);

    // -- P4: run sums, lane = channel ---------------------------------------------
    // Wave w walks candidates [w n / 16, (w + 1) n / 16) of the list in order, for the 4
    // heads at once, 8 at a time: the tokens' value words, then the terms their codes of
    // this lane's channel pick, then the adds; where a head's run changes (at its events,
    // and at the wave's first candidate) the partial sum goes to that run's accumulator with
    // an LDS atomic add.
    const int i0 = (int)((int64_t)wv * n_all / NW), i1 = (int)((int64_t)(wv + 1) * n_all / NW);
    if (work && i1 > i0) {
        const int myn = i1 - i0;                                   // <= 64: n_all <= 1,024
        const uint32_t tokl = lane < myn ? (uint32_t)S.u.ph.clist[i0 + lane] : 0u;
        const uint32_t rixl = S.u.ph.rix[tokl];
        int32_t P[G];
#pragma unroll
        for (int h = 0; h < G; ++h) P[h] = 0;
        uint32_t cur = (uint32_t)__builtin_amdgcn_readlane((int)rixl, 0);   // the open run of each head
        const int wi = (lane * VB) >> 5, sh = (lane * VB) & 31;
        for (int k0 = 0; k0 < myn; k0 += 8) {
            const int nt = myn - k0 < 8 ? myn - k0 : 8;
            int tk[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) tk[k] = __builtin_amdgcn_readlane((int)tokl, k0 + (k < nt ? k : 0));
            uint32_t wd[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) wd[k] = S.u.ph.vw[tk[k]][wi];
            int4 t4[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) t4[k] = S.u.ph.tu.tt[tk[k]][__builtin_amdgcn_ubfe(wd[k], (uint32_t)sh, (uint32_t)VB)];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                if (k < nt) {
                    const uint32_t rx = (uint32_t)__builtin_amdgcn_readlane((int)rixl, k0 + k);
                    if (rx != cur) {
#pragma unroll
                        for (int h = 0; h < G; ++h) {
                            const uint32_t ro = (cur >> (8 * h)) & 255u, rn = (rx >> (8 * h)) & 255u;
                            if (ro != rn) {
                                if (ro < RMAX && P[h]) atomicAdd(&S.runS[h][ro][lane], P[h]);
                                P[h] = 0;
                            }
                        }
                        cur = rx;
                    }
                    P[0] += t4[k].x;
                    P[1] += t4[k].y;
                    P[2] += t4[k].z;
                    P[3] += t4[k].w;
                }
            }
        }
#pragma unroll
        for (int h = 0; h < G; ++h) {
            const uint32_t ro = (cur >> (8 * h)) & 255u;
            if (ro < RMAX && P[h]) atomicAdd(&S.runS[h][ro][lane], P[h]);
        }
    }
    if (work) __syncthreads();                                     // B7 (uniform)
    STAMP(7);

    // -- P5: chunk 0 folds its runs; the others publish theirs ---------------------
    const bool hw = wv < G;        // wave h < G: query head h, lane = channel
    const int h = hw ? wv : 0;
    // The last chunk of the sequence replays (it holds the new token, and its look-back is the
    // longest); every other chunk publishes its runs (chunk 0: its state), waits until they
    // are complete, then publishes its header, and is done. The replayer's runs stay in LDS.
    if (hw && work) {
        const int nr = nruns[h];
        if (nr > RMAX || (!own && !replayer && nr > SLOTS)) flags |= FL_POOL;
        if (own && !(flags & FL_POOL) && fold_runs_certified(S, h, nr, lane, acc0, l0)) {
            nev0 = nr - 1;
        } else if (own && !(flags & FL_POOL)) {
            // acc = floor(acc * f / 2^15) + S per run (run 0 has no rescale), each run certified
            bool unsafe = false;
            for (int r = 0; r < nr; ++r) {
                if (r > 0) {
                    const int64_t f = S.runf[h][r];
                    acc0 = (int32_t)(((int64_t)acc0 * f) >> PROB_FRAC);
                    l0 = (l0 * f) >> PROB_FRAC;
                }
                if (!fits(acc0, (int64_t)S.runB[h][r])) unsafe = true;
                acc0 += S.runS[h][r][lane];
                l0 += S.runL[h][r];
            }
            if (__ballot(unsafe)) flags |= FL_CERT;
            nev0 = nr - 1;
        }
    }
    if (!replayer) {
        if (hw) {
            uint64_t *hp = ck.hdr + (((int64_t)chain * ck.mc + chunk) * G + h) * 2;
            const int64_t hbase = ((int64_t)chain * G + h) * ck.pool;
            int npub = 0;
            if (own) {
                // the state, each word tagged with the epoch: the replayer polls the words
                // themselves, so they need no wait before the header (l < 2^26: at most 1,024
                // values of p <= 2^15; events <= 1,024)
                uint64_t *s0 = ck.st0 + ((int64_t)chain * G + h) * (D + 1);
                const uint64_t tag = (uint64_t)ck.ep << 48;
                pub64(&s0[lane], (uint64_t)(uint32_t)acc0 | tag);
                if (lane == 0) pub64(&s0[D], ((uint64_t)l0 & ((1ull << 26) - 1)) | ((uint64_t)nev0 << 26) | tag);
            } else if ((work || olist) && !(flags & FL_POOL)) {
                const int nr = nruns[h];
                const bool empty = nr == 1 && S.runL[h][0] == 0 && S.runB[h][0] == 0;
                npub = empty ? 0 : nr;
                for (int r = 0; r < npub; ++r) {
                    const int64_t slot = hbase + slot_base(chunk) + r;
                    pub32(&ck.segS[slot * D + lane], (uint32_t)S.runS[h][r][lane]);
                    if (lane == 0) {
                        pub64(&ck.meta[slot * 2], (uint64_t)S.runL[h][r] | ((uint64_t)(uint32_t)S.runf[h][r] << 32));
                        pub64(&ck.meta[slot * 2 + 1], (uint64_t)S.runB[h][r]);
                    }
                }
            }
            if (!own) stores_done();
            if (lane == 0) {
                pub64(hp + 1, ok ? S.mabs : 0ull);
                pub64(hp, (uint64_t)(uint32_t)npub | ((uint64_t)(uint32_t)flags << 16) |
                              ((uint64_t)(ok ? S.ovf & 0xFFFF : 0) << 24) | ((uint64_t)ck.ep << 40));
            }
        }
        STAMP(12);
        STAMP_FLUSH();
        return;
    }
    if (newrow && (wv == G || wv == G + 1)) stores_done();         // the new row, for the serial path
    // the replay's list lies over the chunk list, which the other head waves may still read
    if (!work) __syncthreads();                                    // (uniform)
    STAMP(8);

    // -- P6: the replay --------------------------------------------------------------
    // Wave h < G polls the headers of chunks 1 .. nch - 2 (one per lane and 64 at a time; the
    // wait is bounded, and a head whose wait gives up goes to the serial path), takes their
    // statistics and flags, lists their runs in order and requests them (sums lane = channel,
    // L, f and bounds lane = run); then it polls chunk 0's header and tagged state, which the
    // poll itself delivers, while those loads are in flight, and walks chunk 0's state through
    // the runs and through this chunk's own.
    int32_t aw = acc0;
    int64_t l = l0;
    unsigned long long events = (unsigned long long)nev0;
    int hflags = flags;            // this head's flags over every chunk
    unsigned long long tovf = ok ? S.ovf : 0, tmabs = ok ? S.mabs : 0;
    int total = 0;
    int spins = 0;
    bool gaveup = ck.spin_limit == 0;
    // This chunk's own runs (up to 8), applied last: their sums (lane = channel), factors and L
    // (lane = run) and the sum of their bounds, read now, while the headers are awaited.
    const bool own8 = nch > 1 && hw && (work || olist) && nruns[h] <= 8;
    int32_t vo[8];
    int32_t fko = 1 << PROB_FRAC;
    uint32_t lko = 0;
    int64_t bso = 0;
    if (own8) {
        const int nr = nruns[h];
#pragma unroll
        for (int k = 0; k < 8; ++k) vo[k] = k < nr ? S.runS[h][k][lane] : 0;
        if (lane > 0 && lane < nr) fko = S.runf[h][lane];       // run 0 continues the open run
        if (lane < nr) lko = S.runL[h][lane];
        bso = wave_sum_i64(lane < nr ? (int64_t)S.runB[h][lane] : 0);
    }
    const uint32_t ep = ck.ep;
    const uint64_t *hdr = ck.hdr + ((int64_t)chain * ck.mc * G + h) * 2;    // chunk c: hdr[c * G * 2]
    if (nch > 1 && hw) {
        uint16_t *rl = S.u.rp.rl[h];
        for (int c0 = 1; c0 < nch - 1; c0 += 64) {
            const int c = c0 + lane;
            const bool in = c < nch - 1;
            uint64_t w0 = 0, w1 = 0;
            while (true) {
                if (in) {
                    w0 = get64(&hdr[(int64_t)c * G * 2]);
                    w1 = get64(&hdr[(int64_t)c * G * 2 + 1]);
                }
                if (!__ballot(in && (uint32_t)(w0 >> 40) != ep)) break;
                if (gaveup || ++spins > ck.spin_limit) {
                    gaveup = true;
                    break;
                }
                __builtin_amdgcn_s_sleep(2);
            }
            // A current header lists at most SLOTS runs (a chunk whose runs did not fit
            // publishes none, with FL_POOL); one that lists more would send the loads past the
            // chunk's slots: a fault, and the head takes the serial path.
            const bool cep = in && (uint32_t)(w0 >> 40) == ep;
            const bool over = cep && (int)(w0 & 0xFFFF) > SLOTS;
            if (over && !((w0 >> 16) & FL_POOL)) st->fault = 1;
            const bool cur = cep && !over;
            const int n = cur ? (int)(w0 & 0xFFFF) : 0;
            int fl = cur ? (int)((w0 >> 16) & 0xFF) : 0;
            if (over) fl |= FL_POOL;
            if (in && !cep) fl |= FL_LB;
            const int incl = (int)wave_scan_add32((uint32_t)n);
            const int start = total + incl - n;
            for (int j = 0; j < n && start + j < NSEG; ++j)
                rl[start + j] = (uint16_t)((slot_base(c) + j) | (j ? RUN_EVENT : 0));
            total += __builtin_amdgcn_readlane(incl, 63);
#pragma unroll
            for (int bit = 0; bit < 4; ++bit) hflags |= __ballot((fl >> bit) & 1) ? 1 << bit : 0;
            if (h == 0) {
                // the score statistics, once per chain: counts below 2^16 per chunk
                tovf += (uint32_t)__builtin_amdgcn_readlane(
                    (int)wave_scan_add32(cur ? (uint32_t)((w0 >> 24) & 0xFFFF) : 0u), 63);
                const int64_t mm = wave_max_i64(cur ? (int64_t)w1 : 0);
                tmabs = (unsigned long long)mm > tmabs ? (unsigned long long)mm : tmabs;
            }
        }
        STAMP(14);
        if (total > NSEG) hflags |= FL_POOL;
        if (lane == 0) S.total[h] = hflags ? 0 : total;
    } else if (hw && lane == 0) {
        S.total[h] = 0;
    }
    // Chunk 0's header and state: one poll reads the header (flags, statistics) and the state's
    // tagged words, until every one carries this call's epoch (bounded like the other waits).
    auto take_chunk0 = [&]() __attribute__((always_inline)) {
        const uint64_t *s0 = ck.st0 + ((int64_t)chain * G + h) * (D + 1);
        uint64_t sa = 0, sm = 0, w0 = 0, w1 = 0;
        while (true) {
            sa = get64(&s0[lane]);
            sm = get64(&s0[D]);
            w0 = get64(&hdr[0]);
            w1 = get64(&hdr[1]);
            const bool cur = (uint32_t)(sa >> 48) == ep && (uint32_t)(sm >> 48) == ep && (uint32_t)(w0 >> 40) == ep;
            if (!__ballot(!cur)) break;
            if (gaveup || ++spins > ck.spin_limit) {
                gaveup = true;
                hflags |= FL_LB;
                return;
            }
            __builtin_amdgcn_s_sleep(2);
        }
        hflags |= (int)((w0 >> 16) & 0xF);
        if (h == 0) {
            tovf += (uint32_t)((w0 >> 24) & 0xFFFF);
            tmabs = w1 > tmabs ? w1 : tmabs;
        }
        aw = (int32_t)(uint32_t)sa;
        l = (int64_t)(sm & ((1ull << 26) - 1));
        events = (sm >> 26) & 0xFFF;
    };
    // Each head's wave walks its own runs, RPB at a time: their sums (lane = channel), L, f
    // and bounds (lane = run) loaded into registers together, one round trip, then the walk.
    bool unsafe = false;
    if (hw) {
        const int64_t hbase = ((int64_t)chain * G + h) * ck.pool;
        // this head's slot 0 (unused by the chunks' runs, so that a clamped index reads it),
        // lane = channel, and its meta words
        const int32_t *segh = ck.segS + hbase * D + lane;
        const uint64_t *metah = ck.meta + hbase * 2;
        bool take_c0 = nch > 1;
        const int tot_h = S.total[h];
        for (int g0 = 0; g0 < tot_h && !hflags; g0 += RPB) {
            const int nb = tot_h - g0 < RPB ? tot_h - g0 : RPB;
            const bool mine = lane < nb;
            const uint32_t ent = mine ? (uint32_t)S.u.rp.rl[h][g0 + lane] : 0u;
            // every slot index is checked against the pool before it is read: one past it (a
            // fault: the list is built from checked headers) is not loaded, and sends the head
            // to the serial path
            const int slot = (int)(ent & (RUN_EVENT - 1));
            const bool bad = mine && slot >= ck.pool;
            const bool ld = mine && !bad;
            // Every load first, none of them conditional, so that all are in flight together:
            // each run's L | f << 32 and bound (lane = run) and its sums (lane = channel). A
            // lane past nb, or one whose slot failed the check, reads slot 0, which lies in the
            // pool, and its values count 0.
            const int sl = ld ? slot : 0;
            const uint64_t lfr = get64(metah + 2 * sl);
            const uint64_t bbr = get64(metah + 2 * sl + 1);
            int32_t v[RPB];
#pragma unroll
            for (int k = 0; k < RPB; ++k) v[k] = (int32_t)get32(segh + (int64_t)__builtin_amdgcn_readlane(sl, k) * D);
            const uint64_t lf = ld ? lfr : 0ull;
            const int64_t bb = ld ? (int64_t)bbr : 0;
            if (take_c0) {
                // chunk 0, polled while these loads are in flight
                take_chunk0();
                take_c0 = false;
                if (hflags) break;
            }
            if (__ballot(bad)) {
                st->fault = 1;
                hflags |= FL_POOL;
                break;
            }
            STAMP(15);
            const uint64_t evm = __ballot(mine && (ent & RUN_EVENT));
            // The walk. |acc| only shrinks at a rescale and grows by at most a run's bound B per
            // run, so |acc| + the sum of the nb runs' B certifies them all at once: then a block
            // of 8 runs with no event adds as one tree, and elsewhere only a run that opens with
            // an event rescales first; L comes from a prefix sum over the runs.
            {
                const int64_t bsum_all = wave_sum_i64(mine ? bb : 0);
                const int64_t a0 = aw < 0 ? -(int64_t)aw : (int64_t)aw;
                STAMPV(27, nb);
                STAMPV(28, __ballot(a0 + bsum_all > ACC_HI) ? 2 : 1);
                if (!__ballot(a0 + bsum_all > ACC_HI)) {
                    const uint32_t PLa = wave_scan_add32((uint32_t)lf);   // L < 2^26 a run, 0 past nb
#pragma unroll
                    for (int k0 = 0; k0 < RPB; k0 += 8) {
                        if (k0 >= nb) break;
                        const int kn = nb - k0 < 8 ? nb - k0 : 8;
                        const uint32_t bev = (uint32_t)(evm >> k0) & ((1u << kn) - 1u);
                        const uint32_t lb = k0 ? (uint32_t)__builtin_amdgcn_readlane((int)PLa, k0 - 1) : 0u;
                        if (!bev) {
                            int32_t t[8];
#pragma unroll
                            for (int k = 0; k < 8; ++k) t[k] = k < kn ? v[k0 + k] : 0;
                            aw += ((t[0] + t[1]) + (t[2] + t[3])) + ((t[4] + t[5]) + (t[6] + t[7]));
                            l += (uint32_t)__builtin_amdgcn_readlane((int)PLa, k0 + kn - 1) - lb;
                            continue;
                        }
#pragma unroll
                        for (int k = 0; k < 8; ++k) {
                            if (k < kn) {
                                if ((bev >> k) & 1u) {
                                    const int64_t f = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(lf >> 32), k0 + k);
                                    aw = (int32_t)(((int64_t)aw * f) >> PROB_FRAC);
                                    l = (l * f) >> PROB_FRAC;
                                }
                                aw += v[k0 + k];
                                l += (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)lf, k0 + k);
                            }
                        }
                    }
                    events += (unsigned long long)__popcll(evm);
                    continue;
                }
            }
            // Otherwise block by block: lane k < nb holds run k's list entry, L, f and bound B;
            // prefix sums over the lanes give each block's sums, |acc at a block's start| + the
            // block's B certifies 8 runs at once, and elsewhere the walk goes run by run.
            // 32-bit prefix sums over the RPB = 64 runs: L < 2^26 per run, and bounds below 2^26
            // (a run with a larger one is checked on its own, by the walk run by run)
            static_assert(RPB <= 64, "64 bounds below 2^26 sum below 2^32");
            const uint64_t bigm = __ballot(mine && bb >= (1ll << 26));
            const uint32_t PB = wave_scan_add32(bb < (1ll << 26) ? (uint32_t)bb : 0u);
            const uint32_t PL = wave_scan_add32((uint32_t)lf);
            STAMP(23);
#pragma unroll
            for (int k0 = 0; k0 < RPB; k0 += 8) {
                if (k0 >= nb) break;
                const int kn = nb - k0 < 8 ? nb - k0 : 8;
                const uint32_t bmask = (1u << kn) - 1u;
                const uint32_t bev = (uint32_t)(evm >> k0) & bmask;
                const uint32_t before_b = k0 ? (uint32_t)__builtin_amdgcn_readlane((int)PB, k0 - 1) : 0u;
                const uint32_t before_l = k0 ? (uint32_t)__builtin_amdgcn_readlane((int)PL, k0 - 1) : 0u;
                const int64_t bsum = (uint32_t)__builtin_amdgcn_readlane((int)PB, k0 + kn - 1) - before_b;
                const int64_t a = aw < 0 ? -(int64_t)aw : (int64_t)aw;
                // A rescale never grows |acc|, so the block's bound certifies blocks with events
                // too: then only their rescales are applied in turn, with no check per run.
                const bool cert = !((uint32_t)(bigm >> k0) & bmask) && !__ballot(a + bsum > ACC_HI);
                if (kn < 8) {
#pragma unroll
                    for (int k = 1; k < 8; ++k) v[k0 + k] = k < kn ? v[k0 + k] : 0;
                }
                if (cert && !bev) {
                    aw += ((v[k0] + v[k0 + 1]) + (v[k0 + 2] + v[k0 + 3])) + ((v[k0 + 4] + v[k0 + 5]) + (v[k0 + 6] + v[k0 + 7]));
                    l += (uint32_t)__builtin_amdgcn_readlane((int)PL, k0 + kn - 1) - before_l;
                    continue;
                }
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    if (k < kn) {
                        if ((bev >> k) & 1u) {
                            const int64_t f = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(lf >> 32), k0 + k);
                            aw = (int32_t)(((int64_t)aw * f) >> PROB_FRAC);
                            l = (l * f) >> PROB_FRAC;
                            ++events;
                        }
                        if (!cert && !fits(aw, readlane64(bb, k0 + k))) unsafe = true;
                        aw += v[k0 + k];
                        l += (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)lf, k0 + k);
                    }
                }
            }
        }
        if (take_c0) take_chunk0();        // no runs, or the flags sent the head to the serial path
    }
    STAMP(30);
    if (nch > 1 && hw && (work || olist) && !hflags) {
        // this chunk's own runs, last (run 0 continues the run open before it)
        const int nr = nruns[h];
        const int64_t ao = aw < 0 ? -(int64_t)aw : (int64_t)aw;
        bool cert = false;
        if (own8 && !__ballot(ao + bso > ACC_HI)) {
            // certified by |acc| + their bounds: one chain, no branch (factor 2^15 past nr)
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const int64_t f = __builtin_amdgcn_readlane(fko, k);
                aw = (int32_t)(((int64_t)aw * f) >> PROB_FRAC) + vo[k];
                l = ((l * f) >> PROB_FRAC) + (uint32_t)__builtin_amdgcn_readlane((int)lko, k);
            }
            cert = true;
        } else {
            cert = fold_runs_certified(S, h, nr, lane, aw, l);
        }
        if (cert) events += (unsigned long long)(nr - 1);
        for (int r = 0; r < nr && !cert; ++r) {
            if (r > 0) {
                const int64_t f = S.runf[h][r];
                aw = (int32_t)(((int64_t)aw * f) >> PROB_FRAC);
                l = (l * f) >> PROB_FRAC;
                ++events;
            }
            if (!fits(aw, (int64_t)S.runB[h][r])) unsafe = true;
            aw += S.runS[h][r][lane];
            l += S.runL[h][r];
        }
    }
    if (hw && __ballot(unsafe)) hflags |= FL_CERT;
    STAMP(9);
    // The head waves finish alone: the serial path's LDS lies past the replay's list, and the
    // last head wave to finish posts the chain's statistics.
    if (hw) {
        const int qh = kvh * G + h;
        int32_t *orow = out + ((int64_t)b * g.n_q + qh) * D;
        if (hflags) {
            // The serial path counts score statistics only when no chunk did (the query
            // check failed). The new row came from this workgroup's waves G, G + 1, whose
            // stores are complete; the fence orders this wave's loads after them.
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
            serial_head<1, L::RS>(g, tabs, tabs->kc, tabs->vc, &S.qi[h][0], b, kvh, T, 0, !ok, S.u.sr.fb[h], orow, st);
            if (lane == 0) atomicAdd(&st->serial_fallbacks, 1ull);
        } else {
            const Recip rc = reciprocal(l);
            const int64_t acc = aw;
            orow[lane] = (int32_t)(wmul(acc, rc.r) >> rc.shift);
            STAMP(31);
            const int64_t amax = wave_max_i64(acc < 0 ? -acc : acc);
            if (lane == 0) {
                if (events) atomicAdd(&S.sev, events);
                atomicMax(&S.samax, (unsigned long long)amax);
                atomicOr((unsigned int *)&S.sdone, 2u);
            }
        }
        if (h == 0 && lane == 0) {
            S.ovf = tovf;
            S.mabs = tmabs;
        }
        int last = 0;
        if (lane == 0) {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            last = atomicAdd(&S.hfin, 1) == G - 1;
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        }
        if (__builtin_amdgcn_readfirstlane(last) && lane == 0) {
            // the chain's statistics, once: the heads' merged, and the score statistics of
            // every chunk (when the query check passed; the serial path counted them otherwise)
            if (S.sdone & 2) {
                atomicMax(&st->n_tokens, (unsigned long long)T);
                if (S.sev) atomicAdd(&st->rescale_events, S.sev);
                atomicMax(&st->max_abs_acc, S.samax);
            }
            if (ok) {
                if (S.ovf) atomicAdd(&st->score_overflows, S.ovf);
                atomicMax(&st->max_abs_score, S.mabs);
            }
        }
    }
    STAMP(10);
    STAMP_FLUSH();
}

static void carve(const Geom &g, int64_t mc, int64_t pool, uint8_t *p, Sck *ck, size_t *total, size_t *front) {
    const int64_t chains = (int64_t)g.batch * g.n_kv;
    size_t o = 0;
    auto take = [&](size_t n) {
        const size_t at = o;
        o += (n + 255) / 256 * 256;
        return p ? p + at : nullptr;
    };
    Sck c{};
    c.status = (unsigned long long *)take(chains * G * 2 * mc * sizeof(unsigned long long));
    c.hdr = (uint64_t *)take(chains * mc * G * 2 * sizeof(uint64_t));
    c.done = (unsigned int *)take(chains * sizeof(unsigned int));
    c.st0 = (uint64_t *)take(chains * G * (D + 1) * sizeof(uint64_t));
    if (front) *front = o;
    c.meta = (uint64_t *)take(chains * G * pool * 2 * sizeof(uint64_t));
    c.segS = (int32_t *)take(chains * G * pool * D * sizeof(int32_t));
    c.mc = (int32_t)mc;
    c.pool = (int32_t)pool;
    if (ck) *ck = c;
    if (total) *total = o;
}

}  // namespace stepk

bool step_supported(const Geom &g, int64_t capacity) {
    using namespace stepk;
    const int kbytes = g.d * g.kb / 8;
    const int kpl = kbytes / 16 + (kbytes % 16) / 8;
    return g.d == D && g.G == G && g.kb == 4 && g.vb == 2 && g.n_planes == kpl + 2 &&
           (capacity + CHUNK - 1) / CHUNK <= HMAX && g.norm_frac == 9;
}

int64_t step_max_chunks(int64_t capacity) { return (capacity + stepk::CHUNK - 1) / stepk::CHUNK; }

static int64_t step_pool(int64_t mc) { return 1 + (mc - 1) * stepk::SLOTS + 1; }

void step_layout_facts(const Geom &g, int64_t mc, int64_t *f) {
    using namespace stepk;
    // carved at a stand-in base address (never dereferenced): the areas' offsets
    uint8_t *const base = (uint8_t *)((uintptr_t)1 << 40);
    const int64_t pool = step_pool(mc);
    const int64_t chains = (int64_t)g.batch * g.n_kv;
    Sck c;
    size_t total = 0, front = 0;
    carve(g, mc, pool, base, &c, &total, &front);
    auto off = [&](const void *q) { return (int64_t)((const uint8_t *)q - base); };
    const int64_t at[] = {off(c.status), off(c.hdr), off(c.done), off(c.st0), off(c.meta), off(c.segS),
                          (int64_t)total};
    const int64_t sz[] = {chains * G * 2 * mc * 8, chains * mc * G * 2 * 8, chains * 4, chains * G * (D + 1) * 8,
                          chains * G * pool * 2 * 8, chains * G * pool * D * 4};
    bool ok = true;
    for (int i = 0; i < 6; ++i) ok = ok && at[i] % 256 == 0 && at[i] + sz[i] <= at[i + 1];
    ok = ok && (int64_t)front == off(c.meta);
    f[0] = mc;
    f[1] = pool;
    f[2] = SLOTS;
    f[3] = mc > 1 ? slot_base((int)mc - 1) + SLOTS : 1;    // chunk 0: one state slot
    f[4] = NSEG;
    f[5] = HMAX;
    f[6] = (int64_t)total;
    f[7] = (int64_t)front;
    f[8] = ok ? 1 : 0;
    f[9] = CHUNK;
    f[10] = RUN_EVENT;
}

size_t step_scratch_bytes(const Geom &g, int64_t mc) {
    size_t n = 0;
    stepk::carve(g, mc, step_pool(mc), nullptr, nullptr, &n, nullptr);
    return n;
}

hipError_t launch_step(hipStream_t s, const Geom &g, const Tables *t, int32_t *out, const int64_t *len,
                       ChunkScratch &cs, uint32_t ep, int64_t mc, int64_t grid_chunks, const StepIn &si,
                       LaunchEv ev, DevStats *st) {
    using namespace stepk;
    const int64_t chains = (int64_t)g.batch * g.n_kv;
    if (mc > HMAX || chains > 65535 || mc * chains > 0x7fffffff) return hipErrorInvalidValue;
    if (grid_chunks < 1 || grid_chunks > mc) grid_chunks = mc;
    const int64_t pool = step_pool(mc);
    Sck ck;
    size_t bytes = 0, front = 0;
    carve(g, mc, pool, (uint8_t *)cs.p, &ck, &bytes, &front);
    if (bytes > cs.bytes || ep == 0 || ep > EPOCH_MASK) return hipErrorInvalidValue;
    ck.ep = ep;
    ck.spin_limit = cs.spin_limit;
    const uint64_t layout = ((uint64_t)mc << 48) ^ ((uint64_t)pool << 24) ^ ((uint64_t)g.batch << 8) ^
                            (uint64_t)g.n_kv ^ (1ull << 61);
    {
        const hipError_t e = scratch_layout(s, cs, layout, front);
        if (e != hipSuccess) return e;
    }
    dim3 grid((unsigned)(grid_chunks * chains)), block(NT);
    if (g.kb == 4 && g.vb == 2)
        hipExtLaunchKernelGGL((step_kernel<4, 2>), grid, block, 0, s, ev.start, ev.stop, 0, g, t, out, len, ck, st,
                              si);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace insitu
