// The chunked attend: attend_online / attend_two_pass (ops/attention.py:429-513)
// over a context split into 1,024-token chunks, bit-exact with the sequential
// reference.
//
// Why it can be exact. In the online softmax the running maximum m_t is the
// prefix maximum of the scores, so a chunk reproduces the reference's
// arithmetic token for token once it knows the maximum of everything before it
// (M_in): the tokens with s_t > m_{t-1} are the rescale events, the factor
// there is LUT(s_t - m_{t-1}), and every other token contributes the integer
// floor(v_norm * p * c_v[code] / 2^23) with p = LUT(m_t - s_t). Between two
// events these terms only add, so a chunk hands over, per query head, one
// integer sum (and the sum of p) per event-free run, plus the factor opening
// each run. Replaying
//     acc = floor(acc * f / 2^15) + S,   l = floor(l * f / 2^15) + L
// over the runs in order is exactly the reference recurrence, provided the
// per-token int32 clamp of acc (attention.py:502-503) never fires; that is
// proven per run from the exact acc where the run starts plus the largest
// |prefix sum| of the run's terms (measured, per channel in chunk 0, over all
// channels in the published runs), and a head where it fails is recomputed on
// the serial path (serial_head.h). A run's prefix sums are kept in wrapping
// int32, exact because the sum of their |terms| stays below 2^31 (else the
// chunk flags the head wide and it goes serial too).
//
// Sequential (online) mode is one kernel. Workgroups are numbered chunk-major
// (all chunk-0 workgroups, then all chunk-1 ...), score their chunk (lane =
// token, G = 4 query heads per KV head), publish the chunk maximum, and read
// the maxima of their predecessors with a decoupled look-back. A workgroup
// only waits for workgroups with smaller numbers, which the dispatcher has
// already placed and which publish their maximum before they wait on anyone.
// The wait is bounded all the same: a workgroup that gives up marks its
// (sequence, KV head) for the serial path instead of hanging. The look-back
// words carry the value they publish, so they are read with relaxed atomics
// and no cache maintenance. Two-pass mode needs the maximum of the whole
// context, so it runs a chunk-max kernel first and the same chunk kernel second.
//
// Chunk 0 starts the sequence from acc = l = 0, so it replays its own runs as
// it goes and hands over one state. The last workgroup of each (sequence, KV
// head), elected by a completion counter, replays the rest, one thread per
// (query head, channel): it reads the headers of chunks 1 .. n-1 in one batch
// of loads, lists their runs in order in LDS, loads their sums 64 runs at a
// time (one round trip for a typical context, whose rescale events are few),
// walks them from chunk 0's state, finalizes and writes Q16. Chunk 0 counts
// itself done before publishing its state, so when it is the last (it usually
// is: it holds most rescale events) the state never leaves its registers.
// Scores: sum_ch q[ch] * c[code_ch] in fp64 FMA -- every partial sum is an
// integer below 2^51, so it is exact -- then the int64 norm multiply and >>24
// of the reference.
#include <type_traits>

#include "query.h"
#include "row_codec.h"
#include "serial_head.h"
#include "wave.h"

// The file is built twice: with 1,024-token chunks (two tokens per thread, the default) and,
// with INSITU_CHUNK_TPT=1, with 512-token chunks in namespace insitu::c512. A cache picks one
// at creation: the smaller chunks double the workgroups that walk a flat softmax's candidates,
// the larger ones halve the chunks that a peaked softmax looks back over and replays.
#ifndef INSITU_CHUNK_TPT
#define INSITU_CHUNK_TPT 2
#endif
static_assert(INSITU_CHUNK_TPT == 1 || INSITU_CHUNK_TPT == 2, "1,024- or 512-token chunks");

namespace insitu {
#if INSITU_CHUNK_TPT == 1
namespace c512 {
#endif

constexpr int CT = 512;              // threads per workgroup: 8 waves, 2 per SIMD
constexpr int TPT = INSITU_CHUNK_TPT;  // tokens per thread in the score phase
constexpr int CHUNK = CT * TPT;      // tokens per workgroup
constexpr int VB_MAX = 3;            // widest value code staged in LDS
constexpr int HMAX = 512;            // chunks per (sequence, KV head) on the chunked path
constexpr int NSEG = 2048;           // runs per (sequence, KV head, query head) the replay lists
constexpr int SLOTS = 8;             // run slots of every chunk after chunk 0 (which holds one state)
constexpr uint16_t RUN_EVENT = 0x8000;
constexpr int FLAG_POOL = 1;         // run pool exhausted
constexpr int FLAG_WIDE = 2;         // a run sum bound reached 2^31
// Look-back words: flag (bits 62-63) | call epoch (bits 48-61) | score - SCORE_LO
// (bits 0-47). A word whose epoch is not the current call's is unpublished, so
// the words never need resetting between calls.
constexpr unsigned long long ST_AGG = 1ull << 62, ST_INC = 2ull << 62;
constexpr unsigned long long ST_FLAGS = 3ull << 62;
constexpr int EPOCH_BITS = 14;
constexpr unsigned EPOCH_MASK = (1u << EPOCH_BITS) - 1u;
// A run whose sum of |term| bounds stays at or below this publishes that bound as
// its peak |prefix sum|; only blocks of entries where a run may exceed it track
// the actual prefix sums (sequential mode: flat softmax over large values).
constexpr int64_t TRACK_B = 1ll << 24;
constexpr double MAGIC = 6755399441055744.0;   // 1.5 * 2^52
constexpr int64_t MAGIC_BITS = 0x4338000000000000LL;

// What a chunk publishes, per query head: w0 = n_seg | flags << 16 | score
// overflows << 24 | call epoch << 40, w1 = max |score| (the statistics are per
// chunk, all heads). w0 is the flag the replaying workgroup polls: it goes out
// after the head's run slots and w1 have completed. A run slot
// holds lf = L | f << 32 (L = sum of p < 2^26, f = the factor opening the run,
// <= 2^15) and b = the largest |prefix sum| of the run over its tokens and
// channels (sequential mode; the sum of |terms| is < 2^31 unless FLAG_WIDE is set).
// Everything published between workgroups goes through relaxed agent-scope
// atomics, which are coherent across the XCDs without writing back or
// invalidating whole L2 caches.
struct ChunkHdr {
    uint64_t w0, w1;
};
struct SegMeta {
    uint64_t lf, b;
};

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
// The clamp certificate of one run: acc at its start plus every prefix sum of the
// run stays within int32 when |acc| + peak <= 2^31 - 1, peak = max |prefix sum|
// (0 <= peak < 2^31). In 32-bit unsigned: |acc| <= 2^31 - 1 - peak.
__device__ __forceinline__ bool fits(int32_t acc, int32_t peak) {
    const uint32_t a = acc < 0 ? 0u - (uint32_t)acc : (uint32_t)acc;
    return a <= 0x7FFFFFFFu - (uint32_t)peak;
}
__device__ __forceinline__ int32_t run_peak(int32_t hi, int32_t lo) {
    const uint32_t h = (uint32_t)hi, l = 0u - (uint32_t)lo;      // hi >= 0 >= lo
    return (int32_t)(h > l ? h : l);
}
template <int N>
__device__ __forceinline__ int64_t peak_of(const int32_t (&hi)[N], const int32_t (&lo)[N]) {
    int32_t m = run_peak(hi[0], lo[0]);
#pragma unroll
    for (int k = 1; k < N; ++k) m = run_peak(hi[k], lo[k]) > m ? run_peak(hi[k], lo[k]) : m;
    return m;
}
// Wait until this thread's stores (the relaxed atomics above) have completed.
__device__ __forceinline__ void stores_done() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_s_waitcnt(0x0F70);          // vmcnt(0)
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

struct Chunked {
    int64_t *cmax;                 // [chain][max_chunks][GF]   (two-pass)
    unsigned long long *status;    // [chain][GF][2][max_chunks] look-back words: inclusive, aggregate
    ChunkHdr *hdr;                 // [chain][max_chunks][GF]
    SegMeta *meta;                 // [chain][GF][pool]
    int32_t *segS;                 // [chain][GF][pool][d]
    unsigned int *done;            // [chain]  workgroups of the chain done with their runs
    unsigned int *chain_fb;        // [chain]  the call's epoch: recompute this chain serially
    double *qd;                    // [chain][d][GF]  the group's query rows in fp64 (query.h)
    int32_t *qok;                  // [chain]  nonzero: every score of the group is exact in fp64
    int32_t max_chunks, pool;
    uint32_t ep;                   // this call's epoch, 1 .. 2^14 - 1
    int32_t spin_limit;            // polls before a wait gives up (0: at once)
};

template <int D, int KB>
struct KF {
    static constexpr int KBYTES = D * KB / 8;
    static constexpr int KWORDS = KBYTES / 4;
    static constexpr int NFULL = KBYTES / 16;
    static constexpr int HALF = (KBYTES % 16) / 8;
    static constexpr int KPLANES = NFULL + HALF;
    static constexpr int CPL = D / 64;
    static constexpr uint32_t MASK = (1u << KB) - 1u;
    static constexpr int VW = D * VB_MAX / 32;                 // value words staged per token
    static constexpr int RS = ((D * KB / 8 + D * VB_MAX / 8 + 4) + 3) / 4 * 4;
};

__device__ __forceinline__ int64_t dbl_to_i64(double x) {
    // x is an integer with |x| <= 2^51: adding 1.5 * 2^52 puts it in the low mantissa bits.
    return (int64_t)__double_as_longlong(x + MAGIC) - MAGIC_BITS;
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

// A candidate token of a chunk for one head (a rescale event, or a token less
// than delta_max below the running maximum): token index | event << 10 |
// distance << 11. The distance is s - prev at an event and prev - s otherwise,
// clamped to delta_max (< 2^20), so that LUT(distance) is the event's factor f
// or the token's p (an event's own p is LUT(0), the same for every event).
static_assert(CHUNK <= 1024, "ActRec holds a 10-bit token index");
__device__ __forceinline__ uint32_t act_rec(int tl, bool ev, uint32_t dist) {
    return (uint32_t)tl | (ev ? 1u << 10 : 0u) | (dist << 11);
}

// What only the fused step keeps in LDS: the new token's boundaries, rows, codes
// and scores (live through the score phase), and the rotated query rows for the
// serial path.
template <int D>
struct StepLds {
    int64_t bnd[2][255];           // key and value boundaries
    int32_t kv[2][MAX_D];          // the rotated key and value
    uint8_t codes[2][MAX_D];
    int64_t newsc[GF];             // the new token's scores
    int32_t qi[GF][D];             // the rotated query rows
    // the run-sum walk (codes of at most 2 bits at d = 64): each head's entries of the
    // block, their value words word-major, so that a lane reads its word of entry j at a
    // fixed offset
    uint32_t crow[GF][4][64];
};
struct NoStep {};

template <int D, int KB, bool STEP>
struct ChunkLds {
    struct Phase {
        uint32_t rec[GF][CHUNK];   // each head's candidate tokens in order (act_rec)
        uint32_t vw[CHUNK][KF<D, KB>::VW];
        uint32_t vpad;             // the word after the last token's: read as the pair of its last word
        int16_t vn[CHUNK];
    };
    struct Replay {
        uint16_t slot[GF][NSEG];   // the runs in order: slot | RUN_EVENT when a rescale opens it
    };
    union {
        Phase ph;
        Replay rp;
        SerialLds<KF<D, KB>::RS> fb[GF];
    } u;
    typename std::conditional<STEP, StepLds<D>, NoStep>::type nr;
    union alignas(16) {            // 16-byte aligned: the score loop reads the rows as 128-bit words
        double qf[D * GF];         // the group's query rows [c][h] (unless staged), until the scores
        int32_t tt[GF][64][8];     // run sums: a block of 64 entries' terms for every value code
    } qt;
    double kcf[16];
    int64_t kc[16];
    int64_t vc[16];
    int32_t vc32[16];
    int64_t vcmax;
    int32_t expt[256];
    int32_t cntw[GF][CT / 64];     // candidate tokens per head and wave
    int32_t evw[GF][CT / 64];      // rescale events per head and wave
    int64_t min_[GF];              // the maximum before this chunk (two-pass: of all chunks)
    int64_t lmax[GF];              // this chunk's own maximum
    int64_t wt[GF][CT / 64];       // per head, each wave's maximum score
    int64_t red[CT / 64][GF];
    int qok;
    int last;
    int lb_fail;
    unsigned long long ovf, mabs;
};

// Run slots: chunk 0 owns slot 0 (its replayed state), chunk c > 0 owns SLOTS after it.
// The query head that slot h of KV head kvh's chain computes: its own (GF a KV head), or
// with g.gq query heads a KV head (fewer than GF) head h % gq: the slots from gq on compute
// duplicates of the first gq, whose outputs and statistics are dropped.
__device__ __forceinline__ int qhead(const Geom &g, int kvh, int h) {
    return g.gq ? kvh * g.gq + h % g.gq : kvh * GF + h;
}
__device__ __forceinline__ bool real_head(const Geom &g, int h) { return g.gq == 0 || h < g.gq; }
__host__ __device__ __forceinline__ int slot_base(int chunk) { return chunk == 0 ? 0 : 1 + (chunk - 1) * SLOTS; }
static_assert(1 + (HMAX - 1) * SLOTS < RUN_EVENT, "run slots of the chunked path fit 15 bits");

// The key codes and norm words of this thread's TPT consecutive tokens
// (t = t0 + TPT * tid + j): a wave reads one contiguous span of each plane.
template <int D, int KB>
__device__ __forceinline__ void load_keys(const Geom &g, const uint8_t *__restrict__ hb, int64_t t0,
                                          int64_t T, uint32_t (&w)[TPT][KF<D, KB>::KWORDS + 1],
                                          uint32_t (&normw)[TPT]) {
    using K = KF<D, KB>;
    const int tid = threadIdx.x;
    // Plane by plane across the thread's tokens, in the order the score loop
    // uses them, so that it can start on the first plane while the rest land.
    int64_t tc[TPT];
#pragma unroll
    for (int j = 0; j < TPT; ++j) {
        const int64_t t = t0 + tid * TPT + j;
        tc[j] = t < T ? t : 0;                       // past the end: read token 0, unused
        w[j][K::KWORDS] = 0;
    }
#pragma unroll
    for (int p = 0; p < K::NFULL; ++p)
#pragma unroll
        for (int j = 0; j < TPT; ++j) {
            const uint4 v = *(const uint4 *)(hb + p * g.span + tc[j] * 16);
            w[j][4 * p] = v.x;
            w[j][4 * p + 1] = v.y;
            w[j][4 * p + 2] = v.z;
            w[j][4 * p + 3] = v.w;
        }
    if (K::HALF) {
#pragma unroll
        for (int j = 0; j < TPT; ++j) {
            const uint2 v = *(const uint2 *)(hb + K::NFULL * g.span + tc[j] * 8);
            w[j][4 * K::NFULL] = v.x;
            w[j][4 * K::NFULL + 1] = v.y;
        }
    }
#pragma unroll
    for (int j = 0; j < TPT; ++j) normw[j] = *(const uint32_t *)(hb + (g.n_planes - 1) * g.span + tc[j] * 4);
}

// Exact scores of those tokens for the GF heads (attention.py:333-359), in
// groups of 8 channels. Per group the TPT x 8 centroid reads are issued as one
// LDS batch, then the FMAs run channel by channel over all TPT x GF
// accumulators, so an accumulator is reused only every TPT * GF FMAs. The
// query values are the chain's staged fp64 rows qc = [c][h]: the address is
// wave-uniform and the memory read-only in this kernel, so they arrive by
// scalar loads and enter the FMAs as scalar operands. The 8 codes of a group sit in
// one 32-bit window of the key bitstream (8 * KB <= 32 bits), cut out with
// alignbit.
template <int D, int KB>
__device__ __forceinline__ void score_keys(const uint32_t (&w)[TPT][KF<D, KB>::KWORDS + 1],
                                           const uint32_t (&normw)[TPT], const double *__restrict__ qc,
                                           const double *kcf, int score_shift,
                                           int64_t (&s)[TPT][GF]) {
    using K = KF<D, KB>;
    double acc[TPT][GF];
#pragma unroll
    for (int j = 0; j < TPT; ++j)
#pragma unroll
        for (int h = 0; h < GF; ++h) acc[j][h] = 0.0;
#pragma unroll
    for (int grp = 0; grp < D / 8; ++grp) {
        const int bo = 8 * KB * grp, wi = bo >> 5, sh = bo & 31;
        double cv[TPT][8];
#pragma unroll
        for (int j = 0; j < TPT; ++j) {
            const uint32_t win = sh == 0 ? w[j][wi] : __builtin_amdgcn_alignbit(w[j][wi + 1], w[j][wi], sh);
#pragma unroll
            for (int i = 0; i < 8; ++i) cv[j][i] = kcf[(win >> (i * KB)) & K::MASK];
        }
        double qv[8][GF];
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int h = 0; h < GF; ++h) qv[i][h] = qc[(8 * grp + i) * GF + h];
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int j = 0; j < TPT; ++j)
#pragma unroll
                for (int h = 0; h < GF; ++h) acc[j][h] = fma(qv[i][h], cv[j][i], acc[j][h]);
        // Pin the accumulators at every group so the compiler cannot turn the
        // loop nest inside out (load every centroid first, FMA at the end).
#pragma unroll
        for (int j = 0; j < TPT; ++j)
#pragma unroll
            for (int h = 0; h < GF; ++h) asm volatile("" : "+v"(acc[j][h]));
    }
#pragma unroll
    for (int j = 0; j < TPT; ++j) {
        const int64_t kn = sext16(normw[j]);
#pragma unroll
        for (int h = 0; h < GF; ++h) s[j][h] = wmul(dbl_to_i64(acc[j][h]), kn) >> score_shift;
    }
}

// ---------------------------------------------------------------------------
// two-pass pre-pass: the maximum score of every chunk, and the score statistics
// ---------------------------------------------------------------------------

// QS: the query rows are staged (query.h). Otherwise every workgroup stages
// its group's rows from the caller's int32 rows into LDS, and chunk 0's
// workgroup also fills the staging for the chunk kernel that follows.
template <int D, int KB, bool QS>
__global__ void __launch_bounds__(CT) chunk_max_kernel(Geom g, const Tables *__restrict__ tabs,
                                                       const int32_t *__restrict__ q,
                                                       double *qd, int32_t *qok,
                                                       const int64_t *__restrict__ len,
                                                       Chunked ck, DevStats *st) {
    __shared__ double kcf[16];
    __shared__ double qf[QS ? 1 : D * GF];
    __shared__ int qok_s;
    __shared__ int64_t red[CT / 64][GF];
    __shared__ unsigned long long ovf_s, mabs_s;
    const int chunk = blockIdx.x, chain = blockIdx.y;
    const int b = chain / g.n_kv, kvh = chain % g.n_kv;
    const int64_t T = len[b];
    const int64_t nch = T > 0 ? (T + CHUNK - 1) / CHUNK : 1;
    if (chunk >= nch) return;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    // the query rows (unless staged) and the chunk's keys first, then the
    // centroid table while they land
    int32_t q_t[D / 64];
    if (!QS && wv < GF) {
        const int32_t *qrow = q + ((int64_t)b * g.n_q + qhead(g, kvh, wv)) * D;
#pragma unroll
        for (int k = 0; k < D / 64; ++k) q_t[k] = qrow[lane + 64 * k];
    }
    const int64_t t0 = (int64_t)chunk * CHUNK;
    uint32_t nw[TPT];
    uint32_t kw[TPT][KF<D, KB>::KWORDS + 1];
    load_keys<D, KB>(g, plane_ptr(g, b, kvh, 0), t0, T, kw, nw);
    if (tid == 0) ovf_s = mabs_s = 0;
    if (tid == 0) qok_s = 1;
    if (tid < (1 << g.kb)) kcf[tid] = (double)tabs->kc[tid];
    __syncthreads();
    const double *qc = qd + (int64_t)chain * D * GF;
    bool ok;
    if constexpr (QS) {
        ok = qok[chain] != 0;
    } else {
        if (wv < GF) {
            double cmax = 0.0;
            for (int i = 0; i < (1 << g.kb); ++i) cmax = fmax(cmax, fabs(kcf[i]));
            const bool okh = stage_query_head<D / 64>(q_t, D, wv, qf, cmax,
                                                      chunk == 0 && real_head(g, wv) ? &st->range_errors : nullptr);
            if (lane == 0 && !okh) atomicAnd(&qok_s, 0);
        }
        __syncthreads();
        ok = qok_s != 0;
        qc = qf;
        if (chunk == 0) {          // the staging the chunk kernel reads
            for (int i = tid; i < D * GF; i += CT) qd[(int64_t)chain * D * GF + i] = qf[i];
            if (tid == 0) qok[chain] = qok_s;
        }
    }
    int64_t mx[GF];
#pragma unroll
    for (int h = 0; h < GF; ++h) mx[h] = SCORE_LO;
    unsigned long long ovf = 0;
    int64_t mabs = 0;
    if (ok) {
        int64_t s[TPT][GF];
        score_keys<D, KB>(kw, nw, qc, kcf, CENT_FRAC + g.norm_frac, s);
#pragma unroll
        for (int j = 0; j < TPT; ++j) {
            if (t0 + tid * TPT + j >= T) continue;
#pragma unroll
            for (int h = 0; h < GF; ++h) {
                int64_t v = s[j][h];
                if (v < SCORE_LO || v > SCORE_HI) {
                    if (real_head(g, h)) ++ovf;
                    v = v < SCORE_LO ? SCORE_LO : SCORE_HI;
                }
                const int64_t a = v < 0 ? -v : v;
                mabs = a > mabs ? a : mabs;
                mx[h] = v > mx[h] ? v : mx[h];
            }
        }
    }
#pragma unroll
    for (int h = 0; h < GF; ++h) {
        const int64_t m = wave_max_i64(mx[h]);
        if (lane == 0) red[wv][h] = m;
    }
    ovf = (unsigned long long)wave_sum_i64((int64_t)ovf);
    mabs = wave_max_i64(mabs);
    if (lane == 0) {
        if (ovf) atomicAdd(&ovf_s, ovf);
        atomicMax(&mabs_s, (unsigned long long)mabs);
    }
    __syncthreads();
    if (tid < GF) {
        int64_t m = red[0][tid];
        for (int w = 1; w < CT / 64; ++w) m = red[w][tid] > m ? red[w][tid] : m;
        ck.cmax[((int64_t)chain * ck.max_chunks + chunk) * GF + tid] = m;
    }
}

// ---------------------------------------------------------------------------
// the chunk kernel
// ---------------------------------------------------------------------------

// QS: the query rows are staged (query.h) and read by scalar loads. Otherwise
// (a standalone sequential attend, one launch) every workgroup stages its
// group's rows from the caller's int32 rows into LDS.
// STEP (with SEQ, not QS): the fused decode step (kernel.py:271-345) in one
// launch. len holds the lengths before the step and the attend covers one
// token more: every workgroup rotates its group's wire query rows itself, and
// the workgroup of the chunk holding the new token rotates, encodes and packs
// its key/value row, stores it into the planes and scores it from LDS.
template <int D, int KB, bool SEQ, bool QS, bool STEP>
__global__ void __launch_bounds__(CT, 2) chunk_kernel(Geom g, const Tables *__restrict__ tabs,
                                                   const int32_t *__restrict__ q,
                                                   const double *__restrict__ qd,
                                                   const int32_t *__restrict__ qok, int32_t *out,
                                                   const int64_t *__restrict__ len, Chunked ck,
                                                   DevStats *st, StepIn si) {
    static_assert(!STEP || (SEQ && !QS), "the fused step is the sequential kernel with LDS queries");
    using K = KF<D, KB>;
    constexpr int CPL = K::CPL;
    __shared__ ChunkLds<D, KB, STEP> S;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);      // wave index, scalar
    const int n_chains = g.batch * g.n_kv;

    // Sequential mode numbers workgroups chunk-major, so every predecessor of
    // a chunk has a smaller workgroup number.
    int chunk, chain;
    if (SEQ) {
        chunk = (int)(blockIdx.x / (unsigned)n_chains);
        chain = (int)(blockIdx.x % (unsigned)n_chains);
    } else {
        chunk = blockIdx.x;
        chain = blockIdx.y;
    }
    const int b = chain / g.n_kv, kvh = chain % g.n_kv;
    const int64_t T = len[b] + (STEP ? 1 : 0);
    const int64_t nch = T > 0 ? (T + CHUNK - 1) / CHUNK : 1;
    const bool has_work = chunk < nch;
    const bool new_row = STEP && chunk == nch - 1;     // this chunk holds the step's new token
    if (STEP && chunk == 0 && kvh == 0 && tid == 0) si.len_out[b] = T;
    const int nv = 1 << g.vb;
    const int acc_shift = CENT_FRAC + g.norm_frac + PROB_FRAC - ACC_FRAC;
    const int score_shift = CENT_FRAC + g.norm_frac;
    const int64_t t0 = (int64_t)chunk * CHUNK;

    if (has_work) {
        // The small loads first (the tables, and the query rows unless they are
        // staged), then this chunk's keys and values plane by plane. The counter
        // of outstanding vector loads drains in order, so staging the small
        // values must not wait for the chunk's data, and the score loop starts
        // on the first key plane while the others land. Staged query rows come
        // by scalar loads, which do not wait on that counter.
        const int nk = 1 << g.kb;
        const int64_t kc_t = tid < nk ? tabs->kc[tid] : 0;
        const int64_t vc_t = tid < nv ? tabs->vc[tid] : 0;
        const int32_t ex_t = tid < 256 ? tabs->exp_table[tid] : 0;
        int32_t q_t[D / 64];
        int32_t kv_t[D / 64];          // STEP: the new token's key (wave GF) or value (GF + 1)
        if (STEP) {
            if (wv < GF)
                load_vec<D / 64>(si.qw + ((int64_t)b * g.n_q + qhead(g, kvh, wv)) * D, D, q_t);
            else if (new_row && wv < GF + 2)
                load_vec<D / 64>((wv == GF ? si.kw : si.vw) + ((int64_t)b * g.n_kv + kvh) * D, D, kv_t);
        } else if (!QS && wv < GF) {
            const int32_t *qrow = q + ((int64_t)b * g.n_q + qhead(g, kvh, wv)) * D;
#pragma unroll
            for (int k = 0; k < D / 64; ++k) q_t[k] = qrow[lane + 64 * k];
        }
        const uint8_t *hb = plane_ptr(g, b, kvh, 0);
        uint32_t kw[TPT][K::KWORDS + 1];
        uint32_t nw[TPT];
        load_keys<D, KB>(g, hb, t0, T, kw, nw);
        const int vwords = g.value_bytes / 4;
        uint32_t vreg[TPT][K::VW];
#pragma unroll
        for (int j = 0; j < TPT; ++j) {
            const int64_t t = t0 + tid * TPT + j;
            const int64_t tc = t < T ? t : 0;
            // The value field is split into 16-byte planes (the last one narrower),
            // so value word 4 * p + i sits in word i of value plane p.
#pragma unroll
            for (int p = 0; p < (K::VW + 3) / 4; ++p) {
                const int wdt = g.plane_w[K::KPLANES + p];
                const uint32_t *src = (const uint32_t *)(hb + (K::KPLANES + p) * g.span + tc * wdt);
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (4 * p + i < K::VW) vreg[j][4 * p + i] = 4 * p + i < vwords ? src[i] : 0u;
            }
        }
        if (tid < 16) {
            S.kc[tid] = kc_t;
            S.kcf[tid] = (double)kc_t;
            S.vc[tid] = vc_t;
            S.vc32[tid] = (int32_t)vc_t;               // |centroid| < 2^18 (Q1.15)
        }
        if (tid < 256) S.expt[tid] = ex_t;
        if (wv == 0) {
            const int64_t m = wave_max_i64(vc_t < 0 ? -vc_t : vc_t);
            if (lane == 0) S.vcmax = m;
        }
        if (tid == 0) {
            S.ovf = S.mabs = 0;
            S.lb_fail = 0;
            S.qok = 1;
        }
        if (STEP) {
            // The rotations, once the small rows are in: their waits leave the
            // chunk's own loads in flight. Chunk 0 counts the queries' range
            // errors, the new token's chunk those of its key and value.
            if (wv < GF)
                rotate_loaded<D / 64>(q_t, D, si.rounds, si.sg, q_t, chunk == 0 ? &st->range_errors : nullptr);
            else if (new_row && wv < GF + 2)
                rotate_loaded<D / 64>(kv_t, D, si.rounds, si.sg, kv_t, &st->range_errors);
            if constexpr (STEP) {
                if (new_row) {
                    stage_bounds(tabs, g, S.nr.bnd);
                    if (wv == GF || wv == GF + 1) {
#pragma unroll
                        for (int k = 0; k < D / 64; ++k) S.nr.kv[wv - GF][lane + 64 * k] = kv_t[k];
                    }
                }
            }
        }
        __syncthreads();
        // Whether every score of the group stays an exact fp64 integer (query.h).
        const double *qc = qd + (int64_t)chain * D * GF;
        bool ok;
        if constexpr (QS) {
            ok = qok[chain] != 0;
        } else {
            // Chunk 0 counts the range errors of the rotated queries, once per call.
            if (wv < GF) {
                const bool okh = stage_query_head<D / 64>(q_t, D, wv, S.qt.qf, tabs->kc_absmax,
                                                          chunk == 0 && real_head(g, wv) ? &st->range_errors
                                                                                         : nullptr);
                if (lane == 0 && !okh) atomicAnd(&S.qok, 0);
                if constexpr (STEP) {
#pragma unroll
                    for (int k = 0; k < D / 64; ++k) S.nr.qi[wv][lane + 64 * k] = q_t[k];
                }
            }
            __syncthreads();
            ok = S.qok != 0;
            qc = S.qt.qf;
        }
        // The fused step's new token, beside the score phase: wave 0 encodes its
        // key (rotated by wave GF), stores the key words into the planes and
        // scores it for the GF heads (lane = channel; the partial sums are exact
        // integers, so their sum is the score loop's); wave 1 encodes its value,
        // stores the value words and stages them for the run sums. Waves 0 and 1
        // are the older wave of their SIMD, whose instructions issue first, so this
        // latency-bound work runs beside waves GF and GF + 1's scores instead of
        // after them. The stores are agent-coherent: a serial fallback elsewhere
        // reads the row. The thread that holds token T - 1 scores what its loads
        // found there and sets the result aside; it takes the new scores after the
        // score phase.
        int64_t nmx[GF];                  // wave 0, lane 0: the new token's clamped scores
        unsigned long long novf = 0;
        int64_t nmabs = 0;
#pragma unroll
        for (int h = 0; h < GF; ++h) nmx[h] = SCORE_LO;
        if constexpr (STEP) {
            if (new_row && wv < 2) {
                const int f = wv;              // 0: key, 1: value
                int64_t x[D / 64];
#pragma unroll
                for (int k = 0; k < D / 64; ++k) x[k] = S.nr.kv[f][lane + 64 * k];
                const int64_t n = encode_field<D / 64>(x, D, g.norm_frac, S.nr.bnd[f],
                                                       (1 << (f == 0 ? g.kb : g.vb)) - 1, S.nr.codes[f]);
                const int kwords = g.key_bytes / 4, vwords = g.value_bytes / 4, nwords = g.row_bytes / 4;
                const int tln = (int)(T - 1 - t0);
                uint16_t *nword = (uint16_t *)row_word_ptr(g, b, kvh, T - 1, nwords - 1);
                if (f == 0) {
                    if (lane < kwords) pub32(row_word_ptr(g, b, kvh, T - 1, lane), pack_row_word(g, S.nr.codes, n, 0, lane));
                    if (lane == 0) __hip_atomic_store(nword, (uint16_t)(n & 0xFFFF), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    if (ok) {
                        int64_t part[GF];
#pragma unroll
                        for (int h = 0; h < GF; ++h) {
                            double a = 0.0;
#pragma unroll
                            for (int k = 0; k < D / 64; ++k) {
                                const int c = lane + 64 * k;
                                a = fma(S.qt.qf[c * GF + h], S.kcf[S.nr.codes[0][c]], a);
                            }
                            part[h] = dbl_to_i64(a);
                        }
                        const int64_t kn = sext16((uint32_t)(n & 0xFFFF));
#pragma unroll
                        for (int h = 0; h < GF; ++h) {
                            int64_t v = wmul(wave_sum_i64(part[h]), kn) >> score_shift;
                            if (v < SCORE_LO || v > SCORE_HI) {
                                ++novf;
                                v = v < SCORE_LO ? SCORE_LO : SCORE_HI;
                            }
                            const int64_t a = v < 0 ? -v : v;
                            nmabs = a > nmabs ? a : nmabs;
                            if (lane == 0) {
                                nmx[h] = v;
                                S.nr.newsc[h] = v;
                            }
                        }
                        if (lane != 0) novf = 0, nmabs = 0;
                    }
                } else {
                    if (lane < vwords) {
                        const uint32_t w = pack_row_word(g, S.nr.codes, 0, n, kwords + lane);
                        pub32(row_word_ptr(g, b, kvh, T - 1, kwords + lane), w);
                        S.u.ph.vw[tln][lane] = w;
                    }
                    if (lane == 0) {
                        __hip_atomic_store(nword + 1, (uint16_t)(n & 0xFFFF), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        S.u.ph.vn[tln] = (int16_t)(n & 0xFFFF);
                    }
                }
            }
        }

        // -- phase 1: scores of the thread's TPT consecutive tokens, which stay in
        // registers for the scan; value codes into LDS ----------------------------
        int64_t mx[GF];
        int64_t sv[GF][TPT];      // clamped scores, SCORE_LO past the end
#pragma unroll
        for (int h = 0; h < GF; ++h) mx[h] = nmx[h];
        if (ok) {
            int64_t s[TPT][GF];
            score_keys<D, KB>(kw, nw, qc, S.kcf, score_shift, s);
            unsigned long long ovf = novf;
            int64_t mabs = nmabs;
#pragma unroll
            for (int j = 0; j < TPT; ++j) {
                const int tl = tid * TPT + j;
                const int64_t t = t0 + tl;
                const bool fresh = STEP && new_row && t == T - 1;     // scored by wave 0
                if (t < T && !fresh) {
#pragma unroll
                    for (int h = 0; h < GF; ++h) {
                        int64_t v = s[j][h];
                        if (v < SCORE_LO || v > SCORE_HI) {
                            if (real_head(g, h)) ++ovf;
                            v = v < SCORE_LO ? SCORE_LO : SCORE_HI;
                        }
                        const int64_t a = v < 0 ? -v : v;
                        mabs = a > mabs ? a : mabs;
                        mx[h] = v > mx[h] ? v : mx[h];
                        sv[h][j] = v;
                    }
#pragma unroll
                    for (int i = 0; i < K::VW; ++i)
                        if (i < vwords) S.u.ph.vw[tl][i] = vreg[j][i];
                } else {
#pragma unroll
                    for (int h = 0; h < GF; ++h) sv[h][j] = SCORE_LO;
                }
                if (!fresh) S.u.ph.vn[tl] = (int16_t)(nw[j] >> 16);
            }
            ovf = (unsigned long long)wave_sum_i64((int64_t)ovf);
            mabs = wave_max_i64(mabs);
            if (lane == 0) {
                if (ovf) atomicAdd(&S.ovf, ovf);
                atomicMax(&S.mabs, (unsigned long long)mabs);
            }
        }
#pragma unroll
        for (int h = 0; h < GF; ++h) {
            const int64_t m = wave_max_i64(mx[h]);
            if (lane == 0) S.red[wv][h] = m;
        }
        __syncthreads();
        if constexpr (STEP) {
            if (new_row && ok) {
                const int tln = (int)(T - 1 - t0);
                if (tid == tln / TPT) {
#pragma unroll
                    for (int j = 0; j < TPT; ++j)
                        if (j == tln % TPT) {
#pragma unroll
                            for (int h = 0; h < GF; ++h) sv[h][j] = S.nr.newsc[h];
                        }
                }
            }
        }

        // -- phase 2: the maximum before this chunk (sequential) or of all chunks --
        // Two look-back words per (chunk, head): the inclusive maximum and this
        // chunk's own (aggregate). Wave GF + h publishes head h's aggregate (chunk
        // 0: its inclusive maximum) while wave h looks back, so that the polling
        // wave has no store in flight: its loads' waits would drain it.
        static_assert(CT / 64 == 2 * GF, "a publishing wave beside each polling wave");
        if (SEQ) {
            const int h = wv & (GF - 1);
            int64_t local = S.red[0][h];
            for (int w = 1; w < CT / 64; ++w) local = S.red[w][h] > local ? S.red[w][h] : local;
            // [chain][head][inclusive, aggregate][chunk]: the lanes of a poll (consecutive
            // predecessors) read consecutive words
            unsigned long long *wi0 = ck.status + ((int64_t)chain * GF + h) * 2 * ck.max_chunks;
            unsigned long long *wa0 = wi0 + ck.max_chunks;
            if (wv >= GF) {
                if (lane == 0)
                    __hip_atomic_store((chunk == 0 ? wi0 : wa0) + chunk, st_pack(chunk == 0 ? ST_INC : ST_AGG, ck.ep, local),
                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            } else {
                int64_t run = SCORE_LO;
                bool fail = false;
                if (chunk > 0) {
                    int64_t base = chunk - 1;       // the predecessor lane 0 reads
                    int spins = 0;
                    fail = ck.spin_limit == 0;
                    while (!fail) {
                        const int64_t pc = base - lane;
                        unsigned long long flag = ST_INC;
                        int64_t val = SCORE_LO;
                        if (pc >= 0) {
                            const unsigned long long wi = __hip_atomic_load(wi0 + pc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                            const unsigned long long wa = __hip_atomic_load(wa0 + pc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                            const bool has_inc = st_flag(wi, ck.ep) == ST_INC;
                            flag = has_inc ? ST_INC : st_flag(wa, ck.ep);
                            val = st_val(has_inc ? wi : wa);
                        }
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
                }
                if (lane == 0) {
                    S.min_[h] = run;
                    S.lmax[h] = local;
                    if (fail) S.lb_fail = 1;
                }
            }
        } else if (!SEQ && wv < GF) {
            int64_t m = SCORE_LO;
            for (int64_t c = lane; c < nch; c += 64) {
                const int64_t v = ck.cmax[((int64_t)chain * ck.max_chunks + c) * GF + wv];
                m = v > m ? v : m;
            }
            m = wave_max_i64(m);
            if (lane == 0) S.min_[wv] = m;
        }
        __syncthreads();
        if (SEQ && S.lb_fail && tid == 0) pub32(&ck.chain_fb[chain], ck.ep);

        // -- phase 3: events and each head's candidate tokens listed in order ----
        // (the thread owns TPT consecutive tokens). Two exact shortcuts: a head
        // whose chunk maximum does not exceed the maximum before the chunk has no
        // rescale event, so it needs no scan; and a token at or below
        // prev - delta_max has p = 0 for every later prev too (prev only grows),
        // so a wave whose tokens are all that far down records nothing.
        if (ok) {
            const int64_t dm = tabs->delta_max;
            bool evh[GF];
            int64_t excl[GF];
            bool any_ev = false;
#pragma unroll
            for (int h = 0; h < GF; ++h) {
                evh[h] = SEQ && uni64(S.lmax[h]) > uni64(S.min_[h]);
                any_ev = any_ev || evh[h];
                excl[h] = SCORE_LO;
                if (evh[h]) {
                    int64_t run = SCORE_LO;
#pragma unroll
                    for (int j = 0; j < TPT; ++j) run = sv[h][j] > run ? sv[h][j] : run;
                    const int64_t v = wave_scan64<OpMax64>(run, SCORE_LO);
                    if (lane == 63) S.wt[h][wv] = v;
                    excl[h] = wave_shr1_64(v, SCORE_LO);
                }
            }
            if (any_ev) __syncthreads();
            uint32_t rec[GF][TPT];
            uint32_t act[GF];
            uint32_t pos[GF];
#pragma unroll
            for (int h = 0; h < GF; ++h) {
                int64_t prev = uni64(S.min_[h]);
                if (evh[h]) {
                    // the maxima of the waves before this one: independent reads
#pragma unroll
                    for (int w = 0; w < CT / 64 - 1; ++w) {
                        const int64_t m = S.wt[h][w];
                        prev = w < wv && m > prev ? m : prev;
                    }
                    prev = excl[h] > prev ? excl[h] : prev;
                }
                act[h] = 0;
                pos[h] = 0;
                bool live = false;
#pragma unroll
                for (int j = 0; j < TPT; ++j) {
                    rec[h][j] = 0;
                    live = live || (t0 + tid * TPT + j < T && sv[h][j] > prev - dm);
                }
                int32_t tot = 0, evt = 0;
                if (__ballot(live)) {
                    // Per token only compares: the candidates are the events and
                    // the tokens less than delta_max below the running maximum
                    // (the others have p = 0). A candidate records its distance
                    // from the running maximum, clamped to delta_max; the run-sum
                    // phase turns it into f = LUT(s - prev) at an event (whose
                    // own p is LUT(0)) or p = LUT(prev - s), one lane per entry.
                    // Counts and list positions come from one ballot per token
                    // slot: the lanes below hold the earlier tokens.
                    uint32_t before = 0;
#pragma unroll
                    for (int j = 0; j < TPT; ++j) {
                        const int tl = tid * TPT + j;
                        const bool in = t0 + tl < T;
                        const int64_t sj = sv[h][j];
                        const int64_t d = prev - sj;
                        const bool ev = evh[h] && in && d < 0;
                        const bool a = in && d < dm;               // events included
                        const int64_t up = -d < dm ? -d : dm;
                        const uint32_t dd = (uint32_t)(ev ? up : d);   // <= delta_max < 2^20 when a
                        prev = ev ? sj : prev;
                        rec[h][j] = act_rec(tl, ev, dd);
                        act[h] |= a ? 1u << j : 0u;
                        const uint64_t ba = __ballot(a);
                        before += __builtin_amdgcn_mbcnt_hi((uint32_t)(ba >> 32),
                                                            __builtin_amdgcn_mbcnt_lo((uint32_t)ba, 0u));
                        tot += __popcll(ba);
                        if (evh[h]) evt += __popcll(__ballot(ev));
                    }
                    pos[h] = before;
                }
                if (lane == 0) {
                    S.cntw[h][wv] = tot;
                    S.evw[h][wv] = evt;
                }
            }
            __syncthreads();
#pragma unroll
            for (int h = 0; h < GF; ++h) {
                if (!act[h]) continue;
                uint32_t at = pos[h];
#pragma unroll
                for (int w = 0; w < CT / 64 - 1; ++w) at += w < wv ? (uint32_t)S.cntw[h][w] : 0u;
#pragma unroll
                for (int j = 0; j < TPT; ++j)
                    if ((act[h] >> j) & 1u) S.u.ph.rec[h][at++] = rec[h][j];
            }
        }
        __syncthreads();

        // -- phase 4: run sums over the candidate list, wave = head, lane = channel -
        // Chunk 0 starts the sequence (acc = l = 0), so it replays its own runs
        // here: acc and l after its last token stand in for all its runs. Every
        // later chunk publishes its runs. acc stays in 32 bits in sequential
        // mode: |acc at a run's start| + the run's largest |prefix sum| <= 2^31 - 1
        // whenever the result is used (past a failed check the head goes to the
        // serial path); two-pass sums need 64.
        using AccT = typename std::conditional<SEQ, int32_t, int64_t>::type;
        const bool own = chunk == 0;
        AccT acc0[CPL];
#pragma unroll
        for (int k = 0; k < CPL; ++k) acc0[k] = 0;
        int64_t l0 = 0;
        int n_ev0 = 0, flags0 = 0;
        if (ok && wv < GF) {
            const int h = wv;
            int n_act = 0, n_ev = 0;
#pragma unroll
            for (int w = 0; w < CT / 64; ++w) {
                n_act += S.cntw[h][w];
                n_ev += S.evw[h][w];
            }
            n_act = uni32(n_act);
            n_ev = uni32(n_ev);
            const int n_seg = n_ev + 1;
            const int off = slot_base(chunk);
            int flags = 0;
            if (!own && n_seg > SLOTS) flags |= FLAG_POOL;
            if (!flags) {
                int wi[CPL], wi1[CPL], sh[CPL];
#pragma unroll
                for (int k = 0; k < CPL; ++k) {
                    const int bit = (lane + 64 * k) * g.vb;
                    wi[k] = bit >> 5;
                    wi1[k] = wi[k] + 1 < K::VW ? wi[k] + 1 : wi[k];
                    sh[k] = bit & 31;
                }
                const uint32_t vmask = (1u << g.vb) - 1u;
                const bool vcross = (32 % g.vb) != 0;        // a code may straddle two words
                // the fused step at d = 64 copies the block's value words word-major wherever the
                // codes never straddle (1 or 2 bits: 2 or 4 words a row)
                static_assert(VB_MAX <= 3, "codes that never straddle a word are 1 or 2 bits wide");
                const bool crow_ok = STEP && CPL == 1 && !vcross;
                const uint64_t vcmax = (uint64_t)uni64(S.vcmax);
                int32_t vcr[8];                             // the value centroids (0 past nv)
#pragma unroll
                for (int c = 0; c < 8; ++c) vcr[c] = S.vc32[c];
                const int32_t pev = uni32(S.expt[0]);       // p of an event token: LUT(0)
                const int64_t dm = tabs->delta_max;
                SegMeta *meta = ck.meta + ((int64_t)chain * GF + h) * ck.pool + off;
                int32_t *segS = ck.segS + (((int64_t)chain * GF + h) * ck.pool + off) * D;
                // P: the open run's sum of terms so far, in int32: exact, because
                // |every prefix sum| <= B < 2^31 unless FLAG_WIDE is set.
                // hiP, loP: per channel, the largest and smallest P over the open run
                int32_t P[CPL], hiP[CPL], loP[CPL];
#pragma unroll
                for (int k = 0; k < CPL; ++k) P[k] = hiP[k] = loP[k] = 0;
                int seg = 0;                  // runs closed so far
                int64_t Lc = 0, Bc = 0;       // sums of p and of the term bounds so far
                int64_t Ls = 0, Bs = 0;       // the same where the open run began
                int64_t fkey = 0;             // the open run's event: (entry + 1) << 16 | f
                bool wide = false;
                bool trk_prev = false;        // the previous block of entries tracked prefix sums
                for (int a0 = 0; a0 < n_act; a0 += 64) {
                    // Lane = entry: decode entry a0 + lane. An event's p is LUT(0)
                    // and its LUT value is the factor f opening its run; a candidate
                    // whose p is 0 adds exactly nothing, so its bound term is 0.
                    const int e = a0 + lane;
                    const bool in = e < n_act;
                    const uint32_t r = in ? S.u.ph.rec[h][e] : 0u;
                    const int tl_i = (int)(r & 1023u);
                    const bool ev_i = in && ((r >> 10) & 1u);
                    const int val_i = exp_lut((int64_t)(r >> 11), S.expt, dm);
                    const int32_t p_i = in ? (ev_i ? pev : val_i) : 0;
                    const int32_t w_i = (int32_t)S.u.ph.vn[tl_i] * p_i;       // |w| <= 2^30
                    if constexpr (STEP && CPL == 1) {
                        if (crow_ok) {
#pragma unroll
                            for (int w = 0; w < 4; ++w)
                                if (w < 2 * g.vb && w < K::VW) S.nr.crow[h][w][lane] = S.u.ph.vw[tl_i][w];
                        }
                    }
                    // the entry's term for every value code: floor(w * c[code] / 2^acc_shift),
                    // the per-entry 64-bit products done once for all channels
                    if (g.vb <= 2) {
                        // codes of at most 2 bits index the first four terms only
                        int32_t tv[4];
#pragma unroll
                        for (int c = 0; c < 4; ++c) tv[c] = (int32_t)(((int64_t)w_i * vcr[c]) >> acc_shift);
                        *(int4 *)&S.qt.tt[h][lane][0] = make_int4(tv[0], tv[1], tv[2], tv[3]);
                    } else {
                        int32_t tv[8];
#pragma unroll
                        for (int c = 0; c < 8; ++c) tv[c] = (int32_t)(((int64_t)w_i * vcr[c]) >> acc_shift);
                        *(int4 *)&S.qt.tt[h][lane][0] = make_int4(tv[0], tv[1], tv[2], tv[3]);
                        *(int4 *)&S.qt.tt[h][lane][4] = make_int4(tv[4], tv[5], tv[6], tv[7]);
                    }
                    const uint64_t aw = (uint64_t)(w_i < 0 ? -(int64_t)w_i : (int64_t)w_i);
                    const int64_t bw_i = w_i != 0 ? (int64_t)((aw * vcmax) >> acc_shift) + 1 : 0;
                    const uint64_t evm = __ballot(ev_i);
                    // prefix sums of p and of the term bounds over the block (p <= 2^15, so
                    // 64 of them fit 32 bits)
                    const int64_t lp = Lc + (int64_t)wave_scan_add32((uint32_t)p_i);
                    const int64_t bp = Bc + wave_scan64<OpAdd64>(bw_i, 0);
                    // Tracking: any run with entries in this block has a bound of at
                    // most B (block end) - B (where the run open at the block start
                    // began). A run that starts tracking mid-way bounds its earlier
                    // prefix sums by its bound so far; one that tracks keeps tracking
                    // to its end, since its bound only grows.
                    const bool trk = SEQ && readlane64(bp, 63) - Bs > TRACK_B;
                    if (trk && !trk_prev) {
                        const int32_t b0 = (int32_t)(Bc - Bs);    // <= TRACK_B
#pragma unroll
                        for (int k = 0; k < CPL; ++k) {
                            hiP[k] = hiP[k] > b0 ? hiP[k] : b0;
                            loP[k] = loP[k] < -b0 ? loP[k] : -b0;
                        }
                    }
                    trk_prev = trk;
                    // L and B of every run an event of this block closes: prefix sums
                    // over the entries, less their values where that run began (at
                    // the previous event, or where the open run began before the
                    // block -- prefix sums never decrease, so an exclusive max-scan
                    // over the events finds it). f comes the same way, keyed by entry.
                    // Only event entries read them, so a block without one skips them.
                    int64_t Lr = 0, Br = 0;
                    if (evm) {
                        const int64_t lx = lp - p_i, bx = bp - bw_i;              // before the entry
                        const int64_t key = ev_i ? (int64_t)(e + 1) << 16 | val_i : fkey;
                        const int64_t lb = wave_shr1_64(wave_scan64<OpMax64>(ev_i ? lx : Ls, Ls), Ls);
                        const int64_t bb = wave_shr1_64(wave_scan64<OpMax64>(ev_i ? bx : Bs, Bs), Bs);
                        const int64_t kb = wave_shr1_64(wave_scan64<OpMax64>(key, fkey), fkey);
                        Lr = lx - lb;   // at an event: the run it closes
                        Br = bx - bb;
                        if (ev_i) {
                            wide = wide || Br > ACC_HI;
                            if (!own) {
                                const int ri = seg + (int)__builtin_amdgcn_mbcnt_hi(
                                                         (uint32_t)(evm >> 32),
                                                         __builtin_amdgcn_mbcnt_lo((uint32_t)evm, 0u));
                                pub64(&meta[ri].lf, (uint64_t)Lr | ((uint64_t)(kb & 0xFFFF) << 32));
                            }
                        }
                        const int le = 63 - __clzll((long long)evm);        // the block's last event
                        Ls = readlane64(lx, le);
                        Bs = readlane64(bx, le);
                        fkey = readlane64(key, le);
                    }
                    Lc = readlane64(lp, 63);
                    Bc = readlane64(bp, 63);
                    // Lane = channel: each channel's term of the entries in order, NG at
                    // a time (independent LDS reads: the code's word pair, then the table
                    // entry), then the group's entries in one of three ways.
                    constexpr int NG = CPL == 1 ? 16 : 8;
                    const int cnt = n_act - a0 < 64 ? n_act - a0 : 64;
                    const int roff_i = tl_i * (K::VW * 4);       // the entry's value words, bytes
                    if constexpr (STEP && CPL == 1) {
                        if (crow_ok && !evm && cnt == 64) {
                            // A full block without an event (the common block of a flat
                            // softmax): its 64 entries in one straight run, so that the reads
                            // are issued well ahead of the adds that wait for them.
                            // Every word first, then every table read: LDS returns in order, so a
                            // word read issued after a table read would wait for it.
                            uint32_t cw[64];
                            int32_t cb[64];
#pragma unroll
                            for (int j = 0; j < 64; j += 4)
                                *(uint4 *)&cw[j] = *(const uint4 *)&S.nr.crow[h][wi[0]][j];
                            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                            for (int j = 0; j < 64; ++j)
                                cb[j] = S.qt.tt[h][j][__builtin_amdgcn_ubfe(cw[j], (uint32_t)sh[0], (uint32_t)g.vb)];
                            if (SEQ && trk) {
#pragma unroll
                                for (int j = 0; j < 64; ++j) {
                                    P[0] += cb[j];
                                    hiP[0] = P[0] > hiP[0] ? P[0] : hiP[0];
                                    loP[0] = P[0] < loP[0] ? P[0] : loP[0];
                                }
                            } else {
#pragma unroll
                                for (int j = 0; j < 64; ++j) P[0] += cb[j];
                            }
                            continue;
                        }
                    }
                    for (int j0 = 0; j0 < cnt; j0 += NG) {
                        int32_t cv[NG][CPL];
                        if (vcross) {
#pragma unroll
                            for (int jj = 0; jj < NG; ++jj) {
                                // past cnt: token 0 and a stale table row, read but never added
                                const uint32_t *row = (const uint32_t *)((const char *)&S.u.ph.vw[0][0] +
                                                                         __builtin_amdgcn_readlane(roff_i, j0 + jj));
#pragma unroll
                                for (int k = 0; k < CPL; ++k) {
                                    // the code's word and the next (a 3-bit code may cross into it;
                                    // past a row's last word the bits read are never used)
                                    const uint32_t lo = row[wi[k]];
                                    const uint32_t hi = row[wi[k] + 1];
                                    cv[jj][k] = S.qt.tt[h][j0 + jj][__builtin_amdgcn_alignbit(hi, lo, sh[k]) & vmask];
                                }
                            }
                        } else if constexpr (STEP && CPL == 1) {
                            // the block's words word-major (crow_ok holds): entry j's at a fixed
                            // offset, one bit-field extract for the code
#pragma unroll
                            for (int jj = 0; jj < NG; ++jj) {
                                const uint32_t word = S.nr.crow[h][wi[0]][j0 + jj];
                                cv[jj][0] = S.qt.tt[h][j0 + jj][__builtin_amdgcn_ubfe(word, (uint32_t)sh[0],
                                                                                       (uint32_t)g.vb)];
                            }
                            // keeps these table reads in this branch: merged with the other
                            // branch's, their addresses lose the entry's constant offset
                            __builtin_amdgcn_sched_barrier(0);
                        } else {
                            // the codes never cross a word (vb divides 32): one read per entry
#pragma unroll
                            for (int jj = 0; jj < NG; ++jj) {
                                const uint32_t *row = (const uint32_t *)((const char *)&S.u.ph.vw[0][0] +
                                                                         __builtin_amdgcn_readlane(roff_i, j0 + jj));
#pragma unroll
                                for (int k = 0; k < CPL; ++k)
                                    cv[jj][k] = S.qt.tt[h][j0 + jj][(row[wi[k]] >> sh[k]) & vmask];
                            }
                        }
                        const int ng = cnt - j0 < NG ? cnt - j0 : NG;
                        const uint32_t gev = (uint32_t)(evm >> j0) & ((1u << ng) - 1u);
                        if (!gev && !(SEQ && trk)) {
                            // no event and no prefix tracking: the entries only add (only the
                            // chunk's last group is partial)
                            if (ng == NG) {
#pragma unroll
                                for (int jj = 0; jj < NG; ++jj)
#pragma unroll
                                    for (int k = 0; k < CPL; ++k) P[k] += cv[jj][k];
                            } else {
#pragma unroll
                                for (int jj = 0; jj < NG; ++jj)
#pragma unroll
                                    for (int k = 0; k < CPL; ++k) P[k] += jj < ng ? cv[jj][k] : 0;
                            }
                            continue;
                        }
                        if constexpr (SEQ) {
                            if (!trk) {
                                // Events, no tracking: an event closes the open run, whose
                                // bound Br came from the entry pass. Chunk 0 folds the run
                                // into its state, acc = floor((acc + S) * f / 2^15) (no clamp
                                // inside the run), and l alike; a later chunk publishes it.
                                auto events = [&](auto own_c) __attribute__((always_inline)) {
                                    constexpr bool OWN = decltype(own_c)::value;
#pragma unroll
                                    for (int jj = 0; jj < NG; ++jj) {
                                        if ((gev >> jj) & 1u) {
                                            const int j = j0 + jj;
                                            const int32_t bj = __builtin_amdgcn_readlane((int)Br, j);
                                            if (OWN) {
                                                const int32_t f = __builtin_amdgcn_readlane(val_i, j);   // <= 2^15
                                                l0 = ((l0 + (uint32_t)__builtin_amdgcn_readlane((int)Lr, j)) * f) >>
                                                     PROB_FRAC;
#pragma unroll
                                                for (int k = 0; k < CPL; ++k) {
                                                    if (!fits(acc0[k], bj)) wide = true;
                                                    acc0[k] = (AccT)(((int64_t)(acc0[k] + P[k]) * f) >> PROB_FRAC);
                                                }
                                            } else {
#pragma unroll
                                                for (int k = 0; k < CPL; ++k)
                                                    pub32(&segS[(int64_t)seg * D + lane + 64 * k], (uint32_t)P[k]);
                                                if (lane == 0) pub64(&meta[seg].b, (uint64_t)(uint32_t)bj);
                                            }
#pragma unroll
                                            for (int k = 0; k < CPL; ++k) P[k] = 0;
                                            ++seg;
                                        }
#pragma unroll
                                        for (int k = 0; k < CPL; ++k) P[k] += jj < ng ? cv[jj][k] : 0;
                                    }
                                };
                                if (own)
                                    events(std::true_type{});
                                else
                                    events(std::false_type{});
                                continue;
                            }
                        }
                        // Prefix tracking (a run whose bound may pass TRACK_B): entry by entry.
                        if (!gev) {
                            // no event in the group: no branch per entry (an entry past the
                            // chunk adds 0, which leaves P and its extremes as they are; only
                            // the chunk's last group is partial)
                            if (ng == NG) {
#pragma unroll
                                for (int jj = 0; jj < NG; ++jj)
#pragma unroll
                                    for (int k = 0; k < CPL; ++k) {
                                        P[k] += cv[jj][k];
                                        hiP[k] = P[k] > hiP[k] ? P[k] : hiP[k];
                                        loP[k] = P[k] < loP[k] ? P[k] : loP[k];
                                    }
                            } else {
#pragma unroll
                                for (int jj = 0; jj < NG; ++jj)
#pragma unroll
                                    for (int k = 0; k < CPL; ++k) {
                                        P[k] += jj < ng ? cv[jj][k] : 0;
                                        hiP[k] = P[k] > hiP[k] ? P[k] : hiP[k];
                                        loP[k] = P[k] < loP[k] ? P[k] : loP[k];
                                    }
                            }
                            continue;
                        }
#pragma unroll
                        for (int jj = 0; jj < NG; ++jj) {
                            const int j = j0 + jj;
                            if (j < cnt) {
                                if ((evm >> j) & 1ull) {
                                    // the event closes the open run
                                    if (own) {
                                        const int64_t f = (uint32_t)__builtin_amdgcn_readlane(val_i, j);
                                        l0 = ((l0 + readlane64(Lr, j)) * f) >> PROB_FRAC;
                                        const int32_t bj = (int32_t)readlane64(Br, j);
#pragma unroll
                                        for (int k = 0; k < CPL; ++k) {
                                            if (SEQ && !fits(acc0[k], trk ? run_peak(hiP[k], loP[k]) : bj)) wide = true;
                                            acc0[k] = (AccT)(((int64_t)(AccT)(acc0[k] + (AccT)P[k]) * f) >> PROB_FRAC);
                                        }
                                    } else {
#pragma unroll
                                        for (int k = 0; k < CPL; ++k)
                                            pub32(&segS[(int64_t)seg * D + lane + 64 * k], (uint32_t)P[k]);
                                        if (SEQ) {
                                            const int64_t m = trk ? wave_max_i64(peak_of<CPL>(hiP, loP))
                                                                  : readlane64(Br, j);
                                            if (lane == 0) pub64(&meta[seg].b, (uint64_t)m);
                                        }
                                    }
#pragma unroll
                                    for (int k = 0; k < CPL; ++k) P[k] = hiP[k] = loP[k] = 0;
                                    ++seg;
                                }
#pragma unroll
                                for (int k = 0; k < CPL; ++k) {
                                    P[k] += cv[jj][k];
                                    if (SEQ && trk) {
                                        hiP[k] = P[k] > hiP[k] ? P[k] : hiP[k];
                                        loP[k] = P[k] < loP[k] ? P[k] : loP[k];
                                    }
                                }
                            }
                        }
                    }
                }
                // the open run closes at the end of the chunk
                wide = wide || Bc - Bs > ACC_HI;
                if (own) {
#pragma unroll
                    for (int k = 0; k < CPL; ++k) {
                        if (SEQ && !fits(acc0[k], trk_prev ? run_peak(hiP[k], loP[k])
                                                           : (int32_t)(Bc - Bs > ACC_HI ? ACC_HI : Bc - Bs)))
                            wide = true;
                        acc0[k] += (AccT)P[k];
                    }
                    l0 += Lc - Ls;
                } else {
                    const int64_t m = !SEQ ? 0 : trk_prev ? wave_max_i64(peak_of<CPL>(hiP, loP))
                                                          : (Bc - Bs > ACC_HI ? ACC_HI : Bc - Bs);
                    if (lane == 0) {
                        pub64(&meta[seg].lf, (uint64_t)(Lc - Ls) | ((uint64_t)(fkey & 0xFFFF) << 32));
                        pub64(&meta[seg].b, (uint64_t)m);
                    }
#pragma unroll
                    for (int k = 0; k < CPL; ++k)
                        pub32(&segS[(int64_t)seg * D + lane + 64 * k], (uint32_t)P[k]);
                }
                if (__ballot(wide)) flags |= FLAG_WIDE;
            }
            n_ev0 = n_ev;
            flags0 = flags;
            if (!own) {
                // The header goes out with the run sums: the replay reads it only after
                // this wave has counted itself done, which waits for all of them.
                ChunkHdr *hp = &ck.hdr[((int64_t)chain * ck.max_chunks + chunk) * GF + h];
                if (lane == 0) {
                    pub64(&hp->w1, S.mabs);
                    pub64(&hp->w0, (uint64_t)(uint32_t)n_seg | ((uint64_t)(uint32_t)flags << 16) |
                                       ((uint64_t)(S.ovf & 0xFFFF) << 24) | ((uint64_t)ck.ep << 40));
                }
            }
        } else if (!ok && wv < GF && !own) {
            // q failed its range check: the chain goes to the serial path, which counts its own
            ChunkHdr *hp = &ck.hdr[((int64_t)chain * ck.max_chunks + chunk) * GF + wv];
            if (lane == 0) {
                pub64(&hp->w1, 0);
                pub64(&hp->w0, 1ull | ((uint64_t)ck.ep << 40));
            }
        }

        // -- phase 5: the last workgroup of the chain replays -----------------------
        // A chunk counts itself done once the stores of its head waves (their runs
        // and headers; waves 0 and 1 also the new row; wave 0 the chain's fallback
        // flag) have completed, so the workgroup whose count completes the chain
        // finds everything out. One count per chunk: the counts of a chain meet at
        // one address, where the device applies them one at a time. Chunk 0's
        // state stays in the registers when its workgroup is the last (its many
        // rescale events make it the slowest); otherwise it publishes the state
        // after counting, and the last workgroup waits for its header.
        if (wv < GF) stores_done();
        __syncthreads();
        if (tid == 0) {
            const unsigned prior = __hip_atomic_fetch_add(&ck.done[chain], 1u, __ATOMIC_RELAXED,
                                                          __HIP_MEMORY_SCOPE_AGENT);
            S.last = prior == (unsigned)(nch - 1);
        }
        __syncthreads();
        const bool last = S.last != 0;
        if (own && !last && wv < GF) {
            // chunk 0's state in its slot: acc (|acc| < 2^31 whenever it is used)
            // and l | events << 32
            const int h = wv;
            const int64_t base = (int64_t)chain * GF + h;
#pragma unroll
            for (int k = 0; k < CPL; ++k) pub32(&ck.segS[base * ck.pool * D + lane + 64 * k], (uint32_t)acc0[k]);
            ChunkHdr *hp = &ck.hdr[((int64_t)chain * ck.max_chunks) * GF + h];
            if (lane == 0) {
                pub64(&ck.meta[base * ck.pool].lf, (uint64_t)(uint32_t)l0 | ((uint64_t)(uint32_t)n_ev0 << 32));
                pub64(&hp->w1, ok ? S.mabs : 0ull);
            }
            stores_done();
            if (lane == 0)
                pub64(&hp->w0, 1ull | ((uint64_t)(uint32_t)flags0 << 16) |
                                   ((uint64_t)(ok ? S.ovf & 0xFFFF : 0) << 24) | ((uint64_t)ck.ep << 40));
        }
        if (last) {
            // Every head's wave merges its statistics into the call's totals with global
            // atomics. The device applies the atomics on one word one at a time, so with
            // many chains ending together (C3's 512 chains: 132 -> 120 us per launch) the
            // heads merge in LDS first and the chain sends them once. With few chains the
            // heads send their own, in parallel; the fused step (one token per sequence,
            // C2's 8 chains: 28.5 -> 29.0 us the other way, its SGPR spills up by a third
            // with the merge compiled in) always does.
            const bool merge_stats = !STEP && n_chains > 32;
            if (merge_stats && tid < 4) S.red[4][tid] = 0;    // the heads' merged statistics
            if (merge_stats && tid == 4) S.red[5][0] = 0;     // and how many heads have merged theirs
            const bool hw = wv < GF;              // wave h < GF replays query head h, lane = channel
            const int h = hw ? wv : 0;
            constexpr int HPL = HMAX / 64;
            constexpr int SB = 64 / CPL;          // runs per batch
            AccT aw[CPL];
#pragma unroll
            for (int k = 0; k < CPL; ++k) aw[k] = 0;
            int64_t l = 0;
            bool unsafe = false;                  // a run's certificate failed (sequential mode)
            unsigned long long events = 0;
            bool fb = !ok;
            const bool hdr_stats = ok;
            if (hw) {
                const ChunkHdr *hdr = ck.hdr + (int64_t)chain * ck.max_chunks * GF + h;  // chunk c: hdr[c * GF]
                const SegMeta *meta = ck.meta + ((int64_t)chain * GF + h) * ck.pool;
                const int32_t *segS = ck.segS + ((int64_t)chain * GF + h) * ck.pool * D;
                uint16_t *sl = S.u.rp.slot[h];
                const int zslot = ck.pool - 1;    // a valid slot for the lanes past a batch to read
                const uint32_t ep = ck.ep;
                auto cur = [ep](uint64_t w) __attribute__((always_inline)) { return (uint32_t)(w >> 40) == ep; };
                // A chunk whose look-back timed out flagged the chain before its header
                // (every chunk has counted itself done: read with the headers).
                const bool chain_fb = get32(&ck.chain_fb[chain]) == ep;
                // Chunk 0's state: in the registers, or out of its slot once its header is up.
                int flags = 0;
                int64_t ovf = 0, mabs = 0;
                if (own) {
#pragma unroll
                    for (int k = 0; k < CPL; ++k) aw[k] = acc0[k];
                    l = l0;
                    events = (unsigned long long)n_ev0;
                    flags = flags0;
                    if (h == 0 && lane == 0) {
                        ovf = (int64_t)S.ovf;
                        mabs = (int64_t)S.mabs;
                    }
                } else if (!fb) {
                    uint64_t h0 = 0;
                    int spins = 0;
                    fb = ck.spin_limit == 0;
                    while (!fb) {
                        h0 = (uint64_t)uni64((int64_t)get64(&hdr[0].w0));   // all lanes, one word
                        if (cur(h0)) break;
                        if (++spins > ck.spin_limit) {
                            fb = true;
                            break;
                        }
                        __builtin_amdgcn_s_sleep(1);
                    }
                    if (!fb) {
                        flags = (int)((h0 >> 16) & 0xFF);
#pragma unroll
                        for (int k = 0; k < CPL; ++k) aw[k] = (AccT)(int32_t)get32(segS + lane + 64 * k);
                        const uint64_t lf = get64(&meta[0].lf);
                        l = (int64_t)(uint32_t)lf;
                        events = lf >> 32;
                        if (h == 0 && lane == 0) {
                            ovf = (int64_t)((h0 >> 24) & 0xFFFF);
                            mabs = (int64_t)get64(&hdr[0].w1);
                        }
                    }
                }
                // The runs of chunks 1 .. nch-1 in order: one header load per lane and
                // 64 chunks, then a scan of the run counts lists them by slot in LDS.
                int total = 0;
                uint64_t w0[HPL], w1[HPL];
#pragma unroll
                for (int i = 0; i < HPL; ++i) {
                    const int c = 1 + lane + 64 * i;
                    w0[i] = 0;
                    w1[i] = 0;
                    if (c < nch) {
                        w0[i] = get64(&hdr[(int64_t)c * GF].w0);
                        if (h == 0) w1[i] = get64(&hdr[(int64_t)c * GF].w1);
                    }
                }
#pragma unroll
                for (int i = 0; i < HPL; ++i) {
                    if (64 * i + 1 >= nch) break;
                    const int c = 1 + lane + 64 * i;
                    const bool in = c < nch;
                    if (in && !cur(w0[i])) flags |= FLAG_POOL;     // cannot happen: it counted itself done
                    // A header lists more than SLOTS runs only with FLAG_POOL (its runs did not
                    // fit and were not published); one without it would send the walk past the
                    // chunk's slots: a fault. Either way the chain takes the serial path.
                    const bool over = in && (int)(w0[i] & 0xFFFF) > SLOTS;
                    if (over) {
                        if (!((w0[i] >> 16) & FLAG_POOL)) st->fault = 1;
                        flags |= FLAG_POOL;
                    }
                    const int n = in && !over ? (int)(w0[i] & 0xFFFF) : 0;
                    flags |= in ? (int)((w0[i] >> 16) & 0xFF) : 0;
                    ovf += in ? (int64_t)((w0[i] >> 24) & 0xFFFF) : 0;
                    mabs = (int64_t)w1[i] > mabs ? (int64_t)w1[i] : mabs;
                    const int incl = (int)wave_scan_add32((uint32_t)n);
                    const int start = total + incl - n;
                    total += __builtin_amdgcn_readlane(incl, 63);
                    for (int j = 0; j < n && start + j < NSEG; ++j)
                        sl[start + j] = (uint16_t)((slot_base(c) + j) | (j ? RUN_EVENT : 0));
                }
                total = uni32(total);
                if (__ballot(flags != 0) || total > NSEG) fb = true;
                if (chain_fb) fb = true;
                if (h == 0) {
                    ovf = wave_sum_i64(ovf);
                    mabs = wave_max_i64(mabs);
                    if (lane == 0) {
                        S.ovf = (unsigned long long)ovf;
                        S.mabs = (unsigned long long)mabs;
                    }
                }
                fb = __builtin_amdgcn_readfirstlane((int)fb) != 0;
                wave_sync();
                // The walk, SB runs at a time. Lane i < SB holds run i's list entry
                // and loads its L, f and largest |prefix sum| m; every lane loads its
                // channels' run sums (the slot ids read back with readlane). Per run
                // the walk checks |acc| + m against 2^31 (no clamp can fire inside
                // it) and adds the run sum; l is brought up to date from lane prefix
                // sums at each event (before its rescale) and at the end of the batch.
                for (int g0 = 0; g0 < total && !fb; g0 += SB) {
                    const int nb = total - g0 < SB ? total - g0 : SB;     // uniform
                    const int nblk = (nb + 7) >> 3;                        // blocks of 8 runs
                    const bool mine = lane < nb;
                    uint32_t ent = mine ? (uint32_t)sl[g0 + lane] : (uint32_t)zslot;
                    // Every slot index is checked against the pool before its row is read: one
                    // past it (a fault: the list is built from checked headers) is not loaded,
                    // and the chain takes the serial path.
                    if (__ballot((int)(ent & (RUN_EVENT - 1)) >= ck.pool)) {
                        if (lane == 0) st->fault = 1;
                        fb = true;
                        break;
                    }
                    // lane i: the byte offset of run i's row (lanes past the batch: the spare
                    // slot, whose contents are read but never added)
                    const uint32_t roff = (ent & (RUN_EVENT - 1)) * (uint32_t)(D * 4);
                    const char *sbase = (const char *)segS + 4 * lane;
                    int32_t sv[SB][CPL];
#pragma unroll
                    for (int blk = 0; blk < SB / 8; ++blk) {
                        if (blk < nblk) {
                            // no branch between the loads of a block; past the batch
                            // they read the spare slot
#pragma unroll
                            for (int i = 8 * blk; i < 8 * blk + 8; ++i) {
                                const uint32_t o = (uint32_t)__builtin_amdgcn_readlane((int)roff, i);
#pragma unroll
                                for (int k = 0; k < CPL; ++k) sv[i][k] = (int32_t)get32(sbase + o + 256 * k);
                            }
                        } else {
#pragma unroll
                            for (int i = 8 * blk; i < 8 * blk + 8; ++i)
#pragma unroll
                                for (int k = 0; k < CPL; ++k) sv[i][k] = 0;
                        }
                    }
                    uint64_t mlf = 0, mb = 0;
                    if (mine) {
                        const int si = (int)(ent & (RUN_EVENT - 1));
                        mlf = get64(&meta[si].lf);
                        mb = get64(&meta[si].b);
                    }
                    const uint64_t evm = SEQ ? __ballot(mine && (ent & RUN_EVENT)) : 0ull;
                    // inclusive prefix sums of L and B over the batch's runs
                    const int64_t PL = wave_scan64<OpAdd64>(mine ? (int64_t)(uint32_t)mlf : 0, 0);
                    int64_t done_L = 0;                 // prefix sum already added to l
                    // |acc| only shrinks at a rescale (f <= 2^15) and grows by at most a
                    // run's peak per run, so |acc at a block's start| + the sum of the
                    // block's peaks certifies its 8 runs at once; only where that bound
                    // fails does the walk check run by run
                    const int64_t PB = SEQ ? wave_scan64<OpAdd64>(mine ? (int64_t)(uint32_t)mb : 0, 0) : 0;
#pragma unroll
                    for (int blk = 0; blk < SB / 8; ++blk) {
                        if (blk < nblk) {
                            const uint32_t bev = SEQ ? (uint32_t)(evm >> (8 * blk)) & 0xFFu : 0u;
                            bool bcheck = false;
                            if (SEQ) {
                                const int64_t bsum = readlane64(PB, 8 * blk + 7) - (blk ? readlane64(PB, 8 * blk - 1) : 0);
                                int64_t amax = 0;
#pragma unroll
                                for (int k = 0; k < CPL; ++k) {
                                    const int64_t a = aw[k] < 0 ? -(int64_t)aw[k] : (int64_t)aw[k];
                                    amax = a > amax ? a : amax;
                                }
                                bcheck = __ballot(amax + bsum > ACC_HI) != 0ull;
                            }
                            if (!bev && !bcheck) {
                                // no rescale and no certificate to check in these 8 runs:
                                // they only add (the runs past the batch read the spare slot,
                                // which is never added)
#pragma unroll
                                for (int k = 0; k < CPL; ++k) {
                                    AccT v[8];
#pragma unroll
                                    for (int r = 0; r < 8; ++r) v[r] = 8 * blk + r < nb ? (AccT)sv[8 * blk + r][k] : (AccT)0;
                                    aw[k] += ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
                                }
                                continue;
                            }
#pragma unroll
                            for (int i = 8 * blk; i < 8 * blk + 8; ++i) {
                                if (SEQ && ((evm >> i) & 1ull)) {
                                    const int64_t pl = i ? readlane64(PL, i - 1) : 0;
                                    l += pl - done_L;
                                    done_L = pl;
                                    const int64_t f =
                                        (uint32_t)__builtin_amdgcn_readlane((int)(mlf >> 32), i);
#pragma unroll
                                    for (int k = 0; k < CPL; ++k)
                                        aw[k] = (AccT)(((int64_t)aw[k] * f) >> PROB_FRAC);
                                    l = wmul(l, f) >> PROB_FRAC;
                                    ++events;
                                }
                                if (SEQ && bcheck) {
                                    const int32_t m = __builtin_amdgcn_readlane((int)(uint32_t)mb, i);
#pragma unroll
                                    for (int k = 0; k < CPL; ++k) unsafe = unsafe || !fits((int32_t)aw[k], m);
                                }
#pragma unroll
                                for (int k = 0; k < CPL; ++k) aw[k] += i < nb ? (AccT)sv[i][k] : (AccT)0;
                            }
                        }
                    }
                    l += readlane64(PL, nb - 1) - done_L;
                    if (SEQ && __ballot(unsafe)) fb = true;
                }
            }
            int64_t acc[CPL];
#pragma unroll
            for (int k = 0; k < CPL; ++k) acc[k] = (int64_t)aw[k];
            __syncthreads();   // the replay buffers are dead; the serial path reuses the LDS
            const int qh = qhead(g, kvh, h);
            int32_t *orow = out + ((int64_t)b * g.n_q + qh) * D;
            if (!hw || !real_head(g, h)) {
                // (a duplicate slot: no output, no statistics)
            } else if (fb) {
                // The serial path counts score statistics only when the headers did not.
                // The fused step's new row came from another workgroup: acquire it.
                if (STEP) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
                const int32_t *qrow;
                if constexpr (STEP)
                    qrow = &S.nr.qi[h][0];
                else
                    qrow = q + ((int64_t)b * g.n_q + qh) * D;
                serial_head<CPL, K::RS>(g, tabs, S.kc, S.vc, qrow, b, kvh, T, SEQ ? 0 : 1, !hdr_stats,
                                        S.u.fb[h], orow, st);
                if (lane == 0) atomicAdd(&st->serial_fallbacks, 1ull);
            } else {
                unsigned long long aovf = 0;
                if (!SEQ) {
#pragma unroll
                    for (int k = 0; k < CPL; ++k)
                        if (acc[k] < ACC_LO || acc[k] > ACC_HI) {
                            ++aovf;
                            acc[k] = acc[k] < ACC_LO ? ACC_LO : ACC_HI;
                        }
                }
                const Recip rc = reciprocal(l);
                int64_t amax = 0;
#pragma unroll
                for (int k = 0; k < CPL; ++k) {
                    orow[lane + 64 * k] = (int32_t)(wmul(acc[k], rc.r) >> rc.shift);
                    const int64_t a = acc[k] < 0 ? -acc[k] : acc[k];
                    amax = a > amax ? a : amax;
                }
                amax = wave_max_i64(amax);
                if (!SEQ) aovf = (unsigned long long)wave_sum_i64((int64_t)aovf);
                if (lane == 0 && !merge_stats) {
                    atomicMax(&st->n_tokens, (unsigned long long)T);
                    if (events) atomicAdd(&st->rescale_events, events);
                    atomicMax(&st->max_abs_acc, (unsigned long long)amax);
                    if (aovf) atomicAdd(&st->acc_overflows, aovf);
                } else if (lane == 0) {
                    unsigned long long *m = (unsigned long long *)&S.red[4][0];
                    if (events) atomicAdd(&m[0], events);
                    atomicMax(&m[1], (unsigned long long)amax);
                    if (aovf) atomicAdd(&m[2], aovf);
                    atomicOr(&m[3], 1ull);
                }
            }
            if (!merge_stats) {
                // the chain's score statistics, once (from the headers when they cover it)
                if (hw && h == 0 && lane == 0 && hdr_stats) {
                    if (S.ovf) atomicAdd(&st->score_overflows, S.ovf);
                    atomicMax(&st->max_abs_score, S.mabs);
                }
            } else if (hw && lane == 0) {
                // The statistics of the heads that did not take the serial path (which
                // merges its own), merged in LDS; the last head's wave to get here sends
                // them once for the chain.
                unsigned long long *m = (unsigned long long *)&S.red[4][0];
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");    // this head's merge first
                if (atomicAdd((unsigned int *)&S.red[5][0], 1u) == GF - 1) {
                    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
                    if (m[3]) {
                        atomicMax(&st->n_tokens, (unsigned long long)T);
                        if (m[0]) atomicAdd(&st->rescale_events, m[0]);
                        atomicMax(&st->max_abs_acc, m[1]);
                        if (m[2]) atomicAdd(&st->acc_overflows, m[2]);
                    }
                    // the chain's score statistics, once (from the headers when they cover it)
                    if (hdr_stats) {
                        if (S.ovf) atomicAdd(&st->score_overflows, S.ovf);
                        atomicMax(&st->max_abs_score, S.mabs);
                    }
                }
            }
            if (tid == 0) ck.done[chain] = 0;    // every workgroup of the chain has counted itself
        }
    }
}

// ---------------------------------------------------------------------------
// query staging in front of a standalone attend (d = 128)
// ---------------------------------------------------------------------------

// One workgroup per (sequence, KV head); wave h stages query head h of the
// group (query.h).
template <int CPL>
__global__ void __launch_bounds__(GF * 64) qprep_kernel(Geom g, const Tables *__restrict__ tabs,
                                                        const int32_t *__restrict__ q, double *qd,
                                                        int32_t *qok, DevStats *st) {
    __shared__ int ok_s;
    const int chain = blockIdx.x, h = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int b = chain / g.n_kv, kvh = chain % g.n_kv;
    if (threadIdx.x == 0) ok_s = 1;
    __syncthreads();
    int32_t v[CPL];
    load_vec<CPL>(q + ((int64_t)b * g.n_q + qhead(g, kvh, h)) * g.d, g.d, v);
    const bool ok = stage_query_head<CPL>(v, g.d, h, qd + (int64_t)chain * g.d * GF, tabs->kc_absmax,
                                          real_head(g, h) ? &st->range_errors : nullptr);
    if (lane == 0 && !ok) atomicAnd(&ok_s, 0);
    __syncthreads();
    if (threadIdx.x == 0) qok[chain] = ok_s;
}

// Whether a sequential attend reads staged query rows (a small launch first
// when the caller has not staged them) rather than every workgroup staging
// them in LDS. Read as scalar FMA operands they keep the d = 128 chunk kernel
// within 128 VGPRs, two workgroups per CU, where the LDS-query kernel needs
// about 150; at d = 64 both fit, and the extra launch would only add its
// dispatch. The fused decode step is the LDS-query kernel, so it runs at d = 64.
template <int D>
constexpr bool stage_queries_first() { return D > 64; }

bool chunked_fused_step(const Geom &g) { return g.d <= 64; }

template <int D, int KB>
static hipError_t launch_fast(hipStream_t s, const Geom &g, const Tables *t, const int32_t *q,
                              int32_t *out, const int64_t *len, const Chunked &ck, int two_pass,
                              bool q_staged, const StepIn *step, LaunchEv ev, DevStats *st,
                              int64_t grid_chunks) {
    const unsigned chains = (unsigned)(g.batch * g.n_kv);
    const StepIn si = step ? *step : StepIn{};
    if (two_pass) {
        if (step) return hipErrorInvalidValue;
        // the chunk-max kernel stages the query rows for the chunk kernel when the caller has not
        dim3 grid((unsigned)grid_chunks, chains), block(CT);
        if (q_staged)
            hipExtLaunchKernelGGL((chunk_max_kernel<D, KB, true>), grid, block, 0, s, ev.start, nullptr,
                                  0, g, t, q, ck.qd, ck.qok, len, ck, st);
        else
            hipExtLaunchKernelGGL((chunk_max_kernel<D, KB, false>), grid, block, 0, s, ev.start, nullptr,
                                  0, g, t, q, ck.qd, ck.qok, len, ck, st);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        hipExtLaunchKernelGGL((chunk_kernel<D, KB, false, true, false>), grid, block, 0, s, nullptr,
                              ev.stop, 0, g, t, q, ck.qd, ck.qok, out, len, ck, st, si);
        return hipGetLastError();
    }
    dim3 grid((unsigned)grid_chunks * chains), block(CT);
    if constexpr (stage_queries_first<D>()) {
        if (step) return hipErrorInvalidValue;
        if (!q_staged) {
            hipLaunchKernelGGL((qprep_kernel<D / 64>), dim3(chains), dim3(GF * 64), 0, s, g, t, q,
                               ck.qd, ck.qok, st);
            hipError_t e = hipGetLastError();
            if (e != hipSuccess) return e;
        }
        hipExtLaunchKernelGGL((chunk_kernel<D, KB, true, true, false>), grid, block, 0, s, ev.start,
                              ev.stop, 0, g, t, q, ck.qd, ck.qok, out, len, ck, st, si);
    } else if (step) {
        hipExtLaunchKernelGGL((chunk_kernel<D, KB, true, false, true>), grid, block, 0, s, ev.start,
                              ev.stop, 0, g, t, q, ck.qd, ck.qok, out, len, ck, st, si);
    } else {
        // rotated int32 queries in q (staged ones as well: the write kernel also stores them there)
        hipExtLaunchKernelGGL((chunk_kernel<D, KB, true, false, false>), grid, block, 0, s, ev.start,
                              ev.stop, 0, g, t, q, ck.qd, ck.qok, out, len, ck, st, si);
    }
    return hipGetLastError();
}

int64_t chunked_max_chunks(int64_t capacity) { return (capacity + CHUNK - 1) / CHUNK; }

bool chunked_supported(const Geom &g, int64_t capacity) {
    return g.G == GF && (g.d == 64 || g.d == 128) && g.kb >= 2 && g.kb <= 4 && g.vb >= 1 &&
           g.vb <= VB_MAX && chunked_max_chunks(capacity) <= HMAX;
}


// The run slots of every chunk, plus one spare slot that is never written: the
// replay's lanes past the end of a batch load from it (and add nothing), so the
// loads of a batch need no branch.
int64_t chunked_pool_slots(int64_t max_chunks) { return 1 + (max_chunks - 1) * SLOTS + 1; }

static void carve(const Geom &g, int64_t max_chunks, int64_t pool, uint8_t *p, Chunked *ck,
                  size_t *total) {
    const int64_t chains = (int64_t)g.batch * g.n_kv;
    size_t o = 0;
    auto take = [&](size_t n) {
        const size_t at = o;
        o += (n + 255) / 256 * 256;
        return p ? p + at : nullptr;
    };
    // the words read before their epoch is known to be current come first (scratch_layout)
    Chunked c{};
    c.cmax = (int64_t *)take(chains * max_chunks * GF * sizeof(int64_t));
    c.status = (unsigned long long *)take(chains * max_chunks * GF * 2 * sizeof(unsigned long long));
    c.hdr = (ChunkHdr *)take(chains * max_chunks * GF * sizeof(ChunkHdr));
    c.done = (unsigned int *)take(chains * sizeof(unsigned int));
    c.chain_fb = (unsigned int *)take(chains * sizeof(unsigned int));
    c.meta = (SegMeta *)take(chains * GF * pool * sizeof(SegMeta));
    c.segS = (int32_t *)take(chains * GF * pool * g.d * sizeof(int32_t));
    c.qd = (double *)take(chains * g.d * GF * sizeof(double));
    c.qok = (int32_t *)take(chains * sizeof(int32_t));
    c.max_chunks = (int32_t)max_chunks;
    c.pool = (int32_t)pool;
    if (ck) *ck = c;
    if (total) *total = o;
}

void chunked_layout_facts(const Geom &g, int64_t max_chunks, int64_t *f) {
    // carved at a stand-in base address (never dereferenced): the areas' offsets
    uint8_t *const base = (uint8_t *)((uintptr_t)1 << 40);
    const int64_t pool = chunked_pool_slots(max_chunks);
    const int64_t chains = (int64_t)g.batch * g.n_kv;
    Chunked c;
    size_t total = 0;
    carve(g, max_chunks, pool, base, &c, &total);
    auto off = [&](const void *q) { return (int64_t)((const uint8_t *)q - base); };
    // every area 256-aligned, in carve order, each ending at or before the next one's start
    const int64_t at[] = {off(c.cmax), off(c.status), off(c.hdr), off(c.done), off(c.chain_fb),
                          off(c.meta), off(c.segS), off(c.qd), off(c.qok), (int64_t)total};
    const int64_t sz[] = {chains * max_chunks * GF * 8, chains * max_chunks * GF * 2 * 8,
                          chains * max_chunks * GF * (int64_t)sizeof(ChunkHdr), chains * 4, chains * 4,
                          chains * GF * pool * (int64_t)sizeof(SegMeta), chains * GF * pool * g.d * 4,
                          chains * g.d * GF * 8, chains * 4};
    bool ok = true;
    for (int i = 0; i < 9; ++i) ok = ok && at[i] % 256 == 0 && at[i] + sz[i] <= at[i + 1];
    f[0] = max_chunks;
    f[1] = pool;
    f[2] = SLOTS;
    f[3] = max_chunks > 1 ? slot_base((int)max_chunks - 1) + SLOTS : 1;    // chunk 0: one state slot
    f[4] = NSEG;
    f[5] = HMAX;
    f[6] = (int64_t)total;
    f[7] = off(c.meta);
    f[8] = ok ? 1 : 0;
    f[9] = CHUNK;
    f[10] = RUN_EVENT;
}

size_t chunked_scratch_bytes(const Geom &g, int64_t max_chunks, int64_t pool) {
    size_t n = 0;
    carve(g, max_chunks, pool, nullptr, nullptr, &n);
    return n;
}

void chunked_query_area(const Geom &g, int64_t max_chunks, int64_t pool, void *scratch,
                        double **qd, int32_t **qok) {
    Chunked ck;
    carve(g, max_chunks, pool, (uint8_t *)scratch, &ck, nullptr);
    *qd = ck.qd;
    *qok = ck.qok;
}

__global__ void clear_scratch_kernel(uint4 *p, int64_t n16) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += (int64_t)gridDim.x * blockDim.x)
        p[i] = make_uint4(0u, 0u, 0u, 0u);
}

#if INSITU_CHUNK_TPT == 2
// (one definition: the 512-token build uses these)
hipError_t scratch_begin(hipStream_t s, ChunkScratch &cs, uint32_t *ep) {
    const uint32_t call = cs.calls++;
    // 1 .. 2^14 - 1: the zeroed scratch of a new buffer is never current. At
    // the wrap the words go back to zero (no epoch); every chain's completion
    // counter is zero between attends already.
    if (call % EPOCH_MASK == 0 && call > 0) {
        const int64_t n16 = (int64_t)(cs.bytes / 16);     // carve() rounds every area to 256 B
        const unsigned blocks = (unsigned)(n16 < 65536 * 256 ? (n16 + 255) / 256 : 65536);
        if (n16 > 0) {
            hipLaunchKernelGGL(clear_scratch_kernel, dim3(blocks), dim3(256), 0, s, (uint4 *)cs.p, n16);
            const hipError_t e = hipGetLastError();
            if (e != hipSuccess) return e;
        }
    }
    *ep = call % EPOCH_MASK + 1;
    return hipSuccess;
}

hipError_t scratch_layout(hipStream_t s, ChunkScratch &cs, uint64_t layout, size_t front) {
    if (layout == cs.layout) return hipSuccess;
    const int64_t n16 = (int64_t)(front / 16);          // carve() rounds every area to 256 B
    if (n16 > 0) {
        const unsigned blocks = (unsigned)(n16 < 65536 * 256 ? (n16 + 255) / 256 : 65536);
        hipLaunchKernelGGL(clear_scratch_kernel, dim3(blocks), dim3(256), 0, s, (uint4 *)cs.p, n16);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    cs.layout = layout;
    return hipSuccess;
}
#endif

hipError_t launch_attend_chunked(hipStream_t s, const Geom &g, const Tables *t, const int32_t *q,
                                 int32_t *out, const int64_t *len, ChunkScratch &cs,
                                 uint32_t ep, int64_t max_chunks, int64_t pool, int two_pass,
                                 bool q_staged, const StepIn *step, LaunchEv ev, DevStats *st,
                                 int64_t carve_batch, int64_t grid_chunks) {
    const int64_t chains = (int64_t)g.batch * g.n_kv;
    if (max_chunks > HMAX || chains > 65535 || max_chunks * chains > 0x7fffffff)
        return hipErrorInvalidValue;
    // the grid: the chunks of the longest sequence (workgroups past a chain's last
    // chunk have nothing to do), at most the layout's
    if (grid_chunks < 1 || grid_chunks > max_chunks) grid_chunks = max_chunks;
    if (carve_batch < g.batch) carve_batch = g.batch;
    Geom gc = g;
    gc.batch = (int32_t)carve_batch;
    Chunked ck;
    size_t bytes = 0;
    carve(gc, max_chunks, pool, (uint8_t *)cs.p, &ck, &bytes);
    if (bytes > cs.bytes || ep == 0 || ep > EPOCH_MASK) return hipErrorInvalidValue;
    ck.ep = ep;
    ck.spin_limit = cs.spin_limit;
    const uint64_t layout = ((uint64_t)max_chunks << 48) ^ ((uint64_t)pool << 24) ^ ((uint64_t)carve_batch << 8) ^
                            (uint64_t)g.n_kv ^ ((uint64_t)g.d << 40) ^ (1ull << 62);
    {
        const hipError_t e = scratch_layout(s, cs, layout, (size_t)((uint8_t *)ck.meta - (uint8_t *)cs.p));
        if (e != hipSuccess) return e;
    }
#define INSITU_FAST(DD, KK)                                                          \
    if (g.d == DD && g.kb == KK)                                                     \
        return launch_fast<DD, KK>(s, g, t, q, out, len, ck, two_pass, q_staged, step, ev, st, grid_chunks);
    INSITU_FAST(64, 2)
    INSITU_FAST(64, 3)
    INSITU_FAST(64, 4)
    INSITU_FAST(128, 2)
    INSITU_FAST(128, 3)
    INSITU_FAST(128, 4)
#undef INSITU_FAST
    return hipErrorInvalidValue;
}

#if INSITU_CHUNK_TPT == 1
}  // namespace c512
#endif
}  // namespace insitu
