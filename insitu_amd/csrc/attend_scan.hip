// The scan attend: attend_online (ops/attention.py:451-513) over a context split
// into 1,024-token chunks, bit-exact with the sequential reference, laid out for
// the latency of one decode step on MI355X.
//
// One workgroup of 1,024 threads (16 waves, 4 per SIMD) per (chunk, sequence, KV
// head); thread i owns token chunk*1024 + i. Workgroups are numbered chunk-major,
// so every predecessor of a chunk has a smaller number. Phases:
//
//  0. Loads, issued first: the tables, the group's G query rows (waves 0..G-1),
//     the token's key words, value words and norms. In a fused decode step the
//     query rows are the wire rows, and the chunk that holds the new token also
//     loads the wire k and v rows.
//  1. The query waves rotate their rows (fused step), check that every score
//     of the group stays an exact fp64 integer (||q||_1 * max|c| < 2^51), and
//     stage them as fp64 in the workgroup's own slot of global memory. After a
//     barrier every wave reads them with scalar loads, so the score FMAs take q
//     as a scalar operand and the score loop's LDS traffic is the centroid
//     reads alone. The new token's k and v rows are rotated, encoded, packed,
//     stored, and swapped into the registers of the thread that scores it.
//  2. Scores: sum_ch q[ch] * c[code_ch] in fp64 FMA (exact: every partial sum is
//     an integer below 2^51), the int64 norm multiply and >> 24, the 48-bit clamp.
//  3. The chunk maximum, then a decoupled look-back on the maxima of the chunks
//     before (relaxed agent-scope atomics, words tagged with the call's epoch,
//     bounded waits): M_in, the running maximum where the chunk starts.
//  4. Candidates: with M_in known, a prefix-max scan gives every token's running
//     maximum m_t. The rescale events are the tokens above the maximum before
//     them; a token is a candidate if m_t - s_t < delta_max (otherwise p = 0
//     exactly). Each head's candidates are listed in token order with their p,
//     and every candidate carries its run: the number of events up to it. A
//     run is a maximal stretch between events; inside it the terms
//     floor(v_norm * p * c_v[code] / 2^23) only add.
//  5. Run sums, on every wave: units of 64 listed candidates. Lane = candidate:
//     the candidate's terms for every value code, and per run the sums of p (L)
//     and of the term bounds |w| * max|c_v| / 2^23 + 1 (B). Lane = channel: each
//     channel's sum of terms per run (int32, exact while B < 2^31). Runs that
//     cross a unit boundary meet in LDS atomics; int32 addition is associative.
//  6. Chunk 0 replays its own runs from acc = l = 0 and publishes one state;
//     every other chunk but the last publishes its runs (S, L, f, B).
//  7. The last chunk of the chain waits for the headers of all the others, then
//     replays acc = floor(acc * f / 2^15) + S, l = floor(l * f / 2^15) + L over
//     every run in order, finalizes and writes Q16. That is exactly the
//     reference recurrence provided the per-token int32 clamp never fires,
//     which holds if |acc at a run's start| + B <= 2^31 - 1 for every run
//     (checked per channel where acc is exact); a head that fails, or whose
//     chunks flagged a run pool overflow, a run bound past 2^31, inexact fp64
//     scores or a look-back that gave up, is recomputed on the serial path
//     (serial_head.h).
#include "row_codec.h"
#include "serial_head.h"
#include "wave.h"

namespace insitu {

namespace {

constexpr int SC_NT = 1024;                 // threads per workgroup
constexpr int SC_NW = SC_NT / 64;           // waves
constexpr int SC_CHUNK = SC_NT;             // tokens per workgroup, one per thread
constexpr int SC_MAXCH = 4096;              // chunks per sequence (4M tokens)
constexpr int SC_EPOCH_MASK = (1 << 14) - 1;
constexpr int SF_POOL = 1;                  // more runs than the slots hold
constexpr int SF_WIDE = 2;                  // a run's term bound reached 2^31
constexpr int SF_QEXACT = 4;                // the group's fp64 scores may be inexact
constexpr int SF_LOOKBACK = 8;              // a wait on a predecessor gave up

constexpr unsigned long long LB_AGG = 1ull << 62, LB_INC = 2ull << 62, LB_FLAGS = 3ull << 62;
constexpr double SC_DOT_LIMIT = 2251799813685248.0;       // 2^51
constexpr double SC_MAGIC = 6755399441055744.0;           // 1.5 * 2^52
constexpr int64_t SC_MAGIC_BITS = 0x4338000000000000LL;

typedef __attribute__((address_space(4))) const double cdouble;

struct RunMeta {
    uint32_t L;      // sum of p over the run (< 2^26); chunk 0's state: l
    uint32_t f;      // the factor opening the run (run >= 1); chunk 0's state: its event count
    uint64_t B;      // sum of the term bounds over the run
};
// In the replay's copy of a run's metadata, f also says how the run is applied.
constexpr uint32_t RM_RESCALE = 1u << 31;   // a run after a chunk's first: scale by f, then add
constexpr uint32_t RM_STATE = 1u << 30;     // chunk 0's state: acc, l and the event count
constexpr uint32_t RM_VALUE = 0xFFFFu;

// Look-back words: flag (bits 62-63) | epoch (48-61) | score - SCORE_LO (0-47).
__device__ __forceinline__ unsigned long long lb_pack(unsigned long long flag, unsigned ep, int64_t v) {
    return flag | (unsigned long long)ep << 48 | (unsigned long long)(v - SCORE_LO);
}
__device__ __forceinline__ unsigned long long lb_flag(unsigned long long w, unsigned ep) {
    return ((unsigned)(w >> 48) & SC_EPOCH_MASK) == ep ? w & LB_FLAGS : 0ull;
}
__device__ __forceinline__ int64_t lb_val(unsigned long long w) {
    return (int64_t)(w & ((1ull << 48) - 1)) + SCORE_LO;
}
__device__ __forceinline__ void put64(void *p, uint64_t v) {
    __hip_atomic_store((uint64_t *)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void put32(void *p, uint32_t v) {
    __hip_atomic_store((uint32_t *)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t take64(const void *p) {
    return __hip_atomic_load((uint64_t *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t take32(const void *p) {
    return __hip_atomic_load((uint32_t *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Wait until this thread's stores have completed (the vector memory counter).
__device__ __forceinline__ void sc_stores_done() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_s_waitcnt(0x0F70);          // vmcnt(0)
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
__device__ __forceinline__ int64_t sc_dbl_to_i64(double x) {
    return (int64_t)__double_as_longlong(x + SC_MAGIC) - SC_MAGIC_BITS;
}
// exp_lut (ExpLut.__call__, attention.py:153-159) on a delta held as a double: an
// integer >= 0 below 2^49. min(delta, delta_max) < 2^20, its product with
// log2(e) in Q16 is below 2^37 and the scale by 2^-24 is exact, so one fp64
// multiply and a truncation give the flat index floor(d * LOG2E_Q16 / 2^24).
__device__ __forceinline__ int32_t exp_lut_d(double delta, const int32_t *table, double delta_max) {
    constexpr double K = (double)LOG2E_Q16 / (double)(1 << (ACC_FRAC + ACC_FRAC - LUT_BITS));
    const uint32_t u = (uint32_t)(fmin(delta, delta_max) * K);
    const int32_t v = table[u & 255] >> (u >> LUT_BITS);
    return u < (uint32_t)LUT_SPAN ? v : 0;
}
__device__ __forceinline__ int64_t wave_shl1_64(int64_t v, int64_t id) {
    return dpp64<0x130>(id, v);                  // wave_shl:1, lane i <- lane i + 1
}

// Max-reductions and scans on scores held as doubles: a score is an integer
// below 2^48, exact in fp64, and v_max_f64 is one instruction where an int64
// max is three.
template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ double dppd(double fill, double v) {
    return __longlong_as_double(dpp64<CTRL, ROWS>(__double_as_longlong(fill), __double_as_longlong(v)));
}
__device__ __forceinline__ double readlane_d(double v, int l) {
    return __longlong_as_double(readlane64(__double_as_longlong(v), l));
}
__device__ __forceinline__ double wave_max_d(double v) {
    v = fmax(v, dppd<DPP_QUAD_1032>(v, v));
    v = fmax(v, dppd<DPP_QUAD_2301>(v, v));
    v = fmax(v, dppd<DPP_ROW_HALF_MIRROR>(v, v));
    v = fmax(v, dppd<DPP_ROW_MIRROR>(v, v));
    return fmax(fmax(readlane_d(v, 0), readlane_d(v, 16)), fmax(readlane_d(v, 32), readlane_d(v, 48)));
}
// inclusive prefix maximum in lane order over the wave (id: below every value)
__device__ __forceinline__ double wave_scan_max_d(double v, double id) {
    v = fmax(v, dppd<DPP_ROW_SHR1>(id, v));
    v = fmax(v, dppd<DPP_ROW_SHR2>(id, v));
    v = fmax(v, dppd<DPP_ROW_SHR4>(id, v));
    v = fmax(v, dppd<DPP_ROW_SHR8>(id, v));
    v = fmax(v, dppd<DPP_ROW_BCAST15, 0xA>(id, v));
    v = fmax(v, dppd<DPP_ROW_BCAST31, 0xC>(id, v));
    return v;
}
// inclusive prefix maximum and sum within each row of 16 lanes
__device__ __forceinline__ double row_scan_max_d(double v, double id) {
    v = fmax(v, dppd<DPP_ROW_SHR1>(id, v));
    v = fmax(v, dppd<DPP_ROW_SHR2>(id, v));
    v = fmax(v, dppd<DPP_ROW_SHR4>(id, v));
    v = fmax(v, dppd<DPP_ROW_SHR8>(id, v));
    return v;
}
__device__ __forceinline__ uint32_t row_scan_add32(uint32_t v) {
    v += dpp32<DPP_ROW_SHR1>(0u, v);
    v += dpp32<DPP_ROW_SHR2>(0u, v);
    v += dpp32<DPP_ROW_SHR4>(0u, v);
    v += dpp32<DPP_ROW_SHR8>(0u, v);
    return v;
}

template <int D, int KB, int VB, int G>
struct ScanShape {
    static constexpr int CPL = D / 64;
    static constexpr int KBYTES = D * KB / 8, KW = KBYTES / 4;
    static constexpr int KFULL = KBYTES / 16, KHALF = (KBYTES % 16) ? 1 : 0, KPL = KFULL + KHALF;
    static constexpr int VBYTES = D * VB / 8, VWD = VBYTES / 4;
    static constexpr int VFULL = VBYTES / 16, VHALF = (VBYTES % 16) ? 1 : 0, VPL = VFULL + VHALF;
    static constexpr int NK = 1 << KB, NV = 1 << VB;
    static constexpr uint32_t KMASK = NK - 1, VMASK = NV - 1;
    static constexpr int POOL = 16 * G;            // run slots in LDS, shared by the heads
    static constexpr int RP = 8;                   // runs a chunk other than the first publishes per head
    static constexpr int GRP = 32 / G;             // channels per score group
    static constexpr int CB = (8192 / D) / G;      // chunks per replay batch
    static constexpr int RB = CB * G + 32;         // replay run slots: first runs, then those events open
    static constexpr int RS = (KBYTES + VBYTES + 4 + 3) / 4 * 4;
    static_assert(KBYTES % 16 == 0 || KBYTES % 16 == 8, "key planes are 16 or 8 bytes");
    static_assert(VBYTES % 16 == 0 || VBYTES % 16 == 8, "value planes are 16 or 8 bytes");
    static_assert(GRP * KB <= 32, "a score group's codes sit in one 32-bit window");
};

template <int D, int KB, int VB, int G>
struct ScanLds {
    using SH = ScanShape<D, KB, VB, G>;
    // the tables the inner loops read come first: their addresses fit the
    // instructions' 16-bit LDS offset
    double kcf[16];
    int32_t expt[256];
    int32_t vc32[8];
    int64_t kc[16];
    int64_t vc[8];
    int64_t vcmax;
    struct Phase {
        uint32_t rec[G][SC_CHUNK];          // a head's candidates in token order: token | run << 10 | p << 16
        uint32_t vw[SC_CHUNK][SH::VWD];     // value words of every token
        int16_t vn[SC_CHUNK];               // value norms
        int32_t tt[SC_NW][64][SH::NV];      // per wave: a unit's terms [candidate][code]
    };
    struct Replay {
        int32_t rs[SH::RB][D];              // a batch's runs in walk order, head by head
        RunMeta rm[SH::RB];                 // their metadata, flags in f (RM_*)
        uint64_t hw[SH::CB * G];            // the batch's headers, (chunk, head) pairs chunk-major
        int16_t src[SH::CB * G * SH::RP];   // the run behind each slot: pair * RP + run
        int32_t hb[G], hn[G], hbad[G];      // per head: first slot, slots, a pair unusable
        int32_t nslot;                      // slots in use
    };
    struct NewRow {
        int64_t bnd[2][255];
        uint8_t codes[2][MAX_D];
    };
    union {
        Phase ph;
        Replay rp;
        NewRow nr;
        SerialLds<SH::RS> fb[G];
    } u;
    int32_t S[SH::POOL][D];                 // this chunk's run sums: head h's runs from slot rb[h]
    unsigned long long Lr[SH::POOL], Br[SH::POOL];
    uint16_t evf[SH::POOL];                 // the factor opening each run
    int32_t qi[G][D];                       // the group's rotated queries, for the serial path
    uint32_t row[32];                       // the fused step's new row
    int64_t norms[2];
    double red[SC_NW][G];                   // per wave: the largest score per head
    double wt[G][16];                       // per wave: its largest score (heads with events)
    int64_t min_[G], lmax[G];
    uint32_t cnt[G][16], evn[G][16];
    int32_t flags[G];
    int32_t qok, zero;
    unsigned long long ovf, mabs;
};

struct ScanArgs {
    Geom g;
    const Tables *tabs;
    const int32_t *q;           // rotated int32 queries (batch, n_q, d); the wire rows come in si
    int32_t *out;
    const int64_t *len;
    StepIn si;
    DevStats *st;
    unsigned long long *status; // [chain][mc][G][2] look-back words: inclusive, aggregate
    unsigned long long *hdr;    // [chain][mc][G] epoch << 40 | flags << 16 | runs
    RunMeta *meta;              // [chain][mc][G][RP]
    int32_t *runs;              // [chain][mc][G][RP][D]
    double *qd;                 // [chain * mc + chunk][D][G]: each workgroup's staged queries
    int32_t mc;                 // chunks per chain the scratch is laid out for
    uint32_t ep;
    int32_t spin_limit;
};

// A published run's metadata with its RM_* flags. src = pair * RP + run within the
// batch whose first chunk is c0 (pairs are (chunk, head), chunk-major); bp is the
// index of the batch's first run.
template <int G, int RP>
__device__ __forceinline__ RunMeta scan_meta(const ScanArgs &a, int64_t bp, int src, int c0) {
    const uint64_t lf = take64(&a.meta[bp + src]);
    RunMeta m;
    m.L = (uint32_t)lf;
    m.B = take64(&a.meta[bp + src].B);
    const int r = src % RP, c = c0 + src / RP / G;
    m.f = (uint32_t)(lf >> 32) | (c == 0 ? RM_STATE : (r > 0 ? RM_RESCALE : 0u));
    return m;
}

// The value code of channel c in a token's value words.
template <int VB, int VWD>
__device__ __forceinline__ uint32_t vcode(const uint32_t *vw, int c) {
    const int bit = c * VB, wi = bit >> 5, sh = bit & 31;
    if (VB == 1 || VB == 2 || VB == 4 || VB == 8) return (vw[wi] >> sh) & ((1u << VB) - 1u);
    const int wi1 = wi + 1 < VWD ? wi + 1 : wi;      // a code crossing into the next word
    return __builtin_amdgcn_alignbit(vw[wi1], vw[wi], sh) & ((1u << VB) - 1u);
}

// One workgroup per CU: the staged queries live in SGPRs during the score loop,
// and a second 16-wave workgroup would not fit beside them on gfx950. A launch
// of at most 256 workgroups (ctx <= 32,768 at batch 1, 8 KV heads) runs in one
// round; past that the chunks a CU finishes make room for the rest.
template <int D, int KB, int VB, int G, bool STEP>
__global__ void __launch_bounds__(SC_NT, 1) scan_kernel(ScanArgs a) {
    using SH = ScanShape<D, KB, VB, G>;
    constexpr int CPL = SH::CPL;
    __shared__ ScanLds<D, KB, VB, G> S;
    const Geom &g = a.g;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n_chains = g.batch * g.n_kv;
    const int chunk = (int)(blockIdx.x / (unsigned)n_chains);
    const int chain = (int)(blockIdx.x % (unsigned)n_chains);
    const int b = chain / g.n_kv, kvh = chain % g.n_kv;
    const int64_t T = a.len[b] + (STEP ? 1 : 0);
    const int nch = T > 0 ? (int)((T + SC_CHUNK - 1) / SC_CHUNK) : 1;
    if (chunk >= nch) return;
    const bool last = chunk == nch - 1;
    // Stores and returnless atomics count in a wave's vector memory counter until they
    // complete, and the waits of the waves that publish, look back and replay (waves
    // 0 .. G - 1) drain that counter: writes that are on no chain are made by the
    // last wave instead.
    const bool side = tid == SC_NT - 64;
    if (STEP && chunk == 0 && kvh == 0 && side) a.si.len_out[b] = T;
    const int64_t t0 = (int64_t)chunk * SC_CHUNK;
    const int64_t t = t0 + tid;
    const bool in = t < T;
    const int score_shift = CENT_FRAC + g.norm_frac;
    const int acc_shift = CENT_FRAC + g.norm_frac + PROB_FRAC - ACC_FRAC;
    const int64_t wg_slot = (int64_t)chain * a.mc + chunk;
    const int64_t pair0 = wg_slot * G;                   // this chunk's (chain, chunk, head 0)
    const double LO = (double)SCORE_LO;

    // -- phase 0: loads, small ones first ---------------------------------------------
    const int64_t kc_t = tid < SH::NK ? a.tabs->kc[tid] : 0;
    const int64_t vc_t = tid < SH::NV ? a.tabs->vc[tid] : 0;
    const int32_t ex_t = tid < 256 ? a.tabs->exp_table[tid] : 0;
    int32_t qv[CPL];
    int32_t kvv[CPL];
    if (wv < G) {
        const int32_t *src = STEP ? a.si.qw + ((int64_t)b * g.n_q + kvh * G + wv) * D
                                  : a.q + ((int64_t)b * g.n_q + kvh * G + wv) * D;
        load_vec<CPL>(src, D, qv);
    } else if (STEP && last && wv < G + 2) {
        load_vec<CPL>((wv == G ? a.si.kw : a.si.vw) + ((int64_t)b * g.n_kv + kvh) * D, D, kvv);
    }
    const uint8_t *hb = plane_ptr(g, b, kvh, 0);
    const int64_t tc = in ? t : 0;                       // past the end: token 0, unused
    uint32_t kw[SH::KW + 1], vwv[SH::VWD], nw;
    kw[SH::KW] = 0;
#pragma unroll
    for (int p = 0; p < SH::KFULL; ++p) {
        const uint4 v = *(const uint4 *)(hb + p * g.span + tc * 16);
        kw[4 * p] = v.x;
        kw[4 * p + 1] = v.y;
        kw[4 * p + 2] = v.z;
        kw[4 * p + 3] = v.w;
    }
    if (SH::KHALF) {
        const uint2 v = *(const uint2 *)(hb + SH::KFULL * g.span + tc * 8);
        kw[4 * SH::KFULL] = v.x;
        kw[4 * SH::KFULL + 1] = v.y;
    }
#pragma unroll
    for (int p = 0; p < SH::VFULL; ++p) {
        const uint4 v = *(const uint4 *)(hb + (SH::KPL + p) * g.span + tc * 16);
        vwv[4 * p] = v.x;
        vwv[4 * p + 1] = v.y;
        vwv[4 * p + 2] = v.z;
        vwv[4 * p + 3] = v.w;
    }
    if (SH::VHALF) {
        const uint2 v = *(const uint2 *)(hb + (SH::KPL + SH::VFULL) * g.span + tc * 8);
        vwv[4 * SH::VFULL] = v.x;
        vwv[4 * SH::VFULL + 1] = v.y;
    }
    nw = *(const uint32_t *)(hb + (SH::KPL + SH::VPL) * g.span + tc * 4);

    if (tid < 16) {
        S.kc[tid] = kc_t;
        S.kcf[tid] = (double)kc_t;
    }
    if (tid < 8) {
        S.vc[tid] = vc_t;
        S.vc32[tid] = (int32_t)vc_t;
    }
    if (tid < 256) S.expt[tid] = ex_t;
    if (wv == 0) {
        const int64_t m = wave_max_i64(vc_t < 0 ? -vc_t : vc_t);
        if (lane == 0) S.vcmax = m;
    }
    if (tid < G) S.flags[tid] = 0;
    if (tid == 0) {
        S.qok = 1;
        S.zero = 0;
        S.ovf = S.mabs = 0;
    }
    if (STEP && last) stage_bounds(a.tabs, g, S.u.nr.bnd);
    __syncthreads();

    // -- phase 1: stage the queries; the fused step's new row --------------------------
    if (wv < G) {
        if (STEP)
            rotate_loaded<CPL>(qv, D, a.si.rounds, a.si.sg, qv, chunk == 0 ? &a.st->range_errors : nullptr);
        int64_t l1 = 0, bad = 0;
        double *qdst = a.qd + wg_slot * D * G;
#pragma unroll
        for (int k = 0; k < CPL; ++k) {
            const int c = lane + 64 * k;
            const int64_t x = qv[k];
            qdst[c * G + wv] = (double)x;
            S.qi[wv][c] = qv[k];
            l1 += x < 0 ? -x : x;
            bad += (x >= Q_ROT_LIMIT || x <= -Q_ROT_LIMIT) ? 1 : 0;
        }
        l1 = wave_sum_i64(l1);          // < 2^38: exact as a double
        bad = wave_sum_i64(bad);
        if (chunk == 0 && lane == 0 && bad) atomicAdd(&a.st->range_errors, (unsigned long long)bad);
        if (lane == 0 && !((double)l1 * a.tabs->kc_absmax < SC_DOT_LIMIT)) atomicAnd(&S.qok, 0);
        sc_stores_done();               // the staged rows are in memory before the barrier
    } else if (STEP && last && wv < G + 2) {
        const int f = wv - G;           // 0: key, 1: value
        rotate_loaded<CPL>(kvv, D, a.si.rounds, a.si.sg, kvv, &a.st->range_errors);
        int64_t x[CPL];
#pragma unroll
        for (int k = 0; k < CPL; ++k) x[k] = kvv[k];
        const int64_t n = encode_field<CPL>(x, D, g.norm_frac, S.u.nr.bnd[f], (1 << (f == 0 ? KB : VB)) - 1,
                                            S.u.nr.codes[f]);
        if (lane == 0) S.norms[f] = n;
    }
    __syncthreads();
    if (STEP && last) {
        // pack and store the new row, then hand it to the thread of token T - 1
        const int nwords = g.row_bytes / 4;
        if (wv == G && lane < nwords) {
            const uint32_t w = pack_row_word(g, S.u.nr.codes, S.norms[0], S.norms[1], lane);
            S.row[lane] = w;
            *row_word_ptr(g, b, kvh, T - 1, lane) = w;
            sc_stores_done();             // in memory before the serial path could read it
        }
        __syncthreads();
        if (t == T - 1) {
#pragma unroll
            for (int i = 0; i < SH::KW; ++i) kw[i] = S.row[i];
#pragma unroll
            for (int i = 0; i < SH::VWD; ++i) vwv[i] = S.row[SH::KW + i];
            nw = S.row[SH::KW + SH::VWD];
        }
    }

    // -- phase 2: scores ----------------------------------------------------------------
    const bool qok = S.qok != 0;
    double sd[G];                        // the clamped scores as doubles; LO past the end
#pragma unroll
    for (int h = 0; h < G; ++h) sd[h] = LO;
    {
#pragma unroll
        for (int i = 0; i < SH::VWD; ++i) S.u.ph.vw[tid][i] = vwv[i];
        S.u.ph.vn[tid] = (int16_t)(nw >> 16);
    }
    if (qok) {
        // the staged rows by scalar loads: the address depends on an LDS read after the
        // barrier, so the loads cannot move above it
        cdouble *qs = (cdouble *)((uint64_t)(a.qd + wg_slot * D * G) +
                                  (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane(S.zero));
        double acc[G];
#pragma unroll
        for (int h = 0; h < G; ++h) acc[h] = 0.0;
#pragma unroll
        for (int grp = 0; grp < D / SH::GRP; ++grp) {
            const int bo = SH::GRP * KB * grp, wi = bo >> 5, sh = bo & 31;
            const uint32_t win = sh == 0 ? kw[wi] : __builtin_amdgcn_alignbit(kw[wi + 1], kw[wi], sh);
            double cv[SH::GRP];
#pragma unroll
            for (int i = 0; i < SH::GRP; ++i) cv[i] = S.kcf[(win >> (i * KB)) & SH::KMASK];
#pragma unroll
            for (int i = 0; i < SH::GRP; ++i)
#pragma unroll
                for (int h = 0; h < G; ++h) acc[h] = fma(qs[(SH::GRP * grp + i) * G + h], cv[i], acc[h]);
#pragma unroll
            for (int h = 0; h < G; ++h) asm volatile("" : "+v"(acc[h]));
        }
        const int64_t kn = sext16(nw);
        bool over = false;
        double mabs = 0.0;
#pragma unroll
        for (int h = 0; h < G; ++h) {
            int64_t v = wmul(sc_dbl_to_i64(acc[h]), kn) >> score_shift;
            const bool o = in && (v < SCORE_LO || v > SCORE_HI);
            over = over || o;
            v = v < SCORE_LO ? SCORE_LO : (v > SCORE_HI ? SCORE_HI : v);
            sd[h] = in ? (double)v : LO;
            mabs = in ? fmax(mabs, fabs((double)v)) : mabs;
        }
        if (__ballot(over)) {
            unsigned long long n = 0;
#pragma unroll
            for (int h = 0; h < G; ++h) n += in && (sd[h] == LO || sd[h] == (double)SCORE_HI) ? 1 : 0;
            n = (unsigned long long)wave_sum_i64((int64_t)n);
            if (lane == 0 && n) atomicAdd(&S.ovf, n);
        }
        mabs = wave_max_d(mabs);
        if (lane == 0) atomicMax(&S.mabs, (unsigned long long)mabs);
    }
#pragma unroll
    for (int h = 0; h < G; ++h) {
        const double m = wave_max_d(sd[h]);
        if (lane == 0) S.red[wv][h] = m;
    }
    __syncthreads();

    // -- phase 3: the chunk maximum and the maximum before the chunk -----------------------
    // Each (chunk, head) has two look-back words: [0] inclusive (the running maximum at
    // the chunk's end), [1] aggregate (the chunk's own maximum). Wave G + h publishes the
    // aggregate, so that wave h, which looks back, has no store in flight while it polls.
    if (wv >= G && wv < 2 * G) {
        const int h = wv - G;
        const double lm = wave_max_d(lane < SC_NW ? S.red[lane][h] : LO);
        if (chunk > 0 && lane == 0) put64(a.status + (pair0 + h) * 2 + 1, lb_pack(LB_AGG, a.ep, (int64_t)lm));
    }
    if (wv < G) {
        const int h = wv;
        const double lm = wave_max_d(lane < SC_NW ? S.red[lane][h] : LO);
        const int64_t local = (int64_t)lm;
        unsigned long long *my = a.status + (pair0 + h) * 2;
        int64_t run = SCORE_LO;
        bool fail = false;
        if (chunk == 0) {
            if (lane == 0) put64(my, lb_pack(LB_INC, a.ep, local));
        } else {
            int64_t base = chunk - 1;      // the predecessor lane 0 reads
            int spins = 0;
            fail = a.spin_limit == 0;
            while (!fail) {
                const int64_t pc = base - lane;
                unsigned long long flag = LB_INC;
                int64_t val = SCORE_LO;
                if (pc >= 0) {
                    const unsigned long long *w2 = a.status + (((int64_t)chain * a.mc + pc) * G + h) * 2;
                    const unsigned long long wi = take64(w2), wa = take64(w2 + 1);
                    const bool fi = lb_flag(wi, a.ep) == LB_INC;
                    flag = fi ? LB_INC : lb_flag(wa, a.ep) == LB_AGG ? LB_AGG : 0ull;
                    val = lb_val(fi ? wi : wa);
                }
                const unsigned long long inc = __ballot(flag == LB_INC);
                const int nearest = inc ? __ffsll((long long)inc) - 1 : 64;
                const unsigned long long wait = __ballot(flag == 0 && lane <= nearest);
                if (wait) {
                    if (++spins > a.spin_limit) {
                        fail = true;
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
                    continue;
                }
                const int64_t v = (int64_t)wave_max_d(lane <= nearest ? (double)val : LO);
                run = v > run ? v : run;
                if (nearest < 64) break;
                base -= 64;
            }
            const int64_t incl = run > local ? run : local;
            if (lane == 0) put64(my, lb_pack(LB_INC, a.ep, incl));
        }
        if (lane == 0) {
            S.min_[h] = run;
            S.lmax[h] = local;
            if (fail) S.flags[h] |= SF_LOOKBACK;
            if (!qok) S.flags[h] |= SF_QEXACT;
        }
    }
    __syncthreads();
    if (side && qok) {
        // this chunk's score statistics (AttentionStats.merge: overflows add, max |s| is a max)
        if (S.ovf) atomicAdd(&a.st->score_overflows, S.ovf);
        atomicMax(&a.st->max_abs_score, S.mabs);
    }

    // -- phase 4: candidates, listed in token order per head ---------------------------------
    // Lanes of a row of 16 stand for the 16 waves of one head in the cross-wave
    // prefixes (lane = head * 16 + wave, G / 4 passes).
    const double dmd = (double)a.tabs->delta_max;
    bool evh[G];
    bool anyev = false;
#pragma unroll
    for (int h = 0; h < G; ++h) {
        evh[h] = qok && __builtin_amdgcn_readfirstlane((int)(S.lmax[h] > S.min_[h])) != 0;
        anyev = anyev || evh[h];
    }
    double incl[G];
    if (anyev) {
#pragma unroll
        for (int h = 0; h < G; ++h) {
            if (!evh[h]) continue;
            incl[h] = wave_scan_max_d(sd[h], LO);
            if (lane == 63) S.wt[h][wv] = incl[h];
        }
        __syncthreads();
    }
    bool cand[G], ev[G];
    uint32_t pv[G], fv[G];
#pragma unroll
    for (int h0 = 0; h0 < G; h0 += 4) {
        // the running maximum where this wave starts, for heads h0 .. h0 + 3
        double pre[4];
        if (anyev) {
            const int hh = h0 + (lane >> 4), w = lane & 15;
            double v = LO;
            if (hh < G && evh[hh < G ? hh : 0]) v = S.wt[hh][w];
            v = dppd<DPP_ROW_SHR1>(LO, row_scan_max_d(v, LO));          // exclusive
#pragma unroll
            for (int j = 0; j < 4; ++j) pre[j] = readlane_d(v, 16 * j + wv);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int h = h0 + j;
            if (h >= G) break;
            const double M = (double)S.min_[h];
            double mi = M, me = M;                     // running maximum at and before the token
            if (evh[h]) {
                const double p0 = fmax(M, pre[j]);
                const double ex = dppd<DPP_WAVE_SHR1>(LO, incl[h]);
                mi = fmax(p0, incl[h]);
                me = fmax(p0, ex);
            }
            ev[h] = qok && in && sd[h] > me;
            const double dlt = mi - sd[h];              // an exact integer >= 0; 0 at an event
            cand[h] = qok && in && dlt < dmd;
            pv[h] = 0;
            fv[h] = 0;
            if (__ballot(cand[h])) pv[h] = cand[h] ? (uint32_t)exp_lut_d(dlt, S.expt, dmd) : 0u;
            if (__ballot(ev[h])) fv[h] = ev[h] ? (uint32_t)exp_lut_d(sd[h] - me, S.expt, dmd) : 0u;
            const uint64_t cb = __ballot(cand[h]), eb = __ballot(ev[h]);
            if (lane == 0) {
                S.cnt[h][wv] = (uint32_t)__popcll(cb);
                S.evn[h][wv] = (uint32_t)__popcll(eb);
            }
        }
    }
    __syncthreads();
    int n_rec[G], n_run[G], rb[G];
    int pool = 0;
#pragma unroll
    for (int h0 = 0; h0 < G; h0 += 4) {
        const int hh = h0 + (lane >> 4), w = lane & 15;
        const uint32_t c = hh < G ? S.cnt[hh < G ? hh : 0][w] : 0u;
        const uint32_t e = hh < G ? S.evn[hh < G ? hh : 0][w] : 0u;
        const uint32_t ic = row_scan_add32(c), ie = row_scan_add32(e);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int h = h0 + j;
            if (h >= G) break;
            n_rec[h] = __builtin_amdgcn_readlane((int)ic, 16 * j + 15);
            n_run[h] = __builtin_amdgcn_readlane((int)ie, 16 * j + 15) + 1;
            rb[h] = pool;
            pool += n_run[h];
            const int base = wv ? __builtin_amdgcn_readlane((int)ic, 16 * j + wv - 1) : 0;
            const int evb = wv ? __builtin_amdgcn_readlane((int)ie, 16 * j + wv - 1) : 0;
            const uint64_t cb = __ballot(cand[h]), eb = __ballot(ev[h]);
            const int pos = base + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(cb >> 32),
                                                                  __builtin_amdgcn_mbcnt_lo((uint32_t)cb, 0u));
            const int run = evb + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(eb >> 32),
                                                                 __builtin_amdgcn_mbcnt_lo((uint32_t)eb, 0u)) +
                            (ev[h] ? 1 : 0);
            if (cand[h] && run < 64) S.u.ph.rec[h][pos] = (uint32_t)tid | (uint32_t)run << 10 | pv[h] << 16;
            if (ev[h] && rb[h] + run < SH::POOL) S.evf[rb[h] + run] = (uint16_t)fv[h];
        }
    }
    // the run slots: every head's runs in one pool; past it, or past what a chunk
    // publishes, the head goes to the serial path
    // (a record holds a 6-bit run index: a head with 64 runs or more goes serial too)
    const bool pool_full = pool > SH::POOL;
#pragma unroll
    for (int h = 0; h < G; ++h)
        if (tid == 0 && (pool_full || n_run[h] >= 64 || (chunk > 0 && !last && n_run[h] > SH::RP)))
            S.flags[h] |= SF_POOL;
    {
        const int np = pool_full ? 0 : pool;
        for (int i = tid; i < np * D; i += SC_NT) (&S.S[0][0])[i] = 0;
        if (tid < np) {
            S.Lr[tid] = 0;
            S.Br[tid] = 0;
        }
    }
    __syncthreads();

    // -- phase 5: run sums, units of 64 candidates spread over every wave -----------------------
    {
        int nu[G];
#pragma unroll
        for (int h = 0; h < G; ++h)
            nu[h] = __builtin_amdgcn_readfirstlane(S.flags[h]) == 0 ? (n_rec[h] + 63) >> 6 : 0;
        const uint64_t vcmax = (uint64_t)S.vcmax;
        int32_t (*tt)[SH::NV] = S.u.ph.tt[wv];
        for (int u = wv;; u += SC_NW) {
            int h = -1, blk = u;
#pragma unroll
            for (int hh = 0; hh < G; ++hh) {
                if (h < 0 && blk < nu[hh]) h = hh;
                else if (h < 0) blk -= nu[hh];
            }
            if (h < 0) break;
            const int e0 = blk * 64;
            const int cnt = n_rec[h] - e0 < 64 ? n_rec[h] - e0 : 64;
            const int rbase = rb[h];
            // lane = candidate
            const bool valid = lane < cnt;
            const uint32_t rv = valid ? S.u.ph.rec[h][e0 + lane] : 0u;
            const int tok = (int)(rv & 1023u);
            const int run = valid ? (int)((rv >> 10) & 63u) : 0x7FFFFFFF;
            const int32_t p = (int32_t)(rv >> 16);
            const int32_t w = (int32_t)S.u.ph.vn[tok] * p;           // |w| <= 2^30
#pragma unroll
            for (int i = 0; i < SH::NV; ++i) tt[lane][i] = (int32_t)(((int64_t)w * S.vc32[i]) >> acc_shift);
            const uint64_t aw = (uint64_t)(w < 0 ? -(int64_t)w : (int64_t)w);
            const int64_t bnd = p > 0 ? (int64_t)((aw * vcmax) >> acc_shift) + 1 : 0;
            // per run: the sums of p and of the bounds (runs are non-decreasing along the list)
            const int prev = (int)dpp32<DPP_WAVE_SHR1>(0xFFFFFFFFu, (uint32_t)run);
            const int next = (int)dpp32<0x130>(0x7FFFFFFFu, (uint32_t)run);
            const bool start = valid && (lane == 0 || prev != run);
            const bool end = valid && (lane == cnt - 1 || next != run);
            const int64_t ip = wave_scan64<OpAdd64>(p, 0), ib = wave_scan64<OpAdd64>(bnd, 0);
            const int64_t bp = wave_scan64<OpMax64>(start ? ip - p : 0, 0);
            const int64_t bb = wave_scan64<OpMax64>(start ? ib - bnd : 0, 0);
            if (end) {
                atomicAdd(&S.Lr[rbase + run], (unsigned long long)(ip - bp));
                atomicAdd(&S.Br[rbase + run], (unsigned long long)(ib - bb));
            }
            wave_sync();
            // lane = channel, run by run: the runs of the unit start where `start` is set
            uint64_t starts = __ballot(start);
            while (starts) {
                const int j0 = __ffsll((long long)starts) - 1;
                starts &= starts - 1;
                const int j1 = starts ? __ffsll((long long)starts) - 1 : cnt;
                const int r = __builtin_amdgcn_readlane(run, j0);
                int32_t P[CPL];
#pragma unroll
                for (int k = 0; k < CPL; ++k) P[k] = 0;
                // four candidates at a time, their LDS reads issued together (a candidate
                // past the run reads candidate j1 - 1 and adds nothing)
                for (int j = j0; j < j1; j += 4) {
                    int32_t tv[4][CPL];
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        const int jj = j + u < j1 ? j + u : j1 - 1;
                        const int tk = __builtin_amdgcn_readlane(tok, jj);
#pragma unroll
                        for (int k = 0; k < CPL; ++k) tv[u][k] = tt[jj][vcode<VB, SH::VWD>(S.u.ph.vw[tk], lane + 64 * k)];
                    }
#pragma unroll
                    for (int u = 0; u < 4; ++u)
#pragma unroll
                        for (int k = 0; k < CPL; ++k) P[k] += j + u < j1 ? tv[u][k] : 0;
                }
#pragma unroll
                for (int k = 0; k < CPL; ++k) atomicAdd(&S.S[rbase + r][lane + 64 * k], P[k]);
            }
            wave_sync();
        }
    }
    __syncthreads();

    // -- phase 6: chunk 0 replays its runs; the middle chunks publish theirs --------------------
    const bool hw = wv < G;
    const int h = hw ? wv : 0;
    int64_t acc[CPL];
#pragma unroll
    for (int k = 0; k < CPL; ++k) acc[k] = 0;
    int64_t l = 0;
    unsigned long long events = 0;
    bool fb = false;
    if (hw) {
        int flags = __builtin_amdgcn_readfirstlane(S.flags[h]);
        const int nr = n_run[h], r0 = rb[h];
        if (!flags)
            for (int r = 0; r < nr; ++r)
                if (S.Br[r0 + r] > (unsigned long long)ACC_HI) flags |= SF_WIDE;
        if (chunk == 0) {
            bool unsafe = false;
            if (!flags) {
                for (int r = 0; r < nr; ++r) {
                    if (r > 0) {
                        const int64_t f = S.evf[r0 + r];
#pragma unroll
                        for (int k = 0; k < CPL; ++k) acc[k] = (acc[k] * f) >> PROB_FRAC;
                        l = (l * f) >> PROB_FRAC;
                    }
                    const int64_t B = (int64_t)S.Br[r0 + r];
#pragma unroll
                    for (int k = 0; k < CPL; ++k) {
                        const int64_t av = acc[k] < 0 ? -acc[k] : acc[k];
                        unsafe = unsafe || av + B > ACC_HI;
                        acc[k] += S.S[r0 + r][lane + 64 * k];
                    }
                    l += (int64_t)S.Lr[r0 + r];
                }
                events = (unsigned long long)(nr - 1);
            }
            fb = flags != 0 || __ballot(unsafe) != 0ull;
            if (!last) {
                // chunk 0's state, |acc| < 2^31 whenever it is used
                const int64_t pr = pair0 + h;
#pragma unroll
                for (int k = 0; k < CPL; ++k) put32(&a.runs[pr * SH::RP * D + lane + 64 * k], (uint32_t)(int32_t)acc[k]);
                if (lane == 0) {
                    put64(&a.meta[pr * SH::RP], (uint64_t)(uint32_t)l | (uint64_t)(uint32_t)events << 32);
                    put64(&a.meta[pr * SH::RP].B, 0);
                }
                sc_stores_done();
                if (lane == 0)
                    put64(&a.hdr[pr], (uint64_t)a.ep << 40 | (uint64_t)(fb ? (flags | SF_WIDE) : 0) << 16 | 1u);
            }
        } else if (!last) {
            const int64_t pr = pair0 + h;
            const int np = flags ? 0 : nr;
            for (int r = 0; r < np; ++r) {
#pragma unroll
                for (int k = 0; k < CPL; ++k)
                    put32(&a.runs[(pr * SH::RP + r) * D + lane + 64 * k], (uint32_t)S.S[r0 + r][lane + 64 * k]);
                if (lane == 0) {
                    put64(&a.meta[pr * SH::RP + r],
                          (uint64_t)(uint32_t)S.Lr[r0 + r] | (uint64_t)(r > 0 ? S.evf[r0 + r] : 0u) << 32);
                    put64(&a.meta[pr * SH::RP + r].B, (uint64_t)S.Br[r0 + r]);
                }
            }
            sc_stores_done();
            if (lane == 0) put64(&a.hdr[pr], (uint64_t)a.ep << 40 | (uint64_t)flags << 16 | (uint32_t)np);
        } else {
            fb = flags != 0;
        }
    }
    if (!last) return;

    // -- phase 7: the last chunk replays the chain ------------------------------------------------
    if (chunk > 0) {
        constexpr int CB = SH::CB, NP = SH::CB * G;
        __syncthreads();                                    // the phase buffers are dead
        for (int c0 = 0; c0 < nch - 1; c0 += CB) {
            const int nb = nch - 1 - c0 < CB ? nch - 1 - c0 : CB;
            const int64_t bp = ((int64_t)chain * a.mc + c0) * G * SH::RP;   // the batch's first run
            // every (chunk, head) of the batch: wait for its header
            if (tid < nb * G) {
                const uint64_t *hp = (const uint64_t *)&a.hdr[((int64_t)chain * a.mc + c0) * G + tid];
                uint64_t w = 0;
                int spins = 0;
                bool ok = a.spin_limit > 0;
                while (ok) {
                    w = take64(hp);
                    if ((w >> 40) == a.ep) break;
                    if (++spins > a.spin_limit) ok = false;
                    else __builtin_amdgcn_s_sleep(1);
                }
                S.u.rp.hw[tid] = ok ? w : (uint64_t)SF_LOOKBACK << 16;
            }
            __syncthreads();
            // the batch's runs in walk order, head by head (chunk, then run, within a head):
            // an exclusive prefix over the pairs taken head-major, by wave 0, which records
            // the run behind every slot, each head's first slot and count, and the heads
            // with a pair that published nothing usable
            if (wv == 0) {
                if (lane < G) S.u.rp.hbad[lane] = 0;
                int carry = 0;
                for (int i0 = 0; i0 < nb * G; i0 += 64) {
                    const int i = i0 + lane;
                    const bool live = i < nb * G;
                    const int hh = live ? i / nb : 0, cb = live ? i - hh * nb : 0;
                    const int pg = cb * G + hh;
                    const uint64_t w = live ? S.u.rp.hw[pg] : 0ull;
                    const bool ok = live && (w >> 40) == a.ep && ((w >> 16) & 0xFF) == 0 && (w & 0xFFFF) >= 1 &&
                                    (w & 0xFFFF) <= (uint64_t)SH::RP;
                    const int nr = ok ? (int)(w & 0xFFFF) : 0;
                    const int inc = (int)wave_scan_add32((uint32_t)nr);
                    const int x0 = carry + inc - nr;
                    for (int r = 0; r < nr; ++r) S.u.rp.src[x0 + r] = (int16_t)(pg * SH::RP + r);
                    if (live && cb == 0) S.u.rp.hb[hh] = x0;
                    if (live && !ok) S.u.rp.hbad[hh] = 1;
                    carry += __builtin_amdgcn_readlane(inc, 63);
                }
                if (lane < G) S.u.rp.hn[lane] = (lane + 1 < G ? S.u.rp.hb[lane + 1] : carry) - S.u.rp.hb[lane];
                if (lane == 0) S.u.rp.nslot = carry;
            }
            __syncthreads();
            // every slot below RB: its run and metadata. Thread i loads 8 bytes of slot
            // i / (D / 2); all of a thread's loads are issued before the first is used.
            {
                constexpr int H2 = D / 2, NI = (SH::RB * H2 + SC_NT - 1) / SC_NT;
                const int ns = S.u.rp.nslot < SH::RB ? S.u.rp.nslot : SH::RB;
                uint64_t v[NI];
                int at[NI];
#pragma unroll
                for (int j = 0; j < NI; ++j) {
                    const int i = tid + j * SC_NT, sl = i / H2;
                    at[j] = sl < ns ? i : -1;
                    if (sl < ns) v[j] = take64(&a.runs[(bp + S.u.rp.src[sl]) * D + 2 * (i % H2)]);
                }
                RunMeta m{};
                if (tid < ns) m = scan_meta<G, SH::RP>(a, bp, S.u.rp.src[tid], c0);
#pragma unroll
                for (int j = 0; j < NI; ++j) {
                    if (at[j] < 0) continue;
                    int32_t *d2 = &S.u.rp.rs[at[j] / H2][2 * (at[j] % H2)];
                    d2[0] = (int32_t)(uint32_t)v[j];
                    d2[1] = (int32_t)(uint32_t)(v[j] >> 32);
                }
                if (tid < ns) S.u.rp.rm[tid] = m;
            }
            __syncthreads();
            if (hw && !fb) {
                if (S.u.rp.hbad[h]) {
                    fb = true;
                } else {
                    // While the walk is safe, |acc| <= ACC_HI: acc is held in int32 here.
                    // Every run is applied the same way, branch-free: scale by its factor
                    // (2^15 for a run that only adds, an exact identity), check, add.
                    bool unsafe = false;
                    int32_t a32[CPL];
#pragma unroll
                    for (int k = 0; k < CPL; ++k) a32[k] = (int32_t)acc[k];
                    int base = S.u.rp.hb[h], n = S.u.rp.hn[h];
                    if (c0 == 0) {
                        // the head's first run is chunk 0's state
                        RunMeta m0;
                        if (base < SH::RB) {
                            m0 = S.u.rp.rm[base];
#pragma unroll
                            for (int k = 0; k < CPL; ++k) a32[k] = S.u.rp.rs[base][lane + 64 * k];
                        } else {                           // past the batch's slots: from memory
                            m0 = scan_meta<G, SH::RP>(a, bp, S.u.rp.src[base], c0);
#pragma unroll
                            for (int k = 0; k < CPL; ++k)
                                a32[k] = (int32_t)take32(&a.runs[(bp + S.u.rp.src[base]) * D + lane + 64 * k]);
                        }
                        if (!(m0.f & RM_STATE)) unsafe = true;
                        l = m0.L;
                        events += m0.f & RM_VALUE;
                        ++base;
                        --n;
                    }
                    for (int i0 = 0; i0 < n; i0 += 64) {
                        // lane j: run i0 + j's factor, p sum, and the largest |acc| the run
                        // admits at its start, ACC_HI - B (a run with B > ACC_HI, which the
                        // publishing chunk already flags, makes the walk unsafe outright)
                        RunMeta ml{};
                        const bool mine = i0 + lane < n;
                        const int sl = base + i0 + lane;
                        if (mine) ml = sl < SH::RB ? S.u.rp.rm[sl] : scan_meta<G, SH::RP>(a, bp, S.u.rp.src[sl], c0);
                        const bool wide = ml.B > (uint64_t)ACC_HI;
                        const bool resc = mine && (ml.f & RM_RESCALE) != 0u;
                        unsafe = unsafe || __ballot(wide || (mine && (ml.f & RM_STATE) != 0u)) != 0ull;
                        events += (unsigned long long)__popcll(__ballot(resc));
                        const uint32_t lim = wide ? 0u : (uint32_t)(ACC_HI - (int64_t)ml.B);
                        const uint32_t fac = resc ? (ml.f & RM_VALUE) : (1u << PROB_FRAC);
                        const int cnt = n - i0 < 64 ? n - i0 : 64;
                        const bool fast = base + i0 + cnt <= SH::RB;     // every run of the group in LDS
                        for (int j0 = 0; j0 < cnt; j0 += 4) {
                            int32_t sv[4][CPL];
#pragma unroll
                            for (int u = 0; u < 4; ++u) {
                                int ss = base + i0 + j0 + u;
                                ss = ss < SH::RB ? ss : SH::RB - 1;      // past the group: not used
#pragma unroll
                                for (int k = 0; k < CPL; ++k) sv[u][k] = S.u.rp.rs[ss][lane + 64 * k];
                            }
#pragma unroll
                            for (int u = 0; u < 4; ++u) {
                                const int j = j0 + u;
                                if (j >= cnt) break;
                                if (!fast && base + i0 + j >= SH::RB) {  // past the batch's slots: from memory
                                    const int64_t ro = (bp + S.u.rp.src[base + i0 + j]) * D;
#pragma unroll
                                    for (int k = 0; k < CPL; ++k) sv[u][k] = (int32_t)take32(&a.runs[ro + lane + 64 * k]);
                                }
                                const int64_t fv = (uint32_t)__builtin_amdgcn_readlane((int)fac, j);
                                const uint32_t lm = (uint32_t)__builtin_amdgcn_readlane((int)lim, j);
                                l = ((l * fv) >> PROB_FRAC) + (uint32_t)__builtin_amdgcn_readlane((int)ml.L, j);
#pragma unroll
                                for (int k = 0; k < CPL; ++k) {
                                    const uint32_t x = (uint32_t)(int32_t)(((int64_t)a32[k] * fv) >> PROB_FRAC);
                                    unsafe = unsafe || ((int32_t)x < 0 ? 0u - x : x) > lm;
                                    a32[k] = (int32_t)(x + (uint32_t)sv[u][k]);   // wraps only once unsafe
                                }
                            }
                        }
                    }
#pragma unroll
                    for (int k = 0; k < CPL; ++k) acc[k] = a32[k];
                    fb = __ballot(unsafe) != 0ull;
                }
            }
            __syncthreads();
        }
        if (hw && !fb) {
            // this chunk's own runs
            bool unsafe = false;
            const int r0 = rb[h];
            for (int r = 0; r < n_run[h]; ++r) {
                if (r > 0) {
                    const int64_t f = S.evf[r0 + r];
#pragma unroll
                    for (int k = 0; k < CPL; ++k) acc[k] = (acc[k] * f) >> PROB_FRAC;
                    l = (l * f) >> PROB_FRAC;
                    ++events;
                }
                const int64_t B = (int64_t)S.Br[r0 + r];
#pragma unroll
                for (int k = 0; k < CPL; ++k) {
                    const int64_t av = acc[k] < 0 ? -acc[k] : acc[k];
                    unsafe = unsafe || av + B > ACC_HI;
                    acc[k] += S.S[r0 + r][lane + 64 * k];
                }
                l += (int64_t)S.Lr[r0 + r];
            }
            fb = __ballot(unsafe) != 0ull;
        }
    }
    fb = __builtin_amdgcn_readfirstlane((int)fb) != 0;
    __syncthreads();                       // the serial path reuses the LDS
    if (!hw) return;
    const int qh = kvh * G + h;
    int32_t *orow = a.out + ((int64_t)b * g.n_q + qh) * D;
    if (fb) {
        if (STEP) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        serial_head<CPL, SH::RS>(g, a.tabs, S.kc, S.vc, &S.qi[h][0], b, kvh, T, 0, !qok, S.u.fb[h], orow, a.st);
        if (lane == 0) atomicAdd(&a.st->serial_fallbacks, 1ull);
        return;
    }
    const Recip rc = reciprocal(l);
    int64_t amax = 0;
#pragma unroll
    for (int k = 0; k < CPL; ++k) {
        orow[lane + 64 * k] = (int32_t)(wmul(acc[k], rc.r) >> rc.shift);
        const int64_t av = acc[k] < 0 ? -acc[k] : acc[k];
        amax = av > amax ? av : amax;
    }
    amax = wave_max_i64(amax);
    if (lane == 0) {
        atomicMax(&a.st->n_tokens, (unsigned long long)T);
        if (events) atomicAdd(&a.st->rescale_events, events);
        atomicMax(&a.st->max_abs_acc, (unsigned long long)amax);
    }
}

template <int D, int G>
struct ScanLayout {
    static size_t carve(const Geom &g, int64_t mc, uint8_t *p, ScanArgs *a, int rp) {
        const int64_t chains = (int64_t)g.batch * g.n_kv;
        size_t o = 0;
        auto take = [&](size_t n) {
            const size_t at = o;
            o += (n + 255) / 256 * 256;
            return p ? p + at : nullptr;
        };
        const int64_t pairs = chains * mc * G;
        uint8_t *status = take(pairs * 16), *hdr = take(pairs * 8);   // two look-back words per pair
        uint8_t *meta = take(pairs * rp * sizeof(RunMeta));   // 16-byte records
        uint8_t *runs = take(pairs * rp * D * 4);
        uint8_t *qd = take(chains * mc * D * G * 8);
        if (a) {
            a->status = (unsigned long long *)status;
            a->hdr = (unsigned long long *)hdr;
            a->meta = (RunMeta *)meta;
            a->runs = (int32_t *)runs;
            a->qd = (double *)qd;
            a->mc = (int32_t)mc;
        }
        return o;
    }
};

template <int D, int KB, int VB, int G>
hipError_t scan_launch(hipStream_t s, ScanArgs &a, ChunkScratch &cs, int64_t grid_chunks, bool step, LaunchEv ev) {
    using SH = ScanShape<D, KB, VB, G>;
    ScanLayout<D, G>::carve(a.g, a.mc, (uint8_t *)cs.p, &a, SH::RP);
    // the look-back words and headers (the front of the carve) are the words read
    // before their epoch is known to be current: zero them when the buffer was
    // laid out differently by the previous launch
    const uint64_t layout = ((uint64_t)a.mc << 32) ^ ((uint64_t)a.g.batch << 16) ^ ((uint64_t)a.g.n_kv << 8) ^
                            (uint64_t)(D + G) ^ (2ull << 60);
    const hipError_t e = scratch_layout(s, cs, layout, (size_t)((uint8_t *)a.meta - (uint8_t *)cs.p));
    if (e != hipSuccess) return e;
    const dim3 grid((unsigned)(grid_chunks * a.g.batch * a.g.n_kv)), block(SC_NT);
    if (step)
        hipExtLaunchKernelGGL((scan_kernel<D, KB, VB, G, true>), grid, block, 0, s, ev.start, ev.stop, 0, a);
    else
        hipExtLaunchKernelGGL((scan_kernel<D, KB, VB, G, false>), grid, block, 0, s, ev.start, ev.stop, 0, a);
    return hipGetLastError();
}

template <int G>
int scan_rp(int d) {
    (void)d;
    return 8;
}

}  // namespace

int64_t scan_max_chunks(int64_t tokens) { return tokens > 0 ? (tokens + SC_CHUNK - 1) / SC_CHUNK : 1; }

bool scan_supported(const Geom &g, int64_t capacity) {
    const bool fmt = (g.d == 64 && g.kb == 4 && g.vb == 2 && (g.G == 4 || g.G == 8)) ||
                     (g.d == 128 && g.kb == 3 && g.vb == 3 && g.G == 4);
    return fmt && scan_max_chunks(capacity) <= SC_MAXCH;
}

size_t scan_scratch_bytes(const Geom &g, int64_t mc) {
    if (g.G == 4)
        return g.d == 64 ? ScanLayout<64, 4>::carve(g, mc, nullptr, nullptr, scan_rp<4>(64))
                         : ScanLayout<128, 4>::carve(g, mc, nullptr, nullptr, scan_rp<4>(128));
    return g.d == 64 ? ScanLayout<64, 8>::carve(g, mc, nullptr, nullptr, scan_rp<8>(64))
                     : ScanLayout<128, 8>::carve(g, mc, nullptr, nullptr, scan_rp<8>(128));
}

hipError_t launch_attend_scan(hipStream_t s, const Geom &g, const Tables *t, const int32_t *q, int32_t *out,
                              const int64_t *len, ChunkScratch &cs, uint32_t ep, int64_t mc, int64_t grid_chunks,
                              const StepIn *step, LaunchEv ev, DevStats *st) {
    if (!scan_supported(g, mc * SC_CHUNK) || grid_chunks < 1 || grid_chunks > mc || ep == 0 ||
        ep > (uint32_t)SC_EPOCH_MASK)
        return hipErrorInvalidValue;
    if (scan_scratch_bytes(g, mc) > cs.bytes) return hipErrorInvalidValue;
    ScanArgs a{};
    a.g = g;
    a.tabs = t;
    a.q = q;
    a.out = out;
    a.len = len;
    if (step) a.si = *step;
    a.st = st;
    a.mc = (int32_t)mc;
    a.ep = ep;
    a.spin_limit = cs.spin_limit;
#define INSITU_SCAN(DD, KK, VV, GG)                                            \
    if (g.d == DD && g.kb == KK && g.vb == VV && g.G == GG)                    \
        return scan_launch<DD, KK, VV, GG>(s, a, cs, grid_chunks, step != nullptr, ev);
    INSITU_SCAN(64, 4, 2, 4)
    INSITU_SCAN(128, 3, 3, 4)
    INSITU_SCAN(64, 4, 2, 8)
#undef INSITU_SCAN
    return hipErrorInvalidValue;
}

}  // namespace insitu
